"""Write the golden vectors under tests/golden/ from the reference's own kernels.

The vectors come from oracle/_ref/libuaii_ref.so, which `make -C oracle ref`
compiles from the reference's sources in /root/reference (never copied here):
  * tiny_generate.npz — BASELINE config 0 (tiny Llama GGUF, Q8_0, f32 KV cache):
    seeded 32-token prompt, 64 greedy tokens through the reference kernels
    (gguf_dequant, quant_gemm, norm, transformer, softmax, sampling), the last
    step's logits and every layer's resid2 tap; with the GGUF file's SHA-1 so a
    change of the synthetic writer is detected;
  * dequant_blocks.npz — for each of the 10 block formats, 6 rows x 512 random
    block bytes (finite f16 scales) and the reference's dequant_gguf_row output.
Run from the repo root: python3 tests/golden/make_golden.py
"""
import hashlib
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "universal-ai-inference_amd"))
import oracle  # noqa: E402
import uaii_amd  # noqa: E402
from uaii_amd import synth  # noqa: E402

OUT = Path(__file__).resolve().parent
BLOCKQ = [uaii_amd.Q4_0, uaii_amd.Q4_1, uaii_amd.Q5_0, uaii_amd.Q5_1, uaii_amd.Q8_0,
          uaii_amd.Q2_K, uaii_amd.Q3_K, uaii_amd.Q4_K, uaii_amd.Q5_K, uaii_amd.Q6_K]
# byte offsets of the f16 scale fields inside one block, per format
SCALE_OFFS = {uaii_amd.Q4_0: [0], uaii_amd.Q8_0: [0], uaii_amd.Q4_1: [0, 2], uaii_amd.Q5_0: [0],
              uaii_amd.Q5_1: [0, 2], uaii_amd.Q4_K: [0, 2], uaii_amd.Q5_K: [0, 2],
              uaii_amd.Q6_K: [208], uaii_amd.Q2_K: [80, 82], uaii_amd.Q3_K: [108]}


def random_blocks(t, rows, cols, seed):
    rng = np.random.default_rng(seed)
    p = rng.integers(0, 256, size=rows * uaii_amd.row_bytes(t, cols), dtype=np.uint8)
    blocks = p.reshape(-1, uaii_amd.BLOCK[t][1])
    for o in SCALE_OFFS[t]:
        blocks[:, o + 1] &= 0x7b  # f16 exponent < 31: finite scales
    return p


def main():
    if oracle.ref() is None:
        raise SystemExit("build the reference kernels first: make -C oracle ref")
    cfg = synth.PRESETS["tiny"]
    path = synth.cached_model(cfg)
    sha = hashlib.sha1(Path(path).read_bytes()).hexdigest()
    prompt = np.random.default_rng(cfg.seed + 1).integers(0, cfg.vocab, 32).astype(np.int64)
    m = oracle.Model(path)
    ids, logits, resid2 = oracle.ref_generate(path, prompt, 64, n_layers=m.n_layers, dim=m.dim,
                                              vocab=m.vocab)
    np.savez_compressed(OUT / "tiny_generate.npz", prompt=prompt, ids=ids, logits=logits,
                        resid2=resid2, gguf_sha1=np.array(sha))
    arrays = {}
    for t in BLOCKQ:
        rows, cols = 6, 512
        p = random_blocks(t, rows, cols, seed=500 + t)
        arrays[f"bytes_{t}"] = p
        arrays[f"values_{t}"] = oracle.dequant(t, p, rows, cols, use_ref=True)
    np.savez_compressed(OUT / "dequant_blocks.npz", **arrays)
    print("wrote", sorted(x.name for x in OUT.glob("*.npz")), "model sha1", sha)


if __name__ == "__main__":
    main()
