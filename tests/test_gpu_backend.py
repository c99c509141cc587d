"""The ROCm IBackend running the reference's decoder graph op by op.

uaii::backends::RocmBackend (csrc/host/rocm_backend.cpp) takes the operators the
reference's GGUF loader emits for a layer (libs/uaii-loaders/src/gguf.cpp:
916-1209: Embedding, RMSNorm, MatMul with packed weights and transpose_b,
RoPE, Attention with use_kv_cache and layer_id, Add, Silu, Mul, then the final
RMSNorm, the LM-head MatMul and Softmax) through IBackend::dispatch, here via
its C binding (uaii_backend.h). Two layers of a GQA model are run for several
tokens, with the KV cache committed after each token as Session::run does
(session.cpp:1048-1164).

Checks, all against the reference's own CPU kernels (oracle/_ref, compiled
from its sources):
* every op's device output against the reference kernel applied to the same
  inputs (bar 1e-4 tensor-scale relative; the Embedding row bit-exact);
* a complete reference chain of the same ops over the same tokens, on its own
  values: the last token's logits within 2e-3 and the greedy argmax equal at
  every token;
* tokens alternate between host buffers (the reference Session's case, staged
  by the backend) and device buffers (used in place), and the KV cache is f32
  (the reference's) or f16 (K/V rounded to f16 on the reference side too).
"""
import numpy as np
import pytest

import oracle
import uaii_amd
from uaii_amd import synth, DeviceBuffer

pytestmark = pytest.mark.gpu

CFG = synth.ModelConfig(n_layers=2, dim=1024, n_heads=8, n_kv_heads=2, ffn=2816, vocab=1000, ctx_len=64,
                        type_default=uaii_amd.Q4_0, type_attn_v=uaii_amd.Q8_0, seed=301)
EPS = 1e-5


def maxrel(a, b):
    b = np.asarray(b, np.float64)
    return float(np.abs(np.asarray(a, np.float64) - b).max() / max(np.abs(b).max(), 1e-30))


def fp(a):
    import ctypes as C
    return a.ctypes.data_as(C.POINTER(C.c_float))


class Ref:
    """The reference's kernels on numpy arrays (oracle/_ref)."""

    def __init__(self):
        self.R = oracle.ref()

    def matmul(self, x, w):
        t, rows, cols, raw = w
        y = np.zeros(rows, np.float32)
        assert self.R.uref_quant_gemm(t, fp(x), 1, cols, raw.ctypes.data, rows, fp(y)) == 0
        return y

    def rmsnorm(self, x, w):
        y = np.zeros_like(x)
        assert self.R.uref_rmsnorm(fp(x), fp(w), fp(y), x.size, EPS) == 0
        return y

    def rope(self, x, hd, pos, theta, mode):
        y = x.copy()
        assert self.R.uref_rope(fp(y), y.size, hd, float(pos), theta, mode) == 0
        return y

    def attention(self, q, kc, vc, kn, vn, nh, nkv, hd):
        out = np.zeros_like(q)
        past = len(kc)
        K = np.ascontiguousarray(np.array(kc, np.float32).reshape(max(past, 1), -1)) if past else np.zeros(1, np.float32)
        V = np.ascontiguousarray(np.array(vc, np.float32).reshape(max(past, 1), -1)) if past else np.zeros(1, np.float32)
        assert self.R.uref_attention_decode(fp(q), fp(K), fp(V), past, fp(kn), fp(vn), fp(out), nh, nkv, hd) == 0
        return out

    def silu(self, x):
        y = np.zeros_like(x)
        assert self.R.uref_silu(fp(x), fp(y), x.size) == 0
        return y

    def softmax(self, x):
        y = np.zeros_like(x)
        assert self.R.uref_softmax(fp(x), fp(y), x.size) == 0
        return y


class Dev:
    """One op through the backend; activations as host arrays or device buffers."""

    def __init__(self, b):
        self.b = b
        self.device = False

    def run(self, op, inputs, out_shapes, attrs=None):
        ins, keep = [], []
        for x in inputs:
            if isinstance(x, tuple):  # a weight: (gguf type, rows, cols, raw bytes), host memory
                t, rows, cols, raw = x
                if t in (uaii_amd.F32,):
                    arr = raw.view(np.float32).reshape(rows, cols)
                    ins.append(uaii_amd.Backend.view(arr))
                else:
                    ins.append(uaii_amd.Backend.view(raw, shape=(rows, uaii_amd.row_bytes(t, cols)),
                                                     quant=(t, rows, cols)))
            elif self.device:
                buf = DeviceBuffer.from_array(x)
                keep.append(buf)
                ins.append(uaii_amd.Backend.view((buf, x.shape, x.dtype)))
            else:
                ins.append(uaii_amd.Backend.view(x))
        outs, host = [], []
        for shp in out_shapes:
            if self.device:
                buf = DeviceBuffer(int(np.prod(shp)) * 4)
                keep.append(buf)
                outs.append(uaii_amd.Backend.view((buf, shp, np.float32)))
                host.append(buf)
            else:
                a = np.zeros(shp, np.float32)
                outs.append(uaii_amd.Backend.view(a))
                host.append(a)
        self.b.dispatch(op, ins, outs, attrs)
        if self.device:
            self.b.synchronize()
            return [h.to_array(np.float32, int(np.prod(s))).reshape(s) for h, s in zip(host, out_shapes)]
        return host


@pytest.mark.parametrize("kv_f16", [False, True], ids=["f32kv", "f16kv"])
def test_backend_decoder_layers_op_by_op(kv_f16):
    if oracle.ref() is None:
        pytest.skip("reference kernels not built")
    path = synth.cached_model(CFG)
    m = oracle.Model(path)
    D, H, HKV, hd, V = m.dim, m.n_heads, m.n_kv, m.head_dim, m.vocab
    qd, kvd = H * hd, HKV * hd
    theta = 10000.0
    W = {}

    def w(name):
        if name not in W:
            t, rows, cols, raw = m.tensor(name)
            W[name] = (t, rows, cols, np.ascontiguousarray(raw))
        return W[name]

    def f32(name):
        return w(name)[3].view(np.float32).copy()

    ref = Ref()
    b = uaii_amd.Backend()
    assert b.details().startswith("ROCm backend (native")
    b.configure_kv_cache(m.n_layers, 64, kvd, HKV, f16=kv_f16)
    dev = Dev(b)
    prompt = np.random.default_rng(9).integers(0, V, 7)
    rnd = (lambda a: a.astype(np.float16).astype(np.float32)) if kv_f16 else (lambda a: a)
    caches = [([], []) for _ in range(m.n_layers)]          # op-level reference caches
    chain_caches = [([], []) for _ in range(m.n_layers)]    # independent reference chain
    errs = {}

    def check(name, got, want, bar=1e-4):
        e = maxrel(got, want)
        errs[name] = max(errs.get(name, 0.0), e)
        assert e < bar, (name, e)

    for t, tok in enumerate(prompt):
        dev.device = bool(t % 2)
        assert b.past_len() == t
        tokens = np.array([[float(tok)]], np.float32)
        (x,) = dev.run("Embedding", [tokens, w("token_embd.weight")], [(1, D)])
        et, erows, ecols, eraw = w("token_embd.weight")
        want = oracle.dequant(et, eraw[int(tok) * uaii_amd.row_bytes(et, ecols):][:uaii_amd.row_bytes(et, ecols)],
                              1, ecols, use_ref=True)
        assert np.array_equal(x.view(np.uint32), want.view(np.uint32)), "embedding row not bit-exact"
        cx = x[0].copy()  # the independent chain starts from the same exact row
        for li in range(m.n_layers):
            p = f"blk.{li}."
            (n1,) = dev.run("RMSNorm", [x, f32(p + "attn_norm.weight")], [(1, D)], {"eps": EPS})
            check("rmsnorm", n1[0], ref.rmsnorm(x[0], f32(p + "attn_norm.weight")))
            tb = {"transpose_b": True}
            (q,) = dev.run("MatMul", [n1, w(p + "attn_q.weight")], [(1, qd)], tb)
            (k,) = dev.run("MatMul", [n1, w(p + "attn_k.weight")], [(1, kvd)], tb)
            (v,) = dev.run("MatMul", [n1, w(p + "attn_v.weight")], [(1, kvd)], tb)
            check("matmul", q[0], ref.matmul(n1[0], w(p + "attn_q.weight")))
            check("matmul", v[0], ref.matmul(n1[0], w(p + "attn_v.weight")))
            ra = {"theta": theta, "head_dim": hd, "mode": 0}
            (qr,) = dev.run("RoPE", [q], [(1, qd)], ra)
            (kr,) = dev.run("RoPE", [k], [(1, kvd)], ra)
            check("rope", qr[0], ref.rope(q[0], hd, t, theta, 0), 1e-5)
            check("rope", kr[0], ref.rope(k[0], hd, t, theta, 0), 1e-5)
            (att,) = dev.run("Attention", [qr, kr, v], [(1, qd)],
                             {"num_heads": H, "kv_heads": HKV, "causal": True, "use_kv_cache": True,
                              "layer_id": li})
            kc, vc = caches[li]
            want = ref.attention(qr[0], kc, vc, rnd(kr[0]), rnd(v[0]), H, HKV, hd)
            check("attention", att[0], want, 1e-5)
            kc.append(rnd(kr[0]))
            vc.append(rnd(v[0]))
            (o,) = dev.run("MatMul", [att, w(p + "attn_output.weight")], [(1, D)], tb)
            (r1,) = dev.run("Add", [x, o], [(1, D)])
            check("add", r1[0], x[0] + o[0], 1e-7)
            (n2,) = dev.run("RMSNorm", [r1, f32(p + "ffn_norm.weight")], [(1, D)], {"eps": EPS})
            (g,) = dev.run("MatMul", [n2, w(p + "ffn_gate.weight")], [(1, CFG.ffn)], tb)
            (u,) = dev.run("MatMul", [n2, w(p + "ffn_up.weight")], [(1, CFG.ffn)], tb)
            check("matmul", g[0], ref.matmul(n2[0], w(p + "ffn_gate.weight")))
            (ga,) = dev.run("Silu", [g], [(1, CFG.ffn)])
            check("silu", ga[0], ref.silu(g[0]), 1e-6)
            (hdn,) = dev.run("Mul", [ga, u], [(1, CFG.ffn)])
            check("mul", hdn[0], ga[0] * u[0], 1e-7)
            (dn,) = dev.run("MatMul", [hdn, w(p + "ffn_down.weight")], [(1, D)], tb)
            check("matmul", dn[0], ref.matmul(hdn[0], w(p + "ffn_down.weight")))
            (x,) = dev.run("Add", [r1, dn], [(1, D)])

            # the independent chain: the same ops on the reference's own values
            cn1 = ref.rmsnorm(cx, f32(p + "attn_norm.weight"))
            cq = ref.rope(ref.matmul(cn1, w(p + "attn_q.weight")), hd, t, theta, 0)
            ck = rnd(ref.rope(ref.matmul(cn1, w(p + "attn_k.weight")), hd, t, theta, 0))
            cv = rnd(ref.matmul(cn1, w(p + "attn_v.weight")))
            ckc, cvc = chain_caches[li]
            catt = ref.attention(cq, ckc, cvc, ck, cv, H, HKV, hd)
            ckc.append(ck)
            cvc.append(cv)
            cr1 = cx + ref.matmul(catt, w(p + "attn_output.weight"))
            cn2 = ref.rmsnorm(cr1, f32(p + "ffn_norm.weight"))
            ch = ref.silu(ref.matmul(cn2, w(p + "ffn_gate.weight"))) * ref.matmul(cn2, w(p + "ffn_up.weight"))
            cx = cr1 + ref.matmul(ch, w(p + "ffn_down.weight"))
        (normed,) = dev.run("RMSNorm", [x, f32("output_norm.weight")], [(1, D)], {"eps": EPS})
        (logits,) = dev.run("MatMul", [normed, w("output.weight")], [(1, V)], {"transpose_b": True})
        check("matmul", logits[0], ref.matmul(normed[0], w("output.weight")))
        (probs,) = dev.run("Softmax", [logits], [(1, V)], {"axis": -1})
        check("softmax", probs[0], ref.softmax(logits[0]), 1e-5)
        b.commit_kv_step()
        clog = ref.matmul(ref.rmsnorm(cx, f32("output_norm.weight")), w("output.weight"))
        assert int(np.argmax(probs[0])) == int(np.argmax(ref.softmax(clog))), f"argmax differs at token {t}"
        errs["chain_logits"] = max(errs.get("chain_logits", 0.0), maxrel(logits[0], clog))
    print("max rel errors", {k: f"{e:.2e}" for k, e in errs.items()}, flush=True)
    assert errs["chain_logits"] < 2e-3
    b.reset_kv_cache()
    assert b.past_len() == 0
    b.close()


def test_backend_f32_weights_and_refusals():
    """MatMul with f32 weights (the reference's Path A buffers) as [N, K] with
    transpose_b and as [K, N] without, against numpy in f64; the refusals: an op
    without a device kernel (NotImplemented, never a host fallback), a shape
    mismatch and an out-of-range token (InvalidArgument, the reference's
    messages)."""
    b = uaii_amd.Backend()
    rng = np.random.default_rng(4)
    x = rng.standard_normal((3, 256)).astype(np.float32)
    wt = (0.05 * rng.standard_normal((192, 256))).astype(np.float32)
    want = x.astype(np.float64) @ wt.astype(np.float64).T
    y = np.zeros((3, 192), np.float32)
    b.dispatch("MatMul", [b.view(x), b.view(wt)], [b.view(y)], {"transpose_b": True})
    assert maxrel(y, want) < 1e-5
    y2 = np.zeros((3, 192), np.float32)
    wkn = np.ascontiguousarray(wt.T)
    b.dispatch("MatMul", [b.view(x), b.view(wkn)], [b.view(y2)])
    assert maxrel(y2, want) < 1e-5
    with pytest.raises(uaii_amd.UaiiError, match="not_implemented"):
        b.dispatch("LayerNorm", [b.view(x)], [b.view(np.zeros_like(x))])
    with pytest.raises(uaii_amd.UaiiError, match="elementwise numel mismatch"):
        b.dispatch("Add", [b.view(x), b.view(wt)], [b.view(np.zeros_like(x))])
    table = rng.standard_normal((10, 256)).astype(np.float32)
    with pytest.raises(uaii_amd.UaiiError, match="embedding token id out of range: 12 vocab=10"):
        b.dispatch("Embedding", [b.view(np.array([[12.0]], np.float32)), b.view(table)],
                   [b.view(np.zeros((1, 256), np.float32))])
    out = np.zeros((1, 256), np.float32)
    b.dispatch("Embedding", [b.view(np.array([[7.0]], np.float32)), b.view(table)], [b.view(out)])
    assert np.array_equal(out[0], table[7])
    assert lib_no_host_fallback(b)
    b.close()


def lib_no_host_fallback(b):
    return uaii_amd.lib().uaii_backend_uses_host_fallback(b.h) == 0
