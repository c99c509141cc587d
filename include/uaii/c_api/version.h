/* version.h — C API semantic version (matches the reference's C API 0.3.0,
 * include/uaii/c_api/version.h). */
#ifndef UAII_C_API_VERSION_H_
#define UAII_C_API_VERSION_H_

#define UAII_C_API_VERSION_MAJOR 0
#define UAII_C_API_VERSION_MINOR 3
#define UAII_C_API_VERSION_PATCH 0
#define UAII_C_API_VERSION_STRING "0.3.0"

/* Package version of this library. */
#define UAII_AMD_VERSION_MAJOR 0
#define UAII_AMD_VERSION_MINOR 1
#define UAII_AMD_VERSION_PATCH 0
#define UAII_AMD_VERSION_STRING "0.1.0"

#endif /* UAII_C_API_VERSION_H_ */
