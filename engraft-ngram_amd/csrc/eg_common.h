// Host-side helpers shared by the C-ABI entry points: error reporting and the
// translation of the public structs into kernel arguments.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>

#include "eg_device.h"
#include "engraft_ngram.h"

namespace eg {

// Records the calling thread's last error message; returns `code`.
int set_error(int code, const char* fmt, ...);

#define EG_CHECK_ARG(cond, ...)                                   \
  do {                                                            \
    if (!(cond)) return ::eg::set_error(EG_ERR_ARG, __VA_ARGS__); \
  } while (0)

#define EG_CHECK_HIP(expr)                                                                  \
  do {                                                                                      \
    hipError_t e_ = (expr);                                                                 \
    if (e_ != hipSuccess)                                                                   \
      return ::eg::set_error(EG_ERR_HIP, "%s failed: %s", #expr, hipGetErrorString(e_));   \
  } while (0)

// Validates `spec` and fills the kernel-argument form.
int make_layer_hash(const eg_hash_spec* spec, LayerHash* out);

// Validates a table descriptor (base table or overlay rows).
int make_table(const eg_table* t, TableDev* out, const char* what);

inline int launch_status(const char* kernel) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(EG_ERR_HIP, "launch of %s failed: %s", kernel, hipGetErrorString(e));
  return EG_OK;
}

}  // namespace eg
