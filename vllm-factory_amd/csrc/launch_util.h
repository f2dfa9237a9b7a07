// Host-side argument checking shared by the libvfk entry points.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/vfk.h"
#include "vfk_host.h"

namespace vfk {

inline int elem_size(int dtype) {
  switch (dtype) {
    case VFK_F32: return 4;
    case VFK_BF16: return 2;
    case VFK_F16: return 2;
    default: return 0;
  }
}

inline int check_tensor(const vfk_tensor* t, const char* name, int ndim) {
  if (!t) return set_error(VFK_ERR_INVALID, "%s: descriptor is NULL", name);
  if (!t->data) return set_error(VFK_ERR_INVALID, "%s: data is NULL", name);
  if (elem_size(t->dtype) == 0)
    return set_error(VFK_ERR_INVALID, "%s: unknown dtype %d", name, t->dtype);
  if (t->ndim != ndim)
    return set_error(VFK_ERR_INVALID, "%s: expected %d dims, got %d", name,
                     ndim, t->ndim);
  for (int i = 0; i < ndim; ++i)
    if (t->size[i] < 0 || t->stride[i] < 0)
      return set_error(VFK_ERR_INVALID, "%s: negative size/stride", name);
  return VFK_OK;
}

inline bool present(const vfk_tensor* t) { return t && t->data; }

inline bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

inline int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error((int)e, "%s: HIP launch failed: %s", what, hipGetErrorString(e));
    return (int)e;
  }
  return VFK_OK;
}

inline int ceil_div(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

}  // namespace vfk
