// Host-side declarations shared by the libvfk entry points. No HIP types, so
// plain C++ translation units (bucket.cpp) can include it.
#pragma once
#include <stdint.h>

#ifdef __HIPCC__
#define VFK_HD __host__ __device__
#else
#define VFK_HD
#endif

namespace vfk {

// Relative-position bucket as a monotone step function of a >= 0:
//   f(a) = a                          for a < a0
//   f(a) = f0 + #{ i : thr[i] <= a }  for a >= a0
// Built on the host from the exact fp32 reference formulas (bucket.cpp) and
// evaluated on the device with integer arithmetic only.
#define VFK_MAX_THR 320
struct StepFn {
  int32_t a0;
  int32_t f0;
  int32_t nthr;
  int32_t pad;
  int16_t thr[VFK_MAX_THR];
};

// Integer evaluation of a StepFn; the same code runs in the kernels.
VFK_HD inline int step_eval(const StepFn& s, int a) {
  if (a < s.a0) return a;
  int lo = 0, hi = s.nthr;  // number of thresholds <= a
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if ((int)s.thr[mid] <= a)
      lo = mid + 1;
    else
      hi = mid;
  }
  return s.f0 + lo;
}

int set_error(int code, const char* fmt, ...);

// T5 bucket of rel = key - query (fp32 reference formula).
int t5_bucket_host(int64_t rel, int bidirectional, int num_buckets,
                   int max_distance);
// Step function of a = |rel| (bidirectional) or a = max(-rel, 0) (causal)
// giving the bucket without the sign offset. Returns 0 or a VFK_ERR code.
int build_t5_step(int bidirectional, int num_buckets, int max_distance,
                  StepFn* out);

// DeBERTa log bucket of rel = query - key (fp32 reference formula).
int deberta_bucket_host(int64_t rel, int bucket_size, int max_position);
// Step function of a = |rel| giving min(|bucket|, f_cap), exact for
// a <= max_abs.
int build_deberta_step(int bucket_size, int max_position, int max_abs,
                       int f_cap, StepFn* out);

// True when f(a) - f(a - 1) is 0 or 1 for every a >= 1: f0 is a0 - 1 or a0
// and the thresholds strictly increase. The staged and fused DeBERTa kernels
// size their LDS windows on this (a key tile of 64 keys meets at most 64
// consecutive indices of a query row).
bool step_is_unit(const StepFn& s);

}  // namespace vfk
