// Host-side relative-position bucketing, bit-exact with the fp32 eager
// formulas of the reference, plus their conversion into integer step
// functions that the attention kernels evaluate on the device.
//
// Built without -ffast-math and with -ffp-contract=off: every float operation
// below must round exactly once, in the order the reference evaluates it.
#include <limits.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/vfk.h"
#include "vfk_host.h"

namespace vfk {

// models/mt5/mt5_encoder.py:124-148. Every tensor op there runs in fp32:
//   log(rel.float() / max_exact) / log(tensor(max_distance / max_exact))
//   * (num_buckets - max_exact), truncated by .to(torch.long).
// torch.tensor(python_float) is fp32, so the divisor is logf of the fp32
// rounding of max_distance / max_exact.
int t5_bucket_host(int64_t rel, int bidirectional, int num_buckets,
                   int max_distance) {
  int64_t offset = 0;
  int nb = num_buckets;
  int64_t a;
  if (bidirectional) {
    nb /= 2;
    if (rel > 0) offset = nb;
    a = rel < 0 ? -rel : rel;
  } else {
    a = rel < 0 ? -rel : 0;
  }
  const int max_exact = nb / 2;
  if (a < max_exact) return (int)(a + offset);
  const float ratio = (float)a / (float)max_exact;
  const float denom = logf((float)((double)max_distance / (double)max_exact));
  float t = logf(ratio);
  t = t / denom;
  t = t * (float)(nb - max_exact);
  int64_t large = max_exact + (int64_t)t;  // trunc toward zero
  if (large > nb - 1) large = nb - 1;
  return (int)(large + offset);
}

// models/deberta_v2/deberta_v2_encoder.py:70-89 (make_log_bucket_position):
//   abs_pos = |rel| outside (-mid, mid), else mid - 1   (int64)
//   log_pos = ceil(log(abs_pos / mid) / log(tensor((max_position-1)/mid))
//                  * (mid - 1)) + mid                  (fp32)
//   bucket  = rel if abs_pos <= mid else log_pos * sign(rel)
int deberta_bucket_host(int64_t rel, int bucket_size, int max_position) {
  const int mid = bucket_size / 2;
  int64_t a = rel < 0 ? -rel : rel;
  if (a <= mid) return (int)rel;  // covers the (-mid, mid) substitution too
  const float denom = logf((float)((double)(max_position - 1) / (double)mid));
  float t = logf((float)a / (float)mid);
  t = t / denom;
  t = t * (float)(mid - 1);
  float lp = ceilf(t) + (float)mid;
  int v = (int)lp;
  return rel < 0 ? -v : v;
}

static int fill_steps(StepFn* out, int a0, int (*f)(int64_t, const int*),
                      const int* args, int64_t a_end, int f_cap) {
  memset(out, 0, sizeof(*out));
  out->a0 = a0;
  int prev = f(a0, args);
  if (prev > f_cap) prev = f_cap;
  out->f0 = prev;
  int n = 0;
  for (int64_t a = a0 + 1; a <= a_end && prev < f_cap; ++a) {
    int cur = f(a, args);
    if (cur > f_cap) cur = f_cap;
    if (cur < prev)
      return set_error(VFK_ERR_UNSUPPORTED,
                       "bucket function is not monotone at |rel|=%lld",
                       (long long)a);
    while (prev < cur) {
      if (n >= VFK_MAX_THR)
        return set_error(VFK_ERR_UNSUPPORTED,
                         "bucket function needs more than %d steps",
                         VFK_MAX_THR);
      if (a > 32767)
        return set_error(VFK_ERR_UNSUPPORTED,
                         "bucket step at |rel|=%lld exceeds int16",
                         (long long)a);
      out->thr[n++] = (int16_t)a;
      ++prev;
    }
  }
  out->nthr = n;
  return VFK_OK;
}

static int t5_abs_fn(int64_t a, const int* args) {
  // bucket without the (rel > 0) offset as a function of a >= 0: evaluate at
  // rel = -a, where both modes see magnitude a and add no offset.
  return t5_bucket_host(-a, args[0], args[1], args[2]);
}

int build_t5_step(int bidirectional, int num_buckets, int max_distance,
                  StepFn* out) {
  const int nb = bidirectional ? num_buckets / 2 : num_buckets;
  const int max_exact = nb / 2;
  if (max_exact < 1)
    return set_error(VFK_ERR_UNSUPPORTED,
                     "num_buckets=%d gives max_exact=0 (undefined bucket "
                     "formula)",
                     num_buckets);
  if (max_distance <= max_exact)
    return set_error(VFK_ERR_UNSUPPORTED,
                     "max_distance=%d must exceed max_exact=%d", max_distance,
                     max_exact);
  int args[3] = {bidirectional, num_buckets, max_distance};
  // saturates at nb - 1 no later than a = max_distance; scan well past it.
  int64_t a_end = (int64_t)max_distance * 2 + 64;
  int rc = fill_steps(out, max_exact, t5_abs_fn, args, a_end, nb - 1);
  if (rc) return rc;
  if (out->f0 + out->nthr != nb - 1)
    return set_error(VFK_ERR_UNSUPPORTED,
                     "T5 bucket did not saturate by |rel|=%lld",
                     (long long)a_end);
  return VFK_OK;
}

static int deb_abs_fn(int64_t a, const int* args) {
  return deberta_bucket_host(a, args[0], args[1]);
}

int build_deberta_step(int bucket_size, int max_position, int max_abs,
                       int f_cap, StepFn* out) {
  const int mid = bucket_size / 2;
  if (mid < 1 || max_position <= 1)
    return set_error(VFK_ERR_UNSUPPORTED,
                     "position_buckets=%d / max_relative_positions=%d not "
                     "supported",
                     bucket_size, max_position);
  int args[2] = {bucket_size, max_position};
  // |bucket| beyond the gather span only saturates the clamped index, so the
  // kernels stop the step function at f_cap = att_span.
  return fill_steps(out, mid + 1, deb_abs_fn, args, max_abs, f_cap);
}

bool step_is_unit(const StepFn& s) {
  if (s.f0 < s.a0 - 1 || s.f0 > s.a0) return false;
  for (int i = 0; i < s.nthr; ++i) {
    const int prev = i ? s.thr[i - 1] : s.a0;
    if (s.thr[i] <= prev) return false;
  }
  return true;
}

}  // namespace vfk

// ---------------------------------------------------------------------------
// C ABI host helpers
// ---------------------------------------------------------------------------
extern "C" int vfk_t5_bucket(const int64_t* rel, int32_t* out, int64_t n,
                             int32_t bidirectional, int32_t num_buckets,
                             int32_t max_distance) {
  if (n < 0 || (n > 0 && (!rel || !out)))
    return vfk::set_error(VFK_ERR_INVALID, "vfk_t5_bucket: bad arguments");
  // Evaluated through the same integer step function the kernels use.
  vfk::StepFn s;
  int rc = vfk::build_t5_step(bidirectional, num_buckets, max_distance, &s);
  if (rc) return rc;
  const int half = num_buckets / 2;
  for (int64_t i = 0; i < n; ++i) {
    const int64_t r = rel[i];
    if (bidirectional) {
      const int64_t a = r < 0 ? -r : r;
      const int av = a > INT32_MAX ? INT32_MAX : (int)a;
      out[i] = vfk::step_eval(s, av) + (r > 0 ? half : 0);
    } else {
      const int64_t a = r < 0 ? -r : 0;
      out[i] = vfk::step_eval(s, a > INT32_MAX ? INT32_MAX : (int)a);
    }
  }
  return VFK_OK;
}

extern "C" int vfk_deberta_bucket(const int64_t* rel, int32_t* out, int64_t n,
                                  int32_t bucket_size, int32_t max_position) {
  if (n < 0 || (n > 0 && (!rel || !out)))
    return vfk::set_error(VFK_ERR_INVALID, "vfk_deberta_bucket: bad arguments");
  // Evaluated through the same integer step function the kernels use,
  // uncapped up to the largest |rel| asked for.
  int64_t max_abs = 0;
  for (int64_t i = 0; i < n; ++i) {
    const int64_t a = rel[i] < 0 ? -rel[i] : rel[i];
    if (a > max_abs) max_abs = a;
  }
  if (max_abs > 32767)
    return vfk::set_error(VFK_ERR_UNSUPPORTED, "vfk_deberta_bucket: |rel| > 32767");
  vfk::StepFn s;
  int rc = vfk::build_deberta_step(bucket_size, max_position, (int)max_abs,
                                   1 << 30, &s);
  if (rc) return rc;
  for (int64_t i = 0; i < n; ++i) {
    const int64_t r = rel[i];
    const int v = vfk::step_eval(s, (int)(r < 0 ? -r : r));
    out[i] = r < 0 ? -v : v;
  }
  return VFK_OK;
}

extern "C" int vfk_deberta_unit_steps(int32_t position_buckets, int32_t max_relative_distance,
                                      int32_t use_log_bucket, int32_t max_len) {
  // Same span / bucket derivation as the attention entry points
  // (kernels/flash_deberta_attention.py:323, :366-368).
  const int span = position_buckets > 0 ? position_buckets : max_relative_distance;
  if (span <= 0 || max_len < 0)
    return vfk::set_error(VFK_ERR_INVALID, "vfk_deberta_unit_steps: bad arguments");
  if (!use_log_bucket) return 1;  // c = clamp(d + S): unit steps
  const int nb = position_buckets > 0 ? position_buckets : max_relative_distance * 2;
  const int maxd = max_relative_distance > 0 ? max_relative_distance : 512;
  vfk::StepFn s;
  int rc = vfk::build_deberta_step(nb, maxd, max_len, span, &s);
  if (rc) return rc;
  return vfk::step_is_unit(s) ? 1 : 0;
}
