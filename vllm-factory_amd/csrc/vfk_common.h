// Shared definitions for the libvfk HIP kernels (gfx950 / CDNA4 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/vfk.h"
#include "vfk_host.h"

// ---------------------------------------------------------------------------
// Vector types used as MFMA operands and for 128-bit memory traffic.
// ---------------------------------------------------------------------------
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

#define VFK_LOG2E 1.4426950408889634f
#define VFK_NUM_XCD 8

namespace vfk {

// Element type tags. Storage of 16-bit types is raw uint16_t bits.
struct BF16 {
  static constexpr int code = VFK_BF16;
  // largest accepted probability bound of the softmax fast path: keeps the
  // fp32 output accumulators far from overflow
  static constexpr float kPMax = 1099511627776.0f;  // 2^40
  static constexpr float kLog2PMax = 40.0f;
  typedef bf16x8_t vec8;
  __device__ static inline float to_f32(uint16_t b) {
    return __uint_as_float(((uint32_t)b) << 16);
  }
  __device__ static inline uint16_t from_f32(float f) {
    __bf16 h = (__bf16)f;
    return __builtin_bit_cast(uint16_t, h);
  }
  // two floats -> packed pair (lo = a)
  __device__ static inline uint32_t pack2(float a, float b) {
    f32x2_t v = {a, b};
    bf16x2_t h = __builtin_convertvector(v, bf16x2_t);
    return __builtin_bit_cast(uint32_t, h);
  }
  // c + a.lo + a.hi for a packed pair a (the row-sum of two probabilities)
  __device__ static inline float dot2_ones(uint32_t a, float c) {
    const bf16x2_t one = {(__bf16)1.0f, (__bf16)1.0f};
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), one, c, false);
  }
  __device__ static inline f32x16_t mfma32(u32x4_t a, u32x4_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(
        __builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
        0, 0, 0);
  }
  __device__ static inline f32x4_t mfma16(u32x4_t a, u32x4_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(
        __builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
        0, 0, 0);
  }
  static constexpr uint32_t kOnePair = 0x3f803f80u;  // (1.0, 1.0)
};

struct F16 {
  static constexpr int code = VFK_F16;
  // probabilities must stay representable in f16 (max 65504)
  static constexpr float kPMax = 32768.0f;
  static constexpr float kLog2PMax = 15.0f;
  typedef f16x8_t vec8;
  __device__ static inline float to_f32(uint16_t b) {
    return (float)__builtin_bit_cast(_Float16, b);
  }
  __device__ static inline uint16_t from_f32(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);
  }
  __device__ static inline uint32_t pack2(float a, float b) {
    f32x2_t v = {a, b};
    f16x2_t h = __builtin_convertvector(v, f16x2_t);
    return __builtin_bit_cast(uint32_t, h);
  }
  __device__ static inline float dot2_ones(uint32_t a, float c) {
    const f16x2_t one = {(_Float16)1.0f, (_Float16)1.0f};
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, a), one, c, false);
  }
  __device__ static inline f32x16_t mfma32(u32x4_t a, u32x4_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(
        __builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c, 0,
        0, 0);
  }
  __device__ static inline f32x4_t mfma16(u32x4_t a, u32x4_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(
        __builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c, 0,
        0, 0);
  }
  static constexpr uint32_t kOnePair = 0x3c003c00u;  // (1.0, 1.0)
};

// Unpack eight 16-bit values held in a u32x4 into floats.
template <typename E>
__device__ inline void unpack8(u32x4_t v, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = E::to_f32((uint16_t)(v[i] & 0xffffu));
    f[2 * i + 1] = E::to_f32((uint16_t)(v[i] >> 16));
  }
}

template <typename E>
__device__ inline u32x4_t pack8(const float* f) {
  u32x4_t r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = E::pack2(f[2 * i], f[2 * i + 1]);
  return r;
}

// Max of a value with the lane 32 positions away (the two half-waves hold
// the same attention row in the S^T layout used by the attention kernels).
__device__ inline float fmax_ieee(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// max over the lane pair (l, l ^ 32) of x, and of m.
__device__ inline float half_swap_max(float x, float m = -__builtin_inff()) {
  int xi = __float_as_int(x);
  auto r = __builtin_amdgcn_permlane32_swap(xi, xi, false, false);
  return fmax_ieee(fmax_ieee(m, __int_as_float(r[0])), __int_as_float(r[1]));
}
__device__ inline float half_swap_sum(float x) {
  int xi = __float_as_int(x);
  auto r = __builtin_amdgcn_permlane32_swap(xi, xi, false, false);
  return __int_as_float(r[0]) + __int_as_float(r[1]);
}

template <int CTRL>
__device__ inline float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of LANES (4..64) lanes, every lane gets the sum:
// DPP quad permutes and row mirrors inside 16 lanes, then the gfx950
// permlane16/32 swaps across rows; no LDS round trips.
template <int LANES>
__device__ inline float group_sum(float v) {
  static_assert(LANES >= 4 && LANES <= 64 && (LANES & (LANES - 1)) == 0, "group size");
  v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]: lane ^ 1
  v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]: lane ^ 2
  if (LANES >= 8) v += dpp_f<0x141>(v);   // row_half_mirror: other quad of 8
  if (LANES >= 16) v += dpp_f<0x140>(v);  // row_mirror: other 8 of 16
  if (LANES >= 32) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_int(v), __float_as_int(v), false, false);
    v = __int_as_float(r[0]) + __int_as_float(r[1]);  // lane ^ 16
  }
  if (LANES >= 64) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false, false);
    v = __int_as_float(r[0]) + __int_as_float(r[1]);  // lane ^ 32
  }
  return v;
}

// Max over aligned groups of LANES lanes, by the same exchange pattern.
template <int LANES>
__device__ inline float group_max(float v) {
  static_assert(LANES >= 4 && LANES <= 64 && (LANES & (LANES - 1)) == 0, "group size");
  v = fmaxf(v, dpp_f<0xB1>(v));
  v = fmaxf(v, dpp_f<0x4E>(v));
  if (LANES >= 8) v = fmaxf(v, dpp_f<0x141>(v));
  if (LANES >= 16) v = fmaxf(v, dpp_f<0x140>(v));
  if (LANES >= 32) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_int(v), __float_as_int(v), false, false);
    v = fmaxf(__int_as_float(r[0]), __int_as_float(r[1]));
  }
  if (LANES >= 64) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false, false);
    v = fmaxf(__int_as_float(r[0]), __int_as_float(r[1]));
  }
  return v;
}

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Workgroups are dispatched round-robin over the 8 XCDs, each with its own
// L2. Remap the hardware block id so that consecutive work items (which
// share K/V rows) run on the same XCD.
__device__ inline int xcd_remap(int bid, int n) {
  int xcd = bid % VFK_NUM_XCD;
  int slot = bid / VFK_NUM_XCD;
  int per = n / VFK_NUM_XCD;
  int rem = n % VFK_NUM_XCD;
  if (xcd < rem) return xcd * (per + 1) + slot;
  return rem * (per + 1) + (xcd - rem) * per + slot;
}

// Division of a 32-bit index by a runtime divisor d >= 1 with a multiply-high
// (round-up method of Granlund and Montgomery): l = ceil(log2 d),
// m = floor(2^32 (2^l - d) / d) + 1, x / d = (umulhi(x, m) + x) >> l, exact
// for every x < 2^32 (the sum is formed in 64 bits).
struct Magic {
  uint32_t d, m;
  int l;
};
inline Magic magic_for(uint32_t d) {
  Magic r;
  r.d = d;
  r.l = 0;
  while ((1ull << r.l) < d) ++r.l;
  r.m = (uint32_t)((((1ull << 32) * ((1ull << r.l) - d)) / d) + 1);
  return r;
}
__device__ inline uint32_t magic_div(uint32_t x, const Magic& g) {
  return (uint32_t)(((uint64_t)__umulhi(x, g.m) + x) >> g.l);
}

}  // namespace vfk

