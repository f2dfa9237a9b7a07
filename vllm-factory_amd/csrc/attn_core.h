// Building blocks shared by the bf16/fp16 attention kernels (head_dim 64).
//
// Work split: a 256-thread workgroup (4 waves) owns a tile of 128 query rows,
// 32 per wave, and streams 64-key tiles of K and V through LDS.
//
// Layouts (v_mfma_f32_32x32x16, lane l, half h = l / 32, c = l % 32):
//   S^T = K Q^T : A = K rows (key c, d 8h..8h+7 of a 16-wide step),
//                 B = Q^T (query c, same d slots) held in registers.
//                 Result lane l: query c, keys 8*(r/4) + 4h + r%4, r < 16.
//   O^T = V^T P^T: B = P^T taken straight from the S^T registers (query c),
//                 A = V^T rows (d c) read from a transposed V tile whose key
//                 slots follow the same (r/4, h, r%4) order.
// Each lane therefore owns one query row: the softmax needs one exchange
// with lane l^32 for the tile max and one for the final row sum.
#pragma once

#include "vfk_common.h"

namespace vfk {

constexpr int kBM = 128;        // query rows per workgroup
constexpr int kBN = 64;         // keys per tile
constexpr int kHD = 64;         // head dim
constexpr int kKsStride = 72;   // u16 per K-tile row (64 + 8 pad, 16B aligned)
constexpr int kVtStride = 68;   // u16 per V^T-tile row (64 + 4 pad, 8B aligned)
constexpr int kKsElems = kBN * kKsStride;
constexpr int kVtElems = kHD * kVtStride;
constexpr float kRescaleSlack = 8.0f;  // log2 units: defer O rescales < 256x

// Registers holding one K/V tile between its global load and LDS store.
struct KVStage {
  u32x4_t k0, k1;  // K row r = t>>2: d chunks cp=t&3 and cp+4 (d and d+32)
  u32x4_t v0, v1;  // V rows 2*(t>>3) and +1: d chunk t&7
};

// Loads the 64-key tile starting at key0; rows >= kend are zero.
// Kp/Vp point at key 0 of the (batch, head); ksr/vsr are row strides.
__device__ inline void kv_load(KVStage& st, const uint16_t* __restrict__ Kp,
                               int64_t ksr, const uint16_t* __restrict__ Vp,
                               int64_t vsr, int key0, int kend) {
  const int t = threadIdx.x;
  const int kr = key0 + (t >> 2);
  const int cp = t & 3;
  const u32x4_t z = {0u, 0u, 0u, 0u};
  if (kr < kend) {
    const uint16_t* row = Kp + (int64_t)kr * ksr;
    st.k0 = *reinterpret_cast<const u32x4_t*>(row + cp * 8);
    st.k1 = *reinterpret_cast<const u32x4_t*>(row + 32 + cp * 8);
  } else {
    st.k0 = z;
    st.k1 = z;
  }
  const int vr = key0 + 2 * (t >> 3);
  const int c = t & 7;
  st.v0 = vr < kend ? *reinterpret_cast<const u32x4_t*>(Vp + (int64_t)vr * vsr + c * 8) : z;
  st.v1 = vr + 1 < kend ? *reinterpret_cast<const u32x4_t*>(Vp + (int64_t)(vr + 1) * vsr + c * 8) : z;
}

__device__ inline void kv_store(const KVStage& st, uint16_t* __restrict__ Ks,
                                uint16_t* __restrict__ Vt) {
  const int t = threadIdx.x;
  const int kr = t >> 2, cp = t & 3;
  *reinterpret_cast<u32x4_t*>(Ks + kr * kKsStride + cp * 8) = st.k0;
  *reinterpret_cast<u32x4_t*>(Ks + kr * kKsStride + 32 + cp * 8) = st.k1;
  // V^T: pack (key 2kp, key 2kp+1) at each d into one dword
  const int kp = t >> 3, c = t & 7;
  uint32_t* vt32 = reinterpret_cast<uint32_t*>(Vt);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t a = st.v0[i], b = st.v1[i];
    const uint32_t lo = (a & 0xffffu) | (b << 16);    // d = 8c + 2i
    const uint32_t hi = (a >> 16) | (b & 0xffff0000u);  // d = 8c + 2i + 1
    vt32[((c * 8 + 2 * i) * kVtStride) / 2 + kp] = lo;
    vt32[((c * 8 + 2 * i + 1) * kVtStride) / 2 + kp] = hi;
  }
}

// S^T for this wave's 32 queries against the 64-key tile.
template <typename E>
__device__ inline void qk_tile(const uint16_t* __restrict__ Ks,
                               const u32x4_t (&q)[4], f32x16_t& s0,
                               f32x16_t& s1) {
  const int l = threadIdx.x & 63;
  const int c = l & 31, h = l >> 5;
  const f32x16_t z = {};
  s0 = z;
  s1 = z;
#pragma unroll
  for (int ds = 0; ds < 4; ++ds) {
    const u32x4_t a0 = *reinterpret_cast<const u32x4_t*>(Ks + c * kKsStride + ds * 16 + 8 * h);
    const u32x4_t a1 = *reinterpret_cast<const u32x4_t*>(Ks + (32 + c) * kKsStride + ds * 16 + 8 * h);
    s0 = E::mfma32(a0, q[ds], s0);
    s1 = E::mfma32(a1, q[ds], s1);
  }
}

// O^T += V^T P^T, P packed per 16-key step (p[ks] slots = x[8ks .. 8ks+7]).
template <typename E>
__device__ inline void pv_tile(const uint16_t* __restrict__ Vt,
                               const u32x4_t (&p)[4], f32x16_t& o0,
                               f32x16_t& o1) {
  const int l = threadIdx.x & 63;
  const int c = l & 31, h = l >> 5;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const uint16_t* r0 = Vt + c * kVtStride + ks * 16 + 4 * h;
    const uint16_t* r1 = Vt + (32 + c) * kVtStride + ks * 16 + 4 * h;
    const u32x2_t a0l = *reinterpret_cast<const u32x2_t*>(r0);
    const u32x2_t a0h = *reinterpret_cast<const u32x2_t*>(r0 + 8);
    const u32x2_t a1l = *reinterpret_cast<const u32x2_t*>(r1);
    const u32x2_t a1h = *reinterpret_cast<const u32x2_t*>(r1 + 8);
    const u32x4_t a0 = {a0l[0], a0l[1], a0h[0], a0h[1]};
    const u32x4_t a1 = {a1l[0], a1l[1], a1h[0], a1h[1]};
    o0 = E::mfma32(a0, p[ks], o0);
    o1 = E::mfma32(a1, p[ks], o1);
  }
}

// Key offset within the tile of score element x[i], i = kb*16 + r.
__device__ inline int x_key(int i, int h) {
  const int kb = i >> 4, r = i & 15;
  return kb * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
}

// Online softmax over one tile of raw scores x (bias already added, -inf =
// masked); c = softmax scale * log2(e), so p = exp2(c * (x - m)) is one FMA
// and one exp2 per score. m: running reference max in raw units; l: this
// lane's partial row sum.
// exact: evaluate (x - m) * c instead of fma(x, c, -m*c). Needed when x may
// carry a huge finite additive mask (|x| ~ 1e30): the rounding of m*c alone
// would then exceed the whole exponent range, while x - m stays exact.
template <typename E>
__device__ inline void softmax_tile(float (&x)[32], float c, float& m, float& l,
                                    f32x16_t& o0, f32x16_t& o1,
                                    u32x4_t (&p)[4], bool exact = false) {
  float mx = x[0];
#pragma unroll
  for (int i = 1; i < 32; ++i) mx = fmaxf(mx, x[i]);
  mx = half_swap_max(mx);
  const float m_new = fmaxf(m, mx);
  // Rescale only when the max grew by more than 2^kRescaleSlack; otherwise
  // keep the old reference (probabilities may then reach 256, harmless).
  const bool need = (m_new - m) * c > kRescaleSlack;
  if (__builtin_amdgcn_ballot_w64(need)) {
    if (m_new != -INFINITY) {
      const float alpha = fast_exp2((m - m_new) * c);  // m = -inf -> 0
      o0 *= alpha;
      o1 *= alpha;
      l *= alpha;
      m = m_new;
    }
  }
  float sum = 0.f;
  if (exact) {
    const float ms = (m == -INFINITY) ? 0.f : m;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      x[i] = fast_exp2((x[i] - ms) * c);
      sum += x[i];
    }
  } else {
    const float nmc = (m == -INFINITY) ? 0.f : -m * c;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      x[i] = fast_exp2(__builtin_fmaf(x[i], c, nmc));
      sum += x[i];
    }
  }
  l += sum;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) p[ks] = pack8<E>(&x[8 * ks]);
}

// Writes this lane's normalised output row (query c) for d in the O^T layout.
// Rows with no visible key (l == 0) are written as zeros.
template <typename E>
__device__ inline void store_out(uint16_t* __restrict__ orow, f32x16_t o0,
                                 f32x16_t o1, float l_tot) {
  const int h = (threadIdx.x & 63) >> 5;
  const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    u32x2_t w0, w1;
    w0[0] = E::pack2(o0[4 * j] * inv, o0[4 * j + 1] * inv);
    w0[1] = E::pack2(o0[4 * j + 2] * inv, o0[4 * j + 3] * inv);
    w1[0] = E::pack2(o1[4 * j] * inv, o1[4 * j + 1] * inv);
    w1[1] = E::pack2(o1[4 * j + 2] * inv, o1[4 * j + 3] * inv);
    *reinterpret_cast<u32x2_t*>(orow + 8 * j + 4 * h) = w0;
    *reinterpret_cast<u32x2_t*>(orow + 32 + 8 * j + 4 * h) = w1;
  }
}

// Q^T operand for this lane's query row (zeros when the row is invalid).
// Lane (c, h) holds d = 16*ds + 8*h + i, i < 8, for ds = 0..3.
__device__ inline void load_q(u32x4_t (&q)[4], const uint16_t* __restrict__ qrow,
                              bool valid) {
  const int h = (threadIdx.x & 63) >> 5;
  const u32x4_t z = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int ds = 0; ds < 4; ++ds)
    q[ds] = valid ? *reinterpret_cast<const u32x4_t*>(qrow + ds * 16 + 8 * h) : z;
}

// Native sin/cos of 2*pi*r (r in revolutions), range-reduced with fract.
__device__ inline void sincos_rev(float r, float& s, float& c) {
  const float f = __builtin_amdgcn_fractf(r);
  s = __builtin_amdgcn_sinf(f);
  c = __builtin_amdgcn_cosf(f);
}

// Rotates the Q operand in registers (non-interleaved RoPE halves): the lane's
// chunks ds and ds+2 hold d and d+32. inv_freq_rev[f] = inv_freq[f] / (2 pi).
template <typename E>
__device__ inline void rope_q(u32x4_t (&q)[4], int pos, const float* inv_freq_rev) {
  const int h = (threadIdx.x & 63) >> 5;
#pragma unroll
  for (int dl = 0; dl < 2; ++dl) {
    float a[8], b[8];
    unpack8<E>(q[dl], a);
    unpack8<E>(q[dl + 2], b);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float sn, cs;
      sincos_rev((float)pos * inv_freq_rev[16 * dl + 8 * h + i], sn, cs);
      const float x1 = a[i], x2 = b[i];
      a[i] = x1 * cs - x2 * sn;
      b[i] = x2 * cs + x1 * sn;
    }
    q[dl] = pack8<E>(a);
    q[dl + 2] = pack8<E>(b);
  }
}

// Rotates a staged K tile row (thread t holds key t>>2, d chunks cp and cp+4
// with cp = t&3) for key position pos. inv_freq_rev8[i] is the frequency of
// d = 8*cp + i (the caller's 8-entry slice for its cp).
template <typename E>
__device__ inline void rope_k(KVStage& st, int pos, const float (&inv_freq_rev8)[8]) {
  float a[8], b[8];
  unpack8<E>(st.k0, a);
  unpack8<E>(st.k1, b);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float sn, cs;
    sincos_rev((float)pos * inv_freq_rev8[i], sn, cs);
    const float x1 = a[i], x2 = b[i];
    a[i] = x1 * cs - x2 * sn;
    b[i] = x2 * cs + x1 * sn;
  }
  st.k0 = pack8<E>(a);
  st.k1 = pack8<E>(b);
}

}  // namespace vfk
