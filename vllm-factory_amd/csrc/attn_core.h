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

// S^T for this wave's 32 queries against the 64-key tile. All eight K
// operands are read from LDS before the first MFMA so the reads overlap.
template <typename E>
__device__ inline void qk_tile(const uint16_t* __restrict__ Ks,
                               const u32x4_t (&q)[4], f32x16_t& s0,
                               f32x16_t& s1) {
  const int l = threadIdx.x & 63;
  const int c = l & 31, h = l >> 5;
  u32x4_t a0[4], a1[4];
#pragma unroll
  for (int ds = 0; ds < 4; ++ds) {
    a0[ds] = *reinterpret_cast<const u32x4_t*>(Ks + c * kKsStride + ds * 16 + 8 * h);
    a1[ds] = *reinterpret_cast<const u32x4_t*>(Ks + (32 + c) * kKsStride + ds * 16 + 8 * h);
  }
  // keep all eight reads ahead of the MFMAs (the scheduler would otherwise
  // place each read right before its MFMA and expose its latency eight times)
  __builtin_amdgcn_sched_barrier(0);
  const f32x16_t z = {};
  s0 = E::mfma32(a0[0], q[0], z);
  s1 = E::mfma32(a1[0], q[0], z);
#pragma unroll
  for (int ds = 1; ds < 4; ++ds) {
    s0 = E::mfma32(a0[ds], q[ds], s0);
    s1 = E::mfma32(a1[ds], q[ds], s1);
  }
}

// V^T operands of one tile for this lane (8 MFMA A-operands), read ahead of
// the softmax so the LDS latency hides behind it.
struct VOps {
  u32x4_t a[2][4];
};

__device__ inline void pv_load(const uint16_t* __restrict__ Vt, VOps& v) {
  const int l = threadIdx.x & 63;
  const int c = l & 31, h = l >> 5;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
    for (int db = 0; db < 2; ++db) {
      const uint16_t* r = Vt + (db * 32 + c) * kVtStride + ks * 16 + 4 * h;
      const u32x2_t lo = *reinterpret_cast<const u32x2_t*>(r);
      const u32x2_t hi = *reinterpret_cast<const u32x2_t*>(r + 8);
      v.a[db][ks] = u32x4_t{lo[0], lo[1], hi[0], hi[1]};
    }
  }
}

template <typename E>
__device__ inline void pv_mfma(const VOps& v, const u32x4_t (&p)[4], f32x16_t& o0, f32x16_t& o1) {
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    o0 = E::mfma32(v.a[0][ks], p[ks], o0);
    o1 = E::mfma32(v.a[1][ks], p[ks], o1);
  }
}

// O^T += V^T P^T, P packed per 16-key step (p[ks] slots = x[8ks .. 8ks+7]).
template <typename E>
__device__ inline void pv_tile(const uint16_t* __restrict__ Vt,
                               const u32x4_t (&p)[4], f32x16_t& o0,
                               f32x16_t& o1) {
  VOps v;
  pv_load(Vt, v);
  pv_mfma<E>(v, p, o0, o1);
}

// Key offset within the tile of score element x[i], i = kb*16 + r.
__device__ inline int x_key(int i, int h) {
  const int kb = i >> 4, r = i & 15;
  return kb * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
}

// Row sums of the softmax probabilities, two forms; both sum the 16-bit
// probabilities P (the PV operand), so that the denominator is the sum of
// exactly the rounded weights the numerator uses (fp32 sums of the unrounded
// values would be off by the rounding of a row's dominant weight):
//  * RowSumMfma: the 16-bit probabilities P (the PV operand) summed on the
//    matrix core, which takes 31 adds per tile off the vector ALU and makes
//    the denominator the sum of exactly the weights the numerator uses. The
//    P registers are read as the B operand of a 16x16x32 MFMA: lane l gives
//    column n = l % 16 and k = 8 (l / 16) .. +7, i.e. query n + 16 ((l/16) & 1)
//    and 8 of its keys. The A operand selects k-groups by parity:
//    A[m][k] = 1 when (k / 8) % 2 == m % 2, so row m of the product is the
//    16-key sum of query n + 16 (m % 2). Lane l holds rows 4 (l / 16) .. +3:
//    acc[0] = sum of query l % 16, acc[1] = sum of query l % 16 + 16.
//  * RowSumDot: P summed by packed dot products with (1, 1), 16 v_dot2 per
//    tile in one register, for kernels without the 8 registers RowSumMfma
//    needs; each lane sums its 32 keys and total() adds the partner lane's
//    (l ^ 32) share.
template <typename E>
struct RowSumDot {
  float l = 0.f;
  __device__ void scale(float a) { l *= a; }
  __device__ void add_p(const u32x4_t (&p)[4]) {
    float la = 0.f, lb = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      la = E::dot2_ones(p[0][j], la);
      lb = E::dot2_ones(p[1][j], lb);
      la = E::dot2_ones(p[2][j], la);
      lb = E::dot2_ones(p[3][j], lb);
    }
    l += la + lb;
  }
  __device__ float total() const { return half_swap_sum(l); }
};

template <typename E>
struct RowSumMfma {
  f32x4_t acc = {};
  __device__ void scale(float a) { acc *= a; }
  __device__ void add_p(const u32x4_t (&p)[4]) {
    const int l = threadIdx.x & 63;
    const uint32_t s = (((l >> 4) ^ l) & 1) ? 0u : E::kOnePair;
    const u32x4_t sel = {s, s, s, s};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) acc = E::mfma16(sel, p[ks], acc);
  }
  // the row sum of this lane's query c = l % 32
  __device__ float total() const { return (threadIdx.x & 16) ? acc[1] : acc[0]; }
};

// Online softmax over one tile of raw scores (bias already added, -inf =
// masked), held in the two S^T accumulators s0 (keys 0..31) and s1 (32..63).
// c = softmax scale * log2(e), so p = exp2(c * (x - m)) is one FMA and one
// exp2 per score. m: running reference max in raw units; l: the row sum
// (RowSumDot / RowSumMfma). The step is split in two so that a pipelined loop
// can place the parts apart: softmax_ref (row max, O rescale) and softmax_exp
// (probabilities, row sum, 16-bit packing).

// m := max(m, row max of the tile), but only when the max grew by more than
// 2^kRescaleSlack (otherwise the old reference is kept and probabilities may
// reach 256, harmless); O and l are rescaled to the new reference.
template <typename RS>
__device__ inline void softmax_ref(const f32x16_t& s0, const f32x16_t& s1, float c, float& m,
                                   RS& l, f32x16_t& o0, f32x16_t& o1) {
  // IEEE maximum (NaN-propagating) maps to v_maximum3_f32 without the
  // canonicalising moves fmaxf needs: 17 instructions for 32 scores.
  float ma = fmax_ieee(s0[0], s1[0]), mb = fmax_ieee(s0[1], s1[1]);
#pragma unroll
  for (int i = 2; i < 16; i += 2) {
    ma = fmax_ieee(fmax_ieee(ma, s0[i]), s1[i]);
    mb = fmax_ieee(fmax_ieee(mb, s0[i + 1]), s1[i + 1]);
  }
  const float m_new = half_swap_max(fmax_ieee(ma, mb), m);
  const bool need = (m_new - m) * c > kRescaleSlack;
  if (__builtin_amdgcn_ballot_w64(need)) {
    if (m_new != -INFINITY) {
      const float alpha = fast_exp2((m - m_new) * c);  // m = -inf -> 0
      o0 *= alpha;
      o1 *= alpha;
      l.scale(alpha);
      m = m_new;
    }
  }
}

// p := 16-bit exp2((s - m) c) (0 where m = -inf; s is overwritten with the
// fp32 probabilities), and their sum added to l.
// exact: (x - m) * c instead of fma(x, c, -m*c). Needed when x may carry a
// huge finite additive mask (|x| ~ 1e30): the rounding of m*c alone would
// then exceed the whole exponent range, while x - m stays exact.
template <typename E>
__device__ inline void pack_p(const f32x16_t& s0, const f32x16_t& s1, u32x4_t (&p)[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    p[0][j] = E::pack2(s0[2 * j], s0[2 * j + 1]);
    p[1][j] = E::pack2(s0[8 + 2 * j], s0[8 + 2 * j + 1]);
    p[2][j] = E::pack2(s1[2 * j], s1[2 * j + 1]);
    p[3][j] = E::pack2(s1[8 + 2 * j], s1[8 + 2 * j + 1]);
  }
}

template <typename E, typename RS>
__device__ inline void softmax_exp(f32x16_t& s0, f32x16_t& s1, float c, float m, bool exact,
                                   u32x4_t (&p)[4], RS& l) {
  const float ms = (m == -INFINITY) ? 0.f : m;
  if (exact) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      s0[i] = fast_exp2((s0[i] - ms) * c);
      s1[i] = fast_exp2((s1[i] - ms) * c);
    }
  } else {
    const float nmc = -ms * c;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      s0[i] = fast_exp2(__builtin_fmaf(s0[i], c, nmc));
      s1[i] = fast_exp2(__builtin_fmaf(s1[i], c, nmc));
    }
  }
  pack_p<E>(s0, s1, p);
  l.add_p(p);
}

// Probabilities without a reference: p = exp2(c s), no row max, no rescale.
// Callers either know that |c s| <= log2(E::kPMax) (the varlen kernels: a
// bound from |q| and max |k| before the loop, scores already in log2 units,
// c = 1), so p can neither overflow the fp32 accumulators nor underflow the
// 16-bit P operand, or check the row sums and outputs afterwards and run the
// item again with the running max where they are not finite or too small
// (the bf16 RPB kernel).
template <typename E, typename RS>
__device__ inline void softmax_fixed(f32x16_t& s0, f32x16_t& s1, u32x4_t (&p)[4], RS& l,
                                     float c) {
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    s0[i] = fast_exp2(s0[i] * c);
    s1[i] = fast_exp2(s1[i] * c);
  }
  pack_p<E>(s0, s1, p);
  l.add_p(p);
}

template <typename E, typename RS>
__device__ inline void softmax_tile(f32x16_t& s0, f32x16_t& s1, float c, float& m, RS& l,
                                    f32x16_t& o0, f32x16_t& o1,
                                    u32x4_t (&p)[4], bool exact = false) {
  softmax_ref(s0, s1, c, m, l, o0, o1);
  softmax_exp<E>(s0, s1, c, m, exact, p, l);
}

// s_e = f(e, s_e) for the 32 score elements of the accumulator pair.
template <class F>
__device__ inline void map_scores(f32x16_t& s0, f32x16_t& s1, F f) {
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    s0[e] = f(e, s0[e]);
    s1[e] = f(e + 16, s1[e]);
  }
}

// Adds tab[x_key(e, 0)] to score element e of the accumulator pair (e < 16:
// s0[e], else s1[e - 16]); tab already offset by the lane's 4*h.
__device__ inline void add_by_key(f32x16_t& s0, f32x16_t& s1, const float* __restrict__ tab) {
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    s0[e] += tab[x_key(e, 0)];
    s1[e] += tab[x_key(e + 16, 0)];
  }
}

// Score element e of the accumulator pair := tab[x_key(e, 0)] (tab already
// offset by the lane's 4*h), the form of add_by_key that initialises.
__device__ inline void load_by_key(f32x16_t& s0, f32x16_t& s1, const float* __restrict__ tab) {
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    s0[e] = tab[x_key(e, 0)];
    s1[e] = tab[x_key(e + 16, 0)];
  }
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

// ---------------------------------------------------------------------------
// Direct-to-LDS tiles (gfx950 global_load_lds_dwordx4 + ds_read_b64_tr_b16).
//
// A tile is 64 rows (keys) x 64 halves (d) = 64 x 128 B, stored without
// padding; the 16-byte chunk c of row r lives at chunk c ^ swz(r). With this
// swizzle both the QK operand reads (16 B per lane, one row per lane) and the
// transposed V reads (8 B per lane, four rows per 16-lane group) hit distinct
// banks. K and V tiles are written straight from global memory into LDS by
// the load unit (no staging registers, no VALU), double-buffered so the next
// tile streams in while the current one is consumed; one barrier per tile.
// ---------------------------------------------------------------------------
constexpr int kTileElems = 64 * 64;          // u16 per K or V tile (8 KiB)

__device__ inline int swz(int row) { return (((row >> 1) & 1) << 2) | ((row >> 2) & 3); }

// Writes this wave's 32 normalised output rows through LDS so that the global
// stores are whole rows: the lane's values (query row c, d in the O^T layout)
// go to `stage` (32 rows x 128 B, 16-byte chunks swizzled like the tiles),
// then lane l stores the 16-byte chunk l & 7 of rows l >> 3, +8, +16, +24,
// eight lanes per 128-byte row. rowp(r) gives row r's output address (rows
// for which valid(r) is false are skipped). Call with the stage free (after
// the loop's last barrier); the stage is this wave's own.
template <typename E, typename RowP, typename Valid>
__device__ inline void store_out_rows(uint16_t* __restrict__ stage, f32x16_t o0, f32x16_t o1,
                                      float l_tot, RowP rowp, Valid valid) {
  const int lane = threadIdx.x & 63, c = lane & 31, h = lane >> 5;
  const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
  const int f = swz(c);
  char* st = reinterpret_cast<char*>(stage);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    u32x2_t w0, w1;
    w0[0] = E::pack2(o0[4 * j] * inv, o0[4 * j + 1] * inv);
    w0[1] = E::pack2(o0[4 * j + 2] * inv, o0[4 * j + 3] * inv);
    w1[0] = E::pack2(o1[4 * j] * inv, o1[4 * j + 1] * inv);
    w1[1] = E::pack2(o1[4 * j + 2] * inv, o1[4 * j + 3] * inv);
    // d = 8j + 4h (chunk j) and d + 32 (chunk j + 4), 8 bytes at 8h in the chunk
    *reinterpret_cast<u32x2_t*>(st + c * 128 + 16 * (j ^ f) + 8 * h) = w0;
    *reinterpret_cast<u32x2_t*>(st + c * 128 + 16 * ((j + 4) ^ f) + 8 * h) = w1;
  }
  // other lanes of this wave read what each lane wrote
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const int q = lane & 7;
  u32x4_t v[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int r = (lane >> 3) + 8 * k;
    v[k] = *reinterpret_cast<const u32x4_t*>(st + r * 128 + 16 * (q ^ swz(r)));
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int r = (lane >> 3) + 8 * k;
    // non-temporal: the output is not read again by the attention
    if (valid(r)) __builtin_nontemporal_store(v[k], reinterpret_cast<u32x4_t*>(rowp(r) + 8 * q));
  }
}

// Rows [from, to) of one 64-wide 16-bit output slice (row stride rs
// elements, rows 16-byte aligned) written as zeros, eight lanes per 128-byte
// row: the rows of a packed sequence longer than max_seqlen, which the
// varlen kernels do not compute.
__device__ inline void zero_rows_d64(uint16_t* __restrict__ base, int64_t rs, int from, int to) {
  const u32x4_t z = {0u, 0u, 0u, 0u};
  for (int r = from + (int)(threadIdx.x >> 3); r < to; r += (int)(blockDim.x >> 3))
    *reinterpret_cast<u32x4_t*>(base + (int64_t)r * rs + 8 * (threadIdx.x & 7)) = z;
}

typedef __attribute__((address_space(3))) void lds_void_t;
typedef short s16x4_t __attribute__((ext_vector_type(4)));

// Direct-to-LDS tile loads through a buffer resource. The resource covers the
// nvalid rows of one (sequence, head) slice; the hardware range check turns
// every dword past nvalid rows into a zero written to LDS, so tail tiles need
// no clamping, and the tile's row offset travels in the scalar offset, leaving
// no per-tile address arithmetic on the vector ALU.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int kRsrcWord3 = 0x00020000;  // raw buffer, 32-bit data format

struct TileSrc {
  rsrc_t r;
  int rs2;    // row stride in bytes
  int vo[2];  // this lane's byte offsets in the wave's two 1 KiB blocks
};

// rows * rs * 2 must stay below 2^31 (checked by the host).
__device__ inline void tile_src_init(TileSrc& s, const uint16_t* base, int rs, int nvalid) {
  s.r = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(base), 0, nvalid * rs * 2,
                                          kRsrcWord3);
  s.rs2 = rs * 2;
  const int w = threadIdx.x >> 6, p = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int row = 8 * (2 * w + j) + (p >> 3);
    s.vo[j] = row * s.rs2 + 16 * ((p & 7) ^ swz(row));
  }
}

// Loads rows [row0, row0 + 64) into LDS tile t (swizzled 16-byte chunks).
__device__ inline void tile_load_buf(const TileSrc& s, int row0, uint16_t* tile) {
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int soff = row0 * s.rs2;
#pragma unroll
  for (int j = 0; j < 2; ++j)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(s.r, (lds_void_t*)(tile + (2 * w + j) * 512), 16,
                                             s.vo[j], soff, 0, 0);
}

// Buffer resource over nbytes from base, built from readfirstlane'd words:
// the values are uniform, and saying so keeps the compiler from wrapping each
// load through it in a loop over distinct resource values.
__device__ inline rsrc_t uniform_rsrc(const void* base, int nbytes) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)p);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(p >> 32));
  void* ub = reinterpret_cast<void*>(((uint64_t)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(ub, 0, __builtin_amdgcn_readfirstlane(nbytes), kRsrcWord3);
}

// Waits for this wave's outstanding loads and LDS traffic, then joins the
// workgroup barrier: afterwards every direct-loaded tile is visible.
__device__ inline void tile_barrier() {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
}

// Lane offsets are kept in bytes and passed through an empty asm so that the
// compiler adds the (constant) LDS buffer address in the instruction's offset
// field instead of keeping one address register per buffer live across the
// loop. lds_opaque returns an opaque copy (one move per use); lds_refresh
// makes a loop-carried offset opaque in place, once per step, with no move.
__device__ inline int lds_opaque(int x) {
  asm volatile("" : "+v"(x));
  return x;
}
__device__ inline void lds_refresh(int& x) { asm volatile("" : "+v"(x)); }
template <typename T>
__device__ inline T lds_at(const uint16_t* base, int byte_off) {
  return *reinterpret_cast<const T*>(reinterpret_cast<const char*>(base) + byte_off);
}

// Byte offsets of the QK operand reads in a tile: lane (c, h) reads row c
// (+32 for the second key block, +4096 bytes), chunk 2*ds + h.
struct KOff {
  int o[4];
  __device__ void refresh() {
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) lds_refresh(o[ds]);
  }
};
__device__ inline void k_offsets(KOff& k) {
  const int l = threadIdx.x & 63, c = l & 31, h = l >> 5;
  const int f = swz(c);  // swz(kb*32 + c) == swz(c)
#pragma unroll
  for (int ds = 0; ds < 4; ++ds) k.o[ds] = 2 * (c * 64 + 8 * ((2 * ds + h) ^ f));
}

template <typename E>
__device__ inline void qk_tile_sw(const uint16_t* __restrict__ Kt, const KOff& ko,
                                  const u32x4_t (&q)[4], f32x16_t& s0, f32x16_t& s1) {
  u32x4_t a0[4], a1[4];
#pragma unroll
  for (int ds = 0; ds < 4; ++ds) {
    a0[ds] = lds_at<u32x4_t>(Kt, ko.o[ds]);
    a1[ds] = lds_at<u32x4_t>(Kt, ko.o[ds] + 4096);
  }
  // keys 0-31 first, so their softmax can start while keys 32-63 multiply
  const f32x16_t z = {};
  s0 = E::mfma32(a0[0], q[0], z);
#pragma unroll
  for (int ds = 1; ds < 4; ++ds) s0 = E::mfma32(a0[ds], q[ds], s0);
  s1 = E::mfma32(a1[0], q[0], z);
#pragma unroll
  for (int ds = 1; ds < 4; ++ds) s1 = E::mfma32(a1[ds], q[ds], s1);
}

// As qk_tile_sw, accumulating onto s0 / s1, which hold an additive bias of
// the tile's scores on entry (the bias rides on the MFMAs' accumulator input
// instead of costing one add per score).
template <typename E>
__device__ inline void qk_tile_acc(const uint16_t* __restrict__ Kt, const KOff& ko,
                                   const u32x4_t (&q)[4], f32x16_t& s0, f32x16_t& s1) {
  u32x4_t a0[4], a1[4];
#pragma unroll
  for (int ds = 0; ds < 4; ++ds) {
    a0[ds] = lds_at<u32x4_t>(Kt, ko.o[ds]);
    a1[ds] = lds_at<u32x4_t>(Kt, ko.o[ds] + 4096);
  }
#pragma unroll
  for (int ds = 0; ds < 4; ++ds) s0 = E::mfma32(a0[ds], q[ds], s0);
#pragma unroll
  for (int ds = 0; ds < 4; ++ds) s1 = E::mfma32(a1[ds], q[ds], s1);
}

// Byte offsets of the transposed V reads: for 16-key step ks (+2048 bytes), d
// block db and key half hf (keys 16ks + 8hf + 4h + v, v = source-lane row),
// the lane addresses row 16ks + 8hf + 4h + v, columns d0 + 4r of its 16-lane
// group.
struct VOff {
  int o[2][2];  // [db][hf]
  __device__ void refresh() {
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) lds_refresh(o[db][hf]);
  }
};
__device__ inline void v_offsets(VOff& v) {
  const int l = threadIdx.x & 63;
  const int g = l >> 4, sl = l & 15, vv = sl >> 2, r = sl & 3, h = g >> 1;
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
    const int row = 8 * hf + 4 * h + vv;  // + 16*ks (swz unchanged)
    const int f = swz(row);
#pragma unroll
    for (int db = 0; db < 2; ++db) {
      const int d = db * 32 + 16 * (g & 1) + 4 * r;
      v.o[db][hf] = 2 * (row * 64 + 8 * ((d >> 3) ^ f) + (d & 7));
    }
  }
}

__device__ inline uint32_t tr_lo(s16x4_t x) { return __builtin_bit_cast(u32x2_t, x)[0]; }
__device__ inline uint32_t tr_hi(s16x4_t x) { return __builtin_bit_cast(u32x2_t, x)[1]; }

__device__ inline s16x4_t lds_tr16(const uint16_t* base, int byte_off) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4_t*)(reinterpret_cast<const char*>(base) + byte_off));
}

template <typename E>
__device__ inline void pv_tile_sw(const uint16_t* __restrict__ Vt, const VOff& vo,
                                  const u32x4_t (&p)[4], f32x16_t& o0, f32x16_t& o1) {
  const auto& off = vo.o;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    u32x4_t a[2];
#pragma unroll
    for (int db = 0; db < 2; ++db) {
      const s16x4_t lo = lds_tr16(Vt, off[db][0] + ks * 2048);
      const s16x4_t hi = lds_tr16(Vt, off[db][1] + ks * 2048);
      a[db] = u32x4_t{tr_lo(lo), tr_hi(lo), tr_lo(hi), tr_hi(hi)};
    }
    o0 = E::mfma32(a[0], p[ks], o0);
    o1 = E::mfma32(a[1], p[ks], o1);
  }
}

// ---------------------------------------------------------------------------
// Tile loop over direct-to-LDS tiles. Step i:
//   direct loads K(i+1), V(i+1) and meta(i+1) into the other buffers
//   S = K(i) Q^T; bias / masks; online softmax; O += V(i)^T P^T
//   barrier (tile i+1 landed, everyone is done with tile i)
// Each K and V tile has two LDS buffers, distinct __shared__ objects named
// statically in each unrolled step, so the compiler can tell the direct loads
// from the operand reads and does not wait for the former before the latter.
// The policy P supplies, for virtual tile index i in [0, n):
//   int  key0(i)
//   void loadK(int i, uint16_t* Kt), loadV(int i, uint16_t* Vt)   direct loads
//   M    meta_ld(int i)                 per-tile metadata of tile i, loaded
//                                       early (before the tile's DMA) ...
//   void meta_st(M v, int slot)         ... and written to LDS slot i & 1
//                                       late, before the step's barrier
//   bool wave_active()                  the wave has a valid query row
//   static constexpr bool kAllActive    every tile is active for such waves
//   bool active(int i)                  the wave computes tile i
//   bool init(f32x16_t& s0, f32x16_t& s1, int i, int slot)   writes an additive
//                                       bias of tile i's scores into s0 / s1
//                                       (the QK MFMAs accumulate onto it), or
//                                       returns false (zero bias, s0 / s1
//                                       untouched)
//   bool modify(f32x16_t& s0, f32x16_t& s1, int i, int slot)   further bias /
//                                       masks; returns "exact" for softmax_exp
// ---------------------------------------------------------------------------

// Issues the loads and metadata of tiles 0 and 1 (K and V of both); call
// before the Q set-up so that their latency overlaps it, then attn_loop_db.
// With tile 1's V issued here rather than in the first step, the first
// step's barrier waits for no load issued just before it.
template <typename P>
__device__ inline void attn_pipe_start(P& pol, int n, uint16_t* __restrict__ K0,
                                       uint16_t* __restrict__ K1, uint16_t* __restrict__ V0,
                                       uint16_t* __restrict__ V1) {
  if (n <= 0) return;
  const auto m0 = pol.meta_ld(0);
  pol.loadK(0, K0);
  pol.loadV(0, V0);
  pol.meta_st(m0, 0);
  if (n > 1) {
    const auto m1 = pol.meta_ld(1);
    pol.loadK(1, K1);
    pol.loadV(1, V1);
    pol.meta_st(m1, 1);
  }
}

// FIXED: p = exp2(c s) with no running max (softmax_fixed: the caller bounds
// the scores or checks the result); otherwise the online softmax with running
// max m and scale c.
template <typename E, bool FIXED = false, typename P, typename RS>
__device__ inline void attn_loop_db(P& pol, uint16_t* __restrict__ K0, uint16_t* __restrict__ K1,
                                    uint16_t* __restrict__ V0, uint16_t* __restrict__ V1, int n,
                                    const u32x4_t (&qf)[4], float c, float& m, RS& l,
                                    f32x16_t& o0, f32x16_t& o1) {
  if (n <= 0) return;
  KOff ko;
  VOff vo;
  k_offsets(ko);
  v_offsets(vo);
  const bool wave_on = __builtin_amdgcn_readfirstlane((int)pol.wave_active()) != 0;
  tile_barrier();
  auto step = [&](int i, uint16_t* __restrict__ Kc, uint16_t* __restrict__ Vc,
                  uint16_t* __restrict__ Kn, uint16_t* __restrict__ Vn, int b) {
    ko.refresh();
    vo.refresh();
    // tile 1's K, V and meta were issued with tile 0; the next tile's
    // metadata is loaded before its DMA and written to LDS after this tile's
    // compute
    const bool meta_next = i + 1 < n && i > 0;
    const auto mn = pol.meta_ld(meta_next ? i + 1 : i);
    if (meta_next) {
      pol.loadK(i + 1, Kn);
      pol.loadV(i + 1, Vn);
    }
    if (wave_on && (P::kAllActive || __builtin_amdgcn_readfirstlane((int)pol.active(i)) != 0)) {
      f32x16_t s0, s1;
      if (pol.init(s0, s1, i, b))
        qk_tile_acc<E>(Kc, ko, qf, s0, s1);
      else
        qk_tile_sw<E>(Kc, ko, qf, s0, s1);
      const bool exact = pol.modify(s0, s1, i, b);
      u32x4_t p[4];
      if (FIXED)
        softmax_fixed<E>(s0, s1, p, l, c);
      else
        softmax_tile<E>(s0, s1, c, m, l, o0, o1, p, exact);
      pv_tile_sw<E>(Vc, vo, p, o0, o1);
    }
    if (meta_next) pol.meta_st(mn, b ^ 1);
    tile_barrier();
  };
  int i = 0;
  for (; i + 1 < n; i += 2) {
    step(i, K0, V0, K1, V1, 0);
    step(i + 1, K1, V1, K0, V0, 1);
  }
  if (i < n) step(i, K0, V0, K1, V1, 0);
}

// Rotates the Q operand in registers (non-interleaved RoPE halves): the lane's
// chunks ds and ds+2 hold d and d+32. cs = table row of this position:
// cs[2f] = cos(pos * inv_freq[f]), cs[2f+1] = sin(...), f < 32. The table
// values are fetched first (rope_q_fetch: they depend only on the position,
// so a kernel can issue them before anything else) and applied once q has
// landed (rope_q_apply).
// Returns the lane's sum of squares of q before the rotation (the rotation
// keeps each pair's norm; callers bounding |rotated q| allow for the rounding).
struct RopeQ {
  f32x4_t v[2][4];  // [dl][i2]: cos, sin of f = 16dl + 8h + 2*i2 (+1)
};

__device__ inline void rope_q_fetch(RopeQ& r, const float* __restrict__ cs) {
  const int h = (threadIdx.x & 63) >> 5;
#pragma unroll
  for (int dl = 0; dl < 2; ++dl) {
    const f32x4_t* t = reinterpret_cast<const f32x4_t*>(cs + 2 * (16 * dl + 8 * h));
#pragma unroll
    for (int i2 = 0; i2 < 4; ++i2) r.v[dl][i2] = t[i2];
  }
}

template <typename E>
__device__ inline float rope_q_apply(u32x4_t (&q)[4], const RopeQ& r) {
  float ss = 0.f;
#pragma unroll
  for (int dl = 0; dl < 2; ++dl) {
    float a[8], b[8];
    unpack8<E>(q[dl], a);
    unpack8<E>(q[dl + 2], b);
#pragma unroll
    for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(b[i], b[i], __builtin_fmaf(a[i], a[i], ss));
#pragma unroll
    for (int i2 = 0; i2 < 4; ++i2) {
      const f32x4_t v = r.v[dl][i2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int i = 2 * i2 + u;
        const float cs_ = v[2 * u], sn = v[2 * u + 1];
        const float x1 = a[i], x2 = b[i];
        a[i] = x1 * cs_ - x2 * sn;
        b[i] = x2 * cs_ + x1 * sn;
      }
    }
    q[dl] = pack8<E>(a);
    q[dl + 2] = pack8<E>(b);
  }
  return ss;
}

// cos/sin of one K row for one group of 8 rotary frequencies: the 8 (cos,
// sin) pairs of f = 8 grp .. 8 grp + 7 at the row's position.
struct RopeK {
  f32x4_t v[4];
};

__device__ inline void rope_k_fetch(RopeK& r, const float* __restrict__ table, int pos, int grp) {
  const f32x4_t* t = reinterpret_cast<const f32x4_t*>(table + (int64_t)pos * 64 + 16 * grp);
#pragma unroll
  for (int i = 0; i < 4; ++i) r.v[i] = t[i];
}

// One 16-byte half of a rotate-half pair, rotated and multiplied by `scale`
// before the one rounding to 16 bits: own holds dims d .. d + 7 of the row,
// partner the dims 32 away, with the partner negated for the first half
// (pneg = -1: x1 cos - x2 sin) and not for the second (+1: x2 cos + x1 sin).
template <typename E>
__device__ inline u32x4_t rope_k_half(u32x4_t own, u32x4_t partner, const RopeK& r, float pneg,
                                      float scale) {
  float x[8], p[8];
  unpack8<E>(own, x);
  unpack8<E>(partner, p);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float cs_ = r.v[i >> 1][2 * (i & 1)], sn = r.v[i >> 1][2 * (i & 1) + 1];
    x[i] = (x[i] * cs_ + (pneg * p[i]) * sn) * scale;
  }
  return pack8<E>(x);
}

}  // namespace vfk
