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

// Online softmax over one tile of raw scores (bias already added, -inf =
// masked), held in the two S^T accumulators s0 (keys 0..31) and s1 (32..63)
// and updated in place. c = softmax scale * log2(e), so p = exp2(c * (x - m))
// is one FMA and one exp2 per score. m: running reference max in raw units;
// l: this lane's partial row sum.
// exact: evaluate (x - m) * c instead of fma(x, c, -m*c). Needed when x may
// carry a huge finite additive mask (|x| ~ 1e30): the rounding of m*c alone
// would then exceed the whole exponent range, while x - m stays exact.
template <typename E>
__device__ inline void softmax_tile(f32x16_t& s0, f32x16_t& s1, float c, float& m, float& l,
                                    f32x16_t& o0, f32x16_t& o1,
                                    u32x4_t (&p)[4], bool exact = false) {
  // IEEE maximum (NaN-propagating) maps to v_maximum3_f32 without the
  // canonicalising moves fmaxf needs: 17 instructions for 32 scores.
  float ma = fmax_ieee(s0[0], s1[0]), mb = fmax_ieee(s0[1], s1[1]);
#pragma unroll
  for (int i = 2; i < 16; i += 2) {
    ma = fmax_ieee(fmax_ieee(ma, s0[i]), s1[i]);
    mb = fmax_ieee(fmax_ieee(mb, s0[i + 1]), s1[i + 1]);
  }
  const float m_new = half_swap_max(fmax_ieee(ma, mb), m);
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
  if (exact) {
    const float ms = (m == -INFINITY) ? 0.f : m;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      s0[i] = fast_exp2((s0[i] - ms) * c);
      s1[i] = fast_exp2((s1[i] - ms) * c);
    }
  } else {
    const float nmc = (m == -INFINITY) ? 0.f : -m * c;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      s0[i] = fast_exp2(__builtin_fmaf(s0[i], c, nmc));
      s1[i] = fast_exp2(__builtin_fmaf(s1[i], c, nmc));
    }
  }
  // pack to the 16-bit MFMA operand and sum the packed pairs: the row sum is
  // that of exactly the probabilities the PV product uses
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    p[0][j] = E::pack2(s0[2 * j], s0[2 * j + 1]);
    p[1][j] = E::pack2(s0[8 + 2 * j], s0[8 + 2 * j + 1]);
    p[2][j] = E::pack2(s1[2 * j], s1[2 * j + 1]);
    p[3][j] = E::pack2(s1[8 + 2 * j], s1[8 + 2 * j + 1]);
  }
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
#pragma unroll
    for (int j = 0; j < 4; ++j) l = E::dot2_ones(p[ks][j], l);
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
// Software-pipelined tile loop shared by the attention kernels.
//
// K/V tiles rotate through three LDS buffers so a single barrier per tile
// suffices, and each wave's instruction stream interleaves independent work:
//   commit tile t+1 (RoPE, V transpose, LDS stores)   | VALU  - overlaps PV(t-1)
//   issue global loads of tile t+2                    | VMEM
//   barrier
//   S(t+1) = K(t+1) Q^T                               | MFMA  - overlaps softmax(t)
//   softmax(t) (policy bias / masks first)             | VALU
//   O += V(t)^T P(t)^T                                 | MFMA
// The policy P supplies, for virtual tile index i in [0, n):
//   int  key0(i)                                     first key of the tile
//   void fetch(KVStage&, int i)                      global -> registers
//   void commit(KVStage&, int i, int slot, uint16_t* Ks, uint16_t* Vt)
//   bool active(int i)                               this wave computes tile i
//   bool modify(f32x16_t& s0, f32x16_t& s1, int i, int slot)
//                                                    add bias/masks in place;
//                                                    returns "exact" for softmax_tile
// ---------------------------------------------------------------------------
constexpr int kBufElems = kKsElems + kVtElems;   // u16 per LDS buffer
constexpr int kNumBufs = 3;

template <typename E, typename P>
__device__ inline void attn_pipeline(P& pol, uint16_t* __restrict__ lds, int n,
                                     const u32x4_t (&qf)[4], float c, float& m,
                                     float& l, f32x16_t& o0, f32x16_t& o1) {
  if (n <= 0) return;
  KVStage st;
  pol.fetch(st, 0);
  pol.commit(st, 0, 0, lds, lds + kKsElems);
  if (n > 1) pol.fetch(st, 1);
  __syncthreads();
  f32x16_t sa0, sa1, sb0, sb1;
  if (pol.active(0)) qk_tile<E>(lds, qf, sa0, sa1);

  auto step = [&](int i, int slot, f32x16_t& c0, f32x16_t& c1, f32x16_t& n0, f32x16_t& n1) {
    const int ns = slot == kNumBufs - 1 ? 0 : slot + 1;
    uint16_t* nK = lds + ns * kBufElems;
    if (i + 1 < n) {
      pol.commit(st, i + 1, ns, nK, nK + kKsElems);
      if (i + 2 < n) pol.fetch(st, i + 2);
    }
    __syncthreads();
    const bool act = pol.active(i);
    VOps vo;
    if (act) pv_load(lds + slot * kBufElems + kKsElems, vo);
    if (i + 1 < n && pol.active(i + 1)) qk_tile<E>(nK, qf, n0, n1);
    if (act) {
      const bool exact = pol.modify(c0, c1, i, slot);
      u32x4_t p[4];
      softmax_tile<E>(c0, c1, c, m, l, o0, o1, p, exact);
      pv_mfma<E>(vo, p, o0, o1);
    }
  };

  int slot = 0;
  for (int i = 0; i < n; i += 2) {
    step(i, slot, sa0, sa1, sb0, sb1);
    slot = slot == kNumBufs - 1 ? 0 : slot + 1;
    if (i + 1 < n) {
      step(i + 1, slot, sb0, sb1, sa0, sa1);
      slot = slot == kNumBufs - 1 ? 0 : slot + 1;
    }
  }
}

// Single-buffered tile loop with the same policy interface (slot is always
// 0): commit tile i, barrier, prefetch tile i+1 into registers, compute tile
// i, barrier. Fewer live registers than attn_pipeline (no second S tile, no
// early V operands), so more waves fit on each SIMD.
template <typename E, typename P>
__device__ inline void attn_loop(P& pol, uint16_t* __restrict__ lds, int n,
                                 const u32x4_t (&qf)[4], float c, float& m,
                                 float& l, f32x16_t& o0, f32x16_t& o1) {
  if (n <= 0) return;
  KVStage st;
  pol.fetch(st, 0);
  for (int i = 0; i < n; ++i) {
    pol.commit(st, i, 0, lds, lds + kKsElems);
    __syncthreads();
    if (i + 1 < n) pol.fetch(st, i + 1);
    if (pol.active(i)) {
      f32x16_t s0, s1;
      qk_tile<E>(lds, qf, s0, s1);
      // V operands are read while the softmax runs
      VOps vo;
      pv_load(lds + kKsElems, vo);
      __builtin_amdgcn_sched_barrier(0);
      const bool exact = pol.modify(s0, s1, i, 0);
      u32x4_t p[4];
      softmax_tile<E>(s0, s1, c, m, l, o0, o1, p, exact);
      pv_mfma<E>(vo, p, o0, o1);
    }
    __syncthreads();
  }
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
constexpr int kBuf2Elems = 2 * kTileElems;   // one K + one V tile

__device__ inline int swz(int row) { return (((row >> 1) & 1) << 2) | ((row >> 2) & 3); }

typedef __attribute__((address_space(3))) void lds_void_t;
typedef short s16x4_t __attribute__((ext_vector_type(4)));

// Loads tile rows [row0, row0 + 64) of a [rows x 64] matrix with row stride rs
// (elements) into LDS tile t; rows past nvalid read row nvalid - 1 instead
// (finite data whose scores are masked). Each wave moves two 1 KiB blocks.
__device__ inline void tile_load_direct(const uint16_t* __restrict__ base, int64_t rs, int row0,
                                        int nvalid, uint16_t* tile) {
  const int w = threadIdx.x >> 6, p = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int blk = 2 * w + j;  // rows 8*blk .. 8*blk + 7
    const int row = 8 * blk + (p >> 3);
    const int c = (p & 7) ^ swz(row);
    const int grow = min(row0 + row, nvalid - 1);
    __builtin_amdgcn_global_load_lds(base + (int64_t)grow * rs + 8 * c,
                                     (lds_void_t*)(tile + blk * 512), 16, 0, 0);
  }
}

// Waits for this wave's outstanding loads and LDS traffic, then joins the
// workgroup barrier: afterwards every direct-loaded tile is visible.
__device__ inline void tile_barrier() {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
}

// Lane offsets are kept in bytes and passed through an empty asm at each use
// so that the compiler adds the (constant) LDS buffer address in the
// instruction's offset field instead of keeping one address register per
// buffer live across the loop.
__device__ inline int lds_opaque(int x) {
  asm volatile("" : "+v"(x));
  return x;
}
template <typename T>
__device__ inline T lds_at(const uint16_t* base, int byte_off) {
  return *reinterpret_cast<const T*>(reinterpret_cast<const char*>(base) + byte_off);
}

// Byte offsets of the QK operand reads in a tile: lane (c, h) reads row c
// (+32 for the second key block, +4096 bytes), chunk 2*ds + h.
struct KOff {
  int o[4];
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
    const int off = lds_opaque(ko.o[ds]);
    a0[ds] = lds_at<u32x4_t>(Kt, off);
    a1[ds] = lds_at<u32x4_t>(Kt, off + 4096);
  }
  const f32x16_t z = {};
  s0 = E::mfma32(a0[0], q[0], z);
  s1 = E::mfma32(a1[0], q[0], z);
#pragma unroll
  for (int ds = 1; ds < 4; ++ds) {
    s0 = E::mfma32(a0[ds], q[ds], s0);
    s1 = E::mfma32(a1[ds], q[ds], s1);
  }
}

// Byte offsets of the transposed V reads: for 16-key step ks (+2048 bytes), d
// block db and key half hf (keys 16ks + 8hf + 4h + v, v = source-lane row),
// the lane addresses row 16ks + 8hf + 4h + v, columns d0 + 4r of its 16-lane
// group.
struct VOff {
  int o[2][2];  // [db][hf]
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
  int off[2][2];
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) off[db][hf] = lds_opaque(vo.o[db][hf]);
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

// K rows staged through registers when they must be rotated (RoPE) before
// reaching LDS: thread t holds row t>>2, chunks cp = t&3 and cp+4.
struct KStage {
  u32x4_t k0, k1;
};
__device__ inline void kstage_fetch(KStage& st, const uint16_t* __restrict__ base, int64_t rs,
                                    int row0, int nvalid) {
  const int t = threadIdx.x;
  const int row = min(row0 + (t >> 2), nvalid - 1);
  const uint16_t* g = base + (int64_t)row * rs + 8 * (t & 3);
  st.k0 = *reinterpret_cast<const u32x4_t*>(g);
  st.k1 = *reinterpret_cast<const u32x4_t*>(g + 32);
}
__device__ inline void kstage_store(const KStage& st, uint16_t* Kt) {
  const int t = threadIdx.x, row = t >> 2, cp = t & 3, f = swz(row);
  *reinterpret_cast<u32x4_t*>(Kt + row * 64 + 8 * (cp ^ f)) = st.k0;
  *reinterpret_cast<u32x4_t*>(Kt + row * 64 + 8 * ((cp + 4) ^ f)) = st.k1;
}

// ---------------------------------------------------------------------------
// Tile loop over direct-to-LDS tiles. Policy P supplies, for virtual tile i:
//   int  key0(i)
//   void load(int i, uint16_t* Kt, uint16_t* Vt)  issue direct loads (K too
//                                                  unless KSTAGED)
//   void kfetch(KStage&, int i) / void kcommit(KStage&, int i, uint16_t* Kt)
//                                                  (KSTAGED: registers, rotate,
//                                                  store)
//   void meta(int i, int slot)                     per-tile LDS metadata
//   bool active(int i)
//   bool modify(f32x16_t& s0, f32x16_t& s1, int i, int slot)
// LDS: buf0 and buf1 (distinct __shared__ arrays) of kBuf2Elems each, K tile
// then V tile.
// ---------------------------------------------------------------------------
template <typename E, bool KSTAGED, typename P>
__device__ inline void attn_loop_direct(P& pol, uint16_t* __restrict__ buf0,
                                        uint16_t* __restrict__ buf1, int n,
                                        const u32x4_t (&qf)[4], float c, float& m, float& l,
                                        f32x16_t& o0, f32x16_t& o1) {
  if (n <= 0) return;
  KOff ko;
  VOff vo;
  k_offsets(ko);
  v_offsets(vo);
  KStage ks;
  pol.load(0, buf0, buf0 + kTileElems);
  if (KSTAGED) {
    pol.kfetch(ks, 0);
    pol.kcommit(ks, 0, buf0);
  }
  pol.meta(0, 0);
  tile_barrier();
  // buf0 and buf1 are distinct LDS objects and each step names them
  // statically, so the compiler can tell that the direct loads into nxt do not
  // alias the reads of cur and does not wait for them before computing.
  auto step = [&](int i, uint16_t* __restrict__ cur, uint16_t* __restrict__ nxt, int b) {
    if (i + 1 < n) {
      pol.load(i + 1, nxt, nxt + kTileElems);
      if (KSTAGED) pol.kfetch(ks, i + 1);
      pol.meta(i + 1, b ^ 1);
    }
    if (pol.active(i)) {
      f32x16_t s0, s1;
      qk_tile_sw<E>(cur, ko, qf, s0, s1);
      const bool exact = pol.modify(s0, s1, i, b);
      u32x4_t p[4];
      softmax_tile<E>(s0, s1, c, m, l, o0, o1, p, exact);
      pv_tile_sw<E>(cur + kTileElems, vo, p, o0, o1);
    }
    if (KSTAGED && i + 1 < n) pol.kcommit(ks, i + 1, nxt);
    tile_barrier();
  };
  int i = 0;
  for (; i + 1 < n; i += 2) {
    step(i, buf0, buf1, 0);
    step(i + 1, buf1, buf0, 1);
  }
  if (i < n) step(i, buf0, buf1, 0);
}

// Rotates the Q operand in registers (non-interleaved RoPE halves): the lane's
// chunks ds and ds+2 hold d and d+32. cs = table row of this position:
// cs[2f] = cos(pos * inv_freq[f]), cs[2f+1] = sin(...), f < 32.
template <typename E>
__device__ inline void rope_q_table(u32x4_t (&q)[4], const float* __restrict__ cs) {
  const int h = (threadIdx.x & 63) >> 5;
#pragma unroll
  for (int dl = 0; dl < 2; ++dl) {
    float a[8], b[8];
    unpack8<E>(q[dl], a);
    unpack8<E>(q[dl + 2], b);
    const f32x4_t* t = reinterpret_cast<const f32x4_t*>(cs + 2 * (16 * dl + 8 * h));
#pragma unroll
    for (int i2 = 0; i2 < 4; ++i2) {
      const f32x4_t v = t[i2];  // cos, sin of f = 16dl + 8h + 2*i2 (+1)
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
}

// Rotates a staged K tile row (thread t holds key t>>2, d chunks cp and cp+4
// with cp = t&3); cs8 = the 8 (cos, sin) pairs of f = 8*cp .. 8*cp+7 for the
// row's position, as loaded by rope_k_fetch.
struct RopeK {
  f32x4_t v[4];
};

__device__ inline void rope_k_fetch(RopeK& r, const float* __restrict__ table, int pos, bool valid) {
  const int cp = threadIdx.x & 3;
  const f32x4_t z = {0.f, 0.f, 0.f, 0.f};
  const f32x4_t* t = reinterpret_cast<const f32x4_t*>(table + (int64_t)pos * 64 + 16 * cp);
#pragma unroll
  for (int i = 0; i < 4; ++i) r.v[i] = valid ? t[i] : z;
}

template <typename E>
__device__ inline void rope_k_apply(u32x4_t& k0, u32x4_t& k1, const RopeK& r) {
  float a[8], b[8];
  unpack8<E>(k0, a);
  unpack8<E>(k1, b);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float cs_ = r.v[i >> 1][2 * (i & 1)], sn = r.v[i >> 1][2 * (i & 1) + 1];
    const float x1 = a[i], x2 = b[i];
    a[i] = x1 * cs_ - x2 * sn;
    b[i] = x2 * cs_ + x1 * sn;
  }
  k0 = pack8<E>(a);
  k1 = pack8<E>(b);
}

}  // namespace vfk
