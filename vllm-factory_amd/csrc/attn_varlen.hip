// Varlen (packed-sequence) bidirectional attention for ModernBERT, gfx950.
//
// Replaces F.scaled_dot_product_attention over the whole packed stream with
// dense [T, T] block-diagonal / sliding-window masks
// (models/modernbert/modernbert_encoder.py:236-255, :491-550): work is cut per
// sequence by cu_seqlens, so cross-sequence pairs are never computed, and a
// sliding-window layer only visits the key tiles its rows can see.
// RoPE (non-interleaved halves) uses an fp32 cos/sin table (vfk_rope_table,
// the HF ModernBertRotaryEmbedding values). K is rotated once by a pre-pass
// into a head-major workspace [H][T][64] (the role of the reference's separate
// rotary step, kernels/fused_rope_global.py); Q is rotated in registers by the
// attention kernel as it loads its rows.
//
// With RoPE the pre-pass also folds c = softmax_scale * log2(e) into K before
// its one rounding to 16 bits, so the QK^T MFMA yields scores in log2 units,
// and records the largest row norm of each 16 rows of every 64-key tile (four
// partial maxima per tile). From |q| and those
// norms each wave bounds |score| <= |q| max|k| before its loop; where the
// bound stays within log2(kPMax) for all its rows, p = exp2(score) is taken
// directly (no running max, no rescale: it can neither overflow the fp32
// accumulators nor underflow the 16-bit P operand), otherwise the online
// softmax with a running max runs as without RoPE.
#include <math.h>

#include <algorithm>
#include <type_traits>

#include "attn_core.h"
#include "launch_util.h"

namespace vfk {

struct VarlenArgs {
  const void* q; const void* k; const void* v; void* o;
  int64_t qs[2], ks[2], vs[2], os[2];  // [T,H,D] strides of T and H (D stride 1)
  const int32_t* cu; int nseq; int nqt; int H; int window;
  float c2;                 // softmax scale * log2(e)
  const float* rope;        // optional [positions][32][2] (cos, sin) table
  const uint8_t* key_valid; // optional, [T]
  const void* kr;           // RoPE: rotated, scaled K, head-major [H][T][64]
  float* kmax;              // RoPE: max row norm of each 16 rows of each key tile
                            // [H][nseq][nkt][4], or
                            // (kblk32) of each 32-token block of the stream [H][ceil(T / 32)]
  int nkt;                  // key tiles per sequence slot: ceil(max_seqlen / 64)
  int kblk32;               // kmax holds 32-token stream blocks (K from the fused projection)
  int maxlen;               // max_seqlen: longer sequences are cut there, their
                            // rows past it written as zeros
  int64_t T;
};

// cos/sin table of HF rotary embeddings: row p, f < 32:
// (cos(p * inv_freq[f]), sin(p * inv_freq[f])) with fp32 p * inv_freq[f].
struct RopeTableArgs {
  float* out;
  int npos;
  float inv_freq[32];
};

__global__ __launch_bounds__(256) void rope_table_kernel(RopeTableArgs a) {
  const int e = blockIdx.x * 256 + threadIdx.x;
  if (e >= a.npos * 32) return;
  const int p = e >> 5, f = e & 31;
  const float ang = (float)p * a.inv_freq[f];
  float sn, cs;
  sincosf(ang, &sn, &cs);
  f32x2_t v = {cs, sn};
  reinterpret_cast<f32x2_t*>(a.out)[e] = v;
}

// Half-width of the relative-position penalty table used on tiles that cut
// through the sliding window: entry kPenOff + (key - row) is 0 inside the
// window and -inf outside, for |key - row| < kPenOff.
constexpr int kPenOff = 192;
constexpr int kPenLen = 2 * kPenOff;

// K rotation pre-pass: block (s, g, hg) rotates rows [16 g, 16 g + 16) of
// sequence s for heads [2 NPAIR hg, 2 NPAIR hg + 2 NPAIR). Each 16-lane group
// owns one row and covers two heads per load: lane i of a head's 8 holds 16
// bytes of its 128-byte row, chunk i (i < 4) or 11 - i (i >= 4), so that every
// load and store instruction moves whole 128-byte lines (half-line pieces
// held the pass ~30 % below the copy rate), and the rotate-half partners
// (dims d and d + 32) sit in lanes i and 7 - i, swapped by a DPP
// row_half_mirror. All loads are issued before any store, with head indices
// clamped so that the loads are unconditional. The rows are stored multiplied
// by c2 = softmax_scale * log2(e); the largest Euclidean norm of the block's
// stored rows per head goes to kmax[h][s][kt][g & 3] (kt = g / 4, four
// partial maxima per 64-key tile), and the slots of a live tile that lie past
// the sequence end get 0.
constexpr int kPackRows = 16;

// DPP row_half_mirror: the value of lane 7 - i of the lane's group of 8.
__device__ inline uint32_t mirror8(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false);
}

// max over the lanes l, l ^ 16, l ^ 32, l ^ 48 (the 4 rows of a wave)
__device__ inline float rows_max4(float v) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_int(v), __float_as_int(v), false, false);
  v = fmaxf(__int_as_float(r[0]), __int_as_float(r[1]));
  r = __builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false, false);
  return fmaxf(__int_as_float(r[0]), __int_as_float(r[1]));
}

__device__ inline float wave_max(float v) { return group_max<64>(v); }
__device__ inline float max4(f32x4_t v) { return fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3])); }

template <typename E>
__device__ inline float sumsq8(u32x4_t v) {
  float f[8];
  unpack8<E>(v, f);
  float r = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) r = __builtin_fmaf(f[i], f[i], r);
  return r;
}

template <typename E, int NPAIR>
__global__ __launch_bounds__(256) void rope_k_pack_kernel(VarlenArgs a, int ngrp, int nhg) {
  __shared__ float part[4][2 * NPAIR];
  // blocks (s, g, head group) in that order, each XCD a contiguous share:
  // sequence s is rotated on the XCD whose attention workgroups read it
  // (the attention's items are dealt the same way), so those find its rows
  // in their L2
  const int pb = xcd_remap(blockIdx.x, gridDim.x);
  const int hg = pb % nhg;
  const int g = (pb / nhg) % ngrp;
  const int s = pb / (nhg * ngrp);
  const int tok0 = a.cu[s];
  const int nfull = a.cu[s + 1] - tok0;
  const int n = min(nfull, a.maxlen);
  const int h0 = hg * 2 * NPAIR;
  const int t = threadIdx.x;
  if (g == ngrp - 1 && nfull > n) {
    // a sequence longer than max_seqlen: the attention computes its first
    // max_seqlen rows; the rest of its output rows become zeros here
    for (int u = 0; u < 2 * NPAIR && h0 + u < a.H; ++u)
      zero_rows_d64(reinterpret_cast<uint16_t*>(a.o) + (int64_t)tok0 * a.os[0] + (h0 + u) * a.os[1],
                    a.os[0], n, nfull);
  }
  if (g * kPackRows >= n) {  // uniform: no row of the sequence in this block
    if ((g >> 2) * 64 < n && t < 2 * NPAIR && h0 + t < a.H)
      a.kmax[(((int64_t)(h0 + t) * a.nseq + s) * a.nkt + (g >> 2)) * 4 + (g & 3)] = 0.f;
    return;
  }
  const int row = g * kPackRows + (t >> 4);
  const bool valid = row < n;
  const int rr = valid ? row : g * kPackRows;  // tail rows load a valid row, store nothing
  const int l = t & 15, i8 = l & 7, lw = t & 63, w = t >> 6;
  const int ch = i8 < 4 ? i8 : 11 - i8;  // the lane's 16-byte chunk of the head row
  RopeK rk;
  rope_k_fetch(rk, a.rope, rr, ch & 3);
  const uint16_t* src = reinterpret_cast<const uint16_t*>(a.k) + (int64_t)(tok0 + rr) * a.ks[0] + 8 * ch;
  u32x4_t kv[NPAIR];
#pragma unroll
  for (int j = 0; j < NPAIR; ++j) {
    const int h = min(h0 + 2 * j + (l >> 3), a.H - 1);
    // non-temporal: K is read once here (the attention reads the rotated copy)
    kv[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(src + (int64_t)h * a.ks[1]));
  }
  uint16_t* dst = const_cast<uint16_t*>(reinterpret_cast<const uint16_t*>(a.kr)) +
                  (int64_t)(tok0 + row) * 64 + 8 * ch;
  const int64_t hs = (int64_t)a.T * 64;
  const float pneg = i8 < 4 ? -1.f : 1.f;
#pragma unroll
  for (int j = 0; j < NPAIR; ++j) {
    const int h = h0 + 2 * j + (l >> 3);
    u32x4_t pv;
#pragma unroll
    for (int e = 0; e < 4; ++e) pv[e] = mirror8(kv[j][e]);
    const u32x4_t r = rope_k_half<E>(kv[j], pv, rk, pneg, a.c2);
    float nrm = 0.f;
    if (valid && h < a.H) {
      *reinterpret_cast<u32x4_t*>(dst + h * hs) = r;
      nrm = sumsq8<E>(r);
    }
    // squared row norm (the head row's 8 lanes), then the max over the wave's rows
    nrm = rows_max4(group_sum<8>(nrm));
    if ((lw & ~8) == 0) part[w][2 * j + (lw >> 3)] = nrm;
  }
  __syncthreads();
  if (t < 2 * NPAIR && h0 + t < a.H) {
    const float m = fmaxf(fmaxf(part[0][t], part[1][t]), fmaxf(part[2][t], part[3][t]));
    a.kmax[(((int64_t)(h0 + t) * a.nseq + s) * a.nkt + (g >> 2)) * 4 + (g & 3)] = sqrtf(m);
  }
}

// Output rows past max_seqlen of every (sequence, head), as zeros: block
// (s, h). Launched by the attention over the fused projection's K, where no
// pre-pass runs.
__global__ __launch_bounds__(256) void zero_cut_rows_kernel(VarlenArgs a) {
  const int s = blockIdx.x / a.H, h = blockIdx.x % a.H;
  const int tok0 = a.cu[s];
  const int nfull = a.cu[s + 1] - tok0;
  if (nfull > a.maxlen)
    zero_rows_d64(reinterpret_cast<uint16_t*>(a.o) + (int64_t)tok0 * a.os[0] + h * a.os[1],
                  a.os[0], a.maxlen, nfull);
}

template <typename E, bool ROPE, bool LOCAL, bool KVALID>
struct VarlenPolicy {
  const VarlenArgs* a;
  TileSrc ksrc, vsrc;
  int tok0, n, kt0, t, hl, qrow, wq_lo, wq_hi, window, tail0;
  float* kmask;  // KVALID: [2][kBN], 0 or -inf per key of the tile in slot i & 1;
                 // else [kBN]: the mask of the sequence's last, partial tile
  int* kflag;    // KVALID: [2], any key of the tile masked
  const float* pen;

  __device__ int key0(int i) const { return (kt0 + i) * kBN; }
  __device__ void loadK(int i, uint16_t* Kt) { tile_load_buf(ksrc, key0(i), Kt); }
  __device__ void loadV(int i, uint16_t* Vt) { tile_load_buf(vsrc, key0(i), Vt); }
  // wave 0, one key per lane: key_valid of the tile's keys
  __device__ bool meta_ld(int i) const {
    if (!KVALID || t >= kBN) return true;
    const int j = key0(i) + t;
    return j < n && a->key_valid[tok0 + j] != 0;
  }
  __device__ void meta_st(bool ok, int slot) {
    if (!KVALID || t >= kBN) return;
    kmask[slot * kBN + t] = ok ? 0.f : -INFINITY;
    const unsigned long long dead = __builtin_amdgcn_ballot_w64(!ok);
    if (t == 0) kflag[slot] = dead != 0ull;
  }
  static constexpr bool kAllActive = !LOCAL;
  __device__ bool wave_active() const { return wq_lo < n; }
  __device__ bool active(int i) const {
    if (wq_lo >= n) return false;
    if (!LOCAL) return true;
    const int k0 = key0(i);
    return k0 <= wq_hi + window && k0 + kBN - 1 >= wq_lo - window;
  }
  // the tile cuts through the sliding window of some row of the wave
  __device__ bool pen_tile(int k0) const {
    return LOCAL && (wq_hi - k0 > window || k0 + kBN - 1 - wq_lo > window);
  }
  // 0 / -inf per key of tile i (key_valid, or the partial last tile), or null
  __device__ const float* key_tab(int i, int slot) const {
    if (KVALID) return kflag[slot] ? kmask + slot * kBN + 4 * hl : nullptr;
    return key0(i) == tail0 ? kmask + 4 * hl : nullptr;
  }
  // one of the tile's additive terms (window penalty, else the key mask)
  // enters as the QK MFMAs' accumulator input; modify adds the other
  __device__ bool init(f32x16_t& s0, f32x16_t& s1, int i, int slot) const {
    const int k0 = key0(i);
    if (pen_tile(k0)) {
      // entry kPenOff + key - qrow, key = k0 + 4*hl + x_key(e, 0)
      load_by_key(s0, s1, pen + (kPenOff + k0 + 4 * hl - qrow));
      return true;
    }
    const float* kt = key_tab(i, slot);
    if (kt) {
      load_by_key(s0, s1, kt);
      return true;
    }
    return false;
  }
  __device__ bool modify(f32x16_t& s0, f32x16_t& s1, int i, int slot) const {
    if (pen_tile(key0(i))) {
      const float* kt = key_tab(i, slot);
      if (kt) add_by_key(s0, s1, kt);
    }
    return false;
  }
};

// LDS of one workgroup of the 16-bit kernels.
template <bool LOCAL>
struct VarlenLds {
  uint16_t* K0; uint16_t* K1; uint16_t* V0; uint16_t* V1;
  float* kmask; int* kflag; float* pen;
};

// Loads of an item that need only its (sequence, head, query tile) indices:
// the table row of the Q rotation and the key norms of the tiles the
// workgroup may visit. Issued before the sequence offsets (cu_seqlens)
// arrive, they keep the item's set-up to two memory round trips (kernel
// arguments and offsets, then Q and the first K/V tiles) instead of three.
template <bool ROPE, bool LOCAL>
__device__ inline void varlen_item_prefetch(const VarlenArgs& a, int s, int h, int qt, RopeQ& rq,
                                            f32x4_t& kx) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int q0 = qt * kBM;
  const int qrow = q0 + w * 32 + (lane & 31);
  const int kt_lo = LOCAL ? max(0, q0 - a.window) / kBN : 0;
  kx = f32x4_t{0.f, 0.f, 0.f, 0.f};
  if (ROPE) {
    // rows past the sequence end rotate zeros: any table row will do
    rope_q_fetch(rq, a.rope + (int64_t)min(qrow, a.maxlen - 1) * 64);
    // lanes past the last tile slot load slot nkt - 1 (no branch: a divergent
    // one here would make the offsets loaded next vector loads)
    if (!a.kblk32)
      kx = *reinterpret_cast<const f32x4_t*>(
          a.kmax + (((int64_t)h * a.nseq + s) * a.nkt + min(kt_lo + lane, a.nkt - 1)) * 4);
  }
}

// The same loads in two steps: the addresses (they need the kernel
// arguments, not the sequence offsets), then the loads themselves.
template <bool ROPE, bool LOCAL>
struct ItemPrefetch {
  const float* tab;  // the lane's Q-rotation table row
  const float* km;   // the lane's key-norm slot (the tile's 4 partial maxima)
  __device__ ItemPrefetch(const VarlenArgs& a, int s, int h, int qt) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int q0 = qt * kBM;
    const int qrow = q0 + w * 32 + (lane & 31);
    const int kt_lo = LOCAL ? max(0, q0 - a.window) / kBN : 0;
    tab = ROPE ? a.rope + (int64_t)min(qrow, a.maxlen - 1) * 64 : nullptr;
    km = (ROPE && !a.kblk32)
             ? a.kmax + (((int64_t)h * a.nseq + s) * a.nkt + min(kt_lo + lane, a.nkt - 1)) * 4
             : nullptr;
  }
  __device__ void issue(RopeQ& rq, f32x4_t& kx) const {
    kx = f32x4_t{0.f, 0.f, 0.f, 0.f};
    if (ROPE) {
      rope_q_fetch(rq, tab);
      if (km) kx = *reinterpret_cast<const f32x4_t*>(km);
    }
  }
};

// One item: query rows q0 .. q0 + 127 (qt = q0 / 128) of head h of sequence
// s (rows tok0 .. tok0 + n - 1 of the stream), n > q0, against every key of
// the sequence the layer lets them see; rq / kx4 as varlen_item_prefetch
// left them. Leaves the item's output rows written and every LDS buffer free
// once all waves have passed a barrier.
template <typename E, bool ROPE, bool LOCAL, bool KVALID>
__device__ inline void varlen_item(const VarlenArgs& a, const VarlenLds<LOCAL>& L, int s, int h,
                                   int qt, int tok0, int n, const RopeQ& rq, f32x4_t kx4) {
  const int t = threadIdx.x, lane = t & 63, w = t >> 6, hl = lane >> 5;
  const int q0 = qt * kBM;
  const int wq_lo = q0 + w * 32;
  const int qrow = wq_lo + (lane & 31);
  const uint16_t* Qp = reinterpret_cast<const uint16_t*>(a.q) + (int64_t)tok0 * a.qs[0] + h * a.qs[1];

  // key tiles of the workgroup (sequence-relative)
  int klo = 0, khi = n;
  if (LOCAL) {
    klo = max(0, q0 - a.window);
    khi = min(n, q0 + kBM + a.window);
    for (int e = t; e < kPenLen; e += 256) {
      const int d = e - kPenOff;
      L.pen[e] = (d <= a.window && d >= -a.window) ? 0.f : -INFINITY;
    }
  }
  const int kt_begin = klo / kBN;
  const int kt_end = (khi + kBN - 1) / kBN;
  // start of the sequence's partial last key tile (none: -1)
  const int tail0 = (n % kBN) ? (n / kBN) * kBN : -1;
  if (!KVALID && t < kBN) L.kmask[t] = (tail0 + t < n) ? 0.f : -INFINITY;

  const bool qvalid = qrow < n;

  VarlenPolicy<E, ROPE, LOCAL, KVALID> pol;
  pol.a = &a;
  if (ROPE)
    tile_src_init(pol.ksrc, reinterpret_cast<const uint16_t*>(a.kr) + ((int64_t)h * a.T + tok0) * 64,
                  64, n);
  else
    tile_src_init(pol.ksrc, reinterpret_cast<const uint16_t*>(a.k) + (int64_t)tok0 * a.ks[0] + h * a.ks[1],
                  (int)a.ks[0], n);
  tile_src_init(pol.vsrc, reinterpret_cast<const uint16_t*>(a.v) + (int64_t)tok0 * a.vs[0] + h * a.vs[1],
                (int)a.vs[0], n);
  pol.tok0 = tok0; pol.n = n; pol.kt0 = kt_begin; pol.t = t; pol.hl = hl; pol.qrow = qrow;
  pol.wq_lo = wq_lo; pol.wq_hi = min(wq_lo + 31, n - 1); pol.window = a.window; pol.tail0 = tail0;
  pol.kmask = L.kmask; pol.kflag = L.kflag; pol.pen = L.pen;

  attn_pipe_start(pol, kt_end - kt_begin, L.K0, L.K1, L.V0, L.V1);

  u32x4_t qf[4];
  load_q(qf, Qp + (int64_t)qrow * a.qs[0], qvalid);
  // q2: the lane's share of |q|^2 before the rotation
  float q2 = 0.f;
  if (ROPE) q2 = rope_q_apply<E>(qf, rq);

  float m = -INFINITY;
  // row sums on the matrix core where the 8 extra registers fit (global
  // layers); the sliding-window variants would spill and sum the same
  // rounded weights by packed dots
  typename std::conditional<LOCAL, RowSumDot<E>, RowSumMfma<E>>::type l;
  f32x16_t o0 = {}, o1 = {};
  const int ntiles = kt_end - kt_begin;
  if (ROPE) {
    // |score| <= |q| max|k| over the workgroup's key tiles (scores are in
    // log2 units: K carries c2); the margin covers the fp32 norms and the
    // MFMA's fp32 accumulation
    // the 4 partial maxima of the lane's tile, reduced only here so that the
    // prologue never waits for their load
    float kx = max4(kx4);
    if (a.kblk32) {
      // (kx is 0 here: no norms were prefetched) stream blocks covering the workgroup's keys (a superset: still a bound)
      const float* km = a.kmax + (int64_t)h * ((a.T + 31) >> 5);
      const int b0 = (tok0 + kt_begin * kBN) >> 5, b1 = (tok0 + min(kt_end * kBN, n) - 1) >> 5;
      for (int j = b0 + lane; j <= b1; j += 64) kx = fmaxf(kx, km[j]);
    } else {
      // the prefetched norms of tiles kt_begin + lane, kept where inside the
      // workgroup's range; tiles past the first 64 (sequences > 4096) here
      if (kt_begin + lane >= kt_end) kx = 0.f;
      const f32x4_t* km = reinterpret_cast<const f32x4_t*>(a.kmax) + ((int64_t)h * a.nseq + s) * a.nkt;
      for (int j = kt_begin + 64 + lane; j < kt_end; j += 64) kx = fmaxf(kx, max4(km[j]));
    }
    kx = wave_max(kx);
    // the rotation keeps |q|; rounding the rotated q to 16 bits grows each
    // element, and so |q|, by at most 2^-8 relative
    q2 = half_swap_sum(q2);
    const float ub = sqrtf(q2) * 1.00390625f * kx * 1.0078125f + 0.0625f;
    if (__builtin_amdgcn_ballot_w64(ub > E::kLog2PMax) == 0ull)
      attn_loop_db<E, true>(pol, L.K0, L.K1, L.V0, L.V1, ntiles, qf, 1.f, m, l, o0, o1);
    else
      attn_loop_db<E, false>(pol, L.K0, L.K1, L.V0, L.V1, ntiles, qf, 1.f, m, l, o0, o1);
  } else {
    attn_loop_db<E, false>(pol, L.K0, L.K1, L.V0, L.V1, ntiles, qf, a.c2, m, l, o0, o1);
  }

  const float l_tot = l.total();
  // whole-row stores through this wave's half of K0 / K1 (free after the
  // loop's last barrier; a workgroup with no key tile never touched them)
  uint16_t* ob = reinterpret_cast<uint16_t*>(a.o) + (int64_t)tok0 * a.os[0] + h * a.os[1];
  store_out_rows<E>((w < 2 ? L.K0 : L.K1) + (w & 1) * 2048, o0, o1, l_tot,
                    [&](int r) { return ob + (int64_t)(wq_lo + r) * a.os[0]; },
                    [&](int r) { return wq_lo + r < n; });
}

// One workgroup per (sequence, head, query tile) work item, four workgroups
// per CU (128 VGPRs). The sliding-window kernels with a key mask fit that
// with their row sums as packed dots: 1 (RoPE) or 2 registers are spilled
// outside the tile loops, and the 22-layer ModernBERT forward at 163 736
// tokens runs 0.15 ms faster than at three workgroups per CU.
template <typename E, bool ROPE, bool LOCAL, bool KVALID>
__global__ __launch_bounds__(256, 4) void varlen_fwd_kernel(VarlenArgs a) {
  __shared__ __align__(16) uint16_t K0[kTileElems];
  __shared__ __align__(16) uint16_t K1[kTileElems];
  __shared__ __align__(16) uint16_t V0[kTileElems];
  __shared__ __align__(16) uint16_t V1[kTileElems];
  __shared__ float kmask[2 * kBN];
  __shared__ int kflag[2];
  __shared__ float pen[LOCAL ? kPenLen : 1];

  const int work = xcd_remap(blockIdx.x, gridDim.x);
  const int qt = work % a.nqt;
  const int h = (work / a.nqt) % a.H;
  const int s = work / (a.nqt * a.H);
  // The loads that need only the item's indices (the Q-rotation table row
  // and the key norms of the tiles the workgroup may visit) go out with the
  // sequence offsets, before anything waits on either, so the set-up is two
  // memory round trips (offsets, then Q and the first K/V tiles) rather than
  // three. Global layers request the offsets first, with the other addresses
  // formed beforehand so that no wait for the kernel arguments falls between
  // the requests (an A/B on config 2: global call 142-144 against 145-146 us
  // with the offsets requested last); the sliding-window kernels keep the
  // offsets last, which holds them at 128 VGPRs without a spill.
  RopeQ rq;
  f32x4_t kx;
  int tok0, nfull;
  if (LOCAL) {
    varlen_item_prefetch<ROPE, LOCAL>(a, s, h, qt, rq, kx);
    tok0 = a.cu[s];
    nfull = a.cu[s + 1] - tok0;
  } else {
    const ItemPrefetch<ROPE, LOCAL> pre(a, s, h, qt);
    __builtin_amdgcn_sched_barrier(0);
    tok0 = a.cu[s];
    nfull = a.cu[s + 1] - tok0;
    __builtin_amdgcn_sched_barrier(0);
    pre.issue(rq, kx);
  }
  const int n = min(nfull, a.maxlen);
  // rows past max_seqlen are written as zeros: without RoPE by the last
  // query tile, with RoPE by the K pre-pass (or, after the fused projection,
  // by zero_cut_rows_kernel), which keeps the RoPE kernels' registers free
  if (qt * kBM >= n) {  // whole workgroup: uniform exit
    if (!ROPE && qt == a.nqt - 1 && nfull > n)
      zero_rows_d64(reinterpret_cast<uint16_t*>(a.o) + (int64_t)tok0 * a.os[0] + h * a.os[1],
                    a.os[0], n, nfull);
    return;
  }
  const VarlenLds<LOCAL> L = {K0, K1, V0, V1, kmask, kflag, pen};
  varlen_item<E, ROPE, LOCAL, KVALID>(a, L, s, h, qt, tok0, n, rq, kx);
  if (!ROPE && qt == a.nqt - 1 && nfull > n)
    zero_rows_d64(reinterpret_cast<uint16_t*>(a.o) + (int64_t)tok0 * a.os[0] + h * a.os[1],
                  a.os[0], n, nfull);
}

// fp32: one thread per query row, exact fp32 arithmetic, accurate sin/cos.
__global__ __launch_bounds__(64) void varlen_fwd_f32_kernel(VarlenArgs a) {
  __shared__ float Kt[64][kHD + 1];
  __shared__ float Vt32[64][kHD + 1];
  const int nqt64 = a.nqt * 2;
  const int qt = blockIdx.x % nqt64;
  const int h = (blockIdx.x / nqt64) % a.H;
  const int s = blockIdx.x / (nqt64 * a.H);
  const int tok0 = a.cu[s];
  const int nfull = a.cu[s + 1] - tok0;
  const int n = min(nfull, a.maxlen);
  const int q0 = qt * 64;
  if (qt == nqt64 - 1 && nfull > n) {  // rows past max_seqlen: zeros
    float* ob = reinterpret_cast<float*>(a.o) + (int64_t)tok0 * a.os[0] + h * a.os[1];
    for (int e = threadIdx.x; e < (nfull - n) * kHD; e += 64)
      ob[(int64_t)(n + e / kHD) * a.os[0] + e % kHD] = 0.f;
  }
  if (q0 >= n) return;
  const int qrow = q0 + threadIdx.x;
  const bool qvalid = qrow < n;
  const float* Qp = reinterpret_cast<const float*>(a.q) + (int64_t)tok0 * a.qs[0] + h * a.qs[1];
  const float* Kp = reinterpret_cast<const float*>(a.k) + (int64_t)tok0 * a.ks[0] + h * a.ks[1];
  const float* Vp = reinterpret_cast<const float*>(a.v) + (int64_t)tok0 * a.vs[0] + h * a.vs[1];
  float qv[kHD], acc[kHD];
#pragma unroll
  for (int d = 0; d < kHD; ++d) {
    qv[d] = qvalid ? Qp[(int64_t)qrow * a.qs[0] + d] : 0.f;
    acc[d] = 0.f;
  }
  if (a.rope && qvalid) {
#pragma unroll
    for (int f = 0; f < 32; ++f) {
      const float cs = a.rope[(int64_t)qrow * 64 + 2 * f], sn = a.rope[(int64_t)qrow * 64 + 2 * f + 1];
      const float x1 = qv[f], x2 = qv[f + 32];
      qv[f] = x1 * cs - x2 * sn;
      qv[f + 32] = x2 * cs + x1 * sn;
    }
  }
  float m = -INFINITY, l = 0.f;
  int klo = 0, khi = n;
  if (a.window >= 0) {
    klo = max(0, q0 - a.window);
    khi = min(n, q0 + 64 + a.window);
  }
  for (int key0 = klo; key0 < khi; key0 += 64) {
    __syncthreads();
    for (int e = threadIdx.x; e < 64 * 32; e += 64) {
      const int r = e / 32, f = e % 32;
      const int j = key0 + r;
      float k1 = 0.f, k2 = 0.f, v1 = 0.f, v2 = 0.f;
      if (j < khi) {
        k1 = Kp[(int64_t)j * a.ks[0] + f];
        k2 = Kp[(int64_t)j * a.ks[0] + f + 32];
        v1 = Vp[(int64_t)j * a.vs[0] + f];
        v2 = Vp[(int64_t)j * a.vs[0] + f + 32];
        if (a.rope) {
          const float cs = a.rope[(int64_t)j * 64 + 2 * f], sn = a.rope[(int64_t)j * 64 + 2 * f + 1];
          const float x1 = k1, x2 = k2;
          k1 = x1 * cs - x2 * sn;
          k2 = x2 * cs + x1 * sn;
        }
      }
      Kt[r][f] = k1; Kt[r][f + 32] = k2;
      Vt32[r][f] = v1; Vt32[r][f + 32] = v2;
    }
    __syncthreads();
    const int nk = min(64, khi - key0);
    for (int r = 0; r < nk; ++r) {
      const int j = key0 + r;
      if (a.window >= 0 && (j - qrow > a.window || qrow - j > a.window)) continue;
      if (a.key_valid && !a.key_valid[tok0 + j]) continue;
      float sc = 0.f;
#pragma unroll
      for (int d = 0; d < kHD; ++d) sc += qv[d] * Kt[r][d];
      sc *= a.c2;
      const float mn = fmaxf(m, sc);
      const float alpha = exp2f(m - mn);
      const float p = exp2f(sc - mn);
      l = l * alpha + p;
#pragma unroll
      for (int d = 0; d < kHD; ++d) acc[d] = acc[d] * alpha + p * Vt32[r][d];
      m = mn;
    }
  }
  if (!qvalid) return;
  float* op = reinterpret_cast<float*>(a.o) + (int64_t)(tok0 + qrow) * a.os[0] + h * a.os[1];
  const float inv = l > 0.f ? 1.0f / l : 0.f;
#pragma unroll
  for (int d = 0; d < kHD; ++d) op[d] = acc[d] * inv;
}

}  // namespace vfk

using namespace vfk;

static int check_thd(const vfk_tensor* t, const char* name, int dtype, int64_t T, int64_t H) {
  int rc = check_tensor(t, name, 3);
  if (rc) return rc;
  if (t->dtype != dtype)
    return set_error(VFK_ERR_INVALID, "%s: dtype differs from q", name);
  if (t->size[0] != T || t->size[1] != H)
    return set_error(VFK_ERR_INVALID, "%s: expected [%lld, %lld, 64]", name, (long long)T, (long long)H);
  if (t->size[2] != kHD)
    return set_error(VFK_ERR_UNSUPPORTED, "%s: head_dim %lld (only 64 is built)", name,
                     (long long)t->size[2]);
  if (t->stride[2] != 1)
    return set_error(VFK_ERR_INVALID, "%s: head_dim must be contiguous", name);
  if (dtype != VFK_F32 && (!aligned16(t->data) || t->stride[0] % 8 || t->stride[1] % 8))
    return set_error(VFK_ERR_INVALID, "%s: rows must be 16-byte aligned", name);
  return VFK_OK;
}

static int64_t kr_bytes(int64_t T, int64_t H) { return (T * H * kHD * 2 + 255) / 256 * 256; }

static int launch_varlen(VarlenArgs& a, int dt, bool rope, int max_seqlen, hipStream_t st,
                         const char* nm);


extern "C" int64_t vfk_varlen_attn_workspace_bytes(int32_t dtype, int64_t total_tokens,
                                                  int32_t num_heads, int32_t rope,
                                                  int32_t num_seqs, int32_t max_seqlen) {
  if (!rope || dtype == VFK_F32 || total_tokens <= 0 || num_heads <= 0 || num_seqs <= 0 ||
      max_seqlen <= 0)
    return 0;
  // four partial key-norm maxima (one per 16 rows) per 64-key tile
  const int64_t nkt = (max_seqlen + 63) / 64;
  return kr_bytes(total_tokens, num_heads) + (int64_t)num_heads * num_seqs * nkt * 16;
}

extern "C" int vfk_varlen_attn_fwd(const vfk_tensor* q, const vfk_tensor* k,
                                   const vfk_tensor* v, const int32_t* cu_seqlens,
                                   int32_t num_seqs, int32_t max_seqlen,
                                   int32_t window, const float* rope_cos_sin,
                                   int32_t rope_positions, const uint8_t* key_valid,
                                   float softmax_scale, void* workspace,
                                   int64_t workspace_bytes, vfk_tensor* out, void* stream) {
  int rc = check_tensor(q, "q", 3);
  if (rc) return rc;
  const int dt = q->dtype;
  const int64_t T = q->size[0], H = q->size[1];
  if ((rc = check_thd(q, "q", dt, T, H)) || (rc = check_thd(k, "k", dt, T, H)) ||
      (rc = check_thd(v, "v", dt, T, H)) || (rc = check_thd(out, "out", dt, T, H)))
    return rc;
  if (!cu_seqlens) return set_error(VFK_ERR_INVALID, "cu_seqlens is NULL");
  if (num_seqs < 0 || max_seqlen < 0)
    return set_error(VFK_ERR_INVALID, "num_seqs/max_seqlen must be >= 0");
  if (T >= (1ll << 31) || H > 4096 || max_seqlen > (1 << 24))
    return set_error(VFK_ERR_UNSUPPORTED, "vfk_varlen_attn_fwd: sizes too large");
  if (num_seqs == 0 || max_seqlen == 0 || H == 0) return VFK_OK;
  VarlenArgs a = {};
  a.q = q->data; a.k = k->data; a.v = v->data; a.o = out->data;
  for (int i = 0; i < 2; ++i) {
    a.qs[i] = q->stride[i]; a.ks[i] = k->stride[i];
    a.vs[i] = v->stride[i]; a.os[i] = out->stride[i];
  }
  a.cu = cu_seqlens; a.nseq = num_seqs; a.H = (int)H; a.T = T; a.maxlen = max_seqlen;
  a.window = window < 0 ? -1 : window;
  if (!(softmax_scale > 0.f) || !isfinite(softmax_scale))
    return set_error(VFK_ERR_UNSUPPORTED, "vfk_varlen_attn_fwd: softmax_scale must be > 0");
  a.c2 = softmax_scale * VFK_LOG2E;
  a.key_valid = key_valid;
  if (rope_cos_sin) {
    if (rope_positions < max_seqlen)
      return set_error(VFK_ERR_INVALID, "rope table has %d positions < max_seqlen %d",
                       rope_positions, max_seqlen);
    if (!aligned16(rope_cos_sin))
      return set_error(VFK_ERR_INVALID, "rope table must be 16-byte aligned");
  }
  a.rope = rope_cos_sin;
  hipStream_t st = (hipStream_t)stream;
  if (dt == VFK_F32) {
    a.nqt = ceil_div(max_seqlen, 128);
    const int64_t blocks = (int64_t)a.nqt * 2 * H * num_seqs;
    hipLaunchKernelGGL(varlen_fwd_f32_kernel, dim3((unsigned)blocks), dim3(64), 0, st, a);
    return launch_status("vfk_varlen_attn_fwd");
  }
  // buffer resources cover max_seqlen rows of one slice: byte sizes < 2^31
  const int64_t span = (int64_t)max_seqlen * 2;
  if (span * std::max<int64_t>(a.ks[0], 64) >= (1ll << 31) || span * a.vs[0] >= (1ll << 31))
    return set_error(VFK_ERR_UNSUPPORTED, "vfk_varlen_attn_fwd: max_seqlen x row stride too large");
  const bool rope = a.rope != nullptr;
  if (rope) {
    const int64_t need = vfk_varlen_attn_workspace_bytes(dt, T, (int32_t)H, 1, num_seqs, max_seqlen);
    if (!workspace || workspace_bytes < need)
      return set_error(VFK_ERR_INVALID, "vfk_varlen_attn_fwd: RoPE needs a workspace of %lld bytes",
                       (long long)need);
    if (!aligned16(workspace))
      return set_error(VFK_ERR_INVALID, "workspace must be 16-byte aligned");
    a.kr = workspace;
    const int nkt = ceil_div(max_seqlen, 64);
    a.nkt = nkt;
    a.kmax = reinterpret_cast<float*>(static_cast<char*>(workspace) + kr_bytes(T, H));
    const int ngrp = nkt * (64 / kPackRows);
    // 4 head pairs per block where H is a multiple of 8 but not of 12, else 6
    const int npair = (H % 8 == 0 && H % 12 != 0) ? 4 : 6;
    const int nhg = (int)ceil_div(H, 2 * npair);
    const int64_t pblocks = (int64_t)num_seqs * ngrp * nhg;
    if (pblocks >= (1ll << 31))
      return set_error(VFK_ERR_UNSUPPORTED, "vfk_varlen_attn_fwd: grid too large");
#define VFK_PACK(E, NP) \
  hipLaunchKernelGGL((rope_k_pack_kernel<E, NP>), dim3((unsigned)pblocks), dim3(256), 0, st, a, ngrp, nhg)
    if (dt == VFK_BF16) {
      if (npair == 4) VFK_PACK(BF16, 4);
      else VFK_PACK(BF16, 6);
    } else {
      if (npair == 4) VFK_PACK(F16, 4);
      else VFK_PACK(F16, 6);
    }
#undef VFK_PACK
  }
  return launch_varlen(a, dt, rope, max_seqlen, st, "vfk_varlen_attn_fwd");
}

// Attention over K already rotated, scaled by c2 and laid out head-major by
// the fused q | k | v projection (vfk_qkv_rope_linear_fwd): no pre-pass.
extern "C" int vfk_varlen_attn_krot_fwd(const vfk_tensor* q, const vfk_tensor* v,
                                        const void* krot, int64_t krot_bytes,
                                        const int32_t* cu_seqlens, int32_t num_seqs,
                                        int32_t max_seqlen, int32_t window,
                                        const float* rope_cos_sin, int32_t rope_positions,
                                        const uint8_t* key_valid, float softmax_scale,
                                        vfk_tensor* out, void* stream) {
  const char* nm = "vfk_varlen_attn_krot_fwd";
  int rc = check_tensor(q, "q", 3);
  if (rc) return rc;
  const int dt = q->dtype;
  const int64_t T = q->size[0], H = q->size[1];
  if (dt != VFK_BF16 && dt != VFK_F16) return set_error(VFK_ERR_UNSUPPORTED, "%s: q must be bf16 or fp16", nm);
  if ((rc = check_thd(q, "q", dt, T, H)) || (rc = check_thd(v, "v", dt, T, H)) ||
      (rc = check_thd(out, "out", dt, T, H)))
    return rc;
  if (!cu_seqlens) return set_error(VFK_ERR_INVALID, "cu_seqlens is NULL");
  if (num_seqs < 0 || max_seqlen < 0)
    return set_error(VFK_ERR_INVALID, "num_seqs/max_seqlen must be >= 0");
  if (T >= (1ll << 31) || H > 4096 || max_seqlen > (1 << 24))
    return set_error(VFK_ERR_UNSUPPORTED, "%s: sizes too large", nm);
  if (num_seqs == 0 || max_seqlen == 0 || H == 0) return VFK_OK;
  if (!(softmax_scale > 0.f) || !isfinite(softmax_scale))
    return set_error(VFK_ERR_UNSUPPORTED, "%s: softmax_scale must be > 0", nm);
  if (!rope_cos_sin || rope_positions < max_seqlen || !aligned16(rope_cos_sin))
    return set_error(VFK_ERR_INVALID, "%s: rope table missing, unaligned or shorter than max_seqlen", nm);
  const int64_t need = kr_bytes(T, H) + H * ((T + 31) / 32) * 4;
  if (!krot || krot_bytes < need || !aligned16(krot))
    return set_error(VFK_ERR_INVALID, "%s: krot needs %lld 16-byte aligned bytes", nm, (long long)need);
  VarlenArgs a = {};
  a.q = q->data; a.k = nullptr; a.v = v->data; a.o = out->data;
  for (int i = 0; i < 2; ++i) {
    a.qs[i] = q->stride[i]; a.vs[i] = v->stride[i]; a.os[i] = out->stride[i];
  }
  a.cu = cu_seqlens; a.nseq = num_seqs; a.H = (int)H; a.T = T; a.maxlen = max_seqlen;
  a.window = window < 0 ? -1 : window;
  a.c2 = softmax_scale * VFK_LOG2E;
  a.key_valid = key_valid;
  a.rope = rope_cos_sin;
  a.kr = krot;
  a.kmax = reinterpret_cast<float*>(static_cast<char*>(const_cast<void*>(krot)) + kr_bytes(T, H));
  a.kblk32 = 1;
  const int64_t span = (int64_t)max_seqlen * 2;
  if (span * 64 >= (1ll << 31) || span * a.vs[0] >= (1ll << 31))
    return set_error(VFK_ERR_UNSUPPORTED, "%s: max_seqlen x row stride too large", nm);
  if ((int64_t)num_seqs * H >= (1ll << 31))
    return set_error(VFK_ERR_UNSUPPORTED, "%s: grid too large", nm);
  // rows past max_seqlen (no pre-pass runs on this path to clear them)
  hipLaunchKernelGGL(zero_cut_rows_kernel, dim3((unsigned)(num_seqs * H)), dim3(256), 0,
                     (hipStream_t)stream, a);
  return launch_varlen(a, dt, true, max_seqlen, (hipStream_t)stream, nm);
}

// Launch of the 16-bit attention kernel for prepared arguments.
static int launch_varlen(VarlenArgs& a, int dt, bool rope, int max_seqlen, hipStream_t st,
                         const char* nm) {
  const int64_t H = a.H, num_seqs = a.nseq;
  if (a.window >= 0 && a.window >= max_seqlen) a.window = -1;  // window covers every pair
  if (a.window > kPenOff - kBM)
    return set_error(VFK_ERR_UNSUPPORTED, "%s: window %d > %d", nm, a.window, kPenOff - kBM);
  a.nqt = ceil_div(max_seqlen, kBM);
  const int64_t blocks = (int64_t)a.nqt * H * num_seqs;
  if (blocks >= (1ll << 31))
    return set_error(VFK_ERR_UNSUPPORTED, "%s: grid too large", nm);
  const bool local = a.window >= 0, kv = a.key_valid != nullptr;
#define VFK_VL(E, R, L, K) \
  hipLaunchKernelGGL((varlen_fwd_kernel<E, R, L, K>), dim3((unsigned)blocks), dim3(256), 0, st, a)
#define VFK_VL_E(E)                                                   \
  if (rope) {                                                         \
    if (local) { if (kv) VFK_VL(E, true, true, true); else VFK_VL(E, true, true, false); } \
    else { if (kv) VFK_VL(E, true, false, true); else VFK_VL(E, true, false, false); }    \
  } else {                                                            \
    if (local) { if (kv) VFK_VL(E, false, true, true); else VFK_VL(E, false, true, false); } \
    else { if (kv) VFK_VL(E, false, false, true); else VFK_VL(E, false, false, false); }    \
  }
  if (dt == VFK_BF16) {
    VFK_VL_E(BF16)
  } else {
    VFK_VL_E(F16)
  }
#undef VFK_VL_E
#undef VFK_VL
  return launch_status(nm);
}

extern "C" int vfk_rope_table(float theta, int32_t max_positions, float* out, void* stream) {
  if (!out || max_positions < 0) return set_error(VFK_ERR_INVALID, "vfk_rope_table: bad arguments");
  if (!(theta > 0.f)) return set_error(VFK_ERR_INVALID, "vfk_rope_table: theta must be > 0");
  if (max_positions == 0) return VFK_OK;
  RopeTableArgs a = {};
  a.out = out;
  a.npos = max_positions;
  // inv_freq exactly as the HF rotary module computes it in fp32:
  // 1 / theta ** (arange(0, 64, 2).float() / 64)
  for (int f = 0; f < 32; ++f) a.inv_freq[f] = 1.0f / powf(theta, (float)(2 * f) / 64.0f);
  const int64_t n = (int64_t)max_positions * 32;
  hipLaunchKernelGGL(rope_table_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, a);
  return launch_status("vfk_rope_table");
}
