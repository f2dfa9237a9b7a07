// T5 relative-position-bias flash attention (forward), kernels for gfx950.
//
// Reference behaviour: kernels/flash_attention_rpb.py:61-230 (Triton kernel)
// and its eager twin models/mt5/mt5_encoder.py:150-164, :285-320.
//   out = softmax(q k^T * scale + table[bucket(k - q), h] + mask) v
// The bucket of every relative position the workgroup can meet is evaluated
// once into an LDS table of bias values (already multiplied by log2 e), so the
// inner loop does one LDS read per score instead of a log and a gather.
#include <math.h>

#include <algorithm>
#include <type_traits>

#include "attn_core.h"
#include "launch_util.h"

namespace vfk {

enum { MASK_NONE = 0, MASK_KEY = 1, MASK_FULL = 2 };
// LDS copy of the step thresholds: VFK_MAX_THR int16 rounded to 16 bytes
constexpr int kThrPad = (VFK_MAX_THR + 7) & ~7;

struct RpbArgs {
  const void* q; const void* k; const void* v; void* o;
  int64_t qs[4], ks[4], vs[4], os[4];  // [B,H,L,D] strides, D stride is 1
  const void* table; int table_dt; int64_t tb0, tb1; int total_buckets;
  const void* mask; int mask_dt; int64_t ms[4];
  int B, H, Lq, Lk;
  float c2;     // softmax_scale * log2(e)
  float inv_scale;  // 1 / softmax_scale: bias and mask in raw score units
  int bidir, causal, offset_pos;  // offset added for rel > 0 (bidirectional)
  int lut_len;  // ntiles * kBN + kBM (LDS bias table entries)
  StepFn step;
  // packed sequences (nullptr: the padded batch): "batch" b is sequence b,
  // tokens cu[b] .. cu[b + 1] - 1 of [T, H, D] tensors (strides [.][1] =
  // head, [.][2] = token); Lq = Lk = the longest sequence
  const int32_t* cu;
};

__device__ inline float ld_f(const void* p, int dt, int64_t i) {
  if (dt == VFK_F32) return reinterpret_cast<const float*>(p)[i];
  if (dt == VFK_BF16) return BF16::to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
  return F16::to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
}

// Additive mask value in raw score units (mask / softmax_scale). Clamped at
// -1e30: still absorbs any score exactly (so a row whose keys are all masked
// averages uniformly, like the reference's finite mask), while the softmax's
// later multiply by scale*log2(e) cannot overflow.
__device__ inline float mask_raw(float m, float inv_scale) {
  return fmaxf(m * inv_scale, -1.0e30f);
}
// fp32 kernel works in log2 units.
__device__ inline float mask_l2(float m) {
  return fmaxf(m * VFK_LOG2E, -3.0e38f);
}

__device__ inline int rpb_bucket(const RpbArgs& a, int rel) {
  int b;
  if (a.bidir) {
    const int mag = rel < 0 ? -rel : rel;
    b = step_eval(a.step, mag) + (rel > 0 ? a.offset_pos : 0);
  } else {
    b = step_eval(a.step, rel < 0 ? -rel : 0);
  }
  return min(max(b, 0), a.total_buckets - 1);
}

// ---------------------------------------------------------------------------
// bf16 / fp16 MFMA kernel on the shared direct-to-LDS tile loop.
// ---------------------------------------------------------------------------
template <typename E, int MASK, bool CAUSAL>
struct RpbPolicy {
  const RpbArgs* a;
  TileSrc ksrc, vsrc;
  const int* tiles;      // live key tiles (MASK_KEY) or nullptr = all in order
  const int* tflag;      // MASK_KEY: per key tile, bit0 = some nonzero mask
  float* maskt;          // MASK_KEY: [2][kBN] mask values of the tile in slot i & 1
  const float* tailm;    // [kBN]: 0 / -inf per key of the partial last key tile
  const float* lut;      // bias per relative position (raw score units) or nullptr
  int lut_base, b, h, t, hl, qrow, wq_lo, wq_hi;
  int Lq, Lk;            // query / key rows of this (batch, head) or sequence
  bool nolive;           // MASK_KEY: every key of the row range masked away

  static constexpr bool kAllActive = !CAUSAL;
  __device__ int tile(int i) const { return tiles ? tiles[i] : i; }
  __device__ int key0(int i) const { return tile(i) * kBN; }
  __device__ void loadK(int i, uint16_t* Kt) { tile_load_buf(ksrc, key0(i), Kt); }
  __device__ void loadV(int i, uint16_t* Vt) { tile_load_buf(vsrc, key0(i), Vt); }
  // key-mask values of the tile, wave 0 one key per lane; only tiles that
  // hold a nonzero value are loaded (right padding leaves one such tile)
  __device__ float meta_ld(int i) const {
    if (MASK != MASK_KEY || t >= kBN || !(tflag[tile(i)] & 1)) return 0.f;
    const int j = key0(i) + t;
    return j < Lk ? mask_raw(ld_f(a->mask, a->mask_dt, b * a->ms[0] + h * a->ms[1] + j * a->ms[3]),
                                a->inv_scale)
                     : 0.f;
  }
  __device__ void meta_st(float v, int slot) {
    if (MASK == MASK_KEY && t < kBN) maskt[slot * kBN + t] = v;
  }
  __device__ bool wave_active() const { return wq_lo < Lq; }
  __device__ bool active(int i) const {
    if (wq_lo >= Lq) return false;
    return !CAUSAL || key0(i) <= wq_hi;
  }
  // the relative-position bias enters as the QK MFMAs' accumulator input
  __device__ bool init(f32x16_t& s0, f32x16_t& s1, int i, int) const {
    if (!lut || (MASK == MASK_KEY && nolive)) return false;
    load_by_key(s0, s1, lut + key0(i) + lut_base);
    return true;
  }
  __device__ bool modify(f32x16_t& s0, f32x16_t& s1, int i, int slot) const {
    const int k0 = key0(i);
    bool exact = false;
    if (MASK == MASK_KEY && nolive) {
      // every key's mask is below -1e30 (raw units): scores and biases are
      // absorbed by it, so the row averages V over its keys
      s0 = f32x16_t{};
      s1 = f32x16_t{};
    } else {
      // masked keys (-1e30) fall far below the row max of the live keys:
      // the fma exponent form underflows them to 0 without an exact path
      if (MASK == MASK_KEY && (tflag[tile(i)] & 1)) add_by_key(s0, s1, maskt + slot * kBN + 4 * hl);
    }
    if (MASK == MASK_FULL) {
      if (qrow < Lq) {
        const int64_t mo = b * a->ms[0] + h * a->ms[1] + (int64_t)qrow * a->ms[2];
        map_scores(s0, s1, [&](int e, float v) {
          const int j = k0 + x_key(e, hl);
          return j < Lk ? v + mask_raw(ld_f(a->mask, a->mask_dt, mo + (int64_t)j * a->ms[3]),
                                          a->inv_scale)
                           : v;
        });
      }
      exact = true;
    }
    // the partial tile's keys from the LDS table (with a full mask the
    // compare form keeps the kernel within its registers)
    if (!CAUSAL && MASK != MASK_FULL) {
      if (k0 + kBN > Lk) add_by_key(s0, s1, tailm + 4 * hl);
    } else if (k0 + kBN > Lk || (CAUSAL && k0 + kBN - 1 > wq_lo)) {
      map_scores(s0, s1, [&](int e, float v) {
        const int j = k0 + x_key(e, hl);
        return (j >= Lk || (CAUSAL && j > qrow)) ? -INFINITY : v;
      });
    }
    return exact;
  }
};

template <typename E, int MASK, bool CAUSAL>
__global__ __launch_bounds__(256, 4) void rpb_fwd_kernel(RpbArgs a) {
  __shared__ __align__(16) uint16_t K0[kTileElems];
  __shared__ __align__(16) uint16_t K1[kTileElems];
  __shared__ __align__(16) uint16_t V0[kTileElems];
  __shared__ __align__(16) uint16_t V1[kTileElems];
  __shared__ float maskt[MASK == MASK_KEY ? 2 * kBN : 1];
  __shared__ float tailm[kBN];
  __shared__ int ntl;
  __shared__ int nolive_s;
  __shared__ int spec_bad;  // some row of the fixed-softmax pass failed its check
  extern __shared__ __align__(16) unsigned char smem[];
  const int nqt = (a.Lq + kBM - 1) / kBM;
  const int work = xcd_remap(blockIdx.x, gridDim.x);
  const int qt = work % nqt;
  const int bh = work / nqt;
  const int h = bh % a.H, b = bh / a.H;
  const int q0 = qt * kBM;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6, hl = lane >> 5;
  // rows of this (batch, head) or sequence, and their offsets in q, k, v, o
  int Lq = a.Lq, Lk = a.Lk;
  int64_t qo = b * a.qs[0], ko = b * a.ks[0], vo = b * a.vs[0], oo = b * a.os[0];
  if (a.cu) {
    const int tok0 = a.cu[b];
    // rows past max_seqlen (a.Lq) are not computed (the LDS tables are sized
    // for a.Lk keys): the last query tile writes them as zeros
    const int nfull = a.cu[b + 1] - tok0;
    Lq = Lk = min(nfull, a.Lq);
    qo = (int64_t)tok0 * a.qs[2]; ko = (int64_t)tok0 * a.ks[2];
    vo = (int64_t)tok0 * a.vs[2]; oo = (int64_t)tok0 * a.os[2];
    if (qt == nqt - 1 && nfull > Lq)
      zero_rows_d64(reinterpret_cast<uint16_t*>(a.o) + oo + h * a.os[1], a.os[2], Lq, nfull);
    if (q0 >= Lq) return;  // whole workgroup: uniform exit
  }
  // the host sizes the dynamic LDS for a.Lk keys, an upper bound of Lk
  const int ntiles_all = (Lk + kBN - 1) / kBN;
  const int nt4 = (ntiles_all + 3) & ~3;
  const int nt4_lds = (((a.Lk + kBN - 1) / kBN) + 3) & ~3;
  int* tflag = reinterpret_cast<int*>(smem);  // [nt4]
  int* tiles = tflag + nt4_lds;               // [nt4]
  float* lut = reinterpret_cast<float*>(tiles + nt4_lds);
  (void)nt4;

  // keys past Lk in the partial last tile (read before the first barrier)
  if (t < kBN) tailm[t] = ((Lk - 1) / kBN) * kBN + t < Lk ? 0.f : -INFINITY;
  if (t == 0) spec_bad = 0;

  // ---- bias table over rel = key - query, rel in [-(q0+127), Lk-1-q0] ----
  // the step thresholds and the head's table column go to LDS first, so each
  // entry is a binary search and a lookup in LDS
  const bool has_table = a.table != nullptr;
  if (has_table) {
    int16_t* thr = reinterpret_cast<int16_t*>(lut + a.lut_len);
    float* tcol = reinterpret_cast<float*>(thr + kThrPad);
    for (int e = t; e < a.step.nthr; e += 256) thr[e] = a.step.thr[e];
    for (int e = t; e < a.total_buckets; e += 256)
      tcol[e] = ld_f(a.table, a.table_dt, e * a.tb0 + h * a.tb1) * a.inv_scale;
    __syncthreads();
    const int a0 = a.step.a0, f0 = a.step.f0, nthr = a.step.nthr;
    for (int e = t; e < a.lut_len; e += 256) {
      const int rel = e - q0 - (kBM - 1);
      const int mag = a.bidir ? (rel < 0 ? -rel : rel) : (rel < 0 ? -rel : 0);
      int bk = mag;
      if (mag >= a0) {
        int lo = 0, hi = nthr;
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          if ((int)thr[mid] <= mag) lo = mid + 1; else hi = mid;
        }
        bk = f0 + lo;
      }
      if (a.bidir && rel > 0) bk += a.offset_pos;
      lut[e] = tcol[min(max(bk, 0), a.total_buckets - 1)];
    }
  }
  // ---- key tiles: causal limit, and (key mask) the tiles with a live key ----
  int kt_end = ntiles_all;
  if (CAUSAL) kt_end = min(kt_end, (min(q0 + kBM, Lq) - 1) / kBN + 1);
  int n = kt_end;
  bool direct = true;  // live tiles are 0 .. n-1 (no list indirection)
  if (MASK == MASK_KEY) {
    // pass i: thread t reads key 256 i + t, so wave w holds key tile 4 i + w
    // and its ballots give that tile's flags (no atomics)
    const char* mb = reinterpret_cast<const char*>(a.mask);
    for (int j0 = 0; j0 < ntiles_all * kBN; j0 += 256) {
      const int j = j0 + t;
      float mv = 0.f;
      if (j < Lk) mv = ld_f(mb, a.mask_dt, b * a.ms[0] + h * a.ms[1] + j * a.ms[3]);
      // bit0: some nonzero value; bit1: some key that is not clamped away
      const unsigned long long nz = __builtin_amdgcn_ballot_w64(mv != 0.f);
      const unsigned long long lv = __builtin_amdgcn_ballot_w64(j < Lk && mask_raw(mv, a.inv_scale) > -1.0e30f);
      const int tile = (j0 >> 6) + w;
      if (lane == 0 && tile < ntiles_all) tflag[tile] = (nz ? 1 : 0) | (lv ? 2 : 0);
    }
    __syncthreads();
    // tiles whose every key is masked away are skipped, unless no key of the
    // row range is live (then the reference averages all of them); wave 0
    // compacts the list, 64 tiles per pass
    if (w == 0) {
      unsigned long long live_any = 0;
      for (int i0 = 0; i0 < kt_end; i0 += 64)
        live_any |= __builtin_amdgcn_ballot_w64(i0 + lane < kt_end && (tflag[i0 + lane] & 2));
      int c = 0;
      bool prefix = true;
      for (int i0 = 0; i0 < kt_end; i0 += 64) {
        const int i = i0 + lane;
        const bool keep = i < kt_end && (!live_any || (tflag[i] & 2));
        const unsigned long long kb = __builtin_amdgcn_ballot_w64(keep);
        const int pos = c + __builtin_amdgcn_mbcnt_hi((unsigned)(kb >> 32), __builtin_amdgcn_mbcnt_lo((unsigned)kb, 0u));
        if (keep) tiles[pos] = i;
        prefix = prefix && __builtin_amdgcn_ballot_w64(keep && pos != i) == 0ull;
        c += __builtin_popcountll(kb);
      }
      if (lane == 0) {
        ntl = prefix ? -c : c;  // negative: the list is 0 .. c-1
        nolive_s = live_any == 0ull;
      }
    }
    __syncthreads();
    n = ntl < 0 ? -ntl : ntl;
    direct = ntl < 0;
  }

  RpbPolicy<E, MASK, CAUSAL> pol;
  pol.a = &a;
  tile_src_init(pol.ksrc, reinterpret_cast<const uint16_t*>(a.k) + ko + h * a.ks[1], (int)a.ks[2], Lk);
  tile_src_init(pol.vsrc, reinterpret_cast<const uint16_t*>(a.v) + vo + h * a.vs[1], (int)a.vs[2], Lk);
  pol.Lq = Lq; pol.Lk = Lk;
  pol.tiles = (MASK == MASK_KEY && !direct) ? tiles : nullptr;
  pol.tflag = tflag;
  pol.maskt = maskt;
  pol.tailm = tailm;
  pol.lut = has_table ? lut : nullptr;
  pol.nolive = MASK == MASK_KEY && nolive_s != 0;
  pol.b = b; pol.h = h; pol.t = t; pol.hl = hl;
  pol.wq_lo = q0 + w * 32;
  pol.qrow = pol.wq_lo + (lane & 31);
  pol.wq_hi = min(pol.wq_lo + 31, Lq - 1);
  // lut index of element e in the tile at key0: key0 + x_key(e, 0) + lut_base
  pol.lut_base = 4 * hl - w * 32 - (lane & 31) + (kBM - 1);
  attn_pipe_start(pol, n, K0, K1, V0, V1);

  const bool qvalid = pol.qrow < Lq;
  u32x4_t qf[4];
  load_q(qf, reinterpret_cast<const uint16_t*>(a.q) + qo + h * a.qs[1] + (int64_t)pol.qrow * a.qs[2],
         qvalid);

  // bf16: first p = exp2(c2 s) with no running max. T5 does not scale its
  // scores, so no bound known before the loop keeps them small, but bf16 and
  // the fp32 sums hold p up to 2^127: the pass fails only for rows whose sum
  // or outputs overflow, or whose sum is below 2^-64 (every score far below
  // 0, where low probabilities would flush to zero). Such a workgroup runs
  // the item again with the running max. fp16 (p at most 65504) and the full
  // [L, L] mask (whose second loop would not fit the registers) always take
  // the running max.
  constexpr bool kSpec = std::is_same<E, BF16>::value && MASK != MASK_FULL;
  float m = -INFINITY, l_tot = 0.f;
  RowSumDot<E> l;
  f32x16_t o0 = {}, o1 = {};
  bool rerun = !kSpec;
  if (kSpec) {
    attn_loop_db<E, true>(pol, K0, K1, V0, V1, n, qf, a.c2, m, l, o0, o1);
    l_tot = l.total();
    float fin = l_tot * 0.f;  // NaN when anything below is not finite
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      fin = __builtin_fmaf(o0[i], 0.f, fin);
      fin = __builtin_fmaf(o1[i], 0.f, fin);
    }
    const bool bad = qvalid && n > 0 && (fin != 0.f || !(l_tot >= 0x1p-64f));
    if (__builtin_amdgcn_ballot_w64(bad) != 0ull && lane == 0) spec_bad = 1;
    __syncthreads();
    rerun = spec_bad != 0;
    if (rerun) {
      l = RowSumDot<E>{};
      o0 = f32x16_t{};
      o1 = f32x16_t{};
      attn_pipe_start(pol, n, K0, K1, V0, V1);  // the first tiles again
    }
  }
  if (rerun) {
    attn_loop_db<E>(pol, K0, K1, V0, V1, n, qf, a.c2, m, l, o0, o1);
    l_tot = l.total();
  }
  // whole-row stores through this wave's half of K0 / K1 (free after the loop)
  uint16_t* ob = reinterpret_cast<uint16_t*>(a.o) + oo + h * a.os[1];
  const int wq_lo = pol.wq_lo;
  store_out_rows<E>((w < 2 ? K0 : K1) + (w & 1) * 2048, o0, o1, l_tot,
                    [&](int r) { return ob + (int64_t)(wq_lo + r) * a.os[2]; },
                    [&](int r) { return wq_lo + r < Lq; });
}

// ---------------------------------------------------------------------------
// fp32 kernel: one thread per query row, exact fp32 arithmetic throughout.
// ---------------------------------------------------------------------------
template <int MASK>
__global__ __launch_bounds__(64) void rpb_fwd_f32_kernel(RpbArgs a) {
  __shared__ float Kt[64][kHD + 1];
  __shared__ float Vt32[64][kHD + 1];
  const int nqt = (a.Lq + 63) / 64;
  const int qt = blockIdx.x % nqt;
  const int bh = blockIdx.x / nqt;
  const int h = bh % a.H, b = bh / a.H;
  const int qrow = qt * 64 + threadIdx.x;
  const bool qvalid = qrow < a.Lq;
  const float* Qp = reinterpret_cast<const float*>(a.q) + b * a.qs[0] + h * a.qs[1];
  const float* Kp = reinterpret_cast<const float*>(a.k) + b * a.ks[0] + h * a.ks[1];
  const float* Vp = reinterpret_cast<const float*>(a.v) + b * a.vs[0] + h * a.vs[1];
  float qv[kHD], acc[kHD];
#pragma unroll
  for (int d = 0; d < kHD; ++d) {
    qv[d] = qvalid ? Qp[(int64_t)qrow * a.qs[2] + d] : 0.f;
    acc[d] = 0.f;
  }
  float m = -INFINITY, l = 0.f;
  int kend = a.Lk;
  if (a.causal) kend = min(kend, min(qt * 64 + 64, a.Lq));
  for (int key0 = 0; key0 < kend; key0 += 64) {
    __syncthreads();
    for (int e = threadIdx.x; e < 64 * kHD; e += 64) {
      const int r = e / kHD, d = e % kHD;
      const int j = key0 + r;
      Kt[r][d] = j < a.Lk ? Kp[(int64_t)j * a.ks[2] + d] : 0.f;
      Vt32[r][d] = j < a.Lk ? Vp[(int64_t)j * a.vs[2] + d] : 0.f;
    }
    __syncthreads();
    const int nk = min(64, kend - key0);
    for (int r = 0; r < nk; ++r) {
      const int j = key0 + r;
      if (a.causal && j > qrow) break;
      float s = 0.f;
#pragma unroll
      for (int d = 0; d < kHD; ++d) s += qv[d] * Kt[r][d];
      s = s * a.c2;
      if (a.table) s += ld_f(a.table, a.table_dt, rpb_bucket(a, j - qrow) * a.tb0 + h * a.tb1) * VFK_LOG2E;
      if (MASK != MASK_NONE)
        s += mask_l2(ld_f(a.mask, a.mask_dt, b * a.ms[0] + h * a.ms[1] + (int64_t)qrow * a.ms[2] + (int64_t)j * a.ms[3]));
      const float mn = fmaxf(m, s);
      const float alpha = exp2f(m - mn);
      const float p = exp2f(s - mn);
      l = l * alpha + p;
#pragma unroll
      for (int d = 0; d < kHD; ++d) acc[d] = acc[d] * alpha + p * Vt32[r][d];
      m = mn;
    }
  }
  if (!qvalid) return;
  float* op = reinterpret_cast<float*>(a.o) + b * a.os[0] + h * a.os[1] + (int64_t)qrow * a.os[2];
  const float inv = l > 0.f ? 1.0f / l : 0.f;
#pragma unroll
  for (int d = 0; d < kHD; ++d) op[d] = acc[d] * inv;
}

}  // namespace vfk

using namespace vfk;

static int check_bhld(const vfk_tensor* t, const char* name, int dtype) {
  int rc = check_tensor(t, name, 4);
  if (rc) return rc;
  if (t->dtype != dtype)
    return set_error(VFK_ERR_INVALID, "%s: dtype %d differs from q", name, t->dtype);
  if (t->size[3] != kHD)
    return set_error(VFK_ERR_UNSUPPORTED, "%s: head_dim %lld (only 64 is built)",
                     name, (long long)t->size[3]);
  if (t->stride[3] != 1)
    return set_error(VFK_ERR_INVALID, "%s: head_dim must be contiguous", name);
  if (dtype != VFK_F32) {
    if (!aligned16(t->data) || t->stride[0] % 8 || t->stride[1] % 8 || t->stride[2] % 8)
      return set_error(VFK_ERR_INVALID, "%s: rows must be 16-byte aligned", name);
  }
  return VFK_OK;
}

// Scale, bucket step function and bias table of a launch (shared by the
// padded and packed entry points).
static int rpb_setup(RpbArgs& a, const vfk_tensor* rpb_table, int32_t num_buckets,
                     int32_t max_distance, int32_t is_decoder, float softmax_scale, int64_t H,
                     const char* name) {
  if (!(softmax_scale > 0.f) || !isfinite(softmax_scale))
    return set_error(VFK_ERR_UNSUPPORTED, "%s: softmax_scale must be > 0", name);
  a.c2 = softmax_scale * VFK_LOG2E;
  a.inv_scale = 1.0f / softmax_scale;
  a.bidir = is_decoder ? 0 : 1;
  a.causal = is_decoder ? 1 : 0;
  if (present(rpb_table)) {
    int rc;
    if ((rc = check_tensor(rpb_table, "rpb_table", 2))) return rc;
    if (rpb_table->size[1] != H)
      return set_error(VFK_ERR_INVALID, "rpb_table: expected [buckets, %lld]", (long long)H);
    if (rpb_table->size[0] < 1)
      return set_error(VFK_ERR_INVALID, "rpb_table: no buckets");
    a.table = rpb_table->data; a.table_dt = rpb_table->dtype;
    a.tb0 = rpb_table->stride[0]; a.tb1 = rpb_table->stride[1];
    a.total_buckets = (int)rpb_table->size[0];
    if ((rc = build_t5_step(a.bidir, num_buckets, max_distance, &a.step))) return rc;
    a.offset_pos = num_buckets / 2;
  }
  return VFK_OK;
}

// MFMA launch over a.B x a.H x ceil(a.Lq / 128) workgroups, LDS sized for
// a.Lk keys.
static int rpb_launch(RpbArgs& a, int mode, int dt, hipStream_t st, const char* name) {
  // tile buffer resources span Lk rows of one (batch, head): byte sizes < 2^31
  if ((int64_t)a.Lk * std::max(a.ks[2], a.vs[2]) * 2 >= (1ll << 31))
    return set_error(VFK_ERR_UNSUPPORTED, "%s: Lk x row stride too large", name);
  const int ntiles = ceil_div(a.Lk, kBN);
  a.lut_len = a.table ? ntiles * kBN + kBM : 0;
  // dynamic LDS: tile flags and list, bias table, step thresholds and the
  // head's table column (tiles and masks are static)
  const size_t lds = (size_t)((ntiles + 3) & ~3) * 8 + (size_t)a.lut_len * 4 +
                     (a.table ? (size_t)kThrPad * 2 + (size_t)a.total_buckets * 4 : 0);
  if (lds + 4 * kTileElems * 2 + 2 * kBN * 4 > 160 * 1024)
    return set_error(VFK_ERR_UNSUPPORTED, "%s: Lk=%d needs too much LDS", name, a.Lk);
  const int nqt = ceil_div(a.Lq, kBM);
  dim3 grid((unsigned)((int64_t)nqt * a.B * a.H));
#define VFK_RPB_GO(E, M, C) hipLaunchKernelGGL((rpb_fwd_kernel<E, M, C>), grid, dim3(256), lds, st, a)
#define VFK_RPB_LAUNCH(E)                                                               \
  switch (mode) {                                                                       \
    case MASK_NONE: if (a.causal) VFK_RPB_GO(E, MASK_NONE, true); else VFK_RPB_GO(E, MASK_NONE, false); break; \
    case MASK_KEY: if (a.causal) VFK_RPB_GO(E, MASK_KEY, true); else VFK_RPB_GO(E, MASK_KEY, false); break;    \
    default: if (a.causal) VFK_RPB_GO(E, MASK_FULL, true); else VFK_RPB_GO(E, MASK_FULL, false); break;        \
  }
  if (dt == VFK_BF16) {
    VFK_RPB_LAUNCH(BF16)
  } else {
    VFK_RPB_LAUNCH(F16)
  }
#undef VFK_RPB_LAUNCH
#undef VFK_RPB_GO
  return launch_status(name);
}

extern "C" int vfk_flash_rpb_fwd(const vfk_tensor* q, const vfk_tensor* k,
                                 const vfk_tensor* v, const vfk_tensor* rpb_table,
                                 int32_t num_buckets, int32_t max_distance,
                                 int32_t is_decoder, const vfk_tensor* mask,
                                 float softmax_scale, vfk_tensor* out,
                                 void* stream) {
  const char* name = "vfk_flash_rpb_fwd";
  int rc = check_tensor(q, "q", 4);
  if (rc) return rc;
  const int dt = q->dtype;
  if ((rc = check_bhld(q, "q", dt)) || (rc = check_bhld(k, "k", dt)) ||
      (rc = check_bhld(v, "v", dt)) || (rc = check_bhld(out, "out", dt)))
    return rc;
  const int64_t B = q->size[0], H = q->size[1], Lq = q->size[2], Lk = k->size[2];
  if (k->size[0] != B || k->size[1] != H || v->size[0] != B || v->size[1] != H ||
      v->size[2] != Lk)
    return set_error(VFK_ERR_INVALID, "vfk_flash_rpb_fwd: q/k/v shapes disagree");
  for (int i = 0; i < 4; ++i)
    if (out->size[i] != q->size[i])
      return set_error(VFK_ERR_INVALID, "vfk_flash_rpb_fwd: out shape must equal q");
  if (Lq > (1 << 20) || Lk > (1 << 20) || B * H > (1 << 24))
    return set_error(VFK_ERR_UNSUPPORTED, "vfk_flash_rpb_fwd: sizes too large");
  RpbArgs a = {};
  a.q = q->data; a.k = k->data; a.v = v->data; a.o = out->data;
  for (int i = 0; i < 4; ++i) {
    a.qs[i] = q->stride[i]; a.ks[i] = k->stride[i];
    a.vs[i] = v->stride[i]; a.os[i] = out->stride[i];
  }
  a.B = (int)B; a.H = (int)H; a.Lq = (int)Lq; a.Lk = (int)Lk;
  if ((rc = rpb_setup(a, rpb_table, num_buckets, max_distance, is_decoder, softmax_scale, H, name)))
    return rc;
  int mode = MASK_NONE;
  if (present(mask)) {
    if ((rc = check_tensor(mask, "padding_mask", 4))) return rc;
    const int64_t want[4] = {B, H, Lq, Lk};
    for (int i = 0; i < 4; ++i) {
      if (mask->size[i] != want[i] && mask->size[i] != 1)
        return set_error(VFK_ERR_INVALID, "padding_mask: dim %d not broadcastable", i);
      a.ms[i] = mask->size[i] == 1 ? 0 : mask->stride[i];
    }
    a.mask = mask->data; a.mask_dt = mask->dtype;
    mode = (a.ms[2] == 0) ? MASK_KEY : MASK_FULL;
  }
  if (B == 0 || H == 0 || Lq == 0) return VFK_OK;
  if (Lk == 0)
    return set_error(VFK_ERR_INVALID, "vfk_flash_rpb_fwd: no keys");
  hipStream_t st = (hipStream_t)stream;
  if (dt == VFK_F32) {
    const int nqt = ceil_div(Lq, 64);
    dim3 grid((unsigned)(nqt * B * H));
    if (mode == MASK_NONE)
      hipLaunchKernelGGL(rpb_fwd_f32_kernel<MASK_NONE>, grid, dim3(64), 0, st, a);
    else
      hipLaunchKernelGGL(rpb_fwd_f32_kernel<MASK_FULL>, grid, dim3(64), 0, st, a);
    return launch_status(name);
  }
  return rpb_launch(a, mode, dt, st, name);
}

// [T, H, 64] tensor of a packed stream (token stride [0], head stride [1]).
static int check_thd_rpb(const vfk_tensor* t, const char* name, int dtype, int64_t T, int64_t H) {
  int rc = check_tensor(t, name, 3);
  if (rc) return rc;
  if (t->dtype != dtype) return set_error(VFK_ERR_INVALID, "%s: dtype differs from q", name);
  if (t->size[0] != T || t->size[1] != H)
    return set_error(VFK_ERR_INVALID, "%s: expected [%lld, %lld, 64]", name, (long long)T, (long long)H);
  if (t->size[2] != kHD)
    return set_error(VFK_ERR_UNSUPPORTED, "%s: head_dim %lld (only 64 is built)", name, (long long)t->size[2]);
  if (t->stride[2] != 1) return set_error(VFK_ERR_INVALID, "%s: head_dim must be contiguous", name);
  if (!aligned16(t->data) || t->stride[0] % 8 || t->stride[1] % 8)
    return set_error(VFK_ERR_INVALID, "%s: rows must be 16-byte aligned", name);
  return VFK_OK;
}

extern "C" int vfk_flash_rpb_varlen_fwd(const vfk_tensor* q, const vfk_tensor* k, const vfk_tensor* v,
                                        const int32_t* cu_seqlens, int32_t num_seqs, int32_t max_seqlen,
                                        const vfk_tensor* rpb_table, int32_t num_buckets,
                                        int32_t max_distance, int32_t is_decoder, float softmax_scale,
                                        vfk_tensor* out, void* stream) {
  const char* name = "vfk_flash_rpb_varlen_fwd";
  int rc = check_tensor(q, "q", 3);
  if (rc) return rc;
  const int dt = q->dtype;
  if (dt != VFK_BF16 && dt != VFK_F16)
    return set_error(VFK_ERR_UNSUPPORTED, "%s: bf16 or fp16 only", name);
  const int64_t T = q->size[0], H = q->size[1];
  if ((rc = check_thd_rpb(q, "q", dt, T, H)) || (rc = check_thd_rpb(k, "k", dt, T, H)) ||
      (rc = check_thd_rpb(v, "v", dt, T, H)) || (rc = check_thd_rpb(out, "out", dt, T, H)))
    return rc;
  if (!cu_seqlens) return set_error(VFK_ERR_INVALID, "%s: NULL cu_seqlens", name);
  if (num_seqs < 0 || max_seqlen < 0 || max_seqlen > (1 << 20) || (int64_t)num_seqs * H > (1 << 24))
    return set_error(VFK_ERR_INVALID, "%s: bad num_seqs / max_seqlen", name);
  RpbArgs a = {};
  a.q = q->data; a.k = k->data; a.v = v->data; a.o = out->data;
  // [T, H, D] as the padded kernel's [., H, L, D]: head stride [1], row stride [2]
  a.qs[1] = q->stride[1]; a.qs[2] = q->stride[0]; a.qs[3] = 1;
  a.ks[1] = k->stride[1]; a.ks[2] = k->stride[0]; a.ks[3] = 1;
  a.vs[1] = v->stride[1]; a.vs[2] = v->stride[0]; a.vs[3] = 1;
  a.os[1] = out->stride[1]; a.os[2] = out->stride[0]; a.os[3] = 1;
  a.B = num_seqs; a.H = (int)H; a.Lq = max_seqlen; a.Lk = max_seqlen;
  a.cu = cu_seqlens;
  if ((rc = rpb_setup(a, rpb_table, num_buckets, max_distance, is_decoder, softmax_scale, H, name)))
    return rc;
  if (num_seqs == 0 || H == 0 || max_seqlen == 0 || T == 0) return VFK_OK;
  return rpb_launch(a, MASK_NONE, dt, (hipStream_t)stream, name);
}
