// DeBERTa-v2/v3 disentangled flash attention (forward), gfx950.
//
// Reference behaviour: kernels/flash_deberta_attention.py:144-299 (Triton) and
// its eager twin :375-448, with the model-side bucket formula of
// models/deberta_v2/deberta_v2_encoder.py:70-89:
//   s(i,j) = (q_i.k_j + pos_key[i, c(i-j)] + pos_query[j, c(i-j)]) * sm_scale
//   c(d)   = clamp(bucket(d) + att_span, 0, 2*att_span - 1)
// keys j >= seq_len[b] are masked and query rows >= seq_len[b] are written as
// zeros (the reference kernel's pre-zeroed output).
//
// The clamped index c(i-j) of every relative position a workgroup meets is
// evaluated once into an LDS table (integer step function built on the host
// from the exact fp32 formula); the inner loop reads it with immediate offsets.
#include <math.h>

#include "attn_core.h"
#include "launch_util.h"

namespace vfk {

struct DebArgs {
  const void* q; const void* k; const void* v; void* o;
  int64_t qs[4], ks[4], vs[4], os[4];
  const void* pk; int64_t pks[4];   // pos_key [B,H,M,2S] or null
  const void* pq; int64_t pqs[4];   // pos_query [B,H,N,2S] or null
  const int32_t* seq_lengths;       // [B] or null (all N valid)
  int B, H, M, N, span;             // span = att_span S
  int causal, log_bucket;
  float c2;                         // sm_scale * log2(e)
  int lut_len;                      // ntiles_k*64 + kBM
  const void* kr; int64_t krs[2];   // fused: key_rel [H, 2S, 64] (c2p) or null
  const void* qr; int64_t qrs[2];   // fused: query_rel [H, 2S, 64] (p2c) or null
  StepFn step;                      // |bucket| as a function of |d| (log mode)
};

__device__ inline int deb_index(const DebArgs& a, int d) {
  int bk;
  if (a.log_bucket) {
    const int mag = step_eval(a.step, d < 0 ? -d : d);
    bk = d < 0 ? -mag : mag;
  } else {
    bk = d;
  }
  return min(max(bk + a.span, 0), 2 * a.span - 1);
}

template <typename E>
__global__ __launch_bounds__(256, 2) void deberta_gather_kernel(DebArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  uint16_t* Ks = reinterpret_cast<uint16_t*>(smem);
  uint16_t* Vt = Ks + kKsElems;
  int16_t* lut = reinterpret_cast<int16_t*>(Vt + kVtElems);  // c(i - j)

  const int nqt = (a.M + kBM - 1) / kBM;
  const int work = xcd_remap(blockIdx.x, gridDim.x);
  const int qt = work % nqt;
  const int bh = work / nqt;
  const int h = bh % a.H, b = bh / a.H;
  const int q0 = qt * kBM;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6, hl = lane >> 5;
  const int len = a.seq_lengths ? min(max(a.seq_lengths[b], 0), a.N) : a.N;
  const int qrow = q0 + w * 32 + (lane & 31);
  const bool qstore = qrow < a.M;
  const bool qvalid = qrow < min(len, a.M);
  uint16_t* orow = reinterpret_cast<uint16_t*>(a.o) + b * a.os[0] + h * a.os[1] + (int64_t)qrow * a.os[2];

  // key tiles: keys < len (and <= row + N - M when causal)
  int kend = len;
  if (a.causal) kend = min(kend, min(q0 + kBM, a.M) + (a.N - a.M));
  const int kt_end = (max(kend, 0) + kBN - 1) / kBN;
  if (q0 >= len || kt_end == 0) {  // every row of the tile is padding: zeros
    if (qstore) {
      f32x16_t z = {};
      store_out<E>(orow, z, z, 0.f);
    }
    return;
  }

  // c(i - j) for d = i - j in [q0 - (kt_end*64 - 1), q0 + 127]
  const int dmin = q0 - (kt_end * kBN - 1);
  for (int e = t; e < a.lut_len; e += 256) lut[e] = (int16_t)deb_index(a, dmin + e);

  const uint16_t* Qp = reinterpret_cast<const uint16_t*>(a.q) + b * a.qs[0] + h * a.qs[1];
  const uint16_t* Kp = reinterpret_cast<const uint16_t*>(a.k) + b * a.ks[0] + h * a.ks[1];
  const uint16_t* Vp = reinterpret_cast<const uint16_t*>(a.v) + b * a.vs[0] + h * a.vs[1];
  const uint16_t* PKrow = a.pk ? reinterpret_cast<const uint16_t*>(a.pk) + b * a.pks[0] + h * a.pks[1] +
                                     (int64_t)min(qrow, a.M - 1) * a.pks[2]
                               : nullptr;
  const uint16_t* PQp = a.pq ? reinterpret_cast<const uint16_t*>(a.pq) + b * a.pqs[0] + h * a.pqs[1] : nullptr;

  u32x4_t qf[4];
  load_q(qf, Qp + (int64_t)qrow * a.qs[2], qvalid);
  float m = -INFINITY, l = 0.f;
  f32x16_t o0 = {}, o1 = {};
  // lut index of element e in tile kt: qrow - key - dmin
  const int lut_lane = qrow - 4 * hl - dmin;

  KVStage st;
  kv_load(st, Kp, a.ks[2], Vp, a.vs[2], 0, kend);
  __syncthreads();  // lut ready
  for (int kt = 0; kt < kt_end; ++kt) {
    const int key0 = kt * kBN;
    kv_store(st, Ks, Vt);
    __syncthreads();
    if (kt + 1 < kt_end) kv_load(st, Kp, a.ks[2], Vp, a.vs[2], (kt + 1) * kBN, kend);

    f32x16_t s0, s1;
    qk_tile<E>(Ks, qf, s0, s1);
    const int16_t* lp = lut + (lut_lane - key0);
    map_scores(s0, s1, [&](int e, float v) {
      const int xk = x_key(e, 0);           // key - key0 - 4*hl
      const int key = key0 + xk + 4 * hl;
      const int c = lp[-xk];
      float bias = 0.f;
      if (PKrow && qvalid) bias += E::to_f32(PKrow[(int64_t)c * a.pks[3]]);
      if (PQp && key < kend) bias += E::to_f32(PQp[(int64_t)key * a.pqs[2] + (int64_t)c * a.pqs[3]]);
      v += bias;
      return (key >= kend || (a.causal && key > qrow + (a.N - a.M))) ? -INFINITY : v;
    });
    u32x4_t p[4];
    softmax_tile<E>(s0, s1, a.c2, m, l, o0, o1, p);
    pv_tile<E>(Vt, p, o0, o1);
    __syncthreads();
  }
  const float l_tot = half_swap_sum(l);
  if (qstore) {
    if (!qvalid) {
      f32x16_t z = {};
      store_out<E>(orow, z, z, 0.f);
    } else {
      store_out<E>(orow, o0, o1, l_tot);
    }
  }
}

// fp32: one thread per query row.
__global__ __launch_bounds__(64) void deberta_gather_f32_kernel(DebArgs a) {
  __shared__ float Kt[64][kHD + 1];
  __shared__ float Vt32[64][kHD + 1];
  const int nqt = (a.M + 63) / 64;
  const int qt = blockIdx.x % nqt;
  const int bh = blockIdx.x / nqt;
  const int h = bh % a.H, b = bh / a.H;
  const int qrow = qt * 64 + threadIdx.x;
  const int len = a.seq_lengths ? min(max(a.seq_lengths[b], 0), a.N) : a.N;
  const bool qstore = qrow < a.M;
  const bool qvalid = qrow < min(len, a.M);
  const float* Qp = reinterpret_cast<const float*>(a.q) + b * a.qs[0] + h * a.qs[1];
  const float* Kp = reinterpret_cast<const float*>(a.k) + b * a.ks[0] + h * a.ks[1];
  const float* Vp = reinterpret_cast<const float*>(a.v) + b * a.vs[0] + h * a.vs[1];
  const float* PK = reinterpret_cast<const float*>(a.pk);
  const float* PQ = reinterpret_cast<const float*>(a.pq);
  float qv[kHD], acc[kHD];
#pragma unroll
  for (int d = 0; d < kHD; ++d) {
    qv[d] = qvalid ? Qp[(int64_t)qrow * a.qs[2] + d] : 0.f;
    acc[d] = 0.f;
  }
  float m = -INFINITY, l = 0.f;
  int kend = len;
  if (a.causal) kend = min(kend, min(qt * 64 + 64, a.M) + (a.N - a.M));
  for (int key0 = 0; key0 < kend; key0 += 64) {
    __syncthreads();
    for (int e = threadIdx.x; e < 64 * kHD; e += 64) {
      const int r = e / kHD, d = e % kHD;
      const int j = key0 + r;
      Kt[r][d] = j < kend ? Kp[(int64_t)j * a.ks[2] + d] : 0.f;
      Vt32[r][d] = j < kend ? Vp[(int64_t)j * a.vs[2] + d] : 0.f;
    }
    __syncthreads();
    if (!qvalid) continue;
    const int nk = min(64, kend - key0);
    for (int r = 0; r < nk; ++r) {
      const int j = key0 + r;
      if (a.causal && j > qrow + (a.N - a.M)) break;
      float s = 0.f;
#pragma unroll
      for (int d = 0; d < kHD; ++d) s += qv[d] * Kt[r][d];
      const int c = deb_index(a, qrow - j);
      if (PK) s += PK[b * a.pks[0] + h * a.pks[1] + (int64_t)qrow * a.pks[2] + (int64_t)c * a.pks[3]];
      if (PQ) s += PQ[b * a.pqs[0] + h * a.pqs[1] + (int64_t)j * a.pqs[2] + (int64_t)c * a.pqs[3]];
      s *= a.c2;
      const float mn = fmaxf(m, s);
      const float alpha = exp2f(m - mn);
      const float p = exp2f(s - mn);
      l = l * alpha + p;
#pragma unroll
      for (int d = 0; d < kHD; ++d) acc[d] = acc[d] * alpha + p * Vt32[r][d];
      m = mn;
    }
  }
  if (!qstore) return;
  float* op = reinterpret_cast<float*>(a.o) + b * a.os[0] + h * a.os[1] + (int64_t)qrow * a.os[2];
  const float inv = (qvalid && l > 0.f) ? 1.0f / l : 0.f;
#pragma unroll
  for (int d = 0; d < kHD; ++d) op[d] = acc[d] * inv;
}


// ---------------------------------------------------------------------------
// Fused form: c2p / p2c computed in the kernel from the per-head projections
// key_rel = Kr [2S, 64] and query_rel = Qr [2S, 64]:
//   c2p(i,j) = q_i . Kr[c(i-j)],   p2c(i,j) = k_j . Qr[c(i-j)].
// For a workgroup (128 rows from q0) and a key tile (64 keys from key0) the
// indices c(i-j) lie in a window of at most 191 rows starting at
// wbase = c(q0 - key0 - 63) (c is monotone). Per tile:
//   P^T[idx][key] = Qr[wbase+idx] . K[key]  (MFMA, shared, LDS "PT")
//   C^T[idx][row] = Kr[cw+idx] . q[row]     (MFMA, per wave, 96-row window)
// then every score gathers C[c - cw][row] and PT[key][c - wbase].
// ---------------------------------------------------------------------------
constexpr int kPwin = 192;              // WG window rows (6 blocks of 32)
constexpr int kCwin = 96;               // wave window rows (3 blocks of 32)
constexpr int kPTs = kPwin + 8;         // PT row stride (u16), 8B-aligned rows
constexpr int kCs = 33;                 // C row stride (u16): conflict-free reads
constexpr int kPTElems = kBN * kPTs;
constexpr int kCElems = kCwin * kCs;    // per wave

// Rel-table MFMA operand: row r (clamped into the table), d chunk of lane.
__device__ inline u32x4_t rel_row(const uint16_t* __restrict__ base, int64_t rs, int r, int rmax, int ds) {
  const int h = (threadIdx.x & 63) >> 5;
  r = min(r, rmax);
  return *reinterpret_cast<const u32x4_t*>(base + (int64_t)r * rs + ds * 16 + 8 * h);
}

template <typename E>
__global__ __launch_bounds__(256, 2) void deberta_fused_kernel(DebArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  uint16_t* Ks = reinterpret_cast<uint16_t*>(smem);
  uint16_t* Vt = Ks + kKsElems;
  uint16_t* PT = Vt + kVtElems;
  uint16_t* Cw0 = PT + kPTElems;
  int16_t* lut = reinterpret_cast<int16_t*>(Cw0 + 4 * kCElems);

  const int nqt = (a.M + kBM - 1) / kBM;
  const int work = xcd_remap(blockIdx.x, gridDim.x);
  const int qt = work % nqt;
  const int bh = work / nqt;
  const int h = bh % a.H, b = bh / a.H;
  const int q0 = qt * kBM;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6, hl = lane >> 5, cl = lane & 31;
  const int len = a.seq_lengths ? min(max(a.seq_lengths[b], 0), a.N) : a.N;
  const int qrow = q0 + w * 32 + cl;
  const bool qstore = qrow < a.M;
  const bool qvalid = qrow < min(len, a.M);
  uint16_t* orow = reinterpret_cast<uint16_t*>(a.o) + b * a.os[0] + h * a.os[1] + (int64_t)qrow * a.os[2];
  const int kend = len;
  const int kt_end = (max(kend, 0) + kBN - 1) / kBN;
  if (q0 >= len || kt_end == 0) {
    if (qstore) {
      f32x16_t z = {};
      store_out<E>(orow, z, z, 0.f);
    }
    return;
  }
  const int dmin = q0 - (kt_end * kBN - 1);
  for (int e = t; e < a.lut_len; e += 256) lut[e] = (int16_t)deb_index(a, dmin + e);

  const uint16_t* Qp = reinterpret_cast<const uint16_t*>(a.q) + b * a.qs[0] + h * a.qs[1];
  const uint16_t* Kp = reinterpret_cast<const uint16_t*>(a.k) + b * a.ks[0] + h * a.ks[1];
  const uint16_t* Vp = reinterpret_cast<const uint16_t*>(a.v) + b * a.vs[0] + h * a.vs[1];
  const uint16_t* Kr = a.kr ? reinterpret_cast<const uint16_t*>(a.kr) + h * a.krs[0] : nullptr;
  const uint16_t* Qr = a.qr ? reinterpret_cast<const uint16_t*>(a.qr) + h * a.qrs[0] : nullptr;
  const int rmax = 2 * a.span - 1;
  uint16_t* Cw = Cw0 + w * kCElems;

  u32x4_t qf[4];
  load_q(qf, Qp + (int64_t)qrow * a.qs[2], qvalid);
  float m = -INFINITY, l = 0.f;
  f32x16_t o0 = {}, o1 = {};
  const int lut_lane = qrow - 4 * hl - dmin;
  const int qw0 = q0 + w * 32;

  KVStage st;
  kv_load(st, Kp, a.ks[2], Vp, a.vs[2], 0, kend);
  __syncthreads();  // lut ready
  for (int kt = 0; kt < kt_end; ++kt) {
    const int key0 = kt * kBN;
    kv_store(st, Ks, Vt);
    const int wbase = lut[q0 - key0 - 63 - dmin];
    const int whi = lut[min(q0 + kBM - 1, a.M - 1) - key0 - dmin];
    const int cw = lut[qw0 - key0 - 63 - dmin];
    const int cwhi = lut[min(qw0 + 31, a.M - 1) - key0 - dmin];
    __syncthreads();  // K tile in LDS
    if (kt + 1 < kt_end) kv_load(st, Kp, a.ks[2], Vp, a.vs[2], (kt + 1) * kBN, kend);

    // ---- P^T blocks (WG-shared): wave w takes blocks w, w+4, w+8 of 6x2
    if (Qr) {
      const int nbp = (whi - wbase) / 32 + 1;
#pragma unroll
      for (int bi = 0; bi < 3; ++bi) {
        const int blk = w + 4 * bi;
        const int ib = blk >> 1, kb = blk & 1;
        if (ib < nbp) {
          f32x16_t acc = {};
#pragma unroll
          for (int ds = 0; ds < 4; ++ds) {
            const u32x4_t av = rel_row(Qr, a.qrs[1], wbase + ib * 32 + cl, rmax, ds);
            const u32x4_t bv = *reinterpret_cast<const u32x4_t*>(Ks + (kb * 32 + cl) * kKsStride + ds * 16 + 8 * hl);
            acc = E::mfma32(av, bv, acc);
          }
          // lane holds key kb*32+cl, idx ib*32 + 8*(r/4) + 4*hl + r%4
          uint16_t* prow = PT + (kb * 32 + cl) * kPTs + ib * 32 + 4 * hl;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            u32x2_t wv;
            wv[0] = E::pack2(acc[4 * j], acc[4 * j + 1]);
            wv[1] = E::pack2(acc[4 * j + 2], acc[4 * j + 3]);
            *reinterpret_cast<u32x2_t*>(prow + 8 * j) = wv;
          }
        }
      }
    }
    // ---- C^T for this wave's 32 rows over [cw, cw + 96)
    if (Kr) {
      const int nbc = (cwhi - cw) / 32 + 1;
#pragma unroll
      for (int ib = 0; ib < 3; ++ib) {
        if (ib < nbc) {
          f32x16_t acc = {};
#pragma unroll
          for (int ds = 0; ds < 4; ++ds) {
            const u32x4_t av = rel_row(Kr, a.krs[1], cw + ib * 32 + cl, rmax, ds);
            acc = E::mfma32(av, qf[ds], acc);
          }
          // lane holds row cl, idx ib*32 + 8*(r/4) + 4*hl + r%4
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int idx = ib * 32 + 8 * (r >> 2) + 4 * hl + (r & 3);
            Cw[idx * kCs + cl] = E::from_f32(acc[r]);
          }
        }
      }
    }
    __syncthreads();  // PT and C complete

    f32x16_t s0, s1;
    qk_tile<E>(Ks, qf, s0, s1);
    const int16_t* lp = lut + (lut_lane - key0);
    map_scores(s0, s1, [&](int e, float v) {
      const int xk = x_key(e, 0);
      const int c = lp[-xk];
      float bias = 0.f;
      if (Kr) bias += E::to_f32(Cw[(c - cw) * kCs + cl]);
      if (Qr) bias += E::to_f32(PT[(xk + 4 * hl) * kPTs + (c - wbase)]);
      v += bias;
      return (key0 + xk + 4 * hl >= kend) ? -INFINITY : v;
    });
    u32x4_t p[4];
    softmax_tile<E>(s0, s1, a.c2, m, l, o0, o1, p);
    pv_tile<E>(Vt, p, o0, o1);
    __syncthreads();
  }
  const float l_tot = half_swap_sum(l);
  if (qstore) {
    if (!qvalid) {
      f32x16_t z = {};
      store_out<E>(orow, z, z, 0.f);
    } else {
      store_out<E>(orow, o0, o1, l_tot);
    }
  }
}

// fp32 fused: one thread per query row, c2p/p2c as dot products.
__global__ __launch_bounds__(64) void deberta_fused_f32_kernel(DebArgs a) {
  __shared__ float Kt[64][kHD + 1];
  __shared__ float Vt32[64][kHD + 1];
  const int nqt = (a.M + 63) / 64;
  const int qt = blockIdx.x % nqt;
  const int bh = blockIdx.x / nqt;
  const int h = bh % a.H, b = bh / a.H;
  const int qrow = qt * 64 + threadIdx.x;
  const int len = a.seq_lengths ? min(max(a.seq_lengths[b], 0), a.N) : a.N;
  const bool qstore = qrow < a.M;
  const bool qvalid = qrow < min(len, a.M);
  const float* Qp = reinterpret_cast<const float*>(a.q) + b * a.qs[0] + h * a.qs[1];
  const float* Kp = reinterpret_cast<const float*>(a.k) + b * a.ks[0] + h * a.ks[1];
  const float* Vp = reinterpret_cast<const float*>(a.v) + b * a.vs[0] + h * a.vs[1];
  const float* Kr = a.kr ? reinterpret_cast<const float*>(a.kr) + h * a.krs[0] : nullptr;
  const float* Qr = a.qr ? reinterpret_cast<const float*>(a.qr) + h * a.qrs[0] : nullptr;
  float qv[kHD], acc[kHD];
#pragma unroll
  for (int d = 0; d < kHD; ++d) {
    qv[d] = qvalid ? Qp[(int64_t)qrow * a.qs[2] + d] : 0.f;
    acc[d] = 0.f;
  }
  float m = -INFINITY, l = 0.f;
  for (int key0 = 0; key0 < len; key0 += 64) {
    __syncthreads();
    for (int e = threadIdx.x; e < 64 * kHD; e += 64) {
      const int r = e / kHD, d = e % kHD;
      const int j = key0 + r;
      Kt[r][d] = j < len ? Kp[(int64_t)j * a.ks[2] + d] : 0.f;
      Vt32[r][d] = j < len ? Vp[(int64_t)j * a.vs[2] + d] : 0.f;
    }
    __syncthreads();
    if (!qvalid) continue;
    const int nk = min(64, len - key0);
    for (int r = 0; r < nk; ++r) {
      const int j = key0 + r;
      const int c = deb_index(a, qrow - j);
      float s = 0.f;
#pragma unroll
      for (int d = 0; d < kHD; ++d) {
        float kk = Kt[r][d];
        if (Qr) s += kk * Qr[(int64_t)c * a.qrs[1] + d];
        if (Kr) s += qv[d] * Kr[(int64_t)c * a.krs[1] + d];
        s += qv[d] * kk;
      }
      s *= a.c2;
      const float mn = fmaxf(m, s);
      const float alpha = exp2f(m - mn);
      const float p = exp2f(s - mn);
      l = l * alpha + p;
#pragma unroll
      for (int d = 0; d < kHD; ++d) acc[d] = acc[d] * alpha + p * Vt32[r][d];
      m = mn;
    }
  }
  if (!qstore) return;
  float* op = reinterpret_cast<float*>(a.o) + b * a.os[0] + h * a.os[1] + (int64_t)qrow * a.os[2];
  const float inv = (qvalid && l > 0.f) ? 1.0f / l : 0.f;
#pragma unroll
  for (int d = 0; d < kHD; ++d) op[d] = acc[d] * inv;
}

}  // namespace vfk

using namespace vfk;

static int check_bhld_deb(const vfk_tensor* t, const char* name, int dtype) {
  int rc = check_tensor(t, name, 4);
  if (rc) return rc;
  if (t->dtype != dtype) return set_error(VFK_ERR_INVALID, "%s: dtype differs from q", name);
  if (t->size[3] != kHD)
    return set_error(VFK_ERR_UNSUPPORTED, "%s: head_dim %lld (only 64 is built)", name,
                     (long long)t->size[3]);
  if (t->stride[3] != 1) return set_error(VFK_ERR_INVALID, "%s: head_dim must be contiguous", name);
  if (dtype != VFK_F32 && (!aligned16(t->data) || t->stride[0] % 8 || t->stride[1] % 8 || t->stride[2] % 8))
    return set_error(VFK_ERR_INVALID, "%s: rows must be 16-byte aligned", name);
  return VFK_OK;
}

static int setup_common(DebArgs& a, const vfk_tensor* q, const vfk_tensor* k, const vfk_tensor* v,
                        const int32_t* seq_lengths, float sm_scale, int position_buckets,
                        int max_relative_distance, int use_log_bucket, vfk_tensor* out,
                        const char* name) {
  int rc = check_tensor(q, "q", 4);
  if (rc) return rc;
  const int dt = q->dtype;
  if ((rc = check_bhld_deb(q, "q", dt)) || (rc = check_bhld_deb(k, "k", dt)) ||
      (rc = check_bhld_deb(v, "v", dt)) || (rc = check_bhld_deb(out, "out", dt)))
    return rc;
  const int64_t B = q->size[0], H = q->size[1], M = q->size[2], N = k->size[2];
  if (k->size[0] != B || k->size[1] != H || v->size[0] != B || v->size[1] != H || v->size[2] != N)
    return set_error(VFK_ERR_INVALID, "%s: q/k/v shapes disagree", name);
  for (int i = 0; i < 4; ++i)
    if (out->size[i] != q->size[i]) return set_error(VFK_ERR_INVALID, "%s: out must match q", name);
  if (M > 32767 || N > 32767 || B * H > (1 << 24))
    return set_error(VFK_ERR_UNSUPPORTED, "%s: sizes too large", name);
  if (!(sm_scale > 0.f) || !isfinite(sm_scale))
    return set_error(VFK_ERR_UNSUPPORTED, "%s: sm_scale must be > 0", name);
  a.q = q->data; a.k = k->data; a.v = v->data; a.o = out->data;
  for (int i = 0; i < 4; ++i) {
    a.qs[i] = q->stride[i]; a.ks[i] = k->stride[i]; a.vs[i] = v->stride[i]; a.os[i] = out->stride[i];
  }
  a.B = (int)B; a.H = (int)H; a.M = (int)M; a.N = (int)N;
  a.seq_lengths = seq_lengths;
  a.c2 = sm_scale * VFK_LOG2E;
  // flash_deberta_attention.py:323, :366-368
  a.span = position_buckets > 0 ? position_buckets : max_relative_distance;
  const int nb = position_buckets > 0 ? position_buckets : max_relative_distance * 2;
  const int maxd = max_relative_distance > 0 ? max_relative_distance : 512;
  a.log_bucket = use_log_bucket ? 1 : 0;
  if (a.span <= 0) return set_error(VFK_ERR_INVALID, "%s: att_span must be > 0", name);
  if (a.log_bucket) {
    const int max_abs = (int)(M > N ? M : N);
    if ((rc = build_deberta_step(nb, maxd, max_abs, a.span, &a.step))) return rc;
  }
  return VFK_OK;
}

static int check_pos(const vfk_tensor* p, const char* name, const DebArgs& a, int rows, int dt) {
  int rc = check_tensor(p, name, 4);
  if (rc) return rc;
  if (p->dtype != dt) return set_error(VFK_ERR_INVALID, "%s: dtype differs from q", name);
  if (p->size[0] != a.B || p->size[1] != a.H || p->size[2] != rows || p->size[3] < 2 * a.span)
    return set_error(VFK_ERR_INVALID, "%s: expected [B, H, %d, >= %d]", name, rows, 2 * a.span);
  return VFK_OK;
}

extern "C" int vfk_flash_deberta_fwd(const vfk_tensor* q, const vfk_tensor* k, const vfk_tensor* v,
                                     const int32_t* seq_lengths, const vfk_tensor* pos_key,
                                     const vfk_tensor* pos_query, int32_t causal, float sm_scale,
                                     int32_t position_buckets, int32_t max_relative_distance,
                                     int32_t use_log_bucket, vfk_tensor* out, void* stream) {
  DebArgs a = {};
  int rc = setup_common(a, q, k, v, seq_lengths, sm_scale, position_buckets, max_relative_distance,
                        use_log_bucket, out, "vfk_flash_deberta_fwd");
  if (rc) return rc;
  a.causal = causal ? 1 : 0;
  if (present(pos_key)) {
    if ((rc = check_pos(pos_key, "pos_key", a, a.M, q->dtype))) return rc;
    a.pk = pos_key->data;
    for (int i = 0; i < 4; ++i) a.pks[i] = pos_key->stride[i];
  }
  if (present(pos_query)) {
    if ((rc = check_pos(pos_query, "pos_query", a, a.N, q->dtype))) return rc;
    a.pq = pos_query->data;
    for (int i = 0; i < 4; ++i) a.pqs[i] = pos_query->stride[i];
  }
  if (a.B == 0 || a.H == 0 || a.M == 0) return VFK_OK;
  hipStream_t st = (hipStream_t)stream;
  if (q->dtype == VFK_F32) {
    const int nqt = ceil_div(a.M, 64);
    hipLaunchKernelGGL(deberta_gather_f32_kernel, dim3((unsigned)(nqt * a.B * a.H)), dim3(64), 0, st, a);
    return launch_status("vfk_flash_deberta_fwd");
  }
  const int ntk = ceil_div(a.N, kBN);
  a.lut_len = ntk * kBN + kBM;
  const size_t lds = (size_t)(kKsElems + kVtElems) * 2 + (size_t)a.lut_len * 2;
  if (lds > 160 * 1024) return set_error(VFK_ERR_UNSUPPORTED, "vfk_flash_deberta_fwd: N too large");
  const int nqt = ceil_div(a.M, kBM);
  dim3 grid((unsigned)(nqt * a.B * a.H));
  if (q->dtype == VFK_BF16)
    hipLaunchKernelGGL(deberta_gather_kernel<BF16>, grid, dim3(256), lds, st, a);
  else
    hipLaunchKernelGGL(deberta_gather_kernel<F16>, grid, dim3(256), lds, st, a);
  return launch_status("vfk_flash_deberta_fwd");
}

extern "C" int vfk_deberta_fused_fwd(const vfk_tensor* q, const vfk_tensor* k, const vfk_tensor* v,
                                     const int32_t* seq_lengths, const vfk_tensor* key_rel,
                                     const vfk_tensor* query_rel, float sm_scale,
                                     int32_t position_buckets, int32_t max_relative_distance,
                                     int32_t use_log_bucket, vfk_tensor* out, void* stream) {
  DebArgs a = {};
  int rc = setup_common(a, q, k, v, seq_lengths, sm_scale, position_buckets, max_relative_distance,
                        use_log_bucket, out, "vfk_deberta_fused_fwd");
  if (rc) return rc;
  if (a.M != a.N)
    return set_error(VFK_ERR_UNSUPPORTED, "vfk_deberta_fused_fwd: self-attention only (M == N)");
  const vfk_tensor* rel[2] = {key_rel, query_rel};
  const char* names[2] = {"key_rel", "query_rel"};
  for (int i = 0; i < 2; ++i) {
    if (!present(rel[i])) continue;
    const vfk_tensor* r = rel[i];
    if ((rc = check_tensor(r, names[i], 3))) return rc;
    if (r->dtype != q->dtype) return set_error(VFK_ERR_INVALID, "%s: dtype differs from q", names[i]);
    if (r->size[0] != a.H || r->size[1] < 2 * a.span || r->size[2] != kHD || r->stride[2] != 1)
      return set_error(VFK_ERR_INVALID, "%s: expected [H, >= %d, 64] with unit last stride", names[i],
                       2 * a.span);
    if (q->dtype != VFK_F32 && (!aligned16(r->data) || r->stride[0] % 8 || r->stride[1] % 8))
      return set_error(VFK_ERR_INVALID, "%s: rows must be 16-byte aligned", names[i]);
    if (i == 0) { a.kr = r->data; a.krs[0] = r->stride[0]; a.krs[1] = r->stride[1]; }
    else { a.qr = r->data; a.qrs[0] = r->stride[0]; a.qrs[1] = r->stride[1]; }
  }
  if (a.B == 0 || a.H == 0 || a.M == 0) return VFK_OK;
  hipStream_t st = (hipStream_t)stream;
  if (q->dtype == VFK_F32) {
    const int nqt = ceil_div(a.M, 64);
    hipLaunchKernelGGL(deberta_fused_f32_kernel, dim3((unsigned)(nqt * a.B * a.H)), dim3(64), 0, st, a);
    return launch_status("vfk_deberta_fused_fwd");
  }
  const int ntk = ceil_div(a.N, kBN);
  a.lut_len = ntk * kBN + kBM;
  const size_t lds = (size_t)(kKsElems + kVtElems + kPTElems + 4 * kCElems) * 2 + (size_t)a.lut_len * 2;
  if (lds > 160 * 1024) return set_error(VFK_ERR_UNSUPPORTED, "vfk_deberta_fused_fwd: N too large");
  const int nqt = ceil_div(a.M, kBM);
  dim3 grid((unsigned)(nqt * a.B * a.H));
  if (q->dtype == VFK_BF16)
    hipLaunchKernelGGL(deberta_fused_kernel<BF16>, grid, dim3(256), lds, st, a);
  else
    hipLaunchKernelGGL(deberta_fused_kernel<F16>, grid, dim3(256), lds, st, a);
  return launch_status("vfk_deberta_fused_fwd");
}
