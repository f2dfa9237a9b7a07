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
  int rel_cm;                       // both tables chunk-major [H][8][2S][8] (head stride in [0])
  StepFn step;                      // |bucket| as a function of |d| (log mode)
  int unit;                         // c(d) moves by at most 1 per unit of d
  int lin_lo, lin_hi;               // c(d) = d + span for lin_lo <= d <= lin_hi
  // packed sequences (fused kernel; nullptr: the padded batch): "batch" b is
  // sequence b, tokens cu[b] .. cu[b + 1] - 1 of [T, H, D] tensors (strides
  // [.][1] = head, [.][2] = token); M = N = the longest sequence
  const int32_t* cu;
};

__host__ __device__ inline int deb_index(const DebArgs& a, int d) {
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
  float m = -INFINITY;
  RowSumMfma<E> l;
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
  const float l_tot = l.total();
  if (qstore) {
    if (!qvalid) {
      f32x16_t z = {};
      store_out<E>(orow, z, z, 0.f);
    } else {
      store_out<E>(orow, o0, o1, l_tot);
    }
  }
}

// Staged form of deberta_gather_kernel for row-contiguous pos tensors. The
// gather above issues two 2-byte loads per score, spread over 32 rows per
// instruction. Here each key tile first copies, with 16-byte loads, the
// column windows it needs into LDS: c(i - j) is non-decreasing in i - j with
// steps of at most 1, so the 64 keys of a tile meet at most 64 consecutive
// pos_key columns of a query row, and the 128 query rows of the workgroup
// meet at most 128 consecutive pos_query columns of a key row. Windows start
// on an 8-column boundary (kPkW = 64 + 8, kPqW = 128 + 8) and are clamped
// into [0, 2S). The scores then read their biases from LDS.
constexpr int kPkW = kBN + 8;        // staged pos_key columns per query row
constexpr int kPqW = kBM + 8;        // staged pos_query columns per key row
constexpr int kPkChunks = kPkW / 8;  // 16-byte chunks per staged row
constexpr int kPqChunks = kPqW / 8;

__host__ __device__ constexpr size_t deb_staged_lds(int lut_len) {
  return (size_t)(kKsElems + kVtElems + kBM * kPkW + kBN * kPqW) * 2 + (size_t)(kBM + kBN) * 4 +
         (size_t)lut_len * 2;
}

template <typename E, bool PK, bool PQ>
__global__ __launch_bounds__(256, 2) void deberta_gather_staged_kernel(DebArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  uint16_t* Ks = reinterpret_cast<uint16_t*>(smem);
  uint16_t* Vt = Ks + kKsElems;
  uint16_t* PKs = Vt + kVtElems;                            // [kBM][kPkW]
  uint16_t* PQs = PKs + kBM * kPkW;                         // [kBN][kPqW]
  int* pko = reinterpret_cast<int*>(PQs + kBN * kPqW);      // [kBM] row * kPkW - window start
  int* pqo = pko + kBM;                                     // [kBN] row * kPqW - window start
  int16_t* lut = reinterpret_cast<int16_t*>(pqo + kBN);    // c(i - j)

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

  int kend = len;
  if (a.causal) kend = min(kend, min(q0 + kBM, a.M) + (a.N - a.M));
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
  const uint16_t* PKp = PK ? reinterpret_cast<const uint16_t*>(a.pk) + b * a.pks[0] + h * a.pks[1] : nullptr;
  const uint16_t* PQp = PQ ? reinterpret_cast<const uint16_t*>(a.pq) + b * a.pqs[0] + h * a.pqs[1] : nullptr;
  const int span2 = 2 * a.span;

  u32x4_t qf[4];
  load_q(qf, Qp + (int64_t)qrow * a.qs[2], qvalid);
  float m = -INFINITY;
  RowSumMfma<E> l;
  f32x16_t o0 = {}, o1 = {};
  const int lut_lane = qrow - 4 * hl - dmin;
  const int prow = w * 32 + (lane & 31);  // this lane's staged pos_key row

  KVStage st;
  kv_load(st, Kp, a.ks[2], Vp, a.vs[2], 0, kend);
  __syncthreads();  // lut ready
  for (int kt = 0; kt < kt_end; ++kt) {
    const int key0 = kt * kBN;
    // pos windows of this tile: global -> registers (clamped rows and
    // chunks, so every load is unconditional; surplus chunks are not stored)
    u32x4_t pkv[5], pqv[5];
#pragma unroll
    for (int u = 0; u < 5 && PK; ++u) {
      const int c = min(t + 256 * u, kBM * kPkChunks - 1);
      const int r = c / kPkChunks, j = c - r * kPkChunks;
      const int cmin = lut[q0 + r - key0 - (kBN - 1) - dmin];
      const int start = min(cmin & ~7, span2 - kPkW);
      pkv[u] = *reinterpret_cast<const u32x4_t*>(PKp + (int64_t)min(q0 + r, a.M - 1) * a.pks[2] +
                                                 start + 8 * j);
    }
#pragma unroll
    for (int u = 0; u < 5 && PQ; ++u) {
      const int c = min(t + 256 * u, kBN * kPqChunks - 1);
      const int r = c / kPqChunks, j = c - r * kPqChunks;
      const int cmin = lut[q0 - key0 - r - dmin];
      const int start = min(cmin & ~7, span2 - kPqW);
      pqv[u] = *reinterpret_cast<const u32x4_t*>(PQp + (int64_t)min(key0 + r, a.N - 1) * a.pqs[2] +
                                                 start + 8 * j);
    }
    kv_store(st, Ks, Vt);
    if (PK && t < kBM) {
      const int cmin = lut[q0 + t - key0 - (kBN - 1) - dmin];
      pko[t] = t * kPkW - min(cmin & ~7, span2 - kPkW);
    } else if (PQ && t >= kBM && t < kBM + kBN) {
      const int r = t - kBM;
      const int cmin = lut[q0 - key0 - r - dmin];
      pqo[r] = r * kPqW - min(cmin & ~7, span2 - kPqW);
    }
    __syncthreads();
    if (kt + 1 < kt_end) kv_load(st, Kp, a.ks[2], Vp, a.vs[2], (kt + 1) * kBN, kend);

    f32x16_t s0, s1;
    qk_tile<E>(Ks, qf, s0, s1);
#pragma unroll
    for (int u = 0; u < 5; ++u) {
      const int c = t + 256 * u;
      if (PK && c < kBM * kPkChunks) {
        const int r = c / kPkChunks, j = c - r * kPkChunks;
        *reinterpret_cast<u32x4_t*>(PKs + r * kPkW + 8 * j) = pkv[u];
      }
      if (PQ && c < kBN * kPqChunks) {
        const int r = c / kPqChunks, j = c - r * kPqChunks;
        *reinterpret_cast<u32x4_t*>(PQs + r * kPqW + 8 * j) = pqv[u];
      }
    }
    __syncthreads();

    const int16_t* lp = lut + (lut_lane - key0);
    const uint16_t* pkr = PKs + (PK ? pko[prow] : 0);
    map_scores(s0, s1, [&](int e, float v) {
      const int xk = x_key(e, 0);  // key - key0 - 4*hl
      const int kr = xk + 4 * hl;
      const int key = key0 + kr;
      const int c = lp[-xk];
      float bias = 0.f;  // summed as the per-score gather does: bit-equal
      if (PK) bias += E::to_f32(pkr[c]);
      if (PQ) bias += E::to_f32(PQs[pqo[kr] + c]);
      v += bias;
      return (key >= kend || (a.causal && key > qrow + (a.N - a.M))) ? -INFINITY : v;
    });
    u32x4_t p[4];
    softmax_tile<E>(s0, s1, a.c2, m, l, o0, o1, p);
    pv_tile<E>(Vt, p, o0, o1);
    __syncthreads();
  }
  const float l_tot = l.total();
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
// wlo = c(q0 - key0 - 63) (c is monotone); for one wave's 32 rows, in a window
// of at most 95 rows from cwl = c(qw0 - key0 - 63). Per tile:
//   P^T[key][idx] = Qr[wlo+idx] . K[key]  (MFMA, shared by the workgroup:
//                   wave w computes index blocks w and w + 4 for both key
//                   blocks, so every Qr row is fetched once)
//   C[row][idx]   = Kr[cwl+idx] . q[row]  (MFMA, per wave)
// only over the 32-row index blocks that hold a used c (fewer where the log
// buckets compress distances), both rounded to the element type (the
// precision of the reference's pos_key / pos_query tensors) and written to
// LDS as 8-byte runs; every score then adds C[row][c - cwl] and
// P^T[key][c - wlo], with c read from a table of 2 c(d) over the
// workgroup's relative positions. The Qr and Kr operands of tile i + 1 are
// fetched into registers during tile i.
//
// Step for key tile i (K(i), and the Qr and Kr operands, resident since the
// previous step):
//   direct load V(i); P^T and C blocks; S = K(i) Q^T; barrier;
//   direct load K(i+1), Qr and Kr loads of tile i + 1; bias gathers; online
//   softmax; O += V(i)^T P; barrier (K(i+1) landed, V / P^T / C free again)
// ---------------------------------------------------------------------------
constexpr int kPTs = 204;               // P^T row stride (u16): 8-byte rows, odd dword pairs
constexpr int kCs = 100;                // C row stride (u16): 8-byte rows
constexpr int kPTElems = kBN * kPTs;
constexpr int kCElems = 32 * kCs;       // per wave
constexpr int kFusedStaticLds = (3 * kTileElems + kPTElems + 4 * kCElems) * 2;

// Rel-table MFMA operand (rows row0 .. row0 + 31, k-step ds) through a buffer
// resource over one head's table. Row-major [2S][64] rows: lane byte offset
// voff = row-in-block * rs2 + 16 h, soff = row0 * rs2, dsb = 32, and each
// wave load touches 32 rows' lines. Chunk-major [8][2S][8] (chunk q = k / 8
// holds 16 bytes of every row): voff = (h * 2S + row-in-block) * 16,
// soff = row0 * 16, dsb = 2 * 2S * 16, so a wave load reads two contiguous
// 512-byte runs whatever row0 is. Rows past the table read as zeros, or (chunk
// major) as rows of the next chunk; their products are never used.
struct RelSrc {
  rsrc_t r;
  int lane, rowb, dsb;  // lane byte offset, bytes per row step, bytes per k-step
};

__device__ inline u32x4_t rel_ld(const RelSrc& t, int row0, int ds) {
  return __builtin_bit_cast(u32x4_t,
                            __builtin_amdgcn_raw_buffer_load_b128(t.r, t.lane, row0 * t.rowb + ds * t.dsb, 0));
}

__device__ inline RelSrc rel_src(const void* base, int64_t hstride, int64_t rs, int cm, int span, int cl,
                                 int hl) {
  RelSrc t;
  const int rowb = cm ? 16 : (int)rs * 2;
  t.r = uniform_rsrc(base ? reinterpret_cast<const uint16_t*>(base) + hstride : nullptr,
                     base ? 2 * span * (cm ? 128 : rowb) : 0);
  t.lane = cm ? (hl * 2 * span + cl) * 16 : cl * rowb + 16 * hl;
  t.rowb = rowb;
  t.dsb = cm ? 64 * span : 32;
  return t;
}

// Writes the lane's four 4-element runs of an MFMA output block (rows
// 8j + 4h .. +3 of the block, this lane's column) to a row-major array:
// run j lands at byte offset off + 16 j.
template <typename E>
__device__ inline void store_runs(uint16_t* __restrict__ base, int off, const f32x16_t& acc) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    u32x2_t wv;
    wv[0] = E::pack2(acc[4 * j], acc[4 * j + 1]);
    wv[1] = E::pack2(acc[4 * j + 2], acc[4 * j + 3]);
    *reinterpret_cast<u32x2_t*>(reinterpret_cast<char*>(base) + off + 16 * j) = wv;
  }
}

// C blocks ib < NB of one wave: C[row][idx] = Kr[cwl + idx] . q[row].
template <int NB>
__device__ inline void c_loads(const RelSrc& kr, int cwl, u32x4_t (&ca)[3][4]) {
#pragma unroll
  for (int ib = 0; ib < NB; ++ib)
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) ca[ib][ds] = rel_ld(kr, cwl + ib * 32, ds);
}
template <typename E, int NB>
__device__ inline void c_blocks(const u32x4_t (&ca)[3][4], const u32x4_t (&qf)[4],
                                uint16_t* __restrict__ Cm, int c_row) {
  f32x16_t acc[NB] = {};
#pragma unroll
  for (int ds = 0; ds < 4; ++ds)
#pragma unroll
    for (int ib = 0; ib < NB; ++ib) acc[ib] = E::mfma32(ca[ib][ds], qf[ds], acc[ib]);
  // lane holds row cl, indices ib*32 + 8j + 4h + 0..3
  const int hl = (threadIdx.x & 63) >> 5;
#pragma unroll
  for (int ib = 0; ib < NB; ++ib) store_runs<E>(Cm, c_row + (ib * 32 + 4 * hl) * 2, acc[ib]);
}

template <typename E, bool C2P, bool P2C>
__global__ __launch_bounds__(256, 2) void deberta_fused_kernel(DebArgs a) {
  __shared__ __align__(16) uint16_t K0[kTileElems];
  __shared__ __align__(16) uint16_t K1[kTileElems];
  __shared__ __align__(16) uint16_t Vs[kTileElems];
  __shared__ __align__(16) uint16_t PT[P2C ? kPTElems : 8];
  __shared__ __align__(16) uint16_t Cm[C2P ? 4 * kCElems : 8];
  extern __shared__ __align__(16) unsigned char smem[];
  int16_t* lut = reinterpret_cast<int16_t*>(smem);  // 2 c(dmin + e)

  const int nqt = (a.M + kBM - 1) / kBM;
  const int work = xcd_remap(blockIdx.x, gridDim.x);
  const int qt = work % nqt;
  const int bh = work / nqt;
  const int h = bh % a.H, b = bh / a.H;
  const int q0 = qt * kBM;
  const int t = threadIdx.x, lane = t & 63, hl = lane >> 5, cl = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);
  // rows of this (batch, head) or sequence and their offsets in q, k, v, o;
  // packed sequences have no rows past their length to write
  int len, mrows;
  int64_t qb, kb, vb, ob;
  if (a.cu) {
    const int tok0 = a.cu[b];
    const int nfull = a.cu[b + 1] - tok0;
    len = mrows = min(max(nfull, 0), a.N);
    qb = (int64_t)tok0 * a.qs[2]; kb = (int64_t)tok0 * a.ks[2];
    vb = (int64_t)tok0 * a.vs[2]; ob = (int64_t)tok0 * a.os[2];
    // rows past max_seqlen (a.N) are not computed: the last query tile
    // writes them as zeros
    if (qt == nqt - 1 && nfull > len)
      zero_rows_d64(reinterpret_cast<uint16_t*>(a.o) + ob + h * a.os[1], a.os[2], len, nfull);
  } else {
    len = a.seq_lengths ? min(max(a.seq_lengths[b], 0), a.N) : a.N;
    mrows = a.M;
    qb = b * a.qs[0]; kb = b * a.ks[0]; vb = b * a.vs[0]; ob = b * a.os[0];
  }
  const int qw0 = q0 + w * 32;
  const int qrow = qw0 + cl;
  const bool qstore = qrow < mrows;
  const bool qvalid = qrow < min(len, mrows);
  uint16_t* orow = reinterpret_cast<uint16_t*>(a.o) + ob + h * a.os[1] + (int64_t)qrow * a.os[2];
  if (q0 >= len) {  // every row of the tile is padding (len may be 0): zeros
    if (qstore) {
      f32x16_t z = {};
      store_out<E>(orow, z, z, 0.f);
    }
    return;
  }
  const int kt_end = (len + kBN - 1) / kBN;
  const int dmin = q0 - (kt_end * kBN - 1);
  for (int e = t; e < a.lut_len; e += 256) lut[e] = (int16_t)(2 * deb_index(a, dmin + e));

  const uint16_t* Qp = reinterpret_cast<const uint16_t*>(a.q) + qb + h * a.qs[1];
  TileSrc ksrc, vsrc;
  tile_src_init(ksrc, reinterpret_cast<const uint16_t*>(a.k) + kb + h * a.ks[1], (int)a.ks[2], len);
  tile_src_init(vsrc, reinterpret_cast<const uint16_t*>(a.v) + vb + h * a.vs[1], (int)a.vs[2], len);
  tile_load_buf(ksrc, 0, K0);
  const RelSrc krt = rel_src(C2P ? a.kr : nullptr, h * a.krs[0], a.krs[1], a.rel_cm, a.span, cl, hl);
  const RelSrc qrt = rel_src(P2C ? a.qr : nullptr, h * a.qrs[0], a.qrs[1], a.rel_cm, a.span, cl, hl);

  u32x4_t qf[4];
  load_q(qf, Qp + (int64_t)qrow * a.qs[2], qvalid);
  float m = -INFINITY;
  RowSumMfma<E> l;
  f32x16_t o0 = {}, o1 = {};
  KOff ko;
  VOff vo;
  k_offsets(ko);
  v_offsets(vo);
  const bool wave_on = __builtin_amdgcn_readfirstlane((int)(qw0 < min(len, mrows))) != 0;
  const int lut_lane = qrow - 4 * hl - dmin;  // table index of (qrow, key0 + 4hl) is lut_lane - key0
  const int c_row = (w * 32 + cl) * kCs * 2;  // byte offset of this lane's C row
  const int pt_row = 4 * hl * kPTs * 2;       // byte offset of P^T row 4h
  tile_barrier();  // table and K(0) ready

  // P^T blocks of this wave: index blocks w and (waves 0, 1) w + 4, both key
  // blocks; their Qr operands are loaded one tile ahead into pa
  const bool two = w < 2;
  u32x4_t pa[2][4];
  // index blocks of the workgroup's window that hold a used c (1 to 6)
  auto pt_blocks = [&](int i) {
    const int wl = __builtin_amdgcn_readfirstlane(lut[q0 - i * kBN - 63 - dmin]) >> 1;
    const int wh = __builtin_amdgcn_readfirstlane(lut[q0 + kBM - 1 - i * kBN - dmin]) >> 1;
    return (wh - wl) / 32 + 1;
  };
  auto pt_loads = [&](int i) {
    const int wl = __builtin_amdgcn_readfirstlane(lut[q0 - i * kBN - 63 - dmin]) >> 1;
    const int nbp = pt_blocks(i);
    if (w < nbp) {
#pragma unroll
      for (int ds = 0; ds < 4; ++ds) pa[0][ds] = rel_ld(qrt, wl + w * 32, ds);
    }
    if (two && w + 4 < nbp) {
#pragma unroll
      for (int ds = 0; ds < 4; ++ds) pa[1][ds] = rel_ld(qrt, wl + (w + 4) * 32, ds);
    }
  };
  if (P2C) pt_loads(0);
  // C operands (Kr rows of the wave's window), also loaded one tile ahead:
  // always 3 blocks (rows past the table read as zeros), of which the tile
  // multiplies the nbc that hold a used c
  u32x4_t ca[3][4];
  auto c_prefetch = [&](int i) {
    const int cwl = __builtin_amdgcn_readfirstlane(lut[qw0 - i * kBN - 63 - dmin]) >> 1;
    c_loads<3>(krt, cwl, ca);
  };
  if (C2P && wave_on) c_prefetch(0);

  auto step = [&](int i, const uint16_t* __restrict__ Kc, uint16_t* __restrict__ Kn) {
    ko.refresh();
    vo.refresh();
    const int key0 = i * kBN;
    tile_load_buf(vsrc, key0, Vs);
    const int wlo = __builtin_amdgcn_readfirstlane(lut[q0 - key0 - 63 - dmin]) >> 1;
    const int cwl = __builtin_amdgcn_readfirstlane(lut[qw0 - key0 - 63 - dmin]) >> 1;
    // C blocks of the wave's window that hold a used c (1 to 3)
    const int cwh = __builtin_amdgcn_readfirstlane(lut[qw0 + 31 - key0 - dmin]) >> 1;
    const int nbc = (cwh - cwl) / 32 + 1;
    const int nbp = P2C ? pt_blocks(i) : 0;
    const bool two_i = two && w + 4 < nbp;
    if (P2C && w < nbp) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        u32x4_t kf[4];
#pragma unroll
        for (int ds = 0; ds < 4; ++ds) kf[ds] = lds_at<u32x4_t>(Kc, ko.o[ds] + kb * 4096);
        // lane holds key kb*32 + cl, indices ib*32 + 8j + 4h + 0..3
        f32x16_t acc = E::mfma32(pa[0][0], kf[0], f32x16_t{});
#pragma unroll
        for (int ds = 1; ds < 4; ++ds) acc = E::mfma32(pa[0][ds], kf[ds], acc);
        store_runs<E>(PT, ((kb * 32 + cl) * kPTs + w * 32 + 4 * hl) * 2, acc);
        if (two_i) {
          acc = E::mfma32(pa[1][0], kf[0], f32x16_t{});
#pragma unroll
          for (int ds = 1; ds < 4; ++ds) acc = E::mfma32(pa[1][ds], kf[ds], acc);
          store_runs<E>(PT, ((kb * 32 + cl) * kPTs + (w + 4) * 32 + 4 * hl) * 2, acc);
        }
      }
    }
    if (C2P && wave_on) {
      if (nbc >= 3) c_blocks<E, 3>(ca, qf, Cm, c_row);
      else if (nbc == 2) c_blocks<E, 2>(ca, qf, Cm, c_row);
      else c_blocks<E, 1>(ca, qf, Cm, c_row);
    }
    f32x16_t s0, s1;
    if (wave_on) qk_tile_sw<E>(Kc, ko, qf, s0, s1);
    tile_barrier();  // V(i), P^T and C visible
    if (i + 1 < kt_end) {
      tile_load_buf(ksrc, key0 + kBN, Kn);
      if (P2C) pt_loads(i + 1);
      if (C2P && wave_on) c_prefetch(i + 1);
    }
    // the wave's relative distances qrow - key all lie where c(d) = d + span:
    // the gather addresses are a lane base plus a per-score immediate
    const bool lin = qw0 - key0 - (kBN - 1) >= a.lin_lo && qw0 + 31 - key0 <= a.lin_hi;
    if (wave_on && lin) {
      // 2 c(d) for d = qrow - key, key = key0 + 4 hl + x_key(e, 0)
      const int rel2 = 2 * (qrow - 4 * hl - key0 + a.span);
      const int cb = lds_opaque(c_row - 2 * cwl + rel2 - 2 * (kBN - 1));
      const int pb = lds_opaque(pt_row - 2 * wlo + rel2);
      map_scores(s0, s1, [&](int e, float v) {
        const int xk = x_key(e, 0);
        const int co = cb + 2 * (kBN - 1 - xk), po = pb + xk * (kPTs * 2 - 2);
        if (C2P && P2C) {
          const uint32_t cv = lds_at<uint16_t>(Cm, co);
          const uint32_t pv = lds_at<uint16_t>(PT, po);
          return E::dot2_ones(cv | (pv << 16), v);
        }
        if (C2P) v += E::to_f32(lds_at<uint16_t>(Cm, co));
        if (P2C) v += E::to_f32(lds_at<uint16_t>(PT, po));
        return v;
      });
    } else if (wave_on) {
      const int lb = lut_lane - key0;
      const int cb = lds_opaque(c_row - 2 * cwl), pb = lds_opaque(pt_row - 2 * wlo);
      map_scores(s0, s1, [&](int e, float v) {
        const int xk = x_key(e, 0);
        const int c2 = lut[lb - xk];
        if (C2P && P2C) {
          // both 16-bit terms in one register, added by one packed dot
          const uint32_t cv = lds_at<uint16_t>(Cm, cb + c2);
          const uint32_t pv = lds_at<uint16_t>(PT, pb + xk * (kPTs * 2) + c2);
          return E::dot2_ones(cv | (pv << 16), v);
        }
        if (C2P) v += E::to_f32(lds_at<uint16_t>(Cm, cb + c2));
        if (P2C) v += E::to_f32(lds_at<uint16_t>(PT, pb + xk * (kPTs * 2) + c2));
        return v;
      });
    }
    if (wave_on) {
      if (key0 + kBN > len) {
        map_scores(s0, s1, [&](int e, float v) { return key0 + x_key(e, hl) >= len ? -INFINITY : v; });
      }
      u32x4_t p[4];
      softmax_tile<E>(s0, s1, a.c2, m, l, o0, o1, p);
      pv_tile_sw<E>(Vs, vo, p, o0, o1);
    }
    tile_barrier();  // K(i+1) landed; V, P^T, C free
  };
  int i = 0;
  for (; i + 1 < kt_end; i += 2) {
    step(i, K0, K1);
    step(i + 1, K1, K0);
  }
  if (i < kt_end) step(i, K0, K1);

  const float l_tot = l.total();
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

// Chunk-major copies of up to two relative tables in one launch: thread i
// of table j moves the 16 bytes of (head h, row r, chunk c), reading them at
// row r of the [H, R, 64] source and writing them to [h][c][r] of the
// [H, 8, 2S, 8] destination; a row's eight chunks come from consecutive
// threads, so the reads are whole rows.
struct RelCmArgs {
  const uint16_t* src[2];
  int64_t ss[2][2];  // head and row strides of each source, in elements
  uint16_t* dst[2];
  int64_t ds[2];     // head stride of each destination, in elements
  int span, H;
  int64_t n0;        // 16-byte items of table 0 (H * 2S * 8); table 1 follows
};

__global__ __launch_bounds__(256) void rel_cm_kernel(RelCmArgs a) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int j = i >= a.n0 ? 1 : 0;
  const int64_t e = i - (j ? a.n0 : 0);
  if (e >= a.n0 || !a.src[j]) return;
  const int rows = 2 * a.span;
  const int c = (int)(e & 7);
  const int64_t hr = e >> 3;
  const int r = (int)(hr % rows);
  const int h = (int)(hr / rows);
  const u32x4_t v = *reinterpret_cast<const u32x4_t*>(a.src[j] + h * a.ss[j][0] + r * a.ss[j][1] + 8 * c);
  *reinterpret_cast<u32x4_t*>(a.dst[j] + h * a.ds[j] + ((int64_t)c * rows + r) * 8) = v;
}

}  // namespace vfk

using namespace vfk;

extern "C" int vfk_deberta_rel_chunk_major(const vfk_tensor* key_rel, vfk_tensor* key_out,
                                           const vfk_tensor* query_rel, vfk_tensor* query_out,
                                           int32_t att_span, void* stream) {
  const vfk_tensor* src[2] = {key_rel, query_rel};
  vfk_tensor* dst[2] = {key_out, query_out};
  const char* names[2] = {"key_rel", "query_rel"};
  if (att_span <= 0 || att_span > 8192)
    return set_error(VFK_ERR_INVALID, "deberta_rel_chunk_major: att_span %d out of range", att_span);
  RelCmArgs a = {};
  a.span = att_span;
  int dt = -1, H = -1;
  for (int j = 0; j < 2; ++j) {
    if (!present(src[j]) && !present(dst[j])) continue;
    int rc;
    if ((rc = check_tensor(src[j], names[j], 3)) || (rc = check_tensor(dst[j], "out", 4))) return rc;
    const vfk_tensor* s = src[j];
    const vfk_tensor* d = dst[j];
    if (s->dtype != VFK_BF16 && s->dtype != VFK_F16)
      return set_error(VFK_ERR_UNSUPPORTED, "deberta_rel_chunk_major: %s must be bf16 or fp16", names[j]);
    if ((dt >= 0 && s->dtype != dt) || d->dtype != s->dtype || (H >= 0 && s->size[0] != H))
      return set_error(VFK_ERR_INVALID, "deberta_rel_chunk_major: tables differ in dtype or heads");
    dt = s->dtype;
    H = (int)s->size[0];
    if (s->size[1] < 2 * att_span || s->size[2] != kHD || s->stride[2] != 1 || !aligned16(s->data) ||
        s->stride[0] % 8 || s->stride[1] % 8)
      return set_error(VFK_ERR_INVALID,
                       "deberta_rel_chunk_major: %s must be [H, >= %d, 64] with 16-byte aligned rows",
                       names[j], 2 * att_span);
    if (d->size[0] != H || d->size[1] != 8 || d->size[2] != 2 * att_span || d->size[3] != 8 ||
        d->stride[3] != 1 || d->stride[2] != 8 || d->stride[1] != 16 * (int64_t)att_span ||
        d->stride[0] < 128 * (int64_t)att_span || d->stride[0] % 8 || !aligned16(d->data))
      return set_error(VFK_ERR_INVALID,
                       "deberta_rel_chunk_major: out must be [H, 8, %d, 8], contiguous per head, "
                       "16-byte aligned", 2 * att_span);
    a.src[j] = static_cast<const uint16_t*>(s->data);
    a.ss[j][0] = s->stride[0];
    a.ss[j][1] = s->stride[1];
    a.dst[j] = static_cast<uint16_t*>(d->data);
    a.ds[j] = d->stride[0];
  }
  if (H <= 0) return VFK_OK;
  a.H = H;
  a.n0 = (int64_t)H * 2 * att_span * 8;
  const int64_t n = 2 * a.n0;
  hipLaunchKernelGGL(rel_cm_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a);
  return launch_status("deberta_rel_chunk_major");
}

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

// Scale, attention span and bucket step function (max_abs: the largest
// |i - j| the launch can meet + 1).
static int setup_scalars(DebArgs& a, float sm_scale, int position_buckets, int max_relative_distance,
                         int use_log_bucket, int max_abs, const char* name) {
  if (!(sm_scale > 0.f) || !isfinite(sm_scale))
    return set_error(VFK_ERR_UNSUPPORTED, "%s: sm_scale must be > 0", name);
  a.c2 = sm_scale * VFK_LOG2E;
  // flash_deberta_attention.py:323, :366-368
  a.span = position_buckets > 0 ? position_buckets : max_relative_distance;
  const int nb = position_buckets > 0 ? position_buckets : max_relative_distance * 2;
  const int maxd = max_relative_distance > 0 ? max_relative_distance : 512;
  a.log_bucket = use_log_bucket ? 1 : 0;
  if (a.span <= 0) return set_error(VFK_ERR_INVALID, "%s: att_span must be > 0", name);
  a.unit = 1;
  if (a.log_bucket) {
    int rc;
    if ((rc = build_deberta_step(nb, maxd, max_abs, a.span, &a.step))) return rc;
    a.unit = step_is_unit(a.step) ? 1 : 0;
  }
  // the run of distances around 0 where c(d) = d + span (empty: lo > hi)
  a.lin_lo = 1;
  a.lin_hi = 0;
  if (deb_index(a, 0) == a.span) {
    int lo = 0, hi = 0;
    while (hi + 1 < max_abs && deb_index(a, hi + 1) == hi + 1 + a.span) ++hi;
    while (1 - lo < max_abs && deb_index(a, lo - 1) == lo - 1 + a.span) --lo;
    a.lin_lo = lo;
    a.lin_hi = hi;
  }
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
  a.q = q->data; a.k = k->data; a.v = v->data; a.o = out->data;
  for (int i = 0; i < 4; ++i) {
    a.qs[i] = q->stride[i]; a.ks[i] = k->stride[i]; a.vs[i] = v->stride[i]; a.os[i] = out->stride[i];
  }
  a.B = (int)B; a.H = (int)H; a.M = (int)M; a.N = (int)N;
  a.seq_lengths = seq_lengths;
  return setup_scalars(a, sm_scale, position_buckets, max_relative_distance, use_log_bucket,
                       (int)(M > N ? M : N), name);
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
  // staged form: both pos tensors with contiguous, 16-byte aligned rows, a
  // span whose 2S columns hold the widest window, and LDS within 64 KB
  auto rows16 = [](const void* p, const int64_t* s) {
    return s[3] == 1 && s[0] % 8 == 0 && s[1] % 8 == 0 && s[2] % 8 == 0 &&
           (reinterpret_cast<uintptr_t>(p) & 15) == 0;
  };
  const size_t slds = deb_staged_lds(a.lut_len);
  if (a.unit && (a.pk || a.pq) && (!a.pk || rows16(a.pk, a.pks)) && (!a.pq || rows16(a.pq, a.pqs)) &&
      a.span % 4 == 0 && 2 * a.span >= kPqW && slds <= 64 * 1024) {
#define VFK_DEB_STAGED(E)                                                                         \
  if (a.pk && a.pq)                                                                               \
    hipLaunchKernelGGL((deberta_gather_staged_kernel<E, true, true>), grid, dim3(256), slds, st, a); \
  else if (a.pk)                                                                                  \
    hipLaunchKernelGGL((deberta_gather_staged_kernel<E, true, false>), grid, dim3(256), slds, st, a); \
  else                                                                                            \
    hipLaunchKernelGGL((deberta_gather_staged_kernel<E, false, true>), grid, dim3(256), slds, st, a);
    if (q->dtype == VFK_BF16) {
      VFK_DEB_STAGED(BF16)
    } else {
      VFK_DEB_STAGED(F16)
    }
#undef VFK_DEB_STAGED
    return launch_status("vfk_flash_deberta_fwd");
  }
  if (q->dtype == VFK_BF16)
    hipLaunchKernelGGL(deberta_gather_kernel<BF16>, grid, dim3(256), lds, st, a);
  else
    hipLaunchKernelGGL(deberta_gather_kernel<F16>, grid, dim3(256), lds, st, a);
  return launch_status("vfk_flash_deberta_fwd");
}

// Relative-table checks and the launch of the fused kernel (padded and
// packed entry points).
static int deb_fused_launch(DebArgs& a, int dt, const vfk_tensor* key_rel, const vfk_tensor* query_rel,
                            hipStream_t st, const char* name) {
  int rc;
  const vfk_tensor* rel[2] = {key_rel, query_rel};
  const char* names[2] = {"key_rel", "query_rel"};
  a.rel_cm = -1;
  for (int i = 0; i < 2; ++i) {
    if (!present(rel[i])) continue;
    const vfk_tensor* r = rel[i];
    const int cm = r->ndim == 4;
    if (a.rel_cm >= 0 && a.rel_cm != cm)
      return set_error(VFK_ERR_INVALID, "%s: key_rel and query_rel must share one layout", name);
    a.rel_cm = cm;
    if ((rc = check_tensor(r, names[i], cm ? 4 : 3))) return rc;
    if (r->dtype != dt) return set_error(VFK_ERR_INVALID, "%s: dtype differs from q", names[i]);
    if (cm) {
      // chunk-major [H, 8, 2S, 8]: chunk c holds k = 8 c .. 8 c + 7 of every row
      if (dt == VFK_F32)
        return set_error(VFK_ERR_UNSUPPORTED, "%s: the chunk-major layout is for 16-bit types", names[i]);
      if (r->size[0] != a.H || r->size[1] != 8 || r->size[2] != 2 * a.span || r->size[3] != 8 ||
          r->stride[3] != 1 || r->stride[2] != 8 || r->stride[1] != 16 * a.span ||
          r->stride[0] < 128 * (int64_t)a.span || r->stride[0] % 8 || !aligned16(r->data))
        return set_error(VFK_ERR_INVALID,
                         "%s: expected a chunk-major [H, 8, %d, 8], contiguous per head and 16-byte "
                         "aligned", names[i], 2 * a.span);
    } else {
      if (r->size[0] != a.H || r->size[1] < 2 * a.span || r->size[2] != kHD || r->stride[2] != 1)
        return set_error(VFK_ERR_INVALID, "%s: expected [H, >= %d, 64] with unit last stride", names[i],
                         2 * a.span);
      if (dt != VFK_F32 && (!aligned16(r->data) || r->stride[0] % 8 || r->stride[1] % 8))
        return set_error(VFK_ERR_INVALID, "%s: rows must be 16-byte aligned", names[i]);
    }
    if (i == 0) { a.kr = r->data; a.krs[0] = r->stride[0]; a.krs[1] = cm ? 0 : r->stride[1]; }
    else { a.qr = r->data; a.qrs[0] = r->stride[0]; a.qrs[1] = cm ? 0 : r->stride[1]; }
  }
  if (a.rel_cm < 0) a.rel_cm = 0;
  if (a.B == 0 || a.H == 0 || a.M == 0) return VFK_OK;
  if (dt == VFK_F32) {
    const int nqt = ceil_div(a.M, 64);
    hipLaunchKernelGGL(deberta_fused_f32_kernel, dim3((unsigned)(nqt * a.B * a.H)), dim3(64), 0, st, a);
    return launch_status(name);
  }
  const int ntk = ceil_div(a.N, kBN);
  a.lut_len = ntk * kBN + kBM;
  const size_t dyn = (size_t)a.lut_len * 2;
  if (kFusedStaticLds + dyn > 160 * 1024)
    return set_error(VFK_ERR_UNSUPPORTED, "%s: N too large", name);
  // the table holds 2 c in int16; the K / V buffer resources span N rows
  if (a.span > 8192)
    return set_error(VFK_ERR_UNSUPPORTED, "%s: att_span above 8192", name);
  if ((a.kr && 4 * (int64_t)a.span * a.krs[1] >= ((int64_t)1 << 31)) ||
      (a.qr && 4 * (int64_t)a.span * a.qrs[1] >= ((int64_t)1 << 31)))
    return set_error(VFK_ERR_UNSUPPORTED, "%s: rel tables span 2 GiB or more", name);
  if ((int64_t)a.N * (a.ks[2] > a.vs[2] ? a.ks[2] : a.vs[2]) * 2 >= ((int64_t)1 << 31))
    return set_error(VFK_ERR_UNSUPPORTED, "%s: K / V rows span 2 GiB or more", name);
  const int nqt = ceil_div(a.M, kBM);
  dim3 grid((unsigned)(nqt * a.B * a.H));
#define VFK_DEB_GO(E, C, P) \
  hipLaunchKernelGGL((deberta_fused_kernel<E, C, P>), grid, dim3(256), dyn, st, a)
  const bool c2p = a.kr != nullptr, p2c = a.qr != nullptr;
  if (dt == VFK_BF16) {
    if (c2p && p2c) VFK_DEB_GO(BF16, true, true);
    else if (c2p) VFK_DEB_GO(BF16, true, false);
    else if (p2c) VFK_DEB_GO(BF16, false, true);
    else VFK_DEB_GO(BF16, false, false);
  } else {
    if (c2p && p2c) VFK_DEB_GO(F16, true, true);
    else if (c2p) VFK_DEB_GO(F16, true, false);
    else if (p2c) VFK_DEB_GO(F16, false, true);
    else VFK_DEB_GO(F16, false, false);
  }
#undef VFK_DEB_GO
  return launch_status(name);
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
  // the per-tile index windows (at most 3 C and 6 P^T blocks of 32) hold
  // only for indices that move by at most 1 per unit of distance
  if (!a.unit)
    return set_error(VFK_ERR_UNSUPPORTED,
                     "vfk_deberta_fused_fwd: position_buckets=%d / max_relative_positions=%d give "
                     "bucket steps above 1 (use flash_deberta_attention)",
                     position_buckets, max_relative_distance);
  return deb_fused_launch(a, q->dtype, key_rel, query_rel, (hipStream_t)stream, "vfk_deberta_fused_fwd");
}

// [T, H, 64] tensor of a packed stream (token stride [0], head stride [1]).
static int check_thd_deb(const vfk_tensor* t, const char* name, int dtype, int64_t T, int64_t H) {
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

extern "C" int vfk_deberta_fused_varlen_fwd(const vfk_tensor* q, const vfk_tensor* k, const vfk_tensor* v,
                                            const int32_t* cu_seqlens, int32_t num_seqs,
                                            int32_t max_seqlen, const vfk_tensor* key_rel,
                                            const vfk_tensor* query_rel, float sm_scale,
                                            int32_t position_buckets, int32_t max_relative_distance,
                                            int32_t use_log_bucket, vfk_tensor* out, void* stream) {
  const char* name = "vfk_deberta_fused_varlen_fwd";
  int rc = check_tensor(q, "q", 3);
  if (rc) return rc;
  const int dt = q->dtype;
  if (dt != VFK_BF16 && dt != VFK_F16) return set_error(VFK_ERR_UNSUPPORTED, "%s: bf16 or fp16 only", name);
  const int64_t T = q->size[0], H = q->size[1];
  if ((rc = check_thd_deb(q, "q", dt, T, H)) || (rc = check_thd_deb(k, "k", dt, T, H)) ||
      (rc = check_thd_deb(v, "v", dt, T, H)) || (rc = check_thd_deb(out, "out", dt, T, H)))
    return rc;
  if (!cu_seqlens) return set_error(VFK_ERR_INVALID, "%s: NULL cu_seqlens", name);
  if (num_seqs < 0 || max_seqlen < 0 || max_seqlen > 32767 || (int64_t)num_seqs * H > (1 << 24))
    return set_error(VFK_ERR_INVALID, "%s: bad num_seqs / max_seqlen", name);
  DebArgs a = {};
  a.q = q->data; a.k = k->data; a.v = v->data; a.o = out->data;
  // [T, H, D] as the padded kernel's [., H, L, D]: head stride [1], row stride [2]
  a.qs[1] = q->stride[1]; a.qs[2] = q->stride[0]; a.qs[3] = 1;
  a.ks[1] = k->stride[1]; a.ks[2] = k->stride[0]; a.ks[3] = 1;
  a.vs[1] = v->stride[1]; a.vs[2] = v->stride[0]; a.vs[3] = 1;
  a.os[1] = out->stride[1]; a.os[2] = out->stride[0]; a.os[3] = 1;
  a.B = num_seqs; a.H = (int)H; a.M = max_seqlen; a.N = max_seqlen;
  a.cu = cu_seqlens;
  if ((rc = setup_scalars(a, sm_scale, position_buckets, max_relative_distance, use_log_bucket,
                          max_seqlen, name)))
    return rc;
  if (!a.unit)
    return set_error(VFK_ERR_UNSUPPORTED,
                     "%s: position_buckets=%d / max_relative_positions=%d give bucket steps above 1",
                     name, position_buckets, max_relative_distance);
  if (num_seqs == 0 || T == 0 || max_seqlen == 0) return VFK_OK;
  return deb_fused_launch(a, dt, key_rel, query_rel, (hipStream_t)stream, name);
}
