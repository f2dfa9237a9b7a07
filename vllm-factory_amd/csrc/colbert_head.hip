// ColBERT output head on gfx950: LayerNorm -> projection -> L2 normalisation.
//
// Replaces the last steps of the reference's ModernBERT ColBERT plugin
// (plugins/moderncolbert/model.py:260-267: the final LayerNorm of the encoder,
// then the PyLate Dense projection, then projected / projected.norm()
// clamped at 1e-8) with one pass over the hidden rows: the normalised rows
// never go back to HBM unless the caller asks for them.
//
// Two kernels. The folded one (vfk_colbert_head_folded_fwd, further down)
// multiplies the LayerNorm weight into the projection and projects the raw
// rows; it is what callers that do not want the normalised rows back run.
// The staged one (vfk_colbert_head_fwd) LayerNorms rows into LDS first and
// can return them:
//
// A workgroup takes 32 tokens. Phase 1: each wave LayerNorms 8 rows (x, plus
// an optional residual, fp32 statistics in two passes as the reference's
// LayerNorm) into a 16-bit LDS tile [32][D]. Phase 2: wave w computes output
// columns 32w .. 32w+31 for the 32 tokens with v_mfma_f32_32x32x16 (A = rows
// of W, streamed from L2, where the whole [N, D] matrix stays resident,
// through a register ring: from W in operand order, as vfk_pack_weight_mfma32
// lays it out, each load of a wave is one contiguous KiB; from the [N, D]
// rows, each lane reads whole 64-byte runs of its row;
// B = the tokens' normalised rows from LDS;
// all of a wave's row loads are issued before any row is reduced), so lane (c, h) ends
// with token c and 16 of the wave's columns. Phase 3: per-token sums of
// squares are combined across the waves through LDS, and each lane scales
// and stores its 16 outputs.
#include <math.h>

#include <algorithm>
#include <atomic>
#include <type_traits>

#include "attn_core.h"
#include "launch_util.h"
#include "vfk_common.h"

namespace vfk {

constexpr int kHeadRows = 32;
constexpr int kHeadPad = 8;  // u16 of padding per LDS row

struct HeadArgs {
  const uint16_t* x; int64_t xs;  // [T, D], row stride in elements
  const uint16_t* r; int64_t rs;  // residual [T, D] or null
  const uint16_t* lnw;            // [D] or null: no LayerNorm (rows used as given)
  const uint16_t* lnb;            // [D] or null
  float eps;
  const uint16_t* w; int64_t ws;  // [N, D]
  const uint16_t* bias;           // [N] or null
  uint16_t* h; int64_t hs;        // normalised rows [T, D] or null
  uint16_t* y; int64_t ys;        // [T, N]
  int64_t T;
  int D, N;
};

template <typename E>
__device__ inline void load4(const uint16_t* p, float (&f)[4]) {
  const u32x2_t v = *reinterpret_cast<const u32x2_t*>(p);
  f[0] = E::to_f32((uint16_t)(v[0] & 0xffffu));
  f[1] = E::to_f32((uint16_t)(v[0] >> 16));
  f[2] = E::to_f32((uint16_t)(v[1] & 0xffffu));
  f[3] = E::to_f32((uint16_t)(v[1] >> 16));
}

__device__ inline float wave_sum(float v) { return group_sum<64>(v); }

// NCH = D / 256: 4-element chunks per lane and row. PACKED: a.w is the weight
// in operand order [N/32][D/16][64][8].
template <typename E, int NCH, bool PACKED>
__global__ __launch_bounds__(256) void colbert_head_kernel(HeadArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int D = NCH * 256;
  const int ld = D + kHeadPad;
  uint16_t* At = reinterpret_cast<uint16_t*>(smem);                  // [32][ld]
  float* red = reinterpret_cast<float*>(At + kHeadRows * ld);        // [4][32]
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int64_t r0 = (int64_t)blockIdx.x * kHeadRows;

  // ---- phase 1: rows of the tile, LayerNorm into LDS ----
  float gw[NCH][4], gb[NCH][4];
  if (a.lnw) {
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      load4<E>(a.lnw + (c * 64 + lane) * 4, gw[c]);
      if (a.lnb) load4<E>(a.lnb + (c * 64 + lane) * 4, gb[c]);
      else gb[c][0] = gb[c][1] = gb[c][2] = gb[c][3] = 0.f;
    }
  }
  // all eight rows' loads of this wave are issued before any row is reduced
  constexpr int kRW = kHeadRows / 4;  // rows per wave
  u32x2_t xr[kRW][NCH], rv[kRW][NCH];
#pragma unroll
  for (int i = 0; i < kRW; ++i) {
    const int64_t row = r0 + w + 4 * i;
    const bool ok = row < a.T;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const u32x2_t z = {0u, 0u};
      xr[i][c] = ok ? *reinterpret_cast<const u32x2_t*>(a.x + row * a.xs + (c * 64 + lane) * 4) : z;
      rv[i][c] = (ok && a.r) ? *reinterpret_cast<const u32x2_t*>(a.r + row * a.rs + (c * 64 + lane) * 4)
                             : z;
    }
  }
#pragma unroll
  for (int i = 0; i < kRW; ++i) {
    const int rr = w + 4 * i;
    const int64_t row = r0 + rr;
    float v[NCH][4];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      v[c][0] = E::to_f32((uint16_t)(xr[i][c][0] & 0xffffu)) + E::to_f32((uint16_t)(rv[i][c][0] & 0xffffu));
      v[c][1] = E::to_f32((uint16_t)(xr[i][c][0] >> 16)) + E::to_f32((uint16_t)(rv[i][c][0] >> 16));
      v[c][2] = E::to_f32((uint16_t)(xr[i][c][1] & 0xffffu)) + E::to_f32((uint16_t)(rv[i][c][1] & 0xffffu));
      v[c][3] = E::to_f32((uint16_t)(xr[i][c][1] >> 16)) + E::to_f32((uint16_t)(rv[i][c][1] >> 16));
    }
    if (a.lnw) {
      float s = 0.f;
#pragma unroll
      for (int c = 0; c < NCH; ++c) s += (v[c][0] + v[c][1]) + (v[c][2] + v[c][3]);
      const float mean = wave_sum(s) / (float)D;
      float q = 0.f;
#pragma unroll
      for (int c = 0; c < NCH; ++c)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float d = v[c][j] - mean;
          q += d * d;
        }
      const float rstd = 1.0f / sqrtf(wave_sum(q) / (float)D + a.eps);
#pragma unroll
      for (int c = 0; c < NCH; ++c)
#pragma unroll
        for (int j = 0; j < 4; ++j) v[c][j] = (v[c][j] - mean) * rstd * gw[c][j] + gb[c][j];
    }
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const u32x2_t pk = {E::pack2(v[c][0], v[c][1]), E::pack2(v[c][2], v[c][3])};
      *reinterpret_cast<u32x2_t*>(At + rr * ld + (c * 64 + lane) * 4) = pk;
      if (a.h && row < a.T) *reinterpret_cast<u32x2_t*>(a.h + row * a.hs + (c * 64 + lane) * 4) = pk;
    }
  }
  __syncthreads();

  // ---- phase 2: projection, wave w -> columns 32w .. 32w+31 ----
  const int c = lane & 31, hh = lane >> 5;
  const bool on = 32 * w < a.N;
  f32x16_t acc = {};
  if (on) {
    // Packed: k-step s of the wave's 32 rows is the KiB block w * D/16 + s,
    // lane half hh holding k = 16 s + 8 hh .. +7 (the standard operand order).
    // Rows: the reduction order over k is free as long as both operands
    // follow it: in each 64-wide chunk, MFMA step j gives lane half hh the k
    // values 32 hh + 8 j .. +7, so a lane reads one contiguous 64-byte run of
    // its W row per chunk and the two halves cover the row's 128-byte line.
    const uint16_t* wrow = PACKED ? a.w + ((int64_t)w * (D / 16) * 64 + lane) * 8
                                  : a.w + (int64_t)(32 * w + c) * a.ws + 32 * hh;
    const uint16_t* arow = At + c * ld + (PACKED ? 8 : 32) * hh;
    auto wsrc = [&](int m, int j) { return PACKED ? wrow + (4 * m + j) * 512 : wrow + 64 * m + 8 * j; };
    auto asrc = [&](int m, int j) { return PACKED ? arow + 64 * m + 16 * j : arow + 64 * m + 8 * j; };
    // W streams from L2 through a ring of kWC chunks (4 MFMA steps each)
    constexpr int kWC = 4, NK = NCH * 4;  // chunks in flight, chunks in D
    u32x4_t wq[kWC][4];
#pragma unroll
    for (int m = 0; m < kWC; ++m)
#pragma unroll
      for (int j = 0; j < 4; ++j) wq[m][j] = *reinterpret_cast<const u32x4_t*>(wsrc(m, j));
#pragma unroll
    for (int m = 0; m < NK; ++m) {
      __builtin_amdgcn_sched_barrier(0);
      u32x4_t xb[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) xb[j] = *reinterpret_cast<const u32x4_t*>(asrc(m, j));
#pragma unroll
      for (int j = 0; j < 4; ++j) acc = E::mfma32(wq[m % kWC][j], xb[j], acc);
      if (m + kWC < NK) {
#pragma unroll
        for (int j = 0; j < 4; ++j) wq[m % kWC][j] = *reinterpret_cast<const u32x4_t*>(wsrc(m + kWC, j));
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    // lane (c, hh): token c, columns 32w + 8(e/4) + 4hh + e%4
    if (a.bias) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float b4[4];
        load4<E>(a.bias + 32 * w + 8 * j + 4 * hh, b4);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[4 * j + e] += b4[e];
      }
    }
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) ss += acc[e] * acc[e];
    ss = half_swap_sum(ss);
    if (hh == 0) red[w * 32 + c] = ss;
  }
  __syncthreads();

  // ---- phase 3: per-token norm over all N columns, scale, store ----
  if (on) {
    float tot = 0.f;
    for (int j = 0; 32 * j < a.N; ++j) tot += red[j * 32 + c];
    const float inv = 1.0f / fmaxf(sqrtf(tot), 1e-8f);
    const int64_t tok = r0 + c;
    if (tok < a.T) {
      uint16_t* yrow = a.y + tok * a.ys + 32 * w + 4 * hh;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const u32x2_t pk = {E::pack2(acc[4 * j] * inv, acc[4 * j + 1] * inv),
                            E::pack2(acc[4 * j + 2] * inv, acc[4 * j + 3] * inv)};
        *reinterpret_cast<u32x2_t*>(yrow + 8 * j) = pk;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Folded form (no normalised rows returned). With u = x + residual rounded to
// the element type (the encoder's residual sum), its mean mu and rstd =
// 1 / sqrt(var + eps):
//   LN(u)_k = (u_k - mu) rstd gamma_k + beta_k
//   y_n     = sum_k LN(u)_k W_nk + b_n = rstd (P_n - mu G_n) + C_n
// where P_n = sum_k u_k W'_nk, W'_nk = gamma_k W_nk rounded to the element
// type and packed in MFMA operand order, G_n = sum_k W'_nk and
// C_n = sum_k beta_k W_nk + b_n in fp32 (vfk_colbert_fold_weight makes the
// three once per weight). The raw rows then feed the MFMAs directly: there is
// no normalised copy to stage, so the four waves of a workgroup take 128
// tokens (32 each) and share one stream of the folded weight through LDS, in
// 64-wide K slices double-buffered by direct loads: a quarter of the weight
// bytes of 32-token workgroups. Each wave loads its rows' slice one slice
// ahead into registers with whole-line loads (eight lanes per 128-byte piece
// of a row), forms u and passes it through its own LDS stage into the
// operand layout (lane: token c, k = 16 s + 8 hh .. +7); each lane keeps
// sums of u - u_first and of its square over its half of the row, and the
// two halves are combined at the end (the pairwise form of the variance).
// Measured on the ColBERT workload (163 736 tokens, 768 -> 128, residual +
// LayerNorm): 108 us, 63 % of HBM peak; the non-temporal hints on the row
// loads and output stores are worth about 12 %, the whole-line loads
// (against one 32-byte piece of 32 rows per load) about 15 %, the output
// stores through LDS (whole 128-byte pieces) about 6 %.
// ---------------------------------------------------------------------------
constexpr int kFoldTok = 128;  // tokens per chunk (32 per wave)

struct FoldArgs {
  const uint16_t* x; int64_t xs;
  const uint16_t* r; int64_t rs;  // residual or null
  const uint16_t* w;              // folded weight [N/32][D/16][64][8]
  const float* g;                 // [N] column sums of W' (read with the LayerNorm only)
  const float* c;                 // [N] constant term
  float eps;
  uint16_t* y; int64_t ys;
  int64_t T;
  int64_t per;                    // tokens per workgroup
  int D, N;
};

// The lane pair (l, l ^ 32)'s other value.
__device__ inline float half_partner(float x) {
  const int xi = __float_as_int(x);
  const auto r = __builtin_amdgcn_permlane32_swap(xi, xi, false, false);
  return __int_as_float((threadIdx.x & 32) ? r[0] : r[1]);
}

// Waits until at most the wave's NLEFT newest vector loads are in flight
// (the row loads issued after the next weight slice's direct loads; loads
// complete in issue order) and its LDS reads are done, then joins the
// workgroup barrier. One asm statement with a memory clobber, so that no
// load moves across it.
template <int NLEFT>
__device__ inline void fold_barrier() {
  if (NLEFT == 8)
    asm volatile("s_waitcnt vmcnt(8) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  else
    asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// NB = N / 32 output blocks; RES: a residual is added; LN: the LayerNorm is
// applied (else the rows are projected as given).
//
// Workgroup b takes the tokens [b per, (b + 1) per) (the grid holds as many
// workgroups as fit on the device at once, so every one streams the same
// number of bytes), in chunks of 128 (the last one partial): one pipeline
// of 64-wide K slices runs through all its chunks, so the first slice of the
// next chunk is in flight while a chunk's outputs are formed and stored.
template <typename E, int NB, bool RES, bool LN>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void colbert_fold_kernel(FoldArgs a) {
  __shared__ __align__(16) uint16_t Ws0[NB * 4 * 512];
  __shared__ __align__(16) uint16_t Ws1[NB * 4 * 512];
  __shared__ __align__(16) uint16_t Us[4][32 * 64];  // each wave's u slice, 32 rows x 128 B
  __shared__ __align__(16) float GC[2][NB * 32];     // G and C
  constexpr int kLeft = RES ? 8 : 4;  // row loads issued per slice
  const int t = threadIdx.x, lane = t & 63, w = t >> 6, c = lane & 31, hh = lane >> 5;
  const int64_t wbeg = (int64_t)blockIdx.x * a.per;
  const int64_t wend = wbeg + a.per < a.T ? wbeg + a.per : a.T;
  const int nch = (int)((wend - wbeg + kFoldTok - 1) / kFoldTok);
  const int nks = a.D / 16;  // k-steps
  const int nsl = nks / 4;   // slices
  const rsrc_t wr = uniform_rsrc(a.w, a.N * a.D * 2);
  // slice sl of output block f is the KiB blocks 4 sl .. 4 sl + 3 of f, one
  // contiguous 4 KiB run; wave w copies the KiB of k-step 4 sl + w
  const int wu = __builtin_amdgcn_readfirstlane(w);  // uniform: LDS base and scalar offset
  auto wload = [&](int sl, uint16_t* buf) {
#pragma unroll
    for (int f = 0; f < NB; ++f)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (lds_void_t*)(buf + f * 2048 + wu * 512), 16, lane * 16,
                                               ((f * nks + 4 * sl) * 512 + wu * 512) * 2, 0, 0);
  };
  // Row loads cover whole 128-byte lines: load i of a slice takes the wave's
  // rows 8 i + lane / 8 of the chunk, eight lanes per row (16-byte chunk
  // lane % 8), through buffer resources over the wave's rows (rows past the
  // workgroup's range read as zeros and are never stored); the row and slice
  // offsets are uniform.
  const int q = lane & 7;
  rsrc_t xr, rr;
  auto rows_of = [&](int ch) {
    const int64_t tok0 = wbeg + (int64_t)ch * kFoldTok + wu * 32;
    const int nrow = (int)(wend - tok0 < 32 ? (wend - tok0 > 0 ? wend - tok0 : 0) : 32);
    const int64_t t0 = nrow > 0 ? tok0 : 0;
    xr = uniform_rsrc(a.x + t0 * a.xs, nrow * (int)a.xs * 2);
    if (RES) rr = uniform_rsrc(a.r + t0 * a.rs, nrow * (int)a.rs * 2);
  };
  const int xo = ((lane >> 3) * (int)a.xs + 8 * q) * 2;
  const int ro = RES ? ((lane >> 3) * (int)a.rs + 8 * q) * 2 : 0;
  u32x4_t xq[4], rq[4];
  constexpr int kNT = 2;  // cache policy: non-temporal (each row byte is read once)
  auto rload = [&](int sl) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      xq[i] = __builtin_amdgcn_raw_buffer_load_b128(xr, xo, 16 * i * (int)a.xs + 128 * sl, kNT);
      if (RES) rq[i] = __builtin_amdgcn_raw_buffer_load_b128(rr, ro, 16 * i * (int)a.rs + 128 * sl, kNT);
    }
  };
  // u = x + r rounded, into the wave's stage: chunk q of row r at chunk q ^ swz(r)
  char* us = reinterpret_cast<char*>(Us[w]);
  auto ustore = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v[8];
      unpack8<E>(xq[i], v);
      if (RES) {
        float rv[8];
        unpack8<E>(rq[i], rv);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] += rv[e];
      }
      const int r = 8 * i + (lane >> 3);
      *reinterpret_cast<u32x4_t*>(us + r * 128 + 16 * (q ^ swz(r))) = pack8<E>(v);
    }
    // the wave's other lanes read what each lane wrote
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
  const int fc = swz(c);

  // G and C into LDS (published by the first slice's barrier); their loads
  // are older than every counted load below
  const bool gct = t < NB * 8;
  f32x4_t gq = {0.f, 0.f, 0.f, 0.f}, cq = {0.f, 0.f, 0.f, 0.f};
  if (gct) {
    cq = *reinterpret_cast<const f32x4_t*>(a.c + 4 * t);
    if (LN) gq = *reinterpret_cast<const f32x4_t*>(a.g + 4 * t);
  }
  f32x16_t acc[NB];
#pragma unroll
  for (int f = 0; f < NB; ++f) acc[f] = f32x16_t{};
  rows_of(0);
  // the fences keep every row load behind the weight's direct loads, which
  // the counted waits rely on
  asm volatile("" ::: "memory");
  wload(0, Ws0);
  asm volatile("" ::: "memory");
  rload(0);
  fold_barrier<kLeft>();  // slice 0 landed
  if (gct) {
    *reinterpret_cast<f32x4_t*>(&GC[0][4 * t]) = gq;
    *reinterpret_cast<f32x4_t*>(&GC[1][4 * t]) = cq;
  }
  float sh = 0.f, s1 = 0.f, s2 = 0.f;

  // slice j from buf; more: a slice follows (slice jn, into nbuf, its rows
  // through the current resources). One loop body for every slice pair keeps
  // the accumulators in place (a peeled last pair makes the register
  // allocator rotate them).
  auto slice = [&](bool more, int j, int jn, const uint16_t* buf, uint16_t* nbuf) {
    ustore();
    if (more) {
      asm volatile("" ::: "memory");
      wload(jn, nbuf);
      asm volatile("" ::: "memory");
      rload(jn);
    }
    // B operand: lane (c, hh) takes row c, k = 16 s4 + 8 hh .. +7 (chunk 2 s4 + hh)
    u32x4_t bop[4];
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4)
      bop[s4] = *reinterpret_cast<const u32x4_t*>(us + c * 128 + 16 * ((2 * s4 + hh) ^ fc));
    if (LN) {
      // the half-row's first value shifts its sums (no cancellation for rows
      // far from zero mean)
      if (j == 0) sh = E::to_f32((uint16_t)(bop[0][0] & 0xffffu));
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        float u[8];
        unpack8<E>(bop[s4], u);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float d = u[e] - sh;
          s1 += d;
          s2 = __builtin_fmaf(d, d, s2);
        }
      }
    }
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
      for (int f = 0; f < NB; ++f) {
        const u32x4_t aop = *reinterpret_cast<const u32x4_t*>(buf + f * 2048 + s4 * 512 + lane * 8);
        acc[f] = E::mfma32(aop, bop[s4], acc[f]);
      }
    fold_barrier<kLeft>();  // slice jn landed, slice j free
  };

  for (int ch = 0; ch < nch; ++ch) {
    // nsl is even (D a multiple of 128): slice pairs, W slice 2 m in Ws0
    for (int j = 0; j < nsl; j += 2) {
      slice(true, j, j + 1, Ws0, Ws1);
      const bool last = j + 2 >= nsl;
      if (last && ch + 1 < nch) rows_of(ch + 1);
      slice(!last || ch + 1 < nch, j + 1, last ? 0 : j + 2, Ws1, Ws0);
    }

    // LayerNorm statistics of the row: the two halves' means and squared
    // deviations, combined pairwise
    float mean = 0.f, rstd = 1.f;
    if (LN) {
      const float nh = 0.5f * (float)a.D;
      const float ma = sh + s1 / nh;
      const float qa = fmaxf(s2 - s1 * (s1 / nh), 0.f);
      const float mb = half_partner(ma), qb = half_partner(qa);
      const float d = ma - mb;
      mean = 0.5f * (ma + mb);
      rstd = 1.0f / sqrtf((qa + qb + d * d * (0.25f * (float)a.D)) / (float)a.D + a.eps);
      s1 = s2 = 0.f;
    }
    // lane (c, hh): token c, outputs n = 32 f + 8 jj + 4 hh + e in
    // acc[f][4 jj + e]. y is rounded to the element type first and its norm
    // taken from the rounded values, as the reference's 16-bit projection
    // output is; the packed pairs are all that stays live until the scale
    // is known.
    u32x2_t yp[NB][4];
    float ss = 0.f;
#pragma unroll
    for (int f = 0; f < NB; ++f)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int n0 = 32 * f + 8 * jj + 4 * hh;
        const f32x4_t cv = *reinterpret_cast<const f32x4_t*>(&GC[1][n0]);
        f32x4_t gv = {0.f, 0.f, 0.f, 0.f};
        if (LN) gv = *reinterpret_cast<const f32x4_t*>(&GC[0][n0]);
        float yv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float p = acc[f][4 * jj + e];
          yv[e] = LN ? __builtin_fmaf(rstd, __builtin_fmaf(-mean, gv[e], p), cv[e]) : p + cv[e];
        }
        yp[f][jj] = u32x2_t{E::pack2(yv[0], yv[1]), E::pack2(yv[2], yv[3])};
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const float lo = E::to_f32((uint16_t)(yp[f][jj][i] & 0xffffu));
          const float hi = E::to_f32((uint16_t)(yp[f][jj][i] >> 16));
          ss = __builtin_fmaf(lo, lo, __builtin_fmaf(hi, hi, ss));
        }
      }
#pragma unroll
    for (int f = 0; f < NB; ++f) acc[f] = f32x16_t{};
    ss = half_swap_sum(ss);
    const float inv = 1.0f / fmaxf(sqrtf(ss), 1e-8f);
    // Stores go through the wave's stage so that eight lanes write each
    // 128-byte piece of a row (16-byte pieces per lane leave partly written
    // lines behind): output blocks f0, f0 + 1 are 32 rows x 128 B.
    const int64_t ctok = wbeg + (int64_t)ch * kFoldTok + w * 32;  // the wave's first row
    const int fcs = swz(c);
    auto out_blocks = [&](auto fb_, int f0) {
      constexpr int FB = decltype(fb_)::value;  // blocks written together (1 or 2)
#pragma unroll
      for (int fi = 0; fi < FB; ++fi)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          u32x2_t pk;
#pragma unroll
          for (int i = 0; i < 2; ++i)
            pk[i] = E::pack2(E::to_f32((uint16_t)(yp[f0 + fi][jj][i] & 0xffffu)) * inv,
                             E::to_f32((uint16_t)(yp[f0 + fi][jj][i] >> 16)) * inv);
          *reinterpret_cast<u32x2_t*>(us + c * 128 + 16 * ((4 * fi + jj) ^ fcs) + 8 * hh) = pk;
        }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      constexpr int LPR = 4 * FB;   // lanes per row (16 B each)
      constexpr int RPI = 64 / LPR;  // rows per store
      const int qq = lane % LPR;
#pragma unroll
      for (int k = 0; k < 32 / RPI; ++k) {
        const int r = lane / LPR + RPI * k;
        const u32x4_t v = *reinterpret_cast<const u32x4_t*>(us + r * 128 + 16 * (qq ^ swz(r)));
        // streaming stores: the embeddings are not read again here
        if (ctok + r < wend)
          __builtin_nontemporal_store(v, reinterpret_cast<u32x4_t*>(a.y + (ctok + r) * a.ys + 32 * f0 + 8 * qq));
      }
      // the next writes to the stage follow these reads (LDS order within a wave)
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
#pragma unroll
    for (int f0 = 0; f0 + 1 < NB; f0 += 2) out_blocks(std::integral_constant<int, 2>{}, f0);
    if (NB & 1) out_blocks(std::integral_constant<int, 1>{}, NB - 1);
  }
}

// One block per output row n: W'_n = gamma * W_n rounded, written in operand
// order; G_n = sum_k W'_nk and C_n = sum_k beta_k W_nk + b_n in fp32.
template <typename E>
__global__ __launch_bounds__(256) void colbert_fold_weight_kernel(const uint16_t* w, int64_t ws,
                                                                  const uint16_t* gamma,
                                                                  const uint16_t* beta,
                                                                  const uint16_t* bias, int D,
                                                                  uint16_t* wp, float* G, float* C) {
  __shared__ float red[2][4];
  const int n = blockIdx.x, f = n / 32, cr = n % 32;
  const int t = threadIdx.x;
  float gs = 0.f, cs = 0.f;
  for (int k = t; k < D; k += 256) {
    const float wk = E::to_f32(w[(int64_t)n * ws + k]);
    const float gk = gamma ? E::to_f32(gamma[k]) : 1.f;
    const uint16_t q = E::from_f32(gk * wk);
    const int s = k / 16, h = (k / 8) & 1, e = k & 7;
    wp[(((int64_t)f * (D / 16) + s) * 64 + cr + 32 * h) * 8 + e] = q;
    gs += E::to_f32(q);
    if (beta) cs = __builtin_fmaf(E::to_f32(beta[k]), wk, cs);
  }
  gs = group_sum<64>(gs);
  cs = group_sum<64>(cs);
  if ((t & 63) == 0) {
    red[0][t >> 6] = gs;
    red[1][t >> 6] = cs;
  }
  __syncthreads();
  if (t == 0) {
    G[n] = (red[0][0] + red[0][1]) + (red[0][2] + red[0][3]);
    C[n] = (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]) + (bias ? E::to_f32(bias[n]) : 0.f);
  }
}

// Workgroups of this kernel that the current device holds at once (CUs x
// blocks per CU), found once per device.
template <typename E, int NB, bool RES, bool LN>
static int fold_slots() {
  static std::atomic<int> slots[64];
  int dev = 0;
  (void)hipGetDevice(&dev);
  std::atomic<int>& s = slots[dev & 63];
  int v = s.load();
  if (v > 0) return v;
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, colbert_fold_kernel<E, NB, RES, LN>, 256, 0) !=
          hipSuccess ||
      per_cu <= 0)
    per_cu = 1;
  v = cus * per_cu;
  s.store(v);
  return v;
}

template <typename E, int NB, bool RES, bool LN>
static void launch_fold(FoldArgs a, hipStream_t st) {
  // as many workgroups as fit at once, each with an equal share of tokens
  const int64_t chunks = (a.T + kFoldTok - 1) / kFoldTok;
  const int64_t grid = std::min<int64_t>(chunks, fold_slots<E, NB, RES, LN>());
  a.per = (a.T + grid - 1) / grid;
  hipLaunchKernelGGL((colbert_fold_kernel<E, NB, RES, LN>), dim3((unsigned)grid), dim3(256), 0, st, a);
}

template <typename E, int NCH, bool PACKED>
static void launch_head(const HeadArgs& a, hipStream_t st) {
  const size_t lds = (size_t)kHeadRows * (NCH * 256 + kHeadPad) * 2 + 4 * 32 * sizeof(float);
  const unsigned grid = (unsigned)((a.T + kHeadRows - 1) / kHeadRows);
  if (lds > 65536) {
    // above the default dynamic-LDS limit: raise it once per device (bit d)
    static std::atomic<uint64_t> raised{0};
    int dev = 0;
    (void)hipGetDevice(&dev);
    const uint64_t bit = 1ull << (dev & 63);
    if (!(raised.load() & bit)) {
      (void)hipFuncSetAttribute((const void*)colbert_head_kernel<E, NCH, PACKED>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      raised.fetch_or(bit);
    }
  }
  hipLaunchKernelGGL((colbert_head_kernel<E, NCH, PACKED>), dim3(grid), dim3(256), lds, st, a);
}

}  // namespace vfk

using namespace vfk;

static int check_vec(const vfk_tensor* t, const char* name, int dt, int64_t n) {
  int rc = check_tensor(t, name, 1);
  if (rc) return rc;
  if (t->dtype != dt) return set_error(VFK_ERR_INVALID, "%s: dtype differs from x", name);
  if (t->size[0] != n || (n > 1 && t->stride[0] != 1))
    return set_error(VFK_ERR_INVALID, "%s: expected a contiguous [%lld]", name, (long long)n);
  if (reinterpret_cast<uintptr_t>(t->data) & 7)
    return set_error(VFK_ERR_INVALID, "%s: must be 8-byte aligned", name);
  return VFK_OK;
}

static int check_rows(const vfk_tensor* t, const char* name, int dt, int64_t rows, int64_t cols,
                      int align_elems) {
  int rc = check_tensor(t, name, 2);
  if (rc) return rc;
  if (t->dtype != dt) return set_error(VFK_ERR_INVALID, "%s: dtype differs from x", name);
  if (t->size[0] != rows || t->size[1] != cols)
    return set_error(VFK_ERR_INVALID, "%s: expected [%lld, %lld]", name, (long long)rows,
                     (long long)cols);
  if (t->stride[1] != 1) return set_error(VFK_ERR_INVALID, "%s: rows must be contiguous", name);
  if (t->stride[0] % align_elems ||
      (reinterpret_cast<uintptr_t>(t->data) & (uintptr_t)(align_elems * 2 - 1)))
    return set_error(VFK_ERR_INVALID, "%s: rows must be %d-byte aligned", name, align_elems * 2);
  return VFK_OK;
}

extern "C" int vfk_colbert_head_fwd(const vfk_tensor* x, const vfk_tensor* residual,
                                    const vfk_tensor* ln_weight, const vfk_tensor* ln_bias,
                                    float eps, const vfk_tensor* weight, const vfk_tensor* bias,
                                    vfk_tensor* hidden_out, vfk_tensor* out, void* stream) {
  int rc = check_tensor(x, "x", 2);
  if (rc) return rc;
  const int dt = x->dtype;
  if (dt != VFK_BF16 && dt != VFK_F16)
    return set_error(VFK_ERR_UNSUPPORTED, "vfk_colbert_head_fwd: x must be bf16 or fp16");
  const int64_t T = x->size[0], D = x->size[1];
  if (!present(weight)) return set_error(VFK_ERR_INVALID, "vfk_colbert_head_fwd: weight is NULL");
  const bool packed = weight->ndim == 4;
  rc = check_tensor(weight, "weight", packed ? 4 : 2);
  if (rc) return rc;
  const int64_t N = packed ? 32 * weight->size[0] : weight->size[0];
  if (D % 256 || D < 256 || D > 1024)
    return set_error(VFK_ERR_UNSUPPORTED, "vfk_colbert_head_fwd: hidden size %lld (needs a multiple "
                     "of 256 up to 1024)", (long long)D);
  if (N % 32 || N < 32 || N > 128)
    return set_error(VFK_ERR_UNSUPPORTED, "vfk_colbert_head_fwd: output size %lld (needs 32, 64, 96 "
                     "or 128)", (long long)N);
  if (packed) {
    if (weight->dtype != dt || weight->size[1] != D / 16 || weight->size[2] != 64 || weight->size[3] != 8 ||
        weight->stride[3] != 1 || weight->stride[2] != 8 || weight->stride[1] != 512 ||
        weight->stride[0] != 512 * (D / 16) || (reinterpret_cast<uintptr_t>(weight->data) & 15))
      return set_error(VFK_ERR_INVALID,
                       "vfk_colbert_head_fwd: a packed weight must be a contiguous, 16-byte aligned "
                       "[N / 32, %lld, 64, 8] of x's dtype (vfk_pack_weight_mfma32)", (long long)(D / 16));
  } else if ((rc = check_rows(weight, "weight", dt, N, D, 8))) {
    return rc;
  }
  if ((rc = check_rows(x, "x", dt, T, D, 4)) || (rc = check_rows(out, "out", dt, T, N, 4)))
    return rc;
  if (present(residual) && (rc = check_rows(residual, "residual", dt, T, D, 4))) return rc;
  if (present(hidden_out) && (rc = check_rows(hidden_out, "hidden_out", dt, T, D, 4))) return rc;
  if (present(ln_weight) && (rc = check_vec(ln_weight, "ln_weight", dt, D))) return rc;
  if (present(ln_bias)) {
    if (!present(ln_weight))
      return set_error(VFK_ERR_INVALID, "vfk_colbert_head_fwd: ln_bias needs ln_weight");
    if ((rc = check_vec(ln_bias, "ln_bias", dt, D))) return rc;
  }
  if (present(bias) && (rc = check_vec(bias, "bias", dt, N))) return rc;
  if (T == 0) return VFK_OK;
  if (T >= (1ll << 36)) return set_error(VFK_ERR_UNSUPPORTED, "vfk_colbert_head_fwd: too many rows");
  HeadArgs a = {};
  a.x = static_cast<const uint16_t*>(x->data); a.xs = x->stride[0];
  if (present(residual)) { a.r = static_cast<const uint16_t*>(residual->data); a.rs = residual->stride[0]; }
  if (present(ln_weight)) a.lnw = static_cast<const uint16_t*>(ln_weight->data);
  if (present(ln_bias)) a.lnb = static_cast<const uint16_t*>(ln_bias->data);
  a.eps = eps;
  a.w = static_cast<const uint16_t*>(weight->data); a.ws = packed ? 0 : weight->stride[0];
  if (present(bias)) a.bias = static_cast<const uint16_t*>(bias->data);
  if (present(hidden_out)) { a.h = static_cast<uint16_t*>(hidden_out->data); a.hs = hidden_out->stride[0]; }
  a.y = static_cast<uint16_t*>(out->data); a.ys = out->stride[0];
  a.T = T; a.D = (int)D; a.N = (int)N;
  hipStream_t st = (hipStream_t)stream;
  const int nch = (int)(D / 256);
#define VFK_HEAD(E, P)                                \
  switch (nch) {                                      \
    case 1: launch_head<E, 1, P>(a, st); break;       \
    case 2: launch_head<E, 2, P>(a, st); break;       \
    case 3: launch_head<E, 3, P>(a, st); break;       \
    default: launch_head<E, 4, P>(a, st); break;      \
  }
  if (dt == VFK_BF16) {
    if (packed) { VFK_HEAD(BF16, true) } else { VFK_HEAD(BF16, false) }
  } else {
    if (packed) { VFK_HEAD(F16, true) } else { VFK_HEAD(F16, false) }
  }
#undef VFK_HEAD
  return launch_status("vfk_colbert_head_fwd");
}

static int check_f32_vec(const vfk_tensor* t, const char* name, int64_t n) {
  int rc = check_tensor(t, name, 1);
  if (rc) return rc;
  if (t->dtype != VFK_F32) return set_error(VFK_ERR_INVALID, "%s: must be fp32", name);
  if (t->size[0] != n || t->stride[0] != 1 || (reinterpret_cast<uintptr_t>(t->data) & 15))
    return set_error(VFK_ERR_INVALID, "%s: expected a contiguous, 16-byte aligned [%lld]", name,
                     (long long)n);
  return VFK_OK;
}

static int check_folded(const vfk_tensor* t, int dt, int64_t N, int64_t D, const char* fn) {
  int rc = check_tensor(t, "folded", 4);
  if (rc) return rc;
  if (t->dtype != dt || t->size[0] != N / 32 || t->size[1] != D / 16 || t->size[2] != 64 ||
      t->size[3] != 8 || t->stride[3] != 1 || t->stride[2] != 8 || t->stride[1] != 512 ||
      t->stride[0] != 512 * (D / 16) || (reinterpret_cast<uintptr_t>(t->data) & 15))
    return set_error(VFK_ERR_INVALID, "%s: folded must be a contiguous, 16-byte aligned "
                     "[%lld, %lld, 64, 8] of the weight's dtype", fn, (long long)(N / 32),
                     (long long)(D / 16));
  return VFK_OK;
}

static int check_fold_sizes(int64_t D, int64_t N, const char* fn) {
  if (D % 128 || D < 128 || D > 4096)
    return set_error(VFK_ERR_UNSUPPORTED, "%s: hidden size %lld (needs a multiple of 128 up to 4096)",
                     fn, (long long)D);
  if (N % 32 || N < 32 || N > 128)
    return set_error(VFK_ERR_UNSUPPORTED, "%s: output size %lld (needs 32, 64, 96 or 128)", fn,
                     (long long)N);
  return VFK_OK;
}

extern "C" int vfk_colbert_fold_weight(const vfk_tensor* weight, const vfk_tensor* ln_weight,
                                       const vfk_tensor* ln_bias, const vfk_tensor* bias,
                                       vfk_tensor* folded, vfk_tensor* gsum, vfk_tensor* cvec,
                                       void* stream) {
  static const char* fn = "vfk_colbert_fold_weight";
  int rc = check_tensor(weight, "weight", 2);
  if (rc) return rc;
  const int dt = weight->dtype;
  if (dt != VFK_BF16 && dt != VFK_F16)
    return set_error(VFK_ERR_UNSUPPORTED, "%s: weight must be bf16 or fp16", fn);
  const int64_t N = weight->size[0], D = weight->size[1];
  if ((rc = check_fold_sizes(D, N, fn))) return rc;
  if (weight->stride[1] != 1) return set_error(VFK_ERR_INVALID, "%s: weight rows must be contiguous", fn);
  if ((rc = check_folded(folded, dt, N, D, fn)) || (rc = check_f32_vec(gsum, "gsum", N)) ||
      (rc = check_f32_vec(cvec, "cvec", N)))
    return rc;
  if (present(ln_weight) && (rc = check_vec(ln_weight, "ln_weight", dt, D))) return rc;
  if (present(ln_bias)) {
    if (!present(ln_weight)) return set_error(VFK_ERR_INVALID, "%s: ln_bias needs ln_weight", fn);
    if ((rc = check_vec(ln_bias, "ln_bias", dt, D))) return rc;
  }
  if (present(bias) && (rc = check_vec(bias, "bias", dt, N))) return rc;
  const uint16_t* w = static_cast<const uint16_t*>(weight->data);
  const uint16_t* g = present(ln_weight) ? static_cast<const uint16_t*>(ln_weight->data) : nullptr;
  const uint16_t* b = present(ln_bias) ? static_cast<const uint16_t*>(ln_bias->data) : nullptr;
  const uint16_t* bb = present(bias) ? static_cast<const uint16_t*>(bias->data) : nullptr;
  uint16_t* wp = static_cast<uint16_t*>(folded->data);
  float* G = static_cast<float*>(gsum->data);
  float* C = static_cast<float*>(cvec->data);
  hipStream_t st = (hipStream_t)stream;
  if (dt == VFK_BF16)
    hipLaunchKernelGGL(colbert_fold_weight_kernel<BF16>, dim3((unsigned)N), dim3(256), 0, st, w,
                       weight->stride[0], g, b, bb, (int)D, wp, G, C);
  else
    hipLaunchKernelGGL(colbert_fold_weight_kernel<F16>, dim3((unsigned)N), dim3(256), 0, st, w,
                       weight->stride[0], g, b, bb, (int)D, wp, G, C);
  return launch_status(fn);
}

extern "C" int vfk_colbert_head_folded_fwd(const vfk_tensor* x, const vfk_tensor* residual,
                                           const vfk_tensor* folded, const vfk_tensor* gsum,
                                           const vfk_tensor* cvec, float eps, vfk_tensor* out,
                                           void* stream) {
  static const char* fn = "vfk_colbert_head_folded_fwd";
  int rc = check_tensor(x, "x", 2);
  if (rc) return rc;
  const int dt = x->dtype;
  if (dt != VFK_BF16 && dt != VFK_F16) return set_error(VFK_ERR_UNSUPPORTED, "%s: x must be bf16 or fp16", fn);
  const int64_t T = x->size[0], D = x->size[1];
  if ((rc = check_tensor(folded, "folded", 4))) return rc;
  const int64_t N = 32 * folded->size[0];
  if ((rc = check_fold_sizes(D, N, fn)) || (rc = check_folded(folded, dt, N, D, fn)) ||
      (rc = check_f32_vec(cvec, "cvec", N)))
    return rc;
  if (present(gsum) && (rc = check_f32_vec(gsum, "gsum", N))) return rc;
  if ((rc = check_rows(x, "x", dt, T, D, 8)) || (rc = check_rows(out, "out", dt, T, N, 8))) return rc;
  if (present(residual) && (rc = check_rows(residual, "residual", dt, T, D, 8))) return rc;
  if (T == 0) return VFK_OK;
  if (T >= (1ll << 36)) return set_error(VFK_ERR_UNSUPPORTED, "%s: too many rows", fn);
  // a wave's 32 rows are addressed with 32-bit byte offsets
  if (x->stride[0] >= (1ll << 25) || (present(residual) && residual->stride[0] >= (1ll << 25)))
    return set_error(VFK_ERR_UNSUPPORTED, "%s: row stride too large", fn);
  FoldArgs a = {};
  a.x = static_cast<const uint16_t*>(x->data); a.xs = x->stride[0];
  const bool res = present(residual), ln = present(gsum);
  if (res) { a.r = static_cast<const uint16_t*>(residual->data); a.rs = residual->stride[0]; }
  a.w = static_cast<const uint16_t*>(folded->data);
  if (ln) a.g = static_cast<const float*>(gsum->data);
  a.c = static_cast<const float*>(cvec->data);
  a.eps = eps;
  a.y = static_cast<uint16_t*>(out->data); a.ys = out->stride[0];
  a.T = T; a.D = (int)D; a.N = (int)N;
  hipStream_t st = (hipStream_t)stream;
  const int nb = (int)(N / 32);
#define VFK_FOLD_NB(E, R, L)                            \
  switch (nb) {                                         \
    case 1: launch_fold<E, 1, R, L>(a, st); break;      \
    case 2: launch_fold<E, 2, R, L>(a, st); break;      \
    case 3: launch_fold<E, 3, R, L>(a, st); break;      \
    default: launch_fold<E, 4, R, L>(a, st); break;     \
  }
#define VFK_FOLD(E)                                     \
  if (res) {                                            \
    if (ln) { VFK_FOLD_NB(E, true, true) } else { VFK_FOLD_NB(E, true, false) } \
  } else {                                              \
    if (ln) { VFK_FOLD_NB(E, false, true) } else { VFK_FOLD_NB(E, false, false) } \
  }
  if (dt == VFK_BF16) { VFK_FOLD(BF16) } else { VFK_FOLD(F16) }
#undef VFK_FOLD
#undef VFK_FOLD_NB
  return launch_status(fn);
}
