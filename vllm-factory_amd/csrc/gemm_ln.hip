// Dense projection with the bias, residual add and LayerNorm in the epilogue
// (bf16 / fp16 on v_mfma_f32_32x32x16, gfx950).
//
// out[t] = LayerNorm(round(x[t] W^T + bias) + residual[t]) for x [M, K] and
// W [N, K]: DeBERTa's post-LN output blocks, DebertaV2SelfOutput and
// DebertaV2Output (models/deberta_v2/deberta_v2_encoder.py:494-510 and
// 553-568; dropout is the identity at inference). The dense output is rounded
// to the storage type, as the unfused Linear writes it, and the LayerNorm
// runs in fp32 on that value plus the residual, as vfk_layernorm_fwd does;
// the [M, N] dense output never reaches memory.
//
// A LayerNorm needs whole rows, so a 512-thread workgroup owns 64 tokens and
// all N = 256 NB features (N <= 1024): 64 x 1024 fp32 sums are 256 KiB, half
// of a CU's register file, held by 8 waves (2 per SIMD). Wave w owns features
// 32 NB w .. +32 NB: NB feature blocks x 2 token blocks of 32 x 32. A = weight
// rows, B = token rows, so lane (c, h) of a result block holds token c and
// features 8 (r / 4) + 4 h + r % 4 (r < 16).
//
// Every workgroup streams the whole weight, and an MFMA operand puts a
// different row in every lane: loaded from [N, K] rows, each 1 KiB wave load
// would touch 32 cache lines. The weight is therefore packed once
// (vfk_pack_weight_mfma32) into operand order, [N/32][K/16][64 lanes][8]:
// block (F, s) holds rows 32 F .. +32 and k = 16 s .. +16, lane c + 32 h's
// 16 bytes being row 32 F + c, k = 16 s + 8 h .. +8. A wave's operand load is
// then one contiguous KiB, straight into registers (a weight row is used by
// one wave only), issued three 16-wide k-steps ahead of its MFMAs into four
// rotating buffers.
//
// The 64 token rows are shared by all 8 waves: each 64-wide K slice is read
// with one coalesced 16-byte load per thread, written to one of two LDS
// stages (rows padded to 144 bytes: the operand reads of 8 lanes hit distinct
// banks) and read back as B operands after one barrier per slice. The next
// slice's load is issued before the current slice's MFMAs.
//
// Epilogue: the bias is added, the sums are rounded and written to LDS as
// [64][N] rows (over the token stages), and after one barrier each wave
// normalises 8 rows, 16 bytes per lane and chunk, with wave reductions; the
// residual rows are read with 16-byte loads issued before the barrier.
#include "attn_core.h"
#include "launch_util.h"

#include <type_traits>

namespace vfk {
namespace {

constexpr int kDlRows = 64;            // tokens per workgroup
constexpr int kDlXRow = 144;           // LDS bytes of one token row of a 64-wide K slice
constexpr int kDlXStage = kDlRows * kDlXRow;

struct DenseLnArgs {
  const uint16_t* x;
  const uint16_t* wp;    // packed weight [N/32][K/16][64][8]
  const uint16_t* bias;  // [N] or null
  const uint16_t* res;   // [M, N]
  const uint16_t* g;     // LayerNorm weight [N] or null (ones)
  const uint16_t* b;     // LayerNorm bias [N] or null (zeros)
  uint16_t* out;         // [M, N]; may be the residual itself
  uint16_t* rout;        // [M, N] or null: the sum (rounded); may be the residual itself
  int64_t M;
  int K;
  int xs2, rs2;  // row strides of x and residual in bytes
  int64_t os;    // row stride of out in elements
  int64_t ros;   // row stride of rout in elements
  float eps;
};

// LDS barrier that leaves outstanding global loads in flight (a release
// fence would wait for the weight prefetch too).
__device__ inline void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// weight operands of 16-wide k-step q: one contiguous KiB per feature block
template <int NB>
__device__ inline void dl_load_w(u32x4_t (&wa)[NB], rsrc_t wr, const int (&wo)[NB], int q) {
#pragma unroll
  for (int f = 0; f < NB; ++f) wa[f] = __builtin_amdgcn_raw_buffer_load_b128(wr, wo[f], 1024 * q, 0);
}

// B operands of k-step j (0..3) of the 64-wide slice in an LDS stage
__device__ inline void dl_read_x(u32x4_t (&xb)[2], const char* stage, int c, int h, int j) {
#pragma unroll
  for (int tb = 0; tb < 2; ++tb)
    xb[tb] = *reinterpret_cast<const u32x4_t*>(stage + (32 * tb + c) * kDlXRow + 16 * (2 * j + h));
}

template <typename E, int NB>
__device__ inline void dl_mfma(f32x16_t (&acc)[NB][2], const u32x4_t (&wa)[NB], const u32x4_t (&xb)[2]) {
#pragma unroll
  for (int f = 0; f < NB; ++f)
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) acc[f][tb] = E::mfma32(wa[f], xb[tb], acc[f][tb]);
}

template <typename E, int NB>
__global__ __launch_bounds__(512) void dense_ln_kernel(DenseLnArgs a) {
  constexpr int N = 256 * NB;
  constexpr int RS = 2 * N + 16;      // LDS row stride of the result rows (16-byte aligned)
  constexpr int NCH = N / 8;          // 16-byte chunks of a row
  constexpr int CH = (NCH + 63) / 64; // chunks per lane
  constexpr int kLds = kDlRows * RS > 2 * kDlXStage ? kDlRows * RS : 2 * kDlXStage;
  __shared__ __attribute__((aligned(16))) char smem[kLds];
  char* const ytile = smem;

  const int t = threadIdx.x, lane = t & 63, w = t >> 6, c = lane & 31, h = lane >> 5;
  const int64_t tok0 = (int64_t)blockIdx.x * kDlRows;
  const int rows = (int)min((int64_t)kDlRows, a.M - tok0);
  const int fbase = 32 * NB * w;
  const int KS = a.K >> 4;  // 16-wide k-steps

  // token rows past M read as zeros through the range check
  const rsrc_t xr = uniform_rsrc(a.x + tok0 * (a.xs2 >> 1), rows * a.xs2);
  const rsrc_t wr = uniform_rsrc(a.wp, N * a.K * 2);
  int wo[NB];
#pragma unroll
  for (int f = 0; f < NB; ++f) wo[f] = ((fbase >> 5) + f) * KS * 1024 + 16 * lane;
  // this thread's 16 bytes of a token slice: row t / 8, chunk t % 8
  const int xo = (t >> 3) * a.xs2 + 16 * (t & 7);
  const int xl = (t >> 3) * kDlXRow + 16 * (t & 7);

  f32x16_t acc[NB][2];
#pragma unroll
  for (int f = 0; f < NB; ++f)
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) acc[f][tb] = f32x16_t{};

  const int T = a.K >> 6;  // 64-wide slices
  // four k-step buffers: k-step q's operands are loaded three k-steps
  // (3/4 of a slice) before its MFMAs, into the buffer of k-step q - 1
  u32x4_t wq[4][NB], xb[2];
  u32x4_t xn = __builtin_amdgcn_raw_buffer_load_b128(xr, xo, 0, 0);
  dl_load_w<NB>(wq[0], wr, wo, 0);
  dl_load_w<NB>(wq[1], wr, wo, 1);
  dl_load_w<NB>(wq[2], wr, wo, 2);
  *reinterpret_cast<u32x4_t*>(smem + xl) = xn;
  lds_barrier();
  // slice s (k-steps 4 s .. 4 s + 3): its tokens are in stage s % 2; MORE:
  // slice s + 1 exists (its tokens are loaded now and written to the other
  // stage after the MFMAs: that stage was last read before the previous
  // barrier). The last slice is peeled off so that the loop body has no
  // branch, and each wait counts exactly the loads issued after the one it
  // waits for.
  auto step = [&](int s, auto more_tag) {
    constexpr bool MORE = decltype(more_tag)::value;
    const char* stage = smem + (s & 1) * kDlXStage;
    if (MORE) xn = __builtin_amdgcn_raw_buffer_load_b128(xr, xo, 128 * (s + 1), 0);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (MORE || j == 0) dl_load_w<NB>(wq[(j + 3) & 3], wr, wo, 4 * s + j + 3);
      dl_read_x(xb, stage, c, h, j);
      __builtin_amdgcn_sched_barrier(0);
      dl_mfma<E, NB>(acc, wq[j], xb);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (MORE) *reinterpret_cast<u32x4_t*>(smem + ((s + 1) & 1) * kDlXStage + xl) = xn;
    lds_barrier();
  };
  for (int s = 0; s < T - 1; ++s) step(s, std::true_type{});
  step(T - 1, std::false_type{});

  // bias (absent: a range of 0 bytes, every load reads zero), issued before
  // the residual loads so that waiting for it leaves those in flight
  const rsrc_t br = uniform_rsrc(a.bias, a.bias ? 2 * N : 0);
  u32x2_t bq[NB][4];
#pragma unroll
  for (int f = 0; f < NB; ++f)
#pragma unroll
    for (int g = 0; g < 4; ++g)
      bq[f][g] = __builtin_amdgcn_raw_buffer_load_b64(br, 2 * (fbase + 32 * f + 4 * h + 8 * g), 0, 0);

  // this lane's 16-byte chunks of a row: lane + 64 q; a lane past the row
  // repeats chunk `lane` with no weight in the statistics and no store
  int ch[CH];
  float keep[CH];
#pragma unroll
  for (int q = 0; q < CH; ++q) {
    const int cq = lane + 64 * q;
    keep[q] = cq < NCH ? 1.f : 0.f;
    ch[q] = cq < NCH ? cq : lane;
  }
  // residual rows 8 w .. 8 w + 7 of the tile (rows past M read as zeros)
  const rsrc_t rr = uniform_rsrc(a.res + tok0 * (a.rs2 >> 1), rows * a.rs2);
  u32x4_t rv[8][CH];
#pragma unroll
  for (int r = 0; r < 8; ++r)
#pragma unroll
    for (int q = 0; q < CH; ++q)
      rv[r][q] = __builtin_amdgcn_raw_buffer_load_b128(rr, (8 * w + r) * a.rs2 + 16 * ch[q], 0, 0);

  // bias, rounding to the storage type, rows [64][N] in LDS (the token
  // stages are free: every wave passed the loop's last barrier)
#pragma unroll
  for (int f = 0; f < NB; ++f) {
    const int f0 = fbase + 32 * f + 4 * h;  // features f0 + 8 g + i
    float bv[16];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      bv[4 * g] = E::to_f32((uint16_t)(bq[f][g][0] & 0xffffu));
      bv[4 * g + 1] = E::to_f32((uint16_t)(bq[f][g][0] >> 16));
      bv[4 * g + 2] = E::to_f32((uint16_t)(bq[f][g][1] & 0xffffu));
      bv[4 * g + 3] = E::to_f32((uint16_t)(bq[f][g][1] >> 16));
    }
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
      char* row = ytile + (32 * tb + c) * RS + 2 * f0;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x16_t& s = acc[f][tb];
        u32x2_t p;
        p[0] = E::pack2(s[4 * g] + bv[4 * g], s[4 * g + 1] + bv[4 * g + 1]);
        p[1] = E::pack2(s[4 * g + 2] + bv[4 * g + 2], s[4 * g + 3] + bv[4 * g + 3]);
        *reinterpret_cast<u32x2_t*>(row + 16 * g) = p;
      }
    }
  }
  __syncthreads();

  // LayerNorm weight and bias (absent: ones and zeros)
  const rsrc_t gr = uniform_rsrc(a.g, a.g ? 2 * N : 0), bbr = uniform_rsrc(a.b, a.b ? 2 * N : 0);
  const float gdef = a.g ? 0.f : 1.f;
  float gv[CH][8], bv[CH][8];
#pragma unroll
  for (int q = 0; q < CH; ++q) {
    unpack8<E>(__builtin_amdgcn_raw_buffer_load_b128(gr, 16 * ch[q], 0, 0), gv[q]);
    unpack8<E>(__builtin_amdgcn_raw_buffer_load_b128(bbr, 16 * ch[q], 0, 0), bv[q]);
#pragma unroll
    for (int i = 0; i < 8; ++i) gv[q][i] += gdef;
  }
  const float inv_n = 1.0f / (float)N;
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const int row = 8 * w + r;
    if (row >= rows) break;  // wave-uniform
    float v[CH][8];
    float s = 0.f;
#pragma unroll
    for (int q = 0; q < CH; ++q) {
      float y[8], x[8];
      unpack8<E>(*reinterpret_cast<const u32x4_t*>(ytile + row * RS + 16 * ch[q]), y);
      unpack8<E>(rv[r][q], x);
      float tq = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        v[q][i] = y[i] + x[i];
        tq += v[q][i];
      }
      s += keep[q] * tq;
    }
    const float mean = group_sum<64>(s) * inv_n;
    float d2 = 0.f;
#pragma unroll
    for (int q = 0; q < CH; ++q) {
      float tq = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float d = v[q][i] - mean;
        tq += d * d;
      }
      d2 += keep[q] * tq;
    }
    const float rstd = 1.0f / sqrtf(group_sum<64>(d2) * inv_n + a.eps);
    uint16_t* orow = a.out + (tok0 + row) * a.os;
#pragma unroll
    for (int q = 0; q < CH; ++q) {
      if (keep[q] != 0.f) {
        float o[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = (v[q][i] - mean) * rstd * gv[q][i] + bv[q][i];
        *reinterpret_cast<u32x4_t*>(orow + 8 * ch[q]) = pack8<E>(o);
        if (a.rout)
          *reinterpret_cast<u32x4_t*>(a.rout + (tok0 + row) * a.ros + 8 * ch[q]) = pack8<E>(v[q]);
      }
    }
  }
}

template <typename E>
static void launch_dense_ln(const DenseLnArgs& a, int nb, unsigned grid, hipStream_t st) {
  switch (nb) {
    case 1: hipLaunchKernelGGL((dense_ln_kernel<E, 1>), dim3(grid), dim3(512), 0, st, a); break;
    case 2: hipLaunchKernelGGL((dense_ln_kernel<E, 2>), dim3(grid), dim3(512), 0, st, a); break;
    case 3: hipLaunchKernelGGL((dense_ln_kernel<E, 3>), dim3(grid), dim3(512), 0, st, a); break;
    default: hipLaunchKernelGGL((dense_ln_kernel<E, 4>), dim3(grid), dim3(512), 0, st, a); break;
  }
}

// packed[F][s][l][i] = w[32 F + l % 32][16 s + 8 (l / 32) + i]: one thread
// per 16 bytes of the packed weight
__global__ __launch_bounds__(256) void dense_ln_pack_kernel(const uint16_t* __restrict__ w,
                                                            int64_t ws, int K, int64_t n16,
                                                            uint16_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n16) return;
  const int l = (int)(i & 63);
  const int64_t blk = i >> 6;
  const int KS = K >> 4;
  const int64_t F = blk / KS;
  const int s = (int)(blk - F * KS);
  const uint16_t* src = w + (32 * F + (l & 31)) * ws + 16 * s + 8 * (l >> 5);
  *reinterpret_cast<u32x4_t*>(out + 8 * i) = *reinterpret_cast<const u32x4_t*>(src);
}

// N in {256, 512, 768, 1024}, K a positive multiple of 64
int check_dense_dims(int64_t N, int64_t K) {
  if (N < 256 || N > 1024 || N % 256 != 0)
    return set_error(VFK_ERR_UNSUPPORTED, "dense_layernorm: N must be 256, 512, 768 or 1024, got %lld",
                     (long long)N);
  if (K < 64 || K % 64 != 0)
    return set_error(VFK_ERR_UNSUPPORTED, "dense_layernorm: K must be a positive multiple of 64, got %lld",
                     (long long)K);
  return VFK_OK;
}

}  // namespace
}  // namespace vfk

using namespace vfk;

extern "C" int vfk_pack_weight_mfma32(const vfk_tensor* w, vfk_tensor* packed, void* stream) {
  int rc;
  if ((rc = check_tensor(w, "w", 2)) || (rc = check_tensor(packed, "packed", 4))) return rc;
  const int dt = w->dtype;
  if (dt != VFK_BF16 && dt != VFK_F16)
    return set_error(VFK_ERR_UNSUPPORTED, "pack_weight_mfma32: w must be bf16 or fp16");
  const int64_t N = w->size[0], K = w->size[1];
  if (N < 32 || N % 32 || K < 16 || K % 16)
    return set_error(VFK_ERR_UNSUPPORTED,
                     "pack_weight_mfma32: w [%lld, %lld] needs rows a multiple of 32 and columns a "
                     "multiple of 16", (long long)N, (long long)K);
  if (packed->dtype != dt || packed->size[0] != N / 32 || packed->size[1] != K / 16 ||
      packed->size[2] != 64 || packed->size[3] != 8)
    return set_error(VFK_ERR_INVALID, "pack_weight_mfma32: packed must be [%lld, %lld, 64, 8] of w's dtype",
                     (long long)(N / 32), (long long)(K / 16));
  if (packed->stride[3] != 1 || packed->stride[2] != 8 || packed->stride[1] != 512 ||
      packed->stride[0] != 512 * (K / 16) || !aligned16(packed->data))
    return set_error(VFK_ERR_INVALID, "pack_weight_mfma32: packed must be contiguous and 16-byte aligned");
  if (w->stride[1] != 1 || w->stride[0] < K || w->stride[0] % 8 || !aligned16(w->data))
    return set_error(VFK_ERR_UNSUPPORTED,
                     "pack_weight_mfma32: w rows must be contiguous and 16-byte aligned");
  const int64_t n16 = N * K / 8;
  hipLaunchKernelGGL(dense_ln_pack_kernel, dim3((unsigned)((n16 + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(w->data),
                     w->stride[0], (int)K, n16, static_cast<uint16_t*>(packed->data));
  return launch_status("pack_weight_mfma32");
}

extern "C" int vfk_dense_residual_layernorm_fwd(const vfk_tensor* x, const vfk_tensor* w_packed,
                                                const vfk_tensor* bias, const vfk_tensor* residual,
                                                const vfk_tensor* ln_weight,
                                                const vfk_tensor* ln_bias, float eps,
                                                vfk_tensor* out, vfk_tensor* residual_out,
                                                void* stream) {
  int rc;
  if ((rc = check_tensor(x, "x", 2)) || (rc = check_tensor(w_packed, "w_packed", 4)) ||
      (rc = check_tensor(residual, "residual", 2)) || (rc = check_tensor(out, "out", 2)))
    return rc;
  if (present(bias) && (rc = check_tensor(bias, "bias", 1))) return rc;
  if (present(ln_weight) && (rc = check_tensor(ln_weight, "ln_weight", 1))) return rc;
  if (present(ln_bias) && (rc = check_tensor(ln_bias, "ln_bias", 1))) return rc;
  const bool rsum = present(residual_out);
  if (rsum && (rc = check_tensor(residual_out, "residual_out", 2))) return rc;
  const int dt = x->dtype;
  if (dt != VFK_BF16 && dt != VFK_F16)
    return set_error(VFK_ERR_UNSUPPORTED, "dense_layernorm: x must be bf16 or fp16");
  const int64_t M = x->size[0], K = x->size[1], N = 32 * w_packed->size[0];
  if (w_packed->dtype != dt || residual->dtype != dt || out->dtype != dt)
    return set_error(VFK_ERR_INVALID, "dense_layernorm: x, w, residual and out must share one dtype");
  if (w_packed->size[1] * 16 != K || w_packed->size[2] != 64 || w_packed->size[3] != 8)
    return set_error(VFK_ERR_INVALID,
                     "dense_layernorm: w_packed must be [N / 32, K / 16, 64, 8] for x [M, K] (K = %lld)",
                     (long long)K);
  if (w_packed->stride[3] != 1 || w_packed->stride[2] != 8 || w_packed->stride[1] != 512 ||
      w_packed->stride[0] != 512 * w_packed->size[1] || !aligned16(w_packed->data))
    return set_error(VFK_ERR_INVALID, "dense_layernorm: w_packed must be contiguous and 16-byte aligned");
  if ((rc = check_dense_dims(N, K))) return rc;
  if (residual->size[0] != M || residual->size[1] != N || out->size[0] != M || out->size[1] != N)
    return set_error(VFK_ERR_INVALID, "dense_layernorm: residual and out must be [M, N] = [%lld, %lld]",
                     (long long)M, (long long)N);
  if (rsum && (residual_out->dtype != dt || residual_out->size[0] != M || residual_out->size[1] != N ||
               residual_out->stride[1] != 1 || !aligned16(residual_out->data) ||
               residual_out->stride[0] % 8 || residual_out->stride[0] < N))
    return set_error(VFK_ERR_INVALID,
                     "dense_layernorm: residual_out must be [M, N] of x's dtype, rows contiguous and "
                     "16-byte aligned");
  const vfk_tensor* params[3] = {bias, ln_weight, ln_bias};
  const char* pnames[3] = {"bias", "ln_weight", "ln_bias"};
  for (int i = 0; i < 3; ++i) {
    const vfk_tensor* p = params[i];
    if (!present(p)) continue;
    if (p->dtype != dt || p->size[0] != N || p->stride[0] != 1 || !aligned16(p->data))
      return set_error(VFK_ERR_INVALID,
                       "dense_layernorm: %s must be a contiguous, 16-byte aligned [%lld] of x's dtype",
                       pnames[i], (long long)N);
  }
  if (x->stride[1] != 1 || residual->stride[1] != 1 || out->stride[1] != 1)
    return set_error(VFK_ERR_UNSUPPORTED, "dense_layernorm: rows must be contiguous");
  if (!aligned16(x->data) || !aligned16(residual->data) || !aligned16(out->data) ||
      x->stride[0] % 8 || residual->stride[0] % 8 || out->stride[0] % 8)
    return set_error(VFK_ERR_UNSUPPORTED,
                     "dense_layernorm: base pointers and row strides must be 16-byte aligned");
  if (x->stride[0] < K || residual->stride[0] < N || out->stride[0] < N)
    return set_error(VFK_ERR_INVALID, "dense_layernorm: overlapping rows");
  // a workgroup's buffer ranges: 64 rows of x and residual, the whole weight
  if ((int64_t)kDlRows * x->stride[0] * 2 >= (1ll << 31) ||
      (int64_t)kDlRows * residual->stride[0] * 2 >= (1ll << 31) || N * K * 2 >= (1ll << 31))
    return set_error(VFK_ERR_UNSUPPORTED, "dense_layernorm: row strides or w too large");
  if (!(eps >= 0.f)) return set_error(VFK_ERR_INVALID, "dense_layernorm: eps must be >= 0");
  // each output either is the residual (same rows) or overlaps neither input,
  // and the two outputs do not overlap
  auto overlap = [M](const vfk_tensor* p, const vfk_tensor* q) {
    const char* pb = static_cast<const char*>(p->data);
    const char* pe = pb + ((M - 1) * p->stride[0] + p->size[1]) * 2;
    const char* qb = static_cast<const char*>(q->data);
    const char* qe = qb + ((M - 1) * q->stride[0] + q->size[1]) * 2;
    return pb < qe && qb < pe;
  };
  const vfk_tensor* outs[2] = {out, rsum ? residual_out : nullptr};
  if (M > 0) {
    for (const vfk_tensor* o : outs) {
      if (!o) continue;
      const bool is_res = o->data == residual->data && o->stride[0] == residual->stride[0];
      if (overlap(o, x) || (!is_res && overlap(o, residual)))
        return set_error(VFK_ERR_INVALID,
                         "dense_layernorm: an output overlaps an input other than the residual");
    }
    if (rsum && overlap(out, residual_out))
      return set_error(VFK_ERR_INVALID, "dense_layernorm: out and residual_out overlap");
  }
  if (M == 0) return VFK_OK;
  const int64_t grid = (M + kDlRows - 1) / kDlRows;
  if (grid >= (1ll << 31)) return set_error(VFK_ERR_UNSUPPORTED, "dense_layernorm: too many rows");
  DenseLnArgs a = {};
  a.x = static_cast<const uint16_t*>(x->data);
  a.wp = static_cast<const uint16_t*>(w_packed->data);
  a.bias = present(bias) ? static_cast<const uint16_t*>(bias->data) : nullptr;
  a.res = static_cast<const uint16_t*>(residual->data);
  a.g = present(ln_weight) ? static_cast<const uint16_t*>(ln_weight->data) : nullptr;
  a.b = present(ln_bias) ? static_cast<const uint16_t*>(ln_bias->data) : nullptr;
  a.out = static_cast<uint16_t*>(out->data);
  a.rout = rsum ? static_cast<uint16_t*>(residual_out->data) : nullptr;
  a.ros = rsum ? residual_out->stride[0] : 0;
  a.M = M;
  a.K = (int)K;
  a.xs2 = (int)(x->stride[0] * 2);
  a.rs2 = (int)(residual->stride[0] * 2);
  a.os = out->stride[0];
  a.eps = eps;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int nb = (int)(N / 256);
  if (dt == VFK_BF16)
    launch_dense_ln<BF16>(a, nb, (unsigned)grid, st);
  else
    launch_dense_ln<F16>(a, nb, (unsigned)grid, st);
  return launch_status("dense_layernorm");
}
