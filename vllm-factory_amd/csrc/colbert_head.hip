// ColBERT output head on gfx950: LayerNorm -> projection -> L2 normalisation.
//
// Replaces the last steps of the reference's ModernBERT ColBERT plugin
// (plugins/moderncolbert/model.py:260-267: the final LayerNorm of the encoder,
// then the PyLate Dense projection, then projected / projected.norm()
// clamped at 1e-8) with one pass over the hidden rows: the normalised rows
// never go back to HBM unless the caller asks for them.
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

#include <atomic>

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
