// Memory-bound epilogues: RoPE (table form), LayerNorm, RMSNorm, gated
// activations and residual add. All arithmetic is fp32 in registers; every
// HBM access on the fast path is a 128-bit load or store.
#include <math.h>

#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "activation.h"
#include "launch_util.h"
#include "vfk_common.h"

namespace vfk {

// ---------------------------------------------------------------------------
// Element access: VEC elements = 16 bytes.
// ---------------------------------------------------------------------------
template <int DT>
struct Elt;

template <>
struct Elt<VFK_F32> {
  static constexpr int VEC = 4;
  __device__ static inline void load(const void* base, int64_t i, float* f) {
    f32x4_t v = *reinterpret_cast<const f32x4_t*>(
        reinterpret_cast<const float*>(base) + i);
    f[0] = v[0]; f[1] = v[1]; f[2] = v[2]; f[3] = v[3];
  }
  __device__ static inline void store(void* base, int64_t i, const float* f) {
    f32x4_t v = {f[0], f[1], f[2], f[3]};
    *reinterpret_cast<f32x4_t*>(reinterpret_cast<float*>(base) + i) = v;
  }
  __device__ static inline void load_nt(const void* base, int64_t i, float* f) {
    const f32x4_t v = __builtin_nontemporal_load(
        reinterpret_cast<const f32x4_t*>(reinterpret_cast<const float*>(base) + i));
    f[0] = v[0]; f[1] = v[1]; f[2] = v[2]; f[3] = v[3];
  }
  __device__ static inline float ld1(const void* base, int64_t i) {
    return reinterpret_cast<const float*>(base)[i];
  }
  __device__ static inline void st1(void* base, int64_t i, float v) {
    reinterpret_cast<float*>(base)[i] = v;
  }
};

template <typename E>
struct Elt16 {
  static constexpr int VEC = 8;
  __device__ static inline void load(const void* base, int64_t i, float* f) {
    u32x4_t v = *reinterpret_cast<const u32x4_t*>(
        reinterpret_cast<const uint16_t*>(base) + i);
    unpack8<E>(v, f);
  }
  __device__ static inline void store(void* base, int64_t i, const float* f) {
    *reinterpret_cast<u32x4_t*>(reinterpret_cast<uint16_t*>(base) + i) =
        pack8<E>(f);
  }
  // streaming load for the large, read-once operands of the gated
  // activations (the FFN up/gate projections, larger than the last-level
  // cache): they are kept out of the caches, which then still hold the output
  // for the GEMM that consumes it. Inputs that a previous kernel has just
  // written and that fit in the caches (the norms' rows) use plain loads.
  __device__ static inline void load_nt(const void* base, int64_t i, float* f) {
    const u32x4_t v = __builtin_nontemporal_load(
        reinterpret_cast<const u32x4_t*>(reinterpret_cast<const uint16_t*>(base) + i));
    unpack8<E>(v, f);
  }
  __device__ static inline float ld1(const void* base, int64_t i) {
    return E::to_f32(reinterpret_cast<const uint16_t*>(base)[i]);
  }
  __device__ static inline void st1(void* base, int64_t i, float v) {
    reinterpret_cast<uint16_t*>(base)[i] = E::from_f32(v);
  }
};
template <>
struct Elt<VFK_BF16> : Elt16<BF16> {};
template <>
struct Elt<VFK_F16> : Elt16<F16> {};

// Generic scalar access for mixed-dtype parameters (weights may differ).
__device__ inline float ld_any(const void* base, int dt, int64_t i) {
  if (dt == VFK_F32) return reinterpret_cast<const float*>(base)[i];
  if (dt == VFK_BF16) return BF16::to_f32(reinterpret_cast<const uint16_t*>(base)[i]);
  return F16::to_f32(reinterpret_cast<const uint16_t*>(base)[i]);
}

// ---------------------------------------------------------------------------
// LayerNorm / RMSNorm (one group of LANES lanes per row)
// ---------------------------------------------------------------------------
struct NormArgs {
  const void* x; int64_t x_rs;
  const void* res; int64_t res_rs;        // optional residual added first
  void* res_out; int64_t res_out_rs;      // optional: writes x + res
  const void* w; int w_dt;                // optional weight
  const void* b; int b_dt;                // optional bias (LayerNorm only)
  int w_vec, b_vec;                       // 16-byte aligned: 128-bit loads allowed
  void* y; int64_t y_rs;
  int64_t rows; int n; float eps;
};

// Grid-stride over rows: each lane owns the same columns in every row, so its
// weight / bias slices are loaded once into registers; only x (and the
// residual) stream through, as 128-bit loads. The row loop is instantiated
// per residual mode so that its body is straight-line: all loads of a row are
// issued before the first use, partial chunks and rows past the end load a
// clamped in-bounds address and are masked arithmetically.
// This lane's slice of a [n] parameter vector (weight or bias) as fp32, or
// `fill` where absent. 128-bit loads when its dtype matches x (the common
// case), element loads otherwise; all issued before any use.
template <int DT, int LANES, int CH>
__device__ inline void load_param(const void* p, int p_dt, int p_vec, int nch, int l, float fill,
                                  float (&v)[CH][Elt<DT>::VEC]) {
  using L = Elt<DT>;
  constexpr int VEC = L::VEC;
  if (!p) {
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
      for (int i = 0; i < VEC; ++i) v[c][i] = fill;
    return;
  }
  if (p_dt == DT && p_vec) {
#pragma unroll
    for (int c = 0; c < CH; ++c) L::load(p, (int64_t)min(c * LANES + l, nch - 1) * VEC, v[c]);
  } else {
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
      for (int i = 0; i < VEC; ++i)
        v[c][i] = ld_any(p, p_dt, (int64_t)min(c * LANES + l, nch - 1) * VEC + i);
  }
}

template <int DT, int LANES, int CH, bool RES>
__device__ inline void norm_load_row(const NormArgs& a, int64_t row, int l, int nch,
                                     float (&x)[CH][Elt<DT>::VEC]) {
  using L = Elt<DT>;
  constexpr int VEC = L::VEC;
  const int64_t rr = row < a.rows ? row : a.rows - 1;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int ch = min(c * LANES + l, nch - 1);
    L::load(a.x, rr * a.x_rs + (int64_t)ch * VEC, x[c]);
  }
  if (RES) {
    float r[CH][VEC];
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int ch = min(c * LANES + l, nch - 1);
      L::load(a.res, rr * a.res_rs + (int64_t)ch * VEC, r[c]);
    }
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
      for (int i = 0; i < VEC; ++i) x[c][i] += r[c][i];
  }
}

template <int DT, int LANES, int CH, bool RMS, bool RES, bool RES_OUT>
__device__ inline void norm_rows(const NormArgs& a, const float (&w)[CH][Elt<DT>::VEC],
                                 const float (&bb)[CH][Elt<DT>::VEC]) {
  using L = Elt<DT>;
  constexpr int VEC = L::VEC;
  constexpr int RPW = 64 / LANES;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int sub = lane / LANES;
  const int l = lane % LANES;
  const int nch = a.n / VEC;
  const float inv_n = 1.0f / (float)a.n;
  const int64_t step = (int64_t)gridDim.x * 4 * RPW;
  int64_t row0 = ((int64_t)blockIdx.x * 4 + wave) * RPW;  // wave-uniform
  if (row0 >= a.rows) return;
  float x[CH][VEC];
  norm_load_row<DT, LANES, CH, RES>(a, row0 + sub, l, nch, x);
  for (; row0 < a.rows; row0 += step) {
    const int64_t row = row0 + sub;
    // the next row's loads are in flight while this row is reduced
    float xn[CH][VEC];
    const bool more = row0 + step < a.rows;
    if (more) norm_load_row<DT, LANES, CH, RES>(a, row + step, l, nch, xn);
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const float keep = (c * LANES + l < nch) ? 1.f : 0.f;  // duplicate chunk: no weight
      float t = 0.f;
#pragma unroll
      for (int i = 0; i < VEC; ++i) t += RMS ? x[c][i] * x[c][i] : x[c][i];
      s += keep * t;
    }
    s = group_sum<LANES>(s);
    float mean = 0.f, rstd;
    if (RMS) {
      rstd = 1.0f / sqrtf(s * inv_n + a.eps);
    } else {
      mean = s * inv_n;
      float v = 0.f;
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const float keep = (c * LANES + l < nch) ? 1.f : 0.f;
        float t = 0.f;
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          const float d = x[c][i] - mean;
          t += d * d;
        }
        v += keep * t;
      }
      v = group_sum<LANES>(v);
      rstd = 1.0f / sqrtf(v * inv_n + a.eps);
    }
    if (row < a.rows) {
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const int ch = c * LANES + l;
        if (ch < nch) {
          if (RES_OUT) L::store(a.res_out, row * a.res_out_rs + (int64_t)ch * VEC, x[c]);
          float y[VEC];
#pragma unroll
          for (int i = 0; i < VEC; ++i) y[i] = (x[c][i] - mean) * rstd * w[c][i] + bb[c][i];
          L::store(a.y, row * a.y_rs + (int64_t)ch * VEC, y);
        }
      }
    }
    if (more) {
#pragma unroll
      for (int c = 0; c < CH; ++c)
#pragma unroll
        for (int i = 0; i < VEC; ++i) x[c][i] = xn[c][i];
    }
  }
}

template <int DT, int LANES, int CH, bool RMS>
__global__ __launch_bounds__(256) void norm_vec_kernel(NormArgs a) {
  constexpr int VEC = Elt<DT>::VEC;
  const int l = (threadIdx.x & 63) % LANES;
  const int nch = a.n / VEC;
  float w[CH][VEC], bb[CH][VEC];
  load_param<DT, LANES, CH>(a.w, a.w_dt, a.w_vec, nch, l, 1.f, w);
  load_param<DT, LANES, CH>(RMS ? nullptr : a.b, a.b_dt, a.b_vec, nch, l, 0.f, bb);
  if (!a.res)
    norm_rows<DT, LANES, CH, RMS, false, false>(a, w, bb);
  else if (!a.res_out)
    norm_rows<DT, LANES, CH, RMS, true, false>(a, w, bb);
  else
    norm_rows<DT, LANES, CH, RMS, true, true>(a, w, bb);
}

// Any width / alignment: one 256-thread block per row, LDS reduction.
template <int DT, bool RMS>
__global__ __launch_bounds__(256) void norm_scalar_kernel(NormArgs a) {
  using L = Elt<DT>;
  const int64_t row = blockIdx.x;
  __shared__ float red[8];
  float s = 0.f;
  for (int c = threadIdx.x; c < a.n; c += 256) {
    float v = L::ld1(a.x, row * a.x_rs + c);
    if (a.res) v += L::ld1(a.res, row * a.res_rs + c);
    s += RMS ? v * v : v;
  }
  s = group_sum<64>(s);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  s = red[0] + red[1] + red[2] + red[3];
  __syncthreads();
  const float inv_n = 1.0f / (float)a.n;
  float mean = 0.f, rstd;
  if (RMS) {
    rstd = 1.0f / sqrtf(s * inv_n + a.eps);
  } else {
    mean = s * inv_n;
    float v2 = 0.f;
    for (int c = threadIdx.x; c < a.n; c += 256) {
      float v = L::ld1(a.x, row * a.x_rs + c);
      if (a.res) v += L::ld1(a.res, row * a.res_rs + c);
      v2 += (v - mean) * (v - mean);
    }
    v2 = group_sum<64>(v2);
    if ((threadIdx.x & 63) == 0) red[4 + (threadIdx.x >> 6)] = v2;
    __syncthreads();
    v2 = red[4] + red[5] + red[6] + red[7];
    rstd = 1.0f / sqrtf(v2 * inv_n + a.eps);
  }
  for (int c = threadIdx.x; c < a.n; c += 256) {
    float v = L::ld1(a.x, row * a.x_rs + c);
    if (a.res) {
      v += L::ld1(a.res, row * a.res_rs + c);
      if (a.res_out) L::st1(a.res_out, row * a.res_out_rs + c, v);
    }
    float t = (v - mean) * rstd;
    if (a.w) t *= ld_any(a.w, a.w_dt, c);
    if (!RMS && a.b) t += ld_any(a.b, a.b_dt, c);
    L::st1(a.y, row * a.y_rs + c, t);
  }
}

template <int DT, int LANES, bool RMS>
static void launch_norm_vec(const NormArgs& a, int ch, hipStream_t st) {
  const int rows_per_block = 4 * (64 / LANES);
  // at most 2048 blocks (8 per CU), each striding over the same number of
  // row groups so that no block is left with a partial last round
  const int64_t groups = ceil_div(a.rows, rows_per_block);
  const int64_t per = ceil_div(groups, 2048);
  dim3 grid((unsigned)ceil_div(groups, per));
#define VFK_NORM_CASE(C)                                                   \
  case C:                                                                  \
    hipLaunchKernelGGL((norm_vec_kernel<DT, LANES, C, RMS>), grid, dim3(256), \
                       0, st, a);                                          \
    break;
  switch (ch) {
    VFK_NORM_CASE(1)
    VFK_NORM_CASE(2)
    VFK_NORM_CASE(3)
    VFK_NORM_CASE(4)
    VFK_NORM_CASE(6)
    VFK_NORM_CASE(8)
    VFK_NORM_CASE(12)
    VFK_NORM_CASE(16)
  }
#undef VFK_NORM_CASE
}

static int pick_ch(int need) {
  static const int opts[] = {1, 2, 3, 4, 6, 8, 12, 16};
  for (int o : opts)
    if (o >= need) return o;
  return 0;
}

template <int DT, bool RMS>
static void dispatch_norm(const NormArgs& a, bool vec_ok, hipStream_t st) {
  constexpr int VEC = Elt<DT>::VEC;
  const int nch = a.n / VEC;
  if (vec_ok) {
    const int lanes = (nch % 64 == 0 || nch > 96) ? 64 : 32;
    const int ch = pick_ch((nch + lanes - 1) / lanes);
    if (ch) {
      if (lanes == 64)
        launch_norm_vec<DT, 64, RMS>(a, ch, st);
      else
        launch_norm_vec<DT, 32, RMS>(a, ch, st);
      return;
    }
  }
  hipLaunchKernelGGL((norm_scalar_kernel<DT, RMS>), dim3((unsigned)a.rows),
                     dim3(256), 0, st, a);
}

static int norm_entry(const vfk_tensor* x, const vfk_tensor* residual,
                      const vfk_tensor* weight, const vfk_tensor* bias,
                      float eps, vfk_tensor* out, vfk_tensor* residual_out,
                      void* stream, bool rms, const char* name) {
  int rc;
  if ((rc = check_tensor(x, "x", 2)) || (rc = check_tensor(out, "out", 2)))
    return rc;
  const int64_t rows = x->size[0], n = x->size[1];
  if (n <= 0 || rows < 0 || n > (1 << 30))
    return set_error(VFK_ERR_INVALID, "%s: bad shape [%lld, %lld]", name,
                     (long long)rows, (long long)n);
  if (out->size[0] != rows || out->size[1] != n || out->dtype != x->dtype)
    return set_error(VFK_ERR_INVALID, "%s: out must match x", name);
  if (x->stride[1] != 1 || out->stride[1] != 1)
    return set_error(VFK_ERR_INVALID, "%s: last dim must be contiguous", name);
  NormArgs a = {};
  a.x = x->data; a.x_rs = x->stride[0];
  a.y = out->data; a.y_rs = out->stride[0];
  a.rows = rows; a.n = (int)n; a.eps = eps;
  bool vec_ok = aligned16(x->data) && aligned16(out->data);
  const int es = elem_size(x->dtype);
  const int VEC = 16 / es;
  if (n % VEC || a.x_rs % VEC || a.y_rs % VEC) vec_ok = false;
  if (present(residual)) {
    if ((rc = check_tensor(residual, "residual", 2))) return rc;
    if (residual->size[0] != rows || residual->size[1] != n ||
        residual->dtype != x->dtype || residual->stride[1] != 1)
      return set_error(VFK_ERR_INVALID, "%s: residual must match x", name);
    a.res = residual->data; a.res_rs = residual->stride[0];
    if (!aligned16(a.res) || a.res_rs % VEC) vec_ok = false;
    if (present(residual_out)) {
      if ((rc = check_tensor(residual_out, "residual_out", 2))) return rc;
      if (residual_out->size[0] != rows || residual_out->size[1] != n ||
          residual_out->dtype != x->dtype || residual_out->stride[1] != 1)
        return set_error(VFK_ERR_INVALID, "%s: residual_out must match x", name);
      a.res_out = residual_out->data; a.res_out_rs = residual_out->stride[0];
      if (!aligned16(a.res_out) || a.res_out_rs % VEC) vec_ok = false;
    }
  } else if (present(residual_out)) {
    return set_error(VFK_ERR_INVALID, "%s: residual_out needs residual", name);
  }
  if (present(weight)) {
    if ((rc = check_tensor(weight, "weight", 1))) return rc;
    if (weight->size[0] != n || weight->stride[0] != 1)
      return set_error(VFK_ERR_INVALID, "%s: weight must be contiguous [n]", name);
    a.w = weight->data; a.w_dt = weight->dtype; a.w_vec = aligned16(a.w);
  }
  if (present(bias)) {
    if ((rc = check_tensor(bias, "bias", 1))) return rc;
    if (bias->size[0] != n || bias->stride[0] != 1)
      return set_error(VFK_ERR_INVALID, "%s: bias must be contiguous [n]", name);
    a.b = bias->data; a.b_dt = bias->dtype; a.b_vec = aligned16(a.b);
  }
  if (rows == 0) return VFK_OK;
  hipStream_t st = (hipStream_t)stream;
  switch (x->dtype) {
    case VFK_F32:
      rms ? dispatch_norm<VFK_F32, true>(a, vec_ok, st)
          : dispatch_norm<VFK_F32, false>(a, vec_ok, st);
      break;
    case VFK_BF16:
      rms ? dispatch_norm<VFK_BF16, true>(a, vec_ok, st)
          : dispatch_norm<VFK_BF16, false>(a, vec_ok, st);
      break;
    case VFK_F16:
      rms ? dispatch_norm<VFK_F16, true>(a, vec_ok, st)
          : dispatch_norm<VFK_F16, false>(a, vec_ok, st);
      break;
  }
  return launch_status(name);
}

// ---------------------------------------------------------------------------
// Gated activations and residual add over [rows, n] with row strides.
// ---------------------------------------------------------------------------
struct BinArgs {
  const void* a; int64_t a_rs;
  const void* b; int64_t b_rs;
  void* y; int64_t y_rs;
  int64_t rows; int64_t n;
};

#define VFK_OP_ADD 100
#define VFK_OP_UNARY 200  // VFK_OP_UNARY + act: act(a), b unused

template <int OP>
__device__ inline float apply_op(float a, float b) {
  if (OP >= VFK_OP_UNARY) return act_f<OP - VFK_OP_UNARY>(a);
  if (OP == VFK_OP_ADD) return a + b;
  return act_f<OP>(a) * b;
}

// 128-bit chunks. FLAT: every operand is one dense [rows * n] run, so chunk c
// sits at element c * VEC of each. Otherwise chunk c is (row c / cpr, column
// chunk c % cpr), with the quotient from a multiply-high by a host-computed
// magic number (exact for c < 2^32: q = (umulhi(c, m) + c) >> l with
// l = ceil(log2 cpr), m = 2^32 (2^l - cpr) / cpr + 1).
// Each thread takes kBinU chunks per pass (blockDim apart, so a wave's
// accesses stay contiguous) and issues all their loads before any use.
constexpr int kBinU = 8;
template <int DT, int OP, bool FLAT>
__global__ __launch_bounds__(256) void binary_vec_kernel(BinArgs p, uint32_t cpr, uint32_t magic,
                                                         int shift, uint32_t total) {
  using L = Elt<DT>;
  constexpr int VEC = L::VEC;
  const uint32_t stride = gridDim.x * 256 * kBinU;
  for (uint32_t c0 = blockIdx.x * 256 * kBinU + threadIdx.x; c0 < total; c0 += stride) {
    int64_t ao[kBinU], bo[kBinU], yo[kBinU];
    bool ok[kBinU];
#pragma unroll
    for (int u = 0; u < kBinU; ++u) {
      const uint32_t c = c0 + u * 256;
      ok[u] = c < total;
      const uint32_t cc = ok[u] ? c : c0;  // in-bounds address for masked chunks
      if (FLAT) {
        ao[u] = bo[u] = yo[u] = (int64_t)cc * VEC;
      } else {
        const uint32_t r = (uint32_t)(((uint64_t)__umulhi(cc, magic) + cc) >> shift);
        const int64_t col = (int64_t)(cc - r * cpr) * VEC;
        ao[u] = (int64_t)r * p.a_rs + col;
        bo[u] = (int64_t)r * p.b_rs + col;
        yo[u] = (int64_t)r * p.y_rs + col;
      }
    }
    float x[kBinU][VEC], y[kBinU][VEC];
#pragma unroll
    for (int u = 0; u < kBinU; ++u) {
      L::load_nt(p.a, ao[u], x[u]);
      if (OP < VFK_OP_UNARY) L::load_nt(p.b, bo[u], y[u]);
    }
#pragma unroll
    for (int u = 0; u < kBinU; ++u) {
#pragma unroll
      for (int i = 0; i < VEC; ++i) x[u][i] = apply_op<OP>(x[u][i], y[u][i]);
      if (ok[u]) L::store(p.y, yo[u], x[u]);
    }
  }
}

template <int DT, int OP>
__global__ __launch_bounds__(256) void binary_scalar_kernel(BinArgs p) {
  using L = Elt<DT>;
  const int64_t total = p.rows * p.n;
  for (int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x; c < total;
       c += (int64_t)gridDim.x * 256) {
    const int64_t r = c / p.n;
    const int64_t col = c - r * p.n;
    const float bv = OP < VFK_OP_UNARY ? L::ld1(p.b, r * p.b_rs + col) : 0.f;
    L::st1(p.y, r * p.y_rs + col, apply_op<OP>(L::ld1(p.a, r * p.a_rs + col), bv));
  }
}

template <int DT, int OP>
static void launch_binary(const BinArgs& p, bool vec_ok, hipStream_t st) {
  constexpr int VEC = Elt<DT>::VEC;
  const int64_t work = vec_ok ? p.rows * (p.n / VEC) : p.rows * p.n;
  // enough blocks to fill 256 CUs several times; the loop covers the rest
  int64_t blocks = (work + 255) / 256;
  if (blocks > 256 * 16) blocks = 256 * 16;
  if (blocks < 1) blocks = 1;
  if (vec_ok && work < (1ll << 31)) {
    blocks = std::min<int64_t>(blocks, (work + 256 * kBinU - 1) / (256 * kBinU));
    const uint32_t cpr = (uint32_t)(p.n / VEC);
    const bool flat = p.rows == 1 || (p.a_rs == p.n && p.y_rs == p.n &&
                                      (OP >= VFK_OP_UNARY || p.b_rs == p.n));
    if (flat) {
      hipLaunchKernelGGL((binary_vec_kernel<DT, OP, true>), dim3((unsigned)blocks), dim3(256), 0, st,
                         p, cpr, 0u, 0, (uint32_t)work);
    } else {
      int l = 0;
      while ((1ull << l) < cpr) ++l;
      const uint32_t m = (uint32_t)((((1ull << 32) * ((1ull << l) - cpr)) / cpr) + 1);
      hipLaunchKernelGGL((binary_vec_kernel<DT, OP, false>), dim3((unsigned)blocks), dim3(256), 0, st,
                         p, cpr, m, l, (uint32_t)work);
    }
  } else {
    hipLaunchKernelGGL((binary_scalar_kernel<DT, OP>), dim3((unsigned)blocks), dim3(256), 0, st, p);
  }
}

template <int OP>
static void dispatch_binary(int dt, const BinArgs& p, bool vec_ok, hipStream_t st) {
  switch (dt) {
    case VFK_F32: launch_binary<VFK_F32, OP>(p, vec_ok, st); break;
    case VFK_BF16: launch_binary<VFK_BF16, OP>(p, vec_ok, st); break;
    case VFK_F16: launch_binary<VFK_F16, OP>(p, vec_ok, st); break;
  }
}

static int binary_entry(int op, const vfk_tensor* a, const vfk_tensor* b,
                        vfk_tensor* out, void* stream, const char* name) {
  int rc;
  if ((rc = check_tensor(a, "a", 2)) || (rc = check_tensor(b, "b", 2)) ||
      (rc = check_tensor(out, "out", 2)))
    return rc;
  const int64_t rows = a->size[0], n = a->size[1];
  if (b->size[0] != rows || b->size[1] != n || out->size[0] != rows ||
      out->size[1] != n)
    return set_error(VFK_ERR_INVALID, "%s: shape mismatch", name);
  if (b->dtype != a->dtype || out->dtype != a->dtype)
    return set_error(VFK_ERR_INVALID, "%s: dtype mismatch", name);
  if (a->stride[1] != 1 || b->stride[1] != 1 || out->stride[1] != 1)
    return set_error(VFK_ERR_INVALID, "%s: last dim must be contiguous", name);
  if (rows == 0 || n == 0) return VFK_OK;
  BinArgs p = {a->data, a->stride[0], b->data, b->stride[0],
               out->data, out->stride[0], rows, n};
  const int VEC = 16 / elem_size(a->dtype);
  const bool vec_ok = aligned16(a->data) && aligned16(b->data) &&
                      aligned16(out->data) && n % VEC == 0 &&
                      p.a_rs % VEC == 0 && p.b_rs % VEC == 0 &&
                      p.y_rs % VEC == 0;
  hipStream_t st = (hipStream_t)stream;
  switch (op) {
    case VFK_ACT_GELU_ERF: dispatch_binary<VFK_ACT_GELU_ERF>(a->dtype, p, vec_ok, st); break;
    case VFK_ACT_GELU_TANH: dispatch_binary<VFK_ACT_GELU_TANH>(a->dtype, p, vec_ok, st); break;
    case VFK_ACT_SILU: dispatch_binary<VFK_ACT_SILU>(a->dtype, p, vec_ok, st); break;
    case VFK_ACT_RELU: dispatch_binary<VFK_ACT_RELU>(a->dtype, p, vec_ok, st); break;
    case VFK_OP_ADD: dispatch_binary<VFK_OP_ADD>(a->dtype, p, vec_ok, st); break;
    case VFK_OP_UNARY + VFK_ACT_GELU_ERF:
      dispatch_binary<VFK_OP_UNARY + VFK_ACT_GELU_ERF>(a->dtype, p, vec_ok, st); break;
    case VFK_OP_UNARY + VFK_ACT_GELU_TANH:
      dispatch_binary<VFK_OP_UNARY + VFK_ACT_GELU_TANH>(a->dtype, p, vec_ok, st); break;
    case VFK_OP_UNARY + VFK_ACT_SILU:
      dispatch_binary<VFK_OP_UNARY + VFK_ACT_SILU>(a->dtype, p, vec_ok, st); break;
    case VFK_OP_UNARY + VFK_ACT_RELU:
      dispatch_binary<VFK_OP_UNARY + VFK_ACT_RELU>(a->dtype, p, vec_ok, st); break;
    default: return set_error(VFK_ERR_INVALID, "%s: unknown activation %d", name, op);
  }
  return launch_status(name);
}

// ---------------------------------------------------------------------------
// RoPE with explicit cos/sin tables, x [B,S,H,D], cos/sin [B,S,D].
// ---------------------------------------------------------------------------
struct RopeArgs {
  const void* x; int64_t xs[4];
  const void* c; int64_t cs[3];
  const void* s; int64_t ss[3];
  void* y; int64_t ys[4];
  int64_t B, S, H; int D;
};

// Thread item t = ((b * S + s) * H + h) * cpr + c (chunk pair c of head h of
// row (b, s)), consecutive items covering consecutive 16-byte chunks of the
// row; kRopeU items per thread and pass, all loads issued before any use.
constexpr int kRopeU = 4;
template <int DT>
__global__ __launch_bounds__(256) void rope_item_kernel(RopeArgs p, Magic gc, Magic gh, Magic gs,
                                                        uint32_t total) {
  using L = Elt<DT>;
  constexpr int VEC = L::VEC;
  const int half = p.D / 2;
  const uint32_t stride = gridDim.x * 256 * kRopeU;
  for (uint32_t t0 = blockIdx.x * 256 * kRopeU + threadIdx.x; t0 < total; t0 += stride) {
    int64_t xo[kRopeU], yo[kRopeU], co[kRopeU], so[kRopeU];
    bool ok[kRopeU];
#pragma unroll
    for (int u = 0; u < kRopeU; ++u) {
      const uint32_t t = t0 + u * 256;
      ok[u] = t < total;
      const uint32_t tt = ok[u] ? t : t0;
      const uint32_t rh = magic_div(tt, gc);
      const int d0 = (int)(tt - rh * gc.d) * VEC;
      const uint32_t r = magic_div(rh, gh);
      const uint32_t h = rh - r * gh.d;
      const uint32_t b = magic_div(r, gs);
      const uint32_t sq = r - b * gs.d;
      xo[u] = (int64_t)b * p.xs[0] + (int64_t)sq * p.xs[1] + (int64_t)h * p.xs[2] + d0;
      yo[u] = (int64_t)b * p.ys[0] + (int64_t)sq * p.ys[1] + (int64_t)h * p.ys[2] + d0;
      co[u] = (int64_t)b * p.cs[0] + (int64_t)sq * p.cs[1] + d0;
      so[u] = (int64_t)b * p.ss[0] + (int64_t)sq * p.ss[1] + d0;
    }
    float x1[kRopeU][VEC], x2[kRopeU][VEC], c1[kRopeU][VEC], c2[kRopeU][VEC], s1[kRopeU][VEC],
        s2[kRopeU][VEC];
#pragma unroll
    for (int u = 0; u < kRopeU; ++u) {
      L::load(p.x, xo[u], x1[u]);
      L::load(p.x, xo[u] + half, x2[u]);
      L::load(p.c, co[u], c1[u]);
      L::load(p.c, co[u] + half, c2[u]);
      L::load(p.s, so[u], s1[u]);
      L::load(p.s, so[u] + half, s2[u]);
    }
#pragma unroll
    for (int u = 0; u < kRopeU; ++u) {
      float y1[VEC], y2[VEC];
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        y1[i] = x1[u][i] * c1[u][i] - x2[u][i] * s1[u][i];
        y2[i] = x2[u][i] * c2[u][i] + x1[u][i] * s2[u][i];
      }
      if (ok[u]) {
        L::store(p.y, yo[u], y1);
        L::store(p.y, yo[u] + half, y2);
      }
    }
  }
}

template <int DT>
__global__ __launch_bounds__(256) void rope_vec_kernel(RopeArgs p) {
  using L = Elt<DT>;
  constexpr int VEC = L::VEC;
  const int half = p.D / 2;
  const int cpr = half / VEC;  // chunk pairs per row
  const int64_t total = p.B * p.S * p.H * cpr;
  for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * 256) {
    int64_t r = t / cpr;
    const int d0 = (int)(t - r * cpr) * VEC;
    const int64_t h = r % p.H; r /= p.H;
    const int64_t s = r % p.S;
    const int64_t b = r / p.S;
    const int64_t xo = b * p.xs[0] + s * p.xs[1] + h * p.xs[2];
    const int64_t yo = b * p.ys[0] + s * p.ys[1] + h * p.ys[2];
    const int64_t co = b * p.cs[0] + s * p.cs[1];
    const int64_t so = b * p.ss[0] + s * p.ss[1];
    float x1[VEC], x2[VEC], c1[VEC], c2[VEC], s1[VEC], s2[VEC];
    L::load(p.x, xo + d0, x1);
    L::load(p.x, xo + d0 + half, x2);
    L::load(p.c, co + d0, c1);
    L::load(p.c, co + d0 + half, c2);
    L::load(p.s, so + d0, s1);
    L::load(p.s, so + d0 + half, s2);
    float y1[VEC], y2[VEC];
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      y1[i] = x1[i] * c1[i] - x2[i] * s1[i];
      y2[i] = x2[i] * c2[i] + x1[i] * s2[i];
    }
    L::store(p.y, yo + d0, y1);
    L::store(p.y, yo + d0 + half, y2);
  }
}

// Any strides and any even D; cos / sin in the element type or fp32 (CT).
template <int DT, int CT>
__global__ __launch_bounds__(256) void rope_scalar_kernel(RopeArgs p) {
  using L = Elt<DT>;
  using LC = Elt<CT>;
  const int half = p.D / 2;
  const int64_t total = p.B * p.S * p.H * p.D;
  for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * 256) {
    int64_t r = t / p.D;
    const int d = (int)(t - r * p.D);
    const int64_t h = r % p.H; r /= p.H;
    const int64_t s = r % p.S;
    const int64_t b = r / p.S;
    const int64_t xo = b * p.xs[0] + s * p.xs[1] + h * p.xs[2];
    const float x = L::ld1(p.x, xo + d * p.xs[3]);
    const int pd = d < half ? d + half : d - half;
    const float xp = L::ld1(p.x, xo + pd * p.xs[3]);
    const float c = LC::ld1(p.c, b * p.cs[0] + s * p.cs[1] + d * p.cs[2]);
    const float sn = LC::ld1(p.s, b * p.ss[0] + s * p.ss[1] + d * p.ss[2]);
    float y;
    {
      // products rounded separately, as in the unfused fp32 formula
#pragma clang fp contract(off)
      y = d < half ? x * c - xp * sn : x * c + xp * sn;
    }
    L::st1(p.y, b * p.ys[0] + s * p.ys[1] + h * p.ys[2] + d * p.ys[3], y);
  }
}

// ---------------------------------------------------------------------------
// RoPE of q and k in one launch (kernels/fused_rope_global.py:108-166 makes
// one launch per tensor). Thread = (row (b, s), chunk pair cp): it loads the
// cos / sin values of d in chunk cp and of d + D/2 once, in the table's own
// dtype (fp32 or the element type), and applies them to kRopeHG heads of the
// concatenated head list (q heads, then k heads), all loads of those heads in
// flight before the first use. Grid y = head groups.
// ---------------------------------------------------------------------------
struct RopeQKArgs {
  const void* x[2]; int64_t xs[2][3];  // q, k: strides of B, S, H (D contiguous)
  void* y[2]; int64_t ys[2][3];
  int nh[2];                           // heads of q, k (k: 0 when absent)
  const void* c; int64_t cs[2];        // cos: strides of B (0: shared), S
  const void* s; int64_t ss[2];
  int half;                            // D / 2
  uint32_t rows;                       // B * S
};

constexpr int kRopeHG = 6;

// VEC table values at element i as fp32 (VEC = the x chunk's element count).
template <int CT, int VEC>
__device__ inline void load_tab(const void* base, int64_t i, float* f) {
  if constexpr (CT == VFK_F32) {
#pragma unroll
    for (int j = 0; j < VEC / 4; ++j) Elt<VFK_F32>::load(base, i + 4 * j, f + 4 * j);
  } else {
    static_assert(VEC == Elt<CT>::VEC, "16-bit table with a 16-bit element type");
    Elt<CT>::load(base, i, f);
  }
}

template <int DT, int CT>
__global__ __launch_bounds__(256) void rope_qk_kernel(RopeQKArgs p, Magic gcp, Magic gs) {
  using L = Elt<DT>;
  constexpr int VEC = L::VEC;
  const uint32_t t = blockIdx.x * 256u + threadIdx.x;
  const uint32_t row = magic_div(t, gcp);
  if (row >= p.rows) return;
  const int d0 = (int)(t - row * gcp.d) * VEC;
  const uint32_t b = magic_div(row, gs);
  const uint32_t sq = row - b * gs.d;
  float c1[VEC], c2[VEC], s1[VEC], s2[VEC];
  const int64_t co = (int64_t)b * p.cs[0] + (int64_t)sq * p.cs[1] + d0;
  const int64_t so = (int64_t)b * p.ss[0] + (int64_t)sq * p.ss[1] + d0;
  load_tab<CT, VEC>(p.c, co, c1);
  load_tab<CT, VEC>(p.c, co + p.half, c2);
  load_tab<CT, VEC>(p.s, so, s1);
  load_tab<CT, VEC>(p.s, so + p.half, s2);
  const int nh = p.nh[0] + p.nh[1];
  const int h0 = blockIdx.y * kRopeHG;
  float x1[kRopeHG][VEC], x2[kRopeHG][VEC];
  int64_t yo[kRopeHG];
#pragma unroll
  for (int u = 0; u < kRopeHG; ++u) {
    // head index uniform over the grid row: the tensor choice is scalar
    const int hh = min(h0 + u, nh - 1);
    const int ti = hh >= p.nh[0] ? 1 : 0;
    const int h = hh - ti * p.nh[0];
    const int64_t xo = (int64_t)b * p.xs[ti][0] + (int64_t)sq * p.xs[ti][1] + (int64_t)h * p.xs[ti][2] + d0;
    yo[u] = (int64_t)b * p.ys[ti][0] + (int64_t)sq * p.ys[ti][1] + (int64_t)h * p.ys[ti][2] + d0;
    L::load(p.x[ti], xo, x1[u]);
    L::load(p.x[ti], xo + p.half, x2[u]);
  }
#pragma unroll
  for (int u = 0; u < kRopeHG; ++u) {
    if (h0 + u >= nh) break;
    const int ti = h0 + u >= p.nh[0] ? 1 : 0;
    float y1[VEC], y2[VEC];
    {
      // products rounded separately, as in the unfused fp32 formula
#pragma clang fp contract(off)
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        y1[i] = x1[u][i] * c1[i] - x2[u][i] * s1[i];
        y2[i] = x2[u][i] * c2[i] + x1[u][i] * s2[i];
      }
    }
    L::store(p.y[ti], yo[u], y1);
    L::store(p.y[ti], yo[u] + p.half, y2);
  }
}

// Unit layout of the same operation for D = CPU * VEC: a unit is one (row,
// head) vector of D contiguous elements and CPU consecutive lanes own its
// chunks, so a wave's load and store instructions cover whole units (for
// D = 64 and 16-bit types: 2 rows x 4 adjacent heads, two 512-byte runs).
// Lane j owns chunk j and also loads the chunk j +- CPU/2 that pairs with it
// in the rotation (the wave's own first load has just brought that line into
// the vector cache). A thread takes the heads hs, hs + kRopeSlots, ... of one
// row, in q and then in k (the tensor is uniform over the wave, so its
// strides stay scalar), and loads its cos/sin chunks once. Products are
// rounded separately before the add (x cos, then the partner times sin), as
// in the unfused fp32 formula.
constexpr int kRopeSlots = 4;  // head slots per row
constexpr int kRopeUnits = 3;  // heads per slot and tensor loaded together
template <int DT, int CT, int CPU>
__global__ __launch_bounds__(256) void rope_unit_kernel(RopeQKArgs p, Magic gs) {
  using L = Elt<DT>;
  constexpr int VEC = L::VEC;
  constexpr int RB = 256 / (CPU * kRopeSlots);  // rows per block
  static_assert(RB >= 1 && CPU % 2 == 0, "unit layout");
  const int t = threadIdx.x;
  const int j = t % CPU;
  const int hs = (t / CPU) % kRopeSlots;
  const uint32_t row = blockIdx.x * (uint32_t)RB + (uint32_t)(t / (CPU * kRopeSlots));
  if (row >= p.rows) return;
  const uint32_t b = magic_div(row, gs);
  const uint32_t sq = row - b * gs.d;
  const bool lo = j < CPU / 2;
  const int d0 = j * VEC;
  const int dp = lo ? d0 + p.half : d0 - p.half;
  float c[VEC], s[VEC];
  load_tab<CT, VEC>(p.c, (int64_t)b * p.cs[0] + (int64_t)sq * p.cs[1] + d0, c);
  load_tab<CT, VEC>(p.s, (int64_t)b * p.ss[0] + (int64_t)sq * p.ss[1] + d0, s);
  // first half: x cos - partner sin = x cos + partner (-sin), exactly
  if (lo) {
#pragma unroll
    for (int i = 0; i < VEC; ++i) s[i] = -s[i];
  }
  using U16 = typename std::conditional<DT == VFK_F32, float, uint16_t>::type;
#pragma unroll
  for (int ti = 0; ti < 2; ++ti) {
    const int nh = p.nh[ti];
    // row bases in 64 bits, head offsets in 32 (heads * head stride < 2^31)
    const U16* xb = reinterpret_cast<const U16*>(p.x[ti]) + (int64_t)b * p.xs[ti][0] + (int64_t)sq * p.xs[ti][1];
    U16* yb = reinterpret_cast<U16*>(p.y[ti]) + (int64_t)b * p.ys[ti][0] + (int64_t)sq * p.ys[ti][1];
    const int xh = (int)p.xs[ti][2], yh = (int)p.ys[ti][2];
    for (int hb = hs; hb < nh; hb += kRopeUnits * kRopeSlots) {
      float x[kRopeUnits][VEC], xq[kRopeUnits][VEC];
#pragma unroll
      for (int u = 0; u < kRopeUnits; ++u) {
        const int xo = min(hb + u * kRopeSlots, nh - 1) * xh;
        L::load(xb, xo + d0, x[u]);
        L::load(xb, xo + dp, xq[u]);
      }
#pragma unroll
      for (int u = 0; u < kRopeUnits; ++u) {
        const int h = hb + u * kRopeSlots;
        if (h >= nh) break;
        float y[VEC];
        {
#pragma clang fp contract(off)
#pragma unroll
          for (int i = 0; i < VEC; ++i) y[i] = x[u][i] * c[i] + xq[u][i] * s[i];
        }
        L::store(yb, h * yh + d0, y);
      }
    }
  }
}

}  // namespace vfk

using namespace vfk;

extern "C" int vfk_layernorm_fwd(const vfk_tensor* x, const vfk_tensor* residual,
                                 const vfk_tensor* weight, const vfk_tensor* bias,
                                 float eps, vfk_tensor* out,
                                 vfk_tensor* residual_out, void* stream) {
  return norm_entry(x, residual, weight, bias, eps, out, residual_out, stream,
                    false, "vfk_layernorm_fwd");
}

extern "C" int vfk_rmsnorm_fwd(const vfk_tensor* x, const vfk_tensor* residual,
                               const vfk_tensor* weight, float eps,
                               vfk_tensor* out, vfk_tensor* residual_out,
                               void* stream) {
  return norm_entry(x, residual, weight, nullptr, eps, out, residual_out,
                    stream, true, "vfk_rmsnorm_fwd");
}

extern "C" int vfk_glu_fwd(int32_t act, const vfk_tensor* a,
                           const vfk_tensor* b, vfk_tensor* out, void* stream) {
  if (act < VFK_ACT_GELU_ERF || act > VFK_ACT_RELU)
    return set_error(VFK_ERR_INVALID, "vfk_glu_fwd: unknown activation %d", act);
  return binary_entry(act, a, b, out, stream, "vfk_glu_fwd");
}

extern "C" int vfk_act_fwd(int32_t act, const vfk_tensor* x, vfk_tensor* out, void* stream) {
  if (act < VFK_ACT_GELU_ERF || act > VFK_ACT_RELU)
    return set_error(VFK_ERR_INVALID, "vfk_act_fwd: unknown activation %d", act);
  // b is not read for unary ops; x stands in for its shape checks
  return binary_entry(VFK_OP_UNARY + act, x, x, out, stream, "vfk_act_fwd");
}

extern "C" int vfk_residual_add(const vfk_tensor* a, const vfk_tensor* b,
                                vfk_tensor* out, void* stream) {
  return binary_entry(VFK_OP_ADD, a, b, out, stream, "vfk_residual_add");
}

extern "C" int vfk_rope_fwd(const vfk_tensor* x, const vfk_tensor* cos,
                            const vfk_tensor* sin, vfk_tensor* out,
                            void* stream) {
  int rc;
  if ((rc = check_tensor(x, "x", 4)) || (rc = check_tensor(out, "out", 4)) ||
      (rc = check_tensor(cos, "cos", 3)) || (rc = check_tensor(sin, "sin", 3)))
    return rc;
  const int64_t B = x->size[0], S = x->size[1], H = x->size[2], D = x->size[3];
  for (int i = 0; i < 4; ++i)
    if (out->size[i] != x->size[i])
      return set_error(VFK_ERR_INVALID, "vfk_rope_fwd: out shape mismatch");
  if (D % 2 || D <= 0)
    return set_error(VFK_ERR_INVALID, "vfk_rope_fwd: head_dim must be even");
  const vfk_tensor* cs[2] = {cos, sin};
  for (const vfk_tensor* t : cs) {
    if ((t->size[0] != B && t->size[0] != 1) || t->size[1] != S || t->size[2] != D)
      return set_error(VFK_ERR_INVALID, "vfk_rope_fwd: cos/sin must be [B|1,S,D]");
    if (t->dtype != x->dtype && t->dtype != VFK_F32)
      return set_error(VFK_ERR_INVALID, "vfk_rope_fwd: cos/sin dtype must be x's or fp32");
  }
  if (cos->dtype != sin->dtype)
    return set_error(VFK_ERR_INVALID, "vfk_rope_fwd: cos and sin dtypes differ");
  const bool f32t = cos->dtype == VFK_F32 && x->dtype != VFK_F32;
  if (out->dtype != x->dtype)
    return set_error(VFK_ERR_INVALID, "vfk_rope_fwd: out dtype must match x");
  RopeArgs p = {};
  p.x = x->data; p.c = cos->data; p.s = sin->data; p.y = out->data;
  for (int i = 0; i < 4; ++i) { p.xs[i] = x->stride[i]; p.ys[i] = out->stride[i]; }
  for (int i = 0; i < 3; ++i) { p.cs[i] = cos->stride[i]; p.ss[i] = sin->stride[i]; }
  if (cos->size[0] == 1) p.cs[0] = 0;
  if (sin->size[0] == 1) p.ss[0] = 0;
  p.B = B; p.S = S; p.H = H; p.D = (int)D;
  const int64_t rows = B * S * H;
  if (rows == 0) return VFK_OK;
  const int VEC = 16 / elem_size(x->dtype);
  bool vec_ok = !f32t && (D / 2) % VEC == 0 && x->stride[3] == 1 && out->stride[3] == 1 &&
                cos->stride[2] == 1 && sin->stride[2] == 1 &&
                aligned16(x->data) && aligned16(out->data) &&
                aligned16(cos->data) && aligned16(sin->data);
  for (int i = 0; i < 3; ++i)
    vec_ok = vec_ok && p.xs[i] % VEC == 0 && p.ys[i] % VEC == 0;
  for (int i = 0; i < 2; ++i)
    vec_ok = vec_ok && p.cs[i] % VEC == 0 && p.ss[i] % VEC == 0;
  const int64_t work = vec_ok ? rows * (D / 2 / VEC) : rows * D;
  int64_t blocks = (work + 255) / 256;
  if (blocks > 256 * 16) blocks = 256 * 16;
  hipStream_t st = (hipStream_t)stream;
  const bool by_item = vec_ok && work < (1ll << 31);
  const Magic gc = magic_for((uint32_t)std::max<int64_t>(1, D / 2 / VEC));
  const Magic gh = magic_for((uint32_t)std::max<int64_t>(1, H));
  const Magic gs = magic_for((uint32_t)std::max<int64_t>(1, S));
  const unsigned item_blocks =
      (unsigned)std::min<int64_t>(blocks, (work + 256 * kRopeU - 1) / (256 * kRopeU));
#define VFK_ROPE(DT)                                                               \
  if (by_item)                                                                     \
    hipLaunchKernelGGL((rope_item_kernel<DT>), dim3(item_blocks), dim3(256), 0, st, p, gc, gh, \
                       gs, (uint32_t)work);                                        \
  else if (vec_ok)                                                                 \
    hipLaunchKernelGGL((rope_vec_kernel<DT>), dim3((unsigned)blocks), dim3(256), 0, st, p); \
  else if (f32t)                                                                   \
    hipLaunchKernelGGL((rope_scalar_kernel<DT, VFK_F32>), dim3((unsigned)blocks), dim3(256), 0, st, p); \
  else                                                                             \
    hipLaunchKernelGGL((rope_scalar_kernel<DT, DT>), dim3((unsigned)blocks), dim3(256), 0, st, p);
  switch (x->dtype) {
    case VFK_F32: VFK_ROPE(VFK_F32); break;
    case VFK_BF16: VFK_ROPE(VFK_BF16); break;
    case VFK_F16: VFK_ROPE(VFK_F16); break;
  }
#undef VFK_ROPE
  return launch_status("vfk_rope_fwd");
}

static int rope_x_ok(const vfk_tensor* t, const char* name, int dt) {
  int rc = check_tensor(t, name, 4);
  if (rc) return rc;
  if (t->dtype != dt) return set_error(VFK_ERR_INVALID, "vfk_rope_qk_fwd: %s dtype differs from q", name);
  const int vec = 16 / elem_size(dt);
  if (t->stride[3] != 1 || !aligned16(t->data) || t->stride[0] % vec || t->stride[1] % vec ||
      t->stride[2] % vec)
    return set_error(VFK_ERR_INVALID, "vfk_rope_qk_fwd: %s needs a contiguous last dim and "
                     "16-byte aligned rows", name);
  return VFK_OK;
}

extern "C" int vfk_rope_qk_fwd(const vfk_tensor* q, const vfk_tensor* k, const vfk_tensor* cos,
                               const vfk_tensor* sin, vfk_tensor* q_out, vfk_tensor* k_out,
                               void* stream) {
  int rc;
  if ((rc = check_tensor(q, "q", 4))) return rc;
  const int dt = q->dtype;
  const bool has_k = present(k);
  if (has_k != present(k_out))
    return set_error(VFK_ERR_INVALID, "vfk_rope_qk_fwd: k and k_out go together");
  if ((rc = rope_x_ok(q, "q", dt)) || (rc = rope_x_ok(q_out, "q_out", dt))) return rc;
  if (has_k && ((rc = rope_x_ok(k, "k", dt)) || (rc = rope_x_ok(k_out, "k_out", dt)))) return rc;
  const int64_t B = q->size[0], S = q->size[1], D = q->size[3];
  for (int i = 0; i < 4; ++i)
    if (q_out->size[i] != q->size[i] || (has_k && k_out->size[i] != k->size[i]))
      return set_error(VFK_ERR_INVALID, "vfk_rope_qk_fwd: out shape mismatch");
  if (has_k && (k->size[0] != B || k->size[1] != S || k->size[3] != D))
    return set_error(VFK_ERR_INVALID, "vfk_rope_qk_fwd: q and k must share B, S and D");
  const int vec = 16 / elem_size(dt);
  if (D <= 0 || D % (2 * vec))
    return set_error(VFK_ERR_UNSUPPORTED, "vfk_rope_qk_fwd: head_dim %lld is not a multiple of %d",
                     (long long)D, 2 * vec);
  const vfk_tensor* cs[2] = {cos, sin};
  for (int i = 0; i < 2; ++i) {
    const vfk_tensor* t = cs[i];
    if ((rc = check_tensor(t, i ? "sin" : "cos", 3))) return rc;
    if ((t->size[0] != B && t->size[0] != 1) || t->size[1] != S || t->size[2] != D)
      return set_error(VFK_ERR_INVALID, "vfk_rope_qk_fwd: cos/sin must be [B|1, S, D]");
    if (t->dtype != dt && t->dtype != VFK_F32)
      return set_error(VFK_ERR_INVALID, "vfk_rope_qk_fwd: cos/sin dtype must be q's or fp32");
    const int tv = 16 / elem_size(t->dtype);
    if (t->stride[2] != 1 || !aligned16(t->data) || t->stride[1] % tv ||
        (t->size[0] != 1 && t->stride[0] % tv))
      return set_error(VFK_ERR_INVALID, "vfk_rope_qk_fwd: cos/sin need 16-byte aligned rows");
  }
  if (cos->dtype != sin->dtype)
    return set_error(VFK_ERR_INVALID, "vfk_rope_qk_fwd: cos and sin dtypes differ");
  const int64_t rows = B * S;
  const int64_t cpr = D / 2 / vec;
  if (rows * cpr >= (1ll << 32) - 256)
    return set_error(VFK_ERR_UNSUPPORTED, "vfk_rope_qk_fwd: too many rows");
  const int nh = (int)q->size[2] + (has_k ? (int)k->size[2] : 0);
  if (rows == 0 || nh == 0) return VFK_OK;
  RopeQKArgs p = {};
  p.x[0] = q->data; p.y[0] = q_out->data; p.nh[0] = (int)q->size[2];
  p.x[1] = has_k ? k->data : q->data; p.y[1] = has_k ? k_out->data : q_out->data;
  p.nh[1] = has_k ? (int)k->size[2] : 0;
  for (int i = 0; i < 3; ++i) {
    p.xs[0][i] = q->stride[i]; p.ys[0][i] = q_out->stride[i];
    p.xs[1][i] = has_k ? k->stride[i] : 0; p.ys[1][i] = has_k ? k_out->stride[i] : 0;
  }
  p.c = cos->data; p.cs[0] = cos->size[0] == 1 ? 0 : cos->stride[0]; p.cs[1] = cos->stride[1];
  p.s = sin->data; p.ss[0] = sin->size[0] == 1 ? 0 : sin->stride[0]; p.ss[1] = sin->stride[1];
  p.half = (int)(D / 2);
  p.rows = (uint32_t)rows;
  const Magic gcp = magic_for((uint32_t)cpr);
  const Magic gs = magic_for((uint32_t)std::max<int64_t>(1, S));
  hipStream_t st = (hipStream_t)stream;
  const bool f32t = cos->dtype == VFK_F32;
  // unit layout when a D-vector is 8 or 16 chunks (D = 64 or 128 for 16-bit types)
  const int64_t cpu = 2 * cpr;
  bool unit_ok = dt != VFK_F32 && (cpu == 8 || cpu == 16);
  for (int i = 0; i < 2 && unit_ok; ++i) {
    const vfk_tensor* xt = i ? (has_k ? k : q) : q;
    const vfk_tensor* yt = i ? (has_k ? k_out : q_out) : q_out;
    unit_ok = xt->size[2] * (std::llabs(xt->stride[2]) + 1) + D < (1ll << 31) &&
              yt->size[2] * (std::llabs(yt->stride[2]) + 1) + D < (1ll << 31);
  }
  if (unit_ok) {
#define VFK_RU(DT, CT, C)                                                              \
  hipLaunchKernelGGL((rope_unit_kernel<DT, CT, C>),                                    \
                     dim3((unsigned)((rows + 256 / (C * kRopeSlots) - 1) / (256 / (C * kRopeSlots)))), \
                     dim3(256), 0, st, p, gs)
    if (dt == VFK_BF16) {
      if (cpu == 8) { if (f32t) VFK_RU(VFK_BF16, VFK_F32, 8); else VFK_RU(VFK_BF16, VFK_BF16, 8); }
      else { if (f32t) VFK_RU(VFK_BF16, VFK_F32, 16); else VFK_RU(VFK_BF16, VFK_BF16, 16); }
    } else {
      if (cpu == 8) { if (f32t) VFK_RU(VFK_F16, VFK_F32, 8); else VFK_RU(VFK_F16, VFK_F16, 8); }
      else { if (f32t) VFK_RU(VFK_F16, VFK_F32, 16); else VFK_RU(VFK_F16, VFK_F16, 16); }
    }
#undef VFK_RU
    return launch_status("vfk_rope_qk_fwd");
  }
  const dim3 grid((unsigned)((rows * cpr + 255) / 256), (unsigned)((nh + kRopeHG - 1) / kRopeHG));
#define VFK_RQK(DT, CT) hipLaunchKernelGGL((rope_qk_kernel<DT, CT>), grid, dim3(256), 0, st, p, gcp, gs)
  switch (dt) {
    case VFK_F32: VFK_RQK(VFK_F32, VFK_F32); break;
    case VFK_BF16: if (f32t) VFK_RQK(VFK_BF16, VFK_F32); else VFK_RQK(VFK_BF16, VFK_BF16); break;
    case VFK_F16: if (f32t) VFK_RQK(VFK_F16, VFK_F32); else VFK_RQK(VFK_F16, VFK_F16); break;
  }
#undef VFK_RQK
  return launch_status("vfk_rope_qk_fwd");
}
