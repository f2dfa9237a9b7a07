// Packed-sequence metadata from vLLM's flat position ids, on the device.
//
// Replaces the reference's dense-mask construction for packed ModernBERT
// batches (models/modernbert/modernbert_encoder.py:491-516,
// _build_seq_block_mask): a new sequence starts at token 0 and wherever the
// position does not increase (pos[i] <= pos[i-1]); the reference then turns
// the segment ids (cumsum of those starts) into [T, T] masks. Here the starts
// become cu_seqlens directly, in three passes over 1024-token blocks:
//   1. count the starts of each block,
//   2. one workgroup scans the block counts (exclusive) and writes the
//      totals,
//   3. each block writes the indices of its starts at its offset, checks that
//      positions count up from 0 inside every sequence (the positions the
//      varlen attention's RoPE uses are t - cu_seqlens[s]), and folds the
//      lengths of the sequences that start in it into the maximum.
// meta[0] = number of sequences, meta[1] = longest sequence, meta[2] = breaks
// in the run of positions (a start whose position is not 0, or a token whose
// position is not its predecessor's + 1; 0 exactly when every position equals
// index - sequence start), meta[3] = T.
#include <stdint.h>

#include <algorithm>

#include "launch_util.h"
#include "vfk_common.h"

namespace vfk {

constexpr int kMetaBlock = 1024;  // tokens per block (256 threads x 4)

template <typename P>
__device__ inline bool seq_start(const P* pos, int64_t i) {
  return i == 0 || pos[i] <= pos[i - 1];
}

template <typename P>
__global__ __launch_bounds__(256) void meta_count_kernel(const P* __restrict__ pos, int64_t T,
                                                         int32_t* __restrict__ counts) {
  __shared__ int red[4];
  const int64_t base = (int64_t)blockIdx.x * kMetaBlock;
  int c = 0;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int64_t i = base + u * 256 + threadIdx.x;
    if (i < T && seq_start(pos, i)) ++c;
  }
  for (int o = 32; o > 0; o >>= 1) c += __shfl_xor(c, o, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = c;
  __syncthreads();
  if (threadIdx.x == 0) counts[blockIdx.x] = red[0] + red[1] + red[2] + red[3];
}

// One workgroup: offsets[b] = counts[0] + ... + counts[b-1] (in place);
// meta[0] = total starts, meta[1] = meta[2] = 0, meta[3] = T; cu[total] = T.
__global__ __launch_bounds__(1024) void meta_scan_kernel(int32_t* __restrict__ counts, int nblk,
                                                         int64_t T, int32_t* __restrict__ cu,
                                                         int32_t* __restrict__ meta) {
  __shared__ int part[1024];
  __shared__ int carry;
  if (threadIdx.x == 0) carry = 0;
  __syncthreads();
  for (int b0 = 0; b0 < nblk; b0 += 1024) {
    const int b = b0 + threadIdx.x;
    const int v = b < nblk ? counts[b] : 0;
    part[threadIdx.x] = v;
    __syncthreads();
    for (int o = 1; o < 1024; o <<= 1) {  // inclusive Hillis-Steele scan
      const int add = threadIdx.x >= o ? part[threadIdx.x - o] : 0;
      __syncthreads();
      part[threadIdx.x] += add;
      __syncthreads();
    }
    const int c0 = carry;
    if (b < nblk) counts[b] = c0 + part[threadIdx.x] - v;
    __syncthreads();
    if (threadIdx.x == 1023) carry = c0 + part[1023];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    meta[0] = carry;
    meta[1] = 0;
    meta[2] = 0;
    meta[3] = (int32_t)T;
    cu[carry] = (int32_t)T;
  }
}

template <typename P>
__global__ __launch_bounds__(256) void meta_write_kernel(const P* __restrict__ pos, int64_t T,
                                                         const int32_t* __restrict__ offsets,
                                                         int32_t* __restrict__ cu,
                                                         int32_t* __restrict__ meta) {
  __shared__ int red[4];
  const int64_t base = (int64_t)blockIdx.x * kMetaBlock;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  // rank of each start inside the block: 4 rounds of 256 tokens, each a
  // workgroup-wide exclusive count built from wave ballots
  int off = offsets[blockIdx.x];
  int bad = 0;
  for (int u = 0; u < 4; ++u) {
    const int64_t i = base + u * 256 + threadIdx.x;
    const bool st = i < T && seq_start(pos, i);
    if (i < T && !st && pos[i] != pos[i - 1] + 1) ++bad;
    if (i < T && st && pos[i] != 0) ++bad;
    const unsigned long long m = __builtin_amdgcn_ballot_w64(st);
    const int before_in_wave = __builtin_popcountll(m & ((1ull << lane) - 1ull));
    if (lane == 0) red[w] = __builtin_popcountll(m);
    __syncthreads();
    int before = before_in_wave;
    for (int j = 0; j < w; ++j) before += red[j];
    const int total = red[0] + red[1] + red[2] + red[3];
    if (st) cu[off + before] = (int32_t)i;
    off += total;
    __syncthreads();
  }
  for (int o = 32; o > 0; o >>= 1) bad += __shfl_xor(bad, o, 64);
  if (lane == 0 && bad) atomicAdd(&meta[2], bad);
}

// Longest sequence: one pass over cu once it is complete.
__global__ __launch_bounds__(256) void meta_maxlen_kernel(const int32_t* __restrict__ cu,
                                                          int32_t* __restrict__ meta) {
  const int ns = meta[0];
  int mx = 0;
  for (int s = blockIdx.x * 256 + threadIdx.x; s < ns; s += gridDim.x * 256)
    mx = max(mx, cu[s + 1] - cu[s]);
  for (int o = 32; o > 0; o >>= 1) mx = max(mx, __shfl_xor(mx, o, 64));
  if ((threadIdx.x & 63) == 0 && mx > 0) atomicMax(&meta[1], mx);
}

}  // namespace vfk

using namespace vfk;

extern "C" int64_t vfk_varlen_meta_workspace_bytes(int64_t total_tokens) {
  if (total_tokens <= 0) return 0;
  return ((total_tokens + kMetaBlock - 1) / kMetaBlock) * (int64_t)sizeof(int32_t);
}

extern "C" int vfk_varlen_meta(const void* positions, int32_t pos_dtype_bytes, int64_t total_tokens,
                               int32_t* cu_seqlens, int32_t* meta, void* workspace,
                               int64_t workspace_bytes, void* stream) {
  if (!positions || !cu_seqlens || !meta)
    return set_error(VFK_ERR_INVALID, "vfk_varlen_meta: NULL pointer");
  if (pos_dtype_bytes != 4 && pos_dtype_bytes != 8)
    return set_error(VFK_ERR_INVALID, "vfk_varlen_meta: positions must be int32 or int64");
  if (total_tokens <= 0 || total_tokens >= (1ll << 31) - 1)
    return set_error(VFK_ERR_INVALID, "vfk_varlen_meta: total_tokens must be in [1, 2^31 - 2]");
  const int64_t need = vfk_varlen_meta_workspace_bytes(total_tokens);
  if (!workspace || workspace_bytes < need)
    return set_error(VFK_ERR_INVALID, "vfk_varlen_meta: needs a workspace of %lld bytes",
                     (long long)need);
  const int nblk = ceil_div(total_tokens, kMetaBlock);
  int32_t* counts = reinterpret_cast<int32_t*>(workspace);
  hipStream_t st = (hipStream_t)stream;
  if (pos_dtype_bytes == 8) {
    const int64_t* p = reinterpret_cast<const int64_t*>(positions);
    hipLaunchKernelGGL(meta_count_kernel<int64_t>, dim3(nblk), dim3(256), 0, st, p, total_tokens,
                       counts);
    hipLaunchKernelGGL(meta_scan_kernel, dim3(1), dim3(1024), 0, st, counts, nblk, total_tokens,
                       cu_seqlens, meta);
    hipLaunchKernelGGL(meta_write_kernel<int64_t>, dim3(nblk), dim3(256), 0, st, p, total_tokens,
                       counts, cu_seqlens, meta);
  } else {
    const int32_t* p = reinterpret_cast<const int32_t*>(positions);
    hipLaunchKernelGGL(meta_count_kernel<int32_t>, dim3(nblk), dim3(256), 0, st, p, total_tokens,
                       counts);
    hipLaunchKernelGGL(meta_scan_kernel, dim3(1), dim3(1024), 0, st, counts, nblk, total_tokens,
                       cu_seqlens, meta);
    hipLaunchKernelGGL(meta_write_kernel<int32_t>, dim3(nblk), dim3(256), 0, st, p, total_tokens,
                       counts, cu_seqlens, meta);
  }
  const int mblocks = std::min(nblk, 1024);
  hipLaunchKernelGGL(meta_maxlen_kernel, dim3(mblocks), dim3(256), 0, st, cu_seqlens, meta);
  return launch_status("vfk_varlen_meta");
}
