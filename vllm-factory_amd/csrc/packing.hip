// Packed-stream plumbing on the device: sequence metadata from vLLM's flat
// position ids, and the flat <-> padded row copies around padded encoders.
//
// Metadata replaces the reference's host/dense constructions for packed
// batches: ModernBERT's block mask (models/modernbert/modernbert_encoder.py:
// 491-516, _build_seq_block_mask: a sequence starts at token 0 and wherever
// pos[i] <= pos[i-1]) and the GLiNER plugins' split at zero positions
// (plugins/deberta_gliner/model.py:166-170: starts = (pos == 0).nonzero()).
// The starts become cu_seqlens directly, in three passes over 1024-token
// blocks:
//   1. count the starts of each block,
//   2. one workgroup scans the block counts (exclusive) and writes the
//      totals,
//   3. each block writes the indices of its starts at its offset and counts
//      breaks in the run of positions; a fourth small pass takes the longest
//      sequence from cu_seqlens.
// meta[0] = number of sequences, meta[1] = longest sequence, meta[2] = breaks
// in the run of positions (a start whose position is not 0, or a token whose
// position is not its predecessor's + 1; 0 exactly when every position equals
// index - sequence start), meta[3] = T.
//
// Pad / unpad replace the per-row Python loop of plugins/deberta_gliner/
// model.py:171-202 (batched_ids[row, :length] = input_ids[start:end], then
// torch.cat of encoded[row, :length]). Sequence b's rows are contiguous in
// both layouts, so workgroup row b copies len_b rows' bytes as one run and
// fills the rest of its padded block; no per-element index arithmetic.
//
// The GLiNER pooler front-end gathers replace the per-request loop of
// poolers/gliner.py:219-255 around _extract_gliner_reps (:313-347): the class
// tokens of all requests are compacted with the same count / scan / write
// passes, then one wave per row copies prompt rows and first-subtoken word
// rows.
#include <stdint.h>

#include <algorithm>
#include <mutex>

#include "launch_util.h"
#include "vfk_common.h"

namespace vfk {

constexpr int kMetaBlock = 1024;  // tokens per block (256 threads x 4)

// RULE 0 (VFK_SEQ_RESET): start where the position does not increase;
// RULE 1 (VFK_SEQ_ZERO): start where the position is 0. Token 0 always starts.
template <int RULE, typename P>
__device__ inline bool seq_start(const P* pos, int64_t i) {
  if (i == 0) return true;
  return RULE == 0 ? pos[i] <= pos[i - 1] : pos[i] == 0;
}

template <int RULE, typename P>
__global__ __launch_bounds__(256) void meta_count_kernel(const P* __restrict__ pos, int64_t T,
                                                         int32_t* __restrict__ counts) {
  __shared__ int red[4];
  const int64_t base = (int64_t)blockIdx.x * kMetaBlock;
  int c = 0;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int64_t i = base + u * 256 + threadIdx.x;
    if (i < T && seq_start<RULE>(pos, i)) ++c;
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

template <int RULE, typename P>
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
    const bool st = i < T && seq_start<RULE>(pos, i);
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

// ---------------------------------------------------------------------------
// flat [T, row] <-> padded [B, L, row]
// ---------------------------------------------------------------------------
constexpr int kPadU = 4;  // units per thread and pass, issued loads-first

// Workgroup row b = sequence b. Units t < min(len_b, L) * upr of the padded
// block come from flat row cu[b] + t / upr; the rest get `fill`. The main loop
// takes kPadU units per thread with every load and store unconditional (loads
// at indices clamped into the sequence, so the compiler cannot sink them into
// predicated stores and serialise them); one predicated pass takes the tail.
template <typename U>
__global__ __launch_bounds__(256) void pad_rows_kernel(const U* __restrict__ src,
                                                       U* __restrict__ dst,
                                                       const int32_t* __restrict__ cu,
                                                       int32_t* __restrict__ seq_lengths,
                                                       uint32_t L, uint32_t upr, U fill) {
  const int b = blockIdx.y;
  const int start = cu[b];
  const int len = cu[b + 1] - start;
  if (seq_lengths && blockIdx.x == 0 && threadIdx.x == 0) seq_lengths[b] = len;
  const uint32_t n = L * upr;
  const uint32_t valid = (uint32_t)min(max(len, 0), (int)L) * upr;
  U* d = dst + (size_t)b * n;
  const uint32_t step = gridDim.x * 256 * kPadU;
  uint32_t t0 = blockIdx.x * 256 * kPadU + threadIdx.x;
  if (valid == 0) {  // empty sequence: its flat rows may not exist, fill only
    for (uint32_t t = blockIdx.x * 256 + threadIdx.x; t < n; t += gridDim.x * 256) d[t] = fill;
    return;
  }
  const U* s = src + (size_t)start * upr;
  const uint32_t last = valid - 1;
  for (; t0 + (kPadU - 1) * 256 < n; t0 += step) {
    U v[kPadU];
#pragma unroll
    for (int u = 0; u < kPadU; ++u) {
      const uint32_t t = t0 + u * 256;
      const U x = s[min(t, last)];
      v[u] = t < valid ? x : fill;
    }
#pragma unroll
    for (int u = 0; u < kPadU; ++u) d[t0 + u * 256] = v[u];
  }
  if (t0 < n) {
#pragma unroll
    for (int u = 0; u < kPadU; ++u) {
      const uint32_t t = t0 + u * 256;
      const U x = s[min(t, last)];
      if (t < n) d[t] = t < valid ? x : fill;
    }
  }
}

// Workgroup row b = sequence b: its first min(len_b, L) padded rows go to
// flat rows cu[b]...; workgroups past the end of a short sequence exit. Same
// main-loop / tail split as pad_rows_kernel.
template <typename U>
__global__ __launch_bounds__(256) void unpad_rows_kernel(const U* __restrict__ src,
                                                         U* __restrict__ dst,
                                                         const int32_t* __restrict__ cu,
                                                         uint32_t L, uint32_t upr) {
  const int b = blockIdx.y;
  const int start = cu[b];
  const int len = cu[b + 1] - start;
  const uint32_t valid = (uint32_t)min(max(len, 0), (int)L) * upr;
  const U* s = src + (size_t)b * L * upr;
  U* d = dst + (size_t)start * upr;
  const uint32_t step = gridDim.x * 256 * kPadU;
  uint32_t t0 = blockIdx.x * 256 * kPadU + threadIdx.x;
  for (; t0 + (kPadU - 1) * 256 < valid; t0 += step) {
    U v[kPadU];
#pragma unroll
    for (int u = 0; u < kPadU; ++u) v[u] = s[t0 + u * 256];
#pragma unroll
    for (int u = 0; u < kPadU; ++u) d[t0 + u * 256] = v[u];
  }
  if (t0 < valid) {
#pragma unroll
    for (int u = 0; u < kPadU; ++u) {
      const uint32_t t = t0 + u * 256;
      const U x = s[min(t, valid - 1)];
      if (t < valid) d[t] = x;
    }
  }
}


// ---------------------------------------------------------------------------
// GLiNER pooler front-end gathers over a packed stream
// (poolers/gliner.py:312-345, _extract_gliner_reps, once per request there).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void class_count_kernel(const int64_t* __restrict__ ids, int64_t T,
                                                          int64_t ent, int32_t* __restrict__ counts) {
  __shared__ int red[4];
  const int64_t base = (int64_t)blockIdx.x * kMetaBlock;
  int c = 0;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int64_t i = base + u * 256 + threadIdx.x;
    if (i < T && ids[i] == ent) ++c;
  }
  for (int o = 32; o > 0; o >>= 1) c += __shfl_xor(c, o, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = c;
  __syncthreads();
  if (threadIdx.x == 0) counts[blockIdx.x] = red[0] + red[1] + red[2] + red[3];
}

// Sequence of token p: the last s with cu[s] <= p (cu[0] = 0 <= p).
__device__ inline int seq_of(const int32_t* cu, int n, int64_t p) {
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (cu[mid] <= p) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

// Indices of the class tokens, in stream order, at the scanned block offsets.
// A class token whose row + shift leaves its request (the reference's
// index_select on the per-request rows raises there) sets status[0] = 1.
__global__ __launch_bounds__(256) void class_write_kernel(const int64_t* __restrict__ ids, int64_t T,
                                                          int64_t ent,
                                                          const int32_t* __restrict__ offsets,
                                                          const int32_t* __restrict__ cu, int n,
                                                          int shift, int32_t* __restrict__ idx,
                                                          int32_t* __restrict__ status) {
  __shared__ int red[4];
  const int64_t base = (int64_t)blockIdx.x * kMetaBlock;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int off = offsets[blockIdx.x];
  for (int u = 0; u < 4; ++u) {
    const int64_t i = base + u * 256 + threadIdx.x;
    const bool hit = i < T && ids[i] == ent;
    const unsigned long long m = __builtin_amdgcn_ballot_w64(hit);
    const int before_in_wave = __builtin_popcountll(m & ((1ull << lane) - 1ull));
    if (lane == 0) red[w] = __builtin_popcountll(m);
    __syncthreads();
    int before = before_in_wave;
    for (int j = 0; j < w; ++j) before += red[j];
    if (hit) {
      idx[off + before] = (int32_t)i;
      const int sq = seq_of(cu, n, i);
      const int64_t from = i + shift;
      if (status && (from < cu[sq] || from >= cu[sq + 1])) status[0] = 1;
    }
    off += red[0] + red[1] + red[2] + red[3];
    __syncthreads();
  }
}

// out_cu[s] = number of class tokens before cu[s] (lower bound in idx).
__global__ __launch_bounds__(256) void class_cu_kernel(const int32_t* __restrict__ idx,
                                                       const int32_t* __restrict__ meta,
                                                       const int32_t* __restrict__ cu, int n,
                                                       int32_t* __restrict__ out_cu) {
  const int s = blockIdx.x * 256 + threadIdx.x;
  if (s > n) return;
  const int key = cu[s];
  int lo = 0, hi = meta[0];
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (idx[mid] < key) lo = mid + 1;
    else hi = mid;
  }
  out_cu[s] = lo;
}

// One wave per destination row, 16 bytes per lane and pass; all of a
// lane's loads are issued before its stores. src == nullptr writes zeros.
template <int MAXC>
__device__ inline void copy_row(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                int chunks, int lane) {
  const u32x4_t* sp = reinterpret_cast<const u32x4_t*>(src);
  u32x4_t* dp = reinterpret_cast<u32x4_t*>(dst);
  u32x4_t v[MAXC];
  if (src) {  // clamped, unconditional loads: no per-lane branch around them
#pragma unroll
    for (int j = 0; j < MAXC; ++j) v[j] = sp[min(lane + 64 * j, chunks - 1)];
  } else {
#pragma unroll
    for (int j = 0; j < MAXC; ++j) v[j] = u32x4_t{0, 0, 0, 0};
  }
#pragma unroll
  for (int j = 0; j < MAXC; ++j) {
    const int c = lane + 64 * j;
    if (c < chunks) dp[c] = v[j];
  }
}

// Rows of up to MAXC * 1 KiB (64 lanes x 16 bytes per pass); wider rows loop.
template <int MAXC>
__device__ inline void copy_row_any(const uint8_t* src, uint8_t* dst, int64_t row_bytes, int lane) {
  const int64_t chunks = row_bytes / 16;
  for (int64_t c0 = 0; c0 < chunks; c0 += 64 * MAXC) {
    copy_row<MAXC>(src ? src + c0 * 16 : nullptr, dst + c0 * 16,
                   (int)min<int64_t>(chunks - c0, 64 * MAXC), lane);
  }
}

// pe[r] = tok[class_idx[r] + shift] for r < meta[0], the shifted row clamped
// into the stream (an out-of-request row was flagged by the index pass).
__global__ __launch_bounds__(256) void prompt_rows_kernel(const uint8_t* __restrict__ tok,
                                                          int64_t row_bytes, int64_t T,
                                                          const int32_t* __restrict__ idx,
                                                          const int32_t* __restrict__ meta, int shift,
                                                          uint8_t* __restrict__ pe) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= meta[0]) return;
  const int64_t from = min<int64_t>(max<int64_t>((int64_t)idx[r] + shift, 0), T - 1);
  copy_row_any<2>(tok + from * row_bytes, pe + r * row_bytes, row_bytes, threadIdx.x & 63);
}

// One thread per token. Token p with words_mask[p] = w > 0 is the first
// subtoken of word w when no earlier token of its request has a positive
// mask, or the nearest one that has holds another word (the reference's
// keep[1:] = tgt[1:] != tgt[:-1] over the positive-mask tokens). Its index
// goes to word_src[word_cu[s] + w - 1] as p + 1; a word id past the
// request's word count sets status[0] = 1 instead (an IndexError in the
// reference). The predecessor decides almost every token; lanes whose
// predecessor has mask 0 (the first text token after the prompt, gaps) look
// further back one at a time with the whole wave, 64 tokens per step.
__global__ __launch_bounds__(256) void word_index_kernel(const int64_t* __restrict__ wm, int64_t T,
                                                         const int32_t* __restrict__ cu, int n,
                                                         const int32_t* __restrict__ word_cu,
                                                         int32_t* __restrict__ word_src,
                                                         int32_t* __restrict__ status) {
  const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int lane = threadIdx.x & 63;
  const bool in = p < T;
  const int64_t w = in ? wm[p] : 0;
  const bool pos = w > 0;
  int s = 0;
  int64_t first = 0;
  if (pos) {
    s = seq_of(cu, n, p);
    first = max<int64_t>(cu[s], 0);
  }
  int64_t prev = -1;  // mask of the nearest earlier positive token, 0 if none
  if (pos) prev = p - 1 >= first ? wm[p - 1] : 0;
  bool keep = pos && prev != w;
  unsigned long long todo = __builtin_amdgcn_ballot_w64(pos && prev == 0 && p - 1 >= first);
  while (todo) {
    const int l = __builtin_ctzll(todo);
    todo &= todo - 1;
    const int64_t pl = __shfl(p, l, 64), fl = __shfl(first, l, 64);
    int64_t found = 0;
    for (int64_t hi = pl - 2; hi >= fl; hi -= 64) {
      const int64_t q = hi - lane;
      const int64_t v = q >= fl ? wm[q] : 0;
      const unsigned long long m = __builtin_amdgcn_ballot_w64(v > 0);
      if (m) {
        found = __shfl(v, __builtin_ctzll(m), 64);
        break;
      }
    }
    if (lane == l) keep = found != w;
  }
  if (!keep) return;
  const int64_t slot = w - 1;
  if (slot >= (int64_t)(word_cu[s + 1] - word_cu[s])) {
    if (status) status[0] = 1;
    return;
  }
  word_src[word_cu[s] + slot] = (int32_t)(p + 1);
}

// we[j] = tok[word_src[j] - 1], or zeros where word_src[j] == 0.
__global__ __launch_bounds__(256) void word_rows_kernel(const uint8_t* __restrict__ tok,
                                                        int64_t row_bytes, int64_t T,
                                                        const int32_t* __restrict__ word_src,
                                                        int64_t W, uint8_t* __restrict__ we) {
  const int64_t j = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (j >= W) return;
  const int64_t p = (int64_t)word_src[j] - 1;
  const uint8_t* src = (p >= 0 && p < T) ? tok + p * row_bytes : nullptr;
  copy_row_any<2>(src, we + j * row_bytes, row_bytes, threadIdx.x & 63);
}

// ReLU on the raw bits of a 16-byte chunk: a negative value (sign set, not
// NaN) becomes +0, everything else (NaN included) passes, as torch.relu's
// NaN-propagating maximum does. EB: element bytes (2 = bf16, 3 = fp16, 4 = fp32;
// bf16 and fp16 differ only in where NaN starts).
template <int EB>
__device__ inline u32x4_t relu_bits(u32x4_t v) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t w = v[i];
    if (EB == 4) {
      if ((w & 0x80000000u) && (w & 0x7fffffffu) <= 0x7f800000u) w = 0u;
    } else {
      constexpr uint32_t kInf = EB == 2 ? 0x7f80u : 0x7c00u;
      const uint32_t lo = w & 0xffffu, hi = w >> 16;
      const uint32_t lo2 = ((lo & 0x8000u) && (lo & 0x7fffu) <= kInf) ? 0u : lo;
      const uint32_t hi2 = ((hi & 0x8000u) && (hi & 0x7fffu) <= kInf) ? 0u : hi;
      w = lo2 | (hi2 << 16);
    }
    v[i] = w;
  }
  return v;
}

// Span pair rows of SpanMarkerV0 (poolers/gliner.py:131-145 with
// extract_elements :40-45), for span s of request r (span_cu[r] <= s <
// span_cu[r + 1]) over r's L = row_cu[r + 1] - row_cu[r] word rows:
// i = clamp(span_idx[s][0] * m, 0, L - 1), j = clamp(span_idx[s][1] * m, 0,
// L - 1) with m = span_mask[s] (the reference multiplies the indices by the
// mask value), out[s] = relu(cat(start[row_cu[r] + i], end[row_cu[r] + j])).
// L == 0 gives a zero row. Each wave writes kSpansPerWave consecutive spans:
// lanes 0.. resolve their span's source rows in parallel, then every lane
// issues all of its 16-byte loads (addresses selected per lane, rows clamped
// so that no load is conditional) before its stores.
constexpr int kSpansPerWave = 4;
constexpr int kSpanPass = 3;  // 16-byte chunks per lane and span in one pass

template <int EB>
__global__ __launch_bounds__(256) void span_rows_kernel(const uint8_t* __restrict__ start,
                                                        const uint8_t* __restrict__ end,
                                                        int64_t row_bytes, int64_t W,
                                                        const int32_t* __restrict__ row_cu,
                                                        const int64_t* __restrict__ idx,
                                                        const int64_t* __restrict__ mask,
                                                        const int32_t* __restrict__ span_cu, int n,
                                                        int64_t S, uint8_t* __restrict__ out) {
  const int64_t s0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * kSpansPerWave;
  const int lane = threadIdx.x & 63;
  if (s0 >= S) return;
  const int chunks = (int)(row_bytes / 16), total = 2 * chunks;
  const u32x4_t zero = {0u, 0u, 0u, 0u};
  if (W <= 0) {  // no rows at all: every span is a zero row
    for (int64_t sp = s0; sp < min(S, s0 + kSpansPerWave); ++sp)
      for (int c = lane; c < total; c += 64)
        reinterpret_cast<u32x4_t*>(out + sp * 2 * row_bytes)[c] = zero;
    return;
  }
  int64_t ra = -1, rb = -1;  // source rows of span s0 + lane (-1: zero row)
  if (lane < kSpansPerWave && s0 + lane < S) {
    const int64_t sp = s0 + lane;
    const int r = seq_of(span_cu, n, sp);
    const int64_t base = row_cu[r], L = (int64_t)row_cu[r + 1] - base;
    if (L > 0) {
      const int64_t m = mask[sp];
      const int64_t i = idx[2 * sp] * m, j = idx[2 * sp + 1] * m;
      ra = base + min(max(i, (int64_t)0), L - 1);
      rb = base + min(max(j, (int64_t)0), L - 1);
    }
  }
  for (int c0 = 0; c0 < total; c0 += 64 * kSpanPass) {
    u32x4_t v[kSpansPerWave][kSpanPass];
#pragma unroll
    for (int u = 0; u < kSpansPerWave; ++u) {
      const int64_t a = __shfl(ra, u, 64), b = __shfl(rb, u, 64);
#pragma unroll
      for (int k = 0; k < kSpanPass; ++k) {
        const int c = min(c0 + lane + 64 * k, total - 1);
        const bool first = c < chunks;
        const int64_t row = min(max(first ? a : b, (int64_t)0), W - 1);
        const uint8_t* src = (first ? start : end) + row * row_bytes + (int64_t)(first ? c : c - chunks) * 16;
        const u32x4_t x = *reinterpret_cast<const u32x4_t*>(src);
        v[u][k] = a >= 0 ? relu_bits<EB>(x) : zero;
      }
    }
#pragma unroll
    for (int u = 0; u < kSpansPerWave; ++u) {
      if (s0 + u >= S) break;
      u32x4_t* dst = reinterpret_cast<u32x4_t*>(out + (s0 + u) * 2 * row_bytes);
#pragma unroll
      for (int k = 0; k < kSpanPass; ++k) {
        const int c = c0 + lane + 64 * k;
        // non-temporal: the pair rows stream out without displacing the
        // source rows that neighbouring spans read again from L2
        if (c < total) __builtin_nontemporal_store(v[u][k], dst + c);
      }
    }
  }
}

// Source rows of span sp under the pair-row rules above, or -1 for a request
// without rows.
__device__ inline void span_rows_of(const int32_t* __restrict__ row_cu, const int64_t* __restrict__ idx,
                                    const int64_t* __restrict__ mask, const int32_t* __restrict__ span_cu,
                                    int n, int64_t sp, int64_t& ra, int64_t& rb) {
  const int r = seq_of(span_cu, n, sp);
  const int64_t base = row_cu[r], L = (int64_t)row_cu[r + 1] - base;
  ra = rb = -1;
  if (L > 0) {
    const int64_t m = mask[sp];
    ra = base + min(max(idx[2 * sp] * m, (int64_t)0), L - 1);
    rb = base + min(max(idx[2 * sp + 1] * m, (int64_t)0), L - 1);
  }
}

// 16 bytes of a row as fp32 and back; EB is the type tag of span_rows_kernel
// (2 bf16, 3 fp16: 8 values; 4 fp32: 4 values).
template <int EB>
__device__ inline void ld16(const uint8_t* p, float* f) {
  const u32x4_t v = *reinterpret_cast<const u32x4_t*>(p);
  if constexpr (EB == 4) {
#pragma unroll
    for (int i = 0; i < 4; ++i) f[i] = __uint_as_float(v[i]);
  } else if constexpr (EB == 2) {
    unpack8<BF16>(v, f);
  } else {
    unpack8<F16>(v, f);
  }
}
// The store is non-temporal: output rows stream out without displacing the
// source rows that neighbouring spans read again from L2.
template <int EB>
__device__ inline void st16_nt(uint8_t* p, const float* f) {
  u32x4_t v;
  if constexpr (EB == 4) {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = __float_as_uint(f[i]);
  } else if constexpr (EB == 2) {
    v = pack8<BF16>(f);
  } else {
    v = pack8<F16>(f);
  }
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4_t*>(p));
}

// SpanMarkerV0's out_project first layer without the pair rows: with
// a = relu(start) W1[:, :D]^T and b = relu(end) W1[:, D:]^T computed per word
// row, the layer's output for span s is relu(a[i] + b[j] + b1) (the ReLU of
// cat(start[i], end[j]) distributes over the halves, and W1 splits with
// them). out[s] = relu(a[ra] + b[rb] + bias), summed in fp32 in that order and
// rounded once; ra, rb as for the pair rows (a request without rows adds
// nothing: relu(bias)).
//
// Each wave writes kHidSpans consecutive spans. The row loads, served from
// L2, bound this kernel (its output stream alone runs near the HBM write
// rate). Where the wave's spans are kHidStarts consecutive starts of the
// default span list with all kHidWidths widths valid (span u = (i + u / 12,
// i + u / 12 + u % 12)), the wave loads each of its 4 start rows and 15 end
// rows once per chunk for all 48 spans: 20 row loads for 48 outputs where
// span-by-span loading takes 96. Other span lists, and the starts whose
// widths run past the text, run the wave's spans in groups of
// kSpansPerWave, every span loading both of its rows.
constexpr int kHidWidths = 12;
constexpr int kHidStarts = 4;
constexpr int kHidSpans = kHidStarts * kHidWidths;
constexpr int kHidPass = 2;  // 16-byte chunks per lane and span in one pass of the group form

__device__ inline int64_t readlane64(int64_t v, int l) {
  const int lo = __builtin_amdgcn_readlane((int)(uint32_t)v, l);
  const int hi = __builtin_amdgcn_readlane((int)(v >> 32), l);
  return (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}

template <int EB>
__device__ inline void unpack16(u32x4_t v, float* f) {
  if constexpr (EB == 4) {
#pragma unroll
    for (int i = 0; i < 4; ++i) f[i] = __uint_as_float(v[i]);
  } else if constexpr (EB == 2) {
    unpack8<BF16>(v, f);
  } else {
    unpack8<F16>(v, f);
  }
}

// Three waves per SIMD (<= 168 VGPRs): the 48-span form holds 20 packed row
// chunks and 4 unpacked start rows per lane; the compiler's own choice, 177
// VGPRs and two waves, ran ~1 % slower.
template <int EB>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void span_hidden_kernel(const uint8_t* __restrict__ a,
                                                          const uint8_t* __restrict__ b,
                                                          const uint8_t* __restrict__ bias,
                                                          int64_t row_bytes, int64_t W,
                                                          const int32_t* __restrict__ row_cu,
                                                          const int64_t* __restrict__ idx,
                                                          const int64_t* __restrict__ mask,
                                                          const int32_t* __restrict__ span_cu, int n,
                                                          int64_t S, uint8_t* __restrict__ out) {
  constexpr int V = EB == 4 ? 4 : 8;  // values per 16 bytes (EB: 2 bf16, 3 fp16, 4 fp32)
  // each XCD takes a contiguous run of spans, so the rows that neighbouring
  // spans share are reused from that XCD's L2
  const int64_t blk = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t s0 = (blk * 4 + (threadIdx.x >> 6)) * kHidSpans;
  const int lane = threadIdx.x & 63;
  if (s0 >= S) return;
  const int chunks = (int)(row_bytes / 16);
  const int ns = (int)min((int64_t)kHidSpans, S - s0);
  int64_t ra = -1, rb = -1;  // source rows of span s0 + lane
  if (lane < ns && W > 0) span_rows_of(row_cu, idx, mask, span_cu, n, s0 + lane, ra, rb);
  // every load is unconditional: sources that do not exist (no bias, no
  // rows at all) are read from a valid row and their values replaced by 0
  const bool hb = bias != nullptr, hr = W > 0;
  const uint8_t* src_a = hr ? a : (hb ? bias : out);
  const uint8_t* src_b = hr ? b : (hb ? bias : out);
  const uint8_t* src_c = hb ? bias : src_a;
  const int64_t rs = hr ? row_bytes : 0, wmax = hr ? W - 1 : 0;
  const int64_t a0 = readlane64(ra, 0);
  const bool grid = hr && a0 >= 0 && ns == kHidSpans &&
                    __builtin_amdgcn_ballot_w64(lane < kHidSpans &&
                                                (ra != a0 + lane / kHidWidths ||
                                                 rb != ra + lane % kHidWidths)) == 0ull;
  if (grid) {
    // start rows a0 .. a0 + 3 and end rows a0 .. a0 + 14, all valid rows
    const uint8_t* arow = src_a + a0 * rs;
    const uint8_t* brow = src_b + a0 * rs;
    for (int c0 = 0; c0 < chunks; c0 += 64) {
      const int c = c0 + lane;
      const uint32_t off = (uint32_t)min(c, chunks - 1) * 16u;
      const u32x4_t cq = *reinterpret_cast<const u32x4_t*>(src_c + off);
      u32x4_t aq[kHidStarts], bq[kHidStarts + kHidWidths - 1];
#pragma unroll
      for (int i = 0; i < kHidStarts; ++i) aq[i] = *reinterpret_cast<const u32x4_t*>(arow + i * rs + off);
#pragma unroll
      for (int j = 0; j < kHidStarts + kHidWidths - 1; ++j)
        bq[j] = *reinterpret_cast<const u32x4_t*>(brow + j * rs + off);
      float cv[V], av[kHidStarts][V];
      unpack16<EB>(cq, cv);
#pragma unroll
      for (int i = 0; i < kHidStarts; ++i) unpack16<EB>(aq[i], av[i]);
      // end row j serves start i at width j - i; each end row is unpacked once
      // and its outputs written before the next (predicated, not branched
      // out of: the loops must unroll fully so that bq stays in registers)
#pragma unroll
      for (int j = 0; j < kHidStarts + kHidWidths - 1; ++j) {
        float bv[V];
        unpack16<EB>(bq[j], bv);
#pragma unroll
        for (int i = 0; i < kHidStarts; ++i) {
          const int w = j - i;
          if (w < 0 || w >= kHidWidths) continue;  // compile-time: fully unrolled
          float y[V];
#pragma unroll
          for (int e = 0; e < V; ++e) {
            const float v = (av[i][e] + bv[e]) + (hb ? cv[e] : 0.f);
            y[e] = v < 0.f ? 0.f : v;
          }
          if (c < chunks) st16_nt<EB>(out + (s0 + i * kHidWidths + w) * row_bytes + (int64_t)c * 16, y);
        }
      }
    }
    return;
  }
  for (int g0 = 0; g0 < ns; g0 += kSpansPerWave) {
    int64_t sa[kSpansPerWave], sb[kSpansPerWave];
#pragma unroll
    for (int u = 0; u < kSpansPerWave; ++u) {
      sa[u] = readlane64(ra, min(g0 + u, kHidSpans - 1));
      sb[u] = readlane64(rb, min(g0 + u, kHidSpans - 1));
    }
    for (int c0 = 0; c0 < chunks; c0 += 64 * kHidPass) {
      float bv[kHidPass][V], av[kSpansPerWave][kHidPass][V], cv[kSpansPerWave][kHidPass][V];
#pragma unroll
      for (int k = 0; k < kHidPass; ++k) {
        const int64_t c16 = (int64_t)min(c0 + lane + 64 * k, chunks - 1) * 16;
        ld16<EB>(src_c + c16, bv[k]);
#pragma unroll
        for (int u = 0; u < kSpansPerWave; ++u) {
          ld16<EB>(src_a + min(max(sa[u], (int64_t)0), wmax) * rs + c16, av[u][k]);
          ld16<EB>(src_b + min(max(sb[u], (int64_t)0), wmax) * rs + c16, cv[u][k]);
        }
      }
#pragma unroll
      for (int u = 0; u < kSpansPerWave; ++u) {
        if (g0 + u >= ns) break;
        const bool has = hr && sa[u] >= 0;
#pragma unroll
        for (int k = 0; k < kHidPass; ++k) {
          const int c = c0 + lane + 64 * k;
          if (c >= chunks) continue;
          float y[V];
#pragma unroll
          for (int e = 0; e < V; ++e) {
            const float bb = hb ? bv[k][e] : 0.f;
            const float v = has ? (av[u][k][e] + cv[u][k][e]) + bb : bb;
            y[e] = v < 0.f ? 0.f : v;
          }
          st16_nt<EB>(out + (s0 + g0 + u) * row_bytes + (int64_t)c * 16, y);
        }
      }
    }
  }
}

}  // namespace vfk

using namespace vfk;

extern "C" int64_t vfk_varlen_meta_workspace_bytes(int64_t total_tokens) {
  if (total_tokens <= 0) return 0;
  return ((total_tokens + kMetaBlock - 1) / kMetaBlock) * (int64_t)sizeof(int32_t);
}

template <int RULE, typename P>
static void launch_meta(const P* p, int64_t T, int nblk, int32_t* counts, int32_t* cu,
                        int32_t* meta, hipStream_t st) {
  hipLaunchKernelGGL((meta_count_kernel<RULE, P>), dim3(nblk), dim3(256), 0, st, p, T, counts);
  hipLaunchKernelGGL(meta_scan_kernel, dim3(1), dim3(1024), 0, st, counts, nblk, T, cu, meta);
  hipLaunchKernelGGL((meta_write_kernel<RULE, P>), dim3(nblk), dim3(256), 0, st, p, T, counts, cu,
                     meta);
  hipLaunchKernelGGL(meta_maxlen_kernel, dim3(std::min(nblk, 1024)), dim3(256), 0, st, cu, meta);
}

extern "C" int vfk_varlen_meta(const void* positions, int32_t pos_dtype_bytes, int64_t total_tokens,
                               int32_t rule, int32_t* cu_seqlens, int32_t* meta, void* workspace,
                               int64_t workspace_bytes, void* stream) {
  if (!positions || !cu_seqlens || !meta)
    return set_error(VFK_ERR_INVALID, "vfk_varlen_meta: NULL pointer");
  if (pos_dtype_bytes != 4 && pos_dtype_bytes != 8)
    return set_error(VFK_ERR_INVALID, "vfk_varlen_meta: positions must be int32 or int64");
  if (rule != VFK_SEQ_RESET && rule != VFK_SEQ_ZERO)
    return set_error(VFK_ERR_INVALID, "vfk_varlen_meta: unknown boundary rule %d", rule);
  if (total_tokens <= 0 || total_tokens >= (1ll << 31) - 1)
    return set_error(VFK_ERR_INVALID, "vfk_varlen_meta: total_tokens must be in [1, 2^31 - 2]");
  const int64_t need = vfk_varlen_meta_workspace_bytes(total_tokens);
  if (!workspace || workspace_bytes < need)
    return set_error(VFK_ERR_INVALID, "vfk_varlen_meta: needs a workspace of %lld bytes",
                     (long long)need);
  const int nblk = ceil_div(total_tokens, kMetaBlock);
  int32_t* counts = reinterpret_cast<int32_t*>(workspace);
  hipStream_t st = (hipStream_t)stream;
  const bool wide = pos_dtype_bytes == 8;
  const int64_t T = total_tokens;
  if (rule == VFK_SEQ_RESET) {
    if (wide) launch_meta<0>(static_cast<const int64_t*>(positions), T, nblk, counts, cu_seqlens, meta, st);
    else launch_meta<0>(static_cast<const int32_t*>(positions), T, nblk, counts, cu_seqlens, meta, st);
  } else {
    if (wide) launch_meta<1>(static_cast<const int64_t*>(positions), T, nblk, counts, cu_seqlens, meta, st);
    else launch_meta<1>(static_cast<const int32_t*>(positions), T, nblk, counts, cu_seqlens, meta, st);
  }
  return launch_status("vfk_varlen_meta");
}

// ---------------------------------------------------------------------------
// vfk_varlen_meta without a caller workspace: the per-block start counts live
// in a file-scope device array (one copy per GPU, kept for the life of the
// process). Host code never passes the array's name to a kernel: its device
// address is looked up once per device with hipGetSymbolAddress and cached.
// ---------------------------------------------------------------------------
constexpr int kNoAllocMetaBlocks = (int)(VFK_NOALLOC_MAX_TOKENS / kMetaBlock);  // 64 KiB of counts
static_assert((int64_t)kNoAllocMetaBlocks * kMetaBlock == VFK_NOALLOC_MAX_TOKENS, "whole blocks");
static __device__ __align__(256) int32_t scratch[kNoAllocMetaBlocks];

static std::mutex g_scratch_mu;
static int32_t* g_scratch_ptr[64];

// scratch's device address on the current device (looked up on first use)
static int scratch_ptr(int32_t** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error((int)e, "vfk_varlen_meta_noalloc: hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= 64) return set_error(VFK_ERR_UNSUPPORTED, "vfk_varlen_meta_noalloc: device %d", dev);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_error(e != hipSuccess ? (int)e : VFK_ERR_INVALID,
                       "vfk_varlen_meta_noalloc: hipGetSymbolAddress: %s", hipGetErrorString(e));
    g_scratch_ptr[dev] = static_cast<int32_t*>(p);
  }
  *out = g_scratch_ptr[dev];
  return VFK_OK;
}

extern "C" int vfk_varlen_meta_noalloc(const void* positions, int32_t pos_dtype_bytes,
                                       int64_t total_tokens, int32_t rule, int32_t* cu_seqlens,
                                       int32_t* meta, void* stream) {
  if (total_tokens > VFK_NOALLOC_MAX_TOKENS)
    return set_error(VFK_ERR_UNSUPPORTED,
                     "vfk_varlen_meta_noalloc: total_tokens %lld above the %lld this entry point "
                     "holds (use vfk_varlen_meta with a workspace)",
                     (long long)total_tokens, (long long)VFK_NOALLOC_MAX_TOKENS);
  int32_t* counts = nullptr;
  int rc = scratch_ptr(&counts);
  if (rc) return rc;
  // every count the kernels read is written by the same call first
  return vfk_varlen_meta(positions, pos_dtype_bytes, total_tokens, rule, cu_seqlens, meta, counts,
                         (int64_t)kNoAllocMetaBlocks * (int64_t)sizeof(int32_t), stream);
}

// Copy unit: the widest of 16/8/4/2/1 bytes dividing the row size and both
// base addresses.
static int unit_bytes(int64_t row_bytes, const void* a, const void* b) {
  const uintptr_t m = (uintptr_t)row_bytes | reinterpret_cast<uintptr_t>(a) |
                      reinterpret_cast<uintptr_t>(b);
  for (int u = 16; u > 1; u >>= 1)
    if ((m & (uintptr_t)(u - 1)) == 0) return u;
  return 1;
}

static int check_rows(const char* name, const void* src, const void* dst, const int32_t* cu,
                      int64_t row_bytes, int32_t num_seqs, int32_t max_len) {
  if (!src || !dst || !cu) return set_error(VFK_ERR_INVALID, "%s: NULL pointer", name);
  if (row_bytes <= 0) return set_error(VFK_ERR_INVALID, "%s: row_bytes must be positive", name);
  if (num_seqs <= 0 || num_seqs > 65535)
    return set_error(VFK_ERR_INVALID, "%s: num_seqs must be in [1, 65535]", name);
  if (max_len <= 0) return set_error(VFK_ERR_INVALID, "%s: max_len must be positive", name);
  // unit indices within one padded block, plus a grid stride, stay in 32 bits
  if ((int64_t)max_len * row_bytes >= (1ll << 31))
    return set_error(VFK_ERR_INVALID, "%s: max_len * row_bytes must be below 2^31", name);
  return VFK_OK;
}

template <typename U>
static void fill_unit(U& u, uint64_t bits, int elem_bytes) {
  unsigned char* p = reinterpret_cast<unsigned char*>(&u);
  for (int i = 0; i < (int)sizeof(U); ++i) p[i] = (unsigned char)(bits >> (8 * (i % elem_bytes)));
}

template <typename U>
static void launch_pad(const void* src, void* dst, const int32_t* cu, int32_t* lens, int B, int L,
                       int64_t row_bytes, uint64_t fill_bits, int elem_bytes, hipStream_t st) {
  U fill;
  fill_unit(fill, fill_bits, elem_bytes);
  const uint32_t upr = (uint32_t)(row_bytes / (int64_t)sizeof(U));
  const int64_t n = (int64_t)L * upr;
  const int gx = (int)std::min<int64_t>(ceil_div(n, 256 * kPadU), 1024);
  hipLaunchKernelGGL(pad_rows_kernel<U>, dim3(gx, B), dim3(256), 0, st,
                     static_cast<const U*>(src), static_cast<U*>(dst), cu, lens, (uint32_t)L, upr,
                     fill);
}

template <typename U>
static void launch_unpad(const void* src, void* dst, const int32_t* cu, int B, int L,
                         int64_t row_bytes, hipStream_t st) {
  const uint32_t upr = (uint32_t)(row_bytes / (int64_t)sizeof(U));
  const int64_t n = (int64_t)L * upr;
  const int gx = (int)std::min<int64_t>(ceil_div(n, 256 * kPadU), 1024);
  hipLaunchKernelGGL(unpad_rows_kernel<U>, dim3(gx, B), dim3(256), 0, st,
                     static_cast<const U*>(src), static_cast<U*>(dst), cu, (uint32_t)L, upr);
}

extern "C" int vfk_pad_rows(const void* src, int64_t row_bytes, const int32_t* cu_seqlens,
                            int32_t num_seqs, int32_t max_len, int32_t elem_bytes,
                            uint64_t fill_bits, void* dst, int32_t* seq_lengths, void* stream) {
  const char* name = "vfk_pad_rows";
  if (int rc = check_rows(name, src, dst, cu_seqlens, row_bytes, num_seqs, max_len)) return rc;
  if (elem_bytes != 1 && elem_bytes != 2 && elem_bytes != 4 && elem_bytes != 8)
    return set_error(VFK_ERR_INVALID, "%s: elem_bytes must be 1, 2, 4 or 8", name);
  const int ub = unit_bytes(row_bytes, src, dst);
  if (ub < elem_bytes)
    return set_error(VFK_ERR_INVALID,
                     "%s: row_bytes and both addresses must be multiples of elem_bytes", name);
  hipStream_t st = (hipStream_t)stream;
  switch (ub) {
    case 16: launch_pad<u32x4_t>(src, dst, cu_seqlens, seq_lengths, num_seqs, max_len, row_bytes, fill_bits, elem_bytes, st); break;
    case 8: launch_pad<u32x2_t>(src, dst, cu_seqlens, seq_lengths, num_seqs, max_len, row_bytes, fill_bits, elem_bytes, st); break;
    case 4: launch_pad<uint32_t>(src, dst, cu_seqlens, seq_lengths, num_seqs, max_len, row_bytes, fill_bits, elem_bytes, st); break;
    case 2: launch_pad<uint16_t>(src, dst, cu_seqlens, seq_lengths, num_seqs, max_len, row_bytes, fill_bits, elem_bytes, st); break;
    default: launch_pad<uint8_t>(src, dst, cu_seqlens, seq_lengths, num_seqs, max_len, row_bytes, fill_bits, elem_bytes, st); break;
  }
  return launch_status(name);
}

extern "C" int vfk_unpad_rows(const void* src, int64_t row_bytes, const int32_t* cu_seqlens,
                              int32_t num_seqs, int32_t max_len, void* dst, void* stream) {
  const char* name = "vfk_unpad_rows";
  if (int rc = check_rows(name, src, dst, cu_seqlens, row_bytes, num_seqs, max_len)) return rc;
  hipStream_t st = (hipStream_t)stream;
  switch (unit_bytes(row_bytes, src, dst)) {
    case 16: launch_unpad<u32x4_t>(src, dst, cu_seqlens, num_seqs, max_len, row_bytes, st); break;
    case 8: launch_unpad<u32x2_t>(src, dst, cu_seqlens, num_seqs, max_len, row_bytes, st); break;
    case 4: launch_unpad<uint32_t>(src, dst, cu_seqlens, num_seqs, max_len, row_bytes, st); break;
    case 2: launch_unpad<uint16_t>(src, dst, cu_seqlens, num_seqs, max_len, row_bytes, st); break;
    default: launch_unpad<uint8_t>(src, dst, cu_seqlens, num_seqs, max_len, row_bytes, st); break;
  }
  return launch_status(name);
}

extern "C" int64_t vfk_gliner_class_workspace_bytes(int64_t total_tokens) {
  return vfk_varlen_meta_workspace_bytes(total_tokens);
}

extern "C" int vfk_gliner_class_index(const int64_t* input_ids, int64_t total_tokens,
                                      int64_t ent_token_id, int32_t shift,
                                      const int32_t* cu_seqlens, int32_t num_seqs,
                                      int32_t* class_idx, int32_t* class_cu, int32_t* meta,
                                      int32_t* status, void* workspace, int64_t workspace_bytes,
                                      void* stream) {
  const char* name = "vfk_gliner_class_index";
  if (!input_ids || !cu_seqlens || !class_idx || !class_cu || !meta)
    return set_error(VFK_ERR_INVALID, "%s: NULL pointer", name);
  if (total_tokens <= 0 || total_tokens >= (1ll << 31) - 1)
    return set_error(VFK_ERR_INVALID, "%s: total_tokens must be in [1, 2^31 - 2]", name);
  if (num_seqs <= 0) return set_error(VFK_ERR_INVALID, "%s: num_seqs must be positive", name);
  const int64_t need = vfk_varlen_meta_workspace_bytes(total_tokens);
  if (!workspace || workspace_bytes < need)
    return set_error(VFK_ERR_INVALID, "%s: needs a workspace of %lld bytes", name, (long long)need);
  const int nblk = ceil_div(total_tokens, kMetaBlock);
  int32_t* counts = reinterpret_cast<int32_t*>(workspace);
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(class_count_kernel, dim3(nblk), dim3(256), 0, st, input_ids, total_tokens,
                     ent_token_id, counts);
  hipLaunchKernelGGL(meta_scan_kernel, dim3(1), dim3(1024), 0, st, counts, nblk, total_tokens,
                     class_idx, meta);
  hipLaunchKernelGGL(class_write_kernel, dim3(nblk), dim3(256), 0, st, input_ids, total_tokens,
                     ent_token_id, counts, cu_seqlens, (int)num_seqs, (int)shift, class_idx, status);
  hipLaunchKernelGGL(class_cu_kernel, dim3(ceil_div(num_seqs + 1, 256)), dim3(256), 0, st, class_idx,
                     meta, cu_seqlens, num_seqs, class_cu);
  return launch_status(name);
}

static int check_rows(const char* name, const void* a, const void* b, int64_t row_bytes) {
  if (row_bytes <= 0 || row_bytes % 16)
    return set_error(VFK_ERR_INVALID, "%s: row_bytes must be a positive multiple of 16", name);
  if ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b)) & 15)
    return set_error(VFK_ERR_INVALID, "%s: rows must be 16-byte aligned", name);
  return VFK_OK;
}

extern "C" int vfk_gliner_prompt_rows(const void* tok, int64_t row_bytes, int64_t total_tokens,
                                      const int32_t* class_idx, const int32_t* meta, int32_t shift,
                                      int64_t max_rows, void* pe, void* stream) {
  const char* name = "vfk_gliner_prompt_rows";
  if (!tok || !class_idx || !meta || !pe) return set_error(VFK_ERR_INVALID, "%s: NULL pointer", name);
  if (int rc = check_rows(name, tok, pe, row_bytes)) return rc;
  if (total_tokens <= 0 || max_rows < 0 || max_rows >= (1ll << 31) - 1)
    return set_error(VFK_ERR_INVALID, "%s: bad sizes", name);
  if (max_rows == 0) return VFK_OK;
  hipLaunchKernelGGL(prompt_rows_kernel, dim3((unsigned)ceil_div(max_rows, 4)), dim3(256), 0,
                     (hipStream_t)stream, static_cast<const uint8_t*>(tok), row_bytes, total_tokens,
                     class_idx, meta, (int)shift, static_cast<uint8_t*>(pe));
  return launch_status(name);
}

extern "C" int vfk_gliner_word_index(const int64_t* words_mask, int64_t total_tokens,
                                     const int32_t* cu_seqlens, int32_t num_seqs,
                                     const int32_t* word_cu, int32_t* word_src, int32_t* status,
                                     void* stream) {
  const char* name = "vfk_gliner_word_index";
  if (!words_mask || !cu_seqlens || !word_cu || !word_src)
    return set_error(VFK_ERR_INVALID, "%s: NULL pointer", name);
  if (total_tokens <= 0 || total_tokens >= (1ll << 31) - 1 || num_seqs <= 0)
    return set_error(VFK_ERR_INVALID, "%s: bad sizes", name);
  hipLaunchKernelGGL(word_index_kernel, dim3(ceil_div(total_tokens, 256)), dim3(256), 0,
                     (hipStream_t)stream, words_mask, total_tokens, cu_seqlens, (int)num_seqs,
                     word_cu, word_src, status);
  return launch_status(name);
}

extern "C" int vfk_gliner_word_rows(const void* tok, int64_t row_bytes, int64_t total_tokens,
                                    const int32_t* word_src, int64_t num_words, void* we,
                                    void* stream) {
  const char* name = "vfk_gliner_word_rows";
  if (!tok || !word_src || !we) return set_error(VFK_ERR_INVALID, "%s: NULL pointer", name);
  if (int rc = check_rows(name, tok, we, row_bytes)) return rc;
  if (total_tokens <= 0 || num_words < 0 || num_words >= (1ll << 31) - 1)
    return set_error(VFK_ERR_INVALID, "%s: bad sizes", name);
  if (num_words == 0) return VFK_OK;
  hipLaunchKernelGGL(word_rows_kernel, dim3((unsigned)ceil_div(num_words, 4)), dim3(256), 0,
                     (hipStream_t)stream, static_cast<const uint8_t*>(tok), row_bytes, total_tokens,
                     word_src, num_words, static_cast<uint8_t*>(we));
  return launch_status(name);
}

extern "C" int vfk_gliner_span_rows(const void* start_rep, const void* end_rep, int64_t row_bytes,
                                    int64_t num_rows, int32_t dtype, const int32_t* row_cu, int32_t num_requests,
                                    const int64_t* span_idx, const int64_t* span_mask,
                                    const int32_t* span_cu, int64_t num_spans, void* out,
                                    void* stream) {
  const char* name = "vfk_gliner_span_rows";
  if (!start_rep || !end_rep || !row_cu || !span_idx || !span_mask || !span_cu || !out)
    return set_error(VFK_ERR_INVALID, "%s: NULL pointer", name);
  if (int rc = check_rows(name, start_rep, out, row_bytes)) return rc;
  if (int rc = check_rows(name, end_rep, out, row_bytes)) return rc;
  if (num_requests <= 0 || num_rows < 0 || num_spans < 0 || num_spans >= (1ll << 31) - 1)
    return set_error(VFK_ERR_INVALID, "%s: bad sizes", name);
  if (num_spans == 0) return VFK_OK;
  const dim3 grid((unsigned)ceil_div(num_spans, 4 * kSpansPerWave));
  hipStream_t st = (hipStream_t)stream;
  const uint8_t* sp = static_cast<const uint8_t*>(start_rep);
  const uint8_t* ep = static_cast<const uint8_t*>(end_rep);
  uint8_t* op = static_cast<uint8_t*>(out);
  if (dtype == VFK_BF16)
    hipLaunchKernelGGL(span_rows_kernel<2>, grid, dim3(256), 0, st, sp, ep, row_bytes, num_rows, row_cu, span_idx,
                       span_mask, span_cu, (int)num_requests, num_spans, op);
  else if (dtype == VFK_F16)
    hipLaunchKernelGGL(span_rows_kernel<3>, grid, dim3(256), 0, st, sp, ep, row_bytes, num_rows, row_cu, span_idx,
                       span_mask, span_cu, (int)num_requests, num_spans, op);
  else if (dtype == VFK_F32)
    hipLaunchKernelGGL(span_rows_kernel<4>, grid, dim3(256), 0, st, sp, ep, row_bytes, num_rows, row_cu, span_idx,
                       span_mask, span_cu, (int)num_requests, num_spans, op);
  else
    return set_error(VFK_ERR_INVALID, "%s: dtype must be bf16, fp16 or fp32", name);
  return launch_status(name);
}

extern "C" int vfk_gliner_span_hidden(const void* a, const void* b, const void* bias, int64_t row_bytes,
                                      int64_t num_rows, int32_t dtype, const int32_t* row_cu,
                                      int32_t num_requests, const int64_t* span_idx,
                                      const int64_t* span_mask, const int32_t* span_cu,
                                      int64_t num_spans, void* out, void* stream) {
  const char* name = "vfk_gliner_span_hidden";
  if (!a || !b || !row_cu || !span_idx || !span_mask || !span_cu || !out)
    return set_error(VFK_ERR_INVALID, "%s: NULL pointer", name);
  if (int rc = check_rows(name, a, out, row_bytes)) return rc;
  if (int rc = check_rows(name, b, bias ? bias : out, row_bytes)) return rc;
  if (num_requests <= 0 || num_rows < 0 || num_spans < 0 || num_spans >= (1ll << 31) - 1)
    return set_error(VFK_ERR_INVALID, "%s: bad sizes", name);
  if (num_spans == 0) return VFK_OK;
  const dim3 grid((unsigned)ceil_div(num_spans, 4 * kHidSpans));
  hipStream_t st = (hipStream_t)stream;
  const uint8_t* ap = static_cast<const uint8_t*>(a);
  const uint8_t* bp = static_cast<const uint8_t*>(b);
  const uint8_t* cp = static_cast<const uint8_t*>(bias);
  uint8_t* op = static_cast<uint8_t*>(out);
#define VFK_SH(EB)                                                                                  \
  hipLaunchKernelGGL(span_hidden_kernel<EB>, grid, dim3(256), 0, st, ap, bp, cp, row_bytes, num_rows, \
                     row_cu, span_idx, span_mask, span_cu, (int)num_requests, num_spans, op)
  if (dtype == VFK_BF16) VFK_SH(2);
  else if (dtype == VFK_F16) VFK_SH(3);
  else if (dtype == VFK_F32) VFK_SH(4);
  else return set_error(VFK_ERR_INVALID, "%s: dtype must be bf16, fp16 or fp32", name);
#undef VFK_SH
  return launch_status(name);
}
