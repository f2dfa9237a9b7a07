// GLU projection with the activation and gate product in the epilogue
// (bf16 / fp16 on v_mfma_f32_32x32x16, gfx950).
//
// out[t, f] = act(x[t] . w[f]) * (x[t] . w[I + f]) for a projection weight
// w [2I, K] whose first I rows give the activation input and the last I rows
// the gate: ModernBERT's MLP (Wi, chunk, GELU(input) * gate) and the T5 gated
// FF (wi_0 / wi_1 stacked) without writing the [M, 2I] projection.
//
// Work split: a 256-thread workgroup owns 256 tokens x 128 output features.
// Wave (wm, wn) = (w / 2, w % 2) owns tokens 128 wm .. +128 and features
// 64 wn .. +64 of both weight halves: 4 token blocks x 2 feature blocks x
// {input, gate} = 16 accumulator blocks. A = weight rows, B = token rows, so
// lane (c, h) of a result block holds token c and features
// 8 (r / 4) + 4 h + r % 4 (r < 16): the input and gate sums of one output sit
// in the same lane and register index.
//
// K loop: 64-wide K slices of the 256 token rows and of the 256 weight rows
// (input rows f0 .. +128, then gate rows I + f0 .. +128) go from global memory
// straight into LDS (global_load_lds_dwordx4): three 32 KiB token stages and
// two 32 KiB weight stages, one barrier per slice. Each row is a 128-byte LDS row whose 16-byte chunks are
// XOR-swizzled by swz(row), the layout of the attention kernels' K tiles.
// Rows past the end of x or w read as zeros through the buffer range check.
//
// Persistent: one workgroup per CU. Workgroup i runs on XCD i % 8 and walks
// every g8-th tile of that XCD's share (tiles numbered feature-fastest), so the
// workgroups of one XCD hold the feature tiles of the same token tiles at any
// time: a token tile comes from HBM once and from that XCD's L2 after. The K
// slices of all of a workgroup's tiles form one stream, so the next tile's
// first slices load while the previous tile's epilogue runs.
#include "activation.h"
#include "attn_core.h"
#include "launch_util.h"

#include <algorithm>

namespace vfk {
namespace {

constexpr int kGRows = 256;          // tokens per workgroup tile
constexpr int kGFeat = 128;          // output features per workgroup tile
constexpr int kGSlice = 32768;       // bytes of one K slice of 256 rows (128 B each)
constexpr int kGWBase = 3 * kGSlice; // token rows: 3 stages, then weight rows: 2 stages
constexpr int kGLds = 5 * kGSlice;   // 160 KiB, all of a CU's LDS

// Waits until at most the wave's 8 newest vector-memory loads are in flight
// (the token rows two slices ahead, issued after everything the next slice
// needs; loads complete in issue order) and its LDS reads are done, then
// joins the workgroup barrier. One asm statement with a memory clobber: a
// release fence on LDS would make the compiler wait for every direct-to-LDS
// load, the two-slice lead included.
__device__ inline void slice_barrier() {
  asm volatile("s_waitcnt vmcnt(8) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

struct GluArgs {
  const uint16_t* x;
  const uint16_t* w;
  uint16_t* out;
  int64_t M;
  int K, I;       // head-pair mode: I = 3 H 64 / 2 (half the weight rows)
  int xs2, ws2;   // row strides of x and w in bytes
  int64_t os;     // row stride of out in elements
  int mt, nt;
  int per_xcd;  // tiles of one XCD: XCD x owns tiles x * per_xcd .. +per_xcd
  int g8;       // workgroups per XCD
  // head-pair mode (the fused q | k | v projection with RoPE on the k heads)
  int H;                  // heads per projection
  const int32_t* pos;     // [M] rotary position of each token
  const float* rope;      // fp32 [npos][32][2] (cos, sin)
  int npos;
  float c2;               // softmax scale * log2(e), folded into the rotated k
  uint16_t* qo;           // q rows [M, H, 64] (token stride qs)
  uint16_t* vo;           // v rows [M, H, 64] (token stride vs)
  int64_t qs, vs;
  uint16_t* kr;           // rotated k, head-major [H][M][64]
  float* kmax;            // [H][nb32]: largest row norm of each 32-token block
  int64_t nb32;
};

// One 64-wide K slice from stage st: 4 MFMA k-steps of 16 accumulator blocks,
// the operands of k-step ds + 1 read from LDS while k-step ds multiplies.
// ko[ds]: the lane's byte offset of chunk 2 ds + h in row c of a block.
struct GluFrags {
  u32x4_t x[4], w[4];  // token blocks tb; weight blocks 2 g + fb
};

__device__ inline void glu_frags(GluFrags& f, const char* xs, const char* ws, int ox, int ow) {
#pragma unroll
  for (int tb = 0; tb < 4; ++tb) f.x[tb] = *reinterpret_cast<const u32x4_t*>(xs + ox + 4096 * tb);
#pragma unroll
  for (int g = 0; g < 2; ++g)
#pragma unroll
    for (int fb = 0; fb < 2; ++fb)
      f.w[2 * g + fb] = *reinterpret_cast<const u32x4_t*>(ws + ow + 16384 * g + 4096 * fb);
}

template <typename E>
__device__ inline void glu_mfma(const GluFrags& f, f32x16_t (&acc)[2][2][4]) {
#pragma unroll
  for (int g = 0; g < 2; ++g)
#pragma unroll
    for (int fb = 0; fb < 2; ++fb)
#pragma unroll
      for (int tb = 0; tb < 4; ++tb)
        acc[g][fb][tb] = E::mfma32(f.w[2 * g + fb], f.x[tb], acc[g][fb][tb]);
}

// Instruction order of one k-step: its 16 MFMAs with the next k-step's 8 LDS
// reads between them, or, with loads, the 8 reads after the first MFMA and the
// next slices' 16 direct-to-LDS loads between the rest, so that operand and
// tile traffic overlap the matrix pipe.
__device__ inline void glu_order(bool with_loads) {
  if (with_loads) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
    for (int k = 0; k < 15; ++k) {
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
  } else {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    }
  }
}

// Epilogue of the head-pair mode for one wave: accumulator block fb of the
// input half holds d = 8 (r / 4) + 4 h + r % 4 of head 4 ni + 2 wn + fb (over
// the 3H heads of q | k | v), the gate half d + 32 of the same head, for the
// tokens t0 + 32 tb (lane c). q and v heads are stored as they are; k heads
// are rotated with the (cos, sin) row of the token's position (the rotate-half
// pairs d, d + 32 sit in one lane and register index), multiplied by c2,
// rounded once and stored head-major, and the largest norm of the rounded
// rows of each 32-token block goes to kmax.
// Stores a lane's four 4-value runs (run j: d = 8 j + 4 h .. +3) of one 32-d
// half as two 16-byte stores: lanes c and c + 32 trade runs so that lane h = 0
// holds d = 0..7 and 16..23, lane h = 1 holds 8..15 and 24..31.
__device__ inline void store_runs16(uint16_t* row, const u32x2_t (&run)[4]) {
  const int h = (threadIdx.x & 63) >> 5;
#pragma unroll
  for (int jp = 0; jp < 2; ++jp) {
    const u32x2_t a = run[2 * jp], b = run[2 * jp + 1];
    const u32x2_t send = h ? a : b;
    const u32x2_t got = {(uint32_t)__shfl_xor((int)send[0], 32), (uint32_t)__shfl_xor((int)send[1], 32)};
    const u32x4_t v = h ? u32x4_t{got[0], got[1], b[0], b[1]} : u32x4_t{a[0], a[1], got[0], got[1]};
    *reinterpret_cast<u32x4_t*>(row + 16 * jp + 8 * h) = v;
  }
}

template <typename E>
__device__ inline void qkv_epilogue(const GluArgs& a, const f32x16_t (&acc)[2][2][4], int mi,
                                    int ni, int wm, int wn) {
  const int l = threadIdx.x & 63, c = l & 31, h = l >> 5;
  const int64_t tb0 = (int64_t)mi * kGRows + 128 * wm;  // first token of block tb = 0
#pragma unroll
  for (int fb = 0; fb < 2; ++fb) {
    const int hh = 4 * ni + 2 * wn + fb;
    if (hh >= 3 * a.H) continue;  // uniform: past the last head
    const int region = hh / a.H, hd = hh - region * a.H;
    if (region != 1) {
      uint16_t* base = (region == 0 ? a.qo : a.vo) + hd * 64;
      const int64_t rs = region == 0 ? a.qs : a.vs;
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        const int64_t t = tb0 + 32 * tb + c;
        if (t >= a.M) continue;
        uint16_t* row = base + t * rs;
        const f32x16_t& lo = acc[0][fb][tb];
        const f32x16_t& hi = acc[1][fb][tb];
        u32x2_t p0[4], p1[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          p0[j] = u32x2_t{E::pack2(lo[4 * j], lo[4 * j + 1]), E::pack2(lo[4 * j + 2], lo[4 * j + 3])};
          p1[j] = u32x2_t{E::pack2(hi[4 * j], hi[4 * j + 1]), E::pack2(hi[4 * j + 2], hi[4 * j + 3])};
        }
        // lanes c and c + 32 (one token) are active together
        store_runs16(row, p0);
        store_runs16(row + 32, p1);
      }
      continue;
    }
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
      const int64_t t = tb0 + 32 * tb + c;
      const bool tv = t < a.M;
      const int p = tv ? min(max(a.pos[t], 0), a.npos - 1) : 0;
      const float* cs = a.rope + (int64_t)p * 64;
      uint16_t* row = a.kr + ((int64_t)hd * a.M + (tv ? t : 0)) * 64;
      float nrm = 0.f;
      u32x2_t r0[4], r1[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d0 = 8 * j + 4 * h;
        const f32x4_t c01 = *reinterpret_cast<const f32x4_t*>(cs + 2 * d0);
        const f32x4_t c23 = *reinterpret_cast<const f32x4_t*>(cs + 2 * d0 + 4);
        const float cv[4] = {c01[0], c01[2], c23[0], c23[2]};
        const float sv[4] = {c01[1], c01[3], c23[1], c23[3]};
        float k1[4], k2[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float x1 = acc[0][fb][tb][4 * j + e], x2 = acc[1][fb][tb][4 * j + e];
          k1[e] = (x1 * cv[e] - x2 * sv[e]) * a.c2;
          k2[e] = (x2 * cv[e] + x1 * sv[e]) * a.c2;
        }
        const u32x2_t p0 = {E::pack2(k1[0], k1[1]), E::pack2(k1[2], k1[3])};
        const u32x2_t p1 = {E::pack2(k2[0], k2[1]), E::pack2(k2[2], k2[3])};
        // squared norm of the rounded values (the ones the attention uses)
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const float a0 = E::to_f32((uint16_t)(p0[u] & 0xffffu)), a1 = E::to_f32((uint16_t)(p0[u] >> 16));
          const float b0 = E::to_f32((uint16_t)(p1[u] & 0xffffu)), b1 = E::to_f32((uint16_t)(p1[u] >> 16));
          nrm = __builtin_fmaf(a0, a0, nrm);
          nrm = __builtin_fmaf(a1, a1, nrm);
          nrm = __builtin_fmaf(b0, b0, nrm);
          nrm = __builtin_fmaf(b1, b1, nrm);
        }
        r0[j] = p0;
        r1[j] = p1;
      }
      if (tv) {  // lanes c and c + 32 (one token) are active together
        store_runs16(row, r0);
        store_runs16(row + 32, r1);
      }
      // lanes c and c + 32 hold the two halves of the token's d values; then
      // the largest over the block's 32 tokens (rows past M are zeros)
      nrm += __shfl_xor(nrm, 32);
#pragma unroll
      for (int o = 1; o < 32; o <<= 1) nrm = fmaxf(nrm, __shfl_xor(nrm, o));
      const int64_t blk = (tb0 + 32 * tb) >> 5;
      if (l == 0 && tb0 + 32 * tb < a.M) a.kmax[hd * a.nb32 + blk] = sqrtf(nrm);
    }
  }
}

// QKV: head-pair mode (weight rows of heads in halves d < 32 / d >= 32, the
// qkv_epilogue); otherwise the GLU product act(input) * gate.
template <typename E, int ACT, bool QKV = false>
__global__ __launch_bounds__(256, 1) void gemm_glu_kernel(GluArgs a) {
  __shared__ __attribute__((aligned(1024))) char smem[kGLds];
  // Workgroup i runs on XCD i % 8 and takes every g8-th tile of that XCD's
  // range from i / 8 on, so the g8 workgroups of an XCD work on consecutive
  // tiles (feature tiles of the same token tile) at any time.
  const int ntiles = a.mt * a.nt;
  const int lo = (blockIdx.x & 7) * a.per_xcd, j0 = blockIdx.x >> 3;
  const int span = min(a.per_xcd, ntiles - lo);
  if (j0 >= span) return;
  const int nk = a.K >> 6;
  const int total = ((span - j0 + a.g8 - 1) / a.g8) * nk;  // K slices of all my tiles
  const int l = threadIdx.x & 63, c = l & 31, h = l >> 5;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = w >> 1, wn = w & 1;
  // An AGPR operand tells the compiler that this kernel uses AGPRs, which
  // selects the MFMA form that keeps the 256 accumulators there.
  asm volatile("" ::"a"(0));

  // Wave w loads LDS rows 64 w .. +64 of the token tile and of the weight
  // tile (rows 0-127: input rows f0 .., rows 128-255: gate rows I + f0 ..).
  // The buffer resources start at the wave's first row and end at the last
  // row that exists, so rows past M or 2I read as zeros. Head-pair mode: LDS
  // row r of a wave's weight rows is weight row r + 32 (r / 32) from the
  // wave's base, the first (or second) 32 rows of two consecutive heads.
  int vx[8], vw[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int r = 8 * j + (l >> 3);  // swz(64 w + r) == swz(r)
    const int ch = 16 * ((l & 7) ^ swz(r));
    vx[j] = r * a.xs2 + ch;
    vw[j] = (QKV ? r + 32 * (r >> 5) : r) * a.ws2 + ch;
  }
  // slice gs of the stream: K slice ks of my tile gs / nk at (mi, ni)
  auto slice_of = [&](int gs, int& ks, int& mi, int& ni) {
    const int k = gs / nk;
    ks = gs - k * nk;
    const int L = lo + j0 + k * a.g8;
    mi = L / a.nt;
    ni = L - mi * a.nt;
  };
  auto load_x = [&](int ks, int mi, char* st) {
    const int64_t r0 = (int64_t)mi * kGRows + 64 * w;
    const int64_t n = a.M - r0;
    const int rows = n <= 0 ? 0 : (n >= 64 ? 64 : (int)n);
    const rsrc_t r = uniform_rsrc(a.x + (rows > 0 ? r0 : 0) * (a.xs2 >> 1), rows * a.xs2);
#pragma unroll
    for (int j = 0; j < 8; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)(st + (8 * w + j) * 1024), 16,
                                               vx[j], ks * 128, 0, 0);
  };
  auto load_w = [&](int ks, int ni, char* st) {
    // head pairs: heads 4 ni + 2 (w & 1) and + 1, rows d < 32 (waves 0, 1) or
    // d >= 32 (waves 2, 3); the lane rows reach 95 rows past the base
    const int r0 = QKV ? 64 * (4 * ni + 2 * (w & 1)) + (w < 2 ? 0 : 32)
                       : (w < 2 ? 0 : a.I) + ni * kGFeat + 64 * (w & 1);
    const int n = 2 * a.I - r0;
    const int rmax = QKV ? 96 : 64;
    const int rows = n <= 0 ? 0 : (n >= rmax ? rmax : n);
    const rsrc_t r =
        uniform_rsrc(a.w + (int64_t)(rows > 0 ? r0 : 0) * (a.ws2 >> 1), rows * a.ws2);
#pragma unroll
    for (int j = 0; j < 8; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)(st + (8 * w + j) * 1024), 16,
                                               vw[j], ks * 128, 0, 0);
  };
  // Position of a load stream in the slice stream: slice ks of tile (mi, ni),
  // `left` slices after it. step() moves to the next slice without branches
  // and stays on the last one at the end.
  const int dn = a.g8 % a.nt, dm = a.g8 / a.nt;
  struct Pos {
    int ks, mi, ni, left;
  };
  auto pos_at = [&](int gs) {
    Pos p;
    slice_of(gs, p.ks, p.mi, p.ni);
    p.left = total - 1 - gs;
    return p;
  };
  auto step = [&](Pos& p) {
    const int adv = p.left > 0 ? 1 : 0;
    p.left -= adv;
    const int ks1 = p.ks + adv;
    const bool wrap = ks1 == nk;
    p.ks = wrap ? 0 : ks1;
    const int ni1 = p.ni + (wrap ? dn : 0);
    const int mi1 = p.mi + (wrap ? dm : 0);
    const bool over = ni1 >= a.nt;
    p.ni = over ? ni1 - a.nt : ni1;
    p.mi = over ? mi1 + 1 : mi1;
  };

  int ko[4];
#pragma unroll
  for (int ds = 0; ds < 4; ++ds) ko[ds] = 128 * c + 16 * ((2 * ds + h) ^ swz(c));
  const int xo = 16384 * wm, wo = 8192 * wn;

  f32x16_t acc[2][2][4];
#pragma unroll
  for (int g = 0; g < 2; ++g)
#pragma unroll
    for (int fb = 0; fb < 2; ++fb)
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) acc[g][fb][tb] = f32x16_t{};

  // Slice gs of the stream sits in token stage gs % 3 and weight stage
  // gs % 2. Iteration gs issues the weight loads of slice gs + 1 and the token
  // loads of slice gs + 2 during k-step 0 (token rows come from HBM the first
  // time, so they get two slices of lead), takes the barrier after k-step 2
  // (every wave has then read all of slice gs, and slice gs + 1 has landed),
  // reads k-step 0 of slice gs + 1 while k-step 3 of slice gs multiplies, and
  // after a tile's last slice writes that tile while the next tile's first
  // slices arrive (reading k-step 0 after the epilogue there, which keeps the
  // epilogue's registers free). Past the end the loads repeat the last slice into the free
  // stage, which keeps the barrier's wait count fixed.
  char* const xsm = smem;
  char* const wsm = smem + kGWBase;
  Pos px = pos_at(0);
  load_x(px.ks, px.mi, xsm);
  load_w(px.ks, px.ni, wsm);
  step(px);
  Pos pw = px;  // weight stream: slice gs + 1
  load_x(px.ks, px.mi, xsm + kGSlice);
  step(px);     // token stream: slice gs + 2
  slice_barrier();
  GluFrags fa, fb;
  glu_frags(fa, xsm, wsm, ko[0] + xo, ko[0] + wo);
  int xc = 0, wc = 0;  // byte offsets of the current slice's stages
  // k-steps 0-2 of the current slice with the stream's next loads, then the
  // barrier; returns with the stages advanced and k-step 3's operands in fb
  auto slice_head = [&]() {
    const int xn = xc == 2 * kGSlice ? 0 : xc + kGSlice;
    const int xnn = xn == 2 * kGSlice ? 0 : xn + kGSlice;
    const int wn1 = wc ^ kGSlice;
    const char* xs = xsm + xc;
    const char* ws = wsm + wc;
    // reads of this stage first: the compiler keeps LDS reads behind earlier
    // direct-to-LDS writes, which it cannot tell apart from this stage
    glu_frags(fb, xs, ws, ko[1] + xo, ko[1] + wo);
    load_w(pw.ks, pw.ni, wsm + wn1);
    load_x(px.ks, px.mi, xsm + xnn);
    step(pw);
    step(px);
    glu_mfma<E>(fa, acc);
    glu_order(true);
    glu_frags(fa, xs, ws, ko[2] + xo, ko[2] + wo);
    glu_mfma<E>(fb, acc);
    glu_order(false);
    glu_frags(fb, xs, ws, ko[3] + xo, ko[3] + wo);
    glu_mfma<E>(fa, acc);
    glu_order(false);
    __builtin_amdgcn_sched_barrier(0);
    slice_barrier();
    __builtin_amdgcn_sched_barrier(0);
    xc = xn;
    wc = wn1;
  };
  const int ntile = total / nk;
  for (int tile = 0; tile < ntile; ++tile) {
    for (int kk = 0; kk + 1 < nk; ++kk) {
      slice_head();
      glu_frags(fa, xsm + xc, wsm + wc, ko[0] + xo, ko[0] + wo);
      glu_mfma<E>(fb, acc);
      glu_order(false);
      __builtin_amdgcn_sched_barrier(0);
    }
    slice_head();
    glu_mfma<E>(fb, acc);
    // epilogue of this tile: act(input) * gate, runs of 4 features per
    // store, then cleared accumulators and k-step 0 of the next tile's first
    // slice (its loads are on their way meanwhile)
    int kk, mi, ni;
    slice_of(tile * nk, kk, mi, ni);
    const int64_t t0 = (int64_t)mi * kGRows + 128 * wm + c;
    const int fl = ni * kGFeat + 64 * wn + 4 * h;
    if (QKV) qkv_epilogue<E>(a, acc, mi, ni, wm, wn);
#pragma unroll
    for (int tb = 0; tb < 4 && !QKV; ++tb) {
      const int64_t t = t0 + 32 * tb;
      if (t >= a.M) continue;
      uint16_t* orow = a.out + t * a.os;
#pragma unroll
      for (int fb2 = 0; fb2 < 2; ++fb2)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          const int f = fl + 32 * fb2 + 8 * g4;
          if (f >= a.I) continue;
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e)
            v[e] = act_f<ACT>(acc[0][fb2][tb][4 * g4 + e]) * acc[1][fb2][tb][4 * g4 + e];
          const u32x2_t pk = {E::pack2(v[0], v[1]), E::pack2(v[2], v[3])};
          *reinterpret_cast<u32x2_t*>(orow + f) = pk;
        }
    }
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
      for (int fb2 = 0; fb2 < 2; ++fb2)
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) acc[g][fb2][tb] = f32x16_t{};
    glu_frags(fa, xsm + xc, wsm + wc, ko[0] + xo, ko[0] + wo);
  }
  __builtin_amdgcn_s_waitcnt(0);  // the repeated last slices
}

template <typename E>
void launch_glu(int act, const GluArgs& a, int grid, hipStream_t st) {
  switch (act) {
    case VFK_ACT_GELU_ERF:
      gemm_glu_kernel<E, VFK_ACT_GELU_ERF><<<grid, 256, 0, st>>>(a);
      break;
    case VFK_ACT_GELU_TANH:
      gemm_glu_kernel<E, VFK_ACT_GELU_TANH><<<grid, 256, 0, st>>>(a);
      break;
    case VFK_ACT_SILU:
      gemm_glu_kernel<E, VFK_ACT_SILU><<<grid, 256, 0, st>>>(a);
      break;
    default:
      gemm_glu_kernel<E, VFK_ACT_RELU><<<grid, 256, 0, st>>>(a);
      break;
  }
}

// Tiles per XCD and workgroups per XCD (one per CU: the kernel takes all of a
// CU's LDS); returns the grid size.
int persistent_grid(GluArgs& a) {
  a.per_xcd = (int)(((int64_t)a.mt * a.nt + VFK_NUM_XCD - 1) / VFK_NUM_XCD);
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus < VFK_NUM_XCD)
    cus = 256;
  a.g8 = std::min(cus / VFK_NUM_XCD, a.per_xcd);
  return a.g8 * VFK_NUM_XCD;
}

}  // namespace
}  // namespace vfk

using namespace vfk;

extern "C" int vfk_glu_linear_fwd(int32_t act, const vfk_tensor* x, const vfk_tensor* w,
                                  vfk_tensor* out, void* stream) {
  int rc;
  if ((rc = check_tensor(x, "x", 2)) || (rc = check_tensor(w, "w", 2)) ||
      (rc = check_tensor(out, "out", 2)))
    return rc;
  if (act < VFK_ACT_GELU_ERF || act > VFK_ACT_RELU)
    return set_error(VFK_ERR_INVALID, "glu_linear: unknown activation %d", act);
  const int dt = x->dtype;
  if (dt != VFK_BF16 && dt != VFK_F16)
    return set_error(VFK_ERR_UNSUPPORTED, "glu_linear: x must be bf16 or fp16");
  if (w->dtype != dt || out->dtype != dt)
    return set_error(VFK_ERR_INVALID, "glu_linear: x, w and out must share one dtype");
  const int64_t M = x->size[0], K = x->size[1], I2 = w->size[0];
  if (w->size[1] != K || I2 % 2 != 0)
    return set_error(VFK_ERR_INVALID, "glu_linear: w must be [2I, K] for x [M, K]");
  const int64_t I = I2 / 2;
  if (out->size[0] != M || out->size[1] != I)
    return set_error(VFK_ERR_INVALID, "glu_linear: out must be [M, I] = [%lld, %lld]",
                     (long long)M, (long long)I);
  if (x->stride[1] != 1 || w->stride[1] != 1 || out->stride[1] != 1)
    return set_error(VFK_ERR_UNSUPPORTED, "glu_linear: rows must be contiguous");
  if (K < 64 || K % 64 != 0)
    return set_error(VFK_ERR_UNSUPPORTED, "glu_linear: K must be a positive multiple of 64, got %lld",
                     (long long)K);
  if (I < 8 || I % 8 != 0)
    return set_error(VFK_ERR_UNSUPPORTED, "glu_linear: I must be a positive multiple of 8, got %lld",
                     (long long)I);
  if (!aligned16(x->data) || !aligned16(w->data) || !aligned16(out->data) || x->stride[0] % 8 ||
      w->stride[0] % 8 || out->stride[0] % 8)
    return set_error(VFK_ERR_UNSUPPORTED,
                     "glu_linear: base pointers and row strides must be 16-byte aligned");
  if (x->stride[0] < K || w->stride[0] < K || out->stride[0] < I)
    return set_error(VFK_ERR_INVALID, "glu_linear: overlapping rows");
  // lane offsets reach 255 x-rows and weight row 2I + 127 (past the end: zeros)
  if ((int64_t)kGRows * x->stride[0] * 2 >= (1ll << 31) ||
      (2 * I + kGFeat) * w->stride[0] * 2 >= (1ll << 31))
    return set_error(VFK_ERR_UNSUPPORTED, "glu_linear: x row stride or w too large");
  if (M == 0) return VFK_OK;
  const int64_t mt = (M + kGRows - 1) / kGRows, nt = (I + kGFeat - 1) / kGFeat;
  if (mt * nt >= (1ll << 30)) return set_error(VFK_ERR_UNSUPPORTED, "glu_linear: too many tiles");
  GluArgs a = {};
  a.x = static_cast<const uint16_t*>(x->data);
  a.w = static_cast<const uint16_t*>(w->data);
  a.out = static_cast<uint16_t*>(out->data);
  a.M = M;
  a.K = (int)K;
  a.I = (int)I;
  a.xs2 = (int)(x->stride[0] * 2);
  a.ws2 = (int)(w->stride[0] * 2);
  a.os = out->stride[0];
  a.mt = (int)mt;
  a.nt = (int)nt;
  const int grid = persistent_grid(a);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dt == VFK_BF16)
    launch_glu<BF16>(act, a, grid, st);
  else
    launch_glu<F16>(act, a, grid, st);
  return launch_status("glu_linear");
}

static int64_t qkv_kr_bytes(int64_t M, int64_t H) { return (M * H * 64 * 2 + 255) / 256 * 256; }
static int64_t qkv_nb32(int64_t M) { return (M + 31) / 32; }

extern "C" int64_t vfk_qkv_rope_workspace_bytes(int64_t tokens, int32_t num_heads) {
  if (tokens <= 0 || num_heads <= 0) return 0;
  return qkv_kr_bytes(tokens, num_heads) + (int64_t)num_heads * qkv_nb32(tokens) * 4;
}

extern "C" int vfk_qkv_rope_linear_fwd(const vfk_tensor* x, const vfk_tensor* w,
                                       const int32_t* positions, const float* rope_cos_sin,
                                       int32_t rope_positions, int32_t num_heads,
                                       float softmax_scale, vfk_tensor* q_out, vfk_tensor* v_out,
                                       void* workspace, int64_t workspace_bytes, void* stream) {
  const char* nm = "qkv_rope_linear";
  int rc;
  if ((rc = check_tensor(x, "x", 2)) || (rc = check_tensor(w, "w", 2)) ||
      (rc = check_tensor(q_out, "q_out", 3)) || (rc = check_tensor(v_out, "v_out", 3)))
    return rc;
  const int dt = x->dtype;
  if (dt != VFK_BF16 && dt != VFK_F16)
    return set_error(VFK_ERR_UNSUPPORTED, "%s: x must be bf16 or fp16", nm);
  if (w->dtype != dt || q_out->dtype != dt || v_out->dtype != dt)
    return set_error(VFK_ERR_INVALID, "%s: x, w, q_out and v_out must share one dtype", nm);
  const int64_t M = x->size[0], K = x->size[1], H = num_heads;
  if (H <= 0 || H > 4096) return set_error(VFK_ERR_INVALID, "%s: num_heads %lld", nm, (long long)H);
  if (w->size[0] != 3 * H * 64 || w->size[1] != K)
    return set_error(VFK_ERR_INVALID, "%s: w must be [3 * %lld * 64, K] for x [M, K]", nm,
                     (long long)H);
  for (const vfk_tensor* t : {q_out, v_out}) {
    if (t->size[0] != M || t->size[1] != H || t->size[2] != 64)
      return set_error(VFK_ERR_INVALID, "%s: q_out / v_out must be [M, %lld, 64]", nm, (long long)H);
    if (t->stride[2] != 1 || t->stride[1] % 4 || t->stride[0] % 4 || !aligned16(t->data))
      return set_error(VFK_ERR_UNSUPPORTED, "%s: q_out / v_out rows must be 8-byte aligned runs", nm);
  }
  if (x->stride[1] != 1 || w->stride[1] != 1)
    return set_error(VFK_ERR_UNSUPPORTED, "%s: rows must be contiguous", nm);
  if (K < 64 || K % 64 != 0)
    return set_error(VFK_ERR_UNSUPPORTED, "%s: K must be a positive multiple of 64, got %lld", nm,
                     (long long)K);
  if (!aligned16(x->data) || !aligned16(w->data) || x->stride[0] % 8 || w->stride[0] % 8)
    return set_error(VFK_ERR_UNSUPPORTED, "%s: base pointers and row strides must be 16-byte aligned",
                     nm);
  if (x->stride[0] < K || w->stride[0] < K) return set_error(VFK_ERR_INVALID, "%s: overlapping rows", nm);
  if (!positions) return set_error(VFK_ERR_INVALID, "%s: positions is NULL", nm);
  if (!rope_cos_sin || rope_positions <= 0 || !aligned16(rope_cos_sin))
    return set_error(VFK_ERR_INVALID, "%s: rope table missing, empty or not 16-byte aligned", nm);
  if (!(softmax_scale > 0.f) || !isfinite(softmax_scale))
    return set_error(VFK_ERR_UNSUPPORTED, "%s: softmax_scale must be > 0", nm);
  if (M == 0) return VFK_OK;
  const int64_t need = vfk_qkv_rope_workspace_bytes(M, num_heads);
  if (!workspace || workspace_bytes < need || !aligned16(workspace))
    return set_error(VFK_ERR_INVALID, "%s: workspace needs %lld 16-byte aligned bytes", nm,
                     (long long)need);
  // lane offsets reach 255 x-rows; weight rows reach the last tile's base + 95
  if ((int64_t)kGRows * x->stride[0] * 2 >= (1ll << 31) ||
      (3 * H * 64 + 256) * w->stride[0] * 2 >= (1ll << 31) || M * H * 64 >= (1ll << 40))
    return set_error(VFK_ERR_UNSUPPORTED, "%s: x row stride, w or M too large", nm);
  const int64_t mt = (M + kGRows - 1) / kGRows, nt = (3 * H + 3) / 4;  // four heads per tile
  if (mt * nt >= (1ll << 30)) return set_error(VFK_ERR_UNSUPPORTED, "%s: too many tiles", nm);
  GluArgs a = {};
  a.x = static_cast<const uint16_t*>(x->data);
  a.w = static_cast<const uint16_t*>(w->data);
  a.M = M;
  a.K = (int)K;
  a.I = (int)(3 * H * 32);
  a.xs2 = (int)(x->stride[0] * 2);
  a.ws2 = (int)(w->stride[0] * 2);
  a.mt = (int)mt;
  a.nt = (int)nt;
  a.H = (int)H;
  a.pos = positions;
  a.rope = rope_cos_sin;
  a.npos = rope_positions;
  a.c2 = softmax_scale * VFK_LOG2E;
  a.qo = static_cast<uint16_t*>(q_out->data);
  a.vo = static_cast<uint16_t*>(v_out->data);
  a.qs = q_out->stride[0];
  a.vs = v_out->stride[0];
  a.kr = static_cast<uint16_t*>(workspace);
  a.nb32 = qkv_nb32(M);
  a.kmax = reinterpret_cast<float*>(static_cast<char*>(workspace) + qkv_kr_bytes(M, H));
  const int grid = persistent_grid(a);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dt == VFK_BF16)
    gemm_glu_kernel<BF16, VFK_ACT_RELU, true><<<grid, 256, 0, st>>>(a);
  else
    gemm_glu_kernel<F16, VFK_ACT_RELU, true><<<grid, 256, 0, st>>>(a);
  return launch_status(nm);
}
