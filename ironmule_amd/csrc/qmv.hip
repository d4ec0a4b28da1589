// MI355X (gfx950, CDNA4) kernels and C ABI for the 4-bit affine group-64
// matrix-vector product.  The ABI is declared in include/ironmule_qmv.h.
//
// Arithmetic (the reference's per-group identity, ironmule/qmv_k3840.py:93-109 and
// ironmule/cuda_native.py:101-104):
//     sum_k (s*q_k + b) * x_k  =  s * sum_k q_k x_k  +  b * sum_k x_k
// accumulated in fp32, with the weight never materialised.
//
// How the nibbles meet the activations.  A nibble q placed in the low mantissa bits of
// the bf16 pattern 0x4300 (= 128.0) is the bf16 value 128 + q, exactly.  One
// v_and_or_b32 turns a word shifted by 4p into the bf16 pair (128+q_p, 128+q_{p+4}).
// The matching x values are therefore used in the pair order (x0,x4) (x1,x5) (x2,x6)
// (x3,x7) of each word.  The offset is removed with the group's sum of x:
//     s * sum (128+q) x  +  (b - 128 s) * sum x.
// The MFMA kernels place q in mantissa bits 3..6 of bf16 1.0 instead (the value 1 + q/16,
// same pair order): 16 s * sum (1 + q/16) x + (b - 16 s) * sum x, whose fp32 sums carry
// terms near |x| rather than 128 |x| (an MFMA sum starts from zero, not from the offset).
//
// Kernels sharing that arithmetic:
//   * qmv_m1_kernel / qmv_m1c_kernel / qmv_rows_kernel (one or two rows): v_dot2_f32_bf16
//     chains, x staged once per workgroup in LDS already in pair order, each chain
//     started at -128 * sum(x);
//   * the MFMA kernels (3 to 32 rows): v_mfma_f32_32x32x16_bf16 with the activation rows
//     as the A operand and 32 weight rows as the B operand, four MFMAs per group of 64,
//     and the group's sums of x from MFMAs against a ones operand or dot2 against (1, 1).
//
// Layout in HBM is the reference's own (row-major w (N, K/8) uint32, s and b (N, K/64)
// bf16), so a caller passes its buffers unchanged.  One launch may serve up to
// IMQ_MAX_PROBLEMS weights (for example q/k/v, or gate/up, which read the same x).

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <string>

#include "../../include/ironmule_qmv.h"
#include "common.h"
#include "runtime.h"

namespace {

using namespace imq_dev;

constexpr int kThreads = 256;  // 4 wavefronts of 64
constexpr int kGroup = 64;
constexpr int kMaxProblems = IMQ_MAX_PROBLEMS;

// ------------------------------------------------------------------ kernel args

struct Problem {
  const uint32_t* w;
  const uint16_t* s;
  const uint16_t* b;
  const uint16_t* x;  // row m at x + m * ldx (unless the pointer table is used)
  void* y;            // row m at y + m * ldy elements
  int64_t ldx;
  int64_t ldy;
  int32_t N;
  int32_t K;
  int32_t nch;        // one-row VALU kernel: 16-byte weight chunks per lane
  int32_t lpr_shift;  // VALU kernels: log2 of the lanes that share one weight row
  int32_t pad0;
  int32_t pad1;
};

struct LaunchArgs {
  Problem p[kMaxProblems];
  const uint16_t* xt[IMQ_MAX_ROWS];  // per-row pointers when `table` (single problem)
  void* yt[IMQ_MAX_ROWS];
  int32_t count;
  int32_t M;
  int32_t y_f32;
  int32_t table;
  int32_t pad[2];
};

// Every kernel runs on a (tiles, problems) grid: blockIdx.y names the problem, so a
// workgroup reads its problem's arguments in one round trip, and blockIdx.x the tile.
// The grid is as wide as the problem with the most tiles; the surplus workgroups of the
// other problems return at once.

__device__ __forceinline__ const uint16_t* x_row(const LaunchArgs& a, const Problem& P, int m) {
  return a.table ? a.xt[m] : P.x + (size_t)m * P.ldx;
}

__device__ __forceinline__ void store_y(const LaunchArgs& a, const Problem& P, int m, int row,
                                        float v) {
  if (a.y_f32) {
    float* y = a.table ? static_cast<float*>(a.yt[m])
                       : static_cast<float*>(P.y) + (size_t)m * P.ldy;
    y[row] = v;
  } else {
    uint16_t* y = a.table ? static_cast<uint16_t*>(a.yt[m])
                          : static_cast<uint16_t*>(P.y) + (size_t)m * P.ldy;
    y[row] = f32_to_bf16_bits(v);
  }
}

// ------------------------------------------------- an RMSNorm folded into projections
//
// rms_norm(h) W^T = inv (h * w) W^T per row, inv = 1 / sqrt(sum(h^2) / dim + eps): the
// kernel that produces h writes x' = bf16(h * w) and, per 64-column tile of h, the row's
// partial sum of squares; the kernel that consumes x' scales its product rows by inv.  No
// launch of its own and no round trip through a normalised copy of h.
struct NormIn {
  const float* ssq;  // row m's partials at ssq[m * ld + t], t < tiles (nullptr: off)
  int32_t tiles;     // 1 .. kNormMaxTiles
  int32_t ld;        // a multiple of 4, >= tiles
  int32_t dim;
  float eps;
};
struct ResidualOut {
  float* h;            // h[m][n] += bf16(y[m][n]), rows ldh apart (nullptr: off)
  int64_t ldh;
  const uint16_t* w;   // the next RMSNorm's weight (nullptr: h only)
  uint16_t* x;         // x'[m][n] = bf16(h[m][n] * w[n]), rows ldx apart
  int64_t ldx;
  float* ssq;          // ssq[m * ld + tile] = sum over the tile's columns of h^2 (nullptr: none)
  int32_t ld;
  int32_t pad;
};
constexpr int kNormMaxTiles = 128;
constexpr int kNormSlots = IMQ_MAX_ROWS * kNormMaxTiles / 4;  // (row, four partials) pairs

// One b128 of the partials of pair p = (row p % 32, partials 4 (p / 32) ..): the offset to
// load, or past the buffer (zeros, no traffic) for pairs past the rows or the partials.
__device__ __forceinline__ uint32_t norm_pair_offset(const NormIn& ni, int M, int p) {
  const int m = p & 31, j = p >> 5;
  return m < M && 4 * j < ni.tiles ? (uint32_t)(m * ni.ld + 4 * j) * 4u : kPastBuffer;
}

// The four partials of pair p, added in order, those past `tiles` as zeros.
__device__ __forceinline__ float norm_pair_sum(const NormIn& ni, int p, uint4 v) {
  const int t0 = 4 * (p >> 5);
  const float a = __uint_as_float(v.x), b = t0 + 1 < ni.tiles ? __uint_as_float(v.y) : 0.0f;
  const float c = t0 + 2 < ni.tiles ? __uint_as_float(v.z) : 0.0f;
  const float d = t0 + 3 < ni.tiles ? __uint_as_float(v.w) : 0.0f;
  return ((a + b) + c) + d;
}

// inv of row m from the pair sums in LDS (sums[j][m]), added in pair order.
__device__ __forceinline__ float norm_row_inv(const NormIn& ni, const float (*sums)[32], int m) {
  float ss = 0.0f;
  for (int j = 0; 4 * j < ni.tiles; ++j) ss += sums[j][m];
  return 1.0f / sqrtf(ss / (float)ni.dim + ni.eps);
}

// ----------------------------------------------------------- VALU kernel (few rows)
//
// One workgroup per tile of weight rows of one problem (no persistent loop: the
// hardware dispatcher keeps every CU fed as tiles retire).  LPR lanes share a weight
// row (LPR = 16, 32 or 64, chosen per problem so that each lane gets several 16-byte
// chunks); lane j of a row takes chunks kc = j, j+LPR, ... (32 nibbles, half a group
// each).  A tile is 4 wavefronts x 64/LPR rows.  The chunks are loaded in batches of B,
// the next batch in flight while the current one computes; the first batch is issued
// before x is staged, so the staging round trip overlaps the first weight loads.
//
// LDS holds this problem's x in pair order: xq[m][t][kc] (uint4: word t of chunk kc),
// then sx[m][kc] (the chunk's sum of x).

template <int B>
struct Batch {
  uint4 w[B];
  uint32_t s[B];
  uint32_t b[B];
};

template <int B>
__device__ __forceinline__ void load_batch(Batch<B>& t, const uint32_t* wrow, const uint16_t* srow,
                                           const uint16_t* brow, int j, int sh, int batch, int C) {
#pragma unroll
  for (int q = 0; q < B; ++q) {
    const int kc = j + ((batch * B + q) << sh);
    const int kk = kc < C ? kc : 0;
    // streamed once: the non-temporal cache policy
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(wrow + kk * 4));
    t.w[q] = make_uint4(v.x, v.y, v.z, v.w);
    t.s[q] = srow[kk >> 1];
    t.b[q] = brow[kk >> 1];
  }
}

template <int M, int B>
__device__ __forceinline__ void compute_batch(const Batch<B>& t, float (&acc)[M], const uint4* xq,
                                              const float* sx, int j, int sh, int batch, int C,
                                              uint32_t magic) {
#pragma unroll
  for (int q = 0; q < B; ++q) {
    const int kc = j + ((batch * B + q) << sh);
    const bool valid = kc < C;
    const int kk = valid ? kc : 0;
    const float sc = bf16_bits_to_f32(t.s[q]);
    const float bi = bf16_bits_to_f32(t.b[q]);
    const uint4 wv = t.w[q];
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const uint4 x0 = xq[(m * 4 + 0) * C + kk];
      const uint4 x1 = xq[(m * 4 + 1) * C + kk];
      const uint4 x2 = xq[(m * 4 + 2) * C + kk];
      const uint4 x3 = xq[(m * 4 + 3) * C + kk];
      const float sxm = sx[m * C + kk];
      float d = -128.0f * sxm;
      d = dot2(nibble_pair(wv.x, 0, magic), x0.x, d);
      d = dot2(nibble_pair(wv.x, 1, magic), x0.y, d);
      d = dot2(nibble_pair(wv.x, 2, magic), x0.z, d);
      d = dot2(nibble_pair(wv.x, 3, magic), x0.w, d);
      d = dot2(nibble_pair(wv.y, 0, magic), x1.x, d);
      d = dot2(nibble_pair(wv.y, 1, magic), x1.y, d);
      d = dot2(nibble_pair(wv.y, 2, magic), x1.z, d);
      d = dot2(nibble_pair(wv.y, 3, magic), x1.w, d);
      d = dot2(nibble_pair(wv.z, 0, magic), x2.x, d);
      d = dot2(nibble_pair(wv.z, 1, magic), x2.y, d);
      d = dot2(nibble_pair(wv.z, 2, magic), x2.z, d);
      d = dot2(nibble_pair(wv.z, 3, magic), x2.w, d);
      d = dot2(nibble_pair(wv.w, 0, magic), x3.x, d);
      d = dot2(nibble_pair(wv.w, 1, magic), x3.y, d);
      d = dot2(nibble_pair(wv.w, 2, magic), x3.z, d);
      d = dot2(nibble_pair(wv.w, 3, magic), x3.w, d);
      const float v = fmaf(sc, d, fmaf(bi, sxm, acc[m]));
      acc[m] = valid ? v : acc[m];
    }
  }
}

template <int M, int B>
__global__ __launch_bounds__(kThreads) void qmv_rows_kernel(LaunchArgs a) {
  extern __shared__ uint4 smem[];
  const Problem& P = a.p[blockIdx.y];
  const int K = P.K, N = P.N, sh = P.lpr_shift;
  if ((int)(blockIdx.x * (kThreads >> sh)) >= N) return;  // past this problem's tiles
  const int C = K >> 5;  // 32-value chunks per row
  const int G = K >> 6;  // groups per row
  const int W = K >> 3;  // words per row
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int j = lane & ((1 << sh) - 1);
  const int row = ((blockIdx.x * 4 + wave) << (6 - sh)) + (lane >> sh);
  const int r = row < N ? row : N - 1;  // clamp loads; the store is guarded
  const uint32_t* wrow = P.w + (size_t)r * W;
  const uint16_t* srow = P.s + (size_t)r * G;
  const uint16_t* brow = P.b + (size_t)r * G;
  const int nb = (((C + (1 << sh) - 1) >> sh) + B - 1) / B;
  uint4* xq = smem;
  float* sx = reinterpret_cast<float*>(smem + M * 4 * C);
  const uint32_t magic = in_vgpr(kMagic);

  // x first (loads complete in order, so x issued before the weights can be staged
  // while the first weight batch is still in flight), then the first weight batch.
  constexpr int XR = 4;  // x words per thread per staging round
  uint4 xs[M][XR];
#pragma unroll
  for (int m = 0; m < M; ++m) {
    const uint4* xv = reinterpret_cast<const uint4*>(x_row(a, P, m));
#pragma unroll
    for (int t = 0; t < XR; ++t) {
      const int i = tid + kThreads * t;
      if (i < W) xs[m][t] = xv[i];
    }
  }
  Batch<B> ping, pong;
  load_batch(ping, wrow, srow, brow, j, sh, 0, C);

  for (int base = 0; base < W; base += kThreads * XR) {
    if (base > 0) {  // x longer than one round (K > 8192)
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const uint4* xv = reinterpret_cast<const uint4*>(x_row(a, P, m));
#pragma unroll
        for (int t = 0; t < XR; ++t) {
          const int i = base + tid + kThreads * t;
          if (i < W) xs[m][t] = xv[i];
        }
      }
    }
#pragma unroll
    for (int m = 0; m < M; ++m) {
#pragma unroll
      for (int t = 0; t < XR; ++t) {
        const int i = base + tid + kThreads * t;
        if (i < W) {  // the four words of a chunk are four aligned lanes (W % 4 == 0)
          xq[(m * 4 + (i & 3)) * C + (i >> 2)] = pair_order(xs[m][t]);
          float part = sum8(xs[m][t]);
          part += dpp<0xB1>(part);  // lane ^ 1
          part += dpp<0x4E>(part);  // lane ^ 2
          if ((i & 3) == 0) sx[m * C + (i >> 2)] = part;
        }
      }
    }
  }
  lds_barrier();

  float acc[M];
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m] = 0.0f;
  for (int batch = 0; batch < nb; batch += 2) {
    if (batch + 1 < nb) load_batch(pong, wrow, srow, brow, j, sh, batch + 1, C);
    compute_batch<M, B>(ping, acc, xq, sx, j, sh, batch, C, magic);
    if (batch + 1 < nb) {
      if (batch + 2 < nb) load_batch(ping, wrow, srow, brow, j, sh, batch + 2, C);
      compute_batch<M, B>(pong, acc, xq, sx, j, sh, batch + 1, C, magic);
    }
  }

#pragma unroll
  for (int m = 0; m < M; ++m) {
    float v = row16_sum(acc[m]);
    if (sh >= 5) v = add_xor16(v);
    if (sh >= 6) v = add_xor32(v);
    if (j == 0 && row < N) store_y(a, P, m, row, v);
  }
}

// ---------------------------------------------------- VALU kernel, one activation row
//
// One workgroup per tile of 256/LPR weight rows of one problem; LPR = 1 << lpr_shift
// lanes share a row and lane j takes the 16-byte chunks kc = j, j+LPR, ... (at most NCH,
// nch for this problem).  The lane shape is a per-problem runtime value, so one launch
// serves projections of different K (all seven of a decoder layer, for example).
//
// Every load of the workgroup is issued at the start, in the order it is consumed: x
// (XR 16-byte pieces per thread), the tile's scales and biases (one contiguous span of
// each, read as dwords by consecutive threads), then the weight chunks.  They are raw
// buffer loads issued unconditionally: a piece that is not needed gets an offset past
// its buffer, for which the hardware returns zero without touching memory, so the
// outstanding-load count is the same on every path and each wait is exact.  x goes to
// LDS in pair order with its per-chunk sums, the (scale, bias) pairs as one dword per
// (row, group); then each chunk is consumed as it arrives.

// LDS layout of the one-row kernel, sized by its template so that every staging write
// is unconditional (pieces past the data are written as zeros): x in pair order as four
// planes of XR * 64 chunks, their chunk sums, and 2 * SBR * 256 (scale, bias) dwords.
template <int NCH, int XR, int MR = 1>
struct M1Lds {
  static constexpr int kChunks = XR * 64;                        // per plane, >= K / 32
  static constexpr int kSbr = (64 * NCH + kThreads - 1) / kThreads;  // dwords per thread
  static constexpr size_t kBytes =
      (size_t)MR * kChunks * (64 + 4) + (size_t)kSbr * kThreads * 8;
};

// Activation rows 1 .. MR-1 of a few-row tile (row 0 comes in xp / yp).
struct MoreRows {
  const uint16_t* x[3];
  void* y[3];
};

// One tile of the one-row kernel, its problem's arguments already in scalar registers.
// With MR > 1 the tile serves MR activation rows (xp, more.x -> yp, more.y) from one read
// of the weights; each row's chunk order and sums are those of MR = 1, so each output
// row is the one-row result, bit for bit.
template <int NCH, int XR, int MR = 1>
__device__ __forceinline__ void m1_tile(const uint32_t* wp, const uint16_t* sp, const uint16_t* bp,
                                        const uint16_t* xp, void* yp, int K, int N, int sh,
                                        int nch, int yf32, int row0, const MoreRows& more = {}) {
  static_assert(MR >= 1 && MR <= 4, "one to four activation rows");
  using L = M1Lds<NCH, XR, MR>;
  constexpr int CP = L::kChunks, SBR = L::kSbr;
  extern __shared__ uint4 smem[];
  const int C = K >> 5, G = K >> 6, W = K >> 3;
  const int tid = threadIdx.x;
  const int j = tid & ((1 << sh) - 1);
  const int rl = tid >> sh;  // the lane's row within the tile
  const int row = row0 + rl;
  uint4* xq = smem;                                          // [MR][4][CP]
  float* sx = reinterpret_cast<float*>(smem + MR * 4 * CP);  // [MR][CP]
  uint32_t* sbl = reinterpret_cast<uint32_t*>(sx + MR * CP);  // [rows][G], padded
  const uint32_t magic = in_vgpr(kMagic);

  // x: XR pieces of 8 values per thread and row
  const uint16_t* xps[4] = {xp, more.x[0], more.x[1], more.x[2]};
  uint4 xs[MR][XR];
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    const __amdgpu_buffer_rsrc_t xrsrc = buffer_rsrc(xps[m], (uint32_t)K * 2u);
#pragma unroll
    for (int t = 0; t < XR; ++t) {
      const int i = tid + kThreads * t;
      xs[m][t] = load_b128(xrsrc, i < W ? 16u * i : kPastBuffer);
    }
  }
  // the tile's scales and biases: rows * G halves from row0 * G on, as dwords (rows is
  // even, so the span starts 4-byte aligned); rows past N read as zero.  The range is
  // rounded up to whole dwords (an odd N * G ends mid-dword, and a dword that crosses the
  // range would read as zero); the extra half lies in the same aligned dword as the last
  // one, so it is mapped, and it belongs to no row.
  const int D = ((kThreads >> sh) * G) >> 1;
  const uint32_t sb_bytes = ((uint32_t)N * (uint32_t)G * 2u + 3u) & ~3u;
  const __amdgpu_buffer_rsrc_t srsrc = buffer_rsrc(sp, sb_bytes);
  const __amdgpu_buffer_rsrc_t brsrc = buffer_rsrc(bp, sb_bytes);
  const uint32_t sb0 = (uint32_t)row0 * (uint32_t)G * 2u;
  uint32_t sv[SBR], bv[SBR];
#pragma unroll
  for (int q = 0; q < SBR; ++q) {
    const int d = tid + kThreads * q;
    const uint32_t off = d < D ? sb0 + 4u * d : kPastBuffer;
    sv[q] = __builtin_amdgcn_raw_buffer_load_b32(srsrc, off, 0, 0);
    bv[q] = __builtin_amdgcn_raw_buffer_load_b32(brsrc, off, 0, 0);
  }
  // the weight chunks (rows past N read as zero and are never stored)
  const __amdgpu_buffer_rsrc_t wrsrc = buffer_rsrc(wp, (uint32_t)N * (uint32_t)W * 4u);
  const uint32_t wrow = (uint32_t)row * (uint32_t)W * 4u;
  uint4 wv[NCH];
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int kc = j + (i << sh);
    wv[i] = load_b128_nt(wrsrc, (i < nch && kc < C && row < N) ? wrow + 16u * kc : kPastBuffer);
  }

  // staging, unconditionally (pieces past x and past the span are zeros)
#pragma unroll
  for (int m = 0; m < MR; ++m) {
#pragma unroll
    for (int t = 0; t < XR; ++t) {
      const int i = tid + kThreads * t;  // the four words of a chunk are four aligned lanes
      xq[(m * 4 + (i & 3)) * CP + (i >> 2)] = pair_order(xs[m][t]);
      float part = sum8(xs[m][t]);
      part += dpp<0xB1>(part);  // lane ^ 1
      part += dpp<0x4E>(part);  // lane ^ 2
      if ((i & 3) == 0) sx[m * CP + (i >> 2)] = part;
    }
  }
#pragma unroll
  for (int q = 0; q < SBR; ++q) {
    const int d = tid + kThreads * q;
    *reinterpret_cast<uint2*>(sbl + 2 * d) =
        make_uint2((sv[q] & 0xffffu) | (bv[q] << 16), (sv[q] >> 16) | (bv[q] & 0xffff0000u));
  }
  lds_barrier();

  float acc[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) acc[m] = 0.0f;
  const uint32_t* sbr = sbl + rl * G;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    if (i < nch) {  // uniform over the workgroup's problem
      const int kc = j + (i << sh);
      const bool valid = kc < C;
      const int kk = valid ? kc : 0;
      const uint32_t sb = sbr[kk >> 1];
      const float sc = __uint_as_float(sb << 16);
      const float bi = __uint_as_float(sb & 0xffff0000u);
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        const uint4* xm = xq + m * 4 * CP;
        const float sxm = sx[m * CP + kk];
        const float d = chunk_dot(wv[i], xm[kk], xm[CP + kk], xm[2 * CP + kk], xm[3 * CP + kk],
                                  -128.0f * sxm, magic);
        const float v = fmaf(sc, d, fmaf(bi, sxm, acc[m]));
        acc[m] = valid ? v : acc[m];
      }
    }
  }
  void* yps[4] = {yp, more.y[0], more.y[1], more.y[2]};
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    float v = row16_sum(acc[m]);
    if (sh >= 5) v = add_xor16(v);
    if (sh >= 6) v = add_xor32(v);
    if (j == 0 && row < N) {
      if (yf32)
        static_cast<float*>(yps[m])[row] = v;
      else
        static_cast<uint16_t*>(yps[m])[row] = f32_to_bf16_bits(v);
    }
  }
}

// MR = 2..4 activation rows: blockIdx.y is the problem, blockIdx.x its tile.
template <int NCH, int XR, int MR>
__global__ __launch_bounds__(kThreads) void qmv_mr_kernel(LaunchArgs a) {
  const Problem& P = a.p[blockIdx.y];
  const int K = P.K, N = P.N, sh = P.lpr_shift, nch = P.nch, yf32 = a.y_f32;
  const int row0 = blockIdx.x * (kThreads >> sh);
  if (row0 >= N) return;  // past this problem's tiles
  const size_t ybytes = yf32 ? 4 : 2;
  MoreRows more = {};
#pragma unroll
  for (int m = 1; m < MR; ++m) {
    more.x[m - 1] = x_row(a, P, m);
    more.y[m - 1] = a.table ? a.yt[m] : static_cast<char*>(P.y) + (size_t)m * P.ldy * ybytes;
  }
  m1_tile<NCH, XR, MR>(P.w, P.s, P.b, x_row(a, P, 0), a.table ? a.yt[0] : P.y, K, N, sh, nch,
                       yf32, row0, more);
}

// Any number of problems: blockIdx.y is the problem, blockIdx.x its tile.
template <int NCH, int XR>
__global__ __launch_bounds__(kThreads) void qmv_m1_kernel(LaunchArgs a) {
  const Problem& P = a.p[blockIdx.y];
  const uint32_t* wp = P.w;
  const uint16_t* sp = P.s;
  const uint16_t* bp = P.b;
  const uint16_t *x0 = P.x, *x1 = a.xt[0];
  void *y0 = P.y, *y1 = a.yt[0];
  const int K = P.K, N = P.N, sh = P.lpr_shift, nch = P.nch, yf32 = a.y_f32, table = a.table;
  // every argument in one round trip: without this the exit test below would fetch N
  // and the lane shape first, and the rest only after that answer arrived
  asm volatile("" ::"s"(wp), "s"(sp), "s"(bp), "s"(x0), "s"(x1), "s"(y0), "s"(y1), "s"(K),
               "s"(N), "s"(sh), "s"(nch), "s"(yf32), "s"(table));
  const int row0 = blockIdx.x * (kThreads >> sh);
  if (row0 >= N) return;  // past this problem's tiles
  m1_tile<NCH, XR>(wp, sp, bp, table ? x1 : x0, table ? y1 : y0, K, N, sh, nch, yf32, row0);
}

// Up to kM1Compact problems on a linear grid with no idle workgroups: all their
// arguments arrive in the first round trip and the workgroup picks its problem with
// scalar selects (an indexed read would cost a second, dependent round trip).
constexpr int kM1Compact = 4;

struct M1Args {
  int32_t count;
  int32_t y_f32;
  int32_t pad[2];
  int32_t tile_end[kM1Compact];  // one past the last workgroup of each problem
  int32_t N[kM1Compact];
  int32_t K[kM1Compact];
  int32_t sh[kM1Compact];
  int32_t nch[kM1Compact];
  const uint32_t* w[kM1Compact];
  const uint16_t* s[kM1Compact];
  const uint16_t* b[kM1Compact];
  const uint16_t* x[kM1Compact];
  void* y[kM1Compact];
};

template <typename T>
__device__ __forceinline__ T pick4(int i, T v0, T v1, T v2, T v3) {
  return i == 0 ? v0 : i == 1 ? v1 : i == 2 ? v2 : v3;
}

template <int NCH, int XR>
__global__ __launch_bounds__(kThreads) void qmv_m1c_kernel(M1Args a) {
  asm volatile("" ::"s"(a.count), "s"(a.y_f32), "s"(a.tile_end[0]), "s"(a.tile_end[1]),
               "s"(a.tile_end[2]), "s"(a.N[0]), "s"(a.N[1]), "s"(a.N[2]), "s"(a.N[3]),
               "s"(a.K[0]), "s"(a.K[1]), "s"(a.K[2]), "s"(a.K[3]), "s"(a.sh[0]), "s"(a.sh[1]),
               "s"(a.sh[2]), "s"(a.sh[3]), "s"(a.nch[0]), "s"(a.nch[1]), "s"(a.nch[2]),
               "s"(a.nch[3]));
  asm volatile("" ::"s"(a.w[0]), "s"(a.w[1]), "s"(a.w[2]), "s"(a.w[3]), "s"(a.s[0]), "s"(a.s[1]),
               "s"(a.s[2]), "s"(a.s[3]), "s"(a.b[0]), "s"(a.b[1]), "s"(a.b[2]), "s"(a.b[3]));
  asm volatile("" ::"s"(a.x[0]), "s"(a.x[1]), "s"(a.x[2]), "s"(a.x[3]), "s"(a.y[0]), "s"(a.y[1]),
               "s"(a.y[2]), "s"(a.y[3]));
  const int bx = blockIdx.x;
  const int pi = (a.count > 1 && bx >= a.tile_end[0]) + (a.count > 2 && bx >= a.tile_end[1]) +
                 (a.count > 3 && bx >= a.tile_end[2]);
  const int first = pick4(pi, 0, a.tile_end[0], a.tile_end[1], a.tile_end[2]);
  const int sh = pick4(pi, a.sh[0], a.sh[1], a.sh[2], a.sh[3]);
  m1_tile<NCH, XR>(pick4(pi, a.w[0], a.w[1], a.w[2], a.w[3]),
                   pick4(pi, a.s[0], a.s[1], a.s[2], a.s[3]),
                   pick4(pi, a.b[0], a.b[1], a.b[2], a.b[3]),
                   pick4(pi, a.x[0], a.x[1], a.x[2], a.x[3]),
                   pick4(pi, a.y[0], a.y[1], a.y[2], a.y[3]),
                   pick4(pi, a.K[0], a.K[1], a.K[2], a.K[3]),
                   pick4(pi, a.N[0], a.N[1], a.N[2], a.N[3]), sh,
                   pick4(pi, a.nch[0], a.nch[1], a.nch[2], a.nch[3]), a.y_f32,
                   (bx - first) * (kThreads >> sh));
}

// ---------------------------------------------------- MoE gather (one row per pair)
//
// Pair p of a gather call computes y[p] = W[idx[p]] x[p / xs] with the one-row tile above
// (the same lane shape, chunk order and sums, so each pair's row equals imq_qmv on that
// expert's weights, bit for bit).  blockIdx.y is the pair and blockIdx.x its tile; the
// expert index is read once per workgroup from device memory.  An index outside
// [0, experts) gives a row of zeros.

struct GatherArgs {
  const uint32_t* w;  // (E, N, K/8)
  const uint16_t* s;  // (E, N, K/64)
  const uint16_t* b;
  const uint16_t* x;  // row p / xs at x + (p / xs) * ldx
  void* y;            // row p at y + p * ldy elements
  const uint32_t* idx;
  int64_t ldx, ldy;
  int64_t w_stride, sb_stride;  // words / halves per expert
  int32_t E, N, K, xs, sh, nch, y_f32, pad;
};

template <int NCH, int XR>
__global__ __launch_bounds__(kThreads) void qmv_gather_kernel(GatherArgs a) {
  const int pair = blockIdx.y;
  const int row0 = blockIdx.x * (kThreads >> a.sh);
  if (row0 >= a.N) return;
  const uint32_t ex = __builtin_amdgcn_readfirstlane(a.idx[pair]);
  void* yp = a.y_f32 ? static_cast<void*>(static_cast<float*>(a.y) + (int64_t)pair * a.ldy)
                     : static_cast<void*>(static_cast<uint16_t*>(a.y) + (int64_t)pair * a.ldy);
  if (ex >= (uint32_t)a.E) {
    const int row = row0 + (int)(threadIdx.x >> a.sh);
    if ((threadIdx.x & ((1 << a.sh) - 1)) == 0 && row < a.N) {
      if (a.y_f32)
        static_cast<float*>(yp)[row] = 0.0f;
      else
        static_cast<uint16_t*>(yp)[row] = 0;
    }
    return;
  }
  m1_tile<NCH, XR>(a.w + (int64_t)ex * a.w_stride, a.s + (int64_t)ex * a.sb_stride,
                   a.b + (int64_t)ex * a.sb_stride, a.x + (int64_t)(pair / a.xs) * a.ldx, yp,
                   a.K, a.N, a.sh, a.nch, a.y_f32, row0);
}

// ------------------------------------------------------- MFMA operand helpers

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) {
  u32x4_t t = {v.x, v.y, v.z, v.w};
  return __builtin_bit_cast(bf16x8_t, t);
}

// The MFMA kernels' weight operand.  Word u's nibble pair (p, p + 4) as the bf16 pair
// (1 + q_p/16, 1 + q_{p+4}/16), exact: with s v x summed for v = 1 + q/16, a group's
// sum (s q + b) x = 16 s sum v x + (b - 16 s) sum x, and the fp32 sum of v x carries
// terms within 2x of |x|, so its rounding stays near that of the direct sum (a 128 + q
// operand would carry terms 128x larger into the same fp32 accumulator).
// `one` must be in_vgpr(kNibOne).
constexpr uint32_t kNibOne = 0x3f803f80u;   // bf16 pair (1.0, 1.0)
constexpr uint32_t kNibMask = 0x00780078u;  // mantissa bits 3..6 of each half
template <int P>
__device__ __forceinline__ uint32_t nib16(uint32_t u, uint32_t one) {
  uint32_t t;
  if constexpr (P == 0)
    t = u << 3;
  else
    t = u >> (4 * P - 3);
  return (t & kNibMask) | one;
}

__device__ __forceinline__ bf16x8_t unpack16(uint32_t u, uint32_t one) {
  u32x4_t t = {nib16<0>(u, one), nib16<1>(u, one), nib16<2>(u, one), nib16<3>(u, one)};
  return __builtin_bit_cast(bf16x8_t, t);
}

// ------------------------------------------------ MFMA kernel, 32 x 32 tiles (M >= 3)
//
// A wavefront computes a 32 (activation rows) x 32 (weight rows) tile of y over its share
// of the groups with v_mfma_f32_32x32x16_bf16, x as the A operand and the weights as the
// B operand.  For a group of 64 values, lane (r = lane % 32, h = lane / 32) holds
//   * 16 bytes of weight row r, words 4h .. 4h+3: word 4h+s (as unpack16 bf16 pairs)
//     is the lane's B operand of k-step s;
//   * 64 bytes of activation row r, x[32h .. 32h+32): its piece s in pair order is the
//     lane's A operand of k-step s.
// So both operands come from one contiguous load each.  The output lane (n = lane % 32,
// h) holds rows m = 8(i/4) + 4h + i%4 (i < 16) of column n, so a lane's scale and bias are
// scalars.  Per group
//     acc += 16 s * P + (b - 16 s) * P1,
// P1 being the four k-steps against a ones operand (the row sums of x over the group).
// Rows m >= M read row M-1 and are never stored.
//
// A workgroup's four wavefronts split its groups in quarters and add through LDS in a
// fixed order.  A weight's groups may also be split over SPLITS workgroups (more
// workgroups when N is small): each split writes an fp32 partial of its tile, and the
// last split of the tile to finish (a counter per tile, in the caller's workspace) adds
// the partials in split order and writes y, then returns the counter to zero.  One
// launch, and the same bits whatever order the splits finish in.  Partials and counters
// go through sc1 accesses (coherent across the XCDs' L2 caches): every thread waits for
// its partial stores before the workgroup's one atomic add, and the last split reads the
// partials with sc1 loads, so no cache write-back or invalidate is needed.  Loads are
// issued a stage of MS groups ahead, unconditionally (past the range: offsets past the
// buffer, zero, no traffic).

typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kMmaStage = 1;
constexpr int kMaxSplits = 16;  // partials the last split of a tile adds

// One stage: GS groups of NT weight tiles (32 rows each), the matching x pieces and the
// tiles' scales and biases.
template <int NT, int GS>
struct MmaStage {
  uint4 w[GS][NT];
  uint4 x[GS][4];
  uint32_t s[GS][NT], b[GS][NT];
};

template <int NT, int GS>
__device__ __forceinline__ void mma_load(MmaStage<NT, GS>& st, __amdgpu_buffer_rsrc_t wrsrc,
                                         __amdgpu_buffer_rsrc_t srsrc, __amdgpu_buffer_rsrc_t brsrc,
                                         const uint32_t (&woff)[NT], const uint32_t (&sboff)[NT],
                                         const uint16_t* xr, int g, int g1) {
#pragma unroll
  for (int i = 0; i < GS; ++i) {
    const bool in = g + i < g1;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      st.w[i][t] = load_b128_nt(wrsrc, in ? woff[t] + 32u * (g + i) : kPastBuffer);
      st.s[i][t] = __builtin_amdgcn_raw_buffer_load_b16(srsrc, in ? sboff[t] + 2u * (g + i) : kPastBuffer, 0, 0);
      st.b[i][t] = __builtin_amdgcn_raw_buffer_load_b16(brsrc, in ? sboff[t] + 2u * (g + i) : kPastBuffer, 0, 0);
    }
  }
#pragma unroll
  for (int i = 0; i < GS; ++i) {
    const int gg = g + i < g1 ? g + i : g1 - 1;  // x rows end at K: stay inside them
    const uint4* xv = reinterpret_cast<const uint4*>(xr + 64 * gg);
#pragma unroll
    for (int q = 0; q < 4; ++q) st.x[i][q] = xv[q];
  }
}

template <int NT, int GS>
__device__ __forceinline__ void mma_compute(const MmaStage<NT, GS>& st, int g, int g1,
                                            f32x16_t (&acc)[NT], uint32_t one) {
  const u32x4_t ones_u = {kOnes, kOnes, kOnes, kOnes};
  const bf16x8_t ones = __builtin_bit_cast(bf16x8_t, ones_u);
  const f32x16_t zero = {};
#pragma unroll
  for (int i = 0; i < GS; ++i) {
    if (g + i >= g1) break;
    bf16x8_t a[4];
    f32x16_t p1 = zero;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      a[s] = as_bf16x8(pair_order(st.x[i][s]));
      p1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[s], ones, p1, 0, 0, 0);
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const uint32_t wd[4] = {st.w[i][t].x, st.w[i][t].y, st.w[i][t].z, st.w[i][t].w};
      f32x16_t p = zero;
#pragma unroll
      for (int s = 0; s < 4; ++s)
        p = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[s], unpack16(wd[s], one), p, 0, 0, 0);
      const float sc = bf16_bits_to_f32(st.s[i][t]);
      const float c = fmaf(-16.0f, sc, bf16_bits_to_f32(st.b[i][t]));
      const float s16 = 16.0f * sc;
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[t][e] = fmaf(s16, p[e], fmaf(c, p1[e], acc[t][e]));
    }
  }
}

// The end of a workgroup's tile: acc[t] (in the wavefronts with `holder`) covers rows
// nbase + 32 t + r of y, the workgroup's tile rows [row0, row0 + cols).  Without splits the
// holders store y.  With splits each split stores its fp32 partial, and the last split of
// the tile to arrive (the tile's counter in the workspace) adds the partials in split order,
// writes y and returns the counter to zero.  Every thread waits for its partial stores
// before the workgroup's one atomic add; partials and counters use sc1 accesses.
template <int NT, bool PARTIAL, int MAXS = kMaxSplits>
__device__ __forceinline__ void finish_tiles(const LaunchArgs& a, const Problem& P, int pi,
                                             int split, int splits, float* partial,
                                             int64_t pstride, uint32_t* counters, int tiles_max,
                                             const f32x16_t (&acc)[NT], bool holder, int nbase,
                                             int row0, int cols, int* last) {
  const int N = P.N, M = a.M, tid = threadIdx.x, lane = tid & 63;
  const int r = lane & 31, h = lane >> 5;
  if (!PARTIAL) {
    if (!holder) return;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int n = nbase + 32 * t + r;
      if (n >= N) continue;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int m = 8 * (e >> 2) + 4 * h + (e & 3);
        if (m < M) store_y(a, P, m, n, acc[t][e]);
      }
    }
    return;
  }
  const __amdgpu_buffer_rsrc_t prs =
      buffer_rsrc(partial + pi * pstride, (uint32_t)((int64_t)splits * M * N * 4));
  if (holder) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int n = nbase + 32 * t + r;
      if (n >= N) continue;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int m = 8 * (e >> 2) + 4 * h + (e & 3);
        if (m < M)
          store_b32_sc1(prs, (uint32_t)(((split * M + m) * N + n) * 4), __float_as_uint(acc[t][e]));
      }
    }
  }
  wait_vmem();
  __syncthreads();
  uint32_t* cnt = counters + (int64_t)pi * tiles_max + blockIdx.x;
  if (tid == 0)
    *last = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
            (uint32_t)(splits - 1);
  __syncthreads();
  if (!*last) return;
  // the last split: every thread's partials loaded at once (at most MAXS per output), then
  // added in split order
  const uint32_t step = (uint32_t)(M * N * 4);
  for (int i = tid; i < M * cols; i += kThreads) {
    const int m = i / cols, n = row0 + i % cols;
    const bool in = n < N;
    const uint32_t o = (uint32_t)((m * N + n) * 4);
    float t[MAXS];
#pragma unroll
    for (int q = 0; q < MAXS; ++q)
      t[q] = __uint_as_float(load_b32_sc1(prs, in && q < splits ? o + q * step : kPastBuffer));
    float v = 0.0f;
#pragma unroll
    for (int q = 0; q < MAXS; ++q)
      if (q < splits) v += t[q];
    if (in) store_y(a, P, m, n, v);
  }
  if (tid == 0) st_sc1(cnt, 0u);  // ready for the next call
}

// NT weight tiles of 32 rows per wavefront (x, its pair order and the row sums shared by
// them), four wavefronts splitting the groups of a workgroup's 32 * NT rows.
template <int NT, bool PARTIAL>
__global__ __launch_bounds__(kThreads) void qmv_mma_kernel(LaunchArgs a, int splits,
                                                           float* __restrict__ partial,
                                                           int64_t pstride,
                                                           uint32_t* __restrict__ counters,
                                                           int tiles_max) {
  __shared__ f32x16_t red[3][NT][64];
  const int pi = blockIdx.y / splits, split = blockIdx.y - pi * splits;
  const Problem& P = a.p[pi];
  const int K = P.K, N = P.N, M = a.M;
  const int row0 = blockIdx.x * 32 * NT;
  if (row0 >= N) return;  // past this problem's tiles
  const int G = K >> 6, W = K >> 3;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int r = lane & 31, h = lane >> 5;
  const uint32_t one = in_vgpr(kNibOne);

  // this workgroup's groups, and this wavefront's quarter of them
  const int gs0 = (G * split) / splits, gs1 = (G * (split + 1)) / splits;
  const int g0 = gs0 + ((gs1 - gs0) * wave >> 2), g1 = gs0 + ((gs1 - gs0) * (wave + 1) >> 2);

  const __amdgpu_buffer_rsrc_t wrsrc = buffer_rsrc(P.w, (uint32_t)N * (uint32_t)W * 4u);
  const uint32_t sb_bytes = (uint32_t)N * (uint32_t)G * 2u;
  const __amdgpu_buffer_rsrc_t srsrc = buffer_rsrc(P.s, sb_bytes);
  const __amdgpu_buffer_rsrc_t brsrc = buffer_rsrc(P.b, sb_bytes);
  uint32_t woff[NT], sboff[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int row = row0 + 32 * t + r < N ? row0 + 32 * t + r : N - 1;
    woff[t] = (uint32_t)row * (uint32_t)W * 4u + 16u * h;
    sboff[t] = (uint32_t)row * (uint32_t)G * 2u;
  }
  const uint16_t* xr = x_row(a, P, r < M ? r : M - 1) + 32 * h;

  f32x16_t acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = f32x16_t{};
  MmaStage<NT, kMmaStage> sa, sb;
  mma_load<NT, kMmaStage>(sa, wrsrc, srsrc, brsrc, woff, sboff, xr, g0, g1 > g0 ? g1 : g0 + 1);
  for (int g = g0; g < g1; g += 2 * kMmaStage) {
    mma_load<NT, kMmaStage>(sb, wrsrc, srsrc, brsrc, woff, sboff, xr, g + kMmaStage, g1);
    mma_compute<NT, kMmaStage>(sa, g, g1, acc, one);
    if (g + kMmaStage >= g1) break;
    mma_load<NT, kMmaStage>(sa, wrsrc, srsrc, brsrc, woff, sboff, xr, g + 2 * kMmaStage, g1);
    mma_compute<NT, kMmaStage>(sb, g + kMmaStage, g1, acc, one);
  }

  // add the four quarters in order: waves 1..3 park theirs, wave 0 adds
  if (wave > 0)
#pragma unroll
    for (int t = 0; t < NT; ++t) red[wave - 1][t][lane] = acc[t];
  __syncthreads();
  if (wave == 0)
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int q = 0; q < 3; ++q) acc[t] += red[q][t][lane];
  __shared__ int last;
  finish_tiles<NT, PARTIAL>(a, P, pi, split, splits, partial, pstride, counters, tiles_max, acc,
                            wave == 0, row0, row0, 32 * NT, &last);
}

// ------------------------------ MFMA kernel, weights and x staged through LDS (M >= 3)
//
// The same 32 x 32 MFMA tiles and per-group arithmetic as qmv_mma_kernel, fed from LDS.  A
// load instruction of qmv_mma_kernel's layout touches 32 rows for 32 bytes each; here
// every global load reads whole 128-byte lines, and the MFMA layout is read back from LDS.
//
// Workgroup: 64 weight rows (two wavefronts along N, one 32-row tile each) times two
// K-ranges (two wavefronts along K), so the two N-wavefronts of a K-range share its x.  A
// stage is 4 groups (256 values of k) of both K-ranges:
//   * weights: 2 x 64 rows x 128 B (one line per row), 144-byte LDS rows;
//   * x: 2 x 32 rows x 512 B, stored in pair order, 528-byte LDS rows;
//   * scales and biases: 2 x 64 rows x 8 B each.
// (The row paddings make the MFMA-layout reads conflict-free.)  A stage's loads are issued
// into registers ahead of it (x one stage ahead, weights, scales and biases two) and
// written to LDS after the previous stage is computed, one barrier on each side.  Rows
// m >= M read row M-1 and are never stored; groups past a
// K-range read zero (buffer offsets past the end).  The bias term is one fp32 MFMA
// (v_mfma_f32_32x32x2_f32) per pair of groups: A = the two groups' row sums of x, B = the
// two groups' c = b - 16 s per weight row; the weights enter the MFMAs as 1 + q/16.
// Requires K % 256 == 0 and x rows at x + m * ldx (no row-pointer table).
#ifndef IMQ_STAGED_DEPTH
#define IMQ_STAGED_DEPTH 2
#endif
namespace staged {
constexpr int kMaxPairParts = 4;  // K-parts of a gate/up tile of the last round
constexpr int kWN = 2, kWK = 2;                   // wavefronts along N and along K
constexpr int kRows = 32 * kWN;                   // weight rows per workgroup
constexpr int kWRow = 144, kXRow = 528;           // LDS row strides (bytes)
constexpr int kWBytes = kWK * kRows * kWRow;      // weights of a stage
constexpr int kXBytes = kWK * 32 * kXRow;         // x of a stage
constexpr int kSBBytes = kWK * kRows * 16;        // scales (8 B) and biases (8 B) per row
constexpr int kStage = kWBytes + kXBytes + kSBBytes;
constexpr int kWP = kWK * kRows * 8 / kThreads;   // 16-byte weight pieces per thread
constexpr int kXP = kWK * 32 * 32 / kThreads;     // 16-byte x pieces per thread
constexpr int kXPK = kXP / kWK;                   // ... per K-range
constexpr int kMaxSplitsStaged = 8;
static_assert(kWK * kRows * 2 == kThreads, "one scale or bias piece per thread");
static_assert(kStage >= kWN * 64 * 64, "the K-range reduction reuses the stage");
}  // namespace staged

// PAIR: the gate/up form.  p[0] is the gate weight, p[1] the up weight (same x, N and K);
// workgroup i computes gate rows [32 i, 32 i + 32) on its N-wavefront 0 and the same up rows
// on N-wavefront 1, and writes act[m][n] = bf16(silu(bf16(gate)) * bf16(up)) to p[0].y
// (row stride p[0].ldy): silu_mul_kernel's expression on the values the grouped launch
// and its bf16 outputs would give, bit for bit (the rows' sums run the same way).
template <bool PARTIAL, bool PAIR = false>
__global__ __launch_bounds__(kThreads) void qmv_mma_staged_kernel(LaunchArgs a, int splits,
                                                                  float* __restrict__ partial,
                                                                  int64_t pstride,
                                                                  uint32_t* __restrict__ counters,
                                                                  int tiles_max, NormIn ni) {
  using namespace staged;
  __shared__ __attribute__((aligned(16))) char lds[kStage];
  __shared__ float nsum[PAIR ? kNormMaxTiles / 4 : 1][32];  // input norm: pair sums [j][row]
  __shared__ float ninv[32];                                // input norm: 1/rms per row
  __shared__ int last;
  // PAIR: the first `tiles_max` workgroups take whole tiles; with `splits` > 1 every later
  // tile (the launch's last, partial round over the CUs) is cut into `splits` K-parts, one
  // workgroup each, whose last part to finish adds them (the launch then ends after about
  // one tile per CU instead of two on some); `partial` and `counters` hold the parts
  int tile_p = blockIdx.x, part = 0, parts = 1;
  if (PAIR && splits > 1 && (int)blockIdx.x >= tiles_max) {
    const int q = blockIdx.x - tiles_max;
    tile_p = tiles_max + q / splits;
    part = q - (q / splits) * splits;
    parts = splits;
  }
  const int pi = PAIR ? 0 : blockIdx.y / splits;
  const int split = PAIR ? part : blockIdx.y - pi * splits;
  const int nsplit = PAIR ? parts : splits;
  const Problem& P = a.p[pi];
  const int K = P.K, N = P.N, M = a.M;
  // a tile's row slot r (0..63) is weight row row0 + r, or (PAIR) row rp0 + r % 32 of the
  // gate (r < 32) or up (r >= 32) weight
  const int row0 = PAIR ? 0 : blockIdx.x * kRows;
  const int rp0 = tile_p * 32;
  if ((PAIR ? rp0 : row0) >= N) return;  // past this problem's tiles
  const int G = K >> 6, W = K >> 3;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int wn = wave % kWN, wk = wave / kWN;
  const int r = lane & 31, h = lane >> 5;
  const uint32_t one = in_vgpr(kNibOne);

  // the split's groups (whole stages), then the two K-ranges of whole stages
  const int gs0 = (G * split) / nsplit / 4 * 4;
  const int gs1 = split + 1 == nsplit ? G : (G * (split + 1)) / nsplit / 4 * 4;
  const int span = ((gs1 - gs0 + kWK - 1) / kWK + 3) / 4 * 4;
  const int nst = span / 4;
  int klo[kWK], khi[kWK];
#pragma unroll
  for (int k = 0; k < kWK; ++k) {
    klo[k] = gs0 + k * span;
    khi[k] = klo[k] + span < gs1 ? klo[k] + span : gs1;
  }

  const __amdgpu_buffer_rsrc_t wrsrc = buffer_rsrc(P.w, (uint32_t)N * (uint32_t)W * 4u);
  const uint32_t sb_bytes = (uint32_t)N * (uint32_t)G * 2u;
  const __amdgpu_buffer_rsrc_t srsrc = buffer_rsrc(P.s, sb_bytes);
  const __amdgpu_buffer_rsrc_t brsrc = buffer_rsrc(P.b, sb_bytes);
  const Problem& Pu = a.p[PAIR ? 1 : 0];
  const __amdgpu_buffer_rsrc_t wrsrc_u = buffer_rsrc(Pu.w, (uint32_t)N * (uint32_t)W * 4u);
  const __amdgpu_buffer_rsrc_t srsrc_u = buffer_rsrc(Pu.s, sb_bytes);
  const __amdgpu_buffer_rsrc_t brsrc_u = buffer_rsrc(Pu.b, sb_bytes);
  const __amdgpu_buffer_rsrc_t xrsrc =
      buffer_rsrc(P.x, (uint32_t)((M - 1) * P.ldx * 2 + K * 2));
  auto slot_row = [&](int r) {  // weight row of tile slot r, clamped to the weight
    const int n = PAIR ? rp0 + (r & 31) : row0 + r;
    return n < N ? n : N - 1;
  };

  // Staging.  x piece i of a thread: K-range i / kXPK, row (tid >> 5) + 8 (i % kXPK), piece
  // tid & 31 of the row's 512 bytes.  Weight piece i: row slot (tid >> 3) + 32 i (row =
  // slot % kRows, K-range slot / kRows), piece tid & 7 of the row's 128 bytes.  Scale or
  // bias piece: threads [0, 128) scales, [128, 256) biases (uniform per wavefront), K-range
  // and row from tid % 128.
  const int xp = tid & 31, wp = tid & 7;
  const uint32_t ldx2 = (uint32_t)P.ldx * 2u;
  const uint32_t xdst0 = (uint32_t)(kWBytes + (tid >> 5) * kXRow + 16 * xp);
  const uint32_t wdst0 = (uint32_t)((tid >> 3) * kWRow + 16 * wp);
  const int sb_is_b = __builtin_amdgcn_readfirstlane(tid / (kWK * kRows));
  const int sb_rem = tid % (kWK * kRows), sb_k = sb_rem / kRows;
  const int sb_n = slot_row(sb_rem % kRows);
  const bool sb_up = PAIR && sb_rem % kRows >= 32;  // per lane: the up weight's row
  const uint32_t sb_src = (uint32_t)sb_n * (uint32_t)G * 2u;
  const uint32_t sb_dst = (uint32_t)(kWBytes + kXBytes + sb_rem * 16 + 8 * sb_is_b);

  // A stage's loads in registers: x one stage ahead (from L2), the weights, scales and
  // biases IMQ_STAGED_DEPTH stages ahead (from HBM) in DEPTH register sets.  Each stage
  // issues the next x before the weights DEPTH ahead: loads return in issue order, so the
  // wait for the next stage's x never waits for those weights.
  struct WRegs {
    uint4 w[kWP];
    u32x2_t sb;
  };
  // Each piece's offset at stage 0 is computed once; stage st adds its bytes as the loads'
  // scalar offset, and a piece whose group lies past its K-range gets the past-the-buffer
  // bit (the groups of a stage past the range are the same for every piece of a K-range
  // with the same group slot, so one compare per slot and stage).
  uint32_t xoff[kXP], woff[kWP];
#pragma unroll
  for (int i = 0; i < kXP; ++i) {
    const int k = i / kXPK, m = (tid >> 5) + 8 * (i % kXPK);
    xoff[i] = (uint32_t)(m < M ? m : M - 1) * ldx2 + 16u * (xp & 7) + 128u * (uint32_t)(klo[k] + (xp >> 3));
  }
#pragma unroll
  for (int i = 0; i < kWP; ++i) {
    const int slot = (tid >> 3) + 32 * i, k = slot / kRows;
    woff[i] = (uint32_t)slot_row(slot % kRows) * (uint32_t)W * 4u + 16u * (wp & 1) +
              32u * (uint32_t)(klo[k] + (wp >> 1));
  }
  uint4 xreg[kXP];
  auto fetch_x = [&](int st) {
    uint32_t past[kWK];
#pragma unroll
    for (int k = 0; k < kWK; ++k) past[k] = (xp >> 3) >= khi[k] - klo[k] - 4 * st ? kPastBuffer : 0u;
#pragma unroll
    for (int i = 0; i < kXP; ++i) {
      const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(xrsrc, xoff[i] | past[i / kXPK], 512 * st, 0);
      xreg[i] = make_uint4(v.x, v.y, v.z, v.w);
    }
  };
  auto fetch_w = [&](WRegs& R, int st) {
    uint32_t past[kWK];
#pragma unroll
    for (int k = 0; k < kWK; ++k) past[k] = (wp >> 1) >= khi[k] - klo[k] - 4 * st ? kPastBuffer : 0u;
#pragma unroll
    for (int i = 0; i < kWP; ++i) {
      const int k = ((tid >> 3) + 32 * i) / kRows;
      // slot % kRows < 32 exactly for even i: the weight is uniform per instruction
      const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(PAIR && (i & 1) ? wrsrc_u : wrsrc,
                                                              woff[i] | past[k], 128 * st, kNt);
      R.w[i] = make_uint4(v.x, v.y, v.z, v.w);
    }
    const int g = klo[sb_k] + 4 * st;
    const uint32_t off = (sb_src + 2u * (uint32_t)g) | ((uint32_t)(g >= khi[sb_k]) << 31);
    if (PAIR) {  // gate and up rows share the wavefront: each lane reads from one of them
      const u32x2_t sg = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(
          sb_is_b ? brsrc : srsrc, sb_up ? kPastBuffer : off, 0, 0));
      const u32x2_t su = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(
          sb_is_b ? brsrc_u : srsrc_u, sb_up ? off : kPastBuffer, 0, 0));
      R.sb = u32x2_t{sg[0] | su[0], sg[1] | su[1]};
    } else {
      R.sb = __builtin_bit_cast(u32x2_t,
                                 __builtin_amdgcn_raw_buffer_load_b64(sb_is_b ? brsrc : srsrc, off, 0, 0));
    }
  };
  auto store = [&](const WRegs& R) {
#pragma unroll
    for (int i = 0; i < kXP; ++i)
      *reinterpret_cast<uint4*>(lds + xdst0 + (i / kXPK) * 32 * kXRow + 8 * (i % kXPK) * kXRow) =
          pair_order(xreg[i]);
#pragma unroll
    for (int i = 0; i < kWP; ++i) *reinterpret_cast<uint4*>(lds + wdst0 + 32 * i * kWRow) = R.w[i];
    *reinterpret_cast<u32x2_t*>(lds + sb_dst) = R.sb;
  };

  f32x16_t acc = {}, accb = {};
  const u32x4_t ones_u = {kOnes, kOnes, kOnes, kOnes};
  const bf16x8_t ones = __builtin_bit_cast(bf16x8_t, ones_u);
  const f32x16_t zero = {};
  const int wrow = 32 * wn + r;  // this lane's weight row in the workgroup
  const uint32_t xrd = (uint32_t)(kWBytes + wk * 32 * kXRow + r * kXRow + 64 * h);
  const uint32_t wrd = (uint32_t)(wk * kRows * kWRow + wrow * kWRow + 16 * h);
  const uint32_t sbrd = (uint32_t)(kWBytes + kXBytes + (wk * kRows + wrow) * 16);

  // the input norm's partial sums (gate/up form): two b128 per thread cover 32 rows x
  // kNormMaxTiles partials; their sums are published by the stage loop's barriers
  const bool norm_in = PAIR && ni.ssq != nullptr;  // uniform
  uint4 nq[kNormSlots / kThreads];
  if (norm_in) {
    const __amdgpu_buffer_rsrc_t qrs = buffer_rsrc(ni.ssq, (uint32_t)(M * ni.ld * 4));
#pragma unroll
    for (int r = 0; r < kNormSlots / kThreads; ++r) nq[r] = load_b128(qrs, norm_pair_offset(ni, M, tid + kThreads * r));
  }
  constexpr int DEPTH = IMQ_STAGED_DEPTH;
  static_assert(DEPTH == 1 || DEPTH == 2, "one or two stages in flight");
  WRegs ra, rb;
  fetch_w(ra, 0);
  fetch_x(0);
  if (DEPTH > 1) fetch_w(rb, 1);
  if (norm_in) {
#pragma unroll
    for (int r = 0; r < kNormSlots / kThreads; ++r) {
      const int p = tid + kThreads * r;
      nsum[PAIR ? p >> 5 : 0][p & 31] = norm_pair_sum(ni, p, nq[r]);
    }
  }
  // one stage: its registers to LDS, the next x and the weights DEPTH ahead into the same
  // registers (past the last stage every offset is past its buffer: no traffic), then the
  // stage's MFMAs
  auto stage = [&](WRegs& R, int st) {
    __builtin_amdgcn_sched_barrier(0);
    store(R);
    lds_barrier();
    __builtin_amdgcn_sched_barrier(0);
    fetch_x(st + 1);
    fetch_w(R, st + DEPTH);
    __builtin_amdgcn_sched_barrier(0);
    const u32x2_t s2 = *reinterpret_cast<const u32x2_t*>(lds + sbrd);
    const u32x2_t b2 = *reinterpret_cast<const u32x2_t*>(lds + sbrd + 8);
    float spair = 0.0f, cpair = 0.0f;
#pragma unroll
    for (int gi = 0; gi < 4; ++gi) {
      bf16x8_t xa[4];
      f32x16_t p1 = zero;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        xa[s] = as_bf16x8(*reinterpret_cast<const uint4*>(lds + xrd + gi * 128 + 16 * s));
        p1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ones, xa[s], p1, 0, 0, 0);  // row sums
      }
      const uint4 wv = *reinterpret_cast<const uint4*>(lds + wrd + gi * 32);
      const uint32_t wd[4] = {wv.x, wv.y, wv.z, wv.w};
      f32x16_t pp = zero;
#pragma unroll
      for (int s = 0; s < 4; ++s)
        pp = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xa[s], unpack16(wd[s], one), pp, 0, 0, 0);
      const uint32_t sw = gi < 2 ? s2.x : s2.y, bw = gi < 2 ? b2.x : b2.y;
      const float sc = __uint_as_float((gi & 1) ? (sw & 0xffff0000u) : (sw << 16));
      const float bb = __uint_as_float((gi & 1) ? (bw & 0xffff0000u) : (bw << 16));
      const float cg = fmaf(-16.0f, sc, bb);
      const float s16 = 16.0f * sc;
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[e] = fmaf(s16, pp[e], acc[e]);
      if (gi & 1)  // lanes h = 0 / 1 carry the pair's first / second group
        accb = __builtin_amdgcn_mfma_f32_32x32x2f32(h ? p1[0] : spair, h ? cg : cpair, accb, 0, 0, 0);
      else {
        spair = p1[0];
        cpair = cg;
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    lds_barrier();  // every wavefront is done with this stage
  };
  for (int st = 0; st < nst; st += DEPTH) {
    stage(ra, st);
    if (DEPTH > 1 && st + 1 < nst) stage(rb, st + 1);
  }
  acc += accb;

  // the two K-ranges of each tile add through LDS (K-range 0 holds the sum)
  f32x16_t* red = reinterpret_cast<f32x16_t*>(lds);
  if (wk > 0) red[wn * 64 + lane] = acc;
  __syncthreads();
  if (wk == 0) acc += red[wn * 64 + lane];
  if (PAIR) {
    // the gate and up tiles to LDS as [tile][e][lane], then every thread writes four of the
    // 32 x 32 SiLU(gate) * up values (with an input norm, of the rows scaled by 1/rms)
    float* tiles2 = reinterpret_cast<float*>(lds);
    if (norm_in && tid < 32) ninv[tid] = norm_row_inv(ni, nsum, tid);
    __syncthreads();  // every wavefront is done with the K-range sums in LDS
    if (wk == 0)
#pragma unroll
      for (int e = 0; e < 16; ++e) tiles2[(wn * 16 + e) * 64 + lane] = acc[e];
    __syncthreads();
    float gsum[4], usum[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int idx = tid + kThreads * q;
      gsum[q] = tiles2[idx];
      usum[q] = tiles2[1024 + idx];
    }
    if (parts > 1) {
      // a K-part: park its gate and up sums ([16][64] floats each), count the tile's parts;
      // the last adds them in part order (sc1 accesses, coherent across the XCDs' L2s)
      const int tt = tile_p - tiles_max;
      const __amdgpu_buffer_rsrc_t prs =
          buffer_rsrc(partial + (int64_t)tt * parts * 2048, (uint32_t)(parts * 2048 * 4));
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int idx = tid + kThreads * q;
        store_b32_sc1(prs, (uint32_t)((part * 2048 + idx) * 4), __float_as_uint(tiles2[idx]));
      }
      wait_vmem();
      __syncthreads();
      uint32_t* cnt = counters + tt;
      if (tid == 0)
        last = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               (uint32_t)(parts - 1);
      __syncthreads();
      if (!last) return;
      float gp[kMaxPairParts][4], up[kMaxPairParts][4];  // every part's load in flight
#pragma unroll
      for (int sp = 0; sp < kMaxPairParts; ++sp)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int idx = tid + kThreads * q;
          const uint32_t o = (uint32_t)((sp * 2048 + idx) * 4);
          gp[sp][q] = __uint_as_float(load_b32_sc1(prs, sp < parts ? o : kPastBuffer));
          up[sp][q] = __uint_as_float(load_b32_sc1(prs, sp < parts ? o + 4096u : kPastBuffer));
        }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        gsum[q] = usum[q] = 0.0f;
#pragma unroll
        for (int sp = 0; sp < kMaxPairParts; ++sp)
          if (sp < parts) {
            gsum[q] += gp[sp][q];
            usum[q] += up[sp][q];
          }
      }
      if (tid == 0) st_sc1(cnt, 0u);  // ready for the next call
    }
    uint16_t* act = static_cast<uint16_t*>(P.y);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int idx = tid + kThreads * q, e = idx >> 6, l = idx & 63;
      const int m = 8 * (e >> 2) + 4 * (l >> 5) + (e & 3), n = rp0 + (l & 31);
      if (m < M && n < N) {
        const float sc = norm_in ? ninv[m] : 1.0f;
        const float gs = gsum[q], us = usum[q];
        const float g0 = bf16_bits_to_f32(f32_to_bf16_bits(norm_in ? gs * sc : gs));
        const float u0 = bf16_bits_to_f32(f32_to_bf16_bits(norm_in ? us * sc : us));
        act[(size_t)m * P.ldy + n] = f32_to_bf16_bits(g0 / (1.0f + expf(-g0)) * u0);
      }
    }
    return;
  }
  f32x16_t tiles[1] = {acc};
  finish_tiles<1, PARTIAL, kMaxSplitsStaged>(a, P, pi, split, splits, partial, pstride, counters,
                                             tiles_max, tiles,
                                             wk == 0, row0 + 32 * wn, row0, kRows, &last);
}

// ------------------------------ MFMA kernel with the activations held in registers (M >= 3)
//
// The x-stationary kernel, for launches with many 32-row weight tiles per CU (the LM head).
// A workgroup owns a set of tiles of one weight, every r-th one.  Each of its wavefronts
// owns a slice of K (at most GW groups) and loads that slice of every activation row into
// registers once, in the A-operand layout of v_mfma_f32_16x16x32_bf16: lane
// (i = lane % 16, kb = lane / 16) of m-block mb holds x[16 mb + i][64 g + 16 kb ..+16] in
// pair order, k-step j using the 8 values of word 2 kb + j of the group.  The slice is read
// coalesced (lane l: row l / 8 + 8 t, 16-byte piece l % 8 of a group's 128 bytes, eight
// whole rows per instruction) ahead of every weight load, and put through the wavefront's
// own LDS area into that layout (loads straight in the operand layout touch 16 rows per 16
// lanes, and issued behind the weights they waited for them: the LM head at M = 32 took
// 73.0 us that way, 68.8 this way, on one MI355X).  The staging areas share the LDS of the
// parked partials, which are written only after the first tile's barrier.  Tile after tile
// only weights stream: lane (j = lane % 16, kb) reads the 8 bytes of row 16 nb + j at words
// 2kb, 2kb+1 of each group (16 rows x 32 bytes per load instruction), so the activations
// are read from L2 once per workgroup rather than once per tile.  MB = 1 m-block serves
// M <= 16 with 16 wavefronts of at most 4 groups, MB = 2 serves M <= 32 with 8 wavefronts of
// at most 8 groups (the register file holds the x slices of all of them).
//
// Nibbles become bf16 in the form 1 + q/16 (q in mantissa bits 3..6 of bf16 1.0, exact),
// so with v = 1 + q/16 the group's contribution is
//     sum (s q + b) x  =  16 s * sum v x  +  (b - 16 s) * sum x,
// the first term from two bf16 MFMAs per (m-block, n-block) and one fp32 multiply-add
// per output, the second from one v_mfma_f32_16x16x4_f32 per block of four groups (A =
// the rows' sums of x over the four groups, B = b - 16 s per weight row).
//
// Per tile every wavefront parks its partial in LDS and the workgroup adds them in
// wavefront order (the same bits on every run).  Each tile's scales and biases are staged
// in LDS by the whole workgroup (8-byte pieces).  The next tile's weights are loaded group
// by group right after the current tile's group is multiplied (into the registers just
// freed), its scales and biases at the start of the tile; every load is unconditional (past
// the weight or the range: an offset past the buffer, zero, no traffic), so the number of
// loads between any load and its use is the same on every path and every wait is exact;
// MB = 1 keeps two tiles of weights in flight (two register sets, the tile loop unrolled by
// two), MB = 2 one.  Groups past a wavefront's share contribute nothing (x, its sums and the
// scales read as zero).  Requires K % 256 == 0 and K <= 4096.
namespace xs {
constexpr int kRows = 32;                 // weight rows per tile (two 16-row n-blocks)
constexpr int kXStage = 144;              // LDS bytes per staged x row (128, padded)
constexpr uint32_t kOne = kNibOne;
template <int MB>
struct Shape {
  static constexpr int kWaves = MB == 1 ? 16 : 8;   // wavefronts per workgroup
  static constexpr int kAcc = 8 * MB;               // accumulator floats per lane
  static constexpr int kRange = 64;                 // most groups per K-range
  static constexpr int kDepth = MB == 1 ? 2 : 1;    // tiles of weights in flight
};
template <int MB>
constexpr size_t red_bytes() {
  return (size_t)Shape<MB>::kWaves * 64 * (Shape<MB>::kAcc + 1) * sizeof(float);
}
// the wavefronts' x staging areas (16 MB rows each), used before the first tile and sharing
// the parked partials' area
template <int MB>
constexpr size_t stage_bytes() {
  return (size_t)Shape<MB>::kWaves * 16 * MB * kXStage;
}
template <int MB>
constexpr size_t area_bytes() {
  return red_bytes<MB>() > stage_bytes<MB>() ? red_bytes<MB>() : stage_bytes<MB>();
}
}  // namespace xs

struct XsProblem {
  const uint32_t* w;
  const uint16_t* s;
  const uint16_t* b;
  const uint16_t* x;  // row m at x + m * ldx
  void* y;            // row m at y + m * ldy elements
  int64_t ldx;
  int64_t ldy;
  int32_t N;
  int32_t K;
  int32_t wgs;        // workgroups
  int32_t wg0;        // this problem's first workgroup
  int32_t tiles;      // 32-row tiles
  int32_t pad;
};

struct XsArgs {
  XsProblem p[kMaxProblems];
  int32_t count;
  int32_t M;
  int32_t y_f32;
  int32_t scs;        // LDS row stride of the staged scales/biases (odd, >= every Gs)
};

// Stores issued from inline assembly, so the compiler's wait-count model does not see
// them.  Inside a loop that keeps loads in flight from one iteration to the next, a store
// the compiler knows of sits between those loads and their uses and makes it wait for every
// older load; hidden stores only make each of its waits count more operations than it
// assumed, so every wait is at least as strict as it computed (loads complete in issue
// order).  Everything that must see a hidden store waits for it with wait_vmem().
__device__ __forceinline__ u32x4_t rsrc_words(const void* base, uint32_t bytes) {
  const uint64_t u = reinterpret_cast<uint64_t>(base);
  u32x4_t w;
  w.x = __builtin_amdgcn_readfirstlane((uint32_t)u);
  w.y = __builtin_amdgcn_readfirstlane((uint32_t)(u >> 32)) & 0xffffu;  // stride 0
  w.z = __builtin_amdgcn_readfirstlane(bytes);
  w.w = 0x00020000u;
  return w;
}
__device__ __forceinline__ void hidden_store_b16(u32x4_t rs, uint32_t off, uint32_t v) {
  asm volatile("buffer_store_short %0, %1, %2, 0 offen" ::"v"(v), "v"(off), "s"(rs) : "memory");
}
__device__ __forceinline__ void hidden_store_b32(u32x4_t rs, uint32_t off, uint32_t v) {
  asm volatile("buffer_store_dword %0, %1, %2, 0 offen" ::"v"(v), "v"(off), "s"(rs) : "memory");
}

template <int MB, int GW, int D, bool Y32>
__global__ __launch_bounds__(64 * xs::Shape<MB>::kWaves) void qmv_xs_kernel(XsArgs a) {
  using namespace xs;
  constexpr int NW = Shape<MB>::kWaves, NT = 64 * NW, RS = Shape<MB>::kAcc + 1;
  constexpr int NBLK = (GW + 3) / 4;  // blocks of four groups (bias MFMAs)
  extern __shared__ __attribute__((aligned(16))) char lds[];
  float* red = reinterpret_cast<float*>(lds);  // [NW][64][RS] parked partials
  const int scs = a.scs;
  // [32][scs] 16 * scale, then [32][scs] bias, then spare slots for idle threads
  float* s16l = reinterpret_cast<float*>(lds + area_bytes<MB>());
  float* bl = s16l + kRows * scs;

  // this workgroup's problem, K-range and tiles
  const int bid = blockIdx.x;
  int pi = 0;
#pragma unroll
  for (int i = 1; i < kMaxProblems; ++i)
    if (i < a.count && bid >= a.p[i].wg0) pi = i;
  const XsProblem& P = a.p[pi];
  const int c = bid - P.wg0;
  const int T = P.tiles, C = P.wgs;
  if (c >= T) return;
  const int ntiles = (T - c + C - 1) / C;
  const int N = P.N, K = P.K, M = a.M;
  const int G = K >> 6, W = K >> 3;
  const int gs0 = 0, Gs = G;  // the whole K is this workgroup's range
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int j16 = lane & 15, kb = lane >> 4;
  const int wl0 = (Gs * wave) / NW;              // first group of this wavefront (in the range)
  const int gc = (Gs * (wave + 1)) / NW - wl0;   // its groups (<= GW)
  const int wg0 = gs0 + wl0;
  const uint32_t one = in_vgpr(kOne);

  const __amdgpu_buffer_rsrc_t wrsrc = buffer_rsrc(P.w, (uint32_t)N * (uint32_t)W * 4u);
  const uint32_t sb_bytes = (uint32_t)N * (uint32_t)G * 2u;
  const __amdgpu_buffer_rsrc_t srsrc = buffer_rsrc(P.s, sb_bytes);
  const __amdgpu_buffer_rsrc_t brsrc = buffer_rsrc(P.b, sb_bytes);
  const __amdgpu_buffer_rsrc_t xrsrc = buffer_rsrc(P.x, (uint32_t)((M - 1) * P.ldx * 2 + K * 2));
  const int ysz = Y32 ? 4 : 2;
  const u32x4_t yrs = rsrc_words(P.y, (uint32_t)(((int64_t)(M - 1) * P.ldy + N) * ysz));

  // Scale and bias pieces of a tile: piece q < 8 Gs of each is the quad of row q / (Gs/4)
  // at groups gs0 + 4 (q % (Gs/4)) .. +3 (8 bytes); thread tid takes piece tid of the
  // scales and of the biases.  Rows past N lie past the buffer and read zero; threads
  // without a piece load nothing and park their (zero) values in a spare LDS slot.
  // (An offset with bit 31 set lies past every buffer here: the load reads zero and moves
  // nothing, the store is dropped.  Adding a row offset to it cannot carry out of bit 31
  // because every buffer is below 2 GiB.)
  uint32_t sbrel, sbdst;
  {
    const int quarter = Gs >> 2;
    const int row = tid / quarter, pr = tid - row * quarter;
    const bool in = tid < 8 * Gs;
    sbrel = (uint32_t)(row * G + gs0 + 4 * pr) * 2u | ((uint32_t)!in << 31);
    sbdst = in ? (uint32_t)(row * scs + 4 * pr) : (uint32_t)(2 * kRows * scs);
  }
  u32x2_t sv[D], bv[D];
  auto load_sb = [&](int d, int row0, bool valid) {
    const uint32_t off = sbrel + ((uint32_t)row0 * (uint32_t)G * 2u | ((uint32_t)!valid << 31));
    sv[d] = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(srsrc, off, 0, 0));
    bv[d] = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(brsrc, off, 0, 0));
  };
  auto store_sb = [&](int d) {
    float* ds = s16l + sbdst;
    float* db = bl + sbdst;
    ds[0] = 16.0f * bf16_bits_to_f32(sv[d].x & 0xffffu);
    ds[1] = 16.0f * bf16_bits_to_f32(sv[d].x >> 16);
    ds[2] = 16.0f * bf16_bits_to_f32(sv[d].y & 0xffffu);
    ds[3] = 16.0f * bf16_bits_to_f32(sv[d].y >> 16);
    db[0] = bf16_bits_to_f32(bv[d].x & 0xffffu);
    db[1] = bf16_bits_to_f32(bv[d].x >> 16);
    db[2] = bf16_bits_to_f32(bv[d].y & 0xffffu);
    db[3] = bf16_bits_to_f32(bv[d].y >> 16);
  };

  // Weight loads: lane (j16, kb) reads, for n-block nb, row row0 + 16 nb + j16 (rows past N
  // read zero) at words 2 kb, 2 kb + 1 of each of its groups.
  // D register sets: tile i of this workgroup's list lives in set i % D, and its loads are
  // issued while tile i - D is computed (the first D tiles' at the start).
  u32x2_t wv[D][GW][2];
  const uint32_t wlane = (uint32_t)j16 * (uint32_t)W * 4u + 32u * (uint32_t)wg0 + 8u * kb;
  auto load_w = [&](int d, int g, int row0, bool valid) {
    const uint32_t dead = (uint32_t)!(valid && g < gc) << 31;
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const uint32_t off = (wlane + (uint32_t)(row0 + 16 * nb) * (uint32_t)W * 4u + 32u * g) | dead;
      wv[d][g][nb] = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(wrsrc, off, 0, 0));
    }
  };

  // x of this wavefront's groups first (coalesced pieces, staged below), so that staging it
  // waits for x alone
  uint4 xc[GW][2 * MB];
  const int c8 = lane & 7, r8 = lane >> 3;
#pragma unroll
  for (int g = 0; g < GW; ++g)
#pragma unroll
    for (int t = 0; t < 2 * MB; ++t) {
      const int r = r8 + 8 * t;
      const uint32_t off = (uint32_t)r * (uint32_t)P.ldx * 2u + (uint32_t)(64 * (wg0 + g)) * 2u + 16u * (uint32_t)c8;
      xc[g][t] = load_b128(xrsrc, off | ((uint32_t)!(r < M && g < gc) << 31));
    }
  __builtin_amdgcn_sched_barrier(0);
  // The first D tiles' scale/bias and weight loads, in the order the loop issues them (so
  // that every path into the loop has the same loads in flight in the same order), then
  // x of this wavefront's groups into registers and the groups' row sums.
#pragma unroll
  for (int d = 0; d < D; ++d) {
    load_sb(d, (c + d * C) * kRows, d < ntiles);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int g = 0; g < GW; ++g) {
      load_w(d, g, (c + d * C) * kRows, d < ntiles);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  bf16x8_t xa[MB][GW][2];
  float sxa[MB][NBLK];
  {
    // group by group through this wavefront's LDS area (16 MB rows of kXStage bytes) into
    // the operand layout; the wavefront's LDS instructions run in order, so the fences only
    // keep the compiler from moving them
    char* xst = lds + wave * (16 * MB * kXStage);
    uint4 xv[MB][GW][2];
#pragma unroll
    for (int g = 0; g < GW; ++g) {
#pragma unroll
      for (int t = 0; t < 2 * MB; ++t)
        *reinterpret_cast<uint4*>(xst + (r8 + 8 * t) * kXStage + 16 * c8) = xc[g][t];
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int p = 0; p < 2; ++p)
          xv[mb][g][p] = *reinterpret_cast<const uint4*>(xst + (16 * mb + j16) * kXStage + 32 * kb + 16 * p);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
    }
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t ones = in_vgpr(kOnes);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int b = 0; b < NBLK; ++b) sxa[mb][b] = 0.0f;
#pragma unroll
    for (int g = 0; g < GW; ++g) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        float part = 0.0f;
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          const uint4 v = xv[mb][g][p];
          part = dot2(v.x, ones, part);
          part = dot2(v.y, ones, part);
          part = dot2(v.z, ones, part);
          part = dot2(v.w, ones, part);
          xa[mb][g][p] = as_bf16x8(pair_order(v));
        }
        part = add_xor16(part);
        part = add_xor32(part);  // the row's sum over the group, in every kb lane
        if (kb == (g & 3)) sxa[mb][g >> 2] = part;
      }
      __builtin_amdgcn_sched_barrier(0);  // group by group: the raw x dies as it is converted
    }
  }

  const f32x4_t zero = {};
  for (int it = 0; it < ntiles; it += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
    // tile it + d of the list (past the list's end when ntiles is not a multiple of D:
    // its loads read zero and its stores are dropped)
    const int ti = it + d;
    const bool live = ti < ntiles;
    const int row0 = (c + ti * C) * kRows;
    const int nrow0 = (c + (ti + D) * C) * kRows;
    const bool has_next = ti + D < ntiles;
    __builtin_amdgcn_sched_barrier(0);
    store_sb(d);
    lds_barrier();
    __builtin_amdgcn_sched_barrier(0);
    load_sb(d, nrow0, has_next);
    f32x4_t acc[MB][2];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb][0] = acc[mb][1] = zero;
    float cbv[2] = {0.0f, 0.0f};
#pragma unroll
    for (int g = 0; g < GW; ++g) {
      // (LDS reads past a wavefront's groups stay inside the staged area; their values are
      // replaced by zero)
      float s16v[2];
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const int base = (16 * nb + j16) * scs + wl0;
        s16v[nb] = s16l[base + g];
        if ((g & 3) == 0) cbv[nb] = bl[base + g + kb] - s16l[base + g + kb];
      }
      f32x4_t pp[MB][2];
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const bf16x8_t w0 = unpack16(wv[d][g][nb].x, one), w1 = unpack16(wv[d][g][nb].y, one);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          pp[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[mb][g][0], w0, zero, 0, 0, 0);
          pp[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[mb][g][1], w1, pp[mb][nb], 0, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);  // one n-block's unpacked weights at a time
      }
      load_w(d, g, nrow0, has_next);  // tile ti + D's group g, into the registers just freed
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const float s16 = g < gc ? s16v[nb] : 0.0f;
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[mb][nb][e] = fmaf(s16, pp[mb][nb][e], acc[mb][nb][e]);
      }
      if ((g & 3) == 3 || g == GW - 1) {  // the block of four groups g & ~3 ..: lane kb its group
        const int gg = (g & ~3) + kb;
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
          const float cb = gg < gc && gg <= g ? cbv[nb] : 0.0f;
#pragma unroll
          for (int mb = 0; mb < MB; ++mb)
            acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(sxa[mb][g >> 2], cb, acc[mb][nb], 0, 0, 0);
        }
      }
      __builtin_amdgcn_sched_barrier(0);  // one group at a time: bounds the live registers
    }
    // park this wavefront's partial; the workgroup adds them in order
    {
      float* dst = red + (wave * 64 + lane) * RS;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
#pragma unroll
          for (int e = 0; e < 4; ++e) dst[(mb * 2 + nb) * 4 + e] = acc[mb][nb][e];
    }
    lds_barrier();
    // element e of the tile: row n = e % 32 of the tile, activation row m = e / 32; its
    // holder lane is 16 (m % 16 / 4) + n % 16, register (m / 16, n / 16, m % 4)
    constexpr int kPer = (kRows * 16 * MB + NT - 1) / NT;
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
      const int e0 = tid + NT * q;
      const bool ein = e0 < kRows * 16 * MB;
      const int e = ein ? e0 : 0;
      const int m = e >> 5, n = e & 31;
      const int hl = 16 * ((m & 15) >> 2) + (n & 15);
      const int reg = ((m >> 4) * 2 + (n >> 4)) * 4 + (m & 3);
      const float* src = red + hl * RS + reg;
      float sum = 0.0f;
#pragma unroll
      for (int w = 0; w < NW; ++w) sum += src[w * 64 * RS];
      const uint32_t dead = (uint32_t)!(live && ein && m < M && row0 + n < N) << 31;
      if (Y32)
        hidden_store_b32(yrs, (uint32_t)((m * P.ldy + row0 + n) * 4) | dead, __float_as_uint(sum));
      else
        hidden_store_b16(yrs, (uint32_t)((m * P.ldy + row0 + n) * 2) | dead, f32_to_bf16_bits(sum));
    }
    }
  }
}

// ------------------------------ MFMA kernel fed by direct-to-LDS weight loads (M >= 5)
//
// Every workgroup owns 64 weight rows (two 32 x 32 MFMA tiles) over a K-range of whole
// groups (the whole K, or one of SPLITS ranges of four-group multiples), and each of its W
// wavefronts owns GMAX consecutive groups of that range, so each weight byte and each
// activation byte reaches a workgroup once.
//   * Activations: lane (m, kb) of a wavefront loads the 64 bytes x[m][64 g + 32 kb ..+32]
//     of each of its groups g (four 16-byte loads, IMQ_DMA_XDEPTH groups ahead of their
//     use; rows m >= M read zeros), which in pair order are its A operands of the group's
//     four k-steps of v_mfma_f32_32x32x16_bf16.  The group's row sums come from the same
//     registers (sixteen dot2 against (1, 1) and one exchange with lane m + 32).
//   * Weights go from memory to LDS by the buffer loads' LDS path (16 bytes a lane): an
//     instruction moves 8 rows x 128 bytes (four groups of a row: whole lines), lane l to
//     LDS byte 16 l, piece c of row r stored at slot c ^ ((r >> 1) & 7) so that the reads
//     in MFMA-operand order are free of bank conflicts.  One LDS array per four groups: the
//     first four groups' weights are loaded at the start, the next four while the second
//     group is computed, so that a wavefront is not held at issue by loads it needs late
//     (every wavefront of a CU issuing its whole range at once kept the CU's first
//     computation waiting for most of the launch's traffic).
//   * The workgroup's scales and biases (64 rows x the range's groups, one contiguous block
//     of each array) go to LDS the same way, 4 bytes a lane, first of all; one barrier
//     publishes them.
// Per group: P = sum_k v x from four bf16 MFMAs (v = 1 + q/16, exact), acc += 16 s * P; per
// pair of groups one v_mfma_f32_32x32x2_f32 adds (b - 16 s) * sum x.  Groups past a
// wavefront's range are not computed (their loads read valid bytes or zeros).  At the end
// the wavefronts' accumulators are added in wavefront order (K order) through LDS.  Without
// splits the workgroup writes its 64 rows of y.  With splits it writes an fp32 partial of
// them, and the last split of the tile to finish (a counter per tile in the caller's
// workspace) adds the partials in split order, writes y and returns the counter to zero
// (the same bits whatever order the splits finish in; partials and counters through sc1
// accesses, coherent across the XCDs' L2 caches).  Requires K % 256 == 0, a range of at
// most 64 groups and x rows 16-byte aligned.
#ifndef IMQ_DMA_XDEPTH
#define IMQ_DMA_XDEPTH 2
#endif
namespace dm {
constexpr int kRows = 64;                  // weight rows per workgroup
constexpr int kChunkBytes = kRows * 128;   // a wavefront's four groups of the 64 rows
constexpr int kMaxGroups = 64;             // groups of a workgroup's K-range
constexpr int kMaxSplits = 16;             // K-ranges of a tile
__device__ __forceinline__ int swz(int r) { return (r >> 1) & 7; }
// s_waitcnt immediate that waits for vmcnt <= n and nothing else (gfx9 encoding)
constexpr int vmcnt_imm(int n) { return (n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8); }
}  // namespace dm

struct DmaArgs {
  float* partial;                // split partials: problem i at partial + i * pstride
  uint32_t* counters;            // per (problem, tile) arrival counters, zero between calls
  int64_t pstride;
  int32_t splits;                // K-ranges per tile (1: no partials)
  int32_t range;                 // groups per K-range (a multiple of 4)
  int32_t tiles_max;             // counters per problem
  NormIn nin;                    // input rows scaled by 1/rms (nin.ssq == nullptr: off)
  ResidualOut res;               // residual epilogue instead of y (res.h == nullptr: off)
  int32_t planes;                // 1: every K-range's partial is an output plane (no y)
  int32_t pad;
};

template <int W, int GMAX, bool SPLIT>
__global__ __launch_bounds__(64 * W) void qmv_dma_kernel(LaunchArgs a, DmaArgs d) {
  constexpr int NC = GMAX / 4;  // LDS arrays of four groups per wavefront
  static_assert(NC == 1 || NC == 2, "GMAX is 4 or 8");
  constexpr int XD = IMQ_DMA_XDEPTH < GMAX ? IMQ_DMA_XDEPTH : GMAX;  // x groups in flight
  __shared__ __attribute__((aligned(16))) char wb0[W * dm::kChunkBytes];
  __shared__ __attribute__((aligned(16))) char wb1[NC > 1 ? W * dm::kChunkBytes : 16];
  __shared__ __attribute__((aligned(16))) uint32_t sbl[dm::kRows * W * GMAX];
  __shared__ float nsum[kNormMaxTiles / 4][32];  // input norm: pair sums [j][row]
  __shared__ int last;
  const int pi = blockIdx.y;
  const Problem& P = a.p[pi];
  const int N = P.N, K = P.K, M = a.M, G = K >> 6;
  const int splits = SPLIT ? d.splits : 1;
  const int tile = SPLIT ? (int)blockIdx.x / splits : (int)blockIdx.x;
  const int split = SPLIT ? (int)blockIdx.x - tile * splits : 0;
  const int row0 = tile * dm::kRows;
  if (row0 >= N) return;  // past this problem's tiles
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 31, kb = lane >> 5;

  // this workgroup's K-range [gs0, gs1) and this wavefront's groups [g0, g0 + nw) of it
  const int gs0 = SPLIT ? split * d.range : 0;
  const int gs1 = SPLIT ? min(G, gs0 + d.range) : G;
  const int Gs = gs1 - gs0;
  const int g0 = gs0 + wave * GMAX;
  const int nw = __builtin_amdgcn_readfirstlane(min(GMAX, max(0, gs1 - g0)));

  const __amdgpu_buffer_rsrc_t wrs = buffer_rsrc(P.w, (uint32_t)N * (uint32_t)(K >> 1));
  const uint32_t sb_bytes = (uint32_t)N * (uint32_t)G * 2u;
  const __amdgpu_buffer_rsrc_t srs = buffer_rsrc(P.s, sb_bytes);
  const __amdgpu_buffer_rsrc_t brs = buffer_rsrc(P.b, sb_bytes);
  // x as rows, or in the tile layout (ldx == 0: group g's piece t at 4096 g + 1024 t)
  const bool xt = P.ldx == 0;  // uniform
  const __amdgpu_buffer_rsrc_t xrs =
      buffer_rsrc(P.x, xt ? (uint32_t)K * 64u : (uint32_t)(((int64_t)(M - 1) * P.ldx + K) * 2));
  const uint32_t xrow = j >= M ? kPastBuffer : xt ? 16u * (uint32_t)lane : (uint32_t)j * (uint32_t)P.ldx * 2u + 64u * (uint32_t)kb;
  const uint32_t xgs = xt ? 4096u : 128u, xts = xt ? 1024u : 16u;

  // 0. the input norm's partial sums of squares, before every other load (the first wait
  //    below then covers them): NQ b128 per thread cover 32 rows x kNormMaxTiles partials
  constexpr int NQ = (kNormSlots + 64 * W - 1) / (64 * W);
  const bool norm_in = d.nin.ssq != nullptr;  // uniform
  uint4 nq[NQ];
  if (norm_in) {
    const __amdgpu_buffer_rsrc_t qrs = buffer_rsrc(d.nin.ssq, (uint32_t)(M * d.nin.ld * 4));
#pragma unroll
    for (int r = 0; r < NQ; ++r) {
      const int p = tid + 64 * W * r;
      nq[r] = load_b128(qrs, p < kNormSlots ? norm_pair_offset(d.nin, M, p) : kPastBuffer);
    }
  }

  // 1. scales, then biases, of rows [row0, row0 + 64) over the range: Gs instructions of 64
  //    dwords, dword dd of an array at LDS dword array * 32 Gs + dd
  {
    const int hp = Gs >> 1;  // dwords per row and array
    for (int i = wave; i < Gs; i += W) {
      const int arr = i >= hp ? 1 : 0;
      const int dd = (i - arr * hp) * 64 + lane;
      const int r = dd / hp, pr = dd - r * hp;
      const int row = row0 + r < N ? row0 + r : N - 1;
      const uint32_t off = (uint32_t)row * (uint32_t)G * 2u + 2u * (uint32_t)gs0 + 4u * (uint32_t)pr;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          arr ? brs : srs, (__attribute__((address_space(3))) void*)(sbl + arr * 32 * Gs + (i - arr * hp) * 64),
          4, off, 0, 0, 0);
    }
  }
  // 2. weights: per four groups, 8 instructions of 8 rows x 128 bytes
  auto load_w = [&](char* buf, int q) {
#pragma unroll
    for (int i8 = 0; i8 < 8; ++i8) {
      const int r = 8 * i8 + (lane >> 3);
      const int c = (lane & 7) ^ dm::swz(r);
      int gg = g0 + 4 * q + (c >> 1);
      gg = gg < gs1 ? gg : gs1 - 1;
      const int row = row0 + r < N ? row0 + r : N - 1;
      const uint32_t off = (uint32_t)row * (uint32_t)(K >> 1) + 32u * (uint32_t)gg + 16u * (uint32_t)(c & 1);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          wrs, (__attribute__((address_space(3))) void*)(buf + wave * dm::kChunkBytes + i8 * 1024), 16, off,
          0, 0, kNt);
    }
  };
  // 3. this lane's 64 bytes of x for group gi (rows m >= M and groups past the range:
  //    zeros, no traffic)
  struct XG {
    uint4 v[4];
  };
  auto load_x = [&](XG& xg, int gi) {
    const int g = g0 + gi;
    const uint32_t off = g < gs1 ? xrow + xgs * (uint32_t)g : kPastBuffer;
#pragma unroll
    for (int t = 0; t < 4; ++t) xg.v[t] = load_b128(xrs, off + xts * (uint32_t)t);
  };

  XG xq[GMAX];
  __builtin_amdgcn_sched_barrier(0);  // the wait below counts the loads issued after these
  load_w(wb0, 0);
#pragma unroll
  for (int gi = 0; gi < XD; ++gi) load_x(xq[gi], gi);
  __builtin_amdgcn_sched_barrier(0);
  // this wavefront's scales and biases have landed (the weight and x loads issued after
  // them may not have); past the barrier every wavefront's have
  __builtin_amdgcn_s_waitcnt(dm::vmcnt_imm(8 + 4 * XD));
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);

  const uint32_t one = in_vgpr(kNibOne);
  const f32x16_t zero = {};
  f32x16_t acc[2] = {zero, zero}, accb[2] = {zero, zero};
  uint32_t sp[2] = {0u, 0u}, bp[2] = {0u, 0u};
  float sum_even = 0.0f;  // row j's sum of x over the pair's first group
  const int gl0 = g0 - gs0;  // this wavefront's first group within the range
#pragma unroll
  for (int gi = 0; gi < GMAX; ++gi) {
    if (gi + XD < GMAX) load_x(xq[gi + XD], gi + XD);
    if (NC > 1 && gi == 1) load_w(wb1, 1);  // the next four groups, behind the second x
    if (gi < nw) {
      const char* wb = (gi >> 2) ? wb1 : wb0;
      const XG& xg = xq[gi];
      bf16x8_t xa[4];
      float half = 0.0f;  // this lane's 32 values of row j
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        xa[t] = as_bf16x8(pair_order(xg.v[t]));
        half = dot2(xg.v[t].x, one, half);
        half = dot2(xg.v[t].y, one, half);
        half = dot2(xg.v[t].z, one, half);
        half = dot2(xg.v[t].w, one, half);
      }
      const float gsum = add_xor32(half);  // row j over the whole group
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int r = 32 * t + j;
        if ((gi & 1) == 0) {
          const int gl = gl0 + gi;
          sp[t] = sbl[r * (Gs >> 1) + (gl >> 1)];
          bp[t] = sbl[32 * Gs + r * (Gs >> 1) + (gl >> 1)];
        }
        const int c = 2 * (gi & 3) + kb;
        const uint4 wv = *reinterpret_cast<const uint4*>(
            wb + wave * dm::kChunkBytes + (r >> 3) * 1024 + 16 * (8 * (r & 7) + (c ^ dm::swz(r))));
        f32x16_t p = zero;
        p = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xa[0], unpack16(wv.x, one), p, 0, 0, 0);
        p = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xa[1], unpack16(wv.y, one), p, 0, 0, 0);
        p = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xa[2], unpack16(wv.z, one), p, 0, 0, 0);
        p = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xa[3], unpack16(wv.w, one), p, 0, 0, 0);
        const float s16 = 16.0f * __uint_as_float((gi & 1) ? (sp[t] & 0xffff0000u) : (sp[t] << 16));
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[t][e] = fmaf(s16, p[e], acc[t][e]);
        // the pair's offset term once its second group is done (or at an unpaired last
        // one): A = the rows' sums (lanes kb = 0 / 1: the pair's first / second group),
        // B = b - 16 s of the same groups per weight row
        if ((gi & 1) || gi + 1 == nw) {
          const uint32_t sw = kb ? (sp[t] & 0xffff0000u) : (sp[t] << 16);
          const uint32_t bw = kb ? (bp[t] & 0xffff0000u) : (bp[t] << 16);
          float cg = fmaf(-16.0f, __uint_as_float(sw), __uint_as_float(bw));
          cg = (kb && !(gi & 1)) ? 0.0f : cg;
          const float xs = (gi & 1) ? (kb ? gsum : sum_even) : gsum;
          accb[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(xs, cg, accb[t], 0, 0, 0);
        }
      }
      sum_even = gsum;
    }
  }
  acc[0] += accb[0];
  acc[1] += accb[1];

  // the wavefronts' accumulators, added in wavefront order: wave w's slice of wb0 holds
  // [tile][e][lane] floats (a wavefront without groups never waited for its weight loads
  // into that slice: wait for them first)
  wait_vmem();
  if (norm_in) {  // the input norm's pair sums, published by the barrier below
#pragma unroll
    for (int r = 0; r < NQ; ++r) {
      const int p = tid + 64 * W * r;
      if (p < kNormSlots) nsum[p >> 5][p & 31] = norm_pair_sum(d.nin, p, nq[r]);
    }
  }
  float* red = reinterpret_cast<float*>(wb0);
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int e = 0; e < 16; ++e) red[((wave * 2 + t) * 16 + e) * 64 + lane] = acc[t][e];
  __syncthreads();
  // with an input norm, lane m of every wavefront holds row m's 1/rms (norm_row_inv of the
  // pair sums the barrier above published); an output of row m reads it from that lane
  const float inv_lane = norm_in && lane < 32 ? norm_row_inv(d.nin, nsum, lane) : 1.0f;
  auto row_inv = [&](int m) { return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, inv_lane), m)); };
  // thread (wave, nl) adds rows m = wave, wave + W, ... of tile row nl; every LDS read before
  // the first store
  constexpr int MI = (32 + W - 1) / W;
  const int nl = tid & 63, t = nl >> 5, jn = nl & 31, n = row0 + nl;
  float sums[MI];
#pragma unroll
  for (int i = 0; i < MI; ++i) {
    const int m = min(wave + i * W, 31);
    const int h = (m >> 2) & 1, e = 4 * (m >> 3) + (m & 3);
    float v = 0.0f;
#pragma unroll
    for (int w2 = 0; w2 < W; ++w2) v += red[((w2 * 2 + t) * 16 + e) * 64 + jn + 32 * h];
    sums[i] = v;
  }
  // The outputs of this thread: y[m][n] for m = wave + i W (uniform across the wavefront),
  // scaled by the row's 1/rms with an input norm; with a residual epilogue y is not stored:
  // h += bf16(y), x' = bf16(h * w) and the tile's sums of squares of h per row instead.
  const bool res = d.res.h != nullptr;  // uniform
  auto finish = [&](const float (&v)[MI], const float (&hv)[MI], float wn) {
    float sq[MI];  // the new h squared (residual epilogue), 0 outside the rows and columns
#pragma unroll
    for (int i = 0; i < MI; ++i) {
      const int m = wave + i * W;
      sq[i] = 0.0f;
      if (m >= M) continue;
      const float y = norm_in ? v[i] * row_inv(m) : v[i];
      if (!res) {
        if (n < N) store_y(a, P, m, n, y);
        continue;
      }
      const float hn = hv[i] + bf16_bits_to_f32(f32_to_bf16_bits(y));
      if (n < N) {
        d.res.h[(size_t)m * d.res.ldh + n] = hn;
        if (d.res.w)
          d.res.x[d.res.ldx == 0 ? (size_t)tile_elem(m, n) : (size_t)m * d.res.ldx + n] = f32_to_bf16_bits(hn * wn);
        sq[i] = hn * hn;
      }
    }
    if (res && d.res.ssq) {
      // the rows' sums over the tile's 64 columns: the DPP stages of all rows first (their
      // chains interleave), then each row's four 16-lane sums, as wave_sum adds them
#pragma unroll
      for (int i = 0; i < MI; ++i) sq[i] = row16_sum(sq[i]);
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        const int m = wave + i * W;
        const float ss = (lane_value(sq[i], 0) + lane_value(sq[i], 16)) +
                         (lane_value(sq[i], 32) + lane_value(sq[i], 48));
        if (m < M && lane == 0) d.res.ssq[m * d.res.ld + tile] = ss;
      }
    }
  };
  // h and the norm weight of this thread's outputs (residual epilogue)
  float hv[MI] = {}, wn = 0.0f;
  auto load_res = [&]() {
#pragma unroll
    for (int i = 0; i < MI; ++i) {
      const int m = wave + i * W;
      hv[i] = m < M && n < N ? d.res.h[(size_t)m * d.res.ldh + n] : 0.0f;
    }
    wn = d.res.w && n < N ? bf16_bits_to_f32(d.res.w[n]) : 0.0f;
  };
  if (!SPLIT && !d.planes) {
    if (res) load_res();
    finish(sums, hv, wn);
    return;
  }
  // split: park the partial, count the tile's arrivals; the last one adds them in order.
  // As output planes (d.planes): each range's partial, scaled by the rows' 1/rms, is the
  // output, and the reader adds the planes in range order.
  const __amdgpu_buffer_rsrc_t prs =
      buffer_rsrc(d.partial + pi * d.pstride, (uint32_t)((int64_t)splits * M * N * 4));
#pragma unroll
  for (int i = 0; i < MI; ++i) {
    const int m = wave + i * W;
    if (m < M && n < N) {
      const float v = d.planes && norm_in ? sums[i] * row_inv(m) : sums[i];
      store_b32_sc1(prs, (uint32_t)(((split * M + m) * N + n) * 4), __float_as_uint(v));
    }
  }
  if (d.planes) return;
  wait_vmem();
  __syncthreads();
  uint32_t* cnt = d.counters + (int64_t)pi * d.tiles_max + tile;
  if (tid == 0)
    last = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
           (uint32_t)(splits - 1);
  __syncthreads();
  if (!last) return;
  if (res) load_res();  // in flight with the partials
  // QB partials of each output in flight at a time (one round trip for up to eight ranges
  // where a thread has at most four outputs), added in split order
  constexpr int QB = MI <= 4 ? 8 : 4;
  const uint32_t step = (uint32_t)(M * N * 4);
  float tot[MI];
#pragma unroll
  for (int i = 0; i < MI; ++i) tot[i] = 0.0f;
  for (int q0 = 0; q0 < splits; q0 += QB) {
    float v[MI][QB];
#pragma unroll
    for (int i = 0; i < MI; ++i) {
      const int m = wave + i * W;
      const bool in = m < M && n < N;
      const uint32_t o = (uint32_t)((m * N + n) * 4) + (uint32_t)q0 * step;
#pragma unroll
      for (int q = 0; q < QB; ++q)
        v[i][q] = __uint_as_float(load_b32_sc1(prs, in && q0 + q < splits ? o + q * step : kPastBuffer));
    }
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int q = 0; q < QB; ++q)
        if (q0 + q < splits) tot[i] += v[i][q];
  }
  finish(tot, hv, wn);
  if (tid == 0) st_sc1(cnt, 0u);  // ready for the next call
}

// ------------------- gate/up with SiLU * up over bands of rows (direct-to-LDS, M <= 32)
//
// The gate/up launch with the input RMSNorm folded in, laid out so that every CU streams
// about the same share of the two weights, once, with no K-split partials to add across
// workgroups.  The weights' rows are U = ceil(N / 8) units of 8; workgroup i of nwg owns
// units [i U / nwg, (i + 1) U / nwg) (at most pr::kMaxUnits), i.e. R gate rows and the same
// R up rows from row r0, over the whole K, with W = K / 256 wavefronts, wavefront w owning
// groups [4 w, 4 w + 4).  The 2R rows are the workgroup's slots (slot s < R: gate row
// r0 + s, else up row r0 + s - R), 32 to an MFMA block.
//   * Weights go from memory to LDS by the buffer loads' LDS path, an instruction per 8
//     slots x 128 bytes (a slot's four groups: whole lines), swizzled as in qmv_dma_kernel,
//     in block order, block b into LDS array b: the compiler tells the arrays apart, so a
//     wavefront's reads of block b wait for block b's loads only, and it computes block b
//     as soon as they have landed.
//   * Scales and biases: lane (j, kb) loads the 8 bytes of slot 32 b + j's four groups of
//     each array straight into registers, from the gate or the up array by its own address
//     (slots past the rows read a valid row: their columns are never stored).
//   * x: lane (m, kb) holds the 64 bytes x[m][64 g + 32 kb ..+32] of each of its groups g,
//     as in qmv_dma_kernel; all four groups are in flight before the first weight wait.
// Per group and block: P = sum_k v x from four bf16 MFMAs (v = 1 + q/16), acc += 16 s P;
// per pair of groups one v_mfma_f32_32x32x2_f32 adds (b - 16 s) sum x.  The wavefronts'
// accumulators are added in wavefront order (K order) through LDS, then
// act[m][n] = bf16(silu(g) * u) with g, u = bf16(the gate, up sums times row m's 1/rms)
// (silu_mul_kernel's expression).  Rows m >= M read zeros and are never stored.  Requires
// K % 256 == 0, K / 256 == W and x rows 16-byte aligned.
namespace pr {
constexpr int kMaxUnits = 5;                // 8-row units of a workgroup: R <= 40
constexpr int kLoadOctets = 2 * kMaxUnits;  // 8-slot weight loads of a wavefront
constexpr int kBlocks = 3;                  // 32-slot MFMA blocks: 2R <= 96
constexpr int kChunk = 4 * 1024;            // a wavefront's block: 32 slots x 128 bytes
}  // namespace pr

template <int W>
__global__ __launch_bounds__(64 * W) void qmv_pair_rows_kernel(LaunchArgs a, NormIn ni, int nwg, int units) {
  static_assert(pr::kLoadOctets <= 4 * pr::kBlocks, "the loads fit the blocks");
  static_assert(16 * 64 * 4 <= pr::kChunk, "a block's accumulators fit its chunk");
  __shared__ __attribute__((aligned(16))) char lds0[W * pr::kChunk];
  __shared__ __attribute__((aligned(16))) char lds1[W * pr::kChunk];
  __shared__ __attribute__((aligned(16))) char lds2[W * pr::kChunk];
  __shared__ float nsum[kNormMaxTiles / 4][32];  // input norm: pair sums [j][row]
  const Problem& Pg = a.p[0];
  const Problem& Pu = a.p[1];
  const int N = Pg.N, K = Pg.K, M = a.M, G = K >> 6;
  const int u0 = (int)(((int64_t)blockIdx.x * units) / nwg);
  const int u1 = (int)(((int64_t)(blockIdx.x + 1) * units) / nwg);
  const int R = 8 * (u1 - u0), r0 = 8 * u0;
  const int nb = (2 * R + 31) >> 5;  // blocks with slots (uniform)
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 31, kb = lane >> 5;
  const int g0 = 4 * wave;

  const uint32_t wbytes = (uint32_t)N * (uint32_t)(K >> 1);
  const __amdgpu_buffer_rsrc_t wgr = buffer_rsrc(Pg.w, wbytes), wur = buffer_rsrc(Pu.w, wbytes);
  const bool xt = Pg.ldx == 0;  // x in the tile layout (uniform)
  const __amdgpu_buffer_rsrc_t xrs =
      buffer_rsrc(Pg.x, xt ? (uint32_t)K * 64u : (uint32_t)(((int64_t)(M - 1) * Pg.ldx + K) * 2));

  // 0. the input norm's partial sums of squares, before every other load
  constexpr int NQ = (kNormSlots + 64 * W - 1) / (64 * W);
  const bool norm_in = ni.ssq != nullptr;  // uniform
  uint4 nq[NQ];
  if (norm_in) {
    const __amdgpu_buffer_rsrc_t qrs = buffer_rsrc(ni.ssq, (uint32_t)(M * ni.ld * 4));
#pragma unroll
    for (int r = 0; r < NQ; ++r) {
      const int p = tid + 64 * W * r;
      nq[r] = load_b128(qrs, p < kNormSlots ? norm_pair_offset(ni, M, p) : kPastBuffer);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  // 1. scales and biases of this lane's slot in each block, this wavefront's four groups
  u32x2_t sv[pr::kBlocks], bv[pr::kBlocks];
#pragma unroll
  for (int b = 0; b < pr::kBlocks; ++b) {
    const int s = 32 * b + j;
    const bool up = s >= R;
    int n = r0 + (up ? s - R : s);
    n = s < 2 * R && n < N ? n : r0;
    const size_t o = (size_t)n * G + g0;  // 8-byte aligned: G and g0 are multiples of 4
    sv[b] = *reinterpret_cast<const u32x2_t*>((up ? Pu.s : Pg.s) + o);
    bv[b] = *reinterpret_cast<const u32x2_t*>((up ? Pu.b : Pg.b) + o);
  }
  // 2. x: four groups of 64 bytes a lane
  const uint32_t xrow = j >= M ? kPastBuffer : xt ? 16u * (uint32_t)lane : (uint32_t)j * (uint32_t)Pg.ldx * 2u + 64u * (uint32_t)kb;
  const uint32_t xgs = xt ? 4096u : 128u, xts = xt ? 1024u : 16u;
  uint4 xq[4][4];
#pragma unroll
  for (int gi = 0; gi < 4; ++gi)
#pragma unroll
    for (int t = 0; t < 4; ++t) xq[gi][t] = load_b128(xrs, xrow + xgs * (uint32_t)(g0 + gi) + xts * (uint32_t)t);
  // 3. weights: octet o = slots [8 o, 8 o + 8) x this wavefront's 128 bytes of each, to
  //    byte (o % 4) * 1024 + 16 lane of the wavefront's chunk of block o / 4 (octets past
  //    the slots or the rows read zeros, no traffic)
  char* const chunk[pr::kBlocks] = {lds0 + wave * pr::kChunk, lds1 + wave * pr::kChunk, lds2 + wave * pr::kChunk};
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int o = 0; o < pr::kLoadOctets; ++o) {
    const bool up = 8 * o >= R;  // uniform: R is a multiple of 8
    const int r = 8 * o + (lane >> 3);
    const int c = (lane & 7) ^ dm::swz(r);
    const int n = r0 + (up ? r - R : r);
    const uint32_t off = 8 * o < 2 * R && n < N
                             ? (uint32_t)n * (uint32_t)(K >> 1) + 32u * (uint32_t)(g0 + (c >> 1)) + 16u * (uint32_t)(c & 1)
                             : kPastBuffer;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(up ? wur : wgr,
                                             (__attribute__((address_space(3))) void*)(chunk[o >> 2] + (o & 3) * 1024),
                                             16, off, 0, 0, kNt);
  }
  __builtin_amdgcn_sched_barrier(0);

  // x in pair order (the MFMAs' A operands) and its row sums per group
  const uint32_t one = in_vgpr(kNibOne);
  bf16x8_t xa[4][4];
  float gsum[4];
#pragma unroll
  for (int gi = 0; gi < 4; ++gi) {
    float half = 0.0f;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      xa[gi][t] = as_bf16x8(pair_order(xq[gi][t]));
      half = dot2(xq[gi][t].x, one, half);
      half = dot2(xq[gi][t].y, one, half);
      half = dot2(xq[gi][t].z, one, half);
      half = dot2(xq[gi][t].w, one, half);
    }
    gsum[gi] = add_xor32(half);
  }

  const f32x16_t zero = {};
  f32x16_t acc[pr::kBlocks] = {zero, zero, zero};
  auto block = [&](const int b) {
    const int r = 32 * b + j;
#pragma unroll
    for (int gi = 0; gi < 4; ++gi) {
      const int c = 2 * gi + kb;
      const uint4 wv = *reinterpret_cast<const uint4*>(chunk[b] + ((r >> 3) & 3) * 1024 +
                                                       16 * (8 * (r & 7) + (c ^ dm::swz(r))));
      f32x16_t p = zero;
      p = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xa[gi][0], unpack16(wv.x, one), p, 0, 0, 0);
      p = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xa[gi][1], unpack16(wv.y, one), p, 0, 0, 0);
      p = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xa[gi][2], unpack16(wv.z, one), p, 0, 0, 0);
      p = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xa[gi][3], unpack16(wv.w, one), p, 0, 0, 0);
      const uint32_t sw = sv[b][gi >> 1];
      const float s16 = 16.0f * __uint_as_float((gi & 1) ? (sw & 0xffff0000u) : (sw << 16));
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[b][e] = fmaf(s16, p[e], acc[b][e]);
      if (gi & 1) {
        // the pair's offset term: A = the rows' sums (lanes kb = 0 / 1: the pair's first /
        // second group), B = b - 16 s of the same groups per slot
        const uint32_t sp = sv[b][gi >> 1], bp = bv[b][gi >> 1];
        const uint32_t sk = kb ? (sp & 0xffff0000u) : (sp << 16);
        const uint32_t bk = kb ? (bp & 0xffff0000u) : (bp << 16);
        const float cg = fmaf(-16.0f, __uint_as_float(sk), __uint_as_float(bk));
        const float xs = kb ? gsum[gi] : gsum[gi - 1];
        acc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(xs, cg, acc[b], 0, 0, 0);
      }
    }
  };
  // block b once its octets 4 b .. 4 b + 3 have landed (the loads after them may not have)
  static_assert(pr::kBlocks == 3 && pr::kLoadOctets == 10, "the waits count the octets");
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(dm::vmcnt_imm(6));
  __builtin_amdgcn_sched_barrier(0);
  block(0);
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(dm::vmcnt_imm(2));
  __builtin_amdgcn_sched_barrier(0);
  if (nb > 1) block(1);
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(dm::vmcnt_imm(0));
  __builtin_amdgcn_sched_barrier(0);
  if (nb > 2) block(2);

  // the wavefronts' accumulators through LDS: wavefront w's chunk of block b holds [e][lane]
  // (its own weight reads are done: LDS accesses of a wavefront complete in order)
#pragma unroll
  for (int b = 0; b < pr::kBlocks; ++b)
    if (b < nb)
#pragma unroll
      for (int e = 0; e < 16; ++e) reinterpret_cast<float*>(chunk[b])[e * 64 + lane] = acc[b][e];
  if (norm_in) {
#pragma unroll
    for (int r = 0; r < NQ; ++r) {
      const int p = tid + 64 * W * r;
      if (p < kNormSlots) nsum[p >> 5][p & 31] = norm_pair_sum(ni, p, nq[r]);
    }
  }
  __syncthreads();
  // outputs (m, n = r0 + nl), nl fastest across the threads: the gate sum at slot nl, the up
  // sum at slot R + nl, each added over the wavefronts in order
  uint16_t* act = static_cast<uint16_t*>(Pg.y);
  auto slot_sum = [&](int s, int m) {
    const float* red = reinterpret_cast<const float*>((s >> 5) == 0 ? lds0 : (s >> 5) == 1 ? lds1 : lds2);
    const int at = (4 * (m >> 3) + (m & 3)) * 64 + (s & 31) + 32 * ((m >> 2) & 1);
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < W; ++w) v += red[w * (pr::kChunk / 4) + at];
    return v;
  };
  // row m's 1/rms in lane m of every wavefront (the pair sums in order), fetched per output
  const float inv_lane = norm_in && lane < 32 ? norm_row_inv(ni, nsum, lane) : 1.0f;
  for (int idx = tid; idx < 32 * R; idx += 64 * W) {
    const int m = idx / R, nl = idx - m * R, n = r0 + nl;
    const float sc = __int_as_float(__builtin_amdgcn_ds_bpermute(4 * m, __float_as_int(inv_lane)));
    if (m >= M || n >= N) continue;
    const float gs = slot_sum(nl, m), us = slot_sum(R + nl, m);
    const float g0v = bf16_bits_to_f32(f32_to_bf16_bits(norm_in ? gs * sc : gs));
    const float u0v = bf16_bits_to_f32(f32_to_bf16_bits(norm_in ? us * sc : us));
    act[Pg.ldy == 0 ? (size_t)tile_elem(m, n) : (size_t)m * Pg.ldy + n] =
        f32_to_bf16_bits(g0v / (1.0f + expf(-g0v)) * u0v);
  }
}

// -------------- one projection over bands of 32 rows and the whole K (the residual form)
//
// The o and down projections of the batched decode step with their residual epilogue, and
// no K-ranges: workgroup i owns weight rows [32 i, 32 i + 32) (one MFMA block) over the whole
// K with 16 wavefronts, wavefront w owning a run of whole 4-group chunks (the C = K / 256
// chunks dealt as evenly as they go, at most three each: K <= 9728), so no partial leaves
// the workgroup and no second launch adds planes.  A wavefront issues its scales and biases,
// its chunks' weights (by the LDS path: 32 rows x 128 bytes, chunk j of every wavefront in
// LDS array j), then x for its first rb::kXAhead groups; each computed group issues x for
// the group rb::kXAhead ahead, so the x stream (the whole of x per workgroup, from L2) runs
// under the arithmetic.  x in the tile layout (ldx == 0) reads as contiguous 1 KB pieces,
// rows as in qmv_dma_kernel otherwise.  Per group: four bf16 MFMAs, acc += 16 s P, and per
// pair of groups the bias MFMA, as in qmv_dma_kernel.  The wavefronts' accumulators add in
// K order through LDS; thread (m, n) then writes h += bf16(y), x' = bf16(h * w) and the
// band's sum of squares of row m's new h (ssq[m * ld + band]).
namespace rb {
constexpr int kWaves = 16;
constexpr int kChunk = 4096;                       // a chunk's weights: 32 rows x 128 bytes
constexpr int kMaxChunks = 38;                     // K <= 9728
constexpr int kThird = kMaxChunks - 2 * kWaves;    // wavefronts with a third chunk
constexpr int kXAhead = 2;                         // groups of x in flight
// s_waitcnt vmcnt(n) for the n the unrolled loop folds to (0, 4 or 8; else vmcnt(0))
__device__ __forceinline__ void wait_younger(int n) {
  switch (n) {
    case 8: __builtin_amdgcn_s_waitcnt(dm::vmcnt_imm(8)); break;
    case 4: __builtin_amdgcn_s_waitcnt(dm::vmcnt_imm(4)); break;
    default: __builtin_amdgcn_s_waitcnt(dm::vmcnt_imm(0)); break;
  }
}
}  // namespace rb

template <int NI>
__device__ __forceinline__ void rowband_wave(const Problem& P, int M, int r0, int c0, int wave, int lane,
                                             char* const (&arr)[3], f32x16_t& acc) {
  const int N = P.N, K = P.K, G = K >> 6;
  const int j = lane & 31, kb = lane >> 5;
  const bool tiled = P.ldx == 0;  // uniform
  const int nr = r0 + j < N ? r0 + j : N - 1;  // this lane's weight row (clamped)
  // scales and biases of row nr, four groups per chunk, straight into registers
  u32x2_t sv[NI > 0 ? NI : 1], bv[NI > 0 ? NI : 1];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const size_t o = (size_t)nr * G + 4 * (c0 + i);
    sv[i] = *reinterpret_cast<const u32x2_t*>(P.s + o);
    bv[i] = *reinterpret_cast<const u32x2_t*>(P.b + o);
  }
  // the chunks' weights: instruction q of chunk i = rows 8q .. 8q + 7 x 128 bytes
  const __amdgpu_buffer_rsrc_t wrs = buffer_rsrc(P.w, (uint32_t)N * (uint32_t)(K >> 1));
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int r = 8 * q + (lane >> 3);
      const int c = (lane & 7) ^ dm::swz(r);
      const uint32_t off = r0 + r < N ? (uint32_t)(r0 + r) * (uint32_t)(K >> 1) + 32u * (uint32_t)(4 * (c0 + i) + (c >> 1)) +
                                            16u * (uint32_t)(c & 1)
                                      : kPastBuffer;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          wrs, (__attribute__((address_space(3))) void*)(arr[i] + wave * rb::kChunk + q * 1024), 16, off, 0, 0, kNt);
    }
  __builtin_amdgcn_sched_barrier(0);
  // x: lane (m, kb)'s 64 bytes of group g (rows m >= M: zeros, no traffic)
  const __amdgpu_buffer_rsrc_t xrs =
      buffer_rsrc(P.x, tiled ? (uint32_t)K * 64u : (uint32_t)(((int64_t)(M - 1) * P.ldx + K) * 2));
  const bool xin = j < M;
  const uint32_t xbase = tiled ? 16u * (uint32_t)lane : (uint32_t)j * (uint32_t)P.ldx * 2u + 64u * (uint32_t)kb;
  constexpr int NG = 4 * NI;  // this wavefront's groups
  uint4 xq[NG > 0 ? NG : 1][4];
  auto load_x = [&](int s) {
    const uint32_t g = (uint32_t)(4 * c0 + s);
#pragma unroll
    for (int t = 0; t < 4; ++t)
      xq[s][t] = load_b128(xrs, xin ? xbase + (tiled ? (g * 4u + t) * 1024u : 128u * g + 16u * t) : kPastBuffer);
  };
#pragma unroll
  for (int s = 0; s < rb::kXAhead && s < NG; ++s) load_x(s);
  const uint32_t one = in_vgpr(kNibOne);
  const f32x16_t zero = {};
  float sum_even = 0.0f;
#pragma unroll
  for (int s = 0; s < NG; ++s) {
    const int i = s >> 2, gi = s & 3;
    __builtin_amdgcn_sched_barrier(0);
    if (s + rb::kXAhead < NG) load_x(s + rb::kXAhead);
    __builtin_amdgcn_sched_barrier(0);
    // x of group s has landed, and with it every weight load (issued before it): only the
    // x loads of the groups after s may be in flight
    rb::wait_younger(4 * (s + rb::kXAhead < NG ? rb::kXAhead : NG - 1 - s));
    __builtin_amdgcn_sched_barrier(0);
    bf16x8_t xa[4];
    float half = 0.0f;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      xa[t] = as_bf16x8(pair_order(xq[s][t]));
      half = dot2(xq[s][t].x, one, half);
      half = dot2(xq[s][t].y, one, half);
      half = dot2(xq[s][t].z, one, half);
      half = dot2(xq[s][t].w, one, half);
    }
    const float gsum = add_xor32(half);
    const int c = 2 * gi + kb;
    const uint4 wv = *reinterpret_cast<const uint4*>(arr[i] + wave * rb::kChunk + (j >> 3) * 1024 +
                                                     16 * (8 * (j & 7) + (c ^ dm::swz(j))));
    f32x16_t p = zero;
    p = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xa[0], unpack16(wv.x, one), p, 0, 0, 0);
    p = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xa[1], unpack16(wv.y, one), p, 0, 0, 0);
    p = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xa[2], unpack16(wv.z, one), p, 0, 0, 0);
    p = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xa[3], unpack16(wv.w, one), p, 0, 0, 0);
    const uint32_t sw = sv[i][gi >> 1];
    const float s16 = 16.0f * __uint_as_float((gi & 1) ? (sw & 0xffff0000u) : (sw << 16));
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = fmaf(s16, p[e], acc[e]);
    if (gi & 1) {
      // the pair's offset term: A = the rows' sums (lanes kb = 0 / 1: the pair's first /
      // second group), B = b - 16 s of the same groups per weight row
      const uint32_t bw = bv[i][gi >> 1];
      const uint32_t sk = kb ? (sw & 0xffff0000u) : (sw << 16);
      const uint32_t bk = kb ? (bw & 0xffff0000u) : (bw << 16);
      const float cg = fmaf(-16.0f, __uint_as_float(sk), __uint_as_float(bk));
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(kb ? gsum : sum_even, cg, acc, 0, 0, 0);
    }
    sum_even = gsum;
  }
}

// The launch: up to rb::kMaxProblems projections of one x (the same K), bands [band0[i],
// band0[i + 1]) of the grid for problem i; either the residual epilogue (one problem, res.h
// set) or an fp32 output plane per problem, planes + i * pstride + m * N_i + n, scaled by
// row m's 1/rms when the input norm is folded in (ni.ssq set).
struct RowbandArgs {
  Problem p[3];
  int32_t band0[4];
  int32_t count, M;
  NormIn ni;
  ResidualOut res;
  float* planes;
  int64_t pstride;
};

__global__ __launch_bounds__(64 * rb::kWaves) void qmv_rowband_kernel(RowbandArgs A) {
  __shared__ __attribute__((aligned(16))) char arr0[rb::kWaves * rb::kChunk];
  __shared__ __attribute__((aligned(16))) char arr1[rb::kWaves * rb::kChunk];
  __shared__ __attribute__((aligned(16))) char arr2[rb::kThird * rb::kChunk];
  __shared__ float nsum[kNormMaxTiles / 4][32];  // input norm: pair sums [j][row]
  const int M = A.M;
  // the problem of this band (uniform), its fields selected from static loads of all three
  // (an indexed load would wait for the band test before fetching them)
  const int bx = blockIdx.x;
  const int pi = A.count > 1 && bx >= A.band0[1] ? (A.count > 2 && bx >= A.band0[2] ? 2 : 1) : 0;
  const Problem P = pi == 0 ? A.p[0] : pi == 1 ? A.p[1] : A.p[2];
  const int N = P.N, C = P.K >> 8;
  const int band = blockIdx.x - A.band0[pi], r0 = band * 32;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // the input norm's partial sums of squares, before every other load
  constexpr int NQ = (kNormSlots + 64 * rb::kWaves - 1) / (64 * rb::kWaves);
  const bool norm_in = A.ni.ssq != nullptr;  // uniform
  uint4 nq[NQ];
  if (norm_in) {
    const __amdgpu_buffer_rsrc_t qrs = buffer_rsrc(A.ni.ssq, (uint32_t)(M * A.ni.ld * 4));
#pragma unroll
    for (int r = 0; r < NQ; ++r) {
      const int p = tid + 64 * rb::kWaves * r;
      nq[r] = load_b128(qrs, p < kNormSlots ? norm_pair_offset(A.ni, M, p) : kPastBuffer);
    }
  }
  // this wavefront's chunks [c0, c0 + nc): C / 16 each, one more for the first C % 16
  const int base = C / rb::kWaves, extra = C - base * rb::kWaves;
  const int nc = base + (wave < extra ? 1 : 0);
  const int c0 = wave * base + (wave < extra ? wave : extra);
  char* const arr[3] = {arr0, arr1, arr2};
  const f32x16_t zero = {};
  f32x16_t acc = zero;
  switch (nc) {  // uniform
    case 1: rowband_wave<1>(P, M, r0, c0, wave, lane, arr, acc); break;
    case 2: rowband_wave<2>(P, M, r0, c0, wave, lane, arr, acc); break;
    case 3: rowband_wave<3>(P, M, r0, c0, wave, lane, arr, acc); break;
    default: break;
  }

  // this thread's output: row m = tid / 32, column n = r0 + tid % 32; the residual rows in
  // flight with the reduction
  const ResidualOut& res = A.res;
  const bool plane = res.h == nullptr;  // uniform
  const int m = tid >> 5, n = r0 + (tid & 31);
  const bool mine = m < M && n < N;
  const float hv = mine && !plane ? res.h[(size_t)m * res.ldh + n] : 0.0f;
  const float wn = mine && !plane && res.w ? bf16_bits_to_f32(res.w[n]) : 0.0f;
  // the accumulators through LDS: wavefront w's [e][lane] in its chunk-0 slot (its own
  // weight reads are done: a wavefront's LDS accesses complete in order)
  float* red = reinterpret_cast<float*>(arr0);
#pragma unroll
  for (int e = 0; e < 16; ++e) red[wave * (rb::kChunk / 4) + e * 64 + lane] = acc[e];
  if (norm_in) {  // the input norm's pair sums, published by the barrier below
#pragma unroll
    for (int r = 0; r < NQ; ++r) {
      const int p = tid + 64 * rb::kWaves * r;
      if (p < kNormSlots) nsum[p >> 5][p & 31] = norm_pair_sum(A.ni, p, nq[r]);
    }
  }
  __syncthreads();
  const int at = (4 * (m >> 3) + (m & 3)) * 64 + (tid & 31) + 32 * ((m >> 2) & 1);
  float y = 0.0f;
#pragma unroll
  for (int w = 0; w < rb::kWaves; ++w) y += red[w * (rb::kChunk / 4) + at];
  if (plane) {
    // row m's 1/rms in lane m of every wavefront (the pair sums in order), fetched per output
    const float inv_lane = norm_in && lane < 32 ? norm_row_inv(A.ni, nsum, lane) : 1.0f;
    const float inv = __int_as_float(__builtin_amdgcn_ds_bpermute(4 * m, __float_as_int(inv_lane)));
    if (mine) A.planes[pi * A.pstride + (int64_t)m * N + n] = norm_in ? y * inv : y;
    return;
  }
  float sq = 0.0f;
  if (mine) {
    const float hn = hv + bf16_bits_to_f32(f32_to_bf16_bits(y));
    res.h[(size_t)m * res.ldh + n] = hn;
    if (res.w) res.x[res.ldx == 0 ? (size_t)tile_elem(m, n) : (size_t)m * res.ldx + n] = f32_to_bf16_bits(hn * wn);
    sq = hn * hn;
  }
  if (res.ssq) {
    // row m's sum over the band's 32 columns: lanes 0-31 hold row 2w, 32-63 row 2w + 1
    sq = row16_sum(sq);
    const float lo = lane_value(sq, 0) + lane_value(sq, 16), hi = lane_value(sq, 32) + lane_value(sq, 48);
    if ((lane & 31) == 0 && m < M) res.ssq[m * res.ld + band] = lane ? hi : lo;
  }
}

// ------------------------- the residual epilogue over K-range planes, a launch of its own
//
// qmv_dma_kernel's residual epilogue for a projection computed as K-range output planes
// (imq_qmv_norm_planes): y[m][n] = the planes added in plane order from zero, then
// h += bf16(y), x' = bf16(h * w) and each row's sum of squares of the new h over every
// 64-column tile.  The expressions and reduction orders are those of the last K-range of
// a split qmv_dma_kernel tile, so the two forms give the same bits.  A wavefront per
// (row, 64-column tile), lane l on column 64 tile + l: the epilogue that one workgroup per
// tile ran after the split counter's round trips is spread over every CU (at batch 32 the
// o projection's launch ran 6.4 us longer per layer with it than as planes alone).
constexpr int kResPlanes = 16;   // planes one launch adds
constexpr int kResRowsPerGroup = 4;
template <int S>  // at most S planes: the loads past the call's planes are not issued
__global__ __launch_bounds__(64 * kResRowsPerGroup) void residual_planes_kernel(const float* __restrict__ planes,
                                                                               int nplanes, int M, int N,
                                                                               ResidualOut r) {
  const int tile = blockIdx.x, lane = threadIdx.x & 63;
  const int m = blockIdx.y * kResRowsPerGroup + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (m >= M) return;  // uniform per wavefront
  const int n = tile * 64 + lane;
  const bool in = n < N;
  const __amdgpu_buffer_rsrc_t prs = buffer_rsrc(planes, (uint32_t)((int64_t)nplanes * M * N * 4));
  float v[S];
#pragma unroll
  for (int q = 0; q < S; ++q)
    v[q] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
        prs, in && q < nplanes ? (uint32_t)(((q * M + m) * N + n) * 4) : kPastBuffer, 0, 0));
  const float hv = in ? r.h[(size_t)m * r.ldh + n] : 0.0f;
  const float wn = r.w && in ? bf16_bits_to_f32(r.w[n]) : 0.0f;
  float tot = 0.0f;
#pragma unroll
  for (int q = 0; q < S; ++q)
    if (q < nplanes) tot += v[q];
  const float hn = hv + bf16_bits_to_f32(f32_to_bf16_bits(tot));
  float sq = 0.0f;
  if (in) {
    r.h[(size_t)m * r.ldh + n] = hn;
    if (r.w) r.x[r.ldx == 0 ? (size_t)tile_elem(m, n) : (size_t)m * r.ldx + n] = f32_to_bf16_bits(hn * wn);
    sq = hn * hn;
  }
  if (r.ssq) {
    sq = row16_sum(sq);
    const float ss = (lane_value(sq, 0) + lane_value(sq, 16)) + (lane_value(sq, 32) + lane_value(sq, 48));
    if (lane == 0) r.ssq[m * r.ld + tile] = ss;
  }
}

// -------------------------------------------- MFMA kernel over 256-row bands (M >= 5)
//
// The direct-to-LDS kernel's 64-row workgroup reads, at 32 activation rows, twice as many
// activation bytes as weight bytes (x: 64 bytes per K column, the 64 rows' weights 36).
// Where that kernel would split K anyway, or declines (more 64-row tiles than CUs), the
// activation bytes are cut by a wider tile.  Here a workgroup of eight wavefronts
// owns a band of 256 weight rows (wavefront w: rows 32 w .. 32 w + 31, one 32 x 32 MFMA
// tile) over a K-range of at most 16 groups, so that the range's x is read once for 256
// rows (x: 64 bytes per K column against 144 of weights), and the bands' K-ranges are
// split toward one workgroup per CU.
//   * x: the range's activations go memory -> LDS by the buffer loads' LDS path, 16 bytes
//     a lane, in MFMA A-operand order (slot [group][k-step][lane] holds x[m][64 g + 32 kb
//     + 8 t ..+8] for lane (m, kb)); rows m >= M read row M - 1 (never stored).  After one
//     barrier each thread (group, row) puts its eight slots in pair order and writes the
//     row's group sum, so the per-group activation work is done once per workgroup instead
//     of once per wavefront.
//   * Weights: per wavefront, chunks of four groups of its 32 rows (whole 128-byte lines,
//     the direct-to-LDS kernel's swizzled slots) in a two-buffer ring: chunks 0 and 1 at
//     the start, chunk q + 2 once chunk q is read.
//   * Scales and biases of the band's rows over the range: LDS, 4 bytes a lane, with x.
// Per group (the direct-to-LDS kernel's arithmetic): P = sum_k v x from four bf16 MFMAs (v =
// 1 + q/16, exact), acc += 16 s P; per pair of groups one v_mfma_f32_32x32x2_f32 adds (b -
// 16 s) sum x.  A wavefront's tile needs no other wavefront's sums.  Without splits it
// writes its rows of y; with splits an fp32 partial, and the last split of the band to
// finish (a counter per band in the caller's workspace) adds the partials in split order
// (the same bits whatever order the splits finish in; partials and counters through sc1
// accesses).  Requires K % 256 == 0, ranges of four-group multiples and x rows 16-byte
// aligned.  Measured at M = 32 on MI355X (against the kernel the plan took before): 19456 x
// 2560 18.7 us (20.2, staged), 8192 x 4096 20.3 (21.6, direct-to-LDS in three ranges),
// 50000 x 1024 14.2 (21.8); at K = 3840 x 15360 20.5 against the direct-to-LDS kernel's
// whole-K tiles' 16.5 (the last split's serial add of three 32 KB partials costs some
// 4.5 us), so whole-K direct-to-LDS plans keep precedence.  Weights loaded straight into
// registers (16 bytes a lane, the whole range in flight) measured 20-40% slower than the
// whole-line LDS loads.
namespace bd {
constexpr int kWaves = 8;
constexpr int kRows = 32 * kWaves;       // weight rows per workgroup
constexpr int kMaxGroups = 16;           // groups of a K-range
constexpr int kChunkBytes = 32 * 128;    // four groups of a wavefront's 32 rows
constexpr int kMaxSplits = 16;
}  // namespace bd

template <bool SPLIT>
__global__ __launch_bounds__(64 * bd::kWaves) void qmv_band_kernel(LaunchArgs a, DmaArgs d) {
  __shared__ __attribute__((aligned(16))) uint4 xl[bd::kMaxGroups * 4 * 64];
  __shared__ __attribute__((aligned(16))) char wb[bd::kWaves * 2 * bd::kChunkBytes];
  __shared__ __attribute__((aligned(16))) uint32_t sbl[bd::kRows * bd::kMaxGroups];
  __shared__ float xsum[bd::kMaxGroups][32];
  __shared__ int last;
  const int pi = blockIdx.y;
  const Problem& P = a.p[pi];
  const int N = P.N, K = P.K, M = a.M, G = K >> 6;
  const int splits = SPLIT ? d.splits : 1;
  const int band = SPLIT ? (int)blockIdx.x / splits : (int)blockIdx.x;
  const int split = SPLIT ? (int)blockIdx.x - band * splits : 0;
  const int row0 = band * bd::kRows;
  if (row0 >= N) return;  // past this problem's bands
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 31, kb = lane >> 5;
  const int gs0 = SPLIT ? split * d.range : 0;
  const int gs1 = SPLIT ? min(G, gs0 + d.range) : G;
  const int Gs = __builtin_amdgcn_readfirstlane(gs1 - gs0);  // a multiple of four, <= 16
  const int nq = Gs >> 2;                                     // chunks of four groups
  const int hp = Gs >> 1;                                     // scale dwords per row
  const int wrow0 = row0 + 32 * wave;

  const __amdgpu_buffer_rsrc_t wrs = buffer_rsrc(P.w, (uint32_t)N * (uint32_t)(K >> 1));
  const uint32_t sb_bytes = (uint32_t)N * (uint32_t)G * 2u;
  const __amdgpu_buffer_rsrc_t srs = buffer_rsrc(P.s, sb_bytes);
  const __amdgpu_buffer_rsrc_t brs = buffer_rsrc(P.b, sb_bytes);
  const __amdgpu_buffer_rsrc_t xrs = buffer_rsrc(P.x, (uint32_t)(((int64_t)(M - 1) * P.ldx + K) * 2));

  __builtin_amdgcn_sched_barrier(0);
  // 1. x of the range: instruction i = 4 gl + t, lane l -> slot i * 64 + l
  {
    const uint32_t xro = (uint32_t)min(j, M - 1) * (uint32_t)P.ldx * 2u + 64u * (uint32_t)kb;
    for (int i = wave; i < 4 * Gs; i += bd::kWaves) {
      const uint32_t off = xro + 128u * (uint32_t)(gs0 + (i >> 2)) + 16u * (uint32_t)(i & 3);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          xrs, (__attribute__((address_space(3))) void*)(xl + i * 64), 16, off, 0, 0, 0);
    }
  }
  // 2. scales, then biases: 4 hp instructions of 64 dwords per array; dword dd of an array
  //    (row dd / hp, pair dd % hp of the range's groups) at LDS dword array * 256 hp + dd
  {
    const int per = 4 * hp;
    for (int i = wave; i < 2 * per; i += bd::kWaves) {
      const int arr = i >= per ? 1 : 0;
      const int ii = i - arr * per;
      const int dd = ii * 64 + lane;
      const int r = dd / hp, pr = dd - r * hp;
      const int row = row0 + r < N ? row0 + r : N - 1;
      const uint32_t off = (uint32_t)row * (uint32_t)G * 2u + 2u * (uint32_t)gs0 + 4u * (uint32_t)pr;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          arr ? brs : srs, (__attribute__((address_space(3))) void*)(sbl + arr * bd::kRows * hp + ii * 64),
          4, off, 0, 0, 0);
    }
  }
  // 3. weights: chunk q of this wavefront's rows into its buffer q & 1, 4 instructions of
  //    8 rows x 128 bytes
  char* const wbuf = wb + wave * 2 * bd::kChunkBytes;
  auto load_w = [&](int q) {
#pragma unroll
    for (int i8 = 0; i8 < 4; ++i8) {
      const int r = 8 * i8 + (lane >> 3);
      const int c = (lane & 7) ^ dm::swz(r);
      int gg = gs0 + 4 * q + (c >> 1);
      gg = gg < gs1 ? gg : gs1 - 1;
      const int row = wrow0 + r < N ? wrow0 + r : N - 1;
      const uint32_t off = (uint32_t)row * (uint32_t)(K >> 1) + 32u * (uint32_t)gg + 16u * (uint32_t)(c & 1);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          wrs, (__attribute__((address_space(3))) void*)(wbuf + (q & 1) * bd::kChunkBytes + i8 * 1024), 16, off,
          0, 0, kNt);
    }
  };
  __builtin_amdgcn_sched_barrier(0);
  load_w(0);
  if (nq > 1) load_w(1);
  __builtin_amdgcn_sched_barrier(0);
  // this wavefront's x, scales and biases have landed (its weight loads, issued after
  // them, may not have); past the barrier every wavefront's have
  if (nq > 1)
    asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  else
    asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);

  // 4. x in pair order and the rows' group sums: thread (group g, row m)
  const uint32_t one = in_vgpr(kNibOne);
  {
    const int g = tid >> 5, m = tid & 31;
    if (g < Gs) {
      uint4 v[8];
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int t = 0; t < 4; ++t) v[4 * h + t] = xl[(4 * g + t) * 64 + 32 * h + m];
      float half[2] = {0.0f, 0.0f};
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const uint4 u = v[4 * h + t];
          half[h] = dot2(u.x, one, half[h]);
          half[h] = dot2(u.y, one, half[h]);
          half[h] = dot2(u.z, one, half[h]);
          half[h] = dot2(u.w, one, half[h]);
          xl[(4 * g + t) * 64 + 32 * h + m] = pair_order(u);
        }
      xsum[g][m] = half[0] + half[1];
    }
  }
  __syncthreads();

  // 5. the range's groups, four per chunk
  const f32x16_t zero = {};
  f32x16_t acc = zero, accb = zero;
  const int rl = 32 * wave + j;  // this lane's weight row within the band
#pragma unroll
  for (int q = 0; q < bd::kMaxGroups / 4; ++q) {
    if (q >= nq) break;
    if (q + 1 < nq)
      asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    const char* buf = wbuf + (q & 1) * bd::kChunkBytes;
    uint32_t sp = 0u, bp = 0u;
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      const int gl = 4 * q + gq;
      bf16x8_t xa[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) xa[t] = as_bf16x8(xl[(4 * gl + t) * 64 + lane]);
      if ((gq & 1) == 0) {
        sp = sbl[rl * hp + (gl >> 1)];
        bp = sbl[bd::kRows * hp + rl * hp + (gl >> 1)];
      }
      const int c = 2 * gq + kb;
      const uint4 wv = *reinterpret_cast<const uint4*>(buf + (j >> 3) * 1024 + 16 * (8 * (j & 7) + (c ^ dm::swz(j))));
      f32x16_t p = zero;
      p = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xa[0], unpack16(wv.x, one), p, 0, 0, 0);
      p = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xa[1], unpack16(wv.y, one), p, 0, 0, 0);
      p = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xa[2], unpack16(wv.z, one), p, 0, 0, 0);
      p = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xa[3], unpack16(wv.w, one), p, 0, 0, 0);
      const float s16 = 16.0f * __uint_as_float((gq & 1) ? (sp & 0xffff0000u) : (sp << 16));
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[e] = fmaf(s16, p[e], acc[e]);
      if (gq & 1) {  // the pair's offset term: lanes kb = 0 / 1 take its first / second group
        const uint32_t sw = kb ? (sp & 0xffff0000u) : (sp << 16);
        const uint32_t bw = kb ? (bp & 0xffff0000u) : (bp << 16);
        const float cg = fmaf(-16.0f, __uint_as_float(sw), __uint_as_float(bw));
        accb = __builtin_amdgcn_mfma_f32_32x32x2f32(xsum[gl - 1 + kb][j], cg, accb, 0, 0, 0);
      }
    }
    if (q + 2 < nq) {
      // every read of this chunk's buffer has returned before the buffer is refilled
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
      load_w(q + 2);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  acc += accb;

  // 6. lane (n = j, kb) holds y[m][wrow0 + j] for m = 8 (e / 4) + 4 kb + e % 4
  const int n = wrow0 + j;
  if (!SPLIT) {
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int m = 8 * (e >> 2) + 4 * kb + (e & 3);
      if (m < M && n < N) store_y(a, P, m, n, acc[e]);
    }
    return;
  }
  const __amdgpu_buffer_rsrc_t prs =
      buffer_rsrc(d.partial + pi * d.pstride, (uint32_t)((int64_t)splits * M * N * 4));
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int m = 8 * (e >> 2) + 4 * kb + (e & 3);
    if (m < M && n < N) store_b32_sc1(prs, (uint32_t)(((split * M + m) * N + n) * 4), __float_as_uint(acc[e]));
  }
  wait_vmem();
  __syncthreads();
  uint32_t* cnt = d.counters + (int64_t)pi * d.tiles_max + band;
  if (tid == 0)
    last = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)(splits - 1);
  __syncthreads();
  if (!last) return;
  // four partials of each output in flight at a time, added in split order
  const uint32_t step = (uint32_t)(M * N * 4);
  float tot[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) tot[e] = 0.0f;
  for (int q0 = 0; q0 < splits; q0 += 4) {
    float v[16][4];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int m = 8 * (e >> 2) + 4 * kb + (e & 3);
      const bool in = m < M && n < N;
      const uint32_t o = (uint32_t)((m * N + n) * 4) + (uint32_t)q0 * step;
#pragma unroll
      for (int s = 0; s < 4; ++s)
        v[e][s] = __uint_as_float(load_b32_sc1(prs, in && q0 + s < splits ? o + s * step : kPastBuffer));
    }
#pragma unroll
    for (int e = 0; e < 16; ++e)
#pragma unroll
      for (int s = 0; s < 4; ++s)
        if (q0 + s < splits) tot[e] += v[e][s];
  }
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int m = 8 * (e >> 2) + 4 * kb + (e & 3);
    if (m < M && n < N) store_y(a, P, m, n, tot[e]);
  }
  if (tid == 0) st_sc1(cnt, 0u);  // ready for the next call
}

// ------------------------------------------------------------------ dequantise
//
// One thread per packed word: eight outputs.  fp32 output is fl32(s*q + b), which is
// the same value with or without a fused multiply-add because s*q is exact in fp32.

template <int OUT>  // 0 bf16, 1 fp32, 2 fp16
__global__ __launch_bounds__(kThreads) void dequant_kernel(const uint32_t* __restrict__ w,
                                                           const uint16_t* __restrict__ s,
                                                           const uint16_t* __restrict__ b,
                                                           void* __restrict__ out, int64_t words,
                                                           int32_t K) {
  const int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (t >= words) return;
  const int32_t W = K >> 3;
  const int64_t n = t / W;
  const int32_t wi = (int32_t)(t - n * W);
  const int64_t gidx = n * (K >> 6) + (wi >> 3);
  const float sc = bf16_bits_to_f32(s[gidx]);
  const float bi = bf16_bits_to_f32(b[gidx]);
  const uint32_t u = w[t];
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = fmaf(sc, (float)((u >> (4 * e)) & 0xFu), bi);
  if (OUT == 1) {
    float4* o = reinterpret_cast<float4*>(reinterpret_cast<float*>(out) + t * 8);
    o[0] = make_float4(v[0], v[1], v[2], v[3]);
    o[1] = make_float4(v[4], v[5], v[6], v[7]);
  } else {
    uint32_t h[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      uint32_t lo, hi;
      if (OUT == 0) {
        lo = f32_to_bf16_bits(v[2 * e]);
        hi = f32_to_bf16_bits(v[2 * e + 1]);
      } else {
        lo = __half_as_ushort(__float2half_rn(v[2 * e]));
        hi = __half_as_ushort(__float2half_rn(v[2 * e + 1]));
      }
      h[e] = lo | (hi << 16);
    }
    *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(out) + t * 8) =
        make_uint4(h[0], h[1], h[2], h[3]);
  }
}

// Zeroes `words` 32-bit words (the split counters before a call that uses the library's
// static scratch; a kernel rather than a memset so the call stays capturable in a graph).
__global__ __launch_bounds__(kThreads) void clear_words_kernel(uint32_t* __restrict__ p, int words) {
  const int i = blockIdx.x * kThreads + threadIdx.x;
  if (i < words) p[i] = 0u;
}

}  // namespace

// ------------------------------------------------------ static split scratch
//
// The split workspace of imq_qmv_grouped_noalloc: device memory of the library itself, one
// copy per device (each holds it until the process ends), so that entry point calls no
// allocator.  Host code never passes `scratch` itself to a kernel (on the host the name is
// a stand-in, not a device address): the per-device address comes from
// hipGetSymbolAddress, once per device, and only that address is used.
static __device__ __align__(256) char scratch[IMQ_NOALLOC_SCRATCH_BYTES];

namespace {

struct ScratchSlot {
  std::once_flag once;
  void* ptr = nullptr;
  hipError_t err = hipSuccess;
};
ScratchSlot g_scratch[imq_rt::kMaxDevices];

// The current device's address of `scratch` (looked up once per device, with that device
// current), or nullptr with *code set.
void* scratch_address(int32_t* code) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= imq_rt::kMaxDevices) {
    *code = imq_rt::fail(IMQ_EUNAVAILABLE, "no HIP device is available");
    return nullptr;
  }
  ScratchSlot& s = g_scratch[dev];
  std::call_once(s.once, [&s] { s.err = hipGetSymbolAddress(&s.ptr, HIP_SYMBOL(scratch)); });
  if (s.err != hipSuccess || s.ptr == nullptr) {
    *code = imq_rt::fail(IMQ_ELAUNCH, std::string("hipGetSymbolAddress(scratch) failed: ") +
                                          hipGetErrorString(s.err));
    return nullptr;
  }
  return s.ptr;
}

// ================================================================== host side

using imq_rt::aligned;
using imq_rt::current_device;
using imq_rt::DeviceInfo;
using imq_rt::fail;
using imq_rt::ok;


int32_t check_format(int32_t N, int32_t K, int32_t group_size, int32_t bits) {
  if (bits != 4) return fail(IMQ_EUNSUPPORTED, "only 4-bit weights are supported");
  if (group_size != kGroup) return fail(IMQ_EUNSUPPORTED, "only group size 64 is supported");
  if (N < 1) return fail(IMQ_EINVAL, "N must be >= 1");
  if (K < kGroup || K % kGroup != 0) return fail(IMQ_EINVAL, "K must be a positive multiple of 64");
  return IMQ_OK;
}

int32_t check_weights(const uint32_t* w, const uint16_t* s, const uint16_t* b) {
  if (!w || !s || !b) return fail(IMQ_EINVAL, "w, scales and biases must be non-null");
  if (!aligned(w, 16)) return fail(IMQ_EINVAL, "w must be 16-byte aligned");
  if (!aligned(s, 2) || !aligned(b, 2)) return fail(IMQ_EINVAL, "scales/biases must be 2-byte aligned");
  return IMQ_OK;
}

int32_t check_dtype(int32_t y_dtype) {
  if (y_dtype != IMQ_BF16 && y_dtype != IMQ_F32) return fail(IMQ_EINVAL, "y_dtype must be bf16 or fp32");
  return IMQ_OK;
}

int32_t check_rows(const uint16_t* x, int64_t ldx, const void* y, int64_t ldy, int32_t M, int32_t N,
                   int32_t K, int32_t y_dtype) {
  if (M < 1) return fail(IMQ_EINVAL, "M must be >= 1");
  if (M > IMQ_MAX_ROWS) return fail(IMQ_EUNSUPPORTED, "M must be <= 32");
  if (!x || !y) return fail(IMQ_EINVAL, "x and y must be non-null");
  if (M > 1 && (ldx < K || ldx % 8 != 0)) return fail(IMQ_EINVAL, "ldx must be >= K and a multiple of 8");
  if (M > 1 && ldy < N) return fail(IMQ_EINVAL, "ldy must be >= N");
  if (!aligned(x, 16)) return fail(IMQ_EINVAL, "x must be 16-byte aligned");
  if (!aligned(y, y_dtype == IMQ_F32 ? 4 : 2)) return fail(IMQ_EINVAL, "y is misaligned");
  return IMQ_OK;
}

// Which kernel serves M rows: the VALU dot2 kernel while M is small and the largest x of
// the launch fits in LDS, the MFMA kernel otherwise.
constexpr int kValuMaxRows = 2;
constexpr size_t kValuLdsLimit = 64 * 1024;

// Lanes per weight row for the VALU kernels: the widest of 64/32/16 that still gives
// each lane at least four 16-byte chunks with at most 10% of the lanes' chunks idle.
int choose_lpr_shift(int K) {
  const int C = K / 32;
  for (int sh = 6; sh >= 4; --sh) {
    const int lpr = 1 << sh;
    const int nch = (C + lpr - 1) / lpr;
    if (nch >= 4 && 10 * C >= 9 * lpr * nch) return sh;
  }
  return 4;
}

// Tiles of the generic VALU kernel: 4 wavefronts x 64/LPR rows.  Returns the LDS bytes
// for the largest x of the launch (0 if some x does not fit) and the grid width.
size_t plan_rows(LaunchArgs& a, int* grid_x) {
  size_t lds = 0;
  int tiles = 0;
  for (int i = 0; i < a.count; ++i) {
    Problem& P = a.p[i];
    P.lpr_shift = choose_lpr_shift(P.K);
    const int rows = kThreads >> P.lpr_shift;
    const int t = (P.N + rows - 1) / rows;
    tiles = t > tiles ? t : tiles;
    const size_t need = (size_t)a.M * (P.K / 32) * (64 + 4);
    lds = need > lds ? need : lds;
  }
  if (lds > kValuLdsLimit) return 0;
  *grid_x = tiles;
  return lds;
}

// Batch size (16-byte chunks per lane) that wastes the fewest chunk slots, weighted by
// each problem's weight bytes.
int choose_batch(const LaunchArgs& a, const int* options, int n_options) {
  int best = options[0];
  double best_waste = 1e300;
  for (int o = 0; o < n_options; ++o) {
    const int B = options[o];
    double waste = 0;
    for (int i = 0; i < a.count; ++i) {
      const Problem& P = a.p[i];
      const int lpr = 1 << P.lpr_shift;
      const int nch = (P.K / 32 + lpr - 1) / lpr;
      const int nb = (nch + B - 1) / B;
      waste += (double)P.N * P.K * (nb * B - nch) / (nb * B);
    }
    if (waste < best_waste) {
      best_waste = waste;
      best = B;
    }
  }
  return best;
}

// The one-row kernel's plan: per problem the lane shape of m1_lane_shift (the narrowest
// row of 16, 32 or 64 lanes with at most 5 chunks per lane, else 8), then the launch's
// chunk and x-piece bounds.  Returns false when some problem does not qualify (K over
// 16384, scales/biases not 4-byte aligned, weights of 2 GiB or more).

struct M1Plan {
  int nch = 0;  // chunks per lane, largest over the problems
  int xr = 0;   // x pieces per thread, largest over the problems
  int grid_x = 0;
};

bool plan_m1(LaunchArgs& a, M1Plan* plan) {
  M1Plan pl;
  for (int i = 0; i < a.count; ++i) {
    Problem& P = a.p[i];
    const int C = P.K / 32;
    const int sh = m1_lane_shift(P.K);
    if (sh < 0) return false;
    if (!aligned(P.s, 4) || !aligned(P.b, 4)) return false;
    if ((int64_t)P.N * (P.K / 2) >= ((int64_t)1 << 31)) return false;
    P.lpr_shift = sh;
    P.nch = (C + (1 << sh) - 1) >> sh;
    const int rows = kThreads >> sh;
    const int tiles = (P.N + rows - 1) / rows;
    const int xr = (P.K / 8 + kThreads - 1) / kThreads;
    pl.nch = P.nch > pl.nch ? P.nch : pl.nch;
    pl.xr = xr > pl.xr ? xr : pl.xr;
    pl.grid_x = tiles > pl.grid_x ? tiles : pl.grid_x;
  }
  if (pl.xr > 8) return false;
  *plan = pl;
  return true;
}

template <int NCH, int XR>
hipError_t launch_m1(const LaunchArgs& a, const M1Plan& pl, hipStream_t stream) {
  constexpr size_t lds = M1Lds<NCH, XR>::kBytes;
  if (a.count <= kM1Compact) {
    M1Args c;
    memset(&c, 0, sizeof(c));
    c.count = a.count;
    c.y_f32 = a.y_f32;
    int tiles = 0;
    for (int i = 0; i < a.count; ++i) {
      const Problem& P = a.p[i];
      tiles += (P.N + (kThreads >> P.lpr_shift) - 1) / (kThreads >> P.lpr_shift);
      c.tile_end[i] = tiles;
      c.N[i] = P.N;
      c.K[i] = P.K;
      c.sh[i] = P.lpr_shift;
      c.nch[i] = P.nch;
      c.w[i] = P.w;
      c.s[i] = P.s;
      c.b[i] = P.b;
      c.x[i] = a.table ? a.xt[0] : P.x;
      c.y[i] = a.table ? a.yt[0] : P.y;
    }
    hipLaunchKernelGGL((qmv_m1c_kernel<NCH, XR>), dim3(tiles), dim3(kThreads), lds, stream, c);
  } else {
    hipLaunchKernelGGL((qmv_m1_kernel<NCH, XR>), dim3(pl.grid_x, a.count), dim3(kThreads), lds,
                       stream, a);
  }
  return hipGetLastError();
}

// The instantiation that covers the plan with the fewest idle loads: 2, 5 or 8 chunks
// per lane, 2, 5 or 8 x pieces per thread (NCH <= 2 means K <= 1024, so XR = 2 there).
hipError_t launch_m1_for(const LaunchArgs& a, const M1Plan& pl, hipStream_t stream) {
  if (pl.nch <= 2 && pl.xr <= 2) return launch_m1<2, 2>(a, pl, stream);
  if (pl.nch <= 5) {
    if (pl.xr <= 2) return launch_m1<5, 2>(a, pl, stream);
    if (pl.xr <= 5) return launch_m1<5, 5>(a, pl, stream);
  }
  if (pl.xr <= 2) return launch_m1<8, 2>(a, pl, stream);
  if (pl.xr <= 5) return launch_m1<8, 5>(a, pl, stream);
  return launch_m1<8, 8>(a, pl, stream);
}

template <int NCH, int XR, int MR>
hipError_t launch_mr(const LaunchArgs& a, const M1Plan& pl, hipStream_t stream) {
  constexpr size_t lds = M1Lds<NCH, XR, MR>::kBytes;
  static_assert(lds <= 64 * 1024, "the few-row tile stays within 64 KiB of LDS");
  hipLaunchKernelGGL((qmv_mr_kernel<NCH, XR, MR>), dim3(pl.grid_x, a.count), dim3(kThreads), lds,
                     stream, a);
  return hipGetLastError();
}

// Two to four rows through the one-row tile: two rows with x pieces per thread <= 5 (K <=
// 10240), three or four with <= 2 (K <= 4096); false for the other plans.
template <int MR>
bool launch_mr_for(const LaunchArgs& a, const M1Plan& pl, hipStream_t stream, hipError_t* e) {
  if (pl.nch <= 2 && pl.xr <= 2) *e = launch_mr<2, 2, MR>(a, pl, stream);
  else if (pl.nch <= 5 && pl.xr <= 2) *e = launch_mr<5, 2, MR>(a, pl, stream);
  else if (pl.xr <= 2) *e = launch_mr<8, 2, MR>(a, pl, stream);
  else if (MR > 2) return false;
  else if (pl.nch <= 5 && pl.xr <= 5) *e = launch_mr<5, 5, 2>(a, pl, stream);
  else if (pl.xr <= 5) *e = launch_mr<8, 5, 2>(a, pl, stream);
  else return false;
  return true;
}

template <int M, int B>
hipError_t launch_rows(const LaunchArgs& a, int grid_x, size_t lds, hipStream_t stream) {
  hipLaunchKernelGGL((qmv_rows_kernel<M, B>), dim3(grid_x, a.count), dim3(kThreads), lds, stream,
                     a);
  return hipGetLastError();
}

// The 32 x 32 MFMA kernel's plan: tiles of 32 rows and, when a workspace is given,
// enough splits of the groups that the launch has about two workgroups per CU, each
// split keeping at least 8 groups (2 per wavefront), at most kMaxSplits of them, and the
// partials' traffic small next to the weights' (8 * splits * M * N bytes against
// N * K / 2).  Workspace layout: a fixed region of kCounterBytes for the per-tile
// counters (problem i's tile t at word i * grid_x + t; zero before the first call, and
// every call leaves them at zero), then each problem's fp32 partials (splits * M * N,
// pstride floats apart).  The counter region has the same place and size for every
// launch, so calls of different shapes can share one workspace.
constexpr size_t kCounterBytes = 64 * 1024;

struct MmaPlan {
  bool staged = false;  // qmv_mma_staged_kernel (else qmv_mma_kernel)
  int nt = 1;           // qmv_mma_kernel: 32-row weight tiles per wavefront
  int grid_x = 0;
  int splits = 1;
  int64_t pstride = 0;  // floats per problem in the workspace
  size_t bytes = 0;     // workspace the plan uses (0: no split)
};

#ifndef IMQ_MMA_NT_ROWS
#define IMQ_MMA_NT_ROWS 8192
#endif

// The staged kernel's plan, when it applies: every K a multiple of 256, x rows strided (no
// pointer table) with every row offset inside a 2 GiB buffer, and either at least 0.3
// workgroups per CU without splitting (64-row tiles), or K >= 4096 with a workspace, the
// groups split toward about one workgroup per CU (at most kMaxSplitsStaged ways, at least
// 16 groups per split).  (Measured on MI355X at M = 4..32, Qwen3-4B projections and the
// K = 3840 shape: these are the launches where it beats qmv_mma_kernel.)
bool plan_staged(const LaunchArgs& a, size_t ws_bytes, int cu_count, MmaPlan* pl) {
  if (a.table) return false;
  int tiles = 0, gmin = 1 << 30, nmax = 0, grid_x = 0;
  for (int i = 0; i < a.count; ++i) {
    const Problem& P = a.p[i];
    if (P.K % 256 != 0) return false;
    if ((int64_t)(a.M - 1) * P.ldx * 2 + (int64_t)P.K * 2 >= ((int64_t)1 << 31)) return false;
    const int t = (P.N + staged::kRows - 1) / staged::kRows;
    tiles += t;
    grid_x = t > grid_x ? t : grid_x;
    gmin = P.K / 64 < gmin ? P.K / 64 : gmin;
    nmax = P.N > nmax ? P.N : nmax;
  }
  if ((size_t)a.count * grid_x * 4 > kCounterBytes) return false;
  int sp = 1;
  if (10 * tiles < 3 * cu_count) {
    if (gmin < 64 || ws_bytes <= kCounterBytes) return false;
    sp = (15 * cu_count + 16 * tiles - 1) / (16 * tiles);
    sp = sp < staged::kMaxSplitsStaged ? sp : staged::kMaxSplitsStaged;
    sp = sp < gmin / 16 ? sp : gmin / 16;
    while (sp > 1 && kCounterBytes + (size_t)a.count * sp * a.M * nmax * sizeof(float) > ws_bytes) --sp;
    if (sp < 2 || (int64_t)sp * a.M * nmax * 4 >= ((int64_t)1 << 31)) return false;
  }
  pl->staged = true;
  pl->grid_x = grid_x;
  pl->splits = sp;
  if (sp > 1) {
    pl->pstride = (int64_t)sp * a.M * nmax;
    pl->bytes = kCounterBytes + (size_t)a.count * pl->pstride * sizeof(float);
  }
  return true;
}

MmaPlan plan_mma(const LaunchArgs& a, size_t ws_bytes, int cu_count) {
  MmaPlan pl;
  if (plan_staged(a, ws_bytes, cu_count, &pl)) return pl;
  int ntotal = 0;
  for (int i = 0; i < a.count; ++i) ntotal += a.p[i].N;
  pl.nt = ntotal >= IMQ_MMA_NT_ROWS ? 2 : 1;  // wide launches share x over two tiles
  int tiles = 0, gmin = 1 << 30, kmin = 1 << 30, nmax = 0;
  for (int i = 0; i < a.count; ++i) {
    const int t = (a.p[i].N + 32 * pl.nt - 1) / (32 * pl.nt);
    pl.grid_x = t > pl.grid_x ? t : pl.grid_x;
    tiles += t;
    gmin = a.p[i].K / 64 < gmin ? a.p[i].K / 64 : gmin;
    kmin = a.p[i].K < kmin ? a.p[i].K : kmin;
    nmax = a.p[i].N > nmax ? a.p[i].N : nmax;
  }
  if (ws_bytes <= kCounterBytes || (size_t)a.count * pl.grid_x * 4 > kCounterBytes) return pl;
  int sp = (2 * cu_count + tiles - 1) / tiles;
  sp = sp < gmin / 8 ? sp : gmin / 8;
  sp = sp < kmin / (16 * a.M) ? sp : kmin / (16 * a.M);
  sp = sp < kMaxSplits ? sp : kMaxSplits;
  while (sp > 1 && kCounterBytes + (size_t)a.count * sp * a.M * nmax * sizeof(float) > ws_bytes) --sp;
  if (sp > 1 && (int64_t)sp * a.M * nmax * 4 < ((int64_t)1 << 31)) {
    pl.splits = sp;
    pl.pstride = (int64_t)sp * a.M * nmax;
    pl.bytes = kCounterBytes + (size_t)a.count * pl.pstride * sizeof(float);
  }
  return pl;
}

template <int NT>
void launch_mma_nt(const LaunchArgs& a, const MmaPlan& pl, void* ws, hipStream_t stream) {
  if (pl.splits == 1) {
    hipLaunchKernelGGL((qmv_mma_kernel<NT, false>), dim3(pl.grid_x, a.count), dim3(kThreads), 0,
                       stream, a, 1, nullptr, (int64_t)0, nullptr, 0);
  } else {
    uint32_t* counters = static_cast<uint32_t*>(ws);
    float* partial = reinterpret_cast<float*>(static_cast<char*>(ws) + kCounterBytes);
    hipLaunchKernelGGL((qmv_mma_kernel<NT, true>), dim3(pl.grid_x, a.count * pl.splits),
                       dim3(kThreads), 0, stream, a, pl.splits, partial, pl.pstride, counters,
                       pl.grid_x);
  }
}

hipError_t launch_mma(const LaunchArgs& a, const MmaPlan& pl, void* ws, hipStream_t stream) {
  if (pl.staged) {
    if (pl.splits == 1) {
      hipLaunchKernelGGL((qmv_mma_staged_kernel<false>), dim3(pl.grid_x, a.count), dim3(kThreads),
                         0, stream, a, 1, nullptr, (int64_t)0, nullptr, 0, NormIn{});
    } else {
      uint32_t* counters = static_cast<uint32_t*>(ws);
      float* partial = reinterpret_cast<float*>(static_cast<char*>(ws) + kCounterBytes);
      hipLaunchKernelGGL((qmv_mma_staged_kernel<true>), dim3(pl.grid_x, a.count * pl.splits),
                         dim3(kThreads), 0, stream, a, pl.splits, partial, pl.pstride, counters,
                         pl.grid_x, NormIn{});
    }
    return hipGetLastError();
  }
  if (pl.nt == 2)
    launch_mma_nt<2>(a, pl, ws, stream);
  else
    launch_mma_nt<1>(a, pl, ws, stream);
  return hipGetLastError();
}

// The x-stationary kernel's plan: per problem 32-row tiles and the whole K in one range
// (at most Shape<MB>::kRange groups: K <= 4096), MB = 1 m-block for M <= 16, else 2.  Each
// workgroup takes every r-th tile of its problem, r = ceil(tiles / CUs), so that its x is
// loaded once for r tiles.  The kernel carries a fixed cost per workgroup (x into
// registers) and per tile (the cross-wavefront reduction and the staged scales) that only
// many tiles per workgroup amortise: measured on MI355X it beats the staged MFMA kernel on
// the LM head (151936 x 2560: 72 against 84-95 us at M = 32) and loses on launches of 1-3
// tiles per CU (C3 15360 x 3840, the decoder layer's projections), so it takes launches with
// at least kXsMinTilesPerCu tiles per CU.  Not applicable: K % 256 != 0, K > 4096, or a
// pointer table.
#ifndef IMQ_XS_MIN_TILES_PER_CU
#define IMQ_XS_MIN_TILES_PER_CU 8
#endif

struct XsPlan {
  int mb = 1;           // m-blocks of 16 activation rows
  int gw = 0;           // groups per wavefront of the instantiation
  int grid = 0;
  size_t lds = 0;
};

bool plan_xs(const LaunchArgs& a, int cu_count, XsArgs* xa, XsPlan* pl) {
  if (a.count > kMaxProblems || a.table) return false;
  const int mb = a.M <= 16 ? 1 : 2;
  const int waves = mb == 1 ? xs::Shape<1>::kWaves : xs::Shape<2>::kWaves;
  int ttot = 0, gmax = 0;
  for (int i = 0; i < a.count; ++i) {
    const Problem& P = a.p[i];
    if (P.K % 256 != 0 || P.K / 64 > xs::Shape<1>::kRange) return false;
    if ((int64_t)(a.M - 1) * P.ldx * 2 + (int64_t)P.K * 2 >= ((int64_t)1 << 31)) return false;
    if (((int64_t)(a.M - 1) * P.ldy + P.N) * 4 >= ((int64_t)1 << 31)) return false;
    ttot += (P.N + xs::kRows - 1) / xs::kRows;
    gmax = P.K / 64 > gmax ? P.K / 64 : gmax;
  }
  if (ttot < IMQ_XS_MIN_TILES_PER_CU * cu_count) return false;
  const int per_wave = (gmax + waves - 1) / waves;
  if (per_wave > (mb == 1 ? 4 : 8)) return false;
  pl->mb = mb;
  pl->gw = per_wave <= 2 ? 2 : per_wave == 7 ? 8 : per_wave;
  const int r = (ttot + cu_count - 1) / cu_count;
  memset(xa, 0, sizeof(*xa));
  int wg = 0;
  for (int i = 0; i < a.count; ++i) {
    const Problem& P = a.p[i];
    XsProblem& X = xa->p[i];
    X.w = P.w;
    X.s = P.s;
    X.b = P.b;
    X.x = P.x;
    X.y = P.y;
    X.ldx = P.ldx;
    X.ldy = P.ldy;
    X.N = P.N;
    X.K = P.K;
    X.tiles = (P.N + xs::kRows - 1) / xs::kRows;
    X.wgs = (X.tiles + r - 1) / r;
    X.wg0 = wg;
    wg += X.wgs;
  }
  xa->count = a.count;
  xa->M = a.M;
  xa->y_f32 = a.y_f32;
  xa->scs = gmax | 1;
  pl->grid = wg;
  // the parked partials (the x staging areas before them), then the staged scales and
  // biases and the spare slots (bl's spare at 2 * 32 * scs from bl: 3 * 32 * scs + 4 floats
  // from the start of the staging)
  pl->lds = (mb == 1 ? xs::area_bytes<1>() : xs::area_bytes<2>()) +
            ((size_t)3 * xs::kRows * xa->scs + 4) * sizeof(float);
  return true;
}

template <int MB, int GW, bool Y32>
hipError_t launch_xs_one(const XsArgs& x, const XsPlan& pl, hipStream_t stream) {
  auto kern = qmv_xs_kernel<MB, GW, xs::Shape<MB>::kDepth, Y32>;
  static_assert(xs::area_bytes<MB>() + ((size_t)3 * xs::kRows * 65 + 4) * sizeof(float) <= 64 * 1024,
                "every plan (scs <= 65) stays within the default 64 KiB of dynamic LDS");
  hipLaunchKernelGGL(kern, dim3(pl.grid), dim3(64 * xs::Shape<MB>::kWaves), pl.lds, stream, x);
  return hipGetLastError();
}

template <int MB, int GW>
hipError_t launch_xs_gw(const XsArgs& x, const XsPlan& pl, hipStream_t stream) {
  return x.y_f32 ? launch_xs_one<MB, GW, true>(x, pl, stream) : launch_xs_one<MB, GW, false>(x, pl, stream);
}

hipError_t launch_xs(const XsArgs& x, const XsPlan& pl, hipStream_t stream) {
  if (pl.mb == 1) {
    switch (pl.gw) {
      case 2: return launch_xs_gw<1, 2>(x, pl, stream);
      case 3: return launch_xs_gw<1, 3>(x, pl, stream);
      default: return launch_xs_gw<1, 4>(x, pl, stream);
    }
  }
  switch (pl.gw) {
    case 2: return launch_xs_gw<2, 2>(x, pl, stream);
    case 3: return launch_xs_gw<2, 3>(x, pl, stream);
    case 4: return launch_xs_gw<2, 4>(x, pl, stream);
    case 5: return launch_xs_gw<2, 5>(x, pl, stream);
    case 6: return launch_xs_gw<2, 6>(x, pl, stream);
    default: return launch_xs_gw<2, 8>(x, pl, stream);
  }
}

// The direct-to-LDS kernel's plan.  64-row tiles; the groups of a tile split into K-ranges
// (multiples of four groups, at most 64) so that the launch has about three quarters of a
// workgroup per CU (dma_splits), GMAX = 4 groups per wavefront for ranges up to 32 groups,
// else 8, and W = range / GMAX wavefronts.  The workspace holds the split counters and
// partials (none without splits).  Not applicable: a pointer table, M outside [3, 32],
// K % 256 != 0, problems of different K with splits, x rows not 16-byte aligned, offsets
// past 2 GiB, or more tile counters than the counter region holds.
#ifndef IMQ_DMA_MIN_ROWS
#define IMQ_DMA_MIN_ROWS 5
#endif


struct DmaPlan {
  int waves = 0;
  int gmax = 0;
  int grid_x = 0;          // tiles of the largest problem
  int splits = 1;
  int range = 0;           // groups per K-range
  size_t pstride = 0;      // partial floats per problem
  size_t bytes = 0;        // workspace the plan uses
};

int dma_splits(int tiles, int groups, int cu_count);

bool plan_dma(const LaunchArgs& a, int cu_count, DmaPlan* pl) {
  if (a.table || a.M < 3 || a.M > 32 || a.count < 1 || a.count > kMaxProblems) return false;
  int tiles = 0, grid_x = 0, gmax = 0, gmin = 1 << 30, nmax = 0;
  for (int i = 0; i < a.count; ++i) {
    const Problem& P = a.p[i];
    if (P.K % 256 != 0 || P.N < 1) return false;
    if ((int64_t)P.N * (P.K / 2) >= ((int64_t)1 << 31)) return false;
    if (P.ldx % 8 != 0 || !imq_rt::aligned(P.x, 16)) return false;
    if (((int64_t)(a.M - 1) * P.ldx + P.K) * 2 >= ((int64_t)1 << 31)) return false;
    if (((int64_t)(a.M - 1) * P.ldy + P.N) * 4 >= ((int64_t)1 << 31)) return false;
    const int t = (P.N + dm::kRows - 1) / dm::kRows;
    tiles += t;
    grid_x = t > grid_x ? t : grid_x;
    gmax = P.K / 64 > gmax ? P.K / 64 : gmax;
    gmin = P.K / 64 < gmin ? P.K / 64 : gmin;
    nmax = P.N > nmax ? P.N : nmax;
  }
  int splits = dma_splits(tiles, gmax, cu_count);
  if (splits == 0 || (splits > 1 && gmin != gmax)) return false;  // one range layout for all
  int range = (gmax + splits - 1) / splits;
  range = (range + 3) / 4 * 4;
  if (range > dm::kMaxGroups) return false;
  splits = (gmax + range - 1) / range;
  if (splits > dm::kMaxSplits) return false;
  if ((size_t)a.count * grid_x * 4 > kCounterBytes) return false;
  if (splits > 1 && ((int64_t)splits * a.M * nmax) * 4 >= ((int64_t)1 << 31)) return false;
  pl->splits = splits;
  pl->range = range;
  pl->gmax = range <= 32 ? 4 : 8;
  const int w = (range + pl->gmax - 1) / pl->gmax;
  pl->waves = w <= 2 ? 2 : w <= 6 ? w : 8;  // instantiated: 2, 3, 4, 5, 6, 8
  pl->grid_x = grid_x;
  pl->pstride = splits > 1 ? (size_t)splits * a.M * nmax : 0;
  pl->bytes = splits > 1 ? kCounterBytes + (size_t)a.count * pl->pstride * sizeof(float) : 0;
  return true;
}

// The direct-to-LDS plan for the fused-norm calls, which only this kernel serves: the
// usual plan where it applies, else whole-K tiles (or the fewest K-ranges of at most 64
// groups) at any M from 1 and any tile count.
bool plan_dma_norm(const LaunchArgs& a, int cu_count, DmaPlan* pl) {
  if (a.M >= 3 && plan_dma(a, cu_count, pl)) return true;
  if (a.table || a.M < 1 || a.M > 32 || a.count < 1 || a.count > kMaxProblems) return false;
  int grid_x = 0, gmax = 0, gmin = 1 << 30, nmax = 0;
  for (int i = 0; i < a.count; ++i) {
    const Problem& P = a.p[i];
    if (P.K % 256 != 0 || P.N < 1) return false;
    if ((int64_t)P.N * (P.K / 2) >= ((int64_t)1 << 31)) return false;
    if (P.ldx % 8 != 0 || !imq_rt::aligned(P.x, 16)) return false;
    if (((int64_t)(a.M - 1) * P.ldx + P.K) * 2 >= ((int64_t)1 << 31)) return false;
    const int t = (P.N + dm::kRows - 1) / dm::kRows;
    grid_x = t > grid_x ? t : grid_x;
    gmax = P.K / 64 > gmax ? P.K / 64 : gmax;
    gmin = P.K / 64 < gmin ? P.K / 64 : gmin;
    nmax = P.N > nmax ? P.N : nmax;
  }
  int splits = (gmax + dm::kMaxGroups - 1) / dm::kMaxGroups;
  if (splits > 1 && gmin != gmax) return false;
  int range = ((gmax + splits - 1) / splits + 3) / 4 * 4;
  splits = (gmax + range - 1) / range;
  if (splits > dm::kMaxSplits || (size_t)a.count * grid_x * 4 > kCounterBytes) return false;
  if (splits > 1 && ((int64_t)splits * a.M * nmax) * 4 >= ((int64_t)1 << 31)) return false;
  pl->splits = splits;
  pl->range = range;
  pl->gmax = range <= 32 ? 4 : 8;
  const int w = (range + pl->gmax - 1) / pl->gmax;
  pl->waves = w <= 2 ? 2 : w <= 6 ? w : 8;
  pl->grid_x = grid_x;
  pl->pstride = splits > 1 ? (size_t)splits * a.M * nmax : 0;
  pl->bytes = splits > 1 ? kCounterBytes + (size_t)a.count * pl->pstride * sizeof(float) : 0;
  return true;
}

// K-ranges per tile, 0 to decline.  Measured on MI355X at M = 32 (one call, against the
// other kernels' best): launches of more than half a tile per CU run whole-K tiles (K =
// 3840 x 15360, 240 tiles: 16.3 us against 19.5; any split lost); smaller ones split into
// ranges of at most 28 groups and into at least 0.6 workgroups per CU: the q/k/v
// projections of a 2560-wide decoder layer (96 tiles) in two ranges 11.4 us against 14.0,
// its o projection (K = 4096, 40 tiles) in four 10.1 against 12.4, its down projection (K =
// 9728) in six 12.6 against 15.5, K = 2560 x 2560 in four 10.0 against 11.2.  Launches of
// more tiles than CUs stay with the staged kernel (the 2 x 9728 x 2560 gate/up launch: 21.3
// at best against 19.9), and so do splits into ranges under 8 groups.
int dma_splits(int tiles, int groups, int cu_count) {
  if (tiles > cu_count) return 0;
  if (2 * tiles > cu_count) return (groups + dm::kMaxGroups - 1) / dm::kMaxGroups;
  const int by_range = (groups + 27) / 28;
  const int by_count = (6 * cu_count + 5 * tiles) / (10 * tiles);
  const int s = by_range > by_count ? by_range : by_count;
  if (s <= 1) return 1;
  const int range = ((groups + s - 1) / s + 3) / 4 * 4;
  return range >= 8 ? s : 0;
}

// The launches the direct-to-LDS kernel takes: from IMQ_DMA_MIN_ROWS rows any it plans,
// and from 3 rows those of whole-K tiles, where the few-row VALU tile is slower (K = 3840 x
// 15360: 16.3 us at M = 4 against about 13 us here) while it stays ahead on smaller
// launches (K = 2560 x 2560 at M = 4: 5.9 us against about 10).
bool take_dma(const LaunchArgs& a, int cu_count, DmaPlan* pl) {
  if (a.M < 3 || !plan_dma(a, cu_count, pl)) return false;
  return a.M >= IMQ_DMA_MIN_ROWS || pl->splits == 1;
}

// The 256-row band kernel's plan: K-ranges of at most 16 groups (four-group multiples)
// toward one workgroup per CU, and at least half a workgroup per CU.  Single-weight
// launches only: grouped launches keep the staged and direct-to-LDS plans, whose bits the
// fused gate/up entry (imq_qmv_gate_up_silu) reproduces.  Not applicable either: a pointer
// table, M outside [IMQ_BAND_MIN_ROWS, 32], K % 256 != 0, x rows not 16-byte aligned,
// offsets past 2 GiB, or more band counters than the counter region holds.
// From 5 rows, as the direct-to-LDS kernel (measured at M = 5 / 8 / 12: 50000 x 1024 11.4 /
// 11.5 / 12.0 us against 17.8 / 17.9 / 19.0, 19456 x 2560 15.5 / 15.6 / 16.3 against 17.7 /
// 17.7 / 18.3, 8192 x 4096 16.1 / 16.1 / 17.2 against 17.7 / 18.0 / 18.5)
#ifndef IMQ_BAND_MIN_ROWS
#define IMQ_BAND_MIN_ROWS 5
#endif

struct BandPlan {
  int grid_x = 0;      // bands of the largest problem
  int splits = 1;
  int range = 0;       // groups per K-range
  size_t pstride = 0;  // partial floats per problem
  size_t bytes = 0;    // workspace the plan uses
};

bool plan_band(const LaunchArgs& a, int cu_count, BandPlan* pl) {
  if (a.table || a.M < IMQ_BAND_MIN_ROWS || a.M > 32 || a.count != 1) return false;
  int bands = 0, grid_x = 0, gmax = 0, gmin = 1 << 30, nmax = 0;
  for (int i = 0; i < a.count; ++i) {
    const Problem& P = a.p[i];
    if (P.K % 256 != 0 || P.N < 1) return false;
    if ((int64_t)P.N * (P.K / 2) >= ((int64_t)1 << 31)) return false;
    if (P.ldx % 8 != 0 || !imq_rt::aligned(P.x, 16)) return false;
    if (((int64_t)(a.M - 1) * P.ldx + P.K) * 2 >= ((int64_t)1 << 31)) return false;
    if (((int64_t)(a.M - 1) * P.ldy + P.N) * 4 >= ((int64_t)1 << 31)) return false;
    const int t = (P.N + bd::kRows - 1) / bd::kRows;
    bands += t;
    grid_x = t > grid_x ? t : grid_x;
    gmax = P.K / 64 > gmax ? P.K / 64 : gmax;
    gmin = P.K / 64 < gmin ? P.K / 64 : gmin;
    nmax = P.N > nmax ? P.N : nmax;
  }
  int splits = (gmax + bd::kMaxGroups - 1) / bd::kMaxGroups;
  const int by_count = (cu_count + bands / 2) / bands;
  splits = by_count > splits ? by_count : splits;
  int range = ((gmax + splits - 1) / splits + 3) / 4 * 4;
  range = range < 8 ? (gmax < 8 ? gmax : 8) : range;
  splits = (gmax + range - 1) / range;
  if (2 * bands * splits < cu_count) return false;
  if (splits > bd::kMaxSplits || (splits > 1 && gmin != gmax)) return false;
  if ((size_t)a.count * grid_x * 4 > kCounterBytes) return false;
  if (splits > 1 && ((int64_t)splits * a.M * nmax) * 4 >= ((int64_t)1 << 31)) return false;
  pl->splits = splits;
  pl->range = range;
  pl->grid_x = grid_x;
  pl->pstride = splits > 1 ? (size_t)splits * a.M * nmax : 0;
  pl->bytes = splits > 1 ? kCounterBytes + (size_t)a.count * pl->pstride * sizeof(float) : 0;
  return true;
}

hipError_t launch_band(const LaunchArgs& a, const BandPlan& pl, void* ws, hipStream_t stream) {
  DmaArgs d;
  memset(&d, 0, sizeof(d));
  if (pl.splits > 1) {
    char* base = static_cast<char*>(ws);
    d.counters = reinterpret_cast<uint32_t*>(base);
    d.partial = reinterpret_cast<float*>(base + kCounterBytes);
  }
  d.pstride = (int64_t)pl.pstride;
  d.splits = pl.splits;
  d.range = pl.range;
  d.tiles_max = pl.grid_x;
  if (pl.splits > 1)
    hipLaunchKernelGGL((qmv_band_kernel<true>), dim3(pl.grid_x * pl.splits, a.count), dim3(64 * bd::kWaves), 0,
                       stream, a, d);
  else
    hipLaunchKernelGGL((qmv_band_kernel<false>), dim3(pl.grid_x, a.count), dim3(64 * bd::kWaves), 0, stream, a, d);
  return hipGetLastError();
}

template <int W, int GMAX>
hipError_t launch_dma_w(const LaunchArgs& a, const DmaArgs& d, const DmaPlan& pl, hipStream_t stream) {
  if (pl.splits > 1)
    hipLaunchKernelGGL((qmv_dma_kernel<W, GMAX, true>), dim3(pl.grid_x * pl.splits, a.count), dim3(64 * W), 0,
                       stream, a, d);
  else
    hipLaunchKernelGGL((qmv_dma_kernel<W, GMAX, false>), dim3(pl.grid_x, a.count), dim3(64 * W), 0, stream, a, d);
  return hipGetLastError();
}

template <int GMAX>
hipError_t launch_dma_g(const LaunchArgs& a, const DmaArgs& d, const DmaPlan& pl, hipStream_t stream) {
  switch (pl.waves) {
    case 2: return launch_dma_w<2, GMAX>(a, d, pl, stream);
    case 3: return launch_dma_w<3, GMAX>(a, d, pl, stream);
    case 4: return launch_dma_w<4, GMAX>(a, d, pl, stream);
    case 5: return launch_dma_w<5, GMAX>(a, d, pl, stream);
    case 6: return launch_dma_w<6, GMAX>(a, d, pl, stream);
    default: return launch_dma_w<8, GMAX>(a, d, pl, stream);
  }
}

hipError_t launch_dma(const LaunchArgs& a, const DmaPlan& pl, void* ws, hipStream_t stream,
                      const NormIn* nin = nullptr, const ResidualOut* res = nullptr,
                      float* planes = nullptr, int64_t plane_pstride = 0) {
  DmaArgs d;
  memset(&d, 0, sizeof(d));
  if (nin) d.nin = *nin;
  if (res) d.res = *res;
  if (planes) {  // the partials are the outputs: no counters, no workspace
    d.partial = planes;
    d.planes = 1;
  } else if (pl.splits > 1) {
    char* base = static_cast<char*>(ws);
    d.counters = reinterpret_cast<uint32_t*>(base);
    d.partial = reinterpret_cast<float*>(base + kCounterBytes);
  }
  d.pstride = planes ? plane_pstride : (int64_t)pl.pstride;
  d.splits = pl.splits;
  d.range = pl.range;
  d.tiles_max = pl.grid_x;
  return pl.gmax == 4 ? launch_dma_g<4>(a, d, pl, stream) : launch_dma_g<8>(a, d, pl, stream);
}

#ifndef IMQ_XS_MIN_ROWS
#define IMQ_XS_MIN_ROWS 3
#endif

// Workspace bytes the launch would use given as much as it wants (0: no split).
size_t wanted_workspace(const LaunchArgs& a, int cu_count) {
  if (a.M < 3) return 0;
  XsArgs x;
  XsPlan xp;
  if (a.M >= IMQ_XS_MIN_ROWS && plan_xs(a, cu_count, &x, &xp)) return 0;
  DmaPlan dp;
  if (take_dma(a, cu_count, &dp) && dp.splits == 1) return 0;
  BandPlan bp;
  if (plan_band(a, cu_count, &bp)) return bp.bytes;
  if (take_dma(a, cu_count, &dp)) return dp.bytes;
  return plan_mma(a, (size_t)1 << 40, cu_count).bytes;
}

template <int NCH, int XR>
hipError_t launch_gather_nx(const GatherArgs& a, int P, hipStream_t stream) {
  const int rows = kThreads >> a.sh;
  constexpr size_t lds = M1Lds<NCH, XR>::kBytes;
  hipLaunchKernelGGL((qmv_gather_kernel<NCH, XR>), dim3((a.N + rows - 1) / rows, P), dim3(kThreads),
                     lds, stream, a);
  return hipGetLastError();
}

hipError_t launch_gather(const GatherArgs& a, int P, hipStream_t stream) {
  const int xr = (a.K / 8 + kThreads - 1) / kThreads;
  if (a.nch <= 2 && xr <= 2) return launch_gather_nx<2, 2>(a, P, stream);
  if (a.nch <= 5) {
    if (xr <= 2) return launch_gather_nx<5, 2>(a, P, stream);
    if (xr <= 5) return launch_gather_nx<5, 5>(a, P, stream);
  }
  if (xr <= 2) return launch_gather_nx<8, 2>(a, P, stream);
  if (xr <= 5) return launch_gather_nx<8, 5>(a, P, stream);
  return launch_gather_nx<8, 8>(a, P, stream);
}

// Plans the work of every problem and launches one kernel for all of them.
int32_t launch(LaunchArgs& a, const DeviceInfo* dev, hipStream_t stream, void* ws = nullptr,
               size_t ws_bytes = 0) {
  const int M = a.M;
  hipError_t e;
  M1Plan m1;
  int grid_x = 0;
  size_t lds = 0;
  XsArgs xa;
  XsPlan xp;
  bool big = false;
  for (int i = 0; i < a.count; ++i)
    big = big || (int64_t)a.p[i].N * (a.p[i].K / 2) >= ((int64_t)1 << 31);
  DmaPlan dp;
  BandPlan bp;
  if (M >= IMQ_XS_MIN_ROWS && !big && plan_xs(a, dev->cu_count, &xa, &xp)) {
    e = launch_xs(xa, xp, stream);
  } else if (take_dma(a, dev->cu_count, &dp) && dp.splits == 1) {
    e = launch_dma(a, dp, ws, stream);
  } else if (!big && plan_band(a, dev->cu_count, &bp) && (bp.bytes == 0 || (ws && bp.bytes <= ws_bytes))) {
    e = launch_band(a, bp, ws, stream);
  } else if (take_dma(a, dev->cu_count, &dp) &&
             (dp.bytes == 0 || (ws && dp.bytes <= ws_bytes))) {
    e = launch_dma(a, dp, ws, stream);
  } else if (M == 1 && plan_m1(a, &m1)) {
    e = launch_m1_for(a, m1, stream);
  } else if (M == 2 && plan_m1(a, &m1) && launch_mr_for<2>(a, m1, stream, &e)) {
    // launched
  } else if (M == 3 && plan_m1(a, &m1) && launch_mr_for<3>(a, m1, stream, &e)) {
    // launched
  } else if (M == 4 && plan_m1(a, &m1) && launch_mr_for<4>(a, m1, stream, &e)) {
    // launched
  } else if (M <= kValuMaxRows && (lds = plan_rows(a, &grid_x)) > 0) {
    if (M == 1) {
      static const int opts[] = {4, 5};
      e = choose_batch(a, opts, 2) == 4 ? launch_rows<1, 4>(a, grid_x, lds, stream)
                                        : launch_rows<1, 5>(a, grid_x, lds, stream);
    } else {
      e = launch_rows<2, 2>(a, grid_x, lds, stream);
    }
  } else {
    for (int i = 0; i < a.count; ++i)
      if ((int64_t)a.p[i].N * (a.p[i].K / 2) >= ((int64_t)1 << 31))
        return fail(IMQ_EUNSUPPORTED, "a weight of 2 GiB or more exceeds the MFMA kernel's offsets");
    const MmaPlan pl = plan_mma(a, ws ? ws_bytes : 0, dev->cu_count);
    e = launch_mma(a, pl, ws, stream);
  }
  if (e != hipSuccess)
    return fail(IMQ_ELAUNCH, std::string("qmv launch failed: ") + hipGetErrorString(e));
  return ok();
}

}  // namespace

// ==================================================================== C ABI

extern "C" {

int32_t imq_abi_version(void) { return IMQ_ABI_VERSION; }

int32_t imq_device_check(char* arch, size_t arch_len, int32_t* cu_count) {
  int32_t code = IMQ_OK;
  int dev = -1;
  if (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < imq_rt::kMaxDevices) {
    current_device(&code);
    const imq_rt::DeviceInfo& info = imq_rt::device_info(dev);
    if (arch && arch_len) {
      strncpy(arch, info.arch, arch_len - 1);
      arch[arch_len - 1] = 0;
    }
    if (cu_count) *cu_count = info.cu_count;
    return code == IMQ_OK ? ok() : code;
  }
  return fail(IMQ_EUNAVAILABLE, "no HIP device is available");
}

int32_t imq_qmv(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                const uint16_t* x, int64_t ldx, void* y, int64_t ldy, int32_t M, int32_t N,
                int32_t K, int32_t group_size, int32_t bits, int32_t y_dtype, void* stream) {
  int32_t code = check_format(N, K, group_size, bits);
  if (code != IMQ_OK) return code;
  if ((code = check_weights(w, scales, biases)) != IMQ_OK) return code;
  if ((code = check_dtype(y_dtype)) != IMQ_OK) return code;
  if ((code = check_rows(x, ldx, y, ldy, M, N, K, y_dtype)) != IMQ_OK) return code;
  const DeviceInfo* dev = current_device(&code);
  if (!dev) return code;
  LaunchArgs a;
  memset(&a, 0, sizeof(a));
  a.p[0] = Problem{w, scales, biases, x, y, M > 1 ? ldx : K, M > 1 ? ldy : N, N, K, 0, 0, 0, 0};
  a.count = 1;
  a.M = M;
  a.y_f32 = (y_dtype == IMQ_F32);
  return launch(a, dev, static_cast<hipStream_t>(stream));
}

int32_t imq_qmv_multi(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                      const uint16_t* const* xs, void* const* ys, int32_t count, int32_t N,
                      int32_t K, int32_t group_size, int32_t bits, int32_t y_dtype,
                      void* stream) {
  int32_t code = check_format(N, K, group_size, bits);
  if (code != IMQ_OK) return code;
  if ((code = check_weights(w, scales, biases)) != IMQ_OK) return code;
  if ((code = check_dtype(y_dtype)) != IMQ_OK) return code;
  if (count < 1) return fail(IMQ_EINVAL, "count must be >= 1");
  if (count > IMQ_MAX_ROWS) return fail(IMQ_EUNSUPPORTED, "count must be <= 32");
  if (!xs || !ys) return fail(IMQ_EINVAL, "xs and ys must be non-null");
  for (int i = 0; i < count; ++i) {
    if (!xs[i] || !ys[i]) return fail(IMQ_EINVAL, "every xs[i] and ys[i] must be non-null");
    if (!aligned(xs[i], 16)) return fail(IMQ_EINVAL, "every xs[i] must be 16-byte aligned");
    if (!aligned(ys[i], y_dtype == IMQ_F32 ? 4 : 2)) return fail(IMQ_EINVAL, "ys[i] is misaligned");
  }
  const DeviceInfo* dev = current_device(&code);
  if (!dev) return code;
  LaunchArgs a;
  memset(&a, 0, sizeof(a));
  a.p[0] = Problem{w, scales, biases, xs[0], ys[0], K, N, N, K, 0, 0, 0, 0};
  for (int i = 0; i < count; ++i) {
    a.xt[i] = xs[i];
    a.yt[i] = ys[i];
  }
  a.count = 1;
  a.M = count;
  a.y_f32 = (y_dtype == IMQ_F32);
  a.table = 1;
  return launch(a, dev, static_cast<hipStream_t>(stream));
}

}  // extern "C"

namespace {

// Validates `problems` into `a`; IMQ_OK or the error code.
int32_t build_grouped(LaunchArgs& a, const imq_problem* problems, int32_t count, int32_t M,
                      int32_t group_size, int32_t bits, int32_t y_dtype) {
  if (!problems) return fail(IMQ_EINVAL, "problems must be non-null");
  if (count < 1) return fail(IMQ_EINVAL, "count must be >= 1");
  if (count > IMQ_MAX_PROBLEMS)
    return fail(IMQ_EUNSUPPORTED, "at most IMQ_MAX_PROBLEMS problems per call");
  int32_t code = check_dtype(y_dtype);
  if (code != IMQ_OK) return code;
  memset(&a, 0, sizeof(a));
  for (int i = 0; i < count; ++i) {
    const imq_problem& q = problems[i];
    if ((code = check_format(q.N, q.K, group_size, bits)) != IMQ_OK) return code;
    if ((code = check_weights(q.w, q.scales, q.biases)) != IMQ_OK) return code;
    if ((code = check_rows(q.x, q.ldx, q.y, q.ldy, M, q.N, q.K, y_dtype)) != IMQ_OK) return code;
    a.p[i] = Problem{q.w, q.scales, q.biases, q.x, q.y, M > 1 ? q.ldx : q.K,
                     M > 1 ? q.ldy : q.N, q.N, q.K, 0, 0, 0, 0};
  }
  a.count = count;
  a.M = M;
  a.y_f32 = (y_dtype == IMQ_F32);
  return IMQ_OK;
}

}  // namespace

extern "C" {

int32_t imq_qmv_grouped(const imq_problem* problems, int32_t count, int32_t M,
                        int32_t group_size, int32_t bits, int32_t y_dtype, void* stream) {
  LaunchArgs a;
  int32_t code = build_grouped(a, problems, count, M, group_size, bits, y_dtype);
  if (code != IMQ_OK) return code;
  const DeviceInfo* dev = current_device(&code);
  if (!dev) return code;
  return launch(a, dev, static_cast<hipStream_t>(stream));
}

size_t imq_qmv_grouped_workspace(const imq_problem* problems, int32_t count, int32_t M) {
  if (!problems || count < 1 || count > IMQ_MAX_PROBLEMS || M < 3 || M > IMQ_MAX_ROWS) return 0;
  int32_t code;
  const DeviceInfo* dev = current_device(&code);
  if (!dev) return 0;
  LaunchArgs a;
  memset(&a, 0, sizeof(a));
  for (int i = 0; i < count; ++i) {
    if (problems[i].N < 1 || problems[i].K < 64 || problems[i].K % 64) return 0;
    a.p[i].N = problems[i].N;
    a.p[i].K = problems[i].K;
    a.p[i].ldx = problems[i].ldx > problems[i].K ? problems[i].ldx : problems[i].K;
  }
  a.count = count;
  a.M = M;
  return wanted_workspace(a, dev->cu_count);
}

int32_t imq_qmv_grouped_ws(const imq_problem* problems, int32_t count, int32_t M,
                           int32_t group_size, int32_t bits, int32_t y_dtype, float* workspace,
                           size_t workspace_bytes, void* stream) {
  LaunchArgs a;
  int32_t code = build_grouped(a, problems, count, M, group_size, bits, y_dtype);
  if (code != IMQ_OK) return code;
  if (workspace_bytes > 0 && (!workspace || !aligned(workspace, 16)))
    return fail(IMQ_EINVAL, "workspace must be non-null and 16-byte aligned");
  const DeviceInfo* dev = current_device(&code);
  if (!dev) return code;
  return launch(a, dev, static_cast<hipStream_t>(stream), workspace, workspace_bytes);
}

int32_t imq_qmv_grouped_noalloc(const imq_problem* problems, int32_t count, int32_t M,
                                int32_t group_size, int32_t bits, int32_t y_dtype, void* stream) {
  LaunchArgs a;
  int32_t code = build_grouped(a, problems, count, M, group_size, bits, y_dtype);
  if (code != IMQ_OK) return code;
  const DeviceInfo* dev = current_device(&code);
  if (!dev) return code;
  // the plan imq_qmv_grouped_ws makes with a workspace of imq_qmv_grouped_workspace bytes,
  // so both entry points split the same way and give the same bits
  const size_t need = wanted_workspace(a, dev->cu_count);
  if (need > IMQ_NOALLOC_SCRATCH_BYTES)
    return fail(IMQ_EUNSUPPORTED,
                "this call's split workspace (" + std::to_string(need) +
                    " bytes) exceeds the library's static scratch of " +
                    std::to_string((size_t)IMQ_NOALLOC_SCRATCH_BYTES) +
                    " bytes; use imq_qmv_grouped_ws with a caller workspace");
  if (need == 0) return launch(a, dev, static_cast<hipStream_t>(stream));
  void* ws = scratch_address(&code);
  if (!ws) return code;
  hipStream_t st = static_cast<hipStream_t>(stream);
  // the counters must start at zero; the split kernels leave them at zero, but a kernel
  // fill before every call keeps that true whatever ran on the device before
  constexpr int words = (int)(kCounterBytes / 4);
  hipLaunchKernelGGL(clear_words_kernel, dim3(words / kThreads), dim3(kThreads), 0, st,
                     static_cast<uint32_t*>(ws), words);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(IMQ_ELAUNCH, std::string("scratch clear failed: ") + hipGetErrorString(e));
  return launch(a, dev, st, ws, need);
}

int32_t imq_gather_qmv(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                       int32_t experts, const uint16_t* x, int64_t ldx, int32_t rows_per_x,
                       const uint32_t* idx, int32_t pairs, void* y, int64_t ldy, int32_t N,
                       int32_t K, int32_t group_size, int32_t bits, int32_t y_dtype,
                       void* stream) {
  int32_t code = check_format(N, K, group_size, bits);
  if (code != IMQ_OK) return code;
  if ((code = check_weights(w, scales, biases)) != IMQ_OK) return code;
  if ((code = check_dtype(y_dtype)) != IMQ_OK) return code;
  if (experts < 1) return fail(IMQ_EINVAL, "experts must be >= 1");
  if (pairs < 1 || pairs > 65535) return fail(IMQ_EINVAL, "pairs must be in 1..65535");
  if (rows_per_x < 1) return fail(IMQ_EINVAL, "rows_per_x must be >= 1");
  if (!x || !y || !idx) return fail(IMQ_EINVAL, "x, y and idx must be non-null");
  if (!aligned(x, 16) || (pairs > rows_per_x && ldx % 8)) return fail(IMQ_EINVAL, "x rows must be 16-byte aligned");
  if (pairs > rows_per_x && ldx < K) return fail(IMQ_EINVAL, "ldx must be >= K");
  if (pairs > 1 && ldy < N) return fail(IMQ_EINVAL, "ldy must be >= N");
  if (!aligned(y, y_dtype == IMQ_F32 ? 4 : 2) || !aligned(idx, 4)) return fail(IMQ_EINVAL, "y or idx is misaligned");
  const int sh = m1_lane_shift(K);
  if (sh < 0) return fail(IMQ_EUNSUPPORTED, "K over 16384");
  if (((int64_t)N * (K / 64)) % 2) return fail(IMQ_EUNSUPPORTED, "N * K / 64 must be even (4-byte aligned expert scales)");
  if ((int64_t)N * (K / 2) >= ((int64_t)1 << 31)) return fail(IMQ_EUNSUPPORTED, "an expert of 2 GiB or more");
  const DeviceInfo* dev = current_device(&code);
  if (!dev) return code;
  GatherArgs a;
  memset(&a, 0, sizeof(a));
  a.w = w;
  a.s = scales;
  a.b = biases;
  a.x = x;
  a.y = y;
  a.idx = idx;
  a.ldx = ldx;
  a.ldy = ldy;
  a.w_stride = (int64_t)N * (K / 8);
  a.sb_stride = (int64_t)N * (K / 64);
  a.E = experts;
  a.N = N;
  a.K = K;
  a.xs = rows_per_x;
  a.sh = sh;
  a.nch = ((K / 32) + (1 << sh) - 1) >> sh;
  a.y_f32 = y_dtype == IMQ_F32;
  const hipError_t e = launch_gather(a, pairs, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(IMQ_ELAUNCH, std::string("gather launch failed: ") + hipGetErrorString(e));
  return ok();
}

int32_t imq_dequant(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                    void* out, int32_t out_dtype, int32_t N, int32_t K, int32_t group_size,
                    int32_t bits, void* stream) {
  int32_t code = check_format(N, K, group_size, bits);
  if (code != IMQ_OK) return code;
  if ((code = check_weights(w, scales, biases)) != IMQ_OK) return code;
  if (!out) return fail(IMQ_EINVAL, "out must be non-null");
  if (out_dtype != IMQ_BF16 && out_dtype != IMQ_F32 && out_dtype != IMQ_F16)
    return fail(IMQ_EINVAL, "out_dtype must be bf16, fp32 or fp16");
  if (!aligned(out, 16)) return fail(IMQ_EINVAL, "out must be 16-byte aligned");
  const DeviceInfo* dev = current_device(&code);
  if (!dev) return code;
  const int64_t words = (int64_t)N * (K / 8);
  const int64_t blocks = (words + kThreads - 1) / kThreads;
  if (blocks > 0x7fffffff) return fail(IMQ_EUNSUPPORTED, "weight too large for one launch");
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (out_dtype) {
    case IMQ_BF16:
      hipLaunchKernelGGL(dequant_kernel<0>, dim3((uint32_t)blocks), dim3(kThreads), 0, st, w,
                         scales, biases, out, words, K);
      break;
    case IMQ_F32:
      hipLaunchKernelGGL(dequant_kernel<1>, dim3((uint32_t)blocks), dim3(kThreads), 0, st, w,
                         scales, biases, out, words, K);
      break;
    default:
      hipLaunchKernelGGL(dequant_kernel<2>, dim3((uint32_t)blocks), dim3(kThreads), 0, st, w,
                         scales, biases, out, words, K);
      break;
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return fail(IMQ_ELAUNCH, std::string("dequant launch failed: ") + hipGetErrorString(e));
  return ok();
}

int32_t imq_last_error(char* buf, size_t len) { return imq_rt::last_error(buf, len); }

}  // extern "C"

// ============================================ the RMSNorm folded into projections

namespace {

int32_t check_norm_in(const imq_norm_in* in) {
  if (!in->ssq || !aligned(in->ssq, 16)) return fail(IMQ_EINVAL, "norm ssq must be non-null and 16-byte aligned");
  if (in->tiles < 1 || in->tiles > kNormMaxTiles)
    return fail(IMQ_EUNSUPPORTED, "norm partials per row must be 1..64");
  if (in->ld < in->tiles || in->ld % 4) return fail(IMQ_EINVAL, "norm ld must be a multiple of 4 and >= tiles");
  if (in->dim < 1 || !(in->eps >= 0.0f)) return fail(IMQ_EINVAL, "norm dim must be >= 1 and eps >= 0");
  if ((int64_t)IMQ_MAX_ROWS * in->ld * 4 >= ((int64_t)1 << 31)) return fail(IMQ_EINVAL, "norm ld too large");
  return IMQ_OK;
}

NormIn to_norm_in(const imq_norm_in* in) {
  NormIn n;
  memset(&n, 0, sizeof(n));
  if (in) n = NormIn{in->ssq, in->tiles, in->ld, in->dim, in->eps};
  return n;
}

// imq_qmv_norm_planes over the row-band kernel (one plane per problem) instead of K-range
// planes: x in the tile layout, at most three problems of one K, K a multiple of 256 and at
// most IMQ_ROWBAND_PLANES_MAX_K (the q/k/v projections of the batched decode step: 7.0
// against 9.1 us at K = 2560 and 32 rows).
#ifndef IMQ_ROWBAND_PLANES_MAX_K
#define IMQ_ROWBAND_PLANES_MAX_K 4096
#endif
bool rowband_planes(const imq_problem* problems, int32_t count) {
  if (count < 1 || count > 3) return false;
  for (int i = 0; i < count; ++i) {
    const imq_problem& q = problems[i];
    if (q.ldx != IMQ_LD_TILED || q.K != problems[0].K || q.K % 256 != 0 || q.K > IMQ_ROWBAND_PLANES_MAX_K)
      return false;
  }
  return true;
}

// x' of a residual epilogue: rows ldx apart, or the tile layout (ldx == IMQ_LD_TILED, N a
// multiple of 64); the row stride the kernels take (0: tiled).
int32_t check_x_out(const imq_residual_out* out, int32_t M, int32_t N) {
  if (!out->weight) return IMQ_OK;
  if (!aligned(out->weight, 2) || !out->x || !aligned(out->x, 2))
    return fail(IMQ_EINVAL, "norm weight and x' must be non-null and 2-byte aligned");
  if (out->ldx == IMQ_LD_TILED) {
    if (N % 64 != 0 || M > IMQ_MAX_ROWS) return fail(IMQ_EINVAL, "a tiled x' needs N a multiple of 64");
    return IMQ_OK;
  }
  if (M > 1 && out->ldx < N) return fail(IMQ_EINVAL, "x' ldx must be >= N");
  return IMQ_OK;
}
int64_t x_out_ld(const imq_residual_out* out, int32_t M, int32_t N) {
  return out->ldx == IMQ_LD_TILED ? 0 : M > 1 ? out->ldx : N;
}

// Validates a fused-norm call into `a`, the plan `pl` and the device arguments.
int32_t build_norm(LaunchArgs& a, DmaPlan* pl, NormIn* nin, ResidualOut* res,
                   const imq_problem* problems, int32_t count, int32_t M, int32_t group_size,
                   int32_t bits, const imq_norm_in* in, const imq_residual_out* out,
                   const DeviceInfo** dev) {
  if (!problems) return fail(IMQ_EINVAL, "problems must be non-null");
  if (count < 1 || count > IMQ_MAX_PROBLEMS) return fail(IMQ_EINVAL, "count must be 1..IMQ_MAX_PROBLEMS");
  if (out && count != 1) return fail(IMQ_EINVAL, "a residual epilogue takes one problem");
  imq_problem probs[IMQ_MAX_PROBLEMS];
  bool xt[IMQ_MAX_PROBLEMS] = {};
  for (int i = 0; i < count; ++i) {
    probs[i] = problems[i];
    if (probs[i].ldx == IMQ_LD_TILED) {  // the tile layout: validated as K-element rows
      if (probs[i].K % 64 != 0) return fail(IMQ_EINVAL, "a tiled x needs K a multiple of 64");
      xt[i] = true;
      probs[i].ldx = probs[i].K;
    }
  }
  if (out) {  // y is not written: validate the rows against the residual rows instead
    if (!out->h || !aligned(out->h, 4)) return fail(IMQ_EINVAL, "residual h must be non-null and 4-byte aligned");
    if (M > 1 && out->ldh < probs[0].N) return fail(IMQ_EINVAL, "residual ldh must be >= N");
    probs[0].y = out->h;
    probs[0].ldy = out->ldh;
  }
  int32_t code = build_grouped(a, probs, count, M, group_size, bits, IMQ_BF16);
  if (code != IMQ_OK) return code;
  for (int i = 0; i < count; ++i)
    if (xt[i]) a.p[i].ldx = 0;
  memset(nin, 0, sizeof(*nin));
  memset(res, 0, sizeof(*res));
  if (in) {
    if ((code = check_norm_in(in)) != IMQ_OK) return code;
    *nin = to_norm_in(in);
  }
  if (out) {
    const int N = probs[0].N, tiles = (N + 63) / 64;
    if ((code = check_x_out(out, M, N)) != IMQ_OK) return code;
    if (out->ssq && (!aligned(out->ssq, 4) || out->ld < tiles || out->ld % 4))
      return fail(IMQ_EINVAL, "residual ssq must be 4-byte aligned with ld >= ceil(N / 64), a multiple of 4");
    *res = ResidualOut{out->h, M > 1 ? out->ldh : N, out->weight, out->x, x_out_ld(out, M, N), out->ssq, out->ld, 0};
  }
  *dev = current_device(&code);
  if (!*dev) return code;
  if (!plan_dma_norm(a, (*dev)->cu_count, pl))
    return fail(IMQ_EUNSUPPORTED, "the fused-norm projections need K % 256 == 0, 16-byte aligned x rows "
                                  "(ldx a multiple of 8), one K per call when K-ranges split and "
                                  "offsets under 2 GiB");
  return IMQ_OK;
}

// The gate/up launch's plan: whole tiles of 32 gate and 32 up rows, and with a workspace the
// tiles past the last whole round over the CUs cut into K-parts (0 parts: none).
#ifndef IMQ_PAIR_ROWS
#define IMQ_PAIR_ROWS 1
#endif
struct PairPlan {
  int whole = 0, tail = 0, parts = 1;
  size_t bytes = 0;
};
PairPlan plan_pair(int N, int K, int cu_count) {
  PairPlan pl;
  const int T = (N + 31) / 32;
  pl.whole = T;
  const int r = T > cu_count ? T % cu_count : 0;
  if (r > 0 && K / 64 >= 4 * staged::kMaxPairParts) {
    pl.whole = T - r;
    pl.tail = r;
    pl.parts = staged::kMaxPairParts;
    pl.bytes = kCounterBytes + (size_t)r * pl.parts * 2048 * sizeof(float);
  }
  return pl;
}

// The gate/up launch over bands of rows (qmv_pair_rows_kernel, the folded-norm form): one
// workgroup per CU, each with at most pr::kMaxUnits units of 8 gate and 8 up rows.  Not
// applicable: K / 256 not an instantiated wavefront count, x rows not 16-byte aligned.
struct PairRowsPlan {
  int waves = 0, nwg = 0, units = 0;
};
bool plan_pair_rows(int M, int N, int K, int64_t ldx, const void* x, int cu_count, PairRowsPlan* pl) {
  const int w = K / 256;
  if (K % 256 != 0 || !(w == 4 || w == 8 || w == 10 || w == 12)) return false;
  if (M < 1 || M > 32 || ldx % 8 != 0 || !imq_rt::aligned(x, 16)) return false;
  const int units = (N + 7) / 8;
  int nwg = units < cu_count ? units : cu_count;
  if ((units + nwg - 1) / nwg > pr::kMaxUnits) nwg = (units + pr::kMaxUnits - 1) / pr::kMaxUnits;
  pl->waves = w;
  pl->nwg = nwg;
  pl->units = units;
  return true;
}

hipError_t launch_pair_rows(const LaunchArgs& a, const NormIn& ni, const PairRowsPlan& pl, hipStream_t stream) {
  switch (pl.waves) {
    case 4: hipLaunchKernelGGL((qmv_pair_rows_kernel<4>), dim3(pl.nwg), dim3(64 * 4), 0, stream, a, ni, pl.nwg, pl.units); break;
    case 8: hipLaunchKernelGGL((qmv_pair_rows_kernel<8>), dim3(pl.nwg), dim3(64 * 8), 0, stream, a, ni, pl.nwg, pl.units); break;
    case 10: hipLaunchKernelGGL((qmv_pair_rows_kernel<10>), dim3(pl.nwg), dim3(64 * 10), 0, stream, a, ni, pl.nwg, pl.units); break;
    case 12: hipLaunchKernelGGL((qmv_pair_rows_kernel<12>), dim3(pl.nwg), dim3(64 * 12), 0, stream, a, ni, pl.nwg, pl.units); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

int32_t gate_up_silu(const uint32_t* w_gate, const uint16_t* s_gate, const uint16_t* b_gate,
                     const uint32_t* w_up, const uint16_t* s_up, const uint16_t* b_up,
                     const uint16_t* x, int64_t ldx, uint16_t* act, int64_t ld_act, int32_t M,
                     int32_t N, int32_t K, int32_t group_size, int32_t bits, const imq_norm_in* in,
                     void* stream, float* workspace = nullptr, size_t workspace_bytes = 0) {
  int32_t code = check_format(N, K, group_size, bits);
  if (code != IMQ_OK) return code;
  if ((code = check_weights(w_gate, s_gate, b_gate)) != IMQ_OK) return code;
  if ((code = check_weights(w_up, s_up, b_up)) != IMQ_OK) return code;
  // the norm form takes x and act in the tile layout too (row stride IMQ_LD_TILED)
  const bool xt = in && ldx == IMQ_LD_TILED, at = in && ld_act == IMQ_LD_TILED;
  if ((xt && K % 64 != 0) || (at && N % 64 != 0))
    return fail(IMQ_EINVAL, "the tile layout needs K (x) or N (act) a multiple of 64");
  if ((code = check_rows(x, xt ? K : ldx, act, at ? N : ld_act, M, N, K, IMQ_BF16)) != IMQ_OK) return code;
  if (in && (code = check_norm_in(in)) != IMQ_OK) return code;
  // without the folded norm the launch keeps the bits of the grouped launch and silu_mul,
  // whose plans take the few-row VALU kernel below 5 rows
  if (M < (in ? 1 : 5) || K % 256 != 0)
    return fail(IMQ_EUNSUPPORTED, in ? "the fused gate/up launch with the input norm takes K a multiple of 256"
                                     : "the fused gate/up launch takes 5 to 32 rows and K a multiple of 256");
  if ((int64_t)N * (K / 2) >= ((int64_t)1 << 31) || ((int64_t)(M - 1) * ldx + K) * 2 >= ((int64_t)1 << 31))
    return fail(IMQ_EUNSUPPORTED, "a weight or activation of 2 GiB or more exceeds the kernel's offsets");
  const DeviceInfo* dev = current_device(&code);
  if (!dev) return code;
  LaunchArgs a;
  memset(&a, 0, sizeof(a));
  const int64_t lx = xt ? 0 : M > 1 ? ldx : K, la = at ? 0 : M > 1 ? ld_act : N;
  a.p[0] = Problem{w_gate, s_gate, b_gate, x, act, lx, la, N, K, 0, 0, 0, 0};
  a.p[1] = Problem{w_up, s_up, b_up, x, nullptr, lx, la, N, K, 0, 0, 0, 0};
  a.count = 2;
  a.M = M;
  PairRowsPlan rp;
  if (in && IMQ_PAIR_ROWS && plan_pair_rows(M, N, K, lx, x, dev->cu_count, &rp)) {
    const hipError_t e = launch_pair_rows(a, to_norm_in(in), rp, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail(IMQ_ELAUNCH, std::string("gate/up launch failed: ") + hipGetErrorString(e));
    return ok();
  }
  if (xt || at)
    return fail(IMQ_EUNSUPPORTED, "the tile layout takes the row-band gate/up kernel: K of 4, 8, 10 or 12 times 256");
  PairPlan pl = plan_pair(N, K, dev->cu_count);
  if (pl.parts > 1 && (!workspace || workspace_bytes < pl.bytes)) pl = PairPlan{(N + 31) / 32, 0, 1, 0};
  if (pl.parts > 1 && !aligned(workspace, 16)) return fail(IMQ_EINVAL, "workspace must be 16-byte aligned");
  char* ws = reinterpret_cast<char*>(workspace);
  hipLaunchKernelGGL((qmv_mma_staged_kernel<false, true>), dim3(pl.whole + pl.tail * pl.parts, 1),
                     dim3(kThreads), 0, static_cast<hipStream_t>(stream), a, pl.parts,
                     pl.parts > 1 ? reinterpret_cast<float*>(ws + kCounterBytes) : nullptr, (int64_t)0,
                     pl.parts > 1 ? reinterpret_cast<uint32_t*>(ws) : nullptr, pl.whole, to_norm_in(in));
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(IMQ_ELAUNCH, std::string("gate/up launch failed: ") + hipGetErrorString(e));
  return ok();
}

}  // namespace

extern "C" {

size_t imq_qmv_norm_workspace(const imq_problem* problems, int32_t count, int32_t M) {
  if (!problems || count < 1 || count > IMQ_MAX_PROBLEMS || M < 1 || M > IMQ_MAX_ROWS) return 0;
  int32_t code;
  const DeviceInfo* dev = current_device(&code);
  if (!dev) return 0;
  LaunchArgs a;
  memset(&a, 0, sizeof(a));
  for (int i = 0; i < count; ++i) {
    if (problems[i].N < 1 || problems[i].K < 64 || problems[i].K % 64) return 0;
    a.p[i].N = problems[i].N;
    a.p[i].K = problems[i].K;
    a.p[i].x = problems[i].x;
    a.p[i].ldx = M > 1 ? problems[i].ldx : problems[i].K;
  }
  a.count = count;
  a.M = M;
  DmaPlan pl;
  return plan_dma_norm(a, dev->cu_count, &pl) ? pl.bytes : 0;
}

int32_t imq_qmv_norm(const imq_problem* problems, int32_t count, int32_t M, int32_t group_size,
                     int32_t bits, const imq_norm_in* in, const imq_residual_out* out,
                     float* workspace, size_t workspace_bytes, void* stream) {
  LaunchArgs a;
  DmaPlan pl;
  NormIn nin;
  ResidualOut res;
  const DeviceInfo* dev = nullptr;
  int32_t code = build_norm(a, &pl, &nin, &res, problems, count, M, group_size, bits, in, out, &dev);
  if (code != IMQ_OK) return code;
  if (pl.bytes > 0 && (!workspace || !aligned(workspace, 16) || workspace_bytes < pl.bytes))
    return fail(IMQ_EINVAL, "this call needs a 16-byte aligned workspace of imq_qmv_norm_workspace bytes (" +
                                std::to_string(pl.bytes) + ")");
  const hipError_t e = launch_dma(a, pl, workspace, static_cast<hipStream_t>(stream), &nin, &res);
  if (e != hipSuccess) return fail(IMQ_ELAUNCH, std::string("fused-norm qmv launch failed: ") + hipGetErrorString(e));
  return ok();
}

int32_t imq_qmv_residual_bands(const imq_problem* problem, int32_t M, int32_t group_size, int32_t bits,
                               const imq_residual_out* out, void* stream) {
  if (!problem) return fail(IMQ_EINVAL, "problem must be non-null");
  if (!out) return fail(IMQ_EINVAL, "out must be non-null");
  const imq_problem& p = *problem;
  int32_t code = check_format(p.N, p.K, group_size, bits);
  if (code != IMQ_OK) return code;
  if ((code = check_weights(p.w, p.scales, p.biases)) != IMQ_OK) return code;
  if (M < 1 || M > IMQ_MAX_ROWS) return fail(IMQ_EINVAL, "M must be 1..32");
  if (!p.x) return fail(IMQ_EINVAL, "x must be non-null");
  const bool tiled = p.ldx == IMQ_LD_TILED;
  if (!tiled && (p.ldx < p.K || p.ldx % 8 != 0 || !aligned(p.x, 16)))
    return fail(IMQ_EINVAL, "x rows must be 16-byte aligned, ldx >= K and a multiple of 8 (or IMQ_LD_TILED)");
  if (tiled && !aligned(p.x, 16)) return fail(IMQ_EINVAL, "a tiled x must be 16-byte aligned");
  if (p.K % 256 != 0 || p.K / 256 > rb::kMaxChunks)
    return fail(IMQ_EUNSUPPORTED, "the row-band projection takes K a multiple of 256, at most 9728");
  const int64_t xbytes = tiled ? (int64_t)p.K * 64 : ((int64_t)(M - 1) * p.ldx + p.K) * 2;
  if ((int64_t)p.N * (p.K / 2) >= ((int64_t)1 << 31) || xbytes >= ((int64_t)1 << 31))
    return fail(IMQ_EUNSUPPORTED, "a weight or activation of 2 GiB or more exceeds the kernel's offsets");
  const int N = p.N, bands = (N + 31) / 32;
  if (!out->h || !aligned(out->h, 4)) return fail(IMQ_EINVAL, "residual h must be non-null and 4-byte aligned");
  if (M > 1 && out->ldh < N) return fail(IMQ_EINVAL, "residual ldh must be >= N");
  if ((code = check_x_out(out, M, N)) != IMQ_OK) return code;
  if (out->ssq && (!aligned(out->ssq, 4) || out->ld < bands || out->ld % 4))
    return fail(IMQ_EINVAL, "residual ssq must be 4-byte aligned with ld >= ceil(N / 32), a multiple of 4");
  if (!current_device(&code)) return code;
  RowbandArgs A;
  memset(&A, 0, sizeof(A));
  A.p[0] = Problem{p.w, p.scales, p.biases, p.x, nullptr, tiled ? 0 : p.ldx, 0, N, p.K, 0, 0, 0, 0};
  A.band0[1] = bands;
  A.count = 1;
  A.M = M;
  A.res = ResidualOut{out->h, M > 1 ? out->ldh : N, out->weight, out->x, x_out_ld(out, M, N), out->ssq, out->ld, 0};
  hipLaunchKernelGGL(qmv_rowband_kernel, dim3(bands), dim3(64 * rb::kWaves), 0, static_cast<hipStream_t>(stream), A);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(IMQ_ELAUNCH, std::string("row-band launch failed: ") + hipGetErrorString(e));
  return ok();
}

int32_t imq_residual_planes(const float* planes, int32_t nplanes, int32_t M, int32_t N,
                            const imq_residual_out* out, void* stream) {
  if (!planes || !aligned(planes, 4)) return fail(IMQ_EINVAL, "planes must be non-null and 4-byte aligned");
  if (!out) return fail(IMQ_EINVAL, "out must be non-null");
  if (nplanes < 1 || nplanes > kResPlanes) return fail(IMQ_EINVAL, "nplanes must be 1..16");
  if (M < 1 || M > IMQ_MAX_ROWS) return fail(IMQ_EINVAL, "M must be 1..32");
  if (N < 1) return fail(IMQ_EINVAL, "N must be >= 1");
  if ((int64_t)nplanes * M * N * 4 >= ((int64_t)1 << 31)) return fail(IMQ_EUNSUPPORTED, "planes of 2 GiB or more");
  if (!out->h || !aligned(out->h, 4)) return fail(IMQ_EINVAL, "residual h must be non-null and 4-byte aligned");
  if (M > 1 && out->ldh < N) return fail(IMQ_EINVAL, "residual ldh must be >= N");
  const int tiles = (N + 63) / 64;
  int32_t code = check_x_out(out, M, N);
  if (code != IMQ_OK) return code;
  if (out->ssq && (!aligned(out->ssq, 4) || out->ld < tiles || out->ld % 4))
    return fail(IMQ_EINVAL, "residual ssq must be 4-byte aligned with ld >= ceil(N / 64), a multiple of 4");
  if (!current_device(&code)) return code;
  const ResidualOut r{out->h, M > 1 ? out->ldh : N, out->weight, out->x, x_out_ld(out, M, N), out->ssq,
                      out->ld, 0};
  const dim3 grid(tiles, (M + kResRowsPerGroup - 1) / kResRowsPerGroup), block(64 * kResRowsPerGroup);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (nplanes <= 4)
    hipLaunchKernelGGL(residual_planes_kernel<4>, grid, block, 0, st, planes, nplanes, M, N, r);
  else if (nplanes <= 8)
    hipLaunchKernelGGL(residual_planes_kernel<8>, grid, block, 0, st, planes, nplanes, M, N, r);
  else
    hipLaunchKernelGGL(residual_planes_kernel<kResPlanes>, grid, block, 0, st, planes, nplanes, M, N, r);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(IMQ_ELAUNCH, std::string("residual planes launch failed: ") + hipGetErrorString(e));
  return ok();
}

int32_t imq_qmv_norm_splits(const imq_problem* problems, int32_t count, int32_t M) {
  if (!problems || count < 1 || count > IMQ_MAX_PROBLEMS || M < 1 || M > IMQ_MAX_ROWS) return 0;
  if (rowband_planes(problems, count)) return 1;
  int32_t code;
  const DeviceInfo* dev = current_device(&code);
  if (!dev) return 0;
  LaunchArgs a;
  memset(&a, 0, sizeof(a));
  for (int i = 0; i < count; ++i) {
    if (problems[i].N < 1 || problems[i].K < 64 || problems[i].K % 64) return 0;
    a.p[i].N = problems[i].N;
    a.p[i].K = problems[i].K;
    a.p[i].x = problems[i].x;
    a.p[i].ldx = M > 1 ? problems[i].ldx : problems[i].K;
  }
  a.count = count;
  a.M = M;
  DmaPlan pl;
  return plan_dma_norm(a, dev->cu_count, &pl) ? pl.splits : 0;
}

int32_t imq_qmv_norm_planes(const imq_problem* problems, int32_t count, int32_t M,
                            int32_t group_size, int32_t bits, const imq_norm_in* in, float* planes,
                            int64_t pstride, int32_t* splits, void* stream) {
  if (!planes || !aligned(planes, 4) || !splits) return fail(IMQ_EINVAL, "planes and splits must be non-null");
  if (!problems) return fail(IMQ_EINVAL, "problems must be non-null");
  // the problems' y are not written: validate against the planes
  imq_problem probs[IMQ_MAX_PROBLEMS];
  if (count < 1 || count > IMQ_MAX_PROBLEMS) return fail(IMQ_EINVAL, "count must be 1..IMQ_MAX_PROBLEMS");
  for (int i = 0; i < count; ++i) {
    probs[i] = problems[i];
    probs[i].y = planes;
    probs[i].ldy = problems[i].N;
  }
  LaunchArgs a;
  DmaPlan pl;
  NormIn nin;
  ResidualOut res;
  const DeviceInfo* dev = nullptr;
  int32_t code = build_norm(a, &pl, &nin, &res, probs, count, M, group_size, bits, in, nullptr, &dev);
  if (code != IMQ_OK) return code;
  int64_t need = 0;
  for (int i = 0; i < count; ++i) need = std::max(need, (int64_t)pl.splits * M * probs[i].N);
  if (pstride < need) return fail(IMQ_EINVAL, "pstride must hold every plane of the widest problem (" +
                                                  std::to_string(need) + " floats)");
  if (((int64_t)count * pstride) * 4 >= ((int64_t)1 << 31)) return fail(IMQ_EUNSUPPORTED, "planes of 2 GiB or more");
  if (rowband_planes(problems, count)) {  // one plane per problem from the row-band kernel
    RowbandArgs A;
    memset(&A, 0, sizeof(A));
    for (int i = 0; i < count; ++i) {
      A.p[i] = a.p[i];
      A.band0[i + 1] = A.band0[i] + (a.p[i].N + 31) / 32;
    }
    A.count = count;
    A.M = M;
    A.ni = nin;
    A.planes = planes;
    A.pstride = pstride;
    *splits = 1;
    hipLaunchKernelGGL(qmv_rowband_kernel, dim3(A.band0[count]), dim3(64 * rb::kWaves), 0,
                       static_cast<hipStream_t>(stream), A);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(IMQ_ELAUNCH, std::string("row-band launch failed: ") + hipGetErrorString(e));
    return ok();
  }
  *splits = pl.splits;
  const hipError_t e = launch_dma(a, pl, nullptr, static_cast<hipStream_t>(stream), &nin, &res, planes, pstride);
  if (e != hipSuccess) return fail(IMQ_ELAUNCH, std::string("fused-norm qmv launch failed: ") + hipGetErrorString(e));
  return ok();
}

int32_t imq_qmv_gate_up_silu(const uint32_t* w_gate, const uint16_t* s_gate,
                             const uint16_t* b_gate, const uint32_t* w_up, const uint16_t* s_up,
                             const uint16_t* b_up, const uint16_t* x, int64_t ldx, uint16_t* act,
                             int64_t ld_act, int32_t M, int32_t N, int32_t K, int32_t group_size,
                             int32_t bits, void* stream) {
  return gate_up_silu(w_gate, s_gate, b_gate, w_up, s_up, b_up, x, ldx, act, ld_act, M, N, K, group_size,
                      bits, nullptr, stream);
}

size_t imq_qmv_gate_up_silu_norm_workspace(int32_t M, int32_t N, int32_t K) {
  if (M < 1 || M > IMQ_MAX_ROWS || N < 1 || K < 256 || K % 256) return 0;
  int32_t code;
  const DeviceInfo* dev = current_device(&code);
  if (!dev) return 0;
  PairRowsPlan rp;
  if (IMQ_PAIR_ROWS && plan_pair_rows(M, N, K, K, nullptr, dev->cu_count, &rp)) return 0;
  return plan_pair(N, K, dev->cu_count).bytes;
}

int32_t imq_qmv_gate_up_silu_norm(const uint32_t* w_gate, const uint16_t* s_gate,
                                  const uint16_t* b_gate, const uint32_t* w_up, const uint16_t* s_up,
                                  const uint16_t* b_up, const uint16_t* x, int64_t ldx, uint16_t* act,
                                  int64_t ld_act, int32_t M, int32_t N, int32_t K, int32_t group_size,
                                  int32_t bits, const imq_norm_in* in, float* workspace,
                                  size_t workspace_bytes, void* stream) {
  if (!in) return fail(IMQ_EINVAL, "in must be non-null (imq_qmv_gate_up_silu takes no norm)");
  return gate_up_silu(w_gate, s_gate, b_gate, w_up, s_up, b_up, x, ldx, act, ld_act, M, N, K, group_size,
                      bits, in, stream, workspace, workspace_bytes);
}

}  // extern "C"
