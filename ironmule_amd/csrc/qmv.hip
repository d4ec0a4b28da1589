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
//
// Kernels sharing that arithmetic:
//   * qmv_fixed_kernel / qmv_rows_kernel (one or two activation rows): v_dot2_f32_bf16
//     chains, x staged once per workgroup in LDS already in pair order, each chain
//     started at -128 * sum(x);
//   * qmv_mfma_kernel (more rows): v_mfma_f32_16x16x32_bf16 with the activation rows as
//     the A operand and 16 weight rows as the B operand, one MFMA pair per group of 64,
//     and a second MFMA pair against a ones operand that yields sum(x) per group.
//
// Layout in HBM is the reference's own (row-major w (N, K/8) uint32, s and b (N, K/64)
// bf16), so a caller passes its buffers unchanged.  One launch may serve up to
// IMQ_MAX_PROBLEMS weights (for example q/k/v, or gate/up, which read the same x).

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include <mutex>
#include <string>

#include "../../include/ironmule_qmv.h"

namespace {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// Raw buffer resource over `bytes` bytes at `base` (gfx9 word 3: 32-bit data format).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

constexpr int kThreads = 256;  // 4 wavefronts of 64
constexpr int kGroup = 64;
constexpr int kMaxProblems = IMQ_MAX_PROBLEMS;

// ------------------------------------------------------------------ bf16 helpers

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
  return __uint_as_float(h << 16);
}

// Round to nearest even; NaN becomes the quiet NaN 0x7fc0 (ironmule/cuda_native.py:46-51).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// A constant held in a VGPR.  gfx9 VOP3 instructions take no literal operand and at
// most one SGPR, so (u & mask) | magic becomes one v_and_or_b32 only when `magic` is
// already in a vector register (the mask then comes from an SGPR).
__device__ __forceinline__ uint32_t in_vgpr(uint32_t c) {
  uint32_t r;
  asm("v_mov_b32 %0, %1" : "=v"(r) : "i"(c));
  return r;
}

constexpr uint32_t kMagic = 0x43004300u;  // bf16 pair (128.0, 128.0)
constexpr uint32_t kOnes = 0x3f803f80u;   // bf16 pair (1.0, 1.0)

// Nibbles p and p+4 of word u as the bf16 pair (128 + q_p, 128 + q_{p+4}).
// `magic` must be in_vgpr(kMagic).
__device__ __forceinline__ uint32_t nibble_pair(uint32_t u, int p, uint32_t magic) {
  return ((u >> (4 * p)) & 0x000F000Fu) | magic;
}

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}

// Eight natural-order bf16 values (x0..x7 in d.x..d.w) -> the pair order of nibble_pair.
__device__ __forceinline__ uint4 pair_order(uint4 d) {
  uint4 p;
  p.x = (d.x & 0xffffu) | (d.z << 16);      // (x0, x4)
  p.y = (d.x >> 16) | (d.z & 0xffff0000u);  // (x1, x5)
  p.z = (d.y & 0xffffu) | (d.w << 16);      // (x2, x6)
  p.w = (d.y >> 16) | (d.w & 0xffff0000u);  // (x3, x7)
  return p;
}

__device__ __forceinline__ float sum8(uint4 d) {
  const float a = bf16_bits_to_f32(d.x & 0xffffu) + bf16_bits_to_f32(d.x >> 16);
  const float b = bf16_bits_to_f32(d.y & 0xffffu) + bf16_bits_to_f32(d.y >> 16);
  const float c = bf16_bits_to_f32(d.z & 0xffffu) + bf16_bits_to_f32(d.z >> 16);
  const float e = bf16_bits_to_f32(d.w & 0xffffu) + bf16_bits_to_f32(d.w >> 16);
  return (a + b) + (c + e);
}

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over each aligned row of 16 lanes; every lane of the row receives the sum.
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp<0x141>(v);  // row_half_mirror
  v += dpp<0x140>(v);  // row_mirror
  return v;
}

// LDS-only barrier: waits for this wave's LDS traffic, not for its outstanding global
// loads (a full __syncthreads() would also drain the weight loads issued before it).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

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
  int32_t first;      // first workgroup of this problem
  int32_t lpr_shift;  // VALU kernel: log2 of the lanes that share one weight row
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
  int32_t items;  // VALU kernel: workgroups over all problems
  int32_t pad;
};

// The problem that owns workgroup `idx`; `first` increases with i.
__device__ __forceinline__ int find_problem(const LaunchArgs& a, int idx) {
  int pi = 0;
#pragma unroll
  for (int i = 1; i < kMaxProblems; ++i)
    if (i < a.count && idx >= a.p[i].first) pi = i;
  return pi;
}

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
    t.w[q] = *reinterpret_cast<const uint4*>(wrow + kk * 4);
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
  const Problem& P = a.p[find_problem(a, blockIdx.x)];
  const int K = P.K, N = P.N, sh = P.lpr_shift;
  const int C = K >> 5;  // 32-value chunks per row
  const int G = K >> 6;  // groups per row
  const int W = K >> 3;  // words per row
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int j = lane & ((1 << sh) - 1);
  const int row = (((blockIdx.x - P.first) * 4 + wave) << (6 - sh)) + (lane >> sh);
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
          part += __shfl_xor(part, 1);
          part += __shfl_xor(part, 2);
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
    if (sh >= 5) v += __shfl_xor(v, 16);
    if (sh >= 6) v += __shfl_xor(v, 32);
    if (j == 0 && row < N) store_y(a, P, m, row, v);
  }
}

// ------------------------------------- VALU kernel, lanes and chunks fixed at compile time
//
// The same arithmetic and LDS layout as qmv_rows_kernel, for launches whose problems
// all share the lanes per row (LPR = 1 << SH) and the chunks per lane (NCH).  Every
// chunk of a lane's row is loaded at once (no second buffer), addresses are one base
// plus immediate offsets, and only the last chunk can fall past the row (when
// NCH * LPR > K / 32), so only it is guarded.  Fewer registers let more wavefronts share
// each SIMD, so one launch's workgroups are resident together instead of in two rounds.

__device__ __forceinline__ float chunk_dot(uint4 wv, uint4 x0, uint4 x1, uint4 x2, uint4 x3,
                                           float d, uint32_t magic) {
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
  return d;
}

template <int M, int SH, int NCH>
__global__ __launch_bounds__(kThreads) void qmv_fixed_kernel(LaunchArgs a) {
  constexpr int LPR = 1 << SH;
  constexpr int XR = (NCH * LPR + 63) / 64;  // x words per thread: W <= NCH * LPR * 4
  extern __shared__ uint4 smem[];
  const Problem& P = a.p[find_problem(a, blockIdx.x)];
  const int K = P.K, N = P.N;
  const int C = K >> 5, G = K >> 6, W = K >> 3;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int j = lane & (LPR - 1);
  const int row = (((blockIdx.x - P.first) * 4 + wave) << (6 - SH)) + (lane >> SH);
  const int r = row < N ? row : N - 1;  // clamp loads; the store is guarded
  const bool last_ok = j + (NCH - 1) * LPR < C;
  const int kc_last = last_ok ? j + (NCH - 1) * LPR : 0;
  const uint32_t* wp = P.w + (size_t)r * W;
  const uint16_t* sp = P.s + (size_t)r * G;
  const uint16_t* bp = P.b + (size_t)r * G;
  uint4* xq = smem;
  float* sx = reinterpret_cast<float*>(smem + M * 4 * C);
  const uint32_t magic = in_vgpr(kMagic);

  // x first (its loads then complete before the weights'), then every weight chunk.
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
  uint4 wv[NCH];
  uint32_t s16[NCH], b16[NCH];
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int kc = i + 1 < NCH ? j + i * LPR : kc_last;
    wv[i] = *reinterpret_cast<const uint4*>(wp + kc * 4);
    s16[i] = sp[kc >> 1];
    b16[i] = bp[kc >> 1];
  }
#pragma unroll
  for (int m = 0; m < M; ++m) {
#pragma unroll
    for (int t = 0; t < XR; ++t) {
      const int i = tid + kThreads * t;
      if (i < W) {  // the four words of a chunk are four aligned lanes (W % 4 == 0)
        xq[(m * 4 + (i & 3)) * C + (i >> 2)] = pair_order(xs[m][t]);
        float part = sum8(xs[m][t]);
        part += __shfl_xor(part, 1);
        part += __shfl_xor(part, 2);
        if ((i & 3) == 0) sx[m * C + (i >> 2)] = part;
      }
    }
  }
  lds_barrier();

  float acc[M];
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m] = 0.0f;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int kc = i + 1 < NCH ? j + i * LPR : kc_last;
    const float sc = bf16_bits_to_f32(s16[i]);
    const float bi = bf16_bits_to_f32(b16[i]);
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const float sxm = sx[m * C + kc];
      const float d = chunk_dot(wv[i], xq[(m * 4 + 0) * C + kc], xq[(m * 4 + 1) * C + kc],
                                xq[(m * 4 + 2) * C + kc], xq[(m * 4 + 3) * C + kc],
                                -128.0f * sxm, magic);
      const float v = fmaf(sc, d, fmaf(bi, sxm, acc[m]));
      acc[m] = (i + 1 < NCH || last_ok) ? v : acc[m];
    }
  }

#pragma unroll
  for (int m = 0; m < M; ++m) {
    float v = row16_sum(acc[m]);
    if (SH >= 5) v += __shfl_xor(v, 16);
    if (SH >= 6) v += __shfl_xor(v, 32);
    if (j == 0 && row < N) store_y(a, P, m, row, v);
  }
}

// ------------------------------------------------------- MFMA kernel (more rows)
//
// A workgroup owns 16*NT weight rows of one problem; its four wavefronts split the
// groups of 64 into quarters and add their partial sums through LDS at the end.  In a
// wavefront, lane (n = lane%16, kg = lane/16) holds, per group g and per 16-row tile,
// the two words 8g+2kg and 8g+2kg+1 of weight row n (one 8-byte load): as B operands of
// two v_mfma_f32_16x16x32_bf16 they cover the group's words {0,2,4,6} and {1,3,5,7}.
// The A operands are the matching x words of activation row m = lane%16 (+16 per
// m-tile), read from memory with the weights of the same stage (x stays in L2) and put
// in pair order.
// D[m][n] lands in lane (n, kg) as rows m = 4*kg + r, r < 4.  Per group:
//     acc += s * P + (b - 128 s) * P1,
// where P1 is the same MFMA pair against a ones operand, i.e. sum x over the group.
//
// Memory-level parallelism: the weight words of GS groups are loaded at once, and the
// next GS groups are in flight while these compute.  The scales and biases of the
// workgroup's rows are staged once in LDS as (s | b << 16) words, [row][group].

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) {
  u32x4_t t = {v.x, v.y, v.z, v.w};
  return __builtin_bit_cast(bf16x8_t, t);
}

__device__ __forceinline__ bf16x8_t unpack_word(uint32_t u, uint32_t magic) {
  u32x4_t t = {nibble_pair(u, 0, magic), nibble_pair(u, 1, magic), nibble_pair(u, 2, magic),
               nibble_pair(u, 3, magic)};
  return __builtin_bit_cast(bf16x8_t, t);
}

// One stage: the weight words (per tile) and the x words (per m-tile) of GS groups.
template <int MT, int NT, int GS>
struct MfmaStage {
  uint2 w[GS][NT];
  uint4 x0[GS][MT];
  uint4 x1[GS][MT];
};

// Weight words of groups g .. g+GS-1 as raw buffer loads (one lane offset per tile plus
// immediate offsets; reads past the matrix return zero, so no group needs a clamp), and
// the matching x words.  Groups past the wavefront's range are loaded but never used.
//
// Every stage is always issued, so the number of loads in flight is the same on every
// path and the compiler's waits stay exact (a conditional stage would make it wait for
// everything).  Groups past the range get an offset past the buffer: the hardware
// returns zero for them without touching memory.
constexpr uint32_t kPastBuffer = 0x80000000u;

template <int MT, int NT, int GS>
__device__ __forceinline__ void load_stage(MfmaStage<MT, NT, GS>& st, __amdgpu_buffer_rsrc_t wrsrc,
                                           const uint32_t (&voff)[NT],
                                           const uint16_t* const (&xr)[MT], int g, int g1) {
#pragma unroll
  for (int i = 0; i < GS; ++i) {
    const uint32_t goff = g + i < g1 ? 32u * (g + i) : kPastBuffer;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(wrsrc, voff[t] + goff, 0, 0);
      st.w[i][t] = make_uint2(v.x, v.y);
    }
  }
#pragma unroll
  for (int i = 0; i < GS; ++i) {
    const int gg = g + i < g1 ? g + i : g1 - 1;  // x rows end at K: stay inside them
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const uint4* xv = reinterpret_cast<const uint4*>(xr[mt] + 64 * gg);
      st.x0[i][mt] = xv[0];
      st.x1[i][mt] = xv[1];
    }
  }
}

template <int MT, int NT, int GS>
__device__ __forceinline__ void compute_stage(const MfmaStage<MT, NT, GS>& st, const uint32_t* sb,
                                              int G, int g, int g1, f32x4_t (&acc)[NT][MT],
                                              uint32_t magic) {
  const u32x4_t ones_u = {kOnes, kOnes, kOnes, kOnes};
  const bf16x8_t ones = __builtin_bit_cast(bf16x8_t, ones_u);
  const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < GS; ++i) {
    if (g + i >= g1) break;
    bf16x8_t a0[MT], a1[MT];
    f32x4_t sumx[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      a0[mt] = as_bf16x8(pair_order(st.x0[i][mt]));
      a1[mt] = as_bf16x8(pair_order(st.x1[i][mt]));
      sumx[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0[mt], ones, zero, 0, 0, 0);
      sumx[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1[mt], ones, sumx[mt], 0, 0, 0);
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const bf16x8_t b0 = unpack_word(st.w[i][t].x, magic);
      const bf16x8_t b1 = unpack_word(st.w[i][t].y, magic);
      const uint32_t pk = sb[t * 16 * G + g + i];
      const float sc = bf16_bits_to_f32(pk & 0xffffu);
      const float bp = fmaf(-128.0f, sc, __uint_as_float(pk & 0xffff0000u));
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        f32x4_t p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0[mt], b0, zero, 0, 0, 0);
        p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1[mt], b1, p, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r)
          acc[t][mt][r] = fmaf(sc, p[r], fmaf(bp, sumx[mt][r], acc[t][mt][r]));
      }
    }
  }
}

template <int MT, int NT, int GS>
__global__ __launch_bounds__(kThreads) void qmv_mfma_kernel(LaunchArgs a) {
  extern __shared__ uint32_t sb_lds[];  // (s | b << 16) per [row of the workgroup][group]
  __shared__ f32x4_t red[3][NT][MT][64];
  const Problem& P = a.p[find_problem(a, blockIdx.x)];
  const int K = P.K, N = P.N, M = a.M;
  const int G = K >> 6, W = K >> 3;
  const int tid = threadIdx.x;
  // the wave index is uniform across the wavefront: keep it (and the group range and
  // loop control derived from it) in scalar registers, so branches are scalar
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int n = lane & 15, kg = lane >> 4;
  const int row0 = (blockIdx.x - P.first) * (16 * NT);
  const uint32_t magic = in_vgpr(kMagic);

  // Scales and biases of the workgroup's rows (one contiguous span each), loaded first
  // so they land before the weights: 16-byte loads when aligned and whole, else halves.
  constexpr int SBV = 4;  // uint4 per thread: spans up to 8192 halves (G <= 8192 / (16 NT))
  const int span = 16 * NT * G;
  const uint16_t* s0 = P.s + (size_t)row0 * G;
  const uint16_t* b0 = P.b + (size_t)row0 * G;
  const bool vec = ((reinterpret_cast<uintptr_t>(s0) | reinterpret_cast<uintptr_t>(b0)) & 15) == 0 &&
                   row0 + 16 * NT <= N && span % 8 == 0 && span <= 8 * kThreads * SBV;
  uint4 sv[SBV], bv[SBV];
  if (vec) {
#pragma unroll
    for (int q = 0; q < SBV; ++q) {
      const int idx = tid + kThreads * q;
      if (idx * 8 < span) {
        sv[q] = reinterpret_cast<const uint4*>(s0)[idx];
        bv[q] = reinterpret_cast<const uint4*>(b0)[idx];
      }
    }
  }

  // the host guarantees N * K / 2 < 2^31, so byte offsets fit the buffer's 32 bits
  const __amdgpu_buffer_rsrc_t wrsrc = buffer_rsrc(P.w, (uint32_t)((size_t)N * W * 4));
  uint32_t voff[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int row = row0 + 16 * t + n;
    const int r = row < N ? row : N - 1;
    voff[t] = ((uint32_t)r * (uint32_t)W + 2u * kg) * 4u;
  }
  // rows m >= M feed MFMA rows whose results are never stored: read row M-1 for them
  const uint16_t* xr[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = n + 16 * mt;
    xr[mt] = x_row(a, P, m < M ? m : M - 1) + 16 * kg;
  }

  // this wavefront's quarter of the groups, in double-buffered stages of GS groups
  const int g0 = (G * wave) >> 2, g1 = (G * (wave + 1)) >> 2;
  MfmaStage<MT, NT, GS> sa, sb2;
  load_stage<MT, NT, GS>(sa, wrsrc, voff, xr, g0, g1 > g0 ? g1 : g0 + 1);

  if (vec) {
#pragma unroll
    for (int q = 0; q < SBV; ++q) {
      const int idx = tid + kThreads * q;
      if (idx * 8 < span) {
        const uint32_t ss[4] = {sv[q].x, sv[q].y, sv[q].z, sv[q].w};
        const uint32_t bb[4] = {bv[q].x, bv[q].y, bv[q].z, bv[q].w};
        uint4 lo, hi;  // entries idx*8 .. idx*8+7: (s | b << 16)
        lo.x = (ss[0] & 0xffffu) | (bb[0] << 16);
        lo.y = (ss[0] >> 16) | (bb[0] & 0xffff0000u);
        lo.z = (ss[1] & 0xffffu) | (bb[1] << 16);
        lo.w = (ss[1] >> 16) | (bb[1] & 0xffff0000u);
        hi.x = (ss[2] & 0xffffu) | (bb[2] << 16);
        hi.y = (ss[2] >> 16) | (bb[2] & 0xffff0000u);
        hi.z = (ss[3] & 0xffffu) | (bb[3] << 16);
        hi.w = (ss[3] >> 16) | (bb[3] & 0xffff0000u);
        reinterpret_cast<uint4*>(sb_lds)[2 * idx] = lo;
        reinterpret_cast<uint4*>(sb_lds)[2 * idx + 1] = hi;
      }
    }
  } else {
    for (int idx = tid; idx < span; idx += kThreads) {  // tail tile or unaligned scales
      const int rr = idx / G, g = idx - rr * G;
      const int row = row0 + rr < N ? row0 + rr : N - 1;
      sb_lds[idx] = (uint32_t)P.s[(size_t)row * G + g] | ((uint32_t)P.b[(size_t)row * G + g] << 16);
    }
  }
  lds_barrier();

  const uint32_t* sbl = sb_lds + n * G;
  f32x4_t acc[NT][MT];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[t][mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  for (int g = g0; g < g1; g += 2 * GS) {
    load_stage<MT, NT, GS>(sb2, wrsrc, voff, xr, g + GS, g1);
    compute_stage<MT, NT, GS>(sa, sbl, G, g, g1, acc, magic);
    if (g + GS >= g1) break;
    load_stage<MT, NT, GS>(sa, wrsrc, voff, xr, g + 2 * GS, g1);
    compute_stage<MT, NT, GS>(sb2, sbl, G, g + GS, g1, acc, magic);
  }

  // add the four quarters: waves 1..3 park their sums in LDS, wave 0 adds and stores
  if (wave > 0) {
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) red[wave - 1][t][mt][lane] = acc[t][mt];
  }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int row = row0 + 16 * t + n;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        f32x4_t v = acc[t][mt];
#pragma unroll
        for (int q = 0; q < 3; ++q) v += red[q][t][mt][lane];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = 16 * mt + 4 * kg + r;
          if (m < M && row < N) store_y(a, P, m, row, v[r]);
        }
      }
    }
  }
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

// ================================================================== host side

thread_local int32_t g_last_code = IMQ_OK;
thread_local std::string g_last_msg;

int32_t fail(int32_t code, const std::string& msg) {
  g_last_code = code;
  g_last_msg = msg;
  return code;
}

int32_t ok() {
  g_last_code = IMQ_OK;
  g_last_msg.clear();
  return IMQ_OK;
}

struct DeviceInfo {
  int state = 0;  // 0 unknown, 1 gfx950, -1 unsupported
  int cu_count = 0;
  char arch[64] = {0};
};

constexpr int kMaxDevices = 64;
DeviceInfo g_devices[kMaxDevices];
std::mutex g_device_mutex;

// Checks once per device that it is a gfx950; returns its info or nullptr.
const DeviceInfo* current_device(int32_t* code) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    *code = fail(IMQ_EUNAVAILABLE, "no HIP device is available");
    return nullptr;
  }
  DeviceInfo& info = g_devices[dev];
  if (__atomic_load_n(&info.state, __ATOMIC_ACQUIRE) == 0) {
    std::lock_guard<std::mutex> lock(g_device_mutex);
    if (info.state == 0) {
      hipDeviceProp_t prop;
      if (hipGetDeviceProperties(&prop, dev) != hipSuccess) {
        *code = fail(IMQ_EUNAVAILABLE, "hipGetDeviceProperties failed");
        return nullptr;
      }
      strncpy(info.arch, prop.gcnArchName, sizeof(info.arch) - 1);
      info.cu_count = prop.multiProcessorCount;
      const bool is950 = strncmp(prop.gcnArchName, "gfx950", 6) == 0;
      __atomic_store_n(&info.state, is950 ? 1 : -1, __ATOMIC_RELEASE);
    }
  }
  if (info.state != 1) {
    *code = fail(IMQ_EUNAVAILABLE,
                 std::string("device architecture ") + info.arch + " is not gfx950");
    return nullptr;
  }
  return &info;
}

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

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
constexpr int kMfmaTiles = 2;  // 16-row tiles per MFMA workgroup
constexpr size_t kMfmaLdsLimit = 48 * 1024;  // its (scale, bias) table; K up to 24576

// Lanes per weight row for the VALU kernel: the widest of 64/32/16 that still gives
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

// Tiles of the VALU kernel: 4 wavefronts x 64/LPR rows.  Returns the LDS bytes for the
// largest x of the launch, or 0 if some x does not fit.
size_t plan_rows(LaunchArgs& a) {
  size_t lds = 0;
  int64_t tiles = 0;
  for (int i = 0; i < a.count; ++i) {
    Problem& P = a.p[i];
    P.lpr_shift = choose_lpr_shift(P.K);
    const int rows = 256 >> P.lpr_shift;
    P.first = (int32_t)tiles;
    tiles += (P.N + rows - 1) / rows;
    const size_t need = (size_t)a.M * (P.K / 32) * (64 + 4);
    lds = need > lds ? need : lds;
  }
  if (lds > kValuLdsLimit || tiles > 0x7fffffff) return 0;
  a.items = (int32_t)tiles;
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

template <int M, int SH, int NCH>
hipError_t launch_fixed(const LaunchArgs& a, size_t lds, hipStream_t stream) {
  hipLaunchKernelGGL((qmv_fixed_kernel<M, SH, NCH>), dim3(a.items), dim3(kThreads), lds, stream,
                     a);
  return hipGetLastError();
}

// The compile-time kernel for (M, SH, NCH) if one is built: SH 4 with 1..8 chunks per
// lane, SH 5 and 6 with 4..8.  Returns false when none matches.
template <int M>
bool launch_fixed_for(const LaunchArgs& a, int sh, int nch, size_t lds, hipStream_t stream,
                      hipError_t* e) {
#define IMQ_FIXED(S, NC) \
  if (sh == S && nch == NC) { *e = launch_fixed<M, S, NC>(a, lds, stream); return true; }
  IMQ_FIXED(4, 1) IMQ_FIXED(4, 2) IMQ_FIXED(4, 3) IMQ_FIXED(4, 4)
  IMQ_FIXED(4, 5) IMQ_FIXED(4, 6) IMQ_FIXED(4, 7) IMQ_FIXED(4, 8)
  IMQ_FIXED(5, 4) IMQ_FIXED(5, 5) IMQ_FIXED(5, 6) IMQ_FIXED(5, 7) IMQ_FIXED(5, 8)
  IMQ_FIXED(6, 4) IMQ_FIXED(6, 5) IMQ_FIXED(6, 6) IMQ_FIXED(6, 7) IMQ_FIXED(6, 8)
#undef IMQ_FIXED
  return false;
}

template <int M, int B>
hipError_t launch_rows(const LaunchArgs& a, size_t lds, hipStream_t stream) {
  hipLaunchKernelGGL((qmv_rows_kernel<M, B>), dim3(a.items), dim3(kThreads), lds, stream, a);
  return hipGetLastError();
}

constexpr int kMfmaStage = 4;  // groups of weight and x words loaded at once per wavefront

template <int MT>
hipError_t launch_mfma(const LaunchArgs& a, int grid, size_t lds, hipStream_t stream) {
  hipLaunchKernelGGL((qmv_mfma_kernel<MT, kMfmaTiles, kMfmaStage>), dim3(grid), dim3(kThreads),
                     lds, stream, a);
  return hipGetLastError();
}

// Plans the work of every problem and launches one kernel for all of them.
int32_t launch(LaunchArgs& a, const DeviceInfo* dev, hipStream_t stream) {
  (void)dev;
  const int M = a.M;
  hipError_t e;
  const size_t lds = M <= kValuMaxRows ? plan_rows(a) : 0;
  if (lds > 0) {
    // one (lanes per row, chunks per lane) shape for every problem: the fixed kernel
    int sh = a.p[0].lpr_shift, nch = -1;
    for (int i = 0; i < a.count; ++i) {
      const int lpr = 1 << a.p[i].lpr_shift;
      const int n = (a.p[i].K / 32 + lpr - 1) / lpr;
      if (a.p[i].lpr_shift != sh || (nch >= 0 && n != nch)) sh = -1;
      nch = n;
    }
    if (sh >= 0 && M == 1) {  // at M = 2 the fixed kernel needs too many registers
      if (launch_fixed_for<1>(a, sh, nch, lds, stream, &e)) {
        if (e != hipSuccess)
          return fail(IMQ_ELAUNCH, std::string("qmv launch failed: ") + hipGetErrorString(e));
        return ok();
      }
    }
    if (M == 1) {
      static const int opts[] = {4, 5};
      e = choose_batch(a, opts, 2) == 4 ? launch_rows<1, 4>(a, lds, stream)
                                        : launch_rows<1, 5>(a, lds, stream);
    } else {
      e = launch_rows<2, 2>(a, lds, stream);
    }
  } else {
    const int rows_per_wg = 16 * kMfmaTiles;
    int64_t tiles = 0;
    for (int i = 0; i < a.count; ++i) {
      a.p[i].first = (int32_t)tiles;
      tiles += (a.p[i].N + rows_per_wg - 1) / rows_per_wg;
    }
    if (tiles > 0x7fffffff) return fail(IMQ_EUNSUPPORTED, "too many rows for one launch");
    int kmax = 0;
    for (int i = 0; i < a.count; ++i) kmax = a.p[i].K > kmax ? a.p[i].K : kmax;
    const size_t lds = (size_t)rows_per_wg * (kmax / 64) * 4;  // (s, b) per row and group
    if (lds > kMfmaLdsLimit) return fail(IMQ_EUNSUPPORTED, "K too large for the MFMA kernel");
    for (int i = 0; i < a.count; ++i)
      if ((int64_t)a.p[i].N * (a.p[i].K / 2) >= ((int64_t)1 << 31))
        return fail(IMQ_EUNSUPPORTED, "a weight of 2 GiB or more exceeds the MFMA kernel's offsets");
    e = (M <= 16) ? launch_mfma<1>(a, (int)tiles, lds, stream)
                  : launch_mfma<2>(a, (int)tiles, lds, stream);
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
  if (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < kMaxDevices) {
    current_device(&code);
    if (arch && arch_len) {
      strncpy(arch, g_devices[dev].arch, arch_len - 1);
      arch[arch_len - 1] = 0;
    }
    if (cu_count) *cu_count = g_devices[dev].cu_count;
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

int32_t imq_qmv_grouped(const imq_problem* problems, int32_t count, int32_t M,
                        int32_t group_size, int32_t bits, int32_t y_dtype, void* stream) {
  if (!problems) return fail(IMQ_EINVAL, "problems must be non-null");
  if (count < 1) return fail(IMQ_EINVAL, "count must be >= 1");
  if (count > IMQ_MAX_PROBLEMS)
    return fail(IMQ_EUNSUPPORTED, "at most IMQ_MAX_PROBLEMS problems per call");
  int32_t code = check_dtype(y_dtype);
  if (code != IMQ_OK) return code;
  LaunchArgs a;
  memset(&a, 0, sizeof(a));
  for (int i = 0; i < count; ++i) {
    const imq_problem& q = problems[i];
    if ((code = check_format(q.N, q.K, group_size, bits)) != IMQ_OK) return code;
    if ((code = check_weights(q.w, q.scales, q.biases)) != IMQ_OK) return code;
    if ((code = check_rows(q.x, q.ldx, q.y, q.ldy, M, q.N, q.K, y_dtype)) != IMQ_OK) return code;
    a.p[i] = Problem{q.w, q.scales, q.biases, q.x, q.y, M > 1 ? q.ldx : q.K,
                     M > 1 ? q.ldy : q.N, q.N, q.K, 0, 0, 0, 0};
  }
  const DeviceInfo* dev = current_device(&code);
  if (!dev) return code;
  a.count = count;
  a.M = M;
  a.y_f32 = (y_dtype == IMQ_F32);
  return launch(a, dev, static_cast<hipStream_t>(stream));
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

int32_t imq_last_error(char* buf, size_t len) {
  if (buf && len) {
    strncpy(buf, g_last_msg.c_str(), len - 1);
    buf[len - 1] = 0;
  }
  return g_last_code;
}

}  // extern "C"
