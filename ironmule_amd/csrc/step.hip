// Persistent decode-step engine for MI355X (gfx950): one kernel launch runs a whole
// program of stages (C ABI: include/ironmule_step.h).
//
// Scheduling.  The tasks of all stages form one list in stage order.  The grid holds as
// many workgroups as the device keeps resident at once, and workgroup w runs tasks
// w, w + G, w + 2G, ... in order.  A task first issues its weight loads, then waits
// until every task of its input stage has finished, then reads its activations, computes
// and publishes its outputs.  Because every workgroup is resident and runs its tasks in
// increasing order, the smallest unfinished task can always run, so the program always
// completes; the waits are bounded anyway (a stalled run stops and reports it).
//
// Completion.  Each stage has kSub counters, each on its own cache line and the lines of
// one stage's counters 4 KiB apart: one atomic counter serialises its increments (about
// 11 ns each on MI355X), so a stage's tasks spread theirs over kSub of them.  A waiting
// workgroup sums the kSub counters with one round of loads per poll.
//
// Coherence inside a launch.  Activations produced by one task and read by another
// (the residual stream h, q/k/v, the attention partials and output, SiLU*up) are
// written with sc1 stores and read with sc1 loads (common.h), and a producer waits for
// its stores before it bumps a counter.  No cache write-back or invalidate is used: an
// agent-scope acquire (a full L2 invalidate) costs tens of microseconds when thousands of
// workgroups issue it.
//
// Arithmetic.  A qmv tile is the one-row VALU tile of qmv.hip (the same lane shape, chunk
// order, dot2 chains and cross-lane sums); the fused RMSNorm, the residual add, SiLU*up,
// q/k norm + rotary embedding and attention use the expressions and reduction orders of
// the decode.hip kernels.  A program's results therefore equal the per-kernel path's bit
// for bit.

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <string>
#include <type_traits>
#include <vector>

#include "../../include/ironmule_decode.h"
#include "../../include/ironmule_step.h"
#include "common.h"
#include "runtime.h"

namespace {

using namespace imq_dev;
using imq_rt::aligned;
using imq_rt::current_device;
using imq_rt::DeviceInfo;
using imq_rt::fail;
using imq_rt::ok;

constexpr int kThreads = 256;
constexpr int kD = 128;           // attention head dimension
constexpr int kChunk = 64;        // keys per attention chunk
constexpr int kSub = 16;          // completion counters per stage
constexpr int kLineWords = 32;    // one 128-byte line per counter
constexpr int kMaxPolls = 1 << 22;
constexpr int kMaxStageProblems = 3;
constexpr int kMaxHidden = 4096;  // the fused RMSNorm stages one row of h whole
constexpr int kNormVpt = kMaxHidden / kThreads;

enum : int32_t { kKindQmv = 0, kKindAttention = 1 };
// x sources: a bf16 row; the RMSNorm of the fp32 row of h computed in the task; or x' =
// bf16(h * w) with the rows' outputs scaled by 1/rms(h) from the producer's partial sums of
// squares (the RMSNorm folded into the projections around it)
enum : int32_t { kXVector = 0, kXNorm = 1, kXScaled = 2 };
// epilogues: bf16 or fp32 y; h += bf16(y); SiLU(gate) * up; h += bf16(y) with the next
// RMSNorm's x' = bf16(h * w_next) and the tile's sum of squares of h
enum : int32_t { kEpiBf16 = 0, kEpiF32 = 1, kEpiResidual = 2, kEpiSiluPair = 3, kEpiResidualNorm = 4 };
constexpr int kMaxNormParts = 4096;  // partial sums of squares a kXScaled stage reads
// (chunks per lane, x pieces per thread) of the qmv tile instantiations
enum : int32_t { kShape22 = 0, kShape52 = 1, kShape82 = 2, kShape55 = 3 };

struct QProb {
  const uint32_t* w;
  const uint16_t* s;
  const uint16_t* b;
  void* y;
  int32_t N, K, sh, nch;
  int32_t tile_end;  // one past the problem's last tile, counted within the stage
  int32_t pad[3];
};

struct Stage {
  int32_t kind, first, count, wait;  // wait: stage index, or -1
  int32_t wait_count, shape, xsrc, epi;
  int32_t nprob, nssq, pad1, pad2a;  // nssq: kXScaled's partial sums of squares
  float eps, log2_theta, scale, pad2;
  const uint16_t* x;       // bf16 activation row (kXVector, kXScaled)
  float* h;                // residual stream (kXNorm source, kEpiResidual(Norm) target)
  const uint16_t* norm_w;  // kXNorm weight
  uint16_t* act;           // kEpiSiluPair output
  const float* ssq_in;         // kXScaled: the producer's per-tile sums of squares of h
  float* ssq_out;              // kEpiResidualNorm: this stage's per-tile sums of squares
  uint16_t* xn_out;            // kEpiResidualNorm: x' = bf16(h * norm_next)
  const uint16_t* norm_next;   // kEpiResidualNorm: the next RMSNorm's weight
  QProb p[kMaxStageProblems];
  // attention
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* q_norm;
  const uint16_t* k_norm;
  uint16_t* k_pool;
  uint16_t* v_pool;
  uint16_t* attn_out;
  const int32_t* positions;
  const int32_t* slots;
  float* part;
  float* ml;
  uint32_t* combine;  // one counter per (request, KV head)
  int32_t Hq, Hkv, capacity, num_slots, max_len, splits, cps;
  int32_t out_tiled;  // 1: the attention output in the 32-row tile layout (else rows Hq * 128 apart)
  // q, k and v as fp32 output planes of a split projection instead (staged launches only):
  // problem i (q, k, v), plane s, request b at qkv + i * qkv_pstride + (s * qkv_rows + b) * N_i
  const float* qkv;
  int64_t qkv_pstride;
  int32_t qkv_splits, qkv_rows;
};

constexpr int kMaxQkvPlanes = 4;

struct StepArgs {
  uint32_t* done;
  uint32_t* status;
  int32_t ntasks;
  int32_t sub_stride;  // counters between the same sub-counter of consecutive stages
  int32_t staged;      // 1: one launch per stage (stream order replaces the waits)
  int32_t pad;
};

__device__ __forceinline__ float bf(uint32_t h) { return bf16_bits_to_f32(h); }
__device__ __forceinline__ uint16_t to_bf(float f) { return f32_to_bf16_bits(f); }

// A value the whole workgroup agrees on, kept in a scalar register (a vector load of a
// uniform address would otherwise make everything derived from it look divergent).
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }

// threadIdx.x made opaque at the start of each task, so that values derived from it are
// computed inside the task loop rather than hoisted and kept live across every task.
__device__ __forceinline__ int task_tid() {
  int t = threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}
// A stage descriptor seen through the global address space: loads of its fields are then
// known to be the same for every lane (flat loads might reach per-lane scratch).
typedef const struct Stage __attribute__((address_space(1)))& StageRef;
__device__ __forceinline__ StageRef global_stage(const Stage* p);

template <typename T>
__device__ __forceinline__ T* uni(T* p) {
  const uint64_t u = reinterpret_cast<uint64_t>(p);
  const uint64_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)u);
  const uint64_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(u >> 32));
  return reinterpret_cast<T*>((hi << 32) | lo);
}

__device__ __forceinline__ StageRef global_stage(const Stage* p) {
  return *reinterpret_cast<const Stage __attribute__((address_space(1)))*>(
      reinterpret_cast<uint64_t>(uni(p)));
}

__device__ __forceinline__ uint32_t* counter(const StepArgs& a, int stage, int sub) {
  return a.done + ((size_t)sub * a.sub_stride + stage) * kLineWords;
}

// Waits until the kSub counters of `stage` add up to `count`.  Wavefront 0 polls (lane i
// reads counter i), with a short sleep between polls.  Returns false (and raises the
// status word) if the wait times out or another workgroup raised it.
__device__ bool wait_stage(const StepArgs& a, int stage, uint32_t count) {
  __shared__ int s_ok;
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    const uint32_t* c = counter(a, stage, lane < kSub ? lane : 0);
    int polls = 0, good = 1;
    for (;;) {
      uint32_t v = lane < kSub ? ld_sc1(c) : 0u;
#pragma unroll
      for (int o = 8; o > 0; o >>= 1) v += __shfl_xor(v, o);
      v = __shfl(v, 0);
      if (v >= count) break;
      if (++polls >= kMaxPolls || ((polls & 63) == 0 && ld_sc1(a.status) != 0)) {
        good = 0;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (lane == 0) {
      if (!good) st_sc1(a.status, 1u);
      s_ok = good;
    }
  }
  __syncthreads();
  return s_ok != 0;
}

// After the task's sc1 stores: every thread waits for its own, then one atomic.
__device__ __forceinline__ void signal(uint32_t* c) {
  wait_vmem();
  __syncthreads();
  if (threadIdx.x == 0) __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ------------------------------------------------------------------ qmv tile
//
// LDS of a qmv task: x in pair order as four planes of CP chunks, their chunk sums, the
// tile's (scale, bias) dwords, then (fused RMSNorm) the normalised row as bf16 and the
// block sums, and the SiLU*up exchange.
template <int NCH, int XR>
struct QLds {
  static constexpr int kChunks = XR * 64;
  static constexpr int kSbr = (64 * NCH + kThreads - 1) / kThreads;
  static constexpr size_t kX = 0;
  static constexpr size_t kSx = kX + (size_t)4 * kChunks * 16;
  static constexpr size_t kSb = kSx + (size_t)kChunks * 4;
  static constexpr size_t kPair = kSb + (size_t)kSbr * kThreads * 8;  // 8 floats
  static constexpr size_t kRed = kPair + 8 * 4;  // the wavefronts' sums of squares (4 floats)
  static constexpr size_t kBytes = kRed + 4 * 4;
};

// The fused RMSNorm holds the fp32 row of h at the start of LDS (it is consumed before
// the x planes are written over it) and its block sums after the largest row.
constexpr size_t kNormRed = (size_t)kMaxHidden * 4;
constexpr size_t kNormBytes = kNormRed + 16;

// Loads that may see data written earlier in the same launch use sc1 (`kSc1` true);
// in a staged launch the previous stage ended with its kernel, and plain loads do.
template <bool kSc1Load>
__device__ __forceinline__ uint4 load_act(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return kSc1Load ? load_b128_sc1(r, off) : load_b128(r, off);
}

// x for the tile from a bf16 row.  Pieces past the row lie past the buffer and read as
// zero.
template <int XR, bool kSc1Load>
__device__ __forceinline__ void load_x(const uint16_t* x, int K, int tid, uint4 (&xs)[XR]) {
  const __amdgpu_buffer_rsrc_t r = buffer_rsrc(x, (uint32_t)K * 2u);
#pragma unroll
  for (int t = 0; t < XR; ++t) xs[t] = load_act<kSc1Load>(r, 16u * (tid + kThreads * t));
}

// The fp32 row of h as each thread's own 8-value pieces (values 8i .. 8i+7 of piece
// i = tid + 256 t; zeros past the row).
template <int XR, bool kSc1Load>
__device__ __forceinline__ void load_h(const float* h, int K, int tid, uint4 (&h0)[XR],
                                       uint4 (&h1)[XR]) {
  const __amdgpu_buffer_rsrc_t hr = buffer_rsrc(h, (uint32_t)K * 4u);
#pragma unroll
  for (int t = 0; t < XR; ++t) {
    const uint32_t off = 32u * (tid + kThreads * t);
    h0[t] = load_act<kSc1Load>(hr, off);
    h1[t] = load_act<kSc1Load>(hr, off + 16u);
  }
}

// x = bf16(rms_norm(h) * w) for the tile from the pieces of h and of the norm weight,
// with the sum of squares in the order of add_rmsnorm_kernel (thread t adds the squares
// of h[t + 256 i] in increasing i, then the wavefront butterfly, then the four
// wavefronts as (w0 + w1) + (w2 + w3)): the row goes through LDS for the strided sums.
template <int XR>
__device__ __forceinline__ void norm_x(const uint4 (&h0)[XR], const uint4 (&h1)[XR],
                                       const uint4 (&wn)[XR], int K, float eps, int tid,
                                       float* hl, float* red, uint4 (&xs)[XR]) {
#pragma unroll
  for (int t = 0; t < XR; ++t) {
    uint4* dst = reinterpret_cast<uint4*>(hl) + 2 * (tid + kThreads * t);
    dst[0] = h0[t];
    dst[1] = h1[t];
  }
  lds_barrier();
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < kNormVpt; ++i) {
    const int idx = tid + kThreads * i;
    if (idx < K) ss = fmaf(hl[idx], hl[idx], ss);
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  lds_barrier();
  const float total = (red[0] + red[1]) + (red[2] + red[3]);
  const float inv = 1.0f / sqrtf(total / (float)K + eps);
#pragma unroll
  for (int t = 0; t < XR; ++t) {
    const uint32_t ww[4] = {wn[t].x, wn[t].y, wn[t].z, wn[t].w};
    const float hv[8] = {__uint_as_float(h0[t].x), __uint_as_float(h0[t].y),
                         __uint_as_float(h0[t].z), __uint_as_float(h0[t].w),
                         __uint_as_float(h1[t].x), __uint_as_float(h1[t].y),
                         __uint_as_float(h1[t].z), __uint_as_float(h1[t].w)};
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      o[e] = (uint32_t)to_bf(hv[2 * e] * inv * bf(ww[e] & 0xffffu)) |
             ((uint32_t)to_bf(hv[2 * e + 1] * inv * bf(ww[e] >> 16)) << 16);
    xs[t] = make_uint4(o[0], o[1], o[2], o[3]);
  }
  lds_barrier();  // the x planes are written over the row
}

// One qmv task: one tile of one problem (tiles are numbered across the stage's
// problems), or for a SiLU*up pair stage one tile of the gate/up pair, whose rows 0-7
// are gate rows and rows 8-15 the same up rows (wavefronts 0-1 and 2-3).
//
// The persistent form (kStaged false) issues the weight loads first and then waits for its
// input stage; a staged launch (kStaged true) has its inputs ready, and issues their loads
// first so that staging x overlaps the weight stream (loads return in issue order).
template <int NCH, int XR, int XSRC, int EPI, bool kStaged, typename SRef>
__device__ __forceinline__ bool qmv_task(SRef S, int task, const StepArgs& a, uint4* smem) {
  using L = QLds<NCH, XR>;
  constexpr int CP = L::kChunks, SBR = L::kSbr;
  constexpr bool kPair = EPI == kEpiSiluPair;
  const int tid = task_tid();
  const int wave = uni(tid >> 6);
  int pi = 0, tile = task;
  if (!kPair) {
    if (S.nprob > 1 && task >= S.p[0].tile_end) pi = 1;
    if (S.nprob > 2 && task >= S.p[1].tile_end) pi = 2;
    if (pi > 0) tile = task - S.p[pi - 1].tile_end;
  }
  const int qi = kPair ? (wave >= 2 ? 1 : 0) : pi;  // this wavefront's problem
  const uint32_t* wp = S.p[qi].w;
  const uint16_t* sp = S.p[qi].s;
  const uint16_t* bp = S.p[qi].b;
  const int K = S.p[0].K, N = S.p[qi].N, sh = S.p[0].sh, nch = S.p[0].nch;
  const int C = K >> 5, G = K >> 6, W = K >> 3;
  const int j = tid & ((1 << sh) - 1);
  const int rl = tid >> sh;  // the lane's row within the tile
  const int rows = kPair ? 8 : (kThreads >> sh);
  const int row0 = tile * rows;
  const int row = row0 + (kPair ? (rl & 7) : rl);
  uint4* xq = smem;
  float* sx = reinterpret_cast<float*>(reinterpret_cast<char*>(smem) + L::kSx);
  uint32_t* sbl = reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(smem) + L::kSb);
  const uint32_t magic = in_vgpr(kMagic);

  // the activation inputs: x, or the row of h and the norm weight (or x' and the partial
  // sums of squares); a residual stage also reads its rows of h (final once the input
  // stage is done) and, folding the next RMSNorm, that norm's weights of its rows
  const bool owner = j == 0 && row < N;
  constexpr bool kScaled = XSRC == kXScaled;
  constexpr bool kResNorm = EPI == kEpiResidualNorm;
  constexpr int HX = XSRC == kXNorm ? XR : 1;
  constexpr int NQ = kScaled ? kMaxNormParts / (4 * kThreads) : 1;
  uint4 xs[XR], h0[HX], h1[HX], wn[HX], nq[NQ];
  float hres = 0.0f;
  uint32_t wnext = 0u;
  auto load_inputs = [&]() {
    if constexpr (XSRC == kXNorm)
      load_h<XR, !kStaged>(S.h, K, tid, h0, h1);
    else
      load_x<XR, !kStaged>(S.x, K, tid, xs);
    if constexpr (kScaled) {
      const __amdgpu_buffer_rsrc_t qr = buffer_rsrc(S.ssq_in, (uint32_t)S.nssq * 4u);
#pragma unroll
      for (int t = 0; t < NQ; ++t) nq[t] = load_act<!kStaged>(qr, 16u * (tid + kThreads * t));
    }
    // (branch-free: a lane that owns no row reads past the buffers, zeros; under a branch
    // the compiler widened the weight inside it and waited there for every earlier load,
    // x's included, before issuing any of the tile's weights)
    if constexpr (EPI == kEpiResidual || kResNorm) {
      const __amdgpu_buffer_rsrc_t hr = buffer_rsrc(S.h, (uint32_t)N * 4u);
      const uint32_t off = owner ? 4u * (uint32_t)row : kPastBuffer;
      hres = __uint_as_float(kStaged ? __builtin_amdgcn_raw_buffer_load_b32(hr, off, 0, 0) : load_b32_sc1(hr, off));
    }
    if constexpr (kResNorm)
      wnext = __builtin_amdgcn_raw_buffer_load_b16(buffer_rsrc(S.norm_next, (uint32_t)N * 2u),
                                                   owner ? 2u * (uint32_t)row : kPastBuffer, 0, 0);
  };
  auto load_norm_weight = [&]() {
    if constexpr (XSRC == kXNorm) {
      const __amdgpu_buffer_rsrc_t nr = buffer_rsrc(S.norm_w, (uint32_t)K * 2u);
#pragma unroll
      for (int t = 0; t < XR; ++t) wn[t] = load_b128(nr, 16u * (tid + kThreads * t));
    }
  };
  if constexpr (kStaged) {
    load_inputs();
    load_norm_weight();
  }

  // the tile's (scale, bias) span (a pair tile: threads 0-127 the 8 gate rows, 128-255
  // the 8 up rows), rounded up to whole dwords (the extra half lies in the same aligned
  // dword as the last one and belongs to no row)
  const uint32_t sb_bytes = ((uint32_t)N * (uint32_t)G * 2u + 3u) & ~3u;
  const __amdgpu_buffer_rsrc_t srsrc = buffer_rsrc(sp, sb_bytes);
  const __amdgpu_buffer_rsrc_t brsrc = buffer_rsrc(bp, sb_bytes);
  const int st = kPair ? (tid & 127) : tid;
  const int D = (rows * G) >> 1;
  const uint32_t sb0 = (uint32_t)row0 * (uint32_t)G * 2u;
  uint32_t sv[SBR], bv[SBR];
#pragma unroll
  for (int q = 0; q < SBR; ++q) {
    const int d = st + (kPair ? kThreads / 2 : kThreads) * q;
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
  // every load is issued before the first wait: left to itself the scheduler moves the x
  // staging below (and the wait for x it needs) ahead of the last weight chunks' loads
  __builtin_amdgcn_sched_barrier(0);

  if constexpr (!kStaged) {
    load_norm_weight();
    if (S.wait >= 0 && !wait_stage(a, S.wait, (uint32_t)S.wait_count)) return false;
    load_inputs();
  }
  if constexpr (XSRC == kXNorm)
    norm_x<XR>(h0, h1, wn, K, S.eps, tid, reinterpret_cast<float*>(smem),
               reinterpret_cast<float*>(reinterpret_cast<char*>(smem) + kNormRed), xs);
#pragma unroll
  for (int t = 0; t < XR; ++t) {
    const int i = tid + kThreads * t;  // the four words of a chunk are four aligned lanes
    xq[(i & 3) * CP + (i >> 2)] = pair_order(xs[t]);
    float part = sum8(xs[t]);
    part += dpp<0xB1>(part);  // lane ^ 1
    part += dpp<0x4E>(part);  // lane ^ 2
    if ((i & 3) == 0) sx[i >> 2] = part;
  }
  // 1/rms(h) from the partial sums: each thread adds its pieces in order, the wavefronts
  // their lanes (wave_sum), the four wavefront sums meet after the barrier below
  float* red = reinterpret_cast<float*>(reinterpret_cast<char*>(smem) + L::kRed);
  if constexpr (kScaled) {
    float ss = 0.0f;
#pragma unroll
    for (int t = 0; t < NQ; ++t)
      ss += (__uint_as_float(nq[t].x) + __uint_as_float(nq[t].y)) +
            (__uint_as_float(nq[t].z) + __uint_as_float(nq[t].w));
    ss = wave_sum(ss);
    if ((tid & 63) == 0) red[wave] = ss;
  }
  const int sbase = kPair && tid >= 128 ? 4 * G : 0;  // dword offset of the up rows' span
#pragma unroll
  for (int q = 0; q < SBR; ++q) {
    const int d = st + (kPair ? kThreads / 2 : kThreads) * q;
    if (d < D)
      *reinterpret_cast<uint2*>(sbl + 2 * (sbase + d)) =
          make_uint2((sv[q] & 0xffffu) | (bv[q] << 16), (sv[q] >> 16) | (bv[q] & 0xffff0000u));
  }
  lds_barrier();

  float acc = 0.0f;
  const uint32_t* sbr = sbl + rl * G;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    if (i < nch) {
      const int kc = j + (i << sh);
      const bool valid = kc < C;
      const int kk = valid ? kc : 0;
      const uint32_t sb = sbr[kk >> 1];
      const float sc = __uint_as_float(sb << 16);
      const float bi = __uint_as_float(sb & 0xffff0000u);
      const float sxm = sx[kk];
      const float d = chunk_dot(wv[i], xq[kk], xq[CP + kk], xq[2 * CP + kk], xq[3 * CP + kk],
                                -128.0f * sxm, magic);
      const float v = fmaf(sc, d, fmaf(bi, sxm, acc));
      acc = valid ? v : acc;
    }
  }
  float v = row16_sum(acc);
  if (sh >= 5) v = add_xor16(v);
  if (sh >= 6) v = add_xor32(v);
  if constexpr (kScaled) v *= 1.0f / sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (float)K + S.eps);

  if (EPI == kEpiBf16) {
    if (owner) store_b16_sc1(buffer_rsrc(S.p[qi].y, (uint32_t)N * 2u), 2u * row, to_bf(v));
  } else if (EPI == kEpiF32) {
    if (owner) static_cast<float*>(S.p[qi].y)[row] = v;
  } else if (EPI == kEpiResidual) {
    if (owner) stf_sc1(S.h + row, hres + bf(to_bf(v)));
  } else if (EPI == kEpiResidualNorm) {
    // h += bf16(y), x' = bf16(h * w_next), and the tile's sum of squares of the new h: the
    // owners' squares summed per wavefront (wave_sum), then the four wavefronts in order
    float sq = 0.0f;
    if (owner) {
      const float hn = hres + bf(to_bf(v));
      stf_sc1(S.h + row, hn);
      store_b16_sc1(buffer_rsrc(S.xn_out, (uint32_t)N * 2u), 2u * row, to_bf(hn * bf(wnext)));
      sq = hn * hn;
    }
    sq = wave_sum(sq);
    if ((tid & 63) == 0) red[wave] = sq;
    lds_barrier();
    if (tid == 0) stf_sc1(S.ssq_out + tile, (red[0] + red[1]) + (red[2] + red[3]));
  } else {  // SiLU * up: the up rows hand their values to the gate rows
    float* pairx = reinterpret_cast<float*>(reinterpret_cast<char*>(smem) + L::kPair);
    if (j == 0 && rl >= 8) pairx[rl - 8] = v;
    lds_barrier();
    if (owner && rl < 8) {
      const float g0 = bf(to_bf(v));
      const float u = bf(to_bf(pairx[rl]));
      store_b16_sc1(buffer_rsrc(S.act, (uint32_t)N * 2u), 2u * row,
                    to_bf(g0 / (1.0f + expf(-g0)) * u));
    }
  }
  return true;
}

// ------------------------------------------------------------------ attention
//
// Task (request b, KV head, split s) over keys [s * cps * 64, ...) of the request's
// length pos + 1.  The task rotates its G query heads and the new key itself (the
// arithmetic of qk_norm_rope_kernel), takes the new key and value from registers at
// row pos (the split that holds pos also writes them into the pools), and runs the
// chunk loop of attention_partial_kernel with q in LDS and K then V of a chunk sharing
// one LDS region.  The last split of a (request, KV head) to finish merges the partials
// in split order (attention_combine_kernel's arithmetic) into the bf16 output.

constexpr int kMergeBatch = 16;  // splits whose partials a merge loads at once
constexpr uint32_t kNegZeroPair = 0x80008000u;  // the bf16 pair (-0, -0)

constexpr int kAttnWaves = kThreads / 64;
constexpr int kUnit = 16;  // keys a wavefront takes at a time (the chunk's four wavefronts: 64)
// Dwords per row of a wavefront's V^T tile: 16 keys (8 dwords) and 2 of padding, so that the
// MFMA operand reads (16 lanes: 16 dimensions of one key quad) touch distinct banks.
constexpr int kVtStride = 10;

template <int W>
struct AttnLdsT {
  union {
    struct {
      uint32_t vt[W][kD][kVtStride];  // per wavefront: V^T of its 16 keys, bf16 pairs of keys
      // per wavefront (the wide launch only): its 16 keys, 16-byte piece p of key r at
      // r * 16 + (p ^ r)
      uint4 ks[W > kAttnWaves ? W : 1][16 * 16];
    } tile;
    struct {
      float acc[W][8][kD];  // per wavefront and query head: its chunks' weighted sum
      float ml[W][8][2];    // and their (max, sum of exponentials)
    } merge;
  } u;
  uint32_t qs[8][kD / 2];  // rotated q of the task's heads, bf16 pairs
  uint32_t knew[kD / 2];
  uint32_t vnew[kD / 2];
  int last;
};
using AttnLds = AttnLdsT<kAttnWaves>;

// a if m is all ones, b if m is zero (a value select the compiler keeps in registers)
__device__ __forceinline__ uint4 select4(uint32_t m, uint4 a, uint4 b) {
  return make_uint4((a.x & m) | (b.x & ~m), (a.y & m) | (b.y & ~m), (a.z & m) | (b.z & ~m),
                    (a.w & m) | (b.w & ~m));
}

__device__ __forceinline__ uint16_t ld16_sc1(const uint16_t* base, uint32_t bytes, uint32_t off) {
  return (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(buffer_rsrc(base, bytes), off, 0, kSc1);
}

// kPlanes (staged launches only): q, k and v arrive as the fp32 K-range planes of the q/k/v
// launch (Stage::qkv) rather than as bf16 rows; one instantiation per form, so that each has
// one sequence of loads and its waits count them exactly.
template <bool kStaged, typename SRef, int W = kAttnWaves, bool kPlanes = false>
__device__ __forceinline__ bool attention_task(SRef S, int task, const StepArgs& a, uint4* smem) {
  AttnLdsT<W>& L = *reinterpret_cast<AttnLdsT<W>*>(smem);
  constexpr int kRounds = (8 + W - 1) / W;  // query heads (at most 8) per wavefront
  const int splits = S.splits, Hkv = S.Hkv, Hq = S.Hq, G = Hq / Hkv;
  const int s = task % splits, kvh = (task / splits) % Hkv, b = task / (splits * Hkv);
  const int tid = task_tid(), wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  // Every load that needs only the task goes out first: the position and slot, then (staged)
  // q, the new key and value (or their planes) and the norm weights.  The K/V loads need the
  // position and follow as soon as it has landed; the q/k/v values are used only after them
  // (loads return in issue order, so each wait covers exactly the loads before it).  With
  // the q/k/v values first read after the position, the first K/V load left 4 us into the
  // launch at batch 32.
  const int pos_in = S.positions[b], slot_in = S.slots[b];
  const float eps = S.eps;
  const uint32_t qbytes = (uint32_t)(b + 1) * Hq * kD * 2u;
  const uint32_t kvbytes = (uint32_t)(b + 1) * Hkv * kD * 2u;
  const uint32_t kvoff = (uint32_t)((b * Hkv + kvh) * kD) * 2u;
  auto ld16 = [&](const uint16_t* p, uint32_t bytes, uint32_t off) -> uint32_t {
    return kStaged ? (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(buffer_rsrc(p, bytes), off, 0, 0)
                   : (uint32_t)ld16_sc1(p, bytes, off);
  };
  // q of the task's heads (a wavefront per head: element e of head g at lane e % 64, slot
  // e / 64) and, on wavefront 0, the new key and value: as bf16 values, or as the fp32
  // planes of a q/k/v launch that left its K-ranges to the reader (added below in plane
  // order from zero and rounded to bf16).  Loads a wavefront does not need read past their
  // buffer (zeros, no traffic), so every wavefront issues the same loads.
  constexpr bool use_planes = kStaged && kPlanes;
  const int np = S.qkv_splits, prow = S.qkv_rows;
  const int nq = Hq * kD, nkv = Hkv * kD;
  const __amdgpu_buffer_rsrc_t qkv_rs = buffer_rsrc(S.qkv, use_planes ? (uint32_t)(3 * S.qkv_pstride * 4) : 0u);
  // (bit 31 of an offset puts it past every buffer here, every buffer being under 2 GiB.  The
  // flag is made opaque to the optimizer, which would otherwise branch on it, and a load into
  // a register another path also loads then waits for every load before it.)
  auto plane_loads = [&](int pi, int nw, int elem, bool need, float (&v)[kMaxQkvPlanes]) {
    uint32_t skip = need ? 0u : kPastBuffer;
    asm("" : "+s"(skip));
#pragma unroll
    for (int sp = 0; sp < kMaxQkvPlanes; ++sp) {
      const uint32_t off = (uint32_t)(pi * S.qkv_pstride + (int64_t)(sp * prow + b) * nw + elem) * 4u;
      v[sp] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(qkv_rs, off | (sp < np ? skip : kPastBuffer), 0, 0));
    }
  };
  auto plane_sum = [&](const float (&v)[kMaxQkvPlanes]) -> uint32_t {
    float t = 0.0f;
#pragma unroll
    for (int sp = 0; sp < kMaxQkvPlanes; ++sp)
      if (sp < np) t += v[sp];
    return to_bf(t);
  };
  uint32_t qx[kRounds][2], kx[2] = {0u, 0u}, vx[2] = {0u, 0u};
  float pq[kRounds][2][kMaxQkvPlanes], pk[2][kMaxQkvPlanes], pv[2][kMaxQkvPlanes];
  auto fetch_qkv = [&]() __attribute__((always_inline)) {
    if (use_planes) {
#pragma unroll
      for (int r = 0; r < kRounds; ++r) {
        const int g = wave + W * r;
        const int e0 = (kvh * G + (g < G ? g : 0)) * kD;
        plane_loads(0, nq, e0 + lane, g < G, pq[r][0]);
        plane_loads(0, nq, e0 + lane + 64, g < G, pq[r][1]);
      }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        plane_loads(1, nkv, kvh * kD + lane + 64 * h, wave == 0, pk[h]);
        plane_loads(2, nkv, kvh * kD + lane + 64 * h, wave == 0, pv[h]);
      }
    } else {
#pragma unroll
      for (int r = 0; r < kRounds; ++r) {
        const int g = wave + W * r;
        uint32_t skip = g < G ? 0u : kPastBuffer;
        asm("" : "+s"(skip));
        const uint32_t off = (uint32_t)((b * Hq + kvh * G + (g < G ? g : 0)) * kD) * 2u;
        qx[r][0] = ld16(S.q, qbytes, (off + 2u * lane) | skip);
        qx[r][1] = ld16(S.q, qbytes, (off + 2u * (lane + 64)) | skip);
      }
      uint32_t skip = wave == 0 ? 0u : kPastBuffer;
      asm("" : "+s"(skip));
      kx[0] = ld16(S.k, kvbytes, (kvoff + 2u * lane) | skip);
      kx[1] = ld16(S.k, kvbytes, (kvoff + 2u * (lane + 64)) | skip);
      vx[0] = ld16(S.v, kvbytes, (kvoff + 2u * lane) | skip);
      vx[1] = ld16(S.v, kvbytes, (kvoff + 2u * (lane + 64)) | skip);
    }
  };
  if (kStaged) fetch_qkv();
  const float qn0 = bf(S.q_norm[lane]), qn1 = bf(S.q_norm[lane + 64]);
  const float kn0 = bf(S.k_norm[lane]), kn1 = bf(S.k_norm[lane + 64]);
  const int pos = uni(pos_in), slot = uni(slot_in);
  const bool slot_ok = slot >= 0 && slot < S.num_slots;
  const bool write_ok = slot_ok && pos >= 0 && pos < S.capacity;
  int len = pos + 1;
  len = len < S.max_len ? len : S.max_len;
  len = len < S.capacity ? len : S.capacity;
  if (!write_ok || len < 0) len = 0;
  const int span = S.cps * kChunk;
  const int first = s * span;
  const int last = min(len, first + span);
  const int used = (len + span - 1) / span;
  const int newrow = write_ok && pos < len ? pos : -1;
  const int writer = write_ok ? min(pos / span, splits - 1) : -1;
  const size_t base = (((size_t)(slot_ok ? slot : 0) * Hkv + kvh) * S.capacity) * kD;

  // This wavefront's keys: units of 16, units wave, wave + W, ... of the split's keys
  // [first, last).  K ends up in the A-operand layout of v_mfma_f32_16x16x32_bf16 (lane
  // (key h16 = lane % 16, quarter q4 = lane / 16): dimensions 32 j + 8 q4 .. + 8 of k-step
  // j), V in the wavefront's transposed LDS tile, read as 16-byte pieces of whole 256-byte
  // rows (lane (key quad vq = lane % 4, dimension group vg = lane / 4); load kk takes keys
  // 4 vq + kk).  The wide launch reads K the same way and re-lays it through the
  // wavefront's swizzled LDS tile: loading it straight in the operand layout reads half a
  // cache line per row and load, which measured slower when the CU's load path is full
  // (batch 32), while the tile's LDS round trip measured slower at batch 1.  Both are
  // streamed with the non-temporal policy: every key is read once per launch.  Rows at or
  // past `last` read row last - 1 (their scores are masked), a unit at or past `last`
  // reads past the buffer (zeros, no traffic).
  constexpr bool kRowK = W > kAttnWaves;
  const uint32_t pool_bytes = (uint32_t)(((size_t)(slot_ok ? slot : 0) * Hkv + kvh + 1) * S.capacity * kD * 2);
  const __amdgpu_buffer_rsrc_t krs = buffer_rsrc(S.k_pool, pool_bytes);
  const __amdgpu_buffer_rsrc_t vrs = buffer_rsrc(S.v_pool, pool_bytes);
  const int h16 = lane & 15, q4 = lane >> 4;  // MFMA coordinates: row / column, k quarter
  const int vq = lane & 3, vg = lane >> 2;    // K and V pieces: key quad, dimension group
  auto row_bytes = [&](int key) __attribute__((always_inline)) -> uint32_t {
    return (uint32_t)((base + (size_t)(key < last ? key : last - 1) * kD) * 2);
  };
  uint4 kr[4], vr[4];  // K [key of the quad] (kRowK) or [k-step]; V [key of the quad]
  auto load_k = [&](int start) __attribute__((always_inline)) {
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
      kr[kk] = load_b128_nt(krs, start >= last ? kPastBuffer
                                 : kRowK ? row_bytes(start + 4 * vq + kk) + 16u * vg
                                         : row_bytes(start + h16) + 64u * kk + 16u * q4);
  };
  auto load_v = [&](int start) __attribute__((always_inline)) {
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
      vr[kk] = load_b128_nt(vrs, start < last ? row_bytes(start + 4 * vq + kk) + 16u * vg : kPastBuffer);
  };
  const int start0 = first + kUnit * wave;

  // The persistent form puts the chunk in flight, waits for its input stage and reads q,
  // k and v through sc1; the staged form has them in flight already.
  if (!kStaged) {
    load_k(start0);
    load_v(start0);
    if (!wait_stage(a, S.wait, (uint32_t)S.wait_count)) return false;
    fetch_qkv();
  } else {
    load_k(start0);
    load_v(start0);
    // q, k and v are first used here, behind the K/V loads: an empty asm that reads and
    // writes each value (ordered after the loads by its memory clobber) keeps the compiler
    // from adding the planes, and so waiting for them, before those loads are issued
#pragma unroll
    for (int r = 0; r < kRounds; ++r)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        asm volatile("" : "+v"(qx[r][h]) :: "memory");
#pragma unroll
        for (int sp = 0; sp < kMaxQkvPlanes; ++sp) asm volatile("" : "+v"(pq[r][h][sp]) :: "memory");
      }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      asm volatile("" : "+v"(kx[h]), "+v"(vx[h]) :: "memory");
#pragma unroll
      for (int sp = 0; sp < kMaxQkvPlanes; ++sp) asm volatile("" : "+v"(pk[h][sp]), "+v"(pv[h][sp]) :: "memory");
    }
  }
  if (use_planes) {
#pragma unroll
    for (int r = 0; r < kRounds; ++r) {
      qx[r][0] = plane_sum(pq[r][0]);
      qx[r][1] = plane_sum(pq[r][1]);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      kx[h] = plane_sum(pk[h]);
      vx[h] = plane_sum(pv[h]);
    }
  }
  const float inv_freq = exp2f(-(float)lane * (S.log2_theta / 64.0f));
  float sn, cs;
  sincosf((float)pos * inv_freq, &sn, &cs);
  auto rotate = [&](uint32_t h0, uint32_t h1, float nw0, float nw1, uint16_t* dst) {
    float x0 = bf(h0), x1 = bf(h1);
    const float ss = wave_sum(fmaf(x0, x0, x1 * x1));
    const float inv = 1.0f / sqrtf(ss / (float)kD + eps);
    x0 = bf(to_bf(x0 * inv * nw0));
    x1 = bf(to_bf(x1 * inv * nw1));
    const float r0 = x0 * cs - x1 * sn;
    const float r1 = x0 * sn + x1 * cs;
    dst[lane] = to_bf(r0);
    dst[lane + 64] = to_bf(r1);
  };
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    const int g = wave + W * r;
    if (g < G) rotate(qx[r][0], qx[r][1], qn0, qn1, reinterpret_cast<uint16_t*>(L.qs[g]));
  }
  if (wave == 0) {
    uint16_t* kn = reinterpret_cast<uint16_t*>(L.knew);
    uint16_t* vn = reinterpret_cast<uint16_t*>(L.vnew);
    rotate(kx[0], kx[1], kn0, kn1, kn);
    vn[lane] = (uint16_t)vx[0];
    vn[lane + 64] = (uint16_t)vx[1];
    if (s == writer) {  // this step's key and value into the pools (read by later launches)
      uint16_t* kd = S.k_pool + base + (size_t)pos * kD;
      uint16_t* vd = S.v_pool + base + (size_t)pos * kD;
      kd[lane] = kn[lane];
      kd[lane + 64] = kn[lane + 64];
      vd[lane] = vn[lane];
      vd[lane + 64] = vn[lane + 64];
    }
  }
  __syncthreads();

  uint16_t* out = S.attn_out;
  const uint32_t out_bytes = S.out_tiled ? 64u * (uint32_t)Hq * kD : (uint32_t)(b + 1) * Hq * kD * 2u;
  // byte offset of the output pair (request b, head hd, dimensions 2 lane, 2 lane + 1)
  auto out_at = [&](int hd) {
    return S.out_tiled ? tile_elem((uint32_t)b, (uint32_t)(hd * kD + 2 * lane)) * 2u
                       : (uint32_t)((b * Hq + hd) * kD + 2 * lane) * 2u;
  };
  if (first >= last) {
    if (used == 0 && s == 0) {  // nothing to attend to: zeros
#pragma unroll
      for (int r = 0; r < kRounds; ++r) {
        const int g = wave + W * r;
        if (g < G)
          store_b32_sc1(buffer_rsrc(out, out_bytes), out_at(kvh * G + g), 0u);
      }
    }
    return true;
  }

  float M[kRounds], Ls[kRounds], a0[kRounds], a1[kRounds];
#pragma unroll
  for (int r = 0; r < kRounds; ++r) M[r] = -INFINITY, Ls[r] = a0[r] = a1[r] = 0.0f;
  {
    // q^T as the B operand: lane (head h16, quarter q4) holds dimensions 32 j + 8 q4 .. + 8
    // of head h16 for k-step j (zeros for the columns past the task's G heads)
    bf16x8_t qb[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      qb[j] = __builtin_bit_cast(bf16x8_t, h16 < G ? reinterpret_cast<const uint4*>(L.qs[h16])[4 * j + q4]
                                                   : make_uint4(0u, 0u, 0u, 0u));
    const uint4* kn4 = reinterpret_cast<const uint4*>(L.knew);
    const uint4* vn4 = reinterpret_cast<const uint4*>(L.vnew);
    uint32_t(*vt)[kVtStride] = L.u.tile.vt[wave];
    uint4* ks = L.u.tile.ks[kRowK ? wave : 0];
    // lane (h16, q4) carries head h16's running max and sum (the same in its four quarters)
    // and acc[dblk][i] = its weighted sum for dimension 16 dblk + 4 q4 + i
    float Mw = -INFINITY, Lw = 0.0f;
    f32x4_t acc[8];
#pragma unroll
    for (int d = 0; d < 8; ++d) acc[d] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    for (int start = start0; start < last; start += W * kUnit) {
      const int next = start + W * kUnit;
      // the unit that holds the new key: its row takes the rotated key (and below, the
      // value) from LDS
      const bool has_new = newrow >= start && newrow < start + kUnit;  // uniform
      // K (through the tile: key r = 4 vq + kk, piece vg in; key h16, piece 4 j + q4 out;
      // the 16 lanes of each quarter wavefront touch 16 distinct 16-byte bank groups)
      uint4 ka[4];
      if constexpr (kRowK) {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const int r = 4 * vq + kk;
          ks[r * 16 + (vg ^ r)] = kr[kk];
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) ka[j] = ks[h16 * 16 + ((4 * j + q4) ^ h16)];
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) ka[j] = kr[j];
      }
      if (has_new) {
#pragma unroll
        for (int j = 0; j < 4; ++j) ka[j] = select4(start + h16 == newrow ? ~0u : 0u, kn4[4 * j + q4], ka[j]);
      }
      // scores: S^T (16 keys x heads) = K (keys x 128) q^T
      f32x4_t sc = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int j = 0; j < 4; ++j)
        sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, ka[j]), qb[j], sc, 0, 0, 0);
      load_k(next);
      // online softmax: lane (h16, q4) holds head h16's scores of keys start + 4 q4 + i
      float mloc = -INFINITY;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float v = start + 4 * q4 + i < last ? sc[i] * S.scale : -INFINITY;
        sc[i] = v;
        mloc = fmaxf(mloc, v);
      }
      mloc = max_xor32(max_xor16(mloc));
      const float mnew = fmaxf(Mw, mloc);
      const float alpha = expf(Mw - mnew);
      float lsum = 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = expf(sc[i] - mnew);
        sc[i] = p;
        lsum += p;
      }
      lsum = add_xor32(add_xor16(lsum));
      Lw = fmaf(Lw, alpha, lsum);
      Mw = mnew;
#pragma unroll
      for (int d = 0; d < 8; ++d) acc[d] *= alpha;
      // P^T as the B operand of v_mfma_f32_16x16x16_bf16 (lane (h16, q4): keys 4 q4 .. + 3,
      // the scores' own layout), split into bf16 high and low parts (p = hi + lo to about
      // 2^-16)
      uint32_t hi[2], lo[2];
#pragma unroll
      for (int w = 0; w < 2; ++w) {
        const uint32_t h0 = to_bf(sc[2 * w]), h1 = to_bf(sc[2 * w + 1]);
        hi[w] = h0 | (h1 << 16);
        lo[w] = (uint32_t)to_bf(sc[2 * w] - bf(h0)) | ((uint32_t)to_bf(sc[2 * w + 1] - bf(h1)) << 16);
      }
      const s16x4_t phi = __builtin_bit_cast(s16x4_t, make_uint2(hi[0], hi[1]));
      const s16x4_t plo = __builtin_bit_cast(s16x4_t, make_uint2(lo[0], lo[1]));
      // V^T of the unit's keys into this wavefront's tile: for each of the 8 dimensions of
      // the lane's group, the values of its quad's four keys as two dwords
      {
        uint4 r[4];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) r[kk] = vr[kk];
        if (has_new) {
#pragma unroll
          for (int kk = 0; kk < 4; ++kk) r[kk] = select4(start + 4 * vq + kk == newrow ? ~0u : 0u, vn4[vg], r[kk]);
        }
        const uint32_t w0[4] = {r[0].x, r[0].y, r[0].z, r[0].w}, w1[4] = {r[1].x, r[1].y, r[1].z, r[1].w};
        const uint32_t w2[4] = {r[2].x, r[2].y, r[2].z, r[2].w}, w3[4] = {r[3].x, r[3].y, r[3].z, r[3].w};
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          *reinterpret_cast<uint2*>(&vt[8 * vg + 2 * w][2 * vq]) =
              make_uint2((w0[w] & 0xffffu) | (w1[w] << 16), (w2[w] & 0xffffu) | (w3[w] << 16));
          *reinterpret_cast<uint2*>(&vt[8 * vg + 2 * w + 1][2 * vq]) =
              make_uint2((w0[w] >> 16) | (w1[w] & 0xffff0000u), (w2[w] >> 16) | (w3[w] & 0xffff0000u));
        }
      }
      load_v(next);
      // O^T (dims x heads) += V^T (dims x keys) P^T: lane (h16, q4) reads dimension
      // 16 dblk + h16's keys 4 q4 .. + 3
#pragma unroll
      for (int d = 0; d < 8; ++d) {
        const s16x4_t av = __builtin_bit_cast(s16x4_t, *reinterpret_cast<const uint2*>(&vt[16 * d + h16][2 * q4]));
        acc[d] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(av, phi, acc[d], 0, 0, 0);
        acc[d] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(av, plo, acc[d], 0, 0, 0);
      }
    }
    // the wavefronts' partials through LDS (the V^T tiles are done with), merged in
    // wavefront order by the wavefront of each head
    __syncthreads();
    if (h16 < G) {
#pragma unroll
      for (int d = 0; d < 8; ++d)
        *reinterpret_cast<f32x4_t*>(&L.u.merge.acc[wave][h16][16 * d + 4 * q4]) = acc[d];
      if (q4 == 0) {
        L.u.merge.ml[wave][h16][0] = Mw;
        L.u.merge.ml[wave][h16][1] = Lw;
      }
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kRounds; ++r) {
      const int g = wave + W * r;
      if (g < G) {
        float mx = -INFINITY;
#pragma unroll
        for (int w = 0; w < W; ++w) mx = fmaxf(mx, L.u.merge.ml[w][g][0]);
        float ls = 0.0f, c0 = 0.0f, c1 = 0.0f;
#pragma unroll
        for (int w = 0; w < W; ++w) {
          const float e = expf(L.u.merge.ml[w][g][0] - mx);  // a wavefront without keys: 0
          ls = fmaf(L.u.merge.ml[w][g][1], e, ls);
          const float2 x = *reinterpret_cast<const float2*>(&L.u.merge.acc[w][g][2 * lane]);
          c0 = fmaf(x.x, e, c0);
          c1 = fmaf(x.y, e, c1);
        }
        M[r] = mx;
        Ls[r] = ls;
        a0[r] = c0;
        a1[r] = c1;
      }
    }
  }

  if (used == 1) {
    // the only split with keys: the merge of one partial is c / L with c = fma(a, 1, 0),
    // L = fma(l, 1, 0) (exp(0) = 1), so it is written here with the same bits and no
    // partial round trip
#pragma unroll
    for (int r = 0; r < kRounds; ++r) {
      const int g = wave + W * r;
      if (g < G) {
        const float lx = Ls[r] + 0.0f;
        const uint32_t o = (uint32_t)to_bf((a0[r] + 0.0f) / lx) | ((uint32_t)to_bf((a1[r] + 0.0f) / lx) << 16);
        store_b32_sc1(buffer_rsrc(out, out_bytes), out_at(kvh * G + g), o);
      }
    }
    return true;
  }
  // this split's partial, then the last split of (b, kvh) merges them in split order
  const uint32_t part_bytes = (uint32_t)((b + 1) * Hq * splits) * kD * 4u;
  const uint32_t ml_bytes = (uint32_t)((b + 1) * Hq * splits) * 8u;
  const __amdgpu_buffer_rsrc_t prs = buffer_rsrc(S.part, part_bytes);
  const __amdgpu_buffer_rsrc_t mrs = buffer_rsrc(S.ml, ml_bytes);
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    const int g = wave + W * r;
    if (g < G) {
      const uint32_t po = (uint32_t)((b * Hq + kvh * G + g) * splits + s);
      store_b32_sc1(prs, (po * kD + 2 * lane) * 4u, __float_as_uint(a0[r]));
      store_b32_sc1(prs, (po * kD + 2 * lane + 1) * 4u, __float_as_uint(a1[r]));
      if (lane == 0) {
        store_b32_sc1(mrs, po * 8u, __float_as_uint(M[r]));
        store_b32_sc1(mrs, po * 8u + 4u, __float_as_uint(Ls[r]));
      }
    }
  }
  wait_vmem();
  __syncthreads();
  if (tid == 0)
    L.last = __hip_atomic_fetch_add(S.combine + b * Hkv + kvh, 1u, __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)(used - 1);
  __syncthreads();
  if (!L.last) return true;
  // every split has arrived: the counter is ready for the next launch
  if (tid == 0) st_sc1(S.combine + b * Hkv + kvh, 0u);
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    const int g = wave + W * r;
    if (g < G) {
      const int hh = kvh * G + g;
      const uint32_t p0 = (uint32_t)((b * Hq + hh) * splits);
      // the partials of kMergeBatch splits are loaded together before any is used (all of
      // them in one round when they fit); the arithmetic runs in split order
      // (attention_combine_kernel's)
      if (used <= kMergeBatch) {
        float mq[kMergeBatch], lq[kMergeBatch], xq[kMergeBatch], yq[kMergeBatch];
#pragma unroll
        for (int q = 0; q < kMergeBatch; ++q) {
          const bool in = q < used;
          const uint32_t po = p0 + q;
          mq[q] = __uint_as_float(load_b32_sc1(mrs, in ? po * 8u : kPastBuffer));
          lq[q] = __uint_as_float(load_b32_sc1(mrs, in ? po * 8u + 4u : kPastBuffer));
          xq[q] = __uint_as_float(load_b32_sc1(prs, in ? (po * kD + 2 * lane) * 4u : kPastBuffer));
          yq[q] = __uint_as_float(load_b32_sc1(prs, in ? (po * kD + 2 * lane + 1) * 4u : kPastBuffer));
        }
        float Mx = -INFINITY;
#pragma unroll
        for (int q = 0; q < kMergeBatch; ++q)
          if (q < used) Mx = fmaxf(Mx, mq[q]);
        float Lx = 0.0f, c0 = 0.0f, c1 = 0.0f;
#pragma unroll
        for (int q = 0; q < kMergeBatch; ++q) {
          if (q < used) {
            const float e = expf(mq[q] - Mx);
            Lx = fmaf(lq[q], e, Lx);
            c0 = fmaf(xq[q], e, c0);
            c1 = fmaf(yq[q], e, c1);
          }
        }
        const uint32_t o = (uint32_t)to_bf(c0 / Lx) | ((uint32_t)to_bf(c1 / Lx) << 16);
        store_b32_sc1(buffer_rsrc(out, out_bytes), out_at(hh), o);
        continue;
      }
      float Mx = -INFINITY;
      for (int s0 = 0; s0 < used; s0 += kMergeBatch) {
        float mv[kMergeBatch];
#pragma unroll
        for (int q = 0; q < kMergeBatch; ++q)
          mv[q] = __uint_as_float(load_b32_sc1(mrs, s0 + q < used ? (p0 + s0 + q) * 8u : kPastBuffer));
#pragma unroll
        for (int q = 0; q < kMergeBatch; ++q)
          if (s0 + q < used) Mx = fmaxf(Mx, mv[q]);
      }
      float Lx = 0.0f, c0 = 0.0f, c1 = 0.0f;
      for (int s0 = 0; s0 < used; s0 += kMergeBatch) {
        float mq[kMergeBatch], lq[kMergeBatch], xq[kMergeBatch], yq[kMergeBatch];
#pragma unroll
        for (int q = 0; q < kMergeBatch; ++q) {
          const bool in = s0 + q < used;
          const uint32_t po = p0 + s0 + q;
          mq[q] = __uint_as_float(load_b32_sc1(mrs, in ? po * 8u : kPastBuffer));
          lq[q] = __uint_as_float(load_b32_sc1(mrs, in ? po * 8u + 4u : kPastBuffer));
          xq[q] = __uint_as_float(load_b32_sc1(prs, in ? (po * kD + 2 * lane) * 4u : kPastBuffer));
          yq[q] = __uint_as_float(load_b32_sc1(prs, in ? (po * kD + 2 * lane + 1) * 4u : kPastBuffer));
        }
#pragma unroll
        for (int q = 0; q < kMergeBatch; ++q) {
          if (s0 + q < used) {
            const float e = expf(mq[q] - Mx);
            Lx = fmaf(lq[q], e, Lx);
            c0 = fmaf(xq[q], e, c0);
            c1 = fmaf(yq[q], e, c1);
          }
        }
      }
      const uint32_t o = (uint32_t)to_bf(c0 / Lx) | ((uint32_t)to_bf(c1 / Lx) << 16);
      store_b32_sc1(buffer_rsrc(out, out_bytes), out_at(hh), o);
    }
  }
  return true;
}

// ------------------------------------------------------------------ the kernels

// One qmv instantiation per (x source, epilogue, tile shape) that a program can hold.
#define IMQ_QMV_CASE(NCH, XR, XSRC, EPI, SHAPE)                   \
  case (XSRC) * 32 + (EPI) * 4 + (SHAPE):                          \
    good = qmv_task<NCH, XR, XSRC, EPI, false, StageRef>(S, task, a, smem); \
    break;
#define IMQ_QMV_SHAPES_X2(XSRC, EPI)         \
  IMQ_QMV_CASE(2, 2, XSRC, EPI, kShape22)    \
  IMQ_QMV_CASE(5, 2, XSRC, EPI, kShape52)    \
  IMQ_QMV_CASE(8, 2, XSRC, EPI, kShape82)

__device__ __forceinline__ bool run_task(StageRef S, int task, const StepArgs& a, uint4* smem) {
  bool good = false;
  if (S.kind == kKindAttention) {
    good = attention_task<false, StageRef>(S, task, a, smem);
  } else {
    switch (S.xsrc * 32 + S.epi * 4 + S.shape) {
      IMQ_QMV_SHAPES_X2(kXVector, kEpiBf16)
      IMQ_QMV_CASE(5, 5, kXVector, kEpiBf16, kShape55)
      IMQ_QMV_SHAPES_X2(kXVector, kEpiResidual)
      IMQ_QMV_CASE(5, 5, kXVector, kEpiResidual, kShape55)
      IMQ_QMV_SHAPES_X2(kXVector, kEpiResidualNorm)
      IMQ_QMV_CASE(5, 5, kXVector, kEpiResidualNorm, kShape55)
      IMQ_QMV_SHAPES_X2(kXNorm, kEpiBf16)
      IMQ_QMV_SHAPES_X2(kXNorm, kEpiSiluPair)
      IMQ_QMV_SHAPES_X2(kXNorm, kEpiF32)
      IMQ_QMV_SHAPES_X2(kXScaled, kEpiBf16)
      IMQ_QMV_SHAPES_X2(kXScaled, kEpiSiluPair)
      IMQ_QMV_SHAPES_X2(kXScaled, kEpiF32)
      default: break;  // the host plans only the cases above
    }
  }
  return good;
}

// The persistent form: every stage in one launch.
__global__ __launch_bounds__(kThreads) void step_kernel(const Stage* __restrict__ stages,
                                                        StepArgs a) {
  extern __shared__ uint4 smem[];
  int si = 0;
  for (int t = blockIdx.x; t < a.ntasks; t += gridDim.x) {
    while (t >= stages[si].first + stages[si].count) ++si;
    StageRef S = global_stage(stages + si);
    const int task = t - S.first;
    if (!run_task(S, task, a, smem)) return;
    signal(counter(a, si, task % kSub));
  }
}

// The staged form: one launch per stage, one task per workgroup, the launches' stream
// order standing in for the waits.  Each stage gets the kernel of its own task variant, so
// it carries only that variant's registers.
// The stage descriptor is a kernel argument here, so its fields arrive with the
// argument block instead of a second dependent load.
template <int NCH, int XR, int XSRC, int EPI>
__global__ __launch_bounds__(kThreads) void qmv_stage_kernel(const Stage S, StepArgs a) {
  extern __shared__ uint4 smem[];
  qmv_task<NCH, XR, XSRC, EPI, true, const Stage&>(S, blockIdx.x, a, smem);
}

template <int W, bool kPlanes>
__global__ __launch_bounds__(64 * W) void attention_stage_kernel(const Stage S, StepArgs a) {
  extern __shared__ uint4 smem[];
  attention_task<true, const Stage&, W, kPlanes>(S, blockIdx.x, a, smem);
}

#undef IMQ_QMV_SHAPES_X2
#undef IMQ_QMV_CASE

__global__ __launch_bounds__(kThreads) void reset_kernel(uint32_t* words, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i < n) words[i] = 0u;
}

// ------------------------------------------------------------------ host side

size_t lds_bytes_for(int shape) {
  switch (shape) {
    case kShape22: return QLds<2, 2>::kBytes;
    case kShape52: return QLds<5, 2>::kBytes;
    case kShape82: return QLds<8, 2>::kBytes;
    default: return QLds<5, 5>::kBytes;
  }
}

// The one-row tile's lane shape of qmv.hip's plan_m1 (16, 32 or 64 lanes per row, at
// most 8 chunks per lane), and the instantiation that covers it.  -1: not served.
struct TileShape {
  int sh, nch, xr, shape;
};

TileShape tile_shape(int K) {
  TileShape t{-1, 0, 0, -1};
  const int C = K / 32;
  const int sh = m1_lane_shift(K);
  if (sh < 0) return t;
  t.sh = sh;
  t.nch = (C + (1 << sh) - 1) >> sh;
  t.xr = (K / 8 + kThreads - 1) / kThreads;
  if (t.nch <= 2 && t.xr <= 2) t.shape = kShape22;
  else if (t.nch <= 5 && t.xr <= 2) t.shape = kShape52;
  else if (t.nch <= 8 && t.xr <= 2) t.shape = kShape82;
  else if (t.nch <= 5 && t.xr <= 5) t.shape = kShape55;
  return t;
}

int32_t check_qweight(const imq_qweight& q, int64_t N, int64_t K, const char* what) {
  if (!q.w || !q.scales || !q.biases) return fail(IMQ_EINVAL, std::string(what) + ": null weight pointer");
  if (!aligned(q.w, 16) || !aligned(q.scales, 4) || !aligned(q.biases, 4))
    return fail(IMQ_EINVAL, std::string(what) + ": w must be 16-byte and scales/biases 4-byte aligned");
  if (N < 1 || K < 64 || K % 64) return fail(IMQ_EINVAL, std::string(what) + ": bad shape");
  if (N * (K / 2) >= ((int64_t)1 << 31))
    return fail(IMQ_EUNSUPPORTED, std::string(what) + ": weights of 2 GiB or more");
  return IMQ_OK;
}

}  // namespace

struct imq_program {
  int device = -1;
  std::vector<size_t> stage_lds;  // LDS bytes of each stage's staged launch
  std::vector<Stage> stages;
  Stage* d_stages = nullptr;
  uint32_t* d_words = nullptr;  // completion counters, then combine counters, then status
  int64_t reset_words = 0;      // words zeroed before each run (all but the status word)
  uint32_t* d_status = nullptr;
  void* d_scratch = nullptr;    // activations and attention partials
  int ntasks = 0;
  int sub_stride = 0;
  int grid = 0;
  size_t lds = 0;
};

namespace {

void free_program(imq_program* p) {
  if (!p) return;
  if (p->d_stages) (void)hipFree(p->d_stages);
  if (p->d_words) (void)hipFree(p->d_words);
  if (p->d_scratch) (void)hipFree(p->d_scratch);
  delete p;
}

// Adds a qmv stage of one-row tiles over `probs` (same K); pair: a gate/up pair.
int32_t add_qmv_stage(imq_program* prog, const std::vector<QProb>& probs, int xsrc, int epi,
                      int wait, const uint16_t* x, float* h,
                      const uint16_t* norm_w, float eps, uint16_t* act) {
  Stage S;
  memset(&S, 0, sizeof(S));
  S.kind = kKindQmv;
  S.wait = wait;
  S.xsrc = xsrc;
  S.epi = epi;
  S.nprob = (int)probs.size();
  S.eps = eps;
  S.x = x;
  S.h = h;
  S.norm_w = norm_w;
  S.act = act;
  const TileShape ts = tile_shape(probs[0].K);
  if (ts.shape < 0) return fail(IMQ_EUNSUPPORTED, "K outside the persistent qmv tiles (K <= 16384 with 2/5/8 chunks per lane)");
  if (xsrc == kXNorm && (ts.xr > 2 || probs[0].K > kMaxHidden))
    return fail(IMQ_EUNSUPPORTED, "a fused RMSNorm row is limited to 4096 values");
  if (epi == kEpiSiluPair && ts.sh != 4)
    return fail(IMQ_EUNSUPPORTED, "the gate/up pair tile needs 16 lanes per row (K <= 4096)");
  S.shape = ts.shape;
  int tiles = 0;
  for (size_t i = 0; i < probs.size(); ++i) {
    QProb q = probs[i];
    if (q.K != probs[0].K) return fail(IMQ_EINVAL, "every problem of a stage has the same K");
    q.sh = ts.sh;
    q.nch = ts.nch;
    const int rows = epi == kEpiSiluPair ? 8 : (kThreads >> ts.sh);
    const int t = (q.N + rows - 1) / rows;
    tiles = epi == kEpiSiluPair ? t : tiles + t;
    q.tile_end = tiles;
    S.p[i] = q;
  }
  S.count = tiles;
  S.first = prog->ntasks;
  if (wait >= 0) S.wait_count = prog->stages[wait].count;
  prog->ntasks += S.count;
  prog->stages.push_back(S);
  return IMQ_OK;
}

// Device tables, counters and the launch geometry of a planned program.
int32_t finish_program(imq_program* prog) {
  const int nstages = (int)prog->stages.size();
  if (nstages == 0 || prog->ntasks == 0) return fail(IMQ_EINVAL, "empty program");
  size_t lds = 0;
  prog->stage_lds.clear();
  for (const Stage& S : prog->stages) {
    const size_t b = S.kind == kKindQmv
                         ? std::max(lds_bytes_for(S.shape), S.xsrc == kXNorm ? kNormBytes : 0)
                         : sizeof(AttnLds);
    prog->stage_lds.push_back((b + 15) & ~(size_t)15);
    lds = std::max(lds, b);
  }
  prog->lds = (lds + 15) & ~(size_t)15;

  // counters: kSub lines per stage; the same sub-counter of consecutive stages are
  // neighbours, and consecutive sub-counters of one stage >= 4 KiB apart
  prog->sub_stride = std::max(nstages, 32);
  const int64_t counter_words = (int64_t)kSub * prog->sub_stride * kLineWords;
  int64_t combine_total = 0;
  for (Stage& S : prog->stages)
    if (S.kind == kKindAttention) combine_total += (int64_t)S.count / S.splits;
  prog->reset_words = counter_words + combine_total;
  const int64_t words = prog->reset_words + 1;
  if (hipMalloc(&prog->d_words, (size_t)words * 4) != hipSuccess)
    return fail(IMQ_ELAUNCH, "hipMalloc of the program counters failed");
  if (hipMemset(prog->d_words, 0, (size_t)words * 4) != hipSuccess)
    return fail(IMQ_ELAUNCH, "hipMemset of the program counters failed");
  prog->d_status = prog->d_words + prog->reset_words;
  int64_t cw = counter_words;
  for (Stage& S : prog->stages)
    if (S.kind == kKindAttention) {
      S.combine = prog->d_words + cw;
      cw += S.count / S.splits;
    }
  if (hipMalloc(&prog->d_stages, sizeof(Stage) * nstages) != hipSuccess)
    return fail(IMQ_ELAUNCH, "hipMalloc of the stage table failed");
  if (hipMemcpy(prog->d_stages, prog->stages.data(), sizeof(Stage) * nstages,
                hipMemcpyHostToDevice) != hipSuccess)
    return fail(IMQ_ELAUNCH, "copying the stage table failed");
  int32_t code;
  const DeviceInfo* dev = current_device(&code);
  if (!dev) return code;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(step_kernel),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)prog->lds) != hipSuccess)
    return fail(IMQ_ELAUNCH, "cannot give the persistent kernel its LDS");
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, step_kernel, kThreads, prog->lds) !=
          hipSuccess ||
      per_cu < 1)
    return fail(IMQ_ELAUNCH, "the persistent kernel does not fit on a CU");
  prog->grid = std::min(per_cu * dev->cu_count, prog->ntasks);
  return ok();
}

// Attention splits: the per-kernel path's plan (attention_splits, common.h): a split's
// chunks of 64 keys are shared by the workgroup's four wavefronts, 16 keys each.
void attention_split(int B, int Hkv, int span, int* splits, int* cps) {
  static_assert(kChunk == kAttnWaves * kUnit, "a chunk is one unit per wavefront");
  attention_splits(B, Hkv, span, splits, cps);
}

#ifndef IMQ_ATTN_WIDE_WAVES
#define IMQ_ATTN_WIDE_WAVES 12
#endif
// From 64 (request, KV head) pairs (8 requests over 8 KV heads): at 8 requests the fused
// launch took 12.0 us against 13.5 with 4 wavefronts per workgroup, at 4 requests 11.7
// against 10.6.
#ifndef IMQ_ATTN_WIDE_PAIRS
#define IMQ_ATTN_WIDE_PAIRS 64
#endif
#ifndef IMQ_ATTN_WIDE_WORKGROUPS
#define IMQ_ATTN_WIDE_WORKGROUPS 256
#endif
constexpr int kWideWaves = IMQ_ATTN_WIDE_WAVES;

// The wide plan, from IMQ_ATTN_WIDE_PAIRS (request, KV head) pairs: a workgroup of
// kWideWaves wavefronts takes a split of at least one unit per wavefront, and the splits
// target one workgroup per CU.  Never more splits than attention_split's plan, so its
// workspace size holds.
bool attention_wide_split(int B, int Hkv, int span, int* splits, int* cps) {
  const int pairs = B * Hkv;
  if (pairs < IMQ_ATTN_WIDE_PAIRS) return false;
  const int chunks = (span + kChunk - 1) / kChunk;
  const int min_c = (kWideWaves * kUnit + kChunk - 1) / kChunk;
  int sp = (IMQ_ATTN_WIDE_WORKGROUPS + pairs - 1) / pairs;
  sp = sp < chunks ? sp : chunks;
  sp = sp > 1 ? sp : 1;
  int c = (chunks + sp - 1) / sp;
  c = c > min_c ? c : min_c;
  c = c < chunks ? c : chunks;
  *cps = c;
  *splits = (chunks + c - 1) / c;
  int base_splits, base_cps;
  attention_split(B, Hkv, span, &base_splits, &base_cps);
  return *splits <= base_splits;
}

int32_t attention_fused(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* planes,
                        int64_t pstride, int32_t nplanes,
                            const uint16_t* q_norm, const uint16_t* k_norm,
                            const int32_t* positions, const int32_t* slots, uint16_t* k_pool,
                            uint16_t* v_pool, uint16_t* out, int32_t B, int32_t Hq, int32_t Hkv,
                            int32_t capacity, int32_t num_slots, int32_t max_len, float theta,
                            float eps, float* workspace, uint32_t* counters, void* stream,
                            bool out_tiled = false) {
  if ((planes ? false : (!q || !k || !v)) || !q_norm || !k_norm || !positions || !slots || !k_pool ||
      !v_pool || !out || !workspace || !counters)
    return fail(IMQ_EINVAL, "null pointer");
  if (planes && (nplanes < 1 || nplanes > kMaxQkvPlanes || !aligned(planes, 4) ||
                 pstride < (int64_t)nplanes * B * (Hq > Hkv ? Hq : Hkv) * kD ||
                 3 * pstride * 4 >= ((int64_t)1 << 31)))
    return fail(IMQ_EINVAL, "q/k/v planes: 1 to 4 planes, 4-byte aligned, pstride >= planes * B * Hq * 128, under 2 GiB");
  if (B < 1 || Hq < 1 || Hkv < 1 || Hq % Hkv || Hq / Hkv > 8)
    return fail(IMQ_EINVAL, "bad head counts (Hq a multiple of Hkv, at most 8 query heads per KV head)");
  if (capacity < 1 || num_slots < 1 || max_len < 1 || !(theta > 0.0f) || !(eps >= 0.0f))
    return fail(IMQ_EINVAL, "bad capacity, slot count, max_len, theta or eps");
  // the same layout requirements as imq_attention_decode, whose attention this computes
  if ((!planes && !aligned(q, 16)) || !aligned(k_pool, 16) || !aligned(v_pool, 16) || !aligned(workspace, 16))
    return fail(IMQ_EINVAL, "q, pools and workspace must be 16-byte aligned");
  if (!aligned(counters, 4)) return fail(IMQ_EINVAL, "counters must be 4-byte aligned");
  if (B > 65535 || Hkv > 65535 || Hq > 65535)
    return fail(IMQ_EINVAL, "B and the head counts must be <= 65535");
  if ((int64_t)num_slots * Hkv * capacity * kD * 2 >= ((int64_t)1 << 31))
    return fail(IMQ_EUNSUPPORTED, "a KV pool of 2 GiB or more exceeds the attention's offsets");
  int32_t code;
  if (!current_device(&code)) return code;
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= imq_rt::kMaxDevices)
    return fail(IMQ_EUNAVAILABLE, "no current HIP device");
  const int span = std::min(max_len, capacity);
  int splits, cps;
  const bool wide = attention_wide_split(B, Hkv, span, &splits, &cps);
  if (!wide) attention_split(B, Hkv, span, &splits, &cps);
  Stage A;
  memset(&A, 0, sizeof(A));
  A.kind = kKindAttention;
  A.wait = -1;
  A.count = B * Hkv * splits;
  A.eps = eps;
  A.log2_theta = log2f(theta);
  A.scale = 1.0f / sqrtf((float)kD);
  A.q = q;
  A.k = k;
  A.v = v;
  A.q_norm = q_norm;
  A.k_norm = k_norm;
  A.k_pool = k_pool;
  A.v_pool = v_pool;
  A.attn_out = out;
  A.out_tiled = out_tiled ? 1 : 0;
  A.positions = positions;
  A.slots = slots;
  A.part = workspace;
  A.ml = workspace + (size_t)B * Hq * splits * kD;
  A.combine = counters;
  A.Hq = Hq;
  A.Hkv = Hkv;
  A.capacity = capacity;
  A.num_slots = num_slots;
  A.max_len = span;
  A.splits = splits;
  A.cps = cps;
  A.qkv = planes;
  A.qkv_pstride = pstride;
  A.qkv_splits = planes ? nplanes : 0;
  A.qkv_rows = B;
  StepArgs a;
  memset(&a, 0, sizeof(a));
  a.ntasks = A.count;
  a.staged = 1;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (wide) {
    const size_t lds = (sizeof(AttnLdsT<kWideWaves>) + 15) & ~(size_t)15;
    // the launch's LDS is above the default dynamic limit: raised once per device, for both
    // forms of the kernel
    static std::atomic<bool> raised[imq_rt::kMaxDevices];
    if (!raised[device].load(std::memory_order_acquire)) {
      for (const void* fn : {reinterpret_cast<const void*>(attention_stage_kernel<kWideWaves, true>),
                             reinterpret_cast<const void*>(attention_stage_kernel<kWideWaves, false>)}) {
        const hipError_t attr = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (attr != hipSuccess)
          return fail(IMQ_ELAUNCH, std::string("fused attention LDS size: ") + hipGetErrorString(attr));
      }
      raised[device].store(true, std::memory_order_release);
    }
    if (planes)
      hipLaunchKernelGGL((attention_stage_kernel<kWideWaves, true>), dim3(A.count), dim3(64 * kWideWaves), lds, st, A, a);
    else
      hipLaunchKernelGGL((attention_stage_kernel<kWideWaves, false>), dim3(A.count), dim3(64 * kWideWaves), lds, st, A, a);
  } else {
    const size_t lds = (sizeof(AttnLds) + 15) & ~(size_t)15;
    if (planes)
      hipLaunchKernelGGL((attention_stage_kernel<kAttnWaves, true>), dim3(A.count), dim3(kThreads), lds, st, A, a);
    else
      hipLaunchKernelGGL((attention_stage_kernel<kAttnWaves, false>), dim3(A.count), dim3(kThreads), lds, st, A, a);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(IMQ_ELAUNCH, std::string("fused attention launch: ") + hipGetErrorString(e));
  return ok();
}

}  // namespace

extern "C" {

int32_t imq_attention_fused(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                            const uint16_t* q_norm, const uint16_t* k_norm,
                            const int32_t* positions, const int32_t* slots, uint16_t* k_pool,
                            uint16_t* v_pool, uint16_t* out, int32_t B, int32_t Hq, int32_t Hkv,
                            int32_t capacity, int32_t num_slots, int32_t max_len, float theta,
                            float eps, float* workspace, uint32_t* counters, void* stream) {
  return attention_fused(q, k, v, nullptr, 0, 0, q_norm, k_norm, positions, slots, k_pool, v_pool, out, B,
                         Hq, Hkv, capacity, num_slots, max_len, theta, eps, workspace, counters, stream);
}

int32_t imq_attention_fused_planes(const float* planes, int64_t pstride, int32_t nplanes,
                                   const uint16_t* q_norm, const uint16_t* k_norm,
                                   const int32_t* positions, const int32_t* slots, uint16_t* k_pool,
                                   uint16_t* v_pool, uint16_t* out, int64_t ld_out, int32_t B, int32_t Hq,
                                   int32_t Hkv, int32_t capacity, int32_t num_slots, int32_t max_len,
                                   float theta, float eps, float* workspace, uint32_t* counters, void* stream) {
  if (!planes) return fail(IMQ_EINVAL, "planes must be non-null");
  if (ld_out != IMQ_LD_TILED && ld_out != (int64_t)Hq * kD)
    return fail(IMQ_EINVAL, "ld_out must be Hq * 128 (rows) or IMQ_LD_TILED");
  if (ld_out == IMQ_LD_TILED && (B > 32 || !aligned(out, 4)))
    return fail(IMQ_EINVAL, "a tiled attention output takes at most 32 requests, 4-byte aligned");
  return attention_fused(nullptr, nullptr, nullptr, planes, pstride, nplanes, q_norm, k_norm, positions,
                         slots, k_pool, v_pool, out, B, Hq, Hkv, capacity, num_slots, max_len, theta, eps,
                         workspace, counters, stream, ld_out == IMQ_LD_TILED);
}

int32_t imq_qmv_program_create(const imq_qmv_stage* stages, int32_t count, imq_program** out) {
  if (!out) return fail(IMQ_EINVAL, "out must be non-null");
  *out = nullptr;
  if (!stages || count < 1) return fail(IMQ_EINVAL, "need at least one stage");
  int32_t code;
  if (!current_device(&code)) return code;
  imq_program* prog = new imq_program();
  (void)hipGetDevice(&prog->device);
  for (int i = 0; i < count; ++i) {
    const imq_qmv_stage& st = stages[i];
    if (st.count < 1 || st.count > kMaxStageProblems) {
      free_program(prog);
      return fail(IMQ_EINVAL, "a stage has 1 to 3 problems");
    }
    std::vector<QProb> probs;
    for (int k = 0; k < st.count; ++k) {
      const imq_problem& q = st.problems[k];
      const imq_qweight qw{q.w, q.scales, q.biases};
      code = check_qweight(qw, q.N, q.K, "qmv stage");
      if (code == IMQ_OK && (!q.x || !q.y || !aligned(q.x, 16) || !aligned(q.y, 2)))
        code = fail(IMQ_EINVAL, "x must be 16-byte aligned and y 2-byte aligned");
      if (code == IMQ_OK && q.x != st.problems[0].x)
        code = fail(IMQ_EINVAL, "the problems of a stage share one x");
      if (code != IMQ_OK) {
        free_program(prog);
        return code;
      }
      QProb p;
      memset(&p, 0, sizeof(p));
      p.w = q.w;
      p.s = q.scales;
      p.b = q.biases;
      p.y = q.y;
      p.N = q.N;
      p.K = q.K;
      probs.push_back(p);
    }
    const int wait = st.wait_previous && i > 0 ? i - 1 : -1;
    if ((code = add_qmv_stage(prog, probs, kXVector, kEpiBf16, wait, st.problems[0].x, nullptr,
                              nullptr, 0.0f, nullptr)) != IMQ_OK) {
      free_program(prog);
      return code;
    }
  }
  if ((code = finish_program(prog)) != IMQ_OK) {
    free_program(prog);
    return code;
  }
  *out = prog;
  return IMQ_OK;
}

int32_t imq_decode_program_create(const imq_step_desc* d, imq_program** out) {
  if (!out) return fail(IMQ_EINVAL, "out must be non-null");
  *out = nullptr;
  if (!d || !d->layer || !d->final_norm || !d->positions || !d->slots || !d->h || !d->logits)
    return fail(IMQ_EINVAL, "null pointer in the step description");
  if (d->batch != 1) return fail(IMQ_EUNSUPPORTED, "the persistent decode step runs batch 1");
  if (d->layers < 1 || d->hidden < 64 || d->hidden % 64 || d->hidden > kMaxHidden)
    return fail(IMQ_EINVAL, "need layers >= 1 and hidden a multiple of 64 up to 4096");
  if (d->heads < 1 || d->kv_heads < 1 || d->heads % d->kv_heads || d->heads / d->kv_heads > 8)
    return fail(IMQ_EINVAL, "need kv_heads | heads with at most 8 query heads per KV head");
  if (d->intermediate < 64 || d->intermediate % 64 || d->vocab < 1)
    return fail(IMQ_EINVAL, "bad intermediate size or vocabulary");
  if (d->capacity < 1 || d->num_slots < 1 || d->max_len < 1)
    return fail(IMQ_EINVAL, "capacity, num_slots and max_len must be >= 1");
  if (!(d->theta > 1.0f) || !(d->eps >= 0.0f)) return fail(IMQ_EINVAL, "bad theta or eps");
  if (!aligned(d->h, 16)) return fail(IMQ_EINVAL, "h must be 16-byte aligned");
  int32_t code;
  if (!current_device(&code)) return code;
  const int B = d->batch, D = d->hidden, Hq = d->heads, Hkv = d->kv_heads, I = d->intermediate;
  const int qd = Hq * kD, kvd = Hkv * kD;
  for (int i = 0; i < d->layers; ++i) {
    const imq_step_layer& Ly = d->layer[i];
    if ((code = check_qweight(Ly.q, qd, D, "q")) || (code = check_qweight(Ly.k, kvd, D, "k")) ||
        (code = check_qweight(Ly.v, kvd, D, "v")) || (code = check_qweight(Ly.o, D, qd, "o")) ||
        (code = check_qweight(Ly.gate, I, D, "gate")) || (code = check_qweight(Ly.up, I, D, "up")) ||
        (code = check_qweight(Ly.down, D, I, "down")))
      return code;
    if (!Ly.input_norm || !Ly.post_norm || !Ly.q_norm || !Ly.k_norm || !Ly.k_pool || !Ly.v_pool)
      return fail(IMQ_EINVAL, "null norm weight or KV pool");
    if (!aligned(Ly.k_pool, 16) || !aligned(Ly.v_pool, 16))
      return fail(IMQ_EINVAL, "the KV pools must be 16-byte aligned");
  }
  if ((code = check_qweight(d->head, d->vocab, D, "head")) != IMQ_OK) return code;
  if ((int64_t)d->num_slots * Hkv * d->capacity * kD * 2 >= ((int64_t)1 << 31))
    return fail(IMQ_EUNSUPPORTED, "a KV pool of 2 GiB or more exceeds the attention's offsets");

  // the RMSNorms folded into the projections around them (every one but the first layer's
  // input norm): the o and down stages write x' = bf16(h * w_next) and one sum of squares
  // of the new h per tile, which the next stage reads
  const TileShape ts_o = tile_shape(qd), ts_d = tile_shape(I);
  if (ts_o.shape < 0 || ts_d.shape < 0)
    return fail(IMQ_EUNSUPPORTED, "o or down outside the persistent qmv tiles");
  const int tiles_o = (D + (kThreads >> ts_o.sh) - 1) / (kThreads >> ts_o.sh);
  const int tiles_d = (D + (kThreads >> ts_d.sh) - 1) / (kThreads >> ts_d.sh);
  if (tiles_o > kMaxNormParts || tiles_d > kMaxNormParts)
    return fail(IMQ_EUNSUPPORTED, "more tiles of o or down than the folded norm reads");

  imq_program* prog = new imq_program();
  (void)hipGetDevice(&prog->device);
  const int span = std::min(d->max_len, d->capacity);
  int splits, cps;
  attention_split(B, Hkv, span, &splits, &cps);
  // activations: q, k, v, attention output, SiLU*up, x' (bf16), then the partials and the
  // sums of squares (fp32)
  const size_t off_q = 0, off_k = off_q + (size_t)B * qd * 2, off_v = off_k + (size_t)B * kvd * 2;
  const size_t off_attn = off_v + (size_t)B * kvd * 2, off_act = off_attn + (size_t)B * qd * 2;
  const size_t off_xn = off_act + (size_t)B * I * 2;
  const size_t off_part = (off_xn + (size_t)B * D * 2 + 255) & ~(size_t)255;
  const size_t off_ml = off_part + (size_t)B * Hq * splits * kD * 4;
  const size_t off_sso = (off_ml + (size_t)B * Hq * splits * 8 + 255) & ~(size_t)255;
  const size_t off_ssd = off_sso + (size_t)tiles_o * 4;
  const size_t scratch = off_ssd + (size_t)tiles_d * 4;
  if (hipMalloc(&prog->d_scratch, scratch) != hipSuccess) {
    free_program(prog);
    return fail(IMQ_ELAUNCH, "hipMalloc of the program activations failed");
  }
  char* sc = static_cast<char*>(prog->d_scratch);
  uint16_t* q = reinterpret_cast<uint16_t*>(sc + off_q);
  uint16_t* k = reinterpret_cast<uint16_t*>(sc + off_k);
  uint16_t* v = reinterpret_cast<uint16_t*>(sc + off_v);
  uint16_t* attn = reinterpret_cast<uint16_t*>(sc + off_attn);
  uint16_t* act = reinterpret_cast<uint16_t*>(sc + off_act);
  uint16_t* xn = reinterpret_cast<uint16_t*>(sc + off_xn);
  float* part = reinterpret_cast<float*>(sc + off_part);
  float* ml = reinterpret_cast<float*>(sc + off_ml);
  float* ssq_o = reinterpret_cast<float*>(sc + off_sso);
  float* ssq_d = reinterpret_cast<float*>(sc + off_ssd);
  // the last stage added takes x' and 1/rms from `ssq` (`parts` sums of squares) ...
  auto scaled = [&](const float* ssq, int parts) {
    Stage& S = prog->stages.back();
    S.ssq_in = ssq;
    S.nssq = parts;
  };
  // ... or writes them for the next stage
  auto residual_norm = [&](const uint16_t* w_next, float* ssq) {
    Stage& S = prog->stages.back();
    S.norm_next = w_next;
    S.xn_out = xn;
    S.ssq_out = ssq;
  };
  auto qp = [](const imq_qweight& w, void* y, int N, int K) {
    QProb p;
    memset(&p, 0, sizeof(p));
    p.w = w.w;
    p.s = w.scales;
    p.b = w.biases;
    p.y = y;
    p.N = N;
    p.K = K;
    return p;
  };
  int prev = -1;
  for (int i = 0; i < d->layers && code == IMQ_OK; ++i) {
    const imq_step_layer& Ly = d->layer[i];
    // the first layer's input norm runs in its q/k/v stage; later ones were folded into the
    // previous layer's down stage
    code = add_qmv_stage(prog, {qp(Ly.q, q, qd, D), qp(Ly.k, k, kvd, D), qp(Ly.v, v, kvd, D)},
                         i == 0 ? kXNorm : kXScaled, kEpiBf16, prev, i == 0 ? nullptr : xn, d->h,
                         Ly.input_norm, d->eps, nullptr);
    if (code) break;
    if (i > 0) scaled(ssq_d, tiles_d);
    const int s_qkv = (int)prog->stages.size() - 1;
    Stage A;
    memset(&A, 0, sizeof(A));
    A.kind = kKindAttention;
    A.wait = s_qkv;
    A.wait_count = prog->stages[s_qkv].count;
    A.count = B * Hkv * splits;
    A.first = prog->ntasks;
    A.eps = d->eps;
    A.log2_theta = log2f(d->theta);
    A.scale = 1.0f / sqrtf((float)kD);
    A.q = q;
    A.k = k;
    A.v = v;
    A.q_norm = Ly.q_norm;
    A.k_norm = Ly.k_norm;
    A.k_pool = Ly.k_pool;
    A.v_pool = Ly.v_pool;
    A.attn_out = attn;
    A.positions = d->positions;
    A.slots = d->slots;
    A.part = part;
    A.ml = ml;
    A.Hq = Hq;
    A.Hkv = Hkv;
    A.capacity = d->capacity;
    A.num_slots = d->num_slots;
    A.max_len = span;
    A.splits = splits;
    A.cps = cps;
    prog->ntasks += A.count;
    prog->stages.push_back(A);
    const int s_attn = (int)prog->stages.size() - 1;
    code = add_qmv_stage(prog, {qp(Ly.o, nullptr, D, qd)}, kXVector, kEpiResidualNorm, s_attn,
                         attn, d->h, nullptr, d->eps, nullptr);
    if (code) break;
    residual_norm(Ly.post_norm, ssq_o);
    const int s_o = (int)prog->stages.size() - 1;
    code = add_qmv_stage(prog, {qp(Ly.gate, nullptr, I, D), qp(Ly.up, nullptr, I, D)}, kXScaled,
                         kEpiSiluPair, s_o, xn, d->h, nullptr, d->eps, act);
    if (code) break;
    scaled(ssq_o, tiles_o);
    const int s_gu = (int)prog->stages.size() - 1;
    code = add_qmv_stage(prog, {qp(Ly.down, nullptr, D, I)}, kXVector, kEpiResidualNorm, s_gu, act,
                         d->h, nullptr, d->eps, nullptr);
    if (code) break;
    residual_norm(i + 1 < d->layers ? d->layer[i + 1].input_norm : d->final_norm, ssq_d);
    prev = (int)prog->stages.size() - 1;
  }
  if (code == IMQ_OK) {
    code = add_qmv_stage(prog, {qp(d->head, d->logits, d->vocab, D)}, kXScaled, kEpiF32, prev, xn,
                         d->h, nullptr, d->eps, nullptr);
    if (code == IMQ_OK) scaled(ssq_d, tiles_d);
  }
  if (code == IMQ_OK) code = finish_program(prog);
  if (code != IMQ_OK) {
    free_program(prog);
    return code;
  }
  *out = prog;
  return IMQ_OK;
}

int32_t imq_program_launch(imq_program* p, void* stream) {
  if (!p) return fail(IMQ_EINVAL, "null program");
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev != p->device)
    return fail(IMQ_EINVAL, "the program was created on another device");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t n = p->reset_words;
  hipLaunchKernelGGL(reset_kernel, dim3((uint32_t)((n + kThreads - 1) / kThreads)), dim3(kThreads),
                     0, st, p->d_words, n);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(IMQ_ELAUNCH, std::string("reset launch failed: ") + hipGetErrorString(e));
  StepArgs a;
  a.done = p->d_words;
  a.status = p->d_status;
  a.ntasks = p->ntasks;
  a.sub_stride = p->sub_stride;
  a.staged = 0;
  a.pad = 0;
  hipLaunchKernelGGL(step_kernel, dim3(p->grid), dim3(kThreads), p->lds, st,
                     static_cast<const Stage*>(p->d_stages), a);
  e = hipGetLastError();
  if (e != hipSuccess) return fail(IMQ_ELAUNCH, std::string("persistent launch failed: ") + hipGetErrorString(e));
  return ok();
}

int32_t imq_program_launch_staged(imq_program* p, void* stream) {
  if (!p) return fail(IMQ_EINVAL, "null program");
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev != p->device)
    return fail(IMQ_EINVAL, "the program was created on another device");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t n = p->reset_words;
  hipLaunchKernelGGL(reset_kernel, dim3((uint32_t)((n + kThreads - 1) / kThreads)), dim3(kThreads),
                     0, st, p->d_words, n);
  StepArgs a;
  a.done = p->d_words;
  a.status = p->d_status;
  a.ntasks = p->ntasks;
  a.sub_stride = p->sub_stride;
  a.staged = 1;
  a.pad = 0;
  for (size_t i = 0; i < p->stages.size(); ++i) {
    const Stage& S = p->stages[i];
    const dim3 grid(S.count), block(kThreads);
    const size_t lds = p->stage_lds[i];
    if (S.kind == kKindAttention) {
      hipLaunchKernelGGL((attention_stage_kernel<kAttnWaves, false>), grid, block, lds, st, S, a);
      continue;
    }
#define IMQ_STAGE_CASE(NCH, XR, XSRC, EPI, SHAPE)                                              \
  case (XSRC) * 32 + (EPI) * 4 + (SHAPE):                                                   \
    hipLaunchKernelGGL((qmv_stage_kernel<NCH, XR, XSRC, EPI>), grid, block, lds, st, S, a);   \
    break;
#define IMQ_STAGE_SHAPES_X2(XSRC, EPI)      \
  IMQ_STAGE_CASE(2, 2, XSRC, EPI, kShape22) \
  IMQ_STAGE_CASE(5, 2, XSRC, EPI, kShape52) \
  IMQ_STAGE_CASE(8, 2, XSRC, EPI, kShape82)
    switch (S.xsrc * 32 + S.epi * 4 + S.shape) {
      IMQ_STAGE_SHAPES_X2(kXVector, kEpiBf16)
      IMQ_STAGE_CASE(5, 5, kXVector, kEpiBf16, kShape55)
      IMQ_STAGE_SHAPES_X2(kXVector, kEpiResidual)
      IMQ_STAGE_CASE(5, 5, kXVector, kEpiResidual, kShape55)
      IMQ_STAGE_SHAPES_X2(kXVector, kEpiResidualNorm)
      IMQ_STAGE_CASE(5, 5, kXVector, kEpiResidualNorm, kShape55)
      IMQ_STAGE_SHAPES_X2(kXNorm, kEpiBf16)
      IMQ_STAGE_SHAPES_X2(kXNorm, kEpiSiluPair)
      IMQ_STAGE_SHAPES_X2(kXNorm, kEpiF32)
      IMQ_STAGE_SHAPES_X2(kXScaled, kEpiBf16)
      IMQ_STAGE_SHAPES_X2(kXScaled, kEpiSiluPair)
      IMQ_STAGE_SHAPES_X2(kXScaled, kEpiF32)
      default:
        return fail(IMQ_EUNSUPPORTED, "stage variant without a kernel");
    }
#undef IMQ_STAGE_SHAPES_X2
#undef IMQ_STAGE_CASE
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(IMQ_ELAUNCH, std::string("stage launch failed: ") + hipGetErrorString(e));
  return ok();
}

int32_t imq_program_status(imq_program* p, int32_t* failed) {
  if (!p || !failed) return fail(IMQ_EINVAL, "null argument");
  if (hipDeviceSynchronize() != hipSuccess) return fail(IMQ_ELAUNCH, "device synchronisation failed");
  uint32_t s = 0;
  if (hipMemcpy(&s, p->d_status, 4, hipMemcpyDeviceToHost) != hipSuccess)
    return fail(IMQ_ELAUNCH, "reading the status word failed");
  *failed = s != 0;
  if (s && hipMemset(p->d_status, 0, 4) != hipSuccess) return fail(IMQ_ELAUNCH, "clearing the status word failed");
  return ok();
}

int32_t imq_program_info(const imq_program* p, int32_t* tasks, int32_t* stages, int32_t* workgroups,
                         int32_t* lds_bytes) {
  if (!p) return fail(IMQ_EINVAL, "null program");
  if (tasks) *tasks = p->ntasks;
  if (stages) *stages = (int32_t)p->stages.size();
  if (workgroups) *workgroups = p->grid;
  if (lds_bytes) *lds_bytes = (int32_t)p->lds;
  return ok();
}

void imq_program_destroy(imq_program* p) { free_program(p); }

}  // extern "C"
