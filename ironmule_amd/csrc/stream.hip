// Streaming engine for chains of one-row (M = 1) 4-bit qmv stages on MI355X (gfx950):
// one persistent launch streams the weights of every stage of a program.
// C ABI: include/ironmule_step.h (imq_stream_*).
//
// Work.  Every stage is cut into wavefront tiles of 64 / LPR weight rows (LPR lanes per
// row, the one-row kernel's lane shape, so every output equals imq_qmv's bit for bit).
// The tiles of all stages form one list in stage order.  For independent stages the
// list is cut into runs of R consecutive tiles (16 or a little more, sized on the host
// so that the runs split the list into whole rounds) and wavefront v of the V in the
// grid runs runs v, v + V, ...: the device streams one compact window of the weights, and
// a wavefront resolves a problem's descriptors once per run, jumping to a run's problem
// through a per-program run table.  For chained stages wavefront v runs tiles v, v + V,
// ... of each stage (counted from the stage's first tile), v numbering the wavefronts
// across the workgroups first, so that every stage is spread over the whole device.
//
// Pipelining.  A wavefront keeps two tiles in registers: while it computes one, the
// loads of the next are in flight.  Loads are raw buffer loads issued unconditionally
// (a piece that is not needed reads past its buffer, which returns zero without a memory
// access), and a pass over the two tiles has no exit in between, so the number of loads
// in flight is the same on every path and the waits the compiler places before each tile
// are exact.  Weights are read with the non-temporal cache policy.
//
// Two modes:
//   * independent stages (no stage reads another's output): every distinct x of the
//     program is staged in LDS once, at the start, in the pair order of the dot2 chains;
//     after that a wavefront streams its tiles from the first stage to the last with no
//     barrier and no wait, the next tile's loads always in flight;
//   * chained stages (a stage may wait for an earlier one): all wavefronts enter every
//     stage in order.  Entering a stage, a workgroup signals the previous stage if a later
//     stage waits for it (each wavefront waits for its own stores, then one atomic add),
//     issues the loads of its first two tiles of the new stage, waits for the stage's
//     input (wavefront 0 polls), stages x in LDS (double-buffered by stage parity) and
//     computes.  The weight loads are issued before the wait, so the weight stream of a
//     stage overlaps the completion of the one it depends on.
//
// Completion counters.  A stage has kSubs counters, each on its own 128-byte line; the
// workgroups of the grid spread their increments over them (one atomic counter
// serialises its increments).  A waiter sums the kSubs counters with one load per lane.
// Activations written and read inside a launch go through sc1 stores and loads, which
// are coherent across the XCDs' L2 caches; every wait is bounded.

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <string>
#include <vector>

#include "../../include/ironmule_step.h"
#include "common.h"
#include "runtime.h"
#include "stream_runs.h"

namespace {

using namespace imq_dev;
using imq_rt::aligned;
using imq_rt::current_device;
using imq_rt::DeviceInfo;
using imq_rt::fail;
using imq_rt::ok;

#ifndef IMQ_STREAM_THREADS
#define IMQ_STREAM_THREADS 768
#endif
// One workgroup of 12 wavefronts per CU: every distinct x of a program is loaded and
// staged once per CU (with three workgroups of 4 wavefronts a CU read and staged it three
// times, about as many bytes at the start of a launch as the first two tiles' weights).
constexpr int kThreads = IMQ_STREAM_THREADS;
constexpr int kWaves = kThreads / 64;
constexpr int kNch = 5;                // 16-byte chunks per lane: m1_lane_shift gives <= 5 for K <= 10240
constexpr int kMaxK = 10240;           // m1_lane_shift gives <= kNch chunks per lane up to here
constexpr int kXr = (kMaxK + kThreads * 8 - 1) / (kThreads * 8);  // x pieces of 8 values per thread
constexpr int kSubs = 16;              // completion counters per stage
constexpr int kLine = 32;              // words per counter line
constexpr int kMaxPolls = 1 << 22;
constexpr int kMaxStageProblems = 3;
constexpr int kMaxSlots = 8;           // distinct x rows of an independent-stage program
constexpr size_t kSlotLds = 64 * 1024;  // LDS for those rows
constexpr int kSbWords = 256;           // per wavefront: the span's scale halves, then at kBiasArea its bias halves
constexpr int kBiasArea = 512;          // byte offset of the bias halves in the area
constexpr int kDepth = 2;                // tiles in flight per wavefront (independent stages)
constexpr int kShards = 16;              // claim counters (independent stages)
#ifndef IMQ_STREAM_PRE_SLOTS
#define IMQ_STREAM_PRE_SLOTS 3
#endif
constexpr int kPreSlots = IMQ_STREAM_PRE_SLOTS;  // x rows loaded ahead of the first weights

// LDS bytes of one staged x row of K values: C = K/32 chunks of 80 bytes each, the
// chunk's four words in pair order (64 bytes), its sum and -128 times its sum (8 bytes)
// and 8 bytes of padding.
// A lane reads all five pieces of its chunk from one address (immediate offsets), and the
// 20-dword chunk stride puts the lanes of a quarter-wave on distinct banks.
constexpr int kXChunk = 80;
constexpr size_t x_bytes(int K) { return (size_t)(K / 32) * kXChunk; }

struct SProb {
  const uint32_t* w;
  const uint16_t* s;
  const uint16_t* b;
  uint16_t* y;
  int32_t N;
  int32_t tile_end;  // one past the problem's last tile, counted within the stage
  int32_t live;      // 1: a later stage of the launch reads y (sc1 stores)
  int32_t pad;
};

struct SStage {
  const uint16_t* x;
  int32_t K, sh, nch, nprob;
  int32_t tiles, first;  // the stage's tiles are first .. first + tiles - 1 of the program
  int32_t wait;          // index of the stage this one waits for, or -1
  int32_t signal;        // 1: a later stage waits for this one
  int32_t x_live;        // 1: x is written by an earlier stage of the same launch
  int32_t xoff;          // byte offset of the stage's staged x in LDS
  int32_t pad0, pad1;
  SProb p[kMaxStageProblems];
};

struct XSlot {
  const uint16_t* x;
  int32_t K, off;
};

struct SArgs {
  uint32_t* counters;  // kSubs lines per stage
  uint32_t* status;
  const int32_t* run_site;  // independent stages: (stage << 2) | problem of each run's first tile
  uint32_t* claim;          // independent stages: kShards claim counters, kLine words apart
  int32_t nstages, total, waves, sb_off;  // sb_off: LDS byte offset of the scale/bias areas
  int32_t nslots, pad;
  // chained stages: per (stage, wavefront) four s_memrealtime stamps, or nullptr
  uint64_t* trace;
  imq_runs::ShardPlan runs;  // independent stages: dealt and claimed runs, claim shards
  XSlot slot[kMaxSlots];
};
static_assert(kShards == imq_runs::kMaxShards, "one claim counter line per shard");

typedef const struct SStage __attribute__((address_space(4)))& StageRef;

template <typename T>
__device__ __forceinline__ T* uniform_ptr(T* p) {
  const uint64_t u = reinterpret_cast<uint64_t>(p);
  const uint64_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)u);
  const uint64_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(u >> 32));
  return reinterpret_cast<T*>((hi << 32) | lo);
}

// Stage i's descriptor, seen through the constant address space (nothing writes the table
// while a launch runs) at a uniform address, so its fields are read with scalar loads
// that wait on nothing but each other.
__device__ __forceinline__ StageRef stage_at(const SStage* __restrict__ st, int i) {
  return *reinterpret_cast<const SStage __attribute__((address_space(4)))*>(
      reinterpret_cast<uint64_t>(uniform_ptr(st + i)));
}

__device__ __forceinline__ uint32_t* counter(const SArgs& a, int stage, int sub) {
  return a.counters + ((size_t)stage * kSubs + sub) * kLine;
}

// One tile's loads: kNch weight chunks per lane, and the tile's scales and biases (the
// span of its rows, adjacent in memory: at most 81 dwords, read 16 bytes per lane by the
// first 21 lanes).
struct Tile {
  uint4 w[kNch];
  uint4 s, b;
};

// One problem of a stage (global tiles t0 .. tend-1 of the program), resolved once while
// a wavefront works through its tiles, with what every tile needs: the buffer descriptors
// and row stride (scalar), and per lane its chunk column j, its row in the tile rl, how
// many of its kNch chunk slots hold chunks of the row, and for each slot the offsets
// that slot reads: in the tile's weights, in the staged x and in the scale/bias area.
struct Site {
  __amdgpu_buffer_rsrc_t wr, sr, br, yr;
  uint16_t* y;
  int N, K, sh, nch, xoff, live, t0, tend;
  int rows;        // rows per tile: 64 >> sh
  uint32_t w4;     // bytes per weight row (K / 2)
  // per lane
  uint32_t woff[kNch];  // weight byte offset from the tile's first row; kPastBuffer past the lane's chunks
  uint32_t xo[kNch];    // LDS byte offset of the slot's staged x chunk
  uint32_t so[kNch];    // byte offset of the slot's scale half in the area, before the span's misalignment
  int rl, j, nvalid;
  int cls;  // 0: every lane has kNch chunks, 1: every lane has kNch - 1, 2: lanes differ
};

__device__ __forceinline__ Site site_at(const SStage* __restrict__ st, int si, int pi) {
  StageRef S = stage_at(st, si);
  Site c;
  c.y = S.p[pi].y;
  c.N = S.p[pi].N;
  c.live = S.p[pi].live;
  c.K = S.K;
  c.sh = S.sh;
  c.nch = S.nch;
  c.xoff = S.xoff;
  c.t0 = S.first + (pi == 0 ? 0 : S.p[pi - 1].tile_end);
  c.tend = S.first + S.p[pi].tile_end;
  const int G = c.K >> 6, C = c.K >> 5;
  c.w4 = (uint32_t)c.K >> 1;
  // the scale/bias range rounded up to whole dwords: the extra half lies in the same
  // aligned dword as the last one, so it is mapped, and it belongs to no row
  const uint32_t sbb = ((uint32_t)c.N * (uint32_t)G * 2u + 3u) & ~3u;
  c.wr = buffer_rsrc(S.p[pi].w, (uint32_t)c.N * c.w4);
  c.sr = buffer_rsrc(S.p[pi].s, sbb);
  c.br = buffer_rsrc(S.p[pi].b, sbb);
  c.yr = buffer_rsrc(c.y, (uint32_t)c.N * 2u);
  c.rows = 64 >> c.sh;
  const int lane = threadIdx.x & 63;
  c.j = lane & ((1 << c.sh) - 1);
  c.rl = lane >> c.sh;
  // chunks j, j + 2^sh, ... below C, at most nch of them
  const int nv = (C - c.j + (1 << c.sh) - 1) >> c.sh;
  c.nvalid = nv < c.nch ? nv : c.nch;
  // lane j = 0 has the most chunks, lane j = 2^sh - 1 the fewest
  const int nv_hi = min((C + (1 << c.sh) - 1) >> c.sh, c.nch), nv_lo = min(C >> c.sh, c.nch);
  c.cls = nv_lo != nv_hi ? 2 : nv_hi == kNch ? 0 : nv_hi == kNch - 1 ? 1 : 2;
  // chunk slot i is chunk j + i 2^sh of the row; a slot past the lane's chunks reads no
  // weights and rereads the lane's first chunk of x and its scale/bias word
  const uint32_t wlane = (uint32_t)c.rl * c.w4 + 16u * (uint32_t)c.j;
#pragma unroll
  for (int i = 0; i < kNch; ++i) {
    const bool in = i < c.nvalid;
    const int ii = in ? i : 0;
    c.woff[i] = in ? wlane + ((16u << c.sh) * (uint32_t)i) : kPastBuffer;
    c.xo[i] = (uint32_t)c.xoff + (uint32_t)kXChunk * (uint32_t)(c.j + (ii << c.sh));
    c.so[i] = 2u * (uint32_t)(c.rl * G + (c.j >> 1) + (ii << (c.sh - 1)));
  }
  return c;
}

// Moves (stage si, problem pi) forward to the problem holding global tile g, reading only
// the problems' tile ranges on the way.
__device__ __forceinline__ void advance(const SStage* __restrict__ st, int& si, int& pi, int g) {
  for (;;) {
    StageRef S = stage_at(st, si);
    if (g < S.first + S.p[pi].tile_end) return;
    if (pi + 1 < S.nprob) {
      ++pi;
    } else {
      ++si;
      pi = 0;
    }
  }
}

// Moves a cursor (stage si, problem pi, resolved site c) forward to the problem holding
// global tile g; the site is resolved once, at the end.
__device__ __forceinline__ void seek(const SStage* __restrict__ st, int& si, int& pi, Site& c, int g) {
  if (g < c.tend) return;
  advance(st, si, pi, g);
  c = site_at(st, si, pi);
}

// The scale/bias span of a tile: the halves of rows row0 .. row0 + R - 1 (R = 64 >> sh),
// R * G of them from half row0 * G on, read as dwords from the dword boundary at or below
// its start; `mis` is 1 when that start is odd.  At most 5 * 64 + 2 bytes: 81 dwords.
struct Span {
  uint32_t a0;
  int mis, nd;
};

__device__ __forceinline__ Span span_of(const Site& c, int row0) {
  const int G = c.K >> 6;
  const uint32_t h0 = (uint32_t)row0 * (uint32_t)G;
  const uint32_t h1 = min((uint32_t)(row0 + (64 >> c.sh)), (uint32_t)c.N) * (uint32_t)G;
  Span sp;
  sp.a0 = (h0 & ~1u) * 2u;
  sp.mis = (int)(h0 & 1u);
  sp.nd = (int)((h1 - (h0 & ~1u) + 1u) >> 1);
  return sp;
}

// Issues the loads of global tile g of site c (valid false: every load reads past its
// buffer, which returns zero without a memory access).  The tile's first row offset is
// added with saturation, so that a slot past the lane's chunks (kPastBuffer) stays past
// the buffer on every row.
__device__ __forceinline__ void load_site(const Site& c, int g, bool valid, int lane, Tile& T) {
  const int row0 = (g - c.t0) * c.rows;
  // scales and biases first: the tile's compute needs them before its first chunk
  const Span sp = span_of(c, row0);
  const uint32_t off = valid && 4 * lane < sp.nd ? sp.a0 + 16u * lane : kPastBuffer;
  T.s = load_b128(c.sr, off);
  T.b = load_b128(c.br, off);
  const uint32_t base = valid && row0 + c.rl < c.N ? (uint32_t)row0 * c.w4 : kPastBuffer;
#pragma unroll
  for (int i = 0; i < kNch; ++i) T.w[i] = load_b128_nt(c.wr, __builtin_elementwise_add_sat(base, c.woff[i]));
}

// Adds lane 15 of the previous row of 16 lanes (CTRL row_bcast:15) or lane 31 (row_bcast:31)
// to the rows of ROWS; the other rows are left as they are.
template <int CTRL, int ROWS>
__device__ __forceinline__ float add_bcast(float v) {
  return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                                   CTRL, ROWS, 0xF, false));
}

// The sum over a lane's first NS chunk slots of one tile: scale * (chunk dot) + bias *
// (chunk sum), accumulated slot by slot; with SEL a slot past the lane's chunks is
// discarded by a select (its zero weights stand for q = 0, not for nothing).  No branch,
// so the LDS reads of all slots can be issued early.
template <int NS, bool SEL>
__device__ __forceinline__ float lane_sum(const Site& c, const Tile& T, const char* smem,
                                          const char* sbm, uint32_t magic) {
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < NS; ++i) {
    const char* sb = sbm + c.so[i];
    const float sc = __uint_as_float((uint32_t)*reinterpret_cast<const uint16_t*>(sb) << 16);
    const float bi = __uint_as_float((uint32_t)*reinterpret_cast<const uint16_t*>(sb + kBiasArea) << 16);
    const uint4* xc = reinterpret_cast<const uint4*>(smem + c.xo[i]);
    const float2 sum = reinterpret_cast<const float2*>(xc + 4)[0];  // (chunk sum, -128 sum)
    const float d = chunk_dot(T.w[i], xc[0], xc[1], xc[2], xc[3], sum.y, magic);
    const float v = fmaf(sc, d, fmaf(bi, sum.x, acc));
    acc = !SEL || i < c.nvalid ? v : acc;
  }
  return acc;
}

// Computes global tile g of site c from its loads, the staged x (LDS at smem) and this
// wavefront's scale/bias area `sbw` (kSbWords dwords of LDS), and stores the tile's rows
// as bf16 unless `keep` is false: with sc1 stores when a later stage of the launch reads
// them.  The chunk order and the dot2 chains are the one-row kernel's; its cross-lane sums
// (row of 16, then lanes 16 and 32 apart) are formed here by row broadcasts, the same
// additions with their operands swapped, so the row sums have the same bits and end in
// the row's last lane.
__device__ __forceinline__ void compute_site(const Site& c, int g, int lane, const Tile& T,
                                             const char* smem, uint32_t* sbw, uint32_t magic,
                                             bool keep = true) {
  const int row0 = (g - c.t0) * c.rows;
  const int row = row0 + c.rl;
  // the span's scale and bias halves as loaded, in this wavefront's own LDS area (lanes
  // past the first 32 hold nothing of the span)
  if (lane < 32) {
    reinterpret_cast<uint4*>(sbw)[lane] = T.s;
    reinterpret_cast<uint4*>(reinterpret_cast<char*>(sbw) + kBiasArea)[lane] = T.b;
  }
  const char* sbm = reinterpret_cast<const char*>(sbw) + 2 * span_of(c, row0).mis;
  const float acc = c.cls == 0   ? lane_sum<kNch, false>(c, T, smem, sbm, magic)
                    : c.cls == 1 ? lane_sum<kNch - 1, false>(c, T, smem, sbm, magic)
                                 : lane_sum<kNch, true>(c, T, smem, sbm, magic);
  float v = row16_sum(acc);
  if (c.sh >= 5) v = add_bcast<0x142, 0xA>(v);  // rows 1 and 3 add rows 0 and 2
  if (c.sh >= 6) v = add_bcast<0x143, 0xC>(v);  // rows 2 and 3 add lane 31 (rows 0 + 1)
  if (keep && c.j == (1 << c.sh) - 1 && row < c.N) {
    if (c.live)
      store_b16_sc1(c.yr, 2u * row, f32_to_bf16_bits(v));
    else
      c.y[row] = f32_to_bf16_bits(v);
  }
}

// Stages the bf16 row x (K values) in LDS at `dst` in pair order with its chunk sums; the
// whole workgroup takes part.  `live`: x was written earlier in this launch (sc1 loads).
__device__ __forceinline__ void load_x(const uint16_t* x, int K, bool live, int tid, uint4 (&xs)[kXr]) {
  const int W = K >> 3;
  const __amdgpu_buffer_rsrc_t r = buffer_rsrc(x, (uint32_t)K * 2u);
#pragma unroll
  for (int t = 0; t < kXr; ++t) {
    const int i = tid + kThreads * t;
    const uint32_t off = i < W ? 16u * i : kPastBuffer;
    xs[t] = live ? load_b128_sc1(r, off) : load_b128(r, off);
  }
}

__device__ __forceinline__ void store_x(const uint4 (&xs)[kXr], int K, char* dst, int tid) {
  const int W = K >> 3;
#pragma unroll
  for (int t = 0; t < kXr; ++t) {
    const int i = tid + kThreads * t;  // the four words of a chunk are four aligned lanes
    float part = sum8(xs[t]);
    part += dpp<0xB1>(part);  // lane ^ 1
    part += dpp<0x4E>(part);  // lane ^ 2
    if (i < W) {
      char* chunk = dst + (size_t)kXChunk * (i >> 2);
      reinterpret_cast<uint4*>(chunk)[i & 3] = pair_order(xs[t]);
      if ((i & 3) == 0) reinterpret_cast<float2*>(chunk + 64)[0] = make_float2(part, -128.0f * part);
    }
  }
}

__device__ __forceinline__ void stage_x(const uint16_t* x, int K, bool live, char* dst, int tid) {
  uint4 xs[kXr];
  load_x(x, K, live, tid, xs);
  store_x(xs, K, dst, tid);
}

// ------------------------------------------------------------ independent stages

// Wavefront v takes runs of R consecutive tiles: run v, v + V, v + 2V, ... of the program
// (V wavefronts), so at any moment the device streams one compact window of the weights,
// and a wavefront resolves a problem's descriptors once per run rather than once per
// tile.  R (16 or a little more) is chosen so that the runs split the program evenly over
// the wavefronts.  Dealt runs cover whole rounds of the program's first tiles; the rest is
// cut into runs of dyn_run tiles (the last ending at the program's last tile) that the
// wavefronts claim one at a time from a counter (an atomic add), so that the wavefronts
// that stream faster take more of them and all finish together (measured on MI355X: with
// every run dealt, the last wavefronts of a 20-layer launch ended 35 us after the median
// one; claiming the last 25% in runs of 8 tiles took that launch from 5.83 to 6.13 TB/s,
// while runs of 4 or 16 tiles and a 12% share gained less; each shard's last 30% in single
// tiles then ended a 20-layer launch about 2 us earlier than runs of 2).  The claimed runs are split
// between `shards` counters, each on its own line (one counter serialises its atomic adds:
// 16K claims on one counter cost a 20-layer launch 100 us).  The plan, the claim count
// that returns a shard's counter to zero and the two cursors' steps are in stream_runs.h,
// which a host simulation of this protocol compiles as well.  kDepth tiles are in flight
// (one at the start, until the first is computed): the loads of a wavefront's tile
// k + kDepth are issued as soon as its tile k has been computed; the load cursor claims the
// runs and the compute cursor, at most kDepth tiles behind, takes them from a two-entry
// queue.
constexpr int kRunTarget = 16;
#ifndef IMQ_STREAM_DYN_RUN
#define IMQ_STREAM_DYN_RUN 8
#endif
#ifndef IMQ_STREAM_DYN_PERCENT
#define IMQ_STREAM_DYN_PERCENT 25
#endif
#ifndef IMQ_STREAM_TAIL_RUN
#define IMQ_STREAM_TAIL_RUN 1
#endif
#ifndef IMQ_STREAM_TAIL_PERCENT
#define IMQ_STREAM_TAIL_PERCENT 30
#endif
// workgroups in a row that land on distinct XCDs (workgroup b runs on XCD b % 8)
constexpr int kXcdSpread = 8;
static_assert(IMQ_STREAM_DYN_RUN > kDepth, "a claimed run is longer than the cursors' distance");

__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(3))) void stream_kernel(const SStage* __restrict__ st, SArgs a) {
  extern __shared__ uint4 smem_raw[];
  char* smem = reinterpret_cast<char*>(smem_raw);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int v = blockIdx.x * kWaves + wave;
  const imq_runs::RunPlan& P = a.runs.plan;
  const int total = P.total;
  uint32_t* sbw = reinterpret_cast<uint32_t*>(smem + a.sb_off) + kSbWords * wave;
  const uint32_t magic = in_vgpr(kMagic);
  using imq_runs::Pos;
  const int shard = imq_runs::shard_of_group(blockIdx.x, a.runs.shards, a.runs.spread);
  const imq_runs::ShardRuns sh = a.runs.shard[shard];
  auto tile = [&](const Pos& p) { return imq_runs::tile_of(P, sh, p); };
  imq_runs::ClaimQueue cq;
  uint32_t* ctr = a.claim + shard * kLine;
  const uint32_t last_claim = imq_runs::last_claim_of(sh.count, a.runs.shard_waves[shard]);
  auto claim = [&]() {
    uint32_t old = 0;
    if (lane == 0) old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    old = __builtin_amdgcn_readfirstlane(old);
    if (old == last_claim && lane == 0) st_sc1(ctr, 0u);
    return imq_runs::claimed_run(old, sh, P.runs);
  };
  auto step_load = [&](Pos& p) { imq_runs::step_load(P, sh, p, cq, claim); };
  auto step_compute = [&](Pos& p) { imq_runs::step_compute(P, sh, p, cq); };

  // the load cursor (stage ls, problem lp) and the compute cursor (cs, cp); a cursor that
  // leaves its problem starts from the problem of its run's first tile (a table lookup)
  // rather than walking through the problems in between
  int ls = 0, lp = 0, cs = 0, cp = 0;
  Site lc = site_at(st, 0, 0), cc = lc;
  const int32_t __attribute__((address_space(4)))* runs =
      reinterpret_cast<const int32_t __attribute__((address_space(4)))*>(
          reinterpret_cast<uint64_t>(uniform_ptr(a.run_site)));
  auto move = [&](int& si, int& pi, Site& c, int g, int r) {
    if (g < c.tend) return;
    const int e = runs[r];
    si = e >> 2;
    pi = e & 3;
    advance(st, si, pi, g);
    c = site_at(st, si, pi);
  };
  Tile T[kDepth];
  Pos lpos{v, 0}, cpos{v, 0};
  auto issue = [&](Tile& t) {
    const int g = tile(lpos);
    if (g < total) move(ls, lp, lc, g, lpos.r);
    load_site(lc, g, g < total, lane, t);
    step_load(lpos);
  };
  // x first: the loads of the first kPreSlots distinct x rows go ahead of the first tiles'
  // weights (loads return in issue order, so staging x then waits for x alone), the rest
  // after them
  uint4 xs[kPreSlots > 0 ? kPreSlots : 1][kXr];
#pragma unroll
  for (int k = 0; k < kPreSlots; ++k)
    load_x(a.slot[k].x, k < a.nslots ? a.slot[k].K : 0, false, tid, xs[k]);
  // The pipeline starts one tile deep: the first tile's loads go out behind x, the
  // wavefront computes that tile as soon as x is staged and it has landed, and only then
  // issues the next two.  (With both tiles issued up front, issuing them held every
  // wavefront until its CU's load queue drained, about 5 us, so no tile was computed before
  // the whole first wave of weights had arrived and HBM then waited for new requests.)
  static_assert(kDepth == 2, "the start peels one tile of a two-tile pipeline");
  issue(T[1]);
#pragma unroll
  for (int k = 0; k < kPreSlots; ++k)
    if (k < a.nslots) store_x(xs[k], a.slot[k].K, smem + a.slot[k].off, tid);
  for (int k = kPreSlots; k < a.nslots; ++k) stage_x(a.slot[k].x, a.slot[k].K, false, smem + a.slot[k].off, tid);
  lds_barrier();
  {
    const int gf = tile(cpos);
    if (gf >= total) return;  // uniform: no tiles (its one load read past its buffer)
    move(cs, cp, cc, gf, cpos.r);
    compute_site(cc, gf, lane, T[1], smem, sbw, magic, true);
    step_compute(cpos);
    issue(T[0]);
    issue(T[1]);
  }

  // Every pass runs all kDepth tiles with no exit in between, so that every path into the
  // loop head has issued the tiles' loads in the same order and each tile's compute waits
  // only for its own loads.  A tile past the end (the last pass) was loaded as zeros; it
  // is computed at the pass's first tile's site and not stored.
  for (;;) {
    const Pos p0 = cpos;
    const int g0 = tile(p0);
    if (g0 >= total) break;
#pragma unroll
    for (int d = 0; d < kDepth; ++d) {
      const int gd = tile(cpos);
      const bool in = gd < total;
      move(cs, cp, cc, in ? gd : g0, in ? cpos.r : p0.r);
      compute_site(cc, in ? gd : g0, lane, T[d], smem, sbw, magic, in);
      step_compute(cpos);
      issue(T[d]);
    }
  }
}

// ------------------------------------------------------------ chained stages

// Wavefront 0 polls the kSubs counters of `stage` until they add up to `count`; the
// workgroup then agrees on the outcome (false: timed out, or another workgroup did).
__device__ bool wait_for(const SArgs& a, int stage, uint32_t count, int* flag) {
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    const uint32_t* c = counter(a, stage, lane < kSubs ? lane : 0);
    int polls = 0, good = 1;
    for (;;) {
      uint32_t n = lane < kSubs ? ld_sc1(c) : 0u;
#pragma unroll
      for (int o = 8; o > 0; o >>= 1) n += __shfl_xor(n, o);
      n = __shfl(n, 0);
      if (n >= count) break;
      if (++polls >= kMaxPolls || ((polls & 63) == 0 && ld_sc1(a.status) != 0)) {
        good = 0;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (lane == 0) {
      if (!good) st_sc1(a.status, 1u);
      *flag = good;
    }
  }
  lds_barrier();
  return *flag != 0;
}

// Every workgroup enters every stage in order.  Within a stage the tiles are dealt
// round-robin: wavefront v runs the stage's tiles v, v + V, ... (counted from the
// stage's first), so a stage is spread over the whole device.
__global__ __launch_bounds__(kThreads) void stream_chain_kernel(const SStage* __restrict__ st,
                                                                SArgs a) {
  extern __shared__ uint4 smem_raw[];
  char* smem = reinterpret_cast<char*>(smem_raw);
  __shared__ int flag;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // wavefronts numbered across the workgroups first (wavefront w of workgroup b is w * grid
  // + b), so that a stage of fewer tiles than wavefronts is spread over every CU rather
  // than over the first workgroups' CUs
  const int v = wave * (int)gridDim.x + (int)blockIdx.x;
  const int V = a.waves;
  uint32_t* sbw = reinterpret_cast<uint32_t*>(smem + a.sb_off) + kSbWords * wave;
  const uint32_t magic = in_vgpr(kMagic);
  const uint32_t groups = gridDim.x;
  Tile A, B;

  // the optional trace: per (stage, wavefront) the stage's start (after signalling the
  // previous one), its input ready, its x staged and its last tile done
  uint64_t* const trace = uniform_ptr(a.trace);
  uint64_t stamp[4];
  auto mark = [&](int i) {
    if (trace) stamp[i] = __builtin_amdgcn_s_memrealtime();
  };
  for (int s = 0; s < a.nstages; ++s) {
    StageRef S = stage_at(st, s);
    if (s > 0 && stage_at(st, s - 1).signal) {  // this workgroup is done with stage s-1
      wait_vmem();
      lds_barrier();
      if (tid == 0)
        __hip_atomic_fetch_add(counter(a, s - 1, blockIdx.x % kSubs), 1u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
    mark(0);
    const int first = S.first, end = S.first + S.tiles;
    // this wavefront's first tile of the stage: the smallest g >= first with g - first = v mod V
    int g = first + v;
    int lp = 0, cp = 0, ls = s, cs = s;
    Site lc = site_at(st, s, 0), cc = lc;
    if (g < end) seek(st, ls, lp, lc, g);
    load_site(lc, g, g < end, lane, A);
    if (g + V < end) seek(st, ls, lp, lc, g + V);
    load_site(lc, g + V, g + V < end, lane, B);
    if (S.wait >= 0 && !wait_for(a, S.wait, groups, &flag)) return;
    mark(1);
    stage_x(S.x, S.K, S.x_live != 0, smem + S.xoff, tid);
    lds_barrier();
    mark(2);
    while (g < end) {
      seek(st, cs, cp, cc, g);
      compute_site(cc, g, lane, A, smem, sbw, magic);
      if (g + 2 * V < end) seek(st, ls, lp, lc, g + 2 * V);
      load_site(lc, g + 2 * V, g + 2 * V < end, lane, A);
      g += V;
      if (g >= end) break;
      seek(st, cs, cp, cc, g);
      compute_site(cc, g, lane, B, smem, sbw, magic);
      if (g + 2 * V < end) seek(st, ls, lp, lc, g + 2 * V);
      load_site(lc, g + 2 * V, g + 2 * V < end, lane, B);
      g += V;
    }
    if (trace) {
      mark(3);
      if (lane == 0) {
        uint64_t* row = trace + ((size_t)s * V + v) * 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) row[i] = stamp[i];
      }
    }
  }
}

__global__ __launch_bounds__(kThreads) void clear_kernel(uint32_t* words, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i < n) words[i] = 0u;
}

}  // namespace

struct imq_stream {
  int device = -1;
  bool chained = false;
  std::vector<SStage> stages;
  SStage* d_stages = nullptr;
  uint32_t* d_words = nullptr;  // counters, then the status word
  int32_t* d_runs = nullptr;    // independent stages: the problem of each run's first tile
  int64_t counter_words = 0;
  SArgs args;
  int grid = 0;
  size_t lds = 0;
};

namespace {

void free_stream(imq_stream* p) {
  if (!p) return;
  if (p->d_stages) (void)hipFree(p->d_stages);
  if (p->d_runs) (void)hipFree(p->d_runs);
  if (p->d_words) (void)hipFree(p->d_words);
  delete p;
}

}  // namespace

extern "C" {

int32_t imq_stream_create(const imq_qmv_stage* stages, int32_t count, int32_t workgroups,
                          imq_stream** out) {
  if (!out) return fail(IMQ_EINVAL, "out must be non-null");
  *out = nullptr;
  if (!stages || count < 1) return fail(IMQ_EINVAL, "need at least one stage");
  int32_t code;
  const DeviceInfo* dev = current_device(&code);
  if (!dev) return code;
  imq_stream* p = new imq_stream();
  (void)hipGetDevice(&p->device);
  memset(&p->args, 0, sizeof(p->args));
  int tiles = 0;
  for (int i = 0; i < count; ++i) {
    const imq_qmv_stage& st = stages[i];
    if (st.count < 1 || st.count > kMaxStageProblems) {
      free_stream(p);
      return fail(IMQ_EINVAL, "a stage has 1 to 3 problems");
    }
    SStage S;
    memset(&S, 0, sizeof(S));
    const imq_problem& q0 = st.problems[0];
    S.x = q0.x;
    S.K = q0.K;
    S.nprob = st.count;
    S.wait = st.wait_previous ? i - 1 : -1;
    if (S.wait >= 0) p->chained = true;
    if (i == 0 && st.wait_previous) {
      free_stream(p);
      return fail(IMQ_EINVAL, "the first stage has nothing to wait for");
    }
    if (q0.K < 64 || q0.K % 64 || q0.K > kMaxK) {
      free_stream(p);
      return fail(IMQ_EUNSUPPORTED, "the streaming engine takes K in 64 .. 10240, a multiple of 64");
    }
    S.sh = m1_lane_shift(q0.K);
    S.nch = ((q0.K / 32) + (1 << S.sh) - 1) >> S.sh;
    const int rows = 64 >> S.sh;
    int t = 0;
    for (int k = 0; k < st.count; ++k) {
      const imq_problem& q = st.problems[k];
      if (!q.w || !q.scales || !q.biases || !q.x || !q.y || !aligned(q.w, 16) ||
          !aligned(q.scales, 2) || !aligned(q.biases, 2) || !aligned(q.x, 16) ||
          !aligned(q.y, 2) || q.N < 1) {
        free_stream(p);
        return fail(IMQ_EINVAL, "bad pointer, alignment or shape in a stage");
      }
      if (q.x != q0.x || q.K != q0.K) {
        free_stream(p);
        return fail(IMQ_EINVAL, "the problems of a stage share one x");
      }
      if ((int64_t)q.N * (q.K / 2) >= ((int64_t)1 << 31)) {
        free_stream(p);
        return fail(IMQ_EUNSUPPORTED, "weights of 2 GiB or more");
      }
      SProb& P = S.p[k];
      P.w = q.w;
      P.s = q.scales;
      P.b = q.biases;
      P.y = static_cast<uint16_t*>(q.y);
      P.N = q.N;
      t += (q.N + rows - 1) / rows;
      P.tile_end = t;
    }
    S.tiles = t;
    S.first = tiles;
    tiles += t;
    p->stages.push_back(S);
  }
  for (SStage& S : p->stages)
    if (S.wait >= 0) p->stages[S.wait].signal = 1;
  // x rows that overlap an earlier stage's output are read with sc1 loads, and those
  // outputs are written with sc1 stores
  for (size_t i = 0; i < p->stages.size(); ++i) {
    SStage& S = p->stages[i];
    const uintptr_t x0 = reinterpret_cast<uintptr_t>(S.x), x1 = x0 + (uintptr_t)S.K * 2u;
    for (size_t e = 0; e < i; ++e)
      for (int k = 0; k < p->stages[e].nprob; ++k) {
        SProb& P = p->stages[e].p[k];
        const uintptr_t y0 = reinterpret_cast<uintptr_t>(P.y), y1 = y0 + (uintptr_t)P.N * 2u;
        if (x0 < y1 && y0 < x1) {
          S.x_live = 1;
          P.live = 1;
        }
      }
  }
  if (!p->chained) {
    for (const SStage& S : p->stages)
      if (S.x_live) {
        free_stream(p);
        return fail(IMQ_EINVAL, "a stage reads an output of the program but waits for nothing");
      }
    // every distinct x once in LDS
    int off = 0;
    for (SStage& S : p->stages) {
      int k = 0;
      while (k < p->args.nslots && p->args.slot[k].x != S.x) ++k;
      if (k == p->args.nslots) {
        if (k == kMaxSlots || off + x_bytes(S.K) > kSlotLds) {
          free_stream(p);
          return fail(IMQ_EUNSUPPORTED, "the distinct x rows of the program exceed 8 or 64 KiB of LDS");
        }
        p->args.slot[k] = XSlot{S.x, S.K, off};
        off += (int)((x_bytes(S.K) + 15) & ~(size_t)15);
        p->args.nslots = k + 1;
      } else if (p->args.slot[k].K != S.K) {
        free_stream(p);
        return fail(IMQ_EINVAL, "one x used with two different K");
      }
      S.xoff = p->args.slot[k].off;
    }
    p->args.sb_off = off;
  } else {
    // two x buffers (stages alternate), each sized for the program's largest K
    int kmax = 0;
    for (const SStage& S : p->stages) kmax = std::max(kmax, (int)S.K);
    const int xb = (int)((x_bytes(kmax) + 15) & ~(size_t)15);
    for (size_t i = 0; i < p->stages.size(); ++i) p->stages[i].xoff = (int)(i & 1) * xb;
    p->args.sb_off = 2 * xb;
  }
  p->lds = (size_t)p->args.sb_off + (size_t)kWaves * kSbWords * 4;
  const int nstages = (int)p->stages.size();
  p->counter_words = p->chained ? (int64_t)nstages * kSubs * kLine : 0;
  // the counters, the status word, and (each on a line of its own) the claim counters
  const size_t words = (size_t)(p->counter_words + kLine + kShards * kLine);
  if (hipMalloc(&p->d_words, words * 4) != hipSuccess || hipMemset(p->d_words, 0, words * 4) != hipSuccess) {
    free_stream(p);
    return fail(IMQ_ELAUNCH, "hipMalloc of the stream counters failed");
  }
  if (hipMalloc(&p->d_stages, sizeof(SStage) * nstages) != hipSuccess ||
      hipMemcpy(p->d_stages, p->stages.data(), sizeof(SStage) * nstages, hipMemcpyHostToDevice) !=
          hipSuccess) {
    free_stream(p);
    return fail(IMQ_ELAUNCH, "copying the stage table failed");
  }
  const void* fn = p->chained ? reinterpret_cast<const void*>(stream_chain_kernel)
                              : reinterpret_cast<const void*>(stream_kernel);
  if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)p->lds) != hipSuccess) {
    free_stream(p);
    return fail(IMQ_ELAUNCH, "cannot give the streaming kernel its LDS");
  }
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kThreads, p->lds) != hipSuccess ||
      per_cu < 1) {
    free_stream(p);
    return fail(IMQ_ELAUNCH, "the streaming kernel does not fit on a CU");
  }
  // chained stages need every workgroup resident at once (they wait for each other)
  const int resident = per_cu * dev->cu_count;
  int grid = workgroups > 0 ? workgroups : resident;
  if (p->chained) grid = std::min(grid, resident);
  grid = std::max(1, std::min(grid, (tiles + kWaves - 1) / kWaves));
  p->grid = grid;
  p->args.counters = p->d_words;
  p->args.status = p->d_words + p->counter_words;
  p->args.claim = p->d_words + p->counter_words + kLine;
  p->args.nstages = nstages;
  p->args.total = tiles;
  p->args.waves = grid * kWaves;
  if (!p->chained) {
    // runs of kRunTarget tiles or a little more, in whole rounds of one run per wavefront,
    // the last IMQ_STREAM_DYN_PERCENT of the rounds claimed from as many shards as there
    // are groups of kXcdSpread workgroups (up to kShards), each shard's tiles in runs of
    // IMQ_STREAM_DYN_RUN and its last IMQ_STREAM_TAIL_PERCENT in runs of
    // IMQ_STREAM_TAIL_RUN; and the problem of the first tile of every run
    const imq_runs::ShardPlan& plan = p->args.runs = imq_runs::plan_runs(
        tiles, grid, kWaves, kRunTarget, IMQ_STREAM_DYN_RUN, IMQ_STREAM_DYN_PERCENT,
        IMQ_STREAM_TAIL_RUN, IMQ_STREAM_TAIL_PERCENT, kXcdSpread);
    const imq_runs::RunPlan& P = plan.plan;
    const int nruns = P.runs;
    std::vector<int32_t> runs((size_t)nruns);
    int si = 0, pi = 0, shard = 0;
    for (int r = 0; r < nruns; ++r) {
      while (r >= P.static_runs && r >= plan.shard[shard].lo + plan.shard[shard].count) ++shard;
      const int g = P.start_of(r, plan.shard[shard]);
      while (g >= p->stages[si].first + p->stages[si].p[pi].tile_end) {
        if (pi + 1 < p->stages[si].nprob) {
          ++pi;
        } else {
          ++si;
          pi = 0;
        }
      }
      runs[(size_t)r] = (si << 2) | pi;
    }
    if (hipMalloc(&p->d_runs, sizeof(int32_t) * (size_t)nruns) != hipSuccess ||
        hipMemcpy(p->d_runs, runs.data(), sizeof(int32_t) * (size_t)nruns, hipMemcpyHostToDevice) !=
            hipSuccess) {
      free_stream(p);
      return fail(IMQ_ELAUNCH, "copying the run table failed");
    }
    p->args.run_site = p->d_runs;
  }
  *out = p;
  return ok();
}

int32_t imq_stream_launch(imq_stream* p, void* stream) {
  if (!p) return fail(IMQ_EINVAL, "null program");
  int dev = -1;
  (void)hipGetDevice(&dev);
  if (dev != p->device) return fail(IMQ_EINVAL, "the program belongs to another device");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (p->chained) {
    const int64_t n = p->counter_words;
    clear_kernel<<<(unsigned)((n + kThreads - 1) / kThreads), kThreads, 0, s>>>(p->d_words, n);
    stream_chain_kernel<<<p->grid, kThreads, p->lds, s>>>(p->d_stages, p->args);
  } else {
    stream_kernel<<<p->grid, kThreads, p->lds, s>>>(p->d_stages, p->args);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(IMQ_ELAUNCH, std::string("stream launch: ") + hipGetErrorString(e));
  return ok();
}

int32_t imq_stream_status(imq_stream* p, int32_t* failed) {
  if (!p || !failed) return fail(IMQ_EINVAL, "null argument");
  uint32_t v = 0;
  if (hipDeviceSynchronize() != hipSuccess ||
      hipMemcpy(&v, p->d_words + p->counter_words, 4, hipMemcpyDeviceToHost) != hipSuccess)
    return fail(IMQ_ELAUNCH, "reading the stream status failed");
  *failed = v != 0;
  if (v && hipMemset(p->d_words + p->counter_words, 0, 4) != hipSuccess)
    return fail(IMQ_ELAUNCH, "clearing the stream status failed");
  return ok();
}

int32_t imq_stream_trace(imq_stream* p, uint64_t* buffer, int64_t words) {
  if (!p) return fail(IMQ_EINVAL, "null program");
  if (!p->chained) return fail(IMQ_EUNSUPPORTED, "only chained programs record a stage trace");
  if (buffer && (!aligned(buffer, 8) || words < (int64_t)p->args.nstages * p->args.waves * 4))
    return fail(IMQ_EINVAL, "the trace needs stages * workgroups * wavefronts * 4 8-byte-aligned words");
  p->args.trace = buffer;
  return ok();
}

int32_t imq_stream_info(const imq_stream* p, int32_t* tiles, int32_t* stages, int32_t* workgroups,
                        int32_t* lds_bytes, int32_t* chained) {
  if (!p) return fail(IMQ_EINVAL, "null program");
  if (tiles) *tiles = p->args.total;
  if (stages) *stages = p->args.nstages;
  if (workgroups) *workgroups = p->grid;
  if (lds_bytes) *lds_bytes = (int32_t)p->lds;
  if (chained) *chained = p->chained ? 1 : 0;
  return ok();
}

void imq_stream_destroy(imq_stream* p) { free_stream(p); }

}  // extern "C"
