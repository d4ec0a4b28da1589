// Device helpers shared by the library's kernels (gfx950): bf16 conversions, the
// nibble-to-bf16 pair trick, dot2 chains, cross-lane sums, raw buffer loads and the
// device-coherent ("sc1") accesses used between workgroups of one launch.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace imq_dev {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));  // 4 bf16, the _1k MFMA operands

// Raw buffer resource over `bytes` bytes at `base` (gfx9 word 3: 32-bit data format).
// Every caller passes a value the whole wavefront agrees on; taking it through
// readfirstlane keeps the descriptor in scalar registers even when the value was loaded
// by a vector load (a descriptor in vector registers makes every buffer access a loop
// over the distinct descriptors of the lanes).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
  const uint64_t u = reinterpret_cast<uint64_t>(base);
  const uint64_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)u);
  const uint64_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(u >> 32));
  return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>((hi << 32) | lo), (short)0,
                                           (int)__builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}

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

// Eight natural-order bf16 values (x0..x7 in d.x..d.w) -> the pair order of nibble_pair,
// one v_perm_b32 per output word (selector bytes 0-3 pick the second operand's bytes,
// 4-7 the first's).
__device__ __forceinline__ uint4 pair_order(uint4 d) {
  uint4 p;
  p.x = __builtin_amdgcn_perm(d.z, d.x, 0x05040100u);  // (x0, x4)
  p.y = __builtin_amdgcn_perm(d.z, d.x, 0x07060302u);  // (x1, x5)
  p.z = __builtin_amdgcn_perm(d.w, d.y, 0x05040100u);  // (x2, x6)
  p.w = __builtin_amdgcn_perm(d.w, d.y, 0x07060302u);  // (x3, x7)
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

// The 32-row tile layout of an activation (row stride IMQ_LD_TILED: a row stride of 0): element (m, k) at element offset tile_elem(m, k).  Each 64-column group
// is 4 KB, and the 16 bytes lane (m, kb) of an MFMA kernel reads for k-step t of group g lie
// at byte (4 g + t) * 1024 + 16 (32 kb + m): a contiguous 1 KB per load instruction.
__host__ __device__ constexpr uint32_t tile_elem(uint32_t m, uint32_t k) {
  return ((((k >> 6) * 4 + ((k >> 3) & 3)) * 2 + ((k >> 5) & 1)) * 32 + m) * 8 + (k & 7);
}

constexpr uint32_t kPastBuffer = 0x80000000u;  // a buffer offset that reads as zero

// Lane shape of the one-row (M = 1) tile, shared by every kernel that computes it so
// that they all produce the same bits: LPR = 1 << shift lanes share a weight row and
// lane j takes the 16-byte chunks j, j + LPR, ... of it.  The fewest lanes (16, 32 or
// 64) that give each lane at most 5 chunks, else at most 8; -1 when even 64 lanes
// would need more than 8 (K > 16384).
__host__ __device__ inline int m1_lane_shift(int K) {
  const int C = K / 32;
  for (int cap = 5; cap <= 8; cap += 3)
    for (int sh = 4; sh <= 6; ++sh)
      if ((C + (1 << sh) - 1) >> sh <= cap) return sh;
  return -1;
}

// Decode attention's split of each (request, KV head) pair's keys: whole 64-key chunks per
// split, as many splits as it takes to give the launch about IMQ_ATTN_WORKGROUPS
// workgroups (at most one split per chunk).  Shared by every attention path so that they
// merge the same partials in the same order.  At 32 requests x 8 KV heads over 512 keys
// the fused attention launch measured 31.5 us at 4096 workgroups (one chunk per split),
// 28.1 at 2048, 22.6 at 1024 (three chunks per split) and 25.3 at 512; one request keeps
// a split per chunk at any of these.
#ifndef IMQ_ATTN_WORKGROUPS
#define IMQ_ATTN_WORKGROUPS 1024
#endif
__host__ inline void attention_splits(int B, int Hkv, int span, int* splits, int* chunks_per_split) {
  const int chunks = (span + 63) / 64;
  const int pairs = B * Hkv;
  int sp = (IMQ_ATTN_WORKGROUPS + pairs - 1) / pairs;
  sp = sp < chunks ? sp : chunks;
  sp = sp > 1 ? sp : 1;
  const int c = (chunks + sp - 1) / sp;
  *chunks_per_split = c;
  *splits = (chunks + c - 1) / c;
}

__device__ __forceinline__ uint4 load_b128(__amdgpu_buffer_rsrc_t rsrc, uint32_t off) {
  const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Loads of data read once per launch (streamed weights), with the nt (non-temporal)
// cache-policy bit: the lines are not kept for reuse, which measured 2-3% faster on the
// weight stream than the default policy.
constexpr int kNt = 2;  // cache-policy operand of the raw buffer intrinsics: nt
__device__ __forceinline__ uint4 load_b128_nt(__amdgpu_buffer_rsrc_t rsrc, uint32_t off) {
  const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, kNt);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// ------------------------------------------------------------------ wavefront sums

// v plus the value of lane l ^ 16 (l ^ 32) in every lane l, by the lane-swap instructions
// (no LDS round trip); the same sums as v + __shfl_xor(v, 16 / 32).
__device__ __forceinline__ float add_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_int(v), __float_as_int(v), false, false);
  return __int_as_float(r[0]) + __int_as_float(r[1]);
}
__device__ __forceinline__ float add_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false, false);
  return __int_as_float(r[0]) + __int_as_float(r[1]);
}
// The same with the larger of the two.
__device__ __forceinline__ float max_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_int(v), __float_as_int(v), false, false);
  return fmaxf(__int_as_float(r[0]), __int_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false, false);
  return fmaxf(__int_as_float(r[0]), __int_as_float(r[1]));
}

// Sum (max) over the wavefront, in every lane: each 16-lane row by DPP, then the four row
// results read from lanes 0, 16, 32 and 48 and combined as (r0 + r1) + (r2 + r3).  No LDS
// round trips (a __shfl_xor butterfly costs six of them in a chain).
__device__ __forceinline__ float lane_value(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  return (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp<0xB1>(v));
  v = fmaxf(v, dpp<0x4E>(v));
  v = fmaxf(v, dpp<0x141>(v));
  v = fmaxf(v, dpp<0x140>(v));
  return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)), fmaxf(lane_value(v, 32), lane_value(v, 48)));
}

// ------------------------------------------------ device-coherent accesses (sc1)
//
// Data that one workgroup writes and another reads within the same launch goes through
// accesses with the sc1 cache-policy bit: the form the compiler gives agent-scope relaxed
// atomic loads and stores on gfx950, so they are coherent across the XCDs' L2 caches
// without a cache write-back or invalidate.  A producer issues its sc1 stores, waits for
// them (s_waitcnt vmcnt(0)), then bumps a counter; a consumer that has seen the counter
// reads the data with sc1 loads.
constexpr int kSc1 = 16;  // cache-policy operand of the raw buffer intrinsics: sc1

__device__ __forceinline__ uint32_t ld_sc1(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_sc1(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ldf_sc1(const float* p) {
  return __uint_as_float(ld_sc1(reinterpret_cast<const uint32_t*>(p)));
}
__device__ __forceinline__ void stf_sc1(float* p, float v) {
  st_sc1(reinterpret_cast<uint32_t*>(p), __float_as_uint(v));
}
__device__ __forceinline__ uint4 load_b128_sc1(__amdgpu_buffer_rsrc_t rsrc, uint32_t off) {
  const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, kSc1);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint32_t load_b32_sc1(__amdgpu_buffer_rsrc_t rsrc, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(rsrc, off, 0, kSc1);
}
__device__ __forceinline__ void store_b16_sc1(__amdgpu_buffer_rsrc_t rsrc, uint32_t off, uint16_t v) {
  __builtin_amdgcn_raw_buffer_store_b16(v, rsrc, off, 0, kSc1);
}
__device__ __forceinline__ void store_b32_sc1(__amdgpu_buffer_rsrc_t rsrc, uint32_t off, uint32_t v) {
  __builtin_amdgcn_raw_buffer_store_b32(v, rsrc, off, 0, kSc1);
}
__device__ __forceinline__ void store_b128_sc1(__amdgpu_buffer_rsrc_t rsrc, uint32_t off, uint4 v) {
  const u32x4_t t = {v.x, v.y, v.z, v.w};
  __builtin_amdgcn_raw_buffer_store_b128(t, rsrc, off, 0, kSc1);
}
// Waits until every vector memory access this thread issued has completed.
__device__ __forceinline__ void wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

}  // namespace imq_dev
