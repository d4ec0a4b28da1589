// MI355X (gfx950) kernels for the decode step around the 4-bit projections, and their C
// ABI (include/ironmule_decode.h): embedding rows, residual add + RMSNorm, per-head
// q/k norm + rotary embedding + KV write, grouped-query decode attention, SiLU * up.
//
// All of them are small next to the weight stream; they are written to keep every
// launch to one pass over its data with coalesced 16-byte accesses where the data is
// large (the KV chunks), and to be deterministic (fixed reduction orders).

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <string>

#include "../../include/ironmule_decode.h"
#include "common.h"
#include "runtime.h"

namespace {

using namespace imq_dev;

using imq_rt::aligned;
using imq_rt::current_device;
using imq_rt::fail;
using imq_rt::ok;

constexpr int kThreads = 256;
constexpr int kD = IMQ_HEAD_DIM;  // head dimension
constexpr int kChunk = 64;        // keys per attention workgroup
constexpr int kMaxNormDim = 8192;
constexpr int kNormVpt = kMaxNormDim / kThreads;  // values per thread of the row norm

__device__ __forceinline__ float bf(uint32_t h) { return bf16_bits_to_f32(h); }
__device__ __forceinline__ uint16_t to_bf(float f) { return f32_to_bf16_bits(f); }

// ------------------------------------------------------------------ embedding rows

// One thread per packed word (8 values) of row tokens[b]: fp32 s * q + b.
__global__ __launch_bounds__(kThreads) void embed_kernel(const uint32_t* __restrict__ w,
                                                         const uint16_t* __restrict__ s,
                                                         const uint16_t* __restrict__ b,
                                                         const int32_t* __restrict__ tokens,
                                                         float* __restrict__ h, int vocab, int dim) {
  const int row = blockIdx.y;
  const int W = dim >> 3;
  const int word = blockIdx.x * kThreads + threadIdx.x;
  if (word >= W) return;
  const int t = tokens[row];
  float* out = h + (size_t)row * dim + (size_t)word * 8;
  if (t < 0 || t >= vocab) {
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = __uint_as_float(0x7fc00000u);
    return;
  }
  const uint32_t u = w[(size_t)t * W + word];
  const size_t g = (size_t)t * (dim >> 6) + ((word * 8) >> 6);
  const float sc = bf(s[g]), bi = bf(b[g]);
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = fmaf(sc, (float)((u >> (4 * e)) & 0xFu), bi);
  reinterpret_cast<float4*>(out)[0] = make_float4(v[0], v[1], v[2], v[3]);
  reinterpret_cast<float4*>(out)[1] = make_float4(v[4], v[5], v[6], v[7]);
}

// ------------------------------------------------------- residual add + RMSNorm

// One workgroup per row.  Thread t holds values t, t + 256, ... (VPT of them).  Every
// load is issued before the first is used (indices past the row are clamped to its last
// value and masked), so the row costs one memory round trip.  The sum of squares is added
// per thread, then over each wavefront (butterfly), then over the four wavefronts in
// order, so the result does not depend on scheduling.
//
// PRE (the RMSNorm folded into the next projection): out = bf16(h * weight), unnormalised,
// and ssq[row * ld] = the row's sum of squares, from which that projection scales its
// output rows.
template <int VPT, bool PRE = false>
__global__ __launch_bounds__(kThreads) void add_rmsnorm_kernel(float* __restrict__ h,
                                                               const uint16_t* __restrict__ delta,
                                                               const uint16_t* __restrict__ weight,
                                                               uint16_t* __restrict__ out, int dim,
                                                               float eps, float* __restrict__ ssq = nullptr,
                                                               int ld = 0) {
  __shared__ float red[kThreads / 64];
  const int row = blockIdx.x, tid = threadIdx.x;
  float* hr = h + (size_t)row * dim;
  const uint16_t* dr = delta ? delta + (size_t)row * dim : nullptr;
  float v[VPT];
  uint32_t d[VPT], wv[VPT];
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int idx = min(tid + kThreads * i, dim - 1);
    v[i] = hr[idx];
    d[i] = dr ? dr[idx] : 0u;
    wv[i] = weight[idx];
  }
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int idx = tid + kThreads * i;
    if (dr) v[i] += bf(d[i]);
    if (idx < dim) {
      if (dr) hr[idx] = v[i];
      ss = fmaf(v[i], v[i], ss);
    }
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  const float total = (red[0] + red[1]) + (red[2] + red[3]);
  const float inv = PRE ? 1.0f : 1.0f / sqrtf(total / (float)dim + eps);
  if (PRE && tid == 0) ssq[(size_t)row * ld] = total;
  uint16_t* orow = out + (size_t)row * dim;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int idx = tid + kThreads * i;
    if (idx < dim) orow[idx] = to_bf(PRE ? v[i] * bf(wv[i]) : v[i] * inv * bf(wv[i]));
  }
}

// ------------------------------------------- q/k norm + rotary embedding + KV write

// One wavefront per (request, head) of q, k or v.  Lane i holds dimensions i and i + 64:
// exactly the pair the non-interleaved rotary embedding mixes.
__global__ __launch_bounds__(64) void qk_norm_rope_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const uint16_t* __restrict__ q_norm, const uint16_t* __restrict__ k_norm,
    const int32_t* __restrict__ positions, const int32_t* __restrict__ slots,
    uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_pool, uint16_t* __restrict__ v_pool,
    int Hq, int Hkv, int capacity, int num_slots, float log2_theta, float eps) {
  const int b = blockIdx.x, hh = blockIdx.y, lane = threadIdx.x;
  const int pos = positions[b], slot = slots[b];
  if (pos < 0 || pos >= capacity || slot < 0 || slot >= num_slots) return;  // refused
  const bool is_q = hh < Hq, is_k = !is_q && hh < Hq + Hkv;
  const int head = is_q ? hh : (is_k ? hh - Hq : hh - Hq - Hkv);
  const uint16_t* src = is_q ? q + ((size_t)b * Hq + head) * kD
                             : (is_k ? k : v) + ((size_t)b * Hkv + head) * kD;
  float x0 = bf(src[lane]), x1 = bf(src[lane + 64]);
  if (is_q || is_k) {
    const uint16_t* nw = is_q ? q_norm : k_norm;
    const float ss = wave_sum(fmaf(x0, x0, x1 * x1));
    const float inv = 1.0f / sqrtf(ss / (float)kD + eps);
    // the norm module's output is bf16 in the reference, and the rotation reads it
    x0 = bf(to_bf(x0 * inv * bf(nw[lane])));
    x1 = bf(to_bf(x1 * inv * bf(nw[lane + 64])));
    // angle = pos * theta^(-i / 64) for the pair (i, i + 64)
    const float inv_freq = exp2f(-(float)lane * (log2_theta / 64.0f));
    float sn, cs;
    sincosf((float)pos * inv_freq, &sn, &cs);
    const float r0 = x0 * cs - x1 * sn;
    const float r1 = x0 * sn + x1 * cs;
    x0 = r0;
    x1 = r1;
  }
  uint16_t* dst = is_q ? q_out + ((size_t)b * Hq + head) * kD
                       : (is_k ? k_pool : v_pool) +
                             (((size_t)slot * Hkv + head) * capacity + pos) * kD;
  dst[lane] = to_bf(x0);
  dst[lane + 64] = to_bf(x1);
}

// ------------------------------------------------------------ decode attention
//
// Two launches, no communication between workgroups inside either.
//
// attention_partial_kernel: workgroup (split s, KV head, request b) walks its share of
// the request's keys in 64-key chunks (the next chunk's loads in flight while one
// computes) and serves the G query heads that read that KV head (one wavefront per head,
// G <= 8, their q staged in LDS once).  Per chunk, lane t scores key t (64 bf16 dot2
// against the head's q), the chunk max and sum come from butterflies, lane i accumulates
// dimensions 2i, 2i+1 of p . V, and the chunk is merged into the running (max, sum, acc)
// of the split.  The split's partial goes to the workspace.
//
// attention_combine_kernel: one wavefront per (request, query head) merges the splits in
// split order and writes the bf16 head.  Both orders are fixed, so results do not depend
// on scheduling.

constexpr int kMergeBatch = 16;  // splits whose partials a merge loads at once
constexpr uint32_t kNegZeroPair = 0x80008000u;  // the bf16 pair (-0, -0)

struct AttnLds {
  uint4 k[kChunk][17];        // a key row is 16 uint4; one of padding keeps lanes on
                              // distinct banks when lane t reads row t
  uint32_t v[kChunk][kD / 2];  // lane i reads dword i of a row: conflict-free
  float p[4][kChunk];
  uint4 q[8][kD / 8];         // the workgroup's query heads (read as broadcasts)
};

struct AttnGeometry {
  int len;    // keys to attend over (0: none)
  int slot;
};

__device__ __forceinline__ AttnGeometry attn_geometry(const int32_t* lengths, const int32_t* slots,
                                                      int b, int max_len, int capacity,
                                                      int num_slots) {
  AttnGeometry g;
  g.slot = slots[b];
  int len = lengths[b];
  len = len < max_len ? len : max_len;
  len = len < capacity ? len : capacity;
  g.len = (g.slot < 0 || g.slot >= num_slots || len < 0) ? 0 : len;
  return g;
}

__global__ __launch_bounds__(kThreads) void attention_partial_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k_pool,
    const uint16_t* __restrict__ v_pool, const int32_t* __restrict__ lengths,
    const int32_t* __restrict__ slots, int Hq, int Hkv, int capacity, int max_len, int num_slots,
    float scale, int chunks_per_split, int splits, float* __restrict__ part,
    float* __restrict__ ml) {
  __shared__ AttnLds L;
  const int s = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int G = Hq / Hkv;
  const AttnGeometry geo = attn_geometry(lengths, slots, b, max_len, capacity, num_slots);
  const int first = s * chunks_per_split * kChunk;
  if (first >= geo.len) return;  // the combine skips this split
  const int last = min(geo.len, first + chunks_per_split * kChunk);
  const size_t base = (((size_t)geo.slot * Hkv + kvh) * capacity) * kD;

  // q of this wavefront's heads, as bf16 pairs (uniform across the wavefront)
  float M[2] = {-INFINITY, -INFINITY}, Ls[2] = {0.0f, 0.0f};
  float a0[2] = {0.0f, 0.0f}, a1[2] = {0.0f, 0.0f};

  // The chunk's K and V rows, four 16-byte pieces each per thread, in named registers (an
  // array filled through a reference would be kept in scratch memory).  Rows past `last`
  // read row last-1, which stays inside the slot.
  const uint4* kb = reinterpret_cast<const uint4*>(k_pool + base);
  const uint4* vb = reinterpret_cast<const uint4*>(v_pool + base);
  auto piece = [&](int start, int i) {
    const int p = tid + kThreads * i;
    const int t = start + (p >> 4) < last ? start + (p >> 4) : last - 1;
    return (size_t)t * (kD / 8) + (p & 15);
  };
  uint4 k0 = kb[piece(first, 0)], k1 = kb[piece(first, 1)], k2 = kb[piece(first, 2)],
        k3 = kb[piece(first, 3)];
  uint4 v0 = vb[piece(first, 0)], v1 = vb[piece(first, 1)], v2 = vb[piece(first, 2)],
        v3 = vb[piece(first, 3)];
  // the G query heads of this KV head, once (the loop's first barrier publishes them)
  if (tid < G * (kD / 8))
    L.q[tid / (kD / 8)][tid % (kD / 8)] =
        reinterpret_cast<const uint4*>(q + ((size_t)b * Hq + kvh * G) * kD)[tid];
  for (int start = first; start < last; start += kChunk) {
    const int count = min(kChunk, last - start);
    __syncthreads();  // the previous chunk's readers are done
    {
      const uint4 kr[4] = {k0, k1, k2, k3}, vr[4] = {v0, v1, v2, v3};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int p = tid + kThreads * i;
        const int row = p >> 4, col = p & 15;
        L.k[row][col] = kr[i];
        // rows past the chunk's keys hold -0: their weight p is +0, so each adds -0,
        // which leaves any sum unchanged (the value loop then needs no bound)
        const uint32_t z = start + row < last ? 0u : kNegZeroPair, keep = start + row < last ? ~0u : 0u;
        *reinterpret_cast<uint4*>(&L.v[row][col * 4]) =
            make_uint4((vr[i].x & keep) | z, (vr[i].y & keep) | z, (vr[i].z & keep) | z, (vr[i].w & keep) | z);
      }
    }
    __syncthreads();
    if (start + kChunk < last) {  // next chunk in flight
      k0 = kb[piece(start + kChunk, 0)];
      k1 = kb[piece(start + kChunk, 1)];
      k2 = kb[piece(start + kChunk, 2)];
      k3 = kb[piece(start + kChunk, 3)];
      v0 = vb[piece(start + kChunk, 0)];
      v1 = vb[piece(start + kChunk, 1)];
      v2 = vb[piece(start + kChunk, 2)];
      v3 = vb[piece(start + kChunk, 3)];
    }

#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int g = wave + 4 * r;
      if (g >= G) break;
      float sc = -INFINITY;
      if (lane < count) {
        float d = 0.0f;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const uint4 a = L.q[g][j], kk = L.k[lane][j];
          d = dot2(a.x, kk.x, d);
          d = dot2(a.y, kk.y, d);
          d = dot2(a.z, kk.z, d);
          d = dot2(a.w, kk.w, d);
        }
        sc = d * scale;
      }
      const float mc = wave_max(sc);
      const float p = lane < count ? expf(sc - mc) : 0.0f;
      const float lc = wave_sum(p);
      L.p[wave][lane] = p;
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      float c0 = 0.0f, c1 = 0.0f;
#pragma unroll
      for (int t = 0; t < kChunk; ++t) {  // t >= count: p = +0 times -0
        const float pt = L.p[wave][t];
        const uint32_t vd = L.v[t][lane];
        c0 = fmaf(pt, bf(vd & 0xffffu), c0);
        c1 = fmaf(pt, bf(vd >> 16), c1);
      }
      __builtin_amdgcn_wave_barrier();  // L.p is rewritten by this wave's next head
      // merge the chunk into the split's running result
      const float mn = fmaxf(M[r], mc);
      const float eo = expf(M[r] - mn), ec = expf(mc - mn);
      Ls[r] = fmaf(Ls[r], eo, lc * ec);
      a0[r] = fmaf(a0[r], eo, c0 * ec);
      a1[r] = fmaf(a1[r], eo, c1 * ec);
      M[r] = mn;
    }
  }
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int g = wave + 4 * r;
    if (g >= G) break;
    const size_t po = ((size_t)b * Hq + kvh * G + g) * splits + s;
    reinterpret_cast<float2*>(part + po * kD)[lane] = make_float2(a0[r], a1[r]);
    if (lane == 0) reinterpret_cast<float2*>(ml)[po] = make_float2(M[r], Ls[r]);
  }
}

__global__ __launch_bounds__(64) void attention_combine_kernel(
    const int32_t* __restrict__ lengths, const int32_t* __restrict__ slots,
    uint16_t* __restrict__ out, int Hq, int capacity, int max_len, int num_slots,
    int chunks_per_split, int splits, const float* __restrict__ part, const float* __restrict__ ml) {
  const int h = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
  const AttnGeometry geo = attn_geometry(lengths, slots, b, max_len, capacity, num_slots);
  uint16_t* o = out + ((size_t)b * Hq + h) * kD;
  const int used = (geo.len + chunks_per_split * kChunk - 1) / (chunks_per_split * kChunk);
  if (used == 0) {  // nothing to attend to: zeros
    o[2 * lane] = 0;
    o[2 * lane + 1] = 0;
    return;
  }
  const size_t p0 = ((size_t)b * Hq + h) * splits;
  // the partials of kMergeBatch splits are loaded together before any is used (all of them
  // in one round when they fit); the arithmetic runs in split order
  if (used <= kMergeBatch) {
    float2 mlq[kMergeBatch], pq[kMergeBatch];
#pragma unroll
    for (int q = 0; q < kMergeBatch; ++q) {
      const size_t sq = p0 + (q < used ? q : 0);
      mlq[q] = reinterpret_cast<const float2*>(ml)[sq];
      pq[q] = reinterpret_cast<const float2*>(part + sq * kD)[lane];
    }
    float M = -INFINITY;
#pragma unroll
    for (int q = 0; q < kMergeBatch; ++q)
      if (q < used) M = fmaxf(M, mlq[q].x);
    float Ls = 0.0f, a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int q = 0; q < kMergeBatch; ++q) {
      if (q < used) {
        const float e = expf(mlq[q].x - M);
        Ls = fmaf(mlq[q].y, e, Ls);
        a0 = fmaf(pq[q].x, e, a0);
        a1 = fmaf(pq[q].y, e, a1);
      }
    }
    o[2 * lane] = to_bf(a0 / Ls);
    o[2 * lane + 1] = to_bf(a1 / Ls);
    return;
  }
  float M = -INFINITY;
  for (int s0 = 0; s0 < used; s0 += kMergeBatch) {
    float mv[kMergeBatch];
#pragma unroll
    for (int q = 0; q < kMergeBatch; ++q) mv[q] = s0 + q < used ? ml[2 * (p0 + s0 + q)] : -INFINITY;
#pragma unroll
    for (int q = 0; q < kMergeBatch; ++q) M = fmaxf(M, mv[q]);
  }
  float Ls = 0.0f, a0 = 0.0f, a1 = 0.0f;
  for (int s0 = 0; s0 < used; s0 += kMergeBatch) {
    float2 mlq[kMergeBatch], pq[kMergeBatch];
#pragma unroll
    for (int q = 0; q < kMergeBatch; ++q) {
      const size_t sq = p0 + (s0 + q < used ? s0 + q : s0);
      mlq[q] = reinterpret_cast<const float2*>(ml)[sq];
      pq[q] = reinterpret_cast<const float2*>(part + sq * kD)[lane];
    }
#pragma unroll
    for (int q = 0; q < kMergeBatch; ++q) {
      if (s0 + q < used) {
        const float e = expf(mlq[q].x - M);
        Ls = fmaf(mlq[q].y, e, Ls);
        a0 = fmaf(pq[q].x, e, a0);
        a1 = fmaf(pq[q].y, e, a1);
      }
    }
  }
  o[2 * lane] = to_bf(a0 / Ls);
  o[2 * lane + 1] = to_bf(a1 / Ls);
}

// ------------------------------------------------------------------ SiLU * up

__global__ __launch_bounds__(kThreads) void silu_mul_kernel(const uint16_t* __restrict__ gate,
                                                            const uint16_t* __restrict__ up,
                                                            uint16_t* __restrict__ out, int64_t n) {
  const int64_t i8 = ((int64_t)blockIdx.x * kThreads + threadIdx.x) * 8;
  if (i8 >= n) return;
  if (i8 + 8 <= n) {
    const uint4 g = *reinterpret_cast<const uint4*>(gate + i8);
    const uint4 u = *reinterpret_cast<const uint4*>(up + i8);
    const uint32_t gw[4] = {g.x, g.y, g.z, g.w}, uw[4] = {u.x, u.y, u.z, u.w};
    uint32_t r[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float g0 = bf(gw[e] & 0xffffu), g1 = bf(gw[e] >> 16);
      const float o0 = g0 / (1.0f + expf(-g0)) * bf(uw[e] & 0xffffu);
      const float o1 = g1 / (1.0f + expf(-g1)) * bf(uw[e] >> 16);
      r[e] = (uint32_t)to_bf(o0) | ((uint32_t)to_bf(o1) << 16);
    }
    *reinterpret_cast<uint4*>(out + i8) = make_uint4(r[0], r[1], r[2], r[3]);
  } else {
    for (int64_t i = i8; i < n; ++i) {
      const float g0 = bf(gate[i]);
      out[i] = to_bf(g0 / (1.0f + expf(-g0)) * bf(up[i]));
    }
  }
}

int32_t launched(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(IMQ_ELAUNCH, std::string(what) + " launch failed: " + hipGetErrorString(e));
  return ok();
}

// Splits per (request, KV head): attention_splits (common.h).
struct AttnPlan {
  int splits;
  int chunks_per_split;
};

AttnPlan attention_plan(int32_t B, int32_t Hkv, int32_t span) {
  static_assert(kChunk == 64, "attention_splits counts 64-key chunks");
  AttnPlan pl;
  attention_splits(B, Hkv, span, &pl.splits, &pl.chunks_per_split);
  return pl;
}

}  // namespace

// ==================================================================== C ABI

extern "C" {

int32_t imq_embed(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                  const int32_t* tokens, float* h, int32_t B, int32_t vocab, int32_t dim,
                  void* stream) {
  if (!w || !scales || !biases || !tokens || !h) return fail(IMQ_EINVAL, "null pointer");
  if (B < 1 || vocab < 1) return fail(IMQ_EINVAL, "B and vocab must be >= 1");
  if (dim < 64 || dim % 64) return fail(IMQ_EINVAL, "dim must be a positive multiple of 64");
  if (!aligned(w, 4) || !aligned(h, 16)) return fail(IMQ_EINVAL, "w or h is misaligned");
  int32_t code;
  if (!current_device(&code)) return code;
  const int W = dim / 8;
  hipLaunchKernelGGL(embed_kernel, dim3((W + kThreads - 1) / kThreads, B), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), w, scales, biases, tokens, h, vocab, dim);
  return launched("embed");
}

int32_t imq_add_rmsnorm(float* h, const uint16_t* delta, const uint16_t* weight, uint16_t* out,
                        int32_t B, int32_t dim, float eps, void* stream) {
  if (!h || !weight || !out) return fail(IMQ_EINVAL, "null pointer");
  if (B < 1 || dim < 1 || dim > kMaxNormDim) return fail(IMQ_EINVAL, "B >= 1 and 1 <= dim <= 8192");
  if (!(eps >= 0.0f)) return fail(IMQ_EINVAL, "eps must be >= 0");
  int32_t code;
  if (!current_device(&code)) return code;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int vpt = (dim + kThreads - 1) / kThreads;
  if (vpt <= 4)
    hipLaunchKernelGGL(add_rmsnorm_kernel<4>, dim3(B), dim3(kThreads), 0, st, h, delta, weight, out, dim, eps);
  else if (vpt <= 10)
    hipLaunchKernelGGL(add_rmsnorm_kernel<10>, dim3(B), dim3(kThreads), 0, st, h, delta, weight, out, dim, eps);
  else if (vpt <= 16)
    hipLaunchKernelGGL(add_rmsnorm_kernel<16>, dim3(B), dim3(kThreads), 0, st, h, delta, weight, out, dim, eps);
  else
    hipLaunchKernelGGL(add_rmsnorm_kernel<kNormVpt>, dim3(B), dim3(kThreads), 0, st, h, delta, weight, out, dim, eps);
  return launched("add_rmsnorm");
}

int32_t imq_rmsnorm_prescale(float* h, const uint16_t* delta, const uint16_t* weight, uint16_t* out,
                             float* ssq, int32_t ld, int32_t B, int32_t dim, void* stream) {
  if (!h || !weight || !out || !ssq) return fail(IMQ_EINVAL, "null pointer");
  if (B < 1 || dim < 1 || dim > kMaxNormDim) return fail(IMQ_EINVAL, "B >= 1 and 1 <= dim <= 8192");
  if (ld < 4 || ld % 4 || !aligned(ssq, 16)) return fail(IMQ_EINVAL, "ssq must be 16-byte aligned, ld a multiple of 4");
  int32_t code;
  if (!current_device(&code)) return code;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int vpt = (dim + kThreads - 1) / kThreads;
  if (vpt <= 4)
    hipLaunchKernelGGL((add_rmsnorm_kernel<4, true>), dim3(B), dim3(kThreads), 0, st, h, delta, weight, out, dim, 0.0f, ssq, ld);
  else if (vpt <= 10)
    hipLaunchKernelGGL((add_rmsnorm_kernel<10, true>), dim3(B), dim3(kThreads), 0, st, h, delta, weight, out, dim, 0.0f, ssq, ld);
  else if (vpt <= 16)
    hipLaunchKernelGGL((add_rmsnorm_kernel<16, true>), dim3(B), dim3(kThreads), 0, st, h, delta, weight, out, dim, 0.0f, ssq, ld);
  else
    hipLaunchKernelGGL((add_rmsnorm_kernel<kNormVpt, true>), dim3(B), dim3(kThreads), 0, st, h, delta, weight, out, dim, 0.0f, ssq, ld);
  return launched("rmsnorm_prescale");
}

int32_t imq_qk_norm_rope(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                         const uint16_t* q_norm, const uint16_t* k_norm, const int32_t* positions,
                         const int32_t* slots, uint16_t* q_out, uint16_t* k_pool, uint16_t* v_pool,
                         int32_t B, int32_t Hq, int32_t Hkv, int32_t capacity, int32_t num_slots,
                         float theta, float eps, void* stream) {
  if (!q || !k || !v || !q_norm || !k_norm || !positions || !slots || !q_out || !k_pool || !v_pool)
    return fail(IMQ_EINVAL, "null pointer");
  if (B < 1 || Hq < 1 || Hkv < 1 || Hq % Hkv) return fail(IMQ_EINVAL, "need B, Hkv >= 1 and Hkv | Hq");
  if (capacity < 1 || num_slots < 1) return fail(IMQ_EINVAL, "capacity and num_slots must be >= 1");
  if (!(theta > 1.0f)) return fail(IMQ_EINVAL, "theta must be > 1");
  int32_t code;
  if (!current_device(&code)) return code;
  hipLaunchKernelGGL(qk_norm_rope_kernel, dim3(B, Hq + 2 * Hkv), dim3(64), 0,
                     static_cast<hipStream_t>(stream), q, k, v, q_norm, k_norm, positions, slots,
                     q_out, k_pool, v_pool, Hq, Hkv, capacity, num_slots, log2f(theta), eps);
  return launched("qk_norm_rope");
}

size_t imq_attention_workspace(int32_t B, int32_t Hq, int32_t max_len) {
  if (B < 1 || Hq < 1 || max_len < 1) return 0;
  const size_t chunks = (size_t)((max_len + kChunk - 1) / kChunk);  // splits <= chunks
  return (size_t)B * Hq * chunks * (kD + 2) * sizeof(float);
}

int32_t imq_attention_decode(const uint16_t* q, const uint16_t* k_pool, const uint16_t* v_pool,
                             const int32_t* lengths, const int32_t* slots, uint16_t* out, int32_t B,
                             int32_t Hq, int32_t Hkv, int32_t capacity, int32_t num_slots,
                             int32_t max_len, float scale, float* workspace, void* stream) {
  if (!q || !k_pool || !v_pool || !lengths || !slots || !out || !workspace)
    return fail(IMQ_EINVAL, "null pointer");
  if (B < 1 || Hq < 1 || Hkv < 1 || Hq % Hkv || Hq / Hkv > 8)
    return fail(IMQ_EINVAL, "need Hkv | Hq with at most 8 query heads per KV head");
  if (capacity < 1 || num_slots < 1 || max_len < 1) return fail(IMQ_EINVAL, "capacity, num_slots, max_len >= 1");
  if (!aligned(q, 16) || !aligned(k_pool, 16) || !aligned(v_pool, 16) || !aligned(workspace, 16))
    return fail(IMQ_EINVAL, "q, pools and workspace must be 16-byte aligned");
  if (B > 65535 || Hkv > 65535 || Hq > 65535) return fail(IMQ_EINVAL, "B and the head counts must be <= 65535");
  int32_t code;
  if (!current_device(&code)) return code;
  const int32_t span = max_len < capacity ? max_len : capacity;
  const AttnPlan pl = attention_plan(B, Hkv, span);
  float* part = workspace;
  float* mlp = workspace + (size_t)B * Hq * pl.splits * kD;
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(attention_partial_kernel, dim3(pl.splits, Hkv, B), dim3(kThreads), 0, st, q,
                     k_pool, v_pool, lengths, slots, Hq, Hkv, capacity, span, num_slots, scale,
                     pl.chunks_per_split, pl.splits, part, mlp);
  if ((code = launched("attention")) != IMQ_OK) return code;
  hipLaunchKernelGGL(attention_combine_kernel, dim3(Hq, B), dim3(64), 0, st, lengths, slots, out,
                     Hq, capacity, span, num_slots, pl.chunks_per_split, pl.splits, part, mlp);
  return launched("attention combine");
}

int32_t imq_silu_mul(const uint16_t* gate, const uint16_t* up, uint16_t* out, int64_t n,
                     void* stream) {
  if (!gate || !up || !out) return fail(IMQ_EINVAL, "null pointer");
  if (n < 1) return fail(IMQ_EINVAL, "n must be >= 1");
  if (!aligned(gate, 16) || !aligned(up, 16) || !aligned(out, 16))
    return fail(IMQ_EINVAL, "gate, up and out must be 16-byte aligned");
  int32_t code;
  if (!current_device(&code)) return code;
  const int64_t threads = (n + 7) / 8;
  const int64_t blocks = (threads + kThreads - 1) / kThreads;
  if (blocks > 0x7fffffff) return fail(IMQ_EINVAL, "n too large");
  hipLaunchKernelGGL(silu_mul_kernel, dim3((uint32_t)blocks), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), gate, up, out, n);
  return launched("silu_mul");
}

}  // extern "C"
