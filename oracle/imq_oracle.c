/*
 * CPU oracle for the affine, group-quantised 4-bit matrix-vector product (qmv).
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product links, loads or calls this
 * file: only the tests, the smoke check and the bench's CPU-baseline leg do, and
 * only as the checker (or as the timed CPU baseline), never as the thing that is
 * measured on the GPU or shipped.
 *
 * Format (pinned by the reference's code):
 *   w       uint32 (N, K/8): eight 4-bit values per word, LOW NIBBLE FIRST, so
 *           element j of word u is (u >> 4j) & 0xF
 *           (ironmule/cuda_native.py:54-56, 91; masks in ironmule/qmv_k3840.py:103-106)
 *   scales  bf16 (N, K/gs), biases bf16 (N, K/gs), gs = 64 on the path
 *           (ironmule/qmv_k3840.py:379-408)
 *   weight  w[n][k] = scale * q + bias  (ironmule/numeric_plans.py:450-452,
 *           ironmule/cuda_native.py:265-266)
 *   x       bf16 (M, K); y bf16 or fp32 (M, N).
 *
 * Functions, each with the reference lines it restates:
 *   imo_bf16_to_f32      widening by a 16-bit shift (cuda_native.py:43-45)
 *   imo_f32_to_bf16      round-to-nearest-even, NaN -> 0x7fc0 (cuda_native.py:46-51)
 *   imo_unpack           low-nibble-first unpack (cuda_native.py:91)
 *   imo_dequant_f32      fl32(s*q + b) with fp32 s, b (cuda_native.py:265;
 *                        numeric_plans.py:462-464).  s*q is exact in fp32 (an
 *                        8-bit mantissa times a 4-bit integer), so only the add
 *                        rounds and the result does not depend on FMA use.
 *   imo_qmv_dequant_f32  fp32 dequantise-then-matmul, the parity reference of
 *                        cuda_native.py:265-268: fp32 weights, then an fp32 fma
 *                        chain in increasing k order (MLX's own matmul order is
 *                        not recoverable here).
 *   imo_qmv_f64          the same product in fp64, plus sum_k |w*x| per output,
 *                        which bounds every fp32 summation order's error.
 *   imo_qmv_rowkernel    the reference CUDA row kernel's exact arithmetic
 *                        (cuda_native.py:57-128): per lane c = lane, lane+32, ...
 *                        over 32-value chunks, sx and qx chains, acc +=
 *                        fma(s, qx, b*sx), shuffle-down tree, RNE to bf16.
 *   imo_qmv_mlx          the reference Metal kernels' arithmetic order
 *                        (qmv_k3840.py:62-244 for 8 values per lane;
 *                        qmv_fast_shared.py:30-131 for 16): prescaled x, masked
 *                        nibbles, result += s*accum + sum*b per block, then a
 *                        32-lane reduction.  Two details are Metal's own and are
 *                        NOT pinned here: whether x[i]+x[i+1]+.. adds in bfloat
 *                        (done in fp32 here) and simd_sum's tree order (a xor
 *                        butterfly here).  Contraction is off, as in MLX's
 *                        "safe" math mode.
 *
 * Build: oracle/Makefile (gcc -O3 -fopenmp -ffp-contract=off).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define IMO_EXPORT __attribute__((visibility("default")))

/* ---------------------------------------------------------------- bf16 -- */

IMO_EXPORT float imo_bf16_to_f32(uint16_t h) {
  uint32_t u = ((uint32_t)h) << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

IMO_EXPORT uint16_t imo_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

IMO_EXPORT void imo_f32_to_bf16_array(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = imo_f32_to_bf16(in[i]);
}

IMO_EXPORT void imo_bf16_to_f32_array(const uint16_t* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = imo_bf16_to_f32(in[i]);
}

/* ------------------------------------------------------- unpack/dequant -- */

IMO_EXPORT void imo_unpack(const uint32_t* w, uint8_t* q, int64_t n_words) {
  for (int64_t i = 0; i < n_words; ++i) {
    uint32_t u = w[i];
    for (int j = 0; j < 8; ++j) q[i * 8 + j] = (uint8_t)((u >> (4 * j)) & 0xFu);
  }
}

static inline uint32_t nibble(const uint32_t* row, int64_t k) {
  return (row[k >> 3] >> (4 * (k & 7))) & 0xFu;
}

IMO_EXPORT void imo_dequant_f32(const uint32_t* w, const uint16_t* s, const uint16_t* b,
                                float* out, int64_t N, int64_t K, int32_t gs) {
  const int64_t G = K / gs;
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < N; ++n) {
    const uint32_t* row = w + n * (K / 8);
    for (int64_t k = 0; k < K; ++k) {
      const float sc = imo_bf16_to_f32(s[n * G + k / gs]);
      const float bi = imo_bf16_to_f32(b[n * G + k / gs]);
      const float q = (float)nibble(row, k);
      volatile float sq = sc * q; /* exact; kept separate so no FMA can form */
      out[n * K + k] = sq + bi;
    }
  }
}

/* ---------------------------------------------------- reference products -- */

IMO_EXPORT void imo_qmv_dequant_f32(const uint32_t* w, const uint16_t* s, const uint16_t* b,
                                    const uint16_t* x, float* y, int64_t M, int64_t N,
                                    int64_t K, int32_t gs, int32_t threads) {
  const int64_t G = K / gs;
  float* xf = (float*)malloc(sizeof(float) * (size_t)(M * K));
  for (int64_t i = 0; i < M * K; ++i) xf[i] = imo_bf16_to_f32(x[i]);
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : 1)
  for (int64_t n = 0; n < N; ++n) {
    const uint32_t* row = w + n * (K / 8);
    float acc[64];
    const int64_t mb = M < 64 ? M : 64;
    for (int64_t m0 = 0; m0 < M; m0 += mb) {
      const int64_t mc = (M - m0) < mb ? (M - m0) : mb;
      for (int64_t m = 0; m < mc; ++m) acc[m] = 0.0f;
      for (int64_t k = 0; k < K; ++k) {
        const float sc = imo_bf16_to_f32(s[n * G + k / gs]);
        const float bi = imo_bf16_to_f32(b[n * G + k / gs]);
        volatile float sq = sc * (float)nibble(row, k);
        const float wk = sq + bi;
        for (int64_t m = 0; m < mc; ++m) acc[m] = fmaf(wk, xf[(m0 + m) * K + k], acc[m]);
      }
      for (int64_t m = 0; m < mc; ++m) y[(m0 + m) * N + n] = acc[m];
    }
  }
  free(xf);
}

IMO_EXPORT void imo_qmv_f64(const uint32_t* w, const uint16_t* s, const uint16_t* b,
                            const uint16_t* x, double* y, double* abssum, int64_t M,
                            int64_t N, int64_t K, int32_t gs, int32_t threads) {
  const int64_t G = K / gs;
  double* xd = (double*)malloc(sizeof(double) * (size_t)(M * K));
  for (int64_t i = 0; i < M * K; ++i) xd[i] = (double)imo_bf16_to_f32(x[i]);
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : 1)
  for (int64_t n = 0; n < N; ++n) {
    const uint32_t* row = w + n * (K / 8);
    for (int64_t m = 0; m < M; ++m) {
      double acc = 0.0, mag = 0.0;
      for (int64_t k = 0; k < K; ++k) {
        const double sc = (double)imo_bf16_to_f32(s[n * G + k / gs]);
        const double bi = (double)imo_bf16_to_f32(b[n * G + k / gs]);
        const double wk = sc * (double)nibble(row, k) + bi; /* exact for finite bf16 */
        const double t = wk * xd[m * K + k];
        acc += t;
        mag += fabs(t);
      }
      y[m * N + n] = acc;
      if (abssum) abssum[m * N + n] = mag;
    }
  }
  free(xd);
}

/* The reference CUDA row kernel (cuda_native.py:57-128), one output row at a time.
 * The result of a row depends on neither M nor R (rows per warp), as the
 * reference states (cuda_native.py:19-21), so rows are independent here. */
IMO_EXPORT void imo_qmv_rowkernel(const uint32_t* w, const uint16_t* s, const uint16_t* b,
                                  const uint16_t* x, void* y, int32_t y_f32, int64_t M,
                                  int64_t N, int64_t K, int32_t gs, int32_t threads) {
  const int64_t G = K / gs;
  const int64_t chunks = K / 32;
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : 1)
  for (int64_t n = 0; n < N; ++n) {
    const uint32_t* row = w + n * (K / 8);
    for (int64_t m = 0; m < M; ++m) {
      const uint16_t* xm = x + m * K;
      float lanes[32];
      for (int lane = 0; lane < 32; ++lane) {
        float acc = 0.0f;
        for (int64_t c = lane; c < chunks; c += 32) {
          const int64_t g = (c * 32) / gs;
          float xf[32];
          float sx = 0.0f;
          for (int i = 0; i < 32; ++i) {
            xf[i] = imo_bf16_to_f32(xm[c * 32 + i]);
            sx = sx + xf[i];
          }
          float qx = 0.0f;
          for (int i = 0; i < 32; ++i) {
            const float q = (float)((row[c * 4 + i / 8] >> (4 * (i % 8))) & 0xFu);
            qx = fmaf(q, xf[i], qx);
          }
          const float sc = imo_bf16_to_f32(s[n * G + g]);
          const float bi = imo_bf16_to_f32(b[n * G + g]);
          volatile float bsx = bi * sx;
          acc = acc + fmaf(sc, qx, bsx);
        }
        lanes[lane] = acc;
      }
      /* __shfl_down_sync tree: lane l reads lane l+o, or keeps its own value past 31 */
      for (int o = 16; o > 0; o >>= 1) {
        float next[32];
        for (int l = 0; l < 32; ++l) next[l] = lanes[l] + (l + o < 32 ? lanes[l + o] : lanes[l]);
        memcpy(lanes, next, sizeof(lanes));
      }
      if (y_f32)
        ((float*)y)[m * N + n] = lanes[0];
      else
        ((uint16_t*)y)[m * N + n] = imo_f32_to_bf16(lanes[0]);
    }
  }
}

/* The reference Metal qmv_impl / qmv_fast_impl arithmetic (see header). */
IMO_EXPORT void imo_qmv_mlx(const uint32_t* w, const uint16_t* s, const uint16_t* b,
                            const uint16_t* x, void* y, int32_t y_f32, int64_t M, int64_t N,
                            int64_t K, int32_t gs, int32_t values_per_thread,
                            int32_t threads) {
  const int64_t G = K / gs;
  const int vpt = values_per_thread; /* 8 (qmv_impl) or 16 (qmv_fast_impl) */
  const int64_t block = (int64_t)vpt * 32;
  const int64_t row_bytes = K / 2;
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : 1)
  for (int64_t n = 0; n < N; ++n) {
    const uint8_t* wrow = (const uint8_t*)(w + n * (K / 8));
    for (int64_t m = 0; m < M; ++m) {
      const uint16_t* xm = x + m * K;
      float result[32];
      for (int lid = 0; lid < 32; ++lid) {
        float res = 0.0f;
        for (int64_t k0 = 0; k0 < K; k0 += block) {
          const int64_t base = k0 + (int64_t)lid * vpt;
          int remaining = (int)(K - base);
          if (remaining <= 0) continue;
          if (remaining > vpt) remaining = vpt;
          float xt[16];
          float sum = 0.0f;
          for (int i = 0; i < remaining; i += 4) {
            const float a0 = imo_bf16_to_f32(xm[base + i]);
            const float a1 = imo_bf16_to_f32(xm[base + i + 1]);
            const float a2 = imo_bf16_to_f32(xm[base + i + 2]);
            const float a3 = imo_bf16_to_f32(xm[base + i + 3]);
            sum += ((a0 + a1) + a2) + a3;
            xt[i] = a0;
            xt[i + 1] = a1 / 16.0f;
            xt[i + 2] = a2 / 256.0f;
            xt[i + 3] = a3 / 4096.0f;
          }
          const uint16_t* ws = (const uint16_t*)(wrow + base / 2);
          float accum = 0.0f;
          for (int i = 0; i < remaining / 4; ++i) {
            const uint16_t h = ws[i];
            volatile float p0 = xt[4 * i] * (float)(h & 0x000f);
            volatile float p1 = xt[4 * i + 1] * (float)(h & 0x00f0);
            volatile float p2 = xt[4 * i + 2] * (float)(h & 0x0f00);
            volatile float p3 = xt[4 * i + 3] * (float)(h & 0xf000);
            accum += ((p0 + p1) + p2) + p3;
          }
          const int64_t g = base / gs;
          const float sc = imo_bf16_to_f32(s[n * G + g]);
          const float bi = imo_bf16_to_f32(b[n * G + g]);
          volatile float t0 = sc * accum;
          volatile float t1 = sum * bi;
          res += t0 + t1;
        }
        result[lid] = res;
      }
      (void)row_bytes;
      for (int o = 16; o > 0; o >>= 1) {
        float next[32];
        for (int l = 0; l < 32; ++l) next[l] = result[l] + result[l ^ o];
        memcpy(result, next, sizeof(result));
      }
      if (y_f32)
        ((float*)y)[m * N + n] = result[0];
      else
        ((uint16_t*)y)[m * N + n] = imo_f32_to_bf16(result[0]);
    }
  }
}

IMO_EXPORT int32_t imo_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
