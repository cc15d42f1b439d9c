/*
 * CPU oracle for tilec's matmul path — TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker (or the timed CPU baseline);
 * the product path (the tilec package) never calls it and has no CPU fallback.
 *
 * What it restates
 *   oracle_matmul_tiled_f32  — the reference tile kernel `_matmul_tiled`
 *       (tilec/ext.py:13-24) literally: for each BM x BN output tile an fp32
 *       accumulator starts at zero (`tl.zeros`, :18); for k in
 *       range(0, K, BK) (:19) the A and B tiles are loaded with masks and
 *       `other=0.0` (:21-22) and `acc = acc + tl.dot(x, y)` (:23), where the
 *       dot of one K step is an fp32 sum over that step's k in increasing
 *       order; then a masked store (:24).  The order of the products inside
 *       one `tl.dot` is not fixed by the reference (it runs on Apple
 *       simdgroup MMA, examples/_matmul_tiled.metal:312-411); increasing k is
 *       the order chosen here.
 *   oracle_matmul_f64        — the same product with every sum in double:
 *       the diagnostic "truth" the GPU's fp32 results are measured against
 *       with rel-L2 (the reference's own oracle is `x1 @ x2`,
 *       tests/test_matmul.py:40).
 *   oracle_matmul_bf16_f64 / oracle_matmul_tiled_bf16 — the same two on
 *       bfloat16 inputs, which are widened exactly to fp32 first.
 *   oracle_bf16_from_f32     — round-to-nearest-even fp32 -> bf16 (NaN kept
 *       quiet), the rounding torch's `.to(torch.bfloat16)` applies.
 *
 * How it is pinned (tests/test_oracle.py): against torch.matmul (the
 * reference's oracle routine) on the reference's five parity shapes
 * (tests/test_matmul.py:33), brute-force fp64 triple loops on tiny shapes,
 * exact integer products, identity / all-ones closed forms, linearity,
 * transpose and K-split invariants, and known bf16 roundings.
 *
 * Build: oracle/Makefile (gcc, OpenMP, no FMA contraction).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

int oracle_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void oracle_set_num_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

static inline float bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, sizeof f);
  return f;
}

void oracle_bf16_from_f32(const float* x, uint16_t* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    uint32_t u;
    memcpy(&u, &x[i], sizeof u);
    if ((u & 0x7fffffffu) > 0x7f800000u) {  /* NaN: keep sign, force quiet */
      y[i] = (uint16_t)((u >> 16) | 0x0040u);
      continue;
    }
    const uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;                         /* round to nearest, ties to even */
    y[i] = (uint16_t)(u >> 16);
  }
}

/* Element loaders with the reference's masks (`other=0.0`). */
static inline float ld_f32(const float* p, int64_t r, int64_t c, int64_t ld, int64_t R, int64_t C) {
  return (r < R && c < C) ? p[r * ld + c] : 0.0f;
}
static inline float ld_bf16(const uint16_t* p, int64_t r, int64_t c, int64_t ld, int64_t R, int64_t C) {
  return (r < R && c < C) ? bf16_to_f32(p[r * ld + c]) : 0.0f;
}

/*
 * Shared body of the tiled restatement.  `get_a(i, k)` / `get_b(k, j)` are
 * the masked loads of tilec/ext.py:21-22.
 */
#define TILED_BODY(GET_A, GET_B)                                                   \
  const int64_t tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;          \
  _Pragma("omp parallel")                                                          \
  {                                                                                \
    float* acc = (float*)malloc(sizeof(float) * BM * BN);                          \
    float* d = (float*)malloc(sizeof(float) * BN);                                 \
    float* brow = (float*)malloc(sizeof(float) * BK * BN);                         \
    _Pragma("omp for schedule(dynamic)")                                           \
    for (int64_t t = 0; t < tiles_m * tiles_n; ++t) {                              \
      const int64_t m0 = (t / tiles_n) * BM, n0 = (t % tiles_n) * BN;              \
      for (int64_t e = 0; e < BM * BN; ++e) acc[e] = 0.0f; /* tl.zeros */          \
      for (int64_t k0 = 0; k0 < K; k0 += BK) {             /* range(0, K, BK) */   \
        for (int64_t kk = 0; kk < BK; ++kk)                                        \
          for (int64_t j = 0; j < BN; ++j) brow[kk * BN + j] = GET_B(k0 + kk, n0 + j); \
        for (int64_t i = 0; i < BM; ++i) {                                         \
          for (int64_t j = 0; j < BN; ++j) d[j] = 0.0f;                            \
          for (int64_t kk = 0; kk < BK; ++kk) {                                    \
            const float x = GET_A(m0 + i, k0 + kk);                                \
            const float* y = brow + kk * BN;                                       \
            for (int64_t j = 0; j < BN; ++j) d[j] = d[j] + x * y[j];               \
          }                                                                        \
          float* ar = acc + i * BN;                                                \
          for (int64_t j = 0; j < BN; ++j) ar[j] = ar[j] + d[j]; /* acc + dot */   \
        }                                                                          \
      }                                                                            \
      for (int64_t i = 0; i < BM && m0 + i < M; ++i)       /* masked store */      \
        for (int64_t j = 0; j < BN && n0 + j < N; ++j) c[(m0 + i) * ldc + n0 + j] = acc[i * BN + j]; \
    }                                                                              \
    free(acc);                                                                     \
    free(d);                                                                       \
    free(brow);                                                                    \
  }

void oracle_matmul_tiled_f32(const float* a, const float* b, float* c, int64_t M, int64_t N, int64_t K,
                             int64_t lda, int64_t ldb, int64_t ldc, int64_t BM, int64_t BN, int64_t BK) {
#define GA(i, k) ld_f32(a, (i), (k), lda, M, K)
#define GB(k, j) ld_f32(b, (k), (j), ldb, K, N)
  TILED_BODY(GA, GB)
#undef GA
#undef GB
}

void oracle_matmul_tiled_bf16(const uint16_t* a, const uint16_t* b, float* c, int64_t M, int64_t N, int64_t K,
                              int64_t lda, int64_t ldb, int64_t ldc, int64_t BM, int64_t BN, int64_t BK) {
#define GA(i, k) ld_bf16(a, (i), (k), lda, M, K)
#define GB(k, j) ld_bf16(b, (k), (j), ldb, K, N)
  TILED_BODY(GA, GB)
#undef GA
#undef GB
}

/* c[i][j] = sum_k (double)a[i][k] * (double)b[k][j], k increasing. */
void oracle_matmul_f64(const float* a, const float* b, double* c, int64_t M, int64_t N, int64_t K, int64_t lda,
                       int64_t ldb, int64_t ldc) {
#pragma omp parallel for schedule(dynamic)
  for (int64_t i = 0; i < M; ++i) {
    double* cr = c + i * ldc;
    for (int64_t j = 0; j < N; ++j) cr[j] = 0.0;
    for (int64_t k = 0; k < K; ++k) {
      const double x = a[i * lda + k];
      const float* br = b + k * ldb;
      for (int64_t j = 0; j < N; ++j) cr[j] += x * (double)br[j];
    }
  }
}

void oracle_matmul_bf16_f64(const uint16_t* a, const uint16_t* b, double* c, int64_t M, int64_t N, int64_t K,
                            int64_t lda, int64_t ldb, int64_t ldc) {
#pragma omp parallel
  {
    double* brow = (double*)malloc(sizeof(double) * (N > 0 ? N : 1));
#pragma omp for schedule(dynamic)
    for (int64_t i = 0; i < M; ++i) {
      double* cr = c + i * ldc;
      for (int64_t j = 0; j < N; ++j) cr[j] = 0.0;
      for (int64_t k = 0; k < K; ++k) {
        const double x = bf16_to_f32(a[i * lda + k]);
        const uint16_t* br = b + k * ldb;
        for (int64_t j = 0; j < N; ++j) cr[j] += x * (double)bf16_to_f32(br[j]);
      }
    }
    free(brow);
  }
}
