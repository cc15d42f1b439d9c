// LDS-staged bf16 GEMM on CDNA4 matrix cores (v_mfma_f32_32x32x16_bf16):
//   C[M,N] (fp32) = A[M,K] (bf16) · B[K,N] (bf16), fp32 accumulate.
//
// Same tile semantics as the reference tile kernel `_matmul_tiled`
// (tilec/ext.py:13-24) — zero accumulator, masked K steps with `other=0.0`,
// masked store — on bf16 inputs, which the reference (fp32 only,
// src/lib.rs:19) does not take.  Layout in LDS:
//   As[m][k]  k-contiguous rows, padded by 16 bytes so the 16-byte operand
//             reads of 16 consecutive rows fall in distinct banks;
//   Bs[n][k]  B transposed while it is written to LDS, so the B operand of
//             every MFMA is also one 16-byte LDS read per lane.
// A and B tiles are double-buffered with one barrier per K step and the next
// tile's global loads issued before the current tile's MFMAs.
#include "common.h"
#include "../../include/tilec.h"

namespace tilec {

namespace {

typedef unsigned short u16;
typedef u16 u16x8 __attribute__((ext_vector_type(8)));

template <int BM, int BN, int BK, int WM, int WN>
struct GemmBf16 {
  static constexpr int NT = WM * WN * 64;
  static constexpr int WTM = BM / WM, WTN = BN / WN;
  static constexpr int TM = WTM / 32, TN = WTN / 32;
  static constexpr int LDS_K = BK + 8;  // row length in elements (16-byte pad)
  static constexpr int A_Q = BM * BK / 8 / NT;  // 16-byte loads of A per thread
  static constexpr int B_Q = BK * BN / 8 / NT;  // 16-byte loads of B per thread
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be whole 32x32 blocks");
  static_assert(BM * BK % (8 * NT) == 0 && BK * BN % (8 * NT) == 0, "tile loads must divide evenly");
  static_assert(BK % 16 == 0, "BK");
  static constexpr size_t kLds = sizeof(u16) * 2 * LDS_K * (BM + BN);
};

template <bool VEC>
__device__ __forceinline__ u16x8 ld8(const u16* __restrict__ p, bool ok_all, int valid) {
  if (VEC) {
    const u16x8 v = *reinterpret_cast<const u16x8*>(p);
    const u16x8 z = {0, 0, 0, 0, 0, 0, 0, 0};
    return ok_all ? v : z;
  } else {
    u16x8 v;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const u16 x = p[c < valid ? c : 0];
      v[c] = c < valid ? x : (u16)0;
    }
    return v;
  }
}

template <int BM, int BN, int BK, int WM, int WN, bool VEC>
__global__ __launch_bounds__(WM * WN * 64) void gemm_bf16_kernel(
    const u16* __restrict__ A, const u16* __restrict__ B, float* __restrict__ C, int M, int N, int K,
    int64_t lda, int64_t ldb, int64_t ldc, int group_m, int split_steps, float* __restrict__ ws,
    unsigned* __restrict__ counters) {
  using P = GemmBf16<BM, BN, BK, WM, WN>;
  extern __shared__ __align__(16) u16 lds_u16[];
  __shared__ int last_flag;
  u16* As = lds_u16;                          // [2][BM][LDS_K]
  u16* Bs = lds_u16 + 2 * BM * P::LDS_K;      // [2][BN][LDS_K]

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  int tm, tn;
  tile_of(blockIdx.x, tiles_m, tiles_n, group_m, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const bool interior = (m0 + BM <= M) && (n0 + BN <= N);
  // K steps [kt0, kt1) of this workgroup (grid y = K splits).
  const int split = blockIdx.y, S = gridDim.y;
  const int kt0 = split * split_steps;
  const int kt1 = min((K + BK - 1) / BK, kt0 + split_steps);
  const int nk_full = K / BK;

  u16x8 ra[P::A_Q], rb[P::B_Q];

  auto gload = [&](int kt, bool mask) {
    const int k0 = kt * BK;
#pragma unroll
    for (int p = 0; p < P::A_Q; ++p) {
      const int e = tid + p * P::NT;
      const int i = e / (BK / 8), kq = e % (BK / 8);
      const int gm = m0 + i, gk = k0 + 8 * kq;
      if (!mask) {
        ra[p] = ld8<VEC>(A + (int64_t)gm * lda + gk, true, 8);
      } else {
        const int valid = gm < M ? max(0, min(8, K - gk)) : 0;
        const int64_t off = valid > 0 ? (int64_t)gm * lda + gk : 0;
        ra[p] = ld8<VEC>(A + off, valid == 8, valid);
      }
    }
#pragma unroll
    for (int p = 0; p < P::B_Q; ++p) {
      const int e = tid + p * P::NT;
      const int k = e / (BN / 8), jq = e % (BN / 8);
      const int gk = k0 + k, gn = n0 + 8 * jq;
      if (!mask) {
        rb[p] = ld8<VEC>(B + (int64_t)gk * ldb + gn, true, 8);
      } else {
        const int valid = gk < K ? max(0, min(8, N - gn)) : 0;
        const int64_t off = valid > 0 ? (int64_t)gk * ldb + gn : 0;
        rb[p] = ld8<VEC>(B + off, valid == 8, valid);
      }
    }
  };

  auto sstore = [&](int buf) {
    u16* as = As + buf * BM * P::LDS_K;
    u16* bs = Bs + buf * BN * P::LDS_K;
#pragma unroll
    for (int p = 0; p < P::A_Q; ++p) {
      const int e = tid + p * P::NT;
      const int i = e / (BK / 8), kq = e % (BK / 8);
      *reinterpret_cast<u16x8*>(as + i * P::LDS_K + 8 * kq) = ra[p];
    }
#pragma unroll
    for (int p = 0; p < P::B_Q; ++p) {
      const int e = tid + p * P::NT;
      const int k = e / (BN / 8), jq = e % (BN / 8);
#pragma unroll
      for (int c = 0; c < 8; ++c) bs[(8 * jq + c) * P::LDS_K + k] = rb[p][c];
    }
  };

  f32x16 acc[P::TM][P::TN];
#pragma unroll
  for (int i = 0; i < P::TM; ++i)
#pragma unroll
    for (int j = 0; j < P::TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  if (kt0 < kt1) {
    gload(kt0, !(interior && kt0 < nk_full));
    sstore(0);
    __syncthreads();
  }

  const int arow = wm * P::WTM + (lane & 31);
  const int bcol = wn * P::WTN + (lane & 31);
  const int khalf = lane >> 5;

  for (int kt = kt0; kt < kt1; ++kt) {
    const int buf = (kt - kt0) & 1;
    const bool more = kt + 1 < kt1;
    if (more) gload(kt + 1, !(interior && kt + 1 < nk_full));
    const u16* as = As + buf * BM * P::LDS_K;
    const u16* bs = Bs + buf * BN * P::LDS_K;
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      const int k = 16 * ks + 8 * khalf;
      bf16x8 a[P::TM], b[P::TN];
#pragma unroll
      for (int i = 0; i < P::TM; ++i)
        a[i] = *reinterpret_cast<const bf16x8*>(as + (arow + 32 * i) * P::LDS_K + k);
#pragma unroll
      for (int j = 0; j < P::TN; ++j)
        b[j] = *reinterpret_cast<const bf16x8*>(bs + (bcol + 32 * j) * P::LDS_K + k);
#pragma unroll
      for (int i = 0; i < P::TM; ++i)
#pragma unroll
        for (int j = 0; j < P::TN; ++j) acc[i][j] = mfma32x32x16bf16(a[i], b[j], acc[i][j]);
    }
    if (more) sstore(buf ^ 1);
    __syncthreads();
  }

  const int row_base = m0 + wm * P::WTM + 4 * khalf;
  const int col_base = n0 + bcol;
  if (S > 1 && !splitk_tile<P::TM, P::TN, P::NT>(acc, split, S, blockIdx.x, gridDim.x, ws, counters, &last_flag,
                                                  row_base, col_base, M, N))
    return;
#pragma unroll
  for (int i = 0; i < P::TM; ++i)
#pragma unroll
    for (int j = 0; j < P::TN; ++j) {
      const int gn = col_base + 32 * j;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int gm = row_base + 32 * i + 8 * (r >> 2) + (r & 3);
        if (interior || (gm < M && gn < N)) C[(int64_t)gm * ldc + gn] = acc[i][j][r];
      }
    }
}

template <int BM, int BN, int BK, int WM, int WN, bool VEC>
hipError_t launch_one(const MatmulArgs& a, dim3 grid) {
  using P = GemmBf16<BM, BN, BK, WM, WN>;
  auto k = gemm_bf16_kernel<BM, BN, BK, WM, WN, VEC>;
  const SplitGeom g = gemm_split_geom(a.K, BK, a.split_k);
  if (g.splits > 1 && P::TM * P::TN * 16 > kSplitMaxAccPerThread) return hipErrorInvalidConfiguration;
  grid.y = (unsigned)g.splits;
  const size_t lds = GemmBf16<BM, BN, BK, WM, WN>::kLds;
  static bool attr_set = false;
  if (lds > 65536 && !attr_set) {
    hipError_t e = hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  hipLaunchKernelGGL(k, grid, dim3(WM * WN * 64), lds, a.stream, static_cast<const u16*>(a.x1),
                     static_cast<const u16*>(a.x2), a.out, (int)a.M, (int)a.N, (int)a.K, a.ldx1, a.ldx2, a.ldo,
                     8, (int)g.steps, g.splits > 1 ? static_cast<float*>(a.workspace) : nullptr, g.splits > 1 ? a.counters : nullptr);
  return hipGetLastError();
}

}  // namespace

template <int BM, int BN, int BK, int NBUF, int WM, int WN>
hipError_t launch_gemm_bf16_lds(const MatmulArgs& a);  // gemm_bf16_lds.hip

namespace {

// Aligned operands (16-byte base, K, N, lda, ldb multiples of 8) whose tile
// offsets fit 32 bits run the LDS-DMA kernel of gemm_bf16_lds.hip with a
// ring of NBUF stage buffers of BK; everything else runs the generic kernel
// above with the same output tile (NBUF == 0: generic kernel only).  Both
// use the variant's WM x WN waves, so a K split is possible in one exactly
// when it is in the other.
template <int BM, int BN, int BK, int NBUF, int WM = 2, int WN = 2>
hipError_t launch_gemm_bf16(const MatmulArgs& a) {
  const int64_t tiles = cdiv(a.M, BM) * cdiv(a.N, BN);
  if (tiles == 0) return hipSuccess;
  const bool vec = (a.K % 8 == 0) && (a.N % 8 == 0) && (a.ldx1 % 8 == 0) && (a.ldx2 % 8 == 0) &&
                   (reinterpret_cast<uintptr_t>(a.x1) % 16 == 0) && (reinterpret_cast<uintptr_t>(a.x2) % 16 == 0);
  if constexpr (NBUF > 0) {
    if (vec && a.ldx1 < (int64_t(1) << 22) && a.ldx2 < (int64_t(1) << 24))
      return launch_gemm_bf16_lds<BM, BN, BK, NBUF, WM, WN>(a);
  }
  dim3 grid((unsigned)tiles);
  return vec ? launch_one<BM, BN, 64, WM, WN, true>(a, grid) : launch_one<BM, BN, 64, WM, WN, false>(a, grid);
}

}  // namespace

// Variant table for this family (its order is part of the variant numbering).
// BK is the K step of the LDS-DMA kernel and `unroll` its ring depth.
const VariantDesc* gemm_bf16_variants(int* count) {
  static const VariantDesc t[] = {
      {"gemm_bf16_256x256x32_r4", TILEC_FAMILY_GEMM, TILEC_BF16, 256, 256, 32, 4, 0, 4,
       launch_gemm_bf16<256, 256, 32, 4>},
      {"gemm_bf16_256x256x64_r2", TILEC_FAMILY_GEMM, TILEC_BF16, 256, 256, 64, 8, 0, 2,
       launch_gemm_bf16<256, 256, 64, 2, 2, 4>},
      {"gemm_bf16_256x128x64_r3", TILEC_FAMILY_GEMM, TILEC_BF16, 256, 128, 64, 8, 0, 3,
       launch_gemm_bf16<256, 128, 64, 3, 4, 2>},
      {"gemm_bf16_256x128x32_r4", TILEC_FAMILY_GEMM, TILEC_BF16, 256, 128, 32, 4, 0, 4,
       launch_gemm_bf16<256, 128, 32, 4>},
      {"gemm_bf16_128x128x64_r4", TILEC_FAMILY_GEMM, TILEC_BF16, 128, 128, 64, 8, 0, 4,
       launch_gemm_bf16<128, 128, 64, 4, 2, 4>},
      {"gemm_bf16_64x64x64_w2x2", TILEC_FAMILY_GEMM, TILEC_BF16, 64, 64, 64, 4, 0, 1,
       launch_gemm_bf16<64, 64, 64, 0>},
  };
  *count = (int)(sizeof(t) / sizeof(t[0]));
  return t;
}
}  // namespace tilec
