// LDS-staged fp32 GEMM on CDNA4 matrix cores (v_mfma_f32_32x32x2f32):
//   C[M,N] = A[M,K] · B[K,N], fp32 row-major, fp32 accumulate.
//
// Semantics follow the reference tile kernel `_matmul_tiled`
// (tilec/ext.py:13-24): one workgroup per BM x BN output tile, an accumulator
// that starts at zero, a K loop in steps of BK over masked tiles of A and B
// (`other=0.0`), and a masked store.  What runs underneath is MI355X-native:
//   * 64-wide waves arranged WM x WN, each owning a (BM/WM) x (BN/WN) block of
//     32x32 MFMA accumulators held in registers for the whole K loop;
//   * A and B tiles double-buffered in LDS with one barrier per K step; the
//     next tile's global loads are issued before the current tile's MFMAs;
//   * A stored k-major in LDS (As[k][m]) so every MFMA operand read is one
//     conflict-free 32-bit LDS read per lane for both operands;
//   * branch-free edges, as the reference's if-converted masked loads
//     (README.md:50): with row strides that fit 32-bit offsets (BUF), every
//     tile loads through buffer resources that end at the matrix's last
//     element — rows past M (A) or K (B) get an out-of-range offset and load
//     zeros, and when K or N is not a multiple of 4 a per-element select
//     clears the columns past the edge of the quad that straddles it — so
//     edge tiles cost what interior ones do; otherwise clamped addresses plus
//     selects on edge tiles and the K tail;
//   * XCD-aware, grouped tile order (tile_of in common.h).
#include "common.h"
#include "../../include/tilec.h"

namespace tilec {

namespace {

template <int BM, int BN, int BK, int WM, int WN, bool VEC>
struct GemmF32 {
  static constexpr int NT = WM * WN * 64;
  static constexpr int WTM = BM / WM, WTN = BN / WN;
  static constexpr int TM = WTM / 32, TN = WTN / 32;
  static constexpr int LDA_S = BM + 4;  // As[k][m] row length (floats)
  static constexpr int LDB_S = BN + 4;  // Bs[k][n] row length (floats)
  static constexpr int A_Q = BM * BK / 4 / NT;  // float4 loads of A per thread
  static constexpr int B_Q = BK * BN / 4 / NT;  // float4 loads of B per thread
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be whole 32x32 blocks");
  static_assert(BM * BK % (4 * NT) == 0 && BK * BN % (4 * NT) == 0, "tile loads must divide evenly");
  static_assert(BK % 4 == 0 && BK % 2 == 0, "BK");
  static constexpr size_t kLds = sizeof(float) * 2 * BK * (LDA_S + LDB_S);
};

// Four consecutive floats at a 4-byte aligned address: one dwordx4 load,
// which CDNA performs for any dword-aligned address.
typedef float f32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));

template <bool VEC>
__device__ __forceinline__ f32x4 ld4(const float* __restrict__ p, bool ok_all, int valid) {
  // valid: number of leading elements in bounds (0..4); VEC => valid in {0,4}
  if (VEC) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(p);
    return ok_all ? v : f32x4{0.f, 0.f, 0.f, 0.f};
  } else {
    f32x4 v;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float x = p[c < valid ? c : 0];
      v[c] = c < valid ? x : 0.f;
    }
    return v;
  }
}

template <int BM, int BN, int BK, int WM, int WN, bool VEC, bool BUF>
__global__ __launch_bounds__(WM * WN * 64) void gemm_f32_kernel(
    const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, int M, int N, int K,
    int64_t lda, int64_t ldb, int64_t ldc, int group_m, int split_steps, float* __restrict__ ws,
    unsigned* __restrict__ counters) {
  using P = GemmF32<BM, BN, BK, WM, WN, VEC>;
  extern __shared__ __align__(16) float lds[];
  __shared__ int last_flag;
  float* As = lds;                          // [2][BK][LDA_S]
  float* Bs = lds + 2 * BK * P::LDA_S;      // [2][BK][LDB_S]

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

  f32x4 ra[P::A_Q], rb[P::B_Q];

  // BUF: per-thread quad coordinates are fixed for the whole K loop; the
  // resources move with k0.  Columns a quad keeps: A's K edge moves with the
  // step, B's N edge is fixed per tile.
  int a_row[P::A_Q], a_k[P::A_Q], b_k[P::B_Q], b_valid[P::B_Q];
  uint32_t a_off[P::A_Q], b_off[P::B_Q];
  if constexpr (BUF) {
#pragma unroll
    for (int p = 0; p < P::A_Q; ++p) {
      const int e = tid + p * P::NT;
      a_row[p] = e / (BK / 4);
      a_k[p] = 4 * (e % (BK / 4));
      a_off[p] = m0 + a_row[p] < M ? 4u * ((uint32_t)a_row[p] * (uint32_t)lda + (uint32_t)a_k[p]) : kOob;
    }
#pragma unroll
    for (int p = 0; p < P::B_Q; ++p) {
      const int e = tid + p * P::NT;
      b_k[p] = e / (BN / 4);
      const int n = 4 * (e % (BN / 4));
      b_valid[p] = max(0, min(4, N - (n0 + n)));
      b_off[p] = b_valid[p] > 0 ? 4u * ((uint32_t)b_k[p] * (uint32_t)ldb + (uint32_t)n) : kOob;
    }
  }
  // Bytes from p to the end of a matrix of `rows` rows (row stride ld, last
  // row `cols` long), clamped to a buffer's 31-bit range; 0 if none.
  auto extent = [](int64_t rows_left, int64_t ld, int64_t cols_left) -> uint32_t {
    if (rows_left <= 0 || cols_left <= 0) return 0u;
    const int64_t bytes = 4 * ((rows_left - 1) * ld + cols_left);
    return bytes > 0x7FFFFFFF ? 0x7FFFFFFFu : (uint32_t)bytes;
  };
  auto gload_buf = [&](int kt) {
    const int k0 = kt * BK;
    const BufRsrc rA = make_rsrc(A + (int64_t)m0 * lda + k0, extent(M - m0, lda, K - k0));
    const BufRsrc rB = make_rsrc(B + (int64_t)k0 * ldb + n0, extent(K - k0, ldb, N - n0));
#pragma unroll
    for (int p = 0; p < P::A_Q; ++p) {
      f32x4 v = load_f32x4(rA, k0 + a_k[p] < K ? a_off[p] : kOob);
      if constexpr (!VEC) {
        const int valid = K - (k0 + a_k[p]);
#pragma unroll
        for (int c = 1; c < 4; ++c) v[c] = c < valid ? v[c] : 0.f;
      }
      ra[p] = v;
    }
#pragma unroll
    for (int p = 0; p < P::B_Q; ++p) {
      f32x4 v = load_f32x4(rB, k0 + b_k[p] < K ? b_off[p] : kOob);
      if constexpr (!VEC) {
#pragma unroll
        for (int c = 1; c < 4; ++c) v[c] = c < b_valid[p] ? v[c] : 0.f;
      }
      rb[p] = v;
    }
  };

  // Global -> registers for K tile kt.  MASK: clamp + select at every edge.
  auto gload = [&](int kt, bool mask) {
    if constexpr (BUF) {
      gload_buf(kt);
      return;
    }
    const int k0 = kt * BK;
#pragma unroll
    for (int p = 0; p < P::A_Q; ++p) {
      const int e = tid + p * P::NT;
      const int i = e / (BK / 4), kq = e % (BK / 4);
      const int gm = m0 + i, gk = k0 + 4 * kq;
      if (!mask) {  // whole quad in bounds: one (dword-aligned) 16-byte load
        ra[p] = *reinterpret_cast<const f32x4_a4*>(A + (int64_t)gm * lda + gk);
      } else {
        const bool rok = gm < M;
        const int valid = rok ? max(0, min(4, K - gk)) : 0;
        const int64_t off = valid > 0 ? (int64_t)gm * lda + gk : 0;
        ra[p] = ld4<VEC>(A + off, valid == 4, valid);
      }
    }
#pragma unroll
    for (int p = 0; p < P::B_Q; ++p) {
      const int e = tid + p * P::NT;
      const int k = e / (BN / 4), jq = e % (BN / 4);
      const int gk = k0 + k, gn = n0 + 4 * jq;
      if (!mask) {
        rb[p] = *reinterpret_cast<const f32x4_a4*>(B + (int64_t)gk * ldb + gn);
      } else {
        const int valid = gk < K ? max(0, min(4, N - gn)) : 0;
        const int64_t off = valid > 0 ? (int64_t)gk * ldb + gn : 0;
        rb[p] = ld4<VEC>(B + off, valid == 4, valid);
      }
    }
  };

  auto sstore = [&](int buf) {
    float* as = As + buf * BK * P::LDA_S;
    float* bs = Bs + buf * BK * P::LDB_S;
#pragma unroll
    for (int p = 0; p < P::A_Q; ++p) {
      const int e = tid + p * P::NT;
      const int i = e / (BK / 4), kq = e % (BK / 4);
#pragma unroll
      for (int c = 0; c < 4; ++c) as[(4 * kq + c) * P::LDA_S + i] = ra[p][c];
    }
#pragma unroll
    for (int p = 0; p < P::B_Q; ++p) {
      const int e = tid + p * P::NT;
      const int k = e / (BN / 4), jq = e % (BN / 4);
      *reinterpret_cast<f32x4*>(bs + k * P::LDB_S + 4 * jq) = rb[p];
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
    const float* as = As + buf * BK * P::LDA_S;
    const float* bs = Bs + buf * BK * P::LDB_S;
#pragma unroll
    for (int ks = 0; ks < BK / 2; ++ks) {
      const int k = 2 * ks + khalf;
      float a[P::TM], b[P::TN];
#pragma unroll
      for (int i = 0; i < P::TM; ++i) a[i] = as[k * P::LDA_S + arow + 32 * i];
#pragma unroll
      for (int j = 0; j < P::TN; ++j) b[j] = bs[k * P::LDB_S + bcol + 32 * j];
#pragma unroll
      for (int i = 0; i < P::TM; ++i)
#pragma unroll
        for (int j = 0; j < P::TN; ++j) acc[i][j] = mfma32x32x2(a[i], b[j], acc[i][j]);
    }
    if (more) sstore(buf ^ 1);
    __syncthreads();
  }

  // Epilogue: lane holds D[8*(r/4) + 4*(lane/32) + r%4][lane%32] of each block.
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

template <int BM, int BN, int BK, int WM, int WN, bool VEC, bool BUF>
hipError_t launch_one(const MatmulArgs& a, dim3 grid) {
  using P = GemmF32<BM, BN, BK, WM, WN, VEC>;
  auto k = gemm_f32_kernel<BM, BN, BK, WM, WN, VEC, BUF>;
  const SplitGeom g = gemm_split_geom(a.K, BK, a.split_k);
  if (g.splits > 1 && P::TM * P::TN * 16 > kSplitMaxAccPerThread) return hipErrorInvalidConfiguration;
  grid.y = (unsigned)g.splits;
  const size_t lds = GemmF32<BM, BN, BK, WM, WN, VEC>::kLds;
  static bool attr_set = false;
  if (lds > 65536 && !attr_set) {
    hipError_t e = hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  hipLaunchKernelGGL(k, grid, dim3(WM * WN * 64), lds, a.stream, static_cast<const float*>(a.x1),
                     static_cast<const float*>(a.x2), a.out, (int)a.M, (int)a.N, (int)a.K, a.ldx1, a.ldx2, a.ldo,
                     8, (int)g.steps, g.splits > 1 ? static_cast<float*>(a.workspace) : nullptr, g.splits > 1 ? a.counters : nullptr);
  return hipGetLastError();
}

template <int BM, int BN, int BK, int WM, int WN>
hipError_t launch_gemm_f32(const MatmulArgs& a) {
  const int64_t tiles = cdiv(a.M, BM) * cdiv(a.N, BN);
  if (tiles == 0) return hipSuccess;
  const bool vec = (a.K % 4 == 0) && (a.N % 4 == 0) && (a.ldx1 % 4 == 0) && (a.ldx2 % 4 == 0) &&
                   (reinterpret_cast<uintptr_t>(a.x1) % 16 == 0) && (reinterpret_cast<uintptr_t>(a.x2) % 16 == 0);
  // Buffer offsets inside one K step: row * ld * 4 + 16 * quad < 2^31.
  const bool buf = (int64_t)BM * a.ldx1 * 4 + 4 * BK < (int64_t(1) << 31) &&
                   (int64_t)BK * a.ldx2 * 4 + 4 * BN < (int64_t(1) << 31);
  dim3 grid((unsigned)tiles);
  if (buf)
    return vec ? launch_one<BM, BN, BK, WM, WN, true, true>(a, grid) : launch_one<BM, BN, BK, WM, WN, false, true>(a, grid);
  return vec ? launch_one<BM, BN, BK, WM, WN, true, false>(a, grid) : launch_one<BM, BN, BK, WM, WN, false, false>(a, grid);
}

}  // namespace

// Variant table for this family (its order is part of the variant numbering).
const VariantDesc* gemm_f32_variants(int* count) {
  static const VariantDesc t[] = {
      {"gemm_f32_256x256x16_w2x2", TILEC_FAMILY_GEMM, TILEC_F32, 256, 256, 16, 4, 0, 1,
       launch_gemm_f32<256, 256, 16, 2, 2>},
      {"gemm_f32_256x128x16_w2x2", TILEC_FAMILY_GEMM, TILEC_F32, 256, 128, 16, 4, 0, 1,
       launch_gemm_f32<256, 128, 16, 2, 2>},
      {"gemm_f32_128x128x16_w2x2", TILEC_FAMILY_GEMM, TILEC_F32, 128, 128, 16, 4, 0, 1,
       launch_gemm_f32<128, 128, 16, 2, 2>},
      {"gemm_f32_128x64x16_w2x2", TILEC_FAMILY_GEMM, TILEC_F32, 128, 64, 16, 4, 0, 1,
       launch_gemm_f32<128, 64, 16, 2, 2>},
      {"gemm_f32_64x64x16_w2x2", TILEC_FAMILY_GEMM, TILEC_F32, 64, 64, 16, 4, 0, 1,
       launch_gemm_f32<64, 64, 16, 2, 2>},
  };
  *count = (int)(sizeof(t) / sizeof(t[0]));
  return t;
}

}  // namespace tilec
