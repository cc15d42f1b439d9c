// Output-stationary streaming kernel for skinny products, M <= 16:
//   out[M,N] = x1[M,K] · x2[K,N]   (fp32 in, fp32 out)
//
// Replaces, for small M, the reference's threadgroup-split dot product with a
// SIMD-group reduction (the legacy `_matrix_mul` described at README.md:57,73,
// whose config space survives in tilec/ext.py:29-51): here every lane owns a
// fixed group of output columns, so no reduction across lanes is needed for
// the columns, and x2 — the only large operand — is streamed from HBM exactly
// once with 16-byte coalesced loads.
//
// Mapping (one wave of 64 lanes):
//   lane l: r = l / 16 picks one of 4 consecutive x2 rows, q = l % 16 picks a
//   4-column quad.  One wave load therefore covers rows k..k+3 × 64 columns
//   (four 256-byte row segments).  Those 4 rows are the K=4 reduction slots of
//   v_mfma_f32_16x16x4f32, and each of the 4 columns of a lane's quad feeds
//   one MFMA:  D_c[m][q] += sum_r x1[m][k+r] * x2[k+r][64*slab + 4q + c].
//   The A operand (lane l holds x1[l%16][k + l/16]) is the x1 tile, rows >= M
//   zero.  So the reduction over K stays inside the MFMA; nothing is shuffled.
//   Per 1 KiB of x2 a wave issues 4 MFMAs (128 cycles), 2.5x the rate the HBM
//   share of a SIMD needs, for any M <= 16.
//
// Grid: x = 64-column slabs, y = K splits ("split_k").  The waves of a
// workgroup take interleaved 4-row groups of the workgroup's K chunk, are
// summed through LDS, and when K is split across workgroups each workgroup
// writes its [M x 64] partial to the workspace; the last workgroup of a slab to
// finish (completion counter) adds the partials in split order, so results do
// not depend on scheduling.  The counter is reset to zero by that workgroup.
#include "common.h"
#include "../../include/tilec.h"

namespace tilec {

namespace {

constexpr int kSlab = 64;    // output columns per workgroup
constexpr int kMaxM = 16;    // MFMA rows

struct SkinnyGeom {
  int64_t nslabs, splits, kc;
};

// K chunk per split: a multiple of 4 rows; splits recomputed so none is empty.
SkinnyGeom skinny_geom(int64_t N, int64_t K, int split_k) {
  SkinnyGeom g;
  g.nslabs = cdiv(N, kSlab);
  if (split_k < 1) split_k = 1;
  if (K <= 0) {
    g.splits = 1;
    g.kc = 0;
    return g;
  }
  int64_t kc = cdiv(K, split_k);
  kc = cdiv(kc, 4) * 4;
  g.kc = kc;
  g.splits = cdiv(K, kc);
  return g;
}

template <bool VEC>
__device__ __forceinline__ f32x4 load_quad(const float* __restrict__ row, int col, bool col_ok, int N) {
  if (VEC) {
    // N % 4 == 0, so a quad is either wholly inside or wholly outside.
    const f32x4 v = *reinterpret_cast<const f32x4*>(row + (col_ok ? col : 0));
    return col_ok ? v : f32x4{0.f, 0.f, 0.f, 0.f};
  } else {
    f32x4 v;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const bool ok = col + c < N;
      const float x = row[ok ? col + c : 0];
      v[c] = ok ? x : 0.f;
    }
    return v;
  }
}

template <bool VEC>
__device__ __forceinline__ void store_quad(float* __restrict__ row, int col, int N, f32x4 v) {
  if (VEC) {
    if (col < N) *reinterpret_cast<f32x4*>(row + col) = v;
  } else {
#pragma unroll
    for (int c = 0; c < 4; ++c)
      if (col + c < N) row[col + c] = v[c];
  }
}

template <int WAVES, int UNROLL, bool VEC>
__global__ __launch_bounds__(WAVES * 64) void skinny_f32_kernel(
    const float* __restrict__ x1, const float* __restrict__ x2, float* __restrict__ out,
    int M, int N, int K, int64_t ldx1, int64_t ldx2, int64_t ldo, int kc,
    unsigned* __restrict__ counters, float* __restrict__ part) {
  static_assert(WAVES >= 4, "the epilogue uses 256 threads");
  __shared__ f32x4 red[WAVES][kMaxM][kSlab / 4];
  __shared__ int last_flag;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int r = lane >> 4, q = lane & 15;
  const int slab = blockIdx.x, split = blockIdx.y;
  const int nslabs = gridDim.x, S = gridDim.y;
  const int col = slab * kSlab + 4 * q;
  const bool col_ok = col < N;
  const int kbeg = split * kc;
  const int kend = min(K, kbeg + kc);
  const int ngroups = kend > kbeg ? (kend - kbeg + 3) >> 2 : 0;

  const bool arow_ok = q < M;
  const float* __restrict__ arow = x1 + (int64_t)(arow_ok ? q : 0) * ldx1;

  f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = acc0, acc2 = acc0, acc3 = acc0;

  // Row group g of this chunk: rows kbeg + 4g .. +3; this lane takes row +r.
  auto load = [&](int g, f32x4& b, float& a) {
    const int k = kbeg + 4 * g + r;
    const bool ok = (g < ngroups) & (k < kend);
    const int kk = ok ? k : kbeg;  // in bounds whenever ngroups > 0
    const f32x4 v = load_quad<VEC>(x2 + (int64_t)kk * ldx2, col, col_ok, N);
    const float x = arow[kk];
    b = ok ? v : f32x4{0.f, 0.f, 0.f, 0.f};
    a = (ok & arow_ok) ? x : 0.f;
  };

  constexpr int STEP = WAVES * UNROLL;
  if (wave < ngroups) {
    f32x4 bc[UNROLL];
    float ac[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) load(wave + u * WAVES, bc[u], ac[u]);
    for (int g0 = wave; g0 < ngroups; g0 += STEP) {
      const int g1 = g0 + STEP;
      f32x4 bn[UNROLL];
      float an[UNROLL];
      const bool more = g1 < ngroups;
      if (more) {
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) load(g1 + u * WAVES, bn[u], an[u]);
      }
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        acc0 = mfma16x16x4(ac[u], bc[u][0], acc0);
        acc1 = mfma16x16x4(ac[u], bc[u][1], acc1);
        acc2 = mfma16x16x4(ac[u], bc[u][2], acc2);
        acc3 = mfma16x16x4(ac[u], bc[u][3], acc3);
      }
      if (more) {
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
          bc[u] = bn[u];
          ac[u] = an[u];
        }
      }
    }
  }

  // Lane l holds D_c[4r + v][q] in acc_c[v]: out row 4r+v, columns col..col+3.
#pragma unroll
  for (int v = 0; v < 4; ++v) red[wave][4 * r + v][q] = f32x4{acc0[v], acc1[v], acc2[v], acc3[v]};
  __syncthreads();

  const int m = tid >> 4, cq = tid & 15;  // epilogue thread -> (row, quad), tid < 256
  const int ocol = slab * kSlab + 4 * cq;
  f32x4 s = {0.f, 0.f, 0.f, 0.f};
  if (tid < 256) {
#pragma unroll
    for (int w = 0; w < WAVES; ++w) s += red[w][m][cq];
  }

  if (S == 1) {
    if (tid < 256 && m < M) store_quad<VEC>(out + (int64_t)m * ldo, ocol, N, s);
    return;
  }

  float* __restrict__ my_part = part + ((int64_t)(split * nslabs + slab) * kMaxM) * kSlab;
  if (tid < 256 && m < M) *reinterpret_cast<f32x4*>(my_part + m * kSlab + 4 * cq) = s;
  __threadfence();  // release this thread's partial at device scope
  __syncthreads();
  if (tid == 0) {
    const unsigned prev =
        __hip_atomic_fetch_add(&counters[slab], 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    last_flag = prev == (unsigned)(S - 1);
  }
  __syncthreads();
  if (!last_flag) return;
  __threadfence();  // acquire: the other workgroups' partials are visible

  if (tid < 256 && m < M) {
    f32x4 t = {0.f, 0.f, 0.f, 0.f};
    for (int sp = 0; sp < S; ++sp)
      t += *reinterpret_cast<const f32x4*>(part + ((int64_t)(sp * nslabs + slab) * kMaxM + m) * kSlab +
                                           4 * cq);
    store_quad<VEC>(out + (int64_t)m * ldo, ocol, N, t);
  }
  if (tid == 0) __hip_atomic_store(&counters[slab], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int WAVES, int UNROLL>
hipError_t launch_skinny(const MatmulArgs& a) {
  const SkinnyGeom g = skinny_geom(a.N, a.K, a.split_k);
  const float* x1 = static_cast<const float*>(a.x1);
  const float* x2 = static_cast<const float*>(a.x2);
  const bool vec = (a.N % 4 == 0) && (a.ldx2 % 4 == 0) && (a.ldo % 4 == 0) &&
                   (reinterpret_cast<uintptr_t>(x2) % 16 == 0) &&
                   (reinterpret_cast<uintptr_t>(a.out) % 16 == 0);
  unsigned* counters = nullptr;
  float* part = nullptr;
  if (g.splits > 1) {
    counters = static_cast<unsigned*>(a.workspace);
    const size_t cbytes = cdiv(g.nslabs * sizeof(unsigned), 256) * 256;
    part = reinterpret_cast<float*>(static_cast<char*>(a.workspace) + cbytes);
  }
  dim3 grid((unsigned)g.nslabs, (unsigned)g.splits);
  dim3 block(WAVES * 64);
  if (vec)
    hipLaunchKernelGGL((skinny_f32_kernel<WAVES, UNROLL, true>), grid, block, 0, a.stream, x1, x2, a.out,
                       (int)a.M, (int)a.N, (int)a.K, a.ldx1, a.ldx2, a.ldo, (int)g.kc, counters, part);
  else
    hipLaunchKernelGGL((skinny_f32_kernel<WAVES, UNROLL, false>), grid, block, 0, a.stream, x1, x2, a.out,
                       (int)a.M, (int)a.N, (int)a.K, a.ldx1, a.ldx2, a.ldo, (int)g.kc, counters, part);
  return hipGetLastError();
}

}  // namespace

// Variant table for this family (its order is part of the variant numbering).
const VariantDesc* skinny_variants(int* count) {
  static const VariantDesc t[] = {
      {"skinny_f32_w4_u4", TILEC_FAMILY_SKINNY, TILEC_F32, 16, kSlab, 4, 4, kMaxM, 4, launch_skinny<4, 4>},
      {"skinny_f32_w4_u8", TILEC_FAMILY_SKINNY, TILEC_F32, 16, kSlab, 4, 4, kMaxM, 8, launch_skinny<4, 8>},
      {"skinny_f32_w8_u4", TILEC_FAMILY_SKINNY, TILEC_F32, 16, kSlab, 4, 8, kMaxM, 4, launch_skinny<8, 4>},
      {"skinny_f32_w8_u8", TILEC_FAMILY_SKINNY, TILEC_F32, 16, kSlab, 4, 8, kMaxM, 8, launch_skinny<8, 8>},
      {"skinny_f32_w16_u4", TILEC_FAMILY_SKINNY, TILEC_F32, 16, kSlab, 4, 16, kMaxM, 4, launch_skinny<16, 4>},
  };
  *count = (int)(sizeof(t) / sizeof(t[0]));
  return t;
}

// Workspace layout: counters (one uint32 per slab, padded to 256 B), then
// partials [splits][nslabs][16][64] fp32.
size_t skinny_counter_bytes(int64_t N, int64_t K, int split_k) {
  const SkinnyGeom g = skinny_geom(N, K, split_k);
  if (g.splits <= 1) return 0;
  return cdiv(g.nslabs * sizeof(unsigned), 256) * 256;
}
size_t skinny_workspace_bytes(int64_t N, int64_t K, int split_k) {
  const SkinnyGeom g = skinny_geom(N, K, split_k);
  if (g.splits <= 1) return 0;
  return skinny_counter_bytes(N, K, split_k) + (size_t)g.splits * g.nslabs * kMaxM * kSlab * sizeof(float);
}
int64_t skinny_effective_splits(int64_t N, int64_t K, int split_k) { return skinny_geom(N, K, split_k).splits; }

}  // namespace tilec
