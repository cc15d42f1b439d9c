// Output-stationary streaming kernel for products with a small output:
//   out[M,N] = x1[M,K] · x2[K,N]   (fp32 in, fp32 out)
// built for M <= 16 (one 16-row block) and used for any M whose output is
// too small to fill the chip with tile-GEMM workgroups (each further 16 rows
// of x1 is one more row block of the grid).
//
// Replaces, for small M, the reference's threadgroup-split dot product with a
// SIMD-group reduction (the legacy `_matrix_mul` described at README.md:57,73,
// whose config space survives in tilec/ext.py:29-51): here every lane owns a
// fixed group of output columns, so no reduction across lanes is needed for
// the columns, and x2 — the only large operand — is streamed from HBM exactly
// once with 16-byte coalesced loads.
//
// Mapping.  A workgroup owns a 64-column slab of the output and one K chunk.
// The chunk is walked in 16-row blocks; waves take interleaved blocks.  In a
// block, lane l (r = l / 16, q = l % 16) loads the 4-column quad q of rows
// 4r + u, u = 0..3 (four 16-byte loads; each wave load covers four 256-byte
// row segments) and the 16-byte quad x1[q][4r .. 4r+3].  Row 4r + u is MFMA
// k-slot r of step u of v_mfma_f32_16x16x4f32, and the 4 columns of the x2
// quad feed 4 MFMAs:
//   D_c[m][q] += sum_r x1[m][4r+u] * x2[4r+u][64*slab + 4q + c],
// the A operand being exactly the lane's x1 value for (m = q, k-slot r).
// Masking is done on addresses only: rows past the chunk, columns past N and
// x1 rows past M get an out-of-range buffer offset and load zeros without
// touching memory, so loaded registers go straight into the MFMAs.  Per
// 4 KiB of x2 a wave issues 16 MFMAs (512 cycles), 2.5x the rate the HBM
// share of a SIMD needs, for any M <= 16.
//
// Grid: x = 64-column slabs, y = K splits, z = 16-row blocks of x1 and out.
// Waves are summed through LDS; with a split K each workgroup writes its
// [16 x 64] partial to the workspace, and the last workgroup of a (row
// block, slab) to finish (completion counter) adds the partials in split
// order, so results do not depend on scheduling; it resets the counter to
// zero.
#include "common.h"
#include "../../include/tilec.h"

namespace tilec {

namespace {

constexpr int kSlab = 64;      // output columns per workgroup
constexpr int kMaxM = 16;      // MFMA rows
constexpr int kBlock = 16;     // x2 rows per block (4 MFMA steps of 4 rows)
constexpr int kKcMax = 1024;   // rows per K chunk at most
constexpr int kCounterStride = 64;  // uint32s between completion counters (own 256-byte line each)

struct SkinnyGeom {
  int64_t nslabs, splits, kc, nrb;
};

// K chunk per split: a multiple of kBlock rows, at most kKcMax; the number of
// splits is raised to what kKcMax needs and recomputed so that none is empty.
SkinnyGeom skinny_geom(int64_t M, int64_t N, int64_t K, int split_k) {
  SkinnyGeom g;
  g.nslabs = cdiv(N, kSlab);
  g.nrb = cdiv(M, kMaxM);
  if (K <= 0) {
    g.splits = 1;
    g.kc = 0;
    return g;
  }
  int64_t s = split_k < 1 ? 1 : split_k;
  if (s < cdiv(K, kKcMax)) s = cdiv(K, kKcMax);
  g.kc = cdiv(cdiv(K, s), kBlock) * kBlock;
  g.splits = cdiv(K, g.kc);
  return g;
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

// One 16-row block of the chunk as this lane holds it: x2 rows 4r + u
// (u = 0..3) of the lane's column quad, and x1[q][4r .. 4r+3].
struct Block {
  f32x4 b[4];
  f32x4 a;
};

template <int WAVES, int UB, bool VEC>
__global__ __launch_bounds__(WAVES * 64) void skinny_f32_kernel(
    const float* __restrict__ x1, const float* __restrict__ x2, float* __restrict__ out,
    int M_all, int N, int K, int64_t ldx1, int64_t ldx2, int64_t ldo, int kc,
    unsigned* __restrict__ counters, float* __restrict__ part) {
  __shared__ f32x4 red[WAVES * kMaxM * 16];  // [wave][row][quad]
  __shared__ int last_flag;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int r = lane >> 4, q = lane & 15;
  const int slab = blockIdx.x, split = blockIdx.y, rb = blockIdx.z;
  const int nslabs = gridDim.x, S = gridDim.y;
  // This workgroup's row block: rows 16*rb .. of x1 and out, M of them.
  const int M = min(kMaxM, M_all - kMaxM * rb);
  x1 += (int64_t)kMaxM * rb * ldx1;
  out += (int64_t)kMaxM * rb * ldo;
  const int cell = rb * nslabs + slab;  // (row block, slab): partial slot and counter
  const int col = slab * kSlab + 4 * q;
  const bool col_ok = col < N;
  const int kbeg = split * kc;
  const int nrows = max(0, min(K, kbeg + kc) - kbeg);
  const int nblocks = (nrows + kBlock - 1) / kBlock;

  // Block b covers rows kbeg + 16b .. +15.  Resources are based at the
  // block, so byte offsets stay small (host checks ldx1, ldx2 < 2^25).
  // Every mask is an out-of-range offset: the loaded registers feed the
  // MFMAs directly, and a block past the chunk is all zeros (A and B).
  const uint32_t col_off = 4u * (uint32_t)col;
  const uint32_t a_off = 4u * (uint32_t)q * (uint32_t)ldx1 + 16u * (uint32_t)r;
  const bool a_row = q < M;
  auto load_block = [&](int b, Block& blk) {
    const int brow = 16 * b;  // wave-uniform, relative to kbeg
    const BufRsrc rx2 = make_rsrc(x2 + (int64_t)(kbeg + brow) * ldx2);
    const BufRsrc rx1 = make_rsrc(x1 + kbeg + brow);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int row = 4 * r + u;
      const bool ok = brow + row < nrows;
      const uint32_t roff = 4u * (uint32_t)row * (uint32_t)ldx2;
      if (VEC) {
        blk.b[u] = load_f32x4(rx2, (ok & col_ok) ? roff + col_off : kOob);
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c)
          blk.b[u][c] = load_f32(rx2, (ok & (col + c < N)) ? roff + col_off + 4u * c : kOob);
      }
    }
    if (VEC) {  // K % 4 == 0: the 4 rows of a quad are all valid or all past the chunk
      blk.a = load_f32x4(rx1, (a_row & (brow + 4 * r < nrows)) ? a_off : kOob);
    } else {
#pragma unroll
      for (int u = 0; u < 4; ++u) blk.a[u] = load_f32(rx1, (a_row & (brow + 4 * r + u < nrows)) ? a_off + 4u * u : kOob);
    }
  };

  f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = acc0, acc2 = acc0, acc3 = acc0;
  auto mma_block = [&](const Block& blk) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      acc0 = mfma16x16x4(blk.a[u], blk.b[u][0], acc0);
      acc1 = mfma16x16x4(blk.a[u], blk.b[u][1], acc1);
      acc2 = mfma16x16x4(blk.a[u], blk.b[u][2], acc2);
      acc3 = mfma16x16x4(blk.a[u], blk.b[u][3], acc3);
    }
  };

  // Batch i of this wave: blocks wave + (i*UB + j) * WAVES, j < UB.
  auto blk_id = [&](int i, int j) { return wave + (i * UB + j) * WAVES; };
  const int nmine = wave < nblocks ? (nblocks - wave + WAVES - 1) / WAVES : 0;
  const int nb = (nmine + UB - 1) / UB;

  // Two register sets used in turn: the next batch's loads are in flight
  // while the current batch's MFMAs run.  The body is one basic block and
  // sched_barrier keeps "issue the next batch, then the MFMAs of the current
  // one".  Loads past the chunk return zeros without memory traffic.
  Block A[UB], B[UB];
  if (nb > 0) {
#pragma unroll
    for (int j = 0; j < UB; ++j) load_block(blk_id(0, j), A[j]);
  }
  for (int i = 0; i + 1 < nb; i += 2) {
#pragma unroll
    for (int j = 0; j < UB; ++j) load_block(blk_id(i + 1, j), B[j]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < UB; ++j) mma_block(A[j]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < UB; ++j) load_block(blk_id(i + 2, j), A[j]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < UB; ++j) mma_block(B[j]);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (nb & 1) {
#pragma unroll
    for (int j = 0; j < UB; ++j) mma_block(A[j]);
  }

  // Lane l holds D_c[4r + v][q] in acc_c[v]: out row 4r+v, columns col..col+3.
#pragma unroll
  for (int v = 0; v < 4; ++v)
    red[(wave * kMaxM + 4 * r + v) * 16 + q] = f32x4{acc0[v], acc1[v], acc2[v], acc3[v]};
  __syncthreads();

  // The first 256 threads finish the slab, one (row m, quad cq) item each.
  const bool item = tid < kMaxM * 16;
  const int m = (tid >> 4) & (kMaxM - 1), cq = tid & 15;
  const int ocol = slab * kSlab + 4 * cq;
  const bool mine = item & (m < M);
  f32x4 sum = red[m * 16 + cq];
#pragma unroll
  for (int w = 1; w < WAVES; ++w) sum += red[(w * kMaxM + m) * 16 + cq];

  if (S == 1) {
    if (mine) store_quad<VEC>(out + (int64_t)m * ldo, ocol, N, sum);
    return;
  }

  // Split K: publish this workgroup's partial, count it in, and let the last
  // workgroup of the slab add the partials in split order.
  //
  // Cross-workgroup protocol without cache-wide fences.  An agent-scope
  // release/acquire fence would write back / invalidate this XCD's whole L2
  // (buffer_wbl2 / buffer_inv), and with hundreds of workgroups doing so the
  // tail dominated the kernel.  Instead the only data shared across
  // workgroups — the partials — are written and read with agent-coherent
  // (sc1) buffer accesses, the same cache policy agent-scope atomic loads and
  // stores use, so they bypass the non-coherent L2 state.  Each thread waits
  // for its partial store to complete (vmcnt(0)) before the barrier; wave 0
  // then bumps the slab's counter with an agent-scope atomic; the workgroup
  // that brings it to S reads the partials after seeing that value.
  const BufRsrc prs = make_rsrc(part + (int64_t)cell * kMaxM * kSlab);
  const uint32_t split_stride = 4u * (uint32_t)(gridDim.z * nslabs) * kMaxM * kSlab;  // bytes between splits
  const uint32_t item_off = 4u * (uint32_t)(m * kSlab + 4 * cq);
  if (mine) store_f32x4_coherent(prs, (uint32_t)split * split_stride + item_off, sum);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (wave == 0) {
    unsigned prev = 0;
    if (lane == 0)
      prev = __hip_atomic_fetch_add(&counters[cell * kCounterStride], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    prev = (unsigned)__shfl((int)prev, 0);
    if (lane == 0) last_flag = prev == (unsigned)(S - 1);
  }
  __syncthreads();
  if (!last_flag) return;

  // Partials of split sp for this cell start at (sp * cells + cell) * 1024
  // floats.  The M*16 live items are spread over the whole workgroup: thread
  // t = g*items + item adds the contiguous split range [g*S/G, (g+1)*S/G) of
  // its item, up to 8 loads in flight, so any S costs about one memory round
  // trip; the G group sums then meet in LDS and are added in group order.
  // The order of additions depends only on S, M and the block size.
  if (tid == 0) __hip_atomic_store(&counters[cell * kCounterStride], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const int items = M * 16;
  const int G = min(S, (WAVES * 64) / items);
  const int g = tid / items, it = tid - g * items;
  const int im = it >> 4, icq = it & 15;
  if (g < G) {
    const int s_beg = (g * S) / G, s_end = ((g + 1) * S) / G;
    const uint32_t off = 4u * (uint32_t)(im * kSlab + 4 * icq);
    f32x4 t = {0.f, 0.f, 0.f, 0.f};
    for (int s0 = s_beg; s0 < s_end; s0 += 8) {
      f32x4 v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j)
        v[j] = load_f32x4_coherent(prs, s0 + j < s_end ? (uint32_t)(s0 + j) * split_stride + off : kOob);
#pragma unroll
      for (int j = 0; j < 8; ++j) t += v[j];
    }
    red[tid] = t;  // red[g * items + it]; every read of red above finished before the last barrier
  }
  __syncthreads();
  if (tid < items) {
    f32x4 t = red[tid];
    for (int j = 1; j < G; ++j) t += red[j * items + tid];
    store_quad<VEC>(out + (int64_t)im * ldo, slab * kSlab + 4 * icq, N, t);
  }
}

template <int WAVES, int UB, bool VEC>
hipError_t launch_one(const MatmulArgs& a, const SkinnyGeom& g, unsigned* counters, float* part) {
  hipLaunchKernelGGL((skinny_f32_kernel<WAVES, UB, VEC>), dim3((unsigned)g.nslabs, (unsigned)g.splits, (unsigned)g.nrb),
                     dim3(WAVES * 64), 0, a.stream, static_cast<const float*>(a.x1),
                     static_cast<const float*>(a.x2), a.out, (int)a.M, (int)a.N, (int)a.K, a.ldx1, a.ldx2, a.ldo,
                     (int)g.kc, counters, part);
  return hipGetLastError();
}

template <int WAVES, int UB>
hipError_t launch_skinny(const MatmulArgs& a) {
  const SkinnyGeom g = skinny_geom(a.M, a.N, a.K, a.split_k);
  const bool vec = (a.N % 4 == 0) && (a.ldx2 % 4 == 0) && (a.ldo % 4 == 0) && (a.K % 4 == 0) &&
                   (a.ldx1 % 4 == 0) && (reinterpret_cast<uintptr_t>(a.x1) % 16 == 0) &&
                   (reinterpret_cast<uintptr_t>(a.x2) % 16 == 0) &&
                   (reinterpret_cast<uintptr_t>(a.out) % 16 == 0);
  unsigned* counters = g.splits > 1 ? a.counters : nullptr;
  float* part = g.splits > 1 ? static_cast<float*>(a.workspace) : nullptr;
  return vec ? launch_one<WAVES, UB, true>(a, g, counters, part)
             : launch_one<WAVES, UB, false>(a, g, counters, part);
}

}  // namespace

// Variant table for this family (its order is part of the variant numbering).
// BM = rows per row block, BN = slab width, BK = the largest K chunk of one
// workgroup, unroll = 16-row blocks per batch; max_m 0 = any M.
const VariantDesc* skinny_variants(int* count) {
  static const VariantDesc t[] = {
      {"skinny_f32_w4_b1", TILEC_FAMILY_SKINNY, TILEC_F32, kMaxM, kSlab, kKcMax, 4, 0, 1, launch_skinny<4, 1>},
      {"skinny_f32_w4_b2", TILEC_FAMILY_SKINNY, TILEC_F32, kMaxM, kSlab, kKcMax, 4, 0, 2, launch_skinny<4, 2>},
      {"skinny_f32_w8_b1", TILEC_FAMILY_SKINNY, TILEC_F32, kMaxM, kSlab, kKcMax, 8, 0, 1, launch_skinny<8, 1>},
      {"skinny_f32_w8_b2", TILEC_FAMILY_SKINNY, TILEC_F32, kMaxM, kSlab, kKcMax, 8, 0, 2, launch_skinny<8, 2>},
      {"skinny_f32_w16_b1", TILEC_FAMILY_SKINNY, TILEC_F32, kMaxM, kSlab, kKcMax, 16, 0, 1, launch_skinny<16, 1>},
  };
  *count = (int)(sizeof(t) / sizeof(t[0]));
  return t;
}

// Split K needs partials [splits][row blocks][slabs][16][64] fp32 (scratch)
// and one completion counter per (row block, slab), each on its own 256-byte
// line so workgroups of different cells do not contend on one line.
size_t skinny_counter_bytes(int64_t M, int64_t N, int64_t K, int split_k) {
  const SkinnyGeom g = skinny_geom(M, N, K, split_k);
  if (g.splits <= 1) return 0;
  return (size_t)g.nrb * g.nslabs * kCounterStride * sizeof(unsigned);
}
size_t skinny_workspace_bytes(int64_t M, int64_t N, int64_t K, int split_k) {
  const SkinnyGeom g = skinny_geom(M, N, K, split_k);
  if (g.splits <= 1) return 0;
  return (size_t)g.splits * g.nrb * g.nslabs * kMaxM * kSlab * sizeof(float);
}
int64_t skinny_effective_splits(int64_t N, int64_t K, int split_k) { return skinny_geom(1, N, K, split_k).splits; }

}  // namespace tilec
