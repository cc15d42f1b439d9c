// Output-stationary streaming kernel for products with a small output:
//   out[M,N] = x1[M,K] · x2[K,N]   (fp32 or bf16 in, fp32 out)
// built for M <= 16 (one 16-row block) and used for any M whose output is
// too small to fill the chip with tile-GEMM workgroups (each further 16 rows
// of x1 is one more row block of the grid).  bf16 inputs are widened to fp32
// exactly (a 16-bit shift) in registers, right before the MFMAs that use
// them, and run the same fp32 MFMAs: the kernel is bound by reading x2, and
// bf16 halves those bytes.
//
// Replaces, for small M, the reference's threadgroup-split dot product with a
// SIMD-group reduction (the legacy `_matrix_mul` described at README.md:57,73,
// whose config space survives in tilec/ext.py:29-51): here every lane owns a
// fixed group of output columns, so no reduction across lanes is needed for
// the columns, and x2 — the only large operand — is streamed from HBM exactly
// once with 16-byte coalesced loads.
//
// Mapping.  A lane's 16-byte load of an x2 row holds CPL columns (4 fp32 or
// 8 bf16); a workgroup owns a slab of 16*CPL output columns and one K split.
// K is cut into 16-row blocks; with row-major x2 and M <= 16, split s of S
// takes blocks s, s + S, s + 2S, ... (the workgroups in flight then read
// neighbouring x2 rows), otherwise a contiguous chunk of them; waves take
// interleaved blocks of their workgroup's share.  In a
// block, lane l (r = l / 16, q = l % 16) loads columns CPL*q .. of rows
// 4r + u, u = 0..3 (four 16-byte loads; each wave load covers four 256-byte
// row segments) and x1[q][4r .. 4r+3].  Row 4r + u is MFMA k-slot r of step
// u of v_mfma_f32_16x16x4f32, and each of the CPL columns feeds one MFMA:
//   D_c[m][q] += sum_r x1[m][4r+u] * x2[4r+u][SLAB*slab + CPL*q + c],
// the A operand being exactly the lane's x1 value for (m = q, k-slot r).
// Masking is done on addresses only: rows past K, columns past N and
// x1 rows past M get an out-of-range buffer offset and load zeros without
// touching memory, so loaded registers go straight into the MFMAs.  Per
// 4 KiB of x2 a wave issues 16 MFMAs for fp32 (512 cycles, 2.5x the rate the
// HBM share of a SIMD needs) and 32 for bf16 (1.25x), for any M <= 16.
//
// Column-major x2 (x @ W.T with W [N, K] row-major, read in place): a
// column of x2 is a contiguous run of K, so a block is the slab's 16*CPL
// columns by 4 E consecutive k (E = 4 fp32 or 8 bf16 per 16 bytes): lane l
// loads columns 16g + q (g < CPL) at k = E*r .. E*r + E-1 and x1[q][E*r ..].
// That is the MFMA A operand with x2's columns as its rows (A[i=q][k]) and
// x1 as the B operand (B[k][j=q]), so D_g[n][m] accumulates out^T; bf16
// needs no widening here, the 8 consecutive k of a lane being exactly the
// v_mfma_f32_16x16x32_bf16 operand.  Lane l then holds out[q][16g + 4r ..
// 16g + 4r + 3], which is one float4 item of the same LDS reduction.  A wave
// load covers 16 columns x 64 bytes; the waves' interleaved blocks make up
// contiguous runs.  Column-major x1 is read element by element (it is small
// and cache-resident).
//
// Grid: x = slabs of 16*CPL columns, y = K splits, z = 16-row blocks of x1
// and out.
//
// x @ W.T with M <= 16 has two more kernels below, neither with a K split:
// gemv_rows_kernel (one wave per row of W over all of K, FMAs, M <= 4) and
// gemv_wt_kernel (16 rows of W per workgroup over all of K, MFMAs fed
// through LDS).
// Waves are summed through LDS; with a split K each workgroup writes its
// [16 x SLAB] partial to the workspace, and the last workgroup of a (row
// block, slab) to finish (completion counter) adds the partials in split
// order, so results do not depend on scheduling; it resets the counter to
// zero.
#include <type_traits>

#include "common.h"
#include "../../include/tilec.h"

namespace tilec {

namespace {

constexpr int kMaxM = 16;      // MFMA rows
constexpr int kBlock = 16;     // K chunks are whole multiples of 16 rows
constexpr int kKcMax = 1024;   // rows per K chunk at most
constexpr int kCounterStride = 64;  // uint32s between completion counters (own 256-byte line each)
// Cache policy of the x2 loads: non-temporal, as x2 is streamed once (the
// hint took 6-10 % off the fp32 GEMV at K = N = 4096).
constexpr int kCpolX2 = 2;

typedef unsigned short u16;  // bf16 bit pattern
typedef int i32x2 __attribute__((ext_vector_type(2)));

// Element type: CPL columns per 16-byte row load, slab = 16 * CPL columns,
// NQ = CPL / 4 output float4 per lane and row, E elements per 16 bytes.
template <typename T>
struct Elem;
template <>
struct Elem<float> {
  static constexpr int CPL = 4, BYTES = 4;
};
template <>
struct Elem<u16> {
  static constexpr int CPL = 8, BYTES = 2;
};
template <typename T>
constexpr int kSlabOf = 16 * Elem<T>::CPL;

// One block of a wave's share of x2 and the x1 values it multiplies.
//   x2 row-major (CB = false): x2 rows 4r + u (u < 4), CPL columns each, and
//     x1[q][4r .. 4r+3]; the block covers 16 rows of K.
//   x2 column-major (CB = true): columns 16g + q (g < CPL) of x2, E
//     consecutive k each (k = E*r ..), and x1[q][E*r .. E*r + E-1]; the block
//     covers 4E rows of K.
// bf16 values are kept as raw pairs (low half = lower column / k).
template <typename T, bool CB>
struct Blk;
template <>
struct Blk<float, false> {
  static constexpr int KB = 16;
  f32x4 b[4];
  f32x4 a;
};
template <>
struct Blk<u16, false> {
  static constexpr int KB = 16;
  i32x4 b[4];
  i32x2 a;
};
template <>
struct Blk<float, true> {
  static constexpr int KB = 16;
  f32x4 b[4];
  f32x4 a;
};
template <>
struct Blk<u16, true> {
  static constexpr int KB = 32;
  i32x4 b[8];
  i32x4 a;
};

// FMA path (MV > 0, row-major x2 only): the same x2 block and, for each of
// the MV output rows m, x1[m][4r .. 4r+3] (every lane needs every row).
template <typename T, int MV>
struct BlkV;
template <int MV>
struct BlkV<float, MV> {
  static constexpr int KB = 16;
  f32x4 b[4];
  f32x4 a[MV];
};
template <int MV>
struct BlkV<u16, MV> {
  static constexpr int KB = 16;
  i32x4 b[4];
  i32x2 a[MV];
};

__device__ __forceinline__ float bf16_lo(int w) { return __int_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(int w) { return __int_as_float(w & (int)0xffff0000u); }

struct SkinnyGeom {
  int64_t nslabs, splits, kc, nrb;
};

// K chunk per split: a multiple of kBlock rows, at most kKcMax; the number of
// splits is raised to what kKcMax needs and recomputed so that none is empty.
// Column-major x2, and row-major x2 with more than one 16-row block of x1,
// read each split's chunk; row-major x2 with M <= 16 only uses the split
// count (its splits take interleaved blocks, kc rows each give or take one
// block, and none is empty since splits <= cdiv(K, kBlock)).
SkinnyGeom skinny_geom(int64_t M, int64_t N, int64_t K, int split_k, int slab) {
  SkinnyGeom g;
  g.nslabs = cdiv(N, slab);
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

// MV = 0: MFMA path (any M <= 16 per row block).  MV in 1..4: FMA path for
// M <= MV with row-major x2 — lane (r, q) accumulates out[m][col + c] over
// its own rows 4r + u of each block in plain FMAs, and the four lanes of a
// column group (r = 0..3) meet in the LDS reduction as four more "waves".
// Per 4 KiB of x2 a wave then spends 16 MV FMAs (fp32) where the MFMA path
// issues 16 MFMAs of 8 passes, and bf16 needs no widening to 32 MFMAs.
template <typename T, int WAVES, int UB, bool VEC, bool CA, bool CB, int MV>
__global__ __launch_bounds__(WAVES * 64) void skinny_kernel(
    const T* __restrict__ x1, const T* __restrict__ x2, float* __restrict__ out,
    int M_all, int N, int K, int64_t ldx1, int64_t ldx2, int64_t ldo, int kc,
    unsigned* __restrict__ counters, float* __restrict__ part) {
  static_assert(MV >= 0 && MV <= 4 && (MV == 0 || !CB), "FMA path: M <= 4, row-major x2");
  using E = Elem<T>;
  using Block = std::conditional_t<(MV > 0), BlkV<T, (MV > 0 ? MV : 1)>, Blk<T, CB>>;
  constexpr int CPL = E::CPL, NQ = CPL / 4, SLAB = kSlabOf<T>, NT = WAVES * 64;
  constexpr int EPL = 16 / E::BYTES;  // elements per 16-byte load
  constexpr int KB = Block::KB;       // rows of K per block
  constexpr uint32_t EB = E::BYTES;
  __shared__ f32x4 red[WAVES * kMaxM * 16 * NQ];  // [wave][row][lane column group q][h]
  __shared__ int last_flag;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int r = lane >> 4, q = lane & 15;
  const int slab = blockIdx.x, split = blockIdx.y, rb = blockIdx.z;
  const int nslabs = gridDim.x, S = gridDim.y;
  // This workgroup's row block: rows 16*rb .. of x1 and out, M of them.
  const int M = min(kMaxM, M_all - kMaxM * rb);
  x1 += CA ? (int64_t)kMaxM * rb : (int64_t)kMaxM * rb * ldx1;
  out += (int64_t)kMaxM * rb * ldo;
  const int cell = rb * nslabs + slab;  // (row block, slab): partial slot and counter
  const int n0 = slab * SLAB;
  const int col = n0 + CPL * q;
  const bool col_ok = col < N;
  // Blocks of this split.  Row-major x2 with one row block (M <= 16): split
  // s takes the KB-row blocks s, s + S, s + 2S, ... of K, so the workgroups
  // in flight read one window of S neighbouring blocks of x2 rather than S
  // chunks far apart (a single 64 MiB read pass measured ~1 us faster in
  // that order).  Otherwise the contiguous chunk kbeg .. kbeg + kc: with
  // more row blocks x1 is large, and interleaved 16-row blocks would cut its
  // rows into 64-byte pieces whose 128-byte lines two splits both fetch.
  const bool inter = !CB && gridDim.z == 1;  // workgroup-uniform
  const int kbeg = split * kc;
  const int nrows = max(0, min(K, kbeg + kc) - kbeg);
  const int kblocks = (K + KB - 1) / KB;
  const int nblocks = inter ? (split < kblocks ? (kblocks - split + S - 1) / S : 0) : (nrows + KB - 1) / KB;
  // First row of block b and the rows of K left from there (<= 0: past the
  // end; such blocks load zeros).
  auto blk_row = [&](int b) -> int { return inter ? KB * (b * S + split) : kbeg + KB * b; };
  auto blk_lim = [&](int b) -> int { return inter ? K - KB * (b * S + split) : nrows - KB * b; };

  // Resources are based at the block, so byte offsets stay small (the host
  // bounds ldx1 and ldx2).  Every mask is an out-of-range offset: the loaded
  // registers feed the MFMAs directly, and a block past the split's share is
  // all zeros (A and B).
  const uint32_t col_off = EB * (uint32_t)col;
  const bool a_row = q < M;
  // x1 element (row q, k = block row + kr) of this lane: 0 if masked.
  auto x1_off = [&](int lim, int kr) -> uint32_t {
    if (!(a_row & (kr < lim))) return kOob;
    return CA ? EB * ((uint32_t)kr * (uint32_t)ldx1 + (uint32_t)q) : EB * ((uint32_t)q * (uint32_t)ldx1 + (uint32_t)kr);
  };
  auto x1_rsrc = [&](int k0) {
    return make_rsrc(CA ? x1 + (int64_t)k0 * ldx1 : x1 + k0);
  };
  // Dword w of a 16-byte group from its elements' bit patterns h[].
  auto pack = [](const int* h, int w) -> int { return E::BYTES == 4 ? h[w] : (h[2 * w] | (h[2 * w + 1] << 16)); };
  auto put = [&](auto& v, const int* h) __attribute__((always_inline)) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      if constexpr (E::BYTES == 4) v[w] = __builtin_bit_cast(float, pack(h, w));
      else v[w] = pack(h, w);
    }
  };
  auto ld_elem = [&](const BufRsrc& rs, uint32_t o) -> int {
    if constexpr (E::BYTES == 4) return __builtin_bit_cast(int, load_f32(rs, o));
    else return (int)__builtin_amdgcn_raw_buffer_load_b16(rs, (int)o, 0, 0);
  };
  auto load_block = [&](int b, Block& blk) __attribute__((always_inline)) {
    const int k0 = blk_row(b), lim = blk_lim(b);  // wave-uniform
    const BufRsrc rx1 = x1_rsrc(k0);
    if constexpr (!CB) {
      const BufRsrc rx2 = make_rsrc(x2 + (int64_t)k0 * ldx2);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int row = 4 * r + u;
        const bool ok = row < lim;
        const uint32_t roff = EB * (uint32_t)row * (uint32_t)ldx2;
        if constexpr (VEC) {
          const uint32_t o = (ok & col_ok) ? roff + col_off : kOob;
          if constexpr (CPL == 4) blk.b[u] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rx2, (int)o, 0, kCpolX2));
          else blk.b[u] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(rx2, (int)o, 0, kCpolX2));
        } else {
          int h[CPL];
#pragma unroll
          for (int c = 0; c < CPL; ++c) h[c] = ld_elem(rx2, (ok & (col + c < N)) ? roff + col_off + EB * c : kOob);
          put(blk.b[u], h);
        }
      }
      if constexpr (MV > 0) {
        // x1[m][4r .. 4r+3] for every row m < MV: 0 past M or past K
#pragma unroll
        for (int m = 0; m < (MV > 0 ? MV : 1); ++m) {
          auto off = [&](int kr) -> uint32_t {
            if (!((m < M) & (kr < lim))) return kOob;
            return CA ? EB * ((uint32_t)kr * (uint32_t)ldx1 + (uint32_t)m) : EB * ((uint32_t)m * (uint32_t)ldx1 + (uint32_t)kr);
          };
          if constexpr (VEC && !CA) {
            if constexpr (CPL == 4) blk.a[m] = load_f32x4(rx1, off(4 * r));
            else blk.a[m] = __builtin_bit_cast(i32x2, __builtin_amdgcn_raw_buffer_load_b64(rx1, (int)off(4 * r), 0, 0));
          } else {
            int h[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) h[u] = ld_elem(rx1, off(4 * r + u));
            if constexpr (CPL == 4) {
              put(blk.a[m], h);
            } else {
              blk.a[m][0] = h[0] | (h[1] << 16);
              blk.a[m][1] = h[2] | (h[3] << 16);
            }
          }
        }
      } else if constexpr (VEC && !CA) {  // x1[q][4r .. 4r+3]; K % 4 == 0: the 4 k of a lane are all valid or all past K
        const uint32_t o = x1_off(lim, 4 * r);
        if constexpr (CPL == 4) blk.a = load_f32x4(rx1, o);
        else blk.a = __builtin_bit_cast(i32x2, __builtin_amdgcn_raw_buffer_load_b64(rx1, (int)o, 0, 0));
      } else {
        int h[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) h[u] = ld_elem(rx1, x1_off(lim, 4 * r + u));
        if constexpr (CPL == 4) {
          put(blk.a, h);
        } else {
          blk.a[0] = h[0] | (h[1] << 16);
          blk.a[1] = h[2] | (h[3] << 16);
        }
      }
    } else {
      // x2 column-major: columns n0 + 16g + q, k = k0 + EPL*r ..
      const BufRsrc rx2 = make_rsrc(x2 + (int64_t)n0 * ldx2 + k0);
      const int kr = EPL * r;
#pragma unroll
      for (int g = 0; g < CPL; ++g) {
        const int n = 16 * g + q;
        const bool nok = n0 + n < N;
        const uint32_t noff = EB * ((uint32_t)n * (uint32_t)ldx2 + (uint32_t)kr);
        if constexpr (VEC) {  // K % EPL == 0: a lane's EPL k are all valid or all past the chunk
          const uint32_t o = (nok & (kr < lim)) ? noff : kOob;
          blk.b[g] = __builtin_bit_cast(decltype(blk.a), __builtin_amdgcn_raw_buffer_load_b128(rx2, (int)o, 0, kCpolX2));
        } else {
          int h[EPL];
#pragma unroll
          for (int e = 0; e < EPL; ++e) h[e] = ld_elem(rx2, (nok & (kr + e < lim)) ? noff + EB * e : kOob);
          put(blk.b[g], h);
        }
      }
      // x1[q][kr .. kr + EPL-1]
      if constexpr (VEC && !CA) {
        blk.a = __builtin_bit_cast(decltype(blk.a), __builtin_amdgcn_raw_buffer_load_b128(rx1, (int)x1_off(lim, kr), 0, 0));
      } else {
        int h[EPL];
#pragma unroll
        for (int e = 0; e < EPL; ++e) h[e] = ld_elem(rx1, x1_off(lim, kr + e));
        put(blk.a, h);
      }
    }
  };

  f32x4 acc[CPL];
#pragma unroll
  for (int c = 0; c < CPL; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
  constexpr int MVA = MV > 0 ? MV : 1;
  f32x4 accv[MVA][NQ];  // FMA path: out[m][col + 4h .. +3] over this lane's rows
#pragma unroll
  for (int m = 0; m < MVA; ++m)
#pragma unroll
    for (int h = 0; h < NQ; ++h) accv[m][h] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto mma_block = [&](const Block& blk) __attribute__((always_inline)) {
    if constexpr (MV > 0) {
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int m = 0; m < MVA; ++m) {
          float a;
          if constexpr (CPL == 4) a = blk.a[m][u];
          else a = (u & 1) ? bf16_hi(blk.a[m][u >> 1]) : bf16_lo(blk.a[m][u >> 1]);
#pragma unroll
          for (int cc = 0; cc < CPL; ++cc) {
            float b;
            if constexpr (CPL == 4) b = blk.b[u][cc];
            else b = (cc & 1) ? bf16_hi(blk.b[u][cc >> 1]) : bf16_lo(blk.b[u][cc >> 1]);
            accv[m][cc / 4][cc % 4] = __builtin_fmaf(a, b, accv[m][cc / 4][cc % 4]);
          }
        }
    } else if constexpr (!CB && CPL == 8) {
      // bf16: the lane's rows 4r + u (u < 4) of column col + c are the B
      // operand of a 16x16x16 bf16 MFMA (k = 4r + u) and x1[q][4r .. 4r+3]
      // its A operand, so a block is CPL MFMAs on bf16 pairs packed by byte
      // permutes, with no widening to fp32.
      //   D_c[m][q] += sum_{r,u} x1[m][4r+u] * x2[4r+u][col + c]
      const s16x4 a = __builtin_bit_cast(s16x4, blk.a);
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const unsigned sel = (c & 1) ? 0x07060302u : 0x05040100u;  // high or low halves of two dwords
        const int lo = (int)__builtin_amdgcn_perm((unsigned)blk.b[1][c >> 1], (unsigned)blk.b[0][c >> 1], sel);
        const int hi = (int)__builtin_amdgcn_perm((unsigned)blk.b[3][c >> 1], (unsigned)blk.b[2][c >> 1], sel);
        acc[c] = mfma16x16x16bf16(a, __builtin_bit_cast(s16x4, i32x2{lo, hi}), acc[c]);
      }
    } else if constexpr (!CB) {
      // D_c[m][q] += sum_r x1[m][4r+u] * x2[4r+u][col + c]
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        float a;
        if constexpr (CPL == 4) a = blk.a[u];
        else a = (u & 1) ? bf16_hi(blk.a[u >> 1]) : bf16_lo(blk.a[u >> 1]);
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
          float b;
          if constexpr (CPL == 4) b = blk.b[u][c];
          else b = (c & 1) ? bf16_hi(blk.b[u][c >> 1]) : bf16_lo(blk.b[u][c >> 1]);
          acc[c] = mfma16x16x4(a, b, acc[c]);
        }
      }
    } else if constexpr (CPL == 4) {
      // D_g[n][m] += sum_r x2[4r+c][n0 + 16g + n] * x1[m][4r+c]: x2's column
      // block is the A operand (A[i=q][k=r]), x1 the B operand (B[k=r][j=q]).
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[g] = mfma16x16x4(blk.b[g][c], blk.a[c], acc[g]);
    } else {
      // bf16: 8 consecutive k per lane is the 16x16x32 bf16 operand layout.
#pragma unroll
      for (int g = 0; g < CPL; ++g)
        acc[g] = mfma16x16x32bf16(__builtin_bit_cast(bf16x8, blk.b[g]), __builtin_bit_cast(bf16x8, blk.a), acc[g]);
    }
  };

  // Batch i of this wave: blocks wave + (i*UB + j) * WAVES, j < UB.
  auto blk_id = [&](int i, int j) { return wave + (i * UB + j) * WAVES; };
  const int nmine = wave < nblocks ? (nblocks - wave + WAVES - 1) / WAVES : 0;
  const int nb = (nmine + UB - 1) / UB;

  // Two register sets used in turn: the next batch's loads are in flight
  // while the current batch's MFMAs run.  The body is one basic block and
  // sched_barrier keeps "issue the next batch, then the MFMAs of the current
  // one".  Loads past the split's share return zeros without memory traffic.
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

  // Item (row m, column group q, half h) holds out[m][n0 + CPL*q + 4h .. +3].
  // The FMA path has kRows = MV rows and kVW = 4 WAVES partials per item
  // (lane rows r = 0..3 of every wave).
  constexpr int kRows = MV > 0 ? MV : kMaxM;
  constexpr int kVW = MV > 0 ? 4 * WAVES : WAVES;
  if constexpr (MV > 0) {
#pragma unroll
    for (int m = 0; m < MVA; ++m)
#pragma unroll
      for (int h = 0; h < NQ; ++h) red[(((wave * 4 + r) * kRows + m) * 16 + q) * NQ + h] = accv[m][h];
  } else if constexpr (!CB) {
    // Lane l holds D_c[4r + v][q] in acc[c][v]: out row 4r+v, column col + c.
#pragma unroll
    for (int v = 0; v < 4; ++v)
#pragma unroll
      for (int h = 0; h < NQ; ++h)
        red[((wave * kMaxM + 4 * r + v) * 16 + q) * NQ + h] =
            f32x4{acc[4 * h][v], acc[4 * h + 1][v], acc[4 * h + 2][v], acc[4 * h + 3][v]};
  } else {
    // Lane l holds D_g[4r + v][q] in acc[g][v]: out row q, column n0 + 16g + 4r + v.
#pragma unroll
    for (int g = 0; g < CPL; ++g) {
      const int c = 16 * g + 4 * r;
      red[((wave * kMaxM + q) * 16 + c / CPL) * NQ + (c % CPL) / 4] = acc[g];
    }
  }
  __syncthreads();

  // Output items: (row m, column group q, half h) -> 4 columns at
  // SLAB*slab + CPL*q + 4h; 256*NQ of them, spread over the workgroup.
  constexpr int kItems = kRows * 16 * NQ;
  static_assert(kVW * kItems <= WAVES * kMaxM * 16 * NQ, "red holds every partial");
  auto item_sum = [&](int it) {
    f32x4 v = red[it];
#pragma unroll
    for (int w = 1; w < kVW; ++w) v += red[w * kItems + it];
    return v;
  };
  auto item_col = [&](int it) { return slab * SLAB + CPL * ((it / NQ) % 16) + 4 * (it % NQ); };

  if (S == 1) {
    for (int it = tid; it < kItems; it += NT) {
      const int m = it / (16 * NQ);
      if (m < M) store_quad<VEC>(out + (int64_t)m * ldo, item_col(it), N, item_sum(it));
    }
    return;
  }

  // Split K: publish this workgroup's partial, count it in, and let the last
  // workgroup of the cell add the partials in split order.
  //
  // Cross-workgroup protocol without cache-wide fences.  An agent-scope
  // release/acquire fence would write back / invalidate this XCD's whole L2
  // (buffer_wbl2 / buffer_inv), and with hundreds of workgroups doing so the
  // tail dominated the kernel.  Instead the only data shared across
  // workgroups — the partials — are written and read with agent-coherent
  // (sc1) buffer accesses, the same cache policy agent-scope atomic loads and
  // stores use, so they bypass the non-coherent L2 state.  Each thread waits
  // for its partial stores to complete (vmcnt(0)) before the barrier; wave 0
  // then bumps the cell's counter with an agent-scope atomic; the workgroup
  // that brings it to S reads the partials after seeing that value.
  // Partial of split sp for this cell: kItems float4 at (sp * cells + cell).
  const BufRsrc prs = make_rsrc(part + (int64_t)cell * kItems * 4);
  const uint32_t split_stride = 16u * (uint32_t)(gridDim.z * nslabs) * kItems;  // bytes between splits
  for (int it = tid; it < kItems; it += NT) {
    const int m = it / (16 * NQ);
    if (m < M) store_f32x4_coherent(prs, (uint32_t)split * split_stride + 16u * it, item_sum(it));
  }
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

  // The M*16*NQ live items are spread over the whole workgroup: unit
  // u = g*items + item adds the contiguous split range [g*S/G, (g+1)*S/G)
  // of its item, up to 8 loads in flight, so any S costs about one memory
  // round trip; the G group sums then meet in LDS (red, whose reads all
  // finished before the last barrier) and are added in group order.  The
  // order of additions depends only on S, M and the block size.
  if (tid == 0) __hip_atomic_store(&counters[cell * kCounterStride], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const int items = M * 16 * NQ;
  const int G = max(1, min(S, NT / items));
  for (int u = tid; u < items * G; u += NT) {
    const int g = u / items, it = u - g * items;
    const int s_beg = (g * S) / G, s_end = ((g + 1) * S) / G;
    f32x4 t = {0.f, 0.f, 0.f, 0.f};
    for (int s0 = s_beg; s0 < s_end; s0 += 8) {
      f32x4 v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j)
        v[j] = load_f32x4_coherent(prs, s0 + j < s_end ? (uint32_t)(s0 + j) * split_stride + 16u * it : kOob);
#pragma unroll
      for (int j = 0; j < 8; ++j) t += v[j];
    }
    red[u] = t;
  }
  __syncthreads();
  for (int it = tid; it < items; it += NT) {
    f32x4 t = red[it];
    for (int g = 1; g < G; ++g) t += red[g * items + it];
    store_quad<VEC>(out + (int64_t)(it / (16 * NQ)) * ldo, item_col(it), N, t);
  }
}

template <typename T, int WAVES, int UB, bool VEC, bool CA, bool CB, int MV>
hipError_t launch_one(const MatmulArgs& a, const SkinnyGeom& g, unsigned* counters, float* part) {
  hipLaunchKernelGGL((skinny_kernel<T, WAVES, UB, VEC, CA, CB, MV>), dim3((unsigned)g.nslabs, (unsigned)g.splits, (unsigned)g.nrb),
                     dim3(WAVES * 64), 0, a.stream, static_cast<const T*>(a.x1), static_cast<const T*>(a.x2), a.out,
                     (int)a.M, (int)a.N, (int)a.K, a.ldx1, a.ldx2, a.ldo, (int)g.kc, counters, part);
  return hipGetLastError();
}

template <typename T, int WAVES, int UB, bool CA, bool CB, int MV>
hipError_t launch_layout(const MatmulArgs& a, const SkinnyGeom& g, unsigned* counters, float* part) {
  constexpr int CPL = Elem<T>::CPL, EPL = 16 / (int)sizeof(T);
  auto aligned = [](const void* p, size_t n) { return reinterpret_cast<uintptr_t>(p) % n == 0; };
  // Vector path: 16-byte loads of x2 that never straddle an edge (CPL
  // columns of a row, or EPL k of a column), x1 loads of 4 (row-major x2) or
  // EPL (column-major x2) consecutive k when x1 is row-major, float4 stores.
  bool vec = a.ldo % 4 == 0 && aligned(a.out, 16) && aligned(a.x2, 16);
  if constexpr (!CB)
    vec = vec && a.N % CPL == 0 && a.ldx2 % CPL == 0 &&
          (CA || (a.K % 4 == 0 && a.ldx1 % 4 == 0 && aligned(a.x1, 4 * sizeof(T))));
  else
    vec = vec && a.N % 4 == 0 && a.K % EPL == 0 && a.ldx2 % EPL == 0 &&
          (CA || (a.ldx1 % EPL == 0 && aligned(a.x1, 16)));
  // The FMA path takes row-major x2; a column-major x2 runs the MFMA path.
  constexpr int MVL = CB ? 0 : MV;
  return vec ? launch_one<T, WAVES, UB, true, CA, CB, MVL>(a, g, counters, part)
             : launch_one<T, WAVES, UB, false, CA, CB, MVL>(a, g, counters, part);
}

template <typename T, int WAVES, int UB, int MV = 0>
hipError_t launch_skinny(const MatmulArgs& a) {
  const SkinnyGeom g = skinny_geom(a.M, a.N, a.K, a.split_k, kSlabOf<T>);
  unsigned* counters = g.splits > 1 ? a.counters : nullptr;
  float* part = g.splits > 1 ? static_cast<float*>(a.workspace) : nullptr;
  switch (a.layout & 3) {
    case 0: return launch_layout<T, WAVES, UB, false, false, MV>(a, g, counters, part);
    case TILEC_X1_COL_MAJOR: return launch_layout<T, WAVES, UB, true, false, MV>(a, g, counters, part);
    case TILEC_X2_COL_MAJOR: return launch_layout<T, WAVES, UB, false, true, MV>(a, g, counters, part);
    default: return launch_layout<T, WAVES, UB, true, true, MV>(a, g, counters, part);
  }
}

// ---------------------------------------------------------------------------
// Row-dot kernel for x @ W.T: x2 column-major, i.e. the rows of W [N, K]
// (row stride ldx2) are the columns of x2, and out[m][n] = sum_k x1[m][k] *
// W[n][k].  Each wave owns RPW rows of W (RPW output columns) for the whole
// of K, so there is no K split and no cross-workgroup combine: a row is a
// contiguous run of K elements, read in 1 KiB wave loads (lane l takes
// elements EPL*l .. of each 64*EPL chunk), dotted with the matching x1
// pieces in FMAs (M <= MR rows of x1, row-major, from the cache), and the 64
// lanes meet in a butterfly at the end.  Rows past N and elements past K are
// masked by the buffer resources' extents (one resource per row, num_records
// = K elements): they load zeros.  W is read with the non-temporal cache
// policy CP (streamed once); x1 stays cached.  No LDS, no barriers.
//
// AL: every row starts on a 16-byte boundary (K, both strides and both
// bases aligned).  Otherwise (any element alignment) each row's resource
// starts at the 16-byte boundary below the row and ends at the one above
// its last element, and a wave load covers 63 lanes' worth of the row
// (chunks 1008 bytes apart, overlapping by 16): lane l < 63 loads the
// aligned 16 bytes at 16 l, takes lane l + 1's with a lane shuffle, and
// shifts the pair into place by the row's byte misalignment (funnel16);
// lane 63 only supplies its load.  Elements past K, which now share a chunk
// with the next row, are cleared in both operands.  No load leaves the
// row's own 16-byte chunks.
// ---------------------------------------------------------------------------
template <typename T, int MR, int RPW, int WAVES, int U, int CP, bool AL>
__global__ __launch_bounds__(WAVES * 64) void gemv_rows_kernel(const T* __restrict__ x1, const T* __restrict__ w,
                                                               float* __restrict__ out, int M, int N, int K,
                                                               int64_t ldx1, int64_t ldw, int64_t ldo) {
  constexpr int EPL = 16 / (int)sizeof(T);  // elements per 16-byte load
  constexpr int CH = (AL ? 64 : 63) * EPL;  // K elements per wave load
  typedef std::conditional_t<sizeof(T) == 4, f32x4, i32x4> V;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row0 = (blockIdx.x * WAVES + wave) * RPW;
  if (row0 >= N) return;
  const uint32_t kbytes = (uint32_t)K * sizeof(T);
  BufRsrc rw[RPW], rx[MR];
  uint32_t bw[RPW], bx[MR];  // byte misalignment of each row (AL: 0)
  auto row_rsrc = [&](const T* p, bool ok, uint32_t& b) -> BufRsrc {
    if constexpr (AL) {
      b = 0;
      return make_rsrc(p, ok ? kbytes : 0u);
    } else {
      const uintptr_t s = reinterpret_cast<uintptr_t>(p);
      b = (uint32_t)(s & 15);
      return make_rsrc(reinterpret_cast<const void*>(s - b), ok ? (b + kbytes + 15u) & ~15u : 0u);
    }
  };
#pragma unroll
  for (int r = 0; r < RPW; ++r) rw[r] = row_rsrc(w + (int64_t)(row0 + r) * ldw, row0 + r < N, bw[r]);
#pragma unroll
  for (int m = 0; m < MR; ++m) rx[m] = row_rsrc(x1 + (int64_t)m * ldx1, m < M, bx[m]);
  auto ld = [&](const BufRsrc& rs, uint32_t off) -> V {
    return __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)off, 0, 0));
  };
  auto ld_w = [&](const BufRsrc& rs, uint32_t off) -> V {
    return __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)off, 0, CP));
  };
  auto elem = [](const V& v, int e) -> float {
    if constexpr (sizeof(T) == 4) return v[e];
    else return (e & 1) ? bf16_hi(v[e >> 1]) : bf16_lo(v[e >> 1]);
  };
  struct Batch {
    V w[U][RPW], x[U][MR];
  };
  float acc[RPW][MR];
#pragma unroll
  for (int r = 0; r < RPW; ++r)
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[r][m] = 0.f;
  const uint32_t lane_off = 16u * (uint32_t)lane;
  auto load = [&](int c0, Batch& b) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      // chunk c0 + u; past K every element is masked (offset >= extent)
      const uint32_t off = (uint32_t)(c0 + u) * (uint32_t)CH * sizeof(T) + lane_off;
#pragma unroll
      for (int r = 0; r < RPW; ++r) b.w[u][r] = ld_w(rw[r], off);
#pragma unroll
      for (int m = 0; m < MR; ++m) b.x[u][m] = ld(rx[m], off);
    }
  };
  // The 16 bytes a lane uses (AL: as loaded).
  auto use = [&](const V& v, uint32_t b, int kvalid) -> V {
    if constexpr (AL) {
      return v;
    } else {
      const u32x4 lo = __builtin_bit_cast(u32x4, v);
      u32x4 hi;
#pragma unroll
      for (int j = 0; j < 4; ++j) hi[j] = (uint32_t)__shfl_down((int)lo[j], 1);
      u32x4 x = funnel16(lo, hi, b);
      if (kvalid < EPL) x = keep_bytes(x, kvalid * (int)sizeof(T));
      return __builtin_bit_cast(V, x);
    }
  };
  auto fma = [&](int c0, const Batch& b) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      // elements of this lane's 16 bytes inside K (the unaligned form's lane
      // 63 has none of its own)
      const int kvalid = (!AL && lane == 63) ? 0 : K - (c0 + u) * CH - EPL * lane;
      V wv[RPW], xv[MR];
#pragma unroll
      for (int r = 0; r < RPW; ++r) wv[r] = use(b.w[u][r], bw[r], kvalid);
#pragma unroll
      for (int m = 0; m < MR; ++m) xv[m] = use(b.x[u][m], bx[m], kvalid);
#pragma unroll
      for (int e = 0; e < EPL; ++e)
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          const float xe = elem(xv[m], e);
#pragma unroll
          for (int r = 0; r < RPW; ++r) acc[r][m] = __builtin_fmaf(elem(wv[r], e), xe, acc[r][m]);
        }
    }
  };
  const int nch = (K + CH - 1) / CH;
  const int nb = (nch + U - 1) / U;
  Batch A, B;
  if (nb > 0) load(0, A);
  for (int i = 0; i + 1 < nb; i += 2) {
    load((i + 1) * U, B);
    __builtin_amdgcn_sched_barrier(0);
    fma(i * U, A);
    __builtin_amdgcn_sched_barrier(0);
    load((i + 2) * U, A);
    __builtin_amdgcn_sched_barrier(0);
    fma((i + 1) * U, B);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (nb & 1) fma((nb - 1) * U, A);
  // Butterfly over the 64 lanes; every lane ends with the full sums.
#pragma unroll
  for (int r = 0; r < RPW; ++r)
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      float v = acc[r][m];
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
      acc[r][m] = v;
    }
  // Lane r * MR + m stores out[m][row0 + r].
#pragma unroll
  for (int r = 0; r < RPW; ++r)
#pragma unroll
    for (int m = 0; m < MR; ++m)
      if (lane == r * MR + m && m < M && row0 + r < N) out[(int64_t)m * ldo + row0 + r] = acc[r][m];
}

// ---------------------------------------------------------------------------
// Row-tile kernel for x @ W.T with up to 16 rows of x1: the MFMA counterpart
// of the row-dot kernel.  A workgroup owns R rows of W (R output columns,
// R <= 16) for the whole of K; its waves take interleaved K chunks of CHB
// bytes per row and meet once, in LDS, at the end: no K split, no partials.
//
// The MFMA wants W as its A operand with one W row per lane group (A[i][k]
// on lane i + 16 * (k-slot group)), which a coalesced load of a W row does
// not give.  So each wave reads its chunk of the R rows with contiguous
// CHB-byte wave loads (lane l: bytes 16 * (l % LPR) of row l / LPR of the
// load) into registers, writes them to its own LDS area (rows CHB + 16 bytes
// apart: the 16-byte skew makes the operand reads below conflict-free), and
// reads them back as MFMA operands: for each 64-byte k group t of the chunk,
// lane l reads 16 bytes of row l % 16 at byte 64 t + 16 (l / 16).  The
// matching x1 pieces, x1[l % 16][same k], are the B operand, so D[i][j]
// accumulates out[j][n0 + i]:
//   fp32: the 16 bytes are k = 4 g + u (g = l / 16, u < 4), one
//         v_mfma_f32_16x16x4f32 per u;
//   bf16: the 16 bytes are 8 consecutive k, one v_mfma_f32_16x16x32_bf16.
// Which k meets which MFMA slot does not matter to the sum as long as A and B
// agree, and they do (same byte offsets in W's row and x1's row).
//
// x1 takes the same route as W: loaded as whole CHB-byte row pieces (8 or 4
// rows of 128 or 256 bytes per wave load), staged in a second LDS area and
// read back in the operand layout.  Read directly in that layout, each load
// of x1 would touch 16 rows at 64 bytes each — twice the cache lines per
// byte of a W load — and every workgroup reads all of x1 from the L2 (as
// many bytes as it reads of W at M = 16).  And workgroup b of G starts its
// sweep over K nch * b / G chunks in (wrapping around): in lockstep, all
// workgroups would read the same K columns of x1 at once, 16 rows at a
// stride of ldx1, which lands on a few L2 channels.  On MI355X at
// K = N = 4096 the two took fp32 M = 16 from 15.3-18.2 us to 14.0 us.
//
// Only a wave's own LDS areas are written and read in the loop (LDS runs a
// wave's operations in order), so the loop has no barrier.  Masking is on
// addresses: W rows past N, x1 rows past M and k past K load zeros (both
// operands, so NaN padding past K cannot leak in).  Rows of the W area past
// R are never written; they only feed D rows that are not stored.  A ring of
// NB register sets keeps the loads of NB - 1 chunks in flight while a chunk
// is multiplied; one or two sets did best (fp32 M = 16: 13.0 us with two,
// 14.0 with four, 15.3 with eight — deeper rings queue more requests behind
// each other without reading faster).  Small chunks (128 or 256 bytes per
// row) and many waves keep each wave's MFMA work per chunk short, so the
// last chunks to arrive are multiplied quickly; 512-byte and 1 KiB chunks
// left fp32 launches waiting on MFMAs after their data had arrived.
// Summing the waves in a fixed order keeps results independent of
// scheduling; the rotation fixes each workgroup's order of chunks too.
// ---------------------------------------------------------------------------
template <typename T, int WAVES, int CHB, int R, int NB>
__global__ __launch_bounds__(WAVES * 64) void gemv_wt_kernel(const T* __restrict__ x1, const T* __restrict__ w,
                                                             float* __restrict__ out, int M, int N, int K,
                                                             int64_t ldx1, int64_t ldw, int64_t ldo) {
  constexpr int LPR = CHB / 16;    // lanes per W row in one wave load
  constexpr int RPI = 64 / LPR;    // W rows per wave load
  constexpr int NLD = R / RPI;     // W wave loads per chunk
  constexpr int KG = CHB / 64;     // 64-byte k groups per chunk
  constexpr int PITCH = CHB + 16;  // LDS bytes per staged row
  static_assert(CHB == 128 || CHB == 256 || CHB == 512 || CHB == 1024, "chunk of 128 to 1024 bytes per row");
  static_assert(R <= 16 && R % RPI == 0, "R rows of W, whole wave loads");
  typedef std::conditional_t<sizeof(T) == 4, f32x4, i32x4> V;
  constexpr int AREA = 2 * 16 * PITCH;  // the wave's W rows, then its x1 rows
  __shared__ __attribute__((aligned(16))) unsigned char lds[WAVES * AREA];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n0 = blockIdx.x * R;
  const int m0 = blockIdx.y * 16;
  const int q = lane & 15, g = lane >> 4;
  const uint32_t kbytes = (uint32_t)K * sizeof(T);
  const uint32_t ldw_b = (uint32_t)ldw * sizeof(T), ldx1_b = (uint32_t)ldx1 * sizeof(T);
  const BufRsrc rw = make_rsrc(w + (int64_t)n0 * ldw);
  const BufRsrc rx = make_rsrc(x1 + (int64_t)m0 * ldx1);
  const int wrow = lane / LPR;                     // row of a wave load this lane reads
  const uint32_t wcol = 16u * (uint32_t)(lane % LPR);  // its byte within the row piece
  unsigned char* const area = lds + wave * AREA;
  unsigned char* const xarea = area + 16 * PITCH;

  struct Batch {
    V w[NLD], x[KG];
  };
  // x1 pieces of chunk c: lane l reads x1[m0 + l % 16][k group t, 16 bytes at 16 (l / 16)]
  auto load_x = [&](int c, V* x) __attribute__((always_inline)) {
    const uint32_t cb = (uint32_t)c * CHB;
    const bool kw = cb + wcol < kbytes;
#pragma unroll
    for (int i = 0; i < KG; ++i) {
      const int r = i * RPI + wrow;
      const bool ok = kw && m0 + r < M;
      x[i] = __builtin_bit_cast(
          V, __builtin_amdgcn_raw_buffer_load_b128(rx, (int)(ok ? (uint32_t)r * ldx1_b + cb + wcol : kOob), 0, 0));
    }
  };
  auto load = [&](int c, Batch& b) __attribute__((always_inline)) {
    const uint32_t cb = (uint32_t)c * CHB;
    const bool kw = cb + wcol < kbytes;
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      const int r = i * RPI + wrow;
      const bool ok = kw && n0 + r < N;
      b.w[i] = __builtin_bit_cast(
          V, __builtin_amdgcn_raw_buffer_load_b128(rw, (int)(ok ? (uint32_t)r * ldw_b + cb + wcol : kOob), 0, kCpolX2));
    }
    load_x(c, b.x);
  };
  f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
  auto mma = [&](const Batch& b) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < NLD; ++i)
      *reinterpret_cast<V*>(area + (i * RPI + wrow) * PITCH + wcol) = b.w[i];
#pragma unroll
    for (int i = 0; i < KG; ++i)
      *reinterpret_cast<V*>(xarea + (i * RPI + wrow) * PITCH + wcol) = b.x[i];
#pragma unroll
    for (int t = 0; t < KG; ++t) {
      const V a = *reinterpret_cast<const V*>(area + q * PITCH + 64 * t + 16 * g);
      const V xb = *reinterpret_cast<const V*>(xarea + q * PITCH + 64 * t + 16 * g);
      if constexpr (sizeof(T) == 4) {
#pragma unroll
        for (int u = 0; u < 4; ++u) acc[t & 1] = mfma16x16x4(a[u], xb[u], acc[t & 1]);
      } else {
        acc[t & 1] = mfma16x16x32bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, xb), acc[t & 1]);
      }
    }
  };
  const int nch = (int)((kbytes + CHB - 1) / CHB);
  const int mine = nch > wave ? (nch - wave + WAVES - 1) / WAVES : 0;  // chunks wave, wave + WAVES, ...
  // Workgroup b starts its sweep nch * b / G chunks into K (G workgroups)
  // and wraps around; chunk numbers past nch stay past it (masked loads).
  const int rot = (int)(((int64_t)blockIdx.x * nch) / (int)gridDim.x);
  auto chunk = [&](int c) {
    const int r = c + rot;
    return c < nch ? (r >= nch ? r - nch : r) : c;
  };
  // Ring of NB register sets: chunk j + NB - 1 is loaded before chunk j is
  // used (loads past the last chunk are masked and touch no memory).
  Batch ring[NB];
#pragma unroll
  for (int s = 0; s < NB - 1; ++s) load(chunk(wave + s * WAVES), ring[s]);
  for (int j = 0; j < mine; j += NB) {
#pragma unroll
    for (int s = 0; s < NB; ++s) {
      load(chunk(wave + (j + s + NB - 1) * WAVES), ring[(s + NB - 1) % NB]);
      __builtin_amdgcn_sched_barrier(0);
      if (j + s < mine) mma(ring[s]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // Each wave parks its sum in its own area (after its own reads, in order);
  // wave 0 adds them in wave order.  Lane l holds out[m0 + q][n0 + 4 g + v].
  *reinterpret_cast<f32x4*>(area + 16 * lane) = acc[0] + acc[1];
  __syncthreads();
  if (wave != 0) return;
  f32x4 s = *reinterpret_cast<const f32x4*>(lds + 16 * lane);
#pragma unroll
  for (int v = 1; v < WAVES; ++v) s += *reinterpret_cast<const f32x4*>(lds + v * AREA + 16 * lane);
  if (m0 + q >= M) return;
  float* orow = out + (int64_t)(m0 + q) * ldo;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int i = 4 * g + v;
    if (i < R && n0 + i < N) orow[n0 + i] = s[v];
  }
}

// x @ W.T with a row-major x1 and W, M <= MR: the row-dot kernel, at any
// element alignment of K, strides and bases; any other layout runs the
// streaming kernel's variant FB.
template <typename T, int MR>
bool rows_fit(const MatmulArgs& a) {
  return (a.layout & 3) == TILEC_X2_COL_MAJOR && a.M <= MR &&
         (int64_t)a.K * (int64_t)sizeof(T) < (int64_t(1) << 31) - 64;
}

// Every row of x1 and W starts on a 16-byte boundary.
template <typename T>
bool rows_aligned(const MatmulArgs& a) {
  constexpr int EPL = 16 / (int)sizeof(T);
  auto aligned = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  return a.K % EPL == 0 && a.ldx1 % EPL == 0 && a.ldx2 % EPL == 0 && aligned(a.x1) && aligned(a.x2);
}

template <typename T, int MR, int RPW, int WAVES, int U, int CP, typename FB>
hipError_t launch_rows(const MatmulArgs& a, FB fallback) {
  if (!rows_fit<T, MR>(a)) return fallback(a);
  const int64_t rows_per_wg = (int64_t)WAVES * RPW;
  auto kern = rows_aligned<T>(a) ? gemv_rows_kernel<T, MR, RPW, WAVES, U, CP, true>
                                 : gemv_rows_kernel<T, MR, RPW, WAVES, U, CP, false>;
  hipLaunchKernelGGL(kern, dim3((unsigned)cdiv(a.N, rows_per_wg)), dim3(WAVES * 64), 0, a.stream,
                     static_cast<const T*>(a.x1), static_cast<const T*>(a.x2), a.out, (int)a.M, (int)a.N, (int)a.K,
                     a.ldx1, a.ldx2, a.ldo);
  return hipGetLastError();
}

template <typename T, int MR, int RPW, int WAVES, int U>
hipError_t launch_rows_or_skinny(const MatmulArgs& a) {
  return launch_rows<T, MR, RPW, WAVES, U, kCpolX2>(a, [](const MatmulArgs& b) { return launch_skinny<T, 4, 2>(b); });
}

// x @ W.T with M <= 16 under the same layout and alignment conditions: the
// row-tile kernel; anything else runs skinny_*_w4_b2.  Byte offsets within
// the 16 rows of x1 and of W a workgroup reads must fit 31 bits.
template <typename T, int CHB, int R>
bool wt_fits(const MatmulArgs& a) {
  constexpr int EPL = 16 / (int)sizeof(T);
  auto aligned = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  const int64_t esz = (int64_t)sizeof(T), lim = (int64_t(1) << 31) - 2 * CHB;
  return (a.layout & 3) == TILEC_X2_COL_MAJOR && a.M <= 16 && a.K % EPL == 0 && a.ldx1 % EPL == 0 &&
         a.ldx2 % EPL == 0 && aligned(a.x1) && aligned(a.x2) && 15 * a.ldx1 * esz + a.K * esz < lim &&
         (R - 1) * a.ldx2 * esz + a.K * esz < lim;
}

template <typename T, int WAVES, int CHB, int R, int NB>
hipError_t launch_wt_or_skinny(const MatmulArgs& a) {
  if (!wt_fits<T, CHB, R>(a)) return launch_skinny<T, 4, 2>(a);
  hipLaunchKernelGGL((gemv_wt_kernel<T, WAVES, CHB, R, NB>), dim3((unsigned)cdiv(a.N, R), (unsigned)cdiv(a.M, 16)),
                     dim3(WAVES * 64), 0, a.stream, static_cast<const T*>(a.x1), static_cast<const T*>(a.x2), a.out,
                     (int)a.M, (int)a.N, (int)a.K, a.ldx1, a.ldx2, a.ldo);
  return hipGetLastError();
}

}  // namespace

// The streaming kernel as the fallback of other kernels' launchers (the
// panel kernel, panel.hip, for layouts and alignments it does not take).
template <typename T, int WAVES, int UB, int MV>
hipError_t launch_skinny_fallback(const MatmulArgs& a) {
  return launch_skinny<T, WAVES, UB, MV>(a);
}
template hipError_t launch_skinny_fallback<float, 4, 2, 0>(const MatmulArgs&);
template hipError_t launch_skinny_fallback<float, 4, 2, 1>(const MatmulArgs&);
template hipError_t launch_skinny_fallback<float, 4, 2, 4>(const MatmulArgs&);
template hipError_t launch_skinny_fallback<u16, 4, 2, 0>(const MatmulArgs&);
template hipError_t launch_skinny_fallback<u16, 4, 2, 1>(const MatmulArgs&);
template hipError_t launch_skinny_fallback<u16, 4, 2, 4>(const MatmulArgs&);

// A row-dot / row-tile variant: its kernel needs no scratch when `fits`.
static VariantDesc rows_desc(VariantDesc d, bool (*fits)(const MatmulArgs&)) {
  d.own_kernel_runs = fits;
  return d;
}

// Variant table for this family (its order is part of the variant numbering).
// BM = rows per row block, BN = slab width, BK = the largest K chunk of one
// workgroup, unroll = 16-row blocks per batch; max_m 0 = any M.
const VariantDesc* skinny_variants(int* count) {
  static const VariantDesc t[] = {
      {"skinny_f32_w4_b1", TILEC_FAMILY_SKINNY, TILEC_F32, kMaxM, kSlabOf<float>, kKcMax, 4, 0, 1, launch_skinny<float, 4, 1>},
      {"skinny_f32_w4_b2", TILEC_FAMILY_SKINNY, TILEC_F32, kMaxM, kSlabOf<float>, kKcMax, 4, 0, 2, launch_skinny<float, 4, 2>},
      {"skinny_f32_w8_b1", TILEC_FAMILY_SKINNY, TILEC_F32, kMaxM, kSlabOf<float>, kKcMax, 8, 0, 1, launch_skinny<float, 8, 1>},
      {"skinny_f32_w8_b2", TILEC_FAMILY_SKINNY, TILEC_F32, kMaxM, kSlabOf<float>, kKcMax, 8, 0, 2, launch_skinny<float, 8, 2>},
      {"skinny_f32_w16_b1", TILEC_FAMILY_SKINNY, TILEC_F32, kMaxM, kSlabOf<float>, kKcMax, 16, 0, 1, launch_skinny<float, 16, 1>},
      {"skinny_bf16_w4_b1", TILEC_FAMILY_SKINNY, TILEC_BF16, kMaxM, kSlabOf<u16>, kKcMax, 4, 0, 1, launch_skinny<u16, 4, 1>},
      {"skinny_bf16_w4_b2", TILEC_FAMILY_SKINNY, TILEC_BF16, kMaxM, kSlabOf<u16>, kKcMax, 4, 0, 2, launch_skinny<u16, 4, 2>},
      {"skinny_bf16_w8_b1", TILEC_FAMILY_SKINNY, TILEC_BF16, kMaxM, kSlabOf<u16>, kKcMax, 8, 0, 1, launch_skinny<u16, 8, 1>},
      {"skinny_bf16_w8_b2", TILEC_FAMILY_SKINNY, TILEC_BF16, kMaxM, kSlabOf<u16>, kKcMax, 8, 0, 2, launch_skinny<u16, 8, 2>},
      // FMA path for M <= 1 and M <= 4 (row-major x2; column-major x2 runs the MFMA path).
      {"skinny_f32_v1_w4_b2", TILEC_FAMILY_SKINNY, TILEC_F32, kMaxM, kSlabOf<float>, kKcMax, 4, 1, 2, launch_skinny<float, 4, 2, 1>},
      {"skinny_f32_v1_w8_b2", TILEC_FAMILY_SKINNY, TILEC_F32, kMaxM, kSlabOf<float>, kKcMax, 8, 1, 2, launch_skinny<float, 8, 2, 1>},
      {"skinny_f32_v4_w4_b2", TILEC_FAMILY_SKINNY, TILEC_F32, kMaxM, kSlabOf<float>, kKcMax, 4, 4, 2, launch_skinny<float, 4, 2, 4>},
      {"skinny_f32_v4_w8_b2", TILEC_FAMILY_SKINNY, TILEC_F32, kMaxM, kSlabOf<float>, kKcMax, 8, 4, 2, launch_skinny<float, 8, 2, 4>},
      {"skinny_bf16_v1_w4_b2", TILEC_FAMILY_SKINNY, TILEC_BF16, kMaxM, kSlabOf<u16>, kKcMax, 4, 1, 2, launch_skinny<u16, 4, 2, 1>},
      {"skinny_bf16_v1_w8_b2", TILEC_FAMILY_SKINNY, TILEC_BF16, kMaxM, kSlabOf<u16>, kKcMax, 8, 1, 2, launch_skinny<u16, 8, 2, 1>},
      {"skinny_bf16_v4_w4_b2", TILEC_FAMILY_SKINNY, TILEC_BF16, kMaxM, kSlabOf<u16>, kKcMax, 4, 4, 2, launch_skinny<u16, 4, 2, 4>},
      {"skinny_bf16_v4_w8_b2", TILEC_FAMILY_SKINNY, TILEC_BF16, kMaxM, kSlabOf<u16>, kKcMax, 8, 4, 2, launch_skinny<u16, 8, 2, 4>},
      // x @ W.T (column-major x2): row-dot kernel, one or two W rows per wave, no K split (other
      // layouts run skinny_*_w4_b2).  BN = W rows per workgroup.
      rows_desc({"skinny_f32_t1_r1_w4", TILEC_FAMILY_SKINNY, TILEC_F32, kMaxM, 4, kKcMax, 4, 1, 4, launch_rows_or_skinny<float, 1, 1, 4, 4>}, rows_fit<float, 1>),
      rows_desc({"skinny_f32_t1_r2_w4", TILEC_FAMILY_SKINNY, TILEC_F32, kMaxM, 8, kKcMax, 4, 1, 4, launch_rows_or_skinny<float, 1, 2, 4, 4>}, rows_fit<float, 1>),
      rows_desc({"skinny_f32_t4_r2_w4", TILEC_FAMILY_SKINNY, TILEC_F32, kMaxM, 8, kKcMax, 4, 4, 2, launch_rows_or_skinny<float, 4, 2, 4, 2>}, rows_fit<float, 4>),
      rows_desc({"skinny_bf16_t1_r1_w4", TILEC_FAMILY_SKINNY, TILEC_BF16, kMaxM, 4, kKcMax, 4, 1, 4, launch_rows_or_skinny<u16, 1, 1, 4, 4>}, rows_fit<u16, 1>),
      rows_desc({"skinny_bf16_t1_r2_w4", TILEC_FAMILY_SKINNY, TILEC_BF16, kMaxM, 8, kKcMax, 4, 1, 4, launch_rows_or_skinny<u16, 1, 2, 4, 4>}, rows_fit<u16, 1>),
      rows_desc({"skinny_bf16_t4_r2_w4", TILEC_FAMILY_SKINNY, TILEC_BF16, kMaxM, 8, kKcMax, 4, 4, 2, launch_rows_or_skinny<u16, 4, 2, 4, 2>}, rows_fit<u16, 4>),
      // M = 1 with 8 waves per workgroup and batches of 2 chunks (the built-in choice for M = 1).
      rows_desc({"skinny_f32_t1_r1_w8_u2", TILEC_FAMILY_SKINNY, TILEC_F32, kMaxM, 8, kKcMax, 8, 1, 2, launch_rows_or_skinny<float, 1, 1, 8, 2>}, rows_fit<float, 1>),
      rows_desc({"skinny_bf16_t1_r1_w8_u2", TILEC_FAMILY_SKINNY, TILEC_BF16, kMaxM, 8, kKcMax, 8, 1, 2, launch_rows_or_skinny<u16, 1, 1, 8, 2>}, rows_fit<u16, 1>),
      // x @ W.T, M <= 16: row-tile kernel, 16 rows of W per workgroup over all of K (BN), K chunks of
      // 128 or 256 bytes per row, a ring of `unroll` register sets; other layouts run skinny_*_w4_b2.
      rows_desc({"skinny_f32_t16_r16_w16_c128", TILEC_FAMILY_SKINNY, TILEC_F32, kMaxM, 16, kKcMax, 16, 16, 1, launch_wt_or_skinny<float, 16, 128, 16, 1>}, wt_fits<float, 128, 16>),
      rows_desc({"skinny_f32_t16_r16_w8_c128", TILEC_FAMILY_SKINNY, TILEC_F32, kMaxM, 16, kKcMax, 8, 16, 2, launch_wt_or_skinny<float, 8, 128, 16, 2>}, wt_fits<float, 128, 16>),
      rows_desc({"skinny_f32_t16_r16_w8_c256", TILEC_FAMILY_SKINNY, TILEC_F32, kMaxM, 16, kKcMax, 8, 16, 1, launch_wt_or_skinny<float, 8, 256, 16, 1>}, wt_fits<float, 256, 16>),
      rows_desc({"skinny_bf16_t16_r16_w16_c128", TILEC_FAMILY_SKINNY, TILEC_BF16, kMaxM, 16, kKcMax, 16, 16, 1, launch_wt_or_skinny<u16, 16, 128, 16, 1>}, wt_fits<u16, 128, 16>),
      rows_desc({"skinny_bf16_t16_r16_w8_c128", TILEC_FAMILY_SKINNY, TILEC_BF16, kMaxM, 16, kKcMax, 8, 16, 2, launch_wt_or_skinny<u16, 8, 128, 16, 2>}, wt_fits<u16, 128, 16>),
      rows_desc({"skinny_bf16_t16_r16_w8_c256", TILEC_FAMILY_SKINNY, TILEC_BF16, kMaxM, 16, kKcMax, 8, 16, 1, launch_wt_or_skinny<u16, 8, 256, 16, 1>}, wt_fits<u16, 256, 16>),
  };
  *count = (int)(sizeof(t) / sizeof(t[0]));
  return t;
}

// Split K needs partials [splits][row blocks][slabs][16][SLAB] fp32 (scratch)
// and one completion counter per (row block, slab), each on its own 256-byte
// line so workgroups of different cells do not contend on one line.
static int slab_for(int dtype) { return dtype == TILEC_BF16 ? kSlabOf<u16> : kSlabOf<float>; }
size_t skinny_counter_bytes(int dtype, int64_t M, int64_t N, int64_t K, int split_k) {
  const SkinnyGeom g = skinny_geom(M, N, K, split_k, slab_for(dtype));
  if (g.splits <= 1) return 0;
  return (size_t)g.nrb * g.nslabs * kCounterStride * sizeof(unsigned);
}
size_t skinny_workspace_bytes(int dtype, int64_t M, int64_t N, int64_t K, int split_k) {
  const int slab = slab_for(dtype);
  const SkinnyGeom g = skinny_geom(M, N, K, split_k, slab);
  if (g.splits <= 1) return 0;
  return (size_t)g.splits * g.nrb * g.nslabs * kMaxM * slab * sizeof(float);
}
int64_t skinny_effective_splits(int64_t N, int64_t K, int split_k) { return skinny_geom(1, N, K, split_k, 64).splits; }

}  // namespace tilec
