// bf16 GEMM for aligned operands, C[M,N] (fp32) = A[M,K] · B[K,N] (bf16,
// each row- or column-major, read in place), fp32 accumulate, on
// v_mfma_f32_32x32x16_bf16.
//
// Same tile semantics as the reference tile kernel `_matmul_tiled`
// (tilec/ext.py:13-24): zero accumulator, K steps over masked tiles with
// `other=0.0`, masked store.  Built for gfx950:
//   * Global -> LDS with buffer_load_dwordx4 ... lds: each lane moves 16 bytes
//     straight into LDS, asynchronously, with no VGPR staging.  K steps of BK
//     cycle through a ring of NBUF stage buffers: the loads of step k+NBUF-1
//     are issued while step k is multiplied, so NBUF-1 steps (up to 96 KiB
//     per CU) are in flight — the global->LDS stream, not the matrix cores,
//     is what a shallower pipeline is limited by.
//   * The stage buffers are distinct LDS objects and the K loop is unrolled
//     over the ring, so every access names its buffer statically and the
//     compiler knows reads of one buffer do not wait on loads into another.
//   * Each operand lives in LDS as it is in memory.  One whose memory runs
//     along K (row-major A, column-major B) is stored in rows of BK with its
//     16-byte chunks XOR-swizzled per row, so the 16-byte operand reads of
//     16 consecutive rows hit distinct banks.  One whose memory runs along M
//     or N (row-major B, column-major A) is stored in rows of k, and its MFMA
//     operand (8 consecutive k of one row or column per lane) comes from two
//     ds_read_b64_tr_b16 transposing reads; chunks of row k are swizzled by
//     4 * (k & 3) so the 8 rows one read touches spread over the banks.
//   * Masking is done on addresses: chunks past M, N or K get an out-of-range
//     buffer offset and land in LDS as zeros.  Operands must be 16-byte
//     aligned with contiguous extents and strides multiples of 8 (the
//     launcher checks; other shapes go to the generic kernel in
//     gemm_bf16.hip).
//   * Per K step, the MFMAs of the previous step's last k-slice (read into
//     registers before the barrier) run right after it, threaded one-for-one
//     with the next step's loads, so neither the barrier nor the load issue
//     leaves the matrix cores idle.  With 8 waves (2 per SIMD) one wave's
//     MFMAs also cover the other's LDS waits.
//   * XCD-aware grouped tile order (tile_of in common.h).
#include <type_traits>

#include "common.h"
#include "../../include/tilec.h"

namespace tilec {

namespace {

typedef unsigned short u16;
typedef short i16x4v __attribute__((ext_vector_type(4)));
typedef short i16x8v __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) void* lds_ptr_t;

// A k-contiguous stage: chunk c of row i is stored at (c ^ swz_a) within the
// row; BK=64 rows are 128 B (8 chunks, 2 rows per 256-byte bank line), BK=32
// rows 64 B (4 chunks), swizzled by rows (row >> 2) for the 32x32 blocks'
// reads and (row >> 1) for the 16x16 blocks' (each measured free of bank
// conflicts for its own read pattern, and conflicting for the other's).  An r-contiguous stage: chunks of k-row r are
// swizzled by 4 * (r & 3) ^ 2 * ((r >> 3) & 1).  A transposing read serves 32
// lanes per pass; with 32x32 blocks they read 4 k-rows x 32 columns (four
// chunks, spread over all 64 banks by the first term), with 16x16 blocks two
// groups of 4 k-rows 8 apart x 16 columns each: the second term moves the
// upper group's chunks onto the banks the lower group leaves free.
template <int BK, int MF>
__device__ __forceinline__ int swz_a(int row) {
  return BK == 64 ? (row >> 1) & 7 : (row >> (MF == 16 ? 1 : 2)) & 3;
}
__device__ __forceinline__ int swz_b(int krow) { return (4 * (krow & 3)) ^ (2 * ((krow >> 3) & 1)); }

// How one operand's tile (R rows of its outer dimension — M for x1, N for
// x2 — by BK of K) sits in a stage buffer.
//   KC (k contiguous in memory: row-major x1, column-major x2): R rows of BK
//     elements, chunks swizzled by swz_a; an MFMA fragment (8 consecutive k
//     of one row) is one 16-byte read.
//   otherwise (r contiguous: row-major x2, column-major x1): BK rows of R
//     elements, chunks swizzled by swz_b; a fragment comes from two
//     ds_read_b64_tr_b16 transposing reads.
template <int R, int BK, int NW, bool KC, int MF>
struct Stage {
  static constexpr bool kKC = KC;
  static constexpr int ROW_CHUNKS = KC ? BK / 8 : R / 8;  // 16-byte chunks per stored row
  static constexpr int CHUNKS = R * BK / 8;
  static constexpr int INSTR = CHUNKS / 64 / NW;  // DMA instructions per wave per step
  static constexpr int BYTES = R * BK * 2;
  static_assert(CHUNKS % (64 * NW) == 0, "DMA must divide evenly");
  static_assert(KC || R % 128 == 0, "transposed-read swizzle needs rows of >= 16 chunks");
  static_assert(!KC || BK == 32 || BK == 64, "row swizzle covers 4 or 8 chunks per row");
  __device__ __forceinline__ static int swz(int row) { return KC ? swz_a<BK, MF>(row) : swz_b(row); }
  // Stored row and logical chunk of physical chunk p.
  __device__ __forceinline__ static void chunk(int p, int& row, int& lc) {
    row = p / ROW_CHUNKS;
    lc = (p % ROW_CHUNKS) ^ swz(row);
  }
};

// MF: the MFMA block, 32 (v_mfma_f32_32x32x16_bf16: k-slices of 16, f32x16
// accumulators) or 16 (v_mfma_f32_16x16x32_bf16: k-slices of 32, f32x4).
// For the same flops the 16x16 form moves less accumulator data per cycle; a
// stream of it holds a higher clock under the power limit.
template <int BM, int BN, int BK, int NBUF, int WM, int WN, bool CA, bool CB, int MF>
struct LdsGemm {
  static constexpr int NW = WM * WN;
  static constexpr int NT = NW * 64;
  static constexpr int WTM = BM / WM, WTN = BN / WN;
  static constexpr int TM = WTM / MF, TN = WTN / MF;
  static constexpr int KG = MF == 32 ? 2 : 4;  // 8-k groups per k-slice (lane / MF picks one)
  static constexpr int KS = BK / (8 * KG);     // MFMA k-slices per step
  static constexpr int ACC = MF * MF / 64;     // accumulator floats per lane per block
  using Acc = std::conditional_t<MF == 32, f32x16, f32x4>;
  using SA = Stage<BM, BK, NW, !CA, MF>;
  using SB = Stage<BN, BK, NW, CB, MF>;
  static constexpr int A_INSTR = SA::INSTR, B_INSTR = SB::INSTR;
  static constexpr int IPS = A_INSTR + B_INSTR;
  static constexpr int A_BYTES = SA::BYTES, B_BYTES = SB::BYTES;
  static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
  static_assert(MF == 32 || MF == 16, "32x32x16 or 16x16x32 MFMAs");
  static_assert(WTM % MF == 0 && WTN % MF == 0, "wave tile must be whole MFMA blocks");
  static_assert(MF == 16 || KS % 2 == 0, "a step's last k-slice ends in the second fragment set");
  static_assert(KS % 2 == 0 || NBUF % 2 == 0, "odd k-slice counts alternate fragment sets by step parity");
  // 16x16 pipeline: one B fragment set for an even k-slice count.
  static constexpr bool B1 = KS % 2 == 0;
  static_assert(NBUF >= 2 && NBUF <= 4, "ring of 2..4 stage buffers");
  static_assert((size_t)NBUF * STAGE_BYTES <= 160 * 1024, "LDS is 160 KiB");
  static_assert((NBUF - 2) * IPS <= 63, "vmcnt is 6 bits");
};

// s_waitcnt vmcnt(N) with expcnt and lgkmcnt left unconstrained (gfx9
// encoding: vmcnt[3:0] in bits 3:0, vmcnt[5:4] in bits 15:14).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Barrier between K steps, without the memory fence of __syncthreads.  The
// wait before it (vmcnt(WAIT) lgkmcnt(0)) already completes this wave's
// copies of the next step and its reads of the slot the next copies reuse;
// a workgroup fence would in addition wait for every copy in flight
// (vmcnt(0)), draining the ring of stage buffers at each step.  The empty
// asm statements keep the compiler from moving LDS accesses across it.
__device__ __forceinline__ void step_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Scheduling groups "1 MFMA, then its share of the IPS loads", NM times.
template <int NM, int IPS, int X = 0>
__device__ __forceinline__ void sched_mfma_vmem() {
  if constexpr (X < NM) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    constexpr int n = (X + 1) * IPS / NM - X * IPS / NM;
    if constexpr (n > 0) __builtin_amdgcn_sched_group_barrier(0x020, n, 0);
    sched_mfma_vmem<NM, IPS, X + 1>();
  }
}

// Scheduling groups for the 16x16 pipeline: the B reads of the next k-slice
// (TN fragments of RB reads; RB = 0 when they follow instead) first, then per
// row block x: 1 MFMA, its share of IPS loads, the other TN - 1 MFMAs, the RA
// reads refilling its A fragment.
template <int TM, int TN, int IPS, int RA, int RB, int X = -1>
__device__ __forceinline__ void sched_rows() {
  if constexpr (X < 0) {
    if constexpr (RB > 0) __builtin_amdgcn_sched_group_barrier(0x100, TN * RB, 0);
    sched_rows<TM, TN, IPS, RA, RB, 0>();
  } else if constexpr (X < TM) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    constexpr int n = (X + 1) * IPS / TM - X * IPS / TM;
    if constexpr (n > 0) __builtin_amdgcn_sched_group_barrier(0x020, n, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, TN - 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, RA, 0);
    sched_rows<TM, TN, IPS, RA, RB, X + 1>();
  }
}

template <int BM, int BN, int BK, int NBUF, int WM, int WN, bool KFULL, bool CA, bool CB, int MF>
__global__ __launch_bounds__(WM * WN * 64, 1) void gemm_bf16_lds_kernel(
    const u16* __restrict__ A, const u16* __restrict__ B, float* __restrict__ C, int M, int N, int K,
    int64_t lda, int64_t ldb, int64_t ldc, int group_m, int xcds, int split_steps, float* __restrict__ ws,
    unsigned* __restrict__ counters) {
  using P = LdsGemm<BM, BN, BK, NBUF, WM, WN, CA, CB, MF>;
  using SA = typename P::SA;
  using SB = typename P::SB;
  constexpr int KS = P::KS;
  __shared__ int last_flag;
  // The ring: distinct LDS objects (those past NBUF are never referenced).
  __shared__ __align__(16) char lds0[P::STAGE_BYTES];
  __shared__ __align__(16) char lds1[P::STAGE_BYTES];
  __shared__ __align__(16) char lds2[NBUF > 2 ? P::STAGE_BYTES : 16];
  __shared__ __align__(16) char lds3[NBUF > 3 ? P::STAGE_BYTES : 16];
  auto buf = [&](auto I) -> char* {
    constexpr int i = decltype(I)::value;
    if constexpr (i == 0) return lds0;
    else if constexpr (i == 1) return lds1;
    else if constexpr (i == 2) return lds2;
    else return lds3;
  };

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  int tm, tn;
  tile_of(blockIdx.x, xcds, tiles_m, tiles_n, group_m, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  // This workgroup's K steps: [kt0, kt0 + nk) of the cdiv(K, BK) steps
  // (grid y = K splits of split_steps steps each; one split = all of K).
  const int split = blockIdx.y, S = gridDim.y;
  const int kt0 = split * split_steps;
  const int nk = max(0, min((K + BK - 1) / BK, kt0 + split_steps) - kt0);

  // ---- global -> LDS for K step kt (local: absolute step kt0 + kt) ----------
  // Physical chunk p of an operand's stage area holds stored row
  // p / ROW_CHUNKS, logical chunk (p % ROW_CHUNKS) ^ swz(row) (Stage).
  // Instruction i of this wave fills physical chunks [64 * (wave * INSTR +
  // i), +64), lane l the l-th of them.  A lane's byte offset from the step's
  // base is the same in every step; chunks past M or N get kOob once, here.
  // A step past this workgroup's range gets a resource of zero records, so
  // its loads touch nothing.  When K % BK != 0 (!KFULL) the last step also
  // masks K: per lane for a k-contiguous operand (its chunk's k column), by
  // the resource's size for an r-contiguous one (whole stored rows of K).
  uint32_t off_a[P::A_INSTR], off_b[P::B_INSTR];
  // The K column of this lane's chunk of instruction i of a k-contiguous
  // operand; recomputed where needed rather than held in registers.
  auto kcol = [&](auto st, int i) {
    using T = decltype(st);
    int row, lc;
    T::chunk(64 * (wave * T::INSTR + i) + lane, row, lc);
    return 8 * lc;
  };
#pragma unroll
  for (int i = 0; i < P::A_INSTR; ++i) {
    int row, lc;
    SA::chunk(64 * (wave * P::A_INSTR + i) + lane, row, lc);
    const bool in = CA ? m0 + 8 * lc < M : m0 + row < M;  // stored row = k (CA) or m
    off_a[i] = in ? 2u * ((uint32_t)row * (uint32_t)lda + 8u * lc) : kOob;
  }
#pragma unroll
  for (int i = 0; i < P::B_INSTR; ++i) {
    int row, lc;
    SB::chunk(64 * (wave * P::B_INSTR + i) + lane, row, lc);
    const bool in = CB ? n0 + row < N : n0 + 8 * lc < N;  // stored row = n (CB) or k
    off_b[i] = in ? 2u * ((uint32_t)row * (uint32_t)ldb + 8u * lc) : kOob;
  }
  // The copies of a step read from resources based at that step's first
  // element of each operand tile.  Steps are copied in order (0 .. NBUF-2 in
  // the prologue, then step kt + NBUF - 1 during step kt), so the bases are
  // kept running: one 64-bit scalar add per operand per step instead of a
  // multiply-add chain from the tile origin.  A step past this workgroup's
  // range gets zero records, so its loads touch nothing.  When K % BK != 0
  // (!KFULL) the last step also masks K: per lane for a k-contiguous operand
  // (its chunk's k column), by the resource's size for an r-contiguous one
  // (whole stored rows of K).
  const u16* a_next = !CA ? A + (int64_t)m0 * lda + (int64_t)kt0 * BK : A + (int64_t)kt0 * BK * lda + m0;
  const u16* b_next = CB ? B + (int64_t)n0 * ldb + (int64_t)kt0 * BK : B + (int64_t)kt0 * BK * ldb + n0;
  const int64_t a_step = !CA ? BK : (int64_t)BK * lda;
  const int64_t b_step = CB ? BK : (int64_t)BK * ldb;
  auto op_recs = [&](bool kcontig, int64_t ld, int k0, bool live) -> uint32_t {
    if (!live) return 0u;
    if (!KFULL && !kcontig) return (uint32_t)min<int64_t>((int64_t)(K - k0) * ld * 2, 0x7FFFFFFF);
    return 0x7FFFFFFFu;
  };
  // The resources of step kt (the next step to copy); each advances its base.
  // Every input is wave-uniform; they go through readfirstlane so the
  // compiler keeps the resources in scalar registers (a divergent-looking
  // resource wraps every direct-to-LDS copy in a waterfall loop).
  auto rsrc_a = [&](int kt) __attribute__((always_inline)) {
    const BufRsrc r = make_rsrc_uniform(a_next, op_recs(!CA, lda, (kt0 + kt) * BK, kt < nk));
    a_next += a_step;
    return r;
  };
  auto rsrc_b = [&](int kt) __attribute__((always_inline)) {
    const BufRsrc r = make_rsrc_uniform(b_next, op_recs(CB, ldb, (kt0 + kt) * BK, kt < nk));
    b_next += b_step;
    return r;
  };
  // Instruction q (0 <= q < IPS) of step kt: A instructions first, then B.
  // (Offsets are copied out of the arrays before the builtin: passed straight
  // to it, an array element makes the host pass drop the kernel's stub.)
  auto dma_one = [&](BufRsrc ra, BufRsrc rb, int q, int kt, char* st) __attribute__((always_inline)) {
    const int k0 = (kt0 + kt) * BK;
    if (q < P::A_INSTR) {
      uint32_t off = off_a[q];
      if constexpr (!KFULL && !CA) off = k0 + kcol(SA{}, q) < K ? off : kOob;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_ptr_t)(st + 16 * 64 * (wave * P::A_INSTR + q)), 16, off, 0,
                                               0, 0);
    } else {
      const int i = q - P::A_INSTR;
      uint32_t off = off_b[i];
      if constexpr (!KFULL && CB) off = k0 + kcol(SB{}, i) < K ? off : kOob;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_ptr_t)(st + P::A_BYTES + 16 * 64 * (wave * P::B_INSTR + i)),
                                               16, off, 0, 0, 0);
    }
  };
  auto dma = [&](int kt, char* st) __attribute__((always_inline)) {
    const BufRsrc ra = rsrc_a(kt), rb = rsrc_b(kt);
#pragma unroll
    for (int q = 0; q < P::IPS; ++q) dma_one(ra, rb, q, kt, st);
  };

  typename P::Acc acc[P::TM][P::TN];
#pragma unroll
  for (int i = 0; i < P::TM; ++i)
#pragma unroll
    for (int j = 0; j < P::TN; ++j)
#pragma unroll
      for (int r = 0; r < P::ACC; ++r) acc[i][j][r] = 0.f;

  // Per-lane fragment addressing (bytes within an operand's stage area).
  // A fragment is 8 consecutive k of one of the wave's MF rows (MFMA operand
  // layout: row lane % MF, 8-k group kg = lane / MF of the k-slice's KG).
  // From a k-contiguous stage it is the 16-byte chunk KG ks + kg of that row;
  // from an r-contiguous stage two transposing reads return it.  Each read
  // gives lane jj of a 16-lane group (g = lane / 16) the 4 k-rows tr_krow ..
  // of column jj of the group's 16 columns, which the group's lanes address
  // as 4 k-rows x 4 pieces of 4 columns: k-rows 8 KG ks + tr_krow (+4 for the
  // second read), columns tr_row .. + 3 of the block.
  const int kg = lane / MF;
  const int g = lane >> 4, jj = lane & 15;
  const int tr_row = (MF == 32 ? 16 * (g & 1) : 0) + 4 * (jj & 3);
  const int tr_krow = (MF == 32 ? 8 * (g >> 1) : 8 * g) + (jj >> 2);
  int a_r[P::TM];
#pragma unroll
  for (int i = 0; i < P::TM; ++i) a_r[i] = wm * P::WTM + MF * i + (CA ? tr_row : (lane % MF));
  int b_r[P::TN];
#pragma unroll
  for (int j = 0; j < P::TN; ++j) b_r[j] = wn * P::WTN + MF * j + (CB ? (lane % MF) : tr_row);

  // Transposing reads: the lane's byte offset from the stage base for k-slice
  // 0 (for B including the A area), kept opaque so that every read's address
  // is that one offset plus a constant (k-slice ks and second read add
  // 16 * ROW_CHUNKS * (8 KG ks + 4)).  With shallow address chains the
  // compiler's per-object LDS alias scopes reach every read, so the waits it
  // places before LDS reads cover only the DMA copies into the same stage
  // buffer; a read it cannot place waits for every DMA copy in flight,
  // including the next step's.
  uint32_t tr_a[P::TM], tr_b[P::TN];
  auto tr_off = [&](auto st_t, int r) -> uint32_t {
    using T = decltype(st_t);
    return 16u * (uint32_t)(tr_krow * T::ROW_CHUNKS + ((r >> 3) ^ T::swz(tr_krow))) + 8u * (uint32_t)((r >> 2) & 1);
  };
#pragma unroll
  for (int i = 0; i < P::TM; ++i) {
    tr_a[i] = SA::kKC ? 0u : tr_off(SA{}, a_r[i]);
    asm volatile("" : "+v"(tr_a[i]));
  }
#pragma unroll
  for (int j = 0; j < P::TN; ++j) {
    tr_b[j] = SB::kKC ? 0u : (uint32_t)P::A_BYTES + tr_off(SB{}, b_r[j]);
    asm volatile("" : "+v"(tr_b[j]));
  }

  // kc stage: `area` is the operand's area, r its row.  r-contiguous stage:
  // `area` is the stage base, `off` the lane's offset from tr_a / tr_b.
  auto frag = [&](auto st_t, const char* area, int r, uint32_t off, int ks) __attribute__((always_inline)) -> bf16x8 {
    using T = decltype(st_t);
    if constexpr (T::kKC) {
      const int c = P::KG * ks + kg;
      return *reinterpret_cast<const bf16x8*>(area + 16 * (r * T::ROW_CHUNKS + (c ^ T::swz(r))));
    } else {
      typedef __attribute__((address_space(3))) i16x4v lds_i16x4;
      constexpr uint32_t kRow = 16u * T::ROW_CHUNKS;  // bytes per stored k-row
      const char* p = area + off;
      const i16x4v lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p + kRow * (8 * P::KG * ks)));
      const i16x4v hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p + kRow * (8 * P::KG * ks + 4)));
      return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    }
  };

  // The operands of one k-slice: A rows of the wave's 32-row blocks, B
  // columns of its MF-column blocks (8 consecutive k each).
  struct Frag {
    bf16x8 a[P::TM], b[P::TN];
  };
  auto read = [&](const char* st, int ks, Frag& f) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < P::TM; ++i) f.a[i] = frag(SA{}, st, a_r[i], tr_a[i], ks);
#pragma unroll
    for (int j = 0; j < P::TN; ++j) f.b[j] = frag(SB{}, SB::kKC ? st + P::A_BYTES : st, b_r[j], tr_b[j], ks);
  };
  auto mfma_blk = [](bf16x8 a, bf16x8 b, typename P::Acc c) __attribute__((always_inline)) {
    if constexpr (MF == 32) return mfma32x32x16bf16(a, b, c);
    else return mfma16x16x32bf16(a, b, c);
  };
  auto mma = [&](const Frag& f) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < P::TM; ++i)
#pragma unroll
      for (int j = 0; j < P::TN; ++j) acc[i][j] = mfma_blk(f.a[i], f.b[j], acc[i][j]);
  };
  // The MFMAs of f with the loads of step kt threaded between them, so the
  // loads issue while the matrix cores are busy.
  auto mma_dma = [&](const Frag& f, int kt, char* st) __attribute__((always_inline)) {
    constexpr int NM = P::TM * P::TN;
    const BufRsrc ra = rsrc_a(kt), rb = rsrc_b(kt);
#pragma unroll
    for (int x = 0; x < NM; ++x) {
      const int i = x / P::TN, j = x % P::TN;
      acc[i][j] = mfma_blk(f.a[i], f.b[j], acc[i][j]);
#pragma unroll
      for (int q = x * P::IPS / NM; q < (x + 1) * P::IPS / NM; ++q) dma_one(ra, rb, q, kt, st);
    }
    sched_mfma_vmem<NM, P::IPS>();
  };

  // Software pipeline over K steps.  Entering step kt (ring slot I): f[0]
  // holds (or is loading) k-slice 0 of step kt; f[1] holds the last k-slice
  // of step kt-1, whose MFMAs have not been issued (zeros before step 0).
  // Step kt:
  //   1. MFMAs of f[1], threaded with the loads of step kt+NBUF-1 into the
  //      slot step kt-1 used — every wave finished reading that slot before
  //      the last barrier — so the matrix cores stay busy across it;
  //   2. k-slices 0 .. KS-2 of step kt, each one's MFMAs overlapping the LDS
  //      reads of the next; the last k-slice is read into f[1];
  //   3. wait for those reads and for this wave's loads of step kt+1 (at most
  //      NBUF-2 later steps in flight; loads complete in issue order), then
  //      the barrier: step kt+1 is in LDS for every wave and no wave reads
  //      step kt's slot again;
  //   4. read k-slice 0 of step kt+1 into f[0].
  constexpr int WAIT = (NBUF - 2) * P::IPS;
  if constexpr (MF == 32) {
  Frag f[2];
#pragma unroll
  for (int i = 0; i < P::TM; ++i) f[1].a[i] = bf16x8{};
#pragma unroll
  for (int j = 0; j < P::TN; ++j) f[1].b[j] = bf16x8{};

  auto step = [&](auto I, int kt) __attribute__((always_inline)) {
    constexpr int i = decltype(I)::value;
    char* const cur = buf(I);
    mma_dma(f[1], kt + NBUF - 1, buf(std::integral_constant<int, (i + NBUF - 1) % NBUF>{}));
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int ks = 0; ks + 1 < KS; ++ks) {
      read(cur, ks + 1, f[(ks + 1) & 1]);
      mma(f[ks & 1]);
    }
    // The step's MFMAs stay ahead of the wait: nothing crosses this point.
    __builtin_amdgcn_sched_barrier(0);
    // vmcnt(WAIT) lgkmcnt(0) (gfx9 encoding, expcnt unconstrained)
    __builtin_amdgcn_s_waitcnt((WAIT & 15) | ((WAIT >> 4) << 14) | (7 << 4));
    step_barrier();
    read(buf(std::integral_constant<int, (i + 1) % NBUF>{}), 0, f[0]);
    __builtin_amdgcn_sched_barrier(0);
  };

  // Prologue: steps 0 .. NBUF-2 in flight, step 0 landed everywhere, its
  // first k-slice being read.
  if (nk > 0) {
    dma(0, lds0);
    if constexpr (NBUF > 2) dma(1, lds1);
    if constexpr (NBUF > 3) dma(2, lds2);
    wait_vmcnt<WAIT>();
    step_barrier();
    read(lds0, 0, f[0]);
  }
  int kt = 0;
  for (; kt + NBUF <= nk; kt += NBUF) {
    step(std::integral_constant<int, 0>{}, kt);
    step(std::integral_constant<int, 1>{}, kt + 1);
    if constexpr (NBUF > 2) step(std::integral_constant<int, 2>{}, kt + 2);
    if constexpr (NBUF > 3) step(std::integral_constant<int, 3>{}, kt + 3);
  }
  // Remaining steps (fewer than NBUF): same slots in order.
  if (kt < nk) step(std::integral_constant<int, 0>{}, kt);
  if (kt + 1 < nk) step(std::integral_constant<int, 1>{}, kt + 1);
  if constexpr (NBUF > 2) {
    if (kt + 2 < nk) step(std::integral_constant<int, 2>{}, kt + 2);
  }
  mma(f[1]);  // last k-slice of the last step (zeros if K == 0)
  } else {
    // 16x16x32 blocks: a k-slice's fragments take twice the registers of a
    // 32x32x16 slice for the same wave tile.  A has one set: right after the
    // MFMAs of row block x are issued, fa[x] is refilled from the next
    // k-slice.  B has one set too when a step has an even number of k-slices
    // (read right after the MFMAs that used the previous slice); 32-deep steps
    // (one k-slice) keep two B sets, read a step ahead.  Entering step kt (its stage landed everywhere):
    // Entering step kt (its stage landed everywhere), fa and one B set hold
    // the last k-slice of step kt-1, MFMAs not yet issued (zeros before step
    // 0).  Step kt, an even number of k-slices:
    //   1. MFMAs of (fa, fb[0]), row block by row block, each followed by its
    //      A refill from k-slice 0, with the loads of step kt+NBUF-1 threaded
    //      between them (into the slot step kt-1 used; every wave finished
    //      reading it before the last barrier); then read B of k-slice 0 into
    //      fb[0];
    //   2. per further k-slice ks: the MFMAs of k-slice ks-1, each row block
    //      refilled from ks, then B of ks into fb[0];
    //   3. wait for every read of this stage and for this wave's loads of
    //      step kt+1, then the barrier.
    // One k-slice per step (BK = 32): B of the step's k-slice is read into
    // the set the previous step's MFMAs do not use, before them; the sets
    // alternate by step parity (ring slot i = step % NBUF, NBUF even) and the
    // step count is rounded up to even, so the last step's ends in fb[0]: the
    // extra step's stage holds zeros (its copies were issued past nk, with
    // zero records) and adds nothing.
    bf16x8 fa[P::TM], fb[2][P::TN];
#pragma unroll
    for (int i = 0; i < P::TM; ++i) fa[i] = bf16x8{};
#pragma unroll
    for (int j = 0; j < P::TN; ++j) fb[0][j] = fb[1][j] = bf16x8{};
    constexpr int RA = SA::kKC ? 1 : 2, RB = SB::kKC ? 1 : 2;  // LDS reads per fragment
    auto read_b = [&](const char* st, int ks, bf16x8 (&b)[P::TN]) __attribute__((always_inline)) {
#pragma unroll
      for (int j = 0; j < P::TN; ++j) b[j] = frag(SB{}, SB::kKC ? st + P::A_BYTES : st, b_r[j], tr_b[j], ks);
    };
    // MFMAs of (fa, b), refilling fa from k-slice ks of stage st.
    auto mma_refill = [&](const bf16x8 (&b)[P::TN], const char* st, int ks) __attribute__((always_inline)) {
#pragma unroll
      for (int x = 0; x < P::TM; ++x) {
#pragma unroll
        for (int j = 0; j < P::TN; ++j) acc[x][j] = mfma_blk(fa[x], b[j], acc[x][j]);
        fa[x] = frag(SA{}, st, a_r[x], tr_a[x], ks);
      }
      sched_rows<P::TM, P::TN, 0, RA, P::B1 ? 0 : RB>();
    };
    auto mma_refill_dma = [&](const bf16x8 (&b)[P::TN], const char* st, int kt, char* dst)
        __attribute__((always_inline)) {
      const BufRsrc ra = rsrc_a(kt), rb = rsrc_b(kt);
#pragma unroll
      for (int x = 0; x < P::TM; ++x) {
#pragma unroll
        for (int j = 0; j < P::TN; ++j) {
          acc[x][j] = mfma_blk(fa[x], b[j], acc[x][j]);
          if (j == 0) {
#pragma unroll
            for (int q = x * P::IPS / P::TM; q < (x + 1) * P::IPS / P::TM; ++q) dma_one(ra, rb, q, kt, dst);
          }
        }
        fa[x] = frag(SA{}, st, a_r[x], tr_a[x], 0);
      }
      sched_rows<P::TM, P::TN, P::IPS, RA, P::B1 ? 0 : RB>();
    };
    auto step16 = [&](auto I, int kt) __attribute__((always_inline)) {
      constexpr int i = decltype(I)::value;
      constexpr int pv = P::B1 ? 1 : (i & 1);  // set holding the previous step's last B
      constexpr int s0 = pv ^ 1;                     // set receiving k-slice 0's B
      char* const cur = buf(I);
      if constexpr (P::B1) {
        // One B set: each k-slice's B is read right after the MFMAs that
        // used the previous one were issued.  On the 256x256 tile the
        // wave's priority is raised over each MFMA block and lowered for the
        // B reads: of the two waves on a SIMD, the one in its MFMA block
        // issues first, so the other's LDS reads run under it rather than
        // both waves alternating MFMAs and then both waiting on LDS (8192^3
        // on MI355X: 1.3 % faster row-major, 2.4 % with x1 column-major,
        // level for x2 column-major; on the 128x128 tile 0.4-2 % slower,
        // and in the two-B-set form below 1.5-4x slower).
        constexpr bool PRIO = BM == 256 && BN == 256;
        if constexpr (PRIO) __builtin_amdgcn_s_setprio(1);
        mma_refill_dma(fb[0], cur, kt + NBUF - 1, buf(std::integral_constant<int, (i + NBUF - 1) % NBUF>{}));
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (PRIO) __builtin_amdgcn_s_setprio(0);
        read_b(cur, 0, fb[0]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int ks = 1; ks < KS; ++ks) {
          if constexpr (PRIO) __builtin_amdgcn_s_setprio(1);
          mma_refill(fb[0], cur, ks);
          __builtin_amdgcn_sched_barrier(0);
          if constexpr (PRIO) __builtin_amdgcn_s_setprio(0);
          read_b(cur, ks, fb[0]);
          __builtin_amdgcn_sched_barrier(0);
        }
      } else {
        read_b(cur, 0, fb[s0]);
        mma_refill_dma(fb[pv], cur, kt + NBUF - 1, buf(std::integral_constant<int, (i + NBUF - 1) % NBUF>{}));
        __builtin_amdgcn_sched_barrier(0);
      }
      // vmcnt(WAIT) lgkmcnt(0) (gfx9 encoding, expcnt unconstrained)
      __builtin_amdgcn_s_waitcnt((WAIT & 15) | ((WAIT >> 4) << 14) | (7 << 4));
      step_barrier();
      __builtin_amdgcn_sched_barrier(0);
    };
    const int nrun = P::B1 ? nk : nk + (nk & 1);
    if (nrun > 0) {
      dma(0, lds0);
      if constexpr (NBUF > 2) dma(1, lds1);
      if constexpr (NBUF > 3) dma(2, lds2);
      wait_vmcnt<WAIT>();
      step_barrier();
    }
    int kt = 0;
    for (; kt + NBUF <= nrun; kt += NBUF) {
      step16(std::integral_constant<int, 0>{}, kt);
      step16(std::integral_constant<int, 1>{}, kt + 1);
      if constexpr (NBUF > 2) step16(std::integral_constant<int, 2>{}, kt + 2);
      if constexpr (NBUF > 3) step16(std::integral_constant<int, 3>{}, kt + 3);
    }
    if (kt < nrun) step16(std::integral_constant<int, 0>{}, kt);
    if (kt + 1 < nrun) step16(std::integral_constant<int, 1>{}, kt + 1);
    if constexpr (NBUF > 2) {
      if (kt + 2 < nrun) step16(std::integral_constant<int, 2>{}, kt + 2);
    }
    // last k-slice of the last step (zeros if K == 0)
    auto mma_last = [&](const bf16x8 (&b)[P::TN]) __attribute__((always_inline)) {
#pragma unroll
      for (int x = 0; x < P::TM; ++x)
#pragma unroll
        for (int j = 0; j < P::TN; ++j) acc[x][j] = mfma_blk(fa[x], b[j], acc[x][j]);
    };
    mma_last(fb[0]);
  }
  // Loads issued for steps past K still write (zeros) into LDS: let them
  // land before this workgroup can finish and release its LDS.
  __builtin_amdgcn_s_waitcnt(0);

  // Split K: publish this workgroup's partial tile; the last of the tile's
  // splits adds them in split order and writes C.
  // Epilogue: a lane holds, of each block, D[8*(r/4) + 4*(lane/32) + r%4][lane%32]
  // (MF = 32, r < 16) or D[4*(lane/16) + r][lane%16] (MF = 16, r < 4).
  const bool interior = (m0 + BM <= M) && (n0 + BN <= N);
  const int row_base = m0 + wm * P::WTM + 4 * (MF == 32 ? kg : g);
  const int col_base = n0 + wn * P::WTN + (lane % MF);
  if constexpr (MF == 32) {
    if (S > 1 && !splitk_tile<P::TM, P::TN, P::NT>(acc, split, S, blockIdx.x, gridDim.x, ws, counters, &last_flag,
                                                    row_base, col_base, M, N))
      return;
  } else {
    if (S > 1 && !splitk_tile16<P::TM, P::TN, P::NT>(acc, split, S, blockIdx.x, gridDim.x, ws, counters,
                                                      &last_flag, row_base, col_base, M, N))
      return;
  }
#pragma unroll
  for (int i = 0; i < P::TM; ++i)
#pragma unroll
    for (int j = 0; j < P::TN; ++j) {
      const int gn = col_base + MF * j;
#pragma unroll
      for (int r = 0; r < P::ACC; ++r) {
        const int gm = row_base + MF * i + (MF == 32 ? 8 * (r >> 2) + (r & 3) : r);
        if (interior || (gm < M && gn < N)) C[(int64_t)gm * ldc + gn] = acc[i][j][r];
      }
    }
}

}  // namespace

// Launch the LDS-DMA kernel; the caller has checked alignment (16-byte
// operands, contiguous extents and strides multiples of 8) and the 32-bit
// offset limits.
template <int BM, int BN, int BK, int NBUF, int WM, int WN, bool CA, bool CB, int MF>
hipError_t launch_gemm_bf16_lds(const MatmulArgs& a) {
  using P = LdsGemm<BM, BN, BK, NBUF, WM, WN, CA, CB, MF>;
  const int64_t tiles = cdiv(a.M, BM) * cdiv(a.N, BN);
  if (tiles == 0) return hipSuccess;
  const SplitGeom g = gemm_split_geom(a.K, BK, a.split_k);
  if (g.splits > 1 && P::TM * P::TN * P::ACC > kSplitMaxAccPerThread) return hipErrorInvalidConfiguration;
  // The 16x16 pipeline holds more fragment registers; with K % BK != 0 its
  // per-lane K masks no longer fit in 256 VGPRs, so that case runs the 32x32
  // kernel of the same tile.
  if constexpr (MF == 16) {
    if (a.K % BK != 0) return launch_gemm_bf16_lds<BM, BN, BK, NBUF, WM, WN, CA, CB, 32>(a);
  }
  auto kern = gemm_bf16_lds_kernel<BM, BN, BK, NBUF, WM, WN, true, CA, CB, MF>;
  if constexpr (MF == 32) {
    if (a.K % BK != 0) kern = gemm_bf16_lds_kernel<BM, BN, BK, NBUF, WM, WN, false, CA, CB, MF>;
  }
  hipLaunchKernelGGL(kern, dim3((unsigned)tiles, (unsigned)g.splits), dim3(P::NT), 0, a.stream,
                     static_cast<const u16*>(a.x1), static_cast<const u16*>(a.x2), a.out, (int)a.M, (int)a.N,
                     (int)a.K, a.ldx1, a.ldx2, a.ldo, 4, device_xcds(), (int)g.steps, g.splits > 1 ? static_cast<float*>(a.workspace) : nullptr,
                     g.splits > 1 ? a.counters : nullptr);
  return hipGetLastError();
}

#define TILEC_LDS_VARIANT(BM, BN, BK, NBUF, WM, WN, MF)                                                \
  template hipError_t launch_gemm_bf16_lds<BM, BN, BK, NBUF, WM, WN, false, false, MF>(const MatmulArgs&); \
  template hipError_t launch_gemm_bf16_lds<BM, BN, BK, NBUF, WM, WN, true, false, MF>(const MatmulArgs&);  \
  template hipError_t launch_gemm_bf16_lds<BM, BN, BK, NBUF, WM, WN, false, true, MF>(const MatmulArgs&);  \
  template hipError_t launch_gemm_bf16_lds<BM, BN, BK, NBUF, WM, WN, true, true, MF>(const MatmulArgs&);
TILEC_LDS_VARIANT(256, 256, 32, 4, 2, 2, 32)
TILEC_LDS_VARIANT(256, 256, 64, 2, 2, 4, 32)
TILEC_LDS_VARIANT(256, 128, 64, 3, 4, 2, 32)
TILEC_LDS_VARIANT(256, 128, 32, 4, 2, 2, 32)
TILEC_LDS_VARIANT(128, 128, 64, 4, 2, 4, 32)
TILEC_LDS_VARIANT(256, 256, 32, 4, 2, 4, 32)
TILEC_LDS_VARIANT(256, 256, 64, 2, 2, 4, 16)
TILEC_LDS_VARIANT(256, 256, 32, 4, 2, 4, 16)
TILEC_LDS_VARIANT(256, 128, 64, 3, 4, 2, 16)
TILEC_LDS_VARIANT(128, 128, 64, 4, 2, 4, 16)
#undef TILEC_LDS_VARIANT

}  // namespace tilec
