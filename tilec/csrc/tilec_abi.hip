// C ABI of libtilec_hip.so (declared in include/tilec.h).
//
// Validates arguments the way the reference's host code does before it
// launches (`_matrix_mul_tiled`, tilec/ext.py:55-61, and `_arg_type`,
// tilec/jit.py:34-39), resolves the variant and split, and enqueues one
// kernel on the caller's stream.  No allocation, no synchronization.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <vector>

#include "common.h"
#include "../../include/tilec.h"

namespace tilec {
const VariantDesc* skinny_variants(int* count);
const VariantDesc* gemm_f32_variants(int* count);
const VariantDesc* gemm_bf16_variants(int* count);
const VariantDesc* panel_variants(int* count);
const VariantDesc* direct_variants(int* count);
int64_t direct_effective_splits(int64_t K, int split_k);
size_t skinny_counter_bytes(int dtype, int64_t M, int64_t N, int64_t K, int split_k);
size_t skinny_workspace_bytes(int dtype, int64_t M, int64_t N, int64_t K, int split_k);
int64_t skinny_effective_splits(int64_t N, int64_t K, int split_k);
struct ReduceGeom {
  int64_t cells, splits, span;
  int lpr;
};
ReduceGeom reduce_geom(int64_t R, int64_t C, int esz, int axis);
size_t reduce_workspace_bytes(const ReduceGeom& g);
size_t reduce_counter_bytes(const ReduceGeom& g);
hipError_t launch_reduce(const void* x, float* out, int64_t R, int64_t C, int64_t ld, int dtype, int axis, float* ws,
                         unsigned* counters, hipStream_t stream);
hipError_t launch_read_floor(const void* x, int64_t bytes, float* sink, int workgroups, hipStream_t stream);
}  // namespace tilec

using namespace tilec;

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

const std::vector<const VariantDesc*>& table() {
  static std::vector<const VariantDesc*> t;
  static std::once_flag once;
  std::call_once(once, [] {
    for (auto fam : {skinny_variants, gemm_f32_variants, gemm_bf16_variants, panel_variants, direct_variants}) {
      int n = 0;
      const VariantDesc* v = fam(&n);
      for (int i = 0; i < n; ++i) t.push_back(&v[i]);
    }
  });
  return t;
}

int find(const char* name) {
  const auto& t = table();
  for (size_t i = 0; i < t.size(); ++i)
    if (strcmp(t[i]->name, name) == 0) return (int)i;
  return -1;
}

constexpr int64_t kMaxDim = (int64_t(1) << 31) - 1024;  // kernels index rows/cols in int32

// Compute units of the current device (MI355X: 256; fewer in a partitioned
// mode), read once per device; 256 if the query fails.
int device_cus() {
  constexpr int kMaxDev = 64;
  static std::atomic<int> cache[kMaxDev];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (dev >= 0 && dev < kMaxDev) {
    const int c = cache[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
  if (dev >= 0 && dev < kMaxDev) cache[dev].store(cus, std::memory_order_relaxed);
  return cus;
}

// The skinny kernel addresses its operands within one block with 32-bit byte
// offsets: row-major x2 over 16 rows (16 * ldx2 * 4 bytes < 2^31), x1 over 16
// rows or (column-major) up to 32 columns of K (32 * ldx1 * 2 bytes), and
// column-major x2 over a slab's 64 fp32 / 128 bf16 columns (256 * ldx2
// bytes < 2^31); its split-K partials also take 32-bit offsets (splits * row
// blocks * slabs * 16 * slab width * 4 bytes < 2^31).  Row blocks of 16 are
// its grid's z dimension (at most 65535).
constexpr int64_t kSkinnyMaxLdx1 = int64_t(1) << 25;
constexpr int64_t kSkinnyMaxLdx2 = int64_t(1) << 25;
constexpr int64_t kSkinnyMaxLdx2ColMajor = int64_t(1) << 23;
constexpr int64_t kSkinnyMaxRowBlocks = 65535;

bool skinny_fits(int64_t ldx1, int64_t ldx2, int layout) {
  return ldx1 < kSkinnyMaxLdx1 && ldx2 < ((layout & TILEC_X2_COL_MAJOR) ? kSkinnyMaxLdx2ColMajor : kSkinnyMaxLdx2);
}

// Output tiles of the smallest tile GEMM (64 x 64): below one per CU the
// tile GEMMs cannot fill the chip and the streaming kernel, which splits K,
// takes the product.
bool small_output(int64_t M, int64_t N) { return cdiv(M, 64) * cdiv(N, 64) < device_cus(); }

// Tile-GEMM split-K partials are addressed with 32-bit byte offsets
// (splits * tiles * BM * BN * 4 < 2^31) and splits are grid y (<= 65535).
constexpr int64_t kGemmMaxPartialBytes = (int64_t(1) << 31) - 1;

int64_t gemm_tiles(const VariantDesc* d, int64_t M, int64_t N) { return cdiv(M, d->bm) * cdiv(N, d->bn); }

size_t gemm_workspace_bytes(const VariantDesc* d, int64_t M, int64_t N, int64_t K, int s) {
  if (d->prep) return K > 0 ? prep_workspace_bytes(M, N, K) : 0;
  const SplitGeom g = gemm_split_geom(K, d->bk, s);
  if (g.splits <= 1) return 0;
  return (size_t)g.splits * gemm_tiles(d, M, N) * d->bm * d->bn * sizeof(float);
}
size_t gemm_counter_bytes(const VariantDesc* d, int64_t M, int64_t N, int64_t K, int s) {
  if (d->prep || gemm_split_geom(K, d->bk, s).splits <= 1) return 0;
  return (size_t)gemm_tiles(d, M, N) * kSplitCounterStride * sizeof(unsigned);
}

// Scratch a variant needs for a split K.
size_t variant_workspace_bytes(const VariantDesc* d, int dtype, int64_t M, int64_t N, int64_t K, int s) {
  if (d->workspace_bytes) return d->workspace_bytes(*d, M, N, K, s);
  return d->family == TILEC_FAMILY_SKINNY ? skinny_workspace_bytes(dtype, M, N, K, s)
                                          : gemm_workspace_bytes(d, M, N, K, s);
}
size_t variant_counter_bytes(const VariantDesc* d, int dtype, int64_t M, int64_t N, int64_t K, int s) {
  if (d->counter_bytes) return d->counter_bytes(*d, M, N, K, s);
  return d->family == TILEC_FAMILY_SKINNY ? skinny_counter_bytes(dtype, M, N, K, s)
                                          : gemm_counter_bytes(d, M, N, K, s);
}

// Built-in rule (used when the caller passes TILEC_VARIANT_AUTO).
int auto_variant(int64_t M, int64_t N, int64_t K, int dtype, int64_t ldx1, int64_t ldx2, int layout) {
  const int cus = device_cus();
  // x @ W.T with M <= 16: the row-dot kernel for M = 1, the row-tile kernel
  // above (no K split; both run the streaming kernel themselves when the
  // operands are not 16-byte aligned).  Their workspace and counter needs
  // (those of that fallback, at the split auto_split gives them, which is
  // never above the streaming variant's) never exceed those of the streaming
  // variant chosen below for the same shape in another layout, so sizes
  // queried with TILEC_VARIANT_AUTO still suffice.
  const int64_t epl = dtype == TILEC_F32 ? 4 : 8;  // elements per 16-byte load
  // (the row-dot kernel takes any element alignment, the row-tile kernel
  // whole 16-byte rows)
  if ((layout & 3) == TILEC_X2_COL_MAJOR && M == 1 && skinny_fits(ldx1, ldx2, layout))
    return find(dtype == TILEC_F32 ? "skinny_f32_t1_r1_w8_u2" : "skinny_bf16_t1_r1_w8_u2");
  if ((layout & 3) == TILEC_X2_COL_MAJOR && M >= 2 && M <= 16 && K % epl == 0 && ldx1 % epl == 0 &&
      ldx2 % epl == 0 && skinny_fits(ldx1, ldx2, layout)) {
    // one workgroup per 16 rows of W: with fewer than half the CUs busy
    // and a long K, the streaming kernel's K split (below) is faster
    if (cdiv(N, 16) >= cus / 2 || K <= 2048)
      return find(dtype == TILEC_F32 ? "skinny_f32_t16_r16_w8_c128" : "skinny_bf16_t16_r16_w8_c128");
  }
  // Row-major x2 with M == 1: the panel kernel (512-byte row pieces, about
  // one workgroup per CU; it runs the streaming kernel itself for operands it
  // does not take).  Its M <= 4 variants are the tuner's to pick: at
  // K = N = 4096 they trail the streaming kernel for 2 <= M <= 4.
  if (!(layout & TILEC_X2_COL_MAJOR) && M == 1 && skinny_fits(ldx1, ldx2, layout))
    return find(dtype == TILEC_F32 ? "skinny_f32_p_v1_w8" : "skinny_bf16_p_v1_w8");
  if (dtype == TILEC_F32) {
    if (M <= 16 && skinny_fits(ldx1, ldx2, layout)) return find("skinny_f32_w8_b1");
    // Few output tiles past 16 rows: the direct-operand MFMA kernel, K split
    // across workgroups (on MI355X within 1.15x of the best measured config
    // for such shapes, geometric mean; the streaming kernel: 1.9x).
    if (small_output(M, N)) return find("direct_f32_32x64_w4");
    // Up to four 64x64 tiles per CU but too few 128x128 tiles to give each CU
    // one (1024^2-sized outputs): the direct kernel's 32x64 tile with two
    // register sets, unsplit or nearly (on MI355X within 1.10x of the best
    // measured config over the 53 such and larger fp32 shapes timed,
    // geometric mean; the tile GEMMs below alone: 1.37x).
    // Where its 64x64 tiles give every CU one or two, the direct-to-LDS 64x64
    // tile GEMM instead (1024^3 on MI355X: 18.4 us against 23.4 us).
    if (cdiv(M, 128) * cdiv(N, 128) < cus && cdiv(M, 64) * cdiv(N, 64) <= 4 * (int64_t)cus) {
      const int64_t t64 = cdiv(M, 64) * cdiv(N, 64);
      if (t64 >= cus && t64 <= 2 * (int64_t)cus) return find("gemm_f32_64x64x32_w2x2_lds");
      return find("direct_f32_32x64_w4_db");
    }
    // (the *_lds tiles run the register-staged kernel of the same tile for
    // operands their direct-to-LDS copies do not take)
    static const char* order[] = {"gemm_f32_256x256x32_w2x4_lds", "gemm_f32_256x128x16_w2x2",
                                  "gemm_f32_128x128x32_w2x4_lds", "gemm_f32_128x64x16_w2x2"};
    for (const char* nm : order) {
      const int v = find(nm);
      const VariantDesc* d = table()[v];
      if (cdiv(M, d->bm) * cdiv(N, d->bn) >= cus) return v;
    }
    return find("gemm_f32_64x64x16_w2x2");
  }
  // bf16: the streaming kernel for M <= 16 (it runs fp32 MFMAs on widened
  // inputs, so more rows are better served by the bf16 tile GEMMs).
  if (M <= 16 && skinny_fits(ldx1, ldx2, layout)) return find("skinny_bf16_w8_b1");
  static const char* order[] = {"gemm_bf16_256x256x64_r2_m16", "gemm_bf16_256x128x64_r3_m16",
                                "gemm_bf16_128x128x64_r4"};
  for (const char* nm : order) {
    const int v = find(nm);
    const VariantDesc* d = table()[v];
    if (cdiv(M, d->bm) * cdiv(N, d->bn) >= cus) return v;
  }
  // Few output tiles: the 128 x 128 LDS kernel, with K split to fill the chip.
  return find("gemm_bf16_128x128x64_r4");
}

// split_k == 0.  Streaming kernels: enough workgroups for the variant's
// workgroups per CU (2 for the streaming kernel, 1 for the panel kernel), while
// every wave still gets at least one full unrolled batch of rows.  Tile
// GEMMs: unsplit when the tiles alone fill the CUs, else about one workgroup
// per CU, keeping at least 4 K steps per split (at most 16 splits).
int auto_split(const VariantDesc* d, int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 1;
  const int cus = device_cus();
  if (d->family == TILEC_FAMILY_GEMM) {
    const int64_t tiles = gemm_tiles(d, M, N);
    if (tiles >= cus || d->prep || !tile_can_split(d->bm, d->bn, d->waves)) return 1;
    int64_t s = cdiv(cus, tiles);
    const int64_t s_max = cdiv(K, d->bk) / 4;
    if (s > s_max) s = s_max;
    if (s > 16) s = 16;
    return s < 1 ? 1 : (int)s;
  }
  // Streaming kernels: enough workgroups for the variant's workgroups per
  // CU.  Direct kernels: at most that many, so no CU runs more chunks than
  // the others (a grid a little over the CU count leaves a few CUs with two
  // chunks each, and every tile then waits for them).
  const int64_t cells = cdiv(N, d->bn) * cdiv(M, d->bm);
  int64_t s = d->family == TILEC_FAMILY_DIRECT ? (int64_t)d->wgs_per_cu * cus / cells
                                              : cdiv((int64_t)d->wgs_per_cu * cus, cells);
  const int64_t rows_per_split_min = 16LL * d->waves;  // one 16-row block per wave
  const int64_t s_max = K / rows_per_split_min;
  if (s > s_max) s = s_max;
  if (s < 1) s = 1;
  if (s > 1024) s = 1024;
  return (int)s;
}

// The streaming kernel's split-K partials take 32-bit byte offsets.
int skinny_partials_check(const VariantDesc* d, int64_t M, int64_t N, int64_t K, int s) {
  const int64_t splits = skinny_effective_splits(N, K, s);
  const int64_t cells = cdiv(N, d->bn) * cdiv(M, d->bm);
  if (splits > 1 && splits * cells * d->bm * d->bn * 4 >= (int64_t(1) << 31))
    return fail(TILEC_ERR_UNSUPPORTED, "tilec: %s: %lld splits x %lld output blocks of partials is too many",
                d->name, (long long)splits, (long long)cells);
  return TILEC_OK;
}

// ldx1 / ldx2 <= 0 mean "contiguous" (K and N for row-major operands, M and
// K for column-major ones).
int resolve(int64_t M, int64_t N, int64_t K, int32_t dtype, int32_t variant, int32_t split_k,
            const VariantDesc** out_d, int* out_split, int64_t ldx1 = 0, int64_t ldx2 = 0, int layout = 0) {
  if (dtype != TILEC_F32 && dtype != TILEC_BF16)
    return fail(TILEC_ERR_TYPE, "tilec: unsupported dtype code %d (use float32 or bfloat16)", dtype);
  if (M < 0 || N < 0 || K < 0 || M > kMaxDim || N > kMaxDim || K > kMaxDim)
    return fail(TILEC_ERR_VALUE, "tilec: bad shape M=%lld N=%lld K=%lld", (long long)M, (long long)N,
                (long long)K);
  if (split_k < 0) return fail(TILEC_ERR_VALUE, "tilec: split_k must be >= 0 (got %d)", split_k);
  if (layout & ~(TILEC_X1_COL_MAJOR | TILEC_X2_COL_MAJOR))
    return fail(TILEC_ERR_VALUE, "tilec: unknown layout bits 0x%x", layout);
  if (ldx1 <= 0) ldx1 = (layout & TILEC_X1_COL_MAJOR) ? M : K;
  if (ldx2 <= 0) ldx2 = (layout & TILEC_X2_COL_MAJOR) ? K : N;
  const auto& t = table();
  int v = variant;
  if (v == TILEC_VARIANT_AUTO) {
    v = auto_variant(M, N, K, dtype, ldx1, ldx2, layout);
  } else if (v < 0 || v >= (int)t.size()) {
    return fail(TILEC_ERR_UNSUPPORTED, "tilec: unknown variant %d (have %d)", v, (int)t.size());
  }
  const VariantDesc* d = t[v];
  if (d->dtype != dtype)
    return fail(TILEC_ERR_UNSUPPORTED, "tilec: variant %s is for dtype %d, not %d", d->name, d->dtype, dtype);
  if (d->max_m > 0 && M > d->max_m)
    return fail(TILEC_ERR_UNSUPPORTED, "tilec: variant %s takes M <= %d (got %lld)", d->name, d->max_m,
                (long long)M);
  if (d->family == TILEC_FAMILY_SKINNY && !skinny_fits(ldx1, ldx2, layout))
    return fail(TILEC_ERR_UNSUPPORTED, "tilec: %s needs ldx1 < 2^25 and ldx2 < 2^%d", d->name,
                (layout & TILEC_X2_COL_MAJOR) ? 23 : 25);
  int s = split_k == 0 ? auto_split(d, M, N, K) : split_k;
  if (d->family == TILEC_FAMILY_GEMM) {
    const SplitGeom g = gemm_split_geom(K, d->bk, s);
    if (g.splits > 1 && (d->prep || !tile_can_split(d->bm, d->bn, d->waves)))
      return fail(TILEC_ERR_UNSUPPORTED, "tilec: variant %s does not split K (split_k=%d)", d->name, s);
    if (d->prep && M * K * 2 + K * N * 2 >= (int64_t(1) << 40))
      return fail(TILEC_ERR_UNSUPPORTED, "tilec: %s: operands too large to transpose", d->name);
    if (g.splits > 65535)
      return fail(TILEC_ERR_VALUE, "tilec: split_k=%d gives more than 65535 splits", s);
    if (g.splits > 1 && (int64_t)gemm_workspace_bytes(d, M, N, K, s) > kGemmMaxPartialBytes)
      return fail(TILEC_ERR_UNSUPPORTED, "tilec: %s: %lld splits of %lld tiles of partials is too many", d->name,
                  (long long)g.splits, (long long)gemm_tiles(d, M, N));
  }
  if (d->family == TILEC_FAMILY_DIRECT) {
    const int64_t splits = direct_effective_splits(K, s);
    const int64_t tiles = cdiv(N, d->bn) * cdiv(M, d->bm);
    if (splits > 65535)
      return fail(TILEC_ERR_VALUE, "tilec: split_k=%d gives more than 65535 splits", s);
    if (tiles > 0x7FFFFFFF)
      return fail(TILEC_ERR_UNSUPPORTED, "tilec: %s: %lld output tiles is too many", d->name, (long long)tiles);
    if (splits > 1 && (int64_t)d->workspace_bytes(*d, M, N, K, s) >= (int64_t(1) << 31))
      return fail(TILEC_ERR_UNSUPPORTED, "tilec: %s: %lld splits x %lld tiles of partials is too many", d->name,
                  (long long)splits, (long long)tiles);
  }
  if (d->family == TILEC_FAMILY_SKINNY) {
    if (cdiv(M, d->bm) > kSkinnyMaxRowBlocks)
      return fail(TILEC_ERR_UNSUPPORTED, "tilec: %s takes M <= %lld (got %lld)", d->name,
                  (long long)(kSkinnyMaxRowBlocks * d->bm), (long long)M);
    if (skinny_effective_splits(N, K, s) > 65535)
      return fail(TILEC_ERR_VALUE, "tilec: split_k=%d gives more than 65535 splits", s);
    // Row-dot / row-tile variants: checked by tilec_matmul once it knows
    // whether their own kernel (no partials) or the streaming fallback runs.
    if (!d->own_kernel_runs) {
      const int rc = skinny_partials_check(d, M, N, K, s);
      if (rc != TILEC_OK) return rc;
    }
    // Variants with their own split geometry (the panel kernel: at least
    // K / KC splits, partials addressed with 32-bit offsets).  Their size
    // query covers both their own kernel and the streaming fallback.
    if (d->effective_splits && d->effective_splits(*d, N, K, s) > 65535)
      return fail(TILEC_ERR_VALUE, "tilec: %s: K=%lld with split_k=%d gives more than 65535 splits", d->name,
                  (long long)K, s);
    if (d->workspace_bytes && M > 0 && N > 0 &&
        (int64_t)d->workspace_bytes(*d, M, N, K, s) >= (int64_t(1) << 31))
      return fail(TILEC_ERR_UNSUPPORTED, "tilec: %s: K=%lld needs 2 GiB or more of split-K partials", d->name,
                  (long long)K);
  }
  *out_d = d;
  *out_split = s;
  return TILEC_OK;
}

// Sums: validate, then express a column-major x as the row-major view of its
// transpose (swap R and C, flip the axis).  The kernels address the rows of
// one wave (axis 1: 64 / lpr rows) or one 16-row block (axis 0) with 32-bit
// byte offsets, and their split partials likewise.
struct SumPlan {
  int64_t R, C;
  int axis, esz;
  ReduceGeom g;
};

int sum_plan(int64_t R, int64_t C, int64_t ldx, int32_t layout, int32_t dtype, int32_t axis, SumPlan* p) {
  if (dtype != TILEC_F32 && dtype != TILEC_BF16)
    return fail(TILEC_ERR_TYPE, "tilec: unsupported dtype code %d (use float32 or bfloat16)", dtype);
  if (R < 0 || C < 0 || R > kMaxDim || C > kMaxDim)
    return fail(TILEC_ERR_VALUE, "tilec: bad shape R=%lld C=%lld", (long long)R, (long long)C);
  if (axis != 0 && axis != 1) return fail(TILEC_ERR_VALUE, "tilec: axis must be 0 or 1 (got %d)", axis);
  if (layout & ~TILEC_X1_COL_MAJOR) return fail(TILEC_ERR_VALUE, "tilec: unknown layout bits 0x%x", layout);
  const bool col = layout & TILEC_X1_COL_MAJOR;
  p->R = col ? C : R;
  p->C = col ? R : C;
  p->axis = col ? 1 - axis : axis;
  p->esz = dtype == TILEC_BF16 ? 2 : 4;
  if (ldx > 0 && ldx >= (int64_t(1) << 40)) return fail(TILEC_ERR_VALUE, "tilec: ldx=%lld is too large", (long long)ldx);
  if (p->axis == 1 && p->C * p->esz >= (int64_t(1) << 31) - 64)
    return fail(TILEC_ERR_UNSUPPORTED, "tilec: rows of %lld elements are too long to sum", (long long)p->C);
  if (p->axis == 0 && ldx > 0 && 16 * ldx * p->esz >= (int64_t(1) << 31) - 64)
    return fail(TILEC_ERR_UNSUPPORTED, "tilec: a row stride of %lld elements is too large for column sums",
                (long long)ldx);
  p->g = reduce_geom(p->R, p->C, p->esz, p->axis);
  // Row sums address a wave's 64 / lpr rows from its first one.
  if (p->axis == 1 && ldx > 0 && (64 / p->g.lpr) * ldx * p->esz + p->C * p->esz >= (int64_t(1) << 31) - 64)
    return fail(TILEC_ERR_UNSUPPORTED, "tilec: a row stride of %lld elements is too large for sums of short rows",
                (long long)ldx);
  if (p->g.splits > 65535 || p->g.cells > 0x7FFFFFFF ||
      (int64_t)reduce_workspace_bytes(p->g) >= (int64_t(1) << 31))
    return fail(TILEC_ERR_UNSUPPORTED, "tilec: sum of %lld x %lld is too large", (long long)R, (long long)C);
  return TILEC_OK;
}

// ---------------------------------------------------------------------------
// Scratch of tilec_matmul_noalloc: one static device array per GPU, held
// until the process ends.  Split-K partials in the first kWsMax bytes,
// completion counters (zero at rest) in the next kCntMax.
// ---------------------------------------------------------------------------
constexpr size_t kNoallocWsMax = size_t(16) << 20;
constexpr size_t kNoallocCntMax = size_t(1) << 20;
static __device__ __align__(256) unsigned char scratch[kNoallocWsMax + kNoallocCntMax];

constexpr int kMaxDevices = 64;
std::atomic<unsigned char*> g_scratch[kMaxDevices];  // device address of `scratch` per device (set up once)
std::mutex g_scratch_mu;

__global__ void zero_words(unsigned* __restrict__ p, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = 0u;
}

// Device address of `scratch` on the current device.  The first call on a
// device looks it up (the array's name in host code is only a stand-in) and
// clears the counter area with a fill kernel on `stream` (no memset node, so
// a captured first call replays correctly); the device's static memory is
// zero at load anyway.
int scratch_of_current_device(hipStream_t stream, unsigned char** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(TILEC_ERR_HIP, "tilec: hipGetDevice failed: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(TILEC_ERR_UNSUPPORTED, "tilec: device %d: tilec_matmul_noalloc serves devices 0..%d", dev,
                kMaxDevices - 1);
  unsigned char* p = g_scratch[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      void* addr = nullptr;
      e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
      if (e != hipSuccess || addr == nullptr)
        return fail(TILEC_ERR_HIP, "tilec: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                    hipGetErrorString(e));
      p = static_cast<unsigned char*>(addr);
      hipLaunchKernelGGL(zero_words, dim3(64), dim3(256), 0, stream, reinterpret_cast<unsigned*>(p + kNoallocWsMax),
                         kNoallocCntMax / sizeof(unsigned));
      e = hipGetLastError();
      if (e != hipSuccess)
        return fail(TILEC_ERR_HIP, "tilec: clearing the scratch counters failed: %s", hipGetErrorString(e));
      g_scratch[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return TILEC_OK;
}

}  // namespace

extern "C" {

int tilec_sum(const void* x, float* out, int64_t R, int64_t C, int64_t ldx, int32_t layout, int32_t dtype,
              int32_t axis, void* workspace, size_t workspace_bytes, void* counters, size_t counter_bytes,
              void* stream) {
  g_err[0] = 0;
  SumPlan p;
  const int rc = sum_plan(R, C, ldx, layout, dtype, axis, &p);
  if (rc != TILEC_OK) return rc;
  const int64_t outputs = axis == 1 ? R : C;
  if (outputs == 0) return TILEC_OK;
  if (out == nullptr) return fail(TILEC_ERR_VALUE, "tilec: out is NULL");
  if (R > 0 && C > 0) {
    if (x == nullptr) return fail(TILEC_ERR_VALUE, "tilec: x is NULL");
    if (ldx < p.C)
      return fail(TILEC_ERR_VALUE, "tilec: ldx=%lld < %s=%lld", (long long)ldx,
                  (layout & TILEC_X1_COL_MAJOR) ? "R" : "C", (long long)p.C);
  }
  const size_t need = reduce_workspace_bytes(p.g), need_cnt = reduce_counter_bytes(p.g);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need))
    return fail(TILEC_ERR_WORKSPACE, "tilec: sum needs %zu workspace bytes (got %zu)", need,
                workspace == nullptr ? (size_t)0 : workspace_bytes);
  if (need_cnt > 0 && (counters == nullptr || counter_bytes < need_cnt))
    return fail(TILEC_ERR_WORKSPACE, "tilec: sum needs %zu bytes of counters (got %zu)", need_cnt,
                counters == nullptr ? (size_t)0 : counter_bytes);
  const hipError_t e = launch_reduce(x, out, p.R, p.C, ldx > 0 ? ldx : std::max<int64_t>(p.C, 1), dtype, p.axis,
                                     static_cast<float*>(workspace), static_cast<unsigned*>(counters),
                                     static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(TILEC_ERR_HIP, "tilec: launching the sum failed: %s", hipGetErrorString(e));
  return TILEC_OK;
}

int tilec_read_floor(const void* x, size_t bytes, float* sink, int32_t workgroups, void* stream) {
  g_err[0] = 0;
  constexpr size_t kPiece = 16384;
  if (bytes % kPiece != 0)
    return fail(TILEC_ERR_VALUE, "tilec: read floor: bytes=%zu is not a multiple of 16 KiB", bytes);
  if (bytes > (size_t(1) << 40)) return fail(TILEC_ERR_VALUE, "tilec: read floor: bytes=%zu is too large", bytes);
  if (workgroups < 0) return fail(TILEC_ERR_VALUE, "tilec: read floor: workgroups=%d < 0", workgroups);
  if (bytes == 0) return TILEC_OK;
  if (x == nullptr || sink == nullptr) return fail(TILEC_ERR_VALUE, "tilec: read floor: x/sink is NULL");
  if (reinterpret_cast<uintptr_t>(x) % 16 != 0)
    return fail(TILEC_ERR_VALUE, "tilec: read floor: x is not 16-byte aligned");
  const int64_t pieces = (int64_t)(bytes / kPiece);
  int64_t g = workgroups > 0 ? workgroups : 2 * (int64_t)device_cus();
  if (g > pieces) g = pieces;
  const hipError_t e = launch_read_floor(x, (int64_t)bytes, sink, (int)g, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(TILEC_ERR_HIP, "tilec: launching the read floor failed: %s", hipGetErrorString(e));
  return TILEC_OK;
}

size_t tilec_sum_workspace_bytes(int64_t R, int64_t C, int32_t layout, int32_t dtype, int32_t axis) {
  SumPlan p;
  if (sum_plan(R, C, 0, layout, dtype, axis, &p) != TILEC_OK || (axis == 1 ? R : C) == 0) return 0;
  return reduce_workspace_bytes(p.g);
}

size_t tilec_sum_counter_bytes(int64_t R, int64_t C, int32_t layout, int32_t dtype, int32_t axis) {
  SumPlan p;
  if (sum_plan(R, C, 0, layout, dtype, axis, &p) != TILEC_OK || (axis == 1 ? R : C) == 0) return 0;
  return reduce_counter_bytes(p.g);
}

int tilec_matmul(const void* x1, const void* x2, float* out, int64_t M, int64_t N, int64_t K, int64_t ldx1,
                 int64_t ldx2, int64_t ldo, int32_t layout, int32_t dtype, int32_t variant, int32_t split_k,
                 void* workspace, size_t workspace_bytes, void* counters, size_t counter_bytes, void* stream) {
  g_err[0] = 0;
  const VariantDesc* d = nullptr;
  int s = 1;
  int rc = resolve(M, N, K, dtype, variant, split_k, &d, &s, ldx1, ldx2, layout);
  if (rc != TILEC_OK) return rc;
  if (M == 0 || N == 0) return TILEC_OK;
  if (ldo < N) return fail(TILEC_ERR_VALUE, "tilec: ldo=%lld < N=%lld", (long long)ldo, (long long)N);
  if (out == nullptr) return fail(TILEC_ERR_VALUE, "tilec: out is NULL");
  if (K > 0) {
    if (x1 == nullptr || x2 == nullptr) return fail(TILEC_ERR_VALUE, "tilec: x1/x2 is NULL");
    const bool c1 = layout & TILEC_X1_COL_MAJOR, c2 = layout & TILEC_X2_COL_MAJOR;
    const int64_t need1 = c1 ? M : K, need2 = c2 ? K : N;
    if (ldx1 < need1)
      return fail(TILEC_ERR_VALUE, "tilec: ldx1=%lld < %s=%lld", (long long)ldx1, c1 ? "M" : "K", (long long)need1);
    if (ldx2 < need2)
      return fail(TILEC_ERR_VALUE, "tilec: ldx2=%lld < %s=%lld", (long long)ldx2, c2 ? "K" : "N", (long long)need2);
  }
  MatmulArgs a;
  a.x1 = x1;
  a.x2 = x2;
  a.out = out;
  a.M = M;
  a.N = N;
  a.K = K;
  a.ldx1 = ldx1 > 0 ? ldx1 : 1;
  a.ldx2 = ldx2 > 0 ? ldx2 : 1;
  a.ldo = ldo;
  a.layout = layout;
  a.split_k = s;
  a.workspace = workspace;
  a.workspace_bytes = workspace_bytes;
  a.counters = static_cast<unsigned*>(counters);
  a.counter_bytes = counter_bytes;
  a.stream = static_cast<hipStream_t>(stream);
  // Scratch is required only where a kernel that splits K will run: a
  // row-dot / row-tile variant whose own kernel takes these operands needs
  // none (the size queries, which cannot see the pointers, stay
  // conservative).
  if (!(d->own_kernel_runs && d->own_kernel_runs(a))) {
    if (d->own_kernel_runs) {
      rc = skinny_partials_check(d, M, N, K, s);
      if (rc != TILEC_OK) return rc;
    }
    const size_t need = variant_workspace_bytes(d, dtype, M, N, K, s);
    if (need > 0 && (workspace == nullptr || workspace_bytes < need))
      return fail(TILEC_ERR_WORKSPACE, "tilec: %s needs %zu workspace bytes (got %zu)", d->name, need,
                  workspace == nullptr ? (size_t)0 : workspace_bytes);
    const size_t need_cnt = variant_counter_bytes(d, dtype, M, N, K, s);
    if (need_cnt > 0 && (counters == nullptr || counter_bytes < need_cnt))
      return fail(TILEC_ERR_WORKSPACE, "tilec: %s needs %zu bytes of counters (got %zu)", d->name, need_cnt,
                  counters == nullptr ? (size_t)0 : counter_bytes);
  }
  const hipError_t e = d->launch(a);
  if (e != hipSuccess)
    return fail(TILEC_ERR_HIP, "tilec: launching %s failed: %s", d->name, hipGetErrorString(e));
  return TILEC_OK;
}

int tilec_matmul_noalloc(const void* x1, const void* x2, float* out, int64_t M, int64_t N, int64_t K,
                         int64_t ldx1, int64_t ldx2, int64_t ldo, int32_t layout, int32_t dtype, int32_t variant,
                         int32_t split_k, void* stream) {
  g_err[0] = 0;
  size_t ws = 0, cnt = 0;
  const int qrc = tilec_matmul_scratch_bytes(M, N, K, ldx1, ldx2, layout, dtype, variant, split_k, &ws, &cnt);
  if (qrc != TILEC_OK) return qrc;
  if (ws > kNoallocWsMax || cnt > kNoallocCntMax)
    return fail(TILEC_ERR_WORKSPACE,
                "tilec: this call needs %zu bytes of scratch and %zu of counters; tilec_matmul_noalloc has %zu and "
                "%zu (use tilec_matmul with caller-owned buffers)",
                ws, cnt, kNoallocWsMax, kNoallocCntMax);
  unsigned char* base = nullptr;
  if (ws > 0 || cnt > 0) {
    const int rc = scratch_of_current_device(static_cast<hipStream_t>(stream), &base);
    if (rc != TILEC_OK) return rc;
  }
  return tilec_matmul(x1, x2, out, M, N, K, ldx1, ldx2, ldo, layout, dtype, variant, split_k,
                      base, base ? kNoallocWsMax : 0, base ? base + kNoallocWsMax : nullptr,
                      base ? kNoallocCntMax : 0, stream);
}

int tilec_matmul_scratch_bytes(int64_t M, int64_t N, int64_t K, int64_t ldx1, int64_t ldx2, int32_t layout,
                               int32_t dtype, int32_t variant, int32_t split_k, size_t* workspace_bytes,
                               size_t* counter_bytes) {
  g_err[0] = 0;
  if (workspace_bytes) *workspace_bytes = 0;
  if (counter_bytes) *counter_bytes = 0;
  const VariantDesc* d = nullptr;
  int s = 1;
  const int rc = resolve(M, N, K, dtype, variant, split_k, &d, &s, ldx1, ldx2, layout);
  if (rc != TILEC_OK) return rc;
  if (M == 0 || N == 0) return TILEC_OK;
  if (workspace_bytes) *workspace_bytes = variant_workspace_bytes(d, dtype, M, N, K, s);
  if (counter_bytes) *counter_bytes = variant_counter_bytes(d, dtype, M, N, K, s);
  return TILEC_OK;
}

size_t tilec_matmul_workspace_bytes(int64_t M, int64_t N, int64_t K, int32_t dtype, int32_t variant,
                                    int32_t split_k) {
  const VariantDesc* d = nullptr;
  int s = 1;
  if (resolve(M, N, K, dtype, variant, split_k, &d, &s) != TILEC_OK) return 0;
  if (M == 0 || N == 0) return 0;
  return variant_workspace_bytes(d, dtype, M, N, K, s);
}

size_t tilec_matmul_counter_bytes(int64_t M, int64_t N, int64_t K, int32_t dtype, int32_t variant,
                                  int32_t split_k) {
  const VariantDesc* d = nullptr;
  int s = 1;
  if (resolve(M, N, K, dtype, variant, split_k, &d, &s) != TILEC_OK) return 0;
  if (M == 0 || N == 0) return 0;
  return variant_counter_bytes(d, dtype, M, N, K, s);
}

int32_t tilec_select_variant_layout(int64_t M, int64_t N, int64_t K, int32_t dtype, int32_t layout,
                                    int64_t ldx1, int64_t ldx2) {
  const VariantDesc* d = nullptr;
  int s = 1;
  const int rc = resolve(M, N, K, dtype, TILEC_VARIANT_AUTO, 0, &d, &s, ldx1, ldx2, layout);
  if (rc != TILEC_OK) return -rc;
  if (ldx1 <= 0) ldx1 = (layout & TILEC_X1_COL_MAJOR) ? M : K;
  if (ldx2 <= 0) ldx2 = (layout & TILEC_X2_COL_MAJOR) ? K : N;
  return auto_variant(M, N, K, dtype, ldx1, ldx2, layout);
}

int32_t tilec_select_variant(int64_t M, int64_t N, int64_t K, int32_t dtype) {
  return tilec_select_variant_layout(M, N, K, dtype, 0, 0, 0);
}

int32_t tilec_auto_split_k(int64_t M, int64_t N, int64_t K, int32_t dtype, int32_t variant) {
  const VariantDesc* d = nullptr;
  int s = 1;
  const int rc = resolve(M, N, K, dtype, variant, 0, &d, &s);
  if (rc != TILEC_OK) return -rc;
  return s;
}

int32_t tilec_num_variants(void) { return (int32_t)table().size(); }

int tilec_variant_info(int32_t variant, int32_t info[8], const char** name) {
  const auto& t = table();
  if (variant < 0 || variant >= (int)t.size())
    return fail(TILEC_ERR_UNSUPPORTED, "tilec: unknown variant %d", variant);
  const VariantDesc* d = t[variant];
  if (info) {
    info[0] = d->family;
    info[1] = d->dtype;
    info[2] = d->bm;
    info[3] = d->bn;
    info[4] = d->bk;
    info[5] = d->waves;
    info[6] = d->max_m;
    info[7] = d->unroll;
  }
  if (name) *name = d->name;
  return TILEC_OK;
}

const char* tilec_last_error(void) { return g_err; }

int32_t tilec_version(void) { return 10100; }

}  // extern "C"
