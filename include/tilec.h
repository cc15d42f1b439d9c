/*
 * tilec.h — C ABI of libtilec_hip.so, the MI355X (gfx950) implementation of
 * tilec's matmul op.
 *
 * The reference crosses its host→device boundary in one place: the launch of
 * the tile kernel `_matmul_tiled[(cdiv(M,BM), cdiv(N,BN))](a, b, c, M, N, K,
 * BM=, BN=, BK=)` issued by `_matrix_mul_tiled` (tilec/ext.py:54-63), which
 * goes through `JITFunction.run` / `_launch` (tilec/jit.py:81-105) into
 * `torch.mps.compile_shader(...)(*buffers, threads=..., group_size=...)`.
 * Every entry point below replaces a piece of that path; the Python caller is
 * tilec/ext.py (via ctypes), which keeps the reference's public signature
 * `matrix_mul(x1, x2)` (tilec/ext.py:66-67).
 *
 * Conventions shared by all entry points
 *   - The output is row-major with unit column stride; ldo is its row stride
 *     in elements (>= N).  Each input is row-major (ld* = row stride >= its
 *     number of columns) or, when its `layout` bit is set, column-major
 *     (ld* = column stride >= its number of rows) — the transposed view
 *     x.T of a contiguous matrix, read in place.  The reference makes every
 *     input row-major contiguous first (`.contiguous()`, tilec/ext.py:59-60;
 *     then ld == the number of columns); strided and transposed views skip
 *     that copy here.
 *   - Outputs are float32.  Inputs are float32, or bfloat16 (fp32 accumulate).
 *   - Nothing here allocates device memory, synchronizes, or reads the device
 *     back: work is enqueued on `stream` (a hipStream_t; NULL = the legacy
 *     default stream) and returns at once, like the reference's asynchronous
 *     MPS launch (tilec/jit.py:105).
 *   - Functions return a status code (TILEC_OK == 0).  On failure
 *     tilec_last_error() returns a message for the calling thread.  The Python
 *     caller maps TILEC_ERR_VALUE to ValueError (the reference's shape error,
 *     tilec/ext.py:57-58), TILEC_ERR_TYPE to TypeError (tilec/jit.py:34-39)
 *     and the rest to RuntimeError.
 */
#ifndef TILEC_H
#define TILEC_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
#define TILEC_OK 0
#define TILEC_ERR_VALUE 1       /* bad shape, stride, pointer or split   */
#define TILEC_ERR_TYPE 2        /* unsupported dtype                      */
#define TILEC_ERR_UNSUPPORTED 3 /* variant unknown or not valid for shape */
#define TILEC_ERR_WORKSPACE 4   /* workspace missing or too small         */
#define TILEC_ERR_HIP 5         /* HIP runtime error at launch            */

/* Element types of x1 / x2 (the output is always float32). */
#define TILEC_F32 0
#define TILEC_BF16 1

/* Kernel families (tilec_variant_info, info[0]). */
#define TILEC_FAMILY_SKINNY 0 /* output-stationary streaming kernel, split K:   */
                              /* M <= 16, or outputs of few 64x64 tiles         */
#define TILEC_FAMILY_GEMM 1   /* LDS-staged MFMA tile GEMM                      */
#define TILEC_FAMILY_DIRECT 2 /* fp32 MFMA on operands loaded straight into     */
                              /* registers, split K: GEMV and small outputs     */

/* Operand layouts: bits of tilec_matmul's `layout` (0 = both row-major). */
#define TILEC_X1_COL_MAJOR 1 /* x1 element (m, k) at x1[m + k * ldx1], ldx1 >= M */
#define TILEC_X2_COL_MAJOR 2 /* x2 element (k, n) at x2[k + n * ldx2], ldx2 >= K */

/* Pass as `variant` to let the library pick with its built-in rule. */
#define TILEC_VARIANT_AUTO (-1)

/*
 * out[M,N] = x1[M,K] · x2[K,N]
 *
 * Replaces the launch `_matmul_tiled[grid](x1, x2, out, M, N, K, BM, BN, BK)`
 * (tilec/ext.py:62; kernel semantics tilec/ext.py:13-24; launch
 * tilec/jit.py:88-105).  `variant` selects a compiled kernel (see
 * tilec_num_variants / tilec_variant_info) the way the reference's constexpr
 * tile sizes select a compiled specialization (tilec/jit.py:66-76);
 * `split_k` (0 = automatic) splits the reduction dimension across
 * workgroups, the role of the legacy `split` config (tilec/ext.py:37,48-51).
 *
 * `layout` (TILEC_X1_COL_MAJOR | TILEC_X2_COL_MAJOR) says how x1 and x2 are
 * stored; every variant takes every layout.  The reference has no such
 * argument: it copies each input to row-major first (tilec/ext.py:59-60).
 *
 * M == 0 or N == 0 enqueues nothing.  K == 0 writes zeros (the reference's
 * accumulator starts at zero and its K loop runs no iterations).
 *
 * A split K needs two device buffers (NULL/0 when their size is 0):
 *   `workspace` — tilec_matmul_workspace_bytes(...) bytes of scratch for the
 *                 partial sums; any contents;
 *   `counters`  — tilec_matmul_counter_bytes(...) bytes of completion
 *                 counters that must be zero before the call.  Every call
 *                 that completes leaves them zero again, so a buffer zeroed
 *                 once at allocation serves all later calls on one stream,
 *                 whatever their shapes, as long as it is large enough.
 * Calls that run concurrently (different streams) need their own buffers.
 */
int tilec_matmul(const void* x1, const void* x2, float* out,
                 int64_t M, int64_t N, int64_t K,
                 int64_t ldx1, int64_t ldx2, int64_t ldo, int32_t layout,
                 int32_t dtype, int32_t variant, int32_t split_k,
                 void* workspace, size_t workspace_bytes,
                 void* counters, size_t counter_bytes, void* stream);

/*
 * Bytes of scratch (`workspace`) tilec_matmul needs for these arguments
 * with both operands row-major and contiguous (0 if none).  For a named
 * variant the size is the same for every layout; TILEC_VARIANT_AUTO may pick
 * another variant for another layout or stride, which
 * tilec_matmul_scratch_bytes accounts for.  Replaces nothing in the
 * reference (its kernel needs no scratch); the caller allocates it the way
 * `_matrix_mul_tiled` allocates `out` (tilec/ext.py:61).
 */
size_t tilec_matmul_workspace_bytes(int64_t M, int64_t N, int64_t K,
                                    int32_t dtype, int32_t variant,
                                    int32_t split_k);

/* Bytes of zero-initialised completion counters (`counters`) it needs. */
size_t tilec_matmul_counter_bytes(int64_t M, int64_t N, int64_t K,
                                  int32_t dtype, int32_t variant,
                                  int32_t split_k);

/*
 * Both scratch sizes for exactly the arguments tilec_matmul gets (layout
 * bits and strides included; ldx1 / ldx2 <= 0: contiguous), so that
 * TILEC_VARIANT_AUTO is resolved as the call will resolve it.  Returns
 * TILEC_OK, or the status tilec_matmul would return for an argument it
 * rejects (sizes are then 0).  Like the two queries above it replaces
 * nothing in the reference; it cannot see pointers, so for the row-dot and
 * row-tile variants it counts the scratch of their streaming fallback.
 */
int tilec_matmul_scratch_bytes(int64_t M, int64_t N, int64_t K,
                               int64_t ldx1, int64_t ldx2, int32_t layout,
                               int32_t dtype, int32_t variant, int32_t split_k,
                               size_t* workspace_bytes, size_t* counter_bytes);

/*
 * tilec_matmul without the caller's scratch: for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation).  No counterpart in the reference, whose
 * kernel needs no scratch.  Same arguments, semantics and status codes as
 * tilec_matmul, minus the four buffer arguments.
 *
 * A split K uses a static array of the library on the current device: at
 * most 16 MiB of partial sums and 1 MiB of counters (each GPU the library
 * runs on holds 17 MiB until the process ends).  A call that needs more
 * (tilec_matmul_scratch_bytes for the same arguments) fails with
 * TILEC_ERR_WORKSPACE before anything is enqueued; use tilec_matmul then.
 * The first call on a device looks the array up and enqueues a small kernel
 * that clears its counters.  Nothing is allocated.
 *
 * Every call on one GPU shares that GPU's array and leaves its counters at
 * zero: calls that overlap on one GPU (concurrent streams, host threads)
 * race and must be serialized by the caller.
 */
int tilec_matmul_noalloc(const void* x1, const void* x2, float* out,
                         int64_t M, int64_t N, int64_t K,
                         int64_t ldx1, int64_t ldx2, int64_t ldo, int32_t layout,
                         int32_t dtype, int32_t variant, int32_t split_k,
                         void* stream);

/*
 * The variant the library's built-in rule picks for a shape with both
 * operands row-major and contiguous (what TILEC_VARIANT_AUTO runs for layout
 * 0), or a negative status.  The reference's equivalent is the fixed
 * BM=BN=64, BK=16 default of `_matrix_mul_tiled` (tilec/ext.py:54); the
 * trained per-shape choice lives host-side in tilec/tune.py, as
 * `tune.pick` does in the reference (tilec/tune.py:143-151).
 */
int32_t tilec_select_variant(int64_t M, int64_t N, int64_t K, int32_t dtype);

/*
 * The same for any layout and strides (ldx1 / ldx2 <= 0: contiguous): what
 * TILEC_VARIANT_AUTO runs for tilec_matmul with these arguments (x @ W.T,
 * for instance, takes the row-dot or row-tile kernels).  No counterpart in
 * the reference, whose operands are always made contiguous
 * (tilec/ext.py:59-60).
 */
int32_t tilec_select_variant_layout(int64_t M, int64_t N, int64_t K, int32_t dtype, int32_t layout,
                                    int64_t ldx1, int64_t ldx2);

/* The split_k that split_k == 0 resolves to for this variant and shape. */
int32_t tilec_auto_split_k(int64_t M, int64_t N, int64_t K, int32_t dtype,
                           int32_t variant);

/*
 * Variant enumeration, for the tuner (the reference enumerates its config
 * space in Python: `mm_configs`, tilec/ext.py:48-51).
 *   info[0] family (TILEC_FAMILY_*)  info[1] dtype (TILEC_F32/BF16)
 *   info[2] BM     info[3] BN        info[4] BK
 *   info[5] waves per workgroup      info[6] max M (0 = unbounded)
 *   info[7] unroll / pipeline depth
 * `name` (may be NULL) receives a static string.
 */
int32_t tilec_num_variants(void);
int tilec_variant_info(int32_t variant, int32_t info[8], const char** name);

/*
 * Row or column sums of a matrix, fp32 accumulate, fp32 out:
 *   axis 1:  out[r] = sum_c x[r][c]   (R outputs)
 *   axis 0:  out[c] = sum_r x[r][c]   (C outputs)
 * x is R x C, float32 or bfloat16, row-major with row stride ldx (>= C), or
 * column-major when `layout` is TILEC_X1_COL_MAJOR (column stride ldx >= R).
 * A sum over zero elements is 0.
 *
 * The reduction the reference plans as `tl.sum` (README.md:88) and shows as
 * the `row_sum` kernel (kernel1.py:8-15: out[r] = tl.sum(x[r, :]); the
 * op-level spelling `tl.ext.sum(x_ptr, axis=1)` at kernel1.py:15).  Long
 * reductions with few outputs are split across workgroups and combined in
 * a fixed order, so results do not depend on scheduling; they need the
 * `workspace` and zeroed `counters` that tilec_sum_workspace_bytes /
 * tilec_sum_counter_bytes give (0 when not split), under the same rules as
 * tilec_matmul's (counters are left zero; concurrent calls need their own).
 */
int tilec_sum(const void* x, float* out, int64_t R, int64_t C, int64_t ldx,
              int32_t layout, int32_t dtype, int32_t axis,
              void* workspace, size_t workspace_bytes,
              void* counters, size_t counter_bytes, void* stream);
size_t tilec_sum_workspace_bytes(int64_t R, int64_t C, int32_t layout,
                                 int32_t dtype, int32_t axis);
size_t tilec_sum_counter_bytes(int64_t R, int64_t C, int32_t layout,
                               int32_t dtype, int32_t axis);

/*
 * The HBM read floor, a measurement aid with no counterpart in the
 * reference: one pass over `bytes` of x (a multiple of 16 KiB, 16-byte
 * aligned), in the order the GEMV kernels are measured against —
 * `workgroups` workgroups (<= 0: two per CU; at most one per 16 KiB piece)
 * read the 16 KiB pieces g, g + G, g + 2G, ... with non-temporal 16-byte
 * loads (four waves per workgroup), so the chip reads one moving window.
 * Wave w of workgroup g writes the fp32 sum of the floats it read to
 * sink[4 g + w] (the caller provides four floats per workgroup); nothing is
 * combined across workgroups.  Asynchronous on `stream`, allocates nothing.
 */
int tilec_read_floor(const void* x, size_t bytes, float* sink, int32_t workgroups, void* stream);

/* Message describing the last failure on this thread ("" if none). */
const char* tilec_last_error(void);

/* ABI version (major * 10000 + minor * 100 + patch). */
int32_t tilec_version(void);

#ifdef __cplusplus
}
#endif

#endif /* TILEC_H */
