/*
 * gomlx-hip: C ABI of the MI355X (gfx950) GoMLX backend.
 *
 * This header is the drop-in boundary beneath the GoMLX `backends` plugin API.
 * It replaces the reference's MPSGraph bridge
 * (mpsgraph/gomlx/internal/bridge/bridge.h) with a HIP implementation: the same
 * opaque-handle + error-struct conventions, with device-resident buffers instead
 * of per-call host copies.  Every pointer argument named `x`, `y`, `a`, `b`, `c`,
 * `table`, `ids`, `out`, `gamma`, `beta` in the "direct op" section is a DEVICE
 * pointer; `stream` is a hipStream_t (NULL = the null stream).  No torch types
 * cross this boundary.
 *
 * Errors: every entry point returns 0 on success or a non-zero GHIP_ERR_* code,
 * and, when `err` is non-NULL, fills it; err->message is heap-allocated and the
 * caller releases it with free() or ghip_error_clear() (the reference's rule,
 * bridge.h:16-20, freed by the Go side at bridge.go:77-87).
 */
#ifndef GOMLX_HIP_H
#define GOMLX_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Error reporting; mirrors MPSGraphError (bridge.h:17-20). */
typedef struct {
  int code;
  const char* message;
} GHipError;

enum {
  GHIP_OK = 0,
  GHIP_ERR_INVALID_ARG = 1,   /* bad shape / dtype / axis / null pointer */
  GHIP_ERR_UNSUPPORTED = 2,   /* valid request this backend does not lower */
  GHIP_ERR_HIP = 3,           /* a HIP runtime call failed */
  GHIP_ERR_OOM = 4,           /* device allocation failed */
  GHIP_ERR_STATE = 5,         /* use after finalize, compile twice, ... */
};

/* Data types; numbering is the reference's MPSGraphDType (bridge.h:23-37). */
typedef enum {
  GHIP_DTYPE_BOOL = 0,
  GHIP_DTYPE_INT8 = 1,
  GHIP_DTYPE_INT16 = 2,
  GHIP_DTYPE_INT32 = 3,
  GHIP_DTYPE_INT64 = 4,
  GHIP_DTYPE_FLOAT16 = 5,
  GHIP_DTYPE_BFLOAT16 = 6,
  GHIP_DTYPE_FLOAT32 = 7,
  GHIP_DTYPE_FLOAT64 = 8,
  GHIP_DTYPE_UINT8 = 9,
  GHIP_DTYPE_UINT16 = 10,
  GHIP_DTYPE_UINT32 = 11,
  GHIP_DTYPE_UINT64 = 12,
} GHipDType;

/* Releases err->message (if any) and resets err. */
void ghip_error_clear(GHipError* err);

/* Library / device information. */
const char* ghip_version(void);
/* Writes the device name of `device` into buf (NUL-terminated).  Replaces
 * mpsgraph_device_name (bridge.h:53). */
int ghip_device_name(int device, char* buf, size_t buflen, GHipError* err);

/* ===========================================================================
 * Direct op entry points (device pointers, async on `stream`).
 * These are the kernels the graph lowering launches; they are exported so a
 * host without Go (tests, benchmarks) can drive them through the same ABI.
 * dtype: GHIP_DTYPE_FLOAT32, GHIP_DTYPE_BFLOAT16 or GHIP_DTYPE_FLOAT16 unless
 * stated (16-bit values are raw bit patterns; statistics and accumulation fp32).
 * ======================================================================== */

/* Softmax (log_softmax != 0: log-softmax) of each length-n row of x [rows, n].
 * Replaces Function.FusedSoftmax -> mpsgraph_softmax (function.go:2276-2286,
 * bridge.m:1448-1461) for a last-axis softmax. */
int ghip_softmax_rows(int dtype, const void* x, void* y, int64_t rows, int64_t n,
                      int log_softmax, void* stream, GHipError* err);

/* Fused attention-score softmax: y = softmax(x * scale + mask) along rows of
 * x [batch*sq, sk], where mask is causal (keep col <= row % sq) when causal != 0,
 * and/or a boolean keep-mask bmask [sq, sk] (uint8, may be NULL).
 * Replaces the Mul(scale) -> Where(mask, s, -inf) -> FusedSoftmax chain of
 * FusedScaledDotProductAttention (function.go:2755-2886). */
int ghip_scale_mask_softmax_rows(int dtype, const void* x, void* y, int64_t rows,
                                 int64_t sq, int64_t sk, float scale, int causal,
                                 const uint8_t* bmask, void* stream, GHipError* err);
/* The same over scores [B, H, sq, sk] with the reference's full mask surface
 * (function.go:2840-2878, broadcastMaskToScores :2959-2974): `mask` is a bool
 * keep-mask (mask_dtype GHIP_DTYPE_BOOL: Where(mask, s, -inf)) or an additive mask
 * in the scores' dtype (s + mask), read at mask + b*ms[0] + h*ms[1] + q*ms[2] +
 * key*ms[3] (element strides, 0 on broadcast axes); NULL for none.  Causal keys
 * are -inf whatever the mask holds. */
int ghip_scale_mask_softmax_rows_ex(int dtype, const void* x, void* y, int64_t B, int64_t H,
                                    int64_t sq, int64_t sk, float scale, int causal,
                                    const void* mask, int mask_dtype, const int64_t* mask_strides,
                                    void* stream, GHipError* err);

/* Softmax (log_softmax != 0: log-softmax) over the middle axis of a dense
 * x [outer, n, inner] (the axis of length n; y in the same layout).  Replaces
 * Function.FusedSoftmax with an axis other than the last (function.go:2276-2286,
 * bridge.m:1448-1461: MPSGraph takes any axis) without moving the axis last. */
int ghip_softmax_cols(int dtype, const void* x, void* y, int64_t outer, int64_t n, int64_t inner,
                      int log_softmax, void* stream, GHipError* err);
/* LayerNorm over the middle axis of a dense x [outer, n, inner], fp32 statistics;
 * gamma / beta [n] in x's dtype, each may be NULL.  Replaces Function.FusedLayerNorm
 * with one normalized axis that is not the last (function.go:2416-2427). */
int ghip_layernorm_cols(int dtype, const void* x, const void* gamma, const void* beta, void* y,
                        int64_t outer, int64_t n, int64_t inner, float eps, void* stream,
                        GHipError* err);

/* RMSNorm over the last axis: y = x * rsqrt(mean(x^2) + eps) * gamma.
 * gamma [n] has x's dtype and may be NULL.  Statistics in fp32.  No reference op:
 * replaces the primitive Mul/ReduceSum/Div/Add/Rsqrt/Mul chain (function.go:
 * 686-688, 808-818, 1184-1186). */
int ghip_rmsnorm_rows(int dtype, const void* x, const void* gamma, void* y, int64_t rows,
                      int64_t n, float eps, void* stream, GHipError* err);

/* LayerNorm over the last axis with fp32 statistics; gamma/beta [n] in x's dtype,
 * each may be NULL.  Replaces Function.FusedLayerNorm (function.go:2410-2565). */
int ghip_layernorm_rows(int dtype, const void* x, const void* gamma, const void* beta,
                        void* y, int64_t rows, int64_t n, float eps, void* stream,
                        GHipError* err);

/* dst[i] = src[i] over `dims` (rank <= 8), both sides addressed by ELEMENT strides
 * of elem_bytes-byte elements (1, 2, 4, 8 or 16): the copy that materialises
 * transposed, broadcast, sliced or reversed views and writes outputs.  Axes that
 * both sides step through as one run are merged first; a dense copy moves
 * 16-byte vectors with nontemporal loads and stores.  No reference op:
 * MPSGraph does these copies inside the graph (e.g. the rhs transposes of
 * dotgeneral.go:116-145). */
int ghip_copy_strided(int elem_bytes, const void* src, void* dst, int rank, const int64_t* dims,
                      const int64_t* src_strides, const int64_t* dst_strides, void* stream,
                      GHipError* err);

/* Batched matrix product, the lowering target of Function.DotGeneral
 * (dotgeneral.go:65-164 -> mpsgraph_matmul, bridge.m:684-700):
 *   c[b, m, n] = sum_k a[b, m, k] * b[b, k, n]
 * with every operand addressed by ELEMENT strides (so transposed / permuted
 * views need no copy).  ab_dtype is the dtype of a and b (FLOAT32, BFLOAT16 or
 * FLOAT16); c_dtype the output dtype (FLOAT32, or ab_dtype when that is 16-bit).
 * Accumulation is fp32.  Operands of any size: a batch slice may span more than
 * 4 GiB (the MFMA cores then run their 64-bit-addressing form, bit-identical);
 * row strides of 2^22 elements (16-bit) / 2^21 (fp32) or more, unaligned or
 * negative strides run a generic (non-MFMA) kernel.
 * Requires sc_n == 1. */
int ghip_gemm_batched(int ab_dtype, int c_dtype, int64_t batch, int64_t M, int64_t N,
                      int64_t K, const void* a, int64_t sa_b, int64_t sa_m, int64_t sa_k,
                      const void* b, int64_t sb_b, int64_t sb_k, int64_t sb_n, void* c,
                      int64_t sc_b, int64_t sc_m, int64_t sc_n, void* stream,
                      GHipError* err);

/* Several DotGenerals that share the left operand (dotgeneral.go:65-164 once per
 * product; the projections Q, K, V of an attention block, function.go:2976-3075,
 * are such a set), in one launch:
 *   c[g][m, n] = sum_k a[m, k] * b[g][k, n],   g < groups (1 .. 4)
 * with one set of element strides for a, for every b[g] and every c[g] (unit n
 * stride).  Each c[g] equals what ghip_gemm_batched gives for that product alone
 * (the same kernel core and summation order).  16-bit a / b with a K-contiguous
 * and every b[g] N-contiguous run as one grid of groups x tiles workgroups; other
 * layouts and dtypes run product by product. */
int ghip_gemm_grouped(int ab_dtype, int c_dtype, int groups, int64_t M, int64_t N, int64_t K,
                      const void* a, int64_t sa_m, int64_t sa_k, const void* const* b, int64_t sb_k,
                      int64_t sb_n, void* const* c, int64_t sc_m, void* stream, GHipError* err);

/* Device workspace bytes ghip_gemm_batched_ws / ghip_gemm_grouped_ws can use for a
 * product of these sizes (per product), or 0 when such a product never splits.
 * A split applies to batch 1, at most 256 (16-bit operands) or 128 (fp32) output
 * tiles of 128 x 128 and a long contraction (K >= 1024, K / s a multiple of 64): the
 * contraction runs as s ranges in one grid, each writing its fp32 partial
 * product [M, N] into the workspace (s x M x N x 4 bytes), and a second kernel
 * adds the s partials in range order and rounds once.  The result is
 * deterministic, but its rounding differs from the unsplit product's (another
 * fp32 summation order).  Same DotGeneral as ghip_gemm_batched
 * (dotgeneral.go:65-164); the reference has no workspace. */
int64_t ghip_gemm_workspace_bytes(int ab_dtype, int c_dtype, int64_t batch, int64_t M, int64_t N,
                                  int64_t K);

/* ghip_gemm_batched with a caller-owned device workspace (16-byte aligned) that
 * allows the contraction split described above.  workspace NULL: exactly
 * ghip_gemm_batched (no split).  A workspace smaller than
 * ghip_gemm_workspace_bytes reports for a product that splits is an error
 * (GHIP_ERR_INVALID_ARG).  The workspace is written on `stream`: calls sharing
 * one workspace must be ordered (one stream). */
int ghip_gemm_batched_ws(int ab_dtype, int c_dtype, int64_t batch, int64_t M, int64_t N,
                         int64_t K, const void* a, int64_t sa_b, int64_t sa_m, int64_t sa_k,
                         const void* b, int64_t sb_b, int64_t sb_k, int64_t sb_n, void* c,
                         int64_t sc_b, int64_t sc_m, int64_t sc_n, void* workspace,
                         int64_t workspace_bytes, void* stream, GHipError* err);

/* ghip_gemm_grouped with a workspace: products that split (per
 * ghip_gemm_workspace_bytes with batch 1) run one after another, each as
 * ghip_gemm_batched_ws gives it with the same workspace, so c[g] keeps the
 * stand-alone bits; others as ghip_gemm_grouped. */
int ghip_gemm_grouped_ws(int ab_dtype, int c_dtype, int groups, int64_t M, int64_t N, int64_t K,
                         const void* a, int64_t sa_m, int64_t sa_k, const void* const* b,
                         int64_t sb_k, int64_t sb_n, void* const* c, int64_t sc_m, void* workspace,
                         int64_t workspace_bytes, void* stream, GHipError* err);

/* Fused attention forward, the one-kernel lowering of
 * Function.FusedScaledDotProductAttention (function.go:2669-2907; the composite
 * it replaces is DotGeneral -> scale -> causal Where -> FusedSoftmax -> DotGeneral,
 * :2746-2897):
 *   o[b, h, i, :] = sum_j softmax_j(scale * q[b,h,i,:].k[b,hk,j,:] [j > i masked
 *                   when causal]) v[b, hk, j, :],   hk = h / (H / Hkv)  (GQA, :2911-2956)
 * Operands are addressed by ELEMENT strides (batch, head, sequence) with the head
 * dim contiguous, so BHSD and BSHD layouts both work without copies.  Supported:
 * dtype BFLOAT16 or FLOAT16 with D a multiple of 8 up to 256, strides multiples of
 * 8 (4 for o), o 8-byte aligned; or FLOAT32 with D a multiple of 4 up to 128,
 * strides multiples of 4, o 16-byte aligned; scale > 0 and q/k/v 16-byte aligned;
 * K / V sequence strides below 32 MiB.  One (batch, kv head) slice of K / V may
 * span more than 4 GiB with 16-bit operands (long contexts), below 2 GiB with
 * FLOAT32 ones.  Anything else returns GHIP_ERR_UNSUPPORTED (the graph lowering then uses the
 * composite).  Softmax statistics and accumulation are fp32 (fp32 products too for
 * FLOAT32); weights below 2^-126 of a row's largest are flushed to zero. */
int ghip_sdpa_fwd(int dtype, const void* q, const void* k, const void* v, void* o,
                  int64_t B, int64_t H, int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D,
                  const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
                  const int64_t* o_strides, float scale, int causal, void* stream,
                  GHipError* err);

/* ghip_sdpa_fwd with the reference's mask operand (function.go:2840-2878): a bool
 * keep-mask (mask_dtype GHIP_DTYPE_BOOL: scores where false are -inf, :2847-2871)
 * or an additive mask in the operands' dtype (scale * q.k + mask, :2872-2878), of
 * any rank broadcast to the scores [B, H, Sq, Sk] (:2959-2974): mask_strides are
 * its element strides over (b, h, query, key), 0 on broadcast axes.  mask NULL:
 * no mask.  A query whose keys are all masked gets NaN, as the reference's softmax
 * of a row of -inf does. */
int ghip_sdpa_fwd_masked(int dtype, const void* q, const void* k, const void* v, void* o,
                         int64_t B, int64_t H, int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D,
                         const int64_t* q_strides, const int64_t* k_strides,
                         const int64_t* v_strides, const int64_t* o_strides, const void* mask,
                         int mask_dtype, const int64_t* mask_strides, float scale, int causal,
                         void* stream, GHipError* err);

/* ghip_sdpa_fwd_masked with a caller-provided workspace (the same
 * FusedScaledDotProductAttention, function.go:2669-2907).  With a workspace of
 * ghip_sdpa_workspace_bytes() bytes (16-byte aligned) a grid of few (batch, head,
 * 128-query block) workgroups (decoding, short prefills; 16-bit operands) splits
 * each workgroup's key range over several workgroups and merges their outputs by
 * log-sum-exp in a second kernel (without a causal mask, grouped-query heads of
 * one kv head also share workgroups when Sq < 128, with or without a workspace): the result agrees with the unsplit one to
 * rounding (same tolerance against the reference), and is the same bits every
 * run.  workspace NULL or ghip_sdpa_workspace_bytes() == 0: no split.  Calls that
 * share one workspace on different streams race. */
int64_t ghip_sdpa_workspace_bytes(int dtype, int64_t B, int64_t H, int64_t Hkv, int64_t Sq, int64_t Sk,
                                  int64_t D, int causal);
int ghip_sdpa_fwd_masked_ws(int dtype, const void* q, const void* k, const void* v, void* o,
                            int64_t B, int64_t H, int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D,
                            const int64_t* q_strides, const int64_t* k_strides,
                            const int64_t* v_strides, const int64_t* o_strides, const void* mask,
                            int mask_dtype, const int64_t* mask_strides, float scale, int causal,
                            void* workspace, int64_t workspace_bytes, void* stream, GHipError* err);

/* Embedding lookup: out[i, :] = table[clamp(ids[i], 0, V-1), :] (row_bytes per
 * row, copied bit-exactly).  Replaces the gather fast path
 * (gather.go:61-203 -> mpsgraph_gather_along_axis, bridge.m:764-782). */
int ghip_gather_rows(const void* table, int64_t V, int64_t row_bytes, const int32_t* ids,
                     int64_t n, void* out, void* stream, GHipError* err);

/* ArgMax (is_min = 0) / ArgMin (is_min = 1) of x viewed as [outer, n, inner]
 * along the middle axis; out has out_dtype (INT32 or INT64).  Ties -> lowest
 * index, NaN wins (first NaN).  Replaces Function.ArgMinMax (function.go:
 * 1204-1242). x dtype FLOAT32, BFLOAT16, FLOAT16 or any integer type (compared
 * as int64 / uint64). */
int ghip_argminmax(int dtype, const void* x, int64_t outer, int64_t n, int64_t inner,
                   int is_min, int out_dtype, void* out, void* stream, GHipError* err);

/* Iota: out viewed as [outer, n, inner] gets the index along the middle axis,
 * converted to dtype (INT32, INT64, FLOAT32, BFLOAT16).  Replaces Function.Iota
 * (function.go:1127-1135, bridge.m:237-259). */
int ghip_iota(int dtype, void* out, int64_t outer, int64_t n, int64_t inner, void* stream,
              GHipError* err);

/* ===========================================================================
 * Graph API: the GoMLX backends plugin surface (Backend / Builder / Function /
 * Executable / Buffer) as a C ABI a cgo layer binds one-to-one.  It replaces the
 * MPSGraph context / tensor / exec calls of bridge.h (context :48-53, op
 * constructors :55-156, compile :159-163, execute :167-172).
 *
 * Values are small integer ids inside their Function (GHipValue, -1 = none);
 * every constructor returns the new id or -1 with err filled.  Shapes follow
 * XLA / GoMLX semantics (the upstream shapeinference rules).  Compile lowers the
 * whole graph once: it fuses softmax / RMSNorm / LayerNorm / attention patterns
 * into the row kernels above, DotGeneral into the batched GEMM with operand
 * transposes folded into strides, and chains of elementwise ops into generated
 * kernels (hipRTC, gfx950).  Execute enqueues the plan on the backend's stream
 * with device-resident buffers and returns without synchronizing (results are
 * ordered on that stream; BufferToFlatData waits for them).  Graphs with While /
 * If synchronize inside Execute to read their predicates.
 * ======================================================================== */
typedef struct GHipBackend GHipBackend;
typedef struct GHipBuilder GHipBuilder;
typedef struct GHipFunction GHipFunction;
typedef struct GHipExecutable GHipExecutable;
typedef struct GHipBuffer GHipBuffer;
typedef int32_t GHipValue;

/* Unary ops (backends.Function Abs ... Identity, function.go:658-782). */
enum {
  GHIP_UNARY_ABS = 0, GHIP_UNARY_NEG, GHIP_UNARY_SQRT, GHIP_UNARY_RSQRT, GHIP_UNARY_EXP,
  GHIP_UNARY_EXPM1, GHIP_UNARY_LOG, GHIP_UNARY_LOG1P, GHIP_UNARY_SIN, GHIP_UNARY_COS,
  GHIP_UNARY_TANH, GHIP_UNARY_LOGISTIC, GHIP_UNARY_ERF, GHIP_UNARY_FLOOR, GHIP_UNARY_CEIL,
  GHIP_UNARY_ROUND, GHIP_UNARY_SIGN, GHIP_UNARY_LOGICAL_NOT, GHIP_UNARY_BITWISE_NOT,
  GHIP_UNARY_IS_FINITE, GHIP_UNARY_IS_NAN, GHIP_UNARY_IDENTITY, GHIP_UNARY_COUNT
};
/* Binary ops (function.go:788-903). */
enum {
  GHIP_BINARY_ADD = 0, GHIP_BINARY_SUB, GHIP_BINARY_MUL, GHIP_BINARY_DIV, GHIP_BINARY_REM,
  GHIP_BINARY_POW, GHIP_BINARY_MAX, GHIP_BINARY_MIN, GHIP_BINARY_ATAN2,
  GHIP_BINARY_LOGICAL_AND, GHIP_BINARY_LOGICAL_OR, GHIP_BINARY_LOGICAL_XOR,
  GHIP_BINARY_BITWISE_AND, GHIP_BINARY_BITWISE_OR, GHIP_BINARY_BITWISE_XOR,
  GHIP_BINARY_SHIFT_LEFT, GHIP_BINARY_SHIFT_RIGHT_ARITHMETIC, GHIP_BINARY_SHIFT_RIGHT_LOGICAL,
  GHIP_BINARY_COUNT
};
/* Comparisons (function.go:923-963); results are Bool. */
enum {
  GHIP_CMP_EQ = 0, GHIP_CMP_NE, GHIP_CMP_GT, GHIP_CMP_GE, GHIP_CMP_LT, GHIP_CMP_LE, GHIP_CMP_COUNT
};
/* Reductions; numbering is the reference's MPSGraphReduceType (bridge.h:40-45). */
enum { GHIP_REDUCE_SUM = 0, GHIP_REDUCE_PRODUCT = 1, GHIP_REDUCE_MAX = 2, GHIP_REDUCE_MIN = 3 };
/* Attention axes layout (backends.AxesLayout). */
enum { GHIP_LAYOUT_BHSD = 0, GHIP_LAYOUT_BSHD = 1 };

/* --- Backend (mpsgraph/gomlx/backend.go:22-167) ------------------------- */
/* New (backend.go:33-43).  config: "" or "hip:device=N"; "plan" builds a
 * backend that compiles (lowers, generates kernels) but cannot execute — it
 * needs no GPU and exists so the lowering can be inspected anywhere. */
GHipBackend* ghip_backend_new(const char* config, GHipError* err);
void ghip_backend_finalize(GHipBackend* b);               /* Finalize (:80-92) */
int ghip_backend_is_finalized(GHipBackend* b);            /* IsFinalized (:95-99) */
int ghip_backend_description(GHipBackend* b, char* buf, size_t buflen); /* Description */
int ghip_backend_num_devices(GHipBackend* b);             /* NumDevices (:57) */
void* ghip_backend_stream(GHipBackend* b);                /* stream Execute uses */
/* Capabilities (backend.go:64-67, capabilities.go:14-166): writes
 * "functions=1;ops=<OpType names>;dtypes=<DType names>" (comma-separated, the
 * GoMLX names without the OpType prefix) into buf, truncated to buflen; returns
 * the full length. */
int ghip_backend_capabilities(char* buf, size_t buflen);

/* --- Buffers (buffer.go:20-119, DataInterface backend.go:103-167) ------- */
/* BufferFromFlatData: device buffer of `shape` holding a copy of host `data`. */
GHipBuffer* ghip_buffer_from_host(GHipBackend* b, int dtype, const int64_t* dims, int rank,
                                  const void* data, size_t nbytes, GHipError* err);
/* NewSharedBuffer (device memory, contents undefined). */
GHipBuffer* ghip_buffer_new(GHipBackend* b, int dtype, const int64_t* dims, int rank,
                            GHipError* err);
/* BufferToFlatData: copies the buffer into host `data` (nbytes must match). */
int ghip_buffer_to_host(GHipBuffer* buf, void* data, size_t nbytes, GHipError* err);
/* BufferShape: writes dtype and up to max_rank dims; returns the rank (-1: bad buffer). */
int ghip_buffer_shape(GHipBuffer* buf, int* dtype, int64_t* dims, int max_rank);
/* BufferData: the device pointer (zero-copy; valid until finalize). */
void* ghip_buffer_device_ptr(GHipBuffer* buf);
void ghip_buffer_finalize(GHipBuffer* buf);               /* BufferFinalize */

/* --- Builder (builder.go:16-109) ---------------------------------------- */
GHipBuilder* ghip_builder_new(GHipBackend* b, const char* name, GHipError* err);
void ghip_builder_finalize(GHipBuilder* bl);
GHipFunction* ghip_builder_main(GHipBuilder* bl);         /* Main (:50-55) */
/* Compile (:72-91): errors on a second call, without Main, or without Return. */
GHipExecutable* ghip_builder_compile(GHipBuilder* bl, GHipError* err);

/* --- Function (function.go, dotgeneral.go, gather.go) ------------------ */
GHipValue ghip_fn_parameter(GHipFunction* f, const char* name, int dtype, const int64_t* dims,
                            int rank, GHipError* err);                  /* :285-295 */
GHipValue ghip_fn_constant(GHipFunction* f, int dtype, const int64_t* dims, int rank,
                           const void* data, size_t nbytes, GHipError* err); /* :298-334 */
GHipValue ghip_fn_iota(GHipFunction* f, int dtype, const int64_t* dims, int rank, int axis,
                       GHipError* err);                                 /* :1127-1135 */
GHipValue ghip_fn_unary(GHipFunction* f, int op, GHipValue x, GHipError* err);
GHipValue ghip_fn_binary(GHipFunction* f, int op, GHipValue lhs, GHipValue rhs, GHipError* err);
GHipValue ghip_fn_compare(GHipFunction* f, int op, GHipValue lhs, GHipValue rhs, GHipError* err);
GHipValue ghip_fn_where(GHipFunction* f, GHipValue cond, GHipValue on_true, GHipValue on_false,
                        GHipError* err);                                /* :1044-1058 */
GHipValue ghip_fn_clamp(GHipFunction* f, GHipValue lo, GHipValue x, GHipValue hi,
                        GHipError* err);                                /* :1060-1072 */
GHipValue ghip_fn_convert_dtype(GHipFunction* f, GHipValue x, int dtype, GHipError* err);
GHipValue ghip_fn_reshape(GHipFunction* f, GHipValue x, const int64_t* dims, int rank,
                          GHipError* err);                              /* :969-981 */
GHipValue ghip_fn_transpose(GHipFunction* f, GHipValue x, const int* perm, int rank,
                            GHipError* err);                            /* :983-996 */
GHipValue ghip_fn_broadcast_in_dim(GHipFunction* f, GHipValue x, const int64_t* dims, int rank,
                                   const int* axes, int naxes, GHipError* err); /* :1013-1042 */
GHipValue ghip_fn_reduce(GHipFunction* f, int op, GHipValue x, const int* axes, int naxes,
                         GHipError* err);                               /* :1147-1198 */
GHipValue ghip_fn_arg_min_max(GHipFunction* f, GHipValue x, int axis, int out_dtype, int is_min,
                              GHipError* err);                          /* :1204-1242 */
GHipValue ghip_fn_dot_general(GHipFunction* f, GHipValue lhs, const int* lhs_contracting,
                              int nlc, const int* lhs_batch, int nlb, GHipValue rhs,
                              const int* rhs_contracting, int nrc, const int* rhs_batch,
                              int nrb, GHipError* err);                 /* dotgeneral.go:65-164 */
GHipValue ghip_fn_gather(GHipFunction* f, GHipValue operand, GHipValue start_indices,
                         int index_vector_axis, const int* offset_output_axes, int n_offset,
                         const int* collapsed_slice_axes, int n_collapsed,
                         const int* start_index_map, int n_map, const int64_t* slice_sizes,
                         int n_sizes, int indices_are_sorted, GHipError* err); /* gather.go:24-56 */
GHipValue ghip_fn_slice(GHipFunction* f, GHipValue x, const int64_t* starts, const int64_t* limits,
                        const int64_t* strides, int rank, GHipError* err);  /* :1074-1091 */
GHipValue ghip_fn_concatenate(GHipFunction* f, int axis, const GHipValue* operands, int n,
                              GHipError* err);                          /* :1093-1113 */
GHipValue ghip_fn_reverse(GHipFunction* f, GHipValue x, const int* axes, int naxes,
                          GHipError* err);                              /* :1115-1125 */
/* Pad (:1533-1569): per axis `start` / `end` elements of the scalar `fill`
 * (negative values crop); a non-zero `interior` (may be NULL) is refused with
 * GHIP_ERR_UNSUPPORTED, as the reference refuses it. */
GHipValue ghip_fn_pad(GHipFunction* f, GHipValue x, GHipValue fill, const int64_t* start,
                      const int64_t* end, const int64_t* interior, int rank, GHipError* err);
/* ReduceLogicalAnd (is_or = 0) / ReduceLogicalOr (is_or = 1) over a Bool
 * operand (:2262-2270); empty axes reduce everything. */
GHipValue ghip_fn_reduce_logical(GHipFunction* f, int is_or, GHipValue x, const int* axes,
                                 int naxes, GHipError* err);
GHipValue ghip_fn_fused_softmax(GHipFunction* f, GHipValue x, int axis, GHipError* err); /* :2276 */
/* gamma / beta may be -1 (absent). */
GHipValue ghip_fn_fused_layer_norm(GHipFunction* f, GHipValue x, const int* axes, int naxes,
                                   double epsilon, GHipValue gamma, GHipValue beta,
                                   GHipError* err);                     /* :2410-2565 */
/* mask may be -1; layout GHIP_LAYOUT_*. */
GHipValue ghip_fn_fused_sdpa(GHipFunction* f, GHipValue q, GHipValue k, GHipValue v,
                             GHipValue mask, int num_heads, int num_kv_heads, int layout,
                             double scale, int causal, GHipError* err); /* :2669-2907 */
/* DynamicSlice (function.go:1571-1594): a `sizes` window of operand at the
 * run-time start indices `starts` (one integer scalar value per axis), each
 * clamped to [0, dim - size] (XLA semantics). */
GHipValue ghip_fn_dynamic_slice(GHipFunction* f, GHipValue operand, const GHipValue* starts,
                                int nstarts, const int64_t* sizes, int nsizes, GHipError* err);
/* DynamicUpdateSlice (function.go:1596-1621): operand with `update` written at the
 * run-time start indices, clamped to [0, dim - update dim]. */
GHipValue ghip_fn_dynamic_update_slice(GHipFunction* f, GHipValue operand, GHipValue update,
                                       const GHipValue* starts, int nstarts, GHipError* err);
/* ScatterSum / ScatterMax / ScatterMin (gather.go:441-640): XLA scatter of
 * `updates` into `operand` combining with +, max or min.  A window whose start
 * (from `indices`) does not fit inside the operand is skipped. */
enum { GHIP_SCATTER_SUM = 0, GHIP_SCATTER_MAX = 1, GHIP_SCATTER_MIN = 2 };
GHipValue ghip_fn_scatter(GHipFunction* f, int mode, GHipValue operand, GHipValue indices,
                          GHipValue updates, int index_vector_axis, const int* update_window_axes,
                          int n_update_window_axes, const int* inserted_window_axes,
                          int n_inserted_window_axes, const int* scatter_axes_to_operand_axes,
                          int n_scatter_axes, int indices_are_sorted, int unique_indices,
                          GHipError* err);
/* Composite fused ops, built from the primitives above in the order the
 * reference composes them, so the lowering fuses them like any other chain
 * (bias / activation / slicing run in the GEMM epilogue).
 * FusedGelu (:2288-2408): exact = x/2 (1 + erf(x/sqrt 2)); otherwise the tanh
 * approximation with the reference's constants. */
GHipValue ghip_fn_fused_gelu(GHipFunction* f, GHipValue x, int exact, GHipError* err);
/* backends.ActivationType values FusedDense takes (names as in GoMLX; a cgo
 * binding maps GoMLX's constants onto these by name). */
enum {
  GHIP_ACTIVATION_NONE = 0, GHIP_ACTIVATION_GELU, GHIP_ACTIVATION_RELU, GHIP_ACTIVATION_SILU,
  GHIP_ACTIVATION_TANH
};
/* FusedDense (:2567-2667): x [..., din] . weight [din, ...] + bias (broadcast over
 * the trailing axes; -1 = none), then the activation (GELU = tanh approximation,
 * as the reference calls FusedGelu with exact = false). */
GHipValue ghip_fn_fused_dense(GHipFunction* f, GHipValue x, GHipValue weight, GHipValue bias,
                              int activation, GHipError* err);
/* FusedAttentionQKVProjection (:2976-3075): x . wQKV sliced on the last axis into
 * [0, qdim), [qdim, qdim+kvdim), [qdim+kvdim, qdim+2 kvdim), each plus its bias
 * (-1 = none).  Writes the three values; returns GHIP_OK or the error code. */
int ghip_fn_fused_qkv_projection(GHipFunction* f, GHipValue x, GHipValue w_qkv, GHipValue bias_q,
                                 GHipValue bias_k, GHipValue bias_v, int query_dim,
                                 int key_value_dim, GHipValue* query, GHipValue* key,
                                 GHipValue* value, GHipError* err);
int ghip_fn_return(GHipFunction* f, const GHipValue* outputs, int n, GHipError* err); /* :337-345 */
/* OpShape (builder.go:63-69): dtype + dims of a value; returns rank or -1. */
int ghip_fn_value_shape(GHipFunction* f, GHipValue v, int* dtype, int64_t* dims, int max_rank);

/* --- Functions and control flow (builder.go:57-70, function.go:120-133,
 * 354-660, executable.go:112-577) ------------------------------------------
 * Value ids are unique within a builder, so a closure may use values of the
 * functions that enclose it: they are captured (passed to it as extra inputs
 * after its parameters).  Call / While / If write their outputs' value ids into
 * outs (room for max_outs) and return the number of outputs, or -1 with err set.
 * The loops and branches run on the host, between launches of the compiled
 * closures on the backend's stream; state stays in device memory.  An If reads
 * back one bool.  A While enqueues cond and body in speculative batches (1, 2,
 * 4, then up to 8 iterations) and reads back each batch's predicates in one
 * copy, keeping the state before the first false one; a While whose cond or body
 * itself contains Call / While / If runs without speculation (one predicate read
 * per iteration, the body only when it is true). */
/* NewFunction (builder.go:57-70): a named function, the target of Call. */
GHipFunction* ghip_builder_new_function(GHipBuilder* bl, const char* name, GHipError* err);
/* Closure (function.go:120-133): a function nested in f. */
GHipFunction* ghip_fn_closure(GHipFunction* f, GHipError* err);
/* Call (function.go:354-405): target's outputs for these inputs. */
int ghip_fn_call(GHipFunction* f, GHipFunction* target, const GHipValue* inputs, int n,
                 GHipValue* outs, int max_outs, GHipError* err);
/* While (function.go:407-493): state = init; while cond(state): state = body(state).
 * At most 1,000,000 iterations (Execute then fails, as the reference does). */
int ghip_fn_while(GHipFunction* f, GHipFunction* cond, GHipFunction* body, const GHipValue* init,
                  int n, GHipValue* outs, int max_outs, GHipError* err);
/* If (function.go:495-560): the outputs of true_branch or false_branch (closures
 * without parameters) by the scalar bool pred. */
int ghip_fn_if(GHipFunction* f, GHipValue pred, GHipFunction* true_branch,
               GHipFunction* false_branch, GHipValue* outs, int max_outs, GHipError* err);

/* Sort (function.go:562-655): the n inputs (same dims) reordered along `axis` so
 * that comparator (a closure of 2n scalar parameters lhs_0, rhs_0, lhs_1, rhs_1,
 * ..., returning a scalar bool "lhs before rhs") holds; ties keep their input
 * order (every sort is stable).  The comparator is compiled into the sort kernel:
 * it may use elementwise ops, scalar constants and captured scalars.  Each row
 * along the axis is sorted by one workgroup: in LDS when its keys and indices fit
 * (about 16K elements for one 4-byte key), otherwise over an index array in the
 * executable's arena (chunks sorted in LDS, larger stages in global memory), for
 * rows of up to 2^30 elements. */
int ghip_fn_sort(GHipFunction* f, GHipFunction* comparator, int axis, int is_stable,
                 const GHipValue* inputs, int n, GHipValue* outs, int max_outs, GHipError* err);

/* --- Executable (executable.go:19-112) ---------------------------------- */
int ghip_exec_num_inputs(GHipExecutable* e);
int ghip_exec_num_outputs(GHipExecutable* e);
int ghip_exec_input_shape(GHipExecutable* e, int i, int* dtype, int64_t* dims, int max_rank);
int ghip_exec_output_shape(GHipExecutable* e, int i, int* dtype, int64_t* dims, int max_rank);
/* Execute (:50-112): validates count and shapes of `inputs`, runs the plan, and
 * returns `nout` new output buffers (owned by the caller).  donate may be NULL;
 * a donated input buffer may be reused for an output of identical shape.
 * Calls on one executable are serialized. */
int ghip_exec_execute(GHipExecutable* e, GHipBuffer* const* inputs, int n, const uint8_t* donate,
                      GHipBuffer** outputs, int nout, GHipError* err);
/* Execute without allocating device memory.  No counterpart in the reference:
 * this is for callers that cannot allocate (serving loops that must not call
 * hipMalloc, code run under stream capture).  The caller passes the `nout`
 * output buffers (shapes as ghip_exec_output_shape reports, distinct from the
 * inputs); the intermediates live in a file-scope device array of
 * ghip_exec_noalloc_scratch_bytes() (256 MiB) per GPU, shared by every call on
 * that GPU, so calls that overlap on one GPU race.  A plan needing more than
 * that, or one with Call / While / If (whose sub-functions have arenas of their
 * own), is refused with an error.  Inputs are checked like Execute's. */
int ghip_exec_execute_noalloc(GHipExecutable* e, GHipBuffer* const* inputs, int n,
                              GHipBuffer* const* outputs, int nout, GHipError* err);
size_t ghip_exec_noalloc_scratch_bytes(void);
/* Human-readable lowering plan (one line per launch), for inspection / tests.
 * Returns the full length; writes at most buflen-1 chars. */
size_t ghip_exec_plan(GHipExecutable* e, char* buf, size_t buflen);
void ghip_exec_finalize(GHipExecutable* e);

#ifdef __cplusplus
}
#endif
#endif /* GOMLX_HIP_H */
