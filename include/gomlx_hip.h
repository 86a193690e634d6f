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
 * dtype: GHIP_DTYPE_FLOAT32 or GHIP_DTYPE_BFLOAT16 unless stated.
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

/* Batched matrix product, the lowering target of Function.DotGeneral
 * (dotgeneral.go:65-164 -> mpsgraph_matmul, bridge.m:684-700):
 *   c[b, m, n] = sum_k a[b, m, k] * b[b, k, n]
 * with every operand addressed by ELEMENT strides (so transposed / permuted
 * views need no copy).  ab_dtype is the dtype of a and b (FLOAT32 or BFLOAT16);
 * c_dtype the output dtype (FLOAT32 or BFLOAT16).  Accumulation is fp32.
 * Requires sc_n == 1. */
int ghip_gemm_batched(int ab_dtype, int c_dtype, int64_t batch, int64_t M, int64_t N,
                      int64_t K, const void* a, int64_t sa_b, int64_t sa_m, int64_t sa_k,
                      const void* b, int64_t sb_b, int64_t sb_k, int64_t sb_n, void* c,
                      int64_t sc_b, int64_t sc_m, int64_t sc_n, void* stream,
                      GHipError* err);

/* Embedding lookup: out[i, :] = table[clamp(ids[i], 0, V-1), :] (row_bytes per
 * row, copied bit-exactly).  Replaces the gather fast path
 * (gather.go:61-203 -> mpsgraph_gather_along_axis, bridge.m:764-782). */
int ghip_gather_rows(const void* table, int64_t V, int64_t row_bytes, const int32_t* ids,
                     int64_t n, void* out, void* stream, GHipError* err);

/* ArgMax (is_min = 0) / ArgMin (is_min = 1) of x viewed as [outer, n, inner]
 * along the middle axis; out has out_dtype (INT32 or INT64).  Ties -> lowest
 * index, NaN wins (first NaN).  Replaces Function.ArgMinMax (function.go:
 * 1204-1242). x dtype FLOAT32 or BFLOAT16. */
int ghip_argminmax(int dtype, const void* x, int64_t outer, int64_t n, int64_t inner,
                   int is_min, int out_dtype, void* out, void* stream, GHipError* err);

/* Iota: out viewed as [outer, n, inner] gets the index along the middle axis,
 * converted to dtype (INT32, INT64, FLOAT32, BFLOAT16).  Replaces Function.Iota
 * (function.go:1127-1135, bridge.m:237-259). */
int ghip_iota(int dtype, void* out, int64_t outer, int64_t n, int64_t inner, void* stream,
              GHipError* err);

#ifdef __cplusplus
}
#endif
#endif /* GOMLX_HIP_H */
