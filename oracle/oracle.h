/*
 * CPU oracle for the gomlx-hip backend — TEST INFRASTRUCTURE ONLY.
 *
 * This library restates, on the CPU, what the reference GoMLX backend computes
 * on its hot path (softmax, layer/RMS norm, DotGeneral, scaled dot-product
 * attention, embedding gather, argmin/argmax, iota).  It is the checker the
 * parity tests compare the HIP kernels against.  Only tests/, the smoke() entry
 * of __graft_entry__.py and the cpu_baseline leg of bench.py may load it; the
 * product path never does.
 *
 * Numerics: every function accumulates in fp64 ("truth") unless `mode` is
 * ORC_MODE_F32SEQ, in which case sums run sequentially in fp32 the way a plain
 * Go loop over float32 would (the error profile of the pure-Go CPU backend).
 * Inputs are fp32 (bf16 inputs are widened exactly by the caller); outputs are
 * fp64 so the caller can measure the error of a GPU result against the truth.
 *
 * Pinning (what each function is checked against, in tests/test_oracle.py):
 *   orc_softmax      reference known answers (mpsgraph_test.go:1178-1189),
 *                    row sums = 1, shift invariance, brute force in numpy.
 *   orc_layernorm    reference known answers (mpsgraph_test.go:2598-2623),
 *                    mean 0 / var 1 invariants.
 *   orc_rmsnorm      closed form mean(y^2) = 1 (gamma 1), scale invariance,
 *                    hand-computed 2-row case.
 *   orc_dot_general  reference known answers (mpsgraph_test.go:529-594,
 *                    3142-3155), numpy.einsum on random axis layouts.
 *   orc_dot_sampled  orc_dot_general on small shapes (entry by entry).
 *   orc_sdpa         reference known answers (mpsgraph_test.go:1689-1723,
 *                    2996-3015, 3036-3057), numpy composition.
 *   orc_gather_rows  reference known answers (mpsgraph_test.go:648-672).
 *   orc_argminmax    reference known answer (mpsgraph_test.go:973-990),
 *                    numpy.argmax/argmin on tie-free data.
 *   orc_argminmax_int numpy.argmax/argmin (first occurrence of the extreme) on
 *                    int8..int64 / uint8..uint64 data with many ties, including
 *                    uint64 values above INT64_MAX.
 *   orc_iota         reference known answer (mpsgraph_test.go:795-821).
 *   orc_dynamic_slice / orc_dynamic_update_slice
 *                    reference known answers (mpsgraph_test.go:993-1062,
 *                    1064-1131); numpy slicing with the clamped starts.
 *   orc_scatter      reference known answer (mpsgraph_test.go:1192-1262);
 *                    numpy.add.at / maximum.at / minimum.at on the embedding
 *                    pattern; sum invariant and update-order invariance on a
 *                    general multi-axis case.
 *   orc_activation   reference known answers for GELU (mpsgraph_test.go:2645-2656)
 *                    and ReLU through FusedDense (:2841-2852); odd-part identity
 *                    g(x) - g(-x) = x for both GELU forms; exact GELU against
 *                    x * Phi(x) from the normal CDF (scipy); tanh approximation
 *                    within 1e-3 of exact; SiLU against x / (1 + e^-x).
 */
#ifndef GOMLX_HIP_ORACLE_H
#define GOMLX_HIP_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_MODE_F64 = 0, ORC_MODE_F32SEQ = 1 };

/* Softmax (or log-softmax when `log` != 0) of x viewed as [outer, n, inner]
 * along the middle axis. */
void orc_softmax(const float* x, double* y, int64_t outer, int64_t n, int64_t inner,
                 int log, int mode);

/* LayerNorm over the trailing `n` elements of each of `rows` rows.
 * gamma/beta may be NULL (then 1 / 0). */
void orc_layernorm(const float* x, const float* gamma, const float* beta, double* y,
                   int64_t rows, int64_t n, double eps, int mode);

/* RMSNorm: y = x * rsqrt(mean(x^2) + eps) * gamma.  gamma may be NULL. */
void orc_rmsnorm(const float* x, const float* gamma, double* y, int64_t rows, int64_t n,
                 double eps, int mode);

/* RMSNorm, fp32 output, fp32 sequential statistics (the CPU baseline's form;
 * equal to orc_rmsnorm in ORC_MODE_F32SEQ rounded to float32). */
void orc_rmsnorm_f32(const float* x, const float* gamma, float* y, int64_t rows, int64_t n,
                     double eps);

/* General DotGeneral with XLA semantics.  Output axis order is
 * [batch..., lhs free..., rhs free...].  Returns 0 on success, -1 on bad axes. */
int orc_dot_general(const float* lhs, int lrank, const int64_t* ldims,
                    const int* lcontract, int nlc, const int* lbatch, int nlb,
                    const float* rhs, int rrank, const int64_t* rdims,
                    const int* rcontract, int nrc, const int* rbatch, int nrb,
                    double* out, int mode);

/* Sampled entries of a canonical batched product C[b,m,n] = sum_k A[b,m,k] B[b,k,n],
 * with A and B addressed by element strides (sa_* / sb_*).  Computes the
 * `count` entries listed in (bs[i], ms[i], ns[i]) into out[i]. */
void orc_dot_sampled(const float* a, int64_t sa_b, int64_t sa_m, int64_t sa_k,
                     const float* b, int64_t sb_b, int64_t sb_k, int64_t sb_n, int64_t K,
                     const int64_t* bs, const int64_t* ms, const int64_t* ns, int64_t count,
                     double* out);

/* Scaled dot-product attention in BHSD layout: q [B,H,Sq,D], k/v [B,Hkv,Sk,D].
 * mask (optional, may be NULL) is a boolean [Sq,Sk] (1 = keep).  causal keeps
 * j <= i.  out [B,H,Sq,D]. */
enum { ORC_MASK_NONE = 0, ORC_MASK_BOOL = 1, ORC_MASK_ADD = 2 };
void orc_sdpa(const float* q, const float* k, const float* v, const void* mask, int mask_kind,
              const int64_t* mask_strides, int64_t B, int64_t H, int64_t Hkv, int64_t Sq, int64_t Sk,
              int64_t D, double scale, int causal, double* out);

/* Embedding lookup: out[i, :] = table[clamp(ids[i], 0, V-1), :] byte for byte. */
void orc_gather_rows(const void* table, int64_t V, int64_t row_bytes, const int32_t* ids,
                     int64_t n, void* out);

/* ArgMax (is_min = 0) / ArgMin (is_min = 1) of x viewed as [outer, n, inner]
 * along the middle axis.  Ties resolve to the lowest index; a NaN wins over
 * every number and the first NaN is returned. */
void orc_argminmax(const float* x, int64_t outer, int64_t n, int64_t inner, int is_min,
                   int64_t* out);
void orc_argminmax_int(const int64_t* x, int64_t outer, int64_t n, int64_t inner, int is_min,
                       int is_unsigned, int64_t* out);

/* Iota: out viewed as [outer, n, inner], out[o, i, j] = i. */
void orc_iota(double* out, int64_t outer, int64_t n, int64_t inner);

/* Activation functions of FusedDense / FusedGelu in fp64, elementwise over n
 * values: ORC_ACT_NONE, ORC_ACT_GELU (tanh approximation), ORC_ACT_RELU,
 * ORC_ACT_SILU, ORC_ACT_TANH, ORC_ACT_GELU_EXACT. */
enum { ORC_ACT_NONE = 0, ORC_ACT_GELU = 1, ORC_ACT_RELU = 2, ORC_ACT_SILU = 3, ORC_ACT_TANH = 4,
       ORC_ACT_GELU_EXACT = 5 };
void orc_activation(const double* x, double* y, int64_t n, int act);

/* DynamicSlice: out (dims `sizes`, contiguous) = the window of x (dims, contiguous,
 * elem_bytes per element) at `starts`, each clamped to [0, dims[k] - sizes[k]]. */
void orc_dynamic_slice(const void* x, int elem_bytes, int rank, const int64_t* dims, const int64_t* starts,
                       const int64_t* sizes, void* out);
/* DynamicUpdateSlice: out = x with `upd` (dims udims) written at `starts`, each
 * clamped to [0, dims[k] - udims[k]]. */
void orc_dynamic_update_slice(const void* x, int elem_bytes, int rank, const int64_t* dims, const void* upd,
                              const int64_t* udims, const int64_t* starts, void* out);
/* XLA scatter in fp64: out = operand (dims odims, rank r) combined (mode 0 sum,
 * 1 max, 2 min; NaN propagates through max / min) with every element of updates
 * (dims udims, rank ur) whose window start fits in the operand.  indices are
 * int64 (dims idims, rank ir), the index vector along axis iva (iva == ir: an
 * implicit trailing axis of size 1).  Updates are visited in row-major order. */
void orc_scatter(int mode, const double* operand, int r, const int64_t* odims, const int64_t* indices, int ir,
                 const int64_t* idims, int iva, const double* updates, int ur, const int64_t* udims,
                 const int* uwa, int n_uwa, const int* iwa, int n_iwa, const int* sato, int n_sato, double* out);

/* fp32 -> bf16 (round to nearest even; NaN stays NaN), as 16-bit patterns. */
void orc_f32_to_bf16(const float* x, uint16_t* y, int64_t n);

#ifdef __cplusplus
}
#endif
#endif
