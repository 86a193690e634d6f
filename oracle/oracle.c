/*
 * CPU oracle for the gomlx-hip backend — TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Each function cites the reference code whose semantics it restates.  The
 * reference runs these ops inside Apple's MPSGraph (closed), and its intended
 * parity target, GoMLX's pure-Go "simplego" backend, is an un-vendored module
 * (github.com/gomlx/gomlx@v0.26.1-0.20260223064152-358aaf0bc270,
 * mpsgraph/gomlx/go.mod:6), so what is restated here is the op semantics the
 * reference's Go code and tests fix, computed in fp64.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define ORC_MAX_RANK 16

/* ---------------------------------------------------------------------------
 * Softmax / log-softmax.
 * Reference: Function.FusedSoftmax (mpsgraph/gomlx/function.go:2276-2286)
 * delegates to MPSGraph softMaxWithTensor:axis: (internal/bridge/bridge.m:1448-1461):
 * y = exp(x - max) / sum(exp(x - max)) along `axis`, output shape = input shape.
 * log-softmax has no reference op; it is x - max - log(sum(exp(x - max))).
 * ------------------------------------------------------------------------- */
void orc_softmax(const float* x, double* y, int64_t outer, int64_t n, int64_t inner,
                 int log_, int mode) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t o = 0; o < outer; ++o) {
    for (int64_t j = 0; j < inner; ++j) {
      const float* xr = x + o * n * inner + j;
      double* yr = y + o * n * inner + j;
      double mx = -INFINITY;
      for (int64_t i = 0; i < n; ++i) {
        double v = xr[i * inner];
        if (v > mx || isnan(v)) mx = v;
      }
      if (mode == ORC_MODE_F32SEQ) {
        float mxf = (float)mx, s = 0.0f;
        for (int64_t i = 0; i < n; ++i) s += expf(xr[i * inner] - mxf);
        for (int64_t i = 0; i < n; ++i) {
          float d = xr[i * inner] - mxf;
          yr[i * inner] = log_ ? (double)(d - logf(s)) : (double)(expf(d) / s);
        }
      } else {
        double s = 0.0;
        for (int64_t i = 0; i < n; ++i) s += exp((double)xr[i * inner] - mx);
        double ls = log(s);
        for (int64_t i = 0; i < n; ++i) {
          double d = (double)xr[i * inner] - mx;
          yr[i * inner] = log_ ? d - ls : exp(d) / s;
        }
      }
    }
  }
}

/* ---------------------------------------------------------------------------
 * LayerNorm.
 * Reference: Function.FusedLayerNorm (mpsgraph/gomlx/function.go:2410-2565):
 * mean = sum(x)/count (:2429-2452), diff = x - mean (:2455), var = sum(diff^2)/count
 * (:2461-2473), normalized = diff * rsqrt(var + eps) (:2476-2496), then * gamma
 * (:2533-2546) and + beta (:2549-2562).  Statistics here are fp64 (the reference
 * keeps them in x's dtype, which the build deliberately does not copy).
 * ------------------------------------------------------------------------- */
void orc_layernorm(const float* x, const float* gamma, const float* beta, double* y,
                   int64_t rows, int64_t n, double eps, int mode) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * n;
    double* yr = y + r * n;
    if (mode == ORC_MODE_F32SEQ) {
      float s = 0.0f;
      for (int64_t i = 0; i < n; ++i) s += xr[i];
      float mean = s / (float)n, v = 0.0f;
      for (int64_t i = 0; i < n; ++i) { float d = xr[i] - mean; v += d * d; }
      float inv = 1.0f / sqrtf(v / (float)n + (float)eps);
      for (int64_t i = 0; i < n; ++i) {
        float o = (xr[i] - mean) * inv;
        if (gamma) o *= gamma[i];
        if (beta) o += beta[i];
        yr[i] = o;
      }
    } else {
      double s = 0.0;
      for (int64_t i = 0; i < n; ++i) s += xr[i];
      double mean = s / (double)n, v = 0.0;
      for (int64_t i = 0; i < n; ++i) { double d = xr[i] - mean; v += d * d; }
      double inv = 1.0 / sqrt(v / (double)n + eps);
      for (int64_t i = 0; i < n; ++i) {
        double o = ((double)xr[i] - mean) * inv;
        if (gamma) o *= gamma[i];
        if (beta) o += beta[i];
        yr[i] = o;
      }
    }
  }
}

/* ---------------------------------------------------------------------------
 * RMSNorm: no reference op exists (mpsgraph/gomlx/capabilities.go:134-140 lists
 * no RMSNorm); GoMLX graphs express it as the primitive chain Mul(x,x) ->
 * ReduceSum (function.go:1184-1186) -> Div/Mul by 1/n -> Add eps (:808-810) ->
 * Rsqrt (:686-688) -> Mul x -> Mul gamma (BroadcastInDim :1013-1042).
 * ------------------------------------------------------------------------- */
void orc_rmsnorm(const float* x, const float* gamma, double* y, int64_t rows, int64_t n,
                 double eps, int mode) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * n;
    double* yr = y + r * n;
    if (mode == ORC_MODE_F32SEQ) {
      float s = 0.0f;
      for (int64_t i = 0; i < n; ++i) s += xr[i] * xr[i];
      float inv = 1.0f / sqrtf(s / (float)n + (float)eps);
      for (int64_t i = 0; i < n; ++i) {
        float o = xr[i] * inv;
        if (gamma) o *= gamma[i];
        yr[i] = o;
      }
    } else {
      double s = 0.0;
      for (int64_t i = 0; i < n; ++i) s += (double)xr[i] * xr[i];
      double inv = 1.0 / sqrt(s / (double)n + eps);
      for (int64_t i = 0; i < n; ++i) {
        double o = (double)xr[i] * inv;
        if (gamma) o *= gamma[i];
        yr[i] = o;
      }
    }
  }
}

/* RMSNorm with fp32 output and fp32 sequential statistics: the same arithmetic
 * as orc_rmsnorm's ORC_MODE_F32SEQ (a plain loop over float32, the way a pure-Go
 * backend would write it), stored as float32.  This is the CPU baseline that
 * bench.py times; the parity tests use the fp64 forms. */
void orc_rmsnorm_f32(const float* x, const float* gamma, float* y, int64_t rows, int64_t n,
                     double eps) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * n;
    float* yr = y + r * n;
    float s = 0.0f;
    for (int64_t i = 0; i < n; ++i) s += xr[i] * xr[i];
    const float inv = 1.0f / sqrtf(s / (float)n + (float)eps);
    for (int64_t i = 0; i < n; ++i) {
      float o = xr[i] * inv;
      if (gamma) o *= gamma[i];
      yr[i] = o;
    }
  }
}

/* ---------------------------------------------------------------------------
 * DotGeneral.
 * Reference: dotGeneralOutputShape (mpsgraph/gomlx/dotgeneral.go:15-53) fixes the
 * output order [batch (lhs batch-axes order)..., lhs free (ascending)..., rhs free
 * (ascending)...] and dtype; classifyAxes (:186-227) pairs lhsContracting[i] with
 * rhsContracting[i] and lhsBatch[i] with rhsBatch[i]; DotGeneral (:65-164) sums over
 * the contracting axes.
 * ------------------------------------------------------------------------- */
static int in_list(int a, const int* l, int n) {
  for (int i = 0; i < n; ++i) if (l[i] == a) return 1;
  return 0;
}

/* Offsets (in elements) of every multi-index over `axes` (row-major over the
 * listed axis order) for a tensor with row-major `dims`. */
static int64_t* axis_offsets(const int64_t* dims, int rank, const int* axes, int naxes,
                             int64_t* count_out) {
  int64_t strides[ORC_MAX_RANK];
  int64_t s = 1;
  for (int i = rank - 1; i >= 0; --i) { strides[i] = s; s *= dims[i]; }
  int64_t count = 1;
  for (int i = 0; i < naxes; ++i) count *= dims[axes[i]];
  int64_t* off = (int64_t*)malloc(sizeof(int64_t) * (size_t)(count > 0 ? count : 1));
  for (int64_t c = 0; c < count; ++c) {
    int64_t rem = c, o = 0;
    for (int i = naxes - 1; i >= 0; --i) {
      int64_t d = dims[axes[i]];
      o += (rem % d) * strides[axes[i]];
      rem /= d;
    }
    off[c] = o;
  }
  *count_out = count;
  return off;
}

int orc_dot_general(const float* lhs, int lrank, const int64_t* ldims,
                    const int* lcontract, int nlc, const int* lbatch, int nlb,
                    const float* rhs, int rrank, const int64_t* rdims,
                    const int* rcontract, int nrc, const int* rbatch, int nrb,
                    double* out, int mode) {
  if (nlc != nrc || nlb != nrb || lrank > ORC_MAX_RANK || rrank > ORC_MAX_RANK) return -1;
  for (int i = 0; i < nlc; ++i)
    if (ldims[lcontract[i]] != rdims[rcontract[i]]) return -1;
  for (int i = 0; i < nlb; ++i)
    if (ldims[lbatch[i]] != rdims[rbatch[i]]) return -1;
  int lfree[ORC_MAX_RANK], rfree[ORC_MAX_RANK], nlf = 0, nrf = 0;
  for (int i = 0; i < lrank; ++i)
    if (!in_list(i, lcontract, nlc) && !in_list(i, lbatch, nlb)) lfree[nlf++] = i;
  for (int i = 0; i < rrank; ++i)
    if (!in_list(i, rcontract, nrc) && !in_list(i, rbatch, nrb)) rfree[nrf++] = i;
  int64_t nb, nm, nk, nn, tmp;
  int64_t* lb = axis_offsets(ldims, lrank, lbatch, nlb, &nb);
  int64_t* lm = axis_offsets(ldims, lrank, lfree, nlf, &nm);
  int64_t* lk = axis_offsets(ldims, lrank, lcontract, nlc, &nk);
  int64_t* rb = axis_offsets(rdims, rrank, rbatch, nrb, &tmp);
  int64_t* rn = axis_offsets(rdims, rrank, rfree, nrf, &nn);
  int64_t* rk = axis_offsets(rdims, rrank, rcontract, nrc, &tmp);
  /* k-outer / n-inner so rows of rhs stream; each output still accumulates its
   * terms in k order (sequentially for ORC_MODE_F32SEQ). */
#pragma omp parallel
  {
    double* acc = (double*)malloc(sizeof(double) * (size_t)(nn > 0 ? nn : 1));
    float* acc32 = (float*)malloc(sizeof(float) * (size_t)(nn > 0 ? nn : 1));
#pragma omp for collapse(2) schedule(static)
    for (int64_t b = 0; b < nb; ++b) {
      for (int64_t m = 0; m < nm; ++m) {
        const float* lp = lhs + lb[b] + lm[m];
        for (int64_t n = 0; n < nn; ++n) { acc[n] = 0.0; acc32[n] = 0.0f; }
        for (int64_t k = 0; k < nk; ++k) {
          const float* rp = rhs + rb[b] + rk[k];
          if (mode == ORC_MODE_F32SEQ) {
            const float a = lp[lk[k]];
            for (int64_t n = 0; n < nn; ++n) acc32[n] += a * rp[rn[n]];
          } else {
            const double a = lp[lk[k]];
            for (int64_t n = 0; n < nn; ++n) acc[n] += a * (double)rp[rn[n]];
          }
        }
        double* o = out + (b * nm + m) * nn;
        for (int64_t n = 0; n < nn; ++n) o[n] = mode == ORC_MODE_F32SEQ ? (double)acc32[n] : acc[n];
      }
    }
    free(acc);
    free(acc32);
  }
  free(lb); free(lm); free(lk); free(rb); free(rn); free(rk);
  return 0;
}

/* Sampled entries of the canonical batched product (a size-independent check
 * of a full-size DotGeneral: each sampled entry is an fp64 dot product). */
void orc_dot_sampled(const float* a, int64_t sa_b, int64_t sa_m, int64_t sa_k,
                     const float* b, int64_t sb_b, int64_t sb_k, int64_t sb_n, int64_t K,
                     const int64_t* bs, const int64_t* ms, const int64_t* ns, int64_t count,
                     double* out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < count; ++i) {
    const float* ap = a + bs[i] * sa_b + ms[i] * sa_m;
    const float* bp = b + bs[i] * sb_b + ns[i] * sb_n;
    double acc = 0.0;
    for (int64_t k = 0; k < K; ++k) acc += (double)ap[k * sa_k] * (double)bp[k * sb_k];
    out[i] = acc;
  }
}

/* ---------------------------------------------------------------------------
 * Scaled dot-product attention.
 * Reference: Function.FusedScaledDotProductAttention (mpsgraph/gomlx/function.go:
 * 2669-2907): scores = DotGeneral(Q, K) contracting D with batch [B,H] (:2746-2753);
 * scores *= scale (:2755-2770); causal keeps rowIota >= colIota over [Sq,Sk]
 * (:2773-2790); boolean mask: Where(mask, scores, -inf) (:2847-2871); additive
 * mask: scores + mask (:2872-2878); a mask of any rank broadcasts to the scores
 * over its trailing axes (broadcastMaskToScores :2959-2974; here element strides
 * over (b, h, query, key), 0 on broadcast axes); softmax over
 * the last axis (:2880-2886); output = DotGeneral(P, V) (:2888-2897).  GQA repeats
 * each KV head numHeads/numKVHeads times consecutively (repeatHeads :2911-2956),
 * so query head h reads KV head h / (H / Hkv).
 * ------------------------------------------------------------------------- */
void orc_sdpa(const float* q, const float* k, const float* v, const void* mask, int mask_kind,
              const int64_t* mstr, int64_t B, int64_t H, int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D,
              double scale, int causal, double* out) {
  int64_t rep = H / Hkv;
#pragma omp parallel
  {
    double* p = (double*)malloc(sizeof(double) * (size_t)Sk);
#pragma omp for collapse(3) schedule(static)
    for (int64_t bb = 0; bb < B; ++bb)
      for (int64_t h = 0; h < H; ++h)
        for (int64_t i = 0; i < Sq; ++i) {
          int64_t hk = h / rep;
          const float* qr = q + ((bb * H + h) * Sq + i) * D;
          const float* kb = k + (bb * Hkv + hk) * Sk * D;
          const float* vb = v + (bb * Hkv + hk) * Sk * D;
          const int64_t mrow = mask_kind ? bb * mstr[0] + h * mstr[1] + i * mstr[2] : 0;
          double mx = -INFINITY;
          for (int64_t j = 0; j < Sk; ++j) {
            double s = 0.0;
            for (int64_t d = 0; d < D; ++d) s += (double)qr[d] * (double)kb[j * D + d];
            s *= scale;
            if (mask_kind == ORC_MASK_BOOL && !((const uint8_t*)mask)[mrow + j * mstr[3]]) s = -INFINITY;
            if (mask_kind == ORC_MASK_ADD) s += (double)((const float*)mask)[mrow + j * mstr[3]];
            if (causal && !(i >= j)) s = -INFINITY;
            p[j] = s;
            if (p[j] > mx) mx = p[j];
          }
          /* a row with every key masked: exp(-inf - -inf) = NaN, as the reference's
           * softmax of a row of -inf gives */
          double sum = 0.0;
          for (int64_t j = 0; j < Sk; ++j) { p[j] = exp(p[j] - mx); sum += p[j]; }
          double* orow = out + ((bb * H + h) * Sq + i) * D;
          for (int64_t d = 0; d < D; ++d) orow[d] = 0.0;
          for (int64_t j = 0; j < Sk; ++j) {
            double w = p[j] / sum;
            for (int64_t d = 0; d < D; ++d) orow[d] += w * (double)vb[j * D + d];
          }
        }
    free(p);
  }
}

/* ---------------------------------------------------------------------------
 * Embedding gather.
 * Reference: Function.Gather (mpsgraph/gomlx/gather.go:24-56) takes the
 * embedding fast path gatherEmbeddingLookup (:61-203) when startIndexMap = [axis],
 * sliceSizes[axis] = 1, axis collapsed and the other slice sizes full: the result
 * is the indexed rows of the operand, in index order.  Out-of-range start indices
 * are clamped into [0, V-1], XLA's Gather rule (the rule of the GoMLX graph
 * layer; parity with simplego for out-of-range ids is otherwise unpinned).
 * ------------------------------------------------------------------------- */
void orc_gather_rows(const void* table, int64_t V, int64_t row_bytes, const int32_t* ids,
                     int64_t n, void* out) {
  const unsigned char* t = (const unsigned char*)table;
  unsigned char* o = (unsigned char*)out;
  for (int64_t i = 0; i < n; ++i) {
    int64_t id = ids[i];
    if (id < 0) id = 0;
    if (id > V - 1) id = V - 1;
    memcpy(o + i * row_bytes, t + id * row_bytes, (size_t)row_bytes);
  }
}

/* ---------------------------------------------------------------------------
 * ArgMinMax.
 * Reference: Function.ArgMinMax (mpsgraph/gomlx/function.go:1204-1242): index of the
 * max (min) along `axis`, with that axis removed from the output shape.  Tie and
 * NaN rules are not fixed by the reference (MPSGraph decides); the rule used here
 * is numpy's (first occurrence; NaN propagates as the extreme).
 * ------------------------------------------------------------------------- */
void orc_argminmax(const float* x, int64_t outer, int64_t n, int64_t inner, int is_min,
                   int64_t* out) {
  for (int64_t o = 0; o < outer; ++o)
    for (int64_t j = 0; j < inner; ++j) {
      const float* xr = x + o * n * inner + j;
      int64_t best = 0;
      float bv = xr[0];
      if (!isnan(bv)) {
        for (int64_t i = 1; i < n; ++i) {
          float v = xr[i * inner];
          if (isnan(v)) { best = i; break; }
          if (is_min ? (v < bv) : (v > bv)) { bv = v; best = i; }
        }
      }
      out[o * inner + j] = best;
    }
}

/* ArgMin / ArgMax of integers (x widened to int64, or to uint64 when
 * is_unsigned): the extreme value, ties to the lowest index. */
void orc_argminmax_int(const int64_t* x, int64_t outer, int64_t n, int64_t inner, int is_min,
                       int is_unsigned, int64_t* out) {
  for (int64_t o = 0; o < outer; ++o)
    for (int64_t j = 0; j < inner; ++j) {
      const int64_t* xr = x + o * n * inner + j;
      int64_t best = 0;
      for (int64_t i = 1; i < n; ++i) {
        const int64_t v = xr[i * inner], b = xr[best * inner];
        int better;
        if (is_unsigned)
          better = is_min ? ((uint64_t)v < (uint64_t)b) : ((uint64_t)v > (uint64_t)b);
        else
          better = is_min ? (v < b) : (v > b);
        if (better) best = i;
      }
      out[o * inner + j] = best;
    }
}

/* ---------------------------------------------------------------------------
 * Iota.
 * Reference: Function.Iota (mpsgraph/gomlx/function.go:1127-1135) ->
 * coordinateAlongAxis + cast (internal/bridge/bridge.m:237-259): the index along
 * `iotaAxis`, converted to the output dtype.
 * ------------------------------------------------------------------------- */
void orc_iota(double* out, int64_t outer, int64_t n, int64_t inner) {
  for (int64_t o = 0; o < outer; ++o)
    for (int64_t i = 0; i < n; ++i)
      for (int64_t j = 0; j < inner; ++j) out[(o * n + i) * inner + j] = (double)i;
}

/* ---------------------------------------------------------------------------
 * DynamicSlice / DynamicUpdateSlice.
 * Reference: Function.DynamicSlice / DynamicUpdateSlice (mpsgraph/gomlx/
 * function.go:1571-1621) -> bridge.m:918-1104: a window of the operand at
 * run-time start indices.  Starts are clamped to [0, dim - window] (XLA's
 * definition of both ops, which GoMLX's backend API follows; the reference's
 * tests only use in-range starts, mpsgraph_test.go:993-1131).
 * ------------------------------------------------------------------------- */
static int64_t clamp64(int64_t v, int64_t lo, int64_t hi) { return v < lo ? lo : (v > hi ? hi : v); }

void orc_dynamic_slice(const void* x, int elem_bytes, int rank, const int64_t* dims, const int64_t* starts,
                       const int64_t* sizes, void* out) {
  int64_t st[ORC_MAX_RANK], xs[ORC_MAX_RANK], n = 1, acc = 1;
  for (int k = rank - 1; k >= 0; --k) {
    xs[k] = acc;
    acc *= dims[k];
  }
  for (int k = 0; k < rank; ++k) {
    st[k] = clamp64(starts[k], 0, dims[k] - sizes[k]);
    n *= sizes[k];
  }
  for (int64_t i = 0; i < n; ++i) {
    int64_t q = i, off = 0;
    for (int k = rank - 1; k >= 0; --k) {
      off += (st[k] + q % sizes[k]) * xs[k];
      q /= sizes[k];
    }
    memcpy((char*)out + i * elem_bytes, (const char*)x + off * elem_bytes, (size_t)elem_bytes);
  }
}

void orc_dynamic_update_slice(const void* x, int elem_bytes, int rank, const int64_t* dims, const void* upd,
                              const int64_t* udims, const int64_t* starts, void* out) {
  int64_t st[ORC_MAX_RANK], xs[ORC_MAX_RANK], n = 1, total = 1;
  for (int k = rank - 1; k >= 0; --k) {
    xs[k] = total;
    total *= dims[k];
  }
  memcpy(out, x, (size_t)(total * elem_bytes));
  for (int k = 0; k < rank; ++k) {
    st[k] = clamp64(starts[k], 0, dims[k] - udims[k]);
    n *= udims[k];
  }
  for (int64_t i = 0; i < n; ++i) {
    int64_t q = i, off = 0;
    for (int k = rank - 1; k >= 0; --k) {
      off += (st[k] + q % udims[k]) * xs[k];
      q /= udims[k];
    }
    memcpy((char*)out + off * elem_bytes, (const char*)upd + i * elem_bytes, (size_t)elem_bytes);
  }
}

/* ---------------------------------------------------------------------------
 * Scatter.
 * Reference: Function.ScatterSum / ScatterMax / ScatterMin (mpsgraph/gomlx/
 * gather.go:441-640) -> MPSGraph scatterAlongAxis / scatterND with mode add /
 * max / min (bridge.m:789-815, 1624-1660): XLA scatter.  For update element u:
 * its scatter coordinates select an index vector in `indices`; component k
 * gives the start along operand axis sato[k]; its window coordinates (the
 * update axes listed in uwa) run, in order, over the operand axes not listed
 * in iwa.  Windows that do not fit are skipped (XLA); out-of-range behaviour is
 * not fixed by the reference's tests.
 * ------------------------------------------------------------------------- */
void orc_scatter(int mode, const double* operand, int r, const int64_t* odims, const int64_t* indices, int ir,
                 const int64_t* idims, int iva, const double* updates, int ur, const int64_t* udims,
                 const int* uwa, int n_uwa, const int* iwa, int n_iwa, const int* sato, int n_sato, double* out) {
  int64_t ostr[ORC_MAX_RANK], istr[ORC_MAX_RANK + 1], total = 1, nu = 1;
  for (int k = r - 1; k >= 0; --k) {
    ostr[k] = total;
    total *= odims[k];
  }
  memcpy(out, operand, (size_t)total * sizeof(double));
  int64_t acc = 1;
  for (int k = ir - 1; k >= 0; --k) {
    istr[k] = acc;
    acc *= idims[k];
  }
  for (int k = 0; k < ur; ++k) nu *= udims[k];
  int win_od[ORC_MAX_RANK];  /* operand axis of each update window axis */
  int64_t wsize[ORC_MAX_RANK];
  for (int k = 0; k < r; ++k) wsize[k] = 1;
  {
    int j = 0;
    for (int k = 0; k < r; ++k) {
      if (in_list(k, iwa, n_iwa)) continue;
      win_od[j] = k;
      wsize[k] = udims[uwa[j]];
      ++j;
    }
  }
  for (int64_t u = 0; u < nu; ++u) {
    int64_t c[ORC_MAX_RANK], q = u;
    for (int k = ur - 1; k >= 0; --k) {
      c[k] = q % udims[k];
      q /= udims[k];
    }
    /* indices position: batch coordinates in order, skipping iva */
    int64_t ipos = 0;
    int bi = 0, wj = 0;
    int64_t w[ORC_MAX_RANK];
    for (int k = 0; k < r; ++k) w[k] = 0;
    for (int k = 0; k < ur; ++k) {
      if (in_list(k, uwa, n_uwa)) {
        w[win_od[wj++]] = c[k];
      } else {
        if (bi == iva) ++bi;
        ipos += c[k] * istr[bi];
        ++bi;
      }
    }
    int64_t start[ORC_MAX_RANK];
    for (int k = 0; k < r; ++k) start[k] = 0;
    for (int k = 0; k < n_sato; ++k) start[sato[k]] = indices[ipos + (iva < ir ? k * istr[iva] : 0)];
    int ok = 1;
    for (int k = 0; k < r; ++k)
      if (start[k] < 0 || start[k] > odims[k] - wsize[k]) ok = 0;
    if (!ok) continue;
    int64_t off = 0;
    for (int k = 0; k < r; ++k) off += (start[k] + w[k]) * ostr[k];
    const double v = updates[u], o = out[off];
    if (mode == 0) out[off] = o + v;
    else if (isnan(o) || isnan(v)) out[off] = NAN;
    else out[off] = mode == 1 ? (v > o ? v : o) : (v < o ? v : o);
  }
}

/* ---------------------------------------------------------------------------
 * Activations of FusedDense / FusedGelu.
 * Reference: Function.FusedGelu (mpsgraph/gomlx/function.go:2288-2408):
 *   exact:  x * 0.5 * (1 + erf(x / sqrt 2));
 *   approx: 0.5 * x * (1 + tanh(0.7978845608 * (x + 0.044715 x^3)));
 * FusedDense (function.go:2620-2664): GELU is the approximate form, ReLU
 * max(x, 0), SiLU x * sigmoid(x), Tanh tanh(x).
 * ------------------------------------------------------------------------- */
void orc_activation(const double* x, double* y, int64_t n, int act) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    const double v = x[i];
    double r = v;
    switch (act) {
      case ORC_ACT_GELU: r = 0.5 * v * (1.0 + tanh(0.7978845608 * (v + 0.044715 * v * v * v))); break;
      case ORC_ACT_GELU_EXACT: r = 0.5 * v * (1.0 + erf(v * 0.7071067811865475)); break;
      case ORC_ACT_RELU: r = isnan(v) ? v : (v > 0.0 ? v : 0.0); break;
      case ORC_ACT_SILU: r = v / (1.0 + exp(-v)); break;
      case ORC_ACT_TANH: r = tanh(v); break;
      default: break;
    }
    y[i] = r;
  }
}

void orc_f32_to_bf16(const float* x, uint16_t* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    uint32_t u;
    memcpy(&u, &x[i], 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) { y[i] = (uint16_t)((u >> 16) | 0x40); continue; }
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    y[i] = (uint16_t)(u >> 16);
  }
}
