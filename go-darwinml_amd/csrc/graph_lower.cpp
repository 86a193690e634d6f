// Compile-time lowering: graph -> launch plan.
//
// What the reference leaves to MPSGraph's closed compiler (bridge.m:1112-1240) is
// done here, explicitly:
//   * Views, not copies: Reshape of contiguous data, Transpose, BroadcastInDim and
//     Slice only rewrite (offset, strides).  Consumers that take strided operands
//     (generated elementwise kernels, the GEMM, reductions) read through them;
//     others get one strided-copy materialisation.
//   * Pattern fusion into the hand-written row kernels: FusedSoftmax, the
//     primitive softmax and log-softmax chains, the RMSNorm chain
//     (x * rsqrt(mean(x^2) + eps) * gamma), FusedLayerNorm, and
//     FusedScaledDotProductAttention = GEMM -> scale+mask+softmax -> GEMM.
//   * DotGeneral -> batched MFMA GEMM with batch / free / contracting axis groups
//     folded into single strides whenever the operand layout allows (no
//     transposes, unlike dotgeneral.go:97-148), output [batch, lhs free, rhs free].
//   * Elementwise clusters (Unary / Binary / Compare / Where / Clamp / Convert,
//     plus Iota leaves and scalar constants inlined as literals) become one
//     generated kernel each (rtc.cpp), so adjacent elementwise chains make one
//     HBM round trip.
//   * Intermediates live in one arena per executable; offsets come from a
//     first-fit interval allocation over step lifetimes.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <array>
#include <map>
#include <set>
#include <sstream>

#include "common.h"
#include "gemm_bf16_dev.h"
#include "graph.h"

namespace ghip {
namespace {

struct Fusion {
  enum Kind { None, RmsNorm, Softmax, LogSoftmax, LayerNorm } kind = None;
  int x = -1, gamma = -1, beta = -1;
  double eps = 0;
};

// Helpers shared by every generated elementwise kernel: bf16 / f16 rounding
// (round to nearest even, NaN kept quiet; for bf16 gfx950's v_cvt_pk_bf16_f32,
// which computes exactly that), NaN-propagating min/max, integer pow.
const char kRtcPrelude[] = R"(typedef unsigned short u16;
__device__ __forceinline__ float bf2f(u16 b) { return __uint_as_float(((unsigned)b) << 16); }
__device__ __forceinline__ u16 f2bf(float f) { return __builtin_bit_cast(u16, (__bf16)f); }
// f rounded to bf16 and widened back, in one v_cvt_pk_bf16_f32: the pair (0, f)
// converts to the 32-bit word (bf16(f) << 16) | bf16(0), which is that float.
typedef float rbf_f2 __attribute__((ext_vector_type(2)));
typedef __bf16 rbf_b2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float rbf(float f) {
  const rbf_f2 v = {0.0f, f};
  return __builtin_bit_cast(float, __builtin_convertvector(v, rbf_b2));
}
__device__ __forceinline__ float rhf(float f) { return (float)(_Float16)f; }
// exp / logistic / tanh for ops whose result is rounded to bf16 or f16: the
// hardware exp2 and reciprocal (relative error below 1e-5 over the whole range,
// far inside half an ulp of a 16-bit result), instead of the correctly rounded
// fp32 library routines with their range reductions.
__device__ __forceinline__ float hexp(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }
__device__ __forceinline__ float hsigmoid(float x) { return __builtin_amdgcn_rcpf(1.0f + hexp(-x)); }
__device__ __forceinline__ float htanh(float x) {
  const float ax = __builtin_fabsf(x), p = x * x;
  // |x| < 1/16: the odd series x - x^3/3 + 2x^5/15; else 1 - 2 / (e^(2|x|) + 1) with
  // e^(2|x|) = exp2(|x| * 2 log2(e)).  Explicit FMAs (generated code compiles without
  // contraction): 12 instructions.
  const float small = __builtin_fmaf(x * p, __builtin_fmaf(p, 0.13333333f, -0.33333333f), x);
  const float e2 = __builtin_amdgcn_exp2f(ax * 2.8853900817779268f);
  const float big = __builtin_copysignf(__builtin_fmaf(-2.0f, __builtin_amdgcn_rcpf(e2 + 1.0f), 1.0f), x);
  return ax < 0.0625f ? small : big;
}
template <typename T> __device__ __forceinline__ T fmax_nan(T a, T b) { return (a > b || a != a) ? a : b; }
template <typename T> __device__ __forceinline__ T fmin_nan(T a, T b) { return (a < b || a != a) ? a : b; }
__device__ __forceinline__ long long ipow(long long b, long long e) {
  if (e < 0) return b == 1 ? 1 : (b == -1 ? ((e & 1) ? -1 : 1) : 0);
  long long r = 1;
  while (e) { if (e & 1) r *= b; b *= b; e >>= 1; }
  return r;
}
)";

// Text of gemm_bf16_dev.h (the bf16 MFMA GEMM core), compiled with hipRTC in
// front of generated epilogues.
const char kGemmDevSrc[] =
#include "gemm_bf16_dev.inc"
    ;

std::string fmt(const char* f, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, f);
  vsnprintf(buf, sizeof buf, f, ap);
  va_end(ap);
  return buf;
}

// Strides that present a strided view of dims `od` (strides `os`, row-major
// element order) as dims `nd` without moving data, when they exist: every run of
// old dims that the new dims regroup must be laid out as one row-major block
// (os[k] == od[k+1] * os[k+1] inside the run).  Size-1 dims impose nothing.
static bool reshape_strides(const std::vector<int64_t>& od, const std::vector<int64_t>& os,
                            const std::vector<int64_t>& nd, std::vector<int64_t>* ns) {
  std::vector<int64_t> d, st;
  int64_t total = 1;
  for (size_t i = 0; i < od.size(); ++i) {
    total *= od[i];
    if (od[i] != 1) d.push_back(od[i]), st.push_back(os[i]);
  }
  ns->assign(nd.size(), 1);
  if (total == 0) {
    *ns = contiguous_strides(nd);
    return true;
  }
  size_t i = 0, j = 0;
  const size_t n_old = d.size(), n_new = nd.size();
  while (i < n_old && j < n_new) {
    const size_t i0 = i, j0 = j;
    int64_t po = d[i], pn = nd[j];
    while (po != pn) {
      if (pn < po) {
        if (++j >= n_new) return false;
        pn *= nd[j];
      } else {
        if (++i >= n_old) return false;
        po *= d[i];
      }
    }
    for (size_t k = i0; k < i; ++k)
      if (st[k] != d[k + 1] * st[k + 1]) return false;
    (*ns)[j] = st[i];
    for (size_t k = j; k > j0; --k) (*ns)[k - 1] = (*ns)[k] * nd[k];
    ++i;
    ++j;
  }
  if (i != n_old) return false;
  for (; j < n_new; ++j)
    if (nd[j] != 1) return false;
  return true;
}

struct Lowerer {
  GHipBackend* be;
  GHipFunction* fn;
  Plan* plan;
  GHipError* err;
  std::deque<Node>& N;
  std::vector<char> live;
  std::vector<std::vector<int>> users;
  std::vector<int> cluster;  // elementwise cluster id (= root node) or -1
  std::vector<Fusion> fusion;
  std::vector<char> have;
  std::vector<View> views;
  std::vector<std::vector<int>> reads, writes;
  std::vector<std::vector<int>> inplace_slots;  // per step: read slots its output may alias
  std::vector<std::vector<uint8_t>> const_data;  // per slot (Const slots)
  bool failed = false;

  Lowerer(GHipBackend* b, GHipFunction* f, Plan* p, GHipError* e)
      : be(b), fn(f), plan(p), err(e), N(f->nodes) {}

  View bad() {
    failed = true;
    return View{};
  }
  View fail(int code, const char* what) {
    if (!failed) set_error(err, code, "Compile: %s", what);
    return bad();
  }

  // ------------------------------------------------------------------ slots
  int new_slot(SlotKind k, size_t bytes, int index = 0) {
    Slot s;
    s.kind = k;
    s.bytes = bytes;
    s.index = index;
    plan->slots.push_back(s);
    const_data.emplace_back();
    return static_cast<int>(plan->slots.size()) - 1;
  }
  View contig(int slot, const Shape& s) {
    View v;
    v.slot = slot;
    v.strides = contiguous_strides(s.dims);
    return v;
  }
  View fresh(const Shape& s) { return contig(new_slot(SlotKind::Arena, s.bytes()), s); }

  void add_step(const std::string& desc, std::vector<int> r, std::vector<int> w, StepFn f,
                std::vector<int> inplace = {}) {
    plan->steps.push_back(Step{desc, std::move(f)});
    reads.push_back(std::move(r));
    writes.push_back(std::move(w));
    inplace_slots.push_back(std::move(inplace));
  }

  // ------------------------------------------------------------------ analysis
  void analyse() {
    const int n = static_cast<int>(N.size());
    live.assign(n, 0);
    users.assign(n, {});
    std::vector<int> stack(fn->outputs.begin(), fn->outputs.end());
    while (!stack.empty()) {
      int v = stack.back();
      stack.pop_back();
      if (v < 0 || live[v]) continue;
      live[v] = 1;
      for (int o : N[v].in)
        if (o >= 0) stack.push_back(o);
    }
    for (int v = 0; v < n; ++v)
      if (live[v])
        for (int o : N[v].in)
          if (o >= 0) users[o].push_back(v);
    fusion.assign(n, Fusion{});
    for (int v = n - 1; v >= 0; --v)
      if (live[v]) match_patterns(v);
    build_clusters();
    find_reduce_fusions();
  }

  // ------------------------------------------------------------------ patterns
  int strip_reshape(int v) {
    while (v >= 0 && N[v].kind == Kind::Reshape) v = N[v].in[0];
    return v;
  }
  // Scalar constant behind Reshape/Broadcast chains: returns true and its value.
  bool scalar_const(int v, double* val) {
    while (v >= 0 && (N[v].kind == Kind::Reshape || N[v].kind == Kind::Broadcast)) v = N[v].in[0];
    if (v < 0 || N[v].kind != Kind::Const || N[v].shape.size() != 1) return false;
    *val = const_as_double(N[v], 0);
    return true;
  }
  static double const_as_double(const Node& c, int64_t i) {
    const uint8_t* p = c.data.data() + i * dtype_size(c.shape.dtype);
    switch (c.shape.dtype) {
      case GHIP_DTYPE_FLOAT32: { float f; memcpy(&f, p, 4); return f; }
      case GHIP_DTYPE_FLOAT64: { double d; memcpy(&d, p, 8); return d; }
      case GHIP_DTYPE_BFLOAT16: { uint16_t b; memcpy(&b, p, 2); return bf16_to_f32(b); }
      case GHIP_DTYPE_FLOAT16: { _Float16 h; memcpy(&h, p, 2); return static_cast<double>(h); }
      case GHIP_DTYPE_INT8: { int8_t x; memcpy(&x, p, 1); return x; }
      case GHIP_DTYPE_INT16: { int16_t x; memcpy(&x, p, 2); return x; }
      case GHIP_DTYPE_INT32: { int32_t x; memcpy(&x, p, 4); return x; }
      case GHIP_DTYPE_INT64: { int64_t x; memcpy(&x, p, 8); return static_cast<double>(x); }
      case GHIP_DTYPE_UINT8: case GHIP_DTYPE_BOOL: { uint8_t x; memcpy(&x, p, 1); return x; }
      case GHIP_DTYPE_UINT16: { uint16_t x; memcpy(&x, p, 2); return x; }
      case GHIP_DTYPE_UINT32: { uint32_t x; memcpy(&x, p, 4); return x; }
      case GHIP_DTYPE_UINT64: { uint64_t x; memcpy(&x, p, 8); return static_cast<double>(x); }
      default: return NAN;
    }
  }
  // v (shape == xs) broadcasts a per-row value along the last axis of xs; returns
  // the per-row value (through reshapes) in *u.
  bool row_broadcast(int v, const Shape& xs, int* u) {
    const int r = xs.rank();
    if (r == 0 || v < 0) return false;
    const int64_t rows = xs.size() / std::max<int64_t>(xs.dims[r - 1], 1);
    const Node& b = N[v];
    int src = -1;
    if (b.kind == Kind::Broadcast && b.shape.dims == xs.dims) {
      const Node& s = N[b.in[0]];
      const int sr = s.shape.rank();
      bool ok = true;
      for (int i = 0; i < sr; ++i) {
        const int64_t ax = b.a0[i];
        if (ax == r - 1) ok = ok && s.shape.dims[i] == 1;
        else ok = ok && s.shape.dims[i] == xs.dims[ax];
      }
      // every non-last axis of xs must be covered (else it is broadcast too)
      std::set<int64_t> cov(b.a0.begin(), b.a0.end());
      for (int a = 0; a < r - 1; ++a) ok = ok && (cov.count(a) || xs.dims[a] == 1);
      if (!ok) return false;
      src = b.in[0];
    } else if (b.shape.rank() == r && b.shape.dims[r - 1] == 1 && b.shape.size() == rows && xs.dims[r - 1] != 1) {
      src = v;  // implicit numpy broadcast of a [..., 1] operand
    } else {
      return false;
    }
    if (N[src].shape.size() != rows) return false;
    *u = strip_reshape(src);
    return true;
  }
  // v is a [n]-vector broadcast along the leading axes of xs (gamma / beta).
  bool col_broadcast(int v, const Shape& xs, int* g) {
    const int r = xs.rank();
    if (r == 0) return false;
    const int64_t n = xs.dims[r - 1];
    const Node& b = N[v];
    if (b.kind == Kind::Broadcast && b.shape.dims == xs.dims) {
      const Node& s = N[b.in[0]];
      if (s.shape.size() != n) return false;
      for (int i = 0; i < s.shape.rank(); ++i)
        if (s.shape.dims[i] != 1 && b.a0[i] != r - 1) return false;
      *g = b.in[0];
      return true;
    }
    if (b.shape.size() == n && b.shape.rank() <= r && (b.shape.rank() == 0 ? false : b.shape.dims.back() == n)) {
      *g = v;
      return true;
    }
    return false;
  }
  bool is_binary(int v, int op) { return v >= 0 && N[v].kind == Kind::Binary && N[v].sub == op; }
  bool is_unary(int v, int op) { return v >= 0 && N[v].kind == Kind::Unary && N[v].sub == op; }
  bool is_last_axis_reduce(int v, int op, int x) {
    if (v < 0 || N[v].kind != Kind::Reduce || N[v].sub != op || N[v].in[0] != x) return false;
    const int r = N[x].shape.rank();
    return N[v].a0.size() == 1 && N[v].a0[0] == r - 1;
  }

  // The dtypes the row kernels take; a primitive chain in any other float dtype
  // (Float64) stays unfused and runs as elementwise and reduce kernels.
  static bool row_dtype(int dt) {
    return dt == GHIP_DTYPE_FLOAT32 || dt == GHIP_DTYPE_BFLOAT16 || dt == GHIP_DTYPE_FLOAT16;
  }

  // v = ReduceSum(t, last axis) / n, as Div by the constant n or Mul by 1/n
  // (through reshapes); returns t.
  int mean_last(int v, double n) {
    v = strip_reshape(v);
    int s = -1;
    if (is_binary(v, GHIP_BINARY_MUL)) {
      for (int q = 0; q < 2; ++q) {
        double c;
        if (scalar_const(N[v].in[q], &c) && fabs(c * n - 1.0) < 1e-5) s = strip_reshape(N[v].in[1 - q]);
      }
    } else if (is_binary(v, GHIP_BINARY_DIV)) {
      double c;
      if (scalar_const(N[v].in[1], &c) && fabs(c - n) < 1e-6 * n) s = strip_reshape(N[v].in[0]);
    }
    if (s < 0 || N[s].kind != Kind::Reduce || N[s].sub != GHIP_REDUCE_SUM) return -1;
    const int t = N[s].in[0];
    return is_last_axis_reduce(s, GHIP_REDUCE_SUM, t) ? t : -1;
  }
  // LayerNorm core as the reference composes it (function.go:2429-2497):
  // v = d * bcast(rsqrt(mean(d * d) + eps)) with d = x - bcast(mean(x)).
  bool ln_core(int v, int* xo, double* eps) {
    if (!is_binary(v, GHIP_BINARY_MUL)) return false;
    for (int o = 0; o < 2; ++o) {
      const int d = N[v].in[o], rb = N[v].in[1 - o];
      if (!is_binary(d, GHIP_BINARY_SUB) || N[d].shape.dims != N[v].shape.dims) continue;
      const int x = N[d].in[0];
      if (N[x].shape.dims != N[v].shape.dims || !row_dtype(N[x].shape.dtype)) continue;
      const double n = static_cast<double>(N[x].shape.dims.back());
      int mb, u;
      if (!row_broadcast(N[d].in[1], N[x].shape, &mb) || mean_last(mb, n) != x) continue;
      if (!row_broadcast(rb, N[x].shape, &u) || !is_unary(u, GHIP_UNARY_RSQRT)) continue;
      const int add = strip_reshape(N[u].in[0]);
      if (!is_binary(add, GHIP_BINARY_ADD)) continue;
      for (int p = 0; p < 2; ++p) {
        double e;
        if (!scalar_const(N[add].in[p], &e)) continue;
        const int sq = mean_last(N[add].in[1 - p], n);
        if (!is_binary(sq, GHIP_BINARY_MUL) || N[sq].in[0] != d || N[sq].in[1] != d) continue;
        *xo = x;
        *eps = e;
        return true;
      }
    }
    return false;
  }

  // RMSNorm core: v = x * bcast(rsqrt(mean(x*x) + eps)).
  bool rms_core(int v, int* xo, double* eps) {
    if (!is_binary(v, GHIP_BINARY_MUL)) return false;
    for (int o = 0; o < 2; ++o) {
      const int x = N[v].in[o], rb = N[v].in[1 - o];
      if (N[x].shape.dims != N[v].shape.dims || !row_dtype(N[x].shape.dtype)) continue;
      int u;
      if (!row_broadcast(rb, N[x].shape, &u) || !is_unary(u, GHIP_UNARY_RSQRT)) continue;
      const int add = strip_reshape(N[u].in[0]);
      if (!is_binary(add, GHIP_BINARY_ADD)) continue;
      for (int p = 0; p < 2; ++p) {
        double e;
        if (!scalar_const(N[add].in[p], &e)) continue;
        const int m = strip_reshape(N[add].in[1 - p]);
        const double n = static_cast<double>(N[x].shape.dims.back());
        int s = -1;
        if (is_binary(m, GHIP_BINARY_MUL)) {
          for (int q = 0; q < 2; ++q) {
            double c;
            if (scalar_const(N[m].in[q], &c) && fabs(c * n - 1.0) < 1e-5) s = strip_reshape(N[m].in[1 - q]);
          }
        } else if (is_binary(m, GHIP_BINARY_DIV)) {
          double c;
          if (scalar_const(N[m].in[1], &c) && fabs(c - n) < 1e-6 * n) s = strip_reshape(N[m].in[0]);
        }
        if (s < 0 || N[s].kind != Kind::Reduce || N[s].sub != GHIP_REDUCE_SUM) continue;
        const int sq = N[s].in[0];
        if (!is_last_axis_reduce(s, GHIP_REDUCE_SUM, sq)) continue;
        bool square = is_binary(sq, GHIP_BINARY_MUL) && N[sq].in[0] == x && N[sq].in[1] == x;
        double two;
        square = square || (is_binary(sq, GHIP_BINARY_POW) && N[sq].in[0] == x && scalar_const(N[sq].in[1], &two) && two == 2.0);
        if (!square) continue;
        *xo = x;
        *eps = e;
        return true;
      }
    }
    return false;
  }

  void match_patterns(int v) {
    const Node& n = N[v];
    if (n.kind != Kind::Binary) return;
    // LayerNorm: core [* bcast(gamma)] [+ bcast(beta)] (function.go:2429-2562).
    // Checked first: its core is an RMSNorm of x - mean.
    if ((n.sub == GHIP_BINARY_ADD || n.sub == GHIP_BINARY_MUL) && row_dtype(n.shape.dtype) && n.shape.rank() >= 1) {
      int x, g = -1, b = -1, core = -1;
      double eps;
      if (n.sub == GHIP_BINARY_ADD) {
        for (int o = 0; o < 2 && core < 0; ++o) {
          int bb;
          if (!col_broadcast(n.in[1 - o], n.shape, &bb)) continue;
          const int m = n.in[o];
          int gg;
          for (int q = 0; q < 2 && is_binary(m, GHIP_BINARY_MUL) && core < 0; ++q)
            if (col_broadcast(N[m].in[1 - q], n.shape, &gg) && ln_core(N[m].in[q], &x, &eps)) core = N[m].in[q], g = gg, b = bb;
          if (core < 0 && ln_core(m, &x, &eps)) core = m, b = bb;
        }
      } else {
        for (int o = 0; o < 2 && core < 0; ++o) {
          int gg;
          if (col_broadcast(N[v].in[1 - o], n.shape, &gg) && ln_core(N[v].in[o], &x, &eps)) core = N[v].in[o], g = gg;
        }
        if (core < 0 && ln_core(v, &x, &eps)) core = v;
      }
      if (core >= 0) {
        fusion[v] = Fusion{Fusion::LayerNorm, x, g, b, eps};
        return;
      }
    }
    // RMSNorm, with or without gamma.
    if (n.sub == GHIP_BINARY_MUL && row_dtype(n.shape.dtype) && n.shape.rank() >= 1) {
      int x, g;
      double eps;
      for (int o = 0; o < 2; ++o) {
        if (col_broadcast(n.in[1 - o], n.shape, &g) && rms_core(n.in[o], &x, &eps)) {
          fusion[v] = Fusion{Fusion::RmsNorm, x, g, -1, eps};
          return;
        }
      }
      if (rms_core(v, &x, &eps)) {
        fusion[v] = Fusion{Fusion::RmsNorm, x, -1, -1, eps};
        return;
      }
    }
    // Softmax: exp(x - bmax) / bcast(sum(exp(x - bmax))).
    if (n.sub == GHIP_BINARY_DIV && row_dtype(n.shape.dtype) && n.shape.rank() >= 1) {
      const int e = n.in[0];
      int s;
      if (is_unary(e, GHIP_UNARY_EXP) && row_broadcast(n.in[1], n.shape, &s) &&
          is_last_axis_reduce(s, GHIP_REDUCE_SUM, e)) {
        int x;
        if (shifted_by_max(N[e].in[0], &x)) {
          fusion[v] = Fusion{Fusion::Softmax, x};
          return;
        }
      }
    }
    // Log-softmax: (x - bmax) - bcast(log(sum(exp(x - bmax)))).
    if (n.sub == GHIP_BINARY_SUB && row_dtype(n.shape.dtype) && n.shape.rank() >= 1) {
      const int d = n.in[0];
      int x, l;
      if (shifted_by_max(d, &x) && row_broadcast(n.in[1], n.shape, &l) && is_unary(l, GHIP_UNARY_LOG)) {
        const int s = strip_reshape(N[l].in[0]);
        if (s >= 0 && N[s].kind == Kind::Reduce && is_unary(N[s].in[0], GHIP_UNARY_EXP) &&
            N[N[s].in[0]].in[0] == d && is_last_axis_reduce(s, GHIP_REDUCE_SUM, N[s].in[0])) {
          fusion[v] = Fusion{Fusion::LogSoftmax, x};
          return;
        }
      }
    }
  }
  // d = x - bcast(max(x, last axis)).
  bool shifted_by_max(int d, int* xo) {
    if (!is_binary(d, GHIP_BINARY_SUB)) return false;
    const int x = N[d].in[0];
    int m;
    if (N[x].shape.dims != N[d].shape.dims) return false;
    if (!row_broadcast(N[d].in[1], N[x].shape, &m)) return false;
    if (!is_last_axis_reduce(m, GHIP_REDUCE_MAX, x)) return false;
    *xo = x;
    return true;
  }

  // ------------------------------------------------------------------ clusters
  bool clusterable(int v) {
    if (!live[v] || fusion[v].kind != Fusion::None) return false;
    const Kind k = N[v].kind;
    return is_elementwise(k);
  }
  void build_clusters() {
    const int n = static_cast<int>(N.size());
    cluster.assign(n, -1);
    std::set<int> outs(fn->outputs.begin(), fn->outputs.end());
    for (int v = n - 1; v >= 0; --v) {
      if (!clusterable(v) || cluster[v] >= 0) continue;
      cluster[v] = v;  // new root
      std::vector<int> work{v};
      while (!work.empty()) {
        const int u = work.back();
        work.pop_back();
        for (int o : N[u].in) {
          if (o < 0 || cluster[o] >= 0 || !clusterable(o) || outs.count(o)) continue;
          if (N[o].shape.dims != N[v].shape.dims) continue;
          bool all_in = true;
          for (int w : users[o]) all_in = all_in && cluster[w] == v;
          if (!all_in) continue;
          cluster[o] = v;
          work.push_back(o);
        }
      }
    }
  }

  // Reduce fusion candidates (after the clusters are known).
  void find_reduce_fusions() {
    const int n = static_cast<int>(N.size());
    reduce_prod.assign(n, -1);
    cons_reduce.assign(n, -1);
    if (!fuse_reductions) return;
    std::set<int> outs(fn->outputs.begin(), fn->outputs.end());
    for (int v = 0; v < n; ++v) {
      if (!live[v] || N[v].kind != Kind::Reduce || fusion[v].kind != Fusion::None) continue;
      if (N[v].shape.dtype == GHIP_DTYPE_BOOL) continue;  // no boolean Reduce kernel to mirror
      const int p = N[v].in[0];
      if (p >= 0 && cluster[p] == p && users[p].size() == 1 && !outs.count(p)) reduce_prod[v] = p;
      if (users[v].size() == 1 && !outs.count(v)) {
        const int u = users[v][0];
        const int c = u >= 0 ? cluster[u] : -1;
        if (c >= 0 && cons_reduce[c] < 0 && N[c].shape.dims == N[v].shape.dims) {
          // a cluster fed by a DotGeneral prefers the GEMM epilogue
          bool has_dot = false;
          for (int w = 0; w <= c; ++w)
            if (cluster[w] == c)
              for (int o : N[w].in) has_dot = has_dot || (o >= 0 && N[o].kind == Kind::Dot);
          if (!has_dot) cons_reduce[c] = v;
        }
      }
    }
  }

  // ------------------------------------------------------------------ views
  View get(int v) {
    if (failed) return View{};
    if (have[v]) return views[v];
    View r;
    const Node& n = N[v];
    if (fusion[v].kind != Fusion::None) {
      r = emit_fusion(v);
    } else {
      switch (n.kind) {
        case Kind::Param: r = contig(new_slot(SlotKind::Input, n.shape.bytes(), static_cast<int>(n.i0)), n.shape); break;
        case Kind::Capture:  // inputs after the params, in capture order
          r = contig(new_slot(SlotKind::Input, n.shape.bytes(), static_cast<int>(fn->params.size() + n.i0)), n.shape);
          break;
        case Kind::TupleGet: {
          const int cf = n.in[0];
          if (!cf_out.count(cf)) emit_control_flow(cf);
          if (failed) return bad();
          r = cf_out[cf][n.i0];
          break;
        }
        case Kind::Call: case Kind::While: case Kind::If: case Kind::Sort:
          return fail(GHIP_ERR_STATE, "control-flow tuple used as a value");
        case Kind::Const: {
          r = contig(new_slot(SlotKind::Const, n.shape.bytes()), n.shape);
          const_data[r.slot] = n.data;
          break;
        }
        case Kind::Reshape: {
          View s = get(n.in[0]);
          if (failed) return bad();
          std::vector<int64_t> st;
          if (reshape_strides(N[n.in[0]].shape.dims, s.strides, n.shape.dims, &st)) {
            r = s;  // zero-copy: the new dims group the old ones without crossing a stride break
            r.strides = st;
          } else {
            s = materialize(s, N[n.in[0]].shape);
            r = s;
            r.strides = contiguous_strides(n.shape.dims);
          }
          break;
        }
        case Kind::Transpose: {
          View s = get(n.in[0]);
          if (failed) return bad();
          r = s;
          for (size_t i = 0; i < n.a0.size(); ++i) r.strides[i] = s.strides[n.a0[i]];
          break;
        }
        case Kind::Broadcast: {
          View s = get(n.in[0]);
          if (failed) return bad();
          r.slot = s.slot;
          r.offset = s.offset;
          r.strides.assign(n.shape.rank(), 0);
          const Shape& ss = N[n.in[0]].shape;
          for (int i = 0; i < ss.rank(); ++i)
            if (ss.dims[i] != 1) r.strides[n.a0[i]] = s.strides[i];
          break;
        }
        case Kind::Slice: {
          View s = get(n.in[0]);
          if (failed) return bad();
          r = s;
          for (int i = 0; i < n.shape.rank(); ++i) {
            r.offset += n.a0[i] * s.strides[i];
            r.strides[i] = s.strides[i] * n.a2[i];
          }
          break;
        }
        case Kind::Reverse: {  // negative-stride view
          View s = get(n.in[0]);
          if (failed) return bad();
          r = s;
          for (auto a : n.a0) {
            r.offset += (n.shape.dims[a] - 1) * s.strides[a];
            r.strides[a] = -s.strides[a];
          }
          break;
        }
        case Kind::Iota: r = emit_iota(v); break;
        case Kind::Unary: case Kind::Binary: case Kind::Compare: case Kind::Where:
        case Kind::Clamp: case Kind::Convert:
          r = emit_cluster(cluster[v] == v ? v : -1, v);
          break;
        case Kind::Concat: r = emit_concat(v); break;
        case Kind::Reduce: r = emit_reduce(v); break;
        case Kind::ArgMinMax: r = emit_argminmax(v); break;
        case Kind::Dot: r = emit_dot(v); break;
        case Kind::Gather: r = emit_gather(v); break;
        case Kind::Softmax: r = emit_softmax(v); break;
        case Kind::LayerNorm: r = emit_layernorm(v); break;
        case Kind::SDPA: r = emit_sdpa(v); break;
        case Kind::DynSlice: r = emit_dyn_slice(v); break;
        case Kind::DynUpdate: r = emit_dyn_update(v); break;
        case Kind::Scatter: r = emit_scatter(v); break;
      }
    }
    if (failed) return bad();
    views[v] = r;
    have[v] = 1;
    return r;
  }

  CopyDesc copy_desc(const Shape& s, const View& src, const View& dst) {
    CopyDesc d;
    d.rank = s.rank();
    for (int i = 0; i < d.rank; ++i) {
      d.dims[i] = s.dims[i];
      d.sst[i] = src.strides[i];
      d.dst[i] = dst.strides[i];
    }
    return d;
  }

  void emit_copy(const Shape& s, const View& src, const View& dst, const char* why) {
    const CopyDesc d = copy_desc(s, src, dst);
    const int eb = dtype_size(s.dtype);
    const int dt = s.dtype;
    add_step(fmt("strided_copy %s %s", s.str().c_str(), why), {src.slot}, {dst.slot},
             [=](ExecState& st, GHipError* e) {
               return launch_strided_copy(eb, st.ptr(src, dt), st.ptr(dst, dt), d, st.stream, e);
             });
  }

  View materialize(const View& src, const Shape& s, const char* why = "(materialise)") {
    if (failed) return bad();
    if (src.contiguous(s)) {
      View r = src;
      r.strides = contiguous_strides(s.dims);
      return r;
    }
    View dst = fresh(s);
    emit_copy(s, src, dst, why);
    return dst;
  }

  // Permuted view helper: result dims[i] = dims[perm[i]].
  static View permute(const View& v, const std::vector<int64_t>& perm) {
    View r = v;
    for (size_t i = 0; i < perm.size(); ++i) r.strides[i] = v.strides[perm[i]];
    return r;
  }
  static Shape permute_shape(const Shape& s, const std::vector<int64_t>& perm) {
    Shape r = s;
    for (size_t i = 0; i < perm.size(); ++i) r.dims[i] = s.dims[perm[i]];
    return r;
  }
  static std::vector<int64_t> inverse(const std::vector<int64_t>& p) {
    std::vector<int64_t> q(p.size());
    for (size_t i = 0; i < p.size(); ++i) q[p[i]] = static_cast<int64_t>(i);
    return q;
  }

  // ------------------------------------------------------------------ row kernels
  struct Vec {
    bool present = false;
    View view;
    Shape shape;
  };
  Vec vec_of(int v) {
    Vec r;
    if (v < 0) return r;
    r.present = true;
    r.view = get(v);
    r.shape = N[v].shape;
    return r;
  }
  View emit_rows(int op, const Shape& xs, const View& xv, const Vec& gamma, const Vec& beta, double eps,
                 const std::string& why) {
    const int r = xs.rank();
    const int64_t n = r ? xs.dims[r - 1] : 1;
    const int64_t rows = n ? xs.size() / n : 0;
    const int dt = xs.dtype;
    if (!row_dtype(dt))
      return fail(GHIP_ERR_UNSUPPORTED, fmt("row kernels take float32 / bfloat16 / float16, got %s", dtype_name(dt)).c_str());
    View x = materialize(xv, xs);
    View g, b;
    std::vector<int> rd{x.slot};
    if (gamma.present) {
      g = materialize(gamma.view, gamma.shape);
      rd.push_back(g.slot);
    }
    if (beta.present) {
      b = materialize(beta.view, beta.shape);
      rd.push_back(b.slot);
    }
    if (failed) return bad();
    View y = fresh(xs);
    const bool hg = gamma.present, hb = beta.present;
    const float fe = static_cast<float>(eps);
    static const char* names[] = {"softmax_rows", "log_softmax_rows", "rmsnorm_rows", "layernorm_rows"};
    add_step(fmt("%s %s rows=%lld n=%lld%s%s %s", names[op], dtype_name(dt), (long long)rows, (long long)n,
                 hg ? " +gamma" : "", hb ? " +beta" : "", why.c_str()),
             rd, {y.slot}, [=](ExecState& st, GHipError* e) {
               const void* xp = st.ptr(x, dt);
               void* yp = st.ptr(y, dt);
               const void* gp = hg ? st.ptr(g, dt) : nullptr;
               const void* bp = hb ? st.ptr(b, dt) : nullptr;
               switch (op) {
                 case 0: return ghip_softmax_rows(dt, xp, yp, rows, n, 0, st.stream, e);
                 case 1: return ghip_softmax_rows(dt, xp, yp, rows, n, 1, st.stream, e);
                 case 2: return ghip_rmsnorm_rows(dt, xp, gp, yp, rows, n, fe, st.stream, e);
                 default: return ghip_layernorm_rows(dt, xp, gp, bp, yp, rows, n, fe, st.stream, e);
               }
             });
    return y;
  }

  View emit_fusion(int v) {
    const Fusion& f = fusion[v];
    const Shape& xs = N[f.x].shape;
    View xv = get(f.x);
    if (failed) return bad();
    switch (f.kind) {
      case Fusion::RmsNorm: {
        // gamma must be contiguous [n] data.
        return emit_rows(2, xs, xv, vec_of(f.gamma), Vec{}, f.eps, "(fused primitive RMSNorm chain)");
      }
      case Fusion::Softmax: return emit_rows(0, xs, xv, Vec{}, Vec{}, 0, "(fused primitive softmax chain)");
      case Fusion::LogSoftmax: return emit_rows(1, xs, xv, Vec{}, Vec{}, 0, "(fused primitive log-softmax chain)");
      case Fusion::LayerNorm:
        return emit_rows(3, xs, xv, vec_of(f.gamma), vec_of(f.beta), f.eps, "(fused primitive LayerNorm chain)");
      default: return fail(GHIP_ERR_STATE, "unknown fusion");
    }
  }

  // Softmax (op 0) or LayerNorm (op 3) over axis `axis` of x, which is not the
  // last one: the column kernels on x read as dense [outer, n, inner], writing y in
  // x's own layout (no transposing copy of x, none of y).
  View emit_cols(int op, const Shape& xs, const View& xv, int axis, const Vec& gamma, const Vec& beta,
                 double eps, const char* why) {
    const int dt = xs.dtype;
    if (!row_dtype(dt))
      return fail(GHIP_ERR_UNSUPPORTED, fmt("row kernels take float32 / bfloat16 / float16, got %s", dtype_name(dt)).c_str());
    int64_t outer = 1, inner = 1;
    for (int i = 0; i < axis; ++i) outer *= xs.dims[i];
    for (int i = axis + 1; i < xs.rank(); ++i) inner *= xs.dims[i];
    const int64_t n = xs.dims[axis];
    View x = materialize(xv, xs);
    View g, b;
    std::vector<int> rd{x.slot};
    if (gamma.present) {
      g = materialize(gamma.view, gamma.shape);
      rd.push_back(g.slot);
    }
    if (beta.present) {
      b = materialize(beta.view, beta.shape);
      rd.push_back(b.slot);
    }
    if (failed) return bad();
    View y = fresh(xs);
    const bool hg = gamma.present, hb = beta.present;
    const float fe = static_cast<float>(eps);
    add_step(fmt("%s %s outer=%lld n=%lld inner=%lld%s%s %s", op == 0 ? "softmax_cols" : "layernorm_cols",
                 dtype_name(dt), (long long)outer, (long long)n, (long long)inner, hg ? " +gamma" : "",
                 hb ? " +beta" : "", why),
             rd, {y.slot}, [=](ExecState& st, GHipError* e) {
               const void* xp = st.ptr(x, dt);
               void* yp = st.ptr(y, dt);
               if (op == 0) return ghip_softmax_cols(dt, xp, yp, outer, n, inner, 0, st.stream, e);
               return ghip_layernorm_cols(dt, xp, hg ? st.ptr(g, dt) : nullptr, hb ? st.ptr(b, dt) : nullptr, yp,
                                          outer, n, inner, fe, st.stream, e);
             });
    return y;
  }

  View emit_softmax(int v) {
    const Node& n = N[v];
    const Shape& xs = N[n.in[0]].shape;
    View xv = get(n.in[0]);
    if (failed) return bad();
    const int r = xs.rank(), axis = static_cast<int>(n.i0);
    if (axis == r - 1) return emit_rows(0, xs, xv, Vec{}, Vec{}, 0, "(FusedSoftmax)");
    return emit_cols(0, xs, xv, axis, Vec{}, Vec{}, 0, "(FusedSoftmax over a middle axis)");
  }

  View emit_layernorm(int v) {
    const Node n = N[v];
    const Shape xs = N[n.in[0]].shape;
    View xv = get(n.in[0]);
    if (failed) return bad();
    const int r = xs.rank();
    const int k = static_cast<int>(n.a0.size());
    bool trailing = true;
    for (int i = 0; i < k; ++i) trailing = trailing && n.a0[i] == r - k + i;
    if (k == 1 && !trailing) {
      // One normalized axis before the last: the column kernel, when gamma / beta
      // hold exactly that axis's n values (shape [n], or x's rank with every other
      // axis of size 1).
      const int ax = static_cast<int>(n.a0[0]);
      auto along_axis = [&](int w) {
        if (w < 0) return true;
        const Shape& gs = N[w].shape;
        if (gs.size() != xs.dims[ax]) return false;
        return gs.rank() == 1 || (gs.rank() == r && gs.dims[ax] == xs.dims[ax]);
      };
      if (along_axis(n.in[1]) && along_axis(n.in[2]))
        return emit_cols(3, xs, xv, ax, vec_of(n.in[1]), vec_of(n.in[2]), n.f0, "(FusedLayerNorm over a middle axis)");
    }
    std::vector<int64_t> perm;
    for (int i = 0; i < r; ++i)
      if (std::find(n.a0.begin(), n.a0.end(), i) == n.a0.end()) perm.push_back(i);
    for (auto a : n.a0) perm.push_back(a);
    // Collapse to [rows, prod(normalized)] and run the row kernel.
    Shape ps = permute_shape(xs, perm);
    View pv = trailing ? xv : permute(xv, perm);
    View x2 = materialize(pv, ps);
    if (failed) return bad();
    Shape flat = ps;
    int64_t nn = 1;
    for (int i = r - k; i < r; ++i) nn *= ps.dims[i];
    flat.dims.assign(ps.dims.begin(), ps.dims.begin() + (r - k));
    flat.dims.push_back(nn);
    View fv = contig(x2.slot, flat);
    fv.offset = x2.offset;
    // gamma / beta of x's rank with non-normalized axes of size 1 follow x's
    // permutation; lower-rank ones are already in normalized-axes order.
    Vec gb[2] = {vec_of(n.in[1]), vec_of(n.in[2])};
    for (int w = 0; w < 2; ++w) {
      if (!gb[w].present || trailing || gb[w].shape.rank() != r) continue;
      gb[w].view = materialize(permute(gb[w].view, perm), permute_shape(gb[w].shape, perm));
      gb[w].shape = permute_shape(gb[w].shape, perm);
    }
    if (failed) return bad();
    View y = emit_rows(3, flat, fv, gb[0], gb[1], n.f0, "(FusedLayerNorm)");
    if (failed) return bad();
    View yv = contig(y.slot, ps);
    return trailing ? yv : permute(yv, inverse(perm));
  }

  // ------------------------------------------------------------------ iota / concat / reduce / arg
  View emit_iota(int v) {
    const Node& n = N[v];
    const int dt = n.shape.dtype;
    if (dt != GHIP_DTYPE_INT32 && dt != GHIP_DTYPE_INT64 && dt != GHIP_DTYPE_FLOAT32 && dt != GHIP_DTYPE_BFLOAT16)
      return emit_cluster(-1, v);  // generated kernel handles the other dtypes
    View y = fresh(n.shape);
    int64_t outer = 1, inner = 1;
    const int ax = static_cast<int>(n.i0);
    for (int i = 0; i < ax; ++i) outer *= n.shape.dims[i];
    for (int i = ax + 1; i < n.shape.rank(); ++i) inner *= n.shape.dims[i];
    const int64_t len = n.shape.dims[ax];
    add_step(fmt("iota %s axis=%d", n.shape.str().c_str(), ax), {}, {y.slot},
             [=](ExecState& st, GHipError* e) { return ghip_iota(dt, st.ptr(y, dt), outer, len, inner, st.stream, e); });
    return y;
  }

  View emit_concat(int v) {
    const Node& n = N[v];
    View y = fresh(n.shape);
    int64_t off = 0;
    const int ax = static_cast<int>(n.i0);
    for (int o : n.in) {
      View s = get(o);
      if (failed) return bad();
      View d = y;
      d.offset = off * y.strides[ax];
      emit_copy(N[o].shape, s, d, "(Concatenate)");
      off += N[o].shape.dims[ax];
    }
    return y;
  }

  View emit_reduce(int v) {
    if (reduce_prod[v] >= 0) return emit_reduce_fused(v, reduce_prod[v], -1);
    const Node& n = N[v];
    const Shape& xs = N[n.in[0]].shape;
    View x = get(n.in[0]);
    if (failed) return bad();
    ReduceDesc d;
    for (int i = 0; i < xs.rank(); ++i) {
      if (std::find(n.a0.begin(), n.a0.end(), i) != n.a0.end()) {
        d.rdims[d.rrank] = xs.dims[i];
        d.rst[d.rrank++] = x.strides[i];
      } else {
        d.odims[d.orank] = xs.dims[i];
        d.ost[d.orank++] = x.strides[i];
      }
    }
    if (d.orank == 0) {  // scalar output
      d.odims[0] = 1;
      d.ost[0] = 0;
      d.orank = 1;
    }
    if (d.rrank == 0) {
      d.rdims[0] = 1;
      d.rst[0] = 0;
      d.rrank = 1;
    }
    View y = fresh(n.shape);
    const int dt = xs.dtype, op = n.sub;
    static const char* names[] = {"sum", "product", "max", "min"};
    add_step(fmt("reduce_%s %s -> %s", names[op], xs.str().c_str(), n.shape.str().c_str()), {x.slot}, {y.slot},
             [=](ExecState& st, GHipError* e) { return launch_reduce(dt, op, st.ptr(x, dt), d, st.ptr(y, dt), st.stream, e); });
    return y;
  }

  View emit_argminmax(int v) {
    const Node& n = N[v];
    const Shape& xs = N[n.in[0]].shape;
    if (xs.dtype == GHIP_DTYPE_BOOL || xs.dtype == GHIP_DTYPE_FLOAT64)
      return fail(GHIP_ERR_UNSUPPORTED, "ArgMinMax lowers float32 / bfloat16 / float16 and integer inputs");
    View x = materialize(get(n.in[0]), xs);
    if (failed) return bad();
    const int ax = static_cast<int>(n.i0);
    int64_t outer = 1, inner = 1;
    for (int i = 0; i < ax; ++i) outer *= xs.dims[i];
    for (int i = ax + 1; i < xs.rank(); ++i) inner *= xs.dims[i];
    const int64_t len = xs.dims[ax];
    View y = fresh(n.shape);
    const int dt = xs.dtype, odt = n.shape.dtype, is_min = static_cast<int>(n.i1);
    add_step(fmt("arg%s %s axis=%d", is_min ? "min" : "max", xs.str().c_str(), ax), {x.slot}, {y.slot},
             [=](ExecState& st, GHipError* e) {
               return ghip_argminmax(dt, st.ptr(x, dt), outer, len, inner, is_min, odt, st.ptr(y, odt), st.stream, e);
             });
    return y;
  }

  // ------------------------------------------------------------------ control flow
  // Call / While / If run their compiled functions from one step, on the host,
  // between launches on the stream (executable.go:112-577 orchestrates the same
  // way); every value stays in device memory and a loop or branch reads back one
  // bool per decision.  Inputs are passed as contiguous views, outputs land in
  // fresh contiguous slots.
  std::map<int, std::vector<View>> cf_out;  // control-flow node -> output views
  static constexpr long kMaxWhileIterations = 1000000;  // executable.go:269

  // Comparator / scalar closure as device code: statements and the result
  // expression, its params named p<i>, its captures c<i>.  False when it holds
  // anything but scalar elementwise ops and constants.
  bool scalar_fn_source(std::string* body, std::string* result) {
    std::vector<char> lv(N.size(), 0);
    std::vector<int> stack(fn->outputs.begin(), fn->outputs.end());
    while (!stack.empty()) {
      const int u = stack.back();
      stack.pop_back();
      if (u < 0 || lv[u]) continue;
      lv[u] = 1;
      for (int o : N[u].in) stack.push_back(o);
    }
    std::map<int, std::string> expr;
    std::ostringstream b;
    for (int u = 0; u < static_cast<int>(N.size()); ++u) {
      if (!lv[u]) continue;
      const Node& n = N[u];
      if (n.shape.rank() != 0) return false;
      switch (n.kind) {
        case Kind::Param: expr[u] = "p" + std::to_string(n.i0); break;
        case Kind::Capture: expr[u] = "c" + std::to_string(n.i0); break;
        case Kind::Const: expr[u] = literal(n.shape.dtype, const_as_double(n, 0)); break;
        case Kind::Reshape: case Kind::Broadcast: expr[u] = expr[n.in[0]]; break;
        default:
          if (!is_elementwise(n.kind)) return false;
          b << member_stmt(u, expr, "t" + std::to_string(u));
      }
    }
    *body = b.str();
    *result = expr[fn->outputs[0]];
    return true;
  }

  // Sort: one workgroup per row along the axis; the row's keys in LDS, a bitonic
  // network over an index array ordered by the comparator, ties by index (so the
  // order is total and the sort stable).
  void emit_sort(int v) {
    const Node n = N[v];
    GHipFunction* cf = n.fns[0];
    const int nin = static_cast<int>(n.i2), axis = static_cast<int>(n.i0);
    const Shape s0 = n.outs[0];
    int64_t outer = 1, inner = 1;
    for (int d = 0; d < axis; ++d) outer *= s0.dims[d];
    for (int d = axis + 1; d < s0.rank(); ++d) inner *= s0.dims[d];
    const int64_t L = s0.dims[axis];
    Plan cplan;
    Lowerer C(be, cf, &cplan, err);
    std::string cbody, cres;
    if (!C.scalar_fn_source(&cbody, &cres)) {
      fail(GHIP_ERR_UNSUPPORTED, "Sort: the comparator may only use scalar elementwise ops, constants and captured scalars");
      return;
    }
    for (size_t k = nin; k < n.in.size(); ++k)
      if (N[n.in[k]].shape.rank() != 0) {
        fail(GHIP_ERR_UNSUPPORTED, "Sort: the comparator may only capture scalars");
        return;
      }
    int64_t P = 2;
    while (P < L) P <<= 1;
    int64_t lds = P * 4;
    for (int i = 0; i < nin; ++i) lds += L * dtype_size(n.outs[i].dtype);
    if (lds > 150 * 1024) {
      emit_sort_global(v, cbody, cres, outer, inner, L, P);
      return;
    }
    const int NT = static_cast<int>(std::min<int64_t>(1024, std::max<int64_t>(64, P / 2)));
    std::ostringstream src;
    src << kRtcPrelude << "extern \"C\" __global__ void __launch_bounds__(" << NT << ") sort_rows(\n";
    for (int i = 0; i < nin; ++i) src << "    const void* __restrict__ in" << i << ",\n";
    for (int i = 0; i < nin; ++i) src << "    void* __restrict__ out" << i << ",\n";
    for (size_t k = nin; k < n.in.size(); ++k) src << "    const void* __restrict__ cap" << (k - nin) << ",\n";
    src << "    long long inner) {\n";
    for (int i = 0; i < nin; ++i) src << "  __shared__ " << stype(n.outs[i].dtype) << " k" << i << "[" << L << "];\n";
    src << "  __shared__ int ix[" << P << "];\n"
        << "  const long long row = blockIdx.x, o = row / inner, j = row % inner;\n"
        << "  const long long base = o * " << L << "LL * inner + j;\n"
        << "  for (int k = threadIdx.x; k < " << L << "; k += " << NT << ") {\n";
    for (int i = 0; i < nin; ++i)
      src << "    k" << i << "[k] = ((const " << stype(n.outs[i].dtype) << "*)in" << i << ")[base + k * inner];\n";
    src << "  }\n  for (int k = threadIdx.x; k < " << P << "; k += " << NT << ") ix[k] = k;\n";
    for (size_t k = nin; k < n.in.size(); ++k) {
      const int dt = N[n.in[k]].shape.dtype;
      src << "  const " << ctype(dt) << " c" << (k - nin) << " = "
          << load_expr(dt, "((const " + stype(dt) + "*)cap" + std::to_string(k - nin) + ")[0]") << ";\n";
    }
    src << "  __syncthreads();\n"
        << "  auto cmp = [&](int a, int b) -> bool {\n";
    for (int i = 0; i < nin; ++i) {
      const int dt = n.outs[i].dtype;
      src << "    const " << ctype(dt) << " p" << 2 * i << " = " << load_expr(dt, "k" + std::to_string(i) + "[a]") << ";\n"
          << "    const " << ctype(dt) << " p" << 2 * i + 1 << " = " << load_expr(dt, "k" + std::to_string(i) + "[b]") << ";\n";
    }
    src << cbody << "    return " << cres << ";\n  };\n"
        << "  auto lt = [&](int a, int b) -> bool {\n"
        << "    if (a >= " << L << ") return false;\n    if (b >= " << L << ") return true;\n"
        << "    if (cmp(a, b)) return true;\n    if (cmp(b, a)) return false;\n    return a < b;\n  };\n"
        << "  for (int k = 2; k <= " << P << "; k <<= 1)\n"
        << "    for (int jj = k >> 1; jj > 0; jj >>= 1) {\n"
        << "      for (int t = threadIdx.x; t < " << P / 2 << "; t += " << NT << ") {\n"
        << "        const int a = ((t & ~(jj - 1)) << 1) | (t & (jj - 1)), b = a + jj;\n"
        << "        const int xa = ix[a], xb = ix[b];\n"
        << "        if ((a & k) == 0 ? lt(xb, xa) : lt(xa, xb)) { ix[a] = xb; ix[b] = xa; }\n"
        << "      }\n      __syncthreads();\n    }\n"
        << "  for (int k = threadIdx.x; k < " << L << "; k += " << NT << ") {\n    const int s = ix[k];\n";
    for (int i = 0; i < nin; ++i)
      src << "    ((" << stype(n.outs[i].dtype) << "*)out" << i << ")[base + k * inner] = k" << i << "[s];\n";
    src << "  }\n}\n";
    RtcKernel kern;
    if (rtc_get(be, src.str(), "sort_rows", &kern, err) != GHIP_OK) {
      failed = true;
      return;
    }
    std::vector<View> ins, outs;
    std::vector<int> idt, odt, rd, wr;
    for (int o : n.in) {
      View w = materialize(get(o), N[o].shape, "(Sort input)");
      if (failed) return;
      ins.push_back(w);
      idt.push_back(N[o].shape.dtype);
      rd.push_back(w.slot);
    }
    for (const Shape& sh : n.outs) {
      outs.push_back(fresh(sh));
      odt.push_back(sh.dtype);
      wr.push_back(outs.back().slot);
    }
    cf_out[v] = outs;
    const int64_t rows = outer * inner;
    add_step(fmt("sort_rows %s axis=%d inputs=%d (comparator compiled in; bitonic in LDS, stable)", s0.str().c_str(), axis,
                 nin),
             rd, wr, [=](ExecState& st, GHipError* e) -> int {
               if (rows == 0 || L == 0) return GHIP_OK;
               std::vector<void*> ptr;
               for (int i = 0; i < nin; ++i) ptr.push_back(st.ptr(ins[i], idt[i]));
               for (int i = 0; i < nin; ++i) ptr.push_back(st.ptr(outs[i], odt[i]));
               for (size_t k = nin; k < ins.size(); ++k) ptr.push_back(st.ptr(ins[k], idt[k]));
               long long in_ = inner;
               std::vector<void*> args;
               for (auto& p : ptr) args.push_back(&p);
               args.push_back(&in_);
               int64_t done = 0;
               while (done < rows) {  // grid x <= 2^31 - 1 per launch
                 const int64_t g = std::min<int64_t>(rows - done, 1 << 30);
                 if (done) return set_error(e, GHIP_ERR_UNSUPPORTED, "Sort: more than 2^30 rows");
                 const hipError_t h = hipModuleLaunchKernel(kern.func, static_cast<unsigned>(g), 1, 1, NT, 1, 1, 0,
                                                            st.stream, args.data(), nullptr);
                 if (h != hipSuccess) return check_hip(h, e, "sort launch");
                 done += g;
               }
               return GHIP_OK;
             });
  }

  // Sort of rows too long for one workgroup's LDS: the same bitonic network over an
  // index array, held per row in an arena scratch buffer.  One workgroup per row;
  // each chunk of CH indices is sorted in LDS first, then for every larger stage the
  // exchanges across chunks run in global memory and the ones inside a chunk in LDS.
  // The comparator reads the keys from the input rows (no copy).  The network, the
  // tie rule (index order) and so the result are those of the LDS kernel.
  void emit_sort_global(int v, const std::string& cbody, const std::string& cres, int64_t outer, int64_t inner,
                        int64_t L, int64_t P) {
    const Node n = N[v];
    const int nin = static_cast<int>(n.i2), axis = static_cast<int>(n.i0);
    const Shape s0 = n.outs[0];
    const int64_t rows = outer * inner;
    if (L > (int64_t{1} << 30)) {
      fail(GHIP_ERR_UNSUPPORTED, "Sort: rows longer than 2^30 elements");
      return;
    }
    const int64_t CH = std::min<int64_t>(P, 16384);  // indices per LDS chunk (64 KiB)
    const int NT = 1024;
    // Rows per launch: index scratch of at most 256 MiB.
    const int64_t batch = std::max<int64_t>(1, std::min<int64_t>(rows, (int64_t{256} << 20) / (P * 4)));
    std::ostringstream src;
    src << kRtcPrelude << "extern \"C\" __global__ void __launch_bounds__(" << NT << ") sort_rows_global(\n";
    for (int i = 0; i < nin; ++i) src << "    const void* __restrict__ in" << i << ",\n";
    for (int i = 0; i < nin; ++i) src << "    void* __restrict__ out" << i << ",\n";
    for (size_t k = nin; k < n.in.size(); ++k) src << "    const void* __restrict__ cap" << (k - nin) << ",\n";
    src << "    int* __restrict__ ixg, long long inner, long long row0) {\n"
        << "  __shared__ int ix[" << CH << "];\n"
        << "  const long long row = row0 + blockIdx.x, o = row / inner, j = row % inner;\n"
        << "  const long long base = o * " << L << "LL * inner + j;\n"
        << "  int* g = ixg + (long long)blockIdx.x * " << P << "LL;\n";
    for (size_t k = nin; k < n.in.size(); ++k) {
      const int dt = N[n.in[k]].shape.dtype;
      src << "  const " << ctype(dt) << " c" << (k - nin) << " = "
          << load_expr(dt, "((const " + stype(dt) + "*)cap" + std::to_string(k - nin) + ")[0]") << ";\n";
    }
    src << "  auto cmp = [&](int a, int b) -> bool {\n";
    for (int i = 0; i < nin; ++i) {
      const int dt = n.outs[i].dtype;
      const std::string arr = "((const " + stype(dt) + "*)in" + std::to_string(i) + ")";
      src << "    const " << ctype(dt) << " p" << 2 * i << " = " << load_expr(dt, arr + "[base + (long long)a * inner]")
          << ";\n"
          << "    const " << ctype(dt) << " p" << 2 * i + 1 << " = " << load_expr(dt, arr + "[base + (long long)b * inner]")
          << ";\n";
    }
    src << cbody << "    return " << cres << ";\n  };\n"
        << "  auto lt = [&](int a, int b) -> bool {\n"
        << "    if (a >= " << L << ") return false;\n    if (b >= " << L << ") return true;\n"
        << "    if (cmp(a, b)) return true;\n    if (cmp(b, a)) return false;\n    return a < b;\n  };\n"
        // exchange of the pair at positions (a, a + jj) of stage k, a taken in the whole row
        << "  auto local = [&](int c, int k, int jtop) {\n"  // stages jj = jtop .. 1 of stage k inside chunk c (in LDS)
        << "    for (int jj = jtop; jj > 0; jj >>= 1) {\n"
        << "      for (int t = threadIdx.x; t < " << CH / 2 << "; t += " << NT << ") {\n"
        << "        const int a = ((t & ~(jj - 1)) << 1) | (t & (jj - 1)), b = a + jj;\n"
        << "        const int ga = c * " << CH << " + a;\n"
        << "        const int xa = ix[a], xb = ix[b];\n"
        << "        if ((ga & k) == 0 ? lt(xb, xa) : lt(xa, xb)) { ix[a] = xb; ix[b] = xa; }\n"
        << "      }\n      __syncthreads();\n    }\n  };\n"
        << "  for (int c = 0; c < " << P / CH << "; ++c) {\n"
        << "    for (int t = threadIdx.x; t < " << CH << "; t += " << NT << ") ix[t] = c * " << CH << " + t;\n"
        << "    __syncthreads();\n"
        << "    for (int k = 2; k <= " << CH << "; k <<= 1) local(c, k, k >> 1);\n"
        << "    for (int t = threadIdx.x; t < " << CH << "; t += " << NT << ") g[c * " << CH << " + t] = ix[t];\n"
        << "    __syncthreads();\n  }\n"
        << "  for (int k = " << 2 * CH << "; k <= " << P << "; k <<= 1) {\n"
        << "    for (int jj = k >> 1; jj >= " << CH << "; jj >>= 1) {\n"
        << "      for (int t = threadIdx.x; t < " << P / 2 << "; t += " << NT << ") {\n"
        << "        const int a = ((t & ~(jj - 1)) << 1) | (t & (jj - 1)), b = a + jj;\n"
        << "        const int xa = g[a], xb = g[b];\n"
        << "        if ((a & k) == 0 ? lt(xb, xa) : lt(xa, xb)) { g[a] = xb; g[b] = xa; }\n"
        << "      }\n      __syncthreads();\n    }\n"
        << "    for (int c = 0; c < " << P / CH << "; ++c) {\n"
        << "      for (int t = threadIdx.x; t < " << CH << "; t += " << NT << ") ix[t] = g[c * " << CH << " + t];\n"
        << "      __syncthreads();\n"
        << "      local(c, k, " << CH / 2 << ");\n"
        << "      for (int t = threadIdx.x; t < " << CH << "; t += " << NT << ") g[c * " << CH << " + t] = ix[t];\n"
        << "      __syncthreads();\n    }\n  }\n"
        << "  for (int t = threadIdx.x; t < " << L << "; t += " << NT << ") {\n"
        // padding indices sort last, so g[t] < L; the clamp only keeps reads in bounds
        << "    const long long s = g[t] < " << L << " ? g[t] : " << L - 1 << ";\n";
    for (int i = 0; i < nin; ++i)
      src << "    ((" << stype(n.outs[i].dtype) << "*)out" << i << ")[base + t * inner] = ((const "
          << stype(n.outs[i].dtype) << "*)in" << i << ")[base + s * inner];\n";
    src << "  }\n}\n";
    RtcKernel kern;
    if (rtc_get(be, src.str(), "sort_rows_global", &kern, err) != GHIP_OK) {
      failed = true;
      return;
    }
    std::vector<View> ins, outs;
    std::vector<int> idt, odt, rd, wr;
    for (int o : n.in) {
      View w = materialize(get(o), N[o].shape, "(Sort input)");
      if (failed) return;
      ins.push_back(w);
      idt.push_back(N[o].shape.dtype);
      rd.push_back(w.slot);
    }
    for (const Shape& sh : n.outs) {
      outs.push_back(fresh(sh));
      odt.push_back(sh.dtype);
      wr.push_back(outs.back().slot);
    }
    Shape ish;
    ish.dtype = GHIP_DTYPE_INT32;
    ish.dims = {batch, P};
    const View scratch = fresh(ish);
    wr.push_back(scratch.slot);
    cf_out[v] = outs;
    add_step(fmt("sort_rows_global %s axis=%d inputs=%d (comparator compiled in; bitonic over an index array in "
                 "global memory, chunks of %lld in LDS, stable)",
                 s0.str().c_str(), axis, nin, static_cast<long long>(CH)),
             rd, wr, [=](ExecState& st, GHipError* e) -> int {
               if (rows == 0 || L == 0) return GHIP_OK;
               std::vector<void*> ptr;
               for (int i = 0; i < nin; ++i) ptr.push_back(st.ptr(ins[i], idt[i]));
               for (int i = 0; i < nin; ++i) ptr.push_back(st.ptr(outs[i], odt[i]));
               for (size_t k = nin; k < ins.size(); ++k) ptr.push_back(st.ptr(ins[k], idt[k]));
               void* ixg = st.ptr(scratch, GHIP_DTYPE_INT32);
               long long in_ = inner, r0 = 0;
               std::vector<void*> args;
               for (auto& q : ptr) args.push_back(&q);
               args.push_back(&ixg);
               args.push_back(&in_);
               args.push_back(&r0);
               for (r0 = 0; r0 < rows; r0 += batch) {
                 const int64_t gsz = std::min<int64_t>(rows - r0, batch);
                 const hipError_t h = hipModuleLaunchKernel(kern.func, static_cast<unsigned>(gsz), 1, 1, NT, 1, 1, 0,
                                                            st.stream, args.data(), nullptr);
                 if (h != hipSuccess) return check_hip(h, e, "sort launch");
               }
               return GHIP_OK;
             });
  }

  void emit_control_flow(int v) {
    const Node n = N[v];
    if (n.kind == Kind::Sort) {
      emit_sort(v);
      return;
    }
    std::vector<GHipExecutable*> subs;
    for (GHipFunction* g : n.fns) {
      auto ex = compile_function(be, g, err);
      if (!ex) {
        failed = true;
        return;
      }
      plan->subs.push_back(ex);
      subs.push_back(ex.get());
    }
    std::vector<View> ins;
    std::vector<int> idt, rd, wr;
    std::vector<size_t> ibytes;
    for (int o : n.in) {
      View w = materialize(get(o), N[o].shape, "(control-flow input)");
      if (failed) return;
      ins.push_back(w);
      idt.push_back(N[o].shape.dtype);
      ibytes.push_back(N[o].shape.bytes());
      rd.push_back(w.slot);
    }
    std::vector<View> outs;
    std::vector<int> odt;
    std::vector<size_t> obytes;
    for (const Shape& s : n.outs) {
      outs.push_back(fresh(s));
      odt.push_back(s.dtype);
      obytes.push_back(s.bytes());
      wr.push_back(outs.back().slot);
    }
    cf_out[v] = outs;
    auto ptrs = [](ExecState& st, const std::vector<View>& vs, const std::vector<int>& dts, size_t from, size_t to) {
      std::vector<void*> p;
      for (size_t i = from; i < to; ++i) p.push_back(st.ptr(vs[i], dts[i]));
      return p;
    };
    // Reads one bool from device memory (the only host round trip per decision).
    auto read_bool = [](const void* p, hipStream_t s, bool* out, GHipError* e) -> int {
      uint8_t h = 0;
      hipError_t he = hipMemcpyAsync(&h, p, 1, hipMemcpyDeviceToHost, s);
      if (he == hipSuccess) he = hipStreamSynchronize(s);
      if (he != hipSuccess) return check_hip(he, e, "control flow: reading the predicate");
      *out = h != 0;
      return GHIP_OK;
    };
    const size_t nin = ins.size();
    if (n.kind == Kind::Call) {
      GHipExecutable* sub = subs[0];
      add_step(fmt("call %s (%zu inputs, %zu outputs)", n.fns[0]->name.c_str(), nin, outs.size()), rd, wr,
               [=](ExecState& st, GHipError* e) {
                 auto in = ptrs(st, ins, idt, 0, nin);
                 auto out = ptrs(st, outs, odt, 0, outs.size());
                 return run_plan(sub, in.data(), out.data(), e);
               });
      return;
    }
    if (n.kind == Kind::If) {
      const size_t ntc = static_cast<size_t>(n.i0);
      GHipExecutable* tb = subs[0];
      GHipExecutable* fb = subs[1];
      add_step(fmt("if (%zu outputs; branches run from the host after reading the predicate)", outs.size()), rd, wr,
               [=](ExecState& st, GHipError* e) {
                 bool pred = false;
                 int rc = read_bool(st.ptr(ins[0], GHIP_DTYPE_BOOL), st.stream, &pred, e);
                 if (rc != GHIP_OK) return rc;
                 auto in = pred ? ptrs(st, ins, idt, 1, 1 + ntc) : ptrs(st, ins, idt, 1 + ntc, nin);
                 auto out = ptrs(st, outs, odt, 0, outs.size());
                 return run_plan(pred ? tb : fb, in.data(), out.data(), e);
               });
      return;
    }
    if (n.kind == Kind::While) {
      // Speculative batches: cond and body run k iterations ahead on the stream
      // (each iteration's state in its own slot of a ring of kMaxBatch + 1 state
      // sets, each predicate in its own byte), then the k predicates come back in
      // one copy; the state before the first false predicate is the result.  Extra
      // iterations past the exit only compute (every kernel here is bounds-safe:
      // clamped indices, skipped out-of-range windows), and their results are
      // never used.  Batches grow 1, 2, 4, ... up to kMaxBatch, so a loop of N
      // iterations reads back O(log N + N / kMaxBatch) times and runs at most
      // about twice its body launches.  The ring's size is bounded by a byte
      // budget for large states.
      //
      // When cond or body itself runs host-driven steps (a nested While, If or
      // Call, i.e. a plan with sub-plans), an iteration past the exit is not just
      // computation: a nested loop on post-exit state may not terminate, and an
      // error from it would fail a program the sequential loop completes.  Such
      // loops run without speculation: cond, read its predicate, then the body
      // only when it is true.
      const size_t ns = static_cast<size_t>(n.i0), ncc = static_cast<size_t>(n.i1);
      GHipExecutable* cond = subs[0];
      GHipExecutable* body = subs[1];
      const bool speculate = cond->plan.subs.empty() && body->plan.subs.empty();
      size_t state_bytes = 0;
      for (size_t i = 0; i < ns; ++i) state_bytes += n.outs[i].bytes();
      constexpr size_t kRingBudget = size_t{256} << 20;
      int kmax = speculate ? 8 : 1;
      while (kmax > 1 && (static_cast<size_t>(kmax) + 1) * state_bytes > kRingBudget) kmax /= 2;
      std::vector<std::vector<View>> H(kmax + 1);
      for (int r = 0; r <= kmax; ++r)
        for (size_t i = 0; i < ns; ++i) {
          H[r].push_back(fresh(n.outs[i]));
          wr.push_back(H[r].back().slot);
        }
      Shape bs;
      bs.dtype = GHIP_DTYPE_BOOL;
      bs.dims = {kmax};
      View pv = fresh(bs);
      wr.push_back(pv.slot);
      const std::string desc =
          speculate ? fmt("while (%zu state values; cond and body enqueued in speculative batches of up to %d "
                          "iterations, one predicate read per batch)", ns, kmax)
                    : fmt("while (%zu state values; cond or body runs host-driven control flow, so no "
                          "speculation: one predicate read per iteration, body only when it is true)", ns);
      add_step(desc, rd, wr, [=](ExecState& st, GHipError* e) -> int {
                 std::vector<std::vector<void*>> h(kmax + 1);
                 for (int r = 0; r <= kmax; ++r) h[r] = ptrs(st, H[r], odt, 0, ns);
                 for (size_t i = 0; i < ns; ++i) {
                   const hipError_t he = hipMemcpyAsync(h[0][i], st.ptr(ins[i], idt[i]), ibytes[i],
                                                        hipMemcpyDeviceToDevice, st.stream);
                   if (he != hipSuccess) return check_hip(he, e, "While: initial state");
                 }
                 const std::vector<void*> ccap = ptrs(st, ins, idt, ns, ns + ncc);
                 const std::vector<void*> bcap = ptrs(st, ins, idt, ns + ncc, nin);
                 uint8_t* pp = reinterpret_cast<uint8_t*>(st.ptr(pv, GHIP_DTYPE_BOOL));
                 int base = 0, k = 1, last = -1;
                 if (!speculate) {
                   for (long done = 0; last < 0; ++done) {
                     if (done >= kMaxWhileIterations)
                       return set_error(e, GHIP_ERR_STATE, "While: exceeded maximum iterations (%ld)",
                                        kMaxWhileIterations);
                     const int cur = base, nxt = base ^ 1;
                     std::vector<void*> cin(h[cur]);
                     cin.insert(cin.end(), ccap.begin(), ccap.end());
                     void* p0 = pp;
                     int rc = run_plan(cond, cin.data(), &p0, e);
                     if (rc != GHIP_OK) return rc;
                     bool pred = false;
                     rc = read_bool(pp, st.stream, &pred, e);
                     if (rc != GHIP_OK) return rc;
                     if (!pred) {
                       last = cur;
                       break;
                     }
                     std::vector<void*> bin(h[cur]);
                     bin.insert(bin.end(), bcap.begin(), bcap.end());
                     rc = run_plan(body, bin.data(), h[nxt].data(), e);
                     if (rc != GHIP_OK) return rc;
                     base = nxt;
                   }
                 }
                 for (long done = 0; last < 0;) {
                   if (done >= kMaxWhileIterations)
                     return set_error(e, GHIP_ERR_STATE, "While: exceeded maximum iterations (%ld)", kMaxWhileIterations);
                   for (int j = 0; j < k; ++j) {
                     const int cur = (base + j) % (kmax + 1), nxt = (base + j + 1) % (kmax + 1);
                     std::vector<void*> cin(h[cur]);
                     cin.insert(cin.end(), ccap.begin(), ccap.end());
                     void* pj = pp + j;
                     int rc = run_plan(cond, cin.data(), &pj, e);
                     if (rc != GHIP_OK) return rc;
                     std::vector<void*> bin(h[cur]);
                     bin.insert(bin.end(), bcap.begin(), bcap.end());
                     rc = run_plan(body, bin.data(), h[nxt].data(), e);
                     if (rc != GHIP_OK) return rc;
                   }
                   uint8_t hp[64];
                   hipError_t he = hipMemcpyAsync(hp, pp, static_cast<size_t>(k), hipMemcpyDeviceToHost, st.stream);
                   if (he == hipSuccess) he = hipStreamSynchronize(st.stream);
                   if (he != hipSuccess) return check_hip(he, e, "While: reading the predicates");
                   for (int j = 0; j < k && last < 0; ++j)
                     if (!hp[j]) last = (base + j) % (kmax + 1);
                   if (last < 0) {
                     base = (base + k) % (kmax + 1);
                     done += k;
                     k = k * 2 > kmax ? kmax : k * 2;
                   }
                 }
                 for (size_t i = 0; i < ns; ++i) {
                   const hipError_t he = hipMemcpyAsync(st.ptr(outs[i], odt[i]), h[last][i], obytes[i],
                                                        hipMemcpyDeviceToDevice, st.stream);
                   if (he != hipSuccess) return check_hip(he, e, "While: final state");
                 }
                 return GHIP_OK;
               });
      return;
    }
    fail(GHIP_ERR_UNSUPPORTED, "control flow: unsupported operation");
  }

  // ------------------------------------------------------------------ DynamicSlice / UpdateSlice / Scatter
  // Views of the run-time start scalars in[first..] (read by the kernels).
  bool start_views(const Node& n, int first, std::vector<View>* sv, std::vector<int>* sdt, std::vector<int>* rd) {
    for (size_t k = first; k < n.in.size(); ++k) {
      sv->push_back(get(n.in[k]));
      sdt->push_back(N[n.in[k]].shape.dtype);
      rd->push_back(sv->back().slot);
    }
    return !failed;
  }

  View emit_dyn_slice(int v) {
    const Node n = N[v];
    const Shape os = N[n.in[0]].shape;
    if (os.rank() > kMaxRank) return fail(GHIP_ERR_UNSUPPORTED, "DynamicSlice: rank > 8");
    View src = get(n.in[0]);
    std::vector<View> sv;
    std::vector<int> sdt, rd{src.slot};
    if (failed || !start_views(n, 1, &sv, &sdt, &rd)) return bad();
    View y = fresh(n.shape);
    DynDesc d;
    d.rank = os.rank();
    for (int k = 0; k < d.rank; ++k) {
      d.dims[k] = os.dims[k];
      d.win[k] = n.shape.dims[k];
      d.sst[k] = src.strides[k];
      d.dst[k] = y.strides[k];
    }
    const int dt = os.dtype, eb = dtype_size(dt);
    add_step(fmt("dynamic_slice %s -> %s", os.str().c_str(), n.shape.str().c_str()), rd, {y.slot},
             [=](ExecState& st, GHipError* e) {
               DynDesc dd = d;
               for (int k = 0; k < dd.rank; ++k) {
                 dd.start[k] = st.ptr(sv[k], sdt[k]);
                 dd.sdt[k] = sdt[k];
               }
               return launch_window_copy(eb, st.ptr(src, dt), st.ptr(y, dt), dd, 0, st.stream, e);
             });
    return y;
  }

  View emit_dyn_update(int v) {
    const Node n = N[v];
    const Shape os = n.shape, us = N[n.in[1]].shape;
    if (os.rank() > kMaxRank) return fail(GHIP_ERR_UNSUPPORTED, "DynamicUpdateSlice: rank > 8");
    View op = get(n.in[0]);
    View up = get(n.in[1]);
    std::vector<View> sv;
    std::vector<int> sdt, rd{up.slot};
    if (failed || !start_views(n, 2, &sv, &sdt, &rd)) return bad();
    View y = fresh(os);
    emit_copy(os, op, y, "(DynamicUpdateSlice operand)");
    DynDesc d;
    d.rank = os.rank();
    for (int k = 0; k < d.rank; ++k) {
      d.dims[k] = os.dims[k];
      d.win[k] = us.dims[k];
      d.sst[k] = up.strides[k];
      d.dst[k] = y.strides[k];
    }
    const int dt = os.dtype, eb = dtype_size(dt);
    add_step(fmt("dynamic_update_slice %s <- %s", os.str().c_str(), us.str().c_str()), rd, {y.slot},
             [=](ExecState& st, GHipError* e) {
               DynDesc dd = d;
               for (int k = 0; k < dd.rank; ++k) {
                 dd.start[k] = st.ptr(sv[k], sdt[k]);
                 dd.sdt[k] = sdt[k];
               }
               return launch_window_copy(eb, st.ptr(up, dt), st.ptr(y, dt), dd, 1, st.stream, e);
             });
    return y;
  }

  // ScatterSum in the embedding-gradient form (axis 0 of the operand, one index
  // per update row, whole rows, float data): the deterministic sorted-row path.
  // Returns a view with slot -1 when the scatter is not of that form.
  View emit_scatter_rows(const Node& n, const View& op, const View& ix, const View& up) {
    const Shape os = n.shape, is = N[n.in[1]].shape, us = N[n.in[2]].shape;
    const int dt = os.dtype, r = os.rank(), ur = us.rank(), iva = static_cast<int>(n.i0);
    View none;
    if (n.sub != GHIP_SCATTER_SUM || r < 1) return none;
    if (dt != GHIP_DTYPE_FLOAT32 && dt != GHIP_DTYPE_BFLOAT16 && dt != GHIP_DTYPE_FLOAT16) return none;
    if (is.dtype != GHIP_DTYPE_INT32 && is.dtype != GHIP_DTYPE_INT64) return none;
    if (n.a2 != std::vector<int64_t>{0} || n.a1 != std::vector<int64_t>{0}) return none;
    const int nw = static_cast<int>(n.a0.size()), nb = ur - nw;  // window / scatter dims of updates
    int64_t D = 1;
    for (int k = 0; k < nw; ++k) {
      if (n.a0[k] != nb + k || us.dims[nb + k] != os.dims[1 + k]) return none;  // trailing, whole rows
      D *= os.dims[1 + k];
    }
    std::vector<int64_t> bax, wax, iax;
    for (int k = 0; k < nb; ++k) bax.push_back(k);
    for (int k = nb; k < ur; ++k) wax.push_back(k);
    for (int k = 0; k < is.rank(); ++k)
      if (k != iva) iax.push_back(k);
    int64_t rows = 1, upd_row = 0, dsz = 0, dst_ = 0, isz = 1, ist = 0;
    if (!merge(us, up, bax, &rows, &upd_row) || !merge(us, up, wax, &dsz, &dst_) || !merge(is, ix, iax, &isz, &ist))
      return none;
    if (D > 1 && dst_ != 1) return none;
    if (rows > 1 && upd_row < D) return none;
    if (rows == 0 || rows > kScatterRowsMax || os.dims[0] > kScatterRowsMaxTable) return none;
    View y = fresh(os);
    // A contiguous operand is copied by the launch that sorts (its other
    // workgroups), otherwise by a strided copy first.
    const bool fuse_copy = op.contiguous(os) && os.bytes() % 16 == 0 && op.offset * dtype_size(dt) % 16 == 0;
    if (!fuse_copy) emit_copy(os, op, y, "(Scatter operand)");
    Shape ss;
    ss.dtype = GHIP_DTYPE_INT32;
    ss.dims = {2 * rows + 2};
    View sc = fresh(ss);
    const int64_t V = os.dims[0];
    const int idt = is.dtype;
    std::vector<int> rd{up.slot, ix.slot, sc.slot};
    if (fuse_copy) rd.push_back(op.slot);
    add_step(fmt("scatter_rows_sum %s updates=%s ids=%s (sorted segments, deterministic%s)", os.str().c_str(),
                 us.str().c_str(), is.str().c_str(), fuse_copy ? "; operand copied by the sorting launch" : ""),
             rd, {y.slot, sc.slot}, [=](ExecState& st, GHipError* e) {
               return launch_scatter_rows(dt, st.ptr(up, dt), upd_row, st.ptr(ix, idt), idt, ist, rows, st.ptr(y, dt), V,
                                          D, st.ptr(sc, GHIP_DTYPE_INT32), fuse_copy ? st.ptr(op, dt) : nullptr,
                                          st.stream, e);
             });
    return y;
  }

  View emit_scatter(int v) {
    const Node n = N[v];
    const Shape os = n.shape, is = N[n.in[1]].shape, us = N[n.in[2]].shape;
    if (os.rank() > kMaxRank || us.rank() > kMaxRank || is.rank() > kMaxRank)
      return fail(GHIP_ERR_UNSUPPORTED, "Scatter: rank > 8");
    View op = get(n.in[0]);
    View ix = get(n.in[1]);
    View up = get(n.in[2]);
    if (failed) return bad();
    const int dt = os.dtype, adt = scatter_acc_dtype(dt);
    if (View y = emit_scatter_rows(n, op, ix, up); y.slot >= 0 || failed) return y;
    View y = fresh(os);
    View acc = y;
    CopyDesc cd = copy_desc(os, op, y);
    if (adt != dt) {
      Shape as = os;
      as.dtype = adt;
      acc = fresh(as);
      add_step(fmt("convert %s -> %s (scatter accumulator)", os.str().c_str(), dtype_name(adt)), {op.slot}, {acc.slot},
               [=](ExecState& st, GHipError* e) { return launch_convert(dt, adt, st.ptr(op, dt), st.ptr(acc, adt), cd, st.stream, e); });
    } else {
      emit_copy(os, op, y, "(Scatter operand)");
    }
    ScatterDesc d;
    d.ur = us.rank();
    d.r = os.rank();
    const int iva = static_cast<int>(n.i0);
    std::vector<int64_t> non_inserted;
    for (int k = 0; k < d.r; ++k) {
      d.odims[k] = os.dims[k];
      d.ost[k] = acc.strides[k];
      d.wsize[k] = 1;
      if (std::find(n.a1.begin(), n.a1.end(), k) == n.a1.end()) non_inserted.push_back(k);
    }
    int wi = 0, bi = 0;
    for (int k = 0; k < d.ur; ++k) {
      d.udims[k] = us.dims[k];
      d.ust[k] = up.strides[k];
      d.ibatch_st[k] = 0;
      if (std::find(n.a0.begin(), n.a0.end(), k) != n.a0.end()) {
        const int od = static_cast<int>(non_inserted[wi++]);
        d.uwin_od[k] = od;
        d.wsize[od] = us.dims[k];
      } else {
        if (bi == iva) ++bi;
        d.uwin_od[k] = -1;
        d.ibatch_st[k] = ix.strides[bi++];
      }
    }
    d.nidx = static_cast<int>(n.a2.size());
    d.ivec_st = iva < is.rank() ? ix.strides[iva] : 0;
    for (int k = 0; k < d.nidx; ++k) d.sato[k] = static_cast<int>(n.a2[k]);
    d.idx_dt = is.dtype;
    d.idx_es = dtype_size(is.dtype);
    static const char* mn[] = {"sum", "max", "min"};
    const int mode = n.sub, idt = is.dtype;
    add_step(fmt("scatter_%s %s updates=%s indices=%s", mn[mode], os.str().c_str(), us.str().c_str(), is.str().c_str()),
             {up.slot, ix.slot}, {acc.slot}, [=](ExecState& st, GHipError* e) {
               return launch_scatter(dt, mode, st.ptr(up, dt), st.ptr(ix, idt), st.ptr(acc, adt), d, st.stream, e);
             });
    if (adt != dt) {
      CopyDesc back = copy_desc(os, acc, y);
      add_step(fmt("convert %s -> %s (scatter result)", dtype_name(adt), os.str().c_str()), {acc.slot}, {y.slot},
               [=](ExecState& st, GHipError* e) { return launch_convert(adt, dt, st.ptr(acc, adt), st.ptr(y, dt), back, st.stream, e); });
    }
    return y;
  }

  // ------------------------------------------------------------------ DotGeneral
  // Merges `axes` (in flatten order) of a strided view into one (size, stride).
  static bool merge(const Shape& s, const View& v, const std::vector<int64_t>& axes, int64_t* size, int64_t* stride) {
    int64_t sz = 1, st = 0;
    bool have_st = false;
    // innermost-first
    for (int i = static_cast<int>(axes.size()) - 1; i >= 0; --i) {
      const int64_t a = axes[i], d = s.dims[a];
      if (d == 1) continue;
      if (!have_st) {
        st = v.strides[a];
        have_st = true;
      } else if (v.strides[a] != st * sz) {
        return false;
      }
      sz *= d;
    }
    if (!have_st) st = 0;
    // size-1 dims were skipped: total size
    int64_t total = 1;
    for (auto a : axes) total *= s.dims[a];
    *size = total;
    *stride = st;
    return true;
  }

  // A DotGeneral folded to one batched GEMM: operand views and (batch, M, N, K)
  // sizes with one stride per axis group.
  struct DotPlan {
    View lv, rv;
    int64_t B = 0, sab = 0, sbb = 0, M = 0, sam = 0, K = 0, sak = 0, N = 0, sbn = 0, sbk = 0;
    int nbatch = 0, nlfree = 0;  // output dims: [batch (nbatch), lhs free (nlfree), rhs free]
    std::string how;
  };

  // Folds Dot node v's axis groups into single strides.  Operands whose groups
  // do not fold are materialised in [batch, free, contracting] order, unless
  // allow_copy is false (then returns false with no step emitted).
  bool plan_dot(int v, bool allow_copy, DotPlan* d) {
    const Node& n = N[v];
    const int L = n.in[0], R = n.in[1];
    Shape ls = N[L].shape, rs = N[R].shape;
    View lv = get(L), rv = get(R);
    if (failed) return false;
    std::vector<int64_t> lfree, rfree;
    for (int i = 0; i < ls.rank(); ++i)
      if (std::find(n.a0.begin(), n.a0.end(), i) == n.a0.end() && std::find(n.a1.begin(), n.a1.end(), i) == n.a1.end())
        lfree.push_back(i);
    for (int i = 0; i < rs.rank(); ++i)
      if (std::find(n.a2.begin(), n.a2.end(), i) == n.a2.end() && std::find(n.a3.begin(), n.a3.end(), i) == n.a3.end())
        rfree.push_back(i);
    int64_t B, sab, sbb, M, sam, K, sak, N_, sbn, K2, sbk, B2;
    auto try_merge = [&]() {
      return merge(ls, lv, n.a1, &B, &sab) && merge(ls, lv, lfree, &M, &sam) && merge(ls, lv, n.a0, &K, &sak) &&
             merge(rs, rv, n.a3, &B2, &sbb) && merge(rs, rv, rfree, &N_, &sbn) && merge(rs, rv, n.a2, &K2, &sbk);
    };
    std::string how = "strides folded";
    if (!try_merge()) {
      if (!allow_copy) return false;
      // Materialise each operand in canonical [batch, free, contracting] order.
      std::vector<int64_t> lp(n.a1.begin(), n.a1.end()), rp(n.a3.begin(), n.a3.end());
      lp.insert(lp.end(), lfree.begin(), lfree.end());
      lp.insert(lp.end(), n.a0.begin(), n.a0.end());
      rp.insert(rp.end(), rfree.begin(), rfree.end());
      rp.insert(rp.end(), n.a2.begin(), n.a2.end());
      auto canon = [&](const Shape& s, const View& vw, const std::vector<int64_t>& p) {
        View m = materialize(permute(vw, p), permute_shape(s, p), "(DotGeneral operand to [batch, free, contracting])");
        // re-express as a view of the ORIGINAL axes
        View back = m;
        auto inv = inverse(p);
        for (size_t i = 0; i < p.size(); ++i) back.strides[i] = m.strides[inv[i]];
        return back;
      };
      lv = canon(ls, lv, lp);
      rv = canon(rs, rv, rp);
      if (failed) return false;
      how = "operands materialised";
      if (!try_merge()) {
        fail(GHIP_ERR_STATE, "DotGeneral: stride merge failed after canonicalisation");
        return false;
      }
    }
    if (K != K2 || B != B2) {
      fail(GHIP_ERR_STATE, "DotGeneral: inconsistent sizes");
      return false;
    }
    d->lv = lv;
    d->rv = rv;
    d->B = B; d->sab = sab; d->sbb = sbb; d->M = M; d->sam = sam; d->K = K; d->sak = sak;
    d->N = N_; d->sbn = sbn; d->sbk = sbk;
    d->nbatch = static_cast<int>(n.a1.size());
    d->nlfree = static_cast<int>(lfree.size());
    d->how = how;
    return true;
  }

  // Dots that share Dot v's left operand view, sizes and right-operand strides run
  // as one grouped launch (ghip_gemm_grouped: the Q, K, V projections of an
  // attention block).  A sibling joins when no elementwise cluster uses it (one
  // could absorb it as a GEMM epilogue), its right operand is a leaf or already
  // lowered (lowering it here cannot reach back to v), and it folds without an
  // operand copy.  Returns an empty view when v has no sibling.
  bool group_dots = true;
  View emit_dot_group(int v, const DotPlan& d) {
    const Node& n = N[v];
    const int L = n.in[0];
    const int dt = N[L].shape.dtype, odt = n.shape.dtype;
    if (d.B != 1 || (dt != GHIP_DTYPE_BFLOAT16 && dt != GHIP_DTYPE_FLOAT16)) return View{};
    std::vector<int> grp{v};
    std::vector<DotPlan> plans{d};
    for (int u : users[L]) {
      if (static_cast<int>(grp.size()) == kGemmMaxGroups) break;
      if (u == v || !live[u] || have[u] || N[u].kind != Kind::Dot || fusion[u].kind != Fusion::None) continue;
      const Node& m = N[u];
      if (m.in[0] != L || m.a0 != n.a0 || m.a1 != n.a1 || m.a2 != n.a2 || m.a3 != n.a3 || m.shape.dtype != odt ||
          m.shape.dims != n.shape.dims || N[m.in[1]].shape.dims != N[n.in[1]].shape.dims ||
          N[m.in[1]].shape.dtype != N[n.in[1]].shape.dtype)
        continue;
      bool absorbable = false;
      for (int w : users[u]) absorbable = absorbable || cluster[w] >= 0;
      if (absorbable || std::find(grp.begin(), grp.end(), u) != grp.end()) continue;
      const Kind rk = N[m.in[1]].kind;
      if (!have[m.in[1]] && rk != Kind::Param && rk != Kind::Const && rk != Kind::Capture) continue;
      DotPlan du;
      if (!plan_dot(u, false, &du)) {
        if (failed) return bad();
        continue;
      }
      if (du.lv.slot != d.lv.slot || du.lv.offset != d.lv.offset || du.lv.strides != d.lv.strides ||
          du.sam != d.sam || du.sak != d.sak || du.B != 1 || du.M != d.M || du.N != d.N || du.K != d.K ||
          du.sbk != d.sbk || du.sbn != d.sbn)
        continue;
      grp.push_back(u);
      plans.push_back(du);
    }
    if (grp.size() < 2) return View{};
    const int G = static_cast<int>(grp.size());
    std::vector<View> ys, rvs;
    std::vector<int> rd{d.lv.slot}, wr;
    for (int g = 0; g < G; ++g) {
      ys.push_back(fresh(N[grp[g]].shape));
      rvs.push_back(plans[g].rv);
      rd.push_back(plans[g].rv.slot);
      wr.push_back(ys.back().slot);
    }
    const View lv = d.lv;
    const int64_t M = d.M, N_ = d.N, K = d.K, sam = d.sam, sak = d.sak, sbk = d.sbk, sbn = d.sbn;
    // Products that split their contraction run one after another, sharing one
    // workspace in the arena.
    const int64_t ws_bytes = ghip_gemm_workspace_bytes(dt, odt, 1, M, N_, K);
    const View wsv = gemm_workspace_view(ws_bytes, &wr);
    add_step(fmt("gemm_grouped %s G=%d M=%lld N=%lld K=%lld (products sharing a; a strides m=%lld k=%lld, b strides "
                 "k=%lld n=%lld%s)",
                 dtype_name(dt), G, (long long)M, (long long)N_, (long long)K, (long long)sam, (long long)sak,
                 (long long)sbk, (long long)sbn, split_note(ws_bytes, 1, M, N_, K, dt).c_str()),
             rd, wr, [=](ExecState& st, GHipError* e) {
               const void* bp[kGemmMaxGroups];
               void* cp[kGemmMaxGroups];
               for (int g = 0; g < G; ++g) {
                 bp[g] = st.ptr(rvs[g], dt);
                 cp[g] = st.ptr(ys[g], odt);
               }
               void* ws = ws_bytes > 0 ? st.ptr(wsv, GHIP_DTYPE_FLOAT32) : nullptr;
               return ghip_gemm_grouped_ws(dt, odt, G, M, N_, K, st.ptr(lv, dt), sam, sak, bp, sbk, sbn, cp, N_, ws,
                                           ws_bytes, st.stream, e);
             });
    for (int g = 1; g < G; ++g) {
      views[grp[g]] = ys[g];
      have[grp[g]] = 1;
    }
    return ys[0];
  }

  View emit_dot(int v) {
    const Node& n = N[v];
    DotPlan d;
    if (!plan_dot(v, true, &d)) return bad();
    if (group_dots) {
      const View y = emit_dot_group(v, d);
      if (failed) return bad();
      if (y.slot >= 0) return y;
    }
    const View lv = d.lv, rv = d.rv;
    const int64_t B = d.B, sab = d.sab, sbb = d.sbb, M = d.M, sam = d.sam, K = d.K, sak = d.sak, N_ = d.N,
                  sbn = d.sbn, sbk = d.sbk;
    View y = fresh(n.shape);
    const int dt = N[n.in[0]].shape.dtype, odt = n.shape.dtype;
    const int64_t scb = M * N_, scm = N_;
    std::vector<int> wr{y.slot};
    const int64_t ws_bytes = ghip_gemm_workspace_bytes(dt, odt, B, M, N_, K);
    const View wsv = gemm_workspace_view(ws_bytes, &wr);
    add_step(fmt("gemm_batched %s B=%lld M=%lld N=%lld K=%lld (%s; a strides b=%lld m=%lld k=%lld, b strides b=%lld k=%lld n=%lld%s)",
                 dtype_name(dt), (long long)B, (long long)M, (long long)N_, (long long)K, d.how.c_str(), (long long)sab,
                 (long long)sam, (long long)sak, (long long)sbb, (long long)sbk, (long long)sbn,
                 split_note(ws_bytes, B, M, N_, K, dt).c_str()),
             {lv.slot, rv.slot}, wr, [=](ExecState& st, GHipError* e) {
               void* ws = ws_bytes > 0 ? st.ptr(wsv, GHIP_DTYPE_FLOAT32) : nullptr;
               return ghip_gemm_batched_ws(dt, odt, B, M, N_, K, st.ptr(lv, dt), sab, sam, sak, st.ptr(rv, dt), sbb, sbk,
                                           sbn, st.ptr(y, odt), scb, scm, 1, ws, ws_bytes, st.stream, e);
             });
    return y;
  }

  // The arena view of a GEMM step's contraction-split workspace (none for 0
  // bytes), appended to the step's written slots.
  View gemm_workspace_view(int64_t ws_bytes, std::vector<int>* wr) {
    if (ws_bytes <= 0) return View{};
    Shape wss;
    wss.dtype = GHIP_DTYPE_FLOAT32;
    wss.dims = {(ws_bytes + 3) / 4};
    const View w = fresh(wss);
    wr->push_back(w.slot);
    return w;
  }
  static std::string split_note(int64_t ws_bytes, int64_t B, int64_t M, int64_t N_, int64_t K, int dt) {
    if (ws_bytes <= 0) return "";
    return fmt("; contraction split in %d", gemm_k_split(B, M, N_, K, dt == GHIP_DTYPE_FLOAT32 ? 4 : 2).s);
  }

  // ------------------------------------------------------------------ GEMM epilogue fusion
  // An elementwise cluster whose inputs include one DotGeneral (or two that share
  // the left operand and all sizes) consumed only inside the cluster runs as
  // one GEMM whose epilogue evaluates the cluster: the Dot results never touch
  // HBM.  The Dot value enters the epilogue rounded to the Dot's dtype, and the
  // members' code is the same generated code the stand-alone cluster kernel
  // runs, so fused and unfused plans give bit-identical results.
  bool fuse_epilogues = true;
  bool fuse_reductions = true;
  // Reduce fusion: the elementwise cluster (root) a Reduce absorbs as its
  // producer, and the consumer cluster (root) a Reduce's value feeds; -1: none.
  std::vector<int> reduce_prod, cons_reduce;
  View emit_reduce_fused(int R, int prod_root, int cons_root);
  View emit_gemm_epilogue(int v, const std::vector<int>& mem, bool* fused);
  bool emit_split_partials(int o, const Shape& os, const std::set<int>& inset, View* wsv, int* splits);
  std::string member_stmt(int u, std::map<int, std::string>& expr, const std::string& name);

  // ------------------------------------------------------------------ Gather
  View emit_gather(int v) {
    const Node& n = N[v];
    const Shape& os = N[n.in[0]].shape;
    const Shape& is = N[n.in[1]].shape;
    const int r = os.rank(), ir = is.rank();
    const int ivax = static_cast<int>(n.i0);
    // Embedding-lookup pattern (gather.go:61-98).
    bool emb = n.a2.size() == 1 && n.a1.size() == 1 && n.a1[0] == n.a2[0] && n.a3[n.a2[0]] == 1 &&
               (ivax == ir - 1 || ivax == ir);
    const int g = emb ? static_cast<int>(n.a2[0]) : -1;
    for (int i = 0; emb && i < r; ++i)
      if (i != g && n.a3[i] != os.dims[i]) emb = false;
    const int batch_rank = n.shape.rank() - static_cast<int>(n.a0.size());
    for (size_t i = 0; emb && i < n.a0.size(); ++i)
      if (n.a0[i] != batch_rank + static_cast<int64_t>(i)) emb = false;  // offset axes trailing
    if (!emb) return fail(GHIP_ERR_UNSUPPORTED, "Gather: only the embedding-lookup form is lowered");
    View tv = get(n.in[0]), iv = get(n.in[1]);
    if (failed) return bad();
    // Bring the gathered axis first, the rest in order: rows of the table.
    std::vector<int64_t> perm{g};
    for (int i = 0; i < r; ++i)
      if (i != g) perm.push_back(i);
    View tab = materialize(permute(tv, perm), permute_shape(os, perm), "(Gather table, gathered axis first)");
    View ids = materialize(iv, is);
    if (failed) return bad();
    View y = fresh(n.shape);
    const int64_t V = os.dims[g];
    const int64_t row_bytes = V ? static_cast<int64_t>(os.bytes() / V) : 0;
    const int64_t cnt = is.size() / (ivax < ir ? is.dims[ivax] : 1);
    const int idt = is.dtype, tdt = os.dtype;
    add_step(fmt("gather_rows table=%s ids=%s rows=%lld", os.str().c_str(), is.str().c_str(), (long long)cnt),
             {tab.slot, ids.slot}, {y.slot}, [=](ExecState& st, GHipError* e) {
               return launch_gather_rows(st.ptr(tab, tdt), V, row_bytes, st.ptr(ids, idt), idt, cnt, st.ptr(y, tdt), st.stream, e);
             });
    if (g != 0) {
      // Output rows follow the permuted table: [batch..., other axes in order] — that
      // is already the XLA output order for trailing offset axes.
    }
    return y;
  }

  // ------------------------------------------------------------------ SDPA
  View emit_sdpa(int v) {
    const Node& n = N[v];
    const int qv_ = n.in[0], kv_ = n.in[1], vv_ = n.in[2], mv_ = n.in[3];
    const int H = static_cast<int>(n.i0), Hkv = static_cast<int>(n.i1);
    const bool bshd = n.i2 == GHIP_LAYOUT_BSHD;
    const bool causal = n.i3 != 0;
    const int dt = N[qv_].shape.dtype;
    if (dt != GHIP_DTYPE_FLOAT32 && dt != GHIP_DTYPE_BFLOAT16 && dt != GHIP_DTYPE_FLOAT16)
      return fail(GHIP_ERR_UNSUPPORTED, "SDPA: float32 / bfloat16 / float16 only");
    const std::vector<int64_t> to_bhsd{0, 2, 1, 3};
    auto as_bhsd = [&](int id, Shape* s) {
      View w = get(id);
      *s = N[id].shape;
      if (bshd) {
        w = permute(w, to_bhsd);
        *s = permute_shape(*s, to_bhsd);
      }
      return w;
    };
    Shape qs, ks, vs;
    View q = as_bhsd(qv_, &qs), k = as_bhsd(kv_, &ks), vw = as_bhsd(vv_, &vs);
    if (failed) return bad();
    const int64_t B = qs.dims[0], Sq = qs.dims[2], D = qs.dims[3], Sk = ks.dims[2], Dv = vs.dims[3];
    // Mask (function.go:2840-2878): a rank-4 mask follows Q's layout (:2709-2718);
    // any rank broadcasts to the scores [B, H, Sq, Sk] over its trailing axes
    // (broadcastMaskToScores, :2959-2974): strides 0 on size-1 and missing axes.
    View mview;
    int mdt = -1;
    std::array<int64_t, 4> mst{0, 0, 0, 0};
    if (mv_ >= 0) {
      Shape ms = N[mv_].shape;
      View mw = get(mv_);
      if (failed) return bad();
      if (bshd && ms.rank() == 4) {
        mw = permute(mw, to_bhsd);
        ms = permute_shape(ms, to_bhsd);
      }
      const int64_t sd[4] = {B, H, Sq, Sk};
      const int off = 4 - ms.rank();
      for (int i = 0; i < ms.rank(); ++i) {
        if (ms.dims[i] == 1) continue;
        if (ms.dims[i] != sd[off + i])
          return fail(GHIP_ERR_INVALID_ARG, fmt("SDPA: mask %s does not broadcast to the scores [%lld,%lld,%lld,%lld]",
                                                ms.str().c_str(), (long long)B, (long long)H, (long long)Sq,
                                                (long long)Sk).c_str());
        mst[off + i] = mw.strides[i];
      }
      mview = mw;
      mdt = ms.dtype;
    }
    const bool has_mask = mv_ >= 0;
    // One fused kernel when the operands fit it: Q, K, V (and the mask) are read
    // through their views (BHSD or BSHD, GQA heads shared in place, broadcast mask
    // axes at stride 0) and the output is written in the layout the graph expects.
    if (D == Dv && q.strides[3] == 1 && k.strides[3] == 1 && vw.strides[3] == 1) {
      Shape os;
      os.dtype = dt;
      os.dims = {B, H, Sq, Dv};
      const int64_t qst[3] = {q.strides[0], q.strides[1], q.strides[2]};
      const int64_t kst[3] = {k.strides[0], k.strides[1], k.strides[2]};
      const int64_t vst[3] = {vw.strides[0], vw.strides[1], vw.strides[2]};
      // BHSD strides of the contiguous output in the caller's layout.
      const int64_t ostr[3] = {H * Sq * Dv, bshd ? Dv : Sq * Dv, bshd ? H * Dv : Dv};
      bool mask_ok = true;
      for (int i = 0; i < 4 && has_mask; ++i) mask_ok = mask_ok && mst[i] >= 0;
      const int64_t a16 = 16 / dtype_size(dt);  // elements in 16 bytes
      const bool al = q.offset % a16 == 0 && k.offset % a16 == 0 && vw.offset % a16 == 0;
      const float scale = static_cast<float>(n.f0);
      if (al && mask_ok && sdpa_fused_supported(dt, H, Hkv, Sq, Sk, D, qst, kst, vst, ostr, scale, mdt)) {
        Shape os_layout = bshd ? permute_shape(os, to_bhsd) : os;
        View out_l = fresh(os_layout);
        View ov = bshd ? permute(out_l, to_bhsd) : out_l;
        std::array<int64_t, 3> aq{qst[0], qst[1], qst[2]}, ak{kst[0], kst[1], kst[2]},
            av{vst[0], vst[1], vst[2]}, ao{ov.strides[0], ov.strides[1], ov.strides[2]};
        std::vector<int> rd{q.slot, k.slot, vw.slot};
        if (has_mask) rd.push_back(mview.slot);
        const View mv = mview;
        const std::array<int64_t, 4> ms4 = mst;
        // Few (batch, head, query block) workgroups: the key range splits over a
        // workspace in the arena (partial outputs merged by log-sum-exp).
        const int64_t ws_bytes = ghip_sdpa_workspace_bytes(dt, B, H, Hkv, Sq, Sk, D, causal ? 1 : 0);
        std::vector<int> wr{ov.slot};
        View wsv;
        if (ws_bytes > 0) {
          Shape wss;
          wss.dtype = GHIP_DTYPE_FLOAT32;
          wss.dims = {(ws_bytes + 3) / 4};
          wsv = fresh(wss);
          wr.push_back(wsv.slot);
        }
        add_step(fmt("sdpa_fwd %s B=%lld H=%lld Hkv=%d Sq=%lld Sk=%lld D=%lld causal=%d mask=%s (fused attention%s)",
                     dtype_name(dt), (long long)B, (long long)H, Hkv, (long long)Sq, (long long)Sk, (long long)D,
                     causal ? 1 : 0, has_mask ? dtype_name(mdt) : "none", ws_bytes > 0 ? ", key range split" : ""),
                 rd, wr, [=](ExecState& st, GHipError* e) {
                   const void* mp = has_mask ? st.ptr(mv, mdt) : nullptr;
                   void* ws = ws_bytes > 0 ? st.ptr(wsv, GHIP_DTYPE_FLOAT32) : nullptr;
                   return ghip_sdpa_fwd_masked_ws(dt, st.ptr(q, dt), st.ptr(k, dt), st.ptr(vw, dt), st.ptr(ov, dt), B,
                                                  H, Hkv, Sq, Sk, D, aq.data(), ak.data(), av.data(), ao.data(), mp, mdt,
                                                  ms4.data(), scale, causal ? 1 : 0, ws, ws_bytes, st.stream, e);
                 });
        return out_l;
      }
    }
    // GQA: repeat each KV head H/Hkv times (function.go:2731-2744) as a broadcast view.
    auto repeat = [&](View w, Shape s) {
      if (Hkv == H) return std::make_pair(w, s);
      const int rep = H / Hkv;
      Shape s5 = s;
      s5.dims = {s.dims[0], s.dims[1], rep, s.dims[2], s.dims[3]};
      View w5;
      w5.slot = w.slot;
      w5.offset = w.offset;
      w5.strides = {w.strides[0], w.strides[1], 0, w.strides[2], w.strides[3]};
      View m = materialize(w5, s5, "(SDPA repeat KV heads)");
      Shape s4 = s;
      s4.dims[1] = H;
      View m4 = contig(m.slot, s4);
      m4.offset = m.offset;
      return std::make_pair(m4, s4);
    };
    auto kk = repeat(k, ks);
    auto vvv = repeat(vw, vs);
    k = kk.first; ks = kk.second;
    vw = vvv.first; vs = vvv.second;
    // Batch (b, h) must merge into one GEMM batch stride; else materialise BHSD.
    auto bstride = [&](const View& w, const Shape& s) -> int64_t {
      if (s.dims[1] == 1) return w.strides[0];
      if (s.dims[0] == 1 || w.strides[0] == w.strides[1] * s.dims[1]) return w.strides[1];
      return -1;
    };
    if (bstride(q, qs) < 0) q = materialize(q, qs, "(SDPA Q to BHSD)");
    if (bstride(k, ks) < 0) k = materialize(k, ks, "(SDPA K to BHSD)");
    if (bstride(vw, vs) < 0) vw = materialize(vw, vs, "(SDPA V to BHSD)");
    if (failed) return bad();
    const int64_t BH = B * H;
    Shape ss;
    ss.dtype = dt;
    ss.dims = {B, H, Sq, Sk};
    View scores = fresh(ss);
    View probs = fresh(ss);
    Shape os;
    os.dtype = dt;
    os.dims = {B, H, Sq, Dv};
    View out = fresh(os);
    const int64_t qbs = bstride(q, qs), qms = q.strides[2], qks = q.strides[3];
    const int64_t kbs = bstride(k, ks), kns = k.strides[2], kks = k.strides[3];
    const int64_t vbs = bstride(vw, vs), vks = vw.strides[2], vns = vw.strides[3];
    const float scale = static_cast<float>(n.f0);
    add_step(fmt("gemm_batched %s B=%lld M=%lld N=%lld K=%lld (SDPA scores = Q.K^T)", dtype_name(dt), (long long)BH,
                 (long long)Sq, (long long)Sk, (long long)D),
             {q.slot, k.slot}, {scores.slot}, [=](ExecState& st, GHipError* e) {
               return ghip_gemm_batched(dt, dt, BH, Sq, Sk, D, st.ptr(q, dt), qbs, qms, qks, st.ptr(k, dt), kbs, kks, kns,
                                        st.ptr(scores, dt), Sq * Sk, Sk, 1, st.stream, e);
             });
    std::vector<int> rd{scores.slot};
    if (has_mask) rd.push_back(mview.slot);
    const View mv = mview;
    const std::array<int64_t, 4> ms4 = mst;
    add_step(fmt("scale_mask_softmax_rows %s rows=%lld sk=%lld scale=%g causal=%d mask=%s", dtype_name(dt),
                 (long long)(BH * Sq), (long long)Sk, n.f0, causal ? 1 : 0, has_mask ? dtype_name(mdt) : "none"),
             rd, {probs.slot}, [=](ExecState& st, GHipError* e) {
               const void* mp = has_mask ? st.ptr(mv, mdt) : nullptr;
               return ghip_scale_mask_softmax_rows_ex(dt, st.ptr(scores, dt), st.ptr(probs, dt), B, H, Sq, Sk, scale,
                                                      causal ? 1 : 0, mp, mdt, ms4.data(), st.stream, e);
             });
    add_step(fmt("gemm_batched %s B=%lld M=%lld N=%lld K=%lld (SDPA out = P.V)", dtype_name(dt), (long long)BH,
                 (long long)Sq, (long long)Dv, (long long)Sk),
             {probs.slot, vw.slot}, {out.slot}, [=](ExecState& st, GHipError* e) {
               return ghip_gemm_batched(dt, dt, BH, Sq, Dv, Sk, st.ptr(probs, dt), Sq * Sk, Sk, 1, st.ptr(vw, dt), vbs, vks,
                                        vns, st.ptr(out, dt), Sq * Dv, Dv, 1, st.stream, e);
             });
    return bshd ? permute(out, to_bhsd) : out;
  }

  // ------------------------------------------------------------------ elementwise codegen
  View emit_cluster(int root, int v);
  std::string ctype(int dt) {
    switch (dt) {
      case GHIP_DTYPE_BOOL: return "bool";
      case GHIP_DTYPE_INT8: return "signed char";
      case GHIP_DTYPE_INT16: return "short";
      case GHIP_DTYPE_INT32: return "int";
      case GHIP_DTYPE_INT64: return "long long";
      case GHIP_DTYPE_UINT8: return "unsigned char";
      case GHIP_DTYPE_UINT16: return "unsigned short";
      case GHIP_DTYPE_UINT32: return "unsigned int";
      case GHIP_DTYPE_UINT64: return "unsigned long long";
      case GHIP_DTYPE_FLOAT64: return "double";
      default: return "float";  // f16 / bf16 / f32 compute in fp32
    }
  }
  std::string stype(int dt) {
    switch (dt) {
      case GHIP_DTYPE_BOOL: return "unsigned char";
      case GHIP_DTYPE_BFLOAT16: return "unsigned short";
      case GHIP_DTYPE_FLOAT16: return "_Float16";
      default: return ctype(dt);
    }
  }
  std::string load_expr(int dt, const std::string& e) {
    if (dt == GHIP_DTYPE_BFLOAT16) return "bf2f(" + e + ")";
    if (dt == GHIP_DTYPE_FLOAT16) return "(float)(" + e + ")";
    if (dt == GHIP_DTYPE_BOOL) return "(" + e + " != 0)";
    return e;
  }
  std::string store_expr(int dt, const std::string& e) {
    if (dt == GHIP_DTYPE_BFLOAT16) return "f2bf(" + e + ")";
    if (dt == GHIP_DTYPE_FLOAT16) return "(_Float16)(" + e + ")";
    if (dt == GHIP_DTYPE_BOOL) return "(unsigned char)(" + e + ")";
    return e;
  }
  std::string round_expr(int dt, const std::string& e) {
    if (dt == GHIP_DTYPE_BFLOAT16) return "rbf(" + e + ")";
    if (dt == GHIP_DTYPE_FLOAT16) return "rhf(" + e + ")";
    return e;
  }
  std::string literal(int dt, double val) {
    char b[64];
    if (dt == GHIP_DTYPE_FLOAT64) snprintf(b, sizeof b, "%a", val);
    else if (dtype_is_float(dt)) {
      if (isnan(val)) return "__builtin_nanf(\"\")";
      if (isinf(val)) return val > 0 ? "__builtin_inff()" : "(-__builtin_inff())";
      snprintf(b, sizeof b, "%af", static_cast<float>(val));
    } else if (dt == GHIP_DTYPE_BOOL) snprintf(b, sizeof b, "%s", val != 0 ? "true" : "false");
    else snprintf(b, sizeof b, "((%s)%lldLL)", ctype(dt).c_str(), static_cast<long long>(val));
    return b;
  }
  std::string int_limits(int dt, bool hi) {
    switch (dt) {
      case GHIP_DTYPE_INT8: return hi ? "127" : "-128";
      case GHIP_DTYPE_INT16: return hi ? "32767" : "-32768";
      case GHIP_DTYPE_INT32: return hi ? "2147483647" : "(-2147483647-1)";
      case GHIP_DTYPE_INT64: return hi ? "9223372036854775807LL" : "(-9223372036854775807LL-1)";
      case GHIP_DTYPE_UINT8: return hi ? "255" : "0";
      case GHIP_DTYPE_UINT16: return hi ? "65535" : "0";
      case GHIP_DTYPE_UINT32: return hi ? "4294967295u" : "0";
      default: return hi ? "18446744073709551615ull" : "0";
    }
  }
  std::string op_expr(const Node& n, const std::vector<std::string>& a, const std::vector<int>& adt);

  // ------------------------------------------------------------------ outputs / memory
  int finish();
};

// Expression for one elementwise node given operand expressions (compute types).
std::string Lowerer::op_expr(const Node& n, const std::vector<std::string>& a, const std::vector<int>& adt) {
  const int dt = n.shape.dtype;
  const int it = adt.empty() ? dt : adt[0];
  const bool fl = dtype_is_float(it);
  const bool f64 = it == GHIP_DTYPE_FLOAT64;
  const std::string T = ctype(dt);
  auto fn1 = [&](const char* f32, const char* f64n) { return std::string(f64 ? f64n : f32) + "(" + a[0] + ")"; };
  // 16-bit float results: the hardware transcendental forms (see hexp in the prelude).
  const bool half = dt == GHIP_DTYPE_BFLOAT16 || dt == GHIP_DTYPE_FLOAT16;
  switch (n.kind) {
    case Kind::Unary:
      switch (n.sub) {
        case GHIP_UNARY_ABS: return fl ? fn1("fabsf", "fabs") : (dtype_is_unsigned(it) ? a[0] : "(" + T + ")(" + a[0] + " < 0 ? -" + a[0] + " : " + a[0] + ")");
        case GHIP_UNARY_NEG: return "(" + T + ")(-" + a[0] + ")";
        case GHIP_UNARY_SQRT: return fn1("sqrtf", "sqrt");
        case GHIP_UNARY_RSQRT: return f64 ? "(1.0 / sqrt(" + a[0] + "))" : "rsqrtf(" + a[0] + ")";
        case GHIP_UNARY_EXP: return half ? "hexp(" + a[0] + ")" : fn1("expf", "exp");
        case GHIP_UNARY_EXPM1: return fn1("expm1f", "expm1");
        case GHIP_UNARY_LOG: return fn1("logf", "log");
        case GHIP_UNARY_LOG1P: return fn1("log1pf", "log1p");
        case GHIP_UNARY_SIN: return fn1("sinf", "sin");
        case GHIP_UNARY_COS: return fn1("cosf", "cos");
        case GHIP_UNARY_TANH: return half ? "htanh(" + a[0] + ")" : fn1("tanhf", "tanh");
        case GHIP_UNARY_LOGISTIC:
          if (half) return "hsigmoid(" + a[0] + ")";
          return f64 ? "(1.0 / (1.0 + exp(-" + a[0] + ")))" : "(1.0f / (1.0f + expf(-" + a[0] + ")))";
        case GHIP_UNARY_ERF: return fn1("erff", "erf");
        case GHIP_UNARY_FLOOR: return fn1("floorf", "floor");
        case GHIP_UNARY_CEIL: return fn1("ceilf", "ceil");
        case GHIP_UNARY_ROUND: return fn1("rintf", "rint");  // round half to even
        case GHIP_UNARY_SIGN:
          if (fl) return "(" + a[0] + " > 0 ? (" + T + ")1 : (" + a[0] + " < 0 ? (" + T + ")-1 : " + a[0] + "))";
          return "(" + T + ")(" + a[0] + " > 0 ? 1 : (" + a[0] + " < 0 ? -1 : 0))";
        case GHIP_UNARY_LOGICAL_NOT: return "(!" + a[0] + ")";
        case GHIP_UNARY_BITWISE_NOT: return "(" + T + ")(~" + a[0] + ")";
        case GHIP_UNARY_IS_FINITE: return "(bool)isfinite(" + a[0] + ")";
        case GHIP_UNARY_IS_NAN: return "(bool)isnan(" + a[0] + ")";
        default: return a[0];
      }
    case Kind::Binary: {
      const std::string& x = a[0];
      const std::string& y = a[1];
      const int bits = dtype_size(it) * 8;
      switch (n.sub) {
        case GHIP_BINARY_ADD: return "(" + T + ")(" + x + " + " + y + ")";
        case GHIP_BINARY_SUB: return "(" + T + ")(" + x + " - " + y + ")";
        case GHIP_BINARY_MUL: return "(" + T + ")(" + x + " * " + y + ")";
        case GHIP_BINARY_DIV:
          if (fl) return "(" + x + " / " + y + ")";
          if (dtype_is_unsigned(it)) return "(" + T + ")(" + y + " == 0 ? (" + T + ")~(" + T + ")0 : " + x + " / " + y + ")";
          return "(" + T + ")(" + y + " == 0 ? (" + T + ")-1 : ((" + y + " == -1 && " + x + " == " + int_limits(it, false) + ") ? " + x + " : " + x + " / " + y + "))";
        case GHIP_BINARY_REM:
          if (fl) return std::string(f64 ? "fmod(" : "fmodf(") + x + ", " + y + ")";
          if (dtype_is_unsigned(it)) return "(" + T + ")(" + y + " == 0 ? " + x + " : " + x + " % " + y + ")";
          return "(" + T + ")(" + y + " == 0 ? " + x + " : (" + y + " == -1 ? 0 : " + x + " % " + y + "))";
        case GHIP_BINARY_POW:
          if (fl) return std::string(f64 ? "pow(" : "powf(") + x + ", " + y + ")";
          return "(" + T + ")ipow((long long)" + x + ", (long long)" + y + ")";
        case GHIP_BINARY_MAX: return fl ? "fmax_nan(" + x + ", " + y + ")" : "(" + x + " > " + y + " ? " + x + " : " + y + ")";
        case GHIP_BINARY_MIN: return fl ? "fmin_nan(" + x + ", " + y + ")" : "(" + x + " < " + y + " ? " + x + " : " + y + ")";
        case GHIP_BINARY_ATAN2: return std::string(f64 ? "atan2(" : "atan2f(") + x + ", " + y + ")";
        case GHIP_BINARY_LOGICAL_AND: return "(" + x + " && " + y + ")";
        case GHIP_BINARY_LOGICAL_OR: return "(" + x + " || " + y + ")";
        case GHIP_BINARY_LOGICAL_XOR: return "(" + x + " != " + y + ")";
        case GHIP_BINARY_BITWISE_AND: return "(" + T + ")(" + x + " & " + y + ")";
        case GHIP_BINARY_BITWISE_OR: return "(" + T + ")(" + x + " | " + y + ")";
        case GHIP_BINARY_BITWISE_XOR: return "(" + T + ")(" + x + " ^ " + y + ")";
        case GHIP_BINARY_SHIFT_LEFT:
          return "(" + T + ")((" + y + " < 0 || " + y + " >= " + std::to_string(bits) + ") ? 0 : (" + T + ")(" + x + " << " + y + "))";
        case GHIP_BINARY_SHIFT_RIGHT_ARITHMETIC:
          if (dtype_is_unsigned(it)) return "(" + T + ")((" + y + " >= " + std::to_string(bits) + ") ? 0 : (" + x + " >> " + y + "))";
          return "(" + T + ")((" + y + " < 0 || " + y + " >= " + std::to_string(bits) + ") ? (" + x + " < 0 ? -1 : 0) : (" + x + " >> " + y + "))";
        default: {  // logical right shift: shift the unsigned bit pattern
          static const char* ut[] = {"", "unsigned char", "unsigned short", "", "unsigned int", "", "", "", "unsigned long long"};
          const std::string U = ut[dtype_size(it)];
          return "(" + T + ")((" + y + " < 0 || " + y + " >= " + std::to_string(bits) + ") ? 0 : (" + U + ")((" + U + ")" + x + " >> " + y + "))";
        }
      }
    }
    case Kind::Compare: {
      static const char* ops[] = {"==", "!=", ">", ">=", "<", "<="};
      return "(" + a[0] + " " + ops[n.sub] + " " + a[1] + ")";
    }
    case Kind::Where: return "(" + a[0] + " ? " + a[1] + " : " + a[2] + ")";
    case Kind::Clamp:
      if (fl) return "fmin_nan(fmax_nan(" + a[1] + ", " + a[0] + "), " + a[2] + ")";
      return "(" + a[1] + " < " + a[0] + " ? " + a[0] + " : (" + a[1] + " > " + a[2] + " ? " + a[2] + " : " + a[1] + "))";
    case Kind::Convert: {
      const int src = it;
      if (dt == GHIP_DTYPE_BOOL) return "(" + a[0] + " != 0)";
      if (dtype_is_float(dt)) return "(" + T + ")(" + a[0] + ")";
      if (dtype_is_float(src))  // truncate toward zero, saturating; NaN -> 0
        return "(" + T + ")((" + a[0] + " != " + a[0] + ") ? 0 : ((" + a[0] + ") <= (" + ctype(src) + ")" + int_limits(dt, false) +
               " ? " + int_limits(dt, false) + " : ((" + a[0] + ") >= (" + ctype(src) + ")" + int_limits(dt, true) + " ? " +
               int_limits(dt, true) + " : (" + T + ")(" + a[0] + "))))";
      return "(" + T + ")(" + a[0] + ")";
    }
    default: return a.empty() ? "0" : a[0];
  }
}

// Statement computing elementwise member u (in its compute type, rounded to its
// dtype) from the expressions of its operands; records u's expression.
std::string Lowerer::member_stmt(int u, std::map<int, std::string>& expr, const std::string& name) {
  const Node& n = N[u];
  std::vector<std::string> a;
  std::vector<int> adt;
  for (int o : n.in) {
    a.push_back(expr[o]);
    adt.push_back(N[o].shape.dtype);
  }
  // Where / Clamp: the dtype driving op semantics is the value operands'.
  std::vector<int> sem = adt;
  if (n.kind == Kind::Where) sem = {adt[1]};
  if (n.kind == Kind::Clamp) sem = {adt[1]};
  expr[u] = name;
  return "    const " + ctype(n.shape.dtype) + " " + name + " = " + round_expr(n.shape.dtype, op_expr(n, a, sem)) + ";\n";
}


// One generated kernel for Reduce R, evaluating its producer cluster (rooted at
// prod_root, over R's input shape) on the fly instead of reading it from HBM,
// and, when cons_root >= 0, the consumer cluster (over R's output shape) on the
// reduced value before the one store.  The accumulation order is the generic
// reduce kernels' (one wave per output, lanes striding the reduced index, then a
// butterfly, when >= 64 values are reduced; else one thread per output in
// order), and the reduced value is rounded to R's dtype before the consumers
// see it, so results are bit-identical to the unfused plan.
View Lowerer::emit_reduce_fused(int R, int prod_root, int cons_root) {
  const Node& rn = N[R];
  const int x = rn.in[0];
  const Shape& xs = N[x].shape;
  const Shape& rs = rn.shape;
  const int rx = xs.rank();
  std::vector<int> kept, red;
  for (int i = 0; i < rx; ++i)
    (std::find(rn.a0.begin(), rn.a0.end(), i) != rn.a0.end() ? red : kept).push_back(i);
  int64_t osize = 1, rsize = 1;
  for (int i : kept) osize *= xs.dims[i];
  for (int i : red) rsize *= xs.dims[i];
  const int rdt = rs.dtype, xdt = xs.dtype;
  const bool wave = rsize >= 64;
  // Accumulator type of the generic reduce kernels (RAcc).
  std::string acc_t = "float";
  if (rdt == GHIP_DTYPE_FLOAT64) acc_t = "double";
  else if (dtype_is_int(rdt)) acc_t = dtype_is_unsigned(rdt) ? "unsigned long long" : "long long";
  struct In {
    View view;
    int dt;
    std::string off;  // element offset expression
  };
  std::vector<In> ins;
  std::ostringstream pbody, cbody;
  std::map<int, std::string> expr;
  // Input coordinates: x_i for input axis i (kept axes from the output index,
  // reduced axes from the reduced index); output coordinates o_k.
  auto load_input = [&](int o, const std::vector<std::string>& coord, const Shape& cs, std::ostringstream& body) {
    View w = get(o);
    if (failed) return;
    const Shape& sh = N[o].shape;
    const int off = cs.rank() - sh.rank();
    std::string e = "0";
    for (int d = 0; d < sh.rank(); ++d)
      if (sh.dims[d] != 1 && w.strides[d] != 0) e += " + " + coord[off + d] + " * " + std::to_string(w.strides[d]) + "LL";
    const int k = static_cast<int>(ins.size());
    body << "      const " << ctype(sh.dtype) << " in" << k << " = "
         << load_expr(sh.dtype, "((const " + stype(sh.dtype) + "*)p_in" + std::to_string(k) + ")[" + e + "]") << ";\n";
    expr[o] = "in" + std::to_string(k);
    ins.push_back(In{w, sh.dtype, e});
  };
  auto cluster_code = [&](int root, const Shape& cs, const std::vector<std::string>& coord, std::ostringstream& body,
                          const std::set<int>& preset) {
    std::vector<int> mem;
    for (int u = 0; u <= root; ++u)
      if (cluster[u] == root) mem.push_back(u);
    std::set<int> inset(mem.begin(), mem.end());
    for (int u : mem) {
      for (int o : N[u].in) {
        if (o < 0 || inset.count(o) || expr.count(o) || preset.count(o)) continue;
        double c;
        if (scalar_const(o, &c) && (dtype_is_float(N[o].shape.dtype) || fabs(c) < 9007199254740992.0)) {
          expr[o] = literal(N[o].shape.dtype, c);
          continue;
        }
        if (N[o].kind == Kind::Iota && N[o].shape.dims == cs.dims) {
          expr[o] = "((" + ctype(N[o].shape.dtype) + ")" + coord[N[o].i0] + ")";
          continue;
        }
        load_input(o, coord, cs, body);
        if (failed) return;
      }
      if (N[u].kind == Kind::Iota) {
        const std::string name = "v" + std::to_string(u);
        body << "      const " << ctype(N[u].shape.dtype) << " " << name << " = "
             << round_expr(N[u].shape.dtype, "((" + ctype(N[u].shape.dtype) + ")" + coord[N[u].i0] + ")") << ";\n";
        expr[u] = name;
      } else {
        body << "  " << member_stmt(u, expr, "v" + std::to_string(u));
      }
    }
  };
  std::vector<std::string> xc(rx), oc(rs.rank());
  for (size_t k = 0; k < kept.size(); ++k) xc[kept[k]] = "o" + std::to_string(k);
  for (size_t k = 0; k < red.size(); ++k) xc[red[k]] = "r" + std::to_string(k);
  for (int k = 0; k < rs.rank(); ++k) oc[k] = "o" + std::to_string(k);
  // element value fed to the accumulator
  std::string val;
  if (prod_root >= 0) {
    cluster_code(prod_root, xs, xc, pbody, {});
    if (failed) return bad();
    val = round_expr(xdt, expr[prod_root]);
  } else {
    load_input(x, xc, xs, pbody);
    if (failed) return bad();
    val = expr[x];
  }
  // consumer cluster over the output shape, with R's value preset
  std::string outv = "red", odt_s;
  int out_v = R, odt = rdt;
  if (cons_root >= 0) {
    expr.clear();  // the producer's names are scoped to the reduction loop
    expr[R] = "red";
    cluster_code(cons_root, rs, oc, cbody, {R});
    if (failed) return bad();
    out_v = cons_root;
    odt = N[cons_root].shape.dtype;
    outv = expr[cons_root];
  }
  const std::vector<std::string> ops = {"a + b", "a * b", "((a > b || a != a) ? a : b)", "((a < b || a != a) ? a : b)"};
  std::string init;
  switch (rn.sub) {
    case GHIP_REDUCE_SUM: init = "(" + acc_t + ")0"; break;
    case GHIP_REDUCE_PRODUCT: init = "(" + acc_t + ")1"; break;
    case GHIP_REDUCE_MAX:
      init = acc_t == "float" ? "(-__builtin_inff())" : acc_t == "double" ? "(-__builtin_inf())"
           : acc_t == "long long" ? "(-9223372036854775807LL-1)" : "0ull";
      break;
    default:
      init = acc_t == "float" ? "__builtin_inff()" : acc_t == "double" ? "__builtin_inf()"
           : acc_t == "long long" ? "9223372036854775807LL" : "18446744073709551615ull";
  }
  std::ostringstream src;
  src << kRtcPrelude << "__device__ __forceinline__ " << acc_t << " comb(" << acc_t << " a, " << acc_t << " b) { return "
      << ops[rn.sub] << "; }\n";
  src << "extern \"C\" __global__ void __launch_bounds__(256) fused_reduce(\n";
  for (size_t k = 0; k < ins.size(); ++k) src << "    const void* __restrict__ p_in" << k << ",\n";
  src << "    void* __restrict__ p_out) {\n";
  if (wave)
    src << "  const long long o = (long long)blockIdx.x * 4 + threadIdx.x / 64;\n  const int lane = threadIdx.x % 64;\n";
  else
    src << "  const long long o = (long long)blockIdx.x * 256 + threadIdx.x;\n";
  src << "  if (o >= " << osize << "LL) return;\n";
  // output coordinates
  if (kept.size() == 1) {
    src << "  const long long o0 = o;\n";
  } else if (!kept.empty()) {
    src << "  long long q = o;\n";
    for (int k = static_cast<int>(kept.size()) - 1; k >= 0; --k)
      src << "  const long long o" << k << " = q % " << xs.dims[kept[k]] << "LL; q /= " << xs.dims[kept[k]] << "LL;\n";
  }
  src << "  " << acc_t << " acc = " << init << ";\n";
  src << (wave ? "  for (long long r = lane; r < " : "  for (long long r = 0; r < ") << rsize << "LL; r += " << (wave ? 64 : 1)
      << ") {\n";
  if (red.size() == 1) {
    src << "      const long long r0 = r;\n";
  } else {
    src << "      long long t = r;\n";
    for (int k = static_cast<int>(red.size()) - 1; k >= 0; --k)
      src << "      const long long r" << k << " = t % " << xs.dims[red[k]] << "LL; t /= " << xs.dims[red[k]] << "LL;\n";
  }
  src << pbody.str() << "      acc = comb(acc, (" << acc_t << ")(" << val << "));\n  }\n";
  if (wave) {
    src << "#pragma unroll\n  for (int off = 32; off >= 1; off >>= 1) acc = comb(acc, __shfl_xor(acc, off, 64));\n"
        << "  if (lane != 0) return;\n";
  }
  // the reduced value as the unfused plan stores it, read back in compute type
  src << "  const " << ctype(rdt) << " red = " << load_expr(rdt, "(" + stype(rdt) + ")(" + store_expr(rdt, "(" + ctype(rdt) + ")acc") + ")") << ";\n";
  src << cbody.str();
  src << "  ((" << stype(odt) << "*)p_out)[o] = " << store_expr(odt, outv) << ";\n}\n";
  RtcKernel kern;
  if (rtc_get(be, src.str(), "fused_reduce", &kern, err) != GHIP_OK) return bad();
  const Shape& os = N[out_v].shape;
  View y = fresh(os);
  std::vector<int> rd;
  std::vector<View> in_views;
  std::vector<int> in_dt;
  for (auto& in : ins) {
    rd.push_back(in.view.slot);
    in_views.push_back(in.view);
    in_dt.push_back(in.dt);
  }
  static const char* names[] = {"sum", "product", "max", "min"};
  std::string desc = fmt("fused_reduce_%s %s -> %s", names[rn.sub], xs.str().c_str(), os.str().c_str());
  if (prod_root >= 0) desc += " (producer fused)";
  if (cons_root >= 0) desc += " (consumer fused)";
  const int64_t blocks = wave ? (osize + 3) / 4 : (osize + 255) / 256;
  add_step(desc, rd, {y.slot}, [=](ExecState& st, GHipError* e) -> int {
    if (osize == 0) return GHIP_OK;
    std::vector<void*> ptrs(in_views.size());
    std::vector<void*> args;
    for (size_t k = 0; k < in_views.size(); ++k) ptrs[k] = st.ptr(in_views[k], in_dt[k]);
    void* outp = st.ptr(y, odt);
    for (size_t k = 0; k < ptrs.size(); ++k) args.push_back(&ptrs[k]);
    args.push_back(&outp);
    hipError_t h = hipModuleLaunchKernel(kern.func, static_cast<unsigned>(blocks), 1, 1, 256, 1, 1, 0, st.stream,
                                         args.data(), nullptr);
    if (h != hipSuccess) return check_hip(h, e, "generated reduce kernel launch");
    return GHIP_OK;
  });
  if (cons_root >= 0) {
    views[R] = View{};  // R itself is never materialised
  }
  return y;
}

View Lowerer::emit_cluster(int root, int v) {
  // Members: root's cluster (or, for a value requested outside its cluster, the
  // value alone plus any Iota leaves) in node order.
  std::vector<int> mem;
  if (root >= 0 && cons_reduce[root] >= 0 && !have[cons_reduce[root]])
    return emit_reduce_fused(cons_reduce[root], reduce_prod[cons_reduce[root]], root);
  if (root >= 0) {
    for (int u = 0; u <= root; ++u)
      if (cluster[u] == root) mem.push_back(u);
    if (fuse_epilogues) {
      bool fused = false;
      View y = emit_gemm_epilogue(v, mem, &fused);
      if (failed) return bad();
      if (fused) return y;
    }
  } else {
    mem.push_back(v);
  }
  const Shape& os = N[v].shape;
  std::set<int> inset(mem.begin(), mem.end());
  // Inputs: operands outside the cluster (scalar constants become literals;
  // Iota operands of the cluster's shape are computed from the index).
  struct In {
    int value;
    View view;
    std::vector<int64_t> eff;  // effective strides over os.dims
    bool linear;
    bool partial = false;      // a split Dot's fp32 partials, read at i + j * size
  };
  std::vector<In> ins;
  int n_partial = 0;
  std::map<int, std::string> expr;  // value -> C expression
  std::ostringstream body;
  bool need_idx = false;
  std::vector<std::string> idx_names;
  for (int d = 0; d < os.rank(); ++d) idx_names.push_back("d" + std::to_string(d));
  auto iota_expr = [&](int u) {
    need_idx = true;
    return "((" + ctype(N[u].shape.dtype) + ")" + idx_names[N[u].i0] + ")";
  };
  for (int u : mem) {
    for (int o : N[u].in) {
      if (o < 0 || inset.count(o) || expr.count(o)) continue;
      double c;
      if (scalar_const(o, &c) && (dtype_is_float(N[o].shape.dtype) || fabs(c) < 9007199254740992.0)) {
        expr[o] = literal(N[o].shape.dtype, c);
        continue;
      }
      if (N[o].kind == Kind::Iota && N[o].shape.dims == os.dims) {
        expr[o] = iota_expr(o);
        continue;
      }
      // A DotGeneral read only here whose contraction splits: its fp32 partials
      // come from a GEMM step of their own and are summed here, in range order,
      // then rounded to the Dot's dtype: the value the stand-alone sum kernel
      // stores, without its launch.
      View pw;
      int ps = 0;
      if (fuse_epilogues && emit_split_partials(o, os, inset, &pw, &ps)) {
        const int k = static_cast<int>(ins.size());
        In in{o, pw, contiguous_strides(os.dims), true};
        in.partial = true;
        const std::string pk = "((const float*)p_in" + std::to_string(k) + ")";
        const std::string acc = "acc" + std::to_string(k);
        body << "    float " << acc << " = " << pk << "[i];\n";
        body << "    for (int j = 1; j < " << ps << "; ++j) " << acc << " += " << pk << "[i + (long long)j * "
             << os.size() << "LL];\n";
        body << "    const " << ctype(N[o].shape.dtype) << " in" << k << " = " << round_expr(N[o].shape.dtype, acc)
             << ";\n";
        expr[o] = "in" + std::to_string(k);
        ins.push_back(in);
        ++n_partial;
        continue;
      }
      if (failed) return bad();
      View w = get(o);
      if (failed) return bad();
      In in{o, w, {}, true};
      // right-aligned implicit broadcast to os.dims
      const Shape& s = N[o].shape;
      const int off = os.rank() - s.rank();
      in.eff.assign(os.rank(), 0);
      for (int d = 0; d < s.rank(); ++d)
        if (s.dims[d] != 1) in.eff[off + d] = w.strides[d];
      auto cs = contiguous_strides(os.dims);
      for (int d = 0; d < os.rank(); ++d)
        if (os.dims[d] != 1 && in.eff[d] != cs[d]) in.linear = false;
      if (!in.linear) need_idx = true;
      const int k = static_cast<int>(ins.size());
      std::string off_e = "i";
      if (!in.linear) {
        off_e = "0";
        for (int d = 0; d < os.rank(); ++d)
          if (in.eff[d] != 0 && os.dims[d] != 1) off_e += " + " + idx_names[d] + " * " + std::to_string(in.eff[d]) + "LL";
      }
      body << "    const " << ctype(s.dtype) << " in" << k << " = "
           << load_expr(s.dtype, "((const " + stype(s.dtype) + "*)p_in" + std::to_string(k) + ")[" + off_e + "]") << ";\n";
      expr[o] = "in" + std::to_string(k);
      ins.push_back(in);
    }
    if (failed) return bad();
    if (N[u].kind == Kind::Iota) {
      const std::string name = "v" + std::to_string(u);
      body << "    const " << ctype(N[u].shape.dtype) << " " << name << " = " << round_expr(N[u].shape.dtype, iota_expr(u)) << ";\n";
      expr[u] = name;
    } else {
      body << member_stmt(u, expr, "v" + std::to_string(u));
    }
  }
  // Slots every read of which is at the output's own element index (linear,
  // offset 0, same element size): the output may overwrite them in place (a
  // donated input), so those operands and the output are not declared
  // __restrict__: with donation they are one buffer.
  std::vector<int> inplace;
  for (auto& in : ins) {
    bool ok = !in.partial;
    for (auto& o2 : ins)
      if (o2.view.slot == in.view.slot)
        ok = ok && !o2.partial && o2.linear && o2.view.offset == 0 &&
             dtype_size(N[o2.value].shape.dtype) == dtype_size(os.dtype);
    if (ok && std::find(inplace.begin(), inplace.end(), in.view.slot) == inplace.end()) inplace.push_back(in.view.slot);
  }
  auto may_alias = [&](const View& w) { return std::find(inplace.begin(), inplace.end(), w.slot) != inplace.end(); };
  std::ostringstream src;
  src << kRtcPrelude << R"(extern "C" __global__ void __launch_bounds__(256) fused(
)";
  for (size_t k = 0; k < ins.size(); ++k)
    src << "    const void* " << (may_alias(ins[k].view) ? "" : "__restrict__ ") << "p_in" << k << ",\n";
  src << "    void* " << (inplace.empty() ? "__restrict__ " : "") << "p_out, long long n) {\n";
  src << "  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long long)gridDim.x * 256) {\n";
  if (need_idx) {
    src << "    long long q = i;\n";
    for (int d = os.rank() - 1; d >= 0; --d) {
      src << "    const long long " << idx_names[d] << " = q % " << os.dims[d] << "LL;";
      if (d > 0) src << " q /= " << os.dims[d] << "LL;";
      src << "\n";
    }
  }
  src << body.str();
  src << "    ((" << stype(os.dtype) << "*)p_out)[i] = " << store_expr(os.dtype, expr[v]) << ";\n  }\n}\n";
  const std::string code = src.str();
  RtcKernel kern;
  if (rtc_get(be, code, "fused", &kern, err) != GHIP_OK) return bad();
  View y = fresh(os);
  const int64_t total = os.size();
  std::vector<int> rd;
  std::vector<View> in_views;
  std::vector<int> in_dt;
  for (auto& in : ins) {
    rd.push_back(in.view.slot);
    in_views.push_back(in.view);
    in_dt.push_back(in.partial ? GHIP_DTYPE_FLOAT32 : N[in.value].shape.dtype);
  }
  std::ostringstream d;
  d << "fused_elementwise " << os.str() << " ops=" << mem.size() << " inputs=" << ins.size() << " [";
  for (size_t i = 0; i < mem.size(); ++i) {
    const Node& n = N[mem[i]];
    d << (i ? "," : "") << kind_name(n.kind);
    if (n.kind == Kind::Unary || n.kind == Kind::Binary || n.kind == Kind::Compare) d << "#" << n.sub;
  }
  d << "]";
  if (n_partial) d << " (sums the split partials of " << n_partial << " product" << (n_partial > 1 ? "s" : "") << ")";
  const int odt = os.dtype;
  add_step(d.str(), rd, {y.slot}, [=](ExecState& st, GHipError* e) -> int {
    if (total == 0) return GHIP_OK;
    std::vector<void*> ptrs(in_views.size());
    std::vector<void*> args;
    for (size_t k = 0; k < in_views.size(); ++k) ptrs[k] = st.ptr(in_views[k], in_dt[k]);
    void* outp = st.ptr(y, odt);
    long long nn = total;
    for (size_t k = 0; k < ptrs.size(); ++k) args.push_back(&ptrs[k]);
    args.push_back(&outp);
    args.push_back(&nn);
    int64_t g = (total + 255) / 256;
    if (g > 16384) g = 16384;
    hipError_t h = hipModuleLaunchKernel(kern.func, static_cast<unsigned>(g), 1, 1, 256, 1, 1, 0, st.stream, args.data(), nullptr);
    if (h != hipSuccess) return check_hip(h, e, "generated elementwise kernel launch");
    return GHIP_OK;
  }, inplace);
  return y;
}

// Compile-time image of the run-time checks ghip_gemm_batched makes before it
// takes the bf16 MFMA path (slot bases are 256-byte aligned, so a view's base is
// 16-byte aligned iff its element offset is a multiple of 8).
static int mfma_majorness(int64_t offset, int64_t s_b, int64_t s_mn, int64_t s_k, int64_t MN, int64_t K,
                          int64_t batch) {
  if (offset % 8 != 0) return -1;
  const bool b_ok = batch == 1 || s_b % 8 == 0;
  if (s_k == 1 && K % 8 == 0 && (MN == 1 || s_mn % 8 == 0) && b_ok) return 1;
  if (s_mn == 1 && MN % 8 == 0 && (K == 1 || s_k % 8 == 0) && b_ok) return 0;
  return -1;
}

// A DotGeneral o that only the elementwise cluster being emitted reads (its
// members: inset), with 16-bit operands on the MFMA path, batch 1, o's shape the
// cluster's, and a contraction that splits: emits the GEMM step that writes o's
// fp32 partials into a fresh workspace view (*wsv, *splits ranges) and returns
// true; otherwise emits nothing of o and returns false.
bool Lowerer::emit_split_partials(int o, const Shape& os, const std::set<int>& inset, View* wsv, int* splits) {
  const Node& n = N[o];
  if (n.kind != Kind::Dot || !live[o] || have[o] || fusion[o].kind != Fusion::None || n.shape.dims != os.dims)
    return false;
  for (int r : fn->outputs)
    if (r == o) return false;
  for (int w : users[o])
    if (!inset.count(w)) return false;
  const int dt = N[n.in[0]].shape.dtype, odt = n.shape.dtype;
  if ((dt != GHIP_DTYPE_BFLOAT16 && dt != GHIP_DTYPE_FLOAT16) || N[n.in[1]].shape.dtype != dt) return false;
  if (odt != dt && odt != GHIP_DTYPE_FLOAT32) return false;
  DotPlan d;
  if (!plan_dot(o, false, &d)) return false;
  if (d.B != 1 || d.M <= 0 || d.N <= 0 || d.K <= 0) return false;
  const int64_t wsb = ghip_gemm_workspace_bytes(dt, odt, 1, d.M, d.N, d.K);
  if (wsb <= 0 || d.sam < 0 || d.sak < 0 || d.sbk < 0 || d.sbn < 0) return false;
  if (mfma_majorness(d.lv.offset, 0, d.sam, d.sak, d.M, d.K, 1) < 0 ||
      mfma_majorness(d.rv.offset, 0, d.sbn, d.sbk, d.N, d.K, 1) < 0)
    return false;
  if (!gemm_rows_fit(d.sam, d.sak, 2) || !gemm_rows_fit(d.sbn, d.sbk, 2)) return false;
  const int64_t ea = ((d.M - 1) * d.sam + (d.K - 1) * d.sak + 1) * 2;
  const int64_t eb = ((d.N - 1) * d.sbn + (d.K - 1) * d.sbk + 1) * 2;
  if (ea >= (int64_t{1} << 31) || eb >= (int64_t{1} << 31)) return false;
  const int S = gemm_k_split(1, d.M, d.N, d.K, 2).s;
  Shape wss;
  wss.dtype = GHIP_DTYPE_FLOAT32;
  wss.dims = {(wsb + 3) / 4};
  const View w = fresh(wss);
  const View lv = d.lv, rv = d.rv;
  const int64_t M = d.M, N_ = d.N, K = d.K, sam = d.sam, sak = d.sak, sbk = d.sbk, sbn = d.sbn;
  add_step(fmt("gemm_split_partials %s M=%lld N=%lld K=%lld (%s; a strides m=%lld k=%lld, b strides k=%lld n=%lld; "
               "contraction split in %d, summed by the consumer)",
               dtype_name(dt), (long long)M, (long long)N_, (long long)K, d.how.c_str(), (long long)sam,
               (long long)sak, (long long)sbk, (long long)sbn, S),
           {lv.slot, rv.slot}, {w.slot}, [=](ExecState& st, GHipError* e) {
             return gemm_split_partials(dt, M, N_, K, st.ptr(lv, dt), sam, sak, st.ptr(rv, dt), sbk, sbn,
                                        reinterpret_cast<float*>(st.ptr(w, GHIP_DTYPE_FLOAT32)), wsb, S, st.stream, e);
           });
  *wsv = w;
  *splits = S;
  return true;
}

View Lowerer::emit_gemm_epilogue(int v, const std::vector<int>& mem, bool* fused) {
  *fused = false;
  const Shape& os = N[v].shape;
  std::set<int> inset(mem.begin(), mem.end());
  std::set<int> outs(fn->outputs.begin(), fn->outputs.end());
  // Dot inputs, in first-use order.
  std::vector<int> dots;
  for (int u : mem) {
    if (N[u].kind == Kind::Iota) return View{};
    for (int o : N[u].in)
      if (o >= 0 && !inset.count(o) && N[o].kind == Kind::Dot &&
          std::find(dots.begin(), dots.end(), o) == dots.end())
        dots.push_back(o);
  }
  if (dots.empty() || dots.size() > 2) return View{};
  for (int d : dots) {
    const Node& n = N[d];
    if (!live[d] || have[d] || outs.count(d) || fusion[d].kind != Fusion::None) return View{};
    if (n.shape.dims != os.dims) return View{};
    for (int w : users[d])
      if (!inset.count(w)) return View{};
    if (N[n.in[0]].shape.dtype != GHIP_DTYPE_BFLOAT16 || N[n.in[1]].shape.dtype != GHIP_DTYPE_BFLOAT16) return View{};
    if (n.shape.dtype != GHIP_DTYPE_BFLOAT16 && n.shape.dtype != GHIP_DTYPE_FLOAT32) return View{};
  }
  if (dots.size() == 2) {
    const Node& a = N[dots[0]];
    const Node& b = N[dots[1]];
    if (a.in[0] != b.in[0] || a.shape.dtype != b.shape.dtype || N[a.in[1]].shape.dims != N[b.in[1]].shape.dims ||
        a.a0 != b.a0 || a.a1 != b.a1 || a.a2 != b.a2 || a.a3 != b.a3)
      return View{};
  }
  const int NB = static_cast<int>(dots.size());
  DotPlan dp[2];
  for (int k = 0; k < NB; ++k) {
    if (!plan_dot(dots[k], false, &dp[k])) return View{};  // (failed is checked by the caller)
  }
  const DotPlan& d = dp[0];
  if (NB == 2 && (dp[1].sbb != d.sbb || dp[1].sbk != d.sbk || dp[1].sbn != d.sbn)) return View{};
  // A product the stand-alone GEMM step would run with its contraction split stays
  // unfused (the split's fp32 partials are summed by a kernel of their own, which
  // the generated epilogue kernel does not reproduce).
  if (ghip_gemm_workspace_bytes(GHIP_DTYPE_BFLOAT16, N[dots[0]].shape.dtype, d.B, d.M, d.N, d.K) > 0) return View{};
  // The bf16 MFMA path's operand conditions, decided here because the fused
  // kernel has no generic fallback.
  if (d.B > 65535 || d.M == 0 || d.N == 0 || d.K == 0) return View{};
  if (d.sab < 0 || d.sam < 0 || d.sak < 0 || d.sbb < 0 || d.sbk < 0 || d.sbn < 0) return View{};
  const int ma = mfma_majorness(d.lv.offset, d.sab, d.sam, d.sak, d.M, d.K, d.B);
  int mb = mfma_majorness(d.rv.offset, d.sbb, d.sbn, d.sbk, d.N, d.K, d.B);
  if (NB == 2 && mfma_majorness(dp[1].rv.offset, d.sbb, d.sbn, d.sbk, d.N, d.K, d.B) != mb) mb = -1;
  if (ma < 0 || mb < 0) return View{};
  const int64_t ea = ((d.M - 1) * d.sam + (d.K - 1) * d.sak + 1) * 2;
  const int64_t eb = ((d.N - 1) * d.sbn + (d.K - 1) * d.sbk + 1) * 2;
  if (!gemm_rows_fit(d.sam, d.sak, 2) || !gemm_rows_fit(d.sbn, d.sbk, 2)) return View{};
  // Operand slices of 2 GiB or more: the cores' 64-bit-records form (BIG).
  const bool big = ea >= (int64_t{1} << 31) || eb >= (int64_t{1} << 31);
  const char* big_arg = big ? ", true" : "";

  // Extra operands: each must fold to one stride per (batch, m, n) group of the
  // output dims [batch (nbatch), lhs free (nlfree), rhs free].
  std::vector<int64_t> gb, gm, gn;
  for (int i = 0; i < os.rank(); ++i)
    (i < d.nbatch ? gb : i < d.nbatch + d.nlfree ? gm : gn).push_back(i);
  struct In {
    View view;
    int dt;
    int64_t sb, sm, sn;
    bool vin;  // 4-element vector loads: unit n stride, rows and base 4-element aligned
  };
  std::vector<In> ins;
  std::map<int, std::string> expr;
  // The GEMM stages each product in the Dot's own dtype (bf16 bits, or fp32), so
  // the value read back is exactly what the stand-alone Dot would have stored.
  const int dot_dt = N[dots[0]].shape.dtype;
  const bool stage_bf16 = dot_dt == GHIP_DTYPE_BFLOAT16;
  const int CH = stage_bf16 ? 8 : 4;  // outputs per epilogue call (16 staged bytes)
  for (int k = 0; k < NB; ++k) expr[dots[k]] = stage_bf16 ? (k == 0 ? "bf2f(acc0[e])" : "bf2f(acc1[e])")
                                                           : (k == 0 ? "acc0[e]" : "acc1[e]");
  std::ostringstream body;
  for (size_t ui = 0; ui < mem.size(); ++ui) {
    const int u = mem[ui];
    for (int o : N[u].in) {
      if (o < 0 || inset.count(o) || expr.count(o)) continue;
      double c;
      if (scalar_const(o, &c) && (dtype_is_float(N[o].shape.dtype) || fabs(c) < 9007199254740992.0)) {
        expr[o] = literal(N[o].shape.dtype, c);
        continue;
      }
      if (N[o].kind == Kind::Iota || static_cast<int>(ins.size()) == kEpiMaxIn) return View{};
      View w = get(o);
      if (failed) return View{};
      const Shape& s = N[o].shape;
      View eff;
      eff.slot = w.slot;
      eff.offset = w.offset;
      eff.strides.assign(os.rank(), 0);
      const int off = os.rank() - s.rank();
      for (int i = 0; i < s.rank(); ++i)
        if (s.dims[i] != 1) eff.strides[off + i] = w.strides[i];
      In in{w, s.dtype, 0, 0, 0, false};
      int64_t sz;
      if (!merge(os, eff, gb, &sz, &in.sb) || !merge(os, eff, gm, &sz, &in.sm) || !merge(os, eff, gn, &sz, &in.sn))
        return View{};
      in.vin = in.sn == 1 && (in.sm % CH == 0 || d.M == 1) && (in.sb % CH == 0 || d.B == 1) && w.offset % CH == 0;
      const int k = static_cast<int>(ins.size());
      const std::string ks = std::to_string(k);
      body << "      const " << ctype(s.dtype) << " in" << ks << " = " << load_expr(s.dtype, "pr.x" + ks + "[e]") << ";\n";
      expr[o] = "in" + ks;
      ins.push_back(in);
    }
    body << "  " << member_stmt(u, expr, "t" + std::to_string(ui));
  }

  // Tile shape: the precompiled kernels' choice for one operand; with two, a
  // 256 x (2 x 128) tile does the MMA work of one 256 x 256 tile.
  int BM = 128, BN = 128, WM = 2, WN = 2;
  bool four_wave = false;
  const int64_t t256 = d.B * ((d.M + 255) / 256) * ((d.N + 255) / 256);
  // A VALU-heavy epilogue (transcendentals, long chains) runs faster on an 8-wave
  // core: with one wave per SIMD a wave issues a VALU instruction every few cycles,
  // with two the SIMD's VALU stays busy (FusedDense + tanh-GELU: 894 -> 953 TFLOP/s
  // against the 4-wave core), while the 4-wave MN-contiguous core's main loop is a
  // few percent faster for light epilogues.
  int valu_weight = 0;
  for (int u : mem) {
    const Node& n = N[u];
    valu_weight += 1;
    if (n.kind == Kind::Unary &&
        (n.sub == GHIP_UNARY_EXP || n.sub == GHIP_UNARY_EXPM1 || n.sub == GHIP_UNARY_LOG ||
         n.sub == GHIP_UNARY_LOG1P || n.sub == GHIP_UNARY_SIN || n.sub == GHIP_UNARY_COS ||
         n.sub == GHIP_UNARY_TANH || n.sub == GHIP_UNARY_LOGISTIC || n.sub == GHIP_UNARY_ERF ||
         n.sub == GHIP_UNARY_SQRT || n.sub == GHIP_UNARY_RSQRT))
      valu_weight += 6;
  }
  const bool heavy_epilogue = valu_weight >= 8;
  // Otherwise A K-contiguous, B MN-contiguous: the 8-wave 32-deep core.  Other
  // layouts: the 8-wave 64-deep 16x16x32 core, except both operands MN-contiguous
  // with a light epilogue (4-wave 32-deep core).
  //
  // A K-, B MN-contiguous grids of >= 128 tiles with a light epilogue, or two
  // products: the 4-wave core (128 x 128 waves, one per SIMD, a third fewer LDS
  // reads per MFMA; on the block's residual and SwiGLU epilogues 2.5% faster than
  // the 8-wave core under sustained load).  A VALU-heavy epilogue of one product
  // (FusedDense + tanh-GELU) stays on the 8-wave core (4% faster there).
  //
  // One product on a grid of at most 128 256 x 256 tiles: the 128 x 128 core (two
  // workgroups per CU), as the precompiled GEMMs do (a 256 x 256 grid that small
  // leaves half the CUs or more idle).
  bool eight_km = false, eight_x = false, four_km = false;
  const int64_t t4 = d.B * ((d.M + 255) / 256) * ((d.N + 256 / NB - 1) / (256 / NB));
  if (ma && !mb && d.M >= 256 && d.N >= 256 / NB && (NB == 2 || !heavy_epilogue) && (NB == 2 ? t4 >= 128 : t4 > 128)) {
    BM = 256, BN = 256 / NB, WM = 2, WN = 2, four_km = true;
  } else if (NB == 1) {
    if (d.M >= 256 && d.N >= 256 && t256 > 128 && ma && !mb) BM = 256, BN = 256, WM = 2, WN = 4, eight_km = true;
    else if (d.M >= 256 && d.N >= 256 && t256 > 128 && (mb || heavy_epilogue))
      BM = 256, BN = 256, WM = 2, WN = 4, eight_x = true;
    else if (d.M >= 256 && d.N >= 256 && t256 > 128) BM = 256, BN = 256, WM = 2, WN = 2, four_wave = true;
  } else if (d.M >= 256 && d.N >= 128) {
    BM = 256, BN = 128, WM = 2, WN = 4;
    eight_km = ma && !mb && d.B * ((d.M + 255) / 256) * ((d.N + 127) / 128) >= 128;
    eight_x = !eight_km;
  }
  const int nt = WM * WN * 64;
  const int odt = os.dtype;
  std::ostringstream src;
  src << kGemmDevSrc << "\n" << kRtcPrelude;
  // Pre: the CH raw elements of each extra operand for one call (one row chunk),
  // loaded by prefetch() ahead of the stores of the previous chunk.  FULL: the
  // tile lies inside the output, so no column bounds checks.
  const bool vec = d.N % CH == 0;
  const std::string CHs = std::to_string(CH);
  src << "namespace ghip {\nstruct GenEpi {\n  using Stage = " << (stage_bf16 ? "unsigned short" : "float") << ";\n"
      << "  __device__ __forceinline__ static Stage stage(float v) { return " << (stage_bf16 ? "f2bf(v)" : "v")
      << "; }\n  struct Pre {";
  for (size_t k = 0; k < ins.size(); ++k) src << " " << stype(ins[k].dt) << " x" << k << "[" << CH << "];";
  src << " };\n  EpiArgs a;\n"
      << "  template <bool FULL>\n"
      << "  __device__ __forceinline__ void prefetch(int64_t bb, int64_t m, int64_t n, Pre& pr) const {\n";
  for (size_t k = 0; k < ins.size(); ++k) {
    const std::string T = stype(ins[k].dt), ks = std::to_string(k);
    const int vbytes = std::min(CH * dtype_size(ins[k].dt), 16);
    src << "    {\n      const " << T << "* src = (const " << T << "*)a.in[" << ks << "] + bb * a.s_b[" << ks
        << "] + m * a.s_m[" << ks << "] + n * a.s_n[" << ks << "];\n";
    if (ins[k].vin)
      src << "      if (FULL || n + " << CH - 1 << " < a.N) {\n"
          << "        struct __attribute__((aligned(" << vbytes << "))) V { " << T << " x[" << CHs << "]; };\n"
          << "        const V w = *(const V*)src;\n"
          << "#pragma unroll\n        for (int e = 0; e < " << CHs << "; ++e) pr.x" << ks << "[e] = w.x[e];\n"
          << "      } else {\n";
    else
      src << "      {\n";
    src << "#pragma unroll\n        for (int e = 0; e < " << CHs << "; ++e) pr.x" << ks << "[e] = (FULL || n + e < a.N) ? src[e * a.s_n[" << ks
        << "]] : (" << T << ")0;\n      }\n    }\n";
  }
  src << "  }\n"
      << "  template <bool FULL>\n"
      << "  __device__ __forceinline__ void store(int64_t bb, int64_t m, int64_t n, const Stage* acc0,\n"
      << "                                        const Stage* acc1, const Pre& pr) const {\n"
      << "    " << ctype(odt) << " r[" << CH << "];\n"
      << "#pragma unroll\n    for (int e = 0; e < " << CHs << "; ++e) {\n      const int64_t nn = n + e;\n"
      << "      if (!FULL && nn >= a.N) { r[e] = 0; continue; }\n"
      << body.str()
      << "      r[e] = " << expr[v] << ";\n    }\n"
      << "    " << stype(odt) << "* o = (" << stype(odt) << "*)a.out + bb * a.so_b + m * a.so_m + n;\n";
  if (vec) {
    const int obytes = std::min(CH * dtype_size(odt), 16);
    src << "    if (FULL || n + " << CH - 1 << " < a.N) {\n"
        << "      struct __attribute__((aligned(" << obytes << "))) V { " << stype(odt) << " x[" << CHs << "]; } w;\n"
        << "#pragma unroll\n      for (int e = 0; e < " << CHs << "; ++e) w.x[e] = " << store_expr(odt, "r[e]") << ";\n"
        << "      *(V*)o = w;\n      return;\n    }\n";
  }
  src << "#pragma unroll\n    for (int e = 0; e < " << CHs << "; ++e)\n      if (FULL || n + e < a.N) o[e] = " << store_expr(odt, "r[e]")
      << ";\n  }\n};\n}  // namespace ghip\n";
  src << "extern \"C\" __global__ void __launch_bounds__(" << nt << ", 1) gemm_epilogue(ghip::GemmParams p, ghip::EpiArgs a) {\n"
      << "  const ghip::GenEpi epi{a};\n";
  if (four_km)
    src << "  ghip::gemm_bf16_body4km<ghip::GenEpi, false, " << NB << big_arg << ">(p, epi);\n}\n";
  else if (eight_km)
    src << "  ghip::gemm_bf16_body8km<ghip::GenEpi, false, " << NB << big_arg << ">(p, epi);\n}\n";
  else if (eight_x)
    src << "  ghip::gemm_bf16_body8x<" << (ma ? "true" : "false") << ", " << (mb ? "true" : "false")
        << ", ghip::GenEpi, false, " << NB << big_arg << ">(p, epi);\n}\n";
  else if (four_wave)
    src << "  ghip::gemm_bf16_body4mn<ghip::GenEpi, false" << big_arg << ">(p, epi);\n}\n";
  else
    src << "  ghip::gemm_bf16_body<" << BM << ", " << BN << ", " << WM << ", " << WN << ", " << (ma ? "true" : "false") << ", "
        << (mb ? "true" : "false") << ", " << NB << ", ghip::GenEpi, false" << big_arg << ">(p, epi);\n}\n";
  RtcKernel kern;
  if (rtc_get(be, src.str(), "gemm_epilogue", &kern, err) != GHIP_OK) {
    failed = true;
    return View{};
  }

  View y = fresh(os);
  GemmParams gp{};
  gp.sa_b = d.sab; gp.sa_m = d.sam; gp.sa_k = d.sak;
  gp.sb_b = d.sbb; gp.sb_k = d.sbk; gp.sb_n = d.sbn;
  gp.batch = d.B; gp.M = d.M; gp.N = d.N; gp.K = d.K;
  gp.tiles_m = static_cast<int>((d.M + BM - 1) / BM);
  gp.tiles_n = static_cast<int>((d.N + BN - 1) / BN);
  gp.a_extent = big ? 0u : static_cast<uint32_t>(ea);
  gp.b_extent = big ? 0u : static_cast<uint32_t>(eb);
  gp.a_extent64 = ea;
  gp.b_extent64 = eb;
  const int64_t blocks = d.B * gp.tiles_m * gp.tiles_n;
  const int64_t so_b = d.M * d.N, so_m = d.N;
  const View lv = d.lv, rv0 = d.rv, rv1 = dp[NB - 1].rv;
  std::vector<int> rd{lv.slot, rv0.slot};
  if (NB == 2) rd.push_back(rv1.slot);
  for (auto& in : ins) rd.push_back(in.view.slot);
  std::ostringstream desc;
  // core: waves and k-depth of the main loop (km32: A in 64-deep, B in 32-deep stages)
  const char* core = four_km ? "4w-km32" : eight_km ? "8w-km32" : eight_x ? "8w-k64" : four_wave ? "4w-mn32" : "small";
  desc << fmt("gemm_batched+epilogue bf16 B=%lld M=%lld N=%lld K=%lld dots=%d tile=%dx%d waves=%d core=%s (%s) ops=%zu "
              "inputs=%zu [",
              (long long)d.B, (long long)d.M, (long long)d.N, (long long)d.K, NB, BM, BN * NB, WM * WN, core,
              d.how.c_str(), mem.size(), ins.size());
  for (size_t i = 0; i < mem.size(); ++i) {
    const Node& n = N[mem[i]];
    desc << (i ? "," : "") << kind_name(n.kind);
    if (n.kind == Kind::Unary || n.kind == Kind::Binary || n.kind == Kind::Compare) desc << "#" << n.sub;
  }
  desc << "]";
  add_step(desc.str(), rd, {y.slot}, [=](ExecState& st, GHipError* e) -> int {
    GemmParams p = gp;
    p.a = st.ptr(lv, GHIP_DTYPE_BFLOAT16);
    p.b = st.ptr(rv0, GHIP_DTYPE_BFLOAT16);
    p.b1 = st.ptr(rv1, GHIP_DTYPE_BFLOAT16);
    p.c = st.ptr(y, odt);
    if ((reinterpret_cast<uintptr_t>(p.a) | reinterpret_cast<uintptr_t>(p.b) | reinterpret_cast<uintptr_t>(p.b1)) & 15u)
      return set_error(e, GHIP_ERR_STATE, "fused GEMM epilogue: operand base not 16-byte aligned");
    EpiArgs a{};
    for (size_t k = 0; k < ins.size(); ++k) {
      const int es = dtype_size(ins[k].dt);
      a.in[k] = st.ptr(ins[k].view, ins[k].dt);
      a.s_b[k] = ins[k].sb;
      a.s_m[k] = ins[k].sm;
      a.s_n[k] = ins[k].sn;
      a.vin[k] = ins[k].vin;
      const int va = std::min(CH * es, 16);
      if (ins[k].vin && reinterpret_cast<uintptr_t>(a.in[k]) % va != 0)
        return set_error(e, GHIP_ERR_STATE, "fused GEMM epilogue: operand %zu not %d-byte aligned", k, va);
    }
    a.out = p.c;
    a.so_b = so_b;
    a.so_m = so_m;
    a.N = p.N;
    a.vec = vec;
    if (vec && reinterpret_cast<uintptr_t>(p.c) % std::min(CH * dtype_size(odt), 16) != 0)
      return set_error(e, GHIP_ERR_STATE, "fused GEMM epilogue: output not aligned for %d-element stores", CH);
    void* args[] = {&p, &a};
    hipError_t h = hipModuleLaunchKernel(kern.func, static_cast<unsigned>(blocks), 1, 1, nt, 1, 1, 0, st.stream, args,
                                         nullptr);
    if (h != hipSuccess) return check_hip(h, e, "fused GEMM epilogue launch");
    return GHIP_OK;
  });
  for (int k = 0; k < NB; ++k) have[dots[k]] = 1;  // consumed here; never materialised
  *fused = true;
  return y;
}

int Lowerer::finish() {
  // Outputs: reuse the producing arena slot when the value is a dense,
  // exclusively-owned buffer; otherwise copy into a fresh output slot.
  std::set<int> converted;
  const int nout = static_cast<int>(fn->outputs.size());
  plan->out_slot.assign(nout, -1);
  for (int i = 0; i < nout; ++i) {
    const int v = fn->outputs[i];
    View w = get(v);
    if (failed) return err ? err->code : GHIP_ERR_STATE;
    const Shape& s = N[v].shape;
    Slot& sl = plan->slots[w.slot];
    if (sl.kind == SlotKind::Arena && w.offset == 0 && w.contiguous(s) && sl.bytes == s.bytes() && !converted.count(w.slot)) {
      sl.kind = SlotKind::Output;
      sl.index = i;
      converted.insert(w.slot);
      plan->out_slot[i] = w.slot;
    } else {
      View o = contig(new_slot(SlotKind::Output, s.bytes(), i), s);
      emit_copy(s, w, o, "(copy to output)");
      plan->out_slot[i] = o.slot;
    }
  }
  // Arena: first-fit offsets over [first write, last use] step intervals.
  const int ns = static_cast<int>(plan->slots.size());
  std::vector<int> first(ns, INT32_MAX), last(ns, -1);
  for (size_t st = 0; st < plan->steps.size(); ++st) {
    for (int s : writes[st]) { first[s] = std::min(first[s], static_cast<int>(st)); last[s] = std::max(last[s], static_cast<int>(st)); }
    for (int s : reads[st]) { first[s] = std::min(first[s], static_cast<int>(st)); last[s] = std::max(last[s], static_cast<int>(st)); }
  }
  std::vector<int> order;
  for (int s = 0; s < ns; ++s)
    if (plan->slots[s].kind == SlotKind::Arena && last[s] >= 0) order.push_back(s);
  std::sort(order.begin(), order.end(), [&](int a, int b) { return plan->slots[a].bytes > plan->slots[b].bytes; });
  struct Placed { size_t off, end; int first, last; };
  std::vector<Placed> placed;
  size_t arena = 0;
  for (int s : order) {
    const size_t sz = (plan->slots[s].bytes + 255) & ~size_t(255);
    std::vector<std::pair<size_t, size_t>> busy;
    for (auto& p : placed)
      if (!(p.last < first[s] || last[s] < p.first)) busy.emplace_back(p.off, p.end);
    std::sort(busy.begin(), busy.end());
    size_t off = 0;
    for (auto& b : busy) {
      if (off + sz <= b.first) break;
      off = std::max(off, b.second);
    }
    plan->slots[s].arena_off = off;
    placed.push_back(Placed{off, off + sz, first[s], last[s]});
    arena = std::max(arena, off + sz);
  }
  plan->arena_bytes = arena;
  // Donation: last read of each input, first write of each output, and per step
  // the inputs an elementwise step reads at its output's own element index.
  const int nin = static_cast<int>(fn->params.size() + fn->captures.size());
  plan->in_last_read.assign(nin, -1);
  plan->out_first_write.assign(nout, INT32_MAX);
  plan->inplace_inputs.assign(plan->steps.size(), {});
  for (size_t st = 0; st < plan->steps.size(); ++st) {
    for (int s : reads[st])
      if (plan->slots[s].kind == SlotKind::Input)
        plan->in_last_read[plan->slots[s].index] = std::max(plan->in_last_read[plan->slots[s].index], static_cast<int>(st));
    for (int s : writes[st])
      if (plan->slots[s].kind == SlotKind::Output)
        plan->out_first_write[plan->slots[s].index] = std::min(plan->out_first_write[plan->slots[s].index], static_cast<int>(st));
    for (int s : inplace_slots[st])
      if (plan->slots[s].kind == SlotKind::Input) plan->inplace_inputs[st].push_back(plan->slots[s].index);
  }
  for (auto& st : plan->steps) plan->log.push_back(st.desc);
  return GHIP_OK;
}

}  // namespace

int lower(GHipBackend* be, GHipFunction* fn, Plan* plan, GHipError* err) {
  Lowerer L(be, fn, plan, err);
  // GHIP_EPILOGUE_FUSION=0 keeps every DotGeneral a stand-alone GEMM (the
  // unfused plan the fused one is checked against).
  const char* ef = getenv("GHIP_EPILOGUE_FUSION");
  L.fuse_epilogues = !(ef && ef[0] == '0');
  const char* rf = getenv("GHIP_REDUCE_FUSION");
  L.fuse_reductions = !(rf && rf[0] == '0');
  // GHIP_DOT_GROUPING=0 keeps DotGenerals that share a left operand separate.
  const char* gf = getenv("GHIP_DOT_GROUPING");
  L.group_dots = !(gf && gf[0] == '0');
  L.have.assign(fn->nodes.size(), 0);
  L.views.assign(fn->nodes.size(), View{});
  L.analyse();
  int rc = L.finish();
  if (rc != GHIP_OK) return rc;
  // Const payloads travel with the plan (uploaded by Compile).
  plan->const_data = std::move(L.const_data);
  return GHIP_OK;
}

}  // namespace ghip
