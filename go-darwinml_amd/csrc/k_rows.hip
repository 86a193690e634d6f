// Row kernels: softmax / log-softmax, attention-score softmax (scale + causal /
// boolean mask), RMSNorm and LayerNorm over the last axis.
//
// All of them are HBM-bound: one read of x, one write of y (plus a [n] parameter
// vector that stays in L2).  The fast path keeps a whole row in registers, so x is
// read from HBM exactly once:
//   * a row is split into 16-byte vectors; vector v of lane l covers elements
//     [(v*L + l)*VEC, +VEC) where L is the number of lanes on the row, so each
//     vector step of a wave touches one contiguous 1 KiB span (fully coalesced
//     128-bit loads/stores);
//   * a row is spread over WPR = 1, 2 or 4 waves so that each lane holds about
//     four 16-byte vectors (kept packed; widened to fp32 as they are used):
//     short per-lane work and many waves in flight keep more requests in the
//     memory system than one long row per wave;
//   * x and y move with nontemporal loads/stores (they are touched once), so they
//     do not evict the L2 / Infinity Cache lines that gamma/beta live in;
//     measured on MI355X this lifts e.g. RMSNorm bf16 [8192, 4096] from 50% to
//     67% of the 8 TB/s HBM peak;
//   * WPR > 1 combines the per-wave partial sums through LDS (one barrier per
//     reduction);
//   * anything else (unaligned rows, n not a multiple of the vector width, or
//     rows beyond the register budget) takes a generic multi-pass kernel.
// Statistics are fp32 for fp32, bf16 and f16 I/O.
#include <stdarg.h>

#include <atomic>
#include <type_traits>

#include "common.h"

namespace ghip {

enum RowOp { kSoftmax = 0, kLogSoftmax = 1, kRmsNorm = 2, kLayerNorm = 3, kMaskedSoftmax = 4 };

struct RowParams {
  // The fields every kernel reads first, adjacent (one scalar load fetches them).
  const void* x;
  void* y;
  int64_t rows;
  int64_t n;
  const void* gamma;
  const void* beta;
  // kMaskedSoftmax: a boolean keep-mask (uint8) or an additive mask in the
  // scores' dtype, addressed as mask + b m_sb + h m_sh + q m_sq + key m_sk for row
  // (b, h, q) of the [B, H, Sq, Sk] scores (strides 0 where it broadcasts).
  const void* mask;
  int mask_kind;         // 0 none, 1 keep-mask, 2 additive
  int64_t m_sb, m_sh, m_sq, m_sk;
  int64_t sq;            // rows per attention matrix (kMaskedSoftmax)
  int64_t heads;         // H (kMaskedSoftmax)
  float eps;
  float scale;
  int causal;
};

typedef unsigned u32x4_nt __attribute__((ext_vector_type(4)));

// 16-byte nontemporal load / store of packed elements.
__device__ __forceinline__ uint4 ld_nt(const void* p) {
  const u32x4_nt v = __builtin_nontemporal_load(static_cast<const u32x4_nt*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void st_nt(void* p, uint4 v) {
  const u32x4_nt w = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(w, static_cast<u32x4_nt*>(p));
}

// Packed 16-byte vector <-> fp32 values.
__device__ __forceinline__ void unpack(const uint4& r, float* f, float) {
  f[0] = __uint_as_float(r.x); f[1] = __uint_as_float(r.y);
  f[2] = __uint_as_float(r.z); f[3] = __uint_as_float(r.w);
}
__device__ __forceinline__ void unpack(const uint4& r, float* f, bf16_t) {
  const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(w[i] << 16);
    f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}
__device__ __forceinline__ void unpack(const uint4& r, float* f, f16_t) {
  const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = f16_to_f32(static_cast<uint16_t>(w[i]));
    f[2 * i + 1] = f16_to_f32(static_cast<uint16_t>(w[i] >> 16));
  }
}
__device__ __forceinline__ uint4 pack(const float* f, float) {
  return make_uint4(__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]),
                    __float_as_uint(f[3]));
}
__device__ __forceinline__ uint4 pack(const float* f, bf16_t) {
  return make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]),
                    pack_bf16x2(f[6], f[7]));
}
__device__ __forceinline__ uint4 pack(const float* f, f16_t) {
  return make_uint4(pack_f16x2(f[0], f[1]), pack_f16x2(f[2], f[3]), pack_f16x2(f[4], f[5]),
                    pack_f16x2(f[6], f[7]));
}

// Sum / max over the WPR waves of a row (slot: which LDS pair to use, so two
// back-to-back reductions need no extra barrier).
template <int WPR>
__device__ __forceinline__ float row_reduce_sum(float v, float (*lds)[4], int slot) {
  v = wave_sum(v);
  if constexpr (WPR == 1) {
    return v;
  } else {
    const int w = threadIdx.x / kWave;
    const int first = (w / WPR) * WPR;
    if ((threadIdx.x % kWave) == 0) lds[slot][w] = v;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < WPR; ++i) t += lds[slot][first + i];
    return t;
  }
}
template <int WPR>
__device__ __forceinline__ float row_reduce_max(float v, float (*lds)[4], int slot) {
  v = wave_max(v);
  if constexpr (WPR == 1) {
    return v;
  } else {
    const int w = threadIdx.x / kWave;
    const int first = (w / WPR) * WPR;
    if ((threadIdx.x % kWave) == 0) lds[slot][w] = v;
    __syncthreads();
    float t = lds[slot][first];
#pragma unroll
    for (int i = 1; i < WPR; ++i) t = fmaxf(t, lds[slot][first + i]);
    return t;
  }
}

// Row statistics of RMSNorm (mean 0, rstd = 1/sqrt(mean(x^2) + eps)) or
// LayerNorm (mean, rstd = 1/sqrt(var + eps)) from the row values of the calling
// lanes: xget(i, f) gives vector i as fp32 (live[i]: vector i lies on the row).
template <typename T, int OP, int NV, int WPR, typename XG>
__device__ __forceinline__ void norm_stats(XG xget, const bool (&live)[NV], int64_t n, float eps, float (*lds)[4],
                                           float& mean, float& rstd) {
  // Contraction only within one expression (s += x * x is one fma; a product is
  // never fused into a later statement's sum): otherwise the backend may fuse
  // either product of x0*x0 + x1*x1, and the two norm kernels (which must give
  // identical results for a row whichever of them runs it) would round
  // differently.
#pragma clang fp contract(on)
  constexpr int VEC = Elem<T>::kVec;
  const float inv_n = 1.0f / static_cast<float>(n);
  mean = 0.f;
  if constexpr (OP == kLayerNorm && WPR > 1) {
    // Each wave reduces its part of the row to (count, mean, M2) in registers
    // and one LDS exchange combines the WPR parts (Chan, Golub and LeVeque's
    // pairwise update: M2 = sum M2_w + n_w (mean_w - mean)^2), instead of a
    // reduction for the mean followed by a second one for the variance.
    float cnt = 0.f, sw = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      if (!live[i]) continue;
      float f[VEC];
      xget(i, f);
      cnt += VEC;
#pragma unroll
      for (int j = 0; j < VEC; ++j) sw += f[j];
    }
    cnt = wave_sum(cnt);
    sw = wave_sum(sw);
    const float mw = cnt > 0.f ? sw / cnt : 0.f;
    float qw = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      if (!live[i]) continue;
      float f[VEC];
      xget(i, f);
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        const float d = f[j] - mw;
        qw += d * d;
      }
    }
    qw = wave_sum(qw);
    const int w = threadIdx.x / kWave, first = (w / WPR) * WPR;
    if ((threadIdx.x % kWave) == 0) {
      lds[0][w] = cnt;
      lds[1][w] = mw;
      lds[2][w] = qw;
    }
    __syncthreads();
    float sum = 0.f;
#pragma unroll
    for (int k = 0; k < WPR; ++k) sum += lds[0][first + k] * lds[1][first + k];
    mean = sum * inv_n;
    float m2 = 0.f;
#pragma unroll
    for (int k = 0; k < WPR; ++k) {
      const float d = lds[1][first + k] - mean;
      m2 += lds[2][first + k] + lds[0][first + k] * d * d;
    }
    rstd = rsqrtf(m2 * inv_n + eps);
  } else {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      float f[VEC];
      xget(i, f);
#pragma unroll
      for (int j = 0; j < VEC; ++j) s += (OP == kRmsNorm) ? f[j] * f[j] : f[j];
    }
    s = row_reduce_sum<WPR>(s, lds, 0);
    if constexpr (OP == kRmsNorm) {
      rstd = rsqrtf(s * inv_n + eps);
    } else {
      mean = s * inv_n;
      float q = 0.f;
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        if (!live[i]) continue;
        float f[VEC];
      xget(i, f);
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
          const float d = f[j] - mean;
          q += d * d;
        }
      }
      q = row_reduce_sum<WPR>(q, lds, 1);
      rstd = rsqrtf(q * inv_n + eps);
    }
  }
}

// Store pass of the norms: y = (x - mean) * rstd [* gamma] [+ beta], one copy per
// (gamma, beta) presence (tested per element, the uniform pointer checks became a
// select per value); gfetch / bfetch(i, c0, out) supply vector i of gamma / beta.
template <typename T, int NV, int LANES, typename XG, typename HG, typename HB, typename GF, typename BF>
__device__ __forceinline__ void norm_store(XG xget, const bool (&live)[NV], float mean, float rstd, T* yr, int l, HG,
                                           HB, GF gfetch, BF bfetch) {
#pragma clang fp contract(on)
  constexpr int VEC = Elem<T>::kVec;
  constexpr bool G = HG::value, B = HB::value;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t c0 = (static_cast<int64_t>(i) * LANES + l) * VEC;
    if (!live[i]) continue;
    float x[VEC], f[VEC], gv[VEC], bv[VEC];
    xget(i, x);
    if constexpr (G) gfetch(i, c0, gv);
    if constexpr (B) bfetch(i, c0, bv);
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const float t = (x[j] - mean) * rstd;
      if constexpr (G && B) f[j] = fmaf(t, gv[j], bv[j]);
      else if constexpr (G) f[j] = t * gv[j];
      else if constexpr (B) f[j] = t + bv[j];
      else f[j] = t;
    }
    st_nt(yr + c0, pack(f, T{}));
  }
}

// One row per WPR waves; a 256-thread workgroup handles 4 / WPR rows (row group
// `blk`).  NV packed 16-byte vectors per lane.
template <typename T, int OP, int NV, int WPR>
__device__ __forceinline__ void rows_reg_group(const RowParams& p, int64_t blk, float (*lds)[4]) {
  constexpr int VEC = Elem<T>::kVec;
  constexpr int LANES = kWave * WPR;
  constexpr int ROWS_PER_BLOCK = 4 / WPR;

  const int sub = threadIdx.x / LANES;  // row slot within the block
  const int l = threadIdx.x % LANES;    // lane index within the row
  const int64_t row = blk * ROWS_PER_BLOCK + sub;
  // With WPR > 1 every wave of a row slot shares the row, and the grid covers
  // whole blocks only when rows % ROWS_PER_BLOCK == 0; the early exit is taken
  // by all waves of a row slot together.  Reductions sync the whole block, so a
  // block whose trailing slots are empty must still reach every barrier: those
  // waves run with no live vectors instead of returning.
  const bool row_ok = row < p.rows;
  if (WPR == 1 && !row_ok) return;
  const int64_t n = p.n;
  const T* xr = static_cast<const T*>(p.x) + (row_ok ? row : 0) * n;
  T* yr = static_cast<T*>(p.y) + (row_ok ? row : 0) * n;

  uint4 v[NV];
  bool live[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t c0 = (static_cast<int64_t>(i) * LANES + l) * VEC;
    live[i] = row_ok && c0 < n;
  }

  if constexpr (OP == kSoftmax || OP == kLogSoftmax || OP == kMaskedSoftmax) {
    const int64_t qrow = (OP == kMaskedSoftmax) ? ((row_ok ? row : 0) % p.sq) : 0;
    int64_t moff = 0;
    if constexpr (OP == kMaskedSoftmax) {
      const int64_t bh = (row_ok ? row : 0) / p.sq;
      moff = (bh / p.heads) * p.m_sb + (bh % p.heads) * p.m_sh + qrow * p.m_sq;
    }
    // Value j of vector i after scale / masks (-inf where masked or not live).
    auto val = [&](int i, float* f) {
      const int64_t c0 = (static_cast<int64_t>(i) * LANES + l) * VEC;
      // Causal: a vector whose first column is past the diagonal is fully masked
      // and is never read from HBM.
      const bool skip = (OP == kMaskedSoftmax) && p.causal && c0 > qrow;
      if (!live[i] || skip) {
#pragma unroll
        for (int j = 0; j < VEC; ++j) f[j] = -INFINITY;
        return;
      }
      unpack(v[i], f, T{});
      if constexpr (OP == kMaskedSoftmax) {
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
          float s = f[j] * p.scale;
          if (p.mask_kind == 1 && !static_cast<const uint8_t*>(p.mask)[moff + (c0 + j) * p.m_sk]) s = -INFINITY;
          if (p.mask_kind == 2) s += Elem<T>::load1(static_cast<const T*>(p.mask) + moff + (c0 + j) * p.m_sk);
          if (p.causal && c0 + j > qrow) s = -INFINITY;
          f[j] = s;
        }
      }
    };
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int64_t c0 = (static_cast<int64_t>(i) * LANES + l) * VEC;
      const bool skip = (OP == kMaskedSoftmax) && p.causal && c0 > qrow;
      if (live[i] && !skip) v[i] = ld_nt(xr + c0);
    }
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      float f[VEC];
      val(i, f);
#pragma unroll
      for (int j = 0; j < VEC; ++j) mx = fmaxf(mx, f[j]);
    }
    mx = row_reduce_max<WPR>(mx, lds, 0);
    // fp32 softmax keeps each exp in the register its input came from (a
    // vector holds 4 fp32 either way), so the store pass only scales.
    constexpr bool kKeepExp = OP != kLogSoftmax && Elem<T>::kVec == 4;
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      float f[VEC];
      val(i, f);
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        f[j] = fast_exp(f[j] - mx);
        s += f[j];
      }
      if constexpr (kKeepExp) v[i] = make_uint4(__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]),
                                               __float_as_uint(f[3]));
    }
    s = row_reduce_sum<WPR>(s, lds, 1);
    const float shift = mx + logf(s);
    const float inv = 1.0f / s;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      if (!live[i]) continue;
      const int64_t c0 = (static_cast<int64_t>(i) * LANES + l) * VEC;
      float f[VEC];
      if constexpr (kKeepExp) {
        f[0] = __uint_as_float(v[i].x) * inv;
        f[1] = __uint_as_float(v[i].y) * inv;
        f[2] = __uint_as_float(v[i].z) * inv;
        f[3] = __uint_as_float(v[i].w) * inv;
      } else {
        val(i, f);
#pragma unroll
        for (int j = 0; j < VEC; ++j)
          f[j] = (OP == kLogSoftmax) ? f[j] - shift : fast_exp(f[j] - mx) * inv;
      }
      st_nt(yr + c0, pack(f, T{}));
    }
  } else {
    // RMSNorm / LayerNorm.
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int64_t c0 = (static_cast<int64_t>(i) * LANES + l) * VEC;
      v[i] = live[i] ? ld_nt(xr + c0) : make_uint4(0, 0, 0, 0);
    }
    // RMSNorm fp32: gamma is fetched with x, so its (L2) latency overlaps the
    // loads of x instead of following the statistics ([8192, 4096]: +3.5..5%).
    // For 16-bit data and for LayerNorm (gamma and beta) the extra registers cost
    // more than the overlap gains (measured -1..2%); beyond 4 vectors per lane
    // they would halve the waves in flight.
    constexpr bool kEarlyParams = Elem<T>::kVec == 4 && OP == kRmsNorm && NV <= 4;
    uint4 gr[kEarlyParams ? NV : 1];
#pragma unroll
    for (int i = 0; i < NV && kEarlyParams; ++i) {
      const int64_t c0 = (static_cast<int64_t>(i) * LANES + l) * VEC;
      gr[i] = (p.gamma && live[i]) ? *reinterpret_cast<const uint4*>(static_cast<const T*>(p.gamma) + c0)
                                   : make_uint4(0, 0, 0, 0);
    }
    // Kept packed: each pass widens the vectors as it reads them (a shift or a
    // mask per 16-bit value), which needs half the registers of an fp32 copy.
    float mean, rstd;
    auto xget = [&](int i, float* f) { unpack(v[i], f, T{}); };
    norm_stats<T, OP, NV, WPR>(xget, live, n, p.eps, lds, mean, rstd);
    const T* g = static_cast<const T*>(p.gamma);
    const T* b = static_cast<const T*>(p.beta);
    auto gfetch = [&](int i, int64_t c0, float* gv) {
      if constexpr (kEarlyParams) unpack(gr[i], gv, T{});
      else load_vec(g + c0, gv);
    };
    auto bfetch = [&](int i, int64_t c0, float* bv) { load_vec(b + c0, bv); };
    using yes = std::true_type;
    using no = std::false_type;
    if (g && b) norm_store<T, NV, LANES>(xget, live, mean, rstd, yr, l, yes{}, yes{}, gfetch, bfetch);
    else if (g) norm_store<T, NV, LANES>(xget, live, mean, rstd, yr, l, yes{}, no{}, gfetch, bfetch);
    else if (b) norm_store<T, NV, LANES>(xget, live, mean, rstd, yr, l, no{}, yes{}, gfetch, bfetch);
    else norm_store<T, NV, LANES>(xget, live, mean, rstd, yr, l, no{}, no{}, gfetch, bfetch);
  }
}

// x, y, the row count and the row width come first as kernel arguments of their
// own, preloaded into SGPRs like rows_norm_stream_kernel's: the row's loads are
// addressed without waiting for a kernel-argument fetch (at the config's 6 us per
// launch, that fetch is a visible part of the kernel).
template <typename T, int OP, int NV, int WPR>
__global__ __launch_bounds__(256) void rows_reg_kernel(const void* x, void* y, int64_t rows, int64_t n,
                                                       RowParams p) {
  __shared__ float lds[3][4];
  RowParams q = p;
  q.x = x;
  q.y = y;
  q.rows = rows;
  q.n = n;
  rows_reg_group<T, OP, NV, WPR>(q, blockIdx.x, lds);
}

// Streaming RMSNorm / LayerNorm for rows that exactly fill NV vectors of every
// lane (n == NV * 64 * WPR * VEC): a grid of a few workgroups per CU, each looping
// over row groups with the next group's x loaded (into a second register set)
// before the current group's statistics, so HBM reads of one row overlap the
// reduction, scaling and stores of the previous; gamma and beta are read into
// registers once per workgroup instead of once per row.  The loop has no
// divergent branch and issues no load between a group's stores and the wait for
// the next group's x, so that wait never covers the stores (vmcnt counts loads
// and stores in issue order).  Same arithmetic as rows_reg_group.
//
// x, y, the row count and the group count are the first kernel arguments, which
// this file preloads into SGPRs (-amdgpu-kernarg-preload-count), and the row width
// is a compile-time constant: a wave issues its first group's loads before any
// kernel-argument fetch, and gamma / beta follow them, so their latency overlaps
// instead of preceding the first loads.
template <typename T, int OP, int NV, int WPR>
__global__ __launch_bounds__(256) void rows_norm_stream_kernel(const void* x, void* y, int64_t rows,
                                                               int64_t groups, RowParams p) {
  constexpr int VEC = Elem<T>::kVec;
  constexpr int LANES = kWave * WPR;
  constexpr int RPB = 4 / WPR;
  __shared__ float lds[2][3][4];
  // The row slot is the same for the whole wave (LANES is a multiple of 64).
  const int sub = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / LANES);
  const int l = threadIdx.x % LANES;
  constexpr int64_t n = static_cast<int64_t>(NV) * LANES * VEC;
  int64_t blk = blockIdx.x;
  if (blk >= groups) return;  // whole workgroup
  bool live[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) live[i] = true;
  // Rows past the end (the last group of an odd row count) load the last row
  // again and store nothing.
  auto load = [&](int64_t k, uint4 (&v)[NV]) {
    int64_t row = k * RPB + sub;
    if (row >= rows) row = rows - 1;
    const T* xr = static_cast<const T*>(x) + row * n;
#pragma unroll
    for (int i = 0; i < NV; ++i) v[i] = ld_nt(xr + (static_cast<int64_t>(i) * LANES + l) * VEC);
  };
  uint4 va[NV], vb[NV];
  load(blk, va);
  const T* g = static_cast<const T*>(p.gamma);
  const T* b = OP == kLayerNorm ? static_cast<const T*>(p.beta) : nullptr;
  // gamma / beta widened once (the grid has two workgroups per CU, so registers
  // are not what limits the waves in flight).
  float gf[NV][VEC], bfl[NV][VEC];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t c0 = (static_cast<int64_t>(i) * LANES + l) * VEC;
    unpack(g ? *reinterpret_cast<const uint4*>(g + c0) : make_uint4(0, 0, 0, 0), gf[i], T{});
    unpack(b ? *reinterpret_cast<const uint4*>(b + c0) : make_uint4(0, 0, 0, 0), bfl[i], T{});
  }
  // Wait for the first group and gamma / beta here, once: left pending into the
  // loop, the registers gamma / beta land in make the compiler wait for every
  // outstanding load and store at the top of each iteration (it cannot tell the
  // first iteration apart).
  __builtin_amdgcn_s_waitcnt(0);
  auto process = [&](int64_t k, const uint4 (&v)[NV], float (*L)[4]) {
    const int64_t row = k * RPB + sub;
    // x widened once for the statistics passes and the store pass.
    float xf[NV][VEC];
#pragma unroll
    for (int i = 0; i < NV; ++i) unpack(v[i], xf[i], T{});
    auto xget = [&](int i, float* f) {
#pragma unroll
      for (int j = 0; j < VEC; ++j) f[j] = xf[i][j];
    };
    float mean, rstd;
    norm_stats<T, OP, NV, WPR>(xget, live, n, p.eps, L, mean, rstd);
    if (row >= rows) return;
    T* yr = static_cast<T*>(y) + row * n;
    auto gfetch = [&](int i, int64_t, float* gv) {
#pragma unroll
      for (int j = 0; j < VEC; ++j) gv[j] = gf[i][j];
    };
    auto bfetch = [&](int i, int64_t, float* bv) {
#pragma unroll
      for (int j = 0; j < VEC; ++j) bv[j] = bfl[i][j];
    };
    using yes = std::true_type;
    using no = std::false_type;
    if (g && b) norm_store<T, NV, LANES>(xget, live, mean, rstd, yr, l, yes{}, yes{}, gfetch, bfetch);
    else if (g) norm_store<T, NV, LANES>(xget, live, mean, rstd, yr, l, yes{}, no{}, gfetch, bfetch);
    else if (b) norm_store<T, NV, LANES>(xget, live, mean, rstd, yr, l, no{}, yes{}, gfetch, bfetch);
    else norm_store<T, NV, LANES>(xget, live, mean, rstd, yr, l, no{}, no{}, gfetch, bfetch);
  };
  // The loop body handles two groups (register sets va, vb) and has no exit in
  // between, so no path reaches a prefetch with that register set's previous
  // loads still pending; it runs while both of its prefetches are in range, and
  // the last one or two groups follow it without a prefetch past the end.  The
  // scheduling fences keep the compiler from sinking a prefetch below the
  // statistics or the stores that follow it.
  const int64_t G = gridDim.x;
  const int64_t iters = (groups - blk + G - 1) / G;
  int64_t it = 0;
  for (; it + 2 < iters; it += 2) {
    load(blk + G, vb);
    __builtin_amdgcn_sched_barrier(0);
    process(blk, va, lds[0]);
    blk += G;
    load(blk + G, va);
    __builtin_amdgcn_sched_barrier(0);
    process(blk, vb, lds[1]);
    blk += G;
  }
  if (iters - it == 2) {
    load(blk + G, vb);
    __builtin_amdgcn_sched_barrier(0);
    process(blk, va, lds[0]);
    process(blk + G, vb, lds[1]);
  } else {
    process(blk, va, lds[0]);
  }
}

// Generic fallback: one 256-thread workgroup per row, scalar accesses, several
// passes over the row (the second and third normally hit L2).
template <typename T, int OP>
__global__ __launch_bounds__(256) void rows_generic_kernel(RowParams p) {
  __shared__ float lds[3][4];
  const int64_t row = blockIdx.x;
  if (row >= p.rows) return;
  const int64_t n = p.n;
  const T* xr = static_cast<const T*>(p.x) + row * n;
  T* yr = static_cast<T*>(p.y) + row * n;
  const int t = threadIdx.x;

  if constexpr (OP == kSoftmax || OP == kLogSoftmax || OP == kMaskedSoftmax) {
    const int64_t qrow = (OP == kMaskedSoftmax) ? (row % p.sq) : 0;
    int64_t moff = 0;
    if constexpr (OP == kMaskedSoftmax) {
      const int64_t bh = row / p.sq;
      moff = (bh / p.heads) * p.m_sb + (bh % p.heads) * p.m_sh + qrow * p.m_sq;
    }
    auto val = [&](int64_t c) -> float {
      float s = Elem<T>::load1(xr + c);
      if constexpr (OP == kMaskedSoftmax) {
        s *= p.scale;
        if (p.mask_kind == 1 && !static_cast<const uint8_t*>(p.mask)[moff + c * p.m_sk]) s = -INFINITY;
        if (p.mask_kind == 2) s += Elem<T>::load1(static_cast<const T*>(p.mask) + moff + c * p.m_sk);
        if (p.causal && c > qrow) s = -INFINITY;
      }
      return s;
    };
    float mx = -INFINITY;
    for (int64_t c = t; c < n; c += 256) mx = fmaxf(mx, val(c));
    mx = row_reduce_max<4>(mx, lds, 0);
    float s = 0.f;
    for (int64_t c = t; c < n; c += 256) s += fast_exp(val(c) - mx);
    s = row_reduce_sum<4>(s, lds, 1);
    const float shift = mx + logf(s);
    const float inv = 1.0f / s;
    for (int64_t c = t; c < n; c += 256) {
      const float d = val(c);
      Elem<T>::store1(yr + c, OP == kLogSoftmax ? d - shift : fast_exp(d - mx) * inv);
    }
  } else {
    float s = 0.f;
    for (int64_t c = t; c < n; c += 256) {
      const float a = Elem<T>::load1(xr + c);
      s += (OP == kRmsNorm) ? a * a : a;
    }
    s = row_reduce_sum<4>(s, lds, 1);
    const float inv_n = 1.0f / static_cast<float>(n);
    float mean = 0.f, rstd;
    if constexpr (OP == kRmsNorm) {
      rstd = rsqrtf(s * inv_n + p.eps);
    } else {
      mean = s * inv_n;
      float q = 0.f;
      for (int64_t c = t; c < n; c += 256) {
        const float d = Elem<T>::load1(xr + c) - mean;
        q += d * d;
      }
      q = row_reduce_sum<4>(q, lds, 2);
      rstd = rsqrtf(q * inv_n + p.eps);
    }
    const T* g = static_cast<const T*>(p.gamma);
    const T* b = static_cast<const T*>(p.beta);
    for (int64_t c = t; c < n; c += 256) {
      float o = (Elem<T>::load1(xr + c) - mean) * rstd;
      if (g) o *= Elem<T>::load1(g + c);
      if (b) o += Elem<T>::load1(b + c);
      Elem<T>::store1(yr + c, o);
    }
  }
}

static inline bool aligned16(const void* ptr) {
  return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0;
}

// CUs of the current device (cached per device).
static int device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int c = cache[dev].load(std::memory_order_relaxed);
  if (c == 0) {
    if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) c = 256;
    cache[dev].store(c, std::memory_order_relaxed);
  }
  return c;
}

template <typename T, int OP, int NV, int WPR>
static hipError_t launch_reg(const RowParams& p, hipStream_t s) {
  const int rows_per_block = 4 / WPR;
  const int64_t groups = (p.rows + rows_per_block - 1) / rows_per_block;
  hipLaunchKernelGGL((rows_reg_kernel<T, OP, NV, WPR>), dim3(static_cast<unsigned>(groups)), dim3(256), 0, s, p.x, p.y,
                     p.rows, p.n, p);
  return hipGetLastError();
}

template <typename T, int OP, int NV, int WPR>
static hipError_t launch_norm_stream(const RowParams& p, hipStream_t s, int64_t grid_cap) {
  const int rows_per_block = 4 / WPR;
  const int64_t groups = (p.rows + rows_per_block - 1) / rows_per_block;
  const int64_t grid = groups > grid_cap ? grid_cap : groups;
  hipLaunchKernelGGL((rows_norm_stream_kernel<T, OP, NV, WPR>), dim3(static_cast<unsigned>(grid)), dim3(256), 0, s,
                     p.x, p.y, p.rows, groups, p);
  return hipGetLastError();
}

// RMSNorm / LayerNorm rows that exactly fill NV vectors per lane, with at least
// four row groups per workgroup of a (normally) two-per-CU grid, stream through
// rows_norm_stream_kernel (measured on MI355X, [8192, 4096]: fp32 71% -> 76% of
// the HBM peak, bf16 RMSNorm 69% -> 72%, bf16 LayerNorm 67% -> 70%; grids of one
// or two workgroups per CU beat larger ones and uneven multiples of the CU
// count); everything else takes one workgroup per row group.
// Workgroups of rows_norm_stream_kernel<...> per CU for the streaming grid: two,
// or one where the kernel's registers allow only one (a second, non-resident
// workgroup per CU would start its share of the rows only after the first ends).
template <typename T, int OP, int NV, int WPR>
static int stream_blocks_per_cu() {
  static std::atomic<int> cached{0};
  int c = cached.load(std::memory_order_relaxed);
  if (c == 0) {
    int b = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, rows_norm_stream_kernel<T, OP, NV, WPR>, 256, 0) !=
            hipSuccess ||
        b <= 0)
      b = 1;
    c = b < 2 ? b : 2;
    cached.store(c, std::memory_order_relaxed);
  }
  return c;
}

template <typename T, int OP, int NV, int WPR>
static hipError_t launch_norm(const RowParams& p, hipStream_t s) {
  if constexpr (NV <= 8) {
    const int rows_per_block = 4 / WPR;
    const int64_t groups = (p.rows + rows_per_block - 1) / rows_per_block;
    const int64_t grid = stream_blocks_per_cu<T, OP, NV, WPR>() * static_cast<int64_t>(device_cus());
    if (p.n == static_cast<int64_t>(NV) * kWave * WPR * Elem<T>::kVec && groups >= 4 * grid)
      return launch_norm_stream<T, OP, NV, WPR>(p, s, grid);
  }
  return launch_reg<T, OP, NV, WPR>(p, s);
}

template <typename T, int OP>
static hipError_t launch_rows(const RowParams& p, hipStream_t s) {
  constexpr int VEC = Elem<T>::kVec;
  if (p.rows == 0 || p.n == 0) return hipSuccess;
  const bool vec_ok = (p.n % VEC == 0) && aligned16(p.x) && aligned16(p.y) &&
                      (!p.gamma || aligned16(p.gamma)) && (!p.beta || aligned16(p.beta));
  if (vec_ok) {
    // Waves per row: aim for about four 16-byte vectors per lane.
    const int64_t vecs = p.n / VEC;  // 16-byte vectors per row
    constexpr bool kNorm = OP == kRmsNorm || OP == kLayerNorm;
    auto go = [&](auto nv, auto wpr) {
      if constexpr (kNorm) return launch_norm<T, OP, decltype(nv)::value, decltype(wpr)::value>(p, s);
      else return launch_reg<T, OP, decltype(nv)::value, decltype(wpr)::value>(p, s);
    };
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I4 = std::integral_constant<int, 4>;
    using I8 = std::integral_constant<int, 8>;
    using I16 = std::integral_constant<int, 16>;
    if (vecs <= 64 * 1) return go(I1{}, I1{});
    if (vecs <= 64 * 2) return go(I2{}, I1{});
    if (vecs <= 64 * 4) return go(I4{}, I1{});
    if (vecs <= 128 * 4) return go(I4{}, I2{});
    if (vecs <= 256 * 4) return go(I4{}, I4{});
    if (vecs <= 256 * 8) return go(I8{}, I4{});
    if (vecs <= 256 * 16) return go(I16{}, I4{});
  }
  hipLaunchKernelGGL((rows_generic_kernel<T, OP>), dim3(static_cast<unsigned>(p.rows)),
                     dim3(256), 0, s, p);
  return hipGetLastError();
}

template <int OP>
static int dispatch_rows(int dtype, const RowParams& p, void* stream, GHipError* err,
                         const char* what) {
  if (p.rows < 0 || p.n < 0) return set_error(err, GHIP_ERR_INVALID_ARG, "%s: negative size", what);
  if (p.rows > 0 && p.n > 0 && (!p.x || !p.y))
    return set_error(err, GHIP_ERR_INVALID_ARG, "%s: null pointer", what);
  if (p.rows > 0x7fffffffLL)
    return set_error(err, GHIP_ERR_INVALID_ARG, "%s: too many rows (%lld)", what,
                     static_cast<long long>(p.rows));
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e;
  if (dtype == GHIP_DTYPE_FLOAT32) e = launch_rows<float, OP>(p, s);
  else if (dtype == GHIP_DTYPE_BFLOAT16) e = launch_rows<bf16_t, OP>(p, s);
  else if (dtype == GHIP_DTYPE_FLOAT16) e = launch_rows<f16_t, OP>(p, s);
  else return set_error(err, GHIP_ERR_UNSUPPORTED, "%s: dtype %d not supported", what, dtype);
  if (e != hipSuccess) return check_hip(e, err, what);
  return GHIP_OK;
}

// ---------------------------------------------------------------------------
// Column kernels: softmax / log-softmax / LayerNorm over a middle axis of a dense
// [outer, n, inner] tensor (inner > 1), in place of moving the axis last with a
// transposing copy (and copying the result back).  A workgroup takes 64 adjacent
// columns i of one outer index as 64 lanes x 4 row phases: lane c of phase ph
// walks rows ph, ph + 4, ... of column i0 + c, so each wave instruction reads 64
// consecutive elements of one row.  Per-column statistics in fp32 (softmax: a
// running max and a sum of exponents rescaled when the max moves; LayerNorm: a
// running count, mean and squared-deviation sum, Welford's update), combined
// over the 4 phases through LDS (Chan, Golub and LeVeque's pairwise update for
// LayerNorm), then a second pass writes y in the same layout (its reads of x
// are mostly served by the L2 / Infinity Cache).  -inf inputs contribute nothing
// to the sums; a column of -inf gives NaN, as the row kernels do.
struct ColParams {
  const void* x;
  void* y;
  const void* gamma;  // [n] or null (LayerNorm)
  const void* beta;   // [n] or null (LayerNorm)
  int64_t n, inner, col_blocks;
  float eps;
};

template <typename T, int OP>
__global__ __launch_bounds__(256) void cols_kernel(ColParams p) {
  __shared__ float red[3][4][64];
  const int c = threadIdx.x & 63, ph = threadIdx.x >> 6;
  const int64_t o = blockIdx.x / p.col_blocks;
  const int64_t i = (blockIdx.x % p.col_blocks) * 64 + c;
  const bool ok = i < p.inner;
  const int64_t n = p.n, inner = p.inner;
  const T* x = static_cast<const T*>(p.x) + o * n * inner + (ok ? i : 0);
  T* y = static_cast<T*>(p.y) + o * n * inner + (ok ? i : 0);
  if constexpr (OP == kSoftmax || OP == kLogSoftmax) {
    float m = -INFINITY, s = 0.f;
    if (ok)
      for (int64_t k = ph; k < n; k += 4) {
        const float v = Elem<T>::load1(x + k * inner);
        if (v == -INFINITY) continue;
        if (v > m) {
          s = m == -INFINITY ? 0.f : s * fast_exp(m - v);
          m = v;
        }
        s += fast_exp(v - m);  // NaN inputs make s NaN
      }
    red[0][ph][c] = m;
    red[1][ph][c] = s;
    __syncthreads();
    float M = red[0][0][c];
#pragma unroll
    for (int q = 1; q < 4; ++q) M = fmaxf(M, red[0][q][c]);
    float S = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float mq = red[0][q][c];
      if (mq != -INFINITY) S += red[1][q][c] * fast_exp(mq - M);
    }
    if (!ok) return;
    const float inv = 1.0f / S, shift = M + logf(S);
    for (int64_t k = ph; k < n; k += 4) {
      const float v = Elem<T>::load1(x + k * inner);
      Elem<T>::store1(y + k * inner, OP == kLogSoftmax ? v - shift : fast_exp(v - M) * inv);
    }
  } else {
    static_assert(OP == kLayerNorm, "softmax, log-softmax or LayerNorm");
    float cnt = 0.f, mean = 0.f, m2 = 0.f;
    if (ok)
      for (int64_t k = ph; k < n; k += 4) {
        const float v = Elem<T>::load1(x + k * inner);
        cnt += 1.f;
        const float d = v - mean;
        mean += d / cnt;
        m2 += d * (v - mean);
      }
    red[0][ph][c] = cnt;
    red[1][ph][c] = mean;
    red[2][ph][c] = m2;
    __syncthreads();
    float na = red[0][0][c], ma = red[1][0][c], qa = red[2][0][c];
#pragma unroll
    for (int q = 1; q < 4; ++q) {
      const float nb = red[0][q][c], mb = red[1][q][c], qb = red[2][q][c];
      const float nt = na + nb;
      if (nb > 0.f) {
        const float d = mb - ma;
        ma += d * (nb / nt);
        qa += qb + d * d * (na * nb / nt);
        na = nt;
      }
    }
    if (!ok) return;
    const float rstd = 1.0f / sqrtf(qa / static_cast<float>(n) + p.eps);
    const T* g = static_cast<const T*>(p.gamma);
    const T* b = static_cast<const T*>(p.beta);
    for (int64_t k = ph; k < n; k += 4) {
      float r = (Elem<T>::load1(x + k * inner) - ma) * rstd;
      if (g) r *= Elem<T>::load1(g + k);
      if (b) r += Elem<T>::load1(b + k);
      Elem<T>::store1(y + k * inner, r);
    }
  }
}

template <int OP>
static int dispatch_cols(int dtype, ColParams p, int64_t outer, void* stream, GHipError* err, const char* what) {
  if (outer < 0 || p.n < 0 || p.inner < 0) return set_error(err, GHIP_ERR_INVALID_ARG, "%s: negative size", what);
  if (outer == 0 || p.n == 0 || p.inner == 0) return GHIP_OK;
  if (!p.x || !p.y) return set_error(err, GHIP_ERR_INVALID_ARG, "%s: null pointer", what);
  p.col_blocks = (p.inner + 63) / 64;
  const int64_t grid = outer * p.col_blocks;
  if (grid > 0x7fffffffLL) return set_error(err, GHIP_ERR_INVALID_ARG, "%s: too many columns", what);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 g(static_cast<unsigned>(grid));
  if (dtype == GHIP_DTYPE_FLOAT32) hipLaunchKernelGGL((cols_kernel<float, OP>), g, dim3(256), 0, s, p);
  else if (dtype == GHIP_DTYPE_BFLOAT16) hipLaunchKernelGGL((cols_kernel<bf16_t, OP>), g, dim3(256), 0, s, p);
  else if (dtype == GHIP_DTYPE_FLOAT16) hipLaunchKernelGGL((cols_kernel<f16_t, OP>), g, dim3(256), 0, s, p);
  else return set_error(err, GHIP_ERR_UNSUPPORTED, "%s: dtype %d not supported", what, dtype);
  GHIP_CHECK(hipGetLastError(), err);
  return GHIP_OK;
}

}  // namespace ghip

using namespace ghip;

extern "C" int ghip_softmax_rows(int dtype, const void* x, void* y, int64_t rows, int64_t n,
                                 int log_softmax, void* stream, GHipError* err) {
  RowParams p{};
  p.x = x; p.y = y; p.rows = rows; p.n = n;
  if (log_softmax) return dispatch_rows<kLogSoftmax>(dtype, p, stream, err, "softmax_rows");
  return dispatch_rows<kSoftmax>(dtype, p, stream, err, "softmax_rows");
}

extern "C" int ghip_scale_mask_softmax_rows_ex(int dtype, const void* x, void* y, int64_t B, int64_t H,
                                               int64_t sq, int64_t sk, float scale, int causal, const void* mask,
                                               int mask_dtype, const int64_t* mask_strides, void* stream,
                                               GHipError* err) {
  if (B < 0 || H <= 0 || sq <= 0 || sk < 0)
    return set_error(err, GHIP_ERR_INVALID_ARG, "scale_mask_softmax_rows: bad sizes");
  RowParams p{};
  p.x = x; p.y = y; p.rows = B * H * sq; p.n = sk; p.sq = sq; p.heads = H; p.scale = scale;
  p.causal = causal;
  if (mask) {
    if (!mask_strides) return set_error(err, GHIP_ERR_INVALID_ARG, "scale_mask_softmax_rows: mask without strides");
    if (mask_dtype != GHIP_DTYPE_BOOL && mask_dtype != dtype)
      return set_error(err, GHIP_ERR_INVALID_ARG, "scale_mask_softmax_rows: mask must be bool or the scores' dtype");
    p.mask = mask;
    p.mask_kind = mask_dtype == GHIP_DTYPE_BOOL ? 1 : 2;
    p.m_sb = mask_strides[0]; p.m_sh = mask_strides[1]; p.m_sq = mask_strides[2]; p.m_sk = mask_strides[3];
  }
  return dispatch_rows<kMaskedSoftmax>(dtype, p, stream, err, "scale_mask_softmax_rows");
}

extern "C" int ghip_scale_mask_softmax_rows(int dtype, const void* x, void* y, int64_t rows,
                                            int64_t sq, int64_t sk, float scale, int causal,
                                            const uint8_t* bmask, void* stream,
                                            GHipError* err) {
  if (sq <= 0 || (rows % sq) != 0)
    return set_error(err, GHIP_ERR_INVALID_ARG,
                     "scale_mask_softmax_rows: rows (%lld) must be a multiple of sq (%lld)",
                     static_cast<long long>(rows), static_cast<long long>(sq));
  const int64_t ms[4] = {0, 0, sk, 1};
  return ghip_scale_mask_softmax_rows_ex(dtype, x, y, rows / sq, 1, sq, sk, scale, causal, bmask,
                                         GHIP_DTYPE_BOOL, ms, stream, err);
}

extern "C" int ghip_rmsnorm_rows(int dtype, const void* x, const void* gamma, void* y,
                                 int64_t rows, int64_t n, float eps, void* stream,
                                 GHipError* err) {
  RowParams p{};
  p.x = x; p.y = y; p.gamma = gamma; p.rows = rows; p.n = n; p.eps = eps;
  return dispatch_rows<kRmsNorm>(dtype, p, stream, err, "rmsnorm_rows");
}

extern "C" int ghip_layernorm_rows(int dtype, const void* x, const void* gamma, const void* beta,
                                   void* y, int64_t rows, int64_t n, float eps, void* stream,
                                   GHipError* err) {
  RowParams p{};
  p.x = x; p.y = y; p.gamma = gamma; p.beta = beta; p.rows = rows; p.n = n; p.eps = eps;
  return dispatch_rows<kLayerNorm>(dtype, p, stream, err, "layernorm_rows");
}

extern "C" int ghip_softmax_cols(int dtype, const void* x, void* y, int64_t outer, int64_t n, int64_t inner,
                                 int log_softmax, void* stream, GHipError* err) {
  ColParams p{};
  p.x = x; p.y = y; p.n = n; p.inner = inner;
  if (log_softmax) return dispatch_cols<kLogSoftmax>(dtype, p, outer, stream, err, "softmax_cols");
  return dispatch_cols<kSoftmax>(dtype, p, outer, stream, err, "softmax_cols");
}

extern "C" int ghip_layernorm_cols(int dtype, const void* x, const void* gamma, const void* beta, void* y,
                                   int64_t outer, int64_t n, int64_t inner, float eps, void* stream,
                                   GHipError* err) {
  ColParams p{};
  p.x = x; p.y = y; p.gamma = gamma; p.beta = beta; p.n = n; p.inner = inner; p.eps = eps;
  return dispatch_cols<kLayerNorm>(dtype, p, outer, stream, err, "layernorm_cols");
}
