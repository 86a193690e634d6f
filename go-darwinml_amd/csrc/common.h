// Shared device/host helpers for the gomlx-hip kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gomlx_hip.h"

namespace ghip {

// ---------------------------------------------------------------------------
// bf16 stored as raw 16-bit patterns.  Conversion fp32 -> bf16 rounds to nearest
// even (NaN kept quiet); bf16 -> fp32 is exact.
// ---------------------------------------------------------------------------
struct bf16_t {
  uint16_t bits;
};

__device__ __host__ __forceinline__ float bf16_to_f32(uint16_t b) {
  const uint32_t u = static_cast<uint32_t>(b) << 16;
  return __builtin_bit_cast(float, u);
}

// Round to nearest even; a NaN keeps its sign and upper payload bits and comes
// out quiet.  On gfx950 this is exactly v_cvt_pk_bf16_f32 (the device path:
// one instruction per pair of values); the integer formulation (host path) is
// the definition both are tested against.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
#else
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
#endif
}

// Packs two fp32 into two bf16 (RNE) in one dword: lo in bits 0..15.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
#if defined(__HIP_DEVICE_COMPILE__)
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
#else
  return static_cast<uint32_t>(f32_to_bf16(lo)) | (static_cast<uint32_t>(f32_to_bf16(hi)) << 16);
#endif
}

// IEEE binary16 stored as raw 16-bit patterns; conversions through the
// hardware's v_cvt_f32_f16 / v_cvt_f16_f32 (round to nearest even).
struct f16_t {
  uint16_t bits;
};
__device__ __forceinline__ float f16_to_f32(uint16_t b) {
  return static_cast<float>(__builtin_bit_cast(_Float16, b));
}
// Round to nearest even from the fp32 value.  The empty asm makes f an opaque
// fp32 register, so the compiler cannot fold the rounding into the producing
// fma / multiply (v_fma_mixlo_f16 rounds the exact product to f16 once, which can
// differ from rounding the fp32 result): every kernel rounds the same way.
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  asm volatile("" : "+v"(f));
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  return static_cast<uint32_t>(f32_to_f16(lo)) | (static_cast<uint32_t>(f32_to_f16(hi)) << 16);
}

// ---------------------------------------------------------------------------
// Element traits: how many elements one 16-byte vector holds and how to widen.
// ---------------------------------------------------------------------------
template <typename T> struct Elem;
template <> struct Elem<float> {
  static constexpr int kVec = 4;
  __device__ static float load1(const float* p) { return *p; }
  __device__ static void store1(float* p, float v) { *p = v; }
};
template <> struct Elem<bf16_t> {
  static constexpr int kVec = 8;
  __device__ static float load1(const bf16_t* p) { return bf16_to_f32(p->bits); }
  __device__ static void store1(bf16_t* p, float v) { p->bits = f32_to_bf16(v); }
};
template <> struct Elem<f16_t> {
  static constexpr int kVec = 8;
  __device__ static float load1(const f16_t* p) { return f16_to_f32(p->bits); }
  __device__ static void store1(f16_t* p, float v) { p->bits = f32_to_f16(v); }
};

// Loads 16 bytes (kVec elements) and widens them to fp32.
__device__ __forceinline__ void load_vec(const float* p, float* out) {
  float4 v = *reinterpret_cast<const float4*>(p);
  out[0] = v.x; out[1] = v.y; out[2] = v.z; out[3] = v.w;
}
__device__ __forceinline__ void load_vec(const bf16_t* p, float* out) {
  uint4 v = *reinterpret_cast<const uint4*>(p);
  uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = __uint_as_float(w[i] << 16);
    out[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}
__device__ __forceinline__ void load_vec(const f16_t* p, float* out) {
  uint4 v = *reinterpret_cast<const uint4*>(p);
  uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = f16_to_f32(static_cast<uint16_t>(w[i]));
    out[2 * i + 1] = f16_to_f32(static_cast<uint16_t>(w[i] >> 16));
  }
}
__device__ __forceinline__ void store_vec(float* p, const float* v) {
  *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ void store_vec(bf16_t* p, const float* v) {
  uint4 o;
  o.x = pack_bf16x2(v[0], v[1]);
  o.y = pack_bf16x2(v[2], v[3]);
  o.z = pack_bf16x2(v[4], v[5]);
  o.w = pack_bf16x2(v[6], v[7]);
  *reinterpret_cast<uint4*>(p) = o;
}
__device__ __forceinline__ void store_vec(f16_t* p, const float* v) {
  *reinterpret_cast<uint4*>(p) =
      make_uint4(pack_f16x2(v[0], v[1]), pack_f16x2(v[2], v[3]), pack_f16x2(v[4], v[5]), pack_f16x2(v[6], v[7]));
}

// ---------------------------------------------------------------------------
// Wave64 reductions with every lane receiving the result (all 64 lanes active).  Within each row of
// 16 lanes four DPP steps (quad_perm [1,0,3,2], quad_perm [2,3,0,1],
// row_half_mirror, row_mirror) leave the row's total in all 16 lanes; the four
// row totals are then read as scalars (v_readlane) and combined.  Each DPP step
// is one VALU instruction with its source operand permuted, so a reduction
// costs ~12 instructions and no LDS round trip (a ds_bpermute butterfly takes
// six LDS-latency steps).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float row_lane(float x, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), lane));
}
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f32<0xb1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f32<0x4e>(v);   // quad_perm [2,3,0,1]
  v += dpp_f32<0x141>(v);  // row_half_mirror
  v += dpp_f32<0x140>(v);  // row_mirror
  return (row_lane(v, 0) + row_lane(v, 16)) + (row_lane(v, 32) + row_lane(v, 48));
}
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f32<0xb1>(v));
  v = fmaxf(v, dpp_f32<0x4e>(v));
  v = fmaxf(v, dpp_f32<0x141>(v));
  v = fmaxf(v, dpp_f32<0x140>(v));
  return fmaxf(fmaxf(row_lane(v, 0), row_lane(v, 16)), fmaxf(row_lane(v, 32), row_lane(v, 48)));
}

// exp(x) through the hardware base-2 exponential: exp(x) = 2^(x * log2(e)),
// one v_exp_f32 (results below 2^-126 flush to zero; exp2f would add a
// denormal-range rescale of five more instructions per value).
__device__ __forceinline__ float fast_exp(float x) {
  return __builtin_amdgcn_exp2f(x * 1.4426950408889634f);
}

constexpr int kWave = 64;

}  // namespace ghip

// ---------------------------------------------------------------------------
// Host-side error plumbing shared by every C entry point.
// ---------------------------------------------------------------------------
namespace ghip {
int set_error(GHipError* err, int code, const char* fmt, ...);
int check_hip(hipError_t e, GHipError* err, const char* what);
}  // namespace ghip

#define GHIP_CHECK(expr, err)                                      \
  do {                                                             \
    hipError_t _e = (expr);                                        \
    if (_e != hipSuccess) return ghip::check_hip(_e, (err), #expr); \
  } while (0)
