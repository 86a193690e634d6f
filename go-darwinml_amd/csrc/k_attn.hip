// Fused scaled-dot-product attention (forward), the single-kernel lowering of
// Function.FusedScaledDotProductAttention (mpsgraph/gomlx/function.go:2669-2907):
//   out = softmax(scale * Q K^T + mask  [causal: -inf where key > query]) V
// for bf16 or f16 Q/K/V/O with a head dim that is a multiple of 8 up to 256, or
// fp32 with a multiple of 4 up to 128 (a second kernel, at the end), fp32 softmax
// statistics and accumulation.  The mask is the reference's: a boolean keep-mask (Where(mask,
// scores, -inf), :2847-2871) or an additive one (scores + mask, :2872-2878), of
// any rank broadcast to the scores [B, H, Sq, Sk] (:2959-2974), read through
// element strides (0 on broadcast axes).  GQA reads KV head h / (H / Hkv)
// directly (function.go:2911-2956 repeats it).
//
// Never materialises the [B, H, Sq, Sk] scores (the composite path writes and
// re-reads them: 1 GiB of bf16 traffic at B4 H16 S2048).  Per workgroup: 128
// queries (4 waves x 32); K and V stream through LDS in 64-key tiles:
//   * everything is computed transposed: S^T = K Q^T and O^T = V^T P^T with
//     v_mfma_f32_32x32x16_bf16, so each lane owns one query column -- its running
//     max, running sum and output rescale stay in the lane (one cross-half-wave
//     exchange per tile for the max);
//   * Q stays in registers for the whole kernel (B operand of S^T);
//   * the softmaxed S^T accumulators become the bf16 B operand of the second MFMA
//     without leaving registers: the 16 values a lane holds for key step s are
//     keys 16s + {0..3, 8..11} + 4 * (lane / 32), and V^T is read in that same key
//     order with two ds_read_b64_tr_b16 per fragment;
//   * K / V tiles arrive by buffer_load ... lds (16 B per lane; keys past Sk lie
//     beyond the buffer descriptor's extent and read zeros) into one 32 KiB LDS
//     stage per workgroup, XOR-swizzled so the ds_read_b128 (K) and transpose
//     reads (V) are bank-conflict free.  Two schedules: (plain) each tile's K and
//     V are loaded at its start and waited for before its first LDS read, the
//     other workgroups resident on the CU (three at the D = 128 kernel's 168
//     VGPRs) computing meanwhile; (split, unmasked) V_t loads while the scores of
//     tile t are computed and K_{t+1} while P V of tile t is, in the same 32 KiB,
//     at three barriers a tile instead of two: 4% faster at B4 H16 S2048 causal,
//     6-7% at longer or non-causal shapes, 6% slower when every causal workgroup
//     is short (<= 16 key tiles: the block's S1024), where the plain one is used;
//   * the output rescale of the online softmax is lazy: the reference max moves
//     only when a tile's max exceeds it by more than 2^8 (exponents stay <= 2^8);
//   * causal: tiles past a workgroup's last query are never loaded, a wave skips
//     the tiles past its own last query, and only diagonal tiles apply the
//     element mask; the grid runs all (batch, head) pairs of the last query block
//     first, so the longest workgroups start first.
#include "common.h"

#define GHIP_ALDS __attribute__((address_space(3)))

namespace ghip {
namespace attn {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));

enum MaskKind { kNoMask = 0, kBoolMask = 1, kAddMask = 2 };

struct Params {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  const void* mask;             // bool (uint8) keep-mask, or additive in Q's dtype
  int64_t q_sb, q_sh, q_ss;     // element strides of batch, head, sequence (d stride 1)
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh, o_ss;
  int64_t m_sb, m_sh, m_sq, m_sk;  // mask element strides (0 where it broadcasts)
  int B, H, Hkv, Sq, Sk;
  int D;                        // head dim (<= the kernel's padded width DP)
  float scale_log2;             // softmax scale * log2(e)
  float inv_scale;              // 1 / scale (additive masks are added to raw scores / scale)
  int causal;
  int mask_vec;                 // m_sk == 1 and 4-key groups are aligned: vector mask loads
  uint32_t k_extent, v_extent;  // bytes addressable from one (batch, kv head) slice (< 2 GiB)
  int64_t k_extent64, v_extent64;  // the same for the BIG kernels (any size)
  // Key range split over blockIdx.y (16-bit kernels): kv_chunk keys per split (a
  // multiple of the 64-key tile), each split writing its normalised output and its
  // log2-sum-exp of the scaled scores for the combine kernel; 0: no split.
  int kv_chunk;
  float* part_o;    // [split][b][h][query][D]
  float* part_lse;  // [split][b][h][query]
  // Grouped-query rows (16-bit kernels, no causal mask): a workgroup holds up to
  // 128 (head, query) rows of one kv head's group of H / Hkv heads, head-major, so
  // the group's heads read each K / V tile once; grid (row blocks, b, kv head).
  int gqa_pack;
};

constexpr int kBKV = 64;    // keys per tile
constexpr int kQW = 32;     // queries per wave
constexpr int kWaves = 4;   // waves per workgroup
constexpr int kBQ = kQW * kWaves;
constexpr float kLazyLog2 = 8.f;  // the reference max may trail the true max by 2^8
// A buffer offset past every descriptor's records (< 2 GiB, or capped at it in the
// BIG kernels): a DMA lane given it loads zeros.
constexpr uint32_t kPastEnd = 0x80000000u;

__device__ __forceinline__ i32x4_t make_rsrc(const void* base, uint32_t bytes) {
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  i32x4_t r;
  r.x = __builtin_amdgcn_readfirstlane(static_cast<int>(b));
  r.y = __builtin_amdgcn_readfirstlane(static_cast<int>((b >> 32) & 0xffff));
  r.z = __builtin_amdgcn_readfirstlane(static_cast<int>(bytes));
  r.w = 0x00020000;
  return r;
}
// Byte offsets of a key tile within a K / V slice, and the records of a descriptor
// based there.  BIG = false (slices below 2 GiB): 32-bit arithmetic.  BIG = true
// (16-bit kernels, slices of any size): 64-bit offsets and the bytes left in the
// slice capped at kPastEnd; a key tile lies within 2 GiB of its first row (the
// host checks the sequence strides), so the cap cuts nothing a tile reads.  Kept
// as separate instantiations: the 64-bit arithmetic made the 32-bit cases 3-8%
// slower (measured).
template <bool BIG>
struct KvOff {
  using T = uint32_t;
  __device__ __forceinline__ static uint32_t rec(uint32_t ext, int64_t, T d) { return ext - d; }
};
template <>
struct KvOff<true> {
  using T = int64_t;
  __device__ __forceinline__ static uint32_t rec(uint32_t, int64_t ext64, T d) {
    const int64_t left = ext64 - d;
    return left <= 0 ? 0u : left >= static_cast<int64_t>(kPastEnd) ? kPastEnd : static_cast<uint32_t>(left);
  }
};
// 16 bytes per lane from buffer offset voff straight into LDS byte address
// la + lane*16 (la wave-uniform).
// m0 is set and consumed inside this one asm statement, and no compiler-generated
// code in these kernels reads or writes m0 (none appears in their ISA apart from
// these pairs), so clang's warning that a reserved-register clobber is not
// preserved does not apply here.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(i32x4_t rsrc, uint32_t la, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               ::"s"(la), "v"(voff), "s"(rsrc) : "memory", "m0");
}
#pragma clang diagnostic pop

// LDS tiles are [64 keys][DP] 16-bit values: rows of C = DP / 8 chunks of 16 B.
// K: chunk kc of key row r sits at slot kc ^ (r % C), so the 8 or 16 rows of a
// ds_read_b128 phase land in distinct bank groups.
template <int DP>
__device__ __forceinline__ int swz_k(int r) { return r & (DP / 8 - 1); }
// V: chunk j of key row r sits at slot j ^ f(r & 3): a transpose read touches 4
// consecutive rows x 2 (DP = 64) or 2-4 (DP >= 128) chunks.  DP >= 128: f = {0, 6,
// 10, 12} (rows are whole multiples of the 128-byte bank period, so the bank group
// is the slot mod 8 at DP = 256 as at 128); DP = 64 (8 chunks a row): f = {0, 2, 4,
// 6}, which keeps the chunk pairs of a 32-byte read together and spreads the 4 rows
// over all 8 bank groups.
template <int DP>
__device__ __forceinline__ int swz_v(int r) {
  if constexpr (DP >= 128) return (0xCA60u >> ((r & 3) * 4)) & 15u;
  else return 2 * (r & 3);
}

// K fragment (A operand of S^T = K Q^T): key row kb*32 + lane%32, d = 16s + 8*(lane/32).
template <int DP>
__device__ __forceinline__ bf16x8_t frag_k(const uint16_t* lds, int kb, int s, int lane) {
  const int row = kb * 32 + (lane & 31);
  const int slot = (2 * s + (lane >> 5)) ^ swz_k<DP>(row);
  return *reinterpret_cast<const bf16x8_t*>(lds + row * DP + slot * 8);
}
// V^T fragment (A operand of O^T = V^T P^T), d block db, key step s: lane
// (d = 32 db + lane%32, h = lane/32) gets keys 16s + 4h + {0..3} and
// 16s + 8 + 4h + {0..3}.  ds_read_b64_tr_b16 hands lane j of each 16-lane group
// element j of the four 4-element rows the group points at.
template <int DP>
__device__ __forceinline__ bf16x8_t frag_v(const uint16_t* lds, int db, int s, int lane) {
  const int kl = 16 * s + 4 * (lane >> 5) + ((lane & 15) >> 2);
  const int nl = db * 32 + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  const uint16_t* p0 = lds + kl * DP + (((nl >> 3) ^ swz_v<DP>(kl)) * 8) + (nl & 7);
  const uint16_t* p1 = p0 + 8 * DP;  // key + 8 keeps key & 3, hence the swizzle
  bf16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((GHIP_ALDS bf16x4_t*)(p0));
  bf16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((GHIP_ALDS bf16x4_t*)(p1));
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// 32x32x16 MFMA on 16-bit operands held as bf16 bits: bf16, or f16 when F16.
template <bool F16>
__device__ __forceinline__ f32x16_t mma(const bf16x8_t& a, const bf16x8_t& b, const f32x16_t& c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                  0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
template <bool F16>
__device__ __forceinline__ float from16(uint16_t b) {
  if constexpr (F16) return f16_to_f32(b);
  else return bf16_to_f32(b);
}
template <bool F16>
__device__ __forceinline__ uint32_t pack16x2(float lo, float hi) {
  if constexpr (F16) return pack_f16x2(lo, hi);
  else return pack_bf16x2(lo, hi);
}
// acc + lo + hi of a packed pair of 16-bit values (v_dot2c against (1, 1)).
template <bool F16>
__device__ __forceinline__ float dot2_ones(uint32_t w, float acc) {
  if constexpr (F16) {
    typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
    const f16x2_t one = {static_cast<_Float16>(1.0f), static_cast<_Float16>(1.0f)};
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, w), one, acc, false);
  } else {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    const bf16x2_t one = {static_cast<__bf16>(1.0f), static_cast<__bf16>(1.0f)};
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w), one, acc, false);
  }
}

// DP: the padded head dim the LDS tiles, Q fragments and output accumulators are
// laid out for (64, 128 or 256); the head dim D = p.D is any multiple of 8 up to
// DP.  The 16-byte chunks of a row past D are loaded as zeros (their DMA offsets lie
// beyond the buffer's extent) and Q's are zero, so they add nothing to the scores
// and their output columns are not stored.  The MFMAs still run over the full DP
// (no branch in the tile loop: at D = DP the loop is exactly the unpadded one).
// SPLIT: the split K / V load schedule (below); the host picks it unless the
// mask is causal and no workgroup has more than 16 key tiles, where the plain
// schedule measured faster (short workgroups).
template <int DP, bool F16, int MK, bool SPLIT, bool BIG = false>
// Three workgroups (so three waves a SIMD) per CU for the unmasked kernels up to
// DP = 128: without the bound the compiler took 172 VGPRs for the plain schedule
// (two a SIMD, 12% slower on the block's attention) once the decoding forms added
// per-lane row indices; with it, 168 and no scratch.
__global__ __launch_bounds__(256, DP >= 256 ? 1 : (MK == kNoMask ? 3 : 2)) void sdpa_fwd_kernel(Params p) {
  constexpr int NCH = DP / 8;  // 16-byte chunks per key row
  constexpr int NDMA = kBKV * DP * 2 / 1024 / kWaves;  // DMA instructions per wave per K (or V) tile
  constexpr int RPI = 1024 / (DP * 2);                 // key rows per DMA instruction
  // [stage][K | V][64 keys x DP]
  __shared__ __attribute__((aligned(1024))) uint16_t smem[1][2][kBKV * DP];
  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((GHIP_ALDS void*)&smem[0][0][0]));

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h2 = lane >> 5;  // half of the wave
  const int D = p.D;
  int b, h, hk, q0, qw, qi;
  bool qv;  // this lane's row exists
  if (p.gqa_pack) {
    // Row r of the group (head hk * G + r / Sq, query r % Sq); no causal mask, so
    // q0 / qw (the causal bounds) go unused.
    const int G = p.H / p.Hkv;
    const int nbk = p.B * p.Hkv;
    const int bk = static_cast<int>(blockIdx.x % nbk);
    b = bk / p.Hkv;
    hk = bk % p.Hkv;
    const int r = static_cast<int>(blockIdx.x / nbk) * kBQ + wave * kQW + (lane & 31);
    qv = r < G * p.Sq;
    const int rc = qv ? r : 0;
    h = hk * G + rc / p.Sq;
    qi = rc % p.Sq;
    q0 = 0;
    qw = 0;
  } else {
    const int nqb = (p.Sq + kBQ - 1) / kBQ;
    const int nbh = p.B * p.H;
    // Longest first over the whole grid: every (batch, head) of the last query
    // block, then of the one before it, ... (causal: later blocks see more keys).
    const int qb = p.causal ? (nqb - 1 - static_cast<int>(blockIdx.x / nbh)) : static_cast<int>(blockIdx.x / nbh);
    const int bh = blockIdx.x % nbh;
    b = bh / p.H;
    h = bh % p.H;
    hk = h / (p.H / p.Hkv);
    q0 = qb * kBQ;
    qw = q0 + wave * kQW;    // first query of this wave
    qi = qw + (lane & 31);   // this lane's query
    qv = qi < p.Sq;
  }

  const uint16_t* Q = static_cast<const uint16_t*>(p.q) + b * p.q_sb + h * p.q_sh;
  const uint16_t* Kb = static_cast<const uint16_t*>(p.k) + b * p.k_sb + hk * p.k_sh;
  const uint16_t* Vb = static_cast<const uint16_t*>(p.v) + b * p.v_sb + hk * p.v_sh;

  // Q fragments (B operand of S^T): query qi, d = 16s + 8*h2 .. +8.
  bf16x8_t qf[DP / 16];
#pragma unroll
  for (int s = 0; s < DP / 16; ++s) {
    if (qv && 16 * s + 8 * h2 < D)
      qf[s] = *reinterpret_cast<const bf16x8_t*>(Q + static_cast<int64_t>(qi) * p.q_ss + 16 * s + 8 * h2);
    else
      qf[s] = bf16x8_t{};
  }
  // This lane's mask row (query qi of (b, h)); keys step by m_sk.
  const int64_t mrow = b * p.m_sb + h * p.m_sh + static_cast<int64_t>(qv ? qi : 0) * p.m_sq;

  // Keys [kv_beg, kv_end) in tiles t0 .. ntiles-1; with a split key range the
  // chunk bounds are multiples of the tile, so a split's tiles hold its keys only.
  const int split = static_cast<int>(blockIdx.y);
  const int kv_all = p.causal ? min(p.Sk, q0 + kBQ) : p.Sk;
  const int kv_beg = p.kv_chunk ? split * p.kv_chunk : 0;
  const int kv_end = p.kv_chunk ? min(kv_all, kv_beg + p.kv_chunk) : kv_all;
  const int t0 = kv_beg / kBKV;
  const int ntiles = (kv_end + kBKV - 1) / kBKV;
  // scale_log2 > 0, so the running max is kept on the raw scores and the scale
  // is folded into one FMA per exponent: exp2(s * c - m * c).
  const float c = p.scale_log2;

  // Per-lane byte offsets of this wave's NDMA K and NDMA V DMA instructions within
  // a tile (instruction i fills key rows RPI (NDMA wave + i) .. +RPI, NCH lanes a
  // row).  Keys past Sk lie beyond the descriptor's extent and read zeros.
  uint32_t koff[NDMA], voff[NDMA];
#pragma unroll
  for (int i = 0; i < NDMA; ++i) {
    const int r = (wave * NDMA + i) * RPI + lane / NCH;
    const int cc = lane % NCH;
    const int gk = cc ^ swz_k<DP>(r), gv = cc ^ swz_v<DP>(r);  // global chunks this lane loads
    koff[i] = 8 * gk < D ? static_cast<uint32_t>((static_cast<int64_t>(r) * p.k_ss + gk * 8) * 2) : kPastEnd;
    voff[i] = 8 * gv < D ? static_cast<uint32_t>((static_cast<int64_t>(r) * p.v_ss + gv * 8) * 2) : kPastEnd;
  }
  using Off = typename KvOff<BIG>::T;
  const Off kstep = static_cast<Off>(kBKV * p.k_ss * 2), vstep = static_cast<Off>(kBKV * p.v_ss * 2);
  auto issue = [&](int t, int st) {
    const Off dk = static_cast<Off>(t) * kstep, dv = static_cast<Off>(t) * vstep;
    const i32x4_t rk = make_rsrc(reinterpret_cast<const char*>(Kb) + dk, KvOff<BIG>::rec(p.k_extent, p.k_extent64, dk));
    const i32x4_t rv = make_rsrc(reinterpret_cast<const char*>(Vb) + dv, KvOff<BIG>::rec(p.v_extent, p.v_extent64, dv));
    const uint32_t lk = lds0 + static_cast<uint32_t>(st) * (2 * kBKV * DP * 2) + wave * NDMA * 1024;
    const uint32_t lv = lk + kBKV * DP * 2;
#pragma unroll
    for (int i = 0; i < NDMA; ++i) dma16(rk, lk + i * 1024, koff[i]);
#pragma unroll
    for (int i = 0; i < NDMA; ++i) dma16(rv, lv + i * 1024, voff[i]);
  };
  auto issue_k = [&](int t) {
    const Off dk = static_cast<Off>(t) * kstep;
    const i32x4_t rk = make_rsrc(reinterpret_cast<const char*>(Kb) + dk, KvOff<BIG>::rec(p.k_extent, p.k_extent64, dk));
    const uint32_t lk = lds0 + wave * NDMA * 1024;
#pragma unroll
    for (int i = 0; i < NDMA; ++i) dma16(rk, lk + i * 1024, koff[i]);
  };
  auto issue_v = [&](int t) {
    const Off dv = static_cast<Off>(t) * vstep;
    const i32x4_t rv = make_rsrc(reinterpret_cast<const char*>(Vb) + dv, KvOff<BIG>::rec(p.v_extent, p.v_extent64, dv));
    const uint32_t lv = lds0 + kBKV * DP * 2 + wave * NDMA * 1024;
#pragma unroll
    for (int i = 0; i < NDMA; ++i) dma16(rv, lv + i * 1024, voff[i]);
  };

  f32x16_t o[DP / 32];
#pragma unroll
  for (int db = 0; db < DP / 32; ++db)
#pragma unroll
    for (int v = 0; v < 16; ++v) o[db][v] = 0.f;
  float m = -INFINITY;  // reference max (raw scores) the exponents are taken against
  float l = 0.f;        // running sum over this half-wave's keys

  // Mask values of the 4-key group g (keys key0 + 32 kb + 4 h2 + 8 g + 0..3) for
  // score register pair v = 4 g .. 4 g + 3 of s{kb}: keep flags or additive terms.
  auto mask_group = [&](int key, float* out) {
    if constexpr (MK == kBoolMask) {
      const uint8_t* mp = static_cast<const uint8_t*>(p.mask) + mrow;
      if (p.mask_vec && key + 3 < p.Sk) {
        const uint32_t w = *reinterpret_cast<const uint32_t*>(mp + key);
#pragma unroll
        for (int e = 0; e < 4; ++e) out[e] = ((w >> (8 * e)) & 0xffu) ? 0.f : -INFINITY;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          out[e] = (key + e < p.Sk && !mp[static_cast<int64_t>(key + e) * p.m_sk]) ? -INFINITY : 0.f;
      }
    } else {
      const uint16_t* mp = static_cast<const uint16_t*>(p.mask) + mrow;
      if (p.mask_vec && key + 3 < p.Sk) {
        const uint2 w = *reinterpret_cast<const uint2*>(mp + key);
        out[0] = from16<F16>(static_cast<uint16_t>(w.x));
        out[1] = from16<F16>(static_cast<uint16_t>(w.x >> 16));
        out[2] = from16<F16>(static_cast<uint16_t>(w.y));
        out[3] = from16<F16>(static_cast<uint16_t>(w.y >> 16));
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          out[e] = key + e < p.Sk ? from16<F16>(mp[static_cast<int64_t>(key + e) * p.m_sk]) : 0.f;
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) out[e] *= p.inv_scale;
    }
  };

  // Scores, softmax and the P^T operand of tile t (keys t * 64 ..) from the K tile
  // in LDS; the caller has checked that the wave has keys to process there.
  auto scores = [&](int t, bf16x8_t (&pb)[4]) {
    const int key0 = t * kBKV;
    // The mask terms of this tile, fetched before the MFMAs so their latency
    // overlaps them.
    float mk[2][16];
    if constexpr (MK != kNoMask) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int g = 0; g < 4; ++g) mask_group(key0 + 32 * kb + 4 * h2 + 8 * g, &mk[kb][4 * g]);
    }
    const uint16_t* sk = &smem[0][0][0];
    f32x16_t s0, s1;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      s0[v] = 0.f;
      s1[v] = 0.f;
    }
#pragma unroll
    for (int s = 0; s < DP / 16; ++s) {
      s0 = mma<F16>(frag_k<DP>(sk, 0, s, lane), qf[s], s0);
      s1 = mma<F16>(frag_k<DP>(sk, 1, s, lane), qf[s], s1);
    }
    // s{kb}[v] is key key0 + 32 kb + 4 h2 + kv, kv = (v/4)*8 + v%4, for query qi.
    if constexpr (MK != kNoMask) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        s0[v] += mk[0][v];
        s1[v] += mk[1][v];
      }
    }
    // Only the diagonal tile(s) and a ragged last tile need the element mask:
    // visible iff kv (+32 for s1) < lim.
    if ((p.causal && key0 + kBKV - 1 > qw) || key0 + kBKV > p.Sk) {
      const int lim = min(p.Sk, p.causal ? qi + 1 : p.Sk) - key0 - 4 * h2;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int kv = (v >> 2) * 8 + (v & 3);
        s0[v] = kv < lim ? s0[v] : -INFINITY;
        s1[v] = kv + 32 < lim ? s1[v] : -INFINITY;
      }
    }
    // v_max3_f32 directly: fmaxf would first quiet every MFMA result with a
    // second v_max (MFMA results are never signaling NaNs).
    float mx = -INFINITY;
#pragma unroll
    for (int v = 0; v < 16; ++v) asm("v_max3_f32 %0, %1, %2, %3" : "=v"(mx) : "v"(mx), "v"(s0[v]), "v"(s1[v]));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    // Lazy rescale: the reference max only moves (with o and l rescaled) when
    // some lane's tile max exceeds it by more than kLazyLog2, so exponents stay
    // <= 2^kLazyLog2 and the multiplies of the rescale are rare.  The result
    // o / l does not depend on the reference chosen.
    if (__builtin_amdgcn_ballot_w64((mx - m) * c > kLazyLog2)) {
      const float mnew = fmaxf(m, mx);
      // v_exp_f32 directly: weights below 2^-126 flush to zero.
      const float alpha = mnew == -INFINITY ? 1.f : __builtin_amdgcn_exp2f((m - mnew) * c);
      m = mnew;
      l *= alpha;
#pragma unroll
      for (int db = 0; db < DP / 32; ++db)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[db][v] *= alpha;
    }
    // A query with nothing unmasked yet keeps m = -inf and exponent offset 0.
    const float nb = m == -INFINITY ? 0.f : -m * c;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      s0[v] = __builtin_amdgcn_exp2f(__builtin_fmaf(s0[v], c, nb));
      s1[v] = __builtin_amdgcn_exp2f(__builtin_fmaf(s1[v], c, nb));
    }
    // P^T operand of key step s: s{s/2}[8 (s%2) .. +8] rounded to the 16-bit type,
    // two values per conversion.  The running sum adds the same rounded weights
    // (one dot2 against (1, 1) per pair), so the normalisation divides by exactly
    // the weights the P V product used.
    uint32_t pw[16];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      pw[i] = pack16x2<F16>(s0[2 * i], s0[2 * i + 1]);
      pw[8 + i] = pack16x2<F16>(s1[2 * i], s1[2 * i + 1]);
    }
    float ls0 = 0.f, ls1 = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      ls0 = dot2_ones<F16>(pw[2 * i], ls0);
      ls1 = dot2_ones<F16>(pw[2 * i + 1], ls1);
    }
    l += ls0 + ls1;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      pb[k] = __builtin_bit_cast(bf16x8_t, make_uint4(pw[4 * k], pw[4 * k + 1], pw[4 * k + 2], pw[4 * k + 3]));
  };
  // O^T += V^T P^T over the V tile in LDS.
  auto pv = [&](const bf16x8_t (&pb)[4]) {
    const uint16_t* sv = &smem[0][1][0];
#pragma unroll
    for (int s = 0; s < kBKV / 16; ++s)
#pragma unroll
      for (int db = 0; db < DP / 32; ++db) o[db] = mma<F16>(frag_v<DP>(sv, db, s, lane), pb[s], o[db]);
  };
  // Causal: a wave whose last query precedes tile t's first key has nothing to do
  // there; neither has a wave without rows (decoding: a handful of rows in the
  // first wave).  It still takes part in the barriers and loads.
  const bool wave_rows = __builtin_amdgcn_ballot_w64(qv) != 0;
  auto skip = [&](int t) { return !wave_rows || (p.causal && t * kBKV > qw + kQW - 1); };

  if constexpr (!SPLIT) {
    // Two barriers per tile: the first once every wave has finished reading tile
    // t-1 (the stage may be refilled), the second once tile t has landed.
    auto tile = [&](int t) {
      __syncthreads();
      issue(t, 0);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (!skip(t)) {
        bf16x8_t pb[4];
        scores(t, pb);
        pv(pb);
      }
      // The stage's LDS reads complete before the next barrier, after which it is
      // refilled.
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    };
    for (int t = t0; t < ntiles; t += 2) {
      tile(t);
      if (t + 1 < ntiles) tile(t + 1);
    }
  } else {
    // K and V load separately, each under the other half of the tile: V_t during
    // the scores of tile t, K_{t+1} during P V of tile t (three barriers a tile; the
    // first tile's K and V are both issued up front).  vmcnt counts this wave's
    // DMA instructions in issue order: NDMA of them per K or V tile.
    constexpr int kWaitOneTile = NDMA | (7 << 4) | (15 << 8);  // vmcnt(NDMA), other counters not waited
    static_assert(NDMA < 16, "vmcnt immediate");
    // (A split with no keys for this query block issues nothing.)
    if (t0 < ntiles) {
      issue_k(t0);
      issue_v(t0);
    }
    for (int t = t0; t < ntiles; ++t) {
      if (t == t0) __builtin_amdgcn_s_waitcnt(kWaitOneTile);  // K_t0 landed (V_t0 may be in flight)
      else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // K_t landed
      __syncthreads();  // K_t visible; every wave done with P V of tile t-1
      if (t > t0) issue_v(t);
      bf16x8_t pb[4];
      const bool sk = skip(t);
      if (!sk) scores(t, pb);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __syncthreads();  // every wave done reading K_t
      if (t + 1 < ntiles) {
        issue_k(t + 1);
        __builtin_amdgcn_s_waitcnt(kWaitOneTile);  // V_t landed, K_{t+1} in flight
      } else {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      }
      __syncthreads();  // V_t visible
      if (!sk) pv(pb);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
  }

  // o[db][v] is d = 32 db + (v/4)*8 + 4 h2 + v%4 of query qi.  A query whose keys
  // are all masked has l = 0: its output is NaN, as the reference's softmax of a
  // row of -inf gives.
  const float lt = l + __shfl_xor(l, 32, 64);
  if (p.kv_chunk) {
    // One split's share: o / l in fp32 and the log2-sum-exp m c + log2 l of its
    // scaled scores (-inf, with o = 0, when none of its keys is visible).
    if (qv) {
      const int64_t row = ((static_cast<int64_t>(split) * p.B + b) * p.H + h) * p.Sq + qi;
      const float winv = lt > 0.f ? 1.0f / lt : 0.f;
      float* po = p.part_o + row * D;
#pragma unroll
      for (int db = 0; db < DP / 32; ++db)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d = db * 32 + g * 8 + 4 * h2;
          if (d >= D) continue;
          *reinterpret_cast<float4*>(po + d) = make_float4(o[db][g * 4 + 0] * winv, o[db][g * 4 + 1] * winv,
                                                           o[db][g * 4 + 2] * winv, o[db][g * 4 + 3] * winv);
        }
      if (h2 == 0) p.part_lse[row] = lt > 0.f ? m * c + __builtin_amdgcn_logf(lt) : -INFINITY;
    }
    return;
  }
  const float inv = 1.0f / lt;
  if (qv) {
    uint16_t* O = static_cast<uint16_t*>(p.o) + b * p.o_sb + h * p.o_sh + static_cast<int64_t>(qi) * p.o_ss;
#pragma unroll
    for (int db = 0; db < DP / 32; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = db * 32 + g * 8 + 4 * h2;
        if (d >= D) continue;  // D is a multiple of 8: d < D covers d .. d + 3
        const float r0 = lt > 0.f ? o[db][g * 4 + 0] * inv : __builtin_nanf("");
        const float r1 = lt > 0.f ? o[db][g * 4 + 1] * inv : __builtin_nanf("");
        const float r2 = lt > 0.f ? o[db][g * 4 + 2] * inv : __builtin_nanf("");
        const float r3 = lt > 0.f ? o[db][g * 4 + 3] * inv : __builtin_nanf("");
        *reinterpret_cast<uint2*>(O + d) = make_uint2(pack16x2<F16>(r0, r1), pack16x2<F16>(r2, r3));
      }
  }
}

template <int DP, bool F16, bool SPLIT, bool BIG>
static void launch_dm(const Params& p, int mk, dim3 grid, hipStream_t s) {
  static_assert(!SPLIT, "masked kernels use the plain schedule");
  if (mk == kBoolMask) hipLaunchKernelGGL((sdpa_fwd_kernel<DP, F16, kBoolMask, SPLIT, BIG>), grid, dim3(256), 0, s, p);
  else if (mk == kAddMask) hipLaunchKernelGGL((sdpa_fwd_kernel<DP, F16, kAddMask, SPLIT, BIG>), grid, dim3(256), 0, s, p);
  else hipLaunchKernelGGL((sdpa_fwd_kernel<DP, F16, kNoMask, SPLIT, BIG>), grid, dim3(256), 0, s, p);
}
// The split schedule only without a mask: with one, the compiler's waits for the
// mask loads also wait for the K / V DMA (vmcnt counts both in issue order), and
// the masked variants would spill at the extra barrier.
// BIG: K / V slices of 2 GiB or more (KvOff).
template <int DP, bool F16, bool BIG>
static void launch_db(const Params& p, int mk, dim3 grid, bool split, hipStream_t s) {
  if (split && mk == kNoMask) hipLaunchKernelGGL((sdpa_fwd_kernel<DP, F16, kNoMask, true, BIG>), grid, dim3(256), 0, s, p);
  else launch_dm<DP, F16, false, BIG>(p, mk, grid, s);
}
template <int DP, bool F16>
static void launch_d(const Params& p, int mk, dim3 grid, bool split, bool big, hipStream_t s) {
  if (big) launch_db<DP, F16, true>(p, mk, grid, split, s);
  else launch_db<DP, F16, false>(p, mk, grid, split, s);
}


// fp32 Q / K / V / O: the same structure on v_mfma_f32_32x32x2_f32 (fp32 products
// and sums throughout, P never rounded), with 32-key K / V tiles held as fp32 in LDS
// (32 KiB at DP = 128).  Each lane again owns one query column:
//   * S^T = K Q^T: MFMA step (g, e), g < DP / 8, e < 4, takes head dim d = 8g + 4h +
//     e in lane half h.  A lane reads those 4 values of its key row with one
//     ds_read_b128 (16-byte chunk c of row r sits at slot c ^ (r % 8), so the 8 rows
//     of a b128 phase land in distinct bank groups) and holds Q's in registers;
//   * O^T = V^T P^T: MFMA step j < 16 takes key 8 (j / 4) + 4h + j % 4 in lane half
//     h, which is where register j of that lane's S^T accumulator lies, so P enters
//     the MFMA straight from the accumulator; V^T is read one value a lane (the 32
//     lanes of a half on 32 consecutive head-dim values of one key row).
// Head dims below DP are padded as in the 16-bit kernel (zero chunks, unstored
// output columns); D is a multiple of 4.
constexpr int kKT32 = 32;  // keys per fp32 tile

// Two workgroups a CU, except DP = 128 with a boolean mask, whose ~260 registers
// a lane need the accumulation registers of a one-wave-per-SIMD launch.
template <int DP, int MK>
__global__ __launch_bounds__(256, DP >= 128 && MK == kBoolMask ? 1 : 2) void sdpa_fwd_f32_kernel(Params p) {
  constexpr int KT = kKT32;
  constexpr int NCH = DP / 4;                         // 16-byte chunks per row
  constexpr int NDMA = KT * DP * 4 / 1024 / kWaves;   // DMA instructions per wave per K (or V) tile
  constexpr int RPI = 256 / DP;                       // rows per DMA instruction
  __shared__ __attribute__((aligned(1024))) float smem[2][KT * DP];  // K | V
  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((GHIP_ALDS void*)&smem[0][0]));

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h2 = lane >> 5;
  const int D = p.D;
  const int nqb = (p.Sq + kBQ - 1) / kBQ;
  const int nbh = p.B * p.H;
  const int qb = p.causal ? (nqb - 1 - static_cast<int>(blockIdx.x / nbh)) : static_cast<int>(blockIdx.x / nbh);
  const int bh = blockIdx.x % nbh;
  const int b = bh / p.H, h = bh % p.H;
  const int hk = h / (p.H / p.Hkv);
  const int q0 = qb * kBQ;
  const int qw = q0 + wave * kQW;
  const int qi = qw + (lane & 31);

  const float* Q = static_cast<const float*>(p.q) + b * p.q_sb + h * p.q_sh;
  const float* Kb = static_cast<const float*>(p.k) + b * p.k_sb + hk * p.k_sh;
  const float* Vb = static_cast<const float*>(p.v) + b * p.v_sb + hk * p.v_sh;

  // Q values of this lane: query qi, d = 8g + 4 h2 .. +4.
  float4 qf[DP / 8];
#pragma unroll
  for (int g = 0; g < DP / 8; ++g) {
    const int d = 8 * g + 4 * h2;
    qf[g] = qi < p.Sq && d < D ? *reinterpret_cast<const float4*>(Q + static_cast<int64_t>(qi) * p.q_ss + d)
                               : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  const int64_t mrow = b * p.m_sb + h * p.m_sh + static_cast<int64_t>(qi < p.Sq ? qi : 0) * p.m_sq;

  const int kv_end = p.causal ? min(p.Sk, q0 + kBQ) : p.Sk;
  const int ntiles = (kv_end + KT - 1) / KT;
  const float c = p.scale_log2;

  uint32_t koff[NDMA], voff[NDMA];
#pragma unroll
  for (int i = 0; i < NDMA; ++i) {
    const int r = (wave * NDMA + i) * RPI + lane / NCH;
    const int cc = lane % NCH;
    const int gk = cc ^ (r & 7);
    koff[i] = 4 * gk < D ? static_cast<uint32_t>((static_cast<int64_t>(r) * p.k_ss + gk * 4) * 4) : kPastEnd;
    voff[i] = 4 * cc < D ? static_cast<uint32_t>((static_cast<int64_t>(r) * p.v_ss + cc * 4) * 4) : kPastEnd;
  }
  const uint32_t kstep = static_cast<uint32_t>(KT * p.k_ss * 4), vstep = static_cast<uint32_t>(KT * p.v_ss * 4);
  auto issue = [&](int t) {
    const uint32_t dk = static_cast<uint32_t>(t) * kstep, dv = static_cast<uint32_t>(t) * vstep;
    const i32x4_t rk = make_rsrc(reinterpret_cast<const char*>(Kb) + dk, p.k_extent - dk);
    const i32x4_t rv = make_rsrc(reinterpret_cast<const char*>(Vb) + dv, p.v_extent - dv);
    const uint32_t lk = lds0 + wave * NDMA * 1024;
    const uint32_t lv = lk + KT * DP * 4;
#pragma unroll
    for (int i = 0; i < NDMA; ++i) dma16(rk, lk + i * 1024, koff[i]);
#pragma unroll
    for (int i = 0; i < NDMA; ++i) dma16(rv, lv + i * 1024, voff[i]);
  };

  f32x16_t o[DP / 32];
#pragma unroll
  for (int db = 0; db < DP / 32; ++db)
#pragma unroll
    for (int v = 0; v < 16; ++v) o[db][v] = 0.f;
  float m = -INFINITY, l = 0.f;

  // Keep flags of keys key .. key + 3 (score registers 4g .. 4g + 3), one byte each
  // of a word (keys past Sk are kept: the element mask drops them).
  auto keep_group = [&](int key) -> uint32_t {
    const uint8_t* mp = static_cast<const uint8_t*>(p.mask) + mrow;
    if (p.mask_vec && key + 3 < p.Sk) return *reinterpret_cast<const uint32_t*>(mp + key);
    uint32_t w = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      w |= (key + e >= p.Sk || mp[static_cast<int64_t>(key + e) * p.m_sk]) ? (1u << (8 * e)) : 0u;
    return w;
  };
  // Additive terms of keys key .. key + 3, divided by the scale.
  auto add_group = [&](int key, float* out) {
    {
      const float* mp = static_cast<const float*>(p.mask) + mrow;
      if (p.mask_vec && key + 3 < p.Sk) {
        const float4 w = *reinterpret_cast<const float4*>(mp + key);
        out[0] = w.x; out[1] = w.y; out[2] = w.z; out[3] = w.w;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) out[e] = key + e < p.Sk ? mp[static_cast<int64_t>(key + e) * p.m_sk] : 0.f;
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) out[e] *= p.inv_scale;
    }
  };

  const float* sk = &smem[0][0];
  const float* sv = &smem[1][0];
  for (int t = 0; t < ntiles; ++t) {
    __syncthreads();
    issue(t);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    const int key0 = t * KT;
    if (p.causal && key0 > qw + kQW - 1) continue;
    float mk[MK == kAddMask ? 16 : 1];
    uint32_t mw[4];
    if constexpr (MK == kAddMask) {
#pragma unroll
      for (int g = 0; g < 4; ++g) add_group(key0 + 4 * h2 + 8 * g, &mk[4 * g]);
    } else if constexpr (MK == kBoolMask) {
#pragma unroll
      for (int g = 0; g < 4; ++g) mw[g] = keep_group(key0 + 4 * h2 + 8 * g);
    }
    f32x16_t sc;
#pragma unroll
    for (int v = 0; v < 16; ++v) sc[v] = 0.f;
    const int row = lane & 31;
#pragma unroll
    for (int g = 0; g < DP / 8; ++g) {
      const float4 kf = *reinterpret_cast<const float4*>(sk + row * DP + (((2 * g + h2) ^ (row & 7)) * 4));
      sc = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.x, qf[g].x, sc, 0, 0, 0);
      sc = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.y, qf[g].y, sc, 0, 0, 0);
      sc = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.z, qf[g].z, sc, 0, 0, 0);
      sc = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.w, qf[g].w, sc, 0, 0, 0);
    }
    // sc[v] is key key0 + 4 h2 + kv, kv = (v/4)*8 + v%4, for query qi.
    if constexpr (MK == kAddMask) {
#pragma unroll
      for (int v = 0; v < 16; ++v) sc[v] += mk[v];
    } else if constexpr (MK == kBoolMask) {
#pragma unroll
      for (int v = 0; v < 16; ++v) sc[v] = (mw[v >> 2] >> (8 * (v & 3))) & 0xffu ? sc[v] : -INFINITY;
    }
    if ((p.causal && key0 + KT - 1 > qw) || key0 + KT > p.Sk) {
      const int lim = min(p.Sk, p.causal ? qi + 1 : p.Sk) - key0 - 4 * h2;
#pragma unroll
      for (int v = 0; v < 16; ++v) sc[v] = (v >> 2) * 8 + (v & 3) < lim ? sc[v] : -INFINITY;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int v = 0; v < 16; v += 2) asm("v_max3_f32 %0, %1, %2, %3" : "=v"(mx) : "v"(mx), "v"(sc[v]), "v"(sc[v + 1]));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    if (__builtin_amdgcn_ballot_w64((mx - m) * c > kLazyLog2)) {
      const float mnew = fmaxf(m, mx);
      const float alpha = mnew == -INFINITY ? 1.f : __builtin_amdgcn_exp2f((m - mnew) * c);
      m = mnew;
      l *= alpha;
#pragma unroll
      for (int db = 0; db < DP / 32; ++db)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[db][v] *= alpha;
    }
    const float nb = m == -INFINITY ? 0.f : -m * c;
    float ls = 0.f;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      sc[v] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[v], c, nb));
      ls += sc[v];
    }
    l += ls;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int key = 8 * (j >> 2) + 4 * h2 + (j & 3);
#pragma unroll
      for (int db = 0; db < DP / 32; ++db)
        o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(sv[key * DP + 32 * db + row], sc[j], o[db], 0, 0, 0);
      // V reads are not hoisted more than 4 keys ahead (registers: 2 waves a SIMD).
      if ((j & 3) == 3) __builtin_amdgcn_sched_barrier(0);
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  }

  // o[db][v] is d = 32 db + (v/4)*8 + 4 h2 + v%4 of query qi.
  const float lt = l + __shfl_xor(l, 32, 64);
  const float inv = 1.0f / lt;
  if (qi < p.Sq) {
    float* O = static_cast<float*>(p.o) + b * p.o_sb + h * p.o_sh + static_cast<int64_t>(qi) * p.o_ss;
#pragma unroll
    for (int db = 0; db < DP / 32; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = db * 32 + g * 8 + 4 * h2;
        if (d >= D) continue;  // D is a multiple of 4
        const float nan = __builtin_nanf("");
        *reinterpret_cast<float4*>(O + d) =
            make_float4(lt > 0.f ? o[db][g * 4 + 0] * inv : nan, lt > 0.f ? o[db][g * 4 + 1] * inv : nan,
                        lt > 0.f ? o[db][g * 4 + 2] * inv : nan, lt > 0.f ? o[db][g * 4 + 3] * inv : nan);
      }
  }
}

template <int DP>
static void launch_f32(const Params& p, int mk, dim3 grid, hipStream_t s) {
  if (mk == kBoolMask) hipLaunchKernelGGL((sdpa_fwd_f32_kernel<DP, kBoolMask>), grid, dim3(256), 0, s, p);
  else if (mk == kAddMask) hipLaunchKernelGGL((sdpa_fwd_f32_kernel<DP, kAddMask>), grid, dim3(256), 0, s, p);
  else hipLaunchKernelGGL((sdpa_fwd_f32_kernel<DP, kNoMask>), grid, dim3(256), 0, s, p);
}

// Combine of a split key range (16-bit outputs): for each (b, h, query) row the
// splits' outputs weighted by 2^(lse_i - max lse), summed in split order (the same
// bits every run); a row none of whose keys is visible gets NaN, as without the
// split.  One wave per row, four head-dim values a lane (D <= 256).
template <bool F16>
__global__ __launch_bounds__(256) void sdpa_combine_kernel(Params p, int ns) {
  const int64_t rows = static_cast<int64_t>(p.B) * p.H * p.Sq;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + threadIdx.x / 64;
  const int d = (threadIdx.x % 64) * 4;
  if (row >= rows || d >= p.D) return;
  // The row is the same for the whole wave.  The splits' loads do not depend on
  // each other: they are issued kC at a time before any of them is used (the max
  // pass, then the weighted sum), so a row waits for ceil(ns / kC) + 1 memory
  // latencies rather than one per split.
  constexpr int kC = 16;
  const float* lse = p.part_lse + row;
  const float* po = p.part_o + row * p.D + d;
  const int64_t so = rows * p.D;  // one split's outputs
  float mx = -INFINITY;
  for (int i0 = 0; i0 < ns; i0 += kC) {
    float l[kC];
#pragma unroll
    for (int j = 0; j < kC; ++j) l[j] = i0 + j < ns ? lse[(i0 + j) * rows] : -INFINITY;
#pragma unroll
    for (int j = 0; j < kC; ++j) mx = fmaxf(mx, l[j]);
  }
  float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f, wsum = 0.f;
  for (int i0 = 0; i0 < ns; i0 += kC) {
    float l[kC];
    float4 v[kC];
#pragma unroll
    for (int j = 0; j < kC; ++j)
      if (i0 + j < ns) {
        l[j] = lse[(i0 + j) * rows];
        v[j] = *reinterpret_cast<const float4*>(po + (i0 + j) * so);
      }
    // Split order: the same sums every run.
#pragma unroll
    for (int j = 0; j < kC; ++j)
      if (i0 + j < ns) {
        // A split with no visible key (lse -inf) adds nothing, whatever its o holds.
        const bool live = l[j] != -INFINITY;
        const float w = live ? __builtin_amdgcn_exp2f(l[j] - mx) : 0.f;
        a0 += live ? w * v[j].x : 0.f;
        a1 += live ? w * v[j].y : 0.f;
        a2 += live ? w * v[j].z : 0.f;
        a3 += live ? w * v[j].w : 0.f;
        wsum += w;
      }
  }
  const bool none = mx == -INFINITY;
  const float inv = none ? 0.f : 1.0f / wsum;
  const float nan = __builtin_nanf("");
  const int qi = static_cast<int>(row % p.Sq);
  const int64_t bh = row / p.Sq;
  const int h = static_cast<int>(bh % p.H), b = static_cast<int>(bh / p.H);
  uint16_t* O = static_cast<uint16_t*>(p.o) + b * p.o_sb + h * p.o_sh + static_cast<int64_t>(qi) * p.o_ss + d;
  *reinterpret_cast<uint2*>(O) = make_uint2(pack16x2<F16>(none ? nan : a0 * inv, none ? nan : a1 * inv),
                                            pack16x2<F16>(none ? nan : a2 * inv, none ? nan : a3 * inv));
}

// Key-range splits for grids of few workgroups, 16-bit operands: below 384
// workgroups (half of the 768 that fit at three per CU) each one's keys are split
// so that the grid comes near 768, every split keeping at least 4 key tiles (at
// most 64 splits).  When the grid holds several row blocks per (b, h) (prefill),
// only for 64 key tiles or more: the partial outputs of many rows cost more than
// the extra parallelism gains below that (B1 H16 S2048, causal or not, 12-22%
// slower split; Sq 1024 over 8192 keys 2.2x faster).  ns = 1: no split.
struct KvSplit {
  int ns;
  int chunk;  // keys per split (a multiple of kBKV)
};
// Workgroups of the kernel's grid (x): (query block, b, h), or with grouped-query
// rows (16-bit, no causal mask, GQA, Sq < 128: decoding) (row block, b, kv head).
struct SdpaGrid {
  int64_t wgs;
  bool pack;
  bool one_block;  // one row block per (b, h) or per (b, kv head) group
  int64_t kv;      // keys of the longest workgroup (causal: up to its last query)
};
static SdpaGrid sdpa_grid(int dtype, int64_t B, int64_t H, int64_t Hkv, int64_t Sq, int64_t Sk, int causal) {
  const bool pack = dtype != GHIP_DTYPE_FLOAT32 && !causal && Hkv > 0 && Hkv < H && H % Hkv == 0 && Sq < kBQ;
  const int64_t nqb = (Sq + kBQ - 1) / kBQ;
  const int64_t kv = causal ? std::min<int64_t>(Sk, nqb * kBQ) : Sk;
  if (pack) {
    const int64_t nrb = (H / Hkv * Sq + kBQ - 1) / kBQ;
    return SdpaGrid{nrb * B * Hkv, true, nrb == 1, kv};
  }
  return SdpaGrid{nqb * B * H, false, nqb == 1, kv};
}
static KvSplit kv_split(int dtype, const SdpaGrid& g) {
  const KvSplit none{1, 0};
  const int64_t grid = g.wgs;
  if (dtype == GHIP_DTYPE_FLOAT32 || grid <= 0 || g.kv <= 0) return none;
  const int64_t tiles = (g.kv + kBKV - 1) / kBKV;
  if (grid >= 384 || tiles < 8 || (!g.one_block && tiles < 64)) return none;
  int64_t ns = std::min<int64_t>((768 + grid - 1) / grid, tiles / 4);
  ns = std::min<int64_t>(ns, 64);
  if (ns < 2) return none;
  const int64_t per = (tiles + ns - 1) / ns;
  ns = (tiles + per - 1) / per;
  if (ns < 2) return none;
  return KvSplit{static_cast<int>(ns), static_cast<int>(per * kBKV)};
}
static int64_t kv_split_bytes(const KvSplit& ks, int64_t B, int64_t H, int64_t Sq, int64_t D) {
  return ks.ns > 1 ? static_cast<int64_t>(ks.ns) * B * H * Sq * (D + 1) * 4 : 0;
}

}  // namespace attn

// Whether ghip_sdpa_fwd_masked takes these operands (checked again, with the
// pointers, by the entry point).  Strides are in elements, ordered (batch, head,
// sequence); the head dim must be contiguous.  mask_dtype < 0: no mask.
//   bf16 / f16: head dim a multiple of 8 up to 256; strides multiples of 8 (4 for
//   the output).  fp32: head dim a multiple of 4 up to 128; strides multiples of 4.
bool sdpa_fused_supported(int dtype, int64_t H, int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D,
                          const int64_t* qs, const int64_t* ks, const int64_t* vs, const int64_t* os,
                          float scale, int mask_dtype) {
  const bool f32 = dtype == GHIP_DTYPE_FLOAT32;
  if (!f32 && dtype != GHIP_DTYPE_BFLOAT16 && dtype != GHIP_DTYPE_FLOAT16) return false;
  const int64_t es = f32 ? 4 : 2;
  const int64_t in_al = 16 / es;  // 16-byte rows for the DMA and Q loads
  const int64_t out_al = 4;  // 16 bytes (fp32) or 8 (16-bit): the output stores
  if (D <= 0 || D % in_al != 0 || D > (f32 ? 128 : 256)) return false;
  if (Hkv <= 0 || H % Hkv != 0) return false;
  if (mask_dtype >= 0 && mask_dtype != GHIP_DTYPE_BOOL && mask_dtype != dtype) return false;
  if (!(scale > 0.f) || !(scale < 1e30f)) return false;  // positive and finite
  if (Sq <= 0 || Sk <= 0 || Sq > (int64_t{1} << 30) || Sk > (int64_t{1} << 30)) return false;
  for (const int64_t* s : {qs, ks, vs})
    for (int i = 0; i < 3; ++i)
      if (s[i] < 0 || s[i] % in_al != 0) return false;
  for (int i = 0; i < 3; ++i)
    if (os[i] < 0 || os[i] % out_al != 0) return false;
  // A key tile (64 keys) of K / V lies within 2 GiB of its first row; the slice of
  // one (batch, kv head) may be any size with 16-bit operands (the BIG kernels),
  // below 2 GiB with fp32 ones.
  if ((64 * ks[2] + 256) * es >= (int64_t{1} << 31) || (64 * vs[2] + 256) * es >= (int64_t{1} << 31)) return false;
  if (f32 && (((Sk - 1) * ks[2] + D) * es >= (int64_t{1} << 31) || ((Sk - 1) * vs[2] + D) * es >= (int64_t{1} << 31)))
    return false;
  return true;
}

}  // namespace ghip

using namespace ghip;

extern "C" int64_t ghip_sdpa_workspace_bytes(int dtype, int64_t B, int64_t H, int64_t Hkv, int64_t Sq, int64_t Sk,
                                             int64_t D, int causal) {
  if (B <= 0 || H <= 0 || Hkv <= 0 || Sq <= 0 || Sk <= 0 || D <= 0) return 0;
  const attn::SdpaGrid g = attn::sdpa_grid(dtype, B, H, Hkv, Sq, Sk, causal);
  return attn::kv_split_bytes(attn::kv_split(dtype, g), B, H, Sq, D);
}

extern "C" int ghip_sdpa_fwd_masked_ws(int dtype, const void* q, const void* k, const void* v, void* o,
                                       int64_t B, int64_t H, int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D,
                                       const int64_t* q_strides, const int64_t* k_strides,
                                       const int64_t* v_strides, const int64_t* o_strides, const void* mask,
                                       int mask_dtype, const int64_t* mask_strides, float scale, int causal,
                                       void* workspace, int64_t workspace_bytes, void* stream, GHipError* err) {
  if (B < 0 || H <= 0 || Hkv <= 0 || Sq < 0 || Sk < 0 || D <= 0)
    return set_error(err, GHIP_ERR_INVALID_ARG, "sdpa_fwd: bad sizes");
  if (H % Hkv != 0)
    return set_error(err, GHIP_ERR_INVALID_ARG, "sdpa_fwd: num_heads (%lld) must be a multiple of num_kv_heads (%lld)",
                     static_cast<long long>(H), static_cast<long long>(Hkv));
  if (!q_strides || !k_strides || !v_strides || !o_strides)
    return set_error(err, GHIP_ERR_INVALID_ARG, "sdpa_fwd: null strides");
  if (mask && !mask_strides) return set_error(err, GHIP_ERR_INVALID_ARG, "sdpa_fwd: mask without strides");
  if (B == 0 || Sq == 0) return GHIP_OK;
  if (!q || !k || !v || !o) return set_error(err, GHIP_ERR_INVALID_ARG, "sdpa_fwd: null pointer");
  const int mdt = mask ? mask_dtype : -1;
  if (!sdpa_fused_supported(dtype, H, Hkv, Sq, Sk, D, q_strides, k_strides, v_strides, o_strides, scale, mdt))
    return set_error(err, GHIP_ERR_UNSUPPORTED,
                     "sdpa_fwd: needs bfloat16 or float16 with a head dim that is a multiple of 8 up to 256, "
                     "or float32 with a multiple of 4 up to 128; a bool mask or one in the operands' dtype, a "
                     "positive finite scale, non-negative strides that are multiples of 16 bytes (8 bytes for "
                     "a 16-bit output), K / V sequence strides below 32 MiB and, for float32, < 2 GiB per "
                     "K/V head");
  const bool f32 = dtype == GHIP_DTYPE_FLOAT32;
  const int64_t es = f32 ? 4 : 2;
  auto al = [](const void* ptr, uintptr_t a) { return (reinterpret_cast<uintptr_t>(ptr) & (a - 1)) == 0; };
  if (!al(q, 16) || !al(k, 16) || !al(v, 16) || !al(o, 4 * es))
    return set_error(err, GHIP_ERR_UNSUPPORTED, "sdpa_fwd: q/k/v must be 16-byte aligned, o %d-byte aligned",
                     static_cast<int>(4 * es));
  const int64_t nqb = (Sq + attn::kBQ - 1) / attn::kBQ;
  const attn::SdpaGrid sg = attn::sdpa_grid(dtype, B, H, Hkv, Sq, Sk, causal);
  if (nqb * B * H > 0x7fffffffLL || sg.wgs > 0x7fffffffLL)
    return set_error(err, GHIP_ERR_INVALID_ARG, "sdpa_fwd: problem too large");
  attn::Params p{};
  p.q = q; p.k = k; p.v = v; p.o = o;
  p.q_sb = q_strides[0]; p.q_sh = q_strides[1]; p.q_ss = q_strides[2];
  p.k_sb = k_strides[0]; p.k_sh = k_strides[1]; p.k_ss = k_strides[2];
  p.v_sb = v_strides[0]; p.v_sh = v_strides[1]; p.v_ss = v_strides[2];
  p.o_sb = o_strides[0]; p.o_sh = o_strides[1]; p.o_ss = o_strides[2];
  p.B = static_cast<int>(B); p.H = static_cast<int>(H); p.Hkv = static_cast<int>(Hkv);
  p.Sq = static_cast<int>(Sq); p.Sk = static_cast<int>(Sk);
  p.scale_log2 = scale * 1.4426950408889634f;
  p.inv_scale = 1.0f / scale;
  p.causal = causal ? 1 : 0;
  p.D = static_cast<int>(D);
  p.k_extent64 = ((Sk - 1) * p.k_ss + D) * es;
  p.v_extent64 = ((Sk - 1) * p.v_ss + D) * es;
  const bool big = p.k_extent64 >= (int64_t{1} << 31) || p.v_extent64 >= (int64_t{1} << 31);
  p.k_extent = big ? 0u : static_cast<uint32_t>(p.k_extent64);
  p.v_extent = big ? 0u : static_cast<uint32_t>(p.v_extent64);
  int mk = attn::kNoMask;
  if (mask) {
    mk = mask_dtype == GHIP_DTYPE_BOOL ? attn::kBoolMask : attn::kAddMask;
    p.mask = mask;
    p.m_sb = mask_strides[0]; p.m_sh = mask_strides[1]; p.m_sq = mask_strides[2]; p.m_sk = mask_strides[3];
    // Vector loads of 4-key groups (keys are multiples of 4 apart): unit key stride
    // and every row start aligned to 4 elements.
    const int64_t mes = mask_dtype == GHIP_DTYPE_BOOL ? 1 : es;
    p.mask_vec = p.m_sk == 1 && p.m_sb % 4 == 0 && p.m_sh % 4 == 0 && p.m_sq % 4 == 0 && al(mask, 4 * mes);
  }
  // A split key range when a workspace is given and the grid is small.
  p.gqa_pack = sg.pack ? 1 : 0;
  const attn::KvSplit kvs = workspace ? attn::kv_split(dtype, sg) : attn::KvSplit{1, 0};
  const int64_t rows = B * H * Sq;
  if (kvs.ns > 1) {
    const int64_t need = attn::kv_split_bytes(kvs, B, H, Sq, D);
    if (workspace_bytes < need)
      return set_error(err, GHIP_ERR_INVALID_ARG, "sdpa_fwd: workspace of %lld bytes, %lld needed",
                       static_cast<long long>(workspace_bytes), static_cast<long long>(need));
    if (!al(workspace, 16)) return set_error(err, GHIP_ERR_INVALID_ARG, "sdpa_fwd: workspace must be 16-byte aligned");
    p.kv_chunk = kvs.chunk;
    p.part_o = static_cast<float*>(workspace);
    p.part_lse = p.part_o + static_cast<int64_t>(kvs.ns) * rows * D;
  }
  const dim3 grid(static_cast<unsigned>(sg.wgs), static_cast<unsigned>(kvs.ns));
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const bool f16 = dtype == GHIP_DTYPE_FLOAT16;
  // Key tiles of the longest workgroup: the split K / V schedule (no mask) unless
  // causal workgroups are all short (<= 16 tiles: B8 H16 S1024 measured 6% faster
  // with the plain schedule, S2048 4% and S4096 / S8192 6-7% slower).
  const int64_t kv_max = causal ? std::min<int64_t>(Sk, nqb * attn::kBQ) : Sk;
  const bool split = !causal || (kv_max + attn::kBKV - 1) / attn::kBKV > 16;
  // The smallest padded width that holds D.
  if (f32) {
    if (D <= 64) attn::launch_f32<64>(p, mk, grid, s);
    else attn::launch_f32<128>(p, mk, grid, s);
  } else if (D <= 64) {
    if (f16) attn::launch_d<64, true>(p, mk, grid, split, big, s);
    else attn::launch_d<64, false>(p, mk, grid, split, big, s);
  } else if (D <= 128) {
    if (f16) attn::launch_d<128, true>(p, mk, grid, split, big, s);
    else attn::launch_d<128, false>(p, mk, grid, split, big, s);
  } else {
    if (f16) attn::launch_d<256, true>(p, mk, grid, split, big, s);
    else attn::launch_d<256, false>(p, mk, grid, split, big, s);
  }
  GHIP_CHECK(hipGetLastError(), err);
  if (kvs.ns > 1) {
    const dim3 cgrid(static_cast<unsigned>((rows + 3) / 4));
    if (f16) hipLaunchKernelGGL((attn::sdpa_combine_kernel<true>), cgrid, dim3(256), 0, s, p, kvs.ns);
    else hipLaunchKernelGGL((attn::sdpa_combine_kernel<false>), cgrid, dim3(256), 0, s, p, kvs.ns);
    GHIP_CHECK(hipGetLastError(), err);
  }
  return GHIP_OK;
}

extern "C" int ghip_sdpa_fwd_masked(int dtype, const void* q, const void* k, const void* v, void* o,
                                    int64_t B, int64_t H, int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D,
                                    const int64_t* q_strides, const int64_t* k_strides,
                                    const int64_t* v_strides, const int64_t* o_strides, const void* mask,
                                    int mask_dtype, const int64_t* mask_strides, float scale, int causal,
                                    void* stream, GHipError* err) {
  return ghip_sdpa_fwd_masked_ws(dtype, q, k, v, o, B, H, Hkv, Sq, Sk, D, q_strides, k_strides, v_strides, o_strides,
                                 mask, mask_dtype, mask_strides, scale, causal, nullptr, 0, stream, err);
}

extern "C" int ghip_sdpa_fwd(int dtype, const void* q, const void* k, const void* v, void* o,
                             int64_t B, int64_t H, int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D,
                             const int64_t* q_strides, const int64_t* k_strides,
                             const int64_t* v_strides, const int64_t* o_strides, float scale,
                             int causal, void* stream, GHipError* err) {
  return ghip_sdpa_fwd_masked(dtype, q, k, v, o, B, H, Hkv, Sq, Sk, D, q_strides, k_strides, v_strides, o_strides,
                              nullptr, -1, nullptr, scale, causal, stream, err);
}
