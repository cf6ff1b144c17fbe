// Device helpers shared by the gfx950 kernel files (s14_device.hip,
// s14_prefill.hip): buffer-resource loads, the decoders, SwiGLU, wavefront
// DPP reductions and the top-k selection of one token's router scores.
// Everything sits in an unnamed namespace: each kernel file gets its own
// inline copy.
#pragma once

#include <hip/hip_runtime.h>

#include <climits>

#include "s14_device.hpp"
#include "s14_e4m3.h"
#include "s14_expf.h"

namespace s14 {
namespace {

typedef float v2f __attribute__((ext_vector_type(2)));
typedef unsigned v2u __attribute__((ext_vector_type(2)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));
typedef __amdgpu_buffer_rsrc_t Rsrc;

// ---------------------------------------------------------------------------
// buffer-resource loads: page addresses come from memory (generic pointers),
// which would otherwise become flat loads that also occupy the LDS counter;
// raw buffer loads keep weight traffic on the vector-memory counter only and
// return 0 past num_records instead of faulting.
// ---------------------------------------------------------------------------

constexpr uint32_t kRsrcWord3 = 0x00020000u;  // gfx9 raw buffer descriptor flags

__device__ __forceinline__ Rsrc make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, int(bytes), int(kRsrcWord3));
}
__device__ __forceinline__ uint4 ld16(Rsrc r, uint32_t off) {
  const v4u v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 ld8(Rsrc r, uint32_t off) {
  const v2u v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
  return make_uint2(v.x, v.y);
}
__device__ __forceinline__ uint32_t ld4(Rsrc r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
__device__ __forceinline__ uint32_t ld1(Rsrc r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b8(r, off, 0, 0);
}
__device__ __forceinline__ float ldf(Rsrc r, uint32_t off) { return __uint_as_float(ld4(r, off)); }

// Where a row's bytes come from: one matrix (codes and scales may be
// separate buffers), or two pages split by lane half (lanes 32-63 read page
// b), each page holding its codes and scales.
struct Src1 {
  Rsrc w, s;
};
struct Src2 {
  Rsrc a, b;
  bool hi;
};
// A per-lane source: wavefronts that serve two pages (lanes 0-31 one, 32-63
// the other) load through a per-lane global pointer.  A buffer descriptor
// that differs between lanes has to be made uniform first, and the compiler
// does that with a loop over the distinct descriptors around every load.
// No bounds clamp: callers keep every load inside its row.
typedef const __attribute__((address_space(1))) uint8_t *GPtr;
struct SrcP {
  GPtr p;
};
__device__ __forceinline__ uint2 gld8(GPtr p) {
  const uint64_t v = *(const __attribute__((address_space(1))) uint64_t *)p;
  return make_uint2(uint32_t(v), uint32_t(v >> 32));
}
__device__ __forceinline__ uint32_t gld4(GPtr p) { return *(const __attribute__((address_space(1))) uint32_t *)p; }

// ---------------------------------------------------------------------------
// decoders (bit patterns; equal to s14_vulkan_numeric.rs:1716-1743)
// ---------------------------------------------------------------------------

// 2^(c-127) as f32; c = 0 is the subnormal 2^-127, c = 255 is +inf.
__device__ __forceinline__ float ue8m0_f32(uint32_t c) {
  return c == 0u ? __uint_as_float(0x00400000u) : __uint_as_float(c << 23);
}

// E2M1 nibble: magnitudes {0, .5, 1, 1.5, 2, 3, 4, 6}; for m >= 2 the f32
// bit pattern is (m + 252) << 22, m == 1 is 0.5; bit 3 is the sign.
__device__ __forceinline__ float e2m1_f32(uint32_t nib) {
  const uint32_t m = nib & 7u;
  const uint32_t bits = m == 0u ? 0u : (m == 1u ? 0x3F000000u : ((m + 252u) << 22));
  return __uint_as_float(bits | ((nib & 8u) << 28));
}

// OCP E4M3FN: exponent 0 is m * 2^-9, otherwise (1 + m/8) * 2^(e-7).  The
// NaN codes decode as 480 like the reference CPU decoder; they are rejected
// on the host before upload (s14_vulkan.rs:151-156).
__device__ __forceinline__ float e4m3_f32(uint32_t code) {
  const uint32_t e = (code >> 3) & 15u, m = code & 7u;
  const float mag = e == 0u ? float(m) * 0x1p-9f : __uint_as_float(((e + 120u) << 23) | (m << 20));
  return (code & 0x80u) ? -mag : mag;
}

__device__ __forceinline__ float bf16_f32(uint32_t b) { return __uint_as_float(b << 16); }

// v rounded to bf16 (ties to even; a NaN stays a quiet NaN), as an f32: the
// rounding of torch's .to(bfloat16) that the official expert semantics apply
// to every linear output (executor.py:717-727).
__device__ __forceinline__ float bf16_round(float v) {
  uint32_t u = __float_as_uint(v);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return __uint_as_float((u | 0x00400000u) & 0xffff0000u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return __uint_as_float(u & 0xffff0000u);
}

// E8M0 code of an activation-requant group: 127 + ceil(log2(max(amax, 1e-4)
// / 448)) (l42_reference.py:390-403), the f32 quotient rounded to nearest,
// ceil(log2) taken exactly from its bits.
__device__ __forceinline__ uint32_t requant_code(float amax) {
  if (amax < 1.0e-4f) amax = 1.0e-4f;
  const float r = __fdiv_rn(amax, 448.0f);
  const uint32_t u = __float_as_uint(r);
  const int e = int((u >> 23) & 255u) - 127;  // r is normal: amax/448 >= 2.2e-7
  const int c = (u & 0x7fffffu) ? e + 1 : e;  // ceil(log2 r)
  return uint32_t(c + 127);
}

// The prefill's activation requant (bit-identical to the oracle's
// s14o_requant_e4m3): X [T, 4096] f32 -> Q [T, 4096] e4m3 + S [T, 128]
// E8M0, one thread (gid) per 32-value group.  kOfficial: the official
// act_quant's group of 128 (l42_reference.py:390-403): the maximum over the
// four adjacent threads of a 128-value group, whose four E8M0 bytes then
// hold the same code (a token's 128 groups and a workgroup's 256 threads are
// whole quads, so a quad returns early together or not at all).
template <bool kOfficial>
__device__ __forceinline__ void requant_x_group(uint32_t gid, uint32_t tokens, const float *__restrict__ X,
                                                uint8_t *__restrict__ Q, uint8_t *__restrict__ S) {
  constexpr uint32_t kGroup = 32, groups = kHidden / kGroup;
  if (gid >= tokens * groups) return;
  const uint32_t t = gid / groups, g = gid % groups;
  const float4 *src = reinterpret_cast<const float4 *>(X + size_t(t) * kHidden + g * kGroup);
  float v[32];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float4 q = src[i];
    v[4 * i] = q.x;
    v[4 * i + 1] = q.y;
    v[4 * i + 2] = q.z;
    v[4 * i + 3] = q.w;
  }
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 32; ++i) amax = fabsf(v[i]) > amax ? fabsf(v[i]) : amax;
  if constexpr (kOfficial) {
    // NaN never compares greater, as in the scan above
    const float a1 = __shfl_xor(amax, 1);
    amax = a1 > amax ? a1 : amax;
    const float a2 = __shfl_xor(amax, 2);
    amax = a2 > amax ? a2 : amax;
  }
  const uint32_t code = requant_code(amax);
  const float inv = __uint_as_float((254u - code) << 23);  // 2^-(code-127)
  uint32_t w[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    uint32_t word = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) word |= s14x::e4m3_rne_sat(__fmul_rn(v[4 * i + j], inv)) << (8 * j);
    w[i] = word;
  }
  uint8_t *dst = Q + size_t(t) * kHidden + kGroup * g;
  *reinterpret_cast<uint4 *>(dst) = make_uint4(w[0], w[1], w[2], w[3]);
  *reinterpret_cast<uint4 *>(dst + 16u) = make_uint4(w[4], w[5], w[6], w[7]);
  S[size_t(t) * groups + g] = uint8_t(code);
}

// expf's 32 table entries in LDS (see s14x::expf_glibc_with): filled by the
// first 32 lanes of a wavefront, then a barrier before any use.
struct LdsExpTable {
  const double *t;
  __device__ double operator()(uint32_t i) const { return t[i]; }
};
__device__ __forceinline__ void exp_table_fill(double *lds) {
  const uint32_t lane = threadIdx.x & 63;
  if (threadIdx.x < 32) lds[lane] = s14x::exp_table_entry(lane);
}

template <class Tab>
__device__ __forceinline__ float swiglu_exact_with(float gate, float up, const Tab &tab) {
  // s14_vulkan_numeric.rs:1543-1556: gate.min(10) keeps -0 and maps NaN to
  // 10; clamp passes NaN through.
  const float g = (gate <= 10.0f) ? gate : 10.0f;
  float u = up;
  if (u < -10.0f) u = -10.0f;
  if (u > 10.0f) u = 10.0f;
  const float e = s14x::expf_glibc_with(-g, tab);
  return __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, e)), u);
}
__device__ __forceinline__ float swiglu_exact(float gate, float up) {
  return swiglu_exact_with(gate, up, s14x::ConstExpTable{});
}
__device__ __forceinline__ float swiglu_exact(float gate, float up, const double *lds_table) {
  return swiglu_exact_with(gate, up, LdsExpTable{lds_table});
}

// ---------------------------------------------------------------------------
// wavefront reductions and lane movement
// ---------------------------------------------------------------------------

// DPP row operations.  dpp_f/dpp_i read the source lane given by CTRL; lanes
// without a source (or in rows outside ROW_MASK) get `old`.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_f(float old, float v) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), CTRL, ROW_MASK, 0xf, false));
}
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ int dpp_i(int old, int v) {
  return __builtin_amdgcn_update_dpp(old, v, CTRL, ROW_MASK, 0xf, false);
}

// Wavefront minimum / maximum of an int, returned to every lane: DPP row
// steps (lanes without a DPP source contribute the identity), then lane 63.
// No LDS permutes, so the dependent steps cost VALU latency only.
__device__ __forceinline__ int wave_min_i(int v) {
  v = min(v, dpp_i<0xb1>(INT_MAX, v));        // quad_perm [1,0,3,2]
  v = min(v, dpp_i<0x4e>(INT_MAX, v));        // quad_perm [2,3,0,1]
  v = min(v, dpp_i<0x114>(INT_MAX, v));       // row_shr:4
  v = min(v, dpp_i<0x118>(INT_MAX, v));       // row_shr:8
  v = min(v, dpp_i<0x142, 0xa>(INT_MAX, v));  // row_bcast:15
  v = min(v, dpp_i<0x143, 0xc>(INT_MAX, v));  // row_bcast:31
  return __builtin_amdgcn_readlane(v, 63);
}
__device__ __forceinline__ int wave_max_i(int v) {
  v = max(v, dpp_i<0xb1>(INT_MIN, v));
  v = max(v, dpp_i<0x4e>(INT_MIN, v));
  v = max(v, dpp_i<0x114>(INT_MIN, v));
  v = max(v, dpp_i<0x118>(INT_MIN, v));
  v = max(v, dpp_i<0x142, 0xa>(INT_MIN, v));
  v = max(v, dpp_i<0x143, 0xc>(INT_MIN, v));
  return __builtin_amdgcn_readlane(v, 63);
}

// The value of lane ^ 32 (gfx950's permlane32 swap, a VALU op: the swap
// returns {first operand with lanes 32-63 replaced by the second's lanes
// 0-31, second operand with lanes 0-31 replaced by the first's lanes 32-63}).
__device__ __forceinline__ float lane_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float((threadIdx.x & 32u) ? r[0] : r[1]);
}

// Value of the odd lane of each lane pair (quad_perm [1,1,3,3]); every lane
// has a source, so the move folds into the consuming VALU op as a DPP operand.
__device__ __forceinline__ float from_odd(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xF5, 0xf, 0xf, true));
}
// Value of the even lane of each lane pair (quad_perm [0,0,2,2]).
__device__ __forceinline__ float from_even(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xA0, 0xf, 0xf, true));
}

// The xor butterfly sum of a wavefront's 64 values: for m = 32, 16, 8, 4, 2,
// 1 every lane adds the value of lane ^ m (a + a[lane ^ m], so lanes l and
// l ^ m hold the same sum after each step and every lane ends with the
// total).  The exchanges stay in the VALU: gfx950's permlane swaps for 32
// and 16 (the swap returns {first operand with its upper rows replaced,
// second operand with its lower rows replaced}; each lane takes the half that
// holds its partner), DPP row_ror:8 for 8, two bank-masked row shifts for 4,
// quad_perm for 2 and 1.  `__shfl_xor` would issue an LDS permute per step.
__device__ __forceinline__ float xor_butterfly_sum(float a) {
  const uint32_t lane = threadIdx.x & 63;
  a = __fadd_rn(a, lane_xor32(a));
  {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(a), false, false);
    a = __fadd_rn(a, __uint_as_float((lane & 16u) ? r[0] : r[1]));
  }
  a = __fadd_rn(a, dpp_f<0x128>(0.0f, a));  // row_ror:8: lane ^ 8 within each 16-lane row
  {
    // row_shl:4 into banks 0 and 2 (lanes 0-3, 8-11 of a row), row_shr:4
    // into banks 1 and 3
    int t = __builtin_amdgcn_update_dpp(0, __float_as_int(a), 0x104, 0xf, 0x5, false);
    t = __builtin_amdgcn_update_dpp(t, __float_as_int(a), 0x114, 0xf, 0xa, false);
    a = __fadd_rn(a, __int_as_float(t));
  }
  a = __fadd_rn(a, dpp_f<0x4e>(0.0f, a));  // quad_perm [2,3,0,1]: lane ^ 2
  a = __fadd_rn(a, dpp_f<0xb1>(0.0f, a));  // quad_perm [1,0,3,2]: lane ^ 1
  return a;
}

// Full-wavefront sum (order-changing; FAST mode only), returned to every lane.
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += dpp_f<0xb1>(0.0f, v);        // quad_perm [1,0,3,2]
  v += dpp_f<0x4e>(0.0f, v);        // quad_perm [2,3,0,1]
  v += dpp_f<0x114>(0.0f, v);       // row_shr:4
  v += dpp_f<0x118>(0.0f, v);       // row_shr:8
  v += dpp_f<0x142, 0xa>(0.0f, v);  // row_bcast:15
  v += dpp_f<0x143, 0xc>(0.0f, v);  // row_bcast:31
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Wavefront max of a u32 (DPP row steps, then lane 63), returned to every
// lane.  Lanes without a DPP source contribute the identity.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, uint32_t(dpp_i<0xb1>(0, int(v))));
  v = max(v, uint32_t(dpp_i<0x4e>(0, int(v))));
  v = max(v, uint32_t(dpp_i<0x114>(0, int(v))));
  v = max(v, uint32_t(dpp_i<0x118>(0, int(v))));
  v = max(v, uint32_t(dpp_i<0x142, 0xa>(0, int(v))));
  v = max(v, uint32_t(dpp_i<0x143, 0xc>(0, int(v))));
  return uint32_t(__builtin_amdgcn_readlane(int(v), 63));
}

// Order-preserving key of a score for the top-k selection: larger float ->
// larger key; -0 and +0 share a key (they compare equal); NaN gets key 0,
// below every number (a NaN score is never preferred).
__device__ __forceinline__ uint32_t score_key(float f) {
  if (f != f) return 0u;
  const uint32_t u = __float_as_uint(f + 0.0f);  // -0 + 0 = +0
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Top-k of one token's scores, computed by one whole wavefront
// (executor.py:647-667 semantics, orders fixed here): largest score + bias
// first, equal values to the lower expert index (as the oracle's strict '>'
// scan), sum of the chosen unbiased scores sequential in selection order.
// Lane i < k receives the i-th choice: expert id, unbiased score and the
// expert's page address (0 when `pages` is NULL).  All loads are issued
// before the first selection, so no memory access waits on one.
struct TopK {
  uint32_t id;
  float s;
  uint64_t page;
  float sum;
};
// Plain loads of scores, biased scores and pages (written before the kernel).
struct PlainScoreLoad {
  const float *biased, *scores;
  const uint64_t *pages;
  __device__ float b(uint32_t e) const { return biased[e]; }
  __device__ float s(uint32_t e) const { return scores[e]; }
  __device__ uint64_t p(uint32_t e) const { return pages ? pages[e] : 0ull; }
};

template <class Load>
__device__ __forceinline__ TopK select_topk_from(const Load &ld, uint32_t n_experts, uint32_t k);

__device__ __forceinline__ TopK select_topk(const float *__restrict__ biased, const float *__restrict__ scores,
                                            const uint64_t *__restrict__ pages, uint32_t n_experts, uint32_t k) {
  return select_topk_from(PlainScoreLoad{biased, scores, pages}, n_experts, k);
}

// The selection with the scores and pages read through `ld` (b(e), s(e),
// p(e)): e.g. device-scope loads of scores other workgroups of the same
// launch wrote.
template <class Load>
__device__ __forceinline__ TopK select_topk_from(const Load &ld, uint32_t n_experts, uint32_t k) {
  const uint32_t lane = threadIdx.x & 63;
  // lane l holds experts 4l .. 4l+3, so a lower lane holds only lower
  // indices: the lowest lane with the maximum key, then its lowest slot, is
  // the lowest expert index among the ties.  Key 0 marks an absent or
  // already chosen expert; a real score's key is >= 1 unless it is NaN.
  uint32_t kv[4];
  float sv[4];
  uint64_t pv[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t ee = 4u * lane + uint32_t(j);
    const bool absent = ee >= n_experts;
    kv[j] = absent ? 0u : max(score_key(ld.b(ee)), 1u);
    sv[j] = absent ? 0.0f : ld.s(ee);
    pv[j] = absent ? 0ull : ld.p(ee);
  }
  TopK mine{0u, 0.0f, 0ull, 0.0f};
  float sum = 0.0f;
#pragma unroll
  for (uint32_t i = 0; i < uint32_t(kTopK); ++i) {
    if (i >= k) break;
    const uint32_t top = wave_max_u32(max(max(kv[0], kv[1]), max(kv[2], kv[3])));
    const uint32_t jl = kv[0] == top ? 0u : kv[1] == top ? 1u : kv[2] == top ? 2u : 3u;  // this lane's first hit
    const uint64_t hit = __ballot(kv[0] == top || kv[1] == top || kv[2] == top || kv[3] == top);
    const int wl = __builtin_ctzll(hit | (1ull << 63));  // lowest lane holding the maximum
    const uint32_t wj = uint32_t(__builtin_amdgcn_readlane(int(jl), wl));
    float cand = sv[0];
    uint64_t cpg = pv[0];
#pragma unroll
    for (int j = 1; j < 4; ++j) {
      cand = wj == uint32_t(j) ? sv[j] : cand;
      cpg = wj == uint32_t(j) ? pv[j] : cpg;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (int(lane) == wl && wj == uint32_t(j)) kv[j] = 0u;
    const float s = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cand), wl));
    const uint64_t pg = (uint64_t(uint32_t(__builtin_amdgcn_readlane(int(cpg >> 32), wl))) << 32) |
                        uint32_t(__builtin_amdgcn_readlane(int(uint32_t(cpg)), wl));
    sum = __fadd_rn(sum, s);
    if (lane == i) {
      mine.id = 4u * uint32_t(wl) + wj;
      mine.s = s;
      mine.page = pg;
    }
  }
  mine.sum = sum;
  return mine;
}

// The same selection when scores and pages are in LDS: the rounds carry the
// keys alone (the chosen lane and slot are uniform), lane i < k reads its
// choice's score and page by id afterwards, and the sum is formed in
// selection order from those.  About a third fewer instructions per round.
__device__ __forceinline__ TopK select_topk_lds(const float *biased, const float *scores, const uint64_t *pages,
                                                uint32_t n_experts, uint32_t k) {
  const uint32_t lane = threadIdx.x & 63;
  uint32_t kv[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t ee = 4u * lane + uint32_t(j);
    kv[j] = ee >= n_experts ? 0u : max(score_key(biased[ee]), 1u);
  }
  uint32_t my_id = 0;
#pragma unroll
  for (uint32_t i = 0; i < uint32_t(kTopK); ++i) {
    if (i >= k) break;
    const uint32_t lmax = max(max(kv[0], kv[1]), max(kv[2], kv[3]));
    const uint32_t top = wave_max_u32(lmax);
    const uint32_t jl = kv[0] == top ? 0u : kv[1] == top ? 1u : kv[2] == top ? 2u : 3u;  // this lane's first hit
    const int wl = __builtin_ctzll(__ballot(lmax == top) | (1ull << 63));  // lowest lane holding the maximum
    const uint32_t wj = uint32_t(__builtin_amdgcn_readlane(int(jl), wl));
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (int(lane) == wl && wj == uint32_t(j)) kv[j] = 0u;
    if (lane == i) my_id = 4u * uint32_t(wl) + wj;
  }
  const bool chosen = lane < k;
  TopK mine{my_id, chosen ? scores[my_id] : 0.0f, (chosen && pages) ? pages[my_id] : 0ull, 0.0f};
  float sum = 0.0f;
#pragma unroll
  for (uint32_t i = 0; i < uint32_t(kTopK); ++i) {
    if (i >= k) break;
    sum = __fadd_rn(sum, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine.s), int(i))));
  }
  mine.sum = sum;
  if (!chosen) mine.id = 0u;
  return mine;
}

// Route weight of a choice: s / sum, then * route_scale unless it is 1.
__device__ __forceinline__ float route_weight(const TopK &c, float route_scale) {
  float w = __fdiv_rn(c.s, c.sum);
  if (route_scale != 1.0f) w = __fmul_rn(w, route_scale);
  return w;
}

// Scores and pages held in LDS.
struct LdsScoreLoad {
  const float *scores;
  const uint64_t *pages;
  __device__ float s(uint32_t e) const { return scores[e]; }
  __device__ uint64_t p(uint32_t e) const { return pages ? pages[e] : 0ull; }
};

// Hash route of token t (the reference's layers 0-2, executor.py:643-667),
// computed by one whole wavefront: lane j < k takes expert
// tid2eid[token_ids[t]][j] (row order is route order), its unbiased score
// and page through `ld`; the sum of the k scores is sequential in row order,
// as for the top-k.  `bad` (uniform): the token id is outside [0, vocab), or
// an entry is outside [0, n_experts) or repeats an earlier one (the
// executor's ContractError cases); such lanes then hold expert 0.
template <class Load>
__device__ __forceinline__ TopK select_hash_from(const Load &ld, const RouterArgs &r, uint32_t t, bool &bad) {
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t k = r.topk;
  const int32_t tok = r.token_ids[t];
  const bool tok_ok = tok >= 0 && uint32_t(tok) < r.vocab;
  int64_t e = -1;
  if (lane < k && tok_ok) e = r.tid2eid[size_t(tok) * k + lane];
  const bool in_range = e >= 0 && e < int64_t(r.n_experts);
  const uint32_t id = in_range ? uint32_t(e) : 0u;
  bool dup = false;
#pragma unroll
  for (uint32_t j = 0; j < uint32_t(kTopK); ++j) {
    const uint32_t other = uint32_t(__builtin_amdgcn_readlane(int(id), int(j)));
    dup = dup || (j < lane && j < k && other == id);
  }
  bad = __ballot(lane < k && (!tok_ok || !in_range || dup)) != 0ull;
  TopK mine{id, 0.0f, 0ull, 0.0f};
  if (lane < k) {
    mine.s = ld.s(id);
    mine.page = ld.p(id);
  }
  float sum = 0.0f;
#pragma unroll
  for (uint32_t i = 0; i < uint32_t(kTopK); ++i) {
    if (i >= k) break;
    sum = __fadd_rn(sum, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine.s), int(i))));
  }
  mine.sum = sum;
  return mine;
}

// The weight checks of RouteDecision::validate_for (runner.rs:128-180) on a
// device route, lane j < k holding weight j: every weight finite and >= 0,
// and their f32 sum, sequential in route order from 0, within 1e-4 of
// route_scale (the reference's 1.5).  Uniform result.
__device__ __forceinline__ bool route_weights_valid(float w, uint32_t k, float route_scale) {
  const uint32_t lane = threadIdx.x & 63;
  const bool lane_ok = lane >= k || (__builtin_isfinite(w) && w >= 0.0f);
  float sum = 0.0f;
#pragma unroll
  for (uint32_t i = 0; i < uint32_t(kTopK); ++i) {
    if (i >= k) break;
    sum = __fadd_rn(sum, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), int(i))));
  }
  return __ballot(!lane_ok) == 0ull && fabsf(__fsub_rn(sum, route_scale)) <= 1e-4f;
}

// Lane K % 16 of each 16-lane row of `v`, in every lane of that row (DPP
// row_newbcast, folded into the consuming instruction as its operand).
template <int K>
__device__ __forceinline__ float bcast16(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x150 + (K & 15), 0xf, 0xf, false));
}

}  // namespace
}  // namespace s14
