// Activation-quantised FP8 linear on gfx950: the adjacent FP8 projections of
// the S14 layer (wq_b [32768, 1024], wkv [512, 4096], wo_a [8192, 4096],
// wo_b [4096, 8192]; l42_reference.py:89-102) in fp8_linear's semantics
// (local_s14_primitives/fp8.py:111-193):
//
//   x  e4m3 codes [m][k], one scale per (token, 128 k)       (activation)
//   w  e4m3 codes [n][k], one scale per (128 rows, 128 k)    (weight)
//   y[t][r] = sum over groups g ascending of
//               partial_g = sum_k (dec(x) * sa[t][g]) * (dec(w) * sb[r/128][g])
//             then + bias[r]; f32 throughout (acc = 0; acc += partial_g).
//
// Scales are UE8M0 codes or f32 values (fp8.py:37-46).  The reference sums
// each group's products with torch addmm, whose order is the BLAS's; EXACT
// fixes it to k ascending, multiply then add, so its results are bit-equal
// to the CPU oracle's s14o_fp8_linear.  FAST computes each group's dot
// products on the bf16 MFMA (v_mfma_f32_32x32x16_bf16) from operands decoded
// exactly (every e4m3 value is a bf16 value), so products are exact and sums
// f32, and folds the group scales in afterwards: not order-exact.  The fp8
// MFMA (v_mfma_scale_f32_32x32x64_f8f6f4) is not used here: measured on
// MI355X, its internal sum keeps about 16 bits below the largest product of
// a step (256 * 256 + 1 * 1 comes back as 65536), which put FAST 5e-5 of a
// row's sum of |products| away from the oracle on uniformly drawn codes.
//
// The activation requant that produces x (l42_reference.py:390-403: e4m3
// RNE saturating, scale 2^ceil(log2(max(amax, 1e-4) / 448)) per group) is
// k_act_quant; group 128 feeds this linear, group 32 the prefill.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>
#include <utility>

#include "s14_device.hpp"
#include "s14_device_util.hpp"
#include "s14_e4m3.h"
#include "s14_linear.hpp"

namespace s14 {
namespace {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

// Eight e4m3 codes (two little-endian words) as eight bf16, exactly.
__device__ __forceinline__ v8bf e4m3x8_bf16(uint32_t w0, uint32_t w1) {
  const v4u v = {__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, false)),
                 __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, true)),
                 __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, false)),
                 __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, true))};
  return __builtin_bit_cast(v8bf, v);
}

// ---------------------------------------------------------------------------
// activation requant: one thread per group of `group` values along k
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void k_act_quant(uint32_t n_groups, uint32_t group, const float *__restrict__ X,
                                                   uint8_t *__restrict__ Q, uint8_t *__restrict__ S) {
  const uint32_t gid = blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= n_groups) return;
  const float *src = X + size_t(gid) * group;
  float amax = 0.0f;  // strict '>' scan: a NaN never becomes the maximum
  for (uint32_t i = 0; i < group; ++i) amax = fabsf(src[i]) > amax ? fabsf(src[i]) : amax;
  const uint32_t code = requant_code(amax);
  const float inv = __uint_as_float((254u - code) << 23);
  uint8_t *dst = Q + size_t(gid) * group;
  for (uint32_t i = 0; i < group; ++i) dst[i] = uint8_t(s14x::e4m3_rne_sat(__fmul_rn(src[i], inv)));
  S[gid] = uint8_t(code);
}

__device__ __forceinline__ float lin_scale(Rsrc r, uint32_t i, int is_f32) {
  return is_f32 ? ldf(r, 4u * i) : ue8m0_f32(ld1(r, i));
}

__device__ __forceinline__ uint32_t byte_of(uint4 v, int b) {
  const uint32_t w = b < 4 ? v.x : b < 8 ? v.y : b < 12 ? v.z : v.w;
  return (w >> (8 * (b & 3))) & 0xffu;
}

// ---------------------------------------------------------------------------
// EXACT: one lane per (row, group) computes partial_g for MT tokens, k
// ascending; the row's partials meet in LDS and one lane per (token, row)
// adds them in group order.  A workgroup holds R = max(1, 256 / G) rows.
// kVec: k % 16 == 0 and 16-byte aligned operands (16-byte loads).
// ---------------------------------------------------------------------------

template <int MT, bool kVec>
__global__ __launch_bounds__(256) void k_linear_exact(LinearArgs a) {
  extern __shared__ float lpart[];  // [MT][R][G]
  const uint32_t G = a.groups, K = a.k, N = a.n, M = a.m;
  const uint32_t R = G >= 256u ? 1u : 256u / G;
  const uint32_t row0 = blockIdx.x * R, m0 = blockIdx.y * uint32_t(MT);
  const Rsrc rw = make_rsrc(a.w, N * K);
  const Rsrc rx = make_rsrc(a.x, M * K);
  const uint32_t n_sw = (N + 127u) / 128u * G, n_sx = M * G;
  const Rsrc rsw = make_rsrc(a.w_scale, a.w_scale_f32 ? 4u * n_sw : n_sw);
  const Rsrc rsx = make_rsrc(a.x_scale, a.x_scale_f32 ? 4u * n_sx : n_sx);
  for (uint32_t task = threadIdx.x; task < R * G; task += 256u) {
    const uint32_t r = task / G, g = task % G, row = row0 + r;
    float p[MT];
#pragma unroll
    for (int j = 0; j < MT; ++j) p[j] = 0.0f;
    if (row < N) {
      const float sb = lin_scale(rsw, (row / 128u) * G + g, a.w_scale_f32);
      float sa[MT];
#pragma unroll
      for (int j = 0; j < MT; ++j) sa[j] = m0 + j < M ? lin_scale(rsx, (m0 + j) * G + g, a.x_scale_f32) : 0.0f;
      const uint32_t k0 = g * kLinGroup, len = min(kLinGroup, K - k0);
      const uint32_t wo = row * K + k0;
      if constexpr (kVec) {
        for (uint32_t c = 0; c < len; c += 16u) {
          const uint4 w16 = ld16(rw, wo + c);
          uint4 x16[MT];
#pragma unroll
          for (int j = 0; j < MT; ++j) x16[j] = m0 + j < M ? ld16(rx, (m0 + j) * K + k0 + c) : make_uint4(0, 0, 0, 0);
#pragma unroll
          for (int b = 0; b < 16; ++b) {
            const float wv = __fmul_rn(e4m3_f32(byte_of(w16, b)), sb);
#pragma unroll
            for (int j = 0; j < MT; ++j)
              p[j] = __fadd_rn(p[j], __fmul_rn(__fmul_rn(e4m3_f32(byte_of(x16[j], b)), sa[j]), wv));
          }
        }
      } else {
        for (uint32_t c = 0; c < len; ++c) {
          const float wv = __fmul_rn(e4m3_f32(ld1(rw, wo + c)), sb);
#pragma unroll
          for (int j = 0; j < MT; ++j) {
            const uint32_t xc = m0 + j < M ? ld1(rx, (m0 + j) * K + k0 + c) : 0u;
            p[j] = __fadd_rn(p[j], __fmul_rn(__fmul_rn(e4m3_f32(xc), sa[j]), wv));
          }
        }
      }
    }
#pragma unroll
    for (int j = 0; j < MT; ++j) lpart[(j * R + r) * G + g] = p[j];
  }
  __syncthreads();
  for (uint32_t t = threadIdx.x; t < uint32_t(MT) * R; t += 256u) {
    const uint32_t j = t / R, r = t % R, row = row0 + r, m = m0 + j;
    if (row >= N || m >= M) continue;
    const float *pp = lpart + (j * R + r) * G;
    float acc = 0.0f;
    for (uint32_t g = 0; g < G; ++g) acc = __fadd_rn(acc, pp[g]);
    if (a.bias) acc = __fadd_rn(acc, a.bias[row]);
    if (a.round_bf16) acc = bf16_round(acc);
    a.y[size_t(m) * N + row] = acc;
  }
}

// ---------------------------------------------------------------------------
// EXACT, tiled (k % 128 == 0, 16-byte aligned x and w): one wavefront per
// (64-row tile, scale group g, block of MT tokens), four independent
// wavefronts per workgroup.  The wavefront DMA-loads its 64 rows x 128 bytes
// of weight into LDS (buffer_load ... lds: 8 lanes per row, whole lines per
// quarter-wave; piece q of row r lands at piece q ^ (r & 7), so the later
// row-per-lane reads take distinct banks), and its tokens' 128 activation
// codes, decoded and scaled once: a = dec(x) * sa.  Lane l then owns row
// r0 + l: per 16 k it decodes b = dec(w) * sb and, for each token, adds
// a * b in k order, a reaching every lane as the multiply's DPP
// row-broadcast operand (lane i of each 16-lane row holds a[16c + i]).  The
// group partials go to the workspace, part[g][t][row]; k_linear_sum adds
// them in group order (acc = 0; acc += partial_g), adds the bias and rounds.
// Products and sums are the oracle's (fp8.py:173-191 with k ascending).
// ---------------------------------------------------------------------------
constexpr uint32_t kLTRows = 64;                    // rows per wavefront
constexpr uint32_t kLTWaves = 4;                    // wavefronts per workgroup
constexpr uint32_t kLTSlot = kLTRows * kLinGroup;   // 8 KiB of weight per wavefront
__shared__ __attribute__((aligned(16))) uint8_t lt_w[kLTWaves][kLTSlot];
__shared__ __attribute__((aligned(16))) uint8_t lt_x[kLTWaves][8][kLinGroup];

typedef __attribute__((address_space(3))) void lt_lds_void;

// One 16-k block: p[t] += a[t][16c + i] * b[i], i = 0..15 ascending, for
// MT tokens.  a reaches every lane as the DPP row-broadcast operand of the
// multiply (lane i of each 16-lane row: row_newbcast:i), written as asm
// because the compiler kept the broadcast as a separate move (plus a zeroed
// register) per product.  The MT multiplies of a step come before its MT
// adds, so no add waits on the one before it when MT > 1.  The DPP source
// a is written long before the block (no DPP wait states needed).
#define S14_LT_MUL(t, i) \
  "v_mul_f32_dpp %[q" #t "], %[a" #t "], %[b" #i "] row_newbcast:" #i " row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
#define S14_LT_ADD(t) "v_add_f32 %[p" #t "], %[q" #t "], %[p" #t "]\n"
#define S14_LT_STEP1(i) S14_LT_MUL(0, i) S14_LT_ADD(0)
#define S14_LT_STEP2(i) S14_LT_MUL(0, i) S14_LT_MUL(1, i) S14_LT_ADD(0) S14_LT_ADD(1)
#define S14_LT_STEP4(i) \
  S14_LT_MUL(0, i) S14_LT_MUL(1, i) S14_LT_MUL(2, i) S14_LT_MUL(3, i) \
  S14_LT_ADD(0) S14_LT_ADD(1) S14_LT_ADD(2) S14_LT_ADD(3)
#define S14_LT_STEP8(i) \
  S14_LT_MUL(0, i) S14_LT_MUL(1, i) S14_LT_MUL(2, i) S14_LT_MUL(3, i) S14_LT_MUL(4, i) S14_LT_MUL(5, i) \
  S14_LT_MUL(6, i) S14_LT_MUL(7, i) S14_LT_ADD(0) S14_LT_ADD(1) S14_LT_ADD(2) S14_LT_ADD(3) S14_LT_ADD(4) \
  S14_LT_ADD(5) S14_LT_ADD(6) S14_LT_ADD(7)
#define S14_LT_BLOCK(STEP) \
  STEP(0) STEP(1) STEP(2) STEP(3) STEP(4) STEP(5) STEP(6) STEP(7) STEP(8) STEP(9) STEP(10) STEP(11) STEP(12) \
  STEP(13) STEP(14) STEP(15)
#define S14_LT_B                                                                                               \
  [b0] "v"(bv[0]), [b1] "v"(bv[1]), [b2] "v"(bv[2]), [b3] "v"(bv[3]), [b4] "v"(bv[4]), [b5] "v"(bv[5]),         \
      [b6] "v"(bv[6]), [b7] "v"(bv[7]), [b8] "v"(bv[8]), [b9] "v"(bv[9]), [b10] "v"(bv[10]), [b11] "v"(bv[11]), \
      [b12] "v"(bv[12]), [b13] "v"(bv[13]), [b14] "v"(bv[14]), [b15] "v"(bv[15])

template <int MT>
__device__ __forceinline__ void lt_block16(float (&p)[MT], const float (&ac)[MT], const float (&bv)[16]);
template <>
__device__ __forceinline__ void lt_block16<1>(float (&p)[1], const float (&ac)[1], const float (&bv)[16]) {
  float q[1];
  asm volatile(S14_LT_BLOCK(S14_LT_STEP1) : [p0] "+v"(p[0]), [q0] "=&v"(q[0]) : [a0] "v"(ac[0]), S14_LT_B);
}
template <>
__device__ __forceinline__ void lt_block16<2>(float (&p)[2], const float (&ac)[2], const float (&bv)[16]) {
  float q[2];
  asm volatile(S14_LT_BLOCK(S14_LT_STEP2)
               : [p0] "+v"(p[0]), [p1] "+v"(p[1]), [q0] "=&v"(q[0]), [q1] "=&v"(q[1])
               : [a0] "v"(ac[0]), [a1] "v"(ac[1]), S14_LT_B);
}
template <>
__device__ __forceinline__ void lt_block16<4>(float (&p)[4], const float (&ac)[4], const float (&bv)[16]) {
  float q[4];
  asm volatile(S14_LT_BLOCK(S14_LT_STEP4)
               : [p0] "+v"(p[0]), [p1] "+v"(p[1]), [p2] "+v"(p[2]), [p3] "+v"(p[3]), [q0] "=&v"(q[0]),
                 [q1] "=&v"(q[1]), [q2] "=&v"(q[2]), [q3] "=&v"(q[3])
               : [a0] "v"(ac[0]), [a1] "v"(ac[1]), [a2] "v"(ac[2]), [a3] "v"(ac[3]), S14_LT_B);
}
template <>
__device__ __forceinline__ void lt_block16<8>(float (&p)[8], const float (&ac)[8], const float (&bv)[16]) {
  float q[8];
  asm volatile(S14_LT_BLOCK(S14_LT_STEP8)
               : [p0] "+v"(p[0]), [p1] "+v"(p[1]), [p2] "+v"(p[2]), [p3] "+v"(p[3]), [p4] "+v"(p[4]),
                 [p5] "+v"(p[5]), [p6] "+v"(p[6]), [p7] "+v"(p[7]), [q0] "=&v"(q[0]), [q1] "=&v"(q[1]),
                 [q2] "=&v"(q[2]), [q3] "=&v"(q[3]), [q4] "=&v"(q[4]), [q5] "=&v"(q[5]), [q6] "=&v"(q[6]),
                 [q7] "=&v"(q[7])
               : [a0] "v"(ac[0]), [a1] "v"(ac[1]), [a2] "v"(ac[2]), [a3] "v"(ac[3]), [a4] "v"(ac[4]),
                 [a5] "v"(ac[5]), [a6] "v"(ac[6]), [a7] "v"(ac[7]), S14_LT_B);
}
#undef S14_LT_B
#undef S14_LT_BLOCK
#undef S14_LT_STEP8
#undef S14_LT_STEP4
#undef S14_LT_STEP2
#undef S14_LT_STEP1
#undef S14_LT_ADD
#undef S14_LT_MUL

template <int MT, bool kXsF32, bool kWsF32>
__global__ __launch_bounds__(64 * kLTWaves) void k_linear_tile(LinearArgs a, float *__restrict__ part) {
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const uint32_t G = a.groups, K = a.k, N = a.n, M = a.m;
  const uint32_t task = blockIdx.x * kLTWaves + wave;
  const uint32_t tiles = (N + kLTRows - 1) / kLTRows;
  if (task >= tiles * G) return;  // uniform per wavefront; no workgroup barrier below
  const uint32_t tile = task / G, g = task % G;
  const uint32_t r0 = tile * kLTRows, k0 = g * kLinGroup, m0 = blockIdx.y * uint32_t(MT);
  const Rsrc rw = make_rsrc(a.w, N * K), rx = make_rsrc(a.x, M * K);
  const uint32_t n_sw = (N + 127u) / 128u * G, n_sx = M * G;
  const Rsrc rsw = make_rsrc(a.w_scale, kWsF32 ? 4u * n_sw : n_sw);
  const Rsrc rsx = make_rsrc(a.x_scale, kXsF32 ? 4u * n_sx : n_sx);
  uint8_t *slot = lt_w[wave];
  // weight tile: instruction j moves rows 8j .. 8j+7 (lane l: row 8j + l/8,
  // piece (l % 8) ^ (row & 7), landing at position l % 8 of that row)
#pragma unroll
  for (uint32_t j = 0; j < 8; ++j) {
    const uint32_t dr = 8u * j + (lane >> 3);
    const uint32_t off = (r0 + dr) * K + k0 + 16u * ((lane & 7u) ^ (dr & 7u));
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lt_lds_void *)(slot + 1024u * j), 16, off, 0, 0, 0);
  }
  // activation codes: lane l < 8 MT moves 16 bytes of token l / 8 (tokens
  // past m read zeros through the resource's bounds; their sums are not
  // stored)
  uint8_t(*xs)[kLinGroup] = lt_x[wave];
  if (lane < 8u * MT) {
    const uint32_t t = lane >> 3, piece = lane & 7u;
    const uint4 v = (m0 + t < M) ? ld16(rx, (m0 + t) * K + k0 + 16u * piece) : make_uint4(0u, 0u, 0u, 0u);
    *reinterpret_cast<uint4 *>(&xs[t][16u * piece]) = v;
  }
  float sa[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t)
    sa[t] = (m0 + t < M) ? (kXsF32 ? ldf(rsx, 4u * ((m0 + t) * G + g)) : ue8m0_f32(ld1(rsx, (m0 + t) * G + g))) : 0.0f;
  const float sb = kWsF32 ? ldf(rsw, 4u * ((r0 / 128u) * G + g)) : ue8m0_f32(ld1(rsw, (r0 / 128u) * G + g));
  // a[t][16c + i] in lane i of each 16-lane row: dec(x) * sa, the oracle's
  // f32 product
  float av[MT][8];
  const uint32_t li = lane & 15u;
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const uint32_t code = xs[t][16 * c + li];
      const v2f d = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(code, 1.0f, false);
      av[t][c] = __fmul_rn(d.x, sa[t]);
    }
  // the lane's row: 8 pieces of 16 codes (the DMA's writes are waited for
  // by the compiler before these reads)
  uint4 wr[8];
#pragma unroll
  for (int q = 0; q < 8; ++q)
    wr[q] = *reinterpret_cast<const uint4 *>(slot + 128u * lane + 16u * (uint32_t(q) ^ (lane & 7u)));
  float p[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) p[t] = 0.0f;
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const uint32_t words[4] = {wr[c].x, wr[c].y, wr[c].z, wr[c].w};
    float bv[16];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const v2f lo = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(words[d], 1.0f, false);
      const v2f hi = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(words[d], 1.0f, true);
      bv[4 * d + 0] = __fmul_rn(lo.x, sb);
      bv[4 * d + 1] = __fmul_rn(lo.y, sb);
      bv[4 * d + 2] = __fmul_rn(hi.x, sb);
      bv[4 * d + 3] = __fmul_rn(hi.y, sb);
    }
    float ac[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) ac[t] = av[t][c];
    lt_block16<MT>(p, ac, bv);  // k = 16c + i ascending
  }
  const uint32_t row = r0 + lane;
  if (row < N) {
#pragma unroll
    for (int t = 0; t < MT; ++t)
      if (m0 + t < M) part[(size_t(g) * M + (m0 + t)) * N + row] = p[t];
  }
}

// y[t][row] = (((0 + part_0) + part_1) + ...) + bias, rounded to bf16 when
// asked: one thread per (token, row), rows across lanes.  kLSumBatch groups'
// partials are requested at once (8 .. 64 by the group count: one round
// trip for k <= 8192).
template <uint32_t kLSumBatch>
__global__ __launch_bounds__(256) void k_linear_sum(LinearArgs a, const float *__restrict__ part) {
  const uint32_t N = a.n, M = a.m, G = a.groups;
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  if (i >= M * N) return;
  const uint32_t t = i / N, row = i % N;
  // the partials (at most kLinPartBytes) through a buffer descriptor: the
  // lane's offset in a VGPR, each group's in the scalar offset; groups past
  // G read zeros and are not added
  const uint32_t stride = 4u * M * N;
  const Rsrc rp = make_rsrc(part, G * stride);
  const uint32_t lane_off = 4u * (t * N + row);
  float acc = 0.0f;
  for (uint32_t g0 = 0; g0 < G; g0 += kLSumBatch) {
    float v[kLSumBatch];
#pragma unroll
    for (uint32_t j = 0; j < kLSumBatch; ++j)
      v[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rp, lane_off, (g0 + j) * stride, 0));
#pragma unroll
    for (uint32_t j = 0; j < kLSumBatch; ++j)
      if (g0 + j < G) acc = __fadd_rn(acc, v[j]);
  }
  if (a.bias) acc = __fadd_rn(acc, a.bias[row]);
  if (a.round_bf16) acc = bf16_round(acc);
  a.y[size_t(t) * N + row] = acc;
}

// ---------------------------------------------------------------------------
// FAST: one wavefront per (32-row tile, K split, 32-token block).  A chunk is
// one scale group: 32 rows x 128 k of weight (4 KiB), DMA-loaded into a ring
// of four LDS slots with four chunks in flight (buffer_load ... lds, 8 lanes
// per row so each quarter-wave moves two whole 128-byte rows).  Before the
// ring starts, the wavefront stages its tokens' activations for all of its
// chunks in LDS, decoded to bf16; with UE8M0 scales the power of two
// sa[t][g] * sb[g] is folded into them exactly, so the MFMAs accumulate the
// whole K range into one f32 accumulator; with f32 scales each chunk's sums
// are scaled after its MFMAs (acc += part * sa[t][g] * sb[g]).  Only the
// weight DMA is then on the vector-memory counter, so waiting for a chunk
// never waits for the chunks behind it.
//
// Operand layout (32x32x16 bf16, lane l = column l % 32, half h = l / 32;
// value j of an A lane pairs with value j of the B lane of the same half):
// for steps 2q and 2q + 1 lane (r, h) reads the 16 bytes k = 16 (2q + h) ..
// +15 of weight row r (one LDS read) and uses bytes 0-7 in step 2q, bytes
// 8-15 in step 2q + 1; lane (t, h) reads the same 16 k of token t.  D
// element i of lane l: row 8 (i / 4) + 4 h + i % 4, column l % 32.  Lanes
// of tokens past m read token 0's activations: an MFMA column depends on its
// own B column only, and those columns are never stored.
//
// Splits > 1: each wavefront stores its 32 x 32 partial tile; the last to
// arrive at the tile's counter adds the partials in split order, adds the
// bias and writes y, and resets the counter for the next launch.
// ---------------------------------------------------------------------------

constexpr uint32_t kLChunkBytes = kLinTile * kLinGroup;
__shared__ __attribute__((aligned(16))) uint8_t lin_slot0[kLChunkBytes];
__shared__ __attribute__((aligned(16))) uint8_t lin_slot1[kLChunkBytes];
__shared__ __attribute__((aligned(16))) uint8_t lin_slot2[kLChunkBytes];
__shared__ __attribute__((aligned(16))) uint8_t lin_slot3[kLChunkBytes];

// Each slot is its own LDS array, so the compiler waits for one slot's DMA
// without draining the others.
template <int S>
__device__ __forceinline__ uint8_t *lin_slot() {
  if constexpr (S == 0) return lin_slot0;
  else if constexpr (S == 1) return lin_slot1;
  else if constexpr (S == 2) return lin_slot2;
  else return lin_slot3;
}
template <int S>
struct LSlot {
  static constexpr int value = S;
};
// f(LSlot<S>{}) for S = B .. E - 1, in order, unrolled
template <int B, int E, class F>
__device__ __forceinline__ void for_slots(F &&f) {
  if constexpr (B < E) {
    f(LSlot<B>{});
    for_slots<B + 1, E>(f);
  }
}

typedef __attribute__((address_space(3))) void lds_void;
__device__ __forceinline__ void lin_dma16(Rsrc r, uint8_t *lds, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)(lds), 16, off, 0, 0, 0);
}
// Before a DMA load refills a slot, the LDS reads of its previous chunk have
// returned.
__device__ __forceinline__ void lin_lds_reads_done() { __builtin_amdgcn_s_waitcnt(0xc07f); }
// 16-byte piece q of row r sits at piece q ^ lin_swz(r): the 32 rows of a
// read pass spread over the banks.
__device__ __forceinline__ uint32_t lin_swz(uint32_t r) { return (r + (r >> 3)) & 7u; }

// Cache policy of the split-K partials' loads: agent scope (sc1), coherent
// with the write-through stores of the other XCDs.
constexpr int kCacheAgent = 0x10;

// Sixteen e4m3 codes times a power of two (or 1) as sixteen bf16, exact.
__device__ __forceinline__ v4u e4m3x4_bf16s(uint32_t w0, uint32_t w1, float s) {
  return v4u{__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, s, false)),
             __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, s, true)),
             __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, s, false)),
             __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, s, true))};
}

template <bool kXsF32, bool kWsF32, int kRing>
__global__ __launch_bounds__(64) void k_linear_fast(LinearArgs a, LinearWorkspace ws, uint32_t cw, uint32_t splits) {
  constexpr bool kFold = !kXsF32 && !kWsF32;  // power-of-two scales ride in the bf16 activations
  extern __shared__ __attribute__((aligned(16))) uint8_t lin_x[];  // [ntok][cw * 128] bf16, then [ntok][cw] f32
  const uint32_t tile = blockIdx.x, sidx = blockIdx.y, cb = blockIdx.z, ncb = gridDim.z;
  const uint32_t lane = threadIdx.x & 63u, col = lane & 31u, h = lane >> 5;
  const uint32_t K = a.k, N = a.n, M = a.m, G = a.groups;
  const uint32_t g0 = sidx * cw;
  const uint32_t tok0 = cb * kLinTile, ntok = min(kLinTile, M - tok0);
  const Rsrc rw = make_rsrc(a.w, N * K);
  const Rsrc rx = make_rsrc(a.x, M * K);
  const uint32_t n_sw = (N + 127u) / 128u * G, n_sx = M * G;
  const Rsrc rsw = make_rsrc(a.w_scale, kWsF32 ? 4u * n_sw : n_sw);
  const Rsrc rsx = make_rsrc(a.x_scale, kXsF32 ? 4u * n_sx : n_sx);
  const uint32_t sbrow = (tile * kLinTile / 128u) * G;
  // DMA lane map: load j of a chunk covers rows 8j..8j+7 of the tile; lane
  // -> row 8j + lane / 8, LDS piece lane % 8 holding source piece
  // (lane % 8) ^ lin_swz(row), lin_swz(8j + r) = (j + r) % 8
  const uint32_t lrow = lane >> 3;
  uint32_t dma_off[4];
#pragma unroll
  for (uint32_t j = 0; j < 4; ++j)
    dma_off[j] = (tile * kLinTile + 8u * j + lrow) * K + 16u * ((lane & 7u) ^ ((j + lrow) & 7u));
  auto issue = [&](auto slot_tag, uint32_t c) {
    uint8_t *dst = lin_slot<decltype(slot_tag)::value>();
    lin_lds_reads_done();
    const uint32_t kb = (g0 + c) * kLinGroup;
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) lin_dma16(rw, dst + 1024u * j, dma_off[j] + kb);
  };
  // the first kRing chunks' weights are in flight while the activations are staged
  for_slots<0, kRing>([&](auto sl) { issue(sl, uint32_t(decltype(sl)::value)); });
  // stage: item = (token, chunk, 16-k piece), one 16-byte load per item
  const uint32_t row_elems = cw * kLinGroup;  // bf16 per staged token
  float *stage_scale = reinterpret_cast<float *>(lin_x + size_t(ntok) * row_elems * 2u);
  for (uint32_t item = lane; item < ntok * cw * 8u; item += 64u) {
    const uint32_t t = item / (cw * 8u), pc = item % (cw * 8u), c = pc >> 3, piece = pc & 7u;
    const uint32_t g = g0 + c;
    const uint4 codes = ld16(rx, (tok0 + t) * K + g * kLinGroup + 16u * piece);
    float s = 1.0f;
    if constexpr (kFold) s = ue8m0_f32(ld1(rsx, (tok0 + t) * G + g)) * ue8m0_f32(ld1(rsw, sbrow + g));
    v4u *dst = reinterpret_cast<v4u *>(lin_x + (size_t(t) * row_elems + c * kLinGroup + 16u * piece) * 2u);
    dst[0] = e4m3x4_bf16s(codes.x, codes.y, s);
    dst[1] = e4m3x4_bf16s(codes.z, codes.w, s);
    if constexpr (!kFold) {
      if (piece == 0) {
        const float sa = kXsF32 ? ldf(rsx, 4u * ((tok0 + t) * G + g)) : ue8m0_f32(ld1(rsx, (tok0 + t) * G + g));
        const float sb = kWsF32 ? ldf(rsw, 4u * (sbrow + g)) : ue8m0_f32(ld1(rsw, sbrow + g));
        stage_scale[t * cw + c] = sa * sb;
      }
    }
  }
  __syncthreads();
  const uint32_t my_tok = col < ntok ? col : 0u;
  const uint8_t *xrow = lin_x + size_t(my_tok) * row_elems * 2u + 32u * h;
  v16f acc;
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
  const uint32_t sw = lin_swz(col);
  auto consume = [&](auto slot_tag, uint32_t c) {
    constexpr int S = decltype(slot_tag)::value;
    const uint8_t *src = lin_slot<S>() + 128u * col;
    const uint8_t *xb = xrow + c * (kLinGroup * 2u);
    v16f part;
    if constexpr (!kFold) {
#pragma unroll
      for (int i = 0; i < 16; ++i) part[i] = 0.0f;
    }
#pragma unroll
    for (uint32_t q = 0; q < 4; ++q) {
      const uint4 w = *reinterpret_cast<const uint4 *>(src + 16u * ((2u * q + h) ^ sw));
      const v8bf b0 = *reinterpret_cast<const v8bf *>(xb + 64u * q);
      const v8bf b1 = *reinterpret_cast<const v8bf *>(xb + 64u * q + 16u);
      if constexpr (kFold) {
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(e4m3x8_bf16(w.x, w.y), b0, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(e4m3x8_bf16(w.z, w.w), b1, acc, 0, 0, 0);
      } else {
        part = __builtin_amdgcn_mfma_f32_32x32x16_bf16(e4m3x8_bf16(w.x, w.y), b0, part, 0, 0, 0);
        part = __builtin_amdgcn_mfma_f32_32x32x16_bf16(e4m3x8_bf16(w.z, w.w), b1, part, 0, 0, 0);
      }
    }
    if constexpr (!kFold) {
      const float s = stage_scale[my_tok * cw + c];
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[i] = fmaf(part[i], s, acc[i]);
    }
  };
  // cw is a multiple of kRing (host): whole rounds of the ring; a slot is
  // refilled as soon as it has been read
#pragma unroll 1
  for (uint32_t c = 0; c + kRing < cw; c += kRing) {
    for_slots<0, kRing>([&](auto sl) {
      constexpr uint32_t S = decltype(sl)::value;
      consume(sl, c + S);
      issue(sl, c + kRing + S);
    });
  }
  for_slots<0, kRing>([&](auto sl) { consume(sl, cw - kRing + uint32_t(decltype(sl)::value)); });
  // pin the accumulators in uniform control flow before the per-lane epilogue
  asm volatile("" : "+v"(acc));
  const uint32_t token = tok0 + col;
  const bool live = col < ntok;
  const uint32_t rbase = tile * kLinTile + 4u * h;  // + 8 q + v
  if (splits > 1u) {
    // The partials are written and read with agent-scope atomics (coherent
    // across the XCDs' L2s without a whole-L2 write-back, which an
    // agent-scope release fence per wavefront would cost); the arrival
    // counts after this wavefront's partial stores have completed.
    const uint32_t slot = tile * ncb + cb;
    float *mine = ws.part + (size_t(slot) * splits + sidx) * (kLinTile * kLinTile) + col * kLinTile + 4u * h;
    if (live) {
#pragma unroll
      for (int i = 0; i < 16; ++i)
        __hip_atomic_store(mine + 8 * (i / 4) + (i % 4), acc[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wavefront's stores are done
    uint32_t prev = 0;
    if (lane == 0) prev = __hip_atomic_fetch_add(ws.count + slot, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    prev = uint32_t(__shfl(int(prev), 0));
    if (prev + 1u != splits) return;
    // last arrival: every other split's partial is complete (and no load of
    // them may move above this point)
    asm volatile("" ::: "memory");
    if (lane == 0) __hip_atomic_store(ws.count + slot, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (!live) return;
    // agent-scope loads, four splits' partials in flight at a time, summed
    // in split order
    const Rsrc rp = make_rsrc(ws.part + size_t(slot) * splits * (kLinTile * kLinTile),
                              splits * (kLinTile * kLinTile) * 4u);
    const uint32_t lo = 4u * (col * kLinTile + 4u * h);
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
    for (uint32_t s0 = 0; s0 < splits; s0 += 4u) {
      v4u v[4][4];
#pragma unroll
      for (uint32_t j = 0; j < 4; ++j)
#pragma unroll
        for (uint32_t q = 0; q < 4; ++q)  // past the last split: zeros (descriptor range)
          v[j][q] = __builtin_amdgcn_raw_buffer_load_b128(rp, ((s0 + j) * (kLinTile * kLinTile)) * 4u + lo + 32u * q,
                                                          0, kCacheAgent);
#pragma unroll
      for (uint32_t j = 0; j < 4; ++j)
#pragma unroll
        for (uint32_t q = 0; q < 4; ++q) {
          acc[4 * q] += __uint_as_float(v[j][q].x);
          acc[4 * q + 1] += __uint_as_float(v[j][q].y);
          acc[4 * q + 2] += __uint_as_float(v[j][q].z);
          acc[4 * q + 3] += __uint_as_float(v[j][q].w);
        }
    }
  }
  if (!live) return;
  float *yrow = a.y + size_t(token) * N;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const uint32_t row = rbase + 8u * uint32_t(i / 4) + uint32_t(i % 4);
    if (row >= N) continue;
    float v = acc[i];
    if (a.bias) v += a.bias[row];
    if (a.round_bf16) v = bf16_round(v);
    yrow[row] = v;
  }
}

// FAST for one or two tokens (up to four where n is small) and k a multiple
// of 1,024: a VALU GEMV,
// where the MFMA path would spend 32-token tiles on one token.  One
// wavefront per R rows, R = 8 / (k / 1,024) (at least 1), so that a
// wavefront's eight coalesced 1 KiB code loads (R rows x its k / 1,024
// chunks) are all in flight at once and every projection shape gets ~4,096
// wavefronts, four per SIMD; a longer k takes its chunks in batches of
// eight, the next batch in flight during this one.  In chunk c (1,024 k)
// lane l holds k 1024 c + 16 l .. + 15, which lie in group 8 c + l / 8.
// e4m3 x e4m3 products are exact in f32; each lane sums its 16 per (row,
// token) by fused multiply-adds, scales the sum by the group's two scales
// and accumulates; the wavefront sum (DPP) gives the row.  (Splitting k
// across wavefronts instead, with the split partials met as k_linear_fast
// meets them, was slower at wo_a and wo_b: 13.3 and 14.9 us.)
constexpr uint32_t kGvChunk = 1024, kGvLoads = 8, kGvWaves = 4;
template <int MT, int R, bool kXsF32, bool kWsF32>
__global__ __launch_bounds__(64 * kGvWaves) void k_linear_gemv(LinearArgs a) {
  constexpr uint32_t kB = kGvLoads / uint32_t(R);  // chunks per batch
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t r0 = (blockIdx.x * kGvWaves + (threadIdx.x >> 6)) * uint32_t(R);
  const uint32_t K = a.k, N = a.n, M = a.m, G = a.groups;
  if (r0 >= N) return;  // whole wavefronts
  const uint32_t chunks = K / kGvChunk;
  const Rsrc rw = make_rsrc(a.w, N * K);
  const Rsrc rx = make_rsrc(a.x, M * K);
  const uint32_t n_sw = (N + 127u) / 128u * G, n_sx = M * G;
  const Rsrc rsw = make_rsrc(a.w_scale, kWsF32 ? 4u * n_sw : n_sw);
  const Rsrc rsx = make_rsrc(a.x_scale, kXsF32 ? 4u * n_sx : n_sx);
  const uint32_t sbrow = (r0 / 128u) * G;  // the R rows share a 128-row scale block
  uint32_t woff[R];
#pragma unroll
  for (int r = 0; r < R; ++r) woff[r] = min(r0 + uint32_t(r), N - 1u) * K + 16u * lane;  // rows past n: unused
  float acc[R][MT];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[r][t] = 0.0f;
  uint4 cur[kB][R], nxt[kB][R];
  auto load = [&](uint4 (&dst)[kB][R], uint32_t c0) {
#pragma unroll
    for (uint32_t b = 0; b < kB; ++b)
#pragma unroll
      for (int r = 0; r < R; ++r) dst[b][r] = ld16(rw, woff[r] + min(c0 + b, chunks - 1u) * kGvChunk);
  };
  load(cur, 0);
#pragma unroll 1
  for (uint32_t c0 = 0; c0 < chunks; c0 += kB) {
    if (c0 + kB < chunks) load(nxt, c0 + kB);
#pragma unroll
    for (uint32_t b = 0; b < kB; ++b) {
      const uint32_t c = c0 + b;
      if (c >= chunks) break;  // uniform (a shorter last batch)
      const uint32_t g = c * (kGvChunk / kLinGroup) + lane / 8u;  // this lane's group
      const float sb = kWsF32 ? ldf(rsw, 4u * (sbrow + g)) : ue8m0_f32(ld1(rsw, sbrow + g));
      float xv[MT][16], s[MT];
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        const uint32_t tt = min(uint32_t(t), M - 1u);  // tokens past m: unused
        const uint4 q = ld16(rx, tt * K + c * kGvChunk + 16u * lane);
        const float sa = kXsF32 ? ldf(rsx, 4u * (tt * G + g)) : ue8m0_f32(ld1(rsx, tt * G + g));
        s[t] = sa * sb;
        const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const auto lo = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(qw[j], 1.0f, false);
          const auto hi = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(qw[j], 1.0f, true);
          xv[t][4 * j] = lo[0];
          xv[t][4 * j + 1] = lo[1];
          xv[t][4 * j + 2] = hi[0];
          xv[t][4 * j + 3] = hi[1];
        }
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const uint32_t ww[4] = {cur[b][r].x, cur[b][r].y, cur[b][r].z, cur[b][r].w};
        float wf[16];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const auto lo = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(ww[j], 1.0f, false);
          const auto hi = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(ww[j], 1.0f, true);
          wf[4 * j] = lo[0];
          wf[4 * j + 1] = lo[1];
          wf[4 * j + 2] = hi[0];
          wf[4 * j + 3] = hi[1];
        }
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          float p = 0.0f;
#pragma unroll
          for (int j = 0; j < 16; ++j) p = fmaf(xv[t][j], wf[j], p);
          acc[r][t] = fmaf(p, s[t], acc[r][t]);
        }
      }
    }
#pragma unroll
    for (uint32_t b = 0; b < kB; ++b)
#pragma unroll
      for (int r = 0; r < R; ++r) cur[b][r] = nxt[b][r];
  }
  // every lane gets every (row, token) total; lane r MT + t writes (r, t)
  float mine = 0.0f;
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const float v = wave_sum_dpp(acc[r][t]);
      mine = lane == uint32_t(r * MT + t) ? v : mine;
    }
  const uint32_t orow = r0 + lane / uint32_t(MT), otok = lane % uint32_t(MT);
  if (lane >= uint32_t(R * MT) || orow >= N || otok >= M) return;
  float v = mine;
  if (a.bias) v += a.bias[orow];
  if (a.round_bf16) v = bf16_round(v);
  a.y[size_t(otok) * N + orow] = v;
}

// EXACT for one token and k of 1,024, 2,048, 4,096 or 8,192 (G = k / 128
// groups): one launch where the tiled kernel takes two.  A wavefront owns
// R = 64 / G rows, lane (r, g) = (lane / G, lane % G) one group of one row,
// summed in the oracle's order (k ascending; a = dec(x) * sa, b = dec(w) *
// sb, partial += a * b; with UE8M0 scales the scaled converter forms each
// exactly); the row's lanes then fold their partials in group order
// (acc = 0; acc += partial_g) and one lane adds the bias.  The wavefront's
// R x k weight block (8 KiB) arrives by eight coalesced DMA loads into LDS,
// x's codes once per workgroup; piece q of a group's 128 bytes sits at
// q ^ swz (w: (swz8(g) + r) % 8, x: swz8(g)), so a read pass of 16 lanes
// hits distinct banks.
constexpr uint32_t kGxWaves = 4;
__device__ __forceinline__ uint32_t gx_swz8(uint32_t g) { return (g + (g >> 3)) & 7u; }
template <int R, bool kXsF32, bool kWsF32>
__global__ __launch_bounds__(64 * kGxWaves) void k_linear_gemv_exact(LinearArgs a) {
  constexpr uint32_t G = 64u / uint32_t(R), K = G * kLinGroup;
  __shared__ __attribute__((aligned(16))) uint8_t gx_w[kGxWaves][uint32_t(R) * K];
  __shared__ __attribute__((aligned(16))) uint8_t gx_x[K];
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63u;
  const uint32_t N = a.n;
  const uint32_t r0 = (blockIdx.x * kGxWaves + wave) * uint32_t(R);
  const Rsrc rw = make_rsrc(a.w, N * K), rx = make_rsrc(a.x, K);
  const uint32_t n_sw = (N + 127u) / 128u * G;
  const Rsrc rsw = make_rsrc(a.w_scale, kWsF32 ? 4u * n_sw : n_sw);
  const Rsrc rsx = make_rsrc(a.x_scale, kXsF32 ? 4u * G : G);
  if (r0 < N) {  // uniform per wavefront: its weight block, in flight during the x copy
#pragma unroll
    for (uint32_t j = 0; j < 8; ++j) {
      const uint32_t r = (1024u * j) / K, u = (1024u * j) % K / 16u + lane;  // row, 16-byte unit of the row
      const uint32_t g = u / 8u, q = (u % 8u) ^ ((gx_swz8(g) + r) & 7u);
      const uint32_t off = min(r0 + r, N - 1u) * K + kLinGroup * g + 16u * q;  // rows past n: unused
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lt_lds_void *)(gx_w[wave] + 1024u * j), 16, off, 0, 0, 0);
    }
  }
  for (uint32_t i = threadIdx.x; i < K / 16u; i += 64u * kGxWaves) {
    const uint32_t g = i / 8u, q = i % 8u;
    *reinterpret_cast<uint4 *>(gx_x + kLinGroup * g + 16u * (q ^ gx_swz8(g))) = ld16(rx, 16u * i);
  }
  __syncthreads();
  if (r0 >= N) return;
  const uint32_t r = lane / G, g = lane % G;
  const uint32_t row = min(r0 + r, N - 1u);
  const uint32_t si = (row / 128u) * G + g;
  const uint32_t cx = kXsF32 ? 0u : ld1(rsx, g), cw = kWsF32 ? 0u : ld1(rsw, si);
  const float sa = kXsF32 ? ldf(rsx, 4u * g) : ue8m0_f32(cx);
  const float sb = kWsF32 ? ldf(rsw, 4u * si) : ue8m0_f32(cw);
  // UE8M0 scales whose every a, b and a * b stays normal or zero (|dec| in
  // [2^-9, 448]): the converters' scale operand forms a and b exactly, the
  // same values as the separate multiplies
  const bool scaled = !kXsF32 && !kWsF32 && cx >= 10u && cx <= 246u && cw >= 10u && cw <= 246u &&
                      cx + cw >= 146u && cx + cw <= 364u;
  const uint8_t *wp = gx_w[wave] + r * K + kLinGroup * g;
  const uint8_t *xp = gx_x + kLinGroup * g;
  const uint32_t sw = (gx_swz8(g) + r) & 7u, sx = gx_swz8(g);
  float partial = 0.0f;
  auto group_sum = [&](auto scaled_tag) {
    constexpr bool kScaled = decltype(scaled_tag)::value;
#pragma unroll
    for (uint32_t j = 0; j < 8; ++j) {
      const uint4 wq = *reinterpret_cast<const uint4 *>(wp + 16u * (j ^ sw));
      const uint4 xq = *reinterpret_cast<const uint4 *>(xp + 16u * (j ^ sx));
      const uint32_t ww[4] = {wq.x, wq.y, wq.z, wq.w}, xw[4] = {xq.x, xq.y, xq.z, xq.w};
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        float av[4], bv[4];
        if constexpr (kScaled) {
          const v2f xl = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(xw[d], sa, false);
          const v2f xh = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(xw[d], sa, true);
          const v2f wl = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(ww[d], sb, false);
          const v2f wh = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(ww[d], sb, true);
          av[0] = xl.x, av[1] = xl.y, av[2] = xh.x, av[3] = xh.y;
          bv[0] = wl.x, bv[1] = wl.y, bv[2] = wh.x, bv[3] = wh.y;
        } else {
          const v2f xl = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(xw[d], 1.0f, false);
          const v2f xh = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(xw[d], 1.0f, true);
          const v2f wl = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(ww[d], 1.0f, false);
          const v2f wh = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(ww[d], 1.0f, true);
          av[0] = __fmul_rn(xl.x, sa), av[1] = __fmul_rn(xl.y, sa), av[2] = __fmul_rn(xh.x, sa), av[3] = __fmul_rn(xh.y, sa);
          bv[0] = __fmul_rn(wl.x, sb), bv[1] = __fmul_rn(wl.y, sb), bv[2] = __fmul_rn(wh.x, sb), bv[3] = __fmul_rn(wh.y, sb);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) partial = __fadd_rn(partial, __fmul_rn(av[e], bv[e]));  // k ascending
      }
    }
  };
  if (scaled)
    group_sum(std::true_type{});
  else
    group_sum(std::false_type{});
  // row rr's sum in group order, the same in every lane; lane rr writes it
  float mine = 0.0f;
#pragma unroll
  for (int rr = 0; rr < R; ++rr) {
    float acc = 0.0f;
#pragma unroll
    for (uint32_t gg = 0; gg < G; ++gg)
      acc = __fadd_rn(acc, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(partial), int(uint32_t(rr) * G + gg))));
    mine = lane == uint32_t(rr) ? acc : mine;
  }
  if (lane >= uint32_t(R) || r0 + lane >= N) return;
  float v = mine;
  if (a.bias) v = __fadd_rn(v, a.bias[r0 + lane]);
  if (a.round_bf16) v = bf16_round(v);
  a.y[r0 + lane] = v;
}

}  // namespace

hipError_t launch_act_quant(hipStream_t s, uint32_t rows, uint32_t k, uint32_t group, const float *x, uint8_t *q,
                            uint8_t *scales) {
  const uint32_t n = rows * (k / group);
  k_act_quant<<<(n + 255) / 256, 256, 0, s>>>(n, group, x, q, scales);
  return hipGetLastError();
}

// Slots in flight per wavefront.  Eight (a wavefront's whole K range at the
// projections' shapes requested at once) measured slower than four at every
// shape: wq_b 10.7 -> 12.2 us, and 12.7 -> 19.1 us for 8 tokens.
constexpr int kLinRing = 4;

template <int kRing>
static void launch_fast_ring(hipStream_t s, const LinearArgs &a, const LinearWorkspace &ws, uint32_t cw,
                             uint32_t splits, dim3 grid, size_t lds) {
  if (a.x_scale_f32 && a.w_scale_f32)
    k_linear_fast<true, true, kRing><<<grid, 64, lds, s>>>(a, ws, cw, splits);
  else if (a.x_scale_f32)
    k_linear_fast<true, false, kRing><<<grid, 64, lds, s>>>(a, ws, cw, splits);
  else if (a.w_scale_f32)
    k_linear_fast<false, true, kRing><<<grid, 64, lds, s>>>(a, ws, cw, splits);
  else
    k_linear_fast<false, false, kRing><<<grid, 64, lds, s>>>(a, ws, cw, splits);
}

template <int MT>
static hipError_t launch_exact_mt(hipStream_t s, const LinearArgs &a, bool vec) {
  const uint32_t G = a.groups;
  const uint32_t R = G >= 256u ? 1u : 256u / G;
  const dim3 grid((a.n + R - 1) / R, (a.m + MT - 1) / MT);
  const size_t lds = sizeof(float) * MT * R * G;
  if (vec)
    k_linear_exact<MT, true><<<grid, 256, lds, s>>>(a);
  else
    k_linear_exact<MT, false><<<grid, 256, lds, s>>>(a);
  return hipGetLastError();
}

template <int MT>
static void launch_tile_mt(hipStream_t s, const LinearArgs &a, float *part) {
  const uint32_t tasks = (a.n + kLTRows - 1) / kLTRows * a.groups;
  const dim3 grid((tasks + kLTWaves - 1) / kLTWaves, (a.m + MT - 1) / MT);
  if (a.x_scale_f32 && a.w_scale_f32)
    k_linear_tile<MT, true, true><<<grid, 64 * kLTWaves, 0, s>>>(a, part);
  else if (a.x_scale_f32)
    k_linear_tile<MT, true, false><<<grid, 64 * kLTWaves, 0, s>>>(a, part);
  else if (a.w_scale_f32)
    k_linear_tile<MT, false, true><<<grid, 64 * kLTWaves, 0, s>>>(a, part);
  else
    k_linear_tile<MT, false, false><<<grid, 64 * kLTWaves, 0, s>>>(a, part);
}

// The tiled EXACT path, in token chunks whose group partials fit the
// workspace (kLinPartBytes): tile kernel, then the ordered group sum.
static hipError_t launch_exact_tiled(hipStream_t s, const LinearArgs &a, const LinearWorkspace &ws) {
  const size_t per_token = size_t(a.groups) * a.n * sizeof(float);
  const uint32_t chunk = uint32_t(std::min<size_t>(a.m, kLinPartBytes / per_token));
  if (chunk == 0) return hipErrorInvalidValue;  // one token's partials exceed the workspace (the caller checks)
  const uint32_t xs_stride = a.x_scale_f32 ? 4u : 1u;
  for (uint32_t m0 = 0; m0 < a.m; m0 += chunk) {
    LinearArgs c = a;
    c.m = std::min(chunk, a.m - m0);
    c.x = a.x + size_t(m0) * a.k;
    c.x_scale = static_cast<const uint8_t *>(a.x_scale) + size_t(m0) * a.groups * xs_stride;
    c.y = a.y + size_t(m0) * a.n;
    if (c.m == 1)
      launch_tile_mt<1>(s, c, ws.part);
    else if (c.m == 2)
      launch_tile_mt<2>(s, c, ws.part);
    else if (c.m <= 4)
      launch_tile_mt<4>(s, c, ws.part);
    else
      launch_tile_mt<8>(s, c, ws.part);
    const dim3 sum_grid((c.m * c.n + 255u) / 256u);
    if (c.groups <= 8u)
      k_linear_sum<8><<<sum_grid, 256, 0, s>>>(c, ws.part);
    else if (c.groups <= 16u)
      k_linear_sum<16><<<sum_grid, 256, 0, s>>>(c, ws.part);
    else if (c.groups <= 32u)
      k_linear_sum<32><<<sum_grid, 256, 0, s>>>(c, ws.part);
    else
      k_linear_sum<64><<<sum_grid, 256, 0, s>>>(c, ws.part);
    if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
  }
  return hipSuccess;
}

template <int MT, int R>
static void launch_gemv(hipStream_t s, const LinearArgs &a) {
  const uint32_t waves = (a.n + R - 1) / R;
  const dim3 grid((waves + kGvWaves - 1) / kGvWaves);
  if (a.x_scale_f32 && a.w_scale_f32)
    k_linear_gemv<MT, R, true, true><<<grid, 64 * kGvWaves, 0, s>>>(a);
  else if (a.x_scale_f32)
    k_linear_gemv<MT, R, true, false><<<grid, 64 * kGvWaves, 0, s>>>(a);
  else if (a.w_scale_f32)
    k_linear_gemv<MT, R, false, true><<<grid, 64 * kGvWaves, 0, s>>>(a);
  else
    k_linear_gemv<MT, R, false, false><<<grid, 64 * kGvWaves, 0, s>>>(a);
}
template <int MT>
static void launch_gemv_mt(hipStream_t s, const LinearArgs &a) {
  const uint32_t chunks = a.k / kGvChunk;
  if (chunks == 1)
    launch_gemv<MT, 8>(s, a);
  else if (chunks == 2)
    launch_gemv<MT, 4>(s, a);
  else if (chunks <= 4)
    launch_gemv<MT, 2>(s, a);
  else
    launch_gemv<MT, 1>(s, a);
}

template <int R>
static void launch_gemv_exact(hipStream_t s, const LinearArgs &a) {
  const uint32_t waves = (a.n + R - 1) / R;
  const dim3 grid((waves + kGxWaves - 1) / kGxWaves);
  if (a.x_scale_f32 && a.w_scale_f32)
    k_linear_gemv_exact<R, true, true><<<grid, 64 * kGxWaves, 0, s>>>(a);
  else if (a.x_scale_f32)
    k_linear_gemv_exact<R, true, false><<<grid, 64 * kGxWaves, 0, s>>>(a);
  else if (a.w_scale_f32)
    k_linear_gemv_exact<R, false, true><<<grid, 64 * kGxWaves, 0, s>>>(a);
  else
    k_linear_gemv_exact<R, false, false><<<grid, 64 * kGxWaves, 0, s>>>(a);
}

hipError_t launch_fp8_linear(hipStream_t s, const LinearArgs &a, int mode, const LinearWorkspace &ws) {
  // the GEMV where it measured faster than the MFMA tiles (graph replays,
  // us: wq_b m = 1 8.5 against 10.4, m = 2 10.9 against 10.7; wo_a m = 2 11.2
  // against 12.6, m = 3 14.7 against 13.1; wkv m = 4 4.9 against 7.9)
  const bool gemv = a.m == 1u || (a.m == 2u && a.n <= 8192u) || (a.m <= 4u && a.n <= 1024u);
  if (mode == S14_MODE_FAST && gemv && a.k % kGvChunk == 0u && uint64_t(a.n) * a.k <= 0xFFFFFFFFull) {
    if (a.m == 1)
      launch_gemv_mt<1>(s, a);
    else if (a.m == 2)
      launch_gemv_mt<2>(s, a);
    else
      launch_gemv_mt<4>(s, a);
    return hipGetLastError();
  }
  const bool fast = mode == S14_MODE_FAST && a.k % (4u * kLinGroup) == 0u;
  const LinFastPlan plan = fast ? lin_fast_plan(a.m, a.n, a.groups) : LinFastPlan{0, 0};
  if (plan.cw) {
    // one launch per plan.blocks token blocks, each within the workspace's
    // partials and counters (a smaller last launch fits whatever fits more)
    const uint32_t tiles = (a.n + kLinTile - 1) / kLinTile, per = plan.blocks * kLinTile;
    const uint32_t xs_stride = a.x_scale_f32 ? 4u : 1u;
    for (uint32_t m0 = 0; m0 < a.m; m0 += per) {
      LinearArgs c = a;
      c.m = std::min(per, a.m - m0);
      c.x = a.x + size_t(m0) * a.k;
      c.x_scale = static_cast<const uint8_t *>(a.x_scale) + size_t(m0) * a.groups * xs_stride;
      c.y = a.y + size_t(m0) * a.n;
      const uint32_t ncb = (c.m + kLinTile - 1) / kLinTile, ntok = std::min(c.m, kLinTile);
      const uint32_t cw = lin_fast_chunks(a.groups, tiles, ncb, ntok);
      const uint32_t splits = cw ? a.groups / cw : 0u;
      if (!cw || lin_part_bytes(tiles, ncb, splits) > kLinPartBytes ||
          (splits > 1u && uint64_t(tiles) * ncb > kLinMaxCounters))
        return hipErrorInvalidValue;  // unreachable: the plan fits every launch
      launch_fast_ring<kLinRing>(s, c, ws, cw, splits, dim3(tiles, splits, ncb), lin_stage_bytes(ntok, cw));
      if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    }
    return hipSuccess;
  }
  const bool vec = a.k % 16u == 0u &&
                   ((reinterpret_cast<uintptr_t>(a.x) | reinterpret_cast<uintptr_t>(a.w)) & 15u) == 0u;
  if (a.m == 1u && vec && uint64_t(a.n) * a.k <= 0xFFFFFFFFull &&
      (a.k == 1024u || a.k == 2048u || a.k == 4096u || a.k == 8192u)) {
    switch (a.k) {
      case 1024u: launch_gemv_exact<8>(s, a); break;
      case 2048u: launch_gemv_exact<4>(s, a); break;
      case 4096u: launch_gemv_exact<2>(s, a); break;
      default: launch_gemv_exact<1>(s, a); break;
    }
    return hipGetLastError();
  }
  // tiled: whole groups, one token's partials within the workspace, and the
  // last tile's row offsets within 32 bits (rows past n read zeros)
  if (vec && a.k % kLinGroup == 0u && size_t(a.groups) * a.n * sizeof(float) <= kLinPartBytes &&
      uint64_t(a.n + kLTRows - 1) * a.k <= 0xFFFFFFFFull)
    return launch_exact_tiled(s, a, ws);
  if (a.m == 1) return launch_exact_mt<1>(s, a, vec);
  if (a.m == 2) return launch_exact_mt<2>(s, a, vec);
  if (a.m <= 4) return launch_exact_mt<4>(s, a, vec);
  return launch_exact_mt<8>(s, a, vec);
}

}  // namespace s14
