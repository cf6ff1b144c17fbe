// The EXACT row engine of the gfx950 kernels (device code shared by the
// kernel files): x/h staging into LDS and
// the decode window, lane-pair row chains in the reference CPU oracle's
// order (scheduler/ssd_inference/examples/s14_vulkan_numeric.rs:1669-1714:
// per row k strictly ascending, multiply then add, no FMA) for MXFP4 and FP8
// rows.  Everything sits in an unnamed namespace: each kernel file gets its
// own inline copy.
//
// A row is owned by a lane pair: in every group of 32 k the even lane forms
// the products of k 0..15 and the odd lane those of k 16..31; the running
// sum passes to the even lane, which adds its 16 products, then back to the
// odd lane, which adds its own 16, in k order (each hand-over a DPP
// quad_perm operand of v_add).
#pragma once

#include <hip/hip_runtime.h>

#include "s14_device.hpp"
#include "s14_device_util.hpp"
#include "s14_log1pf.h"

namespace s14 {
namespace {
// Biased-exponent range of the nonzero finite values seen by this lane.
__device__ __forceinline__ void exp_range_acc(float v, int &lo, int &hi) {
  const uint32_t u = __float_as_uint(v);
  const int e = int((u >> 23) & 255u);
  if ((u & 0x7fffffffu) != 0u && e != 255) {
    lo = min(lo, e);
    hi = max(hi, e);
  }
}

// Scale codes for which x * (e2m1 * 2^(c-127)) rounds exactly like the
// oracle's (x * e2m1) * 2^(c-127): both products stay normal and the scaled
// decode is exact.  With every nonzero finite x in [2^(emin-127),
// 2^(emax-126)): requires emin >= 2 (x*0.5 normal), emax <= 251 (x*6
// finite); then c in [max(2, 129 - emin), 252].  (Infinite or NaN x give
// the same inf/NaN either way.)  Batches holding other codes take the
// literal two-multiply path.
struct CodeWindow {
  int cmin, cmax;
};
__device__ __forceinline__ CodeWindow mx_window(int emin, int emax) {
  if (emin < 2 || emax > 251) return {256, 0};
  return {max(2, 129 - emin), 252};
}

// The copy alone, for vectors whose window is known (phase 2's h), in two
// steps so that other loads can go out while the copy's are in flight:
// stage_load_wave issues the calling wavefront's loads (lane-strided
// float4), stage_store_wave writes them to LDS.
template <int N, int S>
struct StageRegs {
  float4 v[S][N / 256];
};
template <int N, int S>
__device__ __forceinline__ void stage_load_wave(StageRegs<N, S> &r, const float *const (&src)[S]) {
  static_assert(N % 256 == 0, "whole float4 sweeps");
  const int lane = int(threadIdx.x & 63);
#pragma unroll
  for (int s = 0; s < S; ++s)
#pragma unroll
    for (int it = 0; it < N / 256; ++it) r.v[s][it] = *reinterpret_cast<const float4 *>(src[s] + it * 256 + lane * 4);
}
template <int N, int S>
__device__ __forceinline__ void stage_store_wave(float *const (&dst)[S], const StageRegs<N, S> &r) {
  const int lane = int(threadIdx.x & 63);
#pragma unroll
  for (int s = 0; s < S; ++s)
#pragma unroll
    for (int it = 0; it < N / 256; ++it) *reinterpret_cast<float4 *>(dst[s] + it * 256 + lane * 4) = r.v[s][it];
}

// Stage one vector of N f32 into LDS with the whole workgroup of NT threads
// (thread-strided float4) and return its exponent window to every thread;
// red: LDS scratch of 2 NT / 64 ints.  Ends with a barrier, after which the
// copy is visible to the workgroup.
template <int N, int NT>
__device__ __forceinline__ CodeWindow stage_x_block(float *dst, const float *__restrict__ src, int *red) {
  static_assert(N % (4 * NT) == 0 && NT % 64 == 0, "whole float4 sweeps");
  constexpr int IT = N / (4 * NT);
  constexpr int W = NT / 64;
  const int t = int(threadIdx.x);
  float4 v[IT];
#pragma unroll
  for (int it = 0; it < IT; ++it) v[it] = *reinterpret_cast<const float4 *>(src + (it * NT + t) * 4);
  int lo = 255, hi = 0;
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    *reinterpret_cast<float4 *>(dst + (it * NT + t) * 4) = v[it];
    exp_range_acc(v[it].x, lo, hi);
    exp_range_acc(v[it].y, lo, hi);
    exp_range_acc(v[it].z, lo, hi);
    exp_range_acc(v[it].w, lo, hi);
  }
  lo = wave_min_i(lo);
  hi = wave_max_i(hi);
  if ((t & 63) == 0) {
    red[2 * (t >> 6)] = lo;
    red[2 * (t >> 6) + 1] = hi;
  }
  __syncthreads();
#pragma unroll
  for (int w = 0; w < W; ++w) {
    lo = min(lo, red[2 * w]);
    hi = max(hi, red[2 * w + 1]);
  }
  return mx_window(lo, hi);
}

// Window of one pair's h from the exponent ranges its exact phase-1 tiles
// recorded (lo | hi << 16 per tile): the same range stage_x_block would find
// by scanning h.
constexpr int kP1Tiles = kInter / kP1ExactRows;
__device__ __forceinline__ CodeWindow h_window(const uint32_t *__restrict__ tiles) {
  static_assert(kP1Tiles == 128, "two tile words per lane");
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t a = tiles[lane], b = tiles[lane + 64];
  const int lo = min(int(a & 0xffffu), int(b & 0xffffu)), hi = max(int(a >> 16), int(b >> 16));
  return mx_window(wave_min_i(lo), wave_max_i(hi));
}

// Copy n f32 (n % 4 == 0) into LDS with the calling wavefront, eight float4
// loads in flight per lane.
__device__ __forceinline__ void stage_chunk_wave(float *dst, const float *__restrict__ src, uint32_t n) {
  const uint32_t lane = threadIdx.x & 63;
  uint32_t i = lane * 4;
  for (; i + 7 * 256 < n; i += 8 * 256) {
    float4 v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = *reinterpret_cast<const float4 *>(src + i + j * 256);
#pragma unroll
    for (int j = 0; j < 8; ++j) *reinterpret_cast<float4 *>(dst + i + j * 256) = v[j];
  }
  for (; i < n; i += 256) *reinterpret_cast<float4 *>(dst + i) = *reinterpret_cast<const float4 *>(src + i);
}

// ---------------------------------------------------------------------------
// EXACT row engine (lane pairs)
// ---------------------------------------------------------------------------

// The 16 x values of a lane's half-group, from LDS (two distinct addresses
// per wavefront: even and odd lanes).
struct X16 {
  float v[16];
};
__device__ __forceinline__ void load_x16(X16 &x, const float *__restrict__ xs) {
  const float4 *p = reinterpret_cast<const float4 *>(xs);
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const float4 q = p[d];
    x.v[4 * d + 0] = q.x;
    x.v[4 * d + 1] = q.y;
    x.v[4 * d + 2] = q.z;
    x.v[4 * d + 3] = q.w;
  }
}

// One group of a lane pair's row chain, in k order: the running sum, held by
// the odd lane between groups, passes to the even lane, which adds its 16
// products; it passes back to the odd lane, which adds its own 16.  Each
// hand-over is a DPP operand of the add that follows it (the other lane's
// adds in each half are discarded), so a group costs 32 adds of which only
// the two hand-overs read a just-written register across lanes and need
// wait states.  A row starts from 0 in both lanes and ends with from_odd.
__device__ __forceinline__ float pair_chain16(float acc, const float (&p)[16]) {
  acc = __fadd_rn(from_odd(acc), p[0]);
#pragma unroll
  for (int j = 1; j < 16; ++j) acc = __fadd_rn(acc, p[j]);
  acc = __fadd_rn(from_even(acc), p[0]);
#pragma unroll
  for (int j = 1; j < 16; ++j) acc = __fadd_rn(acc, p[j]);
  return acc;
}

// pair_chain16 over p with the next group's scaled products q = x * (e2m1
// * 2^(c-127)) (as mx_products_scaled forms them) in its gaps.  An add
// waits about 8 cycles for the one before it and issues in about 4.6, so
// an independent instruction between two adds costs no time; the
// compiler gathers such code into runs of its own whatever barriers stand
// between (its instruction selection orders arithmetic by data dependence
// only), so the group is one asm statement: one independent instruction
// before each add, two before each hand-over add (0 and 16, a DPP read of
// the sum the add before it has just written, which needs two wait
// states).  The eight converters (byte b of a code word chosen by op_sel)
// write three register pairs in turn, v[0:1], v[2:3] and v[4:5], named in
// the statement (an operand cannot name one half of a pair) and so listed
// as clobbered; each pair's two multiplies follow its converter a gap or
// more later.  sc: the converters' scale operand (2^(c-127); they read its
// exponent field only).  The statement ends on an add of acc, so a DPP
// read of acc by compiled code after it takes asm_chain_end first.
__device__ __forceinline__ float pair_chain16_asm(float acc, const float (&p)[16], float (&q)[16], uint2 w, float sc,
                                                  const X16 &x) {
#define S14_A(k) "v_add_f32 %[acc], %[acc], %[p" #k "]\n\t"
#define S14_AD(sel) "v_add_f32_dpp %[acc], %[acc], %[p0] quad_perm:" sel " row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
#define S14_C(t, w, sel) "v_cvt_scalef32_pk_f32_fp4 v[" t "], %[" #w "], %[sc]" sel "\n\t"
#define S14_M(k, r) "v_mul_f32 %[q" #k "], %[x" #k "], v" r "\n\t"
  asm volatile(
      // the even lane's half: the sum from the odd lane, then 16 products
      S14_C("0:1", wx, "") S14_C("2:3", wx, " op_sel:[1,0,0]") S14_AD("[1,1,3,3]")
      S14_C("4:5", wx, " op_sel:[0,1,0]") S14_A(1)
      S14_M(0, "0") S14_A(2)
      S14_M(1, "1") S14_A(3)
      S14_C("0:1", wx, " op_sel:[1,1,0]") S14_A(4)
      S14_M(2, "2") S14_A(5)
      S14_M(3, "3") S14_A(6)
      S14_C("2:3", wy, "") S14_A(7)
      S14_M(4, "4") S14_A(8)
      S14_M(5, "5") S14_A(9)
      S14_C("4:5", wy, " op_sel:[1,0,0]") S14_A(10)
      S14_M(6, "0") S14_A(11)
      S14_M(7, "1") S14_A(12)
      S14_C("0:1", wy, " op_sel:[0,1,0]") S14_A(13)
      S14_M(8, "2") S14_A(14)
      S14_M(9, "3") S14_A(15)
      // the odd lane's half: the sum from the even lane
      S14_C("2:3", wy, " op_sel:[1,1,0]") S14_M(10, "4") S14_AD("[0,0,2,2]")
      S14_M(11, "5") S14_A(1)
      S14_M(12, "0") S14_A(2)
      S14_M(13, "1") S14_A(3)
      S14_M(14, "2") S14_A(4)
      S14_M(15, "3") S14_A(5)
      S14_A(6) S14_A(7) S14_A(8) S14_A(9) S14_A(10) S14_A(11) S14_A(12) S14_A(13) S14_A(14) S14_A(15)
      : [acc] "+v"(acc), [q0] "=&v"(q[0]), [q1] "=&v"(q[1]), [q2] "=&v"(q[2]), [q3] "=&v"(q[3]),
        [q4] "=&v"(q[4]), [q5] "=&v"(q[5]), [q6] "=&v"(q[6]), [q7] "=&v"(q[7]), [q8] "=&v"(q[8]),
        [q9] "=&v"(q[9]), [q10] "=&v"(q[10]), [q11] "=&v"(q[11]), [q12] "=&v"(q[12]), [q13] "=&v"(q[13]),
        [q14] "=&v"(q[14]), [q15] "=&v"(q[15])
      : [p0] "v"(p[0]), [p1] "v"(p[1]), [p2] "v"(p[2]), [p3] "v"(p[3]), [p4] "v"(p[4]), [p5] "v"(p[5]),
        [p6] "v"(p[6]), [p7] "v"(p[7]), [p8] "v"(p[8]), [p9] "v"(p[9]), [p10] "v"(p[10]), [p11] "v"(p[11]),
        [p12] "v"(p[12]), [p13] "v"(p[13]), [p14] "v"(p[14]), [p15] "v"(p[15]), [x0] "v"(x.v[0]),
        [x1] "v"(x.v[1]), [x2] "v"(x.v[2]), [x3] "v"(x.v[3]), [x4] "v"(x.v[4]), [x5] "v"(x.v[5]),
        [x6] "v"(x.v[6]), [x7] "v"(x.v[7]), [x8] "v"(x.v[8]), [x9] "v"(x.v[9]), [x10] "v"(x.v[10]),
        [x11] "v"(x.v[11]), [x12] "v"(x.v[12]), [x13] "v"(x.v[13]), [x14] "v"(x.v[14]), [x15] "v"(x.v[15]),
        [wx] "v"(w.x), [wy] "v"(w.y), [sc] "v"(sc)
      : "v0", "v1", "v2", "v3", "v4", "v5");
#undef S14_A
#undef S14_AD
#undef S14_C
#undef S14_M
  return acc;
}
// Two wait states after an asm chain statement's last write of acc
// (pair_chain16_asm, fp8_quad_chain8_asm, mx_quad_chain8_asm), before
// compiled code reads it through DPP (acc passes through the statement, so
// that read cannot move above it).
__device__ __forceinline__ float asm_chain_end(float acc) {
  asm volatile("s_nop 1" : "+v"(acc));
  return acc;
}
// The converters' scale operand for byte j of scale word sw.
__device__ __forceinline__ float pair_scale_operand(uint32_t sw, int j) {
  return __uint_as_float(j < 3 ? sw << (23 - 8 * j) : sw >> 1);
}

// MXFP4 products of the lane's 8 code bytes (16 k, low nibble first).
// Scaled: p = x * (e2m1 * 2^(c-127)) via the gfx950 scaled converter — equal
// to the oracle's (x * e2m1) * 2^(c-127) for codes inside the window.
__device__ __forceinline__ void mx_products_scaled(float (&p)[16], uint2 w, uint32_t c, const X16 &x) {
  const float sc = __uint_as_float(c << 23);
  const uint32_t words[2] = {w.x, w.y};
#pragma unroll
  for (int d = 0; d < 2; ++d) {
    const v2f q[4] = {__builtin_amdgcn_cvt_scalef32_pk_f32_fp4(words[d], sc, 0),
                      __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(words[d], sc, 1),
                      __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(words[d], sc, 2),
                      __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(words[d], sc, 3)};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      p[8 * d + 2 * s] = __fmul_rn(x.v[8 * d + 2 * s], q[s].x);
      p[8 * d + 2 * s + 1] = __fmul_rn(x.v[8 * d + 2 * s + 1], q[s].y);
    }
  }
}
// Literal: p = (x * e2m1) * ue8m0(c), any code.
__device__ __forceinline__ void mx_products_literal(float (&p)[16], uint2 w, uint32_t c, const X16 &x) {
  const float s = ue8m0_f32(c);
  const uint32_t words[2] = {w.x, w.y};
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const float e = e2m1_f32((words[j >> 3] >> (4 * (j & 7))) & 15u);
    p[j] = __fmul_rn(__fmul_rn(x.v[j], e), s);
  }
}

template <int PF>
struct MxBatch {
  uint2 w[PF];
  uint32_t c[PF / 4];
};

// Codes of groups [g0, g0+PF): the lane's 8 bytes at woff + 16 g (woff
// includes the lane's half-group offset), scale codes at soff + g.  Loads
// past a row's end read neighbouring bytes or, past num_records, zeros;
// such values are never consumed.
template <int PF>
__device__ __forceinline__ void mx_load(MxBatch<PF> &b, const Src1 &src, uint32_t woff, uint32_t soff, int g0) {
#pragma unroll
  for (int i = 0; i < PF; ++i) b.w[i] = ld8(src.w, woff + 16u * uint32_t(g0 + i));
#pragma unroll
  for (int j = 0; j < PF / 4; ++j) b.c[j] = ld4(src.s, soff + uint32_t(g0) + 4u * j);
}
template <int PF>
__device__ __forceinline__ void mx_load(MxBatch<PF> &b, const Src2 &src, uint32_t woff, uint32_t soff, int g0) {
  if (src.hi)
    mx_load<PF>(b, Src1{src.b, src.b}, woff, soff, g0);
  else
    mx_load<PF>(b, Src1{src.a, src.a}, woff, soff, g0);
}

template <int PF>
__device__ __forceinline__ void mx_load(MxBatch<PF> &b, const SrcP &src, uint32_t woff, uint32_t soff, int g0) {
#pragma unroll
  for (int i = 0; i < PF; ++i) b.w[i] = gld8(src.p + woff + 16u * uint32_t(g0 + i));
#pragma unroll
  for (int j = 0; j < PF / 4; ++j) b.c[j] = gld4(src.p + soff + uint32_t(g0) + 4u * j);
}

__device__ __forceinline__ bool codes_in(uint32_t word, CodeWindow win) {
  bool ok = true;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = int((word >> (8 * i)) & 255u);
    ok = ok && c >= win.cmin && c <= win.cmax;
  }
  return ok;
}

template <int PF>
__device__ __forceinline__ uint32_t batch_code(const MxBatch<PF> &b, int i) {
  return (b.c[i >> 2] >> (8 * (i & 3))) & 255u;
}

// Single loads through either source form (the literal path re-reads its
// codes rather than index the register batch dynamically).
__device__ __forceinline__ uint2 src_ld8(const Src1 &s, uint32_t off) { return ld8(s.w, off); }
__device__ __forceinline__ uint32_t src_ld1(const Src1 &s, uint32_t off) { return ld1(s.s, off); }
__device__ __forceinline__ uint2 src_ld8(const Src2 &s, uint32_t off) {
  uint2 v;
  if (s.hi)
    v = ld8(s.b, off);
  else
    v = ld8(s.a, off);
  return v;
}
__device__ __forceinline__ uint2 src_ld8(const SrcP &s, uint32_t off) { return gld8(s.p + off); }
__device__ __forceinline__ uint32_t src_ld1(const SrcP &s, uint32_t off) { return s.p[off]; }
__device__ __forceinline__ uint32_t src_ld1(const Src2 &s, uint32_t off) {
  uint32_t v;
  if (s.hi)
    v = ld1(s.b, off);
  else
    v = ld1(s.a, off);
  return v;
}

// The scale codes of a lane pair's row, split between its lanes (the even
// lane holds groups [0, G/2), the odd lane [G/2, G)), loaded ahead of the
// row so that one check decides the decode of the whole row.
template <int G>
struct RowCodes {
  uint4 v[G / 32];
};
template <int G>
__device__ __forceinline__ void load_row_codes(RowCodes<G> &rc, const Src1 &src, uint32_t soff) {
  const uint32_t base = soff + (threadIdx.x & 1u) * uint32_t(G / 2);
#pragma unroll
  for (int i = 0; i < G / 32; ++i) rc.v[i] = ld16(src.s, base + 16u * i);
}
template <int G>
__device__ __forceinline__ void load_row_codes(RowCodes<G> &rc, const SrcP &src, uint32_t soff) {
  const uint32_t base = soff + (threadIdx.x & 1u) * uint32_t(G / 2);
#pragma unroll
  for (int i = 0; i < G / 32; ++i) {
    const v4u v = *(const __attribute__((address_space(1))) v4u *)(src.p + base + 16u * i);
    rc.v[i] = make_uint4(v.x, v.y, v.z, v.w);
  }
}

// True (in every lane) when every scale code of every row of the wavefront
// lies in its lane's window: byte minimum and maximum through packed 16-bit
// min/max of the even and odd bytes.
template <int G>
__device__ __forceinline__ bool row_codes_in(const RowCodes<G> &rc, CodeWindow win) {
  typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
  u16x2 mn = {255, 255}, mx = {0, 0};
#pragma unroll
  for (int i = 0; i < G / 32; ++i) {
    const uint32_t w[4] = {rc.v[i].x, rc.v[i].y, rc.v[i].z, rc.v[i].w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const u16x2 lo = __builtin_bit_cast(u16x2, w[j] & 0x00ff00ffu);
      const u16x2 hi = __builtin_bit_cast(u16x2, (w[j] >> 8) & 0x00ff00ffu);
      mn = __builtin_elementwise_min(mn, __builtin_elementwise_min(lo, hi));
      mx = __builtin_elementwise_max(mx, __builtin_elementwise_max(lo, hi));
    }
  }
  const int cmin = min(int(mn.x), int(mn.y)), cmax = max(int(mx.x), int(mx.y));
  const bool ok = cmin >= win.cmin && cmax <= win.cmax;
  return __builtin_amdgcn_ballot_w64(!ok) == 0;
}

// One batch: if every lane's codes are inside its window the batch runs the
// scaled decode as straight-line code, software-pipelined: group i+1's x
// reads and products are issued ahead of group i's add chain, so LDS latency
// and the chain's DPP read-after-write waits overlap independent work.
// Otherwise the batch takes the literal decode, group by group, re-reading
// its codes (compact code for a path real scale codes do not take).
template <int PF, bool kCheck = true, class Src>
__device__ __forceinline__ float mx_consume(float acc, const MxBatch<PF> &b, const Src &src, uint32_t woff,
                                            uint32_t soff, const float *__restrict__ xh, int g0, CodeWindow win) {
  bool ok = true;
  if constexpr (kCheck) {
#pragma unroll
    for (int j = 0; j < PF / 4; ++j) ok = ok && codes_in(b.c[j], win);
  }
  if constexpr (!kCheck) {
    // the row's codes were checked once: each group's chain interleaved
    // with the next group's products (pair_chain16_asm)
    X16 xa, xb;
    float p[16], q[16];
    load_x16(xa, xh + g0 * 32);
    load_x16(xb, xh + (g0 + 1) * 32);
    mx_products_scaled(p, b.w[0], batch_code(b, 0), xa);
#pragma unroll
    for (int i = 0; i < PF; i += 2) {
      if (i + 2 < PF) load_x16(xa, xh + (g0 + i + 2) * 32);
      acc = pair_chain16_asm(acc, p, q, b.w[i + 1], pair_scale_operand(b.c[(i + 1) >> 2], (i + 1) & 3), xb);
      if (i + 3 < PF) load_x16(xb, xh + (g0 + i + 3) * 32);
      if (i + 2 < PF) {
        acc = pair_chain16_asm(acc, q, p, b.w[i + 2], pair_scale_operand(b.c[(i + 2) >> 2], (i + 2) & 3), xa);
      } else {
        acc = pair_chain16(asm_chain_end(acc), q);
      }
    }
  } else if (__builtin_amdgcn_ballot_w64(!ok) == 0) {
    X16 xa, xb;
    float p[16], q[16];
    load_x16(xa, xh + g0 * 32);
    load_x16(xb, xh + (g0 + 1) * 32);
    mx_products_scaled(p, b.w[0], batch_code(b, 0), xa);
#pragma unroll
    for (int i = 0; i < PF; i += 2) {
      // p holds group i's products; xb holds group i+1's x
      if (i + 2 < PF) load_x16(xa, xh + (g0 + i + 2) * 32);
      mx_products_scaled(q, b.w[i + 1], batch_code(b, i + 1), xb);
      acc = pair_chain16(acc, p);
      if (i + 3 < PF) load_x16(xb, xh + (g0 + i + 3) * 32);
      if (i + 2 < PF) mx_products_scaled(p, b.w[i + 2], batch_code(b, i + 2), xa);
      acc = pair_chain16(acc, q);
    }
  } else {
#pragma unroll 1
    for (int g = g0; g < g0 + PF; ++g) {
      float p[16];
      X16 x;
      load_x16(x, xh + g * 32);
      mx_products_literal(p, src_ld8(src, woff + 16u * uint32_t(g)), src_ld1(src, soff + uint32_t(g)), x);
      acc = pair_chain16(acc, p);
    }
  }
  return acc;
}

// Dot of one MXFP4 row of G groups (G % PF == 0) with x in LDS (xh = x +
// 16 * (lane & 1)); result in both lanes.  `ba` arrives holding groups
// [0, PF) (loaded by the caller with mx_load, ahead of its own set-up work);
// two register batches of PF groups then ping-pong so that batch b+1 is in
// flight while batch b is consumed.  (The loop prefetches one batch past
// the row's end: neighbouring bytes or zeros, never consumed.)
template <int PF, class Src>
__device__ __forceinline__ float mx_row_pair(float acc, MxBatch<PF> &ba, const Src &src, uint32_t woff,
                                             uint32_t soff, int G, const float *__restrict__ xh, CodeWindow win) {
  static_assert(PF % 4 == 0, "scale words hold 4 codes");
  MxBatch<PF> bb;
  int g0 = 0;
  for (; g0 + 2 * PF <= G; g0 += 2 * PF) {
    mx_load<PF>(bb, src, woff, soff, g0 + PF);
    acc = mx_consume<PF>(acc, ba, src, woff, soff, xh, g0, win);
    mx_load<PF>(ba, src, woff, soff, g0 + 2 * PF);
    acc = mx_consume<PF>(acc, bb, src, woff, soff, xh, g0 + PF, win);
  }
  if (g0 < G) acc = mx_consume<PF>(acc, ba, src, woff, soff, xh, g0, win);  // one batch left
  return from_odd(acc);
}

// The same for a compile-time group count G (G % (2 PF) == 0), with the
// last two batches peeled so that no load reaches past the row (decode
// chosen batch by batch).
template <int PF, int G, class Src>
__device__ __forceinline__ float mx_row_pair_fixed(float acc, MxBatch<PF> &ba, const Src &src, uint32_t woff,
                                                   uint32_t soff, const float *__restrict__ xh, CodeWindow win) {
  static_assert(PF % 4 == 0 && G % (2 * PF) == 0, "whole batch pairs");
  MxBatch<PF> bb;
#pragma unroll 1
  for (int g0 = 0; g0 < G - 2 * PF; g0 += 2 * PF) {
    mx_load<PF>(bb, src, woff, soff, g0 + PF);
    acc = mx_consume<PF>(acc, ba, src, woff, soff, xh, g0, win);
    mx_load<PF>(ba, src, woff, soff, g0 + 2 * PF);
    acc = mx_consume<PF>(acc, bb, src, woff, soff, xh, g0 + PF, win);
  }
  mx_load<PF>(bb, src, woff, soff, G - PF);
  acc = mx_consume<PF>(acc, ba, src, woff, soff, xh, G - 2 * PF, win);
  acc = mx_consume<PF>(acc, bb, src, woff, soff, xh, G - PF, win);
  return from_odd(acc);
}

// The same with the decode chosen once for the whole row from its codes (rc,
// loaded by the caller with load_row_codes): the scaled batches with no
// per-batch check, or the literal decode group by group.
template <int PF, int G, class Src>
__device__ __forceinline__ float mx_row_pair_fixed(float acc, MxBatch<PF> &ba, const Src &src, uint32_t woff,
                                                   uint32_t soff, const float *__restrict__ xh, CodeWindow win,
                                                   const RowCodes<G> &rc) {
  static_assert(PF % 4 == 0 && G % (2 * PF) == 0, "whole batch pairs");
  if (row_codes_in<G>(rc, win)) {
    MxBatch<PF> bb;
#pragma unroll 1
    for (int g0 = 0; g0 < G - 2 * PF; g0 += 2 * PF) {
      mx_load<PF>(bb, src, woff, soff, g0 + PF);
      acc = mx_consume<PF, false>(acc, ba, src, woff, soff, xh, g0, win);
      mx_load<PF>(ba, src, woff, soff, g0 + 2 * PF);
      acc = mx_consume<PF, false>(acc, bb, src, woff, soff, xh, g0 + PF, win);
    }
    mx_load<PF>(bb, src, woff, soff, G - PF);
    acc = mx_consume<PF, false>(acc, ba, src, woff, soff, xh, G - 2 * PF, win);
    acc = mx_consume<PF, false>(acc, bb, src, woff, soff, xh, G - PF, win);
  } else {
#pragma unroll 1
    for (int g = 0; g < G; ++g) {
      float p[16];
      X16 x;
      load_x16(x, xh + g * 32);
      mx_products_literal(p, src_ld8(src, woff + 16u * uint32_t(g)), src_ld1(src, soff + uint32_t(g)), x);
      acc = pair_chain16(acc, p);
    }
  }
  return from_odd(acc);
}

// FP8 products of the lane's 16 code bytes: p = (x * e4m3) * s
// (s14_vulkan_numeric.rs:1698-1714).
__device__ __forceinline__ void fp8_products(float (&p)[16], uint4 w, float s, const X16 &x) {
  const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const v2f lo = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(words[d], 1.0f, false);
    const v2f hi = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(words[d], 1.0f, true);
    p[4 * d + 0] = __fmul_rn(__fmul_rn(x.v[4 * d + 0], lo.x), s);
    p[4 * d + 1] = __fmul_rn(__fmul_rn(x.v[4 * d + 1], lo.y), s);
    p[4 * d + 2] = __fmul_rn(__fmul_rn(x.v[4 * d + 2], hi.x), s);
    p[4 * d + 3] = __fmul_rn(__fmul_rn(x.v[4 * d + 3], hi.y), s);
  }
}

// FP8 batch: 4 groups of 32 k (one 128-wide scale tile when g0 % 4 == 0).
struct Fp8Batch {
  uint4 w[4];
  float s;
};
__device__ __forceinline__ float fp8_scale(Rsrc r, uint32_t soff, uint32_t tile, int scale_f32) {
  return scale_f32 ? ldf(r, soff + 4u * tile) : ue8m0_f32(ld1(r, soff + tile));
}
__device__ __forceinline__ void fp8_load(Fp8Batch &b, const Src1 &src, uint32_t woff, uint32_t soff, int scale_f32,
                                         int g0) {
#pragma unroll
  for (int i = 0; i < 4; ++i) b.w[i] = ld16(src.w, woff + 32u * uint32_t(g0 + i));
  b.s = fp8_scale(src.s, soff, uint32_t(g0) / 4u, scale_f32);
}
__device__ __forceinline__ void fp8_load(Fp8Batch &b, const Src2 &src, uint32_t woff, uint32_t soff, int scale_f32,
                                         int g0) {
  if (src.hi)
    fp8_load(b, Src1{src.b, src.b}, woff, soff, scale_f32, g0);
  else
    fp8_load(b, Src1{src.a, src.a}, woff, soff, scale_f32, g0);
}
// Four groups, pipelined like mx_consume.
__device__ __forceinline__ float fp8_consume(float acc, const Fp8Batch &b, const float *__restrict__ xh, int g0) {
  X16 xa, xb;
  float p[16], q[16];
  load_x16(xa, xh + g0 * 32);
  load_x16(xb, xh + (g0 + 1) * 32);
  fp8_products(p, b.w[0], b.s, xa);
#pragma unroll
  for (int i = 0; i < 4; i += 2) {
    if (i + 2 < 4) load_x16(xa, xh + (g0 + i + 2) * 32);
    fp8_products(q, b.w[i + 1], b.s, xb);
    acc = pair_chain16(acc, p);
    if (i + 3 < 4) load_x16(xb, xh + (g0 + i + 3) * 32);
    if (i + 2 < 4) fp8_products(p, b.w[i + 2], b.s, xa);
    acc = pair_chain16(acc, q);
  }
  return acc;
}

// Dot of one FP8 row of G groups of 32 k with x in LDS (woff includes the
// lane's 16-byte half-group offset; soff is the byte offset of the row's
// first tile scale); result in both lanes.
template <class Src>
__device__ __forceinline__ float fp8_row_pair(float acc, const Src &src, uint32_t woff, uint32_t soff,
                                              int scale_f32, int G, const float *__restrict__ xh) {
  const int G4 = G & ~3;
  Fp8Batch ba, bb;
  fp8_load(ba, src, woff, soff, scale_f32, 0);
  int g0 = 0;
  for (; g0 + 8 <= G4; g0 += 8) {
    fp8_load(bb, src, woff, soff, scale_f32, g0 + 4);
    acc = fp8_consume(acc, ba, xh, g0);
    fp8_load(ba, src, woff, soff, scale_f32, g0 + 8);
    acc = fp8_consume(acc, bb, xh, g0 + 4);
  }
  if (g0 < G4) {
    acc = fp8_consume(acc, ba, xh, g0);
    g0 += 4;
  }
  for (; g0 < G; ++g0) {  // groups of a last partial tile
    Fp8Batch t;
    fp8_load(t, src, woff, soff, scale_f32, g0);  // loads 4 groups, uses one
    float p[16];
    X16 x;
    load_x16(x, xh + g0 * 32);
    fp8_products(p, t.w[0], t.s, x);
    acc = pair_chain16(acc, p);
  }
  return from_odd(acc);
}

// The same row with NB batches (4 NB groups) in flight instead of one: for
// launches with few wavefronts (the standalone matvec at N = 1024 runs 32),
// where one batch ahead leaves every wavefront waiting a load latency per
// batch.  G % (4 NB) == 0; same products and order as fp8_row_pair.
template <int NB>
__device__ __forceinline__ float fp8_row_pair_deep(float acc, const Src1 &src, uint32_t woff, uint32_t soff,
                                                   int scale_f32, int G, const float *__restrict__ xh) {
  Fp8Batch b[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) fp8_load(b[j], src, woff, soff, scale_f32, 4 * j);
  for (int g0 = 0; g0 < G; g0 += 4 * NB) {
    const bool refill = g0 + 4 * NB < G;  // uniform
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      acc = fp8_consume(acc, b[j], xh, g0 + 4 * j);
      if (refill) fp8_load(b[j], src, woff, soff, scale_f32, g0 + 4 * NB + 4 * j);
    }
  }
  return from_odd(acc);
}

// ---------------------------------------------------------------------------
// Lane quads, for launches with few rows (the standalone FP8 matvec at
// N = 1024 has 1,024 row chains for 1,024 SIMDs): each row is owned by four
// lanes, lane q forming the products of k 8q..8q+7 of every 32-k group, and
// the running sum goes round the quad, lane q taking it from lane q - 1 (a
// quad_perm DPP operand of its first add of the step).  A group is four
// steps of 8 adds, each add the running sum plus one product in k order;
// in step s only lane s's adds are kept.  Twice the lanes of a pair, so
// half the wavefront instruction stream per row (fewer products per lane).
// ---------------------------------------------------------------------------

// Value of the previous lane of each quad, lane 0 taking lane 3's
// (quad_perm [3,0,1,2]).
__device__ __forceinline__ float from_prev_in_quad(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x93, 0xf, 0xf, true));
}
// Value of lane 3 of each quad (quad_perm [3,3,3,3]).
__device__ __forceinline__ float from_quad_last(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xFF, 0xf, 0xf, true));
}
__device__ __forceinline__ float quad_chain8(float acc, const float (&p)[8]) {
#pragma unroll
  for (int step = 0; step < 4; ++step) {
    acc = __fadd_rn(from_prev_in_quad(acc), p[0]);
#pragma unroll
    for (int j = 1; j < 8; ++j) acc = __fadd_rn(acc, p[j]);
  }
  return acc;
}
// FP8 products of the lane's 8 code bytes: p = (x * e4m3) * s.
__device__ __forceinline__ void fp8_products8(float (&p)[8], uint2 w, float s, const float *__restrict__ x) {
  const float4 xa = *reinterpret_cast<const float4 *>(x), xb = *reinterpret_cast<const float4 *>(x + 4);
  const float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
  const uint32_t words[2] = {w.x, w.y};
#pragma unroll
  for (int d = 0; d < 2; ++d) {
    const v2f lo = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(words[d], 1.0f, false);
    const v2f hi = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(words[d], 1.0f, true);
    p[4 * d + 0] = __fmul_rn(__fmul_rn(xv[4 * d + 0], lo.x), s);
    p[4 * d + 1] = __fmul_rn(__fmul_rn(xv[4 * d + 1], lo.y), s);
    p[4 * d + 2] = __fmul_rn(__fmul_rn(xv[4 * d + 2], hi.x), s);
    p[4 * d + 3] = __fmul_rn(__fmul_rn(xv[4 * d + 3], hi.y), s);
  }
}
// Four groups of a quad lane's codes (one 128-wide scale tile).
struct Fp8QBatch {
  uint2 w[4];
  float s;
};
__device__ __forceinline__ void fp8q_load(Fp8QBatch &b, Rsrc w, Rsrc sc, uint32_t woff, uint32_t soff, int scale_f32,
                                          int g0) {
#pragma unroll
  for (int i = 0; i < 4; ++i) b.w[i] = ld8(w, woff + 32u * uint32_t(g0 + i));
  b.s = fp8_scale(sc, soff, uint32_t(g0) / 4u, scale_f32);
}
// quad_chain8 over p with the next group's FP8 products q = (x * e4m3) * s
// formed in its gaps, written as one asm statement because the compiler
// gathers such code into runs of its own whatever barriers stand between
// (its instruction selection orders arithmetic by data dependence only):
// each of the 32 dependent adds leaves room for one independent
// instruction, and each hand-over add (0, 8, 16, 24: a DPP read of the sum
// that the add before it has just written, which needs two wait states)
// gets two (or, once the independent work runs out, two wait states).
// Gap schedule: the four conversions (two codes each, the word's low or
// high half chosen by op_sel) write three register pairs in turn, v[0:1],
// v[2:3] and v[4:5], named in the statement (an operand cannot name one
// half of a pair) and so listed as clobbered; then the x products, then
// the scalings, each at least one gap after what it reads.  The statement
// ends on an add of acc, so a DPP read of acc by compiled code after it
// takes asm_chain_end first.
__device__ __forceinline__ float fp8_quad_chain8_asm(float acc, const float (&p)[8], float (&q)[8], uint2 w, float s,
                                                     const float (&xv)[8]) {
#define S14_DPP "quad_perm:[3,0,1,2] row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
#define S14_A(k) "v_add_f32 %[acc], %[acc], %[p" #k "]\n\t"
#define S14_AD "v_add_f32_dpp %[acc], %[acc], %[p0] " S14_DPP
#define S14_C(t, w, sel) "v_cvt_scalef32_pk_f32_fp8 v[" t "], %[" #w "], 1.0" sel "\n\t"
#define S14_M(k, r) "v_mul_f32 %[q" #k "], %[x" #k "], v" r "\n\t"
#define S14_S(k) "v_mul_f32 %[q" #k "], %[q" #k "], %[s]\n\t"
  asm volatile(
      // step 0
      S14_C("0:1", wx, "") S14_C("2:3", wx, " op_sel:[1,0,0]") S14_AD
      S14_C("4:5", wy, "") S14_A(1)
      S14_M(0, "0") S14_A(2)
      S14_M(1, "1") S14_A(3)
      S14_C("0:1", wy, " op_sel:[1,0,0]") S14_A(4)
      S14_M(2, "2") S14_A(5)
      S14_M(3, "3") S14_A(6)
      S14_M(4, "4") S14_A(7)
      // step 1
      S14_M(5, "5") S14_M(6, "0") S14_AD
      S14_M(7, "1") S14_A(1)
      S14_S(0) S14_A(2)
      S14_S(1) S14_A(3)
      S14_S(2) S14_A(4)
      S14_S(3) S14_A(5)
      S14_S(4) S14_A(6)
      S14_S(5) S14_A(7)
      // step 2
      S14_S(6) S14_S(7) S14_AD
      S14_A(1) S14_A(2) S14_A(3) S14_A(4) S14_A(5) S14_A(6) S14_A(7)
      // step 3
      "s_nop 1\n\t" S14_AD
      S14_A(1) S14_A(2) S14_A(3) S14_A(4) S14_A(5) S14_A(6) S14_A(7)
      : [acc] "+v"(acc), [q0] "=&v"(q[0]), [q1] "=&v"(q[1]), [q2] "=&v"(q[2]), [q3] "=&v"(q[3]),
        [q4] "=&v"(q[4]), [q5] "=&v"(q[5]), [q6] "=&v"(q[6]), [q7] "=&v"(q[7])
      : [p0] "v"(p[0]), [p1] "v"(p[1]), [p2] "v"(p[2]), [p3] "v"(p[3]), [p4] "v"(p[4]), [p5] "v"(p[5]),
        [p6] "v"(p[6]), [p7] "v"(p[7]), [x0] "v"(xv[0]), [x1] "v"(xv[1]), [x2] "v"(xv[2]), [x3] "v"(xv[3]),
        [x4] "v"(xv[4]), [x5] "v"(xv[5]), [x6] "v"(xv[6]), [x7] "v"(xv[7]), [wx] "v"(w.x), [wy] "v"(w.y),
        [s] "v"(s)
      : "v0", "v1", "v2", "v3", "v4", "v5");
#undef S14_DPP
#undef S14_A
#undef S14_AD
#undef S14_C
#undef S14_M
#undef S14_S
  return acc;
}
// x of one group for a quad lane (8 values from LDS).
__device__ __forceinline__ void quad_x8(float (&xv)[8], const float *__restrict__ x) {
  const float4 xa = *reinterpret_cast<const float4 *>(x), xb = *reinterpret_cast<const float4 *>(x + 4);
  xv[0] = xa.x, xv[1] = xa.y, xv[2] = xa.z, xv[3] = xa.w, xv[4] = xb.x, xv[5] = xb.y, xv[6] = xb.z, xv[7] = xb.w;
}
// Dot of one FP8 row of G groups (G % (4 NB) == 0) with x in LDS (xq = x +
// 8 q); NB batches in flight.  Result in every lane of the quad.
template <int NB>
__device__ __forceinline__ float fp8_row_quad(Rsrc w, Rsrc sc, uint32_t woff, uint32_t soff, int scale_f32, int G,
                                              const float *__restrict__ xq) {
  Fp8QBatch b[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) fp8q_load(b[j], w, sc, woff, soff, scale_f32, 4 * j);
  float acc = 0.0f;
  for (int g0 = 0; g0 < G; g0 += 4 * NB) {
    const bool refill = g0 + 4 * NB < G;  // uniform
    // software-pipelined: group n+1's products formed in the gaps of group
    // n's chain, from x read from LDS a group before that
    float pc[8], pn[8], xn[8];
    fp8_products8(pc, b[0].w[0], b[0].s, xq + 32 * g0);
    quad_x8(xn, xq + 32 * (g0 + 1));
#pragma unroll
    for (int n = 0; n < 4 * NB; ++n) {
      const int j = n / 4, i = n % 4;
      if (n + 1 < 4 * NB) {
        const int jn = (n + 1) / 4, in = (n + 1) % 4;
        float xa[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) xa[k] = xn[k];
        if (n + 2 < 4 * NB) quad_x8(xn, xq + 32 * (g0 + n + 2));
        acc = fp8_quad_chain8_asm(acc, pc, pn, b[jn].w[in], b[jn].s, xa);
        if (n + 2 == 4 * NB) acc = asm_chain_end(acc);
      } else {
        acc = quad_chain8(acc, pc);
      }
      if (i == 3 && refill) fp8q_load(b[j], w, sc, woff, soff, scale_f32, g0 + 4 * NB + 4 * j);
#pragma unroll
      for (int k = 0; k < 8; ++k) pc[k] = pn[k];
    }
  }
  return from_quad_last(acc);
}

// MXFP4 rows by lane quads (the single-expert chain, whose 4,096 + 4,096
// phase-1 rows and 4,096 phase-2 rows leave most SIMDs idle with lane
// pairs): lane q of each quad holds the 4 code bytes of k 8q .. 8q+7 of
// every 32-k group (woff includes 4 q) and the group's scale code; xq = x +
// 8 q.  Products as the pair engine's: scaled (one converter step per two
// codes, then x times the decoded value) when every code of the
// wavefront's rows is inside the window, else literal ((x * e2m1) * s).
struct MxQBatch {
  uint32_t w[4];  // groups g0 .. g0+3
  uint32_t c;     // their scale codes, one byte each
};
__device__ __forceinline__ void mxq_load(MxQBatch &b, Rsrc r, uint32_t woff, uint32_t soff, int g0) {
#pragma unroll
  for (int i = 0; i < 4; ++i) b.w[i] = ld4(r, woff + 16u * uint32_t(g0 + i));
  b.c = ld4(r, soff + uint32_t(g0));
}
template <bool kScaled>
__device__ __forceinline__ void mx_products8(float (&p)[8], uint32_t w, uint32_t c, const float *__restrict__ x) {
  const float4 xa = *reinterpret_cast<const float4 *>(x), xb = *reinterpret_cast<const float4 *>(x + 4);
  const float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
  if constexpr (kScaled) {
    const float sc = __uint_as_float(c << 23);
    const v2f q[4] = {__builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, sc, 0),
                      __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, sc, 1),
                      __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, sc, 2),
                      __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, sc, 3)};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      p[2 * s] = __fmul_rn(xv[2 * s], q[s].x);
      p[2 * s + 1] = __fmul_rn(xv[2 * s + 1], q[s].y);
    }
  } else {
    const float s = ue8m0_f32(c);
#pragma unroll
    for (int j = 0; j < 8; ++j) p[j] = __fmul_rn(__fmul_rn(xv[j], e2m1_f32((w >> (4 * j)) & 15u)), s);
  }
}
// A quad lane's share of its row's G scale codes (lane q: bytes G/4 q ..
// G/4 q + G/4 - 1), loaded ahead so that one check decides the decode of
// the whole row; quad_codes_in is true (in every lane) when every code of
// every row of the wavefront lies in the window.
template <int G>
struct QuadCodes {
  static_assert(G == 128 || G == 64, "a quad lane holds 32 or 16 codes");
  uint4 v[G / 64];
};
template <int G>
__device__ __forceinline__ void load_quad_codes(QuadCodes<G> &qc, Rsrc r, uint32_t soff_row) {
  const uint32_t q = threadIdx.x & 3u;
#pragma unroll
  for (int i = 0; i < G / 64; ++i) qc.v[i] = ld16(r, soff_row + uint32_t(G / 4) * q + 16u * uint32_t(i));
}
template <int G>
__device__ __forceinline__ bool quad_codes_in(const QuadCodes<G> &qc, CodeWindow win) {
  typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
  u16x2 mn = {255, 255}, mx = {0, 0};
#pragma unroll
  for (int i = 0; i < G / 64; ++i) {
    const uint32_t w[4] = {qc.v[i].x, qc.v[i].y, qc.v[i].z, qc.v[i].w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const u16x2 lo = __builtin_bit_cast(u16x2, w[j] & 0x00ff00ffu);
      const u16x2 hi = __builtin_bit_cast(u16x2, (w[j] >> 8) & 0x00ff00ffu);
      mn = __builtin_elementwise_min(mn, __builtin_elementwise_min(lo, hi));
      mx = __builtin_elementwise_max(mx, __builtin_elementwise_max(lo, hi));
    }
  }
  const bool ok = int(min(mn.x, mn.y)) >= win.cmin && int(max(mx.x, mx.y)) <= win.cmax;
  return __builtin_amdgcn_ballot_w64(!ok) == 0;
}
// quad_chain8 over p with the next group's scaled products q = x * (e2m1 *
// 2^(c-127)) (as mx_products8 forms them) in its gaps, one asm statement
// as pair_chain16_asm: the four converters write v[0:1], v[2:3] and
// v[4:5] in turn (clobbered), each pair's multiplies a gap or more later;
// each hand-over add gets two independent instructions before it, or,
// once those run out, two wait states.  sc: the converters' scale operand;
// xv: that group's x.  Ends on an add of acc (asm_chain_end before a DPP
// read by compiled code).
__device__ __forceinline__ float mx_quad_chain8_asm(float acc, const float (&p)[8], float (&q)[8], uint32_t w,
                                                    float sc, const float (&xv)[8]) {
#define S14_A(k) "v_add_f32 %[acc], %[acc], %[p" #k "]\n\t"
#define S14_AD "v_add_f32_dpp %[acc], %[acc], %[p0] quad_perm:[3,0,1,2] row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
#define S14_C(t, sel) "v_cvt_scalef32_pk_f32_fp4 v[" t "], %[w], %[sc]" sel "\n\t"
#define S14_M(k, r) "v_mul_f32 %[q" #k "], %[x" #k "], v" r "\n\t"
  asm volatile(
      // step 0
      S14_C("0:1", "") S14_C("2:3", " op_sel:[1,0,0]") S14_AD
      S14_C("4:5", " op_sel:[0,1,0]") S14_A(1)
      S14_M(0, "0") S14_A(2)
      S14_M(1, "1") S14_A(3)
      S14_C("0:1", " op_sel:[1,1,0]") S14_A(4)
      S14_M(2, "2") S14_A(5)
      S14_A(6) S14_A(7)
      // step 1
      S14_M(3, "3") S14_M(4, "4") S14_AD
      S14_M(5, "5") S14_A(1)
      S14_A(2) S14_A(3) S14_A(4) S14_A(5) S14_A(6) S14_A(7)
      // step 2
      S14_M(6, "0") S14_M(7, "1") S14_AD
      S14_A(1) S14_A(2) S14_A(3) S14_A(4) S14_A(5) S14_A(6) S14_A(7)
      // step 3
      "s_nop 1\n\t" S14_AD
      S14_A(1) S14_A(2) S14_A(3) S14_A(4) S14_A(5) S14_A(6) S14_A(7)
      : [acc] "+v"(acc), [q0] "=&v"(q[0]), [q1] "=&v"(q[1]), [q2] "=&v"(q[2]), [q3] "=&v"(q[3]),
        [q4] "=&v"(q[4]), [q5] "=&v"(q[5]), [q6] "=&v"(q[6]), [q7] "=&v"(q[7])
      : [p0] "v"(p[0]), [p1] "v"(p[1]), [p2] "v"(p[2]), [p3] "v"(p[3]), [p4] "v"(p[4]), [p5] "v"(p[5]),
        [p6] "v"(p[6]), [p7] "v"(p[7]), [x0] "v"(xv[0]), [x1] "v"(xv[1]), [x2] "v"(xv[2]), [x3] "v"(xv[3]),
        [x4] "v"(xv[4]), [x5] "v"(xv[5]), [x6] "v"(xv[6]), [x7] "v"(xv[7]), [w] "v"(w), [sc] "v"(sc)
      : "v0", "v1", "v2", "v3", "v4", "v5");
#undef S14_A
#undef S14_AD
#undef S14_C
#undef S14_M
  return acc;
}

// Dot of one MXFP4 row of G groups (G % (4 NB) == 0) with x in LDS, NB
// batches of 4 groups in flight; the caller issued batches 0 .. NB-1.
// Result in every lane of the quad.
template <int NB, int G, bool kScaled>
__device__ __forceinline__ float mx_row_quad_as(MxQBatch (&b)[NB], Rsrc r, uint32_t woff, uint32_t soff,
                                                const float *__restrict__ xq) {
  static_assert(G % (4 * NB) == 0, "whole rounds of batches");
  float acc = 0.0f;
#pragma unroll 1
  for (int g0 = 0; g0 < G; g0 += 4 * NB) {
    const bool refill = g0 + 4 * NB < G;  // uniform
    // software-pipelined: group n+1's products are formed in the gaps of
    // group n's chain (scaled decode), from x read from LDS a group before
    float pc[8], pn[8], xn[8];
    mx_products8<kScaled>(pc, b[0].w[0], b[0].c & 255u, xq + 32 * g0);
    if constexpr (kScaled) quad_x8(xn, xq + 32 * (g0 + 1));
#pragma unroll
    for (int n = 0; n < 4 * NB; ++n) {
      const int j = n / 4, i = n % 4;
      if (n + 1 < 4 * NB) {
        const int jn = (n + 1) / 4, in = (n + 1) % 4;
        if constexpr (kScaled) {
          float xa[8];
#pragma unroll
          for (int k = 0; k < 8; ++k) xa[k] = xn[k];
          if (n + 2 < 4 * NB) quad_x8(xn, xq + 32 * (g0 + n + 2));
          acc = mx_quad_chain8_asm(acc, pc, pn, b[jn].w[in], pair_scale_operand(b[jn].c, in), xa);
          if (n + 2 == 4 * NB) acc = asm_chain_end(acc);
        } else {
          mx_products8<kScaled>(pn, b[jn].w[in], (b[jn].c >> (8 * in)) & 255u, xq + 32 * (g0 + n + 1));
          acc = quad_chain8(acc, pc);
        }
      } else {
        acc = quad_chain8(acc, pc);
      }
      if (i == 3 && refill) mxq_load(b[j], r, woff, soff, g0 + 4 * NB + 4 * j);
#pragma unroll
      for (int k = 0; k < 8; ++k) pc[k] = pn[k];
    }
  }
  return from_quad_last(acc);
}
// The decode chosen once per wavefront (`scaled` uniform).
template <int NB, int G>
__device__ __forceinline__ float mx_row_quad(MxQBatch (&b)[NB], Rsrc r, uint32_t woff, uint32_t soff,
                                             const float *__restrict__ xq, bool scaled) {
  return scaled ? mx_row_quad_as<NB, G, true>(b, r, woff, soff, xq) : mx_row_quad_as<NB, G, false>(b, r, woff, soff, xq);
}

// ---------------------------------------------------------------------------
// act_quant of the official expert semantics (l42_reference.py:390-403,
// group 128): a vector in LDS is replaced, in place, by its requantised
// values e4m3(v / s) * s with s = 2^(code-127) per 128 values, each exactly
// representable in f32; the decode window of the result is returned.
// ---------------------------------------------------------------------------

// Groups g = first, first + stride, ... of v (128 values each), by one
// wavefront, two values per lane; accumulates the exponent range.
__device__ __forceinline__ void requant128_groups(float *v, int n_groups, int first, int stride, int &lo, int &hi) {
  const uint32_t lane = threadIdx.x & 63;
  for (int g = first; g < n_groups; g += stride) {
    float2 *p = reinterpret_cast<float2 *>(v + 128 * g) + lane;
    const float2 a = *p;
    // amax over the group (NaN ignored, as the oracle's strict '>' scan does:
    // a lane whose two values are NaN contributes 0)
    float m = 0.0f;
    m = fabsf(a.x) > m ? fabsf(a.x) : m;
    m = fabsf(a.y) > m ? fabsf(a.y) : m;
    const float amax = __uint_as_float(uint32_t(wave_max_i(int(__float_as_uint(m)))));  // m >= 0: bits order as values
    const uint32_t code = requant_code(amax);
    const float inv = __uint_as_float((254u - code) << 23), sc = __uint_as_float(code << 23);
    const float qa = __fmul_rn(e4m3_f32(s14x::e4m3_rne_sat(__fmul_rn(a.x, inv))), sc);
    const float qb = __fmul_rn(e4m3_f32(s14x::e4m3_rne_sat(__fmul_rn(a.y, inv))), sc);
    *p = make_float2(qa, qb);
    exp_range_acc(qa, lo, hi);
    exp_range_acc(qb, lo, hi);
  }
}
// A whole vector by the W = NT / 64 wavefronts of a workgroup (groups
// strided over the wavefronts), between two barriers; red: LDS scratch of
// 2 W ints.  Every thread gets the window.
template <int NT>
__device__ __forceinline__ CodeWindow requant128_block(float *v, int n, int *red) {
  constexpr int W = NT / 64;
  const int wave = int(threadIdx.x >> 6);
  __syncthreads();  // the staged vector is complete
  int lo = 255, hi = 0;
  requant128_groups(v, n / 128, wave, W, lo, hi);
  lo = wave_min_i(lo);
  hi = wave_max_i(hi);
  if ((threadIdx.x & 63) == 0) {
    red[2 * wave] = lo;
    red[2 * wave + 1] = hi;
  }
  __syncthreads();
#pragma unroll
  for (int w = 0; w < W; ++w) {
    lo = min(lo, red[2 * w]);
    hi = max(hi, red[2 * w + 1]);
  }
  return mx_window(lo, hi);
}

// Groups per register batch in the fused exact kernels.  Larger batches hide
// more load latency but inline a longer straight-line body; on the box 8
// beat 16 by 10 % per layer (instruction supply) and 4 (batch overhead).
constexpr int kPF = 8;

// Router: one wavefront per (expert, token).  Logit order (fixed here; the
// reference uses torch F.linear, executor.py:641, whose order is the
// BLAS's): lane l sums k = 256c + 4l + j (c ascending, j = 0..3), each
// step one fused multiply-add acc = fma(w_k, x_k, acc) (one rounding per
// term, as a BLAS dot kernel's FMA), then the xor butterfly over lanes
// (plain adds).  Score: sigmoid (north-star config) or
// sqrt(softplus) with torch's threshold 20 (executor.py:642), exp and log1p
// bit-identical to the C library's (s14_expf.h, s14_log1pf.h) as the
// oracle's.  Score and biased score of expert e from its logit.
__device__ __forceinline__ float2 router_finish(const RouterArgs &r, float logit, uint32_t e) {
  float sc;
  if (r.score_fn == S14_SCORE_SIGMOID) {
    sc = __fdiv_rn(1.0f, __fadd_rn(1.0f, s14x::expf_glibc(-logit)));
  } else {
    const float sp = logit > 20.0f ? logit : s14x::log1pf_glibc(s14x::expf_glibc(logit));
    // IEEE square root (HIP's __fsqrt_rn is the approximate native one unless
    // OCML_BASIC_ROUNDED_OPERATIONS is defined; measured 15 % of results one
    // ulp off on the softplus range)
    sc = __builtin_sqrtf(sp);
  }
  return make_float2(sc, __fadd_rn(sc, r.bias[e]));
}

// Score of expert e for token t, computed by one whole wavefront; valid in
// lane 0 (the biased score in .y).  xwin != NULL (uniform): also store the
// exponent range of the token's x there (lo | hi << 16, as stage_x_block
// finds it), from the registers the logit already loaded.
__device__ __forceinline__ float2 router_score(const RouterArgs &r, const float *__restrict__ X, uint32_t t,
                                               uint32_t e, uint32_t *xwin = nullptr) {
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t K = kHidden;
  const float *x = X + size_t(t) * K;
  const float *row = r.weight + size_t(e) * K;
  float4 wv[K / 256], xv[K / 256];
#pragma unroll
  for (uint32_t c = 0; c < K / 256; ++c) {
    wv[c] = *reinterpret_cast<const float4 *>(row + c * 256 + lane * 4);
    xv[c] = *reinterpret_cast<const float4 *>(x + c * 256 + lane * 4);
  }
  float acc = 0.0f;
#pragma unroll
  for (uint32_t c = 0; c < K / 256; ++c) {
    acc = __fmaf_rn(wv[c].x, xv[c].x, acc);
    acc = __fmaf_rn(wv[c].y, xv[c].y, acc);
    acc = __fmaf_rn(wv[c].z, xv[c].z, acc);
    acc = __fmaf_rn(wv[c].w, xv[c].w, acc);
  }
  if (xwin) {
    int lo = 255, hi = 0;
#pragma unroll
    for (uint32_t c = 0; c < K / 256; ++c) {
      exp_range_acc(xv[c].x, lo, hi);
      exp_range_acc(xv[c].y, lo, hi);
      exp_range_acc(xv[c].z, lo, hi);
      exp_range_acc(xv[c].w, lo, hi);
    }
    lo = wave_min_i(lo);
    hi = wave_max_i(hi);
    if (lane == 0) *xwin = uint32_t(lo) | (uint32_t(hi) << 16);
  }
  return router_finish(r, xor_butterfly_sum(acc), e);
}

}  // namespace
}  // namespace s14
