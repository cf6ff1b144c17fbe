// EXACT row engine for blocks of 2..8 tokens (the K <= 8 speculative-verify
// block): one output row per lane.  The same kernels, instantiated with
// kOfficial, run official blocks (the official expert semantics: the route
// launch's act_quant of x, bf16 roundings, the route weight before w2, h's
// act_quant at the end of phase 1).
//
// The reference CPU oracle's order is a dependent chain of adds per (row,
// token): acc += (x_k * e2m1(w_k)) * s, k ascending
// (scheduler/ssd_inference/examples/s14_vulkan_numeric.rs:1669-1696).  At
// batch 1 the lane-pair engine (s14_exact.hpp) keeps two lanes per row so
// that every SIMD gets a row chain; a block has up to 56 (token, expert)
// pairs, enough chains for one lane each, and one lane per row drops the
// lane pair's discarded adds and LDS x reads:
//
//   - a lane owns one row of w1 (lanes 0-31) or the same row of w3 (lanes
//     32-63) in phase 1, one row of w2 in phase 2;
//   - per group of 32 k it reads its row's 16 code bytes (from LDS, where the
//     wavefront's DMA loads put them) and scale code, converts them with 16
//     scaled v_cvt (2 values each, e2m1 * 2^(c-127)), multiplies each by x_k
//     and adds the product into its chain;
//   - x_k reaches every lane through the multiply's own DPP operand
//     (row_newbcast:i broadcasts lane i of each 16-lane row): a register
//     holding x[32g + j] in lane j (+16, +32, +48) serves 16 products, so x
//     costs two loads per group, no VALU instruction;
//   - a group is 16 + 32 + 32 VALU instructions for 64 rows, against the
//     lane pair's 56 for 32.
//
// The scaled decode equals the oracle's two multiplies while both products
// stay normal (the window of s14_exact.hpp: codes within [max(2, 129 - emin),
// 252] for x's biased exponent range [emin, emax], emin >= 2, emax <= 251);
// a chunk with a code outside the window takes the literal two-multiply
// decode.
//
// Phase 2 writes each pair's w2 output; a small kernel then accumulates each
// token's slots in route order, shared last (s14_vulkan_numeric.rs:929-946).
//
// Each distinct routed page is read once per block: the workgroups of one
// page's tokens (adjacent in the expert-major pair order) for the same tile
// group get workgroup ids 8 apart, so they run on the same XCD one after the
// other and the later tokens' reads of the rows hit that XCD's L2.
//
// The launches take a range of pairs [p0, p0 + n): the host may run the
// block's pairs as two halves on two streams, so that one half's phase 2
// fills the idle SIMDs of the other half's phase-1 tail (each phase is 3.5
// wavefronts per SIMD of equal length, two resident at a time).
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <utility>

#include "s14_device.hpp"
#include "s14_device_util.hpp"
#include "s14_exact.hpp"

namespace s14 {
namespace {

constexpr int kBTileGroups = 16;  // workgroups per pair in each phase: 128 rows of h, 256 rows of w2
constexpr int kXcds = 8;
static_assert(kBTileGroups % kXcds == 0, "tile groups spread evenly over the XCDs");
static_assert(kInter / 32 <= kInter / kP1ExactRows, "32-row h windows fit the workspace's per-pair records");

// The 32 decoded values of one group, e2m1 * scale (scale = 2^(c-127) in
// the scaled form, 1 in the literal one), k = 2i, 2i+1 in q[i].
__device__ __forceinline__ void decode32(v2f (&q)[16], uint4 w, float scale) {
  const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    q[4 * d + 0] = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(words[d], scale, 0);
    q[4 * d + 1] = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(words[d], scale, 1);
    q[4 * d + 2] = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(words[d], scale, 2);
    q[4 * d + 3] = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(words[d], scale, 3);
  }
}

template <int K>
__device__ __forceinline__ float qv(const v2f (&q)[16]) {
  return (K & 1) ? q[K >> 1].y : q[K >> 1].x;
}

// acc + sum of x_k * q_k (scaled: the product is the oracle's), k = 0..31 in
// order; xa holds x[k] for k < 16 in lane k % 16, xb for k >= 16.
template <int... K>
__device__ __forceinline__ float chain_scaled(float acc, const v2f (&q)[16], float xa, float xb,
                                              std::integer_sequence<int, K...>) {
  const float p[32] = {__fmul_rn(bcast16<K>(K < 16 ? xa : xb), qv<K>(q))...};
  ((acc = __fadd_rn(acc, p[K])), ...);
  return acc;
}
// The literal form: (x_k * e2m1_k) * s.
template <int... K>
__device__ __forceinline__ float chain_literal(float acc, const v2f (&q)[16], float s, float xa, float xb,
                                               std::integer_sequence<int, K...>) {
  const float p[32] = {__fmul_rn(__fmul_rn(bcast16<K>(K < 16 ? xa : xb), qv<K>(q)), s)...};
  ((acc = __fadd_rn(acc, p[K])), ...);
  return acc;
}
using K32 = std::make_integer_sequence<int, 32>;

// FP8 rows (the reference's FP8 shared page): 32 code bytes per group, one
// UE8M0 scale per 128 x 128 tile; p = (x * e4m3) * s
// (s14_vulkan_numeric.rs:1698-1714), literal always.
__device__ __forceinline__ void decode32_fp8(v2f (&q)[16], uint4 a, uint4 b) {
  const uint32_t words[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
  for (int d = 0; d < 8; ++d) {
    q[2 * d + 0] = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(words[d], 1.0f, false);
    q[2 * d + 1] = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(words[d], 1.0f, true);
  }
}

// ---------------------------------------------------------------------------
// Codes through LDS.  A wavefront's 64 rows are read one row per lane, but
// loading them that way from memory has every load instruction touch 64
// cache lines (measured: 3.3x the time of the same loop on register data).
// So a wavefront DMA-loads (buffer_load_dwordx4 ... lds) each chunk of 8
// groups (128 bytes of each of its 64 rows, 8 KB) with 8 lanes per row
// segment, full lines per quarter-wave, into one of two LDS slots; lane l's
// 16-byte piece q of row r lands at piece q ^ (r & 7), so the 8 rows of each
// read pass take distinct banks.  The next chunk's DMA is in flight while
// the current one is consumed.
// ---------------------------------------------------------------------------
constexpr int kBChunk = 8;                       // groups per chunk: 128 bytes of a row
constexpr int kBRowsW = 64;                      // rows per wavefront
// Wavefronts per workgroup: 4 (two 64 KB workgroups per CU) measured faster
// than 2 (five 32 KB workgroups per CU: phase 1 109 -> 127 us at K=8).
constexpr int kBWaves = 4;
constexpr uint32_t kBSlot = kBRowsW * 16u * kBChunk;  // 8 KB per wavefront and slot
__shared__ __attribute__((aligned(16))) uint8_t b_slot0[kBWaves][kBSlot];
__shared__ __attribute__((aligned(16))) uint8_t b_slot1[kBWaves][kBSlot];

template <int S>
__device__ __forceinline__ uint8_t *b_slot(uint32_t wave) {
  if constexpr (S == 0) return b_slot0[wave];
  else return b_slot1[wave];
}

typedef __attribute__((address_space(3))) void lds_void;
__device__ __forceinline__ void dma16(Rsrc r, uint8_t *lds, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)(lds), 16, off, 0, 0, 0);
}
// Before a DMA refills a slot: every LDS read of its previous chunk returned.
__device__ __forceinline__ void lds_reads_done() { __builtin_amdgcn_s_waitcnt(0xc07f); }

// Per-lane state of one wavefront's row stream: the DMA source offsets of
// its 8 instructions per chunk (instruction j: row 8j + lane/8, piece
// (lane % 8) ^ (row & 7)) and the lane's own row's scale-code offset.
struct RowStream {
  Rsrc r;
  uint32_t dma[8];
  uint32_t soff;
  const float *x;  // the vector the rows multiply (global memory; L2-resident)
};


template <int S>
__device__ __forceinline__ void stream_issue(const RowStream &st, uint32_t wave, int c) {
  uint8_t *dst = b_slot<S>(wave);
  lds_reads_done();
#pragma unroll
  for (int j = 0; j < 8; ++j) dma16(st.r, dst + 1024u * j, st.dma[j] + 128u * uint32_t(c));
}

// Scale codes and x of chunk c (registers).
struct ChunkRegs {
  uint2 c;
  float a[kBChunk], b[kBChunk];
};
__device__ __forceinline__ void chunk_regs(ChunkRegs &cr, const RowStream &st, int c) {
  cr.c = ld8(st.r, st.soff + uint32_t(c * kBChunk));
  const uint32_t j = threadIdx.x & 15u;
#pragma unroll
  for (int i = 0; i < kBChunk; ++i) {
    cr.a[i] = st.x[32 * (c * kBChunk + i) + j];
    cr.b[i] = st.x[32 * (c * kBChunk + i) + 16 + j];
  }
}
__device__ __forceinline__ uint32_t chunk_code(const ChunkRegs &cr, int i) {
  return ((i < 4 ? cr.c.x : cr.c.y) >> (8 * (i & 3))) & 255u;
}

// Consume chunk c from slot S: 8 groups of the lane's row, k ascending.
template <int S>
__device__ __forceinline__ float chunk_consume(float acc, const ChunkRegs &cr, uint32_t wave, CodeWindow win,
                                               const RowStream &st, int c) {
  const uint32_t lane = threadIdx.x & 63;
  const uint8_t *row = b_slot<S>(wave) + 128u * lane;
  bool ok = true;
#pragma unroll
  for (int i = 0; i < kBChunk; ++i) {
    const int code = int(chunk_code(cr, i));
    ok = ok && code >= win.cmin && code <= win.cmax;
  }
  if (__builtin_amdgcn_ballot_w64(!ok) == 0ull) {
#pragma unroll
    for (int i = 0; i < kBChunk; ++i) {
      const uint4 w = *reinterpret_cast<const uint4 *>(row + 16u * (uint32_t(i) ^ (lane & 7u)));
      v2f q[16];
      decode32(q, w, __uint_as_float(chunk_code(cr, i) << 23));
      acc = chain_scaled(acc, q, cr.a[i], cr.b[i], K32{});
    }
  } else {
    // literal decode (a code outside the window): group by group, codes from
    // LDS, scale codes and x from memory: nothing in `cr` is indexed by the
    // loop variable (that would move the register arrays to scratch memory on
    // every path)
    const uint32_t j = threadIdx.x & 15u;
#pragma unroll 1
    for (int i = 0; i < kBChunk; ++i) {
      const uint4 w = *reinterpret_cast<const uint4 *>(row + 16u * (uint32_t(i) ^ (lane & 7u)));
      v2f q[16];
      decode32(q, w, 1.0f);
      const int g = c * kBChunk + i;
      acc = chain_literal(acc, q, ue8m0_f32(ld1(st.r, st.soff + uint32_t(g))), st.x[32 * g + j],
                          st.x[32 * g + 16 + j], K32{});
    }
  }
  return acc;
}

// Dot of the lane's MXFP4 row (NC chunks) with st.x, k ascending.
template <int NC>
__device__ __forceinline__ float row_dot_stream(const RowStream &st, uint32_t wave, CodeWindow win) {
  static_assert(NC % 2 == 0, "chunk pairs");
  ChunkRegs c0, c1;
  stream_issue<0>(st, wave, 0);
  chunk_regs(c0, st, 0);
  float acc = 0.0f;
#pragma unroll 1
  for (int c = 0; c < NC; c += 2) {
    stream_issue<1>(st, wave, c + 1);
    chunk_regs(c1, st, c + 1);
    acc = chunk_consume<0>(acc, c0, wave, win, st, c);
    if (c + 2 < NC) {
      stream_issue<0>(st, wave, c + 2);
      chunk_regs(c0, st, c + 2);
    }
    acc = chunk_consume<1>(acc, c1, wave, win, st, c + 1);
  }
  return acc;
}

// FP8 rows (the reference's FP8 shared page): 32 code bytes per group, one
// UE8M0 scale per 128 x 128 tile; p = (x * e4m3) * s
// (s14_vulkan_numeric.rs:1698-1714), literal always; rare (that variant's
// shared page only), read straight from memory.
template <int G>
__device__ __forceinline__ float row_dot_fp8(Rsrc r, uint32_t woff, uint32_t soff_tiles, const float *x) {
  float acc = 0.0f;
  const uint32_t j = threadIdx.x & 15u;
#pragma unroll 1
  for (int g0 = 0; g0 < G; g0 += 4) {
    uint4 wa[4], wb[4];
    float xa[4], xb[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      wa[i] = ld16(r, woff + 32u * uint32_t(g0 + i));
      wb[i] = ld16(r, woff + 32u * uint32_t(g0 + i) + 16u);
      xa[i] = x[32 * (g0 + i) + j];
      xb[i] = x[32 * (g0 + i) + 16 + j];
    }
    const float s = ue8m0_f32(ld1(r, soff_tiles + uint32_t(g0 / 4)));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v2f q[16];
      decode32_fp8(q, wa[i], wb[i]);
      acc = chain_literal(acc, q, s, xa[i], xb[i], K32{});
    }
  }
  return acc;
}

__device__ __forceinline__ uint32_t b_page_bytes(uint32_t fmt) {
  return fmt == S14_PAGE_MXFP4 ? uint32_t(S14_EXPERT_PAGE_BYTES) : uint32_t(S14_SHARED_EXPERT_PAGE_BYTES);
}

// Workgroup id -> (tile group q of 16, pair p): XCD id % 8 = q % 8, and one
// XCD's ids enumerate (q / 8, p), so the pairs of one page (adjacent in the
// expert-major order) with the same tile group run on one XCD back to back.
__device__ __forceinline__ void b_decode_id(uint32_t n_pairs, uint32_t p0, uint32_t &q, uint32_t &p) {
  const uint32_t id = blockIdx.x, xcd = id % kXcds, j = id / kXcds;
  q = (j / n_pairs) * kXcds + xcd;
  p = p0 + j % n_pairs;
}

// Phase 1: workgroup -> (pair, 128 rows of h), wavefront -> 32 rows of w1
// (lanes 0-31) and the same rows of w3 (lanes 32-63); h = swiglu(g, u).
// kOfficial (the official expert semantics, executor.py:705-731): x is the
// route launch's act_quant of x (ws.xq, with its window in ws.xwin); g and
// u are rounded to bf16, h = bf16(swiglu(g, u) * w) with w the pair's route
// weight; then h's act_quant for w2 (group 128, l42_reference.py:390-403):
// the workgroup's 128 rows are exactly one group, so the group's maximum is
// one exchange through LDS and no separate requant launch is needed.
static_assert(kBWaves * 32 == 128, "a phase-1 workgroup's rows are one act_quant group of h");
template <bool kOfficial>
__global__ __launch_bounds__(64 * kBWaves) void k_block_phase1(const PairTable *__restrict__ tab, Workspace ws,
                                                               const float *__restrict__ X, uint32_t p0,
                                                               uint32_t n_pairs, PageOffsets mx, PageOffsets f8) {
  uint32_t q, p;
  b_decode_id(n_pairs, p0, q, p);
  const uint32_t lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // every token's x window (lane i: token i % 8), loaded beside the table
  // words rather than after them
  const uint32_t xw_all = ws.xwin[lane & uint32_t(kMaxTokens - 1)];
  const uint8_t *page = reinterpret_cast<const uint8_t *>(tab->page[p]);
  const uint32_t fmt = tab->fmt[p], t = tab->token[p];
  const float *x = (kOfficial ? ws.xq : X) + size_t(t) * kHidden;
  const uint32_t tile = q * kBWaves + wave;  // 32-row tile of h
  const uint32_t row0 = tile * 32u;
  const bool upper = lane >= 32;
  const uint32_t row = row0 + (lane & 31u);
  const Rsrc r = make_rsrc(page, b_page_bytes(fmt));
  float acc;
  if (fmt == S14_PAGE_MXFP4) {
    RowStream st;
    st.r = r;
    st.x = x;
    st.soff = uint32_t(upper ? mx.s3 : mx.s1) + row * (kHidden / 32);
#pragma unroll
    for (uint32_t j = 0; j < 8; ++j) {
      const uint32_t dr = 8u * j + (lane >> 3);  // 0..63: rows 0-31 of w1, then of w3
      const uint32_t base = uint32_t(dr < 32 ? mx.w1 : mx.w3) + (row0 + (dr & 31u)) * (kHidden / 2);
      st.dma[j] = base + 16u * ((lane & 7u) ^ (dr & 7u));
    }
    // x's decode window: the exponent range the route kernel recorded
    const uint32_t xw = uint32_t(__builtin_amdgcn_readlane(int(xw_all), int(t)));
    const CodeWindow win = mx_window(int(xw & 0xffffu), int(xw >> 16));
    acc = row_dot_stream<kHidden / 32 / kBChunk>(st, wave, win);
  } else {
    acc = row_dot_fp8<kHidden / 32>(r, uint32_t(upper ? f8.w3 : f8.w1) + row * kHidden,
                                    uint32_t(upper ? f8.s3 : f8.s1) + (row / 128) * (kHidden / 128), x);
  }
  const float u = lane_xor32(acc);
  int lo = 255, hi = 0;
  if constexpr (kOfficial) {
    __shared__ int b_amax[kBWaves];
    float hv = 0.0f, m = 0.0f;
    if (!upper) {
      hv = bf16_round(__fmul_rn(swiglu_exact(bf16_round(acc), bf16_round(u)), tab->weight[p]));
      m = fabsf(hv) > m ? fabsf(hv) : m;  // a NaN never compares greater, as in the oracle's scan
    }
    const int mw = wave_max_i(int(__float_as_uint(m)));  // m >= 0: bits order as values
    if (lane == 0) b_amax[wave] = mw;
    __syncthreads();
    int mb = b_amax[0];
#pragma unroll
    for (int w = 1; w < kBWaves; ++w) mb = max(mb, b_amax[w]);
    const uint32_t code = requant_code(__uint_as_float(uint32_t(mb)));
    const float inv = __uint_as_float((254u - code) << 23), sc = __uint_as_float(code << 23);
    if (!upper) {
      const float q = __fmul_rn(e4m3_f32(s14x::e4m3_rne_sat(__fmul_rn(hv, inv))), sc);
      ws.h[size_t(p) * kInter + row] = q;
      exp_range_acc(q, lo, hi);
    }
  } else if (!upper) {
    // once per row: expf's table from constant memory
    const float hv = swiglu_exact(acc, u);
    ws.h[size_t(p) * kInter + row] = hv;
    exp_range_acc(hv, lo, hi);
  }
  lo = wave_min_i(lo);
  hi = wave_max_i(hi);
  if (lane == 0) ws.hwin[size_t(p) * kP1Tiles + tile] = uint32_t(lo) | (uint32_t(hi) << 16);
}

// Phase 2: workgroup -> (pair, 256 rows of w2), wavefront -> 64 rows, one
// per lane; down[pair][row] without the route weight (kOfficial: the
// weight is already in h, and the output is rounded to bf16).
template <bool kOfficial>
__global__ __launch_bounds__(64 * kBWaves) void k_block_phase2(const PairTable *__restrict__ tab, Workspace ws,
                                                               uint32_t p0, uint32_t n_pairs, PageOffsets mx,
                                                               PageOffsets f8) {
  uint32_t q, p;
  b_decode_id(n_pairs, p0, q, p);
  const uint32_t lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // h's window records (64 tiles of 32 rows), loaded beside the table words
  const uint32_t wrec = ws.hwin[size_t(p) * kP1Tiles + lane];
  const uint8_t *page = reinterpret_cast<const uint8_t *>(tab->page[p]);
  const uint32_t fmt = tab->fmt[p];
  const float *h = ws.h + size_t(p) * kInter;
  const uint32_t row0 = (q * kBWaves + wave) * kBRowsW;
  const uint32_t row = row0 + lane;
  const Rsrc r = make_rsrc(page, b_page_bytes(fmt));
  float acc;
  if (fmt == S14_PAGE_MXFP4) {
    RowStream st;
    st.r = r;
    st.x = h;
    st.soff = uint32_t(mx.s2) + row * (kInter / 32);
#pragma unroll
    for (uint32_t j = 0; j < 8; ++j) {
      const uint32_t dr = 8u * j + (lane >> 3);
      st.dma[j] = uint32_t(mx.w2) + (row0 + dr) * (kInter / 2) + 16u * ((lane & 7u) ^ (dr & 7u));
    }
    const CodeWindow win = mx_window(wave_min_i(int(wrec & 0xffffu)), wave_max_i(int(wrec >> 16)));
    acc = row_dot_stream<kInter / 32 / kBChunk>(st, wave, win);
  } else {
    acc = row_dot_fp8<kInter / 32>(r, uint32_t(f8.w2) + row * kInter, uint32_t(f8.s2) + (row / 128) * (kInter / 128),
                                   h);
  }
  if constexpr (kOfficial) acc = bf16_round(acc);
  ws.down[size_t(p) * kHidden + row] = acc;
}

// y[t][r] = sum_j w_j down_j[r] (routed, route order) + down_shared[r]
// (s14_vulkan_numeric.rs:929-946); 4 rows per thread.  kOfficial: each
// slot's bf16 output already carries its weight; y = bf16(sum in route
// order, shared last) (executor.py:712-739).
template <bool kOfficial>
__global__ __launch_bounds__(256) void k_block_combine(const PairTable *__restrict__ tab, Workspace ws,
                                                       float *__restrict__ Y, uint32_t tokens) {
  const uint32_t gid = blockIdx.x * 256u + threadIdx.x;
  if (gid >= tokens * (kHidden / 4)) return;
  const uint32_t t = gid / (kHidden / 4), r = 4u * (gid % (kHidden / 4));
  // every slot record in one round trip (with the count), then every used
  // slot's down row in a second, then the adds in route order
  const uint32_t np = tab->npairs[t];
  uint32_t sp[kSlots], sh[kSlots];
  float sw[kSlots];
#pragma unroll
  for (uint32_t j = 0; j < uint32_t(kSlots); ++j) {
    sp[j] = tab->slot_pair[t][j];
    sh[j] = tab->slot_shared[t][j];
    sw[j] = tab->slot_weight[t][j];
  }
  float4 d[kSlots];
#pragma unroll
  for (uint32_t j = 0; j < uint32_t(kSlots); ++j)
    d[j] = j < np ? *reinterpret_cast<const float4 *>(ws.down + size_t(sp[j]) * kHidden + r)
                  : make_float4(0.f, 0.f, 0.f, 0.f);
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (uint32_t j = 0; j < uint32_t(kSlots); ++j) {
    if (j >= np) break;
    if (kOfficial || sh[j]) {
      acc.x = __fadd_rn(acc.x, d[j].x);
      acc.y = __fadd_rn(acc.y, d[j].y);
      acc.z = __fadd_rn(acc.z, d[j].z);
      acc.w = __fadd_rn(acc.w, d[j].w);
    } else {
      acc.x = __fadd_rn(acc.x, __fmul_rn(sw[j], d[j].x));
      acc.y = __fadd_rn(acc.y, __fmul_rn(sw[j], d[j].y));
      acc.z = __fadd_rn(acc.z, __fmul_rn(sw[j], d[j].z));
      acc.w = __fadd_rn(acc.w, __fmul_rn(sw[j], d[j].w));
    }
  }
  if constexpr (kOfficial) acc = make_float4(bf16_round(acc.x), bf16_round(acc.y), bf16_round(acc.z), bf16_round(acc.w));
  *reinterpret_cast<float4 *>(Y + size_t(t) * kHidden + r) = acc;
}

}  // namespace

hipError_t launch_block_phase1(hipStream_t s, const Workspace &ws, uint32_t p0, uint32_t n_pairs,
                               const PageOffsets &mx, const PageOffsets &fp8, const float *x, bool official,
                               KernelEvents ev) {
  hipExtLaunchKernelGGL(official ? k_block_phase1<true> : k_block_phase1<false>, dim3(kBTileGroups * n_pairs),
                        dim3(64 * kBWaves), 0, s, ev.start, ev.stop, 0, ws.table, ws, x, p0, n_pairs, mx, fp8);
  return hipGetLastError();
}

hipError_t launch_block_phase2(hipStream_t s, const Workspace &ws, uint32_t p0, uint32_t n_pairs,
                               const PageOffsets &mx, const PageOffsets &fp8, bool official, hipEvent_t ev_start) {
  hipExtLaunchKernelGGL(official ? k_block_phase2<true> : k_block_phase2<false>,
                        dim3((kHidden / (kBRowsW * kBWaves)) * n_pairs), dim3(64 * kBWaves), 0, s, ev_start, nullptr,
                        0, ws.table, ws, p0, n_pairs, mx, fp8);
  return hipGetLastError();
}

hipError_t launch_block_combine(hipStream_t s, const Workspace &ws, uint32_t tokens, float *y, bool official,
                                hipEvent_t ev_stop) {
  hipExtLaunchKernelGGL(official ? k_block_combine<true> : k_block_combine<false>,
                        dim3((tokens * (kHidden / 4) + 255) / 256), dim3(256), 0, s, nullptr, ev_stop, 0, ws.table, ws,
                        y, tokens);
  return hipGetLastError();
}

}  // namespace s14
