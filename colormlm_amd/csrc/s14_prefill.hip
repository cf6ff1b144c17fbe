// Prefill through the S14 MoE layer (config 4) on gfx950: T tokens, each
// routed to its top-k experts plus the shared expert, computed per expert as
// grouped GEMMs on the CDNA4 scaled MFMA (v_mfma_scale_f32_32x32x64_f8f6f4):
// MXFP4 weights (A, E8M0 per 32 k) times e4m3-requantised activations (B,
// E8M0 per 32 k), f32 accumulation.
//
// There is no reference GPU code for this row; its semantics are the layer's
// (s14_vulkan_numeric.rs:929-946 accumulation, :1543-1556 SwiGLU) with the
// activation requant the north-star config names (e4m3 RNE, saturating,
// per-32 scale 2^ceil(log2(max(amax, 1e-4) / 448)), l42_reference.py:390-403
// with group 32).  The MFMA sums each 64-k step in its own precision, so
// this path is not order-exact; its tolerance against the CPU oracle is
// measured (tests/test_gpu_parity.py).
//
// Operand layout of the 32x32x64 scaled MFMA (established on the hardware,
// lane l, half h = l / 32):
//   A (fp4, 16 bytes)  row l % 32; bytes 0..7 hold k 16h..16h+15 and bytes
//                      8..15 hold k 32+16h..32+16h+15 (low nibble first)
//                      when B is laid out as below; scale_a of lane l covers
//                      the 32 k it holds, i.e. weight block h of the step.
//   B (fp8, 32 bytes)  column l % 32; byte j pairs with A as above, so B must
//                      hold {k 16h..16h+15, k 32+16h..32+16h+15} of the step;
//                      a product from A half h is scaled by scale_b of lane
//                      (column, h).
//   D (16 f32)         element i of lane l is row 8(i/4) + 4h + i%4, column
//                      l % 32.
// Loading each weight row's 16 contiguous bytes per lane-half (32 k, one
// E8M0 block) therefore pairs with activations stored per 64-k step in the
// order [k 0..15 | 32..47 | 16..31 | 48..63]: requant_x and the phase-1
// epilogue write x and h in that order.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include "s14_device.hpp"
#include "s14_device_util.hpp"
#include "s14_prefill.hpp"

namespace s14 {
namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr uint32_t kQGroup = 32;  // requant group (k values per E8M0 scale)

// ---------------------------------------------------------------------------
// requant (bit-identical to the oracle's s14o_requant_e4m3)
// ---------------------------------------------------------------------------

// E8M0 code of a group: 127 + ceil(log2(max(amax, 1e-4) / 448)), the f32
// quotient rounded to nearest, ceil(log2) taken exactly from its bits.
__device__ __forceinline__ uint32_t requant_code(float amax) {
  if (amax < 1.0e-4f) amax = 1.0e-4f;
  const float r = __fdiv_rn(amax, 448.0f);
  const uint32_t u = __float_as_uint(r);
  const int e = int((u >> 23) & 255u) - 127;  // r is normal: amax/448 >= 2.2e-7
  const int c = (u & 0x7fffffu) ? e + 1 : e;  // ceil(log2 r)
  return uint32_t(c + 127);
}

// OCP e4m3fn, round to nearest even, saturating to +-448 (NaN -> 0x7f).
__device__ __forceinline__ uint32_t e4m3_rne_sat(float v) {
  if (v != v) return 0x7fu;
  const uint32_t sign = (__float_as_uint(v) >> 24) & 0x80u;
  const float a = fabsf(v);
  if (a >= 448.0f) return sign | 0x7eu;
  if (a < 0x1p-6f) return sign | uint32_t(__builtin_rintf(__fmul_rn(a, 512.0f)));  // m * 2^-9 grid
  const uint32_t u = __float_as_uint(a);
  int e = int((u >> 23) & 255u) - 127;                     // a = m * 2^e, m in [1, 2)
  const float m = __uint_as_float((u & 0x7fffffu) | 0x3f800000u);
  float mant = __builtin_rintf(__fmul_rn(__fsub_rn(m, 1.0f), 8.0f));
  if (mant >= 8.0f) {
    mant = 0.0f;
    e += 1;
  }
  const int biased = e + 7;
  if (biased > 15 || (biased == 15 && mant >= 7.0f)) return sign | 0x7eu;
  return sign | uint32_t((biased << 3) | int(mant));
}

// X [T, 4096] f32 -> Q [T, 4096] e4m3 in MFMA order + S [T, 128] E8M0.
// One thread per 32-value group.
__global__ __launch_bounds__(256) void k_requant_x(uint32_t tokens, const float *__restrict__ X,
                                                   uint8_t *__restrict__ Q, uint8_t *__restrict__ S) {
  const uint32_t gid = blockIdx.x * blockDim.x + threadIdx.x;
  const uint32_t groups = kHidden / kQGroup;
  if (gid >= tokens * groups) return;
  const uint32_t t = gid / groups, g = gid % groups;
  const float4 *src = reinterpret_cast<const float4 *>(X + size_t(t) * kHidden + g * kQGroup);
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
  const uint32_t code = requant_code(amax);
  const float inv = __uint_as_float((254u - code) << 23);  // 2^-(code-127)
  uint32_t w[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    uint32_t word = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) word |= e4m3_rne_sat(__fmul_rn(v[4 * i + j], inv)) << (8 * j);
    w[i] = word;
  }
  // group g = 32 consecutive k at offset 32*(g%2) of step g/2
  uint8_t *dst = Q + size_t(t) * kHidden + 64u * (g >> 1);
  const uint32_t b = g & 1u;
  *reinterpret_cast<uint4 *>(dst + 16u * b) = make_uint4(w[0], w[1], w[2], w[3]);        // k 0..15 of the group
  *reinterpret_cast<uint4 *>(dst + 32u + 16u * b) = make_uint4(w[4], w[5], w[6], w[7]);  // k 16..31
  S[size_t(t) * groups + g] = uint8_t(code);
}

// The same requant in natural layout (the standalone dispatch): rows x k,
// groups of 32 along k.
__global__ __launch_bounds__(256) void k_requant_rows(uint32_t rows, uint32_t k, const float *__restrict__ X,
                                                      uint8_t *__restrict__ Q, uint8_t *__restrict__ S) {
  const uint32_t gid = blockIdx.x * blockDim.x + threadIdx.x;
  const uint32_t groups = k / kQGroup;
  if (gid >= rows * groups) return;
  const float *src = X + size_t(gid) * kQGroup;  // group gid of the row-major matrix
  float amax = 0.0f;
  for (int i = 0; i < 32; ++i) amax = fabsf(src[i]) > amax ? fabsf(src[i]) : amax;
  const uint32_t code = requant_code(amax);
  const float inv = __uint_as_float((254u - code) << 23);
  for (int i = 0; i < 32; ++i) Q[size_t(gid) * kQGroup + i] = uint8_t(e4m3_rne_sat(__fmul_rn(src[i], inv)));
  S[gid] = uint8_t(code);
}

// ---------------------------------------------------------------------------
// routing and grouping
// ---------------------------------------------------------------------------

__global__ void k_zero_u32(uint32_t n, uint32_t *__restrict__ p) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

// One wavefront per token: top-k, route weights, and the expert's token bit.
__global__ __launch_bounds__(256) void k_prefill_topk(PrefillArgs a, PrefillWorkspace ws) {
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t t = blockIdx.x * 4u + (threadIdx.x >> 6);
  if (t >= a.tokens) return;
  const uint32_t k = a.r.topk;
  const TopK c = select_topk(ws.biased + size_t(t) * kMaxExperts, ws.scores + size_t(t) * kMaxExperts, nullptr,
                             a.r.n_experts, k);
  if (lane < k) {
    const float w = route_weight(c, a.r.route_scale);
    ws.ids[t * kTopK + lane] = c.id;
    ws.weights[t * kTopK + lane] = w;
    if (a.ids_out) a.ids_out[t * k + lane] = uint16_t(c.id);
    if (a.weights_out) a.weights_out[t * k + lane] = w;
    atomicOr(&ws.token_bits[c.id * kPrefillBitWords + (t >> 5)], 1u << (t & 31));
  }
}

// One workgroup: per-expert token counts from the bitmaps, pair offsets
// (experts ascending, the shared expert last), each pair's token in token
// order within its expert, and the GEMM work items (<= kItemTokens tokens of
// one expert each).  Deterministic: positions come from bit counts.
__global__ __launch_bounds__(1024) void k_prefill_group(PrefillArgs a, PrefillWorkspace ws) {
  __shared__ uint32_t cnt[kMaxExperts + 1];
  __shared__ uint32_t off[kMaxExperts + 2];
  __shared__ uint32_t items_of[kMaxExperts + 1];
  __shared__ uint32_t item_off[kMaxExperts + 2];
  const uint32_t tid = threadIdx.x;
  const uint32_t T = a.tokens, words = (T + 31) / 32;
  for (uint32_t e = tid; e <= kMaxExperts; e += blockDim.x) {
    uint32_t c = 0;
    if (e < kMaxExperts)
      for (uint32_t w = 0; w < words; ++w) c += __popc(ws.token_bits[e * kPrefillBitWords + w]);
    else
      c = T;  // shared expert: every token
    cnt[e] = c;
    items_of[e] = (c + kItemTokens - 1) / kItemTokens;
  }
  __syncthreads();
  if (tid == 0) {  // 257 entries: a serial scan is cheaper than a barrier tree
    uint32_t o = 0, io = 0, distinct = 0, mx = 0;
    for (uint32_t e = 0; e <= kMaxExperts; ++e) {
      off[e] = o;
      item_off[e] = io;
      o += cnt[e];
      io += items_of[e];
      if (e < kMaxExperts && cnt[e]) {
        ++distinct;
        mx = cnt[e] > mx ? cnt[e] : mx;
      }
    }
    off[kMaxExperts + 1] = o;
    item_off[kMaxExperts + 1] = io;
    ws.stats[0] = io;  // number of work items
    ws.stats[1] = distinct;
    ws.stats[2] = mx;
    ws.stats[3] = o;  // number of pairs
  }
  __syncthreads();
  // work items
  for (uint32_t e = tid; e <= kMaxExperts; e += blockDim.x) {
    for (uint32_t j = 0; j < items_of[e]; ++j) {
      const uint32_t first = j * kItemTokens;
      const uint32_t n = min(kItemTokens, cnt[e] - first);
      ws.items[item_off[e] + j] = PrefillItem{e, off[e] + first, n};
    }
  }
  // pairs: routed (token t, slot s) -> position = tokens of the expert below t
  for (uint32_t t = tid; t < T; t += blockDim.x) {
    for (uint32_t s = 0; s < a.r.topk; ++s) {
      const uint32_t e = ws.ids[t * kTopK + s];
      const uint32_t *bits = ws.token_bits + e * kPrefillBitWords;
      uint32_t rank = 0;
      for (uint32_t w = 0; w < (t >> 5); ++w) rank += __popc(bits[w]);
      rank += __popc(bits[t >> 5] & ((1u << (t & 31)) - 1u));
      const uint32_t p = off[e] + rank;
      ws.pair_token[p] = t;
      ws.token_pair[t * kSlots + s] = p;
    }
    const uint32_t ps = off[kMaxExperts] + t;
    ws.pair_token[ps] = t;
    ws.token_pair[t * kSlots + a.r.topk] = ps;
  }
}

// ---------------------------------------------------------------------------
// grouped GEMMs
// ---------------------------------------------------------------------------

__device__ __forceinline__ Rsrc page_rsrc(const PrefillArgs &a, uint32_t e) {
  const uint8_t *page = e < kMaxExperts ? reinterpret_cast<const uint8_t *>(a.expert_pages[e]) : a.shared_page;
  return make_rsrc(page, uint32_t(S14_EXPERT_PAGE_BYTES));
}

__device__ __forceinline__ v8i a_operand(uint4 w) {
  v8i v = {int(w.x), int(w.y), int(w.z), int(w.w), 0, 0, 0, 0};
  return v;
}
__device__ __forceinline__ v8i b_operand(uint4 lo, uint4 hi) {
  v8i v = {int(lo.x), int(lo.y), int(lo.z), int(lo.w), int(hi.x), int(hi.y), int(hi.z), int(hi.w)};
  return v;
}

// Pins the accumulators in uniform control flow.  The epilogues store only
// columns < count, a per-lane condition; without this the compiler may sink
// the last K step's MFMA into that branch, and an MFMA issued under a partial
// EXEC mask does not take the inactive lanes' A rows and scales (their output
// rows come back as garbage).
template <int NT>
__device__ __forceinline__ void mfma_settle(v16f (&acc)[NT]) {
#pragma unroll
  for (int j = 0; j < NT; ++j) asm volatile("" : "+a"(acc[j]));
}

template <int NT>
struct BStep {
  uint4 lo[NT], hi[NT];
  uint32_t sc[NT];
};

// B operands of step s for NT token tiles: lane (c, h) loads 32 bytes of
// its token's requantised row at 64 s + 32 h and the scale of block 2 s + h.
// Columns past the item's token count read token 0's row (never stored).
template <int NT>
__device__ __forceinline__ void load_b(BStep<NT> &b, const uint8_t *__restrict__ q, const uint8_t *__restrict__ sc,
                                       const uint32_t (&row)[NT], uint32_t row_bytes, uint32_t s, uint32_t h) {
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const uint4 *p = reinterpret_cast<const uint4 *>(q + size_t(row[j]) * row_bytes + 64u * s + 32u * h);
    b.lo[j] = p[0];
    b.hi[j] = p[1];
    b.sc[j] = sc[size_t(row[j]) * (row_bytes / kQGroup) + 2u * s + h];
  }
}

// Phase 1: one wavefront per (32-row tile of w1/w3, work item of <= 128
// tokens of one expert).  K loop of 64 steps, NT token tiles at once; then
// h = swiglu(g, u), requantised per token over the tile's 32 rows (one E8M0
// group of phase 2's K) and stored in MFMA order.
template <int NT>
__device__ __forceinline__ void prefill_up_tiles(const PrefillArgs &a, const PrefillWorkspace &ws,
                                                 const PrefillItem &it, uint32_t rt) {
  const uint32_t lane = threadIdx.x & 63, col = lane & 31, h = lane >> 5;
  const Rsrc rp = page_rsrc(a, it.expert);
  const uint32_t row = rt * 32u + col;  // A row of this lane
  const uint32_t w1 = uint32_t(a.mx.w1) + row * (kHidden / 2) + 16u * h;
  const uint32_t w3 = uint32_t(a.mx.w3) + row * (kHidden / 2) + 16u * h;
  const uint32_t s1 = uint32_t(a.mx.s1) + row * (kHidden / 32) + h;
  const uint32_t s3 = uint32_t(a.mx.s3) + row * (kHidden / 32) + h;
  uint32_t xrow[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const uint32_t i = 32u * j + col;
    xrow[j] = ws.pair_token[it.first + (i < it.count ? i : 0u)];
  }
  v16f g[NT], u[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j)
#pragma unroll
    for (int i = 0; i < 16; ++i) g[j][i] = u[j][i] = 0.0f;
  uint4 a1 = ld16(rp, w1), a3 = ld16(rp, w3);
  uint32_t c1 = ld1(rp, s1), c3 = ld1(rp, s3);
  BStep<NT> b;
  load_b<NT>(b, ws.xq, ws.xs, xrow, kHidden, 0, h);
  constexpr uint32_t kSteps = kHidden / 64;
  for (uint32_t s = 0; s < kSteps; ++s) {
    // next step's operands in flight during this step's MFMAs (past the
    // last step: reads inside the page or of token rows, never consumed)
    const uint32_t sn = s + 1 < kSteps ? s + 1 : s;
    const uint4 na1 = ld16(rp, w1 + 32u * sn), na3 = ld16(rp, w3 + 32u * sn);
    const uint32_t nc1 = ld1(rp, s1 + 2u * sn), nc3 = ld1(rp, s3 + 2u * sn);
    BStep<NT> nb;
    load_b<NT>(nb, ws.xq, ws.xs, xrow, kHidden, sn, h);
    const v8i A1 = a_operand(a1), A3 = a_operand(a3);
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const v8i B = b_operand(b.lo[j], b.hi[j]);
      g[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(A1, B, g[j], 4, 0, 0, int(c1), 0, int(b.sc[j]));
      u[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(A3, B, u[j], 4, 0, 0, int(c3), 0, int(b.sc[j]));
    }
    a1 = na1;
    a3 = na3;
    c1 = nc1;
    c3 = nc3;
    b = nb;
  }
  mfma_settle<NT>(g);
  mfma_settle<NT>(u);
  // epilogue: lane (col, h) holds rows 8q + 4h + v (q, v = 0..3) of token col
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    float hv[16];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      hv[i] = swiglu_exact(g[j][i], u[j][i]);
      amax = fabsf(hv[i]) > amax ? fabsf(hv[i]) : amax;
    }
    const float other = __shfl_xor(amax, 32);  // the other 16 rows of the column
    amax = other > amax ? other : amax;
    const uint32_t code = requant_code(amax);
    const float inv = __uint_as_float((254u - code) << 23);
    const uint32_t i_tok = 32u * j + col;
    if (i_tok >= it.count) continue;
    const uint32_t p = it.first + i_tok;
    uint8_t *dst = ws.hq + size_t(p) * kInter + 64u * (rt >> 1);
    const uint32_t blk = rt & 1u;  // this tile's 32 rows are group rt of phase 2's K
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      uint32_t word = 0;
#pragma unroll
      for (int v = 0; v < 4; ++v) word |= e4m3_rne_sat(__fmul_rn(hv[4 * q4 + v], inv)) << (8 * v);
      const uint32_t r0 = 8u * q4 + 4u * h;  // first of 4 consecutive rows (k of the group)
      const uint32_t pos = r0 < 16u ? 16u * blk + r0 : 32u + 16u * blk + (r0 - 16u);
      *reinterpret_cast<uint32_t *>(dst + pos) = word;
    }
    if (h == 0) ws.hs[size_t(p) * (kInter / kQGroup) + rt] = uint8_t(code);
  }
}

__global__ __launch_bounds__(64) void k_prefill_up(PrefillArgs a, PrefillWorkspace ws) {
  const uint32_t n_items = ws.stats[0];
  if (blockIdx.y >= n_items) return;
  const PrefillItem it = ws.items[blockIdx.y];
  const uint32_t nt = (it.count + 31) / 32;
  if (nt <= 1)
    prefill_up_tiles<1>(a, ws, it, blockIdx.x);
  else if (nt == 2)
    prefill_up_tiles<2>(a, ws, it, blockIdx.x);
  else if (nt == 3)
    prefill_up_tiles<3>(a, ws, it, blockIdx.x);
  else
    prefill_up_tiles<4>(a, ws, it, blockIdx.x);
}

// Phase 2: one wavefront per (32-row tile of w2, work item): down rows of
// every pair of the item, f32, route weight not applied.
template <int NT>
__device__ __forceinline__ void prefill_down_tiles(const PrefillArgs &a, const PrefillWorkspace &ws,
                                                   const PrefillItem &it, uint32_t rt) {
  const uint32_t lane = threadIdx.x & 63, col = lane & 31, h = lane >> 5;
  const Rsrc rp = page_rsrc(a, it.expert);
  const uint32_t row = rt * 32u + col;
  const uint32_t w2 = uint32_t(a.mx.w2) + row * (kInter / 2) + 16u * h;
  const uint32_t s2 = uint32_t(a.mx.s2) + row * (kInter / 32) + h;
  uint32_t prow[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const uint32_t i = 32u * j + col;
    prow[j] = it.first + (i < it.count ? i : 0u);
  }
  v16f d[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j)
#pragma unroll
    for (int i = 0; i < 16; ++i) d[j][i] = 0.0f;
  uint4 aw = ld16(rp, w2);
  uint32_t cw = ld1(rp, s2);
  BStep<NT> b;
  load_b<NT>(b, ws.hq, ws.hs, prow, kInter, 0, h);
  constexpr uint32_t kSteps = kInter / 64;
  for (uint32_t s = 0; s < kSteps; ++s) {
    const uint32_t sn = s + 1 < kSteps ? s + 1 : s;
    const uint4 naw = ld16(rp, w2 + 32u * sn);
    const uint32_t ncw = ld1(rp, s2 + 2u * sn);
    BStep<NT> nb;
    load_b<NT>(nb, ws.hq, ws.hs, prow, kInter, sn, h);
    const v8i A = a_operand(aw);
#pragma unroll
    for (int j = 0; j < NT; ++j)
      d[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(A, b_operand(b.lo[j], b.hi[j]), d[j], 4, 0, 0, int(cw),
                                                              0, int(b.sc[j]));
    aw = naw;
    cw = ncw;
    b = nb;
  }
  mfma_settle<NT>(d);
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const uint32_t i_tok = 32u * j + col;
    if (i_tok >= it.count) continue;
    float *dst = ws.down + size_t(it.first + i_tok) * kHidden + rt * 32u;
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4)
      *reinterpret_cast<float4 *>(dst + 8u * q4 + 4u * h) =
          make_float4(d[j][4 * q4], d[j][4 * q4 + 1], d[j][4 * q4 + 2], d[j][4 * q4 + 3]);
  }
}

__global__ __launch_bounds__(64) void k_prefill_down(PrefillArgs a, PrefillWorkspace ws) {
  const uint32_t n_items = ws.stats[0];
  if (blockIdx.y >= n_items) return;
  const PrefillItem it = ws.items[blockIdx.y];
  const uint32_t nt = (it.count + 31) / 32;
  if (nt <= 1)
    prefill_down_tiles<1>(a, ws, it, blockIdx.x);
  else if (nt == 2)
    prefill_down_tiles<2>(a, ws, it, blockIdx.x);
  else if (nt == 3)
    prefill_down_tiles<3>(a, ws, it, blockIdx.x);
  else
    prefill_down_tiles<4>(a, ws, it, blockIdx.x);
}

// y[t] = 0; y += w_s * down_s in route order; y += shared down
// (s14_vulkan_numeric.rs:929-946).  One thread per (token, 4 features).
__global__ __launch_bounds__(256) void k_prefill_combine(PrefillArgs a, PrefillWorkspace ws) {
  const uint32_t gid = blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= a.tokens * (kHidden / 4)) return;
  const uint32_t t = gid / (kHidden / 4), r = 4u * (gid % (kHidden / 4));
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (uint32_t s = 0; s <= a.r.topk; ++s) {
    const uint32_t p = ws.token_pair[t * kSlots + s];
    const float4 d = *reinterpret_cast<const float4 *>(ws.down + size_t(p) * kHidden + r);
    if (s < a.r.topk) {
      const float w = ws.weights[t * kTopK + s];
      acc.x = __fadd_rn(acc.x, __fmul_rn(w, d.x));
      acc.y = __fadd_rn(acc.y, __fmul_rn(w, d.y));
      acc.z = __fadd_rn(acc.z, __fmul_rn(w, d.z));
      acc.w = __fadd_rn(acc.w, __fmul_rn(w, d.w));
    } else {
      acc.x = __fadd_rn(acc.x, d.x);
      acc.y = __fadd_rn(acc.y, d.y);
      acc.z = __fadd_rn(acc.z, d.z);
      acc.w = __fadd_rn(acc.w, d.w);
    }
  }
  *reinterpret_cast<float4 *>(a.y + size_t(t) * kHidden + r) = acc;
}

}  // namespace

hipError_t launch_requant_e4m3(hipStream_t s, uint32_t rows, uint32_t k, const float *x, uint8_t *q,
                               uint8_t *scales) {
  const uint32_t n = rows * (k / kQGroup);
  k_requant_rows<<<(n + 255) / 256, 256, 0, s>>>(rows, k, x, q, scales);
  return hipGetLastError();
}

hipError_t launch_prefill(hipStream_t s, const PrefillArgs &a, const PrefillWorkspace &ws) {
  const uint32_t T = a.tokens;
  // scores of every (token, expert)
  Workspace rws{};
  rws.scores = ws.scores;
  rws.biased = ws.biased;
  hipError_t e = launch_router_scores(s, rws, a.r, T, a.x);
  if (e != hipSuccess) return e;
  const uint32_t nbits = kMaxExperts * kPrefillBitWords;
  k_zero_u32<<<(nbits + 255) / 256, 256, 0, s>>>(nbits, ws.token_bits);
  k_prefill_topk<<<(T + 3) / 4, 256, 0, s>>>(a, ws);
  k_prefill_group<<<1, 1024, 0, s>>>(a, ws);
  k_requant_x<<<(T * (kHidden / kQGroup) + 255) / 256, 256, 0, s>>>(T, a.x, ws.xq, ws.xs);
  const uint32_t max_items = prefill_max_items(T);
  k_prefill_up<<<dim3(kInter / 32, max_items), 64, 0, s>>>(a, ws);
  k_prefill_down<<<dim3(kHidden / 32, max_items), 64, 0, s>>>(a, ws);
  k_prefill_combine<<<(T * (kHidden / 4) + 255) / 256, 256, 0, s>>>(a, ws);
  return hipGetLastError();
}

}  // namespace s14
