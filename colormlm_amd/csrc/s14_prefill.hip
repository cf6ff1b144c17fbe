// Prefill through the S14 MoE layer (config 4) on gfx950: T tokens, each
// routed to its top-k experts plus the shared expert, computed per expert as
// grouped GEMMs on the CDNA4 bf16 MFMA (v_mfma_f32_32x32x16_bf16): MXFP4
// weights (A, E8M0 per 32 k) and e4m3-requantised activations (B, E8M0 per
// 32 k) are decoded to bf16 in registers by the gfx950 scaled converters,
// exactly (an e2m1 value has two significant bits, an e4m3 value four, the
// E8M0 scale is a power of two), so every product is exact in f32 and only
// the f32 accumulation order differs from the CPU oracle's sequential sum.
//
// There is no reference GPU code for this row; its semantics are the layer's
// (s14_vulkan_numeric.rs:929-946 accumulation, :1543-1556 SwiGLU) with the
// activation requant the north-star config names (e4m3 RNE, saturating,
// per-32 scale 2^ceil(log2(max(amax, 1e-4) / 448)), l42_reference.py:390-403
// with group 32).  Its tolerance against the CPU oracle is measured
// (tests/test_gpu_parity.py).
//
// The gfx950 scaled MFMA (v_mfma_scale_f32_32x32x64_f8f6f4) would take the
// MXFP4 and e4m3 operands undecoded, but it sums each 64-k step at its own
// internal precision (it returns 256 * 256 + 1 * 1 as 65,536 when the two
// products share a step): GEMM results 5.7e-5 of the output's scale away
// from the oracle's, against 8e-7 here.
//
// Operand layout of v_mfma_f32_32x32x16_bf16 (lane l, half h = l / 32):
// A is row l % 32, B column l % 32, each 8 bf16 at k 8h..8h+7 of the MFMA's
// 16; D element i of lane l is row 8(i/4) + 4h + i%4, column l % 32.  A 64-k
// step is four MFMAs: in MFMA j, lane half h supplies k 32h + 8j .. +7 of
// the step, so a lane's 16 weight bytes (k 32h..32h+31 of its row, one
// E8M0 block) and its column's 32 activations at the same k (one E8M0
// block) feed it.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include "s14_device.hpp"
#include "s14_device_util.hpp"
#include "s14_e4m3.h"
#include "s14_prefill.hpp"

namespace s14 {
namespace {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

constexpr uint32_t kQGroup = 32;  // requant group (k values per E8M0 scale)

// ---------------------------------------------------------------------------
// requant (bit-identical to the oracle's s14o_requant_e4m3)
// ---------------------------------------------------------------------------

using s14x::e4m3_rne_sat;  // s14_e4m3.h: straight-line, checked against the oracle on the CPU

// The activation requant X [T, 4096] f32 -> Q [T, 4096] e4m3 + S [T, 128]
// E8M0 (requant_x_group) runs in extra workgroups of the router's launch
// (launch_router_scores), beside the scoring it does not depend on.

// ---------------------------------------------------------------------------
// routing and grouping
// ---------------------------------------------------------------------------

// One wavefront per token: top-k, route weights, and the expert's token bit.
__global__ __launch_bounds__(256) void k_prefill_topk(PrefillArgs a, PrefillWorkspace ws) {
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t t = blockIdx.x * 4u + (threadIdx.x >> 6);
  if (t >= a.tokens) return;
  const uint32_t k = a.r.topk;
  const float *bt = ws.biased + size_t(t) * kMaxExperts, *st = ws.scores + size_t(t) * kMaxExperts;
  bool bad = false;
  const TopK c = a.r.tid2eid ? select_hash_from(PlainScoreLoad{bt, st, nullptr}, a.r, t, bad)
                             : select_topk(bt, st, nullptr, a.r.n_experts, k);
  float w = lane < k ? route_weight(c, a.r.route_scale) : 0.0f;
  bad = bad || !route_weights_valid(w, k, a.r.route_scale);
  if (bad && lane == 0) __hip_atomic_fetch_or(a.status, kStatusBadRoute, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (lane < k) {
    // a route that fails validate_for takes distinct placeholder experts
    // with NaN weights
    const uint32_t id = bad ? lane : c.id;
    if (bad) w = __builtin_nanf("");
    // the pairs of an expert without a resident page combine with a NaN
    // weight (their GEMM tiles read the shared page instead)
    const bool resident = a.expert_pages[id] != 0ull;
    if (!resident) __hip_atomic_fetch_or(a.status, kStatusNullPage, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    ws.ids[t * kTopK + lane] = id;
    ws.weights[t * kTopK + lane] = resident ? w : __builtin_nanf("");
    if (a.ids_out) a.ids_out[t * k + lane] = uint16_t(id);
    if (a.weights_out) a.weights_out[t * k + lane] = w;
    atomicOr(&ws.token_bits[id * kPrefillBitWords + (t >> 5)], 1u << (t & 31));
  }
}

// One workgroup: per-expert token counts from the bitmaps, pair offsets
// (experts ascending, the shared expert last), each pair's token in token
// order within its expert, and the GEMM work items (<= kItemTokens tokens of
// one expert each).  Deterministic: positions come from bit counts.
__global__ __launch_bounds__(1024) void k_prefill_group(PrefillArgs a, PrefillWorkspace ws) {
  __shared__ uint32_t bits[kMaxExperts][kPrefillBitWords];  // the token bitmaps, read once
  __shared__ uint16_t below[kMaxExperts][kPrefillBitWords];  // tokens of the expert in words < w
  __shared__ uint32_t cnt[kMaxExperts + 1];
  __shared__ uint32_t off[kMaxExperts + 2];
  __shared__ uint32_t items_of[kMaxExperts + 1];
  __shared__ uint32_t item_off[kMaxExperts + 2];
  const uint32_t tid = threadIdx.x;
  const uint32_t T = a.tokens, words = (T + 31) / 32;
  // read the bitmaps and leave them clear for the next call's top-k (the
  // workspace starts clear), which saves a clearing launch per call; all of
  // a thread's loads are issued before the first is used
  constexpr uint32_t kBitIters = kMaxExperts * kPrefillBitWords / 1024;
  static_assert(kMaxExperts * kPrefillBitWords % 1024 == 0, "whole sweeps of the 1024 threads");
  uint32_t bv[kBitIters];
#pragma unroll
  for (uint32_t j = 0; j < kBitIters; ++j) {
    const uint32_t i = tid + 1024u * j;
    bv[j] = i % kPrefillBitWords < words ? ws.token_bits[i] : 0u;
  }
#pragma unroll
  for (uint32_t j = 0; j < kBitIters; ++j) {
    const uint32_t i = tid + 1024u * j, w = i % kPrefillBitWords;
    if (w < words) ws.token_bits[i] = 0u;
    bits[i / kPrefillBitWords][w] = bv[j];
  }
  __syncthreads();
  for (uint32_t e = tid; e <= kMaxExperts; e += blockDim.x) {
    uint32_t c = 0;
    if (e < kMaxExperts) {
      for (uint32_t w = 0; w < words; ++w) {
        below[e][w] = uint16_t(c);
        c += __popc(bits[e][w]);
      }
    } else {
      c = T;  // shared expert: every token
    }
    cnt[e] = c;
    items_of[e] = (c + kItemTokens - 1) / kItemTokens;
  }
  __syncthreads();
  if (tid < 64) {
    // exclusive scans of the 257 counts and item counts by one wavefront:
    // lane l sums experts 5l .. 5l+4, then an inclusive scan over lanes
    constexpr uint32_t kPer = (kMaxExperts + 1 + 63) / 64;  // 5
    uint32_t c[kPer], n[kPer], sc = 0, sn = 0, distinct = 0, mx = 0;
#pragma unroll
    for (uint32_t j = 0; j < kPer; ++j) {
      const uint32_t e = kPer * tid + j;
      c[j] = e <= kMaxExperts ? cnt[e] : 0u;
      n[j] = e <= kMaxExperts ? items_of[e] : 0u;
      sc += c[j];
      sn += n[j];
      if (e < kMaxExperts && c[j]) {
        ++distinct;
        mx = c[j] > mx ? c[j] : mx;
      }
    }
    uint32_t ic = sc, in = sn;
#pragma unroll
    for (uint32_t d = 1; d < 64; d <<= 1) {
      const uint32_t pc = __shfl_up(ic, d), pn = __shfl_up(in, d);
      if (tid >= d) {
        ic += pc;
        in += pn;
      }
    }
    uint32_t oc = ic - sc, on = in - sn;  // exclusive starts of this lane's experts
#pragma unroll
    for (uint32_t j = 0; j < kPer; ++j) {
      const uint32_t e = kPer * tid + j;
      if (e <= kMaxExperts) {
        off[e] = oc;
        item_off[e] = on;
      }
      oc += c[j];
      on += n[j];
    }
    for (uint32_t m = 32; m >= 1; m >>= 1) {
      distinct += __shfl_xor(distinct, m);
      const uint32_t o = __shfl_xor(mx, m);
      mx = o > mx ? o : mx;
    }
    if (tid == 63) {
      off[kMaxExperts + 1] = ic;
      item_off[kMaxExperts + 1] = in;
      ws.stats[0] = in;  // number of work items
      ws.stats[1] = distinct;
      ws.stats[2] = mx;
      ws.stats[3] = ic;  // number of pairs
    }
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
  // pairs: routed (token t, slot s) -> position = tokens of the expert below
  // t; the token's ids and weights loaded before the first is used
  for (uint32_t t = tid; t < T; t += blockDim.x) {
    uint32_t ids[kTopK];
    float wts[kTopK];
#pragma unroll
    for (uint32_t s = 0; s < uint32_t(kTopK); ++s) {
      ids[s] = s < a.r.topk ? ws.ids[t * kTopK + s] : 0u;
      wts[s] = s < a.r.topk ? ws.weights[t * kTopK + s] : 0.0f;
    }
#pragma unroll
    for (uint32_t s = 0; s < uint32_t(kTopK); ++s) {
      if (s >= a.r.topk) break;
      const uint32_t e = ids[s];
      const uint32_t rank = below[e][t >> 5] + __popc(bits[e][t >> 5] & ((1u << (t & 31)) - 1u));
      const uint32_t p = off[e] + rank;
      ws.pair_token[p] = t;
      ws.token_pair[t * kSlots + s] = p;
      ws.pair_weight[p] = wts[s];
    }
    const uint32_t ps = off[kMaxExperts] + t;
    ws.pair_token[ps] = t;
    ws.token_pair[t * kSlots + a.r.topk] = ps;
    ws.pair_weight[ps] = 1.0f;
  }
}

// ---------------------------------------------------------------------------
// grouped GEMMs
// ---------------------------------------------------------------------------

// Each work item's x rows into the item's tile.
// Columns past the item's count are not written: the GEMMs never read them.
// One thread per 16 tile bytes; the thread holding part 0 of the first step
// of a chunk also writes that chunk's scale word.
__global__ __launch_bounds__(256) void k_tile_x(PrefillWorkspace ws) {
  constexpr uint32_t kPerItem = kXTileBytes / 16;
  const uint32_t gid = blockIdx.x * 256u + threadIdx.x;
  const uint32_t i = gid / kPerItem;
  if (i >= ws.stats[0]) return;
  const uint32_t r = gid % kPerItem;
  const uint32_t lane = r & 63u, part = (r >> 6) & 1u, s = r >> 7;
  const uint32_t col = lane & 31u, h = lane >> 5;
  const PrefillItem it = ws.items[i];
  if (col >= it.count) return;
  const uint32_t t = ws.pair_token[it.first + col];
  *reinterpret_cast<uint4 *>(ws.xt + size_t(i) * kXTileBytes + 16u * r) =
      *reinterpret_cast<const uint4 *>(ws.xq + size_t(t) * kHidden + 64u * s + 32u * h + 16u * part);
  if (part == 0 && s % kChunkSteps == 0) {
    uint32_t word = 0;
    const uint8_t *sc = ws.xs + size_t(t) * (kHidden / kQGroup) + 2u * s + h;  // group 2 (s + k) + h
#pragma unroll
    for (uint32_t k = 0; k < kChunkSteps; ++k) word |= uint32_t(sc[2u * k]) << (8u * k);
    reinterpret_cast<uint32_t *>(ws.xts + size_t(i) * kXScaleBytes)[(s / kChunkSteps) * 64u + lane] = word;
  }
}

// A page of 0 (an expert that is not resident) reads the shared page instead
// (mapped memory); the top-k step gave its pairs a NaN weight and set the
// status word.
__device__ __forceinline__ Rsrc page_rsrc(const PrefillArgs &a, uint32_t e) {
  const uint8_t *page = e < kMaxExperts ? reinterpret_cast<const uint8_t *>(a.expert_pages[e]) : a.shared_page;
  if (!page) page = a.shared_page;
  return make_rsrc(page, uint32_t(S14_EXPERT_PAGE_BYTES));
}

// E8M0 code c as the scale operand of the gfx950 scaled converters (they
// take only its exponent field: 2^(c-127), code 0 included).
__device__ __forceinline__ float e8m0_operand(uint32_t c) { return __uint_as_float(c << 23); }

// Eight fp4 (four bytes, low nibble first: k ascending) times 2^(c-127) as
// eight bf16, exact.
__device__ __forceinline__ v8bf fp4x8_bf16(uint32_t w, float s) {
  const v4u v = {__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, s, 0)),
                 __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, s, 1)),
                 __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, s, 2)),
                 __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, s, 3))};
  return __builtin_bit_cast(v8bf, v);
}
// Eight e4m3 (two words, byte order = k order) times 2^(c-127) as eight
// bf16, exact.
__device__ __forceinline__ v8bf fp8x8_bf16(uint32_t w0, uint32_t w1, float s) {
  const v4u v = {__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, s, false)),
                 __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, s, true)),
                 __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, s, false)),
                 __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, s, true))};
  return __builtin_bit_cast(v8bf, v);
}
// One 64-k step of a lane's activations (lo: k 32h..32h+15 of the step, hi:
// k 32h+16..32h+31, one E8M0 block) as the B operands of the step's four
// MFMAs: MFMA j takes k 32h+8j..32h+8j+7.
struct BStep {
  v8bf b[4];
};
__device__ __forceinline__ BStep b_step(uint4 lo, uint4 hi, uint32_t code) {
  const float s = e8m0_operand(code);
  return BStep{{fp8x8_bf16(lo.x, lo.y, s), fp8x8_bf16(lo.z, lo.w, s), fp8x8_bf16(hi.x, hi.y, s),
                fp8x8_bf16(hi.z, hi.w, s)}};
}
// acc += A . B over one 64-k step: the lane's 16 weight bytes (k 32h..32h+31
// of its row, one E8M0 block) decoded exactly to bf16 against the step's
// activations, four MFMAs (exact products, f32 accumulation).
__device__ __forceinline__ v16f mfma_step(uint4 w, uint32_t code, const BStep &b, v16f acc) {
  const float s = e8m0_operand(code);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fp4x8_bf16(w.x, s), b.b[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fp4x8_bf16(w.y, s), b.b[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fp4x8_bf16(w.z, s), b.b[2], acc, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(fp4x8_bf16(w.w, s), b.b[3], acc, 0, 0, 0);
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

// Weight operand through LDS.  A wavefront streams its 32-row weight tile in
// chunks of kChunkSteps K steps (128 bytes of each row): the DMA form of the
// buffer load (buffer_load_dwordx4 ... lds) writes each chunk into a ring
// slot with 8 lanes per row, so every quarter-wave reads 256 contiguous bytes
// of two rows; the MFMA then reads one 16-byte piece of 32 rows from LDS.
// Loading the MFMA layout straight from HBM instead has each quarter-wave
// touch 16 rows: the vector L1 then handles one 64-byte sector per 16 useful
// bytes and, not HBM, bounds the kernel.  Row r's piece q sits at piece
// q ^ swz(r) of its 128 bytes, so the 16 rows of a read pass land in
// distinct banks.  Each slot is its own LDS array, which lets the compiler
// wait for one slot's DMA loads without draining the others.
__device__ __forceinline__ uint32_t swz(uint32_t r) { return (r + (r >> 3)) & 7u; }
// The same for the phase-2 scale tile (64-byte rows, 4 pieces).
__device__ __forceinline__ uint32_t swz4(uint32_t r) { return (r + (r >> 2)) & 3u; }

constexpr uint32_t kUpSlotBytes = 2 * 32 * 128;  // w1 and w3 chunks
// w2 rows per phase-2 wavefront: two 32-row MFMA tiles sharing each
// activation operand (with one tile a wavefront read twice as many
// activation bytes as weight bytes: 249 us for the down GEMM at 512 tokens
// against 220 us; four tiles measured no faster)
constexpr uint32_t kDnRows = 64;
constexpr uint32_t kDnSlotBytes = kDnRows * 128;  // w2 chunk
__shared__ __attribute__((aligned(16))) uint8_t up_slot0[kUpSlotBytes];
__shared__ __attribute__((aligned(16))) uint8_t up_slot1[kUpSlotBytes];
__shared__ __attribute__((aligned(16))) uint8_t up_slot2[kUpSlotBytes];
__shared__ __attribute__((aligned(16))) uint8_t up_slot3[kUpSlotBytes];
__shared__ __attribute__((aligned(16))) uint8_t up_scales[2 * 32 * (kHidden / 32)];  // s1, s3 of the tile
__shared__ __attribute__((aligned(16))) uint8_t dn_slot0[kDnSlotBytes];
__shared__ __attribute__((aligned(16))) uint8_t dn_slot1[kDnSlotBytes];
__shared__ __attribute__((aligned(16))) uint8_t dn_slot2[kDnSlotBytes];
__shared__ __attribute__((aligned(16))) uint8_t dn_slot3[kDnSlotBytes];
__shared__ __attribute__((aligned(16))) uint8_t dn_scales[kDnRows * (kInter / 32)];  // s2 of the tile

template <int S>
struct Slot {
  static constexpr int value = S;
};
template <int S>
__device__ __forceinline__ uint8_t *up_slot() {
  if constexpr (S == 0) return up_slot0;
  else if constexpr (S == 1) return up_slot1;
  else if constexpr (S == 2) return up_slot2;
  else return up_slot3;
}
template <int S>
__device__ __forceinline__ uint8_t *dn_slot() {
  if constexpr (S == 0) return dn_slot0;
  else if constexpr (S == 1) return dn_slot1;
  else if constexpr (S == 2) return dn_slot2;
  else return dn_slot3;
}

typedef __attribute__((address_space(3))) void lds_void;
__device__ __forceinline__ void dma16(Rsrc r, uint8_t *lds, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)(lds), 16, off, 0, 0, 0);
}
// Before a DMA load refills a slot: the LDS reads of its previous chunk
// have returned (they fed MFMAs already issued; this makes it explicit).
__device__ __forceinline__ void lds_reads_done() { __builtin_amdgcn_s_waitcnt(0xc07f); }

// Activation operand: a VGPR ring of kRing chunks, each refilled right after
// its last use, from the item tile (two coalesced 1 KiB loads per step).
constexpr int kRing = 4;
struct BChunk {
  uint4 lo[kChunkSteps], hi[kChunkSteps];
  uint32_t sc;  // byte k: scale of step k for this lane's half
};
// Lanes of columns past the item's count read from past the descriptor's
// range: the buffer load returns zeros without a memory access, so a work
// item moves only its pairs' activations (items average ~13 of 32 columns).
constexpr uint32_t kOffRange = 0x40000000u;
__device__ __forceinline__ uint32_t bcol_base(uint32_t lane, bool live) { return live ? 16u * lane : kOffRange; }
__device__ __forceinline__ uint32_t bscale_base(uint32_t lane, bool live) { return live ? 4u * lane : kOffRange; }
__device__ __forceinline__ void load_bchunk(BChunk &b, Rsrc tile, Rsrc scales, uint32_t c, uint32_t tbase,
                                            uint32_t sbase) {
#pragma unroll
  for (uint32_t k = 0; k < kChunkSteps; ++k) {
    const uint32_t s = c * kChunkSteps + k;
    b.lo[k] = ld16(tile, tbase + 2048u * s);
    b.hi[k] = ld16(tile, tbase + 2048u * s + 1024u);
  }
  b.sc = ld4(scales, sbase + c * 256u);
}

// Phase 1: one wavefront per (32-row tile of w1/w3, work item of <= 32
// pairs of one expert).  K = 4096 in 16 chunks; weights kRing - 1 chunks
// ahead in LDS, activations kRing chunks ahead in VGPRs.  Then h =
// swiglu(g, u), requantised per token over the tile's 32 rows (one E8M0
// group of phase 2's K) and stored into the item's phase-2 tile.
// kOfficial: h = bf16(swiglu(bf16(g), bf16(u)) * w), w the pair's route
// weight (1 for the shared expert) (executor.py:717-731), stored in f32 for
// k_requant_h128 (its group of 128 rows spans four of these workgroups).
template <bool kOfficial>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(1, 1))) void k_prefill_up(PrefillArgs a,
                                                                                                PrefillWorkspace ws) {
  const uint32_t n_items = ws.stats[0];
  const uint32_t item = blockIdx.y;
  if (item >= n_items) return;
  const PrefillItem it = ws.items[item];
  const uint32_t rt = blockIdx.x;
  const uint32_t lane = threadIdx.x & 63, col = lane & 31, h = lane >> 5;
  const Rsrc rp = page_rsrc(a, it.expert);
  constexpr uint32_t kRowBytes = kHidden / 2, kScaleRow = kHidden / 32;
  constexpr uint32_t kChunks = kHidden / 64 / kChunkSteps;
  // DMA lane map: load j of a chunk covers rows 8j..8j+7 of the tile, lane
  // -> row 8j + lane/8, piece (lane % 8) ^ swz(row) (swz(8j + r) = (j + r) % 8)
  const uint32_t lrow = lane >> 3;
  uint32_t dma_off[4];
#pragma unroll
  for (uint32_t j = 0; j < 4; ++j)
    dma_off[j] = (rt * 32u + 8u * j + lrow) * kRowBytes + 16u * ((lane & 7u) ^ ((j + lrow) & 7u));
  const uint32_t w1 = uint32_t(a.mx.w1), w3 = uint32_t(a.mx.w3);
  auto issue = [&](auto slot_tag, uint32_t c) {
    uint8_t *dst = up_slot<decltype(slot_tag)::value>();
    lds_reads_done();
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) {
      dma16(rp, dst + 1024u * j, w1 + dma_off[j] + 128u * c);
      dma16(rp, dst + 4096u + 1024u * j, w3 + dma_off[j] + 128u * c);
    }
  };
  // the tile's scales, whole K: 32 rows x 128 bytes per matrix, same swizzle
#pragma unroll
  for (uint32_t j = 0; j < 4; ++j) {
    const uint32_t so = (rt * 32u + 8u * j + lrow) * kScaleRow + 16u * ((lane & 7u) ^ ((j + lrow) & 7u));
    dma16(rp, up_scales + 1024u * j, uint32_t(a.mx.s1) + so);
    dma16(rp, up_scales + 4096u + 1024u * j, uint32_t(a.mx.s3) + so);
  }
  const Rsrc xt = make_rsrc(ws.xt + size_t(item) * kXTileBytes, kXTileBytes);
  const Rsrc xts = make_rsrc(ws.xts + size_t(item) * kXScaleBytes, kXScaleBytes);
  const bool live = col < it.count;
  const uint32_t tb = bcol_base(lane, live), sbb = bscale_base(lane, live);
  // expf's table for the epilogue's 16 SwiGLUs per lane: one entry per lane
  // now, written to a free ring slot after the K loop (an LDS array of its
  // own would cost this kernel its fourth wavefront per CU)
  const double exp_entry = s14x::exp_table_entry(lane & 31u);
  BChunk rb[kRing];
  issue(Slot<0>{}, 0);
  issue(Slot<1>{}, 1);
  issue(Slot<2>{}, 2);
#pragma unroll
  for (int j = 0; j < kRing; ++j) {
    load_bchunk(rb[j], xt, xts, uint32_t(j), tb, sbb);
    __builtin_amdgcn_sched_barrier(0);  // chunk order, so the loop's waits count the ring right
  }
  v16f g, u;
#pragma unroll
  for (int i = 0; i < 16; ++i) g[i] = u[i] = 0.0f;
  const uint32_t sw = swz(col);
  auto chunk = [&](auto slot_tag, uint32_t c, bool refill) {
    constexpr int S = decltype(slot_tag)::value;
    const uint8_t *src = up_slot<S>() + 128u * col;
#pragma unroll
    for (uint32_t k = 0; k < kChunkSteps; ++k) {
      const uint32_t q = (2u * k + h) ^ sw;
      const uint4 a1 = *reinterpret_cast<const uint4 *>(src + 16u * q);
      const uint4 a3 = *reinterpret_cast<const uint4 *>(src + 4096u + 16u * q);
      const uint32_t sb = 2u * (c * kChunkSteps + k) + h;  // scale byte of this lane's weight block
      const uint32_t sp = 128u * col + 16u * ((sb >> 4) ^ sw) + (sb & 15u);
      const uint32_t c1 = up_scales[sp], c3 = up_scales[4096u + sp];
      const BStep B = b_step(rb[S].lo[k], rb[S].hi[k], (rb[S].sc >> (8u * k)) & 0xffu);
      g = mfma_step(a1, c1, B, g);
      u = mfma_step(a3, c3, B, u);
    }
    if (refill) load_bchunk(rb[S], xt, xts, c + kRing, tb, sbb);
    // keep the refill here: left free, the scheduler sinks loads to the end
    // of the loop body, and the next round's first wait then drains the ring
    __builtin_amdgcn_sched_barrier(0);
  };
  static_assert(kRing == 4 && kChunks % 4 == 0 && kChunks >= 8, "four ring slots, whole rounds");
  // Every round but the last refills unconditionally, so the ring stays in
  // fixed registers across the back edge.
#pragma unroll 1
  for (uint32_t c = 0; c + 4 < kChunks; c += 4) {
    issue(Slot<3>{}, c + 3);
    chunk(Slot<0>{}, c, true);
    issue(Slot<0>{}, c + 4);
    chunk(Slot<1>{}, c + 1, true);
    issue(Slot<1>{}, c + 5);
    chunk(Slot<2>{}, c + 2, true);
    issue(Slot<2>{}, c + 6);
    chunk(Slot<3>{}, c + 3, true);
  }
  issue(Slot<3>{}, kChunks - 1);
  chunk(Slot<0>{}, kChunks - 4, false);
  chunk(Slot<1>{}, kChunks - 3, false);
  chunk(Slot<2>{}, kChunks - 2, false);
  chunk(Slot<3>{}, kChunks - 1, false);
  v16f acc[2] = {g, u};
  mfma_settle<2>(acc);
  g = acc[0];
  u = acc[1];
  // epilogue: lane (col, h) holds rows 8q + 4h + v (q, v = 0..3) of column col
  double *exptab = reinterpret_cast<double *>(up_slot0);  // slot 0's last chunk is consumed
  if (lane < 32) exptab[lane] = exp_entry;
  __syncthreads();  // one wavefront: orders the table writes before the lookups
  if constexpr (kOfficial) {
    if (col >= it.count) return;
    const uint32_t pair = it.first + col;
    const float w = ws.pair_weight[pair];
    float *dst = ws.hf + size_t(pair) * kInter + rt * 32u;
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      float o[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int i = 4 * q4 + v;
        o[v] = bf16_round(__fmul_rn(swiglu_exact(bf16_round(g[i]), bf16_round(u[i]), exptab), w));
      }
      *reinterpret_cast<float4 *>(dst + 8u * q4 + 4u * h) = make_float4(o[0], o[1], o[2], o[3]);
    }
    return;
  }
  float hv[16];
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    hv[i] = swiglu_exact(g[i], u[i], exptab);
    amax = fabsf(hv[i]) > amax ? fabsf(hv[i]) : amax;
  }
  const float other = __shfl_xor(amax, 32);  // the other 16 rows of the column
  amax = other > amax ? other : amax;
  const uint32_t code = requant_code(amax);
  const float inv = __uint_as_float((254u - code) << 23);
  if (col >= it.count) return;  // phase 2 never reads absent columns
  // this tile's 32 rows are half blk of phase 2's K step s2 (group rt)
  const uint32_t s2 = rt >> 1, blk = rt & 1u;
  uint8_t *tile = ws.ht + size_t(item) * kHTileBytes + 2048u * s2;
#pragma unroll
  for (int q4 = 0; q4 < 4; ++q4) {
    uint32_t word = 0;
#pragma unroll
    for (int v = 0; v < 4; ++v) word |= e4m3_rne_sat(__fmul_rn(hv[4 * q4 + v], inv)) << (8 * v);
    const uint32_t pos = 32u * blk + 8u * q4 + 4u * h;  // k in the step of the first of 4 consecutive rows
    *reinterpret_cast<uint32_t *>(tile + 1024u * ((pos >> 4) & 1u) + 16u * (col + 32u * (pos >> 5)) + (pos & 15u)) =
        word;
  }
  if (h == 0) ws.hts[size_t(item) * kHScaleBytes + ((s2 / kChunkSteps) * 64u + col + 32u * blk) * 4u + s2 % kChunkSteps] =
      uint8_t(code);
}

// Official mode: the w2 input's act_quant (group 128) of every work item's
// h columns into the item's phase-2 tile and scales, in the layout
// k_prefill_up's epilogue writes otherwise (tile rt holds rows 32 rt .. +31,
// half rt % 2 of K step rt / 2).  Eight lanes per (item, column, 128 rows),
// each lane 16 rows (64 contiguous bytes in, one 16-byte piece out); the
// group's maximum by xor shuffles within the eight.
constexpr uint32_t kHGroups128 = kInter / 128;
__global__ __launch_bounds__(256) void k_requant_h128(PrefillWorkspace ws) {
  const uint32_t gid = blockIdx.x * 256u + threadIdx.x;
  const uint32_t j = gid & 7u, grp = gid >> 3;  // 16-row piece j of group grp = (item, column, m)
  const uint32_t item = grp / (kItemTokens * kHGroups128);
  if (item >= ws.stats[0]) return;  // whole groups of eight lanes return together
  const uint32_t col = (grp / kHGroups128) % kItemTokens, m = grp % kHGroups128;
  const PrefillItem it = ws.items[item];
  if (col >= it.count) return;  // phase 2 never reads absent columns
  const float4 *src =
      reinterpret_cast<const float4 *>(ws.hf + size_t(it.first + col) * kInter + 128u * m + 16u * j);
  float4 q[4];
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    q[i] = src[i];
    amax = fabsf(q[i].x) > amax ? fabsf(q[i].x) : amax;
    amax = fabsf(q[i].y) > amax ? fabsf(q[i].y) : amax;
    amax = fabsf(q[i].z) > amax ? fabsf(q[i].z) : amax;
    amax = fabsf(q[i].w) > amax ? fabsf(q[i].w) : amax;
  }
#pragma unroll
  for (int d = 1; d < 8; d <<= 1) {  // NaN never compares greater, as in the scan above
    const float o = __shfl_xor(amax, d);
    amax = o > amax ? o : amax;
  }
  const uint32_t code = requant_code(amax);
  const float inv = __uint_as_float((254u - code) << 23);
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    w[i] = e4m3_rne_sat(__fmul_rn(q[i].x, inv)) | (e4m3_rne_sat(__fmul_rn(q[i].y, inv)) << 8) |
           (e4m3_rne_sat(__fmul_rn(q[i].z, inv)) << 16) | (e4m3_rne_sat(__fmul_rn(q[i].w, inv)) << 24);
  const uint32_t rt = 4u * m + j / 2u, s2 = rt >> 1, blk = rt & 1u;
  const uint32_t pos = 32u * blk + 16u * (j & 1u);  // k in the step of the piece's first row
  uint8_t *tile = ws.ht + size_t(item) * kHTileBytes;
  *reinterpret_cast<uint4 *>(tile + 2048u * s2 + 1024u * ((pos >> 4) & 1u) + 16u * (col + 32u * (pos >> 5))) =
      make_uint4(w[0], w[1], w[2], w[3]);
  if (j < 4u) {  // the scale byte of tile 4m + j
    const uint32_t rs = 4u * m + j, ss = rs >> 1, bs = rs & 1u;
    ws.hts[size_t(item) * kHScaleBytes + ((ss / kChunkSteps) * 64u + col + 32u * bs) * 4u + ss % kChunkSteps] =
        uint8_t(code);
  }
}

// Phase 2: one wavefront per (64-row tile of w2, work item): down rows of
// every pair of the item, f32, route weight not applied, as two 32-row
// MFMA tiles that share each activation operand.  K = 2048 in 8 chunks, the
// same rings as phase 1.  kOfficial: rounded to bf16.
template <bool kOfficial>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(1, 1))) void k_prefill_down(PrefillArgs a,
                                                                                                  PrefillWorkspace ws) {
  const uint32_t n_items = ws.stats[0];
  const uint32_t item = blockIdx.y;
  if (item >= n_items) return;
  const PrefillItem it = ws.items[item];
  const uint32_t rt = blockIdx.x;  // 64-row tile
  const uint32_t lane = threadIdx.x & 63, col = lane & 31, h = lane >> 5;
  const Rsrc rp = page_rsrc(a, it.expert);
  constexpr uint32_t kRowBytes = kInter / 2, kScaleRow = kInter / 32;
  constexpr uint32_t kChunks = kInter / 64 / kChunkSteps;
  constexpr uint32_t kDma = kDnRows / 8;  // DMA loads per chunk: 8 rows each
  const uint32_t lrow = lane >> 3;
  uint32_t dma_off[kDma];
#pragma unroll
  for (uint32_t j = 0; j < kDma; ++j)
    dma_off[j] =
        uint32_t(a.mx.w2) + (rt * kDnRows + 8u * j + lrow) * kRowBytes + 16u * ((lane & 7u) ^ ((j + lrow) & 7u));
  auto issue = [&](auto slot_tag, uint32_t c) {
    uint8_t *dst = dn_slot<decltype(slot_tag)::value>();
    lds_reads_done();
#pragma unroll
    for (uint32_t j = 0; j < kDma; ++j) dma16(rp, dst + 1024u * j, dma_off[j] + 128u * c);
  };
  // scales: 64 rows x 64 bytes; load j covers rows 16j..16j+15, 4 lanes a row
#pragma unroll
  for (uint32_t j = 0; j < kDnRows / 16; ++j) {
    const uint32_t row = 16u * j + (lane >> 2);
    dma16(rp, dn_scales + 1024u * j,
          uint32_t(a.mx.s2) + (rt * kDnRows + row) * kScaleRow + 16u * ((lane & 3u) ^ swz4(row)));
  }
  const Rsrc ht = make_rsrc(ws.ht + size_t(item) * kHTileBytes, kHTileBytes);
  const Rsrc hts = make_rsrc(ws.hts + size_t(item) * kHScaleBytes, kHScaleBytes);
  const bool live = col < it.count;
  const uint32_t tb = bcol_base(lane, live), sbb = bscale_base(lane, live);
  BChunk rb[kRing];
  issue(Slot<0>{}, 0);
  issue(Slot<1>{}, 1);
  issue(Slot<2>{}, 2);
#pragma unroll
  for (int j = 0; j < kRing; ++j) {
    load_bchunk(rb[j], ht, hts, uint32_t(j), tb, sbb);
    __builtin_amdgcn_sched_barrier(0);  // chunk order, so the loop's waits count the ring right
  }
  constexpr int NT = int(kDnRows / 32);  // MFMA tiles
  v16f d[NT];
#pragma unroll
  for (int tl = 0; tl < NT; ++tl)
#pragma unroll
    for (int i = 0; i < 16; ++i) d[tl][i] = 0.0f;
  // the lane's rows 32 tl + col, one per tile
  uint32_t sw[NT], s4[NT];
#pragma unroll
  for (int tl = 0; tl < NT; ++tl) {
    sw[tl] = swz(32u * uint32_t(tl) + col);
    s4[tl] = swz4(32u * uint32_t(tl) + col);
  }
  auto chunk = [&](auto slot_tag, uint32_t c, bool refill) {
    constexpr int S = decltype(slot_tag)::value;
    const uint8_t *src = dn_slot<S>();
#pragma unroll
    for (uint32_t k = 0; k < kChunkSteps; ++k) {
      const uint32_t p = 2u * k + h;
      const uint32_t sb = 2u * (c * kChunkSteps + k) + h;
      const BStep B = b_step(rb[S].lo[k], rb[S].hi[k], (rb[S].sc >> (8u * k)) & 0xffu);
#pragma unroll
      for (int tl = 0; tl < NT; ++tl) {
        const uint32_t r = 32u * uint32_t(tl) + col;
        const uint4 aw = *reinterpret_cast<const uint4 *>(src + 128u * r + 16u * (p ^ sw[tl]));
        const uint32_t ca = dn_scales[64u * r + 16u * ((sb >> 4) ^ s4[tl]) + (sb & 15u)];
        d[tl] = mfma_step(aw, ca, B, d[tl]);
      }
    }
    if (refill) load_bchunk(rb[S], ht, hts, c + kRing, tb, sbb);
    __builtin_amdgcn_sched_barrier(0);  // as in phase 1
  };
  static_assert(kRing == 4 && kChunks % 4 == 0 && kChunks >= 8, "four ring slots, whole rounds");
#pragma unroll 1
  for (uint32_t c = 0; c + 4 < kChunks; c += 4) {
    issue(Slot<3>{}, c + 3);
    chunk(Slot<0>{}, c, true);
    issue(Slot<0>{}, c + 4);
    chunk(Slot<1>{}, c + 1, true);
    issue(Slot<1>{}, c + 5);
    chunk(Slot<2>{}, c + 2, true);
    issue(Slot<2>{}, c + 6);
    chunk(Slot<3>{}, c + 3, true);
  }
  issue(Slot<3>{}, kChunks - 1);
  chunk(Slot<0>{}, kChunks - 4, false);
  chunk(Slot<1>{}, kChunks - 3, false);
  chunk(Slot<2>{}, kChunks - 2, false);
  chunk(Slot<3>{}, kChunks - 1, false);
  mfma_settle<NT>(d);
  if (col >= it.count) return;
#pragma unroll
  for (int tl = 0; tl < NT; ++tl) {
    float *dst = ws.down + size_t(it.first + col) * kHidden + rt * kDnRows + 32u * uint32_t(tl);
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      float4 o = make_float4(d[tl][4 * q4], d[tl][4 * q4 + 1], d[tl][4 * q4 + 2], d[tl][4 * q4 + 3]);
      if constexpr (kOfficial) o = make_float4(bf16_round(o.x), bf16_round(o.y), bf16_round(o.z), bf16_round(o.w));
      *reinterpret_cast<float4 *>(dst + 8u * q4 + 4u * h) = o;
    }
  }
}

// y[t] = 0; y += w_s * down_s in route order; y += shared down
// (s14_vulkan_numeric.rs:929-946).  One thread per (token, 4 features).
// kOfficial: the route weights are already in h; y = bf16(sum of the bf16
// outputs in route order, shared last, in f32) (executor.py:712-739).
template <bool kOfficial>
__global__ __launch_bounds__(256) void k_prefill_combine(PrefillArgs a, PrefillWorkspace ws) {
  const uint32_t gid = blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= a.tokens * (kHidden / 4)) return;
  const uint32_t t = gid / (kHidden / 4), r = 4u * (gid % (kHidden / 4));
  // the token's pair indices and weights in one round trip, then every slot's
  // down row in a second (all loads issued before the first add)
  const uint32_t k = a.r.topk;  // <= kTopK; slot k is the shared expert
  uint32_t pr[kSlots];
  float wt[kTopK];
#pragma unroll
  for (uint32_t s = 0; s < uint32_t(kSlots); ++s) pr[s] = s <= k ? ws.token_pair[t * kSlots + s] : 0u;
#pragma unroll
  for (uint32_t s = 0; s < uint32_t(kTopK); ++s) wt[s] = s < k ? ws.weights[t * kTopK + s] : 0.0f;
  float4 d[kSlots];
#pragma unroll
  for (uint32_t s = 0; s < uint32_t(kSlots); ++s)
    d[s] = s <= k ? *reinterpret_cast<const float4 *>(ws.down + size_t(pr[s]) * kHidden + r)
                  : make_float4(0.f, 0.f, 0.f, 0.f);
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (uint32_t s = 0; s < uint32_t(kSlots); ++s) {
    if (s > k) break;
    if (s < k && !kOfficial) {
      acc.x = __fadd_rn(acc.x, __fmul_rn(wt[s], d[s].x));
      acc.y = __fadd_rn(acc.y, __fmul_rn(wt[s], d[s].y));
      acc.z = __fadd_rn(acc.z, __fmul_rn(wt[s], d[s].z));
      acc.w = __fadd_rn(acc.w, __fmul_rn(wt[s], d[s].w));
    } else {
      acc.x = __fadd_rn(acc.x, d[s].x);
      acc.y = __fadd_rn(acc.y, d[s].y);
      acc.z = __fadd_rn(acc.z, d[s].z);
      acc.w = __fadd_rn(acc.w, d[s].w);
    }
  }
  if constexpr (kOfficial) acc = make_float4(bf16_round(acc.x), bf16_round(acc.y), bf16_round(acc.z), bf16_round(acc.w));
  *reinterpret_cast<float4 *>(a.y + size_t(t) * kHidden + r) = acc;
}

}  // namespace

hipError_t launch_prefill(hipStream_t s, const PrefillArgs &a, const PrefillWorkspace &ws) {
  const uint32_t T = a.tokens;
  // scores of every (token, expert)
  Workspace rws{};
  rws.scores = ws.scores;
  rws.biased = ws.biased;
  hipError_t e = launch_router_scores(s, rws, a.r, T, a.x, {}, a.official ? 2 : 1, ws.xq, ws.xs);
  if (e != hipSuccess) return e;
  k_prefill_topk<<<(T + 3) / 4, 256, 0, s>>>(a, ws);
  k_prefill_group<<<1, 1024, 0, s>>>(a, ws);
  const uint32_t max_items = prefill_max_items(T);
  k_tile_x<<<max_items * (kXTileBytes / 16 / 256), 256, 0, s>>>(ws);
  const uint32_t cb_blocks = (T * (kHidden / 4) + 255) / 256;
  if (a.official) {
    k_prefill_up<true><<<dim3(kInter / 32, max_items), 64, 0, s>>>(a, ws);
    k_requant_h128<<<max_items * kItemTokens * kHGroups128 * 8u / 256u, 256, 0, s>>>(ws);
    k_prefill_down<true><<<dim3(kHidden / kDnRows, max_items), 64, 0, s>>>(a, ws);
    k_prefill_combine<true><<<cb_blocks, 256, 0, s>>>(a, ws);
  } else {
    k_prefill_up<false><<<dim3(kInter / 32, max_items), 64, 0, s>>>(a, ws);
    k_prefill_down<false><<<dim3(kHidden / kDnRows, max_items), 64, 0, s>>>(a, ws);
    k_prefill_combine<false><<<cb_blocks, 256, 0, s>>>(a, ws);
  }
  return hipGetLastError();
}

}  // namespace s14
