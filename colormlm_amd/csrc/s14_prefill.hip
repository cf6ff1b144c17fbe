// Prefill through the S14 MoE layer (config 4) on gfx950: T tokens, each
// routed to its top-k experts plus the shared expert, computed per expert as
// grouped GEMMs on the CDNA4 bf16 MFMA (v_mfma_f32_16x16x32_bf16): MXFP4
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
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include "s14_device.hpp"
#include "s14_device_util.hpp"
#include "s14_e4m3.h"
#include "s14_prefill.hpp"

namespace s14 {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));
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

// Both GEMMs run on v_mfma_f32_16x16x32_bf16 over 16-column halves of a work
// item's (up to 32) columns, in super-steps of 128 k.  Operand layout, lane
// l = c + 16 q (c = 0..15, q = 0..3): in MFMA j (0..3) of a super-step, lane
// l supplies row c of A and column c of B at the super-step's k values 32 q
// + 8 j .. +7 (8 bf16 each); D element v of lane l is row 4 q + v, column c.
// A lane's 32 k of a super-step are one E8M0 block of A's row (16 weight
// bytes, one LDS read) and of B's column.  Every column of every item goes
// through the same MFMA sequence, so a token's outputs do not depend on the
// item, or the item's width, the grouping gave it.  An item of at most
// kNarrowTokens pairs runs one half: most experts get a few tokens, and one
// half does half the MFMA work, activation loads and activation conversions
// of a 32-column tile.  Wider items run two halves that share each decoded
// A operand.
constexpr uint32_t kSuperK = 128;                          // k per super-step
constexpr uint32_t kChunkSupers = kChunkSteps * 64 / kSuperK;  // super-steps per chunk: 2

// Each work item's x rows into the item's tile: tile[super-step][half][plane
// p][lane][16 bytes], lane = c + 16 q holding the e4m3 codes of k 32 q + 16 p
// .. +15 of the super-step for column 16 half + c; scales [chunk][half][lane]
// u32, byte u = the E8M0 of super-step kChunkSupers * chunk + u for the
// lane's block q.  Columns past the item's count are not written: the GEMMs
// never read them.  One thread per 16 tile bytes; the plane-0 thread of a
// chunk's first super-step also writes that chunk's scale word.
__global__ __launch_bounds__(256) void k_tile_x(PrefillWorkspace ws) {
  constexpr uint32_t kPerItem = kXTileBytes / 16;
  const uint32_t gid = blockIdx.x * 256u + threadIdx.x;
  const uint32_t i = gid / kPerItem;
  if (i >= ws.stats[0]) return;
  const uint32_t r = gid % kPerItem;
  const uint32_t lane = r & 63u, p = (r >> 6) & 1u, half = (r >> 7) & 1u, u = r >> 8;
  const uint32_t col = 16u * half + (lane & 15u), q = lane >> 4;
  const PrefillItem it = ws.items[i];
  if (col >= it.count) return;
  const uint32_t t = ws.pair_token[it.first + col];
  *reinterpret_cast<uint4 *>(ws.xt + size_t(i) * kXTileBytes + 16u * r) =
      *reinterpret_cast<const uint4 *>(ws.xq + size_t(t) * kHidden + kSuperK * u + 32u * q + 16u * p);
  if (p == 0 && u % kChunkSupers == 0) {
    uint32_t word = 0;
    const uint8_t *sc = ws.xs + size_t(t) * (kHidden / kQGroup) + 4u * u + q;  // group 4 (u + k) + q
#pragma unroll
    for (uint32_t k = 0; k < kChunkSupers; ++k) word |= uint32_t(sc[4u * k]) << (8u * k);
    reinterpret_cast<uint32_t *>(ws.xts + size_t(i) * kXScaleBytes)[((u / kChunkSupers) * 2u + half) * 64u + lane] =
        word;
  }
}

// A page of 0 (an expert that is not resident) reads the shared page instead
// (mapped memory); the top-k step gave its pairs a NaN weight and set the
// status word.
// The address is read back through readfirstlane: it is uniform, and with
// the GEMMs' two column-half paths the compiler otherwise kept it in VGPRs
// and wrapped every DMA load in a loop over its lanes' descriptors.
__device__ __forceinline__ Rsrc page_rsrc(const PrefillArgs &a, uint32_t e) {
  const uint8_t *page = e < kMaxExperts ? reinterpret_cast<const uint8_t *>(a.expert_pages[e]) : a.shared_page;
  if (!page) page = a.shared_page;
  const uint64_t pv = reinterpret_cast<uint64_t>(page);
  const uint64_t lo = uint32_t(__builtin_amdgcn_readfirstlane(int(uint32_t(pv))));
  const uint64_t hi = uint32_t(__builtin_amdgcn_readfirstlane(int(uint32_t(pv >> 32))));
  return make_rsrc(reinterpret_cast<const uint8_t *>(lo | (hi << 32)), uint32_t(S14_EXPERT_PAGE_BYTES));
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
// A lane's activations of one half and one super-step (k 32 q .. 32 q + 31
// of its column: planes 0 and 1, one E8M0 block) as the B operands of MFMAs
// j = 0..3.
struct BStep {
  v8bf b[4];
};
__device__ __forceinline__ BStep b_step(uint4 p0, uint4 p1, uint32_t code) {
  const float s = e8m0_operand(code);
  return BStep{{fp8x8_bf16(p0.x, p0.y, s), fp8x8_bf16(p0.z, p0.w, s), fp8x8_bf16(p1.x, p1.y, s),
                fp8x8_bf16(p1.z, p1.w, s)}};
}
// A lane's 16 weight bytes of one super-step (k 32 q .. 32 q + 31 of its
// row, one E8M0 block) as the A operands of MFMAs j = 0..3.
struct AStep {
  v8bf a[4];
};
__device__ __forceinline__ AStep a_step(uint4 w, uint32_t code) {
  const float s = e8m0_operand(code);
  return AStep{{fp4x8_bf16(w.x, s), fp4x8_bf16(w.y, s), fp4x8_bf16(w.z, s), fp4x8_bf16(w.w, s)}};
}
// acc += A . B over one super-step of a 16x16 tile: exact products, f32
// accumulation.
__device__ __forceinline__ v4f mfma_step(const AStep &a, const BStep &b, v4f acc) {
#pragma unroll
  for (int j = 0; j < 4; ++j) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.a[j], b.b[j], acc, 0, 0, 0);
  return acc;
}

// Pins the accumulators in uniform control flow.  The epilogues store only
// columns < count, a per-lane condition; without this the compiler may sink
// the last K step's MFMA into that branch, and an MFMA issued under a partial
// EXEC mask does not take the inactive lanes' A rows and scales (their output
// rows come back as garbage).
template <int NT>
__device__ __forceinline__ void mfma_settle(v4f (&acc)[NT]) {
#pragma unroll
  for (int j = 0; j < NT; ++j) asm volatile("" : "+a"(acc[j]));
}

// Weight operand through LDS.  A wavefront streams its weight tile in chunks
// of kChunkSteps 64-k steps (128 bytes of each row): the DMA form of the
// buffer load (buffer_load_dwordx4 ... lds) writes each chunk into a ring
// slot with 8 lanes per row, so every quarter-wave reads 256 contiguous bytes
// of two rows; each MFMA lane then reads its row's 16-byte piece of a
// super-step from LDS.  Loading the MFMA layout straight from HBM instead
// has each quarter-wave touch 16 rows: the vector L1 then handles one
// 64-byte sector per 16 useful bytes and, not HBM, bounds the kernel.  Row
// r's piece q sits at piece q ^ swz(r) of its 128 bytes, so the 16 rows of a
// read pass land in distinct banks.  Each slot is its own LDS array, which
// lets the compiler wait for one slot's DMA loads without draining the
// others.
__device__ __forceinline__ uint32_t swz(uint32_t r) { return (r + (r >> 3)) & 7u; }
// The same for the phase-2 scale tile (64-byte rows, 4 pieces).
__device__ __forceinline__ uint32_t swz4(uint32_t r) { return (r + (r >> 2)) & 3u; }

constexpr uint32_t kUpSlotBytes = 2 * 32 * 128;  // w1 and w3 chunks
// w2 rows per phase-2 wavefront: four 16-row MFMA tiles sharing each
// activation operand (with 32 rows a wavefront read twice as many activation
// bytes as weight bytes: 249 us for the down GEMM at 512 tokens against 220
// us with 64; 128 measured no faster)
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
// its last use, from the item tile (two coalesced 1 KiB loads per super-step
// and half).
constexpr int kRing = 4;
template <int NH>
struct BChunk {
  uint4 v[NH][kChunkSupers][2];  // [half][super-step][plane]
  uint32_t sc[NH];               // byte u: scale of super-step u for this lane's block
};
// Lanes of columns past the item's count read from past the descriptor's
// range: the buffer load returns zeros without a memory access, so a work
// item moves only its pairs' activations.
constexpr uint32_t kOffRange = 0x40000000u;
template <int NH>
struct BBase {
  uint32_t tile[NH], scale[NH];
};
template <int NH>
__device__ __forceinline__ BBase<NH> b_base(uint32_t lane, uint32_t count) {
  BBase<NH> b;
#pragma unroll
  for (int h = 0; h < NH; ++h) {
    const bool live = 16u * uint32_t(h) + (lane & 15u) < count;
    b.tile[h] = live ? 2048u * uint32_t(h) + 16u * lane : kOffRange;
    b.scale[h] = live ? 256u * uint32_t(h) + 4u * lane : kOffRange;
  }
  return b;
}
template <int NH>
__device__ __forceinline__ void load_bchunk(BChunk<NH> &b, Rsrc tile, Rsrc scales, uint32_t c, const BBase<NH> &bb) {
#pragma unroll
  for (uint32_t u = 0; u < kChunkSupers; ++u)
#pragma unroll
    for (int h = 0; h < NH; ++h)
#pragma unroll
      for (uint32_t p = 0; p < 2; ++p)
        b.v[h][u][p] = ld16(tile, bb.tile[h] + 4096u * (c * kChunkSupers + u) + 1024u * p);
#pragma unroll
  for (int h = 0; h < NH; ++h) b.sc[h] = ld4(scales, bb.scale[h] + 512u * c);
}

// Phase 2's item tile (ht, hts) in the x tile's layout: the byte offset of
// the codes of rows 16 p .. 16 p + 15 of block b of super-step u (phase 2's
// K positions kSuperK u + 32 b + 16 p ..) for column col, and of the scale
// byte of (u, b) for column col.
__device__ __forceinline__ uint32_t h_tile_offset(uint32_t u, uint32_t b, uint32_t p, uint32_t col) {
  return 4096u * u + 2048u * (col >> 4) + 1024u * p + 16u * ((col & 15u) + 16u * b);
}
__device__ __forceinline__ uint32_t h_scale_offset(uint32_t u, uint32_t b, uint32_t col) {
  return (((u / kChunkSupers) * 2u + (col >> 4)) * 64u + (col & 15u) + 16u * b) * 4u + u % kChunkSupers;
}

// Phase 1: one wavefront per (32-row tile of w1/w3, work item of <= 32
// pairs of one expert), NH column halves.  K = 4096 in 16 chunks; weights
// kRing - 1 chunks ahead in LDS, activations kRing chunks ahead in VGPRs.
// Then h = swiglu(g, u), requantised per token over the tile's 32 rows (one
// E8M0 group of phase 2's K) and stored into the item's phase-2 tile.
// kOfficial: h = bf16(swiglu(bf16(g), bf16(u)) * w), w the pair's route
// weight (1 for the shared expert) (executor.py:717-731), stored in f32 for
// k_requant_h128 (its group of 128 rows spans four of these workgroups).
template <bool kOfficial, int NH>
__device__ __forceinline__ void prefill_up_item(const PrefillArgs &a, const PrefillWorkspace &ws,
                                                const PrefillItem &it, uint32_t item, const Rsrc rp) {
  const uint32_t rt = blockIdx.x;
  const uint32_t lane = threadIdx.x & 63, c16 = lane & 15u, q = lane >> 4;
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
  const BBase<NH> bb = b_base<NH>(lane, it.count);
  // expf's table for the epilogue's SwiGLUs: one entry per lane now, written
  // to a free ring slot after the K loop (an LDS array of its own would cost
  // this kernel its fourth wavefront per CU)
  const double exp_entry = s14x::exp_table_entry(lane & 31u);
  BChunk<NH> rb[kRing];
  issue(Slot<0>{}, 0);
  issue(Slot<1>{}, 1);
  issue(Slot<2>{}, 2);
#pragma unroll
  for (int j = 0; j < kRing; ++j) {
    load_bchunk(rb[j], xt, xts, uint32_t(j), bb);
    __builtin_amdgcn_sched_barrier(0);  // chunk order, so the loop's waits count the ring right
  }
  // acc[4 h + i]: g of column half h, rows 16 i .. 16 i + 15 of the tile;
  // acc[4 h + 2 + i]: u of the same
  v4f acc[4 * NH];
#pragma unroll
  for (int t = 0; t < 4 * NH; ++t) acc[t] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  const uint32_t sw[2] = {swz(c16), swz(16u + c16)};  // the lane's A rows c16 and 16 + c16
  auto chunk = [&](auto slot_tag, uint32_t c, bool refill) {
    constexpr int S = decltype(slot_tag)::value;
#pragma unroll
    for (uint32_t u = 0; u < kChunkSupers; ++u) {
      const uint32_t pc = 4u * u + q;                  // the lane's piece of the chunk row
      const uint32_t sb = kChunkSupers * 4u * c + pc;  // and its E8M0 block of the row
      AStep a1[2], a3[2];
#pragma unroll
      for (uint32_t i = 0; i < 2; ++i) {
        const uint32_t R = 16u * i + c16;
        const uint8_t *src = up_slot<S>() + 128u * R + 16u * (pc ^ sw[i]);
        const uint32_t sp = 128u * R + 16u * ((sb >> 4) ^ sw[i]) + (sb & 15u);
        a1[i] = a_step(*reinterpret_cast<const uint4 *>(src), up_scales[sp]);
        a3[i] = a_step(*reinterpret_cast<const uint4 *>(src + 4096u), up_scales[4096u + sp]);
      }
#pragma unroll
      for (int h = 0; h < NH; ++h) {
        const BStep B = b_step(rb[S].v[h][u][0], rb[S].v[h][u][1], (rb[S].sc[h] >> (8u * u)) & 0xffu);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          acc[4 * h + i] = mfma_step(a1[i], B, acc[4 * h + i]);
          acc[4 * h + 2 + i] = mfma_step(a3[i], B, acc[4 * h + 2 + i]);
        }
      }
    }
    if (refill) load_bchunk(rb[S], xt, xts, c + kRing, bb);
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
  mfma_settle(acc);
  double *exptab = reinterpret_cast<double *>(up_slot0);  // slot 0's last chunk is consumed
  if (lane < 32) exptab[lane] = exp_entry;
  __syncthreads();  // one wavefront: orders the table writes before the lookups
  // epilogue: lane (c16, q) holds rows 16 i + 4 q + v (i = 0, 1; v = 0..3)
  // of column 16 h + c16 in element v of acc[4 h + i] (g) and acc[4 h + 2 + i] (u)
  if constexpr (kOfficial) {
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      const uint32_t col = 16u * uint32_t(h) + c16;
      if (col >= it.count) continue;
      const uint32_t pair = it.first + col;
      const float w = ws.pair_weight[pair];
      float *dst = ws.hf + size_t(pair) * kInter + rt * 32u;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        float o[4];
#pragma unroll
        for (int v = 0; v < 4; ++v)
          o[v] = bf16_round(
              __fmul_rn(swiglu_exact(bf16_round(acc[4 * h + i][v]), bf16_round(acc[4 * h + 2 + i][v]), exptab), w));
        *reinterpret_cast<float4 *>(dst + 16u * uint32_t(i) + 4u * q) = make_float4(o[0], o[1], o[2], o[3]);
      }
    }
    return;
  }
  // this tile's 32 rows are block rt % 4 of phase 2's super-step rt / 4
  // (one E8M0 group), read by lane (col % 16) + 16 (rt % 4) of the column's half
  const uint32_t u2 = rt >> 2, b2 = rt & 3u;
#pragma unroll
  for (int h = 0; h < NH; ++h) {
    float hv[8];
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      hv[e] = swiglu_exact(acc[4 * h + e / 4][e % 4], acc[4 * h + 2 + e / 4][e % 4], exptab);
      amax = fabsf(hv[e]) > amax ? fabsf(hv[e]) : amax;
    }
    // the column's other 24 rows: the lanes of the other three blocks
#pragma unroll
    for (int m = 16; m < 64; m <<= 1) {
      const float other = __shfl_xor(amax, m);
      amax = other > amax ? other : amax;
    }
    const uint32_t code = requant_code(amax);
    const float inv = __uint_as_float((254u - code) << 23);
    const uint32_t col = 16u * uint32_t(h) + c16;
    if (col >= it.count) continue;  // phase 2 never reads absent columns
#pragma unroll
    for (int i = 0; i < 2; ++i) {  // rows 16 i + 4 q .. +3: plane i, bytes 4 q .. 4 q + 3
      uint32_t word = 0;
#pragma unroll
      for (int v = 0; v < 4; ++v) word |= e4m3_rne_sat(__fmul_rn(hv[4 * i + v], inv)) << (8 * v);
      *reinterpret_cast<uint32_t *>(ws.ht + size_t(item) * kHTileBytes + h_tile_offset(u2, b2, uint32_t(i), col) +
                                    4u * q) = word;
    }
    if (q == 0) ws.hts[size_t(item) * kHScaleBytes + h_scale_offset(u2, b2, col)] = uint8_t(code);
  }
}

template <bool kOfficial>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(1, 1))) void k_prefill_up(PrefillArgs a,
                                                                                                PrefillWorkspace ws) {
  const uint32_t n_items = ws.stats[0];
  const uint32_t item = blockIdx.y;
  if (item >= n_items) return;
  const PrefillItem it = ws.items[item];
  const Rsrc rp = page_rsrc(a, it.expert);
  if (uint32_t(__builtin_amdgcn_readfirstlane(int(it.count))) <= kNarrowTokens)
    prefill_up_item<kOfficial, 1>(a, ws, it, item, rp);
  else
    prefill_up_item<kOfficial, 2>(a, ws, it, item, rp);
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
  // group m is phase 2's super-step m: piece j is plane j % 2 of block j / 2
  *reinterpret_cast<uint4 *>(ws.ht + size_t(item) * kHTileBytes + h_tile_offset(m, j >> 1, j & 1u, col)) =
      make_uint4(w[0], w[1], w[2], w[3]);
  if ((j & 1u) == 0) ws.hts[size_t(item) * kHScaleBytes + h_scale_offset(m, j >> 1, col)] = uint8_t(code);
}

// Phase 2: one wavefront per (64-row tile of w2, work item): down rows of
// every pair of the item, f32, route weight not applied, as four 16-row
// MFMA tiles per column half, each decoded A operand shared by the halves
// and each activation operand by the four tiles.  K = 2048 in 8 chunks, the
// same rings as phase 1.  kOfficial: rounded to bf16.
template <bool kOfficial, int NH>
__device__ __forceinline__ void prefill_down_item(const PrefillArgs &a, const PrefillWorkspace &ws,
                                                  const PrefillItem &it, uint32_t item, const Rsrc rp) {
  const uint32_t rt = blockIdx.x;  // 64-row tile
  const uint32_t lane = threadIdx.x & 63, c16 = lane & 15u, q = lane >> 4;
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
  const BBase<NH> bb = b_base<NH>(lane, it.count);
  BChunk<NH> rb[kRing];
  issue(Slot<0>{}, 0);
  issue(Slot<1>{}, 1);
  issue(Slot<2>{}, 2);
#pragma unroll
  for (int j = 0; j < kRing; ++j) {
    load_bchunk(rb[j], ht, hts, uint32_t(j), bb);
    __builtin_amdgcn_sched_barrier(0);  // chunk order, so the loop's waits count the ring right
  }
  constexpr int NT = int(kDnRows / 16);  // row tiles
  v4f d[NH * NT];                        // d[NT h + tl]: column half h, rows 16 tl .. 16 tl + 15
#pragma unroll
  for (int t = 0; t < NH * NT; ++t) d[t] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  // the lane's rows 16 tl + c16, one per tile
  uint32_t sw[NT], s4[NT];
#pragma unroll
  for (int tl = 0; tl < NT; ++tl) {
    sw[tl] = swz(16u * uint32_t(tl) + c16);
    s4[tl] = swz4(16u * uint32_t(tl) + c16);
  }
  auto chunk = [&](auto slot_tag, uint32_t c, bool refill) {
    constexpr int S = decltype(slot_tag)::value;
    const uint8_t *src = dn_slot<S>();
#pragma unroll
    for (uint32_t u = 0; u < kChunkSupers; ++u) {
      const uint32_t pc = 4u * u + q;                  // the lane's piece of the chunk row
      const uint32_t sb = kChunkSupers * 4u * c + pc;  // and its E8M0 block of the row
      BStep B[NH];
#pragma unroll
      for (int h = 0; h < NH; ++h) B[h] = b_step(rb[S].v[h][u][0], rb[S].v[h][u][1], (rb[S].sc[h] >> (8u * u)) & 0xffu);
#pragma unroll
      for (int tl = 0; tl < NT; ++tl) {
        const uint32_t r = 16u * uint32_t(tl) + c16;
        const uint4 aw = *reinterpret_cast<const uint4 *>(src + 128u * r + 16u * (pc ^ sw[tl]));
        const AStep A = a_step(aw, dn_scales[64u * r + 16u * ((sb >> 4) ^ s4[tl]) + (sb & 15u)]);
#pragma unroll
        for (int h = 0; h < NH; ++h) d[NT * h + tl] = mfma_step(A, B[h], d[NT * h + tl]);
      }
    }
    if (refill) load_bchunk(rb[S], ht, hts, c + kRing, bb);
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
  mfma_settle(d);
  // lane (c16, q) holds rows 16 tl + 4 q + v of column 16 h + c16 in element v of d[NT h + tl]
#pragma unroll
  for (int h = 0; h < NH; ++h) {
    const uint32_t col = 16u * uint32_t(h) + c16;
    if (col >= it.count) continue;
    float *dst = ws.down + size_t(it.first + col) * kHidden + rt * kDnRows + 4u * q;
#pragma unroll
    for (int tl = 0; tl < NT; ++tl) {
      const v4f v = d[NT * h + tl];
      float4 o = make_float4(v[0], v[1], v[2], v[3]);
      if constexpr (kOfficial) o = make_float4(bf16_round(o.x), bf16_round(o.y), bf16_round(o.z), bf16_round(o.w));
      *reinterpret_cast<float4 *>(dst + 16u * uint32_t(tl)) = o;
    }
  }
}

template <bool kOfficial>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(1, 1))) void k_prefill_down(PrefillArgs a,
                                                                                                  PrefillWorkspace ws) {
  const uint32_t n_items = ws.stats[0];
  const uint32_t item = blockIdx.y;
  if (item >= n_items) return;
  const PrefillItem it = ws.items[item];
  const Rsrc rp = page_rsrc(a, it.expert);
  if (uint32_t(__builtin_amdgcn_readfirstlane(int(it.count))) <= kNarrowTokens)
    prefill_down_item<kOfficial, 1>(a, ws, it, item, rp);
  else
    prefill_down_item<kOfficial, 2>(a, ws, it, item, rp);
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
