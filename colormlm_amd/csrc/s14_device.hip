// gfx950 (CDNA4) kernels of the S14 quantized expert path.
//
// Two reduction orders:
//   EXACT  one output row per lane, k strictly ascending, multiply then add
//          (no FMA) — the operation order of the reference CPU oracle
//          (scheduler/ssd_inference/examples/s14_vulkan_numeric.rs:1669-1714),
//          so outputs are bit-identical to it.  At batch 1 this is bound by
//          the per-lane dependent-add chain, not by HBM.
//   FAST   K split across the 64 lanes of a wavefront, products fused
//          (v_fma), cross-lane tree reduction; HBM-bound.
// The reference's five shaders (shaders/s14_*.comp) are one workgroup per
// row with a 128-way LDS tree; neither order here follows them.
//
// Build: hipcc --offload-arch=gfx950 -ffp-contract=off (contraction would
// fuse the exact kernels' multiply-then-add).
#include <hip/hip_runtime.h>

#include "s14_device.hpp"
#include "s14_expf.h"

namespace s14 {
namespace {

typedef float v2f __attribute__((ext_vector_type(2)));
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
__device__ __forceinline__ uint32_t ld4(Rsrc r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
__device__ __forceinline__ uint32_t ld1(Rsrc r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b8(r, off, 0, 0);
}
__device__ __forceinline__ float ldf(Rsrc r, uint32_t off) { return __uint_as_float(ld4(r, off)); }

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

__device__ __forceinline__ float swiglu_exact(float gate, float up) {
  // s14_vulkan_numeric.rs:1543-1556: gate.min(10) keeps -0 and maps NaN to
  // 10; clamp passes NaN through.
  const float g = (gate <= 10.0f) ? gate : 10.0f;
  float u = up;
  if (u < -10.0f) u = -10.0f;
  if (u > 10.0f) u = 10.0f;
  const float e = s14x::expf_glibc(-g);
  return __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, e)), u);
}

// ---------------------------------------------------------------------------
// wavefront reductions
// ---------------------------------------------------------------------------

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
  return v;
}
__device__ __forceinline__ int wave_min_i(int v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = min(v, __shfl_xor(v, m));
  return v;
}
__device__ __forceinline__ int wave_max_i(int v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = max(v, __shfl_xor(v, m));
  return v;
}

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
// finite); then c in [max(2, 129 - emin), 252].  Other groups take the
// literal two-multiply path.
struct CodeWindow {
  int cmin, cmax;
};
__device__ __forceinline__ CodeWindow mx_window(int emin, int emax) {
  if (emin < 2 || emax > 251) return {256, 0};
  return {max(2, 129 - emin), 252};
}

// ---------------------------------------------------------------------------
// EXACT row kernels
// ---------------------------------------------------------------------------

// One group of 32 k values (16 code bytes, one scale code) of an MXFP4 row,
// in the oracle's order: pair by pair, low nibble (even k) then high nibble.
__device__ __forceinline__ float mx_group_exact(float acc, const uint4 w, uint32_t c,
                                                const float *__restrict__ xs, CodeWindow win) {
  const float4 *x4 = reinterpret_cast<const float4 *>(xs);
  const uint32_t words[4] = {w.x, w.y, w.z, w.w};
  if (c >= uint32_t(win.cmin) && c <= uint32_t(win.cmax)) {
    const float sc = __uint_as_float(c << 23);
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const float4 xa = x4[2 * d], xb = x4[2 * d + 1];
      const v2f p0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(words[d], sc, 0);
      const v2f p1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(words[d], sc, 1);
      const v2f p2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(words[d], sc, 2);
      const v2f p3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(words[d], sc, 3);
      acc = __fadd_rn(acc, __fmul_rn(xa.x, p0.x));
      acc = __fadd_rn(acc, __fmul_rn(xa.y, p0.y));
      acc = __fadd_rn(acc, __fmul_rn(xa.z, p1.x));
      acc = __fadd_rn(acc, __fmul_rn(xa.w, p1.y));
      acc = __fadd_rn(acc, __fmul_rn(xb.x, p2.x));
      acc = __fadd_rn(acc, __fmul_rn(xb.y, p2.y));
      acc = __fadd_rn(acc, __fmul_rn(xb.z, p3.x));
      acc = __fadd_rn(acc, __fmul_rn(xb.w, p3.y));
    }
  } else {
    const float s = ue8m0_f32(c);
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const float4 xa = x4[2 * d], xb = x4[2 * d + 1];
      const float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float e = e2m1_f32((words[d] >> (4 * j)) & 15u);
        acc = __fadd_rn(acc, __fmul_rn(__fmul_rn(xv[j], e), s));
      }
    }
  }
  return acc;
}

// Dot of one MXFP4 row (G groups of 32) with x staged in LDS, k ascending.
// Code bytes live at r[woff + 16 g], scale codes at rs[soff + g]; they are
// prefetched PF groups ahead (PF * 16 B per lane in flight).
template <int PF>
__device__ __forceinline__ float mx_row_exact(float acc, Rsrc r, uint32_t woff, Rsrc rs, uint32_t soff,
                                              int G, const float *__restrict__ xs, CodeWindow win) {
  static_assert(PF % 4 == 0, "scale words hold 4 codes");
  uint4 cur[PF];
  uint32_t cs[PF / 4];
#pragma unroll
  for (int i = 0; i < PF; ++i) cur[i] = ld16(r, woff + 16u * i);
#pragma unroll
  for (int j = 0; j < PF / 4; ++j) cs[j] = ld4(rs, soff + 4u * j);
  for (int g0 = 0; g0 < G; g0 += PF) {
    uint4 nxt[PF];
    uint32_t ns[PF / 4];
    const bool more = (g0 + PF) < G;
    if (more) {
#pragma unroll
      for (int i = 0; i < PF; ++i) nxt[i] = ld16(r, woff + 16u * (g0 + PF + i));
#pragma unroll
      for (int j = 0; j < PF / 4; ++j) ns[j] = ld4(rs, soff + uint32_t(g0 + PF) + 4u * j);
    }
#pragma unroll
    for (int i = 0; i < PF; ++i)
      acc = mx_group_exact(acc, cur[i], (cs[i >> 2] >> (8 * (i & 3))) & 255u, xs + (g0 + i) * 32, win);
    if (more) {
#pragma unroll
      for (int i = 0; i < PF; ++i) cur[i] = nxt[i];
#pragma unroll
      for (int j = 0; j < PF / 4; ++j) cs[j] = ns[j];
    }
  }
  return acc;
}

// Dot of one FP8 row with x in LDS: sum += (x * e4m3) * scale, k ascending
// (s14_vulkan_numeric.rs:1698-1714).  Codes at rw[woff + k]; the row's tile
// scales (ceil(K/128) of them, ue8m0 bytes or f32) at rs[soff + ...].
// K16: K % 16 == 0 and woff % 16 == 0.
template <bool K16>
__device__ __forceinline__ float fp8_row_exact(float acc, Rsrc rw, uint32_t woff, Rsrc rs, uint32_t soff,
                                               int scale_f32, int K, const float *__restrict__ xs) {
  if (K16) {
    uint4 cur = ld16(rw, woff);
    for (int k0 = 0; k0 < K; k0 += 16) {
      uint4 nxt = cur;
      if (k0 + 16 < K) nxt = ld16(rw, woff + uint32_t(k0) + 16u);
      const uint32_t t = uint32_t(k0 >> 7);
      const float s = scale_f32 ? ldf(rs, soff + 4u * t) : ue8m0_f32(ld1(rs, soff + t));
      const uint32_t words[4] = {cur.x, cur.y, cur.z, cur.w};
      const float4 *x4 = reinterpret_cast<const float4 *>(xs + k0);
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const float4 xv = x4[d];
        const v2f lo = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(words[d], 1.0f, false);
        const v2f hi = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(words[d], 1.0f, true);
        acc = __fadd_rn(acc, __fmul_rn(__fmul_rn(xv.x, lo.x), s));
        acc = __fadd_rn(acc, __fmul_rn(__fmul_rn(xv.y, lo.y), s));
        acc = __fadd_rn(acc, __fmul_rn(__fmul_rn(xv.z, hi.x), s));
        acc = __fadd_rn(acc, __fmul_rn(__fmul_rn(xv.w, hi.y), s));
      }
      cur = nxt;
    }
  } else {
    for (int k = 0; k < K; ++k) {
      const uint32_t t = uint32_t(k >> 7);
      const float s = scale_f32 ? ldf(rs, soff + 4u * t) : ue8m0_f32(ld1(rs, soff + t));
      acc = __fadd_rn(acc, __fmul_rn(__fmul_rn(xs[k], e4m3_f32(ld1(rw, woff + uint32_t(k)))), s));
    }
  }
  return acc;
}

// Stage n f32 (n % 4 == 0) from global to LDS with the whole block, and
// return the block-uniform exponent range (1-wave blocks only).
__device__ __forceinline__ void stage_f32_range(float *dst, const float *__restrict__ src, int n,
                                                int &emin, int &emax) {
  int lo = 255, hi = 0;
  for (int i = int(threadIdx.x) * 4; i < n; i += int(blockDim.x) * 4) {
    const float4 v = *reinterpret_cast<const float4 *>(src + i);
    *reinterpret_cast<float4 *>(dst + i) = v;
    exp_range_acc(v.x, lo, hi);
    exp_range_acc(v.y, lo, hi);
    exp_range_acc(v.z, lo, hi);
    exp_range_acc(v.w, lo, hi);
  }
  emin = wave_min_i(lo);
  emax = wave_max_i(hi);
  __syncthreads();
}

constexpr int kExactChunk = 4096;  // x staged in LDS in chunks of this many k

// Standalone EXACT MXFP4 matvec: one wavefront per 64 rows.
__global__ __launch_bounds__(64) void k_mxfp4_matvec_exact(uint32_t N, uint32_t K,
                                                           const float *__restrict__ x,
                                                           const uint8_t *__restrict__ w,
                                                           const uint8_t *__restrict__ sc,
                                                           float *__restrict__ y) {
  __shared__ float xs[kExactChunk];
  int lo = 255, hi = 0;
  for (uint32_t i = threadIdx.x; i < K; i += 64) exp_range_acc(x[i], lo, hi);
  const CodeWindow win = mx_window(wave_min_i(lo), wave_max_i(hi));
  const Rsrc rw = make_rsrc(w, N * (K / 2));
  const Rsrc rs = make_rsrc(sc, N * (K / 32));
  const uint32_t row = blockIdx.x * 64u + threadIdx.x;
  const bool active = row < N;
  const uint32_t rr = active ? row : 0u;
  float acc = 0.0f;
  for (uint32_t c0 = 0; c0 < K; c0 += kExactChunk) {
    const uint32_t n = min(uint32_t(kExactChunk), K - c0);
    __syncthreads();
    for (uint32_t i = threadIdx.x * 4; i < n; i += 256)
      *reinterpret_cast<float4 *>(xs + i) = *reinterpret_cast<const float4 *>(x + c0 + i);
    __syncthreads();
    // one resource per matrix; only the row offsets differ between lanes
    const uint32_t woff = rr * (K / 2) + c0 / 2, soff = rr * (K / 32) + c0 / 32;
    acc = (((n / 32) & 15) == 0) ? mx_row_exact<16>(acc, rw, woff, rs, soff, int(n / 32), xs, win)
                                 : mx_row_exact<4>(acc, rw, woff, rs, soff, int(n / 32), xs, win);
  }
  if (active) y[row] = acc;
}

// Standalone EXACT FP8 matvec: one wavefront per 64 rows.
template <bool K16>
__global__ __launch_bounds__(64) void k_fp8_matvec_exact(uint32_t N, uint32_t K, const void *x,
                                                         int x_bf16, const uint8_t *__restrict__ w,
                                                         const void *__restrict__ sc, int scale_f32,
                                                         float *__restrict__ y) {
  __shared__ float xs[kExactChunk];
  const uint32_t row = blockIdx.x * 64u + threadIdx.x;
  const bool active = row < N;
  const uint32_t rr = active ? row : 0u;
  const uint32_t kg = (K + 127) / 128;
  const uint32_t ntile = ((N + 127) / 128) * kg;
  const Rsrc rw = make_rsrc(w, N * K);
  const Rsrc rs = make_rsrc(sc, scale_f32 ? 4u * ntile : ntile);
  const uint32_t tile_row = (rr / 128) * kg;
  float acc = 0.0f;
  for (uint32_t c0 = 0; c0 < K; c0 += kExactChunk) {
    const uint32_t n = min(uint32_t(kExactChunk), K - c0);
    __syncthreads();
    if (x_bf16)
      for (uint32_t i = threadIdx.x; i < n; i += 64) xs[i] = bf16_f32(reinterpret_cast<const uint16_t *>(x)[c0 + i]);
    else
      for (uint32_t i = threadIdx.x; i < n; i += 64) xs[i] = reinterpret_cast<const float *>(x)[c0 + i];
    __syncthreads();
    const uint32_t soff = (scale_f32 ? 4u : 1u) * (tile_row + c0 / 128);
    acc = fp8_row_exact<K16>(acc, rw, rr * K + c0, rs, soff, scale_f32, int(n), xs);
  }
  if (active) y[row] = acc;
}

// ---------------------------------------------------------------------------
// FAST row kernels: lane l owns k in [2048 s + 32 l, +32) for each 2048-wide
// segment s (MXFP4), x held in registers; rows streamed with coalesced
// 16-byte loads; one cross-lane reduction per row.
// ---------------------------------------------------------------------------

template <int NSEG>
struct XReg {
  float v[NSEG * 32];
};

template <int NSEG>
__device__ __forceinline__ void load_x_mx(XReg<NSEG> &xr, const float *__restrict__ x, int K) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int s = 0; s < NSEG; ++s) {
    const int k0 = s * 2048 + lane * 32;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (k0 < K) v = *reinterpret_cast<const float4 *>(x + k0 + 4 * j);
      xr.v[s * 32 + 4 * j + 0] = v.x;
      xr.v[s * 32 + 4 * j + 1] = v.y;
      xr.v[s * 32 + 4 * j + 2] = v.z;
      xr.v[s * 32 + 4 * j + 3] = v.w;
    }
  }
}

struct MxRowFrag {
  uint4 w;
  uint32_t c;
};

// Fragments of one MXFP4 row whose codes start at rw[woff] and scale codes
// at rs[soff]; lanes past K read zeros (code 0 = +0).
template <int NSEG>
__device__ __forceinline__ void load_mx_row_frag(MxRowFrag (&f)[NSEG], Rsrc rw, uint32_t woff, Rsrc rs,
                                                 uint32_t soff, int K) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int s = 0; s < NSEG; ++s) {
    const int k0 = s * 2048 + lane * 32;
    if (k0 < K) {
      f[s].w = ld16(rw, woff + uint32_t(k0 / 2));
      f[s].c = ld1(rs, soff + uint32_t(k0 / 32));
    } else {
      f[s].w = make_uint4(0u, 0u, 0u, 0u);
      f[s].c = 127u;
    }
  }
}

template <int NSEG>
__device__ __forceinline__ float mx_row_fast_partial(const MxRowFrag (&f)[NSEG], const XReg<NSEG> &xr) {
  float acc = 0.0f;
#pragma unroll
  for (int s = 0; s < NSEG; ++s) {
    const uint32_t words[4] = {f[s].w.x, f[s].w.y, f[s].w.z, f[s].w.w};
    float part = 0.0f;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const v2f p0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(words[d], 1.0f, 0);
      const v2f p1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(words[d], 1.0f, 1);
      const v2f p2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(words[d], 1.0f, 2);
      const v2f p3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(words[d], 1.0f, 3);
      const float *xv = &xr.v[s * 32 + d * 8];
      part = fmaf(xv[0], p0.x, part);
      part = fmaf(xv[1], p0.y, part);
      part = fmaf(xv[2], p1.x, part);
      part = fmaf(xv[3], p1.y, part);
      part = fmaf(xv[4], p2.x, part);
      part = fmaf(xv[5], p2.y, part);
      part = fmaf(xv[6], p3.x, part);
      part = fmaf(xv[7], p3.y, part);
    }
    acc = fmaf(part, ue8m0_f32(f[s].c), acc);
  }
  return acc;
}

// Standalone FAST MXFP4 matvec: 4 wavefronts per block, R rows per wavefront.
template <int NSEG, int R>
__global__ __launch_bounds__(256) void k_mxfp4_matvec_fast(uint32_t N, uint32_t K,
                                                           const float *__restrict__ x,
                                                           const uint8_t *__restrict__ w,
                                                           const uint8_t *__restrict__ sc,
                                                           float *__restrict__ y) {
  XReg<NSEG> xr;
  load_x_mx<NSEG>(xr, x, int(K));
  const Rsrc rw = make_rsrc(w, N * (K / 2));
  const Rsrc rs = make_rsrc(sc, N * (K / 32));
  const uint32_t wave = blockIdx.x * 4u + (threadIdx.x >> 6);
  const uint32_t row0 = wave * R;
  MxRowFrag f[R][NSEG];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const uint32_t row = min(row0 + r, N - 1);
    load_mx_row_frag<NSEG>(f[r], rw, row * (K / 2), rs, row * (K / 32), int(K));
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float v = wave_sum(mx_row_fast_partial<NSEG>(f[r], xr));
    if ((threadIdx.x & 63) == 0 && row0 + r < N) y[row0 + r] = v;
  }
}

// FAST FP8 matvec: lane l owns k in [1024 s + 16 l, +16); the 16 k of a lane
// lie in one 128-wide scale tile.  One row per wavefront.
template <int NSEG>
__global__ __launch_bounds__(256) void k_fp8_matvec_fast(uint32_t N, uint32_t K, const void *x,
                                                         int x_bf16, const uint8_t *__restrict__ w,
                                                         const void *__restrict__ sc, int scale_f32,
                                                         float *__restrict__ y) {
  const int lane = threadIdx.x & 63;
  float xv[NSEG * 16];
#pragma unroll
  for (int s = 0; s < NSEG; ++s) {
    const int k0 = s * 1024 + lane * 16;
    if (k0 < int(K)) {
      if (x_bf16) {
        const uint4 b = *reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(x) + k0);
        const uint4 c = *reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(x) + k0 + 8);
        const uint32_t hw[8] = {b.x, b.y, b.z, b.w, c.x, c.y, c.z, c.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          xv[s * 16 + 2 * j] = __uint_as_float(hw[j] << 16);
          xv[s * 16 + 2 * j + 1] = __uint_as_float(hw[j] & 0xffff0000u);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float4 v = *reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(x) + k0 + 4 * j);
          xv[s * 16 + 4 * j + 0] = v.x;
          xv[s * 16 + 4 * j + 1] = v.y;
          xv[s * 16 + 4 * j + 2] = v.z;
          xv[s * 16 + 4 * j + 3] = v.w;
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) xv[s * 16 + j] = 0.0f;
    }
  }
  const uint32_t row = blockIdx.x * 4u + (threadIdx.x >> 6);
  if (row >= N) return;
  const uint32_t kg = (K + 127) / 128;
  const uint32_t ntile = ((N + 127) / 128) * kg;
  const Rsrc rw = make_rsrc(w, N * K);
  const Rsrc rs = make_rsrc(sc, scale_f32 ? 4u * ntile : ntile);
  const uint32_t srow = (row / 128) * kg;
  uint4 wf[NSEG];
  float sv[NSEG];
#pragma unroll
  for (int s = 0; s < NSEG; ++s) {
    const int k0 = s * 1024 + lane * 16;
    if (k0 < int(K)) {
      wf[s] = ld16(rw, row * K + uint32_t(k0));
      const uint32_t t = srow + uint32_t(k0 / 128);
      sv[s] = scale_f32 ? ldf(rs, 4u * t) : ue8m0_f32(ld1(rs, t));
    } else {
      wf[s] = make_uint4(0u, 0u, 0u, 0u);
      sv[s] = 0.0f;
    }
  }
  float acc = 0.0f;
#pragma unroll
  for (int s = 0; s < NSEG; ++s) {
    const uint32_t words[4] = {wf[s].x, wf[s].y, wf[s].z, wf[s].w};
    float part = 0.0f;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const v2f lo = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(words[d], 1.0f, false);
      const v2f hi = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(words[d], 1.0f, true);
      part = fmaf(xv[s * 16 + 4 * d + 0], lo.x, part);
      part = fmaf(xv[s * 16 + 4 * d + 1], lo.y, part);
      part = fmaf(xv[s * 16 + 4 * d + 2], hi.x, part);
      part = fmaf(xv[s * 16 + 4 * d + 3], hi.y, part);
    }
    acc = fmaf(part, sv[s], acc);
  }
  acc = wave_sum(acc);
  if (lane == 0) y[row] = acc;
}

// ---------------------------------------------------------------------------
// element-wise kernels (s14_swiglu_limit.comp, s14_route_mix.comp,
// s14_moe_accumulate.comp semantics; oracle :1543-1556, :1300, :929-946)
// ---------------------------------------------------------------------------

__global__ void k_swiglu(uint32_t n, const float *__restrict__ g, const float *__restrict__ u,
                         float *__restrict__ y) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = swiglu_exact(g[i], u[i]);
}

__global__ void k_route_mix(uint32_t n, float w, const float *__restrict__ e, float *__restrict__ out) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = __fmul_rn(w, e[i]);
}

__global__ void k_moe_accumulate(uint32_t n, float w, const float *__restrict__ e, float *acc) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) acc[i] = __fadd_rn(acc[i], __fmul_rn(w, e[i]));
}

__global__ void k_dequant_mxfp4(uint32_t N, uint32_t K, const uint8_t *__restrict__ w,
                                const uint8_t *__restrict__ sc, float *__restrict__ out) {
  // one thread per code byte: two outputs, through the same scaled-decode
  // window the exact matvec uses (codes 2..252), literal decode otherwise
  const size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const size_t nbytes = size_t(N) * K / 2;
  if (i >= nbytes) return;
  const size_t row = i / (K / 2), pair = i % (K / 2);
  const uint32_t c = sc[row * (K / 32) + (pair * 2) / 32];
  const uint32_t byte = w[i];
  float a, b;
  if (c >= 2u && c <= 252u) {
    const v2f p = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(byte, __uint_as_float(c << 23), 0);
    a = p.x;
    b = p.y;
  } else {
    const float s = ue8m0_f32(c);
    a = __fmul_rn(e2m1_f32(byte & 15u), s);
    b = __fmul_rn(e2m1_f32(byte >> 4), s);
  }
  out[row * K + pair * 2] = a;
  out[row * K + pair * 2 + 1] = b;
}

__global__ void k_dequant_fp8(uint32_t N, uint32_t K, const uint8_t *__restrict__ w,
                              const void *__restrict__ sc, int scale_f32, float *__restrict__ out) {
  const size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= size_t(N) * K) return;
  const size_t row = i / K, k = i % K;
  const size_t si = (row / 128) * ((K + 127) / 128) + k / 128;
  const float s = scale_f32 ? reinterpret_cast<const float *>(sc)[si]
                            : ue8m0_f32(reinterpret_cast<const uint8_t *>(sc)[si]);
  const v2f p = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(uint32_t(w[i]), 1.0f, false);
  out[i] = __fmul_rn(p.x, s);
}

// ---------------------------------------------------------------------------
// synthetic page fill: the oracle generator's integer hash, on the device
// ---------------------------------------------------------------------------

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ULL;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}
__device__ __forceinline__ uint64_t rand_u64(uint64_t key, uint64_t index) {
  return mix64(key + index * 0xD1B54A32D192ED03ULL);
}
__device__ __forceinline__ uint64_t stream_key(uint64_t seed, uint64_t stream) {
  return mix64(seed ^ mix64(stream));
}

__global__ void k_fill_page(uint8_t *__restrict__ page, uint64_t seed, uint32_t layer, uint32_t expert,
                            uint64_t up_w, uint64_t up_s, uint64_t dn_w, uint64_t dn_s, int lo, int hi,
                            PageOffsets off) {
  const uint64_t regions_w[3] = {off.w1, off.w3, off.w2};
  const uint64_t regions_s[3] = {off.s1, off.s3, off.s2};
  const uint64_t nw[3] = {up_w, up_w, dn_w};
  const uint64_t ns[3] = {up_s, up_s, dn_s};
  const uint64_t span = uint64_t(hi - lo + 1);
  const uint64_t tid = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const uint64_t stride = uint64_t(gridDim.x) * blockDim.x;
  for (int m = 0; m < 3; ++m) {
    const uint64_t kw = stream_key(seed, (uint64_t(layer) << 32) | (uint64_t(expert) << 8) | uint64_t(2 * m));
    uint64_t *dst = reinterpret_cast<uint64_t *>(page + regions_w[m]);
    for (uint64_t i = tid; i < nw[m] / 8; i += stride) dst[i] = rand_u64(kw, i);
    const uint64_t ks = stream_key(seed, (uint64_t(layer) << 32) | (uint64_t(expert) << 8) | uint64_t(2 * m + 1));
    uint8_t *ds = page + regions_s[m];
    for (uint64_t i = tid; i < ns[m]; i += stride)
      ds[i] = uint8_t(127 + lo + int(rand_u64(ks, i) % span));
  }
}

// ---------------------------------------------------------------------------
// fused layer / block path
// ---------------------------------------------------------------------------

// Agent-scope acquire-release counter increment; returns the old value.
__device__ __forceinline__ uint32_t counter_arrive(uint32_t *c) {
  return __hip_atomic_fetch_add(c, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void counter_reset(uint32_t *c) {
  __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ T load_agent(const T *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__global__ void k_plan_from_host(PairTable plan, PairTable *__restrict__ out) {
  const uint32_t *src = reinterpret_cast<const uint32_t *>(&plan);
  uint32_t *dst = reinterpret_cast<uint32_t *>(out);
  for (uint32_t i = threadIdx.x; i < sizeof(PairTable) / 4; i += blockDim.x) dst[i] = src[i];
}

// Router: one wavefront per (expert, token).  Logit order (fixed here; the
// reference uses torch F.linear, executor.py:641, whose order is the
// BLAS's): lane l sums k = 256c + 4l + j (c ascending, j = 0..3), then the
// xor butterfly over lanes.  The last block of a token picks the top-k of
// score + bias (ties to the lower index) and the renormalised weights; the
// last token to finish writes the expert-major PairTable.
__global__ __launch_bounds__(256) void k_router_plan(RouterArgs r, uint32_t T, const float *__restrict__ X,
                                                     Workspace ws, const uint64_t *__restrict__ expert_pages,
                                                     const uint8_t *shared_page, int shared_fmt,
                                                     uint16_t *ids_out, float *weights_out, int build_plan) {
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t t = blockIdx.y;
  const uint32_t e = blockIdx.x * 4u + wave;
  const uint32_t K = kHidden;
  const float *x = X + size_t(t) * K;
  if (e < r.n_experts) {
    const float *row = r.weight + size_t(e) * K;
    float acc = 0.0f;
    for (uint32_t c = 0; c < K / 256; ++c) {
      const uint32_t k = c * 256 + lane * 4;
      const float4 wv = *reinterpret_cast<const float4 *>(row + k);
      const float4 xv = *reinterpret_cast<const float4 *>(x + k);
      acc = __fadd_rn(acc, __fmul_rn(wv.x, xv.x));
      acc = __fadd_rn(acc, __fmul_rn(wv.y, xv.y));
      acc = __fadd_rn(acc, __fmul_rn(wv.z, xv.z));
      acc = __fadd_rn(acc, __fmul_rn(wv.w, xv.w));
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) acc = __fadd_rn(acc, __shfl_xor(acc, m));
    if (lane == 0) {
      float s;
      if (r.score_fn == S14_SCORE_SIGMOID) {
        s = __fdiv_rn(1.0f, __fadd_rn(1.0f, s14x::expf_glibc(-acc)));
      } else {
        const float sp = acc > 20.0f ? acc : log1pf(s14x::expf_glibc(acc));
        s = __fsqrt_rn(sp);
      }
      ws.scores[t * kMaxExperts + e] = s;
      ws.biased[t * kMaxExperts + e] = __fadd_rn(s, r.bias[e]);
    }
  }
  __threadfence();
  __syncthreads();
  __shared__ uint32_t s_old;
  if (threadIdx.x == 0) s_old = counter_arrive(&ws.counters[t]);
  __syncthreads();
  if (s_old != gridDim.x - 1u || wave != 0) return;
  // ---- last block of token t: top-k on wavefront 0 ----
  if (lane == 0) counter_reset(&ws.counters[t]);
  float v[4];
  bool taken[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t ee = lane + 64u * j;
    taken[j] = ee >= r.n_experts;
    v[j] = taken[j] ? 0.0f : load_agent(&ws.biased[t * kMaxExperts + ee]);
  }
  uint32_t sel[kTopK];
  for (uint32_t i = 0; i < r.topk; ++i) {
    float bv = 0.0f;
    int bi = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (!taken[j] && (bi == 0x7fffffff || v[j] > bv)) {
        bv = v[j];
        bi = int(lane + 64u * j);
      }
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
      const float ov = __shfl_xor(bv, m);
      const int oi = __shfl_xor(bi, m);
      const bool better = (oi != 0x7fffffff) && (bi == 0x7fffffff || ov > bv || (ov == bv && oi < bi));
      if (better) {
        bv = ov;
        bi = oi;
      }
    }
    sel[i] = uint32_t(bi);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (int(lane + 64u * j) == bi) taken[j] = true;
  }
  if (lane == 0) {
    float sc[kTopK];
    float sum = 0.0f;
    for (uint32_t i = 0; i < r.topk; ++i) {
      sc[i] = load_agent(&ws.scores[t * kMaxExperts + sel[i]]);
      sum = __fadd_rn(sum, sc[i]);
    }
    for (uint32_t i = 0; i < r.topk; ++i) {
      float wgt = __fdiv_rn(sc[i], sum);
      if (r.route_scale != 1.0f) wgt = __fmul_rn(wgt, r.route_scale);
      ws.ids[t * kTopK + i] = uint16_t(sel[i]);
      ws.weights[t * kTopK + i] = wgt;
      if (ids_out) ids_out[t * r.topk + i] = uint16_t(sel[i]);
      if (weights_out) weights_out[t * r.topk + i] = wgt;
    }
  }
  if (!build_plan) return;
  __threadfence();
  uint32_t old = 0;
  if (lane == 0) old = counter_arrive(&ws.counters[kCntPlan]);
  old = __shfl(old, 0);
  if (old != T - 1u) return;
  // ---- last token: expert-major PairTable ----
  if (lane == 0) counter_reset(&ws.counters[kCntPlan]);
  const uint32_t npr = T * kTopK;  // routed (token, expert) pairs, <= 48
  const bool mine = lane < npr;
  const uint32_t mt = mine ? lane / kTopK : 0u, mr = mine ? lane % kTopK : 0u;
  const uint32_t me = mine ? uint32_t(load_agent(&ws.ids[mt * kTopK + mr])) : 0u;
  const float mw = mine ? load_agent(&ws.weights[mt * kTopK + mr]) : 0.0f;
  const uint32_t key = mine ? me * 8u + mt : 0xffffffffu;
  uint32_t rank = 0, first = 1;
  for (uint32_t j = 0; j < npr; ++j) {
    const uint32_t kj = __shfl(key, int(j));
    rank += kj < key ? 1u : 0u;
    if ((kj >> 3) == (key >> 3) && kj < key) first = 0;
  }
  PairTable *tab = ws.table;
  if (mine) {
    tab->page[rank] = expert_pages[me];
    tab->fmt[rank] = S14_PAGE_MXFP4;
    tab->token[rank] = mt;
    tab->weight[rank] = mw;
    tab->is_shared[rank] = 0u;
    tab->token_pairs[mt][mr] = rank;
  }
  const uint64_t firsts = __ballot(mine && first);
  if (lane < T) {
    const uint32_t sp = npr + lane;
    tab->page[sp] = reinterpret_cast<uint64_t>(shared_page);
    tab->fmt[sp] = uint32_t(shared_fmt);
    tab->token[sp] = lane;
    tab->weight[sp] = 1.0f;
    tab->is_shared[sp] = 1u;
    tab->token_pairs[lane][kTopK] = sp;
    tab->token_npairs[lane] = kTopK + 1;
  }
  if (lane == 0) {
    tab->n_pairs = npr + T;
    tab->n_tokens = T;
    tab->n_distinct = uint32_t(__popcll(firsts));
    tab->chain = 0u;
  }
}

// Final per-token accumulation of one row tile, run by the last block to
// finish that (token, tile): acc = 0; acc += w * down in route order; acc +=
// shared down (s14_vulkan_numeric.rs:929-946); or y = w * down for the chain
// (:1300).
__device__ __forceinline__ void accumulate_tail(const PairTable *__restrict__ tab, uint32_t p,
                                                uint32_t tile, uint32_t rows_per_tile,
                                                const float *down, float *__restrict__ Y,
                                                uint32_t *counters) {
  __threadfence();
  __syncthreads();
  __shared__ uint32_t s_old;
  const uint32_t t = tab->token[p];
  uint32_t *cnt = &counters[kCntAcc + t * kMaxTiles + tile];
  if (threadIdx.x == 0) s_old = counter_arrive(cnt);
  __syncthreads();
  const uint32_t np = tab->token_npairs[t];
  if (s_old != np - 1u) return;
  if (threadIdx.x == 0) counter_reset(cnt);
  for (uint32_t i = threadIdx.x; i < rows_per_tile; i += blockDim.x) {
    const uint32_t row = tile * rows_per_tile + i;
    float acc = 0.0f;
    if (tab->chain) {
      const uint32_t pr = tab->token_pairs[t][0];
      acc = __fmul_rn(tab->weight[pr], load_agent(&down[size_t(pr) * kHidden + row]));
    } else {
      for (uint32_t j = 0; j < np; ++j) {
        const uint32_t pr = tab->token_pairs[t][j];
        const float d = load_agent(&down[size_t(pr) * kHidden + row]);
        acc = tab->is_shared[pr] ? __fadd_rn(acc, d) : __fadd_rn(acc, __fmul_rn(tab->weight[pr], d));
      }
    }
    Y[size_t(t) * kHidden + row] = acc;
  }
}

// Phase 1 EXACT: one wavefront per (pair, 32-row tile); lanes 0-31 take rows
// of w1, lanes 32-63 the same rows of w3; h = swiglu(g, u) after a lane swap.
__global__ __launch_bounds__(64) void k_phase1_exact(const PairTable *__restrict__ tab,
                                                     const float *__restrict__ X, float *__restrict__ H,
                                                     PageOffsets mx, PageOffsets f8, uint32_t mx_bytes,
                                                     uint32_t f8_bytes) {
  __shared__ float xs[kHidden];
  const uint32_t p = blockIdx.y;
  if (p >= tab->n_pairs) return;
  const uint32_t lane = threadIdx.x;
  int emin, emax;
  stage_f32_range(xs, X + size_t(tab->token[p]) * kHidden, kHidden, emin, emax);
  const uint8_t *page = reinterpret_cast<const uint8_t *>(tab->page[p]);
  const bool upper = lane >= 32;
  const uint32_t row = blockIdx.x * kP1ExactRows + (lane & 31u);
  float acc;
  if (tab->fmt[p] == S14_PAGE_MXFP4) {
    const Rsrc r = make_rsrc(page, mx_bytes);
    const uint32_t woff = uint32_t(upper ? mx.w3 : mx.w1) + row * (kHidden / 2);
    const uint32_t soff = uint32_t(upper ? mx.s3 : mx.s1) + row * (kHidden / 32);
    acc = mx_row_exact<16>(0.0f, r, woff, r, soff, kHidden / 32, xs, mx_window(emin, emax));
  } else {
    const Rsrc r = make_rsrc(page, f8_bytes);
    const uint32_t woff = uint32_t(upper ? f8.w3 : f8.w1) + row * kHidden;
    const uint32_t soff = uint32_t(upper ? f8.s3 : f8.s1) + (row / 128) * (kHidden / 128);
    acc = fp8_row_exact<true>(0.0f, r, woff, r, soff, 0, kHidden, xs);
  }
  const float other = __shfl_xor(acc, 32);
  if (!upper) H[size_t(p) * kInter + row] = swiglu_exact(acc, other);
}

// Phase 2 EXACT: one wavefront per (pair, 64-row tile) of w2.
__global__ __launch_bounds__(64) void k_phase2_exact(const PairTable *__restrict__ tab,
                                                     const float *__restrict__ H, float *D,
                                                     float *__restrict__ Y, uint32_t *counters,
                                                     PageOffsets mx, PageOffsets f8, uint32_t mx_bytes,
                                                     uint32_t f8_bytes) {
  __shared__ float hs[kInter];
  const uint32_t p = blockIdx.y;
  if (p >= tab->n_pairs) return;
  int emin, emax;
  stage_f32_range(hs, H + size_t(p) * kInter, kInter, emin, emax);
  const uint8_t *page = reinterpret_cast<const uint8_t *>(tab->page[p]);
  const uint32_t row = blockIdx.x * kP2ExactRows + threadIdx.x;
  float acc;
  if (tab->fmt[p] == S14_PAGE_MXFP4) {
    const Rsrc r = make_rsrc(page, mx_bytes);
    acc = mx_row_exact<16>(0.0f, r, uint32_t(mx.w2) + row * (kInter / 2), r,
                           uint32_t(mx.s2) + row * (kInter / 32), kInter / 32, hs, mx_window(emin, emax));
  } else {
    const Rsrc r = make_rsrc(page, f8_bytes);
    acc = fp8_row_exact<true>(0.0f, r, uint32_t(f8.w2) + row * kInter, r,
                              uint32_t(f8.s2) + (row / 128) * (kInter / 128), 0, kInter, hs);
  }
  D[size_t(p) * kHidden + row] = acc;
  accumulate_tail(tab, p, blockIdx.x, kP2ExactRows, D, Y, counters);
}

// FAST helpers for FP8 pages: lane l owns k in [2048 s + 32 l, +32) as for
// MXFP4, i.e. two 16-byte loads per segment, one ue8m0 tile scale.
template <int NSEG>
__device__ __forceinline__ float fp8_row_fast_partial(Rsrc r, uint32_t woff, uint32_t soff_tiles,
                                                      const XReg<NSEG> &xr) {
  const int lane = threadIdx.x & 63;
  float acc = 0.0f;
#pragma unroll
  for (int s = 0; s < NSEG; ++s) {
    const uint32_t k0 = uint32_t(s * 2048 + lane * 32);
    const uint4 a = ld16(r, woff + k0);
    const uint4 b = ld16(r, woff + k0 + 16u);
    const float sc = ue8m0_f32(ld1(r, soff_tiles + k0 / 128));
    const uint32_t words[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    float part = 0.0f;
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      const v2f lo = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(words[d], 1.0f, false);
      const v2f hi = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(words[d], 1.0f, true);
      part = fmaf(xr.v[s * 32 + 4 * d + 0], lo.x, part);
      part = fmaf(xr.v[s * 32 + 4 * d + 1], lo.y, part);
      part = fmaf(xr.v[s * 32 + 4 * d + 2], hi.x, part);
      part = fmaf(xr.v[s * 32 + 4 * d + 3], hi.y, part);
    }
    acc = fmaf(part, sc, acc);
  }
  return acc;
}

// Phase 1 FAST: 4 wavefronts per block, each kP1FastRowsPerWave rows of w1
// and w3 (x for the lane's k slices held in registers).
__global__ __launch_bounds__(256) void k_phase1_fast(const PairTable *__restrict__ tab,
                                                     const float *__restrict__ X, float *__restrict__ H,
                                                     PageOffsets mx, PageOffsets f8, uint32_t mx_bytes,
                                                     uint32_t f8_bytes) {
  constexpr int NSEG = kHidden / 2048;
  constexpr int R = kP1FastRowsPerWave;
  const uint32_t p = blockIdx.y;
  if (p >= tab->n_pairs) return;
  XReg<NSEG> xr;
  load_x_mx<NSEG>(xr, X + size_t(tab->token[p]) * kHidden, kHidden);
  const uint8_t *page = reinterpret_cast<const uint8_t *>(tab->page[p]);
  const uint32_t row0 = blockIdx.x * kP1FastRows + (threadIdx.x >> 6) * R;
  float g[R], u[R];
  if (tab->fmt[p] == S14_PAGE_MXFP4) {
    const Rsrc r = make_rsrc(page, mx_bytes);
    MxRowFrag f1[R][NSEG], f3[R][NSEG];
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const uint32_t row = row0 + i;
      load_mx_row_frag<NSEG>(f1[i], r, uint32_t(mx.w1) + row * (kHidden / 2), r,
                             uint32_t(mx.s1) + row * (kHidden / 32), kHidden);
      load_mx_row_frag<NSEG>(f3[i], r, uint32_t(mx.w3) + row * (kHidden / 2), r,
                             uint32_t(mx.s3) + row * (kHidden / 32), kHidden);
    }
#pragma unroll
    for (int i = 0; i < R; ++i) {
      g[i] = wave_sum(mx_row_fast_partial<NSEG>(f1[i], xr));
      u[i] = wave_sum(mx_row_fast_partial<NSEG>(f3[i], xr));
    }
  } else {
    const Rsrc r = make_rsrc(page, f8_bytes);
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const uint32_t row = row0 + i;
      g[i] = wave_sum(fp8_row_fast_partial<NSEG>(r, uint32_t(f8.w1) + row * kHidden,
                                                 uint32_t(f8.s1) + (row / 128) * (kHidden / 128), xr));
      u[i] = wave_sum(fp8_row_fast_partial<NSEG>(r, uint32_t(f8.w3) + row * kHidden,
                                                 uint32_t(f8.s3) + (row / 128) * (kHidden / 128), xr));
    }
  }
  const int lane = threadIdx.x & 63;
  if (lane < R) {
    float gv = g[0], uv = u[0];
#pragma unroll
    for (int i = 1; i < R; ++i)
      if (lane == i) {
        gv = g[i];
        uv = u[i];
      }
    H[size_t(p) * kInter + row0 + lane] = swiglu_exact(gv, uv);
  }
}

// Phase 2 FAST: 4 wavefronts per block, kP2FastRowsPerWave rows of w2 each.
__global__ __launch_bounds__(256) void k_phase2_fast(const PairTable *__restrict__ tab,
                                                     const float *__restrict__ H, float *D,
                                                     float *__restrict__ Y, uint32_t *counters,
                                                     PageOffsets mx, PageOffsets f8, uint32_t mx_bytes,
                                                     uint32_t f8_bytes) {
  constexpr int NSEG = kInter / 2048;
  constexpr int R = kP2FastRowsPerWave;
  const uint32_t p = blockIdx.y;
  if (p >= tab->n_pairs) return;
  XReg<NSEG> xr;
  load_x_mx<NSEG>(xr, H + size_t(p) * kInter, kInter);
  const uint8_t *page = reinterpret_cast<const uint8_t *>(tab->page[p]);
  const uint32_t row0 = blockIdx.x * kP2FastRows + (threadIdx.x >> 6) * R;
  float d[R];
  if (tab->fmt[p] == S14_PAGE_MXFP4) {
    const Rsrc r = make_rsrc(page, mx_bytes);
    MxRowFrag f[R][NSEG];
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const uint32_t row = row0 + i;
      load_mx_row_frag<NSEG>(f[i], r, uint32_t(mx.w2) + row * (kInter / 2), r,
                             uint32_t(mx.s2) + row * (kInter / 32), kInter);
    }
#pragma unroll
    for (int i = 0; i < R; ++i) d[i] = wave_sum(mx_row_fast_partial<NSEG>(f[i], xr));
  } else {
    const Rsrc r = make_rsrc(page, f8_bytes);
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const uint32_t row = row0 + i;
      d[i] = wave_sum(fp8_row_fast_partial<NSEG>(r, uint32_t(f8.w2) + row * kInter,
                                                 uint32_t(f8.s2) + (row / 128) * (kInter / 128), xr));
    }
  }
  const int lane = threadIdx.x & 63;
  if (lane < R) {
    float v = d[0];
#pragma unroll
    for (int i = 1; i < R; ++i)
      if (lane == i) v = d[i];
    D[size_t(p) * kHidden + row0 + lane] = v;
  }
  accumulate_tail(tab, p, blockIdx.x, kP2FastRows, D, Y, counters);
}

inline unsigned blocks_for(size_t n, unsigned threads) { return unsigned((n + threads - 1) / threads); }

}  // namespace

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------

hipError_t launch_mxfp4_matvec(hipStream_t s, const s14_mxfp4_dispatch &d) {
  const uint32_t N = d.shape.n, K = d.shape.k;
  if (d.mode == S14_MODE_FAST && K <= 8192) {
    const unsigned rows_per_block = 4 * 4;
    const unsigned grid = blocks_for(N, rows_per_block);
    if (K <= 2048)
      k_mxfp4_matvec_fast<1, 4><<<grid, 256, 0, s>>>(N, K, d.x, d.weight, d.scale, d.y);
    else if (K <= 4096)
      k_mxfp4_matvec_fast<2, 4><<<grid, 256, 0, s>>>(N, K, d.x, d.weight, d.scale, d.y);
    else
      k_mxfp4_matvec_fast<4, 4><<<grid, 256, 0, s>>>(N, K, d.x, d.weight, d.scale, d.y);
  } else {
    k_mxfp4_matvec_exact<<<blocks_for(N, 64), 64, 0, s>>>(N, K, d.x, d.weight, d.scale, d.y);
  }
  return hipGetLastError();
}

hipError_t launch_fp8_matvec(hipStream_t s, const s14_fp8_dispatch &d) {
  const uint32_t N = d.shape.n, K = d.shape.k;
  const int xb = d.x_dtype == S14_X_BF16, sf = d.scale_dtype == S14_SCALE_F32;
  const bool k16 = (K % 16) == 0;
  if (d.mode == S14_MODE_FAST && k16 && K <= 8192) {
    const unsigned grid = blocks_for(N, 4);
    if (K <= 1024)
      k_fp8_matvec_fast<1><<<grid, 256, 0, s>>>(N, K, d.x, xb, d.weight, d.scale, sf, d.y);
    else if (K <= 2048)
      k_fp8_matvec_fast<2><<<grid, 256, 0, s>>>(N, K, d.x, xb, d.weight, d.scale, sf, d.y);
    else if (K <= 4096)
      k_fp8_matvec_fast<4><<<grid, 256, 0, s>>>(N, K, d.x, xb, d.weight, d.scale, sf, d.y);
    else
      k_fp8_matvec_fast<8><<<grid, 256, 0, s>>>(N, K, d.x, xb, d.weight, d.scale, sf, d.y);
  } else if (k16) {
    k_fp8_matvec_exact<true><<<blocks_for(N, 64), 64, 0, s>>>(N, K, d.x, xb, d.weight, d.scale, sf, d.y);
  } else {
    k_fp8_matvec_exact<false><<<blocks_for(N, 64), 64, 0, s>>>(N, K, d.x, xb, d.weight, d.scale, sf, d.y);
  }
  return hipGetLastError();
}

hipError_t launch_swiglu(hipStream_t s, const s14_swiglu_dispatch &d) {
  k_swiglu<<<blocks_for(d.n, 256), 256, 0, s>>>(d.n, d.gate, d.up, d.y);
  return hipGetLastError();
}

hipError_t launch_route_mix(hipStream_t s, const s14_scale_dispatch &d) {
  k_route_mix<<<blocks_for(d.n, 256), 256, 0, s>>>(d.n, d.weight, d.expert, d.out);
  return hipGetLastError();
}

hipError_t launch_moe_accumulate(hipStream_t s, const s14_scale_dispatch &d) {
  k_moe_accumulate<<<blocks_for(d.n, 256), 256, 0, s>>>(d.n, d.weight, d.expert, d.out);
  return hipGetLastError();
}

hipError_t launch_dequant_mxfp4(hipStream_t s, s14_shape shape, const uint8_t *w, const uint8_t *sc,
                                float *out) {
  const size_t nbytes = size_t(shape.n) * shape.k / 2;
  k_dequant_mxfp4<<<blocks_for(nbytes, 256), 256, 0, s>>>(shape.n, shape.k, w, sc, out);
  return hipGetLastError();
}

hipError_t launch_dequant_fp8(hipStream_t s, s14_shape shape, const uint8_t *w, const void *sc,
                              int scale_dtype, float *out) {
  const size_t n = size_t(shape.n) * shape.k;
  k_dequant_fp8<<<blocks_for(n, 256), 256, 0, s>>>(shape.n, shape.k, w, sc,
                                                     scale_dtype == S14_SCALE_F32, out);
  return hipGetLastError();
}

hipError_t launch_fill_mxfp4_page(hipStream_t s, uint8_t *page, uint64_t seed, uint32_t layer,
                                  uint32_t expert, uint32_t hidden, uint32_t inter, int lo, int hi,
                                  const PageOffsets &off) {
  const uint64_t up_w = uint64_t(inter) * hidden / 2, up_s = uint64_t(inter) * hidden / 32;
  const uint64_t dn_w = uint64_t(hidden) * inter / 2, dn_s = uint64_t(hidden) * inter / 32;
  k_fill_page<<<1024, 256, 0, s>>>(page, seed, layer, expert, up_w, up_s, dn_w, dn_s, lo, hi, off);
  return hipGetLastError();
}

hipError_t launch_plan_from_host(hipStream_t s, const Workspace &ws, const PairTable &plan) {
  k_plan_from_host<<<1, 256, 0, s>>>(plan, ws.table);
  return hipGetLastError();
}

hipError_t launch_router_plan(hipStream_t s, const Workspace &ws, const RouterArgs &r, uint32_t tokens,
                              const float *x, const uint64_t *expert_pages, const uint8_t *shared_page,
                              int shared_fmt, uint16_t *ids_out, float *weights_out, int build_plan) {
  dim3 grid((r.n_experts + 3) / 4, tokens);
  k_router_plan<<<grid, 256, 0, s>>>(r, tokens, x, ws, expert_pages, shared_page, shared_fmt, ids_out,
                                     weights_out, build_plan);
  return hipGetLastError();
}

hipError_t launch_layer_phases(hipStream_t s, const Workspace &ws, uint32_t n_pairs, uint32_t tokens,
                               const PageOffsets &mx, const PageOffsets &fp8, const float *x, float *y,
                               int mode) {
  (void)tokens;
  const uint32_t mx_bytes = uint32_t(S14_EXPERT_PAGE_BYTES);
  const uint32_t f8_bytes = uint32_t(S14_SHARED_EXPERT_PAGE_BYTES);
  if (mode == S14_MODE_FAST) {
    k_phase1_fast<<<dim3(kInter / kP1FastRows, n_pairs), 256, 0, s>>>(ws.table, x, ws.h, mx, fp8, mx_bytes,
                                                                      f8_bytes);
    k_phase2_fast<<<dim3(kHidden / kP2FastRows, n_pairs), 256, 0, s>>>(ws.table, ws.h, ws.down, y,
                                                                       ws.counters, mx, fp8, mx_bytes,
                                                                       f8_bytes);
  } else {
    k_phase1_exact<<<dim3(kInter / kP1ExactRows, n_pairs), 64, 0, s>>>(ws.table, x, ws.h, mx, fp8, mx_bytes,
                                                                       f8_bytes);
    k_phase2_exact<<<dim3(kHidden / kP2ExactRows, n_pairs), 64, 0, s>>>(ws.table, ws.h, ws.down, y,
                                                                        ws.counters, mx, fp8, mx_bytes,
                                                                        f8_bytes);
  }
  return hipGetLastError();
}

}  // namespace s14
