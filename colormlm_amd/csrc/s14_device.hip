// gfx950 (CDNA4) kernels of the S14 quantized expert path.
//
// Two reduction orders:
//   EXACT  k strictly ascending, multiply then add (no FMA): the operation
//          order of the reference CPU oracle
//          (scheduler/ssd_inference/examples/s14_vulkan_numeric.rs:1669-1714),
//          so outputs are bit-identical to it.  Each row is owned by a lane
//          pair: in every group of 32 k the even lane forms the products of
//          k 0..15 and the odd lane those of k 16..31; the running sum passes
//          to the even lane, which adds its 16 products, then back to the odd
//          lane, which adds its own 16, in k order (each hand-over a DPP
//          quad_perm operand of v_add).  The per-row dependent add chain and
//          the instruction issue around it, not HBM, bound this order at
//          batch 1.
//   FAST   K split across the 64 lanes of a wavefront, products fused
//          (v_fma), DPP cross-lane reduction; HBM-bound.
// The reference's five shaders (shaders/s14_*.comp) are one workgroup per
// row with a 128-way LDS tree; neither order here follows them.
//
// Build: hipcc --offload-arch=gfx950 -ffp-contract=off (contraction would
// fuse the exact kernels' multiply-then-add).
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include "s14_device.hpp"
#include "s14_device_util.hpp"
#include "s14_exact.hpp"

namespace s14 {
namespace {

// ---------------------------------------------------------------------------
// standalone EXACT matvecs: 32 rows per wavefront (one row per lane pair),
// x staged in LDS in chunks of kExactChunk
// ---------------------------------------------------------------------------

constexpr int kExactChunk = 4096;

__global__ __launch_bounds__(64) void k_mxfp4_matvec_exact(uint32_t N, uint32_t K,
                                                           const float *__restrict__ x,
                                                           const uint8_t *__restrict__ w,
                                                           const uint8_t *__restrict__ sc,
                                                           float *__restrict__ y) {
  __shared__ float xs[kExactChunk];
  const uint32_t lane = threadIdx.x, h = lane & 1u;
  int lo = 255, hi = 0;
  for (uint32_t i = lane; i < K; i += 64) exp_range_acc(x[i], lo, hi);
  const CodeWindow win = mx_window(wave_min_i(lo), wave_max_i(hi));
  const Src1 src{make_rsrc(w, N * (K / 2)), make_rsrc(sc, N * (K / 32))};
  const uint32_t row = blockIdx.x * 32u + (lane >> 1);
  const bool active = row < N;
  const uint32_t rr = active ? row : 0u;
  float acc = 0.0f;
  for (uint32_t c0 = 0; c0 < K; c0 += kExactChunk) {
    const uint32_t n = min(uint32_t(kExactChunk), K - c0);
    const uint32_t woff = rr * (K / 2) + c0 / 2 + 8u * h, soff = rr * (K / 32) + c0 / 32;
    const int G = int(n / 32);
    __syncthreads();
    if (G % 16 == 0) {
      MxBatch<16> ba;
      mx_load<16>(ba, src, woff, soff, 0);
      stage_chunk_wave(xs, x + c0, n);
      __syncthreads();
      acc = mx_row_pair<16>(acc, ba, src, woff, soff, G, xs + 16 * h, win);
    } else {
      MxBatch<4> ba;
      mx_load<4>(ba, src, woff, soff, 0);
      stage_chunk_wave(xs, x + c0, n);
      __syncthreads();
      acc = mx_row_pair<4>(acc, ba, src, woff, soff, G, xs + 16 * h, win);
    }
  }
  if (active && h == 0) y[row] = acc;
}

// K % 32 == 0: lane pairs as above.  Otherwise every lane computes its pair's
// whole row itself, element by element.
template <bool K32>
__global__ __launch_bounds__(64) void k_fp8_matvec_exact(uint32_t N, uint32_t K, const void *x,
                                                         int x_bf16, const uint8_t *__restrict__ w,
                                                         const void *__restrict__ sc, int scale_f32,
                                                         float *__restrict__ y) {
  __shared__ float xs[kExactChunk];
  const uint32_t lane = threadIdx.x, h = lane & 1u;
  const uint32_t row = blockIdx.x * 32u + (lane >> 1);
  const bool active = row < N;
  const uint32_t rr = active ? row : 0u;
  const uint32_t kg = (K + 127) / 128;
  const uint32_t ntile = ((N + 127) / 128) * kg;
  const Src1 src{make_rsrc(w, N * K), make_rsrc(sc, scale_f32 ? 4u * ntile : ntile)};
  const uint32_t tile_row = (rr / 128) * kg;
  float acc = 0.0f;
  for (uint32_t c0 = 0; c0 < K; c0 += kExactChunk) {
    const uint32_t n = min(uint32_t(kExactChunk), K - c0);
    __syncthreads();
    // element-wise (x may be unaligned), eight loads in flight per lane
    for (uint32_t i0 = lane; i0 < n; i0 += 64 * 8) {
      float t[8];
#pragma unroll
      for (uint32_t j = 0; j < 8; ++j) {
        const uint32_t i = i0 + 64 * j;
        t[j] = i >= n ? 0.0f
                      : (x_bf16 ? bf16_f32(reinterpret_cast<const uint16_t *>(x)[c0 + i])
                                : reinterpret_cast<const float *>(x)[c0 + i]);
      }
#pragma unroll
      for (uint32_t j = 0; j < 8; ++j)
        if (i0 + 64 * j < n) xs[i0 + 64 * j] = t[j];
    }
    __syncthreads();
    const uint32_t soff = (scale_f32 ? 4u : 1u) * (tile_row + c0 / 128);
    if (K32) {
      constexpr int kDeep = 8;  // batches in flight: 32 groups (the launch has N / 32 wavefronts)
      if ((n / 32) % (4 * kDeep) == 0)
        acc = fp8_row_pair_deep<kDeep>(acc, src, rr * K + c0 + 16u * h, soff, scale_f32, int(n / 32), xs + 16 * h);
      else
        acc = fp8_row_pair(acc, src, rr * K + c0 + 16u * h, soff, scale_f32, int(n / 32), xs + 16 * h);
    } else {
      for (uint32_t k = 0; k < n; ++k) {
        const float s = fp8_scale(src.s, soff, k / 128, scale_f32);
        acc = __fadd_rn(acc, __fmul_rn(__fmul_rn(xs[k], e4m3_f32(ld1(src.w, rr * K + c0 + k))), s));
      }
    }
  }
  if (active && h == 0) y[row] = acc;
}

// ---------------------------------------------------------------------------
// FAST row engine: lane l owns k in [2048 s + 32 l, +32) for each 2048-wide
// segment s (MXFP4), x held in registers; rows streamed with coalesced
// 16-byte loads; one DPP reduction per row.
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

// FP8 pages, same lane ownership: two 16-byte loads and one ue8m0 tile
// scale per segment.
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
    const float v = wave_sum_dpp(mx_row_fast_partial<NSEG>(f[r], xr));
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
      sv[s] = fp8_scale(rs, 0u, srow + uint32_t(k0 / 128), scale_f32);
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
  acc = wave_sum_dpp(acc);
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
// synthetic page fill: the host generator's integer hash, on the device
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
// fused layer / block path: router -> plan -> phase 1 -> phase 2
//
// No workgroup waits on another inside a kernel (an agent-scope release on
// gfx950 writes back the L2, and one per workgroup serialised an earlier
// design); each hand-off is a kernel boundary:
//   router   scores and biased scores of every (token, expert)
//   plan     one workgroup: top-k of every token, the renormalised weights,
//            and the pair table sorted expert-major (each distinct routed
//            page's tokens are adjacent in the grid)
//   phase 1  h = swiglu(w1 x, w3 x) for every (token, expert) pair
//   phase 2  one workgroup per (row tile, token) computes the token's routed
//            and shared w2 rows and accumulates them in route order, shared
//            last, in LDS (s14_vulkan_numeric.rs:929-946)
// ---------------------------------------------------------------------------

// Router scores of many tokens (the prefill's first step): one wavefront per
// tile of kRtE experts x kRtT tokens, every logit summed in router_score's
// order (bit-identical), each weight and x chunk loaded once per tile
// instead of once per (expert, token).  (Staging the token tile's x chunks
// once per workgroup in LDS instead, shared by its four wavefronts, measured
// 30.9 us against 29.3.)
constexpr uint32_t kRtE = 8, kRtT = 8;
static_assert(kRtE * kRtT == 64, "one logit per lane after the reduction");
// One step of the transposing xor butterfly: v holds 2H values (compact
// logit indices k, top bit = bit log2(M) of the logit); the lanes whose
// lane bit M is 0 keep the logits with that bit 0 and the others the rest,
// each adding its own value and its partner's (lane ^ M), the operands and
// the order of router_score's butterfly step (a + a[lane ^ M]; f32 addition
// is commutative, so the two partners' sums are the same value).
template <uint32_t M>
__device__ __forceinline__ float rt_xor_get(float v) {
  if constexpr (M == 8) return dpp_f<0x128>(0.0f, v);  // row_ror:8: lane ^ 8 within each 16-lane row
  else if constexpr (M == 4) {
    int t = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x104, 0xf, 0x5, false);
    t = __builtin_amdgcn_update_dpp(t, __float_as_int(v), 0x114, 0xf, 0xa, false);
    return __int_as_float(t);
  } else if constexpr (M == 2) return dpp_f<0x4e>(0.0f, v);  // quad_perm [2,3,0,1]
  else return dpp_f<0xb1>(0.0f, v);                          // quad_perm [1,0,3,2]
}
template <uint32_t H, uint32_t M>
__device__ __forceinline__ void rt_reduce_step(const float (&v)[2 * H], float (&out)[H]) {
  const bool up = (threadIdx.x & M) != 0u;
#pragma unroll
  for (uint32_t k = 0; k < H; ++k) {
    const float lo = v[k], hi = v[k + H];  // logits with the bit 0 / 1
    if constexpr (M == 32 || M == 16) {
      // lanes M..2M-1 of each 2M-lane block swap with lanes 0..M-1: lo's
      // upper block receives hi's lower one and the other way round
      const auto r = M == 32 ? __builtin_amdgcn_permlane32_swap(__float_as_uint(lo), __float_as_uint(hi), false, false)
                             : __builtin_amdgcn_permlane16_swap(__float_as_uint(lo), __float_as_uint(hi), false, false);
      out[k] = up ? __fadd_rn(hi, __uint_as_float(r[0])) : __fadd_rn(lo, __uint_as_float(r[1]));
    } else {
      const float mine = up ? hi : lo, send = up ? lo : hi;
      out[k] = __fadd_rn(mine, rt_xor_get<M>(send));
    }
  }
}
// kRq (1: default, 2: official): the grid's rows past the token tiles
// requantise X into Q and S (requant_x_group, 256 groups a workgroup) beside
// the scoring, which does not depend on them (a launch of its own took
// ~6 us of the prefill).
template <int kRq>
__global__ __launch_bounds__(256) void k_router_scores(RouterArgs r, uint32_t tokens, const float *__restrict__ X,
                                                       float *__restrict__ scores, float *__restrict__ biased,
                                                       uint8_t *__restrict__ Q, uint8_t *__restrict__ S) {
  if constexpr (kRq != 0) {
    const uint32_t tiles = (tokens + kRtT - 1) / kRtT;
    if (blockIdx.y >= tiles) {  // uniform per workgroup
      const uint32_t b = (blockIdx.y - tiles) * gridDim.x + blockIdx.x;
      requant_x_group<kRq == 2>(b * 256u + threadIdx.x, tokens, X, Q, S);
      return;
    }
  }
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t e0 = (blockIdx.x * 4u + wave) * kRtE, t0 = blockIdx.y * kRtT;
  if (e0 >= r.n_experts) return;
  const float *wrow[kRtE];
  const float *xrow[kRtT];
#pragma unroll
  for (uint32_t i = 0; i < kRtE; ++i) wrow[i] = r.weight + size_t(min(e0 + i, r.n_experts - 1)) * kHidden + lane * 4;
#pragma unroll
  for (uint32_t j = 0; j < kRtT; ++j) xrow[j] = X + size_t(min(t0 + j, tokens - 1)) * kHidden + lane * 4;
  float acc[kRtE][kRtT];
#pragma unroll
  for (uint32_t i = 0; i < kRtE; ++i)
#pragma unroll
    for (uint32_t j = 0; j < kRtT; ++j) acc[i][j] = 0.0f;
#pragma unroll 1
  for (uint32_t c = 0; c < kHidden / 256; ++c) {
    float4 wv[kRtE], xv[kRtT];
#pragma unroll
    for (uint32_t i = 0; i < kRtE; ++i) wv[i] = *reinterpret_cast<const float4 *>(wrow[i] + c * 256);
#pragma unroll
    for (uint32_t j = 0; j < kRtT; ++j) xv[j] = *reinterpret_cast<const float4 *>(xrow[j] + c * 256);
#pragma unroll
    for (uint32_t i = 0; i < kRtE; ++i)
#pragma unroll
      for (uint32_t j = 0; j < kRtT; ++j) {
        float a = acc[i][j];
        a = __fmaf_rn(wv[i].x, xv[j].x, a);
        a = __fmaf_rn(wv[i].y, xv[j].y, a);
        a = __fmaf_rn(wv[i].z, xv[j].z, a);
        a = __fmaf_rn(wv[i].w, xv[j].w, a);
        acc[i][j] = a;
      }
  }
  // router_score's xor butterfly for all 64 logits at once, transposed: after
  // the six steps lane l holds logit l = (expert l / kRtT, token l % kRtT)
  float v64[64], v32[32], v16[16], v8[8], v4[4], v2[2], v1[1];
#pragma unroll
  for (uint32_t i = 0; i < kRtE; ++i)
#pragma unroll
    for (uint32_t j = 0; j < kRtT; ++j) v64[i * kRtT + j] = acc[i][j];
  rt_reduce_step<32, 32>(v64, v32);
  rt_reduce_step<16, 16>(v32, v16);
  rt_reduce_step<8, 8>(v16, v8);
  rt_reduce_step<4, 4>(v8, v4);
  rt_reduce_step<2, 2>(v4, v2);
  rt_reduce_step<1, 1>(v2, v1);
  const uint32_t e = e0 + lane / kRtT, t = t0 + lane % kRtT;
  if (e < r.n_experts && t < tokens) {
    const float2 sc = router_finish(r, v1[0], e);
    scores[t * kMaxExperts + e] = sc.x;
    biased[t * kMaxExperts + e] = sc.y;
  }
}

// Plan of one token (one wavefront): top-k of score + bias (ties to the
// lower index) and its weights s/sum (sum sequential in selection order)
// times route_scale (executor.py:647-667), into the LDS lists.  `lead`: this
// wavefront also reports (status bits, ids_out, weights_out); several
// workgroups may plan the same token, one of them reports.
struct PlanLds {
  uint32_t ids[kMaxTokens][kTopK];
  float wts[kMaxTokens][kTopK];
  uint64_t pgs[kMaxTokens][kTopK];
};
__device__ __forceinline__ void plan_token(const RouteSpec &rs, uint32_t t, const float *biased, const float *scores,
                                           const uint64_t *pages, PlanLds &pl, bool lead = true) {
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t k = rs.r.topk;
  bool bad = false;
  const TopK c = rs.r.tid2eid ? select_hash_from(LdsScoreLoad{scores, pages}, rs.r, t, bad)
                              : select_topk_lds(biased, scores, pages, rs.r.n_experts, k);
  float wgt = lane < k ? route_weight(c, rs.r.route_scale) : 0.0f;
  bad = bad || !route_weights_valid(wgt, k, rs.r.route_scale);
  if (bad && lead && lane == 0)
    __hip_atomic_fetch_or(rs.status, kStatusBadRoute, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (lane < k) {
    uint32_t id = c.id;
    uint64_t pg = c.page;
    if (bad) {
      // a route that fails validate_for: distinct placeholder experts (so the
      // pair table stays well formed) on the shared page, NaN weights
      id = lane;
      pg = reinterpret_cast<uint64_t>(rs.shared_page);
      wgt = __builtin_nanf("");
    } else if (pages && pg == 0ull) {
      // a chosen expert without a resident page: its pair reads the shared
      // page instead (mapped memory; the result is discarded) and its NaN
      // weight makes the token's output NaN; the status word says why
      if (lead) __hip_atomic_fetch_or(rs.status, kStatusNullPage, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      pg = reinterpret_cast<uint64_t>(rs.shared_page);
      wgt = __builtin_nanf("");
    }
    pl.ids[t][lane] = id;
    pl.wts[t][lane] = wgt;
    pl.pgs[t][lane] = pg;
    if (lead && rs.ids_out) rs.ids_out[t * k + lane] = uint16_t(id);
    if (lead && rs.weights_out) rs.weights_out[t * k + lane] = wgt;
  }
}

// Publication of the pair table by one wavefront: the (expert, token) pairs
// sorted expert-major, the shared pairs appended, the per-token slot records.
__device__ __forceinline__ void plan_publish(const RouteSpec &rs, PairTable *tab, const PlanLds &pl) {
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t k = rs.r.topk;
  const uint32_t T = rs.tokens, npr = T * k;  // routed pairs, <= 48
  const bool mine = lane < npr;
  const uint32_t mt = mine ? lane / k : 0u, mr = mine ? lane % k : 0u;
  const uint32_t me = mine ? pl.ids[mt][mr] : 0u;
  const uint32_t key = mine ? me * 8u + mt : 0xffffffffu;  // unique: an expert appears once per token
  uint32_t rank = 0, first = 1;
  for (uint32_t j = 0; j < npr; ++j) {
    const uint32_t kj = uint32_t(__builtin_amdgcn_readlane(int(key), int(j)));
    rank += kj < key ? 1u : 0u;
    if ((kj >> 3) == (key >> 3) && kj < key) first = 0;
  }
  if (mine) {
    const uint64_t pg = pl.pgs[mt][mr];
    tab->page[rank] = pg;
    tab->fmt[rank] = S14_PAGE_MXFP4;
    tab->token[rank] = mt;
    tab->weight[rank] = pl.wts[mt][mr];
    tab->slot_pair[mt][mr] = rank;
    tab->slot_page[mt][mr] = pg;
    tab->slot_fmt[mt][mr] = S14_PAGE_MXFP4;
    tab->slot_weight[mt][mr] = pl.wts[mt][mr];
    tab->slot_shared[mt][mr] = 0u;
  }
  const uint64_t firsts = __ballot(mine && first);
  if (lane < T) {
    const uint32_t sp = npr + lane;
    const uint64_t pg = reinterpret_cast<uint64_t>(rs.shared_page);
    tab->page[sp] = pg;
    tab->fmt[sp] = uint32_t(rs.shared_fmt);
    tab->token[sp] = lane;
    tab->weight[sp] = 1.0f;
    tab->slot_pair[lane][k] = sp;
    tab->slot_page[lane][k] = pg;
    tab->slot_fmt[lane][k] = uint32_t(rs.shared_fmt);
    tab->slot_weight[lane][k] = 1.0f;
    tab->slot_shared[lane][k] = 1u;
    tab->npairs[lane] = k + 1;
  }
  if (lane == 0) {
    tab->n_pairs = npr + T;
    tab->n_tokens = T;
    tab->n_distinct = uint32_t(__popcll(firsts));
    tab->chain = 0u;
  }
}

// Router and plan in one launch.  Every workgroup (W = blockDim.x / 64
// wavefronts, W = route_waves(T)) scores W experts of one token, one
// wavefront each; the last workgroup to finish gathers all scores, selects
// every token's top-k (wavefront w takes tokens w, w + W, ...) and publishes
// the pair table.  Completion is counted in two levels so that no counter
// takes more than kRouteGroup increments: workgroups in groups of
// kRouteGroup (by linear index), then groups; each level's last arrival
// resets its counter.  expert_pages == NULL: route only.  Saves a dependent
// kernel launch per layer.
//
// kScoresOnly (single-token layers): the launch only scores; every phase-1
// workgroup of a routed pair then selects the top-k itself from the scores
// (route_pair), so no workgroup waits for a last arrival.
//
// kRequantX (official layers): one more column of workgroups, past the
// scoring ones (one per token), requantises the token's x for the official
// expert (group 128, l42_reference.py:390-403) into ws.xq, in parallel with
// the scoring, and (blocks) records the exponent range of the requantised
// values in ws.xwin (the block engine's decode window); phase 1 then reads those
// values as the exact phase 1 reads x, instead of every phase-1 workgroup
// requantising x itself.  These workgroups are not counted in the
// last-arrival hand-off, so the plan never waits for them.
constexpr uint32_t kRouteGroup = 16;
constexpr uint32_t kSingleRouteWaves = 4;  // route_waves(1)

// The requant workgroup of token t, NT = blockDim.x threads, x's loads all
// in flight at once; kWindow: also x's window (the block engine's).
// xs: LDS for kHidden floats, red: 2 NT / 64 ints.
template <uint32_t NT, bool kWindow>
__device__ __forceinline__ void route_requant_x(const Workspace &ws, const float *__restrict__ X, uint32_t t,
                                                float *xs, int *red) {
  static_assert(NT % 64 == 0 && NT <= 64 * kMaxTokens, "whole wavefronts, at most the route workgroup's");
  // no bounds test on the loads: the compiler cannot prove threadIdx.x < NT,
  // so a test would put each load behind a branch and a wait
  static_assert((kHidden / 4) % NT == 0, "whole float4 sweeps");
  constexpr uint32_t W = NT / 64, IT = kHidden / 4 / NT;
  const uint32_t wave = threadIdx.x >> 6;
  const float4 *src = reinterpret_cast<const float4 *>(X + size_t(t) * kHidden);
  float4 v[IT];
#pragma unroll
  for (uint32_t it = 0; it < IT; ++it) v[it] = src[it * NT + threadIdx.x];
#pragma unroll
  for (uint32_t it = 0; it < IT; ++it) reinterpret_cast<float4 *>(xs)[it * NT + threadIdx.x] = v[it];
  __syncthreads();
  int lo = 255, hi = 0;
  requant128_groups(xs, kHidden / 128, int(wave), int(W), lo, hi);
  if constexpr (kWindow) {
    lo = wave_min_i(lo);
    hi = wave_max_i(hi);
    if ((threadIdx.x & 63) == 0) {
      red[2 * wave] = lo;
      red[2 * wave + 1] = hi;
    }
  }
  __syncthreads();
  float4 *dst = reinterpret_cast<float4 *>(ws.xq + size_t(t) * kHidden);
  for (uint32_t i = threadIdx.x; i < kHidden / 4; i += blockDim.x) dst[i] = reinterpret_cast<const float4 *>(xs)[i];
  if (kWindow && threadIdx.x == 0) {
    for (uint32_t w = 0; w < W; ++w) {
      lo = min(lo, red[2 * w]);
      hi = max(hi, red[2 * w + 1]);
    }
    ws.xwin[t] = uint32_t(lo) | (uint32_t(hi) << 16);
  }
}

template <bool kScoresOnly, bool kRequantX = false>
__global__ __launch_bounds__(64 * kMaxTokens) void k_route(RouteSpec rs, Workspace ws, const float *__restrict__ X) {
  if constexpr (kRequantX) {
    // the requant column (uniform): past the scoring columns; tested with
    // the values the scoring needs anyway (gridDim would be one more
    // dependent scalar load ahead of every scoring workgroup's loads)
    if (blockIdx.x * (blockDim.x >> 6) >= rs.r.n_experts) {
      __shared__ float rq_xs[kHidden];
      __shared__ int rq_red[2 * kMaxTokens];
      if (blockDim.x == 256)
        route_requant_x<256, !kScoresOnly>(ws, X, blockIdx.y, rq_xs, rq_red);
      else
        route_requant_x<64 * kMaxTokens, !kScoresOnly>(ws, X, blockIdx.y, rq_xs, rq_red);
      return;
    }
  }
  // the scoring workgroups' grid (without the requant column)
  const uint32_t gx = kRequantX ? gridDim.x - 1 : gridDim.x;
  __shared__ float sc[kMaxTokens][kMaxExperts];
  __shared__ float bs[kMaxTokens][kMaxExperts];
  __shared__ uint64_t pages[kMaxExperts];
  __shared__ PlanLds pl;
  __shared__ uint32_t is_last;
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t W = blockDim.x >> 6;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t t = blockIdx.y;
  const uint32_t e = blockIdx.x * W + wave;
  if (e < rs.r.n_experts) {
    // blocks: expert 0's wavefront also records the token's x window for
    // the block engine's phase 1 (official: the requant column records xq's)
    const float2 s = router_score(rs.r, X, t, e, (!kScoresOnly && !kRequantX && e == 0) ? ws.xwin + t : nullptr);
    if (lane == 0) {
      // device-coherent stores (no cache writeback needed to publish them)
      __hip_atomic_store(&ws.scores[t * kMaxExperts + e], s.x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&ws.biased[t * kMaxExperts + e], s.y, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  if constexpr (kScoresOnly) return;  // the kernel boundary publishes the scores
  // Why the last workgroup sees every score without a release/acquire pair:
  //  1. the scores are agent-scope atomic stores (global_store ... sc1),
  //     written through to the device's coherence point rather than left
  //     dirty in this XCD's L2;
  //  2. s_waitcnt 0 returns only when this wavefront's stores are
  //     acknowledged there, and the barrier below puts every wavefront's
  //     wait before thread 0's counter increment;
  //  3. the counters are agent-scope atomics, performed at that same point,
  //     so the increment that completes the count comes after every counted
  //     workgroup's stores;
  //  4. the gather's loads are agent-scope atomic loads (sc1, served at the
  //     coherence point, not from a stale L2 line), issued only after the
  //     last increment returned (they depend on is_last through a barrier).
  // A device-scope release fence per wavefront would do the same by writing
  // the whole L2 back (buffer_wbl2), measured at several us per launch.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t n = gx * gridDim.y, id = blockIdx.y * gx + blockIdx.x;
    const uint32_t g = id / kRouteGroup, ng = (n + kRouteGroup - 1) / kRouteGroup;
    const uint32_t gsize = min(kRouteGroup, n - g * kRouteGroup);
    uint32_t *grp = ws.route_count + kRouteCounterStride * (1 + g);
    bool last = __hip_atomic_fetch_add(grp, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gsize - 1;
    if (last) {
      __hip_atomic_store(grp, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last = __hip_atomic_fetch_add(ws.route_count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == ng - 1;
      if (last) __hip_atomic_store(ws.route_count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    is_last = last;
  }
  __syncthreads();
  if (!is_last) return;  // uniform per workgroup
  // gather every (token, expert) score and the page table: all loads issued
  // before any is used
  // route_waves(T) >= T, so the T x 256 scores take at most kPer sweeps of the workgroup
  constexpr int kPer = kMaxExperts / 64;
  const uint32_t T = rs.tokens;
  const uint32_t nthr = blockDim.x, need = T * kMaxExperts;
  const bool with_pages = rs.expert_pages != nullptr;
  float gs[kPer], gb[kPer];
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const uint32_t i = threadIdx.x + uint32_t(j) * nthr;  // token i / 256, expert i % 256
    const bool in = i < need;
    gs[j] = in ? __hip_atomic_load(&ws.scores[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0.0f;
    gb[j] = in ? __hip_atomic_load(&ws.biased[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0.0f;
    if (uint32_t(j + 1) * nthr >= need) break;
  }
  for (uint32_t i = threadIdx.x; i < kMaxExperts; i += nthr)
    pages[i] = (with_pages && i < rs.r.n_experts) ? rs.expert_pages[i] : 0ull;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const uint32_t i = threadIdx.x + uint32_t(j) * nthr;
    if (i < need) {
      sc[i / kMaxExperts][i % kMaxExperts] = gs[j];
      bs[i / kMaxExperts][i % kMaxExperts] = gb[j];
    }
    if (uint32_t(j + 1) * nthr >= need) break;
  }
  __syncthreads();
  for (uint32_t tt = wave; tt < T; tt += W) plan_token(rs, tt, bs[tt], sc[tt], with_pages ? pages : nullptr, pl);
  if (!rs.expert_pages) return;  // route only (uniform)
  __syncthreads();
  if (wave == 0) plan_publish(rs, ws.table, pl);
}

// Wavefronts per route workgroup for T tokens: the last workgroup plans the
// tokens W at a time, and fewer wavefronts spread the scoring over more CUs.
inline uint32_t route_waves(uint32_t tokens) { return tokens <= 4 ? 4u : 8u; }
static_assert(kMaxTokens <= 8, "route_waves covers at most 8 tokens");

// Pair p of phase 1: from the host plan (by value; workgroup (0,0) also
// publishes it for phase 2), from the table the route kernel wrote, or
// planned here from the route kernel's scores (single token).
struct PairRef {
  const uint8_t *page;
  uint32_t fmt;
  uint32_t token;
  float weight;
};
enum : int { kPairFromTable = 0, kPairFromHost = 1, kPairFromScores = 2 };

// The single token's plan by a whole workgroup: its scores, biased scores
// and expert pages into LDS, then one wavefront selects the top-k exactly
// as the route kernel's last workgroup does (plan_token).  lead: that
// wavefront also reports the route and publishes the pair table for phase 2.
__device__ __forceinline__ const PlanLds &token_plan(const RouteSpec &rs, const Workspace &ws, bool lead) {
  __shared__ float rp_sc[kMaxExperts], rp_bs[kMaxExperts];
  __shared__ uint64_t rp_pages[kMaxExperts];
  __shared__ PlanLds rp_pl;
  const uint32_t n = rs.r.n_experts;
  for (uint32_t i = threadIdx.x; i < kMaxExperts; i += blockDim.x) {
    const bool in = i < n;
    rp_sc[i] = in ? ws.scores[i] : 0.0f;
    rp_bs[i] = in ? ws.biased[i] : 0.0f;
    rp_pages[i] = in ? rs.expert_pages[i] : 0ull;
  }
  __syncthreads();
  if (threadIdx.x < 64) {
    plan_token(rs, 0, rp_bs, rp_sc, rp_pages, rp_pl, lead);
    if (lead) plan_publish(rs, ws.table, rp_pl);
  }
  return rp_pl;
}

// Pair p of a single-token layer from the scores (whole workgroup, uniform
// result): the token's plan (token_plan) and its p-th choice in expert
// order, which is the pair table's order (plan_publish sorts pairs by
// expert, then token).  The shared pair (p = topk) needs no plan; its first
// workgroup reports the route and publishes the pair table after its rows
// (phase1_publish), where it has time to spare: the routed workgroups'
// rows start only after their plan.
__device__ __forceinline__ PairRef route_pair(const RouteSpec &rs, const Workspace &ws, uint32_t p) {
  __shared__ PairRef rp_mine;
  const uint32_t k = rs.r.topk;
  if (p >= k) return PairRef{rs.shared_page, uint32_t(rs.shared_fmt), 0u, 1.0f};
  const PlanLds &rp_pl = token_plan(rs, ws, false);
  if (threadIdx.x < 64) {
    const uint32_t lane = threadIdx.x;
    if (lane < k) {
      const uint32_t id = rp_pl.ids[0][lane];
      uint32_t rank = 0;
      for (uint32_t j = 0; j < k; ++j) rank += rp_pl.ids[0][j] < id ? 1u : 0u;
      if (rank == p)
        rp_mine = PairRef{reinterpret_cast<const uint8_t *>(rp_pl.pgs[0][lane]), uint32_t(S14_PAGE_MXFP4), 0u,
                          rp_pl.wts[0][lane]};
    }
  }
  __syncthreads();
  // the same in every lane: keep it in scalar registers (a per-lane page
  // address would put every buffer load in a readfirstlane loop)
  const uint64_t pg = reinterpret_cast<uint64_t>(rp_mine.page);
  return PairRef{reinterpret_cast<const uint8_t *>(
                     (uint64_t(uint32_t(__builtin_amdgcn_readfirstlane(int(pg >> 32)))) << 32) |
                     uint32_t(__builtin_amdgcn_readfirstlane(int(uint32_t(pg))))),
                 uint32_t(__builtin_amdgcn_readfirstlane(int(rp_mine.fmt))),
                 uint32_t(__builtin_amdgcn_readfirstlane(int(rp_mine.token))),
                 __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(rp_mine.weight)))};
}

// End of a phase-1 workgroup that planned from the scores: the shared
// pair's first workgroup reports the route and publishes the pair table
// (uniform per workgroup: every thread reaches token_plan's barrier).
template <int kSrc>
__device__ __forceinline__ void phase1_publish(const RouteSpec &rs, const Workspace &ws) {
  if constexpr (kSrc == kPairFromScores) {
    if (blockIdx.y == rs.r.topk && blockIdx.x == 0) (void)token_plan(rs, ws, true);
  }
}

template <int kSrc>
__device__ __forceinline__ PairRef phase1_pair(const PairTable &plan, const RouteSpec &rs, const Workspace &ws,
                                               uint32_t p) {
  PairTable *__restrict__ tab = ws.table;
  if constexpr (kSrc == kPairFromScores) return route_pair(rs, ws, p);
  if (kSrc == kPairFromHost) {
    if (blockIdx.x == 0 && blockIdx.y == 0) {
      const uint32_t *src = reinterpret_cast<const uint32_t *>(&plan);
      uint32_t *dst = reinterpret_cast<uint32_t *>(tab);
      for (uint32_t i = threadIdx.x; i < sizeof(PairTable) / 4; i += blockDim.x) dst[i] = src[i];
    }
    return PairRef{reinterpret_cast<const uint8_t *>(plan.page[p]), plan.fmt[p], plan.token[p], plan.weight[p]};
  }
  return PairRef{reinterpret_cast<const uint8_t *>(tab->page[p]), tab->fmt[p], tab->token[p], tab->weight[p]};
}

__device__ __forceinline__ uint32_t page_bytes(uint32_t fmt) {
  return fmt == S14_PAGE_MXFP4 ? uint32_t(S14_EXPERT_PAGE_BYTES) : uint32_t(S14_SHARED_EXPERT_PAGE_BYTES);
}

// Phase 1 EXACT: one workgroup of kP1ExactWaves wavefronts per (tile group,
// pair), the pair's x staged in LDS once for all of them; each wavefront
// takes one 16-row tile: lanes 0-31 its rows of w1, lanes 32-63 the same
// rows of w3, one row per lane pair; h = swiglu(g, u) after a half swap.
// Single-token layers only (blocks of 2..8 tokens run the block engine);
// kTier = 1 keeps the kernel's name in line with the FAST kernels', whose
// tier picks their shape.
template <int kSrc, int kTier, bool kOfficial>
__global__ __launch_bounds__(64 * kP1ExactWaves) void k_phase1_exact(PairTable plan, RouteSpec rs, Workspace ws,
                                                                     const float *__restrict__ X, PageOffsets mx,
                                                                     PageOffsets f8) {
  static_assert(kTier == 1, "blocks run the block engine");
  __shared__ float xs[kHidden];
  __shared__ double exptab[32];
  __shared__ int red[2 * kP1ExactWaves];
  exp_table_fill(exptab);  // published by the barrier in the x copy
  const uint32_t p = blockIdx.y;
  const PairRef pr = phase1_pair<kSrc>(plan, rs, ws, p);
  const uint32_t lane = threadIdx.x & 63, h = lane & 1u;
  const uint32_t tile = blockIdx.x * kP1ExactWaves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const bool upper = lane >= 32;
  const uint32_t row = tile * kP1ExactRows + ((lane & 31u) >> 1);
  const Rsrc r = make_rsrc(pr.page, page_bytes(pr.fmt));
  const Src1 src{r, r};
  // official, one token: the route launch already requantised x (ws.xq)
  constexpr bool kXq = kOfficial && kSrc == kPairFromScores;
  const float *const srcx = (kXq ? ws.xq : X) + size_t(pr.token) * kHidden;
  float acc;
  if (pr.fmt == S14_PAGE_MXFP4) {
    const uint32_t woff = uint32_t(upper ? mx.w3 : mx.w1) + row * (kHidden / 2) + 8u * h;
    const uint32_t soff = uint32_t(upper ? mx.s3 : mx.s1) + row * (kHidden / 32);
    MxBatch<kPF> ba;
    mx_load<kPF>(ba, src, woff, soff, 0);  // first weights in flight during the x copy
    // one wavefront per SIMD, issue-bound: one code check per row
    RowCodes<kHidden / 32> rc;
    load_row_codes<kHidden / 32>(rc, src, soff);
    CodeWindow win = stage_x_block<kHidden, 64 * kP1ExactWaves>(xs, srcx, red);
    if constexpr (kOfficial && !kXq) win = requant128_block<64 * kP1ExactWaves>(xs, kHidden, red);
    acc = mx_row_pair_fixed<kPF, kHidden / 32>(0.0f, ba, src, woff, soff, xs + 16 * h, win, rc);
  } else {
    const uint32_t woff = uint32_t(upper ? f8.w3 : f8.w1) + row * kHidden + 16u * h;
    const uint32_t soff = uint32_t(upper ? f8.s3 : f8.s1) + (row / 128) * (kHidden / 128);
    stage_x_block<kHidden, 64 * kP1ExactWaves>(xs, srcx, red);
    if constexpr (kOfficial && !kXq) requant128_block<64 * kP1ExactWaves>(xs, kHidden, red);
    acc = fp8_row_pair(0.0f, src, woff, soff, 0, kHidden / 32, xs + 16 * h);
  }
  const float other = lane_xor32(acc);
  const bool writer = !upper && h == 0;
  int lo = 255, hi = 0;
  if (writer) {
    float hv;
    if constexpr (kOfficial) {
      // g and u rounded to bf16; h = bf16(swiglu(g, u) * w), the route weight
      // before w2 (1 for the shared expert) (executor.py:717-731)
      hv = bf16_round(__fmul_rn(swiglu_exact(bf16_round(acc), bf16_round(other), exptab), pr.weight));
    } else {
      hv = swiglu_exact(acc, other, exptab);
    }
    ws.h[size_t(p) * kInter + row] = hv;
    exp_range_acc(hv, lo, hi);
  }
  // the tile's exponent range, so that phase 2 gets h's decode window
  // without scanning h
  lo = wave_min_i(lo);
  hi = wave_max_i(hi);
  if (lane == 0) ws.hwin[size_t(p) * kP1Tiles + tile] = uint32_t(lo) | (uint32_t(hi) << 16);
  phase1_publish<kSrc>(rs, ws);
}

// Phase 1 FAST: 4 wavefronts per workgroup; each streams p1_fast_rows_per_wave
// row pairs (the same row of w1 and of w3) with kP1FastDepth row pairs of
// codes in flight, x for the lane's k slices held in registers throughout
// (read from one LDS copy per workgroup).
// The grid stays within one round of resident workgroups: a workgroup that
// starts only when another finishes costs a whole extra load latency.
template <int kSrc, int kTier>
__global__ __launch_bounds__(256) void k_phase1_fast(PairTable plan, RouteSpec rs, Workspace ws,
                                                     const float *__restrict__ X, PageOffsets mx, PageOffsets f8) {
  constexpr int NSEG = kHidden / 2048;
  constexpr int R = p1_fast_rows_per_wave(kTier);
  constexpr int D = kP1FastDepth;
  const uint32_t p = blockIdx.y;
  const PairRef pr = phase1_pair<kSrc>(plan, rs, ws, p);
  const uint32_t row0 = blockIdx.x * p1_fast_rows(kTier) + (threadIdx.x >> 6) * R;
  const Rsrc r = make_rsrc(pr.page, page_bytes(pr.fmt));
  const int lane = threadIdx.x & 63;
  float gv = 0.0f, uv = 0.0f;  // lane i keeps row pair i
  __shared__ float xs[kHidden];
  XReg<NSEG> xr;
  if (pr.fmt == S14_PAGE_MXFP4) {
    MxRowFrag f1[D][NSEG], f3[D][NSEG];
    auto load = [&](int slot, uint32_t row) {
      load_mx_row_frag<NSEG>(f1[slot], r, uint32_t(mx.w1) + row * (kHidden / 2), r,
                             uint32_t(mx.s1) + row * (kHidden / 32), kHidden);
      load_mx_row_frag<NSEG>(f3[slot], r, uint32_t(mx.w3) + row * (kHidden / 2), r,
                             uint32_t(mx.s3) + row * (kHidden / 32), kHidden);
    };
#pragma unroll
    for (int i = 0; i < D && i < R; ++i) load(i, row0 + i);
    {
      // x once per workgroup through LDS (each wavefront loading all 16 KiB of
      // it from L2 cost 29 MB of L2 reads per K=1 launch), while the first
      // row pairs are in flight
      const float *src = X + size_t(pr.token) * kHidden;
      float4 v[kHidden / 1024];
#pragma unroll
      for (int it = 0; it < kHidden / 1024; ++it) v[it] = *reinterpret_cast<const float4 *>(src + (it * 256 + threadIdx.x) * 4);
#pragma unroll
      for (int it = 0; it < kHidden / 1024; ++it) *reinterpret_cast<float4 *>(xs + (it * 256 + threadIdx.x) * 4) = v[it];
      __syncthreads();
      load_x_mx<NSEG>(xr, xs, kHidden);
    }
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int slot = i % D;
      const float g = wave_sum_dpp(mx_row_fast_partial<NSEG>(f1[slot], xr));
      const float u = wave_sum_dpp(mx_row_fast_partial<NSEG>(f3[slot], xr));
      if (i + D < R) load(slot, row0 + i + D);
      if (lane == i) {
        gv = g;
        uv = u;
      }
    }
  } else {
    load_x_mx<NSEG>(xr, X + size_t(pr.token) * kHidden, kHidden);
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const uint32_t row = row0 + i;
      const float g = wave_sum_dpp(fp8_row_fast_partial<NSEG>(r, uint32_t(f8.w1) + row * kHidden,
                                                              uint32_t(f8.s1) + (row / 128) * (kHidden / 128), xr));
      const float u = wave_sum_dpp(fp8_row_fast_partial<NSEG>(r, uint32_t(f8.w3) + row * kHidden,
                                                              uint32_t(f8.s3) + (row / 128) * (kHidden / 128), xr));
      if (lane == i) {
        gv = g;
        uv = u;
      }
    }
  }
  if (lane < R) ws.h[size_t(p) * kInter + row0 + lane] = swiglu_exact(gv, uv);
  phase1_publish<kSrc>(rs, ws);
}

// What every phase-2 workgroup needs about its token, read in one round trip
// at kernel start: lane j (< kSlots) holds slot j's route weight and shared
// flag.
struct SlotInfo {
  uint32_t np, chain;
  float w;
  uint32_t shared;
};
__device__ __forceinline__ SlotInfo load_slot_info(const PairTable *__restrict__ tab, uint32_t t) {
  const uint32_t j = min(threadIdx.x & 63, uint32_t(kSlots - 1));
  return SlotInfo{tab->npairs[t], tab->chain, tab->slot_weight[t][j], tab->slot_shared[t][j]};
}

// Phase 2 accumulation of one row tile of token t from part[slot][row]:
// acc = 0; acc += w * down (routed, route order); acc += down (shared) — or
// y = w * down for the single-expert chain (s14_vulkan_numeric.rs:929-946,
// :1300).  Called by one whole wavefront.
template <int ROWS, bool kOfficial = false>
__device__ __forceinline__ void phase2_accumulate(const SlotInfo &si, const float (*part)[ROWS], uint32_t t,
                                                  uint32_t row0, float *__restrict__ Y) {
  const uint32_t lane = threadIdx.x & 63;
  const bool row_lane = lane < uint32_t(ROWS);
  // every slot's value first (the LDS reads pipeline), then the adds in
  // route order
  float d[kSlots];
#pragma unroll
  for (uint32_t j = 0; j < uint32_t(kSlots); ++j) d[j] = (row_lane && j < si.np) ? part[j][lane] : 0.0f;
  float acc = 0.0f;
  if constexpr (kOfficial) {
    // official semantics: each slot's bf16 output already carries its route
    // weight; acc = 0; acc += out_j in route order, shared last; y =
    // bf16(acc) (executor.py:712-739)
#pragma unroll
    for (uint32_t j = 0; j < uint32_t(kSlots); ++j) {
      if (j >= si.np) break;
      acc = __fadd_rn(acc, d[j]);
    }
    acc = bf16_round(acc);
  } else if (si.chain) {
    const float w = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(si.w), 0));
    acc = __fmul_rn(w, d[0]);
  } else {
#pragma unroll
    for (uint32_t j = 0; j < uint32_t(kSlots); ++j) {
      if (j >= si.np) break;
      const float w = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(si.w), int(j)));
      const uint32_t shared = uint32_t(__builtin_amdgcn_readlane(int(si.shared), int(j)));
      acc = shared ? __fadd_rn(acc, d[j]) : __fadd_rn(acc, __fmul_rn(w, d[j]));
    }
  }
  if (row_lane) Y[size_t(t) * kHidden + row0 + lane] = acc;
}

// Phase 2 EXACT: one workgroup of kP2ExactWaves wavefronts per (16-row tile,
// token).  Wavefront w serves the token's pair slots 2w (lanes 0-31) and
// 2w+1 (lanes 32-63), one row per lane pair, with each slot's h staged in
// LDS (row stride padded so the two slots' reads fall in different banks).
constexpr int kHStride = kInter + 8;

// Official mode: the w2 input's act_quant (group 128, l42_reference.py:390-403)
// of every pair's h, in place, once per launch, between phase 1 and phase
// 2 (each phase-2 workgroup requantising its own copies of its slots' h
// took phase 2 from 12.5 to 26 us at K=1).  Eight lanes per (pair, 128
// values), each lane one 16-value phase-1 tile: the group's maximum by xor
// shuffles within the eight (a NaN never compares greater, as in the
// oracle's scan), and the tile's exponent range into hwin, which gives
// phase 2 the decode window of the requantised h.
constexpr uint32_t kHGroups128 = kInter / 128;
__global__ __launch_bounds__(256) void k_requant_h_official(Workspace ws, uint32_t n_pairs) {
  const uint32_t gid = blockIdx.x * 256u + threadIdx.x;
  const uint32_t j = gid & 7u, grp = gid >> 3;  // tile j of group grp = (pair, m)
  const uint32_t p = grp / kHGroups128, m = grp % kHGroups128;
  if (p >= n_pairs) return;  // whole groups of eight lanes return together
  float4 *v = reinterpret_cast<float4 *>(ws.h + size_t(p) * kInter + 128u * m + 16u * j);
  float4 q[4];
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    q[i] = v[i];
    amax = fabsf(q[i].x) > amax ? fabsf(q[i].x) : amax;
    amax = fabsf(q[i].y) > amax ? fabsf(q[i].y) : amax;
    amax = fabsf(q[i].z) > amax ? fabsf(q[i].z) : amax;
    amax = fabsf(q[i].w) > amax ? fabsf(q[i].w) : amax;
  }
#pragma unroll
  for (int d = 1; d < 8; d <<= 1) {
    const float o = __shfl_xor(amax, d);
    amax = o > amax ? o : amax;
  }
  const uint32_t code = requant_code(amax);
  const float inv = __uint_as_float((254u - code) << 23), sc = __uint_as_float(code << 23);
  auto rq = [&](float a) { return __fmul_rn(e4m3_f32(s14x::e4m3_rne_sat(__fmul_rn(a, inv))), sc); };
  int lo = 255, hi = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    q[i] = make_float4(rq(q[i].x), rq(q[i].y), rq(q[i].z), rq(q[i].w));
    exp_range_acc(q[i].x, lo, hi);
    exp_range_acc(q[i].y, lo, hi);
    exp_range_acc(q[i].z, lo, hi);
    exp_range_acc(q[i].w, lo, hi);
    v[i] = q[i];
  }
  ws.hwin[size_t(p) * kP1Tiles + 8u * m + j] = uint32_t(lo) | (uint32_t(hi) << 16);
}

template <int kTier, bool kOfficial>
__global__ __launch_bounds__(64 * kP2ExactWaves) void k_phase2_exact(const PairTable *__restrict__ tab,
                                                                     const float *__restrict__ H,
                                                                     const uint32_t *__restrict__ hwin,
                                                                     float *__restrict__ Y, PageOffsets mx,
                                                                     PageOffsets f8) {
  static_assert(kTier == 1, "blocks run the block engine");
  __shared__ float hs[kSlots][kHStride];
  __shared__ float part[kSlots][kP2ExactRows];
  const uint32_t t = blockIdx.y;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  // slot records of both of this wavefront's slots, read unconditionally (in
  // one round trip with the token's pair count); b falls back to a when absent
  const uint32_t sa = 2 * wave, sb = min(2 * wave + 1, uint32_t(kSlots - 1));
  const SlotInfo si = load_slot_info(tab, t);
  const uint32_t qa = tab->slot_pair[t][sa], qb = tab->slot_pair[t][sb];
  const uint32_t ga = tab->slot_fmt[t][sa], gb = tab->slot_fmt[t][sb];
  const uint64_t ua = tab->slot_page[t][sa], ub = tab->slot_page[t][sb];
  const uint32_t np = si.np;
  const bool has_a = sa < np, has_b = 2 * wave + 1 < np;
  const uint32_t pa = qa, pb = has_b ? qb : qa;
  const uint32_t fa = ga, fb = has_b ? gb : ga;
  const bool hi = lane >= 32;
  const uint32_t h = lane & 1u, r = (lane & 31u) >> 1;
  const uint32_t row = blockIdx.x * kP2ExactRows + r;
  const uint32_t slot = (hi && has_b) ? sb : sa;
  const Src2 src{make_rsrc(reinterpret_cast<const uint8_t *>(ua), page_bytes(fa)),
                 make_rsrc(reinterpret_cast<const uint8_t *>(has_b ? ub : ua), page_bytes(fb)), hi};
  const bool mine_mx = (hi ? fb : fa) == S14_PAGE_MXFP4;
  const uint32_t mx_woff = uint32_t(mx.w2) + row * (kInter / 2) + 8u * h;
  const uint32_t mx_soff = uint32_t(mx.s2) + row * (kInter / 32);
  // both halves MXFP4 (the normal case): per-lane page pointers
  const SrcP srcp{(GPtr)(hi && has_b ? ub : ua)};
  MxBatch<kPF> ba;
  RowCodes<kInter / 32> rc;
  if (has_a && fa == S14_PAGE_MXFP4 && fb == S14_PAGE_MXFP4) {
    mx_load<kPF>(ba, srcp, mx_woff, mx_soff, 0);  // first weights and the row's codes in flight during the h copy
    load_row_codes<kInter / 32>(rc, srcp, mx_soff);
  }
  // h loads first, then the window words (whose reduction waits for them)
  CodeWindow win[2] = {{256, 0}, {256, 0}};
  if (has_b) {
    float *const dst[2] = {hs[sa], hs[sb]};
    const float *const srch[2] = {H + size_t(pa) * kInter, H + size_t(pb) * kInter};
    StageRegs<kInter, 2> hr;
    stage_load_wave<kInter, 2>(hr, srch);
    win[0] = h_window(hwin + size_t(pa) * kP1Tiles);
    win[1] = h_window(hwin + size_t(pb) * kP1Tiles);
    stage_store_wave<kInter, 2>(dst, hr);
  } else if (has_a) {
    float *const dst[1] = {hs[sa]};
    const float *const srch[1] = {H + size_t(pa) * kInter};
    StageRegs<kInter, 1> hr;
    stage_load_wave<kInter, 1>(hr, srch);
    win[0] = win[1] = h_window(hwin + size_t(pa) * kP1Tiles);
    stage_store_wave<kInter, 1>(dst, hr);
  }
  __syncthreads();
  if (has_a) {
    const float *xh = hs[slot] + 16 * h;
    float acc;
    if (fa == S14_PAGE_MXFP4 && fb == S14_PAGE_MXFP4) {
      acc = mx_row_pair_fixed<kPF, kInter / 32>(0.0f, ba, srcp, mx_woff, mx_soff, xh, (hi ? win[1] : win[0]), rc);
    } else if (mine_mx) {  // formats differ between the halves
      MxBatch<kPF> bm;
      mx_load<kPF>(bm, src, mx_woff, mx_soff, 0);
      acc = mx_row_pair<kPF>(0.0f, bm, src, mx_woff, mx_soff, kInter / 32, xh, (hi ? win[1] : win[0]));
    } else {
      acc = fp8_row_pair(0.0f, src, uint32_t(f8.w2) + row * kInter + 16u * h,
                         uint32_t(f8.s2) + (row / 128) * (kInter / 128), 0, kInter / 32, xh);
    }
    if constexpr (kOfficial) acc = bf16_round(acc);  // w2's output rounded to bf16
    if (h == 0 && (!hi || has_b)) part[slot][r] = acc;
  }
  __syncthreads();
  if (wave == 0) phase2_accumulate<kP2ExactRows, kOfficial>(si, part, t, blockIdx.x * kP2ExactRows, Y);
}

// Phase 2 FAST: wavefront j computes kP2FastRows w2 rows of the token's j-th
// pair.
constexpr int kP2FastWaves = kTopK + 1;

template <int kTier>
__global__ __launch_bounds__(64 * kP2FastWaves) void k_phase2_fast(const PairTable *__restrict__ tab,
                                                                   const float *__restrict__ H,
                                                                   float *__restrict__ Y, PageOffsets mx,
                                                                   PageOffsets f8) {
  constexpr int NSEG = kInter / 2048;
  constexpr int R = kP2FastRows;
  __shared__ float part[kP2FastWaves][R];
  const uint32_t t = blockIdx.y;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const uint32_t j = min(wave, uint32_t(kSlots - 1));
  const SlotInfo si = load_slot_info(tab, t);
  const uint32_t p = tab->slot_pair[t][j], fmt = tab->slot_fmt[t][j];
  const uint64_t page = tab->slot_page[t][j];
  const uint32_t row0 = blockIdx.x * R;
  if (wave < si.np) {
    XReg<NSEG> xr;
    load_x_mx<NSEG>(xr, H + size_t(p) * kInter, kInter);
    const Rsrc r = make_rsrc(reinterpret_cast<const uint8_t *>(page), page_bytes(fmt));
    float mine = 0.0f;
    if (fmt == S14_PAGE_MXFP4) {
      MxRowFrag f[R][NSEG];
#pragma unroll
      for (int i = 0; i < R; ++i) {
        const uint32_t row = row0 + i;
        load_mx_row_frag<NSEG>(f[i], r, uint32_t(mx.w2) + row * (kInter / 2), r,
                               uint32_t(mx.s2) + row * (kInter / 32), kInter);
      }
#pragma unroll
      for (int i = 0; i < R; ++i) {
        const float v = wave_sum_dpp(mx_row_fast_partial<NSEG>(f[i], xr));
        if (lane == uint32_t(i)) mine = v;
      }
    } else {
#pragma unroll
      for (int i = 0; i < R; ++i) {
        const uint32_t row = row0 + i;
        const float v = wave_sum_dpp(fp8_row_fast_partial<NSEG>(r, uint32_t(f8.w2) + row * kInter,
                                                                 uint32_t(f8.s2) + (row / 128) * (kInter / 128), xr));
        if (lane == uint32_t(i)) mine = v;
      }
    }
    if (lane < uint32_t(R)) part[wave][lane] = mine;
  }
  __syncthreads();
  if (wave == 0) phase2_accumulate<kP2FastRows>(si, part, t, row0, Y);
}

// The single-expert chain in EXACT order with lane quads (config 0: one
// pair, so lane pairs would leave seven of eight SIMDs idle).  Phase 1:
// workgroups of 4 wavefronts, each wavefront 8 rows of w1 (lanes 0-31) and
// the same 8 rows of w3 (lanes 32-63), x staged once per workgroup, h =
// swiglu(g, u) into ws.h (pair 0).  Phase 2: 16 rows of w2 per wavefront,
// h staged per workgroup, y = w * down (s14_vulkan_numeric.rs:1300).
constexpr int kChainQNB = 8;             // batches of 4 groups in flight per lane
constexpr uint32_t kChainP1Rows = 32;    // rows of h per workgroup
constexpr uint32_t kChainP2Rows = 64;    // rows of y per workgroup
__global__ __launch_bounds__(256) void k_chain_phase1_quad(const uint8_t *page, const float *__restrict__ X,
                                                           Workspace ws, PageOffsets mx) {
  __shared__ float xs[kHidden];
  __shared__ double exptab[32];
  __shared__ int red[8];
  exp_table_fill(exptab);  // published by the barrier in the x copy
  const uint32_t lane = threadIdx.x & 63, q = lane & 3u, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const bool upper = lane >= 32;
  const uint32_t row = blockIdx.x * kChainP1Rows + wave * 8u + ((lane & 31u) >> 2);
  const Rsrc r = make_rsrc(page, uint32_t(S14_EXPERT_PAGE_BYTES));
  const uint32_t woff = uint32_t(upper ? mx.w3 : mx.w1) + row * (kHidden / 2) + 4u * q;
  const uint32_t soff = uint32_t(upper ? mx.s3 : mx.s1) + row * (kHidden / 32);
  MxQBatch b[kChainQNB];
#pragma unroll
  for (int j = 0; j < kChainQNB; ++j) mxq_load(b[j], r, woff, soff, 4 * j);  // in flight during the x copy
  QuadCodes<kHidden / 32> qc;
  load_quad_codes<kHidden / 32>(qc, r, soff);
  const CodeWindow win = stage_x_block<kHidden, 256>(xs, X, red);
  const bool scaled = quad_codes_in<kHidden / 32>(qc, win);
  const float acc = mx_row_quad<kChainQNB, kHidden / 32>(b, r, woff, soff, xs + 8u * q, scaled);
  const float other = lane_xor32(acc);
  if (!upper && q == 0) ws.h[row] = swiglu_exact(acc, other, exptab);
}

__global__ __launch_bounds__(256) void k_chain_phase2_quad(const uint8_t *page, Workspace ws, float weight,
                                                           float *__restrict__ Y, PageOffsets mx) {
  __shared__ float hs[kInter];
  __shared__ int red[8];
  const uint32_t lane = threadIdx.x & 63, q = lane & 3u, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t row = blockIdx.x * kChainP2Rows + wave * 16u + (lane >> 2);
  const Rsrc r = make_rsrc(page, uint32_t(S14_EXPERT_PAGE_BYTES));
  const uint32_t woff = uint32_t(mx.w2) + row * (kInter / 2) + 4u * q;
  const uint32_t soff = uint32_t(mx.s2) + row * (kInter / 32);
  MxQBatch b[kChainQNB];
#pragma unroll
  for (int j = 0; j < kChainQNB; ++j) mxq_load(b[j], r, woff, soff, 4 * j);  // in flight during the h copy
  QuadCodes<kInter / 32> qc;
  load_quad_codes<kInter / 32>(qc, r, soff);
  const CodeWindow win = stage_x_block<kInter, 256>(hs, ws.h, red);
  const bool scaled = quad_codes_in<kInter / 32>(qc, win);
  const float acc = mx_row_quad<kChainQNB, kInter / 32>(b, r, woff, soff, hs + 8u * q, scaled);
  if (q == 0) Y[row] = __fmul_rn(weight, acc);
}

// EXACT FP8 matvec with lane quads (k % 32 == 0, k <= kQuadMaxK): 4
// wavefronts of 16 rows per workgroup, x staged once per workgroup as f32.
constexpr uint32_t kQuadMaxK = 8192;
__global__ __launch_bounds__(256) void k_fp8_matvec_exact_quad(uint32_t N, uint32_t K, const void *x, int x_bf16,
                                                              const uint8_t *__restrict__ w,
                                                              const void *__restrict__ sc, int scale_f32,
                                                              float *__restrict__ y) {
  __shared__ __attribute__((aligned(16))) float xs[kQuadMaxK];
  for (uint32_t i = threadIdx.x; i < K; i += blockDim.x)
    xs[i] = x_bf16 ? bf16_f32(reinterpret_cast<const uint16_t *>(x)[i]) : reinterpret_cast<const float *>(x)[i];
  __syncthreads();
  const uint32_t lane = threadIdx.x & 63u, q = lane & 3u;
  const uint32_t row = blockIdx.x * 64u + (threadIdx.x >> 6) * 16u + (lane >> 2);
  const uint32_t rr = row < N ? row : N - 1u;
  const uint32_t kg = K / 128u + (K % 128u ? 1u : 0u);
  const uint32_t ntile = ((N + 127u) / 128u) * kg;
  const Rsrc rw = make_rsrc(w, N * K), rs = make_rsrc(sc, scale_f32 ? 4u * ntile : ntile);
  const uint32_t soff = (scale_f32 ? 4u : 1u) * ((rr / 128u) * kg);
  constexpr int kNB = 8;
  const float v = fp8_row_quad<kNB>(rw, rs, rr * K + 8u * q, soff, scale_f32, int(K / 32u), xs + 8u * q);
  if (q == 0 && row < N) y[row] = v;
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
    k_mxfp4_matvec_exact<<<blocks_for(N, 32), 64, 0, s>>>(N, K, d.x, d.weight, d.scale, d.y);
  }
  return hipGetLastError();
}

hipError_t launch_fp8_matvec(hipStream_t s, const s14_fp8_dispatch &d) {
  const uint32_t N = d.shape.n, K = d.shape.k;
  const int xb = d.x_dtype == S14_X_BF16, sf = d.scale_dtype == S14_SCALE_F32;
  if (d.mode == S14_MODE_FAST && K % 16 == 0 && K <= 8192) {
    const unsigned grid = blocks_for(N, 4);
    if (K <= 1024)
      k_fp8_matvec_fast<1><<<grid, 256, 0, s>>>(N, K, d.x, xb, d.weight, d.scale, sf, d.y);
    else if (K <= 2048)
      k_fp8_matvec_fast<2><<<grid, 256, 0, s>>>(N, K, d.x, xb, d.weight, d.scale, sf, d.y);
    else if (K <= 4096)
      k_fp8_matvec_fast<4><<<grid, 256, 0, s>>>(N, K, d.x, xb, d.weight, d.scale, sf, d.y);
    else
      k_fp8_matvec_fast<8><<<grid, 256, 0, s>>>(N, K, d.x, xb, d.weight, d.scale, sf, d.y);
  } else if (K % 32 == 0 && K <= kQuadMaxK && (K / 32) % 32 == 0) {
    // lane quads: the standalone matvec has few rows per SIMD
    k_fp8_matvec_exact_quad<<<blocks_for(N, 64), 256, 0, s>>>(N, K, d.x, xb, d.weight, d.scale, sf, d.y);
  } else if (K % 32 == 0) {
    k_fp8_matvec_exact<true><<<blocks_for(N, 32), 64, 0, s>>>(N, K, d.x, xb, d.weight, d.scale, sf, d.y);
  } else {
    k_fp8_matvec_exact<false><<<blocks_for(N, 32), 64, 0, s>>>(N, K, d.x, xb, d.weight, d.scale, sf, d.y);
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

namespace {
__global__ void k_clear_u32(uint32_t *p, uint32_t n) {
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0u;
}
}  // namespace

hipError_t launch_clear_route_counters(hipStream_t s, const Workspace &ws) {
  k_clear_u32<<<1, 256, 0, s>>>(ws.route_count, kRouteCounters);
  k_clear_u32<<<1, 256, 0, s>>>(ws.sync, kSyncLines * kRouteCounterStride);
  return hipGetLastError();
}

hipError_t launch_router_scores(hipStream_t s, const Workspace &ws, const RouterArgs &r, uint32_t tokens,
                                const float *x, KernelEvents ev, int requant, uint8_t *q, uint8_t *qs) {
  const uint32_t gx = (r.n_experts + 4 * kRtE - 1) / (4 * kRtE), tiles = (tokens + kRtT - 1) / kRtT;
  if (requant == 0) {
    hipExtLaunchKernelGGL(k_router_scores<0>, dim3(gx, tiles), dim3(256), 0, s, ev.start, ev.stop, 0, r, tokens, x,
                          ws.scores, ws.biased, q, qs);
    return hipGetLastError();
  }
  const uint32_t rq_blocks = (tokens * (kHidden / 32) + 255) / 256;
  const dim3 grid(gx, tiles + (rq_blocks + gx - 1) / gx);
  if (requant == 2)
    hipExtLaunchKernelGGL(k_router_scores<2>, grid, dim3(256), 0, s, ev.start, ev.stop, 0, r, tokens, x, ws.scores,
                          ws.biased, q, qs);
  else
    hipExtLaunchKernelGGL(k_router_scores<1>, grid, dim3(256), 0, s, ev.start, ev.stop, 0, r, tokens, x, ws.scores,
                          ws.biased, q, qs);
  return hipGetLastError();
}

hipError_t launch_route(hipStream_t s, const Workspace &ws, const RouteSpec &rs, const float *x, KernelEvents ev,
                        bool requant_x) {
  const uint32_t w = route_waves(rs.tokens);
  static_assert(kMaxTokens == 8, "the requant column runs 256 or 512 threads");
  const uint32_t groups = (rs.r.n_experts + w - 1) / w, blocks = groups * rs.tokens;
  // the workspace holds counters for at most kRouteCounters / kRouteCounterStride - 1 groups
  if ((blocks + kRouteGroup - 1) / kRouteGroup > kRouteCounters / kRouteCounterStride - 1) return hipErrorInvalidValue;
  if (requant_x)
    hipExtLaunchKernelGGL(k_route<false, true>, dim3(groups + 1, rs.tokens), dim3(64 * w), 0, s, ev.start, ev.stop,
                          0, rs, ws, x);
  else
    hipExtLaunchKernelGGL(k_route<false>, dim3(groups, rs.tokens), dim3(64 * w), 0, s, ev.start, ev.stop, 0, rs, ws,
                          x);
  return hipGetLastError();
}

hipError_t launch_route_scores(hipStream_t s, const Workspace &ws, const RouteSpec &rs, const float *x,
                               KernelEvents ev, bool official) {
  const uint32_t w = route_waves(rs.tokens);
  const uint32_t groups = (rs.r.n_experts + w - 1) / w;
  if (official) {
    if (rs.tokens != 1 || w != kSingleRouteWaves) return hipErrorInvalidValue;
    hipExtLaunchKernelGGL(k_route<true, true>, dim3(groups + 1, rs.tokens), dim3(64 * w), 0, s, ev.start, ev.stop,
                          0, rs, ws, x);
  } else {
    hipExtLaunchKernelGGL(k_route<true>, dim3(groups, rs.tokens), dim3(64 * w), 0, s, ev.start, ev.stop, 0, rs, ws,
                          x);
  }
  return hipGetLastError();
}

namespace {
template <int kSrc, int kTier>
void phase1_launch(hipStream_t s, const Workspace &ws, const PairTable &plan, const RouteSpec &rs, uint32_t n_pairs,
                   const PageOffsets &mx, const PageOffsets &fp8, const float *x, int mode, KernelEvents ev) {
  if (mode == S14_MODE_FAST) {
    const dim3 grid(kInter / p1_fast_rows(kTier), n_pairs);
    hipExtLaunchKernelGGL(k_phase1_fast<kSrc, kTier>, grid, dim3(256), 0, s, ev.start, ev.stop, 0, plan, rs, ws, x,
                          mx, fp8);
  } else if constexpr (kTier == 1) {  // blocks in these modes run the block engine
    const dim3 grid(kInter / (kP1ExactRows * kP1ExactWaves), n_pairs);
    const dim3 blk(64 * kP1ExactWaves);
    if (mode == S14_MODE_OFFICIAL) {
      // the phase-1 stage includes the h requant that follows it
      hipExtLaunchKernelGGL(k_phase1_exact<kSrc, kTier, true>, grid, blk, 0, s, ev.start, nullptr, 0, plan, rs, ws, x,
                            mx, fp8);
      hipExtLaunchKernelGGL(k_requant_h_official, dim3((n_pairs * kHGroups128 * 8u + 255u) / 256u), dim3(256), 0, s,
                            nullptr, ev.stop, 0, ws, n_pairs);
    } else
      hipExtLaunchKernelGGL(k_phase1_exact<kSrc, kTier, false>, grid, blk, 0, s, ev.start, ev.stop, 0, plan, rs, ws,
                            x, mx, fp8);
  }
}

template <int kTier>
void phase1_tier(hipStream_t s, const Workspace &ws, const PairTable *host_plan, const RouteSpec *route,
                 uint32_t n_pairs, const PageOffsets &mx, const PageOffsets &fp8, const float *x, int mode,
                 KernelEvents ev) {
  PairTable plan{};
  if (host_plan) plan = *host_plan;
  RouteSpec rs{};
  if (route) rs = *route;
  if (host_plan) {
    phase1_launch<kPairFromHost, kTier>(s, ws, plan, rs, n_pairs, mx, fp8, x, mode, ev);
  } else if (route) {
    if constexpr (kTier == 1) phase1_launch<kPairFromScores, kTier>(s, ws, plan, rs, n_pairs, mx, fp8, x, mode, ev);
  } else {
    phase1_launch<kPairFromTable, kTier>(s, ws, plan, rs, n_pairs, mx, fp8, x, mode, ev);
  }
}

template <int kTier>
void phase2_tier(hipStream_t s, const Workspace &ws, uint32_t tokens, const PageOffsets &mx, const PageOffsets &fp8,
                 float *y, int mode, KernelEvents ev) {
  const PairTable *tab = ws.table;
  const float *h = ws.h;
  if (mode == S14_MODE_FAST) {
    hipExtLaunchKernelGGL(k_phase2_fast<kTier>, dim3(kHidden / kP2FastRows, tokens), dim3(64 * kP2FastWaves), 0, s,
                          ev.start, ev.stop, 0, tab, h, y, mx, fp8);
  } else if constexpr (kTier == 1) {  // blocks in these modes run the block engine
    if (mode == S14_MODE_OFFICIAL)
      hipExtLaunchKernelGGL(k_phase2_exact<kTier, true>, dim3(kHidden / kP2ExactRows, tokens),
                            dim3(64 * kP2ExactWaves), 0, s, ev.start, ev.stop, 0, tab, h, ws.hwin, y, mx, fp8);
    else
      hipExtLaunchKernelGGL(k_phase2_exact<kTier, false>, dim3(kHidden / kP2ExactRows, tokens),
                            dim3(64 * kP2ExactWaves), 0, s, ev.start, ev.stop, 0, tab, h, ws.hwin, y, mx, fp8);
  }
}
}  // namespace

hipError_t launch_chain_quad(hipStream_t s, const Workspace &ws, const uint8_t *page, const PageOffsets &mx,
                             const float *x, float weight, float *y, KernelEvents ev1, KernelEvents ev2) {
  hipExtLaunchKernelGGL(k_chain_phase1_quad, dim3(kInter / kChainP1Rows), dim3(256), 0, s, ev1.start, ev1.stop, 0,
                        page, x, ws, mx);
  hipExtLaunchKernelGGL(k_chain_phase2_quad, dim3(kHidden / kChainP2Rows), dim3(256), 0, s, ev2.start, ev2.stop, 0,
                        page, ws, weight, y, mx);
  return hipGetLastError();
}

hipError_t launch_phase1(hipStream_t s, const Workspace &ws, const PairTable *host_plan, uint32_t n_pairs,
                         uint32_t tokens, const PageOffsets &mx, const PageOffsets &fp8, const float *x, int mode,
                         KernelEvents ev, const RouteSpec *route) {
  if (route && (host_plan || tokens != 1)) return hipErrorInvalidValue;  // in-kernel planning: one routed token
  if (tokens > 1 && mode != S14_MODE_FAST) return hipErrorInvalidValue;  // the block engine's
  if (tokens <= 1)
    phase1_tier<1>(s, ws, host_plan, route, n_pairs, mx, fp8, x, mode, ev);
  else
    phase1_tier<kMaxTokens>(s, ws, host_plan, route, n_pairs, mx, fp8, x, mode, ev);
  return hipGetLastError();
}

hipError_t launch_phase2(hipStream_t s, const Workspace &ws, uint32_t tokens, const PageOffsets &mx,
                         const PageOffsets &fp8, float *y, int mode, KernelEvents ev) {
  if (tokens > 1 && mode != S14_MODE_FAST) return hipErrorInvalidValue;  // the block engine's
  if (tokens <= 1)
    phase2_tier<1>(s, ws, tokens, mx, fp8, y, mode, ev);
  else
    phase2_tier<kMaxTokens>(s, ws, tokens, mx, fp8, y, mode, ev);
  return hipGetLastError();
}

}  // namespace s14
