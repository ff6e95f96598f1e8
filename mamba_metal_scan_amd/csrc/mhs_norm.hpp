// Fused RMSNorm of the TinyMamba residual stream for gfx950. The reference
// normalises each row of C features as
//   y = x * rsqrt(mean(x^2) + eps) * weight        (mamba_metal/model.py:85-95)
// before every block's in_proj and before the head. With r = rsqrt(mean(x^2)
// + eps) per row and g = dy * weight:
//   dx = r * g - x * r^3 * (sum_j g_j x_j) / C  (+ the residual stream's
//        gradient, added in the same pass),
//   dweight = sum over rows of dy * x * r.
// The framework's fused rms_norm takes one kernel forward and three backward
// (input gradient, then the weight gradient in two passes), and the
// residual stream's two gradients are added by a kernel of their own. Here
// the backward reads dy, x and the residual gradient once and writes dx once,
// with the weight gradient's per-block partials summed by a small second
// kernel in a fixed order.
//
// HBM-bound. One wave per row at a time: each lane holds NV float4 of the
// row (C <= 256 NV, C a multiple of 4, rows 16-byte aligned), the row's sum
// by xor shuffles (every lane ends with the same bits: each stage adds the
// same two values in either lane).
#pragma once

#include "mhs_common.hpp"

namespace mhs {

constexpr int kNormThreads = 256;          // 4 waves; one row per wave at a time
constexpr int kNormMaxNV = 8;              // rows of at most 2048 features
constexpr int kNormReduceCols = 4;         // float4 columns per reduction block
constexpr int kNormBwdBlocks = 512;        // backward blocks (weight-gradient partials)

__device__ __forceinline__ float wave_sum64(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ float4 f4_zero() { return make_float4(0.f, 0.f, 0.f, 0.f); }

// y (rows, C) = x * r * w; rstd (rows) = r. ADD: the row is x + delta (the
// residual stream's update by the previous block), written to x_out, and
// normalised.
template <int NV, bool ADD = false>
__global__ void __launch_bounds__(kNormThreads)
rmsnorm_fwd_kernel(const float* __restrict__ x, const float* __restrict__ delta,
                   const float* __restrict__ w, float* __restrict__ y, float* __restrict__ x_out,
                   float* __restrict__ rstd, int rows, int C, float eps) {
  const int lane = threadIdx.x & 63;
  const int nw = gridDim.x * (kNormThreads / 64);
  const int C4 = C >> 2;
  float4 wv[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int i = lane + 64 * v;
    wv[v] = i < C4 ? reinterpret_cast<const float4*>(w)[i] : f4_zero();
  }
  const float inv_c = 1.f / (float)C;
  for (int r = blockIdx.x * (kNormThreads / 64) + (threadIdx.x >> 6); r < rows; r += nw) {
    const size_t o = (size_t)r * C;
    const float4* xr = reinterpret_cast<const float4*>(x + o);
    float4 xv[NV];
    float ss = 0.f;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int i = lane + 64 * v;
      xv[v] = i < C4 ? xr[i] : f4_zero();
      if constexpr (ADD) {
        if (i < C4) {
          const float4 dv = reinterpret_cast<const float4*>(delta + o)[i];
          xv[v] = make_float4(xv[v].x + dv.x, xv[v].y + dv.y, xv[v].z + dv.z, xv[v].w + dv.w);
          reinterpret_cast<float4*>(x_out + o)[i] = xv[v];
        }
      }
      ss = __builtin_fmaf(xv[v].x, xv[v].x, ss);
      ss = __builtin_fmaf(xv[v].y, xv[v].y, ss);
      ss = __builtin_fmaf(xv[v].z, xv[v].z, ss);
      ss = __builtin_fmaf(xv[v].w, xv[v].w, ss);
    }
    const float rs = 1.f / __fsqrt_rn(__builtin_fmaf(wave_sum64(ss), inv_c, eps));
    float4* yr = reinterpret_cast<float4*>(y + o);
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int i = lane + 64 * v;
      if (i < C4)
        yr[i] = make_float4(xv[v].x * rs * wv[v].x, xv[v].y * rs * wv[v].y,
                            xv[v].z * rs * wv[v].z, xv[v].w * rs * wv[v].w);
    }
    if (lane == 0) rstd[r] = rs;
  }
}

// dx (rows, C) from dy, x, w, rstd and, if not null, the residual stream's
// gradient dres (added); dwp (gridDim.x, C): the block's partial sums of
// dy * x * r over its rows (its waves' sums added in wave order).
template <int NV>
__global__ void __launch_bounds__(kNormThreads)
rmsnorm_bwd_kernel(const float* __restrict__ dy, const float* __restrict__ x,
                   const float* __restrict__ w, const float* __restrict__ rstd,
                   const float* __restrict__ dres, float* __restrict__ dx,
                   float* __restrict__ dwp, int rows, int C) {
  __shared__ float4 red[kNormThreads / 64 - 1][64 * NV];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nw = gridDim.x * (kNormThreads / 64);
  const int C4 = C >> 2;
  const float inv_c = 1.f / (float)C;
  float4 wv[NV], acc[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int i = lane + 64 * v;
    wv[v] = i < C4 ? reinterpret_cast<const float4*>(w)[i] : f4_zero();
    acc[v] = f4_zero();
  }
  for (int r = blockIdx.x * (kNormThreads / 64) + wave; r < rows; r += nw) {
    const size_t o = (size_t)r * C;
    const float4* dyr = reinterpret_cast<const float4*>(dy + o);
    const float4* xr = reinterpret_cast<const float4*>(x + o);
    const float4* dresr = dres != nullptr ? reinterpret_cast<const float4*>(dres + o) : nullptr;
    float4 dyv[NV], xv[NV], dv[NV];
    float dot = 0.f;   // sum_j (dy_j w_j) x_j over the lane's features
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int i = lane + 64 * v;
      const bool in = i < C4;
      dyv[v] = in ? dyr[i] : f4_zero();
      xv[v] = in ? xr[i] : f4_zero();
      dv[v] = in && dres != nullptr ? dresr[i] : f4_zero();
      dot = __builtin_fmaf(dyv[v].x * wv[v].x, xv[v].x, dot);
      dot = __builtin_fmaf(dyv[v].y * wv[v].y, xv[v].y, dot);
      dot = __builtin_fmaf(dyv[v].z * wv[v].z, xv[v].z, dot);
      dot = __builtin_fmaf(dyv[v].w * wv[v].w, xv[v].w, dot);
    }
    const float rs = rstd[r];
    const float k = rs * rs * rs * wave_sum64(dot) * inv_c;
    float4* dxr = reinterpret_cast<float4*>(dx + o);
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int i = lane + 64 * v;
      if (i >= C4) continue;
      // dx = (dy w) r - x k (+ dres); dweight += dy (x r)
      dxr[i] = make_float4(
          __builtin_fmaf(dyv[v].x * wv[v].x, rs, __builtin_fmaf(-xv[v].x, k, dv[v].x)),
          __builtin_fmaf(dyv[v].y * wv[v].y, rs, __builtin_fmaf(-xv[v].y, k, dv[v].y)),
          __builtin_fmaf(dyv[v].z * wv[v].z, rs, __builtin_fmaf(-xv[v].z, k, dv[v].z)),
          __builtin_fmaf(dyv[v].w * wv[v].w, rs, __builtin_fmaf(-xv[v].w, k, dv[v].w)));
      acc[v].x = __builtin_fmaf(dyv[v].x, xv[v].x * rs, acc[v].x);
      acc[v].y = __builtin_fmaf(dyv[v].y, xv[v].y * rs, acc[v].y);
      acc[v].z = __builtin_fmaf(dyv[v].z, xv[v].z * rs, acc[v].z);
      acc[v].w = __builtin_fmaf(dyv[v].w, xv[v].w * rs, acc[v].w);
    }
  }
  if (wave > 0) {
#pragma unroll
    for (int v = 0; v < NV; ++v) red[wave - 1][lane + 64 * v] = acc[v];
  }
  __syncthreads();
  if (wave != 0) return;
  float4* out = reinterpret_cast<float4*>(dwp + (size_t)blockIdx.x * C);
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int i = lane + 64 * v;
    if (i >= C4) continue;
    float4 s = acc[v];
#pragma unroll
    for (int q = 0; q < kNormThreads / 64 - 1; ++q) {
      const float4 t = red[q][i];
      s.x += t.x; s.y += t.y; s.z += t.z; s.w += t.w;
    }
    out[i] = s;
  }
}

// dw (C) = the sum of the P partial rows of dwp (P, C), in a fixed order:
// a block owns kNormReduceCols float4 columns; its G = 256 / kNormReduceCols
// thread groups each add every G-th partial row (g, g + G, ...), then the
// groups' sums are added pairwise in LDS (a fixed tree of log2 G steps).
__global__ void __launch_bounds__(256)
rmsnorm_dw_reduce_kernel(const float* __restrict__ dwp, float* __restrict__ dw, int P, int C) {
  constexpr int G = 256 / kNormReduceCols;
  __shared__ float4 red[G][kNormReduceCols];
  const int cq = threadIdx.x % kNormReduceCols, g = threadIdx.x / kNormReduceCols;
  const int C4 = C >> 2;
  const int i = blockIdx.x * kNormReduceCols + cq;
  float4 s = f4_zero();
  if (i < C4) {
    const float4* p = reinterpret_cast<const float4*>(dwp) + i;
    int k = g;
    for (; k + 3 * G < P; k += 4 * G) {
      const float4 a = p[(size_t)k * C4], b = p[(size_t)(k + G) * C4],
                   c = p[(size_t)(k + 2 * G) * C4], d = p[(size_t)(k + 3 * G) * C4];
      s.x += a.x; s.y += a.y; s.z += a.z; s.w += a.w;
      s.x += b.x; s.y += b.y; s.z += b.z; s.w += b.w;
      s.x += c.x; s.y += c.y; s.z += c.z; s.w += c.w;
      s.x += d.x; s.y += d.y; s.z += d.z; s.w += d.w;
    }
    for (; k < P; k += G) {
      const float4 a = p[(size_t)k * C4];
      s.x += a.x; s.y += a.y; s.z += a.z; s.w += a.w;
    }
  }
  red[g][cq] = s;
  __syncthreads();
  // The groups' sums added pairwise, a fixed tree: g += g + h for h = G/2 .. 1.
#pragma unroll
  for (int h = G / 2; h >= 1; h >>= 1) {
    if (g < h) {
      const float4 t = red[g + h][cq];
      float4& u = red[g][cq];
      u.x += t.x; u.y += t.y; u.z += t.z; u.w += t.w;
    }
    __syncthreads();
  }
  if (g == 0 && i < C4) reinterpret_cast<float4*>(dw)[i] = red[0][cq];
}

}  // namespace mhs
