// Causal depthwise conv1d + SiLU for gfx950 (the MambaBlock's conv, in the
// reference nn.Conv1d(d_inner, d_inner, kernel_size=K, padding=K-1,
// groups=d_inner) cut to the first T outputs, then F.silu:
// mamba_metal/model.py:174-175 and :244):
//   pre[b,t,d] = bias[d] + sum_{k<K} w[d,k] * x[b, t-K+1+k, d]   (x = 0 before t = 0)
//   out[b,t,d] = silu(pre) = pre * sigmoid(pre)
// Layouts: x (B,T,D) rows of stride x_rs >= D floats (the block passes the x
// half of its in_proj output without a copy), out / dout / dx (B,T,D)
// contiguous, w (D,K), bias (D).
//
// Both kernels are HBM-bound stencils over (b, t, d): a thread owns one
// channel d (consecutive threads, consecutive channels: coalesced rows) and
// a run of TPT consecutive steps, keeping the K-1 step halo in registers.
#pragma once

#include "mhs_common.hpp"

namespace mhs {

constexpr int kConvMaxK = 8;
constexpr int kConvCh = 64;    // channels per block
constexpr int kConvTG = 4;     // step groups per block (block = 64 x 4 threads)

// Forward: thread (d, step group g) of block (db, tb, b) computes TPT
// outputs t in [t0, t0 + TPT).
template <int K, int TPT>
__global__ void __launch_bounds__(kConvCh * kConvTG)
conv_silu_fwd_kernel(const float* __restrict__ x, long long x_rs, const float* __restrict__ w,
                     const float* __restrict__ bias, float* __restrict__ out, int T, int D) {
  const int d = blockIdx.x * kConvCh + (threadIdx.x % kConvCh);
  const int g = threadIdx.x / kConvCh;
  const int b = blockIdx.z;
  const int t0 = (blockIdx.y * kConvTG + g) * TPT;
  if (d >= D || t0 >= T) return;
  float wk[K];
#pragma unroll
  for (int k = 0; k < K; ++k) wk[k] = w[(size_t)d * K + k];
  const float bi = bias[d];
  const float* xb = x + (size_t)b * T * x_rs + d;
  float* ob = out + (size_t)b * T * D + d;
  // window[j] = x[t0 - K + 1 + j], j in [0, TPT + K - 1)
  float win[TPT + K - 1];
#pragma unroll
  for (int j = 0; j < TPT + K - 1; ++j) {
    const int t = t0 - K + 1 + j;
    win[j] = (t >= 0 && t < T) ? xb[(size_t)t * x_rs] : 0.f;
  }
#pragma unroll
  for (int i = 0; i < TPT; ++i) {
    if (t0 + i >= T) break;
    float pre = bi;
#pragma unroll
    for (int k = 0; k < K; ++k) pre = __builtin_fmaf(wk[k], win[i + k], pre);
    ob[(size_t)(t0 + i) * D] = pre * sigmoid_f(pre);
  }
}

// Backward. With s = dout * silu'(pre), silu'(p) = sig(p) * (1 + p * (1 - sig(p))):
//   dx[t]    = sum_k w[k] * s[t + K - 1 - k]          (s = 0 past T - 1)
//   dw[k]    = sum_{b,t} s[t] * x[t - K + 1 + k]
//   dbias    = sum_{b,t} s[t]
// Thread (d, g) produces dx for its TPT steps and partial dw, dbias over
// them; the block adds its kConvTG step groups in a fixed order and writes one
// partial per (block row of steps, b, d) to the workspace.
template <int K, int TPT>
__global__ void __launch_bounds__(kConvCh * kConvTG)
conv_silu_bwd_kernel(const float* __restrict__ x, long long x_rs, const float* __restrict__ w,
                     const float* __restrict__ bias, const float* __restrict__ dout,
                     float* __restrict__ dx, long long dx_rs, float* __restrict__ wsp, int T,
                     int D) {
  __shared__ float part[kConvTG][K + 1][kConvCh];
  const int c = threadIdx.x % kConvCh;
  const int d = blockIdx.x * kConvCh + c;
  const int g = threadIdx.x / kConvCh;
  const int b = blockIdx.z;
  const int t0 = (blockIdx.y * kConvTG + g) * TPT;
  const bool act = d < D && t0 < T;
  float pw[K + 1];
#pragma unroll
  for (int k = 0; k <= K; ++k) pw[k] = 0.f;
  if (act) {
    float wk[K];
#pragma unroll
    for (int k = 0; k < K; ++k) wk[k] = w[(size_t)d * K + k];
    const float bi = bias[d];
    const float* xb = x + (size_t)b * T * x_rs + d;
    const float* gb = dout + (size_t)b * T * D + d;
    float* dxb = dx + (size_t)b * T * dx_rs + d;   // rows dx_rs apart (>= D)
    // x[t0 - K + 1 .. t0 + TPT + K - 2]: inputs of pre over [t0, t0 + TPT + K - 1)
    constexpr int NX = TPT + 2 * (K - 1);
    float xw[NX];
#pragma unroll
    for (int j = 0; j < NX; ++j) {
      const int t = t0 - K + 1 + j;
      xw[j] = (t >= 0 && t < T) ? xb[(size_t)t * x_rs] : 0.f;
    }
    // s over [t0, t0 + TPT + K - 1)
    constexpr int NS = TPT + K - 1;
    float sw[NS];
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      const int t = t0 + j;
      float pre = bi;
#pragma unroll
      for (int k = 0; k < K; ++k) pre = __builtin_fmaf(wk[k], xw[j + k], pre);
      const float sg = sigmoid_f(pre);
      const float gv = t < T ? gb[(size_t)t * D] : 0.f;
      sw[j] = gv * sg * __builtin_fmaf(pre, 1.f - sg, 1.f);
    }
#pragma unroll
    for (int i = 0; i < TPT; ++i) {
      if (t0 + i >= T) break;
      float acc = 0.f;
#pragma unroll
      for (int k = 0; k < K; ++k) acc = __builtin_fmaf(wk[k], sw[i + K - 1 - k], acc);
      dxb[(size_t)(t0 + i) * dx_rs] = acc;
      // dw[k] += s[t] * x[t - K + 1 + k]; dbias += s[t]  (t = t0 + i < T)
#pragma unroll
      for (int k = 0; k < K; ++k) pw[k] = __builtin_fmaf(sw[i], xw[i + k], pw[k]);
      pw[K] += sw[i];
    }
  }
#pragma unroll
  for (int k = 0; k <= K; ++k) part[g][k][c] = pw[k];
  __syncthreads();
  if (g == 0 && d < D) {
    // Fixed order over the step groups; partial slot (blockIdx.y, b).
    float* dst = wsp + ((size_t)blockIdx.y * gridDim.z + b) * (size_t)(K + 1) * D;
#pragma unroll
    for (int k = 0; k <= K; ++k) {
      float s = part[0][k][c];
#pragma unroll
      for (int gg = 1; gg < kConvTG; ++gg) s += part[gg][k][c];
      dst[(size_t)k * D + d] = s;
    }
  }
}

// dw[d,k], dbias[d]: sums of the nparts partials. One wave per output: lane
// l adds partials l, l+64, ... in order, then a fixed DPP / permlane tree sums
// the 64 lanes (a fixed summation order: bit-for-bit reproducible).
__global__ void __launch_bounds__(256)
conv_reduce_kernel(const float* __restrict__ wsp, float* __restrict__ dw, float* __restrict__ dbias,
                   int nparts, int K, int D) {
  const int i = blockIdx.x * 4 + (threadIdx.x >> 6);   // (k, d), d fastest
  const int lane = threadIdx.x & 63;
  if (i >= (K + 1) * D) return;                        // uniform per wave
  const size_t stride = (size_t)(K + 1) * D;
  float s = 0.f;
  for (int p = lane; p < nparts; p += 64) s += wsp[(size_t)p * stride + i];
  s = group_sum<16>(s);                                // row totals
  const auto h32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(s), __float_as_uint(s), false,
                                                    false);
  s = __uint_as_float(h32[0]) + __uint_as_float(h32[1]);
  const auto h16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(s), __float_as_uint(s), false,
                                                    false);
  s = __uint_as_float(h16[0]) + __uint_as_float(h16[1]);
  if (lane == 0) {
    const int k = i / D, d = i % D;
    if (k < K) dw[(size_t)d * K + k] = s;
    else dbias[d] = s;
  }
}

}  // namespace mhs
