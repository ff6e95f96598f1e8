// The block's output gate for gfx950 (mamba_metal/model.py:255-256):
//   out[b,t,d] = (y[b,t,d] + Dskip[d]) * silu(z[b,t,d])
// and its backward, with s = sigmoid(z):
//   dy = dout * z * s
//   dz = dout * (y + Dskip) * s * (1 + z * (1 - s))
//   dDskip[d] = sum_{b,t} dy[b,t,d]
// Layouts: y, out, dout, dy, dz (B,T,D) contiguous; z (B,T,D) with rows
// z_rs >= D floats apart (the block passes the z half of its in_proj output
// without a copy).
//
// HBM-bound elementwise work: a thread owns one channel (consecutive threads,
// consecutive channels: coalesced rows) and TPT consecutive steps, in blocks
// of 64 channels x 4 step groups like the conv kernels. The backward adds its
// dy over the block's steps in a fixed order and leaves one partial per
// (block row of steps, b, d); conv_reduce_kernel (K = 0) sums them.
#pragma once

#include "mhs_common.hpp"
#include "mhs_conv.hpp"

namespace mhs {

template <int TPT>
__global__ void __launch_bounds__(kConvCh * kConvTG)
out_gate_fwd_kernel(const float* __restrict__ y, const float* __restrict__ dskip,
                    const float* __restrict__ z, long long z_rs, float* __restrict__ out, int T,
                    int D) {
  const int d = blockIdx.x * kConvCh + (threadIdx.x % kConvCh);
  const int g = threadIdx.x / kConvCh;
  const int b = blockIdx.z;
  const int t0 = (blockIdx.y * kConvTG + g) * TPT;
  if (d >= D || t0 >= T) return;
  const float ds = dskip[d];
  const float* yb = y + (size_t)b * T * D + d;
  const float* zb = z + (size_t)b * T * z_rs + d;
  float* ob = out + (size_t)b * T * D + d;
  const int n = min(TPT, T - t0);
  float yv[TPT], zv[TPT];
#pragma unroll
  for (int i = 0; i < TPT; ++i) {
    const int t = t0 + (i < n ? i : 0);
    yv[i] = yb[(size_t)t * D];
    zv[i] = zb[(size_t)t * z_rs];
  }
#pragma unroll
  for (int i = 0; i < TPT; ++i)
    if (i < n) ob[(size_t)(t0 + i) * D] = (yv[i] + ds) * (zv[i] * sigmoid_f(zv[i]));
}

template <int TPT>
__global__ void __launch_bounds__(kConvCh * kConvTG)
out_gate_bwd_kernel(const float* __restrict__ y, const float* __restrict__ dskip,
                    const float* __restrict__ z, long long z_rs, const float* __restrict__ dout,
                    float* __restrict__ dy, float* __restrict__ dz, long long dz_rs,
                    float* __restrict__ wsp, int T, int D) {
  __shared__ float part[kConvTG][kConvCh];
  const int c = threadIdx.x % kConvCh;
  const int d = blockIdx.x * kConvCh + c;
  const int g = threadIdx.x / kConvCh;
  const int b = blockIdx.z;
  const int t0 = (blockIdx.y * kConvTG + g) * TPT;
  float acc = 0.f;
  if (d < D && t0 < T) {
    const float ds = dskip[d];
    const size_t row = (size_t)b * T * D + d;
    const float* zb = z + (size_t)b * T * z_rs + d;
    float* dzb = dz + (size_t)b * T * dz_rs + d;   // rows dz_rs apart (>= D)
    const int n = min(TPT, T - t0);
    float yv[TPT], zv[TPT], gv[TPT];
#pragma unroll
    for (int i = 0; i < TPT; ++i) {
      const int t = t0 + (i < n ? i : 0);
      yv[i] = y[row + (size_t)t * D];
      zv[i] = zb[(size_t)t * z_rs];
      gv[i] = dout[row + (size_t)t * D];
    }
#pragma unroll
    for (int i = 0; i < TPT; ++i) {
      if (i >= n) break;
      const float s = sigmoid_f(zv[i]);
      const float dyv = gv[i] * (zv[i] * s);
      const size_t o = row + (size_t)(t0 + i) * D;
      dy[o] = dyv;
      dzb[(size_t)(t0 + i) * dz_rs] = gv[i] * (yv[i] + ds) * s * __builtin_fmaf(zv[i], 1.f - s, 1.f);
      acc += dyv;
    }
  }
  part[g][c] = acc;
  __syncthreads();
  if (g == 0 && d < D) {
    float s = part[0][c];
#pragma unroll
    for (int gg = 1; gg < kConvTG; ++gg) s += part[gg][c];
    wsp[((size_t)blockIdx.y * gridDim.z + b) * D + d] = s;
  }
}

}  // namespace mhs
