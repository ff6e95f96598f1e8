// One recurrent decode step (the reference does this in pure torch,
// mamba_metal/model.py:234-241):
//   h[b,d,:] <- h[b,d,:] * exp(-dt[b,d] * Aneg[d,:]) + dt[b,d] * x[b,d] * B[b,:]
//   y[b,d]    = sum_n C[b,n] * h[b,d,n]
// Memory-bound (h is read and written once). Four lanes share a channel, each
// holding a float4 of its state, so one wave touches 16 channels x 64 B = 1 KiB
// of contiguous h per access; the y sum is a two-level DPP add inside the quad.
#pragma once

#include "mhs_common.hpp"

namespace mhs {

// N % 4 == 0 and N <= 16: lane q of a quad owns n in [4q, 4q+4) of one channel
// (lanes beyond N/4 in the quad idle). One thread per (b, d, quad-lane).
__global__ void __launch_bounds__(256)
step_kernel_vec(float* __restrict__ h, const float* __restrict__ x,
                const float* __restrict__ dt, const float* __restrict__ aneg,
                const float* __restrict__ Bm, const float* __restrict__ Cm,
                float* __restrict__ y, int batch, int D, int N) {
  const long long gid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long ch = gid >> 2;           // (b, d)
  const int q = (int)(gid & 3);
  const bool valid = ch < (long long)batch * D;
  const bool own = valid && 4 * q < N;
  float part = 0.f;
  if (own) {
    const int b = (int)(ch / D);
    const int d = (int)(ch % D);
    const float dtv = dt[ch];
    const float bx = dtv * x[ch];
    const int n = 4 * q;
    float4 hv = *reinterpret_cast<const float4*>(h + ch * N + n);
    const float4 av = *reinterpret_cast<const float4*>(aneg + (size_t)d * N + n);
    const float4 bv = *reinterpret_cast<const float4*>(Bm + (size_t)b * N + n);
    const float4 cv = *reinterpret_cast<const float4*>(Cm + (size_t)b * N + n);
    hv.x = __builtin_fmaf(exp2_hw(-dtv * av.x * kLog2e), hv.x, bv.x * bx);
    hv.y = __builtin_fmaf(exp2_hw(-dtv * av.y * kLog2e), hv.y, bv.y * bx);
    hv.z = __builtin_fmaf(exp2_hw(-dtv * av.z * kLog2e), hv.z, bv.z * bx);
    hv.w = __builtin_fmaf(exp2_hw(-dtv * av.w * kLog2e), hv.w, bv.w * bx);
    *reinterpret_cast<float4*>(h + ch * N + n) = hv;
    part = cv.x * hv.x + cv.y * hv.y + cv.z * hv.z + cv.w * hv.w;
  }
  part = group_sum<4>(part);
  if (valid && q == 0) y[ch] = part;
}

// Any N: one thread per (b, d).
__global__ void __launch_bounds__(256)
step_kernel_any(float* __restrict__ h, const float* __restrict__ x,
                const float* __restrict__ dt, const float* __restrict__ aneg,
                const float* __restrict__ Bm, const float* __restrict__ Cm,
                float* __restrict__ y, int batch, int D, int N) {
  const long long ch = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (ch >= (long long)batch * D) return;
  const int b = (int)(ch / D);
  const int d = (int)(ch % D);
  const float dtv = dt[ch];
  const float bx = dtv * x[ch];
  float s = 0.f;
  for (int n = 0; n < N; ++n) {
    const float hv = __builtin_fmaf(exp2_hw(-dtv * aneg[(size_t)d * N + n] * kLog2e),
                                    h[ch * N + n], Bm[(size_t)b * N + n] * bx);
    h[ch * N + n] = hv;
    s = __builtin_fmaf(Cm[(size_t)b * N + n], hv, s);
  }
  y[ch] = s;
}

}  // namespace mhs
