// Fused cross-entropy of the TinyMamba head for gfx950. The reference
// computes F.cross_entropy(logits.reshape(-1, V), targets.reshape(-1))
// (mamba_metal/model.py:296-297): the framework's log_softmax over the
// vocabulary, which writes the (rows, V) log-probabilities and keeps them for
// the backward, then nll_loss, mean over the rows whose target is not
// ignore_index. Per row r of logits x:
//   lse_r  = log sum_j exp(x_rj),   loss_r = lse_r - x_r,t_r   (t_r the target)
//   dx_rj  = scale * (exp(x_rj - lse_r) - [j == t_r]),  scale = dloss / n_valid
// and 0 for ignored rows. Here the forward reads the logits once and keeps
// only lse_r (4 bytes per row); the backward reads them once more and writes
// the gradient: 3 passes over the (rows, V) tensor instead of the
// framework's six.
//
// HBM-bound: one 256-thread block per row, 16-byte loads, a running maximum
// and rescaled sum per thread (in base 2: y = x log2 e, so that each term is
// one v_exp_f32), combined over the block in a fixed order.
#pragma once

#include "mhs_common.hpp"

namespace mhs {

constexpr int kXentThreads = 256;
constexpr float kLn2 = 0.6931471805599453f;

// (m, s) represents s * 2^m; combine two such partial sums. The side that
// holds the maximum is scaled by exactly 1 (m - mm is not formed for it):
// with both maxima -inf (a row, or a thread's share of it, masked with -inf
// logits) 2^(-inf - -inf) would be NaN, where the sum is 0 * 2^-inf. An
// empty side (s = 0) adds 0. A NaN partial sum (from a NaN logit) is not 0
// and propagates.
__device__ __forceinline__ void lse2_combine(float& m, float& s, float m2, float s2) {
  const float mm = fmaxf(m, m2);
  const float a = s != 0.f ? (m == mm ? s : s * exp2_hw(m - mm)) : 0.f;
  const float b = s2 != 0.f ? (m2 == mm ? s2 : s2 * exp2_hw(m2 - mm)) : 0.f;
  m = mm;
  s = a + b;
}

// The shift of a group's terms 2^(y - mc): its maximum mc, or 0 when every
// term is -inf (the group's sum is then 2^-inf = 0, not 2^(-inf - -inf)).
__device__ __forceinline__ float lse2_shift(float mc) { return mc == -INFINITY ? 0.f : mc; }

// The block's (m, s) combined over its threads in a fixed order: within each
// wave by xor shuffles, then the waves' results in order through LDS. Every
// thread returns the total.
__device__ __forceinline__ void block_lse2(float& m, float& s) {
  __shared__ float red[2][kXentThreads / 64];
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float m2 = __shfl_xor(m, off, 64), s2 = __shfl_xor(s, off, 64);
    lse2_combine(m, s, m2, s2);
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    red[0][wave] = m;
    red[1][wave] = s;
  }
  __syncthreads();
  m = red[0][0];
  s = red[1][0];
#pragma unroll
  for (int w = 1; w < kXentThreads / 64; ++w) lse2_combine(m, s, red[0][w], red[1][w]);
}

// VEC: 4 (vocab a multiple of 4, rows 16-byte aligned: float4 loads) or 1.
// A target outside [0, vocab) that is not ignore_index gives loss NaN (the
// framework raises a device-side assertion there).
template <int VEC>
__global__ void __launch_bounds__(kXentThreads)
xent_fwd_kernel(const float* __restrict__ logits, const long long* __restrict__ targets,
                float* __restrict__ lse, float* __restrict__ loss_rows, long long vocab,
                long long ignore_index) {
  const long long r = blockIdx.x;
  const float* x = logits + r * vocab;
  float m = -INFINITY, s = 0.f;
  if constexpr (VEC == 4) {
    const float4* x4 = reinterpret_cast<const float4*>(x);
    const long long n4 = vocab / 4;
    constexpr int U = 4;   // float4 loads per update of the running maximum
    long long i = threadIdx.x;
    for (; i + (U - 1) * kXentThreads < n4; i += U * kXentThreads) {
      float y[4 * U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const float4 v = x4[i + u * kXentThreads];
        y[4 * u] = v.x * kLog2e;
        y[4 * u + 1] = v.y * kLog2e;
        y[4 * u + 2] = v.z * kLog2e;
        y[4 * u + 3] = v.w * kLog2e;
      }
      float mc = y[0];
#pragma unroll
      for (int k = 1; k < 4 * U; ++k) mc = fmaxf(mc, y[k]);
      const float sh = lse2_shift(mc);
      float sc = 0.f;
#pragma unroll
      for (int k = 0; k < 4 * U; ++k) sc += exp2_hw(y[k] - sh);
      lse2_combine(m, s, mc, sc);
    }
    for (; i < n4; i += kXentThreads) {
      const float4 v = x4[i];
      const float y0 = v.x * kLog2e, y1 = v.y * kLog2e, y2 = v.z * kLog2e, y3 = v.w * kLog2e;
      const float mc = fmaxf(fmaxf(y0, y1), fmaxf(y2, y3));
      const float sh = lse2_shift(mc);
      lse2_combine(m, s, mc,
                   exp2_hw(y0 - sh) + exp2_hw(y1 - sh) + exp2_hw(y2 - sh) + exp2_hw(y3 - sh));
    }
  } else {
    for (long long j = threadIdx.x; j < vocab; j += kXentThreads) {
      const float y = x[j] * kLog2e;
      lse2_combine(m, s, y, 1.f);
    }
  }
  block_lse2(m, s);
  if (threadIdx.x == 0) {
    const float l = (m + log2f(s)) * kLn2;
    const long long t = targets[r];
    lse[r] = l;
    float lr = 0.f;
    if (t != ignore_index) lr = (t >= 0 && t < vocab) ? l - x[t] : __builtin_nanf("");
    loss_rows[r] = lr;
  }
}

template <int VEC>
__global__ void __launch_bounds__(kXentThreads)
xent_bwd_kernel(const float* __restrict__ logits, const long long* __restrict__ targets,
                const float* __restrict__ lse, const float* __restrict__ scale,
                float* __restrict__ dlogits, long long vocab, long long ignore_index) {
  const long long r = blockIdx.x;
  const float* x = logits + r * vocab;
  float* dx = dlogits + r * vocab;
  const long long t = targets[r];
  const bool ignored = t == ignore_index;
  const float g = ignored ? 0.f : scale[0];
  const float l2 = lse[r] * kLog2e;
  if constexpr (VEC == 4) {
    const float4* x4 = reinterpret_cast<const float4*>(x);
    float4* d4 = reinterpret_cast<float4*>(dx);
    const long long n4 = vocab / 4;
    for (long long i = threadIdx.x; i < n4; i += kXentThreads) {
      const float4 v = x4[i];
      float4 p = make_float4(exp2_hw(__builtin_fmaf(v.x, kLog2e, -l2)),
                             exp2_hw(__builtin_fmaf(v.y, kLog2e, -l2)),
                             exp2_hw(__builtin_fmaf(v.z, kLog2e, -l2)),
                             exp2_hw(__builtin_fmaf(v.w, kLog2e, -l2)));
      if ((t >> 2) == i) {   // the target's element: p - 1 (one thread, once)
        const int k = (int)(t & 3);
        if (k == 0) p.x -= 1.f;
        if (k == 1) p.y -= 1.f;
        if (k == 2) p.z -= 1.f;
        if (k == 3) p.w -= 1.f;
      }
      d4[i] = make_float4(g * p.x, g * p.y, g * p.z, g * p.w);
    }
  } else {
    for (long long j = threadIdx.x; j < vocab; j += kXentThreads) {
      const float p = exp2_hw(__builtin_fmaf(x[j], kLog2e, -l2));
      dx[j] = g * (j == t ? p - 1.f : p);
    }
  }
}

}  // namespace mhs
