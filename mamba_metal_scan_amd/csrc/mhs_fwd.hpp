// Forward selective scan for gfx950.
//
// Follows the math of the reference's ssm_fwd (mamba_metal/scan.py:78-127):
//   da = exp(-dt * Aneg); h = da * h + B * (dt * x); y = sum_n C * h;
//   h is written to ckpt at the end of every chunk of K steps (and at T-1).
//
// MI355X mapping (not the reference's one-thread-per-channel layout):
//   grid (ceil(D/64), batch), block 64*G. Wave w of the block owns state lanes
//   n in [w*NPL, w*NPL+NPL) of the block's 64 channels, so the N-vector of one
//   channel is spread over G waves (filling 256 CUs at batch 16 x D 1.5k) and
//   each lane keeps NPL recurrences in VGPRs for the whole sequence.
//   Time advances in sub-chunks of KI steps. Per sub-chunk the block stages
//   x, dt (KI x 64) and B, C (KI x N) in LDS with one coalesced float4 per
//   thread, prefetched one sub-chunk ahead in VGPRs. The per-wave partial sums
//   of y (over the wave's NPL states) are combined across the G waves through
//   LDS and written once, coalesced along d.
#pragma once

#include "mhs_common.hpp"

namespace mhs {

struct FwdArgs {
  const float* x;
  const float* dt;
  const float* aneg;
  const float* B;
  const float* C;
  float* y;        // may be null: then no y traffic at all
  float* ckpt;     // may be null
  float* h_last;   // may be null
  int T, D, K, nchunk;
  int vec4;        // x, dt 16-byte aligned and D % 4 == 0
};

// LDS floats used by fwd_kernel for G waves.
__host__ __device__ constexpr int fwd_lds_floats(int KI, int G, int NPL) {
  return KI * 64 * 2          // x, dt tiles
         + 2 * KI * G * NPL   // B, C tiles
         + G * KI * 64;       // per-wave y partials
}

template <int NPL, int KI, int MAXG, int PER, int PERS>
__global__ void __launch_bounds__(64 * MAXG)
fwd_kernel(FwdArgs a) {
  extern __shared__ float lds[];
  const int G = blockDim.x >> 6;
  const int N = G * NPL;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int b = blockIdx.y;
  const int d0 = blockIdx.x * 64;
  const int d = d0 + lane;
  const bool act = d < a.D;
  const int n0 = wave * NPL;
  const int T = a.T, D = a.D;

  float* tX = lds;
  float* tD = tX + KI * 64;
  float* tB = tD + KI * 64;
  float* tC = tB + KI * N;
  float* tY = tC + KI * N;
  const float* wB = tB + wave * KI * NPL;  // this wave's [KI][NPL] slice
  const float* wC = tC + wave * KI * NPL;

  float a2[NPL], h[NPL];
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    a2[j] = act ? -a.aneg[(size_t)d * N + n0 + j] * kLog2e : 0.f;
    h[j] = 0.f;
  }

  const size_t row0 = (size_t)b * T;
  const float* xb = a.x + row0 * D + d0;
  const float* db = a.dt + row0 * D + d0;
  const float* Bb = a.B + row0 * N;
  const float* Cb = a.C + row0 * N;

  const TileLoader<KI, PER> tl(tid, blockDim.x);
  const RowLoader<PERS, KI, NPL> rl(tid, blockDim.x, N);
  float4 px[PER], pd[PER];
  float pb[PERS], pc[PERS];
  {
    const int len = min(KI, T);
    tl.load(px, xb, len, D, d0, a.vec4);
    tl.load(pd, db, len, D, d0, a.vec4);
    rl.load(pb, Bb, len, N);
    rl.load(pc, Cb, len, N);
  }

  int next_ck = min(a.K, T);
  int ck = 0;
  for (int t0 = 0; t0 < T; t0 += KI) {
    const int len = min(KI, T - t0);
    tl.store(tX, px);
    tl.store(tD, pd);
    rl.store(tB, pb);
    rl.store(tC, pc);
    if (t0 + KI < T) {
      const int nlen = min(KI, T - t0 - KI);
      const size_t off = (size_t)(t0 + KI);
      tl.load(px, xb + off * D, nlen, D, d0, a.vec4);
      tl.load(pd, db + off * D, nlen, D, d0, a.vec4);
      rl.load(pb, Bb + off * N, nlen, N);
      rl.load(pc, Cb + off * N, nlen, N);
    }
    __syncthreads();

    // Steps k >= len of the last sub-chunk see zero-filled tiles: dA = 1 and
    // b = 0 there, so h passes through unchanged and nothing is written.
    float dtv = tD[lane], xv = tX[lane];
    float Bv[NPL], Cv[NPL];
    load_vec<NPL>(Bv, wB);
    load_vec<NPL>(Cv, wC);
#pragma unroll
    for (int k = 0; k < KI; ++k) {
      // Operands of step k+1, read while step k computes.
      float dtn = 0.f, xn = 0.f, Bn[NPL], Cn[NPL];
      if (k + 1 < KI) {
        dtn = tD[(k + 1) * 64 + lane];
        xn = tX[(k + 1) * 64 + lane];
        load_vec<NPL>(Bn, wB + (k + 1) * NPL);
        load_vec<NPL>(Cn, wC + (k + 1) * NPL);
      }
      const float bx = dtv * xv;
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < NPL; ++j) {
        const float da = exp2_hw(dtv * a2[j]);
        h[j] = __builtin_fmaf(da, h[j], Bv[j] * bx);
        acc = __builtin_fmaf(Cv[j], h[j], acc);
      }
      // Written immediately (not kept for after the loop), so the y FMAs stay
      // inside the step and the compiler cannot keep KI steps of h live.
      if (a.y != nullptr) tY[(wave * KI + k) * 64 + lane] = acc;
      if (t0 + k + 1 == next_ck) {
        if (a.ckpt != nullptr && act)
          store_vec<NPL>(a.ckpt + (((size_t)b * a.nchunk + ck) * D + d) * N + n0, h);
        ++ck;
        next_ck = min(next_ck + a.K, T);
      }
      step_fence();
      if (k + 1 < KI) {
        dtv = dtn;
        xv = xn;
#pragma unroll
        for (int j = 0; j < NPL; ++j) {
          Bv[j] = Bn[j];
          Cv[j] = Cn[j];
        }
      }
    }

    if (a.y != nullptr) {
      __syncthreads();
      float* yb = a.y + (row0 + t0) * D + d;
      for (int k = wave; k < len; k += G) {
        float s = 0.f;
        for (int g = 0; g < G; ++g) s += tY[(g * KI + k) * 64 + lane];
        if (act) yb[(size_t)k * D] = s;
      }
    }
    __syncthreads();
  }

  if (a.h_last != nullptr && act)
    store_vec<NPL>(a.h_last + ((size_t)b * D + d) * N + n0, h);
}

}  // namespace mhs
