// Backward selective scan for gfx950.
//
// Gradients (the reference derives them at mamba_metal/scan.py:22-34 and
// computes them in ssm_bwd, scan.py:132-261). With G_t the adjoint of h_t and
// hm_t = dA_t * h_{t-1} (= h_t - b_t):
//   G_t    = dy_t * C_t + dA_{t+1} * G_{t+1}          (G_{T-1} also gets dh_last)
//   dx_t   = dt_t * sum_n G_tn B_tn
//   ddt_t  = x_t * sum_n G_tn B_tn - sum_n Aneg_n G_tn hm_tn
//   dAneg  = -sum_{b,t} dt_t G_tn hm_tn
//   dB_tn  = sum_d G_tdn dt_td x_td          dC_tn = sum_d dy_td h_tdn
//
// MI355X mapping. Same block decomposition as the forward (64 channels x one
// batch row per block, G waves x NPL states). Chunks of K <= KI steps are
// walked last to first. For each chunk the block stages x, dt, dy and B, C in
// LDS (prefetched one chunk ahead), every lane recomputes its chunk of h and
// dA from the checkpoint into VGPRs (hs[KI][NPL], da[KI][NPL]; nothing goes to
// global scratch), then walks the chunk backwards carrying G in VGPRs across
// chunk boundaries. It uses hm = dA * h_{t-1} from the recomputed chunk, so it
// never subtracts h_t - b_t.
//   dx / ddt: the per-wave partial sums over the wave's NPL states are
//             combined across the G waves through LDS, written once.
//   dAneg:    accumulated per lane over the whole walk (no cross-lane traffic),
//             written once per (b, d, n) to a workspace slot.
//   dB / dC:  sums over the 64 channels of the block. Each wave writes its
//             per-lane G (weight dt*x) and h (weight dy) rows to LDS and
//             reduces RROWS rows at a time: LPR = 64/RROWS lanes per row, each
//             doing RROWS fused multiply-adds over its slice of channels,
//             then a DPP tree over the LPR lanes. The per-block sums go to a
//             workspace slot; bwd_reduce_kernel adds the blocks in a fixed
//             order, so the result does not depend on scheduling.
#pragma once

#include "mhs_common.hpp"

namespace mhs {

struct BwdArgs {
  const float* x;
  const float* dt;
  const float* aneg;
  const float* B;
  const float* C;
  const float* dy;
  const float* dh_last;  // may be null
  const float* ckpt;     // (batch, nchunk, D, N), stride K
  float* dx;
  float* ddt;
  float* wsB;            // (nblk, batch, T, N)
  float* wsC;            // (nblk, batch, T, N)
  float* wsA;            // (batch, D, N)
  int batch, T, D, K, nchunk;
  int vec4;              // x, dt, dy 16-byte aligned and D % 4 == 0
};

__host__ __device__ constexpr int bwd_lds_floats(int KI, int G, int NPL, int RROWS) {
  return KI * 64 * 3                        // x, dt, dy tiles
         + 2 * KI * G * NPL                 // B, C tiles
         + G * KI * 64 * 2                  // per-wave (s1, s2) partials
         + G * RROWS * 64                   // per-wave reduction rows
         + G * (RROWS / (2 * NPL)) * 2 * 64;  // per-wave reduction weights
}

template <int NPL, int KI, int MAXG, int PER, int PERS, int RROWS>
__global__ void __launch_bounds__(64 * MAXG)
bwd_kernel(BwdArgs a) {
  constexpr int RPS = 2 * NPL;          // reduction rows per time step
  constexpr int SB = RROWS / RPS;       // time steps per reduction batch
  constexpr int LPR = 64 / RROWS;       // lanes per reduced row
  static_assert(RROWS % RPS == 0 && 64 % RROWS == 0 && KI % SB == 0, "bad reduction shape");
  static_assert(RROWS % 4 == 0, "rows are read as float4");

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
  const int T = a.T, D = a.D, K = a.K;

  float* tX = lds;
  float* tD = tX + KI * 64;
  float* tY = tD + KI * 64;
  float* tB = tY + KI * 64;
  float* tC = tB + KI * N;
  float2* tS = reinterpret_cast<float2*>(tC + KI * N);
  const float* wB = tB + wave * KI * NPL;  // this wave's [KI][NPL] slice
  const float* wC = tC + wave * KI * NPL;
  float* tR = reinterpret_cast<float*>(tS + G * KI * 64) + wave * RROWS * 64;
  float* tW = reinterpret_cast<float*>(tS + G * KI * 64) + G * RROWS * 64 + wave * SB * 2 * 64;

  float an[NPL], a2[NPL], g[NPL], acc[NPL], dan[NPL];
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    an[j] = act ? a.aneg[(size_t)d * N + n0 + j] : 0.f;
    a2[j] = -an[j] * kLog2e;
    g[j] = (a.dh_last != nullptr && act) ? a.dh_last[((size_t)b * D + d) * N + n0 + j] : 0.f;
    acc[j] = 0.f;
    dan[j] = 1.f;
  }

  const size_t row0 = (size_t)b * T;
  const float* xb = a.x + row0 * D + d0;
  const float* db = a.dt + row0 * D + d0;
  const float* yb = a.dy + row0 * D + d0;
  const float* Bb = a.B + row0 * N;
  const float* Cb = a.C + row0 * N;
  const float* ckb = a.ckpt + (size_t)b * a.nchunk * D * N + (size_t)d * N + n0;

  const TileLoader<KI, PER> tl(tid, blockDim.x);
  const RowLoader<PERS, KI, NPL> rl(tid, blockDim.x, N);
  float4 px[PER], pd[PER], py[PER];
  float pb[PERS], pc[PERS], ph[NPL];

  // Prefetch the last chunk.
  {
    const int c = a.nchunk - 1;
    const int t0 = c * K;
    const int len = min(K, T - t0);
    const size_t off = (size_t)t0;
    tl.load(px, xb + off * D, len, D, d0, a.vec4);
    tl.load(pd, db + off * D, len, D, d0, a.vec4);
    tl.load(py, yb + off * D, len, D, d0, a.vec4);
    rl.load(pb, Bb + off * N, len, N);
    rl.load(pc, Cb + off * N, len, N);
#pragma unroll
    for (int j = 0; j < NPL; ++j) ph[j] = 0.f;
    if (c > 0 && act) load_vec<NPL>(ph, ckb + (size_t)(c - 1) * D * N);
  }

  for (int c = a.nchunk - 1; c >= 0; --c) {
    const int t0 = c * K;
    const int len = min(K, T - t0);
    float hc[NPL];
#pragma unroll
    for (int j = 0; j < NPL; ++j) hc[j] = ph[j];
    tl.store(tX, px);
    tl.store(tD, pd);
    tl.store(tY, py);
    rl.store(tB, pb);
    rl.store(tC, pc);
    if (c > 0) {
      const size_t off = (size_t)(t0 - K);
      tl.load(px, xb + off * D, K, D, d0, a.vec4);
      tl.load(pd, db + off * D, K, D, d0, a.vec4);
      tl.load(py, yb + off * D, K, D, d0, a.vec4);
      rl.load(pb, Bb + off * N, K, N);
      rl.load(pc, Cb + off * N, K, N);
#pragma unroll
      for (int j = 0; j < NPL; ++j) ph[j] = 0.f;
      if (c > 1 && act) load_vec<NPL>(ph, ckb + (size_t)(c - 2) * D * N);
    }
    __syncthreads();

    // Recompute the chunk's h and dA in registers. Steps k >= len of a short
    // chunk see zero-filled tiles (dt = x = dy = B = C = 0): dA = 1 and b = 0
    // there, so they are exact identity steps for h and for G, contribute
    // zero to every accumulated gradient, and their outputs are not written.
    // That keeps this loop free of per-step branches.
    float hs[KI][NPL], da[KI][NPL];
    {
      float dtv = tD[lane], xv = tX[lane], Bv[NPL];
      load_vec<NPL>(Bv, wB);
#pragma unroll
      for (int k = 0; k < KI; ++k) {
        float dtn = 0.f, xn = 0.f, Bn[NPL];
        if (k + 1 < KI) {
          dtn = tD[(k + 1) * 64 + lane];
          xn = tX[(k + 1) * 64 + lane];
          load_vec<NPL>(Bn, wB + (k + 1) * NPL);
        }
        const float dtx = dtv * xv;
#pragma unroll
        for (int j = 0; j < NPL; ++j) {
          da[k][j] = exp2_hw(dtv * a2[j]);
          hs[k][j] = __builtin_fmaf(da[k][j], k == 0 ? hc[j] : hs[k - 1][j], Bv[j] * dtx);
        }
        step_fence();
        if (k + 1 < KI) {
          dtv = dtn;
          xv = xn;
#pragma unroll
          for (int j = 0; j < NPL; ++j) Bv[j] = Bn[j];
        }
      }
    }

    // Reverse walk.
    lds_reload_point();
    float dtv = tD[(KI - 1) * 64 + lane], xv = tX[(KI - 1) * 64 + lane];
    float dyv = tY[(KI - 1) * 64 + lane];
    float Bv[NPL], Cv[NPL];
    load_vec<NPL>(Bv, wB + (KI - 1) * NPL);
    load_vec<NPL>(Cv, wC + (KI - 1) * NPL);
#pragma unroll
    for (int k = KI - 1; k >= 0; --k) {
      const int slot = k % SB;
      float dtn = 0.f, xn = 0.f, dyn = 0.f, Bn[NPL], Cn[NPL];
      if (k > 0) {
        dtn = tD[(k - 1) * 64 + lane];
        xn = tX[(k - 1) * 64 + lane];
        dyn = tY[(k - 1) * 64 + lane];
        load_vec<NPL>(Bn, wB + (k - 1) * NPL);
        load_vec<NPL>(Cn, wC + (k - 1) * NPL);
      }
      {
        const float dtx = dtv * xv;
        float s1 = 0.f, s2 = 0.f;
#pragma unroll
        for (int j = 0; j < NPL; ++j) {
          const float gj = __builtin_fmaf(dan[j], g[j], dyv * Cv[j]);
          const float hm = da[k][j] * (k == 0 ? hc[j] : hs[k - 1][j]);
          s1 = __builtin_fmaf(gj, Bv[j], s1);
          const float q = gj * hm;
          s2 = __builtin_fmaf(an[j], q, s2);
          acc[j] = __builtin_fmaf(dtv, q, acc[j]);
          g[j] = gj;
          dan[j] = da[k][j];
        }
        tS[(wave * KI + k) * 64 + lane] = make_float2(s1, s2);
#pragma unroll
        for (int j = 0; j < NPL; ++j) {
          tR[(slot * RPS + j) * 64 + lane] = g[j];
          tR[(slot * RPS + NPL + j) * 64 + lane] = hs[k][j];
        }
        tW[(slot * 2 + 0) * 64 + lane] = dtx;
        tW[(slot * 2 + 1) * 64 + lane] = dyv;
      }
      if (slot == 0) {
        // Rows for steps k .. k+SB-1 are in place; rows of steps >= len are
        // identity-step rows and are not written out.
        wave_lds_sync();
        const int r = lane / LPR;
        const int seg = lane % LPR;
        const int slot_r = r / RPS;
        const int kind = (r % RPS) / NPL;
        const int j = r % NPL;
        const float* rr = tR + r * 64 + seg * RROWS;
        const float* ww = tW + (slot_r * 2 + kind) * 64 + seg * RROWS;
        float sum = 0.f;
#pragma unroll
        for (int i = 0; i < RROWS; i += 4) {
          const float4 v = *reinterpret_cast<const float4*>(rr + i);
          const float4 w = *reinterpret_cast<const float4*>(ww + i);
          sum = __builtin_fmaf(v.x, w.x, sum);
          sum = __builtin_fmaf(v.y, w.y, sum);
          sum = __builtin_fmaf(v.z, w.z, sum);
          sum = __builtin_fmaf(v.w, w.w, sum);
        }
        sum = group_sum<LPR>(sum);
        const int kk = k + slot_r;
        if (seg == 0 && kk < len) {
          float* dst = kind ? a.wsC : a.wsB;
          dst[(((size_t)blockIdx.x * a.batch + b) * T + t0 + kk) * N + n0 + j] = sum;
        }
        wave_lds_sync();
      }
      step_fence();
      if (k > 0) {
        dtv = dtn;
        xv = xn;
        dyv = dyn;
#pragma unroll
        for (int j = 0; j < NPL; ++j) {
          Bv[j] = Bn[j];
          Cv[j] = Cn[j];
        }
      }
    }
    __syncthreads();

    // dx, ddt for this chunk: wave w finalizes steps k with k % G == w.
    float* dxb = a.dx + (row0 + t0) * D + d;
    float* ddtb = a.ddt + (row0 + t0) * D + d;
    for (int k = wave; k < len; k += G) {
      float s1 = 0.f, s2 = 0.f;
      for (int w = 0; w < G; ++w) {
        const float2 v = tS[(w * KI + k) * 64 + lane];
        s1 += v.x;
        s2 += v.y;
      }
      if (act) {
        dxb[(size_t)k * D] = tD[k * 64 + lane] * s1;
        ddtb[(size_t)k * D] = __builtin_fmaf(tX[k * 64 + lane], s1, -s2);
      }
    }
    __syncthreads();
  }

  if (act) {
    float out[NPL];
#pragma unroll
    for (int j = 0; j < NPL; ++j) out[j] = -acc[j];
    store_vec<NPL>(a.wsA + ((size_t)b * D + d) * N + n0, out);
  }
}

// dB, dC: sum the per-block partials over the nblk channel blocks;
// dAneg: sum the per-batch partials over the batch. Fixed summation order.
__global__ void __launch_bounds__(256)
bwd_reduce_kernel(const float* __restrict__ wsB, const float* __restrict__ wsC,
                  const float* __restrict__ wsA, float* __restrict__ dB,
                  float* __restrict__ dC, float* __restrict__ daneg,
                  int nblk, int batch, long long S, long long A) {
  const long long stride = (long long)gridDim.x * blockDim.x;
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < S + A; i += stride) {
    if (i < S) {
      float sb = 0.f, sc = 0.f;
      for (int cb = 0; cb < nblk; ++cb) {
        sb += wsB[(size_t)cb * S + i];
        sc += wsC[(size_t)cb * S + i];
      }
      dB[i] = sb;
      dC[i] = sc;
    } else {
      const long long j = i - S;
      float s = 0.f;
      for (int bb = 0; bb < batch; ++bb) s += wsA[(size_t)bb * A + j];
      daneg[j] = s;
    }
  }
}

}  // namespace mhs
