// Shared device helpers for the gfx950 selective-scan kernels.
//
// Layout conventions (all fp32, contiguous, row-major; see include/mamba_hip_scan.h):
//   x, dt, y, dy, dx, ddt : (batch, T, D)      B, C, dB, dC : (batch, T, N)
//   aneg                  : (D, N)             ckpt         : (batch, nchunk, D, N)
//
// Work decomposition used by the forward and backward kernels: one workgroup
// owns one batch row b and a block of 64 consecutive channels d; its G waves
// split the N state lanes into G groups of NPL (wave w owns n in
// [w*NPL, (w+1)*NPL)). Every lane therefore carries NPL independent
// recurrences in VGPRs, B/C are wave-uniform within a group, and x / dt / dy
// rows are shared by the whole workgroup through LDS.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mhs {

constexpr float kLog2e = 1.4426950408889634f;

// v_exp_f32: 2^v, the hardware transcendental (one instruction, flushes
// results below the fp32 normal range to zero, which the recurrence tolerates:
// such a decay factor erases the state exactly as an exact underflow would).
__device__ __forceinline__ float exp2_hw(float v) { return __builtin_amdgcn_exp2f(v); }

// v_add_f32 with a DPP source permutation: a cross-lane add in one VALU slot.
template <int CTRL>
__device__ __forceinline__ float dpp_add(float v) {
  const int p = __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true);
  return v + __int_as_float(p);
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // lane i <-> 7-i inside each group of 8
constexpr int kDppMirror = 0x140;     // lane i <-> 15-i inside each row of 16

// Sum v over aligned groups of L lanes (L in {1,2,4,8,16}); every lane of the
// group ends with the group total.
template <int L>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (L >= 2) v = dpp_add<kDppXor1>(v);
  if constexpr (L >= 4) v = dpp_add<kDppXor2>(v);
  if constexpr (L >= 8) v = dpp_add<kDppHalfMirror>(v);
  if constexpr (L >= 16) v = dpp_add<kDppMirror>(v);
  static_assert(L <= 16, "group_sum covers at most one DPP row");
  return v;
}

// Ordering point for LDS traffic that stays inside one wavefront: the wave's
// LDS instructions execute in issue order, so only the compiler must be kept
// from moving accesses across this point.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Compiler-only memory clobber: values read from LDS before this point are
// re-read after it instead of being kept live in VGPRs across it.
__device__ __forceinline__ void lds_reload_point() { asm volatile("" ::: "memory"); }

// Scheduling fence: the compiler may not move instructions across it. Used
// once per time step so that LDS reads are issued one step ahead (by hand)
// rather than hoisted for the whole unrolled sub-chunk, which would hold
// KI steps of operands in VGPRs at once.
__device__ __forceinline__ void step_fence() { __builtin_amdgcn_sched_barrier(0); }

// NPL consecutive floats: vector load/store (NPL in {1, 2, 4}).
template <int NPL>
__device__ __forceinline__ void load_vec(float (&v)[NPL], const float* p) {
  if constexpr (NPL == 4) {
    const float4 t = *reinterpret_cast<const float4*>(p);
    v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
  } else if constexpr (NPL == 2) {
    const float2 t = *reinterpret_cast<const float2*>(p);
    v[0] = t.x; v[1] = t.y;
  } else {
    v[0] = p[0];
  }
}

template <int NPL>
__device__ __forceinline__ void store_vec(float* p, const float (&v)[NPL]) {
  if constexpr (NPL == 4) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  } else if constexpr (NPL == 2) {
    *reinterpret_cast<float2*>(p) = make_float2(v[0], v[1]);
  } else {
    p[0] = v[0];
  }
}

// Cooperative staging of one chunk of a (batch, T, D) tensor into a
// [KI][64] LDS tile: the workgroup's 64 channels for KI time steps. The tile
// is KI*16 float4 quads; thread tid moves quads tid, tid+nthreads, ... (at
// most PER of them, PER*nthreads >= KI*16 is checked on the host). Rows at or
// beyond `len` and channels at or beyond D are zero-filled.
template <int KI, int PER>
struct TileLoader {
  int tid, nthreads;
  __device__ __forceinline__ TileLoader(int tid_, int nthreads_) : tid(tid_), nthreads(nthreads_) {}

  // base points at element (b, t0, d0) of the tensor; row stride D.
  // vec4: base is 16-byte aligned and D % 4 == 0.
  __device__ __forceinline__ void load(float4 (&v)[PER], const float* base, int len, int D,
                                       int d0, bool vec4) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int e = tid + i * nthreads;
      const int k = e >> 4, q = e & 15;
      v[i] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (e < KI * 16 && k < len) {
        const int dq = d0 + 4 * q;
        const float* p = base + (size_t)k * D + 4 * q;
        if (vec4 && dq + 3 < D) {
          v[i] = *reinterpret_cast<const float4*>(p);
        } else {
          if (dq + 0 < D) v[i].x = p[0];
          if (dq + 1 < D) v[i].y = p[1];
          if (dq + 2 < D) v[i].z = p[2];
          if (dq + 3 < D) v[i].w = p[3];
        }
      }
    }
  }
  __device__ __forceinline__ void store(float* tile, const float4 (&v)[PER]) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int e = tid + i * nthreads;
      if (e < KI * 16) *reinterpret_cast<float4*>(tile + 4 * e) = v[i];
    }
  }
};

// Cooperative staging of KI rows of a (batch, T, N) tensor (B or C) into an
// LDS tile laid out wave-major, [G][KI][NPL]: wave w reads its NPL states of
// step k at w*KI*NPL + k*NPL, a compile-time offset from a per-wave base.
// Thread tid moves elements e = tid, tid+nthreads, ... (at most PERS of them)
// of the row-major global block; rows at or beyond `len` are zero-filled.
template <int PERS, int KI, int NPL>
struct RowLoader {
  int src[PERS];  // element index in the global [KI][N] block, or -1
  int dst[PERS];  // its slot in the wave-major tile
  __device__ __forceinline__ RowLoader(int tid, int nthreads, int N) {
#pragma unroll
    for (int i = 0; i < PERS; ++i) {
      const int e = tid + i * nthreads;
      const int k = e / N, n = e % N;
      src[i] = e < KI * N ? e : -1;
      dst[i] = (n / NPL) * (KI * NPL) + k * NPL + (n % NPL);
    }
  }
  // base points at (b, t0, 0).
  __device__ __forceinline__ void load(float (&v)[PERS], const float* base, int len, int N) const {
#pragma unroll
    for (int i = 0; i < PERS; ++i) v[i] = (src[i] >= 0 && src[i] < len * N) ? base[src[i]] : 0.f;
  }
  __device__ __forceinline__ void store(float* tile, const float (&v)[PERS]) const {
#pragma unroll
    for (int i = 0; i < PERS; ++i)
      if (src[i] >= 0) tile[dst[i]] = v[i];
  }
};

}  // namespace mhs
