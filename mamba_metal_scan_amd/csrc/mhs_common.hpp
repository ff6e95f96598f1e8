// Shared device helpers for the gfx950 selective-scan kernels.
//
// Layout conventions (all fp32, contiguous, row-major; see include/mamba_hip_scan.h):
//   x, dt, y, dy, dx, ddt : (batch, T, D)      B, C, dB, dC : (batch, T, N)
//   aneg                  : (D, N)             ckpt         : (batch, nchunk, D, N)
//
// Work decomposition used by the forward and backward kernels: one workgroup
// owns one batch row b and a block of CH consecutive channels d. The N states
// are split into NQ groups of NPL; each wave holds NH = 64/CH groups (NH = 2:
// lanes 0-31 and 32-63 carry the same 32 channels for two different groups),
// so a block has G = NQ/NH waves. Every lane carries NPL independent
// recurrences in VGPRs for the whole sequence; x / dt / dy and B / C are
// staged per block in LDS and shared by its waves.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mhs {

constexpr float kLog2e = 1.4426950408889634f;

// v_exp_f32: 2^v, the hardware transcendental (one instruction, flushes
// results below the fp32 normal range to zero, which the recurrence tolerates:
// such a decay factor erases the state exactly as an exact underflow would).
__device__ __forceinline__ float exp2_hw(float v) { return __builtin_amdgcn_exp2f(v); }

// sigmoid(v) = 1 / (1 + 2^(-v log2 e)) with the hardware exp2 and reciprocal
// (about 2 ulp; v -> -inf gives 0, v -> +inf gives 1).
__device__ __forceinline__ float sigmoid_f(float v) {
  return __builtin_amdgcn_rcpf(1.f + exp2_hw(-v * kLog2e));
}

// The block's dt gate (mamba_metal/model.py:197): dt = lo + span * sigmoid(raw).
__device__ __forceinline__ float gate_dt(float raw, float lo, float span) {
  return __builtin_fmaf(span, sigmoid_f(raw), lo);
}

// softplus(a) = log(1 + e^a) (mamba_metal/model.py:200, Aneg = softplus(A)),
// written as max(a, 0) + log1p(e^-|a|) so that it neither overflows for large
// a nor loses the small values for very negative a.
__device__ __forceinline__ float softplus_f(float a) {
  return fmaxf(a, 0.f) + log1pf(expf(-fabsf(a)));
}

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

constexpr int kDppRor8 = 0x128;       // row_ror:8: lane i <-> i^8 inside each row of 16

template <int CTRL>
__device__ __forceinline__ float dpp_get(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}

// One reduce-scatter stage over lane bit b: the values are paired (v[2i],
// v[2i+1]); a lane whose bit b is 0 keeps the pair sum of v[2i] over itself
// and its partner, a lane whose bit is 1 the sum of v[2i+1]. The partner
// (DPP control CTRL) must differ from the lane in bit b and otherwise only in
// bits not yet reduced.
template <int CTRL, int M>
__device__ __forceinline__ void rs_stage_dpp(const float (&v)[M], float (&o)[M / 2], bool bit) {
#pragma unroll
  for (int i = 0; i < M / 2; ++i) {
    const float send = bit ? v[2 * i] : v[2 * i + 1];
    const float keep = bit ? v[2 * i + 1] : v[2 * i];
    o[i] = keep + dpp_get<CTRL>(send);
  }
}

// The reduce-scatter stages over lane bits 3 and 2 as bank-masked DPP adds
// (a bank is 4 lanes of a 16-lane row; bit 3 splits banks {0,1} from {2,3},
// bit 2 banks {0,2} from {1,3}): the pair (x, y) becomes x + x' in the banks
// whose bit is 0 and y + y' in the others (x' the partner's x: row_ror:8 is
// lane i <-> i^8, row_half_mirror lane i <-> 7-i), two instructions per
// pair. Same sums, in the same order, as rs_stage_dpp (a + b == b + a).
// The s_nop's give the 2 wait states a DPP read of a VGPR needs after a VALU
// write of it (the compiler does not look inside the asm): before the first
// reads of inputs written by compiled code, between the two stages, and
// after the block for compiled DPP reads of its outputs.
__device__ __forceinline__ float rs_bits32_8(const float (&a)[4]) {
  float b0, b1, c;
  asm("s_nop 1\n\t"
      "v_add_f32_dpp %1, %3, %3 row_ror:8 row_mask:0xf bank_mask:0x3\n\t"
      "v_add_f32_dpp %1, %4, %4 row_ror:8 row_mask:0xf bank_mask:0xc\n\t"
      "v_add_f32_dpp %2, %5, %5 row_ror:8 row_mask:0xf bank_mask:0x3\n\t"
      "v_add_f32_dpp %2, %6, %6 row_ror:8 row_mask:0xf bank_mask:0xc\n\t"
      "s_nop 0\n\t"
      "v_add_f32_dpp %0, %1, %1 row_half_mirror row_mask:0xf bank_mask:0x5\n\t"
      "v_add_f32_dpp %0, %2, %2 row_half_mirror row_mask:0xf bank_mask:0xa\n\t"
      "s_nop 1"
      : "=&v"(c), "=&v"(b0), "=&v"(b1)
      : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]));
  return c;
}
__device__ __forceinline__ void rs_bits32_16(const float (&a)[8], float (&c)[2]) {
  float b0, b1, b2, b3;
  asm("s_nop 1\n\t"
      "v_add_f32_dpp %2, %6, %6 row_ror:8 row_mask:0xf bank_mask:0x3\n\t"
      "v_add_f32_dpp %2, %7, %7 row_ror:8 row_mask:0xf bank_mask:0xc\n\t"
      "v_add_f32_dpp %3, %8, %8 row_ror:8 row_mask:0xf bank_mask:0x3\n\t"
      "v_add_f32_dpp %3, %9, %9 row_ror:8 row_mask:0xf bank_mask:0xc\n\t"
      "v_add_f32_dpp %4, %10, %10 row_ror:8 row_mask:0xf bank_mask:0x3\n\t"
      "v_add_f32_dpp %4, %11, %11 row_ror:8 row_mask:0xf bank_mask:0xc\n\t"
      "v_add_f32_dpp %5, %12, %12 row_ror:8 row_mask:0xf bank_mask:0x3\n\t"
      "v_add_f32_dpp %5, %13, %13 row_ror:8 row_mask:0xf bank_mask:0xc\n\t"
      "v_add_f32_dpp %0, %2, %2 row_half_mirror row_mask:0xf bank_mask:0x5\n\t"
      "v_add_f32_dpp %0, %3, %3 row_half_mirror row_mask:0xf bank_mask:0xa\n\t"
      "v_add_f32_dpp %1, %4, %4 row_half_mirror row_mask:0xf bank_mask:0x5\n\t"
      "v_add_f32_dpp %1, %5, %5 row_half_mirror row_mask:0xf bank_mask:0xa\n\t"
      "s_nop 1"
      : "=&v"(c[0]), "=&v"(c[1]), "=&v"(b0), "=&v"(b1), "=&v"(b2), "=&v"(b3)
      : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(a[4]), "v"(a[5]), "v"(a[6]),
        "v"(a[7]));
}

// The stages over lane bits 3 and 2 of the row-partial reduce-scatter of 8
// values per lane (see row_partial_pairs): a = (x0, x1, y0, y1). Bit 3 by
// bank-masked row_ror:8 adds (pairs (x0, y0) and (x1, y1): x in the banks
// whose bit 3 is 0, y in the others), then bit 2 by bank-masked row shifts
// (partner lane i ^ 4: row_shl:4, lane i reads lane i + 4, in banks 0 and
// 2; row_shr:4, lane i reads lane i - 4, in banks 1 and 3): the first
// result in the banks whose bit 2 is 0, the second in the others. Wait
// states as in rs_bits32_8.
__device__ __forceinline__ float rs_bits32_shift(const float (&a)[4]) {
  float b0, b1, c;
  asm("s_nop 1\n\t"
      "v_add_f32_dpp %1, %3, %3 row_ror:8 row_mask:0xf bank_mask:0x3\n\t"
      "v_add_f32_dpp %1, %5, %5 row_ror:8 row_mask:0xf bank_mask:0xc\n\t"
      "v_add_f32_dpp %2, %4, %4 row_ror:8 row_mask:0xf bank_mask:0x3\n\t"
      "v_add_f32_dpp %2, %6, %6 row_ror:8 row_mask:0xf bank_mask:0xc\n\t"
      "s_nop 0\n\t"
      "v_add_f32_dpp %0, %1, %1 row_shl:4 row_mask:0xf bank_mask:0x5\n\t"
      "v_add_f32_dpp %0, %2, %2 row_shr:4 row_mask:0xf bank_mask:0xa\n\t"
      "s_nop 1"
      : "=&v"(c), "=&v"(b0), "=&v"(b1)
      : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]));
  return c;
}

// Partial sums over each 16-lane row of 8 products per lane, with the lanes
// of odd index holding their two states in swapped order (the lane's
// register j holds state j ^ (lane & 1)). Products x_j * q: kind 0 / 1 (x
// the adjoint G or the state h, q the channel's dt * x or dy), slot 0 / 1
// (two steps), j the register of the state. Stage over lane bit 0
// (quad_perm [1, 0, 3, 2]): the lane's product of register 0 plus the
// partner's product of register 1 is the pair sum of one state, state n0 +
// (lane & 1), in every lane. pair_sum_xor1 forms it from the factors, with
// the partner's operand q' held by this lane: the partner's product in one
// v_mul_f32_dpp (the compiler folds the DPP read into a plain multiply),
// rounded as the partner would round it, then fma(x0, q, x1' * q'), two
// VALU per pair, where products formed first and a DPP read of the
// partner's take three.
__device__ __forceinline__ float pair_sum_xor1(float x0, float x1, float q, float qp) {
  return __builtin_fmaf(x0, q, dpp_get<kDppXor1>(x1) * qp);
}
// The rest of the row partial, from the pair sums a = (kind 0 slot 0, kind 0
// slot 1, kind 1 slot 0, kind 1 slot 1): bit 3 (kind) and bit 2 (slot) as
// bank-masked stages, and bit 1 (quad_perm [2, 3, 0, 1]) as a plain add, 7
// instructions. Lane l returns the sum over the 16 lanes of its row of the
// product (kind (l >> 3) & 1, slot (l >> 2) & 1, state n0 + (l & 1)); the
// two rows of a half-wave (lane bit 4) are added later, in a fixed order.
__device__ __forceinline__ float row_partial_pairs(const float (&a)[4]) {
  return dpp_add<kDppXor2>(rs_bits32_shift(a));
}

// The stage over lane bit 3 alone, for a pair: (x, y) becomes x + x' in the
// banks whose bit 3 is 0 and y + y' in the others (as in rs_bits32_8).
__device__ __forceinline__ float rs_bit3_4(const float (&a)[2]) {
  float b;
  asm("s_nop 1\n\t"
      "v_add_f32_dpp %0, %1, %1 row_ror:8 row_mask:0xf bank_mask:0x3\n\t"
      "v_add_f32_dpp %0, %2, %2 row_ror:8 row_mask:0xf bank_mask:0xc\n\t"
      "s_nop 1"
      : "=&v"(b)
      : "v"(a[0]), "v"(a[1]));
  return b;
}

// Sums M values (M in {4, 8, 16}) over the 32 lanes of each half-wave, as a
// reduce-scatter: v_permlane16_swap across lane bit 4, then DPP row_ror:8
// (bit 3), row_half_mirror (bit 2) and quad_perm xor 2 (bit 1), each halving
// the values a lane holds, then plain DPP adds over the lane bits left. Lane l
// returns the half-wave total of v[rs_index<M>(l)]. Summation order is fixed:
// the result is bit-for-bit reproducible.
template <int M>
__device__ __forceinline__ float half_wave_reduce_scatter(const float (&v)[M], int lane) {
  static_assert(M == 4 || M == 8 || M == 16, "4, 8 or 16 values per lane");
  float a[M / 2];
#pragma unroll
  for (int i = 0; i < M / 2; ++i) {
    const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[2 * i]),
                                                    __float_as_uint(v[2 * i + 1]), false, false);
    a[i] = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
  }
  if constexpr (M == 4) {
    // Bits 2, 1, 0 are all left: a plain sum over each group of 8 lanes.
    return group_sum<8>(rs_bit3_4(a));
  } else {
    float c[M / 8];
    if constexpr (M == 8) {
      c[0] = rs_bits32_8(a);
    } else {
      rs_bits32_16(a, c);
    }
    float r;
    if constexpr (M == 8) {
      r = dpp_add<kDppXor2>(c[0]);
    } else {
      float d[1];
      rs_stage_dpp<kDppXor2>(c, d, (lane >> 1) & 1);
      r = d[0];
    }
    return dpp_add<kDppXor1>(r);
  }
}
// Index of the value whose total half_wave_reduce_scatter<M> leaves in lane l.
template <int M>
__device__ __forceinline__ int rs_index(int lane) {
  if constexpr (M == 4) return 2 * ((lane >> 3) & 1) + ((lane >> 4) & 1);
  const int i = 4 * ((lane >> 2) & 1) + 2 * ((lane >> 3) & 1) + ((lane >> 4) & 1);
  return M == 8 ? i : i + 8 * ((lane >> 1) & 1);
}

// Ordering point for LDS traffic that stays inside one wavefront: the wave's
// LDS instructions execute in issue order, so only the compiler must be kept
// from moving accesses across this point.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Wave issue priority from progress: 3 for the first 40% of a block's
// iterations, 2 to 70%, 1 to 90% and 0 for the rest (shorter levels towards
// the end, where the order of finishing is set). A CU holds several blocks
// that all run the whole sequence; the issue arbiter favours the oldest waves
// at equal priority, so without this the blocks of a CU finish one after the
// other and the last one runs its final stretch alone, its latencies no
// longer hidden by other waves. A block ahead of the others drops below them
// and yields its issue slots until they catch up. (The wave's own
// arbitration priority only.)
//
// The levels change only at three iterations, computed once before the walk
// (iteration i has level 3 - #{k : i >= ceil(k n / 10), k = 4, 7, 9}): per
// iteration the walk pays one scalar compare, not a division and a chain of
// branches (scalar instructions take issue slots from the wave's VALU work).
struct ProgressPriority {
  int th[3];   // first iterations of levels 2, 1, 0
  int next;    // the next iteration at which the level changes
  __device__ __forceinline__ explicit ProgressPriority(int n) {
    n = max(n, 1);
    th[0] = (4 * n + 9) / 10;
    th[1] = (7 * n + 9) / 10;
    th[2] = (9 * n + 9) / 10;
    next = 0;
  }
  __device__ __forceinline__ void step(int i) {
    if (i != next) return;
    const int lvl = 3 - (i >= th[0]) - (i >= th[1]) - (i >= th[2]);
    switch (lvl) {
      case 3: __builtin_amdgcn_s_setprio(3); break;
      case 2: __builtin_amdgcn_s_setprio(2); break;
      case 1: __builtin_amdgcn_s_setprio(1); break;
      default: __builtin_amdgcn_s_setprio(0); break;
    }
    next = i < th[0] ? th[0] : i < th[1] ? th[1] : i < th[2] ? th[2] : 0x7FFFFFFF;
  }
};

// An opaque register copy. A loop-carried value that comes from a global
// load on some path into the loop (a state or parameter read before it) is
// copied once before the loop: the wait for the load is then placed at the
// copy, once, instead of at the value's first use inside the loop, where it
// would be repeated every iteration and, the counter being in order, would
// also wait for every later load or store still in flight.
__device__ __forceinline__ float opaque_copy(float v) {
  float r;
  asm volatile("v_mov_b32 %0, %1" : "=v"(r) : "v"(v));
  return r;
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

// ---------------------------------------------------------------- LDS tiles
//
// Time is processed in sub-chunks of 16 steps ("quads" of 4 steps). Per-lane
// operands live in channel-major tiles: row c holds the 16 steps of channel
// c, so a lane reads 4 consecutive steps with one 128-bit LDS read (gfx950
// moves ~2x the bytes per clock with ds_read_b128 than with b32/b64). The
// quad slot inside a row is m ^ c ^ (c >> 2) (mod 4): measured on gfx950,
// this makes both the 128-bit reads (lane c reads row c) and the 128-bit
// writes of such tiles free of bank conflicts, where a rotation by c/4 costs
// 8 conflict cycles per 128-bit write.
constexpr int kSteps = 16;   // steps per sub-chunk
constexpr int kQuads = 4;    // quads per sub-chunk

__device__ __forceinline__ int cm_quad(int row, int m) {
  return row * kSteps + (((m ^ row ^ (row >> 2)) & 3) << 2);
}
__device__ __forceinline__ int cm_elem(int row, int k) { return cm_quad(row, k >> 2) + (k & 3); }
// The padded channel-major layout: rows kCmRow = 20 floats apart (80 bytes:
// the 16 rows of any 16 consecutive lanes start on 16 distinct 4-bank
// groups), quads in order. A lane's four quads are then one base register
// plus immediates 0, 16, 32, 48 bytes, where the swizzle needs a register per
// quad (an address add per quad for each buffer switch).
constexpr int kCmRow = 20;
enum class CmLayout { kSwizzled, kPadded };
template <CmLayout L>
__device__ __forceinline__ int cml_quad(int row, int m) {
  if constexpr (L == CmLayout::kPadded) return row * kCmRow + 4 * m;
  else return cm_quad(row, m);
}
template <CmLayout L>
__device__ __forceinline__ int cml_elem(int row, int k) {
  if constexpr (L == CmLayout::kPadded) return row * kCmRow + k;
  else return cm_elem(row, k);
}
template <CmLayout L>
__host__ __device__ constexpr int cml_tile_floats(int ch) {
  return L == CmLayout::kPadded ? ch * kCmRow : ch * kSteps;
}

__device__ __forceinline__ float4 lds4(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ __forceinline__ float2 lds2(const float* p) { return *reinterpret_cast<const float2*>(p); }


// ------------------------------------------------------------- buffer I/O
//
// Global memory is accessed through raw buffer resources: an access whose
// byte offset is at or beyond the resource's size returns 0 (loads) or is
// dropped (stores) by the hardware. Edges (steps past T, channels past
// d_inner, padded states) therefore need no branches: their offsets are set
// to kOOB, and the hot loops stay single basic blocks.
constexpr unsigned kOOB = 0x80000000u;   // resources are < 2 GiB (checked on the host)

// Cache policy of a buffer access (the instruction's aux bits): kStream marks
// it non-temporal (NT), so that data used once streams through the caches
// without evicting the tiles that other blocks or later steps reuse.
constexpr int kStream = 2;

// Base and size must be wave-uniform; they are moved to SGPRs explicitly
// (readfirstlane), so that the compiler never has to wrap an access in a
// loop over the distinct descriptors of the wave. __builtin_amdgcn_readfirstlane
// moves 32 bits: the 64-bit base goes through it as two halves.
__device__ __forceinline__ float* uniform_ptr(const float* p) {
  const uint64_t v = reinterpret_cast<uintptr_t>(p);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
  return reinterpret_cast<float*>(((uint64_t)hi << 32) | lo);
}
struct GBuf {
  __amdgpu_buffer_rsrc_t r;
  __device__ __forceinline__ GBuf(const float* base, unsigned bytes)
      : r(__builtin_amdgcn_make_buffer_rsrc(uniform_ptr(base), 0,
                                            __builtin_amdgcn_readfirstlane((int)bytes), 0x00020000)) {}
  // The b32 builtins move raw 32-bit words (unsigned int): bit-cast, never convert.
  // POL is the cache policy (kStream: non-temporal, for data that is touched
  // once and must not evict what is reused).
  template <int POL = 0>
  __device__ __forceinline__ float ld(unsigned byte_off) const {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, POL));
  }
  template <int POL = 0>
  __device__ __forceinline__ void st(float v, unsigned byte_off) const {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, byte_off, 0, POL);
  }
  // fp32 atomic add at device (agent) scope, no return value
  // (buffer_atomic_add_f32 without glc; no cache-policy bits, as the compiler
  // emits for an agent-scope atomicrmw on gfx950). Out of range offsets are
  // dropped like stores.
  __device__ __forceinline__ void atomic_add(float v, unsigned byte_off) const {
    __builtin_amdgcn_raw_ptr_buffer_atomic_fadd_f32(v, r, byte_off, 0, 0);
  }
};

// Element storage of the (batch, T, D) and (batch, T, N) activations: fp32
// (ES = 4) or bf16 (ES = 2, the upper half of an fp32: loads widen exactly,
// stores round to nearest even). Arithmetic is fp32 either way; states,
// checkpoints and Aneg are always fp32.
__device__ __forceinline__ unsigned short f32_to_bf16(float v) {
  const unsigned u = __float_as_uint(v);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (unsigned short)((u >> 16) | 0x40u);   // quiet NaN
  return (unsigned short)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}
template <int ES, int POL = 0>
__device__ __forceinline__ float ld_elem(const GBuf& g, unsigned byte_off) {
  static_assert(ES == 4 || ES == 2, "fp32 or bf16 elements");
  if constexpr (ES == 4) {
    return g.ld<POL>(byte_off);
  } else {
    return __uint_as_float((unsigned)__builtin_amdgcn_raw_buffer_load_b16(g.r, byte_off, 0, POL)
                           << 16);
  }
}
template <int ES, int POL = 0>
__device__ __forceinline__ void st_elem(const GBuf& g, float v, unsigned byte_off) {
  if constexpr (ES == 4) {
    g.st<POL>(v, byte_off);
  } else {
    __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16(v), g.r, byte_off, 0, POL);
  }
}
// Element idx of an activation tensor of ES-byte elements, as the float
// pointer GBuf takes (a byte address; only GBuf dereferences it).
template <int ES>
__device__ __forceinline__ const float* elem_at(const void* base, size_t idx) {
  return reinterpret_cast<const float*>(static_cast<const char*>(base) + idx * ES);
}

// One (batch, T, ·) operand walked a chunk of `steps` steps at a time. The
// resource over chunk i covers its rows from column c0 (row stride ld, width
// columns): [p0 + i * step, + bytes(i)), with bytes the full chunk's, the
// short last chunk's (index ilast, last_len rows) or 0 for indices outside
// [lo, hi). The base is linear in i (no clamping: outside the range the
// resource is empty and never dereferenced), so that the compiler turns
// i * step into one 64-bit scalar add per operand and iteration instead of
// the 64-bit product (row0 + t0) * ld (scalar instructions take issue slots
// from the wave's VALU work).
template <int ES>
struct SubStream {
  const char* p0;
  size_t step;
  unsigned full, last;
  int lo, hi, ilast;
  __device__ __forceinline__ SubStream(const void* base, size_t row, int ld, int c0, int width,
                                       int steps, int lo_, int hi_, int ilast_, int last_len)
      : p0(static_cast<const char*>(base) + ((size_t)row * ld + c0) * ES),
        step((size_t)steps * ld * ES),
        full((unsigned)ES * (unsigned)((steps - 1) * ld + width - c0)),
        last((unsigned)ES * (unsigned)((last_len - 1) * ld + width - c0)),
        lo(lo_), hi(hi_), ilast(ilast_) {}
  __device__ __forceinline__ unsigned bytes(int i) const {
    return i < lo || i >= hi ? 0u : i == ilast ? last : full;
  }
  __device__ __forceinline__ const char* base(int i) const {
    return p0 + (ptrdiff_t)i * (ptrdiff_t)step;
  }
  __device__ __forceinline__ GBuf at(int i) const {
    return GBuf(reinterpret_cast<const float*>(base(i)), bytes(i));
  }
};

// A SubStream walked backwards one chunk per loop iteration: the current
// chunk's pointer, moved down by one step (a 64-bit scalar subtract) instead
// of recomputed from the index.
template <int ES>
struct StreamCursor {
  const char* p;
  int i;
  __device__ __forceinline__ StreamCursor(const SubStream<ES>& s, int i0) : p(s.base(i0)), i(i0) {}
  __device__ __forceinline__ GBuf get(const SubStream<ES>& s) const {
    return GBuf(reinterpret_cast<const float*>(p), s.bytes(i));
  }
  __device__ __forceinline__ void down(const SubStream<ES>& s) {
    p -= s.step;
    --i;
  }
};

// NPL consecutive states of one lane at byte offset `off` (kOOB: none);
// states at or beyond `nvalid` are padding and are not stored. Register j
// holds state j ^ sw of the lane's group (sw: 0, or 1 for a lane that keeps
// its two states in swapped order; see the backward's channel sums).
template <int NPL, int POL = 0>
__device__ __forceinline__ void store_states(const GBuf& g, unsigned off, int nvalid,
                                             const float (&v)[NPL], int sw = 0) {
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    const int n = j ^ sw;
    g.st<POL>(v[j], (off != kOOB && n < nvalid) ? off + 4u * n : kOOB);
  }
}
template <int NPL, int POL = 0>
__device__ __forceinline__ void load_states(float (&v)[NPL], const GBuf& g, unsigned off,
                                            int nvalid, int sw = 0) {
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    const int n = j ^ sw;
    v[j] = g.ld<POL>((off != kOOB && n < nvalid) ? off + 4u * n : kOOB);
  }
}

__device__ __forceinline__ void sts4(float* p, float4 v) { *reinterpret_cast<float4*>(p) = v; }

// Marks loaded registers as used here, without an instruction: the wait for
// their loads is placed at this point on every path, also on the paths where
// a branch skipped their real use (threads without a staging task), rather
// than at a later reuse of the registers, where the in-order counter would
// make it wait for every later load or store in flight as well.
__device__ __forceinline__ void consume(const float4& v) {
  asm volatile("" ::"v"(v.x), "v"(v.y), "v"(v.z), "v"(v.w));
}

// Staging of one sub-chunk of a (batch, T, D) tensor for the block's CH
// channels: task (c, quad m) holds steps 4m..4m+3 of channel d0+c. Tasks are
// numbered c-fastest so that each load instruction reads consecutive
// channels. Thread tid owns tasks tid, tid+nthreads, ... (PER of them; tasks
// beyond TASKS and channels beyond d_inner load zeros).
template <int CH, int PER, int ES = 4>
struct QuadLoader {
  static constexpr int TASKS = CH * kQuads;
  int tid, nthreads;
  int w0;               // the wave's first thread index (wave-uniform)
  unsigned rs;          // row (time step) stride in bytes
  unsigned toff[PER];   // byte offset of step 4m of channel c from the sub-chunk base, or kOOB
  // D: channels; ld: elements between consecutive time steps (>= D; D for a
  // contiguous (batch, T, D) tensor, more for a column slice of a wider one).
  __device__ __forceinline__ QuadLoader(int tid_, int nthreads_, int D, int d0, int ld)
      : tid(tid_), nthreads(nthreads_), w0(__builtin_amdgcn_readfirstlane(tid_) & ~63),
        rs((unsigned)ES * (unsigned)ld) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int e = tid + i * nthreads;
      const int c = e % CH, m = e / CH;
      toff[i] = (e < TASKS && d0 + c < D)
                    ? (unsigned)ES * ((unsigned)(4 * m) * (unsigned)ld + (unsigned)c)
                    : kOOB;
    }
  }
  // Whether task i of this thread exists. With whole waves of tasks (TASKS a
  // multiple of 64, as nthreads is) it is the same for every lane of a wave,
  // and the test reads the wave's first thread index from an SGPR: a scalar
  // branch around the LDS store instead of an exec-mask save and restore.
  __device__ __forceinline__ bool valid(int i) const {
    if ((i + 1) * nthreads <= TASKS) return true;
    if constexpr (TASKS % 64 == 0) {
      return w0 + i * nthreads < TASKS;
    } else {
      return tid + i * nthreads < TASKS;
    }
  }
  __device__ __forceinline__ int chan(int i) const { return (tid + i * nthreads) % CH; }
  __device__ __forceinline__ int quad(int i) const { return (tid + i * nthreads) / CH; }
  // g covers (b, t0.., d0..) up to the end of the batch row (steps past T
  // are out of range).
  template <int POL = 0>
  __device__ __forceinline__ void load(float4 (&v)[PER], const GBuf& g) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const unsigned o = toff[i];
      const bool ok = o != kOOB;
      v[i].x = ld_elem<ES, POL>(g, o);
      v[i].y = ld_elem<ES, POL>(g, ok ? o + rs : kOOB);
      v[i].z = ld_elem<ES, POL>(g, ok ? o + 2 * rs : kOOB);
      v[i].w = ld_elem<ES, POL>(g, ok ? o + 3 * rs : kOOB);
    }
  }
  // Per task, the element of a per-channel vector (the dt gate's bias) for
  // its channel d0 + chan(i); 0 for tasks past the tile, channels past
  // d_inner, or no vector.
  __device__ __forceinline__ void load_channel(float (&v)[PER], const float* vec, int d0) const {
#pragma unroll
    for (int i = 0; i < PER; ++i)
      v[i] = (vec != nullptr && toff[i] != kOOB) ? vec[d0 + chan(i)] : 0.f;
  }
  // Gate staged dt values in place: dt = lo + span * sigmoid(raw + bias) for
  // the steps below len (bias: the task's channel bias, see load_channel);
  // steps at or past len (and channels past d_inner) get dt = 0, which makes
  // them identity steps of the recurrence, as the zeros an ungated load
  // returns there.
  __device__ __forceinline__ void gate(float4 (&v)[PER], int len, float lo, float span,
                                       const float (&bias)[PER]) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int s0 = toff[i] != kOOB ? 4 * quad(i) : kSteps;
      v[i].x = s0 < len ? gate_dt(v[i].x + bias[i], lo, span) : 0.f;
      v[i].y = s0 + 1 < len ? gate_dt(v[i].y + bias[i], lo, span) : 0.f;
      v[i].z = s0 + 2 < len ? gate_dt(v[i].z + bias[i], lo, span) : 0.f;
      v[i].w = s0 + 3 < len ? gate_dt(v[i].w + bias[i], lo, span) : 0.f;
    }
  }
  // Channel-major tile [CH][16] (swizzled) or [CH][kCmRow] (padded).
  template <CmLayout L = CmLayout::kSwizzled>
  __device__ __forceinline__ void store_cm(float* tile, const float4 (&v)[PER]) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      if (valid(i)) sts4(tile + cml_quad<L>(chan(i), quad(i)), v[i]);
      consume(v[i]);
    }
  }
  template <CmLayout L = CmLayout::kSwizzled>
  __device__ __forceinline__ void store_cm_product(float* tile, const float4 (&a)[PER],
                                                   const float4 (&b)[PER]) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      if (valid(i))
        sts4(tile + cml_quad<L>(chan(i), quad(i)),
             make_float4(a[i].x * b[i].x, a[i].y * b[i].y, a[i].z * b[i].z, a[i].w * b[i].w));
      consume(a[i]);
      consume(b[i]);
    }
  }
  // Step-major tile [16][CH] (consecutive channels contiguous).
  __device__ __forceinline__ void store_sm(float* tile, const float4 (&v)[PER]) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      if (!valid(i)) continue;
      float* p = tile + 4 * quad(i) * CH + chan(i);
      p[0] = v[i].x;
      p[CH] = v[i].y;
      p[2 * CH] = v[i].z;
      p[3 * CH] = v[i].w;
    }
  }
  __device__ __forceinline__ void store_sm_product(float* tile, const float4 (&a)[PER],
                                                   const float4 (&b)[PER]) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      if (!valid(i)) continue;
      float* p = tile + 4 * quad(i) * CH + chan(i);
      p[0] = a[i].x * b[i].x;
      p[CH] = a[i].y * b[i].y;
      p[2 * CH] = a[i].z * b[i].z;
      p[3 * CH] = a[i].w * b[i].w;
    }
  }
};

// B / C tiles in LDS: per state group q (NPL states), the 16 steps x NPL
// states of the group, [16][NPL], followed by kBCPad floats of padding. The
// padding puts the two half-waves' groups (read at the same instant, each
// half-wave broadcasting one address) 16 bytes apart modulo the bank width
// instead of on the same banks, and keeps consecutive staging slots on
// consecutive banks across a group boundary.
constexpr int kBCPad = 4;
__host__ __device__ constexpr int bc_group_floats(int NPL) { return kSteps * NPL + kBCPad; }
// A B or C tile of NQ state groups.
__host__ __device__ constexpr int bc_tile_floats(int NQ, int NPL) {
  return NQ * bc_group_floats(NPL);
}

// Staging of 16 rows of a (batch, T, N) tensor (B or C) into an LDS tile of
// NP >= N (padded) states laid out per state group (see bc_group_floats):
// group q reads NPL states of 4 steps as NPL float4s at
// q*bc_group_floats(NPL) + 4*m*NPL. Thread tid moves tile elements tid,
// tid+nthreads, ... (PERS of them), state fastest, so that a wave's loads
// read whole rows; with the groups' padding the states of one step then fall
// on distinct banks (SQ_LDS_BANK_CONFLICT reads 0 for the forward at
// 16x512x1536x16; unpadded, the 16 states of a step shared two banks).
// Padded states and steps past T are zero.
template <int PERS, int NPL, int ES = 4>
struct RowLoader {
  unsigned src[PERS];  // byte offset in the sub-chunk's global [16][ld] block, or kOOB
  int dst[PERS];       // slot in the tile, or -1
  int tid, nthreads, ntile;
  int w0;              // the wave's first thread index (wave-uniform)
  // ld: elements between consecutive time steps (>= N).
  __device__ __forceinline__ RowLoader(int tid_, int nthreads_, int N, int NP, int ld)
      : tid(tid_), nthreads(nthreads_), ntile(kSteps * NP),
        w0(__builtin_amdgcn_readfirstlane(tid_) & ~63) {
#pragma unroll
    for (int i = 0; i < PERS; ++i) {
      const int e = tid + i * nthreads;       // tile element (k, n), n fastest
      const int k = e / NP, n = e % NP;
      const bool in_tile = e < kSteps * NP;
      src[i] = (in_tile && n < N) ? (unsigned)ES * (unsigned)(k * ld + n) : kOOB;
      dst[i] = in_tile ? (n / NPL) * bc_group_floats(NPL) + k * NPL + (n % NPL) : -1;
    }
  }
  __device__ __forceinline__ void load(float (&v)[PERS], const GBuf& g) const {
#pragma unroll
    for (int i = 0; i < PERS; ++i) v[i] = ld_elem<ES>(g, src[i]);
  }
  __device__ __forceinline__ void store(float* tile, const float (&v)[PERS]) const {
#pragma unroll
    for (int i = 0; i < PERS; ++i) {
      if (valid(i)) tile[dst[i]] = v[i];
      asm volatile("" ::"v"(v[i]));   // as consume(): the wait happens here on every path
    }
  }
  // Whether element i of this thread lies in the tile (dst[i] >= 0): true
  // at compile time when the threads cover the tile exactly, else a scalar
  // test of the wave's first thread index when the tile is whole waves.
  __device__ __forceinline__ bool valid(int i) const {
    if ((i + 1) * nthreads <= ntile) return true;
    if (ntile % 64 == 0) return w0 + i * nthreads < ntile;
    return dst[i] >= 0;
  }
};

// Broadcast tiles of B and C for two states per lane: per state group q
// and quad m, 16 floats (the group's 2 states x 4 steps x {B, C}). Two
// layouts:
// * kRow (the forward's row broadcasts): [kind][k % 4][n % 2], one float
//   per lane of a 16-lane row; groups kBCGroup2 floats apart (16 banks),
//   so that the two half-waves' groups fall on disjoint banks;
// * kQuad (the backward's quad broadcasts): [kind][(k % 2) * 2 + n % 2][(k
//   % 4) / 2], so that lane p of a quad reads 2 floats of B and 2 of C with
//   two 64-bit loads and holds B (then C) of steps 4m + (p >> 1) and 4m + 2
//   + (p >> 1), each of state n0 + (p & 1) (qp_get); groups kBCGroupQ
//   floats apart (8 banks): the staging writes of a wave (8 groups x 8
//   contiguous floats) then hit 64 distinct banks and the half-waves' reads
//   disjoint ones.
constexpr int kBCGroup2 = kQuads * 16 + 16;
constexpr int kBCGroupQ = kQuads * 16 + 8;
enum class BCLayout { kRow, kQuad };

// Staging of 16 rows of B and C (fp32 or bf16, rows ld apart) into such a
// tile: thread tid moves tile elements tid, tid + nthreads, ... (PERS of
// them), state fastest, of both B and C. Padded states and steps past T are
// zero.
template <int PERS, int ES = 4, BCLayout L = BCLayout::kRow>
struct BCRowLoader {
  unsigned src[PERS];  // byte offset in the sub-chunk's global [16][ld] block, or kOOB
  int dst[PERS];       // B's slot in the tile (C's is 8 further), or -1
  int tid, nthreads, ntile;
  int w0;
  static constexpr int kGroup = L == BCLayout::kRow ? kBCGroup2 : kBCGroupQ;
  __device__ __forceinline__ BCRowLoader(int tid_, int nthreads_, int N, int NP, int ld)
      : tid(tid_), nthreads(nthreads_), ntile(kSteps * NP),
        w0(__builtin_amdgcn_readfirstlane(tid_) & ~63) {
#pragma unroll
    for (int i = 0; i < PERS; ++i) {
      const int e = tid + i * nthreads;       // tile element (k, n), n fastest
      const int k = e / NP, n = e % NP;
      const bool in_tile = e < kSteps * NP;
      src[i] = (in_tile && n < N) ? (unsigned)ES * (unsigned)(k * ld + n) : kOOB;
      const int in_quad = L == BCLayout::kRow ? (k % 4) * 2 + (n % 2)
                                              : ((k % 2) * 2 + (n % 2)) * 2 + (k % 4) / 2;
      dst[i] = in_tile ? (n / 2) * kGroup + (k / 4) * 16 + in_quad : -1;
    }
  }
  __device__ __forceinline__ void load(float (&v)[PERS], const GBuf& g) const {
#pragma unroll
    for (int i = 0; i < PERS; ++i) v[i] = ld_elem<ES>(g, src[i]);
  }
  __device__ __forceinline__ bool valid(int i) const {
    if ((i + 1) * nthreads <= ntile) return true;
    if (ntile % 64 == 0) return w0 + i * nthreads < ntile;
    return dst[i] >= 0;
  }
  // kind 0 (B) or 1 (C)
  __device__ __forceinline__ void store(float* tile, const float (&v)[PERS], int kind) const {
#pragma unroll
    for (int i = 0; i < PERS; ++i) {
      if (valid(i)) tile[dst[i] + 8 * kind] = v[i];
      asm volatile("" ::"v"(v[i]));
    }
  }
};

// Quad broadcasts from a kQuad tile. Lane p of a quad holding its two states
// in swapped order when p is odd (register j: state n0 + (j ^ (p & 1))), the
// value of step 4m + s, register j, is in the quad's B (or C) register
// (s >> 1) of lane ((s & 1) << 1) | (j ^ (p & 1)): sel = (s & 1) * 2
// + j picks one of four quad_perm patterns, [0,1,0,1], [1,0,1,0], [2,3,2,3]
// and [3,2,3,2]. With sel a constant after unrolling, each switch below
// folds to one case.
__host__ __device__ constexpr int qp_sel(int s, int j) { return (s & 1) * 2 + j; }
// The broadcast value itself (the compiler folds the DPP read into the
// multiply that uses it: v_mul_f32_dpp).
__device__ __forceinline__ float qp_get(float r, int sel) {
  switch (sel) {
    case 0: return dpp_get<0x44>(r);
    case 1: return dpp_get<0x11>(r);
    case 2: return dpp_get<0xEE>(r);
    default: return dpp_get<0xBB>(r);
  }
}
// acc += (the broadcast value of r) * x, one v_fmac_f32_dpp (the compiler
// does not fold a DPP read into v_fmac). r must come from an LDS load, not
// from a VALU instruction: a DPP read of a VGPR needs 2 wait states after a
// VALU write of it, which the compiler does not check inside the asm
// (build.py's dpp_hazards rejects compiled assembly where it fails).
__device__ __forceinline__ void qp_fmac(float& acc, float r, float x, int sel) {
  switch (sel) {
    case 0:
      asm("v_fmac_f32_dpp %0, %1, %2 quad_perm:[0,1,0,1] row_mask:0xf bank_mask:0xf"
          : "+v"(acc) : "v"(r), "v"(x));
      break;
    case 1:
      asm("v_fmac_f32_dpp %0, %1, %2 quad_perm:[1,0,1,0] row_mask:0xf bank_mask:0xf"
          : "+v"(acc) : "v"(r), "v"(x));
      break;
    case 2:
      asm("v_fmac_f32_dpp %0, %1, %2 quad_perm:[2,3,2,3] row_mask:0xf bank_mask:0xf"
          : "+v"(acc) : "v"(r), "v"(x));
      break;
    default:
      asm("v_fmac_f32_dpp %0, %1, %2 quad_perm:[3,2,3,2] row_mask:0xf bank_mask:0xf"
          : "+v"(acc) : "v"(r), "v"(x));
      break;
  }
}

// NPL states x 4 steps of a group's B or C tile: v[s][j] = tile[(4m+s)*NPL + j].
template <int NPL>
__device__ __forceinline__ void load_quad_rows(float (&v)[4][NPL], const float* g, int m) {
  const float* p = g + 4 * m * NPL;
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    const float4 t = lds4(p + 4 * i);
    const float tv[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) v[(4 * i + e) / NPL][(4 * i + e) % NPL] = tv[e];
  }
}

__device__ __forceinline__ void f4_to(float (&v)[4], float4 t) {
  v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
}

}  // namespace mhs
