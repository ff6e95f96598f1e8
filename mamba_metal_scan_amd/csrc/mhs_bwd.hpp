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
// MI355X mapping. Same block decomposition as the forward (32 channels x one
// batch row per block; lane = (wave, half, channel), NPL states per lane,
// d_state padded with zero states to NP = 2*G*NPL). Chunks of K <= 16 steps
// are walked last to first. Each chunk takes two phases and two barriers:
//   recompute: every lane rebuilds its chunk of dA and h from the checkpoint
//     into VGPRs (da[16][NPL], hs[16][NPL]; nothing goes to global scratch):
//     all dA and inputs b = B*dt*x first (independent), then the short chain
//     h = dA*h + b. In the same straight-line code the waves also finish the
//     previous (later-in-time) chunk: dx, ddt from the per-wave sums and the
//     x, dt tiles still in that chunk's LDS buffer, and the dB/dC block sums.
//   reverse: walks the chunk backwards carrying G in VGPRs across chunk
//     boundaries, with hm = dA * h_{t-1} from the recomputed chunk (no
//     h_t - b_t cancellation). In the same code the waves store the staged
//     inputs of the next chunk into the other LDS buffer (free once the
//     previous chunk is finished) and issue the global loads of the chunk
//     after that. All global accesses are bounds-checked buffer accesses
//     whose resources end at the chunk's last step, so chunk and tensor edges
//     need no branches.
// Steps k >= len of a chunk (K < 16, or the tail of the sequence) see zero
// inputs: dA = 1 and b = 0 there, so they are identity steps for h and G, add
// zero to every accumulated gradient, and their outputs are not written.
//   dx / ddt: per lane s1 = sum G*B, s2 = sum Aneg*G*hm over its NPL states.
//             The two half-waves (same channels, different states) are added
//             with one v_permlane32_swap (lanes 0-31 keep s1, 32-63 s2); the
//             per-wave values go to LDS and, in the next chunk's recompute
//             phase, are summed over the G waves in a fixed order and written
//             once, coalesced.
//   dAneg:    accumulated per lane over the whole walk, written once per
//             (b, d, n) to a workspace slot.
//   dB / dC:  sums over the block's 32 channels, i.e. over the 32 lanes of a
//             half-wave. Every two steps each lane forms its 4*NPL products
//             G*(dt*x) and h*dy and the wave sums them over its half-waves
//             with a register-only reduce-scatter (v_permlane16_swap, then
//             DPP stages): no LDS round trip, and each lane ends with one
//             total, which goes to the chunk's LDS tile of block sums. These
//             are copied to a workspace slot; bwd_reduce_kernel adds the
//             blocks in a fixed order, so the backward is bit-for-bit
//             reproducible.
#pragma once

#include "mhs_common.hpp"
#include "mhs_fwd.hpp"

namespace mhs {

struct BwdArgs {
  // x, dt, B, C, dy, dx, ddt: ES-byte elements (fp32 or bf16, see the
  // kernel's ES); everything else fp32.
  const void* x;
  const void* dt;
  const float* aneg;
  const void* B;
  const void* C;
  const void* dy;
  const float* dh_last;  // may be null
  const float* ckpt;     // (batch, nchunk, D, N), stride K
  void* dx;
  void* ddt;
  float* wsB;            // (nblk, batch, T, N)
  float* wsC;            // (nblk, batch, T, N)
  float* wsA;            // (batch, D, N)
  int batch, T, D, N, K, nchunk;
  // Gated kernels only (GATED): dt holds the raw gate input and aneg holds A
  // (dt = dt_lo + dt_span * sigmoid(raw + dt_bias[d]), Aneg = softplus(A);
  // mamba_metal/model.py:197, :200), and ddt receives the gradient of the raw
  // input. dt_bias may be null. wsDB (nseg, batch, D), if not null, receives
  // per block the sum over its steps of that gradient: the bias gradient's
  // partials.
  float dt_lo, dt_span, dt_inv_span;
  const float* dt_bias;
  float* wsDB;
  // Time segments (the chunk-parallel-over-time variant): the chunks split
  // into nseg segments of cps chunks, one block per (channel block, batch
  // row, segment), blockIdx.y = seg * batch + b. The carry pass (CARRY) runs
  // over carry units of cps / cunits chunks (cunits per segment: a grid with
  // enough blocks to hide its dependent chains), launched with cps = the
  // unit's chunks and one block per unit of segments 1..nseg-1. With
  // nseg > 1:
  //   carryL   (nunits, batch, D, N): slot u >= cunits holds L_u = dA_a * G_a
  //            of unit u walked from a zero adjoint (a = its first step);
  //   carrySdt (nunits, batch, D):    slot u >= cunits holds sum dt over unit u.
  // The adjoint entering segment s from the later ones is then folded from
  // the last unit down to the first unit after segment s:
  //   K = dh_last (or 0);  K <- L_u + exp(-Aneg * Sdt_u) * K.
  int nseg, cps;
  float* carryL;
  float* carrySdt;
  int cunits = 1, nunits = 0;
  // In-kernel sweep kernels only (SWEEP > 0): ckpt holds the caller's
  // checkpoints at stride km x 16 steps (ck_nchunk of them per batch row),
  // K is 16 and nchunk counts 16-step chunks.
  int km = 1, ck_nchunk = 0;
  // Row strides (elements between consecutive time steps) of dt, of B and C,
  // and of ddt: D, N and D for contiguous tensors, more for column slices of
  // a wider projection output (and its gradient). x, dy, dx are contiguous.
  int ld_dt, ld_bc, ld_ddt;
  // Atomic kernels only (ATOM): the fp32 gradients the blocks add into with
  // fp32 atomics instead of writing partials (wsB, wsC, wsA, wsDB unused),
  // zeroed beforehand: dB, dC (rows ld_dbc apart), dAneg (or the gated
  // kernels' dA), the gated kernels' dt-bias gradient (may be null).
  float* dB = nullptr;
  float* dC = nullptr;
  float* daneg = nullptr;
  float* dbias = nullptr;
  int ld_dbc = 0;
};

// Largest number of 16-step chunks per caller checkpoint that the backward
// sweeps inside the kernel (checkpoint stride 32 steps); larger strides
// recompute stride-16 checkpoints in a separate pass. From three windows on
// the separate pass is the faster (backward launch at 16x512x1536x16, chunk
// 48: 153.2 against 155.0 us, chunk 64: 154.2 against 158.7 us; at
// 4x16384x2048x16 1793 against 1827 and 1800 against 1881 us), at two the
// sweep (149.9 against 154.0 us, 1763 against 1797 us).
constexpr int kSweepMax = 2;

// Channel sums of the two-state plans' gradient kernels (RL): the lanes of
// odd channel hold their two states in swapped order, and the dB / dC
// products are summed over each 16-lane row in registers (pair_sum_xor1, then
// row_partial_pairs: each lane reads its partner channel's dt * x and dy too).
// Such kernels stage B and C in a quad broadcast tile (BCLayout::kQuad, two
// 64-bit reads per lane and quad) and take each value from the right lane of
// the quad with quad_perm DPP (qp_get, qp_fmac), which serves both state
// orders. The two rows of a half-wave are then added in the finishing step
// (RP: the kernels without the in-kernel sweep, which keep two row partials per block
// sum: tile [row][kind][16 steps][rp_step_floats], the kinds rp_kind_floats
// apart and the rows twice that, so that the 32 lanes of a half-wave that
// write one step pair's partials hit 32 distinct banks), or in registers by one more
// v_permlane16_swap stage (the swept kernels, whose LDS, with the sweep's
// state slots, has no room for the partials). Both add the two rows in the
// same order, so every checkpoint stride gives the same sums.
__host__ __device__ constexpr int rp_step_floats(int NP) { return NP <= 16 ? 16 : 48; }
__host__ __device__ constexpr int rp_kind_floats(int NP) {
  return kSteps * rp_step_floats(NP) + 4;
}
__host__ __device__ constexpr bool bwd_relabel(int NPL, bool CARRY) { return NPL == 2 && !CARRY; }
__host__ __device__ constexpr bool bwd_row_partial(int NPL, bool CARRY, int SWEEP) {
  return bwd_relabel(NPL, CARRY) && SWEEP == 0;
}

// The layout of the backward's channel-major tiles (dt, dy, x, dt*x): padded
// in the gradient kernels, whose walk switches staging buffers every chunk
// (one address add per tile row and switch, not per quad); swizzled in the
// adjoint-carry pass, whose occupancy its LDS sets (4 blocks per CU at d_state
// 16, 3 with the padding).
__host__ __device__ constexpr CmLayout bwd_cm(bool carry) {
  return carry ? CmLayout::kSwizzled : CmLayout::kPadded;
}

// One staging buffer (the kernel keeps two) and the single-buffered rest.
__host__ __device__ constexpr int bwd_buf_floats(int G, int NPL, bool rl, bool carry) {
  return 4 * (carry ? cml_tile_floats<CmLayout::kSwizzled>(kCH)
                    : cml_tile_floats<CmLayout::kPadded>(kCH))   // dt, dy, x, dt*x
         + (rl ? 2 * G * kBCGroupQ      // B, C quad broadcast tile
               : 2 * bc_tile_floats(2 * G, NPL));   // B, C tiles
}
__host__ __device__ constexpr int bwd_lds_floats(int G, int NPL, bool rl, bool rp, bool carry) {
  return 2 * bwd_buf_floats(G, NPL, rl, carry)
         + G * 64 * kSteps                       // (s1, s2) per wave
         + (rp ? 4 * rp_kind_floats(2 * G * NPL)  // dB, dC row partials of a chunk
               : 2 * kSteps * 2 * G * NPL);      // dB, dC block sums of a chunk
}
// The swept kernels (SWEEP > 0) keep each lane's swept states in LDS after
// that: kSweepMax slots of NPL floats per thread, [slot][thread][NPL].
__host__ __device__ constexpr int bwd_sweep_lds_floats(int G, int NPL) {
  return bwd_lds_floats(G, NPL, bwd_relabel(NPL, false), false, false) + kSweepMax * 64 * G * NPL;
}

// GATED: see BwdArgs. The staging threads gate each dt once per block as they
// move it to LDS; finalize turns ddt into the raw input's gradient
// ddt * span * s * (1 - s), s = sigmoid(raw) = (dt - lo) / span.
// CARRY: the adjoint-carry pass of the time segments (see BwdArgs): blocks of
// segments 1..nseg-1 walk their segment backwards carrying only the adjoint
// (dA and G, no state, no gradients, no x or B traffic) and write L_s and
// the segment's sum of dt.
// ES: bytes per element of x, dt, B, C, dy, dx, ddt (4: fp32, 2: bf16).
// ATOM: the block sums of dB and dC, each lane's dAneg and the block's
// dt-bias sums are added into zeroed fp32 gradients with fp32 atomics (no
// partials, no reduction kernel; the order of the additions, and so the
// rounding, varies from run to run). For bf16 activations dB and dC go to
// fp32 buffers that a later pass rounds to bf16.
template <int NPL, int G, int MINW, bool GATED, bool CARRY, int ES = 4, bool ATOM = false,
          int SWEEP = 0>
__global__ void __launch_bounds__(64 * G, MINW)
bwd_kernel(BwdArgs a) {
  constexpr int NT = 64 * G;
  constexpr int NP = 2 * G * NPL;
  constexpr bool RL = bwd_relabel(NPL, CARRY);
  constexpr bool RP = bwd_row_partial(NPL, CARRY, SWEEP);
  constexpr int BUF = bwd_buf_floats(G, NPL, RL, CARRY);
  constexpr CmLayout kBwdCm = bwd_cm(CARRY);
  constexpr int kBwdCmTile = cml_tile_floats<kBwdCm>(kCH);
  constexpr int PER = (kCH * kQuads + NT - 1) / NT;
  constexpr int PERS = (kSteps * NP + NT - 1) / NT;
  constexpr int FT = (kSteps / 2 * kCH + NT - 1) / NT;      // dx/ddt tasks per thread
  constexpr int FK = (kSteps * NP + NT - 1) / NT;           // dB (or dC) copies per thread
  // One state per lane gives a tile of kSteps * NP = NT / 2 sums: half the
  // threads copy one each. Two or four: every thread copies FK.
  constexpr bool kFKExact = FK * NT == kSteps * NP;
  constexpr int M = 4 * NPL;            // dB/dC products per lane per two steps
  static_assert(NPL == 1 || NPL == 2 || NPL == 4, "one, two or four states per lane");
  static_assert(!ATOM || !CARRY, "atomics: gradient pass only");

  extern __shared__ float lds[];
  const int N = a.N;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int hh = lane >> 5;
  const int c = lane & 31;
  const int q = wave * 2 + hh;
  const int n0 = q * NPL;
  // RL: lanes of odd channel hold their two states in swapped order
  // (register j holds state n0 + (j ^ sw)); memory layouts are unchanged.
  const int sw = RL ? (lane & 1) : 0;
  const int b = blockIdx.y % a.batch;
  const int seg = blockIdx.y / a.batch + (CARRY ? a.cunits : 0);   // CARRY: the unit
  const int d0 = blockIdx.x * kCH;
  const int d = d0 + c;
  const bool act = d < a.D;
  const int T = a.T, D = a.D, K = a.K;
  const int nvalid = N - n0;
  const int nch = a.nchunk;
  const int c_lo = seg * a.cps;                      // this block's chunks [c_lo, c_hi)
  const int c_hi = min(c_lo + a.cps, nch);

  constexpr int RPS = rp_step_floats(NP), RPK = rp_kind_floats(NP);
  // LDS: the (s1, s2) tile tS at 0 (its finishing-step reads then take their
  // offsets from one loop-invariant register: read2's 8-bit fields reach the
  // four waves' partials), the dB / dC tile tDBC, then the two staging
  // buffers (sbuf).
  float* tS = lds;                                    // [8 pairs][G][64][2]
  float* tDBC = tS + G * 64 * kSteps;                 // [2][16][NP], RP: [2][2][16][RPS]
  float* sbuf = tDBC + (RP ? 4 * RPK : 2 * kSteps * NP);
  // Staging buffer j: dt, dy, x (channel-major), B, C (per lane group; with
  // RL one quad broadcast tile of both, at oB).
  constexpr int oDY = kBwdCmTile, oX = 2 * kBwdCmTile, oDTX = 3 * kBwdCmTile,
                oB = 4 * kBwdCmTile, oC = oB + bc_tile_floats(2 * G, NPL);
  // The reduce-scatter leaves lane `lane` with the total of product rs_index:
  // products are numbered kind * 2NPL + slot * NPL + j (kind 0: dB, 1: dC;
  // slot: step k + slot; j: state n0 + j of this half-wave's group). With RL
  // it leaves the sum over the lane's 16-lane row (RP), or over its
  // half-wave, of product (kind (lane >> 3) & 1, slot (lane >> 2) & 1, state
  // n0 + (lane & 1)).
  const int rs = rs_index<M>(lane);
  const int rs_kind = RL ? (lane >> 3) & 1 : rs / (2 * NPL);
  const int rs_slot = RL ? (lane >> 2) & 1 : (rs / NPL) & 1;
  const int rs_n = RL ? (lane & 1) : rs % NPL;
  float* const dbc_out =
      RP ? tDBC + ((lane >> 4) & 1) * 2 * RPK + rs_kind * RPK + rs_slot * RPS + n0 + rs_n
         : tDBC + rs_kind * kSteps * NP + rs_slot * NP + n0 + rs_n;
  constexpr int kDbcStep = RP ? RPS : NP;   // dbc_out's stride per step
  // The dB / dC products of a step pair summed as dbc_out holds them: from
  // the products pv (numbered as for rs_index) or, with RL, from their
  // bit-0 pair sums pa (kind * 2 + slot, pair_sum_xor1).
  auto channel_sums = [&](const float (&pv)[M], const float (&pa)[4]) {
    if constexpr (RP) {
      return row_partial_pairs(pa);
    } else if constexpr (RL) {
      // the two rows of the half-wave added in registers (row 0's first)
      const float r = row_partial_pairs(pa);
      const auto sw16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(r), __float_as_uint(r),
                                                         false, false);
      return __uint_as_float(sw16[0]) + __uint_as_float(sw16[1]);
    } else {
      return half_wave_reduce_scatter<M>(pv, lane);
    }
  };
  // RL: the partner channel's row of the channel-major tiles (its dt * x and
  // dy for pair_sum_xor1).
  const int cp = c ^ 1;

  const size_t slice = (size_t)D * N;
  const unsigned slice_bytes = 4u * (unsigned)slice;
  const unsigned st_lane = act ? 4u * ((unsigned)d * (unsigned)N + (unsigned)n0) : kOOB;
  // u = dA_{t+1} * G_{t+1}, the adjoint already decayed into step t: the walk
  // carries u, so that G_t = dy_t C_t + u and dA_t h_{t-1} G_t = u_t h_{t-1}
  // each take one operation.
  float an[NPL], a2[NPL], u[NPL], acc[NPL];
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    const int nj = j ^ sw;
    an[j] = (act && nj < nvalid) ? a.aneg[(size_t)d * N + n0 + nj] : 0.f;
    if constexpr (GATED) an[j] = (act && nj < nvalid) ? softplus_f(an[j]) : 0.f;
    a2[j] = -an[j] * kLog2e;
    acc[j] = 0.f;
    u[j] = 0.f;
  }
  if constexpr (!CARRY) {
    // The adjoint entering this segment: dh_last for the last one, folded
    // with the carries of the later segments for the others.
    const float* dhl = a.dh_last != nullptr ? a.dh_last + (size_t)b * slice : a.aneg;
    load_states<NPL>(u, GBuf(dhl, a.dh_last != nullptr ? slice_bytes : 0u), st_lane, nvalid,
                     sw);
    for (int s2 = a.nunits - 1; s2 >= (seg + 1) * a.cunits; --s2) {
      float lv[NPL];
      const size_t slot = (size_t)s2 * a.batch + b;
      load_states<NPL>(lv, GBuf(a.carryL + slot * slice, slice_bytes), st_lane, nvalid, sw);
      const float sdt = act ? a.carrySdt[slot * D + d] : 0.f;
#pragma unroll
      for (int j = 0; j < NPL; ++j) u[j] = __builtin_fmaf(exp2_hw(sdt * a2[j]), u[j], lv[j]);
    }
  }
  // u (dh_last) and Aneg come from loads before the walk.
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    u[j] = opaque_copy(u[j]);
    an[j] = opaque_copy(an[j]);
  }
  // CARRY: the sum of dt over the segment, per staging task (the dt of 4
  // steps of one channel as staged), added over the channels' tasks at the
  // end: a quarter of the adds that every lane summing its steps would take.
  float sdt_part = 0.f;

  const size_t row0 = (size_t)b * T;
  // Only the gated kernels read dt, B, C from (and write ddt into) column
  // slices of wider tensors; the others keep compile-time-contiguous
  // addressing.
  const int ld_dt = GATED ? a.ld_dt : D, ld_bc = GATED ? a.ld_bc : N;
  const int ld_ddt = GATED ? a.ld_ddt : D;
  const QuadLoader<kCH, PER, ES> ql(tid, NT, D, d0, D);
  const QuadLoader<kCH, PER, ES> qdt(tid, NT, D, d0, ld_dt);
  const RowLoader<PERS, NPL, ES> rl(tid, NT, N, NP, ld_bc);
  const BCRowLoader<PERS, ES, BCLayout::kQuad> rlq(tid, NT, N, NP, ld_bc);   // RL: stores
  float4 px[PER], pd[PER], py[PER];
  float pb[PERS], pc[PERS], ph[NPL];
  float gbias[PER];   // GATED: the dt bias of each staging task's channel
  if constexpr (GATED) qdt.load_channel(gbias, a.dt_bias, d0);
  float dbias_acc = 0.f;   // GATED: this thread's sum of the raw dt gradient (channel tid % 32)

  // Chunk ci (any integer): its length (0 outside this block's segment, so
  // that every load and store of a chunk outside it is empty). The swept
  // kernel also reads dt, x and B from the chunks of the segment's first
  // caller chunk that lie before the segment (from c_in): their states are
  // swept, not walked.
  const int last_len = T - (nch - 1) * K;
  const int c_in = SWEEP > 0 ? c_lo / a.km * a.km : c_lo;
  auto chunk_len = [&](int ci) {
    return (ci < c_lo || ci >= c_hi) ? 0 : ci == nch - 1 ? last_len : K;
  };
  auto in_len = [&](int ci) {
    return (ci < c_in || ci >= c_hi) ? 0 : ci == nch - 1 ? last_len : K;
  };
  // Resources over chunk ci of the operands (channels d0 .. D-1 of the
  // (batch, T, D) ones, all N states of B, C and of the dB / dC rows; see
  // SubStream): empty outside [c_lo, c_hi) ([c_in, c_hi) for dt, x, B).
  auto stream = [&](const void* base, int ld, int c0, int width, int lo) {
    return SubStream<ES>(base, row0, ld, c0, width, K, lo, c_hi, nch - 1, last_len);
  };
  const SubStream<ES> sx = stream(a.x, D, d0, D, c_in), sdt = stream(a.dt, ld_dt, d0, D, c_in),
                      sdy = stream(a.dy, D, d0, D, c_lo), sB = stream(a.B, ld_bc, 0, N, c_in),
                      sC = stream(a.C, ld_bc, 0, N, c_lo), sdx = stream(a.dx, D, d0, D, c_lo),
                      sddt = stream(a.ddt, ld_ddt, d0, D, c_lo);
  // global -> staging registers: chunk ci (the prologue), or the chunk of
  // the loop's load cursors (two below the chunk walked).
  auto load_sub = [&](int ci) {
    if constexpr (!CARRY) ql.load(px, sx.at(ci));
    qdt.load(pd, sdt.at(ci));
    ql.load(py, sdy.at(ci));
    if constexpr (!CARRY) rl.load(pb, sB.at(ci));
    rl.load(pc, sC.at(ci));
  };
  StreamCursor<ES> lx(sx, c_hi - 3), ldt(sdt, c_hi - 3), ldy(sdy, c_hi - 3), lB(sB, c_hi - 3),
      lC(sC, c_hi - 3);
  auto load_next = [&]() {
    if constexpr (!CARRY) ql.load(px, lx.get(sx));
    qdt.load(pd, ldt.get(sdt));
    ql.load(py, ldy.get(sdy));
    if constexpr (!CARRY) rl.load(pb, lB.get(sB));
    rl.load(pc, lC.get(sC));
  };
  auto load_down = [&]() {
    lx.down(sx);
    ldt.down(sdt);
    ldy.down(sdy);
    lB.down(sB);
    lC.down(sC);
  };
  // h at the start of chunk ci: checkpoint ci-1, or 0 for the first chunk
  // (empty for ci <= 0). The loop walks it with a pointer moved down by one
  // (D, N) slice per chunk.
  const float* ck_row = a.ckpt + ((size_t)b * nch - 1) * slice;
  auto load_h0 = [&](int ci) {
    load_states<NPL>(ph, GBuf(ck_row + (ptrdiff_t)ci * (ptrdiff_t)slice, ci > 0 ? slice_bytes : 0u),
                     st_lane, nvalid, sw);
  };
  const float* ck_next = ck_row + (ptrdiff_t)(c_hi - 3) * (ptrdiff_t)slice;
  int ck_i = c_hi - 3;
  auto store_sub = [&](int j, int ci) {   // staging registers (chunk ci) -> buffer j
    float* s0 = sbuf + j * BUF;
    if constexpr (GATED) qdt.gate(pd, in_len(ci), a.dt_lo, a.dt_span, gbias);
    if constexpr (CARRY) {
#pragma unroll
      for (int f = 0; f < PER; ++f) sdt_part += (pd[f].x + pd[f].y) + (pd[f].z + pd[f].w);
    }
    ql.template store_cm<kBwdCm>(s0, pd);
    ql.template store_cm<kBwdCm>(s0 + oDY, py);
    if constexpr (!CARRY) ql.template store_cm<kBwdCm>(s0 + oX, px);
    if constexpr (!CARRY)   // dt * x, once per block
      ql.template store_cm_product<kBwdCm>(s0 + oDTX, pd, px);
    if constexpr (RL) {
      rlq.store(s0 + oB, pb, 0);
      rlq.store(s0 + oB, pc, 1);
    } else {
      if constexpr (!CARRY) rl.store(s0 + oB, pb);
      rl.store(s0 + oC, pc);
    }
  };
  // The fp32 rows of the dB / dC block sums of chunk ci: this block's
  // partials (rows of N), or with ATOM the gradients themselves (rows ld_dbc
  // apart).
  const size_t prow = ((size_t)blockIdx.x * a.batch + b) * T;
  const SubStream<4> swB(a.wsB, prow, N, 0, N, K, c_lo, c_hi, nch - 1, last_len),
                     swC(a.wsC, prow, N, 0, N, K, c_lo, c_hi, nch - 1, last_len),
                     sdB(a.dB, row0, a.ld_dbc, 0, N, K, c_lo, c_hi, nch - 1, last_len),
                     sdC(a.dC, row0, a.ld_dbc, 0, N, K, c_lo, c_hi, nch - 1, last_len);
  const SubStream<4>& sBsum = ATOM ? sdB : swB;
  const SubStream<4>& sCsum = ATOM ? sdC : swC;
  // dx, ddt and the dB, dC block sums of chunk ci (len steps), staged in
  // buffer j, into gdx, gddt and the dB / dC rows gbs, gcs: from tS and tDBC
  // (which hold them until the next reverse phase) and the chunk's x and dt
  // tiles.
  auto finalize = [&](int j, int len, const GBuf& gdx, const GBuf& gddt, const GBuf& gbs,
                      const GBuf& gcs) {
    const float* tx = sbuf + j * BUF + oX;
    const float* tdt = sbuf + j * BUF;
#pragma unroll
    for (int f = 0; f < FT; ++f) {
      const int task0 = tid + f * NT;
      const bool ok = task0 < kSteps / 2 * kCH;
      const int task = ok ? task0 : 0;
      const int cc = task % kCH, k = 2 * (task / kCH);
      const bool okc = ok && d0 + cc < D;
      const unsigned o0 = okc ? (unsigned)ES * ((unsigned)k * (unsigned)D + cc) : kOOB;
      const unsigned o1 = okc ? o0 + (unsigned)ES * (unsigned)D : kOOB;
      const unsigned od0 = okc ? (unsigned)ES * ((unsigned)k * (unsigned)ld_ddt + cc) : kOOB;
      const unsigned od1 = okc ? od0 + (unsigned)ES * (unsigned)ld_ddt : kOOB;
      const float2 xv = lds2(tx + cml_elem<kBwdCm>(cc, k));
      const float2 dtv = lds2(tdt + cml_elem<kBwdCm>(cc, k));
      const float x0 = xv.x, x1 = xv.y, t0v = dtv.x, t1v = dtv.y;
      // The waves' partials summed in order from wave 0's (not from 0.f:
      // an add of zero that the compiler keeps, for the sign of zero).
      float s1a = 0.f, s1b = 0.f, s2a = 0.f, s2b = 0.f;
#pragma unroll
      for (int w = 0; w < G; ++w) {
        const float2 v1 = lds2(tS + ((k / 2) * G + w) * 128 + cc * 2);
        const float2 v2 = lds2(tS + ((k / 2) * G + w) * 128 + (kCH + cc) * 2);
        if (w == 0) {
          s1a = v1.x; s1b = v1.y;
          s2a = v2.x; s2b = v2.y;
        } else {
          s1a += v1.x; s1b += v1.y;
          s2a += v2.x; s2b += v2.y;
        }
      }
      // dx, ddt: written once, not read again here (NT).
      st_elem<ES, kStream>(gdx, t0v * s1a, o0);
      st_elem<ES, kStream>(gdx, t1v * s1b, o1);
      float g0 = __builtin_fmaf(x0, s1a, -s2a), g1 = __builtin_fmaf(x1, s1b, -s2b);
      if constexpr (GATED) {
        const float u0 = t0v - a.dt_lo, u1 = t1v - a.dt_lo;   // span * s
        g0 *= u0 * (a.dt_span - u0) * a.dt_inv_span;
        g1 *= u1 * (a.dt_span - u1) * a.dt_inv_span;
        // Task f's channel is tid % 32 for every f (NT is a multiple of 32).
        dbias_acc += (okc && k < len ? g0 : 0.f) + (okc && k + 1 < len ? g1 : 0.f);
      }
      st_elem<ES, kStream>(gddt, g0, od0);
      st_elem<ES, kStream>(gddt, g1, od1);
    }
    // The block's sums: partials (rows of N), or with ATOM added into rows
    // (b, t) of dB and dC (ld_dbc apart). The resources end after the
    // chunk's last row.
    const int ldr = ATOM ? a.ld_dbc : N;
#pragma unroll
    for (int f = 0; f < FK; ++f) {
      const int r0 = tid + f * NT;                // (k, n) of the tile, n fastest
      const bool okr = kFKExact || r0 < kSteps * NP;
      const int r = okr ? r0 : 0;
      const int k = r / NP, n = r % NP;
      const unsigned o = okr && n < N ? 4u * (unsigned)(k * ldr + n) : kOOB;
      float vb, vc;
      if constexpr (RP) {
        // the two rows' partials of the half-wave, added in a fixed order
        const int rr = k * RPS + n;
        vb = tDBC[rr] + tDBC[2 * RPK + rr];
        vc = tDBC[RPK + rr] + tDBC[3 * RPK + rr];
      } else {
        vb = tDBC[r];
        vc = tDBC[kSteps * NP + r];
      }
      if constexpr (ATOM) {
        gbs.atomic_add(vb, o);
        gcs.atomic_add(vc, o);
      } else {
        // plain stores: the reduction kernel reads the partials right after
        // this kernel, and they are then still cached (measured: 11.9 ->
        // 11.1 us for its 50 MB at 16x512x1536x16 against non-temporal ones)
        gbs.st(vb, o);
        gcs.st(vc, o);
      }
    }
  };
  // finalize's output resources walked down with the loop (chunk ci + 1).
  StreamCursor<ES> fdx(sdx, c_hi), fddt(sddt, c_hi);
  StreamCursor<4> fbs(sBsum, c_hi), fcs(sCsum, c_hi);

  float hc[NPL];                          // h at the start of the current chunk
  int last_par;                           // LDS buffer of the segment's last chunk
  if constexpr (SWEEP > 0) {
    // Checkpoint stride a.km x 16 steps (2 <= a.km <= SWEEP), the caller's
    // own checkpoints: the walk goes over 16-step chunks as usual, and the
    // states at the 16-step boundaries inside a caller chunk are rebuilt in
    // this kernel, by "sweep" items of the same pipeline. For each caller
    // chunk cc (last to first), holding n walk chunks: sweep its chunks 0 ..
    // n-2 forward from the caller's checkpoint (each rebuilds its dA and h
    // as the walk's recompute phase does, and keeps only the end state, in
    // H[l + 1]), then walk chunks n-1 .. 0 backwards from H[l] (in a time
    // segment that starts inside a caller chunk, only its own chunks of
    // that caller chunk are walked: the segments are the stride-16 ones, so
    // the results equal those at stride 16 bit for bit). The sweeps
    // stage dt, x and B only (their dy and C loads are empty). An item
    // that follows a walk has the walk's two barriers (the first after that
    // walk's finishing step), one that follows a sweep only the last.
    static_assert(!CARRY, "the in-kernel sweep: gradient pass only");
    const int KM = a.km;
    const int cc_lo = c_lo / KM, cc_top = (c_hi - 1) / KM;
    const int n_top = c_hi - cc_top * KM;
    const int lo_first = c_lo - cc_lo * KM;   // the segment may start inside a caller chunk
    // Per caller chunk cc: n walk chunks (n_top for the segment's last
    // caller chunk), of which those from lo (lo_first in its first, else 0)
    // belong to this segment: n - 1 sweeps, then n - lo walks.
    const int nitem = 2 * (c_hi - cc_lo * KM) - (cc_top - cc_lo + 1) - lo_first;
    // Position in the item sequence: caller chunk cc, item l of its
    // 2n - 1 - lo. Advanced by one per item (no divisions in the loop).
    struct Pos {
      int cc, l, n, lo;
    };
    auto advance = [&](Pos p) {
      if (++p.l == 2 * p.n - 1 - p.lo) {
        --p.cc;
        p.l = 0;
        p.n = KM;
        p.lo = p.cc == cc_lo ? lo_first : 0;
      }
      return p;
    };
    struct Item {
      int ci;      // walk chunk (16 steps); -1: none (empty resources)
      int loc;     // its index inside the caller chunk
      bool sweep;  // sweep (forward, end state only) or walk (gradients)
      bool first;  // the caller chunk's first item
    };
    auto item_at = [&](const Pos& p) {
      Item it{-1, 0, false, false};
      if (p.cc < cc_lo) return it;   // past the segment's first chunk
      it.sweep = p.l < p.n - 1;
      it.loc = it.sweep ? p.l : 2 * (p.n - 1) - p.l;
      it.ci = p.cc * KM + it.loc;
      it.first = p.l == 0;
      return it;
    };
    // The caller's checkpoint before caller chunk cc (0 for the first).
    const float* ckc = a.ckpt + ((size_t)b * a.ck_nchunk - 1) * slice;
    auto load_h0c = [&](int cc) {
      load_states<NPL>(ph, GBuf(ckc + (ptrdiff_t)cc * (ptrdiff_t)slice, cc > 0 ? slice_bytes : 0u),
                       st_lane, nvalid, sw);
    };
    auto load_item = [&](const Item& it) {
      const int cy = it.sweep ? -1 : it.ci;
      ql.load(px, sx.at(it.ci));
      qdt.load(pd, sdt.at(it.ci));
      ql.load(py, sdy.at(cy));
      rl.load(pb, sB.at(it.ci));
      rl.load(pc, sC.at(cy));
    };
    // H[l], the state at the start of walk chunk l of the caller chunk, in
    // this thread's LDS slot l (lanes contiguous: conflict-free 32 / 64 /
    // 128-bit accesses); registers are what the walk is short of.
    static_assert(SWEEP <= kSweepMax, "LDS slots for the swept states");
    float* const tH = lds + bwd_lds_floats(G, NPL, RL, RP, false) + tid * NPL;
    auto h_slot = [&](int l) { return tH + l * NT * NPL; };
    Pos pos{cc_top, 0, n_top, cc_top == cc_lo ? lo_first : 0};
    const Item it0 = item_at(pos);
    load_h0c(cc_top);
    load_item(it0);
    store_sub(0, it0.ci);
    load_item(item_at(advance(pos)));
    __syncthreads();

    Item itp{-1, 0, false, false};   // the previous item
    ProgressPriority prio(nitem);
    for (int k = 0; k < nitem; ++k) {
      prio.step(k);
      const Item it = item_at(pos);
      const Pos pos1 = advance(pos);
      const Item it1 = item_at(pos1), it2 = item_at(advance(pos1));
      const float* s0 = sbuf + (k & 1) * BUF;
      const float* gB = s0 + oB + q * bc_group_floats(NPL);
      const float* gC = s0 + oC + q * bc_group_floats(NPL);
      const float* gQ = s0 + oB + q * kBCGroupQ + (lane & 3) * 2;   // RL
      if (it.first) {
        float h0[NPL];
#pragma unroll
        for (int j = 0; j < NPL; ++j) h0[j] = opaque_copy(ph[j]);
        store_vec<NPL>(h_slot(0), h0);
        load_h0c(it.ci / KM - 1);   // the next caller chunk's
      }
      load_vec<NPL>(hc, h_slot(it.loc));
      // The previous item's gradients (if it was a walk) are finished here,
      // in this item's first phase; only then does the item need a barrier
      // between its phases (finalize reads the previous buffer and the
      // (s1, s2) and dB / dC tiles that this item's second phase rewrites).
      const bool fin = !itp.sweep && itp.ci >= 0;

      // ---- recompute (walk) or sweep: dA and h of the chunk
      float da[kSteps][NPL], hs[kSteps][NPL];
#pragma unroll
      for (int m = 0; m < kQuads; ++m) {
        float dts[4], dtxs[4], Bq[4][NPL];
        float2 qb;   // RL: B of the quad broadcast tile
        f4_to(dts, lds4(s0 + cml_quad<kBwdCm>(c, m)));
        f4_to(dtxs, lds4(s0 + oDTX + cml_quad<kBwdCm>(c, m)));
        if constexpr (RL) {
          qb = lds2(gQ + 16 * m);
        } else {
          load_quad_rows<NPL>(Bq, gB, m);
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
#pragma unroll
          for (int j = 0; j < NPL; ++j) {
            da[4 * m + s][j] = exp2_hw(dts[s] * a2[j]);
            const float bv = RL ? qp_get((s >> 1) ? qb.y : qb.x, qp_sel(s, j)) : Bq[s][j];
            hs[4 * m + s][j] = bv * dtxs[s];
          }
        }
        if (m == 0 && fin)
          finalize((k + 1) & 1, chunk_len(itp.ci), sdx.at(itp.ci), sddt.at(itp.ci),
                   sBsum.at(itp.ci), sCsum.at(itp.ci));
      }
#pragma unroll
      for (int kk = 0; kk < kSteps; ++kk)
#pragma unroll
        for (int j = 0; j < NPL; ++j)
          hs[kk][j] = __builtin_fmaf(da[kk][j], kk == 0 ? hc[j] : hs[kk - 1][j], hs[kk][j]);
      if (it.sweep) {
        store_vec<NPL>(h_slot(it.loc + 1), hs[kSteps - 1]);
        if (fin) __syncthreads();   // finalize(previous) is done with its buffer
        store_sub((k + 1) & 1, it1.ci);
        load_item(it2);
        __syncthreads();   // the next item staged
        itp = it;
        pos = pos1;
        continue;
      }
      if (fin) __syncthreads();   // finalize(previous) is done with tS, tDBC and its buffer

      // ---- reverse phase (the walk's)
#pragma unroll
      for (int m = kQuads - 1; m >= 0; --m) {
        float dts[4], dys[4], dtxs[4], Bq[4][NPL], Cq[4][NPL], s1q[4], s2q[4];
        float dysp[4], dtxsp[4];   // RL: the partner channel's
        f4_to(dts, lds4(s0 + cml_quad<kBwdCm>(c, m)));
        f4_to(dys, lds4(s0 + oDY + cml_quad<kBwdCm>(c, m)));
        f4_to(dtxs, lds4(s0 + oDTX + cml_quad<kBwdCm>(c, m)));
        if constexpr (RL) {
          f4_to(dysp, lds4(s0 + oDY + cml_quad<kBwdCm>(cp, m)));
          f4_to(dtxsp, lds4(s0 + oDTX + cml_quad<kBwdCm>(cp, m)));
        }
        float2 qb, qc;   // RL: B and C of the quad broadcast tile
        if constexpr (RL) {
          qb = lds2(gQ + 16 * m);
          qc = lds2(gQ + 16 * m + 8);
        } else {
          load_quad_rows<NPL>(Bq, gB, m);
          load_quad_rows<NPL>(Cq, gC, m);
        }
        float pv[M], pa[4];
#pragma unroll
        for (int s = 3; s >= 0; --s) {
          const int kk = 4 * m + s;
          const int slot = kk & 1;
          float s1 = 0.f, s2 = 0.f, gk[NPL];
#pragma unroll
          for (int j = 0; j < NPL; ++j) {
            if constexpr (RL) {
              gk[j] = u[j];
              qp_fmac(gk[j], (s >> 1) ? qc.y : qc.x, dys[s], qp_sel(s, j));
            } else {
              gk[j] = __builtin_fmaf(dys[s], Cq[s][j], u[j]);
            }
            u[j] = da[kk][j] * gk[j];
            const float qv = u[j] * (kk == 0 ? hc[j] : hs[kk - 1][j]);
            if constexpr (RL) {
              const float br = (s >> 1) ? qb.y : qb.x;
              if (j == 0) s1 = qp_get(br, qp_sel(s, 0)) * gk[0];
              else qp_fmac(s1, br, gk[j], qp_sel(s, j));
            } else {
              s1 = __builtin_fmaf(gk[j], Bq[s][j], s1);
            }
            s2 = __builtin_fmaf(an[j], qv, s2);
            acc[j] = __builtin_fmaf(dts[s], qv, acc[j]);
          }
          s1q[s] = s1;
          s2q[s] = s2;
          if constexpr (RL) {
            pa[slot] = pair_sum_xor1(gk[0], gk[1], dtxs[s], dtxsp[s]);
            pa[2 + slot] = pair_sum_xor1(hs[kk][0], hs[kk][1], dys[s], dysp[s]);
          } else {
#pragma unroll
            for (int j = 0; j < NPL; ++j) {
              pv[slot * NPL + j] = gk[j] * dtxs[s];
              pv[2 * NPL + slot * NPL + j] = hs[kk][j] * dys[s];
            }
          }
          if (slot == 0) *(dbc_out + kk * kDbcStep) = channel_sums(pv, pa);
        }
        float o[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(s1q[s]),
                                                          __float_as_uint(s2q[s]), false, false);
          o[s] = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
        }
        float* const ts = tS + wave * 128 + lane * 2;
        *reinterpret_cast<float2*>(ts + 2 * m * G * 128) = make_float2(o[0], o[1]);
        *reinterpret_cast<float2*>(ts + (2 * m + 1) * G * 128) = make_float2(o[2], o[3]);
        if (m == 2) store_sub((k + 1) & 1, it1.ci);
        if (m == 1) load_item(it2);
      }
      __syncthreads();   // tS / tDBC complete; the next item staged
      itp = it;
      pos = pos1;
    }
    last_par = (nitem - 1) & 1;
  } else {
    // Prologue: the segment's last chunk staged in LDS buffer 0, the one
    // before it in the staging registers.
    load_sub(c_hi - 1);
    if constexpr (!CARRY) load_h0(c_hi - 1);
    store_sub(0, c_hi - 1);
    if constexpr (!CARRY) {
#pragma unroll
      for (int j = 0; j < NPL; ++j) hc[j] = opaque_copy(ph[j]);
    }
    load_sub(c_hi - 2);
    if constexpr (!CARRY) load_h0(c_hi - 2);
    __syncthreads();

    const int nit = c_hi - c_lo;
    ProgressPriority prio(nit);
    for (int i = 0; i < nit; ++i) {
      prio.step(i);
      const int ci = c_hi - 1 - i;
      const float* s0 = sbuf + (i & 1) * BUF;
      const float* gB = s0 + oB + q * bc_group_floats(NPL);
      const float* gC = s0 + oC + q * bc_group_floats(NPL);
      // RL: this lane's floats of each quad of the quad broadcast tile (B;
      // C 8 further)
      const float* gQ = s0 + oB + q * kBCGroupQ + (lane & 3) * 2;

      if constexpr (CARRY) {
        // The adjoint alone: G_t = dy_t C_t + dA_{t+1} G_{t+1}, dA formed on
        // the way (no state needed).
#pragma unroll
        for (int m = kQuads - 1; m >= 0; --m) {
          float dts[4], dys[4], Cq[4][NPL];
          f4_to(dts, lds4(s0 + cml_quad<kBwdCm>(c, m)));
          f4_to(dys, lds4(s0 + oDY + cml_quad<kBwdCm>(c, m)));
          load_quad_rows<NPL>(Cq, gC, m);
#pragma unroll
          for (int s = 3; s >= 0; --s) {
#pragma unroll
            for (int j = 0; j < NPL; ++j)
              u[j] = exp2_hw(dts[s] * a2[j]) * __builtin_fmaf(dys[s], Cq[s][j], u[j]);
          }
          if (m == 2) store_sub((i + 1) & 1, ci - 1);
          if (m == 1) load_next();
        }
        load_down();
        __syncthreads();   // chunk ci-1 staged
        continue;
      }

      // ---- recompute phase, with the pipeline work of the neighbouring chunks
      float da[kSteps][NPL], hs[kSteps][NPL];
#pragma unroll
      for (int m = 0; m < kQuads; ++m) {
        float dts[4], dtxs[4], Bq[4][NPL];
        float2 qb;   // RL: B of the quad broadcast tile
        f4_to(dts, lds4(s0 + cml_quad<kBwdCm>(c, m)));
        f4_to(dtxs, lds4(s0 + oDTX + cml_quad<kBwdCm>(c, m)));
        if constexpr (RL) {
          qb = lds2(gQ + 16 * m);
        } else {
          load_quad_rows<NPL>(Bq, gB, m);
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
#pragma unroll
          for (int j = 0; j < NPL; ++j) {
            da[4 * m + s][j] = exp2_hw(dts[s] * a2[j]);
            const float bv = RL ? qp_get((s >> 1) ? qb.y : qb.x, qp_sel(s, j)) : Bq[s][j];
            hs[4 * m + s][j] = bv * dtxs[s];       // b_k, turned into h_k below
          }
        }
        if (m == 0)   // no-op stores past the sequence end
          finalize((i + 1) & 1, chunk_len(ci + 1), fdx.get(sdx), fddt.get(sddt), fbs.get(sBsum),
                   fcs.get(sCsum));
      }
#pragma unroll
      for (int k = 0; k < kSteps; ++k)
#pragma unroll
        for (int j = 0; j < NPL; ++j)
          hs[k][j] = __builtin_fmaf(da[k][j], k == 0 ? hc[j] : hs[k - 1][j], hs[k][j]);
      __syncthreads();   // finalize(ci+1) is done with tS, tDBC and its buffer

      // ---- reverse phase
#pragma unroll
      for (int m = kQuads - 1; m >= 0; --m) {
        float dts[4], dys[4], dtxs[4], Bq[4][NPL], Cq[4][NPL], s1q[4], s2q[4];
        float dysp[4], dtxsp[4];   // RL: the partner channel's
        f4_to(dts, lds4(s0 + cml_quad<kBwdCm>(c, m)));
        f4_to(dys, lds4(s0 + oDY + cml_quad<kBwdCm>(c, m)));
        f4_to(dtxs, lds4(s0 + oDTX + cml_quad<kBwdCm>(c, m)));
        if constexpr (RL) {
          f4_to(dysp, lds4(s0 + oDY + cml_quad<kBwdCm>(cp, m)));
          f4_to(dtxsp, lds4(s0 + oDTX + cml_quad<kBwdCm>(cp, m)));
        }
        float2 qb, qc;   // RL: B and C of the quad broadcast tile
        if constexpr (RL) {
          qb = lds2(gQ + 16 * m);
          qc = lds2(gQ + 16 * m + 8);
        } else {
          load_quad_rows<NPL>(Bq, gB, m);
          load_quad_rows<NPL>(Cq, gC, m);
        }
        // dB/dC products of the step pair (k, k+1), k even, numbered as for
        // rs_index, or with RL their bit-0 pair sums
        float pv[M], pa[4];
#pragma unroll
        for (int s = 3; s >= 0; --s) {
          const int k = 4 * m + s;
          const int slot = k & 1;
          float s1 = 0.f, s2 = 0.f, gk[NPL];
#pragma unroll
          for (int j = 0; j < NPL; ++j) {
            if constexpr (RL) {
              gk[j] = u[j];                                            // G_k
              qp_fmac(gk[j], (s >> 1) ? qc.y : qc.x, dys[s], qp_sel(s, j));
            } else {
              gk[j] = __builtin_fmaf(dys[s], Cq[s][j], u[j]);          // G_k
            }
            u[j] = da[k][j] * gk[j];                                   // dA_k G_k
            const float qv = u[j] * (k == 0 ? hc[j] : hs[k - 1][j]);   // G_k * hm_k
            if constexpr (RL) {
              // G_k . B_k: the first product a DPP multiply, as the fma
              // into 0 of the other plans rounds it
              const float br = (s >> 1) ? qb.y : qb.x;
              if (j == 0) s1 = qp_get(br, qp_sel(s, 0)) * gk[0];
              else qp_fmac(s1, br, gk[j], qp_sel(s, j));
            } else {
              s1 = __builtin_fmaf(gk[j], Bq[s][j], s1);
            }
            s2 = __builtin_fmaf(an[j], qv, s2);
            acc[j] = __builtin_fmaf(dts[s], qv, acc[j]);
          }
          s1q[s] = s1;
          s2q[s] = s2;
          if constexpr (RL) {
            pa[slot] = pair_sum_xor1(gk[0], gk[1], dtxs[s], dtxsp[s]);            // dB
            pa[2 + slot] = pair_sum_xor1(hs[k][0], hs[k][1], dys[s], dysp[s]);    // dC
          } else {
#pragma unroll
            for (int j = 0; j < NPL; ++j) {
              pv[slot * NPL + j] = gk[j] * dtxs[s];             // dB: G * dt * x
              pv[2 * NPL + slot * NPL + j] = hs[k][j] * dys[s];   // dC: h * dy
            }
          }
          if (slot == 0) *(dbc_out + k * kDbcStep) = channel_sums(pv, pa);
        }
        // Add the two half-waves: lanes 0-31 end with s1, lanes 32-63 with s2.
        float o[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(s1q[s]),
                                                          __float_as_uint(s2q[s]), false, false);
          o[s] = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
        }
        // tS: [8 step pairs][G waves][64 rows][2] (rows 0-31: s1 of the
        // channels, 32-63: s2): a wave's 64-bit writes of one pair are
        // contiguous (no bank conflicts), and finalize's reads of a pair's
        // partials over the waves lie within 2 KB of one address (read2).
        float* const ts = tS + wave * 128 + lane * 2;
        *reinterpret_cast<float2*>(ts + 2 * m * G * 128) = make_float2(o[0], o[1]);
        *reinterpret_cast<float2*>(ts + (2 * m + 1) * G * 128) = make_float2(o[2], o[3]);
        if (m == 2) store_sub((i + 1) & 1, ci - 1);  // unused when ci == 0
        if (m == 1) load_next();             // chunk ci - 2: loads nothing when ci < 2
      }
      // h at the start of chunk ci-1, copied here and now (an opaque copy the
      // compiler cannot sink): ph's registers are then free for the next
      // checkpoint load. A copy left at the loop back-edge would move that load's
      // result, i.e. wait for it, and vmcnt being in order, for every load and
      // store still in flight: a full memory drain per chunk.
#pragma unroll
      for (int j = 0; j < NPL; ++j) hc[j] = opaque_copy(ph[j]);
      load_states<NPL>(ph, GBuf(ck_next, ck_i > 0 ? slice_bytes : 0u), st_lane, nvalid,
                       sw);   // h0(ci-2)
      ck_next -= slice;
      --ck_i;
      load_down();
      fdx.down(sdx);
      fddt.down(sddt);
      fbs.down(sBsum);
      fcs.down(sCsum);
      __syncthreads();   // tS / tDBC complete; chunk ci-1 staged
    }
    last_par = (nit - 1) & 1;
  }
  const size_t slot = (size_t)seg * a.batch + b;
  if constexpr (CARRY) {
    // L_s = dA_a * G_a, a the segment's first step: u after the walk.
    store_states<NPL>(GBuf(a.carryL + slot * slice, slice_bytes), st_lane, nvalid, u, sw);
    // The staging tasks' sums of dt, channel tid % 32 each (NT a multiple of
    // 32; threads without a task hold 0), added per channel in a fixed
    // order. The loop ended on a barrier: LDS is free.
    static_assert(NT % kCH == 0, "staging tasks keep their channel");
    lds[tid] = sdt_part;
    __syncthreads();
    if (q == 0 && act) {
      float sdt = 0.f;
#pragma unroll
      for (int r = 0; r < NT / kCH; ++r) sdt += lds[r * kCH + c];
      a.carrySdt[slot * D + d] = sdt;
    }
    return;
  }
  finalize(last_par, chunk_len(c_lo), sdx.at(c_lo), sddt.at(c_lo), sBsum.at(c_lo),
           sCsum.at(c_lo));

  float out[NPL];
#pragma unroll
  for (int j = 0; j < NPL; ++j) out[j] = -acc[j];
  if constexpr (ATOM) {
    // dAneg, or for the gated kernel dA = dAneg * softplus'(A) = dAneg * sigmoid(A).
    const GBuf gda(a.daneg, slice_bytes);
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
      const int nj = j ^ sw;
      float v = out[j];
      if constexpr (GATED)
        v *= (act && nj < nvalid) ? sigmoid_f(a.aneg[(size_t)d * N + n0 + nj]) : 0.f;
      gda.atomic_add(v, (st_lane != kOOB && nj < nvalid) ? st_lane + 4u * nj : kOOB);
    }
  } else {
    store_states<NPL>(GBuf(a.wsA + slot * slice, slice_bytes), st_lane, nvalid, out, sw);
  }
  if constexpr (GATED) {
    if (ATOM ? a.dbias != nullptr : a.wsDB != nullptr) {
      // The block's sum of the raw dt gradient per channel: the NT / 32
      // threads of channel cc (tid = cc + 32 r) added in a fixed order.
      static_assert(NT % kCH == 0, "finalize tasks keep their channel");
      __syncthreads();   // every finalize read of LDS is done
      lds[tid] = dbias_acc;
      __syncthreads();
      if (tid < kCH && d0 + tid < D) {
        float sum = 0.f;
#pragma unroll
        for (int r = 0; r < NT / kCH; ++r) sum += lds[r * kCH + tid];
        if constexpr (ATOM)
          GBuf(a.dbias, 4u * (unsigned)D).atomic_add(sum, 4u * (unsigned)(d0 + tid));
        else
          a.wsDB[slot * D + d0 + tid] = sum;
      }
    }
  }
}

// dB, dC: sum the per-block partials over the nblk channel blocks;
// dAneg: sum the per-batch partials over the batch. The sums run in a fixed
// order (block 0, 1, ...); the loads are issued eight at a time so that each
// thread keeps 16 loads in flight instead of one dependent load per add.
__device__ __forceinline__ void ordered_sum2(const float* __restrict__ p, const float* __restrict__ q,
                                             size_t stride, int n, float& sp, float& sq) {
  int k = 0;
  for (; k + 8 <= n; k += 8) {
    float vp[8], vq[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      vp[u] = p[(size_t)(k + u) * stride];
      vq[u] = q[(size_t)(k + u) * stride];
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      sp += vp[u];
      sq += vq[u];
    }
  }
  for (; k < n; ++k) {
    sp += p[(size_t)k * stride];
    sq += q[(size_t)k * stride];
  }
}

// a_raw: null, or A for the gated backward: then daneg receives dAneg *
// softplus'(A) = dAneg * sigmoid(A), the gradient of A. dB, dC: ES-byte
// elements (fp32 or bf16), rows of N elements ld_dbc apart. Dn: 0, or D for
// the gated backward's dt-bias gradient: dbias[d] = the sum of wsDB's
// `batch` rows (of Dn) in a fixed order.
template <int ES = 4>
__global__ void __launch_bounds__(256)
bwd_reduce_kernel(const float* __restrict__ wsB, const float* __restrict__ wsC,
                  const float* __restrict__ wsA, const float* __restrict__ a_raw,
                  void* __restrict__ dB, void* __restrict__ dC, float* __restrict__ daneg,
                  int nblk, int batch, long long S, long long A, int N, long long ld_dbc,
                  const float* __restrict__ wsDB, float* __restrict__ dbias, int Dn) {
  const long long stride = (long long)gridDim.x * blockDim.x;
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < S + A + Dn;
       i += stride) {
    if (i < S) {
      float sb = 0.f, sc = 0.f;
      ordered_sum2(wsB + i, wsC + i, (size_t)S, nblk, sb, sc);
      const long long o = ld_dbc == N ? i : (i / N) * ld_dbc + i % N;   // row stride ld_dbc
      if constexpr (ES == 4) {
        static_cast<float*>(dB)[o] = sb;
        static_cast<float*>(dC)[o] = sc;
      } else {
        static_cast<unsigned short*>(dB)[o] = f32_to_bf16(sb);
        static_cast<unsigned short*>(dC)[o] = f32_to_bf16(sc);
      }
    } else if (i < S + A) {
      const long long j = i - S;
      float s = 0.f;
      for (int bb = 0; bb < batch; ++bb) s += wsA[(size_t)bb * A + j];
      daneg[j] = a_raw != nullptr ? s / (1.f + expf(-a_raw[j])) : s;
    } else {
      const long long j = i - S - A;
      float s = 0.f;
      for (int bb = 0; bb < batch; ++bb) s += wsDB[(size_t)bb * Dn + j];
      dbias[j] = s;
    }
  }
}

// Zero the gradients the atomic backward adds into: dB and dC (rows x N,
// rows ld apart), dAneg (A floats) and the dt-bias gradient (Dn floats; null
// when Dn is 0). A kernel rather than hipMemsetAsync, so that the launch
// sequence stays capturable in a HIP graph without memset nodes.
template <int UNUSED = 0>
__global__ void __launch_bounds__(256)
zero_grads_kernel(float* __restrict__ dB, float* __restrict__ dC, long long rows, int N,
                  long long ld, float* __restrict__ daneg, long long A, float* __restrict__ dbias,
                  int Dn) {
  const long long S = rows * N;
  const long long stride = (long long)gridDim.x * blockDim.x;
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < S + A + Dn;
       i += stride) {
    if (i < S) {
      const long long o = ld == N ? i : (i / N) * ld + i % N;
      dB[o] = 0.f;
      dC[o] = 0.f;
    } else if (i < S + A) {
      daneg[i - S] = 0.f;
    } else {
      dbias[i - S - A] = 0.f;
    }
  }
}

}  // namespace mhs
