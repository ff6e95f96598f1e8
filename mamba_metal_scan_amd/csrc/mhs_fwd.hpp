// Forward selective scan for gfx950.
//
// Math of the reference's ssm_fwd (mamba_metal/scan.py:78-127):
//   da = exp(-dt * Aneg); h = da * h + B * (dt * x); y = sum_n C * h;
//   h is written to ckpt at the end of every chunk of K steps (and at T-1).
//
// MI355X mapping (not the reference's one-thread-per-channel layout):
//   grid (ceil(D/32), batch), block 64*G. Lane (wave w, half hh, channel c)
//   owns channel d = blockIdx.x*32 + c and the NPL states n in [q*NPL,
//   q*NPL+NPL), q = 2w + hh: the d_state vector of a channel is spread over
//   2G lane groups (d_state padded with zero states to NP = 2*G*NPL), each
//   lane keeping NPL recurrences in VGPRs for the whole sequence. At batch 16
//   x d_inner 1536 x d_state 16 (NPL 2, G 4) that is 768 blocks of 4 waves:
//   3 blocks per CU and 3 waves per SIMD.
//
//   Time advances in sub-chunks of 16 steps, as a software pipeline with one
//   barrier per sub-chunk. While sub-chunk i is computed, the same waves, in
//   the same straight-line code (all global accesses are bounds-checked
//   buffer accesses, so there are no branches), also
//     - sum the y partials of sub-chunk i-1 over the 2G lane groups in a
//       fixed order and store y, coalesced along d;
//     - store the staged inputs of sub-chunk i+1 into the other LDS buffer
//       (dt and dt*x as channel-major tiles, B and C per lane group);
//     - issue the global loads of sub-chunk i+3 into the staging registers
//       (two register sets, by sub-chunk parity; the loop is unrolled by two
//       sub-chunks, so that both the set and the LDS buffer are constants):
//       a load then has about 1.75 sub-chunks to arrive, against 0.75 with
//       one set (32x2048x4096x16: 1.39 -> 1.30 ms).
//   A lane reads its operands four steps at a time with 128-bit LDS reads,
//   computes the four dA = exp2(dt * -Aneg*log2e) and inputs first
//   (independent), then runs the four dependent h = fma(dA, h, u) steps and
//   the C.h sums, and writes its y partials of the quad as one float4.
#pragma once

#include <type_traits>

#include "mhs_common.hpp"

namespace mhs {

struct FwdArgs {
  // x, dt, B, C, y: ES-byte elements (fp32 or bf16, see the kernel's ES).
  const void* x;
  const void* dt;
  const float* aneg;
  const void* B;
  const void* C;
  void* y;         // may be null: then no y traffic at all
  float* ckpt;     // may be null
  float* h_last;   // may be null
  int T, D, N, K, nchunk;
  // Gated kernels only (GATED): dt holds the raw gate input and aneg holds A;
  // dt = dt_lo + dt_span * sigmoid(raw + dt_bias[d]) and Aneg = softplus(A)
  // are formed in the kernel (mamba_metal/model.py:197, :200; dt_bias, the
  // dt projection's bias, may be null).
  float dt_lo, dt_span;
  const float* dt_bias = nullptr;
  // Time segments: blockIdx.y = seg * batch + b; segment seg covers steps
  // [seg * seg_len, min(T, (seg + 1) * seg_len)), seg_len a multiple of 16
  // (nseg = 1, seg_len >= T: the whole sequence). A segment other than the
  // first starts from h_init, a checkpoint buffer (batch, init_nchunk, D, N)
  // of stride init_K that has a checkpoint at its first step (seg_len is a
  // multiple of init_K): the segments are then independent and exact.
  int batch = 1, seg_len = 0;
  const float* h_init = nullptr;
  int init_K = 1, init_nchunk = 1;
  // Carried segments (no h_init): segment s >= 1 starts from the state folded
  // from the carries of everything before it. The carry pass (FCARRY) runs
  // over carry units of seg_len / cunits steps (cunits per segment, so that
  // its grid has enough blocks to hide its dependent chains) and writes, for
  // unit u, hend_u, the state after unit u scanned from zero, to carryH
  // (units, batch, D, N) and Sdt_u, its sum of dt, to carrySdt (units,
  // batch, D). Segment s folds units 0 .. s*cunits - 1: H_0 = 0 and
  //   H_{u+1} = exp(-Aneg * Sdt_u) * H_u + hend_u.
  float* carryH = nullptr;
  float* carrySdt = nullptr;
  int cunits = 1;
  // Row strides (elements between consecutive time steps) of dt and of B,
  // C: D and N for contiguous tensors, more for column slices of a wider
  // projection output. x and y are contiguous.
  int ld_dt = 0, ld_bc = 0;
};

constexpr int kCH = 32;   // channels per block

// Two states per lane (NPL 2): B and C reach the lanes by DPP row broadcasts
// from a broadcast tile in the row layout (BCLayout::kRow): each lane of a
// 16-lane row reads one float per quad, and the multiply (B) and the fma (C)
// that use a value broadcast it from its lane with row_newbcast. The two
// rows of a half-wave read the same 16 floats.
__host__ __device__ constexpr int fwd_bc_floats(int G, int NPL) {
  return NPL == 2 ? 2 * G * kBCGroup2 : 2 * bc_tile_floats(2 * G, NPL);
}

// One pipeline buffer (the kernel keeps two).
__host__ __device__ constexpr int fwd_buf_floats(int G, int NPL) {
  return 2 * kCH * kSteps               // dt, dt*x tiles (channel-major)
         + fwd_bc_floats(G, NPL)        // B, C tiles
         + G * kCH * kSteps;            // per-wave y partials (both half-waves added)
}

// u[s][j] = B * bx[s] for the quad's 4 steps and 2 states, B broadcast from
// lane 2s + j of the row's value r (read from the broadcast tile). The
// leading s_nop gives the 2 wait states a DPP read of r needs should r have
// been written by a VALU instruction just before.
__device__ __forceinline__ void bcast_mul_b(float (&u)[4][2], float r, const float (&bx)[4]) {
  asm("s_nop 1\n\t"
      "v_mul_f32_dpp %0, %8, %9 row_newbcast:0 row_mask:0xf bank_mask:0xf\n\t"
      "v_mul_f32_dpp %1, %8, %9 row_newbcast:1 row_mask:0xf bank_mask:0xf\n\t"
      "v_mul_f32_dpp %2, %8, %10 row_newbcast:2 row_mask:0xf bank_mask:0xf\n\t"
      "v_mul_f32_dpp %3, %8, %10 row_newbcast:3 row_mask:0xf bank_mask:0xf\n\t"
      "v_mul_f32_dpp %4, %8, %11 row_newbcast:4 row_mask:0xf bank_mask:0xf\n\t"
      "v_mul_f32_dpp %5, %8, %11 row_newbcast:5 row_mask:0xf bank_mask:0xf\n\t"
      "v_mul_f32_dpp %6, %8, %12 row_newbcast:6 row_mask:0xf bank_mask:0xf\n\t"
      "v_mul_f32_dpp %7, %8, %12 row_newbcast:7 row_mask:0xf bank_mask:0xf"
      : "=&v"(u[0][0]), "=&v"(u[0][1]), "=&v"(u[1][0]), "=&v"(u[1][1]), "=&v"(u[2][0]),
        "=&v"(u[2][1]), "=&v"(u[3][0]), "=&v"(u[3][1])
      : "v"(r), "v"(bx[0]), "v"(bx[1]), "v"(bx[2]), "v"(bx[3]));
}
// y[s] = C_0 h[s][0] + C_1 h[s][1] (as fma(C_1, h_1, C_0 h_0)), C_j broadcast
// from lane 8 + 2s + j of r. The trailing s_nop covers DPP or permlane reads
// of y by the compiled code that follows.
__device__ __forceinline__ void bcast_dot_c(float (&y)[4], float r, const float (&h)[4][2]) {
  asm("s_nop 1\n\t"
      "v_mul_f32_dpp %0, %4, %5 row_newbcast:8 row_mask:0xf bank_mask:0xf\n\t"
      "v_mul_f32_dpp %1, %4, %7 row_newbcast:10 row_mask:0xf bank_mask:0xf\n\t"
      "v_mul_f32_dpp %2, %4, %9 row_newbcast:12 row_mask:0xf bank_mask:0xf\n\t"
      "v_mul_f32_dpp %3, %4, %11 row_newbcast:14 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %0, %4, %6 row_newbcast:9 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %1, %4, %8 row_newbcast:11 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %2, %4, %10 row_newbcast:13 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %3, %4, %12 row_newbcast:15 row_mask:0xf bank_mask:0xf\n\t"
      "s_nop 1"
      : "=&v"(y[0]), "=&v"(y[1]), "=&v"(y[2]), "=&v"(y[3])
      : "v"(r), "v"(h[0][0]), "v"(h[0][1]), "v"(h[1][0]), "v"(h[1][1]), "v"(h[2][0]),
        "v"(h[2][1]), "v"(h[3][0]), "v"(h[3][1]));
}
// The two pipeline buffers, then (two states per lane, ck: a launch that
// writes checkpoints) the checkpoint tiles of the two sub-chunk parities,
// [32 channels][NP + 2] each (rows of an odd number of float pairs: the 32
// lanes' 64-bit writes of a column hit 64 distinct banks). A launch without
// checkpoints never touches the tiles and is launched without them (the
// prefill: 5 blocks per CU at d_state 16 instead of 4).
__host__ __device__ constexpr int fwd_ck_row(int G, int NPL) { return 2 * G * NPL + 2; }
__host__ __device__ constexpr int fwd_lds_floats(int G, int NPL, bool ck = true) {
  return 2 * fwd_buf_floats(G, NPL) + (ck && NPL == 2 ? 2 * kCH * fwd_ck_row(G, NPL) : 0);
}

// KALIGNED: the checkpoint stride K is a multiple of 16, so checkpoints fall
// on sub-chunk ends (and the last one on the final state): no per-step tests.
// GATED: dt and Aneg come from the block's raw projections (see FwdArgs); the
// staging threads gate each dt once per block as they move it to LDS.
// PASS: what the kernel produces.
//   kPassFull:  y, checkpoints, final state.
//   kPassCarry: the carry pass of the time segments (see FwdArgs): blocks of
//               segments 0..nseg-2 scan their segment from zero and write
//               only its end state and sum of dt (no C, no y, no checkpoints).
//   kPassCkpt:  checkpoints only (no C, no y): the backward's recompute of
//               finer checkpoints for strides above its register window.
// ES: bytes per element of x, dt, B, C and y (4: fp32, 2: bf16).
constexpr int kPassFull = 0, kPassCarry = 1, kPassCkpt = 2;

template <int NPL, int G, int MINW, bool KALIGNED, bool GATED, int PASS = kPassFull, int ES = 4>
__global__ void __launch_bounds__(64 * G, MINW)
fwd_kernel(FwdArgs a) {
  constexpr bool FCARRY = PASS == kPassCarry;
  constexpr bool NOY = PASS != kPassFull;   // no C operand, no y
  constexpr int NT = 64 * G;                    // threads
  constexpr int NP = 2 * G * NPL;               // padded states
  constexpr int BUF = fwd_buf_floats(G, NPL);
  constexpr int TILE = bc_tile_floats(2 * G, NPL);   // one B or C tile (NPL 1, 4)
  constexpr int BCF = fwd_bc_floats(G, NPL);         // the B and C tiles
  constexpr bool BCAST = NPL == 2;                   // B, C by DPP row broadcasts
  constexpr int PER = (kCH * kQuads + NT - 1) / NT;
  constexpr int PERS = (kSteps * NP + NT - 1) / NT;
  extern __shared__ float lds[];
  const int N = a.N;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int hh = lane >> 5;
  const int c = lane & 31;
  const int q = wave * 2 + hh;
  const int n0 = q * NPL;
  const int b = blockIdx.y % a.batch;
  const int seg = blockIdx.y / a.batch;
  const int d0 = blockIdx.x * kCH;
  const int d = d0 + c;
  const bool act = d < a.D;
  const int T = a.T, D = a.D;
  const int t_beg = seg * a.seg_len;                      // this block's steps [t_beg, t_end)
  const int t_end = min(T, t_beg + a.seg_len);
  const int nsub = (t_end - t_beg + kSteps - 1) / kSteps;

  float a2[NPL], h[NPL];
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    float an = (act && n0 + j < N) ? a.aneg[(size_t)d * N + n0 + j] : 0.f;
    if constexpr (GATED) an = (act && n0 + j < N) ? softplus_f(an) : 0.f;
    a2[j] = -an * kLog2e;
    h[j] = 0.f;
  }

  const size_t row0 = (size_t)b * T;
  // Only the gated kernels read dt, B, C from column slices of a wider
  // tensor; the others keep compile-time-contiguous addressing.
  const int ld_dt = GATED ? a.ld_dt : D, ld_bc = GATED ? a.ld_bc : N;
  const QuadLoader<kCH, PER, ES> ql(tid, NT, D, d0, D);
  const QuadLoader<kCH, PER, ES> qdt(tid, NT, D, d0, ld_dt);
  const RowLoader<PERS, NPL, ES> rl(tid, NT, N, NP, ld_bc);
  const BCRowLoader<PERS, ES> rlb(tid, NT, N, NP, ld_bc);
  // Two staging register sets: set k & 1 holds sub-chunk k, loaded during
  // sub-chunk k - 3 and staged into LDS during sub-chunk k - 1.
  float4 px2[2][PER], pd2[2][PER];
  float pb2[2][PERS], pc2[2][PERS];
  float gbias[PER];   // GATED: the dt bias of each staging task's channel
  if constexpr (GATED) qdt.load_channel(gbias, a.dt_bias, d0);
  // Sub-chunk i of the segment (any i >= 0): its length (0 past the segment).
  const int last_len = t_end - t_beg - (nsub - 1) * kSteps;
  auto sub_len = [&](int i) { return i < nsub - 1 ? kSteps : i == nsub - 1 ? last_len : 0; };
  // Resources over sub-chunk i of the operands (channels d0 .. D-1 of the
  // (batch, T, D) ones, all N states of B and C; see SubStream).
  const size_t r0 = row0 + t_beg;
  const int il = nsub - 1;
  const SubStream<ES> sx(a.x, r0, D, d0, D, kSteps, 0, nsub, il, last_len);
  const SubStream<ES> sdt(a.dt, r0, ld_dt, d0, D, kSteps, 0, nsub, il, last_len);
  const SubStream<ES> sB(a.B, r0, ld_bc, 0, N, kSteps, 0, nsub, il, last_len);
  const SubStream<ES> sC(a.C, r0, ld_bc, 0, N, kSteps, 0, nsub, il, last_len);
  const SubStream<ES> sy(a.y != nullptr ? a.y : a.x, r0, D, d0, D, kSteps, 0,
                         a.y != nullptr ? nsub : 0, il, last_len);
  auto load_sub = [&](int i, auto set) {   // global -> staging registers
    constexpr int S = decltype(set)::value;
    ql.load(px2[S], sx.at(i));
    qdt.load(pd2[S], sdt.at(i));
    rl.load(pb2[S], sB.at(i));
    if constexpr (!NOY) rl.load(pc2[S], sC.at(i));
  };
  // FCARRY: the sum of dt over the segment, per staging task (the dt of 4
  // steps of one channel as staged), added over the channels' tasks at the
  // end: a quarter of the adds that every lane summing its steps would take.
  float sdt_part = 0.f;
  auto store_sub = [&](int i, auto set) {  // staging set i & 1 -> LDS buffer i & 1
    constexpr int S = decltype(set)::value;
    float4 (&px)[PER] = px2[S];
    float4 (&pd)[PER] = pd2[S];
    float (&pb)[PERS] = pb2[S];
    float (&pc)[PERS] = pc2[S];
    float* buf = lds + S * BUF;
    if constexpr (GATED) qdt.gate(pd, sub_len(i), a.dt_lo, a.dt_span, gbias);
    if constexpr (FCARRY) {
#pragma unroll
      for (int f = 0; f < PER; ++f) sdt_part += (pd[f].x + pd[f].y) + (pd[f].z + pd[f].w);
    }
    ql.store_cm(buf, pd);
    ql.store_cm_product(buf + kCH * kSteps, pd, px);
    if constexpr (BCAST) {
      rlb.store(buf + 2 * kCH * kSteps, pb, 0);
      if constexpr (!NOY) rlb.store(buf + 2 * kCH * kSteps, pc, 1);
    } else {
      rl.store(buf + 2 * kCH * kSteps, pb);
      if constexpr (!NOY) rl.store(buf + 2 * kCH * kSteps + TILE, pc);
    }
  };
  // y of sub-chunk i: every wave leaves, per channel and step, the sum over
  // its two half-waves (added in registers), in a step-pair-major tile
  // [8 pairs][32 channels][2] (each 64-bit write or read of a pair by 32
  // lanes is one contiguous, bank-conflict-free run); task (channel cc,
  // step pair p) sums those over the G waves in a fixed order. There are
  // 32 x 8 = 256 tasks: one per thread at G = 4. Split in two so that the LDS
  // reads (y_read) and their use (y_write) sit in different scheduling
  // regions.
  constexpr int YTASKS = kCH * kSteps / 2;
  constexpr int YT = (YTASKS + NT - 1) / NT;             // y tasks per thread
  float2 ypart[YT][G];
  auto y_read = [&](int par) {   // the y partials in LDS buffer par
    const float* yp = lds + par * BUF + 2 * kCH * kSteps + BCF;
#pragma unroll
    for (int f = 0; f < YT; ++f) {
      const int t0 = tid + f * NT;
      const int t = t0 < YTASKS ? t0 : 0;
      const int cc = t % kCH, p = t / kCH;
#pragma unroll
      for (int w = 0; w < G; ++w) ypart[f][w] = lds2(yp + w * kCH * kSteps + (p * kCH + cc) * 2);
    }
  };
  auto y_write = [&](int i) {
    const GBuf yo = sy.at(i);
#pragma unroll
    for (int f = 0; f < YT; ++f) {
      const int t0 = tid + f * NT;
      const bool ok = t0 < YTASKS;
      const int t = ok ? t0 : 0;
      const int cc = t % kCH, p = t / kCH;
      float2 sum = ypart[f][0];
#pragma unroll
      for (int q2 = 1; q2 < G; ++q2) {
        sum.x += ypart[f][q2].x;
        sum.y += ypart[f][q2].y;
      }
      const unsigned o =
          (ok && d0 + cc < D) ? (unsigned)ES * ((unsigned)(2 * p) * (unsigned)D + cc) : kOOB;
      st_elem<ES, kStream>(yo, sum.x, o);                // y: written once (NT)
      st_elem<ES, kStream>(yo, sum.y, o != kOOB ? o + (unsigned)ES * (unsigned)D : kOOB);
    }
  };

  // Prologue: sub-chunk 0 in LDS, sub-chunks 1 and 2 in the staging sets.
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  load_sub(0, I0{});
  store_sub(0, I0{});
  load_sub(1, I1{});
  load_sub(2, I0{});
  __syncthreads();

  // Checkpoints / final state: bounds-checked stores of the lane's states
  // (padded states and channels past d_inner are dropped). Each store gets a
  // resource over one (D, N) slice.
  const size_t ck_stride = (size_t)D * N;
  const unsigned slice_bytes = 4u * (unsigned)ck_stride;
  const unsigned ck_lane = act ? 4u * ((unsigned)d * (unsigned)N + (unsigned)n0) : kOOB;
  const int nvalid = N - n0;
  // A later segment starts from the checkpoint at its first step, or from
  // the state folded from the earlier segments' carries.
  if (seg > 0 && a.h_init != nullptr) {
    load_states<NPL>(h, GBuf(a.h_init + ((size_t)b * a.init_nchunk + t_beg / a.init_K - 1) *
                                            ck_stride, slice_bytes), ck_lane, nvalid);
  } else if (!FCARRY && seg > 0 && a.carryH != nullptr) {
    for (int s2 = 0; s2 < seg * a.cunits; ++s2) {
      const size_t slot = (size_t)s2 * a.batch + b;
      float hv[NPL];
      load_states<NPL>(hv, GBuf(a.carryH + slot * ck_stride, slice_bytes), ck_lane, nvalid);
      const float sdt = act ? a.carrySdt[slot * D + d] : 0.f;
#pragma unroll
      for (int j = 0; j < NPL; ++j) h[j] = __builtin_fmaf(exp2_hw(sdt * a2[j]), h[j], hv[j]);
    }
  }
#pragma unroll
  for (int j = 0; j < NPL; ++j) h[j] = opaque_copy(h[j]);   // h may come from a load
  constexpr int kDone = 0x7FFFFFFF;
  // Step count after the next checkpoint, and its slot.
  int next_ck = a.ckpt != nullptr ? min((t_beg / a.K + 1) * a.K, T) : kDone;
  const float* ck_base = a.ckpt != nullptr ? a.ckpt + (size_t)b * a.nchunk * ck_stride : a.aneg;
  const float* ck_ptr = ck_base + (size_t)(t_beg / a.K) * ck_stride;
  // Staged checkpoints (two states per lane, strides that are multiples of
  // 16): at the end of a sub-chunk each lane writes its states to the LDS
  // tile of the sub-chunk's parity, [32 channels][NP] (the (D, N) slice's
  // layout, rows CKR floats apart), and after the barrier (in quad 2 of the
  // next sub-chunk, away from quad 1's y stores: 49.6 -> 48.8 us at
  // 16x512x1536x16) thread t stores floats 2t and 2t + 1 of it to the
  // checkpoint: each wave writes 512 contiguous bytes, whole lines,
  // where the lanes' own stores (8 bytes every N floats) leave lines for the
  // caches to assemble from the 2G lane groups (measured at 16x512x1536x16:
  // forward 50.5 -> 49.9 us; 4x16384x2048x16 forward 824 -> 797 us).
  constexpr bool CKL = KALIGNED && NPL == 2 && PASS != kPassCarry;
  constexpr int CKR = fwd_ck_row(G, NPL);
  float* const ckt = lds + 2 * BUF;
  const float* ck_pend = nullptr;   // the checkpoint staged, not yet stored
  unsigned ck_off0 = kOOB, ck_off1 = kOOB;
  const int ck_rd = (2 * tid) / NP * CKR + (2 * tid) % NP;   // 2 * NT == kCH * NP
  {
    const int cc = (2 * tid) / NP, nn = (2 * tid) % NP;
    const bool okc = d0 + cc < D;
    ck_off0 = (okc && nn < N) ? 4u * (unsigned)((d0 + cc) * N + nn) : kOOB;
    ck_off1 = (okc && nn + 1 < N) ? 4u * (unsigned)((d0 + cc) * N + nn + 1) : kOOB;
  }
  auto flush_ck = [&](int par) {   // the staged checkpoint of parity par
    const float2 v = lds2(ckt + par * kCH * CKR + ck_rd);
    const GBuf g(ck_pend, slice_bytes);
    g.st(v.x, ck_off0);
    g.st(v.y, ck_off1);
    ck_pend = nullptr;
  };
  ProgressPriority prio(nsub);
  // Sub-chunk i, of parity P (a constant: the loop below is unrolled by two).
  auto iter = [&](int i, auto par) {
    constexpr int P = decltype(par)::value;
    prio.step(i);
    const int t0 = t_beg + i * kSteps;
    const float* buf = lds + P * BUF;
    const float* cDT = buf;
    const float* cBX = buf + kCH * kSteps;
    const float* gB = buf + 2 * kCH * kSteps + q * bc_group_floats(NPL);
    const float* gC = buf + 2 * kCH * kSteps + TILE + q * bc_group_floats(NPL);
    // BCAST: this lane's value of its group's broadcast tile
    const float* gBC = buf + 2 * kCH * kSteps + q * kBCGroup2 + (lane & 15);
    float* myY = lds + P * BUF + 2 * kCH * kSteps + BCF + wave * kCH * kSteps;

    // A quad's LDS operands, read one quad ahead of their use.
    float4 qdt, qbx, qB[NPL], qC[NPL];
    float qr;   // BCAST: B and C of the quad, one value per lane
    auto read_quad = [&](int m) {
      qdt = lds4(cDT + cm_quad(c, m));
      qbx = lds4(cBX + cm_quad(c, m));
      if constexpr (BCAST) {
        qr = gBC[16 * m];
      } else {
#pragma unroll
        for (int j = 0; j < NPL; ++j) {
          qB[j] = lds4(gB + 4 * m * NPL + 4 * j);
          if constexpr (!NOY) qC[j] = lds4(gC + 4 * m * NPL + 4 * j);
        }
      }
    };
    read_quad(0);

    // Steps past T in the last sub-chunk see zero inputs: dA = 1 and u = 0
    // there, so h passes through unchanged and nothing is stored.
#pragma unroll
    for (int m = 0; m < kQuads; ++m) {
      float dts[4], bxs[4], Bq[4][NPL], Cq[4][NPL];
      f4_to(dts, qdt);
      f4_to(bxs, qbx);
      float r = 0.f;
      if constexpr (BCAST) {
        r = qr;
      } else {
#pragma unroll
        for (int e = 0; e < 4 * NPL; ++e) {
          const float4 tb = qB[e / 4], tc = NOY ? tb : qC[e / 4];
          const float vb[4] = {tb.x, tb.y, tb.z, tb.w}, vc[4] = {tc.x, tc.y, tc.z, tc.w};
          Bq[e / NPL][e % NPL] = vb[e % 4];
          Cq[e / NPL][e % NPL] = vc[e % 4];
        }
      }
      if (m + 1 < kQuads) read_quad(m + 1);
      float da[4][NPL], u[4][NPL];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
#pragma unroll
        for (int j = 0; j < NPL; ++j) {
          da[s][j] = exp2_hw(dts[s] * a2[j]);
          if constexpr (!BCAST) u[s][j] = Bq[s][j] * bxs[s];
        }
      }
      if constexpr (BCAST) bcast_mul_b(u, r, bxs);
      float yq[4], hq[4][NPL];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < NPL; ++j) {
          h[j] = __builtin_fmaf(da[s][j], h[j], u[s][j]);
          if constexpr (!NOY && !BCAST) acc = __builtin_fmaf(Cq[s][j], h[j], acc);
          hq[s][j] = h[j];
        }
        yq[s] = acc;
      }
      if constexpr (!NOY && BCAST) bcast_dot_c(yq, r, hq);
      if constexpr (!NOY) {
        // Add the two half-waves (same channels, different states): lanes
        // 0-31 end with steps 0, 1 of the quad, lanes 32-63 with steps 2, 3.
        const auto s02 = __builtin_amdgcn_permlane32_swap(__float_as_uint(yq[0]),
                                                          __float_as_uint(yq[2]), false, false);
        const auto s13 = __builtin_amdgcn_permlane32_swap(__float_as_uint(yq[1]),
                                                          __float_as_uint(yq[3]), false, false);
        *reinterpret_cast<float2*>(myY + ((2 * m + hh) * kCH + c) * 2) =
            make_float2(__uint_as_float(s02[0]) + __uint_as_float(s02[1]),
                        __uint_as_float(s13[0]) + __uint_as_float(s13[1]));
      }

      // Pipeline work for the neighbouring sub-chunks, in this quad's
      // scheduling region. Unconditional: past either end of the sequence the
      // resources are empty (loads return 0, stores are dropped) and the LDS
      // buffer written is not read again.
      if (!NOY && m == 0) y_read(P ^ 1);
      if constexpr (CKL) {
        if (m == 2 && ck_pend != nullptr) flush_ck(P ^ 1);
      }
      if (!NOY && m == 1) y_write(i - 1);
      if (m == 1) store_sub(i + 1, std::integral_constant<int, P ^ 1>{});
      if (m == 2) load_sub(i + 3, std::integral_constant<int, P ^ 1>{});

      if constexpr (!KALIGNED) {
        // Checkpoints inside this quad (any stride; uniform tests per step).
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          if (i < nsub && t0 + 4 * m + s + 1 == next_ck) {
            store_states<NPL>(GBuf(ck_ptr, slice_bytes), ck_lane, nvalid, hq[s]);
            ck_ptr += ck_stride;
            next_ck = next_ck == T ? kDone : min(next_ck + a.K, T);
          }
        }
      }
      step_fence();
    }
    if constexpr (KALIGNED) {
      // A checkpoint at the end of this sub-chunk (uniform test; none in the
      // padding sub-chunk past the segment, whose end may be the position of
      // a checkpoint of the next segment).
      if (next_ck == t0 + kSteps && next_ck < T && i < nsub) {
        if constexpr (CKL) {
          *reinterpret_cast<float2*>(ckt + P * kCH * CKR + c * CKR + n0) = make_float2(h[0], h[1]);
          ck_pend = ck_ptr;
        } else {
          store_states<NPL>(GBuf(ck_ptr, slice_bytes), ck_lane, nvalid, h);
        }
        ck_ptr += ck_stride;
        next_ck += a.K;
      }
    }
    __syncthreads();
  };
  // Pairs of sub-chunks; an odd count is padded with sub-chunk nsub, whose
  // inputs are empty (identity steps: h passes through, nothing is stored).
  // A separate last iteration instead made the compiler copy the staging
  // registers of one set into another at every turn of the loop (10 VALU
  // per pair, and a wait for the loads that fill them).
  for (int i = 0; i < nsub; i += 2) {
    iter(i, I0{});
    iter(i + 1, I1{});
  }
  if constexpr (FCARRY) {
    const size_t slot = (size_t)seg * a.batch + b;
    store_states<NPL>(GBuf(a.carryH + slot * ck_stride, slice_bytes), ck_lane, nvalid, h);
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
  if constexpr (CKL) {
    if (ck_pend != nullptr) flush_ck((nsub - 1) & 1);   // the loop ended on a barrier
  }
  // KALIGNED: the last checkpoint (slot nchunk-1) is the state after step T-1,
  // which is h now in the last segment (steps past T are identity steps).
  const bool last_seg = t_end == T;
  if (KALIGNED && a.ckpt != nullptr && last_seg)
    store_states<NPL>(GBuf(ck_base + (size_t)(a.nchunk - 1) * ck_stride, slice_bytes), ck_lane,
                      nvalid, h);
  if (!NOY && (nsub & 1) == 0) {   // else the padding sub-chunk wrote it
    y_read((nsub - 1) & 1);
    y_write(nsub - 1);
  }

  if (a.h_last != nullptr && last_seg)
    store_states<NPL>(GBuf(a.h_last + (size_t)b * ck_stride, slice_bytes), ck_lane, nvalid, h);
}

}  // namespace mhs
