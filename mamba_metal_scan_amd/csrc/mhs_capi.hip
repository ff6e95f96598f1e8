// C ABI of the gfx950 selective scan (declared in include/mamba_hip_scan.h).
//
// Host-side responsibilities: argument validation, choice of the kernel
// variant for d_state, grid/LDS sizing, workspace carving, and HIP error
// reporting. No allocation happens here: every buffer comes from the caller
// (the Python layer takes it from torch's caching allocator).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <initializer_list>
#include <mutex>
#include <numeric>

#include "mamba_hip_scan.h"
#include "mhs_bwd.hpp"
#include "mhs_conv.hpp"
#include "mhs_fwd.hpp"
#include "mhs_gate.hpp"
#include "mhs_instances.hpp"
#include "mhs_step.hpp"
#include "mhs_xent.hpp"
#include "mhs_norm.hpp"

// The scan kernels are instantiated in the mhs_kern_*.hip units.
namespace mhs {
MHS_FOR_PLANS(MHS_FWD_INST, extern, 4)
MHS_FOR_PLANS(MHS_FWD_INST, extern, 2)
MHS_FOR_PLANS(MHS_BWD_INST, extern, 4)
MHS_FOR_PLANS(MHS_BWD_INST, extern, 2)
MHS_FOR_PLANS(MHS_BWD_ATOM_INST, extern, 4)
MHS_FOR_PLANS(MHS_BWD_ATOM_INST, extern, 2)
}  // namespace mhs

namespace {

constexpr int kVersion = (0 << 16) | (7 << 8) | 0;   // 0.7: quad-broadcast B/C and DPP partner products in the backward

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(MHS_EHIP, "%s: %s", what, hipGetErrorString(e));
  return MHS_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Forced states per lane (0 = automatic); see mhs_set_variant.
std::atomic<int> g_npl_override{0};
// Forced number of backward time segments (0 = automatic); see mhs_set_time_segments.
std::atomic<int> g_seg_override{0};
// Reduction of the backward's sums over channels and (batch, time): see
// mhs_set_reduction (0 = automatic).
std::atomic<int> g_reduction{0};
constexpr int kRedFixed = 1, kRedAtomic = 2;
// The automatic choice, per shape: the fixed order where the backward runs in
// one time segment (the grid fills the GPU), atomics where it runs in several.
// Measured on MI355X (backward launch, same box):
//   16x512x1536x16, one segment:        fixed 126.1 us, atomics 145.4 us;
//   4x16384x2048x16, three segments:    fixed 1597 us,  atomics 1511 us.
// At the first the atomics cost more kernel time than the reduction kernel
// they replace (12 us); at the second the reduction kernel reads 64 channel
// blocks' partials of every (b, t, n), 537 MB in 116 us, more than the
// atomics cost.
bool atomic_reduction(bool segmented) {
  const int m = g_reduction.load(std::memory_order_relaxed);
  return m == 0 ? segmented : m == kRedAtomic;
}

constexpr int kDefaultCUs = 256; // MI355X compute units (used when no device can be queried)
constexpr int kMaxDevices = 64;
constexpr int kMaxSegments = 8;
constexpr int kMinSegChunks = 8; // automatic split: at least 8 chunks per segment

// Forced compute-unit count (0 = query the device); see mhs_set_cu_count.
std::atomic<int> g_cu_override{0};
std::atomic<int> g_cu_cache[kMaxDevices];   // per device, 0 until queried

// Compute units of the current device, queried once per device and cached
// (a partitioned MI355X exposes fewer than 256). Without a usable device the
// MI355X count, so that the host-side size queries still answer.
int device_cus() {
  const int forced = g_cu_override.load(std::memory_order_relaxed);
  if (forced > 0) return forced;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return kDefaultCUs;
  }
  if (dev >= 0 && dev < kMaxDevices) {
    const int cached = g_cu_cache[dev].load(std::memory_order_relaxed);
    if (cached > 0) return cached;
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      n <= 0) {
    (void)hipGetLastError();
    n = kDefaultCUs;
  }
  if (dev >= 0 && dev < kMaxDevices) g_cu_cache[dev].store(n, std::memory_order_relaxed);
  return n;
}

// Time segments for this shape (see FwdArgs in mhs_fwd.hpp and BwdArgs in
// mhs_bwd.hpp), in units of nch chunks (16-step sub-chunks in the forward,
// the backward's chunks in the backward). Automatic: one segment while the
// grid has at least two blocks per CU; below that, enough segments for about
// per_cu blocks per CU, each at least kMinSegChunks chunks long: the
// forward's carry pass costs more of its main pass than the backward's does,
// and the forward plans for kFwdBlocksPerCU, the backward for
// kBwdBlocksPerCU (measured on MI355X at 4x16384x2048x16, 256 blocks:
// forward 821 / 880 / 945 us and backward 1679 / 1597 / 1846 us with 2 / 3 /
// 4 segments). The carry
// passes run over carry units, cunits per segment, chosen so that their grid
// has about kCarryBlocksPerCU blocks per CU (a carry pass is a chain of
// dependent steps per state: it needs the waves to hide them), each at least
// kMinUnitChunks chunks long. Segments that start from exact states
// (carries = false) have no carry pass and a single unit each.
constexpr int kCarryBlocksPerCU = 4;
constexpr int kMinUnitChunks = 2;
constexpr int kFwdBlocksPerCU = 2, kBwdBlocksPerCU = 3;

struct Segments {
  int nseg = 1;    // segments
  int cps = 1;     // chunks per segment (the last may be shorter)
  int cunits = 1;  // carry units per segment
  int ups = 1;     // chunks per carry unit (cps = cunits * ups)
  int nunits = 1;  // carry units over the whole sequence
};

Segments segments_for(int64_t batch, int64_t D, int nch, int per_cu, bool carries = true) {
  Segments r;
  const int64_t blocks = batch * ((D + mhs::kCH - 1) / mhs::kCH);
  const int cus = device_cus();
  int want = g_seg_override.load(std::memory_order_relaxed);
  if (want == 0) {
    want = 1;
    if (blocks < 2 * (int64_t)cus) {
      want = (int)std::min<int64_t>(kMaxSegments, (per_cu * (int64_t)cus + blocks - 1) / blocks);
      want = std::max(1, std::min(want, nch / kMinSegChunks));
    }
  }
  want = std::max(1, std::min(want, nch));
  int cps = (nch + want - 1) / want;
  int nseg = (nch + cps - 1) / cps;    // no empty segment
  int f = 1;
  if (carries && nseg > 1) {
    f = (int)std::max<int64_t>(1, (int64_t)kCarryBlocksPerCU * cus / (blocks * (nseg - 1)));
    f = std::max(1, std::min(f, cps / kMinUnitChunks));
  }
  r.ups = (cps + f - 1) / f;
  r.cunits = f;
  r.cps = r.ups * f;
  r.nseg = (nch + r.cps - 1) / r.cps;
  r.nunits = (nch + r.ups - 1) / r.ups;
  if (r.nseg == 1) {   // no carries
    r.cunits = 1;
    r.ups = r.cps;
    r.nunits = 1;
  }
  return r;
}

using FwdFn = void (*)(mhs::FwdArgs);
using BwdFn = void (*)(mhs::BwdArgs);

constexpr int kKI = mhs::kSteps;           // backward register window (steps)
constexpr int kMaxLdsBytes = 160 * 1024;   // gfx950 LDS per workgroup
constexpr int kMaxG = 8;                   // waves per block

// The kernels of one plan for one activation element type.
struct Kernels {
  FwdFn fwd = nullptr;      // checkpoint stride a multiple of 16 (or >= T)
  FwdFn fwd_any = nullptr;  // any checkpoint stride
  FwdFn fwd_g = nullptr;    // the same two with the dt gate and softplus(A) fused
  FwdFn fwd_any_g = nullptr;
  FwdFn fcarry = nullptr;   // carry pass of the forward's time segments
  FwdFn fcarry_g = nullptr; // gated
  FwdFn fckpt = nullptr;    // checkpoints only (the backward's fine recompute)
  FwdFn fckpt_g = nullptr;  // gated
  BwdFn bwd = nullptr;
  BwdFn bwd_g = nullptr;    // gated
  BwdFn carry = nullptr;    // adjoint-carry pass of the time segments
  BwdFn carry_g = nullptr;  // gated
  BwdFn bwd_atom = nullptr;   // fp32 atomics for the reduced gradients
  BwdFn bwd_atom_g = nullptr; // gated
  // The same four gradient passes with the in-kernel sweep (checkpoint
  // strides of 2..kSweepMax 16-step chunks).
  BwdFn bwd_sw = nullptr, bwd_sw_g = nullptr, bwd_atom_sw = nullptr, bwd_atom_sw_g = nullptr;
  void (*reduce)(const float*, const float*, const float*, const float*, void*, void*, float*,
                 int, int, long long, long long, int, long long, const float*, float*,
                 int) = nullptr;
};

// Activation element types: x, dt, B, C, y, dy, dx, ddt, dB, dC in fp32 or
// bf16 (states, checkpoints, Aneg and all arithmetic stay fp32).
enum Elem { kF32 = 0, kBF16 = 1 };

struct Plan {
  int npl = 0;      // states per lane
  int G = 0;        // waves per block (d_state padded to 2*G*npl)
  Kernels k[2];     // by Elem
  int fwd_lds = 0;       // bytes, a launch that writes checkpoints
  int fwd_lds_nock = 0;  // bytes, one that does not (no checkpoint tiles)
  int bwd_ki = 0;   // largest chunk the backward walks directly
  int bwd_lds = 0;  // bytes, the gradient kernels
  int bwd_carry_lds = 0;  // bytes, the adjoint-carry kernels
  int bwd_sw_lds = 0;  // bytes, the swept kernels
};

// Kernel instantiations: NPL in {2, 4}, G in 1..8 (d_state up to 64).
// MINW is the waves-per-SIMD target the register budget is sized for: 3 for
// two states per lane (<= 168 VGPRs: at batch 16 x d_inner 1536 x d_state 16
// the grid is exactly 3 waves per SIMD), 2 for four (<= 256 VGPRs).
template <int NPL, int G, int MINW, int ES>
void fill_elem(Kernels& k) {
  k.fwd = &mhs::fwd_kernel<NPL, G, MINW, true, false, mhs::kPassFull, ES>;
  k.fwd_any = &mhs::fwd_kernel<NPL, G, MINW, false, false, mhs::kPassFull, ES>;
  k.fwd_g = &mhs::fwd_kernel<NPL, G, MINW, true, true, mhs::kPassFull, ES>;
  k.fwd_any_g = &mhs::fwd_kernel<NPL, G, MINW, false, true, mhs::kPassFull, ES>;
  k.fcarry = &mhs::fwd_kernel<NPL, G, MINW, true, false, mhs::kPassCarry, ES>;
  k.fcarry_g = &mhs::fwd_kernel<NPL, G, MINW, true, true, mhs::kPassCarry, ES>;
  k.fckpt = &mhs::fwd_kernel<NPL, G, MINW, true, false, mhs::kPassCkpt, ES>;
  k.fckpt_g = &mhs::fwd_kernel<NPL, G, MINW, true, true, mhs::kPassCkpt, ES>;
  k.bwd = &mhs::bwd_kernel<NPL, G, MINW, false, false, ES>;
  k.bwd_g = &mhs::bwd_kernel<NPL, G, MINW, true, false, ES>;
  k.carry = &mhs::bwd_kernel<NPL, G, MINW, false, true, ES>;
  k.carry_g = &mhs::bwd_kernel<NPL, G, MINW, true, true, ES>;
  k.bwd_atom = &mhs::bwd_kernel<NPL, G, MINW, false, false, ES, true>;
  k.bwd_atom_g = &mhs::bwd_kernel<NPL, G, MINW, true, false, ES, true>;
  k.bwd_sw = &mhs::bwd_kernel<NPL, G, MINW, false, false, ES, false, mhs::kSweepMax>;
  k.bwd_sw_g = &mhs::bwd_kernel<NPL, G, MINW, true, false, ES, false, mhs::kSweepMax>;
  k.bwd_atom_sw = &mhs::bwd_kernel<NPL, G, MINW, false, false, ES, true, mhs::kSweepMax>;
  k.bwd_atom_sw_g = &mhs::bwd_kernel<NPL, G, MINW, true, false, ES, true, mhs::kSweepMax>;
  k.reduce = &mhs::bwd_reduce_kernel<ES>;
}

template <int NPL, int G>
void fill(Plan& p) {
  constexpr int MINW = NPL == 1 ? 4 : NPL == 2 ? 3 : 2;
  fill_elem<NPL, G, MINW, 4>(p.k[kF32]);
  fill_elem<NPL, G, MINW, 2>(p.k[kBF16]);
  p.fwd_lds = mhs::fwd_lds_floats(G, NPL) * 4;
  p.fwd_lds_nock = mhs::fwd_lds_floats(G, NPL, false) * 4;
  p.bwd_lds = mhs::bwd_lds_floats(G, NPL, mhs::bwd_relabel(NPL, false),
                                   mhs::bwd_row_partial(NPL, false, 0), false) * 4;
  p.bwd_carry_lds = mhs::bwd_lds_floats(G, NPL, mhs::bwd_relabel(NPL, true),
                                         mhs::bwd_row_partial(NPL, true, 0), true) * 4;
  p.bwd_sw_lds = mhs::bwd_sweep_lds_floats(G, NPL) * 4;
}

template <int NPL>
bool fill_g(int G, Plan& p) {
  switch (G) {
    case 1: fill<NPL, 1>(p); break;
    case 2: fill<NPL, 2>(p); break;
    case 3: fill<NPL, 3>(p); break;
    case 4: fill<NPL, 4>(p); break;
    case 5: fill<NPL, 5>(p); break;
    case 6: fill<NPL, 6>(p); break;
    case 7: fill<NPL, 7>(p); break;
    case 8: fill<NPL, 8>(p); break;
    default: return false;
  }
  return true;
}

// One state per lane: plans for d_state 5..8 (G 4) and 9..16 (G 8) only.
bool fill_g1(int G, Plan& p) {
  switch (G) {
    case 4: fill<1, 4>(p); break;
    case 8: fill<1, 8>(p); break;
    default: return false;
  }
  return true;
}

bool plan_for(int N, int npl, Plan& p) {
  // One state per lane: the instantiated plans pad d_state to 8 or 16.
  const int G = npl == 1 ? (N <= 8 ? 4 : N <= 16 ? 8 : 0) : (N + 2 * npl - 1) / (2 * npl);
  if (G < 1 || G > kMaxG) return false;
  const bool ok = npl == 2 ? fill_g<2>(G, p) : npl == 4 ? fill_g<4>(G, p)
                  : npl == 1 ? fill_g1(G, p) : false;
  if (!ok) return false;
  p.npl = npl;
  p.G = G;
  p.bwd_ki = kKI;
  return p.fwd_lds <= kMaxLdsBytes && p.bwd_lds <= kMaxLdsBytes && p.bwd_sw_lds <= kMaxLdsBytes;
}

// Resolve the kernel variant for d_state N. Returns false if unsupported.
bool make_plan(int N, Plan& p) {
  if (N < 1 || N > MHS_MAX_DSTATE) return false;
  const int forced = g_npl_override.load(std::memory_order_relaxed);
  if (forced != 0) return plan_for(N, forced, p);
  // Automatic: two states per lane up to d_state 32 (more, thinner blocks),
  // four beyond.
  return plan_for(N, N <= 32 ? 2 : 4, p);
}

// Dynamic-LDS opt-in, once per kernel function.
std::mutex g_attr_mu;
int ensure_lds(const void* fn, int bytes) {
  static const void* done_fn[64];
  static int done_bytes[64];
  static int ndone = 0;
  std::lock_guard<std::mutex> lk(g_attr_mu);
  for (int i = 0; i < ndone; ++i)
    if (done_fn[i] == fn && done_bytes[i] >= bytes) return MHS_OK;
  const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e != hipSuccess) return fail(MHS_EHIP, "hipFuncSetAttribute(%d B LDS): %s", bytes, hipGetErrorString(e));
  if (ndone < 64) {
    done_fn[ndone] = fn;
    done_bytes[ndone] = bytes;
    ++ndone;
  }
  return MHS_OK;
}

// Dynamic LDS of a forward launch of nblocks blocks of `waves` waves that
// needs lds bytes. A block runs its whole sequence (or time segment), so the
// last round of a grid larger than the blocks the GPU holds at once lasts
// about as long as a full round however few blocks it has. Where the grid
// takes several rounds, the LDS is raised (never lowered) so that the blocks
// per CU minimise rounds x the waves per SIMD a round keeps busy, counted as
// at least 3 (below that one wave's issue latency, not the SIMD's VALU, sets
// a round's length). 32x2048x4096x16 prefill, 4096 blocks: 4 per CU in 4
// rounds instead of 5 per CU in 3.2, 891 against 925 us.
constexpr int kCuLdsBytes = 160 * 1024;   // gfx950 LDS per CU
int fwd_round_lds(const void* fn, int lds, long long nblocks, int waves) {
  struct Entry { const void* fn; int lds; long long nblocks; int waves, cus, out; };
  static Entry cache[32];
  static int ncache = 0, next = 0;
  static std::mutex mu;
  const int cus = device_cus();
  std::lock_guard<std::mutex> lk(mu);
  for (int i = 0; i < ncache; ++i) {
    const Entry& c = cache[i];
    if (c.fn == fn && c.lds == lds && c.nblocks == nblocks && c.waves == waves && c.cus == cus)
      return c.out;
  }
  auto occupancy = [&](int bytes) {
    int b = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, fn, 64 * waves, bytes) != hipSuccess) {
      (void)hipGetLastError();
      return 0;
    }
    return b;
  };
  int out = lds;
  const int bmax = occupancy(lds);
  if (bmax > 1 && nblocks > (long long)cus * bmax) {
    auto cost = [&](int b) {
      const long long per_round = (long long)cus * b;
      return (double)((nblocks + per_round - 1) / per_round) * std::max(b * waves / 4.0, 3.0);
    };
    int best = bmax;
    for (int b = bmax - 1; b >= 1; --b)
      if (cost(b) < cost(best)) best = b;
    // The smallest size, from just above the limit of best + 1 blocks, at
    // which the device holds best blocks per CU.
    for (int bytes = (std::max(lds, kCuLdsBytes / (best + 1) + 1) + 15) & ~15;
         best < bmax && bytes <= kCuLdsBytes / best; bytes += 256) {
      const int b = occupancy(bytes);
      if (b == best) {
        out = bytes;
        break;
      }
      if (b < best) break;
    }
  }
  cache[next] = Entry{fn, lds, nblocks, waves, cus, out};
  next = (next + 1) % 32;
  ncache = std::min(ncache + 1, 32);
  return out;
}

int check_shape(int64_t batch, int64_t seqlen, int64_t d_inner, int64_t d_state, int64_t chunk) {
  if (batch < 1 || seqlen < 1 || d_inner < 1 || d_state < 1)
    return fail(MHS_EINVAL, "sizes must be positive: batch %lld seqlen %lld d_inner %lld d_state %lld",
                (long long)batch, (long long)seqlen, (long long)d_inner, (long long)d_state);
  if (chunk < 1) return fail(MHS_EINVAL, "chunk must be >= 1, got %lld", (long long)chunk);
  if (batch > 65535) return fail(MHS_EINVAL, "batch %lld exceeds 65535", (long long)batch);
  if (seqlen > (1LL << 30)) return fail(MHS_EINVAL, "seqlen %lld too large", (long long)seqlen);
  if (d_state > MHS_MAX_DSTATE)
    return fail(MHS_EINVAL, "d_state %lld unsupported (max %d)", (long long)d_state, MHS_MAX_DSTATE);
  // Buffer resources address at most 2 GiB: one (d_inner, d_state) state
  // slice and 16 steps of one (T, d_inner) row must fit.
  if (d_inner > (1LL << 24) || d_inner * d_state * 4 >= (1LL << 31))
    return fail(MHS_EINVAL, "d_inner %lld x d_state %lld too large", (long long)d_inner,
                (long long)d_state);
  return MHS_OK;
}

size_t round_up(size_t n, size_t m) { return (n + m - 1) / m * m; }

// Backward workspace. Fixed-order reduction: per-block dB / dC partials
// (nblk, batch, T, N), per (segment, batch row) dAneg and dt-bias partials.
// Atomic reduction: fp32 dB / dC accumulators (batch, T, N) for bf16
// activations (fp32 ones accumulate into the outputs). Either way the
// time-segment carries and, for chunk > bwd_ki, the fine checkpoints.
struct WsLayout {
  size_t partB = 0, partC = 0, partA = 0, partDB = 0, carryL = 0, carryS = 0, fine = 0,
         total = 0;
  Segments sg;
  int nseg = 1;
  bool atomic = false;
};

// 16-step chunks per checkpoint when the backward sweeps them inside the
// kernel (an effective stride K = min(chunk, T) of 2..kSweepMax register
// windows, a multiple of the window), else 0.
int sweep_km(int64_t chunk, int64_t T, int bwd_ki) {
  const int64_t K = std::min<int64_t>(chunk, T);
  if (K <= bwd_ki || K % bwd_ki != 0 || K / bwd_ki > mhs::kSweepMax) return 0;
  return (int)(K / bwd_ki);
}

WsLayout ws_layout(int64_t batch, int64_t T, int64_t D, int64_t N, int64_t chunk, int bwd_ki) {
  WsLayout w;
  const size_t nblk = (size_t)((D + mhs::kCH - 1) / mhs::kCH);
  const size_t S = (size_t)batch * T * N;
  const int kb = (int)std::min<int64_t>(chunk, T) > bwd_ki ? bwd_ki : (int)std::min<int64_t>(chunk, T);
  const int km = sweep_km(chunk, T, bwd_ki);
  // Segments of the walk's chunks, the same as at stride bwd_ki (a segment
  // of the swept kernel may start inside a caller chunk).
  w.sg = segments_for(batch, D, (int)((T + kb - 1) / kb), kBwdBlocksPerCU);
  w.nseg = w.sg.nseg;
  w.atomic = atomic_reduction(w.nseg > 1);
  size_t off = 0;
  const size_t parts = w.atomic ? 1 : nblk;
  w.partB = off;
  off += round_up(parts * S * 4, 256);
  w.partC = off;
  off += round_up(parts * S * 4, 256);
  if (!w.atomic) {
    w.partA = off;
    off += round_up((size_t)w.nseg * batch * D * N * 4, 256);
    w.partDB = off;   // the gated backward's dt-bias partials
    off += round_up((size_t)w.nseg * batch * D * 4, 256);
  }
  if (w.nseg > 1) {   // carries per unit
    w.carryL = off;
    off += round_up((size_t)w.sg.nunits * batch * D * N * 4, 256);
    w.carryS = off;
    off += round_up((size_t)w.sg.nunits * batch * D * 4, 256);
  }
  w.fine = off;   // fine checkpoints: strides above the window that are not swept
  if (std::min<int64_t>(chunk, T) > bwd_ki && km == 0)
    off += round_up((size_t)batch * ((T + bwd_ki - 1) / bwd_ki) * D * N * 4, 256);
  w.total = off;
  return w;
}

// The block's dt gate (mamba_metal/model.py:197): dt = lo + span *
// sigmoid(raw + bias), bias the dt projection's (null: none); dbias, if not
// null, receives the backward's gradient of the bias.
struct Gate {
  bool on = false;
  float lo = 0.f, span = 0.f;
  const float* bias = nullptr;
  float* dbias = nullptr;
};

int check_gate(float dt_min, float dt_max, Gate& g) {
  if (!std::isfinite(dt_min) || !std::isfinite(dt_max) || !(dt_max > dt_min))
    return fail(MHS_EINVAL, "need finite dt_min < dt_max, got %g, %g", (double)dt_min,
                (double)dt_max);
  g.on = true;
  g.lo = dt_min;
  g.span = dt_max - dt_min;
  if (!(g.span > 0.f) || !std::isfinite(g.span))
    return fail(MHS_EINVAL, "dt_max - dt_min must be a positive finite float");
  return MHS_OK;
}

// One block per (channel block, batch row, time segment); a.seg_len and
// a.h_init describe the segments (see FwdArgs), nseg = 1 for the whole sequence.
// ckpt_only: the checkpoint-only pass (stride a multiple of 16; no C, no y).
int launch_fwd(const Plan& p, mhs::FwdArgs a, int batch, hipStream_t s, const Gate& g, Elem e,
               int nseg = 1, bool ckpt_only = false) {
  const Kernels& kk = p.k[e];
  const bool aligned = a.K % mhs::kSteps == 0 || a.K >= a.T;
  if (ckpt_only && !aligned) return fail(MHS_EINVAL, "checkpoint-only pass needs a stride of 16k");
  const FwdFn fn = ckpt_only ? (g.on ? kk.fckpt_g : kk.fckpt)
                   : aligned ? (g.on ? kk.fwd_g : kk.fwd) : (g.on ? kk.fwd_any_g : kk.fwd_any);
  a.dt_lo = g.lo;
  a.dt_span = g.span;
  a.dt_bias = g.bias;
  a.batch = batch;
  if (nseg == 1) {
    a.seg_len = a.T;
    a.h_init = nullptr;
  }
  const dim3 grid((unsigned)((a.D + mhs::kCH - 1) / mhs::kCH), (unsigned)(batch * nseg));
  const int lds = fwd_round_lds(reinterpret_cast<const void*>(fn),
                                a.ckpt != nullptr ? p.fwd_lds : p.fwd_lds_nock,
                                (long long)grid.x * grid.y, p.G);
  int rc = ensure_lds(reinterpret_cast<const void*>(fn), std::max(lds, p.fwd_lds));
  if (rc) return rc;
  hipLaunchKernelGGL(fn, grid, dim3(64 * p.G), lds, s, a);
  return check_launch("forward scan kernel");
}

// Workspace of the forward's time segments: carried end states and dt sums
// (see FwdArgs in mhs_fwd.hpp); total 0 when the shape runs unsegmented.
struct FwdWs {
  size_t carryH = 0, carryS = 0, total = 0;
  Segments sg;   // in sub-chunks of 16 steps
};

FwdWs fwd_ws_layout(int64_t batch, int64_t T, int64_t D, int64_t N) {
  FwdWs w;
  w.sg = segments_for(batch, D, (int)((T + mhs::kSteps - 1) / mhs::kSteps), kFwdBlocksPerCU);
  if (w.sg.nseg > 1) {   // carries of the units of segments 0..nseg-2
    const size_t units = (size_t)(w.sg.nseg - 1) * w.sg.cunits;
    w.carryH = 0;
    w.carryS = round_up(units * batch * D * N * 4, 256);
    w.total = w.carryS + round_up(units * batch * D * 4, 256);
  }
  return w;
}

// Row strides (elements between consecutive time steps) of dt, B/C, ddt and
// dB/dC; 0 means contiguous (D, N, D, N).
struct Strides {
  int64_t dt = 0, bc = 0, ddt = 0, dbc = 0;
};

int resolve_strides(const Strides& in, int64_t D, int64_t N, Strides& out) {
  out.dt = in.dt ? in.dt : D;
  out.bc = in.bc ? in.bc : N;
  out.ddt = in.ddt ? in.ddt : D;
  out.dbc = in.dbc ? in.dbc : N;
  if (out.dt < D || out.ddt < D || out.bc < N || out.dbc < N)
    return fail(MHS_EINVAL, "row strides must be at least d_inner (dt, ddt) and d_state (B, C, "
                "dB, dC); got %lld %lld %lld %lld", (long long)out.dt, (long long)out.bc,
                (long long)out.ddt, (long long)out.dbc);
  if (out.dt >= (1LL << 24) || out.ddt >= (1LL << 24) || out.bc >= (1LL << 24) ||
      out.dbc >= (1LL << 24))
    return fail(MHS_EINVAL, "row stride too large");
  return MHS_OK;
}

int scan_fwd(const void* x, const void* dt, const float* aneg, const void* B, const void* C,
             void* y, float* ckpt, float* h_last, void* workspace, size_t workspace_bytes,
             int64_t batch, int64_t seqlen, int64_t d_inner, int64_t d_state, int64_t chunk,
             void* stream, const Gate& g, Elem e, const Strides& st_in = Strides{}) {
  int rc = check_shape(batch, seqlen, d_inner, d_state, chunk);
  if (rc) return rc;
  if (!x || !dt || !aneg || !B || !C) return fail(MHS_EINVAL, "null input pointer");
  Strides st;
  rc = resolve_strides(st_in, d_inner, d_state, st);
  if (rc) return rc;
  const void* ptrs[] = {x, dt, aneg, B, C, y, ckpt, h_last};
  for (const void* q : ptrs)
    if (q && !aligned16(q)) return fail(MHS_EINVAL, "device pointers must be 16-byte aligned");
  Plan p;
  if (!make_plan((int)d_state, p)) return fail(MHS_EINVAL, "d_state %lld unsupported", (long long)d_state);
  mhs::FwdArgs a;
  a.x = x; a.dt = dt; a.aneg = aneg; a.B = B; a.C = C;
  a.y = y; a.ckpt = ckpt; a.h_last = h_last;
  a.T = (int)seqlen; a.D = (int)d_inner; a.N = (int)d_state;
  a.K = (int)std::min<int64_t>(chunk, seqlen);
  a.nchunk = (int)mhs_num_chunks(seqlen, chunk);
  a.ld_dt = (int)st.dt;
  a.ld_bc = (int)st.bc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const FwdWs w = fwd_ws_layout(batch, seqlen, d_inner, d_state);
  if (workspace == nullptr || w.sg.nseg == 1) return launch_fwd(p, a, (int)batch, s, g, e);
  if (workspace_bytes < w.total)
    return fail(MHS_EINVAL, "workspace too small: %zu < %zu bytes", workspace_bytes, w.total);
  if (reinterpret_cast<uintptr_t>(workspace) & 255u)
    return fail(MHS_EINVAL, "workspace must be 256-byte aligned");
  // Time segments: the carry pass over segments 0..nseg-2, then every
  // segment from its folded start state.
  char* ws = static_cast<char*>(workspace);
  a.batch = (int)batch;
  a.seg_len = w.sg.cps * mhs::kSteps;
  a.cunits = w.sg.cunits;
  a.h_init = nullptr;
  a.carryH = reinterpret_cast<float*>(ws + w.carryH);
  a.carrySdt = reinterpret_cast<float*>(ws + w.carryS);
  a.dt_lo = g.lo;
  a.dt_span = g.span;
  a.dt_bias = g.bias;
  const unsigned nblk = (unsigned)((d_inner + mhs::kCH - 1) / mhs::kCH);
  mhs::FwdArgs c = a;   // the carry pass: one "segment" per carry unit
  c.y = nullptr;
  c.ckpt = nullptr;
  c.h_last = nullptr;
  c.seg_len = w.sg.ups * mhs::kSteps;
  const Kernels& kk = p.k[e];
  const FwdFn cfn = g.on ? kk.fcarry_g : kk.fcarry;
  const dim3 cgrid(nblk, (unsigned)(batch * (w.sg.nseg - 1) * w.sg.cunits));
  const int clds = fwd_round_lds(reinterpret_cast<const void*>(cfn), p.fwd_lds_nock,
                                 (long long)cgrid.x * cgrid.y, p.G);
  rc = ensure_lds(reinterpret_cast<const void*>(cfn), std::max(clds, p.fwd_lds));
  if (rc) return rc;
  hipLaunchKernelGGL(cfn, cgrid, dim3(64 * p.G), clds, s, c);
  rc = check_launch("forward carry kernel");
  if (rc) return rc;
  const bool aligned = a.K % mhs::kSteps == 0 || a.K >= a.T;
  const FwdFn fn = aligned ? (g.on ? kk.fwd_g : kk.fwd) : (g.on ? kk.fwd_any_g : kk.fwd_any);
  const dim3 grid(nblk, (unsigned)(batch * w.sg.nseg));
  const int lds = fwd_round_lds(reinterpret_cast<const void*>(fn),
                                a.ckpt != nullptr ? p.fwd_lds : p.fwd_lds_nock,
                                (long long)grid.x * grid.y, p.G);
  rc = ensure_lds(reinterpret_cast<const void*>(fn), std::max(lds, p.fwd_lds));
  if (rc) return rc;
  hipLaunchKernelGGL(fn, grid, dim3(64 * p.G), lds, s, a);
  return check_launch("forward scan kernel");
}

}  // namespace

// ------------------------------------------------- allocation-free forward
//
// The device scratch of mhs_scan_fwd_noalloc_f32: what mhs_scan_fwd_ws_f32's
// workspace holds, the time segments' carried end states and dt sums. Every
// GPU the library runs on holds its own copy from module load until the
// process ends. In host code `scratch` names a host-side shadow, never device
// memory: launches take the address hipGetSymbolAddress returns for the
// current device (scratch_address), looked up once per device.
static __device__ __align__(256) unsigned char scratch[MHS_NOALLOC_SCRATCH_BYTES];

namespace {

std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices] = {};

// The current device's copy of `scratch`; the stream (if not NULL) must
// belong to that device.
int scratch_address(void* stream, void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(MHS_EHIP, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(MHS_EINVAL, "device %d: at most %d devices are supported", dev, kMaxDevices);
  if (stream != nullptr) {
    hipDevice_t sdev = -1;
    e = hipStreamGetDevice(static_cast<hipStream_t>(stream), &sdev);
    if (e != hipSuccess) return fail(MHS_EHIP, "hipStreamGetDevice: %s", hipGetErrorString(e));
    if (sdev != dev)
      return fail(MHS_EINVAL, "the stream belongs to device %d but device %d is current", sdev,
                  dev);
  }
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_dev[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(MHS_EHIP, "hipGetSymbolAddress(scratch) on device %d: %s", dev,
                  hipGetErrorString(e));
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return MHS_OK;
}

int scan_bwd(const void* x, const void* dt, const float* aneg, const void* B, const void* C,
             const void* dy, const float* dh_last, const float* ckpt, void* dx, void* ddt,
             float* daneg, void* dB, void* dC, void* workspace, size_t workspace_bytes,
             int64_t batch, int64_t seqlen, int64_t d_inner, int64_t d_state, int64_t chunk,
             void* stream, const Gate& g, Elem e, const Strides& st_in = Strides{}) {
  int rc = check_shape(batch, seqlen, d_inner, d_state, chunk);
  if (rc) return rc;
  if (!x || !dt || !aneg || !B || !C || !dy || !ckpt || !dx || !ddt || !daneg || !dB || !dC ||
      !workspace)
    return fail(MHS_EINVAL, "null pointer argument");
  Strides st;
  rc = resolve_strides(st_in, d_inner, d_state, st);
  if (rc) return rc;
  const void* ptrs[] = {x, dt, aneg, B, C, dy, dh_last, ckpt, dx, ddt, daneg, dB, dC};
  for (const void* q : ptrs)
    if (q && !aligned16(q)) return fail(MHS_EINVAL, "device pointers must be 16-byte aligned");
  if (reinterpret_cast<uintptr_t>(workspace) & 255u)
    return fail(MHS_EINVAL, "workspace must be 256-byte aligned");
  Plan p;
  if (!make_plan((int)d_state, p)) return fail(MHS_EINVAL, "d_state %lld unsupported", (long long)d_state);
  const int ch = mhs::kCH;
  const WsLayout w = ws_layout(batch, seqlen, d_inner, d_state, chunk, p.bwd_ki);
  if (workspace_bytes < w.total)
    return fail(MHS_EINVAL, "workspace too small: %zu < %zu bytes", workspace_bytes, w.total);
  hipStream_t s = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  const int T = (int)seqlen, D = (int)d_inner, N = (int)d_state;
  const int K = (int)std::min<int64_t>(chunk, seqlen);

  // Checkpoints at the backward's stride: the forward's own if chunk fits the
  // register window; for 2..kSweepMax windows the kernel sweeps the states
  // between the caller's checkpoints itself; else recomputed into the
  // workspace at stride bwd_ki.
  const float* ck = ckpt;
  int Kb = K;
  const int km = sweep_km(chunk, seqlen, p.bwd_ki);
  if (km > 0) {
    Kb = p.bwd_ki;
  } else if (K > p.bwd_ki) {
    mhs::FwdArgs f;
    f.x = x; f.dt = dt; f.aneg = aneg; f.B = B; f.C = C;
    f.y = nullptr;
    f.ckpt = reinterpret_cast<float*>(ws + w.fine);
    f.h_last = nullptr;
    f.T = T; f.D = D; f.N = N; f.K = p.bwd_ki;
    f.ld_dt = (int)st.dt;
    f.ld_bc = (int)st.bc;
    f.nchunk = (int)mhs_num_chunks(T, p.bwd_ki);
    // Time segments that start on the caller's checkpoints (stride K): each
    // is a multiple of lcm(16, K) steps and starts from the exact state, so
    // they run in parallel where the grid alone would leave CUs idle.
    const int64_t unit = std::lcm<int64_t>(mhs::kSteps, K);
    const Segments sg =
        segments_for(batch, D, (int)((T + unit - 1) / unit), kBwdBlocksPerCU, /*carries=*/false);
    const int nseg = sg.nseg;
    f.seg_len = (int)std::min<int64_t>((int64_t)sg.cps * unit, T);
    f.h_init = ckpt;
    f.init_K = K;
    f.init_nchunk = (int)mhs_num_chunks(T, K);
    rc = launch_fwd(p, f, (int)batch, s, g, e, nseg, /*ckpt_only=*/true);
    if (rc) return rc;
    ck = f.ckpt;
    Kb = p.bwd_ki;
  }

  mhs::BwdArgs a;
  a.x = x; a.dt = dt; a.aneg = aneg; a.B = B; a.C = C; a.dy = dy;
  a.dh_last = dh_last; a.ckpt = ck;
  a.dx = dx; a.ddt = ddt;
  a.wsB = reinterpret_cast<float*>(ws + w.partB);
  a.wsC = reinterpret_cast<float*>(ws + w.partC);
  a.wsA = reinterpret_cast<float*>(ws + w.partA);
  a.batch = (int)batch; a.T = T; a.D = D; a.N = N; a.K = Kb;
  a.nchunk = (int)mhs_num_chunks(T, Kb);
  a.km = km > 0 ? km : 1;
  a.ck_nchunk = km > 0 ? (int)mhs_num_chunks(T, K) : 0;
  a.dt_lo = g.lo;
  a.dt_span = g.span;
  a.dt_inv_span = g.on ? 1.f / g.span : 0.f;
  a.dt_bias = g.bias;
  a.wsDB = g.dbias != nullptr ? reinterpret_cast<float*>(ws + w.partDB) : nullptr;
  a.nseg = w.nseg;
  a.cps = w.sg.cps;
  a.cunits = w.sg.cunits;
  a.nunits = w.sg.nunits;
  a.carryL = w.nseg > 1 ? reinterpret_cast<float*>(ws + w.carryL) : nullptr;
  a.carrySdt = w.nseg > 1 ? reinterpret_cast<float*>(ws + w.carryS) : nullptr;
  a.ld_dt = (int)st.dt;
  a.ld_bc = (int)st.bc;
  a.ld_ddt = (int)st.ddt;
  const unsigned nblk = (unsigned)((D + ch - 1) / ch);
  const long long S = (long long)batch * T * N;
  const long long A = (long long)D * N;
  const int Dn = g.dbias != nullptr ? D : 0;
  if (w.atomic) {
    // The kernel adds into zeroed fp32 sums: the outputs themselves for fp32
    // activations, the workspace's accumulators for bf16 (rounded below).
    a.dB = e == kF32 ? static_cast<float*>(dB) : a.wsB;
    a.dC = e == kF32 ? static_cast<float*>(dC) : a.wsC;
    a.ld_dbc = e == kF32 ? (int)st.dbc : N;
    a.daneg = daneg;
    a.dbias = g.dbias;
    const long long n0 = S + A + Dn;
    hipLaunchKernelGGL(mhs::zero_grads_kernel<>, dim3((unsigned)std::min<long long>((n0 + 255) / 256, 2048)),
                       dim3(256), 0, s, a.dB, a.dC, (long long)batch * T, N, (long long)a.ld_dbc,
                       daneg, A, g.dbias, Dn);
    rc = check_launch("backward zero-fill kernel");
    if (rc) return rc;
  }
  if (w.nseg > 1) {
    // Adjoint carries of the units of segments 1..nseg-1 (segment 0 passes
    // nothing on): one block per unit.
    const BwdFn cfn = g.on ? p.k[e].carry_g : p.k[e].carry;
    rc = ensure_lds(reinterpret_cast<const void*>(cfn), p.bwd_carry_lds);
    if (rc) return rc;
    mhs::BwdArgs c = a;
    c.cps = w.sg.ups;
    hipLaunchKernelGGL(cfn, dim3(nblk, (unsigned)(batch * (w.sg.nunits - w.sg.cunits))),
                       dim3(64 * p.G), p.bwd_carry_lds, s, c);
    rc = check_launch("backward carry kernel");
    if (rc) return rc;
  }
  const Kernels& kk = p.k[e];
  const BwdFn fn = km > 0 ? (w.atomic ? (g.on ? kk.bwd_atom_sw_g : kk.bwd_atom_sw)
                                      : (g.on ? kk.bwd_sw_g : kk.bwd_sw))
                         : (w.atomic ? (g.on ? kk.bwd_atom_g : kk.bwd_atom)
                                     : (g.on ? kk.bwd_g : kk.bwd));
  const int lds_bytes = km > 0 ? p.bwd_sw_lds : p.bwd_lds;
  rc = ensure_lds(reinterpret_cast<const void*>(fn), lds_bytes);
  if (rc) return rc;
  hipLaunchKernelGGL(fn, dim3(nblk, (unsigned)(batch * w.nseg)), dim3(64 * p.G), lds_bytes, s, a);
  rc = check_launch("backward scan kernel");
  if (rc) return rc;

  if (w.atomic) {
    if (e == kF32) return MHS_OK;
    // bf16: round the fp32 sums to the bf16 outputs (one "block" of
    // partials, nothing else to reduce).
    const int blocks = (int)std::min<long long>((S + 255) / 256, 4096);
    hipLaunchKernelGGL(kk.reduce, dim3(blocks), dim3(256), 0, s, a.wsB, a.wsC, a.wsA, nullptr, dB,
                       dC, daneg, 1, 1, S, 0LL, N, (long long)st.dbc, nullptr, nullptr, 0);
    return check_launch("backward rounding kernel");
  }
  const long long total = S + A + Dn;
  const int blocks = (int)std::min<long long>((total + 255) / 256, 4096);
  hipLaunchKernelGGL(p.k[e].reduce, dim3(blocks), dim3(256), 0, s, a.wsB, a.wsC, a.wsA,
                     g.on ? aneg : nullptr, dB, dC, daneg, (D + ch - 1) / ch,
                     (int)batch * w.nseg, S, A, N, (long long)st.dbc, a.wsDB, g.dbias, Dn);
  return check_launch("backward reduction kernel");
}

}  // namespace

extern "C" {

int mhs_version(void) { return kVersion; }

const char* mhs_last_error(void) { return g_err; }

int64_t mhs_num_chunks(int64_t seqlen, int64_t chunk) {
  if (seqlen < 1 || chunk < 1) return 0;
  return (seqlen + chunk - 1) / chunk;
}

int mhs_set_variant(int npl) {
  if (npl != 0 && npl != 1 && npl != 2 && npl != 4)
    return fail(MHS_EINVAL, "states per lane must be 0 (auto), 1, 2 or 4; got %d", npl);
  g_npl_override.store(npl, std::memory_order_relaxed);
  return MHS_OK;
}

int mhs_set_time_segments(int segments) {
  if (segments < 0 || segments > kMaxSegments)
    return fail(MHS_EINVAL, "time segments must be 0 (auto) .. %d; got %d", kMaxSegments,
                segments);
  g_seg_override.store(segments, std::memory_order_relaxed);
  return MHS_OK;
}

int mhs_set_reduction(int mode) {
  if (mode != 0 && mode != kRedFixed && mode != kRedAtomic)
    return fail(MHS_EINVAL, "reduction mode must be 0 (auto), 1 (fixed order) or 2 (atomics); "
                "got %d", mode);
  g_reduction.store(mode, std::memory_order_relaxed);
  return MHS_OK;
}

int mhs_deterministic(void) {
  return g_reduction.load(std::memory_order_relaxed) == kRedFixed ? 1 : 0;
}

int mhs_scan_bwd_reduction(int64_t batch, int64_t seqlen, int64_t d_inner, int64_t d_state,
                           int64_t chunk) {
  if (check_shape(batch, seqlen, d_inner, d_state, chunk)) return 0;
  Plan p;
  if (!make_plan((int)d_state, p)) return 0;
  return ws_layout(batch, seqlen, d_inner, d_state, chunk, p.bwd_ki).atomic ? kRedAtomic
                                                                            : kRedFixed;
}

int mhs_set_cu_count(int cus) {
  if (cus < 0 || cus > 65536)
    return fail(MHS_EINVAL, "compute-unit count must be 0 (query the device) .. 65536; got %d",
                cus);
  g_cu_override.store(cus, std::memory_order_relaxed);
  return MHS_OK;
}

int mhs_cu_count(void) { return device_cus(); }

int64_t mhs_preferred_chunk(int64_t d_state) {
  Plan p;
  if (!make_plan((int)d_state, p)) return 0;
  return p.bwd_ki;
}

size_t mhs_scan_bwd_workspace_bytes(int64_t batch, int64_t seqlen, int64_t d_inner,
                                    int64_t d_state, int64_t chunk) {
  if (check_shape(batch, seqlen, d_inner, d_state, chunk)) return 0;
  Plan p;
  if (!make_plan((int)d_state, p)) return 0;
  return ws_layout(batch, seqlen, d_inner, d_state, chunk, p.bwd_ki).total;
}

int mhs_scan_fwd_f32(const float* x, const float* dt, const float* aneg, const float* B,
                     const float* C, float* y, float* ckpt, float* h_last, int64_t batch,
                     int64_t seqlen, int64_t d_inner, int64_t d_state, int64_t chunk,
                     void* stream) {
  g_err[0] = '\0';
  return scan_fwd(x, dt, aneg, B, C, y, ckpt, h_last, nullptr, 0, batch, seqlen, d_inner, d_state,
                  chunk, stream, Gate{}, kF32);
}

size_t mhs_scan_fwd_workspace_bytes(int64_t batch, int64_t seqlen, int64_t d_inner,
                                    int64_t d_state) {
  if (check_shape(batch, seqlen, d_inner, d_state, 1)) return 0;
  return fwd_ws_layout(batch, seqlen, d_inner, d_state).total;
}

int mhs_scan_fwd_ws_f32(const float* x, const float* dt, const float* aneg, const float* B,
                        const float* C, float* y, float* ckpt, float* h_last, void* workspace,
                        size_t workspace_bytes, int64_t batch, int64_t seqlen, int64_t d_inner,
                        int64_t d_state, int64_t chunk, void* stream) {
  g_err[0] = '\0';
  return scan_fwd(x, dt, aneg, B, C, y, ckpt, h_last, workspace, workspace_bytes, batch, seqlen,
                  d_inner, d_state, chunk, stream, Gate{}, kF32);
}

int mhs_scan_fwd_noalloc_f32(const float* x, const float* dt, const float* aneg, const float* B,
                             const float* C, float* y, float* ckpt, float* h_last, int64_t batch,
                             int64_t seqlen, int64_t d_inner, int64_t d_state, int64_t chunk,
                             void* stream) {
  g_err[0] = '\0';
  int rc = check_shape(batch, seqlen, d_inner, d_state, chunk);
  if (rc) return rc;
  const FwdWs w = fwd_ws_layout(batch, seqlen, d_inner, d_state);
  if (w.total > (size_t)MHS_NOALLOC_SCRATCH_BYTES)
    return fail(MHS_EINVAL, "the time segments of this shape need %zu bytes of scratch, more than "
                "the %zu-byte static scratch of mhs_scan_fwd_noalloc_f32; call "
                "mhs_scan_fwd_ws_f32 with a workspace", w.total,
                (size_t)MHS_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  if (w.total > 0) {
    rc = scratch_address(stream, &ws);
    if (rc) return rc;
  }
  // Every slot the segmented passes read is written by the carry pass of the
  // same call first: nothing in the scratch needs clearing.
  return scan_fwd(x, dt, aneg, B, C, y, ckpt, h_last, ws, w.total, batch, seqlen, d_inner,
                  d_state, chunk, stream, Gate{}, kF32);
}

int mhs_scan_bwd_f32(const float* x, const float* dt, const float* aneg, const float* B,
                     const float* C, const float* dy, const float* dh_last, const float* ckpt,
                     float* dx, float* ddt, float* daneg, float* dB, float* dC, void* workspace,
                     size_t workspace_bytes, int64_t batch, int64_t seqlen, int64_t d_inner,
                     int64_t d_state, int64_t chunk, void* stream) {
  g_err[0] = '\0';
  return scan_bwd(x, dt, aneg, B, C, dy, dh_last, ckpt, dx, ddt, daneg, dB, dC, workspace,
                  workspace_bytes, batch, seqlen, d_inner, d_state, chunk, stream, Gate{}, kF32);
}

int mhs_scan_gated_fwd_f32(const float* x, const float* dt_raw, const float* A, const float* B,
                           const float* C, float dt_min, float dt_max, const float* dt_bias,
                           float* y, float* ckpt,
                           float* h_last, void* workspace, size_t workspace_bytes, int64_t batch,
                           int64_t seqlen, int64_t d_inner, int64_t d_state, int64_t chunk,
                           int64_t ld_dt, int64_t ld_bc, void* stream) {
  g_err[0] = '\0';
  Gate g;
  const int rc = check_gate(dt_min, dt_max, g);
  if (rc) return rc;
  g.bias = dt_bias;
  return scan_fwd(x, dt_raw, A, B, C, y, ckpt, h_last, workspace, workspace_bytes, batch, seqlen,
                  d_inner, d_state, chunk, stream, g, kF32, Strides{ld_dt, ld_bc, 0, 0});
}

int mhs_scan_gated_bwd_f32(const float* x, const float* dt_raw, const float* A, const float* B,
                           const float* C, float dt_min, float dt_max, const float* dt_bias,
                           const float* dy, const float* dh_last, const float* ckpt, float* dx,
                           float* ddt_raw, float* dA, float* dB, float* dC, float* ddt_bias,
                           void* workspace,
                           size_t workspace_bytes, int64_t batch, int64_t seqlen, int64_t d_inner,
                           int64_t d_state, int64_t chunk, int64_t ld_dt, int64_t ld_bc,
                           int64_t ld_ddt, int64_t ld_dbc, void* stream) {
  g_err[0] = '\0';
  Gate g;
  const int rc = check_gate(dt_min, dt_max, g);
  if (rc) return rc;
  g.bias = dt_bias;
  g.dbias = ddt_bias;
  return scan_bwd(x, dt_raw, A, B, C, dy, dh_last, ckpt, dx, ddt_raw, dA, dB, dC, workspace,
                  workspace_bytes, batch, seqlen, d_inner, d_state, chunk, stream, g, kF32,
                  Strides{ld_dt, ld_bc, ld_ddt, ld_dbc});
}

int mhs_scan_fwd_bf16(const uint16_t* x, const uint16_t* dt, const float* aneg, const uint16_t* B,
                      const uint16_t* C, uint16_t* y, float* ckpt, float* h_last, void* workspace,
                      size_t workspace_bytes, int64_t batch, int64_t seqlen, int64_t d_inner,
                      int64_t d_state, int64_t chunk, void* stream) {
  g_err[0] = '\0';
  return scan_fwd(x, dt, aneg, B, C, y, ckpt, h_last, workspace, workspace_bytes, batch, seqlen,
                  d_inner, d_state, chunk, stream, Gate{}, kBF16);
}

int mhs_scan_bwd_bf16(const uint16_t* x, const uint16_t* dt, const float* aneg, const uint16_t* B,
                      const uint16_t* C, const uint16_t* dy, const float* dh_last,
                      const float* ckpt, uint16_t* dx, uint16_t* ddt, float* daneg, uint16_t* dB,
                      uint16_t* dC, void* workspace, size_t workspace_bytes, int64_t batch,
                      int64_t seqlen, int64_t d_inner, int64_t d_state, int64_t chunk,
                      void* stream) {
  g_err[0] = '\0';
  return scan_bwd(x, dt, aneg, B, C, dy, dh_last, ckpt, dx, ddt, daneg, dB, dC, workspace,
                  workspace_bytes, batch, seqlen, d_inner, d_state, chunk, stream, Gate{}, kBF16);
}

int mhs_scan_gated_fwd_bf16(const uint16_t* x, const uint16_t* dt_raw, const float* A,
                            const uint16_t* B, const uint16_t* C, float dt_min, float dt_max,
                            const float* dt_bias, uint16_t* y, float* ckpt, float* h_last, void* workspace,
                            size_t workspace_bytes, int64_t batch, int64_t seqlen,
                            int64_t d_inner, int64_t d_state, int64_t chunk, int64_t ld_dt,
                            int64_t ld_bc, void* stream) {
  g_err[0] = '\0';
  Gate g;
  const int rc = check_gate(dt_min, dt_max, g);
  if (rc) return rc;
  g.bias = dt_bias;
  return scan_fwd(x, dt_raw, A, B, C, y, ckpt, h_last, workspace, workspace_bytes, batch, seqlen,
                  d_inner, d_state, chunk, stream, g, kBF16, Strides{ld_dt, ld_bc, 0, 0});
}

int mhs_scan_gated_bwd_bf16(const uint16_t* x, const uint16_t* dt_raw, const float* A,
                            const uint16_t* B, const uint16_t* C, float dt_min, float dt_max,
                            const float* dt_bias, const uint16_t* dy, const float* dh_last,
                            const float* ckpt, uint16_t* dx, uint16_t* ddt_raw, float* dA,
                            uint16_t* dB, uint16_t* dC, float* ddt_bias, void* workspace, size_t workspace_bytes, int64_t batch,
                            int64_t seqlen, int64_t d_inner, int64_t d_state, int64_t chunk,
                            int64_t ld_dt, int64_t ld_bc, int64_t ld_ddt, int64_t ld_dbc,
                            void* stream) {
  g_err[0] = '\0';
  Gate g;
  const int rc = check_gate(dt_min, dt_max, g);
  if (rc) return rc;
  g.bias = dt_bias;
  g.dbias = ddt_bias;
  return scan_bwd(x, dt_raw, A, B, C, dy, dh_last, ckpt, dx, ddt_raw, dA, dB, dC, workspace,
                  workspace_bytes, batch, seqlen, d_inner, d_state, chunk, stream, g, kBF16,
                  Strides{ld_dt, ld_bc, ld_ddt, ld_dbc});
}

int mhs_scan_step_f32(float* h, const float* x, const float* dt, const float* aneg, const float* B,
                      const float* C, float* y, int64_t batch, int64_t d_inner, int64_t d_state,
                      void* stream) {
  g_err[0] = '\0';
  int rc = check_shape(batch, 1, d_inner, d_state, 1);
  if (rc) return rc;
  if (!h || !x || !dt || !aneg || !B || !C || !y) return fail(MHS_EINVAL, "null pointer argument");
  const void* ptrs[] = {h, x, dt, aneg, B, C, y};
  for (const void* q : ptrs)
    if (!aligned16(q)) return fail(MHS_EINVAL, "device pointers must be 16-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const long long ch = batch * d_inner;
  auto vec = [&](auto kernel, int lpc) {
    const long long threads = ch * lpc;
    hipLaunchKernelGGL(kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, h, x, dt,
                       aneg, B, C, y, (int)batch, (int)d_inner);
  };
  // One float4 of state per lane, d_state/4 lanes per channel (measured on
  // MI355X at 32 x 4096 x 16: 3.7 us/step, 5.0 TB/s; a whole channel per
  // lane runs at 2.1 TB/s).
  switch (d_state) {
    case 4: vec(mhs::step_kernel_vec<1, 1>, 1); break;
    case 8: vec(mhs::step_kernel_vec<1, 2>, 2); break;
    case 16: vec(mhs::step_kernel_vec<1, 4>, 4); break;
    case 32: vec(mhs::step_kernel_vec<1, 8>, 8); break;
    case 64: vec(mhs::step_kernel_vec<1, 16>, 16); break;
    default:
      hipLaunchKernelGGL(mhs::step_kernel_any, dim3((unsigned)((ch + 255) / 256)), dim3(256), 0, s,
                         h, x, dt, aneg, B, C, y, (int)batch, (int)d_inner, (int)d_state);
  }
  return check_launch("decode step kernel");
}

}  // extern "C"

// ------------------------------------------------------------- conv1d + SiLU

namespace {

constexpr int kConvTPT = 16;   // steps per thread

int check_conv(int64_t batch, int64_t seqlen, int64_t d_inner, int64_t k, int64_t x_rs) {
  if (batch < 1 || seqlen < 1 || d_inner < 1)
    return fail(MHS_EINVAL, "sizes must be positive: batch %lld seqlen %lld d_inner %lld",
                (long long)batch, (long long)seqlen, (long long)d_inner);
  if (k < 1 || k > mhs::kConvMaxK)
    return fail(MHS_EINVAL, "kernel_size %lld unsupported (1..%d)", (long long)k, mhs::kConvMaxK);
  if (x_rs < d_inner) return fail(MHS_EINVAL, "row stride %lld < d_inner %lld", (long long)x_rs,
                                  (long long)d_inner);
  if (batch > 65535) return fail(MHS_EINVAL, "batch %lld exceeds 65535", (long long)batch);
  if (seqlen > (1LL << 30) || d_inner > (1LL << 30)) return fail(MHS_EINVAL, "sizes too large");
  return MHS_OK;
}

dim3 conv_grid(int64_t batch, int64_t seqlen, int64_t d_inner) {
  return dim3((unsigned)((d_inner + mhs::kConvCh - 1) / mhs::kConvCh),
              (unsigned)((seqlen + mhs::kConvTG * kConvTPT - 1) / (mhs::kConvTG * kConvTPT)),
              (unsigned)batch);
}

template <int K>
void conv_fwd_launch(const float* x, long long x_rs, const float* w, const float* bias, float* out,
                     dim3 grid, int T, int D, hipStream_t s) {
  hipLaunchKernelGGL((mhs::conv_silu_fwd_kernel<K, kConvTPT>), grid, dim3(mhs::kConvCh * mhs::kConvTG),
                     0, s, x, x_rs, w, bias, out, T, D);
}
template <int K>
void conv_bwd_launch(const float* x, long long x_rs, const float* w, const float* bias,
                     const float* dout, float* dx, long long dx_rs, float* wsp, dim3 grid, int T,
                     int D, hipStream_t s) {
  hipLaunchKernelGGL((mhs::conv_silu_bwd_kernel<K, kConvTPT>), grid,
                     dim3(mhs::kConvCh * mhs::kConvTG), 0, s, x, x_rs, w, bias, dout, dx, dx_rs,
                     wsp, T, D);
}

}  // namespace

extern "C" {

int mhs_conv1d_silu_fwd_f32(const float* x, int64_t x_row_stride, const float* w,
                            const float* bias, float* out, int64_t batch, int64_t seqlen,
                            int64_t d_inner, int64_t kernel_size, void* stream) {
  g_err[0] = '\0';
  int rc = check_conv(batch, seqlen, d_inner, kernel_size, x_row_stride);
  if (rc) return rc;
  if (!x || !w || !bias || !out) return fail(MHS_EINVAL, "null pointer argument");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid = conv_grid(batch, seqlen, d_inner);
  const int T = (int)seqlen, D = (int)d_inner;
  switch (kernel_size) {
    case 1: conv_fwd_launch<1>(x, x_row_stride, w, bias, out, grid, T, D, s); break;
    case 2: conv_fwd_launch<2>(x, x_row_stride, w, bias, out, grid, T, D, s); break;
    case 3: conv_fwd_launch<3>(x, x_row_stride, w, bias, out, grid, T, D, s); break;
    case 4: conv_fwd_launch<4>(x, x_row_stride, w, bias, out, grid, T, D, s); break;
    case 5: conv_fwd_launch<5>(x, x_row_stride, w, bias, out, grid, T, D, s); break;
    case 6: conv_fwd_launch<6>(x, x_row_stride, w, bias, out, grid, T, D, s); break;
    case 7: conv_fwd_launch<7>(x, x_row_stride, w, bias, out, grid, T, D, s); break;
    default: conv_fwd_launch<8>(x, x_row_stride, w, bias, out, grid, T, D, s); break;
  }
  return check_launch("conv1d+silu forward kernel");
}

size_t mhs_conv1d_silu_bwd_workspace_bytes(int64_t batch, int64_t seqlen, int64_t d_inner,
                                           int64_t kernel_size) {
  if (check_conv(batch, seqlen, d_inner, kernel_size, d_inner)) return 0;
  const dim3 grid = conv_grid(batch, seqlen, d_inner);
  return (size_t)grid.y * grid.z * (size_t)(kernel_size + 1) * (size_t)d_inner * 4;
}

int mhs_conv1d_silu_bwd_f32(const float* x, int64_t x_row_stride, const float* w,
                            const float* bias, const float* dout, float* dx, int64_t dx_row_stride,
                            float* dw, float* dbias, void* workspace, size_t workspace_bytes,
                            int64_t batch, int64_t seqlen, int64_t d_inner, int64_t kernel_size,
                            void* stream) {
  g_err[0] = '\0';
  int rc = check_conv(batch, seqlen, d_inner, kernel_size, x_row_stride);
  if (rc) return rc;
  const long long dx_rs = dx_row_stride ? dx_row_stride : d_inner;
  if (dx_rs < d_inner) return fail(MHS_EINVAL, "dx row stride %lld < d_inner %lld", dx_rs,
                                   (long long)d_inner);
  if (!x || !w || !bias || !dout || !dx || !dw || !dbias || !workspace)
    return fail(MHS_EINVAL, "null pointer argument");
  const size_t need = mhs_conv1d_silu_bwd_workspace_bytes(batch, seqlen, d_inner, kernel_size);
  if (workspace_bytes < need)
    return fail(MHS_EINVAL, "workspace too small: %zu < %zu bytes", workspace_bytes, need);
  if (reinterpret_cast<uintptr_t>(workspace) & 15u)
    return fail(MHS_EINVAL, "workspace must be 16-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid = conv_grid(batch, seqlen, d_inner);
  const int T = (int)seqlen, D = (int)d_inner;
  float* wsp = static_cast<float*>(workspace);
  switch (kernel_size) {
    case 1: conv_bwd_launch<1>(x, x_row_stride, w, bias, dout, dx, dx_rs, wsp, grid, T, D, s); break;
    case 2: conv_bwd_launch<2>(x, x_row_stride, w, bias, dout, dx, dx_rs, wsp, grid, T, D, s); break;
    case 3: conv_bwd_launch<3>(x, x_row_stride, w, bias, dout, dx, dx_rs, wsp, grid, T, D, s); break;
    case 4: conv_bwd_launch<4>(x, x_row_stride, w, bias, dout, dx, dx_rs, wsp, grid, T, D, s); break;
    case 5: conv_bwd_launch<5>(x, x_row_stride, w, bias, dout, dx, dx_rs, wsp, grid, T, D, s); break;
    case 6: conv_bwd_launch<6>(x, x_row_stride, w, bias, dout, dx, dx_rs, wsp, grid, T, D, s); break;
    case 7: conv_bwd_launch<7>(x, x_row_stride, w, bias, dout, dx, dx_rs, wsp, grid, T, D, s); break;
    default: conv_bwd_launch<8>(x, x_row_stride, w, bias, dout, dx, dx_rs, wsp, grid, T, D, s); break;
  }
  rc = check_launch("conv1d+silu backward kernel");
  if (rc) return rc;
  const int K = (int)kernel_size;
  const int n = (K + 1) * D;
  hipLaunchKernelGGL(mhs::conv_reduce_kernel, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, s,
                     wsp, dw, dbias, (int)(grid.y * grid.z), K, D);
  return check_launch("conv1d+silu reduction kernel");
}

}  // extern "C"

// ------------------------------------------------------------- output gate

extern "C" {

int mhs_out_gate_fwd_f32(const float* y, const float* d_skip, const float* z, int64_t z_row_stride,
                         float* out, int64_t batch, int64_t seqlen, int64_t d_inner,
                         void* stream) {
  g_err[0] = '\0';
  int rc = check_conv(batch, seqlen, d_inner, 1, z_row_stride);
  if (rc) return rc;
  if (!y || !d_skip || !z || !out) return fail(MHS_EINVAL, "null pointer argument");
  const dim3 grid = conv_grid(batch, seqlen, d_inner);
  hipLaunchKernelGGL(mhs::out_gate_fwd_kernel<kConvTPT>, grid, dim3(mhs::kConvCh * mhs::kConvTG),
                     0, static_cast<hipStream_t>(stream), y, d_skip, z, (long long)z_row_stride,
                     out, (int)seqlen, (int)d_inner);
  return check_launch("output gate forward kernel");
}

size_t mhs_out_gate_bwd_workspace_bytes(int64_t batch, int64_t seqlen, int64_t d_inner) {
  if (check_conv(batch, seqlen, d_inner, 1, d_inner)) return 0;
  const dim3 grid = conv_grid(batch, seqlen, d_inner);
  return (size_t)grid.y * grid.z * (size_t)d_inner * 4;
}

int mhs_out_gate_bwd_f32(const float* y, const float* d_skip, const float* z, int64_t z_row_stride,
                         const float* dout, float* dy, float* dz, int64_t dz_row_stride,
                         float* dd_skip, void* workspace, size_t workspace_bytes, int64_t batch,
                         int64_t seqlen, int64_t d_inner, void* stream) {
  g_err[0] = '\0';
  int rc = check_conv(batch, seqlen, d_inner, 1, z_row_stride);
  if (rc) return rc;
  const long long dz_rs = dz_row_stride ? dz_row_stride : d_inner;
  if (dz_rs < d_inner) return fail(MHS_EINVAL, "dz row stride %lld < d_inner %lld", dz_rs,
                                   (long long)d_inner);
  if (!y || !d_skip || !z || !dout || !dy || !dz || !dd_skip || !workspace)
    return fail(MHS_EINVAL, "null pointer argument");
  const size_t need = mhs_out_gate_bwd_workspace_bytes(batch, seqlen, d_inner);
  if (workspace_bytes < need)
    return fail(MHS_EINVAL, "workspace too small: %zu < %zu bytes", workspace_bytes, need);
  if (reinterpret_cast<uintptr_t>(workspace) & 15u)
    return fail(MHS_EINVAL, "workspace must be 16-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid = conv_grid(batch, seqlen, d_inner);
  float* wsp = static_cast<float*>(workspace);
  const int D = (int)d_inner;
  hipLaunchKernelGGL(mhs::out_gate_bwd_kernel<kConvTPT>, grid, dim3(mhs::kConvCh * mhs::kConvTG),
                     0, s, y, d_skip, z, (long long)z_row_stride, dout, dy, dz, dz_rs, wsp,
                     (int)seqlen, D);
  rc = check_launch("output gate backward kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(mhs::conv_reduce_kernel, dim3((unsigned)((D + 3) / 4)), dim3(256), 0, s, wsp,
                     nullptr, dd_skip, (int)(grid.y * grid.z), 0, D);
  return check_launch("output gate reduction kernel");
}

}  // extern "C"

// ------------------------------------------------------------- cross-entropy

namespace {

int check_xent(const float* logits, const int64_t* targets, int64_t rows, int64_t vocab) {
  if (rows < 0 || vocab < 1)
    return fail(MHS_EINVAL, "rows must be >= 0 and vocab >= 1; got %lld, %lld", (long long)rows,
                (long long)vocab);
  if (rows > 0x7FFFFFFF) return fail(MHS_EINVAL, "rows %lld exceeds 2^31 - 1", (long long)rows);
  if (rows > 0 && (!logits || !targets)) return fail(MHS_EINVAL, "null pointer argument");
  return MHS_OK;
}

}  // namespace

extern "C" {

int mhs_xent_fwd_f32(const float* logits, const int64_t* targets, float* lse, float* loss_rows,
                     int64_t rows, int64_t vocab, int64_t ignore_index, void* stream) {
  g_err[0] = '\0';
  int rc = check_xent(logits, targets, rows, vocab);
  if (rc) return rc;
  if (rows == 0) return MHS_OK;
  if (!lse || !loss_rows) return fail(MHS_EINVAL, "null pointer argument");
  const auto* t = reinterpret_cast<const long long*>(targets);
  const bool vec = vocab % 4 == 0 && aligned16(logits);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (vec)
    hipLaunchKernelGGL(mhs::xent_fwd_kernel<4>, dim3((unsigned)rows), dim3(mhs::kXentThreads), 0,
                       s, logits, t, lse, loss_rows, (long long)vocab, (long long)ignore_index);
  else
    hipLaunchKernelGGL(mhs::xent_fwd_kernel<1>, dim3((unsigned)rows), dim3(mhs::kXentThreads), 0,
                       s, logits, t, lse, loss_rows, (long long)vocab, (long long)ignore_index);
  return check_launch("cross-entropy forward kernel");
}

int mhs_xent_bwd_f32(const float* logits, const int64_t* targets, const float* lse,
                     const float* scale, float* dlogits, int64_t rows, int64_t vocab,
                     int64_t ignore_index, void* stream) {
  g_err[0] = '\0';
  int rc = check_xent(logits, targets, rows, vocab);
  if (rc) return rc;
  if (rows == 0) return MHS_OK;
  if (!lse || !scale || !dlogits) return fail(MHS_EINVAL, "null pointer argument");
  if (dlogits == logits) return fail(MHS_EINVAL, "dlogits may not alias logits");
  const auto* t = reinterpret_cast<const long long*>(targets);
  const bool vec = vocab % 4 == 0 && aligned16(logits) && aligned16(dlogits);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (vec)
    hipLaunchKernelGGL(mhs::xent_bwd_kernel<4>, dim3((unsigned)rows), dim3(mhs::kXentThreads), 0,
                       s, logits, t, lse, scale, dlogits, (long long)vocab,
                       (long long)ignore_index);
  else
    hipLaunchKernelGGL(mhs::xent_bwd_kernel<1>, dim3((unsigned)rows), dim3(mhs::kXentThreads), 0,
                       s, logits, t, lse, scale, dlogits, (long long)vocab,
                       (long long)ignore_index);
  return check_launch("cross-entropy backward kernel");
}

}  // extern "C"

// ------------------------------------------------------------------- RMSNorm

namespace {

// Rows of cols features: cols a multiple of 4 in [4, 256 * kNormMaxNV],
// rows < 2^31, 16-byte aligned pointers.
int check_norm(int64_t rows, int64_t cols, std::initializer_list<const void*> ptrs) {
  if (rows < 0 || cols < 4 || cols % 4 != 0 || cols > 256 * mhs::kNormMaxNV)
    return fail(MHS_EINVAL, "rows must be >= 0 and cols a multiple of 4 in [4, %d]; got %lld, %lld",
                256 * mhs::kNormMaxNV, (long long)rows, (long long)cols);
  if (rows > 0x7FFFFFFF) return fail(MHS_EINVAL, "rows %lld exceeds 2^31 - 1", (long long)rows);
  for (const void* q : ptrs) {
    if (!q) return fail(MHS_EINVAL, "null pointer argument");
    if (!aligned16(q)) return fail(MHS_EINVAL, "device pointers must be 16-byte aligned");
  }
  return MHS_OK;
}

int64_t norm_bwd_blocks(int64_t rows) {
  return std::min<int64_t>((rows + 3) / 4, mhs::kNormBwdBlocks);
}

// The norm kernels' operands: forward (x, delta or null, w -> y, x_out,
// rstd), backward (dy = a, x = b, w, rstd, dres -> dx = out, partials = aux).
struct NormArgs {
  const float *a, *b, *w, *rstd, *dres;
  float *out, *out2, *aux;
  int rows, cols;
  float eps;
};

enum NormKind { kNormFwd, kNormAddFwd, kNormBwd };

template <int NV>
void launch_norm(NormKind k, const NormArgs& n, unsigned blocks, hipStream_t s) {
  const dim3 g(blocks), t(mhs::kNormThreads);
  if (k == kNormBwd)
    hipLaunchKernelGGL(mhs::rmsnorm_bwd_kernel<NV>, g, t, 0, s, n.a, n.b, n.w, n.rstd, n.dres,
                       n.out, n.aux, n.rows, n.cols);
  else if (k == kNormAddFwd)
    hipLaunchKernelGGL((mhs::rmsnorm_fwd_kernel<NV, true>), g, t, 0, s, n.a, n.b, n.w, n.out,
                       n.out2, n.aux, n.rows, n.cols, n.eps);
  else
    hipLaunchKernelGGL((mhs::rmsnorm_fwd_kernel<NV, false>), g, t, 0, s, n.a, nullptr, n.w,
                       n.out, nullptr, n.aux, n.rows, n.cols, n.eps);
}

// The kernel instance for cols features (NV float4 per lane).
void dispatch_norm(NormKind k, const NormArgs& n, unsigned blocks, hipStream_t s) {
  static_assert(mhs::kNormMaxNV == 8, "one case per NV");
  switch ((n.cols + 255) / 256) {
    case 1: launch_norm<1>(k, n, blocks, s); break;
    case 2: launch_norm<2>(k, n, blocks, s); break;
    case 3: launch_norm<3>(k, n, blocks, s); break;
    case 4: launch_norm<4>(k, n, blocks, s); break;
    case 5: launch_norm<5>(k, n, blocks, s); break;
    case 6: launch_norm<6>(k, n, blocks, s); break;
    case 7: launch_norm<7>(k, n, blocks, s); break;
    default: launch_norm<8>(k, n, blocks, s); break;
  }
}

int norm_fwd(const float* x, const float* delta, const float* weight, float* x_out, float* y,
             float* rstd, int64_t rows, int64_t cols, float eps, void* stream) {
  g_err[0] = '\0';
  if (!(eps >= 0.f) || eps == INFINITY)
    return fail(MHS_EINVAL, "eps must be finite and >= 0; got %g", (double)eps);
  if (rows == 0) return check_norm(rows, cols, {});
  int rc = check_norm(rows, cols, {x, weight, y, rstd});
  if (rc) return rc;
  if (delta) {
    rc = check_norm(rows, cols, {delta, x_out});
    if (rc) return rc;
    if (x_out == x || x_out == delta || x_out == y)
      return fail(MHS_EINVAL, "x_out may not alias x, delta or y");
    if (y == delta) return fail(MHS_EINVAL, "y may not alias delta");
  }
  if (y == x) return fail(MHS_EINVAL, "y may not alias x");
  const unsigned blocks = (unsigned)std::min<int64_t>((rows + 3) / 4, 8 * 1024);
  NormArgs n{x, delta, weight, nullptr, nullptr, y, x_out, rstd, (int)rows, (int)cols, eps};
  dispatch_norm(delta ? kNormAddFwd : kNormFwd, n, blocks, static_cast<hipStream_t>(stream));
  return check_launch("RMSNorm forward kernel");
}

}  // namespace

extern "C" {

int mhs_rmsnorm_fwd_f32(const float* x, const float* weight, float* y, float* rstd, int64_t rows,
                        int64_t cols, float eps, void* stream) {
  return norm_fwd(x, nullptr, weight, nullptr, y, rstd, rows, cols, eps, stream);
}

int mhs_add_rmsnorm_fwd_f32(const float* x, const float* delta, const float* weight,
                            float* x_out, float* y, float* rstd, int64_t rows, int64_t cols,
                            float eps, void* stream) {
  if (rows > 0 && !delta) {
    g_err[0] = '\0';
    return fail(MHS_EINVAL, "null pointer argument");
  }
  return norm_fwd(x, delta, weight, x_out, y, rstd, rows, cols, eps, stream);
}

size_t mhs_rmsnorm_bwd_workspace_bytes(int64_t rows, int64_t cols) {
  if (rows < 0 || cols < 0) return 0;
  return round_up((size_t)norm_bwd_blocks(rows) * (size_t)cols * 4, 256);
}

int mhs_rmsnorm_bwd_f32(const float* dy, const float* x, const float* weight, const float* rstd,
                        const float* dres, float* dx, float* dweight, void* workspace,
                        size_t workspace_bytes, int64_t rows, int64_t cols, void* stream) {
  g_err[0] = '\0';
  int rc = check_norm(rows, cols, {weight, dweight});
  if (rc) return rc;
  if (rows > 0) {
    rc = check_norm(rows, cols, {dy, x, rstd, dx});
    if (rc) return rc;
    if (dres && !aligned16(dres))
      return fail(MHS_EINVAL, "device pointers must be 16-byte aligned");
    if (dx == x || dx == dy) return fail(MHS_EINVAL, "dx may alias only dres");
  }
  const size_t need = mhs_rmsnorm_bwd_workspace_bytes(rows, cols);
  if (need > 0 && (!workspace || workspace_bytes < need))
    return fail(MHS_EINVAL, "workspace too small: %zu < %zu bytes", workspace_bytes, need);
  if (workspace && (reinterpret_cast<uintptr_t>(workspace) & 255u))
    return fail(MHS_EINVAL, "workspace must be 256-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  float* part = static_cast<float*>(workspace);
  const int64_t P = norm_bwd_blocks(rows);
  if (P > 0) {
    NormArgs n{dy, x, weight, rstd, dres, dx, nullptr, part, (int)rows, (int)cols, 0.f};
    dispatch_norm(kNormBwd, n, (unsigned)P, s);
    rc = check_launch("RMSNorm backward kernel");
    if (rc) return rc;
  }
  // dweight: the partial rows summed in a fixed order (zeros for rows == 0)
  const unsigned rblocks = (unsigned)((cols / 4 + mhs::kNormReduceCols - 1) / mhs::kNormReduceCols);
  hipLaunchKernelGGL(mhs::rmsnorm_dw_reduce_kernel, dim3(rblocks), dim3(256), 0, s, part, dweight,
                     (int)P, (int)cols);
  return check_launch("RMSNorm weight-gradient reduction kernel");
}

}  // extern "C"
