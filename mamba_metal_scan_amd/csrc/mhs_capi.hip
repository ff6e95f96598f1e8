// C ABI of the gfx950 selective scan (declared in include/mamba_hip_scan.h).
//
// Host-side responsibilities: argument validation, choice of the kernel
// variant for d_state, grid/LDS sizing, workspace carving, and HIP error
// reporting. No allocation happens here: every buffer comes from the caller
// (the Python layer takes it from torch's caching allocator).
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "mamba_hip_scan.h"
#include "mhs_bwd.hpp"
#include "mhs_fwd.hpp"
#include "mhs_step.hpp"

namespace {

constexpr int kVersion = (0 << 16) | (1 << 8) | 0;

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

// Forced state-lanes-per-wave (0 = automatic); see mhs_set_variant.
std::atomic<int> g_npl_override{0};

using FwdFn = void (*)(mhs::FwdArgs);
using BwdFn = void (*)(mhs::BwdArgs);

constexpr int kFwdKI = 16;
constexpr int kRows = 16;

struct Plan {
  int npl = 0;      // state lanes per wave
  int G = 0;        // waves per block (= N / npl)
  FwdFn fwd = nullptr;
  int fwd_lds = 0;  // bytes
  BwdFn bwd = nullptr;
  int bwd_ki = 0;   // largest chunk the backward walks directly
  int bwd_lds = 0;  // bytes
};

template <int NPL, int PER>
FwdFn fwd_fn() { return &mhs::fwd_kernel<NPL, kFwdKI, 16, PER, 1>; }

constexpr int kMaxLdsBytes = 160 * 1024;   // gfx950 LDS per workgroup

// Backward instantiations per state-lanes-per-wave, in order of preference:
// the larger register window (KI = 16) for up to 8 waves per block, a
// narrower one (KI = 8) for up to 16 waves. PER: tile float4s per thread.
struct BwdCand {
  int ki, maxg, rows;
  BwdFn narrow;   // for blocks of fewer than 4 waves
  BwdFn wide;     // for blocks of 4 or more waves
};

template <int NPL>
void bwd_cands(const BwdCand*& c, int& n) {
  static const BwdCand t[] = {
      {16, 8, kRows, &mhs::bwd_kernel<NPL, 16, 8, 4, 1, kRows>,
       &mhs::bwd_kernel<NPL, 16, 8, 1, 1, kRows>},
      {8, 16, (NPL == 4 ? 16 : 8), &mhs::bwd_kernel<NPL, 8, 16, 2, 1, (NPL == 4 ? 16 : 8)>,
       &mhs::bwd_kernel<NPL, 8, 16, 1, 1, (NPL == 4 ? 16 : 8)>},
  };
  c = t;
  n = 2;
}

bool plan_for(int N, int npl, Plan& p) {
  if (N % npl != 0) return false;
  const int G = N / npl;
  if (G < 1 || G > 16) return false;
  const bool narrow = G < 4;   // tile loads need more than one float4 per thread
  FwdFn fwd = nullptr;
  const BwdCand* cands = nullptr;
  int nc = 0;
  switch (npl) {
    case 4: fwd = narrow ? fwd_fn<4, 4>() : fwd_fn<4, 1>(); bwd_cands<4>(cands, nc); break;
    case 2: fwd = narrow ? fwd_fn<2, 4>() : fwd_fn<2, 1>(); bwd_cands<2>(cands, nc); break;
    case 1: fwd = narrow ? fwd_fn<1, 4>() : fwd_fn<1, 1>(); bwd_cands<1>(cands, nc); break;
    default: return false;
  }
  const int fwd_lds = mhs::fwd_lds_floats(kFwdKI, G, npl) * 4;
  if (fwd_lds > kMaxLdsBytes) return false;
  for (int i = 0; i < nc; ++i) {
    const BwdCand& c = cands[i];
    const int lds = mhs::bwd_lds_floats(c.ki, G, npl, c.rows) * 4;
    if (G > c.maxg || lds > kMaxLdsBytes) continue;
    if (narrow && c.ki * 16 > 64 * G * (c.ki == 16 ? 4 : 2)) continue;
    p.npl = npl;
    p.G = G;
    p.fwd = fwd;
    p.fwd_lds = fwd_lds;
    p.bwd = narrow ? c.narrow : c.wide;
    p.bwd_ki = c.ki;
    p.bwd_lds = lds;
    return true;
  }
  return false;
}

// Resolve the kernel variant for d_state N. Returns false if unsupported.
bool make_plan(int N, Plan& p) {
  if (N < 1 || N > MHS_MAX_DSTATE) return false;
  const int forced = g_npl_override.load(std::memory_order_relaxed);
  if (forced != 0 && plan_for(N, forced, p)) return true;
  // Automatic: the most state lanes per wave that still gives >= 4 waves.
  if (N % 4 == 0 && N / 4 >= 4 && plan_for(N, 4, p)) return true;
  if (N % 2 == 0 && N / 2 >= 4 && plan_for(N, 2, p)) return true;
  if (plan_for(N, 1, p)) return true;
  if (N % 2 == 0 && plan_for(N, 2, p)) return true;
  return N % 4 == 0 && plan_for(N, 4, p);
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

int check_shape(int64_t batch, int64_t seqlen, int64_t d_inner, int64_t d_state, int64_t chunk) {
  if (batch < 1 || seqlen < 1 || d_inner < 1 || d_state < 1)
    return fail(MHS_EINVAL, "sizes must be positive: batch %lld seqlen %lld d_inner %lld d_state %lld",
                (long long)batch, (long long)seqlen, (long long)d_inner, (long long)d_state);
  if (chunk < 1) return fail(MHS_EINVAL, "chunk must be >= 1, got %lld", (long long)chunk);
  if (batch > 65535) return fail(MHS_EINVAL, "batch %lld exceeds 65535", (long long)batch);
  if (seqlen > (1LL << 30) || d_inner > (1LL << 30))
    return fail(MHS_EINVAL, "seqlen / d_inner too large");
  if (d_state > MHS_MAX_DSTATE)
    return fail(MHS_EINVAL, "d_state %lld unsupported (max %d)", (long long)d_state, MHS_MAX_DSTATE);
  return MHS_OK;
}

size_t round_up(size_t n, size_t m) { return (n + m - 1) / m * m; }

struct WsLayout {
  size_t partB = 0, partC = 0, partA = 0, fine = 0, total = 0;  // offsets / bytes
};

WsLayout ws_layout(int64_t batch, int64_t T, int64_t D, int64_t N, int64_t chunk, int bwd_ki) {
  WsLayout w;
  const size_t nblk = (size_t)((D + 63) / 64);
  const size_t S = (size_t)batch * T * N;
  size_t off = 0;
  w.partB = off;
  off += round_up(nblk * S * 4, 256);
  w.partC = off;
  off += round_up(nblk * S * 4, 256);
  w.partA = off;
  off += round_up((size_t)batch * D * N * 4, 256);
  w.fine = off;
  if (chunk > bwd_ki) off += round_up((size_t)batch * ((T + bwd_ki - 1) / bwd_ki) * D * N * 4, 256);
  w.total = off;
  return w;
}

int launch_fwd(const Plan& p, const mhs::FwdArgs& a, int batch, hipStream_t s) {
  int rc = ensure_lds(reinterpret_cast<const void*>(p.fwd), p.fwd_lds);
  if (rc) return rc;
  const dim3 grid((unsigned)((a.D + 63) / 64), (unsigned)batch);
  hipLaunchKernelGGL(p.fwd, grid, dim3(64 * p.G), p.fwd_lds, s, a);
  return check_launch("forward scan kernel");
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
    return fail(MHS_EINVAL, "state lanes per wave must be 0 (auto), 1, 2 or 4; got %d", npl);
  g_npl_override.store(npl, std::memory_order_relaxed);
  return MHS_OK;
}

int64_t mhs_preferred_chunk(int64_t d_state) {
  Plan p;
  if (!make_plan((int)d_state, p)) return 0;
  return p.bwd_ki;
}

int mhs_scan_fwd_f32(const float* x, const float* dt, const float* aneg, const float* B,
                     const float* C, float* y, float* ckpt, float* h_last, int64_t batch,
                     int64_t seqlen, int64_t d_inner, int64_t d_state, int64_t chunk,
                     void* stream) {
  g_err[0] = '\0';
  int rc = check_shape(batch, seqlen, d_inner, d_state, chunk);
  if (rc) return rc;
  if (!x || !dt || !aneg || !B || !C) return fail(MHS_EINVAL, "null input pointer");
  const void* ptrs[] = {x, dt, aneg, B, C, y, ckpt, h_last};
  for (const void* q : ptrs)
    if (q && !aligned16(q)) return fail(MHS_EINVAL, "device pointers must be 16-byte aligned");
  Plan p;
  if (!make_plan((int)d_state, p)) return fail(MHS_EINVAL, "d_state %lld unsupported", (long long)d_state);
  mhs::FwdArgs a;
  a.x = x; a.dt = dt; a.aneg = aneg; a.B = B; a.C = C;
  a.y = y; a.ckpt = ckpt; a.h_last = h_last;
  a.T = (int)seqlen; a.D = (int)d_inner;
  a.K = (int)std::min<int64_t>(chunk, seqlen);
  a.nchunk = (int)mhs_num_chunks(seqlen, chunk);
  a.vec4 = (d_inner % 4 == 0) ? 1 : 0;
  return launch_fwd(p, a, (int)batch, static_cast<hipStream_t>(stream));
}

size_t mhs_scan_bwd_workspace_bytes(int64_t batch, int64_t seqlen, int64_t d_inner,
                                    int64_t d_state, int64_t chunk) {
  if (check_shape(batch, seqlen, d_inner, d_state, chunk)) return 0;
  Plan p;
  if (!make_plan((int)d_state, p)) return 0;
  return ws_layout(batch, seqlen, d_inner, d_state, chunk, p.bwd_ki).total;
}

int mhs_scan_bwd_f32(const float* x, const float* dt, const float* aneg, const float* B,
                     const float* C, const float* dy, const float* dh_last, const float* ckpt,
                     float* dx, float* ddt, float* daneg, float* dB, float* dC, void* workspace,
                     size_t workspace_bytes, int64_t batch, int64_t seqlen, int64_t d_inner,
                     int64_t d_state, int64_t chunk, void* stream) {
  g_err[0] = '\0';
  int rc = check_shape(batch, seqlen, d_inner, d_state, chunk);
  if (rc) return rc;
  if (!x || !dt || !aneg || !B || !C || !dy || !ckpt || !dx || !ddt || !daneg || !dB || !dC ||
      !workspace)
    return fail(MHS_EINVAL, "null pointer argument");
  const void* ptrs[] = {x, dt, aneg, B, C, dy, dh_last, ckpt, dx, ddt, daneg, dB, dC};
  for (const void* q : ptrs)
    if (q && !aligned16(q)) return fail(MHS_EINVAL, "device pointers must be 16-byte aligned");
  if (reinterpret_cast<uintptr_t>(workspace) & 255u)
    return fail(MHS_EINVAL, "workspace must be 256-byte aligned");
  Plan p;
  if (!make_plan((int)d_state, p)) return fail(MHS_EINVAL, "d_state %lld unsupported", (long long)d_state);
  const WsLayout w = ws_layout(batch, seqlen, d_inner, d_state, chunk, p.bwd_ki);
  if (workspace_bytes < w.total)
    return fail(MHS_EINVAL, "workspace too small: %zu < %zu bytes", workspace_bytes, w.total);
  hipStream_t s = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  const int T = (int)seqlen, D = (int)d_inner, N = (int)d_state;
  const int K = (int)std::min<int64_t>(chunk, seqlen);

  // Checkpoints at the backward's stride: the forward's own if chunk fits the
  // register window, else recomputed into the workspace at stride bwd_ki.
  const float* ck = ckpt;
  int Kb = K;
  if (K > p.bwd_ki) {
    mhs::FwdArgs f;
    f.x = x; f.dt = dt; f.aneg = aneg; f.B = B; f.C = C;
    f.y = nullptr;
    f.ckpt = reinterpret_cast<float*>(ws + w.fine);
    f.h_last = nullptr;
    f.T = T; f.D = D; f.K = p.bwd_ki;
    f.nchunk = (int)mhs_num_chunks(T, p.bwd_ki);
    f.vec4 = (D % 4 == 0) ? 1 : 0;
    rc = launch_fwd(p, f, (int)batch, s);
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
  a.batch = (int)batch; a.T = T; a.D = D; a.K = Kb;
  a.nchunk = (int)mhs_num_chunks(T, Kb);
  a.vec4 = (D % 4 == 0) ? 1 : 0;
  rc = ensure_lds(reinterpret_cast<const void*>(p.bwd), p.bwd_lds);
  if (rc) return rc;
  const dim3 grid((unsigned)((D + 63) / 64), (unsigned)batch);
  hipLaunchKernelGGL(p.bwd, grid, dim3(64 * p.G), p.bwd_lds, s, a);
  rc = check_launch("backward scan kernel");
  if (rc) return rc;

  const long long S = (long long)batch * T * N;
  const long long A = (long long)D * N;
  const long long total = S + A;
  const int blocks = (int)std::min<long long>((total + 255) / 256, 4096);
  hipLaunchKernelGGL(mhs::bwd_reduce_kernel, dim3(blocks), dim3(256), 0, s, a.wsB, a.wsC, a.wsA,
                     dB, dC, daneg, (D + 63) / 64, (int)batch, S, A);
  return check_launch("backward reduction kernel");
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
  if (d_state % 4 == 0 && d_state <= 16) {
    const long long threads = ch * 4;
    hipLaunchKernelGGL(mhs::step_kernel_vec, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                       s, h, x, dt, aneg, B, C, y, (int)batch, (int)d_inner, (int)d_state);
  } else {
    hipLaunchKernelGGL(mhs::step_kernel_any, dim3((unsigned)((ch + 255) / 256)), dim3(256), 0, s,
                       h, x, dt, aneg, B, C, y, (int)batch, (int)d_inner, (int)d_state);
  }
  return check_launch("decode step kernel");
}

}  // extern "C"
