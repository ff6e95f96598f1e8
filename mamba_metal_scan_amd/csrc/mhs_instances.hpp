// The scan kernels' instantiations, listed once. mhs_capi.hip declares them
// `extern template` and takes their addresses; the mhs_kern_*.hip units define
// them, so that the four groups compile in parallel.
//
// Plans: NPL states per lane in {2, 4}, G waves in 1..8, MINW the
// waves-per-SIMD target (3 for NPL 2, 2 for NPL 4); and one state per lane
// for d_state 8 and 16 (G 4 and 8, 512-thread blocks at 16), MINW 4. ES:
// element bytes of the activations (4: fp32, 2: bf16).
#pragma once

#include "mhs_bwd.hpp"
#include "mhs_fwd.hpp"

#define MHS_FOR_PLANS(X, PREFIX, ES)                                                   \
  X(PREFIX, 2, 1, 3, ES) X(PREFIX, 2, 2, 3, ES) X(PREFIX, 2, 3, 3, ES)                 \
  X(PREFIX, 2, 4, 3, ES) X(PREFIX, 2, 5, 3, ES) X(PREFIX, 2, 6, 3, ES)                 \
  X(PREFIX, 2, 7, 3, ES) X(PREFIX, 2, 8, 3, ES)                                        \
  X(PREFIX, 4, 1, 2, ES) X(PREFIX, 4, 2, 2, ES) X(PREFIX, 4, 3, 2, ES)                 \
  X(PREFIX, 4, 4, 2, ES) X(PREFIX, 4, 5, 2, ES) X(PREFIX, 4, 6, 2, ES)                 \
  X(PREFIX, 4, 7, 2, ES) X(PREFIX, 4, 8, 2, ES)                                        \
  X(PREFIX, 1, 4, 4, ES) X(PREFIX, 1, 8, 4, ES)

// Forward: checkpoint stride aligned / any, ungated / gated; the carry pass
// of the time segments and the checkpoint-only pass (ungated / gated).
#define MHS_FWD_INST(PREFIX, NPL, G, MINW, ES)                                                   \
  PREFIX template __global__ void fwd_kernel<NPL, G, MINW, true, false, kPassFull, ES>(FwdArgs);  \
  PREFIX template __global__ void fwd_kernel<NPL, G, MINW, false, false, kPassFull, ES>(FwdArgs); \
  PREFIX template __global__ void fwd_kernel<NPL, G, MINW, true, true, kPassFull, ES>(FwdArgs);   \
  PREFIX template __global__ void fwd_kernel<NPL, G, MINW, false, true, kPassFull, ES>(FwdArgs);  \
  PREFIX template __global__ void fwd_kernel<NPL, G, MINW, true, false, kPassCarry, ES>(FwdArgs); \
  PREFIX template __global__ void fwd_kernel<NPL, G, MINW, true, true, kPassCarry, ES>(FwdArgs);  \
  PREFIX template __global__ void fwd_kernel<NPL, G, MINW, true, false, kPassCkpt, ES>(FwdArgs);  \
  PREFIX template __global__ void fwd_kernel<NPL, G, MINW, true, true, kPassCkpt, ES>(FwdArgs);

// Backward: ungated / gated, gradient pass / adjoint-carry pass; the
// gradient pass with the in-kernel sweep of the checkpoint stride 32
// (kSweepMax 16-step chunks per caller checkpoint), ungated / gated.
#define MHS_BWD_INST(PREFIX, NPL, G, MINW, ES)                                    \
  PREFIX template __global__ void bwd_kernel<NPL, G, MINW, false, false, ES>(BwdArgs); \
  PREFIX template __global__ void bwd_kernel<NPL, G, MINW, true, false, ES>(BwdArgs);  \
  PREFIX template __global__ void bwd_kernel<NPL, G, MINW, false, true, ES>(BwdArgs);  \
  PREFIX template __global__ void bwd_kernel<NPL, G, MINW, true, true, ES>(BwdArgs);   \
  PREFIX template __global__ void bwd_kernel<NPL, G, MINW, false, false, ES, false, kSweepMax>( \
      BwdArgs);                                                                              \
  PREFIX template __global__ void bwd_kernel<NPL, G, MINW, true, false, ES, false, kSweepMax>( \
      BwdArgs);

// Backward with fp32 atomics for dB, dC, dAneg and the dt bias: ungated /
// gated.
#define MHS_BWD_ATOM_INST(PREFIX, NPL, G, MINW, ES)                                    \
  PREFIX template __global__ void bwd_kernel<NPL, G, MINW, false, false, ES, true>(BwdArgs); \
  PREFIX template __global__ void bwd_kernel<NPL, G, MINW, true, false, ES, true>(BwdArgs);  \
  PREFIX template __global__ void bwd_kernel<NPL, G, MINW, false, false, ES, true, kSweepMax>( \
      BwdArgs);                                                                             \
  PREFIX template __global__ void bwd_kernel<NPL, G, MINW, true, false, ES, true, kSweepMax>( \
      BwdArgs);
