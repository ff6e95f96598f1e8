/*
 * mamba_hip_scan.h -- C ABI of the MI355X (gfx950) fused diagonal selective scan.
 *
 * The recurrence (mamba_metal/scan.py:13-15 in the reference):
 *
 *     dA[t,d,n] = exp(-dt[t,d] * Aneg[d,n])
 *     h[t,d,n]  = dA[t,d,n] * h[t-1,d,n] + dt[t,d] * B[t,n] * x[t,d]      h[-1] = 0
 *     y[t,d]    = sum_n C[t,n] * h[t,d,n]
 *
 * Every pointer is a DEVICE pointer to contiguous row-major float32:
 *     x, dt, y, dy, dx, ddt : (batch, seqlen, d_inner)
 *     B, C, dB, dC          : (batch, seqlen, d_state)
 *     aneg, daneg           : (d_inner, d_state)          (Aneg > 0, e.g. softplus(A))
 *     ckpt                  : (batch, ceil(seqlen/chunk), d_inner, d_state),
 *                             h at the END of every chunk of `chunk` steps
 *     h_last, dh_last       : (batch, d_inner, d_state)   (h at t = seqlen-1)
 *
 * All pointers must be 16-byte aligned (torch allocations are). The caller
 * owns every buffer, as the reference's autograd Function allocates every
 * output (scan.py:373-375 and :401-405). Work is enqueued asynchronously on
 * `stream` (a hipStream_t; NULL = the legacy default stream). Functions return 0
 * or an MHS_E* code; mhs_last_error() gives a message for the calling thread.
 * Entry points may be called concurrently from several threads / streams: no
 * buffer is shared between calls (except the static scratch of
 * mhs_scan_fwd_noalloc_f32, see there).
 */
#ifndef MAMBA_HIP_SCAN_H
#define MAMBA_HIP_SCAN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MHS_OK 0
#define MHS_EINVAL 1   /* bad argument: null pointer, size, d_state unsupported */
#define MHS_EHIP 2     /* a HIP runtime call or kernel launch failed */

/* Largest supported d_state; every d_state in [1, MHS_MAX_DSTATE] is supported
 * (padded internally with zero states). The reference's Metal kernels
 * require d_state % 4 == 0 (scan.py:274-276). Also required: d_inner <= 2^24
 * and d_inner * d_state * 4 < 2^31. */
#define MHS_MAX_DSTATE 64

/* Library version, (major << 16) | (minor << 8) | patch. */
int mhs_version(void);

/* Message describing the last failure on the calling thread ("" if none). */
const char* mhs_last_error(void);

/* Number of checkpoint slots the forward writes: ceil(seqlen / chunk). */
int64_t mhs_num_chunks(int64_t seqlen, int64_t chunk);

/* The largest checkpoint stride the backward walks directly (its register
 * window, 16 steps); 0 if d_state is unsupported. Any chunk >= 1 is correct.
 * A stride of 2 windows (32) is swept inside the backward kernel: it
 * rebuilds the states between the caller's checkpoints itself, with no extra
 * workspace. Other strides above the window (the reference's own 64 among
 * them) cost one extra forward pass inside mhs_scan_bwd_f32 and stride-16
 * checkpoints in its workspace (the faster choice from 3 windows on). No
 * counterpart in the reference (its stride is the module constant
 * SSM_CHUNK, mamba_metal/scan.py:58). */
int64_t mhs_preferred_chunk(int64_t d_state);

/* Tuning knob, process-wide: force the number of d_state entries each GPU
 * lane carries per channel (1, 2 or 4; 0 restores the automatic choice: 2 up
 * to d_state 32, 4 above). With 2, d_state above 32 becomes unsupported; with
 * 1, d_state above 16 (d_state is padded to 8 or 16). No
 * counterpart in the reference (its Metal kernels keep all d_state entries of
 * a channel in one thread, scan.py:67-69). */
int mhs_set_variant(int states_per_lane);

/* Tuning knob, process-wide: the number of time segments the forward (with
 * a workspace) and the backward split the sequence into (1..8; 0 restores the
 * automatic choice: one segment while the grid has at least two blocks of 32
 * channels per compute unit, otherwise enough segments of at least 128 steps
 * for about two blocks per compute unit in the forward and three in the
 * backward, at most 8). Segments run in parallel after a short pass that
 * carries the state (forward) or the adjoint (backward) across segment
 * boundaries, over carry units of each segment sized for about four blocks
 * per compute unit; results equal the unsegmented scan up to rounding. The
 * workspace sizes depend on it. No counterpart in the reference (its kernels
 * walk each channel's whole sequence in one thread, scan.py:78-127,
 * :132-261). */
int mhs_set_time_segments(int segments);

/* The compute-unit count the automatic time-segment choice plans for: the
 * current device's (hipDeviceAttributeMultiprocessorCount, queried once per
 * device; 256, MI355X's count, when no device can be queried), unless forced.
 * mhs_set_cu_count forces it process-wide (1..65536; 0 restores the query),
 * for tests and tuning; like the other knobs it is read when a call is made,
 * and the workspace sizes depend on it. No counterpart in the reference. */
int mhs_set_cu_count(int cus);
int mhs_cu_count(void);

/* How the backward reduces its sums over channels (dB, dC) and over batch and
 * time (dAneg, the gated dt-bias gradient), process-wide, read when a call is
 * made (the workspace size depends on it):
 *   1  fixed order: per-block partials in the workspace, added by a reduction
 *      kernel in a fixed order; bit-for-bit reproducible run to run.
 *   2  fp32 atomics: each block adds its (wave64 DPP/permlane + LDS reduced)
 *      sums into the zeroed gradients with device-scope fp32 atomics, as the
 *      reference's kernel does (mamba_metal/scan.py:237-245); no partials and
 *      no reduction kernel, a far smaller workspace, and a rounding that
 *      varies with the order the additions land in (about 1e-7 relative of
 *      each sum: far inside the 1e-4 parity bar).
 *   0  automatic, per shape: 1 where the backward runs in one time segment
 *      (the grid fills the GPU), 2 where it runs in several; each measured
 *      the faster there on MI355X.
 * mhs_deterministic() is 1 when the current setting reproduces bit for bit
 * at every shape (mode 1). mhs_scan_bwd_reduction() returns the mode (1 or
 * 2) a backward of this shape uses under the current setting, 0 for a shape
 * the backward rejects. */
int mhs_set_reduction(int mode);
int mhs_deterministic(void);
int mhs_scan_bwd_reduction(int64_t batch, int64_t seqlen, int64_t d_inner, int64_t d_state,
                           int64_t chunk);

/*
 * Forward scan. Replaces the reference's `lib.ssm_fwd(x, dt, Aneg, Bm, Cm, y,
 * ckpt, Bt, T, D, Kc)` launch (mamba_metal/scan.py:78-127, launched at :377-378).
 *
 *   y      : written (may be NULL: then only ckpt / h_last are produced)
 *   ckpt   : written if non-NULL; checkpoint stride `chunk` (>= 1)
 *   h_last : written if non-NULL (the state after the last step; the reference
 *            returns ckpt[:, -1] for this, scan.py:381-387)
 */
int mhs_scan_fwd_f32(const float* x, const float* dt, const float* aneg,
                     const float* B, const float* C,
                     float* y, float* ckpt, float* h_last,
                     int64_t batch, int64_t seqlen, int64_t d_inner, int64_t d_state,
                     int64_t chunk, void* stream);

/* Bytes of device workspace mhs_scan_fwd_ws_f32 (and the gated forward)
 * can use for this shape: 0 when the forward runs as one time segment (grids
 * of at least two blocks of 32 channels per compute unit), else the carried
 * states of its time segments (see mhs_set_time_segments). */
size_t mhs_scan_fwd_workspace_bytes(int64_t batch, int64_t seqlen, int64_t d_inner,
                                    int64_t d_state);

/*
 * mhs_scan_fwd_f32 with a workspace (>= mhs_scan_fwd_workspace_bytes bytes,
 * 256-byte aligned, contents irrelevant; NULL = none). With it, grids too small
 * for the GPU run as time segments: a pass that scans segments 0..S-2 from a
 * zero state and keeps their end states and dt sums, then all S segments at
 * once, each from the state folded from the earlier ones. Same outputs up to
 * rounding. No counterpart in the reference (its forward runs each channel's
 * whole sequence in one thread, scan.py:78-127).
 */
int mhs_scan_fwd_ws_f32(const float* x, const float* dt, const float* aneg,
                        const float* B, const float* C,
                        float* y, float* ckpt, float* h_last,
                        void* workspace, size_t workspace_bytes,
                        int64_t batch, int64_t seqlen, int64_t d_inner, int64_t d_state,
                        int64_t chunk, void* stream);

/*
 * mhs_scan_fwd_ws_f32 without a workspace argument and without any
 * allocation: the time segments' carries live in a static device array of
 * MHS_NOALLOC_SCRATCH_BYTES (16 MiB) that every GPU the library runs on holds
 * from module load until the process ends. No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). It calls no
 * hipMalloc / hipFree. Same arguments (minus the workspace), outputs and
 * kernels as mhs_scan_fwd_ws_f32. Shapes whose carries need more than the
 * static scratch (mhs_scan_fwd_workspace_bytes > MHS_NOALLOC_SCRATCH_BYTES)
 * fail with MHS_EINVAL before any launch; on MI355X (256 CUs) no automatic
 * split needs more than 8.5 MB (d_state 64); forced splits may. The stream
 * (if not NULL) must belong to the current device. All calls on one GPU
 * share its scratch, which keeps the last call's contents (each call writes
 * every slot it reads first, so nothing needs clearing): calls that overlap
 * in time on one GPU (concurrent streams) race and give wrong results;
 * serialize them.
 */
#define MHS_NOALLOC_SCRATCH_BYTES 16777216u
int mhs_scan_fwd_noalloc_f32(const float* x, const float* dt, const float* aneg,
                             const float* B, const float* C,
                             float* y, float* ckpt, float* h_last,
                             int64_t batch, int64_t seqlen, int64_t d_inner, int64_t d_state,
                             int64_t chunk, void* stream);

/* Bytes of device workspace mhs_scan_bwd_f32 needs for this shape. */
size_t mhs_scan_bwd_workspace_bytes(int64_t batch, int64_t seqlen, int64_t d_inner,
                                    int64_t d_state, int64_t chunk);

/*
 * Backward scan. Replaces the reference's `lib.ssm_bwd(x, dt, Aneg, Bm, Cm, dy,
 * dx, ddt, dAneg, dBm, dCm, ckpt, scratch, Bt, T, D, Kc)` launch
 * (mamba_metal/scan.py:132-261, launched at :408-410).
 *
 *   ckpt     : the forward's checkpoints for the same `chunk`
 *   dh_last  : gradient of the returned final state, or NULL (= zero; the
 *              reference drops it, scan.py:390-393)
 *   dx, ddt, daneg, dB, dC : fully written (no pre-zeroing needed). dB, dC and
 *              daneg are sums over channels / (batch, time), reduced as
 *              mhs_set_reduction selects (fixed order: bit-for-bit
 *              reproducible; atomics: reproducible to rounding; the default
 *              chooses per shape). dx and ddt are reproducible bit for bit
 *              either way.
 *   workspace: >= mhs_scan_bwd_workspace_bytes(...) bytes of device memory,
 *              256-byte aligned; its contents on entry do not matter.
 */
int mhs_scan_bwd_f32(const float* x, const float* dt, const float* aneg,
                     const float* B, const float* C, const float* dy,
                     const float* dh_last, const float* ckpt,
                     float* dx, float* ddt, float* daneg, float* dB, float* dC,
                     void* workspace, size_t workspace_bytes,
                     int64_t batch, int64_t seqlen, int64_t d_inner, int64_t d_state,
                     int64_t chunk, void* stream);

/*
 * Forward scan with the block's dt gate and decay parametrisation fused in.
 * Replaces the reference's `_proj` + `selective_scan` pair
 * (mamba_metal/model.py:197 and :200 feeding scan.py:78-127): the kernels form
 *     dt   = dt_min + (dt_max - dt_min) * sigmoid(dt_raw)    dt_raw : (batch, seqlen, d_inner)
 *     Aneg = softplus(A)                                     A      : (d_inner, d_state)
 * as they stage their inputs (dt is never written to memory), then run the
 * recurrence of mhs_scan_fwd_ws_f32 on (x, dt, Aneg, B, C). Needs finite
 * dt_min < dt_max. Same outputs, layouts, checkpoints and workspace (may be
 * NULL) as mhs_scan_fwd_ws_f32.
 * dt_bias: NULL, or the dt projection's bias (d_inner fp32, any alignment),
 * added to dt_raw before the sigmoid: then dt_raw may be the projection's
 * output without its bias (`dt_proj(x) = x W^T + b`, model.py:197).
 * ld_dt, ld_bc: elements between consecutive time steps of dt_raw and of B,
 * C (0: contiguous, i.e. d_inner and d_state). Larger strides read column
 * slices of one wider tensor, e.g. a single projection whose rows hold
 * [dt_raw | B | C] (ld_dt = ld_bc = d_inner + 2 d_state; the 16-byte
 * alignment applies to the slices' first elements). x is contiguous.
 */
int mhs_scan_gated_fwd_f32(const float* x, const float* dt_raw, const float* A,
                           const float* B, const float* C, float dt_min, float dt_max,
                           const float* dt_bias, float* y, float* ckpt, float* h_last,
                           void* workspace, size_t workspace_bytes,
                           int64_t batch, int64_t seqlen, int64_t d_inner, int64_t d_state,
                           int64_t chunk, int64_t ld_dt, int64_t ld_bc, void* stream);

/*
 * Backward of mhs_scan_gated_fwd_f32 (the autograd of the same reference
 * `_proj` + scan). Writes the gradients of the raw inputs:
 *     ddt_raw = ddt * (dt_max - dt_min) * s * (1 - s),   s = sigmoid(dt_raw)
 *     dA      = dAneg * sigmoid(A)
 * and dx, dB, dC as mhs_scan_bwd_f32. Workspace: mhs_scan_bwd_workspace_bytes
 * of the same shape. Reproducible as mhs_scan_bwd_f32 (bit for bit under the
 * fixed-order reduction).
 * ld_dt, ld_bc: input row strides as in mhs_scan_gated_fwd_f32; ld_ddt,
 * ld_dbc: row strides of the outputs ddt_raw and dB, dC (0: contiguous), so
 * that they can be written into the column slices of one gradient tensor of
 * the projection. dx is contiguous.
 * dt_bias: as in the forward. ddt_bias: NULL, or d_inner fp32 that receive
 * the gradient of the bias, sum over batch and time of ddt_raw (reduced as
 * dAneg is).
 */
int mhs_scan_gated_bwd_f32(const float* x, const float* dt_raw, const float* A,
                           const float* B, const float* C, float dt_min, float dt_max,
                           const float* dt_bias, const float* dy, const float* dh_last,
                           const float* ckpt, float* dx, float* ddt_raw, float* dA, float* dB,
                           float* dC, float* ddt_bias, void* workspace, size_t workspace_bytes,
                           int64_t batch, int64_t seqlen, int64_t d_inner, int64_t d_state,
                           int64_t chunk, int64_t ld_dt, int64_t ld_bc, int64_t ld_ddt,
                           int64_t ld_dbc, void* stream);

/*
 * bf16 activations with fp32 state. The same four scan entry points with x,
 * dt (or dt_raw), B, C, y, dy, dx, ddt (or ddt_raw), dB and dC as bf16
 * (uint16_t bit patterns, the upper half of an fp32); aneg / A, daneg / dA,
 * dt_bias, ddt_bias, dh_last, ckpt and h_last stay fp32. Loads widen exactly; all arithmetic,
 * the recurrent state and the reductions are fp32; each bf16 output is its
 * fp32 value rounded to nearest even. Same layouts, workspaces and
 * determinism as the fp32 entry points. No counterpart in the reference
 * (its kernels are fp32-only, README.md:80).
 */
int mhs_scan_fwd_bf16(const uint16_t* x, const uint16_t* dt, const float* aneg,
                      const uint16_t* B, const uint16_t* C,
                      uint16_t* y, float* ckpt, float* h_last,
                      void* workspace, size_t workspace_bytes,
                      int64_t batch, int64_t seqlen, int64_t d_inner, int64_t d_state,
                      int64_t chunk, void* stream);
int mhs_scan_bwd_bf16(const uint16_t* x, const uint16_t* dt, const float* aneg,
                      const uint16_t* B, const uint16_t* C, const uint16_t* dy,
                      const float* dh_last, const float* ckpt,
                      uint16_t* dx, uint16_t* ddt, float* daneg, uint16_t* dB, uint16_t* dC,
                      void* workspace, size_t workspace_bytes,
                      int64_t batch, int64_t seqlen, int64_t d_inner, int64_t d_state,
                      int64_t chunk, void* stream);
int mhs_scan_gated_fwd_bf16(const uint16_t* x, const uint16_t* dt_raw, const float* A,
                            const uint16_t* B, const uint16_t* C, float dt_min, float dt_max,
                            const float* dt_bias, uint16_t* y, float* ckpt, float* h_last,
                            void* workspace, size_t workspace_bytes,
                            int64_t batch, int64_t seqlen, int64_t d_inner, int64_t d_state,
                            int64_t chunk, int64_t ld_dt, int64_t ld_bc, void* stream);
int mhs_scan_gated_bwd_bf16(const uint16_t* x, const uint16_t* dt_raw, const float* A,
                            const uint16_t* B, const uint16_t* C, float dt_min, float dt_max,
                            const float* dt_bias, const uint16_t* dy, const float* dh_last,
                            const float* ckpt, uint16_t* dx, uint16_t* ddt_raw, float* dA,
                            uint16_t* dB, uint16_t* dC, float* ddt_bias, void* workspace, size_t workspace_bytes,
                            int64_t batch, int64_t seqlen, int64_t d_inner, int64_t d_state,
                            int64_t chunk, int64_t ld_dt, int64_t ld_bc, int64_t ld_ddt,
                            int64_t ld_dbc, void* stream);

/*
 * One recurrent decode step, in place on h. Replaces the pure-torch step of
 * the reference's MambaBlock.forward (mamba_metal/model.py:234-241):
 *     h <- h * exp(-dt * Aneg) + dt * B * x ;  y = sum_n C * h
 *   x, dt, y : (batch, d_inner)    B, C : (batch, d_state)    h : (batch, d_inner, d_state)
 */
int mhs_scan_step_f32(float* h, const float* x, const float* dt, const float* aneg,
                      const float* B, const float* C, float* y,
                      int64_t batch, int64_t d_inner, int64_t d_state, void* stream);

/*
 * Causal depthwise conv1d + SiLU, forward. Replaces the reference block's
 * `F.silu(self.conv(xt)[:, :, :T])` with `self.conv = nn.Conv1d(d_inner,
 * d_inner, kernel_size=K, padding=K-1, groups=d_inner, bias=True)`
 * (mamba_metal/model.py:174-175, applied at :244):
 *     pre[b,t,d] = bias[d] + sum_{k<K} w[d,k] * x[b, t-K+1+k, d]   (x = 0 for t < 0)
 *     out[b,t,d] = pre * sigmoid(pre)
 *   x   : (batch, seqlen, d_inner), rows `x_row_stride` floats apart
 *         (>= d_inner; the block's x half of its in_proj output has 2*d_inner),
 *         batch rows seqlen * x_row_stride apart
 *   w   : (d_inner, K) (the Conv1d weight (d_inner, 1, K)), bias : (d_inner)
 *   out : (batch, seqlen, d_inner) contiguous
 * K in [1, 8]. Pointers need 4-byte alignment only.
 */
int mhs_conv1d_silu_fwd_f32(const float* x, int64_t x_row_stride, const float* w,
                            const float* bias, float* out, int64_t batch, int64_t seqlen,
                            int64_t d_inner, int64_t kernel_size, void* stream);

/* Bytes of device workspace mhs_conv1d_silu_bwd_f32 needs for this shape. */
size_t mhs_conv1d_silu_bwd_workspace_bytes(int64_t batch, int64_t seqlen, int64_t d_inner,
                                           int64_t kernel_size);

/*
 * Backward of mhs_conv1d_silu_fwd_f32 (the autograd of the same reference
 * Conv1d + SiLU): dx (batch, seqlen, d_inner) with rows dx_row_stride apart
 * (0: contiguous; larger writes the x half of the in_proj output's
 * gradient in place), dw (d_inner, K), dbias (d_inner), all fully written.
 * dw and dbias are summed over (batch, time) through the workspace in a
 * fixed order (bit-for-bit reproducible).
 */
int mhs_conv1d_silu_bwd_f32(const float* x, int64_t x_row_stride, const float* w,
                            const float* bias, const float* dout, float* dx,
                            int64_t dx_row_stride, float* dw, float* dbias, void* workspace,
                            size_t workspace_bytes, int64_t batch, int64_t seqlen,
                            int64_t d_inner, int64_t kernel_size, void* stream);

/*
 * The block's output gate, forward. Replaces `y = y + self.D_skip` and the
 * `y * F.silu(z)` feeding out_proj (mamba_metal/model.py:255-256):
 *     out[b,t,d] = (y[b,t,d] + d_skip[d]) * silu(z[b,t,d])
 *   y, out : (batch, seqlen, d_inner) contiguous
 *   z      : (batch, seqlen, d_inner), rows `z_row_stride` floats apart (>= d_inner;
 *            the z half of the block's in_proj output has 2*d_inner), batch rows
 *            seqlen * z_row_stride apart
 * Pointers need 4-byte alignment only.
 */
int mhs_out_gate_fwd_f32(const float* y, const float* d_skip, const float* z,
                         int64_t z_row_stride, float* out,
                         int64_t batch, int64_t seqlen, int64_t d_inner, void* stream);

/* Bytes of device workspace mhs_out_gate_bwd_f32 needs for this shape. */
size_t mhs_out_gate_bwd_workspace_bytes(int64_t batch, int64_t seqlen, int64_t d_inner);

/*
 * Backward of mhs_out_gate_fwd_f32 (the autograd of the same reference ops),
 * with s = sigmoid(z):
 *     dy = dout * z * s ;  dz = dout * (y + d_skip) * s * (1 + z * (1 - s)) ;
 *     dd_skip[d] = sum_{b,t} dy[b,t,d]
 * dy : (batch, seqlen, d_inner) contiguous; dz : the same, rows dz_row_stride
 * apart (0: contiguous; larger writes the z half of the in_proj output's
 * gradient in place); dd_skip : (d_inner); all fully written. dd_skip is
 * summed through the workspace (16-byte aligned) in a fixed order (bit-for-bit
 * reproducible).
 */
int mhs_out_gate_bwd_f32(const float* y, const float* d_skip, const float* z,
                         int64_t z_row_stride, const float* dout,
                         float* dy, float* dz, int64_t dz_row_stride, float* dd_skip,
                         void* workspace, size_t workspace_bytes,
                         int64_t batch, int64_t seqlen, int64_t d_inner, void* stream);

/*
 * Cross-entropy of the model head, forward: for each row r of logits
 * (rows, vocab) fp32 (row-major, contiguous) and int64 targets (rows),
 *     lse[r] = log sum_j exp(logits[r, j]);
 *     loss_rows[r] = lse[r] - logits[r, targets[r]], or 0 where
 *     targets[r] == ignore_index (NaN for any other target outside [0, vocab)).
 * The mean loss is sum(loss_rows) / (rows whose target is not ignore_index).
 * Replaces F.cross_entropy's log_softmax + nll_loss over the tied head's
 * logits (mamba_metal/model.py:296-297), which write and keep the (rows, vocab)
 * log-probabilities; this reads the logits once and keeps lse (4 bytes per
 * row). Each row's sum runs in a fixed order (bit-for-bit reproducible).
 */
int mhs_xent_fwd_f32(const float* logits, const int64_t* targets, float* lse,
                     float* loss_rows, int64_t rows, int64_t vocab, int64_t ignore_index,
                     void* stream);

/*
 * Its backward: dlogits[r, j] = scale[0] * (exp(logits[r, j] - lse[r]) - [j == targets[r]])
 * for rows whose target is not ignore_index, 0 for the others. scale is one
 * device float: the loss's upstream gradient over the count of rows not
 * ignored (the mean's factor). dlogits (rows, vocab) is fully written and may
 * not alias logits. Replaces the log_softmax / nll_loss backward
 * (the autograd of mamba_metal/model.py:296-297).
 */
int mhs_xent_bwd_f32(const float* logits, const int64_t* targets, const float* lse,
                     const float* scale, float* dlogits, int64_t rows, int64_t vocab,
                     int64_t ignore_index, void* stream);

/*
 * RMSNorm of the residual stream, fp32: for each of `rows` rows of `cols`
 * features, y = x * r * weight with r = 1 / sqrt(mean(x^2) + eps); rstd[row]
 * receives r. Replaces the reference's RMSNorm.forward
 * (mamba_metal/model.py:85-95), applied before every block's in_proj
 * (model.py:225) and before the head (model.py:293). cols is a multiple of 4
 * in [4, 2048]; every pointer 16-byte aligned; y may not alias x; eps finite
 * and >= 0. Each row's sum of squares runs in a fixed order.
 */
int mhs_rmsnorm_fwd_f32(const float* x, const float* weight, float* y, float* rstd,
                        int64_t rows, int64_t cols, float eps, void* stream);

/*
 * The residual stream's update and the next norm in one pass: x_out = x +
 * delta, then y and rstd of x_out as mhs_rmsnorm_fwd_f32. Replaces the
 * block's residual add (mamba_metal/model.py:256) followed by the next
 * block's RMSNorm (model.py:225) or the final one (model.py:293). x_out may
 * not alias x, delta or y; y may not alias x or delta. The backward is
 * mhs_rmsnorm_bwd_f32 on x_out, with x_out's own gradient as dres; x and
 * delta both receive the resulting dx.
 */
int mhs_add_rmsnorm_fwd_f32(const float* x, const float* delta, const float* weight,
                            float* x_out, float* y, float* rstd, int64_t rows, int64_t cols,
                            float eps, void* stream);

/* Workspace bytes of mhs_rmsnorm_bwd_f32 for rows x cols. */
size_t mhs_rmsnorm_bwd_workspace_bytes(int64_t rows, int64_t cols);

/*
 * Its backward, the autograd of model.py:85-95: with g = dy * weight,
 * dx = r * g - x * r^3 * sum(g * x) / cols, plus dres (the residual stream's
 * other gradient, may be null) added in the same pass; dweight (cols) = the
 * sum over rows of dy * x * r, fully written (zeros for rows = 0). dx may
 * alias dres, not x or dy. The workspace (mhs_rmsnorm_bwd_workspace_bytes,
 * 256-byte aligned) holds per-block partials of dweight, summed in a fixed
 * order: bit-for-bit reproducible.
 */
int mhs_rmsnorm_bwd_f32(const float* dy, const float* x, const float* weight, const float* rstd,
                        const float* dres, float* dx, float* dweight, void* workspace,
                        size_t workspace_bytes, int64_t rows, int64_t cols, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MAMBA_HIP_SCAN_H */
