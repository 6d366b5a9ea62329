/*
 * ssm_mamba.h -- C ABI of the MI355X (gfx950) selective-scan library
 * (libssm_mamba_hip.so).
 *
 * Plain pointers and sizes only.  Every pointer is a device pointer on the
 * current HIP device unless stated otherwise; tensors are dense row-major.
 * Every call is asynchronous on `stream` (a hipStream_t; NULL = the default
 * stream) and returns SSM_OK or an error code, with a message available from
 * ssm_last_error() (per calling thread).
 *
 * Element types (`dtype`): SSM_F32 or SSM_BF16 for the streamed tensors
 * (u, delta, z, out, dout, du, ddelta, dz, B, C, dB, dC, x, dt); parameters
 * (A, D, delta_bias), states and their gradients are always fp32.  Arithmetic
 * is fp32 throughout.
 *
 * Shapes: u/delta/z/out/dout/du/ddelta/dz (batch, dim, seqlen);
 * B/C/dB/dC (batch, nstate, seqlen); A/dA (dim, nstate); D/delta_bias/dD/
 * ddelta_bias (dim); h_init/h_last/dh_last/dh_init (batch, dim, nstate);
 * h_chunks (batch, ssm_scan_nchunks(seqlen), nstate, dim): the state after
 * each SSM_CHUNK steps, channel-contiguous (h_chunks[:, -1] transposed is the
 * final state); or, with h_pairs = 1, the pair layout
 * (batch, SSM_REF_SLOTS * ssm_scan_ref_nchunks(seqlen), 2 * nstate, dim):
 * slot s holds in row 2n + 1 the state after SSM_CHUNK * (s + 1) steps
 * (s < ssm_scan_nchunks(seqlen)), and slot SSM_REF_SLOTS * c + 7, the last of
 * the reference's 128-step chunk c, holds in row 2n the product of the decays
 * exp(delta_t A) from step 0 to that chunk's end and in row 2n + 1 the state
 * at its end (the final state for the last chunk, also when seqlen is not a
 * multiple of 128): the reference's (prod a, h) chunk carry
 * (csrc/selective_scan/forward_kernel.cu:225-228, chunks of
 * kernel_config::chunk_size = 128 steps, kernel_config.h:4-10), seen in the
 * reference's (batch, dim, nchunks, 2 * nstate) index order as a strided view
 * with chunk stride SSM_REF_SLOTS slots and offset 7 slots; the other slots'
 * even rows are not written;
 * length (batch) int64.
 */
#ifndef SSM_MAMBA_H_
#define SSM_MAMBA_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { SSM_F32 = 0, SSM_BF16 = 1 };
enum { SSM_OK = 0, SSM_ERR_INVALID = 1, SSM_ERR_UNSUPPORTED = 2, SSM_ERR_HIP = 3 };
enum { SSM_CHUNK = 16, SSM_REF_CHUNK = 128, SSM_REF_SLOTS = SSM_REF_CHUNK / SSM_CHUNK };

/* Message for the last failed call on this thread ("" if none). */
const char* ssm_last_error(void);

/* Library ABI version (bumped on any signature change). */
int ssm_abi_version(void);

/*
 * Kernel timing (measurement hook; no counterpart in the reference, whose
 * launches are untimed).  Between ssm_profile_begin() and ssm_profile_end()
 * every kernel this library launches is bracketed by HIP events recorded on
 * its launch stream.  ssm_profile_end() waits for them and writes one line
 * "<kernel> <launches> <total_ms>" per kernel into buf (NUL-terminated,
 * truncated to buf_bytes); it returns the number of timed launches (< 0 on
 * error).  At most 4096 launches are timed per session.
 */
int ssm_profile_begin(void);
int ssm_profile_end(char* buf, size_t buf_bytes);

/* Number of saved states per row: ceil(seqlen / SSM_CHUNK). */
int64_t ssm_scan_nchunks(int64_t seqlen);
/* Number of the reference's chunks per row, ceil(seqlen / SSM_REF_CHUNK)
 * (kernel_config::get_num_chunks, csrc/selective_scan/kernel_config.h:8-10):
 * the chunk count of the pair layout (h_pairs = 1). */
int64_t ssm_scan_ref_nchunks(int64_t seqlen);

/* Device workspace (bytes) for ssm_selective_scan_fwd / _bwd. */
size_t ssm_scan_fwd_workspace_bytes(int64_t batch, int64_t dim, int64_t seqlen, int64_t nstate);
size_t ssm_scan_bwd_workspace_bytes(int64_t batch, int64_t dim, int64_t seqlen, int64_t nstate);

/*
 * Selective-scan forward.  Replaces selective_scan_forward
 * (csrc/selective_scan/selective_scan.cpp:212-292, declared at
 * csrc/selective_scan/selective_scan.h:73-84) behind the pybind binding
 * selective_scan.forward (csrc/selective_scan/bindings.cpp:6).
 *
 *   out      = (D*u + sum_n C*h) [* silu(z)]  with h_t = exp(delta_t*A) h_{t-1}
 *              + delta_t*u_t*B_t, delta = softplus(delta_raw + delta_bias)
 *              (no softplus when delta_softplus == 0)
 *   h_chunks = states after each SSM_CHUNK steps (h_pairs = 1: the pair
 *              layout with the reference's 128-step chunk carry, see above),
 *              or NULL (inference); then h_last (nullable) receives the
 *              final state.
 *   out_ungated (nullable, requires z) = D*u + sum_n C*h, the output before
 *              the gate: the backward needs it for dz.  The reference gates
 *              outside the kernel (modules/mamba.py:182), where autograd
 *              saves the same tensor.
 * D, delta_bias, h_init, length, z are nullable.  padding_right: 1 = valid
 * positions are t < length[b], 0 = t >= seqlen - length[b] (lengths are
 * clamped to [0, seqlen]); padded steps leave the state unchanged.
 * B and C: rows of seqlen, nstate rows per batch row, batch row b starting
 * bc_batch_stride elements after row b-1 (0: nstate * seqlen, contiguous).
 * The reference takes B/C batch strides too (B_batch_stride,
 * csrc/selective_scan/selective_scan.cpp:83-87); a channel slice of the
 * x-projection output can be passed in place.
 * nstate <= 256.  workspace: ssm_scan_fwd_workspace_bytes() bytes.
 */
int ssm_selective_scan_fwd(int64_t batch, int64_t dim, int64_t seqlen, int64_t nstate, int dtype,
                           const void* u, const void* delta, const float* A, const void* B,
                           const void* C, int64_t bc_batch_stride, const float* D,
                           const float* delta_bias,
                           const float* h_init, const int64_t* length, int padding_right,
                           const void* z, int delta_softplus, void* out, void* out_ungated,
                           float* h_chunks, int h_pairs, float* h_last, void* workspace,
                           size_t workspace_bytes, void* stream);

/*
 * Selective-scan forward that allocates nothing and takes no workspace.  No
 * counterpart in the reference: it is for callers that cannot allocate device
 * memory -- code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc.  Arguments and results as ssm_selective_scan_fwd; the
 * workspace is a static device array of SSM_NOALLOC_SCRATCH_BYTES per GPU,
 * held until the process ends.  Shapes whose ssm_scan_fwd_workspace_bytes()
 * exceeds that size are rejected (SSM_ERR_UNSUPPORTED).  The first call on a
 * device looks the array up on that device (hipGetSymbolAddress); no call
 * allocates.  Every call on one GPU shares its array, so calls that overlap
 * on one GPU (concurrent streams or threads) race: serialize them.
 */
#define SSM_NOALLOC_SCRATCH_BYTES (32u << 20)
int ssm_selective_scan_fwd_noalloc(int64_t batch, int64_t dim, int64_t seqlen, int64_t nstate,
                                   int dtype, const void* u, const void* delta, const float* A,
                                   const void* B, const void* C, int64_t bc_batch_stride,
                                   const float* D, const float* delta_bias, const float* h_init,
                                   const int64_t* length, int padding_right, const void* z,
                                   int delta_softplus, void* out, void* out_ungated,
                                   float* h_chunks, int h_pairs, float* h_last, void* stream);

/*
 * Selective-scan forward with the step-size projection fused in: the
 * inference prefill of a Mamba block from its x-projection output to the scan
 * output, replacing modules/mamba.py:149-171 (the split of ssm_params, the
 * delta projection delta_proj.weight @ delta.t(), the channel-major copies of
 * delta, B and C, and SelectiveScanFn's forward).
 *
 *   ssm_params (batch, seqlen, P) bf16, P = dt_rank + 2 * nstate: the
 *              token-major x-projection output (modules/mamba.py:141-145),
 *              each token's row [dt | B | C]; batch row b starts
 *              params_batch_stride elements after row b-1 (0: seqlen * P).
 *   dt_weight  (dim, dt_rank) bf16, delta_proj.weight.
 *   delta_raw  = dt_weight @ dt^T rounded to bf16 per element (the
 *              reference's product in the model dtype), then the scan as
 *              ssm_selective_scan_fwd with delta = delta_raw and B, C read in
 *              place from ssm_params.  Written to delta_out (nullable;
 *              (batch, dim, seqlen) bf16) when given.
 * z_batch_stride: elements between batch rows of z (0: dim * seqlen), so the
 * gate half of the in-projection output is read in place.
 * The other arguments as ssm_selective_scan_fwd; no saved chunk states and no
 * ungated output (inference).  bf16 only, nstate <= 16 and a multiple of 4,
 * dt_rank a multiple of 8 and <= 64, ssm_params and dt_weight 16-byte aligned,
 * params_batch_stride a multiple of 8 (else SSM_ERR_UNSUPPORTED; the caller
 * then runs the projection and ssm_selective_scan_fwd).  workspace:
 * ssm_scan_fwd_workspace_bytes() bytes.
 */
int ssm_selective_scan_fwd_dt_proj(int64_t batch, int64_t dim, int64_t seqlen, int64_t nstate,
                                   int64_t dt_rank, int dtype, const void* u,
                                   const void* ssm_params, int64_t params_batch_stride,
                                   const void* dt_weight, const float* A, const float* D,
                                   const float* delta_bias, const float* h_init,
                                   const int64_t* length, int padding_right, const void* z,
                                   int64_t z_batch_stride, int delta_softplus, void* out,
                                   void* delta_out, float* h_last, void* workspace,
                                   size_t workspace_bytes, void* stream);
/* 1 when ssm_selective_scan_fwd_dt_proj takes this shape and dtype, else 0. */
int ssm_selective_scan_fwd_dt_proj_supported(int64_t batch, int64_t dim, int64_t seqlen,
                                             int64_t nstate, int64_t dt_rank, int dtype);

/*
 * Selective-scan backward.  Replaces selective_scan_backward
 * (csrc/selective_scan/selective_scan.cpp:294-380, declared at
 * csrc/selective_scan/selective_scan.h:86-99) behind selective_scan.backward
 * (csrc/selective_scan/bindings.cpp:7).
 *
 * Inputs as for the forward (B and C with bc_batch_stride; dB and dC are
 * written contiguous) plus h_chunks (from the forward, in the layout h_pairs
 * names; only the states are read), dout (the
 * upstream gradient of out; ignored at padded positions) and dh_last
 * (nullable = zero).  Writes du, ddelta, dA, dB, dC (all overwritten), and
 * when non-NULL dD, ddelta_bias and dh_init (requires h_init).  With z,
 * out_ungated (the forward's ungated output) and dz are required; without z
 * both must be NULL.
 * nstate <= 256, as the reference's backward dispatch (csrc/static_switch.h:
 * 15-37, csrc/selective_scan/backward_kernel.cu:456-478); past 64 states the
 * kernels run in chunks of 64 states.  workspace: ssm_scan_bwd_workspace_bytes()
 * bytes.  The result is deterministic (fixed-order reductions, no atomics on
 * global memory).
 */
int ssm_selective_scan_bwd(int64_t batch, int64_t dim, int64_t seqlen, int64_t nstate, int dtype,
                           const void* u, const void* delta, const float* A, const void* B,
                           const void* C, int64_t bc_batch_stride, const float* D,
                           const float* delta_bias,
                           const float* h_init, const int64_t* length, int padding_right,
                           const void* z, const void* out_ungated, int delta_softplus,
                           const float* h_chunks, int h_pairs, const void* dout,
                           const float* dh_last, void* du, void* ddelta, float* dA, void* dB,
                           void* dC, float* dD, float* ddelta_bias, float* dh_init, void* dz,
                           void* workspace, size_t workspace_bytes, void* stream);

/*
 * One decode step.  Replaces selective_update
 * (csrc/selective_update/selective_update.cpp:78-130, declared at
 * csrc/selective_update/selective_update.h:32-41) behind
 * selective_update.apply (csrc/selective_update/bindings.cpp:6).
 *
 *   new_state = exp(delta*A)*state + delta*x*B,  delta = softplus(dt + dt_bias)
 *   out       = (D*x + sum_n C*new_state) [* silu(z)]
 * state, new_state (batch, dim, nstate) fp32 -- new_state may equal state for
 * an in-place update; x, dt, z, out (batch, dim); B, C (batch, nstate).
 * D, dt_bias, z nullable.  nstate <= 256.
 */
int ssm_selective_state_update(int64_t batch, int64_t dim, int64_t nstate, int dtype,
                               const float* state, float* new_state, const void* x,
                               const void* dt, const float* A, const void* B, const void* C,
                               const float* D, const float* dt_bias, const void* z,
                               int dt_softplus, void* out, void* stream);

/*
 * RMSNorm over the channel axis of channel-major x (batch, channels, seqlen):
 * out[b, c, t] = x[b, c, t] * rsqrt(mean_c x[b, c, t]^2 + eps) * (1 + weight[c]),
 * fp32 statistics, the result in `dtype` -- the reference's RMSNorm
 * (modules/rms_norm.py:11-31) applied to the layout the scan streams.  x, out
 * (batch, channels, seqlen) and weight (channels) have element type `dtype`.
 */
int ssm_rms_norm_cm(int64_t batch, int64_t channels, int64_t seqlen, int dtype, const void* x,
                    const void* weight, float eps, void* out, void* stream);

/*
 * Causal depthwise conv1d (+ SiLU) over channel-major rows: the prefill
 * convolution of the Mamba layer, nn.Conv1d(dim, dim, width, groups=dim,
 * padding=width-1)(x)[..., :seqlen] followed by F.silu
 * (modules/mamba.py:37-44,138-139), which the reference runs as two torch ops.
 *
 *   out[b,c,t] = act(bias[c] + sum_{j<width} weight[c,j] * x[b,c,t-(width-1)+j]),
 *   x = 0 before t = 0; act = silu when silu != 0, else the identity.
 * x, out (batch, dim, seqlen); weight (dim, width) (the (dim, 1, width) conv
 * weight); bias (dim) nullable.  All of x, out, weight, bias, window (and the
 * gradients below) have element type `dtype`; arithmetic is fp32.
 * width <= 8.
 * window (nullable): (batch, dim, width-1) receives the decode cache a
 * prefill leaves (modules/mamba.py:113-135): the width-1 inputs x[b,c,t] for
 * t = len-(width-1) .. len-1, zero for t < 0, with len = lengths[b] clamped to
 * [0, seqlen] (lengths nullable: len = seqlen; lengths requires window).
 * x_batch_stride: elements between batch rows of x (0: dim * seqlen), so a
 * channel slice of a larger activation -- the x half of the in-projection
 * output (modules/mamba.py:104-111) -- is read in place; out is contiguous.
 */
int ssm_causal_conv1d_fwd(int64_t batch, int64_t dim, int64_t seqlen, int64_t width, int dtype,
                          const void* x, int64_t x_batch_stride, const void* weight,
                          const void* bias, int silu, void* out, const int64_t* lengths,
                          void* window, void* stream);

/* Device workspace (bytes) for ssm_causal_conv1d_bwd. */
size_t ssm_causal_conv1d_bwd_workspace_bytes(int64_t batch, int64_t dim, int64_t width);

/*
 * Backward of ssm_causal_conv1d_fwd for the upstream gradient dout: writes dx
 * (batch, dim, seqlen), dweight (dim, width) and, when non-NULL, dbias (dim)
 * (all overwritten; bias NULL counts as zero).  The weight and bias gradients
 * are summed over batch and time in a fixed order (deterministic).
 */
int ssm_causal_conv1d_bwd(int64_t batch, int64_t dim, int64_t seqlen, int64_t width, int dtype,
                          const void* x, const void* weight, const void* bias, const void* dout,
                          int silu, void* dx, void* dweight, void* dbias, void* workspace,
                          size_t workspace_bytes, void* stream);

/*
 * Fused decode step of a Mamba block, for 1 <= batch <= 8 sequences.  The
 * reference's Block.step / Mamba.step (modules/block.py:80-86,
 * modules/mamba.py:189-243) runs about twenty torch ops per layer and token;
 * these four calls do the same work:
 *
 *   ssm_decode_in_proj_conv  xz = W_in @ rmsnorm(x) [+ b_in]; conv step -> xc;
 *                            the conv window rolls
 *   ssm_decode_gemv          params = W_x @ xc                 (batch, rank + 2*nstate)
 *   ssm_decode_ssm_step      state update, y = (C.h + D xc) * silu(z)
 *   ssm_decode_gemv          x' = x + W_out @ y [+ b_out]      (residual set)
 *
 * or three, when ssm_decode_xproj_blocks(dim, rank + 2*nstate) = P > 0: the
 * in-projection call then also takes W_x and writes P fp32 partials of
 * W_x @ xc, and the state-update call adds them in place of params.
 *
 * Every tensor except state has element type `dtype` (weights and the norm,
 * conv, dt and A/D parameters included); state (batch, dim, nstate) is fp32.
 * Row-major throughout.
 */

/*
 * y[b, o] = sum_k W[o, k] v[b, k] (+ bias[o]) (+ residual[b, o]) with
 * v = x, or v = x * rsqrt(mean_k x^2 + norm_eps) * (1 + norm_weight) when
 * norm_weight is non-NULL (the reference's RMSNorm, modules/rms_norm.py:11-31).
 * W (out_dim, in_dim); x (batch, in_dim); y, residual (batch, out_dim).
 * in_dim a multiple of 16 bytes of elements; W, x, norm_weight 16-byte aligned.
 * Also the decode LM head (models/causal_lm.py:93-104) with the final norm.
 */
int ssm_decode_gemv(int64_t batch, int64_t out_dim, int64_t in_dim, int dtype, const void* weight,
                    const void* x, const void* norm_weight, float norm_eps, const void* bias,
                    const void* residual, void* y, void* stream);

/*
 * In-projection with the conv step (modules/mamba.py:199-214): xz (batch,
 * 2*dim) = in_proj_weight (2*dim, in_dim) @ v [+ in_proj_bias], v = x or its
 * RMSNorm (norm_weight non-NULL, as in ssm_decode_gemv); for the x half
 * xs = xz[:, :dim]: xc (batch, dim) = silu(sum_{j<width-1} conv_weight[c, j] *
 * conv_window[b, c, j] + conv_weight[c, width-1] * xs + conv_bias[c]) and the
 * window rolls: conv_window (batch, dim, width-1) <- [window[..., 1:], xs].
 * conv_weight (dim, width); conv_bias nullable; 2 <= width <= 8.
 */
int ssm_decode_in_proj_conv(int64_t batch, int64_t dim, int64_t in_dim, int64_t width, int dtype,
                            const void* in_proj_weight, const void* x, const void* norm_weight,
                            float norm_eps, const void* in_proj_bias, const void* conv_weight,
                            const void* conv_bias, void* conv_window, void* xz, void* xc,
                            const void* x_proj_weight, int64_t params_dim, float* xproj_partials,
                            void* stream);

/*
 * The x-projection folded into the two calls around it (no counterpart call
 * in the reference; it is modules/mamba.py:216-221's x_proj).  Returns the
 * number P of partial blocks, or 0 when the folded form does not apply
 * (params_dim = rank + 2*nstate above 256, or dim not a multiple of 16).
 * With x_proj_weight (params_dim, dim) non-NULL, ssm_decode_in_proj_conv
 * also writes xproj_partials, fp32 (P, batch, params_dim rounded up to 4):
 * block p holds sum over the 16 channels c of block p of
 * x_proj_weight[j, c] * xc[b, c].  ssm_decode_ssm_step with params_blocks = P
 * reads params = xproj_partials and adds the P blocks in a fixed order
 * (the result is bit-reproducible), rounding the sums to dtype as the
 * unfolded x-projection output is.  x_proj_weight and xproj_partials are
 * 16-byte aligned.
 */
int64_t ssm_decode_xproj_blocks(int64_t dim, int64_t params_dim);

/*
 * Step-size projection, state update and gate (modules/mamba.py:223-240 with
 * selective_update/kernel.cu:39-71): delta = dt_proj_weight (dim, rank) @
 * params[:, :rank]; delta' = softplus(delta + dt_bias); A = -exp(log_A);
 * state = exp(delta' A) state + delta' xc B with B = params[:, rank:rank+nstate];
 * y = (sum_n C state + D xc) * silu(z), C = params[:, rank+nstate:],
 * z = xz[:, dim:2*dim] (row stride ld_xz).  params (batch, rank + 2*nstate)
 * with params_blocks = 0, or the x-projection partials of
 * ssm_decode_in_proj_conv with params_blocks = ssm_decode_xproj_blocks(dim,
 * rank + 2*nstate); state (batch, dim, nstate) fp32 updated in place; y
 * (batch, dim).  dt_bias, D nullable; nstate in {4, 8, 16, 32, 64}.
 */
int ssm_decode_ssm_step(int64_t batch, int64_t dim, int64_t nstate, int64_t rank, int dtype,
                        const void* params, int64_t params_blocks, const void* dt_proj_weight,
                        const void* dt_bias, const void* log_A, const void* D, const void* xc,
                        const void* xz, int64_t ld_xz, float* state, void* y, void* stream);

/*
 * The token step of a whole stack of Mamba blocks in one launch: for each of
 * nlayers layers in turn, x <- x + Mamba.step(rmsnorm(x)) (Block.step,
 * modules/block.py:78-90, over the layers as models/causal_lm.py:92-93
 * loops): the work of ssm_decode_in_proj_conv (folded x-projection),
 * ssm_decode_ssm_step and the residual ssm_decode_gemv, with the
 * out-projection's dot products summed in K-slices and the state update's
 * sums split over thread pairs (each a fixed order: the results are
 * deterministic and agree with those calls to fp32 rounding, not bit for
 * bit).  No counterpart call in the reference.
 *
 * One persistent grid runs the three phases of every layer; its workgroups
 * pass activations to each other through the workspace, each waiting for the
 * data it reads, so every workgroup must be resident at once
 * (SSM_ERR_UNSUPPORTED otherwise, before anything runs): do not run other
 * work on the device at the same time.  Shapes: nstate = 16, the in- and
 * out-projections in one pass each (model_dim <= 1024 and dim <= 2048 for
 * bf16, half that for fp32) and at most 8 x-projection partial blocks per
 * state-update thread (SSM_ERR_UNSUPPORTED otherwise).
 *
 * layer_table: device memory, nlayers rows of SSM_LAYER_NPTR pointers in the
 * order of the enum below (NULL allowed for the biases, dt_bias and D; the
 * others 16-byte aligned, the state fp32).  Shapes: in_proj_weight (2*dim,
 * model_dim), norm_weight (model_dim), conv_weight (dim, width), x_proj_weight
 * (rank + 2*nstate, dim), dt_proj_weight (dim, rank), log_A (dim, nstate),
 * out_proj_weight (model_dim, dim), conv_window (batch, dim, width-1), state
 * (batch, dim, nstate).  x, out: (batch, model_dim); out may be x.
 * rank a multiple of 16 bytes of elements, at most 16 such;
 * ssm_decode_xproj_blocks(dim, rank + 2*nstate) > 0; 2 <= width <= 4.
 *
 * workspace: at least ssm_decode_layers_workspace(...) bytes (it grows with
 * nlayers: each layer has its own hand-off buffers), 256-byte aligned,
 * zero-filled before its first use and then left to the launches (it holds a
 * launch counter); one workspace per stream of launches.  Every wait is
 * bounded: should one ever time out, the workgroup that gave up sets the
 * error word (the 32-bit word at byte offset 512 of the workspace, nonzero
 * once set), the launch and every later launch on the workspace do nothing
 * further (their outputs are not written) until ssm_decode_layers_status
 * reports it (SSM_ERR_HIP) and zero-fills the workspace.  The launches
 * advance the layers' SSM states and conv windows in place, so those caches
 * may then have been advanced partly (some layers, some channels): they are
 * invalid as well, and the caller re-runs the prefill.
 */
enum {
  SSM_LAYER_IN_PROJ_W = 0, SSM_LAYER_IN_PROJ_B, SSM_LAYER_NORM_W, SSM_LAYER_CONV_W,
  SSM_LAYER_CONV_B, SSM_LAYER_X_PROJ_W, SSM_LAYER_DT_PROJ_W, SSM_LAYER_DT_BIAS, SSM_LAYER_LOG_A,
  SSM_LAYER_D, SSM_LAYER_OUT_PROJ_W, SSM_LAYER_OUT_PROJ_B, SSM_LAYER_CONV_WINDOW, SSM_LAYER_STATE,
  SSM_LAYER_NPTR
};
int64_t ssm_decode_layers_workspace(int64_t batch, int64_t nlayers, int64_t model_dim,
                                    int64_t dim, int64_t params_dim, int dtype);
int ssm_decode_layers(int64_t batch, int64_t nlayers, int64_t model_dim, int64_t dim, int64_t nstate,
                      int64_t rank, int64_t width, int dtype, const void* layer_table, const void* x,
                      void* out, float norm_eps, void* workspace, int64_t workspace_bytes,
                      void* stream);
/* Synchronises the stream; SSM_OK, or SSM_ERR_HIP after a wait timed out
 * (the workspace is zero-filled then, and the outputs and the layers' caches
 * since the previous check are invalid). */
int ssm_decode_layers_status(void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Greedy pick of the decode loop: token[b] = argmax_v probs[b, v] over the
 * softmax output (batch, vocab) -- the argmax of models/causal_lm.py:117-120,
 * the first maximum, NaN ranking above every number as in torch.argmax --
 * and, with tokens non-NULL, the loop's bookkeeping in the same launch:
 * tokens[b * tokens_ld + min(*pos, tokens_cols - 1)] = token[b], then
 * *pos += 1 (pos nullable: column 0, no increment).  token, tokens, pos are
 * int64.  Rows of a multiple of 16 bytes, 16-byte aligned.  workspace:
 * ssm_decode_pick_workspace(batch) bytes, zero-filled before the first call
 * (a counter each call leaves at zero); calls that share it must not overlap.
 * No counterpart call in the reference (its loop does these as torch ops,
 * models/causal_lm.py:111-129).
 */
int64_t ssm_decode_pick_workspace(int64_t batch);
int ssm_decode_pick(int64_t batch, int64_t vocab, int dtype, const void* probs, int64_t* token,
                    int64_t* tokens, int64_t tokens_ld, int64_t tokens_cols, int64_t* pos,
                    void* workspace, int64_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SSM_MAMBA_H_ */
