/*
 * atlas_scan.h -- C ABI of the MI355X (gfx950) Atlas memory-layer library.
 *
 * Plain C: descriptors, raw device pointers, sizes and an opaque stream
 * handle (a hipStream_t passed as void*; NULL = the default stream).  No C++
 * or framework types cross this boundary, so it can be bound from ctypes,
 * an XLA FFI handler, or any other host.
 *
 * Reference interfaces each entry point replaces (rkstgr/atlas-jax):
 *   atlas_scan_fwd          the chunk loop of AtlasMemoryLayer.__call__
 *                           (atlas_jax/memory_layer.py:662-716) together
 *                           with its loop body _process_chunk_deep (:496-597):
 *                           inner gradient, Omega window, momentum scan,
 *                           Polar-Express, memory scan and read-out, for all
 *                           chunks of a sequence in one call.
 *   atlas_fused_chunk_fwd   the plugin operator fused_chunk_scan
 *                           (atlas_jax/kernels/fused_chunk.py:321-355): one
 *                           chunk from precomputed momentum inputs.
 *   atlas_pe_batched        polar_express / fused_polar_express
 *                           (atlas_jax/memory_layer.py:43-71,
 *                           atlas_jax/kernels/triton_pe.py:26-69) on a batch of
 *                           small matrices; with ATLAS_PE_NORM_NO_EPS it is the
 *                           Muon orthogonalisation block (atlas_jax/optim.py:69-83).
 *   atlas_linear_scan       linear_scan / triton_linear_scan
 *                           (atlas_jax/memory_layer.py:256-296,
 *                           atlas_jax/kernels/triton_scan.py:85-111).
 *   atlas_linear_scan_bwd   the reverse-time scan backward of
 *                           triton_linear_scan (kernels/triton_scan.py:119-161).
 *   atlas_swa_fwd           the sliding-window attention core of the MAG
 *                           blocks (atlas_jax/model.py:83-133), and its
 *                           backward (atlas_swa_bwd).
 *   atlas_layer_prologue    the layer's convolutions, q/k norm + polynomial
 *                           map and gates (atlas_jax/memory_layer.py:606-633).
 *
 * Conventions
 *   - The caller owns every buffer.  The library allocates nothing and never
 *     synchronises the stream; all work is enqueued on `stream`.
 *   - State (W1, W2, S1, S2) is fp32 and updated in place.
 *   - Errors: an atlas_status is returned; atlas_last_error() gives a
 *     thread-local message for the last failing call on this thread.
 *   - Reentrant: no global mutable state besides the thread-local message,
 *     the opt-in kernel-timing records (atlas_profile_enable) and the
 *     per-GPU scratch array of atlas_scan_fwd_noalloc.
 */
#ifndef ATLAS_SCAN_H
#define ATLAS_SCAN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ATLAS_ABI_VERSION 1

typedef enum {
  ATLAS_OK = 0,
  ATLAS_ERR_INVALID_ARGUMENT = 1, /* null pointer, bad size, bad enum    */
  ATLAS_ERR_UNSUPPORTED_SHAPE = 2, /* shape outside the compiled kernels */
  ATLAS_ERR_HIP = 3,               /* a HIP runtime call failed          */
  ATLAS_ERR_WORKSPACE = 4          /* workspace smaller than required    */
} atlas_status;

typedef enum {
  ATLAS_DTYPE_F32 = 0,
  ATLAS_DTYPE_BF16 = 1,
  ATLAS_DTYPE_F16 = 2
} atlas_dtype;

/* Arithmetic of the matrix-core work inside the scan.
 *   ATLAS_COMPUTE_F32: fp32 MFMA everywhere (parity mode, ~1e-6 per chunk).
 *   ATLAS_COMPUTE_F16: inner-gradient GEMMs in fp32 MFMA; momentum assembly,
 *     Polar-Express and read-out products with fp16 MFMA operands, fp32
 *     accumulation and fp32 master copies (~2e-3 per chunk). */
typedef enum {
  ATLAS_COMPUTE_F32 = 0,
  ATLAS_COMPUTE_F16 = 1
} atlas_compute;

/* Shape and layout of one memory-layer scan.
 * q, k, v, y: element (b, t, h, d) at b*x_stride_b + t*x_stride_t + h*x_stride_h + d.
 * gates:      element (b, t, h)    at b*g_stride_b + t*g_stride_t + h.
 * A stride of 0 selects the dense token-major default of the reference,
 * (B, T, H, D) for q/k/v/y and (B, T, H) for gates.
 * W1, S1: dense (B, H, D, E); W2, S2: dense (B, H, E, D). */
typedef struct {
  int32_t B, T, H, D, E;
  int32_t chunk_size;    /* tokens per chunk (reference config.chunk_size)   */
  int32_t omega_window;  /* Omega window; <= 1 or gamma == NULL: no window    */
  int32_t ns_steps;      /* Polar-Express steps, 0..5                         */
  int32_t io_dtype;      /* atlas_dtype of q, k, v and y                      */
  int32_t gate_dtype;    /* atlas_dtype of alpha, eta, theta, gamma           */
  int32_t compute;       /* atlas_compute                                     */
  int32_t n_slices;      /* token slices per chunk (0 = choose automatically) */
  int64_t x_stride_b, x_stride_t, x_stride_h;
  int64_t g_stride_b, g_stride_t;
} atlas_scan_desc;

/* Bytes of device workspace atlas_scan_fwd needs for this descriptor
 * (0 if the descriptor is invalid; see atlas_last_error). */
size_t atlas_scan_workspace_size(const atlas_scan_desc* desc);

/* Runs the whole chunk loop of one memory layer.
 * q, k: feature-mapped queries/keys (after norm + polynomial), v: values.
 * alpha, theta, gamma: post-sigmoid gates; eta: post-sigmoid gate already
 * multiplied by max_lr (memory_layer.py:627-633).  gamma may be NULL.
 * W1, W2, S1, S2: chunk-start state in, final state out (fp32, in place).
 * y: read-out y_t = q_t + W1_t gelu(W2_t q_t) for every token (io_dtype).
 * T need not be a multiple of chunk_size: the tail is padded exactly as
 * memory_layer.py:649-660 (alpha=1, eta=theta=gamma=0, q=k=v=0), so the
 * returned S is zero in that case, as in the reference.
 * Shapes: the phase kernels take D = 32 with E in {32, 64, 128}, D = 64 with
 * E in {64, 128, 256} (E = 256 with ATLAS_COMPUTE_F16) and chunk_size <= 128
 * (a multiple of 4) where their LDS layouts fit a CU (not fp32 at chunk 128
 * with E = 128); every other shape with D and E multiples of 4, D <= 128,
 * E <= 256 and chunk_size <= 4096 (E = 256 in fp32 included) runs on a
 * per-token path (one chunk at a time: momentum and memory scans per
 * element, batched Polar-Express), slower but the same semantics.  Outside
 * that: ATLAS_ERR_UNSUPPORTED_SHAPE. */
atlas_status atlas_scan_fwd(const atlas_scan_desc* desc,
                            const void* q, const void* k, const void* v,
                            const void* alpha, const void* eta,
                            const void* theta, const void* gamma,
                            float* W1, float* W2, float* S1, float* S2,
                            void* y, void* workspace, size_t workspace_bytes,
                            void* stream);

/* atlas_scan_fwd without a caller-provided workspace, for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  No counterpart in the reference.
 * The workspace is a file-scope device array of
 * atlas_scan_noalloc_scratch_bytes() bytes (64 MiB) that each GPU the
 * library runs on holds until the process ends; the call allocates nothing.
 * Shapes whose workspace does not fit it (even with the gate tables of one
 * chunk at a time) return ATLAS_ERR_WORKSPACE: B*H = 64 with D = 64,
 * E = 128, cs = 64 fits (any T), the E = 256 configurations do not.  It
 * runs the phase kernels only: shapes that atlas_scan_fwd sends to its
 * per-token path return ATLAS_ERR_UNSUPPORTED_SHAPE here.  All
 * calls on one GPU share its array: calls that overlap in time on one GPU
 * (other streams, other host threads) race and must be serialised by the
 * caller.  Nothing in the array needs to start at zero. */
size_t atlas_scan_noalloc_scratch_bytes(void);
atlas_status atlas_scan_fwd_noalloc(const atlas_scan_desc* desc,
                                    const void* q, const void* k, const void* v,
                                    const void* alpha, const void* eta,
                                    const void* theta, const void* gamma,
                                    float* W1, float* W2, float* S1, float* S2,
                                    void* y, void* stream);

/* One chunk with precomputed momentum inputs: the operator of
 * fused_chunk.py:321-355 (semantics of its _regular_fwd, :279-314).
 * W1, SW1: (B, H, D, E); W2, SW2: (B, H, E, D) -- in/out, fp32.
 * momW1: (B, cs, H, D, E); momW2: (B, cs, H, E, D); theta, alpha: (B, cs, H);
 * q, y: (B, cs, H, D).  Inputs of io_dtype; gates of gate_dtype.
 * Workspace: atlas_fused_chunk_workspace_size(). */
size_t atlas_fused_chunk_workspace_size(int32_t B, int32_t H, int32_t D,
                                        int32_t E, int32_t cs);
atlas_status atlas_fused_chunk_fwd(int32_t B, int32_t cs, int32_t H, int32_t D,
                                   int32_t E, int32_t ns_steps,
                                   int32_t io_dtype, int32_t gate_dtype,
                                   int32_t compute,
                                   float* W1, float* W2, float* SW1, float* SW2,
                                   const void* momW1, const void* momW2,
                                   const void* theta, const void* alpha,
                                   const void* q, void* y,
                                   void* workspace, size_t workspace_bytes,
                                   void* stream);

/* Polar-Express on n independent (d1 x d2) row-major matrices,
 * min(d1, d2) <= 64 and max(d1, d2) <= 256.
 * X and Y may alias.  dtype applies to both.  norm_mode selects the
 * Frobenius normalisation: ATLAS_PE_NORM_EPS = sqrt(sum X^2 + 1e-12)
 * (memory_layer.py:55), ATLAS_PE_NORM_NO_EPS = sqrt(sum X^2) (optim.py:71). */
#define ATLAS_PE_NORM_EPS 0
#define ATLAS_PE_NORM_NO_EPS 1
atlas_status atlas_pe_batched(int64_t n, int32_t d1, int32_t d2,
                              int32_t ns_steps, int32_t norm_mode,
                              const void* X, void* Y, int32_t dtype,
                              int32_t compute, void* stream);

/* VJP of Polar-Express (the normalisation with the 1e-12 term and ns_steps
 * odd-quintic steps of polar_express, memory_layer.py:43-71; the
 * derivative autodiff takes through them) on n independent (d1 x d2)
 * row-major fp32 matrices: G holds the cotangent of PE(X) on entry and
 * dPE/dX^T G on return.  min(d1, d2) 32 with max 32/64/128, or 64 with
 * 64/128/256.  compute: ATLAS_COMPUTE_F32
 * (fp32 matrix-core operands) or ATLAS_COMPUTE_F16 (fp16 operands, each
 * scaled by a power of two, fp32 accumulation).  Workspace:
 * atlas_pe_vjp_workspace_size bytes (0 = unsupported; enough for either
 * compute mode).  X, G and the workspace 16-byte aligned. */
size_t atlas_pe_vjp_workspace_size(int32_t d1, int32_t d2, int32_t ns_steps);
atlas_status atlas_pe_vjp_batched(int64_t n, int32_t d1, int32_t d2, int32_t ns_steps,
                                  const float* X, float* G, int32_t compute,
                                  void* workspace, size_t workspace_bytes,
                                  void* stream);

/* h_t = g_t * h_{t-1} + x_t along T, for every (b, h) and state element.
 * h_init: (B, H, N) fp32; gates: (B, T, H) fp32; inputs, h_all: (B, T, H, N)
 * fp32; h_final: (B, H, N) fp32 (may alias h_init). */
atlas_status atlas_linear_scan(int32_t B, int32_t T, int32_t H, int64_t N,
                               const float* h_init, const float* gates,
                               const float* inputs, float* h_all,
                               float* h_final, void* stream);

/* Backward of atlas_linear_scan (the reverse-time scan of
 * kernels/triton_scan.py:119-161): from the forward's h_init (B, H, N),
 * gates (B, T, H), h_all (B, T, H, N) and the upstream dh_all (B, T, H, N)
 * and dh_final (B, H, N) (either may be NULL = zero), with
 * G_t = dh_all_t + [t = T-1] dh_final + gates_{t+1} G_{t+1}:
 *   d_inputs = G (B, T, H, N), d_h_init = gates_0 G_0 (B, H, N),
 *   d_gates_t = <G_t, h_{t-1}> (B, T, H), summed in a fixed order.
 * All fp32.  Workspace: atlas_linear_scan_bwd_workspace_size bytes. */
size_t atlas_linear_scan_bwd_workspace_size(int32_t B, int32_t T, int32_t H, int64_t N);
atlas_status atlas_linear_scan_bwd(int32_t B, int32_t T, int32_t H, int64_t N,
                                   const float* h_init, const float* gates,
                                   const float* h_all, const float* dh_all,
                                   const float* dh_final, float* d_h_init,
                                   float* d_gates, float* d_inputs, void* workspace,
                                   size_t workspace_bytes, void* stream);

/* Memory-layer prologue after the input projections: the part of
 * AtlasMemoryLayer.__call__ between the projections and the chunk loop
 * (atlas_jax/memory_layer.py:606-633): causal depthwise convolutions of q, k,
 * v (ShortConv, :303-329), RMS norm (:211-216) and the polynomial map
 * (:459-466) -- q: norm then map, k: map then norm -- and the sigmoid gates
 * with eta times max_lr, plus the retrieve gate sigmoid (:720-722).
 * proj: (B, T, proj_ld) output of one GEMM x @ W_all^T whose leading columns
 *   are [q (H*D) | k (H*D) | v (H*D) | gates (n_gates*H) | retrieve (H)],
 *   n_gates = 3 (alpha, eta, theta) or 4 (+ gamma); gate biases come in gate_b.
 * conv_w: (3, H*D, conv_kernel) and conv_b: (3, H*D) for q, k, v; poly:
 *   (poly_degree) coefficients (poly_degree 0: norm only).
 * q, k, v: (B, T, H, D) dense, out_dtype; gates: (n_gates, B, T, H) fp32;
 * retrieve: (B, T, H) fp32 (ignored unless has_retrieve).  D <= 128. */
atlas_status atlas_layer_prologue(int32_t B, int32_t T, int32_t H, int32_t D,
                                  int32_t conv_kernel, int32_t poly_degree,
                                  int32_t n_gates, int32_t has_retrieve,
                                  const void* proj, int64_t proj_ld,
                                  int32_t proj_dtype, const float* conv_w,
                                  const float* conv_b, const float* poly,
                                  const float* gate_b, float max_lr,
                                  void* q, void* k, void* v, int32_t out_dtype,
                                  float* gates, float* retrieve, void* stream);

/* Sliding-window causal attention with rotary embeddings, the attention of
 * the MAG blocks (atlas_jax/model.py:83-133 between the qkv projection and
 * to_out; atlas_jax/mag_transformer.py:63-79): for every (b, h) and query t,
 *   out_t = sum_{s <= t, t - s <= window} softmax_s(q'_t . k'_s / sqrt(D)) v_s
 * with q', k' the half-split rotary rotation (model.py:64-73) using the
 * caller's cos/sin tables (T, D/2) fp32 (model.py:50-62).  q, k, v:
 * (B, T, H, D) views sharing the element strides (multiples of 8; e.g. the
 * three thirds of the (B, T, 3*H*D) projection output); out: (B, T, H, D)
 * contiguous, same dtype.  io_dtype bf16 (1) or fp16 (2); fp16 matrix-core
 * operands with fp32 scores, softmax and accumulation.  D = 64. */
atlas_status atlas_swa_fwd(int32_t B, int32_t T, int32_t H, int32_t D, int32_t window,
                           const void* q, const void* k, const void* v, void* out,
                           int64_t stride_b, int64_t stride_t, int64_t stride_h,
                           int32_t io_dtype, const float* cos_tab, const float* sin_tab,
                           void* stream);

/* atlas_swa_fwd that also writes lse (B, H, T) fp32: the log of each
 * query's softmax normaliser of the scaled scores (the input of
 * atlas_swa_bwd).  No reference counterpart: the reference's autodiff keeps
 * what it needs itself. */
atlas_status atlas_swa_fwd_lse(int32_t B, int32_t T, int32_t H, int32_t D, int32_t window,
                               const void* q, const void* k, const void* v, void* out,
                               int64_t stride_b, int64_t stride_t, int64_t stride_h,
                               int32_t io_dtype, const float* cos_tab, const float* sin_tab,
                               float* lse, void* stream);

/* Backward of atlas_swa_fwd: the gradients the reference's autodiff takes
 * through SlidingWindowAttention.__call__'s attention core (model.py:109-129,
 * with the rotary rotation model.py:64-73) for the cotangent dout of its
 * output.  q, k, v, strides, io_dtype, cos/sin as for the forward; out and
 * lse: the forward's output and log-normalisers (atlas_swa_fwd_lse); dout:
 * (B, T, H, D) contiguous, io_dtype.  dq, dk, dv: (B, T, H, D) fp32
 * contiguous (written, not accumulated).  P is recomputed from lse; fp16
 * matrix-core operands, fp32 accumulation; no atomics (bitwise
 * reproducible).  Workspace: atlas_swa_bwd_workspace_size bytes (4-byte
 * aligned); out, dout, dq, dk, dv 16-byte aligned.  D = 64. */
size_t atlas_swa_bwd_workspace_size(int32_t B, int32_t T, int32_t H);
atlas_status atlas_swa_bwd(int32_t B, int32_t T, int32_t H, int32_t D, int32_t window,
                           const void* q, const void* k, const void* v, const void* out,
                           const void* dout, const float* lse,
                           int64_t stride_b, int64_t stride_t, int64_t stride_h,
                           int32_t io_dtype, const float* cos_tab, const float* sin_tab,
                           float* dq, float* dk, float* dv,
                           void* workspace, size_t workspace_bytes, void* stream);

/* atlas_scan_fwd that also writes every chunk's start state into
 * state_trace: n_chunks = ceil(T / chunk_size) blocks of four arrays, W1
 * (B, H, D, E), W2 (B, H, E, D), S1 (B, H, D, E), S2 (B, H, E, D), fp32
 * (chunk 0 holds the initial state); the input of atlas_scan_bwd.
 * All forward shapes.  It has no counterpart in the reference, whose autodiff keeps
 * (or, with use_checkpoint, recomputes) the carried states itself. */
atlas_status atlas_scan_fwd_trace(const atlas_scan_desc* desc,
                                  const void* q, const void* k, const void* v,
                                  const void* alpha, const void* eta,
                                  const void* theta, const void* gamma,
                                  float* W1, float* W2, float* S1, float* S2,
                                  void* y, float* state_trace,
                                  void* workspace, size_t workspace_bytes,
                                  void* stream);

/* Backward of atlas_scan_fwd: the VJP of the whole layer's chunk loop
 * (memory_layer.py:649-711 with _process_chunk_deep :496-541, the gradients
 * the reference obtains by differentiating that loop, including the custom
 * VJP of fused_chunk_scan, kernels/fused_chunk.py:357-379, and the reverse
 * scan of kernels/triton_scan.py:119-161).  Recomputes every chunk's forward
 * from its start state (a trace pass stores the start states) and returns:
 *   dq, dk, dv (B, T, H, D); dalpha, deta, dtheta, dgamma (B, T, H);
 *   dW1_0, dS1_0 (B, H, D, E), dW2_0, dS2_0 (B, H, E, D): the gradients of
 *   <dy, y> + <dW1, W1_T> + <dW2, W2_T> + <dS1, S1_T> + <dS2, S2_T>, with
 *   y and the final state (W1_T .. S2_T) the outputs of atlas_scan_fwd for
 *   the same inputs and initial state (W1 .. S2, read only).
 * state_trace: the chunk-start states written by atlas_scan_fwd_trace for the
 * same call (then the backward linearises around exactly the forward's
 * trajectory and skips its own forward pass), or NULL (the backward first
 * runs a fp32 forward pass that stores them in the workspace).
 * dy and the four state cotangents may be NULL (zero); gamma may be NULL
 * (no Omega window, as in atlas_scan_fwd), and dgamma may be NULL (not
 * written); without a window dgamma is written as zeros.
 * flags: ATLAS_BWD_PE_STE = straight-through Polar-Express (backward is the
 * identity, memory_layer.py:74-76); ATLAS_BWD_STOP_GRAD_CHUNKS = the carry
 * is detached at every chunk start (memory_layer.py:665), so the initial
 * state receives no gradient and each chunk's end state only its own.
 * compute: ATLAS_COMPUTE_F32, or ATLAS_COMPUTE_F16 for Polar-Express and
 * its VJP on fp16 matrix-core operands (everything else stays fp32).
 * Restrictions: fp32 inputs (io_dtype, gate_dtype); dense
 * (B, T, H, D) / (B, T, H) strides; T a multiple of chunk_size (pad as the
 * reference does, :649-660: alpha 1, eta = theta = gamma = 0, q = k = v = 0,
 * and drop the padded rows of the gradients); chunk_size <= 256; D 32 with
 * E 32/64/128, or D 64 with E 64/128/256.  q, k, the states, their cotangents,
 * the state gradients and the workspace must be 16-byte aligned.
 * Workspace: atlas_scan_bwd_workspace_size bytes (0 = unsupported desc).
 * Streams: with more than one chunk, the chunks' forward recomputes and
 * backwards alternate between `stream` and a second stream of the
 * library's (one per device, default priority, created on first use and
 * kept for the process), each chunk's recompute beside the backward of the
 * chunk after it; the second stream waits for the work issued on `stream`
 * before the call, and `stream` waits for all of the second stream's work
 * before the call returns, so the call behaves as if everything ran on
 * `stream` (concurrent calls on one device share that second stream). */
#define ATLAS_BWD_PE_STE 1
#define ATLAS_BWD_STOP_GRAD_CHUNKS 2
size_t atlas_scan_bwd_workspace_size(const atlas_scan_desc* desc);
atlas_status atlas_scan_bwd(const atlas_scan_desc* desc, int32_t flags,
                            const float* q, const float* k, const float* v,
                            const float* alpha, const float* eta,
                            const float* theta, const float* gamma,
                            const float* W1, const float* W2,
                            const float* S1, const float* S2,
                            const float* state_trace, const float* dy, const float* dW1, const float* dW2,
                            const float* dS1, const float* dS2,
                            float* dq, float* dk, float* dv,
                            float* dalpha, float* deta, float* dtheta,
                            float* dgamma, float* dW1_0, float* dW2_0,
                            float* dS1_0, float* dS2_0,
                            void* workspace, size_t workspace_bytes,
                            void* stream);

/* Kernel timing for measurement tools (not for production use).
 * While enabled, atlas_scan_fwd brackets every kernel it launches with HIP
 * events on the caller's stream; atlas_profile_read synchronises those events
 * and returns, for one kernel kind, the launch count and the summed duration.
 * Kinds: 0 = prep, 1 = phase W2, 2 = phase W1, 3 = finalize (W_end only when
 * kind 5 runs), 4 = slice prefix, 5 = the next chunk's prep together with this
 * chunk's y (one launch).
 * atlas_profile_enable(1) also clears previous records.  Process-wide state:
 * enable it only around single-threaded measurement runs. */
#define ATLAS_KERNEL_PREP 0
#define ATLAS_KERNEL_PHASE2 1
#define ATLAS_KERNEL_PHASE1 2
#define ATLAS_KERNEL_FIN 3
#define ATLAS_KERNEL_PREFIX 4
#define ATLAS_KERNEL_TAIL 5
atlas_status atlas_profile_enable(int32_t enable);
atlas_status atlas_profile_read(int32_t kind, int64_t* launches, double* total_ms);

/* Matrix-core calibration for measurement tools (no reference counterpart):
 * the sustained dense fp16 rate (TFLOP/s) of independent
 * v_mfma_f32_32x32x16_f16 chains with pseudo-random operands on every CU at
 * waves_per_simd (1..4) waves per SIMD, about 25 ms on `stream`
 * (synchronised).  It measures what the part sustains under its power limit
 * for real data, next to the datasheet's dense peak. */
atlas_status atlas_profile_mfma_rate(int32_t waves_per_simd, double* tflops, void* stream);

/* Thread-local message describing the last error on this thread ("" if none). */
const char* atlas_last_error(void);

/* ATLAS_ABI_VERSION of the loaded library. */
int32_t atlas_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* ATLAS_SCAN_H */
