/*
 * morphottention -- MI355X (gfx950) native fused morpho-attention, C ABI.
 *
 * Drop-in boundary for the reference extension's host launchers
 *   attention_forward_kernel_launcher   packages/morphottention/csrc/cuda/attention/attention.cuh:28-31
 *   attention_backward_kernel_launcher  packages/morphottention/csrc/cuda/attention/attention.cuh:33-38
 * and of the ATen ops that wrap them
 *   morpho_forward / morpho_backward    packages/morphottention/csrc/cuda/attention/attention.cpp:15-117
 *
 * Differences from the reference launchers, all deliberate:
 *   - `causal` is honoured at run time (the reference drops it, attention.cpp:46-54);
 *     its other bits select the reference's compile-time variants (see morpho_mode);
 *   - cube_m in {16, 32, 64} and head_dim_v = D / H in {32, 64, 128} are accepted
 *     (the reference accepts only 64 / 64, attention.cu:494,535);
 *   - the backward returns the complete gradient, including the query-side code
 *     gradient the reference drops (attention.cu:446-451,472-482);
 *   - scratch memory is passed in by the caller (`workspace`), sized by the
 *     *_workspace_size queries, so the library never allocates device memory;
 *   - errors are returned as status codes instead of C++ exceptions.
 *
 * Data layout (all device pointers, row-major, contiguous, float16 = IEEE binary16):
 *   X, out, grad_out, dX   [B, N, D]           float16
 *   W_phi, dW_phi          [D, H * cube_m]     float16  (head h owns columns h*cube_m ..)
 *   gate_q, gate_k, d_*    [H, cube_m]         float16
 *   W_V, dW_V              [D, D]              float16  (head h owns columns h*(D/H) ..)
 *   lse                    [B * H, N]          float32  base-2 log-sum-exp of the row scores
 *
 * All calls are asynchronous on `stream` (a hipStream_t; NULL = legacy default
 * stream) and use the device that is current on the calling thread. Calls that
 * share a workspace must be ordered on one stream.
 */
#ifndef MORPHOTTENTION_H
#define MORPHOTTENTION_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* morpho_stream_t; /* identical to hipStream_t */

/* Bits of the `causal` argument of morpho_forward / morpho_backward. 0 and 1
 * keep their plain meaning (non-causal / causal, sigmoid cube projection, the
 * diagonal kept). The other bits select variants that the reference defines
 * at compile time but never wires: MASK_DIAG (declarations.cuh:79-82) drops
 * key j == query i; HardTanh01 (phi = clamp((z + 1) / 2, 0, 1)) and Identity
 * (phi = z) replace the sigmoid cube projection (cube.cuh:9-17,29-35). Pass
 * the same bits to the backward as to the forward. */
enum morpho_mode {
  MORPHO_MODE_CAUSAL = 1,
  MORPHO_MODE_MASK_DIAG = 2,
  MORPHO_MODE_PROJ_HARDTANH01 = 4,
  MORPHO_MODE_PROJ_IDENTITY = 8,
  /* Soft aggregation only: always use the element-wise kernels instead of the
   * product form on MFMA (which falls back to them by itself when it cannot
   * guarantee its precision). No reference counterpart; for tests and
   * measurement. */
  MORPHO_MODE_SOFT_EXACT = 16,
  /* morpho_backward only (ignored by the forward, rejected by the soft entry
   * points): the gradients are the same bits on every run with the same
   * inputs. The backward's dq and dS row sums are then summed from per-key-
   * block partials in a fixed order instead of by fp32 atomics; the workspace
   * grows by (N / keys per block) x the dq buffer
   * (morpho_backward_workspace_size_for_mode). Without the bit only those
   * two sums depend on the order of atomics. No reference counterpart: the
   * reference adds dX and the weight gradients with fp16 atomics
   * (attention.cu:389-480), so its gradients vary from run to run. */
  MORPHO_MODE_DETERMINISTIC = 32
};

enum morpho_status {
  MORPHO_OK = 0,
  MORPHO_ERR_INVALID_ARGUMENT = 1, /* bad shape, null pointer, unsupported size */
  MORPHO_ERR_UNSUPPORTED = 2,      /* valid request this build does not implement */
  MORPHO_ERR_WORKSPACE = 3,        /* workspace missing or too small */
  MORPHO_ERR_HIP = 4               /* a HIP runtime call failed */
};

/* Library version, MAJOR * 10000 + MINOR * 100 + PATCH. No reference counterpart. */
int morpho_version(void);

/* Short text for a status code. No reference counterpart (the reference throws c10::Error). */
const char* morpho_status_string(int status);

/* Human-readable detail of the last failure on the calling thread, "" if none.
 * Carries the same messages as the reference's TORCH_CHECKs (attention.cpp:9-38,
 * attention.cu:491-495). */
const char* morpho_last_error(void);

/* Bytes of device workspace morpho_forward needs (0 on invalid sizes).
 * The forward workspace holds the projected codes and values; passing it
 * unchanged to morpho_backward lets the backward skip recomputing them.
 * Sizes every entry point accepts: cube_m in {16, 32, 64}, D / H in {32, 64,
 * 128}, B*N <= 2^28, B*N*D <= 2^34, B*N*H*cube_m <= 2^33, D and H*cube_m
 * <= 65536 (every kernel grid then stays below 2^31 work-items); larger
 * problems fail with MORPHO_ERR_INVALID_ARGUMENT. */
size_t morpho_forward_workspace_size(int64_t B, int64_t N, int64_t D, int64_t H, int64_t cube_m);

/* Forward. Replaces attention_forward_kernel_launcher (attention.cuh:28-31) and
 * the launch part of morpho_forward (attention.cpp:15-57).
 * Writes out [B, N, D] (float16) and lse [B*H, N] (float32, base 2;
 * -FLT_MAX, with out = 0, for a row without unmasked keys: only query 0 under
 * MORPHO_MODE_CAUSAL | MORPHO_MODE_MASK_DIAG, or N = 1 with MASK_DIAG).
 * Numeric range: the key codes hold 2 * scale * log2(e) * gate_q[h][c] *
 * gate_k[h][c] * phi in float16, so |scale * gate_q * gate_k * phi| must stay
 * below 22,700 for every code (phi <= 1 except with the Identity projection);
 * beyond it the codes overflow and the outputs are NaN. The reference keeps
 * gate * phi in float16 and applies scale in float32. */
int morpho_forward(const void* X, const void* W_phi, const void* gate_q, const void* gate_k, const void* W_V,
                   void* out, float* lse, int64_t B, int64_t N, int64_t D, int64_t H, int64_t cube_m, float scale,
                   int causal, void* workspace, size_t workspace_bytes, morpho_stream_t stream);

/* Bytes of device memory inside the library used by morpho_forward_noalloc,
 * per GPU. */
#define MORPHO_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)

/* Allocation-free forward. No counterpart in the reference: for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). Same arguments, kernels and
 * results as morpho_forward, without the workspace: the library's own static
 * device array of MORPHO_NOALLOC_SCRATCH_BYTES serves as the workspace (one
 * per GPU, held from the library's first use on that GPU until the process
 * ends). Problems whose forward workspace (morpho_forward_workspace_size)
 * exceeds it are rejected with MORPHO_ERR_WORKSPACE before anything runs; at
 * cube_m = 16 and D / H = 64 that is up to about 90,000 (token, head) pairs,
 * fewer as the weights grow with D: B = 1, N = 4096, D = 1024, H = 16 needs
 * 28 MiB. Every call on a GPU shares that GPU's
 * array: calls that overlap in time on one GPU (unordered streams or
 * threads) race, and the array is not a forward workspace that a later
 * morpho_backward may be given (pass NULL there to recompute). Nothing is
 * allocated or freed. */
int morpho_forward_noalloc(const void* X, const void* W_phi, const void* gate_q, const void* gate_k,
                           const void* W_V, void* out, float* lse, int64_t B, int64_t N, int64_t D, int64_t H,
                           int64_t cube_m, float scale, int causal, morpho_stream_t stream);

/* Bytes of device workspace morpho_backward needs. With `have_forward_workspace`
 * = 0 this includes room to recompute the projection. */
size_t morpho_backward_workspace_size(int64_t B, int64_t N, int64_t D, int64_t H, int64_t cube_m,
                                      int have_forward_workspace);

/* The same for the mode bits `causal` that morpho_backward will be given
 * (0 on invalid sizes or bits). Only MORPHO_MODE_DETERMINISTIC changes the
 * size: it adds the per-key-block partials. No reference counterpart. */
size_t morpho_backward_workspace_size_for_mode(int64_t B, int64_t N, int64_t D, int64_t H, int64_t cube_m,
                                               int have_forward_workspace, int causal);

/* Backward. Replaces attention_backward_kernel_launcher (attention.cuh:33-38)
 * and the launch part of morpho_backward (attention.cpp:59-117).
 * Writes dX, dW_phi, d_gate_q, d_gate_k, dW_V (float16, shaped like their
 * inputs); every output is overwritten, none needs zeroing by the caller.
 * `forward_workspace` is either NULL (the projection is recomputed from X) or
 * the workspace of the morpho_forward call that produced `out` and `lse`,
 * unchanged since. */
int morpho_backward(const void* grad_out, const void* X, const void* W_phi, const void* gate_q, const void* gate_k,
                    const void* W_V, const void* out, const float* lse, void* dX, void* dW_phi, void* d_gate_q,
                    void* d_gate_k, void* dW_V, int64_t B, int64_t N, int64_t D, int64_t H, int64_t cube_m,
                    float scale, int causal, const void* forward_workspace, void* workspace, size_t workspace_bytes,
                    morpho_stream_t stream);

/* Soft tropical aggregation: the morpho scores s_ij combine with the values
 * in a soft max-plus (sgn = +1, dilation) or min-plus (sgn = -1, erosion)
 * product instead of the softmax-weighted sum,
 *     out_ic = sgn * tau * ln sum_j exp(sgn * (s_ij + V_jc) / tau),
 * built from the accumulators of packages/morphottention/csrc/cuda/morfology/
 * soft_morph.cuh:21-69 (lse_update, morph_accumulate, lse_merge,
 * lse_finalize), which the reference defines but never calls; it has no
 * launcher or op for them, so these entry points have no counterpart to
 * replace. Shapes, dtypes, `mode` bits and workspace rules are those of
 * morpho_forward / morpho_backward; the forward workspace size is
 * morpho_soft_forward_workspace_size. `tau` points to one float32 in device
 * memory (> 0; read by the kernels, so it may be a learnable parameter).
 * zb [B*H, N, D/H] float32 receives log2 sum_j 2^(log2e sgn (s_ij + V_jc) /
 * tau), so out = sgn tau ln2 zb (-FLT_MAX, with out = 0, for a row without
 * keys); the backward needs it. */
int morpho_soft_forward(const void* X, const void* W_phi, const void* gate_q, const void* gate_k, const void* W_V,
                        const float* tau, void* out, float* zb, int64_t B, int64_t N, int64_t D, int64_t H,
                        int64_t cube_m, float scale, int mode, int sgn, void* workspace, size_t workspace_bytes,
                        morpho_stream_t stream);

/* Bytes of device workspace morpho_soft_forward needs: the projection of
 * morpho_forward_workspace_size plus the state of the product form. */
size_t morpho_soft_forward_workspace_size(int64_t B, int64_t N, int64_t D, int64_t H, int64_t cube_m);

/* Bytes of device workspace morpho_soft_backward needs (as
 * morpho_backward_workspace_size, plus the dtau partial sums). */
size_t morpho_soft_backward_workspace_size(int64_t B, int64_t N, int64_t D, int64_t H, int64_t cube_m,
                                           int have_forward_workspace);

/* Backward of morpho_soft_forward: dX, dW_phi, d_gate_q, d_gate_k, dW_V as in
 * morpho_backward, and dtau (one float32 in device memory) from
 * morph_dtau_term (soft_morph.cuh:77-80) summed over every output. */
int morpho_soft_backward(const void* grad_out, const void* X, const void* W_phi, const void* gate_q,
                         const void* gate_k, const void* W_V, const float* tau, const float* zb, void* dX,
                         void* dW_phi, void* d_gate_q, void* d_gate_k, void* dW_V, float* dtau, int64_t B, int64_t N,
                         int64_t D, int64_t H, int64_t cube_m, float scale, int mode, int sgn,
                         const void* forward_workspace, void* workspace, size_t workspace_bytes,
                         morpho_stream_t stream);

/* Per-kernel timing for measurement harnesses. No reference counterpart.
 * When enabled (process-wide), every kernel the library launches, from any
 * thread, carries a start and a stop HIP event bound to its dispatch
 * (hipExtLaunchKernel: the kernel's own start and end, no marker packets
 * between kernels, so the timed stream runs as it does untimed).
 * morpho_timing_read
 * synchronises on the recorded events and returns up to `max_entries`
 * (name, milliseconds) pairs, oldest first, then clears the record; names
 * point to static strings. */
int morpho_timing_enable(int enable);
int morpho_timing_read(const char** names, float* ms, int max_entries);
/* Restricts the timing to the launches of one name (as morpho_timing_read
 * reports it, e.g. "attn_bwd"); NULL or "" times every launch again. Each
 * timed dispatch costs a few microseconds of queue time before it, so a
 * harness that times a whole run times only the kernel it reports. */
int morpho_timing_only(const char* name);

#ifdef __cplusplus
}
#endif

#endif /* MORPHOTTENTION_H */
