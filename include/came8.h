/*
 * came8.h -- C ABI of the MI355X CAME 8-bit optimizer step (libcame8.so).
 *
 * Plain pointers, sizes and a hipStream_t; no torch types.  The caller owns
 * every buffer: parameters, gradients, the quantised optimizer state and a
 * workspace sized by came8_workspace_size().  All launches are asynchronous
 * on the given stream; no call synchronises the host with the device.
 *
 * Reference interfaces replaced (paths relative to the reference tree):
 *   came8_step           -- the per-parameter CUDA chains that the full8bit
 *                           optimizers run for one step:
 *                           came_full_factored_sq_step          came_pytorch/came_cuda/csrc/came_bindings.cpp:1406-1453
 *                           came_full_factored_expavg_res_prepare              came_bindings.cpp:1589-1633
 *                           came_full_factored_res_step                        came_bindings.cpp:1507-1549
 *                           came_full_factored_param_update                    came_bindings.cpp:1675-1691
 *                           came_full_nonfactored_step                         came_bindings.cpp:856-915
 *                           came_full_factored_step_multitensor_same_shape_ptrs came_bindings.cpp:1795-1907
 *                           came_full_nonfactored_step_multitensor_ptrs        came_bindings.cpp:1170-1222
 *                         (Python wrappers: came_pytorch/came_cuda/__init__.py:253-963;
 *                          arithmetic: came_pytorch/CAME8bitFull.py:1006-1075);
 *                         and, with fp32 states, CAMECUDA's steps:
 *                           came_fp_factored_step               came_bindings.cpp:1692-1760
 *                         (Python: came_cuda/__init__.py:820-860; arithmetic:
 *                          came_pytorch/CAMECUDA.py:275-326);
 *                         and, with the 8bit2d state layout, CAME8bit2D's step:
 *                           came2d_step                         came_bindings.cpp:617-759
 *                         (Python: came_pytorch/CAME8bit2D.py; kernels:
 *                          came_cuda/csrc/came_kernels.cu:3599-4040).
 *   came8_quantize_blockwise / came8_dequantize_blockwise
 *                        -- blockwise_quant / blockwise_dequant
 *                           came_bindings.cpp:756-801 (Python: came_cuda/__init__.py:205-228;
 *                           arithmetic: came_pytorch/blockwise_quantization.py:66-82,112-124).
 *
 * Errors: every entry point returns CAME8_OK (0) or a negative CAME8_E* code;
 * came8_last_error() returns the message of the last failure on the calling
 * thread (the reference raised RuntimeError from TORCH_CHECK with that text).
 */
#ifndef CAME8_H
#define CAME8_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CAME8_ABI_VERSION 5

/* element types of parameters and gradients */
#define CAME8_F32 0
#define CAME8_BF16 1
#define CAME8_F16 2

/* status codes */
#define CAME8_OK 0
#define CAME8_EINVAL (-1)   /* bad argument: shape, dtype, block size, null pointer */
#define CAME8_ESPACE (-2)   /* workspace smaller than came8_workspace_size() */
#define CAME8_EHIP (-3)     /* a HIP runtime call failed */

/* came8_tensor.state_kind */
#define CAME8_STATE_Q8 0   /* 8-bit states, full8bit layout (CAME8bit, CAME8bitFull, CAME8bitMemory) */
#define CAME8_STATE_FP32 1 /* fp32 states, CAMECUDA layout */
#define CAME8_STATE_8BIT2D 2 /* 8-bit states, 8bit2d layout (CAME8bit2D): momentum in 16x16 tiles */
#define CAME8_STATE_Q8_MATRIX 3 /* 8-bit states of an N-D tensor (ndim >= 3) blocked per matrix, as the
                                   reference's CUDA N-D path keeps them (came_pytorch/CAME8bitFull.py:
                                   790-842, views :188-223): the codes as in CAME8_STATE_Q8, but every one of
                                   the P matrices has blocks of its own -- exp_avg_absmax [P][ceil(R*C/B)],
                                   row_absmax [2][P][ceil(R/B)], col_absmax [2][P][ceil(C/B)] (ABI 5) */

/* flags for came8_hparams.flags.  By default the clip's update norm is the reference's own: torch's
 * CPU norm(2) order (eight fp32 fused-multiply-add chains, came_pytorch/CAME8bitFull.py:121-122,1032),
 * replayed bit for bit in parallel. */
#define CAME8_FLAG_REFERENCE_NORM 1u /* the default; accepted for callers of ABI 3 */
#define CAME8_FLAG_EXACT_NORM 2u     /* opt-in: the update norm as the exactly rounded fp64 sum instead
                                        (one pass less; differs from the reference by the fp32 chains'
                                        rounding error, ~1e-4 relative at 2^22 elements) */
#define CAME8_FLAG_PLAN_ONLY 4u      /* build and upload the launch plan for this workspace and tag, launch
                                        nothing (prepares a later capture into a HIP graph) */
#define CAME8_FLAG_FP16_UPDATE 8u    /* unfactored (1-D) tensors of the 8-bit layout: the momentum takes the
                                        update rsqrt(v) * g rounded to fp16 (round to nearest even), then
                                        divided by the clip, as the reference's fp16-update CUDA kernels
                                        store it (came_pytorch/came_cuda/csrc/came_kernels.cu:1068-1122,
                                        1546-1601; selected by CAME8bitFull.py:488-509, and always by
                                        CAME8bitMemory.py:524-557).  The clip's norm stays that of the fp32
                                        update.  Lossy: the update moves by up to 2^-11 relative. */

/* flags for came8_tensor.tensor_flags */
#define CAME8_TENSOR_FP16_UPDATE 1u  /* this unfactored tensor takes the fp16-update rounding of
                                        CAME8_FLAG_FP16_UPDATE on its own: the reference selects those kernels
                                        per tensor (CAME8bit routes a 1-D tensor to them only on some of its
                                        paths, came_pytorch/CAME8bit.py:224-245,441-529,712-861) */

/*
 * One parameter tensor and its full8bit state, laid out exactly as the
 * reference's CPU branch of CAME8bitFull._init_state keeps it
 * (came_pytorch/CAME8bitFull.py:748-788, 919-923):
 *
 *   shape S = (..., R, C), numel N = P*R*C with P = prod(S[:-2]) (P = 1 for 2-D).
 *   exp_avg_q        int8   [N]                 (row-major, flat 256-element blocks)
 *   exp_avg_absmax   f32    [ceil(N/B)]
 *   factored (ndim >= 2):
 *     row_q          uint8  [2][P*R]  ([0] = exp_avg_sq_row, [1] = exp_avg_res_row)
 *     row_absmax     f32    [2][ceil(P*R/B)]
 *     col_q          uint8  [2][P*C]  ([0] = exp_avg_sq_col, [1] = exp_avg_res_col)
 *     col_absmax     f32    [2][ceil(P*C/B)]
 *   non-factored (ndim == 1; R = 1, C = N, P = 1):
 *     row_q          uint8  [N]       (exp_avg_sq_q)
 *     row_absmax     f32    [ceil(N/B)] (exp_avg_sq_absmax)
 *     col_q, col_absmax unused (NULL)
 *
 * param and grad are contiguous; param is updated in place.
 *
 * With state_kind = CAME8_STATE_FP32 the states are the fp32 tensors of the
 * reference's CAMECUDA (came_pytorch/CAMECUDA.py:83-104), passed through the
 * same fields (cast to the field types):
 *   exp_avg_q      -> exp_avg          float [N]
 *   row_q          -> exp_avg_sq_row   float [P*R]   (1-D: exp_avg_sq float [N])
 *   row_absmax     -> exp_avg_res_row  float [P*R]   (1-D: unused)
 *   col_q          -> exp_avg_sq_col   float [P*C]
 *   col_absmax     -> exp_avg_res_col  float [P*C]
 *   exp_avg_absmax    unused (may be NULL)
 * The arithmetic is CAMECUDA._step_param_generic (CAMECUDA.py:275-326): the
 * 8-bit step's, with the states kept in fp32 and no quantisation.  block_size
 * then only shapes the work decomposition (a power of two in [8, 2048]).
 *
 * With state_kind = CAME8_STATE_8BIT2D the tensor is a 2-D matrix (prefix 1,
 * factored 1) with the reference's 8bit2d state (came_pytorch/came8bit2d_state.py:33-75):
 *   exp_avg_q        int8   [R*C]            row-major momentum codes
 *   exp_avg_absmax   f32    [ceil(R/16)*ceil(C/16)]  one absmax per 16x16 tile,
 *                                            tile (ty, tx) at ty*ceil(C/16)+tx; 0 = no momentum yet
 *   row_q, row_absmax          exp_avg_sq_row   uint8 [R], f32 [ceil(R/B)]
 *   col_q, col_absmax          exp_avg_sq_col   uint8 [C], f32 [ceil(C/B)]
 *   res_row_q, res_row_absmax  exp_avg_res_row  uint8 [R], f32 [ceil(R/B)]
 *   res_col_q, res_col_absmax  exp_avg_res_col  uint8 [C], f32 [ceil(C/B)]
 *   res_row_partial  f32 [R*ceil(C/16)], res_col_partial f32 [C*ceil(R/16)]: the
 *                    reference's state-resident scratch for each tile's residual sums
 *                    per row and per column; used as such when both are given, else
 *                    the workspace holds them (NULL both)
 * and the arithmetic of the reference's CUDA 8bit2d step (came_pytorch/came_cuda/csrc/
 * came_kernels.cu:60-96, 198-243, 298-333, 595-619, 2584-2780, 3333-3367; launch order
 * came_kernels.cu:3599-4040): float32 EMAs (old*beta)+((1-beta)*mean), momentum
 * requantised per tile, multiplicative weight decay p*(1-lr*wd), and the parameter written
 * from the requantised momentum.  block_size must be 256, as the reference requires
 * (came_bindings.cpp:690).  The res_* fields are used only by this kind.
 */
typedef struct came8_tensor {
  void* param;
  const void* grad;
  int8_t* exp_avg_q;
  float* exp_avg_absmax;
  uint8_t* row_q;
  float* row_absmax;
  uint8_t* col_q;
  float* col_absmax;
  int64_t prefix; /* P */
  int64_t rows;   /* R */
  int64_t cols;   /* C */
  int32_t param_dtype; /* CAME8_F32 / CAME8_BF16 / CAME8_F16 */
  int32_t grad_dtype;
  int32_t factored;    /* 1 for ndim >= 2, 0 for 1-D */
  int32_t state_kind;  /* CAME8_STATE_Q8 (0), CAME8_STATE_FP32 or CAME8_STATE_8BIT2D */
  uint8_t* res_row_q;  /* CAME8_STATE_8BIT2D only (NULL otherwise) */
  float* res_row_absmax;
  uint8_t* res_col_q;
  float* res_col_absmax;
  float* res_row_partial;  /* CAME8_STATE_8BIT2D only, optional (NULL: workspace) */
  float* res_col_partial;
  uint32_t tensor_flags;   /* CAME8_TENSOR_* (ABI 5) */
  int32_t reserved;        /* 0 */
} came8_tensor;

/* Hyper-parameters of one param group (the reference's group keys, as Python floats). */
typedef struct came8_hparams {
  double lr;
  double beta1, beta2, beta3;
  double eps0, eps1;
  double clip_threshold;
  double weight_decay;
  int32_t block_size;
  uint32_t flags;
} came8_hparams;

/* Library identification. */
const char* came8_version(void);
int came8_abi_version(void);

/* Message of the last failing call on this thread ("" if none). */
const char* came8_last_error(void);

/*
 * Bytes of device workspace came8_step needs for this tensor list and block
 * size.  Depends only on shapes, dtypes and block size.
 */
int came8_workspace_size(const came8_tensor* tensors, int32_t n_tensors, int32_t block_size, size_t* bytes);

/*
 * Forget every cached launch plan for `workspace` (call when freeing it; frees
 * the host copies the library keeps of its uploads).  No reference
 * counterpart: the reference rebuilt pointer tables on every call
 * (came_pytorch/came_cuda/csrc/came_bindings.cpp:461-478).
 */
int came8_release_workspace(const void* workspace);

/*
 * One CAME 8-bit step over all tensors of a param group: the factored update
 * (row/column second moments, update-RMS clip, beta1 momentum, confidence
 * residual, weight decay, parameter write) for ndim >= 2 tensors, the
 * unfactored update for 1-D tensors, and blockwise int8/uint8 requantisation
 * of every state.  Arithmetic follows came_pytorch/CAME8bitFull.py:1006-1075.
 * Enqueued on `stream`; returns before the device finishes.
 *
 * The head of the workspace holds the launch plan.  `workspace_tag` names the
 * caller's current allocation of `workspace` (a value it never reuses for
 * another allocation, e.g. a process-wide counter): with a nonzero tag the
 * plan is re-uploaded only when the tensor list (pointers, shapes, dtypes) or
 * the block size changes, and the caller must not write to the workspace
 * between calls; tag 0 uploads on every call.
 *
 * Under HIP graph capture of `stream` the call only enqueues kernel launches, so the plan must exist
 * already: a call that would have to build or upload it while the stream is capturing fails with
 * CAME8_EINVAL.  Prepare with one eager call, or with CAME8_FLAG_PLAN_ONLY, before capture.
 */
int came8_step(const came8_tensor* tensors, int32_t n_tensors, const came8_hparams* hp,
               void* workspace, size_t workspace_bytes, uint64_t workspace_tag, void* stream);

/*
 * came8_step without a caller workspace, for callers that cannot allocate device memory (code under
 * HIP graph capture that must not call hipMalloc, tight serving loops, harnesses that forbid
 * allocation).  No counterpart in the reference.  The workspace is a static 32 MiB array in the
 * library's code object (one per GPU, held until the process ends); the call allocates nothing.
 * Tensor lists whose workspace (came8_workspace_size) exceeds 32 MiB fail with CAME8_ESPACE.  Every
 * call on one GPU shares that GPU's array and its cached launch plan: calls that overlap on one GPU
 * (other streams, other threads) race and must be serialised by the caller.  Otherwise as
 * came8_step with a nonzero workspace tag (the plan is rebuilt when the tensor list changes).
 */
int came8_step_static(const came8_tensor* tensors, int32_t n_tensors, const came8_hparams* hp, void* stream);

/*
 * Per-kernel device timing.  While enabled, every launch of came8_step is
 * bracketed by HIP events recorded on the launch stream; came8_profile_read
 * waits for the recorded events and returns, per kernel phase, the number of
 * launches, their summed device time and their summed algorithmic bytes (each
 * operand the kernel must touch counted once).  No reference counterpart
 * beyond its host-side dispatch timing (came_pytorch/CAME8bit.py:695-710).
 */
typedef struct came8_phase_stat {
  char name[32];
  int64_t launches;
  double total_ms;
  double alg_bytes;
} came8_phase_stat;

int came8_profile_enable(int32_t on);
int came8_profile_read(came8_phase_stat* out, int32_t max_phases, int32_t* n_phases, int32_t reset);

/*
 * Inspection: the clip divisor max(rms(u) / clip_threshold, 1) that the last came8_step on this
 * workspace and tag computed for each of its n_tensors tensors, copied to out[] (host memory) after
 * the stream has finished that step.  Synchronises the host with `stream`.  No reference
 * counterpart (the reference keeps the value in a device scratch tensor); it lets a caller check
 * the update norm, the one reduction whose rounding order the reference fixes
 * (came_pytorch/CAME8bitFull.py:121-122,1032).
 */
int came8_read_clip(const void* workspace, uint64_t workspace_tag, int32_t n_tensors, float* out, void* stream);

/*
 * Per-stream resources: came8_step keeps one side stream and two events per (device, caller stream)
 * it has stepped on (launches of a pass with many kernel variants are spread over the caller's
 * stream and that side stream, and the tensors with the longest clip-norm chains take their walk,
 * clip and pass 2 there).  A side stream not in use by a step is idle; at most 16 idle ones
 * are kept, the least recently used released (after its work completes) when another is needed.
 * came8_side_stream_count returns how many are kept now.  No reference counterpart (the reference
 * launches on the caller's stream only).
 */
int came8_side_stream_count(void);

/*
 * Blockwise absmax quantisation of n fp32 values into int8 (is_signed, Q = 127)
 * or uint8 (Q = 255) codes with one fp32 absmax per block of block_size
 * (came_pytorch/blockwise_quantization.py:66-82).
 */
int came8_quantize_blockwise(const float* x, int64_t n, int32_t is_signed, int32_t block_size,
                             void* q, float* absmax, void* stream);

/* Inverse: out[i] = q[i] * (absmax[i / block_size] / Q)  (blockwise_quantization.py:112-124). */
int came8_dequantize_blockwise(const void* q, const float* absmax, int64_t n, int32_t is_signed,
                               int32_t block_size, float* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* CAME8_H */
