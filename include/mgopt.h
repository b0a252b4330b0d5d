/*
 * mgopt.h -- C ABI of the MI355X optimizer-step engine (libmgopt.so).
 *
 * The engine replaces, on one GPU, the four torch calls that the reference's
 * training loop makes once per iteration (train.py:483-491):
 *
 *     scaler.unscale_(optimizer)                      -> deferred into the two passes
 *     clip_grad_norm_(model.parameters(), max_norm)   -> mgopt_grad_norm
 *     scaler.step(optimizer)                          -> mgopt_adamw_step
 *     scaler.update()                                 -> mgopt_scaler_update
 *
 * Conventions
 *   - Every pointer argument named *_dev is a device pointer; buffers are
 *     owned by the caller (PyTorch's allocator in the Python host layer),
 *     except the plan's internal tables, which the plan owns.
 *   - Every call is asynchronous on `stream` (a hipStream_t) and makes no
 *     host<->device synchronisation, except mgopt_plan_create (one blocking
 *     upload of the tables).
 *   - Every function returns 0 on success or a nonzero code (a hipError_t,
 *     or MGOPT_E_* below); mgopt_last_error() then describes the failure of
 *     the most recent failing call on the calling thread.  No C++ exception
 *     crosses this boundary.
 *   - A plan is not safe for concurrent use from two streams.
 */
#ifndef MGOPT_H
#define MGOPT_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MGOPT_API __attribute__((visibility("default")))

/* element types */
#define MGOPT_F32 0
#define MGOPT_F16 1
#define MGOPT_BF16 2
#define MGOPT_NONE (-1)

/* error codes beyond hipError_t values */
#define MGOPT_E_INVALID 10001   /* bad argument */
#define MGOPT_E_ALIGN 10002     /* misaligned buffer */
#define MGOPT_E_LIMIT 10003     /* size above a compiled maximum */

#define MGOPT_MAX_GROUPS 16

/* flags for mgopt_adamw_step */
#define MGOPT_WRITEBACK_GRADS 1  /* store the unscaled, clipped gradient back into each grad */
#define MGOPT_GROUPS_ON_DEVICE 2 /* `groups` is a device pointer, read by the kernel when it runs (so a
                                    launch captured in a HIP graph picks up the values current at replay) */

/* One parameter tensor of the optimizer (one entry of torch.optim.Optimizer's
 * param_groups[*]["params"], torch/optim/optimizer.py:164-189).
 *   param_dev      fp32 values AdamW updates in place: the model parameter
 *                  itself when it is fp32, else the fp32 master copy.
 *   lowp_dev       the model parameter when it is bf16/fp16 (rewritten from the
 *                  master after every update, round to nearest even), or NULL.
 *   exp_avg_dev,
 *   exp_avg_sq_dev fp32 first and second moments (torch/optim/adam.py:177-184).
 *   numel          element count (> 0).
 *   group          index into the group hyper-parameter array.
 *   grad_dtype     MGOPT_F32, MGOPT_F16 or MGOPT_BF16.
 *   lowp_dtype     MGOPT_BF16, MGOPT_F16, or MGOPT_NONE when lowp_dev is NULL.
 *   row_elems      0: param_dev, exp_avg_dev and exp_avg_sq_dev each hold the
 *                  numel values contiguously.  > 0: they hold them in rows of
 *                  row_elems values (row_elems divides numel and is a multiple
 *                  of the plan's chunk_elems), row r of exp_avg / exp_avg_sq at
 *                  exp_avg_dev / exp_avg_sq_dev + r * state_pitch and row r of
 *                  param_dev at param_dev + r * param_pitch (param_pitch =
 *                  row_elems for a contiguous parameter).  This lets a caller
 *                  place one tensor's master, exp_avg and exp_avg_sq rows side
 *                  by side in memory, which keeps the update's reads and
 *                  write-backs of a row in neighbouring DRAM rows; lowp_dev
 *                  and the gradient are always contiguous.
 *   param_pitch,
 *   state_pitch    row strides in elements (>= row_elems) when row_elems > 0. */
typedef struct mgopt_tensor_desc {
    float* param_dev;
    void* lowp_dev;
    float* exp_avg_dev;
    float* exp_avg_sq_dev;
    int64_t numel;
    int32_t group;
    int32_t grad_dtype;
    int32_t lowp_dtype;
    int32_t reserved;
    int64_t row_elems;
    int64_t param_pitch;
    int64_t state_pitch;
} mgopt_tensor_desc;

/* Per-group AdamW hyper-parameters for one step, as host doubles (the values
 * torch/optim/adam.py:214-272 reads from each param group). */
typedef struct mgopt_group_hparams {
    double lr;
    double weight_decay;
    double beta1;
    double beta2;
    double eps;
    int32_t maximize;
    int32_t reserved;
} mgopt_group_hparams;

typedef struct mgopt_plan mgopt_plan;

/* Builds the device chunk tables for a parameter set (the multi-tensor
 * dispatch torch builds per call in torch/optim/adam.py:139-212 _init_group
 * and in _foreach_norm's tensor lists, clip_grad.py:85-96): pass 2 (the AdamW
 * update) works in chunks of chunk_elems elements, which must be a positive
 * multiple of 512; pass 1 (the norm) in chunks of 131,072.  steps_dev is a
 * caller-owned float[n_tensors] holding each tensor's AdamW step count
 * (torch/optim/adam.py:168-176 state["step"]). */
MGOPT_API int mgopt_plan_create(const mgopt_tensor_desc* descs, int32_t n_tensors, int32_t n_groups,
                                float* steps_dev, int64_t chunk_elems, mgopt_plan** out);

MGOPT_API int mgopt_plan_destroy(mgopt_plan* plan);

/* Number of pass-2 chunks of the plan (one work-group each). */
MGOPT_API int64_t mgopt_plan_num_chunks(const mgopt_plan* plan);

/* 1 when the plan runs a step as three kernels (a plan of at most 2,097,152
 * elements, no empty tensor, no tensor of more than 256 pass-2 chunks,
 * MGOPT_FOLD not "0" in the environment at creation; MGOPT_FOLD=1 lifts the
 * two size limits for plans of up to 67,108,864 elements): pass 1 finalizes
 * in its last work-group and pass 2 forms the step counts and constants
 * itself; 0 for the five-kernel form (pass 1, finalize, prologue, pass 2,
 * scaler); -1 for NULL.  Both forms give the same results.  No reference
 * counterpart. */
MGOPT_API int mgopt_plan_folded(const mgopt_plan* plan);

/* Sets the gradient of every tensor for the coming step from a host array of
 * n_tensors device pointers (NULL = this tensor has no grad this step, as
 * p.grad is None is skipped at torch/optim/adam.py:153 and clip_grad.py:228).
 * Uploads only when the pointers changed since the last call. */
MGOPT_API int mgopt_plan_set_grads(mgopt_plan* plan, const void* const* grads_host, void* stream);

/* Pass 1 + finalize: the gradient L2 norm.  Replaces
 *   torch._amp_foreach_non_finite_check_and_unscale_ (torch/amp/grad_scaler.py:280-284),
 *   torch._foreach_norm + vector_norm(stack)       (torch/nn/utils/clip_grad.py:96-108),
 *   the clip coefficient                           (clip_grad.py:165-169).
 * Reads every grad once (one pass-1 launch per gradient dtype, then one
 * finalize launch; a small plan runs the finalize in pass 1's last
 * work-group, see mgopt_plan_folded).  scale_dev: the GradScaler scale (fp32 scalar); when
 * non-NULL each grad element g becomes float(g) * float(1/double(scale))
 * before squaring, and found_inf_dev receives 1.0 if any *input* element is
 * non-finite, else 0.0.  coef_dev (when non-NULL) receives the clip
 * coefficient min(1, max_norm / (norm + 1e-6)) in torch's fp32 arithmetic
 * (NaN propagates).  norm_dev receives the fp32 total norm.  Any output
 * pointer may be NULL. */
MGOPT_API int mgopt_grad_norm(mgopt_plan* plan, const float* scale_dev, double max_norm,
                              float* norm_dev, float* coef_dev, float* found_inf_dev, void* stream);

/* Pass 2: the AdamW update of every tensor that has a grad.  Replaces
 *   GradScaler.step's skip decision  (torch/amp/grad_scaler.py:348-358, 403-454),
 *   clip_grad.py:174 (_foreach_mul_ by the clip coefficient),
 *   torch/optim/adam.py:347-552 (_single_tensor_adam) / 803-899 (_fused_adam).
 * groups: n_groups hyper-parameter sets, passed by value to the kernel, or,
 * with MGOPT_GROUPS_ON_DEVICE in flags, a device array of them that the kernel
 * reads when it runs.  bc_dev: double table bc[(group * bc_cap + t) * 2 + {0,1}]
 * = {1 - beta1**t, (1 - beta2**t) ** 0.5} for 1 <= t < bc_cap, computed on the
 * host with the same expressions as adam.py:529-536, and {beta1, beta2} at
 * t = 0 (the betas the row was computed for).  A step count that is not an
 * integer in [1, bc_cap) -- one written into the state, or reached by graph
 * replays -- or a group whose betas differ from its row's, takes the same
 * expressions evaluated on the device in double (the device
 * pow can differ from the host's by an ulp of the double), and raises the
 * plan's flag (mgopt_plan_flags).  A prologue launch (one thread per tensor)
 * advances the step counts and forms each tensor's fp32 constants; pass 2
 * then reads them once per work-group.  A small plan forms them inside
 * pass 2 instead (mgopt_plan_folded), with the same results.
 * scale_dev (nullable): unscale as in mgopt_grad_norm.  coef_dev (nullable):
 * clip coefficient.  found_inf_dev (nullable): nonzero skips the whole step,
 * leaving params, moments and step counts untouched. */
MGOPT_API int mgopt_adamw_step(mgopt_plan* plan, const mgopt_group_hparams* groups, const double* bc_dev,
                               int64_t bc_cap, const float* scale_dev, const float* coef_dev,
                               const float* found_inf_dev, int32_t flags, void* stream);

/* torch._amp_update_scale_ (torch/amp/grad_scaler.py:469-539, call at 529-536),
 * summing n_found found_inf scalars first as grad_scaler.py:517-527 does. */
MGOPT_API int mgopt_scaler_update(float* scale_dev, int32_t* growth_tracker_dev,
                                  const float* const* found_inf_devs, int32_t n_found, double growth_factor,
                                  double backoff_factor, int32_t growth_interval, void* stream);

/* In-place g *= coef over the plan's grads (clip_grad.py:120-182,
 * _clip_grads_with_norm_), for callers that clip a parameter list that is
 * not an optimizer's.  coef_dev is a device fp32 scalar. */
MGOPT_API int mgopt_scale_grads(mgopt_plan* plan, const float* coef_dev, void* stream);

/* Copies every lowp parameter into its fp32 master (exact widening). */
MGOPT_API int mgopt_sync_master(mgopt_plan* plan, void* stream);

/* Registers a caller-owned 16-byte device buffer (NULL: none) that later
 * calls keep log-window statistics in: float last norm, float running maximum
 * of norms (NaN propagates, as torch.maximum does), uint32 skipped steps,
 * uint32 taken steps.  mgopt_grad_norm updates the norms when it writes a norm;
 * mgopt_adamw_step counts the step.  Replaces the per-step
 * torch.maximum(window_grad_norm_max, grad_norm) and the optimizer-step /
 * skip bookkeeping of train.py:487-489,501-507. */
MGOPT_API int mgopt_plan_set_window(mgopt_plan* plan, void* window_dev);

/* Blocking read of the plan's device flag: nonzero once a pass-2 work-group
 * has computed its bias corrections on the device because its step count was
 * outside the bias-correction table (see mgopt_adamw_step).  No reference
 * counterpart. */
MGOPT_API int mgopt_plan_flags(mgopt_plan* plan, int* out);

/* The gradient L2 norm of one contiguous gradient buffer of n elements (a
 * flat gradient arena), with the outputs, scaling and arithmetic of
 * mgopt_grad_norm.  It sums the same 131,072-element chunks in the same order
 * as mgopt_grad_norm on a plan holding that buffer as its one tensor in the
 * five-kernel form (a plan of more than 2,097,152 elements, or any plan made
 * with MGOPT_FOLD=0 in the environment), and is bit-identical to it there; a
 * plan of at most 2,097,152 elements runs the three-kernel form, whose
 * 16,384-element chunks group the fp64 partial sums differently, so the two
 * can differ in the last bits of the fp64 total.  Allocates nothing: its
 * partial sums live in a static 1 MiB device array that each GPU holds until
 * the process ends, so n is at most 8,589,934,592 (65,536 chunks of 131,072
 * elements; larger n returns MGOPT_E_LIMIT).  Runs on the current device.  Calls that overlap on
 * one GPU share that array and race.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops, harnesses that forbid hipMalloc). */
MGOPT_API int mgopt_grad_norm_noalloc(const void* grads_dev, int32_t grad_dtype, int64_t n, const float* scale_dev,
                                      double max_norm, float* norm_dev, float* coef_dev, float* found_inf_dev,
                                      void* stream);

/* Deterministic test data: dst[i] = synth(key(seed, stream_id), i) in dtype
 * (MGOPT_F32/F16/BF16).  No reference counterpart; used by tests and the
 * benchmark to create identical inputs on the GPU and in the CPU oracle. */
MGOPT_API int mgopt_synth_fill(void* dst_dev, int32_t dtype, int64_t n, uint64_t seed, uint64_t stream_id,
                               double k, uint64_t tail_every, double tail_mult, void* stream);

/* Message for the most recent failure on the calling thread ("" if none). */
MGOPT_API const char* mgopt_last_error(void);

/* Library version string. */
MGOPT_API const char* mgopt_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MGOPT_H */
