/*
 * cresso_hip.h -- C ABI of the MI355X (gfx950) CRESSO5 hot-path library.
 *
 * libcresso_hip.so replaces the reference's JIT-built CUDA extension
 * (/root/reference/cresso_cuda/cresso_cuda.cpp:170-196, kernels in
 * cresso_cuda/cresso_cuda_kernel.cu) behind CRESSO5(params, cuda_ops=...).
 * Every entry point is stream-ordered on the given HIP stream, takes raw
 * device pointers owned by the caller (PyTorch), performs host-side
 * validation before any launch, never synchronizes the device and returns 0
 * on success or a negative CRESSO_E* code; the message of the last failure on
 * the calling thread is returned by cresso_hip_last_error().
 *
 * Plain C types only: no torch or HIP types appear in the signatures
 * (a stream is passed as void*; NULL is the null stream).
 */
#ifndef CRESSO_HIP_H
#define CRESSO_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CRESSO_HIP_ABI_VERSION 1

/* error codes */
#define CRESSO_OK 0
#define CRESSO_E_INVALID (-1)   /* bad argument (shape, dtype, alignment, size)  */
#define CRESSO_E_HIP (-2)       /* a HIP runtime call failed                      */
#define CRESSO_E_UNSUPPORTED (-3) /* valid input outside what this build handles  */

/* element dtypes */
#define CRESSO_F32 0
#define CRESSO_F64 1
#define CRESSO_F16 2
#define CRESSO_BF16 3

/* Hyperparameters of one CRESSO5 param group: the float keyword arguments of
 * CRESSO5.__init__ (cresso_v5.py:621-681, stored in the group at 760-818). */
typedef struct cresso_hyper {
    double lr, weight_decay, energy_power, dt, impulse_friction, contact_gain;
    double restoring, cubic, metric_dt, metric_friction, metric_coupling;
    double local_sharpness, instant_metric_coupling, instant_metric_power;
    double root_channel_mix, echo_mix, transport_mix, hash_decay;
    double hash_impulse_decay, hash_metric_coupling, hash_drive_mix;
    double direct_force_mix, residual_feedback_mix, reservoir_decay;
    double refractory_decay, refractory_gain, confidence_decay, confidence_gain;
    double surprise_gain, surprise_decay, prediction_mix, novelty_mix;
    double surprise_brake, target_update_rms, min_gain, max_gain, drive_clip;
    double spike_mix, eps;
    int32_t warmup_steps;
    int32_t maximize;     /* non-zero: the force is -grad (cresso_v5.py:835-836) */
} cresso_hyper;

/* ---------------------------------------------------------------------------
 * Library identity and errors
 * ------------------------------------------------------------------------- */
int32_t cresso_hip_abi_version(void);
/* Message of the last failing call on this thread ("" if none). */
const char* cresso_hip_last_error(void);

/* ---------------------------------------------------------------------------
 * Scalar (LoRA-thin / small-tensor) route.
 *
 * Replaces scalar_update_2d_cuda (cresso_cuda_kernel.cu:3225-3605; binding
 * cresso_cuda.cpp:190, called at cresso_v5.py:1457-1500) and also covers the
 * ndim != 2 tensors that the reference sends to its PyTorch scalar path
 * (cresso_v5.py:1505-1582).  One launch updates `count` tensors: each
 * descriptor names a param, its grad and the 8 scalar states of
 * cresso_v5.py:885-891 + 857-862 (q, impulse, metric_q, metric_impulse,
 * force_rms, drive_energy, surprise, action), all updated in place.
 * ------------------------------------------------------------------------- */
typedef struct cresso_scalar_desc {
    void* param;          /* contiguous, param_dtype                          */
    const void* grad;     /* contiguous, grad_dtype, same shape                */
    void* state[8];       /* 0-dim state tensors, state dtype (f32, f64 for f64 params) */
    int64_t shape[8];
    int64_t numel;
    int32_t ndim;         /* 0..8                                              */
    int32_t param_dtype;
    int32_t grad_dtype;
    int32_t step;         /* optimizer step BEFORE this call (state["step"])  */
} cresso_scalar_desc;

/* Opaque, host-side plan of one scalar-route batch: the descriptors
 * validated, each tensor assigned a kernel (register-resident for 2D tensors
 * of <= 64 Ki elements with float4-aligned rows, streaming otherwise) and
 * grouped so that one launch runs per kernel variant.  NULL on error. */
typedef struct cresso_scalar_plan cresso_scalar_plan;
cresso_scalar_plan* cresso_scalar_plan_create(const cresso_scalar_desc* host_descs, int32_t count,
                                              const cresso_hyper* hyper);
void cresso_scalar_plan_destroy(cresso_scalar_plan* plan);

/* Device bytes the plan's table needs (descriptors, step counters, grad
 * pointers, axis-sum scratch). */
size_t cresso_scalar_plan_bytes(const cresso_scalar_plan* plan);

/* Copy the plan (descriptors and each tensor's current step) into dev_table.
 * Synchronizes `stream` once; call when the plan is (re)built. */
int32_t cresso_scalar_plan_upload(cresso_scalar_plan* plan, void* dev_table, size_t table_bytes, void* stream);

/* One optimizer step of every tensor of the plan: the fused scalar step of
 * cresso_v5.py:1434-1582 per tensor, param and the 8 states updated in place,
 * each tensor's step counter advanced on the device (state["step"] += 1).
 *   grads : NULL to reuse the grad pointers already in the table, else a host
 *           array of `count` device pointers in descriptor order (autograd
 *           gives fresh grad tensors each step); uploaded from pinned staging
 *   hyper : current hyperparameters (lr may change between steps) */
int32_t cresso_scalar_plan_step(cresso_scalar_plan* plan, void* dev_table, const void* const* grads,
                                const cresso_hyper* hyper, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* CRESSO_HIP_H */
