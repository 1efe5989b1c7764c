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

#define CRESSO_HIP_ABI_VERSION 2

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
    double micro_decay, micro_impulse_decay, micro_drive_mix;
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
 * (cresso_v5.py:1505-1582), and the dense micro-field route of small tensors
 * (micro_field_max_size > 0; PyTorch-only in the reference,
 * cresso_v5.py:1355-1432).  One launch updates `count` tensors: each
 * descriptor names a param, its grad and its states, all updated in place:
 *   route 0 (scalar): the 8 scalar states of cresso_v5.py:885-891 + 857-862
 *     (q, impulse, metric_q, metric_impulse, force_rms, drive_energy,
 *     surprise, action);
 *   route 1 (micro): micro_energy, micro_impulse, micro_refractory (dense,
 *     the param's shape, cresso_v5.py:893-898), then force_rms, drive_energy,
 *     surprise, action (0-dim); state[7] is unused.
 * ------------------------------------------------------------------------- */
typedef struct cresso_scalar_desc {
    void* param;          /* contiguous, param_dtype                          */
    const void* grad;     /* contiguous, grad_dtype, same shape                */
    void* state[8];       /* state tensors, state dtype (f32, f64 for f64 params) */
    int64_t shape[8];
    int64_t numel;
    int32_t ndim;         /* 0..8                                              */
    int32_t param_dtype;
    int32_t grad_dtype;
    int32_t step;         /* optimizer step BEFORE this call (state["step"])  */
    int32_t route;        /* 0 scalar, 1 micro field                          */
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
 * cresso_v5.py:1434-1582 (route 0) or the micro-field step of
 * cresso_v5.py:1355-1432 (route 1) per tensor, param and states updated in place,
 * each tensor's step counter advanced on the device (state["step"] += 1).
 *   grads : NULL to reuse the previous call's grad pointers, else a host
 *           array of `count` device pointers in descriptor order (autograd
 *           gives fresh grad tensors each step).  Copied (host side) into one
 *           of two pinned, device-mapped staging buffers that the kernels read
 *           directly; a call waits only for the kernels of two calls ago.
 *   hyper : current hyperparameters (lr may change between steps) */
int32_t cresso_scalar_plan_step(cresso_scalar_plan* plan, void* dev_table, const void* const* grads,
                                const cresso_hyper* hyper, void* stream);

/* ---------------------------------------------------------------------------
 * Spectral / coordinate-hash route (large tensors).
 *
 * Replaces the reference's per-step op chain of cresso_v5.py:945-1353 as
 * fused by cresso_cuda_kernel.cu (basis_axis_cache_cuda 842,
 * basis_stats_with_cache_cuda 897, basis_project_with_cache_cuda 996,
 * basis_reconstruct_with_cache_cuda 1148, hash_metric_update_log_cuda 1515,
 * hash_impulse_update_gather_cuda 1593, instant_axis_metric_2d_cuda 1766,
 * metric_update_cuda 1829, confidence_update_cuda 1869,
 * contact_update_pair_cuda 1903, drive_update_cuda 2995; bindings
 * cresso_cuda.cpp:170-196) with one call per tensor and step.
 * ------------------------------------------------------------------------- */

/* Opaque plan for one (shape, freqs, hash_bins, hash_tables): geometry,
 * carrier bookkeeping and workspace layout.  freqs is the host copy of
 * state["freqs"] (int64 [rank][ndim], cresso_v5.py:864-868).  rank 1..32,
 * hash_tables 1..8 with tables x bin bytes
 * <= 8, hash_bins <= 65535.  NULL on error (cresso_hip_last_error says why). */
typedef struct cresso_spectral_plan cresso_spectral_plan;
cresso_spectral_plan* cresso_spectral_plan_create(const int64_t* shape, int32_t ndim, const int64_t* freqs,
                                                  int32_t rank, int32_t hash_bins, int32_t hash_tables);
/* The same with the work dtype of the tensors the plan steps: CRESSO_F32
 * (fp32, bf16 and fp16 params; what cresso_spectral_plan_create makes) or
 * CRESSO_F64 (fp64 params: every carrier, field, sum and state update in
 * fp64, the reference's work dtype for them, cresso_v5.py:119-124).  An F64
 * plan's workspace also holds per-axis fp64 carrier tables (rank x sum of the
 * dims x 32 bytes) and an fp64 field (8 bytes per element); it steps fp64
 * params with fp64 grads only, one tensor per call. */
cresso_spectral_plan* cresso_spectral_plan_create_ex(const int64_t* shape, int32_t ndim, const int64_t* freqs,
                                                     int32_t rank, int32_t hash_bins, int32_t hash_tables,
                                                     int32_t work_dtype);
void cresso_spectral_plan_destroy(cresso_spectral_plan* plan);

/* Device bytes of the plan's workspace: per-axis carrier tables, basis stats,
 * cached coordinate-hash bins of every element (data independent), bin
 * counts, the stored tangent field and per-step scratch.  Not optimizer
 * state: it is rebuilt from the shape and freqs. */
size_t cresso_spectral_workspace_bytes(const cresso_spectral_plan* plan);

/* Build the workspace tables on the device (synchronizes `stream` once). */
int32_t cresso_spectral_workspace_init(const cresso_spectral_plan* plan, void* workspace, size_t workspace_bytes,
                                       const cresso_hyper* hyper, void* stream);

typedef struct cresso_spectral_desc {
    void* param;              /* contiguous, param_dtype                    */
    const void* grad;         /* contiguous, grad_dtype                     */
    int32_t param_dtype;
    int32_t grad_dtype;
    int64_t numel;
    /* state of cresso_v5.py:857-883, updated in place: fp32, or fp64 when
     * param_dtype is F64 (the reference's state follows the work dtype,
     * v5.py:119-124; an F64 step computes in fp64 on an F64 plan) */
    void *force_rms, *drive_energy, *surprise, *action;       /* 0-dim       */
    const void* omega;                                         /* [rank]      */
    void *q_cos, *q_sin, *p_cos, *p_sin;                       /* [rank]      */
    void *metric_cos, *metric_sin, *metric_p_cos, *metric_p_sin;
    void *calcium_cos, *calcium_sin, *mode_confidence;
    void *hash_energy, *hash_impulse, *hash_refractory;       /* [T][B] or all NULL */
    int32_t step;             /* state["step"] AFTER the increment          */
    int32_t hard;             /* hard channel on (cresso_v5.py:981-983)     */
} cresso_spectral_desc;

/* One optimizer step of one tensor on the spectral route.  (param, grad)
 * dtype pairs: (F32,F32), (BF16,BF16), (F16,F16), (F32,BF16), (F32,F16) on
 * an F32 plan; (F64,F64) on an F64 plan (cresso_spectral_plan_create_ex). */
int32_t cresso_spectral_step(const cresso_spectral_plan* plan, const cresso_spectral_desc* desc, void* workspace,
                             size_t workspace_bytes, const cresso_hyper* hyper, void* stream);

/* One optimizer step of `count` tensors of one plan, each launch of the step
 * covering all of them (the tensor is the grid's second dimension).  Replaces
 * the reference's loop over a group's same-shape spectral params
 * (cresso_v5.py:828-843 with _spectral_step, v5.py:885), whose per-step basis
 * cache (transient_basis_workspace, v5.py:827) is shared the same way: the
 * plan's shape tables are held once, the per-step scratch once per tensor.
 *
 * descs: host array of `count` descriptors of distinct tensors; they may
 * differ in every pointer and in `step`, not in dtypes, `hard` or whether
 * hash state is given.  The library copies them to the device as kernel
 * arguments on `stream` (no host synchronization).  Every tensor's results
 * are bit-identical to cresso_spectral_step of it.  F64 params are not batched (CRESSO_E_UNSUPPORTED):
 * step them with cresso_spectral_step.
 *
 * The workspace: cresso_spectral_batched_workspace_bytes(plan, count) bytes,
 * set up once by cresso_spectral_batched_workspace_init (which synchronizes
 * `stream` once).  It serves any batch of up to `count` tensors; calls that
 * share it must be ordered (one stream). */
size_t cresso_spectral_batched_workspace_bytes(const cresso_spectral_plan* plan, int32_t count);
int32_t cresso_spectral_batched_workspace_init(const cresso_spectral_plan* plan, int32_t count, void* workspace,
                                               size_t workspace_bytes, const cresso_hyper* hyper, void* stream);
int32_t cresso_spectral_step_batched(const cresso_spectral_plan* plan, const cresso_spectral_desc* descs, int32_t count,
                                     void* workspace, size_t workspace_bytes, const cresso_hyper* hyper, void* stream);

/* cresso_spectral_step without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.
 *
 * The workspace lives in a static device array of
 * CRESSO_SPECTRAL_NOALLOC_MAX_BYTES bytes that every GPU the library runs on
 * holds until the process ends; the call allocates and frees nothing.  A plan
 * whose cresso_spectral_workspace_bytes() exceeds that size is rejected with
 * CRESSO_E_INVALID (at T = 2 tables of <= 256 bins the limit admits about
 * 5 M elements, e.g. a 2048 x 2048 tensor).  The array keeps the last call's
 * contents: when the plan differs from the one of the device's previous
 * no-alloc call, the call first rebuilds the plan's tables in it (as
 * cresso_spectral_workspace_init does, including its one synchronization of
 * `stream`).  All calls on one GPU share the array: calls that overlap (two
 * streams or two host threads) race.  Results are identical to
 * cresso_spectral_step's.
 *
 * Graph capture: a call whose plan's tables are already resident launches
 * kernels only and may be captured.  A call that would rebuild the tables
 * returns CRESSO_E_INVALID when `stream` is capturing (the rebuild copies from
 * host memory and synchronizes).  A captured graph reads the tables of the
 * plan it was captured with: it is valid only while no no-alloc call with
 * another plan has run on that GPU since; after one, make an uncaptured call
 * with the graph's plan before replaying it. */
#define CRESSO_SPECTRAL_NOALLOC_MAX_BYTES (32u << 20)
int32_t cresso_spectral_step_noalloc(const cresso_spectral_plan* plan, const cresso_spectral_desc* desc,
                                     const cresso_hyper* hyper, void* stream);

/* Inspection of an initialised workspace, for parity checks (a step does not
 * need these).
 *
 * cresso_spectral_workspace_bins: the coordinate-hash bin of every element
 * for every table, exactly as the step consumes them, into bins_out (device
 * int32 [hash_tables][numel]); the bin occupancy counts into counts_out
 * (device int64 [hash_tables][hash_bins]).  Counterpart of the index/count
 * half of hash_reduce_mean_cuda (cresso_cuda_kernel.cu:1222; bin function
 * cresso_hash_index, cu:189-201) and of the reference's _hash_index_tensor
 * (cresso_v5.py:495-516).  Fails on a plan with hash_bins = 0.
 *
 * cresso_spectral_workspace_basis: the normalized basis pair (C_r, S_r) of
 * mode `mode` at every element, formed from the separable row/column tables
 * and the closed-form stats as the step's reconstructions combine them
 * (device fp32 [numel] each).  Counterpart of basis_axis_cache_cuda +
 * basis_stats_with_cache_cuda (cu:842, 897) and of the reference's
 * _basis_pair (cresso_v5.py:295-348). */
int32_t cresso_spectral_workspace_bins(const cresso_spectral_plan* plan, const void* workspace, size_t workspace_bytes,
                                       int32_t* bins_out, int64_t* counts_out, void* stream);
int32_t cresso_spectral_workspace_basis(const cresso_spectral_plan* plan, const void* workspace, size_t workspace_bytes,
                                        int32_t mode, float* cos_out, float* sin_out, void* stream);

/* Gram matrix of the normalized basis that the step's closed-form drive
 * statistics use: G[v][w] = mean over elements of Xn_v Xn_w with v = 2r for
 * C_r and v = 2r+1 for S_r, into gram_out (device fp64 [2*rank][2*rank]).
 * The reference evaluates the same quantities element by element
 * (cresso_v5.py:1303-1353; drive_update_cuda, cresso_cuda_kernel.cu:2995). */
int32_t cresso_spectral_workspace_gram(const cresso_spectral_plan* plan, const void* workspace, size_t workspace_bytes,
                                       double* gram_out, void* stream);

/* Projection of a field on the normalized basis, out[2r] = mean(x C_r),
 * out[2r+1] = mean(x S_r) (device fp32 x [numel] -> device fp64 out [2*rank];
 * fp32 products, fp64 sums): the reference's _project / basis_project
 * (cresso_v5.py:351-359; basis_project_with_cache_cuda, cu:996-1084).
 * Uses the workspace's per-step scratch, so it is stream-ordered with steps. */
int32_t cresso_spectral_workspace_project(const cresso_spectral_plan* plan, void* workspace, size_t workspace_bytes,
                                          const float* x, double* out, void* stream);

/* Reconstruction out = shrink * sum_r g_r (cc[r] C_r + sc[r] S_r), shrink =
 * 1/sqrt(max(1, 0.7 log2(rank+1))), a gate of exactly 0 skipping mode r
 * (gates may be NULL: all 1), accumulated in fp32 in mode order (device fp32
 * cc, sc, gates [rank] -> device fp32 out [numel]): the reference's
 * _reconstruct (cresso_v5.py:362-376; basis_reconstruct_with_cache_cuda,
 * cu:1148-1210). */
int32_t cresso_spectral_workspace_reconstruct(const cresso_spectral_plan* plan, const void* workspace,
                                              size_t workspace_bytes, const float* cc, const float* sc,
                                              const float* gates, float* out, void* stream);

/* ---------------------------------------------------------------------------
 * Unit operations of the spectral route.
 *
 * One entry point per op of the reference's fused CUDA path
 * (cresso_cuda.cpp:44-125), with the same arguments and in-place state
 * semantics, on explicit device fields (fp32).  cresso_spectral_step fuses
 * all of them; these serve callers that compose a step themselves and the
 * per-op parity checks.  The hash ops and cresso_drive_update take a
 * caller-allocated scratch workspace (256-byte aligned) of at least
 * cresso_unit_workspace_bytes(bins) bytes (bins = 1 for the drive); calls
 * sharing a workspace must not overlap.  Hash bins and counts follow
 * _hash_index_tensor (cresso_v5.py:495-516) bit for bit.
 * ------------------------------------------------------------------------- */
size_t cresso_unit_workspace_bytes(int32_t bins);

/* Bin means of x [numel] for one hash table (table salt `salt`): the sum of
 * the elements of each bin divided by max(count, 1), into mean_out [bins]
 * (cresso_v5.py:519-526).  Replaces hash_reduce_mean_cuda
 * (cresso_cuda_kernel.cu:1222-1253; binding cresso_cuda.cpp:42).
 * bins <= 4096, as the reference's op. */
int32_t cresso_hash_reduce_mean(const float* x, int64_t numel, int32_t bins, int32_t salt, float* mean_out,
                                void* workspace, size_t workspace_bytes, void* stream);

/* out[i] = values[bin(i)] for i < numel, bin of table salt `salt` over
 * `bins` = the length of values (cresso_v5.py:1024, 1158).  Replaces
 * hash_gather_cuda (cresso_cuda_kernel.cu:1255-1276; binding
 * cresso_cuda.cpp:43).  Needs no workspace. */
int32_t cresso_hash_gather(const float* values, int32_t bins, int64_t numel, int32_t salt, float* out, void* stream);

/* Instant axis metric of a 2-D field rel [rows][cols] (cresso_v5.py:243-262):
 * density d = min(max(rel, eps)^p, 1e6) with p = max(power, 0.25); row and
 * column means of d, each divided by max(mean of its marginal, eps); out =
 * clamp(exp(coupling / (2 p) * (log max(row term, eps) + log max(col term,
 * eps))), 0.08, 12); all ones when coupling = 0 or rows * cols = 1.  Replaces
 * instant_axis_metric_2d_cuda (cresso_cuda_kernel.cu:1766-1827; binding
 * cresso_cuda.cpp:63).  Sums are fp64 in a fixed order.  The workspace
 * (256-byte aligned) holds cresso_instant_axis_metric_2d_workspace_bytes(rows,
 * cols) bytes. */
size_t cresso_instant_axis_metric_2d_workspace_bytes(int64_t rows, int64_t cols);
int32_t cresso_instant_axis_metric_2d(const float* rel, int64_t rows, int64_t cols, double power, double coupling,
                                      double eps, float* out, void* workspace, size_t workspace_bytes, void* stream);

/* One hash table's metric (cresso_v5.py:1014-1026): bin means of
 * density_source [numel] (row-major linear index, table salt `salt`), EMA into
 * hash_energy [bins] in place (copied when step <= 1), normalized by its
 * mean, raised to hash_metric_coupling / max(0.25, energy_power), gathered per
 * element, clamped to [0.08, 12] and logged into term_out [numel].
 * Replaces hash_metric_update_log_cuda (cresso_cuda_kernel.cu:1515-1591;
 * binding cresso_cuda.cpp:44-53).  bins <= 4096. */
int32_t cresso_hash_metric_update_log(const float* density_source, int64_t numel, float* hash_energy, int32_t bins,
                                      int32_t salt, int32_t step, double hash_decay, double hash_metric_coupling,
                                      double energy_power, double eps, float* term_out, void* workspace,
                                      size_t workspace_bytes, void* stream);

/* One hash table's impulse (cresso_v5.py:1153-1160): bin means cp of
 * port_source, hash_refractory <- decay * r + (1 - decay) |cp|, gate
 * 1/(1 + refractory_gain * r), hash_impulse <- impulse_decay * i +
 * (1 - impulse_decay) cp * gate (both [bins], in place), gathered per element
 * into retrieved_out [numel].  Replaces hash_impulse_update_gather_cuda
 * (cresso_cuda_kernel.cu:1593-1661; binding cresso_cuda.cpp:54-62). */
int32_t cresso_hash_impulse_update_gather(const float* port_source, int64_t numel, float* hash_refractory,
                                          float* hash_impulse, int32_t bins, int32_t salt, double hash_decay,
                                          double hash_impulse_decay, double refractory_gain, float* retrieved_out,
                                          void* workspace, size_t workspace_bytes, void* stream);

/* Metric oscillator of both banks, in place (cresso_v5.py:1064-1088).
 * Replaces metric_update_cuda (cresso_cuda_kernel.cu:1829-1867; binding
 * cresso_cuda.cpp:64-73).  rank <= 4096. */
int32_t cresso_metric_update(float* metric_cos, float* metric_sin, float* metric_p_cos, float* metric_p_sin,
                             const float* mcos_port, const float* msin_port, const float* omega, int32_t rank,
                             double metric_dt, double metric_friction, void* stream);

/* Mode confidence, in place, from the port projections and the pre-contact q
 * (cresso_v5.py:1199-1202 and its PyTorch branch).  Replaces
 * confidence_update_cuda (cresso_cuda_kernel.cu:1869-1901; binding
 * cresso_cuda.cpp:74-81).  rank <= 4096. */
int32_t cresso_confidence_update(float* confidence, const float* pcos_port, const float* psin_port, const float* qcos,
                                 const float* qsin, int32_t rank, double confidence_decay, double eps, void* stream);

/* Contact oscillator of one bank (q, p) with its calcium trace, the shared
 * action (0-dim) and the surprise (0-dim, read), in place
 * (cresso_v5.py:914-943; the step calls it for the cos bank, then the sin
 * bank).  Replaces contact_update_pair_cuda (cresso_cuda_kernel.cu:1903-1965;
 * binding cresso_cuda.cpp:82-98).  rank <= 4096. */
int32_t cresso_contact_update_pair(float* q, float* p, const float* port, const float* omega, float* calcium,
                                   float* action, const float* surprise, int32_t rank, double dt,
                                   double refractory_decay, double refractory_gain, double surprise_gain,
                                   double surprise_brake, double impulse_friction, double contact_gain,
                                   double restoring, double cubic, void* stream);

/* Drive shaping, drive-energy reservoir (0-dim drive_energy, in place) and
 * the update param -= lr * cast(drive * gain) (cresso_v5.py:1303-1353) from
 * the tangent, prediction and error fields [numel]; echo and hash_pred may be
 * NULL (no echo / hash term); surprise is read.  param_dtype: CRESSO_F32,
 * CRESSO_BF16 or CRESSO_F16.  Replaces drive_update_cuda
 * (cresso_cuda_kernel.cu:2995-3223; binding cresso_cuda.cpp:99-125). */
int32_t cresso_drive_update(void* param, int32_t param_dtype, const float* tangent, const float* pred,
                            const float* error, const float* echo, const float* hash_pred, const float* surprise,
                            float* drive_energy, int64_t numel, int32_t step, int32_t hard, const cresso_hyper* hyper,
                            void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* CRESSO_HIP_H */
