/*
 * tmnn_hip.h -- C-ABI of the MI355X (gfx950) neural-field hot path.
 *
 * This library replaces the reference's Metal layers (L5 kernel generation,
 * L6 device runtime) under tiny-metal-nn's ITrainerRuntime / FieldEvaluator /
 * RuntimeAuthority boundary. Plain C types only: every array argument is a
 * caller-owned pointer with an explicit element count. Host-pointer entry
 * points copy inputs in and results out before they return (the reference's
 * synchronous step contract); the *_device entry points take device pointers
 * and only enqueue on the trainer's stream.
 *
 * Reference citations are relative to the reference checkout. Every entry
 * point returns TMNN_OK (0) or a negative status; tmnn_last_error() returns
 * the thread-local message of the last failure on the calling thread.
 */
#ifndef TMNN_HIP_H
#define TMNN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes --------------------------------------------------- */
#define TMNN_OK 0
#define TMNN_ERR_INVALID_ARGUMENT (-1) /* std::invalid_argument in the reference */
#define TMNN_ERR_RUNTIME (-2)          /* std::runtime_error in the reference */
#define TMNN_ERR_GPU (-3)              /* a HIP call failed */
#define TMNN_ERR_UNSUPPORTED (-4)      /* geometry outside this build's kernels */

/* ---- enums ------------------------------------------------------------ */
/* Loss kinds: extension::LossKind (include/tiny-metal-nn/extension/
 * kernel_compile_spec.h) plus RelativeL2, which the reference lacks
 * (factory_json_detail.h:368-377). */
#define TMNN_LOSS_L2 0
#define TMNN_LOSS_L1 1
#define TMNN_LOSS_HUBER 2
#define TMNN_LOSS_COSINE 3
#define TMNN_LOSS_RELATIVE_L2 4

/* MLP arithmetic. FP32: fp32 MFMA (v_mfma_f32_16x16x4_f32), the reference's
 * fp32 math. FP16: fp16 MFMA operands, fp32 accumulation and fp32 master
 * parameters. Inference always runs FP32 (default_trainer.cpp:356-379). */
#define TMNN_PRECISION_FP32 0
#define TMNN_PRECISION_FP16 1

/* Hash-table Adam: LAZY updates only entries visited by the step's batch
 * (the reference default, adam_kernel_msl.h:120-164); DENSE updates every
 * entry (the reference's unified kernel, adam_kernel_msl.h:37-109). */
#define TMNN_HASH_ADAM_LAZY 0
#define TMNN_HASH_ADAM_DENSE 1

/* Network families: NetworkFamily (detail/network_planning.h:29-33), same
 * numbering. On this GPU: FULLY_FUSED = the shape-specialised MFMA kernels
 * (weight gradients in registers / owned tiles, inline or separate encode);
 * TILED = the generic kernels (runtime layer count and geometry, weight
 * gradients accumulated in LDS); SAFE_DEBUG = the generic kernels in fp32
 * without the Morton sort. AUTO lets the planner choose. */
#define TMNN_FAMILY_AUTO (-1)
#define TMNN_FAMILY_FULLY_FUSED 0
#define TMNN_FAMILY_TILED 1
#define TMNN_FAMILY_SAFE_DEBUG 2

/* Planner fallback reasons: PlannerFallbackReason (network_planning.h:45-58),
 * same numbering (bit r of tmnn_network_plan.reasons). NO_FUSED_INSTANCE has
 * no reference counterpart: no FULLY_FUSED kernel is instantiated for the
 * shape (compile-time hidden-layer count / widths / geometry). */
#define TMNN_PLAN_NO_GPU_CONTEXT 1
#define TMNN_PLAN_THREADGROUP_MEMORY_EXCEEDED 4
#define TMNN_PLAN_UNSUPPORTED_INPUT_DIMS 6
#define TMNN_PLAN_UNSUPPORTED_OUTPUT_DIMS 7
#define TMNN_PLAN_HIDDEN_DIM_UNSUPPORTED 9
#define TMNN_PLAN_FORCED_TILED 10
#define TMNN_PLAN_FORCED_SAFE_DEBUG 11
#define TMNN_PLAN_NO_FUSED_INSTANCE 13

/* ---- descriptors ------------------------------------------------------ */

/* Model descriptor: HashGridEncoding::Config (hash_grid.h:19-26),
 * FullyFusedMLP::Config (fully_fused_mlp.h:18-23), TrainerConfig
 * (trainer.h:34-61) and WeightInitConfig (weight_init.h:113-141) in one POD.
 * Call tmnn_model_desc_init() for the reference defaults. */
typedef struct tmnn_model_desc {
  uint32_t struct_size;       /* sizeof(tmnn_model_desc) */
  /* encoding */
  int32_t spatial_dims;       /* 2 (the reference lifts to (x,y,0)), 3 or 4 */
  int32_t num_levels;         /* 1..32 */
  int32_t features_per_level; /* 1, 2 or 4 */
  int32_t log2_hashmap_size;  /* 10..24 */
  float base_resolution;
  float per_level_scale;
  /* network */
  int32_t hidden_dim;         /* 1..64; 128 (fp16 training, 16x2 inputs) */
  int32_t num_hidden_layers;  /* 1..8 */
  int32_t num_outputs;        /* 1..16 in this build */
  /* loss */
  int32_t loss_kind;          /* TMNN_LOSS_* */
  float huber_delta;
  /* optimizer (Adam) */
  float lr_encoding;
  float lr_network;
  float beta1;
  float beta2;
  float epsilon;
  float l1_reg;
  float l2_reg;
  float grad_clip;
  float weight_decay;
  /* trainer */
  int32_t batch_size;         /* steps use min(N, batch_size) points */
  int32_t precision;          /* TMNN_PRECISION_* (training / split path) */
  int32_t hash_adam_mode;     /* TMNN_HASH_ADAM_* */
  int32_t morton_sort;        /* 1: sort each batch by Morton code (reference) */
  /* weight init */
  uint64_t seed;
  float hash_init_range;      /* U(-r, r) for the table */
  /* planner: NetworkFactoryOptions::forced_family (network_planning.h:146-158) */
  int32_t forced_family;      /* TMNN_FAMILY_* (AUTO by default) */
} tmnn_model_desc;

/* Device capabilities the planner decides on: DeviceCapabilities of the
 * reference (common.h), MI355X terms. */
typedef struct tmnn_device_caps {
  uint32_t struct_size;       /* sizeof(tmnn_device_caps) */
  int32_t gpu_available;
  int32_t cu_count;
  int32_t lds_bytes_per_cu;   /* LDS one block may use (gfx950: 160 KB) */
  int32_t wave_size;          /* 64 */
  int32_t has_mfma_f16;       /* v_mfma_f32_16x16x32_f16 */
  uint64_t global_mem_bytes;
} tmnn_device_caps;

/* NetworkPlan (network_planning.h:160-174): the selected family, whether the
 * evaluator / training kernels are the fused (specialised) ones, the
 * candidates that were eligible (bit per family) and the recorded fallback
 * reasons (bit per reason). */
typedef struct tmnn_network_plan {
  uint32_t struct_size;       /* sizeof(tmnn_network_plan) */
  int32_t selected_family;    /* TMNN_FAMILY_*; -1 when no family can run the model */
  int32_t fused_eval;
  int32_t fused_train;
  uint64_t planner_fingerprint;  /* FNV-1a of the encoding/network/precision shape */
  uint32_t candidate_families;
  uint32_t reasons;
  int32_t train_lds_bytes;    /* LDS per block of the selected training kernel */
  int32_t train_waves_per_block;
  tmnn_device_caps capabilities;
} tmnn_network_plan;

/* NumericsReport (detail/runtime_stats.h:32-40), filled on sampled steps
 * (tmnn_set_numerics_sampling). The reductions run on the device inside the
 * step's own kernels: the training kernel keeps the largest |output| of its
 * points, the finish kernel (dW reduction + Adam) the gradient and update
 * terms. */
typedef struct tmnn_numerics_report {
  int32_t finite_forward;     /* the step's loss is finite */
  int32_t finite_backward;    /* every gradient is finite (hash int32 / 65536, MLP fp32) */
  int32_t finite_update;      /* every applied update (new weight, m, v, delta) is finite;
                                 0 whenever finite_backward is 0, as in the reference */
  float max_abs_activation;   /* largest |network output| over the batch's points (the
                                 reference declares the field and leaves it 0) */
  float max_abs_gradient;     /* largest |g| over the finite gradients */
  float max_abs_update;       /* largest |w_before - w_after| over the applied updates (lazy
                                 hash Adam: the visited entries; the reference's probe takes
                                 the dense candidate update of every entry) */
  uint32_t first_bad_layer;   /* 0, as the reference */
} tmnn_numerics_report;

/* Result of one fused training step: TrainingStepResult (common.h:97-110).
 * The caller sets struct_size. */
typedef struct tmnn_step_result {
  uint32_t struct_size;       /* sizeof(tmnn_step_result), set by the caller */
  float loss;                 /* sum of per-point losses / N */
  uint32_t step;              /* step counter after the update */
  uint32_t batch_n;           /* points used (after the batch cap) */
  float grad_norm;            /* sqrt(sum of g^2) over the step's gradients (reported steps) */
  int32_t numerics_reported;  /* 1: `numerics` holds this step's report */
  int32_t has_numerics_anomaly; /* a reported non-finite forward, backward or update */
  tmnn_numerics_report numerics;
} tmnn_step_result;

/* NumericsSamplingMode (runtime_policy.h:13-18), same numbering; the
 * sampling rule of NumericsGuard::should_sample (numerics_guard.cpp:12-36)
 * on the step counter after the update: SAMPLED reports step 1, every
 * interval-th step, a host-pointer step whose loss is not finite, and the
 * step after a reported anomaly; PERIODIC every interval-th step and the step
 * after an anomaly; FULL every step; DISABLED none (only a non-finite loss of
 * a host-pointer step is still reported, as finite_forward = 0). */
#define TMNN_NUMERICS_SAMPLED 0
#define TMNN_NUMERICS_PERIODIC 1
#define TMNN_NUMERICS_FULL 2
#define TMNN_NUMERICS_DISABLED 3

/* Realized kernel geometry: TrainerRuntimeInspection (trainer.h:63-87). */
typedef struct tmnn_inspection {
  int32_t family;             /* TMNN_FAMILY_* the trainer runs */
  int32_t precision;          /* TMNN_PRECISION_* of the training kernel */
  int32_t hidden_padded;      /* MFMA tile width of the hidden layers */
  int32_t input_padded;       /* MFMA tile width of the encoded input */
  int32_t points_per_wave_tile;
  int32_t waves_per_block_train;
  int32_t blocks_train;       /* persistent blocks of the training kernel */
  int32_t lds_bytes_train;
  int32_t lds_bytes_infer;
  int32_t cu_count;
  uint32_t hash_param_count;
  uint32_t mlp_param_count;
  uint32_t batch_size;
  int32_t train_fused_scatter; /* 1: the training kernel runs the hash-grid backward of
                                  each tile itself (no separate scatter kernel) */
} tmnn_inspection;

typedef struct tmnn_context tmnn_context;
typedef struct tmnn_trainer tmnn_trainer;

/* ---- errors ----------------------------------------------------------- */
/* Thread-local message of the calling thread's last failure
 * (DiagnosticInfo::message, diagnostics.h:199-245). */
const char *tmnn_last_error(void);
/* ABI version of this header (bumped on incompatible change). */
uint32_t tmnn_abi_version(void);

/* ---- context: MetalContext::create (metal_context.h:105-149) ------------ */
int tmnn_context_create(int32_t device, tmnn_context **out);
int tmnn_context_destroy(tmnn_context *ctx);
int tmnn_context_device_info(tmnn_context *ctx, int32_t *cu_count,
                             uint64_t *global_mem_bytes, char *name,
                             size_t name_capacity);
/* The context's device capabilities (MetalContext::capabilities). */
int tmnn_context_caps(tmnn_context *ctx, tmnn_device_caps *out);
/* Nominal MI355X capabilities (256 CUs, 160 KB LDS, wave 64, MFMA), for
 * planning without a device. */
void tmnn_device_caps_init(tmnn_device_caps *caps);

/* ---- planner: plan_network (network_planning.h:176-190;
 * network_planner.cpp:132-300). Pure host logic, no allocation: family
 * eligibility from the kernels this library instantiates and their LDS plans
 * against caps->lds_bytes_per_cu. tmnn_trainer_create runs the same planner
 * on its context's capabilities and builds its kernels from the result. */
int tmnn_plan_network(const tmnn_device_caps *caps, const tmnn_model_desc *desc,
                      tmnn_network_plan *out);

/* ---- model: try_create_trainer (default_trainer.cpp:2771-2818) ---------- */
void tmnn_model_desc_init(tmnn_model_desc *desc);
int tmnn_trainer_create(tmnn_context *ctx, const tmnn_model_desc *desc,
                        tmnn_trainer **out);
int tmnn_trainer_destroy(tmnn_trainer *tr);
int tmnn_trainer_param_counts(tmnn_trainer *tr, uint32_t *hash_count,
                              uint32_t *mlp_count);
int tmnn_trainer_inspect(tmnn_trainer *tr, tmnn_inspection *out);
/* The plan the trainer was built from. */
int tmnn_trainer_get_plan(tmnn_trainer *tr, tmnn_network_plan *out);

/* ---- compute ------------------------------------------------------------ */
/* ITrainerRuntime::training_step (trainer.h:140-141; default_trainer.cpp:
 * 883-1045). input [N][spatial_dims], target [N][num_outputs], host memory.
 * Synchronous: returns after Adam, with the loss. */
int tmnn_training_step(tmnn_trainer *tr, const float *input,
                       const float *target, int32_t n, tmnn_step_result *out);

/* Device-resident variant of training_step: input/target are device
 * pointers; the step is only enqueued, on the trainer's stream (and its Morton
 * sort on a second stream of the trainer). The inputs must be complete when
 * the call is made (nothing orders the step after work the caller has
 * enqueued elsewhere): use tmnn_training_step_device_after for inputs a
 * caller's stream is still producing. If loss_out (device pointer) is
 * non-null the step's loss is written there when the step executes. On
 * sampled steps the numerics report stays on the device until
 * tmnn_get_last_numerics. */
int tmnn_training_step_device(tmnn_trainer *tr, const float *d_input,
                              const float *d_target, int32_t n,
                              float *d_loss_out);

/* tmnn_training_step_device ordered after a caller's event: every stream of
 * the trainer that reads the inputs (the sort's and the step's) waits for
 * `wait_event` (a hipEvent_t of the trainer's device, recorded by the caller
 * after the work producing d_input / d_target; NULL: no wait) before it
 * reads them. No counterpart in the reference, whose steps take host
 * memory. */
int tmnn_training_step_device_after(tmnn_trainer *tr, const float *d_input,
                                    const float *d_target, int32_t n,
                                    float *d_loss_out, void *wait_event);

/* Records `event` (a hipEvent_t of the trainer's device) on the trainer's
 * stream after everything enqueued so far: a caller's stream that waits for
 * it sees the outputs of the preceding *_device calls (loss, inference
 * outputs, updated weights). */
int tmnn_record_event(tmnn_trainer *tr, void *event);

/* Numerics sampling of the training steps (RuntimePolicy::
 * numerics_sampling_mode / numerics_sample_interval, runtime_policy.h:
 * 30-38): mode TMNN_NUMERICS_*, interval >= 1 (reference default SAMPLED,
 * 128). Resets the anomaly history. */
int tmnn_set_numerics_sampling(tmnn_trainer *tr, int32_t mode, uint32_t interval);

/* The report of the last sampled step (host-pointer or device step): waits
 * for the trainer's stream, then fills out (out->struct_size set by the
 * caller) with that step's loss, step counter, batch size, grad_norm and
 * numerics; numerics_reported = 0 when no step has been sampled yet. */
int tmnn_get_last_numerics(tmnn_trainer *tr, tmnn_step_result *out);

/* Bytes of the per-device scratch behind tmnn_training_step_device_noalloc. */
#define TMNN_NOALLOC_SCRATCH_BYTES (80u << 20)

/* Allocation-free variant of tmnn_training_step_device. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). Same arguments, same result, same kernels; it calls no
 * hipMalloc / hipFree / hipEventCreate: the step's batch-sized buffers (sort
 * keys and values, radix histograms, sorted positions and targets, feature
 * tiles, input-feature gradients) live in a fixed device scratch of
 * TMNN_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends, instead
 * of trainer buffers grown on demand. Trainer state (parameters, moments,
 * gradients, visit flags, dW partial rows) was allocated by
 * tmnn_trainer_create. The scratch needs about
 * (16 + 4 * (spatial_dims + num_outputs) + 4 * (input_padded + L * F)) bytes
 * per point (each region rounded to 256 bytes, plus the radix histograms):
 * the C2 image-fit step (2D, 16x2 features, 3 outputs) fits 2^18 points.
 * Larger batches return TMNN_ERR_INVALID_ARGUMENT; hidden width 128 and the
 * layer-wise (Tiled) path return TMNN_ERR_UNSUPPORTED. Steps are not
 * profiled. Every call on one GPU shares that GPU's scratch, which keeps the
 * last call's contents: calls from trainers on different streams of one GPU
 * are ordered by a per-device event (each waits for the previous call's
 * kernels before its first kernel; the enqueue itself holds a process-wide
 * lock), so they take the scratch in turn, in the order the calls were
 * made. A caller that needs a particular order across threads must impose
 * it itself. */
int tmnn_training_step_device_noalloc(tmnn_trainer *tr, const float *d_input,
                                      const float *d_target, int32_t n,
                                      float *d_loss_out);

/* FieldEvaluator::evaluate / Trainer::inference (evaluator.h:22-59;
 * default_trainer.cpp:321-465): fp32, unsorted, no batch cap.
 * positions [N][spatial_dims] -> output [N][num_outputs], host memory. */
int tmnn_inference(tmnn_trainer *tr, const float *positions, float *output,
                   int32_t n);
/* Device-pointer variant; only enqueues, on the trainer's stream (the
 * positions must be complete when the call is made). */
int tmnn_inference_device(tmnn_trainer *tr, const float *d_positions,
                          float *d_output, int32_t n);
/* tmnn_inference_device ordered after a caller's event (NULL: no wait), as
 * tmnn_training_step_device_after. */
int tmnn_inference_device_after(tmnn_trainer *tr, const float *d_positions,
                                float *d_output, int32_t n, void *wait_event);

/* FieldEvaluator::evaluate_with_gradient (evaluator.h:41-50;
 * default_trainer.cpp:467-620): outputs [N][num_outputs] and the Jacobian
 * gradients [N][num_outputs][spatial_dims] (d output / d position, row-major,
 * evaluator.h:10-12), fp32, unsorted, no batch cap. Host memory. */
int tmnn_evaluate_with_gradient(tmnn_trainer *tr, const float *positions,
                                float *output, float *gradients, int32_t n);

/* ITrainerRuntime::forward_for_training (trainer.h:145-150;
 * default_trainer.cpp:1047-1127): forward in the training precision, output
 * in the caller's point order. *written = min(N, batch_size) * num_outputs. */
int tmnn_forward_for_training(tmnn_trainer *tr, const float *input,
                              float *output, int32_t n, uint32_t *written);

/* ITrainerRuntime::zero_gradients / backward_accumulate / adam_step
 * (trainer.h:160-174; default_trainer.cpp:1300-1443). */
int tmnn_zero_gradients(tmnn_trainer *tr);
int tmnn_backward_accumulate(tmnn_trainer *tr, const float *input,
                             const float *d_output, int32_t n);
int tmnn_adam_step(tmnn_trainer *tr);

/* Block until all work enqueued on the trainer's stream has finished
 * (ITrainerRuntime::sync_weights, trainer.h:182). */
int tmnn_synchronize(tmnn_trainer *tr);

/* ---- state ----------------------------------------------------------------- */
/* ITrainerRuntime::step (trainer.h:183). */
int tmnn_get_step(tmnn_trainer *tr, uint32_t *step);

/* RuntimeAuthority::buffer(HashWeights | MlpWeights) download
 * (runtime_authority.h:68-79). Layouts: hash [L][T][F] fp32;
 * MLP [W0 (in x H), b0, W1, b1, ..., WO (H x M), bO] fp32. Either pointer may
 * be null to skip; counts must match exactly. */
int tmnn_get_weights(tmnn_trainer *tr, float *hash, size_t hash_count,
                     float *mlp, size_t mlp_count);

/* ITrainerRuntime::set_initial_weights (trainer.h:197-207;
 * default_trainer.cpp:1555-1643): replaces weights, resets Adam and step. */
int tmnn_set_initial_weights(tmnn_trainer *tr, const float *hash,
                             size_t hash_count, const float *mlp,
                             size_t mlp_count);

/* OptimizerStateBlob v1 (detail/runtime_authority.h; default_trainer.cpp:
 * 1645-1768): payload = 4 sections [u32 LE byte_len][fp32 bytes] in the
 * order m_hash, v_hash, m_mlp, v_mlp. Export: pass payload=NULL to query
 * *payload_len; version is always 1. */
int tmnn_export_optimizer_state(tmnn_trainer *tr, uint32_t *version,
                                uint32_t *step, uint8_t *payload,
                                size_t capacity, size_t *payload_len);
int tmnn_import_optimizer_state(tmnn_trainer *tr, uint32_t version,
                                uint32_t step, const uint8_t *payload,
                                size_t payload_len);

/* ITrainerRuntime::reset_optimizer / apply_optimizer_config
 * (trainer.h:208-209): zero m, v and the step; set learning rates. */
int tmnn_reset_optimizer(tmnn_trainer *tr);
int tmnn_set_learning_rate(tmnn_trainer *tr, float lr_encoding,
                           float lr_network);

/* ---- runtime authority: RuntimeAuthority (detail/runtime_authority.h:
 * 110-119) and ITrainerRuntime::batch_plan (trainer.h:186) ----------------- */

/* RuntimeBufferRole (runtime_authority.h:68-79), same numbering. */
#define TMNN_BUFFER_CONFIG_WEIGHTS 0
#define TMNN_BUFFER_HASH_WEIGHTS 1
#define TMNN_BUFFER_MLP_WEIGHTS 2
#define TMNN_BUFFER_GRAD_HASH 3
#define TMNN_BUFFER_GRAD_MLP 4
#define TMNN_BUFFER_TRAIN_PARAMS 5
#define TMNN_BUFFER_ADAM_PARAMS 6
#define TMNN_BUFFER_FUSED_WEIGHTS 7
#define TMNN_BUFFER_FUSED_FIRST_MOMENT 8
#define TMNN_BUFFER_FUSED_SECOND_MOMENT 9

/* StorageVisibility / ResourceLifetime (runtime_authority.h:21-31). */
#define TMNN_STORAGE_CPU_VISIBLE 0
#define TMNN_STORAGE_GPU_ONLY 1
#define TMNN_LIFETIME_PERSISTENT 0
#define TMNN_LIFETIME_TRANSIENT 1
#define TMNN_LIFETIME_STAGING 2

/* Element encoding of a buffer view. I32_PACKED_PAIR: the int32 fixed-point
 * hash gradients of F == 2 tables, where each entry's two words hold one
 * 64-bit sum: word 0 is feature 0's int32 sum and feature 1's sum is
 * word 1 + (word 0 < 0 ? 1 : 0) (two's complement, wrapping).
 * tmnn_debug_get_gradients returns the unpacked reference layout. */
#define TMNN_ELEM_F32 0
#define TMNN_ELEM_I32 1
#define TMNN_ELEM_I32_PACKED_PAIR 2
#define TMNN_ELEM_OPAQUE 3

/* RuntimeBufferView (runtime_authority.h:81-93): gpu_buffer + offset is the
 * role's first byte (device_ptr, for convenience). Device memory only
 * (cpu_data is always null in this library): read it with hipMemcpy on the
 * trainer's device, after tmnn_synchronize. The pointers stay valid until the
 * trainer is destroyed. */
typedef struct tmnn_buffer_view {
  uint32_t struct_size;       /* sizeof(tmnn_buffer_view), set by the caller */
  int32_t role;               /* TMNN_BUFFER_* */
  void *gpu_buffer;           /* base of the allocation (NULL: no such buffer) */
  uint64_t offset;            /* byte offset of the role's data in it */
  uint64_t bytes;             /* 0: no such buffer (RuntimeBufferView::valid() false) */
  void *device_ptr;           /* gpu_buffer + offset */
  int32_t element_kind;       /* TMNN_ELEM_* */
  int32_t visibility;         /* TMNN_STORAGE_* */
  int32_t lifetime;           /* TMNN_LIFETIME_* */
} tmnn_buffer_view;

/* ParameterLayout (runtime_authority.h:33-43). This library passes the step
 * parameters and Adam's hyper-parameters as kernel launch arguments, so the
 * TrainParams / AdamParams / config-header float counts are 0. */
typedef struct tmnn_parameter_layout_t {
  uint32_t struct_size;
  uint32_t hash_grid_float_count;
  uint32_t mlp_weight_float_count;
  uint32_t train_params_float_count;
  uint32_t train_params_idx_n;
  uint32_t train_params_idx_unsigned_mode;
  uint32_t train_params_idx_loss_scale;
  uint32_t train_params_idx_num_active_levels;
  uint32_t adam_params_float_count;
  uint32_t config_header_float_count;
  uint32_t config_tail_float_count;
  uint32_t target_dims;
  uint32_t reduction_terms;
  int32_t fused_adam;
} tmnn_parameter_layout_t;

/* TrainerBatchPlan (runtime_authority.h:45-56). max_batch_size is the
 * configured batch_size (no 65536 cap in this library); one step lane. */
typedef struct tmnn_batch_plan_t {
  uint32_t struct_size;
  uint32_t max_batch_size;
  uint32_t lane_count;
  uint32_t input_dims;
  uint32_t target_dims;
  uint32_t reduction_terms;
  uint64_t positions_bytes_per_lane;
  uint64_t targets_bytes_per_lane;
  uint64_t reduction_bytes_per_lane;
  uint32_t threadgroup_size;       /* threads per block of the training kernel */
  uint32_t points_per_threadgroup; /* points one block takes per round */
} tmnn_batch_plan_t;

/* RuntimeStoragePolicy (runtime_authority.h:58-66). */
typedef struct tmnn_storage_policy_t {
  uint32_t struct_size;
  int32_t parameter_weights;  /* TMNN_STORAGE_* */
  int32_t gradients;
  int32_t optimizer_state;
  int32_t control_buffers;
  int32_t step_inputs;        /* TMNN_LIFETIME_* */
  int32_t step_targets;
  int32_t step_reduction;
  int32_t requires_staging_uploads;
} tmnn_storage_policy_t;

/* RuntimeAuthority::buffer(role) (default_trainer.cpp:263-297). out->struct_size
 * must be set. Unknown roles: TMNN_ERR_INVALID_ARGUMENT. */
int tmnn_runtime_buffer(tmnn_trainer *tr, int32_t role, tmnn_buffer_view *out);
/* RuntimeAuthority::parameter_layout (default_trainer.cpp:258-260). */
int tmnn_parameter_layout(tmnn_trainer *tr, tmnn_parameter_layout_t *out);
/* RuntimeAuthority::storage_policy (default_trainer.cpp:261-263). */
int tmnn_storage_policy(tmnn_trainer *tr, tmnn_storage_policy_t *out);
/* ITrainerRuntime::batch_plan (trainer.h:186; default_trainer.cpp:1531-1533). */
int tmnn_batch_plan(tmnn_trainer *tr, tmnn_batch_plan_t *out);

/* ---- step profiling ------------------------------------------------------------ */
/* Opt-in GPU timing of the fused step's phases, the GPU-timestamp fields of
 * TrainingStepProfile (trainer.h:89-133; set_training_step_profiling,
 * trainer.h:214-217,422-431). While enabled, profiled training steps bracket
 * each phase with HIP events on the trainer's stream. The profile holds the
 * sums over the profiled steps since profiling was (re-)enabled; reading it
 * waits for the stream. gpu_*_us are GPU execution microseconds between
 * events (each event pair also costs a few microseconds of stream time). */
typedef struct tmnn_step_profile {
  uint32_t steps;             /* profiled steps summed below */
  uint32_t batch_size;        /* points of the last profiled step */
  double gpu_sort_us;         /* Morton codes + radix sort + gather, weight-image packing */
  double gpu_fwd_bwd_us;      /* the MLP kernel: forward, loss, backward to dx */
  double gpu_scatter_us;      /* hash-grid backward scatter + visit flags */
  double gpu_reduce_us;       /* dW partial reduction + loss reduction */
  double gpu_adam_us;         /* fused Adam pass (+ mask/grad clearing) */
  double gpu_total_us;        /* first event to last event, summed */
  double gpu_encode_us;       /* hash-grid encode forward (features of the batch) */
  uint32_t infer_calls;       /* profiled inference calls summed below */
  double gpu_infer_us;        /* the inference forward kernel (tmnn_inference[_device]) */
  /* the step's main kernels alone, from their dispatches' own start and end
   * timestamps (a phase above also holds the launch gap before its kernel);
   * 0 where the step has no such kernel or (layer-wise path) runs several */
  double gpu_encode_kernel_us;
  double gpu_train_kernel_us;   /* the MLP training kernel (with the fused hash-grid backward) */
  double gpu_scatter_kernel_us;
  double gpu_finish_kernel_us;
} tmnn_step_profile;

/* enabled: 0 off; k >= 1 profiles one training step in k (the first after
 * enabling, then every k-th; 1 = every step, the reference's on), and one
 * inference call in k the same way. Resets the sums. Negative:
 * TMNN_ERR_INVALID_ARGUMENT. */
int tmnn_set_step_profiling(tmnn_trainer *tr, int32_t enabled);
int tmnn_get_step_profile(tmnn_trainer *tr, tmnn_step_profile *out);

/* Per-step times (GPU microseconds) of the profiled training steps since
 * profiling was (re-)enabled, in step order: row i holds
 * TMNN_PROFILE_COLUMNS floats indexed by TMNN_PROFILE_*: the phases, their
 * total, then the main kernels alone (as the *_kernel_us fields of
 * tmnn_step_profile). *count receives the number of profiled steps; at most
 * `capacity` rows are written (out may be NULL to query). Waits for the
 * stream. A phase or kernel without work (the fused step's scatter and
 * reduce phases and scatter kernel) reads 0. */
#define TMNN_PROFILE_SORT 0
#define TMNN_PROFILE_ENCODE 1
#define TMNN_PROFILE_FWD_BWD 2
#define TMNN_PROFILE_SCATTER 3
#define TMNN_PROFILE_REDUCE 4
#define TMNN_PROFILE_ADAM 5
#define TMNN_PROFILE_TOTAL 6
#define TMNN_PROFILE_KERNEL_ENCODE 7
#define TMNN_PROFILE_KERNEL_TRAIN 8
#define TMNN_PROFILE_KERNEL_SCATTER 9
#define TMNN_PROFILE_KERNEL_FINISH 10
#define TMNN_PROFILE_COLUMNS 11
int tmnn_get_step_profile_samples(tmnn_trainer *tr, float *out, uint32_t capacity,
                                  uint32_t *count);

/* ---- inspection hooks of the path (used by the parity tests) --------------- */
/* Encode forward only (emitHashEncodeUnified, mlp_kernel_emitter.cpp:
 * 205-360): features [N][L*F] fp32; corner_index / corner_weight (nullable)
 * [N][L][2^spatial_dims] in the reference's corner order. Host memory. */
int tmnn_debug_encode(tmnn_trainer *tr, const float *positions, int32_t n,
                      float *features, uint32_t *corner_index,
                      float *corner_weight);

/* The training step's own encode (the feature-tile kernels the step launches,
 * point- or level-major by the table size, reading the batch through the
 * step's Morton permutation when `sorted` and the trainer sorts): features
 * [N][L*F] fp32 in the step's point order, i.e. row j belongs to input row
 * perm_out[j] (identity when unsorted). sorted_pos_out [N][spatial_dims]
 * receives the positions the encode wrote for the backward scatter (nullable),
 * *padding_nonzero the count of nonzero padding floats in the feature tiles
 * (padding features and points; 0 when correct; nullable). Host memory.
 * No counterpart in the reference (its training kernel encodes inline). */
int tmnn_debug_encode_tiles(tmnn_trainer *tr, const float *positions, int32_t n,
                            int32_t sorted, float *features, uint32_t *perm_out,
                            float *sorted_pos_out, uint64_t *padding_nonzero);

/* Reference rates of the hash-grid memory operations at this trainer's
 * shape, over n device-resident points (d_positions [n][spatial_dims]; with
 * `sorted`, in the training step's Morton order): the average GPU time of one
 * launch (over `reps`) of a kernel that only (gather) loads every corner's F
 * floats of every level, (atomic) adds a constant with the scatter's atomic
 * per corner and level into a scratch table, (flag) stores the visit byte per
 * corner and level. Each kernel walks the levels as the kernel it stands
 * for does: level-major (one level's table slice at a time) for the gather
 * when the trainer's encode is level-major (level slices over 2 MB), and for
 * the atomic and flag kernels when its scatter is (over 8 MB); else
 * point-major. Trainer state is not touched. The achievable-bandwidth
 * denominators of the encode and scatter; no counterpart in the reference. */
int tmnn_debug_hash_rates(tmnn_trainer *tr, const float *d_positions, int32_t n,
                          int32_t sorted, int32_t reps, double *gather_us,
                          double *atomic_us, double *flag_us);

/* The training kernel's forward outputs of one fused step: runs a regular
 * training step (Adam included, the step counter advances) on host-memory
 * input/target and also writes the network outputs the step's own training
 * kernel computed, [N][num_outputs] in the caller's row order. result as
 * tmnn_training_step (nullable). No counterpart in the reference (a parity
 * read-out of its fused step's forward). */
int tmnn_debug_step_outputs(tmnn_trainer *tr, const float *input, const float *target,
                            int32_t n, float *outputs, tmnn_step_result *result);

/* LDS read bandwidth of the context's device, bytes per second: a kernel of
 * conflict-free 16-byte lane reads (ds_read_b128, as the MLP kernels read
 * their weight fragments and parked operands) on every CU, `reps` timed
 * launches. The LDS peak of the MLP kernels' roofline; no counterpart in the
 * reference. */
int tmnn_debug_lds_rate(tmnn_context *ctx, int32_t reps, double *bytes_per_s);

/* Accumulated gradients in reference layout: int32 fixed-point hash grads
 * [L][T][F] (scale 65536) and fp32 MLP grads. Either pointer may be null. */
int tmnn_debug_get_gradients(tmnn_trainer *tr, int32_t *grad_hash,
                             size_t hash_count, float *grad_mlp,
                             size_t mlp_count);

/* Active-hash mask words (bit per entry pair when F == 2, else per float). */
int tmnn_debug_get_active_mask(tmnn_trainer *tr, uint32_t *words,
                               size_t word_count);

/* The step's Morton sort of a batch (morton_sort_batch, morton_sort.h:
 * 60-110): codes[i] = Morton code of positions[i] (2D: the x/y interleave of
 * the lifted point, which orders identically), perm[j] = input row of the
 * j-th point in sorted order (stable: ties keep input order). Host memory. */
int tmnn_debug_morton_sort(tmnn_trainer *tr, const float *positions, int32_t n,
                           uint32_t *codes, uint32_t *perm);

/* Per-level resolution table used by every kernel (L floats). */
int tmnn_debug_get_resolutions(tmnn_trainer *tr, float *out, int32_t count);

/* The training plan's packed weight image (LDS head: weight fragments,
 * biases, resolution table): `current` as the training step left it (a fused
 * step updates it in place with the new weights) and `repacked` as rebuilt
 * from the parameters now; the two are byte-identical. *bytes receives the
 * image size; pass NULL for both buffers to query it. Host memory. No
 * counterpart in the reference (its weights live in device buffers read by
 * the kernels directly). */
int tmnn_debug_train_image(tmnn_trainer *tr, void *current, void *repacked, uint64_t *bytes);

/* The seeded Philox-4x32-10 uniform fill used for weight init
 * (detail::context_dispatch_init_uniform, metal_context.cpp:731-982):
 * out[count] = low + u * (high - low), counters base, base+1, ...
 * Host output. */
int tmnn_debug_philox_uniform(tmnn_context *ctx, uint64_t seed,
                              uint32_t counter_base, uint32_t count, float low,
                              float high, float *out);

#ifdef __cplusplus
}
#endif

#endif /* TMNN_HIP_H */
