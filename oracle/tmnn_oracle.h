/*
 * tmnn_oracle.h -- CPU restatement of tiny-metal-nn's neural-field hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker for the
 * HIP product library and the CPU baseline timed beside it. Nothing in the
 * product (tiny-metal-nn_amd/) links, loads or calls it; only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may.
 *
 * Every function restates the scalar MSL the reference emits (all paths are
 * relative to the reference checkout):
 *   src/tiny_metal_nn/kernels/mlp_kernel_emitter.cpp   (encode, MLP, loss, bwd)
 *   include/tiny-metal-nn/kernels/adam_kernel_msl.h     (Adam)
 *   src/tiny_metal_nn/runtime/adam_params.h             (bias corrections)
 *   src/tiny_metal_nn/runtime/metal_context.cpp         (Philox init)
 *   src/tiny_metal_nn/runtime/default_trainer.cpp       (init streams, sparse Adam)
 *   src/tiny_metal_nn/runtime/morton_sort.h             (Morton code)
 * Per-function citations are in tmnn_oracle.cpp.
 */
#ifndef TMNN_ORACLE_H
#define TMNN_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_L2 = 0, ORC_L1 = 1, ORC_HUBER = 2, ORC_COSINE = 3, ORC_RELATIVE_L2 = 4 };

typedef struct orc_model {
  int32_t spatial_dims;       /* 2 (evaluated as the reference's lifted (x,y,0)), 3 or 4 */
  int32_t num_levels;
  int32_t features_per_level; /* 1, 2 or 4 */
  int32_t log2_hashmap_size;
  float base_resolution;
  float per_level_scale;
  int32_t hidden_dim;
  int32_t num_hidden_layers;
  int32_t num_outputs;
  int32_t loss_kind;          /* ORC_* */
  float huber_delta;
} orc_model;

typedef struct orc_adam {
  float lr_encoding;
  float lr_network;
  float beta1;
  float beta2;
  float epsilon;
  float l1_reg;
  float l2_reg;
  float grad_clip;
  float weight_decay;
} orc_adam;

/* Sizes. */
uint32_t orc_hash_param_count(const orc_model *m);
uint32_t orc_mlp_param_count(const orc_model *m);
uint32_t orc_mask_word_count(const orc_model *m);

/* Per-level resolution table (L floats). */
void orc_resolutions(const orc_model *m, float *out);

/* Philox-4x32-10 uniform fill (one counter per 4 outputs). */
void orc_philox_uniform(uint64_t seed, uint32_t counter_base, uint32_t count,
                        float low, float high, float *out);

/* Default weight init: hash U(+-hash_range), MLP Kaiming-uniform (ReLU gain)
 * weights and U(+-1/sqrt(fan_in)) biases, all from one Philox stream. */
void orc_init_params(const orc_model *m, uint64_t seed, float hash_range,
                     float *hash_out, float *mlp_out);

/* Encode forward. feats: [N][L*F]. corner_idx / corner_w (nullable):
 * [N][L][C] with C = 8 for 2D/3D, 16 for 4D (2D points are lifted to
 * (x, y, 0) exactly as the reference does; their dz=1 corners carry weight 0).
 * corner_idx holds the hashed entry index h in [0, T). */
void orc_encode(const orc_model *m, const float *table, const float *pos,
                int32_t n, float *feats, uint32_t *corner_idx, float *corner_w);

/* Inference forward: out [N][num_outputs]. */
void orc_forward(const orc_model *m, const float *table, const float *mlp,
                 const float *pos, int32_t n, float *out);

/* Fused forward+backward over a batch. Exactly one of target (internal loss)
 * or d_out_ext (external output gradient) is non-null.
 * Accumulates into grad_hash (int32 fixed point, wraps), grad_mlp (double,
 * order-free sum of the per-point fp32 terms) and mask (bit per tracked slot).
 * loss_sum (nullable) receives the sum of per-point losses (double).
 * out (nullable) receives the forward outputs [N][num_outputs].
 * n_threads <= 1 runs serially. */
void orc_forward_backward(const orc_model *m, const float *table,
                          const float *mlp, const float *pos, int32_t n,
                          const float *target, const float *d_out_ext,
                          int32_t *grad_hash, double *grad_mlp, uint32_t *mask,
                          double *loss_sum, float *out, int32_t n_threads);

/* Bias corrections exactly as the host computes them. */
void orc_adam_bias_corrections(float beta1, float beta2, uint32_t logical_step,
                               float *bc1, float *bc2);

/* Adam update of params = [hash | mlp], m, v (same layout).
 * mask == NULL selects the dense unified kernel for the hash part; otherwise
 * the lazy sparse kernel updates only masked entries. */
void orc_adam_step(const orc_model *m, const orc_adam *a, uint32_t logical_step,
                   float *params, float *mom1, float *mom2,
                   const int32_t *grad_hash, const float *grad_mlp,
                   const uint32_t *mask, int32_t n_threads);

/* Morton code of one point set: codes[N]. dims 2 is lifted to (x, y, 0). */
void orc_morton_codes(const float *pos, int32_t n, int32_t dims, uint32_t *codes);

/* FieldEvaluator::evaluate_with_gradient: out [N][num_outputs] and the
 * Jacobian grads [N][num_outputs][spatial_dims] (d out / d position). */
void orc_evaluate_with_gradient(const orc_model *m, const float *table,
                                const float *mlp, const float *pos, int32_t n,
                                float *out, float *grads);

/* One full reference training step: forward/backward with internal loss,
 * lazy hash Adam + dense MLP Adam (dense hash when dense_hash != 0 or
 * l1_reg != 0), grads and mask consumed. Returns the reported loss
 * (sum of per-point losses / N). */
float orc_training_step(const orc_model *m, const orc_adam *a,
                        uint32_t logical_step, float *params, float *mom1,
                        float *mom2, const float *pos, const float *target,
                        int32_t n, int32_t dense_hash, int32_t n_threads);

#ifdef __cplusplus
}
#endif

#endif /* TMNN_ORACLE_H */
