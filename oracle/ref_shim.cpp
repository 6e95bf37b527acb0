// ref_shim.cpp -- C entry points over the reference's own host-side sources,
// compiled in place from the reference checkout (never copied) into
// oracle/_ref/libtmnn_ref.so. TEST INFRASTRUCTURE ONLY: used by tests/ to pin
// the oracle against the reference's real code where that code is plain C++.
//
// Compiled reference sources (paths relative to the reference checkout):
//   src/tiny_metal_nn/runtime/morton_sort.h        (Morton code + batch sort)
//   src/tiny_metal_nn/kernels/kernel_spec.cpp      (KernelSpec::mlpWeightCount,
//                                                   validate, fromConfigHeader)
//   include/tiny-metal-nn/detail/{l2,l1,huber,cosine}_loss.h (CPU losses)
//   src/tiny_metal_nn/kernels/mlp_kernel_emitter.cpp (the MSL text the
//                                                   reference generates; the
//                                                   tests read it, nothing runs it)
// The reference's GPU arithmetic exists only as MSL text emitted for Metal and
// cannot execute here; see oracle/tmnn_oracle.cpp for its restatement.
#include "tiny_metal_nn/runtime/morton_sort.h"
#include "tiny-metal-nn/kernels/kernel_spec.h"
#include "tiny-metal-nn/detail/l2_loss.h"
#include "tiny-metal-nn/detail/l1_loss.h"
#include "tiny-metal-nn/detail/huber_loss.h"
#include "tiny-metal-nn/detail/cosine_loss.h"
#include "tiny-metal-nn/kernels/mlp_kernel_emitter.h"

#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <vector>

extern "C" {

uint32_t ref_morton_code_3d(float x, float y, float z) {
  return tmnn::detail::morton_code_3d(x, y, z);
}

uint32_t ref_morton_code_4d(float x, float y, float z, float w) {
  return tmnn::detail::morton_code_4d(x, y, z, w);
}

// morton_sort_batch: writes the sorted positions/targets and the permutation
// (indices[sorted_i] = original_i). Returns 0 on success, -1 on error.
int ref_morton_sort_batch(const float *input, const float *target, int n,
                          uint32_t input_dims, uint32_t target_dims,
                          float *sorted_pos, float *sorted_tgt,
                          uint32_t *indices) {
  try {
    std::vector<uint32_t> idx, codes;
    std::vector<float> sp, st;
    tmnn::detail::morton_sort_batch(input, target, n, input_dims, target_dims,
                                    idx, codes, sp, st);
    std::memcpy(sorted_pos, sp.data(), sp.size() * sizeof(float));
    std::memcpy(sorted_tgt, st.data(), st.size() * sizeof(float));
    std::memcpy(indices, idx.data(), idx.size() * sizeof(uint32_t));
    return 0;
  } catch (...) {
    return -1;
  }
}

int ref_mlp_weight_count(int input_dim, int hidden_dim, int num_hidden_layers,
                         int num_outputs) {
  tmnn::KernelSpec s;
  s.input_dim = input_dim;
  s.hidden_dim = hidden_dim;
  s.num_hidden_layers = num_hidden_layers;
  s.num_outputs = num_outputs;
  return s.mlpWeightCount();
}

// KernelSpec::validate on the given geometry: 0 = valid, 1 = rejected.
int ref_kernel_spec_validate(int num_levels, int features_per_level,
                             int log2_hashmap_size, int hidden_dim,
                             int num_hidden_layers, int spatial_dims) {
  tmnn::KernelSpec s;
  s.num_levels = num_levels;
  s.features_per_level = features_per_level;
  s.log2_hashmap_size = log2_hashmap_size;
  s.hidden_dim = hidden_dim;
  s.num_hidden_layers = num_hidden_layers;
  s.spatial_dims = spatial_dims;
  s.input_dim = num_levels * features_per_level;
  s.encoding = spatial_dims == 4 ? tmnn::KernelSpec::FourD
                                 : tmnn::KernelSpec::Standard;
  try {
    s.validate();
    return 0;
  } catch (const std::invalid_argument &) {
    return 1;
  }
}

// CPU loss classes: kind 0 L2, 1 L1, 2 Huber(delta), 3 Cosine(output_dims).
float ref_loss_evaluate_cpu(int kind, const float *pred, const float *target,
                            int n, float delta, uint32_t output_dims) {
  switch (kind) {
    case 0: return tmnn::L2Loss().evaluate_cpu(pred, target, n);
    case 1: return tmnn::L1Loss().evaluate_cpu(pred, target, n);
    case 2: return tmnn::HuberLoss(delta).evaluate_cpu(pred, target, n);
    case 3: return tmnn::CosineLoss(output_dims).evaluate_cpu(pred, target, n);
    default: return -1.0f;
  }
}

// MSL source the reference emits for one geometry (kind 0: scalar training
// kernel with int atomics and the active-hash mask, 1: evaluation kernel).
// Writes up to capacity-1 bytes + NUL; returns the full length, or -1.
long ref_emit_kernel_source(int kind, int spatial_dims, int num_levels,
                            int features_per_level, int log2_hashmap_size,
                            float base_resolution, float per_level_scale,
                            int hidden_dim, int num_hidden_layers,
                            int num_outputs, int loss, char *buf,
                            size_t capacity) {
  try {
    tmnn::KernelSpec s;
    s.num_levels = num_levels;
    s.features_per_level = features_per_level;
    s.log2_hashmap_size = log2_hashmap_size;
    s.base_resolution = base_resolution;
    s.per_level_scale = per_level_scale;
    s.hidden_dim = hidden_dim;
    s.num_hidden_layers = num_hidden_layers;
    s.num_outputs = num_outputs;
    s.input_dim = num_levels * features_per_level;
    s.spatial_dims = spatial_dims;
    s.encoding = spatial_dims == 4 ? tmnn::KernelSpec::FourD
                                   : tmnn::KernelSpec::Standard;
    s.loss = static_cast<tmnn::KernelSpec::LossType>(loss);
    s.use_simd = false;
    s.use_fp16 = false;
    s.use_int_atomics = true;
    s.emit_active_hash_mask = true;
    tmnn::MLPKernelEmitter e;
    const std::string src = kind == 0 ? e.emitTrainKernel(s) : e.emitEvalKernel(s);
    if (buf && capacity > 0) {
      const size_t n = src.size() < capacity - 1 ? src.size() : capacity - 1;
      std::memcpy(buf, src.data(), n);
      buf[n] = '\0';
    }
    return static_cast<long>(src.size());
  } catch (...) {
    return -1;
  }
}

}  // extern "C"
