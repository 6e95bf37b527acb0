// sort.hpp -- stable LSD radix sort of (Morton code, point index) pairs on the
// trainer's stream. Replaces the reference's per-step host std::sort
// (src/tiny_metal_nn/runtime/morton_sort.h:60-110); ties keep input order.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace tmnn_hip {

hipError_t morton_sort_temp_bytes(int n, size_t *bytes);

hipError_t morton_sort_pairs(void *tmp, size_t &tmp_bytes, const uint32_t *keys_in,
                             uint32_t *keys_out, const uint32_t *vals_in,
                             uint32_t *vals_out, int n, int end_bit, hipStream_t stream);

}  // namespace tmnn_hip
