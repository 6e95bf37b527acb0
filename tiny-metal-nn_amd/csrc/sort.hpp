// sort.hpp -- stable LSD radix sort of (Morton code, point index) pairs on the
// trainer's stream. Replaces the reference's per-step host std::sort
// (src/tiny_metal_nn/runtime/morton_sort.h:60-110); ties keep input order.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace tmnn_hip {

// Scratch bytes morton_sort_pairs needs for n keys.
hipError_t morton_sort_temp_bytes(int n, size_t *bytes);

// Sorts keys0[0..n) (bits [0, end_bit)) with the point index as payload.
// keys0/keys1 and vals0/vals1 are ping-pong buffers of n elements; keys0 is
// overwritten. The payload of the first pass is the identity (vals0 is not
// read). On return *keys_sorted / *vals_sorted point at the buffers holding
// the sorted keys and their original indices.
hipError_t morton_sort_pairs(void *tmp, size_t tmp_bytes, uint32_t *keys0, uint32_t *keys1,
                             uint32_t *vals0, uint32_t *vals1, int n, int end_bit,
                             hipStream_t stream, const uint32_t **keys_sorted,
                             const uint32_t **vals_sorted);

}  // namespace tmnn_hip
