// sort.hpp -- stable LSD radix sort of the batch by Morton code on the
// trainer's stream. Replaces the reference's per-step host std::sort
// (src/tiny_metal_nn/runtime/morton_sort.h:60-110); ties keep input order.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace tmnn_hip {

// Scratch bytes morton_sort_batch needs for n points.
hipError_t morton_sort_temp_bytes(int n, size_t *bytes);

// Sorts the n points pos[n][dims] (dims 2..4) by the reference's Morton code,
// which the first radix pass computes from the positions. keys0/keys1 and
// vals0/vals1 are ping-pong buffers of n elements. On return *keys_sorted /
// *vals_sorted point at the buffers holding the sorted codes and, for each
// sorted slot, the point's original index.
hipError_t morton_sort_batch(void *tmp, size_t tmp_bytes, const float *pos, int dims,
                             uint32_t *keys0, uint32_t *keys1, uint32_t *vals0, uint32_t *vals1,
                             int n, hipStream_t stream, const uint32_t **keys_sorted,
                             const uint32_t **vals_sorted);

}  // namespace tmnn_hip
