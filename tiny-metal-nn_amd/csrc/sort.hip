// sort.hip -- Morton-pair radix sort (rocPRIM's onesweep radix sort).
#include "sort.hpp"

#include <rocprim/device/device_radix_sort.hpp>

namespace tmnn_hip {

hipError_t morton_sort_temp_bytes(int n, size_t *bytes) {
  size_t b = 0;
  hipError_t e = rocprim::radix_sort_pairs(nullptr, b, static_cast<const uint32_t *>(nullptr),
                                           static_cast<uint32_t *>(nullptr),
                                           static_cast<const uint32_t *>(nullptr),
                                           static_cast<uint32_t *>(nullptr),
                                           static_cast<size_t>(n), 0u, 32u);
  *bytes = b;
  return e;
}

hipError_t morton_sort_pairs(void *tmp, size_t &tmp_bytes, const uint32_t *keys_in,
                             uint32_t *keys_out, const uint32_t *vals_in,
                             uint32_t *vals_out, int n, int end_bit, hipStream_t stream) {
  return rocprim::radix_sort_pairs(tmp, tmp_bytes, keys_in, keys_out, vals_in, vals_out,
                                   static_cast<size_t>(n), 0u,
                                   static_cast<unsigned int>(end_bit), stream);
}

}  // namespace tmnn_hip
