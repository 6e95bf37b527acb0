// sort.hip -- stable LSD radix sort of (Morton code, point index) pairs on the
// trainer's stream, replacing the reference's per-step host std::sort
// (src/tiny_metal_nn/runtime/morton_sort.h:60-110).
//
// 8-bit digits, ceil(end_bit / 8) passes, three kernels per pass:
//   hist   -- each block counts the digits of its 1024-key chunk (LDS atomics)
//             into hist[digit][block];
//   scan   -- one block per digit: exclusive prefix of the digit's counts over
//             the blocks, and the digit total;
//   scatter-- each block ranks its chunk stably (wave ballots for the rank
//             among equal digits, wave order and round order for the rest),
//             sorts it locally in LDS and writes it out digit run by digit
//             run, so consecutive lanes store consecutive addresses.
// Ties keep input order (stable), so the sorted order is deterministic.
#include "sort.hpp"

#include <algorithm>

namespace tmnn_hip {
namespace {

constexpr int kBins = 256;
constexpr int kSortThreads = 256;
constexpr int kKeysPerThread = 4;
constexpr int kChunk = kSortThreads * kKeysPerThread;  // keys per block
constexpr int kSortWaves = kSortThreads / 64;

__device__ __forceinline__ uint32_t digit_of(uint32_t key, int shift) {
  return (key >> shift) & (kBins - 1);
}

__global__ void __launch_bounds__(kSortThreads)
    radix_hist_kernel(const uint32_t *keys, int n, int shift, int blocks, uint32_t *hist) {
  __shared__ uint32_t cnt[kBins];
  cnt[threadIdx.x] = 0u;
  __syncthreads();
  const int base = blockIdx.x * kChunk;
#pragma unroll 4
  for (int r = 0; r < kKeysPerThread; ++r) {
    const int i = base + r * kSortThreads + static_cast<int>(threadIdx.x);
    if (i < n) atomicAdd(&cnt[digit_of(keys[i], shift)], 1u);
  }
  __syncthreads();
  hist[threadIdx.x * blocks + blockIdx.x] = cnt[threadIdx.x];
}

// Inclusive scan of v over the 64 lanes of a wave.
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v, int lane) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t u = __shfl_up(v, off);
    if (lane >= off) v += u;
  }
  return v;
}

// Exclusive scan over the kSortThreads threads of a block; *total gets the sum.
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t *wsum,
                                                    uint32_t *total) {
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const uint32_t inc = wave_incl_scan(v, lane);
  if (lane == 63) wsum[w] = inc;
  __syncthreads();
  uint32_t before = 0, all = 0;
#pragma unroll
  for (int k = 0; k < kSortWaves; ++k) {
    const uint32_t c = wsum[k];
    before += k < w ? c : 0u;
    all += c;
  }
  __syncthreads();
  *total = all;
  return before + inc - v;
}

// Row d of hist (the G per-block counts of digit d, contiguous): exclusive
// prefix over blocks into pre[d][*], the digit's total into totals[d].
// One block per digit; thread t owns blocks [t*k, (t+1)*k).
__global__ void __launch_bounds__(kSortThreads)
    radix_scan_kernel(const uint32_t *hist, int blocks, uint32_t *pre, uint32_t *totals) {
  __shared__ uint32_t wsum[kSortWaves];
  const int d = blockIdx.x;
  const int t = threadIdx.x;
  const int k = (blocks + kSortThreads - 1) / kSortThreads;
  const uint32_t *row = hist + static_cast<size_t>(d) * blocks;
  uint32_t *out = pre + static_cast<size_t>(d) * blocks;
  const int lo = t * k;
  uint32_t s = 0;
  for (int i = 0; i < k; ++i)
    if (lo + i < blocks) s += row[lo + i];
  uint32_t total = 0;
  uint32_t run = block_excl_scan(s, wsum, &total);
  for (int i = 0; i < k; ++i)
    if (lo + i < blocks) {
      const uint32_t c = row[lo + i];
      out[lo + i] = run;
      run += c;
    }
  if (t == 0) totals[d] = total;
}

__global__ void __launch_bounds__(kSortThreads)
    radix_scatter_kernel(const uint32_t *keys_in, const uint32_t *vals_in, int n, int shift,
                         int blocks, const uint32_t *hist, const uint32_t *pre,
                         const uint32_t *totals, uint32_t *keys_out, uint32_t *vals_out) {
  __shared__ uint32_t s_keys[kChunk];
  __shared__ uint32_t s_vals[kChunk];
  __shared__ uint32_t glob[kBins];     // global start of this block's digit run
  __shared__ uint32_t local[kBins];    // start of the digit run within the chunk
  __shared__ uint32_t running[kBins];  // keys of each digit placed so far
  __shared__ uint32_t wcnt[kSortWaves][kBins];
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int base = blockIdx.x * kChunk;
  const int nblk = std::min(kChunk, n - base);

  __shared__ uint32_t wsum[kSortWaves];
  // global start of each digit (exclusive scan of the digit totals) plus this
  // block's prefix within the digit; chunk-local starts from its own counts
  {
    uint32_t all = 0;
    const uint32_t digit_base = block_excl_scan(totals[t], wsum, &all);
    glob[t] = digit_base + pre[t * blocks + blockIdx.x];
    const uint32_t count = hist[t * blocks + blockIdx.x];
    local[t] = block_excl_scan(count, wsum, &all);
    running[t] = 0u;
  }
  __syncthreads();

  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int r = 0; r < kKeysPerThread; ++r) {
    const int li = r * kSortThreads + t;  // chunk-local index (input order)
    const bool valid = li < nblk;
    const uint32_t key = valid ? keys_in[base + li] : 0u;
    const uint32_t val = valid ? (vals_in ? vals_in[base + li] : static_cast<uint32_t>(base + li))
                               : 0u;
    const uint32_t d = digit_of(key, shift);
    // lanes of this wave holding the same digit
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const bool bit = (d >> b) & 1u;
      const uint64_t m = __ballot(bit);
      peers &= bit ? m : ~m;
    }
    const uint32_t rank = static_cast<uint32_t>(__popcll(peers & lt_mask));
    const bool leader = valid && rank == 0u;
#pragma unroll
    for (int w = 0; w < kSortWaves; ++w) wcnt[w][t] = 0u;
    __syncthreads();
    if (leader) wcnt[wave][d] = static_cast<uint32_t>(__popcll(peers));
    __syncthreads();
    // per digit t: exclusive offsets across waves, then advance the run
    {
      uint32_t acc = running[t];
#pragma unroll
      for (int w = 0; w < kSortWaves; ++w) {
        const uint32_t c = wcnt[w][t];
        wcnt[w][t] = acc;
        acc += c;
      }
      running[t] = acc;
    }
    __syncthreads();
    if (valid) {
      const uint32_t pos = local[d] + wcnt[wave][d] + rank;
      s_keys[pos] = key;
      s_vals[pos] = val;
    }
    __syncthreads();
  }

  // write the locally sorted chunk: position j belongs to the digit run of
  // s_keys[j]; its global slot is glob[d] + (j - local[d]).
  for (int j = t; j < nblk; j += kSortThreads) {
    const uint32_t key = s_keys[j];
    const uint32_t d = digit_of(key, shift);
    const uint32_t dst = glob[d] + (static_cast<uint32_t>(j) - local[d]);
    keys_out[dst] = key;
    vals_out[dst] = s_vals[j];
  }
}

int sort_blocks(int n) { return (n + kChunk - 1) / kChunk; }

}  // namespace

hipError_t morton_sort_temp_bytes(int n, size_t *bytes) {
  // hist[kBins][G] + pre[kBins][G] + totals[kBins]
  *bytes = (2 * static_cast<size_t>(kBins) * std::max(1, sort_blocks(n)) + kBins) *
           sizeof(uint32_t);
  return hipSuccess;
}

hipError_t morton_sort_pairs(void *tmp, size_t tmp_bytes, uint32_t *keys0, uint32_t *keys1,
                             uint32_t *vals0, uint32_t *vals1, int n, int end_bit,
                             hipStream_t stream, const uint32_t **keys_sorted,
                             const uint32_t **vals_sorted) {
  const int blocks = sort_blocks(n);
  size_t need = 0;
  morton_sort_temp_bytes(n, &need);
  if (n <= 0 || tmp_bytes < need) return hipErrorInvalidValue;
  uint32_t *hist = static_cast<uint32_t *>(tmp);
  uint32_t *pre = hist + static_cast<size_t>(kBins) * blocks;
  uint32_t *totals = pre + static_cast<size_t>(kBins) * blocks;
  uint32_t *kin = keys0, *kout = keys1, *vin = nullptr, *vout = vals1;
  uint32_t *vspare = vals0;
  const int passes = std::max(1, (end_bit + 7) / 8);
  for (int pass = 0; pass < passes; ++pass) {
    const int shift = 8 * pass;
    hipLaunchKernelGGL(radix_hist_kernel, dim3(blocks), dim3(kSortThreads), 0, stream, kin, n,
                       shift, blocks, hist);
    hipLaunchKernelGGL(radix_scan_kernel, dim3(kBins), dim3(kSortThreads), 0, stream, hist,
                       blocks, pre, totals);
    hipLaunchKernelGGL(radix_scatter_kernel, dim3(blocks), dim3(kSortThreads), 0, stream, kin,
                       vin, n, shift, blocks, hist, pre, totals, kout, vout);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // next pass reads what this one wrote
    std::swap(kin, kout);
    uint32_t *written = vout;
    vout = (pass == 0) ? vspare : vin;
    vin = written;
  }
  *keys_sorted = kin;
  *vals_sorted = vin;
  return hipSuccess;
}

}  // namespace tmnn_hip
