// sort.hip -- stable LSD radix sort of the batch by Morton code on the
// trainer's stream, replacing the reference's per-step host std::sort
// (src/tiny_metal_nn/runtime/morton_sort.h:60-110).
//
// RB-bit digits (10 for 2D's 20-bit codes: 2 passes; 8 for 3D's 30-bit and
// 4D's 32-bit codes: 4 passes), three kernels per pass:
//   hist   -- each block counts the digits of its 2048-key chunk (LDS atomics)
//             into hist[digit][block]; the first pass computes the Morton
//             codes from the positions itself;
//   scan   -- one block per digit: exclusive prefix of the digit's counts over
//             the blocks, and the digit total;
//   scatter-- each block ranks its chunk stably: every wave ranks a
//             contiguous quarter of it against its own LDS counters (wave
//             ballots for the rank among equal digits, rounds in input
//             order), then a per-digit prefix over the waves; it sorts the
//             chunk locally in LDS and writes it out digit run by digit run,
//             so consecutive lanes store consecutive addresses.
// Ties keep input order (stable), so the sorted order is deterministic.
#include "sort.hpp"

#include <algorithm>

#include "device_common.hpp"

namespace tmnn_hip {
namespace {

constexpr int kSortThreads = 256;
constexpr int kKeysPerThread = 8;
constexpr int kChunk = kSortThreads * kKeysPerThread;  // keys per block
constexpr int kWaveKeys = 64 * kKeysPerThread;         // keys per wave in the scatter
constexpr int kSortWaves = kSortThreads / 64;

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

// key of chunk-local element li: the Morton code of the position (first
// pass) or the previous pass's output
template <bool FIRST>
__device__ __forceinline__ uint32_t load_key(const uint32_t *keys, const float *pos, int dims,
                                             size_t i) {
  if constexpr (FIRST) return morton_code(pos + i * dims, dims);
  return keys[i];
}

template <int RB, bool FIRST>
__global__ void __launch_bounds__(kSortThreads)
    radix_hist_kernel(const uint32_t *keys, const float *pos, int dims, int n, int shift,
                      int blocks, uint32_t *hist) {
  constexpr int kBins = 1 << RB, BPT = kBins / kSortThreads;
  __shared__ uint32_t cnt[kBins];
  const int t = threadIdx.x;
#pragma unroll
  for (int j = 0; j < BPT; ++j) cnt[t + kSortThreads * j] = 0u;
  __syncthreads();
  const int base = blockIdx.x * kChunk;
#pragma unroll
  for (int r = 0; r < kKeysPerThread; ++r) {
    const int i = base + r * kSortThreads + t;
    if (i < n) {
      const uint32_t key = load_key<FIRST>(keys, pos, dims, static_cast<size_t>(i));
      atomicAdd(&cnt[(key >> shift) & (kBins - 1)], 1u);
    }
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < BPT; ++j) {
    const int d = t + kSortThreads * j;
    hist[static_cast<size_t>(d) * blocks + blockIdx.x] = cnt[d];
  }
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

template <int RB, bool FIRST>
__global__ void __launch_bounds__(kSortThreads)
    radix_scatter_kernel(const uint32_t *keys_in, const uint32_t *vals_in, const float *pos,
                         int dims, int n, int shift, int blocks, const uint32_t * /*hist*/,
                         const uint32_t *pre, const uint32_t *totals, uint32_t *keys_out,
                         uint32_t *vals_out) {
  constexpr int kBins = 1 << RB, BPT = kBins / kSortThreads;
  __shared__ uint32_t s_keys[kChunk];
  __shared__ uint32_t s_vals[kChunk];
  __shared__ uint16_t wcnt[kSortWaves][kBins];  // per-wave counts, then offsets (< kChunk)
  __shared__ uint32_t lstart[kBins];            // start of the digit run within the chunk
  __shared__ uint32_t glob[kBins];              // global slot of chunk index 0 of the run
  __shared__ uint32_t wsum[kSortWaves];
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int base = blockIdx.x * kChunk;
  const int nblk = std::min(kChunk, n - base);
  for (int i = t; i < kSortWaves * kBins / 2; i += kSortThreads)
    reinterpret_cast<uint32_t *>(&wcnt[0][0])[i] = 0u;
  __syncthreads();

  // wave w ranks chunk keys [w * kWaveKeys, (w + 1) * kWaveKeys), 64 per
  // round in input order, against its own counters (no barriers): piw = keys
  // of the same digit before it in the wave. All loads are issued first.
  uint32_t key[kKeysPerThread], val[kKeysPerThread], piw[kKeysPerThread];
#pragma unroll
  for (int r = 0; r < kKeysPerThread; ++r) {
    const int li = wave * kWaveKeys + r * 64 + lane;
    const bool valid = li < nblk;
    const size_t gi = static_cast<size_t>(base + (valid ? li : 0));
    if constexpr (FIRST) {
      key[r] = valid ? load_key<true>(nullptr, pos, dims, gi) : 0u;
      val[r] = static_cast<uint32_t>(gi);
    } else {
      key[r] = valid ? keys_in[gi] : 0u;
      val[r] = valid ? vals_in[gi] : 0u;
    }
  }
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
#pragma unroll
  for (int r = 0; r < kKeysPerThread; ++r) {
    const bool valid = wave * kWaveKeys + r * 64 + lane < nblk;
    const uint32_t d = (key[r] >> shift) & (kBins - 1);
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int b = 0; b < RB; ++b) {
      const bool bit = (d >> b) & 1u;
      const uint64_t m = __ballot(bit);
      peers &= bit ? m : ~m;
    }
    const uint32_t rank = static_cast<uint32_t>(__popcll(peers & lt_mask));
    // every lane reads the wave's running count before the leader advances
    // it (the LDS operations of one wave complete in program order)
    const uint32_t c = valid ? wcnt[wave][d] : 0u;
    piw[r] = c + rank;
    if (valid && rank == 0u) wcnt[wave][d] = static_cast<uint16_t>(c + __popcll(peers));
  }
  __syncthreads();

  // thread t owns digits [t*BPT, (t+1)*BPT): offsets across waves, the
  // chunk's count, the run's start in the chunk and its global slot
  // (exclusive scan of the digit totals plus this block's prefix in the digit)
  uint32_t cnt[BPT], tot[BPT], sc = 0, st = 0;
#pragma unroll
  for (int j = 0; j < BPT; ++j) {
    const int dd = t * BPT + j;
    uint32_t acc = 0;
#pragma unroll
    for (int w = 0; w < kSortWaves; ++w) {
      const uint32_t c = wcnt[w][dd];
      wcnt[w][dd] = static_cast<uint16_t>(acc);
      acc += c;
    }
    cnt[j] = acc;
    tot[j] = totals[dd];
    sc += acc;
    st += tot[j];
  }
  uint32_t all = 0;
  uint32_t lb = block_excl_scan(sc, wsum, &all);
  uint32_t gb = block_excl_scan(st, wsum, &all);
#pragma unroll
  for (int j = 0; j < BPT; ++j) {
    const int dd = t * BPT + j;
    lstart[dd] = lb;
    glob[dd] = gb + pre[static_cast<size_t>(dd) * blocks + blockIdx.x] - lb;  // modulo 2^32
    lb += cnt[j];
    gb += tot[j];
  }
  __syncthreads();

  // sort the chunk in LDS (input order within each digit)
#pragma unroll
  for (int r = 0; r < kKeysPerThread; ++r) {
    if (wave * kWaveKeys + r * 64 + lane < nblk) {
      const uint32_t d = (key[r] >> shift) & (kBins - 1);
      const uint32_t p = lstart[d] + wcnt[wave][d] + piw[r];
      s_keys[p] = key[r];
      s_vals[p] = val[r];
    }
  }
  __syncthreads();

  // consecutive threads write consecutive slots of a digit run
  for (int j = t; j < nblk; j += kSortThreads) {
    const uint32_t k = s_keys[j];
    const uint32_t dst = glob[(k >> shift) & (kBins - 1)] + static_cast<uint32_t>(j);
    keys_out[dst] = k;
    vals_out[dst] = s_vals[j];
  }
}

int sort_blocks(int n) { return (n + kChunk - 1) / kChunk; }

// digit width per code width: two 10-bit passes for 2D's 20-bit codes; 8-bit
// digits (4 passes) for 3D/4D, where wider digits measured slower per pass
// than the pass they save
int digit_bits(int end_bit) { return end_bit == 20 ? 10 : 8; }

template <int RB>
hipError_t run_passes(uint32_t *hist, uint32_t *pre, uint32_t *totals, const float *pos,
                      int dims, uint32_t *keys0, uint32_t *keys1, uint32_t *vals0,
                      uint32_t *vals1, int n, int end_bit, hipStream_t stream,
                      const uint32_t **keys_sorted, const uint32_t **vals_sorted) {
  const int blocks = sort_blocks(n);
  uint32_t *kin = keys0, *kout = keys1, *vin = nullptr, *vout = vals1;
  uint32_t *vspare = vals0;
  const int passes = std::max(1, (end_bit + RB - 1) / RB);
  for (int pass = 0; pass < passes; ++pass) {
    const int shift = RB * pass;
    if (pass == 0) {
      hipLaunchKernelGGL((radix_hist_kernel<RB, true>), dim3(blocks), dim3(kSortThreads), 0, stream,
                         nullptr, pos, dims, n, shift, blocks, hist);
    } else {
      hipLaunchKernelGGL((radix_hist_kernel<RB, false>), dim3(blocks), dim3(kSortThreads), 0,
                         stream, kin, nullptr, dims, n, shift, blocks, hist);
    }
    hipLaunchKernelGGL(radix_scan_kernel, dim3(1 << RB), dim3(kSortThreads), 0, stream, hist,
                       blocks, pre, totals);
    if (pass == 0) {
      hipLaunchKernelGGL((radix_scatter_kernel<RB, true>), dim3(blocks), dim3(kSortThreads), 0,
                         stream, nullptr, nullptr, pos, dims, n, shift, blocks, hist, pre, totals,
                         kout, vout);
    } else {
      hipLaunchKernelGGL((radix_scatter_kernel<RB, false>), dim3(blocks), dim3(kSortThreads), 0,
                         stream, kin, vin, nullptr, dims, n, shift, blocks, hist, pre, totals,
                         kout, vout);
    }
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

}  // namespace

hipError_t morton_sort_temp_bytes(int n, size_t *bytes) {
  // hist[kBins][G] + pre[kBins][G] + totals[kBins] at the widest digit
  const size_t bins = size_t(1) << 10;
  *bytes = (2 * bins * std::max(1, sort_blocks(n)) + bins) * sizeof(uint32_t);
  return hipSuccess;
}

hipError_t morton_sort_batch(void *tmp, size_t tmp_bytes, const float *pos, int dims,
                             uint32_t *keys0, uint32_t *keys1, uint32_t *vals0, uint32_t *vals1,
                             int n, hipStream_t stream, const uint32_t **keys_sorted,
                             const uint32_t **vals_sorted) {
  size_t need = 0;
  morton_sort_temp_bytes(n, &need);
  if (n <= 0 || tmp_bytes < need || dims < 2 || dims > 4) return hipErrorInvalidValue;
  // 2D codes interleave x and y only (the lifted z = 0 bits are all zero,
  // which leaves the order unchanged): 20 bits; 3D 30 bits; 4D 32 bits.
  const int end_bit = dims == 2 ? 20 : (dims == 3 ? 30 : 32);
  const int blocks = sort_blocks(n);
  const size_t bins = size_t(1) << digit_bits(end_bit);
  uint32_t *hist = static_cast<uint32_t *>(tmp);
  uint32_t *pre = hist + bins * blocks;
  uint32_t *totals = pre + bins * blocks;
  if (digit_bits(end_bit) == 8)
    return run_passes<8>(hist, pre, totals, pos, dims, keys0, keys1, vals0, vals1, n, end_bit,
                         stream, keys_sorted, vals_sorted);
  return run_passes<10>(hist, pre, totals, pos, dims, keys0, keys1, vals0, vals1, n, end_bit,
                        stream, keys_sorted, vals_sorted);
}

}  // namespace tmnn_hip
