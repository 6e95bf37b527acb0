// sort.hip -- stable radix sort of the batch by Morton code on the trainer's
// stream, replacing the reference's per-step host std::sort
// (src/tiny_metal_nn/runtime/morton_sort.h:60-110).
//
// 3D's 30-bit and 4D's 32-bit codes: LSD with 8-bit digits (4 passes). 2D's
// 20-bit codes: one MSD pass on the top 10 bits, then bucket_sort_kernel
// sorts each of the 1024 buckets by the low 10 bits in one block (one launch
// instead of a second three-kernel pass). Three kernels per radix pass:
//   hist   -- each block counts the digits of its chunk (256 x KPT keys: 2048
//             for 3D/4D, 1536 for 2D) with LDS atomics into its row
//             hist[block][digit] (one coalesced row store); the
//             first pass computes the Morton codes from the positions itself;
//   scan   -- 16 digits per block, 16 threads per digit, each over a
//             contiguous run of blocks: exclusive prefix of every digit's
//             counts over the blocks (pre[block][digit]), and the totals;
//   scatter-- each block ranks its chunk stably: every wave ranks a
//             contiguous quarter of it against its own LDS counters (wave
//             ballots for the rank among equal digits, rounds in input
//             order), then a per-digit prefix over the waves; it sorts the
//             chunk locally in LDS and writes it out digit run by digit run,
//             so consecutive lanes store consecutive addresses; the 2D MSD
//             pass also writes each digit's output start for the buckets.
// Ties keep input order (stable), so the sorted order is deterministic.
#include "sort.hpp"

#include <algorithm>
#include <type_traits>

#include "device_common.hpp"

namespace tmnn_hip {
namespace {

constexpr int kSortThreads = 256;
// keys per thread (a chunk = 256 x KPT keys per block): 8 for the 3D/4D LSD
// passes; 6 for 2D, whose 2^18-point batches gain from more, smaller chunks
constexpr int kKeysPerThread = 8;
constexpr int kKeysPerThread2D = 6;
constexpr int chunk_keys(int kpt) { return kSortThreads * kpt; }
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

// The keys of a thread's KPT elements at global indices gi[r] (each a valid
// index): the Morton codes of the positions (first pass) or the previous
// pass's output. Every load is issued before the first code is formed (the
// uniform branch on dims sits outside the loads), so a thread waits for its
// KPT loads once instead of once per key.
template <bool FIRST, int KPT>
__device__ __forceinline__ void load_keys(const uint32_t *keys, const float *pos, int dims,
                                          const size_t (&gi)[KPT], uint32_t (&key)[KPT]) {
  if constexpr (FIRST) {
    auto codes = [&](auto dc) __attribute__((always_inline)) {
      constexpr int D = decltype(dc)::value;
      float p[KPT][D];
#pragma unroll
      for (int r = 0; r < KPT; ++r)
#pragma unroll
        for (int k = 0; k < D; ++k) p[r][k] = pos[gi[r] * D + k];
#pragma unroll
      for (int r = 0; r < KPT; ++r) key[r] = morton_code_of<D>(p[r]);
    };
    if (dims == 4)
      codes(std::integral_constant<int, 4>{});
    else if (dims == 3)
      codes(std::integral_constant<int, 3>{});
    else
      codes(std::integral_constant<int, 2>{});
  } else {
#pragma unroll
    for (int r = 0; r < KPT; ++r) key[r] = keys[gi[r]];
  }
}

template <int RB, bool FIRST, int KPT>
__global__ void __launch_bounds__(kSortThreads)
    radix_hist_kernel(const uint32_t *keys, const float *pos, int dims, int n, int shift,
                      int blocks, uint32_t *hist) {
  constexpr int kBins = 1 << RB, BPT = kBins / kSortThreads;
  __shared__ uint32_t cnt[kBins];
  const int t = threadIdx.x;
  const int base = blockIdx.x * chunk_keys(KPT);
  size_t gi[KPT];
  bool ok[KPT];
#pragma unroll
  for (int r = 0; r < KPT; ++r) {
    const int i = base + r * kSortThreads + t;
    ok[r] = i < n;
    gi[r] = static_cast<size_t>(ok[r] ? i : 0);
  }
  // the keys are loaded (and coded) while the counters are cleared
  uint32_t key[KPT];
  load_keys<FIRST, KPT>(keys, pos, dims, gi, key);
#pragma unroll
  for (int j = 0; j < BPT; ++j) cnt[t + kSortThreads * j] = 0u;
  __syncthreads();
#pragma unroll
  for (int r = 0; r < KPT; ++r)
    if (ok[r]) atomicAdd(&cnt[(key[r] >> shift) & (kBins - 1)], 1u);
  __syncthreads();
#pragma unroll
  for (int j = 0; j < BPT; ++j) {
    const int d = t + kSortThreads * j;
    hist[static_cast<size_t>(blockIdx.x) * kBins + d] = cnt[d];
  }
}

// Column d of hist (the G per-block counts of digit d, row stride bins):
// exclusive prefix over the blocks into pre[*][d], the digit's total into
// totals[d]. Block x takes digits 16 x .. 16 x + 15; thread t takes digit
// 16 x + t % 16 and the blocks of segment t / 16, a contiguous sixteenth of
// them: it sums its segment (16 loads in flight at a time, from clamped
// addresses), the sixteen segment sums of its digit are scanned through
// LDS, then it writes its segment's prefixes (a segment of at most 16
// blocks, e.g. 2D at 2^18 points, from the registers of the first pass).
constexpr int kScanDigits = 16, kScanSegs = kSortThreads / kScanDigits, kScanChunk = 16;
__global__ void __launch_bounds__(kSortThreads)
    radix_scan_kernel(const uint32_t *__restrict__ hist, int blocks, int bins,
                      uint32_t *__restrict__ pre, uint32_t *__restrict__ totals) {
  __shared__ uint32_t seg[kScanSegs][kScanDigits];
  const int t = threadIdx.x;
  const int dl = t % kScanDigits, sg = t / kScanDigits;
  const int d = blockIdx.x * kScanDigits + dl;
  const int k = (blocks + kScanSegs - 1) / kScanSegs;
  const int lo = sg * k, hi = std::min(blocks, lo + k);
  uint32_t v[kScanChunk];
  auto load_chunk = [&](int c0) {
#pragma unroll
    for (int j = 0; j < kScanChunk; ++j) {
      const int b = c0 + j;
      const uint32_t c = hist[static_cast<size_t>(std::min(b, hi - 1)) * bins + d];
      v[j] = b < hi ? c : 0u;
    }
  };
  uint32_t s = 0;
  for (int c0 = lo; c0 < hi; c0 += kScanChunk) {
    load_chunk(c0);
#pragma unroll
    for (int j = 0; j < kScanChunk; ++j) s += v[j];
  }
  seg[sg][dl] = s;
  __syncthreads();
  uint32_t run = 0, total = 0;
#pragma unroll
  for (int j = 0; j < kScanSegs; ++j) {
    const uint32_t c = seg[j][dl];
    run += j < sg ? c : 0u;
    total += c;
  }
  const bool one_chunk = hi - lo <= kScanChunk;  // v still holds the segment
  for (int c0 = lo; c0 < hi; c0 += kScanChunk) {
    if (!one_chunk) load_chunk(c0);
#pragma unroll
    for (int j = 0; j < kScanChunk; ++j) {
      const int b = c0 + j;
      if (b < hi) pre[static_cast<size_t>(b) * bins + d] = run;
      run += v[j];
    }
  }
  if (sg == 0) totals[d] = total;
}

// LDS of one chunk's stable ranking (radix_scatter_kernel, bucket_sort_kernel).
template <int RB, int KPT>
struct ChunkLds {
  uint32_t keys[chunk_keys(KPT)];
  uint32_t vals[chunk_keys(KPT)];
  uint16_t wcnt[kSortWaves][1 << RB];  // per-wave counts, then offsets (< the chunk)
  uint32_t lstart[1 << RB];            // start of the digit run within the chunk
  uint32_t glob[1 << RB];              // output slot of chunk index 0 of the run
  uint32_t wsum[kSortWaves];
};

// Chunk element of key slot r of this thread: wave w holds the contiguous
// chunk elements [w * 64 KPT, (w + 1) * 64 KPT), 64 per slot.
template <int KPT>
__device__ __forceinline__ int chunk_index(int r) {
  return (threadIdx.x >> 6) * (64 * KPT) + r * 64 + (threadIdx.x & 63);
}

// Clears the per-wave digit counters (the caller's barrier publishes it).
template <int RB, int KPT>
__device__ __forceinline__ void clear_counts(ChunkLds<RB, KPT> &L) {
  for (int i = threadIdx.x; i < kSortWaves * (1 << RB) / 2; i += kSortThreads)
    reinterpret_cast<uint32_t *>(&L.wcnt[0][0])[i] = 0u;
}

// Every wave ranks its keys, 64 per round in input order, against its own
// counters (no barriers): piw = keys of the same digit before it in the wave.
template <int RB, int KPT>
__device__ __forceinline__ void rank_in_waves(ChunkLds<RB, KPT> &L, const uint32_t (&key)[KPT],
                                              int nblk, int shift, uint32_t (&piw)[KPT]) {
  constexpr int kBins = 1 << RB;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
#pragma unroll
  for (int r = 0; r < KPT; ++r) {
    const bool valid = chunk_index<KPT>(r) < nblk;
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
    const uint32_t c = valid ? L.wcnt[wave][d] : 0u;
    piw[r] = c + rank;
    if (valid && rank == 0u) L.wcnt[wave][d] = static_cast<uint16_t>(c + __popcll(peers));
  }
}

// After the ranking's barrier: thread t owns digits [t*BPT, (t+1)*BPT); turns
// their per-wave counts into offsets across the waves and returns the
// chunk's count of each in cnt.
template <int RB, int KPT>
__device__ __forceinline__ void wave_offsets(ChunkLds<RB, KPT> &L,
                                             uint32_t (&cnt)[(1 << RB) / kSortThreads]) {
  constexpr int BPT = (1 << RB) / kSortThreads;
#pragma unroll
  for (int j = 0; j < BPT; ++j) {
    const int dd = threadIdx.x * BPT + j;
    uint32_t acc = 0;
#pragma unroll
    for (int w = 0; w < kSortWaves; ++w) {
      const uint32_t c = L.wcnt[w][dd];
      L.wcnt[w][dd] = static_cast<uint16_t>(acc);
      acc += c;
    }
    cnt[j] = acc;
  }
}

// Sorts the chunk into L.keys / L.vals by digit, input order within a digit
// (after the barrier that published lstart and the wave offsets).
template <int RB, int KPT>
__device__ __forceinline__ void place_chunk(ChunkLds<RB, KPT> &L, const uint32_t (&key)[KPT],
                                            const uint32_t (&val)[KPT], const uint32_t (&piw)[KPT],
                                            int nblk, int shift) {
  constexpr int kBins = 1 << RB;
  const int wave = threadIdx.x >> 6;
#pragma unroll
  for (int r = 0; r < KPT; ++r) {
    if (chunk_index<KPT>(r) < nblk) {
      const uint32_t d = (key[r] >> shift) & (kBins - 1);
      const uint32_t p = L.lstart[d] + L.wcnt[wave][d] + piw[r];
      L.keys[p] = key[r];
      L.vals[p] = val[r];
    }
  }
}

// Writes the sorted chunk out (after the barrier that follows place_chunk):
// consecutive threads write consecutive slots of a digit run.
template <int RB, int KPT>
__device__ __forceinline__ void write_chunk(const ChunkLds<RB, KPT> &L, int nblk, int shift,
                                            uint32_t *keys_out, uint32_t *vals_out) {
  constexpr int kBins = 1 << RB;
  for (int j = threadIdx.x; j < nblk; j += kSortThreads) {
    const uint32_t k = L.keys[j];
    const uint32_t dst = L.glob[(k >> shift) & (kBins - 1)] + static_cast<uint32_t>(j);
    keys_out[dst] = k;
    vals_out[dst] = L.vals[j];
  }
}

template <int RB, bool FIRST, int KPT>
__global__ void __launch_bounds__(kSortThreads)
    radix_scatter_kernel(const uint32_t *keys_in, const uint32_t *vals_in, const float *pos,
                         int dims, int n, int shift, int blocks, uint32_t *starts,
                         const uint32_t *pre, const uint32_t *totals, uint32_t *keys_out,
                         uint32_t *vals_out) {
  constexpr int BPT = (1 << RB) / kSortThreads;
  __shared__ ChunkLds<RB, KPT> L;
  const int t = threadIdx.x;
  const int base = blockIdx.x * chunk_keys(KPT);
  const int nblk = std::min(chunk_keys(KPT), n - base);
  // all loads are issued before the ranking: the owned digits' totals and
  // this block's prefixes first (they do not depend on the keys)
  uint32_t tot[BPT], pv[BPT];
#pragma unroll
  for (int j = 0; j < BPT; ++j) {
    tot[j] = totals[t * BPT + j];
    pv[j] = pre[static_cast<size_t>(blockIdx.x) * (1 << RB) + t * BPT + j];
  }
  clear_counts(L);
  __syncthreads();

  uint32_t key[KPT], val[KPT], piw[KPT];
  size_t gi[KPT];
#pragma unroll
  for (int r = 0; r < KPT; ++r) {
    const int li = chunk_index<KPT>(r);
    gi[r] = static_cast<size_t>(base + (li < nblk ? li : 0));
  }
  load_keys<FIRST, KPT>(keys_in, pos, dims, gi, key);
#pragma unroll
  for (int r = 0; r < KPT; ++r) {
    const bool valid = chunk_index<KPT>(r) < nblk;
    if constexpr (FIRST) {
      val[r] = static_cast<uint32_t>(gi[r]);
    } else {
      const uint32_t v = vals_in[gi[r]];
      val[r] = valid ? v : 0u;
    }
    key[r] = valid ? key[r] : 0u;
  }
  rank_in_waves(L, key, nblk, shift, piw);
  __syncthreads();

  // the chunk's count of each owned digit, the run's start in the chunk and
  // its global slot (exclusive scan of the digit totals plus this block's
  // prefix in the digit)
  uint32_t cnt[BPT], sc = 0, st = 0;
  wave_offsets(L, cnt);
#pragma unroll
  for (int j = 0; j < BPT; ++j) {
    sc += cnt[j];
    st += tot[j];
  }
  uint32_t all = 0;
  uint32_t lb = block_excl_scan(sc, L.wsum, &all);
  uint32_t gb = block_excl_scan(st, L.wsum, &all);
#pragma unroll
  for (int j = 0; j < BPT; ++j) {
    const int dd = t * BPT + j;
    L.lstart[dd] = lb;
    L.glob[dd] = gb + pv[j] - lb;  // modulo 2^32
    // the digits' output starts, for a following bucket pass (nullable)
    if (starts != nullptr && blockIdx.x == 0) starts[dd] = gb;
    lb += cnt[j];
    gb += tot[j];
  }
  __syncthreads();
  place_chunk(L, key, val, piw, nblk, shift);
  __syncthreads();
  write_chunk(L, nblk, shift, keys_out, vals_out);
}

// Second pass of the 2D sort, after an MSD pass on the top RB bits: block b
// sorts bucket b (the keys whose top digit is b, contiguous and in input
// order) stably by the low RB bits, in place of a full LSD pass. A bucket
// that fits one chunk is ranked and written at once; a larger one takes a
// digit histogram of the whole bucket, then its chunks in order, each
// written at the running offsets of its digits (stable across chunks).
template <int RB, int KPT>
__global__ void __launch_bounds__(kSortThreads)
    bucket_sort_kernel(const uint32_t *keys_in, const uint32_t *vals_in, const uint32_t *starts,
                       const uint32_t *totals, uint32_t *keys_out, uint32_t *vals_out) {
  constexpr int kBins = 1 << RB, BPT = kBins / kSortThreads;
  constexpr int kChunk = chunk_keys(KPT);
  __shared__ ChunkLds<RB, KPT> L;
  __shared__ uint32_t offs[kBins];  // running output offset of each digit in the bucket
  const int t = threadIdx.x;
  const int b = blockIdx.x;
  const uint32_t start = starts[b];  // written by the MSD pass's scatter
  const int size = static_cast<int>(totals[b]);
  if (size == 0) return;  // uniform
  const bool one_chunk = size <= kChunk;
  if (!one_chunk) {
    // digit histogram of the whole bucket, then its exclusive scan
    for (int i = t; i < kBins; i += kSortThreads) offs[i] = 0u;
    __syncthreads();
    for (int i = t; i < size; i += kSortThreads)
      atomicAdd(&offs[keys_in[start + i] & (kBins - 1)], 1u);
    __syncthreads();
    uint32_t c[BPT], sum = 0;
#pragma unroll
    for (int j = 0; j < BPT; ++j) {
      c[j] = offs[t * BPT + j];
      sum += c[j];
    }
    uint32_t all = 0;
    uint32_t run = block_excl_scan(sum, L.wsum, &all);
#pragma unroll
    for (int j = 0; j < BPT; ++j) {
      offs[t * BPT + j] = run;
      run += c[j];
    }
  }
  for (int base = 0; base < size; base += kChunk) {
    const int nblk = std::min(kChunk, size - base);
    clear_counts(L);
    __syncthreads();
    uint32_t key[KPT], val[KPT], piw[KPT];
#pragma unroll
    for (int r = 0; r < KPT; ++r) {
      const int li = chunk_index<KPT>(r);
      const bool valid = li < nblk;
      const size_t gi = static_cast<size_t>(start) + base + (valid ? li : 0);
      key[r] = valid ? keys_in[gi] : 0u;
      val[r] = valid ? vals_in[gi] : 0u;
    }
    rank_in_waves(L, key, nblk, 0, piw);
    __syncthreads();
    uint32_t cnt[BPT], sc = 0;
    wave_offsets(L, cnt);
#pragma unroll
    for (int j = 0; j < BPT; ++j) sc += cnt[j];
    uint32_t all = 0;
    uint32_t lb = block_excl_scan(sc, L.wsum, &all);
#pragma unroll
    for (int j = 0; j < BPT; ++j) {
      const int dd = t * BPT + j;
      L.lstart[dd] = lb;
      if (one_chunk) {
        L.glob[dd] = start;  // the sorted chunk is the sorted bucket
      } else {
        L.glob[dd] = start + offs[dd] - lb;  // modulo 2^32
        offs[dd] += cnt[j];
      }
      lb += cnt[j];
    }
    __syncthreads();
    place_chunk(L, key, val, piw, nblk, 0);
    __syncthreads();
    write_chunk(L, nblk, 0, keys_out, vals_out);
    __syncthreads();  // L is reused by the next chunk
  }
}

int sort_blocks(int n, int kpt) { return (n + chunk_keys(kpt) - 1) / chunk_keys(kpt); }

// digit width per code width: two 10-bit passes for 2D's 20-bit codes; 8-bit
// digits (4 passes) for 3D/4D, where wider digits measured slower per pass
// than the pass they save
int digit_bits(int end_bit) { return end_bit == 20 ? 10 : 8; }

template <int RB>
hipError_t run_passes(uint32_t *hist, uint32_t *pre, uint32_t *totals, const float *pos,
                      int dims, uint32_t *keys0, uint32_t *keys1, uint32_t *vals0,
                      uint32_t *vals1, int n, int end_bit, hipStream_t stream,
                      const uint32_t **keys_sorted, const uint32_t **vals_sorted) {
  const int blocks = sort_blocks(n, kKeysPerThread);
  uint32_t *kin = keys0, *kout = keys1, *vin = nullptr, *vout = vals1;
  uint32_t *vspare = vals0;
  const int passes = std::max(1, (end_bit + RB - 1) / RB);
  for (int pass = 0; pass < passes; ++pass) {
    const int shift = RB * pass;
    if (pass == 0) {
      hipLaunchKernelGGL((radix_hist_kernel<RB, true, kKeysPerThread>), dim3(blocks), dim3(kSortThreads), 0, stream,
                         nullptr, pos, dims, n, shift, blocks, hist);
    } else {
      hipLaunchKernelGGL((radix_hist_kernel<RB, false, kKeysPerThread>), dim3(blocks), dim3(kSortThreads), 0,
                         stream, kin, nullptr, dims, n, shift, blocks, hist);
    }
    hipLaunchKernelGGL(radix_scan_kernel, dim3((1 << RB) / kScanDigits), dim3(kSortThreads), 0,
                       stream, hist, blocks, 1 << RB, pre, totals);
    if (pass == 0) {
      hipLaunchKernelGGL((radix_scatter_kernel<RB, true, kKeysPerThread>), dim3(blocks), dim3(kSortThreads), 0,
                         stream, nullptr, nullptr, pos, dims, n, shift, blocks, nullptr, pre, totals,
                         kout, vout);
    } else {
      hipLaunchKernelGGL((radix_scatter_kernel<RB, false, kKeysPerThread>), dim3(blocks), dim3(kSortThreads), 0,
                         stream, kin, vin, nullptr, dims, n, shift, blocks, nullptr, pre, totals,
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
  // hist[G][kBins] + pre[G][kBins] + totals[kBins] + starts[kBins] at the
  // widest digit
  const size_t bins = size_t(1) << 10;
  const int blocks = std::max(sort_blocks(n, kKeysPerThread), sort_blocks(n, kKeysPerThread2D));
  *bytes = (2 * bins * std::max(1, blocks) + 2 * bins) * sizeof(uint32_t);
  return hipSuccess;
}

hipError_t morton_sort_batch(void *tmp, size_t tmp_bytes, const float *pos, int dims,
                             uint32_t *keys0, uint32_t *keys1, uint32_t *vals0, uint32_t *vals1,
                             int n, hipStream_t stream, const uint32_t **keys_sorted,
                             const uint32_t **vals_sorted) {
  size_t need = 0;
  const hipError_t need_err = morton_sort_temp_bytes(n, &need);
  if (need_err != hipSuccess) return need_err;
  if (n <= 0 || tmp_bytes < need || dims < 2 || dims > 4) return hipErrorInvalidValue;
  // 2D codes interleave x and y only (the lifted z = 0 bits are all zero,
  // which leaves the order unchanged): 20 bits; 3D 30 bits; 4D 32 bits.
  const int end_bit = dims == 2 ? 20 : (dims == 3 ? 30 : 32);
  const size_t bins = size_t(1) << digit_bits(end_bit);
  const int blocks = sort_blocks(n, digit_bits(end_bit) == 8 ? kKeysPerThread : kKeysPerThread2D);
  uint32_t *hist = static_cast<uint32_t *>(tmp);
  uint32_t *pre = hist + bins * blocks;
  uint32_t *totals = pre + bins * blocks;
  uint32_t *starts = totals + bins;
  if (digit_bits(end_bit) == 8)
    return run_passes<8>(hist, pre, totals, pos, dims, keys0, keys1, vals0, vals1, n, end_bit,
                         stream, keys_sorted, vals_sorted);
  // 2D: an MSD pass on the top 10 bits (codes computed from the positions),
  // then one block per top digit sorts its bucket by the low 10 bits
  constexpr int K2 = kKeysPerThread2D;
  hipLaunchKernelGGL((radix_hist_kernel<10, true, K2>), dim3(blocks), dim3(kSortThreads), 0,
                     stream, nullptr, pos, dims, n, 10, blocks, hist);
  hipLaunchKernelGGL(radix_scan_kernel, dim3((1 << 10) / kScanDigits), dim3(kSortThreads), 0,
                     stream, hist, blocks, 1 << 10, pre, totals);
  hipLaunchKernelGGL((radix_scatter_kernel<10, true, K2>), dim3(blocks), dim3(kSortThreads), 0,
                     stream, nullptr, nullptr, pos, dims, n, 10, blocks, starts, pre, totals, keys1,
                     vals1);
  hipLaunchKernelGGL((bucket_sort_kernel<10, K2>), dim3(1 << 10), dim3(kSortThreads), 0, stream,
                     keys1, vals1, starts, totals, keys0, vals0);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  *keys_sorted = keys0;
  *vals_sorted = vals0;
  return hipSuccess;
}

}  // namespace tmnn_hip
