// rate_kernels.hpp -- reference-rate kernels at a trainer's own hash-grid
// shape (debug entry tmnn_debug_hash_rates): the throughput of the memory
// operations the encode and scatter kernels are built from, with everything
// else removed, over the same points in the same order. They give the
// "achievable" denominators the encode and scatter are measured against.
//   kRateGather -- every corner of every level, F floats each (the encode's
//                  loads and addresses, no interpolation; one float per point
//                  is written so the loads stay live);
//   kRateAtomic -- one F-wide integer atomic add (64-bit for F = 2, as the
//                  scatter packs it) of a constant nonzero value into a
//                  scratch table per run of lanes on the same entry (corner
//                  and level; the scatter merges such runs);
//   kRateFlag   -- one byte store per run of lanes on the same entry (the
//                  visit flags, as the scatter stores them).
#pragma once

#include "device_common.hpp"

namespace tmnn_hip {

enum : int32_t { kRateGather = 0, kRateAtomic = 1, kRateFlag = 2 };

struct HashRateArgs {
  int32_t n, L;
  uint32_t log2T;
  float res[kMaxLevels];
  const float *pos;    // [n][D]
  const float *table;  // [L][T][F]
  float *out;          // [n] (gather)
  int32_t *acc;        // [L][T][F] scratch (atomic)
  uint8_t *flags;      // [L][T] scratch (flag)
};

template <int D, int F, int KIND>
__global__ void __launch_bounds__(256) hash_rate_kernel(HashRateArgs a) {
  constexpr int C = 1 << D;
  constexpr int G = C >= 16 ? 2 : (C >= 8 ? 4 : 8);  // levels whose loads are in flight together
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  const bool valid = i < a.n;  // lanes past the batch take part in the run test
  const int lane = threadIdx.x & 63;
  float p[D];
#pragma unroll
  for (int k = 0; k < D; ++k) p[k] = a.pos[static_cast<size_t>(valid ? i : 0) * D + k];
  const uint32_t tmask = (1u << a.log2T) - 1u;
  float sum = 0.0f;
  for (int l0 = 0; l0 < a.L; l0 += G) {
    float v[G][C];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int l = l0 + g < a.L ? l0 + g : a.L - 1;
      const Cell<D> c = cell_of<D>(p, a.res[l]);
      const size_t lbase = static_cast<size_t>(l) << a.log2T;
#pragma unroll
      for (int k = 0; k < C; ++k) {
        int co[D];
        float wc[D];
        corner_of<D>(c, k, co, wc);
        const uint32_t local = valid ? hash_corner<D>(co, tmask) : 0xFFFFFFFFu;
        const size_t e = lbase + (valid ? local : 0u);
        // first lane of a run of equal entries (previous lane by DPP wave_shr:1)
        const uint32_t prev = static_cast<uint32_t>(
            __builtin_amdgcn_update_dpp(-1, static_cast<int>(local), 0x138, 0xf, 0xf, false));
        const bool head = valid && (lane == 0 || prev != local);
        if constexpr (KIND == kRateGather) {
          float t = 0.0f;
          if constexpr (F == 1) {
            t = a.table[e];
          } else if constexpr (F == 2) {
            const f32x2 q = *reinterpret_cast<const f32x2 *>(a.table + e * 2);
            t = q[0] + q[1];
          } else {
            const f32x4 q = *reinterpret_cast<const f32x4 *>(a.table + e * 4);
            t = (q[0] + q[1]) + (q[2] + q[3]);
          }
          v[g][k] = t;
        } else if constexpr (KIND == kRateAtomic) {
          if (head && l0 + g < a.L) {
            if constexpr (F == 2) {
              atomicAdd(reinterpret_cast<unsigned long long *>(a.acc + e * 2), 0x100000001ull);
            } else {
#pragma unroll
              for (int f = 0; f < F; ++f) atomicAdd(a.acc + e * F + f, 1);
            }
          }
        } else {
          if (head && l0 + g < a.L) a.flags[e] = 1;
        }
      }
    }
    if constexpr (KIND == kRateGather) {
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int k = 0; k < C; ++k) sum += l0 + g < a.L ? v[g][k] : 0.0f;
    }
  }
  if constexpr (KIND == kRateGather)
    if (valid) a.out[i] = sum;
}

// Level-major variant, for the shapes whose encode or scatter walks the
// levels one at a time (tables over 2 MB or 8 MB per level): blockIdx.y =
// level, one thread per point, so the resident blocks work on one level's
// slice at a time, as encode_level_kernel and hash_scatter_level_kernel do.
// Every lane issues its own corner operations (no lane pairing). The gather
// sums its corners and stores only on an impossible bit pattern, so the
// loads stay live without an output stream.
template <int D, int F, int KIND>
__global__ void __launch_bounds__(256) hash_rate_level_kernel(HashRateArgs a) {
  constexpr int C = 1 << D;
  const int l = blockIdx.y;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  const bool valid = i < a.n;
  const int lane = threadIdx.x & 63;
  float p[D];
#pragma unroll
  for (int k = 0; k < D; ++k) p[k] = a.pos[static_cast<size_t>(valid ? i : 0) * D + k];
  const uint32_t tmask = (1u << a.log2T) - 1u;
  const Cell<D> c = cell_of<D>(p, a.res[l]);
  const size_t lbase = static_cast<size_t>(l) << a.log2T;
  float v[C];
#pragma unroll
  for (int k = 0; k < C; ++k) {
    int co[D];
    float wc[D];
    corner_of<D>(c, k, co, wc);
    const uint32_t local = valid ? hash_corner<D>(co, tmask) : 0xFFFFFFFFu;
    const size_t e = lbase + (valid ? local : 0u);
    const uint32_t prev = static_cast<uint32_t>(
        __builtin_amdgcn_update_dpp(-1, static_cast<int>(local), 0x138, 0xf, 0xf, false));
    const bool head = valid && (lane == 0 || prev != local);
    if constexpr (KIND == kRateGather) {
      if constexpr (F == 1) {
        v[k] = a.table[e];
      } else if constexpr (F == 2) {
        const f32x2 q = *reinterpret_cast<const f32x2 *>(a.table + e * 2);
        v[k] = q[0] + q[1];
      } else {
        const f32x4 q = *reinterpret_cast<const f32x4 *>(a.table + e * 4);
        v[k] = (q[0] + q[1]) + (q[2] + q[3]);
      }
    } else if constexpr (KIND == kRateAtomic) {
      if (head) {
        if constexpr (F == 2) {
          atomicAdd(reinterpret_cast<unsigned long long *>(a.acc + e * 2), 0x100000001ull);
        } else {
#pragma unroll
          for (int f = 0; f < F; ++f) atomicAdd(a.acc + e * F + f, 1);
        }
      }
    } else {
      if (head) a.flags[e] = 1;
    }
  }
  if constexpr (KIND == kRateGather) {
    float sum = 0.0f;
#pragma unroll
    for (int k = 0; k < C; ++k) sum += v[k];
    if (valid && __builtin_bit_cast(uint32_t, sum) == 0x7fc0beefu) a.out[i] = sum;
  }
}

// LDS read rate (debug entry tmnn_debug_lds_rate): the LDS bandwidth the
// MLP kernels' weight fragments and parked operands are read at, as they read
// them (ds_read_b128, one 16-byte slot per lane, consecutive lanes on
// consecutive slots: conflict-free). Each 256-thread block fills 32 KB of LDS
// (four blocks per CU fit), then every lane reads kLdsRateSlots slots per
// iteration. The loaded registers are consumed by an empty asm statement that
// also clobbers memory, so each iteration issues its loads again and no ALU
// work competes with them; out is written only on an impossible value.
constexpr int kLdsRateThreads = 256;
constexpr int kLdsRateSlots = 8;

typedef uint32_t rate_u32x4 __attribute__((ext_vector_type(4)));

__global__ void __launch_bounds__(kLdsRateThreads) lds_rate_kernel(int32_t iters, uint32_t *out) {
  __shared__ rate_u32x4 buf[kLdsRateSlots * kLdsRateThreads];
  const int t = threadIdx.x;
#pragma unroll
  for (int k = 0; k < kLdsRateSlots; ++k) {
    rate_u32x4 w = {static_cast<uint32_t>(t), static_cast<uint32_t>(k),
                    static_cast<uint32_t>(t ^ k), 1u};
    buf[k * kLdsRateThreads + t] = w;
  }
  __syncthreads();
  uint32_t acc = 0u;
  for (int it = 0; it < iters; ++it) {
    rate_u32x4 v[kLdsRateSlots];
#pragma unroll
    for (int k = 0; k < kLdsRateSlots; ++k) v[k] = buf[k * kLdsRateThreads + t];
    asm volatile("" ::"v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3]), "v"(v[4]), "v"(v[5]),
                 "v"(v[6]), "v"(v[7])
                 : "memory");
    acc += v[it & (kLdsRateSlots - 1)].w;
  }
  if (acc == 0x9E3779B9u) out[blockIdx.x] = acc;
}

}  // namespace tmnn_hip
