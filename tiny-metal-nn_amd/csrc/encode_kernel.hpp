// encode_kernel.hpp -- hash-grid encode forward as its own kernel, writing the
// input features of every point straight into the MFMA register layout the
// MLP kernels consume.
//
// The encode is a gather problem: 2^D corners x L levels per point, each an
// F-float load from a table that may not fit in L2. A launch of one thread
// per point, few registers and many waves per SIMD keeps enough loads in
// flight to run at the chip's gather rate; inside an MLP kernel (one wave per
// SIMD, the register file taken by weight-gradient accumulators) the same
// gathers are latency-bound. Each thread issues the loads of a group of
// feature quads (<= 128 floats) before it interpolates any of them.
//
// Arithmetic: as encode_level (the reference's corner order z, y, x
// ascending, weight ((wx * wy) * wz)(* wt), features summed from 0;
// emitHashEncodeUnified, mlp_kernel_emitter.cpp:205-360) -- bit-identical
// features.
//
// With a sort permutation, point i is pos[perm[i]], and the kernel also writes
// the positions in point (sorted) order for the hash-grid backward (the MLP
// kernels read targets through the permutation: per-thread row copies here
// measured slower).
//
// Layout of the feature buffer ("X tiles"): point i = 32 t + 16 nt + p and
// feature f = 16 kt + 4 q + r sit at float offset
//   ((((t * KT0 + kt) * kNT + nt) * 64 + p + 16 q) * 4 + r,
// i.e. one f32x4 per lane of a wave tile, in the order the MLP kernels hold
// X[kt][nt] in registers: a wave loads its tile with 16-byte coalesced loads.
// Padding features (IN <= f < 16 KT0) and padding points (n <= i < 32 t_max)
// are zero.
#pragma once

#include "device_common.hpp"

namespace tmnn_hip {

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

struct EncodeArgs {
  int32_t n;       // points
  int32_t n_pad;   // n rounded up to whole 32-point tiles
  int32_t L;       // levels
  int32_t KT0;     // input K tiles (16 features each)
  uint32_t log2T;
  float res[kMaxLevels];
  const float *pos;       // [n][D]
  const uint32_t *perm;   // nullable: point i is pos[perm[i]] (Morton order)
  float *pos_out;         // nullable: positions in point order, [n][D]
  const float *table;     // [L][T][F]
  float *xfeat;           // X tiles, n_pad * 16 * KT0 floats
};

constexpr int kEncodeThreads = 256;

// float offset of feature quad fq (features 4 fq .. 4 fq + 3) of point i
__host__ __device__ __forceinline__ size_t xtile_offset(int i, int fq, int KT0) {
  const int t = i >> 5, nt = (i >> 4) & 1, p = i & 15;
  const int kt = fq >> 2, q = fq & 3;
  return ((((static_cast<size_t>(t) * KT0 + kt) * 2 + nt) * 64) + p + 16 * q) * 4;
}

template <int D, int F>
__global__ void __launch_bounds__(kEncodeThreads) encode_features_kernel(EncodeArgs a) {
  constexpr int C = 1 << D;        // corners per level
  constexpr int LPQ = 4 / F;       // levels per feature quad
  // quads per group (QG * 4 * C floats in flight): 2D takes 4 (32 gathers,
  // 74 registers: six waves per SIMD hold a whole 2^18 batch at once), 3D and
  // 4D 32 / C
  constexpr int QG = D == 2 ? 4 : (C >= 32 ? 1 : 32 / C);
  const int i = blockIdx.x * kEncodeThreads + threadIdx.x;
  if (i >= a.n_pad) return;
  const bool valid = i < a.n;
  float p[D];
  const size_t src = valid ? (a.perm ? a.perm[i] : static_cast<uint32_t>(i)) : 0u;
#pragma unroll
  for (int k = 0; k < D; ++k) p[k] = valid ? a.pos[src * D + k] : 0.0f;
  if (a.pos_out && valid && blockIdx.y == 0)
#pragma unroll
    for (int k = 0; k < D; ++k) a.pos_out[static_cast<size_t>(i) * D + k] = p[k];
  const uint32_t tmask = (1u << a.log2T) - 1u;
  // gridDim.y > 1 (batches too small to fill the chip): thread (i, y) takes
  // feature quads [y * qps, (y + 1) * qps) of point i, so a small batch's
  // gathers spread over more threads instead of queueing in a few
  const int nquads = 4 * a.KT0;
  const int qps = (nquads + static_cast<int>(gridDim.y) - 1) / static_cast<int>(gridDim.y);
  const int qbeg = static_cast<int>(blockIdx.y) * qps;
  const int qend = qbeg + qps < nquads ? qbeg + qps : nquads;
  for (int q0 = qbeg; q0 < qend; q0 += QG) {
    float v[QG][LPQ][C][F];
#pragma unroll
    for (int g = 0; g < QG; ++g)
#pragma unroll
      for (int lv = 0; lv < LPQ; ++lv) {
        const int l = (q0 + g) * LPQ + lv;
        const bool on = valid && q0 + g < qend && l < a.L;
        const Cell<D> c = cell_of<D>(p, a.res[on ? l : 0]);
        const size_t lbase = static_cast<size_t>(on ? l : 0) << a.log2T;
#pragma unroll
        for (int k = 0; k < C; ++k) {
          int co[D];
          float wc[D];
          corner_of<D>(c, k, co, wc);
          const float *e = a.table + (lbase + hash_corner<D>(co, tmask)) * F;
          if constexpr (F == 1) {
            v[g][lv][k][0] = on ? e[0] : 0.0f;
          } else if constexpr (F == 2) {
            const f32x2 t = on ? *reinterpret_cast<const f32x2 *>(e) : f32x2{0.f, 0.f};
            v[g][lv][k][0] = t[0];
            v[g][lv][k][1] = t[1];
          } else {
            const f32x4 t = on ? *reinterpret_cast<const f32x4 *>(e) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int f = 0; f < 4; ++f) v[g][lv][k][f] = t[f];
          }
        }
      }
#pragma unroll
    for (int g = 0; g < QG; ++g) {
      if (q0 + g >= qend) break;
      f32x4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int lv = 0; lv < LPQ; ++lv) {
        const int l = (q0 + g) * LPQ + lv;
        const Cell<D> c = cell_of<D>(p, a.res[l < a.L ? l : 0]);
        float feat[F];
#pragma unroll
        for (int f = 0; f < F; ++f) feat[f] = 0.0f;
#pragma unroll
        for (int k = 0; k < C; ++k) {
          int co[D];
          float wc[D];
          corner_of<D>(c, k, co, wc);
          const float w = corner_weight<D>(wc);
#pragma unroll
          for (int f = 0; f < F; ++f) feat[f] = feat[f] + w * v[g][lv][k][f];
        }
#pragma unroll
        for (int f = 0; f < F; ++f) o[lv * F + f] = (valid && l < a.L) ? feat[f] : 0.0f;
      }
      // streamed out (non-temporal): the table keeps the caches
      __builtin_nontemporal_store(o, reinterpret_cast<f32x4 *>(a.xfeat + xtile_offset(i, q0 + g, a.KT0)));
    }
  }
}

// Level-major variant for large tables: one thread per (point, level),
// blockIdx.y = level, so the resident blocks gather from one level's slice of
// the table at a time (a 2^22-entry level is 32 MB; all levels together do not
// stay in the caches). Same arithmetic as encode_features_kernel; the thread
// stores its level's F features into their X-tile quad (the whole quad for
// F = 4, half of it for F = 2, one float for F = 1); the last level's threads
// also zero the padding features, level 0's write the sorted position.
template <int D, int F>
__global__ void __launch_bounds__(kEncodeThreads) encode_level_kernel(EncodeArgs a) {
  constexpr int C = 1 << D;  // corners per level
  const int l = blockIdx.y;
  const int i = blockIdx.x * kEncodeThreads + threadIdx.x;
  // every lane of a wave takes part in the lane swaps below: threads past the
  // padded batch gather for position 0 and store nothing
  const bool live = i < a.n_pad;
  const bool valid = i < a.n;
  float p[D];
  const size_t src = valid ? (a.perm ? a.perm[i] : static_cast<uint32_t>(i)) : 0u;
#pragma unroll
  for (int k = 0; k < D; ++k) p[k] = valid ? a.pos[src * D + k] : 0.0f;
  if (l == 0 && a.pos_out && valid)
#pragma unroll
    for (int k = 0; k < D; ++k) a.pos_out[static_cast<size_t>(i) * D + k] = p[k];
  const uint32_t tmask = (1u << a.log2T) - 1u;
  const Cell<D> c = cell_of<D>(p, a.res[l]);
  const float *lt = a.table + (static_cast<size_t>(l) << a.log2T) * F;
  // Corners x and x + 1 (k = 2m, 2m + 1) are neighbouring entries unless x
  // ends in seven 1 bits, so mostly one line. A v_permlane32_swap of their
  // entry indices lets one load instruction fetch both x-corners of 32 points
  // (lanes 0-31 corner x, lanes 32-63 corner x + 1 of the same points, then
  // the other 32 points): half the distinct lines per instruction. A second
  // swap of the loaded values returns each lane its own corners. The values
  // are swapped as the integers they were loaded as: with float operands
  // bit-cast to integers the compiler (ROCm 7.2) used the swap's first result
  // for both.
  float v[C][F];
#pragma unroll
  for (int m = 0; m < C / 2; ++m) {
    int co[D];
    float wc[D];
    corner_of<D>(c, 2 * m, co, wc);
    const uint32_t e0 = hash_corner<D>(co, tmask);
    co[0] += 1;
    const uint32_t e1 = hash_corner<D>(co, tmask);
    const auto r = __builtin_amdgcn_permlane32_swap(e0, e1, false, false);
    uint32_t t[2][F];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t *e = reinterpret_cast<const uint32_t *>(lt) + static_cast<size_t>(r[h]) * F;
      if constexpr (F == 1) {
        t[h][0] = e[0];
      } else if constexpr (F == 2) {
        const u32x2 x = *reinterpret_cast<const u32x2 *>(e);
        t[h][0] = x[0];
        t[h][1] = x[1];
      } else {
        const uint4 x = *reinterpret_cast<const uint4 *>(e);
        t[h][0] = x.x;
        t[h][1] = x.y;
        t[h][2] = x.z;
        t[h][3] = x.w;
      }
    }
#pragma unroll
    for (int f = 0; f < F; ++f) {
      const auto b = __builtin_amdgcn_permlane32_swap(t[0][f], t[1][f], false, false);
      const uint32_t lo = b[0], hi = b[1];
      v[2 * m][f] = __builtin_bit_cast(float, lo);
      v[2 * m + 1][f] = __builtin_bit_cast(float, hi);
    }
  }
  float feat[F];
#pragma unroll
  for (int f = 0; f < F; ++f) feat[f] = 0.0f;
#pragma unroll
  for (int k = 0; k < C; ++k) {
    int co[D];
    float wc[D];
    corner_of<D>(c, k, co, wc);
    const float w = corner_weight<D>(wc);
#pragma unroll
    for (int f = 0; f < F; ++f) feat[f] = feat[f] + w * v[k][f];
  }
  if (!live) return;
  const int f0 = l * F;  // the level's first feature
  float *dst = a.xfeat + xtile_offset(i, f0 / 4, a.KT0) + f0 % 4;
  if constexpr (F == 4) {
    *reinterpret_cast<f32x4 *>(dst) = valid ? f32x4{feat[0], feat[1], feat[2], feat[3]}
                                            : f32x4{0.f, 0.f, 0.f, 0.f};
  } else if constexpr (F == 2) {
    *reinterpret_cast<f32x2 *>(dst) = valid ? f32x2{feat[0], feat[1]} : f32x2{0.f, 0.f};
  } else {
    *dst = valid ? feat[0] : 0.0f;
  }
  if (l == a.L - 1)
    for (int f = a.L * F; f < 16 * a.KT0; ++f)
      a.xfeat[xtile_offset(i, f / 4, a.KT0) + f % 4] = 0.0f;
}

}  // namespace tmnn_hip
