// tile_scatter.hpp -- the hash-grid backward of one 32-point MLP tile, run by
// the MLP training kernel itself (mlp_kernel.hpp) right after the tile's
// input-feature gradients dx come off the matrix cores, instead of storing
// dx for hash_scatter_kernel.
//
// Same arithmetic as hash_scatter_kernel (scatter_kernel.hpp; reference
// emitHashScatter, mlp_kernel_emitter.cpp:672-901, mask :48-71): per corner
// and feature int32(trunc(d * w * 65536)) with w = ((wx * wy) * wz) (F = 2),
// packed 64-bit atomics for the feature pair, every visited corner's flag
// stored; a group of lanes whose contributions all truncate to 0 (the common
// case once training converges) only stores the flags. Lanes that hit the
// same entry each issue their own atomic (no run merging: a converging
// batch's contributions are almost all zero).
//
// Why here: the separate scatter re-read 8 B of dx per feature and spent its
// time on the per-lane memory requests of the flag stores; in the MLP kernel
// the memory pipeline is nearly idle, so the index arithmetic and the stores
// run beside the matrix work, and the dx round trip through HBM disappears.
//
// Lane layout (D layout of dx[kt][nt]): lane p + 16 q holds features
// 16 kt + 4 q + r of point 16 nt + p; for F = 2 items r = 2h, 2h + 1 are the
// two features of level 8 kt + 2 q + h. One wave instruction therefore
// covers 16 points at each of four levels.
#pragma once

#include "field_kernel.hpp"
#include "scatter_kernel.hpp"

namespace tmnn_hip {

// Compile-time shapes with a fused scatter: (D, F) of the hash grid. F = 2
// only (the feature pair of a level lies in one lane).
__host__ __device__ constexpr bool tile_scatter_shape(int D, int F) {
  return F == 2 && (D == 2 || D == 3);
}

// dx: the tile's input-feature gradients (fp32, still carrying the loss
// scale); pos: the lane's point positions per column tile (sorted order);
// res: the per-level resolution table (the LDS image's copy).
// GB, GE: the (K tile, pair) groups [GB, GE) of dx this call covers (group
// 2 kt + h: levels 8 kt + 2 q + h), so a caller can spread one tile's
// backward over several places.
template <int D, int F, int KT0, int GB, int GE>  // defaults: field_kernel.hpp
__device__ __forceinline__ void tile_scatter(const FieldArgs &a, const f32x4 (&dx)[KT0][kNT],
                                             const float (&pos)[kNT][D], const bool (&valid)[kNT],
                                             const float *res, int q) {
  static_assert(tile_scatter_shape(D, F), "fused scatter shape");
  static_assert(0 <= GB && GB <= GE && GE <= 2 * KT0, "group range");
  const uint32_t tmask = (1u << a.log2T) - 1u;
  const __amdgpu_buffer_rsrc_t flags = flag_rsrc(a.mask, a.L, a.log2T);
#pragma unroll
  for (int gi = GB; gi < GE; ++gi) {
      const int kt = gi / 2, h = gi % 2;
      const int l = 8 * kt + 2 * q + h;
      const bool lv = l < a.L;
      const float rl = res[lv ? l : 0];
      const uint32_t lbase = static_cast<uint32_t>(lv ? l : 0) << a.log2T;
#pragma unroll
      for (int nt = 0; nt < kNT; ++nt) {
        const bool on = valid[nt] && lv;
        float d[2];
        d[0] = dx[kt][nt][2 * h] * a.inv_loss_scale;
        d[1] = dx[kt][nt][2 * h + 1] * a.inv_loss_scale;
        const Cell<D> c = cell_of<D>(pos[nt], rl);
        if (__all(!on || grads_vanish<2>(d))) {
          // flags only. Corners x and x + 1 of a cell differ only in the low
          // bits the carry of x + 1 flips, so their flag bytes share a
          // 128-byte line unless x ends in seven 1 bits: one
          // v_permlane32_swap gives each store instruction both x-corners of
          // 32 (point, level) pairs (lanes 0-31 corner x, lanes 32-63 corner
          // x + 1 of the same pairs), half the line requests of one
          // instruction per corner
#pragma unroll
          for (int m = 0; m < (1 << (D - 1)); ++m) {
            int co[D];
            float wc[D];
            corner_of<D>(c, 2 * m, co, wc);
            const uint32_t e0 = on ? lbase + hash_corner<D>(co, tmask) : kNoEntry;
            co[0] += 1;
            const uint32_t e1 = on ? lbase + hash_corner<D>(co, tmask) : kNoEntry;
            const auto r = __builtin_amdgcn_permlane32_swap(e0, e1, false, false);
            mark_flag(flags, r[0]);
            mark_flag(flags, r[1]);
          }
        } else {
          const bool fits = __all(!on || grads_fit<2>(d));
#pragma unroll
          for (int k = 0; k < (1 << D); ++k) {
            int co[D];
            float wc[D];
            corner_of<D>(c, k, co, wc);
            const uint32_t entry = lbase + hash_corner<D>(co, tmask);
            const float w = corner_weight<D>(wc);
            int32_t ci[2];
#pragma unroll
            for (int f = 0; f < 2; ++f) {
              const float v = d[f] * w;
              ci[f] = fits ? static_cast<int32_t>(v * kGradScale) : f2i_trunc(v * kGradScale);
            }
            const int64_t v64 = static_cast<int64_t>(
                (static_cast<uint64_t>(static_cast<uint32_t>(ci[1])) << 32) +
                static_cast<uint64_t>(static_cast<int64_t>(ci[0])));
            if (on && v64 != 0)
              atomicAdd(reinterpret_cast<unsigned long long *>(a.grad_hash + static_cast<size_t>(entry) * 2),
                        static_cast<unsigned long long>(v64));
            mark_flag(flags, on ? entry : kNoEntry);
          }
        }
      }
    }
}

}  // namespace tmnn_hip
