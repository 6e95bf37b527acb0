// grad_kernel.hpp -- position gradient of the field (FieldEvaluator::
// evaluate_with_gradient): given dx = d out_m / d(features) of every point
// (the fused kernel in kModeInputGrad), accumulate
//   d out_m / d pos_a += (dx[l][f] * r_l) * d feat_{l,f} / d frac_a
// over levels l (outer) and features f, with the reference's derivative forms
// (neural_sdf_analytical_eval_gradient_points, mlp_kernel_emitter.cpp:
// 1865-2090): the lerp form of trilinear_feature_grad (:1677-1704) in 3D and
// for the lifted 2D points (fz = 0: the z = 1 terms vanish exactly), the
// product loops (:2034-2056) in 4D.
#pragma once

#include "device_common.hpp"

namespace tmnn_hip {

struct PosGradArgs {
  int32_t n, L, F, M, m;      // points, levels, features/level, outputs, this output
  uint32_t log2T;
  float res[kMaxLevels];
  const float *pos;           // [n][D]
  const float *table;         // [L][T][F]
  const float *dx;            // [n][L*F]
  float *grads;               // [n][M][D]
};

template <int D>
__global__ void __launch_bounds__(256) pos_grad_kernel(PosGradArgs a) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= a.n) return;
  float p[D];
#pragma unroll
  for (int k = 0; k < D; ++k) p[k] = a.pos[static_cast<size_t>(i) * D + k];
  const uint32_t tmask = (1u << a.log2T) - 1u;
  const float *dxi = a.dx + static_cast<size_t>(i) * a.L * a.F;
  float gp[D];
#pragma unroll
  for (int k = 0; k < D; ++k) gp[k] = 0.0f;
  for (int l = 0; l < a.L; ++l) {
    const float r = a.res[l];
    const Cell<D> c = cell_of<D>(p, r);
    const size_t lbase = static_cast<size_t>(l) << a.log2T;
    for (int f = 0; f < a.F; ++f) {
      const float s = dxi[l * a.F + f] * r;
      auto at = [&](int dx, int dy, int dz, int dw) {
        int co[D];
        co[0] = c.bc[0] + dx;
        co[1] = c.bc[1] + dy;
        if constexpr (D >= 3) co[2] = c.bc[2] + dz;
        if constexpr (D == 4) co[3] = c.bc[3] + dw;
        (void)dz;
        (void)dw;
        return a.table[(lbase + hash_corner<D>(co, tmask)) * a.F + f];
      };
      const float fx = c.fr[0], fy = c.fr[1];
      if constexpr (D == 2) {
        const float c000 = at(0, 0, 0, 0), c010 = at(0, 1, 0, 0), c100 = at(1, 0, 0, 0),
                    c110 = at(1, 1, 0, 0);
        gp[0] = gp[0] + s * ((1.0f - fy) * (c100 - c000) + fy * (c110 - c010));
        gp[1] = gp[1] + s * ((1.0f - fx) * (c010 - c000) + fx * (c110 - c100));
      } else if constexpr (D == 3) {
        const float fz = c.fr[2];
        const float c000 = at(0, 0, 0, 0), c001 = at(0, 0, 1, 0), c010 = at(0, 1, 0, 0),
                    c011 = at(0, 1, 1, 0), c100 = at(1, 0, 0, 0), c101 = at(1, 0, 1, 0),
                    c110 = at(1, 1, 0, 0), c111 = at(1, 1, 1, 0);
        gp[0] = gp[0] + s * ((1.0f - fz) * ((1.0f - fy) * (c100 - c000) + fy * (c110 - c010)) +
                             fz * ((1.0f - fy) * (c101 - c001) + fy * (c111 - c011)));
        gp[1] = gp[1] + s * ((1.0f - fz) * ((1.0f - fx) * (c010 - c000) + fx * (c110 - c100)) +
                             fz * ((1.0f - fx) * (c011 - c001) + fx * (c111 - c101)));
        gp[2] = gp[2] + s * ((1.0f - fy) * ((1.0f - fx) * (c001 - c000) + fx * (c101 - c100)) +
                             fy * ((1.0f - fx) * (c011 - c010) + fx * (c111 - c110)));
      } else {
        const float fr[4] = {c.fr[0], c.fr[1], c.fr[2], c.fr[3]};
        float cv[2][2][2][2];
#pragma unroll
        for (int dw = 0; dw < 2; ++dw)
#pragma unroll
          for (int dz = 0; dz < 2; ++dz)
#pragma unroll
            for (int dy = 0; dy < 2; ++dy)
#pragma unroll
              for (int dx = 0; dx < 2; ++dx) cv[dw][dz][dy][dx] = at(dx, dy, dz, dw);
        auto w = [&](int d, int axis) { return d == 0 ? (1.0f - fr[axis]) : fr[axis]; };
        float g4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int dw = 0; dw < 2; ++dw)
#pragma unroll
          for (int dz = 0; dz < 2; ++dz)
#pragma unroll
            for (int dy = 0; dy < 2; ++dy)
              g4[0] += w(dy, 1) * w(dz, 2) * w(dw, 3) * (cv[dw][dz][dy][1] - cv[dw][dz][dy][0]);
#pragma unroll
        for (int dw = 0; dw < 2; ++dw)
#pragma unroll
          for (int dz = 0; dz < 2; ++dz)
#pragma unroll
            for (int dx = 0; dx < 2; ++dx)
              g4[1] += w(dx, 0) * w(dz, 2) * w(dw, 3) * (cv[dw][dz][1][dx] - cv[dw][dz][0][dx]);
#pragma unroll
        for (int dw = 0; dw < 2; ++dw)
#pragma unroll
          for (int dy = 0; dy < 2; ++dy)
#pragma unroll
            for (int dx = 0; dx < 2; ++dx)
              g4[2] += w(dx, 0) * w(dy, 1) * w(dw, 3) * (cv[dw][1][dy][dx] - cv[dw][0][dy][dx]);
#pragma unroll
        for (int dz = 0; dz < 2; ++dz)
#pragma unroll
          for (int dy = 0; dy < 2; ++dy)
#pragma unroll
            for (int dx = 0; dx < 2; ++dx)
              g4[3] += w(dx, 0) * w(dy, 1) * w(dz, 2) * (cv[1][dz][dy][dx] - cv[0][dz][dy][dx]);
#pragma unroll
        for (int k = 0; k < 4; ++k) gp[k] = gp[k] + s * g4[k];
      }
    }
  }
  float *dst = a.grads + (static_cast<size_t>(i) * a.M + a.m) * D;
#pragma unroll
  for (int k = 0; k < D; ++k) dst[k] = gp[k];
}

}  // namespace tmnn_hip
