// step_kernel.hpp -- the end of a training step as one launch: the MLP
// gradient reduction over the train kernel's per-block partial rows, the
// step's loss, and the Adam pass over [hash entries | MLP parameters], with
// each updated MLP weight also written into the training plan's packed LDS
// image (so the next step needs no repack).
//
// Blocks [0, mlp_blocks): 64 MLP columns x 16 row groups each, the same
// fixed summation order as reduce_partials_kernel (row group g sums rows
// g, g + 16, ... ascending, then the groups in order), so the gradient, and
// with it the update, is bit-identical to reduce_partials_kernel followed by
// adam_kernel. Block mlp_blocks: the loss. The rest: hash entries,
// grid-stride.
#pragma once

#include "aux_kernels.hpp"
#include "field_kernel.hpp"

namespace tmnn_hip {

struct FinishArgs {
  AdamArgs adam;
  const float *partials;       // [part_blocks][mlp_count] per-block dW rows
  int32_t part_blocks;
  const float *loss_partials;  // [part_blocks]
  int32_t n;                   // points of the step
  float *loss_out;             // the step's loss (sum of partials / n)
  int32_t mlp_blocks;          // blocks reducing + updating MLP columns
  FieldLayout s;               // layout of the image below (pack_image_kernel's)
  int32_t f16;                 // fp16 fragments (else fp32)
  unsigned char *image;        // the training plan's packed image, updated in place
  // numerics probe (finish_step_kernel<F, true>): per block one row
  // {max |g|, sum g^2, max |update|, non-finite bits}; the loss block's row
  // is {max |output| over amax_partials, the loss, 0, 0}
  const float *amax_partials;  // [part_blocks] largest |output| per training block
  float4 *num_rows;            // [gridDim.x]
};

constexpr int kFinishThreads = kReduceCols * kReduceGroups;

// K-slot coordinates of unit u in an fp16 A fragment (inverse of kslot_f16):
// K step ks, lane quad q, slot j.
__device__ __forceinline__ void kslot_f16_inverse(int u, int &ks, int &q, int &j) {
  ks = u / 32;
  const int r = u % 32;
  q = (r & 15) >> 2;
  j = (r & 3) + (r >= 16 ? 4 : 0);
}

// Writes the image entries of MLP parameter idx (reference layout) with value
// w: the forward (hi, and lo for fp16) and backward fragment slots of a
// weight (the slots frag_value reads it into), or the bias slot. Padding
// slots never change and keep the zeros pack_image_kernel wrote.
__device__ __forceinline__ void write_image_param(const FinishArgs &a, int idx, float w) {
  const FieldLayout &s = a.s;
  for (int k = 0; k <= s.NHL; ++k) {
    const int mreal = k == s.NHL ? s.M : s.H;
    const int bo = s.b_off(k);
    if (idx >= bo + mreal) continue;
    if (idx >= bo) {
      reinterpret_cast<float *>(a.image + s.bias_off(k))[idx - bo] = w;
      return;
    }
    const int i = (idx - s.w_off(k)) / mreal, o = (idx - s.w_off(k)) % mreal;
    const int kin = k == 0 ? s.INP : s.HP;
    const int mout = k == s.NHL ? 16 : s.HP;
    if (a.f16) {
      int ks, q, j;
      kslot_f16_inverse(i, ks, q, j);  // forward A = W^T: input unit along K
      const int ef = (((o / 16) * (kin / 32) + ks) * 64 + 16 * q + (o % 16)) * 8 + j;
      const _Float16 hi = static_cast<_Float16>(w);
      reinterpret_cast<_Float16 *>(a.image + s.fwd_off(k))[ef] = hi;
      reinterpret_cast<_Float16 *>(a.image + s.fwd_lo_off(k))[ef] =
          static_cast<_Float16>(w - static_cast<float>(hi));
      kslot_f16_inverse(o, ks, q, j);  // backward A = W: output unit along K
      const int eb = (((i / 16) * (round_up(mout, 32) / 32) + ks) * 64 + 16 * q + (i % 16)) * 8 + j;
      reinterpret_cast<_Float16 *>(a.image + s.bwd_off(k))[eb] = hi;
    } else {
      const int ef = (((o / 16) * (kin / 16) + i / 16) * 64 + 16 * ((i % 16) / 4) + (o % 16)) * 4 + i % 4;
      reinterpret_cast<float *>(a.image + s.fwd_off(k))[ef] = w;
      const int eb = (((i / 16) * (mout / 16) + o / 16) * 64 + 16 * ((o % 16) / 4) + (i % 16)) * 4 + o % 4;
      reinterpret_cast<float *>(a.image + s.bwd_off(k))[eb] = w;
    }
    return;
  }
}

// Block-wide reduction of the threads' numerics terms into row blockIdx.x.
__device__ __forceinline__ void num_block_row(const FinishArgs &a, NumAcc acc) {
  __shared__ float4 nred[kFinishThreads / 64];
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    acc.gmax = fmaxf(acc.gmax, __shfl_xor(acc.gmax, off));
    acc.g2 += __shfl_xor(acc.g2, off);
    acc.umax = fmaxf(acc.umax, __shfl_xor(acc.umax, off));
    acc.bad |= static_cast<uint32_t>(__shfl_xor(static_cast<int>(acc.bad), off));
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) nred[wave] = make_float4(acc.gmax, acc.g2, acc.umax, __uint_as_float(acc.bad));
  __syncthreads();
  if (threadIdx.x == 0) {
    float4 r = nred[0];
    for (int w = 1; w < static_cast<int>(blockDim.x) / 64; ++w) {
      const float4 o = nred[w];
      r.x = fmaxf(r.x, o.x);
      r.y += o.y;
      r.z = fmaxf(r.z, o.z);
      r.w = __uint_as_float(__float_as_uint(r.w) | __float_as_uint(o.w));
    }
    a.num_rows[blockIdx.x] = r;
  }
}

template <int F, bool NUM = false>
__global__ void __launch_bounds__(kFinishThreads) finish_step_kernel(FinishArgs a) {
  const AdamArgs &ad = a.adam;
  NumAcc acc;
  if (blockIdx.x < static_cast<uint32_t>(a.mlp_blocks)) {
    __shared__ float red[kReduceGroups][kReduceCols + 1];
    const int c = threadIdx.x % kReduceCols;
    const int g = threadIdx.x / kReduceCols;
    const int col = blockIdx.x * kReduceCols + c;
    const int count = static_cast<int>(ad.mlp_count);
    float s = 0.0f;
    if (col < count) {
#pragma unroll 4
      for (int32_t b = g; b < a.part_blocks; b += kReduceGroups)
        s += a.partials[static_cast<size_t>(b) * count + col];
    }
    red[g][c] = s;
    __syncthreads();
    if (g == 0 && col < count) {
      float t = 0.0f;
#pragma unroll
      for (int k = 0; k < kReduceGroups; ++k) t += red[k][c];
      const float w = adam_mlp_param<F, NUM>(ad, col, ad.grad_mlp[col] + t, &acc);
      if (a.image) write_image_param(a, col, w);
    }
    if constexpr (NUM) num_block_row(a, acc);
    return;
  }
  if (blockIdx.x == static_cast<uint32_t>(a.mlp_blocks)) {
    // the step's loss: sum of the per-block loss partials (fixed lane order) / N
    if (threadIdx.x < 64) {
      const int lane = threadIdx.x;
      float t = 0.0f;
      for (int32_t b = lane; b < a.part_blocks; b += 64) t += a.loss_partials[b];
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) t += __shfl_xor(t, off);
      const float loss = a.n > 0 ? t / static_cast<float>(a.n) : 0.0f;
      if (lane == 0 && a.loss_out) *a.loss_out = loss;
      if constexpr (NUM) {
        float m = 0.0f;
        for (int32_t b = lane; b < a.part_blocks; b += 64) m = fmaxf(m, a.amax_partials[b]);
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
        if (lane == 0) a.num_rows[blockIdx.x] = make_float4(m, loss, 0.0f, 0.0f);
      }
    }
    return;
  }
  const uint32_t first = static_cast<uint32_t>(a.mlp_blocks) + 1u;
  const uint32_t stride = (gridDim.x - first) * blockDim.x;
  for (uint32_t j = (blockIdx.x - first) * blockDim.x + threadIdx.x; j < ad.hash_entries; j += stride)
    adam_hash_entry<F, NUM>(ad, j, &acc);
  if constexpr (NUM) num_block_row(a, acc);
}

}  // namespace tmnn_hip
