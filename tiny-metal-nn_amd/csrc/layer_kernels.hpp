// layer_kernels.hpp -- the layer-wise ("tiled") MLP path: one tiled fp32
// matrix product per layer with the activations of the whole batch in global
// memory, for the shapes the fused kernels do not instantiate (hidden widths
// up to 512, up to 128 input features, any number of outputs, fp32 training
// at width 128). This is the MI355X counterpart of the reference's Tiled MLP
// family (network_planner.cpp:132-300: the family a model falls back to when
// the fully fused kernel cannot hold it): correctness over speed, every
// KernelSpec shape (kernel_spec.cpp:12-44) runs.
//
// Products: C[r][c] = sum_k A(r, k) B(k, c) over 64 x 64 output tiles (row
// tiles along blockIdx.x, column tiles along blockIdx.y), K in steps of 16
// staged through LDS, each of the block's four waves a 32 x 32 quadrant on
// the matrix cores (v_mfma_f32_16x16x4_f32: fp32 operands, fp32
// accumulation). The
// operands are read in place: activations row-major, the input features as
// X tiles (encode_kernel.hpp), the weights in the reference layout
// W[in][out] (the backward reads them transposed), and for the weight
// gradients the activations / deltas transposed with the points along K,
// one partial row per chunk of the batch (the rows finish_step_kernel /
// reduce_partials_kernel reduce in a fixed order); the bias gradients are
// the same product with an extra all-ones row of A (the reference layout
// stores b right after W, so that row lands in the bias slots). Epilogues
// fuse the bias and ReLU (forward), the ReLU derivative [h > 0] of the
// stored activation (backward), and the output scale.
#pragma once

#include "encode_kernel.hpp"
#include "field_kernel.hpp"

namespace tmnn_hip {

enum : int32_t {
  kLwEpiHidden = 0,  // out = relu(acc + bias)
  kLwEpiOutput = 1,  // y = acc + bias -> out (row mapped) and out2
  kLwEpiMask = 2,    // out = mask > 0 ? acc : 0
  kLwEpiScale = 3,   // out = acc * scale
  kLwEpiPartial = 4  // partial row of blockIdx.z: dst[z * dst_stride + dst_off + r * C + c]
};

enum : int32_t {
  kLwARow = 0,     // A(r, k) = A[r * lda + k]
  kLwAXTiles = 1,  // A(r, k) = feature k of point r in the X tiles
  kLwACol = 2,     // A(r, k) = A[k * lda + r]
  kLwAXTilesT = 3  // A(r, k) = feature r of point k in the X tiles
};

struct LwGemmArgs {
  int32_t R, C, K;       // output rows, columns; contraction length
  int32_t k_chunk;       // K range of blockIdx.z: [z * k_chunk, min(K, (z + 1) * k_chunk))
  int32_t a_mode, lda, KT0;
  int32_t b_trans, ldb;  // 0: B(k, c) = B[k * ldb + c]; 1: B(k, c) = B[c * ldb + k]
  int32_t epi;
  const float *A;
  const float *B;
  const float *bias;
  float *out;
  int32_t ldo;
  const uint32_t *out_index;  // kLwEpiOutput: row of out for output row r (nullable)
  float *out2;                // kLwEpiOutput: dense copy [R][ldo2] (nullable)
  int32_t ldo2;
  const float *mask;          // kLwEpiMask: [R][ldm]
  int32_t ldm;
  float scale;
  float *dst;                 // kLwEpiPartial
  int64_t dst_stride;
  int32_t dst_off;
  int32_t ones_row;           // 1: A's last row (r == R - 1) is all ones (bias gradients)
};

constexpr int kLwTile = 64;
// Points per chunk of a layer-wise forward pass (inference has no batch cap):
// two activation buffers of kLwForwardChunk x H floats.
constexpr int kLwForwardChunk = 1 << 18;
constexpr int kLwK = 16;

__device__ __forceinline__ float lw_a(const LwGemmArgs &g, int r, int k) {
  if (g.ones_row && r == g.R - 1) return 1.0f;
  switch (g.a_mode) {
    case kLwARow: return g.A[static_cast<size_t>(r) * g.lda + k];
    case kLwACol: return g.A[static_cast<size_t>(k) * g.lda + r];
    case kLwAXTiles: return g.A[xtile_offset(r, k >> 2, g.KT0) + (k & 3)];
    default: return g.A[xtile_offset(k, r >> 2, g.KT0) + (r & 3)];
  }
}

__device__ __forceinline__ float lw_b(const LwGemmArgs &g, int k, int c) {
  return g.b_trans ? g.B[static_cast<size_t>(c) * g.ldb + k] : g.B[static_cast<size_t>(k) * g.ldb + c];
}

// LDS staging of one K step: row (or column) i of the tile holds its kLwK
// operands contiguously (kLwKP floats per row: 16-byte aligned and padded),
// so each lane reads the four K values of an MFMA A or B operand with one
// ds_read_b128.
constexpr int kLwKP = kLwK + 4;
constexpr int kLwStage = kLwTile * kLwK / 256;  // operand elements per thread and K step

__global__ void __launch_bounds__(256) lw_gemm_kernel(LwGemmArgs g) {
  // the tile's A rows and B columns of the current K step, K innermost
  __shared__ __align__(16) float As[kLwTile * kLwKP];
  __shared__ __align__(16) float Bs[kLwTile * kLwKP];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int p = lane & 15, q = lane >> 4;
  // wave w computes the 32 x 32 quadrant (rows (w & 1) * 32, columns
  // (w >> 1) * 32) of the 64 x 64 tile: 2 x 2 MFMA tiles of 16 x 16
  const int wr = (wave & 1) * 32, wc = (wave >> 1) * 32;
  const int r0 = blockIdx.x * kLwTile, c0 = blockIdx.y * kLwTile;
  const int kb = blockIdx.z * g.k_chunk;
  const int ke = min(g.K, kb + g.k_chunk);
  f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  // Operand staging, software-pipelined: the next K step's slices are read
  // from global memory into registers before the current step's products
  // and stored to LDS after them. Consecutive threads walk the operand's
  // contiguous index; elements outside the product are zero.
  const bool a_k_fast = g.a_mode == kLwARow, b_k_fast = g.b_trans != 0;
  float ra[kLwStage], rb[kLwStage];
  auto load = [&](int k0) {
#pragma unroll
    for (int e = 0; e < kLwStage; ++e) {
      const int idx = tid + 256 * e;
      const int rr = a_k_fast ? idx / kLwK : idx % kLwTile;
      const int kk = a_k_fast ? idx % kLwK : idx / kLwTile;
      const int r = r0 + rr, k = k0 + kk;
      ra[e] = (r < g.R && k < ke) ? lw_a(g, r, k) : 0.0f;
      const int cc = b_k_fast ? idx / kLwK : idx % kLwTile;
      const int kc = b_k_fast ? idx % kLwK : idx / kLwTile;
      const int c = c0 + cc, k2 = k0 + kc;
      rb[e] = (c < g.C && k2 < ke) ? lw_b(g, k2, c) : 0.0f;
    }
  };
  auto store = [&]() {
#pragma unroll
    for (int e = 0; e < kLwStage; ++e) {
      const int idx = tid + 256 * e;
      const int rr = a_k_fast ? idx / kLwK : idx % kLwTile;
      const int kk = a_k_fast ? idx % kLwK : idx / kLwTile;
      As[rr * kLwKP + kk] = ra[e];
      const int cc = b_k_fast ? idx / kLwK : idx % kLwTile;
      const int kc = b_k_fast ? idx % kLwK : idx / kLwTile;
      Bs[cc * kLwKP + kc] = rb[e];
    }
  };
  if (kb < ke) {
    load(kb);
    store();
  }
  __syncthreads();
  for (int k0 = kb; k0 < ke; k0 += kLwK) {
    const bool more = k0 + kLwK < ke;  // uniform over the block
    if (more) load(k0 + kLwK);
    // v_mfma_f32_16x16x4_f32: lane p + 16 q supplies A[row p][k] and
    // B[k][column p] of K slot q; the four MFMAs of a 16-wide K group take K
    // values 16 h + 4 q + e (e = 0..3), one ds_read_b128 per operand tile
#pragma unroll
    for (int h = 0; h < kLwK / 16; ++h) {
      f32x4 av[2], bv[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        av[i] = *reinterpret_cast<const f32x4 *>(As + (wr + 16 * i + p) * kLwKP + 16 * h + 4 * q);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        bv[j] = *reinterpret_cast<const f32x4 *>(Bs + (wc + 16 * j + p) * kLwKP + 16 * h + 4 * q);
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i][e], bv[j][e], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
    if (more) {
      store();
      __syncthreads();
    }
  }
  // D layout: lane p + 16 q holds rows 4 q + rr, column p of each 16 x 16 tile
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int r = r0 + wr + 16 * i + 4 * q + rr;
      if (r >= g.R) continue;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int c = c0 + wc + 16 * j + p;
        if (c >= g.C) continue;
        const float v = acc[i][j][rr];
        switch (g.epi) {
          case kLwEpiHidden:
            g.out[static_cast<size_t>(r) * g.ldo + c] = fmaxf(v + g.bias[c], 0.0f);
            break;
          case kLwEpiOutput: {
            const float y = v + g.bias[c];
            if (g.out) {
              const size_t row = g.out_index ? g.out_index[r] : static_cast<uint32_t>(r);
              g.out[row * g.ldo + c] = y;
            }
            if (g.out2) g.out2[static_cast<size_t>(r) * g.ldo2 + c] = y;
            break;
          }
          case kLwEpiMask:
            g.out[static_cast<size_t>(r) * g.ldo + c] =
                g.mask[static_cast<size_t>(r) * g.ldm + c] > 0.0f ? v : 0.0f;
            break;
          case kLwEpiScale:
            g.out[static_cast<size_t>(r) * g.ldo + c] = v * g.scale;
            break;
          default:
            g.dst[blockIdx.z * g.dst_stride + g.dst_off + static_cast<int64_t>(r) * g.C + c] = v;
            break;
        }
      }
    }
}

struct LwLossArgs {
  int32_t n, M, mode, loss_kind, grad_output, chunk;
  float huber_delta, inv_n, loss_scale;
  const float *y;            // [n][M]
  const float *target;       // [rows][M]: targets (TrainLoss) or d_out (TrainExtGrad)
  const uint32_t *tgt_index; // nullable: point i's row is tgt_index[i]
  float *out;                // nullable: outputs [n][M] (kModeInputGrad: row i; training
                             // modes: row out_index[i] or i, the parity read-out of a step)
  const uint32_t *out_index; // nullable: caller row of point i (training modes)
  float *g;                  // [n][M] output gradients
  float *loss_partials;      // [chunks]
  float *amax_partials;      // nullable: [chunks] largest |output| of the chunk's points
};

// Output gradient and loss of each point (emitLoss, mlp_kernel_emitter.cpp:
// 562-670): block z takes the points of chunk z and writes that chunk's loss
// sum (threads in order, then lanes) -- a fixed order.
__global__ void __launch_bounds__(256) lw_loss_kernel(LwLossArgs a) {
  const int i0 = blockIdx.x * a.chunk, i1 = min(a.n, i0 + a.chunk);
  float lsum = 0.0f, amax = 0.0f;
  for (int i = i0 + threadIdx.x; i < i1; i += blockDim.x) {
    const float *y = a.y + static_cast<size_t>(i) * a.M;
    float *g = a.g + static_cast<size_t>(i) * a.M;
    if (a.mode == kModeInputGrad) {
      for (int o = 0; o < a.M; ++o) {
        if (a.out) a.out[static_cast<size_t>(i) * a.M + o] = y[o];
        g[o] = o == a.grad_output ? 1.0f : 0.0f;
      }
      continue;
    }
    const size_t row = a.tgt_index ? a.tgt_index[i] : static_cast<uint32_t>(i);
    const size_t orow = a.out_index ? a.out_index[i] : static_cast<uint32_t>(i);
    for (int o = 0; o < a.M; ++o) {
      amax = fmaxf(amax, fabsf(y[o]));
      if (a.out) a.out[orow * a.M + o] = y[o];
    }
    const float *t = a.target + row * a.M;
    if (a.mode == kModeTrainExtGrad) {
      for (int o = 0; o < a.M; ++o) g[o] = t[o] * a.loss_scale;
      continue;
    }
    if (a.loss_kind == kLossCosine) {
      // emitLoss cosine branch (mlp_kernel_emitter.cpp:643-662)
      float dot = 0.0f, pn = 0.0f, tn = 0.0f;
      for (int o = 0; o < a.M; ++o) {
        dot = dot + y[o] * t[o];
        pn = pn + y[o] * y[o];
        tn = tn + t[o] * t[o];
      }
      const float pnorm = sqrtf(pn + 1e-8f);
      const float tnorm = sqrtf(tn + 1e-8f);
      const float denom = pnorm * tnorm;
      const float cosine = dot / denom;
      const float pdenom = pn + 1e-8f;
      lsum += 1.0f - cosine;
      for (int o = 0; o < a.M; ++o) {
        const float t1 = (cosine * y[o]) / pdenom;
        const float t2 = t[o] / denom;
        g[o] = ((t1 - t2) * a.inv_n) * a.loss_scale;
      }
      continue;
    }
    for (int o = 0; o < a.M; ++o) {
      float d = 0.0f;
      switch (a.loss_kind) {
        case kLossL1: lsum += elem_loss<kLossL1, false>(y[o], t[o], a.huber_delta, a.inv_n, &d); break;
        case kLossHuber: lsum += elem_loss<kLossHuber, false>(y[o], t[o], a.huber_delta, a.inv_n, &d); break;
        case kLossRelL2: lsum += elem_loss<kLossRelL2, false>(y[o], t[o], a.huber_delta, a.inv_n, &d); break;
        default: lsum += elem_loss<kLossL2, false>(y[o], t[o], a.huber_delta, a.inv_n, &d); break;
      }
      g[o] = d * a.loss_scale;
    }
  }
  if (a.mode != kModeTrainLoss) return;
  __shared__ float red[256];
  red[threadIdx.x] = lsum;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (static_cast<int>(threadIdx.x) < s) red[threadIdx.x] += red[threadIdx.x + s];
    __syncthreads();
  }
  if (threadIdx.x == 0) a.loss_partials[blockIdx.x] = red[0];
  if (a.amax_partials == nullptr) return;
  __syncthreads();
  red[threadIdx.x] = amax;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (static_cast<int>(threadIdx.x) < s) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + s]);
    __syncthreads();
  }
  if (threadIdx.x == 0) a.amax_partials[blockIdx.x] = red[0];
}

}  // namespace tmnn_hip
