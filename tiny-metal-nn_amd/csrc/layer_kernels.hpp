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
  // 16-byte accesses allowed (lw_vec_ok; set by lw_set_vec): A rows (kLwARow,
  // kLwACol), B rows, and the epilogue's out / bias / mask rows
  int32_t a_vec, b_vec, o_vec;
};

constexpr int kLwTile = 64;
// Points per chunk of a layer-wise forward pass (inference has no batch cap):
// two activation buffers of kLwForwardChunk x H floats.
constexpr int kLwForwardChunk = 1 << 18;
constexpr int kLwK = 16;

template <int AM>
__device__ __forceinline__ float lw_a(const LwGemmArgs &g, int r, int k) {
  if (g.ones_row && r == g.R - 1) return 1.0f;
  if constexpr (AM == kLwARow) return g.A[static_cast<size_t>(r) * g.lda + k];
  if constexpr (AM == kLwACol) return g.A[static_cast<size_t>(k) * g.lda + r];
  if constexpr (AM == kLwAXTiles) return g.A[xtile_offset(r, k >> 2, g.KT0) + (k & 3)];
  return g.A[xtile_offset(k, r >> 2, g.KT0) + (r & 3)];
}

template <int BT>
__device__ __forceinline__ float lw_b(const LwGemmArgs &g, int k, int c) {
  if constexpr (BT != 0) return g.B[static_cast<size_t>(c) * g.ldb + k];
  return g.B[static_cast<size_t>(k) * g.ldb + c];
}

// LDS staging of one K step: row (or column) i of the tile holds its kLwK
// operands contiguously (kLwKP floats per row: 16-byte aligned and padded),
// so each lane reads the four K values of an MFMA A or B operand with one
// ds_read_b128.
constexpr int kLwKP = kLwK + 4;
// The output tile is staged through LDS for the epilogue (kLwCP floats per
// row), so each thread stores 16 consecutive columns of one row.
constexpr int kLwCP = kLwTile + 4;
constexpr int kLwSmem = kLwTile * kLwCP > 2 * kLwTile * kLwKP ? kLwTile * kLwCP : 2 * kLwTile * kLwKP;
static_assert(kLwTile * kLwK == 256 * 4, "one four-element quad per thread and operand");

// Whether A's and B's rows (of the layouts read with 16-byte loads: lda /
// ldb floats apart, 16-byte aligned) allow vector loads (host-side check).
inline bool lw_vec_ok(const float *ptr, int ld) {
  return ptr != nullptr && (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0 && ld % 4 == 0;
}

// One thread's quad of an operand tile for one K step. k-fast layouts (A
// rows, X tiles, B read transposed): quad = four consecutive K of one tile
// row, thread t takes row t / 4, K offset 4 (t % 4). Row-fast layouts (A
// read by columns, transposed X tiles, B in [K][C]): quad = four consecutive
// rows at one K, thread t takes K offset t / 16, rows 4 (t % 16) .. + 3.
// The four values of a quad lie contiguous in memory; a quad wholly inside
// the product (and aligned) is one 16-byte load, else four bounded scalar
// reads. Elements outside the product are zero.
template <int AM>
__device__ __forceinline__ f32x4 lw_load_a(const LwGemmArgs &g, int r0, int k0, int ke, bool &kfast,
                                           int &rr, int &kk) {
  const int t = threadIdx.x;
  kfast = AM == kLwARow || AM == kLwAXTiles;
  rr = kfast ? t >> 2 : (t & 15) * 4;
  kk = kfast ? (t & 3) * 4 : t >> 4;
  const int r = r0 + rr, k = k0 + kk;
  const int real_rows = g.R - (g.ones_row ? 1 : 0);  // rows read from A
  f32x4 v = {0.f, 0.f, 0.f, 0.f};
  if (kfast) {
    if (r >= g.R || k >= ke) return v;
    if (r < real_rows && k + 3 < ke && (AM == kLwAXTiles || g.a_vec)) {
      const float *src = AM == kLwAXTiles ? g.A + xtile_offset(r, k >> 2, g.KT0)
                                          : g.A + static_cast<size_t>(r) * g.lda + k;
      return *reinterpret_cast<const f32x4 *>(src);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (k + e < ke) v[e] = lw_a<AM>(g, r, k + e);
    return v;
  }
  if (k >= ke || r >= g.R) return v;
  if (r + 3 < real_rows && (AM == kLwAXTilesT || g.a_vec)) {
    const float *src = AM == kLwAXTilesT ? g.A + xtile_offset(k, r >> 2, g.KT0)
                                         : g.A + static_cast<size_t>(k) * g.lda + r;
    return *reinterpret_cast<const f32x4 *>(src);
  }
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (r + e < g.R) v[e] = lw_a<AM>(g, r + e, k);
  return v;
}

template <int BT>
__device__ __forceinline__ f32x4 lw_load_b(const LwGemmArgs &g, int c0, int k0, int ke, bool &kfast,
                                           int &cc, int &kk) {
  const int t = threadIdx.x;
  kfast = BT != 0;
  cc = kfast ? t >> 2 : (t & 15) * 4;
  kk = kfast ? (t & 3) * 4 : t >> 4;
  const int c = c0 + cc, k = k0 + kk;
  f32x4 v = {0.f, 0.f, 0.f, 0.f};
  if (kfast) {
    if (c >= g.C || k >= ke) return v;
    if (k + 3 < ke && g.b_vec)
      return *reinterpret_cast<const f32x4 *>(g.B + static_cast<size_t>(c) * g.ldb + k);
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (k + e < ke) v[e] = lw_b<BT>(g, k + e, c);
    return v;
  }
  if (k >= ke || c >= g.C) return v;
  if (c + 3 < g.C && g.b_vec)
    return *reinterpret_cast<const f32x4 *>(g.B + static_cast<size_t>(k) * g.ldb + c);
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (c + e < g.C) v[e] = lw_b<BT>(g, k, c + e);
  return v;
}

// Stores a quad into the LDS tile (row i's K values contiguous).
__device__ __forceinline__ void lw_stage(float *S, f32x4 v, bool kfast, int i, int kk) {
  if (kfast) {
    *reinterpret_cast<f32x4 *>(S + i * kLwKP + kk) = v;
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) S[(i + e) * kLwKP + kk] = v[e];
  }
}

// Epilogue of one output element (row r, column c, product value v).
template <int EPI>
__device__ __forceinline__ void lw_epilogue(const LwGemmArgs &g, int r, int c, float v) {
  if constexpr (EPI == kLwEpiHidden) {
    g.out[static_cast<size_t>(r) * g.ldo + c] = fmaxf(v + g.bias[c], 0.0f);
  } else if constexpr (EPI == kLwEpiOutput) {
    const float y = v + g.bias[c];
    if (g.out) {
      const size_t row = g.out_index ? g.out_index[r] : static_cast<uint32_t>(r);
      g.out[row * g.ldo + c] = y;
    }
    if (g.out2) g.out2[static_cast<size_t>(r) * g.ldo2 + c] = y;
  } else if constexpr (EPI == kLwEpiMask) {
    g.out[static_cast<size_t>(r) * g.ldo + c] = g.mask[static_cast<size_t>(r) * g.ldm + c] > 0.0f ? v : 0.0f;
  } else if constexpr (EPI == kLwEpiScale) {
    g.out[static_cast<size_t>(r) * g.ldo + c] = v * g.scale;
  } else {
    g.dst[blockIdx.z * g.dst_stride + g.dst_off + static_cast<int64_t>(r) * g.C + c] = v;
  }
}

// One instance per (A layout, B orientation, epilogue) the layer-wise path
// uses (lw_gemm_fn): compiled without the other modes' registers and branches.
template <int AM, int BT, int EPI>
__global__ void __launch_bounds__(256) lw_gemm_kernel(LwGemmArgs g) {
  // the tile's A rows and B columns of the current K step, K innermost; after
  // the products the same memory holds the output tile
  __shared__ __align__(16) float smem[kLwSmem];
  float *As = smem, *Bs = smem + kLwTile * kLwKP, *Cs = smem;
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
  // Operand staging, software-pipelined: the next K step's quads are read
  // from global memory into registers before the current step's products
  // and stored to LDS after them.
  bool akf, bkf;
  int ai, ak, bi, bk;
  f32x4 ra, rb;
  if (kb < ke) {
    ra = lw_load_a<AM>(g, r0, kb, ke, akf, ai, ak);
    rb = lw_load_b<BT>(g, c0, kb, ke, bkf, bi, bk);
    lw_stage(As, ra, akf, ai, ak);
    lw_stage(Bs, rb, bkf, bi, bk);
  }
  __syncthreads();
  for (int k0 = kb; k0 < ke; k0 += kLwK) {
    const bool more = k0 + kLwK < ke;  // uniform over the block
    if (more) {
      ra = lw_load_a<AM>(g, r0, k0 + kLwK, ke, akf, ai, ak);
      rb = lw_load_b<BT>(g, c0, k0 + kLwK, ke, bkf, bi, bk);
    }
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
      lw_stage(As, ra, akf, ai, ak);
      lw_stage(Bs, rb, bkf, bi, bk);
      __syncthreads();
    }
  }
  // the output tile through LDS (D layout: lane p + 16 q holds rows 4 q + rr,
  // column p of each 16 x 16 tile), then row-contiguous stores
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr)
        Cs[(wr + 16 * i + 4 * q + rr) * kLwCP + wc + 16 * j + p] = acc[i][j][rr];
  __syncthreads();
  const int er = tid >> 2, ecol = (tid & 3) * 16;  // this thread: 16 columns of one row
  const int r = r0 + er;
  if (r >= g.R) return;
#pragma unroll
  for (int gq = 0; gq < 4; ++gq) {
    const int c = c0 + ecol + 4 * gq;
    if (c >= g.C) break;
    const f32x4 v = *reinterpret_cast<const f32x4 *>(Cs + er * kLwCP + ecol + 4 * gq);
    constexpr bool kVecEpi = EPI == kLwEpiHidden || EPI == kLwEpiMask || EPI == kLwEpiScale;
    if (kVecEpi && c + 3 < g.C && g.o_vec) {
      f32x4 o;
      const size_t oi = static_cast<size_t>(r) * g.ldo + c;
      if constexpr (EPI == kLwEpiHidden) {
        const f32x4 b = *reinterpret_cast<const f32x4 *>(g.bias + c);
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = fmaxf(v[e] + b[e], 0.0f);
      } else if constexpr (EPI == kLwEpiMask) {
        const f32x4 m = *reinterpret_cast<const f32x4 *>(g.mask + static_cast<size_t>(r) * g.ldm + c);
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = m[e] > 0.0f ? v[e] : 0.0f;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = v[e] * g.scale;
      }
      *reinterpret_cast<f32x4 *>(g.out + oi) = o;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (c + e < g.C) lw_epilogue<EPI>(g, r, c + e, v[e]);
    }
  }
}

using LwGemmFn = void (*)(LwGemmArgs);

// The lw_gemm_kernel instance for g's modes (nullptr: a combination the
// layer-wise path does not use).
inline LwGemmFn lw_gemm_fn(const LwGemmArgs &g) {
  if (g.b_trans == 0 && g.epi == kLwEpiHidden)
    return g.a_mode == kLwAXTiles ? lw_gemm_kernel<kLwAXTiles, 0, kLwEpiHidden>
                                  : lw_gemm_kernel<kLwARow, 0, kLwEpiHidden>;
  if (g.b_trans == 0 && g.epi == kLwEpiOutput)
    return g.a_mode == kLwAXTiles ? lw_gemm_kernel<kLwAXTiles, 0, kLwEpiOutput>
                                  : lw_gemm_kernel<kLwARow, 0, kLwEpiOutput>;
  if (g.b_trans == 0 && g.epi == kLwEpiPartial)
    return g.a_mode == kLwAXTilesT ? lw_gemm_kernel<kLwAXTilesT, 0, kLwEpiPartial>
                                   : lw_gemm_kernel<kLwACol, 0, kLwEpiPartial>;
  if (g.b_trans != 0 && g.a_mode == kLwARow && g.epi == kLwEpiMask)
    return lw_gemm_kernel<kLwARow, 1, kLwEpiMask>;
  if (g.b_trans != 0 && g.a_mode == kLwARow && g.epi == kLwEpiScale)
    return lw_gemm_kernel<kLwARow, 1, kLwEpiScale>;
  return nullptr;
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
