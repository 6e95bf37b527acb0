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

// LDS staging of one K step, laid out so that neither the stores nor the
// MFMA operand reads meet a bank conflict. The LDS serves (measured on
// gfx950 with SQ_LDS_BANK_CONFLICT): 4-byte accesses 32 lanes per cycle
// (lanes 0-31, then 32-63) over 32 banks; 16-byte stores 8 consecutive
// lanes per cycle over 32 banks; 16-byte reads 16 lanes per cycle over 64
// banks, a cycle taking the lane quads (lane / 4) of even, then of odd bit
// parity among lanes 0-31 (0-3, 12-15, 20-23, 24-27 | 4-11, 16-19, 28-31),
// then the same in lanes 32-63. A k-fast operand (A rows, X tiles, B read
// transposed: a quad is four consecutive K of one row) sits row-major,
// [row][16], the four quads of a row permuted by an XOR with
// (-(row / 4)) % 4: 8 lanes storing two rows' quads cover 32 banks, and
// each 16-lane cycle of the operand read (lane p + 16 q: quad q of row p)
// covers the 64 banks once (the XOR with (row / 4) % 4 left two lanes of
// each cycle in one bank). A row-fast operand (A read by columns,
// transposed X tiles, B in [K][C]: a quad is four consecutive rows at one
// K) sits K-major, [16][kLwRS]: a quad is one 16-byte store (8 lanes: 32
// consecutive floats), and a lane reads its row's four K values with four
// scalar reads, each reaching 32 distinct banks per half wave.
constexpr int kLwRS = kLwTile + 4;         // row-fast K-major row stride (floats)
constexpr int kLwOpFloats = kLwK * kLwRS;  // one operand's region (>= kLwTile * kLwK)
// The output tile is staged through LDS for the epilogue (kLwCP floats per
// row), so each thread stores 16 consecutive columns of one row.
constexpr int kLwCP = kLwTile + 4;
// Two K steps (A and B regions each) are staged per pair of barriers.
constexpr int kLwSteps = 2;
constexpr int kLwSmem = kLwTile * kLwCP > 2 * kLwSteps * kLwOpFloats ? kLwTile * kLwCP
                                                                     : 2 * kLwSteps * kLwOpFloats;
static_assert(kLwOpFloats >= kLwTile * kLwK, "operand region");

// Float offset of quad kq (K values 4 kq .. 4 kq + 3) of row `row` of a
// k-fast operand.
__device__ __forceinline__ int lw_kfast_off(int row, int kq) {
  return row * kLwK + 4 * (kq ^ (-(row >> 2) & 3));
}
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

// Stores a quad into an operand's LDS region (k-fast: row i, K kk .. kk +
// 3; row-fast: rows i .. i + 3 at K kk).
__device__ __forceinline__ void lw_stage(float *S, f32x4 v, bool kfast, int i, int kk) {
  if (kfast)
    *reinterpret_cast<f32x4 *>(S + lw_kfast_off(i, kk >> 2)) = v;
  else
    *reinterpret_cast<f32x4 *>(S + kk * kLwRS + i) = v;
}

// The MFMA operand of lane p + 16 q for row `row`: K values 4 q .. 4 q + 3.
template <bool KFAST>
__device__ __forceinline__ f32x4 lw_frag(const float *S, int row, int q) {
  if constexpr (KFAST) {
    return *reinterpret_cast<const f32x4 *>(S + lw_kfast_off(row, q));
  } else {
    return f32x4{S[(4 * q) * kLwRS + row], S[(4 * q + 1) * kLwRS + row], S[(4 * q + 2) * kLwRS + row],
                 S[(4 * q + 3) * kLwRS + row]};
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
  // step h of a staged pair: A at smem + 2 h kLwOpFloats, B right after it
  float *Cs = smem;
  constexpr bool kAKFast = AM == kLwARow || AM == kLwAXTiles, kBKFast = BT != 0;
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
  // Operand staging, software-pipelined: the next pair of K steps' quads are
  // read from global memory into registers before the current pair's
  // products and stored to LDS after them (K past ke loads as zeros, so a
  // pair's second step may be empty).
  bool akf, bkf;
  int ai, ak, bi, bk;
  f32x4 ra[kLwSteps], rb[kLwSteps];
  auto load_pair = [&](int k) {
#pragma unroll
    for (int h = 0; h < kLwSteps; ++h) {
      ra[h] = lw_load_a<AM>(g, r0, k + h * kLwK, ke, akf, ai, ak);
      rb[h] = lw_load_b<BT>(g, c0, k + h * kLwK, ke, bkf, bi, bk);
    }
  };
  auto stage_pair = [&]() {
#pragma unroll
    for (int h = 0; h < kLwSteps; ++h) {
      lw_stage(smem + 2 * h * kLwOpFloats, ra[h], akf, ai, ak);
      lw_stage(smem + (2 * h + 1) * kLwOpFloats, rb[h], bkf, bi, bk);
    }
  };
  if (kb < ke) {
    load_pair(kb);
    stage_pair();
  }
  __syncthreads();
  for (int k0 = kb; k0 < ke; k0 += kLwSteps * kLwK) {
    const bool more = k0 + kLwSteps * kLwK < ke;  // uniform over the block
    if (more) load_pair(k0 + kLwSteps * kLwK);
    // v_mfma_f32_16x16x4_f32: lane p + 16 q supplies A[row p][k] and
    // B[k][column p] of K slot q; the four MFMAs of a K step take K values
    // 4 q + e (e = 0..3)
    static_assert(kLwK == 16, "one 16-wide K group per step");
#pragma unroll
    for (int h = 0; h < kLwSteps; ++h) {
      const float *As = smem + 2 * h * kLwOpFloats, *Bs = As + kLwOpFloats;
      f32x4 av[2], bv[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) av[i] = lw_frag<kAKFast>(As, wr + 16 * i + p, q);
#pragma unroll
      for (int j = 0; j < 2; ++j) bv[j] = lw_frag<kBKFast>(Bs, wc + 16 * j + p, q);
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
      stage_pair();
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

// ---- Narrow products: the output layer's three products have at most 16
// output columns (forward, weight gradient) or at most 16 K (delta), where a
// 64 x 64 tile would multiply 48 or more zero columns. Each is memory-bound
// (one pass over the batch's activations) and gets a kernel of its own
// shape; the host picks them (lw_narrow_*_ok) and falls back to
// lw_gemm_kernel otherwise. Their loads come from clamped, always valid
// addresses and out-of-range values are replaced by zeros afterwards, so
// the loads carry no branches and are issued in batches ahead of their use.
constexpr int kLwNarrow = 16;       // at most this many columns (forward, weight gradient) or K (delta)
constexpr int kLwNarrowMaxK = 512;  // forward: longest K whose B^T fits the block's LDS
constexpr int kLwNarrowKStep = 128; // forward: K per batch of A loads (8 quads per lane)

// Forward output layer y = A B + bias (kLwEpiOutput; A row-major with
// 16-byte aligned rows and K % 4 == 0, B[K][C], C <= 16, K <=
// kLwNarrowMaxK). B^T sits in LDS ([16][Kr], Kr = round128(K), zero beyond
// C and K), the 16-byte quads of row c permuted by an XOR of the quad index
// with c: the 16-byte read of lane p + 16 q (row p, quad 2 q + const) then
// lands in quad slot p ^ 2 q (mod 16), distinct within each 16-lane read
// cycle (lanes 0-3, 12-15 with q = 0 and 20-27 with q = 1, and the other
// three sets alike). Each wave computes 16 rows x 16 columns with
// v_mfma_f32_16x16x4_f32, reading A straight from global memory into the
// operand registers: for each 32 K, lane p + 16 q loads K values 8 q .. + 7
// of row p (the four lanes of a row read 128 contiguous bytes) and MFMA e of
// the eight takes K value 8 q + e in K slot q (a permutation of K applied to
// A and B alike). Two register sets of 128 K each alternate: one is loaded
// while the other feeds the MFMAs.
__global__ void __launch_bounds__(256) lw_narrow_out_kernel(LwGemmArgs g) {
  extern __shared__ __align__(16) float Bt[];
  const int Kr = (g.K + kLwNarrowKStep - 1) / kLwNarrowKStep * kLwNarrowKStep;
  // thread t of each 256-element batch: columns (t & 7) + 8 ((t >> 5) & 1),
  // K (t >> 3) & 3 + 4 (t >> 6): each half wave stores 8 columns x 4 K,
  // which k ^ 4c spreads over the 32 banks of a 4-byte store cycle
  for (int i = threadIdx.x; i < kLwNarrow * Kr; i += 256) {
    const int t = i & 255;
    const int c = (t & 7) | (((t >> 5) & 1) << 3);
    const int k = (i >> 8) * 16 + ((t >> 6) << 2) + ((t >> 3) & 3);
    // k ^ 4c stays inside k's 64-float block, so below Kr
    Bt[c * Kr + (k ^ (4 * c))] = (c < g.C && k < g.K) ? g.B[static_cast<size_t>(k) * g.ldb + c] : 0.0f;
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int p = lane & 15, q = lane >> 4;
  const int groups = (g.R + 15) / 16;
  const int kmax = g.K - 4;  // last quad of a row
  const float *brow = Bt + p * Kr;
  for (int grp = blockIdx.x * 4 + wave; grp < groups; grp += gridDim.x * 4) {
    // rows past R read row R - 1 and are not stored (row p of A feeds only
    // output row p)
    const float *arow = g.A + static_cast<size_t>(min(grp * 16 + p, g.R - 1)) * g.lda;
    auto load = [&](f32x4(&a)[8], int kb) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int k = kb + 32 * (i >> 1) + 8 * q + 4 * (i & 1);
        const f32x4 v = *reinterpret_cast<const f32x4 *>(arow + min(k, kmax));
        a[i] = k < g.K ? v : f32x4{0.f, 0.f, 0.f, 0.f};
      }
    };
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    auto product = [&](const f32x4(&a)[8], int kb) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int k = kb + 32 * (i >> 1) + 8 * q + 4 * (i & 1);  // this lane's quad of row p
        const f32x4 b = *reinterpret_cast<const f32x4 *>(brow + (k ^ (4 * p)));
#pragma unroll
        for (int e = 0; e < 4; ++e) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i][e], b[e], acc, 0, 0, 0);
      }
    };
    f32x4 x[8], y[8];
    load(x, 0);
    for (int kb = 0; kb < Kr; kb += 2 * kLwNarrowKStep) {
      if (kb + kLwNarrowKStep < Kr) load(y, kb + kLwNarrowKStep);
      product(x, kb);
      if (kb + kLwNarrowKStep >= Kr) break;
      if (kb + 2 * kLwNarrowKStep < Kr) load(x, kb + 2 * kLwNarrowKStep);
      product(y, kb + kLwNarrowKStep);
    }
    // D layout: lane p + 16 q holds rows 4 q + v, column p
    if (p < g.C) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = grp * 16 + 4 * q + v;
        if (row < g.R) lw_epilogue<kLwEpiOutput>(g, row, p, acc[v]);
      }
    }
  }
}

// Weight-gradient partial rows of the output layer (kLwEpiPartial, A read by
// columns: A(r, k) = act[k][r] with 16-byte aligned rows, B(k, c) = D[k][c],
// C <= 16, the rows read from A a multiple of 4, an all-ones last row when
// ones_row). Block (x, z): output rows 64 x .. + 63 over the points of
// chunk z; wave w takes the groups of four points 4 w + 16 j of the chunk,
// eight groups per batch of loads, and the four waves' sums are added in
// wave order at the end. Lane p + 16 q loads rows 4 p .. + 3 of point k + q
// (one 16-byte load; the 16 lanes of a point read 256 contiguous bytes) and
// feeds row 4 p + e to MFMA tile e, so output row 4 (4 q + v) + e of the
// block comes back in lane p + 16 q, element v of tile e. A and D are read
// through raw buffer resources over the chunk's points: points past the
// chunk, rows past A's and columns past C lie outside the range and read as
// zeros (chunk bytes < 2^31, a host check).
constexpr uint32_t kLwOutside = 0x80000000u;  // a buffer offset past every range
__device__ __forceinline__ __amdgpu_buffer_rsrc_t lw_rsrc(const float *base, int64_t bytes) {
  // dword 3: 32-bit data format, the raw-buffer setting of gfx9 parts
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(base), 0, static_cast<int>(bytes),
                                           0x00020000);
}
__global__ void __launch_bounds__(256) lw_narrow_wgrad_kernel(LwGemmArgs g) {
  __shared__ f32x4 red[3][4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int p = lane & 15, q = lane >> 4;
  const int real_rows = g.R - (g.ones_row ? 1 : 0);  // rows read from A
  const int u = blockIdx.x * 64 + 4 * p;              // this lane's first row
  const bool ones = g.ones_row && u == real_rows;     // element 0 is the all-ones row
  const bool col = p < g.C;
  const int kb = blockIdx.z * g.k_chunk;
  const int ke = min(g.K, kb + g.k_chunk);
  const int64_t points = max(ke - kb, 0);  // an empty last chunk reads nothing
  const __amdgpu_buffer_rsrc_t ar = lw_rsrc(g.A + static_cast<size_t>(kb) * g.lda, points * g.lda * 4);
  const __amdgpu_buffer_rsrc_t br = lw_rsrc(g.B + static_cast<size_t>(kb) * g.ldb, points * g.ldb * 4);
  // byte offsets of point kb + q; rows past A and columns past C never in range
  const uint32_t a_off = u < real_rows ? static_cast<uint32_t>(q * g.lda + u) * 4u : kLwOutside;
  const uint32_t b_off = col ? static_cast<uint32_t>(q * g.ldb + p) * 4u : kLwOutside;
  f32x4 acc[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) acc[e] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int k0 = 4 * wave; k0 < ke - kb; k0 += 128) {
    f32x4 a[8];
    float b[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int kr = k0 + 16 * j;  // chunk-relative point of K slot 0
      const uint32_t ka = static_cast<uint32_t>(kr * g.lda) * 4u, kbo = static_cast<uint32_t>(kr * g.ldb) * 4u;
      a[j] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(ar, a_off + ka, 0, 0));
      b[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(br, b_off + kbo, 0, 0));
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (ones) a[j][0] = kb + k0 + 16 * j + q < ke ? 1.0f : 0.0f;
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j][e], b[j], acc[e], 0, 0, 0);
    }
  }
  if (wave > 0) {
#pragma unroll
    for (int e = 0; e < 4; ++e) red[wave - 1][e][lane] = acc[e];
  }
  __syncthreads();
  if (wave > 0 || !col) return;
  float *dst = g.dst + blockIdx.z * g.dst_stride + g.dst_off;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const f32x4 s = acc[e] + red[0][e][lane] + red[1][e][lane] + red[2][e][lane];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int r = blockIdx.x * 64 + 4 * (4 * q + v) + e;
      if (r < g.R) dst[static_cast<int64_t>(r) * g.C + p] = s[v];
    }
  }
}

// Delta through the output layer: out[r][c] = mask[r][c] > 0 ? sum_{k < K}
// A[r][k] B(k, c) : 0 with B read transposed (B(k, c) = W[c][k]), K <= 16,
// C % 4 == 0 and 16-byte aligned out / mask rows. Block (x, y): rows
// kLwNarrowRows x .. + kLwNarrowRows - 1 and columns 256 y .. + 255, whose A
// rows and W slice sit in LDS; thread t takes the column quad 4 (t % 64) of
// the rows t / 64 + 4 j (j = 0 .. 7), all eight mask loads issued first.
constexpr int kLwNarrowRows = 32;
__global__ void __launch_bounds__(256) lw_narrow_mask_kernel(LwGemmArgs g) {
  __shared__ __align__(16) float Ws[kLwNarrow][256];
  __shared__ float As[kLwNarrowRows][kLwNarrow];
  const int c0 = blockIdx.y * 256, rb = blockIdx.x * kLwNarrowRows;
  for (int i = threadIdx.x; i < kLwNarrow * 256; i += 256) {
    const int k = i / 256, cc = i % 256;  // columns fastest: conflict-free LDS stores
    Ws[k][cc] = (k < g.K && c0 + cc < g.C) ? g.B[static_cast<size_t>(c0 + cc) * g.ldb + k] : 0.0f;
  }
  for (int i = threadIdx.x; i < kLwNarrowRows * kLwNarrow; i += 256) {
    const int rr = i / kLwNarrow, k = i % kLwNarrow;
    As[rr][k] = (k < g.K && rb + rr < g.R) ? g.A[static_cast<size_t>(rb + rr) * g.lda + k] : 0.0f;
  }
  __syncthreads();
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const int c = c0 + 4 * tx;
  if (c >= g.C) return;
  constexpr int kRows = kLwNarrowRows / 4;
  f32x4 m[kRows];
#pragma unroll
  for (int j = 0; j < kRows; ++j) {
    const int r = min(rb + ty + 4 * j, g.R - 1);
    m[j] = *reinterpret_cast<const f32x4 *>(g.mask + static_cast<size_t>(r) * g.ldm + c);
  }
#pragma unroll
  for (int j = 0; j < kRows; ++j) {
    const int rr = ty + 4 * j;
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
    for (int k = 0; k < g.K; ++k) {
      const float a = As[rr][k];
      const f32x4 w = *reinterpret_cast<const f32x4 *>(&Ws[k][4 * tx]);
#pragma unroll
      for (int e = 0; e < 4; ++e) s[e] = fmaf(a, w[e], s[e]);
    }
    f32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = m[j][e] > 0.0f ? s[e] : 0.0f;
    if (rb + rr < g.R) *reinterpret_cast<f32x4 *>(g.out + static_cast<size_t>(rb + rr) * g.ldo + c) = o;
  }
}

// Host-side checks that a product has the narrow kernels' form (a_vec / o_vec
// as set for the generic kernel).
inline bool lw_narrow_out_ok(const LwGemmArgs &g) {
  return g.epi == kLwEpiOutput && g.a_mode == kLwARow && g.b_trans == 0 && g.C <= kLwNarrow &&
         g.K >= 4 && g.K % 4 == 0 && g.K <= kLwNarrowMaxK && g.k_chunk >= g.K && g.a_vec &&
         !g.ones_row;
}
inline bool lw_narrow_wgrad_ok(const LwGemmArgs &g) {
  const int real_rows = g.R - (g.ones_row ? 1 : 0);
  const int64_t chunk_bytes = static_cast<int64_t>(g.k_chunk + 128) * std::max(g.lda, g.ldb) * 4;
  return g.epi == kLwEpiPartial && g.a_mode == kLwACol && g.b_trans == 0 && g.C <= kLwNarrow &&
         real_rows >= 4 && real_rows % 4 == 0 && g.a_vec && chunk_bytes < (int64_t{1} << 31);
}
inline bool lw_narrow_mask_ok(const LwGemmArgs &g) {
  return g.epi == kLwEpiMask && g.a_mode == kLwARow && g.b_trans != 0 && g.K <= kLwNarrow &&
         g.C % 4 == 0 && g.o_vec && !g.ones_row && g.k_chunk >= g.K;
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
