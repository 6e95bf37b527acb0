// wide_kernel.hpp -- the field kernel for hidden width 128 (
// 32 -> 128 x4 -> 4).
//
// The split-fp16 forward needs hi + lo weight fragments (4 B per weight) and
// the backward another fp16 copy: ~330 KB at 128 wide, more than a CU's LDS.
// So this kernel is block-cooperative: four waves each own a 32-point tile of
// a 128-point block tile, and walk the layers together; before each layer
// the block copies that layer's fragments (from the packed image in global
// memory, L2-resident) into LDS, behind a barrier. Activations stay in
// registers in the forward; the hidden activations also go to global memory
// (fp16, tile-blocked [layer][tile][unit][32 points]) with their ReLU masks
// as one 64-bit word per lane, for the backward.
//
// Weight gradients: per hidden layer the block stages delta and the layer's
// input (fp16) for all 128 points in LDS ([unit][point]), and each wave
// multiplies the rows it owns -- units [32w, 32w+32) -- over the 128 points
// into MFMA accumulators that live in registers across all block tiles. Each
// dW element has exactly one owner, so the per-block partial row needs no
// cross-wave reduction; biases are summed per owned unit from the same stage
// in a fixed order. Deterministic.
//
// Modes: training (fp16 only), the evaluator's input gradient (fp32 or
// fp16; no weight gradients) and forward (fp32 inference, fp16 forward for
// training). Reference math: as field_kernel.hpp.
#pragma once

#include "field_kernel.hpp"

namespace tmnn_hip {

constexpr int kWideHP = 128;
constexpr int kWideHT = kWideHP / 16;
constexpr int kWideWaves = 4;
constexpr int kBlockPts = kWideWaves * kTilePts;  // points per block tile
constexpr int kSPS = kBlockPts + 8;               // stage row stride (fp16 elements)

// LDS plan of the wide kernel (bytes). The weight buffer and the gradient
// stage are never live at the same time and share offset 0.
struct WideLayout {
  int32_t region;  // max(weight buffer, stage)
  int32_t stage_h; // offset of the input stage inside the region
  int32_t bias;    // fp32 biases of every layer (copied from the image)
  int32_t res;     // fp32 resolution table
  int32_t red;     // per-wave loss slots
  int32_t total;
};

__host__ __device__ __forceinline__ WideLayout make_wide_layout(const FieldLayout &fl, bool f16, bool train) {
  WideLayout w;
  const int es = f16 ? 2 : 4;
  const int wbuf = (f16 ? 2 : 1) * kWideHP * kWideHP * es;  // largest layer's forward fragments
  const int bwd = kWideHP * kWideHP * es;
  const int stage = (train && f16) ? 2 * kWideHP * kSPS * 2 : 0;
  w.region = wbuf > bwd ? wbuf : bwd;
  if (stage > w.region) w.region = stage;
  w.stage_h = kWideHP * kSPS * 2;
  w.bias = w.region;
  w.res = w.bias + (fl.res_off - fl.bias_base);
  w.red = w.res + kMaxLevels * 4;
  w.total = w.red + kWideWaves * 4;
  return w;
}

// D-layout tiles -> fp16 rows of a block stage: unit row0 + 16*mt + 4*q + r,
// point pt0 + 16*nt + p.
template <int MT>
__device__ __forceinline__ void stage_store(unsigned char *st, const f32x4 (&t)[MT][kNT],
                                            int row0, int pt0, int p, int q) {
  _Float16 *h = reinterpret_cast<_Float16 *>(st);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        h[(row0 + 16 * mt + 4 * q + r) * kSPS + pt0 + 16 * nt + p] =
            static_cast<_Float16>(t[mt][nt][r]);
}

// acc + sum over the block tile's 128 points of A[arow + i][pt] * B[brow + j][pt].
__device__ __forceinline__ f32x4 dw_stage(const unsigned char *A, int arow,
                                          const unsigned char *B, int brow, int p, int q,
                                          f32x4 acc) {
#pragma unroll
  for (int s = 0; s < kBlockPts / 32; ++s) {
    const half8 av = *reinterpret_cast<const half8 *>(A + ((arow + p) * kSPS + 32 * s + 8 * q) * 2);
    const half8 bv = *reinterpret_cast<const half8 *>(B + ((brow + p) * kSPS + 32 * s + 8 * q) * 2);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, acc, 0, 0, 0);
  }
  return acc;
}

// Sum over the block tile's points of stage row `row` (lane pair 2u, 2u+1
// splits the points; fixed order).
__device__ __forceinline__ float stage_row_sum(const unsigned char *A, int row, int lane) {
  const _Float16 *h = reinterpret_cast<const _Float16 *>(A) + row * kSPS + (lane & 1) * (kBlockPts / 2);
  float s = 0.0f;
#pragma unroll
  for (int c = 0; c < kBlockPts / 2 / 8; ++c) {
    const half8 v = *reinterpret_cast<const half8 *>(h + 8 * c);
#pragma unroll
    for (int j = 0; j < 8; ++j) s += static_cast<float>(v[j]);
  }
  return s + __shfl_xor(s, 1);
}

// ReLU mask bits of a D-layout hidden tile set (bit (mt*kNT + nt)*4 + r).
__device__ __forceinline__ uint64_t relu_bits(const f32x4 (&t)[kWideHT][kNT]) {
  uint64_t b = 0;
#pragma unroll
  for (int mt = 0; mt < kWideHT; ++mt)
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (t[mt][nt][r] > 0.0f) b |= 1ull << ((mt * kNT + nt) * 4 + r);
  return b;
}

__device__ __forceinline__ void apply_bits(f32x4 (&t)[kWideHT][kNT], uint64_t b) {
#pragma unroll
  for (int mt = 0; mt < kWideHT; ++mt)
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (!((b >> ((mt * kNT + nt) * 4 + r)) & 1ull)) t[mt][nt][r] = 0.0f;
}

// XMEM: input features read from a.xfeat (encode_features_kernel) instead
// of encoded here.
template <int D, int F, int NHL, bool F16, bool TRAIN, bool XMEM>
__global__ void __launch_bounds__(kWideWaves * 64)
    __attribute__((amdgpu_waves_per_eu(1, 1))) wide_kernel(FieldArgs a) {
  constexpr int HT = kWideHT;
  constexpr int INP = 32;
  constexpr int KT0 = INP / 16;
  constexpr int OKT = F16 ? 2 : 1;
  constexpr int DF = D * 8 + F;
  constexpr bool kWgrad = TRAIN && F16;  // weight gradients are built for fp16 only
  extern __shared__ __align__(16) unsigned char smem[];

  const FieldLayout fl = make_layout(INP, kWideHP, a.IN, a.H, NHL, a.M, a.mlp_count, F16,
                                     TRAIN, 1);
  const WideLayout wl = make_wide_layout(fl, F16, TRAIN);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int p = lane & 15, q = lane >> 4;
  // biases + resolution table stay in LDS for the whole launch
  copy_to_lds(smem + wl.bias, a.image + fl.bias_base, fl.dw_off - fl.bias_base);
  __syncthreads();
  const float *res = reinterpret_cast<const float *>(smem + wl.res);
  const bool wgrads = kWgrad && a.mode != kModeInputGrad;

  // owned weight-gradient tiles: hidden units [32w, 32w + 32) of every layer
  f32x4 acc0[2][KT0];                              // layer 0: rows u, cols input features
  f32x4 acch[NHL > 1 ? NHL - 1 : 1][2][HT];        // layers 1..NHL-1
  f32x4 acco[2];                                   // output: rows outputs, cols units
  float dbias[NHL + 1];                            // unit 32w + lane/2 of each layer
  if constexpr (kWgrad) {
#pragma unroll
    for (int uu = 0; uu < 2; ++uu) {
#pragma unroll
      for (int ft = 0; ft < KT0; ++ft) acc0[uu][ft] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < (NHL > 1 ? NHL - 1 : 1); ++k)
#pragma unroll
        for (int it = 0; it < HT; ++it) acch[k][uu][it] = f32x4{0.f, 0.f, 0.f, 0.f};
      acco[uu] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int k = 0; k <= NHL; ++k) dbias[k] = 0.0f;
  }
  float lane_loss = 0.0f, lane_amax = 0.0f;
  const int pt0 = wave * kTilePts;  // this wave's points inside the block stage
  const int n_btiles = (a.n_tiles + kWideWaves - 1) / kWideWaves;
  unsigned char *stage_d = smem;
  unsigned char *stage_h = smem + wl.stage_h;

  for (int bt = blockIdx.x; bt < n_btiles; bt += gridDim.x) {
    const int tile = bt * kWideWaves + wave;  // may lie past the batch: then all points invalid
    int pt[kNT];
    bool valid[kNT];
    float P[kNT][4];
    float Tv[kNT][4];
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt) {
      pt[nt] = tile * kTilePts + 16 * nt + p;
      valid[nt] = tile < a.n_tiles && pt[nt] < a.n;
#pragma unroll
      for (int d = 0; d < 4; ++d)
        P[nt][d] = (!XMEM && valid[nt] && d < D) ? a.pos[static_cast<size_t>(pt[nt]) * D + d] : 0.0f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int o = 4 * q + r;
        Tv[nt][r] = (TRAIN && a.mode != kModeInputGrad && valid[nt] && o < a.M)
                        ? a.target[static_cast<size_t>(a.tgt_index ? a.tgt_index[pt[nt]]
                                                                   : static_cast<uint32_t>(pt[nt])) *
                                       a.M + o]
                        : 0.0f;
      }
    }
    f32x4 X[KT0][kNT];
    if constexpr (XMEM) {
      const f32x4 *xt = reinterpret_cast<const f32x4 *>(a.xfeat);
#pragma unroll
      for (int kt = 0; kt < KT0; ++kt)
#pragma unroll
        for (int nt = 0; nt < kNT; ++nt)
          X[kt][nt] = tile < a.n_tiles
                          ? xt[((static_cast<size_t>(tile) * KT0 + kt) * kNT + nt) * 64 + lane]
                          : f32x4{0.f, 0.f, 0.f, 0.f};
    } else {
      encode_tile<KT0, DF>(a, res, q, P, X);
    }

    // ---- forward, one layer's weights in LDS at a time
    f32x4 act[HT][kNT];
    f32x4 y[1][kNT];
    const size_t tile_slot = static_cast<size_t>(tile < a.n_tiles ? tile : 0);
#pragma unroll
    for (int k = 0; k <= NHL; ++k) {
      const int kin = k == 0 ? INP : kWideHP;
      const int mout = k == NHL ? 16 : kWideHP;
      const int fbytes = kin * mout * (F16 ? 2 : 4);
      __syncthreads();  // everyone is done with the previous layer's buffer
      copy_to_lds(smem, a.image + fl.fwd_off(k), fbytes);
      if constexpr (F16) copy_to_lds(smem + fbytes, a.image + fl.fwd_lo_off(k), fbytes);
      __syncthreads();
      if (k == NHL) {
        if constexpr (F16)
          layer_mma_split<HT, 1>(smem, smem + fbytes, act, y, lane);
        else
          layer_mma<false, HT, 1>(smem, act, y, lane);
        break;
      }
      f32x4 nxt[HT][kNT];
      if (k == 0) {
        if constexpr (F16)
          layer_mma_split<KT0, HT>(smem, smem + fbytes, X, nxt, lane);
        else
          layer_mma<false, KT0, HT>(smem, X, nxt, lane);
      } else {
        if constexpr (F16)
          layer_mma_split<HT, HT>(smem, smem + fbytes, act, nxt, lane);
        else
          layer_mma<false, HT, HT>(smem, act, nxt, lane);
      }
      const float *bias = reinterpret_cast<const float *>(smem + wl.bias + k * kWideHP * 4);
#pragma unroll
      for (int mt = 0; mt < HT; ++mt)
#pragma unroll
        for (int nt = 0; nt < kNT; ++nt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float v = nxt[mt][nt][r] + bias[16 * mt + 4 * q + r];
            act[mt][nt][r] = v > 0.0f ? v : 0.0f;
          }
      if constexpr (TRAIN) {
        if (k < NHL - 1) {
          // hidden input of layer k + 1, for the backward: mask bits and fp16 values
          if (tile < a.n_tiles)
            a.wide_mask[(static_cast<size_t>(k) * a.n_tiles + tile_slot) * 64 + lane] = relu_bits(act);
          if (wgrads && tile < a.n_tiles) {
            _Float16 *hg = a.wide_act + (static_cast<size_t>(k) * a.n_tiles + tile_slot) * kWideHP * kTilePts;
#pragma unroll
            for (int mt = 0; mt < HT; ++mt)
#pragma unroll
              for (int nt = 0; nt < kNT; ++nt)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                  hg[(16 * mt + 4 * q + r) * kTilePts + 16 * nt + p] =
                      static_cast<_Float16>(act[mt][nt][r]);
          }
        }
      }
    }
    {
      const float *bias = reinterpret_cast<const float *>(smem + wl.bias + NHL * kWideHP * 4);
#pragma unroll
      for (int nt = 0; nt < kNT; ++nt)
#pragma unroll
        for (int r = 0; r < 4; ++r) y[0][nt][r] = y[0][nt][r] + bias[4 * q + r];
    }

    if constexpr (!TRAIN) {
#pragma unroll
      for (int nt = 0; nt < kNT; ++nt) {
        if (!valid[nt]) continue;
        const size_t row = a.out_index ? a.out_index[pt[nt]] : static_cast<size_t>(pt[nt]);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int o = 4 * q + r;
          if (o < a.M) a.out[row * a.M + o] = y[0][nt][r];
        }
      }
      continue;
    } else {
      f32x4 g[OKT][kNT];
      output_grad<OKT>(a, y, Tv, valid, pt, q, lane_loss, lane_amax, g);
#pragma unroll
      for (int nt = 0; nt < kNT; ++nt)
        if (!valid[nt])
#pragma unroll
          for (int t = 0; t < OKT; ++t) g[t][nt] = f32x4{0.f, 0.f, 0.f, 0.f};

      // ---- output layer: dW_out over the block stage, then delta of the last hidden layer
      const uint64_t last_bits = relu_bits(act);
      if constexpr (kWgrad) {
        if (wgrads) {
          __syncthreads();
          {
            f32x4 g0[1][kNT];
#pragma unroll
            for (int nt = 0; nt < kNT; ++nt) g0[0][nt] = g[0][nt];
            stage_store<1>(stage_d, g0, 0, pt0, p, q);
          }
          stage_store<HT>(stage_h, act, 0, pt0, p, q);
          __syncthreads();
#pragma unroll
          for (int uu = 0; uu < 2; ++uu)
            acco[uu] = dw_stage(stage_d, 0, stage_h, 16 * (2 * wave + uu), p, q, acco[uu]);
          if (wave == 0 && lane < 32) dbias[NHL] += stage_row_sum(stage_d, lane >> 1, lane);
        }
      }
      f32x4 dl[HT][kNT];
      {
        const int kin = kWideHP, ko = F16 ? 32 : 16;
        __syncthreads();
        copy_to_lds(smem, a.image + fl.bwd_off(NHL), kin * ko * (F16 ? 2 : 4));
        __syncthreads();
        layer_mma<F16, OKT, HT>(smem, g, dl, lane);
        apply_bits(dl, last_bits);
      }

      // ---- hidden layers NHL-1 .. 1
#pragma unroll
      for (int k = NHL - 1; k >= 1; --k) {
        const uint64_t bits =
            a.wide_mask[(static_cast<size_t>(k - 1) * a.n_tiles + tile_slot) * 64 + lane];
        if constexpr (kWgrad) {
          if (wgrads) {
            __syncthreads();
            stage_store<HT>(stage_d, dl, 0, pt0, p, q);
            {
              // this wave's 32-point slice of h_{k-1}: 128 rows x 64 bytes
              const uint4 *src = reinterpret_cast<const uint4 *>(
                  a.wide_act + (static_cast<size_t>(k - 1) * a.n_tiles + tile_slot) * kWideHP * kTilePts);
#pragma unroll
              for (int j = 0; j < 8; ++j) {
                const int c = lane + 64 * j;  // 16-byte chunk: row c / 4, part c % 4
                uint4 v = make_uint4(0u, 0u, 0u, 0u);
                if (tile < a.n_tiles) v = src[c];
                *reinterpret_cast<uint4 *>(stage_h + ((c >> 2) * kSPS + pt0 + 8 * (c & 3)) * 2) = v;
              }
            }
            __syncthreads();
#pragma unroll
            for (int uu = 0; uu < 2; ++uu)
#pragma unroll
              for (int it = 0; it < HT; ++it)
                acch[k - 1][uu][it] =
                    dw_stage(stage_d, 16 * (2 * wave + uu), stage_h, 16 * it, p, q, acch[k - 1][uu][it]);
            if (lane < 64) dbias[k] += stage_row_sum(stage_d, 32 * wave + (lane >> 1), lane);
          }
        }
        __syncthreads();
        copy_to_lds(smem, a.image + fl.bwd_off(k), kWideHP * kWideHP * (F16 ? 2 : 4));
        __syncthreads();
        f32x4 nd[HT][kNT];
        layer_mma<F16, HT, HT>(smem, dl, nd, lane);
        apply_bits(nd, bits);
#pragma unroll
        for (int mt = 0; mt < HT; ++mt)
#pragma unroll
          for (int nt = 0; nt < kNT; ++nt) dl[mt][nt] = nd[mt][nt];
      }

      // ---- layer 0: dW0 over the stage, then dx
      if constexpr (kWgrad) {
        if (wgrads) {
          __syncthreads();
          stage_store<HT>(stage_d, dl, 0, pt0, p, q);
          stage_store<KT0>(stage_h, X, 0, pt0, p, q);
          __syncthreads();
#pragma unroll
          for (int uu = 0; uu < 2; ++uu)
#pragma unroll
            for (int ft = 0; ft < KT0; ++ft)
              acc0[uu][ft] = dw_stage(stage_d, 16 * (2 * wave + uu), stage_h, 16 * ft, p, q, acc0[uu][ft]);
          dbias[0] += stage_row_sum(stage_d, 32 * wave + (lane >> 1), lane);
        }
      }
      __syncthreads();
      copy_to_lds(smem, a.image + fl.bwd_off(0), INP * kWideHP * (F16 ? 2 : 4));
      __syncthreads();
      f32x4 dx[KT0][kNT];
      layer_mma<F16, HT, KT0>(smem, dl, dx, lane);
#pragma unroll
      for (int nt = 0; nt < kNT; ++nt) {
        if (!valid[nt]) continue;
        float *row = a.dx_out + static_cast<size_t>(pt[nt]) * a.IN;
#pragma unroll
        for (int kt = 0; kt < KT0; ++kt) {
          const int f0 = 16 * kt + 4 * q;
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (f0 + r < a.IN) row[f0 + r] = dx[kt][nt][r] * a.inv_loss_scale;
        }
      }
    }
  }

  if constexpr (TRAIN) {
    if (a.mode == kModeInputGrad) return;  // uniform: no loss, no weight gradients
    __syncthreads();
    block_loss_partials(a, lane_loss, lane_amax, reinterpret_cast<float *>(smem + wl.red), lane,
                        wave, kWideWaves);
    if constexpr (kWgrad) {
      // each dW element has one owner: write this block's partial row directly
      float *dst = a.grad_partials + static_cast<size_t>(blockIdx.x) * a.mlp_count;
      const float sc = a.inv_loss_scale;
      const int H = a.H, IN = a.IN, M = a.M;
#pragma unroll
      for (int uu = 0; uu < 2; ++uu) {
        const int ut = 2 * wave + uu;
#pragma unroll
        for (int ft = 0; ft < KT0; ++ft)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int u = 16 * ut + 4 * q + r, f = 16 * ft + p;
            if (u < H && f < IN) dst[fl.w_off(0) + f * H + u] = acc0[uu][ft][r] * sc;
          }
#pragma unroll
        for (int k = 1; k < NHL; ++k)
#pragma unroll
          for (int it = 0; it < HT; ++it)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int u = 16 * ut + 4 * q + r, i = 16 * it + p;
              if (u < H && i < H) dst[fl.w_off(k) + i * H + u] = acch[k - 1][uu][it][r] * sc;
            }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int o = 4 * q + r, u = 16 * ut + p;
          if (o < M && u < H) dst[fl.w_off(NHL) + u * M + o] = acco[uu][r] * sc;
        }
      }
      // biases: lane pair (2j, 2j+1) holds unit 32w + j
      if ((lane & 1) == 0) {
        const int u = 32 * wave + (lane >> 1);
#pragma unroll
        for (int k = 0; k < NHL; ++k)
          if (u < H) dst[fl.b_off(k) + u] = dbias[k] * sc;
        if (wave == 0 && (lane >> 1) < M && lane < 32) dst[fl.b_off(NHL) + (lane >> 1)] = dbias[NHL] * sc;
      }
    }
  }
}

}  // namespace tmnn_hip
