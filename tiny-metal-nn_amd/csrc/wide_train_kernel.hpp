// wide_train_kernel.hpp -- fp16 training kernel of the hidden-width-128 MLP
// (32 -> 128 x NHL -> M), on the scheme of
// mlp_train_kernel (mlp_kernel.hpp): transposes on the matrix cores, owned
// weight-gradient tiles accumulated in registers over all rounds, packed fp16
// ReLU' factors, 16-byte lane-private LDS parking slots.
//
// Two things differ from the 64-wide kernel because a 128-wide layer's
// operands are 4x larger:
//  * weights: the split-fp16 forward fragments of one hidden layer (hi + lo,
//    64 KB) plus the backward copy exceed what LDS can hold for every layer,
//    so the block stages one layer's fragments at a time from the packed
//    image (direct global-to-LDS loads, behind barriers);
//  * activations: the packed fp16 activations of hidden layers 0 .. NHL-2
//    (the D-layout B operands, 8 KB per tile and layer) go to global memory
//    in the forward and come back in the backward, where they give both the
//    ReLU' factors and (transposed on the matrix cores) the dW operands; the
//    last hidden layer's stay in registers.
//
// Per round each of the four waves (one per SIMD) owns a 32-point tile. The
// backward parks, per layer, every wave's transposed deltas and layer inputs;
// after a barrier each wave accumulates the dW tiles it owns over all four
// waves' points in wave order (deterministic, no cross-wave reduction), and
// the owners write the block's partial row at the end. Numerics as
// mlp_train_kernel: split-fp16 forward with the bias as the accumulator's
// initial value, fp16 backward with a power-of-two loss scale, ReLU' from the
// fp16 activation. Bias gradients are fp32 sums of the parked fp16 delta^T
// tiles (v_dot2 against ones; the owner of unit tile ut is wave ut % 4, the
// four lanes of a unit are added at the end in a fixed order), which keeps
// them out of the MFMA accumulators.
#pragma once

#include "mlp_kernel.hpp"
#include "wide_kernel.hpp"

namespace tmnn_hip {

// LDS plan of wide_train_kernel (bytes): one layer's staged weight fragments,
// the biases of every layer (fp32, image order), the per-wave loss slots,
// then per wave its parking slots (16 bytes per lane each): [0, 8) delta^T
// tiles, [8, 16) layer-input^T tiles, 16 the output gradient^T; then per
// wave its owned dW_0 and dW_out accumulators (kWideAccSlots f32x4 per lane),
// which are live only during their layer's owner jobs.
constexpr int kWideAccSlots = 6;  // dW_0: 2 * 8 / 4 tiles, dW_out: 8 / 4

struct WideTrainLds {
  int32_t bias, loss, park, park_bytes, acc, total;
};

__host__ __device__ __forceinline__ WideTrainLds wide_train_lds(const FieldLayout &s) {
  WideTrainLds m;
  m.bias = 2 * kWideHP * kWideHP * 2;  // a hidden layer's forward hi + lo fragments
  m.loss = m.bias + round_up(s.res_off - s.bias_base, 16);
  m.park = m.loss + 16 * 4;
  m.park_bytes = (2 * kWideHT + 1) * 64 * 16;
  m.acc = m.park + kWideWaves * m.park_bytes;
  m.total = m.acc + kWideWaves * kWideAccSlots * 64 * 16;
  return m;
}

template <int NHL>
__global__ void __launch_bounds__(kWideWaves * 64)
    __attribute__((amdgpu_waves_per_eu(1, 1))) wide_train_kernel(FieldArgs a) {
  constexpr int HP = kWideHP;
  constexpr int HT = HP / 16;  // unit tiles of a hidden layer
  constexpr int HS = HT / 2;   // K steps over a hidden layer
  constexpr int INP = 32;
  constexpr int KT0 = INP / 16;
  constexpr int XS = KT0 / 2;
  constexpr int W = kWideWaves;
  static_assert(NHL >= 2, "at least two hidden layers");
  constexpr int kJobsOut = HT;        // dW_out tiles (units x outputs)
  constexpr int kJobsHid = HT * HT;   // dW_k tiles
  constexpr int kJobs0 = KT0 * HT;    // dW_0 tiles
  constexpr int kBiasTiles = HT / W;  // owned bias unit tiles per layer: ut = wave + W j
  constexpr int kSlotsOut = (kJobsOut + W - 1) / W;
  constexpr int kSlotsHid = (kJobsHid + W - 1) / W;
  constexpr int kSlots0 = (kJobs0 + W - 1) / W;
  static_assert(kSlots0 + kSlotsOut <= kWideAccSlots, "LDS accumulator slots");
  constexpr int kHSlot = HT;       // first layer-input^T slot
  constexpr int kGSlot = 2 * HT;   // output gradient^T slot
  extern __shared__ __align__(16) unsigned char smem[];

  const FieldLayout s = make_layout(INP, HP, a.IN, a.H, NHL, a.M, a.mlp_count, true, true, 1);
  const WideTrainLds ml = wide_train_lds(s);
  copy_to_lds(smem + ml.bias, a.image + s.bias_base, s.res_off - s.bias_base);
  // parked operands of absent tiles must be finite (they meet zero deltas);
  // the LDS accumulators start at zero (they follow the parking slots)
  for (int e = threadIdx.x; e < (ml.total - ml.park) / 16; e += blockDim.x)
    reinterpret_cast<uint4 *>(smem + ml.park)[e] = make_uint4(0u, 0u, 0u, 0u);
  __syncthreads();

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int p = lane & 15;
  const int q = lane >> 4;
  const bool wgrads = a.mode != kModeInputGrad;
  unsigned char *park0 = smem + ml.park;
  unsigned char *pk = park0 + wave * ml.park_bytes;
  auto opnd = [&](int w, int slot) {
    return *reinterpret_cast<const half8 *>(park0 + w * ml.park_bytes + (slot * 64 + lane) * 16);
  };
  auto bias_of = [&](int k) { return reinterpret_cast<const float *>(smem + ml.bias + k * HP * 4); };
  // this wave's LDS accumulator j: [0, kSlots0) dW_0, then dW_out (lane-private)
  f32x4 *acc_lds = reinterpret_cast<f32x4 *>(smem + ml.acc) + wave * kWideAccSlots * 64 + lane;
  auto acc_at = [&](int j) -> f32x4 & { return acc_lds[j * 64]; };
  // Weight stages, double-buffered: a round walks 3 NHL + 1 stages (below),
  // stage i in buffer (i + par) & 1 of two 32 KB buffers. At each stage
  // boundary the block waits for its loads and meets at one barrier, which
  // both publishes stage i and retires every read of the other buffer
  // (stage i - 1); then the loads of stage i + 1 are issued into that buffer
  // and run under stage i's products.
  constexpr int kBuf = HP * HP * 2;
  constexpr int kStages = 3 * NHL + 1;
  int par = 0;
  auto buf = [&](int i) { return smem + ((i + par) & 1) * kBuf; };
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  auto fetch = [&](unsigned char *dst, int32_t off, int bytes) {  // whole 4 KB groups
    // an opaque image base: the addresses are formed here, not hoisted out
    // of the round loop into registers held across it
    const unsigned char *img = a.image;
    asm volatile("" : "+s"(img));
    for (int j = 0; j < (bytes >> 12); ++j) {
      const int c = wave_s + W * j;  // 1 KB chunk of this wave
      __builtin_amdgcn_global_load_lds(img + off + (c << 10) + lane * 16,
                                       (__attribute__((address_space(3))) void *)(dst + (c << 10)),
                                       16, 0, 0);
    }
  };
  auto boundary = [&]() {
    __builtin_amdgcn_s_waitcnt(0);  // this thread's loads (direct-to-LDS included) landed
    __syncthreads();
  };
  // stage i of a round: 0 F0 (hi | lo), 2k - 1 and 2k the unit tiles [0, 4) and
  // [4, 8) of F_k (hi | lo, 1 <= k < NHL), 2 NHL - 1 F_out (hi | lo), 3 NHL - k
  // B_k (NHL >= k >= 0): F forward fragments, B backward fragments
  auto fetch_stage = [&](int i) {
    unsigned char *d = buf(i);
    if (i == 0 || i == kStages) {  // kStages: the next round's stage 0
      fetch(d, s.fwd_off(0), INP * HP * 2);
      fetch(d + INP * HP * 2, s.fwd_lo_off(0), INP * HP * 2);
    } else if (i < 2 * NHL - 1) {
      const int k = (i + 1) / 2, part = (i + 1) % 2 * (kBuf / 2);
      fetch(d, s.fwd_off(k) + part, kBuf / 2);
      fetch(d + kBuf / 2, s.fwd_lo_off(k) + part, kBuf / 2);
    } else if (i == 2 * NHL - 1) {
      fetch(d, s.fwd_off(NHL), HP * 16 * 2);
      fetch(d + HP * 16 * 2, s.fwd_lo_off(NHL), HP * 16 * 2);
    } else {
      const int k = 3 * NHL - i;
      fetch(d, s.bwd_off(k), k == NHL ? HP * 32 * 2 : k == 0 ? INP * HP * 2 : kBuf);
    }
  };
  half8 sel_lo, sel_hi;
  selection_fragments(p, q, sel_lo, sel_hi);
  uint32_t ones16 = 0x00010001u;  // relu_keep's operand, opaque to the compiler
  asm volatile("" : "+s"(ones16));

  f32x4 accH[NHL - 1][kSlotsHid];
  float bsO = 0.0f;                       // output bias (wave 0): lane partial sums
  float bsH[NHL - 1][kBiasTiles];         // hidden biases of the owned unit tiles
  float bs0[kBiasTiles];
#pragma unroll
  for (int j = 0; j < kBiasTiles; ++j) {
    bs0[j] = 0.0f;
#pragma unroll
    for (int k = 0; k < NHL - 1; ++k) bsH[k][j] = 0.0f;
  }
  const half2v one2 = {static_cast<_Float16>(1.0f), static_cast<_Float16>(1.0f)};
  // partial sum += the 8 fp16 values of a parked tile of this lane
  auto add8 = [&](float acc, half8 v) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc = __builtin_amdgcn_fdot2(half2v{v[2 * j], v[2 * j + 1]}, one2, acc, false);
    return acc;
  };
#pragma unroll
  for (int k = 0; k < NHL - 1; ++k)
#pragma unroll
    for (int j = 0; j < kSlotsHid; ++j) accH[k][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  float lane_loss = 0.0f, lane_amax = 0.0f;
  const f32x4 *xt = reinterpret_cast<const f32x4 *>(a.xfeat);
  half8 *act_store = reinterpret_cast<half8 *>(a.wide_act);
  const bool has_target = a.mode != kModeInputGrad && a.target != nullptr;
  const bool dx_vec = (a.IN & 3) == 0;
  const int n_rounds = (a.n_tiles + W - 1) / W;

  if (static_cast<int>(blockIdx.x) < n_rounds) fetch_stage(0);
  for (int round = blockIdx.x; round < n_rounds; round += gridDim.x) {
    const int tile = round * W + wave;
    const bool have = tile < a.n_tiles;  // waves past the batch park zero deltas
    int pt[kNT];
    bool valid[kNT];
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt) {
      pt[nt] = tile * kTilePts + 16 * nt + p;
      valid[nt] = have && pt[nt] < a.n;
    }
    f32x4 X[KT0][kNT];
#pragma unroll
    for (int kt = 0; kt < KT0; ++kt)
#pragma unroll
      for (int nt = 0; nt < kNT; ++nt)
        X[kt][nt] = have ? xt[((static_cast<size_t>(tile) * KT0 + kt) * kNT + nt) * 64 + lane]
                         : f32x4{0.f, 0.f, 0.f, 0.f};
    float Tv[kNT][4];
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt) {
      const uint32_t pr = valid[nt] ? static_cast<uint32_t>(pt[nt]) : 0u;
      const size_t row = static_cast<size_t>(a.tgt_index ? a.tgt_index[pr] : pr) * a.M;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int o = 4 * q + r;
        const float v = has_target ? a.target[row + (o < a.M ? o : a.M - 1)] : 0.0f;
        Tv[nt][r] = (valid[nt] && o < a.M) ? v : 0.0f;
      }
    }
    // packed activations of hidden layer k of this tile in global memory
    auto act_slot = [&](int k, int ks, int nt) {
      return act_store + ((static_cast<size_t>(k) * a.n_tiles + (have ? tile : 0)) * (HS * kNT) +
                          ks * kNT + nt) * 64 + lane;
    };

    // ---- forward, one layer's fragments in LDS at a time
    f32x4 act[HT][kNT];
    auto relu = [&]() {
#pragma unroll
      for (int mt = 0; mt < HT; ++mt)
#pragma unroll
        for (int nt = 0; nt < kNT; ++nt)
#pragma unroll
          for (int r = 0; r < 4; ++r) act[mt][nt][r] = relu_f32(act[mt][nt][r]);
    };
    {
      // layer 0: forward hi and lo fragments (stage 0)
      boundary();
      fetch_stage(1);
      half8 bh[XS][kNT], bl[XS][kNT];
      pack_split_tiles<KT0>(X, bh, bl);
      mma_split_packed<XS, HT>(buf(0), buf(0) + INP * HP * 2, bh, bl, bias_of(0), act, lane);
      relu();
    }
    uint4 fac[HS][kNT];  // ReLU' masks of the layer whose delta is formed next (relu_keep)
#pragma unroll
    for (int k = 1; k <= NHL; ++k) {
      half8 bh[HS][kNT], bl[HS][kNT];
      pack_split_tiles<HT>(act, bh, bl);
      if (k < NHL) {
        // unit tiles [0, 4) on stage 2k - 1, then [4, 8) on stage 2k
        boundary();
        fetch_stage(2 * k);
        if (have)  // after the fetch: the stores retire under the products
#pragma unroll
          for (int ks = 0; ks < HS; ++ks)
#pragma unroll
            for (int nt = 0; nt < kNT; ++nt) *act_slot(k - 1, ks, nt) = bh[ks][nt];
        {
          f32x4 part[HT / 2][kNT];
          mma_split_packed<HS, HT / 2>(buf(2 * k - 1), buf(2 * k - 1) + kBuf / 2, bh, bl,
                                       bias_of(k), part, lane);
#pragma unroll
          for (int mt = 0; mt < HT / 2; ++mt)
#pragma unroll
            for (int nt = 0; nt < kNT; ++nt) act[mt][nt] = part[mt][nt];
        }
        boundary();
        fetch_stage(2 * k + 1);
        {
          f32x4 part[HT / 2][kNT];
          mma_split_packed<HS, HT / 2>(buf(2 * k), buf(2 * k) + kBuf / 2, bh, bl,
                                       bias_of(k) + HP / 2, part, lane);
#pragma unroll
          for (int mt = 0; mt < HT / 2; ++mt)
#pragma unroll
            for (int nt = 0; nt < kNT; ++nt) act[HT / 2 + mt][nt] = part[mt][nt];
        }
        relu();
      } else {
#pragma unroll
        for (int ks = 0; ks < HS; ++ks)
#pragma unroll
          for (int nt = 0; nt < kNT; ++nt) fac[ks][nt] = relu_keep(bh[ks][nt], ones16);
        boundary();  // stage 2 NHL - 1: F_out
        fetch_stage(2 * NHL);
        f32x4 y[1][kNT];
        mma_split_packed<HS, 1>(buf(2 * NHL - 1), buf(2 * NHL - 1) + HP * 16 * 2, bh, bl,
                                bias_of(NHL), y, lane);
        // loss / output gradient (outputs 0..15 in tile 0, tile 1 zero)
        f32x4 g[2][kNT];
        output_grad<2, true>(a, y, Tv, valid, pt, q, lane_loss, lane_amax, g);
        half8 gb[1][kNT];
        pack_tiles<2>(g, gb);
        {
          half8 gT[2];
          transpose_tiles<1>(gb, sel_lo, sel_hi, gT);
          park(pk, kGSlot, lane, gT[0]);
        }
        {
          half8 hT[HT];
          transpose_tiles<HS>(bh, sel_lo, sel_hi, hT);
#pragma unroll
          for (int it = 0; it < HT; ++it) park(pk, kHSlot + it, lane, hT[it]);
        }
        // owners: dW_out (units x outputs) and b_out over the round's points;
        // the boundary publishes the parks and stage 2 NHL (B_out)
        boundary();
        fetch_stage(2 * NHL + 1);
        if (wgrads) {
          f32x4 accO[kSlotsOut];
#pragma unroll
          for (int j = 0; j < kSlotsOut; ++j) accO[j] = acc_at(kSlots0 + j);
#pragma unroll 1
          for (int w = 0; w < W; ++w)  // waves outermost: one wave's operands live
#pragma unroll
            for (int j = 0; j < kSlotsOut; ++j) {
              const int job = wave + W * j;
              if (job < kJobsOut)
                accO[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(opnd(w, kHSlot + job),
                                                                 opnd(w, kGSlot), accO[j], 0, 0, 0);
              if (j == 0 && wave == 0) bsO = add8(bsO, opnd(w, kGSlot));
            }
#pragma unroll
          for (int j = 0; j < kSlotsOut; ++j) acc_at(kSlots0 + j) = accO[j];
        }
        // delta of the last hidden layer (backward fragments of the output layer)
        mma_packed<1, HT>(buf(2 * NHL), gb, act, lane);  // act now holds W_out g (pre-mask)
      }
    }

    // ---- hidden layers NHL-1 .. 1: delta_k parked over slots [0, 8), the
    // layer input h_{k-1} (reloaded, transposed) over [8, 16); owners add
    // dW_k / b_k; then delta_{k-1} on the staged backward fragments. The
    // reloads of h_{k-1} (and of the input features for dW_0) are issued one
    // layer ahead, before layer k + 1's owner jobs (h_{NHL-2} here), so their
    // latency runs under the owner products.
    half8 hpf[HS][kNT];
    auto load_h = [&](int k) {
#pragma unroll
      for (int ks = 0; ks < HS; ++ks)
#pragma unroll
        for (int nt = 0; nt < kNT; ++nt) hpf[ks][nt] = have ? *act_slot(k, ks, nt) : half8{};
    };
    f32x4 xpf[KT0][kNT];
    auto load_x = [&]() {  // L2-resident: not kept live across the round
#pragma unroll
      for (int kt = 0; kt < KT0; ++kt)
#pragma unroll
        for (int nt = 0; nt < kNT; ++nt)
          xpf[kt][nt] = have ? xt[((static_cast<size_t>(tile) * KT0 + kt) * kNT + nt) * 64 + lane]
                             : f32x4{0.f, 0.f, 0.f, 0.f};
    };
    load_h(NHL - 2);
#pragma unroll
    for (int k = NHL - 1; k >= 0; --k) {
      half8 b[HS][kNT];
      pack_tiles<HT>(act, b);
      __syncthreads();  // every wave is done with the last layer's parked operands
#pragma unroll
      for (int ks = 0; ks < HS; ++ks)
#pragma unroll
        for (int nt = 0; nt < kNT; ++nt) b[ks][nt] = apply_keep(b[ks][nt], fac[ks][nt]);
      {
        half8 dT[HT];
        transpose_tiles<HS>(b, sel_lo, sel_hi, dT);
#pragma unroll
        for (int ut = 0; ut < HT; ++ut) park(pk, ut, lane, dT[ut]);
      }
      if (k > 0) {
        half8 hb[HS][kNT];
#pragma unroll
        for (int ks = 0; ks < HS; ++ks)
#pragma unroll
          for (int nt = 0; nt < kNT; ++nt) hb[ks][nt] = hpf[ks][nt];
        half8 hT[HT];
        transpose_tiles<HS>(hb, sel_lo, sel_hi, hT);
#pragma unroll
        for (int it = 0; it < HT; ++it) park(pk, kHSlot + it, lane, hT[it]);
#pragma unroll
        for (int ks = 0; ks < HS; ++ks)
#pragma unroll
          for (int nt = 0; nt < kNT; ++nt) fac[ks][nt] = relu_keep(hb[ks][nt], ones16);
      } else {
        // the input features again (prefetched by load_x)
        half8 bh[XS][kNT], bl[XS][kNT];
        pack_split_tiles<KT0>(xpf, bh, bl);
        half8 xT[KT0];
        transpose_tiles<XS>(bh, sel_lo, sel_hi, xT);
#pragma unroll
        for (int ft = 0; ft < KT0; ++ft) park(pk, kHSlot + ft, lane, xT[ft]);
      }
      // stage 3 NHL - k (B_k) and the parks published; the next stage is
      // B_{k-1}, or the next round's F0
      boundary();
      if (k > 0)
        fetch_stage(3 * NHL - k + 1);
      else if (round + static_cast<int>(gridDim.x) < n_rounds)
        fetch_stage(kStages);
      if (k >= 2)
        load_h(k - 2);
      else if (k == 1)
        load_x();
      if (wgrads) {
        // waves outermost (not unrolled): one wave's operands live at a
        // time; every accumulator still adds the waves in order
        if (k > 0) {
#pragma unroll 1
          for (int w = 0; w < W; ++w)
#pragma unroll
            for (int j = 0; j < kSlotsHid; ++j) {
              const int job = wave + W * j;  // dW tile (it, ut) = (job / HT, job % HT)
              if (job < kJobsHid)
                accH[k - 1][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    opnd(w, kHSlot + job / HT), opnd(w, job % HT), accH[k - 1][j], 0, 0, 0);
              if (j < kBiasTiles) bsH[k - 1][j] = add8(bsH[k - 1][j], opnd(w, wave + W * j));
            }
        } else {
          f32x4 acc0[kSlots0];
#pragma unroll
          for (int j = 0; j < kSlots0; ++j) acc0[j] = acc_at(j);
#pragma unroll 1
          for (int w = 0; w < W; ++w)
#pragma unroll
            for (int j = 0; j < kSlots0; ++j) {
              const int job = wave + W * j;  // dW tile (ft, ut) = (job / HT, job % HT)
              if (job < kJobs0)
                acc0[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    opnd(w, kHSlot + job / HT), opnd(w, job % HT), acc0[j], 0, 0, 0);
              if (j < kBiasTiles) bs0[j] = add8(bs0[j], opnd(w, wave + W * j));
            }
#pragma unroll
          for (int j = 0; j < kSlots0; ++j) acc_at(j) = acc0[j];
        }
      }
      if (k > 0) {
        mma_packed<HS, HT>(buf(3 * NHL - k), b, act, lane);  // W_k delta_k (pre-mask)
      } else {
        f32x4 dx[KT0][kNT];
        mma_packed<HS, KT0>(buf(3 * NHL), b, dx, lane);
        if (have) {
          // rows past the batch exist (the buffer is padded to whole tiles)
#pragma unroll
          for (int nt = 0; nt < kNT; ++nt) {
            float *row = a.dx_out + static_cast<size_t>(pt[nt]) * a.IN;
#pragma unroll
            for (int kt = 0; kt < KT0; ++kt) {
              const int f0 = 16 * kt + 4 * q;
              f32x4 v = dx[kt][nt];
#pragma unroll
              for (int r = 0; r < 4; ++r) v[r] = v[r] * a.inv_loss_scale;
              if (dx_vec) {
                if (f0 < a.IN) *reinterpret_cast<f32x4 *>(row + f0) = v;
              } else {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                  if (f0 + r < a.IN) row[f0 + r] = v[r];
              }
            }
          }
        }
      }
    }
    par ^= kStages & 1;  // the next round's stage 0 is this round's stage kStages
  }

  if (a.mode == kModeInputGrad) return;  // uniform: no loss, no weight gradients
  // ---- loss partial (wave order) and largest |output| of the block
  __syncthreads();
  block_loss_partials(a, lane_loss, lane_amax, reinterpret_cast<float *>(smem + ml.loss), lane,
                      wave, W);
  // ---- owners write their tiles of the block's partial row (reference layout)
  float *dst = a.grad_partials + static_cast<size_t>(blockIdx.x) * a.mlp_count;
  const float sc = a.inv_loss_scale;
  f32x4 accO[kSlotsOut], acc0[kSlots0];
#pragma unroll
  for (int j = 0; j < kSlotsOut; ++j) accO[j] = acc_at(kSlots0 + j);
#pragma unroll
  for (int j = 0; j < kSlots0; ++j) acc0[j] = acc_at(j);
  const int H = a.H, IN = a.IN, M = a.M;
#pragma unroll
  for (int j = 0; j < kSlotsOut; ++j) {
    const int job = wave + W * j;
    if (job < HT) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int u = 16 * job + 4 * q + r;
        if (u < H && p < M) dst[s.w_off(NHL) + u * M + p] = accO[j][r] * sc;
      }
    }
  }
  // bias of unit 16 ut + p: the four lanes p + 16 q, added in a fixed order
  auto lane_total = [&](float v) {
    v = v + __shfl_xor(v, 16);
    return v + __shfl_xor(v, 32);
  };
  {
    const float t = lane_total(bsO);
    if (wave == 0 && q == 0 && p < M) dst[s.b_off(NHL) + p] = t * sc;
  }
#pragma unroll
  for (int k = 1; k < NHL; ++k)
#pragma unroll
    for (int j = 0; j < kSlotsHid; ++j) {
      const int job = wave + W * j;
      if (job < HT * HT) {
        const int it = job / HT, ut = job % HT;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = 16 * it + 4 * q + r, u = 16 * ut + p;
          if (i < H && u < H) dst[s.w_off(k) + i * H + u] = accH[k - 1][j][r] * sc;
        }
      }
      if (j < kBiasTiles) {
        const float t = lane_total(bsH[k - 1][j]);
        const int u = 16 * (wave + W * j) + p;
        if (q == 0 && u < H) dst[s.b_off(k) + u] = t * sc;
      }
    }
#pragma unroll
  for (int j = 0; j < kSlots0; ++j) {
    const int job = wave + W * j;
    if (job < KT0 * HT) {
      const int ft = job / HT, ut = job % HT;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int f = 16 * ft + 4 * q + r, u = 16 * ut + p;
        if (f < IN && u < H) dst[s.w_off(0) + f * H + u] = acc0[j][r] * sc;
      }
    }
    if (j < kBiasTiles) {
      const float t = lane_total(bs0[j]);
      const int u = 16 * (wave + W * j) + p;
      if (q == 0 && u < H) dst[s.b_off(0) + u] = t * sc;
    }
  }
}

}  // namespace tmnn_hip
