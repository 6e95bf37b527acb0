// mlp_kernel.hpp -- fp16 training kernel of the 64-wide MLP with no LDS
// staging of activations or deltas.
//
// The weight gradients dW_k = sum over points of h_{k-1} delta_k^T contract
// over the points of a tile, so their MFMA operands need the points along K:
// each lane must hold consecutive points of one unit. Layer products leave
// the opposite arrangement in registers (the "D layout": a lane holds four
// consecutive units of one point). Instead of a round trip through LDS, this
// kernel transposes on the matrix cores: an MFMA with the packed fp16 tile
// set as A and a constant 0/1 selection fragment as B returns the transposed
// 16x16 tile exactly (every product is x * 1 or x * 0 in an fp32
// accumulator). Those transposed fp16 tiles are precisely the values the LDS
// path fed to the dW MFMAs (fp16(h), fp16(delta)), so the arithmetic of the
// weight gradients is unchanged.
//
// Occupancy and weight gradients: eight waves per block, two per SIMD (256
// registers each), so one wave's MFMA / LDS latencies hide behind the other's
// work; shapes whose weight image leaves no LDS for eight waves' parking run
// four waves, one per SIMD (mlp_waves). The block walks its tiles in rounds
// of one tile per wave; each
// wave parks the transposed operands of its tile in LDS (lane-private 16-byte
// slots), and after a barrier every wave accumulates the dW tiles it OWNS over
// all eight waves' points, in wave order, in registers that live across all
// rounds. Each dW element has exactly one owner (deterministic sums, no
// cross-wave reduction); the owners write the block's partial row at the end.
// Parking slots are reused as layers die: delta_k goes into the slots of h_k
// once dW_{k+1} (the last reader of h_k) is done. In 8-wave blocks dW_out
// needs no exchange: each wave accumulates it from its own parked last
// hidden layer and its output gradient in registers (no barrier), and the
// waves' partials are added in wave order at the end, as are the bias
// gradients; 4-wave blocks (one job per wave) keep dW_out as owner jobs.
//
// Everything else follows field_body in the fp16 training configuration:
// split-fp16 forward (hi/lo operands, three MFMAs per product), fp16 backward
// with a power-of-two loss scale, input features read as X tiles from
// encode_features_kernel. Details that differ are of fp16 size: the ReLU
// derivative is taken from the fp16 activation (a positive activation below
// 2^-25 rounds to 0 and masks its delta), the bias gradients sum the fp16
// deltas on the matrix cores (each wave its own tiles' column sums, the
// waves' partials added in wave order at the end), each layer's bias is the accumulator's initial value (added
// before the products, not after), and RelativeL2 takes its reciprocal from
// v_rcp_f32.
//
// Instances with SD > 0 also run the hash-grid backward of each tile
// (tile_scatter.hpp, a D = SD, F = SF grid) where the input-feature
// gradients come off the matrix cores, instead of storing them for
// hash_scatter_kernel; the tile's point positions are prefetched with its X
// tiles.
#pragma once

#include "field_kernel.hpp"
#include "tile_scatter.hpp"

namespace tmnn_hip {

// Waves per block of mlp_train_kernel: eight (two per SIMD, 256 registers
// each) where the weight image and eight waves' parking slots fit in LDS,
// else four (one per SIMD with the whole register file).
__host__ __device__ constexpr int mlp_waves(int INP, int NHL) {
  return (INP <= 32 && NHL <= 2) ? 8 : 4;
}

// LDS plan of mlp_train_kernel (bytes): the packed weight image, the per-wave
// loss slots, then per wave its parking slots (16 bytes per lane each): [0, KT0) input features,
// KT0 + k * HT + t hidden layer k (then delta_k), and in 4-wave blocks
// KT0 + NHL * HT the output gradient, in 8-wave blocks KT0 + (NHL + k) * HT + t
// delta_k for k < NHL - 1.
struct MlpLds {
  int32_t loss, park, park_bytes, total;
};

__host__ __device__ __forceinline__ MlpLds mlp_lds(const FieldLayout &s, int waves) {
  MlpLds m;
  m.loss = s.dw_off;
  m.park = m.loss + 16 * 4;
  m.park_bytes =
      (s.INP / 16 + s.NHL * (s.HP / 16) + (waves == 8 ? (s.NHL - 1) * (s.HP / 16) : 1)) * 64 * 16;
  m.total = m.park + waves * m.park_bytes;
  return m;
}

// Lane-private 16-byte LDS slots (slot-major, lane-minor: conflict-free).
__device__ __forceinline__ void park(unsigned char *base, int slot, int lane, half8 v) {
  *reinterpret_cast<half8 *>(base + (slot * 64 + lane) * 16) = v;
}
__device__ __forceinline__ half8 unpark(const unsigned char *base, int slot, int lane) {
  return *reinterpret_cast<const half8 *>(base + (slot * 64 + lane) * 16);
}

// B-operand selection fragments of the transpose MFMA: with a packed tile
// pair (t0 | t1) as A, sel_lo picks t0 and sel_hi picks t1 (lane p + 16 q,
// K slot j: t0 unit 4q + j for j < 4, t1 unit 4q + j - 4 for j >= 4).
__device__ __forceinline__ void selection_fragments(int p, int q, half8 &sel_lo, half8 &sel_hi) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    sel_lo[j] = (j < 4 && 4 * q + j == p) ? static_cast<_Float16>(1.0f) : static_cast<_Float16>(0.0f);
    sel_hi[j] = (j >= 4 && 4 * q + j - 4 == p) ? static_cast<_Float16>(1.0f) : static_cast<_Float16>(0.0f);
  }
}

// Transposed fp16 tiles of a packed D-layout tile set b[KS][nt] (units along
// K, 32 points): T[u] for unit tile u = 2 ks + t holds, in lane p + 16 q,
// slot j, the value of unit 16 u + p at point 4 q + j (j < 4) or
// 16 + 4 q + j - 4 (j >= 4) -- the A/B operand of a dW MFMA over the tile's
// 32 points.
template <int KS>
__device__ __forceinline__ void transpose_tiles(const half8 (&b)[KS][kNT], half8 sel_lo,
                                                half8 sel_hi, half8 (&T)[2 * KS]) {
  const f32x4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const f32x4 a0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(b[ks][0], sel_lo, z, 0, 0, 0);
    const f32x4 a1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(b[ks][1], sel_lo, z, 0, 0, 0);
    const f32x4 c0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(b[ks][0], sel_hi, z, 0, 0, 0);
    const f32x4 c1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(b[ks][1], sel_hi, z, 0, 0, 0);
    T[2 * ks] = pack8(a0, a1);
    T[2 * ks + 1] = pack8(c0, c1);
  }
}

// out[MT][nt] = A(frag) x B for a packed B operand (fp16, K step 32).
template <int KS, int MT>
__device__ __forceinline__ void mma_packed(const unsigned char *frag, const half8 (&b)[KS][kNT],
                                           f32x4 (&out)[MT][kNT], int lane) {
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    f32x4 acc[kNT];
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt) acc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const half8 av = *reinterpret_cast<const half8 *>(frag + ((mt * KS + ks) * 64 + lane) * 16);
#pragma unroll
      for (int nt = 0; nt < kNT; ++nt)
        acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, b[ks][nt], acc[nt], 0, 0, 0);
    }
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt) out[mt][nt] = acc[nt];
  }
}

// Split-fp16 forward product (as layer_mma_split) on prepacked operands,
// accumulated onto the layer's bias (units 16 mt + 4 q + r of bias): the
// bias enters first instead of last, one fp32 rounding apart.
template <int KS, int MT>
__device__ __forceinline__ void mma_split_packed(const unsigned char *frag_hi,
                                                 const unsigned char *frag_lo,
                                                 const half8 (&bh)[KS][kNT],
                                                 const half8 (&bl)[KS][kNT], const float *bias,
                                                 f32x4 (&out)[MT][kNT], int lane) {
  const int q = lane >> 4;
  // unit tiles in pairs (one alone if MT is odd): four independent
  // accumulator chains interleaved; each chain keeps its own product order
  constexpr int MP = MT >= 2 ? 2 : 1;
#pragma unroll
  for (int m0 = 0; m0 < MT; m0 += MP) {
    constexpr int kM = MP;
    f32x4 acc[kM][kNT];
#pragma unroll
    for (int u = 0; u < kM; ++u) {
      const int mt = m0 + u < MT ? m0 + u : MT - 1;
      const f32x4 bv = *reinterpret_cast<const f32x4 *>(bias + 16 * mt + 4 * q);
#pragma unroll
      for (int nt = 0; nt < kNT; ++nt) acc[u][nt] = bv;
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      half8 ah[kM], al[kM];
#pragma unroll
      for (int u = 0; u < kM; ++u) {
        const int mt = m0 + u < MT ? m0 + u : MT - 1;
        const int off = ((mt * KS + ks) * 64 + lane) * 16;
        ah[u] = *reinterpret_cast<const half8 *>(frag_hi + off);
        al[u] = *reinterpret_cast<const half8 *>(frag_lo + off);
      }
#pragma unroll
      for (int u = 0; u < kM; ++u)
#pragma unroll
        for (int nt = 0; nt < kNT; ++nt)
          acc[u][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[u], bh[ks][nt], acc[u][nt], 0, 0, 0);
#pragma unroll
      for (int u = 0; u < kM; ++u)
#pragma unroll
        for (int nt = 0; nt < kNT; ++nt)
          acc[u][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[u], bl[ks][nt], acc[u][nt], 0, 0, 0);
#pragma unroll
      for (int u = 0; u < kM; ++u)
#pragma unroll
        for (int nt = 0; nt < kNT; ++nt)
          acc[u][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[u], bh[ks][nt], acc[u][nt], 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < kM; ++u)
      if (m0 + u < MT)
#pragma unroll
        for (int nt = 0; nt < kNT; ++nt) out[m0 + u][nt] = acc[u][nt];
  }
}

template <int KT>
__device__ __forceinline__ void pack_split_tiles(const f32x4 (&t)[KT][kNT], half8 (&bh)[KT / 2][kNT],
                                                 half8 (&bl)[KT / 2][kNT]) {
#pragma unroll
  for (int ks = 0; ks < KT / 2; ++ks)
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt) pack8_split(t[2 * ks][nt], t[2 * ks + 1][nt], bh[ks][nt], bl[ks][nt]);
}

template <int KT>
__device__ __forceinline__ void pack_tiles(const f32x4 (&t)[KT][kNT], half8 (&b)[KT / 2][kNT]) {
#pragma unroll
  for (int ks = 0; ks < KT / 2; ++ks)
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt) b[ks][nt] = pack8(t[2 * ks][nt], t[2 * ks + 1][nt]);
}

// ReLU' of a packed fp16 activation tile pair (ReLU outputs: +0, positive or
// NaN) as 16-bit masks: 0 - min(bits, 1) is 0x0000 exactly for +0, else
// 0xFFFF; applied to a packed fp16 delta by a 32-bit AND. Two packed integer
// ops per pair to make (the fp16 factors take three), one to apply. `ones`
// holds 0x00010001 in an opaque scalar register (set up once per kernel):
// with a literal the compiler proves the 0/1 range and rewrites the ops into
// per-element compares and selects.
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));
__device__ __forceinline__ uint4 relu_keep(half8 h, uint32_t ones) {
  const u16x8 o = __builtin_bit_cast(u16x8, make_uint4(ones, ones, ones, ones));
  const u16x8 m = static_cast<u16x8>(0) - __builtin_elementwise_min(__builtin_bit_cast(u16x8, h), o);
  return __builtin_bit_cast(uint4, m);
}
__device__ __forceinline__ half8 apply_keep(half8 d, uint4 keep) {
  uint4 v = __builtin_bit_cast(uint4, d);
  v.x &= keep.x;
  v.y &= keep.y;
  v.z &= keep.z;
  v.w &= keep.w;
  return __builtin_bit_cast(half8, v);
}

// max(x, 0) as one v_maximum3_f32 (fmaxf on an MFMA result adds a NaN-quieting
// max(x, x)); -0 maps to +0
__device__ __forceinline__ float relu_f32(float x) { return __builtin_elementwise_maximum(x, 0.0f); }

// Scheduling hint for an owner's run of W products: the LDS reads of four
// products' operands, then those four MFMAs, and so on, so the reads are in
// flight together instead of one read, one wait, one product at a time.
template <int W>
__device__ __forceinline__ void owner_schedule() {
#pragma unroll
  for (int g = 0; g < W / 4; ++g) {
    __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);  // DS reads
    __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);  // MFMA
  }
}

template <int HP, int INP, int NHL, int W = mlp_waves(INP, NHL), int SD = 0, int SF = 0>
__global__ void __launch_bounds__(W * 64)
    __attribute__((amdgpu_waves_per_eu(W / 4, W / 4))) mlp_train_kernel(FieldArgs a) {
  constexpr int HT = HP / 16;    // unit tiles of a hidden layer
  constexpr int HS = HT / 2;     // K steps over a hidden layer
  constexpr int KT0 = INP / 16;  // input feature tiles
  constexpr int XS = KT0 / 2;    // K steps over the input
  static_assert(HT % 2 == 0 && KT0 % 2 == 0 && NHL >= 1 && W % 4 == 0, "shape");
  static_assert(HT <= 4, "bias_mma maps unit tile u to lanes 16 u .. 16 u + 15");
  // owned jobs (dW tiles + bias tiles) per phase, wave w owns jobs w + W j
  // (bias gradients: each wave's own partials, bias_mma below)
  constexpr int kJobsHid = HT * HT;   // dW_k tiles
  constexpr int kJobs0 = KT0 * HT;    // dW_0 tiles
  constexpr int kSlotsHid = (kJobsHid + W - 1) / W;
  constexpr int kSlots0 = (kJobs0 + W - 1) / W;
  extern __shared__ __align__(16) unsigned char smem[];

  const FieldLayout s = make_layout(INP, HP, a.IN, a.H, NHL, a.M, a.mlp_count, true, true, W,
                                    false, true);
  const MlpLds ml = mlp_lds(s, W);
  stage_weights<true, true>(a, s, smem);
  // parked operands of absent tiles must be finite (they meet zero deltas)
  for (int e = threadIdx.x; e < W * ml.park_bytes / 16; e += blockDim.x)
    reinterpret_cast<uint4 *>(smem + ml.park)[e] = make_uint4(0u, 0u, 0u, 0u);
  __syncthreads();

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int p = lane & 15;
  const int q = lane >> 4;
  const bool wgrads = a.mode != kModeInputGrad;
  unsigned char *park0 = smem + ml.park;
  unsigned char *pk = park0 + wave * ml.park_bytes;
  auto hslot = [](int k, int it) { return KT0 + k * HT + it; };
  // operand of wave w's slot
  auto opnd = [&](int w, int slot) {
    return *reinterpret_cast<const half8 *>(park0 + w * ml.park_bytes + (slot * 64 + lane) * 16);
  };
  half8 sel_lo, sel_hi;
  selection_fragments(p, q, sel_lo, sel_hi);
  uint32_t ones16 = 0x00010001u;  // relu_keep's operand, opaque to the compiler
  asm volatile("" : "+s"(ones16));

  // dW_out (units x outputs): 8-wave blocks, this wave's tiles, unit tile u
  // in accO[u] (lane n + 16 q: units 16 u + 4 q + r, output n), the waves'
  // partials added in wave order at the end; 4-wave blocks, owner job
  // wave + W j in accO[j]
  constexpr bool kOwnOut = W == 8;
  constexpr int kSlotsOut = kOwnOut ? HT : (HT + W - 1) / W;
  constexpr int kGSlot = KT0 + NHL * HT;  // 4-wave blocks: the output gradient
  // slot of unit tile ut of delta_k: over h_k in 4-wave blocks and for
  // delta_{NHL-1}; in 8-wave blocks the other deltas follow the hidden layers
  auto dslot = [](int k, int ut) {
    return (!kOwnOut || k == NHL - 1) ? KT0 + k * HT + ut : KT0 + NHL * HT + k * HT + ut;
  };
  f32x4 accO[kSlotsOut];
  f32x4 accH[NHL > 1 ? NHL - 1 : 1][kSlotsHid];
  f32x4 acc0[kSlots0];
  // bias gradient partials of this wave's tiles: lane l holds unit l of
  // hidden layer k (biasH[k]) or output l (biasO, lanes < 16)
  f32x4 biasH[NHL], biasO = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int k = 0; k < NHL; ++k) biasH[k] = f32x4{0.f, 0.f, 0.f, 0.f};
  // Column sums of a transposed delta tile (units along N, the tile's 32
  // points along K) on the matrix cores: the A operand is 1 in rows
  // 4 u .. 4 u + 3 and 0 elsewhere, so unit tile u's sums land in rows
  // 4 u .. 4 u + 3 of the D tile, i.e. lane p + 16 u holds the sum for unit
  // 16 u + p; one accumulator takes all four unit tiles of a layer.
  auto bias_mma = [&](int u, half8 t, f32x4 acc) {
    const half8 one8 = {1, 1, 1, 1, 1, 1, 1, 1}, zero8 = {0, 0, 0, 0, 0, 0, 0, 0};
    return __builtin_amdgcn_mfma_f32_16x16x32_f16((p >> 2) == u ? one8 : zero8, t, acc, 0, 0, 0);
  };
#pragma unroll
  for (int u = 0; u < kSlotsOut; ++u) accO[u] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int k = 0; k < (NHL > 1 ? NHL - 1 : 1); ++k)
#pragma unroll
    for (int j = 0; j < kSlotsHid; ++j) accH[k][j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < kSlots0; ++j) acc0[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  float lane_loss = 0.0f, lane_amax = 0.0f;
  const f32x4 *xt = reinterpret_cast<const f32x4 *>(a.xfeat);
  const bool has_target = a.mode != kModeInputGrad && a.target != nullptr;
  const bool dx_vec = (a.IN & 3) == 0;
  const int n_rounds = (a.n_tiles + W - 1) / W;

  // Software pipeline over the block's rounds: the X tiles and target rows
  // of the next round are requested once this round's X is packed, its
  // targets (a gather through the rows) after this round's loss, so the
  // loads overlap a round of work instead of opening the next one.
  f32x4 Xn[KT0][kNT];
  uint32_t rown[kNT];
  float Tn[kNT][4];
  constexpr int PD = SD > 0 ? SD : 1;
  float Pn[kNT][PD];  // fused scatter: the next tile's point positions
  auto point_valid = [&](int tile, int nt) {
    return tile < a.n_tiles && tile * kTilePts + 16 * nt + p < a.n;
  };
  auto fetch_x = [&](int tile) {
#pragma unroll
    for (int kt = 0; kt < KT0; ++kt)
#pragma unroll
      for (int nt = 0; nt < kNT; ++nt)
        Xn[kt][nt] = tile < a.n_tiles
                         ? xt[((static_cast<size_t>(tile) * KT0 + kt) * kNT + nt) * 64 + lane]
                         : f32x4{0.f, 0.f, 0.f, 0.f};
    if constexpr (SD > 0) {
#pragma unroll
      for (int nt = 0; nt < kNT; ++nt) {
        const bool ok = point_valid(tile, nt);
        const size_t pi = ok ? static_cast<size_t>(tile * kTilePts + 16 * nt + p) : 0u;
#pragma unroll
        for (int k = 0; k < SD; ++k) Pn[nt][k] = ok ? a.spos[pi * SD + k] : 0.0f;
      }
    }
  };
  auto fetch_rows = [&](int tile) {
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt) {
      const uint32_t pr =
          point_valid(tile, nt) ? static_cast<uint32_t>(tile * kTilePts + 16 * nt + p) : 0u;
      rown[nt] = has_target ? (a.tgt_index ? a.tgt_index[pr] : pr) : 0u;
    }
  };
  // raw values: the validity select waits until the round that uses them
  auto fetch_targets = [&]() {
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt) {
      const size_t row = static_cast<size_t>(rown[nt]) * a.M;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int o = 4 * q + r;
        Tn[nt][r] = has_target ? a.target[row + (o < a.M ? o : a.M - 1)] : 0.0f;
      }
    }
  };
  if (blockIdx.x < n_rounds) {
    fetch_x(blockIdx.x * W + wave);
    fetch_rows(blockIdx.x * W + wave);
    fetch_targets();
  }
  // 2D grids (four corners per level, a table the L2 holds): the fused
  // hash-grid backward of the previous round's tile runs in three parts
  // inside this round's forward (after the layer-0, layer-1 and output-layer
  // products are issued), so its index arithmetic and stores use the VALU
  // and memory pipes while the matrix cores run the products; the last
  // round's runs after the loop. The int32 atomic sums and flag stores are
  // order-free. 3D grids (eight corners into tables of tens of MB: a
  // memory-bound backward) run it right after the tile's dW_0 owner jobs
  // instead, where it overlaps other waves' owner jobs; deferred, its
  // stores stalled the forward (C3 MLP kernel 257 -> 313 us).
  constexpr bool kDeferScatter = SD == 2;
  f32x4 sdx[KT0][kNT];
  float sP[kNT][PD];
  bool svalid[kNT];
  bool spend = false;
  const float *sres = reinterpret_cast<const float *>(smem + s.res_off);
  // three parts in proportion to the products they sit behind (layer 0,
  // layer 1, the output layer: 24, 48 and 12 MFMAs at C2): groups [0, G/4),
  // [G/4, 3G/4), [3G/4, G) of the tile's G = 2 KT0 groups
  auto scatter_part = [&](auto part) __attribute__((always_inline)) {
    if constexpr (kDeferScatter) {
      constexpr int G = 2 * KT0, i = decltype(part)::value;
      constexpr int gb = i == 0 ? 0 : (i == 1 ? G / 4 : 3 * G / 4);
      constexpr int ge = i == 0 ? G / 4 : (i == 1 ? 3 * G / 4 : G);
      if (spend) tile_scatter<SD, SF, KT0, gb, ge>(a, sdx, sP, svalid, sres, q);
    }
  };

  for (int round = blockIdx.x; round < n_rounds; round += gridDim.x) {
    const int tile = round * W + wave;
    const int next_tile = (round + gridDim.x) * W + wave;  // >= n_tiles: zeros
    const bool have = tile < a.n_tiles;  // waves past the batch park zero deltas
    int pt[kNT];
    bool valid[kNT];
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt) {
      pt[nt] = tile * kTilePts + 16 * nt + p;
      valid[nt] = point_valid(tile, nt);
    }
    f32x4 X[KT0][kNT];
#pragma unroll
    for (int kt = 0; kt < KT0; ++kt)
#pragma unroll
      for (int nt = 0; nt < kNT; ++nt) X[kt][nt] = Xn[kt][nt];
    float P[kNT][PD];
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt)
#pragma unroll
      for (int k = 0; k < PD; ++k) P[nt][k] = Pn[nt][k];
    float Tv[kNT][4];
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt)
#pragma unroll
      for (int r = 0; r < 4; ++r) Tv[nt][r] = (valid[nt] && 4 * q + r < a.M) ? Tn[nt][r] : 0.0f;
    // the targets arrived during the previous round: take them here, before
    // this round's requests (an empty asm: orders, emits nothing), so that the
    // wait for them does not also wait for the loads issued below
    asm volatile(""
                 : "+v"(Tv[0][0]), "+v"(Tv[0][1]), "+v"(Tv[0][2]), "+v"(Tv[0][3]),
                   "+v"(Tv[1][0]), "+v"(Tv[1][1]), "+v"(Tv[1][2]), "+v"(Tv[1][3])
                 :
                 : "memory");

    // ---- forward; transposed fp16 layer inputs parked, ReLU masks kept
    f32x4 act[HT][kNT];
    uint4 mask[NHL][HS][kNT];  // ReLU' masks of the hidden layers (relu_keep)
    {
      half8 bh[XS][kNT], bl[XS][kNT];
      pack_split_tiles<KT0>(X, bh, bl);
      fetch_x(next_tile);
      fetch_rows(next_tile);
      half8 xT[KT0];
      transpose_tiles<XS>(bh, sel_lo, sel_hi, xT);
#pragma unroll
      for (int ft = 0; ft < KT0; ++ft) park(pk, ft, lane, xT[ft]);
      mma_split_packed<XS, HT>(smem + s.fwd_off(0), smem + s.fwd_lo_off(0), bh, bl,
                               reinterpret_cast<const float *>(smem + s.bias_off(0)), act, lane);
    }
    scatter_part(std::integral_constant<int, 0>{});
    auto relu = [&]() {
#pragma unroll
      for (int mt = 0; mt < HT; ++mt)
#pragma unroll
        for (int nt = 0; nt < kNT; ++nt)
#pragma unroll
          for (int r = 0; r < 4; ++r) act[mt][nt][r] = relu_f32(act[mt][nt][r]);
    };
    auto pack_hidden = [&](int k, half8 (&bh)[HS][kNT], half8 (&bl)[HS][kNT]) {
      pack_split_tiles<HT>(act, bh, bl);
#pragma unroll
      for (int ks = 0; ks < HS; ++ks)
#pragma unroll
        for (int nt = 0; nt < kNT; ++nt) mask[k][ks][nt] = relu_keep(bh[ks][nt], ones16);
      half8 hT[HT];
      transpose_tiles<HS>(bh, sel_lo, sel_hi, hT);
#pragma unroll
      for (int it = 0; it < HT; ++it) park(pk, hslot(k, it), lane, hT[it]);
    };
    relu();
#pragma unroll
    for (int k = 1; k < NHL; ++k) {
      half8 bh[HS][kNT], bl[HS][kNT];
      pack_hidden(k - 1, bh, bl);
      mma_split_packed<HS, HT>(smem + s.fwd_off(k), smem + s.fwd_lo_off(k), bh, bl,
                               reinterpret_cast<const float *>(smem + s.bias_off(k)), act, lane);
      if (k == 1) scatter_part(std::integral_constant<int, 1>{});
      relu();
    }
    if constexpr (NHL == 1) scatter_part(std::integral_constant<int, 1>{});
    f32x4 y[1][kNT];
    {
      half8 bh[HS][kNT], bl[HS][kNT];
      pack_hidden(NHL - 1, bh, bl);
      mma_split_packed<HS, 1>(smem + s.fwd_off(NHL), smem + s.fwd_lo_off(NHL), bh, bl,
                              reinterpret_cast<const float *>(smem + s.bias_off(NHL)), y, lane);
    }
    scatter_part(std::integral_constant<int, 2>{});
    spend = false;

    // ---- loss / output gradient (outputs 0..15 in tile 0, tile 1 zero)
    f32x4 g[2][kNT];
    output_grad<2, true>(a, y, Tv, valid, pt, q, lane_loss, lane_amax, g);
    fetch_targets();
    half8 gb[1][kNT];
    pack_tiles<2>(g, gb);
    {
      half8 gT[2];
      transpose_tiles<1>(gb, sel_lo, sel_hi, gT);
      biasO = bias_mma(0, gT[0], biasO);
      // dW_out of this wave's tile, from its own parked h_{NHL-1} tiles (no
      // other wave reads them: no barrier, and delta_{NHL-1} is parked over
      // them below in this wave's program order)
      if (!kOwnOut) park(pk, kGSlot, lane, gT[0]);
      if (kOwnOut && wgrads) {
        wave_lds_sync();
        half8 hT[HT];
#pragma unroll
        for (int u = 0; u < HT; ++u) hT[u] = unpark(pk, hslot(NHL - 1, u), lane);
#pragma unroll
        for (int u = 0; u < HT; ++u) accO[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(hT[u], gT[0], accO[u], 0, 0, 0);
        wave_lds_sync();
      }
    }
    f32x4 dl[HT][kNT];
    mma_packed<1, HT>(smem + s.bwd_off(NHL), gb, dl, lane);

    if constexpr (!kOwnOut) {  // owners: dW_out (units x outputs) over the round's points
      __syncthreads();
      if (wgrads) {
#pragma unroll
        for (int j = 0; j < kSlotsOut; ++j) {
          const int job = wave + W * j;
          if (job < HT) {
            half8 oa[W], ob[W];  // every operand requested before the first product
#pragma unroll
            for (int w = 0; w < W; ++w) {
              oa[w] = opnd(w, hslot(NHL - 1, job));
              ob[w] = opnd(w, kGSlot);
            }
            f32x4 acc = accO[j];
#pragma unroll
            for (int w = 0; w < W; ++w) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(oa[w], ob[w], acc, 0, 0, 0);
            accO[j] = acc;
            owner_schedule<W>();
          }
        }
      }
      __syncthreads();
    }

    // ---- hidden layers NHL-1 .. 0: delta_k (masked, fp16) parked, owners add
    // dW_k, then delta_{k-1} (or the input-feature gradient). 4-wave blocks
    // park delta_k over h_k once the owners of dW_{k+1} are done (a barrier
    // per layer either side of its owner phase). 8-wave blocks park every
    // delta without a barrier (delta_{NHL-1} over this wave's own
    // h_{NHL-1}, which only its dW_out read; the others in slots of their
    // own), then meet once and run all layers' owner jobs in one phase.
    f32x4 dx[KT0][kNT];  // the input-feature gradients (k == 0)
    // this tile's hash-grid backward: now, or kept for the next round
    auto scatter_tile = [&]() __attribute__((always_inline)) {
      if constexpr (kDeferScatter) {
#pragma unroll
        for (int nt = 0; nt < kNT; ++nt) {
#pragma unroll
          for (int kt = 0; kt < KT0; ++kt) sdx[kt][nt] = dx[kt][nt];
#pragma unroll
          for (int k = 0; k < PD; ++k) sP[nt][k] = P[nt][k];
          svalid[nt] = valid[nt];
        }
        spend = true;
      } else if constexpr (SD > 0) {
        tile_scatter<SD, SF, KT0>(a, dx, P, valid, sres, q);
      }
    };
    auto owners = [&](int k) __attribute__((always_inline)) {
      if (!wgrads) return;
      if (k > 0) {
#pragma unroll
        for (int j = 0; j < kSlotsHid; ++j) {
          const int job = wave + W * j;
          if (job < kJobsHid) {
            const int it = job / HT, ut = job % HT;  // dW tile (it, ut)
            half8 oa[W], ob[W];
#pragma unroll
            for (int w = 0; w < W; ++w) {
              oa[w] = opnd(w, hslot(k - 1, it));
              ob[w] = opnd(w, dslot(k, ut));
            }
            f32x4 acc = accH[k - 1][j];
#pragma unroll
            for (int w = 0; w < W; ++w) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(oa[w], ob[w], acc, 0, 0, 0);
            accH[k - 1][j] = acc;
            owner_schedule<W>();
          }
        }
      } else {
#pragma unroll
        for (int j = 0; j < kSlots0; ++j) {
          const int job = wave + W * j;
          if (job < kJobs0) {
            const int ft = job / HT, ut = job % HT;
            half8 oa[W], ob[W];
#pragma unroll
            for (int w = 0; w < W; ++w) {
              oa[w] = opnd(w, ft);
              ob[w] = opnd(w, dslot(0, ut));
            }
            f32x4 acc = acc0[j];
#pragma unroll
            for (int w = 0; w < W; ++w) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(oa[w], ob[w], acc, 0, 0, 0);
            acc0[j] = acc;
            owner_schedule<W>();
          }
        }
      }
    };
#pragma unroll
    for (int k = NHL - 1; k >= 0; --k) {
      half8 b[HS][kNT];
      pack_tiles<HT>(dl, b);
#pragma unroll
      for (int ks = 0; ks < HS; ++ks)
#pragma unroll
        for (int nt = 0; nt < kNT; ++nt) b[ks][nt] = apply_keep(b[ks][nt], mask[k][ks][nt]);
      {
        half8 dT[HT];
        transpose_tiles<HS>(b, sel_lo, sel_hi, dT);
#pragma unroll
        for (int ut = 0; ut < HT; ++ut) park(pk, dslot(k, ut), lane, dT[ut]);
#pragma unroll
        for (int ut = 0; ut < HT; ++ut) biasH[k] = bias_mma(ut, dT[ut], biasH[k]);
      }
      if (k > 0) {
        mma_packed<HS, HT>(smem + s.bwd_off(k), b, dl, lane);
      } else {
        mma_packed<HS, KT0>(smem + s.bwd_off(0), b, dx, lane);
        if constexpr (SD > 0) {
          // the hash-grid backward runs after this wave's dW_0 owner jobs
          // (below), in the same barrier interval
        } else if (have) {
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
      if constexpr (!kOwnOut) {
        __syncthreads();
        owners(k);
        if constexpr (SD > 0)
          if (k == 0) scatter_tile();
        __syncthreads();
      }
    }
    if constexpr (kOwnOut) {
      __syncthreads();  // every wave's deltas are parked
#pragma unroll
      for (int k = NHL - 1; k >= 0; --k) owners(k);
      if constexpr (SD > 0) scatter_tile();
      __syncthreads();  // the next round parks its operands over these slots
    }
  }
  scatter_part(std::integral_constant<int, 0>{});
  scatter_part(std::integral_constant<int, 1>{});
  scatter_part(std::integral_constant<int, 2>{});

  if (a.mode == kModeInputGrad) return;  // uniform: no loss, no weight gradients
  // ---- loss partial (wave order) and largest |output| of the block
  block_loss_partials(a, lane_loss, lane_amax, reinterpret_cast<float *>(smem + ml.loss), lane,
                      wave, W);
  // ---- owners write their tiles of the block's partial row (reference layout)
  float *dst = a.grad_partials + static_cast<size_t>(blockIdx.x) * a.mlp_count;
  const float sc = a.inv_loss_scale;
  const int H = a.H, IN = a.IN, M = a.M;
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
  }
  // ---- bias gradients: the waves' partials (lane l: unit l) summed in wave
  // order through LDS (the parking slots are free after the last round)
  float *bred = reinterpret_cast<float *>(smem + ml.park);
#pragma unroll
  for (int k = 0; k < NHL; ++k) bred[(wave * (NHL + 1) + k) * 64 + lane] = biasH[k][0];
  bred[(wave * (NHL + 1) + NHL) * 64 + lane] = biasO[0];
  // 8-wave blocks: dW_out partials after them (wave w, unit tile u, lane,
  // item r); 4-wave blocks: the owners' tiles
  float *ored = bred + W * (NHL + 1) * 64;
  if constexpr (kOwnOut) {
#pragma unroll
    for (int u = 0; u < HT; ++u)
      *reinterpret_cast<f32x4 *>(ored + ((wave * HT + u) * 64 + lane) * 4) = accO[u];
  } else {
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
  }
  __syncthreads();
  if constexpr (kOwnOut) {
    for (int e = threadIdx.x; e < HP * 16; e += blockDim.x) {
      const int i = e / 16, n = e % 16;  // unit i, output n
      if (i < H && n < M) {
        const int u = i / 16, qq = (i % 16) / 4, r = i % 4;
        float t = 0.0f;
        for (int w = 0; w < W; ++w) t += ored[((w * HT + u) * 64 + n + 16 * qq) * 4 + r];
        dst[s.w_off(NHL) + i * M + n] = t * sc;
      }
    }
  }
  for (int e = threadIdx.x; e < (NHL + 1) * 64; e += blockDim.x) {
    const int k = e / 64, u = e % 64;
    float t = 0.0f;
    for (int w = 0; w < W; ++w) t += bred[(w * (NHL + 1) + k) * 64 + u];
    if (u < (k == NHL ? M : H)) dst[s.b_off(k) + u] = t * sc;
  }
}

}  // namespace tmnn_hip
