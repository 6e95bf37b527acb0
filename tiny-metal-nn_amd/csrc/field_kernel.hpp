// field_kernel.hpp -- the fused neural-field kernel for gfx950.
//
// One launch runs, per 32-point wave tile:
//   hash-grid encode (gathers straight into MFMA B-operand registers)
//   -> MLP forward on MFMA (weights resident in LDS as A-operand fragments)
//   -> loss + output gradient                          [training modes]
//   -> MLP backward on MFMA, dW accumulated per wave    [training modes]
//   -> input-feature gradient dx, stored per point      [training modes]
// and hash_scatter_kernel then turns dx into the int32 fixed-point hash
// gradients and lazy-Adam visit flags, one thread per (point, level).
//
// Reference semantics (paths relative to the reference checkout):
//   encode      mlp_kernel_emitter.cpp:205-360 (emitHashEncodeUnified)
//   MLP fwd     mlp_kernel_emitter.cpp:362-480, :2987-3036
//   loss        mlp_kernel_emitter.cpp:562-670 (emitLoss)
//   MLP bwd     mlp_kernel_emitter.cpp:3055-3113
//   hash bwd    mlp_kernel_emitter.cpp:672-901 (emitHashScatter),
//               mask :48-71 (emit_active_hash_tracking)
//
// Register layout ("D layout"): within a 64-lane wave, lane = p + 16*q.
// A 16x16 tile of activations over (unit, point) lives as one f32x4 per lane:
// item r is unit 16*t + 4*q + r of point 16*nt + p -- exactly the output
// layout of v_mfma_f32_16x16x{4f32,32f16}. The next layer consumes it as the
// B operand without any data movement; the K order of each A fragment is
// permuted to match (see stage_weights).
#pragma once

#include "device_common.hpp"

namespace tmnn_hip {

// kModeInputGrad: forward + backward from d out_m = 1 for output grad_output,
// storing only dx (the evaluator's position gradient); no weight gradients.
enum : int32_t { kModeForward = 0, kModeTrainLoss = 1, kModeTrainExtGrad = 2, kModeInputGrad = 3 };
enum : int32_t {
  kLossL2 = 0,
  kLossL1 = 1,
  kLossHuber = 2,
  kLossCosine = 3,
  kLossRelL2 = 4
};

constexpr int kNT = 2;             // 16-point MFMA column tiles per wave tile
constexpr int kTilePts = 16 * kNT; // points per wave tile
// LDS row stride (elements) of the [unit][point] staging arrays. fp32: 32
// floats, point index c of row `row` stored at c ^ stage_swz(row); fp16: 40
// halves, rows 16-byte aligned for the 8-half dW operand reads.
__host__ __device__ constexpr int lds_pitch(bool f16) { return f16 ? 40 : 32; }
// fp32 point swizzle (a multiple of 4: 16-byte quads stay whole). The LDS
// serves 4-byte accesses 32 lanes per cycle over 32 banks and 16-byte reads
// 16 lanes per cycle over 64 banks (lane quads of even, then odd, bit parity
// among lanes 0-31, then the same in 32-63). The D-layout stores and ReLU'
// reads (lane p + 16 q: row 4 q + r, point 16 nt + p) and the dW operand
// reads (lane p + 16 q: row p, points 8 q .. 8 q + 7 as two 16-byte reads)
// then each meet every bank of a cycle once.
__device__ __forceinline__ int stage_swz(int row) { return ((row << 1) & 4) | ((row << 2) & 16); }
constexpr int kMaxLayers = 9;      // up to 8 hidden layers + the output layer
constexpr int kBlockThreads = 256;

struct FieldArgs {
  int32_t D, L, F, IN, H, NHL, M;
  uint32_t log2T;
  int32_t n;                // points of this launch
  int32_t n_tiles;          // ceil(n / kTilePts)
  int32_t waves_per_block;
  int32_t mode;             // kMode*
  int32_t grad_output;      // kModeInputGrad: the output row of the Jacobian
  int32_t loss_kind;        // kLoss*
  float huber_delta;
  float inv_n;              // fl(1/N) of the loss (emitScalarTrainKernelImpl)
  float loss_scale;         // power of two applied to d_out in the fp16 path
  float inv_loss_scale;
  int32_t dw_global;        // dW accumulator in grad_partials (LDS too small)
  int32_t mlp_count;
  float res[kMaxLevels];    // per-level resolution table
  const float *pos;         // [n][D]
  const float *xfeat;       // input features as X tiles (encode_kernel.hpp), XMEM kernels
  const float *target;      // [n][M] target (TrainLoss) or d_out (TrainExtGrad)
  const uint32_t *tgt_index;// nullable: point i's target row is tgt_index[i]
  const float *table;       // [L][T][F] fp32
  const float *mlp;         // fp32 master MLP params (reference layout)
  const unsigned char *image; // packed LDS head (pack_image_kernel), s.dw_off bytes
  float *out;               // [n][M] (Forward)
  const uint32_t *out_index;// nullable: row of out[] for point i
  float *dx_out;            // [n][IN] input-feature gradients (training)
  uint64_t *wide_mask;      // wide kernel: ReLU bits of hidden layers [NHL-1][n_tiles][64 lanes]
  _Float16 *wide_act;       // wide kernel: hidden activations [NHL-1][n_tiles][128][32] (fp16 training)
  float *grad_partials;     // [gridDim.x][mlp_count]
  float *loss_partials;     // [gridDim.x]
  float *amax_partials;     // nullable: [gridDim.x] largest |output| of the block's points
  // training kernels with the hash-grid backward fused (tile_scatter.hpp):
  const float *spos;        // [n][D] positions in tile order
  int32_t *grad_hash;       // [L][T][F] int32 fixed point
  uint8_t *mask;            // [L][T] visit flags
};

// LDS plan of one launch, evaluated identically on host and device. All
// per-layer offsets are closed-form in the layer index (no runtime-indexed
// arrays, which would live in scratch memory on the device).
struct FieldLayout {
  int32_t INP, HP, IN, H, NHL, M, es, okt;  // okt: K width of output-layer bwd
  int32_t lo_base;              // fp16: LDS bytes of the forward low-part fragments
  int32_t bwd_base, bias_base;
  int32_t res_off;              // LDS bytes: fp32 resolution table
  int32_t dw_off;               // LDS bytes: fp32 dW accumulator
  int32_t red_off;              // LDS bytes: fp32 per-wave reduction slots
  int32_t wave_off;             // LDS bytes: first wave's activation region
  int32_t wave_bytes;
  int32_t xs_off, hs_off, ds_off;  // within a wave region: X, hidden layers, output grad
  int32_t dw_global;            // 1: dW accumulates in the block's global partial row
  int32_t total;

  // LDS bytes of the forward A fragments (W_k^T) of layer k (k == NHL: output)
  __host__ __device__ __forceinline__ int32_t fwd_off(int k) const {
    if (k == 0) return 0;
    return INP * HP * es + (k - 1) * HP * HP * es;
  }
  // LDS bytes of the forward low-part fragments fp16(W - fp16(W)) of layer k
  __host__ __device__ __forceinline__ int32_t fwd_lo_off(int k) const { return lo_base + fwd_off(k); }
  // LDS bytes of the backward A fragments (W_k) of layer k
  __host__ __device__ __forceinline__ int32_t bwd_off(int k) const {
    if (k == 0) return bwd_base;
    return bwd_base + INP * HP * es + (k - 1) * HP * HP * es;
  }
  // LDS bytes of the fp32 bias of layer k (padded to HP; output to 16)
  __host__ __device__ __forceinline__ int32_t bias_off(int k) const { return bias_base + k * HP * 4; }
  // element offsets in the reference weight layout
  // [W0 (IN x H), b0, (W_k (H x H), b_k)..., WO (H x M), bO]
  __host__ __device__ __forceinline__ int32_t w_off(int k) const {
    return k == 0 ? 0 : IN * H + H + (k - 1) * (H * H + H);
  }
  __host__ __device__ __forceinline__ int32_t b_off(int k) const {
    return w_off(k) + (k == 0 ? IN * H : (k == NHL ? H * M : H * H));
  }
  __host__ __device__ __forceinline__ int32_t mlp_count() const { return b_off(NHL) + M; }
};

__host__ __device__ __forceinline__ int32_t round_up(int32_t v, int32_t m) {
  return (v + m - 1) / m * m;
}

__host__ __device__ __forceinline__ FieldLayout make_layout(int INP, int HP, int IN,
                                                   int H, int NHL, int M,
                                                   int mlp_count, bool f16,
                                                   bool train, int wpb,
                                                   bool dw_global = false,
                                                   bool reg_dw = false) {
  FieldLayout s;
  s.INP = INP; s.HP = HP; s.IN = IN; s.H = H; s.NHL = NHL; s.M = M;
  s.es = f16 ? 2 : 4;
  s.okt = f16 ? 32 : 16;
  const int fwd_bytes = (INP * HP + (NHL - 1) * HP * HP + HP * 16) * s.es;
  const int bwd_bytes = (INP * HP + (NHL - 1) * HP * HP + HP * s.okt) * s.es;
  // fp16: the forward runs on split operands (hi + lo halves, three MFMAs per
  // product), so the low-part fragments follow the high-part ones.
  s.lo_base = fwd_bytes;
  int off = f16 ? 2 * fwd_bytes : fwd_bytes;
  s.bwd_base = off;
  if (train) off += bwd_bytes;
  s.bias_base = off;
  off += (NHL * HP + 16) * 4;
  s.res_off = off;
  off += kMaxLevels * 4;
  off = round_up(off, 16);  // end of the packed image (copied in 16-byte units)
  s.dw_off = off;
  s.dw_global = dw_global ? 1 : 0;
  if (train && !dw_global && !reg_dw) off += round_up(mlp_count, 4) * 4;
  s.red_off = off;
  off += round_up(wpb, 4) * 4;
  off = round_up(off, 16);
  s.wave_off = off;
  s.xs_off = 0;
  const int pitch = lds_pitch(f16) * s.es;
  s.hs_off = INP * pitch;
  s.ds_off = s.hs_off + NHL * HP * pitch;
  // the delta region holds the output gradient's 16-row tile only: a hidden
  // layer's delta is staged over that layer's activations (their ReLU mask is
  // applied before the delta is stored)
  s.wave_bytes = train ? round_up(s.ds_off + 16 * pitch, 16) : 0;
  off += wpb * s.wave_bytes;
  // Register-accumulated dW is reduced across the block's waves through LDS
  // at the end of the kernel, over the then idle weight/activation space.
  // (red_slot permutes within 64-float rows, so the array spans whole rows)
  if (train && reg_dw) off = off > round_up(mlp_count, 64) * 4 ? off : round_up(mlp_count, 64) * 4;
  s.total = off;
  return s;
}

// ---------------------------------------------------------------- helpers --

__device__ __forceinline__ void wave_lds_sync() {
  // LDS traffic of one wave executes in issue order; this only keeps the
  // compiler from moving LDS accesses across the point where lanes start
  // reading what other lanes of the same wave wrote.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ half8 pack8(f32x4 a, f32x4 b) {
  half8 r;
  r[0] = static_cast<_Float16>(a[0]);
  r[1] = static_cast<_Float16>(a[1]);
  r[2] = static_cast<_Float16>(a[2]);
  r[3] = static_cast<_Float16>(a[3]);
  r[4] = static_cast<_Float16>(b[0]);
  r[5] = static_cast<_Float16>(b[1]);
  r[6] = static_cast<_Float16>(b[2]);
  r[7] = static_cast<_Float16>(b[3]);
  return r;
}

// out[MT][nt] = A(frag) x in[KT][nt]: one dense layer over the wave tile.
// f16: K step 32 (two 16-unit input tiles) per v_mfma_f32_16x16x32_f16.
// f32: four v_mfma_f32_16x16x4_f32 per 16-unit input tile.
template <bool F16, int KT, int MT>
__device__ __forceinline__ void layer_mma(const unsigned char *frag,
                                          const f32x4 (&in)[KT][kNT],
                                          f32x4 (&out)[MT][kNT], int lane) {
  if constexpr (F16) {
    static_assert(KT % 2 == 0, "fp16 K tiles come in pairs");
    constexpr int KS = KT / 2;
    half8 b[KS][kNT];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int nt = 0; nt < kNT; ++nt) b[ks][nt] = pack8(in[2 * ks][nt], in[2 * ks + 1][nt]);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      f32x4 acc[kNT];
#pragma unroll
      for (int nt = 0; nt < kNT; ++nt) acc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const half8 av =
            *reinterpret_cast<const half8 *>(frag + ((mt * KS + ks) * 64 + lane) * 16);
#pragma unroll
        for (int nt = 0; nt < kNT; ++nt)
          acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, b[ks][nt], acc[nt], 0, 0, 0);
      }
#pragma unroll
      for (int nt = 0; nt < kNT; ++nt) out[mt][nt] = acc[nt];
    }
  } else {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      f32x4 acc[kNT];
#pragma unroll
      for (int nt = 0; nt < kNT; ++nt) acc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) {
        const f32x4 av =
            *reinterpret_cast<const f32x4 *>(frag + ((mt * KT + kt) * 64 + lane) * 16);
#pragma unroll
        for (int nt = 0; nt < kNT; ++nt)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            acc[nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[r], in[kt][nt][r], acc[nt], 0, 0, 0);
      }
#pragma unroll
      for (int nt = 0; nt < kNT; ++nt) out[mt][nt] = acc[nt];
    }
  }
}

// fp16 split of two D-layout tiles: hi = fp16(v), lo = fp16(v - hi). hi*hi
// products are exact in the fp32 accumulator and hi + lo carries ~22 bits.
// v - hi is exact in fp32, so it is formed as fma(hi, m1, v) with m1 = -1
// held opaque in a scalar register: the compiler then selects v_fma_mix,
// which reads hi straight out of the packed pair (one v_cvt_pk per pair for
// hi, no separate fp16 -> fp32 conversions), with bit-identical results.
__device__ __forceinline__ void pack8_split(f32x4 a, f32x4 b, half8 &hi, half8 &lo) {
  float m1 = -1.0f;
  asm volatile("" : "+s"(m1));  // emits nothing; keeps the fma from folding into a subtraction
#pragma unroll
  for (int r = 0; r < 4; r += 2) {
    const half2v ha = __builtin_convertvector(f32x2{a[r], a[r + 1]}, half2v);
    const half2v hb = __builtin_convertvector(f32x2{b[r], b[r + 1]}, half2v);
    hi[r] = ha[0];
    hi[r + 1] = ha[1];
    hi[r + 4] = hb[0];
    hi[r + 5] = hb[1];
    lo[r] = static_cast<_Float16>(__builtin_fmaf(static_cast<float>(ha[0]), m1, a[r]));
    lo[r + 1] = static_cast<_Float16>(__builtin_fmaf(static_cast<float>(ha[1]), m1, a[r + 1]));
    lo[r + 4] = static_cast<_Float16>(__builtin_fmaf(static_cast<float>(hb[0]), m1, b[r]));
    lo[r + 5] = static_cast<_Float16>(__builtin_fmaf(static_cast<float>(hb[1]), m1, b[r + 1]));
  }
}

// Forward layer on split fp16 operands: out = A x in with A = Ahi + Alo and
// in = Bhi + Blo, accumulated as Alo*Bhi + Ahi*Blo + Ahi*Bhi in fp32 (the
// dropped Alo*Blo term is ~2^-22 relative). Keeps the fp16 training forward
// within fp32 rounding of the reference's fp32 math.
template <int KT, int MT>
__device__ __forceinline__ void layer_mma_split(const unsigned char *frag_hi,
                                                const unsigned char *frag_lo,
                                                const f32x4 (&in)[KT][kNT],
                                                f32x4 (&out)[MT][kNT], int lane) {
  static_assert(KT % 2 == 0, "fp16 K tiles come in pairs");
  constexpr int KS = KT / 2;
  half8 bh[KS][kNT], bl[KS][kNT];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks)
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt)
      pack8_split(in[2 * ks][nt], in[2 * ks + 1][nt], bh[ks][nt], bl[ks][nt]);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    f32x4 acc[kNT];
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt) acc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int off = ((mt * KS + ks) * 64 + lane) * 16;
      const half8 ah = *reinterpret_cast<const half8 *>(frag_hi + off);
      const half8 al = *reinterpret_cast<const half8 *>(frag_lo + off);
#pragma unroll
      for (int nt = 0; nt < kNT; ++nt) {
        acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bh[ks][nt], acc[nt], 0, 0, 0);
        acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bl[ks][nt], acc[nt], 0, 0, 0);
        acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh[ks][nt], acc[nt], 0, 0, 0);
      }
    }
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt) out[mt][nt] = acc[nt];
  }
}

// Forward layer in the kernel's precision: fp32 MFMA, or split fp16.
template <bool F16, int KT, int MT>
__device__ __forceinline__ void layer_fwd(const FieldLayout &s, const unsigned char *smem,
                                          int k, const f32x4 (&in)[KT][kNT],
                                          f32x4 (&out)[MT][kNT], int lane) {
  if constexpr (F16)
    layer_mma_split<KT, MT>(smem + s.fwd_off(k), smem + s.fwd_lo_off(k), in, out, lane);
  else
    layer_mma<false, KT, MT>(smem + s.fwd_off(k), in, out, lane);
}

// acc + one 16x16 tile of sum over the 32 tile points of
// A[row0 + i][pt] * B[col0 + j][pt], both read from [unit][point] LDS arrays.
template <bool F16>
__device__ __forceinline__ f32x4 dw_tile(const unsigned char *A, int row0,
                                         const unsigned char *B, int col0,
                                         int p, int q,
                                         f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f}) {
  if constexpr (F16) {
    constexpr int ps = lds_pitch(true);
    const half8 av = *reinterpret_cast<const half8 *>(A + ((row0 + p) * ps + 8 * q) * 2);
    const half8 bv = *reinterpret_cast<const half8 *>(B + ((col0 + p) * ps + 8 * q) * 2);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, acc, 0, 0, 0);
  } else {
    // K slot q of MFMA step 4 h + e takes point 8 q + 4 h + e (the same
    // permutation of the 32 points in both operands)
    constexpr int ps = lds_pitch(false);
    const float *Ar = reinterpret_cast<const float *>(A) + (row0 + p) * ps;
    const float *Br = reinterpret_cast<const float *>(B) + (col0 + p) * ps;
    const int sa = stage_swz(row0 + p), sb = stage_swz(col0 + p);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const f32x4 av = *reinterpret_cast<const f32x4 *>(Ar + ((8 * q + 4 * h) ^ sa));
      const f32x4 bv = *reinterpret_cast<const f32x4 *>(Br + ((8 * q + 4 * h) ^ sb));
#pragma unroll
      for (int e = 0; e < 4; ++e) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[e], bv[e], acc, 0, 0, 0);
    }
  }
  return acc;
}

// Store a D-layout tile set to an LDS [unit][point] array.
template <bool F16, int MT>
__device__ __forceinline__ void store_tiles(unsigned char *dst,
                                            const f32x4 (&t)[MT][kNT], int p,
                                            int q) {
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 16 * mt + 4 * q + r, pt = 16 * nt + p;
        if constexpr (F16)
          reinterpret_cast<_Float16 *>(dst)[row * lds_pitch(true) + pt] =
              static_cast<_Float16>(t[mt][nt][r]);
        else
          reinterpret_cast<float *>(dst)[row * lds_pitch(false) + (pt ^ stage_swz(row))] = t[mt][nt][r];
      }
}

// delta *= [h > 0] with h read back from the stored forward activations.
template <bool F16, int MT>
__device__ __forceinline__ void relu_mask(f32x4 (&t)[MT][kNT],
                                          const unsigned char *h, int p,
                                          int q) {
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 16 * mt + 4 * q + r, pt = 16 * nt + p;
        float hv;
        if constexpr (F16)
          hv = static_cast<float>(reinterpret_cast<const _Float16 *>(h)[row * lds_pitch(true) + pt]);
        else
          hv = reinterpret_cast<const float *>(h)[row * lds_pitch(false) + (pt ^ stage_swz(row))];
        t[mt][nt][r] = hv > 0.0f ? t[mt][nt][r] : 0.0f;
      }
}

// Sum over the 16 lanes p of one q group.
__device__ __forceinline__ float sum_over_p(float v) {
  v += __shfl_xor(v, 1);
  v += __shfl_xor(v, 2);
  v += __shfl_xor(v, 4);
  v += __shfl_xor(v, 8);
  return v;
}

// ----------------------------------------------------------- encode / hash --

// Features of one level (F values), corner loop in the reference's order.
template <int D, int F>
__device__ __forceinline__ void encode_level(const float *table, uint32_t log2T,
                                             int l, const float *p, float res,
                                             float *feat) {
  const Cell<D> c = cell_of<D>(p, res);
  const uint32_t tmask = (1u << log2T) - 1u;
#pragma unroll
  for (int f = 0; f < F; ++f) feat[f] = 0.0f;
#pragma unroll
  for (int k = 0; k < (1 << D); ++k) {
    int co[D];
    float wc[D];
    corner_of<D>(c, k, co, wc);
    const uint32_t h = hash_corner<D>(co, tmask);
    const float w = corner_weight<D>(wc);
    const float *e = table + ((static_cast<size_t>(l) << log2T) + h) * F;
    if constexpr (F == 1) {
      feat[0] = feat[0] + w * e[0];
    } else if constexpr (F == 2) {
      const f32x2 t = *reinterpret_cast<const f32x2 *>(e);
      feat[0] = feat[0] + w * t[0];
      feat[1] = feat[1] + w * t[1];
    } else {
      const f32x4 t = *reinterpret_cast<const f32x4 *>(e);
#pragma unroll
      for (int f = 0; f < 4; ++f) feat[f] = feat[f] + w * t[f];
    }
  }
}

// Input features fb .. fb+3 of one point (zero past L*F).
template <int D, int F>
__device__ __forceinline__ f32x4 encode_quad_t(const FieldArgs &a,
                                               const float *res, int fb,
                                               const float *p) {
  f32x4 o = {0.f, 0.f, 0.f, 0.f};
  if constexpr (F == 1) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int l = fb + r;
      if (l < a.L) {
        float v[1];
        encode_level<D, 1>(a.table, a.log2T, l, p, res[l], v);
        o[r] = v[0];
      }
    }
  } else if constexpr (F == 2) {
#pragma unroll
    for (int lv = 0; lv < 2; ++lv) {
      const int l = fb / 2 + lv;
      if (l < a.L) {
        float v[2];
        encode_level<D, 2>(a.table, a.log2T, l, p, res[l], v);
        o[2 * lv] = v[0];
        o[2 * lv + 1] = v[1];
      }
    }
  } else {
    const int l = fb / 4;
    if (l < a.L) {
      float v[4];
      encode_level<D, 4>(a.table, a.log2T, l, p, res[l], v);
      o = f32x4{v[0], v[1], v[2], v[3]};
    }
  }
  return o;
}

// Encode every input quad of the wave tile for one (D, F): a runtime loop
// over (kt, nt) keeps one copy of the gather code; results land in the
// register tile through compile-time-indexed selects.
template <int D, int F, int KT0>
__device__ __forceinline__ void encode_tile_t(const FieldArgs &a,
                                              const float *res, int q,
                                              const float (&P)[kNT][4],
                                              f32x4 (&X)[KT0][kNT]) {
#pragma unroll
  for (int nt = 0; nt < kNT; ++nt) {
    const float pp[4] = {P[nt][0], P[nt][1], P[nt][2], P[nt][3]};
#pragma unroll 1
    for (int kt = 0; kt < KT0; ++kt) {
      const f32x4 v = encode_quad_t<D, F>(a, res, 16 * kt + 4 * q, pp);
#pragma unroll
      for (int j = 0; j < KT0; ++j)
        if (j == kt) X[j][nt] = v;
    }
  }
}

// DF = D * 8 + F selects the geometry at compile time; DF == 0 dispatches on
// the runtime geometry.
template <int KT0, int DF>
__device__ __forceinline__ void encode_tile(const FieldArgs &a, const float *res,
                                            int q, const float (&P)[kNT][4],
                                            f32x4 (&X)[KT0][kNT]) {
  if constexpr (DF != 0) {
    encode_tile_t<DF / 8, DF % 8, KT0>(a, res, q, P, X);
    return;
  }
  switch (a.D * 8 + a.F) {
    case 2 * 8 + 1: encode_tile_t<2, 1, KT0>(a, res, q, P, X); break;
    case 2 * 8 + 2: encode_tile_t<2, 2, KT0>(a, res, q, P, X); break;
    case 2 * 8 + 4: encode_tile_t<2, 4, KT0>(a, res, q, P, X); break;
    case 3 * 8 + 1: encode_tile_t<3, 1, KT0>(a, res, q, P, X); break;
    case 3 * 8 + 2: encode_tile_t<3, 2, KT0>(a, res, q, P, X); break;
    case 3 * 8 + 4: encode_tile_t<3, 4, KT0>(a, res, q, P, X); break;
    case 4 * 8 + 1: encode_tile_t<4, 1, KT0>(a, res, q, P, X); break;
    case 4 * 8 + 2: encode_tile_t<4, 2, KT0>(a, res, q, P, X); break;
    default: encode_tile_t<4, 4, KT0>(a, res, q, P, X); break;
  }
}

// ----------------------------------------------- software-pipelined encode --
//
// The geometry-specialised kernels split the encode of a wave tile in two:
// gather_issue computes the corners and issues every table load of the tile
// into registers; gather_finish (one tile later in program order, after the
// previous tile's backward) applies the corner weights. The loads of tile i+1
// are in flight while tile i runs its MLP backward.

template <int D, int F, int KT0>
struct Gathered {
  static constexpr int LPQ = 4 / F;  // levels per feature quad
  static constexpr int C = 1 << D;   // corners per level
  float v[kNT][KT0][LPQ][C][F];
};

template <int D, int F, int KT0>
__device__ __forceinline__ void gather_issue(const FieldArgs &a, const float *res, int q,
                                             const float (&P)[kNT][4],
                                             Gathered<D, F, KT0> &g) {
  constexpr int LPQ = Gathered<D, F, KT0>::LPQ;
  const uint32_t tmask = (1u << a.log2T) - 1u;
#pragma unroll
  for (int nt = 0; nt < kNT; ++nt)
#pragma unroll
    for (int kt = 0; kt < KT0; ++kt)
#pragma unroll
      for (int lv = 0; lv < LPQ; ++lv) {
        const int l = (16 * kt + 4 * q) / F + lv;
        const bool on = l < a.L;
        const Cell<D> c = cell_of<D>(P[nt], res[on ? l : 0]);
#pragma unroll
        for (int k = 0; k < (1 << D); ++k) {
          int co[D];
          float wc[D];
          corner_of<D>(c, k, co, wc);
          const uint32_t h = hash_corner<D>(co, tmask);
          const float *e = a.table + ((static_cast<size_t>(on ? l : 0) << a.log2T) + h) * F;
          if constexpr (F == 1) {
            g.v[nt][kt][lv][k][0] = on ? e[0] : 0.0f;
          } else if constexpr (F == 2) {
            const f32x2 t = on ? *reinterpret_cast<const f32x2 *>(e) : f32x2{0.f, 0.f};
            g.v[nt][kt][lv][k][0] = t[0];
            g.v[nt][kt][lv][k][1] = t[1];
          } else {
            const f32x4 t = on ? *reinterpret_cast<const f32x4 *>(e) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int f = 0; f < 4; ++f) g.v[nt][kt][lv][k][f] = t[f];
          }
        }
      }
}

// Interpolation of gathered corners in the reference's order (features start
// at 0, corners z, y, x ascending, weight ((wx * wy) * wz)(* wt)).
template <int D, int F, int KT0>
__device__ __forceinline__ void gather_finish(const FieldArgs &a, const float *res, int q,
                                              const float (&P)[kNT][4],
                                              const Gathered<D, F, KT0> &g,
                                              f32x4 (&X)[KT0][kNT]) {
  constexpr int LPQ = Gathered<D, F, KT0>::LPQ;
#pragma unroll
  for (int nt = 0; nt < kNT; ++nt)
#pragma unroll
    for (int kt = 0; kt < KT0; ++kt) {
      f32x4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int lv = 0; lv < LPQ; ++lv) {
        const int l = (16 * kt + 4 * q) / F + lv;
        const Cell<D> c = cell_of<D>(P[nt], res[l < a.L ? l : 0]);
        float feat[F];
#pragma unroll
        for (int f = 0; f < F; ++f) feat[f] = 0.0f;
#pragma unroll
        for (int k = 0; k < (1 << D); ++k) {
          int co[D];
          float wc[D];
          corner_of<D>(c, k, co, wc);
          const float w = corner_weight<D>(wc);
#pragma unroll
          for (int f = 0; f < F; ++f) feat[f] = feat[f] + w * g.v[nt][kt][lv][k][f];
        }
#pragma unroll
        for (int f = 0; f < F; ++f) o[lv * F + f] = l < a.L ? feat[f] : 0.0f;
      }
      X[kt][nt] = o;
    }
}

// ------------------------------------------------------------ LDS staging --


// ----------------------------------------------------- weight image packing --
//
// The head of the kernel's LDS plan -- [fwd A fragments (hi) | fwd lo
// fragments (fp16) | bwd A fragments | fp32 biases | resolution table] -- is
// the same for every block, so it is built once per weight update by
// pack_image_kernel (one thread per element) and each block copies it into
// LDS with 16-byte loads.

enum : int32_t { kSecFwd = 0, kSecBwd = 1, kSecBias = 2, kSecRes = 3 };
constexpr int kMaxSections = 3 * kMaxLayers + 1;

struct PackArgs {
  FieldLayout s;
  int32_t f16;
  int32_t L;
  int32_t nsec;
  int32_t sec_start[kMaxSections + 1];  // element prefix over the sections
  int32_t sec_kind[kMaxSections];
  int32_t sec_layer[kMaxSections];
  float res[kMaxLevels];
  const float *mlp;                      // fp32 master MLP params (reference layout)
  unsigned char *image;                  // s.dw_off bytes
};

// K-slot order of one fp16 A fragment: slot (q, j) of K step ks covers unit
// 32*ks + 4*q + j (j < 4) or 32*ks + 16 + 4*q + (j - 4) (j >= 4), matching
// pack8() of two D-layout tiles.
__host__ __device__ __forceinline__ int kslot_f16(int ks, int q, int j) {
  return 32 * ks + (j < 4 ? 4 * q + j : 16 + 4 * q + (j - 4));
}

// Value of element e of layer k's forward (A = W_k^T) or backward (A = W_k)
// fragments: the fragment slot -> (input unit i, output unit o) mapping.
__host__ __device__ __forceinline__ float frag_value(const PackArgs &a, int k, bool bwd, int e) {
  const FieldLayout &s = a.s;
  const int kin = k == 0 ? s.INP : s.HP;
  const int kreal = k == 0 ? s.IN : s.H;
  const int mout = k == s.NHL ? 16 : s.HP;
  const int mreal = k == s.NHL ? s.M : s.H;
  int i, o;
  if (a.f16) {
    const int j = e & 7, lane = (e >> 3) & 63, f = e >> 9;
    if (!bwd) {
      const int ks_n = kin / 32, mt = f / ks_n, ks = f % ks_n;
      i = kslot_f16(ks, lane >> 4, j);
      o = 16 * mt + (lane & 15);
    } else {
      const int ko = round_up(mout, 32);
      const int ks_n = ko / 32, mt = f / ks_n, ks = f % ks_n;
      i = 16 * mt + (lane & 15);
      o = kslot_f16(ks, lane >> 4, j);
    }
  } else {
    const int r = e & 3, lane = (e >> 2) & 63, f = e >> 8;
    if (!bwd) {
      const int kt_n = kin / 16, mt = f / kt_n, kt = f % kt_n;
      i = 16 * kt + 4 * (lane >> 4) + r;
      o = 16 * mt + (lane & 15);
    } else {
      const int kt_n = mout / 16, mt = f / kt_n, kt = f % kt_n;
      i = 16 * mt + (lane & 15);
      o = 16 * kt + 4 * (lane >> 4) + r;
    }
  }
  return (i < kreal && o < mreal) ? a.mlp[s.w_off(k) + i * mreal + o] : 0.0f;
}

__global__ void pack_image_kernel(PackArgs a) {
  const int g = blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= a.sec_start[a.nsec]) return;
  int sec = 0;
  while (g >= a.sec_start[sec + 1]) ++sec;
  const int e = g - a.sec_start[sec];
  const int k = a.sec_layer[sec];
  const FieldLayout &s = a.s;
  switch (a.sec_kind[sec]) {
    case kSecFwd: {
      const float v = frag_value(a, k, false, e);
      if (a.f16) {
        const _Float16 hi = static_cast<_Float16>(v);
        reinterpret_cast<_Float16 *>(a.image + s.fwd_off(k))[e] = hi;
        reinterpret_cast<_Float16 *>(a.image + s.fwd_lo_off(k))[e] =
            static_cast<_Float16>(v - static_cast<float>(hi));
      } else {
        reinterpret_cast<float *>(a.image + s.fwd_off(k))[e] = v;
      }
      break;
    }
    case kSecBwd: {
      const float v = frag_value(a, k, true, e);
      if (a.f16)
        reinterpret_cast<_Float16 *>(a.image + s.bwd_off(k))[e] = static_cast<_Float16>(v);
      else
        reinterpret_cast<float *>(a.image + s.bwd_off(k))[e] = v;
      break;
    }
    case kSecBias: {
      const int mreal = k == s.NHL ? s.M : s.H;
      reinterpret_cast<float *>(a.image + s.bias_off(k))[e] =
          e < mreal ? a.mlp[s.b_off(k) + e] : 0.0f;
      break;
    }
    default:
      reinterpret_cast<float *>(a.image + s.res_off)[e] = e < a.L ? a.res[e] : 0.0f;
      break;
  }
}

// Block-wide copy of `bytes` (a multiple of 16) from global memory into LDS.
// Whole 1 KB chunks go by direct global-to-LDS loads (global_load_lds_dwordx4:
// lane i's 16 bytes land at the wave-uniform LDS base + 16 i), which need no
// registers and keep every chunk of the copy in flight at once; the rest goes
// through registers. Returns once this thread's part has landed; the caller's
// barrier publishes the copy to the block.
__device__ __forceinline__ void copy_to_lds(unsigned char *dst, const unsigned char *src,
                                            int bytes) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const int chunks = bytes >> 10;
  for (int c = wave; c < chunks; c += nw)
    __builtin_amdgcn_global_load_lds(src + (c << 10) + lane * 16,
                                     (__attribute__((address_space(3))) void *)(dst + (c << 10)),
                                     16, 0, 0);
  const uint4 *s = reinterpret_cast<const uint4 *>(src);
  uint4 *d = reinterpret_cast<uint4 *>(dst);
  for (int e = (chunks << 6) + threadIdx.x; e < bytes / 16; e += blockDim.x) d[e] = s[e];
  __builtin_amdgcn_s_waitcnt(0);  // the direct loads (vmcnt) and the stores have completed
}

// Block-wide copy of the packed image into LDS (+ zeroing of an LDS or
// global dW accumulator for the generic kernels).
template <bool TRAIN, bool REGDW>
__device__ __forceinline__ void stage_weights(const FieldArgs &a, const FieldLayout &s,
                                              unsigned char *smem) {
  const int tid = threadIdx.x;
  const int nthr = blockDim.x;
  copy_to_lds(smem, a.image, s.dw_off);
  if constexpr (TRAIN && !REGDW) {
    if (s.dw_global) {
      float *dwg = a.grad_partials + static_cast<size_t>(blockIdx.x) * a.mlp_count;
      for (int e = tid; e < a.mlp_count; e += nthr) dwg[e] = 0.0f;
    } else {
      const int nd = round_up(a.mlp_count, 4);
      for (int e = tid; e < nd; e += nthr)
        reinterpret_cast<float *>(smem + s.dw_off)[e] = 0.0f;
    }
  }
}

// ------------------------------------------------------------------ loss ----

// Loss term and output gradient of one element (emitLoss, L2/L1/Huber; and
// RelativeL2 = r^2/(y^2+0.01) with the denominator held constant). FAST_RCP
// (fp16 training only, whose gradient is rounded to fp16 next) takes the
// RelativeL2 reciprocal from v_rcp_f32 (1 ulp) instead of a division.
template <int KIND, bool FAST_RCP>
__device__ __forceinline__ float elem_loss(float y, float t, float delta, float inv_n, float *d) {
  const float r = y - t;
  if constexpr (KIND == kLossL1) {
    *d = (r > 0.0f ? 1.0f : (r < 0.0f ? -1.0f : 0.0f)) * inv_n;
    return fabsf(r);
  } else if constexpr (KIND == kLossHuber) {
    const float ar = fabsf(r);
    if (ar <= delta) {
      *d = r * inv_n;
      return (0.5f * r) * r;
    }
    *d = (delta * (r > 0.0f ? 1.0f : -1.0f)) * inv_n;
    return delta * (ar - 0.5f * delta);
  } else if constexpr (KIND == kLossRelL2) {
    const float den = y * y + 0.01f;
    const float inv = FAST_RCP ? __builtin_amdgcn_rcpf(den) : 1.0f / den;
    *d = ((2.0f * r) * inv) * inv_n;
    return (r * r) * inv;
  } else {
    *d = (2.0f * r) * inv_n;
    return r * r;
  }
}

// Loss terms and output gradients of the valid outputs of a wave tile for a
// compile-time loss kind (the kind is uniform: one branch per tile).
template <int KIND, bool FAST_RCP>
__device__ __forceinline__ void tile_loss(const FieldArgs &a, const f32x4 (&y)[1][kNT],
                                          const float (&Tv)[kNT][4], const bool (&valid)[kNT],
                                          int q, float &lane_loss, f32x4 &g0, f32x4 &g1) {
#pragma unroll
  for (int nt = 0; nt < kNT; ++nt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int o = 4 * q + r;
      if (valid[nt] && o < a.M) {
        float d;
        lane_loss += elem_loss<KIND, FAST_RCP>(y[0][nt][r], Tv[nt][r], a.huber_delta, a.inv_n, &d);
        (nt == 0 ? g0 : g1)[r] = d * a.loss_scale;
      }
    }
}

// Loss term and output gradient of one wave tile (emitLoss,
// mlp_kernel_emitter.cpp:562-670) in D layout: output 4*q + r of point
// 16*nt + p. kModeInputGrad instead writes the outputs and seeds
// d out_{grad_output} = 1; kModeTrainExtGrad takes d_out from Tv.
// Training modes also keep the largest |output| of the lane's points in
// lane_amax (the numerics report's activation term), and with a.out set
// write the outputs to row a.out_index[pt] (or pt) of a.out (the parity
// read-out of a training step's forward).
template <int OKT, bool FAST_RCP = false>
__device__ __forceinline__ void output_grad(const FieldArgs &a, const f32x4 (&y)[1][kNT],
                                            const float (&Tv)[kNT][4], const bool (&valid)[kNT],
                                            const int (&pt)[kNT], int q, float &lane_loss,
                                            float &lane_amax, f32x4 (&g)[OKT][kNT]) {
#pragma unroll
  for (int t = 0; t < OKT; ++t)
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt) g[t][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (a.mode != kModeInputGrad) {
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (valid[nt] && 4 * q + r < a.M) lane_amax = fmaxf(lane_amax, fabsf(y[0][nt][r]));
    if (a.out) {  // uniform
#pragma unroll
      for (int nt = 0; nt < kNT; ++nt) {
        if (!valid[nt]) continue;
        const size_t row = a.out_index ? a.out_index[pt[nt]] : static_cast<uint32_t>(pt[nt]);
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (4 * q + r < a.M) a.out[row * a.M + 4 * q + r] = y[0][nt][r];
      }
    }
  }
  if (a.mode == kModeInputGrad) {
    // evaluator gradient pass: outputs once, then d out_m = 1
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt) {
      if (!valid[nt]) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int o = 4 * q + r;
        if (a.out && o < a.M) a.out[static_cast<size_t>(pt[nt]) * a.M + o] = y[0][nt][r];
        if (o == a.grad_output) g[0][nt][r] = 1.0f;
      }
    }
  } else if (a.mode == kModeTrainExtGrad) {
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int o = 4 * q + r;
        if (valid[nt] && o < a.M) g[0][nt][r] = Tv[nt][r] * a.loss_scale;
      }
  } else if (a.loss_kind == kLossCosine) {
    // emitLoss cosine branch (mlp_kernel_emitter.cpp:643-662)
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt) {
      float tv[4];
      float dot = 0.0f, pn = 0.0f, tn = 0.0f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int o = 4 * q + r;
        const bool ok = valid[nt] && o < a.M;
        tv[r] = ok ? Tv[nt][r] : 0.0f;
        const float yv = ok ? y[0][nt][r] : 0.0f;
        dot = dot + yv * tv[r];
        pn = pn + yv * yv;
        tn = tn + tv[r] * tv[r];
      }
      dot += __shfl_xor(dot, 16);
      dot += __shfl_xor(dot, 32);
      pn += __shfl_xor(pn, 16);
      pn += __shfl_xor(pn, 32);
      tn += __shfl_xor(tn, 16);
      tn += __shfl_xor(tn, 32);
      const float pnorm = sqrtf(pn + 1e-8f);
      const float tnorm = sqrtf(tn + 1e-8f);
      const float denom = pnorm * tnorm;
      const float cosine = dot / denom;
      const float pdenom = pn + 1e-8f;
      if (valid[nt]) {
        if (q == 0) lane_loss += 1.0f - cosine;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int o = 4 * q + r;
          if (o < a.M) {
            const float t1 = (cosine * y[0][nt][r]) / pdenom;
            const float t2 = tv[r] / denom;
            g[0][nt][r] = ((t1 - t2) * a.inv_n) * a.loss_scale;
          }
        }
      }
    }
  } else {
    static_assert(kNT == 2, "two point tiles per wave tile");
    switch (a.loss_kind) {
      case kLossL1:
        tile_loss<kLossL1, FAST_RCP>(a, y, Tv, valid, q, lane_loss, g[0][0], g[0][1]);
        break;
      case kLossHuber:
        tile_loss<kLossHuber, FAST_RCP>(a, y, Tv, valid, q, lane_loss, g[0][0], g[0][1]);
        break;
      case kLossRelL2:
        tile_loss<kLossRelL2, FAST_RCP>(a, y, Tv, valid, q, lane_loss, g[0][0], g[0][1]);
        break;
      default:
        tile_loss<kLossL2, FAST_RCP>(a, y, Tv, valid, q, lane_loss, g[0][0], g[0][1]);
        break;
    }
  }
}

// End of a training launch: the block's loss partial (each wave's lane sum,
// then the waves in order) into a.loss_partials[blockIdx.x] and, when
// a.amax_partials is set, the largest |output| of the block's points. lred
// holds one float per wave in LDS; every thread of the block calls this.
__device__ __forceinline__ void block_loss_partials(const FieldArgs &a, float lane_loss,
                                                    float lane_amax, float *lred, int lane,
                                                    int wave, int waves) {
  float v = lane_loss;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) v += __shfl_xor(v, off);
  if (lane == 0) lred[wave] = v;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = 0.0f;
    for (int w = 0; w < waves; ++w) t += lred[w];
    a.loss_partials[blockIdx.x] = t;
  }
  if (a.amax_partials == nullptr) return;  // uniform
  float m = lane_amax;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) m = fmaxf(m, __shfl_xor(m, off));
  __syncthreads();
  if (lane == 0) lred[wave] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = 0.0f;
    for (int w = 0; w < waves; ++w) t = fmaxf(t, lred[w]);
    a.amax_partials[blockIdx.x] = t;
  }
}

// ---------------------------------------------------------------- kernel ----

// Compile-time layer index for the unrolled backward (value > 0) and the
// runtime one of the generic kernel (value 0, index in .runtime).
template <int V>
struct LayerC {
  static constexpr int value = V;
  int runtime = 0;
};
struct RuntimeLayer : LayerC<0> {
  __device__ explicit RuntimeLayer(int k) { runtime = k; }
};

// f(LayerC<N>), f(LayerC<N-1>), ..., f(LayerC<1>).
template <int N, class Fn>
__device__ __forceinline__ void static_for_desc(Fn &&f) {
  if constexpr (N >= 1) {
    f(LayerC<N>{});
    static_for_desc<N - 1>(f);
  }
}

// Per-wave dW accumulators, resident in registers across all tiles of a
// wave (used when the hidden-layer count is a compile-time constant). Tile
// orientation matches dw_tile: w0[mt][ft] rows = hidden units 16mt + 4q + r,
// cols = input features 16ft + p; wh[k-1][mt][it] rows = units of layer k,
// cols = units of layer k-1; wo[ut] rows = outputs 4q + r, cols = hidden
// units 16ut + p. b[k][mt][r] / bo[r] hold this lane's share (point lanes p)
// of the bias sums.
template <int HT, int KT0, int NHLT>
struct DwRegs {
  f32x4 w0[HT][KT0];
  f32x4 wh[NHLT > 1 ? NHLT - 1 : 1][HT][HT];
  f32x4 wo[HT];
  float b[NHLT > 0 ? NHLT : 1][HT][4];
  float bo[4];
};

// LDS slot of parameter e in the block's reduction array: a bijection within
// each 64-float row that XORs bits 6-7 of e into bits 0-1 and bits 8-9 into
// bits 3-4. A dW tile's stores (lane p + 16 q: parameter row 16 t + p,
// column 16 m + 4 q + r; rows 64 floats apart at H = 64) then meet 32
// distinct banks in each half wave (unswizzled: 16 lanes per bank).
__device__ __forceinline__ int red_slot(int e) {
  return e ^ (((e >> 6) & 3) | (((e >> 8) & 3) << 3));
}

// red[idx] (+)= v over the block's waves in wave order: wave 0 stores, the
// others add, one wave at a time (deterministic).
__device__ __forceinline__ void red_put(float *red, int idx, float v, bool first) {
  const int i = red_slot(idx);
  red[i] = first ? v : red[i] + v;
}

template <int HT, int KT0, int NHLT>
__device__ __forceinline__ void dw_regs_to_lds(const DwRegs<HT, KT0, NHLT> &R, const FieldArgs &a,
                                               const FieldLayout &s, float *red, int p,
                                               int q, bool first, float scale) {
  const int H = a.H, IN = a.IN, M = a.M;
#pragma unroll
  for (int mt = 0; mt < HT; ++mt)
#pragma unroll
    for (int ft = 0; ft < KT0; ++ft)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int u = 16 * mt + 4 * q + r, f = 16 * ft + p;
        if (u < H && f < IN) red_put(red, s.w_off(0) + f * H + u, R.w0[mt][ft][r] * scale, first);
      }
#pragma unroll
  for (int k = 1; k < NHLT; ++k)
#pragma unroll
    for (int mt = 0; mt < HT; ++mt)
#pragma unroll
      for (int it = 0; it < HT; ++it)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int u = 16 * mt + 4 * q + r, i = 16 * it + p;
          if (u < H && i < H) red_put(red, s.w_off(k) + i * H + u, R.wh[k - 1][mt][it][r] * scale, first);
        }
#pragma unroll
  for (int ut = 0; ut < HT; ++ut)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int o = 4 * q + r, u = 16 * ut + p;
      if (o < M && u < H) red_put(red, s.w_off(NHLT) + u * M + o, R.wo[ut][r] * scale, first);
    }
  // biases: sum the point lanes p, lane p == 0 of each q group writes
#pragma unroll
  for (int k = 0; k < NHLT; ++k)
#pragma unroll
    for (int mt = 0; mt < HT; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float v = sum_over_p(R.b[k][mt][r]);
        const int u = 16 * mt + 4 * q + r;
        if (p == 0 && u < H) red_put(red, s.b_off(k) + u, v * scale, first);
      }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float v = sum_over_p(R.bo[r]);
    const int o = 4 * q + r;
    if (p == 0 && o < M) red_put(red, s.b_off(NHLT) + o, v * scale, first);
  }
}

// The hash-grid backward of one 32-point tile from its dx registers
// (tile_scatter.hpp, which defines it): groups [GB, GE) of (K tile, level
// pair), so a caller may spread a tile's backward over several places.
template <int D, int F, int KT0, int GB = 0, int GE = 2 * KT0>
__device__ __forceinline__ void tile_scatter(const FieldArgs &a, const f32x4 (&dx)[KT0][kNT],
                                             const float (&pos)[kNT][D], const bool (&valid)[kNT],
                                             const float *res, int q);

// The fused kernel body. Template parameters: padded hidden width HP and
// input width INP (MFMA tiles), fp16 (split-fp16 forward, fp16 backward) or
// fp32 MFMA, training or forward only, DF = D * 8 + F (0: runtime geometry),
// NHLT = hidden-layer count (0: runtime count, dW accumulated in LDS;
// > 0: dW accumulated in registers across tiles), XMEM: input features read
// from a.xfeat (written by encode_features_kernel) instead of encoded here,
// SD, SF > 0: the training modes run each tile's hash-grid backward
// (tile_scatter, a D = SD, F = SF grid, positions from a.spos) instead of
// storing dx.
template <int HP, int INP, bool F16, bool TRAIN, int DF, int NHLT, bool XMEM = false, int SD = 0,
          int SF = 0>
__device__ __forceinline__ void field_body(const FieldArgs &a) {
  constexpr int HT = HP / 16;
  constexpr int KT0 = INP / 16;
  constexpr int OKT = F16 ? 2 : 1;  // K tiles of the output-layer backward
  constexpr int es = F16 ? 2 : 4;
  constexpr bool REGDW = TRAIN && NHLT > 0;
  extern __shared__ __align__(16) unsigned char smem[];

  const int NHL = NHLT > 0 ? NHLT : a.NHL;
  const FieldLayout s = make_layout(INP, HP, a.IN, a.H, NHL, a.M,
                                    a.mlp_count, F16, TRAIN, a.waves_per_block,
                                    a.dw_global != 0, REGDW);
  stage_weights<TRAIN, REGDW>(a, s, smem);
  __syncthreads();

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int p = lane & 15;
  const int q = lane >> 4;
  const float *res = reinterpret_cast<const float *>(smem + s.res_off);
  // LDS dW accumulator (runtime layer count): LDS, or (when the model leaves
  // no room) this block's row of grad_partials, zeroed in stage_weights.
  float *dw = s.dw_global
                  ? a.grad_partials + static_cast<size_t>(blockIdx.x) * a.mlp_count
                  : reinterpret_cast<float *>(smem + s.dw_off);
  unsigned char *wb = smem + s.wave_off + wave * s.wave_bytes;
  unsigned char *Xs = wb + s.xs_off;
  unsigned char *Hs = wb + s.hs_off;
  unsigned char *Ds = wb + s.ds_off;
  const int hs_layer_bytes = HP * lds_pitch(F16) * es;
  float lane_loss = 0.0f, lane_amax = 0.0f;

  DwRegs<HT, KT0, NHLT> R;
  if constexpr (REGDW) {
#pragma unroll
    for (int mt = 0; mt < HT; ++mt) {
#pragma unroll
      for (int ft = 0; ft < KT0; ++ft) R.w0[mt][ft] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < (NHLT > 1 ? NHLT - 1 : 1); ++k)
#pragma unroll
        for (int it = 0; it < HT; ++it) R.wh[k][mt][it] = f32x4{0.f, 0.f, 0.f, 0.f};
      R.wo[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < NHLT; ++k)
#pragma unroll
        for (int r = 0; r < 4; ++r) R.b[k][mt][r] = 0.0f;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) R.bo[r] = 0.0f;
  }

  // Positions of a tile (zero past the batch).
  auto load_pos = [&](int t, float (&Pt)[kNT][4]) {
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt) {
      const int i = t * kTilePts + 16 * nt + p;
      const bool ok = t < a.n_tiles && i < a.n;
#pragma unroll
      for (int d = 0; d < 4; ++d)
        Pt[nt][d] = (ok && d < a.D) ? a.pos[static_cast<size_t>(i) * a.D + d] : 0.0f;
    }
  };
  // Specialised kernels pipeline the gathers when the in-flight corner values
  // fit in registers (<= 128 floats per lane; e.g. not for 3D x 4 features).
  constexpr bool kPipe =
      DF != 0 && kNT * KT0 * (DF ? (4 / (DF % 8)) * (1 << (DF / 8)) * (DF % 8) : 0) <= 128;
  // X tile of wave tile t: one 16-byte load per (kt, nt), zero past the batch
  const f32x4 *xt = reinterpret_cast<const f32x4 *>(a.xfeat);
  auto load_x = [&](int t, f32x4 (&Xt)[KT0][kNT]) {
#pragma unroll
    for (int kt = 0; kt < KT0; ++kt)
#pragma unroll
      for (int nt = 0; nt < kNT; ++nt)
        Xt[kt][nt] = t < a.n_tiles
                         ? xt[((static_cast<size_t>(t) * KT0 + kt) * kNT + nt) * 64 + lane]
                         : f32x4{0.f, 0.f, 0.f, 0.f};
  };
  const int tile_stride = gridDim.x * a.waves_per_block;
  int tile = blockIdx.x * a.waves_per_block + wave;
  float P[kNT][4];
  Gathered<(DF ? DF / 8 : 2), (DF ? DF % 8 : 2), KT0> G;
  f32x4 Xn[KT0][kNT];  // XMEM: features of the next tile, in flight
  // the X prefetch runs one tile ahead when its registers are cheap: 32
  // features, or the forward-only kernels (no dW accumulators)
  constexpr bool kPrefetchX = KT0 <= 2 || !TRAIN;
  if constexpr (XMEM) {
    if constexpr (kPrefetchX) load_x(tile, Xn);
  } else {
    load_pos(tile, P);
    if constexpr (kPipe) gather_issue<DF / 8, DF % 8, KT0>(a, res, q, P, G);
  }

  for (; tile < a.n_tiles; tile += tile_stride) {
    const int next = tile + tile_stride;
    int pt[kNT];
    bool valid[kNT];
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt) {
      pt[nt] = tile * kTilePts + 16 * nt + p;
      valid[nt] = pt[nt] < a.n;
    }

    // ---- encode: input features 16*kt + 4*q + r of point 16*nt + p
    f32x4 X[KT0][kNT];
    float Pn[kNT][4];
    if constexpr (XMEM) {
      if constexpr (!kPrefetchX) load_x(tile, Xn);
#pragma unroll
      for (int kt = 0; kt < KT0; ++kt)
#pragma unroll
        for (int nt = 0; nt < kNT; ++nt) X[kt][nt] = Xn[kt][nt];
      if constexpr (kPrefetchX) load_x(next, Xn);
    } else {
      if constexpr (kPipe)
        gather_finish<DF / 8, DF % 8, KT0>(a, res, q, P, G, X);
      else
        encode_tile<KT0, DF>(a, res, q, P, X);
      // prefetch: the next tile's positions
      load_pos(next, Pn);
    }
    // this tile's sorted positions, for the fused hash-grid backward
    constexpr int kSP = SD > 0 ? SD : 1;
    float Ps[kNT][kSP];
    if constexpr (SD > 0) {
      const bool scat = a.mode != kModeInputGrad;  // uniform
#pragma unroll
      for (int nt = 0; nt < kNT; ++nt)
#pragma unroll
        for (int k = 0; k < SD; ++k)
          Ps[nt][k] = (scat && valid[nt]) ? a.spos[static_cast<size_t>(pt[nt]) * SD + k] : 0.0f;
    }
    // this tile's targets / d_out
    float Tv[kNT][4];
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int o = 4 * q + r;
        Tv[nt][r] = (TRAIN && a.mode != kModeInputGrad && valid[nt] && o < a.M)
                        ? a.target[static_cast<size_t>(a.tgt_index ? a.tgt_index[pt[nt]]
                                                                   : static_cast<uint32_t>(pt[nt])) *
                                       a.M + o]
                        : 0.0f;
      }
    if constexpr (TRAIN) store_tiles<F16, KT0>(Xs, X, p, q);

    // ---- MLP forward
    f32x4 act[HT][kNT];
    layer_fwd<F16, KT0, HT>(s, smem, 0, X, act, lane);
    auto hidden_fwd = [&](int k) {
      if (k > 0) {
        f32x4 nxt[HT][kNT];
        layer_fwd<F16, HT, HT>(s, smem, k, act, nxt, lane);
#pragma unroll
        for (int mt = 0; mt < HT; ++mt)
#pragma unroll
          for (int nt = 0; nt < kNT; ++nt) act[mt][nt] = nxt[mt][nt];
      }
      const float *bias = reinterpret_cast<const float *>(smem + s.bias_off(k));
#pragma unroll
      for (int mt = 0; mt < HT; ++mt)
#pragma unroll
        for (int nt = 0; nt < kNT; ++nt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float v = act[mt][nt][r] + bias[16 * mt + 4 * q + r];
            act[mt][nt][r] = v > 0.0f ? v : 0.0f;
          }
      if constexpr (TRAIN) store_tiles<F16, HT>(Hs + k * hs_layer_bytes, act, p, q);
    };
    if constexpr (NHLT > 0) {
#pragma unroll
      for (int k = 0; k < NHLT; ++k) hidden_fwd(k);
    } else {
      for (int k = 0; k < NHL; ++k) hidden_fwd(k);
    }
    f32x4 y[1][kNT];
    layer_fwd<F16, HT, 1>(s, smem, NHL, act, y, lane);
    {
      const float *bias = reinterpret_cast<const float *>(smem + s.bias_off(NHL));
#pragma unroll
      for (int nt = 0; nt < kNT; ++nt)
#pragma unroll
        for (int r = 0; r < 4; ++r) y[0][nt][r] = y[0][nt][r] + bias[4 * q + r];
    }
    // the next tile's gathers fly while this tile finishes
    if constexpr (!XMEM) {
      if constexpr (kPipe)
        if (next < a.n_tiles) gather_issue<DF / 8, DF % 8, KT0>(a, res, q, Pn, G);
#pragma unroll
      for (int nt = 0; nt < kNT; ++nt)
#pragma unroll
        for (int d = 0; d < 4; ++d) P[nt][d] = Pn[nt][d];
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
      // ---- loss / output gradient
      const bool wgrads = a.mode != kModeInputGrad;  // accumulate dW / loss
      f32x4 g[OKT][kNT];
      output_grad<OKT>(a, y, Tv, valid, pt, q, lane_loss, lane_amax, g);

      // ---- output layer backward
      wave_lds_sync();
      {
        f32x4 g0[1][kNT];
#pragma unroll
        for (int nt = 0; nt < kNT; ++nt) g0[0][nt] = g[0][nt];
        store_tiles<F16, 1>(Ds, g0, p, q);
      }
      wave_lds_sync();
      const int last = NHL - 1;
      {
        const unsigned char *Hl = Hs + last * hs_layer_bytes;
        if (!wgrads) {
        } else if constexpr (REGDW) {
#pragma unroll
          for (int ut = 0; ut < HT; ++ut) R.wo[ut] = dw_tile<F16>(Ds, 0, Hl, 16 * ut, p, q, R.wo[ut]);
#pragma unroll
          for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int nt = 0; nt < kNT; ++nt) R.bo[r] += g[0][nt][r];
        } else {
          const int wo = s.w_off(NHL), bo = s.b_off(NHL);
#pragma unroll
          for (int ut = 0; ut < HT; ++ut) {
            const f32x4 acc = dw_tile<F16>(Ds, 0, Hl, 16 * ut, p, q);
            const int u = 16 * ut + p;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int o = 4 * q + r;
              if (o < a.M && u < a.H) atomicAdd(dw + wo + u * a.M + o, acc[r] * a.inv_loss_scale);
            }
          }
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float sv = 0.0f;
#pragma unroll
            for (int nt = 0; nt < kNT; ++nt) sv += g[0][nt][r];
            sv = sum_over_p(sv);
            const int o = 4 * q + r;
            if (p == 0 && o < a.M) atomicAdd(dw + bo + o, sv * a.inv_loss_scale);
          }
        }
      }
      f32x4 dl[HT][kNT];
      layer_mma<F16, OKT, HT>(smem + s.bwd_off(NHL), g, dl, lane);
      relu_mask<F16, HT>(dl, Hs + last * hs_layer_bytes, p, q);

      // ---- hidden layers nhl-1 .. 1
      auto hidden_bwd = [&](auto kc) {
        constexpr int KC = decltype(kc)::value;  // compile-time layer (REGDW) or 0
        const int k = KC > 0 ? KC : kc.runtime;
        // layer k's activations are dead (dl is masked): dl takes their slot
        unsigned char *Dk = Hs + k * hs_layer_bytes;
        wave_lds_sync();
        store_tiles<F16, HT>(Dk, dl, p, q);
        wave_lds_sync();
        const unsigned char *Hin = Hs + (k - 1) * hs_layer_bytes;
        if (!wgrads) {
        } else if constexpr (REGDW) {
#pragma unroll
          for (int mt = 0; mt < HT; ++mt) {
#pragma unroll
            for (int it = 0; it < HT; ++it)
              R.wh[KC - 1][mt][it] =
                  dw_tile<F16>(Dk, 16 * mt, Hin, 16 * it, p, q, R.wh[KC - 1][mt][it]);
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
              for (int nt = 0; nt < kNT; ++nt) R.b[KC][mt][r] += dl[mt][nt][r];
          }
        } else {
          const int wk = s.w_off(k), bk = s.b_off(k);
#pragma unroll
          for (int mt = 0; mt < HT; ++mt) {
#pragma unroll
            for (int it = 0; it < HT; ++it) {
              const f32x4 acc = dw_tile<F16>(Dk, 16 * mt, Hin, 16 * it, p, q);
              const int i = 16 * it + p;
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const int u = 16 * mt + 4 * q + r;
                if (u < a.H && i < a.H) atomicAdd(dw + wk + i * a.H + u, acc[r] * a.inv_loss_scale);
              }
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              float sv = 0.0f;
#pragma unroll
              for (int nt = 0; nt < kNT; ++nt) sv += dl[mt][nt][r];
              sv = sum_over_p(sv);
              const int u = 16 * mt + 4 * q + r;
              if (p == 0 && u < a.H) atomicAdd(dw + bk + u, sv * a.inv_loss_scale);
            }
          }
        }
        f32x4 nd[HT][kNT];
        layer_mma<F16, HT, HT>(smem + s.bwd_off(k), dl, nd, lane);
        relu_mask<F16, HT>(nd, Hin, p, q);
#pragma unroll
        for (int mt = 0; mt < HT; ++mt)
#pragma unroll
          for (int nt = 0; nt < kNT; ++nt) dl[mt][nt] = nd[mt][nt];
      };
      if constexpr (NHLT > 0) {
        static_for_desc<NHLT - 1>([&](auto kc) { hidden_bwd(kc); });
      } else {
        for (int k = NHL - 1; k >= 1; --k) hidden_bwd(RuntimeLayer{k});
      }

      // ---- layer 0: dW0, db0, input-feature gradient, hash scatter
      unsigned char *D0 = Hs;  // over layer 0's activations, as above
      wave_lds_sync();
      store_tiles<F16, HT>(D0, dl, p, q);
      wave_lds_sync();
      if (!wgrads) {
      } else if constexpr (REGDW) {
#pragma unroll
        for (int mt = 0; mt < HT; ++mt) {
#pragma unroll
          for (int ft = 0; ft < KT0; ++ft)
            R.w0[mt][ft] = dw_tile<F16>(D0, 16 * mt, Xs, 16 * ft, p, q, R.w0[mt][ft]);
#pragma unroll
          for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int nt = 0; nt < kNT; ++nt) R.b[0][mt][r] += dl[mt][nt][r];
        }
      } else {
        const int w0 = s.w_off(0), b0 = s.b_off(0);
#pragma unroll
        for (int mt = 0; mt < HT; ++mt) {
#pragma unroll
          for (int ft = 0; ft < KT0; ++ft) {
            const f32x4 acc = dw_tile<F16>(D0, 16 * mt, Xs, 16 * ft, p, q);
            const int f = 16 * ft + p;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int u = 16 * mt + 4 * q + r;
              if (u < a.H && f < a.IN) atomicAdd(dw + w0 + f * a.H + u, acc[r] * a.inv_loss_scale);
            }
          }
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float sv = 0.0f;
#pragma unroll
            for (int nt = 0; nt < kNT; ++nt) sv += dl[mt][nt][r];
            sv = sum_over_p(sv);
            const int u = 16 * mt + 4 * q + r;
            if (p == 0 && u < a.H) atomicAdd(dw + b0 + u, sv * a.inv_loss_scale);
          }
        }
      }
      f32x4 dx[KT0][kNT];
      layer_mma<F16, HT, KT0>(smem + s.bwd_off(0), dl, dx, lane);
      if constexpr (SD > 0) {
        if (a.mode != kModeInputGrad) {  // uniform
          tile_scatter<SD, SF, KT0>(a, dx, Ps, valid, res, q);
          continue;
        }
      }
      // dx (D layout: feature 16*kt + 4*q + r of point 16*nt + p) -> [n][IN]
#pragma unroll
      for (int nt = 0; nt < kNT; ++nt) {
        if (!valid[nt]) continue;
        float *row = a.dx_out + static_cast<size_t>(pt[nt]) * a.IN;
#pragma unroll
        for (int kt = 0; kt < KT0; ++kt) {
          const int f0 = 16 * kt + 4 * q;
          f32x4 v = dx[kt][nt];
#pragma unroll
          for (int r = 0; r < 4; ++r) v[r] = v[r] * a.inv_loss_scale;
          if (f0 + 3 < a.IN && (a.IN & 3) == 0) {
            *reinterpret_cast<f32x4 *>(row + f0) = v;
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r)
              if (f0 + r < a.IN) row[f0 + r] = v[r];
          }
        }
      }
    }
  }

  if constexpr (TRAIN) {
    if (a.mode == kModeInputGrad) return;  // uniform: no loss, no weight gradients
    block_loss_partials(a, lane_loss, lane_amax, reinterpret_cast<float *>(smem + s.red_off), lane,
                        wave, a.waves_per_block);
    float *dst = a.grad_partials + static_cast<size_t>(blockIdx.x) * a.mlp_count;
    if constexpr (REGDW) {
      // every wave is past its tiles (barrier above): reduce the waves'
      // register accumulators through LDS in wave order, then store the row
      __syncthreads();
      float *red = reinterpret_cast<float *>(smem);
      for (int w = 0; w < a.waves_per_block; ++w) {
        if (wave == w) dw_regs_to_lds<HT, KT0, NHLT>(R, a, s, red, p, q, w == 0, a.inv_loss_scale);
        __syncthreads();
      }
      for (int e = threadIdx.x; e < a.mlp_count; e += blockDim.x) dst[e] = red[red_slot(e)];
    } else if (!s.dw_global) {
      for (int e = threadIdx.x; e < a.mlp_count; e += blockDim.x) dst[e] = dw[e];
    }
  }
}

// Training launches are LDS-bound to one 4-wave block per CU (one wave per
// SIMD), so they may use the whole register file. Their input features come
// from encode_features_kernel (XMEM).
template <int HP, int INP, bool F16, int NHLT, int SD = 0, int SF = 0>
__global__ void __launch_bounds__(kBlockThreads)
    __attribute__((amdgpu_waves_per_eu(1, 1))) field_train_kernel(FieldArgs a) {
  field_body<HP, INP, F16, true, 0, NHLT, true, SD, SF>(a);
}

// Forward only (inference, the fp16 forward of the split training API),
// encoding inline: unsorted inference batches gain nothing from the separate
// encode pass, and the gathers of the next tile overlap this tile's MLP.
template <int HP, int INP, bool F16, int DF>
__global__ void __launch_bounds__(kBlockThreads) field_forward_kernel(FieldArgs a) {
  field_body<HP, INP, F16, false, DF, 0>(a);
}

// Forward only over X tiles written by the level-major encode
// (encode_level_kernel), for tables whose level slices exceed 2 MB: there the
// inline gathers of field_forward_kernel miss to HBM at one or two waves per
// SIMD and stall its MFMA work, while the level-major encode keeps one
// level's slice in the caches at full occupancy.
template <int HP, int INP, bool F16>
__global__ void __launch_bounds__(kBlockThreads) field_forward_x_kernel(FieldArgs a) {
  field_body<HP, INP, F16, false, 0, 0, true>(a);
}

}  // namespace tmnn_hip
