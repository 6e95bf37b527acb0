// scatter_kernel.hpp -- hash-grid backward: input-feature gradients dx of a
// batch -> int32 fixed-point table gradients + lazy-Adam visit flags.
//
// One thread per point walking the levels; few registers and no LDS: many
// waves per SIMD hide the atomic latency.
//
// Reference semantics (emitHashScatter, mlp_kernel_emitter.cpp:672-901;
// mask :48-71): per corner and feature, int32(trunc(d * w * 65536)) with
// w = ((wx * wy) * wz) on the float2 path (F == 2, 2D/3D), else
// ((d * wx) * wy) * wz (* wt); every visited corner (zero weight included)
// is marked; for the reference's lifted 2D points the z = 1 corners count as
// visited too, which Adam reads off the z = 0 partner's flag (the z = 1 entry
// of a corner is its z = 0 entry XOR (805459861 mod T) within the level).
//
// A wave whose contributions at a level all truncate to 0 (every lane's
// |d| < 2^-16; with d_out ~ 1/N this is 90-99% of a converging batch's
// levels) only stores that level's visit flags (mark_level).
//
// Lanes of a wave hold consecutive Morton-sorted points of one level. When
// more than kMergeMinLanes lanes of a corner have a nonzero contribution, runs
// of lanes that hit the same entry are summed across lanes first (int32 sums
// per feature) and issue one atomic (and one flag store) per run; otherwise
// every lane issues its own (zero contributions issue no atomic), which is
// cheaper than the merge. Measured: merging always costs 15% on a converging
// batch (most contributions truncate to 0), never merging 2.5x on a batch with
// large gradients; the rule stays within 5% of the better of the two on both.
//
// F == 2 packs both features of an entry into one 64-bit atomic:
//   S += (int64)c1 * 2^32 + (int64)c0   (c0 sign-extended)
// The low word is then exactly the int32 (wrapping) sum of c0, the high word
// the sum of c1 minus one when that low sum is negative. Readers restore
// feature 1 as hi + (lo < 0), exact whenever the true sum of c0 stays in
// int32 range (|gradient| < 32768), as the reference's own sum must (and so
// does each wave-merged run's partial sum, a subset of it).
#pragma once

#include "device_common.hpp"

namespace tmnn_hip {

struct ScatterArgs {
  int32_t n;                 // points
  int32_t IN;                // L * F (row stride of dx)
  uint32_t log2T;
  float res[kMaxLevels];     // per-level resolution table
  const float *pos;          // [n][D], the order dx was produced in
  const float *dx;           // [n][IN]
  int32_t *grad_hash;        // [L][T][F]
  uint8_t *mask;             // [L][T] visit flags
};

constexpr int kScatterThreads = 256;
constexpr int kMergeMinLanes = 8;

// Visit flag of one table entry: a plain byte store. Every writer stores the
// same value, so concurrent marks need no atomics (the reference's bit-mask
// atomic_fetch_or marks the same set: all F floats of a visited corner).
__device__ __forceinline__ void mark_entry(uint8_t *mask, size_t entry) { mask[entry] = 1; }

// Visit flags are stored through a raw buffer resource over the flag array
// (num_records = L * T bytes): the entry index is the store's 32-bit offset
// (no 64-bit address arithmetic), and a lane with nothing to mark passes
// kNoEntry, an offset past num_records, whose store the buffer range check
// drops (no branch around the store). Flag arrays hold at most 32 levels of
// 2^24 entries (the planner's limits), below 2^31.
constexpr uint32_t kNoEntry = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t flag_rsrc(uint8_t *mask, int L, uint32_t log2T) {
  // dword 3: 32-bit data format, the raw-buffer setting of gfx9 parts
  return __builtin_amdgcn_make_buffer_rsrc(mask, 0, static_cast<int>(static_cast<uint32_t>(L) << log2T),
                                           0x00020000);
}

__device__ __forceinline__ void mark_flag(__amdgpu_buffer_rsrc_t r, uint32_t entry) {
  __builtin_amdgcn_raw_buffer_store_b8(static_cast<unsigned char>(1), r, static_cast<int>(entry), 0, 0);
}

// feature 1 of a packed F == 2 gradient entry (see the file comment)
__host__ __device__ __forceinline__ int32_t unpack_hi(int32_t lo, int32_t hi) {
  return static_cast<int32_t>(static_cast<uint32_t>(hi) + (lo < 0 ? 1u : 0u));
}

// Inclusive prefix sum of v over the 64 lanes of the wave (wrapping int32),
// on DPP lane shifts only: row_shr 1, 2, 4, 8 inside each 16-lane row, then
// row 0's total into row 1 and row 2's into row 3 (row_bcast:15), then lanes
// 0..31's total into rows 2 and 3 (row_bcast:31).
__device__ __forceinline__ int32_t wave_incl_sum(int32_t v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, true);   // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, true);   // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, true);   // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, true);   // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31
  return v;
}

// Sums of c[0..N) over the run of equal keys that ends at this lane (runs are
// maximal sequences of equal keys in lane order); *is_tail is set on the last
// lane of each run, which then owns the run's totals. A run total is the
// wave prefix sum at its tail minus the prefix sum just before its head;
// int32 sums wrap, so the totals are exact modulo 2^32 in any order, like the
// int32 atomics they feed.
template <int N>
__device__ __forceinline__ void run_sums(uint32_t key, int32_t (&c)[N], int lane, bool *is_tail) {
  // previous lane's key: DPP wave_shr:1 (lane 0 keeps the old value)
  const uint32_t prev = static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(-1, static_cast<int>(key), 0x138, 0xf, 0xf, false));
  const bool head = lane == 0 || prev != key;
  const uint64_t heads = __ballot(head);
  if (heads == ~0ull) {  // no two neighbours share an entry
    *is_tail = true;
    return;
  }
  const uint64_t le = lane == 63 ? ~0ull : ((2ull << lane) - 1ull);
  const int start = 63 - __clzll(heads & le);  // first lane of this lane's run
  const int src = start > 0 ? start - 1 : 0;
#pragma unroll
  for (int f = 0; f < N; ++f) {
    const int32_t incl = wave_incl_sum(c[f]);
    const int32_t before = __shfl(incl, src);
    c[f] = static_cast<int32_t>(static_cast<uint32_t>(incl) -
                                (start > 0 ? static_cast<uint32_t>(before) : 0u));
  }
  *is_tail = lane == 63 || ((heads >> (lane + 1)) & 1ull);
}

// |d| < 32768 for every feature: then every product d * w (w in [0, 1]) times
// 65536 lies inside int32, and the conversion needs no saturation or NaN
// handling (f2i_trunc's branches)
template <int F>
__device__ __forceinline__ bool grads_fit(const float *d) {
  bool ok = true;
#pragma unroll
  for (int f = 0; f < F; ++f) ok = ok && __builtin_fabsf(d[f]) < 32768.0f;
  return ok;
}

// |d| < 2^-16 for every feature: every corner's contribution truncates to 0.
// The corner weight w is a product of per-axis factors in [0, 1], so each
// rounded product fl(d * w...) is no larger in magnitude than d, and
// fl(d * w) * 65536 (exact: a power of two) stays below 1. NaN is not small.
template <int F>
__device__ __forceinline__ bool grads_vanish(const float *d) {
  bool ok = true;
#pragma unroll
  for (int f = 0; f < F; ++f) ok = ok && __builtin_fabsf(d[f]) < 1.0f / kGradScale;
  return ok;
}

// A level whose contributions all truncate to 0 in every lane of the wave
// (the common case once training converges: |d| ~ 1/N): only the visit flags
// of its corners are stored, the same entries the full path marks. Corners x
// and x + 1 differ only in the low bits the carry of x + 1 flips (x has
// multiplier 1 in the hash), so their flag bytes share a line unless x ends
// in seven 1 bits: a v_permlane32_swap gives each store instruction both
// x-corners of 32 points (lanes 0-31 corner x, lanes 32-63 corner x + 1 of
// the same points, then the other way round), half the line requests of one
// instruction per corner.
template <int D, int F>
__device__ __forceinline__ void mark_level(const ScatterArgs &a, int l, const float *p,
                                           bool valid) {
  const Cell<D> c = cell_of<D>(p, a.res[l]);
  const uint32_t tmask = (1u << a.log2T) - 1u;
  const uint32_t lbase = static_cast<uint32_t>(l) << a.log2T;
  const __amdgpu_buffer_rsrc_t flags = flag_rsrc(a.mask, a.IN / F, a.log2T);
#pragma unroll
  for (int m = 0; m < (1 << (D - 1)); ++m) {
    int co[D];
    float wc[D];
    corner_of<D>(c, 2 * m, co, wc);
    const uint32_t e0 = valid ? lbase + hash_corner<D>(co, tmask) : kNoEntry;
    co[0] += 1;
    const uint32_t e1 = valid ? lbase + hash_corner<D>(co, tmask) : kNoEntry;
    const auto r = __builtin_amdgcn_permlane32_swap(e0, e1, false, false);
    mark_flag(flags, r[0]);
    mark_flag(flags, r[1]);
  }
}

// One thread per point (or per point and share of its levels, blockIdx.y),
// its levels in turn: the thread reads its dx row with
// 16-byte loads (coalesced across the wave) and the lanes of a wave still
// hold consecutive Morton-sorted points at the same level, which keeps the
// run merging. FITS: every lane's d passed grads_fit (plain conversion).
template <int D, int F, bool FITS>
__device__ __forceinline__ void scatter_level(const ScatterArgs &a, int l, const float *p,
                                              const float *d, bool valid, int lane) {
  const Cell<D> c = cell_of<D>(p, a.res[l]);
  const uint32_t tmask = (1u << a.log2T) - 1u;
  const size_t lbase = static_cast<size_t>(l) << a.log2T;
  constexpr bool kVec2 = (F == 2 && D <= 3);
#pragma unroll
  for (int k = 0; k < (1 << D); ++k) {
    int co[D];
    float wc[D];
    corner_of<D>(c, k, co, wc);
    const uint32_t local = valid ? hash_corner<D>(co, tmask) : 0xFFFFFFFFu;
    const size_t entry = lbase + local;
    int32_t ci[F];
#pragma unroll
    for (int f = 0; f < F; ++f) {
      float v;
      if constexpr (kVec2) {
        v = d[f] * corner_weight<D>(wc);
      } else {
        v = d[f] * wc[0];
        v = v * wc[1];
        if constexpr (D >= 3) v = v * wc[2];
        if constexpr (D == 4) v = v * wc[3];
      }
      if constexpr (FITS)
        ci[f] = valid ? static_cast<int32_t>(v * kGradScale) : 0;
      else
        ci[f] = valid ? f2i_trunc(v * kGradScale) : 0;
    }
    bool tail = true;
    bool nz = false;
#pragma unroll
    for (int f = 0; f < F; ++f) nz = nz || ci[f] != 0;
    if (__popcll(__ballot(nz)) > kMergeMinLanes) run_sums<F>(local, ci, lane, &tail);
    if (valid && tail) {
      if constexpr (F == 2) {
        // packed pair (see the file comment)
        const int64_t v64 = static_cast<int64_t>(
            (static_cast<uint64_t>(static_cast<uint32_t>(ci[1])) << 32) +
            static_cast<uint64_t>(static_cast<int64_t>(ci[0])));
        if (v64 != 0)
          atomicAdd(reinterpret_cast<unsigned long long *>(a.grad_hash + entry * 2),
                    static_cast<unsigned long long>(v64));
      } else {
#pragma unroll
        for (int f = 0; f < F; ++f)
          if (ci[f] != 0) atomicAdd(a.grad_hash + entry * F + f, ci[f]);
      }
      mark_entry(a.mask, entry);
    }
  }
}

// One level of one point: flags only when the whole wave's contributions
// vanish, else the full scatter (plain or saturating conversion).
template <int D, int F>
__device__ __forceinline__ void scatter_point_level(const ScatterArgs &a, int l, const float *p,
                                                    const float *d, bool valid, int lane) {
  if (__all(!valid || grads_vanish<F>(d)))
    mark_level<D, F>(a, l, p, valid);
  else if (__all(grads_fit<F>(d)))
    scatter_level<D, F, true>(a, l, p, d, valid, lane);
  else
    scatter_level<D, F, false>(a, l, p, d, valid, lane);
}

template <int D, int F>
__global__ void __launch_bounds__(kScatterThreads) hash_scatter_kernel(ScatterArgs a) {
  const int i = blockIdx.x * kScatterThreads + threadIdx.x;
  const int lane = threadIdx.x & 63;
  // lanes past the batch take part in the wave's run merging with a key no
  // point can have and nothing to add
  const bool valid = i < a.n;
  const int ii = valid ? i : a.n - 1;
  float p[D];
#pragma unroll
  for (int k = 0; k < D; ++k) p[k] = a.pos[static_cast<size_t>(ii) * D + k];
  const float *row = a.dx + static_cast<size_t>(ii) * a.IN;
  // the levels of one 16-byte dx load (4 features: 4 / F levels) at a time
  // blockIdx.y picks this thread's share of the quads (the launch may split
  // a point's levels over several threads)
  const int nq = (a.IN + 3) / 4;
  const int per = (nq + static_cast<int>(gridDim.y) - 1) / static_cast<int>(gridDim.y);
  const int q1 = min(nq, static_cast<int>(blockIdx.y) * per + per);
  for (int fq = static_cast<int>(blockIdx.y) * per; fq < q1; ++fq) {
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    if (fq * 4 + 3 < a.IN && (a.IN & 3) == 0) {
      v = *reinterpret_cast<const f32x4 *>(row + fq * 4);
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (fq * 4 + r < a.IN) v[r] = row[fq * 4 + r];
    }
#pragma unroll
    for (int lv = 0; lv < 4 / F; ++lv) {
      const int l = fq * (4 / F) + lv;
      if (l * F >= a.IN) break;  // IN = L * F
      float d[F];
#pragma unroll
      for (int f = 0; f < F; ++f) d[f] = v[lv * F + f];
      scatter_point_level<D, F>(a, l, p, d, valid, lane);
    }
  }
}

// Level-major variant for large tables: one thread per (point, level),
// blockIdx.y = level, so the resident blocks work in one level's slice of the
// table at a time (a 2^22-entry level is 32 MB; all levels together do not
// stay in the caches).
template <int D, int F>
__global__ void __launch_bounds__(kScatterThreads) hash_scatter_level_kernel(ScatterArgs a) {
  const int l = blockIdx.y;
  const int i = blockIdx.x * kScatterThreads + threadIdx.x;
  const int lane = threadIdx.x & 63;
  const bool valid = i < a.n;
  const int ii = valid ? i : a.n - 1;
  float p[D];
#pragma unroll
  for (int k = 0; k < D; ++k) p[k] = a.pos[static_cast<size_t>(ii) * D + k];
  float d[F];
  const float *src = a.dx + static_cast<size_t>(ii) * a.IN + l * F;
  if constexpr (F == 2) {
    const f32x2 v = *reinterpret_cast<const f32x2 *>(src);
    d[0] = v[0];
    d[1] = v[1];
  } else if constexpr (F == 4) {
    const f32x4 v = *reinterpret_cast<const f32x4 *>(src);
#pragma unroll
    for (int f = 0; f < 4; ++f) d[f] = v[f];
  } else {
    d[0] = src[0];
  }
  scatter_point_level<D, F>(a, l, p, d, valid, lane);
}

}  // namespace tmnn_hip
