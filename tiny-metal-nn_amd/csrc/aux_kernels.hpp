// aux_kernels.hpp -- the bandwidth-bound kernels around the fused field
// kernel: seeded Philox init, Morton codes + batch gather, dW partial
// reduction, the fused (lazy-hash + dense-MLP) Adam pass, loss reduction and
// the encode-only inspection kernel.
#pragma once

#include "device_common.hpp"
#include "scatter_kernel.hpp"

namespace tmnn_hip {

// init_uniform_philox (metal_context.cpp:766-792): thread t writes
// out[4t .. 4t+3] = low + u * (high - low), u = float(r) * 2^-32.
__global__ void philox_uniform_kernel(float *out, uint32_t count, uint32_t k0,
                                      uint32_t k1, uint32_t counter_base,
                                      float low, float high) {
  const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
  const uint32_t base = t * 4u;
  if (base >= count) return;
  uint32_t r[4];
  philox4x32_10(counter_base + t, k0, k1, r);
  const float kScale = 1.0f / 4294967296.0f;
  const float span = high - low;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (base + i < count) {
      const float u = static_cast<float>(r[i]) * kScale;
      out[base + i] = low + u * span;
    }
  }
}

// Morton code per point (morton_code in device_common.hpp).
__global__ void morton_codes_kernel(const float *pos, int32_t n, int32_t dims,
                                    uint32_t *codes) {
  const int32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  codes[i] = morton_code(pos + static_cast<size_t>(i) * dims, dims);
}

// dst_pos[i] = src_pos[perm[i]], dst_tgt[i] = src_tgt[perm[i]].
__global__ void gather_rows_kernel(const float *src_pos, const float *src_tgt,
                                   const uint32_t *perm, int32_t n,
                                   int32_t pos_dims, int32_t tgt_dims,
                                   float *dst_pos, float *dst_tgt) {
  // one thread per element, elements of a row on consecutive lanes: the
  // positions [n][pos_dims], then the targets [n][tgt_dims]
  const size_t e = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const size_t np = static_cast<size_t>(n) * pos_dims;
  if (e < np) {
    const size_t i = e / pos_dims, d = e % pos_dims;
    dst_pos[e] = src_pos[static_cast<size_t>(perm[i]) * pos_dims + d];
    return;
  }
  if (!src_tgt) return;
  const size_t t = e - np;
  if (t >= static_cast<size_t>(n) * tgt_dims) return;
  const size_t i = t / tgt_dims, d = t % tgt_dims;
  dst_tgt[t] = src_tgt[static_cast<size_t>(perm[i]) * tgt_dims + d];
}

// grad_mlp[i] += sum over the per-block partial rows partials[b][i].
// Block = 64 columns x 16 row groups; row group g sums rows g, g+16, ...
// in ascending order, then the 16 group sums are added in group order:
// a fixed order, so the result is bit-reproducible.
constexpr int kReduceCols = 64;
constexpr int kReduceGroups = 16;
__global__ void __launch_bounds__(kReduceCols * kReduceGroups)
    reduce_partials_kernel(const float *partials, int32_t blocks, int32_t count,
                           float *grad_mlp, const float *loss_partials, int32_t n,
                           float *loss_out) {
  __shared__ float red[kReduceGroups][kReduceCols + 1];
  // the extra last block (launched when loss_out is set): the step's loss,
  // sum of the per-block loss partials (fixed lane order) / N
  if (loss_out && blockIdx.x == gridDim.x - 1) {
    if (threadIdx.x < 64) {
      const int lane = threadIdx.x;
      float t = 0.0f;
      for (int32_t b = lane; b < blocks; b += 64) t += loss_partials[b];
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) t += __shfl_xor(t, off);
      if (lane == 0) *loss_out = n > 0 ? t / static_cast<float>(n) : 0.0f;
    }
    return;
  }
  const int c = threadIdx.x % kReduceCols;
  const int g = threadIdx.x / kReduceCols;
  const int col = blockIdx.x * kReduceCols + c;
  float s = 0.0f;
  if (col < count) {
#pragma unroll 4
    for (int32_t b = g; b < blocks; b += kReduceGroups)
      s += partials[static_cast<size_t>(b) * count + col];
  }
  red[g][c] = s;
  __syncthreads();
  if (g == 0 && col < count) {
    float t = 0.0f;
#pragma unroll
    for (int k = 0; k < kReduceGroups; ++k) t += red[k][c];
    grad_mlp[col] = grad_mlp[col] + t;
  }
}

struct AdamArgs {
  float *params;            // [hash | mlp] fp32
  float *m;
  float *v;
  int32_t *grad_hash;       // [hash] int32 fixed point
  float *grad_mlp;          // [mlp]
  const uint8_t *mask;      // per-entry visit flags of this step
  uint8_t *mask_next;       // the other flag buffer: zeroed here for the next step
  uint32_t partner_xor;     // 2D: z = 1 entry = z = 0 entry ^ partner_xor (0: none)
  uint32_t log2T;
  int32_t lazy;             // 1: update visited entries only; 0: every entry
  uint32_t hash_entries;    // L * T (hash floats = hash_entries * F)
  uint32_t mlp_count;
  float lr_hash, lr_mlp, beta1, beta2, eps, bc1, bc2;
  float l1_hash, l2_mlp, grad_clip, weight_decay;
  int32_t clear_grads;      // zero consumed gradients (fused step)
  int32_t clear_mask;       // zero mask_next (the caller then swaps the buffers)
};

// Numerics probe of a training step, per thread (NumericsReport,
// detail/runtime_stats.h:32-40; the terms of probe_backward_numerics and
// accumulate_update_probe_for_range, training_step_execution.cpp:238-344,
// taken from the values the Adam pass already holds instead of a host
// read-back of every buffer).
struct NumAcc {
  float gmax = 0.0f;  // largest |g| over finite raw gradients
  float g2 = 0.0f;    // sum of g^2 over them
  float umax = 0.0f;  // largest |w_before - w_after| over finite updates
  uint32_t bad = 0u;  // bit 0: a non-finite gradient; bit 1: a non-finite update
  __device__ __forceinline__ void grad(float g) {
    if (__builtin_isfinite(g)) {
      gmax = fmaxf(gmax, fabsf(g));
      g2 += g * g;
    } else {
      bad |= 1u;
    }
  }
  __device__ __forceinline__ void update(float w0, float w, float mo, float ve) {
    const float du = w0 - w;
    if (__builtin_isfinite(w) && __builtin_isfinite(mo) && __builtin_isfinite(ve) &&
        __builtin_isfinite(du))
      umax = fmaxf(umax, fabsf(du));
    else
      bad |= 2u;
  }
};

// One Adam element (adam_kernel_msl.h:67-108, :137-163, :183-202).
__device__ __forceinline__ void adam_update(float &w, float &mo, float &ve,
                                            float g, float lr, const AdamArgs &a,
                                            bool is_mlp) {
  if (a.grad_clip > 0.0f) g = fminf(fmaxf(g, -a.grad_clip), a.grad_clip);
  if (a.weight_decay > 0.0f) {
    w = w - (lr * a.weight_decay) * w;
  } else {
    if (!is_mlp && a.l1_hash > 0.0f)
      g = g + a.l1_hash * (w > 0.0f ? 1.0f : (w < 0.0f ? -1.0f : 0.0f));
    if (is_mlp && a.l2_mlp > 0.0f) g = g + a.l2_mlp * w;
  }
  const float mn = a.beta1 * mo + (1.0f - a.beta1) * g;
  const float vn = a.beta2 * ve + ((1.0f - a.beta2) * g) * g;
  mo = mn;
  ve = vn;
  const float mh = mn / a.bc1;
  const float vh = vn / a.bc2;
  w = w - (lr * mh) / (sqrtf(vh) + a.eps);
}

// F contiguous 4-byte values at an F-aligned address, as one access.
template <int F, class T>
__device__ __forceinline__ void load_vec(const T *p, T (&out)[F]) {
  typedef T vec __attribute__((ext_vector_type(F)));
  if constexpr (F == 1) {
    out[0] = p[0];
  } else {
    const vec v = *reinterpret_cast<const vec *>(p);
#pragma unroll
    for (int f = 0; f < F; ++f) out[f] = v[f];
  }
}
template <int F, class T>
__device__ __forceinline__ void store_vec(T *p, const T (&in)[F]) {
  typedef T vec __attribute__((ext_vector_type(F)));
  if constexpr (F == 1) {
    p[0] = in[0];
  } else {
    vec v;
#pragma unroll
    for (int f = 0; f < F; ++f) v[f] = in[f];
    *reinterpret_cast<vec *>(p) = v;
  }
}

// One pass over [hash entries | mlp params]. Thread j < hash_entries owns
// table entry j (its F floats); in lazy mode the entry is updated only if it
// was visited (its flag, or for lifted 2D points its z = 0 partner's flag) -- the lazy sparse semantics of
// neural_sdf_adam_hash_sparse (adam_kernel_msl.h:120-164) without the host
// compaction (default_trainer.cpp:1882-1960). Threads past the table own one
// MLP parameter each (neural_sdf_adam_mlp_dense, adam_kernel_msl.h:166-203).
// Adam of hash entry j (its F floats): skipped in lazy mode unless visited;
// zeroes the entry's flag in the next step's buffer.
template <int F, bool NUM = false>
__device__ __forceinline__ void adam_hash_entry(const AdamArgs &a, uint32_t j,
                                                NumAcc *acc = nullptr) {
  bool visited = a.mask[j] != 0;
  if (a.partner_xor) {  // lifted 2D: also visited as some corner's z = 1 partner
    const uint32_t tmask = (1u << a.log2T) - 1u;
    visited = visited || a.mask[(j & ~tmask) | ((j & tmask) ^ a.partner_xor)] != 0;
  }
  if (a.clear_mask) a.mask_next[j] = 0;
  if (a.lazy && !visited) return;
  // the entry's F floats / ints are contiguous and F-aligned: one vector
  // load and store per array
  int32_t gi[F];
  float w[F], mo[F], ve[F];
  load_vec<F>(a.grad_hash + static_cast<size_t>(j) * F, gi);
  load_vec<F>(a.params + static_cast<size_t>(j) * F, w);
  load_vec<F>(a.m + static_cast<size_t>(j) * F, mo);
  load_vec<F>(a.v + static_cast<size_t>(j) * F, ve);
  // an accumulator that is already zero needs no clearing store (once
  // training converges most contributions truncate to 0: the stores were a
  // seventh of the pass's traffic)
  bool any = false;
#pragma unroll
  for (int f = 0; f < F; ++f) any = any || gi[f] != 0;
  // F == 2 entries accumulate as one packed 64-bit sum (scatter_kernel.hpp)
  if constexpr (F == 2) gi[1] = unpack_hi(gi[0], gi[1]);
#pragma unroll
  for (int f = 0; f < F; ++f) {
    const float g = static_cast<float>(gi[f]) * (1.0f / 65536.0f);
    const float w0 = w[f];
    adam_update(w[f], mo[f], ve[f], g, a.lr_hash, a, false);
    if constexpr (NUM) {
      acc->grad(g);
      acc->update(w0, w[f], mo[f], ve[f]);
    }
  }
  store_vec<F>(a.params + static_cast<size_t>(j) * F, w);
  store_vec<F>(a.m + static_cast<size_t>(j) * F, mo);
  store_vec<F>(a.v + static_cast<size_t>(j) * F, ve);
  if (a.clear_grads && any) {
    int32_t z[F];
#pragma unroll
    for (int f = 0; f < F; ++f) z[f] = 0;
    store_vec<F>(a.grad_hash + static_cast<size_t>(j) * F, z);
  }
}

// Adam of MLP parameter k with gradient g; returns the new weight.
template <int F, bool NUM = false>
__device__ __forceinline__ float adam_mlp_param(const AdamArgs &a, uint32_t k, float g,
                                                NumAcc *acc = nullptr) {
  const size_t i = static_cast<size_t>(a.hash_entries) * F + k;
  float w = a.params[i], mo = a.m[i], ve = a.v[i];
  const float w0 = w;
  adam_update(w, mo, ve, g, a.lr_mlp, a, true);
  if constexpr (NUM) {
    acc->grad(g);
    acc->update(w0, w, mo, ve);
  }
  a.params[i] = w;
  a.m[i] = mo;
  a.v[i] = ve;
  if (a.clear_grads) a.grad_mlp[k] = 0.0f;
  return w;
}

template <int F>
__global__ void adam_kernel(AdamArgs a) {
  const uint32_t total = a.hash_entries + a.mlp_count;
  const uint32_t stride = gridDim.x * blockDim.x;
  for (uint32_t j = blockIdx.x * blockDim.x + threadIdx.x; j < total; j += stride) {
    if (j < a.hash_entries)
      adam_hash_entry<F>(a, j);
    else
      adam_mlp_param<F>(a, j - a.hash_entries, a.grad_mlp[j - a.hash_entries]);
  }
}

// dst[0 .. n) = 0 in 16-byte stores (a kernel rather than hipMemsetAsync, so
// a caller may capture the step in a HIP graph).
__global__ void zero_bytes_kernel(uint8_t *dst, size_t n) {
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  const size_t n16 = n / 16;
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n16; i += stride)
    reinterpret_cast<uint4 *>(dst)[i] = make_uint4(0u, 0u, 0u, 0u);
  for (size_t i = n16 * 16 + static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += stride)
    dst[i] = 0;
}

// Encode-only inspection kernel: thread per (point, level).
template <int D>
__device__ void encode_debug_point(const float *table, uint32_t log2T, int F,
                                   int L, const float *res, const float *p,
                                   int l, float *feat_out, uint32_t *idx_out,
                                   float *w_out) {
  const Cell<D> c = cell_of<D>(p, res[l]);
  const uint32_t tmask = (1u << log2T) - 1u;
  float feat[4] = {0.f, 0.f, 0.f, 0.f};
  for (int k = 0; k < (1 << D); ++k) {
    int co[D];
    float wc[D];
    corner_of<D>(c, k, co, wc);
    const uint32_t h = hash_corner<D>(co, tmask);
    const float w = corner_weight<D>(wc);
    const float *e = table + ((static_cast<size_t>(l) << log2T) + h) * F;
    for (int f = 0; f < F; ++f) feat[f] = feat[f] + w * e[f];
    if (idx_out) idx_out[k] = h;
    if (w_out) w_out[k] = w;
  }
  for (int f = 0; f < F; ++f) feat_out[f] = feat[f];
  (void)L;
}

__global__ void encode_debug_kernel(const float *table, uint32_t log2T,
                                    int32_t D, int32_t F, int32_t L,
                                    const float *res_table, const float *pos,
                                    int32_t n, float *feats, uint32_t *idx,
                                    float *wts) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= static_cast<int64_t>(n) * L) return;
  const int32_t i = static_cast<int32_t>(t / L);
  const int l = static_cast<int>(t % L);
  const int C = 1 << D;
  float p[4] = {0.f, 0.f, 0.f, 0.f};
  for (int d = 0; d < D; ++d) p[d] = pos[static_cast<size_t>(i) * D + d];
  float *fo = feats + static_cast<size_t>(i) * L * F + l * F;
  uint32_t *io = idx ? idx + (static_cast<size_t>(i) * L + l) * C : nullptr;
  float *wo = wts ? wts + (static_cast<size_t>(i) * L + l) * C : nullptr;
  if (D == 2)
    encode_debug_point<2>(table, log2T, F, L, res_table, p, l, fo, io, wo);
  else if (D == 3)
    encode_debug_point<3>(table, log2T, F, L, res_table, p, l, fo, io, wo);
  else
    encode_debug_point<4>(table, log2T, F, L, res_table, p, l, fo, io, wo);
}

}  // namespace tmnn_hip
