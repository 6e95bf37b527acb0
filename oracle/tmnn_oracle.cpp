// tmnn_oracle.cpp -- CPU restatement of the reference's scalar hot-path math.
//
// TEST INFRASTRUCTURE ONLY (parity checker + CPU baseline); see tmnn_oracle.h.
// Built with -ffp-contract=off so every multiply and add rounds separately,
// in the order the reference's MSL source writes them.
//
// Reference paths are relative to the reference checkout.
#include "tmnn_oracle.h"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#ifdef _OPENMP
#include <omp.h>
#endif

namespace {

// mlp_kernel_emitter.cpp:16-18 (hash primes; the GPU 4D prime is 56711039).
constexpr uint32_t kPrimeY = 2654435761u;
constexpr uint32_t kPrimeZ = 805459861u;
constexpr uint32_t kPrimeW = 56711039u;
// mlp_kernel_emitter.cpp:20 / :2741-2744 (int32 fixed-point hash gradients).
constexpr float kGradScale = 65536.0f;
constexpr float kMaxHidden = 512;

struct Geo {
  int D;      // effective spatial dims (2D is lifted to 3)
  int in_D;   // dims of the caller's position rows
  int L, F, H, NHL, M;
  uint32_t T;
  int C;      // corners per level
  bool vec2;  // the reference's float2 path: F == 2 and 3D
};

Geo geo_of(const orc_model *m) {
  Geo g;
  g.in_D = m->spatial_dims;
  g.D = m->spatial_dims == 2 ? 3 : m->spatial_dims;
  g.L = m->num_levels;
  g.F = m->features_per_level;
  g.H = m->hidden_dim;
  g.NHL = m->num_hidden_layers;
  g.M = m->num_outputs;
  g.T = 1u << m->log2_hashmap_size;
  g.C = 1 << g.D;
  g.vec2 = (g.F == 2 && g.D == 3);
  return g;
}

// Constants are baked into MSL with "%.6f" (mlp_kernel_emitter.cpp:91-92) and
// re-read by the shader compiler as float literals.
float baked6(float v) {
  char buf[64];
  std::snprintf(buf, sizeof buf, "%.6f", static_cast<double>(v));
  return std::strtof(buf, nullptr);
}

// Per-level resolution: iterated fp32 product r_l = r_{l-1} * s
// (mlp_kernel_emitter.cpp:224,298 -- the eval / encode path).
void resolutions(const orc_model *m, float *out) {
  float r = baked6(m->base_resolution);
  const float s = baked6(m->per_level_scale);
  for (int l = 0; l < m->num_levels; ++l) {
    out[l] = r;
    r = r * s;
  }
}

// hash_coords / hash_coords_4d: mlp_kernel_emitter.cpp:144-161.
inline uint32_t hash_idx(const int *c, int D, uint32_t T) {
  uint32_t h = static_cast<uint32_t>(c[0]) * 1u;
  h ^= static_cast<uint32_t>(c[1]) * kPrimeY;
  h ^= static_cast<uint32_t>(c[2]) * kPrimeZ;
  if (D == 4) h ^= static_cast<uint32_t>(c[3]) * kPrimeW;
  return h % T;
}

// MSL int(x) on the gradient path; clamp so the C conversion is defined and
// equals the GPU's saturating v_cvt_i32_f32 (NaN -> 0).
inline int32_t to_i32(float x) {
  if (!(x == x)) return 0;
  if (x >= 2147483648.0f) return 2147483647;
  if (x <= -2147483648.0f) return static_cast<int32_t>(0x80000000u);
  return static_cast<int32_t>(x);
}

// Corner set of one level for one point: bc = int(floor(p*r)),
// frac = p*r - floor(p*r)  (mlp_kernel_emitter.cpp:240-254).
struct Level {
  int bc[4];
  float fr[4];
};

inline Level level_of(const Geo &g, const float *p, float res) {
  Level lv;
  for (int a = 0; a < 4; ++a) { lv.bc[a] = 0; lv.fr[a] = 0.0f; }
  for (int a = 0; a < g.D; ++a) {
    const float coord = (a < g.in_D) ? p[a] : 0.0f;  // lifted z = 0
    const float s = coord * res;
    const float fl = std::floor(s);
    lv.bc[a] = static_cast<int>(fl);
    lv.fr[a] = s - fl;
  }
  return lv;
}

// Corner c in the reference's loop order (dw outer, then dz, dy, dx inner):
// corner weight = ((wx*wy)*wz)(*wt), one rounding per multiply
// (mlp_kernel_emitter.cpp:270-274, :2918-2928).
inline void corner_of(const Geo &g, const Level &lv, int c, int *coords,
                      float *wcomp) {
  const int dx = c & 1, dy = (c >> 1) & 1, dz = (c >> 2) & 1, dw = (c >> 3) & 1;
  const int d[4] = {dx, dy, dz, dw};
  for (int a = 0; a < 4; ++a) {
    coords[a] = lv.bc[a] + (a < g.D ? d[a] : 0);
    wcomp[a] = (a < g.D) ? (d[a] == 0 ? (1.0f - lv.fr[a]) : lv.fr[a]) : 1.0f;
  }
}

inline float corner_weight(const Geo &g, const float *wc) {
  float w = wc[0] * wc[1];
  w = w * wc[2];
  if (g.D == 4) w = w * wc[3];
  return w;
}

// Encode one level: feats[f] = sum over corners (loop order) of w*t.
inline void encode_level(const Geo &g, const float *table, const Level &lv,
                         int l, float *feat, uint32_t *idx_out, float *w_out) {
  for (int f = 0; f < g.F; ++f) feat[f] = 0.0f;
  for (int c = 0; c < g.C; ++c) {
    int co[4];
    float wc[4];
    corner_of(g, lv, c, co, wc);
    const uint32_t h = hash_idx(co, g.D, g.T);
    const float w = corner_weight(g, wc);
    const size_t off = static_cast<size_t>(l) * g.T * g.F + static_cast<size_t>(h) * g.F;
    for (int f = 0; f < g.F; ++f) feat[f] = feat[f] + w * table[off + f];
    if (idx_out) idx_out[c] = h;
    if (w_out) w_out[c] = w;
  }
}

struct Offsets {
  int w[9], b[9];  // layer 0 .. NHL-1 hidden, index NHL = output
  int total;
};

// Weight layout: [W0 (in x H), b0, W1 (H x H), b1, ..., WO (H x M), bO]
// (mlp_kernel_emitter.cpp:163-199; kernel_spec.cpp:65-71).
Offsets offsets_of(const Geo &g) {
  Offsets o;
  int off = 0;
  const int in = g.L * g.F;
  o.w[0] = off; off += in * g.H;
  o.b[0] = off; off += g.H;
  for (int k = 1; k < g.NHL; ++k) {
    o.w[k] = off; off += g.H * g.H;
    o.b[k] = off; off += g.H;
  }
  o.w[g.NHL] = off; off += g.H * g.M;
  o.b[g.NHL] = off; off += g.M;
  o.total = off;
  return o;
}

// Forward of one point (scalar train kernel, mlp_kernel_emitter.cpp:2898-3036).
// acts: [NHL][H] post-ReLU activations; out: [M].
void forward_point(const Geo &g, const Offsets &o, const float *res,
                   const float *table, const float *W, const float *p,
                   float *acts, float *out) {
  float *h0 = acts;
  for (int j = 0; j < g.H; ++j) h0[j] = 0.0f;
  for (int l = 0; l < g.L; ++l) {
    const Level lv = level_of(g, p, res[l]);
    float feat[4];
    encode_level(g, table, lv, l, feat, nullptr, nullptr);
    if (g.vec2) {
      // h0[j] += feat.x * W0[fb][j] + feat.y * W0[fb+1][j]  (:2930-2933)
      const float *wa = W + o.w[0] + (l * 2) * g.H;
      const float *wb = W + o.w[0] + (l * 2 + 1) * g.H;
      for (int j = 0; j < g.H; ++j) {
        const float a = feat[0] * wa[j];
        const float b = feat[1] * wb[j];
        h0[j] = h0[j] + (a + b);
      }
    } else {
      for (int f = 0; f < g.F; ++f) {  // (:2979-2984)
        const float *wr = W + o.w[0] + (l * g.F + f) * g.H;
        for (int j = 0; j < g.H; ++j) h0[j] = h0[j] + feat[f] * wr[j];
      }
    }
  }
  for (int j = 0; j < g.H; ++j) {  // (:2987-2988)
    const float v = h0[j] + W[o.b[0] + j];
    h0[j] = v > 0.0f ? v : 0.0f;
  }
  for (int k = 1; k < g.NHL; ++k) {  // (:3001-3008)
    const float *src = acts + (k - 1) * g.H;
    float *dst = acts + k * g.H;
    const float *Wk = W + o.w[k];
    for (int j = 0; j < g.H; ++j) {
      float acc = 0.0f;
      for (int i = 0; i < g.H; ++i) acc = acc + src[i] * Wk[i * g.H + j];
      const float v = acc + W[o.b[k] + j];
      dst[j] = v > 0.0f ? v : 0.0f;
    }
  }
  const float *last = acts + (g.NHL - 1) * g.H;
  for (int mm = 0; mm < g.M; ++mm) {  // (:3025-3035)
    float acc = W[o.b[g.NHL] + mm];
    for (int j = 0; j < g.H; ++j) acc = acc + last[j] * W[o.w[g.NHL] + j * g.M + mm];
    out[mm] = acc;
  }
}

// Loss and output gradient of one point (emitLoss, mlp_kernel_emitter.cpp:562-670).
// RelativeL2 is not in the reference: it follows tcnn's published definition
// r^2 / (y^2 + 0.01) with the denominator held constant in the gradient,
// summed over outputs and divided by N like the reference's L2; one division
// per element (inv = 1 / den, then products), as the GPU kernels compute it.
float loss_point(const orc_model *m, const Geo &g, const float *out,
                 const float *tgt, float inv_n, float *d_out) {
  float loss = 0.0f;
  if (m->loss_kind == ORC_COSINE) {
    float dot = 0.0f, pn = 0.0f, tn = 0.0f;
    for (int k = 0; k < g.M; ++k) {
      dot = dot + out[k] * tgt[k];
      pn = pn + out[k] * out[k];
      tn = tn + tgt[k] * tgt[k];
    }
    const float pnorm = std::sqrt(pn + 1e-8f);
    const float tnorm = std::sqrt(tn + 1e-8f);
    const float denom = pnorm * tnorm;
    const float cosine = dot / denom;
    const float pdenom = pn + 1e-8f;
    for (int k = 0; k < g.M; ++k) {
      const float a = (cosine * out[k]) / pdenom;
      const float b = tgt[k] / denom;
      d_out[k] = (a - b) * inv_n;
    }
    return 1.0f - cosine;
  }
  for (int k = 0; k < g.M; ++k) {
    const float r = out[k] - tgt[k];
    float term, d;
    switch (m->loss_kind) {
      case ORC_L1:
        term = std::fabs(r);
        d = (r > 0.0f ? 1.0f : (r < 0.0f ? -1.0f : 0.0f)) * inv_n;
        break;
      case ORC_HUBER: {
        const float delta = baked6(m->huber_delta);
        const float ar = std::fabs(r);
        if (ar <= delta) {
          term = (0.5f * r) * r;
          d = r * inv_n;
        } else {
          term = delta * (ar - 0.5f * delta);
          d = (delta * (r > 0.0f ? 1.0f : -1.0f)) * inv_n;
        }
        break;
      }
      case ORC_RELATIVE_L2: {
        const float den = out[k] * out[k] + 0.01f;
        const float inv = 1.0f / den;
        term = (r * r) * inv;
        d = ((2.0f * r) * inv) * inv_n;
        break;
      }
      default:  // L2
        term = r * r;
        d = (2.0f * r) * inv_n;
        break;
    }
    loss = loss + term;
    d_out[k] = d;
  }
  return loss;
}

inline void mark_slot(uint32_t *mask, uint32_t slot) {
  std::atomic_ref<uint32_t> w(mask[slot >> 5]);
  w.fetch_or(1u << (slot & 31u), std::memory_order_relaxed);
}

inline void add_i32(int32_t *dst, int32_t v) {
  std::atomic_ref<int32_t> a(*dst);
  a.fetch_add(v, std::memory_order_relaxed);  // two's complement wrap
}

// Backward of one point (mlp_kernel_emitter.cpp:3055-3143 and emitHashScatter
// :672-901). gW accumulates the per-point fp32 terms (thread-local).
void backward_point(const Geo &g, const Offsets &o, const float *res,
                    const float *table, const float *W, const float *p,
                    float *acts, const float *d_out, int32_t *grad_hash,
                    double *gW, uint32_t *mask) {
  // Output layer (:3067-3079): acts of the last layer become delta in place.
  float *last = acts + (g.NHL - 1) * g.H;
  for (int j = 0; j < g.H; ++j) {
    const float hv = last[j];
    float dpre = 0.0f;
    for (int k = 0; k < g.M; ++k) {
      gW[o.w[g.NHL] + j * g.M + k] += static_cast<double>(d_out[k] * hv);
      dpre = dpre + d_out[k] * W[o.w[g.NHL] + j * g.M + k];
    }
    last[j] = dpre * (hv > 0.0f ? 1.0f : 0.0f);
  }
  for (int k = 0; k < g.M; ++k) gW[o.b[g.NHL] + k] += static_cast<double>(d_out[k]);

  // Hidden layers nhl-1 .. 1 (:3096-3113).
  for (int k = g.NHL - 1; k >= 1; --k) {
    float *dl = acts + k * g.H;
    float *hl = acts + (k - 1) * g.H;
    const float *Wk = W + o.w[k];
    for (int i = 0; i < g.H; ++i) {
      const float hv = hl[i];
      for (int j = 0; j < g.H; ++j)
        gW[o.w[k] + i * g.H + j] += static_cast<double>(dl[j] * hv);
      float acc = 0.0f;
      for (int j = 0; j < g.H; ++j) acc = acc + dl[j] * Wk[i * g.H + j];
      hl[i] = acc * (hv > 0.0f ? 1.0f : 0.0f);
    }
    for (int j = 0; j < g.H; ++j) gW[o.b[k] + j] += static_cast<double>(dl[j]);
  }

  // Layer 0 + hash scatter (emitHashScatter).
  const float *d0 = acts;
  for (int l = 0; l < g.L; ++l) {
    const Level lv = level_of(g, p, res[l]);
    uint32_t cidx[16];
    float cw[16];
    float feat[4];
    encode_level(g, table, lv, l, feat, cidx, cw);
    const size_t base = static_cast<size_t>(l) * g.T * g.F;
    if (g.vec2) {
      const int r0 = o.w[0] + (l * 2) * g.H, r1 = o.w[0] + (l * 2 + 1) * g.H;
      float df0 = 0.0f, df1 = 0.0f;
      for (int j = 0; j < g.H; ++j) {  // (:726-735)
        gW[r0 + j] += static_cast<double>(d0[j] * feat[0]);
        gW[r1 + j] += static_cast<double>(d0[j] * feat[1]);
        df0 = df0 + d0[j] * W[r0 + j];
        df1 = df1 + d0[j] * W[r1 + j];
      }
      for (int c = 0; c < g.C; ++c) {  // (:744-768): int((d * w) * 65536)
        const size_t off = base + static_cast<size_t>(cidx[c]) * 2;
        const float w = cw[c];
        add_i32(&grad_hash[off], to_i32((df0 * w) * kGradScale));
        add_i32(&grad_hash[off + 1], to_i32((df1 * w) * kGradScale));
        if (mask) mark_slot(mask, static_cast<uint32_t>(off >> 1));
      }
    } else {
      for (int f = 0; f < g.F; ++f) {
        const int row = o.w[0] + (l * g.F + f) * g.H;
        float df = 0.0f;
        for (int j = 0; j < g.H; ++j) {  // (:823-831)
          gW[row + j] += static_cast<double>(d0[j] * feat[f]);
          df = df + d0[j] * W[row + j];
        }
        for (int c = 0; c < g.C; ++c) {  // (:836-866): int(d*wx*wy*wz(*wt)*S)
          int co[4];
          float wc[4];
          corner_of(g, lv, c, co, wc);
          float v = df * wc[0];
          v = v * wc[1];
          v = v * wc[2];
          if (g.D == 4) v = v * wc[3];
          const size_t off = base + static_cast<size_t>(cidx[c]) * g.F + f;
          add_i32(&grad_hash[off], to_i32(v * kGradScale));
          if (mask) {
            // Entry pairs are tracked when F == 2, single floats otherwise
            // (mlp_kernel_emitter.cpp:870-888).
            const uint32_t slot = (g.F == 2) ? static_cast<uint32_t>(off >> 1)
                                             : static_cast<uint32_t>(off);
            mark_slot(mask, slot);
          }
        }
      }
    }
  }
  for (int j = 0; j < g.H; ++j) gW[o.b[0] + j] += static_cast<double>(d0[j]);
}

// d(feature f of level l)/d(cell fraction) at one point: the 3D lerp form of
// trilinear_feature_grad (mlp_kernel_emitter.cpp:1677-1704; lifted 2D points
// use it with fz = 0) and the 4D loops of the gradient kernel (:2034-2056).
void level_frac_grad(const Geo &g, const float *table, const Level &lv, int l, int f,
                     float *dv) {
  const size_t base = static_cast<size_t>(l) * g.T * g.F;
  auto at = [&](int dx, int dy, int dz, int dw) {
    int c[4] = {lv.bc[0] + dx, lv.bc[1] + dy, lv.bc[2] + dz, lv.bc[3] + dw};
    return table[base + static_cast<size_t>(hash_idx(c, g.D, g.T)) * g.F + f];
  };
  const float fx = lv.fr[0], fy = lv.fr[1], fz = lv.fr[2], fw = lv.fr[3];
  if (g.D == 3) {
    const float c000 = at(0, 0, 0, 0), c001 = at(0, 0, 1, 0), c010 = at(0, 1, 0, 0),
                c011 = at(0, 1, 1, 0), c100 = at(1, 0, 0, 0), c101 = at(1, 0, 1, 0),
                c110 = at(1, 1, 0, 0), c111 = at(1, 1, 1, 0);
    dv[0] = (1.0f - fz) * ((1.0f - fy) * (c100 - c000) + fy * (c110 - c010)) +
            fz * ((1.0f - fy) * (c101 - c001) + fy * (c111 - c011));
    dv[1] = (1.0f - fz) * ((1.0f - fx) * (c010 - c000) + fx * (c110 - c100)) +
            fz * ((1.0f - fx) * (c011 - c001) + fx * (c111 - c101));
    dv[2] = (1.0f - fy) * ((1.0f - fx) * (c001 - c000) + fx * (c101 - c100)) +
            fy * ((1.0f - fx) * (c011 - c010) + fx * (c111 - c110));
    dv[3] = 0.0f;
    return;
  }
  float c[2][2][2][2];
  for (int dw = 0; dw < 2; ++dw)
    for (int dz = 0; dz < 2; ++dz)
      for (int dy = 0; dy < 2; ++dy)
        for (int dx = 0; dx < 2; ++dx) c[dw][dz][dy][dx] = at(dx, dy, dz, dw);
  auto w = [](int d, float fr) { return d == 0 ? (1.0f - fr) : fr; };
  float gx = 0.0f, gy = 0.0f, gz = 0.0f, gt = 0.0f;
  for (int dw = 0; dw < 2; ++dw)
    for (int dz = 0; dz < 2; ++dz)
      for (int dy = 0; dy < 2; ++dy)
        gx += w(dy, fy) * w(dz, fz) * w(dw, fw) * (c[dw][dz][dy][1] - c[dw][dz][dy][0]);
  for (int dw = 0; dw < 2; ++dw)
    for (int dz = 0; dz < 2; ++dz)
      for (int dx = 0; dx < 2; ++dx)
        gy += w(dx, fx) * w(dz, fz) * w(dw, fw) * (c[dw][dz][1][dx] - c[dw][dz][0][dx]);
  for (int dw = 0; dw < 2; ++dw)
    for (int dy = 0; dy < 2; ++dy)
      for (int dx = 0; dx < 2; ++dx)
        gz += w(dx, fx) * w(dy, fy) * w(dw, fw) * (c[dw][1][dy][dx] - c[dw][0][dy][dx]);
  for (int dz = 0; dz < 2; ++dz)
    for (int dy = 0; dy < 2; ++dy)
      for (int dx = 0; dx < 2; ++dx)
        gt += w(dx, fx) * w(dy, fy) * w(dz, fz) * (c[1][dz][dy][dx] - c[0][dz][dy][dx]);
  dv[0] = gx;
  dv[1] = gy;
  dv[2] = gz;
  dv[3] = gt;
}

// Philox-4x32-10 (metal_context.cpp:735-752; Salmon et al., SC'11).
inline void philox(uint32_t ctr_in, uint32_t k0, uint32_t k1, uint32_t out[4]) {
  uint32_t c0 = ctr_in, c1 = 0, c2 = 0, c3 = 0;
  for (int i = 0; i < 10; ++i) {
    const uint64_t p0 = static_cast<uint64_t>(0xD2511F53u) * c0;
    const uint64_t p1 = static_cast<uint64_t>(0xCD9E8D57u) * c2;
    const uint32_t hi0 = static_cast<uint32_t>(p0 >> 32), lo0 = static_cast<uint32_t>(p0);
    const uint32_t hi1 = static_cast<uint32_t>(p1 >> 32), lo1 = static_cast<uint32_t>(p1);
    const uint32_t n0 = hi1 ^ c1 ^ k0, n1 = lo1, n2 = hi0 ^ c3 ^ k1, n3 = lo0;
    c0 = n0; c1 = n1; c2 = n2; c3 = n3;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

// Morton code (morton_sort.h:14-57).
inline uint32_t expand3(uint32_t v) {
  v = (v | (v << 16)) & 0x030000FFu;
  v = (v | (v << 8)) & 0x0300F00Fu;
  v = (v | (v << 4)) & 0x030C30C3u;
  v = (v | (v << 2)) & 0x09249249u;
  return v;
}
inline uint32_t expand4(uint32_t v) {
  v &= 0xFFu;
  v = (v | (v << 16)) & 0x000F000Fu;
  v = (v | (v << 8)) & 0x00C30C03u;
  v = (v | (v << 4)) & 0x09090909u;
  v = (v | (v << 2)) & 0x11111111u;
  return v;
}
inline uint32_t quant(float v, float scale, float top) {
  const float mapped = (v * 0.5f + 0.5f) * scale;
  return static_cast<uint32_t>(std::fmin(std::fmax(mapped, 0.0f), top));
}

int threads_for(int32_t requested) {
#ifdef _OPENMP
  return requested > 1 ? requested : 1;
#else
  (void)requested;
  return 1;
#endif
}

}  // namespace

extern "C" {

uint32_t orc_hash_param_count(const orc_model *m) {
  return static_cast<uint32_t>(m->num_levels) * (1u << m->log2_hashmap_size) *
         static_cast<uint32_t>(m->features_per_level);
}

uint32_t orc_mlp_param_count(const orc_model *m) {
  return static_cast<uint32_t>(offsets_of(geo_of(m)).total);
}

// Tracked slots: entry pairs when F == 2 (default_trainer.cpp:1878-1880).
uint32_t orc_mask_word_count(const orc_model *m) {
  const uint32_t width = m->features_per_level == 2 ? 2u : 1u;
  return (orc_hash_param_count(m) / width + 31u) / 32u;
}

void orc_resolutions(const orc_model *m, float *out) { resolutions(m, out); }

// init_uniform_philox (metal_context.cpp:766-792): u = float(r) * 2^-32,
// v = low + u * (high - low).
void orc_philox_uniform(uint64_t seed, uint32_t counter_base, uint32_t count,
                        float low, float high, float *out) {
  const uint32_t k0 = static_cast<uint32_t>(seed & 0xFFFFFFFFu);
  const uint32_t k1 = static_cast<uint32_t>(seed >> 32);
  const float kScale = 1.0f / 4294967296.0f;
  const float span = high - low;
  const uint32_t threads = (count + 3u) / 4u;
  for (uint32_t t = 0; t < threads; ++t) {
    uint32_t r[4];
    philox(counter_base + t, k0, k1, r);
    for (int i = 0; i < 4; ++i) {
      const uint32_t e = t * 4u + static_cast<uint32_t>(i);
      if (e >= count) break;
      const float u = static_cast<float>(r[i]) * kScale;
      out[e] = low + u * span;
    }
  }
}

// init_weights_with_config (default_trainer.cpp:1978-2180): hash at counter 0,
// then each layer's W and b slice, each advancing the counter by ceil(n/4).
void orc_init_params(const orc_model *m, uint64_t seed, float hash_range,
                     float *hash_out, float *mlp_out) {
  const Geo g = geo_of(m);
  const uint32_t hash_count = orc_hash_param_count(m);
  orc_philox_uniform(seed, 0u, hash_count, -hash_range, hash_range, hash_out);
  uint32_t ctr = (hash_count + 3u) / 4u;
  const float gain = std::sqrt(2.0f);
  struct Slice { int wc, bc, fan_in; };
  std::vector<Slice> layers;
  const int in = g.L * g.F;
  layers.push_back({in * g.H, g.H, in});
  for (int k = 1; k < g.NHL; ++k) layers.push_back({g.H * g.H, g.H, g.H});
  layers.push_back({g.H * g.M, g.M, g.H});
  float *dst = mlp_out;
  for (const Slice &s : layers) {
    const float fin = static_cast<float>(s.fan_in);
    const float bw = gain * std::sqrt(3.0f / fin);
    orc_philox_uniform(seed, ctr, static_cast<uint32_t>(s.wc), -bw, bw, dst);
    ctr += static_cast<uint32_t>((s.wc + 3) / 4);
    dst += s.wc;
    const float bb = 1.0f / std::sqrt(fin);
    orc_philox_uniform(seed, ctr, static_cast<uint32_t>(s.bc), -bb, bb, dst);
    ctr += static_cast<uint32_t>((s.bc + 3) / 4);
    dst += s.bc;
  }
}

void orc_encode(const orc_model *m, const float *table, const float *pos,
                int32_t n, float *feats, uint32_t *corner_idx, float *corner_w) {
  const Geo g = geo_of(m);
  std::vector<float> res(g.L);
  resolutions(m, res.data());
  for (int32_t i = 0; i < n; ++i) {
    const float *p = pos + static_cast<size_t>(i) * g.in_D;
    for (int l = 0; l < g.L; ++l) {
      const Level lv = level_of(g, p, res[l]);
      float feat[4];
      const size_t ci = (static_cast<size_t>(i) * g.L + l) * g.C;
      encode_level(g, table, lv, l, feat, corner_idx ? corner_idx + ci : nullptr,
                   corner_w ? corner_w + ci : nullptr);
      for (int f = 0; f < g.F; ++f)
        feats[static_cast<size_t>(i) * g.L * g.F + l * g.F + f] = feat[f];
    }
  }
}

void orc_forward(const orc_model *m, const float *table, const float *mlp,
                 const float *pos, int32_t n, float *out) {
  const Geo g = geo_of(m);
  const Offsets o = offsets_of(g);
  std::vector<float> res(g.L);
  resolutions(m, res.data());
#pragma omp parallel for schedule(static)
  for (int32_t i = 0; i < n; ++i) {
    float acts[8 * 512];
    forward_point(g, o, res.data(), table, mlp,
                  pos + static_cast<size_t>(i) * g.in_D, acts,
                  out + static_cast<size_t>(i) * g.M);
  }
}

void orc_forward_backward(const orc_model *m, const float *table,
                          const float *mlp, const float *pos, int32_t n,
                          const float *target, const float *d_out_ext,
                          int32_t *grad_hash, double *grad_mlp, uint32_t *mask,
                          double *loss_sum, float *out, int32_t n_threads) {
  const Geo g = geo_of(m);
  const Offsets o = offsets_of(g);
  std::vector<float> res(g.L);
  resolutions(m, res.data());
  const float inv_n = n > 0 ? 1.0f / static_cast<float>(n) : 0.0f;
  const int nt = threads_for(n_threads);
  std::vector<std::vector<double>> part(nt, std::vector<double>(o.total, 0.0));
  std::vector<double> lpart(nt, 0.0);
#pragma omp parallel num_threads(nt)
  {
#ifdef _OPENMP
    const int tid = omp_get_thread_num();
#else
    const int tid = 0;
#endif
    double *gW = part[tid].data();
    double lsum = 0.0;
    float acts[8 * 512];
    float outv[64];
    float dout[64];
#pragma omp for schedule(static)
    for (int32_t i = 0; i < n; ++i) {
      const float *p = pos + static_cast<size_t>(i) * g.in_D;
      forward_point(g, o, res.data(), table, mlp, p, acts, outv);
      if (out)
        for (int k = 0; k < g.M; ++k) out[static_cast<size_t>(i) * g.M + k] = outv[k];
      if (target) {
        lsum += static_cast<double>(
            loss_point(m, g, outv, target + static_cast<size_t>(i) * g.M, inv_n, dout));
      } else {
        for (int k = 0; k < g.M; ++k) dout[k] = d_out_ext[static_cast<size_t>(i) * g.M + k];
      }
      backward_point(g, o, res.data(), table, mlp, p, acts, dout, grad_hash, gW, mask);
    }
    lpart[tid] = lsum;
  }
  for (int t = 0; t < nt; ++t) {
    for (int k = 0; k < o.total; ++k) grad_mlp[k] += part[t][k];
    if (loss_sum) *loss_sum += lpart[t];
  }
}

// adam_params.h:33-52: bc = 1 - std::pow(beta, float(step + 1)) in fp32.
void orc_adam_bias_corrections(float beta1, float beta2, uint32_t logical_step,
                               float *bc1, float *bc2) {
  const float s = static_cast<float>(logical_step + 1);
  *bc1 = 1.0f - std::pow(beta1, s);
  *bc2 = 1.0f - std::pow(beta2, s);
}

}  // extern "C"

namespace {

// One Adam element (adam_kernel_msl.h:67-108 unified; :120-203 split).
inline void adam_elem(float &w, float &mo, float &ve, float g, float lr,
                      float beta1, float beta2, float eps, float bc1, float bc2,
                      float clip, float wd, float l1, float l2, bool is_mlp) {
  if (clip > 0.0f) g = std::fmin(std::fmax(g, -clip), clip);
  if (wd > 0.0f) {
    w = w - (lr * wd) * w;
  } else {
    if (!is_mlp && l1 > 0.0f) g = g + l1 * (w > 0.0f ? 1.0f : (w < 0.0f ? -1.0f : 0.0f));
    if (is_mlp && l2 > 0.0f) g = g + l2 * w;
  }
  const float mn = beta1 * mo + (1.0f - beta1) * g;
  const float vn = beta2 * ve + ((1.0f - beta2) * g) * g;
  mo = mn;
  ve = vn;
  const float mh = mn / bc1;
  const float vh = vn / bc2;
  w = w - (lr * mh) / (std::sqrt(vh) + eps);
}

}  // namespace

extern "C" {

void orc_adam_step(const orc_model *m, const orc_adam *a, uint32_t logical_step,
                   float *params, float *mom1, float *mom2,
                   const int32_t *grad_hash, const float *grad_mlp,
                   const uint32_t *mask, int32_t n_threads) {
  float bc1, bc2;
  orc_adam_bias_corrections(a->beta1, a->beta2, logical_step, &bc1, &bc2);
  const uint32_t nh = orc_hash_param_count(m);
  const uint32_t nm = orc_mlp_param_count(m);
  const float inv_scale = 1.0f / 65536.0f;
  const int nt = threads_for(n_threads);
  const uint32_t width = m->features_per_level == 2 ? 2u : 1u;
#pragma omp parallel for num_threads(nt) schedule(static)
  for (int64_t i = 0; i < static_cast<int64_t>(nh); ++i) {
    if (mask) {
      const uint32_t slot = static_cast<uint32_t>(i) / width;
      if (!((mask[slot >> 5] >> (slot & 31u)) & 1u)) continue;
    }
    const float g = static_cast<float>(grad_hash[i]) * inv_scale;
    adam_elem(params[i], mom1[i], mom2[i], g, a->lr_encoding, a->beta1, a->beta2,
              a->epsilon, bc1, bc2, a->grad_clip, a->weight_decay, a->l1_reg,
              a->l2_reg, false);
  }
  for (uint32_t i = 0; i < nm; ++i) {
    const size_t k = nh + i;
    adam_elem(params[k], mom1[k], mom2[k], grad_mlp[i], a->lr_network, a->beta1,
              a->beta2, a->epsilon, bc1, bc2, a->grad_clip, a->weight_decay,
              a->l1_reg, a->l2_reg, true);
  }
}

void orc_morton_codes(const float *pos, int32_t n, int32_t dims, uint32_t *codes) {
  for (int32_t i = 0; i < n; ++i) {
    const float *p = pos + static_cast<size_t>(i) * dims;
    if (dims == 4) {
      codes[i] = (expand4(quant(p[3], 256.0f, 255.0f)) << 3) |
                 (expand4(quant(p[2], 256.0f, 255.0f)) << 2) |
                 (expand4(quant(p[1], 256.0f, 255.0f)) << 1) |
                 expand4(quant(p[0], 256.0f, 255.0f));
    } else {
      const float z = dims == 3 ? p[2] : 0.0f;
      codes[i] = (expand3(quant(z, 1024.0f, 1023.0f)) << 2) |
                 (expand3(quant(p[1], 1024.0f, 1023.0f)) << 1) |
                 expand3(quant(p[0], 1024.0f, 1023.0f));
    }
  }
}

float orc_training_step(const orc_model *m, const orc_adam *a,
                        uint32_t logical_step, float *params, float *mom1,
                        float *mom2, const float *pos, const float *target,
                        int32_t n, int32_t dense_hash, int32_t n_threads) {
  const uint32_t nh = orc_hash_param_count(m);
  const uint32_t nm = orc_mlp_param_count(m);
  std::vector<int32_t> gh(nh, 0);
  std::vector<double> gm(nm, 0.0);
  std::vector<uint32_t> mask(orc_mask_word_count(m), 0u);
  double loss = 0.0;
  orc_forward_backward(m, params, params + nh, pos, n, target, nullptr, gh.data(),
                       gm.data(), mask.data(), &loss, nullptr, n_threads);
  std::vector<float> gmf(nm);
  for (uint32_t i = 0; i < nm; ++i) gmf[i] = static_cast<float>(gm[i]);
  // Sparse hash Adam needs l1_reg == 0 (default_trainer.cpp:1868-1876).
  const bool dense = dense_hash != 0 || a->l1_reg != 0.0f;
  orc_adam_step(m, a, logical_step, params, mom1, mom2, gh.data(), gmf.data(),
                dense ? nullptr : mask.data(), n_threads);
  return n > 0 ? static_cast<float>(loss / static_cast<double>(n)) : 0.0f;
}

// FieldEvaluator::evaluate_with_gradient (neural_sdf_analytical_eval_gradient_
// points, mlp_kernel_emitter.cpp:1865-2090; host default_trainer.cpp:467-620):
// out[N][M] as orc_forward, grads[N][M][D] = d out_m / d pos. Per output m
// the backward starts from d out_m = 1: g_last[j] = WO[j][m] * [h_last > 0],
// g_prev[i] = (sum_j g[j] * W[i][j]) * [h_prev > 0] (:1966-1990); then
// grad_feat = sum_j g0[j] * W0[feat][j] and grad_pos += (grad_feat * r_l) *
// d(feat)/d(frac) over levels and features (:1995-2060). 2D points are the
// lifted (x, y, 0); their z component is dropped.
void orc_evaluate_with_gradient(const orc_model *m, const float *table, const float *mlp,
                                const float *pos, int32_t n, float *out, float *grads) {
  const Geo g = geo_of(m);
  const Offsets o = offsets_of(g);
  std::vector<float> res(g.L);
  resolutions(m, res.data());
#pragma omp parallel for schedule(static)
  for (int32_t i = 0; i < n; ++i) {
    const float *p = pos + static_cast<size_t>(i) * g.in_D;
    std::vector<float> acts(static_cast<size_t>(g.NHL) * g.H);
    forward_point(g, o, res.data(), table, mlp, p, acts.data(),
                  out + static_cast<size_t>(i) * g.M);
    std::vector<float> cur(g.H), nxt(g.H);
    for (int mm = 0; mm < g.M; ++mm) {
      const float *last = acts.data() + (g.NHL - 1) * g.H;
      for (int j = 0; j < g.H; ++j)
        cur[j] = mlp[o.w[g.NHL] + j * g.M + mm] * (last[j] > 0.0f ? 1.0f : 0.0f);
      for (int k = g.NHL - 1; k >= 1; --k) {
        const float *hp = acts.data() + (k - 1) * g.H;
        for (int ii = 0; ii < g.H; ++ii) {
          float acc = 0.0f;
          for (int j = 0; j < g.H; ++j) acc = acc + cur[j] * mlp[o.w[k] + ii * g.H + j];
          nxt[ii] = acc * (hp[ii] > 0.0f ? 1.0f : 0.0f);
        }
        std::swap(cur, nxt);
      }
      float gp[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      for (int l = 0; l < g.L; ++l) {
        const Level lv = level_of(g, p, res[l]);
        for (int f = 0; f < g.F; ++f) {
          const int row = o.w[0] + (l * g.F + f) * g.H;
          float gf = 0.0f;
          for (int j = 0; j < g.H; ++j) gf = gf + cur[j] * mlp[row + j];
          float dv[4];
          level_frac_grad(g, table, lv, l, f, dv);
          const float s = gf * res[l];
          for (int a = 0; a < g.D; ++a) gp[a] = gp[a] + s * dv[a];
        }
      }
      for (int a = 0; a < g.in_D; ++a)
        grads[(static_cast<size_t>(i) * g.M + mm) * g.in_D + a] = gp[a];
    }
  }
}

}  // extern "C"
