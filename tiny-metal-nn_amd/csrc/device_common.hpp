// device_common.hpp -- gfx950 device helpers shared by the tmnn HIP kernels:
// hash / corner selection, Philox, Morton codes, MFMA operand types.
//
// All device code is compiled with -ffp-contract=off: every multiply and add
// in the encoding, loss and Adam paths rounds on its own, in the order the
// reference's MSL writes it (src/tiny_metal_nn/kernels/mlp_kernel_emitter.cpp).
// MFMA products are the only fused arithmetic.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tmnn_hip {

// Hash primes of the reference's GPU kernels (mlp_kernel_emitter.cpp:16-18);
// the 4D prime is the GPU value 56711039, not tcnn's 3674653429.
constexpr uint32_t kPrimeY = 2654435761u;
constexpr uint32_t kPrimeZ = 805459861u;
constexpr uint32_t kPrimeW = 56711039u;
// int32 fixed-point hash gradient scale (mlp_kernel_emitter.cpp:2741-2744).
constexpr float kGradScale = 65536.0f;
constexpr int kMaxLevels = 32;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// (x*1 ^ y*PY ^ z*PZ [^ w*PW]) mod T with uint32 wraparound
// (hash_coords / hash_coords_4d, mlp_kernel_emitter.cpp:144-161).
// T is a power of two, so "mod T" is "& (T-1)".
template <int D>
__device__ __forceinline__ uint32_t hash_corner(const int *c, uint32_t tmask) {
  uint32_t h = static_cast<uint32_t>(c[0]);
  h ^= static_cast<uint32_t>(c[1]) * kPrimeY;
  if (D >= 3) h ^= static_cast<uint32_t>(c[2]) * kPrimeZ;
  if (D == 4) h ^= static_cast<uint32_t>(c[3]) * kPrimeW;
  return h & tmask;
}

// The reference lifts 2D points to (x, y, 0); the corners of the z = 1 plane
// hash as (x ^ y*PY ^ PZ). Used to mark them for the lazy Adam mask.
__device__ __forceinline__ uint32_t hash_corner_lift_z1(const int *c,
                                                       uint32_t tmask) {
  uint32_t h = static_cast<uint32_t>(c[0]);
  h ^= static_cast<uint32_t>(c[1]) * kPrimeY;
  h ^= kPrimeZ;
  return h & tmask;
}

// Per-level cell: bc = int(floor(p*r)), frac = p*r - floor(p*r)
// (mlp_kernel_emitter.cpp:240-254).
template <int D>
struct Cell {
  int bc[D];
  float fr[D];
};

template <int D>
__device__ __forceinline__ Cell<D> cell_of(const float *p, float res) {
  Cell<D> c;
#pragma unroll
  for (int a = 0; a < D; ++a) {
    const float s = p[a] * res;
    const float fl = floorf(s);
    c.bc[a] = static_cast<int>(fl);
    c.fr[a] = s - fl;
  }
  return c;
}

// Corner k of a cell in the reference's loop order (dw, dz, dy outer, dx
// inner): coordinates and the per-axis weights (1-f or f).
template <int D>
__device__ __forceinline__ void corner_of(const Cell<D> &c, int k, int *co,
                                          float *wc) {
#pragma unroll
  for (int a = 0; a < D; ++a) {
    const int d = (k >> a) & 1;
    co[a] = c.bc[a] + d;
    wc[a] = d ? c.fr[a] : (1.0f - c.fr[a]);
  }
}

// Corner weight ((wx*wy)*wz)(*wt), one rounding per multiply. For native 2D
// the reference's lifted wz is exactly 1 on the z = 0 plane.
template <int D>
__device__ __forceinline__ float corner_weight(const float *wc) {
  float w = wc[0] * wc[1];
  if (D >= 3) w = w * wc[2];
  if (D == 4) w = w * wc[3];
  return w;
}

// MSL int(x) on the gradient path: truncate toward zero; saturate out of
// range and map NaN to 0 explicitly so the result is defined everywhere.
__device__ __forceinline__ int32_t f2i_trunc(float x) {
  if (!(x == x)) return 0;
  if (x >= 2147483648.0f) return 2147483647;
  if (x <= -2147483648.0f) return static_cast<int32_t>(0x80000000u);
  return static_cast<int32_t>(x);
}

// Philox-4x32-10 (Salmon et al., SC'11) with the reference's counter/key
// convention (metal_context.cpp:735-752): ctr = (base + tid, 0, 0, 0),
// key = (seed lo, seed hi).
__device__ __forceinline__ void philox4x32_10(uint32_t ctr, uint32_t k0,
                                              uint32_t k1, uint32_t *out) {
  uint32_t c0 = ctr, c1 = 0u, c2 = 0u, c3 = 0u;
#pragma unroll
  for (int i = 0; i < 10; ++i) {
    const uint32_t hi0 = __umulhi(0xD2511F53u, c0);
    const uint32_t lo0 = 0xD2511F53u * c0;
    const uint32_t hi1 = __umulhi(0xCD9E8D57u, c2);
    const uint32_t lo1 = 0xCD9E8D57u * c2;
    const uint32_t n0 = hi1 ^ c1 ^ k0;
    const uint32_t n2 = hi0 ^ c3 ^ k1;
    c0 = n0;
    c1 = lo1;
    c2 = n2;
    c3 = lo0;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  out[0] = c0;
  out[1] = c1;
  out[2] = c2;
  out[3] = c3;
}

// Morton code of the reference (morton_sort.h:14-57): (v*0.5+0.5)*1024
// clamped to [0, 1023] per axis, 10 bits interleaved x | y<<1 | z<<2;
// 4D uses 8 bits per axis.
__device__ __forceinline__ uint32_t expand_bits_3d(uint32_t v) {
  v = (v | (v << 16)) & 0x030000FFu;
  v = (v | (v << 8)) & 0x0300F00Fu;
  v = (v | (v << 4)) & 0x030C30C3u;
  v = (v | (v << 2)) & 0x09249249u;
  return v;
}

__device__ __forceinline__ uint32_t expand_bits_4d(uint32_t v) {
  v &= 0xFFu;
  v = (v | (v << 16)) & 0x000F000Fu;
  v = (v | (v << 8)) & 0x00C30C03u;
  v = (v | (v << 4)) & 0x09090909u;
  v = (v | (v << 2)) & 0x11111111u;
  return v;
}

__device__ __forceinline__ uint32_t morton_quant(float v, float scale,
                                                 float top) {
  const float mapped = (v * 0.5f + 0.5f) * scale;
  return static_cast<uint32_t>(fminf(fmaxf(mapped, 0.0f), top));
}

__device__ __forceinline__ uint32_t expand_bits_2d(uint32_t v) {
  v &= 0x3FFu;
  v = (v | (v << 8)) & 0x00FF00FFu;
  v = (v | (v << 4)) & 0x0F0F0F0Fu;
  v = (v | (v << 2)) & 0x33333333u;
  v = (v | (v << 1)) & 0x55555555u;
  return v;
}

// Morton code of one point (morton_sort.h:14-57): the reference's 10-bit (3D)
// or 8-bit (4D) quantisation. 2D points are the reference's lifted
// (x, y, 0); their z bits are all zero, so the code keeps only the x/y
// interleave (20 bits), which sorts identically.
template <int D>
__device__ __forceinline__ uint32_t morton_code_of(const float *p) {
  if constexpr (D == 4)
    return (expand_bits_4d(morton_quant(p[3], 256.0f, 255.0f)) << 3) |
           (expand_bits_4d(morton_quant(p[2], 256.0f, 255.0f)) << 2) |
           (expand_bits_4d(morton_quant(p[1], 256.0f, 255.0f)) << 1) |
           expand_bits_4d(morton_quant(p[0], 256.0f, 255.0f));
  else if constexpr (D == 3)
    return (expand_bits_3d(morton_quant(p[2], 1024.0f, 1023.0f)) << 2) |
           (expand_bits_3d(morton_quant(p[1], 1024.0f, 1023.0f)) << 1) |
           expand_bits_3d(morton_quant(p[0], 1024.0f, 1023.0f));
  else
    return (expand_bits_2d(morton_quant(p[1], 1024.0f, 1023.0f)) << 1) |
           expand_bits_2d(morton_quant(p[0], 1024.0f, 1023.0f));
}
__device__ __forceinline__ uint32_t morton_code(const float *p, int dims) {
  if (dims == 4) return morton_code_of<4>(p);
  if (dims == 3) return morton_code_of<3>(p);
  return morton_code_of<2>(p);
}

}  // namespace tmnn_hip
