// Shared device helpers for the GDN HIP kernels (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gdn {

constexpr int kHeadDim = 128;   // K = V = D, fixed by both operators
constexpr int kWave = 64;       // CDNA wavefront width

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// Round-to-nearest-even fp32 -> bf16 (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float x) {
  __bf16 h = (__bf16)x;
  return __builtin_bit_cast(uint16_t, h);
}

// Two bf16 packed in one dword -> two floats.
__device__ __forceinline__ void unpack_bf16x2(uint32_t w, float& lo, float& hi) {
  lo = __uint_as_float(w << 16);
  hi = __uint_as_float(w & 0xffff0000u);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return uint32_t(f32_to_bf16_bits(lo)) | (uint32_t(f32_to_bf16_bits(hi)) << 16);
}

// Decode softplus: x <= 20 ? log(1 + e^x) : x   (reference DEC:21-23).
__device__ __forceinline__ float softplus_thresh20(float x) {
  return x <= 20.0f ? log1pf(expf(x)) : x;
}

// Prefill softplus: x > 0 ? x + log(1 + e^-x) : log(1 + e^x)   (reference PRE:1711-1720).
__device__ __forceinline__ float softplus_stable(float x) {
  return x > 0.0f ? x + log1pf(expf(-x)) : log1pf(expf(x));
}

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }

// DPP helpers.  dpp_ctrl encodings: quad_perm = 0x00..0xFF, row_ror:n = 0x120 + n.
template <int kCtrl>
__device__ __forceinline__ float dpp_f32(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), kCtrl, 0xf, 0xf, false));
}

// DPP move with a row mask: rows outside row_mask receive 0.
template <int kCtrl, int kRowMask>
__device__ __forceinline__ float dpp_f32_rows(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), kCtrl, kRowMask, 0xf, false));
}

// Inclusive prefix sum over the 64 lanes of a wave (lanes shifted in from
// outside a row read 0): a scan within each 16-lane row by row_shr, then the
// row totals carried forward by row_bcast:15 / row_bcast:31.
__device__ __forceinline__ float wave_inclusive_scan(float x) {
  x += dpp_f32<0x111>(x);             // row_shr:1
  x += dpp_f32<0x112>(x);             // row_shr:2
  x += dpp_f32<0x114>(x);             // row_shr:4
  x += dpp_f32<0x118>(x);             // row_shr:8
  x += dpp_f32_rows<0x142, 0xa>(x);   // row_bcast:15 into rows 1 and 3
  x += dpp_f32_rows<0x143, 0xc>(x);   // row_bcast:31 into rows 2 and 3
  return x;
}

// Sum over the 16 lanes of a DPP row; every lane of the row receives the total.
__device__ __forceinline__ float row16_sum(float x) {
  x += dpp_f32<0x128>(x);   // row_ror:8
  x += dpp_f32<0x124>(x);   // row_ror:4
  x += dpp_f32<0x4E>(x);    // quad_perm [2,3,0,1]
  x += dpp_f32<0xB1>(x);    // quad_perm [1,0,3,2]
  return x;
}

// q / k L2 normalisation (optional, GDN_QK_L2NORM): a row x of 128 elements
// is used as x (sum x^2 + 1e-6)^(-1/2), all in fp32 (no intermediate rounding;
// the bf16 squares are exact in fp32, v_rsq_f32 is within 1 ulp).
constexpr float kL2NormEps = 1e-6f;

__device__ __forceinline__ float l2norm_rsqrt(float sum_sq) {
  return __builtin_amdgcn_rsqf(sum_sq + kL2NormEps);
}

// The factor (sum x^2 + 1e-6)^(-1/2) of a row held 8 per lane by the 16 lanes
// of a DPP row (every lane of the row receives it).
__device__ __forceinline__ float l2norm_factor_row16(const float (&x)[8]) {
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss = fmaf(x[e], x[e], ss);
  return l2norm_rsqrt(row16_sum(ss));
}

__device__ __forceinline__ void l2norm_row16(float (&x)[8]) {
  const float r = l2norm_factor_row16(x);
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] *= r;
}

}  // namespace gdn
