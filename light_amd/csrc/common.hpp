// common.hpp -- shared definitions for libhipq (gfx950 / CDNA4 only).
//
// Formats are GGUF block layouts exactly as Light stores them (dtype/dtype.go:53-60,
// quant/q4_0.go:18-27, quant/q5_0.go:11-20, quant/q8_0.go:10-17, quant/q4_k.go:14-24,
// quant/q5_k.go:11-22, quant/q6_k.go:10-20, quant/q8_1.go:10-18):
// a tensor's bytes are the GGUF bytes.  The one exception is Q6_K_R, an opt-in load-time
// layout of Q6_K (q6k_repack.hip) that the caller asks for explicitly.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/hipq.h"

namespace hq {

// Light's dtype.DType codes (dtype/dtype.go:13-37).
enum DType : int {
  F16 = HQ_F16, BF16 = HQ_BF16, F32 = HQ_F32,
  Q4_0 = HQ_Q4_0, Q5_0 = HQ_Q5_0, Q8_0 = HQ_Q8_0, Q8_1 = HQ_Q8_1, Q4_K = HQ_Q4_K, Q5_K = HQ_Q5_K, Q6_K = HQ_Q6_K,
  Q6_K_R = HQ_Q6_K_R,
};

constexpr int kWave = 64;  // CDNA wavefront width

// Prepared activations ("act" layout, internal to libhipq) for x (M, K): a two-level
// int8 quantization of x, stored planar so kernels can use 16-byte loads:
//   q1  int8   [M][K]      at 0                 q8_1's quants of x (d = amax / 127)
//   q2  int8   [M][K]      at act_q2_off(M, K)  quants of the residual x - d*q1, step e = d / 254
//   de  f32x2  [M][K/32]   at act_d_off(M, K)   (d, e) per 32-block (d before q8_1's f16 rounding)
//   sx  f32    [M][K/32]   at act_s_off(M, K)   sum of the block's x (f32)
// x ~= d*q1 + e*q2 with |error| <= e/2: about 2^-15 of the block's amax.  q1 and d are
// bit-identical to the q8_1 quantization of the same x.
__host__ __device__ constexpr int64_t act_q2_off(int64_t M, int64_t K) { return (M * K + 255) & ~(int64_t)255; }
__host__ __device__ constexpr int64_t act_d_off(int64_t M, int64_t K) { return 2 * act_q2_off(M, K); }
__host__ __device__ constexpr int64_t act_s_off(int64_t M, int64_t K) { return act_d_off(M, K) + 8 * M * (K / 32); }
__host__ __device__ constexpr int64_t act_bytes(int64_t M, int64_t K) {
  return (act_s_off(M, K) + 4 * M * (K / 32) + 255) & ~(int64_t)255;
}

// Bytes per block / elements per block (dtype/dtype.go:53-60).
struct BlockInfo { int elems, bytes; };
__host__ __device__ constexpr BlockInfo block_info(int dt) {
  return dt == Q4_0 ? BlockInfo{32, 18}
       : dt == Q5_0 ? BlockInfo{32, 22}
       : dt == Q8_0 ? BlockInfo{32, 34}
       : dt == Q8_1 ? BlockInfo{32, 36}
       : dt == Q4_K ? BlockInfo{256, 144}
       : dt == Q5_K ? BlockInfo{256, 176}
       : dt == Q6_K ? BlockInfo{256, 210}
       : dt == Q6_K_R ? BlockInfo{256, 210}
       : BlockInfo{0, 0};
}

// Row bytes of the Q6_K_R layout: the 210 bytes of each block, padded per row to 16.
__host__ __device__ constexpr int64_t q6kr_row_bytes(int64_t K) { return (K / 256 * 210 + 15) & ~(int64_t)15; }

// f16 -> f32 widening is exact for every finite pattern (v_cvt_f32_f16), which is
// what Half.ToF32 computes (dtype/half.go:84-113).
__device__ __forceinline__ float h2f(uint32_t h16) {
  _Float16 h;
  uint16_t b = (uint16_t)h16;
  __builtin_memcpy(&h, &b, 2);
  return (float)h;
}

// f32 -> f16 as Light's HalfFromF32 (dtype/half.go:15-81): IEEE round-to-nearest-even,
// except that |f| < 2^-24 flushes to signed zero (:43-46) where IEEE would round
// (2^-25, 2^-24) up to the smallest subnormal.
__device__ __forceinline__ uint16_t f2h_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) < (103u << 23)) return (uint16_t)((u >> 16) & 0x8000u);
  _Float16 h = (_Float16)f;
  uint16_t b;
  __builtin_memcpy(&b, &h, 2);
  return b;
}

// BF16FromF32 (dtype/half.go:118-129): RNE, NaNs keep their top bits with the quiet bit set.
__device__ __forceinline__ uint16_t f2bf_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffffu)) return (uint16_t)((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float bf2f(uint32_t b16) { return __uint_as_float(b16 << 16); }

// Signed 4 x int8 dot product accumulate (v_dot4_i32_i8).
__device__ __forceinline__ int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// Full-wave sum (xor butterfly over 64 lanes).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// Q4_K 6-bit (scale, min) of sub-block j from the three scale dwords
// (getScaleMinK4, quant/q4_k.go:83-89): s0 = scales[0..3], s1 = scales[4..7], s2 = scales[8..11].
__device__ __forceinline__ void q4k_scale_min(int j, uint32_t s0, uint32_t s1, uint32_t s2, int &sc, int &m) {
  if (j < 4) {
    sc = (s0 >> (8 * j)) & 63;
    m = (s1 >> (8 * j)) & 63;
  } else {
    int k = j - 4;
    uint32_t a = (s2 >> (8 * k)) & 0xff, lo = (s0 >> (8 * k)) & 0xff, hi = (s1 >> (8 * k)) & 0xff;
    sc = (int)((a & 0x0f) | ((lo >> 6) << 4));
    m = (int)((a >> 4) | ((hi >> 6) << 4));
  }
}

// Light's SiLU (kernels/cpu/unary.go:219-222) and exact GELU (:216, :263-265), the gate
// activation of the gated MLP (HQ_ACT_SILU = 0, HQ_ACT_GELU_ERF = 1).
__device__ __forceinline__ float gate_act(float g, int act) {
  if (act == 1) return 0.5f * g * (1.0f + erff(g * 0.70710678118654752f));
  return g / (1.0f + expf(-g));
}

}  // namespace hq
