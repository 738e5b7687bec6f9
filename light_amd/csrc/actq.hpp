// actq.hpp -- the two-level int8 activation quantization of one 32-element block,
// shared by the quantize kernel and the GEMVs that quantize x in LDS.
//
// Eight lanes of an aligned 8-lane group (lanes 8i .. 8i+7 of a wave) hold one block,
// four elements each, and call act_quant8 together.  Level 1 is q8_1's rounding (encodeQ8_0, quant/quantize.go:70-86):
// d = amax / 127, id = 1 / d, q1 = RoundToEven(v * id).  Level 2 quantizes the residual
// r = v - d*q1 at step e = d / 254 (|q2| <= 127).  sum is the block's f32 sum, reduced
// pairwise in lane order so every caller gets the same bits.
//
// Non-finite x: fmaxf drops a NaN from amax, so a block holding one would quantize to
// finite codes.  A NaN block sum (a NaN, or +Inf with -Inf, in the block) sets d and e to
// NaN instead, and an Inf sets d to Inf: either way every dot over the block is NaN, as
// Light's F32 arithmetic gives a non-finite result for that row.
#pragma once

#include "common.hpp"

namespace hq {

struct ActQ {
  uint32_t q1, q2;  // this lane's four quants per level, packed little-endian
  float d, e, sum;  // block values (equal in all eight lanes)
  int qsum;         // sum of the block's level-1 quants
};

// Exchange inside an aligned 8-lane group with DPP: CTRL 0xB1 = lane ^ 1, 0x4E = lane ^ 2
// (quad_perm), 0x141 = lane 7 - i (row_half_mirror).  After the two quad steps every lane
// of a quad holds the quad's value, so the mirror step reads the other quad, as ^ 4 would.
template <int CTRL>
__device__ __forceinline__ float dpp8f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp8i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}

// d and e of a block whose sum is NaN become NaN (see the header).
template <class Q>
__device__ __forceinline__ void poison_nan_block(Q &r) {
  if (r.sum != r.sum) r.d = r.e = r.sum;
}

__device__ __forceinline__ ActQ act_quant8(const float v[4]) {
  float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
  amax = fmaxf(amax, dpp8f<0xB1>(amax));
  amax = fmaxf(amax, dpp8f<0x4E>(amax));
  amax = fmaxf(amax, dpp8f<0x141>(amax));
  ActQ r;
  r.d = __fdiv_rn(amax, 127.0f);
  const float id = r.d != 0.f ? __fdiv_rn(1.0f, r.d) : 0.f;
  r.e = __fdiv_rn(r.d, 254.0f);
  const float ie = r.e != 0.f ? __fdiv_rn(1.0f, r.e) : 0.f;
  int qs = 0;
  r.q1 = r.q2 = 0;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int q = (int)rintf(__fmul_rn(v[j], id));
    qs += q;
    const float res = __fsub_rn(v[j], __fmul_rn(r.d, (float)q));
    int q2 = (int)rintf(__fmul_rn(res, ie));
    q2 = q2 > 127 ? 127 : (q2 < -127 ? -127 : q2);
    r.q1 |= (uint32_t)(q & 0xff) << (8 * j);
    r.q2 |= (uint32_t)(q2 & 0xff) << (8 * j);
  }
  // Pairwise block sum: ((s0 + s1) + (s2 + s3)) + ((s4 + s5) + (s6 + s7)) over the lanes'
  // partial sums, the same bits in every lane (each step adds two equal-order operands).
  float bsum = __fadd_rn(__fadd_rn(v[0], v[1]), __fadd_rn(v[2], v[3]));
  bsum = __fadd_rn(bsum, dpp8f<0xB1>(bsum));
  bsum = __fadd_rn(bsum, dpp8f<0x4E>(bsum));
  bsum = __fadd_rn(bsum, dpp8f<0x141>(bsum));
  qs += dpp8i<0xB1>(qs);
  qs += dpp8i<0x4E>(qs);
  qs += dpp8i<0x141>(qs);
  r.sum = bsum;
  r.qsum = qs;
  poison_nan_block(r);
  return r;
}

// The same two-level quantization with reciprocal-based scale arithmetic instead of IEEE
// divisions, for activations produced and consumed inside one kernel pair (the fused
// GEMV's own x, the gated GEMV's output).  The stored d and e are the ones the residual
// uses, so x = d*q1 + e*q2 holds to e/2 (up to a rounding of the reciprocals) exactly as
// for act_quant8; q1 may differ from q8_1's in the last unit where v/d is near a tie.
__device__ __forceinline__ ActQ act_quant8_fast(const float v[4]) {
  float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
  amax = fmaxf(amax, dpp8f<0xB1>(amax));
  amax = fmaxf(amax, dpp8f<0x4E>(amax));
  amax = fmaxf(amax, dpp8f<0x141>(amax));
  ActQ r;
  const float ra = amax > 0.f ? __builtin_amdgcn_rcpf(amax) : 0.f;
  r.d = amax * (1.0f / 127.0f);
  r.e = r.d * (1.0f / 254.0f);
  const float id = 127.0f * ra, ie = 254.0f * id;
  r.q1 = r.q2 = 0;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const float qf = rintf(v[j] * id);
    const float res = __fmaf_rn(-r.d, qf, v[j]);
    const float q2f = fminf(fmaxf(rintf(res * ie), -127.f), 127.f);
    r.q1 |= (uint32_t)((int)qf & 0xff) << (8 * j);
    r.q2 |= (uint32_t)((int)q2f & 0xff) << (8 * j);
  }
  float bsum = (v[0] + v[1]) + (v[2] + v[3]);
  bsum += dpp8f<0xB1>(bsum);
  bsum += dpp8f<0x4E>(bsum);
  bsum += dpp8f<0x141>(bsum);
  r.sum = bsum;
  r.qsum = 0;
  poison_nan_block(r);
  return r;
}

// Two-level quantization of one 32-element block held by two adjacent lanes (lanes 2i,
// 2i+1), sixteen elements each: the work per element is four VALU operations.  Same
// scales as act_quant8_fast (d = amax / 127, e = d / 254, reciprocal-based); rounding to
// nearest-even by the magic-number add (2^23 + 2^22: the float's low byte is the rounded
// integer).  |v * id| <= 127 (1 + 2^-22) and |r * ie| <= 127 (1 + 2^-20), so no level
// needs a clamp.  q1 / q2: the lane's sixteen quants per level, little-endian bytes.
struct ActQ16 {
  uint32_t q1[4], q2[4];
  float d, e, sum;
};

__device__ __forceinline__ uint32_t pack_lo_bytes(float a, float b, float c, float d) {
  const uint32_t ab = __builtin_amdgcn_perm(__float_as_uint(b), __float_as_uint(a), 0x0c0c0400u);
  const uint32_t cd = __builtin_amdgcn_perm(__float_as_uint(d), __float_as_uint(c), 0x04000c0cu);
  return ab | cd;
}

__device__ __forceinline__ ActQ16 act_quant16_fast(const float (&v)[16]) {
  constexpr float MAGIC = 12582912.0f;  // 1.5 * 2^23
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < 16; j += 2) amax = __builtin_fmaxf(amax, __builtin_fmaxf(fabsf(v[j]), fabsf(v[j + 1])));
  amax = fmaxf(amax, dpp8f<0xB1>(amax));
  ActQ16 r;
  const float ra = amax > 0.f ? __builtin_amdgcn_rcpf(amax) : 0.f;
  r.d = amax * (1.0f / 127.0f);
  r.e = r.d * (1.0f / 254.0f);
  const float id = 127.0f * ra, ie = 254.0f * id;
  float f1[16], f2[16];
#pragma unroll
  for (int j = 0; j < 16; j++) {
    f1[j] = __fmaf_rn(v[j], id, MAGIC);
    const float res = __fmaf_rn(-r.d, f1[j] - MAGIC, v[j]);
    f2[j] = __fmaf_rn(res, ie, MAGIC);
  }
#pragma unroll
  for (int k = 0; k < 4; k++) {
    r.q1[k] = pack_lo_bytes(f1[4 * k], f1[4 * k + 1], f1[4 * k + 2], f1[4 * k + 3]);
    r.q2[k] = pack_lo_bytes(f2[4 * k], f2[4 * k + 1], f2[4 * k + 2], f2[4 * k + 3]);
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 16; j += 4) s += (v[j] + v[j + 1]) + (v[j + 2] + v[j + 3]);
  r.sum = s + dpp8f<0xB1>(s);
  poison_nan_block(r);
  return r;
}

// One lane's Q4_K contribution from its two sub-blocks A (low nibbles) and B (high
// nibbles) of a 64-element pair: d * sum_s sc_s (d1_s dot1_s + e_s dot2_s)
// - dmin * sum_s m_s sx_s, with de = (dA, eA, dB, eB) and ss = (sxA, sxB).  Every
// rounding is explicit so all Q4_K GEMV kernels produce the same bits.
__device__ __forceinline__ float q4k_pair(float d, float dmin, float scA, float scB, float mnA, float mnB, float4 de,
                                          float2 ss, int dA, int dA2, int dB, int dB2) {
  const float va = __fmaf_rn(de.y, (float)dA2, __fmul_rn(de.x, (float)dA));
  const float vb = __fmaf_rn(de.w, (float)dB2, __fmul_rn(de.z, (float)dB));
  const float v = __fmaf_rn(scB, vb, __fmul_rn(scA, va));
  const float mn = __fmaf_rn(mnB, ss.y, __fmul_rn(mnA, ss.x));
  return __fmaf_rn(d, v, -__fmul_rn(dmin, mn));
}

// q4k_pair with sub-block B's dots taken on 16 * (q - 8) (high nibbles masked in place with
// the sign bit flipped): sum(q x) = dot / 16 + 8 * sum(x), with the exact block sum sx of x
// standing in for the quantized one (the difference is below the activations' own
// quantization error, e/2 per element).
__device__ __forceinline__ float q4k_pair_h16(float d, float dmin, float scA, float scB, float mnA, float mnB,
                                              float4 de, float2 ss, int dA, int dA2, int dB16, int dB216) {
  const float va = __fmaf_rn(de.y, (float)dA2, __fmul_rn(de.x, (float)dA));
  const float vb16 = __fmaf_rn(de.w, (float)dB216, __fmul_rn(de.z, (float)dB16));
  const float vb = __fmaf_rn(vb16, 0.0625f, __fmul_rn(8.0f, ss.y));
  const float v = __fmaf_rn(scB, vb, __fmul_rn(scA, va));
  const float mn = __fmaf_rn(mnB, ss.y, __fmul_rn(mnA, ss.x));
  return __fmaf_rn(d, v, -__fmul_rn(dmin, mn));
}

// Single-level forms of q4k_pair / q4k_pair_h16: x is q1 with its step d only (q8_1).
__device__ __forceinline__ float q4k_pair1(float d, float dmin, float scA, float scB, float mnA, float mnB, float4 de,
                                           float2 ss, int dA, int dB) {
  const float v = __fmaf_rn(scB, __fmul_rn(de.z, (float)dB), __fmul_rn(scA, __fmul_rn(de.x, (float)dA)));
  const float mn = __fmaf_rn(mnB, ss.y, __fmul_rn(mnA, ss.x));
  return __fmaf_rn(d, v, -__fmul_rn(dmin, mn));
}
__device__ __forceinline__ float q4k_pair1_h16(float d, float dmin, float scA, float scB, float mnA, float mnB,
                                               float4 de, float2 ss, int dA, int dB16) {
  const float vb = __fmaf_rn(__fmul_rn(de.z, (float)dB16), 0.0625f, __fmul_rn(8.0f, ss.y));
  const float v = __fmaf_rn(scB, vb, __fmul_rn(scA, __fmul_rn(de.x, (float)dA)));
  const float mn = __fmaf_rn(mnB, ss.y, __fmul_rn(mnA, ss.x));
  return __fmaf_rn(d, v, -__fmul_rn(dmin, mn));
}

}  // namespace hq
