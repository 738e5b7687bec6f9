// decode.hpp -- bit-exact decode of eight consecutive elements of a GGUF row.
//
// Thread t of a block-major walk decodes elements [8t, 8t+8).  The arithmetic is
// Light's CPU decoders', operation for operation and explicitly rounded, so no
// multiply-add is fused:
//   Q8_0  y = d * q                         (kernels/cpu/quant_matmul.go:29-34)
//   Q4_0  y = d * (q - 8)                   (kernels/cpu/quant_matmul.go:35-42)
//   Q5_0  y = d * (q5 - 16)                 (kernels/cpu/quant_matmul.go:43-53)
//   Q5_K  y = (d * sc) * q5 - (dmin * m)    (quant/q5_k.go:50-83)
//   Q4_K  y = (d * sc) * q - (dmin * m)     (kernels/cpu/quant_matmul.go:54-68)
//   Q6_K  y = (d * int8 sc) * (raw - 32)    (kernels/cpu/quant_matmul.go:69-87)
//   Q8_1  y = d * q                         (quant/q8_1.go:21-57)
// Q4_K / Q5_K need a 16-byte aligned block base; the other formats use byte loads.
#pragma once
#include "common.hpp"

namespace hq {

__device__ __forceinline__ uint32_t ld_u16(const uint8_t *p) { return *reinterpret_cast<const uint16_t *>(p); }

template <int DT>
__device__ __forceinline__ void decode8(const uint8_t *__restrict__ w, int64_t t, float y[8]) {
  if constexpr (DT == Q8_0 || DT == Q8_1) {
    constexpr int BB = DT == Q8_0 ? 34 : 36, QO = DT == Q8_0 ? 2 : 4;
    const uint8_t *blk = w + (t >> 2) * BB;
    float d = h2f(ld_u16(blk));
    const uint8_t *q = blk + QO + 8 * (t & 3);
#pragma unroll
    for (int i = 0; i < 8; i++) y[i] = __fmul_rn(d, (float)(int8_t)q[i]);
  } else if constexpr (DT == Q4_0 || DT == Q5_0) {
    // Elements 0..15 are the low nibbles of qs, 16..31 the high; Q5_0's fifth bit of
    // element e is bit e of the little-endian u32 qh.
    constexpr int BB = DT == Q4_0 ? 18 : 22, QO = DT == Q4_0 ? 2 : 6, OFF = DT == Q4_0 ? 8 : 16;
    const uint8_t *blk = w + (t >> 2) * BB;
    const float d = h2f(ld_u16(blk));
    const int e0 = 8 * (int)(t & 3), sh = e0 >= 16 ? 4 : 0;
    const uint8_t *q = blk + QO + (e0 & 15);
    uint32_t qh = 0;
    if constexpr (DT == Q5_0) qh = ld_u16(blk + 2) | ld_u16(blk + 4) << 16;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      int v = (q[i] >> sh) & 15;
      if constexpr (DT == Q5_0) v |= (int)((qh >> (e0 + i)) & 1) << 4;
      y[i] = __fmul_rn(d, (float)(v - OFF));
    }
  } else if constexpr (DT == Q5_K) {
    // Q4_K's header and nibbles; bit j of qh[l] is the fifth bit of element 32 j + l.
    const uint8_t *blk = w + (t >> 5) * 176;
    int e0 = 8 * (int)(t & 31), j = e0 >> 5, p = j >> 1, l0 = e0 & 31;
    float d = h2f(ld_u16(blk)), dmin = h2f(ld_u16(blk + 2));
    const uint32_t *sw = reinterpret_cast<const uint32_t *>(blk + 4);
    int sc, m;
    q4k_scale_min(j, sw[0], sw[1], sw[2], sc, m);
    float ds = __fmul_rn(d, (float)sc), dm = __fmul_rn(dmin, (float)m);
    uint2 qv = *reinterpret_cast<const uint2 *>(blk + 48 + 32 * p + l0);
    uint2 hv = *reinterpret_cast<const uint2 *>(blk + 16 + l0);
    int shift = (j & 1) * 4;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      uint32_t word = i < 4 ? qv.x : qv.y, hw = i < 4 ? hv.x : hv.y;
      int q = ((word >> (8 * (i & 3) + shift)) & 15) | (int)((hw >> (8 * (i & 3) + j)) & 1) << 4;
      y[i] = __fsub_rn(__fmul_rn(ds, (float)q), dm);
    }
  } else if constexpr (DT == Q4_K) {
    const uint8_t *blk = w + (t >> 5) * 144;
    int e0 = 8 * (int)(t & 31), j = e0 >> 5, p = j >> 1, l0 = e0 & 31;
    float d = h2f(ld_u16(blk)), dmin = h2f(ld_u16(blk + 2));
    const uint32_t *sw = reinterpret_cast<const uint32_t *>(blk + 4);
    int sc, m;
    q4k_scale_min(j, sw[0], sw[1], sw[2], sc, m);
    float ds = __fmul_rn(d, (float)sc), dm = __fmul_rn(dmin, (float)m);
    uint2 qv = *reinterpret_cast<const uint2 *>(blk + 16 + 32 * p + l0);
    int shift = (j & 1) * 4;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      uint32_t word = i < 4 ? qv.x : qv.y;
      int q = (word >> (8 * (i & 3) + shift)) & 15;
      y[i] = __fsub_rn(__fmul_rn(ds, (float)q), dm);
    }
  } else {  // Q6_K
    const uint8_t *blk = w + (t >> 5) * 210;
    int e0 = 8 * (int)(t & 31), h = e0 >> 7, g = (e0 >> 5) & 3, l0 = e0 & 31;
    const uint8_t *ql = blk + h * 64 + (g & 1) * 32 + l0;
    const uint8_t *qh = blk + 128 + h * 32 + l0;
    float d = h2f(ld_u16(blk + 208));
    float s = __fmul_rn(d, (float)(int8_t)blk[192 + h * 8 + 2 * g + (l0 >> 4)]);
    int nsh = (g >> 1) * 4, hsh = 2 * g;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      int raw = ((ql[i] >> nsh) & 15) | (((qh[i] >> hsh) & 3) << 4);
      y[i] = __fmul_rn(s, (float)(raw - 32));
    }
  }
}

}  // namespace hq
