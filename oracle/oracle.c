/*
 * oracle.c -- CPU restatement of Light's quantized-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for light_amd's HIP kernels and the
 * timed CPU baseline of bench.py.  Never part of the product path.
 *
 * Build (oracle/Makefile): gcc -O2 -mavx2 -mfma -mf16c -ffp-contract=off.
 * -ffp-contract=off matters: Light's decoders multiply then subtract without
 * fusing (VMULPS then VSUBPS, kernels/cpu/qdecode_amd64.s:171-174), while its
 * dot products fuse (VFMADD231PS, internal/simd/simd_amd64.s:21-24).  Every
 * fused multiply-add below is therefore written explicitly.
 */
#include "oracle.h"

#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* ------------------------------------------------------------------ */
/* dtype/half.go                                                       */
/* ------------------------------------------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* Half.ToF32, dtype/half.go:84-113. */
float or_half_to_f32(uint16_t h) {
  uint32_t bits = h, sign = (bits >> 15) & 1, exp = (bits >> 10) & 0x1f, mant = bits & 0x3ff, out;
  switch (exp) {
    case 0:
      if (mant == 0) {
        out = sign << 31;
      } else {
        float v = (float)mant * (1.0f / (float)(1 << 24));
        return sign ? -v : v;
      }
      break;
    case 0x1f:
      out = mant == 0 ? (sign << 31 | 0x7f800000u) : (sign << 31 | 0x7fc00000u);
      break;
    default:
      out = sign << 31 | (exp + 127 - 15) << 23 | mant << 13;
  }
  return u2f(out);
}

/* HalfFromF32, dtype/half.go:15-81 (round to nearest even). */
uint16_t or_half_from_f32(float f) {
  uint32_t bits = f2u(f);
  uint16_t sign = (uint16_t)((bits >> 31) & 1);
  int32_t exp32 = (int32_t)((bits >> 23) & 0xff);
  uint32_t mant32 = bits & 0x7fffff;
  if (exp32 == 0xff) {
    if (mant32 == 0) return (uint16_t)(sign << 15 | 0x7c00);
    return (uint16_t)(sign << 15 | 0x7c00 | ((uint16_t)(mant32 >> 13) | 0x200));
  }
  if (exp32 == 0) return (uint16_t)(sign << 15);
  int32_t real_exp = exp32 - 127;
  if (real_exp > 15) return (uint16_t)(sign << 15 | 0x7c00);
  if (real_exp < -24) return (uint16_t)(sign << 15);
  if (real_exp < -14) {
    uint32_t mant = mant32 | 0x800000;
    uint32_t shift = (uint32_t)(-real_exp - 14 + 13);
    uint32_t h = mant >> shift;
    uint32_t rem = mant & ((1u << shift) - 1);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (h & 1))) h++;
    return (uint16_t)(sign << 15 | (uint16_t)h);
  }
  uint32_t h_exp = (uint32_t)(real_exp + 15), h_mant = mant32 >> 13, rem = mant32 & 0x1fff;
  if (rem > 0x1000 || (rem == 0x1000 && (h_mant & 1))) {
    h_mant++;
    if (h_mant > 0x3ff) {
      h_mant = 0;
      h_exp++;
      if (h_exp >= 31) return (uint16_t)(sign << 15 | 0x7c00);
    }
  }
  return (uint16_t)(sign << 15 | (uint16_t)(h_exp << 10) | (uint16_t)h_mant);
}

/* BF16FromF32, dtype/half.go:118-129 (RNE, quiet NaN kept). */
uint16_t or_bf16_from_f32(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffff)) return (uint16_t)((u >> 16) | 0x0040);
  u += 0x7fff + ((u >> 16) & 1);
  return (uint16_t)(u >> 16);
}

/* f16RowF16C, kernels/cpu/qdecode_amd64.s:317-339 (VCVTPH2PS). */
void or_half_to_f32_avx2(const uint16_t *src, float *dst, int64_t n) {
  for (int64_t i = 0; i + 8 <= n; i += 8)
    _mm256_storeu_ps(dst + i, _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(src + i))));
}

static inline float f16le(const uint8_t *b) { return or_half_to_f32((uint16_t)(b[0] | b[1] << 8)); }

/* ------------------------------------------------------------------ */
/* Block decoders                                                      */
/* ------------------------------------------------------------------ */

/* scaleMinK4, kernels/cpu/quant_matmul.go:92-97 (= quant/q4_k.go:83-89). */
static inline void scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *m) {
  if (j < 4) {
    *sc = q[j] & 63;
    *m = q[j + 4] & 63;
  } else {
    *sc = (uint8_t)((q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4));
    *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
  }
}

/* Q8_0: kernels/cpu/quant_matmul.go:29-34. */
static void dec_q8_0(const uint8_t *b, float *dst) {
  float d = f16le(b);
  for (int i = 0; i < 32; i++) dst[i] = d * (float)(int8_t)b[2 + i];
}

/* Q4_0: kernels/cpu/quant_matmul.go:35-42 (= quant/q4_0.go dequantQ4_0CPU); y = d*(q - 8). */
static void dec_q4_0(const uint8_t *b, float *dst) {
  float d = f16le(b);
  for (int j = 0; j < 16; j++) {
    uint8_t q = b[2 + j];
    dst[j] = d * (float)((int)(q & 15) - 8);
    dst[j + 16] = d * (float)((int)(q >> 4) - 8);
  }
}

/* Q5_0: kernels/cpu/quant_matmul.go:43-53 (= quant/q5_0.go:56-67); fifth bit of element j is
 * bit j of the little-endian u32 qh; y = d*(q5 - 16). */
static void dec_q5_0(const uint8_t *b, float *dst) {
  float d = f16le(b);
  uint32_t qh = (uint32_t)b[2] | (uint32_t)b[3] << 8 | (uint32_t)b[4] << 16 | (uint32_t)b[5] << 24;
  for (int j = 0; j < 16; j++) {
    uint8_t q = b[6 + j];
    int lo = (q & 15) | (int)((qh >> j) & 1) << 4;
    int hi = (q >> 4) | (int)((qh >> (j + 16)) & 1) << 4;
    dst[j] = d * (float)(lo - 16);
    dst[j + 16] = d * (float)(hi - 16);
  }
}

/* Q5_K: quant/q5_k.go:50-83 (DequantQ5_K; Light's CPU matmul_q has no Q5_K decoder):
 * Q4_K's header, qh[32] where bit 2p / 2p+1 of qh[l] is the fifth bit of element
 * p*64+l / p*64+32+l, then Q4_K's qs; y = (d*sc)*q5 - dmin*m, unfused. */
static void dec_q5_k(const uint8_t *b, float *dst) {
  float d = f16le(b), dmin = f16le(b + 2);
  const uint8_t *scales = b + 4, *qh = b + 16, *qs = b + 48;
  for (int p = 0; p < 4; p++) {
    uint8_t sc0, m0, sc1, m1;
    scale_min_k4(2 * p, scales, &sc0, &m0);
    scale_min_k4(2 * p + 1, scales, &sc1, &m1);
    float d1 = d * (float)sc0, mo1 = dmin * (float)m0;
    float d2 = d * (float)sc1, mo2 = dmin * (float)m1;
    for (int l = 0; l < 32; l++) {
      uint8_t q = qs[p * 32 + l];
      int lo = (q & 15) | ((qh[l] >> (2 * p)) & 1) << 4;
      int hi = (q >> 4) | ((qh[l] >> (2 * p + 1)) & 1) << 4;
      float a = d1 * (float)lo;
      float c = d2 * (float)hi;
      dst[p * 64 + l] = a - mo1;
      dst[p * 64 + 32 + l] = c - mo2;
    }
  }
}

/* Q4_K: kernels/cpu/quant_matmul.go:54-68; y = (d*sc)*q - dmin*m, unfused. */
static void dec_q4_k(const uint8_t *b, float *dst) {
  float d = f16le(b), dmin = f16le(b + 2);
  const uint8_t *scales = b + 4, *qs = b + 16;
  for (int p = 0; p < 4; p++) {
    uint8_t sc0, m0, sc1, m1;
    scale_min_k4(2 * p, scales, &sc0, &m0);
    scale_min_k4(2 * p + 1, scales, &sc1, &m1);
    float d1 = d * (float)sc0, mo1 = dmin * (float)m0;
    float d2 = d * (float)sc1, mo2 = dmin * (float)m1;
    for (int l = 0; l < 32; l++) {
      uint8_t q = qs[p * 32 + l];
      float a = d1 * (float)(q & 15);
      float c = d2 * (float)(q >> 4);
      dst[p * 64 + l] = a - mo1;
      dst[p * 64 + 32 + l] = c - mo2;
    }
  }
}

/* Q6_K: kernels/cpu/quant_matmul.go:69-87; y = (d*int8(sc))*q. */
static void dec_q6_k(const uint8_t *b, float *dst) {
  const uint8_t *ql = b, *qh = b + 128, *sc = b + 192;
  float d = f16le(b + 208);
  for (int half = 0; half < 2; half++) {
    int qlB = half * 64, qhB = half * 32, scB = half * 8, y = half * 128;
    for (int l = 0; l < 32; l++) {
      int is = l >> 4;
      uint8_t h = qh[qhB + l];
      int q1 = ((ql[qlB + l] & 15) | (h & 3) << 4) - 32;
      int q2 = ((ql[qlB + l + 32] & 15) | ((h >> 2) & 3) << 4) - 32;
      int q3 = ((ql[qlB + l] >> 4) | ((h >> 4) & 3) << 4) - 32;
      int q4 = ((ql[qlB + l + 32] >> 4) | ((h >> 6) & 3) << 4) - 32;
      float s1 = d * (float)(int8_t)sc[scB + is], s2 = d * (float)(int8_t)sc[scB + 2 + is];
      float s3 = d * (float)(int8_t)sc[scB + 4 + is], s4 = d * (float)(int8_t)sc[scB + 6 + is];
      dst[y + l] = s1 * (float)q1;
      dst[y + l + 32] = s2 * (float)q2;
      dst[y + l + 64] = s3 * (float)q3;
      dst[y + l + 96] = s4 * (float)q4;
    }
  }
}

/* Q8_1 dequant: quant/q8_1.go:21-57 (y = d*q, the s field ignored). */
static void dec_q8_1(const uint8_t *b, float *dst) {
  float d = f16le(b);
  for (int i = 0; i < 32; i++) dst[i] = d * (float)(int8_t)b[4 + i];
}

static int block_info(int dt, int *elems, int *bytes) {
  switch (dt) {
    case OR_Q4_0: *elems = 32; *bytes = 18; return 0;
    case OR_Q5_0: *elems = 32; *bytes = 22; return 0;
    case OR_Q8_0: *elems = 32; *bytes = 34; return 0;
    case OR_Q8_1: *elems = 32; *bytes = 36; return 0;
    case OR_Q4_K: *elems = 256; *bytes = 144; return 0;
    case OR_Q5_K: *elems = 256; *bytes = 176; return 0;
    case OR_Q6_K: *elems = 256; *bytes = 210; return 0;
  }
  return -1;
}

int or_decode_row(int dt, const uint8_t *raw, int64_t K, float *dst) {
  int be, bb;
  if (block_info(dt, &be, &bb) || K % be) return -1;
  for (int64_t b = 0; b < K / be; b++) {
    const uint8_t *blk = raw + b * bb;
    float *o = dst + b * be;
    switch (dt) {
      case OR_Q4_0: dec_q4_0(blk, o); break;
      case OR_Q5_0: dec_q5_0(blk, o); break;
      case OR_Q5_K: dec_q5_k(blk, o); break;
      case OR_Q8_0: dec_q8_0(blk, o); break;
      case OR_Q8_1: dec_q8_1(blk, o); break;
      case OR_Q4_K: dec_q4_k(blk, o); break;
      case OR_Q6_K: dec_q6_k(blk, o); break;
    }
  }
  return 0;
}

/* AVX2 decoders: q8_0RowAVX2 (qdecode_amd64.s:34-66), q4KBlockAVX2 (:165-204),
 * q6KBlockAVX2 (:206-246), with the per-block scales pre-formed as in
 * decodeRowAVX2 (kernels/cpu/quant_matmul.go:208-250). */
int or_decode_row_avx2(int dt, const uint8_t *raw, int64_t K, float *dst) {
  if (dt == OR_Q8_0) {
    if (K % 32) return -1;
    for (int64_t b = 0; b < K / 32; b++) {
      const uint8_t *s = raw + b * 34;
      __m256 d = _mm256_set1_ps(f16le(s));
      for (int c = 0; c < 4; c++) {
        __m256i v = _mm256_cvtepi8_epi32(_mm_loadl_epi64((const __m128i *)(s + 2 + 8 * c)));
        _mm256_storeu_ps(dst + b * 32 + 8 * c, _mm256_mul_ps(d, _mm256_cvtepi32_ps(v)));
      }
    }
    return 0;
  }
  if (dt == OR_Q4_0 || dt == OR_Q5_0) {
    /* q4_0RowAVX2 / q5_0RowAVX2 (qdecode_amd64.s:68-158): per 8-element half, the low and
     * high nibbles (plus the qh bit for Q5_0) minus the offset, converted, times d. */
    if (K % 32) return -1;
    const int q5 = dt == OR_Q5_0, bb = q5 ? 22 : 18, qo = q5 ? 6 : 2;
    const __m256i m15 = _mm256_set1_epi32(15), one = _mm256_set1_epi32(1);
    const __m256i off = _mm256_set1_epi32(q5 ? 16 : 8), sh0 = _mm256_setr_epi32(0, 1, 2, 3, 4, 5, 6, 7);
    for (int64_t b = 0; b < K / 32; b++) {
      const uint8_t *s = raw + b * bb;
      __m256 d = _mm256_set1_ps(f16le(s));
      uint32_t qhv = q5 ? ((uint32_t)s[2] | (uint32_t)s[3] << 8 | (uint32_t)s[4] << 16 | (uint32_t)s[5] << 24) : 0;
      __m256i qh = _mm256_set1_epi32((int)qhv);
      for (int h = 0; h < 2; h++) {
        __m256i v = _mm256_cvtepu8_epi32(_mm_loadl_epi64((const __m128i *)(s + qo + 8 * h)));
        __m256i lo = _mm256_and_si256(v, m15), hi = _mm256_srli_epi32(v, 4);
        if (q5) {
          __m256i shl = _mm256_add_epi32(sh0, _mm256_set1_epi32(8 * h));
          __m256i shh = _mm256_add_epi32(sh0, _mm256_set1_epi32(16 + 8 * h));
          lo = _mm256_or_si256(lo, _mm256_slli_epi32(_mm256_and_si256(_mm256_srlv_epi32(qh, shl), one), 4));
          hi = _mm256_or_si256(hi, _mm256_slli_epi32(_mm256_and_si256(_mm256_srlv_epi32(qh, shh), one), 4));
        }
        lo = _mm256_sub_epi32(lo, off);
        hi = _mm256_sub_epi32(hi, off);
        _mm256_storeu_ps(dst + b * 32 + 8 * h, _mm256_mul_ps(_mm256_cvtepi32_ps(lo), d));
        _mm256_storeu_ps(dst + b * 32 + 16 + 8 * h, _mm256_mul_ps(_mm256_cvtepi32_ps(hi), d));
      }
    }
    return 0;
  }
  if (dt == OR_Q4_K) {
    if (K % 256) return -1;
    const __m256i m15 = _mm256_set1_epi32(15);
    for (int64_t b = 0; b < K / 256; b++) {
      const uint8_t *blk = raw + b * 144;
      float d = f16le(blk), dmin = f16le(blk + 2), sc[8], mn[8];
      for (int j = 0; j < 8; j++) {
        uint8_t s, m;
        scale_min_k4(j, blk + 4, &s, &m);
        sc[j] = d * (float)s;
        mn[j] = dmin * (float)m;
      }
      const uint8_t *qs = blk + 16;
      float *o = dst + b * 256;
      for (int p = 0; p < 4; p++) {
        __m256 slo = _mm256_set1_ps(sc[2 * p]), mlo = _mm256_set1_ps(mn[2 * p]);
        __m256 shi = _mm256_set1_ps(sc[2 * p + 1]), mhi = _mm256_set1_ps(mn[2 * p + 1]);
        for (int c = 0; c < 4; c++) {
          __m256i v = _mm256_cvtepu8_epi32(_mm_loadl_epi64((const __m128i *)(qs + 32 * p + 8 * c)));
          __m256 lo = _mm256_cvtepi32_ps(_mm256_and_si256(v, m15));
          __m256 hi = _mm256_cvtepi32_ps(_mm256_srli_epi32(v, 4));
          _mm256_storeu_ps(o + 64 * p + 8 * c, _mm256_sub_ps(_mm256_mul_ps(lo, slo), mlo));
          _mm256_storeu_ps(o + 64 * p + 32 + 8 * c, _mm256_sub_ps(_mm256_mul_ps(hi, shi), mhi));
        }
      }
    }
    return 0;
  }
  if (dt == OR_Q6_K) {
    if (K % 256) return -1;
    const __m256i m15 = _mm256_set1_epi32(15), m3 = _mm256_set1_epi32(3), c32 = _mm256_set1_epi32(32);
    for (int64_t b = 0; b < K / 256; b++) {
      const uint8_t *blk = raw + b * 210;
      float d = f16le(blk + 208), sc[16];
      for (int j = 0; j < 16; j++) sc[j] = d * (float)(int8_t)blk[192 + j];
      float *o = dst + b * 256;
      for (int half = 0; half < 2; half++) {
        const uint8_t *ql = blk + 64 * half, *qh = blk + 128 + 32 * half;
        const float *s = sc + 8 * half;
        for (int c = 0; c < 4; c++) {
          int l0 = 8 * c, is = l0 >> 4;
          __m256i a = _mm256_cvtepu8_epi32(_mm_loadl_epi64((const __m128i *)(ql + l0)));
          __m256i bq = _mm256_cvtepu8_epi32(_mm_loadl_epi64((const __m128i *)(ql + l0 + 32)));
          __m256i h = _mm256_cvtepu8_epi32(_mm_loadl_epi64((const __m128i *)(qh + l0)));
          __m256i nib[4] = {_mm256_and_si256(a, m15), _mm256_and_si256(bq, m15), _mm256_srli_epi32(a, 4),
                            _mm256_srli_epi32(bq, 4)};
          for (int g = 0; g < 4; g++) {
            __m256i hb = _mm256_slli_epi32(_mm256_and_si256(_mm256_srli_epi32(h, 2 * g), m3), 4);
            __m256i q = _mm256_sub_epi32(_mm256_or_si256(nib[g], hb), c32);
            __m256 v = _mm256_mul_ps(_mm256_cvtepi32_ps(q), _mm256_set1_ps(s[2 * g + is]));
            _mm256_storeu_ps(o + 128 * half + 32 * g + l0, v);
          }
        }
      }
    }
    return 0;
  }
  return or_decode_row(dt, raw, K, dst);
}

/* int4 canonical row, scalar: kernels/cpu/quant_matmul.go:191-199; s*(q - z). */
void or_int4_row(const uint32_t *codes, const float *s, const float *z, float *dst, int64_t K, int G) {
  for (int64_t g = 0; g < K / G; g++) {
    float sg = s[g], zg = z[g];
    for (int64_t k = g * G; k < (g + 1) * G; k += 8) {
      uint32_t w = codes[k / 8];
      for (int j = 0; j < 8; j++) dst[k + j] = sg * ((float)((w >> (4 * j)) & 15) - zg);
    }
  }
}

/* int4RowAVX2, kernels/cpu/qdecode_amd64.s:251-284: VSUBPS then VMULPS. */
void or_int4_row_avx2(const uint32_t *codes, const float *s, const float *z, float *dst, int64_t K, int G) {
  const __m256i sh = _mm256_setr_epi32(0, 4, 8, 12, 16, 20, 24, 28), m15 = _mm256_set1_epi32(15);
  for (int64_t g = 0; g < K / G; g++) {
    __m256 sg = _mm256_set1_ps(s[g]), zg = _mm256_set1_ps(z[g]);
    for (int64_t k = g * G; k < (g + 1) * G; k += 8) {
      __m256i w = _mm256_set1_epi32((int)codes[k / 8]);
      __m256 q = _mm256_cvtepi32_ps(_mm256_and_si256(_mm256_srlv_epi32(w, sh), m15));
      _mm256_storeu_ps(dst + k, _mm256_mul_ps(sg, _mm256_sub_ps(q, zg)));
    }
  }
}

int or_dequant(int dt, const uint8_t *raw, int64_t n, float *out) { return or_decode_row(dt, raw, n, out); }

/* int4DequantCPU, kernels/cpu/int4.go:19-54: product in F32, rounded once to BF16. */
int or_int4_dequant(const uint32_t *codes, const float *s, const float *z, void *out, int out_dt,
                    int64_t N, int64_t K, int G) {
  if (G <= 0 || K % G || K % 8) return -1;
  int64_t ng = K / G;
  for (int64_t n = 0; n < N; n++) {
    for (int64_t k = 0; k < K; k++) {
      int64_t g = n * ng + k / G;
      float v = s[g] * ((float)((codes[n * (K / 8) + k / 8] >> (4 * (k % 8))) & 0xF) - z[g]);
      if (out_dt == OR_F32)
        ((float *)out)[n * K + k] = v;
      else if (out_dt == OR_BF16)
        ((uint16_t *)out)[n * K + k] = or_bf16_from_f32(v);
      else
        return -1;
    }
  }
  return 0;
}

/* ------------------------------------------------------------------ */
/* internal/simd                                                       */
/* ------------------------------------------------------------------ */

/* HSUM / dotreduce tail: lanes (l0..l7) -> ((l0+l4)+(l1+l5)) + ((l2+l6)+(l3+l7)). */
static inline float hsum256(__m256 v) {
  __m128 x = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
  x = _mm_hadd_ps(x, x);
  x = _mm_hadd_ps(x, x);
  return _mm_cvtss_f32(x);
}

/* dotAVX2, internal/simd/simd_amd64.s:6-58. */
float or_dot_avx2(const float *a, const float *b, int64_t n) {
  __m256 y0 = _mm256_setzero_ps(), y1 = y0, y2 = y0, y3 = y0;
  int64_t i = 0;
  for (; n - i >= 32; i += 32) {
    y0 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), y0);
    y1 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 8), _mm256_loadu_ps(b + i + 8), y1);
    y2 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 16), _mm256_loadu_ps(b + i + 16), y2);
    y3 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 24), _mm256_loadu_ps(b + i + 24), y3);
  }
  for (; n - i >= 8; i += 8) y0 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), y0);
  y0 = _mm256_add_ps(y0, y1);
  y2 = _mm256_add_ps(y2, y3);
  y0 = _mm256_add_ps(y0, y2);
  float r = hsum256(y0);
  for (; i < n; i++) r = fmaf(a[i], b[i], r);
  return r;
}

/* The same order as dotAVX2, written lane by lane with scalar fmaf: an
 * independent encoding used to pin the intrinsics version bit for bit. */
float or_dot_lanes(const float *a, const float *b, int64_t n) {
  float acc[4][8] = {{0}};
  int64_t i = 0;
  for (; n - i >= 32; i += 32)
    for (int r = 0; r < 4; r++)
      for (int l = 0; l < 8; l++) acc[r][l] = fmaf(a[i + 8 * r + l], b[i + 8 * r + l], acc[r][l]);
  for (; n - i >= 8; i += 8)
    for (int l = 0; l < 8; l++) acc[0][l] = fmaf(a[i + l], b[i + l], acc[0][l]);
  float v[8];
  for (int l = 0; l < 8; l++) v[l] = (acc[0][l] + acc[1][l]) + (acc[2][l] + acc[3][l]);
  float x[4];
  for (int l = 0; l < 4; l++) x[l] = v[l] + v[l + 4];
  float r = (x[0] + x[1]) + (x[2] + x[3]);
  for (; i < n; i++) r = fmaf(a[i], b[i], r);
  return r;
}

/* dot4x3AVX2, internal/simd/simd_amd64.s:143-205: 12 accumulators, k step 8, HSUM each. */
void or_dot4x3_avx2(const float *a, int64_t lda, const float *w, int64_t ldw, int64_t k, float *out) {
  __m256 acc[12];
  for (int i = 0; i < 12; i++) acc[i] = _mm256_setzero_ps();
  for (int64_t t = 0; t < k; t += 8) {
    __m256 w0 = _mm256_loadu_ps(w + t), w1 = _mm256_loadu_ps(w + ldw + t), w2 = _mm256_loadu_ps(w + 2 * ldw + t);
    for (int r = 0; r < 4; r++) {
      __m256 av = _mm256_loadu_ps(a + r * lda + t);
      acc[3 * r] = _mm256_fmadd_ps(w0, av, acc[3 * r]);
      acc[3 * r + 1] = _mm256_fmadd_ps(w1, av, acc[3 * r + 1]);
      acc[3 * r + 2] = _mm256_fmadd_ps(w2, av, acc[3 * r + 2]);
    }
  }
  for (int i = 0; i < 12; i++) out[i] = hsum256(acc[i]);
}

/* simd.MatTB, internal/simd/simd.go:63-90 (AVX2 branch). */
void or_mattb(const float *a, int64_t lda, const float *w, int64_t ldw, float *out, int64_t ldo, int64_t m,
              int64_t n, int64_t k) {
  int64_t i = 0;
  if (k % 8 == 0 && k > 0) {
    float t[12];
    for (; i + 4 <= m; i += 4) {
      int64_t j = 0;
      for (; j + 3 <= n; j += 3) {
        or_dot4x3_avx2(a + i * lda, lda, w + j * ldw, ldw, k, t);
        for (int r = 0; r < 4; r++) {
          float *o = out + (i + r) * ldo + j;
          o[0] = t[3 * r];
          o[1] = t[3 * r + 1];
          o[2] = t[3 * r + 2];
        }
      }
      for (; j < n; j++)
        for (int r = 0; r < 4; r++) out[(i + r) * ldo + j] = or_dot_avx2(a + (i + r) * lda, w + j * ldw, k);
    }
  }
  for (; i < m; i++)
    for (int64_t j = 0; j < n; j++) out[i * ldo + j] = or_dot_avx2(a + i * lda, w + j * ldw, k);
}

/* ------------------------------------------------------------------ */
/* internal/parallel                                                   */
/* ------------------------------------------------------------------ */

int or_hw_threads(void) {
  long n = sysconf(_SC_NPROCESSORS_ONLN);
  return n > 0 ? (int)n : 1;
}

typedef void (*range_fn)(void *ctx, int64_t lo, int64_t hi);
typedef struct {
  range_fn fn;
  void *ctx;
  int64_t lo, hi;
} par_task;

static void *par_run(void *p) {
  par_task *t = (par_task *)p;
  t->fn(t->ctx, t->lo, t->hi);
  return NULL;
}

/* parallel.For, internal/parallel/parallel.go:11-37: contiguous chunks of
 * ceil(n / workers), workers = min(threads, n / grain). */
static void par_for(int64_t n, int64_t grain, int threads, range_fn fn, void *ctx) {
  if (n <= 0) return;
  int64_t workers = threads > 0 ? threads : or_hw_threads();
  if (grain < 1) grain = 1;
  if (n / grain < workers) workers = n / grain;
  if (workers <= 1) {
    fn(ctx, 0, n);
    return;
  }
  int64_t chunk = (n + workers - 1) / workers;
  int64_t nt = (n + chunk - 1) / chunk;
  pthread_t *th = (pthread_t *)malloc(sizeof(pthread_t) * nt);
  par_task *tk = (par_task *)malloc(sizeof(par_task) * nt);
  int64_t c = 0;
  for (int64_t lo = 0; lo < n; lo += chunk, c++) {
    tk[c].fn = fn;
    tk[c].ctx = ctx;
    tk[c].lo = lo;
    tk[c].hi = lo + chunk < n ? lo + chunk : n;
    if (pthread_create(&th[c], NULL, par_run, &tk[c])) par_run(&tk[c]), th[c] = 0;
  }
  for (int64_t i = 0; i < c; i++)
    if (th[i]) pthread_join(th[i], NULL);
  free(th);
  free(tk);
}

/* ------------------------------------------------------------------ */
/* rowsTimesX + matmulQCPU / int4MatMulCPU                             */
/* ------------------------------------------------------------------ */

enum { TILE_ROWS = 48 }; /* kernels/cpu/matmul_f32.go:9 */

typedef void (*decode_fn)(void *ctx, int64_t n, float *dst);
typedef struct {
  const float *x;
  float *out;
  int64_t M, K, N;
  decode_fn dec;
  void *dctx;
} rtx_ctx;

static void rtx_range(void *p, int64_t lo, int64_t hi) {
  rtx_ctx *c = (rtx_ctx *)p;
  float *rows = (float *)malloc(sizeof(float) * TILE_ROWS * c->K);
  for (int64_t n0 = lo; n0 < hi; n0 += TILE_ROWS) {
    int64_t n1 = n0 + TILE_ROWS < hi ? n0 + TILE_ROWS : hi;
    for (int64_t n = n0; n < n1; n++) c->dec(c->dctx, n, rows + (n - n0) * c->K);
    or_mattb(c->x, c->K, rows, c->K, c->out + n0, c->N, c->M, n1 - n0, c->K);
  }
  free(rows);
}

/* rowsTimesX, kernels/cpu/quant_matmul.go:123-137. */
static void rows_times_x(const float *x, float *out, int64_t M, int64_t K, int64_t N, decode_fn dec, void *dctx,
                         int threads) {
  rtx_ctx c = {x, out, M, K, N, dec, dctx};
  int64_t grain = 16384 / (K + 1);
  par_for(N, grain < 1 ? 1 : grain, threads, rtx_range, &c);
}

typedef struct {
  const uint8_t *w;
  int64_t row_bytes, K;
  int dt;
} gguf_dctx;

static void gguf_decode(void *p, int64_t n, float *dst) {
  gguf_dctx *c = (gguf_dctx *)p;
  or_decode_row_avx2(c->dt, c->w + n * c->row_bytes, c->K, dst);
}

/* matmulF32Fast's x * W^T case, kernels/cpu/matmul_f32.go:30-48: parallel over output
 * columns with grain max(1, 32768 / (K*M + 1)), MatTB over tiles of 48 weight rows. */
typedef struct {
  const float *x, *w;
  float *out;
  int64_t M, K, N;
} mmt_ctx;

static void mmt_range(void *p, int64_t lo, int64_t hi) {
  mmt_ctx *c = (mmt_ctx *)p;
  for (int64_t j0 = lo; j0 < hi; j0 += TILE_ROWS) {
    int64_t j1 = j0 + TILE_ROWS < hi ? j0 + TILE_ROWS : hi;
    or_mattb(c->x, c->K, c->w + j0 * c->K, c->K, c->out + j0, c->N, c->M, j1 - j0, c->K);
  }
}

int or_matmul_q(const float *x, const uint8_t *w, float *out, int64_t M, int64_t N, int64_t K, int dt,
                int threads) {
  int be, bb;
  if (block_info(dt, &be, &bb) || dt == OR_Q8_1 || K % be) return -1;
  if (dt == OR_Q5_K) {
    /* No CPU matmul_q kernel for Q5_K: ops.MatMulQ falls back to quant.Dequantize + MatMul
     * (ops/matmul_q.go:60-66, 85-95). */
    float *wf = (float *)malloc(sizeof(float) * (size_t)(N * K));
    if (!wf) return -2;
    or_dequant(dt, w, N * K, wf);
    mmt_ctx c = {x, wf, out, M, K, N};
    int64_t grain = 32768 / (K * M + 1);
    par_for(N, grain < 1 ? 1 : grain, threads, mmt_range, &c);
    free(wf);
    return 0;
  }
  gguf_dctx d = {w, K / be * bb, K, dt};
  rows_times_x(x, out, M, K, N, gguf_decode, &d, threads);
  return 0;
}

typedef struct {
  const uint32_t *codes;
  const float *s, *z;
  int64_t K;
  int G;
} int4_dctx;

static void int4_decode(void *p, int64_t n, float *dst) {
  int4_dctx *c = (int4_dctx *)p;
  int64_t ng = c->K / c->G;
  if (c->G % 8 == 0)
    or_int4_row_avx2(c->codes + n * (c->K / 8), c->s + n * ng, c->z + n * ng, dst, c->K, c->G);
  else
    or_int4_row(c->codes + n * (c->K / 8), c->s + n * ng, c->z + n * ng, dst, c->K, c->G);
}

int or_int4_matmul(const float *x, const uint32_t *codes, const float *s, const float *z, float *out,
                   int64_t M, int64_t N, int64_t K, int G, int threads) {
  if (G <= 0 || K % G || K % 8) return -1;
  int4_dctx d = {codes, s, z, K, G};
  rows_times_x(x, out, M, K, N, int4_decode, &d, threads);
  return 0;
}

/* ------------------------------------------------------------------ */
/* MoE                                                                 */
/* ------------------------------------------------------------------ */

/* Stable ascending sort of the flat expert ids: Sort(flat, false) on the CPU
 * is sort.SliceStable (kernels/cpu/shape_ops.go:156-184).  Counting sort is
 * stable and gives the same (value, index) pairs. */
void or_moe_route_from_ids(const int64_t *ids, int64_t M, int64_t *sorted_expts, int64_t *sorted_pairs) {
  int64_t maxe = -1;
  for (int64_t i = 0; i < M; i++)
    if (ids[i] > maxe) maxe = ids[i];
  int64_t *cnt = (int64_t *)calloc((size_t)(maxe + 2), sizeof(int64_t));
  for (int64_t i = 0; i < M; i++) cnt[ids[i] + 1]++;
  for (int64_t e = 0; e <= maxe; e++) cnt[e + 1] += cnt[e];
  for (int64_t i = 0; i < M; i++) {
    int64_t pos = cnt[ids[i]]++;
    sorted_expts[pos] = ids[i];
    sorted_pairs[pos] = i;
  }
  free(cnt);
}

/* MoERoute, ops/moe.go:29-71, on the CPU: TopK(probs, k, largest) -- a stable descending
 * sort of each row (kernels/cpu/topk.go:52-68; an insertion sort is stable) -- then, with
 * normalize, den = Sum over the k values from 0 left to right (kernels/cpu/reduce.go:76-87)
 * and vals / den; then Sort(flat ids) ascending, stable (or_moe_route_from_ids). */
void or_moe_route(const float *probs, int64_t T, int64_t E, int topk, int normalize, int64_t *topk_ids,
                  float *weights, int64_t *sorted_pairs, int64_t *sorted_expts) {
  int64_t *ord = (int64_t *)malloc(sizeof(int64_t) * (size_t)E);
  for (int64_t t = 0; t < T; t++) {
    const float *row = probs + t * E;
    for (int64_t j = 0; j < E; j++) {
      int64_t i = j;
      while (i > 0 && row[j] > row[ord[i - 1]]) {
        ord[i] = ord[i - 1];
        i--;
      }
      ord[i] = j;
    }
    float den = 0.0f;
    for (int s = 0; s < topk; s++) den += row[ord[s]];
    for (int s = 0; s < topk; s++) {
      topk_ids[t * topk + s] = ord[s];
      weights[t * topk + s] = normalize ? row[ord[s]] / den : row[ord[s]];
    }
  }
  free(ord);
  or_moe_route_from_ids(topk_ids, T * topk, sorted_expts, sorted_pairs);
}

typedef struct {
  const float *x, *w, *topk_w;
  const int64_t *pairs, *expts;
  float *out;
  int64_t size_m, N, K;
  int topk, row_per_pair;
} moe_ctx;

static void moe_range(void *p, int64_t lo, int64_t hi) {
  moe_ctx *c = (moe_ctx *)p;
  for (int64_t idx = lo; idx < hi; idx++) {
    int64_t i = idx / c->N, n = idx % c->N, pr = c->pairs[i];
    if (pr < 0 || pr >= c->size_m) continue;
    int64_t r = c->row_per_pair ? pr : pr / c->topk, e = c->expts[i];
    float acc = or_dot_avx2(c->x + r * c->K, c->w + (e * c->N + n) * c->K, c->K);
    if (c->topk_w) acc *= c->topk_w[pr];
    c->out[pr * c->N + n] = acc;
  }
}

int or_moe_gemm_f32(const float *x, const float *w, const int64_t *pairs, const int64_t *expts,
                    const float *topk_w, float *out, int64_t M, int64_t size_m, int64_t N, int64_t K,
                    int topk, int row_per_pair, int threads) {
  moe_ctx c = {x, w, topk_w, pairs, expts, out, size_m, N, K, topk, row_per_pair};
  int64_t grain = 16384 / (K + 1);
  par_for(M * N, grain < 1 ? 1 : grain, threads, moe_range, &c);
  return 0;
}

int or_moe_gemm_q(const float *x, const uint8_t *w, int dt, const int64_t *pairs, const int64_t *expts,
                  const float *topk_w, float *out, int64_t M, int64_t size_m, int64_t E, int64_t N,
                  int64_t K, int topk, int row_per_pair, int threads, float *w_scratch) {
  int be, bb;
  if (block_info(dt, &be, &bb) || K % be) return -1;
  float *wf = w_scratch ? w_scratch : (float *)malloc(sizeof(float) * (size_t)(E * N * K));
  if (!wf) return -2;
  or_dequant(dt, w, E * N * K, wf);
  memset(out, 0, sizeof(float) * (size_t)(size_m * N));
  or_moe_gemm_f32(x, wf, pairs, expts, topk_w, out, M, size_m, N, K, topk, row_per_pair, threads);
  if (!w_scratch) free(wf);
  return 0;
}

/* MoECombine, ops/moe.go:209-240: acc = slot0; acc = acc + slot_s for s = 1.. */
void or_moe_combine(const float *pair_out, float *out, int64_t M, int64_t N, int topk) {
  for (int64_t t = 0; t < M / topk; t++)
    for (int64_t n = 0; n < N; n++) {
      float acc = pair_out[(t * topk) * N + n];
      for (int s = 1; s < topk; s++) acc = acc + pair_out[(t * topk + s) * N + n];
      out[t * N + n] = acc;
    }
}

/* The unfused gated MLP tail: SiLU (kernels/cpu/unary.go:219-222, f32: a / (1 + f32(exp(f64(-a)))))
 * or GeluErf (:216, :263-265, f64 0.5 x (1 + erf(x / sqrt 2)) rounded to f32), then Mul (f32). */
void or_gated(const float *g, const float *u, float *out, int64_t n, int act) {
  for (int64_t i = 0; i < n; i++) {
    const float a = g[i];
    float h;
    if (act == 1)
      h = (float)(0.5 * (double)a * (1.0 + erf((double)a / sqrt(2.0))));
    else
      h = a / (1.0f + (float)exp(-(double)a));
    out[i] = h * u[i];
  }
}

/* ------------------------------------------------------------------ */
/* Quantizers                                                          */
/* ------------------------------------------------------------------ */

static void put16(uint8_t *p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }

/* encodeQ8_0, quant/quantize.go:70-86. */
void or_quantize_q8_0(const float *x, int64_t n, uint8_t *dst) {
  for (int64_t b = 0; b < n / 32; b++) {
    const float *v = x + 32 * b;
    uint8_t *o = dst + 34 * b;
    float amax = 0;
    for (int i = 0; i < 32; i++) {
      float a = fabsf(v[i]);
      if (a > amax) amax = a;
    }
    float d = amax / 127.0f, id = d != 0 ? 1.0f / d : 0.0f;
    put16(o, or_half_from_f32(d));
    for (int i = 0; i < 32; i++) {
      float p = v[i] * id;
      o[2 + i] = (uint8_t)(int8_t)nearbyint((double)p);
    }
  }
}

/* q8_1 activation quantizer.  Light has no q8_1 encoder; the layout is
 * quant/q8_1.go:10-18 ([f16 d][f16 s][i8 q[32]]), the rounding is
 * encodeQ8_0's (quant/quantize.go:77-85: d = amax/127, id = 1/d from the
 * unrounded f32 d, q = RoundToEven(v*id)), and s = f16(f32(sum q) * d). */
void or_quantize_q8_1(const float *x, int64_t n, uint8_t *dst) {
  for (int64_t b = 0; b < n / 32; b++) {
    const float *v = x + 32 * b;
    uint8_t *o = dst + 36 * b;
    float amax = 0;
    for (int i = 0; i < 32; i++) {
      float a = fabsf(v[i]);
      if (a > amax) amax = a;
    }
    float d = amax / 127.0f, id = d != 0 ? 1.0f / d : 0.0f;
    int sum = 0;
    for (int i = 0; i < 32; i++) {
      float p = v[i] * id;
      int q = (int)nearbyint((double)p);
      o[4 + i] = (uint8_t)(int8_t)q;
      sum += q;
    }
    put16(o, or_half_from_f32(d));
    put16(o + 2, or_half_from_f32((float)sum * d));
  }
}

/* ------------------------------------------------------------------ */
/* f64 dequant-then-matmul oracle                                      */
/* ------------------------------------------------------------------ */

typedef struct {
  const float *x, *w;
  int64_t M, N, K;
  double *ref, *mag, *wnorm;
} f64_ctx;

static void f64_range(void *p, int64_t lo, int64_t hi) {
  f64_ctx *c = (f64_ctx *)p;
  for (int64_t n = lo; n < hi; n++) {
    const float *wr = c->w + n * c->K;
    if (c->wnorm) {
      double s = 0;
      for (int64_t k = 0; k < c->K; k++) s += (double)wr[k] * wr[k];
      c->wnorm[n] = sqrt(s);
    }
    for (int64_t m = 0; m < c->M; m++) {
      const float *xr = c->x + m * c->K;
      double acc = 0, mg = 0;
      for (int64_t k = 0; k < c->K; k++) {
        double t = (double)xr[k] * (double)wr[k];
        acc += t;
        mg += fabs(t);
      }
      if (c->ref) c->ref[m * c->N + n] = acc;
      if (c->mag) c->mag[m * c->N + n] = mg;
    }
  }
}

void or_matmul_f64(const float *x, const float *w, int64_t M, int64_t N, int64_t K, double *ref,
                   double *mag, double *wnorm, double *xnorm, int threads) {
  f64_ctx c = {x, w, M, N, K, ref, mag, wnorm};
  par_for(N, 1, threads, f64_range, &c);
  if (xnorm)
    for (int64_t m = 0; m < M; m++) {
      double s = 0;
      for (int64_t k = 0; k < K; k++) s += (double)x[m * K + k] * x[m * K + k];
      xnorm[m] = sqrt(s);
    }
}
