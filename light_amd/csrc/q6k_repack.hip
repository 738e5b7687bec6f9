// q6k_repack.hip -- the Q6_K_R layout: a load-time, value-preserving repack of Q6_K weights.
//
// Q6_K blocks (quant/q6_k.go:10-27) are 210 bytes, so a block starts on a 2-byte boundary and
// its 6-bit quants are split over ql (low nibbles) and qh (2-bit highs of four groups per
// byte).  The decode GEMV wants each lane's 64 weights in aligned 16-byte loads that a wave
// issues as contiguous 1 KB requests.  Q6_K_R stores, per row (K = 256 nb, P = 4 nb units):
//
//   [0, 16 P)        plane 0: unit u's quant bytes 0..15
//   [16 P, 32 P)     plane 1: unit u's quant bytes 16..31
//   [32 P, 48 P)     plane 2: unit u's 16 bytes of 2-bit highs
//   [48 P, 52 P)     unit u's four int8 scales
//   [52 P, 52 P + 2 nb)  the f16 d of each block, then zero padding to a multiple of 16 bytes
//
// Unit u = 4 b + v of block b covers group g = v % 2 (weights "A") and group g + 2 ("B") of
// half h = v / 2: element h*128 + g*32 + i is A[i], element h*128 + (g+2)*32 + i is B[i].
// Both share quant byte ql[64 h + 32 g + i] (A the low nibble, B the high one) and the qh byte
// qh[32 h + i] (A bits 2g..2g+1, B bits 2g+4..2g+5).  High dword m, byte t holds, from bit 0
// up, the 2-bit highs of A[8m+t], A[8m+4+t], B[8m+t], B[8m+4+t], so that quant dword k (four
// weights) gets its highs from dword k/2 with one shift and mask per group.  Scales are
// A's two sub-blocks (scales[8h+2g], [8h+2g+1]) then B's ([8h+2g+4], [8h+2g+5]).
//
// Bytes per row: 210 nb rounded up to 16 -- the same HBM traffic as GGUF, all of it aligned.
#include "internal.hpp"

namespace hq {

namespace {

struct Q6Src {
  const uint8_t *w;
  uint8_t *dst;
  int64_t N;
  int K, nb, P;
  int64_t row_bytes;  // Q6_K_R row bytes
};

// One thread per (row, unit): gathers the unit's bytes from the GGUF block and writes its
// four pieces; unit 0 of each pair of blocks also writes their two d's, and unit 0 of a row
// the row's zero padding.
__global__ __launch_bounds__(256) void repack_q6k_kernel(Q6Src a) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= a.N * a.P) return;
  const int64_t row = t / a.P;
  const int u = (int)(t - row * a.P), b = u >> 2, v = u & 3, h = v >> 1, g = v & 1;
  const uint8_t *blk = a.w + (row * a.nb + b) * 210;
  uint8_t *o = a.dst + row * a.row_bytes;
  const uint8_t *ql = blk + 64 * h + 32 * g, *qh = blk + 128 + 32 * h;
  uint8_t q[32], hi[16];
#pragma unroll
  for (int i = 0; i < 32; i++) q[i] = ql[i];
#pragma unroll
  for (int m = 0; m < 4; m++)
#pragma unroll
    for (int tt = 0; tt < 4; tt++) {
      const uint32_t e0 = qh[8 * m + tt], e1 = qh[8 * m + 4 + tt];
      hi[4 * m + tt] = (uint8_t)(((e0 >> (2 * g)) & 3) | (((e1 >> (2 * g)) & 3) << 2) |
                                 (((e0 >> (2 * g + 4)) & 3) << 4) | (((e1 >> (2 * g + 4)) & 3) << 6));
    }
  uint32_t w4[12];
#pragma unroll
  for (int k = 0; k < 8; k++)
    w4[k] = q[4 * k] | (uint32_t)q[4 * k + 1] << 8 | (uint32_t)q[4 * k + 2] << 16 | (uint32_t)q[4 * k + 3] << 24;
#pragma unroll
  for (int k = 0; k < 4; k++)
    w4[8 + k] = hi[4 * k] | (uint32_t)hi[4 * k + 1] << 8 | (uint32_t)hi[4 * k + 2] << 16 | (uint32_t)hi[4 * k + 3] << 24;
  const int64_t P16 = 16 * (int64_t)a.P;
  *reinterpret_cast<uint4 *>(o + 16 * u) = make_uint4(w4[0], w4[1], w4[2], w4[3]);
  *reinterpret_cast<uint4 *>(o + P16 + 16 * u) = make_uint4(w4[4], w4[5], w4[6], w4[7]);
  *reinterpret_cast<uint4 *>(o + 2 * P16 + 16 * u) = make_uint4(w4[8], w4[9], w4[10], w4[11]);
  const uint8_t *sc = blk + 192 + 8 * h + 2 * g;
  *reinterpret_cast<uint32_t *>(o + 3 * P16 + 4 * u) =
      sc[0] | (uint32_t)sc[1] << 8 | (uint32_t)sc[4] << 16 | (uint32_t)sc[5] << 24;
  if (v == 0) {
    uint8_t *dd = o + 52 * (int64_t)a.P + 2 * b;
    dd[0] = blk[208];
    dd[1] = blk[209];
  }
  if (u == 0)
    for (int64_t i = 52 * (int64_t)a.P + 2 * a.nb; i < a.row_bytes; i++) o[i] = 0;
}

// One thread per (row, unit): the unit's 64 outputs, with the GGUF decoder's arithmetic
// (s = d * sc rounded, then s * (raw - 32)).
template <int ODT>
__global__ __launch_bounds__(256) void dequant_q6kr_kernel(Q6Src a, void *out) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= a.N * a.P) return;
  const int64_t row = t / a.P;
  const int u = (int)(t - row * a.P), b = u >> 2, v = u & 3, h = v >> 1, g = v & 1;
  const uint8_t *o = a.w + row * a.row_bytes;
  const int64_t P16 = 16 * (int64_t)a.P;
  const uint4 q0 = *reinterpret_cast<const uint4 *>(o + 16 * u);
  const uint4 q1 = *reinterpret_cast<const uint4 *>(o + P16 + 16 * u);
  const uint4 hh = *reinterpret_cast<const uint4 *>(o + 2 * P16 + 16 * u);
  const uint32_t sc = *reinterpret_cast<const uint32_t *>(o + 3 * P16 + 4 * u);
  const float d = h2f(*reinterpret_cast<const uint16_t *>(o + 52 * (int64_t)a.P + 2 * b));
  const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
  const uint32_t hw[4] = {hh.x, hh.y, hh.z, hh.w};
  float s[4];
#pragma unroll
  for (int j = 0; j < 4; j++) s[j] = __fmul_rn(d, (float)(int8_t)(sc >> (8 * j)));
  const int64_t base = row * a.K + 256 * (int64_t)b + 128 * h + 32 * g;
#pragma unroll
  for (int side = 0; side < 2; side++) {  // A = group g, B = group g + 2 (64 elements on)
    float y[32];
#pragma unroll
    for (int i = 0; i < 32; i++) {
      const int k = i >> 2, tt = i & 3, m = k >> 1;
      const uint32_t nib = (qw[k] >> (8 * tt + 4 * side)) & 15u;
      const uint32_t hi2 = (hw[m] >> (8 * tt + 2 * (k & 1) + 4 * side)) & 3u;
      y[i] = __fmul_rn(s[2 * side + (i >> 4)], (float)((int)(nib | hi2 << 4) - 32));
    }
    const int64_t e0 = base + 64 * side;
    if constexpr (ODT == F32) {
      float4 *op = reinterpret_cast<float4 *>(static_cast<float *>(out) + e0);
#pragma unroll
      for (int k = 0; k < 8; k++) op[k] = make_float4(y[4 * k], y[4 * k + 1], y[4 * k + 2], y[4 * k + 3]);
    } else {
      uint4 *op = reinterpret_cast<uint4 *>(static_cast<uint16_t *>(out) + e0);
#pragma unroll
      for (int k = 0; k < 4; k++) {
        uint32_t p[4];
#pragma unroll
        for (int j = 0; j < 4; j++) p[j] = f2bf_rne(y[8 * k + 2 * j]) | (uint32_t)f2bf_rne(y[8 * k + 2 * j + 1]) << 16;
        op[k] = make_uint4(p[0], p[1], p[2], p[3]);
      }
    }
  }
}

Q6Src q6src(const void *w, void *dst, int64_t N, int64_t K) {
  Q6Src a;
  a.w = static_cast<const uint8_t *>(w);
  a.dst = static_cast<uint8_t *>(dst);
  a.N = N;
  a.K = (int)K;
  a.nb = (int)(K / 256);
  a.P = (int)(K / 64);
  a.row_bytes = q6kr_row_bytes(K);
  return a;
}

}  // namespace

int launch_repack_q6k(const void *src, void *dst, int64_t N, int64_t K, hipStream_t s) {
  const Q6Src a = q6src(src, dst, N, K);
  repack_q6k_kernel<<<dim3((unsigned)cdiv(N * a.P, 256)), 256, 0, s>>>(a);
  return check_launch("repack_q6k");
}

int launch_dequant_q6kr(const void *src, void *dst, int64_t N, int64_t K, int out_dtype, hipStream_t s) {
  const Q6Src a = q6src(src, nullptr, N, K);
  const dim3 grid((unsigned)cdiv(N * a.P, 256));
  if (out_dtype == F32)
    dequant_q6kr_kernel<F32><<<grid, 256, 0, s>>>(a, dst);
  else
    dequant_q6kr_kernel<BF16><<<grid, 256, 0, s>>>(a, dst);
  return check_launch("dequant_q6kr");
}

}  // namespace hq
