// int4_convert.hip -- GPTQ / AWQ checkpoint tensors -> Light's canonical 4-bit layout
// (quant.Int4: codes U32 (N, K/8), nibble j of codes[n][c] is W[n][8c + j]; scales / zeros F32
// (N, K/G)), on the device, once at load.
//
// Role: quant.FromGPTQ / quant.FromAWQ (quant/int4.go:102-235), which convert on the host;
// here the checkpoint tensors go to HBM as they are stored and are converted there.
//
//  * GPTQ ("gptq" / "gptq_v2"): qweight I32 (K/8, N), nibble j of qweight[r][n] is input row
//    8r + j; qzeros I32 (K/G, N/8), nibble j of qzeros[g][c] is column 8c + j and holds
//    zero - 1 ("gptq") or the zero ("gptq_v2"); scales (K/G, N).  Without act order the
//    canonical word (n, c) is qweight[c][n] itself, so the codes are a 32-bit transpose
//    (32 x 32-word LDS tiles, coalesced on both sides).  With act order, canonical column k
//    takes input row perm[k] (the host sorts K by g_idx, as Light does), one nibble gather per
//    code.
//  * AWQ (AutoAWQ GEMM): qweight I32 (K, N/8) and qzeros I32 (K/G, N/8), both packed along N
//    with nibble i of a word holding column 8c + (0, 2, 4, 6, 1, 3, 5, 7)[i]; scales (K/G, N).
//
// Bound: HBM, 4 bytes read and written per 8 codes; a load-time step, not a hot path.
#include "internal.hpp"

namespace hq {

namespace {

__device__ __forceinline__ uint32_t nib(uint32_t w, int j) { return (w >> (4 * j)) & 0xFu; }

// AutoAWQ's packing: column offset o within a word sits at nibble kAwqInv[o].
__device__ __forceinline__ int awq_inv(int o) { return (0x73625140 >> (4 * o)) & 0xF; }

// codes[n][c] = qweight[c][n] over a (Kw = K/8) x N word matrix.
__global__ __launch_bounds__(256) void gptq_codes_kernel(const uint32_t *__restrict__ qw, uint32_t *__restrict__ codes,
                                                         int64_t Kw, int64_t N) {
  __shared__ uint32_t tile[32][33];
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
  const int64_t n0 = (int64_t)blockIdx.x * 32, c0 = (int64_t)blockIdx.y * 32;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int64_t c = c0 + ty + 8 * i, n = n0 + tx;
    if (c < Kw && n < N) tile[ty + 8 * i][tx] = qw[c * N + n];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int64_t n = n0 + ty + 8 * i, c = c0 + tx;
    if (c < Kw && n < N) codes[n * Kw + c] = tile[tx][ty + 8 * i];
  }
}

// Act order: code (n, k) = nibble (r % 8) of qweight[r / 8][n], r = perm[k] (clamped into range).
__global__ __launch_bounds__(256) void gptq_codes_perm_kernel(const uint32_t *__restrict__ qw,
                                                              const int64_t *__restrict__ perm,
                                                              uint32_t *__restrict__ codes, int64_t K, int64_t N) {
  const int64_t Kw = K / 8;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // n fastest: coalesced qweight reads
  if (i >= N * Kw) return;
  const int64_t n = i % N, c = i / N;
  uint32_t w = 0;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    int64_t r = perm[8 * c + j];
    r = r < 0 ? 0 : (r >= K ? K - 1 : r);
    w |= nib(qw[(r >> 3) * N + n], (int)(r & 7)) << (4 * j);
  }
  codes[n * Kw + c] = w;
}

// AWQ: code (n, k) = nibble awq_inv(n % 8) of qweight[k][n / 8].
__global__ __launch_bounds__(256) void awq_codes_kernel(const uint32_t *__restrict__ qw, uint32_t *__restrict__ codes,
                                                        int64_t K, int64_t N) {
  const int64_t Kw = K / 8, Nw = N / 8;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // n fastest
  if (i >= N * Kw) return;
  const int64_t n = i % N, c = i / N;
  const int sh = awq_inv((int)(n & 7));
  uint32_t w = 0;
#pragma unroll
  for (int j = 0; j < 8; j++) w |= nib(qw[(8 * c + j) * Nw + n / 8], sh) << (4 * j);
  codes[n * Kw + c] = w;
}

// Scales (G, N) -> (N, G) and zeros from qzeros (G, N/8): mode 0 GPTQ (stored zero - 1),
// 1 GPTQ v2 (the zero), 2 AWQ (the zero, AWQ nibble order).
__global__ __launch_bounds__(256) void int4_sz_kernel(const uint32_t *__restrict__ qz, const float *__restrict__ sc,
                                                      float *__restrict__ s_out, float *__restrict__ z_out, int64_t G,
                                                      int64_t N, int mode) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // n fastest: coalesced reads
  if (i >= N * G) return;
  const int64_t n = i % N, g = i / N;
  const int j = mode == 2 ? awq_inv((int)(n & 7)) : (int)(n & 7);
  const uint32_t z = nib(qz[g * (N / 8) + n / 8], j) + (mode == 0 ? 1u : 0u);
  s_out[n * G + g] = sc[g * N + n];
  z_out[n * G + g] = (float)z;
}

}  // namespace

int launch_int4_from_gptq(const uint32_t *qw, const uint32_t *qz, const float *sc, const int64_t *perm, int64_t K,
                          int64_t N, int group, bool v2, uint32_t *codes, float *s_out, float *z_out, hipStream_t s) {
  const int64_t Kw = K / 8, G = K / group;
  if (perm) {
    gptq_codes_perm_kernel<<<(unsigned)cdiv(N * Kw, 256), 256, 0, s>>>(qw, perm, codes, K, N);
  } else {
    dim3 grid((unsigned)cdiv(N, 32), (unsigned)cdiv(Kw, 32));
    gptq_codes_kernel<<<grid, 256, 0, s>>>(qw, codes, Kw, N);
  }
  if (int rc = check_launch("int4_from_gptq")) return rc;
  int4_sz_kernel<<<(unsigned)cdiv(N * G, 256), 256, 0, s>>>(qz, sc, s_out, z_out, G, N, v2 ? 1 : 0);
  return check_launch("int4_from_gptq");
}

int launch_int4_from_awq(const uint32_t *qw, const uint32_t *qz, const float *sc, int64_t K, int64_t N, int group,
                         uint32_t *codes, float *s_out, float *z_out, hipStream_t s) {
  const int64_t Kw = K / 8, G = K / group;
  awq_codes_kernel<<<(unsigned)cdiv(N * Kw, 256), 256, 0, s>>>(qw, codes, K, N);
  if (int rc = check_launch("int4_from_awq")) return rc;
  int4_sz_kernel<<<(unsigned)cdiv(N * G, 256), 256, 0, s>>>(qz, sc, s_out, z_out, G, N, 2);
  return check_launch("int4_from_awq");
}

}  // namespace hq
