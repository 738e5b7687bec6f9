// gemm.hip -- Q4_K prefill GEMM on MFMA (gfx950 v_mfma_f32_32x32x16_bf16).
//
// Role: the M >= 9 leg of Light's matmul_q, which Light runs as a full F32
// dequant + cuBLAS SGEMM (ops/matmul_q.go:52-59, 85-95); here it is one fused
// kernel.  out[m, n] = sum_k x[m, k] * dequant(W)[n, k].
//
// Design:
//  * Activations are converted once to bf16 (RNE) in the workspace: from F32 x
//    (hq_matmul_q) or from prepared q8_1 activations (hq_matmul_q_act).
//  * Workgroup tile BM x BN = 256 x 128 over K steps of BK = 64 (a quarter of a
//    Q4_K super-block: sub-blocks 2p and 2p+1).  4 waves, each 128 x 64 =
//    4 x 2 MFMA 32x32 tiles (128 f32 accumulators per lane).
//  * Each K step, every thread dequantizes 16 quant bytes (32 weights) of one
//    weight row, (d*sc)*q - dmin*m in f32, rounds to bf16 and writes them into
//    the LDS B tile: the 4-bit weights cross HBM once and are expanded only in
//    LDS, amortised over the 256 activation rows of the tile.
//  * LDS is double-buffered; the next step's global loads are issued before the
//    current step's MFMAs.  Rows are padded to 72 bf16 (144 B) so the 32 lanes
//    reading one 16-byte column slice hit distinct banks.
//  * Workgroup -> tile mapping keeps both M tiles of a weight tile on the same
//    XCD (workgroups are dealt round-robin over the 8 XCDs), so a weight tile is
//    fetched from HBM into one L2 once.
//  * Split-K (grid.z) fills the chip when there are few output tiles; partial
//    tiles are summed in split order by a second kernel (deterministic).
#include "internal.hpp"

namespace hq {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int GBM = 256, GBN = 128, GBK = 64, GLD = GBK + 8;  // LDS row stride in bf16
constexpr int G_A_BYTES = GBM * GLD * 2, G_B_BYTES = GBN * GLD * 2;
constexpr int G_STAGE = G_A_BYTES + G_B_BYTES;
constexpr int G_LDS = 2 * G_STAGE;

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Two f32 -> packed bf16 (RNE; one v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  bf16x2 v = {(__bf16)a, (__bf16)b};
  uint32_t u;
  __builtin_memcpy(&u, &v, 4);
  return u;
}

// Dequantize the 8 nibbles of one quant dword: low nibbles (sub-block 2p) -> lo0/lo1,
// high nibbles (sub-block 2p+1) -> hi0/hi1, as packed bf16 pairs in element order.
__device__ __forceinline__ void dq8(uint32_t v, float dA, float mA, float dB, float mB, uint32_t &lo0,
                                    uint32_t &lo1, uint32_t &hi0, uint32_t &hi1) {
  const uint32_t l = v & 0x0F0F0F0Fu, h = (v >> 4) & 0x0F0F0F0Fu;
  lo0 = pack_bf16(dA * (float)(l & 0xff) - mA, dA * (float)((l >> 8) & 0xff) - mA);
  lo1 = pack_bf16(dA * (float)((l >> 16) & 0xff) - mA, dA * (float)(l >> 24) - mA);
  hi0 = pack_bf16(dB * (float)(h & 0xff) - mB, dB * (float)((h >> 8) & 0xff) - mB);
  hi1 = pack_bf16(dB * (float)((h >> 16) & 0xff) - mB, dB * (float)(h >> 24) - mB);
}

struct GemmArgs {
  const uint16_t *x;  // bf16 activations [M][K]
  const uint8_t *w;   // Q4_K (N, K)
  float *out;         // [M][N] or split partials [S][M][N]
  int M, N, K, nb;    // nb = K / 256
  int tiles_m, tiles_n, splits;
  int xcd_map;        // 1: XCD-grouped tile mapping
};

__global__ __launch_bounds__(256) void gemm_q4k_kernel(GemmArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;  // wave tile origin: rows wm*128, cols wn*64

  // Tile mapping.
  int tile = blockIdx.x;
  const int ntiles = a.tiles_m * a.tiles_n;
  if (a.xcd_map) tile = (blockIdx.x % 8) * (ntiles / 8) + blockIdx.x / 8;
  const int tm = tile % a.tiles_m, tn = tile / a.tiles_m;
  const int m0 = tm * GBM, n0 = tn * GBN;
  const int z = blockIdx.z;
  const int blk0 = (int)((int64_t)a.nb * z / a.splits), blk1 = (int)((int64_t)a.nb * (z + 1) / a.splits);
  const int nsteps = (blk1 - blk0) * 4;

  // Global load assignment.
  // A: 256 rows x 128 B per step; load i covers rows 32i + t/8, 16-byte column t%8.
  const int acol = t & 7;
  const uint16_t *xrow[8];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const int r = m0 + 32 * i + (t >> 3);
    xrow[i] = a.x + (int64_t)(r < a.M ? r : a.M - 1) * a.K + acol * 8;
  }
  // W: thread t -> weight row n0 + t/2, quant half h = t & 1 (16 bytes).
  const int wr = t >> 1, wh = t & 1;
  const int wrow = n0 + wr < a.N ? n0 + wr : a.N - 1;
  const uint8_t *wrp = a.w + (int64_t)wrow * a.nb * 144;

  f32x16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

  uint4 ra0, ra1, ra2, ra3, ra4, ra5, ra6, ra7, rq, rh;

#define GEMM_GLOAD(step)                                                                   \
  {                                                                                        \
    const int kb_ = blk0 + ((step) >> 2), p_ = (step) & 3, k0_ = kb_ * 256 + p_ * 64;       \
    ra0 = *reinterpret_cast<const uint4 *>(xrow[0] + k0_);                                 \
    ra1 = *reinterpret_cast<const uint4 *>(xrow[1] + k0_);                                 \
    ra2 = *reinterpret_cast<const uint4 *>(xrow[2] + k0_);                                 \
    ra3 = *reinterpret_cast<const uint4 *>(xrow[3] + k0_);                                 \
    ra4 = *reinterpret_cast<const uint4 *>(xrow[4] + k0_);                                 \
    ra5 = *reinterpret_cast<const uint4 *>(xrow[5] + k0_);                                 \
    ra6 = *reinterpret_cast<const uint4 *>(xrow[6] + k0_);                                 \
    ra7 = *reinterpret_cast<const uint4 *>(xrow[7] + k0_);                                 \
    const uint8_t *bp_ = wrp + (int64_t)kb_ * 144;                                         \
    rq = *reinterpret_cast<const uint4 *>(bp_ + 16 + 32 * p_ + 16 * wh);                   \
    rh = *reinterpret_cast<const uint4 *>(bp_);                                            \
  }

#define GEMM_LSTORE(step, buf)                                                                          \
  {                                                                                                     \
    uint8_t *sa_ = smem + (buf) * G_STAGE;                                                              \
    uint8_t *sb_ = sa_ + G_A_BYTES;                                                                     \
    uint8_t *ad_ = sa_ + ((t >> 3) * GLD + acol * 8) * 2;                                               \
    *reinterpret_cast<uint4 *>(ad_ + 0 * 32 * GLD * 2) = ra0;                                           \
    *reinterpret_cast<uint4 *>(ad_ + 1 * 32 * GLD * 2) = ra1;                                           \
    *reinterpret_cast<uint4 *>(ad_ + 2 * 32 * GLD * 2) = ra2;                                           \
    *reinterpret_cast<uint4 *>(ad_ + 3 * 32 * GLD * 2) = ra3;                                           \
    *reinterpret_cast<uint4 *>(ad_ + 4 * 32 * GLD * 2) = ra4;                                           \
    *reinterpret_cast<uint4 *>(ad_ + 5 * 32 * GLD * 2) = ra5;                                           \
    *reinterpret_cast<uint4 *>(ad_ + 6 * 32 * GLD * 2) = ra6;                                           \
    *reinterpret_cast<uint4 *>(ad_ + 7 * 32 * GLD * 2) = ra7;                                           \
    const int p_ = (step) & 3;                                                                          \
    const float d_ = h2f(rh.x & 0xffffu), dmin_ = h2f(rh.x >> 16);                                      \
    int scA_, mnA_, scB_, mnB_;                                                                         \
    q4k_scale_min(2 * p_, rh.y, rh.z, rh.w, scA_, mnA_);                                                \
    q4k_scale_min(2 * p_ + 1, rh.y, rh.z, rh.w, scB_, mnB_);                                            \
    const float dA_ = d_ * (float)scA_, mA_ = dmin_ * (float)mnA_;                                      \
    const float dB_ = d_ * (float)scB_, mB_ = dmin_ * (float)mnB_;                                      \
    uint32_t lo_[8], hi_[8];                                                                            \
    dq8(rq.x, dA_, mA_, dB_, mB_, lo_[0], lo_[1], hi_[0], hi_[1]);                                      \
    dq8(rq.y, dA_, mA_, dB_, mB_, lo_[2], lo_[3], hi_[2], hi_[3]);                                      \
    dq8(rq.z, dA_, mA_, dB_, mB_, lo_[4], lo_[5], hi_[4], hi_[5]);                                      \
    dq8(rq.w, dA_, mA_, dB_, mB_, lo_[6], lo_[7], hi_[6], hi_[7]);                                      \
    uint4 *bd_ = reinterpret_cast<uint4 *>(sb_ + (wr * GLD + 16 * wh) * 2);                             \
    bd_[0] = make_uint4(lo_[0], lo_[1], lo_[2], lo_[3]);                                                \
    bd_[1] = make_uint4(lo_[4], lo_[5], lo_[6], lo_[7]);                                                \
    uint4 *bh_ = reinterpret_cast<uint4 *>(sb_ + (wr * GLD + 32 + 16 * wh) * 2);                        \
    bh_[0] = make_uint4(hi_[0], hi_[1], hi_[2], hi_[3]);                                                \
    bh_[1] = make_uint4(hi_[4], hi_[5], hi_[6], hi_[7]);                                                \
  }

  if (nsteps > 0) {
    GEMM_GLOAD(0);
    GEMM_LSTORE(0, 0);
  }
  __syncthreads();
  const int fr = lane & 31, fk = (lane >> 5) * 8;  // fragment row / k offset
  for (int s = 0; s < nsteps; s++) {
    const int buf = s & 1;
    if (s + 1 < nsteps) GEMM_GLOAD(s + 1);
    const uint8_t *sa = smem + buf * G_STAGE;
    const uint8_t *sb = sa + G_A_BYTES;
#pragma unroll
    for (int kk = 0; kk < GBK / 16; kk++) {
      bf16x8 af[4], bfr[2];
#pragma unroll
      for (int i = 0; i < 4; i++)
        af[i] = *reinterpret_cast<const bf16x8 *>(sa + ((wm * 128 + i * 32 + fr) * GLD + kk * 16 + fk) * 2);
#pragma unroll
      for (int j = 0; j < 2; j++)
        bfr[j] = *reinterpret_cast<const bf16x8 *>(sb + ((wn * 64 + j * 32 + fr) * GLD + kk * 16 + fk) * 2);
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
    if (s + 1 < nsteps) GEMM_LSTORE(s + 1, buf ^ 1);
    __syncthreads();
  }
#undef GEMM_GLOAD
#undef GEMM_LSTORE

  // Epilogue: lane holds D[8*(r/4) + 4*(lane/32) + r%4][lane%32] of each 32x32 tile.
  float *out = a.out + (int64_t)z * a.M * a.N;
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int col = n0 + wn * 64 + j * 32 + (lane & 31);
      if (col >= a.N) continue;
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int row = m0 + wm * 128 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (row < a.M) out[(int64_t)row * a.N + col] = acc[i][j][r];
      }
    }
}

__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float *__restrict__ part, float *__restrict__ out,
                                                            int64_t n, int splits) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float s = part[i];
  for (int z = 1; z < splits; z++) s += part[(int64_t)z * n + i];
  out[i] = s;
}

// x F32 -> bf16 (RNE, BF16FromF32 semantics).
__global__ __launch_bounds__(256) void f32_to_bf16_kernel(const float *__restrict__ x, uint16_t *__restrict__ y,
                                                          int64_t n4) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n4) return;
  float4 v = reinterpret_cast<const float4 *>(x)[i];
  reinterpret_cast<uint2 *>(y)[i] = make_uint2(pack_bf16(v.x, v.y), pack_bf16(v.z, v.w));
}

// Prepared activations -> bf16 of d * q.
__global__ __launch_bounds__(256) void act_to_bf16_kernel(const uint8_t *__restrict__ act, uint16_t *__restrict__ y,
                                                          int64_t n4, int64_t d_off) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n4) return;
  const uint32_t q = reinterpret_cast<const uint32_t *>(act)[i];
  const float d = reinterpret_cast<const float *>(act + d_off)[i >> 3];
  float v0 = d * (float)(int8_t)(q & 0xff), v1 = d * (float)(int8_t)((q >> 8) & 0xff);
  float v2 = d * (float)(int8_t)((q >> 16) & 0xff), v3 = d * (float)(int8_t)(q >> 24);
  reinterpret_cast<uint2 *>(y)[i] = make_uint2(pack_bf16(v0, v1), pack_bf16(v2, v3));
}

static int gemm_splits(int64_t M, int64_t N, int64_t K) {
  int64_t tiles = cdiv(M, GBM) * cdiv(N, GBN), nb = K / 256;
  int target = device_cus();
  int s = 1;
  while (tiles * (s * 2) <= target && nb / (s * 2) >= 4) s *= 2;
  return s;
}

size_t gemm_q4k_ws_bytes(int64_t M, int64_t K) {
  // bf16 activations + room for split-K partials is sized per call in launch (N unknown here):
  // the bf16 copy only; partials live in a second region sized by gemm_q4k_partial_bytes.
  return ((size_t)M * (size_t)K * 2 + 255) & ~(size_t)255;
}

size_t gemm_q4k_partial_bytes(int64_t M, int64_t N, int64_t K) {
  int s = gemm_splits(M, N, K);
  return s > 1 ? (size_t)s * (size_t)M * (size_t)N * 4 : 0;
}

static bool g_attr_set[64] = {false};

int launch_gemm_q4k_bf16(const uint16_t *xb, const void *w, float *out, float *partials, int64_t M, int64_t N,
                         int64_t K, hipStream_t s) {
  int dev = 0;
  (void)hipGetDevice(&dev);
  if (dev >= 0 && dev < 64 && !g_attr_set[dev]) {
    if (int rc = check(hipFuncSetAttribute((const void *)gemm_q4k_kernel,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, G_LDS),
                       "hipFuncSetAttribute"))
      return rc;
    g_attr_set[dev] = true;
  }
  GemmArgs a;
  a.x = xb;
  a.w = static_cast<const uint8_t *>(w);
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.nb = (int)(K / 256);
  a.tiles_m = (int)cdiv(M, GBM);
  a.tiles_n = (int)cdiv(N, GBN);
  a.splits = gemm_splits(M, N, K);
  const int ntiles = a.tiles_m * a.tiles_n;
  a.xcd_map = ntiles % 8 == 0;
  a.out = a.splits > 1 ? partials : out;
  dim3 grid((unsigned)ntiles, 1, (unsigned)a.splits);
  gemm_q4k_kernel<<<grid, 256, G_LDS, s>>>(a);
  if (int rc = check_launch("gemm_q4k")) return rc;
  if (a.splits > 1) {
    int64_t n = M * N;
    splitk_reduce_kernel<<<(unsigned)cdiv(n, 256), 256, 0, s>>>(partials, out, n, a.splits);
    return check_launch("splitk_reduce");
  }
  return HQ_OK;
}

int launch_to_bf16(const void *src, bool from_act, uint16_t *dst, int64_t M, int64_t K, hipStream_t s) {
  int64_t n4 = M * K / 4;
  if (from_act)
    act_to_bf16_kernel<<<(unsigned)cdiv(n4, 256), 256, 0, s>>>(static_cast<const uint8_t *>(src), dst, n4,
                                                                  act_d_off(M, K));
  else
    f32_to_bf16_kernel<<<(unsigned)cdiv(n4, 256), 256, 0, s>>>(static_cast<const float *>(src), dst, n4);
  return check_launch("to_bf16");
}

}  // namespace hq
