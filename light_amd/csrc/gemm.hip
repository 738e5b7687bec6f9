// gemm.hip -- quantized-weight GEMM on MFMA (gfx950 v_mfma_f32_32x32x16_bf16).
//
// Role: the many-row leg of Light's quantized matmuls, which Light runs as a
// full dequant + cuBLAS GEMM: matmul_q for M >= 8 (ops/matmul_q.go:52-59,
// 85-95) and MatMulInt4 for M > 8 (ops/int4.go:100-126).  Here it is one fused
// kernel: out[m, n] = sum_k x[m, k] * dequant(W)[n, k].
//
// Design:
//  * Activations are converted once to bf16 (RNE) in the workspace (from F32 /
//    F16 x, or from prepared q8_1 activations); bf16 x is used as is.
//  * A workgroup computes a BM x 128 tile over K steps of 64.  Each step, the
//    weight policy loads 16 packed bytes per thread (32 weights of one row),
//    dequantizes them in f32, rounds to bf16 and writes them into the LDS B
//    tile: 4-bit weights cross HBM once and are expanded only in LDS, amortised
//    over the BM activation rows of the tile.
//      Q4_K: a 64-wide K window is sub-blocks 2p, 2p+1 of one super-block;
//            w = (d*sc)*q - dmin*m (quant/q4_k.go:61-77).
//      int4: a 64-wide window lies in one group (G % 64 == 0); w = s*(q - z)
//            (quant/int4.go:239-261).
//  * BM = 256: 4 waves of 128 x 64 (4 x 2 MFMA 32x32 tiles, 128 f32
//    accumulators); BM = 64: 4 waves of 64 x 32.
//  * LDS is double-buffered; the next step's global loads are issued before
//    the current step's MFMAs.  Rows are padded to 72 bf16 (144 B) so the 32
//    lanes reading one 16-byte column slice hit distinct banks.
//  * Workgroup -> tile mapping keeps the M tiles of a weight tile on one XCD
//    (workgroups are dealt round-robin over the 8 XCDs), so a weight tile is
//    fetched from HBM into one L2 once.
//  * Split-K (grid.z) fills the chip when there are few output tiles; partial
//    tiles are summed in split order by a second kernel (deterministic), which
//    also converts to the output dtype.
#include "internal.hpp"

#include <algorithm>

namespace hq {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
// Native 4 x u32 vector: unlike HIP's uint4 (a struct over a union, copied with
// memcpy) arrays of it stay in registers.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int GBN = 128, GBK = 64, GLD = GBK + 8;  // LDS row stride in bf16

template <int BM>
struct GTile {
  static constexpr int WM = BM == 256 ? 2 : 1, WN = 4 / WM;  // waves along M / N
  static constexpr int TM = BM / WM, TN = GBN / WN;          // wave tile
  static constexpr int MT = TM / 32, NT = TN / 32;           // MFMA tiles per wave
  static constexpr int A_BYTES = BM * GLD * 2, B_BYTES = GBN * GLD * 2;
  static constexpr int STAGE = A_BYTES + B_BYTES, LDS = 2 * STAGE;
  static constexpr int AROWS_PER_LOAD = 32, ALOADS = BM / 32;  // 8 lanes per 128-byte row slice
};

// Two f32 -> packed bf16 (RNE; one v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  bf16x2 v = {(__bf16)a, (__bf16)b};
  uint32_t u;
  __builtin_memcpy(&u, &v, 4);
  return u;
}

struct GemmArgs {
  const uint16_t *x;  // bf16 activations [M][K]
  const uint8_t *w;   // Q4_K blocks (N, K) or int4 codes (N, K/8)
  const float *s, *z; // int4 scales / zeros (N, K/G)
  float *out;         // [M][N] or split partials [S][M][N]
  int M, N, K, G;
  int tiles_m, tiles_n, splits;
  int xcd_map;        // 1: XCD-grouped tile mapping
};

// ---- weight policies: registers for one K step and the LDS write ----------

struct Q4kPolicy {
  u32x4 q, h;
  __device__ __forceinline__ void load(const GemmArgs &a, int row, int half, int k0) {
    const uint8_t *bp = a.w + (int64_t)row * (a.K / 256) * 144 + (int64_t)(k0 >> 8) * 144;
    const int p = (k0 >> 6) & 3;
    q = *reinterpret_cast<const u32x4 *>(bp + 16 + 32 * p + 16 * half);
    h = *reinterpret_cast<const u32x4 *>(bp);
  }
  // Low nibbles: sub-block 2p, k = 16*half + i; high nibbles: sub-block 2p+1, k = 32 + 16*half + i.
  __device__ __forceinline__ void store(uint8_t *brow, int half, int k0) const {
    const int p = (k0 >> 6) & 3;
    const float d = h2f(h.x & 0xffffu), dmin = h2f(h.x >> 16);
    int scA, mnA, scB, mnB;
    q4k_scale_min(2 * p, h.y, h.z, h.w, scA, mnA);
    q4k_scale_min(2 * p + 1, h.y, h.z, h.w, scB, mnB);
    const float dA = d * (float)scA, mA = dmin * (float)mnA, dB = d * (float)scB, mB = dmin * (float)mnB;
    const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
    uint32_t lo[8], hi[8];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const uint32_t l = qw[k] & 0x0F0F0F0Fu, hh = (qw[k] >> 4) & 0x0F0F0F0Fu;
      lo[2 * k] = pack_bf16(dA * (float)(l & 0xff) - mA, dA * (float)((l >> 8) & 0xff) - mA);
      lo[2 * k + 1] = pack_bf16(dA * (float)((l >> 16) & 0xff) - mA, dA * (float)(l >> 24) - mA);
      hi[2 * k] = pack_bf16(dB * (float)(hh & 0xff) - mB, dB * (float)((hh >> 8) & 0xff) - mB);
      hi[2 * k + 1] = pack_bf16(dB * (float)((hh >> 16) & 0xff) - mB, dB * (float)(hh >> 24) - mB);
    }
    u32x4 *bd = reinterpret_cast<u32x4 *>(brow + 32 * half);
    bd[0] = u32x4{lo[0], lo[1], lo[2], lo[3]};
    bd[1] = u32x4{lo[4], lo[5], lo[6], lo[7]};
    u32x4 *bh = reinterpret_cast<u32x4 *>(brow + 64 + 32 * half);
    bh[0] = u32x4{hi[0], hi[1], hi[2], hi[3]};
    bh[1] = u32x4{hi[4], hi[5], hi[6], hi[7]};
  }
};

struct Int4Policy {
  u32x4 q;
  float s, z;
  // Codes of k in [k0 + 32*half, +32): words k0/8 + 4*half .. +4.
  __device__ __forceinline__ void load(const GemmArgs &a, int row, int half, int k0) {
    q = *reinterpret_cast<const u32x4 *>(a.w + (int64_t)row * (a.K / 2) + (k0 >> 1) + 16 * half);
    const int64_t gi = (int64_t)row * (a.K / a.G) + k0 / a.G;
    s = a.s[gi];
    z = a.z[gi];
  }
  __device__ __forceinline__ void store(uint8_t *brow, int half, int) const {
    const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
    uint32_t o[16];
#pragma unroll
    for (int k = 0; k < 4; k++)
#pragma unroll
      for (int j = 0; j < 8; j += 2)
        o[4 * k + j / 2] = pack_bf16(s * ((float)((qw[k] >> (4 * j)) & 15) - z),
                                     s * ((float)((qw[k] >> (4 * j + 4)) & 15) - z));
    u32x4 *bd = reinterpret_cast<u32x4 *>(brow + 64 * half);
#pragma unroll
    for (int k = 0; k < 4; k++) bd[k] = u32x4{o[4 * k], o[4 * k + 1], o[4 * k + 2], o[4 * k + 3]};
  }
};

template <class WP, int BM>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs a) {
  using T = GTile<BM>;
  extern __shared__ __align__(16) uint8_t smem[];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave / T::WN, wn = wave % T::WN;

  int tile = blockIdx.x;
  const int ntiles = a.tiles_m * a.tiles_n;
  if (a.xcd_map) tile = (blockIdx.x % 8) * (ntiles / 8) + blockIdx.x / 8;
  const int tm = tile % a.tiles_m, tn = tile / a.tiles_m;
  const int m0 = tm * BM, n0 = tn * GBN;
  const int z = blockIdx.z;
  const int ksteps = a.K / GBK;
  const int st0 = (int)((int64_t)ksteps * z / a.splits), st1 = (int)((int64_t)ksteps * (z + 1) / a.splits);
  const int nsteps = st1 - st0;

  // A: BM rows x 128 B per step; load i covers rows 32i + t/8, 16-byte column t%8.
  const int acol = t & 7;
  const uint16_t *xrow[T::ALOADS];
#pragma unroll
  for (int i = 0; i < T::ALOADS; i++) {
    const int r = m0 + 32 * i + (t >> 3);
    xrow[i] = a.x + (int64_t)(r < a.M ? r : a.M - 1) * a.K + acol * 8;
  }
  // W: thread t -> weight row n0 + t/2, half t & 1.
  const int wr = t >> 1, wh = t & 1;
  const int wrow = n0 + wr < a.N ? n0 + wr : a.N - 1;

  f32x16 acc[T::MT][T::NT];
#pragma unroll
  for (int i = 0; i < T::MT; i++)
#pragma unroll
    for (int j = 0; j < T::NT; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

  u32x4 ra[T::ALOADS];
  WP wp;
  if (nsteps > 0) {
    const int k0 = st0 * GBK;
#pragma unroll
    for (int i = 0; i < T::ALOADS; i++) ra[i] = *reinterpret_cast<const u32x4 *>(xrow[i] + k0);
    wp.load(a, wrow, wh, k0);
    uint8_t *ad = smem + ((t >> 3) * GLD + acol * 8) * 2;
#pragma unroll
    for (int i = 0; i < T::ALOADS; i++) *reinterpret_cast<u32x4 *>(ad + i * 32 * GLD * 2) = ra[i];
    wp.store(smem + T::A_BYTES + wr * GLD * 2, wh, k0);
  }
  __syncthreads();
  const int fr = lane & 31, fk = (lane >> 5) * 8;  // fragment row / k offset
  for (int s = 0; s < nsteps; s++) {
    const int buf = s & 1;
    const int kn = (st0 + s + 1) * GBK;
    if (s + 1 < nsteps) {
#pragma unroll
      for (int i = 0; i < T::ALOADS; i++) ra[i] = *reinterpret_cast<const u32x4 *>(xrow[i] + kn);
      wp.load(a, wrow, wh, kn);
    }
    const uint8_t *sa = smem + buf * T::STAGE;
    const uint8_t *sb = sa + T::A_BYTES;
#pragma unroll
    for (int kk = 0; kk < GBK / 16; kk++) {
      bf16x8 af[T::MT], bfr[T::NT];
#pragma unroll
      for (int i = 0; i < T::MT; i++)
        af[i] = *reinterpret_cast<const bf16x8 *>(sa + ((wm * T::TM + i * 32 + fr) * GLD + kk * 16 + fk) * 2);
#pragma unroll
      for (int j = 0; j < T::NT; j++)
        bfr[j] = *reinterpret_cast<const bf16x8 *>(sb + ((wn * T::TN + j * 32 + fr) * GLD + kk * 16 + fk) * 2);
#pragma unroll
      for (int i = 0; i < T::MT; i++)
#pragma unroll
        for (int j = 0; j < T::NT; j++)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
    if (s + 1 < nsteps) {
      uint8_t *na = smem + (buf ^ 1) * T::STAGE;
      uint8_t *ad = na + ((t >> 3) * GLD + acol * 8) * 2;
#pragma unroll
      for (int i = 0; i < T::ALOADS; i++) *reinterpret_cast<u32x4 *>(ad + i * 32 * GLD * 2) = ra[i];
      wp.store(na + T::A_BYTES + wr * GLD * 2, wh, kn);
    }
    __syncthreads();
  }

  // Epilogue: lane holds D[8*(r/4) + 4*(lane/32) + r%4][lane%32] of each 32x32 tile.
  float *out = a.out + (int64_t)z * a.M * a.N;
#pragma unroll
  for (int i = 0; i < T::MT; i++)
#pragma unroll
    for (int j = 0; j < T::NT; j++) {
      const int col = n0 + wn * T::TN + j * 32 + (lane & 31);
      if (col >= a.N) continue;
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int row = m0 + wm * T::TM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (row < a.M) out[(int64_t)row * a.N + col] = acc[i][j][r];
      }
    }
}

// ---- int4, M <= 64: weights straight into MFMA operands -------------------------
// out[m, n] = sum_k x[m, k] * s[n, g] * (q[n, k] - z[n, g]) for up to 64 rows of x.  Each wave
// owns 32 weight rows and streams their codes through registers, expanding each lane's 8
// codes per 16-k slice directly into its MFMA B fragment (no LDS for the weights); the
// workgroup shares x in LDS, 128 k per stage, double-buffered.  The two halves of a wave
// (lanes l / 32) take the two contiguous 64-k halves of a stage -- A and B use the same
// k permutation, so the sum is unchanged -- which makes every code load a contiguous 16 B.
// Dequant in fma form, s * q + (-s z), rounded once to bf16 (the 64-row path is not the
// bit-exact dequant).  Split K over grid.z; partial tiles summed by splitk_reduce_kernel.
constexpr int SK = 128, SLD = SK + 8;  // x stage: 64 rows x 128 k (bf16), padded row stride

struct SmallI4Args {
  const uint16_t *x;       // bf16 [M][K]
  const uint32_t *codes;   // (N, K/8)
  const float *s, *z;      // (N, K/G)
  float *out;              // [M][N] or split partials [S][M][N]
  int M, N, K, G, splits;
};

template <bool G64>  // G % 64 == 0: one (scale, zero) per lane per stage
__global__ __launch_bounds__(256) void gemm_small_int4_kernel(SmallI4Args a) {
  __shared__ __align__(16) uint16_t xs[2][64 * SLD];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int kh = lane >> 5, fr = lane & 31;
  const int n0 = blockIdx.x * 128 + wave * 32;
  const int row = n0 + fr < a.N ? n0 + fr : a.N - 1;  // this lane's weight row (clamped)
  const int nst = a.K / SK;
  const int c0 = (int)((int64_t)nst * blockIdx.z / a.splits), c1 = (int)((int64_t)nst * (blockIdx.z + 1) / a.splits);
  const int ng = a.K / a.G;
  const uint32_t *crow = a.codes + (int64_t)row * (a.K / 8);
  const float *srow = a.s + (int64_t)row * ng, *zrow = a.z + (int64_t)row * ng;
  // x stage loads: 64 rows x 256 B; thread t -> row t / 4, 64-byte quarter t % 4.
  const int xr = t >> 2, xq = t & 3;
  const uint16_t *xsrc = a.x + (int64_t)(xr < a.M ? xr : a.M - 1) * a.K + xq * 32;

  f32x16 acc[2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int r = 0; r < 16; r++) acc[i][r] = 0.f;
  if (c0 >= c1) return;

  // Stage c + 1's loads go out while stage c is computed.  (A two-stage register ring
  // measured the same: the compiler waits for every outstanding load at the loop's back edge.)
  u32x4 xv[4], cw[2];
  float sc[8], zc[8];
  auto load_stage = [&](int c) __attribute__((always_inline)) {
    const uint16_t *xp = xsrc + (int64_t)c * SK;
#pragma unroll
    for (int i = 0; i < 4; i++) xv[i] = *reinterpret_cast<const u32x4 *>(xp + 8 * i);
    const uint32_t *cp = crow + (c * SK + 64 * kh) / 8;
    cw[0] = *reinterpret_cast<const u32x4 *>(cp);
    cw[1] = *reinterpret_cast<const u32x4 *>(cp + 4);
    if constexpr (G64) {
      const int g = (c * SK + 64 * kh) / a.G;
      sc[0] = srow[g];
      zc[0] = zrow[g];
    } else {
#pragma unroll
      for (int s8 = 0; s8 < 8; s8++) {
        const int g = (c * SK + 64 * kh + 8 * s8) / a.G;
        sc[s8] = srow[g];
        zc[s8] = zrow[g];
      }
    }
  };
  auto store_x = [&](int buf) __attribute__((always_inline)) {
    uint16_t *d = &xs[buf][xr * SLD + xq * 32];
#pragma unroll
    for (int i = 0; i < 4; i++) *reinterpret_cast<u32x4 *>(d + 8 * i) = xv[i];
  };
  load_stage(c0);
  store_x(0);
  u32x4 cur[2] = {cw[0], cw[1]};
  float cs[8], cz[8];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    cs[i] = sc[G64 ? 0 : i];
    cz[i] = zc[G64 ? 0 : i];
  }
  __syncthreads();
  for (int c = c0; c < c1; c++) {
    const int buf = (c - c0) & 1;
    if (c + 1 < c1) load_stage(c + 1);
    const uint16_t *xa = &xs[buf][0];
#pragma unroll
    for (int s8 = 0; s8 < 8; s8++) {
      const uint32_t w = cur[s8 >> 2][s8 & 3];
      const float sg = cs[G64 ? 0 : s8], nz = -sg * cz[G64 ? 0 : s8];
      const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
      bf16x8 b;
      b[0] = (__bf16)__fmaf_rn(sg, (float)(lo & 0xff), nz);
      b[1] = (__bf16)__fmaf_rn(sg, (float)(hi & 0xff), nz);
      b[2] = (__bf16)__fmaf_rn(sg, (float)((lo >> 8) & 0xff), nz);
      b[3] = (__bf16)__fmaf_rn(sg, (float)((hi >> 8) & 0xff), nz);
      b[4] = (__bf16)__fmaf_rn(sg, (float)((lo >> 16) & 0xff), nz);
      b[5] = (__bf16)__fmaf_rn(sg, (float)((hi >> 16) & 0xff), nz);
      b[6] = (__bf16)__fmaf_rn(sg, (float)(lo >> 24), nz);
      b[7] = (__bf16)__fmaf_rn(sg, (float)(hi >> 24), nz);
      const int kx = 64 * kh + 8 * s8;
      const bf16x8 a0 = *reinterpret_cast<const bf16x8 *>(xa + fr * SLD + kx);
      const bf16x8 a1 = *reinterpret_cast<const bf16x8 *>(xa + (32 + fr) * SLD + kx);
      acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b, acc[0], 0, 0, 0);
      acc[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b, acc[1], 0, 0, 0);
    }
    if (c + 1 < c1) {
      store_x(buf ^ 1);
      cur[0] = cw[0];
      cur[1] = cw[1];
#pragma unroll
      for (int i = 0; i < 8; i++) {
        cs[i] = sc[G64 ? 0 : i];
        cz[i] = zc[G64 ? 0 : i];
      }
    }
    __syncthreads();
  }
  // Lane holds D[8*(r/4) + 4*(lane/32) + r%4][lane%32] of each 32 x 32 tile (m, n).
  float *out = a.out + (int64_t)blockIdx.z * a.M * a.N;
  const int col = n0 + fr;
  if (col >= a.N) return;
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int m = 32 * i + 8 * (r >> 2) + 4 * kh + (r & 3);
      if (m < a.M) out[(int64_t)m * a.N + col] = acc[i][r];
    }
}

// ---- MoE grouped GEMM ---------------------------------------------------------
// out[p, n] = w(p) * x[row(p)] . dequant(W[e])[n] for the expert-sorted pairs of
// expert e = blockIdx.y; blockIdx.x is the 128-wide weight-row tile.  The expert's
// pairs are processed in chunks of 32 gathered activation rows (BM = 32, 4 waves of
// 32 x 32), each chunk running the full K loop of gemm_kernel.

// ---- MoE grouped GEMM (prefill-sized routing: more than 4 pairs per expert) ------------
//
// out[p, :] = w(p) * x[row(p)] . dequant(W[e(p)])^T for the expert-sorted pairs (ops.MoEGemmQ,
// ops/moe.go:242-265), Q4_K.  grid = (N / 128, E); a workgroup takes its expert's pair segment
// in chunks of 32 gathered rows and streams the expert's 128 weight rows once per chunk.
//
// With only 16-32 rows per expert, each dequantized weight feeds at most 32 rows, so the
// dequant -- not the MFMAs -- is the work: the bf16 path (convert, FMA, round, 4.4 VALU
// instructions per weight) ran T = 256 gate/up at 108 us for 226 MB.  Here B is f16 and the
// dequant is packed: a nibble pair becomes the f16 pair (1024 + q) with one v_perm_b32
// against 0x64 bytes, one packed add takes away 1024 (exact), one packed FMA applies
// d*sc and -dmin*m (one rounding), about 2 VALU instructions per weight.  x is converted to
// f16 once per row with a power-of-two row scale (rows of |x| above 2^15 are scaled down, the
// output row scaled back up exactly), so the f16 range never clips.
// The raw loads of step s + MD go out while step s computes (a register ring of one 256-k
// block: the block header is loaded with its first step only).

constexpr int MD = 4;  // ring slots: one super-block of 256 k, so slot 0 starts each block
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2v __attribute__((ext_vector_type(2)));

struct MoeGemmArgs {
  GemmArgs g;          // x = f16 rows of x, w = expert stack, N, K
  const float *xscale; // per x row: the power of two the f16 row was divided by
  const int64_t *pairs;
  const int32_t *offsets;
  const float *topk_w;
  float *out;
  int64_t size_m, expert_bytes;
  int topk, rpp;
  int gated_I, act;  // gated: N = 2 I stacked gate / up rows, out (size_m, I) = act(g) * u
};

// x (rows, K) F32 -> f16, row r divided by 2^e_r (e_r = 0 unless the row's max |x| exceeds
// 2^15); xscale[r] = 2^e_r.  One workgroup per row.
__global__ __launch_bounds__(256) void to_f16_rowscale_kernel(const float *__restrict__ x, _Float16 *__restrict__ y,
                                                              float *__restrict__ xscale, int64_t K) {
  __shared__ float red[4];
  const int64_t r = blockIdx.x;
  const float *xr = x + r * K;
  const int t = threadIdx.x;
  // K <= 4096 (K % 256 == 0): the row stays in registers, four floats per load, so it is read
  // once; longer rows are read twice.
  constexpr int KV = 4;
  const int64_t n4 = K / 4;
  const bool reg = n4 <= KV * 256;
  float4 v[KV];
  float m = 0.f;
  if (reg) {
#pragma unroll
    for (int j = 0; j < KV; j++) {
      const int64_t i = t + 256 * j;
      v[j] = i < n4 ? reinterpret_cast<const float4 *>(xr)[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int j = 0; j < KV; j++)
      m = fmaxf(m, fmaxf(fmaxf(fabsf(v[j].x), fabsf(v[j].y)), fmaxf(fabsf(v[j].z), fabsf(v[j].w))));
  } else {
    for (int64_t k = t; k < K; k += 256) m = fmaxf(m, fabsf(xr[k]));
  }
  for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
  if ((t & 63) == 0) red[t >> 6] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  int ex = 0;
  (void)frexpf(m, &ex);  // m < 2^ex
  const int e = ex > 15 && m == m && m < INFINITY ? ex - 15 : 0;
  if (reg) {
#pragma unroll
    for (int j = 0; j < KV; j++) {
      const int64_t i = t + 256 * j;
      if (i < n4) {
        typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
        const f16x4 h = {(_Float16)ldexpf(v[j].x, -e), (_Float16)ldexpf(v[j].y, -e), (_Float16)ldexpf(v[j].z, -e),
                         (_Float16)ldexpf(v[j].w, -e)};
        reinterpret_cast<f16x4 *>(y + r * K)[i] = h;
      }
    }
  } else {
    for (int64_t k = t; k < K; k += 256) y[r * K + k] = (_Float16)ldexpf(xr[k], -e);
  }
  if (t == 0) xscale[r] = ldexpf(1.f, e);
}

// The ring's loads are issued from inline asm and awaited with explicit counts: with plain
// loads the compiler waits for every outstanding load at the K loop's back edge (vmcnt(0)),
// which leaves one step of latency exposed per step.  The wait names the registers it
// completes ("+v"), so nothing reads them -- or reuses them -- before it.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ u32x4 ldg16(const void *p) {
  u32x4 r;
  asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(r) : "v"(p) : "memory");
  return r;
}
template <int N>
__device__ __forceinline__ void wait_ring(u32x4 &a, u32x4 &b, u32x4 &c) {
  asm volatile("s_waitcnt vmcnt(%3)" : "+v"(a), "+v"(b), "+v"(c) : "n"(N) : "memory");
}
template <int N>
__device__ __forceinline__ void wait_ring(u32x4 &a, u32x4 &b) {
  asm volatile("s_waitcnt vmcnt(%2)" : "+v"(a), "+v"(b) : "n"(N) : "memory");
}
#pragma clang diagnostic pop

// Raw Q4_K bytes of one thread's B slot for one 64-k step: (row, half): quant bytes
// 16 * half .. + 16 of the step's pair (low nibbles: sub-block 2p, k = 16 half + i; high:
// sub-block 2p + 1, k = 32 + 16 half + i); the block header h (d, dmin, scales) is loaded
// with the block's first step only and kept for the other three.
struct Q4kF16Slot {
  u32x4 q;
  __device__ __forceinline__ static const uint8_t *block(const GemmArgs &a, int row, int k0) {
    return a.w + (int64_t)row * (a.K / 256) * 144 + (int64_t)(k0 >> 8) * 144;
  }
  __device__ __forceinline__ void load(const GemmArgs &a, int row, int half, int k0) {
    const int p = (k0 >> 6) & 3;
    q = ldg16(block(a, row, k0) + 16 + 32 * p + 16 * half);
  }
  __device__ __forceinline__ void store(uint8_t *brow, int half, int k0, const u32x4 &h) const {
    const int p = (k0 >> 6) & 3;
    const float d = h2f(h.x & 0xffffu), dmin = h2f(h.x >> 16);
    int scA, mnA, scB, mnB;
    q4k_scale_min(2 * p, h.y, h.z, h.w, scA, mnA);
    q4k_scale_min(2 * p + 1, h.y, h.z, h.w, scB, mnB);
    const _Float16 dA = (_Float16)(d * (float)scA), mA = (_Float16)(-(dmin * (float)mnA));
    const _Float16 dB = (_Float16)(d * (float)scB), mB = (_Float16)(-(dmin * (float)mnB));
    const f16x2v sa = {dA, dA}, ma = {mA, mA}, sb = {dB, dB}, mb = {mB, mB};
    const f16x2v k1024 = {(_Float16)-1024.f, (_Float16)-1024.f};
    constexpr uint32_t K64 = 0x64646464u;
    uint32_t lo[8], hi[8];
    const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const uint32_t l = qw[k] & 0x0F0F0F0Fu, hh = (qw[k] >> 4) & 0x0F0F0F0Fu;
      const uint32_t pr[4] = {__builtin_amdgcn_perm(K64, l, 0x04010400u), __builtin_amdgcn_perm(K64, l, 0x04030402u),
                              __builtin_amdgcn_perm(K64, hh, 0x04010400u), __builtin_amdgcn_perm(K64, hh, 0x04030402u)};
      f16x2v v[4];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        f16x2v t;
        __builtin_memcpy(&t, &pr[j], 4);
        t = t + k1024;  // q, exact
        v[j] = j < 2 ? __builtin_elementwise_fma(t, sa, ma) : __builtin_elementwise_fma(t, sb, mb);
      }
      __builtin_memcpy(&lo[2 * k], &v[0], 4);
      __builtin_memcpy(&lo[2 * k + 1], &v[1], 4);
      __builtin_memcpy(&hi[2 * k], &v[2], 4);
      __builtin_memcpy(&hi[2 * k + 1], &v[3], 4);
    }
    u32x4 *bd = reinterpret_cast<u32x4 *>(brow + 32 * half);
    bd[0] = u32x4{lo[0], lo[1], lo[2], lo[3]};
    bd[1] = u32x4{lo[4], lo[5], lo[6], lo[7]};
    u32x4 *bh = reinterpret_cast<u32x4 *>(brow + 64 + 32 * half);
    bh[0] = u32x4{hi[0], hi[1], hi[2], hi[3]};
    bh[1] = u32x4{hi[4], hi[5], hi[6], hi[7]};
  }
};

// GATED: a tile's 128 B rows are gate rows n0 .. n0 + 63 and the matching up rows (I + n0 ..),
// so waves 0-1 hold g and waves 2-3 u of the same 64 output columns; after the K loop waves 2-3
// pass u through LDS and waves 0-1 write act(g) * u (the values the ungated kernel followed by
// the split would give, bit for bit).
// f(integral_constant<int, I>) for I = 0, 1, ... while it returns true.
template <class F, int... I>
__device__ __forceinline__ void unroll_steps(F &&f, std::integer_sequence<int, I...>) {
  (void)(... && f(std::integral_constant<int, I>{}));
}

template <bool GATED>
__global__ __launch_bounds__(256) void moe_gemm_kernel(MoeGemmArgs ma) {
  using T = GTile<32>;
  extern __shared__ __align__(16) uint8_t smem[];
  const int e = blockIdx.y;
  const int seg0 = ma.offsets[e], seg1 = ma.offsets[e + 1];
  if (seg0 >= seg1) return;
  GemmArgs a = ma.g;
  a.w += (int64_t)e * ma.expert_bytes;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wn = wave;  // 4 waves along N, 32 columns each
  const int n0 = blockIdx.x * (GATED ? GBN / 2 : GBN);
  const int ksteps = a.K / GBK;
  const int acol = t & 7, arow = t >> 3;  // A: 32 rows x 128 B per step, one 16-byte load per thread
  const int wr = t >> 1, wh = t & 1;
  int wrow;
  if constexpr (GATED) {
    const int I = ma.gated_I, c = n0 + (wr & (GBN / 2 - 1));
    wrow = (wr >= GBN / 2 ? I : 0) + (c < I ? c : I - 1);
  } else {
    wrow = n0 + wr < a.N ? n0 + wr : a.N - 1;
  }
  const int fr = lane & 31, fk = (lane >> 5) * 8;

  for (int c0 = seg0; c0 < seg1; c0 += 32) {
    // Gathered activation row of this thread's A slot.
    int64_t pp = c0 + arow < seg1 ? ma.pairs[c0 + arow] : -1;
    const int64_t xr = (pp < 0 || pp >= ma.size_m) ? 0 : (ma.rpp ? pp : pp / ma.topk);
    const uint16_t *xrow = a.x + xr * a.K + acol * 8;

    f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; r++) acc[r] = 0.f;
    // Ring slot i holds the raw loads of a step congruent to i mod MD; loads past the last step
    // are clamped to it (unconditional, so the compiler's per-register waits stay exact).
    u32x4 ra[MD], hd, hcur;  // hd: slot 0's block header; hcur: the header being staged
    Q4kF16Slot wp[MD];
    // Loads per step and thread: x and the quant bytes, plus the block header in slot 0 (whose
    // steps start the 256-k blocks: K % 256 == 0), in this order.
    auto load = [&](int st, u32x4 &r, Q4kF16Slot &w, auto SLOT) __attribute__((always_inline)) {
      const int k = (st < ksteps ? st : ksteps - 1) * GBK;
      r = ldg16(xrow + k);
      w.load(a, wrow, wh, k);
      if constexpr (decltype(SLOT)::value == 0) hd = ldg16(Q4kF16Slot::block(a, wrow, k));
    };
    auto stage_in = [&](int buf, int st, const u32x4 &r, const Q4kF16Slot &w, auto SLOT) __attribute__((always_inline)) {
      if constexpr (decltype(SLOT)::value == 0) hcur = hd;
      uint8_t *na = smem + buf * T::STAGE;
      *reinterpret_cast<u32x4 *>(na + (arow * GLD + acol * 8) * 2) = r;
      w.store(na + T::A_BYTES + wr * GLD * 2, wh, (st < ksteps ? st : ksteps - 1) * GBK, hcur);
    };
    // The ring holds one step per slot, so when slot n is awaited the loads issued after its
    // own are one step of every other slot: 2 MD + 1 in all, less slot n's.
    auto wait_slot = [&](auto SLOT) __attribute__((always_inline)) {
      constexpr int n = decltype(SLOT)::value;
      if constexpr (n == 0)
        wait_ring<2 * MD + 1 - 3>(ra[0], wp[0].q, hd);
      else
        wait_ring<2 * MD + 1 - 2>(ra[n], wp[n].q);
    };
    unroll_steps([&](auto I) { return load(decltype(I)::value, ra[decltype(I)::value], wp[decltype(I)::value], I), true; },
                 std::make_integer_sequence<int, MD>{});
    wait_slot(std::integral_constant<int, 0>{});
    stage_in(0, 0, ra[0], wp[0], std::integral_constant<int, 0>{});
    __syncthreads();
    // Step s (ring slot s % MD, a compile-time constant): refill the slot with step s + MD,
    // multiply step s from LDS, stage step s + 1 (slot (s + 1) % MD) into the other buffer.
    // Slot 0 is refilled after step s + 1 .. s + 3 no longer need its header: hcur holds it.
    auto step = [&](int s, auto SLOT) __attribute__((always_inline)) {
      constexpr int slot = decltype(SLOT)::value, nslot = (slot + 1) % MD;
      load(s + MD, ra[slot], wp[slot], SLOT);
      wait_slot(std::integral_constant<int, nslot>{});
      const uint8_t *sa = smem + (s & 1) * T::STAGE;
      const uint8_t *sb = sa + T::A_BYTES;
#pragma unroll
      for (int kk = 0; kk < GBK / 16; kk++) {
        const f16x8 af = *reinterpret_cast<const f16x8 *>(sa + (fr * GLD + kk * 16 + fk) * 2);
        const f16x8 bfr = *reinterpret_cast<const f16x8 *>(sb + ((wn * 32 + fr) * GLD + kk * 16 + fk) * 2);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bfr, acc, 0, 0, 0);
      }
      if (s + 1 < ksteps) stage_in((s + 1) & 1, s + 1, ra[nslot], wp[nslot], std::integral_constant<int, nslot>{});
      __syncthreads();
    };
    // ksteps = K / 64 is a multiple of MD (Q4_K rows are whole 256-k blocks), so each trip runs
    // all MD steps: the loop has no exit between its steps, and every path that reaches the
    // loop head has issued the same loads.
    for (int s = 0; s < ksteps; s += MD)
      unroll_steps([&](auto I) { return step(s + decltype(I)::value, I), true; }, std::make_integer_sequence<int, MD>{});
    // The ring's last (clamped) loads land before its registers can be reused.
    wait_ring<0>(ra[0], wp[0].q, hd);
#pragma unroll
    for (int d = 1; d < MD; d++) wait_ring<0>(ra[d], wp[d].q);
    if constexpr (GATED) {
      // The stage buffers are free (the last step ended with a barrier): waves 2-3 leave u.
      float *ux = reinterpret_cast<float *>(smem);
      if (wn >= 2) {
#pragma unroll
        for (int r = 0; r < 16; r++) ux[((wn - 2) * 16 + r) * 64 + lane] = acc[r];
      }
      __syncthreads();
      const int col = n0 + wn * 32 + (lane & 31);
      if (wn < 2 && col < ma.gated_I) {
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int lr = 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
          const int i = c0 + lr;
          if (i >= seg1) continue;
          const int64_t p = ma.pairs[i];
          if (p < 0 || p >= ma.size_m) continue;
          const int64_t row = ma.rpp ? p : p / ma.topk;
          const float sc = ma.xscale[row];
          const float g = acc[r] * sc, u = ux[(wn * 16 + r) * 64 + lane] * sc;
          ma.out[p * ma.gated_I + col] = gate_act(g, ma.act) * u;
        }
      }
      __syncthreads();  // (u is read before the next chunk's stages overwrite it)
    } else {
      const int col = n0 + wn * 32 + (lane & 31);
      if (col < a.N) {
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int lr = 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
          const int i = c0 + lr;
          if (i >= seg1) continue;
          const int64_t p = ma.pairs[i];
          if (p < 0 || p >= ma.size_m) continue;
          const int64_t row = ma.rpp ? p : p / ma.topk;
          ma.out[p * a.N + col] = acc[r] * ma.xscale[row] * (ma.topk_w ? ma.topk_w[p] : 1.f);
        }
      }
    }
  }
}

// x (rows, K) F32 in, xh = f16 rows (rows * K * 2 bytes, 16-byte aligned) and xs = row scales
// (rows floats) in the workspace.
// gated_I > 0: N = 2 gated_I stacked gate / up rows, out (size_m, gated_I) = act(g) * u.
int launch_moe_gemm_q4k(const float *x, uint16_t *xh, float *xs, const void *w, const int64_t *pairs,
                        const int32_t *offsets, const float *topk_w, float *out, int topk, int64_t size_m,
                        int64_t rows, int64_t E, int64_t N, int64_t K, int rpp, hipStream_t s, int64_t gated_I,
                        int act, bool x_ready) {
  using T = GTile<32>;
  if (K % 256 || K <= 0) return fail(HQ_EINVAL, "moe_gemm_q4k", "K=%lld is not a multiple of 256", (long long)K);
  if (!x_ready) {
    to_f16_rowscale_kernel<<<(unsigned)rows, 256, 0, s>>>(x, reinterpret_cast<_Float16 *>(xh), xs, K);
    if (int rc = check_launch("to_f16_rowscale")) return rc;
  }
  if (moe_stream_ok(rows, size_m, N, K, gated_I))
    return launch_moe_stream_q4k(xh, xs, w, pairs, offsets, topk_w, out, topk, size_m, E, N, K, rpp, gated_I, act, s);
  MoeGemmArgs ma = {};
  ma.g.x = xh;
  ma.g.w = static_cast<const uint8_t *>(w);
  ma.g.N = (int)N;
  ma.g.K = (int)K;
  ma.xscale = xs;
  ma.pairs = pairs;
  ma.offsets = offsets;
  ma.topk_w = topk_w;
  ma.out = out;
  ma.size_m = size_m;
  ma.expert_bytes = N * (K / 256) * 144;
  ma.topk = topk;
  ma.rpp = rpp;
  ma.gated_I = (int)gated_I;
  ma.act = act;
  if (gated_I > 0) {
    dim3 grid((unsigned)cdiv(gated_I, GBN / 2), (unsigned)E);
    moe_gemm_kernel<true><<<grid, 256, T::LDS, s>>>(ma);
  } else {
    dim3 grid((unsigned)cdiv(N, GBN), (unsigned)E);
    moe_gemm_kernel<false><<<grid, 256, T::LDS, s>>>(ma);
  }
  return check_launch("moe_gemm_q4k");
}

// out[i] = sum_z part[z][i] in split order, converted to the output dtype.  Four outputs per
// thread (16-byte loads), and the splits' loads issued eight at a time before they are added
// (in split order): a load-add loop waits out one memory latency per split.
template <int ODT>
__device__ __forceinline__ void splitk_store(void *out, int64_t i, float v) {
  if constexpr (ODT == F32)
    static_cast<float *>(out)[i] = v;
  else if constexpr (ODT == BF16)
    static_cast<uint16_t *>(out)[i] = f2bf_rne(v);
  else
    static_cast<uint16_t *>(out)[i] = f2h_rne(v);
}

template <int ODT>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float *__restrict__ part, void *__restrict__ out,
                                                            int64_t n, int splits) {
  constexpr int U = 8;
  const int64_t i = 4 * ((int64_t)blockIdx.x * blockDim.x + threadIdx.x);
  if (i >= n) return;
  if (i + 4 <= n && (n & 3) == 0) {
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int z0 = 0; z0 < splits; z0 += U) {
      float4 v[U];
#pragma unroll
      for (int u = 0; u < U; u++)
        if (z0 + u < splits) v[u] = *reinterpret_cast<const float4 *>(part + (int64_t)(z0 + u) * n + i);
#pragma unroll
      for (int u = 0; u < U; u++)
        if (z0 + u < splits) {
          if (z0 + u == 0) {
            acc = v[u];
          } else {
            acc.x += v[u].x;
            acc.y += v[u].y;
            acc.z += v[u].z;
            acc.w += v[u].w;
          }
        }
    }
    splitk_store<ODT>(out, i, acc.x);
    splitk_store<ODT>(out, i + 1, acc.y);
    splitk_store<ODT>(out, i + 2, acc.z);
    splitk_store<ODT>(out, i + 3, acc.w);
    return;
  }
  for (int64_t e = i; e < n && e < i + 4; e++) {
    float s = part[e];
    for (int z = 1; z < splits; z++) s += part[(int64_t)z * n + e];
    splitk_store<ODT>(out, e, s);
  }
}

int launch_splitk_reduce(const float *part, void *out, int out_dtype, int64_t n, int splits, hipStream_t s) {
  dim3 rg((unsigned)cdiv(cdiv(n, 4), 256));
  switch (out_dtype) {
    case F32: splitk_reduce_kernel<F32><<<rg, 256, 0, s>>>(part, out, n, splits); break;
    case BF16: splitk_reduce_kernel<BF16><<<rg, 256, 0, s>>>(part, out, n, splits); break;
    default: splitk_reduce_kernel<F16><<<rg, 256, 0, s>>>(part, out, n, splits); break;
  }
  return check_launch("splitk_reduce");
}

// x (F32 or F16) -> bf16 (RNE).
template <int XDT>
__global__ __launch_bounds__(256) void to_bf16_kernel(const void *__restrict__ x, uint16_t *__restrict__ y,
                                                      int64_t n4) {
  // Four groups of four elements per thread, the block's 1024 groups contiguous; every load
  // goes out before the first conversion.
  constexpr int UN = 4;
  const int64_t i0 = (int64_t)blockIdx.x * (UN * 256) + threadIdx.x;
  float v[UN][4];
#pragma unroll
  for (int k = 0; k < UN; k++) {
    const int64_t i = i0 + k * 256 < n4 ? i0 + k * 256 : n4 - 1;
    if constexpr (XDT == F32) {
      const float4 f = static_cast<const float4 *>(x)[i];
      v[k][0] = f.x; v[k][1] = f.y; v[k][2] = f.z; v[k][3] = f.w;
    } else {
      const uint2 u = static_cast<const uint2 *>(x)[i];
      v[k][0] = h2f(u.x & 0xffffu); v[k][1] = h2f(u.x >> 16); v[k][2] = h2f(u.y & 0xffffu); v[k][3] = h2f(u.y >> 16);
    }
  }
#pragma unroll
  for (int k = 0; k < UN; k++)
    if (i0 + k * 256 < n4)
      reinterpret_cast<uint2 *>(y)[i0 + k * 256] = make_uint2(pack_bf16(v[k][0], v[k][1]), pack_bf16(v[k][2], v[k][3]));
}

// Prepared activations -> bf16 of d * q1 + e * q2.
__global__ __launch_bounds__(256) void act_to_bf16_kernel(const uint8_t *__restrict__ act, uint16_t *__restrict__ y,
                                                          int64_t n4, int64_t q2_off, int64_t d_off) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n4) return;
  const uint32_t q = reinterpret_cast<const uint32_t *>(act)[i];
  const uint32_t r = reinterpret_cast<const uint32_t *>(act + q2_off)[i];
  const float2 de = reinterpret_cast<const float2 *>(act + d_off)[i >> 3];
  float v[4];
#pragma unroll
  for (int j = 0; j < 4; j++)
    v[j] = de.x * (float)(int8_t)((q >> (8 * j)) & 0xff) + de.y * (float)(int8_t)((r >> (8 * j)) & 0xff);
  reinterpret_cast<uint2 *>(y)[i] = make_uint2(pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]));
}

// ---- host side ----------------------------------------------------------------

static int gemm_bm(int64_t M) { return M <= 64 ? 64 : 256; }

int gemm_splits(int64_t M, int64_t N, int64_t K) {
  // Split K until the grid fills the CUs: the 64-row tile (4 waves, 55 KB of LDS) up to two
  // workgroups per CU (int4 M = 64, 18944 x 3584: 63 -> 46 us), at most 8 splits.
  int64_t tiles = cdiv(M, gemm_bm(M)) * cdiv(N, GBN), steps = K / GBK;
  const int target = device_cus() * (gemm_bm(M) == 64 ? 2 : 1);
  int s = 1;
  while (tiles * (s * 2) <= target && steps / (s * 2) >= 8 && s < 8) s *= 2;
  return s;
}

size_t gemm_x_bytes(int64_t M, int64_t K) { return ((size_t)M * (size_t)K * 2 + 255) & ~(size_t)255; }

size_t gemm_ws_partial_bytes(int64_t M, int64_t N, int64_t K, bool f32_out);

// int4 at M <= 64 (gemm_small_int4_kernel): split K until about two workgroups per CU,
// keeping at least four 128-k stages per split.
int small_int4_splits(int64_t N, int64_t K) {
  const int64_t tiles = cdiv(N, 128), nst = K / SK;
  const int64_t target = 2 * (int64_t)device_cus();
  int s = 1;
  while (tiles * (s * 2) <= target && nst / (s * 2) >= 4 && s < 16) s *= 2;
  return s;
}

static bool small_int4_ok(int64_t M, int64_t K, int G) { return M <= 64 && K % SK == 0 && G % 32 == 0; }

size_t gemm_partial_bytes(int64_t M, int64_t N, int64_t K, bool f32_out) {
  int s = gemm_splits(M, N, K);
  size_t old = (s > 1 || !f32_out) ? (size_t)s * (size_t)M * (size_t)N * 4 : 0;
  if (M <= 64 && K % SK == 0) {
    const int s2 = std::max(small_int4_splits(N, K), i4f16_splits(N, K));
    old = std::max(old, (s2 > 1 || !f32_out) ? (size_t)s2 * (size_t)M * (size_t)N * 4 : (size_t)0);
  }
  return std::max(std::max(old, gemm_ws_partial_bytes(M, N, K, f32_out)), gemm_q4k2_ws_bytes(M, N, K));
}

static int launch_small_int4(const uint16_t *xb, const uint32_t *codes, const float *sc, const float *zr, void *out,
                             int out_dtype, float *partials, int64_t M, int64_t N, int64_t K, int G, hipStream_t s) {
  SmallI4Args a;
  a.x = xb;
  a.codes = codes;
  a.s = sc;
  a.z = zr;
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.G = G;
  a.splits = small_int4_splits(N, K);
  const bool direct = a.splits == 1 && out_dtype == F32;
  a.out = direct ? static_cast<float *>(out) : partials;
  dim3 grid((unsigned)cdiv(N, 128), 1, (unsigned)a.splits);
  if (G % 64 == 0)
    gemm_small_int4_kernel<true><<<grid, 256, 0, s>>>(a);
  else
    gemm_small_int4_kernel<false><<<grid, 256, 0, s>>>(a);
  if (int rc = check_launch("gemm_small_int4")) return rc;
  if (direct) return HQ_OK;
  return launch_splitk_reduce(partials, out, out_dtype, M * N, a.splits, s);
}

int launch_gemm_ws_q4k(const uint16_t *xb, const void *w, float *out, float *partials, int64_t M, int64_t N,
                       int64_t K, hipStream_t s);
int launch_gemm_ws_int4(const uint16_t *xb, const uint32_t *codes, const float *sc, const float *zr, void *out,
                        int out_dtype, float *partials, int64_t M, int64_t N, int64_t K, int G, hipStream_t s);

template <class WP, int BM>
static int launch_gemm_t(const GemmArgs &a0, int out_dtype, void *out, float *partials, hipStream_t s) {
  using T = GTile<BM>;
  static bool attr_set[64] = {false};
  int dev = 0;
  (void)hipGetDevice(&dev);
  if (dev >= 0 && dev < 64 && !attr_set[dev]) {
    if (int rc = check(hipFuncSetAttribute((const void *)gemm_kernel<WP, BM>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, T::LDS),
                       "hipFuncSetAttribute"))
      return rc;
    attr_set[dev] = true;
  }
  GemmArgs a = a0;
  a.tiles_m = (int)cdiv(a.M, BM);
  a.tiles_n = (int)cdiv(a.N, GBN);
  a.splits = gemm_splits(a.M, a.N, a.K);
  const int ntiles = a.tiles_m * a.tiles_n;
  a.xcd_map = ntiles % 8 == 0;
  const bool direct = a.splits == 1 && out_dtype == F32;
  a.out = direct ? static_cast<float *>(out) : partials;
  dim3 grid((unsigned)ntiles, 1, (unsigned)a.splits);
  gemm_kernel<WP, BM><<<grid, 256, T::LDS, s>>>(a);
  if (int rc = check_launch("gemm")) return rc;
  if (direct) return HQ_OK;
  return launch_splitk_reduce(partials, out, out_dtype, (int64_t)a.M * a.N, a.splits, s);
}

// M <= 64 only (larger M takes the warp-specialised kernel of gemm_ws.hip).
template <class WP>
static int launch_gemm_p(const GemmArgs &a, int out_dtype, void *out, float *partials, hipStream_t s) {
  return launch_gemm_t<WP, 64>(a, out_dtype, out, partials, s);
}

int launch_gemm_q4k_bf16(const uint16_t *xb, const void *w, float *out, float *partials, int64_t M, int64_t N,
                         int64_t K, hipStream_t s) {
  // M > 64: the all-waves Q4_K kernel (gemm_q4k.hip), else the warp-specialised kernel
  // (gemm_ws.hip); small M keeps the 64-row tile.
  if (gemm_q4k_ok(M, N, K, w, xb)) return launch_gemm_q4k2(xb, w, out, partials, M, N, K, s);
  if (M > 64) return launch_gemm_ws_q4k(xb, w, out, partials, M, N, K, s);
  GemmArgs a = {};
  a.x = xb;
  a.w = static_cast<const uint8_t *>(w);
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.G = 256;
  return launch_gemm_p<Q4kPolicy>(a, F32, out, partials, s);
}

int launch_gemm_int4_bf16(const uint16_t *xb, const uint32_t *codes, const float *sc, const float *zr, void *out,
                          int out_dtype, float *partials, int64_t M, int64_t N, int64_t K, int G, hipStream_t s) {
  if (M > 64) return launch_gemm_ws_int4(xb, codes, sc, zr, out, out_dtype, partials, M, N, K, G, s);
  if (small_int4_ok(M, K, G)) return launch_small_int4(xb, codes, sc, zr, out, out_dtype, partials, M, N, K, G, s);
  GemmArgs a = {};
  a.x = xb;
  a.w = reinterpret_cast<const uint8_t *>(codes);
  a.s = sc;
  a.z = zr;
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.G = G;
  return launch_gemm_p<Int4Policy>(a, out_dtype, out, partials, s);
}

size_t gemm_q4k_ws_bytes(int64_t M, int64_t K) { return gemm_x_bytes(M, K); }
size_t gemm_q4k_partial_bytes(int64_t M, int64_t N, int64_t K) { return gemm_partial_bytes(M, N, K, true); }

int launch_to_bf16(const void *src, int src_kind, uint16_t *dst, int64_t M, int64_t K, hipStream_t s) {
  int64_t n4 = M * K / 4;
  dim3 g((unsigned)cdiv(n4, 256)), g4((unsigned)cdiv(n4, 1024));
  switch (src_kind) {
    case F32: to_bf16_kernel<F32><<<g4, 256, 0, s>>>(src, dst, n4); break;
    case F16: to_bf16_kernel<F16><<<g4, 256, 0, s>>>(src, dst, n4); break;
    case BF16:
      return check(hipMemcpyAsync(dst, src, (size_t)M * K * 2, hipMemcpyDeviceToDevice, s), "hipMemcpyAsync");
    default:  // prepared activations
      act_to_bf16_kernel<<<g, 256, 0, s>>>(static_cast<const uint8_t *>(src), dst, n4, act_q2_off(M, K),
                                           act_d_off(M, K));
      break;
  }
  return check_launch("to_bf16");
}

}  // namespace hq
