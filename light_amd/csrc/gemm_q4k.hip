// gemm_q4k.hip -- Q4_K prefill GEMM on MFMA (gfx950): out (M, N) F32 = x (M, K) . dequant(W)^T
// with x rounded to bf16 and each weight dequantized in F32 and rounded once to bf16.
//
// Role: the many-row leg of Light's matmul_q (ops/matmul_q.go:52-59, 85-95: dequant + cuBLAS
// SGEMM on CUDA), fused: the dequantized weight never exists in HBM.
//
// Design (one 512-thread workgroup per CU, tile 256 x BN, BN = 112 or 128, K step 64):
//  * Wave w owns rows [64 (w % 4), 64 (w % 4) + 64) x BN columns over one 32-wide half
//    (w / 4) of every 64-wide K step; the two waves of a row group sit on the same SIMD, so
//    one's fragment reads and dequant overlap the other's MFMAs, and each wave's 64 x BN
//    tile reads 0.39 LDS fragments per v_mfma_f32_16x16x32_bf16.  Their two accumulators
//    are added once, after the K loop.
//  * Per step s every wave (1) issues its direct global->LDS loads of A (bf16 x) for step
//    s + 2 and of the raw Q4_K bytes for step s + 3, (2) dequantizes its share of step
//    s + 1's raw bytes into the bf16 B tile of the other buffer, (3) runs its 28 or 32 MFMAs
//    of step s and (4) waits for its own loads of A(s+1) and raw(s+2); one barrier per step.
//  * BN = 112 gives N = 14336 exactly 128 column tiles, so M = 512 is 256 tiles: one per CU.
//  * A is row-major in LDS, 128 bytes (64 k) per row, the eight 16-byte pieces of row r at
//    piece ^ (r % 8).  B is stored in MFMA fragment order (a 1 KB block per 16 columns and
//    32-wide half, lane l's 16 bytes at l * 16).
//  * Raw bytes per step and row: the 32 quant bytes of the super-block pair the step covers
//    and the block's 16-byte header (d, dmin, 12 scale bytes).  A thread dequantizes 16
//    weights (a quarter of one row's step): (d * sc) * q - dmin * m in F32, rounded to bf16
//    (RNE).  Threads past the tile's 4 * BN tasks write a pad slot (no branch).
//  * K may be split over grid.z; partial tiles then go to F32 slices of the workspace, added in
//    slice order by splitk_reduce_kernel (an in-kernel "last workgroup adds" reduction, with
//    its agent-scope fences, measured slower).
#include "dma.hpp"
#include "internal.hpp"

namespace hq {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int QBM = 256, QBK = 64, QTHREADS = 512;
constexpr int QNA = 3, QNR = 4;  // A stages (loads 2 steps ahead), raw stages (3 ahead)

template <int BN>
struct QT {
  static constexpr int NJ = BN / 16;
  static constexpr int A_STAGE = QBM * QBK * 2;          // 32 KB
  static constexpr int R_STAGE = 6 * 1024;               // 3 * BN 16-byte entries (+ pad)
  static constexpr int B_STAGE = BN * QBK * 2 + 1024;    // 14 / 16 KB + a pad block
  static constexpr int R_OFF = QNA * A_STAGE;
  static constexpr int B_OFF = R_OFF + QNR * R_STAGE;
  static constexpr int LDS = B_OFF + 2 * B_STAGE;       // 150 / 154 KB
  static_assert(4 * 64 * BN * 4 <= LDS, "the final accumulator exchange fits in the stages");
};

__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  bf16x2 v = {(__bf16)a, (__bf16)b};
  uint32_t u;
  __builtin_memcpy(&u, &v, 4);
  return u;
}

}  // namespace

struct Q4kGemmArgs {
  const uint16_t *x;  // bf16 [M][K]
  const uint8_t *w;   // Q4_K blocks (N, K)
  float *out;         // [M][N]
  float *part;        // split-K slices [splits][M][N] (splits > 1)
  int M, N, K, splits, tiles_m;
  int64_t row_bytes;
};

template <int BN>
__global__ __launch_bounds__(QTHREADS) void gemm_q4k_kernel(Q4kGemmArgs a) {
  using T = QT<BN>;
  extern __shared__ __align__(16) uint8_t smem[];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int rg = wave & 3, kh = wave >> 2;  // row group, K half
  const uint32_t lds0 = (uint32_t)(uintptr_t)smem;
  const int tm = blockIdx.x % a.tiles_m, tn = blockIdx.x / a.tiles_m;
  const int m0 = tm * QBM, n0 = tn * BN;
  const int ksteps = a.K / QBK;
  const int st0 = (int)((int64_t)ksteps * blockIdx.z / a.splits);
  const int st1 = (int)((int64_t)ksteps * (blockIdx.z + 1) / a.splits);
  const int nsteps = st1 - st0;  // >= 1 (the host keeps splits <= ksteps)

  // Per-thread load sources, fixed for the kernel.  A: wave w loads rows [32 w, 32 w + 32),
  // four direct loads of 8 rows (lane -> row lane / 8, piece (lane % 8) ^ (row % 8)).
  const uint16_t *asrc[4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int lr = wave * 32 + j * 8 + (lane >> 3);
    const int piece = (lane & 7) ^ (lr & 7);
    const int row = m0 + lr < a.M ? m0 + lr : a.M - 1;
    asrc[j] = a.x + (int64_t)row * a.K + (int64_t)st0 * QBK + piece * 8;
  }
  // Raw: entry e < 2 BN is quant half (e & 1) of row e >> 1, then BN headers, then padding;
  // wave w loads entries [64 w', 64 w' + 64) with w' = w for w < 6, w - 6 otherwise (waves 6
  // and 7 repeat loads 0 and 1: the same bytes to the same place).
  const int rli = wave < 6 ? wave : wave - 6;
  const uint8_t *bsrc;
  int bqs;  // 1: a quant entry (offset by the pair), 0: a header
  {
    const int e = rli * 64 + lane;
    int n;
    if (e < 2 * BN) {
      n = e >> 1;
      bqs = 1;
    } else {
      n = e - 2 * BN < BN ? e - 2 * BN : 0;
      bqs = 0;
    }
    const int row = n0 + n < a.N ? n0 + n : a.N - 1;
    bsrc = a.w + (int64_t)row * a.row_bytes + (bqs ? 16 + 16 * (e & 1) : 0);
  }
  auto clamp = [&](int st) { return st < nsteps ? st : nsteps - 1; };
  auto issue_a = [&](int st) {
    const int k = clamp(st) * QBK;
    const uint32_t base = lds0 + (st % QNA) * T::A_STAGE + wave * 32 * 128;
#pragma unroll
    for (int j = 0; j < 4; j++) dma16(asrc[j] + k, __builtin_amdgcn_readfirstlane(base + j * 8 * 128));
  };
  auto issue_b = [&](int st) {
    const int kg = st0 + clamp(st);  // global 64-wide step: super-block kg / 4, pair kg % 4
    const uint8_t *src = bsrc + (int64_t)(kg >> 2) * 144 + (bqs ? 32 * (kg & 3) : 0);
    dma16(src, __builtin_amdgcn_readfirstlane(lds0 + T::R_OFF + (st % QNR) * T::R_STAGE + rli * 1024));
  };
  // Dequant task t < 4 BN: row tn_ = t / 4, weights 16 tq .. 16 tq + 15 of the step (tq = t % 4):
  // low nibbles of quant bytes 16 tq .. (sub-block 2p) for tq < 2, high nibbles of bytes
  // 16 (tq - 2) .. (sub-block 2p + 1) otherwise.  They fill B fragment (j = tn_ / 16, half
  // tq / 2), lane groups 2 (tq % 2) and 2 (tq % 2) + 1.
  const bool task_ok = t < 4 * BN;
  const int tn_ = task_ok ? t >> 2 : 0, tq = t & 3;
  const int thh = tq >> 1;  // which nibble / sub-block of the pair
  const uint32_t b_slot = task_ok ? (uint32_t)(((thh * T::NJ + (tn_ >> 4)) * 64 + (tq & 1) * 32 + (tn_ & 15)) * 16)
                                  : (uint32_t)(BN * QBK * 2 + (lane & 31) * 16);
  struct Raw {
    u32x4 q, hd;
  };
  auto dequant_load = [&](int st) {
    const uint8_t *raw = smem + T::R_OFF + (st % QNR) * T::R_STAGE;
    Raw r;
    r.q = *reinterpret_cast<const u32x4 *>(raw + tn_ * 32 + (tq & 1) * 16);
    r.hd = *reinterpret_cast<const u32x4 *>(raw + (2 * BN + tn_) * 16);
    return r;
  };
  auto dequant_store = [&](int st, const Raw &r) {
    const int p = (st0 + clamp(st)) & 3;
    const float d = h2f(r.hd[0] & 0xffffu), dmin = h2f(r.hd[0] >> 16);
    int sc, mn;
    q4k_scale_min(2 * p + thh, r.hd[1], r.hd[2], r.hd[3], sc, mn);
    const float dA = d * (float)sc, mA = dmin * (float)mn;
    uint8_t *bs = smem + T::B_OFF + (st & 1) * T::B_STAGE + b_slot;
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const uint32_t l0 = (r.q[2 * h] >> (4 * thh)) & 0x0F0F0F0Fu, l1 = (r.q[2 * h + 1] >> (4 * thh)) & 0x0F0F0F0Fu;
      float v[8];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        v[i] = dA * (float)((l0 >> (8 * i)) & 0xffu) - mA;
        v[4 + i] = dA * (float)((l1 >> (8 * i)) & 0xffu) - mA;
      }
      const u32x4 o = {pk_bf16(v[0], v[1]), pk_bf16(v[2], v[3]), pk_bf16(v[4], v[5]), pk_bf16(v[6], v[7])};
      *reinterpret_cast<u32x4 *>(bs + h * 256) = o;
    }
  };
  auto dequant = [&](int st) { dequant_store(st, dequant_load(st)); };

  f32x4 acc[4][T::NJ];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < T::NJ; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Prologue: raw(0..2) and A(0..1), all landed, then B(0).
  issue_b(0);
  issue_a(0);
  issue_b(1);
  issue_a(1);
  issue_b(2);
  wait_vm<0>();
  __syncthreads();
  dequant(0);
  __syncthreads();

  const int fr = lane & 15, fg = lane >> 4;
  uint32_t a_rd[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int r = rg * 64 + i * 16 + fr;
    a_rd[i] = (uint32_t)(r * 128 + ((((kh << 2) + fg) ^ (r & 7)) << 4));
  }
  const uint32_t b_rd = (uint32_t)((kh * T::NJ * 64 + lane) * 16);
  for (int s = 0; s < nsteps; s++) {
    issue_a(s + 2);
    issue_b(s + 3);
    const uint8_t *sa = smem + (s % QNA) * T::A_STAGE;
    const uint8_t *sb = smem + T::B_OFF + (s & 1) * T::B_STAGE + b_rd;
    // LDS reads in the order they are consumed (the raw bytes for the dequant, A, then B
    // fragment by fragment), so each consumer waits only for its own reads.
    const Raw rw = dequant_load(s + 1);
    bf16x8 af[4], bfr[T::NJ];
#pragma unroll
    for (int i = 0; i < 4; i++) af[i] = *reinterpret_cast<const bf16x8 *>(sa + a_rd[i]);
#pragma unroll
    for (int j = 0; j < T::NJ; j++) bfr[j] = *reinterpret_cast<const bf16x8 *>(sb + j * 1024);
    dequant_store(s + 1, rw);
#pragma unroll
    for (int j = 0; j < T::NJ; j++)
#pragma unroll
      for (int i = 0; i < 4; i++)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    // A(s+1) and raw(s+2) were issued one iteration ago, followed by this iteration's five.
    wait_vm<5>();
    __syncthreads();
  }
  wait_vm<0>();
  __syncthreads();  // every wave's last (clamped) loads have landed before LDS is reused

  // The K-half-1 waves hand their accumulators to the K-half-0 waves through LDS (the stages
  // are free now): wave 4 + rg's lane l, value (i, j, r) at ((rg * 4 + i) * NJ + j) * 256 +
  // r * 64 + l floats.
  float *xch = reinterpret_cast<float *>(smem);
  if (kh == 1) {
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < T::NJ; j++)
#pragma unroll
        for (int r = 0; r < 4; r++) xch[((rg * 4 + i) * T::NJ + j) * 256 + r * 64 + lane] = acc[i][j][r];
  }
  __syncthreads();
  const bool split = a.splits > 1;
  if (kh == 0) {
    float *dst = split ? a.part + (int64_t)blockIdx.z * a.M * a.N : a.out;
    // Lane holds D[4 (lane / 16) + r][lane % 16] of each 16 x 16 tile.
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < T::NJ; j++) {
        const int col = n0 + j * 16 + fr;
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const float v = acc[i][j][r] + xch[((rg * 4 + i) * T::NJ + j) * 256 + r * 64 + lane];
          const int row = m0 + rg * 64 + i * 16 + fg * 4 + r;
          if (row < a.M && col < a.N) dst[(int64_t)row * a.N + col] = v;
        }
      }
  }
}

// ---- host side ------------------------------------------------------------------

// Tile width and K split: the pair minimising (waves of tiles over the CUs) x (tile width) x
// (K steps per split), with a 5% charge for the split's partial traffic.
static void q4k_plan(int64_t M, int64_t N, int64_t K, int *bn_out, int *s_out) {
  const int64_t cus = device_cus(), steps = K / QBK;
  double best = 1e300;
  for (int bn : {112, 128}) {
    const int64_t tiles = cdiv(M, QBM) * cdiv(N, bn);
    for (int s = 1; s <= 8 && s <= steps; s++) {
      if (s > 1 && steps / s < 8) break;
      const double cost = (double)cdiv(tiles * s, cus) * bn * cdiv(steps, s) * (s > 1 ? 1.05 : 1.0) *
                          (N % bn ? 1.02 : 1.0);
      if (cost < best) {
        best = cost;
        *bn_out = bn;
        *s_out = s;
      }
    }
  }
}

bool gemm_q4k_ok(int64_t M, int64_t N, int64_t K, const void *w, const void *x) {
  return M > 64 && K % 256 == 0 && N % 4 == 0 && N >= 16 && N < INT32_MAX && M < INT32_MAX &&
         ((uintptr_t)w & 15) == 0 && ((uintptr_t)x & 15) == 0;
}

size_t gemm_q4k2_ws_bytes(int64_t M, int64_t N, int64_t K) {
  int bn = 128, s = 1;
  q4k_plan(M, N, K, &bn, &s);
  if (s <= 1) return 0;
  return ((size_t)s * M * N * 4 + 255) & ~(size_t)255;
}

template <int BN>
static int launch_q4k_t(Q4kGemmArgs a, hipStream_t s) {
  using T = QT<BN>;
  static bool attr_set[64] = {false};
  int dev = 0;
  (void)hipGetDevice(&dev);
  if (dev >= 0 && dev < 64 && !attr_set[dev]) {
    if (int rc = check(hipFuncSetAttribute((const void *)gemm_q4k_kernel<BN>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, T::LDS),
                       "hipFuncSetAttribute"))
      return rc;
    attr_set[dev] = true;
  }
  a.tiles_m = (int)cdiv(a.M, QBM);
  const int ntiles = a.tiles_m * (int)cdiv(a.N, BN);
  dim3 grid((unsigned)ntiles, 1, (unsigned)a.splits);
  gemm_q4k_kernel<BN><<<grid, QTHREADS, T::LDS, s>>>(a);
  return check_launch("gemm_q4k");
}

int launch_splitk_reduce(const float *part, void *out, int out_dtype, int64_t n, int splits, hipStream_t s);

// ws: gemm_q4k2_ws_bytes(M, N, K) bytes (the split-K slices).
int launch_gemm_q4k2(const uint16_t *xb, const void *w, float *out, void *ws, int64_t M, int64_t N, int64_t K,
                     hipStream_t s) {
  Q4kGemmArgs a = {};
  a.x = xb;
  a.w = static_cast<const uint8_t *>(w);
  a.out = out;
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.row_bytes = K / 256 * 144;
  int bn = 128, splits = 1;
  q4k_plan(M, N, K, &bn, &splits);
  a.splits = splits;
  if (a.splits > 1) a.part = static_cast<float *>(ws);
  if (int rc = bn == 112 ? launch_q4k_t<112>(a, s) : launch_q4k_t<128>(a, s)) return rc;
  if (a.splits == 1) return HQ_OK;
  return launch_splitk_reduce(a.part, out, F32, M * N, a.splits, s);
}

}  // namespace hq
