// gemm_ws.hip -- warp-specialised quantized-weight GEMM on MFMA (gfx950).
//
// Role: the many-row leg of Light's quantized matmuls (matmul_q for M >= 8,
// ops/matmul_q.go:52-59, 85-95; MatMulInt4 for M > 8, ops/int4.go:100-126), fused:
// out[m, n] = sum_k x[m, k] * dequant(W)[n, k] with bf16 x and bf16-rounded weights.
//
// Design (one 512-thread workgroup per CU, tile BM x 128 x 64):
//  * Producer waves (4-7) move data; consumer waves (0-3) only read LDS and issue
//    v_mfma_f32_32x32x16_bf16.  The two roles run concurrently on every SIMD.
//  * A (bf16 x) and the raw weight bytes reach LDS by direct global->LDS loads
//    (global_load_lds_dwordx4): no registers, NA / NR stages deep.  These loads are
//    issued from inline asm with their wait counts managed here: the compiler would
//    otherwise wait for every LDS DMA before any LDS access, which serialises the
//    pipeline.
//  * Producers dequantize the raw bytes of step s+1 (Q4_K: (d*sc)*q - dmin*m; int4:
//    s*(q - z)) while consumers run step s, writing bf16 B in MFMA operand order.
//  * A is stored row-major, 128 bytes (64 k) per row, with the eight 16-byte pieces of
//    row r at piece ^ (r % 8): each direct load fills 8 whole rows from 8 full cache
//    lines, and the fragment reads (32 rows x one piece) hit 8 distinct bank groups.
//    B is stored in MFMA fragment order: a 1 KB block holds one 32-row x 16-k fragment,
//    lane l's 16 bytes at l*16, so its reads are contiguous.
//  * One barrier per K step.  Workgroup -> tile mapping keeps the M tiles of a
//    weight tile on one XCD (its L2 serves the second read of the weights).
#include "dma.hpp"
#include "internal.hpp"

namespace hq {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int WBN = 128, WBK = 64;
constexpr int NR = 4;                 // raw weight stages (loads issued NR-1 steps ahead)
constexpr int B_STAGE = WBN * WBK * 2;  // 16 KB of bf16 B, two stages

// WF::R_WAVE: raw bytes per producer wave per stage.  WF::DIRECT: the raw stage already is
// bf16 B in fragment order (no dequant step, no separate B stages).
template <int BM, class WF>
struct WsTile {
  static constexpr int A_STAGE = BM * WBK * 2;         // bf16 A per step
  static constexpr int NA = BM == 256 ? 3 : 5;          // A stages (loads issued NA-1 steps ahead)
  static constexpr int A_BLOCKS = BM / 8;                // 1 KB (8-row) blocks per step
  static constexpr int A_PER_WAVE = A_BLOCKS / 4;       // direct loads per producer wave per step
  static constexpr int WM = BM == 256 ? 2 : 2, WN = 2;  // consumer waves along M / N
  static constexpr int MT = BM / WM / 32, NT = WBN / WN / 32;
  static constexpr int R_STAGE = 4 * WF::R_WAVE;
  static constexpr int R_OFF = NA * A_STAGE;
  static constexpr int B_OFF = R_OFF + NR * R_STAGE;
  static constexpr int LDS = B_OFF + (WF::DIRECT ? 0 : 2 * B_STAGE);
};

__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
  bf16x2 v = {(__bf16)a, (__bf16)b};
  uint32_t u;
  __builtin_memcpy(&u, &v, 4);
  return u;
}

}  // namespace

struct WsArgs {
  const uint16_t *x;   // bf16 [M][K]
  const uint8_t *w;    // Q4_K blocks (N, K) or int4 codes (N, K/8)
  const float *s, *z;  // int4 scales / zeros (N, K/G)
  float *out;          // [M][N] or split partials [S][M][N]
  int M, N, K, G;
  int tiles_m, tiles_n, splits, xcd_map;
  int64_t row_bytes;
};

// ---- weight formats: raw bytes of one row and one 64-wide K step --------------
// Q4_K: qs bytes [32p, 32p+32) of super-block k0/256 (p = (k0/64) % 4) and the 16-byte
// block header.  Producer wave layout per stage: [0, 1 KB) qs, chunk (row r, half h) at
// (32h + r) * 16; [1 KB, 2 KB) headers, row r at 1024 + 16 r.
struct WsQ4k {
  static constexpr int RAW_LOADS = 2;  // direct loads per producer wave per step
  static constexpr int R_WAVE = 2048;  // 1 KB qs + 1 KB headers
  static constexpr bool DIRECT = false;
  __device__ static void issue_raw(const WsArgs &a, int row_base, int lane, int k0, uint32_t dst) {
    const int p = (k0 >> 6) & 3;
    const int64_t blk = (int64_t)(k0 >> 8) * 144;
    int r = row_base + (lane & 31);
    r = r < a.N ? r : a.N - 1;
    const uint8_t *rp = a.w + (int64_t)r * a.row_bytes + blk;
    dma16(rp + 16 + 32 * p + 16 * (lane >> 5), dst);
    int r2 = row_base + (lane & 31);
    r2 = r2 < a.N ? r2 : a.N - 1;
    dma16(a.w + (int64_t)r2 * a.row_bytes + blk, dst + 1024);
  }
  // Thread (row r of the wave's 32, half h): 32 weights of k = 16h + i (low nibbles,
  // sub-block 2p) and 32 + 16h + i (high nibbles, sub-block 2p+1), i < 16.
  __device__ static void dequant(const WsArgs &a, const uint8_t *raw, int r, int h, int k0, float out_lo[16],
                                 float out_hi[16]) {
    const u32x4 q = *reinterpret_cast<const u32x4 *>(raw + (32 * h + r) * 16);
    const u32x4 hd = *reinterpret_cast<const u32x4 *>(raw + 1024 + 16 * r);
    const int p = (k0 >> 6) & 3;
    const float d = h2f(hd[0] & 0xffffu), dmin = h2f(hd[0] >> 16);
    int scA, mnA, scB, mnB;
    q4k_scale_min(2 * p, hd[1], hd[2], hd[3], scA, mnA);
    q4k_scale_min(2 * p + 1, hd[1], hd[2], hd[3], scB, mnB);
    const float dA = d * (float)scA, mA = dmin * (float)mnA, dB = d * (float)scB, mB = dmin * (float)mnB;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const uint32_t l = q[k] & 0x0F0F0F0Fu, hh = (q[k] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        out_lo[4 * k + j] = dA * (float)((l >> (8 * j)) & 0xff) - mA;
        out_hi[4 * k + j] = dB * (float)((hh >> (8 * j)) & 0xff) - mB;
      }
    }
  }
};

// int4 (quant.Int4, G % 64 == 0): codes words [k0/8, k0/8 + 8) of a row (32 bytes), the
// group's scale and zero.  Layout: [0, 1 KB) codes, (row r, half h) at (32h + r) * 16;
// [1 KB, 1 KB + 128) scales, [1 KB + 128, 1 KB + 256) zeros.
struct WsInt4 {
  static constexpr int RAW_LOADS = 2;
  static constexpr int R_WAVE = 2048;
  static constexpr bool DIRECT = false;
  __device__ static void issue_raw(const WsArgs &a, int row_base, int lane, int k0, uint32_t dst) {
    int r = row_base + (lane & 31);
    r = r < a.N ? r : a.N - 1;
    dma16(a.w + (int64_t)r * (a.K / 2) + (k0 >> 1) + 16 * (lane >> 5), dst);
    int r2 = row_base + (lane & 31);
    r2 = r2 < a.N ? r2 : a.N - 1;
    const int64_t gi = (int64_t)r2 * (a.K / a.G) + k0 / a.G;
    dma4(lane < 32 ? (const void *)(a.s + gi) : (const void *)(a.z + gi), dst + 1024);
  }
  // Thread (row r, half h): codes bytes [16h, 16h+16) = k 32h + i, i < 32 (nibble order).
  // Low 16 -> kk = 2h, high 16 -> kk = 2h + 1 (out_lo / out_hi).
  __device__ static void dequant(const WsArgs &a, const uint8_t *raw, int r, int h, int, float out_lo[16],
                                 float out_hi[16]) {
    const u32x4 q = *reinterpret_cast<const u32x4 *>(raw + (32 * h + r) * 16);
    const float s = reinterpret_cast<const float *>(raw + 1024)[r];
    const float z = reinterpret_cast<const float *>(raw + 1024)[32 + r];
#pragma unroll
    for (int k = 0; k < 4; k++)
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const float v = s * ((float)((q[k] >> (4 * j)) & 15) - z);
        if (k < 2)
          out_lo[8 * k + j] = v;
        else
          out_hi[8 * (k - 2) + j] = v;
      }
  }
};

// bf16 weights (N, K) row-major (a GGUF format dequantized once, bit-exact, to bf16): the
// wave's 32 rows x 64 k land by direct loads straight in MFMA fragment order, 1 KB per
// 16-k piece kk: lane l holds row l % 32, k = 16 kk + 8 (l / 32) .. + 8.
struct WsBf16 {
  static constexpr int RAW_LOADS = 4;
  static constexpr int R_WAVE = 4096;
  static constexpr bool DIRECT = true;
  __device__ static void issue_raw(const WsArgs &a, int row_base, int lane, int k0, uint32_t dst) {
#pragma unroll
    for (int kk = 0; kk < 4; kk++) {
      int r = row_base + (lane & 31);
      r = r < a.N ? r : a.N - 1;
      dma16(a.w + (int64_t)r * a.row_bytes + 2 * (k0 + 16 * kk + 8 * (lane >> 5)), dst + 1024 * kk);
    }
  }
  __device__ static void dequant(const WsArgs &, const uint8_t *, int, int, int, float *, float *) {}
};

template <class WF, int BM>
__global__ __launch_bounds__(512) void gemm_ws_kernel(WsArgs a) {
  using T = WsTile<BM, WF>;
  extern __shared__ __align__(16) uint8_t smem[];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const uint32_t lds0 = (uint32_t)(uintptr_t)smem;

  int tile = blockIdx.x;
  const int ntiles = a.tiles_m * a.tiles_n;
  if (a.xcd_map) tile = (blockIdx.x % 8) * (ntiles / 8) + blockIdx.x / 8;
  const int tm = tile % a.tiles_m, tn = tile / a.tiles_m;
  const int m0 = tm * BM, n0 = tn * WBN;
  const int ksteps = a.K / WBK;
  const int st0 = (int)((int64_t)ksteps * blockIdx.z / a.splits);
  const int st1 = (int)((int64_t)ksteps * (blockIdx.z + 1) / a.splits);
  const int nsteps = st1 - st0;
  if (nsteps <= 0) return;

  if (wave >= 4) {
    // ---------------- producers ----------------
    const int pw = wave - 4;
    const int pt = t - 256;                 // 0..255
    const int bh = (pt >> 5) & 1;           // half of the row's 32 raw bytes
    const int br = pw * 32 + (lane & 31);   // B row (0..127)
    const int rrow = br & 31;               // row within the wave's 32
    // Step index -> clamped global K offset (steps past the end reload the last step into
    // a stage that is never consumed, which keeps every iteration's load count fixed).
    auto kofs = [&](int st) { return (st0 + (st < nsteps ? st : nsteps - 1)) * WBK; };
    auto issue = [&](int st) {
      // Raw weights of step st, then A of step st - (NR - T::NA) ... both at fixed counts.
      const int k0 = kofs(st);
      WF::issue_raw(a, n0 + pw * 32, lane, k0,
                    __builtin_amdgcn_readfirstlane(lds0 + T::R_OFF + (st % NR) * T::R_STAGE + pw * WF::R_WAVE));
    };
    auto issue_a = [&](int st) {
      const int k0 = kofs(st);
      const uint32_t base = lds0 + (st % T::NA) * T::A_STAGE;
#pragma unroll
      for (int j = 0; j < T::A_PER_WAVE; j++) {
        const int bi = pw * T::A_PER_WAVE + j;  // rows 8 bi .. 8 bi + 7
        const int lr = bi * 8 + (lane >> 3);
        const int piece = (lane & 7) ^ (lr & 7);
        int row = m0 + lr;
        row = row < a.M ? row : a.M - 1;
        dma16(a.x + (int64_t)row * a.K + k0 + piece * 8, __builtin_amdgcn_readfirstlane(base + bi * 1024));
      }
    };
    auto dequant = [&](int st) {
      if constexpr (WF::DIRECT) return;
      const uint8_t *raw = smem + T::R_OFF + (st % NR) * T::R_STAGE + pw * WF::R_WAVE;
      float lo[16], hi[16];
      WF::dequant(a, raw, rrow, bh, kofs(st), lo, hi);
      uint8_t *bs = smem + T::B_OFF + (st & 1) * B_STAGE;
      const int nt = br >> 5;
      // Q4_K: lo -> kk = bh, hi -> kk = 2 + bh; int4: lo -> kk = 2bh, hi -> kk = 2bh + 1.
      int kkl, kkh;
      if constexpr (__is_same(WF, WsQ4k)) {
        kkl = bh;
        kkh = 2 + bh;
      } else {
        kkl = 2 * bh;
        kkh = 2 * bh + 1;
      }
#pragma unroll
      for (int half = 0; half < 2; half++) {
        const u32x4 vl = {pk_bf16(lo[8 * half], lo[8 * half + 1]), pk_bf16(lo[8 * half + 2], lo[8 * half + 3]),
                          pk_bf16(lo[8 * half + 4], lo[8 * half + 5]), pk_bf16(lo[8 * half + 6], lo[8 * half + 7])};
        const u32x4 vh = {pk_bf16(hi[8 * half], hi[8 * half + 1]), pk_bf16(hi[8 * half + 2], hi[8 * half + 3]),
                          pk_bf16(hi[8 * half + 4], hi[8 * half + 5]), pk_bf16(hi[8 * half + 6], hi[8 * half + 7])};
        *reinterpret_cast<u32x4 *>(bs + ((nt * 4 + kkl) * 64 + half * 32 + rrow) * 16) = vl;
        *reinterpret_cast<u32x4 *>(bs + ((nt * 4 + kkh) * 64 + half * 32 + rrow) * 16) = vh;
      }
    };
    // Per iteration i, loads are issued in a fixed order: raw(i + NR - 1), then A(i + NA - 1).
    // The prologue runs iterations -(P) .. -1 (P = max(NR, NA) - 1) issuing the loads whose
    // step is >= 0; from iteration 1 - NR on every iteration is full (NA >= NR - 1), which
    // the loop's wait counts rely on.
    static_assert(T::NA >= NR - 1, "wait counts assume NA >= NR - 1");
    constexpr int PER_IT = WF::RAW_LOADS + T::A_PER_WAVE;
    constexpr int P = (NR > T::NA ? NR : T::NA) - 1;
    for (int i = -P; i < 0; i++) {
      if (i + NR - 1 >= 0) issue(i + NR - 1);
      if (i + T::NA - 1 >= 0) issue_a(i + T::NA - 1);
    }
    // raw(0) and A(0) complete.  NA = 3: A(0) (iteration -2) is followed by iteration -1.
    // NA = 5: raw(0) (iteration -3) is followed by A(1) and iterations -2, -1.
    if constexpr (T::NA == 3)
      wait_vm<PER_IT>();
    else
      wait_vm<T::A_PER_WAVE + 2 * PER_IT>();
    dequant(0);
    __syncthreads();
    for (int s = 0; s < nsteps; s++) {
      issue(s + NR - 1);
      issue_a(s + T::NA - 1);
      if (s + 1 < nsteps) {
        // raw(s+1) was issued NR-2 iterations ago; its A part and the later iterations follow.
        wait_vm<T::A_PER_WAVE + PER_IT * (NR - 2)>();
        dequant(s + 1);  // (DIRECT: nothing to convert; the wait alone publishes B(s+1))
      }
      // A(s+1): issued NA-2 iterations ago, followed by the later iterations' loads.
      wait_vm<PER_IT * (T::NA - 2)>();
      __syncthreads();
    }
    wait_vm<0>();
  } else {
    // ---------------- consumers ----------------
    const int wm = wave / T::WN, wn = wave % T::WN;
    f32x16 acc[T::MT][T::NT];
#pragma unroll
    for (int i = 0; i < T::MT; i++)
#pragma unroll
      for (int j = 0; j < T::NT; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;
    __syncthreads();  // matches the producers' prologue barrier
    // A fragment (row, k piece c): byte (row * 128) + ((c ^ (row % 8)) * 16) of the stage.
    const int fr = lane & 31, fh = lane >> 5;
    for (int s = 0; s < nsteps; s++) {
      const uint8_t *sa = smem + (s % T::NA) * T::A_STAGE;
      const uint8_t *sb = WF::DIRECT ? smem + T::R_OFF + (s % NR) * T::R_STAGE : smem + T::B_OFF + (s & 1) * B_STAGE;
      bf16x8 af[2][T::MT], bfr[2][T::NT];
#define WS_LOAD_FRAGS(BUF, KK)                                                                          \
  do {                                                                                                  \
    _Pragma("unroll") for (int i = 0; i < T::MT; i++) {                                                 \
      const int row = (wm * T::MT + i) * 32 + fr;                                                      \
      af[BUF][i] = *reinterpret_cast<const bf16x8 *>(sa + row * 128 + ((((KK) * 2 + fh) ^ (row & 7)) << 4)); \
    }                                                                                                   \
    _Pragma("unroll") for (int j = 0; j < T::NT; j++)                                                  \
      bfr[BUF][j] = *reinterpret_cast<const bf16x8 *>(sb + (((wn * T::NT + j) * 4 + (KK)) * 64 + lane) * 16); \
  } while (0)
      WS_LOAD_FRAGS(0, 0);
#pragma unroll
      for (int kk = 0; kk < 4; kk++) {
        if (kk < 3) WS_LOAD_FRAGS((kk + 1) & 1, kk + 1);
#pragma unroll
        for (int i = 0; i < T::MT; i++)
#pragma unroll
          for (int j = 0; j < T::NT; j++)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[kk & 1][i], bfr[kk & 1][j], acc[i][j], 0, 0, 0);
      }
#undef WS_LOAD_FRAGS
      __syncthreads();
    }
    // Epilogue: lane holds D[8*(r/4) + 4*(lane/32) + r%4][lane%32] of each 32x32 tile.
    float *out = a.out + (int64_t)blockIdx.z * a.M * a.N;
#pragma unroll
    for (int i = 0; i < T::MT; i++)
#pragma unroll
      for (int j = 0; j < T::NT; j++) {
        const int col = n0 + (wn * T::NT + j) * 32 + (lane & 31);
        if (col >= a.N) continue;
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int row = m0 + (wm * T::MT + i) * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
          if (row < a.M) out[(int64_t)row * a.N + col] = acc[i][j][r];
        }
      }
  }
}

// ---- host side ------------------------------------------------------------------

static int ws_bm(int64_t M) { return M > 128 ? 256 : 128; }

static int ws_splits(int64_t M, int64_t N, int64_t K) {
  const int64_t tiles = cdiv(M, ws_bm(M)) * cdiv(N, WBN), steps = K / WBK;
  const int target = device_cus();
  int s = 1;
  while (tiles * (s * 2) <= target && steps / (s * 2) >= 8) s *= 2;
  return s;
}

size_t gemm_ws_partial_bytes(int64_t M, int64_t N, int64_t K, bool f32_out) {
  const int s = ws_splits(M, N, K);
  return (s > 1 || !f32_out) ? (size_t)s * (size_t)M * (size_t)N * 4 : 0;
}

int launch_splitk_reduce(const float *part, void *out, int out_dtype, int64_t n, int splits, hipStream_t s);

template <class WF, int BM>
static int launch_ws_t(WsArgs a, int out_dtype, void *out, float *partials, hipStream_t s) {
  using T = WsTile<BM, WF>;
  static bool attr_set[64] = {false};
  int dev = 0;
  (void)hipGetDevice(&dev);
  if (dev >= 0 && dev < 64 && !attr_set[dev]) {
    if (int rc = check(hipFuncSetAttribute((const void *)gemm_ws_kernel<WF, BM>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, T::LDS),
                       "hipFuncSetAttribute"))
      return rc;
    attr_set[dev] = true;
  }
  a.tiles_m = (int)cdiv(a.M, BM);
  a.tiles_n = (int)cdiv(a.N, WBN);
  a.splits = ws_splits(a.M, a.N, a.K);
  const int ntiles = a.tiles_m * a.tiles_n;
  a.xcd_map = ntiles % 8 == 0;
  const bool direct = a.splits == 1 && out_dtype == F32;
  a.out = direct ? static_cast<float *>(out) : partials;
  dim3 grid((unsigned)ntiles, 1, (unsigned)a.splits);
  gemm_ws_kernel<WF, BM><<<grid, 512, T::LDS, s>>>(a);
  if (int rc = check_launch("gemm_ws")) return rc;
  if (direct) return HQ_OK;
  return launch_splitk_reduce(partials, out, out_dtype, (int64_t)a.M * a.N, a.splits, s);
}

template <class WF>
static int launch_ws(const WsArgs &a, int out_dtype, void *out, float *partials, hipStream_t s) {
  if (ws_bm(a.M) == 128) return launch_ws_t<WF, 128>(a, out_dtype, out, partials, s);
  return launch_ws_t<WF, 256>(a, out_dtype, out, partials, s);
}

int launch_gemm_ws_q4k(const uint16_t *xb, const void *w, float *out, float *partials, int64_t M, int64_t N,
                       int64_t K, hipStream_t s) {
  WsArgs a = {};
  a.x = xb;
  a.w = static_cast<const uint8_t *>(w);
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.G = 256;
  a.row_bytes = K / 256 * 144;
  return launch_ws<WsQ4k>(a, F32, out, partials, s);
}

int launch_gemm_ws_bf16(const uint16_t *xb, const uint16_t *wb, float *out, float *partials, int64_t M, int64_t N,
                        int64_t K, hipStream_t s) {
  WsArgs a = {};
  a.x = xb;
  a.w = reinterpret_cast<const uint8_t *>(wb);
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.G = 0;
  a.row_bytes = K * 2;
  return launch_ws<WsBf16>(a, F32, out, partials, s);
}

int launch_gemm_ws_int4(const uint16_t *xb, const uint32_t *codes, const float *sc, const float *zr, void *out,
                        int out_dtype, float *partials, int64_t M, int64_t N, int64_t K, int G, hipStream_t s) {
  WsArgs a = {};
  a.x = xb;
  a.w = reinterpret_cast<const uint8_t *>(codes);
  a.s = sc;
  a.z = zr;
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.G = G;
  a.row_bytes = K / 2;
  return launch_ws<WsInt4>(a, out_dtype, out, partials, s);
}

}  // namespace hq
