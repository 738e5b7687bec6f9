// int4_small.hip -- GPTQ / AWQ int4 matmul for 8 < M <= 64 rows of F16 activations on f16 MFMA.
//
// Role: Light's MatMulInt4 for prefill-sized M (ops/int4.go:100-126: int4_dequant into
// scratch + cuBLAS), fused: y (M, N) = x (M, K) . W^T, W = s * (q - z) (quant.Int4, group G).
//
// Design (gfx950, 512 threads = 8 waves, 64 rows x 256 weight rows per workgroup, 128-k stages):
//  * The weight is never rounded: the MFMA's B operand holds q - z exactly -- a nibble masked
//    in place and OR'd into the f16 exponent pattern 0x6400 (one v_and_or_b32) is 1024 + q
//    (nibbles 0, 2 of a byte pair) or 1024 + 16 q (nibbles 1, 3, whose x pairs are staged
//    divided by 16, exact), and one packed f16 add of -(1024 + z) or -(1024 + 16 z) leaves
//    q - z or 16 (q - z) (integral zero points, as in every GPTQ / AWQ checkpoint; other zero
//    points take a second add, still within f16 precision) -- and the group scale multiplies
//    the stage's f32 MFMA sum afterwards (acc += s * C, one FMA per output per group; stages
//    never straddle a group, G % 128 == 0).  About 1.1 VALU instructions per weight.
//  * Each lane streams its own weight row's codes (32 contiguous bytes per stage) straight
//    into registers, three stages ahead, with its group's scale and zero; x (64 x 128 f16 per
//    stage) is loaded three stages ahead into registers too and goes through LDS,
//    double-buffered, shared by the eight waves.  x is re-read by every column tile, so the
//    tile is wide (256 weight rows): x traffic was twice the weight traffic at 128.  The loads are issued from inline asm and
//    waited for with explicit vmcnt counts (the compiler would wait for every outstanding load
//    at the loop's back edge).
//  * The two halves of a wave take the two 64-k halves of a stage, and inside each 8-k slice
//    the k order is (0, 4, 1, 5, 2, 6, 3, 7) -- the order the nibble pairs (i, i + 4) of a code
//    word unpack in -- for A (x, permuted once while staged into LDS) and B alike, so the sum
//    is unchanged and every code load is a contiguous 16 bytes.
//  * K is split over grid.z until the grid fills the chip; partial tiles go to f32 slices,
//    summed in slice order by splitk_reduce_kernel.
#include "internal.hpp"

namespace hq {

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int IK = 128, IXLD = IK + 8;  // stage k; x stage row stride (f16), padded
constexpr int ID = 3;                   // weight stages in flight

struct I4F16Args {
  const uint16_t *x;      // f16 (M, K)
  const uint32_t *codes;  // (N, K/8)
  const float *s, *z;     // (N, K/G)
  float *part;            // [splits][M][N] f32
  int M, N, K, G, splits;
};

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ u32x4 ld16(const void *p) {
  u32x4 r;
  asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(r) : "v"(p) : "memory");
  return r;
}
// Wait until at most N loads of this wave are outstanding; the registers named become
// defined only here, so no use of them can be scheduled before the wait.
template <int N>
__device__ __forceinline__ void wait_w(u32x4 &a, u32x4 &b) {
  asm volatile("s_waitcnt vmcnt(%2)" : "+v"(a), "+v"(b) : "n"(N) : "memory");
}
template <int N>
__device__ __forceinline__ void wait_x(u32x4 &a, u32x4 &b) {
  asm volatile("s_waitcnt vmcnt(%2)" : "+v"(a), "+v"(b) : "n"(N) : "memory");
}
#pragma clang diagnostic pop

// (x_i, x_{i+1}) f16 pairs of an 8-k slice -> the (0, 4, 1, 5, 2, 6, 3, 7) order, with the
// pairs (1, 5) and (3, 7) divided by 16 (exact): their weights enter the MFMA as 16 (q - z).
__device__ __forceinline__ u32x4 perm8(const u32x4 v) {
  const f16x2 s16 = {(_Float16)0.0625f, (_Float16)0.0625f};
  uint32_t p1 = __builtin_amdgcn_perm(v[2], v[0], 0x07060302u), p3 = __builtin_amdgcn_perm(v[3], v[1], 0x07060302u);
  f16x2 h1, h3;
  __builtin_memcpy(&h1, &p1, 4);
  __builtin_memcpy(&h3, &p3, 4);
  h1 = h1 * s16;
  h3 = h3 * s16;
  __builtin_memcpy(&p1, &h1, 4);
  __builtin_memcpy(&p3, &h3, 4);
  return u32x4{__builtin_amdgcn_perm(v[2], v[0], 0x05040100u), p1, __builtin_amdgcn_perm(v[3], v[1], 0x05040100u), p3};
}

// (w & mask) | 0x64006400 in one instruction.
__device__ __forceinline__ uint32_t and_or_6400(uint32_t w, uint32_t mask, uint32_t magic) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(w), "s"(mask), "v"(magic));
  return r;
}

}  // namespace

__global__ __launch_bounds__(512) void gemm_i4f16_small_kernel(I4F16Args a) {
  // x stages, then the scales / zeros (sized by the launch: IXS_EXTRA bytes).
  extern __shared__ __align__(16) uint16_t xsm[];
  uint16_t(*xs)[64 * IXLD] = reinterpret_cast<uint16_t(*)[64 * IXLD]>(xsm);
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int kh = lane >> 5, fr = lane & 31;
  const int n0 = blockIdx.x * 256 + wave * 32;
  const int row = n0 + fr < a.N ? n0 + fr : a.N - 1;  // this lane's weight row (clamped)
  const int nst = a.K / IK;
  const int c0 = (int)((int64_t)nst * blockIdx.z / a.splits), c1 = (int)((int64_t)nst * (blockIdx.z + 1) / a.splits);
  const int ng = a.K / a.G;
  const uint32_t *crow = a.codes + (int64_t)row * (a.K / 8) + 8 * kh;  // + 16 words per stage
  // x staging: thread t -> row t / 8, 16-k eighth t % 8 (two 16-byte loads).  Rows past M
  // load row 0 and are stored as zeros.
  const int xr = t >> 3, xq = t & 7;
  const bool xok = xr < a.M;
  const uint16_t *xsrc = a.x + (int64_t)(xok ? xr : 0) * a.K + xq * 16;

  // The split's scales and zeros of the workgroup's 256 weight rows go to LDS once: one load
  // per row and group instead of per lane and stage (those scattered dword loads were most
  // of the kernel's cache requests).  Groups [g0, g1) of K / G.
  const int g0 = c0 * IK / a.G, g1 = (c1 * IK + a.G - 1) / a.G, ngl = g1 - g0;
  float *lsz = reinterpret_cast<float *>(&xs[2][0]);  // [2][256][ngl]
  for (int i = t; i < 256 * ngl; i += 512) {
    const int r = i / ngl, gg = i - r * ngl;
    const int wr = blockIdx.x * 256 + r < a.N ? blockIdx.x * 256 + r : a.N - 1;
    lsz[i] = a.s[(int64_t)wr * ng + g0 + gg];
    lsz[256 * ngl + i] = a.z[(int64_t)wr * ng + g0 + gg];
  }
  // Loads of stage c (clamped into the split's range, so the counts never change).
  auto cl = [&](int c) { return c < c1 ? c : c1 - 1; };
  u32x4 cw[ID][2];
  auto load_w = [&](int c, int slot) __attribute__((always_inline)) {
    const int cc = cl(c);
    cw[slot][0] = ld16(crow + cc * 16);
    cw[slot][1] = ld16(crow + cc * 16 + 4);
  };
  u32x4 xv[ID][2];
  auto load_x = [&](int c, int slot) __attribute__((always_inline)) {
    const uint16_t *p = xsrc + (int64_t)cl(c) * IK;
#pragma unroll
    for (int i = 0; i < 2; i++) xv[slot][i] = ld16(p + 8 * i);
  };
  auto store_x = [&](int buf, int slot) __attribute__((always_inline)) {
    uint16_t *d = &xs[buf][xr * IXLD + xq * 16];
#pragma unroll
    for (int i = 0; i < 2; i++)
      *reinterpret_cast<u32x4 *>(d + 8 * i) = xok ? perm8(xv[slot][i]) : u32x4{0, 0, 0, 0};
  };

  f32x16 acc[2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int r = 0; r < 16; r++) acc[i][r] = 0.f;
  if (c0 >= c1) return;  // (whole workgroup: c0, c1 are uniform)

  // Prologue: x and the weights of stages c0 .. c0 + ID - 1, all landed before the loop (the
  // in-loop counts assume full stages of loads after the ones awaited).
#pragma unroll
  for (int d = 0; d < ID; d++) {
    load_x(c0 + d, d);
    load_w(c0 + d, d);
  }
#pragma unroll
  for (int d = 0; d < ID; d++) {
    wait_x<0>(xv[d][0], xv[d][1]);
    wait_w<0>(cw[d][0], cw[d][1]);
  }
  store_x(0, 0);
  __syncthreads();  // (also publishes the scales / zeros)

  // One stage c (ring slot c - c0 mod ID): its weights are awaited (loads after them: the
  // ID - 1 later stages' four each -- two x, two weight -- stages c < c0 + ID were awaited in
  // the prologue), the 8 MFMA steps run on x(c) in LDS, the group scale is applied, the slot
  // is refilled with x and weights of stage c + ID, x(c + 1) is awaited (loads after it: its
  // stage's two weight loads and the ID - 1 later stages' four each) and stored, then the
  // barrier.
  auto stage = [&](int c, auto SLOT) __attribute__((always_inline)) {
    constexpr int slot = decltype(SLOT)::value, nslot = (slot + 1) % ID;
    const int buf = (c - c0) & 1;
    wait_w<4 * (ID - 1)>(cw[slot][0], cw[slot][1]);
    if (c < c1) {  // (uniform) a padding stage past the split only keeps the ring's loads and waits
      const int gl = c * IK / a.G - g0, lr = wave * 32 + fr;
      const float sgv = lsz[lr * ngl + gl], zgv = lsz[256 * ngl + lr * ngl + gl];
      const uint16_t *xa = &xs[buf][0];
      // Nibbles i = 0, 2 enter as 1024 + q, nibbles 1, 3 as 1024 + 16 q (masked in place, no
      // shift; the x pairs they meet were staged / 16).  Integral zero points (every GPTQ / AWQ
      // checkpoint's): one packed add of -(1024 + z) or -(1024 + 16 z) leaves q - z or 16 (q - z)
      // exactly.  Otherwise (a wave-uniform test) -1024 first, exact, then -z or -16 z.
      const bool zint = __all(zgv == rintf(zgv) && fabsf(zgv) <= 64.f);
      const uint32_t magic = __builtin_amdgcn_readfirstlane(0x64006400u);
      f32x16 cacc[2];
      auto mfma_stage = [&](auto ZI) __attribute__((always_inline)) {
        constexpr bool zi = decltype(ZI)::value;
        const f16x2 c0v = {(_Float16)(zi ? -1024.f - zgv : -1024.f), (_Float16)(zi ? -1024.f - zgv : -1024.f)};
        const f16x2 c0v16 = {(_Float16)(zi ? -1024.f - 16.f * zgv : -1024.f),
                             (_Float16)(zi ? -1024.f - 16.f * zgv : -1024.f)};
        const f16x2 zf = {(_Float16)-zgv, (_Float16)-zgv}, zf16 = {(_Float16)(-16.f * zgv), (_Float16)(-16.f * zgv)};
#pragma unroll
        for (int j = 0; j < 8; j++) {
          const uint32_t w = cw[slot][j >> 2][j & 3], w8 = w >> 8;
          const uint32_t pr[4] = {and_or_6400(w, 0x000F000Fu, magic), and_or_6400(w, 0x00F000F0u, magic),
                                  and_or_6400(w8, 0x000F000Fu, magic), and_or_6400(w8, 0x00F000F0u, magic)};
          f16x8 b;
#pragma unroll
          for (int i = 0; i < 4; i++) {
            f16x2 h;
            __builtin_memcpy(&h, &pr[i], 4);
            h = h + ((i & 1) ? c0v16 : c0v);
            if constexpr (!zi) h = h + ((i & 1) ? zf16 : zf);
            b[2 * i] = h[0];
            b[2 * i + 1] = h[1];
          }
          const int kx = 64 * kh + 8 * j;
          const f16x8 a0 = *reinterpret_cast<const f16x8 *>(xa + fr * IXLD + kx);
          const f16x8 a1 = *reinterpret_cast<const f16x8 *>(xa + (32 + fr) * IXLD + kx);
          if (j == 0) {
            const f32x16 zero = {};
            cacc[0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, b, zero, 0, 0, 0);
            cacc[1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, b, zero, 0, 0, 0);
          } else {
            cacc[0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, b, cacc[0], 0, 0, 0);
            cacc[1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, b, cacc[1], 0, 0, 0);
          }
        }
      };
      if (zint)
        mfma_stage(std::true_type{});
      else
        mfma_stage(std::false_type{});
      const float sc = sgv;
#pragma unroll
      for (int i = 0; i < 2; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[i][r] = __fmaf_rn(sc, cacc[i][r], acc[i][r]);
    }
    load_x(c + ID, slot);
    load_w(c + ID, slot);
    wait_x<2 + 4 * (ID - 1)>(xv[nslot][0], xv[nslot][1]);
    store_x(buf ^ 1, nslot);
    __syncthreads();
  };
  // Every trip runs all ID stages (the last trip's stages past c1 are padding), so each path
  // to the loop head has issued the same loads and the hand-counted waits hold on all of them.
  static_assert(ID == 3, "the trip below unrolls ID stages");
  for (int c = c0; c < c1; c += ID) {
    stage(c, std::integral_constant<int, 0>{});
    stage(c + 1, std::integral_constant<int, 1>{});
    stage(c + 2, std::integral_constant<int, 2>{});
  }
  // The last (clamped) prefetches land before their registers can be reused.
#pragma unroll
  for (int d = 0; d < ID; d++) {
    wait_x<0>(xv[d][0], xv[d][1]);
    wait_w<0>(cw[d][0], cw[d][1]);
  }

  // Lane holds D[8 (r / 4) + 4 (lane / 32) + r % 4][lane % 32] of each 32 x 32 tile (m, n).
  float *out = a.part + (int64_t)blockIdx.z * a.M * a.N;
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

int launch_splitk_reduce(const float *part, void *out, int out_dtype, int64_t n, int splits, hipStream_t s);
int i4f16_splits(int64_t N, int64_t K);

// LDS of one workgroup: the double-buffered x stage, then the scales and zeros of the 256
// weight rows over the groups one split can touch (its stages' span of K / G, plus one for a
// group boundary).
static size_t i4f16_lds(int64_t N, int64_t K, int G) {
  const int64_t nst = K / IK, maxst = cdiv(nst, i4f16_splits(N, K));
  const int64_t ngl = (maxst * IK + G - 1) / G + 1;
  return 2 * 64 * IXLD * 2 + 2 * 256 * (size_t)ngl * 4;
}

// Shapes past the LDS (many groups per split) take the bf16 GEMM instead.
bool i4f16_small_ok(int64_t M, int64_t N, int64_t K, int G, int x_dtype, const void *x, const void *codes) {
  return x_dtype == F16 && M > 8 && M <= 64 && K % IK == 0 && G % IK == 0 && K % G == 0 && N >= 1 &&
         ((uintptr_t)x & 15) == 0 && ((uintptr_t)codes & 15) == 0 && i4f16_lds(N, K, G) <= 160 * 1024;
}

// K split: one workgroup fits a CU (133 registers, eight waves), so the split minimising
// (rounds of workgroups over the CUs) x (stages per split) wins, with a 2% charge per split
// for the partial traffic and at least 4 stages per split (18944 x 3584: 3 splits, 222
// workgroups -- 4 splits made 296, and the 40 CUs holding two ran twice as long).
int i4f16_splits(int64_t N, int64_t K) {
  const int64_t tiles = cdiv(N, 256), nst = K / IK, cus = device_cus();
  int best = 1;
  double bc = 1e300;
  for (int s = 1; s <= 32 && nst / s >= 4; s++) {
    const double c = (double)cdiv(tiles * s, cus) * cdiv(nst, s) * (1.0 + 0.02 * s);
    if (c < bc) {
      bc = c;
      best = s;
    }
  }
  return best;
}

int launch_i4f16_small(const uint16_t *x, const uint32_t *codes, const float *s, const float *z, void *y,
                       float *partials, int64_t M, int64_t N, int64_t K, int G, hipStream_t st) {
  I4F16Args a;
  a.x = x;
  a.codes = codes;
  a.s = s;
  a.z = z;
  a.part = partials;
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.G = G;
  a.splits = i4f16_splits(N, K);
  dim3 grid((unsigned)cdiv(N, 256), 1, (unsigned)a.splits);
  const size_t lds = i4f16_lds(N, K, G);
  if (lds > 160 * 1024) return fail(HQ_EUNSUPPORTED, "int4_matmul", "LDS %zu bytes", lds);
  gemm_i4f16_small_kernel<<<grid, 512, lds, st>>>(a);
  if (int rc = check_launch("gemm_i4f16_small")) return rc;
  return launch_splitk_reduce(partials, y, F16, M * N, a.splits, st);
}

}  // namespace hq
