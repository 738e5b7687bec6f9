// int4_cu.hip -- GPTQ / AWQ int4 matmul for 8 < M <= 64 rows of F16 activations when the
// weight's 80-row column tiles fill the chip: one workgroup per CU over all of K, no split-K
// partials, no second launch.
//
// Role: Light's MatMulInt4 for prefill-sized M (ops/int4.go:100-126: int4_dequant into
// scratch + cuBLAS), fused: y (M, N) = x (M, K) . W^T, W = s * (q - z) (quant.Int4, group G).
//
// Design (gfx950, 512 threads = 8 waves, two per SIMD, one workgroup per CU):
//  * A workgroup owns 80 weight rows (five 16-row MFMA tiles).  The eight waves split its
//    128-k chunks (waves w and w + 4 share SIMD w % 4 and take consecutive shares, so every
//    SIMD holds the same number of chunks to within one), so every x and weight byte the
//    workgroup reads goes to exactly one wave and the waves never wait for each other inside
//    the K loop.  Each wave accumulates the whole 16 MT x 80 tile over its chunks.
//  * A CU's streaming rate is bounded by its memory requests more than by bytes (a load
//    costs about the same per cache line it touches), so x is fetched in whole 128-byte
//    lines: 8 lanes per x row, straight into the wave's LDS ring (global_load_lds_dwordx4, 64 k
//    x 16 MT rows per unit, two units), with the line's 16-byte pieces XOR-swizzled by
//    (row / 2) % 8 so the MFMA fragment reads are conflict-free.  The weight codes go straight
//    into registers: one 16-byte load per lane and tile brings the lane's four code words of a
//    chunk, one chunk ahead.
//  * MFMA v_mfma_f32_16x16x32_f16.  Step s of a chunk multiplies, in lane group q = lane / 16,
//    the 8 k values 32 s + 8 q + [0, 8).  The lane loaded words 4 q + [0, 4) of its weight
//    row's chunk; a 4 x 4 transpose across the lane groups (v_permlane32_swap,
//    v_permlane16_swap) hands lane group q word 4 s + q for step s.
//  * Dequant, four VALU instructions per pair of weights: v_perm_b32 puts the code byte in
//    both halves under an 0x64 exponent byte, an AND keeps the low nibble in the low half and
//    the high nibble in the high half (f16 1024 + q0 and 1024 + 16 q1, exact), a packed FMA
//    by (1, 1/16) with -(1024 + z), -(64 + z) leaves q0 - z, q1 - z exactly (integral zero
//    points, as in every GPTQ / AWQ checkpoint; otherwise -1024, -64 leave q exactly), and a
//    packed FMA by s' (and + (-z s') for other zero points) gives the f16 weight s' (q - z),
//    rounded once.  s' = s 2^e, with 2^e per wave and weight row chosen so the row's largest
//    scale lands in [16, 32): the f16 weights stay clear of the subnormal range, and the
//    row's sum is multiplied by 2^-e (exact) at the end.  (MFMA and VALU work of a SIMD
//    overlap only partly on gfx950, so the VALU count per weight is what the dequant trims.)
//  * Every wave issues its scale / zero loads before a barrier and only then its ring loads,
//    so the CU's request queue serves all scales first.  Loads are issued from inline asm and
//    awaited with explicit vmcnt counts; the loop runs whole trips of two chunks (the second
//    chunk of the last trip may be padding that only keeps the loads and waits), so the
//    counts hold on every path.
//  * The eight waves' tiles are added in LDS in a fixed order, ((w0 + w4) + (w1 + w5)) +
//    ((w2 + w6) + (w3 + w7)), four outputs per thread.
#include "internal.hpp"

namespace hq {

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int CK = 128;            // k per chunk
constexpr int NT = 5;              // 16-row weight tiles per workgroup
constexpr int NR = 16 * NT;        // weight rows per workgroup
constexpr int NW = 8;              // waves per workgroup, two per SIMD
constexpr int NTH = 64 * NW;
constexpr int DB = 2;              // weight chunks in each wave's register ring
constexpr int XU = 2;              // x units (64 k) in each wave's LDS ring
constexpr int RP = NR + 4;         // reduction row pitch (floats)
constexpr int RPW = NR / NW;       // weight rows per wave whose scales / zeros it stages

struct I4CuArgs {
  const uint16_t *x;      // f16 (M, K)
  const uint32_t *codes;  // (N, K/8)
  const float *s, *z;     // (N, K/G)
  uint16_t *y;            // f16 (M, N)
  int M, N, K, G;
};

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// 16 bytes per lane from base (SGPRs) + a 32-bit byte offset + an immediate, into registers.
template <int IMM>
__device__ __forceinline__ u32x4 ld16s(const void *base, uint32_t off) {
  u32x4 r;
  asm volatile("global_load_dwordx4 %0, %1, %2 offset:%3" : "=v"(r) : "v"(off), "s"(base), "n"(IMM) : "memory");
  return r;
}
__device__ __forceinline__ uint32_t ld4(const void *p) {
  uint32_t r;
  asm volatile("global_load_dword %0, %1, off" : "=v"(r) : "v"(p) : "memory");
  return r;
}
// 16 bytes per lane from base + off into LDS at m0 + 16 lane.  (No immediate offset: on an
// LDS DMA load it moves the LDS destination too.)
__device__ __forceinline__ void dma16s(const void *base, uint32_t off, uint32_t m0) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(m0) : "memory", "m0");
}
#pragma clang diagnostic pop

template <int N>
__device__ __forceinline__ void wait_vmem() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ __forceinline__ f16x2 as_h2(uint32_t v) {
  f16x2 h;
  __builtin_memcpy(&h, &v, 4);
  return h;
}
__device__ __forceinline__ uint32_t as_u(f16x2 h) {
  uint32_t v;
  __builtin_memcpy(&v, &h, 4);
  return v;
}

template <int V>
using ic = std::integral_constant<int, V>;

}  // namespace


template <int MT>
__global__ __launch_bounds__(NTH) void int4_cu_kernel(I4CuArgs a) {
  constexpr int XROWS = 16 * MT;      // x rows staged (rows past M repeat row M - 1)
  constexpr int XUB = XROWS * 128;    // bytes per x unit: XROWS rows x 64 k
  constexpr int XIN = XROWS / 8;      // LDS DMA instructions per unit (8 rows each)
  constexpr int XWB = XU * XUB;       // bytes of one wave's ring
  extern __shared__ __align__(16) unsigned char lds[];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int q = lane >> 4, r16 = lane & 15;
  const int n0 = blockIdx.x * NR;
  const int C = a.K / CK, ng = a.K / a.G;
  // The K / G groups' scales and zeros are staged after the x rings with an odd row pitch (the
  // 16 rows a lane group reads fall in distinct banks).
  const int sp = ng | 1;
  float *ls = reinterpret_cast<float *>(lds + NW * XWB), *lz = ls + NR * sp;
  // This wave's chunks [cb, ce): SIMD w % 4 holds waves w and w + 4, which take consecutive
  // shares (each SIMD gets the same number of chunks to within one).
  const int p = 2 * (wave & 3) + (wave >> 2);
  const int cb = (int)((int64_t)C * p / NW), ce = (int)((int64_t)C * (p + 1) / NW);
  const int n = ce - cb;
  const int clast = n > 0 ? ce - 1 : 0;  // loads past the range are clamped here
  auto chunk = [&](int k) { return k < n ? cb + k : clast; };

  // Scales / zeros of the workgroup's rows, issued by every wave ahead of any ring load: wave w
  // stages rows w, w + NW, ..., one row per load with the lane as the group (K / G <= 64).
  const int gl = lane < ng ? lane : ng - 1;
  uint32_t sv[RPW], zv[RPW];
#pragma unroll
  for (int i = 0; i < RPW; i++) {
    const int r = wave + NW * i;
    const int wr = n0 + r < a.N ? n0 + r : a.N - 1;
    sv[i] = ld4(a.s + (int64_t)wr * ng + gl);
    zv[i] = ld4(a.z + (int64_t)wr * ng + gl);
  }
  __syncthreads();

  // x DMA: instruction ii of a unit loads rows 8 ii + lane / 8; the lane's LDS slot holds
  // 16-byte piece p = lane % 8 of the row's 128 bytes, filled from logical piece p ^ f(row),
  // f(row) = (row / 2) % 8.  Byte offsets from x (under 2 GiB).
  uint32_t xg[XIN];
#pragma unroll
  for (int ii = 0; ii < XIN; ii++) {
    const int row = 8 * ii + (lane >> 3);
    const int m = row < a.M ? row : a.M - 1;
    const int piece = (lane & 7) ^ ((row >> 1) & 7);
    xg[ii] = (uint32_t)(((int64_t)m * a.K + 8 * piece) * 2);
  }
  const uint32_t xring = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds + (uint32_t)(wave * XWB));
  // Unit u = 2 k + h of this wave: chunk k, k half h (64 k), into ring slot SLOT.
  auto load_xu = [&](int k, auto H, auto SLOT) __attribute__((always_inline)) {
    const uint32_t off = (uint32_t)chunk(k) * (CK * 2) + 128 * decltype(H)::value;
#pragma unroll
    for (int ii = 0; ii < XIN; ii++) dma16s(a.x, xg[ii] + off, xring + decltype(SLOT)::value * XUB + ii * 1024);
  };
  // Weight code rows n0 + 16 j + r16 (clamped), word offset 4 q.
  uint32_t co[NT];
#pragma unroll
  for (int j = 0; j < NT; j++) {
    const int r = n0 + 16 * j + r16 < a.N ? n0 + 16 * j + r16 : a.N - 1;
    co[j] = (uint32_t)(((int64_t)r * (a.K / 8) + 4 * q) * 4);
  }
  u32x4 wb[DB][NT];
  auto load_w = [&](int k, auto SLOT) __attribute__((always_inline)) {
    const uint32_t off = (uint32_t)chunk(k) * (CK / 2);
#pragma unroll
    for (int j = 0; j < NT; j++) wb[decltype(SLOT)::value][j] = ld16s<0>(a.codes, co[j] + off);
  };

  // Ring order: x unit u + XU is issued right after unit u's last step, W(k + DB) right after
  // chunk k's last step (after its x unit) -- so W(c) follows x unit 2 c - 2 DB + 1 + XU =
  // 2 c - 1, and when a unit is awaited, the loads issued after it are one x unit and one W
  // chunk.  The prologue keeps that order: W0, U0 before the scales are awaited (so the
  // request queue is not filled ahead of them), then U1, W1.
  static_assert(DB == 2 && XU == 2, "the prologue, the waits and the trip below assume two-deep rings");
  load_w(0, ic<0>{});
  load_xu(0, ic<0>{}, ic<0>{});
  wait_vmem<XIN + NT>();  // the scales / zeros have landed
#pragma unroll
  for (int i = 0; i < RPW; i++) asm volatile("" : "+v"(sv[i]), "+v"(zv[i]));  // defined only here
  bool zok = true;
  if (lane < ng) {
#pragma unroll
    for (int i = 0; i < RPW; i++) {
      const int r = wave + NW * i;
      float sf, zf;
      __builtin_memcpy(&sf, &sv[i], 4);
      __builtin_memcpy(&zf, &zv[i], 4);
      ls[r * sp + lane] = sf;
      lz[r * sp + lane] = zf;
      zok = zok && zf == rintf(zf) && fabsf(zf) <= 64.f;
    }
  }
  // Integral zero points in the whole tile: one exact FMA leaves q - z.
  const bool zint = __syncthreads_and(zok);

  // Per-row scale exponent over this wave's groups: s' = s 2^e with max |s'| in [16, 32).
  float fsc[NT];
  {
    const int gl0 = n > 0 ? cb * CK / a.G : 0, gl1 = n > 0 ? (ce * CK - 1) / a.G + 1 : 0;
#pragma unroll
    for (int j = 0; j < NT; j++) {
      float mx = 0.f;
      for (int gl = gl0; gl < gl1; gl++) mx = fmaxf(mx, fabsf(ls[(16 * j + r16) * sp + gl]));
      int ex = 0;
      (void)frexpf(mx, &ex);
      ex = mx > 0.f && mx <= 3.0e38f ? 5 - ex : 0;
      ex = ex < -100 ? -100 : ex > 100 ? 100 : ex;
      fsc[j] = ldexpf(1.f, ex);
    }
  }

  load_xu(0, ic<1>{}, ic<1>{});
  load_w(1, ic<1>{});

  f32x4 acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; i++)
#pragma unroll
    for (int j = 0; j < NT; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Per-chunk dequant constants of the lane's five weight rows.
  uint32_t c1[NT], sk[NT], c2[NT];
  auto chunk_consts = [&](int k) __attribute__((always_inline)) {
    const int gl = (cb + k) * CK / a.G;
#pragma unroll
    for (int j = 0; j < NT; j++) {
      const float s1 = ls[(16 * j + r16) * sp + gl] * fsc[j], z1 = lz[(16 * j + r16) * sp + gl];
      const f16x2 a1 = zint ? f16x2{(_Float16)(-1024.f - z1), (_Float16)(-64.f - z1)} : f16x2{(_Float16)-1024.f, (_Float16)-64.f};
      const f16x2 a2 = zint ? f16x2{(_Float16)0.f, (_Float16)0.f} : f16x2{(_Float16)(-z1 * s1), (_Float16)(-z1 * s1)};
      c1[j] = as_u(a1);
      sk[j] = as_u(f16x2{(_Float16)s1, (_Float16)s1});
      c2[j] = as_u(a2);
    }
  };
  // The lane's A fragment offsets in a unit: row 16 i + r16 (+ 2048 i), logical piece
  // 4 s' + q for step s' of the unit, stored at piece ^ f(row), f(row) = (r16 / 2) % 8.
  const uint32_t aoff0 = (uint32_t)(r16 * 128 + (((0 + q) ^ ((r16 >> 1) & 7)) << 4));
  const uint32_t aoff1 = (uint32_t)(r16 * 128 + (((4 + q) ^ ((r16 >> 1) & 7)) << 4));
  const unsigned char *xr = lds + wave * XWB;
  const uint32_t magic = 0x64646464u;

  // One 32-k step S of chunk k: W slot WS, x unit slot XS (the unit is chunk k's half S / 2).
  auto step = [&](int k, auto S, auto WS, auto XS) __attribute__((always_inline)) {
    constexpr int s = decltype(S)::value, ws = decltype(WS)::value, xs = decltype(XS)::value;
    if constexpr (s % 2 == 0) {
      // The unit's data: loads issued after it are the next x unit and one W chunk.
      wait_vmem<XIN + NT>();
      if constexpr (s == 0) {
#pragma unroll
        for (int j = 0; j < NT; j++) asm volatile("" : "+v"(wb[ws][j]));  // defined only here
      }
    }
    if (k < n) {  // (wave-uniform) a padding chunk only keeps the ring's loads and waits
      if constexpr (s == 0) {
        chunk_consts(k);
        // Lane group g loaded words 4 g + [0, 4) of the chunk; step s needs word 4 s + q in
        // lane group q: a 4 x 4 transpose across lane groups, in place.
#pragma unroll
        for (int j = 0; j < NT; j++) {
          u32x4 &v = wb[ws][j];
          const auto h02 = __builtin_amdgcn_permlane32_swap(v[0], v[2], false, false);
          const auto h13 = __builtin_amdgcn_permlane32_swap(v[1], v[3], false, false);
          const auto o01 = __builtin_amdgcn_permlane16_swap(h02[0], h13[0], false, false);
          const auto o23 = __builtin_amdgcn_permlane16_swap(h02[1], h13[1], false, false);
          v = u32x4{o01[0], o01[1], o23[0], o23[1]};
        }
      }
      const f16x2 f1 = {(_Float16)1.f, (_Float16)0.0625f};
      f16x8 bf[NT];
#pragma unroll
      for (int j = 0; j < NT; j++) {
        const uint32_t w = wb[ws][j][s];
#pragma unroll
        for (int i = 0; i < 4; i++) {
          // bytes (b_i, 0x64, b_i, 0x64), nibbles kept: (1024 + q_2i, 1024 + 16 q_2i+1)
          const uint32_t sel = 0x04000400u | ((uint32_t)i << 16) | (uint32_t)i;
          const uint32_t h = __builtin_amdgcn_perm(magic, w, sel) & 0xFFF0FF0Fu;
          f16x2 v = __builtin_elementwise_fma(as_h2(h), f1, as_h2(c1[j]));
          v = __builtin_elementwise_fma(v, as_h2(sk[j]), as_h2(c2[j]));
          bf[j][2 * i] = v[0];
          bf[j][2 * i + 1] = v[1];
        }
      }
      const unsigned char *xb = xr + xs * XUB + ((s & 1) ? aoff1 : aoff0);
      f16x8 af[MT];
#pragma unroll
      for (int i = 0; i < MT; i++) af[i] = *reinterpret_cast<const f16x8 *>(xb + 2048 * i);
#pragma unroll
      for (int j = 0; j < NT; j++)
#pragma unroll
        for (int i = 0; i < MT; i++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    if constexpr (s % 2 == 1) {
      // Refill the unit's slot with unit 2 k + s / 2 + XU; after the chunk, W(k + DB).
      constexpr int un = s / 2 + XU;  // relative to 2 k
      load_xu(k + un / 2, ic<un % 2>{}, XS);
      if constexpr (s == 3) load_w(k + DB, WS);
    }
  };
  // A chunk's four steps: W slot WS, its two x units in slots 0, 1.
  auto chunk_steps = [&](int k, auto WS) __attribute__((always_inline)) {
    step(k, ic<0>{}, WS, ic<0>{});
    step(k, ic<1>{}, WS, ic<0>{});
    step(k, ic<2>{}, WS, ic<1>{});
    step(k, ic<3>{}, WS, ic<1>{});
  };
  // Whole trips of two chunks (W slots 0, 1); the second chunk of the last trip may be
  // padding, which keeps the ring's loads and waits but does no arithmetic.  The waves of a
  // SIMD hold 3 and 4 chunks (or equal counts), so one wave's padding overlaps the other's work.
  for (int k = 0; k < n; k += 2) {
    chunk_steps(k, ic<0>{});
    chunk_steps(k + 1, ic<1>{});
  }
  // The last (clamped) prefetches land before their registers and LDS can be reused.
  wait_vmem<0>();
#pragma unroll
  for (int j = 0; j < NT; j++)
#pragma unroll
    for (int c = 0; c < DB; c++) asm volatile("" : "+v"(wb[c][j]));

  // Undo the row exponents, then add the eight waves' tiles in LDS (over the x rings).  Lane
  // holds D[4 q + r][r16] of tile (i, j): x row 16 i + 4 q + r, weight row 16 j + r16.
#pragma unroll
  for (int i = 0; i < MT; i++)
#pragma unroll
    for (int j = 0; j < NT; j++) acc[i][j] *= 1.f / fsc[j];  // (a power of two: exact)
  float *red = reinterpret_cast<float *>(lds);
  constexpr int RB = 16 * MT * RP;  // floats per wave tile
  auto put = [&](int b) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
      for (int j = 0; j < NT; j++)
#pragma unroll
        for (int r = 0; r < 4; r++) red[b * RB + (16 * i + 4 * q + r) * RP + 16 * j + r16] = acc[i][j][r];
  };
  __syncthreads();  // every wave is done with its x ring
  if (wave >= 4) put(wave - 4);
  __syncthreads();
  if (wave < 4) {
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
      for (int j = 0; j < NT; j++)
#pragma unroll
        for (int r = 0; r < 4; r++) acc[i][j][r] += red[wave * RB + (16 * i + 4 * q + r) * RP + 16 * j + r16];
  }
  __syncthreads();
  if (wave < 4) put(wave);
  __syncthreads();
  const int rows = a.M < 16 * MT ? a.M : 16 * MT;
  const bool vec = (a.N & 3) == 0;
  for (int e = t; e < rows * (NR / 4); e += NTH) {
    const int m = e / (NR / 4), c = 4 * (e - m * (NR / 4));
    const int o = m * RP + c;
    const f32x4 v0 = *reinterpret_cast<const f32x4 *>(red + o), v1 = *reinterpret_cast<const f32x4 *>(red + RB + o);
    const f32x4 v2 = *reinterpret_cast<const f32x4 *>(red + 2 * RB + o),
                v3 = *reinterpret_cast<const f32x4 *>(red + 3 * RB + o);
    const f32x4 v = (v0 + v1) + (v2 + v3);
    const int64_t go = (int64_t)m * a.N + n0 + c;
    const f16x4 h = {(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
    if (vec && n0 + c + 3 < a.N) {
      __builtin_memcpy(&a.y[go], &h, 8);
    } else {
#pragma unroll
      for (int u = 0; u < 4; u++)
        if (n0 + c + u < a.N) {
          const _Float16 hu = h[u];
          __builtin_memcpy(&a.y[go + u], &hu, 2);
        }
    }
  }
}

static size_t i4cu_lds(int64_t K, int G, int mt) {
  const size_t ring = (size_t)NW * XU * (16 * mt) * 128;
  const size_t red = (size_t)4 * (16 * mt) * RP * 4;
  return (ring > red ? ring : red) + 2 * (size_t)NR * (size_t)((K / G) | 1) * 4;
}

// One workgroup per CU over all of K: taken when the 80-row column tiles fill at least three
// quarters of the CUs (below that, the K-split kernel keeps the chip busy), and the row's
// groups fit one wave's lanes (K / G <= 64), and the LDS of the launch's x tiles fits.
bool i4cu_ok(int64_t M, int64_t N, int64_t K, int G, int x_dtype, const void *x, const void *codes) {
  return x_dtype == F16 && M > 8 && M <= 64 && K % CK == 0 && G % CK == 0 && K % G == 0 && N >= 1 &&
         ((uintptr_t)x & 15) == 0 && ((uintptr_t)codes & 15) == 0 && N * K / 2 < ((int64_t)1 << 31) &&
         M * K * 2 < ((int64_t)1 << 31) && 4 * cdiv(N, NR) >= 3 * (int64_t)device_cus() && K / G <= 64 &&
         i4cu_lds(K, G, (int)cdiv(M, 16)) <= 160 * 1024;
}

int launch_i4cu(const uint16_t *x, const uint32_t *codes, const float *s, const float *z, void *y, int64_t M, int64_t N,
                int64_t K, int G, hipStream_t st) {
  I4CuArgs a;
  a.x = x;
  a.codes = codes;
  a.s = s;
  a.z = z;
  a.y = static_cast<uint16_t *>(y);
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.G = G;
  const int mt = (int)cdiv(M, 16);
  const size_t lds = i4cu_lds(K, G, mt);
  const unsigned grid = (unsigned)cdiv(N, NR);
  switch (mt) {
    case 1: int4_cu_kernel<1><<<grid, NTH, lds, st>>>(a); break;
    case 2: int4_cu_kernel<2><<<grid, NTH, lds, st>>>(a); break;
    case 3: int4_cu_kernel<3><<<grid, NTH, lds, st>>>(a); break;
    default: int4_cu_kernel<4><<<grid, NTH, lds, st>>>(a); break;
  }
  return check_launch("int4_cu");
}

}  // namespace hq
