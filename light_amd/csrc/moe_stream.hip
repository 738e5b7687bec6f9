// moe_stream.hip -- the grouped Q4_K expert matmul of MoE prefill (many pairs per expert) as a
// weight stream: out rows of the pairs routed to expert e = x_pair . W_e^T, optionally gated.
//
// Role: Light's moe_gemm_q for M > 4 E pairs (kernels/cuda/moe.go:78-141, ops/moe.go:124-204:
// a grouped qmatmul over expert segments), fused with the gated epilogue of nn.SparseMoE
// (nn/moe.go:196-236) when gated: h = act(x . Wg^T) * (x . Wu^T).
//
// Design (gfx950, 512 threads = 8 waves, grid = (column blocks, E)):
//  * At T = 256 pairs per 128 experts each expert sees about 16 pair rows, so the grouped GEMM
//    is a weight stream with little reuse.  A workgroup owns 256 weight rows of one expert
//    (gated: 128 gate rows and the matching 128 up rows) and streams them once per pass of up
//    to 32 pair rows; the pass's rows of x (f16, per-row power-of-two scale) go to LDS one
//    256-k block at a time by whole-row LDS DMA, shared by the eight waves, so x is read once
//    per workgroup instead of once per 128 columns.
//  * Wave w owns two 16-row weight tiles (gated: gate tile and up tile of the same 16 output
//    columns, so act(g) * u is formed in registers).  Its raw Q4_K bytes stream straight into
//    registers, one block ahead: per tile and lane 48 bytes per block (the block header and
//    32 quant bytes).  Lane group q loads quant bytes [32 q, 32 q + 32), the sub-block pair q;
//    a 4 x 4 transpose of 8-byte pieces across the lane groups (v_permlane32_swap,
//    v_permlane16_swap on the low and the high dwords) leaves lane group q bytes
//    [32 p + 8 q, 32 p + 8 q + 8) of every pair p: weights 8 q .. 8 q + 7 of sub-blocks 2 p (low
//    nibbles) and 2 p + 1 (high nibbles), the B fragment of v_mfma_f32_16x16x32_f16.
//  * Dequant as the tiled grouped GEMM's: v_perm_b32 puts two code bytes under 0x64 exponent
//    bytes and an AND keeps their low (or high) nibbles, f16 1024 + q (or 1024 + 16 q), exact;
//    a packed add of -1024 (or FMA by 1/16 with -64) leaves q; one packed FMA gives
//    (d sc) q - dmin m, rounded once to f16.
//  * The x block of 256 k x 32 pair rows sits in LDS at 512 bytes per row with its 16-byte
//    pieces XOR-swizzled by row % 16, so the A fragment reads are conflict-free; two buffers.
//  * Loads are issued from inline asm and awaited with explicit vmcnt counts; per block a wave
//    issues the next x block's DMA before its arithmetic and the weight block two ahead after
//    it, so when block b is awaited only the weight block b + 1 was issued after x(b).  The
//    block loop runs whole pairs of blocks (an odd count's last is padding that keeps the
//    waits, the barrier and the loads), so the counts hold on every path.
#include "internal.hpp"

namespace hq {

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int SW = 8;             // waves
constexpr int STH = 64 * SW;      // threads
constexpr int SROWS = 32 * SW;    // weight rows per workgroup (gated: 128 gate + 128 up)
constexpr int SXB = 32 * 512;     // bytes of one x block buffer: 32 pair rows x 256 k

struct StreamArgs {
  const uint16_t *xh;     // f16 x rows (rows, K)
  const float *xscale;    // per x row
  const uint8_t *w;       // Q4_K experts (E, N, K)
  const int64_t *pairs;
  const int32_t *offsets;
  const float *topk_w;
  float *out;
  int64_t size_m, expert_bytes, row_bytes;
  int N, K, topk, rpp, gated_I, act;
};

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
template <int IMM>
__device__ __forceinline__ u32x4 ld16s(const void *base, uint32_t off) {
  u32x4 r;
  asm volatile("global_load_dwordx4 %0, %1, %2 offset:%3" : "=v"(r) : "v"(off), "s"(base), "n"(IMM) : "memory");
  return r;
}
// 16 bytes per lane from base + off into LDS at m0 + 16 lane (no immediate offset: on an LDS
// DMA load it moves the LDS destination too).
__device__ __forceinline__ void dma16s(const void *base, uint32_t off, uint32_t m0) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(m0) : "memory", "m0");
}
#pragma clang diagnostic pop

template <int N>
__device__ __forceinline__ void wait_vmem() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

template <int V>
using ic = std::integral_constant<int, V>;

// A workgroup-uniform pointer in SGPRs (the load's base operand).
__device__ __forceinline__ const void *uniform_ptr(const void *p) {
  const uint64_t v = (uint64_t)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (const void *)(uintptr_t)(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ f16x2 as_h2(uint32_t v) {
  f16x2 h;
  __builtin_memcpy(&h, &v, 4);
  return h;
}

// q4k_scale_min for a sub-block index that differs between lanes, without branches.
__device__ __forceinline__ void q4k_scale_min_lane(int j, uint32_t s0, uint32_t s1, uint32_t s2, int &sc, int &m) {
  const uint32_t sh = 8 * (uint32_t)(j & 3);
  const uint32_t a = (s2 >> sh) & 0xffu, l = (s0 >> sh) & 0xffu, h = (s1 >> sh) & 0xffu;
  const bool low = j < 4;
  sc = (int)(low ? (l & 63u) : ((a & 15u) | ((l >> 6) << 4)));
  m = (int)(low ? (h & 63u) : ((a >> 4) | ((h >> 6) << 4)));
}

// The raw bytes of one weight tile's block for one lane: quant bytes (8 dwords) and header.
struct WTile {
  u32x4 q0, q1, hd;
};

}  // namespace

// One pass of up to 16 MT pair rows [r0, r0 + rows) of the expert's segment.
template <bool GATED, int MT>
__device__ __forceinline__ void stream_pass(const StreamArgs &a, unsigned char *lds, const void *wexp, int seg0,
                                            int r0, int rows, int n0) {
  const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int q = lane >> 4, r16 = lane & 15;
  const int nb = a.K / 256;
  // x DMA: instruction j of a block loads pass rows 2 j, 2 j + 1 (lanes 0-31, 32-63); wave w
  // issues instructions w, w + 8, ...  The lane's LDS slot is piece lane % 32 of its row,
  // filled from logical piece (lane % 32) ^ (row % 16).
  constexpr int XIN = MT;  // instructions per wave and block (16 MT rows / 2 rows / 8 waves)
  uint32_t xo[XIN];
#pragma unroll
  for (int ii = 0; ii < XIN; ii++) {
    const int row = 2 * (wave + SW * ii) + (lane >> 5);
    uint32_t xr = 0;
    if (row < rows) {
      const int64_t p = a.pairs[seg0 + r0 + row];
      if (p >= 0 && p < a.size_m) xr = (uint32_t)(a.rpp ? p : p / a.topk);
    }
    const int piece = (lane & 31) ^ (row & 15);
    xo[ii] = (uint32_t)(((int64_t)xr * a.K + 8 * piece) * 2);
  }
  const uint32_t xlds = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
  auto load_x = [&](int b, int buf) __attribute__((always_inline)) {
    const uint32_t off = (uint32_t)(b < nb ? b : nb - 1) * 512;
#pragma unroll
    for (int ii = 0; ii < XIN; ii++)
      dma16s(a.xh, xo[ii] + off,
             __builtin_amdgcn_readfirstlane(xlds + (uint32_t)buf * SXB + (uint32_t)(wave + SW * ii) * 1024));
  };
  // Weight rows of the wave's two tiles (clamped), byte offsets within the expert.
  uint32_t wo[2];
#pragma unroll
  for (int T = 0; T < 2; T++) {
    int n;
    if constexpr (GATED) {
      const int c = n0 + 16 * wave + r16;
      n = (T ? a.gated_I : 0) + (c < a.gated_I ? c : a.gated_I - 1);
    } else {
      const int r = n0 + 32 * wave + 16 * T + r16;
      n = r < a.N ? r : a.N - 1;
    }
    wo[T] = (uint32_t)((int64_t)n * a.row_bytes);
  }
  WTile wt[2][2];  // [slot][tile]
  auto load_w = [&](int b, auto SLOT) __attribute__((always_inline)) {
    const uint32_t off = (uint32_t)(b < nb ? b : nb - 1) * 144;
#pragma unroll
    for (int T = 0; T < 2; T++) {
      WTile &r = wt[decltype(SLOT)::value][T];
      r.q0 = ld16s<0>(wexp, wo[T] + off + 16 + 32 * q);
      r.q1 = ld16s<16>(wexp, wo[T] + off + 16 + 32 * q);
      r.hd = ld16s<0>(wexp, wo[T] + off);
    }
  };

  f32x4 acc[MT][2];
#pragma unroll
  for (int i = 0; i < MT; i++)
#pragma unroll
    for (int T = 0; T < 2; T++) acc[i][T] = f32x4{0.f, 0.f, 0.f, 0.f};

  // A fragment offset of the lane in a block buffer: row 16 i + r16 (+ 8 KB i), logical piece
  // 4 s + q of sub-block s, stored at (4 s + q) ^ r16.
  const uint32_t arow = (uint32_t)r16 * 512;
  const uint32_t magic = 0x64646464u;
  const f16x2 k1024 = {(_Float16)-1024.f, (_Float16)-1024.f};
  const f16x2 s16 = {(_Float16)0.0625f, (_Float16)0.0625f}, k64 = {(_Float16)-64.f, (_Float16)-64.f};

  // Block b: x buffer b % 2, weight slot SLOT.  A block past the last (an odd count's padding)
  // keeps the wait, the barrier and the (clamped) loads but does no arithmetic.  (Skipping its
  // wait would let the compiler reuse ring registers whose loads are still in flight.)
  auto block = [&](int b, auto SLOT) __attribute__((always_inline)) {
    constexpr int sl = decltype(SLOT)::value;
    // x(b) and everything before it, including W(b): only W(b + 1) was issued after x(b).
    wait_vmem<6>();
#pragma unroll
    for (int T = 0; T < 2; T++) asm volatile("" : "+v"(wt[sl][T].q0), "+v"(wt[sl][T].q1), "+v"(wt[sl][T].hd));
    __syncthreads();  // every wave's share of x(b) has landed; block b - 1's buffer is free
    load_x(b + 1, (b + 1) & 1);
    if (b < nb) {
    const unsigned char *xb = lds + (b & 1) * SXB + arow;
    // Transpose the 8-byte pieces across lane groups: afterwards lane group q holds bytes
    // [32 p + 8 q, + 8) of pair p as (lo[p], hi[p]).
    uint32_t lo[2][4], hi[2][4];
#pragma unroll
    for (int T = 0; T < 2; T++) {
      const WTile &r = wt[sl][T];
      const uint32_t d[8] = {r.q0[0], r.q0[1], r.q0[2], r.q0[3], r.q1[0], r.q1[1], r.q1[2], r.q1[3]};
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const auto a02 = __builtin_amdgcn_permlane32_swap(d[h], d[4 + h], false, false);
        const auto a13 = __builtin_amdgcn_permlane32_swap(d[2 + h], d[6 + h], false, false);
        const auto o01 = __builtin_amdgcn_permlane16_swap(a02[0], a13[0], false, false);
        const auto o23 = __builtin_amdgcn_permlane16_swap(a02[1], a13[1], false, false);
        uint32_t *o = h ? hi[T] : lo[T];
        o[0] = o01[0];
        o[1] = o01[1];
        o[2] = o23[0];
        o[3] = o23[1];
      }
    }
    // Scales: lane group q decodes sub-blocks 2 q and 2 q + 1 of its row into packed f16
    // (d sc, -dmin m), and three permlane swaps hand every lane group all eight.
    uint32_t sm[2][8];
#pragma unroll
    for (int T = 0; T < 2; T++) {
      const WTile &r = wt[sl][T];
      const float d = h2f(r.hd[0] & 0xffffu), dmin = h2f(r.hd[0] >> 16);
#pragma unroll
      for (int u = 0; u < 2; u++) {
        int sc, mn;
        q4k_scale_min_lane(2 * q + u, r.hd[1], r.hd[2], r.hd[3], sc, mn);
        const f16x2 v = {(_Float16)(d * (float)sc), (_Float16)(-(dmin * (float)mn))};
        uint32_t x;
        __builtin_memcpy(&x, &v, 4);
        const auto a = __builtin_amdgcn_permlane16_swap(x, x, false, false);    // (g0 g0 g2 g2), (g1 g1 g3 g3)
        const auto b02 = __builtin_amdgcn_permlane32_swap(a[0], a[0], false, false);  // g0 x4, g2 x4
        const auto b13 = __builtin_amdgcn_permlane32_swap(a[1], a[1], false, false);  // g1 x4, g3 x4
        sm[T][0 + u] = b02[0];
        sm[T][2 + u] = b13[0];
        sm[T][4 + u] = b02[1];
        sm[T][6 + u] = b13[1];
      }
    }
#pragma unroll
    for (int s = 0; s < 8; s++) {
      const int p = s >> 1, nib = s & 1;
      f16x8 bf[2];
#pragma unroll
      for (int T = 0; T < 2; T++) {
        const f16x2 dsm = as_h2(sm[T][s]);
        const f16x2 sv = {dsm[0], dsm[0]}, mv = {dsm[1], dsm[1]};
        const uint32_t wd[2] = {lo[T][p], hi[T][p]};
#pragma unroll
        for (int u = 0; u < 2; u++) {
#pragma unroll
          for (int v = 0; v < 2; v++) {
            // bytes (b_2v, 0x64, b_2v+1, 0x64), the low or the high nibbles kept
            const uint32_t sel = v ? 0x04030402u : 0x04010400u;
            const uint32_t h = __builtin_amdgcn_perm(magic, wd[u], sel) & (nib ? 0xFFF0FFF0u : 0xFF0FFF0Fu);
            const f16x2 qv = nib ? __builtin_elementwise_fma(as_h2(h), s16, k64) : as_h2(h) + k1024;  // q, exact
            const f16x2 wv = __builtin_elementwise_fma(qv, sv, mv);
            bf[T][4 * u + 2 * v] = wv[0];
            bf[T][4 * u + 2 * v + 1] = wv[1];
          }
        }
      }
      const uint32_t pc = (uint32_t)(((4 * s + q) ^ r16) << 4);
#pragma unroll
      for (int i = 0; i < MT; i++) {
        const f16x8 af = *reinterpret_cast<const f16x8 *>(xb + 8192 * i + pc);
#pragma unroll
        for (int T = 0; T < 2; T++) acc[i][T] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[T], acc[i][T], 0, 0, 0);
      }
    }
    }
    load_w(b + 2, SLOT);
  };

  // Prologue in the loop's issue order: W(0), x(0), W(1).
  load_w(0, ic<0>{});
  load_x(0, 0);
  load_w(1, ic<1>{});
  for (int b = 0; b < nb; b += 2) {
    block(b, ic<0>{});
    block(b + 1, ic<1>{});
  }
  // The last (clamped) loads land before their registers and LDS are reused.
  wait_vmem<0>();
#pragma unroll
  for (int sl = 0; sl < 2; sl++)
#pragma unroll
    for (int T = 0; T < 2; T++) asm volatile("" : "+v"(wt[sl][T].q0), "+v"(wt[sl][T].q1), "+v"(wt[sl][T].hd));
  __syncthreads();  // before the next pass's DMA overwrites the buffers

  // Lane holds D[4 q + r][r16] of tile (i, T): pass row 16 i + 4 q + r, output column r16.
#pragma unroll
  for (int i = 0; i < MT; i++)
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int row = 16 * i + 4 * q + r;
      if (row >= rows) continue;
      const int64_t pp = a.pairs[seg0 + r0 + row];
      if (pp < 0 || pp >= a.size_m) continue;
      const int64_t xr = a.rpp ? pp : pp / a.topk;
      const float sc = a.xscale[xr];
      if constexpr (GATED) {
        const int col = n0 + 16 * wave + r16;
        if (col < a.gated_I)
          a.out[(int64_t)pp * a.gated_I + col] = gate_act(acc[i][0][r] * sc, a.act) * (acc[i][1][r] * sc);
      } else {
#pragma unroll
        for (int T = 0; T < 2; T++) {
          const int col = n0 + 32 * wave + 16 * T + r16;
          if (col < a.N) a.out[pp * a.N + col] = acc[i][T][r] * sc * (a.topk_w ? a.topk_w[pp] : 1.f);
        }
      }
    }
}

template <bool GATED>
__global__ __launch_bounds__(STH) void moe_stream_kernel(StreamArgs a) {
  extern __shared__ __align__(16) unsigned char lds[];
  const int e = blockIdx.y;
  const int seg0 = a.offsets[e], seg1 = a.offsets[e + 1];
  if (seg0 >= seg1) return;
  const void *wexp = uniform_ptr(a.w + (int64_t)e * a.expert_bytes);
  const int n0 = blockIdx.x * (GATED ? SROWS / 2 : SROWS);
  // Passes of up to 32 pair rows (two 16-row x tiles).  A one-tile variant for experts with
  // at most 16 rows measured slower: the second instantiation pushed the kernel past 128
  // registers (one workgroup per CU instead of two) or, capped, made it spill.
  for (int r0 = 0; r0 < seg1 - seg0; r0 += 32) {
    const int rows = seg1 - seg0 - r0 < 32 ? seg1 - seg0 - r0 : 32;
    stream_pass<GATED, 2>(a, lds, wexp, seg0, r0, rows, n0);
  }
}

// Gated: N = 2 gated_I rows (gate, then up), out (size_m, gated_I); 16 | gated_I.  Plain: 16 | N.
// Byte offsets within an expert and into x, and pair indices, stay below 2^31.
bool moe_stream_ok(int64_t rows, int64_t size_m, int64_t N, int64_t K, int64_t gated_I) {
  if (K % 256 || K <= 0 || size_m >= ((int64_t)1 << 31)) return false;
  if (gated_I > 0 ? gated_I % 16 != 0 : N % 16 != 0) return false;
  return N * (K / 256) * 144 < ((int64_t)1 << 31) && rows * K * 2 < ((int64_t)1 << 31);
}

int launch_moe_stream_q4k(const uint16_t *xh, const float *xs, const void *w, const int64_t *pairs,
                          const int32_t *offsets, const float *topk_w, float *out, int topk, int64_t size_m, int64_t E,
                          int64_t N, int64_t K, int rpp, int64_t gated_I, int act, hipStream_t s) {
  StreamArgs a;
  a.xh = xh;
  a.xscale = xs;
  a.w = static_cast<const uint8_t *>(w);
  a.pairs = pairs;
  a.offsets = offsets;
  a.topk_w = topk_w;
  a.out = out;
  a.size_m = size_m;
  a.row_bytes = (K / 256) * 144;
  a.expert_bytes = N * a.row_bytes;
  a.N = (int)N;
  a.K = (int)K;
  a.topk = topk;
  a.rpp = rpp;
  a.gated_I = (int)gated_I;
  a.act = act;
  const size_t lds = 2 * (size_t)SXB;
  if (gated_I > 0) {
    dim3 grid((unsigned)cdiv(gated_I, SROWS / 2), (unsigned)E);
    moe_stream_kernel<true><<<grid, STH, lds, s>>>(a);
  } else {
    dim3 grid((unsigned)cdiv(N, SROWS), (unsigned)E);
    moe_stream_kernel<false><<<grid, STH, lds, s>>>(a);
  }
  return check_launch("moe_stream_q4k");
}

}  // namespace hq
