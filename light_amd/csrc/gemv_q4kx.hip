// gemv_q4kx.hip -- decode GEMV (M <= 8) for Q4_K and int4 weights: plain, gated (SwiGLU /
// GELU-erf) and the two-launch MLP (gated gate/up emitting quantized h, then down).
//
// Role: Light's matmul_q for small M (ops/matmul_q.go:61-75, kernels/cuda/matmul_q.go:44-91),
// its int4_gemv (ops/int4.go:87-99, kernels/cuda/int4.go:76-101), and the gated MLP decode
// out = act(x . Wg^T) * (x . Wu^T) followed by the down projection, which Light computes as
// MatMulQ, MatMulQ, SiLU / GeluErf, Mul, MatMulQ (models/llama.go:1306-1333; the dense BF16
// analogue is ops.GatedLinear, ops/gemv.go:80-130).
//
// Design (gfx950, wave64):
//  * Activations are two-level int8 (the act layout of common.hpp).  They come either
//    prepared from global memory (XIN = false) or from x (F32 / BF16 / F16) that each
//    workgroup quantizes into LDS itself (XIN = true, act_quant16_fast: two lanes per
//    32-block), saving a launch.
//  * A lane owns one 64-element unit of a weight row (a weight-format policy: Q4kUnit =
//    one (super-block, 64-element pair) of Q4_K, Int4Unit = two 32-element code blocks of
//    quant.Int4) and keeps the unit's activations in registers for the whole kernel.  A
//    team of TP lanes covers a row; a workgroup holds RW teams.  Products are exact
//    v_dot4_i32_i8 chains scaled once per 32-block.
//  * Workgroups are persistent (two per CU).  One register slot keeps the next row group's
//    loads in flight while the current one is reduced (each weight refilled as soon as its
//    dot is done); every load is unconditional -- inactive lanes read valid addresses and
//    their sums are dropped, rows past N are range-checked buffer loads that fetch nothing --
//    so no load sits in a branch and the compiler's wait counts stay exact.  Long rows carry
//    two rows per team and iteration.
//  * Q4_K high nibbles are masked in place with the sign bit flipped (16 * (q - 8) as a
//    signed byte, one and-xor per dword); the -8 folds into the block-sum term.
//  * Team sums: DPP row sums, then v_readlane over the wave's four rows; teams wider than a
//    wave add their 16-lane row sums through LDS (one barrier per group).  Row sums are added
//    in row order in both cases.
//  * AOUT: the workgroup owns whole 32-row chunks of the output, keeps the chunk's results
//    in LDS and, when a chunk is complete, quantizes it into the act layout for the next
//    matmul (the down projection) -- the gated kernel's output never needs its own
//    quantize launch.
#include "actq.hpp"
#include "internal.hpp"
#include "route.hpp"

#include <algorithm>
#include <atomic>
#include <mutex>

namespace hq {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

struct Q4kxArgs {
  const void *x;           // XIN: (M, K) of x dtype
  const uint8_t *ain;      // !XIN: prepared activations of (M, K)
  const uint8_t *w0, *w1;  // weights (N, K); w1 = up projection (gated mode only)
  const float *s0, *z0, *s1, *z1;  // int4 scales / zeros (N, K/G) of w0 / w1
  void *out;               // (M, N) of the output dtype, may be NULL with AOUT
  uint8_t *aout;           // AOUT: act layout of the (M, N) output
  int M, N, K, P, TP, RW;  // P: units per row (K/64); TP: team lanes; RW: teams per workgroup
  int G;                   // int4 group size
  int gpr = 0;             // int4 scale / zero groups per row of s0 / z0 (0: K / G; a K part: the full row's)
  int64_t row_bytes;
  int64_t in_q2, in_d, in_s;     // act offsets of (M, K)
  int64_t out_q2, out_d, out_s;  // act offsets of (M, N)
  int act;                       // gated epilogue: 0 SiLU, 1 GELU (erf)
};

namespace {

__device__ __forceinline__ float rsum16(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false));
  return v;
}

__device__ __forceinline__ float rl(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

}  // namespace

// LDS: act [MM][K] q1 | [MM][K] q2 | (d, e) [MM][K/32] | sx [MM][K/32]  (XIN only)
//      part [2][RW * NW * MM * TP/16]                                   (TP > 64 only)
//      hbuf [2][MM][32]                                                  (AOUT only)
__host__ __device__ constexpr int64_t q4kx_act_lds(int MM, int64_t K) { return MM * (2 * K + 12 * (K / 32)); }

// Weight loads are buffer loads over a resource that spans exactly the matrix (N rows).  A
// row group past the end loads "row N": every offset lies outside the resource, so the
// load returns zeros without a memory request.  The loads stay unconditional (no branch,
// exact compiler wait counts) and idle teams cost no bandwidth -- clamping them to a valid
// row instead would aim every workgroup's final prefetch at the same bytes, one L2 channel.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t span_rsrc(const void *p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u32x4_t bload16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}
__device__ __forceinline__ float bload_f32(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
__device__ __forceinline__ uint32_t bload_u32(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}

// ---- weight-unit policies --------------------------------------------------------
// Activations of one unit (two 32-blocks of one row of x), as each policy wants them.

// Q4_K / Q5_K unit: super-block b = u / 4, pair p = u % 4 -> 32 quant bytes (low nibbles =
// sub-block 2p, high = 2p+1) and the block header, broadcast in the block's 4-lane quad.
// Q5_K (quant/q5_k.go:11-22) adds the 32 qh bytes of the block: bit 2p / 2p+1 of qh[l] is
// the fifth bit of the pair's low / high element l.
//
// X2 = false: single-level activations (q1 with its step d only -- exactly q8_1), for rows of
// at least kX1MinK = 4096 elements, where the int8 rounding noise of x averages out below the
// error bar (K = 4096, N(0,1) x: at most ~3.6e-4 of |w| |x| per output against f32 x, a third
// of the 1e-3 bar); the q2 loads and dots are skipped (4096 x 14336: 10.9 -> 9.8 us; the MLP
// step's gate/up at K = 4096: 23.0 -> 22.3 us per step).  Shorter rows keep both levels.
template <bool Q5, bool X2 = true>
struct QkUnit {
  static constexpr int BB = Q5 ? 176 : 144, QO = Q5 ? 48 : 16;
  static constexpr bool kX2 = X2;
  struct Lane {
    uint32_t qoff, hoff, qhoff;  // byte offsets of the quant chunk / the block header / qh
    int ja;                      // first 32-block of x
    uint32_t sel, mlo, mhi;
    int ka, sh;
  };
  struct W {
    u32x4_t q0, q1;
    u32x4_t h0, h1;  // Q5_K only
    u32x4_t hd;      // the block header (d, dmin, scales[12]); the quad's four lanes load the same 16 B
  };
  struct X {
    uint32_t xa[8], xb[8], ya[8], yb[8];
    float4 de;  // (dA, eA, dB, eB)
    float2 ss;  // block sums of x
  };
  __device__ static Lane lane(int u) {
    Lane L;
    const int b = u >> 2, p = u & 3;
    L.qoff = b * BB + QO + p * 32;
    L.hoff = b * BB;
    L.qhoff = b * BB + 16;
    L.ja = b * 8 + 2 * p;
    const bool lowj = p < 2;
    L.sel = lowj ? ~0u : 0u;
    L.mlo = lowj ? 0x3F3Fu : 0x0F0Fu;
    L.mhi = lowj ? 0u : 0x3030u;
    L.ka = (2 * p) & 3;
    L.sh = 2 * p;
    return L;
  }
  // Byte offsets are 32-bit: the host checks (N + 1) * row_bytes < 2^32, row N included.
  __device__ static void load(const uint8_t *w, const float *, const float *, const Q4kxArgs &a, int row,
                              const Lane &L, W &r) {
    const __amdgpu_buffer_rsrc_t rs = span_rsrc(w, (uint32_t)a.N * (uint32_t)a.row_bytes);
    const uint32_t ro = (uint32_t)row * (uint32_t)a.row_bytes;
    r.q0 = bload16(rs, ro + L.qoff);
    r.q1 = bload16(rs, ro + L.qoff + 16);
    if constexpr (Q5) {
      r.h0 = bload16(rs, ro + L.qhoff);
      r.h1 = bload16(rs, ro + L.qhoff + 16);
    }
    r.hd = bload16(rs, ro + L.hoff);
  }
  __device__ static void load_x(const uint8_t *q1, const uint8_t *q2, const uint8_t *de, const uint8_t *sx,
                                int64_t blk, X &x) {
    const u32x4_t *s1 = reinterpret_cast<const u32x4_t *>(q1 + blk * 32);
    const u32x4_t v0 = s1[0], v1 = s1[1], v2 = s1[2], v3 = s1[3];
#pragma unroll
    for (int k = 0; k < 4; k++) x.xa[k] = v0[k], x.xa[k + 4] = v1[k], x.xb[k] = v2[k], x.xb[k + 4] = v3[k];
    if constexpr (X2) {
      const u32x4_t *s2 = reinterpret_cast<const u32x4_t *>(q2 + blk * 32);
      const u32x4_t w0 = s2[0], w1 = s2[1], w2 = s2[2], w3 = s2[3];
#pragma unroll
      for (int k = 0; k < 4; k++) x.ya[k] = w0[k], x.ya[k + 4] = w1[k], x.yb[k] = w2[k], x.yb[k + 4] = w3[k];
    }
    x.de = *reinterpret_cast<const float4 *>(de + 8 * blk);
    x.ss = *reinterpret_cast<const float2 *>(sx + 4 * blk);
  }
  template <int MM>
  __device__ static void dot(const W &w, const X (&x)[MM], const Lane &L, float (&out)[MM]) {
    const uint32_t h0 = w.hd[0], h1 = w.hd[1], h2 = w.hd[2], h3 = w.hd[3];
    const float d = h2f(h0 & 0xffffu), dmin = h2f(h0 >> 16);
    // 6-bit (scale, min) of sub-blocks 2p and 2p+1 (getScaleMinK4, quant/q4_k.go:83-89),
    // selected branch-free with lane constants: p < 2 takes the low six bits of
    // scales[j] / scales[j+4]; p >= 2 combines nibbles of scales[j+4] with the top two bits
    // of scales[j-4] / scales[j].
    const uint32_t t1 = (h1 >> (8 * L.ka)) & 0xffffu, t2 = (h2 >> (8 * L.ka)) & 0xffffu;
    const uint32_t t3 = (h3 >> (8 * L.ka)) & 0xffffu;
    const uint32_t srcS = (t1 & L.sel) | (t3 & ~L.sel), srcM = (t2 & L.sel) | ((t3 >> 4) & ~L.sel);
    const uint32_t scp = (srcS & L.mlo) | ((t1 >> 2) & L.mhi), mnp = (srcM & L.mlo) | ((t2 >> 2) & L.mhi);
    const float scA = (float)(scp & 0xffu), scB = (float)(scp >> 8);
    const float mnA = (float)(mnp & 0xffu), mnB = (float)(mnp >> 8);
    uint32_t lo[8], hi[8];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      lo[k] = w.q0[k] & 0x0F0F0F0Fu;
      lo[k + 4] = w.q1[k] & 0x0F0F0F0Fu;
      if constexpr (Q5) {
        hi[k] = (w.q0[k] >> 4) & 0x0F0F0F0Fu;
        hi[k + 4] = (w.q1[k] >> 4) & 0x0F0F0F0Fu;
        lo[k] |= ((w.h0[k] >> L.sh) & 0x01010101u) << 4;
        hi[k] |= ((w.h0[k] >> (L.sh + 1)) & 0x01010101u) << 4;
        lo[k + 4] |= ((w.h1[k] >> L.sh) & 0x01010101u) << 4;
        hi[k + 4] |= ((w.h1[k] >> (L.sh + 1)) & 0x01010101u) << 4;
      } else {
        // High nibbles in place, top bit flipped: the signed byte is 16 * (q - 8), one
        // and-xor per dword instead of a shift and a mask.
        hi[k] = (w.q0[k] & 0xF0F0F0F0u) ^ 0x80808080u;
        hi[k + 4] = (w.q1[k] & 0xF0F0F0F0u) ^ 0x80808080u;
      }
    }
#pragma unroll
    for (int mm = 0; mm < MM; mm++) {
      int dA = 0, dB = 0, dA2 = 0, dB2 = 0;
#pragma unroll
      for (int k = 0; k < 8; k++) {
        dA = dot4((int)lo[k], (int)x[mm].xa[k], dA);
        dB = dot4((int)hi[k], (int)x[mm].xb[k], dB);
        if constexpr (X2) {
          dA2 = dot4((int)lo[k], (int)x[mm].ya[k], dA2);
          dB2 = dot4((int)hi[k], (int)x[mm].yb[k], dB2);
        }
      }
      if constexpr (!X2) {
        if constexpr (Q5)
          out[mm] = q4k_pair1(d, dmin, scA, scB, mnA, mnB, x[mm].de, x[mm].ss, dA, dB);
        else
          out[mm] = q4k_pair1_h16(d, dmin, scA, scB, mnA, mnB, x[mm].de, x[mm].ss, dA, dB);
      } else if constexpr (Q5)
        out[mm] = q4k_pair(d, dmin, scA, scB, mnA, mnB, x[mm].de, x[mm].ss, dA, dA2, dB, dB2);
      else
        out[mm] = q4k_pair_h16(d, dmin, scA, scB, mnA, mnB, x[mm].de, x[mm].ss, dA, dA2, dB, dB2);
    }
  }
};
using Q4kUnit = QkUnit<false>;
using Q5kUnit = QkUnit<true>;

// int4 unit (quant.Int4, quant/int4.go:11-34): 64 elements = code words 8u .. 8u+7 (two
// 32-blocks A, B); nibble j of word c is element 8c + j, so the low / high nibbles of a
// word are its even / odd elements and the lane's activations are stored even / odd
// permuted (v_perm_b32) once.  Per block: s * (d * sum(q q1) + e * sum(q q2) - z * sx).
// X2 = false: single-level activations, as for QkUnit.
template <bool X2 = true>
struct Int4UnitT {
  static constexpr bool kX2 = X2, kInt4 = true;
  struct Lane {
    uint32_t coff;  // byte offset of the unit's codes in a row
    int ja, gA, gB;  // first 32-block of x; group index of blocks A, B
  };
  struct W {
    u32x4_t q0, q1;
    float sA, zA, sB, zB;
  };
  struct X {
    int ev[8], od[8], ev2[8], od2[8];  // blocks A (0..3) and B (4..7)
    float4 de;
    float2 ss;
  };
  __device__ static Lane lane(int u, int G) {
    Lane L;
    L.coff = 32 * u;
    L.ja = 2 * u;
    L.gA = (64 * u) / G;
    L.gB = (64 * u + 32) / G;
    return L;
  }
  __device__ static void load(const uint8_t *w, const float *s, const float *z, const Q4kxArgs &a, int row,
                              const Lane &L, W &r) {
    const __amdgpu_buffer_rsrc_t rs = span_rsrc(w, (uint32_t)a.N * (uint32_t)a.row_bytes);
    const uint32_t gpr = (uint32_t)(a.gpr ? a.gpr : a.K / a.G);
    const uint32_t gbytes = (uint32_t)a.N * gpr * 4u;
    const __amdgpu_buffer_rsrc_t rsc = span_rsrc(s, gbytes), rz = span_rsrc(z, gbytes);
    const uint32_t ro = (uint32_t)row * (uint32_t)a.row_bytes;
    r.q0 = bload16(rs, ro + L.coff);
    r.q1 = bload16(rs, ro + L.coff + 16);
    const uint32_t go = (uint32_t)row * gpr * 4u;
    r.sA = bload_f32(rsc, go + 4u * L.gA);
    r.zA = bload_f32(rz, go + 4u * L.gA);
    r.sB = bload_f32(rsc, go + 4u * L.gB);
    r.zB = bload_f32(rz, go + 4u * L.gB);
  }
  __device__ static void load_x(const uint8_t *q1, const uint8_t *q2, const uint8_t *de, const uint8_t *sx,
                                int64_t blk, X &x) {
    const u32x4_t *s1 = reinterpret_cast<const u32x4_t *>(q1 + blk * 32);
    const u32x4_t *s2 = reinterpret_cast<const u32x4_t *>(q2 + blk * 32);
    const u32x4_t v[4] = {s1[0], s1[1], s1[2], s1[3]};
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const uint32_t a0 = v[k >> 1][2 * (k & 1)], a1 = v[k >> 1][2 * (k & 1) + 1];
      x.ev[k] = (int)__builtin_amdgcn_perm(a1, a0, 0x06040200u);
      x.od[k] = (int)__builtin_amdgcn_perm(a1, a0, 0x07050301u);
    }
    if constexpr (X2) {
      const u32x4_t y[4] = {s2[0], s2[1], s2[2], s2[3]};
#pragma unroll
      for (int k = 0; k < 8; k++) {
        const uint32_t b0 = y[k >> 1][2 * (k & 1)], b1 = y[k >> 1][2 * (k & 1) + 1];
        x.ev2[k] = (int)__builtin_amdgcn_perm(b1, b0, 0x06040200u);
        x.od2[k] = (int)__builtin_amdgcn_perm(b1, b0, 0x07050301u);
      }
    }
    x.de = *reinterpret_cast<const float4 *>(de + 8 * blk);
    x.ss = *reinterpret_cast<const float2 *>(sx + 4 * blk);
  }
  template <int MM>
  __device__ static void dot(const W &w, const X (&x)[MM], const Lane &, float (&out)[MM]) {
    uint32_t lo[8], hi[8];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      lo[k] = w.q0[k] & 0x0F0F0F0Fu;
      hi[k] = (w.q0[k] >> 4) & 0x0F0F0F0Fu;
      lo[k + 4] = w.q1[k] & 0x0F0F0F0Fu;
      hi[k + 4] = (w.q1[k] >> 4) & 0x0F0F0F0Fu;
    }
#pragma unroll
    for (int mm = 0; mm < MM; mm++) {
      int dA = 0, dA2 = 0, dB = 0, dB2 = 0;
#pragma unroll
      for (int k = 0; k < 4; k++) {
        dA = dot4((int)lo[k], x[mm].ev[k], dA);
        dA = dot4((int)hi[k], x[mm].od[k], dA);
        dB = dot4((int)lo[4 + k], x[mm].ev[4 + k], dB);
        dB = dot4((int)hi[4 + k], x[mm].od[4 + k], dB);
        if constexpr (X2) {
          dA2 = dot4((int)lo[k], x[mm].ev2[k], dA2);
          dA2 = dot4((int)hi[k], x[mm].od2[k], dA2);
          dB2 = dot4((int)lo[4 + k], x[mm].ev2[4 + k], dB2);
          dB2 = dot4((int)hi[4 + k], x[mm].od2[4 + k], dB2);
        }
      }
      const float4 de = x[mm].de;
      float yA, yB;
      if constexpr (X2) {
        yA = __fmaf_rn(-w.zA, x[mm].ss.x, __fmaf_rn(de.y, (float)dA2, __fmul_rn(de.x, (float)dA)));
        yB = __fmaf_rn(-w.zB, x[mm].ss.y, __fmaf_rn(de.w, (float)dB2, __fmul_rn(de.z, (float)dB)));
      } else {
        yA = __fmaf_rn(-w.zA, x[mm].ss.x, __fmul_rn(de.x, (float)dA));
        yB = __fmaf_rn(-w.zB, x[mm].ss.y, __fmul_rn(de.z, (float)dB));
      }
      out[mm] = __fmaf_rn(w.sB, yB, __fmul_rn(w.sA, yA));
    }
  }
};

using Int4Unit = Int4UnitT<true>;

// Q6_K_R unit (the planar Q6_K layout of q6k_repack.hip): unit u = 4 b + v of block b pairs
// group g = v % 2 ("A", 32-block ja = 8 b + 4 h + g of x, h = v / 2) with group g + 2 ("B",
// block ja + 2).  Three contiguous 16-byte planes (quant bytes 0..15, 16..31, 2-bit highs),
// four int8 scales and the block's f16 d (read as the dword holding d of blocks b, b ^ 1).
// Per 16-weight sub-block: dot chains start at -32 * (sum of x's quants) (the Q6_K offset),
// c = 254 * dot(q1) + dot(q2) is exact below 2^24 (|dot| <= 16 * 32 * 127), and the sum is
// d * (e_A * (scA0 c_A0 + scA1 c_A1) + e_B * (...)), with e = d_x / 254 the second level's
// step (d_x q1 + e q2 = e (254 q1 + q2) to within an ulp of d_x).  X2 = false: one level, d_x.
template <bool X2 = true>
struct Q6kUnit {
  static constexpr bool kX2 = X2;
  struct Lane {
    uint32_t u, dsh;
    int ja;
  };
  struct W {
    u32x4_t q0, q1, hh;
    uint32_t sc, dd;
  };
  struct X {
    uint32_t xa[8], xb[8], ya[8], yb[8];
    float fA, fB;
    int sA[2], sB[2], tA[2], tB[2];
  };
  __device__ static Lane lane(int u) {
    Lane L;
    const int b = u >> 2, v = u & 3;
    L.u = (uint32_t)u;
    L.dsh = (uint32_t)(b & 1) * 16;
    L.ja = b * 8 + (v >> 1) * 4 + (v & 1);
    return L;
  }
  __device__ static void load(const uint8_t *w, const float *, const float *, const Q4kxArgs &a, int row,
                              const Lane &L, W &r) {
    const __amdgpu_buffer_rsrc_t rs = span_rsrc(w, (uint32_t)a.N * (uint32_t)a.row_bytes);
    const uint32_t ro = (uint32_t)row * (uint32_t)a.row_bytes, P16 = (uint32_t)a.K >> 2;  // 16 * K / 64
    r.q0 = bload16(rs, ro + 16u * L.u);
    r.q1 = bload16(rs, ro + P16 + 16u * L.u);
    r.hh = bload16(rs, ro + 2u * P16 + 16u * L.u);
    r.sc = bload_u32(rs, ro + 3u * P16 + 4u * L.u);
    r.dd = bload_u32(rs, ro + 13u * (P16 >> 2) + 4u * (L.u >> 3));  // 52 P + 4 (b / 2)
  }
  __device__ static void load_x(const uint8_t *q1, const uint8_t *q2, const uint8_t *de, const uint8_t *,
                                int64_t blk, X &x) {
    const u32x4_t *a1 = reinterpret_cast<const u32x4_t *>(q1 + blk * 32);
    const u32x4_t *b1 = reinterpret_cast<const u32x4_t *>(q1 + (blk + 2) * 32);
    const u32x4_t va0 = a1[0], va1 = a1[1], vb0 = b1[0], vb1 = b1[1];
#pragma unroll
    for (int k = 0; k < 4; k++) x.xa[k] = va0[k], x.xa[k + 4] = va1[k], x.xb[k] = vb0[k], x.xb[k + 4] = vb1[k];
    if constexpr (X2) {
      const u32x4_t *a2 = reinterpret_cast<const u32x4_t *>(q2 + blk * 32);
      const u32x4_t *b2 = reinterpret_cast<const u32x4_t *>(q2 + (blk + 2) * 32);
      const u32x4_t wa0 = a2[0], wa1 = a2[1], wb0 = b2[0], wb1 = b2[1];
#pragma unroll
      for (int k = 0; k < 4; k++) x.ya[k] = wa0[k], x.ya[k + 4] = wa1[k], x.yb[k] = wb0[k], x.yb[k + 4] = wb1[k];
    }
    const float2 dA = reinterpret_cast<const float2 *>(de)[blk], dB = reinterpret_cast<const float2 *>(de)[blk + 2];
    x.fA = X2 ? dA.y : dA.x;
    x.fB = X2 ? dB.y : dB.x;
#pragma unroll
    for (int s = 0; s < 2; s++) {
      int sa = 0, sb = 0, ta = 0, tb = 0;
#pragma unroll
      for (int k = 4 * s; k < 4 * s + 4; k++) {
        sa = dot4((int)x.xa[k], 0x01010101, sa);
        sb = dot4((int)x.xb[k], 0x01010101, sb);
        if constexpr (X2) {
          ta = dot4((int)x.ya[k], 0x01010101, ta);
          tb = dot4((int)x.yb[k], 0x01010101, tb);
        }
      }
      x.sA[s] = -32 * sa;
      x.sB[s] = -32 * sb;
      x.tA[s] = -32 * ta;
      x.tB[s] = -32 * tb;
    }
  }
  template <int MM>
  __device__ static void dot(const W &w, const X (&x)[MM], const Lane &L, float (&out)[MM]) {
    const float d = h2f((w.dd >> L.dsh) & 0xffffu);
    // The signed scales pass through an empty asm so that the conversion is a plain
    // v_cvt_f32_i32: folded with the byte extract, hipcc emitted v_cvt_f32_u32_sdwa with a
    // sext source, which reads a negative scale as 2^32 - |sc|.
    float sc[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      int si = __builtin_amdgcn_sbfe((int)w.sc, 8 * j, 8);
      asm volatile("" : "+v"(si));
      sc[j] = (float)si;
    }
    const uint32_t qw[8] = {w.q0[0], w.q0[1], w.q0[2], w.q0[3], w.q1[0], w.q1[1], w.q1[2], w.q1[3]};
    uint32_t qa[8], qb[8];
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const uint32_t hm = w.hh[k >> 1];
      qa[k] = (qw[k] & 0x0F0F0F0Fu) | (((k & 1) ? hm << 2 : hm << 4) & 0x30303030u);
      qb[k] = ((qw[k] >> 4) & 0x0F0F0F0Fu) | (((k & 1) ? hm >> 2 : hm) & 0x30303030u);
    }
#pragma unroll
    for (int mm = 0; mm < MM; mm++) {
      float vA = 0.f, vB = 0.f;
#pragma unroll
      for (int s = 0; s < 2; s++) {
        int a1 = x[mm].sA[s], b1 = x[mm].sB[s], a2 = x[mm].tA[s], b2 = x[mm].tB[s];
#pragma unroll
        for (int k = 4 * s; k < 4 * s + 4; k++) {
          a1 = dot4((int)qa[k], (int)x[mm].xa[k], a1);
          b1 = dot4((int)qb[k], (int)x[mm].xb[k], b1);
          if constexpr (X2) {
            a2 = dot4((int)qa[k], (int)x[mm].ya[k], a2);
            b2 = dot4((int)qb[k], (int)x[mm].yb[k], b2);
          }
        }
        const int cA = X2 ? __mul24(254, a1) + a2 : a1, cB = X2 ? __mul24(254, b1) + b2 : b1;
        vA = __fmaf_rn(sc[s], (float)cA, vA);
        vB = __fmaf_rn(sc[2 + s], (float)cB, vB);
      }
      out[mm] = d * __fmaf_rn(x[mm].fB, vB, x[mm].fA * vA);
    }
  }
};

// Rows of at least this many elements take single-level activations.
constexpr int64_t kX1MinK = 4096;

// Calls f with a default-constructed unit policy for (dt in {Q4_K, Q5_K, Q6_K_R}, K).
template <class F>
static int with_qk_unit(int dt, int64_t K, F &&f) {
  const bool x1 = K >= kX1MinK;
  if (dt == Q5_K) return x1 ? f(QkUnit<true, false>{}) : f(QkUnit<true, true>{});
  if (dt == Q6_K_R) return x1 ? f(Q6kUnit<false>{}) : f(Q6kUnit<true>{});
  return x1 ? f(QkUnit<false, false>{}) : f(QkUnit<false, true>{});
}


template <class U, class = void>
struct is_int4_unit {
  static constexpr bool value = false;
};
template <class U>
struct is_int4_unit<U, decltype(void(U::kInt4))> {
  static constexpr bool value = true;
};

template <class U>
__device__ __forceinline__ typename U::Lane unit_lane(int u, int G) {
  if constexpr (is_int4_unit<U>::value)
    return U::lane(u, G);
  else
    return U::lane(u);
}

template <int XDT>
__device__ __forceinline__ float4 load_x4(const void *x, int64_t i) {
  if constexpr (XDT == F32) {
    return *reinterpret_cast<const float4 *>(static_cast<const float *>(x) + i);
  } else {
    const uint2 u = *reinterpret_cast<const uint2 *>(static_cast<const uint16_t *>(x) + i);
    const uint32_t h[4] = {u.x & 0xffffu, u.x >> 16, u.y & 0xffffu, u.y >> 16};
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; j++) v[j] = XDT == BF16 ? bf2f(h[j]) : h2f(h[j]);
    return make_float4(v[0], v[1], v[2], v[3]);
  }
}

template <int ODT>
__device__ __forceinline__ void store_out(void *out, int64_t i, float y) {
  if constexpr (ODT == F32)
    static_cast<float *>(out)[i] = y;
  else if constexpr (ODT == BF16)
    static_cast<uint16_t *>(out)[i] = f2bf_rne(y);
  else
    static_cast<uint16_t *>(out)[i] = f2h_rne(y);
}

// The kernel body for workgroup bx of G persistent workgroups (grid row blockIdx.y).  ROWS
// (plain GEMV only): a team carries ROWS rows per iteration, rows g*ROWS*RW + team + j*RW, so
// ROWS times the bytes are in flight and the per-iteration reduction is paid once per ROWS
// rows.
template <class U, int MM, bool GATED, bool XIN, bool AOUT, int XDT, int ODT, int ROWS = 1>
__device__ __forceinline__ void q4kx_body(const Q4kxArgs &a, uint8_t *smem, const int bx, const int G) {
  static_assert(ROWS == 1 || !(GATED || AOUT), "ROWS > 1 is for the plain GEMV");
  constexpr int NW = GATED ? 2 : ROWS;  // weight rows in a register slot
  const int t = threadIdx.x, lane = t & 63;
  const int RW = a.RW, KB = a.K >> 5;
  const int team = t / a.TP, u = t - team * a.TP;
  const bool active = u < a.P;
  const typename U::Lane L = unit_lane<U>(active ? u : 0, a.G);
  const int SPAN = ROWS * RW;  // rows per group
  const int ngroups = (a.N + SPAN - 1) / SPAN;
  const int m0 = blockIdx.y * MM;
  // Iteration i of this workgroup -> row group: whole chunks of CG groups (32 rows with
  // AOUT), chunks strided over the grid.  Groups past the end load row N (zeros, no traffic).
  const int CG = AOUT ? 32 / RW : 1;
  const int nchunks = (ngroups + CG - 1) / CG;
  const int niter = ((nchunks - bx + G - 1) / G) * CG;
#define Q4KX_GRP(I) ((bx + ((I) / CG) * G) * CG + (I) % CG)
  // Weight j of a slot: the up weight of the same row (GATED, j = 1), else row j * RW of
  // the group.  Rows past the end load row N (zeros, no traffic).
#define Q4KX_LOAD_J(SLOT, GRP, J)                                             \
  do {                                                                        \
    int row_ = (GRP) * SPAN + team + (GATED ? 0 : (J) * RW);                  \
    row_ = row_ < a.N ? row_ : a.N;                                           \
    U::load((J) && GATED ? a.w1 : a.w0, (J) && GATED ? a.s1 : a.s0,          \
            (J) && GATED ? a.z1 : a.z0, a, row_, L, wr[SLOT][J]);             \
  } while (0)
#define Q4KX_LOAD(SLOT, GRP)                                                  \
  do {                                                                        \
    _Pragma("unroll") for (int j_ = 0; j_ < NW; j_++) Q4KX_LOAD_J(SLOT, GRP, j_); \
  } while (0)

  // One register slot: the next group's loads go out once the current one is reduced.
  // (Deeper rings -- two to four groups in flight per wave -- were measured slower: this
  // kernel is bound by VALU issue as much as by HBM, and more outstanding rows only spread
  // the DRAM traffic.)
  // Prepared activations are loaded before the first weights (measured 0.2-0.3 us faster at
  // 4096 x 14336: the shared x lines are not queued behind the weight stream); x quantized
  // in the kernel goes after them, so the weights stream during the quantization.
  typename U::W wr[1][NW];
  typename U::X xr[MM];
  if constexpr (XIN) Q4KX_LOAD(0, Q4KX_GRP(0));

  const int64_t lds_act = XIN ? q4kx_act_lds(MM, a.K) : 0;
  if constexpr (XIN) {
    // Quantize this workgroup's MM rows of x into LDS: a task is half a 32-block (sixteen
    // elements) on one lane, two lanes per block (act_quant16_fast).
    uint8_t *lq1 = smem, *lq2 = smem + (int64_t)MM * a.K;
    float2 *lde = reinterpret_cast<float2 *>(smem + 2 * (int64_t)MM * a.K);
    float *lsx = reinterpret_cast<float *>(smem + 2 * (int64_t)MM * a.K + 8 * (int64_t)MM * KB);
    const int ntask = MM * KB * 2, bd = (int)blockDim.x;
    // Element index of task i (clamped into range): rows of x are whole blocks, so the
    // tasks of (mm, block, half) are contiguous in x.
    auto xidx = [&](int i) __attribute__((always_inline)) {
      i = i < ntask ? i : ntask - 1;
      const int mm = MM == 1 ? 0 : i / (2 * KB);
      const int m = m0 + mm < a.M ? m0 + mm : a.M - 1;
      return (int64_t)m * a.K + (int64_t)(i - mm * 2 * KB) * 16;
    };
    auto quant_store = [&](const float (&v)[16], int task) __attribute__((always_inline)) {
      const ActQ16 q = act_quant16_fast(v);
      if (task < ntask) {  // both lanes of a block agree (ntask is even)
        const int blk = task >> 1, half = task & 1;
        *reinterpret_cast<u32x4_t *>(lq1 + blk * 32 + half * 16) = u32x4_t{q.q1[0], q.q1[1], q.q1[2], q.q1[3]};
        if constexpr (U::kX2)
          *reinterpret_cast<u32x4_t *>(lq2 + blk * 32 + half * 16) = u32x4_t{q.q2[0], q.q2[1], q.q2[2], q.q2[3]};
        if (half == 0) {
          lde[blk] = make_float2(q.d, q.e);
          lsx[blk] = q.sum;
        }
      }
    };
    constexpr int XR = XDT == F32 ? 4 : 2;  // 16-byte pieces of a task's sixteen elements
    auto to_f32 = [&](const u32x4_t (&raw)[XR], float (&v)[16]) __attribute__((always_inline)) {
#pragma unroll
      for (int j = 0; j < 16; j++) {
        const uint32_t w32 = raw[XDT == F32 ? j / 4 : j / 8][XDT == F32 ? j % 4 : (j % 8) / 2];
        if constexpr (XDT == F32)
          v[j] = __uint_as_float(w32);
        else
          v[j] = XDT == BF16 ? bf2f((j & 1) ? w32 >> 16 : w32 & 0xffffu) : h2f((j & 1) ? w32 >> 16 : w32 & 0xffffu);
      }
    };
    for (int base = 0; base < ntask; base += bd) {
      u32x4_t raw[XR];
      const uint8_t *xp = static_cast<const uint8_t *>(a.x) + xidx(base + t) * (XDT == F32 ? 4 : 2);
#pragma unroll
      for (int r = 0; r < XR; r++) raw[r] = *reinterpret_cast<const u32x4_t *>(xp + 16 * r);
      float v[16];
      to_f32(raw, v);
      if (base + t < ntask) quant_store(v, base + t);
    }
    __syncthreads();
#pragma unroll
    for (int mm = 0; mm < MM; mm++)
      U::load_x(lq1, lq2, reinterpret_cast<const uint8_t *>(lde), reinterpret_cast<const uint8_t *>(lsx),
                mm * KB + L.ja, xr[mm]);
  } else {
#pragma unroll
    for (int mm = 0; mm < MM; mm++) {
      const int m = m0 + mm < a.M ? m0 + mm : a.M - 1;
      U::load_x(a.ain, a.ain + a.in_q2, a.ain + a.in_d, a.ain + a.in_s, (int64_t)m * KB + L.ja, xr[mm]);
    }
  }
  if constexpr (!XIN) Q4KX_LOAD(0, Q4KX_GRP(0));

  const int hpt = a.TP >> 4;  // 16-lane rows per team
  float *part = reinterpret_cast<float *>(smem + lds_act);
  float *hbuf = part + (a.TP > 64 ? 2 * RW * NW * MM * hpt : 0);

  // One iteration: wait for the slot (straight-line form), reduce the group's rows, refill
  // the slot with the group D iterations ahead, write the outputs.  VALID is
  // workgroup-uniform; REFILL is a compile-time constant in the straight-line form.
  for (int it = 0; it < niter; it++) {
    const int grp = Q4KX_GRP(it);
    float res[NW][MM];
#pragma unroll
    for (int j = 0; j < NW; j++) {
      float c[MM];
      U::template dot<MM>(wr[0][j], xr, L, c);
      // Weight j is consumed: refill it with the next group's (unconditionally) before the
      // next weight's arithmetic, so the load has that much longer to arrive.
      Q4KX_LOAD_J(0, Q4KX_GRP(it + 1), j);
#pragma unroll
      for (int mm = 0; mm < MM; mm++) res[j][mm] = rsum16(active ? c[mm] : 0.f);
    }
    const int row = grp * SPAN + team;
    float *hb = hbuf + ((it / CG) & 1) * (MM * 32);
    if (a.TP <= 64) {
      // Team within one wave (TP in {16, 32, 64}): add its 16-lane rows in order.
#pragma unroll
      for (int mm = 0; mm < MM; mm++) {
        float tot[NW];
#pragma unroll
        for (int j = 0; j < NW; j++) {
          const float r0 = rl(res[j][mm], 0), r1 = rl(res[j][mm], 16);
          const float r2 = rl(res[j][mm], 32), r3 = rl(res[j][mm], 48);
          if (a.TP == 64)
            tot[j] = ((r0 + r1) + r2) + r3;
          else if (a.TP == 32)
            tot[j] = lane < 32 ? r0 + r1 : r2 + r3;
          else
            tot[j] = lane < 16 ? r0 : (lane < 32 ? r1 : (lane < 48 ? r2 : r3));
        }
        if (u == 0 && row < a.N) {
          float y = tot[0];
          if (GATED) y = gate_act(tot[0], a.act) * tot[NW - 1];
          if (a.out && m0 + mm < a.M) store_out<ODT>(a.out, (int64_t)(m0 + mm) * a.N + row, y);
          if (AOUT) hb[mm * 32 + (row & 31)] = y;
        }
#pragma unroll
        for (int j = 1; j < (GATED ? 1 : NW); j++)
          if (u == 0 && row + j * RW < a.N && a.out && m0 + mm < a.M)
            store_out<ODT>(a.out, (int64_t)(m0 + mm) * a.N + row + j * RW, tot[j]);
      }
    } else {
      // Team wider than a wave: 16-lane row sums through LDS, added in row order.
      float *pp = part + (it & 1) * (RW * NW * MM * hpt);
#pragma unroll
      for (int j = 0; j < NW; j++) {
#pragma unroll
        for (int mm = 0; mm < MM; mm++)
          if ((lane & 15) == 0) pp[((team * NW + j) * MM + mm) * hpt + (u >> 4)] = res[j][mm];
      }
      __syncthreads();
      if (t < RW * MM) {
        const int tm = t / MM, mm = t - tm * MM;
        float tot[NW];
#pragma unroll
        for (int j = 0; j < NW; j++) {
          float acc = 0.f;
          for (int k = 0; k < hpt; k++) acc += pp[((tm * NW + j) * MM + mm) * hpt + k];
          tot[j] = acc;
        }
        const int r2 = grp * SPAN + tm;
        if (r2 < a.N) {
          float y = tot[0];
          if (GATED) y = gate_act(tot[0], a.act) * tot[NW - 1];
          if (a.out && m0 + mm < a.M) store_out<ODT>(a.out, (int64_t)(m0 + mm) * a.N + r2, y);
          if (AOUT) hb[mm * 32 + (r2 & 31)] = y;
        }
#pragma unroll
        for (int j = 1; j < (GATED ? 1 : NW); j++)
          if (r2 + j * RW < a.N && a.out && m0 + mm < a.M)
            store_out<ODT>(a.out, (int64_t)(m0 + mm) * a.N + r2 + j * RW, tot[j]);
      }
    }
    if (AOUT && it % CG == CG - 1) {
      // The chunk's 32 rows are complete: quantize them into the act layout of (M, N).
      __syncthreads();
      const int chunk = grp / CG;
      if (t < 8 * MM) {
        const int mm = t >> 3, sub = t & 7;
        const float v[4] = {hb[mm * 32 + sub * 4], hb[mm * 32 + sub * 4 + 1], hb[mm * 32 + sub * 4 + 2],
                            hb[mm * 32 + sub * 4 + 3]};
        const ActQ q = act_quant8_fast(v);
        if (m0 + mm < a.M && chunk * 32 < a.N) {
          const int64_t blk = (int64_t)(m0 + mm) * (a.N >> 5) + chunk;
          reinterpret_cast<uint32_t *>(a.aout + blk * 32)[sub] = q.q1;
          reinterpret_cast<uint32_t *>(a.aout + a.out_q2 + blk * 32)[sub] = q.q2;
          if (sub == 0) {
            reinterpret_cast<float2 *>(a.aout + a.out_d)[blk] = make_float2(q.d, q.e);
            reinterpret_cast<float *>(a.aout + a.out_s)[blk] = q.sum;
          }
        }
      }
    }
  }
#undef Q4KX_LOAD
#undef Q4KX_LOAD_J
#undef Q4KX_GRP
}

template <class U, int MM, bool GATED, bool XIN, bool AOUT, int XDT, int ODT, int ROWS = 1>
__global__ __launch_bounds__(512) void gemv_q4kx_kernel(Q4kxArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  q4kx_body<U, MM, GATED, XIN, AOUT, XDT, ODT, ROWS>(a, smem, (int)blockIdx.x, (int)gridDim.x);
}

// ---------------------------------------------------------------------------
// MoE grouped decode GEMV (ops.MoEGemmQ, ops/moe.go:101-111, 242-265):
//   out[p, n] = w(p) * x[row(p)] . dequant(W[e(p)])[n],  row(p) = rpp ? p : p / topk,
// for the expert-sorted pairs.  grid.y = expert.  Each workgroup finds its expert's pair
// segment by binary search over the sorted expert ids (the workgroups with blockIdx.x == 0
// also write Light's counts / offsets scratch), quantizes the x rows of up to MM pairs at
// a time into LDS, and streams the expert's weight rows as the dense GEMV does.  Teams
// fit in one wave (K <= 4096).
// ---------------------------------------------------------------------------
struct MoeXArgs {
  Q4kxArgs g;  // w0 = expert stack, N, K, P, TP, RW, row_bytes; x = F32 rows of x
  const int64_t *pairs, *expts;
  int32_t *counts, *offsets;
  const float *topk_w;
  int64_t size_m, expert_bytes, rows, npairs;
  int64_t up_off;  // GATED: byte offset of the up rows inside an expert (I rows after gate)
  int E, topk, rpp, act;
  // ROUTE: router probabilities (T, E) and MoERoute's outputs, written by workgroup (0, 0).
  const float *probs;
  int64_t *topk_ids, *sorted_pairs_out, *sorted_expts_out;
  float *weights_out;
  int T, normalize;
};

// MoERoute inside a workgroup, for T * topk <= 64 pairs and T <= 8 tokens: wave t selects
// token t's top-k (topk_row_any, as moe_route_kernel; or the rank path below), then wave 0
// places each pair at its rank in the stable expert order (pairs of one expert keep pair
// order).  The LDS arrays end as MoERoute's outputs: re/rw per pair, se/sp in sorted order.
//
// Where the workgroup has a thread per probability (T E <= blockDim.x), the top-k is found by
// rank instead: each thread counts the keys of its row above its own (from LDS, the same
// address for every lane of a row at a time), and the keys of rank < topk are the selection,
// in rank order -- the order the repeated maxima find them (keys are distinct).  One pass
// instead of topk rounds of wave-wide maxima (E = 128, topk = 8: 3 -> ~0.5 us).
__device__ void route_in_workgroup(const MoeXArgs &ma, int *re, float *rw, int *se, int *sp) {
  __shared__ uint64_t rkeys[512];
  __shared__ int rpart[512];
  __shared__ float rsel[64];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int M = (int)ma.npairs;
  if (ma.T * ma.E <= (int)blockDim.x && ma.T * ma.E <= 512) {
    const int E = ma.E, n = ma.T * E;
    // nq threads per key, each counting over its quarter (half, ...) of the row.
    const int nq = (int)blockDim.x / n >= 4 ? 4 : ((int)blockDim.x / n >= 2 ? 2 : 1);
    const int ki = t % n, q = t / n;
    const int tok = ki / E, e = ki - tok * E;
    uint64_t key = 0;
    if (t < n) {
      key = ((uint64_t)ord_f32(ma.probs[t]) << 32) | (uint64_t)(0xffffffffu - (uint32_t)e);
      rkeys[t] = key;
    }
    __syncthreads();
    if (q < nq) {
      key = rkeys[ki];
      const uint64_t *row = rkeys + tok * E;
      const int j0 = E * q / nq, j1 = E * (q + 1) / nq;
      int rank = 0, j = j0;
      // Sixteen independent LDS reads per round (a read-compare loop waits out the LDS latency
      // on every key).
      for (; j + 16 <= j1; j += 16) {
        uint64_t kk[16];
#pragma unroll
        for (int i = 0; i < 16; i++) kk[i] = row[j + i];
#pragma unroll
        for (int i = 0; i < 16; i++) rank += kk[i] > key ? 1 : 0;
      }
      for (; j < j1; j++) rank += row[j] > key ? 1 : 0;
      rpart[t] = rank;
    }
    __syncthreads();
    if (t < n) {
      int rank = 0;
      for (int qq = 0; qq < nq; qq++) rank += rpart[qq * n + t];
      if (rank < ma.topk) {
        re[tok * ma.topk + rank] = e;
        rsel[tok * ma.topk + rank] = unord_f32((uint32_t)(key >> 32));
      }
    }
    __syncthreads();
    if (t < ma.T * ma.topk) {
      // den: the left-to-right f32 sum of the token's selected values in slot order (every
      // lane of a token adds the same values in the same order), then each slot's weight.
      const int tk = t / ma.topk;
      float den = 0.f;
      for (int jj = 0; jj < ma.topk; jj++) den = __fadd_rn(den, rsel[tk * ma.topk + jj]);
      const float v = rsel[t];
      rw[t] = ma.normalize ? __fdiv_rn(v, den) : v;
    }
  } else if (wave < ma.T) {
    float sv, den;
    int si;
    topk_row_any(ma.probs + (int64_t)wave * ma.E, ma.E, ma.topk, lane, sv, si, den);
    if (lane < ma.topk) {
      re[wave * ma.topk + lane] = si;
      rw[wave * ma.topk + lane] = ma.normalize ? __fdiv_rn(sv, den) : sv;
    }
  }
  __syncthreads();
  if (wave == 0) {
    const bool valid = lane < M;
    const int ep = valid ? re[lane] : 0x7fffffff;
    int pos = 0;
    for (int q = 0; q < M; q++) {
      const int eq = __builtin_amdgcn_readlane(ep, q);
      pos += (eq < ep || (eq == ep && q < lane)) ? 1 : 0;
    }
    if (valid) {
      se[pos] = ep;
      sp[pos] = lane;
    }
  }
  __syncthreads();
}


// Segment j of the sorted expert ids (segment starts: i == 0 or v[i] != v[i-1]), found by
// one wave: 256 ids per round as four independent loads per lane, ballots of the start
// flags, and the lane whose start rank is j.  Returns [seg0, seg1), the segment's expert e
// and the expert before it (eprev, -1 for the first); seg0 = -1 when there is no segment j.
struct Seg {
  int64_t seg0, seg1;
  int e, eprev;
};

__device__ __forceinline__ Seg find_segment(const int64_t *__restrict__ v, int64_t n, int j, int lane) {
  Seg sg{-1, n, -1, -1};
  const uint64_t lt = (1ull << lane) - 1;
  int64_t cnt = 0;
  for (int64_t base = 0; base < n; base += 256) {
    int cur[4], prv[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
      int64_t i = base + 64 * c + lane;
      i = i < n ? i : n - 1;
      cur[c] = (int)v[i];
      prv[c] = (int)v[i > 0 ? i - 1 : 0];
    }
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const int64_t i = base + 64 * c + lane;
      const bool st = i < n && (i == 0 || cur[c] != prv[c]);
      const uint64_t m = __ballot(st);
      const int64_t rank = cnt + __popcll(m & lt);
      if (sg.seg0 < 0) {
        const uint64_t hit = __ballot(st && rank == j);
        if (hit) {
          const int pos = __ffsll((unsigned long long)hit) - 1;
          sg.seg0 = base + 64 * c + pos;
          sg.e = __builtin_amdgcn_readlane(cur[c], pos);  // pos is wave-uniform
          sg.eprev = sg.seg0 == 0 ? -1 : __builtin_amdgcn_readlane(prv[c], pos);
        }
      }
      const uint64_t nxt = __ballot(st && rank == (int64_t)j + 1);
      if (nxt && sg.seg1 == n) sg.seg1 = base + 64 * c + (__ffsll((unsigned long long)nxt) - 1);
      cnt += __popcll(m);
    }
    if (sg.seg1 < n || cnt > j + 1) break;  // wave-uniform
  }
  return sg;
}

// Segment j of the expert-sorted ids held in LDS (n <= 64), as find_segment.
__device__ __forceinline__ Seg lds_segment(const int *se, int n, int j, int lane) {
  Seg sg{-1, n, -1, -1};
  const bool st = lane < n && (lane == 0 || se[lane] != se[lane > 0 ? lane - 1 : 0]);
  uint64_t m = __ballot(st);
  for (int i = 0; i < j && m; i++) m &= m - 1;
  if (!m) return sg;
  sg.seg0 = __ffsll((unsigned long long)m) - 1;
  m &= m - 1;
  sg.seg1 = m ? __ffsll((unsigned long long)m) - 1 : n;
  sg.e = se[sg.seg0];
  sg.eprev = sg.seg0 == 0 ? -1 : se[sg.seg0 - 1];
  return sg;
}

// The kernel body for workgroup (bx, by) of a (G, gridDim.y) grid; r_* are the routing's LDS
// arrays (64 entries each, ROUTE only).  A workgroup without work returns after the routing.
template <class U, int MM, bool GATED, bool ROUTE = false, bool COH = false>
__device__ __forceinline__ void moe_x_body(const MoeXArgs &ma, uint8_t *smem, int *r_e, float *r_w, int *r_se,
                                           int *r_sp, const int bx, const int by, const int G) {
  const Q4kxArgs &a = ma.g;
  const int t = threadIdx.x, lane = t & 63;
  // One row of x (a single token's gate/up, plain kernel): every pair reads row 0, so the first slice of
  // x loads (all of x up to K = 2048) goes out now, beside the expert-id search instead of
  // after it.
  constexpr int XT = 4;
  const bool x1 = (!GATED || ROUTE) && ma.rows == 1;  // (the plain gated kernel has no registers to spare)
  const int KB0 = a.K >> 5, ntask0 = MM * KB0 * 8;
  float4 xpre = make_float4(0.f, 0.f, 0.f, 0.f);
  // One row of x and one pair per pass (a single token's experts): the row is quantized into
  // LDS slot 0 once, up front -- in the routed kernel by the waves that do not route, while
  // the routing waves select the top-k -- so it is off the path from the routing to the first
  // dot.  (The barriers of the routing / the pass publish it.)
  const bool xq0 = x1 && MM == 1;
  if (xq0) {
    // Whole waves (act_quant8_fast works on aligned 8-lane groups) past the routing's: one wave
    // per token, or a thread per probability (route_in_workgroup's rank path).
    const int rt = ma.T * ma.E <= (int)blockDim.x && ma.T * ma.E <= 512 ? (ma.T * ma.E + 63) & ~63 : 64 * ma.T;
    const int t0 = ROUTE ? rt : 0;
    const int nth = (int)blockDim.x - t0;
    if (t >= t0 && nth > 0) {
      // The first XP passes' loads go out together (a load-quantize loop waited out one
      // memory latency per pass).
      constexpr int XP = 4;
      float4 xp[XP];
#pragma unroll
      for (int i = 0; i < XP; i++) {
        const int task = i * nth + t - t0, tc = task < ntask0 ? task : ntask0 - 1;
        xp[i] = *reinterpret_cast<const float4 *>(static_cast<const float *>(a.x) + tc * 4);
      }
      for (int base = 0, pass = 0; base < ntask0; base += nth, pass++) {
        const int task = base + t - t0, tc = task < ntask0 ? task : ntask0 - 1;
        const int blk = tc >> 3, sub = tc & 7;
        float4 xq = make_float4(0.f, 0.f, 0.f, 0.f);
        if (pass < XP) {
#pragma unroll
          for (int i = 0; i < XP; i++)
            if (pass == i) xq = xp[i];
        } else {
          xq = *reinterpret_cast<const float4 *>(static_cast<const float *>(a.x) + blk * 32 + sub * 4);
        }
        const float v[4] = {xq.x, xq.y, xq.z, xq.w};
        const ActQ q = act_quant8_fast(v);
        if (task < ntask0) {
          reinterpret_cast<uint32_t *>(smem + blk * 32)[sub] = q.q1;
          reinterpret_cast<uint32_t *>(smem + (int64_t)a.K + blk * 32)[sub] = q.q2;
          if (sub == 0) {
            reinterpret_cast<float2 *>(smem + 2 * (int64_t)a.K)[blk] = make_float2(q.d, q.e);
            reinterpret_cast<float *>(smem + 2 * (int64_t)a.K + 8 * (int64_t)KB0)[blk] = q.sum;
          }
        }
      }
    }
    if constexpr (!ROUTE) __syncthreads();
  } else if (x1) {
    const int task = t < ntask0 ? t : ntask0 - 1;
    const int blk = task >> 3, sub = task & 7, kb = blk % KB0;
    xpre = *reinterpret_cast<const float4 *>(static_cast<const float *>(a.x) + kb * 32 + sub * 4);
  }
  Seg sg;
  if constexpr (ROUTE) {
    route_in_workgroup(ma, r_e, r_w, r_se, r_sp);
    if (bx == 0 && by == 0) {
      for (int i = t; i < (int)ma.npairs; i += blockDim.x) {
        ma.topk_ids[i] = r_e[i];
        ma.weights_out[i] = r_w[i];
        ma.sorted_pairs_out[i] = r_sp[i];
        ma.sorted_expts_out[i] = r_se[i];
      }
    }
    sg = lds_segment(r_se, (int)ma.npairs, by, lane);
  } else {
    sg = find_segment(ma.expts, ma.npairs, by, lane);
  }
  if (sg.seg0 < 0) return;
  const int64_t seg0 = sg.seg0, seg1 = sg.seg1;
  const int e = sg.e;
  if (bx == 0 && ma.counts && ma.offsets) {
    // counts / offsets of the experts (eprev, e], and of (e, E) after the last segment.
    const int lo = sg.eprev + 1 > 0 ? sg.eprev + 1 : 0;
    const int hi = seg1 == ma.npairs ? ma.E - 1 : (e < ma.E ? e : ma.E - 1);
    for (int x = lo + t; x <= hi; x += blockDim.x) {
      ma.counts[x] = x == e ? (int32_t)(seg1 - seg0) : 0;
      ma.offsets[x] = x <= e ? (int32_t)seg0 : (int32_t)seg1;
    }
    if (seg1 == ma.npairs && t == 0) ma.offsets[ma.E] = (int32_t)seg1;
  }
  if (e < 0 || e >= ma.E) return;
  const uint8_t *w = a.w0 + (int64_t)e * ma.expert_bytes;
  const int RW = a.RW, KB = a.K >> 5;
  const int team = t / a.TP, u = t - team * a.TP;
  const bool active = u < a.P;
  const typename U::Lane L = unit_lane<U>(active ? u : 0, a.G);
  const int ngroups = (a.N + RW - 1) / RW;
  const int niter = (ngroups - bx + G - 1) / G;
  if (niter <= 0) return;
  uint8_t *lq1 = smem, *lq2 = smem + (int64_t)MM * a.K;
  float2 *lde = reinterpret_cast<float2 *>(smem + 2 * (int64_t)MM * a.K);
  float *lsx = reinterpret_cast<float *>(smem + 2 * (int64_t)MM * a.K + 8 * (int64_t)MM * KB);

  for (int64_t c0 = seg0; c0 < seg1; c0 += MM) {
    int64_t pid[MM], xrow[MM];
#pragma unroll
    for (int mm = 0; mm < MM; mm++) {
      int64_t p = c0 + mm < seg1 ? (ROUTE ? (int64_t)r_sp[c0 + mm] : ma.pairs[c0 + mm]) : -1;
      if (p < 0 || p >= ma.size_m) p = -1;
      pid[mm] = p;
      int64_t r = p < 0 ? 0 : (ma.rpp ? p : p / ma.topk);
      xrow[mm] = r < ma.rows ? r : ma.rows - 1;
    }
    constexpr int NW = GATED ? 2 : 1;
    typename U::W wr[NW];
    {
      int row = bx * RW + team;
      row = row < a.N ? row : a.N;
      U::load(w, a.s0, a.z0, a, row, L, wr[0]);
      if (GATED) U::load(w + ma.up_off, a.s0, a.z0, a, row, L, wr[NW - 1]);
    }
    if (c0 != seg0) __syncthreads();  // every lane has its activations of the previous chunk
    const int ntask = xq0 ? 0 : MM * KB * 8;
    const float *x = static_cast<const float *>(a.x);
    for (int base = 0; base < ntask; base += XT * (int)blockDim.x) {
      float4 xv[XT];
      {
#pragma unroll
        for (int i = 0; i < XT; i++) {
          if (i == 0 && x1 && c0 == seg0 && base == 0) {
            xv[0] = xpre;
            continue;
          }
          int task = base + i * (int)blockDim.x + t;
          task = task < ntask ? task : ntask - 1;
          const int blk = task >> 3, sub = task & 7, mm = blk / KB, kb = blk - mm * KB;
          int64_t r = 0;
#pragma unroll
          for (int k = 0; k < MM; k++) r = k == mm ? xrow[k] : r;
          xv[i] = *reinterpret_cast<const float4 *>(x + r * a.K + kb * 32 + sub * 4);
        }
      }
#pragma unroll
      for (int i = 0; i < XT; i++) {
        const int task = base + i * (int)blockDim.x + t;
        const int blk = task >> 3, sub = task & 7;
        const float v[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
        const ActQ q = act_quant8_fast(v);
        if (task < ntask) {
          reinterpret_cast<uint32_t *>(lq1 + blk * 32)[sub] = q.q1;
          reinterpret_cast<uint32_t *>(lq2 + blk * 32)[sub] = q.q2;
          if (sub == 0) {
            lde[blk] = make_float2(q.d, q.e);
            lsx[blk] = q.sum;
          }
        }
      }
    }
    __syncthreads();
    typename U::X xr[MM];
#pragma unroll
    for (int mm = 0; mm < MM; mm++)
      U::load_x(lq1, lq2, reinterpret_cast<const uint8_t *>(lde), reinterpret_cast<const uint8_t *>(lsx),
                mm * KB + L.ja, xr[mm]);
    float wp[MM];
#pragma unroll
    for (int mm = 0; mm < MM; mm++) wp[mm] = pid[mm] >= 0 && ma.topk_w ? ma.topk_w[pid[mm]] : 1.f;

    for (int it = 0; it < niter; it++) {
      const int grp = bx + it * G;
      float c[NW][MM];
#pragma unroll
      for (int j = 0; j < NW; j++) U::template dot<MM>(wr[j], xr, L, c[j]);
      {
        int row = (grp + G) * RW + team;
        row = row < a.N ? row : a.N;
        U::load(w, a.s0, a.z0, a, row, L, wr[0]);
        if (GATED) U::load(w + ma.up_off, a.s0, a.z0, a, row, L, wr[NW - 1]);
      }
      const int row = grp * RW + team;
#pragma unroll
      for (int mm = 0; mm < MM; mm++) {
        float tot[NW];
#pragma unroll
        for (int j = 0; j < NW; j++) {
          const float r16 = rsum16(active ? c[j][mm] : 0.f);
          const float r0 = rl(r16, 0), r1 = rl(r16, 16), r2 = rl(r16, 32), r3 = rl(r16, 48);
          if (a.TP == 64)
            tot[j] = ((r0 + r1) + r2) + r3;
          else if (a.TP == 32)
            tot[j] = lane < 32 ? r0 + r1 : r2 + r3;
          else
            tot[j] = lane < 16 ? r0 : (lane < 32 ? r1 : (lane < 48 ? r2 : r3));
        }
        const float y = GATED ? gate_act(tot[0], ma.act) * tot[NW - 1] : tot[0] * wp[mm];
        if (u == 0 && row < a.N && pid[mm] >= 0) {
          float *o = static_cast<float *>(a.out) + pid[mm] * a.N + row;
          if constexpr (COH)  // read by other workgroups in the same launch: agent-coherent
            __hip_atomic_store(o, y, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          else
            *o = y;
        }
      }
    }
  }
}

template <class U, int MM, bool GATED, bool ROUTE = false>
__global__ __launch_bounds__(512) void moe_gemv_x_kernel(MoeXArgs ma) {
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ int r_e[ROUTE ? 64 : 1], r_se[ROUTE ? 64 : 1], r_sp[ROUTE ? 64 : 1];
  __shared__ float r_w[ROUTE ? 64 : 1];
  moe_x_body<U, MM, GATED, ROUTE>(ma, smem, r_e, r_w, r_se, r_sp, (int)blockIdx.x, (int)blockIdx.y, (int)gridDim.x);
}

// ---------------------------------------------------------------------------
// MoE decode down projection with MoECombine in its epilogue (ops.MoEGemmQ with the routing
// weights, then ops.MoECombine: ops/moe.go:209-265, nn/moe.go:230-235):
//   y[t, n] = sum over slots s of w(t,s) * h[t*topk+s] . dequant(W[e(t,s)])[n],
// the slots added in slot order as Light's Add chain does.  Token-major: grid.y = token, and a
// workgroup's teams are (row, slot) pairs -- RW / topk rows times topk slots -- so a team keeps
// one slot's activations in registers for the whole kernel.  Each pair's value is computed by
// exactly the instruction sequence of moe_gemv_x_kernel (same quantization of h, same unit
// dot, same 16-lane and team sums, same multiply by w), and the combine adds them in the order
// of moe_combine_kernel, so y is bit-identical to moe_gemm_q followed by moe_combine.
// ---------------------------------------------------------------------------
struct MoeCombArgs {
  Q4kxArgs g;  // w0 = expert stack (E, N, K); x = F32 h (M, K); out = y (T, N)
  const int64_t *pairs, *expts;
  int32_t *counts, *offsets;  // nullable: written by workgroup (0, 0)
  const float *topk_w;        // nullable
  int64_t expert_bytes, npairs;
  int E, topk;
};

// The kernel body for workgroup bx of G (token tok).  FUSED (the one-launch MoE block): the
// slots' experts and routing weights come from the workgroup's own routing (slot_e, slot_w),
// the first weights go out before hook() -- which waits until h is complete and returns false
// if it gave up -- and h is read with agent-coherent loads after it.  A workgroup whose hook
// gave up writes NaN to its rows of y instead of sums over an h that may be incomplete.
struct NoWait {
  __device__ bool operator()() const { return true; }
};

template <class U, bool FUSED = false, class Hook = NoWait>
__device__ __forceinline__ void moe_comb_body(const MoeCombArgs &ma, uint8_t *smem, const int bx, const int tok,
                                              const int G, const int *slot_e = nullptr,
                                              const float *slot_w = nullptr, const Hook &hook = Hook()) {
  const Q4kxArgs &a = ma.g;
  const int t = threadIdx.x, lane = t & 63;
  const int topk = ma.topk;
  const int RW = a.RW, KB = a.K >> 5, RPW = RW / topk;  // rows per workgroup
  // LDS: act of the token's topk h rows | expert per slot | pair values [RPW][topk]
  uint8_t *lq1 = smem, *lq2 = smem + (int64_t)topk * a.K;
  float2 *lde = reinterpret_cast<float2 *>(smem + 2 * (int64_t)topk * a.K);
  float *lsx = reinterpret_cast<float *>(smem + 2 * (int64_t)topk * a.K + 8 * (int64_t)topk * KB);
  int *lexp = reinterpret_cast<int *>(smem + q4kx_act_lds(topk, a.K));
  float *lval = reinterpret_cast<float *>(lexp + 64);
  // The token's h rows do not depend on the routing: their first loads go out first.
  constexpr int XT = 4;
  const int ntask = topk * KB * 8, bd = (int)blockDim.x;
  const float *x = static_cast<const float *>(a.x) + (int64_t)tok * topk * a.K;
  float4 xv[XT];
  if constexpr (!FUSED) {
#pragma unroll
    for (int i = 0; i < XT; i++) {
      const int task = i * bd + t < ntask ? i * bd + t : ntask - 1;
      xv[i] = *reinterpret_cast<const float4 *>(x + (int64_t)(task >> 3) * 32 + (task & 7) * 4);
    }
  }
  if (!FUSED && bx == 0 && tok == 0 && ma.offsets) {
    for (int e = t; e <= ma.E; e += blockDim.x) {
      auto lower = [&](int64_t v) {
        int64_t lo = 0, hi = ma.npairs;
        while (lo < hi) {
          const int64_t mid = (lo + hi) >> 1;
          if (ma.expts[mid] < v) lo = mid + 1; else hi = mid;
        }
        return lo;
      };
      const int64_t o = lower(e);
      ma.offsets[e] = (int32_t)o;
      if (e < ma.E && ma.counts) ma.counts[e] = (int32_t)(lower(e + 1) - o);
    }
  }
  // Expert of each of the token's slots, from the expert-sorted pair list (-1: none).
  if constexpr (FUSED) {
    if (t < topk) lexp[t] = slot_e[(int64_t)tok * topk + t];
  } else {
    if (t < topk) lexp[t] = -1;
    __syncthreads();
    for (int64_t i = t; i < ma.npairs; i += blockDim.x) {
      const int64_t p = ma.pairs[i];
      if (p >= (int64_t)tok * topk && p < (int64_t)(tok + 1) * topk) lexp[p - (int64_t)tok * topk] = (int)ma.expts[i];
    }
  }
  __syncthreads();
  const int team = t / a.TP, u = t - team * a.TP;
  const int slot = team % topk, rloc = team / topk;
  const bool active = u < a.P && rloc < RPW;
  const typename U::Lane L = unit_lane<U>(active ? u : 0, a.G);
  int e = lexp[slot];
  const bool ok = e >= 0 && e < ma.E;
  e = ok ? e : 0;
  const uint8_t *w = a.w0 + (int64_t)e * ma.expert_bytes;
  const int ngroups = (a.N + RPW - 1) / RPW;
  const int niter = (ngroups - bx + G - 1) / G;
  // The first weights go out as soon as the experts are known, before h is read.
  typename U::W wr;
  {
    int row = bx * RPW + rloc;
    row = row < a.N && rloc < RPW ? row : a.N;
    U::load(w, a.s0, a.z0, a, row, L, wr);
  }
  // FUSED: h is read once the hook returns, agent-coherently (sc1 buffer loads over the token's
  // rows), the first XT tasks per thread all at once.
  __amdgpu_buffer_rsrc_t hr = span_rsrc(x, (uint32_t)ntask * 16u);
  auto hload = [&](int task) __attribute__((always_inline)) {
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(hr, (uint32_t)task * 16u, 0, 16 /* sc1 */);
    return make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]), __uint_as_float(v[3]));
  };
  bool h_ok = true;
  if constexpr (FUSED) {
    h_ok = hook();
#pragma unroll
    for (int i = 0; i < XT; i++) xv[i] = hload(i * bd + t < ntask ? i * bd + t : ntask - 1);
  }
  // Quantize the token's topk rows of h into LDS, as moe_gemv_x_kernel does (eight lanes per
  // 32-block; the first XT tasks per thread were loaded at the start).
  for (int base = 0; base < ntask; base += bd) {
    const int task = base + t < ntask ? base + t : ntask - 1;
    const int blk = task >> 3, sub = task & 7;
    float4 xq;
    if (FUSED && base >= XT * bd) {
      xq = hload(task);
    } else if (base < XT * bd) {
#pragma unroll
      for (int i = 0; i < XT; i++)
        if (base == i * bd) xq = xv[i];
    } else {
      xq = *reinterpret_cast<const float4 *>(x + (int64_t)blk * 32 + sub * 4);
    }
    const float v[4] = {xq.x, xq.y, xq.z, xq.w};
    const ActQ q = act_quant8_fast(v);
    if (base + t < ntask) {
      reinterpret_cast<uint32_t *>(lq1 + blk * 32)[sub] = q.q1;
      reinterpret_cast<uint32_t *>(lq2 + blk * 32)[sub] = q.q2;
      if (sub == 0) {
        lde[blk] = make_float2(q.d, q.e);
        lsx[blk] = q.sum;
      }
    }
  }
  __syncthreads();
  const int64_t p = (int64_t)tok * topk + slot;
  const float wp = FUSED ? slot_w[p] : (ma.topk_w ? ma.topk_w[p] : 1.f);
  typename U::X xr[1];
  U::load_x(lq1, lq2, reinterpret_cast<const uint8_t *>(lde), reinterpret_cast<const uint8_t *>(lsx),
            slot * KB + L.ja, xr[0]);
  for (int it = 0; it < niter; it++) {
    const int grp = bx + it * G;
    float c[1];
    U::template dot<1>(wr, xr, L, c);
    {
      int row = (grp + G) * RPW + rloc;
      row = row < a.N && rloc < RPW ? row : a.N;
      U::load(w, a.s0, a.z0, a, row, L, wr);
    }
    const float r16 = rsum16(active ? c[0] : 0.f);
    const float r0 = rl(r16, 0), r1 = rl(r16, 16), r2 = rl(r16, 32), r3 = rl(r16, 48);
    float tot;
    if (a.TP == 64)
      tot = ((r0 + r1) + r2) + r3;
    else if (a.TP == 32)
      tot = lane < 32 ? r0 + r1 : r2 + r3;
    else
      tot = lane < 16 ? r0 : (lane < 32 ? r1 : (lane < 48 ? r2 : r3));
    float *vb = lval + (it & 1) * (RPW * topk);
    if (u == 0 && rloc < RPW) vb[rloc * topk + slot] = ok ? tot * wp : 0.f;
    __syncthreads();
    const int row = grp * RPW + t;
    if (t < RPW && row < a.N) {
      float acc = vb[t * topk];
      for (int s2 = 1; s2 < topk; s2++) acc = __fadd_rn(acc, vb[t * topk + s2]);
      static_cast<float *>(a.out)[(int64_t)tok * a.N + row] = h_ok ? acc : __builtin_nanf("");
    }
  }
}

template <class U>
__global__ __launch_bounds__(512) void moe_down_combine_kernel(MoeCombArgs ma) {
  extern __shared__ __align__(16) uint8_t smem[];
  moe_comb_body<U>(ma, smem, (int)blockIdx.x, (int)blockIdx.y, (int)gridDim.x);
}

// ---------------------------------------------------------------------------
// The MoE decode block in one launch (one token): MoERoute + routed gated gate/up
// (moe_x_body, ROUTE) and then the down projection with MoECombine (moe_comb_body, FUSED),
// with a grid barrier between them.  Every workgroup routes the token itself, so after its
// gate/up rows it already knows the experts of the down projection: it issues its first
// down-weight loads, waits at the barrier, and only then reads h.  h goes out as
// agent-coherent stores (complete before the workgroup arrives) and comes back as
// agent-coherent loads, so the barrier needs no cache-wide release or acquire.
//
// Barrier words (a file-scope device array; see moe_block_bar): arrival counters k < 16 at
// 64 k (workgroup bx arrives at counter bx % 16), the top counter at 64 * 16, and 16 copies of
// the generation at 64 * (17 + r).  A workgroup reads its copy of the generation before it
// arrives; the last arrival at a counter resets it and arrives at the top counter; the last
// arrival there resets it and bumps every copy; the others poll their copy.  The state
// returns to zero counts after every launch, so graph replays work: a workgroup always
// arrives before it waits, so the last one to arrive completes the barrier even when others
// have already given up.
//
// The wait needs the whole grid resident at once.  The host sizes the grid to the occupancy
// and serves one stream, but kernels of other streams or processes can hold CUs, so the wait
// is bounded (`limit` polls, each a device-scope load and an s_sleep(1): by default 2^22,
// at least 0.1 s and a few seconds at most, against a few microseconds for a normal wait).
// A workgroup that gives up sets the failure word (64 * (17 + 16)) and the host-visible
// flag, and writes NaN to its rows of y; the host reports the failure as an error
// (hq_moe_block_q / hq_moe_block_q_check).
//
// Ordering is carried by the accesses to h themselves, not by release / acquire on the barrier
// words: h goes out as device-scope (sc1) stores, every thread waits for its own stores to
// complete (s_waitcnt vmcnt(0)) before the workgroup barrier that precedes thread 0's arrival
// (so the compiler cannot move the arrival above them either), and after the poll and a
// second workgroup barrier h is read back with device-scope (sc1) loads, which miss any stale
// line of the reader's L2.  The counters and generation words are relaxed device-scope
// atomics.  Agent-scope release / acquire on them instead (an L2 write-back per arrival and
// an invalidate after the poll) measured 32.0 against 20.4 us per block.
// ---------------------------------------------------------------------------
constexpr int kBarSub = 16;
constexpr int kBarFail = 64 * (17 + kBarSub);
constexpr int kBarWords = kBarFail + 64;
constexpr uint32_t kBarSpinLimit = 1u << 22;  // polls; a normal wait takes a few hundred

__device__ __forceinline__ void bar_arrive(uint32_t *w, int bx, int G, uint32_t gen) {
  const int k = bx % kBarSub;
  const uint32_t nk = (uint32_t)((G - 1 - k) / kBarSub + 1);
  if (__hip_atomic_fetch_add(&w[64 * k], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u != nk) return;
  __hip_atomic_store(&w[64 * k], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint32_t nsub = (uint32_t)(G < kBarSub ? G : kBarSub);
  if (__hip_atomic_fetch_add(&w[64 * kBarSub], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u != nsub) return;
  __hip_atomic_store(&w[64 * kBarSub], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  for (int r = 0; r < kBarSub; r++)
    __hip_atomic_store(&w[64 * (17 + r)], gen + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Returns false (for the whole workgroup) if the generation did not change within `limit` polls.
struct BarWait {
  uint32_t *w;
  uint32_t gen;
  int bx;
  uint32_t limit;
  uint32_t *host_flag;  // pinned host word, nullable
  int *ok_lds;
  __device__ bool operator()() const {
    if (threadIdx.x == 0) {
      uint32_t *g = &w[64 * (17 + bx % kBarSub)];
      int ok = 0;
      for (uint32_t n = 0; n < limit; n++) {
        if (__hip_atomic_load(g, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != gen) {
          ok = 1;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
      if (!ok) {
        __hip_atomic_store(&w[kBarFail], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (host_flag) __hip_atomic_store(host_flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      }
      *ok_lds = ok;
    }
    __syncthreads();
    return *ok_lds != 0;
  }
};

template <class U>
__global__ __launch_bounds__(512) void moe_block_kernel(MoeXArgs ma1, MoeCombArgs ma2, uint32_t *bar, int per,
                                                        int nseg, uint32_t limit, uint32_t *host_flag) {
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ int r_e[64], r_se[64], r_sp[64], r_ok;
  __shared__ float r_w[64];
  const int id = (int)blockIdx.x, G = (int)gridDim.x;
  uint32_t gen = 0;
  if (threadIdx.x == 0) gen = __hip_atomic_load(&bar[64 * (17 + id % kBarSub)], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // Gate/up: workgroup (id % per, id / per); ids past per * nseg only route (no segment).
  const int by = id / per < nseg ? id / per : nseg;
  moe_x_body<U, 1, true, true, true>(ma1, smem, r_e, r_w, r_se, r_sp, id % per, by, per);
  __builtin_amdgcn_s_waitcnt(0);  // this wave's h stores are complete
  __syncthreads();
  if (threadIdx.x == 0) bar_arrive(bar, id, G, gen);
  moe_comb_body<U, true>(ma2, smem, id, 0, G, r_e, r_w, BarWait{bar, gen, id, limit, host_flag, &r_ok});
}

// ---------------------------------------------------------------------------
// The MoE decode block for one token in one launch, one workgroup per CU (moe_block1_kernel):
//  * every workgroup loads the router probabilities and x, routes the token (the top-k and
//    the expert sort of route_in_workgroup) and quantizes x into LDS;
//  * gate/up: workgroup b < topk * I / 32 owns slot b / (I / 32) and the 32-row block
//    b % (I / 32) of that slot's gated rows -- all of its row loads go out right after the
//    routing, R1 = 32 / RW1 rows per team -- writes act(g) * u as F32 h and quantizes the
//    block into the act layout (agent-coherent stores: read by other workgroups);
//  * down + MoECombine: workgroup b owns RPW output rows for all topk slots, as (row, slot)
//    team tasks; their weights are requested before the grid barrier (the routing names the
//    experts), h's act blocks are read agent-coherently after it into LDS, and each row's
//    slot values are added in slot order.
// With the previous layout (one 16-row group per workgroup, 384 of them on 256 CUs) the
// second workgroup of a CU got its rows only after the first's, and h went out as F32 to be
// quantized by every down workgroup after the barrier (per-workgroup clock stamps: gate/up
// done at 6.5-11.4 us, h quantized 2.6 us after the barrier).  The arithmetic -- unit dots,
// team sums, act(g) * u, h's quantization (act_quant8_fast on eight lanes per block), pair
// values times the routing weight, the slot-order adds -- is that of hq_moe_route_gated
// followed by hq_moe_gemm_q_combine, so every output is the same bits.  The grid barrier is
// moe_block_kernel's (bounded wait; a workgroup that gives up writes NaN and raises the flag).
// ---------------------------------------------------------------------------
struct MoeBlock1Args {
  Q4kxArgs ga;       // gate/up geometry: K = H, N = 2I (an expert's gate rows then up rows)
  Q4kxArgs da;       // down geometry: K = I, N = H
  MoeXArgs ra;       // routing (probs, E, topk, normalize, outputs)
  const uint8_t *wgu, *wdn;
  float *h;          // (topk, I) F32
  uint8_t *hact;     // act layout of (topk, I), agent-coherent
  float *y;          // (1, H)
  int64_t gu_bytes, dn_bytes;  // bytes per expert
  int I, H, topk, act, rpw;
};

template <class U, int R1, int NR>
__global__ __launch_bounds__(512) void moe_block1_kernel(MoeBlock1Args b, uint32_t *bar, uint32_t limit,
                                                         uint32_t *host_flag) {
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ int r_e[64], r_se[64], r_sp[64], r_ok;
  __shared__ float r_w[64];
  const int t = threadIdx.x, lane = t & 63;
  const int id = (int)blockIdx.x, G = (int)gridDim.x;
  const int topk = b.topk, I = b.I;
  uint32_t gen = 0;
  if (t == 0) gen = __hip_atomic_load(&bar[64 * (17 + id % kBarSub)], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  // x (one row of H) requested first; quantized into LDS after the gate/up loads go out.
  const Q4kxArgs &ga = b.ga;
  const int KB1 = ga.K >> 5, ntask1 = KB1 * 8;  // eight lanes per 32-block (act_quant8_fast)
  constexpr int XT = 2;
  float4 xv[XT];
#pragma unroll
  for (int i = 0; i < XT; i++) {
    const int task = i * 512 + t < ntask1 ? i * 512 + t : ntask1 - 1;
    xv[i] = reinterpret_cast<const float4 *>(ga.x)[task];
  }
  route_in_workgroup(b.ra, r_e, r_w, r_se, r_sp);
  if (id == 0) {
    for (int i = t; i < topk; i += 512) {
      b.ra.topk_ids[i] = r_e[i];
      b.ra.weights_out[i] = r_w[i];
      b.ra.sorted_pairs_out[i] = r_sp[i];
      b.ra.sorted_expts_out[i] = r_se[i];
    }
    if (b.ra.counts && b.ra.offsets) {
      // counts / offsets of the expert-sorted pairs: an exclusive scan over the sorted ids.
      for (int e = t; e <= b.ra.E; e += 512) {
        int lo = 0, cnt = 0;
        for (int i = 0; i < topk; i++) {
          lo += r_se[i] < e ? 1 : 0;
          cnt += r_se[i] == e ? 1 : 0;
        }
        b.ra.offsets[e] = lo;
        if (e < b.ra.E) b.ra.counts[e] = cnt;
      }
    }
  }

  // ---- gate / up: slot s, 32-row block j ----
  const int nblk = I / 32, gwg = topk * nblk;
  const int team1 = t / ga.TP, u1 = t - team1 * ga.TP;
  const bool act1 = u1 < ga.P;
  const typename U::Lane L1 = unit_lane<U>(act1 ? u1 : 0, ga.G);
  const bool gwork = id < gwg;
  const int gs = gwork ? id / nblk : 0, gj = gwork ? id % nblk : 0;
  int ge = r_e[gs];
  const bool gok = gwork && ge >= 0 && ge < b.ra.E;
  ge = gok ? ge : 0;
  const uint8_t *wgu = b.wgu + (int64_t)ge * b.gu_bytes;
  typename U::W wg[R1], wu[R1];
#pragma unroll
  for (int i = 0; i < R1; i++) {
    int row = gj * 32 + team1 + ga.RW * i;
    row = gok && team1 < ga.RW ? row : ga.N;  // no work: row N, zeros, no traffic
    U::load(wgu, ga.s0, ga.z0, ga, row, L1, wg[i]);
    U::load(wgu, ga.s0, ga.z0, ga, row < ga.N ? row + I : ga.N, L1, wu[i]);
  }
  // x into LDS (two-level act layout of one row)
  uint8_t *lq1 = smem, *lq2 = smem + ga.K;
  float2 *lde = reinterpret_cast<float2 *>(smem + 2 * ga.K);
  float *lsx = reinterpret_cast<float *>(smem + 2 * ga.K + 8 * KB1);
#pragma unroll
  for (int i = 0; i < XT; i++) {
    const int task = i * 512 + t;
    if (i * 512 >= ntask1) break;
    const int tc = task < ntask1 ? task : ntask1 - 1;
    const int blk = tc >> 3, sub = tc & 7;
    const float v[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
    const ActQ q = act_quant8_fast(v);
    if (task < ntask1) {
      reinterpret_cast<uint32_t *>(lq1 + blk * 32)[sub] = q.q1;
      reinterpret_cast<uint32_t *>(lq2 + blk * 32)[sub] = q.q2;
      if (sub == 0) {
        lde[blk] = make_float2(q.d, q.e);
        lsx[blk] = q.sum;
      }
    }
  }
  __syncthreads();
  float *hb = reinterpret_cast<float *>(smem + q4kx_act_lds(1, ga.K));  // [32]
  if (gwork) {
    typename U::X xr[1];
    U::load_x(lq1, lq2, reinterpret_cast<const uint8_t *>(lde), reinterpret_cast<const uint8_t *>(lsx), L1.ja, xr[0]);
#pragma unroll
    for (int i = 0; i < R1; i++) {
      float cg[1], cu[1];
      U::template dot<1>(wg[i], xr, L1, cg);
      U::template dot<1>(wu[i], xr, L1, cu);
      const float g16 = rsum16(act1 ? cg[0] : 0.f), u16 = rsum16(act1 ? cu[0] : 0.f);
      const float g0 = rl(g16, 0), g1 = rl(g16, 16), g2 = rl(g16, 32), g3 = rl(g16, 48);
      const float v0 = rl(u16, 0), v1 = rl(u16, 16), v2 = rl(u16, 32), v3 = rl(u16, 48);
      float tg, tu;
      if (ga.TP == 64) {
        tg = ((g0 + g1) + g2) + g3;
        tu = ((v0 + v1) + v2) + v3;
      } else if (ga.TP == 32) {
        tg = lane < 32 ? g0 + g1 : g2 + g3;
        tu = lane < 32 ? v0 + v1 : v2 + v3;
      } else {
        tg = lane < 16 ? g0 : (lane < 32 ? g1 : (lane < 48 ? g2 : g3));
        tu = lane < 16 ? v0 : (lane < 32 ? v1 : (lane < 48 ? v2 : v3));
      }
      const int r = team1 + ga.RW * i;
      if (u1 == 0 && team1 < ga.RW && r < 32) hb[r] = gok ? gate_act(tg, b.act) * tu : 0.f;
    }
  }
  __syncthreads();
  if (gwork && t < 8) {
    const float v[4] = {hb[t * 4], hb[t * 4 + 1], hb[t * 4 + 2], hb[t * 4 + 3]};
    const ActQ q = act_quant8_fast(v);
    const int64_t blk = (int64_t)gs * nblk + gj;
    const int64_t q2 = act_q2_off(topk, I), dof = act_d_off(topk, I), sof = act_s_off(topk, I);
    auto st = [&](int64_t off, uint32_t val) __attribute__((always_inline)) {
      __hip_atomic_store(reinterpret_cast<uint32_t *>(b.hact + off), val, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    st(blk * 32 + 4 * t, q.q1);
    st(q2 + blk * 32 + 4 * t, q.q2);
    if (t == 0) {
      st(dof + 8 * blk, __float_as_uint(q.d));
      st(dof + 8 * blk + 4, __float_as_uint(q.e));
      st(sof + 4 * blk, __float_as_uint(q.sum));
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // this wave's act stores are complete
  __syncthreads();
  if (t == 0) bar_arrive(bar, id, G, gen);
  // F32 h (an output of the call, read by no other workgroup) after the arrival.
  if (gwork && t < 32) b.h[(int64_t)gs * I + gj * 32 + t] = hb[t];

  // ---- down + combine: rows id * rpw .. + rpw, every slot ----
  const Q4kxArgs &da = b.da;
  const int team2 = t / da.TP, u2 = t - team2 * da.TP;
  const bool act2 = u2 < da.P;
  const typename U::Lane L2 = unit_lane<U>(act2 ? u2 : 0, da.G);
  const int slot = team2 % topk;
  int de_ = r_e[slot];
  const bool dok = de_ >= 0 && de_ < b.ra.E;
  de_ = dok ? de_ : 0;
  const uint8_t *wdn = b.wdn + (int64_t)de_ * b.dn_bytes;
  const int ntasks = b.rpw * topk;
  typename U::W wd[NR];
#pragma unroll
  for (int i = 0; i < NR; i++) {
    const int k = team2 + da.RW * i;  // task: (row k / topk, slot k % topk)
    int row = id * b.rpw + k / topk;
    row = k < ntasks && team2 < da.RW && row < da.N ? row : da.N;
    U::load(wdn, da.s0, da.z0, da, row, L2, wd[i]);
  }
  const bool h_ok = BarWait{bar, gen, id, limit, host_flag, &r_ok}();
  // h's act blocks of every slot into LDS (the LDS act layout of (topk, I)), agent-coherently.
  {
    const int KB2 = I >> 5;
    const int64_t gq2 = act_q2_off(topk, I), gd = act_d_off(topk, I), gsx = act_s_off(topk, I);
    const int nq = topk * I / 16;  // 16-byte pieces of q1 (and of q2)
    const __amdgpu_buffer_rsrc_t hr = span_rsrc(b.hact, (uint32_t)act_bytes(topk, I));
    uint8_t *d1 = smem, *d2 = smem + (int64_t)topk * I;
    uint8_t *dd = smem + 2 * (int64_t)topk * I, *ds = dd + 8 * (int64_t)topk * KB2;
    for (int i = t; i < nq; i += 512) {
      *reinterpret_cast<u32x4_t *>(d1 + 16 * i) = __builtin_amdgcn_raw_buffer_load_b128(hr, (uint32_t)(16 * i), 0, 16);
      *reinterpret_cast<u32x4_t *>(d2 + 16 * i) =
          __builtin_amdgcn_raw_buffer_load_b128(hr, (uint32_t)(gq2 + 16 * i), 0, 16);
    }
    for (int i = t; i < topk * KB2; i += 512) {
      reinterpret_cast<uint32_t *>(dd)[2 * i] = __builtin_amdgcn_raw_buffer_load_b32(hr, (uint32_t)(gd + 8 * i), 0, 16);
      reinterpret_cast<uint32_t *>(dd)[2 * i + 1] =
          __builtin_amdgcn_raw_buffer_load_b32(hr, (uint32_t)(gd + 8 * i + 4), 0, 16);
      reinterpret_cast<uint32_t *>(ds)[i] = __builtin_amdgcn_raw_buffer_load_b32(hr, (uint32_t)(gsx + 4 * i), 0, 16);
    }
  }
  __syncthreads();
  typename U::X xr2[1];
  {
    const int KB2 = I >> 5;
    U::load_x(smem, smem + (int64_t)topk * I, smem + 2 * (int64_t)topk * I,
              smem + 2 * (int64_t)topk * I + 8 * (int64_t)topk * KB2, (int64_t)slot * KB2 + L2.ja, xr2[0]);
  }
  float *vb = reinterpret_cast<float *>(smem + q4kx_act_lds(topk, I));  // [rpw][topk]
  const float wp = r_w[slot];
#pragma unroll
  for (int i = 0; i < NR; i++) {
    float c[1];
    U::template dot<1>(wd[i], xr2, L2, c);
    const float r16 = rsum16(act2 ? c[0] : 0.f);
    const float r0 = rl(r16, 0), r1 = rl(r16, 16), r2 = rl(r16, 32), r3 = rl(r16, 48);
    float tot;
    if (da.TP == 64)
      tot = ((r0 + r1) + r2) + r3;
    else if (da.TP == 32)
      tot = lane < 32 ? r0 + r1 : r2 + r3;
    else
      tot = lane < 16 ? r0 : (lane < 32 ? r1 : (lane < 48 ? r2 : r3));
    const int k = team2 + da.RW * i;
    if (u2 == 0 && team2 < da.RW && k < ntasks) vb[k] = dok ? tot * wp : 0.f;
  }
  __syncthreads();
  if (t < b.rpw) {
    const int row = id * b.rpw + t;
    if (row < da.N) {
      float acc = vb[t * topk];
      for (int s2 = 1; s2 < topk; s2++) acc = __fadd_rn(acc, vb[t * topk + s2]);
      b.y[row] = h_ok ? acc : __builtin_nanf("");
    }
  }
}

// ---------------------------------------------------------------------------
// MoEInt4 (ops/int4.go:149-300): the routed gated-MLP expert block with 4-bit (GPTQ / AWQ,
// canonical quant.Int4) experts.  Each expert is a separate quant.Int4, so the kernels read
// per-expert (codes, scales, zeros) pointers from device tables, and only the routed experts'
// rows are read -- nothing is expanded.  Two launches:
//  * moe_int4_gated_kernel: grid.y = routed pair p = t * topk + j.  h[p, n] =
//    act(x[t] . Wgu[e][n]) * (x[t] . Wgu[e][I + n]) for n < I (e = ids[p]), x[t] quantized in
//    LDS, teams streaming gate and up rows together as the gated GEMV does.
//  * moe_int4_down_kernel: grid.y = token, teams = (row, slot) pairs as in
//    moe_down_combine_kernel: y[t, n] = 0 + w(t,0) dot_0 + w(t,1) dot_1 + ..., the slots added
//    in slot order onto zero, as Light's moeInt4Rows does, stored at x's dtype.
// ---------------------------------------------------------------------------
struct MoeInt4Args {
  Q4kxArgs g;                 // K, P, TP, RW, G of the launch; x / out / N set per kernel
  const void *const *tab;     // [6][E]: gate-up codes, scales, zeros; down codes, scales, zeros
  const int64_t *ids;         // (T * topk) expert per pair
  const float *w;             // (T * topk) routing weights
  float *h;                   // (T * topk, I) F32
  int E, topk, T, I, H, act, x_dtype;
};

// Quantize `rows` rows of K elements (x dtype XDT, row r at src + r * K) into the LDS act layout
// (eight lanes per 32-block, act_quant8_fast), rows after each other.
template <int XDT>
__device__ __forceinline__ void quant_rows_lds(const void *src, int rows, int K, uint8_t *smem) {
  const int KB = K >> 5, t = threadIdx.x;
  uint8_t *lq1 = smem, *lq2 = smem + (int64_t)rows * K;
  float2 *lde = reinterpret_cast<float2 *>(smem + 2 * (int64_t)rows * K);
  float *lsx = reinterpret_cast<float *>(smem + 2 * (int64_t)rows * K + 8 * (int64_t)rows * KB);
  const int ntask = rows * KB * 8;
  for (int base = 0; base < ntask; base += (int)blockDim.x) {
    const int task = base + t < ntask ? base + t : ntask - 1;
    const int blk = task >> 3, sub = task & 7;
    const float4 xv = load_x4<XDT>(src, (int64_t)blk * 32 + sub * 4);
    const float v[4] = {xv.x, xv.y, xv.z, xv.w};
    const ActQ q = act_quant8_fast(v);
    if (base + t < ntask) {
      reinterpret_cast<uint32_t *>(lq1 + blk * 32)[sub] = q.q1;
      reinterpret_cast<uint32_t *>(lq2 + blk * 32)[sub] = q.q2;
      if (sub == 0) {
        lde[blk] = make_float2(q.d, q.e);
        lsx[blk] = q.sum;
      }
    }
  }
}

template <class U, int XDT>
__global__ __launch_bounds__(512) void moe_int4_gated_kernel(MoeInt4Args ma) {
  extern __shared__ __align__(16) uint8_t smem[];
  Q4kxArgs a = ma.g;
  const int t = threadIdx.x, lane = t & 63;
  const int p = blockIdx.y, tok = p / ma.topk;
  int64_t e = ma.ids[p];
  const bool ok = e >= 0 && e < ma.E;
  e = ok ? e : 0;
  const uint8_t *wc = static_cast<const uint8_t *>(ma.tab[0 * ma.E + e]);
  const float *ws = static_cast<const float *>(ma.tab[1 * ma.E + e]);
  const float *wz = static_cast<const float *>(ma.tab[2 * ma.E + e]);
  a.N = 2 * ma.I;  // the expert's gate-up rows (the resource spans both halves)
  const int RW = a.RW, KB = a.K >> 5;
  const int team = t / a.TP, u = t - team * a.TP;
  const bool active = u < a.P;
  const typename U::Lane L = unit_lane<U>(active ? u : 0, a.G);
  const int ngroups = (ma.I + RW - 1) / RW, G = gridDim.x;
  const int niter = (ngroups - (int)blockIdx.x + G - 1) / G;
  typename U::W wr[2];
  {
    int row = (int)blockIdx.x * RW + team;
    row = row < ma.I ? row : a.N;
    U::load(wc, ws, wz, a, row, L, wr[0]);
    U::load(wc, ws, wz, a, row < ma.I ? row + ma.I : a.N, L, wr[1]);
  }
  quant_rows_lds<XDT>(static_cast<const uint8_t *>(a.x) + (int64_t)tok * a.K * (XDT == F32 ? 4 : 2), 1, a.K,
                      smem);
  __syncthreads();
  typename U::X xr[1];
  U::load_x(smem, smem + a.K, smem + 2 * a.K, smem + 2 * a.K + 8 * KB, L.ja, xr[0]);
  for (int it = 0; it < niter; it++) {
    const int grp = (int)blockIdx.x + it * G;
    float c[2][1];
    U::template dot<1>(wr[0], xr, L, c[0]);
    U::template dot<1>(wr[1], xr, L, c[1]);
    {
      int row = (grp + G) * RW + team;
      const bool in = row < ma.I;
      U::load(wc, ws, wz, a, in ? row : a.N, L, wr[0]);
      U::load(wc, ws, wz, a, in ? row + ma.I : a.N, L, wr[1]);
    }
    float tot[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const float r16 = rsum16(active ? c[j][0] : 0.f);
      const float r0 = rl(r16, 0), r1 = rl(r16, 16), r2 = rl(r16, 32), r3 = rl(r16, 48);
      if (a.TP == 64)
        tot[j] = ((r0 + r1) + r2) + r3;
      else if (a.TP == 32)
        tot[j] = lane < 32 ? r0 + r1 : r2 + r3;
      else
        tot[j] = lane < 16 ? r0 : (lane < 32 ? r1 : (lane < 48 ? r2 : r3));
    }
    const int row = grp * RW + team;
    if (u == 0 && row < ma.I) ma.h[(int64_t)p * ma.I + row] = ok ? gate_act(tot[0], ma.act) * tot[1] : 0.f;
  }
}

template <class U, int ODT>
__global__ __launch_bounds__(512) void moe_int4_down_kernel(MoeInt4Args ma) {
  extern __shared__ __align__(16) uint8_t smem[];
  Q4kxArgs a = ma.g;  // K = I, N = H
  const int t = threadIdx.x, lane = t & 63;
  const int tok = blockIdx.y, topk = ma.topk;
  const int RW = a.RW, KB = a.K >> 5, RPW = RW / topk;
  float *lval = reinterpret_cast<float *>(smem + q4kx_act_lds(topk, a.K));
  const int team = t / a.TP, u = t - team * a.TP;
  const int slot = team % topk, rloc = team / topk;
  const bool active = u < a.P;
  const typename U::Lane L = unit_lane<U>(active ? u : 0, a.G);
  const int64_t p = (int64_t)tok * topk + slot;
  int64_t e = ma.ids[p];
  const bool ok = e >= 0 && e < ma.E;
  e = ok ? e : 0;
  const uint8_t *wc = static_cast<const uint8_t *>(ma.tab[3 * ma.E + e]);
  const float *ws = static_cast<const float *>(ma.tab[4 * ma.E + e]);
  const float *wz = static_cast<const float *>(ma.tab[5 * ma.E + e]);
  const int ngroups = (a.N + RPW - 1) / RPW, G = gridDim.x;
  const int niter = (ngroups - (int)blockIdx.x + G - 1) / G;
  typename U::W wr;
  {
    int row = (int)blockIdx.x * RPW + rloc;
    row = row < a.N ? row : a.N;
    U::load(wc, ws, wz, a, row, L, wr);
  }
  quant_rows_lds<F32>(ma.h + (int64_t)tok * topk * a.K, topk, a.K, smem);
  __syncthreads();
  const float wp = ma.w[p];
  typename U::X xr[1];
  U::load_x(smem, smem + (int64_t)topk * a.K, smem + 2 * (int64_t)topk * a.K,
            smem + 2 * (int64_t)topk * a.K + 8 * (int64_t)topk * KB, slot * KB + L.ja, xr[0]);
  for (int it = 0; it < niter; it++) {
    const int grp = (int)blockIdx.x + it * G;
    float c[1];
    U::template dot<1>(wr, xr, L, c);
    {
      int row = (grp + G) * RPW + rloc;
      row = row < a.N ? row : a.N;
      U::load(wc, ws, wz, a, row, L, wr);
    }
    const float r16 = rsum16(active ? c[0] : 0.f);
    const float r0 = rl(r16, 0), r1 = rl(r16, 16), r2 = rl(r16, 32), r3 = rl(r16, 48);
    float tot;
    if (a.TP == 64)
      tot = ((r0 + r1) + r2) + r3;
    else if (a.TP == 32)
      tot = lane < 32 ? r0 + r1 : r2 + r3;
    else
      tot = lane < 16 ? r0 : (lane < 32 ? r1 : (lane < 48 ? r2 : r3));
    float *vb = lval + (it & 1) * (RPW * topk);
    if (u == 0) vb[rloc * topk + slot] = ok ? __fmul_rn(wp, tot) : 0.f;
    __syncthreads();
    const int row = grp * RPW + t;
    if (t < RPW && row < a.N) {
      float acc = 0.f;
      for (int s2 = 0; s2 < topk; s2++) acc = __fadd_rn(acc, vb[t * topk + s2]);
      store_out<ODT>(a.out, (int64_t)tok * a.N + row, acc);
    }
  }
}

// Generic MoEInt4 (any H, I multiple of 8 and of G): one wave per output, F32 x, the weight
// decoded on the fly exactly as quant.Int4.Dequant does (s * (q - z), quant/int4.go:239-261),
// F32 products summed lane-strided then by a wave reduction.  Used where the GEMV's
// 64-element units do not tile the shapes.
__device__ __forceinline__ float int4_w(const uint32_t *codes, const float *sc, const float *zr, int64_t n,
                                        int64_t k, int64_t K, int G) {
  const uint32_t q = (codes[n * (K / 8) + k / 8] >> (4 * (k & 7))) & 15u;
  const int64_t gi = n * (K / G) + k / G;
  return __fmul_rn(sc[gi], __fsub_rn((float)q, zr[gi]));
}

template <int XDT>
__global__ __launch_bounds__(256) void moe_int4_generic_gated_kernel(MoeInt4Args ma) {
  const int lane = threadIdx.x & 63;
  const int64_t gw = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // output (pair, row)
  const int64_t M = (int64_t)ma.T * ma.topk;
  if (gw >= M * ma.I) return;
  const int64_t p = gw / ma.I, n = gw % ma.I, tok = p / ma.topk;
  int64_t e = ma.ids[p];
  const bool ok = e >= 0 && e < ma.E;
  e = ok ? e : 0;
  const auto *wc = static_cast<const uint32_t *>(ma.tab[0 * ma.E + e]);
  const auto *ws = static_cast<const float *>(ma.tab[1 * ma.E + e]);
  const auto *wz = static_cast<const float *>(ma.tab[2 * ma.E + e]);
  float g = 0.f, u = 0.f;
  for (int64_t k = lane; k < ma.H; k += 64) {
    float xv;
    if constexpr (XDT == F32)
      xv = static_cast<const float *>(ma.g.x)[tok * ma.H + k];
    else if constexpr (XDT == BF16)
      xv = bf2f(static_cast<const uint16_t *>(ma.g.x)[tok * ma.H + k]);
    else
      xv = h2f(static_cast<const uint16_t *>(ma.g.x)[tok * ma.H + k]);
    g = __fmaf_rn(xv, int4_w(wc, ws, wz, n, k, ma.H, ma.g.G), g);
    u = __fmaf_rn(xv, int4_w(wc, ws, wz, n + ma.I, k, ma.H, ma.g.G), u);
  }
  g = wave_sum(g);
  u = wave_sum(u);
  if (lane == 0) ma.h[p * ma.I + n] = ok ? gate_act(g, ma.act) * u : 0.f;
}

template <int ODT>
__global__ __launch_bounds__(256) void moe_int4_generic_down_kernel(MoeInt4Args ma) {
  const int lane = threadIdx.x & 63;
  const int64_t gw = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // output (token, row)
  if (gw >= (int64_t)ma.T * ma.H) return;
  const int64_t tok = gw / ma.H, n = gw % ma.H;
  float acc = 0.f;
  for (int j = 0; j < ma.topk; j++) {
    const int64_t p = tok * ma.topk + j;
    int64_t e = ma.ids[p];
    const bool ok = e >= 0 && e < ma.E;
    e = ok ? e : 0;
    const auto *wc = static_cast<const uint32_t *>(ma.tab[3 * ma.E + e]);
    const auto *ws = static_cast<const float *>(ma.tab[4 * ma.E + e]);
    const auto *wz = static_cast<const float *>(ma.tab[5 * ma.E + e]);
    float y = 0.f;
    for (int64_t k = lane; k < ma.I; k += 64) y = __fmaf_rn(ma.h[p * ma.I + k], int4_w(wc, ws, wz, n, k, ma.I, ma.g.G), y);
    y = wave_sum(y);
    acc = __fadd_rn(acc, ok ? __fmul_rn(ma.w[p], y) : 0.f);
  }
  if (lane == 0) store_out<ODT>(ma.g.out, tok * ma.H + n, acc);
}

// ---------------------------------------------------------------------------
// Launch
// ---------------------------------------------------------------------------

// Team geometry: P = K/64 lanes (units) per row; TP = 16, 32 or 64 when P fits a wave,
// else P rounded up to whole 16-lane rows (up to 512; e.g. 224 at K = 14336, so no lane of
// the team idles); RW = teams per workgroup of at most 512 lanes.  `kblock` is the
// K granularity of the format (256 for Q4_K, 64 for int4).
static bool q4kx_geom(int64_t K, int kblock, int *P, int *TP, int *RW) {
  if (K % kblock || K > 32768) return false;
  *P = (int)(K / 64);
  if (*P <= 16)
    *TP = 16;
  else if (*P <= 32)
    *TP = 32;
  else if (*P <= 64)
    *TP = 64;
  else
    *TP = (*P + 15) & ~15;  // several waves: whole 16-lane rows (the LDS reduction's unit)
  *RW = *TP >= 512 ? 1 : 512 / *TP;
  return true;
}

// Row bytes of a K-wide row of the Q4_K, Q5_K (GGUF) and Q6_K_R (padded planar) formats.
static int64_t q4kx_row_bytes(int dt, int64_t K) {
  return dt == Q6_K_R ? q6kr_row_bytes(K) : K / 256 * block_info(dt).bytes;
}

static int mm_of(int64_t M) { return M >= 3 ? 4 : (int)M; }

// Quantize x inside the GEMV's workgroups (saves a launch) only for rows up to 8192: each
// workgroup quantizes all of x, which costs ~1 us at K = 4096 but ~4.5 us at K = 14336,
// more than the separate quantize launch.
bool q4kx_xin(int64_t K) { return K <= 8192; }

static size_t q4kx_lds(int MM, int64_t K, int TP, int RW, int nw, bool xin, bool aout) {
  size_t b = xin ? (size_t)q4kx_act_lds(MM, K) : 0;
  if (TP > 64) b += 2 * 4 * (size_t)(RW * (TP >> 4) * nw * MM);
  if (aout) b += 2 * 4 * 32 * (size_t)MM;
  return b;
}

bool q4kx_ok(int64_t M, int64_t N, int64_t K, const void *w0, const void *w1, const void *x, int dt) {
  int P, TP, RW;
  if ((dt != Q4_K && dt != Q5_K && dt != Q6_K_R) || M < 1 || M > kGemvMaxRows || !q4kx_geom(K, 256, &P, &TP, &RW))
    return false;
  if (N > INT32_MAX / 2 || (N + 1) * q4kx_row_bytes(dt, K) > UINT32_MAX) return false;
  if (((uintptr_t)w0 & 15) || (w1 && ((uintptr_t)w1 & 15)) || ((uintptr_t)x & 15)) return false;
  return q4kx_lds(mm_of(M), K, TP, RW, w1 != nullptr ? 2 : 1, true, true) <= 160 * 1024;
}

template <class U, int MM, bool GATED, bool XIN, bool AOUT, int XDT, int ODT, int ROWS = 1>
static int run_q4kx(const Q4kxArgs &a, hipStream_t s) {
  auto *kern = &gemv_q4kx_kernel<U, MM, GATED, XIN, AOUT, XDT, ODT, ROWS>;
  const size_t lds = q4kx_lds(MM, a.K, a.TP, a.RW, GATED ? 2 : ROWS, XIN, AOUT);
  if (lds > 64 * 1024) {
    static std::atomic<bool> attr_done{false};  // (idempotent: racing callers both set it)
    if (!attr_done.load(std::memory_order_acquire)) {
      if (hipFuncSetAttribute(reinterpret_cast<const void *>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                              160 * 1024) != hipSuccess)
        return fail(HQ_EUNSUPPORTED, "gemv_q4kx", "LDS %zu bytes not available", lds);
      attr_done.store(true, std::memory_order_release);
    }
  }
  const int span = ROWS * a.RW;
  const int ngroups = (a.N + span - 1) / span;
  const int units = AOUT ? (ngroups + 32 / a.RW - 1) / (32 / a.RW) : ngroups;
  // Two persistent workgroups per CU, one row group in flight per wave: measured faster
  // than deeper per-wave prefetch (more loads per wave) or more workgroups.
  const int cap = device_cus() * 2;
  dim3 grid((unsigned)(units < cap ? units : cap), (unsigned)cdiv(a.M, MM));
  kern<<<grid, a.TP * a.RW, lds, s>>>(a);
  return check_launch(GATED ? "gemv_q4k_gated" : "gemv_q4kx");
}

template <class U, bool GATED, bool XIN, bool AOUT, int XDT = F32, int ODT = F32, int ROWS = 1>
static int dispatch_q4kx(const Q4kxArgs &a, hipStream_t s) {
  const int MMc = mm_of(a.M);
  if (MMc == 1) return run_q4kx<U, 1, GATED, XIN, AOUT, XDT, ODT, ROWS>(a, s);
  if (MMc == 2) return run_q4kx<U, 2, GATED, XIN, AOUT, XDT, ODT, ROWS>(a, s);
  return run_q4kx<U, 4, GATED, XIN, AOUT, XDT, ODT, ROWS>(a, s);
}

static int q4kx_setup(Q4kxArgs &a, int64_t M, int64_t N, int64_t K, int kblock, int64_t row_bytes,
                      const char *call) {
  if (!q4kx_geom(K, kblock, &a.P, &a.TP, &a.RW) || N > INT32_MAX / 2 || M > 65535 || (N + 1) * row_bytes > UINT32_MAX)
    return fail(HQ_EUNSUPPORTED, call, "K=%lld N=%lld", (long long)K, (long long)N);
  a.x = nullptr;
  a.ain = nullptr;
  a.w0 = a.w1 = nullptr;
  a.s0 = a.z0 = a.s1 = a.z1 = nullptr;
  a.out = nullptr;
  a.aout = nullptr;
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.G = 0;
  a.row_bytes = row_bytes;
  a.in_q2 = act_q2_off(M, K);
  a.in_d = act_d_off(M, K);
  a.in_s = act_s_off(M, K);
  a.out_q2 = act_q2_off(M, N);
  a.out_d = act_d_off(M, N);
  a.out_s = act_s_off(M, N);
  a.act = 0;
  return 0;
}

// ---------------------------------------------------------------------------
// One-token GEMV (plain, or gated with F32 output) on x quantized in the kernel, K in
// (2048, 4096] (one wave per row): one workgroup per CU over a contiguous range of
// N / C rows, x requested first and quantized into LDS while the first rows stream, D rows
// (pairs, gated) in flight per wave, straight-line code.  The arithmetic is
// gemv_q4kx_kernel<U, 1, GATED, XIN = true, AOUT = false, XDT, ODT>'s, bit for bit.
// ---------------------------------------------------------------------------
template <class U, bool GATED, int R, int D, int XDT, int ODT>
__global__ __launch_bounds__(512) void gemv_cu_kernel(Q4kxArgs a) {
  static_assert(D >= 1 && D <= R, "ring depth");
  constexpr int NW = GATED ? 2 : 1;
  extern __shared__ __align__(16) uint8_t smem[];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int KB = a.K >> 5;
  const bool active = lane < a.P;
  const typename U::Lane L = unit_lane<U>(active ? lane : 0, a.G);
  const int C = (int)gridDim.x, b = (int)blockIdx.x;
  const int rs = (int)((int64_t)b * a.N / C), re = (int)((int64_t)(b + 1) * a.N / C);
  auto row_of = [&](int i) __attribute__((always_inline)) {
    const int r = rs + 8 * i + wave;
    return r < re ? r : a.N;  // past the range: row N, zeros, no traffic
  };
  typename U::W wr[D][NW];
  auto load_row = [&](int i) __attribute__((always_inline)) {
    const int row = row_of(i);
    U::load(a.w0, a.s0, a.z0, a, row, L, wr[i % D][0]);
    if constexpr (GATED) U::load(a.w1, a.s1, a.z1, a, row, L, wr[i % D][NW - 1]);
  };
  // x: one 16-element task per thread (K <= 4096: at most 256 tasks).
  const int ntask = KB * 2;
  const int task = t < ntask ? t : ntask - 1;
  constexpr int XR = XDT == F32 ? 4 : 2;
  u32x4_t raw[XR];
  {
    const uint8_t *xp = static_cast<const uint8_t *>(a.x) + (int64_t)task * 16 * (XDT == F32 ? 4 : 2);
#pragma unroll
    for (int r = 0; r < XR; r++) raw[r] = *reinterpret_cast<const u32x4_t *>(xp + 16 * r);
  }
#pragma unroll
  for (int i = 0; i < D; i++) load_row(i);
  uint8_t *lq1 = smem, *lq2 = smem + a.K;
  float2 *lde = reinterpret_cast<float2 *>(smem + 2 * a.K);
  float *lsx = reinterpret_cast<float *>(smem + 2 * a.K + 8 * KB);
  {
    float v[16];
#pragma unroll
    for (int j = 0; j < 16; j++) {
      const uint32_t w32 = raw[XDT == F32 ? j / 4 : j / 8][XDT == F32 ? j % 4 : (j % 8) / 2];
      if constexpr (XDT == F32)
        v[j] = __uint_as_float(w32);
      else
        v[j] = XDT == BF16 ? bf2f((j & 1) ? w32 >> 16 : w32 & 0xffffu) : h2f((j & 1) ? w32 >> 16 : w32 & 0xffffu);
    }
    const ActQ16 q = act_quant16_fast(v);
    if (t < ntask) {
      const int blk = task >> 1, half = task & 1;
      *reinterpret_cast<u32x4_t *>(lq1 + blk * 32 + half * 16) = u32x4_t{q.q1[0], q.q1[1], q.q1[2], q.q1[3]};
      if constexpr (U::kX2)
        *reinterpret_cast<u32x4_t *>(lq2 + blk * 32 + half * 16) = u32x4_t{q.q2[0], q.q2[1], q.q2[2], q.q2[3]};
      if (half == 0) {
        lde[blk] = make_float2(q.d, q.e);
        lsx[blk] = q.sum;
      }
    }
  }
  __syncthreads();
  typename U::X xr[1];
  U::load_x(lq1, lq2, reinterpret_cast<const uint8_t *>(lde), reinterpret_cast<const uint8_t *>(lsx), L.ja, xr[0]);
#pragma unroll
  for (int i = 0; i < R; i++) {
    float tot[NW];
#pragma unroll
    for (int j = 0; j < NW; j++) {
      float c[1];
      U::template dot<1>(wr[i % D][j], xr, L, c);
      const float r16 = rsum16(active ? c[0] : 0.f);
      tot[j] = ((rl(r16, 0) + rl(r16, 16)) + rl(r16, 32)) + rl(r16, 48);
    }
    if (i + D < R) load_row(i + D);
    const int row = row_of(i);
    if (lane == 0 && row < a.N) {
      const float y = GATED ? gate_act(tot[0], a.act) * tot[NW - 1] : tot[0];
      store_out<ODT>(a.out, row, y);
    }
  }
}

// One token, one wave per row (K in (2048, 4096]), 8 to 16 rows per CU.  (At 56 rows per CU,
// 14336 x 4096, the persistent kernel was measured faster: 8.6 against 8.9-9.9 us with one to
// three rows in flight per wave; at 16 rows per CU, Q6_K_R 4096 x 4096, this one: 6.5 -> 5.8 us.)
static bool gemv_cu_ok(const Q4kxArgs &a) {
  return a.M == 1 && a.TP == 64 && a.RW == 8 && a.P > 32 && a.N >= 8 * device_cus() && a.N <= 16 * device_cus();
}

template <class U, bool GATED, int XDT, int ODT>
static int run_gemv_cu(const Q4kxArgs &a, hipStream_t s) {
  const int C = device_cus();
  const int R = (int)cdiv(cdiv(a.N, C), 8);
  const size_t lds = (size_t)q4kx_act_lds(1, a.K);
  const dim3 grid((unsigned)C);
  if (R <= 1)
    gemv_cu_kernel<U, GATED, 1, 1, XDT, ODT><<<grid, 512, lds, s>>>(a);
  else
    gemv_cu_kernel<U, GATED, 2, 2, XDT, ODT><<<grid, 512, lds, s>>>(a);
  return check_launch(GATED ? "gemv_cu_gated" : "gemv_cu");
}

int launch_gemv_q4kx(const float *x, const void *w0, const void *w1, float *out, int64_t M, int64_t N, int64_t K,
                     int act, int dt, hipStream_t s) {
  Q4kxArgs a;
  if (int rc = q4kx_setup(a, M, N, K, 256, q4kx_row_bytes(dt, K), "gemv_q4kx")) return rc;
  a.x = x;
  a.w0 = static_cast<const uint8_t *>(w0);
  a.w1 = static_cast<const uint8_t *>(w1);
  a.out = out;
  a.act = act;
  return with_qk_unit(dt, K, [&](auto unit) {
    using U = decltype(unit);
    if (gemv_cu_ok(a)) return w1 ? run_gemv_cu<U, true, F32, F32>(a, s) : run_gemv_cu<U, false, F32, F32>(a, s);
    return w1 ? dispatch_q4kx<U, true, true, false>(a, s) : dispatch_q4kx<U, false, true, false>(a, s);
  });
}

// ---------------------------------------------------------------------------
// Long-row GEMV on prepared activations at one token (the MLP's down projection, K = 14336):
// one workgroup per CU, its rows requested early.
//
// A CU serves the memory requests of its workgroups roughly in issue order.  With two
// persistent workgroups per CU (gemv_q4kx_kernel) the second one's first rows arrive only
// after the first one's (per-workgroup clock stamps: first data at 2.5 us for workgroups
// 0-255, 5.5 us for 256-511), and each later row group is requested only after a dot, so the
// launch ends several latencies after its first data.  Here one workgroup per CU holds RW
// teams of R rows each: every lane requests its unit's activations first (they gate every
// dot), then D rows, and each dot refills its slot with the row D ahead (straight-line code:
// the compiler's wait before each dot covers that row's loads only).  The teams' 16-lane sums
// meet in LDS once, at the end.  Arithmetic and summation order are gemv_q4kx_kernel's (unit
// dots, 16-lane sums, a team's rows added in order from zero), so the results are the same
// bits.  4096 x 14336: 10.2 -> 8.8 us.
// ---------------------------------------------------------------------------
template <class U, int R, int D, int ODT = F32>
__global__ __launch_bounds__(512) void gemv_rows_kernel(Q4kxArgs a) {
  static_assert(D >= 1 && D <= R, "ring depth");
  extern __shared__ __align__(16) uint8_t smem[];
  const int t = threadIdx.x, lane = t & 63;
  const int team = t / a.TP, u = t - team * a.TP;
  const bool active = u < a.P;
  const typename U::Lane L = unit_lane<U>(active ? u : 0, a.G);
  const int hpt = a.TP >> 4;
  const int row0 = (blockIdx.x * a.RW + team) * R;
  typename U::X xr[1];
  U::load_x(a.ain, a.ain + a.in_q2, a.ain + a.in_d, a.ain + a.in_s, (int64_t)L.ja, xr[0]);
  typename U::W wr[D];
  auto load_row = [&](int r) __attribute__((always_inline)) {
    int row = row0 + r;
    row = row < a.N ? row : a.N;  // past the end: zeros, no traffic
    U::load(a.w0, a.s0, a.z0, a, row, L, wr[r % D]);
  };
#pragma unroll
  for (int r = 0; r < D; r++) load_row(r);
  float *pp = reinterpret_cast<float *>(smem);  // [RW][R][hpt] 16-lane sums
#pragma unroll
  for (int r = 0; r < R; r++) {
    float c[1];
    U::template dot<1>(wr[r % D], xr, L, c);
    if (r + D < R) load_row(r + D);
    const float s16 = rsum16(active ? c[0] : 0.f);
    if ((lane & 15) == 0) pp[(team * R + r) * hpt + (u >> 4)] = s16;
  }
  __syncthreads();
  if (t < a.RW * R) {
    const int tm = t / R, r = t - tm * R;
    float acc = 0.f;
    for (int k = 0; k < hpt; k++) acc += pp[(tm * R + r) * hpt + k];
    const int row = (blockIdx.x * a.RW + tm) * R + r;
    if (row < a.N) store_out<ODT>(a.out, row, acc);
  }
}

// One token, teams wider than a wave (K > 4096) that fill a workgroup.
static bool gemv_rows_ok(const Q4kxArgs &a) { return a.M == 1 && a.TP > 64 && a.TP * a.RW <= 512; }

// R rows per team: as many as put one workgroup on every CU, at most 8 (4 in flight).
template <class U, int ODT = F32>
static int run_gemv_rows(const Q4kxArgs &a, hipStream_t s) {
  const int64_t per = cdiv(a.N, (int64_t)a.RW * device_cus());
  const int R = per >= 8 ? 8 : per >= 4 ? 4 : per >= 2 ? 2 : 1;
  const size_t lds = (size_t)a.RW * R * (a.TP >> 4) * 4;
  const dim3 grid((unsigned)cdiv(a.N, (int64_t)a.RW * R));
  const int nt = a.TP * a.RW;
  switch (R) {
    case 8: gemv_rows_kernel<U, 8, 4, ODT><<<grid, nt, lds, s>>>(a); break;
    case 4: gemv_rows_kernel<U, 4, 4, ODT><<<grid, nt, lds, s>>>(a); break;
    case 2: gemv_rows_kernel<U, 2, 2, ODT><<<grid, nt, lds, s>>>(a); break;
    default: gemv_rows_kernel<U, 1, 1, ODT><<<grid, nt, lds, s>>>(a); break;
  }
  return check_launch("gemv_rows");
}

int launch_gemv_q4kx_act(const void *act_in, const void *w, float *out, int64_t M, int64_t N, int64_t K, int dt,
                         hipStream_t s) {
  Q4kxArgs a;
  if (int rc = q4kx_setup(a, M, N, K, 256, q4kx_row_bytes(dt, K), "gemv_q4kx")) return rc;
  a.ain = static_cast<const uint8_t *>(act_in);
  a.w0 = static_cast<const uint8_t *>(w);
  a.out = out;
  // Long rows (teams of several waves): two rows per team and iteration (measured 10.8 ->
  // 10.6 us at 4096 x 14336; four rows, 130 registers, measured 12.2 us).
  return with_qk_unit(dt, K, [&](auto unit) {
    using U = decltype(unit);
    if (gemv_rows_ok(a)) return run_gemv_rows<U>(a, s);
    if (a.TP > 64) return dispatch_q4kx<U, false, false, false, F32, F32, 2>(a, s);
    return dispatch_q4kx<U, false, false, false>(a, s);
  });
}

// Rows longer than one team (Q4_K / Q5_K, 32768 < K <= 65536, e.g. Llama-3-405B's down
// projection, K = 53248): each x row's dot runs as two launches of the act GEMV above, one
// per K half, on the full rows' stride -- the weight base moves by the first half's blocks
// and the activation bases by its elements, so both halves read the same buffers in place --
// then one launch adds the second half's outputs (in tmp) to the first's.
__global__ void add_rows_kernel(float *out, const float *tmp, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] += tmp[i];
}

bool q4kx_halves_ok(int64_t M, int64_t N, int64_t K, int dt, const void *w, const void *act) {
  if ((dt != Q4_K && dt != Q5_K) || M < 1 || M > kGemvMaxRows || K <= 32768 || K > 65536 || K % 256) return false;
  const int64_t kh = (K / 2 + 255) / 256 * 256;
  return q4kx_ok(1, N, kh, w, nullptr, act, dt) && (N + 1) * q4kx_row_bytes(dt, K) <= UINT32_MAX;
}

int launch_gemv_q4kx_act_halves(const void *act_in, const void *w, float *out, float *tmp, int64_t M, int64_t N,
                                int64_t K, int dt, hipStream_t s) {
  const int64_t kh = (K / 2 + 255) / 256 * 256;
  const int64_t bb = dt == Q4_K ? 144 : 176;  // bytes per 256-element block
  const int64_t q2 = act_q2_off(M, K), d = act_d_off(M, K), so = act_s_off(M, K);
  const uint8_t *act = static_cast<const uint8_t *>(act_in);
  for (int64_t m = 0; m < M; m++) {
    for (int h = 0; h < 2; h++) {
      const int64_t k0 = h ? kh : 0, kn = h ? K - kh : kh, e0 = m * K + k0;  // first element
      Q4kxArgs a;
      if (int rc = q4kx_setup(a, 1, N, kn, 256, q4kx_row_bytes(dt, K), "gemv_q4kx")) return rc;
      a.ain = act + e0;
      a.in_q2 = q2;                      // q2 base: act + q2 + e0
      a.in_d = d + 8 * (e0 / 32) - e0;   // (d, e) base: act + d + 8 e0 / 32
      a.in_s = so + 4 * (e0 / 32) - e0;  // sx base: act + s + 4 e0 / 32
      a.w0 = static_cast<const uint8_t *>(w) + k0 / 256 * bb;
      a.out = (h ? tmp : out) + m * N;
      const int rc = with_qk_unit(dt, kn, [&](auto unit) {
        using U = decltype(unit);
        if (gemv_rows_ok(a)) return run_gemv_rows<U>(a, s);
        return dispatch_q4kx<U, false, false, false, F32, F32, 2>(a, s);
      });
      if (rc) return rc;
    }
  }
  return launch_add_rows(out, tmp, M * N, s);
}

// The same halves for M >= 2 rows of F32 x: each half's columns of x are copied out and
// quantized as an (M, kn) activation, so one launch serves every row of x and the weights
// are read once per half (not once per row).  ws: the half's x, its act layout, then M * N
// floats (q4kx_halves_x_ws_bytes).
size_t q4kx_halves_x_ws_bytes(int64_t M, int64_t N, int64_t K) {
  const int64_t kh = (K / 2 + 255) / 256 * 256;
  auto al = [](int64_t b) { return (b + 255) & ~(int64_t)255; };
  return (size_t)(al(4 * M * kh) + al(act_bytes(M, kh)) + 4 * M * N);
}

int launch_gemv_q4kx_halves_x(const float *x, const void *w, float *out, void *ws, int64_t M, int64_t N, int64_t K,
                              int dt, hipStream_t s) {
  const int64_t kh = (K / 2 + 255) / 256 * 256;
  const int64_t bb = dt == Q4_K ? 144 : 176;
  auto al = [](int64_t b) { return (b + 255) & ~(int64_t)255; };
  float *xb = static_cast<float *>(ws);
  uint8_t *ab = reinterpret_cast<uint8_t *>(ws) + al(4 * M * kh);
  float *tmp = reinterpret_cast<float *>(ab + al(act_bytes(M, kh)));
  for (int h = 0; h < 2; h++) {
    const int64_t k0 = h ? kh : 0, kn = h ? K - kh : kh;
    if (hipError_t e = hipMemcpy2DAsync(xb, (size_t)kn * 4, x + k0, (size_t)K * 4, (size_t)kn * 4, (size_t)M,
                                        hipMemcpyDeviceToDevice, s))
      return fail((int)e, "gemv_q4kx", "hipMemcpy2DAsync: %s", hipGetErrorString(e));
    if (int rc = launch_quantize_act(xb, F32, ab, M, kn, s)) return rc;
    Q4kxArgs a;
    if (int rc = q4kx_setup(a, M, N, kn, 256, q4kx_row_bytes(dt, K), "gemv_q4kx")) return rc;
    a.ain = ab;
    a.w0 = static_cast<const uint8_t *>(w) + k0 / 256 * bb;
    a.out = h ? tmp : out;
    const int rc = with_qk_unit(dt, kn, [&](auto unit) {
      using U = decltype(unit);
      if (gemv_rows_ok(a)) return run_gemv_rows<U>(a, s);
      return dispatch_q4kx<U, false, false, false, F32, F32, 2>(a, s);
    });
    if (rc) return rc;
  }
  return launch_add_rows(out, tmp, M * N, s);
}

int launch_add_rows(float *out, const float *tmp, int64_t n, hipStream_t s) {
  add_rows_kernel<<<(unsigned)cdiv(n, 256), 256, 0, s>>>(out, tmp, n);
  return check_launch("add_rows");
}

// int4 GEMV on x (F32 / BF16 / F16) quantized in the kernel; y at x's dtype.
bool int4x_ok(int64_t M, int64_t N, int64_t K, int G, const void *codes, const void *x) {
  int P, TP, RW;
  if (M < 1 || M > kGemvMaxRows || G <= 0 || G % 32 || K % G || !q4kx_geom(K, 64, &P, &TP, &RW)) return false;
  if (N > INT32_MAX / 2 || (N + 1) * (K / 2) > UINT32_MAX) return false;
  if (((uintptr_t)codes & 15) || ((uintptr_t)x & 15)) return false;
  return q4kx_lds(mm_of(M), K, TP, RW, 1, true, false) <= 160 * 1024;
}

int launch_gemv_int4x(const void *x, int x_dtype, const uint32_t *codes, const float *sc, const float *zr, void *y,
                      int64_t M, int64_t N, int64_t K, int G, void *ws, hipStream_t s) {
  Q4kxArgs a;
  if (int rc = q4kx_setup(a, M, N, K, 64, K / 2, "int4_gemv")) return rc;
  a.w0 = reinterpret_cast<const uint8_t *>(codes);
  a.s0 = sc;
  a.z0 = zr;
  a.G = G;
  a.out = y;
  if (!q4kx_xin(K)) {
    // Long rows: one quantize launch beats every workgroup quantizing all of x.
    if (int rc = launch_quantize_act(x, x_dtype, ws, M, K, s)) return rc;
    a.ain = static_cast<const uint8_t *>(ws);
    // Two rows per team (15.0 -> 13.8 us at 3584 x 18944); rows of at least kX1MinK take
    // single-level activations.
    if (a.TP > 64 && K >= kX1MinK && gemv_rows_ok(a)) switch (x_dtype) {
        case F32: return run_gemv_rows<Int4UnitT<false>, F32>(a, s);
        case BF16: return run_gemv_rows<Int4UnitT<false>, BF16>(a, s);
        case F16: return run_gemv_rows<Int4UnitT<false>, F16>(a, s);
        default: return fail(HQ_EUNSUPPORTED, "int4_gemv", "x dtype %d", x_dtype);
      }
    if (a.TP > 64 && K >= kX1MinK) switch (x_dtype) {
      case F32: return dispatch_q4kx<Int4UnitT<false>, false, false, false, F32, F32, 2>(a, s);
      case BF16: return dispatch_q4kx<Int4UnitT<false>, false, false, false, F32, BF16, 2>(a, s);
      case F16: return dispatch_q4kx<Int4UnitT<false>, false, false, false, F32, F16, 2>(a, s);
      default: return fail(HQ_EUNSUPPORTED, "int4_gemv", "x dtype %d", x_dtype);
    }
    if (a.TP > 64 && gemv_rows_ok(a)) switch (x_dtype) {
        case F32: return run_gemv_rows<Int4Unit, F32>(a, s);
        case BF16: return run_gemv_rows<Int4Unit, BF16>(a, s);
        case F16: return run_gemv_rows<Int4Unit, F16>(a, s);
        default: return fail(HQ_EUNSUPPORTED, "int4_gemv", "x dtype %d", x_dtype);
      }
    if (a.TP > 64) switch (x_dtype) {
      case F32: return dispatch_q4kx<Int4Unit, false, false, false, F32, F32, 2>(a, s);
      case BF16: return dispatch_q4kx<Int4Unit, false, false, false, F32, BF16, 2>(a, s);
      case F16: return dispatch_q4kx<Int4Unit, false, false, false, F32, F16, 2>(a, s);
      default: return fail(HQ_EUNSUPPORTED, "int4_gemv", "x dtype %d", x_dtype);
    }
    switch (x_dtype) {
      case F32: return dispatch_q4kx<Int4Unit, false, false, false, F32, F32>(a, s);
      case BF16: return dispatch_q4kx<Int4Unit, false, false, false, F32, BF16>(a, s);
      case F16: return dispatch_q4kx<Int4Unit, false, false, false, F32, F16>(a, s);
      default: return fail(HQ_EUNSUPPORTED, "int4_gemv", "x dtype %d", x_dtype);
    }
  }
  a.x = x;
  if (gemv_cu_ok(a)) switch (x_dtype) {
      case F32: return run_gemv_cu<Int4Unit, false, F32, F32>(a, s);
      case BF16: return run_gemv_cu<Int4Unit, false, BF16, BF16>(a, s);
      case F16: return run_gemv_cu<Int4Unit, false, F16, F16>(a, s);
      default: return fail(HQ_EUNSUPPORTED, "int4_gemv", "x dtype %d", x_dtype);
    }
  switch (x_dtype) {
    case F32: return dispatch_q4kx<Int4Unit, false, true, false, F32, F32>(a, s);
    case BF16: return dispatch_q4kx<Int4Unit, false, true, false, BF16, BF16>(a, s);
    case F16: return dispatch_q4kx<Int4Unit, false, true, false, F16, F16>(a, s);
    default: return fail(HQ_EUNSUPPORTED, "int4_gemv", "x dtype %d", x_dtype);
  }
}

// int4 rows past one team (32768 < K <= 65536, 256 % G == 0) at M <= 8: x quantized once,
// the act GEMV over each K half on the full rows' strides (codes, scales and zeros bases moved
// to the half; the scales' row stride is the full row's groups), both halves to F32 partials,
// then one launch adds them and rounds once to y's dtype.
template <int ODT>
__global__ void add_halves_kernel(void *y, const float *t0, const float *t1, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) store_out<ODT>(y, i, t0[i] + t1[i]);
}

bool int4_halves_ok(int64_t M, int64_t N, int64_t K, int G, const void *codes, const void *x) {
  if (M < 1 || M > kGemvMaxRows || K <= 32768 || K > 65536 || K % 256 || G <= 0 || 256 % G) return false;
  const int64_t kh = (K / 2 + 255) / 256 * 256;
  return int4x_ok(1, N, kh, G, codes, x) && (N + 1) * (K / 2) <= UINT32_MAX &&
         N * (K / G) * 4 <= (int64_t)UINT32_MAX;
}

int launch_int4_halves(const void *x, int x_dtype, const uint32_t *codes, const float *sc, const float *zr, void *y,
                       int64_t M, int64_t N, int64_t K, int G, void *ws, hipStream_t s) {
  const int64_t kh = (K / 2 + 255) / 256 * 256;
  auto al = [](int64_t b) { return (b + 255) & ~(int64_t)255; };
  if (M > 1) {
    // Several rows of x: each half's columns copied out (x's dtype) and quantized as an
    // (M, kn) activation, one launch per half for every row (weights read once per half).
    const int64_t esz = x_dtype == F32 ? 4 : 2;
    uint8_t *xb = static_cast<uint8_t *>(ws), *ab = xb + al(esz * M * kh);
    float *t0 = reinterpret_cast<float *>(ab + al(act_bytes(M, kh))), *t1 = t0 + M * N;
    for (int h = 0; h < 2; h++) {
      const int64_t k0 = h ? kh : 0, kn = h ? K - kh : kh;
      if (hipError_t e = hipMemcpy2DAsync(xb, (size_t)(kn * esz), static_cast<const uint8_t *>(x) + k0 * esz,
                                          (size_t)(K * esz), (size_t)(kn * esz), (size_t)M, hipMemcpyDeviceToDevice, s))
        return fail((int)e, "int4_gemv", "hipMemcpy2DAsync: %s", hipGetErrorString(e));
      if (int rc = launch_quantize_act(xb, x_dtype, ab, M, kn, s)) return rc;
      Q4kxArgs a;
      if (int rc = q4kx_setup(a, M, N, kn, 64, K / 2, "int4_gemv")) return rc;
      a.ain = ab;
      a.w0 = reinterpret_cast<const uint8_t *>(codes) + k0 / 2;
      a.s0 = sc + k0 / G;
      a.z0 = zr + k0 / G;
      a.G = G;
      a.gpr = (int)(K / G);
      a.out = h ? t1 : t0;
      if (int rc = dispatch_q4kx<Int4UnitT<false>, false, false, false, F32, F32, 2>(a, s)) return rc;
    }
    const int64_t n = M * N;
    const unsigned g = (unsigned)cdiv(n, 256);
    switch (x_dtype) {
      case F32: add_halves_kernel<F32><<<g, 256, 0, s>>>(y, t0, t1, n); break;
      case BF16: add_halves_kernel<BF16><<<g, 256, 0, s>>>(y, t0, t1, n); break;
      case F16: add_halves_kernel<F16><<<g, 256, 0, s>>>(y, t0, t1, n); break;
      default: return fail(HQ_EUNSUPPORTED, "int4_gemv", "x dtype %d", x_dtype);
    }
    return check_launch("int4_halves");
  }
  if (int rc = launch_quantize_act(x, x_dtype, ws, M, K, s)) return rc;
  const uint8_t *act = static_cast<const uint8_t *>(ws);
  float *t0 = reinterpret_cast<float *>(static_cast<uint8_t *>(ws) + ((act_bytes(M, K) + 255) & ~(int64_t)255));
  float *t1 = t0 + M * N;
  const int64_t q2 = act_q2_off(M, K), d = act_d_off(M, K), so = act_s_off(M, K);
  for (int64_t m = 0; m < M; m++) {
    for (int h = 0; h < 2; h++) {
      const int64_t k0 = h ? kh : 0, kn = h ? K - kh : kh, e0 = m * K + k0;
      Q4kxArgs a;
      if (int rc = q4kx_setup(a, 1, N, kn, 64, K / 2, "int4_gemv")) return rc;
      a.ain = act + e0;
      a.in_q2 = q2;
      a.in_d = d + 8 * (e0 / 32) - e0;
      a.in_s = so + 4 * (e0 / 32) - e0;
      a.w0 = reinterpret_cast<const uint8_t *>(codes) + k0 / 2;
      a.s0 = sc + k0 / G;
      a.z0 = zr + k0 / G;
      a.G = G;
      a.gpr = (int)(K / G);
      a.out = (h ? t1 : t0) + m * N;
      const int rc = gemv_rows_ok(a) ? run_gemv_rows<Int4UnitT<false>, F32>(a, s)
                                     : dispatch_q4kx<Int4UnitT<false>, false, false, false, F32, F32, 2>(a, s);
      if (rc) return rc;
    }
  }
  const int64_t n = M * N;
  const unsigned g = (unsigned)cdiv(n, 256);
  switch (x_dtype) {
    case F32: add_halves_kernel<F32><<<g, 256, 0, s>>>(y, t0, t1, n); break;
    case BF16: add_halves_kernel<BF16><<<g, 256, 0, s>>>(y, t0, t1, n); break;
    case F16: add_halves_kernel<F16><<<g, 256, 0, s>>>(y, t0, t1, n); break;
    default: return fail(HQ_EUNSUPPORTED, "int4_gemv", "x dtype %d", x_dtype);
  }
  return check_launch("int4_halves");
}

// ---------------------------------------------------------------------------
// Gated projection and the MLP
// ---------------------------------------------------------------------------

// Unfused gated epilogue: out = act(g) * u, elementwise (the path for layouts the fused
// kernel does not take).
__global__ __launch_bounds__(256) void gated_epilogue_kernel(const float *__restrict__ g, const float *__restrict__ u,
                                                             float *__restrict__ out, int64_t n, int act) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = gate_act(g[i], act) * u[i];
}

static int64_t al256(int64_t b) { return (b + 255) & ~(int64_t)255; }

size_t matmul_q_gated_ws_bytes(int64_t M, int64_t N, int64_t K, int dt) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 32) return 0;
  return (size_t)(2 * al256(4 * M * N)) + matmul_q_ws_bytes(M, N, K, dt);
}

int launch_matmul_q_gated(const float *x, const void *wg, const void *wu, float *out, int64_t M, int64_t N, int64_t K,
                          int dt, int act, void *ws, hipStream_t s) {
  if (q4kx_ok(M, N, K, wg, wu, x, dt)) {
    if (q4kx_xin(K)) return launch_gemv_q4kx(x, wg, wu, out, M, N, K, act, dt, s);
    Q4kxArgs a;
    if (int rc = q4kx_setup(a, M, N, K, 256, q4kx_row_bytes(dt, K), "gemv_q4k_gated")) return rc;
    if (int rc = launch_quantize_act(x, F32, ws, M, K, s)) return rc;
    a.ain = static_cast<const uint8_t *>(ws);
    a.w0 = static_cast<const uint8_t *>(wg);
    a.w1 = static_cast<const uint8_t *>(wu);
    a.out = out;
    a.act = act;
    return with_qk_unit(dt, K, [&](auto unit) { return dispatch_q4kx<decltype(unit), true, false, false>(a, s); });
  }
  float *g = static_cast<float *>(ws);
  float *u = reinterpret_cast<float *>(static_cast<char *>(ws) + al256(4 * M * N));
  void *inner = static_cast<char *>(ws) + 2 * al256(4 * M * N);
  if (int rc = launch_matmul_q(x, wg, g, M, N, K, dt, inner, s)) return rc;
  if (int rc = launch_matmul_q(x, wu, u, M, N, K, dt, inner, s)) return rc;
  gated_epilogue_kernel<<<(unsigned)cdiv(M * N, 256), 256, 0, s>>>(g, u, out, M * N, act);
  return check_launch("gated_epilogue");
}

// The two-launch MLP applies: Q4_K / Q5_K, M <= 8, aligned, I a multiple of 256 (the down
// projection's K) and the gate/up workgroup's teams tile 32-row chunks.
static bool mlp_fused_ok(int64_t M, int64_t H, int64_t I, int dt, const void *wg, const void *wu, const void *wd,
                         const float *x) {
  int P, TP, RW;
  if (I % 256 || !q4kx_ok(M, I, H, wg, wu, x, dt) || !q4kx_ok(M, H, I, wd, nullptr, x, dt)) return false;
  if (!q4kx_geom(H, 256, &P, &TP, &RW) || 32 % RW) return false;
  return q4kx_geom(I, 256, &P, &TP, &RW);
}

size_t mlp_q_ws_bytes(int64_t M, int64_t H, int64_t I, int dt) {
  if (M <= 0 || H <= 0 || I <= 0 || H % 32 || I % 32) return 0;
  const size_t fused = (size_t)act_bytes(M, I);
  const size_t unfused =
      (size_t)al256(4 * M * I) + std::max(matmul_q_gated_ws_bytes(M, I, H, dt), matmul_q_ws_bytes(M, H, I, dt));
  return std::max(fused, unfused);
}

size_t matmul_q_gated_act_ws_bytes(int64_t M, int64_t N, int64_t K, int dt) {
  if (M <= 0 || N <= 0 || K <= 0 || N % 32 || K % 32) return 0;
  return (size_t)al256(4 * M * N) + matmul_q_gated_ws_bytes(M, N, K, dt);
}

// ---------------------------------------------------------------------------
// The gated gate/up launch of the decode MLP at one token, K in (2048, 4096] (one wave per
// row), with the quantized-h epilogue: one workgroup per CU owning whole 32-row chunks --
// chunk bx and, with NCH = 2, chunk bx + G.
//
// Each wave reads rows 8 i + wave of its chunks, gate and up together.  x is requested first
// (every dot waits for it), then the first row pair, and x is quantized into LDS while the
// weights stream.  One row pair is in flight per wave while every CU streams its first chunk
// and two during the second chunk (only the CUs that own two chunks are still streaming then):
// measured against one, two, four, six and eight row pairs in flight throughout, this was the
// fastest -- more requests in flight at once lengthen every request's latency more than they
// add bandwidth, as a plain read shows too (hq_ceiling_read, depth 1-2 against 4-8).  The code
// is straight-line, so the compiler's wait before each dot covers that row pair's loads only.
// The arithmetic -- unit dots, 16-lane sums, the row sum order, act(g) * u, the chunk's
// quantization -- is gemv_q4kx_kernel<U, 1, GATED, XIN, AOUT>'s, bit for bit.
// 14336 x 4096: 15.2 -> 14.2-14.6 us.
// ---------------------------------------------------------------------------
template <class U, int NCH>
__global__ __launch_bounds__(512) void gate_cu_kernel(Q4kxArgs a) {
  constexpr int RC = 4, R = RC * NCH;  // row pairs per wave: 4 per chunk
  static_assert(NCH == 1 || NCH == 2, "one or two chunks");
  extern __shared__ __align__(16) uint8_t smem[];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int KB = a.K >> 5;
  const bool active = lane < a.P;
  const typename U::Lane L = unit_lane<U>(active ? lane : 0, a.G);
  const int nch = a.N / 32;
  const int c0 = blockIdx.x, c1 = NCH > 1 ? blockIdx.x + (int)gridDim.x : nch;
  auto row_of = [&](int i) __attribute__((always_inline)) {
    const int c = i < RC ? c0 : c1;
    return c < nch ? c * 32 + 8 * (i % RC) + wave : a.N;  // past the end: zeros, no traffic
  };
  typename U::W wg[2], wu[2];
  auto load_row = [&](int i) __attribute__((always_inline)) {
    const int row = row_of(i);
    U::load(a.w0, a.s0, a.z0, a, row, L, wg[i & 1]);
    U::load(a.w1, a.s1, a.z1, a, row, L, wu[i & 1]);
  };

  // x: one 16-element task per thread (K <= 4096: at most 256 tasks).
  uint8_t *lq1 = smem, *lq2 = smem + a.K;
  float2 *lde = reinterpret_cast<float2 *>(smem + 2 * a.K);
  float *lsx = reinterpret_cast<float *>(smem + 2 * a.K + 8 * KB);
  const int ntask = KB * 2;
  const int task = t < ntask ? t : ntask - 1;
  float v[16];
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const float4 f = reinterpret_cast<const float4 *>(static_cast<const float *>(a.x) + (int64_t)task * 16)[r];
    v[4 * r] = f.x, v[4 * r + 1] = f.y, v[4 * r + 2] = f.z, v[4 * r + 3] = f.w;
  }
  load_row(0);
  {
    const ActQ16 q = act_quant16_fast(v);
    if (t < ntask) {
      const int blk = task >> 1, half = task & 1;
      *reinterpret_cast<u32x4_t *>(lq1 + blk * 32 + half * 16) = u32x4_t{q.q1[0], q.q1[1], q.q1[2], q.q1[3]};
      if constexpr (U::kX2)
        *reinterpret_cast<u32x4_t *>(lq2 + blk * 32 + half * 16) = u32x4_t{q.q2[0], q.q2[1], q.q2[2], q.q2[3]};
      if (half == 0) {
        lde[blk] = make_float2(q.d, q.e);
        lsx[blk] = q.sum;
      }
    }
  }
  __syncthreads();
  typename U::X xr[1];
  U::load_x(lq1, lq2, reinterpret_cast<const uint8_t *>(lde), reinterpret_cast<const uint8_t *>(lsx), L.ja, xr[0]);

  float *hb = reinterpret_cast<float *>(smem + q4kx_act_lds(1, a.K));  // [NCH][32]
#pragma unroll
  for (int i = 0; i < R; i++) {
    float cg[1], cu[1];
    U::template dot<1>(wg[i & 1], xr, L, cg);
    U::template dot<1>(wu[i & 1], xr, L, cu);
    // Refill: the next row pair during the first chunk, the one after it (two in flight)
    // from the first chunk's last row on.
    if (i < RC - 1) {
      load_row(i + 1);
    } else if (i == RC - 1 && NCH > 1) {
      load_row(RC);
      load_row(RC + 1);
    } else if (i + 2 < R) {
      load_row(i + 2);
    }
    const float g16 = rsum16(active ? cg[0] : 0.f), u16 = rsum16(active ? cu[0] : 0.f);
    const float tg = ((rl(g16, 0) + rl(g16, 16)) + rl(g16, 32)) + rl(g16, 48);
    const float tu = ((rl(u16, 0) + rl(u16, 16)) + rl(u16, 32)) + rl(u16, 48);
    const int row = row_of(i);
    if (lane == 0 && row < a.N) {
      const float y = gate_act(tg, a.act) * tu;
      if (a.out) static_cast<float *>(a.out)[row] = y;
      hb[(i / RC) * 32 + 8 * (i % RC) + wave] = y;
    }
  }
  __syncthreads();
  // Each chunk's 32 values into the act layout of (1, N): eight lanes per chunk.
  if (t < 8 * NCH) {
    const int ch = t >> 3, sub = t & 7, c = ch ? c1 : c0;
    const float hv[4] = {hb[ch * 32 + sub * 4], hb[ch * 32 + sub * 4 + 1], hb[ch * 32 + sub * 4 + 2],
                         hb[ch * 32 + sub * 4 + 3]};
    const ActQ q = act_quant8_fast(hv);
    if (c < nch) {
      reinterpret_cast<uint32_t *>(a.aout + (int64_t)c * 32)[sub] = q.q1;
      reinterpret_cast<uint32_t *>(a.aout + a.out_q2 + (int64_t)c * 32)[sub] = q.q2;
      if (sub == 0) {
        reinterpret_cast<float2 *>(a.aout + a.out_d)[c] = make_float2(q.d, q.e);
        reinterpret_cast<float *>(a.aout + a.out_s)[c] = q.sum;
      }
    }
  }
}

// One token, one wave per row, 8 teams (K in (2048, 4096]), whole chunks, at most two per CU.
static bool gate_cu_ok(const Q4kxArgs &a) {
  return a.M == 1 && a.TP == 64 && a.RW == 8 && a.P > 32 && a.N % 32 == 0 && a.N / 32 <= 2 * device_cus();
}

template <class U>
static int run_gate_cu(const Q4kxArgs &a, hipStream_t s) {
  const int nch = (int)(a.N / 32), cus = device_cus();
  const size_t lds = (size_t)q4kx_act_lds(1, a.K) + 64 * 4;
  if (nch > cus)
    gate_cu_kernel<U, 2><<<(unsigned)cus, 512, lds, s>>>(a);
  else
    gate_cu_kernel<U, 1><<<(unsigned)nch, 512, lds, s>>>(a);
  return check_launch("gate_cu");
}

// Gated projection whose output is written as prepared activations (act layout of (M, N)).
// Q4_K / Q5_K, M <= 8, aligned, with teams that tile 32-row chunks: one kernel (the gated
// GEMV quantizes its own 32-row output chunks in the epilogue).  Otherwise the gated
// projection runs into ws as F32 and a quantize launch follows.
int launch_matmul_q_gated_act(const float *x, const void *wg, const void *wu, uint8_t *aout, int64_t M, int64_t N,
                              int64_t K, int dt, int act, void *ws, hipStream_t s) {
  int P, TP, RW;
  if (N % 256 == 0 && q4kx_ok(M, N, K, wg, wu, x, dt) && q4kx_geom(K, 256, &P, &TP, &RW) && 32 % RW == 0) {
    Q4kxArgs a;
    if (int rc = q4kx_setup(a, M, N, K, 256, q4kx_row_bytes(dt, K), "matmul_q_gated_act")) return rc;
    a.x = x;
    a.w0 = static_cast<const uint8_t *>(wg);
    a.w1 = static_cast<const uint8_t *>(wu);
    a.aout = aout;
    a.act = act;
    return with_qk_unit(dt, K, [&](auto unit) {
      using U = decltype(unit);
      if (gate_cu_ok(a)) return run_gate_cu<U>(a, s);
      return dispatch_q4kx<U, true, true, true>(a, s);
    });
  }
  float *h = static_cast<float *>(ws);
  void *inner = static_cast<char *>(ws) + al256(4 * M * N);
  if (int rc = launch_matmul_q_gated(x, wg, wu, h, M, N, K, dt, act, inner, s)) return rc;
  return launch_quantize_act(h, F32, aout, M, N, s);
}

int launch_mlp_q(const float *x, const void *wg, const void *wu, const void *wd, float *out, int64_t M, int64_t H,
                 int64_t I, int dt, int act, void *ws, hipStream_t s) {
  if (mlp_fused_ok(M, H, I, dt, wg, wu, wd, x)) {
    // Launch 1: gated gate/up on x, output quantized straight into ws (act layout of (M, I)).
    auto *h = static_cast<uint8_t *>(ws);
    if (int rc = launch_matmul_q_gated_act(x, wg, wu, h, M, I, H, dt, act, nullptr, s)) return rc;
    // Launch 2: down projection on the prepared h.
    return launch_gemv_q4kx_act(h, wd, out, M, H, I, dt, s);
  }
  float *h = static_cast<float *>(ws);
  void *inner = static_cast<char *>(ws) + al256(4 * M * I);
  if (int rc = launch_matmul_q_gated(x, wg, wu, h, M, I, H, dt, act, inner, s)) return rc;
  return launch_matmul_q(h, wd, out, M, H, I, dt, inner, s);
}

bool moe_x_ok(int64_t K, int dt, const void *w, const void *x) {
  int P, TP, RW;
  if ((dt != Q4_K && dt != Q5_K) || !q4kx_geom(K, 256, &P, &TP, &RW) || TP > 64) return false;
  return ((uintptr_t)w & 15) == 0 && ((uintptr_t)x & 15) == 0;
}

template <class U, int MM, bool GATED, bool ROUTE = false>
static int run_moe_x(MoeXArgs &ma, int64_t active, hipStream_t s) {
  const Q4kxArgs &a = ma.g;
  const size_t lds = (size_t)q4kx_act_lds(MM, a.K);
  const int ngroups = (a.N + a.RW - 1) / a.RW;
  // Enough workgroups per active expert to fill the chip (those of empty experts exit).
  // grid.y = segment slot (at most min(pairs, E) segments); grid.x balanced so that every
  // workgroup of a slot takes the same number of row groups.
  int64_t per = cdiv((int64_t)device_cus() * 2, active);
  per = per < ngroups ? per : ngroups;
  per = cdiv(ngroups, cdiv(ngroups, per));
  dim3 grid((unsigned)per, (unsigned)active);
  moe_gemv_x_kernel<U, MM, GATED, ROUTE><<<grid, a.TP * a.RW, lds, s>>>(ma);
  return check_launch("moe_gemv_x");
}

int launch_moe_gemv_x(const float *x, const void *w, const int64_t *pairs, const int64_t *expts, int32_t *counts,
                      int32_t *offsets, const float *topk_w, float *out, int topk, int64_t size_m, int64_t M,
                      int64_t rows, int64_t E, int64_t N, int64_t K, int rpp, int dt, int act, hipStream_t s) {
  MoeXArgs ma;
  const int64_t row_bytes = q4kx_row_bytes(dt, K);
  const bool gated = act >= 0;  // N = I; the expert holds gate rows [0, I) then up rows [I, 2I)
  if (int rc = q4kx_setup(ma.g, 1, gated ? 2 * N : N, K, 256, row_bytes, "moe_gemv")) return rc;
  ma.g.N = (int)N;
  ma.g.x = x;
  ma.g.w0 = static_cast<const uint8_t *>(w);
  ma.g.out = out;
  ma.pairs = pairs;
  ma.expts = expts;
  ma.counts = counts;
  ma.offsets = offsets;
  ma.topk_w = topk_w;
  ma.size_m = size_m;
  ma.expert_bytes = (gated ? 2 * N : N) * row_bytes;
  ma.up_off = gated ? N * row_bytes : 0;
  ma.act = gated ? act : 0;
  ma.rows = rows;
  ma.npairs = M;
  ma.E = (int)E;
  ma.topk = topk;
  ma.rpp = rpp;
  const int64_t active = M < E ? M : E;
  const int64_t avg = active > 0 ? (M + active - 1) / active : 1;
  // Gated: at most two pair rows per pass (two weight rows in registers).
  if (gated) {
    if (dt == Q5_K) return avg <= 1 ? run_moe_x<Q5kUnit, 1, true>(ma, active, s) : run_moe_x<Q5kUnit, 2, true>(ma, active, s);
    return avg <= 1 ? run_moe_x<Q4kUnit, 1, true>(ma, active, s) : run_moe_x<Q4kUnit, 2, true>(ma, active, s);
  }
  if (dt == Q5_K) {
    if (avg <= 1) return run_moe_x<Q5kUnit, 1, false>(ma, active, s);
    if (avg <= 2) return run_moe_x<Q5kUnit, 2, false>(ma, active, s);
    return run_moe_x<Q5kUnit, 4, false>(ma, active, s);
  }
  if (avg <= 1) return run_moe_x<Q4kUnit, 1, false>(ma, active, s);
  if (avg <= 2) return run_moe_x<Q4kUnit, 2, false>(ma, active, s);
  return run_moe_x<Q4kUnit, 4, false>(ma, active, s);
}

// The fused down + combine applies to Q4_K / Q5_K decode (K fits one wave's team, topk teams
// fit a workgroup), with every pair row in range (size_m == M).
bool moe_comb_ok(int64_t M, int64_t T, int topk, int64_t K, int dt, const void *w, const void *x) {
  int P, TP, RW;
  if ((dt != Q4_K && dt != Q5_K) || topk > 64 || M != T * topk || T > 65535) return false;
  if (!q4kx_geom(K, 256, &P, &TP, &RW) || TP > 64 || RW % topk) return false;
  return ((uintptr_t)w & 15) == 0 && ((uintptr_t)x & 15) == 0;
}

int launch_moe_down_combine(const float *h, const void *w, const int64_t *pairs, const int64_t *expts,
                            int32_t *counts, int32_t *offsets, const float *topk_w, float *y, int topk, int64_t T,
                            int64_t E, int64_t N, int64_t K, int dt, hipStream_t s) {
  MoeCombArgs ma;
  const int64_t row_bytes = q4kx_row_bytes(dt, K);
  if (int rc = q4kx_setup(ma.g, 1, N, K, 256, row_bytes, "moe_gemm_q_combine")) return rc;
  ma.g.x = h;
  ma.g.w0 = static_cast<const uint8_t *>(w);
  ma.g.out = y;
  ma.pairs = pairs;
  ma.expts = expts;
  ma.counts = counts;
  ma.offsets = offsets;
  ma.topk_w = topk_w;
  ma.expert_bytes = N * row_bytes;
  ma.npairs = T * topk;
  ma.E = (int)E;
  ma.topk = topk;
  const int RPW = ma.g.RW / topk;
  const int64_t ngroups = cdiv(N, RPW);
  // Enough workgroups to fill the chip over all tokens, each taking whole row groups.
  int64_t per = cdiv((int64_t)device_cus() * 2, T);
  per = per < ngroups ? per : ngroups;
  per = cdiv(ngroups, cdiv(ngroups, per));
  const size_t lds = (size_t)q4kx_act_lds(topk, K) + 64 * 4 + 2 * (size_t)RPW * topk * 4;
  dim3 grid((unsigned)per, (unsigned)T);
  // Two-level activations at every K, as moe_gemv_x_kernel uses (Q4kUnit / Q5kUnit).
  if (dt == Q5_K)
    moe_down_combine_kernel<Q5kUnit><<<grid, ma.g.TP * ma.g.RW, lds, s>>>(ma);
  else
    moe_down_combine_kernel<Q4kUnit><<<grid, ma.g.TP * ma.g.RW, lds, s>>>(ma);
  return check_launch("moe_down_combine");
}

// MoERoute + the routed gated gate/up in one launch: every workgroup routes the T tokens
// itself (route_in_workgroup) and takes its expert segment from that.  Applies to Q4_K /
// Q5_K with T <= 8, T * topk <= 64, E <= 1024 and the decode GEMV's geometry.
bool moe_route_gated_ok(int64_t T, int64_t E, int topk, int64_t K, int dt, const void *w, const void *x) {
  const int64_t M = T * topk;
  return T >= 1 && T <= 8 && M <= 64 && E >= 1 && E <= 1024 && topk <= E && M <= 4 * E && moe_x_ok(K, dt, w, x);
}

int launch_moe_route_gated(const float *probs, const float *x, const void *w, float *h, int64_t T, int64_t E,
                           int topk, int normalize, int64_t I, int64_t K, int dt, int act, int64_t *topk_ids,
                           float *weights, int64_t *sorted_pairs, int64_t *sorted_expts, int32_t *counts,
                           int32_t *offsets, hipStream_t s) {
  MoeXArgs ma;
  const int64_t row_bytes = q4kx_row_bytes(dt, K);
  if (int rc = q4kx_setup(ma.g, 1, 2 * I, K, 256, row_bytes, "moe_route_gated")) return rc;
  const int64_t M = T * topk;
  ma.g.N = (int)I;
  ma.g.x = x;
  ma.g.w0 = static_cast<const uint8_t *>(w);
  ma.g.out = h;
  ma.pairs = nullptr;
  ma.expts = nullptr;
  ma.counts = counts;
  ma.offsets = offsets;
  ma.topk_w = nullptr;
  ma.size_m = M;
  ma.expert_bytes = 2 * I * row_bytes;
  ma.up_off = I * row_bytes;
  ma.act = act;
  ma.rows = T;
  ma.npairs = M;
  ma.E = (int)E;
  ma.topk = topk;
  ma.rpp = 0;
  ma.probs = probs;
  ma.topk_ids = topk_ids;
  ma.weights_out = weights;
  ma.sorted_pairs_out = sorted_pairs;
  ma.sorted_expts_out = sorted_expts;
  ma.T = (int)T;
  ma.normalize = normalize;
  const int64_t active = M < E ? M : E;
  const int64_t avg = (M + active - 1) / active;
  if (dt == Q5_K)
    return avg <= 1 ? run_moe_x<Q5kUnit, 1, true, true>(ma, active, s) : run_moe_x<Q5kUnit, 2, true, true>(ma, active, s);
  return avg <= 1 ? run_moe_x<Q4kUnit, 1, true, true>(ma, active, s) : run_moe_x<Q4kUnit, 2, true, true>(ma, active, s);
}

// The one-launch MoE block's barrier words: a file-scope device array (zero when the library
// loads) that serves one stream per device -- the first to run the block; other streams take
// the two launches (two such grids side by side could each hold CUs the other waits for).
// Beside it, per device, a pinned host word that a workgroup giving up at the barrier sets
// (system scope), so the host sees the failure without synchronizing; after a failure the
// device takes the two launches until moe_block_set_spin_limit() re-enables the one launch.
static __device__ __align__(256) uint32_t g_moe_bar[kBarWords];

namespace {
struct MoeBarState {
  uint32_t *bar = nullptr;         // device address of g_moe_bar on this device
  volatile uint32_t *flag = nullptr;  // pinned host word
  hipStream_t owner = nullptr;
  bool init = false, disabled = false;
};
std::mutex g_bar_mu;
MoeBarState g_bar[64];
uint32_t g_bar_limit = kBarSpinLimit;

MoeBarState *moe_bar_state(int *dev_out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    return nullptr;
  }
  *dev_out = dev;
  MoeBarState &st = g_bar[dev];
  if (!st.init) {
    void *p = nullptr, *h = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_moe_bar)) != hipSuccess || !p) {
      (void)hipGetLastError();
      return nullptr;
    }
    if (hipHostMalloc(&h, 256, hipHostMallocCoherent | hipHostMallocMapped) != hipSuccess || !h) {
      (void)hipGetLastError();
      return nullptr;
    }
    st.bar = static_cast<uint32_t *>(p);
    st.flag = static_cast<volatile uint32_t *>(h);
    *st.flag = 0;
    st.init = true;
  }
  return &st;
}

// HQ_OK, or the error of a one-launch block on this device whose barrier gave up since the
// last check (the flag is cleared and the device falls back to the two launches).
int moe_bar_take_failure(MoeBarState &st, const char *call) {
  if (!st.flag || *st.flag == 0) return HQ_OK;
  *st.flag = 0;
  st.disabled = true;
  return fail(HQ_EBARRIER, call,
              "an earlier one-launch MoE block on this device gave up at its grid barrier (the grid was "
              "not resident at once); that call's y holds NaN, and later calls take the two launches");
}
}  // namespace

int moe_block_check(hipStream_t s, const char *call) {
  if (hipError_t e = hipStreamSynchronize(s)) return fail((int)e, call, "hipStreamSynchronize: %s", hipGetErrorString(e));
  std::lock_guard<std::mutex> lk(g_bar_mu);
  int dev = 0;
  MoeBarState *st = moe_bar_state(&dev);
  return st ? moe_bar_take_failure(*st, call) : HQ_OK;
}

void moe_block_forget_stream(hipStream_t s) {
  std::lock_guard<std::mutex> lk(g_bar_mu);
  for (auto &st : g_bar)
    if (st.init && st.owner == s) st.owner = nullptr;
}

void moe_block_set_spin_limit(uint32_t limit) {
  std::lock_guard<std::mutex> lk(g_bar_mu);
  g_bar_limit = limit;
  int dev = 0;
  if (MoeBarState *st = moe_bar_state(&dev)) {
    st->disabled = false;
    st->owner = nullptr;  // the next stream to run the block owns it
  }
}

// MoERoute + gated gate/up + down + MoECombine for one token in one launch; returns 1 (and
// launches nothing) where it does not apply: Q4_K / Q5_K, T = 1, the route_gated and
// down-combine geometries, and a grid that fits the device at once.
// The one-workgroup-per-CU block (moe_block1_kernel); returns 1 where it does not apply.
static int launch_moe_block1(const MoeXArgs &ra, const Q4kxArgs &da0, const uint8_t *wgu, const uint8_t *wdn, float *h,
                             uint8_t *hact, float *y, int64_t H, int64_t I, int topk, int act, int dt, uint32_t *bar,
                             uint32_t limit, uint32_t *host_flag, hipStream_t s) {
  constexpr int kNo = 1;
  MoeBlock1Args b;
  b.ra = ra;
  b.ga = ra.g;
  b.ga.N = (int)(2 * I);  // an expert's gate rows then its up rows
  b.da = da0;
  const int G = device_cus();
  const int TP1 = b.ga.TP, RW1 = b.ga.RW, TP2 = b.da.TP, RW2 = b.da.RW;
  if (TP1 > 64 || 32 % RW1 || I % 32 || TP2 > 64 || RW2 % topk || H > 4096) return kNo;
  if (topk * (I / 32) > G || ((uintptr_t)ra.g.x & 15)) return kNo;
  const int rpw = (int)cdiv(H, G);
  const int nr = (int)cdiv((int64_t)rpw * topk, RW2), r1 = 32 / RW1;
  if (nr > 4 || nr == 3) return kNo;
  const size_t lds = std::max((size_t)q4kx_act_lds(1, H) + 32 * 4, (size_t)q4kx_act_lds(topk, I) + 4 * (size_t)rpw * topk);
  if (lds > 64 * 1024) return kNo;
  b.wgu = wgu;
  b.wdn = wdn;
  b.h = h;
  b.hact = hact;
  b.y = y;
  b.gu_bytes = 2 * I * b.ga.row_bytes;
  b.dn_bytes = H * b.da.row_bytes;
  b.I = (int)I;
  b.H = (int)H;
  b.topk = topk;
  b.act = act;
  b.rpw = rpw;
  auto launch = [&](auto unit) {
    using U = decltype(unit);
    auto go = [&](auto R1c, auto NRc) {
      moe_block1_kernel<U, decltype(R1c)::value, decltype(NRc)::value><<<(unsigned)G, 512, lds, s>>>(b, bar, limit,
                                                                                                     host_flag);
      return check_launch("moe_block1");
    };
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I4 = std::integral_constant<int, 4>;
    if (r1 == 1) return nr == 1 ? go(I1{}, I1{}) : nr == 2 ? go(I1{}, I2{}) : go(I1{}, I4{});
    if (r1 == 2) return nr == 1 ? go(I2{}, I1{}) : nr == 2 ? go(I2{}, I2{}) : go(I2{}, I4{});
    if (r1 == 4) return nr == 1 ? go(I4{}, I1{}) : nr == 2 ? go(I4{}, I2{}) : go(I4{}, I4{});
    return kNo;
  };
  return dt == Q5_K ? launch(Q5kUnit{}) : launch(Q4kUnit{});
}

int launch_moe_block(const float *probs, const float *x, const void *wgu, const void *wdn, float *h, float *y,
                     int64_t T, int64_t E, int topk, int normalize, int64_t H, int64_t I, int dt, int act,
                     int64_t *topk_ids, float *weights, int64_t *sorted_pairs, int64_t *sorted_expts,
                     int32_t *counts, int32_t *offsets, uint8_t *hact, hipStream_t s) {
  constexpr int kNo = 1;
  if (T != 1 || (dt != Q4_K && dt != Q5_K) || topk > 64) return kNo;
  if (!moe_route_gated_ok(T, E, topk, H, dt, wgu, x) || !moe_comb_ok(topk, T, topk, I, dt, wdn, h)) return kNo;
  uint32_t *bar = nullptr;
  uint32_t *host_flag = nullptr;
  uint32_t limit = 0;
  {
    std::lock_guard<std::mutex> lk(g_bar_mu);
    int dev = 0;
    MoeBarState *st = moe_bar_state(&dev);
    if (!st) return kNo;
    if (int rc = moe_bar_take_failure(*st, "hq_moe_block_q")) return rc;
    if (st->disabled) return kNo;
    if (!st->owner) st->owner = s;
    if (st->owner != s) return kNo;
    bar = st->bar;
    host_flag = const_cast<uint32_t *>(st->flag);
    limit = g_bar_limit;
  }
  MoeXArgs ma1;
  const int64_t rb1 = q4kx_row_bytes(dt, H), rb2 = q4kx_row_bytes(dt, I);
  if (q4kx_setup(ma1.g, 1, 2 * I, H, 256, rb1, "moe_block")) return kNo;
  const int64_t M = T * topk;
  ma1.g.N = (int)I;
  ma1.g.x = x;
  ma1.g.w0 = static_cast<const uint8_t *>(wgu);
  ma1.g.out = h;
  ma1.pairs = nullptr;
  ma1.expts = nullptr;
  ma1.counts = counts;
  ma1.offsets = offsets;
  ma1.topk_w = nullptr;
  ma1.size_m = M;
  ma1.expert_bytes = 2 * I * rb1;
  ma1.up_off = I * rb1;
  ma1.act = act;
  ma1.rows = T;
  ma1.npairs = M;
  ma1.E = (int)E;
  ma1.topk = topk;
  ma1.rpp = 0;
  ma1.probs = probs;
  ma1.topk_ids = topk_ids;
  ma1.weights_out = weights;
  ma1.sorted_pairs_out = sorted_pairs;
  ma1.sorted_expts_out = sorted_expts;
  ma1.T = (int)T;
  ma1.normalize = normalize;
  MoeCombArgs ma2;
  if (q4kx_setup(ma2.g, 1, H, I, 256, rb2, "moe_block")) return kNo;
  ma2.g.x = h;
  ma2.g.w0 = static_cast<const uint8_t *>(wdn);
  ma2.g.out = y;
  ma2.pairs = nullptr;
  ma2.expts = nullptr;
  ma2.counts = nullptr;
  ma2.offsets = nullptr;
  ma2.topk_w = nullptr;
  ma2.expert_bytes = H * rb2;
  ma2.npairs = M;
  ma2.E = (int)E;
  ma2.topk = topk;
  if (ma1.g.TP * ma1.g.RW > 512 || ma2.g.TP * ma2.g.RW > 512) return kNo;
  if (hact) {
    const int rc1 = launch_moe_block1(ma1, ma2.g, static_cast<const uint8_t *>(wgu), static_cast<const uint8_t *>(wdn),
                                      h, hact, y, H, I, topk, act, dt, bar, limit, host_flag, s);
    if (rc1 != kNo) return rc1;
  }
  // Gate/up grid as run_moe_x sizes it; the down projection's row groups over the same grid.
  const int64_t nseg = M < E ? M : E;
  const int ngroups1 = (ma1.g.N + ma1.g.RW - 1) / ma1.g.RW;
  int64_t per = cdiv((int64_t)device_cus() * 2, nseg);
  per = per < ngroups1 ? per : ngroups1;
  per = cdiv(ngroups1, cdiv(ngroups1, per));
  const size_t lds = std::max((size_t)q4kx_act_lds(1, H),
                              (size_t)q4kx_act_lds(topk, I) + 64 * 4 + 2 * (size_t)(ma2.g.RW / topk) * topk * 4);
  if (lds > 64 * 1024) return kNo;
  auto *kern = dt == Q5_K ? &moe_block_kernel<Q5kUnit> : &moe_block_kernel<Q4kUnit>;
  static int per_cu[2] = {-1, -1};
  int &pc = per_cu[dt == Q5_K];
  if (pc < 0) {
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, reinterpret_cast<const void *>(kern), 512, lds) !=
        hipSuccess) {
      (void)hipGetLastError();
      nb = 0;
    }
    pc = nb;
  }
  const int64_t resident = (int64_t)device_cus() * (pc < 2 ? pc : 2);
  const int64_t G = std::max<int64_t>(per * nseg, device_cus() * 2);
  if (pc < 1 || G > resident) return kNo;
  kern<<<(unsigned)G, 512, lds, s>>>(ma1, ma2, bar, (int)per, (int)nseg, limit, host_flag);
  if (int rc = check_launch("moe_block")) return rc;
  return HQ_OK;
}

// MoEInt4 on the decode GEMV machinery: H and I multiples of 64, G % 32 == 0, topk teams of
// the down projection fit a workgroup.
bool moe_int4_ok(int64_t H, int64_t I, int G, int topk) {
  int P, TP, RW;
  if (H % 64 || I % 64 || G <= 0 || G % 32 || H % G || I % G || topk < 1 || topk > 64) return false;
  if (!q4kx_geom(H, 64, &P, &TP, &RW) || TP > 64) return false;
  if (!q4kx_geom(I, 64, &P, &TP, &RW) || TP > 64 || RW % topk) return false;
  return q4kx_act_lds(topk, I) + 2 * 4 * 64 <= 64 * 1024;
}

size_t moe_int4_ws_bytes(int64_t T, int topk, int64_t I) { return (size_t)(T * topk * I * 4 + 255) & ~(size_t)255; }

int launch_moe_int4(const void *x, int x_dtype, const void *const *tab, int64_t E, const int64_t *ids,
                    const float *w, void *y, int64_t T, int topk, int64_t H, int64_t I, int G, int act, void *ws,
                    hipStream_t s) {
  MoeInt4Args ma;
  ma.tab = tab;
  ma.ids = ids;
  ma.w = w;
  ma.h = static_cast<float *>(ws);
  ma.E = (int)E;
  ma.topk = topk;
  ma.T = (int)T;
  ma.I = (int)I;
  ma.H = (int)H;
  ma.act = act;
  ma.x_dtype = x_dtype;
  const int64_t M = T * topk;
  if (!moe_int4_ok(H, I, G, topk)) {
    ma.g.G = G;
    ma.g.x = x;
    ma.g.out = y;
    const unsigned b1 = (unsigned)cdiv(M * I, 4), b2 = (unsigned)cdiv(T * H, 4);
    switch (x_dtype) {
      case F32: moe_int4_generic_gated_kernel<F32><<<b1, 256, 0, s>>>(ma); break;
      case BF16: moe_int4_generic_gated_kernel<BF16><<<b1, 256, 0, s>>>(ma); break;
      default: moe_int4_generic_gated_kernel<F16><<<b1, 256, 0, s>>>(ma); break;
    }
    if (int rc = check_launch("moe_int4_gated")) return rc;
    switch (x_dtype) {
      case F32: moe_int4_generic_down_kernel<F32><<<b2, 256, 0, s>>>(ma); break;
      case BF16: moe_int4_generic_down_kernel<BF16><<<b2, 256, 0, s>>>(ma); break;
      default: moe_int4_generic_down_kernel<F16><<<b2, 256, 0, s>>>(ma); break;
    }
    return check_launch("moe_int4_down");
  }
  // Gate / up: K = H, rows I (x2); one workgroup column per routed pair.
  if (int rc = q4kx_setup(ma.g, 1, 2 * I, H, 64, H / 2, "moe_int4")) return rc;
  ma.g.G = G;
  ma.g.x = x;
  {
    const int ngroups = (int)cdiv(I, ma.g.RW);
    int64_t per = cdiv((int64_t)device_cus() * 2, M);
    per = per < ngroups ? per : ngroups;
    per = cdiv(ngroups, cdiv(ngroups, per));
    dim3 grid((unsigned)per, (unsigned)M);
    const size_t lds = (size_t)q4kx_act_lds(1, H);
    const unsigned thr = ma.g.TP * ma.g.RW;
    switch (x_dtype) {
      case F32: moe_int4_gated_kernel<Int4Unit, F32><<<grid, thr, lds, s>>>(ma); break;
      case BF16: moe_int4_gated_kernel<Int4Unit, BF16><<<grid, thr, lds, s>>>(ma); break;
      default: moe_int4_gated_kernel<Int4Unit, F16><<<grid, thr, lds, s>>>(ma); break;
    }
    if (int rc = check_launch("moe_int4_gated")) return rc;
  }
  // Down: K = I, rows H; token-major with the slots combined in the epilogue.
  if (int rc = q4kx_setup(ma.g, 1, H, I, 64, I / 2, "moe_int4")) return rc;
  ma.g.G = G;
  ma.g.out = y;
  const int RPW = ma.g.RW / topk;
  const int64_t ngroups = cdiv(H, RPW);
  int64_t per = cdiv((int64_t)device_cus() * 2, T);
  per = per < ngroups ? per : ngroups;
  per = cdiv(ngroups, cdiv(ngroups, per));
  dim3 grid((unsigned)per, (unsigned)T);
  const size_t lds = (size_t)q4kx_act_lds(topk, I) + 2 * (size_t)RPW * topk * 4;
  const unsigned thr = ma.g.TP * ma.g.RW;
  switch (x_dtype) {
    case F32: moe_int4_down_kernel<Int4Unit, F32><<<grid, thr, lds, s>>>(ma); break;
    case BF16: moe_int4_down_kernel<Int4Unit, BF16><<<grid, thr, lds, s>>>(ma); break;
    default: moe_int4_down_kernel<Int4Unit, F16><<<grid, thr, lds, s>>>(ma); break;
  }
  return check_launch("moe_int4_down");
}

}  // namespace hq

