// gemv_q4kx.hip -- Q4_K decode GEMV (M <= 8): plain, gated (SwiGLU / GELU-erf) and the
// two-launch MLP (gated gate/up emitting quantized h, then down).
//
// Role: Light's matmul_q for small M (ops/matmul_q.go:61-75, kernels/cuda/matmul_q.go:44-91)
// and the gated MLP decode out = act(x . Wg^T) * (x . Wu^T) followed by the down projection,
// which Light computes as MatMulQ, MatMulQ, SiLU / GeluErf, Mul, MatMulQ
// (models/llama.go:1306-1333; the dense BF16 analogue is ops.GatedLinear, ops/gemv.go:80-130).
//
// Design (gfx950, wave64):
//  * Activations are two-level int8 (the act layout of common.hpp).  They come either
//    prepared from global memory (XIN = false) or from F32 x that each workgroup quantizes
//    into LDS itself (XIN = true, act_quant8_fast), which saves a launch.
//  * Lane = one (block, 64-element pair) of a weight row: 32 quant bytes (two 16-byte loads)
//    + one header dword, broadcast in the block's 4-lane quad by DPP.  A team of TP lanes
//    covers a row; a workgroup holds RW teams; each lane keeps its pair's activations in
//    registers for the whole kernel.
//  * Workgroups are persistent (two per CU).  A ring of D register slots (D = 1) keeps the
//    next row group's loads in flight while the current one is reduced; every load is unconditional (inactive lanes and rows past N read valid
//    addresses and their sums are dropped), so no load sits in a branch and the compiler's
//    wait counts stay exact.
//  * Team sums: DPP row sums, then v_readlane over the wave's four rows; teams wider than a
//    wave add their 16-lane row sums through LDS (one barrier per group).  Row sums are added
//    in row order in both cases.
//  * AOUT: the workgroup owns whole 32-row chunks of the output, keeps the chunk's results
//    in LDS and, when a chunk is complete, quantizes it into the act layout for the next
//    matmul (the down projection) -- the gated kernel's output never needs its own
//    quantize launch.
#include "actq.hpp"
#include "internal.hpp"

#include <algorithm>

namespace hq {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

struct Q4kxArgs {
  const float *x;          // XIN: (M, K) F32
  const uint8_t *ain;      // !XIN: prepared activations of (M, K)
  const uint8_t *w0, *w1;  // (N, K) Q4_K; w1 = up projection (gated mode only)
  float *out;              // (M, N) F32, may be NULL with AOUT
  uint8_t *aout;           // AOUT: act layout of the (M, N) output
  int M, N, K, P, TP, RW;  // P: pairs per row (K/64); TP: team lanes; RW: teams per workgroup
  int64_t row_bytes;
  int64_t in_q2, in_d, in_s;     // act offsets of (M, K)
  int64_t out_q2, out_d, out_s;  // act offsets of (M, N)
  int act;                       // gated epilogue: 0 SiLU, 1 GELU (erf)
};

namespace {

template <int K>
__device__ __forceinline__ uint32_t qb(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, K * 0x55, 0xF, 0xF, false);
}

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

// Light's SiLU (kernels/cpu/unary.go:219-222) and exact GELU (:216, :263-265).
__device__ __forceinline__ float gate_act(float g, int act) {
  if (act == 1) return 0.5f * g * (1.0f + erff(g * 0.70710678118654752f));
  return g / (1.0f + expf(-g));
}

}  // namespace

// LDS: act [MM][K] q1 | [MM][K] q2 | (d, e) [MM][K/32] | sx [MM][K/32]  (XIN only)
//      part [2][RW * NW * MM * TP/16]                                   (TP > 64 only)
//      hbuf [2][MM][32]                                                  (AOUT only)
__host__ __device__ constexpr int64_t q4kx_act_lds(int MM, int64_t K) { return MM * (2 * K + 12 * (K / 32)); }

// Byte offsets are 32-bit (the host checks N * row_bytes < 2^32), so loads take the
// scalar-base + vector-offset form.
#define Q4KX_LOAD(S, GRP)                                                             \
  do {                                                                                \
    int row_ = (GRP) * RW + team;                                                     \
    row_ = row_ < a.N ? row_ : a.N - 1;                                               \
    const uint32_t ro_ = (uint32_t)row_ * (uint32_t)a.row_bytes;                      \
    wq0[S][0] = *reinterpret_cast<const u32x4_t *>(a.w0 + (ro_ + qoff));              \
    wq1[S][0] = *reinterpret_cast<const u32x4_t *>(a.w0 + (ro_ + qoff + 16));         \
    wh[S][0] = *reinterpret_cast<const uint32_t *>(a.w0 + (ro_ + hoff));              \
    if (GATED) {                                                                      \
      wq0[S][NW - 1] = *reinterpret_cast<const u32x4_t *>(a.w1 + (ro_ + qoff));       \
      wq1[S][NW - 1] = *reinterpret_cast<const u32x4_t *>(a.w1 + (ro_ + qoff + 16));  \
      wh[S][NW - 1] = *reinterpret_cast<const uint32_t *>(a.w1 + (ro_ + hoff));       \
    }                                                                                 \
  } while (0)

template <int MM, bool GATED, int D, bool XIN, bool AOUT>
__global__ __launch_bounds__(512) void gemv_q4kx_kernel(Q4kxArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  constexpr int NW = GATED ? 2 : 1;
  const int t = threadIdx.x, lane = t & 63;
  const int RW = a.RW, KB = a.K >> 5;
  const int team = t / a.TP, u = t - team * a.TP;
  const bool active = u < a.P;
  const int uu = active ? u : 0;
  const int b = uu >> 2, p = uu & 3;
  const uint32_t qoff = b * 144 + 16 + p * 32, hoff = b * 144 + 4 * p;
  const int ngroups = (a.N + RW - 1) / RW;
  const int m0 = blockIdx.y * MM;
  const int G = gridDim.x;
  // Iteration i of this workgroup -> row group: whole chunks of CG groups (32 rows with
  // AOUT), chunks strided over the grid.
  const int CG = AOUT ? 32 / RW : 1;
  const int nchunks = (ngroups + CG - 1) / CG;
  const int niter = ((nchunks - (int)blockIdx.x + G - 1) / G) * CG;
#define Q4KX_GRP(I) (((int)blockIdx.x + ((I) / CG) * G) * CG + (I) % CG)

  u32x4_t wq0[D][NW], wq1[D][NW];
  uint32_t wh[D][NW];
#pragma unroll
  for (int s = 0; s < D; s++) Q4KX_LOAD(s, Q4KX_GRP(s));

  const int ja = b * 8 + 2 * p;  // this lane's first 32-block in a row of x
  uint32_t xa[MM][8], xb[MM][8], ya[MM][8], yb[MM][8];
  float4 de[MM];
  float2 ss[MM];
  const int64_t lds_act = XIN ? q4kx_act_lds(MM, a.K) : 0;
  if constexpr (XIN) {
    // Quantize this workgroup's MM rows of x into LDS (8 lanes per 32-block).  A chunk's
    // loads are all issued before its quantization.
    uint8_t *lq1 = smem, *lq2 = smem + (int64_t)MM * a.K;
    float2 *lde = reinterpret_cast<float2 *>(smem + 2 * (int64_t)MM * a.K);
    float *lsx = reinterpret_cast<float *>(smem + 2 * (int64_t)MM * a.K + 8 * (int64_t)MM * KB);
    constexpr int XT = 4;
    const int ntask = MM * KB * 8;
    for (int base = 0; base < ntask; base += XT * (int)blockDim.x) {
      float4 xv[XT];
#pragma unroll
      for (int i = 0; i < XT; i++) {
        int task = base + i * (int)blockDim.x + t;
        task = task < ntask ? task : ntask - 1;
        const int blk = task >> 3, sub = task & 7, mm = blk / KB, kb = blk - mm * KB;
        const int m = m0 + mm < a.M ? m0 + mm : a.M - 1;
        xv[i] = *reinterpret_cast<const float4 *>(a.x + (int64_t)m * a.K + kb * 32 + sub * 4);
      }
#pragma unroll
      for (int i = 0; i < XT; i++) {
        const int task = base + i * (int)blockDim.x + t;
        const int blk = task >> 3, sub = task & 7;
        const float v[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
        const ActQ q = act_quant8_fast(v);
        if (task < ntask) {  // uniform over each aligned 8-lane group
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
#pragma unroll
    for (int mm = 0; mm < MM; mm++) {
      const int blk = mm * KB + ja;
      const u32x4_t *s1 = reinterpret_cast<const u32x4_t *>(lq1 + blk * 32);
      const u32x4_t *s2 = reinterpret_cast<const u32x4_t *>(lq2 + blk * 32);
      const u32x4_t v0 = s1[0], v1 = s1[1], v2 = s1[2], v3 = s1[3];
      const u32x4_t w0 = s2[0], w1 = s2[1], w2 = s2[2], w3 = s2[3];
#pragma unroll
      for (int k = 0; k < 4; k++) {
        xa[mm][k] = v0[k], xa[mm][k + 4] = v1[k], xb[mm][k] = v2[k], xb[mm][k + 4] = v3[k];
        ya[mm][k] = w0[k], ya[mm][k + 4] = w1[k], yb[mm][k] = w2[k], yb[mm][k + 4] = w3[k];
      }
      de[mm] = *reinterpret_cast<const float4 *>(lde + blk);
      ss[mm] = *reinterpret_cast<const float2 *>(lsx + blk);
    }
  } else {
#pragma unroll
    for (int mm = 0; mm < MM; mm++) {
      const int m = m0 + mm < a.M ? m0 + mm : a.M - 1;
      const int64_t blk = (int64_t)m * KB + ja;
      const u32x4_t *s1 = reinterpret_cast<const u32x4_t *>(a.ain + blk * 32);
      const u32x4_t *s2 = reinterpret_cast<const u32x4_t *>(a.ain + a.in_q2 + blk * 32);
      const u32x4_t v0 = s1[0], v1 = s1[1], v2 = s1[2], v3 = s1[3];
      const u32x4_t w0 = s2[0], w1 = s2[1], w2 = s2[2], w3 = s2[3];
#pragma unroll
      for (int k = 0; k < 4; k++) {
        xa[mm][k] = v0[k], xa[mm][k + 4] = v1[k], xb[mm][k] = v2[k], xb[mm][k + 4] = v3[k];
        ya[mm][k] = w0[k], ya[mm][k + 4] = w1[k], yb[mm][k] = w2[k], yb[mm][k + 4] = w3[k];
      }
      de[mm] = *reinterpret_cast<const float4 *>(a.ain + a.in_d + 8 * blk);
      ss[mm] = *reinterpret_cast<const float2 *>(a.ain + a.in_s + 4 * blk);
    }
  }

  const bool lowj = p < 2;
  const uint32_t sel = lowj ? ~0u : 0u, mlo = lowj ? 0x3F3Fu : 0x0F0Fu, mhi = lowj ? 0u : 0x3030u;
  const int ka = (2 * p) & 3;
  const int wpt = a.TP >> 6;  // waves per team (0 when a team is narrower than a wave)
  const int hpt = a.TP >> 4;  // 16-lane rows per team
  float *part = reinterpret_cast<float *>(smem + lds_act);
  float *hbuf = part + (wpt > 1 ? 2 * RW * NW * MM * hpt : 0);

  for (int i0 = 0; i0 < niter; i0 += D) {
#pragma unroll
    for (int s = 0; s < D; s++) {
      const int it = i0 + s;
      const int grp = Q4KX_GRP(it);
      float res[NW][MM];
#pragma unroll
      for (int j = 0; j < NW; j++) {
        const uint32_t hd = wh[s][j];
        const uint32_t h0 = qb<0>(hd), h1 = qb<1>(hd), h2 = qb<2>(hd), h3 = qb<3>(hd);
        const float d = h2f(h0 & 0xffffu), dmin = h2f(h0 >> 16);
        // 6-bit (scale, min) of sub-blocks 2p and 2p+1 (getScaleMinK4, quant/q4_k.go:83-89).
        const uint32_t t1 = (h1 >> (8 * ka)) & 0xffffu, t2 = (h2 >> (8 * ka)) & 0xffffu;
        const uint32_t t3 = (h3 >> (8 * ka)) & 0xffffu;
        // Branch-free select with lane constants (v_bfi / v_and_or): p < 2 takes the low six
        // bits of scales[j] / scales[j+4]; p >= 2 combines nibbles of scales[j+4] with the top
        // two bits of scales[j-4] / scales[j].
        const uint32_t srcS = (t1 & sel) | (t3 & ~sel), srcM = (t2 & sel) | ((t3 >> 4) & ~sel);
        const uint32_t scp = (srcS & mlo) | ((t1 >> 2) & mhi), mnp = (srcM & mlo) | ((t2 >> 2) & mhi);
        const float scA = (float)(scp & 0xffu), scB = (float)(scp >> 8);
        const float mnA = (float)(mnp & 0xffu), mnB = (float)(mnp >> 8);
        uint32_t lo[8], hi[8];
#pragma unroll
        for (int k = 0; k < 4; k++) {
          lo[k] = wq0[s][j][k] & 0x0F0F0F0Fu;
          hi[k] = (wq0[s][j][k] >> 4) & 0x0F0F0F0Fu;
          lo[k + 4] = wq1[s][j][k] & 0x0F0F0F0Fu;
          hi[k + 4] = (wq1[s][j][k] >> 4) & 0x0F0F0F0Fu;
        }
#pragma unroll
        for (int mm = 0; mm < MM; mm++) {
          int dA = 0, dB = 0, dA2 = 0, dB2 = 0;
#pragma unroll
          for (int k = 0; k < 8; k++) {
            dA = dot4((int)lo[k], (int)xa[mm][k], dA);
            dB = dot4((int)hi[k], (int)xb[mm][k], dB);
            dA2 = dot4((int)lo[k], (int)ya[mm][k], dA2);
            dB2 = dot4((int)hi[k], (int)yb[mm][k], dB2);
          }
          const float c = q4k_pair(d, dmin, scA, scB, mnA, mnB, de[mm], ss[mm], dA, dA2, dB, dB2);
          res[j][mm] = rsum16(active ? c : 0.f);
        }
      }
      // The slot is consumed: refill it with the group D iterations ahead (unconditionally).
      Q4KX_LOAD(s, Q4KX_GRP(it + D));
      if (it >= niter) break;

      const int row = grp * RW + team;
      float *hb = hbuf + ((it / CG) & 1) * (MM * 32);
      if (wpt <= 1) {
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
            if (a.out && m0 + mm < a.M) a.out[(int64_t)(m0 + mm) * a.N + row] = y;
            if (AOUT) hb[mm * 32 + (row & 31)] = y;
          }
        }
      } else {
        // Team of wpt waves: 16-lane row sums through LDS, added in row order.
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
          const int r2 = grp * RW + tm;
          if (r2 < a.N) {
            float y = tot[0];
            if (GATED) y = gate_act(tot[0], a.act) * tot[NW - 1];
            if (a.out && m0 + mm < a.M) a.out[(int64_t)(m0 + mm) * a.N + r2] = y;
            if (AOUT) hb[mm * 32 + (r2 & 31)] = y;
          }
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
  }
#undef Q4KX_GRP
}

#undef Q4KX_LOAD

// ---------------------------------------------------------------------------
// Launch
// ---------------------------------------------------------------------------

// Team geometry: P = K/64 lanes per row; TP = 16, 32 or 64 when P fits a wave, else a
// multiple of 64 (up to 512); RW = teams per 512-lane workgroup.
static bool q4kx_geom(int64_t K, int *P, int *TP, int *RW) {
  if (K % 256 || K > 32768) return false;
  *P = (int)(K / 64);
  if (*P <= 16)
    *TP = 16;
  else if (*P <= 32)
    *TP = 32;
  else
    *TP = (*P + 63) & ~63;
  *RW = *TP >= 512 ? 1 : 512 / *TP;
  return true;
}

static int mm_of(int64_t M) { return M >= 3 ? 4 : (int)M; }

static size_t q4kx_lds(int MM, int64_t K, int TP, int RW, bool gated, bool xin, bool aout) {
  size_t b = xin ? (size_t)q4kx_act_lds(MM, K) : 0;
  if (TP > 64) b += 2 * 4 * (size_t)(RW * (TP >> 4) * (gated ? 2 : 1) * MM);
  if (aout) b += 2 * 4 * 32 * (size_t)MM;
  return b;
}

bool q4kx_ok(int64_t M, int64_t N, int64_t K, const void *w0, const void *w1, const void *x) {
  int P, TP, RW;
  if (M < 1 || M > kGemvMaxRows || !q4kx_geom(K, &P, &TP, &RW)) return false;
  if (N > INT32_MAX / 2 || N * (K / 256 * 144) > UINT32_MAX) return false;
  if (((uintptr_t)w0 & 15) || (w1 && ((uintptr_t)w1 & 15)) || ((uintptr_t)x & 15)) return false;
  return q4kx_lds(mm_of(M), K, TP, RW, w1 != nullptr, true, true) <= 160 * 1024;
}

template <int MM, bool GATED, int D, bool XIN, bool AOUT>
static int run_q4kx(const Q4kxArgs &a, hipStream_t s) {
  auto *kern = &gemv_q4kx_kernel<MM, GATED, D, XIN, AOUT>;
  const size_t lds = q4kx_lds(MM, a.K, a.TP, a.RW, GATED, XIN, AOUT);
  if (lds > 64 * 1024) {
    static bool attr_done = false;
    if (!attr_done) {
      if (hipFuncSetAttribute(reinterpret_cast<const void *>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                              160 * 1024) != hipSuccess)
        return fail(HQ_EUNSUPPORTED, "gemv_q4kx", "LDS %zu bytes not available", lds);
      attr_done = true;
    }
  }
  const int ngroups = (a.N + a.RW - 1) / a.RW;
  const int units = AOUT ? (ngroups + 32 / a.RW - 1) / (32 / a.RW) : ngroups;
  // Two persistent workgroups per CU, one row group in flight per wave: measured faster
  // than deeper per-wave prefetch (more loads per wave) or more workgroups.
  const int cap = device_cus() * 2;
  dim3 grid((unsigned)(units < cap ? units : cap), (unsigned)cdiv(a.M, MM));
  kern<<<grid, a.TP * a.RW, lds, s>>>(a);
  return check_launch(GATED ? "gemv_q4k_gated" : "gemv_q4kx");
}

template <bool GATED, bool XIN, bool AOUT>
static int dispatch_q4kx(const Q4kxArgs &a, hipStream_t s) {
  const int MMc = mm_of(a.M);
  if (MMc == 1) return run_q4kx<1, GATED, 1, XIN, AOUT>(a, s);
  if (MMc == 2) return run_q4kx<2, GATED, 1, XIN, AOUT>(a, s);
  return run_q4kx<4, GATED, 1, XIN, AOUT>(a, s);
}

static int q4kx_setup(Q4kxArgs &a, int64_t M, int64_t N, int64_t K, const char *call) {
  if (!q4kx_geom(K, &a.P, &a.TP, &a.RW) || N > INT32_MAX / 2 || M > 65535 || N * (K / 256 * 144) > UINT32_MAX)
    return fail(HQ_EUNSUPPORTED, call, "K=%lld N=%lld", (long long)K, (long long)N);
  a.x = nullptr;
  a.ain = nullptr;
  a.w0 = a.w1 = nullptr;
  a.out = nullptr;
  a.aout = nullptr;
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.row_bytes = K / 256 * 144;
  a.in_q2 = act_q2_off(M, K);
  a.in_d = act_d_off(M, K);
  a.in_s = act_s_off(M, K);
  a.out_q2 = act_q2_off(M, N);
  a.out_d = act_d_off(M, N);
  a.out_s = act_s_off(M, N);
  a.act = 0;
  return 0;
}

int launch_gemv_q4kx(const float *x, const void *w0, const void *w1, float *out, int64_t M, int64_t N, int64_t K,
                     int act, hipStream_t s) {
  Q4kxArgs a;
  if (int rc = q4kx_setup(a, M, N, K, "gemv_q4kx")) return rc;
  a.x = x;
  a.w0 = static_cast<const uint8_t *>(w0);
  a.w1 = static_cast<const uint8_t *>(w1);
  a.out = out;
  a.act = act;
  return w1 ? dispatch_q4kx<true, true, false>(a, s) : dispatch_q4kx<false, true, false>(a, s);
}

int launch_gemv_q4kx_act(const void *act_in, const void *w, float *out, int64_t M, int64_t N, int64_t K,
                         hipStream_t s) {
  Q4kxArgs a;
  if (int rc = q4kx_setup(a, M, N, K, "gemv_q4kx")) return rc;
  a.ain = static_cast<const uint8_t *>(act_in);
  a.w0 = static_cast<const uint8_t *>(w);
  a.out = out;
  return dispatch_q4kx<false, false, false>(a, s);
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
  if (dt == Q4_K && q4kx_ok(M, N, K, wg, wu, x)) return launch_gemv_q4kx(x, wg, wu, out, M, N, K, act, s);
  float *g = static_cast<float *>(ws);
  float *u = reinterpret_cast<float *>(static_cast<char *>(ws) + al256(4 * M * N));
  void *inner = static_cast<char *>(ws) + 2 * al256(4 * M * N);
  if (int rc = launch_matmul_q(x, wg, g, M, N, K, dt, inner, s)) return rc;
  if (int rc = launch_matmul_q(x, wu, u, M, N, K, dt, inner, s)) return rc;
  gated_epilogue_kernel<<<(unsigned)cdiv(M * N, 256), 256, 0, s>>>(g, u, out, M * N, act);
  return check_launch("gated_epilogue");
}

// The two-launch MLP applies: Q4_K, M <= 8, aligned, I a multiple of 256 (the down
// projection's K) and the gate/up workgroup's teams tile 32-row chunks.
static bool mlp_fused_ok(int64_t M, int64_t H, int64_t I, int dt, const void *wg, const void *wu, const void *wd,
                         const float *x) {
  int P, TP, RW;
  if (dt != Q4_K || I % 256 || !q4kx_ok(M, I, H, wg, wu, x) || !q4kx_ok(M, H, I, wd, nullptr, x)) return false;
  if (!q4kx_geom(H, &P, &TP, &RW) || 32 % RW) return false;
  return q4kx_geom(I, &P, &TP, &RW);
}

size_t mlp_q_ws_bytes(int64_t M, int64_t H, int64_t I, int dt) {
  if (M <= 0 || H <= 0 || I <= 0 || H % 32 || I % 32) return 0;
  const size_t fused = (size_t)act_bytes(M, I);
  const size_t unfused =
      (size_t)al256(4 * M * I) + std::max(matmul_q_gated_ws_bytes(M, I, H, dt), matmul_q_ws_bytes(M, H, I, dt));
  return std::max(fused, unfused);
}

int launch_mlp_q(const float *x, const void *wg, const void *wu, const void *wd, float *out, int64_t M, int64_t H,
                 int64_t I, int dt, int act, void *ws, hipStream_t s) {
  if (mlp_fused_ok(M, H, I, dt, wg, wu, wd, x)) {
    // Launch 1: gated gate/up on x, output quantized straight into ws (act layout of (M, I)).
    Q4kxArgs a;
    if (int rc = q4kx_setup(a, M, I, H, "mlp_q")) return rc;
    a.x = x;
    a.w0 = static_cast<const uint8_t *>(wg);
    a.w1 = static_cast<const uint8_t *>(wu);
    a.aout = static_cast<uint8_t *>(ws);
    a.act = act;
    if (int rc = dispatch_q4kx<true, true, true>(a, s)) return rc;
    // Launch 2: down projection on the prepared h.
    return launch_gemv_q4kx_act(ws, wd, out, M, H, I, s);
  }
  float *h = static_cast<float *>(ws);
  void *inner = static_cast<char *>(ws) + al256(4 * M * I);
  if (int rc = launch_matmul_q_gated(x, wg, wu, h, M, I, H, dt, act, inner, s)) return rc;
  return launch_matmul_q(h, wd, out, M, H, I, dt, inner, s);
}

}  // namespace hq
