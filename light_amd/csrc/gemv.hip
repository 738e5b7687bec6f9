// gemv.hip -- decode GEMV for GGUF weights (Q4_K, Q8_0, Q6_K) on q8_1 activations.
//
// Role: Light's matmul_q kernels for small M (kernels/cuda/matmul_q.go:44-91,
// kernels/cpu/quant_matmul.go:141-170); y[m, n] = sum_k x[m, k] * dequant(W)[n, k].
//
// Design (gfx950, wave64):
//  * x is quantized once (quantize.hip) into the planar act layout: int8 quants,
//    f32 block scales d and f32 d * sum(q).  Every product is an exact int32
//    v_dot4_i32_i8 chain over one 32-element block, scaled once in f32, so the
//    per-weight VALU work stays well under what HBM speed allows.
//  * A lane owns FIXED K positions and keeps their activations in registers for
//    the whole kernel; weight rows stream past.  Up to MM = 4 activation rows are
//    served per weight read.
//  * Q4_K (144-byte blocks, 16-byte aligned): a "team" of ceil(nb*4/16)*16 lanes
//    covers one weight row; lane = one (block, p) pair = 32 contiguous quant
//    bytes (two global_load_dwordx4) = sub-blocks 2p (low nibbles) and 2p+1
//    (high nibbles).  The 16-byte block header is fetched one dword per lane
//    and broadcast inside the block's 4-lane quad with DPP.  Partial sums are
//    reduced with DPP inside 16-lane rows and across the team in LDS.
//    Workgroups are persistent and prefetch the next rows while computing.
//  * Q8_0 (34 B) and Q6_K (210 B) blocks are only 2-byte aligned.  Each wave
//    streams its rows' raw bytes into LDS with direct global->LDS loads (two slices,
//    the next row group loading while the current one is computed), and lanes read
//    their blocks back with aligned dword reads re-aligned by v_alignbit.  The first
//    group's loads are issued before anything waits on x.  Up to K = 8192 the workgroup
//    quantizes its own F32 x rows into LDS (two lanes per 32-block), which saves the
//    separate quantize launch.
//  * Other shapes take a generic wave-per-row kernel on F32 activations built on
//    the bit-exact decoder of dequant.hip.
#include "actq.hpp"
#include "dma.hpp"
#include "decode.hpp"
#include "internal.hpp"

#include <atomic>
#include <mutex>

namespace hq {

int device_cus() {
  static std::mutex mu;
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  std::lock_guard<std::mutex> lk(mu);
  if (!cached[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// Broadcast lane k of each 4-lane quad to the whole quad (DPP quad_perm).
template <int K>
__device__ __forceinline__ uint32_t quad_bcast(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, K * 0x55, 0xF, 0xF, false);
}

// Sum over each 16-lane DPP row; the result is valid in every lane of the row.
__device__ __forceinline__ float row16_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));   // xor 1
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));   // xor 2
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));  // half mirror
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false));  // mirror
  return v;
}

// Full-wave sum via the four 16-lane row sums.
__device__ __forceinline__ float wave_sum64(float v) {
  v = row16_sum(v);
  // v_readlane: the four row sums come straight from VGPR lanes, no LDS round trips.
  const auto rl = [](float f, int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f), l)); };
  return ((rl(v, 0) + rl(v, 16)) + rl(v, 32)) + rl(v, 48);
}

__device__ __forceinline__ uint4 ld16g(const void *p) { return *reinterpret_cast<const uint4 *>(p); }
__device__ __forceinline__ uint32_t ld32(const uint8_t *p) { return *reinterpret_cast<const uint32_t *>(p); }

// Sum of the four signed bytes of each of n dwords.
__device__ __forceinline__ int byte_sum(const int *v, int n) {
  int s = 0;
  for (int i = 0; i < n; i++) s = dot4(v[i], 0x01010101, s);
  return s;
}

// ---------------------------------------------------------------------------
// Q4_K
// ---------------------------------------------------------------------------
struct Q4kArgs {
  const uint8_t *act;  // planar two-level activations
  const uint8_t *w;
  float *out;
  int M, N, K, P, TP;  // P = pairs per row (nb * 4), TP = team lanes (P rounded up to 16)
  int64_t row_bytes, q2_off, d_off, s_off;
};

template <int R, int MM, bool PF>
__global__ __launch_bounds__(512) void gemv_q4k_kernel(Q4kArgs a) {
  __shared__ float part[512];
  const int t = threadIdx.x;
  const int RW = blockDim.x / a.TP;  // row teams per workgroup
  const int team = t / a.TP, u = t - team * a.TP;
  const bool active = u < a.P;
  const int uu = active ? u : 0;
  const int b = uu >> 2, p = uu & 3;
  const int qoff = b * 144 + 16 + p * 32, hoff = b * 144 + 4 * p;
  const int rows_per_group = RW * R;
  const int ngroups = (a.N + rows_per_group - 1) / rows_per_group;
  const int m0 = blockIdx.y * MM;

  uint4 q0[R], q1[R];
  uint32_t hd[R];
  auto load = [&](int grp, uint4 (&x0)[R], uint4 (&x1)[R], uint32_t (&h)[R]) {
#pragma unroll
    for (int r = 0; r < R; r++) {
      int row = grp * rows_per_group + r * RW + team;
      row = row < a.N ? row : a.N - 1;
      const uint8_t *rp = a.w + (int64_t)row * a.row_bytes;
      if (active) {
        x0[r] = ld16g(rp + qoff);
        x1[r] = ld16g(rp + qoff + 16);
        h[r] = ld32(rp + hoff);
      } else {
        x0[r] = x1[r] = make_uint4(0, 0, 0, 0);
        h[r] = 0;
      }
    }
  };
  int g = blockIdx.x;
  if (g < ngroups) load(g, q0, q1, hd);

  // Activations of this lane's two sub-blocks (both levels), for MM rows of x.
  const int ja = b * 8 + 2 * p;
  int xa[MM][8], xb[MM][8], ya[MM][8], yb[MM][8];
  float4 de[MM];  // (dA, eA, dB, eB)
  float2 ss[MM];  // block sums of x
#pragma unroll
  for (int mm = 0; mm < MM; mm++) {
    const int m = m0 + mm < a.M ? m0 + mm : a.M - 1;
    const int64_t blk = (int64_t)m * (a.K / 32) + ja;
    const uint4 *xs = reinterpret_cast<const uint4 *>(a.act + blk * 32);
    const uint4 *x2 = reinterpret_cast<const uint4 *>(a.act + a.q2_off + blk * 32);
    const uint4 v0 = xs[0], v1 = xs[1], v2 = xs[2], v3 = xs[3];
    const uint4 u0 = x2[0], u1 = x2[1], u2 = x2[2], u3 = x2[3];
    const int A[8] = {(int)v0.x, (int)v0.y, (int)v0.z, (int)v0.w, (int)v1.x, (int)v1.y, (int)v1.z, (int)v1.w};
    const int B[8] = {(int)v2.x, (int)v2.y, (int)v2.z, (int)v2.w, (int)v3.x, (int)v3.y, (int)v3.z, (int)v3.w};
    const int C[8] = {(int)u0.x, (int)u0.y, (int)u0.z, (int)u0.w, (int)u1.x, (int)u1.y, (int)u1.z, (int)u1.w};
    const int D[8] = {(int)u2.x, (int)u2.y, (int)u2.z, (int)u2.w, (int)u3.x, (int)u3.y, (int)u3.z, (int)u3.w};
#pragma unroll
    for (int k = 0; k < 8; k++) {
      xa[mm][k] = A[k];
      xb[mm][k] = B[k];
      ya[mm][k] = C[k];
      yb[mm][k] = D[k];
    }
    de[mm] = *reinterpret_cast<const float4 *>(a.act + a.d_off + 8 * blk);
    ss[mm] = *reinterpret_cast<const float2 *>(a.act + a.s_off + 4 * blk);
  }
  const bool lowj = p < 2;
  const int ka = (2 * p) & 3;
  const int lane = t & 63;
  const int hpt = a.TP >> 4;  // 16-lane rows per team

  for (; g < ngroups; g += gridDim.x) {
    uint4 n0[R], n1[R];
    uint32_t nh[R];
    if (PF && g + (int)gridDim.x < ngroups) load(g + gridDim.x, n0, n1, nh);
#pragma unroll
    for (int r = 0; r < R; r++) {
      const uint32_t h0 = quad_bcast<0>(hd[r]), h1 = quad_bcast<1>(hd[r]);
      const uint32_t h2 = quad_bcast<2>(hd[r]), h3 = quad_bcast<3>(hd[r]);
      const float d = h2f(h0 & 0xffffu), dmin = h2f(h0 >> 16);
      // 6-bit (scale, min) of sub-blocks 2p and 2p+1 (getScaleMinK4, quant/q4_k.go:83-89),
      // unpacked two at a time: bytes ka and ka+1 of each scale dword.
      const uint32_t t1 = (h1 >> (8 * ka)) & 0xffffu, t2 = (h2 >> (8 * ka)) & 0xffffu;
      const uint32_t t3 = (h3 >> (8 * ka)) & 0xffffu;
      const uint32_t scp = lowj ? (t1 & 0x3F3Fu) : ((t3 & 0x0F0Fu) | ((t1 >> 2) & 0x3030u));
      const uint32_t mnp = lowj ? (t2 & 0x3F3Fu) : (((t3 >> 4) & 0x0F0Fu) | ((t2 >> 2) & 0x3030u));
      const float scA = (float)(scp & 0xffu), scB = (float)(scp >> 8);
      const float mnA = (float)(mnp & 0xffu), mnB = (float)(mnp >> 8);
      const uint32_t qw[8] = {q0[r].x, q0[r].y, q0[r].z, q0[r].w, q1[r].x, q1[r].y, q1[r].z, q1[r].w};
      uint32_t lo[8], hi[8];
#pragma unroll
      for (int k = 0; k < 8; k++) {
        lo[k] = qw[k] & 0x0F0F0F0Fu;
        hi[k] = (qw[k] >> 4) & 0x0F0F0F0Fu;
      }
#pragma unroll
      for (int mm = 0; mm < MM; mm++) {
        int dotA = 0, dotB = 0, dotA2 = 0, dotB2 = 0;
#pragma unroll
        for (int k = 0; k < 8; k++) {
          dotA = dot4((int)lo[k], xa[mm][k], dotA);
          dotB = dot4((int)hi[k], xb[mm][k], dotB);
          dotA2 = dot4((int)lo[k], ya[mm][k], dotA2);
          dotB2 = dot4((int)hi[k], yb[mm][k], dotB2);
        }
        const float s = row16_sum(q4k_pair(d, dmin, scA, scB, mnA, mnB, de[mm], ss[mm], dotA, dotA2, dotB, dotB2));
        if ((lane & 15) == 0) part[((r * RW + team) * MM + mm) * hpt + (u >> 4)] = s;
      }
    }
    __syncthreads();
    if (t < rows_per_group * MM) {
      const int slot = t / MM, mm = t - slot * MM;
      const int r = slot / RW, tm = slot - r * RW;
      float acc = 0.f;
      for (int k = 0; k < hpt; k++) acc += part[t * hpt + k];
      const int row = g * rows_per_group + r * RW + tm;
      if (row < a.N && m0 + mm < a.M) a.out[(int64_t)(m0 + mm) * a.N + row] = acc;
    }
    __syncthreads();
    if (PF) {
#pragma unroll
      for (int r = 0; r < R; r++) {
        q0[r] = n0[r];
        q1[r] = n1[r];
        hd[r] = nh[r];
      }
    } else if (g + (int)gridDim.x < ngroups) {
      load(g + gridDim.x, q0, q1, hd);
    }
  }
}

// ---------------------------------------------------------------------------
// MoE grouped Q4_K GEMV: the Q4_K kernel above with an expert dimension
// (grid.y) and the expert's routed pairs as the rows of x (ops/moe.go:101-111):
// out[p, n] = w(p) * x[row(p)] . dequant(W[e])[n], row(p) = rpp ? p : p / topk.
// ---------------------------------------------------------------------------
struct MoeQ4kArgs {
  Q4kArgs base;  // act / w / out / N / K / P / TP / offsets; base.M = rows of x
  const int64_t *pairs;
  const int32_t *offsets;
  const float *topk_w;
  int64_t size_m, expert_bytes;
  int topk, rpp;
};

template <int R, int MM>
__global__ __launch_bounds__(512) void moe_gemv_q4k_kernel(MoeQ4kArgs ma) {
  __shared__ float part[512];
  const Q4kArgs &a = ma.base;
  const int e = blockIdx.y;
  const int seg0 = ma.offsets[e], seg1 = ma.offsets[e + 1];
  if (seg0 >= seg1) return;
  const uint8_t *wexp = a.w + (int64_t)e * ma.expert_bytes;
  const int t = threadIdx.x;
  const int RW = blockDim.x / a.TP;
  const int team = t / a.TP, u = t - team * a.TP;
  const bool active = u < a.P;
  const int uu = active ? u : 0;
  const int b = uu >> 2, p = uu & 3;
  const int qoff = b * 144 + 16 + p * 32, hoff = b * 144 + 4 * p;
  const int rows_per_group = RW * R;
  const int ngroups = (a.N + rows_per_group - 1) / rows_per_group;
  const int ja = b * 8 + 2 * p;
  const bool lowj = p < 2;
  const int ka = (2 * p) & 3;
  const int lane = t & 63;
  const int hpt = a.TP >> 4;

  for (int c0 = seg0; c0 < seg1; c0 += MM) {
    int64_t pid[MM];
    int xa[MM][8], xb[MM][8], ya[MM][8], yb[MM][8];
    float4 de[MM];
    float2 ss[MM];
#pragma unroll
    for (int mm = 0; mm < MM; mm++) {
      const int i = c0 + mm;
      int64_t pp = i < seg1 ? ma.pairs[i] : -1;
      if (pp < 0 || pp >= ma.size_m) pp = -1;
      pid[mm] = pp;
      const int64_t row = pp < 0 ? 0 : (ma.rpp ? pp : pp / ma.topk);
      const int64_t blk = row * (a.K / 32) + ja;
      const uint4 *xs = reinterpret_cast<const uint4 *>(a.act + blk * 32);
      const uint4 *x2 = reinterpret_cast<const uint4 *>(a.act + a.q2_off + blk * 32);
      const uint4 v0 = xs[0], v1 = xs[1], v2 = xs[2], v3 = xs[3];
      const uint4 w0 = x2[0], w1 = x2[1], w2 = x2[2], w3 = x2[3];
      const int A[8] = {(int)v0.x, (int)v0.y, (int)v0.z, (int)v0.w, (int)v1.x, (int)v1.y, (int)v1.z, (int)v1.w};
      const int B[8] = {(int)v2.x, (int)v2.y, (int)v2.z, (int)v2.w, (int)v3.x, (int)v3.y, (int)v3.z, (int)v3.w};
      const int C[8] = {(int)w0.x, (int)w0.y, (int)w0.z, (int)w0.w, (int)w1.x, (int)w1.y, (int)w1.z, (int)w1.w};
      const int D[8] = {(int)w2.x, (int)w2.y, (int)w2.z, (int)w2.w, (int)w3.x, (int)w3.y, (int)w3.z, (int)w3.w};
#pragma unroll
      for (int k = 0; k < 8; k++) {
        xa[mm][k] = A[k];
        xb[mm][k] = B[k];
        ya[mm][k] = C[k];
        yb[mm][k] = D[k];
      }
      de[mm] = *reinterpret_cast<const float4 *>(a.act + a.d_off + 8 * blk);
      ss[mm] = *reinterpret_cast<const float2 *>(a.act + a.s_off + 4 * blk);
    }
    for (int g = blockIdx.x; g < ngroups; g += gridDim.x) {
      uint4 q0[R], q1[R];
      uint32_t hd[R];
#pragma unroll
      for (int r = 0; r < R; r++) {
        int row = g * rows_per_group + r * RW + team;
        row = row < a.N ? row : a.N - 1;
        const uint8_t *rp = wexp + (int64_t)row * a.row_bytes;
        if (active) {
          q0[r] = ld16g(rp + qoff);
          q1[r] = ld16g(rp + qoff + 16);
          hd[r] = ld32(rp + hoff);
        } else {
          q0[r] = q1[r] = make_uint4(0, 0, 0, 0);
          hd[r] = 0;
        }
      }
#pragma unroll
      for (int r = 0; r < R; r++) {
        const uint32_t h0 = quad_bcast<0>(hd[r]), h1 = quad_bcast<1>(hd[r]);
        const uint32_t h2 = quad_bcast<2>(hd[r]), h3 = quad_bcast<3>(hd[r]);
        const float d = h2f(h0 & 0xffffu), dmin = h2f(h0 >> 16);
        const uint32_t t1 = (h1 >> (8 * ka)) & 0xffffu, t2 = (h2 >> (8 * ka)) & 0xffffu;
        const uint32_t t3 = (h3 >> (8 * ka)) & 0xffffu;
        const uint32_t scp = lowj ? (t1 & 0x3F3Fu) : ((t3 & 0x0F0Fu) | ((t1 >> 2) & 0x3030u));
        const uint32_t mnp = lowj ? (t2 & 0x3F3Fu) : (((t3 >> 4) & 0x0F0Fu) | ((t2 >> 2) & 0x3030u));
        const float scA = (float)(scp & 0xffu), scB = (float)(scp >> 8);
        const float mnA = (float)(mnp & 0xffu), mnB = (float)(mnp >> 8);
        const uint32_t qw[8] = {q0[r].x, q0[r].y, q0[r].z, q0[r].w, q1[r].x, q1[r].y, q1[r].z, q1[r].w};
        uint32_t lo[8], hi[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
          lo[k] = qw[k] & 0x0F0F0F0Fu;
          hi[k] = (qw[k] >> 4) & 0x0F0F0F0Fu;
        }
#pragma unroll
        for (int mm = 0; mm < MM; mm++) {
          int dA1 = 0, dB1 = 0, dA2 = 0, dB2 = 0;
#pragma unroll
          for (int k = 0; k < 8; k++) {
            dA1 = dot4((int)lo[k], xa[mm][k], dA1);
            dB1 = dot4((int)hi[k], xb[mm][k], dB1);
            dA2 = dot4((int)lo[k], ya[mm][k], dA2);
            dB2 = dot4((int)hi[k], yb[mm][k], dB2);
          }
          const float s = row16_sum(q4k_pair(d, dmin, scA, scB, mnA, mnB, de[mm], ss[mm], dA1, dA2, dB1, dB2));
          if ((lane & 15) == 0) part[((r * RW + team) * MM + mm) * hpt + (u >> 4)] = s;
        }
      }
      __syncthreads();
      if (t < rows_per_group * MM) {
        const int slot = t / MM, mm = t - slot * MM;
        const int r = slot / RW, tm = slot - r * RW;
        float acc = 0.f;
        for (int k = 0; k < hpt; k++) acc += part[t * hpt + k];
        const int row = g * rows_per_group + r * RW + tm;
        const int64_t pp = pid[mm];
        if (row < a.N && pp >= 0) a.out[pp * a.N + row] = acc * (ma.topk_w ? ma.topk_w[pp] : 1.f);
      }
      __syncthreads();
    }
  }
}

template <int MM>
static void run_moe_q4k(MoeQ4kArgs ma, int64_t active, hipStream_t s) {
  Q4kArgs &a = ma.base;
  const int rw = a.TP >= 256 ? 1 : 256 / a.TP;
  const int R = a.TP <= 128 ? 1 : 2;
  const int ngroups = (a.N + rw * R - 1) / (rw * R);
  // At most `active` experts have pairs: give each enough workgroups to fill the chip
  // (the workgroups of experts without pairs exit at once).
  const int64_t cap = cdiv((int64_t)device_cus() * 4, active);
  dim3 grid((unsigned)(ngroups < cap ? ngroups : cap), (unsigned)a.M /* experts */);
  if (R == 1)
    moe_gemv_q4k_kernel<1, MM><<<grid, a.TP * rw, 0, s>>>(ma);
  else
    moe_gemv_q4k_kernel<2, MM><<<grid, a.TP * rw, 0, s>>>(ma);
}

int launch_moe_gemv_q4k(const void *act, const void *w, const int64_t *pairs, const int32_t *offsets,
                        const float *topk_w, float *out, int topk, int64_t size_m, int64_t M, int64_t rows,
                        int64_t E, int64_t N, int64_t K, int rpp, hipStream_t s) {
  MoeQ4kArgs ma;
  Q4kArgs &a = ma.base;
  a.act = static_cast<const uint8_t *>(act);
  a.w = static_cast<const uint8_t *>(w);
  a.out = out;
  a.M = (int)E;  // grid.y: experts
  a.N = (int)N;
  a.K = (int)K;
  a.P = (int)(K / 256 * 4);
  a.TP = (a.P + 15) & ~15;
  a.row_bytes = K / 256 * 144;
  a.q2_off = act_q2_off(rows, K);
  a.d_off = act_d_off(rows, K);
  a.s_off = act_s_off(rows, K);
  ma.pairs = pairs;
  ma.offsets = offsets;
  ma.topk_w = topk_w;
  ma.size_m = size_m;
  ma.expert_bytes = N * a.row_bytes;
  ma.topk = topk;
  ma.rpp = rpp;
  // Pairs per expert: about M / E on average; serve up to 4 per weight pass.
  const int64_t active = M < E ? M : E;
  const int64_t avg = (M + active - 1) / active;
  if (avg <= 1)
    run_moe_q4k<1>(ma, active, s);
  else if (avg <= 2)
    run_moe_q4k<2>(ma, active, s);
  else
    run_moe_q4k<4>(ma, active, s);
  return check_launch("moe_gemv_q4k");
}

// ---------------------------------------------------------------------------
// Q8_0 / Q4_0 / Q5_0 / Q6_K: LDS-staged rows, one wave per R rows.
// ---------------------------------------------------------------------------
struct StagedArgs {
  const uint8_t *act;
  const float *x;  // XIN: F32 x (M, K), quantized by each workgroup into LDS
  const uint8_t *w;
  float *out;
  int M, N, K, nb;
  int64_t row_bytes, q2_off, d_off, s_off;
  // Row stride in w and the byte offset of the staged part within each row: row_bytes and 0,
  // except for a K part of rows too long to stage whole (then one row per group).
  int64_t row_stride, k0_bytes;
  int lds_wave;  // bytes of one LDS slice (one row group)
  int ns;        // slices per wave: row groups are loaded ns - 1 ahead
};

// NDW dwords starting at LDS byte offset o (o even), re-aligned: out[k] = bytes [o+4k, o+4k+4).
template <int NDW>
__device__ __forceinline__ void lds_unaligned(const uint8_t *lds, int o, uint32_t (&out)[NDW]) {
  const uint32_t *base = reinterpret_cast<const uint32_t *>(lds + (o & ~3));
  const uint32_t sh = (uint32_t)(o & 3) * 8;
  uint32_t w[NDW + 1];
#pragma unroll
  for (int k = 0; k <= NDW; k++) w[k] = base[k];
#pragma unroll
  for (int k = 0; k < NDW; k++) out[k] = __builtin_amdgcn_alignbit(w[k + 1], w[k], sh);
}

// Direct loads of the row group starting at row r0 into an LDS slice: ni = lds_wave / 1 KB
// loads of 1 KB, byte offsets clamped into the weight (the slice's tail past the group
// reloads valid bytes that are never read).  A group past the end issues nothing -- clamping
// it would aim every idle wave at the same last row, one L2 channel -- and the return
// value is the number of loads issued (wave-uniform), for the wait that follows.
__device__ __forceinline__ int staged_issue(const StagedArgs &a, uint8_t *slice, int64_t r0, int lane) {
  if (r0 >= a.N) return 0;
  // Loads stay inside w (N rows of row_stride): lanes past the group's bytes re-read its last
  // 16 bytes or read on into later bytes of w, landing in the slice's slack, which no dot reads.
  const int64_t total = (int64_t)a.N * a.row_stride;
  const int64_t base = r0 * a.row_stride + a.k0_bytes;
  const uint32_t dst = (uint32_t)(uintptr_t)slice;
  const int ni = a.lds_wave >> 10;
  for (int i = 0; i < ni; i++) {
    int64_t off = base + i * 1024 + lane * 16;
    off = off < total - 16 ? off : total - 16;
    dma16(a.w + off, __builtin_amdgcn_readfirstlane(dst + i * 1024));
  }
  return ni;
}

// XIN: the workgroup quantizes x rows m0 .. m0+MM-1 (clamped to M-1) into LDS at xs, in the
// act layout of an MM-row activation: q1 [MM][K] | q2 [MM][K] | (d, e) [MM][K/32] | sx
// [MM][K/32].  Two lanes per 32-block, sixteen elements each (act_quant16_fast: reciprocal
// scales, four VALU operations per element), as the Q4_K GEMV quantizes its own x.
struct ActView {
  const uint8_t *p;
  int64_t q2, d, s;  // byte offsets of q2, (d, e) and sx from p
};

__host__ __device__ constexpr int64_t staged_xin_lds(int MM, int64_t K) { return MM * (2 * K + 12 * (K / 32)); }

template <int MM>
__device__ __forceinline__ ActView staged_quantize_x(const StagedArgs &a, uint8_t *xs, int m0) {
  const int nb = a.K >> 5, ntask = MM * nb * 2;
  const int64_t q2 = (int64_t)MM * a.K, d = 2 * q2, so = d + 8 * (int64_t)MM * nb;
  for (int base = 0; base < ntask; base += 256) {
    const int t = base + (int)threadIdx.x;
    const int tc = t < ntask ? t : ntask - 1;  // ntask is even: both lanes of a block agree
    const int blk = tc >> 1, half = tc & 1, mm = MM == 1 ? 0 : blk / nb;
    const int m = m0 + mm < a.M ? m0 + mm : a.M - 1;
    const float4 *xp = reinterpret_cast<const float4 *>(a.x + (int64_t)m * a.K + (int64_t)(blk - mm * nb) * 32 + half * 16);
    float v[16];
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const float4 f = xp[r];
      v[4 * r] = f.x, v[4 * r + 1] = f.y, v[4 * r + 2] = f.z, v[4 * r + 3] = f.w;
    }
    const ActQ16 q = act_quant16_fast(v);
    if (t < ntask) {
      *reinterpret_cast<uint4 *>(xs + blk * 32 + half * 16) = make_uint4(q.q1[0], q.q1[1], q.q1[2], q.q1[3]);
      *reinterpret_cast<uint4 *>(xs + q2 + blk * 32 + half * 16) = make_uint4(q.q2[0], q.q2[1], q.q2[2], q.q2[3]);
      if (half == 0) {
        reinterpret_cast<float2 *>(xs + d)[blk] = make_float2(q.d, q.e);
        reinterpret_cast<float *>(xs + so)[blk] = q.sum;
      }
    }
  }
  __syncthreads();
  return ActView{xs, q2, d, so};
}

// Bit j of n (j < 4) to bit 0 of byte j.
__device__ __forceinline__ uint32_t spread4(uint32_t n) { return (n * 0x00204081u) & 0x01010101u; }

// 32-element blocks (Q8_0, Q4_0, Q5_0): lane unit = one block.  The block's 32 weights as
// eight dwords of bytes in element order; Q4_0 / Q5_0 give the unsigned stored values
// (the offset 8 / 16 is taken off through the block sum of x).
template <int DT>
__device__ __forceinline__ void b32_quants(const uint8_t *lds, int o, uint32_t (&qd)[8]) {
  if constexpr (DT == Q8_0) {
    lds_unaligned<8>(lds, o + 2, qd);
  } else {
    uint32_t qs[4];
    lds_unaligned<4>(lds, o + (DT == Q4_0 ? 2 : 6), qs);
#pragma unroll
    for (int k = 0; k < 4; k++) {
      qd[k] = qs[k] & 0x0F0F0F0Fu;
      qd[4 + k] = (qs[k] >> 4) & 0x0F0F0F0Fu;
    }
    if constexpr (DT == Q5_0) {
      uint32_t qh[1];
      lds_unaligned<1>(lds, o + 2, qh);
#pragma unroll
      for (int k = 0; k < 8; k++) qd[k] |= spread4((qh[0] >> (4 * k)) & 15u) << 4;
    }
  }
}

template <int DT, int CPL, int R, int MM, bool XIN, bool X1>
__global__ __launch_bounds__(256) void gemv_q80_kernel(StagedArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  constexpr int BB = DT == Q8_0 ? 34 : DT == Q4_0 ? 18 : 22;
  constexpr float OFF = DT == Q8_0 ? 0.f : DT == Q4_0 ? 8.f : 16.f;
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int nwaves = gridDim.x * 4;
  const int m0 = blockIdx.y * MM;

  // The first row group's weight bytes are requested before anything waits on x.
  uint8_t *ring = smem + (threadIdx.x >> 6) * a.ns * a.lds_wave;
  const int64_t stride = (int64_t)nwaves * R;
  for (int k = 0; k < a.ns - 1; k++) staged_issue(a, ring + k * a.lds_wave, (int64_t)wave * R + k * stride, lane);
  ActView av;
  if constexpr (XIN)
    av = staged_quantize_x<MM>(a, smem + 4 * a.ns * a.lds_wave, m0);
  else
    av = ActView{a.act, a.q2_off, a.d_off, a.s_off};

  int xv[MM][CPL][8], yv[MM][CPL][8];
  float2 dx[MM][CPL];
  float ox[MM][CPL];  // OFF * (sum of the block's x)
#pragma unroll
  for (int mm = 0; mm < MM; mm++) {
    const int m = XIN ? mm : (m0 + mm < a.M ? m0 + mm : a.M - 1);
#pragma unroll
    for (int i = 0; i < CPL; i++) {
      const int bl = lane + 64 * i;
      const bool ok = bl < a.nb;
      const int64_t blk = (int64_t)m * a.nb + (ok ? bl : 0);
      const uint4 *xs = reinterpret_cast<const uint4 *>(av.p + blk * 32);
      const uint4 *x2 = reinterpret_cast<const uint4 *>(av.p + av.q2 + blk * 32);
      const uint4 v0 = xs[0], v1 = xs[1];
      const uint4 u0 = X1 ? make_uint4(0, 0, 0, 0) : x2[0], u1 = X1 ? make_uint4(0, 0, 0, 0) : x2[1];
      const int V[8] = {(int)v0.x, (int)v0.y, (int)v0.z, (int)v0.w, (int)v1.x, (int)v1.y, (int)v1.z, (int)v1.w};
      const int U[8] = {(int)u0.x, (int)u0.y, (int)u0.z, (int)u0.w, (int)u1.x, (int)u1.y, (int)u1.z, (int)u1.w};
#pragma unroll
      for (int k = 0; k < 8; k++) {
        xv[mm][i][k] = ok ? V[k] : 0;
        yv[mm][i][k] = ok ? U[k] : 0;
      }
      dx[mm][i] = ok ? reinterpret_cast<const float2 *>(av.p + av.d)[blk] : make_float2(0.f, 0.f);
      ox[mm][i] = 0.f;
      if constexpr (DT != Q8_0) ox[mm][i] = ok ? OFF * reinterpret_cast<const float *>(av.p + av.s)[blk] : 0.f;
    }
  }

  // A ring of ns LDS slices per wave, filled by direct loads ns - 1 row groups ahead.
  const int ni = a.lds_wave >> 10;
  int cur = 0;
  for (int64_t row0 = (int64_t)wave * R; row0 < a.N; row0 += stride, cur = cur + 1 == a.ns ? 0 : cur + 1) {
    const int nrows = (int)(a.N - row0 < R ? a.N - row0 : R);
    uint8_t *lds = ring + cur * a.lds_wave;
    // The group ns - 1 ahead into the slice computed last, then wait for this group: the
    // loads issued after it are the later groups' (those before the end).  Row stores in
    // between only make the wait stricter.
    const int prev = cur == 0 ? a.ns - 1 : cur - 1;
    staged_issue(a, ring + prev * a.lds_wave, row0 + (a.ns - 1) * stride, lane);
    int newer = 0;
    for (int k = 1; k < a.ns; k++) newer += row0 + k * stride < a.N ? ni : 0;
    wait_vm_rt(newer);
#pragma unroll
    for (int r = 0; r < R; r++) {
      if (r >= nrows) break;
      float acc[MM];
#pragma unroll
      for (int mm = 0; mm < MM; mm++) acc[mm] = 0.f;
#pragma unroll
      for (int i = 0; i < CPL; i++) {
        const int bl = lane + 64 * i;
        const int o = r * (int)a.row_bytes + BB * (bl < a.nb ? bl : 0);
        const float d = h2f(*reinterpret_cast<const uint16_t *>(lds + o));
        uint32_t qd[8];
        b32_quants<DT>(lds, o, qd);
#pragma unroll
        for (int mm = 0; mm < MM; mm++) {
          int dot = 0, dot2 = 0;
#pragma unroll
          for (int k = 0; k < 8; k++) {
            dot = dot4((int)qd[k], xv[mm][i][k], dot);
            if constexpr (!X1) dot2 = dot4((int)qd[k], yv[mm][i][k], dot2);
          }
          float v = X1 ? dx[mm][i].x * (float)dot : dx[mm][i].x * (float)dot + dx[mm][i].y * (float)dot2;
          if constexpr (DT != Q8_0) v -= ox[mm][i];
          acc[mm] += d * v;
        }
      }
#pragma unroll
      for (int mm = 0; mm < MM; mm++) {
        const float s = wave_sum64(acc[mm]);
        if (lane == 0 && m0 + mm < a.M) a.out[(int64_t)(m0 + mm) * a.N + row0 + r] = s;
      }
    }
  }
  wait_vm<0>();
}

// Q6_K lane unit = (block b, l8): half h = l8 >> 2, l0 = (l8 & 3) * 8; the unit covers
// elements h*128 + g*32 + l0 + [0, 8) for g = 0..3 (quant/q6_k.go:18-27).
template <int CPL, int R, int MM, bool XIN, bool X1>
__global__ __launch_bounds__(256) void gemv_q6k_kernel(StagedArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int nwaves = gridDim.x * 4;
  const int m0 = blockIdx.y * MM;
  const int units = a.nb * 8;

  // The first row group's weight bytes are requested before anything waits on x.
  uint8_t *ring = smem + (threadIdx.x >> 6) * a.ns * a.lds_wave;
  const int64_t stride = (int64_t)nwaves * R;
  for (int k = 0; k < a.ns - 1; k++) staged_issue(a, ring + k * a.lds_wave, (int64_t)wave * R + k * stride, lane);
  ActView av;
  if constexpr (XIN)
    av = staged_quantize_x<MM>(a, smem + 4 * a.ns * a.lds_wave, m0);
  else
    av = ActView{a.act, a.q2_off, a.d_off, a.s_off};

  // Per (row of x, unit, 32-block g): the quants of both levels, -32 * their sums (the Q6_K
  // offset, folded into the dot chains' start) and d / 254 (the second level's step e is
  // d / 254 to within an ulp, so d q1 + e q2 = (d / 254) (254 q1 + q2)).
  int xv[MM][CPL][8], yv[MM][CPL][8];
  float fs[MM][CPL][4];
  int s32[MM][CPL][4], t32[MM][CPL][4];
#pragma unroll
  for (int i = 0; i < CPL; i++) {
    const int un = lane + 64 * i;
    const bool ok = un < units;
    const int uu = ok ? un : 0, bl = uu >> 3, l8 = uu & 7, h = l8 >> 2, l0 = (l8 & 3) * 8;
#pragma unroll
    for (int mm = 0; mm < MM; mm++) {
      const int m = XIN ? mm : (m0 + mm < a.M ? m0 + mm : a.M - 1);
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const int64_t blk = (int64_t)m * (a.K / 32) + bl * 8 + h * 4 + g;
        const uint2 v = *reinterpret_cast<const uint2 *>(av.p + blk * 32 + l0);
        const uint2 v2 = X1 ? make_uint2(0, 0) : *reinterpret_cast<const uint2 *>(av.p + av.q2 + blk * 32 + l0);
        xv[mm][i][2 * g] = ok ? (int)v.x : 0;
        xv[mm][i][2 * g + 1] = ok ? (int)v.y : 0;
        yv[mm][i][2 * g] = ok ? (int)v2.x : 0;
        yv[mm][i][2 * g + 1] = ok ? (int)v2.y : 0;
        const float dxb = reinterpret_cast<const float2 *>(av.p + av.d)[blk].x;
        fs[mm][i][g] = ok ? (X1 ? dxb : dxb * (1.0f / 254.0f)) : 0.f;
        s32[mm][i][g] = -32 * byte_sum(&xv[mm][i][2 * g], 2);
        t32[mm][i][g] = -32 * byte_sum(&yv[mm][i][2 * g], 2);
      }
    }
  }

  // A ring of ns LDS slices per wave, filled by direct loads ns - 1 row groups ahead.
  const int ni = a.lds_wave >> 10;
  int cur = 0;
  for (int64_t row0 = (int64_t)wave * R; row0 < a.N; row0 += stride, cur = cur + 1 == a.ns ? 0 : cur + 1) {
    const int nrows = (int)(a.N - row0 < R ? a.N - row0 : R);
    uint8_t *lds = ring + cur * a.lds_wave;
    // The group ns - 1 ahead into the slice computed last, then wait for this group: the
    // loads issued after it are the later groups' (those before the end).  Row stores in
    // between only make the wait stricter.
    const int prev = cur == 0 ? a.ns - 1 : cur - 1;
    staged_issue(a, ring + prev * a.lds_wave, row0 + (a.ns - 1) * stride, lane);
    int newer = 0;
    for (int k = 1; k < a.ns; k++) newer += row0 + k * stride < a.N ? ni : 0;
    wait_vm_rt(newer);
#pragma unroll
    for (int r = 0; r < R; r++) {
      if (r >= nrows) break;
      float acc[MM];
#pragma unroll
      for (int mm = 0; mm < MM; mm++) acc[mm] = 0.f;
#pragma unroll
      for (int i = 0; i < CPL; i++) {
        const int un = lane + 64 * i;
        const int uu = un < units ? un : 0, bl = uu >> 3, l8 = uu & 7, h = l8 >> 2, l0 = (l8 & 3) * 8;
        const int o = r * (int)a.row_bytes + 210 * bl;
        uint32_t A[2], B[2], H[2], S[2];
        lds_unaligned<2>(lds, o + h * 64 + l0, A);
        lds_unaligned<2>(lds, o + h * 64 + 32 + l0, B);
        lds_unaligned<2>(lds, o + 128 + h * 32 + l0, H);
        lds_unaligned<2>(lds, o + 192 + h * 8, S);
        const float d = h2f(*reinterpret_cast<const uint16_t *>(lds + o + 208));
        // Sub-block scales 2g + is (int8): bytes is, is + 2 of S[0] (g = 0, 1) and of S[1].
        const int is = l0 >> 4;
        int sc[4];
#pragma unroll
        for (int g = 0; g < 4; g++) sc[g] = __builtin_amdgcn_sbfe((int)S[g >> 1], 8 * (2 * (g & 1) + is), 8);
        // 6-bit quants q = low nibble | 2 high bits << 4, one byte each.
        uint32_t qv[4][2];
#pragma unroll
        for (int k = 0; k < 2; k++) {
          const uint32_t hk = H[k];
          qv[0][k] = (A[k] & 0x0F0F0F0Fu) | ((hk << 4) & 0x30303030u);
          qv[1][k] = (B[k] & 0x0F0F0F0Fu) | ((hk << 2) & 0x30303030u);
          qv[2][k] = ((A[k] >> 4) & 0x0F0F0F0Fu) | (hk & 0x30303030u);
          qv[3][k] = ((B[k] >> 4) & 0x0F0F0F0Fu) | ((hk >> 2) & 0x30303030u);
        }
#pragma unroll
        for (int mm = 0; mm < MM; mm++) {
          float v = 0.f;
#pragma unroll
          for (int g = 0; g < 4; g++) {
            // sum (q - 32) x over the 8 elements, both levels: |dot| <= 8 * 32 * 127, so
            // 254 dot + dot2 stays below 2^23 and sc * (254 dot + dot2) below 2^31.
            int dot = dot4((int)qv[g][0], xv[mm][i][2 * g], s32[mm][i][g]);
            dot = dot4((int)qv[g][1], xv[mm][i][2 * g + 1], dot);
            int c;
            if constexpr (X1) {
              c = __mul24(sc[g], dot);
            } else {
              int dot2 = dot4((int)qv[g][0], yv[mm][i][2 * g], t32[mm][i][g]);
              dot2 = dot4((int)qv[g][1], yv[mm][i][2 * g + 1], dot2);
              c = __mul24(sc[g], __mul24(254, dot) + dot2);
            }
            v = __fmaf_rn((float)c, fs[mm][i][g], v);
          }
          acc[mm] += d * v;
        }
      }
#pragma unroll
      for (int mm = 0; mm < MM; mm++) {
        const float s = wave_sum64(acc[mm]);
        if (lane == 0 && m0 + mm < a.M) a.out[(int64_t)(m0 + mm) * a.N + row0 + r] = s;
      }
    }
  }
  wait_vm<0>();
}

// ---------------------------------------------------------------------------
// Generic fallback: F32 activations, wave per row, bit-exact decode.
// ---------------------------------------------------------------------------
template <int DT>
__global__ __launch_bounds__(256) void gemv_generic_kernel(const float *__restrict__ x, const uint8_t *__restrict__ w,
                                                           float *__restrict__ out, int64_t N, int64_t K,
                                                           int64_t row_bytes) {
  const int lane = threadIdx.x & 63;
  const int64_t nwaves = (int64_t)gridDim.x * 4;
  const float *xr = x + blockIdx.y * K;
  for (int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); row < N; row += nwaves) {
    const uint8_t *rp = w + row * row_bytes;
    float acc = 0.f;
    for (int64_t t = lane; t < K / 8; t += 64) {
      float y[8];
      decode8<DT>(rp, t, y);
#pragma unroll
      for (int j = 0; j < 8; j++) acc += y[j] * xr[8 * t + j];
    }
    acc = wave_sum64(acc);
    if (lane == 0) out[blockIdx.y * N + row] = acc;
  }
}

// ---------------------------------------------------------------------------
// Launch logic
// ---------------------------------------------------------------------------

static const int kCplSteps[] = {1, 2, 3, 4, 6, 8};

// The staged kernels quantize F32 x themselves up to this K (each workgroup re-reads x from
// L2; beyond it one quantize launch is cheaper).
static constexpr int64_t kStagedXinMaxK = 8192;

static int pick_cpl(int64_t units) {
  int64_t need = cdiv(units, 64);
  for (int c : kCplSteps)
    if (c >= need) return c;
  return 0;
}

static int64_t staged_row_bytes(int dt, int64_t K) { return K / block_info(dt).elems * block_info(dt).bytes; }

// The int8 GEMV applies: rows are 16-byte multiples, w is 16-byte aligned and K fits.
bool gemv_fast_ok(int dt, int64_t K, const void *w) {
  if (((uintptr_t)w & 15) != 0 || K % 32) return false;
  BlockInfo bi = block_info(dt);
  if (!bi.elems || K % bi.elems) return false;
  int64_t nb = K / bi.elems, row_bytes = nb * bi.bytes;
  if (row_bytes % 16) return false;
  if (dt == Q4_K || dt == Q5_K) return nb <= 128;  // team of <= 512 lanes
  if (!pick_cpl(dt == Q6_K ? nb * 8 : nb)) return false;
  return staged_row_bytes(dt, K) + 16 <= 16384;  // one row must fit a wave's LDS slice
}

template <int R, int MM, bool PF>
static void run_q4k(const Q4kArgs &a, int rw, int cap, hipStream_t s) {
  int ngroups = (a.N + rw * R - 1) / (rw * R);
  int grid = ngroups < cap ? ngroups : cap;
  dim3 g((unsigned)grid, (unsigned)cdiv(a.M, MM));
  gemv_q4k_kernel<R, MM, PF><<<g, a.TP * rw, 0, s>>>(a);
}

template <int MM>
static void dispatch_q4k(Q4kArgs a, hipStream_t s) {
  const int rw = a.TP >= 256 ? 1 : 256 / a.TP;
  const int cus = device_cus();
  if (a.TP <= 128)
    run_q4k<1, MM, true>(a, rw, cus * 4, s);
  else
    run_q4k<2, MM, false>(a, rw, cus * 2, s);
}

template <typename K>
static void allow_big_lds(K *kern) {
  (void)hipFuncSetAttribute(reinterpret_cast<const void *>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            160 * 1024);
}

// Bytes of one LDS slice: R rows (+16 bytes read past the last block), whole KB.
static int staged_slice(int R, int64_t row_bytes) { return (int)((R * row_bytes + 16 + 1023) & ~(int64_t)1023); }

template <int CPL, int R, int MM, bool XIN, bool X1>
static void run_staged_x(int dt, StagedArgs a, int ns, hipStream_t s) {
  // ns slices per wave; XIN adds the workgroup's quantized x rows.
  a.lds_wave = staged_slice(R, a.row_bytes);
  a.ns = ns;
  const int lds = 4 * ns * a.lds_wave + (XIN ? (int)staged_xin_lds(MM, a.K) : 0);
  static std::atomic<bool> attr_done{false};  // (idempotent: racing callers both set it)
  if (!attr_done.load(std::memory_order_acquire)) {
    allow_big_lds(&gemv_q80_kernel<Q8_0, CPL, R, MM, XIN, X1>);
    allow_big_lds(&gemv_q80_kernel<Q4_0, CPL, R, MM, XIN, X1>);
    allow_big_lds(&gemv_q80_kernel<Q5_0, CPL, R, MM, XIN, X1>);
    allow_big_lds(&gemv_q6k_kernel<CPL, R, MM, XIN, X1>);
    attr_done.store(true, std::memory_order_release);
  }
  const int per_cu = (160 * 1024) / lds;
  // At least two row groups per wave where N allows (the workgroup's x quantization and the
  // activation set-up are paid once per workgroup); at most two workgroups per CU.
  int64_t wgs = cdiv(cdiv(a.N, R), 4 * 2), cap = (int64_t)device_cus() * (per_cu < 2 ? per_cu : 2);
  dim3 g((unsigned)(wgs < cap ? wgs : cap), (unsigned)cdiv(a.M, MM));
  switch (dt) {
    case Q8_0: gemv_q80_kernel<Q8_0, CPL, R, MM, XIN, X1><<<g, 256, lds, s>>>(a); break;
    case Q4_0: gemv_q80_kernel<Q4_0, CPL, R, MM, XIN, X1><<<g, 256, lds, s>>>(a); break;
    case Q5_0: gemv_q80_kernel<Q5_0, CPL, R, MM, XIN, X1><<<g, 256, lds, s>>>(a); break;
    default: gemv_q6k_kernel<CPL, R, MM, XIN, X1><<<g, 256, lds, s>>>(a); break;
  }
}

// Rows of at least kStagedX1MinK elements take single-level activations (q1 alone, exactly
// q8_1), as the Q4_K / Q5_K / int4 GEMVs do from the same length: the second level's loads
// and dots are skipped.
constexpr int64_t kStagedX1MinK = 4096;
// (Three or more units per lane means more than 128 units, i.e. K > 4096: those widths
// exist only with one level.)
template <int CPL, int R, int MM, bool XIN>
static void run_staged(int dt, StagedArgs a, int ns, hipStream_t s) {
  if constexpr (CPL > 2) {
    run_staged_x<CPL, R, MM, XIN, true>(dt, a, ns, s);
  } else {
    if (a.K >= kStagedX1MinK)
      run_staged_x<CPL, R, MM, XIN, true>(dt, a, ns, s);
    else
      run_staged_x<CPL, R, MM, XIN, false>(dt, a, ns, s);
  }
}

template <int CPL, int MM, bool XIN>
static void run_staged_r(int dt, StagedArgs a, hipStream_t s) {
  // Two slices per wave of up to four rows each.  (Four one-row slices, three groups in
  // flight per wave, measured slower on every shape: per-row overheads outweigh the depth.)
  if (4 * a.row_bytes + 16 <= 8192)
    run_staged<CPL, 4, MM, XIN>(dt, a, 2, s);
  else if (2 * a.row_bytes + 16 <= 8192)
    run_staged<CPL, 2, MM, XIN>(dt, a, 2, s);
  else
    run_staged<CPL, 1, MM, XIN>(dt, a, 2, s);
}

// Q6_K holds 16 activation registers per unit and row of x: wide rows (CPL >= 6)
// serve one row of x per pass.
template <int CPL, int MM, bool XIN>
static void run_staged_c(int dt, StagedArgs a, hipStream_t s) {
  if constexpr (CPL >= 6 && MM > 1) {
    if (dt == Q6_K) return run_staged_r<CPL, 1, XIN>(dt, a, s);
  }
  run_staged_r<CPL, MM, XIN>(dt, a, s);
}

// XIN serves K <= kStagedXinMaxK only, so CPL <= 4 there.
template <int MM, bool XIN>
static void run_staged_m(int dt, StagedArgs a, int cpl, hipStream_t s) {
  switch (cpl) {
    case 1: run_staged_c<1, MM, XIN>(dt, a, s); break;
    case 2: run_staged_c<2, MM, XIN>(dt, a, s); break;
    case 3: run_staged_c<3, MM, XIN>(dt, a, s); break;
    case 4: run_staged_c<4, MM, XIN>(dt, a, s); break;
    default:
      if constexpr (!XIN) {
        if (cpl == 6)
          run_staged_c<6, MM, XIN>(dt, a, s);
        else
          run_staged_c<8, MM, XIN>(dt, a, s);
      }
  }
}

// The staged formats (Q8_0, Q4_0, Q5_0, Q6_K) on prepared activations (act != NULL) or on
// F32 x quantized inside the kernel (x != NULL, K <= kStagedXinMaxK).
static int launch_staged(const void *act, const float *x, const uint8_t *w, float *out, int64_t M, int64_t N,
                         int64_t K, int dt, hipStream_t s) {
  StagedArgs a;
  a.act = static_cast<const uint8_t *>(act);
  a.x = x;
  a.w = w;
  a.out = out;
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.nb = (int)(K / block_info(dt).elems);
  a.row_bytes = staged_row_bytes(dt, K);
  a.row_stride = a.row_bytes;
  a.k0_bytes = 0;
  a.q2_off = act_q2_off(M, K);
  a.d_off = act_d_off(M, K);
  a.s_off = act_s_off(M, K);
  a.lds_wave = 0;
  a.ns = 2;
  const int MMc = M >= 3 ? 4 : (int)M;
  int cpl = pick_cpl(dt == Q6_K ? (int64_t)a.nb * 8 : a.nb);
  // Q6_K keeps 16 registers of activations per unit and row of x: cap MM at 2.
  int mm = dt == Q6_K && MMc > 2 ? 2 : MMc;
  if (x) {
    if (mm == 1)
      run_staged_m<1, true>(dt, a, cpl, s);
    else if (mm == 2)
      run_staged_m<2, true>(dt, a, cpl, s);
    else
      run_staged_m<4, true>(dt, a, cpl, s);
  } else {
    if (mm == 1)
      run_staged_m<1, false>(dt, a, cpl, s);
    else if (mm == 2)
      run_staged_m<2, false>(dt, a, cpl, s);
    else
      run_staged_m<4, false>(dt, a, cpl, s);
  }
  return check_launch(dt == Q6_K ? "gemv_q6k" : "gemv_q80");
}

// Rows too long to stage whole (a Q6_K row of K = 53248 is 43,680 bytes; a slice holds at most
// 16 KB): K parts of whole 8-block groups (16-byte aligned in every row), each staged one row
// per group on the full row stride, for one x row at a time; the parts' outputs are summed.
// Every part is longer than 4088 bytes, so the launcher's row-group choice is one row
// (a group of several rows would need them contiguous).
static bool staged_plan(int dt, int64_t nb, int64_t *size, int *parts) {
  const BlockInfo bi = block_info(dt);
  const int64_t upb = dt == Q6_K ? 8 : 1;  // lane units per block; at most 512 units per row part
  const int64_t bmax = std::min<int64_t>((16384 - 16) / bi.bytes, 512 / upb) / 8 * 8;
  if (bmax < 8 || nb % 8) return false;
  const int p = (int)cdiv(nb, bmax);
  if (p < 2 || p > 64) return false;
  const int64_t sz = cdiv(cdiv(nb, p), 8) * 8, last = nb - (p - 1) * sz;
  if (sz > bmax || last <= 0 || last * bi.bytes <= 4088 || sz * bi.bytes <= 4088) return false;
  *size = sz;
  *parts = p;
  return true;
}

bool staged_parts_ok(int64_t M, int64_t N, int64_t K, int dt, const void *w, const void *x) {
  if ((dt != Q8_0 && dt != Q4_0 && dt != Q5_0 && dt != Q6_K) || M < 1 || M > kGemvMaxRows || N < 1 ||
      N > INT32_MAX || K <= 0 || K > INT32_MAX)
    return false;
  if (((uintptr_t)w & 15) || ((uintptr_t)x & 15)) return false;
  const BlockInfo bi = block_info(dt);
  if (K % bi.elems || gemv_fast_ok(dt, K, w)) return false;
  const int64_t nb = K / bi.elems;
  if ((nb * bi.bytes) % 16) return false;
  int64_t sz;
  int p;
  return staged_plan(dt, nb, &sz, &p);
}

int launch_staged_parts(const void *act, const void *w, float *out, float *tmp, int64_t M, int64_t N, int64_t K,
                        int dt, hipStream_t s) {
  const BlockInfo bi = block_info(dt);
  const int64_t nb = K / bi.elems, full = nb * bi.bytes;
  int64_t sz;
  int parts;
  if (!staged_plan(dt, nb, &sz, &parts)) return fail(HQ_EUNSUPPORTED, "gemv", "K=%lld", (long long)K);
  const int64_t q2 = act_q2_off(M, K), d = act_d_off(M, K), so = act_s_off(M, K);
  for (int64_t m = 0; m < M; m++) {
    for (int i = 0; i < parts; i++) {
      const int64_t b0 = i * sz, nbp = std::min<int64_t>(sz, nb - b0), e0 = m * K + b0 * bi.elems;
      StagedArgs a;
      a.act = static_cast<const uint8_t *>(act) + e0;
      a.x = nullptr;
      a.w = static_cast<const uint8_t *>(w);
      a.out = (i ? tmp : out) + m * N;
      a.M = 1;
      a.N = (int)N;
      a.K = (int)(nbp * bi.elems);
      a.nb = (int)nbp;
      a.row_bytes = nbp * bi.bytes;
      a.row_stride = full;
      a.k0_bytes = b0 * bi.bytes;
      a.q2_off = q2;                      // q2 base: act + q2 + e0
      a.d_off = d + 8 * (e0 / 32) - e0;   // (d, e) base
      a.s_off = so + 4 * (e0 / 32) - e0;  // sx base
      a.lds_wave = 0;
      a.ns = 2;
      run_staged_m<1, false>(dt, a, pick_cpl(dt == Q6_K ? nbp * 8 : nbp), s);
      if (int rc = check_launch(dt == Q6_K ? "gemv_q6k_parts" : "gemv_q80_parts")) return rc;
      if (i)
        if (int rc = launch_add_rows(out + m * N, tmp + m * N, N, s)) return rc;
    }
  }
  return HQ_OK;
}

// The same parts for M >= 2 rows of F32 x: each part's columns of x are copied out and
// quantized as an (M, kn) activation, so one launch (the launcher's row tiles) serves every
// row of x.  ws: the part's x, its act layout, then M * N floats.
size_t staged_parts_x_ws_bytes(int dt, int64_t M, int64_t N, int64_t K) {
  const BlockInfo bi = block_info(dt);
  int64_t sz = 0;
  int parts = 0;
  if (!bi.elems || K % bi.elems || !staged_plan(dt, K / bi.elems, &sz, &parts)) return 0;
  const int64_t kmax = sz * bi.elems;
  auto al = [](int64_t b) { return (b + 255) & ~(int64_t)255; };
  return (size_t)(al(4 * M * kmax) + al(act_bytes(M, kmax)) + 4 * M * N);
}

int launch_staged_parts_x(const float *x, const void *w, float *out, void *ws, int64_t M, int64_t N, int64_t K,
                          int dt, hipStream_t s) {
  const BlockInfo bi = block_info(dt);
  const int64_t nb = K / bi.elems, full = nb * bi.bytes;
  int64_t sz;
  int parts;
  if (!staged_plan(dt, nb, &sz, &parts)) return fail(HQ_EUNSUPPORTED, "gemv", "K=%lld", (long long)K);
  auto al = [](int64_t b) { return (b + 255) & ~(int64_t)255; };
  const int64_t kmax = sz * bi.elems;
  float *xb = static_cast<float *>(ws);
  uint8_t *ab = reinterpret_cast<uint8_t *>(ws) + al(4 * M * kmax);
  float *tmp = reinterpret_cast<float *>(ab + al(act_bytes(M, kmax)));
  for (int i = 0; i < parts; i++) {
    const int64_t b0 = i * sz, nbp = std::min<int64_t>(sz, nb - b0), k0 = b0 * bi.elems, kn = nbp * bi.elems;
    if (hipError_t e = hipMemcpy2DAsync(xb, (size_t)kn * 4, x + k0, (size_t)K * 4, (size_t)kn * 4, (size_t)M,
                                        hipMemcpyDeviceToDevice, s))
      return fail((int)e, "gemv", "hipMemcpy2DAsync: %s", hipGetErrorString(e));
    if (int rc = launch_quantize_act(xb, F32, ab, M, kn, s)) return rc;
    StagedArgs a;
    a.act = ab;
    a.x = nullptr;
    a.w = static_cast<const uint8_t *>(w);
    a.out = i ? tmp : out;
    a.M = (int)M;
    a.N = (int)N;
    a.K = (int)kn;
    a.nb = (int)nbp;
    a.row_bytes = nbp * bi.bytes;
    a.row_stride = full;
    a.k0_bytes = b0 * bi.bytes;
    a.q2_off = act_q2_off(M, kn);
    a.d_off = act_d_off(M, kn);
    a.s_off = act_s_off(M, kn);
    a.lds_wave = 0;
    a.ns = 2;
    const int mm = M >= 3 ? (dt == Q6_K ? 2 : 4) : (int)M;  // Q6_K: at most two rows of x per pass
    const int cpl = pick_cpl(dt == Q6_K ? nbp * 8 : nbp);
    if (mm == 1)
      run_staged_m<1, false>(dt, a, cpl, s);
    else if (mm == 2)
      run_staged_m<2, false>(dt, a, cpl, s);
    else
      run_staged_m<4, false>(dt, a, cpl, s);
    if (int rc = check_launch(dt == Q6_K ? "gemv_q6k_parts" : "gemv_q80_parts")) return rc;
    if (i)
      if (int rc = launch_add_rows(out, tmp, M * N, s)) return rc;
  }
  return HQ_OK;
}

int launch_gemv_act(const void *act, const void *wv, float *out, int64_t M, int64_t N, int64_t K, int dt,
                    hipStream_t s) {
  if (N > INT32_MAX || M > 65535 * 4 || K > INT32_MAX)
    return fail(HQ_EUNSUPPORTED, "gemv", "N, M or K too large");
  auto *w = static_cast<const uint8_t *>(wv);
  auto *xa = static_cast<const uint8_t *>(act);
  const int MMc = M >= 3 ? 4 : (int)M;
  if (dt == Q4_K && q4kx_ok(M, N, K, w, nullptr, act, Q4_K)) return launch_gemv_q4kx_act(act, w, out, M, N, K, Q4_K, s);
  if (dt == Q4_K) {
    Q4kArgs a;
    a.act = xa;
    a.w = w;
    a.out = out;
    a.M = (int)M;
    a.N = (int)N;
    a.K = (int)K;
    a.P = (int)(K / 256 * 4);
    a.TP = (a.P + 15) & ~15;
    a.row_bytes = K / 256 * 144;
    a.q2_off = act_q2_off(M, K);
    a.d_off = act_d_off(M, K);
    a.s_off = act_s_off(M, K);
    if (MMc == 1)
      dispatch_q4k<1>(a, s);
    else if (MMc == 2)
      dispatch_q4k<2>(a, s);
    else
      dispatch_q4k<4>(a, s);
    return check_launch("gemv_q4k");
  }
  // Q5_K at any M: the act-input kernel tiles M over grid.y (geometry checked at one row).
  if (dt == Q5_K && q4kx_ok(1, N, K, w, nullptr, act, Q5_K))
    return launch_gemv_q4kx_act(act, w, out, M, N, K, Q5_K, s);
  if (dt != Q8_0 && dt != Q4_0 && dt != Q5_0 && dt != Q6_K) return fail(HQ_EUNSUPPORTED, "gemv", "dtype %d", dt);
  return launch_staged(act, nullptr, w, out, M, N, K, dt, s);
}

static int launch_gemv_generic(const float *x, const void *wv, float *out, int64_t M, int64_t N, int64_t K, int dt,
                               hipStream_t s) {
  auto *w = static_cast<const uint8_t *>(wv);
  BlockInfo bi = block_info(dt);
  int64_t row_bytes = K / bi.elems * bi.bytes;
  int64_t wgs = cdiv(N, 4), cap = (int64_t)device_cus() * 16;
  dim3 grid((unsigned)(wgs < cap ? wgs : cap), (unsigned)M);
  switch (dt) {
    case Q4_K: gemv_generic_kernel<Q4_K><<<grid, 256, 0, s>>>(x, w, out, N, K, row_bytes); break;
    case Q8_0: gemv_generic_kernel<Q8_0><<<grid, 256, 0, s>>>(x, w, out, N, K, row_bytes); break;
    case Q4_0: gemv_generic_kernel<Q4_0><<<grid, 256, 0, s>>>(x, w, out, N, K, row_bytes); break;
    case Q5_0: gemv_generic_kernel<Q5_0><<<grid, 256, 0, s>>>(x, w, out, N, K, row_bytes); break;
    case Q5_K: gemv_generic_kernel<Q5_K><<<grid, 256, 0, s>>>(x, w, out, N, K, row_bytes); break;
    case Q6_K: gemv_generic_kernel<Q6_K><<<grid, 256, 0, s>>>(x, w, out, N, K, row_bytes); break;
    default: return fail(HQ_EUNSUPPORTED, "gemv", "dtype %d", dt);
  }
  return check_launch("gemv_generic");
}

// Many rows: the MFMA GEMM.  Q4_K dequantizes inside the GEMM; the other formats are
// dequantized once, bit-exact, to bf16 in the workspace and run the same GEMM on bf16 B.
// The K argument is checked where it is known (K % 64 for the 64-wide K step).
bool use_gemm(int64_t M, int dt) { return M > kGemvMaxRows; }

static bool gemm_k_ok(int64_t K) { return K % 64 == 0; }

bool matmul_act_takes_gemm(int64_t M, int64_t K, int dt) { return use_gemm(M, dt) && gemm_k_ok(K); }

static int64_t al256(int64_t b) { return (b + 255) & ~(int64_t)255; }

static size_t gemm_ws(int64_t M, int64_t N, int64_t K, int dt) {
  const size_t wb = dt == Q4_K ? 0 : (size_t)al256(N * K * 2);
  return al256((int64_t)gemm_q4k_ws_bytes(M, K)) + al256((int64_t)gemm_q4k_partial_bytes(M, N, K)) + wb;
}

size_t matmul_q_ws_bytes(int64_t M, int64_t N, int64_t K, int dt) {
  if (M <= 0 || K <= 0 || K % 32) return 0;
  if (use_gemm(M, dt) && gemm_k_ok(K)) return gemm_ws(M, N, K, dt);
  // Long Q4_K / Q5_K rows: x quantized once, then the second K half's outputs.
  if ((dt == Q4_K || dt == Q5_K) && K > 32768 && K <= 65536 && K % 256 == 0)
    return std::max((size_t)(al256(act_bytes(M, K)) + 4 * M * N), q4kx_halves_x_ws_bytes(M, N, K));
  // Long staged rows (split into K parts): the parts' outputs as well.
  if ((dt == Q8_0 || dt == Q4_0 || dt == Q5_0 || dt == Q6_K) && staged_row_bytes(dt, K) + 16 > 16384)
    return std::max((size_t)(al256(act_bytes(M, K)) + 4 * M * N), staged_parts_x_ws_bytes(dt, M, N, K));
  return (size_t)act_bytes(M, K);
}

// Long rows split into K parts (act_long_rows_ok) need the later parts' outputs.
static bool long_rows_dt(int64_t K, int dt) {
  return ((dt == Q4_K || dt == Q5_K) && K > 32768 && K <= 65536 && K % 256 == 0) ||
         ((dt == Q8_0 || dt == Q4_0 || dt == Q5_0 || dt == Q6_K) && staged_row_bytes(dt, K) + 16 > 16384);
}

size_t matmul_act_ws_bytes(int64_t M, int64_t N, int64_t K, int dt) {
  if (M <= 0 || K <= 0 || K % 32) return 0;
  if (use_gemm(M, dt) && gemm_k_ok(K)) return gemm_ws(M, N, K, dt);
  return long_rows_dt(K, dt) && N > 0 ? (size_t)(4 * M * N) : 0;
}

bool act_long_rows_ok(int64_t M, int64_t N, int64_t K, int dt, const void *w, const void *act) {
  return !matmul_act_takes_gemm(M, K, dt) &&
         (q4kx_halves_ok(M, N, K, dt, w, act) || staged_parts_ok(M, N, K, dt, w, act));
}

const char *matmul_q_kernel_name(int64_t M, int dt) { return use_gemm(M, dt) ? "matmul_q.gemm" : "matmul_q.gemv"; }

static int run_gemm(const void *src, bool from_act, const void *w, float *out, int64_t M, int64_t N, int64_t K,
                    int dt, void *ws, hipStream_t s) {
  char *base = static_cast<char *>(ws);
  auto *xb = reinterpret_cast<uint16_t *>(base);
  float *partials = reinterpret_cast<float *>(base + al256((int64_t)gemm_q4k_ws_bytes(M, K)));
  if (int rc = launch_to_bf16(src, from_act ? kActSrc : F32, xb, M, K, s)) return rc;
  if (dt == Q4_K) return launch_gemm_q4k_bf16(xb, w, out, partials, M, N, K, s);
  auto *wb = reinterpret_cast<uint16_t *>(base + al256((int64_t)gemm_q4k_ws_bytes(M, K)) +
                                          al256((int64_t)gemm_q4k_partial_bytes(M, N, K)));
  if (int rc = dt == Q6_K_R ? launch_dequant_q6kr(w, wb, N, K, BF16, s) : launch_dequant(w, wb, N * K, dt, BF16, s))
    return rc;
  return launch_gemm_ws_bf16(xb, wb, out, partials, M, N, K, s);
}

int launch_matmul_act(const void *act, const void *w, float *out, int64_t M, int64_t N, int64_t K, int dt, void *ws,
                      hipStream_t s) {
  if (matmul_act_takes_gemm(M, K, dt)) return run_gemm(act, true, w, out, M, N, K, dt, ws, s);
  if (staged_parts_ok(M, N, K, dt, w, act))
    return launch_staged_parts(act, w, out, static_cast<float *>(ws), M, N, K, dt, s);
  if (q4kx_halves_ok(M, N, K, dt, w, act))
    return launch_gemv_q4kx_act_halves(act, w, out, static_cast<float *>(ws), M, N, K, dt, s);
  return launch_gemv_act(act, w, out, M, N, K, dt, s);
}

int launch_matmul_q(const float *x, const void *w, float *out, int64_t M, int64_t N, int64_t K, int dt, void *ws,
                    hipStream_t s) {
  if (use_gemm(M, dt) && gemm_k_ok(K)) return run_gemm(x, false, w, out, M, N, K, dt, ws, s);
  if (dt == Q6_K_R) {
    // The planar Q6_K layout is only read by the team GEMV (and dequantized for the GEMM).
    if (!q4kx_ok(M, N, K, w, nullptr, x, dt))
      return fail(HQ_EUNSUPPORTED, "matmul_q", "Q6_K_R needs 16-byte aligned x and w, M <= %d, K <= 32768",
                  (int)kGemvMaxRows);
    if (q4kx_xin(K)) return launch_gemv_q4kx(x, w, nullptr, out, M, N, K, 0, dt, s);
    if (int rc = launch_quantize_act(x, F32, ws, M, K, s)) return rc;
    return launch_gemv_q4kx_act(ws, w, out, M, N, K, dt, s);
  }
  if ((dt == Q4_K || dt == Q5_K) && q4kx_ok(M, N, K, w, nullptr, x, dt) && q4kx_xin(K))
    return launch_gemv_q4kx(x, w, nullptr, out, M, N, K, 0, dt, s);
  if (staged_parts_ok(M, N, K, dt, w, x)) {
    // Staged rows too long for one slice: x quantized once, then the K parts and their sum
    // (several rows of x: each part's columns quantized on their own, one launch per part).
    if (M > 1) return launch_staged_parts_x(x, w, out, ws, M, N, K, dt, s);
    if (int rc = launch_quantize_act(x, F32, ws, M, K, s)) return rc;
    float *tmp = reinterpret_cast<float *>(static_cast<char *>(ws) + al256(act_bytes(M, K)));
    return launch_staged_parts(ws, w, out, tmp, M, N, K, dt, s);
  }
  if (q4kx_halves_ok(M, N, K, dt, w, x)) {
    // Rows longer than one team: x quantized once, then the two K halves and their sum
    // (several rows of x: each half's columns quantized on their own, one launch per half).
    if (M > 1) return launch_gemv_q4kx_halves_x(x, w, out, ws, M, N, K, dt, s);
    if (int rc = launch_quantize_act(x, F32, ws, M, K, s)) return rc;
    float *tmp = reinterpret_cast<float *>(static_cast<char *>(ws) + al256(act_bytes(M, K)));
    return launch_gemv_q4kx_act_halves(ws, w, out, tmp, M, N, K, dt, s);
  }
  if (!gemv_fast_ok(dt, K, w) || (dt == Q5_K && !q4kx_ok(1, N, K, w, nullptr, x, dt)))
    return launch_gemv_generic(x, w, out, M, N, K, dt, s);
  if (dt != Q4_K && dt != Q5_K && K <= kStagedXinMaxK && ((uintptr_t)x & 15) == 0)
    return launch_staged(nullptr, x, static_cast<const uint8_t *>(w), out, M, N, K, dt, s);
  if (int rc = launch_quantize_act(x, F32, ws, M, K, s)) return rc;
  return launch_gemv_act(ws, w, out, M, N, K, dt, s);
}

}  // namespace hq
