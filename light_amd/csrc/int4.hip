// int4.hip -- GPTQ / AWQ 4-bit group-quantized weights (Light's canonical quant.Int4).
//
// Layout (quant/int4.go:11-34): codes U32 (N, K/8), nibble j of word c is W[n, 8c+j];
// scales / zeros F32 (N, K/G); W[n, k] = s[n, k/G] * (code(n, k) - z[n, k/G]).
//
//  * int4_dequant: one thread per code word, s * (q - z) formed in F32 with explicit
//    rounding (Light's int4DequantCPU, kernels/cpu/int4.go:19-54), BF16 rounded once.
//  * GEMV (M <= 8, Light's int4GEMVMaxM, ops/int4.go:58-59): x is quantized to the
//    planar q8_1 act layout; a team of lanes covers one weight row, each lane owning
//    CPL 32-element blocks (16 code bytes each) with their int8 activations held in
//    registers.  The low / high nibbles of a code word are the even / odd elements of
//    its 8, so the lane permutes its activation bytes once (v_perm_b32) into even /
//    odd order and every product is a v_dot4_i32_i8 chain.  Per 32-block (two
//    activation levels x ~= d*q1 + e*q2, block sum sx):
//    y += s * (d * sum(q * q1) + e * sum(q * q2) - z * sx).
//  * M > 8 with G % 64 == 0: the bf16 MFMA GEMM of gemm.hip with the int4 weight policy.
#include "internal.hpp"

namespace hq {

// ---- dequant --------------------------------------------------------------------

template <int ODT>
__global__ __launch_bounds__(256) void int4_dequant_kernel(const uint32_t *__restrict__ codes,
                                                           const float *__restrict__ sc,
                                                           const float *__restrict__ zr, void *__restrict__ out,
                                                           int64_t N, int64_t K, int G, int64_t off) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t wpr = K / 8;
  if (idx >= N * wpr) return;
  const int64_t n = idx / wpr, c = idx - n * wpr;
  const uint32_t w = codes[idx];
  const int64_t ng = K / G;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const int64_t k = 8 * c + j, g = n * ng + k / G;
    const float v = __fmul_rn(sc[g], __fsub_rn((float)((w >> (4 * j)) & 15), zr[g]));
    if constexpr (ODT == F32)
      static_cast<float *>(out)[off + n * K + k] = v;
    else
      static_cast<uint16_t *>(out)[off + n * K + k] = f2bf_rne(v);
  }
}

int launch_int4_dequant(const uint32_t *codes, const float *s, const float *z, void *out, int out_dtype, int64_t N,
                        int64_t K, int G, int64_t off, hipStream_t st) {
  const int64_t n = N * (K / 8);
  dim3 g((unsigned)cdiv(n, 256));
  if (out_dtype == F32)
    int4_dequant_kernel<F32><<<g, 256, 0, st>>>(codes, s, z, out, N, K, G, off);
  else
    int4_dequant_kernel<BF16><<<g, 256, 0, st>>>(codes, s, z, out, N, K, G, off);
  return check_launch("int4_dequant");
}

// ---- act-order gather -----------------------------------------------------------
// y[m, k] = x[m, idx[k]] (ops.gatherColumns, ops/int4.go:129-147: act-order GPTQ stores
// the weight's K axis sorted by group; x's columns are gathered the same way).
template <typename T>
__global__ __launch_bounds__(256) void gather_cols_kernel(const T *__restrict__ x, const int64_t *__restrict__ idx,
                                                          T *__restrict__ y, int64_t M, int64_t K) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= M * K) return;
  const int64_t m = i / K, k = i - m * K;
  const int64_t j = idx[k];
  y[i] = (j >= 0 && j < K) ? x[m * K + j] : T(0);
}

int launch_gather_cols(const void *x, const int64_t *idx, void *y, int64_t M, int64_t K, int elem_bytes,
                       hipStream_t s) {
  dim3 g((unsigned)cdiv(M * K, 256));
  if (elem_bytes == 4)
    gather_cols_kernel<uint32_t><<<g, 256, 0, s>>>(static_cast<const uint32_t *>(x), idx, static_cast<uint32_t *>(y), M, K);
  else
    gather_cols_kernel<uint16_t><<<g, 256, 0, s>>>(static_cast<const uint16_t *>(x), idx, static_cast<uint16_t *>(y), M, K);
  return check_launch("gather_cols");
}

// ---- GEMV -----------------------------------------------------------------------

__device__ __forceinline__ float row16_sum_i4(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false));
  return v;
}

struct I4Args {
  const uint8_t *act;
  const uint32_t *codes;
  const float *s, *z;
  void *out;
  int odt, M, N, K, G, nb, P, TP;  // nb = K / 32; P = lanes per row; TP = P rounded up to 16
  int64_t q2_off, d_off, s_off;
};

template <int CPL, int R, int MM, bool PF>
__global__ __launch_bounds__(512) void gemv_int4_kernel(I4Args a) {
  __shared__ float part[512];
  const int t = threadIdx.x;
  const int RW = blockDim.x / a.TP;
  const int team = t / a.TP, u = t - team * a.TP;
  const bool active = u < a.P;
  const int ngrp = a.K / a.G;
  const int rows_per_group = RW * R;
  const int ngroups = (a.N + rows_per_group - 1) / rows_per_group;
  const int m0 = blockIdx.y * MM;

  int blk[CPL];
  bool bok[CPL];
#pragma unroll
  for (int c = 0; c < CPL; c++) {
    const int j = u * CPL + c;
    bok[c] = active && j < a.nb;
    blk[c] = bok[c] ? j : 0;
  }

  uint4 q[R][CPL];
  float2 sz[R][CPL];
  uint4 nq[R][CPL];
  float2 nsz[R][CPL];
#define I4_LOAD(grp, Q, SZ)                                                                    \
  {                                                                                            \
    _Pragma("unroll") for (int r = 0; r < R; r++) {                                            \
      int row = (grp) * rows_per_group + r * RW + team;                                        \
      row = row < a.N ? row : a.N - 1;                                                         \
      _Pragma("unroll") for (int c = 0; c < CPL; c++) {                                        \
        if (bok[c]) {                                                                          \
          Q[r][c] = *reinterpret_cast<const uint4 *>(a.codes + (int64_t)row * (a.K / 8) + 4 * blk[c]); \
          const int64_t gi = (int64_t)row * ngrp + (32 * blk[c]) / a.G;                        \
          SZ[r][c] = make_float2(a.s[gi], a.z[gi]);                                            \
        } else {                                                                               \
          Q[r][c] = make_uint4(0, 0, 0, 0);                                                    \
          SZ[r][c] = make_float2(0.f, 0.f);                                                    \
        }                                                                                      \
      }                                                                                        \
    }                                                                                          \
  }

  int g = blockIdx.x;
  if (g < ngroups) I4_LOAD(g, q, sz);

  // Activations: even / odd element bytes of each 8-element group, d and d*sum(q).
  int ev[MM][CPL][4], od[MM][CPL][4], ev2[MM][CPL][4], od2[MM][CPL][4];
  float2 dx[MM][CPL];
  float sx[MM][CPL];
#pragma unroll
  for (int mm = 0; mm < MM; mm++) {
    const int m = m0 + mm < a.M ? m0 + mm : a.M - 1;
#pragma unroll
    for (int c = 0; c < CPL; c++) {
      const int64_t b = (int64_t)m * a.nb + blk[c];
      const uint4 *xs = reinterpret_cast<const uint4 *>(a.act + b * 32);
      const uint4 *x2 = reinterpret_cast<const uint4 *>(a.act + a.q2_off + b * 32);
      const uint4 v0 = xs[0], v1 = xs[1], u0 = x2[0], u1 = x2[1];
      const uint32_t w8[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
      const uint32_t y8[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
      for (int k = 0; k < 4; k++) {
        ev[mm][c][k] = bok[c] ? (int)__builtin_amdgcn_perm(w8[2 * k + 1], w8[2 * k], 0x06040200u) : 0;
        od[mm][c][k] = bok[c] ? (int)__builtin_amdgcn_perm(w8[2 * k + 1], w8[2 * k], 0x07050301u) : 0;
        ev2[mm][c][k] = bok[c] ? (int)__builtin_amdgcn_perm(y8[2 * k + 1], y8[2 * k], 0x06040200u) : 0;
        od2[mm][c][k] = bok[c] ? (int)__builtin_amdgcn_perm(y8[2 * k + 1], y8[2 * k], 0x07050301u) : 0;
      }
      dx[mm][c] = bok[c] ? reinterpret_cast<const float2 *>(a.act + a.d_off)[b] : make_float2(0.f, 0.f);
      sx[mm][c] = bok[c] ? reinterpret_cast<const float *>(a.act + a.s_off)[b] : 0.f;
    }
  }
  const int lane = t & 63;
  const int hpt = a.TP >> 4;

  for (; g < ngroups; g += gridDim.x) {
    if (PF && g + (int)gridDim.x < ngroups) I4_LOAD(g + gridDim.x, nq, nsz);
#pragma unroll
    for (int r = 0; r < R; r++) {
      float acc[MM];
#pragma unroll
      for (int mm = 0; mm < MM; mm++) acc[mm] = 0.f;
#pragma unroll
      for (int c = 0; c < CPL; c++) {
        const uint32_t w4[4] = {q[r][c].x, q[r][c].y, q[r][c].z, q[r][c].w};
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
          lo[k] = w4[k] & 0x0F0F0F0Fu;
          hi[k] = (w4[k] >> 4) & 0x0F0F0F0Fu;
        }
#pragma unroll
        for (int mm = 0; mm < MM; mm++) {
          int dot = 0, dot2 = 0;
#pragma unroll
          for (int k = 0; k < 4; k++) {
            dot = dot4((int)lo[k], ev[mm][c][k], dot);
            dot = dot4((int)hi[k], od[mm][c][k], dot);
            dot2 = dot4((int)lo[k], ev2[mm][c][k], dot2);
            dot2 = dot4((int)hi[k], od2[mm][c][k], dot2);
          }
          acc[mm] += sz[r][c].x * (dx[mm][c].x * (float)dot + dx[mm][c].y * (float)dot2 - sz[r][c].y * sx[mm][c]);
        }
      }
#pragma unroll
      for (int mm = 0; mm < MM; mm++) {
        const float s = row16_sum_i4(acc[mm]);
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
      if (row < a.N && m0 + mm < a.M) {
        const int64_t o = (int64_t)(m0 + mm) * a.N + row;
        if (a.odt == F32)
          static_cast<float *>(a.out)[o] = acc;
        else if (a.odt == BF16)
          static_cast<uint16_t *>(a.out)[o] = f2bf_rne(acc);
        else
          static_cast<uint16_t *>(a.out)[o] = f2h_rne(acc);
      }
    }
    __syncthreads();
    if (PF) {
#pragma unroll
      for (int r = 0; r < R; r++)
#pragma unroll
        for (int c = 0; c < CPL; c++) {
          q[r][c] = nq[r][c];
          sz[r][c] = nsz[r][c];
        }
    } else if (g + (int)gridDim.x < ngroups) {
      I4_LOAD(g + gridDim.x, q, sz);
    }
  }
#undef I4_LOAD
}

template <int CPL, int MM>
static void run_i4(const I4Args &a, hipStream_t s) {
  const int rw = a.TP >= 256 ? 1 : 256 / a.TP;
  const int cus = device_cus();
  dim3 g(0, (unsigned)cdiv(a.M, MM));
  if (a.TP <= 128) {
    int ng = (a.N + rw - 1) / rw;
    g.x = (unsigned)(ng < cus * 4 ? ng : cus * 4);
    gemv_int4_kernel<CPL, 1, MM, true><<<g, a.TP * rw, 0, s>>>(a);
  } else {
    int ng = (a.N + 2 * rw - 1) / (2 * rw);
    g.x = (unsigned)(ng < cus * 2 ? ng : cus * 2);
    gemv_int4_kernel<CPL, 2, MM, false><<<g, a.TP * rw, 0, s>>>(a);
  }
}

// Activation registers grow with CPL * MM: wide rows serve fewer rows of x per pass.
template <int CPL>
static void run_i4_m(const I4Args &a, int mm, hipStream_t s) {
  if constexpr (CPL >= 4) {
    run_i4<CPL, 1>(a, s);
  } else if constexpr (CPL == 2) {
    if (mm == 1)
      run_i4<CPL, 1>(a, s);
    else
      run_i4<CPL, 2>(a, s);
  } else {
    if (mm == 1)
      run_i4<CPL, 1>(a, s);
    else if (mm == 2)
      run_i4<CPL, 2>(a, s);
    else
      run_i4<CPL, 4>(a, s);
  }
}

// The MFMA GEMMs: M > 8, and rows too long for the int8 GEMV (K / 32 > 2048) at any M (their
// x rows past M are clamped and their stores masked).
static bool int4_gemm_ok(int64_t M, int64_t K, int G) { return (M > 8 || K / 32 > 2048) && G % 64 == 0; }

size_t int4_ws_bytes(int64_t M, int64_t N, int64_t K, int G, int x_dtype) {
  if (M <= 0 || K <= 0 || K % 32) return 0;
  if (!int4_gemm_ok(M, K, G)) {
    // Long rows (two K halves): the halves' F32 partials as well.
    const bool halves = M <= 8 && K > 32768 && K <= 65536 && K % 256 == 0 && G > 0 && 256 % G == 0;
    if (!halves) return (size_t)act_bytes(M, K);
    // One row: x's act layout + two F32 partials; several rows: a half's x (up to F32), its
    // act layout + the partials.
    auto al = [](int64_t b) { return (b + 255) & ~(int64_t)255; };
    const int64_t kh = (K / 2 + 255) / 256 * 256;
    return (size_t)std::max(al(act_bytes(M, K)) + 8 * M * N, al(4 * M * kh) + al(act_bytes(M, kh)) + 8 * M * N);
  }
  return (x_dtype == BF16 ? 0 : gemm_x_bytes(M, K)) + gemm_partial_bytes(M, N, K, x_dtype == F32);
}

int launch_int4_matmul(const void *x, int x_dtype, const uint32_t *codes, const float *s, const float *z, void *y,
                       int64_t M, int64_t N, int64_t K, int G, void *ws, hipStream_t st) {
  if (N > INT32_MAX || K > INT32_MAX) return fail(HQ_EUNSUPPORTED, "int4_matmul", "N or K too large");
  if (int4_gemm_ok(M, K, G) && i4cu_ok(M, N, K, G, x_dtype, x, codes)) {
    // F16 x at M <= 64 with enough column tiles to fill the chip: one workgroup per CU over
    // all of K, no split-K partials.
    return launch_i4cu(static_cast<const uint16_t *>(x), codes, s, z, y, M, N, K, G, st);
  }
  if (int4_gemm_ok(M, K, G) && i4f16_small_ok(M, N, K, G, x_dtype, x, codes)) {
    // F16 x at M <= 64: the exact-weight f16 MFMA kernel reads x as given.
    return launch_i4f16_small(static_cast<const uint16_t *>(x), codes, s, z, y,
                              reinterpret_cast<float *>(static_cast<char *>(ws) + gemm_x_bytes(M, K)), M, N, K, G, st);
  }
  if (int4_gemm_ok(M, K, G)) {
    const uint16_t *xb = static_cast<const uint16_t *>(x);
    char *rest = static_cast<char *>(ws);
    if (x_dtype != BF16) {
      xb = static_cast<const uint16_t *>(ws);
      if (int rc = launch_to_bf16(x, x_dtype, static_cast<uint16_t *>(ws), M, K, st)) return rc;
      rest += gemm_x_bytes(M, K);
    }
    return launch_gemm_int4_bf16(xb, codes, s, z, y, x_dtype, reinterpret_cast<float *>(rest), M, N, K, G, st);
  }
  if (int4_halves_ok(M, N, K, G, codes, x)) return launch_int4_halves(x, x_dtype, codes, s, z, y, M, N, K, G, ws, st);
  if (int4x_ok(M, N, K, G, codes, x)) return launch_gemv_int4x(x, x_dtype, codes, s, z, y, M, N, K, G, ws, st);
  if (int rc = launch_quantize_act(x, x_dtype, ws, M, K, st)) return rc;
  I4Args a;
  a.act = static_cast<const uint8_t *>(ws);
  a.codes = codes;
  a.s = s;
  a.z = z;
  a.out = y;
  a.odt = x_dtype;
  a.K = (int)K;
  a.N = (int)N;
  a.G = G;
  a.nb = (int)(K / 32);
  a.q2_off = act_q2_off(M, K);
  a.d_off = act_d_off(M, K);
  a.s_off = act_s_off(M, K);
  const int cpl = a.nb <= 512 ? 1 : a.nb <= 1024 ? 2 : 4;
  if (a.nb > 2048) return fail(HQ_EUNSUPPORTED, "int4_matmul", "K=%lld too large for the GEMV", (long long)K);
  a.P = (a.nb + cpl - 1) / cpl;
  a.TP = (a.P + 15) & ~15;
  // Rows of x are served four at a time (grid.y = ceil(M / 4)).
  if (M > 65535 * 4) return fail(HQ_EUNSUPPORTED, "int4_matmul", "M=%lld too large", (long long)M);
  a.M = (int)M;
  const int mm = M >= 3 ? 4 : (int)M;
  if (cpl == 1)
    run_i4_m<1>(a, mm, st);
  else if (cpl == 2)
    run_i4_m<2>(a, mm, st);
  else
    run_i4_m<4>(a, mm, st);
  return check_launch("gemv_int4");
}

}  // namespace hq
