// gemv.hip -- decode GEMV for GGUF weights (Q4_K, Q8_0, Q6_K) on q8_1 activations.
//
// Role: Light's matmul_q kernels for small M (kernels/cuda/matmul_q.go:44-91,
// kernels/cpu/quant_matmul.go:141-170); y[m, n] = sum_k x[m, k] * dequant(W)[n, k].
//
// Design (gfx950, wave64):
//  * The activation row is quantized once to q8_1 (quantize.hip) and each lane
//    keeps the int8 activations of a FIXED set of K positions in registers for
//    the whole kernel; a wave then streams weight rows past them.  The weight
//    is read exactly once from HBM; the activations are read once per wave.
//  * Inner products run on v_dot4_i32_i8 (4 MACs per op), so the unpack work per
//    weight stays far below the VALU budget needed at HBM speed.
//  * Q4_K (144-byte blocks, 16-byte aligned): lanes load their 16-byte quant
//    chunk straight from HBM (global_load_dwordx4, coalesced); the 16-byte block
//    header is fetched one dword per lane and broadcast inside each 4-lane quad
//    with DPP, so each lane issues 20 bytes of loads per 32 weights.
//  * Q8_0 (34 B) and Q6_K (210 B) blocks are only 2-byte aligned.  A wave copies
//    its rows' bytes into LDS with coalesced 16-byte loads and writes each block
//    at a padded, 4/8-byte-aligned LDS slot; lanes then decode from LDS with
//    aligned reads.
//  * Any other shape (K beyond the register budget, rows not 16-byte multiples)
//    takes a generic wave-per-row kernel on F32 activations that uses the
//    bit-exact decoder of dequant.hip.
//
// Accuracy: activations are quantized per 32 elements (error <= d/2 per element),
// and per-block partial sums are exact integers scaled once in F32.
#include "decode.hpp"
#include "internal.hpp"

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

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Streaming 16-byte load (weights are read once: non-temporal hint).
__device__ __forceinline__ uint4 ld_stream16(const void *p) {
  u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ uint32_t byte_at(uint32_t w, int k) { return (w >> (8 * k)) & 0xffu; }
__device__ __forceinline__ uint32_t ld32(const uint8_t *p) { return *reinterpret_cast<const uint32_t *>(p); }
__device__ __forceinline__ uint32_t ld16(const uint8_t *p) { return *reinterpret_cast<const uint16_t *>(p); }

// Sum of the four signed bytes of each of n dwords.
__device__ __forceinline__ int byte_sum(const int *v, int n) {
  int s = 0;
  for (int i = 0; i < n; i++) s = dot4(v[i], 0x01010101, s);
  return s;
}

// ---------------------------------------------------------------------------
// Q4_K: one "chunk" = 16 quant bytes = 16 elements of sub-block 2p (low
// nibbles) and 16 of sub-block 2p+1 (high nibbles); 8 chunks per block.
// Lane l owns chunks l, l+64, ... of every row.
// ---------------------------------------------------------------------------
template <int CPL, int R>
__global__ __launch_bounds__(256) void gemv_q4k_kernel(const uint8_t *__restrict__ xq, const uint8_t *__restrict__ w,
                                                       float *__restrict__ out, int N, int nchunks,
                                                       int64_t row_bytes, int64_t xq_row_bytes) {
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int nwaves = gridDim.x * 4;
  xq += blockIdx.y * xq_row_bytes;
  out += (int64_t)blockIdx.y * N;

  int xa[CPL][4], xb[CPL][4], qoff[CPL], hoff[CPL], kA[CPL];
  float dA[CPL], dB[CPL], sA[CPL], sB[CPL];
  bool lowj[CPL];
#pragma unroll
  for (int i = 0; i < CPL; i++) {
    int c = lane + 64 * i;
    bool ok = c < nchunks;
    if (!ok) c = 0;
    int b = c >> 3, cc = c & 7, p = cc >> 1, h = cc & 1;
    qoff[i] = b * 144 + 16 + cc * 16;
    hoff[i] = b * 144 + 4 * (cc & 3);
    lowj[i] = p < 2;
    kA[i] = (2 * p) & 3;
    const uint8_t *pa = xq + 36 * (b * 8 + 2 * p);
    const uint8_t *pb = pa + 36;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      xa[i][k] = ok ? (int)ld32(pa + 4 + 16 * h + 4 * k) : 0;
      xb[i][k] = ok ? (int)ld32(pb + 4 + 16 * h + 4 * k) : 0;
    }
    dA[i] = ok ? h2f(ld16(pa)) : 0.f;
    dB[i] = ok ? h2f(ld16(pb)) : 0.f;
    sA[i] = dA[i] * (float)byte_sum(xa[i], 4);
    sB[i] = dB[i] * (float)byte_sum(xb[i], 4);
  }

  for (int64_t row0 = (int64_t)wave * R; row0 < N; row0 += (int64_t)nwaves * R) {
    uint4 q[R][CPL];
    uint32_t hd[R][CPL];
#pragma unroll
    for (int r = 0; r < R; r++) {
      int64_t row = row0 + r < N ? row0 + r : N - 1;
      const uint8_t *rp = w + row * row_bytes;
#pragma unroll
      for (int i = 0; i < CPL; i++) {
        q[r][i] = ld_stream16(rp + qoff[i]);
        hd[r][i] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(rp + hoff[i]));
      }
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
      float acc = 0.f;
#pragma unroll
      for (int i = 0; i < CPL; i++) {
        uint32_t h0 = quad_bcast<0>(hd[r][i]), h1 = quad_bcast<1>(hd[r][i]);
        uint32_t h2 = quad_bcast<2>(hd[r][i]), h3 = quad_bcast<3>(hd[r][i]);
        float d = h2f(h0 & 0xffffu), dmin = h2f(h0 >> 16);
        int ka = kA[i], kb = ka + 1;
        uint32_t sa = byte_at(h1, ka), ma = byte_at(h2, ka), aa = byte_at(h3, ka);
        uint32_t sb = byte_at(h1, kb), mb = byte_at(h2, kb), ab = byte_at(h3, kb);
        int scA = lowj[i] ? (int)(sa & 63) : (int)((aa & 15) | ((sa >> 6) << 4));
        int mnA = lowj[i] ? (int)(ma & 63) : (int)((aa >> 4) | ((ma >> 6) << 4));
        int scB = lowj[i] ? (int)(sb & 63) : (int)((ab & 15) | ((sb >> 6) << 4));
        int mnB = lowj[i] ? (int)(mb & 63) : (int)((ab >> 4) | ((mb >> 6) << 4));
        const uint32_t qw[4] = {q[r][i].x, q[r][i].y, q[r][i].z, q[r][i].w};
        int dotA = 0, dotB = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) {
          dotA = dot4((int)(qw[k] & 0x0F0F0F0Fu), xa[i][k], dotA);
          dotB = dot4((int)((qw[k] >> 4) & 0x0F0F0F0Fu), xb[i][k], dotB);
        }
        float v = (float)scA * dA[i] * (float)dotA + (float)scB * dB[i] * (float)dotB;
        float mn = (float)mnA * sA[i] + (float)mnB * sB[i];
        acc += d * v - dmin * mn;
      }
      acc = wave_sum(acc);
      if (lane == 0 && row0 + r < N) out[row0 + r] = acc;
    }
  }
}

// ---------------------------------------------------------------------------
// Q8_0 / Q6_K: LDS-staged rows.
// ---------------------------------------------------------------------------
template <int DT>
struct Staged;
template <>
struct Staged<Q8_0> {
  static constexpr int BB = 34, SB = 36, LEAD = 2, UPB = 1;  // block at slot+2: d at +2, qs at +4
};
template <>
struct Staged<Q6_K> {
  static constexpr int BB = 210, SB = 216, LEAD = 0, UPB = 8;  // block at slot: ql +0, qh +128, sc +192, d +208
};

template <int DT, int CPL, int R>
__global__ __launch_bounds__(256) void gemv_staged_kernel(const uint8_t *__restrict__ xq,
                                                          const uint8_t *__restrict__ w, float *__restrict__ out,
                                                          int N, int nblk, int64_t row_bytes, int64_t xq_row_bytes,
                                                          int lds_wave_bytes) {
  using S = Staged<DT>;
  extern __shared__ __align__(16) uint8_t smem[];
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int nwaves = gridDim.x * 4;
  uint8_t *lds = smem + (threadIdx.x >> 6) * lds_wave_bytes;
  uint16_t *lds16 = reinterpret_cast<uint16_t *>(lds);
  xq += blockIdx.y * xq_row_bytes;
  out += (int64_t)blockIdx.y * N;
  const int units = nblk * S::UPB;

  // Activations of this lane's units.
  constexpr int XD = DT == Q8_0 ? 8 : 8;  // dwords of int8 activations per unit
  int xv[CPL][XD];
  float dx[CPL][DT == Q8_0 ? 1 : 4];
  int s32[CPL][4];
  int ublk[CPL], uh[CPL], ul0[CPL];
#pragma unroll
  for (int i = 0; i < CPL; i++) {
    int u = lane + 64 * i;
    bool ok = u < units;
    if (!ok) u = 0;
    if constexpr (DT == Q8_0) {
      ublk[i] = u;
      uh[i] = ul0[i] = 0;
      const uint8_t *p = xq + 36 * u;
#pragma unroll
      for (int k = 0; k < 8; k++) xv[i][k] = ok ? (int)ld32(p + 4 + 4 * k) : 0;
      dx[i][0] = ok ? h2f(ld16(p)) : 0.f;
    } else {
      int b = u >> 3, l8 = u & 7, h = l8 >> 2, l0 = (l8 & 3) * 8;
      ublk[i] = b;
      uh[i] = h;
      ul0[i] = l0;
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const uint8_t *p = xq + 36 * (b * 8 + h * 4 + g);
        xv[i][2 * g] = ok ? (int)ld32(p + 4 + l0) : 0;
        xv[i][2 * g + 1] = ok ? (int)ld32(p + 8 + l0) : 0;
        dx[i][g] = ok ? h2f(ld16(p)) : 0.f;
        s32[i][g] = 32 * byte_sum(&xv[i][2 * g], 2);
      }
    }
  }

  for (int64_t row0 = (int64_t)wave * R; row0 < N; row0 += (int64_t)nwaves * R) {
    const int nrows = (int)(N - row0 < R ? N - row0 : R);
    const int nseg = (int)(nrows * row_bytes / 16);
    const uint4 *src = reinterpret_cast<const uint4 *>(w + row0 * row_bytes);
    // Stage: 16-byte coalesced loads, 2-byte scatter into padded block slots.
    for (int s0 = lane; s0 < nseg; s0 += 256) {
      uint4 v[4];
#pragma unroll
      for (int k = 0; k < 4; k++)
        if (s0 + 64 * k < nseg) v[k] = ld_stream16(src + s0 + 64 * k);
#pragma unroll
      for (int k = 0; k < 4; k++) {
        int s = s0 + 64 * k;
        if (s >= nseg) break;
        const uint32_t vw[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
#pragma unroll
        for (int j = 0; j < 8; j++) {
          int ob = 16 * s + 2 * j;
          int gb = ob / S::BB;
          lds16[(gb * S::SB + S::LEAD + ob - gb * S::BB) >> 1] = (uint16_t)(vw[j >> 1] >> (16 * (j & 1)));
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

#pragma unroll
    for (int r = 0; r < R; r++) {
      if (r >= nrows) break;
      float acc = 0.f;
#pragma unroll
      for (int i = 0; i < CPL; i++) {
        const uint8_t *blk = lds + (r * nblk + ublk[i]) * S::SB;
        if constexpr (DT == Q8_0) {
          float d = h2f(ld16(blk + 2));
          int dot = 0;
#pragma unroll
          for (int k = 0; k < 8; k++) dot = dot4((int)ld32(blk + 4 + 4 * k), xv[i][k], dot);
          acc += d * (dx[i][0] * (float)dot);
        } else {
          const int h = uh[i], l0 = ul0[i];
          const uint2 qa = *reinterpret_cast<const uint2 *>(blk + h * 64 + l0);
          const uint2 qb = *reinterpret_cast<const uint2 *>(blk + h * 64 + 32 + l0);
          const uint2 qh = *reinterpret_cast<const uint2 *>(blk + 128 + h * 32 + l0);
          const uint2 sc = *reinterpret_cast<const uint2 *>(blk + 192 + h * 8);
          float d = h2f(ld16(blk + 208));
          const uint32_t A[2] = {qa.x, qa.y}, B[2] = {qb.x, qb.y}, H[2] = {qh.x, qh.y};
          const int is = l0 >> 4;
          float v = 0.f;
#pragma unroll
          for (int g = 0; g < 4; g++) {
            int dot = 0;
#pragma unroll
            for (int k = 0; k < 2; k++) {
              uint32_t nib = g == 0 ? (A[k] & 0x0F0F0F0Fu)
                           : g == 1 ? (B[k] & 0x0F0F0F0Fu)
                           : g == 2 ? ((A[k] >> 4) & 0x0F0F0F0Fu)
                                    : ((B[k] >> 4) & 0x0F0F0F0Fu);
              uint32_t qv = nib | (((H[k] >> (2 * g)) & 0x03030303u) << 4);
              dot = dot4((int)qv, xv[i][2 * g + k], dot);
            }
            int sidx = 2 * g + is;  // scale byte within this half's 8
            int scv = (int)(int8_t)((sidx < 4 ? sc.x >> (8 * sidx) : sc.y >> (8 * (sidx - 4))) & 0xff);
            v += (float)scv * (dx[i][g] * (float)(dot - s32[i][g]));
          }
          acc += d * v;
        }
      }
      acc = wave_sum(acc);
      if (lane == 0) out[row0 + r] = acc;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
  }
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
    acc = wave_sum(acc);
    if (lane == 0) out[blockIdx.y * N + row] = acc;
  }
}

// ---------------------------------------------------------------------------
// Launch logic
// ---------------------------------------------------------------------------

static const int kCplSteps[] = {1, 2, 3, 4, 5, 6, 7, 8, 10, 12, 14, 16};

static int pick_cpl(int64_t units) {
  int64_t need = cdiv(units, 64);
  for (int c : kCplSteps)
    if (c >= need) return c;
  return 0;
}

// Fast (int8) GEMV applies: K fits the register budget and rows are 16-byte multiples.
static bool gemv_fast_ok(int dt, int64_t K, const void *w) {
  if (((uintptr_t)w & 15) != 0) return false;
  BlockInfo bi = block_info(dt);
  int64_t nblk = K / bi.elems, row_bytes = nblk * bi.bytes;
  if (row_bytes % 16) return false;
  int64_t units = dt == Q4_K ? nblk * 8 : dt == Q6_K ? nblk * 8 : nblk;
  if (!pick_cpl(units)) return false;
  if (dt != Q4_K) {
    int sb = dt == Q8_0 ? Staged<Q8_0>::SB : Staged<Q6_K>::SB;
    if (nblk * sb + 16 > 16384) return false;  // one row must fit a wave's LDS slice
  }
  return true;
}

template <int CPL, int R>
static void run_q4k(const uint8_t *xq, const uint8_t *w, float *out, int64_t M, int64_t N, int64_t K, hipStream_t s) {
  int64_t nblk = K / 256;
  int64_t wgs = cdiv(cdiv(N, R), 4);
  int64_t cap = (int64_t)device_cus() * 16;
  dim3 grid((unsigned)(wgs < cap ? wgs : cap), (unsigned)M);
  gemv_q4k_kernel<CPL, R><<<grid, 256, 0, s>>>(xq, w, out, (int)N, (int)(nblk * 8), nblk * 144, (K / 32) * 36);
}

template <int DT, int CPL, int R>
static void run_staged(const uint8_t *xq, const uint8_t *w, float *out, int64_t M, int64_t N, int64_t K,
                       hipStream_t s) {
  using S = Staged<DT>;
  int64_t nblk = K / block_info(DT).elems;
  int lds_wave = (int)(((R * nblk * S::SB + 16) + 15) & ~15);
  int64_t wgs = cdiv(cdiv(N, R), 4);
  int64_t cap = (int64_t)device_cus() * 16;
  dim3 grid((unsigned)(wgs < cap ? wgs : cap), (unsigned)M);
  gemv_staged_kernel<DT, CPL, R><<<grid, 256, 4 * lds_wave, s>>>(xq, w, out, (int)N, (int)nblk,
                                                                  nblk * block_info(DT).bytes, (K / 32) * 36,
                                                                  lds_wave);
}

#define CPL_SWITCH(cpl, CALL)        \
  switch (cpl) {                     \
    case 1: { constexpr int C = 1; CALL; } break;   \
    case 2: { constexpr int C = 2; CALL; } break;   \
    case 3: { constexpr int C = 3; CALL; } break;   \
    case 4: { constexpr int C = 4; CALL; } break;   \
    case 5: { constexpr int C = 5; CALL; } break;   \
    case 6: { constexpr int C = 6; CALL; } break;   \
    case 7: { constexpr int C = 7; CALL; } break;   \
    case 8: { constexpr int C = 8; CALL; } break;   \
    case 10: { constexpr int C = 10; CALL; } break; \
    case 12: { constexpr int C = 12; CALL; } break; \
    case 14: { constexpr int C = 14; CALL; } break; \
    default: { constexpr int C = 16; CALL; } break; \
  }

template <int C>
static void run_q4k_c(const uint8_t *xq, const uint8_t *w, float *out, int64_t M, int64_t N, int64_t K, hipStream_t s) {
  if constexpr (C <= 2)
    run_q4k<C, 4>(xq, w, out, M, N, K, s);
  else if constexpr (C <= 8)
    run_q4k<C, 2>(xq, w, out, M, N, K, s);
  else
    run_q4k<C, 1>(xq, w, out, M, N, K, s);
}

template <int DT, int C>
static void run_staged_c(const uint8_t *xq, const uint8_t *w, float *out, int64_t M, int64_t N, int64_t K,
                         hipStream_t s) {
  using S = Staged<DT>;
  int64_t row_lds = (K / block_info(DT).elems) * S::SB;
  if constexpr (C <= 4) {
    if (4 * row_lds + 16 <= 16384) return run_staged<DT, C, 4>(xq, w, out, M, N, K, s);
  }
  if (2 * row_lds + 16 <= 16384) return run_staged<DT, C, 2>(xq, w, out, M, N, K, s);
  run_staged<DT, C, 1>(xq, w, out, M, N, K, s);
}

int launch_gemv_q8(const void *xqv, const void *wv, float *out, int64_t M, int64_t N, int64_t K, int dt,
                   hipStream_t s) {
  auto *xq = static_cast<const uint8_t *>(xqv);
  auto *w = static_cast<const uint8_t *>(wv);
  if (N > INT32_MAX) return fail(HQ_EUNSUPPORTED, "gemv", "N=%lld too large", (long long)N);
  int64_t nblk = K / block_info(dt).elems;
  int cpl = pick_cpl(dt == Q8_0 ? nblk : nblk * 8);
  switch (dt) {
    case Q4_K: CPL_SWITCH(cpl, (run_q4k_c<C>(xq, w, out, M, N, K, s))); break;
    case Q8_0: CPL_SWITCH(cpl, (run_staged_c<Q8_0, C>(xq, w, out, M, N, K, s))); break;
    case Q6_K: CPL_SWITCH(cpl, (run_staged_c<Q6_K, C>(xq, w, out, M, N, K, s))); break;
    default: return fail(HQ_EUNSUPPORTED, "gemv", "dtype %d", dt);
  }
  return check_launch("gemv_q8");
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
    case Q6_K: gemv_generic_kernel<Q6_K><<<grid, 256, 0, s>>>(x, w, out, N, K, row_bytes); break;
    default: return fail(HQ_EUNSUPPORTED, "gemv", "dtype %d", dt);
  }
  return check_launch("gemv_generic");
}

static size_t q8_bytes(int64_t M, int64_t K) { return ((size_t)M * (size_t)(K / 32) * 36 + 255) & ~(size_t)255; }

static bool use_gemm(int64_t M, int dt) { return dt == Q4_K && M > kGemvMaxRows; }

size_t matmul_q_ws_bytes(int64_t M, int64_t K, int dt) {
  if (M <= 0 || K <= 0 || K % 32) return 0;
  return q8_bytes(M, K) + (use_gemm(M, dt) ? gemm_q4k_ws_bytes(M, K) : 0);
}

const char *matmul_q_kernel_name(int64_t M, int dt) { return use_gemm(M, dt) ? "matmul_q.gemm" : "matmul_q.gemv"; }

int launch_matmul_q(const float *x, const void *w, float *out, int64_t M, int64_t N, int64_t K, int dt, void *ws,
                    hipStream_t s) {
  if (use_gemm(M, dt)) {
    if (int rc = launch_quantize_q8_1(x, F32, ws, M, K, s)) return rc;
    return launch_gemm_q4k(ws, w, out, M, N, K, static_cast<char *>(ws) + q8_bytes(M, K), s);
  }
  if (!gemv_fast_ok(dt, K, w)) return launch_gemv_generic(x, w, out, M, N, K, dt, s);
  if (int rc = launch_quantize_q8_1(x, F32, ws, M, K, s)) return rc;
  return launch_gemv_q8(ws, w, out, M, N, K, dt, s);
}

}  // namespace hq
