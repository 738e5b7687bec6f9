// ceiling.hip -- the hardware ceilings the bench reports beside the roofline fractions: a
// streaming read of a device buffer (how much of the 8 TB/s HBM peak a launch of a given size
// can reach, by access order, loads in flight and cache-line use), a register-only MFMA loop
// (how much of the 2.5 PFLOP/s dense bf16 peak the matrix cores sustain) and an MFMA + VALU
// mix (how far a SIMD overlaps the two).  Measurement kernels, not part of any Light op.
#include "internal.hpp"

namespace hq {

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Every thread xor-folds DEPTH 16-byte loads per trip, all issued before any is used.
//  ORDER 0 (window): trip j of thread g reads items (j DEPTH + k) G + g -- at any time the grid
//    reads one contiguous window of DEPTH * G * 16 bytes, which moves through the buffer.
//  ORDER 1 (slice): workgroup b reads its own contiguous 1 / gridDim slice front to back,
//    the workgroups' slices spread over the whole buffer (the order of a kernel whose
//    workgroups own whole output chunks).
//  ORDER 2 (half lines): the window order's bytes, but each load instruction reads 16 rows x
//    64 bytes -- half of 16 different 128-byte lines, lane 16 q + r at row r, piece q -- and
//    the other halves come a trip later (the pattern of a 16 x 16 MFMA fragment loaded
//    straight from a row-major matrix).  Against ORDER 0 it shows what a load costs per
//    cache line touched rather than per byte.
template <int ORDER, int DEPTH>
__global__ __launch_bounds__(512) void read_kernel(const u32x4 *__restrict__ p, int64_t n, uint32_t *sink) {
  const int64_t G = (int64_t)gridDim.x * blockDim.x;
  if constexpr (ORDER == 2) {
    // Regions of 16 lines (128 units of 16 bytes); wave w's trip t reads DEPTH regions' half h.
    const int64_t W = G / 64, nreg = n / 128;
    const int64_t w = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63, r = lane & 15, q = lane >> 4;
    u32x4 acc = {0, 0, 0, 0};
    for (int64_t t = 0;; t++) {
      const int64_t reg0 = ((t >> 1) * DEPTH) * W + w;
      if (reg0 >= nreg) break;
      const int h = (int)(t & 1);
      u32x4 v[DEPTH];
#pragma unroll
      for (int k = 0; k < DEPTH; k++) {
        const int64_t reg = reg0 + (int64_t)k * W;
        v[k] = reg < nreg ? p[reg * 128 + r * 8 + h * 4 + q] : u32x4{0, 0, 0, 0};
      }
#pragma unroll
      for (int k = 0; k < DEPTH; k++) acc ^= v[k];
    }
    const uint32_t x = acc.x ^ acc.y ^ acc.z ^ acc.w;
    if (x == 0x9e3779b9u) sink[0] = x;
    return;
  }
  int64_t base, step, end;
  if constexpr (ORDER == 0) {
    base = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    step = G;
    end = n;
  } else {
    const int64_t per = (n + gridDim.x - 1) / gridDim.x;
    base = (int64_t)blockIdx.x * per + threadIdx.x;
    step = blockDim.x;
    end = (int64_t)blockIdx.x * per + per < n ? (int64_t)blockIdx.x * per + per : n;
  }
  u32x4 acc = {0, 0, 0, 0};
  for (int64_t i = base; i < end; i += DEPTH * step) {
    u32x4 v[DEPTH];
#pragma unroll
    for (int k = 0; k < DEPTH; k++) {
      const int64_t j = i + k * step;
      v[k] = j < end ? p[j] : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int k = 0; k < DEPTH; k++) acc ^= v[k];
  }
  const uint32_t r = acc.x ^ acc.y ^ acc.z ^ acc.w;
  if (r == 0x9e3779b9u) sink[0] = r;  // keeps the loads; practically never stored
}

// Four independent v_mfma_f32_32x32x16_bf16 chains per wave on register operands.
__global__ __launch_bounds__(256) void mfma_kernel(int64_t iters, float *sink) {
  bf16x8 a, b;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    a[i] = (__bf16)(float)((threadIdx.x + i) & 7);
    b[i] = (__bf16)(float)((threadIdx.x * 3 + i) & 7);
  }
  f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
  for (int64_t it = 0; it < iters; it++) {
    c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c0, 0, 0, 0);
    c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c1, 0, 0, 0);
    c2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c2, 0, 0, 0);
    c3 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c3, 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 16; i++) s += c0[i] + c1[i] + c2[i] + c3[i];
  if (s == -1.f) sink[0] = s;  // never: the sums are non-negative
}

// MODE 0: 20 v_mfma_f32_16x16x32_f16 per iteration (independent accumulators); MODE 1: 80
// v_pk_fma_f16 in 20 independent chains; MODE 2: both, the VALU block before the MFMA block
// (the shape of a dequantize-then-multiply step).  Two waves per SIMD.
template <int MODE>
__global__ __launch_bounds__(512) void mix_kernel(int64_t iters, float *sink) {
  f16x8 a[4], b[5];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int e = 0; e < 8; e++) a[i][e] = (_Float16)(float)((threadIdx.x + i + e) & 3);
#pragma unroll
  for (int j = 0; j < 5; j++)
#pragma unroll
    for (int e = 0; e < 8; e++) b[j][e] = (_Float16)(float)((threadIdx.x * 3 + j + e) & 3);
  f32x4 acc[4][5];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 5; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  f16x2 v[20];
#pragma unroll
  for (int i = 0; i < 20; i++) v[i] = f16x2{(_Float16)(float)(threadIdx.x & 7), (_Float16)1.f};
  const f16x2 m = {(_Float16)0.999f, (_Float16)1.001f}, c = {(_Float16)0.01f, (_Float16)0.02f};
  for (int64_t it = 0; it < iters; it++) {
    if constexpr (MODE != 0) {
#pragma unroll
      for (int r = 0; r < 4; r++)
#pragma unroll
        for (int i = 0; i < 20; i++) v[i] = __builtin_elementwise_fma(v[i], m, c);
    }
    if constexpr (MODE != 1) {
#pragma unroll
      for (int j = 0; j < 5; j++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 5; j++) s += acc[i][j][0] + acc[i][j][1] + acc[i][j][2] + acc[i][j][3];
#pragma unroll
  for (int i = 0; i < 20; i++) s += (float)v[i][0] + (float)v[i][1];
  if (s == -12345.f) sink[0] = s;  // practically never
}

template <int ORDER>
int launch_read(const void *buf, int64_t n16, int depth, uint32_t *sink, unsigned grid, hipStream_t s) {
  const auto *p = static_cast<const u32x4 *>(buf);
  switch (depth) {
    case 1: read_kernel<ORDER, 1><<<grid, 512, 0, s>>>(p, n16, sink); break;
    case 2: read_kernel<ORDER, 2><<<grid, 512, 0, s>>>(p, n16, sink); break;
    case 4: read_kernel<ORDER, 4><<<grid, 512, 0, s>>>(p, n16, sink); break;
    default: read_kernel<ORDER, 8><<<grid, 512, 0, s>>>(p, n16, sink); break;
  }
  return check_launch("ceiling_read");
}

}  // namespace

int launch_ceiling_read(const void *buf, int64_t bytes, int order, int depth, uint32_t *sink, hipStream_t s) {
  if (!buf || !sink || bytes < 16 || bytes % 16 || ((uintptr_t)buf & 15))
    return fail(HQ_EINVAL, "hq_ceiling_read", "buffer of %lld bytes must be 16-byte aligned and sized",
                (long long)bytes);
  if (order < 0 || order > 2) return fail(HQ_EINVAL, "hq_ceiling_read", "order %d", order);
  if (order == 2 && bytes % 2048)
    return fail(HQ_EINVAL, "hq_ceiling_read", "order 2 reads whole 2 KB regions; %lld bytes", (long long)bytes);
  if (depth != 1 && depth != 2 && depth != 4 && depth != 8) return fail(HQ_EINVAL, "hq_ceiling_read", "depth %d", depth);
  const unsigned grid = (unsigned)(2 * device_cus());
  if (order == 2) return launch_read<2>(buf, bytes / 16, depth, sink, grid, s);
  return order == 0 ? launch_read<0>(buf, bytes / 16, depth, sink, grid, s)
                    : launch_read<1>(buf, bytes / 16, depth, sink, grid, s);
}

int launch_ceiling_mfma(int64_t iters, float *sink, hipStream_t s) {
  if (iters < 1 || !sink) return fail(HQ_EINVAL, "hq_ceiling_mfma", "iters %lld", (long long)iters);
  const unsigned grid = (unsigned)(2 * device_cus());
  mfma_kernel<<<grid, 256, 0, s>>>(iters, sink);
  return check_launch("ceiling_mfma");
}

int launch_ceiling_mix(int mode, int64_t iters, float *sink, hipStream_t s) {
  if (iters < 1 || !sink || mode < 0 || mode > 2)
    return fail(HQ_EINVAL, "hq_ceiling_mix", "mode %d, iters %lld", mode, (long long)iters);
  const unsigned grid = (unsigned)device_cus();
  switch (mode) {
    case 0: mix_kernel<0><<<grid, 512, 0, s>>>(iters, sink); break;
    case 1: mix_kernel<1><<<grid, 512, 0, s>>>(iters, sink); break;
    default: mix_kernel<2><<<grid, 512, 0, s>>>(iters, sink); break;
  }
  return check_launch("ceiling_mix");
}

int64_t ceiling_mfma_flops(int64_t iters) { return (int64_t)2 * device_cus() * 4 * iters * 4 * (2 * 32 * 32 * 16); }

}  // namespace hq
