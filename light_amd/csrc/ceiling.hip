// ceiling.hip -- the hardware ceilings the bench reports beside the roofline fractions: a
// streaming read of a device buffer (how much of the 8 TB/s HBM peak a launch of a given size
// can reach, by access order and loads in flight) and a register-only MFMA loop (how much of
// the 2.5 PFLOP/s dense bf16 peak the matrix cores sustain).  Measurement kernels, not part of
// any Light op.
#include "internal.hpp"

namespace hq {

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// Every thread xor-folds DEPTH 16-byte loads per trip, all issued before any is used.
//  ORDER 0 (window): trip j of thread g reads items (j DEPTH + k) G + g -- at any time the grid
//    reads one contiguous window of DEPTH * G * 16 bytes, which moves through the buffer.
//  ORDER 1 (slice): workgroup b reads its own contiguous 1 / gridDim slice front to back,
//    the workgroups' slices spread over the whole buffer (the order of a kernel whose
//    workgroups own whole output chunks).
template <int ORDER, int DEPTH>
__global__ __launch_bounds__(512) void read_kernel(const u32x4 *__restrict__ p, int64_t n, uint32_t *sink) {
  const int64_t G = (int64_t)gridDim.x * blockDim.x;
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
  if (order != 0 && order != 1) return fail(HQ_EINVAL, "hq_ceiling_read", "order %d", order);
  if (depth != 1 && depth != 2 && depth != 4 && depth != 8) return fail(HQ_EINVAL, "hq_ceiling_read", "depth %d", depth);
  const unsigned grid = (unsigned)(2 * device_cus());
  return order == 0 ? launch_read<0>(buf, bytes / 16, depth, sink, grid, s)
                    : launch_read<1>(buf, bytes / 16, depth, sink, grid, s);
}

int launch_ceiling_mfma(int64_t iters, float *sink, hipStream_t s) {
  if (iters < 1 || !sink) return fail(HQ_EINVAL, "hq_ceiling_mfma", "iters %lld", (long long)iters);
  const unsigned grid = (unsigned)(2 * device_cus());
  mfma_kernel<<<grid, 256, 0, s>>>(iters, sink);
  return check_launch("ceiling_mfma");
}

int64_t ceiling_mfma_flops(int64_t iters) { return (int64_t)2 * device_cus() * 4 * iters * 4 * (2 * 32 * 32 * 16); }

}  // namespace hq
