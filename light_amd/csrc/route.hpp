// route.hpp -- device helpers of MoERoute's top-k (ops/moe.go:29-71; Light's CPU TopK is a
// stable descending sort, kernels/cpu/topk.go:52-68): one wave selects the top-k of a row
// by repeated wave-wide maxima of (value, lowest index) keys.  Shared by the routing kernel
// and the MoE decode kernel that routes inside its own workgroups.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hq {
namespace {

// Selection key: the value mapped to an order-preserving u32 (high half; -0 taken as +0,
// as Light's comparisons do) and the complement of the index (low half), so the largest key
// is the largest value at the lowest index.  0 marks a taken or absent slot.
__device__ __forceinline__ uint32_t ord_f32(float v) {
  uint32_t u = __float_as_uint(v == 0.f ? 0.f : v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float unord_f32(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

template <int CTRL>
__device__ __forceinline__ void kmax_dpp(uint32_t &hi, uint32_t &lo) {
  const uint32_t oh = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)hi, CTRL, 0xF, 0xF, false);
  const uint32_t ol = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)lo, CTRL, 0xF, 0xF, false);
  const bool take = oh > hi || (oh == hi && ol > lo);
  hi = take ? oh : hi;
  lo = take ? ol : lo;
}

// Top-k of one row of E <= 64 VPL values by one wave: k rounds of a wave-wide key max (DPP
// within 16-lane rows, then the four row maxima by readlane).  Lane j < topk ends with the
// j-th selection; den is the left-to-right f32 sum of the selected values (uniform).
template <int VPL>
__device__ void topk_row(const float *__restrict__ row, int E, int topk, int lane, float &sel_v, int &sel_i,
                         float &den) {
  uint32_t kh[VPL], kl[VPL];
#pragma unroll
  for (int j = 0; j < VPL; j++) {
    const int e = lane + 64 * j;
    kh[j] = e < E ? ord_f32(row[e]) : 0u;
    kl[j] = e < E ? 0xffffffffu - (uint32_t)e : 0u;
  }
  sel_v = 0.f;
  sel_i = -1;
  den = 0.f;
  for (int r = 0; r < topk; r++) {
    uint32_t hi = kh[0], lo = kl[0];
#pragma unroll
    for (int j = 1; j < VPL; j++) {
      const bool take = kh[j] > hi || (kh[j] == hi && kl[j] > lo);
      hi = take ? kh[j] : hi;
      lo = take ? kl[j] : lo;
    }
    kmax_dpp<0xB1>(hi, lo);   // quad_perm [1,0,3,2]
    kmax_dpp<0x4E>(hi, lo);   // quad_perm [2,3,0,1]
    kmax_dpp<0x141>(hi, lo);  // row_half_mirror
    kmax_dpp<0x140>(hi, lo);  // row_mirror
    uint32_t bh = (uint32_t)__builtin_amdgcn_readlane((int)hi, 0), bl = (uint32_t)__builtin_amdgcn_readlane((int)lo, 0);
#pragma unroll
    for (int q = 16; q < 64; q += 16) {
      const uint32_t h2 = (uint32_t)__builtin_amdgcn_readlane((int)hi, q);
      const uint32_t l2 = (uint32_t)__builtin_amdgcn_readlane((int)lo, q);
      const bool take = h2 > bh || (h2 == bh && l2 > bl);
      bh = take ? h2 : bh;
      bl = take ? l2 : bl;
    }
    const int idx = (int)(0xffffffffu - bl);
    const float v = unord_f32(bh);
    den = __fadd_rn(den, v);  // Sum over the selected values in slot order
#pragma unroll
    for (int j = 0; j < VPL; j++)
      if (lane + 64 * j == idx) kh[j] = kl[j] = 0u;
    if (lane == r) {
      sel_v = v;
      sel_i = idx;
    }
  }
}

// Top-k of one row for any E <= 1024 (values per lane chosen at run time).
__device__ __forceinline__ void topk_row_any(const float *__restrict__ row, int E, int topk, int lane, float &sv,
                                             int &si, float &den) {
  if (E <= 64)
    topk_row<1>(row, E, topk, lane, sv, si, den);
  else if (E <= 128)
    topk_row<2>(row, E, topk, lane, sv, si, den);
  else if (E <= 256)
    topk_row<4>(row, E, topk, lane, sv, si, den);
  else if (E <= 512)
    topk_row<8>(row, E, topk, lane, sv, si, den);
  else
    topk_row<16>(row, E, topk, lane, sv, si, den);
}

}  // namespace
}  // namespace hq
