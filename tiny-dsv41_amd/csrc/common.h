// common.h — shared device helpers and host error plumbing for libdsv41hip.so (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "dsv41_rocm.h"

namespace dsv41 {

// ---------------------------------------------------------------- host errors
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);

#define DSV41_HIP_CHECK(expr)                                                        \
  do {                                                                               \
    hipError_t _e = (expr);                                                          \
    if (_e != hipSuccess)                                                            \
      return ::dsv41::fail(DSV41_E_HIP, std::string(#expr ": ") + hipGetErrorString(_e)); \
  } while (0)

// ------------------------------------------------------------- device helpers
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
__device__ __forceinline__ int wave_min_i(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o));
  return v;
}
// DPP reductions (all 64 lanes must be active).  Within each 16-lane row: swap
// neighbours, swap pairs (quad_perm), rotate by 4 and by 8; the four row results are
// then combined from readlanes, so the returned value is identical in every lane.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  // quad_perm and row_ror only: every lane reads a lane of its own row, so no old value is
  // needed (bound_ctrl), and the move can fold into the instruction that uses it
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ float rl(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_f32<0x4E>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp_f32<0x124>(v));  // row_ror:4
  v = fmaxf(v, dpp_f32<0x128>(v));  // row_ror:8
  return fmaxf(fmaxf(rl(v, 0), rl(v, 16)), fmaxf(rl(v, 32), rl(v, 48)));
}

// inclusive prefix sums across the 64 lanes (all lanes active).  Integer sums are exact in
// any order, so the integer scans go by DPP: shifts of 1, 2, 4 and 8 lanes within each
// 16-lane row (lanes whose source lies before the row read 0), then row 0's total into
// row 1 and row 2's into row 3 (row_bcast:15), then lane 31's into rows 2 and 3
// (row_bcast:31): no LDS crossbar round trips.
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ uint32_t dpp_scan_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROWS, 0xF, false);
}
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ uint64_t dpp_scan_u64(uint64_t v) {
  return ((uint64_t)dpp_scan_u32<CTRL, ROWS>((uint32_t)(v >> 32)) << 32) | dpp_scan_u32<CTRL, ROWS>((uint32_t)v);
}
__device__ __forceinline__ uint64_t wave_incl_scan_u64(uint64_t v, int lane) {
  (void)lane;
  v += dpp_scan_u64<0x111>(v);        // row_shr:1
  v += dpp_scan_u64<0x112>(v);        // row_shr:2
  v += dpp_scan_u64<0x114>(v);        // row_shr:4
  v += dpp_scan_u64<0x118>(v);        // row_shr:8
  v += dpp_scan_u64<0x142, 0xA>(v);   // row_bcast:15 into rows 1 and 3
  v += dpp_scan_u64<0x143, 0xC>(v);   // row_bcast:31 into rows 2 and 3
  return v;
}
__device__ __forceinline__ int wave_incl_scan_i(int v, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    int t = __shfl_up(v, o);
    if (lane >= o) v += t;
  }
  return v;
}

}  // namespace dsv41
