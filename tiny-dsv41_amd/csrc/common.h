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
// Maxima of quiet operands (all 64 lanes active).  In IEEE mode the compiler's fmaxf first
// turns a signaling NaN into a quiet one, a v_max per operand that also keeps the DPP move
// from folding into the max.  For operands that are not signaling NaNs (fmaxf and arithmetic
// results, or values passed through __builtin_canonicalizef) a plain v_max_f32 returns
// fmaxf's value, and maxima of such values are quiet again.  A DPP or permlane read of a
// register that the instruction before wrote needs two wait states (s_nop 1).  Each block
// ends with one too: the compiler does not count the asm as the VALU write that a later
// DPP read of its result must wait for.
//   row_max_q: every lane gets its 16-lane row's maximum (quad_perm swaps, row_ror 4, 8);
//   pair_max_q: rows 0, 1 and rows 2, 3 combined (v_permlane16_swap), so every lane of
//     lanes 0-31 holds their maximum and every lane of 32-63 theirs;
//   halves_max_q: the two 32-lane halves combined (v_permlane32_swap).
__device__ __forceinline__ float row_max_q(float v) {
  asm("s_nop 1\n\t"
      "v_max_f32_dpp %0, %0, %0 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
      "s_nop 1\n\t"
      "v_max_f32_dpp %0, %0, %0 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
      "s_nop 1\n\t"
      "v_max_f32_dpp %0, %0, %0 row_ror:4 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
      "s_nop 1\n\t"
      "v_max_f32_dpp %0, %0, %0 row_ror:8 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
      "s_nop 1"
      : "+v"(v));
  return v;
}
__device__ __forceinline__ float pair_max_q(float v) {
  float w = v;
  asm("s_nop 1\n\t"
      "v_permlane16_swap_b32 %0, %1\n\t"
      "v_max_f32 %0, %0, %1\n\t"
      "s_nop 1"
      : "+v"(v), "+v"(w));
  return v;
}
__device__ __forceinline__ float halves_max_q(float v) {
  float w = v;
  asm("s_nop 1\n\t"
      "v_permlane32_swap_b32 %0, %1\n\t"
      "v_max_f32 %0, %0, %1\n\t"
      "s_nop 1"
      : "+v"(v), "+v"(w));
  return v;
}
// fmaxf over the 64 lanes, the same value in every lane
__device__ __forceinline__ float wave_max_dpp(float v) {
  return halves_max_q(pair_max_q(row_max_q(__builtin_canonicalizef(v))));
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
__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t v) {
  v += dpp_scan_u32<0x111>(v);        // row_shr:1
  v += dpp_scan_u32<0x112>(v);        // row_shr:2
  v += dpp_scan_u32<0x114>(v);        // row_shr:4
  v += dpp_scan_u32<0x118>(v);        // row_shr:8
  v += dpp_scan_u32<0x142, 0xA>(v);   // row_bcast:15 into rows 1 and 3
  v += dpp_scan_u32<0x143, 0xC>(v);   // row_bcast:31 into rows 2 and 3
  return v;
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
// fp64 sum over the 64 lanes (all lanes active), the same value in every lane: the DPP
// inclusive scan above on the double's bits (lanes whose source lies outside read +0.0),
// then lane 63's total.  Its order is fixed, so the sum is deterministic.
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ double dpp_scan_d(double v) {
  return __builtin_bit_cast(double, dpp_scan_u64<CTRL, ROWS>(__builtin_bit_cast(uint64_t, v)));
}
__device__ __forceinline__ double wave_total_d(double v) {
  v += dpp_scan_d<0x111>(v);        // row_shr:1
  v += dpp_scan_d<0x112>(v);        // row_shr:2
  v += dpp_scan_d<0x114>(v);        // row_shr:4
  v += dpp_scan_d<0x118>(v);        // row_shr:8
  v += dpp_scan_d<0x142, 0xA>(v);   // row_bcast:15 into rows 1 and 3
  v += dpp_scan_d<0x143, 0xC>(v);   // row_bcast:31 into rows 2 and 3
  const uint64_t b = __builtin_bit_cast(uint64_t, v);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), 63);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, 63);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
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
