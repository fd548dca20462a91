// zx_attn_common.h -- device helpers shared by the attention kernels that read the FP8
// KV pages (decode: zx_attention.hip, blocks of queries: zx_prefill.hip).
#pragma once

#include "zx_common.h"

namespace zx {

constexpr float ATT_LOG2E = 1.4426950408889634f;

typedef __bf16 att_bf2 __attribute__((ext_vector_type(2)));
// 16 e4m3 codes -> 8 bf16 pairs (exact: every e4m3 value is a bf16 value).
__device__ __forceinline__ void decode16_bf16(uint4 c, uint32_t (&b)[8]) {
  const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    b[2 * i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w[i], 1.0f, false));
    b[2 * i + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w[i], 1.0f, true));
  }
}

template <int CTRL> __device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
// Sum over aligned groups of N lanes inside a 16-lane row, by DPP (quad_perm swaps, then
// half-row and row mirrors, which pair groups whose lanes already agree; every lane of a
// group ends with the result).
template <int N> __device__ __forceinline__ float group_sum(float v) {
  if (N >= 2) v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
  if (N >= 4) v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
  if (N >= 8) v += dpp<0x141>(v);  // row_half_mirror
  if (N >= 16) v += dpp<0x140>(v); // row_mirror
  return v;
}
typedef __bf16 att_bf16x8 __attribute__((ext_vector_type(8)));
typedef float att_f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int att_u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float row16_max(float v) {  // max over lanes 0-15 of each row
  v = fmaxf(v, dpp<0xB1>(v));
  v = fmaxf(v, dpp<0x4E>(v));
  v = fmaxf(v, dpp<0x141>(v));
  return fmaxf(v, dpp<0x140>(v));
}
// Over lanes l, l ^ 16, l ^ 32, l ^ 48 (the four 16-lane rows, lane position kept):
// v_permlane32_swap pairs lane l with l ^ 32 across its two results, v_permlane16_swap
// pairs rows 0/1 and 2/3; both results of a swap together hold the pair's two values.
// (Elements are converted with __uint_as_float: with this compiler __builtin_bit_cast of
// the builtin's vector result reads element 0 for both.)
__device__ __forceinline__ void xrow_pair32(float v, float &x, float &y) {
  auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  x = __uint_as_float(s[0]);
  y = __uint_as_float(s[1]);
}
__device__ __forceinline__ void xrow_pair16(float v, float &x, float &y) {
  auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  x = __uint_as_float(s[0]);
  y = __uint_as_float(s[1]);
}
__device__ __forceinline__ float xrow_max(float v) {
  float x, y;
  xrow_pair32(v, x, y);
  xrow_pair16(fmaxf(x, y), x, y);
  return fmaxf(x, y);
}

}  // namespace zx
