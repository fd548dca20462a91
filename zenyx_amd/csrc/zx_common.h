// zx_common.h -- shared host/device helpers of libzenyx_kv.so (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/zenyx_kv.h"

namespace zx {

// ------------------------------------------------------------------ host side

// Records a message for zx_last_error() and returns `code`.
int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
// Clears the thread's message; entry points call it first.
void clear_error();

inline hipStream_t as_stream(zx_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// Checks the launch that was just enqueued.
int check_launch(const char *what);

#define ZX_TRY_HIP(call)                                                                  \
  do {                                                                                    \
    hipError_t e_ = (call);                                                               \
    if (e_ != hipSuccess) return ::zx::fail(ZX_ERR_HIP, "%s: %s", #call, hipGetErrorString(e_)); \
  } while (0)

#define ZX_REQUIRE(cond, ...)                                                             \
  do {                                                                                    \
    if (!(cond)) return ::zx::fail(ZX_ERR_INVALID, __VA_ARGS__);                          \
  } while (0)

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Number of compute units of the current device (cached per device).
int num_cus();

// ------------------------------------------------------------------ device side

// bf16 halves of a 32-bit word as exact fp32 values.
__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// Two fp32 -> packed bf16 pair, round-to-nearest-even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  bf16x2_t v;
  v[0] = (__bf16)lo;
  v[1] = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, v);
}

// Four fp32 -> four OCP e4m3fn codes (byte k holds value k), nearest-even, via
// v_cvt_pk_fp8_f32.  Callers guarantee |v| <= 464 or handle larger values themselves.
__device__ __forceinline__ uint32_t e4m3x4(float a, float b, float c, float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return (uint32_t)w;
}

// Exact decode of the four e4m3fn codes in a word (v_cvt_pk_f32_fp8).
__device__ __forceinline__ void e4m3x4_decode(uint32_t w, float &a, float &b, float &c, float &d) {
  auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
  auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
  a = lo[0];
  b = lo[1];
  c = hi[0];
  d = hi[1];
}

// Correctly rounded x / s given r = RN(1/s) (Markstein's FMA correction: with r within
// half an ulp of 1/s and q0 within one ulp of x/s, RN(q0 + RN(x - q0*s)*r) = RN(x/s)).
// Valid for finite normal s and finite x; quotients below 2^-126 may differ from RN(x/s)
// in the last place, which no e4m3 code can tell apart (they all encode to +-0).
__device__ __forceinline__ float div_by_scale(float x, float s, float r) {
  float q = x * r;
  float e = __builtin_fmaf(-q, s, x);
  return __builtin_fmaf(e, r, q);
}

// FP8 scale from the largest |x| bit pattern of a slab (fp32 bits; > 0x7F800000 is NaN).
__device__ __forceinline__ float scale_from_amax_bits(uint32_t bits) {
  if (bits > 0x7F800000u) return __uint_as_float(0x7FC00000u);
  float a = __uint_as_float(bits);
  a = a < 1e-8f ? 1e-8f : a;
  return a / 448.0f;
}

// Slab mode from its scale: 0 finite (normal path), 1 +inf, 2 NaN.
__device__ __forceinline__ int scale_mode(float s) {
  uint32_t b = __float_as_uint(s) & 0x7FFFFFFFu;
  return b < 0x7F800000u ? 0 : (b == 0x7F800000u ? 1 : 2);
}

// Code of one value in a slab whose scale is not finite (mode 1 or 2).
__device__ __forceinline__ uint32_t code_nonfinite(uint32_t xbits16, int mode) {
  if (mode == 2) return 0x7Fu;
  uint32_t mag = xbits16 & 0x7FFFu;
  if (mag >= 0x7F80u) return 0x7Fu;  // +-inf or NaN input: inf/inf or NaN
  return (xbits16 >> 8) & 0x80u;     // finite / inf = signed zero
}

// 16 bf16 values (two 16-byte words) -> 16 e4m3 codes (one 16-byte word).
__device__ __forceinline__ uint4 quant16(uint4 a, uint4 b, float s, float r, int mode) {
  uint4 out;
  if (mode == 0) {
    uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    uint32_t o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      uint32_t u0 = w[2 * k], u1 = w[2 * k + 1];
      o[k] = e4m3x4(div_by_scale(bf_lo(u0), s, r), div_by_scale(bf_hi(u0), s, r),
                    div_by_scale(bf_lo(u1), s, r), div_by_scale(bf_hi(u1), s, r));
    }
    out = make_uint4(o[0], o[1], o[2], o[3]);
  } else {
    uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    uint32_t o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      uint32_t u0 = w[2 * k], u1 = w[2 * k + 1];
      o[k] = code_nonfinite(u0 & 0xFFFFu, mode) | (code_nonfinite(u0 >> 16, mode) << 8) |
             (code_nonfinite(u1 & 0xFFFFu, mode) << 16) | (code_nonfinite(u1 >> 16, mode) << 24);
    }
    out = make_uint4(o[0], o[1], o[2], o[3]);
  }
  return out;
}

// 8 bf16 values (one 16-byte word) -> 8 e4m3 codes (one 8-byte word).  Branch-free:
// the non-finite-scale codes are computed alongside and selected, so callers that keep
// several loads in flight see straight-line code.
__device__ __forceinline__ uint2 quant8(uint4 a, float s, float r, int mode) {
  uint32_t w[4] = {a.x, a.y, a.z, a.w};
  uint32_t o[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    uint32_t u0 = w[2 * k], u1 = w[2 * k + 1];
    uint32_t fin = e4m3x4(div_by_scale(bf_lo(u0), s, r), div_by_scale(bf_hi(u0), s, r),
                          div_by_scale(bf_lo(u1), s, r), div_by_scale(bf_hi(u1), s, r));
    uint32_t nf = code_nonfinite(u0 & 0xFFFFu, mode) | (code_nonfinite(u0 >> 16, mode) << 8) |
                  (code_nonfinite(u1 & 0xFFFFu, mode) << 16) | (code_nonfinite(u1 >> 16, mode) << 24);
    o[k] = mode == 0 ? fin : nf;
  }
  return make_uint2(o[0], o[1]);
}

// Largest |bf16| bit pattern among 8 values.
__device__ __forceinline__ uint32_t absmax8(uint4 q) {
  uint32_t m = 0;
  uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    uint32_t u = w[k] & 0x7FFF7FFFu;
    m = max(m, max(u & 0xFFFFu, u >> 16));
  }
  return m;
}

// Largest |bf16| bit pattern among 16 values (as a 16-bit magnitude in a uint32).
__device__ __forceinline__ uint32_t absmax16(uint4 a, uint4 b) {
  uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  uint32_t m = 0;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    uint32_t u = w[k] & 0x7FFF7FFFu;
    m = max(m, max(u & 0xFFFFu, u >> 16));
  }
  return m;
}

// 16 e4m3 codes (one 16-byte word) -> 16 bf16 values (two 16-byte words).
__device__ __forceinline__ void dequant16(uint4 c, float s, uint4 &o0, uint4 &o1) {
  uint32_t w[4] = {c.x, c.y, c.z, c.w};
  uint32_t o[8];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float a, b, cc, d;
    e4m3x4_decode(w[k], a, b, cc, d);
    o[2 * k] = pack_bf16(a * s, b * s);
    o[2 * k + 1] = pack_bf16(cc * s, d * s);
  }
  o0 = make_uint4(o[0], o[1], o[2], o[3]);
  o1 = make_uint4(o[4], o[5], o[6], o[7]);
}

// Wavefront max-reduction over aligned groups of `width` lanes (power of two <= 64).
__device__ __forceinline__ uint32_t group_max(uint32_t v, int width) {
  for (int off = 1; off < width; off <<= 1) v = max(v, (uint32_t)__shfl_xor((int)v, off, 64));
  return v;
}

}  // namespace zx
