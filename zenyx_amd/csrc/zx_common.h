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
// The bulk arrays (activations, code pools, outputs) are moved in 16-byte vectors.
inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Number of compute units of the current device (cached per device).
int num_cus();

// Bound of one inter-workgroup wait of the cooperative kernels without progress, in
// s_memrealtime ticks (100 MHz); set by zx_set_wait_bound_us.
uint64_t wait_bound_ticks();

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
  // the first conversion fills bytes 0-1 and keeps 2-3 of its `old` operand, which the
  // second one overwrites: any register will do, so no zero has to be materialised
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, __builtin_bit_cast(int, a), false);
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
// in the last place, which no e4m3 code can tell apart (they all encode to +-0).  The
// residual is formed as e = RN(q0 s - x) = -RN(x - q0 s) and the result as
// RN(q0 - e r): the same value, and for s > 0 the zero of x = +-0 keeps its sign (with
// x - q0 s, the sum of the two opposite zeros made -0 / s come out +0; a negative s
// reaches here through quant_scale's sign flip, which makes it positive).
__device__ __forceinline__ float div_by_scale(float x, float s, float r) {
  const float q = x * r;
  const float e = __builtin_fmaf(q, s, -x);
  return __builtin_fmaf(-e, r, q);
}

// FP8 scale from the largest |x| bit pattern of a slab (fp32 bits; > 0x7F800000 is NaN).
__device__ __forceinline__ float scale_from_amax_bits(uint32_t bits) {
  if (bits > 0x7F800000u) return __uint_as_float(0x7FC00000u);
  float a = __uint_as_float(bits);
  a = a < 1e-8f ? 1e-8f : a;
  return a / 448.0f;
}

// Encode parameters of one slab (uniform across the slab).  A finite scale s encodes
// RN_e4m3(RN(x / s)) through div_by_scale(x, s, r = RN(1/s)).  The other cases follow
// the torch evaluation of x / s -> e4m3fn:
//   * s = +inf (the slab holds an infinity and no NaN): a finite x gives a zero with
//     the sign of x, +-inf gives inf/inf = NaN -> 0x7F.  The same arithmetic with s' = 1,
//     r' = 0 gives exactly the signed zeros, and a NaN for +-inf;
//   * s = NaN (the slab holds a NaN): every code is 0x7F; s' = r' = NaN make every
//     value a NaN.
// In those two cases the NaN codes that come out (0x7F or 0xFF: the sign of a NaN result
// depends on the operands) are set to 0x7F by nan_codes_positive.  With a finite scale
// the fix-up is switched off (an overflowing negative quotient keeps its 0xFF), so every
// slab takes the same branch-free path.  A negative scale (a static one) divides -x by
// -s instead (the inputs' sign bits flipped as they are unpacked): the same quotient,
// with the zeros signed as IEEE division signs them (-inf: x / -inf = -sign(x) 0).
struct QuantScale {
  float s, r;
  uint32_t nan_fix;  // 0x80808080 for a non-finite scale, else 0
  uint32_t xflip;    // 0x80008000 for a negative scale (flips two bf16 signs), else 0
};
__device__ __forceinline__ QuantScale quant_scale(float sc) {
  const uint32_t b = __float_as_uint(sc) & 0x7FFFFFFFu;
  const bool neg = sc < 0.0f;  // false for NaN and -0
  QuantScale q;
  q.s = b == 0x7F800000u ? 1.0f : (neg ? -sc : sc);
  q.r = b == 0x7F800000u ? 0.0f : 1.0f / q.s;
  q.nan_fix = b >= 0x7F800000u ? 0x80808080u : 0u;
  q.xflip = neg ? 0x80008000u : 0u;
  return q;
}

// Four e4m3 codes of a non-finite-scale slab (each 0x00, 0x80, 0x7F or 0xFF): with
// fix = 0x80808080 clears bit 7 of every byte whose bit 6 is set, i.e. 0xFF -> 0x7F;
// with fix = 0 returns c.  (c << 1) moves each byte's bit 6 to its bit 7; the whole
// expression is one v_bitop3_b32 after the shift.
__device__ __forceinline__ uint32_t nan_codes_positive(uint32_t c, uint32_t fix) {
  return c & ~((c << 1) & fix);
}

// Four bf16 (two 32-bit words) -> four e4m3 codes.
__device__ __forceinline__ uint32_t quant4(uint32_t u0, uint32_t u1, const QuantScale &q) {
  u0 ^= q.xflip;
  u1 ^= q.xflip;
  return nan_codes_positive(e4m3x4(div_by_scale(bf_lo(u0), q.s, q.r), div_by_scale(bf_hi(u0), q.s, q.r),
                                   div_by_scale(bf_lo(u1), q.s, q.r), div_by_scale(bf_hi(u1), q.s, q.r)),
                            q.nan_fix);
}

// 16 bf16 values (two 16-byte words) -> 16 e4m3 codes (one 16-byte word).
__device__ __forceinline__ uint4 quant16(uint4 a, uint4 b, const QuantScale &q) {
  return make_uint4(quant4(a.x, a.y, q), quant4(a.z, a.w, q), quant4(b.x, b.y, q), quant4(b.z, b.w, q));
}

// 8 bf16 values (one 16-byte word) -> 8 e4m3 codes (one 8-byte word).
__device__ __forceinline__ uint2 quant8(uint4 a, const QuantScale &q) {
  return make_uint2(quant4(a.x, a.y, q), quant4(a.z, a.w, q));
}

// |bf16| bit patterns, two per word, folded into a running packed max (v_pk_max_u16);
// fold16 gives the largest of the two halves.  A NaN pattern (> 0x7F80) wins over
// every number, as torch's amax propagates NaN.
typedef unsigned short zx_u16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pkmax(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(zx_u16x2, a),
                                                                 __builtin_bit_cast(zx_u16x2, b)));
}
__device__ __forceinline__ uint32_t absmax_acc(uint32_t acc, uint4 q) {
  const uint32_t m = 0x7FFF7FFFu;
  return pkmax(pkmax(acc, pkmax(q.x & m, q.y & m)), pkmax(q.z & m, q.w & m));
}
__device__ __forceinline__ uint32_t fold16(uint32_t p) { return max(p & 0xFFFFu, p >> 16); }

// Largest |bf16| bit pattern among 8 / 16 values (a 16-bit magnitude in a uint32).
__device__ __forceinline__ uint32_t absmax8(uint4 q) { return fold16(absmax_acc(0u, q)); }
__device__ __forceinline__ uint32_t absmax16(uint4 a, uint4 b) { return fold16(absmax_acc(absmax_acc(0u, a), b)); }

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
