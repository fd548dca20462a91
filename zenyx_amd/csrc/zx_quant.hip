// zx_quant.hip -- quantisation kernels of libzenyx_kv.so (gfx950):
//   * legacy per-tensor int8 (zenyx/streaming/precision.py:8-16)
//   * FP8 e4m3fn per-(outer, head) quant / dequant (FP8KVQuantizer, README.md:157, 329)
//   * per-(layer, kv, head) scales and the paged append with fused quant
// Every kernel streams 16-byte vectors; all are HBM-bound (no MFMA: nothing here is a
// contraction).
#include <mutex>

#include "zx_internal.h"

namespace zx {

__global__ void fill_u32_kernel(uint32_t *p, int64_t n, uint32_t v) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

int fill_u32(uint32_t *p, int64_t n, uint32_t v, hipStream_t st) {
  if (n <= 0) return ZX_OK;
  fill_u32_kernel<<<(unsigned)ceil_div(n, 256), 256, 0, st>>>(p, n, v);
  return check_launch("fill_u32");
}

// Block-wide max of one uint32 per thread; result valid in every thread.
__device__ __forceinline__ uint32_t block_max(uint32_t v) {
  __shared__ uint32_t red[16];
  v = group_max(v, 64);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) red[wid] = v;
  __syncthreads();
  const int nw = (blockDim.x + 63) >> 6;
  uint32_t m = 0;
  for (int i = 0; i < nw; ++i) m = max(m, red[i]);
  __syncthreads();
  return m;
}

// ================================================================== legacy int8

typedef unsigned int nt_u4 __attribute__((ext_vector_type(4)));  // for the nontemporal builtins

// Storage dtypes of the legacy path: magnitude mask and "is NaN" threshold of the raw bits.
template <int DT> struct Dt;
template <> struct Dt<ZX_BF16> {
  __device__ static float load(const void *x, int64_t i) {
    return __uint_as_float((uint32_t)((const uint16_t *)x)[i] << 16);
  }
  __device__ static uint32_t absbits(const void *x, int64_t i) { return ((const uint16_t *)x)[i] & 0x7FFFu; }
  __device__ static float from_absbits(uint32_t b) { return __uint_as_float(b << 16); }
  __device__ static float round(float v) { return (float)(__bf16)v; }
  __device__ static void store(void *p, float v) {
    __bf16 h = (__bf16)v;
    *(uint16_t *)p = __builtin_bit_cast(uint16_t, h);
  }
};
template <> struct Dt<ZX_F16> {
  __device__ static float load(const void *x, int64_t i) {
    return (float)__builtin_bit_cast(_Float16, ((const uint16_t *)x)[i]);
  }
  __device__ static uint32_t absbits(const void *x, int64_t i) { return ((const uint16_t *)x)[i] & 0x7FFFu; }
  __device__ static float from_absbits(uint32_t b) { return (float)__builtin_bit_cast(_Float16, (uint16_t)b); }
  __device__ static float round(float v) { return (float)(_Float16)v; }
  __device__ static void store(void *p, float v) {
    _Float16 h = (_Float16)v;
    *(uint16_t *)p = __builtin_bit_cast(uint16_t, h);
  }
};
template <> struct Dt<ZX_F32> {
  __device__ static float load(const void *x, int64_t i) { return ((const float *)x)[i]; }
  __device__ static uint32_t absbits(const void *x, int64_t i) {
    return ((const uint32_t *)x)[i] & 0x7FFFFFFFu;
  }
  __device__ static float from_absbits(uint32_t b) { return __uint_as_float(b); }
  __device__ static float round(float v) { return v; }
  __device__ static void store(void *p, float v) { *(float *)p = v; }
};

// For all three formats the integer order of |x| bit patterns is the float order, with
// NaN patterns above infinity, so an integer max is the float amax (NaN-propagating).
// Quantisation follows precision.py:10-11 with torch's CPU arithmetic: every intermediate
// is rounded to the storage dtype, division is IEEE fp32 division, round() is
// half-to-even.

// The same functions applied to n_slabs equal slabs in one launch (one scale per slab;
// the per-tensor entry points are the case n_slabs = 1): grid.y = slab, grid.x blocks
// stride through the slab.  VEC: 16-byte lane loads (W = 8 16-bit or 4 fp32 elements;
// int8 codes stored as W-byte words, bf16 dequant output as 16-byte words), which needs
// 16-byte aligned slabs; a slab's last n % W elements go element by element.
constexpr int LEGACY_U = 4;  // vectors per thread per round in the vector loops
// A thread's LEGACY_U vectors per round: with a grid of one tile per block (one round),
// block b takes vectors [b, b + 1) x LEGACY_U x 256 and lane t of it vectors t + 256 u;
// when every thread has at least 8 rounds of work, each wave takes a contiguous chunk of
// LEGACY_U x 64 vectors per round (its loads are adjacent 1 KiB blocks: 12% faster on a
// 1 Gi-element tensor than loads a grid stride apart); in between (many small slabs) the
// vectors are a grid stride apart, which keeps the last round spread over all threads.
struct LegacyRounds {
  int64_t first, step_u, round;
  __device__ LegacyRounds(int64_t t0, int64_t stride, int64_t nv) {
    if (nv <= LEGACY_U * stride) {  // one round: each block a contiguous tile of LEGACY_U x 256 vectors
      first = (t0 >> 8) * (256 * LEGACY_U) + (t0 & 255);
      step_u = 256;
      round = LEGACY_U * stride;
    } else if (nv >= 8 * LEGACY_U * stride) {
      first = (t0 >> 6) * LEGACY_U * 64 + (t0 & 63);
      step_u = 64;
      round = (stride >> 6) * LEGACY_U * 64;
    } else {
      first = t0;
      step_u = stride;
      round = LEGACY_U * stride;
    }
  }
};
template <int DT> struct LegacyVec {
  static constexpr int W = DT == ZX_F32 ? 4 : 8;
  static constexpr int ES = DT == ZX_F32 ? 4 : 2;
  __device__ static uint32_t absmax(uint4 v) {
    if constexpr (DT == ZX_F32) {
      return max(max(v.x & 0x7FFFFFFFu, v.y & 0x7FFFFFFFu), max(v.z & 0x7FFFFFFFu, v.w & 0x7FFFFFFFu));
    } else {
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
      uint32_t m = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) m = max(m, max(w[i] & 0x7FFFu, (w[i] >> 16) & 0x7FFFu));
      return m;
    }
  }
  __device__ static float elem(uint4 v, int j) {  // element j of the vector, as float
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    if constexpr (DT == ZX_F32) {
      return __uint_as_float(w[j]);
    } else {
      const uint16_t h = (uint16_t)(w[j >> 1] >> (16 * (j & 1)));
      return Dt<DT>::load(&h, 0);
    }
  }
};

// FAST: the quotient from r = 1 / s and one Markstein correction instead of a division
// (q0 = x r, e = fma(-q0, s, x), q = fma(e, r, q0); q0 itself when |q0| >= 65536, where the
// code saturates).  For bf16 / f16 input it gives the same int8 code as IEEE division for
// every input and every finite scale the quantiser can produce from such an amax: checked
// exhaustively on the CPU (2,886,336,512 pairs).  fp32 input and non-finite scales divide.
template <int DT, bool FAST>
__device__ __forceinline__ int8_t legacy_code(float xv, float s, float r) {
  float qv;
  if constexpr (FAST) {
    const float q0 = xv * r;
    qv = fabsf(q0) < 65536.0f ? __builtin_fmaf(__builtin_fmaf(-q0, s, xv), r, q0) : q0;
  } else {
    qv = xv / s;
  }
  const float v = __builtin_rintf(Dt<DT>::round(qv));
  return v != v ? (int8_t)0 : (int8_t)fminf(fmaxf(v, -127.0f), 127.0f);  // NaN -> 0, as torch CPU
}

// Four codes (one word) of the fast path, for bf16 / f16 slabs with a finite scale, where
// every input obeys |x| <= amax, so every quotient is finite and below ~170: the quotient
// as in legacy_code with no range guard, rounded to the storage dtype, clamped to +-127
// (v_med3), then rounded to an integer by adding 1.5 * 2^23 (round half to even, as
// rint; the low byte of the sum is the two's-complement code).  The same codes as
// legacy_code for every reachable (scale, x) pair: checked exhaustively on the CPU
// (zxo_legacy_fast_check).
template <int DT>
__device__ __forceinline__ uint32_t legacy_fast4(uint32_t u0, uint32_t u1, float s, float r) {
  const uint32_t w[2] = {u0, u1};
  uint32_t b[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint16_t h = (uint16_t)(w[j >> 1] >> (16 * (j & 1)));
    const float x = Dt<DT>::load(&h, 0);
    const float q0 = x * r;
    const float q = __builtin_fmaf(__builtin_fmaf(-q0, s, x), r, q0);
    b[j] = __float_as_uint(__builtin_amdgcn_fmed3f(Dt<DT>::round(q), -127.0f, 127.0f) + 12582912.0f);
  }
  return __builtin_amdgcn_perm(b[1], b[0], 0x0c0c0400u) | __builtin_amdgcn_perm(b[3], b[2], 0x04000c0cu);
}

// NT: nontemporal loads, for inputs of 256 MiB and more (5% at 1 Gi bf16 elements); below
// that the default policy leaves the input in the Infinity Cache for the quant pass (7% at
// configs[0]'s 151 MB).
template <int DT, bool VEC, bool NT>
__global__ void legacy_amax_slabs_kernel(const void *x, int64_t slab_len, uint32_t *amax_bits) {
  using V = LegacyVec<DT>;
  const int64_t base = (int64_t)blockIdx.y * slab_len;
  const int64_t t0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x, stride = (int64_t)gridDim.x * blockDim.x;
  uint32_t m = 0;
  int64_t done = 0;
  if constexpr (VEC) {
    const uint4 *xv = reinterpret_cast<const uint4 *>((const char *)x + base * V::ES);
    const int64_t nv = slab_len / V::W;
    const LegacyRounds lr(t0, stride, nv);
    for (int64_t v0 = lr.first; v0 < nv; v0 += lr.round) {
      uint4 xw[LEGACY_U];
#pragma unroll
      for (int u = 0; u < LEGACY_U; ++u) {
        const int64_t v = v0 + u * lr.step_u;
        if (v < nv) {
          if constexpr (NT) {
            const nt_u4 t = __builtin_nontemporal_load(reinterpret_cast<const nt_u4 *>(xv) + v);
            xw[u] = make_uint4(t.x, t.y, t.z, t.w);
          } else {
            xw[u] = xv[v];
          }
        } else {
          xw[u] = make_uint4(0u, 0u, 0u, 0u);
        }
      }
#pragma unroll
      for (int u = 0; u < LEGACY_U; ++u) m = max(m, V::absmax(xw[u]));
    }
    done = nv * V::W;
  }
  for (int64_t i = done + t0; i < slab_len; i += stride) m = max(m, Dt<DT>::absbits(x, base + i));
  m = block_max(m);
  if (threadIdx.x == 0) atomicMax(&amax_bits[blockIdx.y], m);
}

template <int DT, bool VEC, bool FAST>
__device__ __forceinline__ void legacy_quant_range(const void *x, int64_t base, int64_t slab_len, int8_t *q, float s,
                                                   float r) {
  using V = LegacyVec<DT>;
  const int64_t t0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x, stride = (int64_t)gridDim.x * blockDim.x;
  int64_t done = 0;
  if constexpr (VEC) {
    const uint4 *xv = reinterpret_cast<const uint4 *>((const char *)x + base * V::ES);
    const int64_t nv = slab_len / V::W;
    // LEGACY_U vectors per thread per round, all loaded before any is encoded (loads in
    // flight); vectors past nv load nothing and store nothing
    const LegacyRounds lr(t0, stride, nv);
    for (int64_t v0 = lr.first; v0 < nv; v0 += lr.round) {
      uint4 xw[LEGACY_U];
#pragma unroll
      for (int u = 0; u < LEGACY_U; ++u) {
        const int64_t v = v0 + u * lr.step_u;
        xw[u] = v < nv ? xv[v] : make_uint4(0u, 0u, 0u, 0u);
      }
#pragma unroll
      for (int u = 0; u < LEGACY_U; ++u) {
        const int64_t v = v0 + u * lr.step_u;
        uint32_t c[V::W / 4];
#pragma unroll
        for (int k = 0; k < V::W / 4; ++k) {
          if constexpr (FAST && DT != ZX_F32) {
            const uint32_t xw4[4] = {xw[u].x, xw[u].y, xw[u].z, xw[u].w};
            c[k] = legacy_fast4<DT>(xw4[2 * k], xw4[2 * k + 1], s, r);
          } else {
            uint32_t w = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j)
              w |= (uint32_t)(uint8_t)legacy_code<DT, FAST>(V::elem(xw[u], 4 * k + j), s, r) << (8 * j);
            c[k] = w;
          }
        }
        if (v < nv) {
          if constexpr (V::W == 8)
            reinterpret_cast<uint2 *>(q + base)[v] = make_uint2(c[0], c[1]);
          else
            reinterpret_cast<uint32_t *>(q + base)[v] = c[0];
        }
      }
    }
    done = nv * V::W;
  }
  for (int64_t i = done + t0; i < slab_len; i += stride)
    q[base + i] = legacy_code<DT, FAST>(Dt<DT>::load(x, base + i), s, r);
}

template <int DT, bool VEC>
__global__ void legacy_quant_slabs_kernel(const void *x, int64_t slab_len, const uint32_t *amax_bits, int8_t *q,
                                          void *scales) {
  using V = LegacyVec<DT>;
  const int64_t base = (int64_t)blockIdx.y * slab_len;
  float a = Dt<DT>::from_absbits(amax_bits[blockIdx.y]);
  const float lo = Dt<DT>::round(1e-8f);
  if (a < lo) a = lo;
  const float s = Dt<DT>::round(a / 127.0f);
  if (blockIdx.x == 0 && threadIdx.x == 0) Dt<DT>::store((char *)scales + V::ES * (int64_t)blockIdx.y, s);
  const float r = 1.0f / s;
  if (DT != ZX_F32 && __builtin_isfinite(s) && __builtin_isfinite(r))  // uniform per slab
    legacy_quant_range<DT, VEC, DT != ZX_F32>(x, base, slab_len, q, s, r);
  else
    legacy_quant_range<DT, VEC, false>(x, base, slab_len, q, s, r);
}

template <int DT, bool VEC>
__global__ void legacy_dequant_slabs_kernel(const int8_t *q, const void *scales, int64_t slab_len, uint16_t *y) {
  const int64_t base = (int64_t)blockIdx.y * slab_len;
  const float s = Dt<DT>::load(scales, blockIdx.y);
  const int64_t t0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x, stride = (int64_t)gridDim.x * blockDim.x;
  int64_t done = 0;
  if constexpr (VEC) {  // 8 codes -> 8 bf16 per lane
    const uint2 *qv = reinterpret_cast<const uint2 *>(q + base);
    uint4 *yv = reinterpret_cast<uint4 *>(y + base);
    const int64_t nv = slab_len / 8;
    const LegacyRounds lr(t0, stride, nv);
    for (int64_t v0 = lr.first; v0 < nv; v0 += lr.round) {
      uint2 cw[LEGACY_U];
#pragma unroll
      for (int u = 0; u < LEGACY_U; ++u) {
        const int64_t v = v0 + u * lr.step_u;
        cw[u] = v < nv ? qv[v] : make_uint2(0u, 0u);
      }
#pragma unroll
      for (int u = 0; u < LEGACY_U; ++u) {
        const int64_t v = v0 + u * lr.step_u;
        uint32_t o[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t w = k < 2 ? cw[u].x : cw[u].y;
          const int8_t c0 = (int8_t)(w >> (16 * (k & 1))), c1 = (int8_t)(w >> (16 * (k & 1) + 8));
          o[k] = pack_bf16((float)c0 * s, (float)c1 * s);
        }
        typedef unsigned int lq_v4u __attribute__((ext_vector_type(4)));
        if (v < nv) __builtin_nontemporal_store(lq_v4u{o[0], o[1], o[2], o[3]}, reinterpret_cast<lq_v4u *>(yv + v));
      }
    }
    done = nv * 8;
  }
  for (int64_t i = done + t0; i < slab_len; i += stride) {
    __bf16 h = (__bf16)((float)q[base + i] * s);
    y[base + i] = __builtin_bit_cast(uint16_t, h);
  }
}

// ================================================================== FP8 per (outer, head)

// Blocks own chunks of CHUNK_VEC 16-element vectors inside one run of one slab.
constexpr int QH_THREADS = 256;
constexpr int QH_VEC_PER_THREAD = 4;
constexpr int64_t QH_CHUNK_VEC = QH_THREADS * QH_VEC_PER_THREAD;

struct HeadsGeom {
  int64_t n_batch, n_heads, vec_per_run, chunks_per_run;
  __device__ void locate(int64_t block, int64_t &run_idx, int64_t &chunk, int64_t &slab) const {
    run_idx = block / chunks_per_run;
    chunk = block - run_idx * chunks_per_run;
    const int64_t h = run_idx % n_heads;
    const int64_t o = run_idx / (n_heads * n_batch);
    slab = o * n_heads + h;
  }
};

// Two-pass kernels: a block is one chunk of a run (2 QH_CHUNK_VEC 16-byte input vectors),
// lane t takes vectors h = chunk 2 QH_CHUNK_VEC + k QH_THREADS + t (each load instruction
// of a wave reads 1 KiB contiguously), and every load is issued before any is used: an
// index past the run is clamped into it and its value dropped.  (With a load, its use and
// a store per step the compiler kept one load in flight per thread: the stores might
// alias the next load.)
constexpr int QH_H = 2 * QH_VEC_PER_THREAD;  // 16-byte input vectors per thread

__global__ void __launch_bounds__(QH_THREADS)
heads_amax_kernel(const uint4 *x, HeadsGeom g, uint32_t *amax_bits) {
  int64_t run_idx, chunk, slab;
  g.locate(blockIdx.x, run_idx, chunk, slab);
  const uint4 *base = x + run_idx * g.vec_per_run * 2;
  const int64_t n_half = 2 * g.vec_per_run, h0 = chunk * 2 * QH_CHUNK_VEC + threadIdx.x;
  uint4 v[QH_H];
#pragma unroll
  for (int k = 0; k < QH_H; ++k) {
    const int64_t h = h0 + k * QH_THREADS;
    v[k] = base[h < n_half ? h : 0];
  }
  uint32_t acc = 0;
#pragma unroll
  for (int k = 0; k < QH_H; ++k)
    if (h0 + k * QH_THREADS < n_half) acc = absmax_acc(acc, v[k]);
  const uint32_t m = block_max(fold16(acc));
  if (threadIdx.x == 0) atomicMax(&amax_bits[slab], m << 16);
}

__global__ void finalize_scales_kernel(float *scales, int64_t n) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) scales[i] = scale_from_amax_bits(__float_as_uint(scales[i]));
}

__global__ void __launch_bounds__(QH_THREADS)
heads_quant_kernel(const uint4 *x, HeadsGeom g, const float *scales, uint4 *codes) {
  int64_t run_idx, chunk, slab;
  g.locate(blockIdx.x, run_idx, chunk, slab);
  const QuantScale q = quant_scale(scales[slab]);
  const uint4 *src = x + run_idx * g.vec_per_run * 2;
  uint2 *dst = reinterpret_cast<uint2 *>(codes + run_idx * g.vec_per_run);  // 8 codes per input vector
  const int64_t n_half = 2 * g.vec_per_run, h0 = chunk * 2 * QH_CHUNK_VEC + threadIdx.x;
  uint4 v[QH_H];
#pragma unroll
  for (int k = 0; k < QH_H; ++k) {
    const int64_t h = h0 + k * QH_THREADS;
    v[k] = src[h < n_half ? h : 0];
  }
#pragma unroll
  for (int k = 0; k < QH_H; ++k) {
    const int64_t h = h0 + k * QH_THREADS;
    if (h < n_half) dst[h] = quant8(v[k], q);
  }
}

// 8 codes -> 8 bf16 (16 bytes)
__device__ __forceinline__ uint4 dequant8(uint2 c, float s) {
  float a, b, cc, d, e, f, gg, h;
  e4m3x4_decode(c.x, a, b, cc, d);
  e4m3x4_decode(c.y, e, f, gg, h);
  return make_uint4(pack_bf16(a * s, b * s), pack_bf16(cc * s, d * s), pack_bf16(e * s, f * s),
                    pack_bf16(gg * s, h * s));
}
// Every lane loads 8 codes and stores their 16 bytes, so that each store instruction of a
// wave writes 1 KiB of whole lines (storing 32 bytes per lane as two 16-byte halves wrote
// every line by halves: 0.635 against 0.550 ms on 1 Gi elements); the stores are
// nontemporal, the loads not (the codes of a recent quantisation may still be in the cache)
// VPT: 16-byte code vectors per thread (two 8-code halves each); the dequant takes half the
// quantiser's chunk (3% faster at 1 Gi elements, where the quantiser's amax pass
// prefers the larger chunk: fewer blocks, fewer atomics)
constexpr int QH_DQ_VPT = 2;
template <int VPT>
__global__ void __launch_bounds__(QH_THREADS)
heads_dequant_kernel(const uint4 *codes, HeadsGeom g, const float *scales, uint4 *y) {
  int64_t run_idx, chunk, slab;
  g.locate(blockIdx.x, run_idx, chunk, slab);
  const float s = scales[slab];
  const uint2 *src = reinterpret_cast<const uint2 *>(codes + run_idx * g.vec_per_run);
  nt_u4 *dst = reinterpret_cast<nt_u4 *>(y + run_idx * g.vec_per_run * 2);
  constexpr int NH = 2 * VPT;  // 8-code halves per thread
  const int64_t n_half = 2 * g.vec_per_run, h0 = chunk * 2 * (QH_THREADS * VPT) + threadIdx.x;
  uint2 c[NH];  // every load issued before any store (see the two-pass kernels)
#pragma unroll
  for (int k = 0; k < NH; ++k) {
    const int64_t h = h0 + k * QH_THREADS;
    c[k] = src[h < n_half ? h : 0];
  }
#pragma unroll
  for (int k = 0; k < NH; ++k) {
    const int64_t h = h0 + k * QH_THREADS;
    if (h < n_half) {
      const uint4 o = dequant8(c[k], s);
      __builtin_nontemporal_store(nt_u4{o.x, o.y, o.z, o.w}, dst + h);
    }
  }
}

static int heads_geom(int64_t n_outer, int64_t n_batch, int64_t n_heads, int64_t run, HeadsGeom &g,
                      int64_t &n_blocks, int64_t chunk_vec = QH_CHUNK_VEC) {
  ZX_REQUIRE(n_outer > 0 && n_batch > 0 && n_heads > 0 && run > 0,
             "fp8 heads: all dimensions must be positive");
  if (run % 16) return fail(ZX_ERR_UNSUPPORTED, "fp8 heads: run (%lld) must be a multiple of 16",
                            (long long)run);
  g.n_batch = n_batch;
  g.n_heads = n_heads;
  g.vec_per_run = run / 16;
  g.chunks_per_run = ceil_div(g.vec_per_run, chunk_vec);
  n_blocks = n_outer * n_batch * n_heads * g.chunks_per_run;
  if (n_blocks >= (1LL << 31)) return fail(ZX_ERR_UNSUPPORTED, "fp8 heads: tensor too large");
  return ZX_OK;
}

// ================================================================== paged KV

// Token-major rows x[n_tok][2][H][D]: thread t of a block owns column (16-element
// vector) c = t % vpr of rows t / vpr + RB * j; every column lies in one (kv, head) slab.
struct RowGeom {
  int32_t vpr;        // 16-element vectors per row = 2*H*D/16
  int32_t rb;         // rows per block iteration
  int32_t vec_per_d;  // D / 16 (lanes sharing a slab)
  int32_t n_slabs;    // 2*H
  int64_t n_tok;
  int64_t x_layer_stride;  // elements
};

static int row_geom(int32_t n_heads, int32_t head_dim, int64_t n_tok, int64_t x_layer_stride,
                    RowGeom &g) {
  ZX_REQUIRE(n_heads > 0 && n_tok >= 0, "kv: n_heads must be positive and n_tok >= 0");
  if (!(head_dim == 64 || head_dim == 128 || head_dim == 256))
    return fail(ZX_ERR_UNSUPPORTED, "kv: head_dim %d not in {64, 128, 256}", head_dim);
  int64_t row = 2LL * n_heads * head_dim;
  if (row > 8192) return fail(ZX_ERR_UNSUPPORTED, "kv: 2*H*D = %lld exceeds 8192", (long long)row);
  g.vpr = (int32_t)(row / 16);
  g.rb = g.vpr >= 256 ? 1 : 256 / g.vpr;
  g.vec_per_d = head_dim / 16;
  g.n_slabs = 2 * n_heads;
  g.n_tok = n_tok;
  g.x_layer_stride = x_layer_stride;
  return ZX_OK;
}

// Row kernels of the two-pass path (used when a share does not fit the single-pass
// kernel's registers, e.g. 524,288-token layers).  Lane t of a block owns the 16-byte
// column c = t % vpr8 of rows t / vpr8 + rpb * k (vpr8 = 2*H*D/8 vectors per row,
// rpb = rows per block step), so its slab c / (D/8) is fixed and one scale / one max
// per lane suffices.  Loads go through a buffer resource based at the block's first row
// whose num_records ends at the last token: rows past the end read zeros.
struct RowGeom8 {
  int32_t vpr8;    // 16-byte vectors per token row = 2*H*D/8
  int32_t rpb;     // rows per block step (vpr8 * rpb threads)
  int32_t lps;     // lanes per slab = D/8
  int32_t n_slabs; // 2*H
  int64_t n_tok;
  int64_t row_bytes;
  int64_t x_layer_stride;  // elements
};
typedef unsigned int q_v4u __attribute__((ext_vector_type(4)));
__device__ __forceinline__ __amdgpu_buffer_rsrc_t q_rsrc(const void *base, int64_t bytes) {
  const int n = bytes < 0 ? 0 : (bytes > 0x7FFFFFF0 ? 0x7FFFFFF0 : (int)bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, n, 0x00020000);
}

// Pass 1: per-(layer, slab) amax.  Persistent grid sweeping the rows front to back with
// default-policy loads; pass 2 runs back to front, so it starts on rows the memory-side
// cache still holds (about 5% of pass 2 at 524,288-token layers on MI355X).  Each block
// ends with one maximum per slab: stored into part[layer][block][slab] when a partials
// buffer is given (reduced by finalize_partials_kernel), else combined by atomicMax into
// amax_bits, which must start at zero.  Atomics from every block onto one line serialize
// at the memory side (about 3 ns each on MI355X), so the partials path is the fast one.
template <int U>
__global__ void __launch_bounds__(1024)
kv_amax_rows_kernel(const uint16_t *x, RowGeom8 g, uint32_t *amax_bits /* [L][2H] */,
                    uint32_t *part /* [L][gridDim.x][2H] or null */) {
  const int t = threadIdx.x;
  const int c = t % g.vpr8, rs = t / g.vpr8;
  const int layer = blockIdx.y;
  const char *xl = reinterpret_cast<const char *>(x + (int64_t)layer * g.x_layer_stride);
  const int64_t step = (int64_t)gridDim.x * U * g.rpb;
  uint32_t m = 0;  // two packed 16-bit maxes
  for (int64_t r0 = (int64_t)blockIdx.x * U * g.rpb; r0 < g.n_tok; r0 += step) {
    const __amdgpu_buffer_rsrc_t rsrc = q_rsrc(xl + r0 * g.row_bytes, (g.n_tok - r0) * g.row_bytes);
    uint4 v[U];
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const q_v4u q = __builtin_amdgcn_raw_buffer_load_b128(
          rsrc, (int)((k * g.rpb + rs) * g.row_bytes) + c * 16, 0, 0);
      v[k] = make_uint4(q.x, q.y, q.z, q.w);
    }
#pragma unroll
    for (int k = 0; k < U; ++k) m = absmax_acc(m, v[k]);
  }
  const uint32_t mx = group_max(fold16(m), g.lps);
  if (!part) {
    if (c % g.lps == 0 && mx) atomicMax(&amax_bits[(int64_t)layer * g.n_slabs + c / g.lps], mx << 16);
    return;
  }
  // one value per slab and block: the block's rpb row groups (threads c, vpr8 + c, ...)
  // hold the same slabs and are folded through LDS (at most 1024 threads)
  __shared__ uint32_t red[1024];
  red[t] = mx;
  __syncthreads();
  if (rs == 0 && c % g.lps == 0) {
    uint32_t v = mx;
    for (int k = 1; k < g.rpb; ++k) v = max(v, red[k * g.vpr8 + c]);
    part[((int64_t)layer * gridDim.x + blockIdx.x) * g.n_slabs + c / g.lps] = v << 16;
  }
}

// Per-(layer, slab) maximum over the gx block partials of kv_amax_rows_kernel, turned into
// the slab's scale.  One 256-thread block per (layer, slab).
__global__ void __launch_bounds__(256)
finalize_partials_kernel(const uint32_t *part, int32_t gx, int32_t n_slabs, float *scales) {
  const int64_t i = blockIdx.x;  // layer * n_slabs + slab
  const int64_t layer = i / n_slabs, slab = i % n_slabs;
  const uint32_t *p = part + layer * gx * (int64_t)n_slabs + slab;
  uint32_t v = 0;
  for (int b = threadIdx.x; b < gx; b += 256) v = max(v, p[(int64_t)b * n_slabs]);
  v = group_max(v, 64);
  __shared__ uint32_t red[4];
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  if (threadIdx.x == 0)
    scales[i] = scale_from_amax_bits(max(max(red[0], red[1]), max(red[2], red[3])));
}

// 0x80 in each byte of w whose low 7 bits are all set (an e4m3 NaN code), else 0.
__device__ __forceinline__ uint32_t nan_code_bytes(uint32_t w) { return ((w & 0x7F7F7F7Fu) + 0x01010101u) & 0x80808080u; }

// NaN codes of 8 inputs v under a finite static scale (sign bit s_sign, 0 or 0x80).  The
// code is the NaN code S.1111.111 when the quotient x / s is NaN or rounds beyond the e4m3
// range; its sign is that of the IEEE quotient: the sign of x for a NaN x, else
// sign(x) ^ sign(s).  (div_by_scale's correction step turns an infinite quotient into a
// NaN whose sign is the device's default, so the sign is set here.)  A finite x with a
// NaN code overflowed: MODE 1 flags it, MODE 2 also stores +-448 (S.1111.110).  The
// per-element look runs only when some code is a NaN code.
template <int MODE>
__device__ __forceinline__ uint2 static_overflow(uint4 v, uint2 cd, uint32_t s_sign, int32_t *err) {
  if (!(nan_code_bytes(cd.x) | nan_code_bytes(cd.y))) return cd;
  const uint32_t in[4] = {v.x, v.y, v.z, v.w};
  uint32_t c[2] = {cd.x, cd.y};
  bool hit = false;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const uint32_t bits = (in[k >> 1] >> (16 * (k & 1))) & 0xFFFFu;
    const uint32_t mag = bits & 0x7FFFu, x_sign = (bits >> 8) & 0x80u;
    const int sh = 8 * (k & 3);
    const uint32_t code = (c[k >> 2] >> sh) & 0xFFu;
    if ((code & 0x7Fu) == 0x7Fu) {
      const uint32_t sign = mag > 0x7F80u ? x_sign : (x_sign ^ s_sign);
      uint32_t fixed = sign | 0x7Fu;
      if (mag < 0x7F80u) {
        hit = true;
        if (MODE == 2) fixed = sign | 0x7Eu;
      }
      c[k >> 2] = (c[k >> 2] & ~(0xFFu << sh)) | (fixed << sh);
    }
  }
  if (hit && err) atomicOr(err, ZX_KERR_OVERFLOW);
  return make_uint2(c[0], c[1]);
}

// Pass 2: encode and scatter.  Block b takes rows [r0, r0 + U*rpb) with tiles taken from
// the end of the batch first.  A row without a page (tok_off < 0) is not stored.
// MODE 0: dynamic scales (no code can overflow, and a slab holding a non-finite input has a
// non-finite scale); 1: static scales, NaN codes signed as the IEEE quotient and overflow
// flagged in *err; 2: as 1, with overflow saturated.
template <int U, int MODE>
__global__ void __launch_bounds__(1024)
kv_quant_rows_kernel(const uint16_t *x, RowGeom8 g, const int64_t *tok_off, const float *scales,
                     uint8_t *pool, int64_t pool_layer_stride, int32_t page_size, int32_t head_dim, int32_t *err) {
  const int t = threadIdx.x;
  const int c = t % g.vpr8, rs = t / g.vpr8;
  const int slab = c / g.lps;
  const int layer = blockIdx.y;
  const float sc = scales[(int64_t)layer * g.n_slabs + slab];
  const QuantScale q = quant_scale(sc);
  const uint32_t s_sign = (__float_as_uint(sc) >> 24) & 0x80u;
  const int64_t tile = (int64_t)gridDim.x - 1 - blockIdx.x;
  const int64_t r0 = tile * U * g.rpb;
  const char *xl = reinterpret_cast<const char *>(x + (int64_t)layer * g.x_layer_stride);
  const __amdgpu_buffer_rsrc_t rsrc = q_rsrc(xl + r0 * g.row_bytes, (g.n_tok - r0) * g.row_bytes);
  uint8_t *pl = pool + (int64_t)layer * pool_layer_stride + (int64_t)slab * page_size * head_dim +
                (c % g.lps) * 8;
  uint4 v[U];
  int64_t off[U];
#pragma unroll
  for (int k = 0; k < U; ++k) {
    const int64_t r = r0 + k * g.rpb + rs;
    off[k] = r < g.n_tok ? tok_off[r] : -1;
    const q_v4u w = __builtin_amdgcn_raw_buffer_load_b128(rsrc, (int)((k * g.rpb + rs) * g.row_bytes) + c * 16,
                                                          0, 2 /* nontemporal: last read */);
    v[k] = make_uint4(w.x, w.y, w.z, w.w);
  }
#pragma unroll
  for (int k = 0; k < U; ++k) {
    if (off[k] < 0) continue;
    uint2 cd = quant8(v[k], q);
    if (MODE != 0 && q.nan_fix == 0) cd = static_overflow<MODE>(v[k], cd, s_sign, err);
    typedef unsigned int v2u __attribute__((ext_vector_type(2)));
    const v2u w2 = {cd.x, cd.y};
    __builtin_nontemporal_store(w2, reinterpret_cast<v2u *>(pl + off[k]));
  }
}

// Pool offset (bytes within one layer) of each token's (page, row) base, or -1.
__global__ void kv_token_offsets_kernel(const int32_t *cu_seqlens, const int32_t *start_pos,
                                        int32_t n_seqs, const int32_t *block_tables,
                                        int32_t max_blocks, int32_t page_size, int64_t n_pages,
                                        int64_t page_bytes, int32_t head_dim, int64_t n_tok,
                                        int64_t *tok_off, int32_t *err) {
  int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n_tok) return;
  int lo = 0, hi = n_seqs - 1;  // last b with cu_seqlens[b] <= t
  while (lo < hi) {
    int mid = (lo + hi + 1) >> 1;
    if (cu_seqlens[mid] <= t) lo = mid;
    else hi = mid - 1;
  }
  const int b = lo;
  int64_t off = -1;
  if (t >= cu_seqlens[b] && t < cu_seqlens[b + 1]) {
    int64_t pos = (start_pos ? start_pos[b] : 0) + (t - cu_seqlens[b]);
    if (pos < 0 || pos >= (int64_t)max_blocks * page_size) {
      if (err) atomicOr(err, ZX_KERR_POS_RANGE);
    } else {
      int64_t page = block_tables[(int64_t)b * max_blocks + pos / page_size];
      if (page < 0 || page >= n_pages) {
        if (err) atomicOr(err, ZX_KERR_PAGE_RANGE);
      } else {
        off = page * page_bytes + (pos % page_size) * head_dim;
      }
    }
  }
  tok_off[t] = off;
}

#ifndef KA_U
#define KA_U 8  // rows per thread per step of the amax pass
#endif
#ifndef KQ_U
#define KQ_U 4  // rows per thread of the two-pass encode
#endif

static RowGeom8 row_geom8(const RowGeom &g) {
  RowGeom8 r;
  r.vpr8 = g.vpr * 2;
  r.rpb = r.vpr8 >= 256 ? 1 : 256 / r.vpr8;
  r.lps = g.vec_per_d * 2;
  r.n_slabs = g.n_slabs;
  r.n_tok = g.n_tok;
  r.row_bytes = (int64_t)g.vpr * 32;
  r.x_layer_stride = g.x_layer_stride;
  return r;
}

#ifndef KA_BPC
#define KA_BPC 4  // amax blocks per CU (of 256 threads at 4 KiB rows)
#endif

// Blocks per layer of the amax pass: KA_BPC per CU over all layers, at most one per tile.
static int64_t amax_grid_x(int64_t n_tok, int32_t rpb, int32_t n_layers) {
  const int64_t tiles = ceil_div(n_tok, (int64_t)KA_U * rpb);
  const int64_t want = std::max<int64_t>(1, ceil_div((int64_t)num_cus() * KA_BPC, n_layers));
  return std::max<int64_t>(1, std::min(tiles, want));
}

// Bytes of the partials buffer kv_scales_impl can use: [L][blocks per layer][2H] words.
static size_t amax_partials_bytes(int32_t n_layers, int32_t n_heads) {
  const int64_t gx = std::max<int64_t>(1, ceil_div((int64_t)num_cus() * KA_BPC, n_layers));
  return align256((size_t)gx * n_layers * 2 * n_heads * sizeof(uint32_t));
}

// Dynamic scales of every (layer, slab).  With `part` (amax_partials_bytes of device
// memory) the blocks store their maxima and one reduction kernel finishes; without it they
// combine by atomics into `scales` (cleared first).
static int kv_scales_impl(const uint16_t *x, const RowGeom &g, int32_t n_layers, float *scales,
                          uint32_t *part, hipStream_t st) {
  const int64_t n = (int64_t)n_layers * g.n_slabs;
  int rc;
  if (part && g.n_tok > 0) {
    const RowGeom8 r = row_geom8(g);
    const unsigned gx = (unsigned)amax_grid_x(g.n_tok, r.rpb, n_layers);
    kv_amax_rows_kernel<KA_U><<<dim3(gx, n_layers), r.vpr8 * r.rpb, 0, st>>>(x, r, nullptr, part);
    if ((rc = check_launch("kv_amax_rows"))) return rc;
    finalize_partials_kernel<<<(unsigned)n, 256, 0, st>>>(part, (int32_t)gx, g.n_slabs, scales);
    return check_launch("finalize_partials");
  }
  if ((rc = fill_u32(reinterpret_cast<uint32_t *>(scales), n, 0, st))) return rc;
  if (g.n_tok > 0) {
    const RowGeom8 r = row_geom8(g);
    const unsigned gx = (unsigned)amax_grid_x(g.n_tok, r.rpb, n_layers);
    kv_amax_rows_kernel<KA_U><<<dim3(gx, n_layers), r.vpr8 * r.rpb, 0, st>>>(
        x, r, reinterpret_cast<uint32_t *>(scales), nullptr);
    if ((rc = check_launch("kv_amax_rows"))) return rc;
  }
  finalize_scales_kernel<<<(unsigned)ceil_div(n, 256), 256, 0, st>>>(scales, n);
  return check_launch("finalize_scales");
}

}  // namespace zx

using namespace zx;

// ================================================================== C ABI

namespace {
// blocks per slab: ~16 per CU over all slabs, at most one per 8 K elements of a slab
unsigned legacy_blocks_per_slab(int64_t n_slabs, int64_t slab_len) {
  const int64_t bps = ceil_div((int64_t)num_cus() * 16, n_slabs);
  int64_t cap = ceil_div(slab_len, 256LL * 32);
  if (cap < 1) cap = 1;
  return (unsigned)(bps < 1 ? 1 : (bps > cap ? cap : bps));
}

template <int DT>
int legacy_quant_launch(const void *x, int64_t n_slabs, int64_t slab_len, int8_t *q, void *scales, uint32_t *amax,
                        hipStream_t st) {
  using V = LegacyVec<DT>;
  const bool vec = (uintptr_t)x % 16 == 0 && (uintptr_t)q % V::W == 0 &&
                   (n_slabs == 1 || (slab_len * V::ES) % 16 == 0);
  const dim3 grid(legacy_blocks_per_slab(n_slabs, slab_len), (unsigned)n_slabs);
  const bool large = (double)n_slabs * slab_len * V::ES >= (double)(256 << 20);
  int rc;
  if (vec) {
    if (large)
      legacy_amax_slabs_kernel<DT, true, true><<<grid, 256, 0, st>>>(x, slab_len, amax);
    else
      legacy_amax_slabs_kernel<DT, true, false><<<grid, 256, 0, st>>>(x, slab_len, amax);
    if ((rc = check_launch("legacy_amax"))) return rc;
    // one contiguous tile per block (6% faster than the amax pass's persistent grid, which
    // stays there because every block ends with an atomic)
    const int64_t qt = ceil_div(slab_len / V::W, 256LL * LEGACY_U);
    legacy_quant_slabs_kernel<DT, true><<<dim3((unsigned)(qt < 1 ? 1 : qt), (unsigned)n_slabs), 256, 0, st>>>(
        x, slab_len, amax, q, scales);
  } else {
    legacy_amax_slabs_kernel<DT, false, false><<<grid, 256, 0, st>>>(x, slab_len, amax);
    if ((rc = check_launch("legacy_amax"))) return rc;
    legacy_quant_slabs_kernel<DT, false><<<grid, 256, 0, st>>>(x, slab_len, amax, q, scales);
  }
  return check_launch("legacy_quant");
}

template <int DT>
int legacy_dequant_launch(const int8_t *q, const void *scales, int64_t n_slabs, int64_t slab_len, uint16_t *y,
                          hipStream_t st) {
  const bool vec = (uintptr_t)q % 8 == 0 && (uintptr_t)y % 16 == 0 && (n_slabs == 1 || slab_len % 8 == 0);
  // vector path: one contiguous tile of LEGACY_U x 256 vectors per block (9% faster than a
  // persistent grid at 1 Gi elements)
  const int64_t tiles = ceil_div(slab_len / 8, 256LL * LEGACY_U);
  const dim3 grid(vec ? (unsigned)(tiles < 1 ? 1 : tiles) : legacy_blocks_per_slab(n_slabs, slab_len),
                  (unsigned)n_slabs);
  if (vec)
    legacy_dequant_slabs_kernel<DT, true><<<grid, 256, 0, st>>>(q, scales, slab_len, y);
  else
    legacy_dequant_slabs_kernel<DT, false><<<grid, 256, 0, st>>>(q, scales, slab_len, y);
  return check_launch("legacy_dequant");
}

int legacy_quant_any(const void *x, int dtype, int64_t n_slabs, int64_t slab_len, int8_t *q, void *scales,
                     void *workspace, hipStream_t st, const char *what) {
  uint32_t *amax = reinterpret_cast<uint32_t *>(workspace);
  int rc = fill_u32(amax, n_slabs, 0, st);
  if (rc) return rc;
  switch (dtype) {
    case ZX_BF16: return legacy_quant_launch<ZX_BF16>(x, n_slabs, slab_len, q, scales, amax, st);
    case ZX_F16: return legacy_quant_launch<ZX_F16>(x, n_slabs, slab_len, q, scales, amax, st);
    case ZX_F32: return legacy_quant_launch<ZX_F32>(x, n_slabs, slab_len, q, scales, amax, st);
    default: return fail(ZX_ERR_INVALID, "%s: unknown dtype %d", what, dtype);
  }
}

int legacy_dequant_any(const int8_t *q, const void *scales, int dtype, int64_t n_slabs, int64_t slab_len, uint16_t *y,
                       hipStream_t st, const char *what) {
  switch (dtype) {
    case ZX_BF16: return legacy_dequant_launch<ZX_BF16>(q, scales, n_slabs, slab_len, y, st);
    case ZX_F16: return legacy_dequant_launch<ZX_F16>(q, scales, n_slabs, slab_len, y, st);
    case ZX_F32: return legacy_dequant_launch<ZX_F32>(q, scales, n_slabs, slab_len, y, st);
    default: return fail(ZX_ERR_INVALID, "%s: unknown dtype %d", what, dtype);
  }
}
}  // namespace

extern "C" int zx_int8_legacy_quant(const void *x, int dtype, int64_t n, int8_t *q, void *scale,
                                    void *workspace, size_t workspace_bytes, zx_stream_t stream) {
  clear_error();
  ZX_REQUIRE(x && q && scale, "int8_legacy_quant: null pointer");
  ZX_REQUIRE(n > 0, "int8_legacy_quant: empty tensor (the reference raises on amax of an empty tensor)");
  if (!workspace || workspace_bytes < 256) return fail(ZX_ERR_WORKSPACE, "int8_legacy_quant: workspace < 256 bytes");
  return legacy_quant_any(x, dtype, 1, n, q, scale, workspace, as_stream(stream), "int8_legacy_quant");
}

extern "C" size_t zx_int8_legacy_quant_slabs_workspace_bytes(int64_t n_slabs) {
  return (size_t)((n_slabs > 0 ? n_slabs : 0) * 4 + 255) / 256 * 256;
}

extern "C" int zx_int8_legacy_quant_slabs(const void *x, int dtype, int64_t n_slabs, int64_t slab_len, int8_t *q,
                                          void *scales, void *workspace, size_t workspace_bytes, zx_stream_t stream) {
  clear_error();
  ZX_REQUIRE(x && q && scales, "int8_legacy_quant_slabs: null pointer");
  ZX_REQUIRE(n_slabs > 0 && n_slabs <= 65535 && slab_len > 0,
             "int8_legacy_quant_slabs: need 1..65535 slabs of at least one element (the reference raises on amax of "
             "an empty tensor)");
  if (!workspace || workspace_bytes < zx_int8_legacy_quant_slabs_workspace_bytes(n_slabs))
    return fail(ZX_ERR_WORKSPACE, "int8_legacy_quant_slabs: workspace < %zu bytes",
                zx_int8_legacy_quant_slabs_workspace_bytes(n_slabs));
  return legacy_quant_any(x, dtype, n_slabs, slab_len, q, scales, workspace, as_stream(stream),
                          "int8_legacy_quant_slabs");
}

extern "C" int zx_int8_legacy_dequant_slabs(const int8_t *q, const void *scales, int scale_dtype, int64_t n_slabs,
                                            int64_t slab_len, uint16_t *y, zx_stream_t stream) {
  clear_error();
  ZX_REQUIRE(q && scales && y, "int8_legacy_dequant_slabs: null pointer");
  ZX_REQUIRE(n_slabs >= 0 && n_slabs <= 65535 && slab_len >= 0, "int8_legacy_dequant_slabs: bad sizes");
  if (n_slabs == 0 || slab_len == 0) return ZX_OK;
  return legacy_dequant_any(q, scales, scale_dtype, n_slabs, slab_len, y, as_stream(stream),
                            "int8_legacy_dequant_slabs");
}

extern "C" int zx_int8_legacy_dequant(const int8_t *q, const void *scale, int scale_dtype, int64_t n, uint16_t *y,
                                      zx_stream_t stream) {
  clear_error();
  ZX_REQUIRE(q && scale && y, "int8_legacy_dequant: null pointer");
  ZX_REQUIRE(n >= 0, "int8_legacy_dequant: negative size");
  if (n == 0) return ZX_OK;
  return legacy_dequant_any(q, scale, scale_dtype, 1, n, y, as_stream(stream), "int8_legacy_dequant");
}

extern "C" size_t zx_fp8_quant_heads_workspace_bytes(int64_t n_outer, int64_t n_batch, int64_t n_heads,
                                                     int64_t run) {
  return heads_fused_workspace_bytes(n_outer, n_batch, n_heads, run);
}

extern "C" int zx_fp8_quant_heads(const uint16_t *x, int64_t n_outer, int64_t n_batch, int64_t n_heads,
                                  int64_t run, uint8_t *codes, float *scales, int32_t flags, int32_t *err,
                                  void *workspace, size_t workspace_bytes, zx_stream_t stream) {
  clear_error();
  ZX_REQUIRE(x && codes && scales, "fp8_quant_heads: null pointer");
  ZX_REQUIRE(aligned16(x) && aligned16(codes), "fp8_quant_heads: x and codes must be 16-byte aligned");
  ZX_REQUIRE(!(flags & ~(ZX_HEADS_TWO_PASS | ZX_HEADS_SINGLE_PASS)), "fp8_quant_heads: unknown flag bits 0x%x",
             (unsigned)flags);
  ZX_REQUIRE((flags & (ZX_HEADS_TWO_PASS | ZX_HEADS_SINGLE_PASS)) != (ZX_HEADS_TWO_PASS | ZX_HEADS_SINGLE_PASS),
             "fp8_quant_heads: ZX_HEADS_TWO_PASS and ZX_HEADS_SINGLE_PASS together");
  HeadsGeom g;
  int64_t nb;
  int rc = heads_geom(n_outer, n_batch, n_heads, run, g, nb);
  if (rc) return rc;
  hipStream_t st = as_stream(stream);
  // Below the 256 MiB Infinity Cache the two passes' second read is served from it and two
  // passes are faster (MI355X: 0.069 vs 0.091 ms at configs[0]'s 151 MB); above it the
  // single pass saves the second HBM read (1 Gi elements: 0.66 vs 1.02 ms).
  const bool large = (double)n_outer * n_batch * n_heads * run * 2 >= (double)(256 << 20);
  if (!(flags & ZX_HEADS_TWO_PASS) && (large || (flags & ZX_HEADS_SINGLE_PASS))) {
    const size_t need = heads_fused_workspace_bytes(n_outer, n_batch, n_heads, run);
    if (!workspace || workspace_bytes < need)
      return fail(ZX_ERR_WORKSPACE, "fp8_quant_heads: workspace %zu < %zu bytes", workspace_bytes, need);
    rc = heads_fused(x, n_outer, n_batch, n_heads, run, codes, scales, err, workspace, workspace_bytes, st);
    if (rc != ZX_ERR_UNSUPPORTED) return rc;
    clear_error();  // shape or device outside the single pass: two passes below
  }
  int64_t ns = n_outer * n_heads;
  if ((rc = fill_u32(reinterpret_cast<uint32_t *>(scales), ns, 0, st))) return rc;
  heads_amax_kernel<<<(unsigned)nb, QH_THREADS, 0, st>>>(reinterpret_cast<const uint4 *>(x), g,
                                                        reinterpret_cast<uint32_t *>(scales));
  if ((rc = check_launch("heads_amax"))) return rc;
  finalize_scales_kernel<<<(unsigned)ceil_div(ns, 256), 256, 0, st>>>(scales, ns);
  if ((rc = check_launch("finalize_scales"))) return rc;
  heads_quant_kernel<<<(unsigned)nb, QH_THREADS, 0, st>>>(reinterpret_cast<const uint4 *>(x), g, scales,
                                                         reinterpret_cast<uint4 *>(codes));
  return check_launch("heads_quant");
}

extern "C" int zx_fp8_dequant_heads(const uint8_t *codes, const float *scales, int64_t n_outer,
                                    int64_t n_batch, int64_t n_heads, int64_t run, uint16_t *y,
                                    zx_stream_t stream) {
  clear_error();
  ZX_REQUIRE(codes && scales && y, "fp8_dequant_heads: null pointer");
  ZX_REQUIRE(aligned16(codes) && aligned16(y), "fp8_dequant_heads: codes and y must be 16-byte aligned");
  HeadsGeom g;
  int64_t nb;
  int rc = heads_geom(n_outer, n_batch, n_heads, run, g, nb, (int64_t)QH_THREADS * QH_DQ_VPT);
  if (rc) return rc;
  heads_dequant_kernel<QH_DQ_VPT><<<(unsigned)nb, QH_THREADS, 0, as_stream(stream)>>>(
      reinterpret_cast<const uint4 *>(codes), g, scales, reinterpret_cast<uint4 *>(y));
  return check_launch("heads_dequant");
}

extern "C" int zx_kv_scales(const uint16_t *x, int64_t x_layer_stride, int32_t n_layers, int64_t n_tok,
                            int32_t n_heads, int32_t head_dim, float *scales, zx_stream_t stream) {
  clear_error();
  ZX_REQUIRE(scales && (x || n_tok == 0), "kv_scales: null pointer");
  ZX_REQUIRE(aligned16(x) && (n_layers == 1 || x_layer_stride % 8 == 0),
             "kv_scales: x (and every layer of it) must be 16-byte aligned");
  ZX_REQUIRE(n_layers > 0 && n_layers <= 65535, "kv_scales: n_layers out of range");
  RowGeom g;
  int rc = row_geom(n_heads, head_dim, n_tok, x_layer_stride, g);
  if (rc) return rc;
  ZX_REQUIRE(n_layers == 1 || x_layer_stride >= n_tok * 2LL * n_heads * head_dim,
             "kv_scales: layer stride smaller than a layer");
  return kv_scales_impl(x, g, n_layers, scales, nullptr, as_stream(stream));
}

extern "C" size_t zx_kv_quant_append_workspace_bytes(int32_t n_layers, int64_t n_tok, int32_t n_heads,
                                                     int32_t head_dim) {
  (void)head_dim;
  return align256((size_t)(n_tok > 0 ? n_tok : 0) * sizeof(int64_t)) +
         std::max(append_fused_workspace_bytes(n_layers, n_heads), amax_partials_bytes(n_layers, n_heads));
}

namespace {
// The body of zx_kv_quant_append and zx_kv_quant_append_noalloc: argument checks, token
// offsets, then the single-pass kernel or the two passes.  Launches kernels only (no
// allocation); everything the workspace must hold at the start is written by kernels on
// `st` (token offsets, the single pass's slots and abort flag), so a workspace's old
// contents never matter.
int kv_quant_append_impl(const uint16_t *x, int64_t x_layer_stride, int32_t n_layers, int64_t n_tok, int32_t n_heads,
                         int32_t head_dim, const int32_t *cu_seqlens, const int32_t *start_pos, int32_t n_seqs,
                         const int32_t *block_tables, int32_t max_blocks, int32_t page_size, uint8_t *pool,
                         int64_t pool_layer_stride, int64_t n_pages, float *scales, int32_t flags, int32_t *err,
                         void *workspace, size_t workspace_bytes, hipStream_t st) {
  ZX_REQUIRE(!(flags & ~(ZX_APPEND_STATIC_SCALES | ZX_APPEND_TWO_PASS | ZX_APPEND_SATURATE | ZX_APPEND_SINGLE_PASS)),
             "kv_quant_append: unknown flag bits 0x%x", (unsigned)flags);
  ZX_REQUIRE((flags & (ZX_APPEND_TWO_PASS | ZX_APPEND_SINGLE_PASS)) != (ZX_APPEND_TWO_PASS | ZX_APPEND_SINGLE_PASS),
             "kv_quant_append: ZX_APPEND_TWO_PASS and ZX_APPEND_SINGLE_PASS together");
  ZX_REQUIRE(scales && cu_seqlens && block_tables && pool, "kv_quant_append: null pointer");
  ZX_REQUIRE(x || n_tok == 0, "kv_quant_append: null x");
  ZX_REQUIRE(aligned16(x) && aligned16(pool) && (n_layers == 1 || (x_layer_stride % 8 == 0 && pool_layer_stride % 16 == 0)),
             "kv_quant_append: x and pool (and every layer of them) must be 16-byte aligned");
  ZX_REQUIRE(n_layers > 0 && n_layers <= 65535, "kv_quant_append: n_layers out of range");
  ZX_REQUIRE(n_seqs > 0 && max_blocks > 0 && page_size > 0 && n_pages > 0,
             "kv_quant_append: n_seqs, max_blocks, page_size and n_pages must be positive");
  ZX_REQUIRE(n_tok < (1LL << 31), "kv_quant_append: n_tok must be below 2^31");
  RowGeom g;
  int rc = row_geom(n_heads, head_dim, n_tok, x_layer_stride, g);
  if (rc) return rc;
  const int64_t page_bytes = 2LL * n_heads * page_size * head_dim;
  ZX_REQUIRE(n_layers == 1 || x_layer_stride >= n_tok * 2LL * n_heads * head_dim,
             "kv_quant_append: x layer stride smaller than a layer");
  ZX_REQUIRE(n_layers == 1 || pool_layer_stride >= n_pages * page_bytes,
             "kv_quant_append: pool layer stride smaller than a layer's pages");
  size_t need = zx_kv_quant_append_workspace_bytes(n_layers, n_tok, n_heads, head_dim);
  if (!workspace || workspace_bytes < need)
    return fail(ZX_ERR_WORKSPACE, "kv_quant_append: workspace %zu < %zu bytes", workspace_bytes, need);
  const bool dynamic = !(flags & ZX_APPEND_STATIC_SCALES);
  if (n_tok == 0) return dynamic ? kv_scales_impl(x, g, n_layers, scales, nullptr, st) : ZX_OK;
  int64_t *tok_off = reinterpret_cast<int64_t *>(workspace);
  kv_token_offsets_kernel<<<(unsigned)ceil_div(n_tok, 256), 256, 0, st>>>(
      cu_seqlens, start_pos, n_seqs, block_tables, max_blocks, page_size, n_pages, page_bytes, head_dim,
      n_tok, tok_off, err);
  if ((rc = check_launch("kv_token_offsets"))) return rc;
  if (dynamic && !(flags & ZX_APPEND_TWO_PASS) &&
      ((flags & ZX_APPEND_SINGLE_PASS) || append_fused_preferred(n_tok, head_dim, (int64_t)n_layers * 2 * n_heads))) {
    void *fws = static_cast<char *>(workspace) + align256((size_t)n_tok * sizeof(int64_t));
    rc = append_fused(x, x_layer_stride, n_layers, n_tok, n_heads, head_dim, tok_off, pool, pool_layer_stride,
                      page_size, scales, err, fws, st);
    if (rc != ZX_ERR_UNSUPPORTED) return rc;
    clear_error();  // this device cannot run the single-pass kernel: two passes below
  }
  // the two passes: the tail of the workspace (the single pass's region) holds the amax partials
  uint32_t *part = reinterpret_cast<uint32_t *>(static_cast<char *>(workspace) + align256((size_t)n_tok * sizeof(int64_t)));
  if (dynamic && (rc = kv_scales_impl(x, g, n_layers, scales, part, st))) return rc;
  const RowGeom8 r = row_geom8(g);
  const int64_t tiles = ceil_div(n_tok, (int64_t)KQ_U * r.rpb);
  if (tiles >= (1LL << 31)) return fail(ZX_ERR_UNSUPPORTED, "kv_quant_append: too many rows");
  const dim3 grid((unsigned)tiles, n_layers);
  const int threads = r.vpr8 * r.rpb;
  if (dynamic)
    kv_quant_rows_kernel<KQ_U, 0><<<grid, threads, 0, st>>>(x, r, tok_off, scales, pool, pool_layer_stride,
                                                            page_size, head_dim, err);
  else if (flags & ZX_APPEND_SATURATE)
    kv_quant_rows_kernel<KQ_U, 2><<<grid, threads, 0, st>>>(x, r, tok_off, scales, pool, pool_layer_stride,
                                                            page_size, head_dim, err);
  else
    kv_quant_rows_kernel<KQ_U, 1><<<grid, threads, 0, st>>>(x, r, tok_off, scales, pool, pool_layer_stride,
                                                            page_size, head_dim, err);
  return check_launch("kv_quant_rows");
}

// Scratch of zx_kv_quant_append_noalloc: one copy per GPU, in the code object (no
// allocation call).  Its host-side name is not a device address: kernels get the address
// hipGetSymbolAddress returns for the current device.
static __device__ __align__(256) uint8_t scratch[ZX_KV_APPEND_NOALLOC_SCRATCH_BYTES];

int noalloc_scratch(void **out) {
  static std::mutex mu;
  static void *ptr[64] = {nullptr};
  int dev = 0;
  ZX_TRY_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= 64) return fail(ZX_ERR_UNSUPPORTED, "device index %d out of range", dev);
  std::lock_guard<std::mutex> lock(mu);
  if (!ptr[dev]) {
    void *p = nullptr;
    ZX_TRY_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) return fail(ZX_ERR_HIP, "hipGetSymbolAddress returned no address for the append scratch");
    ptr[dev] = p;
  }
  *out = ptr[dev];
  return ZX_OK;
}
}  // namespace

extern "C" int zx_kv_quant_append(const uint16_t *x, int64_t x_layer_stride, int32_t n_layers,
                                  int64_t n_tok, int32_t n_heads, int32_t head_dim,
                                  const int32_t *cu_seqlens, const int32_t *start_pos, int32_t n_seqs,
                                  const int32_t *block_tables, int32_t max_blocks, int32_t page_size,
                                  uint8_t *pool, int64_t pool_layer_stride, int64_t n_pages,
                                  float *scales, int32_t flags, int32_t *err, void *workspace,
                                  size_t workspace_bytes, zx_stream_t stream) {
  clear_error();
  return kv_quant_append_impl(x, x_layer_stride, n_layers, n_tok, n_heads, head_dim, cu_seqlens, start_pos, n_seqs,
                              block_tables, max_blocks, page_size, pool, pool_layer_stride, n_pages, scales, flags,
                              err, workspace, workspace_bytes, as_stream(stream));
}

extern "C" int zx_kv_quant_append_noalloc(const uint16_t *x, int64_t x_layer_stride, int32_t n_layers,
                                          int64_t n_tok, int32_t n_heads, int32_t head_dim,
                                          const int32_t *cu_seqlens, const int32_t *start_pos, int32_t n_seqs,
                                          const int32_t *block_tables, int32_t max_blocks, int32_t page_size,
                                          uint8_t *pool, int64_t pool_layer_stride, int64_t n_pages, float *scales,
                                          int32_t flags, int32_t *err, zx_stream_t stream) {
  clear_error();
  const size_t need = zx_kv_quant_append_workspace_bytes(n_layers, n_tok, n_heads, head_dim);
  if (n_tok < 0 || need > (size_t)ZX_KV_APPEND_NOALLOC_SCRATCH_BYTES)
    return fail(ZX_ERR_WORKSPACE,
                "kv_quant_append_noalloc: this call needs %zu bytes of scratch, more than the %u bytes it has "
                "(use zx_kv_quant_append with a workspace)",
                need, (unsigned)ZX_KV_APPEND_NOALLOC_SCRATCH_BYTES);
  void *ws = nullptr;
  int rc = noalloc_scratch(&ws);
  if (rc) return rc;
  return kv_quant_append_impl(x, x_layer_stride, n_layers, n_tok, n_heads, head_dim, cu_seqlens, start_pos, n_seqs,
                              block_tables, max_blocks, page_size, pool, pool_layer_stride, n_pages, scales, flags,
                              err, ws, ZX_KV_APPEND_NOALLOC_SCRATCH_BYTES, as_stream(stream));
}

namespace zx {
__global__ void encode_f32_kernel(const float *v, int64_t n, uint8_t *codes) {
  int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i >= n) return;
  float a[4];
  uint32_t fix = 0, fixmask = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    a[k] = i + k < n ? v[i + k] : 0.0f;
    uint32_t b = __float_as_uint(a[k]);
    if ((b & 0x7FFFFFFFu) > 0x43E80000u) {  // beyond 464 (or Inf/NaN): e4m3fn NaN
      fix |= (((b >> 24) & 0x80u) | 0x7Fu) << (8 * k);
      fixmask |= 0xFFu << (8 * k);
      a[k] = 0.0f;
    }
  }
  uint32_t w = (e4m3x4(a[0], a[1], a[2], a[3]) & ~fixmask) | fix;
#pragma unroll
  for (int k = 0; k < 4; ++k)
    if (i + k < n) codes[i + k] = (uint8_t)(w >> (8 * k));
}
}  // namespace zx

extern "C" int zx_fp8_encode_f32(const float *v, int64_t n, uint8_t *codes, zx_stream_t stream) {
  clear_error();
  ZX_REQUIRE(n >= 0, "fp8_encode_f32: negative size");
  if (n == 0) return ZX_OK;
  ZX_REQUIRE(v && codes, "fp8_encode_f32: null pointer");
  encode_f32_kernel<<<(unsigned)ceil_div(ceil_div(n, 4), 256), 256, 0, as_stream(stream)>>>(v, n, codes);
  return check_launch("fp8_encode_f32");
}
