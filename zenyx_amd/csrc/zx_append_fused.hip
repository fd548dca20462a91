// zx_append_fused.hip -- single-pass paged append with dynamic per-(layer, kv, head) FP8
// scales (sized for a 32-layer append of ~75k tokens, 8 KV heads, D = 128).
//
// A (layer, kv, head) slab's scale needs the amax over all of its tokens before any of
// them can be encoded.  Instead of reading the input twice (amax pass + quant pass), one
// cooperative persistent launch keeps each workgroup's share of a slab on chip:
//   * workgroup w (one per CU) owns tokens [w*T/G, (w+1)*T/G) of every slab;
//   * 15 data waves keep NB = 5 slabs of their share in registers.  At step s a wave
//     reduces the max of slab s+4 (loaded during step s-1), hands it to the workgroup,
//     waits for slab s's scale, encodes slab s and refills that buffer with slab s+5, so
//     loads stay in flight continuously and no block-wide barrier is ever taken;
//   * even and odd workgroups take each layer's slabs in two orders that differ at every
//     step in K/V and in the head, so the reads and the writes in flight are spread over
//     the offsets inside each 4 KiB (see phys_slab);
//   * a wave's max goes to an LDS slot (ds_max + arrival count); the control wave (the
//     16th) stores the workgroup's max plus one into its own device-coherent slot of
//     slab s (slots start at zero), reads all G slots of a slab with one wave-wide load
//     until none is zero, and broadcasts the finished scale through LDS.  It
//     publishes later slabs while still polling slab s, so their round trips overlap,
//     and the data waves keep streaming throughout.
// Loads and stores go through buffer resources, whose range check drops the lanes that
// have nothing to move (past the share, rows without a page, padding steps), so the
// data path has no per-lane branch or select.
// HBM traffic is 2 B read + 1 B written per element.  Tokens of a share beyond what the
// registers hold are re-read from memory (both for the max and for the encode).
// Every wait is bounded in wall time; a timeout raises a global abort flag that
// releases every other waiter, so all waves always exit.
#include <type_traits>

#include "zx_internal.h"

namespace zx {

constexpr int FA_THREADS = 1024;
constexpr int FA_DATA_WAVES = 15;
constexpr int FA_DATA_THREADS = FA_DATA_WAVES * 64;
constexpr int FA_SLOTS = 8;                 // LDS ring of per-slab reduction slots (>= NB + 1)
// A slot holds a workgroup's share max (a bf16 magnitude, at most 0x7FFF) plus one, so the
// zeroed workspace reads as "not published yet" (one fill clears flag and slots together).

struct FusedArgs {
  const uint16_t *x;
  int64_t x_layer_stride;  // elements
  int64_t n_tok;
  int32_t n_layers, n_heads, head_dim, page_size;
  int32_t vpt_log2;  // log2(16-byte vectors per token row of one head) = log2(D / 8)
  const int64_t *tok_off;
  uint8_t *pool;
  int64_t pool_layer_stride;
  float *scales;
  uint32_t *slots;  // [S][G] each workgroup's share max (bf16 magnitude) + 1, 0 until published
  uint32_t *abort_flag;
  int32_t *err;
  uint64_t spin_ticks;  // bound of one wait in s_memrealtime ticks (100 MHz)
};

struct FusedShared {
  uint32_t max[FA_SLOTS];    // running max of the data waves' contributions
  uint32_t cnt[FA_SLOTS];    // data waves that contributed
  uint32_t ready[FA_SLOTS];  // s + 1 once slab s's scale is final
  float scale[FA_SLOTS];
  uint32_t abort;
};

__device__ __forceinline__ uint32_t ld_agent(const uint32_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// LDS flags between the waves of one workgroup.  DS instructions of a wave execute in
// program order, so relaxed LDS atomics plus compiler-only fences order them; acquire /
// release orderings would also drain every outstanding global load (s_waitcnt vmcnt(0))
// and stall the streaming data waves.
#define ZX_COMPILER_FENCE() asm volatile("" ::: "memory")
__device__ __forceinline__ uint32_t ld_lds(const uint32_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Buffer resources (raw, stride 0) let the hardware drop what a lane must not touch: a
// load whose offset is at or past num_records returns zeros, such a store is discarded.
// Lanes past the share, and rows without a page, get offset FA_OOB; a padding step
// stores through a resource with num_records = 0.
constexpr uint32_t FA_OOB = 0x80000000u;
constexpr int FA_RANGE = 0x7FFFFFF0;  // num_records of a live resource (offsets < 2^31 - 16)
typedef unsigned int zx_v4u __attribute__((ext_vector_type(4)));
typedef unsigned int zx_v2u __attribute__((ext_vector_type(2)));
constexpr int FA_NT = 2;  // cache policy: nontemporal (each byte is moved exactly once)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void *base, int num_records) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, num_records, 0x00020000);
}

// Per-thread constants of the register part.  Vector k of a data thread is index
// v = k * FA_DATA_THREADS + tid of the share (token v >> vpt_log2, 16-byte chunk
// v & mask).  src[k] is its byte offset from the share's first row (FA_OOB past the
// share); dst[k] is the offset of its 8 codes inside a layer's pool minus the slab term
// (FA_OOB, or -1 when WIDE, for a row without a page).  WIDE pools (a layer of 2 GiB or
// more) store through 64-bit addresses, a row without a page then writes a dummy
// workspace slot.  The data path has no per-lane branch, so the compiler counts
// outstanding loads exactly (s_waitcnt vmcnt(N) instead of vmcnt(0)) and later slabs'
// loads stay in flight.
template <int K, bool WIDE> struct ThreadMap {
  uint32_t src;  // offset of vector 0 from its row block's first row
  typename std::conditional<WIDE, int64_t, uint32_t>::type dst[K];
  int nreg;         // vectors of the share held in registers (whole workgroup)
  int64_t blk_bytes;  // bytes between row blocks k and k + 1 (FA_DATA_THREADS vectors)
  int range[K];     // bytes of row block k inside the register part (0 if none)
};

__device__ __forceinline__ int64_t vec_src(const FusedArgs &a, int v) {
  const int64_t row_bytes = 4LL * a.n_heads * a.head_dim;
  return (int64_t)(v >> a.vpt_log2) * row_bytes + (v & ((1 << a.vpt_log2) - 1)) * 16;
}

// Slab order.  Concurrent accesses that all sit at the same offset modulo 4 KiB load the
// memory system unevenly, and address bit 11 matters most: on MI355X a walk over one
// 256-byte column of every 4 KiB row reads ~7% slower than one taking column j from half
// the rows and j ^ 8 (the other 2 KiB half) from the other half.  Both sides of the append
// have such offsets: a slab (kv, h) sits at kv * 2 KiB + h * 256 B in a token row [2][H][D]
// of bf16, and at kv * 16 KiB + h * 2 KiB in a pool page [2][H][P][D] of codes (H = 8,
// D = 128, P = 16).  So each layer's slabs go in pairs (K h, V h ^ m), m = H - 1 for a
// power-of-two H (else 1), even workgroups taking K h then V h ^ m and odd ones V h ^ m
// then K h: at every step the two halves of the chip work on slabs whose offsets differ
// in K/V and in every head bit, on the read side and on the write side, and every slab is
// one step apart between the halves (one step of the exchange's look-ahead).  An odd head
// count pairs K h with V h.  Sequence index q -> physical slab l * 2H + kv * H + h: the
// index of scales, exchange slots and pool slabs.
__device__ __forceinline__ int phys_slab(const FusedArgs &a, int q) {
  const int two_h = 2 * a.n_heads;
  const int l = q / two_h, r = q - l * two_h;
  const int i = r >> 1, kv = (r & 1) ^ (int)(blockIdx.x & 1);
  const int m = (a.n_heads & 1) ? 0 : ((a.n_heads & (a.n_heads - 1)) == 0 ? a.n_heads - 1 : 1);
  return l * two_h + kv * a.n_heads + (kv ? (i ^ m) : i);
}

__device__ __forceinline__ const char *slab_src(const FusedArgs &a, int s, int64_t t_lo) {
  const int two_h = 2 * a.n_heads;
  const int l = s / two_h, j = s - l * two_h;
  return reinterpret_cast<const char *>(a.x + (int64_t)l * a.x_layer_stride + t_lo * two_h * a.head_dim +
                                        (int64_t)j * a.head_dim);
}
__device__ __forceinline__ uint8_t *slab_dst(const FusedArgs &a, int s) {
  const int two_h = 2 * a.n_heads;
  const int l = s / two_h, j = s - l * two_h;
  return a.pool + (int64_t)l * a.pool_layer_stride + (int64_t)j * a.page_size * a.head_dim;
}

// Vector k*FA_DATA_THREADS + tid lies FA_DATA_THREADS / vpt rows after vector tid, in
// the same column, so one per-lane offset serves every k: row block k gets a resource
// of its own whose num_records ends at the last row of the register part.
template <int K, bool WIDE>
__device__ __forceinline__ void load_share(const FusedArgs &a, const ThreadMap<K, WIDE> &m, int s, int64_t t_base,
                                           uint4 (&r)[K]) {
  const char *base = slab_src(a, s, t_base);
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const __amdgpu_buffer_rsrc_t rs = rsrc(base + k * m.blk_bytes, m.range[k]);
    const zx_v4u q = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)m.src, 0, FA_NT);
    r[k] = make_uint4(q.x, q.y, q.z, q.w);
  }
}

template <int K, bool SPILL, bool WIDE>
__device__ __forceinline__ uint32_t share_max(const FusedArgs &a, const ThreadMap<K, WIDE> &m, int s, int64_t t_lo,
                                              int nv, const uint4 (&r)[K]) {
  uint32_t mx = 0;  // two packed 16-bit maxes; lanes past the share loaded zeros
#pragma unroll
  for (int k = 0; k < K; ++k) mx = absmax_acc(mx, r[k]);
  if (SPILL && nv > m.nreg) {
    const char *base = slab_src(a, s, t_lo);
    for (int v = m.nreg + threadIdx.x; v < nv; v += FA_DATA_THREADS)
      mx = absmax_acc(mx, *reinterpret_cast<const uint4 *>(base + vec_src(a, v)));
  }
  return fold16(mx);
}

__device__ __forceinline__ void nt_store8(uint8_t *p, uint2 v) {
  zx_v2u w = {v.x, v.y};
  __builtin_nontemporal_store(w, reinterpret_cast<zx_v2u *>(p));
}

// dst: the slab's base in the pool, or nullptr for a padding step (nothing is stored).
template <int K, bool SPILL, bool WIDE>
__device__ __forceinline__ void encode_share(const FusedArgs &a, const ThreadMap<K, WIDE> &m, int s, int64_t t_lo,
                                             int nv, const uint4 (&r)[K], float sc, uint8_t *dst,
                                             uint8_t *dummy) {
  const QuantScale q = quant_scale(sc);
  if constexpr (WIDE) {
#pragma unroll
    for (int k = 0; k < K; ++k) nt_store8(dst && m.dst[k] >= 0 ? dst + m.dst[k] : dummy, quant8(r[k], q));
  } else {
    const __amdgpu_buffer_rsrc_t rd = rsrc(dst ? dst : a.pool, dst ? FA_RANGE : 0);
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const uint2 c = quant8(r[k], q);
      const zx_v2u w = {c.x, c.y};
      __builtin_amdgcn_raw_buffer_store_b64(w, rd, (int)m.dst[k], 0, FA_NT);
    }
  }
  if (SPILL && dst && nv > m.nreg) {
    const char *base = slab_src(a, s, t_lo);
    for (int v = m.nreg + threadIdx.x; v < nv; v += FA_DATA_THREADS) {
      const int64_t off = a.tok_off[t_lo + (v >> a.vpt_log2)];
      const uint4 x = *reinterpret_cast<const uint4 *>(base + vec_src(a, v));
      if (off >= 0) nt_store8(dst + off + (v & ((1 << a.vpt_log2) - 1)) * 8, quant8(x, q));
    }
  }
}

// Data wave: fold its max into the workgroup's LDS slot for slab s.
__device__ __forceinline__ void contribute(FusedShared &sh, int s, uint32_t mx, bool real) {
  mx = group_max(mx, 64);
  if (real && (threadIdx.x & 63) == 0) {
    const int slot = s & (FA_SLOTS - 1);
    __hip_atomic_fetch_max(&sh.max[slot], mx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    ZX_COMPILER_FENCE();
    __hip_atomic_fetch_add(&sh.cnt[slot], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
}

// Data wave: wait for slab s's scale; false if the launch was aborted.
__device__ __forceinline__ bool wait_ready(const FusedShared &sh, int s, float &sc) {
  const int slot = s & (FA_SLOTS - 1);
  while (ld_lds(&sh.ready[slot]) != (uint32_t)(s + 1)) {
    if (ld_lds(&sh.abort)) return false;
    __builtin_amdgcn_s_sleep(1);
  }
  ZX_COMPILER_FENCE();
  sc = __uint_as_float(ld_lds(reinterpret_cast<const uint32_t *>(&sh.scale[slot])));
  return true;
}

// Control wave: workgroup <-> device protocol, all slabs in order.  Publishes a slab as
// soon as the data waves' contributions are in (up to pub_ahead past the oldest
// unresolved one), and resolves the oldest published slab once every workgroup's slot
// is filled.  Returns false on timeout or abort.
__device__ __forceinline__ bool control_loop(const FusedArgs &a, FusedShared &sh, int S, int S_pad,
                                             uint32_t G, int pub_ahead) {
  const int lane = threadIdx.x & 63;
  int next_pub = 0, next_res = 0;
  uint64_t t_progress = __builtin_amdgcn_s_memrealtime();
  while (next_res < S) {
    bool progress = false;
    while (next_pub < S && next_pub < next_res + pub_ahead &&
           ld_lds(&sh.cnt[next_pub & (FA_SLOTS - 1)]) == (uint32_t)FA_DATA_WAVES) {
      const int slot = next_pub & (FA_SLOTS - 1);
      ZX_COMPILER_FENCE();
      const uint32_t mx = ld_lds(&sh.max[slot]);
      if (lane == 0) {
        __hip_atomic_store(&a.slots[(int64_t)phys_slab(a, next_pub) * G + blockIdx.x], mx + 1u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        sh.max[slot] = 0;
        sh.cnt[slot] = 0;
      }
      ++next_pub;
      progress = true;
    }
    if (next_res < next_pub) {
      const uint32_t *row = a.slots + (int64_t)phys_slab(a, next_res) * G;
      uint32_t mx = 0;
      bool full = true;
      for (uint32_t i = lane; i < G; i += 64) {
        const uint32_t v = __hip_atomic_load(&row[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        full = full && v != 0u;
        mx = max(mx, v);
      }
      if (__ballot(!full) == 0) {
        mx = group_max(mx, 64) - 1u;
        const float sc = scale_from_amax_bits(mx << 16);
        const int slot = next_res & (FA_SLOTS - 1);
        if (lane == 0) {
          if (blockIdx.x == 0) a.scales[phys_slab(a, next_res)] = sc;
          sh.scale[slot] = sc;
          ZX_COMPILER_FENCE();
          __hip_atomic_store(&sh.ready[slot], (uint32_t)(next_res + 1), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_WORKGROUP);
        }
        ++next_res;
        progress = true;
      }
    }
    if (progress) {
      t_progress = __builtin_amdgcn_s_memrealtime();
      continue;
    }
    if (ld_agent(a.abort_flag) || __builtin_amdgcn_s_memrealtime() - t_progress > a.spin_ticks) return false;
    __builtin_amdgcn_s_sleep(1);
  }
  // padding steps past the last slab: scale 1, nothing published
  for (int s = S; s < S_pad; ++s) {
    const int slot = s & (FA_SLOTS - 1);
    if (lane == 0) {
      sh.scale[slot] = 1.0f;
      ZX_COMPILER_FENCE();
      __hip_atomic_store(&sh.ready[slot], (uint32_t)(s + 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
  }
  return true;
}

// K: 16-byte vectors per data thread per slab kept in registers; NB: register buffers
// (the data waves run NB - 1 slabs ahead of the oldest unresolved one).
// SPILL: some share holds more vectors than the registers (extra loops re-read them);
// without it the data path is straight-line code between waits.
template <int K, int NB, bool SPILL, bool WIDE>
__global__ void __launch_bounds__(FA_THREADS, 1) kv_append_fused_kernel(FusedArgs a) {
  static_assert(NB + 1 <= FA_SLOTS, "slot ring too small");
  __shared__ FusedShared sh;
  const uint32_t G = gridDim.x;
  const int64_t t_lo = (int64_t)blockIdx.x * a.n_tok / G;
  const int64_t t_hi = (int64_t)(blockIdx.x + 1) * a.n_tok / G;
  const int nv = (int)(t_hi - t_lo) << a.vpt_log2;
  const int S = a.n_layers * 2 * a.n_heads;
  if (threadIdx.x < FA_SLOTS) {
    sh.max[threadIdx.x] = 0;
    sh.cnt[threadIdx.x] = 0;
    sh.ready[threadIdx.x] = 0;
  }
  if (threadIdx.x == 0) sh.abort = 0;
  __syncthreads();

  const int S_pad = (int)ceil_div(S, NB) * NB;
  if (threadIdx.x >= FA_DATA_THREADS) {  // control wave
    if (!control_loop(a, sh, S, S_pad, G, NB) && threadIdx.x == FA_DATA_THREADS) {
      __hip_atomic_fetch_or(a.abort_flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (a.err) atomicOr(a.err, ZX_KERR_SPIN);
      __hip_atomic_store(&sh.abort, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    return;
  }

  ThreadMap<K, WIDE> m;
  m.nreg = nv < K * FA_DATA_THREADS ? nv : K * FA_DATA_THREADS;
  // a workgroup with an empty share bases its (all out-of-range) loads at token 0
  const int64_t t_base = nv > 0 ? t_lo : 0;
  {
    const int64_t row_bytes = 4LL * a.n_heads * a.head_dim;
    const int rows_blk = FA_DATA_THREADS >> a.vpt_log2, rows_reg = m.nreg >> a.vpt_log2;
    m.src = (uint32_t)vec_src(a, threadIdx.x);
    m.blk_bytes = rows_blk * row_bytes;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int rows = rows_reg - k * rows_blk;
      m.range[k] = rows > 0 ? (int)(rows * row_bytes) : 0;
    }
  }
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int v = k * FA_DATA_THREADS + threadIdx.x;
    const bool live = v < m.nreg;
    const int64_t off = live ? a.tok_off[t_lo + (v >> a.vpt_log2)] : -1;
    const int64_t d = off < 0 ? -1 : off + (v & ((1 << a.vpt_log2) - 1)) * 8;
    if constexpr (WIDE) m.dst[k] = d;
    else m.dst[k] = d < 0 ? FA_OOB : (uint32_t)d;
  }
  uint8_t *dummy = reinterpret_cast<uint8_t *>(a.abort_flag) + 64 + 8 * (threadIdx.x & 15);

  // Slabs past the end are clamped to the last one: the loads stay unconditional (and
  // valid) and their maxes are simply not contributed.
  auto slab = [&](int q) { return phys_slab(a, q < S ? q : S - 1); };
  uint4 buf[NB][K];
#pragma unroll
  for (int i = 0; i < NB; ++i) load_share<K, WIDE>(a, m, slab(i), t_base, buf[i]);
#pragma unroll
  for (int i = 0; i + 1 < NB; ++i) contribute(sh, i, share_max<K, SPILL, WIDE>(a, m, slab(i), t_lo, nv, buf[i]), i < S);

  // step q (buffer i = q % NB): reduce q + NB - 1 (loaded during step q - 1), wait for
  // slab q's scale, encode q, refill the buffer with q + NB.  Reducing first hands the
  // max to the control wave before this wave blocks on a scale, so the device-wide round
  // trip of slab q + NB - 1 starts as early as its data allows.  The slab count is padded
  // to a multiple of NB so every unrolled step is unconditional (padded steps encode into
  // the dummy slot; the control wave marks them ready at the end); an aborted wait leaves
  // the kernel directly.
  for (int q0 = 0; q0 < S_pad; q0 += NB) {
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int q = q0 + i;
      const int j = (i + NB - 1) % NB;  // constant after unrolling
      const int r = q + NB - 1;
      contribute(sh, r, share_max<K, SPILL, WIDE>(a, m, slab(r), t_lo, nv, buf[j]), r < S);
      float sc;
      if (!wait_ready(sh, q, sc)) return;
      encode_share<K, SPILL, WIDE>(a, m, slab(q), t_lo, nv, buf[i], sc, q < S ? slab_dst(a, slab(q)) : nullptr, dummy);
      load_share<K, WIDE>(a, m, slab(q + NB), t_base, buf[i]);
    }
  }
}

// ------------------------------------------------------------------ host side

#ifndef FA_K_CHOICE
#define FA_K_CHOICE 5
#endif
// Register buffers: 5 (four slabs of look-ahead, 127 VGPRs) where the data path is
// straight-line code; 4 where the re-read loops (SPILL) or 64-bit stores (WIDE) need the
// registers (NB = 5 spills there).  On configs[1], NB = 3 / 4 / 5 run 3.33 / 3.15 /
// 3.12 ms per call.
constexpr int FA_K = FA_K_CHOICE;
#define FA_KERNEL(spill, wide) kv_append_fused_kernel<FA_K, ((spill) || (wide)) ? 4 : 5, spill, wide>

static int fused_supported() {
  static int cached[64] = {0};
  int dev = 0;
  ZX_TRY_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= 64) return fail(ZX_ERR_UNSUPPORTED, "device index out of range");
  if (!cached[dev]) {
    int coop = 0, fits = 1;
    ZX_TRY_HIP(hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev));
    const void *fns[4] = {reinterpret_cast<const void *>(FA_KERNEL(false, false)),
                          reinterpret_cast<const void *>(FA_KERNEL(true, false)),
                          reinterpret_cast<const void *>(FA_KERNEL(false, true)),
                          reinterpret_cast<const void *>(FA_KERNEL(true, true))};
    for (const void *fn : fns) {
      int per_cu = 0;
      ZX_TRY_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, FA_THREADS, 0));
      fits = fits && per_cu >= 1;
    }
    cached[dev] = (coop && fits) ? 1 : -1;
  }
  if (cached[dev] < 0) return fail(ZX_ERR_UNSUPPORTED, "device cannot co-schedule the single-pass append");
  return ZX_OK;
}

// The single pass pays a device-wide exchange per slab (~3.6 us on MI355X whatever the
// slab's size) and fills its pipeline over the first slabs; two passes move 5 B per
// element against 3 but no exchange, and below the Infinity Cache's size their second
// read comes from it.  Measured whole calls (MI355X, D = 128, H = 8), single / two passes:
// 74,752 tokens x 1 layer 0.147 / 0.128 ms, x 2 layers 0.230 / 0.259, x 16 1.430 / 2.106;
// 32,768 tokens (share = 43% of the registers) x 16 layers 0.917 / 0.890; 131,072 tokens
// (share = 1.7x the registers, tail re-read) x 1 layer 0.228 / 0.217, x 4 0.890 / 0.914.
// So: a share between half and twice what the registers hold, and at least 32 slabs.
bool append_fused_preferred(int64_t n_tok, int32_t head_dim, int64_t n_slabs) {
  const int64_t share = ceil_div(n_tok, num_cus()) * (head_dim / 8);
  const int64_t regs = (int64_t)FA_K * FA_DATA_THREADS;
  return 2 * share >= regs && share <= 2 * regs && n_slabs >= 32;
}

// workspace: abort flag (+ 60 B pad) | dummy store slots (128 B) | slots [S][G]
size_t append_fused_workspace_bytes(int32_t n_layers, int32_t n_heads) {
  const size_t S = (size_t)n_layers * 2 * n_heads;
  return 256 + align256(S * (size_t)num_cus() * 4);
}

int append_fused(const uint16_t *x, int64_t x_layer_stride, int32_t n_layers, int64_t n_tok, int32_t n_heads,
                 int32_t head_dim, const int64_t *tok_off, uint8_t *pool, int64_t pool_layer_stride,
                 int32_t page_size, float *scales, int32_t *err, void *ws, hipStream_t st) {
  int rc = fused_supported();
  if (rc) return rc;
  const int G = num_cus();
  if (ceil_div(n_tok, G) * (head_dim / 8) >= (1LL << 30))
    return fail(ZX_ERR_UNSUPPORTED, "fused append: share too large");
  // source offsets of the register part are 32-bit buffer offsets
  if ((int64_t)(FA_K * FA_DATA_THREADS / (head_dim / 8) + 1) * 4 * n_heads * head_dim > FA_RANGE)
    return fail(ZX_ERR_UNSUPPORTED, "fused append: token rows too long");
  const int64_t S = (int64_t)n_layers * 2 * n_heads;
  char *w = static_cast<char *>(ws);
  FusedArgs a;
  a.x = x;
  a.x_layer_stride = x_layer_stride;
  a.n_tok = n_tok;
  a.n_layers = n_layers;
  a.n_heads = n_heads;
  a.head_dim = head_dim;
  a.page_size = page_size;
  a.vpt_log2 = head_dim == 64 ? 3 : (head_dim == 128 ? 4 : 5);
  a.tok_off = tok_off;
  a.pool = pool;
  a.pool_layer_stride = pool_layer_stride;
  a.scales = scales;
  a.abort_flag = reinterpret_cast<uint32_t *>(w);
  a.slots = reinterpret_cast<uint32_t *>(w + 256);
  a.err = err;
  a.spin_ticks = wait_bound_ticks();  // default 2 s without progress (zx_set_wait_bound_us)
  // the abort flag and every slot start at zero: one fill kernel (not a memset, so the
  // sequence stays valid inside a captured graph) over the header and the slots
  if ((rc = fill_u32(a.abort_flag, (256 + S * G * 4) / 4, 0, st))) return rc;
  void *args[] = {&a};
  const bool spill = ceil_div(n_tok, G) * (head_dim / 8) > (int64_t)FA_K * FA_DATA_THREADS;
  const bool wide = pool_layer_stride > FA_RANGE;  // pool offsets beyond 32-bit buffer offsets
  const void *fn = spill ? (wide ? reinterpret_cast<const void *>(FA_KERNEL(true, true))
                                 : reinterpret_cast<const void *>(FA_KERNEL(true, false)))
                         : (wide ? reinterpret_cast<const void *>(FA_KERNEL(false, true))
                                 : reinterpret_cast<const void *>(FA_KERNEL(false, false)));
  ZX_TRY_HIP(hipLaunchCooperativeKernel(fn, dim3(G), dim3(FA_THREADS), args, 0, st));
  return check_launch("kv_append_fused");
}

}  // namespace zx
