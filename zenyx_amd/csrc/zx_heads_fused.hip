// zx_heads_fused.hip -- single-pass FP8 quantisation with one scale per (outer, head) slab
// (FP8KVQuantizer.quantize, README.md:157, 329; layout [n_outer][n_batch][n_heads][run]).
//
// A slab's scale needs its amax over all n_batch runs before any code can be written.  Each
// run is cut into m contiguous member shares small enough for registers, so a slab has
// g = n_batch * m members, one workgroup each; the grid holds floor(CUs / g) such groups
// (cooperative launch: every workgroup is resident), and group k takes slabs k, k + groups,
// k + 2 groups, ...  Inside a workgroup the protocol of the fused paged append is used:
//   * 15 data waves keep NB steps (slabs) of their member share in registers; at step i a
//     wave reduces step i + NB - 1 (loaded during step i - 1) and hands its max to the
//     workgroup, waits for step i's scale, encodes step i and refills that buffer with step
//     i + NB, so loads stay in flight and no block-wide barrier is taken;
//   * the control wave (the 16th) publishes the workgroup's max (plus one) into its own
//     device-coherent slot of the slab (slots start at zero), reads the g slots of the oldest
//     published slab until none is zero and broadcasts the scale through LDS.
// Each element is read from HBM once (2 B) and its code written once (1 B).  Loads and
// stores go through buffer resources whose range ends at the member share, so lanes past
// it need no branch.  Every wait is bounded in wall time; a timeout raises a global abort
// flag that releases every other waiter, so all waves always exit.
#include "zx_internal.h"

namespace zx {

constexpr int HF_THREADS = 1024;
constexpr int HF_DATA_WAVES = 15;
constexpr int HF_DATA_THREADS = HF_DATA_WAVES * 64;
#ifndef HF_K_CHOICE
#define HF_K_CHOICE 6
#endif
#ifndef HF_PLAN_SEARCH
#define HF_PLAN_SEARCH 1
#endif
constexpr int HF_K = HF_K_CHOICE;           // 16-byte vectors per data thread per step
constexpr int HF_NB = 4;                    // steps in flight (register buffers)
constexpr int HF_SLOTS = 8;                 // LDS ring of per-step reduction slots (>= NB + 1)
constexpr int64_t HF_SHARE_MAX = (int64_t)HF_K * HF_DATA_THREADS;  // vectors per member share
// A slot holds a member's share max (a bf16 magnitude, at most 0x7FFF) plus one, so the
// zeroed workspace reads as "not published yet" (one fill clears flag and slots together).

struct HeadsFusedArgs {
  const uint16_t *x;
  uint8_t *codes;
  float *scales;
  int64_t n_batch, n_heads;
  int64_t vpr;     // 16-byte vectors (8 elements) per run
  int64_t share;   // vectors per member share (the last share of a run may be shorter)
  int32_t m;       // member shares per run
  int32_t g;       // members per slab = n_batch * m
  int32_t n_groups;
  int32_t n_slabs;  // n_outer * n_heads
  uint32_t *slots;  // [n_slabs][g] each member's share max (bf16 magnitude) + 1, 0 until published
  uint32_t *abort_flag;
  int32_t *err;
  uint64_t spin_ticks;  // bound of one wait in s_memrealtime ticks (100 MHz)
};

struct HeadsShared {
  uint32_t max[HF_SLOTS];    // running max of the data waves' contributions
  uint32_t cnt[HF_SLOTS];    // data waves that contributed
  uint32_t ready[HF_SLOTS];  // i + 1 once step i's scale is final
  float scale[HF_SLOTS];
  uint32_t abort;
};

// LDS flags between the waves of one workgroup: DS instructions of a wave execute in
// program order, so relaxed LDS atomics plus compiler-only fences order them (acquire /
// release orderings would drain every outstanding global load of the data waves).
#define HF_COMPILER_FENCE() asm volatile("" ::: "memory")
__device__ __forceinline__ uint32_t hf_ld_lds(const uint32_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

typedef unsigned int hf_v4u __attribute__((ext_vector_type(4)));
typedef unsigned int hf_v2u __attribute__((ext_vector_type(2)));
constexpr int HF_NT = 2;  // nontemporal: each byte is moved exactly once
__device__ __forceinline__ __amdgpu_buffer_rsrc_t hf_rsrc(const void *base, int num_records) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, num_records, 0x00020000);
}

// This workgroup's member share of slab s: first vector (index into x in 16-byte vectors,
// codes in 8-byte words) and length in vectors.
struct Share {
  int64_t v0;
  int32_t n;
};
__device__ __forceinline__ Share member_share(const HeadsFusedArgs &a, int s, int member) {
  const int64_t o = s / a.n_heads, h = s - o * a.n_heads;
  const int b = member / a.m, part = member - b * a.m;
  const int64_t lo = (int64_t)part * a.share;
  const int64_t hi = lo + a.share < a.vpr ? lo + a.share : a.vpr;
  Share r;
  r.v0 = ((o * a.n_batch + b) * a.n_heads + h) * a.vpr + lo;
  r.n = hi > lo ? (int32_t)(hi - lo) : 0;
  return r;
}

__device__ __forceinline__ void hf_load(const HeadsFusedArgs &a, const Share &sh, uint4 (&r)[HF_K]) {
  const __amdgpu_buffer_rsrc_t rs = hf_rsrc(a.x + sh.v0 * 8, sh.n * 16);
#pragma unroll
  for (int k = 0; k < HF_K; ++k) {
    const hf_v4u q =
        __builtin_amdgcn_raw_buffer_load_b128(rs, (k * HF_DATA_THREADS + (int)threadIdx.x) * 16, 0, HF_NT);
    r[k] = make_uint4(q.x, q.y, q.z, q.w);
  }
}

__device__ __forceinline__ uint32_t hf_max(const uint4 (&r)[HF_K]) {
  uint32_t mx = 0;  // two packed 16-bit maxes; lanes past the share loaded zeros
#pragma unroll
  for (int k = 0; k < HF_K; ++k) mx = absmax_acc(mx, r[k]);
  return fold16(mx);
}

// store: false for a padding step (the resource then has no records: nothing is written).
__device__ __forceinline__ void hf_encode(const HeadsFusedArgs &a, const Share &sh, bool store,
                                          const uint4 (&r)[HF_K], float sc) {
  const QuantScale q = quant_scale(sc);
  const __amdgpu_buffer_rsrc_t rd = hf_rsrc(a.codes + sh.v0 * 8, store ? sh.n * 8 : 0);
#pragma unroll
  for (int k = 0; k < HF_K; ++k) {
    const uint2 c = quant8(r[k], q);
    const hf_v2u w = {c.x, c.y};
    __builtin_amdgcn_raw_buffer_store_b64(w, rd, (k * HF_DATA_THREADS + (int)threadIdx.x) * 8, 0, HF_NT);
  }
}

// Data wave: fold its max into the workgroup's LDS slot for step i.
__device__ __forceinline__ void hf_contribute(HeadsShared &sh, int i, uint32_t mx, bool real) {
  mx = group_max(mx, 64);
  if (real && (threadIdx.x & 63) == 0) {
    const int slot = i & (HF_SLOTS - 1);
    __hip_atomic_fetch_max(&sh.max[slot], mx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    HF_COMPILER_FENCE();
    __hip_atomic_fetch_add(&sh.cnt[slot], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
}

// Data wave: wait for step i's scale; false if the launch was aborted.
__device__ __forceinline__ bool hf_wait_ready(const HeadsShared &sh, int i, float &sc) {
  const int slot = i & (HF_SLOTS - 1);
  while (hf_ld_lds(&sh.ready[slot]) != (uint32_t)(i + 1)) {
    if (hf_ld_lds(&sh.abort)) return false;
    __builtin_amdgcn_s_sleep(1);
  }
  HF_COMPILER_FENCE();
  sc = __uint_as_float(hf_ld_lds(reinterpret_cast<const uint32_t *>(&sh.scale[slot])));
  return true;
}

// Control wave: publishes step i (slab group + i * n_groups) once the data waves' maxes are
// in (up to NB steps past the oldest unresolved one) and resolves the oldest published step
// once all g members' slots are filled.  Returns false on timeout or abort.
__device__ bool hf_control_loop(const HeadsFusedArgs &a, HeadsShared &sh, int group, int member, int steps,
                                int steps_pad) {
  const int lane = threadIdx.x & 63;
  const uint32_t g = (uint32_t)a.g;
  int next_pub = 0, next_res = 0;
  uint64_t t_progress = __builtin_amdgcn_s_memrealtime();
  while (next_res < steps) {
    bool progress = false;
    while (next_pub < steps && next_pub < next_res + HF_NB &&
           hf_ld_lds(&sh.cnt[next_pub & (HF_SLOTS - 1)]) == (uint32_t)HF_DATA_WAVES) {
      const int slot = next_pub & (HF_SLOTS - 1);
      HF_COMPILER_FENCE();
      const uint32_t mx = hf_ld_lds(&sh.max[slot]);
      if (lane == 0) {
        const int64_t s = group + (int64_t)next_pub * a.n_groups;
        __hip_atomic_store(&a.slots[s * g + member], mx + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        sh.max[slot] = 0;
        sh.cnt[slot] = 0;
      }
      ++next_pub;
      progress = true;
    }
    if (next_res < next_pub) {
      const int64_t s = group + (int64_t)next_res * a.n_groups;
      const uint32_t *row = a.slots + s * g;
      uint32_t mx = 0;
      bool full = true;
      for (uint32_t i = lane; i < g; i += 64) {
        const uint32_t v = __hip_atomic_load(&row[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        full = full && v != 0u;
        mx = max(mx, v);
      }
      if (__ballot(!full) == 0) {
        mx = group_max(mx, 64) - 1u;
        const float sc = scale_from_amax_bits(mx << 16);
        const int slot = next_res & (HF_SLOTS - 1);
        if (lane == 0) {
          if (member == 0) a.scales[s] = sc;
          sh.scale[slot] = sc;
          HF_COMPILER_FENCE();
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
    if (__hip_atomic_load(a.abort_flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ||
        __builtin_amdgcn_s_memrealtime() - t_progress > a.spin_ticks)
      return false;
    __builtin_amdgcn_s_sleep(1);
  }
  for (int i = steps; i < steps_pad; ++i) {  // padding steps: scale 1, nothing published
    const int slot = i & (HF_SLOTS - 1);
    if (lane == 0) {
      sh.scale[slot] = 1.0f;
      HF_COMPILER_FENCE();
      __hip_atomic_store(&sh.ready[slot], (uint32_t)(i + 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
  }
  return true;
}

__global__ void __launch_bounds__(HF_THREADS, 1) heads_fused_kernel(HeadsFusedArgs a) {
  static_assert(HF_NB + 1 <= HF_SLOTS, "slot ring too small");
  __shared__ HeadsShared sh;
  const int group = blockIdx.x / a.g, member = blockIdx.x - group * a.g;
  // steps of this group: slabs group, group + n_groups, ... (none for a spare group)
  const int steps = group < a.n_slabs ? (a.n_slabs - group + a.n_groups - 1) / a.n_groups : 0;
  if (steps == 0) return;
  const int steps_pad = (steps + HF_NB - 1) / HF_NB * HF_NB;
  if (threadIdx.x < HF_SLOTS) {
    sh.max[threadIdx.x] = 0;
    sh.cnt[threadIdx.x] = 0;
    sh.ready[threadIdx.x] = 0;
  }
  if (threadIdx.x == 0) sh.abort = 0;
  __syncthreads();

  if (threadIdx.x >= HF_DATA_THREADS) {  // control wave
    if (!hf_control_loop(a, sh, group, member, steps, steps_pad) && threadIdx.x == HF_DATA_THREADS) {
      __hip_atomic_fetch_or(a.abort_flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (a.err) atomicOr(a.err, ZX_KERR_SPIN);
      __hip_atomic_store(&sh.abort, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    return;
  }

  // Steps past the last real one load the last real slab again (valid addresses) and
  // neither contribute nor store.
  auto slab_of = [&](int i) { return group + (i < steps ? i : steps - 1) * a.n_groups; };
  uint4 buf[HF_NB][HF_K];
#pragma unroll
  for (int i = 0; i < HF_NB; ++i) hf_load(a, member_share(a, slab_of(i), member), buf[i]);
#pragma unroll
  for (int i = 0; i + 1 < HF_NB; ++i) hf_contribute(sh, i, hf_max(buf[i]), i < steps);

  for (int i0 = 0; i0 < steps_pad; i0 += HF_NB) {
#pragma unroll
    for (int j = 0; j < HF_NB; ++j) {
      const int i = i0 + j;
      const int jr = (j + HF_NB - 1) % HF_NB;  // buffer of step i + NB - 1 (constant after unrolling)
      hf_contribute(sh, i + HF_NB - 1, hf_max(buf[jr]), i + HF_NB - 1 < steps);
      float sc;
      if (!hf_wait_ready(sh, i, sc)) return;
      hf_encode(a, member_share(a, slab_of(i), member), i < steps, buf[j], sc);
      hf_load(a, member_share(a, slab_of(i + HF_NB), member), buf[j]);
    }
  }
}

// ------------------------------------------------------------------ host side

struct HeadsPlan {
  int32_t m, g, n_groups;
  int64_t share;
};

// Member shares per run: m = ceil(vpr / HF_SHARE_MAX), the fewest that fit the registers
// (g = n_batch m members per slab, floor(G / g) groups); with HF_PLAN_SEARCH, the m up to
// twice that which leaves the fewest workgroups idle.  False when one slab needs more
// workgroups than the device holds.
static bool heads_plan(int64_t n_batch, int64_t vpr, int G, HeadsPlan &p) {
  const int64_t m_min = ceil_div(vpr, HF_SHARE_MAX);
  if (n_batch * m_min > G) return false;
  int64_t best_m = m_min, best_used = 0;
  for (int64_t m = m_min; m <= (HF_PLAN_SEARCH ? 2 * m_min : m_min) && n_batch * m <= G; ++m) {
    const int64_t g = n_batch * m, used = (G / g) * g;
    if (used > best_used) best_used = used, best_m = m;
  }
  p.m = (int32_t)best_m;
  p.g = (int32_t)(n_batch * best_m);
  p.n_groups = G / p.g;
  p.share = ceil_div(vpr, best_m);
  return true;
}

static int heads_fused_supported() {
  static int cached[64] = {0};
  int dev = 0;
  ZX_TRY_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= 64) return fail(ZX_ERR_UNSUPPORTED, "device index out of range");
  if (!cached[dev]) {
    int coop = 0, per_cu = 0;
    ZX_TRY_HIP(hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev));
    ZX_TRY_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(
        &per_cu, reinterpret_cast<const void *>(heads_fused_kernel), HF_THREADS, 0));
    cached[dev] = (coop && per_cu >= 1) ? 1 : -1;
  }
  if (cached[dev] < 0) return fail(ZX_ERR_UNSUPPORTED, "device cannot co-schedule the single-pass quantiser");
  return ZX_OK;
}

size_t heads_fused_workspace_bytes(int64_t n_outer, int64_t n_batch, int64_t n_heads, int64_t run) {
  HeadsPlan p;
  if (n_outer <= 0 || n_batch <= 0 || n_heads <= 0 || run <= 0 || !heads_plan(n_batch, ceil_div(run, 8), num_cus(), p))
    return 256;
  return 256 + align256((size_t)n_outer * n_heads * p.g * 4);
}

int heads_fused(const uint16_t *x, int64_t n_outer, int64_t n_batch, int64_t n_heads, int64_t run, uint8_t *codes,
                float *scales, int32_t *err, void *ws, size_t ws_bytes, hipStream_t st) {
  HeadsPlan p;
  if (run % 8 || !heads_plan(n_batch, run / 8, num_cus(), p))
    return fail(ZX_ERR_UNSUPPORTED, "single-pass quantiser: a slab needs more workgroups than the device holds");
  if (n_outer * n_heads >= (1LL << 31) / p.g) return fail(ZX_ERR_UNSUPPORTED, "single-pass quantiser: too many slabs");
  if (ws_bytes < heads_fused_workspace_bytes(n_outer, n_batch, n_heads, run))
    return fail(ZX_ERR_WORKSPACE, "fp8_quant_heads: workspace too small for the single-pass path");
  int rc = heads_fused_supported();
  if (rc) return rc;
  char *w = static_cast<char *>(ws);
  HeadsFusedArgs a;
  a.x = x;
  a.codes = codes;
  a.scales = scales;
  a.n_batch = n_batch;
  a.n_heads = n_heads;
  a.vpr = run / 8;
  a.share = p.share;
  a.m = p.m;
  a.g = p.g;
  a.n_groups = p.n_groups;
  a.n_slabs = (int32_t)(n_outer * n_heads);
  a.abort_flag = reinterpret_cast<uint32_t *>(w);
  a.slots = reinterpret_cast<uint32_t *>(w + 256);
  a.err = err;
  a.spin_ticks = wait_bound_ticks();  // default 2 s without progress (zx_set_wait_bound_us)
  // the abort flag and every slot start at zero: one fill kernel over the header and slots
  if ((rc = fill_u32(a.abort_flag, (256 + (int64_t)a.n_slabs * p.g * 4) / 4, 0, st))) return rc;
  void *args[] = {&a};
  ZX_TRY_HIP(hipLaunchCooperativeKernel(reinterpret_cast<const void *>(heads_fused_kernel),
                                        dim3((unsigned)(p.n_groups * p.g)), dim3(HF_THREADS), args, 0, st));
  return check_launch("heads_fused");
}

}  // namespace zx
