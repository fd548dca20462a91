// zx_tier.hip -- HBM <-> pinned-host tier moves (replaces the synchronous .to(device) /
// .cpu() copies of zenyx/streaming/kv_tiering.py:46, 54, 60).  Runs of pages are merged
// where they are adjacent on both sides and issued as hipMemcpyAsync on the caller's
// (side) stream, so they overlap with kernels on other streams.
#include "zx_common.h"

using namespace zx;

extern "C" int zx_tier_copy_runs(void *dst, const void *src, const int64_t *dst_off, const int64_t *src_off,
                                 int64_t n_runs, int64_t run_bytes, zx_stream_t stream, void *done) {
  clear_error();
  ZX_REQUIRE(n_runs >= 0 && run_bytes > 0, "tier_copy_runs: bad sizes");
  ZX_REQUIRE(n_runs == 0 || (dst && src && dst_off && src_off), "tier_copy_runs: null pointer");
  hipStream_t st = as_stream(stream);
  int64_t i = 0;
  while (i < n_runs) {
    ZX_REQUIRE(dst_off[i] >= 0 && src_off[i] >= 0, "tier_copy_runs: negative offset at run %lld",
               (long long)i);
    int64_t j = i + 1;
    while (j < n_runs && dst_off[j] == dst_off[j - 1] + run_bytes && src_off[j] == src_off[j - 1] + run_bytes)
      ++j;
    ZX_TRY_HIP(hipMemcpyAsync(static_cast<char *>(dst) + dst_off[i], static_cast<const char *>(src) + src_off[i],
                              (size_t)((j - i) * run_bytes), hipMemcpyDefault, st));
    i = j;
  }
  if (done) ZX_TRY_HIP(hipEventRecord(reinterpret_cast<hipEvent_t>(done), st));
  return ZX_OK;
}

// ------------------------------------------------------------------ scattered page moves
//
// One launch moves a whole batch of scattered pages: workgroup w copies pages w, w + G,
// ... with 16-byte loads straight from the source (device memory or pinned host memory
// over PCIe) into the destination.  Each lane keeps ZX_MV_U loads in flight before its
// stores, so a few dozen workgroups cover the PCIe latency; per-page hipMemcpyAsync
// calls would pay a command per 128 KiB instead.
constexpr int ZX_MV_THREADS = 256;
constexpr int ZX_MV_U = 8;
typedef unsigned int zx_mv_v4 __attribute__((ext_vector_type(4)));

__global__ void __launch_bounds__(ZX_MV_THREADS)
tier_move_pages_kernel(char *__restrict__ dst, const char *__restrict__ src, const int64_t *__restrict__ dst_off,
                       const int64_t *__restrict__ src_off, int64_t n, int64_t page_bytes, int64_t dst_bytes,
                       int64_t src_bytes, int32_t *err) {
  const int64_t nv = page_bytes / 16;
  for (int64_t p = blockIdx.x; p < n; p += gridDim.x) {
    const int64_t so = src_off[p], dof = dst_off[p];
    if (so < 0 || dof < 0 || so > src_bytes - page_bytes || dof > dst_bytes - page_bytes) {
      if (threadIdx.x == 0 && err) atomicOr(err, ZX_KERR_PAGE_RANGE);
      continue;
    }
    const zx_mv_v4 *s = reinterpret_cast<const zx_mv_v4 *>(src + so);
    zx_mv_v4 *d = reinterpret_cast<zx_mv_v4 *>(dst + dof);
    for (int64_t i0 = threadIdx.x; i0 < nv; i0 += (int64_t)ZX_MV_THREADS * ZX_MV_U) {
      zx_mv_v4 v[ZX_MV_U];
#pragma unroll
      for (int u = 0; u < ZX_MV_U; ++u) {
        const int64_t i = i0 + (int64_t)u * ZX_MV_THREADS;
        if (i < nv) v[u] = __builtin_nontemporal_load(s + i);
      }
#pragma unroll
      for (int u = 0; u < ZX_MV_U; ++u) {
        const int64_t i = i0 + (int64_t)u * ZX_MV_THREADS;
        if (i < nv) __builtin_nontemporal_store(v[u], d + i);
      }
    }
  }
}

extern "C" int zx_tier_move_pages(void *dst, int64_t dst_bytes, const void *src, int64_t src_bytes,
                                  const int64_t *dst_off, const int64_t *src_off, int64_t n_pages,
                                  int64_t page_bytes, int32_t max_workgroups, int32_t *err, zx_stream_t stream) {
  clear_error();
  ZX_REQUIRE(n_pages >= 0 && page_bytes > 0 && page_bytes % 16 == 0 && dst_bytes >= 0 && src_bytes >= 0,
             "tier_move_pages: bad sizes (page_bytes must be a positive multiple of 16)");
  if (n_pages == 0) return ZX_OK;
  ZX_REQUIRE(dst && src && dst_off && src_off, "tier_move_pages: null pointer");
  ZX_REQUIRE((reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src)) % 16 == 0,
             "tier_move_pages: buffers must be 16-byte aligned");
  const int64_t g = max_workgroups > 0 ? max_workgroups : 32;
  const int blocks = (int)(n_pages < g ? n_pages : g);
  tier_move_pages_kernel<<<blocks, ZX_MV_THREADS, 0, as_stream(stream)>>>(
      static_cast<char *>(dst), static_cast<const char *>(src), dst_off, src_off, n_pages, page_bytes, dst_bytes,
      src_bytes, err);
  return check_launch("tier_move_pages");
}

// ------------------------------------------------------------------ three-tier plan
//
// Belady MIN is a stack algorithm: with one total order of the keys (next use, then
// smaller page id), the pages MIN keeps with capacity c0 are always a subset of those it
// keeps with capacity c0 + c1.  In an exclusive T0 / T1 / T2 hierarchy where T0 sends
// its farthest page to T1 and T1 sends its farthest to T2, T0 is therefore MIN(c0) and
// T0 + T1 is MIN(c0 + c1): the union's victim on a miss is the farthest page of T0 + T1,
// which is either T0's farthest (then it goes from T0 straight to T2) or in T1.  So two
// runs of zx_belady_simulate give the whole three-tier schedule, and this kernel only
// has to line them up per position.

__global__ void tier_plan_src_kernel(const int32_t *__restrict__ prev_use, const uint8_t *__restrict__ miss0,
                                     const uint8_t *__restrict__ miss01, int64_t n, uint8_t *__restrict__ src,
                                     int32_t *__restrict__ v0, int32_t *__restrict__ v1) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const uint8_t s = !miss0[i] ? 0 : (!miss01[i] ? 1 : (prev_use[i] >= 0 ? 2 : 3));
    src[i] = s;
    v0[i] = -1;
    v1[i] = -1;
  }
}

__global__ void tier_plan_victims_kernel(const int32_t *__restrict__ pos, const int32_t *__restrict__ page,
                                         int64_t n_ev, int64_t n, int32_t *__restrict__ v, int32_t *err) {
  for (int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; k < n_ev; k += (int64_t)gridDim.x * blockDim.x) {
    const int32_t p = pos[k];
    if (p >= 0 && p < n) v[p] = page[k];
    else if (err) atomicOr(err, ZX_KERR_POS_RANGE);
  }
}

extern "C" int zx_belady_tier_plan(const int32_t *prev_use, const uint8_t *miss0, const uint8_t *miss01, int64_t n,
                                   const int32_t *e0_pos, const int32_t *e0_page, int64_t n_e0,
                                   const int32_t *e01_pos, const int32_t *e01_page, int64_t n_e01, uint8_t *src,
                                   int32_t *v0, int32_t *v1, int32_t *err, zx_stream_t stream) {
  clear_error();
  ZX_REQUIRE(n >= 0 && n_e0 >= 0 && n_e01 >= 0 && n_e0 <= n && n_e01 <= n, "belady_tier_plan: bad sizes");
  if (n == 0) return ZX_OK;
  ZX_REQUIRE(prev_use && miss0 && miss01 && src && v0 && v1, "belady_tier_plan: null pointer");
  ZX_REQUIRE((n_e0 == 0 || (e0_pos && e0_page)) && (n_e01 == 0 || (e01_pos && e01_page)),
             "belady_tier_plan: null victim list");
  hipStream_t st = as_stream(stream);
  const int blocks = (int)(ceil_div(n, 256) < 8192 ? ceil_div(n, 256) : 8192);
  tier_plan_src_kernel<<<blocks, 256, 0, st>>>(prev_use, miss0, miss01, n, src, v0, v1);
  int rc = check_launch("tier_plan_src");
  if (rc) return rc;
  if (n_e0) {
    const int b = (int)(ceil_div(n_e0, 256) < 8192 ? ceil_div(n_e0, 256) : 8192);
    tier_plan_victims_kernel<<<b, 256, 0, st>>>(e0_pos, e0_page, n_e0, n, v0, err);
    if ((rc = check_launch("tier_plan_victims"))) return rc;
  }
  if (n_e01) {
    const int b = (int)(ceil_div(n_e01, 256) < 8192 ? ceil_div(n_e01, 256) : 8192);
    tier_plan_victims_kernel<<<b, 256, 0, st>>>(e01_pos, e01_page, n_e01, n, v1, err);
    if ((rc = check_launch("tier_plan_victims"))) return rc;
  }
  return ZX_OK;
}
