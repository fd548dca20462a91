// zx_belady.hip -- Belady victim selection (zenyx/streaming/belady.py:39-51) and the
// next-use tables it needs.  The trace-level simulator lives in zx_belady_sim.hip.
#include <hipcub/hipcub.hpp>

#include "zx_internal.h"

namespace zx {

// ------------------------------------------------------------------ argmax

struct Best {
  int64_t key, slot;
};

// a beats b: larger key, ties to the smaller slot; {-1, -1} is "none".
__device__ __forceinline__ bool beats(int64_t ka, int64_t sa, int64_t kb, int64_t sb) {
  if (sa < 0) return false;
  if (sb < 0) return true;
  return ka > kb || (ka == kb && sa < sb);
}

__device__ __forceinline__ void wave_best(int64_t &k, int64_t &s) {
  for (int off = 32; off >= 1; off >>= 1) {
    int64_t k2 = __shfl_xor(k, off, 64);
    int64_t s2 = __shfl_xor(s, off, 64);
    if (beats(k2, s2, k, s)) {
      k = k2;
      s = s2;
    }
  }
}

constexpr int AM_THREADS = 256;
constexpr int AM_MAX_BLOCKS = 1024;

__device__ __forceinline__ void block_best(int64_t &k, int64_t &s) {
  __shared__ int64_t kk[AM_THREADS / 64], ss[AM_THREADS / 64];
  wave_best(k, s);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) {
    kk[wid] = k;
    ss[wid] = s;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < AM_THREADS / 64; ++w)
      if (beats(kk[w], ss[w], k, s)) {
        k = kk[w];
        s = ss[w];
      }
  }
}

__global__ void __launch_bounds__(AM_THREADS)
argmax_partial_kernel(const int64_t *keys, const uint8_t *resident, int64_t n, Best *part) {
  int64_t bk = -1, bs = -1;
  for (int64_t i = (int64_t)blockIdx.x * AM_THREADS + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * AM_THREADS) {
    // belady.py:48-50: a slot qualifies when its key is strictly greater than -1
    if (resident[i] && keys[i] > -1 && beats(keys[i], i, bk, bs)) {
      bk = keys[i];
      bs = i;
    }
  }
  block_best(bk, bs);
  if (threadIdx.x == 0) part[blockIdx.x] = Best{bk, bs};
}

__global__ void __launch_bounds__(AM_THREADS)
argmax_final_kernel(const Best *part, int n_part, int64_t *out) {
  int64_t bk = -1, bs = -1;
  for (int i = threadIdx.x; i < n_part; i += AM_THREADS)
    if (beats(part[i].key, part[i].slot, bk, bs)) {
      bk = part[i].key;
      bs = part[i].slot;
    }
  block_best(bk, bs);
  if (threadIdx.x == 0) {
    out[0] = bs;
    out[1] = bs < 0 ? -1 : bk;
  }
}

// Slot updates of the drop-in cache: keys[slot[i]] = key[i], resident[slot[i]] = res[i]
// (the host passes each slot once).  The update arrays may live in pinned host memory.
__global__ void update_slots_kernel(int64_t *keys, uint8_t *resident, int64_t n_slots, const int64_t *slot,
                                    const int64_t *key, const uint8_t *res, int64_t n, int32_t *err) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int64_t s = slot[i];
  if (s < 0 || s >= n_slots) {
    if (err) atomicOr(err, ZX_KERR_PAGE_RANGE);
    return;
  }
  keys[s] = key[i];
  resident[s] = res[i];
}

static int argmax_blocks(int64_t n) {
  int64_t b = ceil_div(n, (int64_t)AM_THREADS * 8);
  if (b < 1) b = 1;
  if (b > AM_MAX_BLOCKS) b = AM_MAX_BLOCKS;
  return (int)b;
}

// ------------------------------------------------------------------ next use

__global__ void iota_check_kernel(const int32_t *trace, int64_t n, int32_t n_pages, int32_t *pos,
                                  int32_t *err) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  pos[i] = (int32_t)i;
  int32_t p = trace[i];
  if ((p < 0 || p >= n_pages) && err) atomicOr(err, ZX_KERR_PAGE_RANGE);
}

__global__ void next_use_kernel(const int32_t *skey, const int32_t *spos, int64_t n, int32_t *next_use,
                                int32_t *prev_use) {
  int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (k >= n) return;
  const int32_t p = skey[k], pos = spos[k];
  next_use[pos] = (k + 1 < n && skey[k + 1] == p) ? spos[k + 1] : ZX_NEVER;
  prev_use[pos] = (k > 0 && skey[k - 1] == p) ? spos[k - 1] : -1;
}

static int key_bits(int32_t n_pages) {
  int b = 1;
  while (b < 31 && (1LL << b) < (int64_t)n_pages) ++b;
  return b;
}



static size_t sort_temp_bytes(int64_t n, int32_t n_pages) {
  size_t temp = 0;
  (void)hipcub::DeviceRadixSort::SortPairs(nullptr, temp, (const int32_t *)nullptr, (int32_t *)nullptr,
                                     (const int32_t *)nullptr, (int32_t *)nullptr, (int)n, 0,
                                     key_bits(n_pages));
  return temp;
}

}  // namespace zx

using namespace zx;

extern "C" size_t zx_belady_argmax_workspace_bytes(int64_t n_slots) {
  return (size_t)argmax_blocks(n_slots > 0 ? n_slots : 1) * sizeof(Best);
}

extern "C" int zx_belady_argmax(const int64_t *keys, const uint8_t *resident, int64_t n_slots, int64_t *out,
                                void *workspace, size_t workspace_bytes, zx_stream_t stream) {
  clear_error();
  ZX_REQUIRE(out && (n_slots == 0 || (keys && resident)), "belady_argmax: null pointer");
  ZX_REQUIRE(n_slots >= 0, "belady_argmax: negative size");
  const int nb = argmax_blocks(n_slots > 0 ? n_slots : 1);
  if (!workspace || workspace_bytes < (size_t)nb * sizeof(Best))
    return fail(ZX_ERR_WORKSPACE, "belady_argmax: workspace too small");
  hipStream_t st = as_stream(stream);
  Best *part = reinterpret_cast<Best *>(workspace);
  argmax_partial_kernel<<<nb, AM_THREADS, 0, st>>>(keys, resident, n_slots, part);
  int rc = check_launch("belady_argmax_partial");
  if (rc) return rc;
  argmax_final_kernel<<<1, AM_THREADS, 0, st>>>(part, nb, out);
  return check_launch("belady_argmax_final");
}

extern "C" int zx_belady_update_slots(int64_t *keys, uint8_t *resident, int64_t n_slots, const int64_t *slot,
                                      const int64_t *key, const uint8_t *res, int64_t n, int32_t *err,
                                      zx_stream_t stream) {
  clear_error();
  ZX_REQUIRE(n >= 0 && n_slots >= 0, "belady_update_slots: negative size");
  if (n == 0) return ZX_OK;
  ZX_REQUIRE(keys && resident && slot && key && res, "belady_update_slots: null pointer");
  update_slots_kernel<<<(unsigned)ceil_div(n, 256), 256, 0, as_stream(stream)>>>(keys, resident, n_slots, slot, key,
                                                                                res, n, err);
  return check_launch("belady_update_slots");
}

extern "C" size_t zx_belady_next_use_workspace_bytes(int64_t n, int32_t n_pages) {
  if (n <= 0) return 256;
  return 3 * align256((size_t)n * 4) + align256(sort_temp_bytes(n, n_pages > 0 ? n_pages : 1));
}

extern "C" int zx_belady_next_use(const int32_t *trace, int64_t n, int32_t n_pages, int32_t *next_use,
                                  int32_t *prev_use, int32_t *err, void *workspace, size_t workspace_bytes,
                                  zx_stream_t stream) {
  clear_error();
  ZX_REQUIRE(n >= 0 && n < 0x7FFFFFFF, "belady_next_use: n out of range");
  ZX_REQUIRE(n_pages > 0, "belady_next_use: n_pages must be positive");
  if (n == 0) return ZX_OK;
  ZX_REQUIRE(trace && next_use && prev_use, "belady_next_use: null pointer");
  const size_t need = zx_belady_next_use_workspace_bytes(n, n_pages);
  if (!workspace || workspace_bytes < need)
    return fail(ZX_ERR_WORKSPACE, "belady_next_use: workspace %zu < %zu bytes", workspace_bytes, need);
  hipStream_t st = as_stream(stream);
  char *ws = reinterpret_cast<char *>(workspace);
  const size_t a = align256((size_t)n * 4);
  int32_t *pos_in = reinterpret_cast<int32_t *>(ws);
  int32_t *key_out = reinterpret_cast<int32_t *>(ws + a);
  int32_t *pos_out = reinterpret_cast<int32_t *>(ws + 2 * a);
  void *temp = ws + 3 * a;
  size_t temp_bytes = need - 3 * a;
  iota_check_kernel<<<(unsigned)ceil_div(n, 256), 256, 0, st>>>(trace, n, n_pages, pos_in, err);
  int rc = check_launch("belady_iota");
  if (rc) return rc;
  ZX_TRY_HIP(hipcub::DeviceRadixSort::SortPairs(temp, temp_bytes, trace, key_out, pos_in, pos_out, (int)n, 0,
                                                key_bits(n_pages), st));
  next_use_kernel<<<(unsigned)ceil_div(n, 256), 256, 0, st>>>(key_out, pos_out, n, next_use, prev_use);
  return check_launch("belady_next_use");
}
