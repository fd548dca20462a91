// zx_belady.hip -- Belady victim selection (zenyx/streaming/belady.py:39-51) and the
// next-use tables it needs.  The trace-level simulator lives in zx_belady_sim.hip.
#include "zx_internal.h"

namespace zx {

// ------------------------------------------------------------------ argmax

struct Best {
  int64_t key, rank, slot;
};

// a beats b: larger key, ties to the smaller rank, then the smaller slot; slot -1 is
// "none".
__device__ __forceinline__ bool beats(const Best &a, const Best &b) {
  if (a.slot < 0) return false;
  if (b.slot < 0) return true;
  if (a.key != b.key) return a.key > b.key;
  if (a.rank != b.rank) return a.rank < b.rank;
  return a.slot < b.slot;
}

__device__ __forceinline__ Best shfl_best(const Best &b, int off) {
  return Best{__shfl_xor(b.key, off, 64), __shfl_xor(b.rank, off, 64), __shfl_xor(b.slot, off, 64)};
}

__device__ __forceinline__ void wave_best(Best &b) {
  for (int off = 32; off >= 1; off >>= 1) {
    const Best o = shfl_best(b, off);
    if (beats(o, b)) b = o;
  }
}

constexpr int AM_THREADS = 256;
constexpr int AM_MAX_BLOCKS = 1024;

__device__ __forceinline__ void block_best(Best &b) {
  __shared__ Best sb[AM_THREADS / 64];
  wave_best(b);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) sb[wid] = b;
  __syncthreads();
  if (threadIdx.x == 0)
    for (int w = 1; w < AM_THREADS / 64; ++w)
      if (beats(sb[w], b)) b = sb[w];
}

// resident == nullptr: every slot is a candidate; rank == nullptr: a slot's rank is its
// index (ties to the smaller slot).
__global__ void __launch_bounds__(AM_THREADS)
argmax_partial_kernel(const int64_t *keys, const uint8_t *resident, const int64_t *rank, int64_t n, Best *part) {
  Best best{-1, 0, -1};
  for (int64_t i = (int64_t)blockIdx.x * AM_THREADS + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * AM_THREADS) {
    // belady.py:48-50: a slot qualifies when its key is strictly greater than -1
    const Best c{keys[i], rank ? rank[i] : i, i};
    if ((!resident || resident[i]) && c.key > -1 && beats(c, best)) best = c;
  }
  block_best(best);
  if (threadIdx.x == 0) part[blockIdx.x] = best;
}

__global__ void __launch_bounds__(AM_THREADS)
argmax_final_kernel(const Best *part, int n_part, int64_t *out) {
  Best best{-1, 0, -1};
  for (int i = threadIdx.x; i < n_part; i += AM_THREADS)
    if (beats(part[i], best)) best = part[i];
  block_best(best);
  if (threadIdx.x == 0) {
    out[0] = best.slot;
    out[1] = best.slot < 0 ? -1 : best.key;
  }
}

// Slot updates of the drop-in cache: keys[slot[i]] = key[i], and resident[slot[i]] =
// res[i] / rank[slot[i]] = rank_in[i] when those tables are given (the host passes each
// slot once).  The update arrays may live in pinned host memory.
__global__ void update_slots_kernel(int64_t *keys, uint8_t *resident, int64_t *rank, int64_t n_slots,
                                    const int64_t *slot, const int64_t *key, const uint8_t *res,
                                    const int64_t *rank_in, int64_t n, int32_t *err) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int64_t s = slot[i];
  if (s < 0 || s >= n_slots) {
    if (err) atomicOr(err, ZX_KERR_PAGE_RANGE);
    return;
  }
  keys[s] = key[i];
  if (resident) resident[s] = res[i];
  if (rank) rank[s] = rank_in[i];
}

static int argmax_blocks(int64_t n) {
  int64_t b = ceil_div(n, (int64_t)AM_THREADS * 8);
  if (b < 1) b = 1;
  if (b > AM_MAX_BLOCKS) b = AM_MAX_BLOCKS;
  return (int)b;
}

// ------------------------------------------------------------------ next use

// next_use / prev_use come from the trace sorted by page, stably (positions of one page
// stay in trace order): neighbours with the same page are consecutive uses.  The sort is an
// LSD radix sort of (page, position) pairs with 7-bit digits, ceil(bits(n_pages) / 7)
// passes, each:
//   1. rs_hist_kernel: per tile of RS_TILE elements, the count of every digit, stored
//      digit-major (hist[d * n_tiles + tile]);
//   2. an exclusive scan of that table (rs_scan_*): the output position where digit d's
//      elements of each tile start;
//   3. rs_scatter_kernel: each tile ranks its elements stably within their digit and
//      writes (page, position) to the scanned start plus the rank.
// Ranking in a tile runs in RS_ITEMS rounds of 256 consecutive elements (one per thread,
// loads coalesced).  In a round, the lanes of a wave holding the same digit find each other
// with 7 ballots (their rank in the wave = the peers below them); each wave's count per
// digit goes to LDS, and an element's rank in the tile = (count of its digit in earlier
// rounds) + (count in earlier waves of this round) + (rank in its wave).
constexpr int RS_BITS = 7;
constexpr int RS_RADIX = 1 << RS_BITS;
constexpr int RS_THREADS = 256;
constexpr int RS_WAVES = RS_THREADS / 64;
constexpr int RS_ITEMS = 16;
constexpr int RS_TILE = RS_THREADS * RS_ITEMS;
constexpr int RS_SCAN_CHUNK = 4096;  // entries of the digit table per scan block

__global__ void __launch_bounds__(RS_THREADS)
rs_hist_kernel(const int32_t *keys, int64_t n, int shift, int32_t n_pages, uint32_t *hist, int64_t n_tiles,
               int32_t *err) {
  __shared__ uint32_t cnt[RS_RADIX];
  if (threadIdx.x < RS_RADIX) cnt[threadIdx.x] = 0;
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * RS_TILE;
  bool bad = false;
#pragma unroll 4
  for (int r = 0; r < RS_ITEMS; ++r) {
    const int64_t e = base + r * RS_THREADS + threadIdx.x;
    if (e < n) {
      const int32_t k = keys[e];
      bad |= k < 0 || k >= n_pages;
      atomicAdd(&cnt[((uint32_t)k >> shift) & (RS_RADIX - 1)], 1u);
    }
  }
  if (err && shift == 0 && __ballot(bad) && (threadIdx.x & 63) == 0) atomicOr(err, ZX_KERR_PAGE_RANGE);
  __syncthreads();
  if (threadIdx.x < RS_RADIX) hist[(int64_t)threadIdx.x * n_tiles + blockIdx.x] = cnt[threadIdx.x];
}

// Exclusive scan of m entries: block sums of RS_SCAN_CHUNK-entry chunks, a one-block scan of
// those, then each chunk rescanned from its base (in place).
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t &total) {
  __shared__ uint32_t wsum[RS_WAVES];
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  uint32_t x = v;  // inclusive scan inside the wave
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  if (lane == 63) wsum[wid] = x;
  __syncthreads();
  uint32_t before = 0;
  total = 0;
  for (int w = 0; w < RS_WAVES; ++w) {
    before += w < wid ? wsum[w] : 0u;
    total += wsum[w];
  }
  __syncthreads();
  return before + x - v;
}

__global__ void __launch_bounds__(RS_THREADS) rs_scan_sums_kernel(const uint32_t *a, int64_t m, uint32_t *sums) {
  const int64_t c0 = (int64_t)blockIdx.x * RS_SCAN_CHUNK;
  uint32_t s = 0;
  for (int i = threadIdx.x; i < RS_SCAN_CHUNK; i += RS_THREADS)
    if (c0 + i < m) s += a[c0 + i];
  uint32_t total;
  block_excl_scan(s, total);
  if (threadIdx.x == 0) sums[blockIdx.x] = total;
}

__global__ void __launch_bounds__(RS_THREADS) rs_scan_top_kernel(uint32_t *sums, int64_t n_chunks) {
  uint32_t carry = 0;  // one block walks the chunk sums RS_THREADS at a time
  for (int64_t i0 = 0; i0 < n_chunks; i0 += RS_THREADS) {
    const int64_t i = i0 + threadIdx.x;
    const uint32_t v = i < n_chunks ? sums[i] : 0u;
    uint32_t total;
    const uint32_t ex = block_excl_scan(v, total);
    if (i < n_chunks) sums[i] = carry + ex;
    carry += total;
  }
}

__global__ void __launch_bounds__(RS_THREADS)
rs_scan_chunks_kernel(uint32_t *a, int64_t m, const uint32_t *sums) {
  const int64_t c0 = (int64_t)blockIdx.x * RS_SCAN_CHUNK;
  constexpr int PER = RS_SCAN_CHUNK / RS_THREADS;  // consecutive entries per thread
  uint32_t v[PER], s = 0;
  const int64_t i0 = c0 + (int64_t)threadIdx.x * PER;
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    v[k] = i0 + k < m ? a[i0 + k] : 0u;
    s += v[k];
  }
  uint32_t total;
  uint32_t run = sums[blockIdx.x] + block_excl_scan(s, total);
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    if (i0 + k < m) a[i0 + k] = run;
    run += v[k];
  }
}

// vals_in == nullptr: the values are the element indices (the first pass).  The tile is
// ranked, staged in LDS in digit order, then written out: the elements of one digit go to
// consecutive output positions, so neighbouring threads write neighbouring words.
__global__ void __launch_bounds__(RS_THREADS)
rs_scatter_kernel(const int32_t *keys_in, const int32_t *vals_in, int64_t n, int shift, const uint32_t *offs,
                  int64_t n_tiles, int32_t *keys_out, int32_t *vals_out) {
  __shared__ uint32_t gstart[RS_RADIX];              // output position of the tile's first element of digit d
  __shared__ uint32_t lstart[RS_RADIX];              // its position in the tile's digit order
  __shared__ uint32_t run[RS_RADIX];                 // elements of digit d ranked so far (earlier rounds)
  __shared__ uint32_t wcnt[2][RS_WAVES][RS_RADIX];   // per round (parity), per wave, per digit
  __shared__ int32_t lk[RS_TILE], lv[RS_TILE];       // the tile in digit order
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int64_t base = (int64_t)blockIdx.x * RS_TILE;
  const int tile_n = (int)min((int64_t)RS_TILE, n - base);
  uint32_t cnt = 0;
  if (threadIdx.x < RS_RADIX) {
    // digit-major exclusive scan: the next entry is this tile's start plus its count
    const int64_t i = (int64_t)threadIdx.x * n_tiles + blockIdx.x;
    const uint32_t st = offs[i];
    const uint32_t nx = i + 1 < n_tiles * RS_RADIX ? offs[i + 1] : (uint32_t)n;
    gstart[threadIdx.x] = st;
    cnt = nx - st;
    run[threadIdx.x] = 0;
  }
  for (int i = threadIdx.x; i < 2 * RS_WAVES * RS_RADIX; i += RS_THREADS) (&wcnt[0][0][0])[i] = 0;
  uint32_t total;
  const uint32_t ex = block_excl_scan(threadIdx.x < RS_RADIX ? cnt : 0u, total);  // synchronises
  if (threadIdx.x < RS_RADIX) lstart[threadIdx.x] = ex;
  __syncthreads();
  const uint64_t below = (1ull << lane) - 1;
  int led[2] = {-1, -1};  // digit this lane led two rounds ago, per parity (its entry to clear)
  for (int r = 0; r < RS_ITEMS; ++r) {
    const int par = r & 1;
    const int e = r * RS_THREADS + threadIdx.x;  // element of the tile
    const bool valid = e < tile_n;
    const int32_t k = valid ? keys_in[base + e] : 0;
    const int32_t v = valid ? (vals_in ? vals_in[base + e] : (int32_t)(base + e)) : 0;
    const uint32_t d = ((uint32_t)k >> shift) & (RS_RADIX - 1);
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int b = 0; b < RS_BITS; ++b) {
      const uint64_t ones = __ballot((d >> b) & 1u);
      peers &= ((d >> b) & 1u) ? ones : ~ones;
    }
    const uint32_t rank_w = (uint32_t)__popcll(peers & below);
    // clear what this lane wrote two rounds ago (every wave has read it since), then
    // publish this round's count of the digit for the wave
    if (led[par] >= 0) wcnt[par][wid][led[par]] = 0;
    led[par] = -1;
    if (valid && rank_w == 0) {
      wcnt[par][wid][d] = (uint32_t)__popcll(peers);
      led[par] = (int)d;
    }
    __syncthreads();
    if (valid) {
      uint32_t pos = lstart[d] + run[d] + rank_w;
      for (int w = 0; w < wid; ++w) pos += wcnt[par][w][d];
      lk[pos] = k;
      lv[pos] = v;
    }
    __syncthreads();
    if (threadIdx.x < RS_RADIX) {  // the round's elements of digit d follow earlier rounds'
      uint32_t c = 0;
      for (int w = 0; w < RS_WAVES; ++w) c += wcnt[par][w][threadIdx.x];
      run[threadIdx.x] += c;
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < tile_n; i += RS_THREADS) {
    const int32_t k = lk[i];
    const uint32_t d = ((uint32_t)k >> shift) & (RS_RADIX - 1);
    const uint32_t pos = gstart[d] + (uint32_t)i - lstart[d];
    keys_out[pos] = k;
    vals_out[pos] = lv[i];
  }
}

static int key_bits(int32_t n_pages) {
  int b = 1;
  while (b < 31 && (1LL << b) < (int64_t)n_pages) ++b;
  return b;
}

__global__ void next_use_kernel(const int32_t *skey, const int32_t *spos, int64_t n, int32_t *next_use,
                                int32_t *prev_use) {
  int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (k >= n) return;
  const int32_t p = skey[k], pos = spos[k];
  next_use[pos] = (k + 1 < n && skey[k + 1] == p) ? spos[k + 1] : ZX_NEVER;
  prev_use[pos] = (k > 0 && skey[k - 1] == p) ? spos[k - 1] : -1;
}

// Workspace: keys and positions twice (ping-pong), the digit table, the scan's chunk sums.
struct NextUseWs {
  int32_t *k[2], *v[2];
  uint32_t *hist, *sums;
  int64_t n_tiles, m, n_chunks;
  size_t bytes;
};

static NextUseWs next_use_ws(void *base, int64_t n) {
  NextUseWs w;
  w.n_tiles = ceil_div(n, RS_TILE);
  w.m = w.n_tiles * RS_RADIX;
  w.n_chunks = ceil_div(w.m, RS_SCAN_CHUNK);
  char *p = static_cast<char *>(base);
  const size_t a = align256((size_t)n * 4);
  for (int i = 0; i < 2; ++i) {
    w.k[i] = reinterpret_cast<int32_t *>(p + (2 * i) * a);
    w.v[i] = reinterpret_cast<int32_t *>(p + (2 * i + 1) * a);
  }
  w.hist = reinterpret_cast<uint32_t *>(p + 4 * a);
  w.sums = reinterpret_cast<uint32_t *>(p + 4 * a + align256((size_t)w.m * 4));
  w.bytes = 4 * a + align256((size_t)w.m * 4) + align256((size_t)w.n_chunks * 4);
  return w;
}

}  // namespace zx

using namespace zx;

extern "C" size_t zx_belady_argmax_workspace_bytes(int64_t n_slots) {
  return (size_t)argmax_blocks(n_slots > 0 ? n_slots : 1) * sizeof(Best);
}

extern "C" int zx_belady_argmax(const int64_t *keys, const uint8_t *resident, const int64_t *rank, int64_t n_slots,
                                int64_t *out, void *workspace, size_t workspace_bytes, zx_stream_t stream) {
  clear_error();
  ZX_REQUIRE(out && (n_slots == 0 || keys), "belady_argmax: null pointer");
  ZX_REQUIRE(n_slots >= 0, "belady_argmax: negative size");
  const int nb = argmax_blocks(n_slots > 0 ? n_slots : 1);
  if (!workspace || workspace_bytes < (size_t)nb * sizeof(Best))
    return fail(ZX_ERR_WORKSPACE, "belady_argmax: workspace too small");
  hipStream_t st = as_stream(stream);
  Best *part = reinterpret_cast<Best *>(workspace);
  argmax_partial_kernel<<<nb, AM_THREADS, 0, st>>>(keys, resident, rank, n_slots, part);
  int rc = check_launch("belady_argmax_partial");
  if (rc) return rc;
  argmax_final_kernel<<<1, AM_THREADS, 0, st>>>(part, nb, out);
  return check_launch("belady_argmax_final");
}

extern "C" int zx_belady_update_slots(int64_t *keys, uint8_t *resident, int64_t *rank, int64_t n_slots,
                                      const int64_t *slot, const int64_t *key, const uint8_t *res,
                                      const int64_t *rank_in, int64_t n, int32_t *err, zx_stream_t stream) {
  clear_error();
  ZX_REQUIRE(n >= 0 && n_slots >= 0, "belady_update_slots: negative size");
  ZX_REQUIRE(!resident == !res, "belady_update_slots: resident and res must be given together");
  ZX_REQUIRE(!rank == !rank_in, "belady_update_slots: rank and rank_in must be given together");
  if (n == 0) return ZX_OK;
  ZX_REQUIRE(keys && slot && key, "belady_update_slots: null pointer");
  update_slots_kernel<<<(unsigned)ceil_div(n, 256), 256, 0, as_stream(stream)>>>(keys, resident, rank, n_slots, slot,
                                                                                key, res, rank_in, n, err);
  return check_launch("belady_update_slots");
}

extern "C" size_t zx_belady_next_use_workspace_bytes(int64_t n, int32_t n_pages) {
  (void)n_pages;
  if (n <= 0) return 256;
  return next_use_ws(nullptr, n).bytes;
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
  const NextUseWs w = next_use_ws(workspace, n);
  const int bits = key_bits(n_pages), passes = (bits + RS_BITS - 1) / RS_BITS;
  const unsigned tiles = (unsigned)w.n_tiles;
  int rc;
  for (int p = 0; p < passes; ++p) {
    const int shift = p * RS_BITS;
    const int32_t *kin = p == 0 ? trace : w.k[(p + 1) & 1];
    const int32_t *vin = p == 0 ? nullptr : w.v[(p + 1) & 1];
    rs_hist_kernel<<<tiles, RS_THREADS, 0, st>>>(kin, n, shift, n_pages, w.hist, w.n_tiles, err);
    if ((rc = check_launch("radix_hist"))) return rc;
    rs_scan_sums_kernel<<<(unsigned)w.n_chunks, RS_THREADS, 0, st>>>(w.hist, w.m, w.sums);
    if ((rc = check_launch("radix_scan_sums"))) return rc;
    rs_scan_top_kernel<<<1, RS_THREADS, 0, st>>>(w.sums, w.n_chunks);
    if ((rc = check_launch("radix_scan_top"))) return rc;
    rs_scan_chunks_kernel<<<(unsigned)w.n_chunks, RS_THREADS, 0, st>>>(w.hist, w.m, w.sums);
    if ((rc = check_launch("radix_scan_chunks"))) return rc;
    rs_scatter_kernel<<<tiles, RS_THREADS, 0, st>>>(kin, vin, n, shift, w.hist, w.n_tiles, w.k[p & 1], w.v[p & 1]);
    if ((rc = check_launch("radix_scatter"))) return rc;
  }
  const int last = (passes - 1) & 1;
  next_use_kernel<<<(unsigned)ceil_div(n, 256), 256, 0, st>>>(w.k[last], w.v[last], n, next_use, prev_use);
  return check_launch("belady_next_use");
}
