// zx_belady_sim.hip -- trace-level Belady MIN (BeladyKVCacheTieringManager, README.md:93-97;
// per-miss farthest-next-use victim of zenyx/streaming/belady.py:39-51, ties to the
// smallest page id).
//
// Keys as one priority-ordered bitmap.  A resident page is either "never used again"
// (its key is ZX_NEVER) or has a next use at a future trace position j.  Map it to
//     idx = page                            (never again; smaller page first)
//     idx = n_pages + (n_total - 1 - j)     (next use j; farther first)
// and set bit idx of B.  The Belady victim is always the resident page of smallest idx,
// i.e. the lowest set bit.  Per-4096-bit block counts (kept in LDS) find the first E set
// bits quickly.
//
// Windows.  One persistent workgroup walks the trace in windows [t0, t1) of up to 2048
// accesses.  Inside a window:
//   * an access that is not the page's first in the window is a hit, and a page's first
//     access misses iff the page is not resident -- provided at least E resident pages
//     are not accessed in the window ("statics", E = evictions the window needs): a
//     static's key lies beyond t1, so some static always outranks every page whose
//     next use falls inside the window, and such a page is never evicted before it is
//     used again;
//   * misses beyond the free capacity evict, in order;
//   * candidates are the first E statics (the first E set bits) and the window's
//     "dynamic" items: a page's last access in the window makes it a candidate from that
//     time on with key = its next use (beyond t1 or never);
//   * each eviction takes the best candidate available at its time (one wave scans the
//     dynamic items, statics are consumed in order).
// When fewer than E statics exist the window is halved (a window of one access always
// qualifies).  The result equals the sequential algorithm access by access.
#include "zx_internal.h"

namespace zx {

constexpr int BS_THREADS = 1024;
constexpr int BS_IPT = 2;                     // trace positions per thread per window
constexpr int BS_W = BS_THREADS * BS_IPT;     // window size
constexpr int BS_BLOCK_BITS = 4096;           // bits per counted block
constexpr int BS_MAX_BLOCKS = 8192;           // LDS block counters -> at most 2^25 bits
constexpr int64_t BS_MAX_BITS = (int64_t)BS_MAX_BLOCKS * BS_BLOCK_BITS;

struct SimArgs {
  const int32_t *trace, *next_use, *prev_use;
  int64_t n_total, t_begin, t_end;
  int32_t n_pages;
  int64_t capacity;
  uint8_t *resident;
  int32_t *key;
  int64_t *state;
  int32_t *evict_pos, *evict_page;
  int64_t evict_cap;
  uint8_t *miss_flags;
  unsigned long long *bits;  // ceil(nbits / 64) words
  uint32_t *cnt;             // ceil(nbits / 4096) counts (rebuilt on the host side of the call)
  int64_t nbits;
  int32_t nblk;
  int32_t *err;
};

__device__ __forceinline__ int64_t item_idx(const SimArgs &a, int32_t page, int32_t nu) {
  return nu == ZX_NEVER ? (int64_t)page : (int64_t)a.n_pages + (a.n_total - 1 - nu);
}

// Byte of a flag array, read through to L2 (other waves of this workgroup wrote it in
// earlier windows; the per-CU L1 is not kept coherent with those stores).
__device__ __forceinline__ uint32_t ld_flag(const uint8_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ unsigned long long ld_word(const unsigned long long *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void set_bit(const SimArgs &a, uint32_t *cnt, int64_t idx) {
  atomicOr(&a.bits[idx >> 6], 1ull << (idx & 63));
  atomicAdd(&cnt[idx / BS_BLOCK_BITS], 1u);
}
__device__ __forceinline__ void clear_bit(const SimArgs &a, uint32_t *cnt, int64_t idx) {
  atomicAnd(&a.bits[idx >> 6], ~(1ull << (idx & 63)));
  atomicSub(&cnt[idx / BS_BLOCK_BITS], 1u);
}

// Exclusive block-wide prefix sum of one value per thread; *total receives the sum.
__device__ __forceinline__ int block_scan(int v, int *total, int *ws /* [BS_THREADS / 64 + 1] */) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  int x = v;
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  if (lane == 63) ws[wid] = x;
  __syncthreads();
  if (threadIdx.x == 0) {
    int acc = 0;
    for (int i = 0; i < BS_THREADS / 64; ++i) {
      const int t = ws[i];
      ws[i] = acc;
      acc += t;
    }
    ws[BS_THREADS / 64] = acc;
  }
  __syncthreads();
  const int r = ws[wid] + x - v;
  *total = ws[BS_THREADS / 64];
  __syncthreads();
  return r;
}

struct SimShared {
  uint32_t cnt[BS_MAX_BLOCKS];
  int32_t s_idx[BS_W];    // first E set bits (static candidates), in order
  int32_t d_idx[BS_W];    // dynamic candidates: idx, time (window offset), page
  int32_t d_t[BS_W];
  int32_t d_page[BS_W];
  uint8_t d_taken[BS_W];
  int32_t ev_t[BS_W];     // eviction events: window offset of the evicting miss
  int32_t ev_vidx[BS_W];  // victim idx and page per event
  int32_t ev_vpage[BS_W];
  uint8_t ev_dyn[BS_W];
  int32_t blk_list[BS_W];  // blocks holding the first E set bits, and their rank offsets
  int32_t blk_before[BS_W];
  int scan_ws[BS_THREADS / 64 + 1];
  int n_list;
};

// First E set bits of B (E <= BS_W, at least E bits set) into sh.s_idx.
__device__ void select_first(const SimArgs &a, SimShared &sh, int E) {
  const int per = (a.nblk + BS_THREADS - 1) / BS_THREADS;
  const int b0 = threadIdx.x * per;
  int sum = 0;
  for (int b = b0; b < b0 + per && b < a.nblk; ++b) sum += sh.cnt[b];
  int total;
  int before = block_scan(sum, &total, sh.scan_ws);
  if (threadIdx.x == 0) sh.n_list = 0;
  __syncthreads();
  for (int b = b0; b < b0 + per && b < a.nblk && before < E; ++b) {
    const int c = sh.cnt[b];
    if (c) {
      const int slot = atomicAdd(&sh.n_list, 1);
      sh.blk_list[slot] = b;
      sh.blk_before[slot] = before;
    }
    before += c;
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  for (int li = wid; li < sh.n_list; li += BS_THREADS / 64) {
    const int b = sh.blk_list[li];
    const int64_t widx = (int64_t)b * (BS_BLOCK_BITS / 64) + lane;
    unsigned long long w = widx * 64 < a.nbits ? ld_word(&a.bits[widx]) : 0ull;
    const int pc = __popcll(w);
    int x = pc;
    for (int off = 1; off < 64; off <<= 1) {
      const int y = __shfl_up(x, off, 64);
      if (lane >= off) x += y;
    }
    int r = sh.blk_before[li] + x - pc;
    while (w && r < E) {
      const int bit = __ffsll((long long)w) - 1;
      w &= w - 1;
      sh.s_idx[r++] = (int32_t)(widx * 64 + bit);
    }
  }
  __syncthreads();
}

__global__ void __launch_bounds__(BS_THREADS, 1) belady_sim_kernel(SimArgs a) {
  __shared__ SimShared sh;
  __shared__ int64_t st[4];
  for (int b = threadIdx.x; b < a.nblk; b += BS_THREADS) sh.cnt[b] = a.cnt[b];
  if (threadIdx.x < 4) st[threadIdx.x] = a.state[threadIdx.x];
  __syncthreads();
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;

  int w_lim = BS_W;
  int64_t t0 = a.t_begin;
  while (t0 < a.t_end) {
    const int w = (int)((a.t_end - t0) < w_lim ? (a.t_end - t0) : w_lim);
    const int64_t t1 = t0 + w;
    int32_t p[BS_IPT], nu[BS_IPT];
    bool live[BS_IPT], miss[BS_IPT], hitfirst[BS_IPT], last[BS_IPT];
    int mcount = 0, hcount = 0;
#pragma unroll
    for (int j = 0; j < BS_IPT; ++j) {
      const int i = j * BS_THREADS + threadIdx.x;
      live[j] = i < w;
      p[j] = 0;
      nu[j] = ZX_NEVER;
      miss[j] = hitfirst[j] = last[j] = false;
      if (live[j]) {
        const int64_t pos = t0 + i;
        p[j] = a.trace[pos];
        nu[j] = a.next_use[pos];
        const bool first = a.prev_use[pos] < t0;
        last[j] = nu[j] == ZX_NEVER || nu[j] >= t1;
        if (first) {
          const bool res = ld_flag(a.resident + p[j]) != 0;
          miss[j] = !res;
          hitfirst[j] = res;
        }
      }
      mcount += miss[j];
      hcount += hitfirst[j];
    }
    // miss ranks in trace order (positions j * BS_THREADS + tid)
    int m_rank[BS_IPT];
    int M = 0;
#pragma unroll
    for (int j = 0; j < BS_IPT; ++j) {
      int tot;
      m_rank[j] = M + block_scan(miss[j] ? 1 : 0, &tot, sh.scan_ws);
      M += tot;
    }
    int Hf;
    block_scan(hcount, &Hf, sh.scan_ws);
    const int64_t count0 = st[0];
    const int64_t F = a.capacity - count0 > 0 ? a.capacity - count0 : 0;
    const int E = M > F ? (int)(M - F) : 0;
    if (E > 0 && count0 - Hf < E) {  // not enough statics: smaller window
      w_lim = w > 1 ? w / 2 : 1;
      continue;
    }
    w_lim = w_lim < BS_W ? w_lim * 2 : BS_W;

    int dpos[BS_IPT];
#pragma unroll
    for (int j = 0; j < BS_IPT; ++j) dpos[j] = -1;
    if (E > 0) {
      select_first(a, sh, E);
      const int32_t worst = sh.s_idx[E - 1];
      // dynamic candidates that can beat a needed static, in trace order
      int nd = 0;
#pragma unroll
      for (int j = 0; j < BS_IPT; ++j) {
        const bool cand = last[j] && item_idx(a, p[j], nu[j]) < worst;
        int tot;
        const int r = nd + block_scan(cand ? 1 : 0, &tot, sh.scan_ws);
        if (cand) {
          sh.d_idx[r] = (int32_t)item_idx(a, p[j], nu[j]);
          sh.d_t[r] = j * BS_THREADS + threadIdx.x;
          sh.d_page[r] = p[j];
          sh.d_taken[r] = 0;
          dpos[j] = r;
        }
        nd += tot;
        if (miss[j] && m_rank[j] >= F) sh.ev_t[m_rank[j] - F] = j * BS_THREADS + threadIdx.x;
      }
      __syncthreads();
      if (nd == 0) {  // no dynamic candidate can beat a needed static: victims in order
        for (int k = threadIdx.x; k < E; k += BS_THREADS) {
          const int32_t sidx = sh.s_idx[k];
          sh.ev_vidx[k] = sidx;
          sh.ev_vpage[k] = sidx < a.n_pages ? sidx : a.trace[a.n_total - 1 - ((int64_t)sidx - a.n_pages)];
          sh.ev_dyn[k] = 0;
        }
      } else if (wid == 0) {
        int sp = 0;
        for (int k = 0; k < E; ++k) {
          const int tau = sh.ev_t[k];
          int best = 0x7FFFFFFF, bj = -1;
          for (int q = lane; q < nd; q += 64)
            if (!sh.d_taken[q] && sh.d_t[q] < tau && sh.d_idx[q] < best) {
              best = sh.d_idx[q];
              bj = q;
            }
          for (int off = 32; off >= 1; off >>= 1) {
            const int ob = __shfl_xor(best, off, 64), oj = __shfl_xor(bj, off, 64);
            if (ob < best) {
              best = ob;
              bj = oj;
            }
          }
          if (lane == 0) {
            const int32_t sidx = sh.s_idx[sp];
            if (bj >= 0 && best < sidx) {
              sh.ev_vidx[k] = best;
              sh.ev_vpage[k] = sh.d_page[bj];
              sh.ev_dyn[k] = 1;
              sh.d_taken[bj] = 1;
            } else {
              sh.ev_vidx[k] = sidx;
              sh.ev_vpage[k] = sidx < a.n_pages ? sidx : a.trace[a.n_total - 1 - ((int64_t)sidx - a.n_pages)];
              sh.ev_dyn[k] = 0;
            }
          }
          if (!(bj >= 0 && best < sh.s_idx[sp])) ++sp;
          __builtin_amdgcn_wave_barrier();
        }
      }
      __syncthreads();
    }
    // admissions and hits on pages resident since before the window
#pragma unroll
    for (int j = 0; j < BS_IPT; ++j) {
      if (!live[j]) continue;
      const int64_t pos = t0 + j * BS_THREADS + threadIdx.x;
      if (miss[j]) a.resident[p[j]] = 1;
      if (hitfirst[j]) clear_bit(a, sh.cnt, item_idx(a, p[j], (int32_t)pos));
      if (a.miss_flags) a.miss_flags[pos] = miss[j] ? 1 : 0;
    }
    __syncthreads();
    // evictions
    const int64_t ev0 = st[1];
    for (int k = threadIdx.x; k < E; k += BS_THREADS) {
      const int32_t page = sh.ev_vpage[k];
      a.resident[page] = 0;
      if (!sh.ev_dyn[k]) clear_bit(a, sh.cnt, sh.ev_vidx[k]);
      if (ev0 + k < a.evict_cap) {
        a.evict_pos[ev0 + k] = (int32_t)(t0 + sh.ev_t[k]);
        a.evict_page[ev0 + k] = page;
      }
    }
    __syncthreads();
    // pages still resident after their last access in the window get their new key
#pragma unroll
    for (int j = 0; j < BS_IPT; ++j) {
      if (!live[j] || !last[j]) continue;
      if (dpos[j] >= 0 && sh.d_taken[dpos[j]]) continue;
      set_bit(a, sh.cnt, item_idx(a, p[j], nu[j]));
      a.key[p[j]] = nu[j];
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      st[0] = count0 + M - E;
      st[1] = ev0 + E;
      st[2] += M;
      st[3] += w - M;
    }
    __syncthreads();
    t0 = t1;
  }
  if (threadIdx.x < 4) a.state[threadIdx.x] = st[threadIdx.x];
}

// Rebuild B and the block counts from the caller's resident/key arrays.
__global__ void belady_rebuild_kernel(SimArgs a) {
  const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= a.n_pages || !a.resident[p]) return;
  const int32_t k = a.key[p];
  if (k != ZX_NEVER && (k < a.t_begin || k >= a.n_total)) {
    if (a.err) atomicOr(a.err, ZX_KERR_POS_RANGE);
    return;
  }
  const int64_t idx = item_idx(a, (int32_t)p, k);
  atomicOr(&a.bits[idx >> 6], 1ull << (idx & 63));
  atomicAdd(&a.cnt[idx / BS_BLOCK_BITS], 1u);
}

}  // namespace zx

using namespace zx;

extern "C" size_t zx_belady_simulate_workspace_bytes(int64_t n_total, int32_t n_pages) {
  const int64_t nbits = (n_total > 0 ? n_total : 0) + (n_pages > 0 ? n_pages : 0);
  return align256((size_t)ceil_div(nbits, 64) * 8) + align256((size_t)ceil_div(nbits, BS_BLOCK_BITS) * 4);
}

extern "C" int zx_belady_simulate(const int32_t *trace, const int32_t *next_use, const int32_t *prev_use,
                                  int64_t n_total, int64_t t_begin, int64_t t_end, int32_t n_pages,
                                  int64_t capacity, uint8_t *resident, int32_t *key, int64_t *state,
                                  int32_t *evict_pos, int32_t *evict_page, int64_t evict_cap,
                                  uint8_t *miss_flags, void *workspace, size_t workspace_bytes,
                                  zx_stream_t stream) {
  clear_error();
  ZX_REQUIRE(n_pages > 0 && n_total >= 0 && n_total < 0x7FFFFFFF, "belady_simulate: bad sizes");
  ZX_REQUIRE(0 <= t_begin && t_begin <= t_end && t_end <= n_total, "belady_simulate: bad range");
  ZX_REQUIRE(capacity >= 1, "belady_simulate: capacity must be >= 1");
  ZX_REQUIRE(resident && key && state && (evict_cap == 0 || (evict_pos && evict_page)),
             "belady_simulate: null pointer");
  ZX_REQUIRE(n_total == 0 || (trace && next_use && prev_use), "belady_simulate: null trace");
  const int64_t nbits = n_total + n_pages;
  if (nbits > BS_MAX_BITS)
    return fail(ZX_ERR_UNSUPPORTED, "belady_simulate: n_total + n_pages = %lld exceeds %lld", (long long)nbits,
                (long long)BS_MAX_BITS);
  const size_t need = zx_belady_simulate_workspace_bytes(n_total, n_pages);
  if (!workspace || workspace_bytes < need)
    return fail(ZX_ERR_WORKSPACE, "belady_simulate: workspace %zu < %zu bytes", workspace_bytes, need);
  if (t_begin == t_end) return ZX_OK;
  hipStream_t st = as_stream(stream);
  SimArgs a;
  a.trace = trace;
  a.next_use = next_use;
  a.prev_use = prev_use;
  a.n_total = n_total;
  a.t_begin = t_begin;
  a.t_end = t_end;
  a.n_pages = n_pages;
  a.capacity = capacity;
  a.resident = resident;
  a.key = key;
  a.state = state;
  a.evict_pos = evict_pos;
  a.evict_page = evict_page;
  a.evict_cap = evict_cap;
  a.miss_flags = miss_flags;
  const size_t words_bytes = align256((size_t)ceil_div(nbits, 64) * 8);
  a.bits = reinterpret_cast<unsigned long long *>(workspace);
  a.cnt = reinterpret_cast<uint32_t *>(static_cast<char *>(workspace) + words_bytes);
  a.nbits = nbits;
  a.nblk = (int32_t)ceil_div(nbits, BS_BLOCK_BITS);
  a.err = nullptr;
  int rc = fill_u32(reinterpret_cast<uint32_t *>(workspace), (int64_t)(need / 4), 0, st);
  if (rc) return rc;
  belady_rebuild_kernel<<<(unsigned)ceil_div(n_pages, 256), 256, 0, st>>>(a);
  if ((rc = check_launch("belady_rebuild"))) return rc;
  belady_sim_kernel<<<1, BS_THREADS, 0, st>>>(a);
  return check_launch("belady_sim");
}
