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
// Windows.  One persistent workgroup walks the trace in windows [t0, t1) of up to 8192
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
//   * each eviction takes the best candidate available at its time: merged by rank when
//     every dynamic candidate exists before the first eviction, else parked in key order
//     by one wave (park_victims).
// When fewer than E statics exist the window is halved (a window of one access always
// qualifies).  The result equals the sequential algorithm access by access.
#include "zx_internal.h"

namespace zx {

constexpr int BS_THREADS = 1024;
constexpr int BS_IPT = 8;                     // trace positions per thread per window
constexpr int BS_W = BS_THREADS * BS_IPT;     // largest window
constexpr int BS_EMAX = 2048;                 // evictions and dynamic candidates per window
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

__device__ __forceinline__ unsigned long long ld_word(const unsigned long long *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
  if (wid == 0) {  // exclusive scan of the wave totals by the first wave
    constexpr int NW = BS_THREADS / 64;
    const int t = lane < NW ? ws[lane] : 0;
    int u = t;
    for (int off = 1; off < NW; off <<= 1) {
      const int y = __shfl_up(u, off, 64);
      if (lane >= off) u += y;
    }
    if (lane < NW) ws[lane] = u - t;
    if (lane == NW - 1) ws[NW] = u;
  }
  __syncthreads();
  const int r = ws[wid] + x - v;
  *total = ws[BS_THREADS / 64];
  __syncthreads();
  return r;
}

struct SimShared {
  uint32_t cnt[BS_MAX_BLOCKS];
  int32_t s_idx[BS_EMAX];    // first E set bits (static candidates), in order
  int32_t d_idx[BS_EMAX];    // dynamic candidates: idx, time (window offset), page
  int32_t d_t[BS_EMAX];
  int32_t d_page[BS_EMAX];
  uint8_t d_taken[BS_EMAX];
  int32_t ev_t[BS_EMAX];     // eviction events: window offset of the evicting miss
  int32_t ev_vidx[BS_EMAX];  // victim idx and page per event
  int32_t ev_vpage[BS_EMAX];
  uint8_t ev_dyn[BS_EMAX];
  int32_t blk_list[BS_EMAX];  // blocks holding the first E set bits, and their rank offsets
  int32_t blk_before[BS_EMAX];
  int32_t sort_key[BS_EMAX];  // dynamic candidates sorted by idx (key) -> candidate slot
  int32_t sort_val[BS_EMAX];
  int32_t sort_rel[BS_EMAX];  // per sorted candidate: evictions at or before its time
  unsigned long long win_bits[BS_W / 64 + 2];  // words of B covering the window's positions
  unsigned long long win_clr[BS_W / 64 + 2];   // bits of those words cleared in this window
  int scan_ws[BS_THREADS / 64 + 1];
  int n_list;
  int n_dyn_victims;
};

// Sorts sh.sort_key[0, n) ascending with sh.sort_val as payload (bitonic; n <= BS_EMAX).
__device__ void sort_candidates(SimShared &sh, int n) {
  int n2 = 1;
  while (n2 < n) n2 <<= 1;
  for (int i = n + threadIdx.x; i < n2; i += BS_THREADS) {
    sh.sort_key[i] = 0x7FFFFFFF;
    sh.sort_val[i] = -1;
  }
  __syncthreads();
  for (int k = 2; k <= n2; k <<= 1)
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < n2; i += BS_THREADS) {
        const int p = i ^ j;
        if (p > i) {
          const bool up = (i & k) == 0;
          const int ki = sh.sort_key[i], kp = sh.sort_key[p];
          if ((ki > kp) == up) {
            sh.sort_key[i] = kp;
            sh.sort_key[p] = ki;
            const int v = sh.sort_val[i];
            sh.sort_val[i] = sh.sort_val[p];
            sh.sort_val[p] = v;
          }
        }
      }
      __syncthreads();
    }
}

// Number of entries of the ascending array a[0, n) that are <= x.
__device__ __forceinline__ int upper_bound(const int32_t *a, int n, int32_t x) {
  int lo = 0, hi = n;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (a[mid] <= x) lo = mid + 1;
    else hi = mid;
  }
  return lo;
}

__device__ __forceinline__ int32_t lane_of(int32_t v, int lane) { return __builtin_amdgcn_readlane(v, lane); }
__device__ __forceinline__ uint64_t lane_of64(uint64_t v, int lane) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, lane);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), lane);
  return ((uint64_t)hi << 32) | lo;
}

// Victims of a window whose dynamic candidates appear between its evictions (wave 0).
// Eviction k (at window offset ev_t[k]) takes the best (smallest idx) candidate not yet
// taken: any static, or a dynamic one whose time d_t < ev_t[k].  That online order gives
// the same victims as parking the candidates in increasing idx order, each at the first
// free eviction slot it may use (a static: any slot; a dynamic one: slots k with
// ev_t[k] > d_t): the smallest candidate goes to the first eviction that can see it,
// and the rest is the same problem without that candidate and that eviction.  So the wave
// walks the merged idx order of the E statics (sh.s_idx) and the sorted dynamic
// candidates (sh.sort_key / sort_val / sort_rel) once, with the free slots as a bitmap
// in registers (lane l < 32: slots [64 l, 64 l + 64)); each candidate costs a ballot,
// not a scan of the candidates.  Records ev_vidx and ev_dyn per slot, and in ev_vpage the
// candidate slot (dynamic) or -1 (static: its page is read afterwards).  Returns the
// number of dynamic victims.
__device__ int park_victims(SimShared &sh, int E, int nd) {
  const int lane = threadIdx.x & 63;
  uint64_t freem = 0;
  if (lane < 32) {
    const int lo = lane * 64;
    freem = lo >= E ? 0ull : (E - lo >= 64 ? ~0ull : ((1ull << (E - lo)) - 1));
  }
  int sp = 0, dp = 0, filled = 0, n_dyn = 0;
  int sbase = -64, dbase = -64;
  int32_t cs = 0, ck = 0, cv = 0, cr = 0;
  while (filled < E) {
    if (sp - sbase >= 64) {
      sbase = sp;
      cs = sbase + lane < E ? sh.s_idx[sbase + lane] : 0x7FFFFFFF;
    }
    if (dp - dbase >= 64) {
      dbase = dp;
      const bool in = dbase + lane < nd;
      ck = in ? sh.sort_key[dbase + lane] : 0x7FFFFFFF;
      cv = in ? sh.sort_val[dbase + lane] : -1;
      cr = in ? sh.sort_rel[dbase + lane] : E;
    }
    const int32_t skey = sp < E ? lane_of(cs, sp - sbase) : 0x7FFFFFFF;
    const int32_t dkey = dp < nd ? lane_of(ck, dp - dbase) : 0x7FFFFFFF;
    if (skey == 0x7FFFFFFF && dkey == 0x7FFFFFFF) break;  // not reached: E statics fill E slots
    const bool dyn = dkey < skey;
    const int rel = dyn ? lane_of(cr, dp - dbase) : 0;
    const int cand = dyn ? lane_of(cv, dp - dbase) : -1;
    if (dyn) ++dp;
    else ++sp;
    // first free slot >= rel
    const int lo = lane * 64;
    uint64_t m = lo >= rel ? freem : ((rel >> 6) == lane ? freem & (~0ull << (rel & 63)) : 0ull);
    const uint64_t any = __ballot(m != 0ull);
    if (any == 0ull) continue;  // every slot this candidate may use is taken
    const int fl = __ffsll((long long)any) - 1;
    const uint64_t mf = lane_of64(m, fl);
    const int bit = __ffsll((long long)mf) - 1;
    const int slot = fl * 64 + bit;
    if (lane == fl) freem &= ~(1ull << bit);
    if (lane == 0) {
      sh.ev_vidx[slot] = dyn ? dkey : skey;
      sh.ev_vpage[slot] = cand;
      sh.ev_dyn[slot] = dyn ? 1 : 0;
    }
    n_dyn += dyn ? 1 : 0;
    ++filled;
  }
  return n_dyn;
}

// Number of entries of the ascending array a[0, n) that are < x.
__device__ __forceinline__ int lower_bound(const int32_t *a, int n, int32_t x) {
  int lo = 0, hi = n;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (a[mid] < x) lo = mid + 1;
    else hi = mid;
  }
  return lo;
}

// First E set bits of B (E <= BS_EMAX, at least E bits set) into sh.s_idx.
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

// v[j] = src[j] for j < n_valid, fill beyond.  A thread's trace positions are contiguous,
// so a whole run is read as 16-byte loads (4-byte aligned: window starts are arbitrary
// positions); only the thread that holds the window's end takes the element path.
typedef int32_t bs_i4 __attribute__((ext_vector_type(4)));
typedef bs_i4 bs_i4_a4 __attribute__((aligned(4)));
template <int N>
__device__ __forceinline__ void load_run(const int32_t *src, int n_valid, int32_t fill, int32_t (&v)[N]) {
  static_assert(N % 4 == 0, "runs are read 4 elements at a time");
  if (n_valid >= N) {
#pragma unroll
    for (int k = 0; k < N / 4; ++k) {
      const bs_i4 x = *reinterpret_cast<const bs_i4_a4 *>(src + 4 * k);
      v[4 * k] = x.x;
      v[4 * k + 1] = x.y;
      v[4 * k + 2] = x.z;
      v[4 * k + 3] = x.w;
    }
  } else {
#pragma unroll
    for (int j = 0; j < N; ++j) v[j] = j < n_valid ? src[j] : fill;
  }
}

// cnt[b] += c for every lane of the wave (c == 0: nothing), one LDS atomic per distinct
// block: a window's bits fall into a few blocks, and same-address LDS atomics from many
// lanes would serialise.  Called by every lane of the wave.
__device__ __forceinline__ void wave_cnt_add(uint32_t *cnt, int32_t b, int32_t c) {
  unsigned long long pend = __ballot(c != 0);
  while (pend) {
    const int leader = __ffsll((long long)pend) - 1;
    const int32_t b0 = __shfl(b, leader, 64);
    const bool mine = c != 0 && b == b0;
    int32_t v = mine ? c : 0;
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    if ((threadIdx.x & 63) == leader) atomicAdd(&cnt[b0], (uint32_t)v);
    pend &= ~__ballot(mine);
    if (mine) c = 0;
  }
}

// Segmented OR over the lanes of a wave that hold the same word wd (wd < 0: nothing).
// Returns true on the lane that issues the word's atomic, with m = the OR of its run.
// A thread's items are consecutive trace positions whose bits are mostly consecutive
// too, so neighbouring lanes share words; one atomic per run instead of one per lane
// keeps same-address atomics (serialised in the cache) off the window's critical path.
// Runs are contiguous lanes in the usual case; equal words in separate runs just give
// one atomic per run (OR is idempotent, no bit is lost).  Called by every lane.
__device__ __forceinline__ bool wave_word_or(int64_t wd, unsigned long long &m) {
  const int lane = threadIdx.x & 63;
  for (int off = 1; off < 64; off <<= 1) {
    const int64_t ow = __shfl_down(wd, off, 64);
    const unsigned long long om = __shfl_down(m, off, 64);
    if (lane + off < 64 && ow == wd) m |= om;
  }
  const int64_t pw = __shfl_up(wd, 1, 64);
  return wd >= 0 && (lane == 0 || pw != wd);
}

// Makes this wave's global stores and atomics complete, then joins the workgroup, so
// later reads by any wave of the workgroup observe them.
__device__ __forceinline__ void sync_global() {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
}

__global__ void __launch_bounds__(BS_THREADS, 1) belady_sim_kernel(SimArgs a) {
  __shared__ SimShared sh;
  __shared__ int64_t st[4];
  for (int b = threadIdx.x; b < a.nblk; b += BS_THREADS) sh.cnt[b] = a.cnt[b];
  if (threadIdx.x < 4) st[threadIdx.x] = a.state[threadIdx.x];
  __syncthreads();
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int64_t top = (int64_t)a.n_pages + a.n_total - 1;  // idx of position 0

  int w_lim = BS_W;
  int64_t t0 = a.t_begin;
  while (t0 < a.t_end) {
    const int w = (int)((a.t_end - t0) < w_lim ? (a.t_end - t0) : w_lim);
    const int64_t t1 = t0 + w;
    // A page whose first access in the window is at pos is resident iff its key is pos,
    // i.e. iff bit idx(pos) is set: read the window's bits instead of per-page flags.
    const int64_t wlo = (top - (t1 - 1)) >> 6, whi = (top - t0) >> 6;
    for (int64_t q = wlo + threadIdx.x; q <= whi; q += BS_THREADS) {
      sh.win_bits[q - wlo] = ld_word(&a.bits[q]);
      sh.win_clr[q - wlo] = 0;
    }
    // thread-major items: thread tid owns window offsets [tid * BS_IPT, (tid + 1) * BS_IPT)
    int32_t p[BS_IPT], nu[BS_IPT], pu[BS_IPT];
    bool first[BS_IPT];
    const int i0 = threadIdx.x * BS_IPT;
    load_run<BS_IPT>(a.trace + t0 + i0, w - i0, 0, p);
    load_run<BS_IPT>(a.next_use + t0 + i0, w - i0, ZX_NEVER, nu);
    load_run<BS_IPT>(a.prev_use + t0 + i0, w - i0, 0, pu);
#pragma unroll
    for (int j = 0; j < BS_IPT; ++j) first[j] = i0 + j < w && pu[j] < t0;
    __syncthreads();
    uint32_t missm = 0, hitm = 0, lastm = 0;  // bit j: item j
    int mc = 0, hc = 0;
#pragma unroll
    for (int j = 0; j < BS_IPT; ++j) {
      const int i = i0 + j;
      if (i >= w) continue;
      if (nu[j] == ZX_NEVER || nu[j] >= t1) lastm |= 1u << j;
      if (first[j]) {
        const int64_t idx = top - (t0 + i);
        const bool res = (sh.win_bits[(idx >> 6) - wlo] >> (idx & 63)) & 1ull;
        if (res) {
          hitm |= 1u << j;
          ++hc;
        } else {
          missm |= 1u << j;
          ++mc;
        }
      }
    }
    int tot;
    const int pre = block_scan(mc | (hc << 16), &tot, sh.scan_ws);
    const int m_base = pre & 0xFFFF, M = tot & 0xFFFF, Hf = tot >> 16;
    const int64_t count0 = st[0];
    const int64_t F = a.capacity - count0 > 0 ? a.capacity - count0 : 0;
    const int E = M > F ? (int)(M - F) : 0;
    if (E > 0 && (count0 - Hf < E || E > BS_EMAX)) {  // not enough statics, or too many victims
      w_lim = w > 1 ? w / 2 : 1;
      continue;
    }

    if (E == 0) {
      // No eviction: admissions, hit clears, miss flags and new keys are independent of
      // one another (hits clear the bits of this window's positions, new keys lie beyond
      // it; atomics on disjoint bits commute), so they go out in one pass and the window
      // waits for memory once.
      int64_t hw = -1, kw = -1;
      unsigned long long hm = 0, km = 0;
      int32_t hb = -1, hc = 0, kb = -1, kc = 0;
#pragma unroll
      for (int j = 0; j < BS_IPT; ++j) {
        const int i = i0 + j;
        if (i >= w) continue;
        if ((missm >> j) & 1) a.resident[p[j]] = 1;
        if ((hitm >> j) & 1) {
          const int64_t idx = top - (t0 + i);
          if ((idx >> 6) != hw) {
            if (hw >= 0) atomicAnd(&a.bits[hw], ~hm);
            hw = idx >> 6;
            hm = 0;
          }
          hm |= 1ull << (idx & 63);
          const int32_t b = (int32_t)(idx / BS_BLOCK_BITS);
          if (hc == 0 || b == hb) {
            hb = b;
            ++hc;
          } else {
            atomicSub(&sh.cnt[b], 1u);
          }
        }
        if (a.miss_flags) a.miss_flags[t0 + i] = (missm >> j) & 1;
        if ((lastm >> j) & 1) {
          const int64_t idx = item_idx(a, p[j], nu[j]);
          a.key[p[j]] = nu[j];
          if ((idx >> 6) != kw) {
            if (kw >= 0) {
              atomicOr(&a.bits[kw], km);
              const int32_t b = (int32_t)((kw * 64) / BS_BLOCK_BITS);
              if (kc == 0 || b == kb) {
                kb = b;
                kc += __popcll(km);
              } else {
                atomicAdd(&sh.cnt[b], (uint32_t)__popcll(km));
              }
            }
            kw = idx >> 6;
            km = 0;
          }
          km |= 1ull << (idx & 63);
        }
      }
      if (kw >= 0) {
        const int32_t b = (int32_t)((kw * 64) / BS_BLOCK_BITS);
        if (kc == 0 || b == kb) {
          kb = b;
          kc += __popcll(km);
        } else {
          atomicAdd(&sh.cnt[b], (uint32_t)__popcll(km));
        }
      }
      if (wave_word_or(hw, hm)) atomicAnd(&a.bits[hw], ~hm);
      if (wave_word_or(kw, km)) atomicOr(&a.bits[kw], km);
      wave_cnt_add(sh.cnt, hb, -hc);
      wave_cnt_add(sh.cnt, kb, kc);
      if (threadIdx.x == 0) {
        st[0] = count0 + M;
        st[2] += M;
        st[3] += w - M;
      }
      w_lim = w_lim < BS_W ? w_lim * 2 : BS_W;
      sync_global();
      t0 = t1;
      continue;
    }

    uint32_t takenm = 0;  // bit j: item j's dynamic candidate was evicted
    int dbase = 0;
    if (E > 0) {
      select_first(a, sh, E);
      const int32_t worst = sh.s_idx[E - 1];
      // dynamic candidates that can beat a needed static, in trace order
      uint32_t candm = 0;
      int dc = 0;
#pragma unroll
      for (int j = 0; j < BS_IPT; ++j)
        if (((lastm >> j) & 1) && item_idx(a, p[j], nu[j]) < worst) {
          candm |= 1u << j;
          ++dc;
        }
      int nd;
      dbase = block_scan(dc, &nd, sh.scan_ws);
      if (nd > BS_EMAX) {
        w_lim = w > 1 ? w / 2 : 1;
        continue;
      }
      int r = dbase, mr = m_base;
#pragma unroll
      for (int j = 0; j < BS_IPT; ++j) {
        if ((candm >> j) & 1) {
          sh.d_idx[r] = (int32_t)item_idx(a, p[j], nu[j]);
          sh.d_t[r] = i0 + j;
          sh.d_page[r] = p[j];
          sh.d_taken[r] = 0;
          ++r;
        }
        if ((missm >> j) & 1) {
          if (mr >= F) sh.ev_t[mr - F] = i0 + j;
          ++mr;
        }
      }
      __syncthreads();
      if (threadIdx.x == 0) sh.n_dyn_victims = 0;
      if (nd == 0) {  // no dynamic candidate can beat a needed static: victims in order
        for (int k = threadIdx.x; k < E; k += BS_THREADS) {
          const int32_t sidx = sh.s_idx[k];
          sh.ev_vidx[k] = sidx;
          sh.ev_vpage[k] = sidx < a.n_pages ? sidx : a.trace[top - sidx];
          sh.ev_dyn[k] = 0;
        }
      } else if (sh.d_t[nd - 1] < sh.ev_t[0]) {
        // Every dynamic candidate exists before the first eviction, so the victims are the
        // E best of (dynamic candidates U statics): merge the two sorted lists by rank.
        for (int q = threadIdx.x; q < nd; q += BS_THREADS) {
          sh.sort_key[q] = sh.d_idx[q];
          sh.sort_val[q] = q;
        }
        __syncthreads();
        sort_candidates(sh, nd);
        for (int q = threadIdx.x; q < nd; q += BS_THREADS) {
          const int rank = q + lower_bound(sh.s_idx, E, sh.sort_key[q]);
          if (rank < E) {
            const int slot = sh.sort_val[q];
            sh.ev_vidx[rank] = sh.sort_key[q];
            sh.ev_vpage[rank] = sh.d_page[slot];
            sh.ev_dyn[rank] = 1;
            sh.d_taken[slot] = 1;
            atomicAdd(&sh.n_dyn_victims, 1);
          }
        }
        for (int k = threadIdx.x; k < E; k += BS_THREADS) {
          const int32_t sidx = sh.s_idx[k];
          const int rank = k + lower_bound(sh.sort_key, nd, sidx);
          if (rank < E) {
            sh.ev_vidx[rank] = sidx;
            sh.ev_vpage[rank] = sidx < a.n_pages ? sidx : a.trace[top - sidx];
            sh.ev_dyn[rank] = 0;
          }
        }
      } else {  // candidates appear between evictions: park them in idx order (park_victims)
        for (int q = threadIdx.x; q < nd; q += BS_THREADS) {
          sh.sort_key[q] = sh.d_idx[q];
          sh.sort_val[q] = q;
        }
        __syncthreads();
        sort_candidates(sh, nd);
        for (int q = threadIdx.x; q < nd; q += BS_THREADS) sh.sort_rel[q] = upper_bound(sh.ev_t, E, sh.d_t[sh.sort_val[q]]);
        __syncthreads();
        if (wid == 0) {
          const int n_dyn = park_victims(sh, E, nd);
          if (lane == 0) sh.n_dyn_victims = n_dyn;
        }
        __syncthreads();
        for (int k = threadIdx.x; k < E; k += BS_THREADS) {
          if (sh.ev_dyn[k]) {
            const int q = sh.ev_vpage[k];
            sh.ev_vpage[k] = sh.d_page[q];
            sh.d_taken[q] = 1;
          } else {
            const int32_t sidx = sh.ev_vidx[k];
            sh.ev_vpage[k] = sidx < a.n_pages ? sidx : a.trace[top - sidx];
          }
        }
      }
      __syncthreads();
      int rr = dbase;
#pragma unroll
      for (int j = 0; j < BS_IPT; ++j)
        if ((candm >> j) & 1) {
          if (sh.d_taken[rr]) takenm |= 1u << j;
          ++rr;
        }
    }
    // Grow the window again only if this one left room for twice its evictions: in a
    // stretch where every access misses, a doubled window would exceed BS_EMAX evictions
    // and be retried at this size anyway.
    if (2 * E <= BS_EMAX) w_lim = w_lim < BS_W ? w_lim * 2 : BS_W;
    // admissions, and hits on pages resident since before the window (their bits are
    // cleared in the LDS copy first, then one atomic per word).  A thread's hits have
    // consecutive bits, so its LDS updates go out once per word, and its first block's
    // count goes through the wave-level sum (later blocks, rare, directly).
    {
      int64_t cw = -1;
      int32_t cb = -1, cc = 0;
      unsigned long long cm = 0;
#pragma unroll
      for (int j = 0; j < BS_IPT; ++j) {
        const int i = i0 + j;
        if (i >= w) continue;
        if ((missm >> j) & 1) a.resident[p[j]] = 1;
        if ((hitm >> j) & 1) {
          const int64_t idx = top - (t0 + i);
          if ((idx >> 6) != cw) {
            if (cw >= 0) atomicOr(&sh.win_clr[cw - wlo], cm);
            cw = idx >> 6;
            cm = 0;
          }
          cm |= 1ull << (idx & 63);
          const int32_t b = (int32_t)(idx / BS_BLOCK_BITS);
          if (cc == 0 || b == cb) {
            cb = b;
            ++cc;
          } else {
            atomicSub(&sh.cnt[b], 1u);
          }
        }
        if (a.miss_flags) a.miss_flags[t0 + i] = (missm >> j) & 1;
      }
      if (wave_word_or(cw, cm)) atomicOr(&sh.win_clr[cw - wlo], cm);
      wave_cnt_add(sh.cnt, cb, -cc);
    }
    __syncthreads();
    for (int64_t q = wlo + threadIdx.x; q <= whi; q += BS_THREADS) {
      const unsigned long long c = sh.win_clr[q - wlo];
      if (c) atomicAnd(&a.bits[q], ~c);
    }

    // Without evictions there are no records and no bulk clear, and the hit clears above
    // touch bits disjoint from the new keys (this window's positions against positions
    // beyond it; atomics on disjoint bits commute): go straight to the new keys, the end
    // of the window waits for everything.
    const int64_t ev0 = st[1];
    if (E > 0) {
      // evictions: records, residency, and the static victims' bits -- those are exactly
      // the first sp set bits of B, so every word up to the last one is cleared with a
      // single atomic
      const int sp = E - sh.n_dyn_victims;
      for (int k = threadIdx.x; k < E; k += BS_THREADS) {
        const int32_t page = sh.ev_vpage[k];
        a.resident[page] = 0;
        if (ev0 + k < a.evict_cap) {
          a.evict_pos[ev0 + k] = (int32_t)(t0 + sh.ev_t[k]);
          a.evict_page[ev0 + k] = page;
        }
      }
      if (sp > 0) {
        const int64_t bound = sh.s_idx[sp - 1];
        for (int li = wid; li < sh.n_list; li += BS_THREADS / 64) {
          if (sh.blk_before[li] >= sp) continue;
          const int b = sh.blk_list[li];
          const int64_t q = (int64_t)b * (BS_BLOCK_BITS / 64) + lane;
          const int64_t lo = q * 64;
          unsigned long long mask = 0;
          if (lo <= bound && lo < a.nbits) mask = lo + 63 <= bound ? ~0ull : ((2ull << (bound - lo)) - 1);
          int removed = 0;
          if (mask) removed = __popcll(atomicAnd(&a.bits[q], ~mask) & mask);
          for (int off = 32; off >= 1; off >>= 1) removed += __shfl_xor(removed, off, 64);
          if (lane == 0 && removed) atomicSub(&sh.cnt[b], (uint32_t)removed);
        }
      }
      // The bulk clear above must land before the new keys are set (it clears every bit up
      // to the last static victim).
      sync_global();
    }
    // pages still resident after their last access in the window get their new key; a
    // thread's consecutive items often share a word, so their bits go out together
    {
      int64_t cur_w = -1;
      unsigned long long cur_m = 0;
      int32_t kb = -1, kc = 0;  // first block's count, summed over the wave at the end
      auto add_cnt = [&](int64_t word, int32_t n) {
        const int32_t b = (int32_t)((word * 64) / BS_BLOCK_BITS);
        if (kc == 0 || b == kb) {
          kb = b;
          kc += n;
        } else {
          atomicAdd(&sh.cnt[b], (uint32_t)n);
        }
      };
#pragma unroll
      for (int j = 0; j < BS_IPT; ++j) {
        if (!((lastm >> j) & 1) || ((takenm >> j) & 1)) continue;
        const int64_t idx = item_idx(a, p[j], nu[j]);
        a.key[p[j]] = nu[j];
        if ((idx >> 6) != cur_w) {
          if (cur_w >= 0) {
            atomicOr(&a.bits[cur_w], cur_m);
            add_cnt(cur_w, __popcll(cur_m));
          }
          cur_w = idx >> 6;
          cur_m = 0;
        }
        cur_m |= 1ull << (idx & 63);
      }
      if (cur_w >= 0) add_cnt(cur_w, __popcll(cur_m));
      if (wave_word_or(cur_w, cur_m)) atomicOr(&a.bits[cur_w], cur_m);
      wave_cnt_add(sh.cnt, kb, kc);
    }
    if (threadIdx.x == 0) {
      st[0] = count0 + M - E;
      st[1] = ev0 + E;
      st[2] += M;
      st[3] += w - M;
    }
    sync_global();
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
