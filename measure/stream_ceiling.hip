// stream_ceiling.hip -- measures the HBM ceilings that bound the KV append and gather on
// this device, with no arithmetic, no scale exchange and no page indirection:
//
//   plain    plain streams (one 16-byte vector per thread, nontemporal loads and stores)
//            with the read:write mixes of the append (2:1) and the gather (1:2), at the
//            byte counts of BASELINE configs[1] / configs[2];
//   pages    reads of random 2 KiB runs (one (page, K/V, head) run of a 16-token FP8 page)
//            out of a 300,000-page pool, the pattern of the paged gather and of decode
//            attention (4.29 GB read), read-only and with the gather's
//            2 bytes written per byte read;
//   append   the access pattern the single-pass append is forced into: a layer of token
//            rows of 4 KiB (2 x 8 heads x 128 bf16) cannot stay on chip (302 MB at
//            configs[1] versus ~170 MB of registers + LDS on 256 CUs), and a slab's scale
//            needs its amax over all tokens, so each step reads one 256-byte slab of every
//            row, with NB = 4 steps in flight per workgroup, and writes 128 bytes per row,
//            contiguously per slab or (as the append does) into 16-token pages in random order.
//            Run as a persistent grid (one 1024-thread workgroup per CU) with the token
//            share of every workgroup fixed (as the fused append does) and with chunks of
//            64 tokens dealt out per slab by an atomic counter;
//   columns  the same column blocks (W = 256 B .. 2 KiB of every 4 KiB row, W / 2 bytes
//            written per row) read by ordinary launches at full occupancy (256-thread
//            workgroups, one launch per column block), which separates the cost of the
//            pattern from the cost of the persistent structure;
//   cache    whether the memory-side Infinity Cache (256 MB) serves a second read: a
//            buffer of C MiB is read once after a 1 GiB flush, then read again, with
//            default-policy (temporal) and nontemporal loads on the first read;
//   chunked  the two-pass design that would rely on it: 1 Gi bf16 elements (2 GiB) as
//            chunks of C MiB, each read twice (a max pass, then a pass that writes 1 byte
//            per element), against the same passes over the whole buffer;
//   slabs    the same two passes over configs[4]'s layer (524,288 rows of 4 KiB) taken by
//            groups of W-byte columns (W = 256 B is one (kv, head) slab, 128 MiB), each
//            group read twice in a row, so that its second read can come from the cache;
//   heads    the bytes of one single-pass per-head quantisation of 1 Gi bf16 elements
//            (2 GiB read, 1 GiB written) as a plain stream (one 16-byte vector per thread)
//            and as the persistent structure of the single-pass quantiser with nothing
//            else in it: one 1024-thread workgroup per CU, 15 waves holding K = 6 vectors
//            of NB = 4 contiguous 64 KiB shares in registers, each share written (8 bytes
//            per vector) and its buffer refilled in turn; the shares fixed per workgroup
//            (as the quantiser has them) or dealt out at run time by an atomic counter.
//
// Usage: stream_ceiling [plain|pages|append|columns|cache|chunked|slabs|heads|all] (default all).
// Prints one line per measurement.  Every access is in bounds; nothing waits on another
// workgroup.  Built by __graft_entry__.build() into measure/bin/stream_ceiling.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#define SC_CHECK(x)                                                                     \
  do {                                                                                  \
    hipError_t e_ = (x);                                                                \
    if (e_ != hipSuccess) {                                                             \
      fprintf(stderr, "HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__);   \
      exit(1);                                                                          \
    }                                                                                   \
  } while (0)

typedef unsigned int sc_v4u __attribute__((ext_vector_type(4)));
typedef unsigned int sc_v2u __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------- 1. plain streams

// RB bytes read and WB bytes written per thread (16 or 8), n threads.
template <int RB, int WB>
__global__ void plain_stream(const char *__restrict__ src, char *__restrict__ dst, long n) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  unsigned a, b, c, d;
  if (RB == 16) {
    const sc_v4u v = __builtin_nontemporal_load(reinterpret_cast<const sc_v4u *>(src) + i);
    a = v.x, b = v.y, c = v.z, d = v.w;
  } else {
    const sc_v2u v = __builtin_nontemporal_load(reinterpret_cast<const sc_v2u *>(src) + i);
    a = v.x, b = v.y, c = v.x ^ 1u, d = v.y ^ 1u;
  }
  if (WB == 16) {
    const sc_v4u o = {a, b ^ 1u, c, d ^ a};
    __builtin_nontemporal_store(o, reinterpret_cast<sc_v4u *>(dst) + i);
  } else {
    const sc_v2u o = {a ^ b, c ^ d};
    __builtin_nontemporal_store(o, reinterpret_cast<sc_v2u *>(dst) + i);
  }
}

// ---------------------------------------------------------------- 2. random page runs

// Workgroup w reads runs w*R .. w*R + R - 1 of the list (2 KiB each, 8 bytes per lane per
// run); with WRITE it stores 16 bytes per lane per run contiguously (the bf16 output).
template <bool WRITE>
__global__ void __launch_bounds__(256) page_runs(const char *__restrict__ pool, const long *__restrict__ runs,
                                                 long n_runs, char *__restrict__ out, unsigned *sink) {
  constexpr int R = 4;
  unsigned acc = 0;
  sc_v2u v[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const long k = (long)blockIdx.x * R + r;
    v[r] = k < n_runs ? __builtin_nontemporal_load(reinterpret_cast<const sc_v2u *>(pool + runs[k]) + threadIdx.x)
                      : sc_v2u{0, 0};
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const long k = (long)blockIdx.x * R + r;
    if (WRITE && k < n_runs) {
      const sc_v4u o = {v[r].x, v[r].y ^ 1u, v[r].x ^ 2u, v[r].y ^ 3u};
      __builtin_nontemporal_store(o, reinterpret_cast<sc_v4u *>(out + k * 4096) + threadIdx.x);
    }
    acc ^= v[r].x ^ v[r].y;
  }
  if (acc == 0x9E3779B9u) sink[0] = acc;
}

// ---------------------------------------------------------------- 3. append pattern

constexpr int SC_TPB = 1024;
constexpr int SC_ROW = 4096;
// Column width W of one step (256 B: one (kv, head) slab; 512 B: two adjacent slabs taken
// as one step), with the bytes a workgroup holds the same for both: chunks of
// 1024 / (W / 16) tokens (one 16-byte vector per lane), K chunks per step, NB steps in flight.
template <int W> struct ScGeom;
template <> struct ScGeom<256> { static constexpr int K = 6, NB = 4; };
template <> struct ScGeom<512> { static constexpr int K = 12, NB = 2; };
constexpr int SC_CT = 64;  // tokens per chunk at W = 256
constexpr int SC_K = ScGeom<256>::K, SC_NB = ScGeom<256>::NB;
constexpr int SC_SLAB = 256, SC_SLABS_PER_ROW = SC_ROW / SC_SLAB;

struct PatternArgs {
  const char *x;  // [L][T][4096 B]
  char *out;      // [L * 4096 / W][T][W / 2 B], or with `page` the pool [L][T / 16 pages][16 slabs][16][128 B]
  long T;
  int n_slabs, n_chunks, dynamic;  // n_slabs: column steps (L * 4096 / W)
  unsigned *counter;  // [n_slabs], zero at launch (dynamic only)
  const int *page;    // null, or the page of each group of 16 tokens (a permutation): the
                      // append's destination, 2 KiB runs of one slab 32 KiB apart
};

template <int W>
__device__ __forceinline__ sc_v4u pat_load(const PatternArgs &a, int s, int c, int tid) {
  constexpr int LPT = W / 16, CT = SC_TPB / LPT, SPR = SC_ROW / W;
  const long tok = (long)c * CT + tid / LPT;
  if (c < 0 || s >= a.n_slabs || tok >= a.T) return sc_v4u{0, 0, 0, 0};
  const int l = s / SPR, j = s % SPR;
  return __builtin_nontemporal_load(
      reinterpret_cast<const sc_v4u *>(a.x + ((long)l * a.T + tok) * SC_ROW + j * W + (tid % LPT) * 16));
}

template <int W>
__device__ __forceinline__ void pat_store(const PatternArgs &a, int s, int c, int tid, sc_v4u v) {
  constexpr int LPT = W / 16, CT = SC_TPB / LPT, SPR = SC_ROW / W;
  const long tok = (long)c * CT + tid / LPT;
  if (c < 0 || s >= a.n_slabs || tok >= a.T) return;
  const sc_v2u o = {v.x ^ v.y, v.z ^ v.w};
  long off;
  if (a.page) {
    const int l = s / SPR, jj = (s % SPR) * (W / 256) + (tid % LPT) / 16;  // the 256 B slab
    const long pages = (a.T + 15) / 16;
    off = (((long)l * pages + a.page[tok >> 4]) * SC_SLABS_PER_ROW + jj) * 2048 + (tok & 15) * 128 + (tid % 16) * 8;
  } else {
    off = ((long)s * a.T + tok) * (W / 2) + (tid % LPT) * 8;
  }
  __builtin_nontemporal_store(o, reinterpret_cast<sc_v2u *>(a.out + off));
}

template <int W>
__global__ void __launch_bounds__(SC_TPB) append_pattern(PatternArgs a) {
  constexpr int K = ScGeom<W>::K, NB = ScGeom<W>::NB;
  __shared__ int base[NB];
  const int tid = threadIdx.x, w = blockIdx.x, G = gridDim.x;
  sc_v4u buf[NB][K];
  int cid[NB][K];
  // chunk ids of step s for buffer i (the same on every lane of the workgroup)
  auto assign = [&](int s, int i) {
    if (!a.dynamic) {
      const int c0 = (int)((long)w * a.n_chunks / G), c1 = (int)((long)(w + 1) * a.n_chunks / G);
#pragma unroll
      for (int k = 0; k < K; ++k) cid[i][k] = c0 + k < c1 ? c0 + k : -1;
    } else {
      __syncthreads();
      if (tid == 0) base[i] = s < a.n_slabs ? (int)atomicAdd(&a.counter[s], (unsigned)K) : a.n_chunks;
      __syncthreads();
      const int b = base[i];
#pragma unroll
      for (int k = 0; k < K; ++k) cid[i][k] = b + k < a.n_chunks ? b + k : -1;
    }
  };
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    assign(i, i);
#pragma unroll
    for (int k = 0; k < K; ++k) buf[i][k] = pat_load<W>(a, i, cid[i][k], tid);
  }
  const int s_pad = (a.n_slabs + NB - 1) / NB * NB;
  for (int s0 = 0; s0 < s_pad; s0 += NB) {
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int s = s0 + i;
#pragma unroll
      for (int k = 0; k < K; ++k) pat_store<W>(a, s, cid[i][k], tid, buf[i][k]);
      assign(s + NB, i);
#pragma unroll
      for (int k = 0; k < K; ++k) buf[i][k] = pat_load<W>(a, s + NB, cid[i][k], tid);
    }
  }
}

// ---------------------------------------------------------------- 4. column blocks, full occupancy

// One launch per column block j: reads bytes [j W, (j + 1) W) of every 4 KiB row and writes
// W / 2 bytes per row (out: this block's [row][W / 2]).  256 threads cover 256 / (W / 16)
// rows per step, U steps per workgroup, all loads issued before the stores.
template <int U, int POL>
__global__ void __launch_bounds__(256) column_block(const char *__restrict__ x, char *__restrict__ out, long rows,
                                                   int W, int j) {
  const int lpr = W / 16;
  const int rpb = 256 / lpr;
  const long r0 = (long)blockIdx.x * U * rpb + threadIdx.x / lpr;
  const int c = threadIdx.x % lpr;
  sc_v4u v[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const long r = r0 + (long)u * rpb;
    const sc_v4u *p = reinterpret_cast<const sc_v4u *>(x + r * 4096 + (long)j * W) + c;
    v[u] = r < rows ? (POL ? __builtin_nontemporal_load(p) : *p) : sc_v4u{0, 0, 0, 0};
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const long r = r0 + (long)u * rpb;
    if (r < rows) {
      const sc_v2u o = {v[u].x ^ v[u].y, v[u].z ^ v[u].w};
      __builtin_nontemporal_store(o, reinterpret_cast<sc_v2u *>(out + r * (W / 2)) + c);
    }
  }
}

// Column group j of W bytes of every 4 KiB row, U rows per thread in flight: WRITE 0 reads
// and folds (an amax pass), WRITE 1 reads and writes W / 2 bytes per row (an encode pass).
// REV takes the row tiles from the end first.  POL 1: nontemporal loads.
template <int U, int WRITE, int POL, int REV>
__global__ void __launch_bounds__(256) column_pass(const char *__restrict__ x, char *__restrict__ out, long rows,
                                                  int W, int j, unsigned *sink) {
  const int lpr = W / 16;
  const int rpb = 256 / lpr;
  const long tile = REV ? (long)gridDim.x - 1 - blockIdx.x : (long)blockIdx.x;
  const long r0 = tile * U * rpb + threadIdx.x / lpr;
  const int c = threadIdx.x % lpr;
  sc_v4u v[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const long r = r0 + (long)u * rpb;
    const sc_v4u *p = reinterpret_cast<const sc_v4u *>(x + r * 4096 + (long)j * W) + c;
    v[u] = r < rows ? (POL ? __builtin_nontemporal_load(p) : *p) : sc_v4u{0, 0, 0, 0};
  }
  if (WRITE) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const long r = r0 + (long)u * rpb;
      if (r < rows) {
        const sc_v2u o = {v[u].x ^ v[u].y, v[u].z ^ v[u].w};
        __builtin_nontemporal_store(o, reinterpret_cast<sc_v2u *>(out + r * (W / 2)) + c);
      }
    }
  } else {
    unsigned m = 0;
#pragma unroll
    for (int u = 0; u < U; ++u) m = max(m, max(v[u].x ^ v[u].y, v[u].z ^ v[u].w));
    if (m == 0x9E3779B9u) sink[0] = m;
  }
}

// ---------------------------------------------------------------- 5./6. cache reuse, chunked passes

// Read of n 16-byte vectors, 4 in flight per thread, folded into a value that is stored
// only if it matches a constant (so the loads are kept).  Each wave takes a contiguous
// chunk of 4 x 64 vectors per round (its 4 loads are adjacent 1 KiB blocks); the grid
// strides over chunks.  (A thread's 4 loads a grid stride apart read 15-20% slower: 5.57 /
// 5.97 TB/s default / nontemporal against 6.40 / 7.15 on 2 GiB.)  POL 0: default cache
// policy; POL 1: nontemporal.
template <int POL>
__global__ void __launch_bounds__(256) read_fold(const sc_v4u *__restrict__ x, long n, unsigned *sink) {
  const long t = (long)blockIdx.x * 256 + threadIdx.x;
  const long round = (long)gridDim.x * 4 * 256;
  unsigned m = 0;
  for (long i = (t >> 6) * 256 + (t & 63); i < n; i += round) {
    sc_v4u v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const long k = i + u * 64;
      v[u] = k < n ? (POL ? __builtin_nontemporal_load(x + k) : x[k]) : sc_v4u{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) m = max(m, max(v[u].x ^ v[u].y, v[u].z ^ v[u].w));
  }
  if (m == 0x9E3779B9u) sink[0] = m;
}

// The same reads, 8 bytes written per 16 read (nontemporal stores).
template <int POL>
__global__ void __launch_bounds__(256) read_write_half(const sc_v4u *__restrict__ x, sc_v2u *__restrict__ out,
                                                       long n) {
  const long t = (long)blockIdx.x * 256 + threadIdx.x;
  const long round = (long)gridDim.x * 4 * 256;
  for (long i = (t >> 6) * 256 + (t & 63); i < n; i += round) {
    sc_v4u v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const long k = i + u * 64;
      v[u] = k < n ? (POL ? __builtin_nontemporal_load(x + k) : x[k]) : sc_v4u{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const long k = i + u * 64;
      if (k < n) __builtin_nontemporal_store(sc_v2u{v[u].x ^ v[u].y, v[u].z ^ v[u].w}, out + k);
    }
  }
}

// ---------------------------------------------------------------- 7. persistent contiguous shares

constexpr int HP_DATA = 960;  // 15 data waves
constexpr int HP_K = 6, HP_NB = 4;
constexpr long HP_SHARE = 4096;  // vectors per share (64 KiB)

// Workgroup w takes shares w, w + G, w + 2G, ... of n vectors; steps past the end load and
// store nothing.  The 16th wave idles, as the control wave of the quantiser mostly does.
__global__ void __launch_bounds__(1024) heads_pattern(const sc_v4u *__restrict__ x, sc_v2u *__restrict__ out,
                                                      long n) {
  const int t = threadIdx.x;
  if (t >= HP_DATA) return;
  const long G = gridDim.x, n_sh = (n + HP_SHARE - 1) / HP_SHARE;
  const long steps = (n_sh - blockIdx.x + G - 1) / G;
  const long steps_pad = (steps + HP_NB - 1) / HP_NB * HP_NB;
  auto idx = [&](long i, int k) -> long {  // vector of slot k at step i, or -1
    const long sh = blockIdx.x + i * G;
    const long v = (long)k * HP_DATA + t;
    return (i < steps && v < HP_SHARE && sh * HP_SHARE + v < n) ? sh * HP_SHARE + v : -1;
  };
  sc_v4u buf[HP_NB][HP_K];
#pragma unroll
  for (int j = 0; j < HP_NB; ++j)
#pragma unroll
    for (int k = 0; k < HP_K; ++k) {
      const long v = idx(j, k);
      buf[j][k] = v >= 0 ? __builtin_nontemporal_load(x + v) : sc_v4u{0, 0, 0, 0};
    }
  for (long i0 = 0; i0 < steps_pad; i0 += HP_NB) {
#pragma unroll
    for (int j = 0; j < HP_NB; ++j) {
      const long i = i0 + j;
#pragma unroll
      for (int k = 0; k < HP_K; ++k) {
        const long v = idx(i, k);
        if (v >= 0) __builtin_nontemporal_store(sc_v2u{buf[j][k].x ^ buf[j][k].y, buf[j][k].z ^ buf[j][k].w}, out + v);
      }
#pragma unroll
      for (int k = 0; k < HP_K; ++k) {
        const long v = idx(i + HP_NB, k);
        buf[j][k] = v >= 0 ? __builtin_nontemporal_load(x + v) : sc_v4u{0, 0, 0, 0};
      }
    }
  }
}

// The same with the shares dealt out at run time: the 16th wave claims share ids from a
// global counter (zero at launch) into an LDS ring ahead of the data waves, so a workgroup
// on a faster part of the chip takes more shares.  Claims only increase, so a data wave
// stops at the first id past the end.
// LAZY: the share of step c is claimed only once every data wave has stored step c - NB
// (the buffer it goes into is free), as a kernel must that may not hold a claimed share it
// has not loaded; otherwise up to HP_RING claims run ahead of the data waves.
constexpr int HP_RING = 8;  // > HP_NB
template <bool LAZY>
__global__ void __launch_bounds__(1024) heads_pattern_dyn(const sc_v4u *__restrict__ x, sc_v2u *__restrict__ out,
                                                          long n, unsigned *counter) {
  __shared__ long sid[HP_RING];
  __shared__ unsigned ready[HP_RING], used[HP_RING], fin[HP_RING];
  const int t = threadIdx.x;
  const long n_sh = (n + HP_SHARE - 1) / HP_SHARE;
  if (t < HP_RING) {
    ready[t] = 0;
    used[t] = 0;
    fin[t] = 0;
  }
  __syncthreads();
  if (t >= HP_DATA) {  // claimer: lane 0 of the 16th wave
    if (t != HP_DATA) return;
    for (int c = 0;; ++c) {
      const int r = c % HP_RING;
      const unsigned need = (unsigned)(c / HP_RING) * (HP_DATA / 64);  // earlier rounds consumed
      while (__hip_atomic_load(&used[r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != need)
        __builtin_amdgcn_s_sleep(1);
      if (LAZY && c >= HP_NB) {  // step c - NB stored by every data wave
        const int f = c - HP_NB;
        const unsigned want = (unsigned)(f / HP_RING + 1) * (HP_DATA / 64);
        while (__hip_atomic_load(&fin[f % HP_RING], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < want)
          __builtin_amdgcn_s_sleep(1);
      }
      const long s = (long)atomicAdd(counter, 1u);
      sid[r] = s;
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      __hip_atomic_store(&ready[r], (unsigned)(c + 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      if (s >= n_sh) return;
    }
  }
  auto get = [&](int c) -> long {
    const int r = c % HP_RING;
    while (__hip_atomic_load(&ready[r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != (unsigned)(c + 1))
      __builtin_amdgcn_s_sleep(1);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    const long s = sid[r];
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    if ((t & 63) == 0) __hip_atomic_fetch_add(&used[r], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    return s;
  };
  auto vec = [&](long sh, int k) -> long {
    const long v = (long)k * HP_DATA + t;
    return (sh < n_sh && v < HP_SHARE && sh * HP_SHARE + v < n) ? sh * HP_SHARE + v : -1;
  };
  long cur[HP_NB];
  sc_v4u buf[HP_NB][HP_K];
  int c_next = 0;
  bool done = false;
#pragma unroll
  for (int j = 0; j < HP_NB; ++j) {
    cur[j] = done ? n_sh : get(c_next++);
    done = done || cur[j] >= n_sh;
#pragma unroll
    for (int k = 0; k < HP_K; ++k) {
      const long v = vec(cur[j], k);
      buf[j][k] = v >= 0 ? __builtin_nontemporal_load(x + v) : sc_v4u{0, 0, 0, 0};
    }
  }
  // a round refills the buffers in claim order: when the first refill is past the end, so
  // are the others, and nothing is left
  for (int i0 = 0; cur[0] < n_sh; i0 += HP_NB) {
#pragma unroll
    for (int j = 0; j < HP_NB; ++j) {
#pragma unroll
      for (int k = 0; k < HP_K; ++k) {
        const long v = vec(cur[j], k);
        if (v >= 0) __builtin_nontemporal_store(sc_v2u{buf[j][k].x ^ buf[j][k].y, buf[j][k].z ^ buf[j][k].w}, out + v);
      }
      if (LAZY && (t & 63) == 0)  // step i0 + j stored by this wave
        __hip_atomic_fetch_add(&fin[(i0 + j) % HP_RING], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      cur[j] = done ? n_sh : get(c_next++);
      done = done || cur[j] >= n_sh;
#pragma unroll
      for (int k = 0; k < HP_K; ++k) {
        const long v = vec(cur[j], k);
        buf[j][k] = v >= 0 ? __builtin_nontemporal_load(x + v) : sc_v4u{0, 0, 0, 0};
      }
    }
  }
}

static unsigned grid_for(long n_vec) {
  const long g = (n_vec + 1023) / 1024;
  return (unsigned)(g < 1 ? 1 : (g > 16384 ? 16384 : g));
}

// ---------------------------------------------------------------- host

template <typename F>
static float best_ms(F launch, int reps) {
  hipEvent_t e0, e1;
  SC_CHECK(hipEventCreate(&e0));
  SC_CHECK(hipEventCreate(&e1));
  float best = 1e30f;
  for (int r = 0; r < reps; ++r) {
    SC_CHECK(hipEventRecord(e0));
    launch();
    SC_CHECK(hipEventRecord(e1));
    SC_CHECK(hipEventSynchronize(e1));
    float ms = 0;
    SC_CHECK(hipEventElapsedTime(&ms, e0, e1));
    best = std::min(best, ms);
  }
  SC_CHECK(hipEventDestroy(e0));
  SC_CHECK(hipEventDestroy(e1));
  return best;
}

static bool want(const char *sel, const char *group) { return !strcmp(sel, "all") || !strcmp(sel, group); }

int main(int argc, char **argv) {
  const char *sel = argc > 1 ? argv[1] : "all";
  // configs[1] with seed 1: 32 layers x 74,902 tokens x 4 KiB rows
  const int L = 32;
  const long T = 74902;
  const long in_bytes = (long)L * T * SC_ROW;  // 9.82 GB
  const long out_bytes = in_bytes / 2;
  char *x = nullptr, *out = nullptr;
  unsigned *counter = nullptr;
  SC_CHECK(hipMalloc(&x, in_bytes));
  SC_CHECK(hipMalloc(&out, in_bytes));  // large enough for the 1:2 stream too
  SC_CHECK(hipMalloc(&counter, 4096 * sizeof(unsigned)));
  SC_CHECK(hipMemset(x, 0x11, in_bytes));
  int ncu = 0;
  SC_CHECK(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, 0));
  printf("device CUs: %d\n", ncu);
  fflush(stdout);

  if (want(sel, "plain")) {  // 2:1 stream over the append's bytes
    const long n = in_bytes / 16;
    float ms = best_ms([&] { plain_stream<16, 8><<<(unsigned)((n + 255) / 256), 256>>>(x, out, n); }, 5);
    printf("plain stream 2:1 (read %.3f GB, write %.3f GB): %.3f ms, %.1f GB/s\n", in_bytes / 1e9, out_bytes / 1e9,
           ms, (in_bytes + out_bytes) / ms / 1e6);
    // 1:2 stream over the gather's bytes (configs[2]: 4.29 GB codes in, 8.59 GB bf16 out)
    const long n2 = 4294967296L / 8;
    ms = best_ms([&] { plain_stream<8, 16><<<(unsigned)((n2 + 255) / 256), 256>>>(x, out, n2); }, 5);
    printf("plain stream 1:2 (read %.3f GB, write %.3f GB): %.3f ms, %.1f GB/s\n", n2 * 8 / 1e9, n2 * 16 / 1e9, ms,
           n2 * 24.0 / ms / 1e6);
    fflush(stdout);
  }
  if (want(sel, "pages")) {  // random 2 KiB runs of a 300,000-page pool (32 KiB pages: K and V x 8 heads x 2 KiB)
    const long n_pool_pages = 300000, page = 32768;
    const long pool_bytes = n_pool_pages * page;  // 9.83 GB
    char *pool = nullptr;
    SC_CHECK(hipMalloc(&pool, pool_bytes));
    SC_CHECK(hipMemset(pool, 0x22, pool_bytes));
    // 64 sequences x 2048 pages x 2 (K, V) x 8 heads runs, pages drawn at random
    const long n_runs = 64L * 2048 * 2 * 8;
    long *runs_h = (long *)malloc(n_runs * sizeof(long));
    unsigned long long r = 88172645463325252ull;
    for (long i = 0; i < n_runs / 16; ++i) {
      r ^= r << 13, r ^= r >> 7, r ^= r << 17;
      const long pg = (long)(r % (unsigned long long)n_pool_pages);
      for (int j = 0; j < 16; ++j) runs_h[i * 16 + j] = pg * page + j * 2048;  // K and V runs of 8 heads
    }
    long *runs = nullptr;
    SC_CHECK(hipMalloc(&runs, n_runs * sizeof(long)));
    SC_CHECK(hipMemcpy(runs, runs_h, n_runs * sizeof(long), hipMemcpyHostToDevice));
    free(runs_h);
    unsigned *sink = counter;
    const unsigned blocks = (unsigned)((n_runs + 3) / 4);
    float ms = best_ms([&] { page_runs<false><<<blocks, 256>>>(pool, runs, n_runs, out, sink); }, 5);
    printf("random 2 KiB page runs, read only (%.3f GB): %.3f ms, %.1f GB/s\n", n_runs * 2048 / 1e9, ms,
           n_runs * 2048.0 / ms / 1e6);
    ms = best_ms([&] { page_runs<true><<<blocks, 256>>>(pool, runs, n_runs, out, sink); }, 5);
    printf("random 2 KiB page runs + 2 B written per byte read (%.3f GB moved): %.3f ms, %.1f GB/s\n",
           n_runs * 6144 / 1e9, ms, n_runs * 6144.0 / ms / 1e6);
    fflush(stdout);
    SC_CHECK(hipFree(pool));
    SC_CHECK(hipFree(runs));
  }
  if (want(sel, "append")) {
    const int chunks = (int)((T + SC_CT - 1) / SC_CT);
    if ((long)ncu * SC_K < chunks) {
      printf("append pattern skipped: %d CUs x %d chunks < %d chunks per slab\n", ncu, SC_K, chunks);
    } else {
      // a random page order for the paged destination (the same for every layer)
      const long pages = (T + 15) / 16;
      int *page_h = static_cast<int *>(malloc(pages * sizeof(int)));
      for (long i = 0; i < pages; ++i) page_h[i] = (int)i;
      srand(5);
      for (long i = pages - 1; i > 0; --i) {
        const long k = rand() % (i + 1);
        std::swap(page_h[i], page_h[k]);
      }
      int *page_d = nullptr;
      SC_CHECK(hipMalloc(&page_d, pages * sizeof(int)));
      SC_CHECK(hipMemcpy(page_d, page_h, pages * sizeof(int), hipMemcpyHostToDevice));
      free(page_h);
      for (int paged = 0; paged < 2; ++paged)
        for (int dyn = 0; dyn < 2; ++dyn) {
          PatternArgs a{x, out, T, L * SC_SLABS_PER_ROW, chunks, dyn, counter, paged ? page_d : nullptr};
          const float ms = best_ms(
              [&] {
                SC_CHECK(hipMemsetAsync(counter, 0, 4096 * sizeof(unsigned)));
                append_pattern<256><<<ncu, SC_TPB>>>(a);
              },
              5);
          printf("append pattern, %s shares, %s (256 B of each 4 KiB row per step, %d steps in flight): %.3f ms, "
                 "%.1f GB/s\n",
                 dyn ? "dynamic" : "static", paged ? "writes into random pages" : "contiguous writes", SC_NB, ms,
                 (in_bytes + out_bytes) / ms / 1e6);
          fflush(stdout);
        }
      // two adjacent slabs per step (512 B of each row), half as many steps in flight
      const int chunks512 = (int)((T + 31) / 32);
      if ((long)ncu * ScGeom<512>::K >= chunks512) {
        for (int paged = 0; paged < 2; ++paged)
          for (int dyn = 0; dyn < 2; ++dyn) {
            PatternArgs a{x, out, T, L * (SC_ROW / 512), chunks512, dyn, counter, paged ? page_d : nullptr};
            const float ms = best_ms(
                [&] {
                  SC_CHECK(hipMemsetAsync(counter, 0, 4096 * sizeof(unsigned)));
                  append_pattern<512><<<ncu, SC_TPB>>>(a);
                },
                5);
            printf("append pattern, %s shares, %s (512 B of each 4 KiB row per step, %d steps in flight): %.3f ms, "
                   "%.1f GB/s\n",
                   dyn ? "dynamic" : "static", paged ? "writes into random pages" : "contiguous writes",
                   ScGeom<512>::NB, ms, (in_bytes + out_bytes) / ms / 1e6);
            fflush(stdout);
          }
      }
      SC_CHECK(hipFree(page_d));
    }
  }
  if (want(sel, "columns")) {
    const long rows = (long)L * T;
    for (int pol = 1; pol >= 0; --pol) {
      for (int W = 256; W <= 2048; W *= 2) {
        const int lpr = W / 16, rpb = 256 / lpr;
        constexpr int U = 4;
        const unsigned blocks = (unsigned)((rows + (long)U * rpb - 1) / ((long)U * rpb));
        const float ms = best_ms(
            [&] {
              for (int j = 0; j < 4096 / W; ++j) {
                if (pol)
                  column_block<U, 1><<<blocks, 256>>>(x, out + (long)j * rows * (W / 2), rows, W, j);
                else
                  column_block<U, 0><<<blocks, 256>>>(x, out + (long)j * rows * (W / 2), rows, W, j);
              }
            },
            3);
        printf("column blocks of %d B per 4 KiB row, one launch per block (%d launches), %s loads: %.3f ms, %.1f "
               "GB/s\n",
               W, 4096 / W, pol ? "nontemporal" : "default", ms, (in_bytes + out_bytes) / ms / 1e6);
        fflush(stdout);
      }
    }
  }
  if (want(sel, "cache")) {
    const long flush_bytes = 1L << 30;
    char *flush = out;  // a region disjoint from the probed one
    unsigned *sink = counter;
    hipEvent_t e0, e1;
    SC_CHECK(hipEventCreate(&e0));
    SC_CHECK(hipEventCreate(&e1));
    const long sizes_mib[] = {16, 32, 64, 128, 192, 256, 384};
    for (int pol = 0; pol < 2; ++pol) {
      for (long mib : sizes_mib) {
        const long bytes = mib << 20, n = bytes / 16;
        float best1 = 1e30f, best2 = 1e30f;
        for (int rep = 0; rep < 3; ++rep) {
          read_fold<0><<<grid_for(flush_bytes / 16), 256>>>(reinterpret_cast<const sc_v4u *>(flush),
                                                             flush_bytes / 16, sink);
          float t1 = 0, t2 = 0;
          SC_CHECK(hipEventRecord(e0));
          if (pol)
            read_fold<1><<<grid_for(n), 256>>>(reinterpret_cast<const sc_v4u *>(x), n, sink);
          else
            read_fold<0><<<grid_for(n), 256>>>(reinterpret_cast<const sc_v4u *>(x), n, sink);
          SC_CHECK(hipEventRecord(e1));
          SC_CHECK(hipEventSynchronize(e1));
          SC_CHECK(hipEventElapsedTime(&t1, e0, e1));
          SC_CHECK(hipEventRecord(e0));
          read_fold<0><<<grid_for(n), 256>>>(reinterpret_cast<const sc_v4u *>(x), n, sink);
          SC_CHECK(hipEventRecord(e1));
          SC_CHECK(hipEventSynchronize(e1));
          SC_CHECK(hipEventElapsedTime(&t2, e0, e1));
          best1 = std::min(best1, t1);
          best2 = std::min(best2, t2);
        }
        printf("cache reuse, %ld MiB: first read (%s loads, after a 1 GiB flush) %.4f ms = %.1f GB/s; second read "
               "(default loads) %.4f ms = %.1f GB/s\n",
               mib, pol ? "nontemporal" : "default", best1, bytes / best1 / 1e6, best2, bytes / best2 / 1e6);
        fflush(stdout);
      }
    }
    SC_CHECK(hipEventDestroy(e0));
    SC_CHECK(hipEventDestroy(e1));
  }
  if (want(sel, "chunked")) {
    const long total = 2L << 30;  // 1 Gi bf16 elements
    const sc_v4u *xv = reinterpret_cast<const sc_v4u *>(x);
    sc_v2u *ov = reinterpret_cast<sc_v2u *>(out);
    unsigned *sink = counter;
    {
      const long n = total / 16;
      const float ms = best_ms([&] { read_write_half<1><<<grid_for(n), 256>>>(xv, ov, n); }, 5);
      printf("chunked: one pass 2:1 over 2 GiB (read 2 GiB, write 1 GiB): %.4f ms, %.1f GB/s of 3 GiB\n", ms,
             3.0 * (1L << 30) / ms / 1e6);
    }
    const long chunk_mib[] = {32, 64, 128, 256, 2048};
    for (int pol = 0; pol < 2; ++pol) {
      for (long mib : chunk_mib) {
        const long c = std::min(total, mib << 20), n = c / 16;
        const float ms = best_ms(
            [&] {
              for (long off = 0; off < total; off += c) {
                const long v0 = off / 16;
                if (pol)
                  read_fold<1><<<grid_for(n), 256>>>(xv + v0, n, sink);
                else
                  read_fold<0><<<grid_for(n), 256>>>(xv + v0, n, sink);
                read_write_half<1><<<grid_for(n), 256>>>(xv + v0, ov + v0, n);
              }
            },
            3);
        printf("chunked two passes, chunks of %ld MiB (%ld launches), first pass %s loads: %.4f ms, %.1f GB/s of "
               "3 GiB algorithmic\n",
               mib, 2 * (total / c), pol ? "nontemporal" : "default", ms, 3.0 * (1L << 30) / ms / 1e6);
        fflush(stdout);
      }
    }
  }
  if (want(sel, "slabs")) {
    // configs[4]'s layer: 524,288 token rows of 4 KiB; a (kv, head) slab is one 256 B column
    const long rows = 524288, total = rows * 4096;
    unsigned *sink = counter;
    for (int rev = 0; rev < 2; ++rev) {
      for (int W = 256; W <= 4096; W *= 2) {
        for (int pol = 0; pol < 2; ++pol) {
          const int lpr = W / 16, rpb = 256 / lpr;
          constexpr int U = 8;
          const unsigned blocks = (unsigned)((rows + (long)U * rpb - 1) / ((long)U * rpb));
          const float ms = best_ms(
              [&] {
                for (int j = 0; j < 4096 / W; ++j) {
                  char *o = out + (long)j * rows * (W / 2);
                  if (pol)
                    column_pass<U, 0, 1, 0><<<blocks, 256>>>(x, o, rows, W, j, sink);
                  else
                    column_pass<U, 0, 0, 0><<<blocks, 256>>>(x, o, rows, W, j, sink);
                  if (rev)
                    column_pass<U, 1, 1, 1><<<blocks, 256>>>(x, o, rows, W, j, sink);
                  else
                    column_pass<U, 1, 1, 0><<<blocks, 256>>>(x, o, rows, W, j, sink);
                }
              },
              4);
          printf("slabs: two passes per group of %d B columns (%ld MiB, %d groups), first pass %s loads, second "
                 "pass %s: %.4f ms, %.1f GB/s of 3 GiB\n",
                 W, rows * W >> 20, 4096 / W, pol ? "nontemporal" : "default",
                 rev ? "back to front" : "front to back", ms, 1.5 * total / ms / 1e6);
          fflush(stdout);
        }
      }
    }
    for (int W = 256; W <= 4096; W *= 4) {  // the first pass alone
      const int lpr = W / 16, rpb = 256 / lpr;
      constexpr int U = 8;
      const unsigned blocks = (unsigned)((rows + (long)U * rpb - 1) / ((long)U * rpb));
      for (int pol = 0; pol < 2; ++pol) {
        const float ms = best_ms(
            [&] {
              for (int j = 0; j < 4096 / W; ++j) {
                if (pol)
                  column_pass<U, 0, 1, 0><<<blocks, 256>>>(x, out, rows, W, j, sink);
                else
                  column_pass<U, 0, 0, 0><<<blocks, 256>>>(x, out, rows, W, j, sink);
              }
            },
            4);
        printf("slabs: read-only pass per group of %d B columns, %s loads: %.4f ms, %.1f GB/s of 2 GiB\n", W,
               pol ? "nontemporal" : "default", ms, (double)total / ms / 1e6);
        fflush(stdout);
      }
    }
  }
  if (want(sel, "heads")) {
    const long total = 2L << 30;  // 1 Gi bf16 elements read, 1 GiB of codes written
    const long n = total / 16;
    const sc_v4u *xv = reinterpret_cast<const sc_v4u *>(x);
    sc_v2u *ov = reinterpret_cast<sc_v2u *>(out);
    float ms = best_ms([&] { plain_stream<16, 8><<<(unsigned)((n + 255) / 256), 256>>>(x, out, n); }, 5);
    printf("heads: plain stream 2:1 over 2 GiB (one vector per thread): %.4f ms, %.1f GB/s of 3 GiB\n", ms,
           3.0 * (1L << 30) / ms / 1e6);
    ms = best_ms([&] { read_fold<1><<<grid_for(n), 256>>>(xv, n, counter); }, 5);
    printf("heads: read-only stream over 2 GiB (4 vectors in flight per thread, nontemporal): %.4f ms, %.1f GB/s\n",
           ms, 2.0 * (1L << 30) / ms / 1e6);
    ms = best_ms([&] { read_fold<0><<<grid_for(n), 256>>>(xv, n, counter); }, 5);
    printf("heads: read-only stream over 2 GiB (default loads): %.4f ms, %.1f GB/s\n", ms,
           2.0 * (1L << 30) / ms / 1e6);
    ms = best_ms([&] { heads_pattern<<<(unsigned)ncu, 1024>>>(xv, ov, n); }, 5);
    printf("heads: persistent grid (%d x 1024), contiguous 64 KiB shares, K = %d, NB = %d: %.4f ms, %.1f GB/s of "
           "3 GiB\n",
           ncu, HP_K, HP_NB, ms, 3.0 * (1L << 30) / ms / 1e6);
    for (int lazy = 0; lazy < 2; ++lazy) {
      ms = best_ms(
          [&] {
            SC_CHECK(hipMemsetAsync(counter, 0, sizeof(unsigned)));
            if (lazy)
              heads_pattern_dyn<true><<<(unsigned)ncu, 1024>>>(xv, ov, n, counter);
            else
              heads_pattern_dyn<false><<<(unsigned)ncu, 1024>>>(xv, ov, n, counter);
          },
          5);
      printf("heads: persistent grid, shares dealt by an atomic counter, %s (counter reset included): %.4f ms, "
             "%.1f GB/s of 3 GiB\n",
             lazy ? "claimed when a buffer frees" : "claimed up to 8 steps ahead", ms, 3.0 * (1L << 30) / ms / 1e6);
    }
    fflush(stdout);
  }
  SC_CHECK(hipFree(x));
  SC_CHECK(hipFree(out));
  SC_CHECK(hipFree(counter));
  return 0;
}
