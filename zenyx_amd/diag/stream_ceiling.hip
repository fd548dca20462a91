// stream_ceiling.hip -- measures the HBM ceilings that bound the KV append and gather on
// this device, with no arithmetic, no scale exchange and no page indirection:
//
//   1. plain streams (one 16-byte vector per thread, nontemporal loads and stores) with
//      the read:write mixes of the append (2:1) and the gather (1:2), at the byte counts
//      of BASELINE configs[1] / configs[2];
//   2. reads of random 2 KiB runs (one (page, K/V, head) run of a 16-token FP8 page)
//      out of a 300,000-page pool, the pattern of the paged gather and of decode
//      attention (4.29 GB read), read-only and with the gather's
//      2 bytes written per byte read;
//   3. the access pattern the single-pass append is forced into: a layer of token rows
//      of 4 KiB (2 x 8 heads x 128 bf16) cannot stay on chip (302 MB at configs[1] versus
//      ~170 MB of registers + LDS on 256 CUs), and a slab's scale needs its amax over all
//      tokens, so each step reads one 256-byte slab of every row, with NB = 4 steps in
//      flight per workgroup, and writes 128 bytes per row contiguously.  Run as a
//      persistent grid (one 1024-thread workgroup per CU) with the token share of every
//      workgroup fixed (as the fused append does) and with chunks of 64 tokens dealt out
//      per slab by an atomic counter.
//
// Prints one line per measurement.  Every access is in bounds; nothing waits on another
// workgroup.  Built by zenyx_amd/build.py into zenyx_amd/lib/zx_stream_ceiling.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>

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
constexpr int SC_CT = 64;  // tokens per chunk: 64 x 16 vectors = one 16-byte vector per lane
constexpr int SC_K = 6;    // chunks a workgroup holds per slab
constexpr int SC_NB = 4;   // slabs in flight per workgroup
constexpr int SC_ROW = 4096, SC_SLAB = 256, SC_SLABS_PER_ROW = SC_ROW / SC_SLAB;

struct PatternArgs {
  const char *x;  // [L][T][4096 B]
  char *out;      // [L * 16][T][128 B]
  long T;
  int n_slabs, n_chunks, dynamic;
  unsigned *counter;  // [n_slabs], zero at launch (dynamic only)
};

__device__ __forceinline__ sc_v4u pat_load(const PatternArgs &a, int s, int c, int tid) {
  const long tok = (long)c * SC_CT + tid / 16;
  if (c < 0 || s >= a.n_slabs || tok >= a.T) return sc_v4u{0, 0, 0, 0};
  const int l = s / SC_SLABS_PER_ROW, j = s % SC_SLABS_PER_ROW;
  return __builtin_nontemporal_load(
      reinterpret_cast<const sc_v4u *>(a.x + ((long)l * a.T + tok) * SC_ROW + j * SC_SLAB + (tid % 16) * 16));
}

__device__ __forceinline__ void pat_store(const PatternArgs &a, int s, int c, int tid, sc_v4u v) {
  const long tok = (long)c * SC_CT + tid / 16;
  if (c < 0 || s >= a.n_slabs || tok >= a.T) return;
  const sc_v2u o = {v.x ^ v.y, v.z ^ v.w};
  __builtin_nontemporal_store(o, reinterpret_cast<sc_v2u *>(a.out + ((long)s * a.T + tok) * 128 + (tid % 16) * 8));
}

__global__ void __launch_bounds__(SC_TPB) append_pattern(PatternArgs a) {
  __shared__ int base[SC_NB];
  const int tid = threadIdx.x, w = blockIdx.x, G = gridDim.x;
  sc_v4u buf[SC_NB][SC_K];
  int cid[SC_NB][SC_K];
  // chunk ids of slab s for buffer i (the same on every lane of the workgroup)
  auto assign = [&](int s, int i) {
    if (!a.dynamic) {
      const int c0 = (int)((long)w * a.n_chunks / G), c1 = (int)((long)(w + 1) * a.n_chunks / G);
#pragma unroll
      for (int k = 0; k < SC_K; ++k) cid[i][k] = c0 + k < c1 ? c0 + k : -1;
    } else {
      __syncthreads();
      if (tid == 0) base[i] = s < a.n_slabs ? (int)atomicAdd(&a.counter[s], (unsigned)SC_K) : a.n_chunks;
      __syncthreads();
      const int b = base[i];
#pragma unroll
      for (int k = 0; k < SC_K; ++k) cid[i][k] = b + k < a.n_chunks ? b + k : -1;
    }
  };
#pragma unroll
  for (int i = 0; i < SC_NB; ++i) {
    assign(i, i);
#pragma unroll
    for (int k = 0; k < SC_K; ++k) buf[i][k] = pat_load(a, i, cid[i][k], tid);
  }
  const int s_pad = (a.n_slabs + SC_NB - 1) / SC_NB * SC_NB;
  for (int s0 = 0; s0 < s_pad; s0 += SC_NB) {
#pragma unroll
    for (int i = 0; i < SC_NB; ++i) {
      const int s = s0 + i;
#pragma unroll
      for (int k = 0; k < SC_K; ++k) pat_store(a, s, cid[i][k], tid, buf[i][k]);
      assign(s + SC_NB, i);
#pragma unroll
      for (int k = 0; k < SC_K; ++k) buf[i][k] = pat_load(a, s + SC_NB, cid[i][k], tid);
    }
  }
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

int main() {
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

  {  // 2:1 stream over the append's bytes
    const long n = in_bytes / 16;
    const float ms = best_ms([&] { plain_stream<16, 8><<<(unsigned)((n + 255) / 256), 256>>>(x, out, n); }, 5);
    printf("plain stream 2:1 (read %.3f GB, write %.3f GB): %.3f ms, %.1f GB/s\n", in_bytes / 1e9, out_bytes / 1e9,
           ms, (in_bytes + out_bytes) / ms / 1e6);
  }
  {  // 1:2 stream over the gather's bytes (configs[2]: 4.29 GB codes in, 8.59 GB bf16 out)
    const long n = 4294967296L / 8;
    const float ms = best_ms([&] { plain_stream<8, 16><<<(unsigned)((n + 255) / 256), 256>>>(x, out, n); }, 5);
    printf("plain stream 1:2 (read %.3f GB, write %.3f GB): %.3f ms, %.1f GB/s\n", n * 8 / 1e9, n * 16 / 1e9, ms,
           n * 24.0 / ms / 1e6);
  }
  {  // random 2 KiB runs of a 300,000-page pool (32 KiB pages: K and V x 8 heads x 2 KiB)
    const long n_pool_pages = 300000, page = 32768;
    const long pool_bytes = n_pool_pages * page;  // 9.83 GB
    char *pool = nullptr;
    SC_CHECK(hipMalloc(&pool, pool_bytes));
    SC_CHECK(hipMemset(pool, 0x22, pool_bytes));
    // 64 sequences x 2048 pages x 2 (K, V) x 8 heads runs, pages drawn at random
    const long n_runs = 64L * 2048 * 2 * 8;
    long *runs_h = (long *)malloc(n_runs * sizeof(long));
    unsigned long long x = 88172645463325252ull;
    for (long i = 0; i < n_runs / 16; ++i) {
      x ^= x << 13, x ^= x >> 7, x ^= x << 17;
      const long pg = (long)(x % (unsigned long long)n_pool_pages);
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
    SC_CHECK(hipFree(pool));
    SC_CHECK(hipFree(runs));
  }
  const int chunks = (int)((T + SC_CT - 1) / SC_CT);
  if ((long)ncu * SC_K < chunks) {
    printf("append pattern skipped: %d CUs x %d chunks < %d chunks per slab\n", ncu, SC_K, chunks);
    return 0;
  }
  for (int dyn = 0; dyn < 2; ++dyn) {
    PatternArgs a{x, out, T, L * SC_SLABS_PER_ROW, chunks, dyn, counter};
    const float ms = best_ms(
        [&] {
          SC_CHECK(hipMemsetAsync(counter, 0, 4096 * sizeof(unsigned)));
          append_pattern<<<ncu, SC_TPB>>>(a);
        },
        5);
    printf("append pattern, %s shares (256 B of each 4 KiB row per step, %d steps in flight): %.3f ms, %.1f GB/s\n",
           dyn ? "dynamic" : "static", SC_NB, ms, (in_bytes + out_bytes) / ms / 1e6);
  }
  SC_CHECK(hipFree(x));
  SC_CHECK(hipFree(out));
  SC_CHECK(hipFree(counter));
  return 0;
}
