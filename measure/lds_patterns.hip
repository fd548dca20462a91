// LDS throughput of the ring-attention kernel's operand access patterns on gfx950, and of
// the alternatives measured against them: bytes per clock per CU for one 1024-thread
// block per CU (16 waves), each wave issuing independent LDS instructions (8 reads or 4
// writes per iteration, then one wait), every address inside a 64 KiB array.
//
//   measure/bin/lds_patterns
//
// Patterns (n = lane % 16, kg = lane / 16, as the MFMA operands use them):
//   reads (ds_read_b128, 16 bytes per lane):
//     linear           lane * 16                                        (the ceiling)
//     K rows 272       key n at 272-byte rows, channels 32 kg + 8 c     (zx_prefill.hip's K)
//     K chunk-major    chunk q = 4 kg + c of key n at q * 1024 + 16 n    (alternative)
//     V^T rows 144     channel n at 144-byte rows, 16-byte chunk kg ^ jt (zx_prefill.hip's V^T)
//     V^T chunk-major  ((jt * 2 + kbk) * 4 + kg) * 256 + 16 n            (alternative)
//     stride S         lane n at n * S, the four 16-lane groups 4 KiB apart
//   transposing reads (ds_read_b64_tr_b16, 8 bytes per lane) of V key rows of R bytes:
//     lane L of group kg reads key 4 kg + L / 4, channels 16 jt + 4 (L % 4) ..+4
//   writes (ds_write_b128): the K stores of zx_prefill.hip (thread t: keys 2 (t / 8) + j,
//     channels 16 (t % 8) ..+16, 272-byte rows) and of the chunk-major alternative (lane l:
//     key l % 16 of its wave's tile, chunks 4 (l / 16) ..+4).
#include <hip/hip_runtime.h>
#include <cstdio>

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
constexpr int ITERS = 2048;
constexpr int LDS_BYTES = 65536;

template <int PAT>
__device__ __forceinline__ int read_addr(int l, int j) {
  const int n = l & 15, kg = l >> 4;
  if constexpr (PAT == 0) return l * 16 + 1024 * j;
  if constexpr (PAT == 1) return n * 272 + kg * 64 + 16 * (j & 3) + 4352 * (j >> 2);
  if constexpr (PAT == 2) return ((4 * kg + (j & 3)) * 64 + 16 * (j >> 2) + n) * 16;
  if constexpr (PAT == 3) return n * 144 + ((kg ^ j) << 4);
  if constexpr (PAT == 4) return ((j * 2 * 4 + kg) * 16 + n) * 16;
  if constexpr (PAT >= 100) return n * (PAT - 100) + kg * 4096 + 16 * (j & 3);
  return 0;
}
template <int R>
__device__ __forceinline__ int tr_addr(int l, int j) {
  const int L = l & 15, kg = l >> 4;
  return (4 * kg + (L >> 2) + 16 * (j >> 3)) * R + 2 * (16 * (j & 7) + 4 * (L & 3));
}
template <int PAT>
__device__ __forceinline__ int write_addr(int t, int j) {
  const int g8 = t & 7, kk0 = 2 * (t >> 3), w = t >> 6, l = t & 63;
  if constexpr (PAT == 0) return (kk0 + (j >> 1)) * 272 + 32 * g8 + 16 * (j & 1);
  return ((4 * (l >> 4) + j) * 64 + 16 * w + (l & 15)) * 16;
}

template <int PAT>
__global__ void __launch_bounds__(1024) read_probe(unsigned *out, long long *cyc) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[LDS_BYTES];
  for (int i = threadIdx.x; i < LDS_BYTES / 4; i += blockDim.x) reinterpret_cast<unsigned *>(lds)[i] = i;
  __syncthreads();
  const int l = threadIdx.x & 63, w = threadIdx.x >> 6;
  const unsigned base = (unsigned)(size_t)lds;  // the array's LDS offset
  unsigned a[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) a[j] = base + ((read_addr<PAT>(l, j) + (w & 3) * 16384) & (LDS_BYTES - 1));
  u32x4 acc = {0u, 0u, 0u, 0u};
  __syncthreads();
  const long long c0 = clock64();
  for (int it = 0; it < ITERS; ++it) {
    u32x4 r[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) asm volatile("ds_read_b128 %0, %1" : "=v"(r[j]) : "v"(a[j]));
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int j = 0; j < 8; ++j) acc += r[j];
  }
  __syncthreads();
  const long long c1 = clock64();
  out[blockIdx.x * blockDim.x + threadIdx.x] = acc.x ^ acc.y ^ acc.z ^ acc.w;
  if (threadIdx.x == 0) cyc[blockIdx.x] = c1 - c0;
}

template <int R>
__global__ void __launch_bounds__(1024) tr_probe(unsigned *out, long long *cyc) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[LDS_BYTES];
  for (int i = threadIdx.x; i < LDS_BYTES / 4; i += blockDim.x) reinterpret_cast<unsigned *>(lds)[i] = i;
  __syncthreads();
  const int l = threadIdx.x & 63, w = threadIdx.x >> 6;
  const unsigned base = (unsigned)(size_t)lds;
  unsigned a[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) a[j] = base + ((tr_addr<R>(l, j) + (w & 3) * 16384) & (LDS_BYTES - 1));
  u32x2 acc = {0u, 0u};
  __syncthreads();
  const long long c0 = clock64();
  for (int it = 0; it < ITERS; ++it) {
    u32x2 r[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(r[j]) : "v"(a[j]));
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int j = 0; j < 16; ++j) acc += r[j];
  }
  __syncthreads();
  const long long c1 = clock64();
  out[blockIdx.x * blockDim.x + threadIdx.x] = acc.x ^ acc.y;
  if (threadIdx.x == 0) cyc[blockIdx.x] = c1 - c0;
}

template <int PAT>
__global__ void __launch_bounds__(1024) write_probe(unsigned *out, long long *cyc) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[LDS_BYTES];
  const int t = threadIdx.x & 255, grp = threadIdx.x >> 8;  // four groups of 256 threads, 16 KiB each
  const unsigned base = (unsigned)(size_t)lds;
  unsigned a[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) a[j] = base + (write_addr<PAT>(t, j) & 16383) + grp * 16384;
  u32x4 v = {(unsigned)threadIdx.x, 1u, 2u, 3u};
  __syncthreads();
  const long long c0 = clock64();
  for (int it = 0; it < ITERS; ++it) {
#pragma unroll
    for (int j = 0; j < 4; ++j) asm volatile("ds_write_b128 %0, %1" ::"v"(a[j]), "v"(v) : "memory");
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    v.x += 1u;
  }
  __syncthreads();
  const long long c1 = clock64();
  out[blockIdx.x * blockDim.x + threadIdx.x] = reinterpret_cast<unsigned *>(lds)[threadIdx.x];
  if (threadIdx.x == 0) cyc[blockIdx.x] = c1 - c0;
}

static unsigned *g_out;
static long long *g_cyc;
constexpr int BLOCKS = 256;

template <typename K>
static double bytes_per_clock(K kernel, double bytes_per_block) {
  for (int rep = 0; rep < 2; ++rep) kernel<<<BLOCKS, 1024>>>(g_out, g_cyc);
  if (hipDeviceSynchronize() != hipSuccess) return -1.0;
  long long h[BLOCKS];
  if (hipMemcpy(h, g_cyc, sizeof(h), hipMemcpyDeviceToHost) != hipSuccess) return -1.0;
  double s = 0.0;
  for (int b = 0; b < BLOCKS; ++b) s += (double)h[b];
  return bytes_per_block / (s / BLOCKS);
}

int main() {
  if (hipMalloc(&g_out, BLOCKS * 1024 * 4) != hipSuccess || hipMalloc(&g_cyc, BLOCKS * 8) != hipSuccess) return 1;
  const double rb = 16.0 * 1024 * 8 * ITERS, tb = 8.0 * 1024 * 16 * ITERS, wb = 16.0 * 1024 * 4 * ITERS;
  printf("bytes per clock per CU (clock64), one 1024-thread block per CU\n");
  printf("read  linear                    %6.1f\n", bytes_per_clock(read_probe<0>, rb));
  printf("read  K rows 272 (kernel)       %6.1f\n", bytes_per_clock(read_probe<1>, rb));
  printf("read  K chunk-major             %6.1f\n", bytes_per_clock(read_probe<2>, rb));
  printf("read  V^T rows 144 (kernel)     %6.1f\n", bytes_per_clock(read_probe<3>, rb));
  printf("read  V^T chunk-major           %6.1f\n", bytes_per_clock(read_probe<4>, rb));
#define ZX_STRIDE(S) printf("read  stride %4d               %6.1f\n", S, bytes_per_clock(read_probe<100 + S>, rb));
  ZX_STRIDE(16) ZX_STRIDE(32) ZX_STRIDE(48) ZX_STRIDE(64) ZX_STRIDE(128) ZX_STRIDE(144) ZX_STRIDE(256)
  ZX_STRIDE(272) ZX_STRIDE(288)
  printf("trread V rows 256               %6.1f\n", bytes_per_clock(tr_probe<256>, tb));
  printf("trread V rows 272               %6.1f\n", bytes_per_clock(tr_probe<272>, tb));
  printf("trread V rows 288               %6.1f\n", bytes_per_clock(tr_probe<288>, tb));
  printf("write K rows 272 (kernel)       %6.1f\n", bytes_per_clock(write_probe<0>, wb));
  printf("write K chunk-major             %6.1f\n", bytes_per_clock(write_probe<1>, wb));
  return 0;
}
