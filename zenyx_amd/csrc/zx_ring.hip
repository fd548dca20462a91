// zx_ring.hip -- ring-attention page traces for a curriculum of ring degrees
// (RingDegreeScheduler / CurriculumPhase, README.md:162-165, 330, 345: "progressive ring
// degree expansion"; code absent), generalising build_ring_timeline
// (zenyx/streaming/kv_tiering.py:69-73) to degree R with uneven shards.
//
// In step k (degree R, P pages per layer) shard s of a layer holds pages
// [floor(s P / R), floor((s + 1) P / R)); at ring step r simulated device d reads shard
// (d - r) mod R, so the devices of ring step r read shards a, a + 1, ..., R - 1, 0, ...,
// a - 1 with a = (R - r) mod R: one rotation of the layer's pages, starting at
// floor(a P / R).  Every position of the trace is therefore one closed-form expression
// and the kernel is a plain elementwise write (4 bytes per access).
#include "zx_common.h"

using namespace zx;

__global__ void ring_trace_step_kernel(int32_t *__restrict__ out, int64_t half, int64_t R, int64_t P,
                                       int64_t stride) {
  const int64_t RP = R * P;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < 2 * half;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t f = i < half ? i : 2 * half - 1 - i;  // the backward pass reverses the forward
    const int64_t l = f / RP, rem = f - l * RP;
    const int64_t r = rem / P, o = rem - r * P;
    const int64_t a = (R - r) % R;
    const int64_t start = a * P / R;
    int64_t j = start + o;
    if (j >= P) j -= P;
    out[i] = (int32_t)(l * stride + j);
  }
}

extern "C" int64_t zx_ring_curriculum_trace_len(const int32_t *degrees, const int32_t *ctx_pages, int32_t n_steps,
                                                int32_t n_layers) {
  if (!degrees || !ctx_pages || n_steps < 0 || n_layers < 1) return -1;
  int64_t n = 0;
  for (int32_t k = 0; k < n_steps; ++k) {
    if (degrees[k] < 1 || ctx_pages[k] < 1) return -1;
    n += 2LL * n_layers * degrees[k] * ctx_pages[k];
  }
  return n;
}

extern "C" int zx_ring_curriculum_trace(const int32_t *degrees, const int32_t *ctx_pages, int32_t n_steps,
                                        int32_t n_layers, int32_t layer_stride, int32_t *out, int64_t out_len,
                                        zx_stream_t stream) {
  clear_error();
  ZX_REQUIRE(degrees && ctx_pages && n_steps >= 0 && n_layers >= 1, "ring_curriculum_trace: bad arguments");
  const int64_t need = zx_ring_curriculum_trace_len(degrees, ctx_pages, n_steps, n_layers);
  ZX_REQUIRE(need >= 0, "ring_curriculum_trace: degrees and pages per layer must be >= 1");
  for (int32_t k = 0; k < n_steps; ++k)
    ZX_REQUIRE(ctx_pages[k] <= layer_stride, "ring_curriculum_trace: step %d has %d pages per layer > layer_stride %d",
               k, ctx_pages[k], layer_stride);
  ZX_REQUIRE((int64_t)(n_layers - 1) * layer_stride + layer_stride <= 0x7FFFFFFFLL,
             "ring_curriculum_trace: page ids beyond int32");
  ZX_REQUIRE(out || need == 0, "ring_curriculum_trace: null output");
  ZX_REQUIRE(out_len >= need, "ring_curriculum_trace: output holds %lld ids, the trace has %lld",
             (long long)out_len, (long long)need);
  hipStream_t st = as_stream(stream);
  int64_t off = 0;
  for (int32_t k = 0; k < n_steps; ++k) {
    const int64_t half = (int64_t)n_layers * degrees[k] * ctx_pages[k];
    const int64_t blocks = ceil_div(2 * half, 256);
    ring_trace_step_kernel<<<(int)(blocks < 16384 ? blocks : 16384), 256, 0, st>>>(out + off, half, degrees[k],
                                                                                  ctx_pages[k], layer_stride);
    int rc = check_launch("ring_trace_step");
    if (rc) return rc;
    off += 2 * half;
  }
  return ZX_OK;
}
