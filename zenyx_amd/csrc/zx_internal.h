// zx_internal.h -- helpers shared between the translation units of libzenyx_kv.so.
#pragma once

#include "zx_common.h"

namespace zx {

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Sets n 32-bit words to v with a kernel (graph-capture safe, unlike hipMemsetAsync).
int fill_u32(uint32_t *p, int64_t n, uint32_t v, hipStream_t st);

// Single-pass paged append with dynamic scales (zx_append_fused.hip).  Returns
// ZX_ERR_UNSUPPORTED when the device cannot run it (the caller then uses two passes).
// append_fused_preferred: whether the single pass beats two passes for this call (a
// workgroup's share of a slab between half and twice what its registers hold, and enough
// slabs to fill its pipeline; measured on MI355X).
size_t append_fused_workspace_bytes(int32_t n_layers, int32_t n_heads);
bool append_fused_preferred(int64_t n_tok, int32_t head_dim, int64_t n_slabs);
int append_fused(const uint16_t *x, int64_t x_layer_stride, int32_t n_layers, int64_t n_tok, int32_t n_heads,
                 int32_t head_dim, const int64_t *tok_off, uint8_t *pool, int64_t pool_layer_stride,
                 int32_t page_size, float *scales, int32_t *err, void *ws, hipStream_t st);

// Single-pass FP8 quantisation per (outer, head) slab (zx_heads_fused.hip).  Returns
// ZX_ERR_UNSUPPORTED when the shape or the device does not allow it (the caller then uses
// two passes).
size_t heads_fused_workspace_bytes(int64_t n_outer, int64_t n_batch, int64_t n_heads, int64_t run);
int heads_fused(const uint16_t *x, int64_t n_outer, int64_t n_batch, int64_t n_heads, int64_t run, uint8_t *codes,
                float *scales, int32_t *err, void *ws, size_t ws_bytes, hipStream_t st);

}  // namespace zx
