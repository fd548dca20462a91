// zx_belady_sim.hip -- trace-level Belady MIN simulator (BeladyKVCacheTieringManager).
#include "zx_common.h"

using namespace zx;

extern "C" size_t zx_belady_simulate_workspace_bytes(int64_t n_total, int32_t n_pages) {
  (void)n_total;
  (void)n_pages;
  return 256;
}

extern "C" int zx_belady_simulate(const int32_t *trace, const int32_t *next_use, const int32_t *prev_use,
                                  int64_t n_total, int64_t t_begin, int64_t t_end, int32_t n_pages,
                                  int64_t capacity, uint8_t *resident, int32_t *key, int64_t *state,
                                  int32_t *evict_pos, int32_t *evict_page, int64_t evict_cap,
                                  uint8_t *miss_flags, void *workspace, size_t workspace_bytes,
                                  zx_stream_t stream) {
  clear_error();
  return fail(ZX_ERR_UNSUPPORTED, "belady_simulate: not built yet");
}
