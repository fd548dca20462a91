// zx_tier.hip -- HBM <-> pinned-host tier moves (replaces the synchronous .to(device) /
// .cpu() copies of zenyx/streaming/kv_tiering.py:46, 54, 60).  Runs of pages are merged
// where they are adjacent on both sides and issued as hipMemcpyAsync on the caller's
// (side) stream, so they overlap with kernels on other streams.
#include "zx_common.h"

using namespace zx;

extern "C" int zx_tier_copy_runs(void *dst, const void *src, const int64_t *dst_off, const int64_t *src_off,
                                 int64_t n_runs, int64_t run_bytes, zx_stream_t stream, void *done) {
  clear_error();
  ZX_REQUIRE(n_runs >= 0 && run_bytes > 0, "tier_copy_runs: bad sizes");
  ZX_REQUIRE(n_runs == 0 || (dst && src && dst_off && src_off), "tier_copy_runs: null pointer");
  hipStream_t st = as_stream(stream);
  int64_t i = 0;
  while (i < n_runs) {
    ZX_REQUIRE(dst_off[i] >= 0 && src_off[i] >= 0, "tier_copy_runs: negative offset at run %lld",
               (long long)i);
    int64_t j = i + 1;
    while (j < n_runs && dst_off[j] == dst_off[j - 1] + run_bytes && src_off[j] == src_off[j - 1] + run_bytes)
      ++j;
    ZX_TRY_HIP(hipMemcpyAsync(static_cast<char *>(dst) + dst_off[i], static_cast<const char *>(src) + src_off[i],
                              (size_t)((j - i) * run_bytes), hipMemcpyDefault, st));
    i = j;
  }
  if (done) ZX_TRY_HIP(hipEventRecord(reinterpret_cast<hipEvent_t>(done), st));
  return ZX_OK;
}
