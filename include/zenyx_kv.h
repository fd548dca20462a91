/*
 * zenyx_kv.h -- C ABI of libzenyx_kv.so, the MI355X (gfx950) KV-cache hot path.
 *
 * Every entry point takes plain device pointers, element counts and a HIP stream
 * (hipStream_t passed as void*; NULL means the legacy default stream), enqueues its
 * kernels on that stream and returns without synchronising.  Buffers are owned by
 * the caller.  The bulk arrays (activations, code pools, outputs) are moved
 * in 16-byte vectors and must be 16-byte aligned, every layer of them included (hipMalloc
 * and torch allocations are); a misaligned one is refused with ZX_ERR_INVALID.  Scale
 * and index arrays need only their element's alignment.  Return value: ZX_OK (0) or a
 * negative ZX_ERR_* code; a message for the last failure on the calling thread is
 * available from zx_last_error().
 *
 * Reference interfaces each group replaces (paths relative to the zenyx source tree):
 *   - zenyx/streaming/precision.py:8-12   quantize_to_fp8_storage
 *   - zenyx/streaming/precision.py:15-16  dequantize_for_bf16_compute
 *   - zenyx/streaming/belady.py:39-51     BeladyApproxCache._select_victim
 *   - zenyx/streaming/kv_tiering.py:36-66 KVTierManager tier moves (.to / .cpu copies)
 *   - README.md:93-97, 328-331, 343-346   BeladyKVCacheTieringManager / FP8KVQuantizer
 *     (the Phase-7/8 modules named there are absent from the source tree; their
 *      behaviour is defined by this library, see the per-function comments)
 *
 * Numeric contract (shared with the CPU oracle under oracle/):
 *   bf16 values are passed as uint16_t bit patterns, fp8 codes as uint8_t (OCP e4m3fn).
 *   FP8 scale   s = fp32(max(amax, 1e-8f) / 448.0f)   (IEEE division; NaN amax -> NaN s)
 *   FP8 code    c = e4m3fn_RNE(fp32(x) / s)           (IEEE division, RNE, overflow -> NaN)
 *   dequant     y = bf16_RNE(decode(c) * s)
 *   Slabs whose scale is not finite: s = +inf gives code 0x00/0x80 for finite x and
 *   0x7F for non-finite x; s = NaN (any NaN in the slab) gives 0x7F everywhere.
 */
#ifndef ZENYX_KV_H
#define ZENYX_KV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void *zx_stream_t; /* hipStream_t */

enum zx_status {
  ZX_OK = 0,
  ZX_ERR_INVALID = -1,     /* null pointer, negative size, inconsistent arguments */
  ZX_ERR_HIP = -2,         /* a HIP runtime call failed */
  ZX_ERR_UNSUPPORTED = -3, /* shape outside what the kernels handle */
  ZX_ERR_WORKSPACE = -4,   /* workspace missing or too small */
};

enum zx_dtype { ZX_BF16 = 0, ZX_F16 = 1, ZX_F32 = 2 };

/* Error bits a kernel ORs into the caller's device error word (see err arguments). */
enum zx_kernel_error {
  ZX_KERR_PAGE_RANGE = 1, /* a block-table entry outside [0, n_pages) */
  ZX_KERR_POS_RANGE = 2,  /* a token position beyond max_blocks * page_size */
  ZX_KERR_SPIN = 4,       /* a bounded inter-workgroup wait ran out (kernel exited early) */
  ZX_KERR_OVERFLOW = 8,   /* static FP8 scales only: a finite input's quotient x / s rounded
                             beyond the e4m3 range (|x / s| > 464), so its code is the NaN
                             code S.1111.111 (or +-448 with ZX_APPEND_SATURATE) */
};

/* Message describing the last failing call on this thread ("" if none). */
const char *zx_last_error(void);
/* ABI version of the library (bumped on any change of a signature or of a default). */
int zx_abi_version(void);

/* Bound, in microseconds, of one wait without progress inside the cooperative
 * single-pass kernels (zx_kv_quant_append's and zx_fp8_quant_heads' single pass, whose
 * workgroups exchange slab maxima).  When a wait runs out the kernel raises a global
 * abort flag, every wave exits, ZX_KERR_SPIN is ORed into the call's error word and
 * the outputs of that call are undefined.  Default 2,000,000 (2 s); a negative value
 * restores it; 0 makes the first wait without progress give up, which exercises the
 * release path.  Applies to launches issued after the call, process-wide.  No
 * counterpart in the reference (its Phase-8 code is absent); for tests and operators. */
int zx_set_wait_bound_us(int64_t us);

/* ---------------------------------------------------------------------------
 * Legacy per-tensor int8 storage.  Replaces zenyx/streaming/precision.py:8-12.
 *   s = max(amax(|x|), 1e-8) / 127, every step rounded to x's dtype as torch does
 *   q = int8(clamp(round_half_even(dtype(x / s)), -127, 127))
 * x: n elements of `dtype` (ZX_BF16, ZX_F16 or ZX_F32); q: n int8; scale: one
 * element of `dtype` (device).  workspace: >= 256 device bytes.  n must be > 0
 * (the reference raises on an empty tensor, precision.py:10).
 */
int zx_int8_legacy_quant(const void *x, int dtype, int64_t n, int8_t *q, void *scale,
                         void *workspace, size_t workspace_bytes, zx_stream_t stream);

/* Replaces zenyx/streaming/precision.py:15-16: y = bf16_RNE(float(q) * float(scale)).
 * scale: one element of `scale_dtype` (device); y: n bf16. */
int zx_int8_legacy_dequant(const int8_t *q, const void *scale, int scale_dtype, int64_t n,
                           uint16_t *y, zx_stream_t stream);

/* The two functions above applied to n_slabs equal, contiguous slabs of slab_len
 * elements in one launch each, one scale per slab (scales: n_slabs elements of dtype):
 * precision.py:8-16 applied per (layer, kv, head) slab, bit-identical to calling the
 * per-tensor functions on every slab.  1 <= n_slabs <= 65535, slab_len >= 1 for the
 * quant; workspace of zx_int8_legacy_quant_slabs_workspace_bytes(n_slabs) bytes. */
size_t zx_int8_legacy_quant_slabs_workspace_bytes(int64_t n_slabs);
int zx_int8_legacy_quant_slabs(const void *x, int dtype, int64_t n_slabs, int64_t slab_len, int8_t *q,
                               void *scales, void *workspace, size_t workspace_bytes, zx_stream_t stream);
int zx_int8_legacy_dequant_slabs(const int8_t *q, const void *scales, int scale_dtype, int64_t n_slabs,
                                 int64_t slab_len, uint16_t *y, zx_stream_t stream);

/* ---------------------------------------------------------------------------
 * FP8 e4m3fn with one scale per (outer, head): FP8KVQuantizer.quantize
 * (README.md:329, 344; "per-head dynamic scaling" README.md:157).
 * Layout of x / codes / y: [n_outer][n_batch][n_heads][run] (for a KV cache
 * [L][2][B][H][T][D]: n_outer = 2L, run = T*D).  scales: [n_outer][n_heads] fp32,
 * written by quant, read by dequant.  run must be a multiple of 16.
 */
#define ZX_HEADS_TWO_PASS 1    /* flag: amax pass + encode pass instead of the single pass */
#define ZX_HEADS_SINGLE_PASS 2 /* flag: the single pass below 256 MiB too (where it is slower) */
size_t zx_fp8_quant_heads_workspace_bytes(int64_t n_outer, int64_t n_batch, int64_t n_heads, int64_t run);
/* The slab (outer, head) is read once: each of its n_batch runs is cut into shares held in
 * registers by one workgroup each, the workgroups of a slab exchange their maxima through
 * the workspace, then encode what they hold (cooperative launch; every wait is bounded and
 * a timeout sets ZX_KERR_SPIN in *err, device int32, may be NULL).  A slab needing more
 * workgroups than the device holds (n_batch * ceil(run / 46080) > compute units), an input
 * below 256 MiB without ZX_HEADS_SINGLE_PASS (the Infinity Cache serves the second read
 * there, making two passes faster), or ZX_HEADS_TWO_PASS take two passes (same results).
 * workspace: zx_fp8_quant_heads_workspace_bytes() device bytes (unused with two passes,
 * may then be NULL). */
int zx_fp8_quant_heads(const uint16_t *x, int64_t n_outer, int64_t n_batch, int64_t n_heads,
                       int64_t run, uint8_t *codes, float *scales, int32_t flags, int32_t *err,
                       void *workspace, size_t workspace_bytes, zx_stream_t stream);
int zx_fp8_dequant_heads(const uint8_t *codes, const float *scales, int64_t n_outer,
                         int64_t n_batch, int64_t n_heads, int64_t run, uint16_t *y,
                         zx_stream_t stream);

/* Encode already-scaled fp32 values to e4m3fn codes with the same device conversion the
 * kernels above use (utility; no reference counterpart): nearest-even, |v| > 464 or
 * Inf/NaN -> sign | 0x7F. */
int zx_fp8_encode_f32(const float *v, int64_t n, uint8_t *codes, zx_stream_t stream);

/* ---------------------------------------------------------------------------
 * Paged KV cache.  A layer's new tokens arrive token-major, x[n_tok][2][H][D] bf16
 * (K then V), sequences packed by cu_seqlens[n_seqs+1].  Token i of sequence b sits
 * at position start_pos[b] + i, in page block_tables[b][pos / P], row pos % P.
 * Pool layout per layer: [n_pages][2][H][P][D] uint8 codes, so one (page, kv, head)
 * is a contiguous run of P*D bytes.  Scales: [n_layers][2][H] fp32.
 * Supported: head_dim in {64, 128, 256}, 2*H*head_dim <= 8192, page_size >= 1.
 */

/* Per-(layer, kv, head) scales of a token-major batch (dynamic amax). */
int zx_kv_scales(const uint16_t *x, int64_t x_layer_stride, int32_t n_layers, int64_t n_tok,
                 int32_t n_heads, int32_t head_dim, float *scales, zx_stream_t stream);

/* Bytes of device workspace zx_kv_quant_append needs for these arguments. */
size_t zx_kv_quant_append_workspace_bytes(int32_t n_layers, int64_t n_tok, int32_t n_heads,
                                          int32_t head_dim);

#define ZX_APPEND_STATIC_SCALES 1 /* flag: use `scales` as given instead of computing them */
#define ZX_APPEND_SATURATE 4      /* flag, with ZX_APPEND_STATIC_SCALES: a finite input whose
                                     quotient overflows the e4m3 range (ZX_KERR_OVERFLOW) is
                                     stored as +-448 (code S.1111.110, the sign of x / s)
                                     instead of the NaN code; slabs whose static scale is not
                                     finite are unaffected */
#define ZX_APPEND_TWO_PASS 2      /* flag: compute dynamic scales in a separate amax pass
                                     instead of the single-pass cooperative kernel (same
                                     results).  Without this flag or ZX_APPEND_SINGLE_PASS
                                     the library picks: one pass while a CU's share of a
                                     (layer, kv, head) slab is between half and twice what
                                     its registers hold (~38k-150k tokens at D = 128 on
                                     MI355X) and the call has at least 32 slabs, two passes
                                     otherwise and on devices without cooperative launch */
#define ZX_APPEND_SINGLE_PASS 8   /* flag: the single pass whatever the size (where the
                                     device can co-schedule it; same results) */

/* Paged append with fused FP8 quantisation (e.g. 32 layers x ~75k tokens).  Without
 * ZX_APPEND_STATIC_SCALES the scales are computed from this batch (amax over all
 * of its tokens) and written to `scales`; then |x / s| <= 448 (1 + 2^-23) for every
 * finite x and no code overflows (a NaN input makes its slab's scale, and so every code
 * of the slab, NaN, as torch's amax does).  Static scales (a decode step reusing the
 * prefill's scales) may be normal fp32 numbers of either sign, +-inf (finite inputs
 * then encode as the zero x / s signs: sign(x) XOR sign(s)) or NaN; zero and subnormal
 * static scales are outside the contract.  With a finite
 * static scale a token larger than 464 |s| does not fit e4m3: its code is the NaN code
 * (the torch cast's result) and ZX_KERR_OVERFLOW is set in *err, or, with
 * ZX_APPEND_SATURATE, the code is +-448 (and the bit is still set).  Rows whose page id
 * is out of range are skipped and flagged in *err (device int32, may be NULL).  Bits
 * are ORed into *err, never cleared. */
int zx_kv_quant_append(const uint16_t *x, int64_t x_layer_stride, int32_t n_layers,
                       int64_t n_tok, int32_t n_heads, int32_t head_dim,
                       const int32_t *cu_seqlens, const int32_t *start_pos, int32_t n_seqs,
                       const int32_t *block_tables, int32_t max_blocks, int32_t page_size,
                       uint8_t *pool, int64_t pool_layer_stride, int64_t n_pages, float *scales,
                       int32_t flags, int32_t *err, void *workspace, size_t workspace_bytes,
                       zx_stream_t stream);

/* zx_kv_quant_append without a workspace argument, for callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  Same arguments, semantics and results
 * as zx_kv_quant_append; its scratch is a fixed array of
 * ZX_KV_APPEND_NOALLOC_SCRATCH_BYTES in the library's code object, one per GPU, held
 * until the process ends (its address is looked up once per device, on the first call).
 * A call whose zx_kv_quant_append_workspace_bytes() exceeds it fails with
 * ZX_ERR_WORKSPACE before launching anything (at 8 heads, D = 128 and 32 layers: up to
 * about 980,000 tokens).  Calls no allocating routine.  Every call on one GPU uses the
 * same scratch: calls that overlap on one GPU (different streams, or host threads) race;
 * calls in one stream are ordered.  Under stream capture: make one call on the device
 * outside the capture first (it looks up the scratch address and the single pass's
 * occupancy, which are then cached); captured calls (single pass, two passes and static
 * scales alike) replay with the results of an eager call.  A captured graph's replays
 * share the scratch with every other call on that GPU. */
#define ZX_KV_APPEND_NOALLOC_SCRATCH_BYTES (8u << 20)
int zx_kv_quant_append_noalloc(const uint16_t *x, int64_t x_layer_stride, int32_t n_layers,
                               int64_t n_tok, int32_t n_heads, int32_t head_dim,
                               const int32_t *cu_seqlens, const int32_t *start_pos, int32_t n_seqs,
                               const int32_t *block_tables, int32_t max_blocks, int32_t page_size,
                               uint8_t *pool, int64_t pool_layer_stride, int64_t n_pages, float *scales,
                               int32_t flags, int32_t *err, zx_stream_t stream);

/* Paged gather + dequant for decode (e.g. 64 sequences x 32k tokens) of one layer.
 * scales: the layer's [2][H] fp32.  Output k_out, v_out: [n_seqs][H][out_len][D] bf16;
 * positions t >= seq_lens[b] are written as zeros, as are rows whose page id is out of
 * range (flagged in *err, may be NULL). */
int zx_kv_gather_dequant(const uint8_t *pool, int64_t n_pages, int32_t n_heads, int32_t head_dim,
                         int32_t page_size, const float *scales, const int32_t *block_tables,
                         int32_t max_blocks, const int32_t *seq_lens, int32_t n_seqs,
                         int32_t out_len, uint16_t *k_out, uint16_t *v_out, int32_t *err,
                         zx_stream_t stream);

/* Decode attention straight from the FP8 pages (the attention that consumes FP8 pages
 * directly: QuantizedRingAttention, README.md:344, whose code is absent; defined here).
 * q: [n_seqs][n_q_heads][head_dim] bf16, one query token per sequence; query head i reads
 * kv head i / (n_q_heads / n_kv_heads).  For positions t < seq_lens[b]:
 *   s_t = sm_scale * sum_d q[d] * K_t[d],   K_t[d] = decode(code) * scales[0][h]
 *   out = sum_t softmax(s)_t * V_t,         V_t[d] = decode(code) * scales[1][h]
 * computed in fp32 (exp2-domain online softmax, split over positions) and rounded once to
 * bf16: within 1 bf16 ulp of the same expression evaluated exactly.  A sequence of length
 * 0 gives zeros; rows with an out-of-range page id or a position past max_blocks*P are
 * left out and flagged in *err.  out: [n_seqs][n_q_heads][head_dim] bf16.  workspace:
 * zx_paged_attention_decode_workspace_bytes() device bytes (per-split partial results). */
size_t zx_paged_attention_decode_workspace_bytes(int32_t n_seqs, int32_t n_q_heads, int32_t n_kv_heads,
                                                 int32_t head_dim, int32_t max_blocks, int32_t page_size);
int zx_paged_attention_decode(const uint16_t *q, int32_t n_q_heads, const uint8_t *pool, int64_t n_pages,
                              int32_t n_kv_heads, int32_t head_dim, int32_t page_size, const float *scales,
                              const int32_t *block_tables, int32_t max_blocks, const int32_t *seq_lens,
                              int32_t n_seqs, float sm_scale, uint16_t *out, int32_t *err,
                              void *workspace, size_t workspace_bytes, zx_stream_t stream);

/* ---------------------------------------------------------------------------
 * Belady victim selection.  Replaces zenyx/streaming/belady.py:39-51: among the
 * candidate slots (resident[i] != 0; every slot when resident is NULL), pick the
 * largest keys[i] that is > -1; ties go to the smallest rank[i] (when rank is given:
 * the drop-in cache passes each resident id's registration order there, since its
 * slots are reused), then to the smallest slot index.  out (device int64[2]) receives
 * {slot, key}, or {-1, -1} when no slot qualifies.
 * workspace: >= zx_belady_argmax_workspace_bytes(n_slots).
 */
size_t zx_belady_argmax_workspace_bytes(int64_t n_slots);
int zx_belady_argmax(const int64_t *keys, const uint8_t *resident, const int64_t *rank, int64_t n_slots,
                     int64_t *out, void *workspace, size_t workspace_bytes, zx_stream_t stream);

/* Slot updates of the drop-in cache's device tables (BeladyApproxCache.update_future and
 * .touch, belady.py:22-37): for i < n, keys[slot[i]] = key[i], and resident[slot[i]] =
 * res[i] and rank[slot[i]] = rank_in[i] for the tables given (resident with res, rank
 * with rank_in; either pair may be NULL); each slot at most once per call.  slot / key /
 * res / rank_in may live in pinned host memory (the kernel reads them directly) and must
 * stay valid until the update has run.  A slot outside [0, n_slots) is skipped and sets
 * ZX_KERR_PAGE_RANGE in *err (may be NULL). */
int zx_belady_update_slots(int64_t *keys, uint8_t *resident, int64_t *rank, int64_t n_slots,
                           const int64_t *slot, const int64_t *key, const uint8_t *res,
                           const int64_t *rank_in, int64_t n, int32_t *err, zx_stream_t stream);

/* Next/previous use of every trace position: next_use[i] = smallest j > i with
 * trace[j] == trace[i], else ZX_NEVER; prev_use[i] = largest j < i, else -1.
 * trace holds page ids in [0, n_pages); n < 2^31 - 1.  Out-of-range ids set
 * ZX_KERR_PAGE_RANGE in *err (device int32, may be NULL). */
#define ZX_NEVER 0x7FFFFFFF
size_t zx_belady_next_use_workspace_bytes(int64_t n, int32_t n_pages);
int zx_belady_next_use(const int32_t *trace, int64_t n, int32_t n_pages, int32_t *next_use,
                       int32_t *prev_use, int32_t *err, void *workspace, size_t workspace_bytes,
                       zx_stream_t stream);

/* Belady MIN over a page trace (BeladyKVCacheTieringManager, README.md:93-97, 343):
 * a miss with `capacity` (>= 1) pages resident evicts the resident page whose next use
 * is farthest (ZX_NEVER counts as farthest), ties to the smallest page id, then admits
 * the missed page; a hit moves the page's key to its next use.
 * trace/next_use/prev_use cover the whole trace, positions [0, n_total); this call
 * processes positions [t_begin, t_end), so a trace can be fed in pieces.  The cache
 * state lives in the caller's buffers: resident[n_pages] (uint8), key[n_pages] (int32
 * next use of each resident page), state[4] (int64 device: resident count, evictions so
 * far, misses so far, hits so far); zero them all for an empty cache.  Victims are
 * appended to evict_pos/evict_page at index state[1] (stored while < evict_cap, always
 * counted).  miss_flags (uint8[n_total], may be NULL) receives 1 at each miss position
 * of this call and 0 at each hit.
 * workspace: >= zx_belady_simulate_workspace_bytes(n_total, n_pages); n_total + n_pages
 * must not exceed 2^30. */
size_t zx_belady_simulate_workspace_bytes(int64_t n_total, int32_t n_pages);
int zx_belady_simulate(const int32_t *trace, const int32_t *next_use, const int32_t *prev_use,
                       int64_t n_total, int64_t t_begin, int64_t t_end, int32_t n_pages,
                       int64_t capacity, uint8_t *resident, int32_t *key, int64_t *state,
                       int32_t *evict_pos, int32_t *evict_page, int64_t evict_cap,
                       uint8_t *miss_flags, void *workspace, size_t workspace_bytes,
                       zx_stream_t stream);

/* ---------------------------------------------------------------------------
 * Tier moves (replaces the .to(device) / .cpu() copies of kv_tiering.py:46, 54, 60).
 * Copies n_runs runs of `run_bytes` bytes: run i goes from src + src_off[i] to
 * dst + dst_off[i] (offsets in bytes, host arrays).  Adjacent runs are merged into one
 * hipMemcpyAsync.  Host memory must be pinned (hipHostMalloc) for the copy to overlap
 * with kernels on other streams.  `done` (hipEvent_t, may be NULL) is recorded on
 * `stream` after the last copy. */
int zx_tier_copy_runs(void *dst, const void *src, const int64_t *dst_off, const int64_t *src_off,
                      int64_t n_runs, int64_t run_bytes, zx_stream_t stream, void *done);

/* Scattered page moves of a tier (replaces the per-block .to(device) / .cpu() copies of
 * kv_tiering.py:46, 54, 60): page i goes from src + src_off[i] to dst + dst_off[i], each
 * page_bytes (a multiple of 16) long, by one kernel that reads and writes device memory
 * or pinned host memory directly (dst/src 16-byte aligned; pinned host memory must come
 * from hipHostMalloc).  dst_off / src_off hold n_pages int64 byte offsets in memory the
 * device can read (device or pinned host), and must stay valid until the copy is done.
 * A page whose range leaves [0, dst_bytes) or [0, src_bytes) is skipped and sets
 * ZX_KERR_PAGE_RANGE in *err (may be NULL).  max_workgroups <= 0 picks 32 (enough to
 * keep PCIe Gen5 x16 busy on MI355X; more only takes compute units from other work). */
int zx_tier_move_pages(void *dst, int64_t dst_bytes, const void *src, int64_t src_bytes,
                       const int64_t *dst_off, const int64_t *src_off, int64_t n_pages,
                       int64_t page_bytes, int32_t max_workgroups, int32_t *err, zx_stream_t stream);

/* Three-tier Belady plan (README.md:150-154: HBM / DRAM / NVMe tiers with offline-optimal
 * replacement; replaces the LRU spill of kv_tiering.py:57-66).  Inputs are two runs of
 * zx_belady_simulate over the same trace with miss flags: capacity c0 (T0) and c0 + c1
 * (T0 and T1 together), plus the trace's prev_use table.  Per position i writes
 *   src[i]: 0 hit in T0, 1 brought from T1, 2 brought from T2 (seen before), 3 new;
 *   v0[i]:  the page T0 evicts at i (to T1, or to T2 when v1[i] == v0[i]), or -1;
 *   v1[i]:  the page T1 evicts to T2 at i, or -1.
 * Equal to the explicit hierarchy in which T0 sends its farthest page to T1 and T1 its
 * farthest to T2 (Belady MIN is a stack algorithm).  A victim position outside [0, n)
 * sets ZX_KERR_POS_RANGE in *err (may be NULL) and is skipped. */
int zx_belady_tier_plan(const int32_t *prev_use, const uint8_t *miss0, const uint8_t *miss01, int64_t n,
                        const int32_t *e0_pos, const int32_t *e0_page, int64_t n_e0,
                        const int32_t *e01_pos, const int32_t *e01_page, int64_t n_e01, uint8_t *src,
                        int32_t *v0, int32_t *v1, int32_t *err, zx_stream_t stream);

/* Ring-attention page trace of a curriculum of training steps (RingDegreeScheduler /
 * CurriculumPhase, README.md:162-165, 330, 345, code absent; build_ring_timeline of
 * kv_tiering.py:69-73 generalised).  Step k has ring degree degrees[k] = R and
 * ctx_pages[k] = P pages per layer (host arrays); layer l's pages are
 * [l * layer_stride, l * layer_stride + P).  Shard s holds pages
 * [floor(s P / R), floor((s + 1) P / R)).  Forward of a step: per layer, per ring step
 * r, per simulated device d, the pages of shard (d - r) mod R; backward: the exact
 * reverse of the step's forward.  Steps are concatenated into out (device int32, at
 * least zx_ring_curriculum_trace_len() ids; that query returns -1 for a degree or page
 * count below 1). */
int64_t zx_ring_curriculum_trace_len(const int32_t *degrees, const int32_t *ctx_pages, int32_t n_steps,
                                     int32_t n_layers);
int zx_ring_curriculum_trace(const int32_t *degrees, const int32_t *ctx_pages, int32_t n_steps, int32_t n_layers,
                             int32_t layer_stride, int32_t *out, int64_t out_len, zx_stream_t stream);

/* Blocks of queries attending to K/V straight from the paged FP8 pool: one ring step of
 * QuantizedRingAttention (README.md:344, code absent).  Query row i of sequence b (rows
 * [cu_q[b], cu_q[b+1]) of q [n_q][n_q_heads][128] bf16, device) sits at position
 * q_pos0[b] + i - cu_q[b]; query head hq reads kv head hq / (n_q_heads / n_kv_heads) at
 * key positions kp in [kv_begin[b], kv_end[b]) (device int32), with kp <= the query's
 * position when `causal`:
 *   s = sm_scale * q . K_kp,  o = sum_kp softmax(s)_kp V_kp,  K/V = decode(code) * scale,
 *   lse2 = log2(sum_kp exp(s))  (-inf and o = 0 when no key qualifies).
 * Pool layer [n_pages][2][n_kv_heads][page_size][128] e4m3 codes, scales [2][n_kv_heads]
 * fp32, block tables [n_seqs][max_blocks] int32 (an entry outside [0, n_pages) skips its
 * keys and sets ZX_KERR_PAGE_RANGE in *err; kv_end beyond max_blocks * page_size is
 * clipped and sets ZX_KERR_POS_RANGE).  max_q_per_seq >= every sequence's query count
 * (host int; a sequence with more rows has the rest left unwritten and sets
 * ZX_KERR_POS_RANGE).  flags:
 *   ZX_PREFILL_MERGE: merge (o, lse2) into o_acc [n_q][n_q_heads][128] fp32 (normalised
 *     rows) and lse2 [n_q][n_q_heads] fp32, which hold the steps so far;
 *   ZX_PREFILL_INIT (with MERGE): the first step: overwrite instead of merging;
 *   ZX_PREFILL_BF16: also write the (merged) rows to out as bf16;
 *   ZX_PREFILL_LAST (with MERGE and BF16): merge as MERGE does but write the result to out
 *     only, leaving o_acc and lse2 as they were (a ring's last step, when the running
 *     output is not needed afterwards: half of that step's traffic on the running output).
 *   ZX_PREFILL_FINAL (with MERGE and BF16, causal, zx_paged_attention_prefill; ABI
 *     version 7): for a causal ring whose steps cover each sequence's keys in ascending,
 *     contiguous ranges (the first step's kv_begin 0, each later kv_begin the previous
 *     kv_end): a row at a position below kv_begin is left alone (an earlier step finished
 *     it; with INIT no row is); a row below kv_end sees no later key, so it is written to
 *     out as bf16 and not
 *     to o_acc / lse2; the other rows merge into o_acc / lse2 (with LAST: go to out as
 *     well, as final).  Each row then reaches out in the step that completes it, and the
 *     last step converts only the rows it reaches instead of every row.
 * Running every step of a ring with MERGE (INIT on the first) and BF16 on the last (or
 * MERGE | BF16 | FINAL on every step, INIT on the first, LAST on the last) gives
 * attention over the union of the steps' key ranges.  Needs head_dim 128 and a page size
 * that is a multiple of 16.
 * NaN codes (e4m3 0x7F / 0xFF): a NaN K element makes the rows that see its key NaN in
 * every channel (lse2 -inf); a NaN V element makes its channel NaN in the rows that see
 * its key, and may also do so in rows before the key whose 64-key step holds it (the
 * product of the step multiplies their weight 0 by the NaN); a merge keeps a NaN of an
 * earlier step. */
enum {
  ZX_PREFILL_MERGE = 1,
  ZX_PREFILL_INIT = 2,
  ZX_PREFILL_BF16 = 4,
  ZX_PREFILL_FAST_P = 8,
  ZX_PREFILL_EXACT_P = 16,
  ZX_PREFILL_LAST = 32, /* ABI version 6 */
  ZX_PREFILL_FINAL = 64 /* ABI version 7 */
};
/* Precision of P.V.  The row sums use the same rounded softmax weights P as P.V, so a row
 * is an average of V under weights perturbed by at most e relative, which moves it by at
 * most e max|V - out| <= 2 e max|V| (and lse2 by at most log2(1 + e)); steps merged
 * through lse2 stay such an average:
 *   default            P (times 2^7, which keeps it in range) rounded once to fp16, V in
 *                      fp16, one matrix product per tile: e = 2^-11, so |got - exact| <=
 *                      one bf16 ulp + 2^-10 max|V|;
 *   ZX_PREFILL_FAST_P  P rounded once to bf16 (as flash attention usually does), same
 *                      speed: e = 2^-8, one ulp + 2^-7 max|V|;
 *   ZX_PREFILL_EXACT_P P as bf16 hi + lo, two matrix products per tile (~1.3x the time):
 *                      e = 2^-16, one ulp + 2^-15 max|V| at worst (measured within one ulp
 *                      + 2^-17 max|V|). */
/* All R steps of a ring on one GPU in one launch: the same computation as R calls of
 * zx_paged_attention_prefill over key ranges kv_begin[r * n_seqs + b], kv_end[r * n_seqs + b]
 * (r < n_ranges, device int32), except that each block walks the ranges in order with the
 * running row maxima, output and row sums in registers, so nothing is merged through
 * memory between ranges; flags as above (MERGE then merges the union of the ranges into
 * o_acc / lse2 once).  The ranges of a sequence should not overlap (a key in two ranges
 * counts twice).  Within the same tolerance as the per-step composition. */
int zx_paged_attention_prefill(const uint16_t *q, int64_t n_q, const int32_t *cu_q, const int32_t *q_pos0,
                               int32_t n_q_heads, const uint8_t *pool, int64_t n_pages, int32_t n_kv_heads,
                               int32_t head_dim, int32_t page_size, const float *scales,
                               const int32_t *block_tables, int32_t max_blocks, const int32_t *kv_begin,
                               const int32_t *kv_end, int32_t n_seqs, int32_t max_q_per_seq, int32_t causal,
                               float sm_scale, int32_t flags, float *o_acc, float *lse2, uint16_t *out,
                               int32_t *err, zx_stream_t stream);
int zx_paged_attention_ring(const uint16_t *q, int64_t n_q, const int32_t *cu_q, const int32_t *q_pos0,
                            int32_t n_q_heads, const uint8_t *pool, int64_t n_pages, int32_t n_kv_heads,
                            int32_t head_dim, int32_t page_size, const float *scales, const int32_t *block_tables,
                            int32_t max_blocks, const int32_t *kv_begin, const int32_t *kv_end, int32_t n_ranges,
                            int32_t n_seqs, int32_t max_q_per_seq, int32_t causal, float sm_scale, int32_t flags,
                            float *o_acc, float *lse2, uint16_t *out, int32_t *err, zx_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* ZENYX_KV_H */
