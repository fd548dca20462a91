// zx_gather.hip -- paged gather + FP8 dequant for decode (sized for 64 sequences x 32k tokens).
// Pool layout per layer: [n_pages][2][H][P][D] uint8; output [B][H][T][D] bf16 per kv.
// Thread work units are 8 codes (8 B in, 16 B out), so each load instruction of a wave
// reads 512 contiguous bytes and each store writes 1 KB contiguous; both are
// nontemporal (codes are read once, the output is streamed, not re-read here).
// Two kernels: gather_slices_kernel when P is a multiple of the 256-unit slice (every
// slice inside one page: block-uniform page lookups, no per-lane branch), otherwise
// gather_dequant_kernel (per-lane page lookup; 4 units per thread).
// HBM-bound: 1 B read + 2 B written per element, plus one int32 block-table entry per
// P positions.
#include "zx_common.h"

namespace zx {

constexpr int GD_THREADS = 256;
constexpr int GD_UNITS = 4;  // 8-code work units per thread
#ifndef GS_UNITS
#define GS_UNITS 4  // slices per block of the fast path (MI355X, configs[2]: 4 > 8 > 2 >> 1)
#endif

typedef unsigned int v4u_t __attribute__((ext_vector_type(4)));

// 8 e4m3 codes -> 8 bf16 values.
__device__ __forceinline__ uint4 dequant8(uint2 c, float s) {
  float a, b, cc, d, e, f, g, h;
  e4m3x4_decode(c.x, a, b, cc, d);
  e4m3x4_decode(c.y, e, f, g, h);
  return make_uint4(pack_bf16(a * s, b * s), pack_bf16(cc * s, d * s), pack_bf16(e * s, f * s),
                    pack_bf16(g * s, h * s));
}

struct GatherGeom {
  int32_t n_heads, head_dim, page_size, max_blocks, out_len;
  int32_t upt_log2;  // log2(8-code units per token) = log2(D / 8)
  int32_t tt;        // positions per block
  int64_t chunks_per_row;
  int64_t n_pages;
};

__global__ void __launch_bounds__(GD_THREADS)
gather_dequant_kernel(const uint8_t *pool, GatherGeom g, const float *scales,
                      const int32_t *block_tables, const int32_t *seq_lens, uint16_t *k_out,
                      uint16_t *v_out, int32_t *err) {
  const int64_t blk = blockIdx.x;
  const int64_t row = blk / g.chunks_per_row;
  const int64_t chunk = blk - row * g.chunks_per_row;
  const int kv = (int)(row & 1);
  const int64_t bh = row >> 1;
  const int h = (int)(bh % g.n_heads);
  const int64_t b = bh / g.n_heads;
  const float s = scales[kv * g.n_heads + h];
  const int32_t len = seq_lens[b];
  const int32_t *bt = block_tables + b * g.max_blocks;
  const int64_t page_bytes = 2LL * g.n_heads * g.page_size * g.head_dim;
  const uint8_t *pbase = pool + ((int64_t)kv * g.n_heads + h) * g.page_size * g.head_dim;
  uint16_t *out = (kv ? v_out : k_out) + bh * (int64_t)g.out_len * g.head_dim;
  const int umask = (1 << g.upt_log2) - 1;

  uint2 c[GD_UNITS];
  int64_t o_off[GD_UNITS];
  bool live[GD_UNITS], have[GD_UNITS];
  int32_t e = 0;
#pragma unroll
  for (int k = 0; k < GD_UNITS; ++k) {
    const int u = k * GD_THREADS + threadIdx.x;
    const int64_t t = chunk * g.tt + (u >> g.upt_log2);
    const int dc = u & umask;
    live[k] = t < g.out_len;
    have[k] = false;
    o_off[k] = t * g.head_dim + dc * 8;
    c[k] = make_uint2(0, 0);
    if (live[k] && t < len) {
      const int64_t bi = t / g.page_size;
      if (bi < g.max_blocks) {
        const int64_t page = bt[bi];
        if (page >= 0 && page < g.n_pages) {
          c[k] = *reinterpret_cast<const uint2 *>(pbase + page * page_bytes +
                                                   (t - bi * g.page_size) * g.head_dim + dc * 8);
          have[k] = true;
        } else {
          e |= ZX_KERR_PAGE_RANGE;
        }
      } else {
        e |= ZX_KERR_POS_RANGE;
      }
    }
  }
#pragma unroll
  for (int k = 0; k < GD_UNITS; ++k) {
    if (!live[k]) continue;
    const uint4 o = have[k] ? dequant8(c[k], s) : make_uint4(0, 0, 0, 0);
    const v4u_t w = {o.x, o.y, o.z, o.w};
    __builtin_nontemporal_store(w, reinterpret_cast<v4u_t *>(out + o_off[k]));
  }
  if (e && err) atomicOr(err, e);
}

// Fast path, for page sizes that are a multiple of TK = 256 / (D / 8) tokens (P = 16 at
// D = 128): a block covers U slices of TK consecutive positions of one (b, h, kv) row;
// every slice lies inside one page, so its block-table entry, validity and error bits
// are block-uniform (scalar loads and branches).  Lane i moves bytes [8i, 8i + 8) of the
// slice's codes and [16i, 16i + 16) of its output: one 2 KiB read and one 4 KiB write
// per wave-slice, through buffer resources whose num_records ends at the last valid row
// (positions past seq_len load zeros, which dequantise to +0; past out_len nothing is
// stored), so the data path has no per-lane branch.
typedef unsigned int v2u_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ __amdgpu_buffer_rsrc_t gd_rsrc(const void *base, int num_records) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, num_records, 0x00020000);
}
constexpr int GD_NT = 2;  // nontemporal: codes are read once, the output is streamed

template <int U>
__global__ void __launch_bounds__(GD_THREADS)
gather_slices_kernel(const uint8_t *__restrict__ pool, GatherGeom g, const float *__restrict__ scales,
                     const int32_t *__restrict__ block_tables, const int32_t *__restrict__ seq_lens,
                     uint16_t *k_out, uint16_t *v_out, int32_t *err) {
  const int64_t blk = blockIdx.x;
  const int64_t row = blk / g.chunks_per_row;
  const int64_t chunk = blk - row * g.chunks_per_row;
  const int kv = (int)(row & 1);
  const int64_t bh = row >> 1;
  const int h = (int)(bh % g.n_heads);
  const int64_t b = bh / g.n_heads;
  const float s = scales[kv * g.n_heads + h];
  const int32_t len = seq_lens[b];
  const int32_t *bt = block_tables + b * g.max_blocks;
  const int64_t page_bytes = 2LL * g.n_heads * g.page_size * g.head_dim;
  const uint8_t *pbase = pool + ((int64_t)kv * g.n_heads + h) * g.page_size * g.head_dim;
  uint16_t *out = (kv ? v_out : k_out) + bh * (int64_t)g.out_len * g.head_dim;
  const int tk_n = GD_THREADS >> g.upt_log2;  // positions per slice
  const int64_t t0 = chunk * (int64_t)(U * tk_n);

  // all block-table entries first (clamped into the table, so the scalar loads are
  // unconditional and issue back to back), then the code loads
  int32_t page[U];
#pragma unroll
  for (int k = 0; k < U; ++k) {
    const int64_t bi = (t0 + k * tk_n) / g.page_size;
    page[k] = bt[bi < g.max_blocks ? bi : g.max_blocks - 1];
  }
  uint2 c[U];
  int32_t e = 0;
#pragma unroll
  for (int k = 0; k < U; ++k) {
    const int64_t tk = t0 + k * tk_n;
    const int64_t rows = min((int64_t)tk_n, (int64_t)len - tk);  // positions with data
    const int64_t bi = tk / g.page_size;
    int nrec = 0;
    const uint8_t *src = pool;
    if (rows > 0) {
      if (bi >= g.max_blocks) {
        e |= ZX_KERR_POS_RANGE;
      } else if (page[k] < 0 || page[k] >= g.n_pages) {
        e |= ZX_KERR_PAGE_RANGE;
      } else {
        src = pbase + page[k] * page_bytes + (tk - bi * g.page_size) * g.head_dim;
        nrec = (int)rows * g.head_dim;
      }
    }
    const v2u_t q = __builtin_amdgcn_raw_buffer_load_b64(gd_rsrc(src, nrec), (int)threadIdx.x * 8, 0, GD_NT);
    c[k] = make_uint2(q.x, q.y);
  }
#pragma unroll
  for (int k = 0; k < U; ++k) {
    const int64_t tk = t0 + k * tk_n;
    const int64_t rows = min((int64_t)tk_n, (int64_t)g.out_len - tk);
    const int nrec = rows > 0 ? (int)rows * g.head_dim * 2 : 0;
    const uint4 o = dequant8(c[k], s);
    const v4u_t w = {o.x, o.y, o.z, o.w};
    __builtin_amdgcn_raw_buffer_store_b128(w, gd_rsrc(rows > 0 ? out + tk * g.head_dim : out, nrec),
                                           (int)threadIdx.x * 16, 0, GD_NT);
  }
  if (e && err && threadIdx.x == 0) atomicOr(err, e);
}

}  // namespace zx

using namespace zx;

extern "C" int zx_kv_gather_dequant(const uint8_t *pool, int64_t n_pages, int32_t n_heads, int32_t head_dim,
                                    int32_t page_size, const float *scales, const int32_t *block_tables,
                                    int32_t max_blocks, const int32_t *seq_lens, int32_t n_seqs,
                                    int32_t out_len, uint16_t *k_out, uint16_t *v_out, int32_t *err,
                                    zx_stream_t stream) {
  clear_error();
  ZX_REQUIRE(pool && scales && block_tables && seq_lens && k_out && v_out,
             "kv_gather_dequant: null pointer");
  ZX_REQUIRE(aligned16(pool) && aligned16(k_out) && aligned16(v_out),
             "kv_gather_dequant: pool, k_out and v_out must be 16-byte aligned");
  ZX_REQUIRE(n_pages > 0 && n_heads > 0 && page_size > 0 && max_blocks > 0 && n_seqs > 0 && out_len >= 0,
             "kv_gather_dequant: sizes must be positive");
  if (!(head_dim == 64 || head_dim == 128 || head_dim == 256))
    return fail(ZX_ERR_UNSUPPORTED, "kv_gather_dequant: head_dim %d not in {64, 128, 256}", head_dim);
  if (out_len == 0) return ZX_OK;
  GatherGeom g;
  g.n_heads = n_heads;
  g.head_dim = head_dim;
  g.page_size = page_size;
  g.max_blocks = max_blocks;
  g.out_len = out_len;
  g.upt_log2 = head_dim == 64 ? 3 : (head_dim == 128 ? 4 : 5);
  g.tt = (GD_THREADS * GD_UNITS) >> g.upt_log2;
  g.chunks_per_row = ceil_div(out_len, g.tt);
  g.n_pages = n_pages;
  const int tk_n = GD_THREADS >> g.upt_log2;
  if (page_size % tk_n == 0) {  // every slice of tk_n positions lies inside one page
    constexpr int U = GS_UNITS;
    g.chunks_per_row = ceil_div(out_len, (int64_t)U * tk_n);
    const int64_t n_blocks = 2LL * n_seqs * n_heads * g.chunks_per_row;
    if (n_blocks >= (1LL << 31)) return fail(ZX_ERR_UNSUPPORTED, "kv_gather_dequant: output too large");
    gather_slices_kernel<U><<<(unsigned)n_blocks, GD_THREADS, 0, as_stream(stream)>>>(
        pool, g, scales, block_tables, seq_lens, k_out, v_out, err);
    return check_launch("gather_slices");
  }
  const int64_t n_blocks = 2LL * n_seqs * n_heads * g.chunks_per_row;
  if (n_blocks >= (1LL << 31)) return fail(ZX_ERR_UNSUPPORTED, "kv_gather_dequant: output too large");
  gather_dequant_kernel<<<(unsigned)n_blocks, GD_THREADS, 0, as_stream(stream)>>>(
      pool, g, scales, block_tables, seq_lens, k_out, v_out, err);
  return check_launch("gather_dequant");
}
