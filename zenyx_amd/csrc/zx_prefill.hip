// zx_prefill.hip -- blocks of queries attending to K/V straight from the paged FP8 pool:
// one ring step of QuantizedRingAttention (README.md:344), with the step's result merged
// into a running (output, log-sum-exp) so that the steps of a ring compose into full
// attention.  The ring exchange itself needs more than one GPU and is not here.
//
// A block owns (sequence, G query heads of one kv head, a tile of 32 * 4 / G query rows);
// its 4 waves each take one head and 32 rows (two 16-row MFMA tiles), so every K/V tile
// is read from HBM once per block and serves 128 query rows.  Steps of 32 keys (two
// 16-key tiles, each inside one page):
//   * the block loads the step's K and V runs with contiguous 16-byte lane loads (whole
//     cache lines), one step ahead of the compute; K codes go to LDS staging rows as
//     they are, V values go transposed into LDS (V^T[channel][key], bf16), both double
//     buffered so one block barrier per step suffices;
//   * each wave: S = Q . K^T on v_mfma_f32_16x16x32_bf16 (Q rows as A, K codes converted
//     to bf16 exactly as B), key range / causal mask, online softmax per row in the exp2
//     domain (rows live in 16-lane groups of the C layout: DPP reductions), P through
//     LDS into the A layout split into bf16 hi + lo, O += P . V on the same MFMA.
// At the end each row is normalised; with MERGE the step's (O, lse2) is combined with
// the running one in o_acc / lse2 (each (row, head) belongs to one block, so no races);
// with the bf16 flag the merged row is also written as bf16.
#include "zx_attn_common.h"

namespace zx {

constexpr int PF_THREADS = 256;
constexpr int PF_KEYS = 32;                  // keys per step
constexpr int PF_KROW = 144;                 // K staging row (128 codes + 16 pad: conflict-free reads)
constexpr int PF_VROW = 80;                  // V^T row (32 keys bf16 + 16 pad)
constexpr int PF_KBYTES = PF_KEYS * PF_KROW;
constexpr int PF_VBYTES = 128 * PF_VROW;
constexpr int PF_PBYTES = 32 * PF_KEYS * 4;  // one wave's P: 32 rows x 32 keys fp32
constexpr int PF_MERGE = 1, PF_WRITE_BF16 = 2, PF_INIT = 4;

struct PrefillArgs {
  const uint16_t *q;  // [n_q][Hq][128] bf16
  const int32_t *cu_q, *q_pos0;
  const uint8_t *pool;
  const float *scales;  // [2][Hkv]
  const int32_t *bt, *kv_begin, *kv_end;
  float *o_acc;   // [n_q][Hq][128] fp32, normalised
  float *lse2;    // [n_q][Hq]
  uint16_t *out;  // [n_q][Hq][128] bf16 (PF_WRITE_BF16)
  int32_t *err;
  int64_t n_pages;
  int32_t n_q_heads, n_kv_heads, page_size, max_blocks, mode, causal;
  uint32_t p_magic;
  int32_t p_shift;
  float sm_log2e;  // sm_scale * log2 e
};

__device__ __forceinline__ uint32_t pf_page_of(const PrefillArgs &a, uint32_t t) {
  return (uint32_t)(((uint64_t)t * a.p_magic) >> (31 + a.p_shift));
}

template <int G>
__global__ void __launch_bounds__(PF_THREADS) paged_prefill_mfma_kernel(PrefillArgs a) {
  constexpr int D = 128;
  constexpr int QT = 32 * 4 / G;  // query rows per block
  const int b = blockIdx.z;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15, kg = lane >> 4;
  const int64_t q_lo = a.cu_q[b];
  const int64_t n_qb = (int64_t)a.cu_q[b + 1] - q_lo;
  const int64_t row0_blk = (int64_t)blockIdx.x * QT;
  if (row0_blk >= n_qb) return;
  const int grp = a.n_q_heads / a.n_kv_heads;
  const int hq = blockIdx.y * G + wave % G;
  const int h = hq / grp;
  const int64_t wrow0 = row0_blk + 32 * (wave / G);  // this wave's first row (in the sequence)
  const int64_t qp0 = a.q_pos0[b];
  const int64_t page_bytes = 2LL * a.n_kv_heads * a.page_size * D;
  const int64_t head_off = (int64_t)h * a.page_size * D;
  const int64_t v_off = (int64_t)a.n_kv_heads * a.page_size * D;
  const int32_t *bt = a.bt + (int64_t)b * a.max_blocks;
  int32_t e = 0;
  int64_t kb = a.kv_begin[b] > 0 ? a.kv_begin[b] : 0;
  int64_t ke = a.kv_end[b];
  if (ke > (int64_t)a.max_blocks * a.page_size) {
    e |= ZX_KERR_POS_RANGE;
    ke = (int64_t)a.max_blocks * a.page_size;
  }
  // keys past the block's last query position never count when causal
  const int64_t last_row = min(row0_blk + QT, n_qb) - 1;
  const int64_t ke_blk = a.causal ? min(ke, qp0 + last_row + 1) : ke;

  __shared__ __attribute__((aligned(16))) uint8_t kst[2][PF_KBYTES];
  __shared__ __attribute__((aligned(16))) uint8_t vtl[2][PF_VBYTES];
  __shared__ __attribute__((aligned(16))) float pls[4][32 * PF_KEYS];
  float *pl = pls[wave];

  // Q rows as the A operand: lane (n, kg) of row tile rt holds row wrow0 + 16 rt + n,
  // channels 32 kg + 8 c ..+8 for MFMA c (the same channel order as the K operand)
  att_bf16x8 qa[2][4];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    const int64_t r = wrow0 + 16 * rt + n;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      att_u32x4 w = {0u, 0u, 0u, 0u};
      if (r < n_qb) {
        const uint4 x =
            *reinterpret_cast<const uint4 *>(a.q + ((q_lo + r) * a.n_q_heads + hq) * D + kg * 32 + c * 8);
        w = att_u32x4{x.x, x.y, x.z, x.w};
      }
      qa[rt][c] = __builtin_bit_cast(att_bf16x8, w);
    }
  }
  const float qs = a.scales[h] * a.sm_log2e;            // K's dequant scale folds into the scores
  const float vscale = a.scales[a.n_kv_heads + h];

  att_f32x4 o[2][8];
  float m[2][4], l[2][4];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
#pragma unroll
    for (int jt = 0; jt < 8; ++jt) o[rt][jt] = att_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      m[rt][i] = -INFINITY;
      l[rt][i] = 0.0f;
    }
  }

  // block-cooperative load of one step: thread t moves 16 bytes of K and of V of key
  // t / 8 (tile (t / 8) / 16), channels 16 (t % 8) ..+16; tiles past the range or on a
  // bad page load through zero-length resources
  const int kk = threadIdx.x >> 3, g8 = threadIdx.x & 7;
  const int64_t s_first = (kb / 16) * 16;
  auto tile_ok = [&](int64_t tp) -> bool {  // uniform
    if (tp >= ke) return false;
    const int64_t page = bt[pf_page_of(a, (uint32_t)tp)];
    return page >= 0 && page < a.n_pages;
  };
  auto load_step = [&](int64_t s0, uint4 &kc, uint4 &vc) {
    const int64_t tp = s0 + (kk & 16);  // this thread's 16-key tile
    const int live = (int)max((int64_t)0, min((int64_t)16, ke - tp));
    const int64_t tc = tp < ke ? tp : (ke > 0 ? ke - 1 : 0);
    const uint32_t bi = pf_page_of(a, (uint32_t)tc);
    const int64_t page = bt[bi];
    const bool ok = live > 0 && page >= 0 && page < a.n_pages;
    e |= (live > 0 && !ok) ? ZX_KERR_PAGE_RANGE : 0;
    const int nrec = ok ? live * D : 0;
    const uint8_t *src = a.pool + (ok ? page * page_bytes + head_off + (tc - (int64_t)bi * a.page_size) * D : 0);
    const __amdgpu_buffer_rsrc_t rk =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(src), (short)0, nrec, 0x00020000);
    const __amdgpu_buffer_rsrc_t rv =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(src + (ok ? v_off : 0)), (short)0, nrec, 0x00020000);
    const int off = (kk & 15) * D + 16 * g8;
    const att_u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 2);
    const att_u32x4 y = __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, 2);
    kc = make_uint4(x.x, x.y, x.z, x.w);
    vc = make_uint4(y.x, y.y, y.z, y.w);
  };
  auto store_step = [&](int buf, const uint4 &kc, const uint4 &vc) {
    *reinterpret_cast<uint4 *>(&kst[buf][kk * PF_KROW + 16 * g8]) = kc;
    // V^T element (channel c, key k) at c * PF_VROW + 16 ((k / 8) ^ (c / 32)) + 2 (k % 8);
    // this thread's channels c = 16 g8 + 2 p, +1, so c / 32 = g8 / 2
    uint32_t vb[8];
    decode16_bf16(vc, vb);
    const int base = (((kk >> 3) ^ (g8 >> 1)) << 4) + (kk & 7) * 2;
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      uint8_t *row = &vtl[buf][(16 * g8 + 2 * p) * PF_VROW + base];
      *reinterpret_cast<uint16_t *>(row) = (uint16_t)(vb[p] & 0xFFFFu);
      *reinterpret_cast<uint16_t *>(row + PF_VROW) = (uint16_t)(vb[p] >> 16);
    }
  };

  auto compute_step = [&](int buf, int64_t s0) {
    const bool ok0 = tile_ok(s0), ok1 = tile_ok(s0 + 16);
    // scores for both key tiles and both row tiles
    att_f32x4 sc[2][2];
#pragma unroll
    for (int KT = 0; KT < 2; ++KT) {
      uint32_t kbv[16];
      uint32_t (&k0)[8] = *reinterpret_cast<uint32_t (*)[8]>(&kbv[0]);
      uint32_t (&k1)[8] = *reinterpret_cast<uint32_t (*)[8]>(&kbv[8]);
      const uint8_t *kr = &kst[buf][(16 * KT + n) * PF_KROW + kg * 32];
      decode16_bf16(*reinterpret_cast<const uint4 *>(kr), k0);
      decode16_bf16(*reinterpret_cast<const uint4 *>(kr + 16), k1);
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        att_f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int c = 0; c < 4; ++c)
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              qa[rt][c],
              __builtin_bit_cast(att_bf16x8, att_u32x4{kbv[4 * c], kbv[4 * c + 1], kbv[4 * c + 2], kbv[4 * c + 3]}),
              acc, 0, 0, 0);
        sc[rt][KT] = acc;
      }
    }
    // C layout: lane holds rows 16 rt + 4 kg + i, key 16 KT + n
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      float sv[2][4];
#pragma unroll
      for (int KT = 0; KT < 2; ++KT) {
        const int64_t kp = s0 + 16 * KT + n;
        const bool tok = KT == 0 ? ok0 : ok1;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int64_t r = wrow0 + 16 * rt + 4 * kg + i;
          const bool valid = tok && kp >= kb && kp < ke && r < n_qb && (!a.causal || kp <= qp0 + r);
          sv[KT][i] = valid ? sc[rt][KT][i] * qs : -INFINITY;
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float mx = row16_max(fmaxf(sv[0][i], sv[1][i]));
        const float mn = fmaxf(m[rt][i], mx);
        const float alpha = mn == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m[rt][i] - mn);
        m[rt][i] = mn;
        l[rt][i] *= alpha;
#pragma unroll
        for (int jt = 0; jt < 8; ++jt) o[rt][jt][i] *= alpha;
#pragma unroll
        for (int KT = 0; KT < 2; ++KT) {
          const float p = mn == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(sv[KT][i] - mn);
          l[rt][i] += p;
          pl[(16 * rt + 4 * kg + i) * PF_KEYS + 16 * KT + n] = p;
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // A operand: P[row 16 rt + n][keys 8 kg ..+8], split into bf16 hi + lo
    att_bf16x8 ah[2], al[2];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      const float4 x = *reinterpret_cast<const float4 *>(pl + (16 * rt + n) * PF_KEYS + kg * 8);
      const float4 y = *reinterpret_cast<const float4 *>(pl + (16 * rt + n) * PF_KEYS + kg * 8 + 4);
      const float pr[8] = {x.x, x.y, x.z, x.w, y.x, y.y, y.z, y.w};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        ah[rt][i] = (__bf16)pr[i];
        al[rt][i] = (__bf16)(pr[i] - (float)ah[rt][i]);
      }
    }
    // B operand per 16-channel tile: V^T[channel 16 jt + n][keys 8 kg ..+8]
#pragma unroll
    for (int jt = 0; jt < 8; ++jt) {
      const int ch = 16 * jt + n;
      const att_u32x4 w = *reinterpret_cast<const att_u32x4 *>(&vtl[buf][ch * PF_VROW + ((kg ^ (ch >> 5)) << 4)]);
      const att_bf16x8 bv = __builtin_bit_cast(att_bf16x8, w);
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        o[rt][jt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[rt], bv, o[rt][jt], 0, 0, 0);
        o[rt][jt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[rt], bv, o[rt][jt], 0, 0, 0);
      }
    }
  };

  // steps: data of step s + 1 loaded into registers while step s computes; one barrier
  // per step (the LDS buffers alternate)
  uint4 kc, vc;
  int64_t s0 = s_first;
  if (s0 < ke_blk) {
    load_step(s0, kc, vc);
    store_step(0, kc, vc);
  }
  __syncthreads();
  int buf = 0;
  while (s0 < ke_blk) {
    const int64_t s1 = s0 + PF_KEYS;
    const bool more = s1 < ke_blk;  // uniform
    if (more) load_step(s1, kc, vc);
    compute_step(buf, s0);
    if (more) store_step(buf ^ 1, kc, vc);
    __syncthreads();
    buf ^= 1;
    s0 = s1;
  }

  // rows: l over the 16 lanes of the row group; normalise; merge; store
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t r = wrow0 + 16 * rt + 4 * kg + i;
      const float lt = group_sum<16>(l[rt][i]);
      if (r >= n_qb) continue;
      const float lse_new = lt > 0.0f ? m[rt][i] + __builtin_amdgcn_logf(lt) : -INFINITY;
      const float inv = lt > 0.0f ? vscale / lt : 0.0f;  // V's dequant scale applied once, here
      const int64_t row = (q_lo + r) * a.n_q_heads + hq;
      float wa = 0.0f, wb = 1.0f, lse = lse_new;
      if ((a.mode & PF_MERGE) && !(a.mode & PF_INIT)) {
        const float lse_old = a.lse2[row];
        const float mm = fmaxf(lse_old, lse_new);
        if (mm == -INFINITY) {
          wa = 0.0f;
          wb = 0.0f;
          lse = -INFINITY;
        } else {
          const float ea = __builtin_amdgcn_exp2f(lse_old - mm), eb = __builtin_amdgcn_exp2f(lse_new - mm);
          const float den = ea + eb;
          wa = ea / den;
          wb = eb / den;
          lse = mm + __builtin_amdgcn_logf(den);
        }
      }
#pragma unroll
      for (int jt = 0; jt < 8; ++jt) {
        const int64_t idx = row * D + 16 * jt + n;
        float v = o[rt][jt][i] * inv * wb;
        if (wa != 0.0f) v += wa * a.o_acc[idx];
        if (a.mode & PF_MERGE) a.o_acc[idx] = v;
        if (a.mode & PF_WRITE_BF16) a.out[idx] = (uint16_t)(pack_bf16(v, 0.0f) & 0xFFFFu);
      }
      if ((a.mode & PF_MERGE) && n == 0) a.lse2[row] = lse;
    }
  if (e && a.err) atomicOr(a.err, e);
}

}  // namespace zx

using namespace zx;

extern "C" int zx_paged_attention_prefill(const uint16_t *q, int64_t n_q, const int32_t *cu_q, const int32_t *q_pos0,
                                          int32_t n_q_heads, const uint8_t *pool, int64_t n_pages, int32_t n_kv_heads,
                                          int32_t head_dim, int32_t page_size, const float *scales,
                                          const int32_t *block_tables, int32_t max_blocks, const int32_t *kv_begin,
                                          const int32_t *kv_end, int32_t n_seqs, int32_t max_q_per_seq,
                                          int32_t causal, float sm_scale, int32_t flags, float *o_acc, float *lse2,
                                          uint16_t *out, int32_t *err, zx_stream_t stream) {
  clear_error();
  ZX_REQUIRE(q && cu_q && q_pos0 && pool && scales && block_tables && kv_begin && kv_end,
             "paged_attention_prefill: null pointer");
  ZX_REQUIRE(n_q >= 0 && n_q_heads > 0 && n_kv_heads > 0 && n_pages > 0 && page_size > 0 && max_blocks > 0 &&
                 n_seqs > 0 && max_q_per_seq >= 0,
             "paged_attention_prefill: sizes must be positive");
  ZX_REQUIRE(n_q_heads % n_kv_heads == 0, "paged_attention_prefill: n_q_heads must be a multiple of n_kv_heads");
  ZX_REQUIRE((flags & ~(ZX_PREFILL_MERGE | ZX_PREFILL_INIT | ZX_PREFILL_BF16)) == 0,
             "paged_attention_prefill: unknown flags");
  ZX_REQUIRE(!(flags & ZX_PREFILL_MERGE) || (o_acc && lse2), "paged_attention_prefill: merging needs o_acc and lse2");
  ZX_REQUIRE(!(flags & ZX_PREFILL_BF16) || out, "paged_attention_prefill: bf16 output requested without out");
  ZX_REQUIRE(flags & (ZX_PREFILL_MERGE | ZX_PREFILL_BF16), "paged_attention_prefill: nothing to write");
  if (head_dim != 128 || page_size % 16)
    return fail(ZX_ERR_UNSUPPORTED, "paged_attention_prefill: needs head_dim 128 and pages of a multiple of 16 tokens "
                                    "(got %d, %d)", head_dim, page_size);
  if (n_q == 0 || max_q_per_seq == 0) return ZX_OK;
  if ((int64_t)max_blocks * page_size >= (1LL << 31))
    return fail(ZX_ERR_UNSUPPORTED, "paged_attention_prefill: sequences too long");
  const int grp = n_q_heads / n_kv_heads;
  const int G = grp % 4 == 0 ? 4 : (grp % 2 == 0 ? 2 : 1);
  PrefillArgs a;
  a.q = q;
  a.cu_q = cu_q;
  a.q_pos0 = q_pos0;
  a.pool = pool;
  a.scales = scales;
  a.bt = block_tables;
  a.kv_begin = kv_begin;
  a.kv_end = kv_end;
  a.o_acc = o_acc;
  a.lse2 = lse2;
  a.out = out;
  a.err = err;
  a.n_pages = n_pages;
  a.n_q_heads = n_q_heads;
  a.n_kv_heads = n_kv_heads;
  a.page_size = page_size;
  a.max_blocks = max_blocks;
  a.mode = ((flags & ZX_PREFILL_MERGE) ? PF_MERGE : 0) | ((flags & ZX_PREFILL_INIT) ? PF_INIT : 0) |
           ((flags & ZX_PREFILL_BF16) ? PF_WRITE_BF16 : 0);
  a.causal = causal ? 1 : 0;
  a.sm_log2e = sm_scale * ATT_LOG2E;
  {  // t / page_size = (t * magic) >> (31 + shift) for t < 2^31
    int shift = 0;
    while ((1LL << shift) < page_size) ++shift;
    a.p_shift = shift;
    a.p_magic = (uint32_t)(((1ULL << (31 + shift)) + page_size - 1) / page_size);
  }
  const int QT = 32 * 4 / G;
  const dim3 grid((unsigned)ceil_div(max_q_per_seq, QT), (unsigned)(n_q_heads / G), (unsigned)n_seqs);
  ZX_REQUIRE(grid.x < (1u << 31) && n_seqs <= 65535, "paged_attention_prefill: too many query tiles or sequences");
  hipStream_t st = as_stream(stream);
  switch (G) {
    case 4: paged_prefill_mfma_kernel<4><<<grid, PF_THREADS, 0, st>>>(a); break;
    case 2: paged_prefill_mfma_kernel<2><<<grid, PF_THREADS, 0, st>>>(a); break;
    default: paged_prefill_mfma_kernel<1><<<grid, PF_THREADS, 0, st>>>(a); break;
  }
  return check_launch("paged_prefill_mfma");
}
