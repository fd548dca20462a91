// zx_attention.hip -- decode attention straight from the paged FP8 pool.
//
// One query token per sequence attends to its K/V pages without materialising bf16 K/V
// (the attention that consumes FP8 pages directly, QuantizedRingAttention README.md:344):
//   s_t = sm_scale * q . K_t,  K_t = decode(code) * scale_k     (t < seq_len)
//   out = sum_t softmax(s)_t V_t,  V_t = decode(code) * scale_v
// HBM traffic is 1 B per K/V element (the gather + dequant path moves 3 B and then the
// attention reads 2 B more).
//
// Split-K flash decoding.  Pass 1 (paged_decode_partial_kernel): a block owns one
// (sequence, kv head, group of G query heads, split of positions); lane l of a
// wave owns 16 channels (dc = l % LPT, LPT = D / 16 lanes per token) of token slot
// l / LPT, so K and V rows are read as 16-byte loads that cover whole page rows.  Scale
// factors fold into q (q * scale_k * sm_scale * log2 e) and into the end (scale_v), so
// the inner loop works on decoded codes.  Each wave keeps an online softmax (running max
// m, sum l, accumulator acc[G][16] per lane, exp2 domain) over steps of ATT_U passes;
// at the end the token slots and the block's 4 waves are combined and the partial
// (m, l, acc[D]) per query head is written to the workspace.  Pass 2
// (paged_decode_combine_kernel) merges the splits of a (sequence, query head) and writes
// bf16.
#include "zx_attn_common.h"

namespace zx {

constexpr int ATT_THREADS = 256;  // 4 waves
constexpr int ATT_WAVES = ATT_THREADS / 64;
constexpr int ATT_U = 4;          // passes per online-softmax step
constexpr int ATT_SPLIT_MIN = 1024;  // positions per block: a multiple of this, chosen per call

struct AttnGeom {
  int32_t n_q_heads, n_kv_heads, head_dim, page_size, max_blocks, n_seqs;
  int32_t n_splits, split_len;  // blocks per (sequence, head group), positions per block
  uint32_t p_magic;  // t / page_size = (t * p_magic) >> (31 + p_shift) for t < 2^31
  int32_t p_shift;
  int64_t n_pages;
  float sm_scale;
};

__device__ __forceinline__ uint32_t page_of(const AttnGeom &g, uint32_t t) {
  return (uint32_t)(((uint64_t)t * g.p_magic) >> (31 + g.p_shift));
}

// 16 e4m3 codes -> 16 fp32 values (exact).
__device__ __forceinline__ void decode16(uint4 c, float (&f)[16]) {
  e4m3x4_decode(c.x, f[0], f[1], f[2], f[3]);
  e4m3x4_decode(c.y, f[4], f[5], f[6], f[7]);
  e4m3x4_decode(c.z, f[8], f[9], f[10], f[11]);
  e4m3x4_decode(c.w, f[12], f[13], f[14], f[15]);
}

// Across 16-lane rows: the lane 16 and 32 positions away (ds_bpermute).  (The
// v_permlane16/32_swap builtins return one of their two outputs twice with this
// compiler, so they are not used.)
__device__ __forceinline__ float rows_sum(float v) {
  v += __shfl_xor(v, 16, 64);
  return v + __shfl_xor(v, 32, 64);
}
__device__ __forceinline__ float rows_max(float v) {
  v = fmaxf(v, __shfl_xor(v, 16, 64));
  return fmaxf(v, __shfl_xor(v, 32, 64));
}
// Max / sum over the token slots of a wave for each channel group: lanes l, l + LPT,
// l + 2 LPT, ... (row_ror by 4 and 8 inside a 16-lane row keeps l % LPT, then the row
// pairs).
template <int LPT> __device__ __forceinline__ float slots_max(float v) {
  if (LPT <= 4) v = fmaxf(v, dpp<0x124>(v));  // row_ror:4
  if (LPT <= 8) v = fmaxf(v, dpp<0x128>(v));  // row_ror:8
  return rows_max(v);
}
template <int LPT> __device__ __forceinline__ float slots_sum(float v) {
  if (LPT <= 4) v += dpp<0x124>(v);
  if (LPT <= 8) v += dpp<0x128>(v);
  return rows_sum(v);
}

// Partial layout in the workspace: [B][Hq][n_splits][2 + D] fp32 = (m, l, acc[D]) with m
// in the exp2 domain; a split without valid positions writes m = -inf, l = 0, acc = 0.
template <int G, int D, bool FAST>
__global__ void __launch_bounds__(ATT_THREADS)
paged_decode_partial_kernel(const uint16_t *__restrict__ q, AttnGeom g, const uint8_t *__restrict__ pool,
                            const float *__restrict__ scales, const int32_t *__restrict__ block_tables,
                            const int32_t *__restrict__ seq_lens, float *__restrict__ part, int32_t *err) {
  constexpr int LPT = D / 16;   // lanes per token
  constexpr int TPW = 64 / LPT;  // token slots per wave pass
  constexpr int STEP = ATT_U * TPW;
  const int split = blockIdx.x;
  const int grp_blocks = g.n_q_heads / g.n_kv_heads / G;  // query-head groups per kv head
  const int h = blockIdx.y / grp_blocks;
  const int hq0 = h * (g.n_q_heads / g.n_kv_heads) + (blockIdx.y % grp_blocks) * G;
  const int b = blockIdx.z;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: scalar addressing
  const int ts = lane / LPT, dc = lane % LPT;
  const int32_t len = seq_lens[b];
  const int64_t t_begin = (int64_t)split * g.split_len;
  const int64_t t_end = min(min((int64_t)len, (int64_t)g.max_blocks * g.page_size), t_begin + g.split_len);
  const int64_t page_bytes = 2LL * g.n_kv_heads * g.page_size * D;
  const uint8_t *kbase = pool + (int64_t)h * g.page_size * D + dc * 16;
  const int64_t v_off = (int64_t)g.n_kv_heads * g.page_size * D;
  const int32_t *bt = block_tables + (int64_t)b * g.max_blocks;

  // q as bf16 pairs for this lane's 16 channels; the score scale (scale_k * sm_scale *
  // log2 e) multiplies the reduced dot product
  uint32_t qb[G][8];
#pragma unroll
  for (int j = 0; j < G; ++j) {
    const uint4 *qp = reinterpret_cast<const uint4 *>(q + ((int64_t)b * g.n_q_heads + hq0 + j) * D + dc * 16);
    const uint4 a = qp[0], c = qp[1];
    qb[j][0] = a.x; qb[j][1] = a.y; qb[j][2] = a.z; qb[j][3] = a.w;
    qb[j][4] = c.x; qb[j][5] = c.y; qb[j][6] = c.z; qb[j][7] = c.w;
  }
  const float qs = scales[h] * g.sm_scale * ATT_LOG2E;

  float m[G], l[G], acc[G][16];
#pragma unroll
  for (int j = 0; j < G; ++j) {
    m[j] = -INFINITY;
    l[j] = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[j][i] = 0.0f;
  }
  // positions past the block table are not attended to, and flagged once per sequence
  int32_t e = split == 0 && threadIdx.x == 0 && blockIdx.y == 0 && (int64_t)len > (int64_t)g.max_blocks * g.page_size
                  ? ZX_KERR_POS_RANGE : 0;

  // K/V of one step (ATT_U passes of TPW positions) into registers.  FAST (page size a
  // multiple of TPW): the TPW positions of a pass share one page, so the page id is a
  // scalar load and the loads go through a resource whose num_records ends at the last
  // valid row; otherwise every lane looks its page up.  ok marks positions with data.
  auto load_step = [&](int64_t t0, uint4 (&kc)[ATT_U], uint4 (&vc)[ATT_U], bool (&ok)[ATT_U]) {
#pragma unroll
    for (int u = 0; u < ATT_U; ++u) {
      if constexpr (FAST) {
        const int64_t tp = t0 + u * TPW;  // uniform
        const int64_t rows = min((int64_t)TPW, t_end - tp);
        int nrec = 0;
        const uint8_t *src = pool;
        if (rows > 0) {
          const uint32_t bi = page_of(g, (uint32_t)tp);
          const int64_t page = bt[bi];
          if (page < 0 || page >= g.n_pages) e |= ZX_KERR_PAGE_RANGE;
          else {
            src = pool + page * page_bytes + (int64_t)h * g.page_size * D + (tp - (int64_t)bi * g.page_size) * D;
            nrec = (int)rows * D;
          }
        }
        const __amdgpu_buffer_rsrc_t rk =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(src), (short)0, nrec, 0x00020000);
        const __amdgpu_buffer_rsrc_t rv =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(src + (nrec ? v_off : 0)), (short)0, nrec, 0x00020000);
        typedef unsigned int v4u __attribute__((ext_vector_type(4)));
        const v4u a = __builtin_amdgcn_raw_buffer_load_b128(rk, ts * D + dc * 16, 0, 2);
        const v4u c = __builtin_amdgcn_raw_buffer_load_b128(rv, ts * D + dc * 16, 0, 2);
        kc[u] = make_uint4(a.x, a.y, a.z, a.w);
        vc[u] = make_uint4(c.x, c.y, c.z, c.w);
        ok[u] = ts * D < nrec;
      } else {
        const int64_t t = t0 + u * TPW + ts;
        int64_t off = -1;
        if (t < t_end) {
          const uint32_t bi = page_of(g, (uint32_t)t);
          const int64_t page = bt[bi];
          if (page < 0 || page >= g.n_pages) e |= ZX_KERR_PAGE_RANGE;
          else off = page * page_bytes + (t - (int64_t)bi * g.page_size) * D;
        }
        ok[u] = off >= 0;
        const uint8_t *kp = kbase + (off >= 0 ? off : 0);
        kc[u] = ok[u] ? *reinterpret_cast<const uint4 *>(kp) : make_uint4(0, 0, 0, 0);
        vc[u] = ok[u] ? *reinterpret_cast<const uint4 *>(kp + v_off) : make_uint4(0, 0, 0, 0);
      }
    }
  };

  auto compute_step = [&](const uint4 (&kc)[ATT_U], const uint4 (&vc)[ATT_U], const bool (&ok)[ATT_U]) {
    float s[ATT_U][G];
#pragma unroll
    for (int u = 0; u < ATT_U; ++u) {
      uint32_t kb[8];
      decode16_bf16(kc[u], kb);
#pragma unroll
      for (int j = 0; j < G; ++j) {
        float a = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i)
          a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(att_bf2, qb[j][i]), __builtin_bit_cast(att_bf2, kb[i]),
                                              a, false);
        a = group_sum<LPT>(a);
        s[u][j] = ok[u] ? a * qs : -INFINITY;
      }
    }
    // running max per head (the same in every lane); the accumulators are rescaled only
    // on the steps where some head's max grew (a scalar branch: rare after the first
    // steps of a split)
    float m_new[G];
    bool grew = false;
#pragma unroll
    for (int j = 0; j < G; ++j) {
      float mx = s[0][j];
#pragma unroll
      for (int u = 1; u < ATT_U; ++u) mx = fmaxf(mx, s[u][j]);
      mx = slots_max<LPT>(mx);
      m_new[j] = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, fmaxf(m[j], mx))));
      grew = grew || m_new[j] > m[j];
    }
    if (grew) {
#pragma unroll
      for (int j = 0; j < G; ++j) {
        const float alpha = m_new[j] == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m[j] - m_new[j]);
        m[j] = m_new[j];
        l[j] *= alpha;
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[j][i] *= alpha;
      }
    }
#pragma unroll
    for (int j = 0; j < G; ++j) {
#pragma unroll
      for (int u = 0; u < ATT_U; ++u) s[u][j] = m[j] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(s[u][j] - m[j]);
    }
#pragma unroll
    for (int u = 0; u < ATT_U; ++u) {
      float v[16];
      decode16(vc[u], v);
#pragma unroll
      for (int j = 0; j < G; ++j) {
        l[j] += s[u][j];
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[j][i] = __builtin_fmaf(s[u][j], v[i], acc[j][i]);
      }
    }
  };

  // wave w takes steps w, w + 4, ...; the next step's loads are issued before the
  // current step is computed
  const int64_t stride = (int64_t)ATT_WAVES * STEP;
  int64_t t0 = t_begin + (int64_t)wave * STEP;
  uint4 ka[ATT_U], va[ATT_U], kb2[ATT_U], vb2[ATT_U];
  bool oka[ATT_U], okb[ATT_U];
  if (t0 < t_end) load_step(t0, ka, va, oka);
  while (t0 < t_end) {
    if (t0 + stride < t_end) load_step(t0 + stride, kb2, vb2, okb);
    compute_step(ka, va, oka);
    t0 += stride;
    if (t0 >= t_end) break;
    if (t0 + stride < t_end) load_step(t0 + stride, ka, va, oka);
    compute_step(kb2, vb2, okb);
    t0 += stride;
  }

  // token slots of the wave -> one value per (head, channel) in every lane of slot 0
#pragma unroll
  for (int j = 0; j < G; ++j) {
    l[j] = slots_sum<LPT>(l[j]);
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[j][i] = slots_sum<LPT>(acc[j][i]);
  }
  // combine the block's waves through LDS
  __shared__ float sm_m[ATT_WAVES][G], sm_l[ATT_WAVES][G];
  __shared__ float sm_acc[ATT_WAVES][G][D];
  if (ts == 0) {
#pragma unroll
    for (int j = 0; j < G; ++j) {
#pragma unroll
      for (int i = 0; i < 16; ++i) sm_acc[wave][j][dc * 16 + i] = acc[j][i];
      if (dc == 0) {
        sm_m[wave][j] = m[j];
        sm_l[wave][j] = l[j];
      }
    }
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < G * D; idx += ATT_THREADS) {
    const int j = idx / D, d = idx % D;
    float M = sm_m[0][j];
#pragma unroll
    for (int w = 1; w < ATT_WAVES; ++w) M = fmaxf(M, sm_m[w][j]);
    float a = 0.0f, ll = 0.0f;
#pragma unroll
    for (int w = 0; w < ATT_WAVES; ++w) {
      const float f = M == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(sm_m[w][j] - M);
      a += f * sm_acc[w][j][d];
      ll += f * sm_l[w][j];
    }
    float *pp = part + (((int64_t)b * g.n_q_heads + hq0 + j) * g.n_splits + split) * (2 + D);
    pp[2 + d] = a;
    if (d == 0) {
      pp[0] = M;
      pp[1] = ll;
    }
  }
  if (e && err) atomicOr(err, e);
}

// Matrix-core variant of pass 1 for D = 128 and page sizes that are a multiple of 16:
// q.K^T and P.V run on v_mfma_f32_16x16x32_bf16 with the (up to 4) query heads of the
// block as the M rows (padded to 16).  A wave takes steps of 32 positions (two 16-token
// tiles, each inside one page).  The K and V codes of a tile arrive as two contiguous
// 1 KiB loads per run (lane l: token 8 i + l / 8, channels 16 (l % 8) ..+16: whole cache
// lines per instruction) and are rearranged on chip:
//   * K codes go through a staging area (144-byte token rows) and come back as lane
//     (n, kg) = token n, channels 32 kg ..+32, converted to bf16 exactly: the B operand
//     of q.K^T (k = channel; any channel permutation shared with q's A operand works,
//     since the product sums over channels);
//   * V values go into LDS as bf16 token rows (288-byte rows: the four rows a 16-lane
//     group reads fall on distinct banks) with two 16-byte stores per load, and the B
//     operand of P.V (8 consecutive tokens of one channel per lane) comes back through
//     gfx950's transposing LDS read, ds_read_b64_tr_b16 (2% faster than storing V^T with
//     64 two-byte stores per lane and step).
// P goes through LDS as fp32 into the A-operand layout and is split into bf16 hi + lo
// (two MFMAs), which keeps the products at ~2^-17 relative error.  Scores land in the C
// layout: lanes 0-15 hold heads 0-3 of token l % 16, so the softmax bookkeeping is a
// 16-lane DPP reduction; the O accumulators (8 tiles of 16 channels) live in MFMA
// results, rows = heads.
constexpr int AM_VTROW = 288;               // bytes per token row of V (256 + 32 pad)
constexpr int AM_VBYTES = 32 * AM_VTROW;    // one wave's V (32 tokens)
typedef short att_i16x4 __attribute__((ext_vector_type(4)));
constexpr int AM_PBYTES = 4 * 32 * 4;       // one wave's P (4 heads x 32 tokens fp32)
constexpr int AM_KROW = 144;                // bytes per token row of the K staging (128 + 16 pad)
constexpr int AM_KBYTES = 32 * AM_KROW;     // one wave's K codes (32 tokens)


template <int G>
__global__ void __launch_bounds__(ATT_THREADS, 2)
paged_decode_mfma_kernel(const uint16_t *__restrict__ q, AttnGeom g, const uint8_t *__restrict__ pool,
                         const float *__restrict__ scales, const int32_t *__restrict__ block_tables,
                         const int32_t *__restrict__ seq_lens, float *__restrict__ part, int32_t *err) {
  constexpr int D = 128;
  const int split = blockIdx.x;
  const int grp_blocks = g.n_q_heads / g.n_kv_heads / G;
  const int h = blockIdx.y / grp_blocks;
  const int hq0 = h * (g.n_q_heads / g.n_kv_heads) + (blockIdx.y % grp_blocks) * G;
  const int b = blockIdx.z;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15, kg = lane >> 4;  // MFMA column / k-group
  const int32_t len = seq_lens[b];
  const int64_t t_begin = (int64_t)split * g.split_len;
  const int64_t t_end = min(min((int64_t)len, (int64_t)g.max_blocks * g.page_size), t_begin + g.split_len);
  const int64_t page_bytes = 2LL * g.n_kv_heads * g.page_size * D;
  const int64_t head_off = (int64_t)h * g.page_size * D;
  const int64_t v_off = (int64_t)g.n_kv_heads * g.page_size * D;
  const int32_t *bt = block_tables + (int64_t)b * g.max_blocks;
  __shared__ __attribute__((aligned(16))) uint8_t lds[ATT_WAVES][AM_VBYTES + AM_PBYTES + AM_KBYTES];
  uint8_t *vt = lds[wave];
  float *pl = reinterpret_cast<float *>(lds[wave] + AM_VBYTES);
  uint8_t *ks = lds[wave] + AM_VBYTES + AM_PBYTES;

  // q rows (heads) as the A operand: lane l holds head n, channels 32 kg + 8 c .. +8
  att_bf16x8 qa[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    att_u32x4 w = {0u, 0u, 0u, 0u};
    if (n < G) {
      const uint4 x = *reinterpret_cast<const uint4 *>(q + ((int64_t)b * g.n_q_heads + hq0 + n) * D + kg * 32 + c * 8);
      w = att_u32x4{x.x, x.y, x.z, x.w};
    }
    qa[c] = __builtin_bit_cast(att_bf16x8, w);
  }
  const float qs = scales[h] * g.sm_scale * ATT_LOG2E;

  att_f32x4 o[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) o[t] = att_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float m[4], l[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    m[j] = -INFINITY;
    l[j] = 0.0f;
  }
  int32_t e = split == 0 && threadIdx.x == 0 && blockIdx.y == 0 && (int64_t)len > (int64_t)g.max_blocks * g.page_size
                  ? ZX_KERR_POS_RANGE : 0;

  // one 16-token tile: K and V codes of token tp + n, channels 32 kg ..+32; rows = valid tokens.
  // Branch-free: the block-table entry is read for a position clamped into the split
  // (always a valid index), validity is a select, and a tile past the end or on a bad
  // page loads through resources with num_records = 0 (zeros, no memory traffic).  Every
  // step therefore issues the same loads, so the compiler's s_waitcnt counts only wait
  // for the step being computed and the next step's loads stay in flight.
  const int64_t t_last = t_end > t_begin ? t_end - 1 : t_begin;
  // page id of the tile at tp (position clamped into the split: always a valid index)
  auto tile_page = [&](int64_t tp) -> int64_t {
    const int64_t tc = tp < t_last ? tp : t_last;
    return bt[page_of(g, (uint32_t)tc)];
  };
  auto load_tile = [&](int64_t tp, int64_t page, uint4 (&kc)[2], uint4 (&vc)[2], int &rows) {
    const int live = (int)max((int64_t)0, min((int64_t)16, t_end - tp));
    const int64_t tc = tp < t_last ? tp : t_last;
    const uint32_t bi = page_of(g, (uint32_t)tc);
    const bool ok = page >= 0 && page < g.n_pages;
    e |= (live > 0 && !ok) ? ZX_KERR_PAGE_RANGE : 0;
    rows = ok ? live : 0;
    const int nrec = rows * D;
    const uint8_t *src = pool + (ok ? page * page_bytes + head_off + (tc - (int64_t)bi * g.page_size) * D : 0);
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(src), (short)0, nrec,
                                                                        0x00020000);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(src + (ok ? v_off : 0)), (short)0, nrec, 0x00020000);
    // contiguous: load i gives lane l the 16 codes of token 8 i + l / 8, channels
    // 16 (l % 8) ..+16, so one instruction reads 1 KiB of whole cache lines (the mapping
    // that gives each lane its MFMA operand directly touches half lines and was ~20%
    // slower on the same bytes); the operand layout is made on chip
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const att_u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(rk, 16 * lane + 1024 * i, 0, 2);
      const att_u32x4 c = __builtin_amdgcn_raw_buffer_load_b128(rv, 16 * lane + 1024 * i, 0, 2);
      kc[i] = make_uint4(a.x, a.y, a.z, a.w);
      vc[i] = make_uint4(c.x, c.y, c.z, c.w);
    }
  };

  auto compute_step = [&](const uint4 (&kc)[2][2], const uint4 (&vc)[2][2], const int (&rows)[2]) {
    // K codes through the staging rows: written as loaded, read back as lane (n, kg) =
    // token n, channels 32 kg ..+32 (144-byte rows: the 16 rows of a read hit distinct banks)
#pragma unroll
    for (int T = 0; T < 2; ++T)
#pragma unroll
      for (int i = 0; i < 2; ++i)
        *reinterpret_cast<uint4 *>(ks + (T * 16 + 8 * i + (lane >> 3)) * AM_KROW + 16 * (lane & 7)) = kc[T][i];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // scores: S[head][token] for both tiles
    float sv[2][4];
#pragma unroll
    for (int T = 0; T < 2; ++T) {
      uint32_t kb[16];
      uint32_t (&k0)[8] = *reinterpret_cast<uint32_t (*)[8]>(&kb[0]);
      uint32_t (&k1)[8] = *reinterpret_cast<uint32_t (*)[8]>(&kb[8]);
      const uint8_t *kr = ks + (T * 16 + n) * AM_KROW + kg * 32;
      decode16_bf16(*reinterpret_cast<const uint4 *>(kr), k0);
      decode16_bf16(*reinterpret_cast<const uint4 *>(kr + 16), k1);
      att_f32x4 sc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int c = 0; c < 4; ++c)
        sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            qa[c], __builtin_bit_cast(att_bf16x8, att_u32x4{kb[4 * c], kb[4 * c + 1], kb[4 * c + 2], kb[4 * c + 3]}),
            sc, 0, 0, 0);
#pragma unroll
      for (int j = 0; j < 4; ++j) sv[T][j] = (kg == 0 && j < G && n < rows[T]) ? sc[j] * qs : -INFINITY;
    }
    float m_new[4];
    bool grew = false;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float mx = row16_max(fmaxf(sv[0][j], sv[1][j]));
      m_new[j] = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, fmaxf(m[j], mx))));
      grew = grew || m_new[j] > m[j];
    }
    if (grew) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float alpha = m_new[j] == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m[j] - m_new[j]);
        m[j] = m_new[j];
        l[j] *= alpha;
#pragma unroll
        for (int t = 0; t < 8; ++t) o[t][j] *= alpha;
      }
    }
    // P (fp32) into LDS as [head][token]
#pragma unroll
    for (int T = 0; T < 2; ++T)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float p = m[j] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(sv[T][j] - m[j]);
        l[j] += p;
        if (kg == 0) pl[j * 32 + T * 16 + n] = p;
      }
    // V into LDS as token rows (AM_VTROW bytes, channels in order, bf16): load i of tile T
    // gave lane l token t = 16 T + 8 i + l / 8, channels 16 (l % 8) ..+16: 32 bytes
#pragma unroll
    for (int T = 0; T < 2; ++T)
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        uint32_t vb[8];
        decode16_bf16(vc[T][i], vb);
        const int t = T * 16 + 8 * i + (lane >> 3);
        uint4 *row = reinterpret_cast<uint4 *>(vt + t * AM_VTROW + 32 * (lane & 7));
        row[0] = make_uint4(vb[0], vb[1], vb[2], vb[3]);
        row[1] = make_uint4(vb[4], vb[5], vb[6], vb[7]);
      }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // A operand: P[head n][tokens 8 kg ..+8], split into bf16 hi + lo
    att_bf16x8 ah, al;
    {
      float pr[8];
      if (n < G) {
        const float4 a = *reinterpret_cast<const float4 *>(pl + n * 32 + kg * 8);
        const float4 c = *reinterpret_cast<const float4 *>(pl + n * 32 + kg * 8 + 4);
        pr[0] = a.x; pr[1] = a.y; pr[2] = a.z; pr[3] = a.w; pr[4] = c.x; pr[5] = c.y; pr[6] = c.z; pr[7] = c.w;
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) pr[i] = 0.0f;
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        ah[i] = (__bf16)pr[i];
        al[i] = (__bf16)(pr[i] - (float)ah[i]);
      }
    }
    // B operand per 16-channel tile: V^T[channel 16 jt + n][tokens 8 kg ..+8]
#pragma unroll
    for (int jt = 0; jt < 8; ++jt) {
      // two transposing reads (ds_read_b64_tr_b16): within each 16-lane group kg, lane L
      // reads channels 16 jt + 4 (L % 4) ..+4 of token 8 kg + L / 4 (+4), and lane n
      // receives channel 16 jt + n of the four tokens, the B operand's k = 8 kg ..+4 (+4)
      const uint8_t *src = vt + (8 * kg + (n >> 2)) * AM_VTROW + 2 * (16 * jt + 4 * (n & 3));
      const att_i16x4 w0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) att_i16x4 *)(src));
      const att_i16x4 w1 =
          __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) att_i16x4 *)(src + 4 * AM_VTROW));
      const att_bf16x8 bv = __builtin_bit_cast(
          att_bf16x8, att_u32x4{__builtin_bit_cast(uint2, w0).x, __builtin_bit_cast(uint2, w0).y,
                                __builtin_bit_cast(uint2, w1).x, __builtin_bit_cast(uint2, w1).y});
      o[jt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bv, o[jt], 0, 0, 0);
      o[jt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bv, o[jt], 0, 0, 0);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };

  // steps of 32 positions: wave w takes steps w, w + 4, ...; a step's K/V loads are issued
  // two steps ahead and its two page ids one step before that, so no step waits on a
  // block-table read before it can issue its loads (three register buffers: 250 VGPRs
  // with launch bounds for 2 blocks per CU, the most the LDS allows; one step ahead
  // measured 2% slower)
  constexpr int STEP = 32;
  const int64_t stride = (int64_t)ATT_WAVES * STEP;
  int64_t t0 = t_begin + (int64_t)wave * STEP;
  uint4 k0[2][2], v0[2][2], k1[2][2], v1[2][2], k2[2][2], v2[2][2];
  int r0[2], r1[2], r2[2];
  int64_t p0[2], p1[2], p2[2];
  auto pages_of_step = [&](int64_t ts0, int64_t (&p)[2]) {
    p[0] = tile_page(ts0);
    p[1] = tile_page(ts0 + 16);
  };
  auto load_step = [&](int64_t ts0, const int64_t (&p)[2], uint4 (&kc)[2][2], uint4 (&vc)[2][2], int (&rows)[2]) {
    load_tile(ts0, p[0], kc[0], vc[0], rows[0]);
    load_tile(ts0 + 16, p[1], kc[1], vc[1], rows[1]);
  };
  // past the end the loads are zero-length
  pages_of_step(t0, p0);
  load_step(t0, p0, k0, v0, r0);
  pages_of_step(t0 + stride, p1);
  load_step(t0 + stride, p1, k1, v1, r1);
  pages_of_step(t0 + 2 * stride, p2);
  while (t0 < t_end) {
    load_step(t0 + 2 * stride, p2, k2, v2, r2);
    pages_of_step(t0 + 3 * stride, p0);
    compute_step(k0, v0, r0);
    t0 += stride;
    if (t0 >= t_end) break;
    load_step(t0 + 2 * stride, p0, k0, v0, r0);
    pages_of_step(t0 + 3 * stride, p1);
    compute_step(k1, v1, r1);
    t0 += stride;
    if (t0 >= t_end) break;
    load_step(t0 + 2 * stride, p1, k1, v1, r1);
    pages_of_step(t0 + 3 * stride, p2);
    compute_step(k2, v2, r2);
    t0 += stride;
  }

  // l over the 16 token lanes; then the block's waves merge through LDS
#pragma unroll
  for (int j = 0; j < 4; ++j) l[j] = group_sum<16>(l[j]);
  __shared__ float sm_m[ATT_WAVES][4], sm_l[ATT_WAVES][4];
  __shared__ float sm_acc[ATT_WAVES][4][D];
  if (kg == 0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int t = 0; t < 8; ++t) sm_acc[wave][j][16 * t + n] = o[t][j];
      if (n == 0) {
        sm_m[wave][j] = m[j];
        sm_l[wave][j] = l[j];
      }
    }
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < G * D; idx += ATT_THREADS) {
    const int j = idx / D, d = idx % D;
    float M = sm_m[0][j];
#pragma unroll
    for (int w = 1; w < ATT_WAVES; ++w) M = fmaxf(M, sm_m[w][j]);
    float a = 0.0f, ll = 0.0f;
#pragma unroll
    for (int w = 0; w < ATT_WAVES; ++w) {
      const float f = M == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(sm_m[w][j] - M);
      a += f * sm_acc[w][j][d];
      ll += f * sm_l[w][j];
    }
    float *pp = part + (((int64_t)b * g.n_q_heads + hq0 + j) * g.n_splits + split) * (2 + D);
    pp[2 + d] = a;
    if (d == 0) {
      pp[0] = M;
      pp[1] = ll;
    }
  }
  if (e && err) atomicOr(err, e);
}

// Pass 2: out[b][hq][:] = scale_v * sum_s 2^(m_s - M) acc_s / sum_s 2^(m_s - M) l_s.
__global__ void __launch_bounds__(256)
paged_decode_combine_kernel(const float *__restrict__ part, AttnGeom g, const float *__restrict__ scales,
                            uint16_t *__restrict__ out) {
  const int64_t row = blockIdx.x;  // b * Hq + hq
  const int hq = (int)(row % g.n_q_heads);
  const int h = hq / (g.n_q_heads / g.n_kv_heads);
  const int D = g.head_dim;
  const float *pp = part + row * g.n_splits * (2 + D);
  __shared__ float w_s[256];
  __shared__ float l_sum;
  float M = -INFINITY;
  for (int s = 0; s < g.n_splits; ++s) M = fmaxf(M, pp[s * (2 + D)]);
  if (threadIdx.x == 0) {
    float ll = 0.0f;
    for (int s = 0; s < g.n_splits; ++s)
      ll += M == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(pp[s * (2 + D)] - M) * pp[s * (2 + D) + 1];
    l_sum = ll;
  }
  for (int s = threadIdx.x; s < g.n_splits && s < 256; s += blockDim.x)
    w_s[s] = M == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(pp[s * (2 + D)] - M);
  __syncthreads();
  const float sv = scales[g.n_kv_heads + h];
  for (int d = threadIdx.x; d < D; d += blockDim.x) {
    float a = 0.0f;
    for (int s = 0; s < g.n_splits; ++s) {
      const float f = s < 256 ? w_s[s] : (M == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(pp[s * (2 + D)] - M));
      a += f * pp[s * (2 + D) + 2 + d];
    }
    // a sequence without positions (l = 0) gives zeros
    const float o = l_sum == 0.0f ? 0.0f : a / l_sum * sv;
    out[row * D + d] = (uint16_t)(pack_bf16(o, 0.0f) & 0xFFFFu);
  }
}

}  // namespace zx

using namespace zx;

// Positions per block: a multiple of ATT_SPLIT_MIN, as long as the grid still has about
// eight blocks per CU, four per resident slot (long sequences in small batches get more,
// shorter splits).  With one block per slot (configs[2]: 64 sequences x 8 head groups =
// 512 blocks of 32k positions) the launch ends with the slowest CU; four per slot let the
// dispatcher even that out (1% on configs[2]; eight per slot costs more in partials).
static void att_splits(int32_t n_seqs, int32_t head_groups, int32_t max_blocks, int32_t page_size,
                       int64_t &n_splits, int64_t &split_len) {
  const int64_t max_len = (int64_t)max_blocks * page_size;
  const int64_t most = ceil_div(max_len, ATT_SPLIT_MIN);
  int64_t want = ceil_div(8LL * num_cus(), (int64_t)n_seqs * head_groups);
  want = want < 1 ? 1 : (want > most ? most : want);
  split_len = ceil_div(ceil_div(max_len, want), ATT_SPLIT_MIN) * ATT_SPLIT_MIN;
  n_splits = ceil_div(max_len, split_len);
}

static int32_t att_group(int32_t n_q_heads, int32_t n_kv_heads) {  // query heads per block
  const int grp = n_q_heads / n_kv_heads;
  return grp % 4 == 0 ? 4 : (grp % 2 == 0 ? 2 : 1);
}

extern "C" size_t zx_paged_attention_decode_workspace_bytes(int32_t n_seqs, int32_t n_q_heads, int32_t n_kv_heads,
                                                            int32_t head_dim, int32_t max_blocks, int32_t page_size) {
  if (n_seqs <= 0 || n_q_heads <= 0 || n_kv_heads <= 0 || n_q_heads % n_kv_heads || head_dim <= 0 ||
      max_blocks <= 0 || page_size <= 0)
    return 0;
  int64_t n_splits, split_len;
  att_splits(n_seqs, n_q_heads / att_group(n_q_heads, n_kv_heads), max_blocks, page_size, n_splits, split_len);
  return (size_t)n_seqs * n_q_heads * n_splits * (2 + head_dim) * sizeof(float);
}

template <int G, int D>
static int launch_partial(dim3 grid, hipStream_t st, const uint16_t *q, const AttnGeom &g, const uint8_t *pool,
                          const float *scales, const int32_t *bt, const int32_t *sl, float *part, int32_t *err) {
  constexpr int TPW = 64 / (D / 16);
  if (g.page_size % TPW == 0)
    paged_decode_partial_kernel<G, D, true><<<grid, ATT_THREADS, 0, st>>>(q, g, pool, scales, bt, sl, part, err);
  else
    paged_decode_partial_kernel<G, D, false><<<grid, ATT_THREADS, 0, st>>>(q, g, pool, scales, bt, sl, part, err);
  return check_launch("paged_decode_partial");
}

template <int G>
static int launch_mfma(dim3 grid, hipStream_t st, const uint16_t *q, const AttnGeom &g, const uint8_t *pool,
                       const float *scales, const int32_t *bt, const int32_t *sl, float *part, int32_t *err) {
  paged_decode_mfma_kernel<G><<<grid, ATT_THREADS, 0, st>>>(q, g, pool, scales, bt, sl, part, err);
  return check_launch("paged_decode_mfma");
}

template <int D>
static int launch_g(int G, dim3 grid, hipStream_t st, const uint16_t *q, const AttnGeom &g, const uint8_t *pool,
                    const float *scales, const int32_t *bt, const int32_t *sl, float *part, int32_t *err) {
  if (D == 128 && g.page_size % 16 == 0) {  // matrix-core variant
    switch (G) {
      case 1: return launch_mfma<1>(grid, st, q, g, pool, scales, bt, sl, part, err);
      case 2: return launch_mfma<2>(grid, st, q, g, pool, scales, bt, sl, part, err);
      default: return launch_mfma<4>(grid, st, q, g, pool, scales, bt, sl, part, err);
    }
  }
  switch (G) {
    case 1: return launch_partial<1, D>(grid, st, q, g, pool, scales, bt, sl, part, err);
    case 2: return launch_partial<2, D>(grid, st, q, g, pool, scales, bt, sl, part, err);
    default: return launch_partial<4, D>(grid, st, q, g, pool, scales, bt, sl, part, err);
  }
}

extern "C" int zx_paged_attention_decode(const uint16_t *q, int32_t n_q_heads, const uint8_t *pool, int64_t n_pages,
                                         int32_t n_kv_heads, int32_t head_dim, int32_t page_size,
                                         const float *scales, const int32_t *block_tables, int32_t max_blocks,
                                         const int32_t *seq_lens, int32_t n_seqs, float sm_scale, uint16_t *out,
                                         int32_t *err, void *workspace,
                                         size_t workspace_bytes, zx_stream_t stream) {
  clear_error();
  ZX_REQUIRE(q && pool && scales && block_tables && seq_lens && out, "paged_attention_decode: null pointer");
  ZX_REQUIRE(aligned16(q) && aligned16(pool) && aligned16(out),
             "paged_attention_decode: q, pool and out must be 16-byte aligned");
  ZX_REQUIRE(n_q_heads > 0 && n_kv_heads > 0 && n_pages > 0 && page_size > 0 && max_blocks > 0 && n_seqs > 0,
             "paged_attention_decode: sizes must be positive");
  ZX_REQUIRE(n_q_heads % n_kv_heads == 0, "paged_attention_decode: n_q_heads must be a multiple of n_kv_heads");
  if (!(head_dim == 64 || head_dim == 128 || head_dim == 256))
    return fail(ZX_ERR_UNSUPPORTED, "paged_attention_decode: head_dim %d not in {64, 128, 256}", head_dim);
  if (n_seqs > 65535) return fail(ZX_ERR_UNSUPPORTED, "paged_attention_decode: more than 65535 sequences");
  const size_t need =
      zx_paged_attention_decode_workspace_bytes(n_seqs, n_q_heads, n_kv_heads, head_dim, max_blocks, page_size);
  if (!workspace || workspace_bytes < need)
    return fail(ZX_ERR_WORKSPACE, "paged_attention_decode: workspace %zu < %zu bytes", workspace_bytes, need);
  const int grp = n_q_heads / n_kv_heads;
  const int G = att_group(n_q_heads, n_kv_heads);
  AttnGeom g;
  g.n_q_heads = n_q_heads;
  g.n_kv_heads = n_kv_heads;
  g.head_dim = head_dim;
  g.page_size = page_size;
  g.max_blocks = max_blocks;
  g.n_seqs = n_seqs;
  int64_t n_splits, split_len;
  att_splits(n_seqs, n_q_heads / G, max_blocks, page_size, n_splits, split_len);
  if (n_splits >= (1LL << 31) || split_len >= (1LL << 31))
    return fail(ZX_ERR_UNSUPPORTED, "paged_attention_decode: sequences too long");
  g.n_splits = (int32_t)n_splits;
  g.split_len = (int32_t)split_len;
  g.n_pages = n_pages;
  g.sm_scale = sm_scale;
  {  // magic division by the page size for positions below 2^31
    int sh = 0;
    while ((1LL << sh) < page_size) ++sh;
    g.p_shift = sh;
    g.p_magic = (uint32_t)(((1ULL << (31 + sh)) + (uint64_t)page_size - 1) / (uint64_t)page_size);
  }
  const int64_t gy = (int64_t)n_kv_heads * (grp / G);
  if (gy > 65535) return fail(ZX_ERR_UNSUPPORTED, "paged_attention_decode: too many heads");
  hipStream_t st = as_stream(stream);
  float *part = static_cast<float *>(workspace);
  const dim3 grid((unsigned)g.n_splits, (unsigned)gy, (unsigned)n_seqs);
  int rc;
  switch (head_dim) {
    case 64: rc = launch_g<64>(G, grid, st, q, g, pool, scales, block_tables, seq_lens, part, err); break;
    case 128: rc = launch_g<128>(G, grid, st, q, g, pool, scales, block_tables, seq_lens, part, err); break;
    default: rc = launch_g<256>(G, grid, st, q, g, pool, scales, block_tables, seq_lens, part, err); break;
  }
  if (rc) return rc;
  paged_decode_combine_kernel<<<(unsigned)((int64_t)n_seqs * n_q_heads), 256, 0, st>>>(part, g, scales, out);
  return check_launch("paged_decode_combine");
}
