// zx_prefill.hip -- blocks of queries attending to K/V straight from the paged FP8 pool:
// one ring step of QuantizedRingAttention (README.md:344), with the step's result merged
// into a running (output, log-sum-exp) so that the steps of a ring compose into full
// attention.  The ring exchange itself needs more than one GPU and is not here.
//
// A block owns (sequence, G query heads of one kv head, a tile of 32 * 4 / G query rows);
// its 4 waves each take one head and 32 rows (two 16-row MFMA tiles), so every K/V tile
// is read from HBM once per block and serves 128 query rows.  Steps of 64 keys (four
// 16-key tiles, each inside one page):
//   * the block loads the step's K and V runs with contiguous 16-byte lane loads (whole
//     cache lines; a thread takes channels 16 g ..+16 of two adjacent keys), one step
//     ahead of the compute; K goes to LDS decoded to bf16 rows, V goes transposed
//     (V^T[channel][key], bf16, the two keys of a thread as one 32-bit word), both double
//     buffered so one block barrier per step suffices;
//   * each wave computes the transposed problem, so that one query row sits in one lane
//     column of every MFMA tile: S^T = K . Q^T on v_mfma_f32_16x16x32_bf16 (K rows as A,
//     Q rows as B), key range / causal mask only on the steps that cross a boundary,
//     online softmax in the exp2 domain with row maxima over the 4 lane rows by
//     v_permlane32/16_swap, P^T kept in registers as the B operand (fp16 by default,
//     see PM below), O^T += V^T . P^T on the matrix cores, and the row sums of P as a
//     ninth tile against ones (the rescale of O skipped unless a row maximum was raised).
// At the end each row is normalised; with MERGE the step's (O, lse2) is combined with
// the running one in o_acc / lse2 (each (row, head) belongs to one block, so no races);
// with the bf16 flag the merged row is also written as bf16.
#include "zx_attn_common.h"

namespace zx {

constexpr int PF_THREADS = 256;
constexpr int PF_KEYS = 64;                  // keys per step
constexpr int PF_KROW = 272;                 // K row in LDS (128 channels bf16 + 16 pad: conflict-free reads)
constexpr int PF_VROW = 144;                 // V^T row (64 keys bf16 + 16 pad)
constexpr int PF_KBYTES = PF_KEYS * PF_KROW;
constexpr int PF_VBYTES = 128 * PF_VROW;
constexpr int PF_RTAB = 64;  // key ranges whose bounds a block keeps in LDS
constexpr int PF_MERGE = 1, PF_WRITE_BF16 = 2, PF_INIT = 4, PF_LAST = 8, PF_FINAL = 16;
// a row's running maximum m is raised only when a score exceeds it by more than this
// (log2 units), so p = 2^(s - m) <= 2^PF_LAZY and O is rarely rescaled
constexpr float PF_LAZY = 8.0f;

struct PrefillArgs {
  const uint16_t *q;  // [n_q][Hq][128] bf16
  const int32_t *cu_q, *q_pos0;
  const uint8_t *pool;
  const float *scales;  // [2][Hkv]
  const int32_t *bt, *kv_begin, *kv_end;  // [n_ranges][n_seqs] key ranges, walked in order
  float *o_acc;   // [n_q][Hq][128] fp32, normalised
  float *lse2;    // [n_q][Hq]
  uint16_t *out;  // [n_q][Hq][128] bf16 (PF_WRITE_BF16)
  int32_t *err;
  int64_t n_pages;
  int32_t n_q_heads, n_kv_heads, page_size, max_blocks, mode, causal, n_ranges, n_seqs;
  int32_t n_qt;  // query tiles per sequence (the grid is n_qt x head groups x sequences)
  uint32_t p_magic;
  int32_t p_shift;
  float sm_log2e;  // sm_scale * log2 e
};

__device__ __forceinline__ uint32_t pf_page_of(const PrefillArgs &a, uint32_t t) {
  return (uint32_t)(((uint64_t)t * a.p_magic) >> (31 + a.p_shift));
}

// MFMA k order of a step's keys: the 64 keys form two k-blocks of 32 (one PV MFMA each);
// inside k-block kb, k = 8 kg + 4 KT + i is key 32 kb + 16 KT + 4 kg + i, which is where
// the S^T tiles leave that key (tile 2 kb + KT, lane row kg, element i).  V^T rows hold
// the keys in this order, in 16-byte chunks (8 keys) swizzled by channel / 16.
__device__ __forceinline__ int pf_vslot_byte(int c, int key) {
  const int kb = key >> 5, KT = (key >> 4) & 1, kg = (key >> 2) & 3, i = key & 3;
  return c * PF_VROW + ((((kb << 2) + kg) ^ (c >> 4)) << 4) + 2 * (4 * KT + i);
}

// How P enters P.V (and the row sums, which use the same P):
//   PF_P_F16   P * 2^7 rounded once to fp16 (11 significant bits, relative error <= 2^-11;
//              the 2^7 keeps P's range (<= 2^PF_LAZY) inside fp16 and pushes its
//              subnormal range 7 octaves down), V^T in LDS as fp16 (e4m3 values are exact
//              in fp16), one fp16 MFMA per tile;
//   PF_P_BF16  P rounded once to bf16 (relative error <= 2^-9), one bf16 MFMA per tile,
//              the usual flash-attention numerics;
//   PF_P_EXACT P as bf16 hi + lo, two bf16 MFMAs per tile: P carried to ~2^-17.
constexpr int PF_P_F16 = 0, PF_P_BF16 = 1, PF_P_EXACT = 2;
constexpr float PF_F16_SHIFT = 7.0f;  // log2 of the factor P carries in PF_P_F16
typedef _Float16 att_f16x8 __attribute__((ext_vector_type(8)));

// O^T (or the row sums) += A . B on 16x16x32 tiles, A and B given as the bits of 8 values
__device__ __forceinline__ att_f32x4 pf_mfma_bf16(att_u32x4 a, att_u32x4 b, att_f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(att_bf16x8, a), __builtin_bit_cast(att_bf16x8, b),
                                                 c, 0, 0, 0);
}
__device__ __forceinline__ att_f32x4 pf_mfma_f16(att_u32x4 a, att_u32x4 b, att_f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(att_f16x8, a), __builtin_bit_cast(att_f16x8, b), c,
                                                0, 0, 0);
}
__device__ __forceinline__ uint32_t pack_f16(float lo, float hi) {
  typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
  f16x2_t v;
  v[0] = (_Float16)lo;
  v[1] = (_Float16)hi;
  return __builtin_bit_cast(uint32_t, v);
}
// 16 e4m3 codes -> 8 fp16 pairs (exact: every e4m3 value is an fp16 value).
__device__ __forceinline__ void decode16_f16(uint4 c, uint32_t (&b)[8]) {
  const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    b[2 * i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)w[i], 1.0f, false));
    b[2 * i + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)w[i], 1.0f, true));
  }
}

template <int G, int PM>
__global__ void __launch_bounds__(PF_THREADS, 2) paged_prefill_mfma_kernel(PrefillArgs a) {
  constexpr bool EXACT = PM == PF_P_EXACT, F16 = PM == PF_P_F16;
  constexpr int D = 128;
  constexpr int QT = 32 * 4 / G;  // query rows per block
  // one-dimensional grid, query tile slowest: the last query tiles see the most keys under
  // a causal mask, so every (head group, sequence)'s last tile is launched first, then
  // every second-to-last, ... (globally longest first: the shortest blocks make the tail)
  const int n_hg = a.n_q_heads / G;
  const int64_t per_rank = (int64_t)n_hg * a.n_seqs;
  const int64_t qt_rev = (int64_t)blockIdx.x / per_rank;
  const int rem = (int)((int64_t)blockIdx.x - qt_rev * per_rank);
  const int hg = rem % n_hg, b = rem / n_hg;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15, kg = lane >> 4;
  const int grp = a.n_q_heads / a.n_kv_heads;
  const int hq = hg * G + wave % G;
  const int h = (hg * G) / grp;  // the block's KV head (G divides grp: its G query heads share it)
  // What the set-up reads that depends only on the (sequence, head group) is loaded in one
  // round trip: the sequence's queries, its first key range and the head's scales.  Every
  // dependent round trip of a block's set-up or final merge is a wait of that block, and
  // they count where blocks are short: a ring step of 1,024 keys per launch (one launch per
  // step, as a multi-GPU ring runs) took 7% less time per ring with the set-up below (the
  // pages of the first two steps and Q read together, then the first K/V and the block
  // table check) and the running output read in one go at the end.
  const int32_t cq0 = a.cu_q[b], cq1 = a.cu_q[b + 1], qp0_32 = a.q_pos0[b];
  const int32_t kb0 = a.kv_begin[b], ke0 = a.kv_end[b];
  const float sk = a.scales[h], sv = a.scales[a.n_kv_heads + h];
  // (the empty asm takes every value as an operand, so the compiler issues the loads
  // together here instead of sinking each one to its first use past a branch)
  asm volatile("" ::"s"(cq0), "s"(cq1), "s"(qp0_32), "s"(kb0), "s"(ke0), "s"(sk), "s"(sv));
  const int64_t qp0 = qp0_32;
  const int64_t q_lo = cq0;
  const int n_qb = cq1 - cq0;
  const int64_t row0_64 = ((int64_t)a.n_qt - 1 - qt_rev) * QT;
  if (row0_64 >= n_qb) return;
  const int row0_blk = (int)row0_64;
  const int wrow0 = row0_blk + 32 * (wave / G);  // this wave's first row (in the sequence)
  const int64_t page_bytes = 2LL * a.n_kv_heads * a.page_size * D;
  const int64_t head_off = (int64_t)h * a.page_size * D;
  const int64_t v_off = (int64_t)a.n_kv_heads * a.page_size * D;
  const int32_t *bt = a.bt + (int64_t)b * a.max_blocks;
  int32_t e = 0;
  // rows past n_qt * QT (max_q_per_seq too small) are not computed: flag it
  if (qt_rev == 0 && (int64_t)a.n_qt * QT < n_qb) e |= ZX_KERR_POS_RANGE;
  const int kmax = a.max_blocks * a.page_size;  // < 2^31 (checked by the host)
  // keys past the block's last query position never count when causal
  const int last_row = min(row0_blk + QT, n_qb) - 1;
  // Range r of this sequence: keys [kb, ke) (ke clipped to the block table), walked in
  // 64-key steps from s_first (kb rounded down to a 16-key tile) while below ke_blk (ke,
  // or the block's last causal key + 1).  All block-uniform.
  struct Range {
    int kb, ke, s_first, ke_blk;
  };
  // With several ranges, their bounds go to LDS in one round trip here: read where the
  // walk reaches them, each would stall the steps for a dependent load.
  __shared__ int32_t rtab[2][PF_RTAB];
  const int n_tab = a.n_ranges > 1 ? min(a.n_ranges, PF_RTAB) : 0;
  if (n_tab) {  // block-uniform
    for (int r = threadIdx.x; r < n_tab; r += PF_THREADS) {
      const int64_t i = (int64_t)r * a.n_seqs + b;
      rtab[0][r] = a.kv_begin[i];
      rtab[1][r] = a.kv_end[i];
    }
    __syncthreads();
  }
  auto range = [&](int r) -> Range {
    Range g;
    const int64_t i = (int64_t)r * a.n_seqs + b;
    int32_t kbr, ker;
    if (r == 0) {
      kbr = kb0;
      ker = ke0;
    } else if (r < n_tab) {
      kbr = __builtin_amdgcn_readfirstlane(rtab[0][r]);
      ker = __builtin_amdgcn_readfirstlane(rtab[1][r]);
    } else {
      kbr = a.kv_begin[i];
      ker = a.kv_end[i];
    }
    g.kb = kbr > 0 ? kbr : 0;
    g.ke = ker;
    if (g.ke > kmax) {
      e |= ZX_KERR_POS_RANGE;
      g.ke = kmax;
    }
    g.ke_blk = a.causal ? (int)max((int64_t)-1, min((int64_t)g.ke, qp0 + last_row + 1)) : g.ke;
    g.s_first = (g.kb / 16) * 16;
    return g;
  };
  // the first range with a step at or after r (a.n_ranges if none)
  auto next_range = [&](int r, Range &g) -> int {
    for (; r < a.n_ranges; ++r) {
      g = range(r);
      if (g.s_first < g.ke_blk) return r;
    }
    return a.n_ranges;
  };
  Range cur;
  int rc = next_range(0, cur);
  // rows that reach no key still have something to write on a first step (the empty
  // running output), on a step that writes bf16 for every row, and on a FINAL ring's last
  // step (rows beyond the keys, finished now)
  const bool rows_without_keys_write =
      (a.mode & PF_INIT) ||
      ((a.mode & PF_WRITE_BF16) && (!(a.mode & PF_FINAL) || (a.mode & PF_LAST)));
  // a FINAL step leaves rows below kv_begin alone: a block of such rows only would read
  // the running output for nothing
  const bool rows_all_done = (a.mode & PF_FINAL) && !(a.mode & PF_INIT) && qp0 + last_row < (int64_t)kb0;
  if ((rc == a.n_ranges && !rows_without_keys_write) || rows_all_done) {
    // no key of any range reaches the block's rows: merging would leave o_acc and lse2 as
    // they are, and a FINAL step's rows below kv_begin were finished before (block-uniform
    // exit)
    if (e && a.err && threadIdx.x == 0) atomicOr(a.err, e);
    return;
  }

  __shared__ __attribute__((aligned(16))) uint8_t kst[2][PF_KBYTES];
  __shared__ __attribute__((aligned(16))) uint8_t vtl[2][PF_VBYTES];

  // every page the block may load inside the pool? (then the steps skip the per-tile
  // block-table checks; otherwise tiles on bad pages count as masked).  Found below, once
  // the first step's loads are in flight.
  bool all_ok = false;

  // Q rows as the B operand of S^T = K . Q^T: lane (n, kg) of row tile rt holds row
  // wrow0 + 16 rt + n, channels 32 kg + 8 c ..+8 for MFMA c (the K operand's channel order);
  // loaded below, after the first step's page lookup
  att_bf16x8 qa[2][4];
  const float qs = sk * a.sm_log2e;  // K's dequant scale folds into the scores
  const float vscale = sv;

  // O^T tiles: o[rt][jt] holds channels 16 jt + 4 kg ..+4 of row 16 rt + n; m per row.
  // The softmax denominator l is a ninth tile on the matrix cores: V^T rows of ones, so
  // every element of ol[rt] is the row's sum of the same P that O uses.
  att_f32x4 o[2][8], ol[2];
  float m[2];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
#pragma unroll
    for (int jt = 0; jt < 8; ++jt) o[rt][jt] = att_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    ol[rt] = att_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    m[rt] = -INFINITY;
  }
  const uint32_t one2 = F16 ? 0x3C003C00u : 0x3F803F80u;  // two ones (fp16 / bf16)
  const att_u32x4 ones = {one2, one2, one2, one2};
  // the factor 2^PF_F16_SHIFT that P carries in PF_P_F16 (it cancels in O / l)
  const float p_shift = F16 ? PF_F16_SHIFT : 0.0f;

  // block-cooperative load of one step: thread t moves 16 bytes of K and of V of keys
  // 2 (t / 8) and 2 (t / 8) + 1 (so wave w loads 16-key tile w), channels 16 (t % 8) ..+16;
  // tiles past the range or on a bad page load through zero-length resources
  const int kp2 = threadIdx.x >> 3, g8 = threadIdx.x & 7;
  const int kk0 = 2 * kp2;
  auto tile_ok = [&](int tp, int ke) -> bool {  // uniform
    if (tp >= ke) return false;
    if (all_ok) return true;
    const int64_t page = bt[pf_page_of(a, (uint32_t)tp)];
    return page >= 0 && page < a.n_pages;
  };
  // a step's page, looked up one step before its K/V loads are issued, so that the
  // block-table read is never waited for on its own (3% on the ring workload).  The row's
  // byte size fits the resource: page_size >= 16 and max_blocks * page_size < 2^31.
  const __amdgpu_buffer_rsrc_t rbt = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int32_t *>(bt), (short)0, a.max_blocks * (int)sizeof(int32_t), 0x00020000);
  struct StepPage {
    int tc, live;
    uint32_t bi;
    int32_t page;
  };
  auto lookup_step = [&](int s0, int ke) -> StepPage {
    StepPage p;
    const int tp = s0 + 16 * wave;  // this wave's 16-key tile (scalar: the buffer resources stay in SGPRs)
    p.live = max(0, min(16, ke - tp));
    p.tc = tp < ke ? tp : (ke > 0 ? ke - 1 : 0);
    p.bi = pf_page_of(a, (uint32_t)p.tc);
    // a range-checked load (entries past the block table read as 0; a tile with no key
    // never uses its page), issued without a branch so the wait for it can be counted
    p.page = __builtin_amdgcn_raw_buffer_load_b32(rbt, (int)(p.bi * 4u), 0, 0);
    return p;
  };
  auto issue_step = [&](const StepPage &p, att_u32x4 (&kc)[2], att_u32x4 (&vc)[2]) {
    const int64_t page = __builtin_amdgcn_readfirstlane(p.page);
    const bool ok = p.live > 0 && page >= 0 && page < a.n_pages;
    e |= (p.live > 0 && !ok) ? ZX_KERR_PAGE_RANGE : 0;
    const int nrec = ok ? p.live * D : 0;
    const uint8_t *src =
        a.pool + (ok ? page * page_bytes + head_off + (int64_t)(p.tc - (int)p.bi * a.page_size) * D : 0);
    const __amdgpu_buffer_rsrc_t rk =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(src), (short)0, nrec, 0x00020000);
    const __amdgpu_buffer_rsrc_t rv =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(src + (ok ? v_off : 0)), (short)0, nrec, 0x00020000);
    const int off = (kk0 & 15) * D + 16 * g8;
    kc[0] = __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 2);
    kc[1] = __builtin_amdgcn_raw_buffer_load_b128(rk, off + D, 0, 2);
    vc[0] = __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, 2);
    vc[1] = __builtin_amdgcn_raw_buffer_load_b128(rv, off + D, 0, 2);
  };
  // K/V of one step stored into an LDS buffer, in 8 pieces so that the store can be spread
  // over the matrix products of the step before: 0, 1 the two K rows (decoded once per
  // block, read as bf16 by the 4 waves); 2 the V decode into v0, v1; 3 .. 6 two V^T channel
  // pairs each (channel c = 16 g8 + 2 p (+1) gets keys kk0, kk0 + 1, adjacent k slots, as
  // one word); 7 nothing
  auto store_piece = [&](int buf, int j, const att_u32x4 (&kc)[2], const att_u32x4 (&vc)[2], uint32_t (&v0)[8],
                         uint32_t (&v1)[8]) {
    if (j < 2) {
      uint32_t kb8[8];
      decode16_bf16(make_uint4(kc[j].x, kc[j].y, kc[j].z, kc[j].w), kb8);
      uint4 *kd = reinterpret_cast<uint4 *>(&kst[buf][(kk0 + j) * PF_KROW + 32 * g8]);
      kd[0] = make_uint4(kb8[0], kb8[1], kb8[2], kb8[3]);
      kd[1] = make_uint4(kb8[4], kb8[5], kb8[6], kb8[7]);
    } else if (j == 2) {
      if constexpr (F16) {
        decode16_f16(make_uint4(vc[0].x, vc[0].y, vc[0].z, vc[0].w), v0);
        decode16_f16(make_uint4(vc[1].x, vc[1].y, vc[1].z, vc[1].w), v1);
      } else {
        decode16_bf16(make_uint4(vc[0].x, vc[0].y, vc[0].z, vc[0].w), v0);
        decode16_bf16(make_uint4(vc[1].x, vc[1].y, vc[1].z, vc[1].w), v1);
      }
    } else if (j < 7) {
      const int slot0 = pf_vslot_byte(16 * g8, kk0);  // channel 16 g8; the others add c * PF_VROW
#pragma unroll
      for (int pp = 0; pp < 2; ++pp) {
        const int p = 2 * (j - 3) + pp;
        uint8_t *row = &vtl[buf][slot0 + 2 * p * PF_VROW];
        *reinterpret_cast<uint32_t *>(row) = __builtin_amdgcn_perm(v1[p], v0[p], 0x05040100u);
        *reinterpret_cast<uint32_t *>(row + PF_VROW) = __builtin_amdgcn_perm(v1[p], v0[p], 0x07060302u);
      }
    }
  };
  auto store_step = [&](int buf, const att_u32x4 (&kc)[2], const att_u32x4 (&vc)[2]) {
    uint32_t v0[8], v1[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) store_piece(buf, j, kc, vc, v0, v1);
  };

  // one step: S^T, softmax, then the P.V products with the next step's K/V stored between
  // them
  auto compute_step = [&](int buf, int s0, int kb, int ke, const att_u32x4 (&kc)[2], const att_u32x4 (&vc)[2]) {
    bool tok[4];
#pragma unroll
    for (int KT = 0; KT < 4; ++KT) tok[KT] = tile_ok(s0 + 16 * KT, ke);
    // S^T tiles: sc[rt][KT] lane (n, kg) holds keys 16 KT + 4 kg + i of row 16 rt + n
    att_f32x4 sc[2][4];
    // A operand: key 16 KT + n, channels 32 kg + 8 c ..+8, read one tile ahead
    att_bf16x8 kar[2][4];
    auto ld_ka = [&](int KT, att_bf16x8 (&dst)[4]) {
      const uint8_t *kr = &kst[buf][(16 * KT + n) * PF_KROW + kg * 64];
#pragma unroll
      for (int c = 0; c < 4; ++c)
        dst[c] = __builtin_bit_cast(att_bf16x8, *reinterpret_cast<const att_u32x4 *>(kr + 16 * c));
    };
    ld_ka(0, kar[0]);
    // wave priority: low while this wave issues its products, high for its softmax and the
    // rest of the step, so that on a SIMD the other block's wave (in another phase) keeps
    // the matrix core fed while this one's VALU work goes first (3% on the ring workload;
    // the exact mode, with twice the P.V products, loses 1% with it and keeps one level)
    if constexpr (!EXACT) __builtin_amdgcn_s_setprio(0);
#pragma unroll
    for (int KT = 0; KT < 4; ++KT) {
      if (KT + 1 < 4) ld_ka(KT + 1, kar[(KT + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
      const att_bf16x8 (&ka)[4] = kar[KT & 1];
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        att_f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int c = 0; c < 4; ++c) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[c], qa[rt][c], acc, 0, 0, 0);
        sc[rt][KT] = acc;
      }
    }
    if constexpr (!EXACT) __builtin_amdgcn_s_setprio(1);
    // wave-uniform: every (row, key) of the step counts, no mask needed (and qs >= 0, so
    // the row maximum of s * qs is qs times the maximum of s)
    const bool full = tok[0] && tok[1] && tok[2] && tok[3] && s0 >= kb && s0 + PF_KEYS <= ke &&
                      wrow0 + 32 <= n_qb && qs >= 0.0f &&
                      (!a.causal || (int64_t)s0 + PF_KEYS - 1 <= qp0 + wrow0);
    float alpha[2];
    bool grow_any = false;
    att_u32x4 ph[2][2], pl[2][2];  // [rt][k-block] P^T (hi) / lo as 16-bit pairs: word 2 KT + i / 2
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      const int r = wrow0 + 16 * rt + n;
      // last key position the row may see (keys are < 2^31)
      const int lim = (r < n_qb) ? (a.causal ? (int)min(max(qp0 + r, (int64_t)-1), (int64_t)INT32_MAX) : INT32_MAX)
                                 : -1;
      auto valid = [&](int KT, int i) {  // branch-free
        const int kp = s0 + 16 * KT + 4 * kg + i;
        return tok[KT] & (kp >= kb) & (kp < ke) & (kp <= lim);
      };
      float mx = -INFINITY;
      if (full) {
#pragma unroll
        for (int KT = 0; KT < 4; ++KT)
#pragma unroll
          for (int i = 0; i < 4; ++i) mx = fmaxf(mx, sc[rt][KT][i]);
        mx *= qs;
      } else {
#pragma unroll
        for (int KT = 0; KT < 4; ++KT)
#pragma unroll
          for (int i = 0; i < 4; ++i) mx = fmaxf(mx, valid(KT, i) ? sc[rt][KT][i] * qs : -INFINITY);
      }
      mx = xrow_max(mx);
      const bool grow = mx > m[rt] + PF_LAZY;  // a row with no key yet grows at its first key
      const float mn = grow ? mx : m[rt];
      const float ms = mn == -INFINITY ? 0.0f : mn;  // a row with no key yet keeps p = 0
      alpha[rt] = grow ? __builtin_amdgcn_exp2f(m[rt] - ms) : 1.0f;
      grow_any |= grow;
      m[rt] = mn;
      // exponent s qs - m, -inf for the masked (row, key) pairs (qs >= 0 keeps the
      // unmasked exponents <= PF_LAZY; with qs < 0 every step takes the masked branch,
      // where the maximum was taken over s qs itself)
      float xe[4][4];
#pragma unroll
      for (int KT = 0; KT < 4; ++KT)
#pragma unroll
        for (int i = 0; i < 4; ++i) xe[KT][i] = __builtin_fmaf(sc[rt][KT][i], qs, p_shift - ms);
      if (!full) {
#pragma unroll
        for (int KT = 0; KT < 4; ++KT)
#pragma unroll
          for (int i = 0; i < 4; ++i) xe[KT][i] = valid(KT, i) ? xe[KT][i] : -INFINITY;
      }
#pragma unroll
      for (int KT = 0; KT < 4; ++KT)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const float p0 = __builtin_amdgcn_exp2f(xe[KT][2 * j]), p1 = __builtin_amdgcn_exp2f(xe[KT][2 * j + 1]);
          const uint32_t hw = F16 ? pack_f16(p0, p1) : pack_bf16(p0, p1);
          ph[rt][KT >> 1][2 * (KT & 1) + j] = hw;
          if constexpr (EXACT)
            pl[rt][KT >> 1][2 * (KT & 1) + j] =
                pack_bf16(p0 - __uint_as_float(hw << 16), p1 - __uint_as_float(hw & 0xFFFF0000u));
        }
    }
    // rescale O only when some row's maximum was raised
    if (__builtin_amdgcn_ballot_w64(grow_any)) {
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
#pragma unroll
        for (int jt = 0; jt < 8; ++jt) o[rt][jt] *= alpha[rt];
        ol[rt] *= alpha[rt];
      }
    }
    // the next step's K/V goes into the other LDS buffer (free since the last barrier), one
    // store piece per P.V tile, so that its VALU and LDS work sit beside the products (2%
    // on the ring workload against storing it whole before them)
    uint32_t nv0[8], nv1[8];  // the next step's V, decoded by store piece 2
    // A operand per 16-channel tile and k-block: V^T[channel 16 jt + n][k 8 kg ..+8],
    // read PVD tiles ahead of its products (the scheduling barrier keeps the compiler
    // from sinking the reads next to their use: 2% on the ring workload; one tile ahead
    // measured 2% faster than two once the blocks were launched longest first)
    constexpr int PVD = 1;
    att_u32x4 avr[PVD + 1][2];
    auto ld_av = [&](int jt, att_u32x4 (&dst)[2]) {
      const int ch = 16 * jt + n;
#pragma unroll
      for (int kbk = 0; kbk < 2; ++kbk)
        dst[kbk] = *reinterpret_cast<const att_u32x4 *>(&vtl[buf][ch * PF_VROW + ((((kbk << 2) + kg) ^ jt) << 4)]);
    };
#pragma unroll
    for (int jt = 0; jt < PVD; ++jt) ld_av(jt, avr[jt]);
    if constexpr (!EXACT) __builtin_amdgcn_s_setprio(0);
#pragma unroll
    for (int jt = 0; jt < 8; ++jt) {
      if (jt + PVD < 8) ld_av(jt + PVD, avr[(jt + PVD) % (PVD + 1)]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int kbk = 0; kbk < 2; ++kbk) {
        const att_u32x4 av = avr[jt % (PVD + 1)][kbk];
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
          if constexpr (F16) {
            o[rt][jt] = pf_mfma_f16(av, ph[rt][kbk], o[rt][jt]);
          } else {
            o[rt][jt] = pf_mfma_bf16(av, ph[rt][kbk], o[rt][jt]);
            if constexpr (EXACT) o[rt][jt] = pf_mfma_bf16(av, pl[rt][kbk], o[rt][jt]);
          }
        }
      }
      store_piece(buf ^ 1, jt, kc, vc, nv0, nv1);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int kbk = 0; kbk < 2; ++kbk)
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        if constexpr (F16) {
          ol[rt] = pf_mfma_f16(ones, ph[rt][kbk], ol[rt]);
        } else {
          ol[rt] = pf_mfma_bf16(ones, ph[rt][kbk], ol[rt]);
          if constexpr (EXACT) ol[rt] = pf_mfma_bf16(ones, pl[rt][kbk], ol[rt]);
        }
      }
    if constexpr (!EXACT) __builtin_amdgcn_s_setprio(1);
  };

  // steps: data of step s + 1 loaded into registers and the page of step s + 2 looked up
  // while step s computes; one barrier per step (the LDS buffers alternate).  The steps of
  // the ranges follow each other (the step after a range's last one is the next non-empty
  // range's first), with the running row maxima, O and row sums carried in registers from
  // range to range.  The last step also loads and stores a step after it (zero-length
  // loads; that buffer is never read).  Positions: p0 the step being computed, p1 the next
  // one (K/V loading), p2 the one after (page looked up); a position past the last range
  // stays there (s = 0, ke = 0).
  struct Pos {
    int s, rc;
    Range g;
  };
  auto advance = [&](const Pos &p) -> Pos {
    Pos q = p;
    if (p.rc >= a.n_ranges) return q;
    q.s = p.s + PF_KEYS;
    if (q.s >= p.g.ke_blk) {
      q.rc = next_range(p.rc + 1, q.g);
      q.s = q.rc < a.n_ranges ? q.g.s_first : 0;
    }
    return q;
  };
  auto ke_of = [&](const Pos &p) { return p.rc < a.n_ranges ? p.g.ke : 0; };
  att_u32x4 kc[2], vc[2];
  Pos p0 = {cur.s_first, rc, cur};
  // the pages of the first two steps and Q are read together, then the first step's K/V
  // and the block-table check
  StepPage pg0 = {0, 0, 0u, 0};
  if (p0.rc < a.n_ranges) pg0 = lookup_step(p0.s, p0.g.ke);
  Pos p1 = advance(p0);
  StepPage pg1 = lookup_step(p1.s, ke_of(p1));
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    const int r = wrow0 + 16 * rt + n;
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
  if (p0.rc < a.n_ranges) issue_step(pg0, kc, vc);
  {
    bool bad = false;
    for (int r = 0; r < a.n_ranges; ++r) {
      const Range g = range(r);
      if (g.s_first >= g.ke) continue;
      const int p_lo = (int)pf_page_of(a, (uint32_t)g.s_first), p_hi = (int)pf_page_of(a, (uint32_t)(g.ke - 1));
      for (int pi = p_lo + (int)threadIdx.x; pi <= p_hi; pi += PF_THREADS) {
        const int64_t pg = bt[pi];
        bad |= pg < 0 || pg >= a.n_pages;
      }
    }
    all_ok = !__syncthreads_or(bad);
  }
  if (p0.rc < a.n_ranges) store_step(0, kc, vc);
  __syncthreads();
  int buf = 0;
  while (p0.rc < a.n_ranges) {
    const Pos p2 = advance(p1);
    issue_step(pg1, kc, vc);
    const StepPage pg2 = lookup_step(p2.s, ke_of(p2));
    compute_step(buf, p0.s, p0.g.kb, p0.g.ke, kc, vc);
    __syncthreads();
    buf ^= 1;
    p0 = p1;
    p1 = p2;
    pg1 = pg2;
  }

  // rows: normalise; merge; store channels 16 jt + 4 kg ..+4.  The running output and
  // log-sum-exp being merged into are read first, all at once (rows past the sequence's
  // end read its last row and discard it).
  const bool merge_old = (a.mode & PF_MERGE) && !(a.mode & PF_INIT);
  // the merged rows go back into the running output unless this is a ring's last step
  const bool keep = (a.mode & PF_MERGE) && !(a.mode & PF_LAST);
  float lse_prev[2];
  float4 o_prev[2][8];
  if (merge_old) {
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      const int64_t row = (q_lo + min(wrow0 + 16 * rt + n, n_qb - 1)) * a.n_q_heads + hq;
      lse_prev[rt] = a.lse2[row];
#pragma unroll
      for (int jt = 0; jt < 8; ++jt) o_prev[rt][jt] = *reinterpret_cast<const float4 *>(a.o_acc + row * D + 16 * jt + 4 * kg);
    }
  }
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    const int r = wrow0 + 16 * rt + n;
    const float lt = ol[rt][0];
    if (r >= n_qb) continue;
    // FINAL: rows below kv_begin were finished by an earlier step (there is none before
    // the first); rows below kv_end (all rows on the last step) are finished by this one
    // and go to out only
    const int64_t pos = qp0 + r;
    const bool fin_mode = (a.mode & PF_FINAL) != 0;
    if (fin_mode && !(a.mode & PF_INIT) && pos < kb0) continue;
    const bool fin = fin_mode && (pos < ke0 || (a.mode & PF_LAST));
    const bool keep_row = keep && !fin;
    const bool bf16_row = (a.mode & PF_WRITE_BF16) && (!fin_mode || fin);
    const float lse_new = lt > 0.0f ? m[rt] + (__builtin_amdgcn_logf(lt) - p_shift) : -INFINITY;
    const float inv = lt > 0.0f ? vscale / lt : 0.0f;  // V's dequant scale applied once, here
    const int64_t row = (q_lo + r) * a.n_q_heads + hq;
    float wa = 0.0f, wb = 1.0f, lse = lse_new;
    if (merge_old) {
      const float lse_old = lse_prev[rt];
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
      const int64_t idx = row * D + 16 * jt + 4 * kg;
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = o[rt][jt][i] * inv * wb;
      if (merge_old) {  // also at weight 0, so that a NaN of an earlier step stays (0 x NaN)
        const float4 old = o_prev[rt][jt];
        v[0] += wa * old.x;
        v[1] += wa * old.y;
        v[2] += wa * old.z;
        v[3] += wa * old.w;
      }
      if (keep_row) *reinterpret_cast<float4 *>(a.o_acc + idx) = make_float4(v[0], v[1], v[2], v[3]);
      if (bf16_row)
        *reinterpret_cast<uint2 *>(a.out + idx) = make_uint2(pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]));
    }
    if (keep_row && kg == 0) a.lse2[row] = lse;
  }
  if (e && a.err) atomicOr(a.err, e);
}

}  // namespace zx

using namespace zx;

namespace {
int prefill_impl(const uint16_t *q, int64_t n_q, const int32_t *cu_q, const int32_t *q_pos0, int32_t n_q_heads,
                 const uint8_t *pool, int64_t n_pages, int32_t n_kv_heads, int32_t head_dim, int32_t page_size,
                 const float *scales, const int32_t *block_tables, int32_t max_blocks, const int32_t *kv_begin,
                 const int32_t *kv_end, int32_t n_ranges, int32_t n_seqs, int32_t max_q_per_seq, int32_t causal,
                 float sm_scale, int32_t flags, float *o_acc, float *lse2, uint16_t *out, int32_t *err,
                 zx_stream_t stream) {
  ZX_REQUIRE(q && cu_q && q_pos0 && pool && scales && block_tables && kv_begin && kv_end,
             "paged_attention_prefill: null pointer");
  ZX_REQUIRE(n_ranges >= 1, "paged_attention: n_ranges must be positive");
  ZX_REQUIRE(n_q >= 0 && n_q_heads > 0 && n_kv_heads > 0 && n_pages > 0 && page_size > 0 && max_blocks > 0 &&
                 n_seqs > 0 && max_q_per_seq >= 0,
             "paged_attention_prefill: sizes must be positive");
  ZX_REQUIRE(n_q_heads % n_kv_heads == 0, "paged_attention_prefill: n_q_heads must be a multiple of n_kv_heads");
  ZX_REQUIRE((flags & ~(ZX_PREFILL_MERGE | ZX_PREFILL_INIT | ZX_PREFILL_BF16 | ZX_PREFILL_FAST_P | ZX_PREFILL_EXACT_P |
                        ZX_PREFILL_LAST | ZX_PREFILL_FINAL)) == 0,
             "paged_attention_prefill: unknown flags");
  ZX_REQUIRE(!(flags & ZX_PREFILL_FINAL) ||
                 ((flags & ZX_PREFILL_MERGE) && (flags & ZX_PREFILL_BF16) && causal && n_ranges == 1),
             "paged_attention_prefill: ZX_PREFILL_FINAL needs ZX_PREFILL_MERGE, ZX_PREFILL_BF16, causal and one key "
             "range (zx_paged_attention_prefill)");
  ZX_REQUIRE(!(flags & ZX_PREFILL_LAST) || ((flags & ZX_PREFILL_MERGE) && (flags & ZX_PREFILL_BF16)),
             "paged_attention_prefill: ZX_PREFILL_LAST needs ZX_PREFILL_MERGE and ZX_PREFILL_BF16");
  ZX_REQUIRE(!((flags & ZX_PREFILL_FAST_P) && (flags & ZX_PREFILL_EXACT_P)),
             "paged_attention_prefill: ZX_PREFILL_FAST_P and ZX_PREFILL_EXACT_P together");
  ZX_REQUIRE(!(flags & ZX_PREFILL_MERGE) || (o_acc && lse2), "paged_attention_prefill: merging needs o_acc and lse2");
  ZX_REQUIRE(!(flags & ZX_PREFILL_BF16) || out, "paged_attention_prefill: bf16 output requested without out");
  ZX_REQUIRE(flags & (ZX_PREFILL_MERGE | ZX_PREFILL_BF16), "paged_attention_prefill: nothing to write");
  ZX_REQUIRE(aligned16(q) && aligned16(pool) && (!(flags & ZX_PREFILL_MERGE) || aligned16(o_acc)) &&
                 (!(flags & ZX_PREFILL_BF16) || aligned16(out)),
             "paged_attention_prefill: q, pool, o_acc and out must be 16-byte aligned");
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
  a.n_ranges = n_ranges;
  a.n_seqs = n_seqs;
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
           ((flags & ZX_PREFILL_BF16) ? PF_WRITE_BF16 : 0) | ((flags & ZX_PREFILL_LAST) ? PF_LAST : 0) |
           ((flags & ZX_PREFILL_FINAL) ? PF_FINAL : 0);
  a.causal = causal ? 1 : 0;
  a.sm_log2e = sm_scale * ATT_LOG2E;
  {  // t / page_size = (t * magic) >> (31 + shift) for t < 2^31
    int shift = 0;
    while ((1LL << shift) < page_size) ++shift;
    a.p_shift = shift;
    a.p_magic = (uint32_t)(((1ULL << (31 + shift)) + page_size - 1) / page_size);
  }
  const int QT = 32 * 4 / G;
  a.n_qt = (int32_t)ceil_div(max_q_per_seq, QT);
  const int64_t n_blocks = (int64_t)a.n_qt * (n_q_heads / G) * n_seqs;
  ZX_REQUIRE(n_blocks < (1LL << 31), "paged_attention_prefill: too many query tiles or sequences");
  const dim3 grid((unsigned)n_blocks);
  hipStream_t st = as_stream(stream);
  const int pm = (flags & ZX_PREFILL_EXACT_P) ? PF_P_EXACT : ((flags & ZX_PREFILL_FAST_P) ? PF_P_BF16 : PF_P_F16);
  switch (G * 4 + pm) {
#define ZX_PF_CASE(g, m) \
  case g * 4 + m: paged_prefill_mfma_kernel<g, m><<<grid, PF_THREADS, 0, st>>>(a); break;
    ZX_PF_CASE(4, PF_P_F16)
    ZX_PF_CASE(4, PF_P_BF16)
    ZX_PF_CASE(4, PF_P_EXACT)
    ZX_PF_CASE(2, PF_P_F16)
    ZX_PF_CASE(2, PF_P_BF16)
    ZX_PF_CASE(2, PF_P_EXACT)
    ZX_PF_CASE(1, PF_P_F16)
    ZX_PF_CASE(1, PF_P_BF16)
    ZX_PF_CASE(1, PF_P_EXACT)
#undef ZX_PF_CASE
    default: return fail(ZX_ERR_INVALID, "paged_attention_prefill: internal dispatch");
  }
  return check_launch("paged_prefill_mfma");
}
}  // namespace

extern "C" int zx_paged_attention_prefill(const uint16_t *q, int64_t n_q, const int32_t *cu_q, const int32_t *q_pos0,
                                          int32_t n_q_heads, const uint8_t *pool, int64_t n_pages, int32_t n_kv_heads,
                                          int32_t head_dim, int32_t page_size, const float *scales,
                                          const int32_t *block_tables, int32_t max_blocks, const int32_t *kv_begin,
                                          const int32_t *kv_end, int32_t n_seqs, int32_t max_q_per_seq,
                                          int32_t causal, float sm_scale, int32_t flags, float *o_acc, float *lse2,
                                          uint16_t *out, int32_t *err, zx_stream_t stream) {
  clear_error();
  return prefill_impl(q, n_q, cu_q, q_pos0, n_q_heads, pool, n_pages, n_kv_heads, head_dim, page_size, scales,
                      block_tables, max_blocks, kv_begin, kv_end, 1, n_seqs, max_q_per_seq, causal, sm_scale, flags,
                      o_acc, lse2, out, err, stream);
}

extern "C" int zx_paged_attention_ring(const uint16_t *q, int64_t n_q, const int32_t *cu_q, const int32_t *q_pos0,
                                       int32_t n_q_heads, const uint8_t *pool, int64_t n_pages, int32_t n_kv_heads,
                                       int32_t head_dim, int32_t page_size, const float *scales,
                                       const int32_t *block_tables, int32_t max_blocks, const int32_t *kv_begin,
                                       const int32_t *kv_end, int32_t n_ranges, int32_t n_seqs, int32_t max_q_per_seq,
                                       int32_t causal, float sm_scale, int32_t flags, float *o_acc, float *lse2,
                                       uint16_t *out, int32_t *err, zx_stream_t stream) {
  clear_error();
  return prefill_impl(q, n_q, cu_q, q_pos0, n_q_heads, pool, n_pages, n_kv_heads, head_dim, page_size, scales,
                      block_tables, max_blocks, kv_begin, kv_end, n_ranges, n_seqs, max_q_per_seq, causal, sm_scale,
                      flags, o_acc, lse2, out, err, stream);
}
