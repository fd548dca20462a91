/*
 * zx_oracle.c -- CPU restatement of the zenyx KV-cache hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the HIP library is compared
 * against: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * it.  The product (zenyx_amd/, libzenyx_kv.so) never links or calls it.
 *
 * Reference anchors (paths relative to the zenyx source tree):
 *   int8 legacy quant/dequant ........ zenyx/streaming/precision.py:8-12, 15-16
 *   Belady victim selection .......... zenyx/streaming/belady.py:25-51
 *   ring schedule .................... zenyx/streaming/kv_tiering.py:69-73 (generalised)
 *   FP8 per-head quant, paged append/gather, trace-level Belady: specified by the
 *   README (README.md:93-97, 157-159, 328-331, 343-346) whose code is absent from the
 *   tree; the exact semantics restated here are the ones include/zenyx_kv.h documents.
 *
 * Arithmetic is written from the definitions (OCP OFP8 v1.0 for e4m3fn, IEEE-754
 * binary16/bfloat16 round-to-nearest-even) with double-precision helpers, not with the
 * bit tricks the GPU kernels use, so the two implementations are independent.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ZXO_NEVER 0x7FFFFFFF

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ---------------------------------------------------------------- rounding helpers */

/* Round |a| (finite, >= 0) to the grid of a binary format with `mbits` stored mantissa
 * bits and minimum normal exponent `emin`, nearest-even.  Exact in double for every
 * float input because the grid spacing is a power of two. */
static double round_to_grid(double a, int mbits, int emin) {
  if (a == 0.0) return 0.0;
  int e;
  frexp(a, &e); /* a = m * 2^e, m in [0.5, 1) */
  int E = e - 1;
  if (E < emin) E = emin;
  double q = ldexp(1.0, E - mbits);
  return rint(a / q) * q; /* default rounding mode is round-to-nearest-even */
}

/* OCP e4m3fn: bias 7, 3 mantissa bits, no infinities, S.1111.111 is NaN, max 448.
 * Overflow (a value that rounds above 448) and Inf/NaN give NaN with the input sign. */
uint8_t zxo_e4m3_encode(float f) {
  uint8_t sign = (uint8_t)((f2u(f) >> 24) & 0x80);
  if (isnan(f) || isinf(f)) return sign | 0x7F;
  double r = round_to_grid(fabs((double)f), 3, -6);
  if (r > 448.0) return sign | 0x7F;
  if (r == 0.0) return sign;
  int e;
  frexp(r, &e);
  int E = e - 1;
  if (E < -6) return sign | (uint8_t)(r / ldexp(1.0, -9)); /* subnormal: m * 2^-9 */
  int mant = (int)(r / ldexp(1.0, E - 3)) - 8;
  return sign | (uint8_t)(((E + 7) << 3) | mant);
}

float zxo_e4m3_decode(uint8_t c) {
  int s = c >> 7, e = (c >> 3) & 0xF, m = c & 7;
  float v;
  if (e == 15 && m == 7) v = NAN;
  else if (e == 0) v = (float)ldexp((double)m, -9);
  else v = (float)ldexp((double)(8 + m), e - 10);
  return s ? -v : v;
}

/* float -> bfloat16 bits, nearest-even; NaN -> 0x7FC0. */
uint16_t zxo_bf16_rne(float f) {
  if (isnan(f)) return 0x7FC0;
  uint16_t sign = (uint16_t)((f2u(f) >> 16) & 0x8000);
  if (isinf(f)) return sign | 0x7F80;
  double r = round_to_grid(fabs((double)f), 7, -126);
  if (r >= 0x1p128) return sign | 0x7F80; /* rounds past the largest finite bf16 */
  return sign | (uint16_t)(f2u((float)r) >> 16);
}

float zxo_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

/* float -> binary16 bits, nearest-even; NaN -> 0x7E00. */
uint16_t zxo_f16_rne(float f) {
  if (isnan(f)) return 0x7E00;
  uint16_t sign = (uint16_t)((f2u(f) >> 16) & 0x8000);
  if (isinf(f)) return sign | 0x7C00;
  double r = round_to_grid(fabs((double)f), 10, -14);
  if (r > 65504.0) return sign | 0x7C00;
  if (r == 0.0) return sign;
  int e;
  frexp(r, &e);
  int E = e - 1;
  if (E < -14) return sign | (uint16_t)(r / ldexp(1.0, -24));
  int mant = (int)(r / ldexp(1.0, E - 10)) - 1024;
  return sign | (uint16_t)(((E + 15) << 10) | mant);
}

float zxo_f16_to_f32(uint16_t h) {
  int s = h >> 15, e = (h >> 10) & 0x1F, m = h & 0x3FF;
  double v;
  if (e == 31) v = m ? NAN : INFINITY;
  else if (e == 0) v = ldexp((double)m, -24);
  else v = ldexp((double)(1024 + m), e - 25);
  return (float)(s ? -v : v);
}

void zxo_e4m3_encode_array(const float *in, uint8_t *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = zxo_e4m3_encode(in[i]);
}
void zxo_e4m3_decode_array(const uint8_t *in, float *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = zxo_e4m3_decode(in[i]);
}
void zxo_bf16_rne_array(const float *in, uint16_t *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = zxo_bf16_rne(in[i]);
}
void zxo_f16_rne_array(const float *in, uint16_t *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = zxo_f16_rne(in[i]);
}

/* ---------------------------------------------------------------- FP8 per-head */

/* s = fp32(max(amax, 1e-8f) / 448.0f); a NaN amax gives NaN. */
float zxo_fp8_scale(float amax) {
  if (isnan(amax)) return u2f(0x7FC00000u);
  float a = amax < 1e-8f ? 1e-8f : amax;
  return a / 448.0f;
}

/* Code of one value under slab scale s (include/zenyx_kv.h numeric contract). */
uint8_t zxo_fp8_code(float x, float s) {
  if (isnan(s)) return 0x7F;
  if (isinf(s)) {
    if (isnan(x) || isinf(x)) return 0x7F;
    return (uint8_t)(((f2u(x) ^ f2u(s)) >> 24) & 0x80); /* x / +-inf: a zero signed as IEEE */
  }
  return zxo_e4m3_encode(x / s);
}

uint16_t zxo_fp8_dequant_value(uint8_t c, float s) { return zxo_bf16_rne(zxo_e4m3_decode(c) * s); }

/* Layout [n_outer][n_batch][n_heads][run]; scales [n_outer][n_heads]. */
void zxo_fp8_quant_heads(const uint16_t *x, int64_t n_outer, int64_t n_batch, int64_t n_heads,
                         int64_t run, uint8_t *codes, float *scales) {
  for (int64_t o = 0; o < n_outer; ++o)
    for (int64_t h = 0; h < n_heads; ++h) {
      float amax = 0.0f;
      int nan = 0;
      for (int64_t b = 0; b < n_batch; ++b) {
        const uint16_t *p = x + ((o * n_batch + b) * n_heads + h) * run;
        for (int64_t i = 0; i < run; ++i) {
          float v = fabsf(zxo_bf16_to_f32(p[i]));
          if (isnan(v)) nan = 1;
          else if (v > amax) amax = v;
        }
      }
      float s = zxo_fp8_scale(nan ? NAN : amax);
      scales[o * n_heads + h] = s;
      for (int64_t b = 0; b < n_batch; ++b) {
        int64_t base = ((o * n_batch + b) * n_heads + h) * run;
        for (int64_t i = 0; i < run; ++i) codes[base + i] = zxo_fp8_code(zxo_bf16_to_f32(x[base + i]), s);
      }
    }
}

void zxo_fp8_dequant_heads(const uint8_t *codes, const float *scales, int64_t n_outer,
                           int64_t n_batch, int64_t n_heads, int64_t run, uint16_t *y) {
  for (int64_t o = 0; o < n_outer; ++o)
    for (int64_t b = 0; b < n_batch; ++b)
      for (int64_t h = 0; h < n_heads; ++h) {
        float s = scales[o * n_heads + h];
        int64_t base = ((o * n_batch + b) * n_heads + h) * run;
        for (int64_t i = 0; i < run; ++i) y[base + i] = zxo_fp8_dequant_value(codes[base + i], s);
      }
}

/* ---------------------------------------------------------------- paged KV cache */

/* Token-major layer batch x[n_tok][2][H][D] (stride x_layer_stride elements between
 * layers) -> scales[L][2][H]. */
void zxo_kv_scales(const uint16_t *x, int64_t x_layer_stride, int32_t n_layers, int64_t n_tok,
                   int32_t n_heads, int32_t head_dim, float *scales) {
  int64_t row = 2LL * n_heads * head_dim;
  for (int32_t l = 0; l < n_layers; ++l)
    for (int32_t s = 0; s < 2 * n_heads; ++s) {
      float amax = 0.0f;
      int nan = 0;
      for (int64_t t = 0; t < n_tok; ++t) {
        const uint16_t *p = x + l * x_layer_stride + t * row + (int64_t)s * head_dim;
        for (int32_t d = 0; d < head_dim; ++d) {
          float v = fabsf(zxo_bf16_to_f32(p[d]));
          if (isnan(v)) nan = 1;
          else if (v > amax) amax = v;
        }
      }
      scales[(int64_t)l * 2 * n_heads + s] = zxo_fp8_scale(nan ? NAN : amax);
    }
}

/* Paged append; returns the OR of ZX_KERR_* bits (1 page range, 2 position range,
 * 8 overflow).  flags: 1 static scales (scales are input), 4 saturate (with static
 * scales: a finite x whose code under a finite scale is the NaN code, i.e. whose
 * quotient rounds beyond 448, sets bit 8 and is stored as +-448, the quotient's sign;
 * without it the NaN code stays and bit 8 is still set). */
int32_t zxo_kv_quant_append(const uint16_t *x, int64_t x_layer_stride, int32_t n_layers,
                            int64_t n_tok, int32_t n_heads, int32_t head_dim,
                            const int32_t *cu_seqlens, const int32_t *start_pos, int32_t n_seqs,
                            const int32_t *block_tables, int32_t max_blocks, int32_t page_size,
                            uint8_t *pool, int64_t pool_layer_stride, int64_t n_pages,
                            float *scales, int32_t flags) {
  int32_t err = 0;
  const int static_scales = flags & 1, saturate = flags & 4;
  if (!static_scales) zxo_kv_scales(x, x_layer_stride, n_layers, n_tok, n_heads, head_dim, scales);
  int64_t row = 2LL * n_heads * head_dim;
  for (int32_t l = 0; l < n_layers; ++l)
    for (int32_t b = 0; b < n_seqs; ++b)
      for (int64_t t = cu_seqlens[b]; t < cu_seqlens[b + 1]; ++t) {
        int64_t pos = (start_pos ? start_pos[b] : 0) + (t - cu_seqlens[b]);
        if (pos < 0 || pos >= (int64_t)max_blocks * page_size) { err |= 2; continue; }
        int64_t page = block_tables[(int64_t)b * max_blocks + pos / page_size];
        if (page < 0 || page >= n_pages) { err |= 1; continue; }
        int64_t slot = pos % page_size;
        for (int32_t s = 0; s < 2 * n_heads; ++s) {
          float sc = scales[(int64_t)l * 2 * n_heads + s];
          const uint16_t *src = x + l * x_layer_stride + t * row + (int64_t)s * head_dim;
          uint8_t *dst = pool + l * pool_layer_stride +
                         ((page * 2 * n_heads + s) * page_size + slot) * head_dim;
          for (int32_t d = 0; d < head_dim; ++d) {
            const float xv = zxo_bf16_to_f32(src[d]);
            uint8_t c = zxo_fp8_code(xv, sc);
            if (static_scales && isfinite(sc) && isfinite(xv) && (c & 0x7F) == 0x7F) {
              err |= 8;
              if (saturate) c = (uint8_t)((c & 0x80) | 0x7E);
            }
            dst[d] = c;
          }
        }
      }
  return err;
}

/* Paged gather + dequant of one layer -> k_out/v_out [B][H][out_len][D]. */
int32_t zxo_kv_gather_dequant(const uint8_t *pool, int64_t n_pages, int32_t n_heads,
                              int32_t head_dim, int32_t page_size, const float *scales,
                              const int32_t *block_tables, int32_t max_blocks,
                              const int32_t *seq_lens, int32_t n_seqs, int32_t out_len,
                              uint16_t *k_out, uint16_t *v_out) {
  int32_t err = 0;
  for (int32_t b = 0; b < n_seqs; ++b)
    for (int32_t kv = 0; kv < 2; ++kv)
      for (int32_t h = 0; h < n_heads; ++h) {
        uint16_t *out = (kv ? v_out : k_out) + (((int64_t)b * n_heads + h) * out_len) * head_dim;
        float sc = scales[kv * n_heads + h];
        for (int64_t t = 0; t < out_len; ++t) {
          uint16_t *o = out + t * head_dim;
          int64_t page = -1;
          if (t < seq_lens[b]) {
            if (t / page_size < max_blocks) {
              page = block_tables[(int64_t)b * max_blocks + t / page_size];
              if (page < 0 || page >= n_pages) { err |= 1; page = -1; }
            } else {
              err |= 2;
            }
          }
          if (page < 0) { memset(o, 0, (size_t)head_dim * 2); continue; }
          const uint8_t *src = pool + ((page * 2 + kv) * n_heads + h) * (int64_t)page_size * head_dim +
                               (t % page_size) * head_dim;
          for (int32_t d = 0; d < head_dim; ++d) o[d] = zxo_fp8_dequant_value(src[d], sc);
        }
      }
  return err;
}

/* ------------------------------------------------------ paged decode attention */

/* One query token per sequence attending to its paged FP8 K/V (the attention that
 * consumes FP8 pages directly, QuantizedRingAttention README.md:344; semantics defined
 * by include/zenyx_kv.h).  q [B][Hq][D] bf16; kv head of query head hq = hq / (Hq/Hkv);
 *   s_t = sm_scale * sum_d q[d] * K[t][d],  K = decode(code) * scale_k, t < seq_len
 *   out = sum_t softmax(s)_t * V[t],        V = decode(code) * scale_v
 * evaluated in double and rounded once to bf16 (via fp32); a sequence of length 0
 * gives zeros.  Returns the error bits of zxo_kv_gather_dequant (such rows are skipped). */
int32_t zxo_paged_attention_decode(const uint16_t *q, int32_t n_q_heads, const uint8_t *pool,
                                   int64_t n_pages, int32_t n_kv_heads, int32_t head_dim,
                                   int32_t page_size, const float *scales, const int32_t *block_tables,
                                   int32_t max_blocks, const int32_t *seq_lens, int32_t n_seqs,
                                   float sm_scale, uint16_t *out) {
  int32_t err = 0;
  const int32_t grp = n_q_heads / n_kv_heads;
  const int64_t page_bytes = 2LL * n_kv_heads * page_size * head_dim;
  double *s = NULL, *acc = malloc(sizeof(double) * head_dim);
  int64_t *pg = NULL, cap = 0;
  for (int32_t b = 0; b < n_seqs; ++b)
    for (int32_t hq = 0; hq < n_q_heads; ++hq) {
      const int32_t h = hq / grp;
      const uint16_t *qv = q + ((int64_t)b * n_q_heads + hq) * head_dim;
      uint16_t *o = out + ((int64_t)b * n_q_heads + hq) * head_dim;
      const int64_t len = seq_lens[b] > 0 ? seq_lens[b] : 0;
      if (len > cap) {
        cap = len;
        s = realloc(s, sizeof(double) * (size_t)cap);
        pg = realloc(pg, sizeof(int64_t) * (size_t)cap);
      }
      double m = -INFINITY;
      for (int64_t t = 0; t < len; ++t) {  /* scores; pg[t] < 0 marks a skipped row */
        pg[t] = -1;
        if (t / page_size >= max_blocks) { err |= 2; continue; }
        const int64_t page = block_tables[(int64_t)b * max_blocks + t / page_size];
        if (page < 0 || page >= n_pages) { err |= 1; continue; }
        pg[t] = page;
        const uint8_t *kr = pool + page * page_bytes + ((int64_t)h * page_size + t % page_size) * head_dim;
        double dot = 0.0;
        for (int32_t d = 0; d < head_dim; ++d)
          dot += (double)zxo_bf16_to_f32(qv[d]) * ((double)zxo_e4m3_decode(kr[d]) * (double)scales[h]);
        s[t] = dot * (double)sm_scale;
        if (s[t] > m) m = s[t];
      }
      double l = 0.0;
      for (int32_t d = 0; d < head_dim; ++d) acc[d] = 0.0;
      for (int64_t t = 0; t < len; ++t) {
        if (pg[t] < 0) continue;
        const double p = exp(s[t] - m);
        const uint8_t *vr = pool + pg[t] * page_bytes +
                            ((int64_t)(n_kv_heads + h) * page_size + t % page_size) * head_dim;
        l += p;
        for (int32_t d = 0; d < head_dim; ++d)
          acc[d] += p * ((double)zxo_e4m3_decode(vr[d]) * (double)scales[n_kv_heads + h]);
      }
      for (int32_t d = 0; d < head_dim; ++d) o[d] = l > 0.0 || isnan(l) ? zxo_bf16_rne((float)(acc[d] / l)) : 0;
    }
  free(s);
  free(pg);
  free(acc);
  return err;
}

/* ---------------------------------------------------------------- legacy int8 */

/* Block attention over the paged FP8 K/V: one ring step of QuantizedRingAttention
 * (README.md:344; semantics defined by include/zenyx_kv.h).  Query token i of sequence b
 * (rows [cu_q[b], cu_q[b+1]) of q [n_q][Hq][D] bf16) sits at position q_pos0[b] + i -
 * cu_q[b]; query head hq reads kv head hq / (Hq / Hkv) at key positions kp in
 * [kv_begin[b], kv_end[b]) with kp <= the query's position when causal:
 *   s = sm_scale * q . K_kp,  out = sum softmax(s)_kp V_kp   (K, V = decode(code) * scale)
 * in double, out rounded once to bf16 (via fp32); lse2 [n_q][Hq] = log2(sum exp(s)) in
 * fp32 (-inf and out = 0 when no key qualifies).  Returns error bits (1: a block-table
 * entry outside [0, n_pages), whose keys are skipped; 2: kv_end beyond max_blocks *
 * page_size, clipped). */
int32_t zxo_paged_attention_prefill(const uint16_t *q, const int32_t *cu_q, const int32_t *q_pos0,
                                    int32_t n_q_heads, const uint8_t *pool, int64_t n_pages, int32_t n_kv_heads,
                                    int32_t head_dim, int32_t page_size, const float *scales,
                                    const int32_t *block_tables, int32_t max_blocks, const int32_t *kv_begin,
                                    const int32_t *kv_end, int32_t n_seqs, int32_t causal, float sm_scale,
                                    uint16_t *out, float *lse2) {
  int32_t err = 0;
  const int32_t grp = n_q_heads / n_kv_heads;
  const int64_t page_bytes = 2LL * n_kv_heads * page_size * head_dim;
  double *s = NULL, *acc = malloc(sizeof(double) * head_dim);
  int64_t *pg = NULL, cap = 0;
  for (int32_t b = 0; b < n_seqs; ++b) {
    int64_t kb = kv_begin[b] > 0 ? kv_begin[b] : 0, ke = kv_end[b];
    if (ke > (int64_t)max_blocks * page_size) { err |= 2; ke = (int64_t)max_blocks * page_size; }
    const int64_t nk = ke > kb ? ke - kb : 0;
    if (nk > cap) {
      cap = nk;
      s = realloc(s, sizeof(double) * (size_t)cap);
      pg = realloc(pg, sizeof(int64_t) * (size_t)cap);
    }
    for (int64_t i = cu_q[b]; i < cu_q[b + 1]; ++i) {
      const int64_t qp = (int64_t)q_pos0[b] + (i - cu_q[b]);
      for (int32_t hq = 0; hq < n_q_heads; ++hq) {
        const int32_t h = hq / grp;
        const uint16_t *qv = q + (i * n_q_heads + hq) * head_dim;
        uint16_t *o = out + (i * n_q_heads + hq) * head_dim;
        double m = -INFINITY;
        for (int64_t j = 0; j < nk; ++j) {
          const int64_t t = kb + j;
          pg[j] = -1;
          if (causal && t > qp) continue;
          const int64_t page = block_tables[(int64_t)b * max_blocks + t / page_size];
          if (page < 0 || page >= n_pages) { err |= 1; continue; }
          pg[j] = page;
          const uint8_t *kr = pool + page * page_bytes + ((int64_t)h * page_size + t % page_size) * head_dim;
          double dot = 0.0;
          for (int32_t d = 0; d < head_dim; ++d)
            dot += (double)zxo_bf16_to_f32(qv[d]) * ((double)zxo_e4m3_decode(kr[d]) * (double)scales[h]);
          s[j] = dot * (double)sm_scale;
          if (s[j] > m) m = s[j];
        }
        double l = 0.0;
        for (int32_t d = 0; d < head_dim; ++d) acc[d] = 0.0;
        for (int64_t j = 0; j < nk; ++j) {
          if (pg[j] < 0) continue;
          const int64_t t = kb + j;
          const double p = exp(s[j] - m);
          const uint8_t *vr = pool + pg[j] * page_bytes +
                              ((int64_t)(n_kv_heads + h) * page_size + t % page_size) * head_dim;
          l += p;
          for (int32_t d = 0; d < head_dim; ++d)
            acc[d] += p * ((double)zxo_e4m3_decode(vr[d]) * (double)scales[n_kv_heads + h]);
        }
        for (int32_t d = 0; d < head_dim; ++d) o[d] = l > 0.0 || isnan(l) ? zxo_bf16_rne((float)(acc[d] / l)) : 0;
        if (lse2) lse2[i * n_q_heads + hq] = l > 0.0 ? (float)((m + log(l)) / log(2.0)) : -INFINITY;
      }
    }
  }
  free(s);
  free(pg);
  free(acc);
  return err;
}

/* Round a float to the storage dtype and back (0 bf16, 1 f16, 2 f32), as torch stores
 * every intermediate of precision.py:10-11 in the input dtype. */
static float to_dtype(float v, int dtype) {
  if (dtype == 0) return zxo_bf16_to_f32(zxo_bf16_rne(v));
  if (dtype == 1) return zxo_f16_to_f32(zxo_f16_rne(v));
  return v;
}
static float load_dtype(const void *x, int dtype, int64_t i) {
  if (dtype == 0) return zxo_bf16_to_f32(((const uint16_t *)x)[i]);
  if (dtype == 1) return zxo_f16_to_f32(((const uint16_t *)x)[i]);
  return ((const float *)x)[i];
}

/* precision.py:10: scale = tensor.abs().amax().clamp_min(1e-8) / 127.0, all in dtype;
 * precision.py:11: q = clamp(round(tensor / scale), -127, 127).to(int8).
 * Division is true IEEE division computed in fp32 (torch's CPU opmath) and rounded to
 * dtype; round() is half-to-even.  Returns the scale as a float (exactly a dtype value). */
float zxo_int8_legacy_quant(const void *x, int dtype, int64_t n, int8_t *q) {
  float amax = 0.0f;
  int nan = 0;
  for (int64_t i = 0; i < n; ++i) {
    float v = fabsf(load_dtype(x, dtype, i));
    if (isnan(v)) nan = 1;
    else if (v > amax) amax = v;
  }
  float a = nan ? NAN : amax;
  float lo = to_dtype(1e-8f, dtype);
  if (!(a >= lo) && !isnan(a)) a = lo;
  float s = to_dtype(a / 127.0f, dtype);
  for (int64_t i = 0; i < n; ++i) {
    float r = rintf(to_dtype(load_dtype(x, dtype, i) / s, dtype));
    if (isnan(r)) { q[i] = 0; continue; } /* int8 of NaN is not defined by the reference */
    if (r > 127.0f) r = 127.0f;
    if (r < -127.0f) r = -127.0f;
    q[i] = (int8_t)r;
  }
  return s;
}

/* precision.py:16: (q.float() * scale).to(bfloat16). */
void zxo_int8_legacy_dequant(const int8_t *q, float scale, int64_t n, uint16_t *y) {
  for (int64_t i = 0; i < n; ++i) y[i] = zxo_bf16_rne((float)q[i] * scale);
}

/* A check of the division the GPU's legacy quantiser uses for bf16 / f16 input, not part
 * of the restatement: with r = 1 / s (IEEE), q0 = x r, e = fma(-q0, s, x), the quotient
 * fma(e, r, q0) (or q0 itself when |q0| >= 65536, where the code saturates anyway) must
 * give the same int8 code as x / s above.  Every `scale_stride`-th finite scale the
 * quantiser produces from an amax of `dtype` (0 bf16, 1 f16) against every input x of that
 * dtype; returns the number of differing codes, *pairs the number compared. */
int64_t zxo_legacy_reciprocal_check(int dtype, int scale_stride, int64_t *pairs) {
  int64_t bad = 0, n = 0, k = 0;
  float last = -1.0f;
  const float lo = to_dtype(1e-8f, dtype);
  for (uint32_t ab = 0; ab < 0x8000u; ++ab) {
    float a = dtype == 0 ? zxo_bf16_to_f32((uint16_t)ab) : zxo_f16_to_f32((uint16_t)ab);
    if (isnan(a) || isinf(a)) continue;
    if (a < lo) a = lo;
    const float s = to_dtype(a / 127.0f, dtype);
    if (s == last) continue; /* amax values sharing a scale (they come in order) */
    last = s;
    const float r = 1.0f / s;
    if (!isfinite(s) || !isfinite(r) || (k++ % scale_stride)) continue;
    for (uint32_t xb = 0; xb < 0x10000u; ++xb) {
      const float x = dtype == 0 ? zxo_bf16_to_f32((uint16_t)xb) : zxo_f16_to_f32((uint16_t)xb);
      float w = rintf(to_dtype(x / s, dtype));
      const float q0 = x * r;
      const float q = fabsf(q0) < 65536.0f ? fmaf(fmaf(-q0, s, x), r, q0) : q0;
      float g = rintf(to_dtype(q, dtype));
      w = isnan(w) ? 0.0f : fminf(fmaxf(w, -127.0f), 127.0f);
      g = isnan(g) ? 0.0f : fminf(fmaxf(g, -127.0f), 127.0f);
      bad += w != g;
      ++n;
    }
  }
  if (pairs) *pairs = n;
  return bad;
}

/* The GPU's fast encoder for bf16 / f16 slabs with a finite scale, where every input obeys
 * |x| <= amax: q = x / s from r = 1 / s and one Markstein correction (no range guard),
 * rounded to the storage dtype, clamped to +-127, then rounded to an integer by adding
 * 1.5 * 2^23 (the low byte of the sum is the two's-complement code).  Checked against
 * the reference code rint(dtype(x / s)) (clamped, NaN -> 0) for every finite x with |x| at
 * most the largest amax of each scale; every scale_stride-th reachable scale.  Returns
 * the number of differing pairs; *pairs the number compared. */
int64_t zxo_legacy_fast_check(int dtype, int scale_stride, int64_t *pairs) {
  int64_t bad = 0, n = 0, k = 0;
  const float lo = to_dtype(1e-8f, dtype);
  const uint32_t fin = dtype == 0 ? 0x7F80u : 0x7C00u; /* first non-finite magnitude */
  uint32_t ab = 0;
  while (ab < fin) {
    /* the run of amax patterns [ab, ae) sharing one scale */
    float a = dtype == 0 ? zxo_bf16_to_f32((uint16_t)ab) : zxo_f16_to_f32((uint16_t)ab);
    const float s = to_dtype((a < lo ? lo : a) / 127.0f, dtype);
    uint32_t ae = ab + 1;
    while (ae < fin) {
      float a2 = dtype == 0 ? zxo_bf16_to_f32((uint16_t)ae) : zxo_f16_to_f32((uint16_t)ae);
      if (to_dtype((a2 < lo ? lo : a2) / 127.0f, dtype) != s) break;
      ++ae;
    }
    const uint32_t top = ae - 1; /* the largest |x| pattern the run allows */
    ab = ae;
    const float r = 1.0f / s;
    if (!isfinite(s) || !isfinite(r) || (k++ % scale_stride)) continue;
    for (uint32_t mag = 0; mag <= top; ++mag)
      for (uint32_t sg = 0; sg < 2; ++sg) {
        const uint16_t xb = (uint16_t)(mag | (sg << 15));
        const float x = dtype == 0 ? zxo_bf16_to_f32(xb) : zxo_f16_to_f32(xb);
        float w = rintf(to_dtype(x / s, dtype));
        w = isnan(w) ? 0.0f : fminf(fmaxf(w, -127.0f), 127.0f);
        const float q0 = x * r;
        float v = to_dtype(fmaf(fmaf(-q0, s, x), r, q0), dtype);
        v = fminf(fmaxf(v, -127.0f), 127.0f);
        const int8_t g = (int8_t)(f2u(v + 12582912.0f) & 0xFFu);
        bad += (int8_t)w != g;
        ++n;
      }
  }
  if (pairs) *pairs = n;
  return bad;
}

/* Is the Markstein correction of the FP8 encoders needed with dynamic scales?  For every
 * finite bf16 amax a > 0 (s = zxo_fp8_scale(a), r = RN(1 / s)) and every bf16 x with
 * |x| <= a, compares the code of RN(x / s) (the reference) with the code of the plain
 * product RN(x * r).  Every scale_stride-th amax.  Returns the differing pairs; *pairs
 * the number compared. */
int64_t zxo_fp8_product_check(int scale_stride, int64_t *pairs) {
  int64_t bad = 0, n = 0, k = 0;
  for (uint32_t ab = 1; ab < 0x7F80u; ++ab) {
    if (k++ % scale_stride) continue;
    const float a = zxo_bf16_to_f32((uint16_t)ab);
    const float s = zxo_fp8_scale(a);
    const float r = 1.0f / s;
    for (uint32_t mag = 0; mag <= ab; ++mag)
      for (uint32_t sg = 0; sg < 2; ++sg) {
        const float x = zxo_bf16_to_f32((uint16_t)(mag | (sg << 15)));
        bad += zxo_e4m3_encode(x / s) != zxo_e4m3_encode(x * r);
        ++n;
      }
  }
  if (pairs) *pairs = n;
  return bad;
}

/* ---------------------------------------------------------------- Belady */

/* belady.py:39-51 over integer slots: the largest key > -1 among resident slots, ties to
 * the smallest slot (the reference breaks ties by set iteration order, which Python does
 * not fix).  out = {slot, key} or {-1, -1}. */
/* belady.py:44-50 over slots: the largest key > -1 among candidates (resident[i] != 0, or
 * every slot when resident is NULL); ties to the smallest rank (the slot index when rank
 * is NULL), then the smallest slot. */
void zxo_belady_argmax(const int64_t *keys, const uint8_t *resident, const int64_t *rank, int64_t n, int64_t *out) {
  int64_t best = -1, bestk = -1, bestr = 0;
  for (int64_t i = 0; i < n; ++i) {
    if (resident && !resident[i]) continue;
    const int64_t r = rank ? rank[i] : i;
    if (keys[i] > bestk || (best >= 0 && keys[i] == bestk && r < bestr)) {
      bestk = keys[i];
      bestr = r;
      best = i;
    }
  }
  out[0] = best;
  out[1] = best < 0 ? -1 : bestk;
}

/* next_use[i]: next position of trace[i] or ZXO_NEVER; prev_use[i]: previous or -1. */
void zxo_next_use(const int32_t *trace, int64_t n, int32_t n_pages, int32_t *next_use,
                  int32_t *prev_use) {
  int32_t *last = (int32_t *)malloc(sizeof(int32_t) * (size_t)n_pages);
  for (int32_t p = 0; p < n_pages; ++p) last[p] = ZXO_NEVER;
  for (int64_t i = n - 1; i >= 0; --i) {
    next_use[i] = last[trace[i]];
    last[trace[i]] = (int32_t)i;
  }
  for (int32_t p = 0; p < n_pages; ++p) last[p] = -1;
  for (int64_t i = 0; i < n; ++i) {
    prev_use[i] = last[trace[i]];
    last[trace[i]] = (int32_t)i;
  }
  free(last);
}

/* Indexed binary max-heap of resident pages ordered by (key desc, page asc). */
typedef struct {
  int32_t *h;   /* heap array of page ids */
  int32_t *pos; /* page -> index in h, or -1 */
  const int32_t *key;
  int64_t size;
} zxo_heap;

static inline int heap_before(const zxo_heap *H, int32_t a, int32_t b) {
  int32_t ka = H->key[a], kb = H->key[b];
  return ka > kb || (ka == kb && a < b);
}
static void heap_swap(zxo_heap *H, int64_t i, int64_t j) {
  int32_t a = H->h[i], b = H->h[j];
  H->h[i] = b; H->h[j] = a;
  H->pos[b] = (int32_t)i; H->pos[a] = (int32_t)j;
}
static void heap_up(zxo_heap *H, int64_t i) {
  while (i > 0) {
    int64_t p = (i - 1) / 2;
    if (!heap_before(H, H->h[i], H->h[p])) break;
    heap_swap(H, i, p);
    i = p;
  }
}
static void heap_down(zxo_heap *H, int64_t i) {
  for (;;) {
    int64_t l = 2 * i + 1, r = l + 1, m = i;
    if (l < H->size && heap_before(H, H->h[l], H->h[m])) m = l;
    if (r < H->size && heap_before(H, H->h[r], H->h[m])) m = r;
    if (m == i) break;
    heap_swap(H, i, m);
    i = m;
  }
}

/* Belady MIN over a whole trace (include/zenyx_kv.h, zx_belady_simulate): a miss with
 * `capacity` pages resident evicts the page of farthest next use (ties: smallest page),
 * then admits the missed page; a hit moves the page's key to its next use.  The per-miss
 * argmax of belady.py:46-50 is kept exactly, with a heap instead of a linear scan.
 * Returns the number of evictions (entries beyond evict_cap are counted, not stored);
 * stats[0] = misses, stats[1] = hits, stats[2] = final resident count; miss_flags (may be
 * NULL) receives 1 at every miss position. */
int64_t zxo_belady_simulate(const int32_t *trace, int64_t n, int32_t n_pages, int64_t capacity,
                            int32_t *evict_pos, int32_t *evict_page, int64_t evict_cap,
                            int64_t *stats, uint8_t *miss_flags) {
  int32_t *next_use = (int32_t *)malloc(sizeof(int32_t) * (size_t)(n ? n : 1));
  int32_t *prev_use = (int32_t *)malloc(sizeof(int32_t) * (size_t)(n ? n : 1));
  int32_t *key = (int32_t *)malloc(sizeof(int32_t) * (size_t)n_pages);
  zxo_heap H;
  H.h = (int32_t *)malloc(sizeof(int32_t) * (size_t)n_pages);
  H.pos = (int32_t *)malloc(sizeof(int32_t) * (size_t)n_pages);
  H.key = key;
  H.size = 0;
  zxo_next_use(trace, n, n_pages, next_use, prev_use);
  for (int32_t p = 0; p < n_pages; ++p) { H.pos[p] = -1; key[p] = -1; }
  int64_t ev = 0, misses = 0, hits = 0;
  for (int64_t i = 0; i < n; ++i) {
    int32_t p = trace[i];
    if (miss_flags) miss_flags[i] = H.pos[p] < 0;
    if (H.pos[p] >= 0) {
      ++hits;
      key[p] = next_use[i];
      heap_up(&H, H.pos[p]);
      heap_down(&H, H.pos[p]);
      continue;
    }
    ++misses;
    if (H.size >= capacity && H.size > 0) {
      int32_t v = H.h[0];
      heap_swap(&H, 0, H.size - 1);
      H.size--;
      H.pos[v] = -1;
      if (H.size) heap_down(&H, 0);
      if (ev < evict_cap) { evict_pos[ev] = (int32_t)i; evict_page[ev] = v; }
      ++ev;
    }
    key[p] = next_use[i];
    H.h[H.size] = p;
    H.pos[p] = (int32_t)H.size;
    H.size++;
    heap_up(&H, H.size - 1);
  }
  if (stats) { stats[0] = misses; stats[1] = hits; stats[2] = H.size; }
  free(next_use); free(prev_use); free(key); free(H.h); free(H.pos);
  return ev;
}

/* Three-tier Belady hierarchy (README.md:150-154: HBM / DRAM / NVMe, offline-optimal
 * replacement; the reference's T0/T1/T2 manager kv_tiering.py:18-66 with the policy made
 * Belady), simulated explicitly with one heap per tier.  T0 holds at most c0 pages, T1 at
 * most c1; T2 holds everything else.  Access of page p at position i:
 *   * p in T0: hit (src 0), its key becomes its next use;
 *   * otherwise p comes from T1 (src 1, leaving T1), from T2 (src 2: seen before) or is
 *     new (src 3: first access).  If T0 is full, its farthest page r (ties: smallest id)
 *     goes to T1 (v0[i] = r); if T1 then holds more than c1 pages, its farthest page q
 *     (possibly r itself) goes to T2 (v1[i] = q).  p enters T0.
 * src, v0, v1 have n entries (v0/v1 = -1 where nothing moves).  Returns the number of
 * T0 misses.  The hierarchy is exclusive: a page is in exactly one tier. */
int64_t zxo_belady_tiers(const int32_t *trace, int64_t n, int32_t n_pages, int64_t c0, int64_t c1,
                         uint8_t *src, int32_t *v0, int32_t *v1) {
  int32_t *next_use = (int32_t *)malloc(sizeof(int32_t) * (size_t)(n ? n : 1));
  int32_t *prev_use = (int32_t *)malloc(sizeof(int32_t) * (size_t)(n ? n : 1));
  int32_t *key = (int32_t *)malloc(sizeof(int32_t) * (size_t)n_pages);
  uint8_t *seen = (uint8_t *)calloc((size_t)n_pages, 1);
  zxo_heap H0, H1;
  H0.h = (int32_t *)malloc(sizeof(int32_t) * (size_t)n_pages);
  H0.pos = (int32_t *)malloc(sizeof(int32_t) * (size_t)n_pages);
  H1.h = (int32_t *)malloc(sizeof(int32_t) * (size_t)n_pages);
  H1.pos = (int32_t *)malloc(sizeof(int32_t) * (size_t)n_pages);
  H0.key = H1.key = key;
  H0.size = H1.size = 0;
  zxo_next_use(trace, n, n_pages, next_use, prev_use);
  for (int32_t p = 0; p < n_pages; ++p) { H0.pos[p] = H1.pos[p] = -1; key[p] = -1; }
  int64_t misses = 0;
  for (int64_t i = 0; i < n; ++i) {
    const int32_t p = trace[i];
    v0[i] = v1[i] = -1;
    if (H0.pos[p] >= 0) {
      src[i] = 0;
      key[p] = next_use[i];
      heap_up(&H0, H0.pos[p]);
      heap_down(&H0, H0.pos[p]);
      continue;
    }
    ++misses;
    if (H1.pos[p] >= 0) { /* leaves T1: move the last heap entry into its place */
      int64_t at = H1.pos[p];
      heap_swap(&H1, at, H1.size - 1);
      H1.size--;
      H1.pos[p] = -1;
      if (at < H1.size) { heap_up(&H1, at); heap_down(&H1, at); }
      src[i] = 1;
    } else {
      src[i] = seen[p] ? 2 : 3;
    }
    seen[p] = 1;
    if (H0.size >= c0) {
      const int32_t r = H0.h[0];
      heap_swap(&H0, 0, H0.size - 1);
      H0.size--;
      H0.pos[r] = -1;
      if (H0.size) heap_down(&H0, 0);
      v0[i] = r;
      H1.h[H1.size] = r; /* r keeps its key (its next use) */
      H1.pos[r] = (int32_t)H1.size;
      H1.size++;
      heap_up(&H1, H1.size - 1);
      if (H1.size > c1) {
        const int32_t q = H1.h[0];
        heap_swap(&H1, 0, H1.size - 1);
        H1.size--;
        H1.pos[q] = -1;
        if (H1.size) heap_down(&H1, 0);
        v1[i] = q;
      }
    }
    key[p] = next_use[i];
    H0.h[H0.size] = p;
    H0.pos[p] = (int32_t)H0.size;
    H0.size++;
    heap_up(&H0, H0.size - 1);
  }
  free(next_use); free(prev_use); free(key); free(seen);
  free(H0.h); free(H0.pos); free(H1.h); free(H1.pos);
  return misses;
}

/* Ring-attention page accesses over a curriculum of training steps (README.md:162-165,
 * 330, 345: RingDegreeScheduler / CurriculumPhase, "progressive ring degree expansion";
 * code absent).  Step k has ring degree degrees[k] = R and ctx_pages[k] = P pages per
 * layer; layer l's pages are [l * layer_stride, l * layer_stride + P).  Shard s of a
 * layer holds pages [floor(s P / R), floor((s + 1) P / R)) (uneven shards allowed, empty
 * ones too).  Forward of step k: for each layer, for ring step r, for simulated device
 * d, the pages of shard (d - r) mod R in order; backward: the exact reverse of the
 * step's forward (build_ring_timeline, kv_tiering.py:69-73, generalised).  Steps are
 * concatenated; out holds sum_k 2 * L * R_k * P_k ids.  Returns the count. */
int64_t zxo_ring_curriculum_trace(const int32_t *degrees, const int32_t *ctx_pages, int32_t n_steps,
                                  int32_t n_layers, int32_t layer_stride, int32_t *out) {
  int64_t k = 0;
  for (int32_t st = 0; st < n_steps; ++st) {
    const int64_t R = degrees[st], P = ctx_pages[st];
    const int64_t begin = k;
    for (int32_t l = 0; l < n_layers; ++l)
      for (int64_t r = 0; r < R; ++r)
        for (int64_t d = 0; d < R; ++d) {
          const int64_t sh = ((d - r) % R + R) % R;
          const int64_t lo = sh * P / R, hi = (sh + 1) * P / R;
          for (int64_t j = lo; j < hi; ++j) out[k++] = (int32_t)((int64_t)l * layer_stride + j);
        }
    const int64_t n_fwd = k - begin;
    for (int64_t i = 0; i < n_fwd; ++i) out[k + i] = out[k - 1 - i];
    k += n_fwd;
  }
  return k;
}

/* Ring-attention access schedule of degree `ring` on one GPU (kv_tiering.py:69-73
 * generalised).  Layer l owns pages [l*ring*shard_pages, (l+1)*ring*shard_pages), split
 * into `ring` shards of shard_pages pages.  Forward: for each layer, for step s, for each
 * simulated device d, the pages of shard (d - s) mod ring in order.  Backward: the exact
 * reverse of the forward sequence.  out holds 2 * L * ring * ring * shard_pages ids. */
void zxo_ring_trace(int32_t n_layers, int32_t ring, int32_t shard_pages, int32_t *out) {
  int64_t k = 0;
  for (int32_t l = 0; l < n_layers; ++l)
    for (int32_t s = 0; s < ring; ++s)
      for (int32_t d = 0; d < ring; ++d) {
        int32_t shard = ((d - s) % ring + ring) % ring;
        int32_t base = (l * ring + shard) * shard_pages;
        for (int32_t j = 0; j < shard_pages; ++j) out[k++] = base + j;
      }
  for (int64_t i = 0; i < k; ++i) out[k + i] = out[k - 1 - i];
}
