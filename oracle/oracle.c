/*
 * oracle.c — CPU restatement of ds-ocr's quantized-MoE decode arithmetic (test infrastructure).
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this file, as the
 * checker; the product library never links it. Build: oracle/Makefile, with -ffp-contract=off so
 * that the only fused multiply-adds are the explicit fmaf() calls, each placed where GCC contracts
 * the reference expression (-O3, default -ffp-contract=fast, FMA-capable -march).
 *
 * How each function is pinned (tests/test_oracle_*.py):
 *   - quantizer, dequantizer, INT8 matvec, fast-exp, SwiGLU, BF16 truncation, AVX-512-order BF16
 *     matvec/argmax, bf16 dot row, f32 linear, both top-k modes, combine, INT8/BF16 expert, MoE
 *     layer: bit-compared against the reference itself (oracle/_ref, compiled from
 *     /root/reference by oracle/build_ref.sh) on seeded inputs, and against the committed golden
 *     fixtures in tests/golden/ that were written from oracle/_ref.
 *   - quantizer additionally: closed-form invariants (codes in range, row min -> code 0, |deq-w| <=
 *     scale/2 + ulp, constant rows, half-way ties decided away from zero).
 *   - INT8 matvec additionally: f64 brute force through the dequantized matrix.
 *   - argmax additionally: f64 brute force on small vocabularies, NaN rows, duplicate rows, rows
 *     below -1e30.
 *   - or_prefill_moe_f64: the reference prefill runs OpenBLAS sgemm, whose summation order is not
 *     in the reference tree; it is pinned through the decode-path functions above (a one-token
 *     prefill must equal or_moe_layer_decode within f32 rounding) — parity of the sgemm order itself
 *     is unpinned, as documented.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- generators */

uint64_t or_splitmix64(uint64_t *state) {
  uint64_t z = (*state += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

void or_fill_normal_f32(float *out, size_t n, uint64_t seed, float mean, float std_) {
  uint64_t st = seed;
  const double two_pi = 6.283185307179586476925286766559;
  for (size_t i = 0; i < n; i += 2) {
    double u1 = ((double)(or_splitmix64(&st) >> 11) + 1.0) * (1.0 / 9007199254740992.0); /* (0,1] */
    double u2 = (double)(or_splitmix64(&st) >> 11) * (1.0 / 9007199254740992.0);         /* [0,1) */
    double r = sqrt(-2.0 * log(u1));
    double z0 = r * cos(two_pi * u2), z1 = r * sin(two_pi * u2);
    out[i] = (float)((double)mean + (double)std_ * z0);
    if (i + 1 < n) out[i + 1] = (float)((double)mean + (double)std_ * z1);
  }
}

uint16_t or_f32_to_bf16_rne(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return (uint16_t)((u >> 16) | 0x0040u);
  uint32_t lsb = (u >> 16) & 1u;
  u += 0x7FFFu + lsb;
  return (uint16_t)(u >> 16);
}

float or_bf16_to_f32(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

void or_fill_normal_bf16(uint16_t *out, size_t n, uint64_t seed, float std_) {
  const size_t blk = 4096;
  float tmp[4096];
  uint64_t st = seed;
  /* Generate in blocks from one continuous stream so the result equals the f32 fill. */
  const double two_pi = 6.283185307179586476925286766559;
  for (size_t base = 0; base < n; base += blk) {
    size_t m = n - base < blk ? n - base : blk;
    for (size_t i = 0; i < m; i += 2) {
      double u1 = ((double)(or_splitmix64(&st) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
      double u2 = (double)(or_splitmix64(&st) >> 11) * (1.0 / 9007199254740992.0);
      double r = sqrt(-2.0 * log(u1));
      tmp[i] = (float)((double)std_ * (r * cos(two_pi * u2)));
      if (i + 1 < m) tmp[i + 1] = (float)((double)std_ * (r * sin(two_pi * u2)));
    }
    for (size_t i = 0; i < m; i++) out[base + i] = or_f32_to_bf16_rne(tmp[i]);
  }
}

/* test_int4.c:39-41. The expression lo+(hi-lo)*t is contracted by GCC to fma(hi-lo, t, lo). */
float or_lcg_rand(unsigned *seed, float lo, float hi) {
  *seed = *seed * 1103515245u + 12345u;
  float t = (float)(*seed & 0x7fffffffu) / (float)0x7fffffff;
  return fmaf(hi - lo, t, lo);
}

void or_fill_lcg_bf16(uint16_t *out, size_t n, unsigned *seed, float lo, float hi) {
  for (size_t i = 0; i < n; i++) {
    float v = or_lcg_rand(seed, lo, hi);
    uint32_t u;
    memcpy(&u, &v, 4);
    out[i] = (uint16_t)(u >> 16);
  }
}

void or_fill_lcg_f32(float *out, size_t n, unsigned *seed, float lo, float hi) {
  for (size_t i = 0; i < n; i++) out[i] = or_lcg_rand(seed, lo, hi);
}

/* ---------------------------------------------------------------- quantizer */

/* ds_quantize.c:29-47 int8_quantize_row. */
static void quantize_row(int8_t *q, float *row_scale, float *row_offset, const float *v, int n) {
  float mn = 1e30f, mx = -1e30f;
  for (int c = 0; c < n; c++) {
    if (v[c] < mn) mn = v[c];
    if (v[c] > mx) mx = v[c];
  }
  float range = mx - mn;
  float scale = range / 255.0f;
  if (scale < 1e-10f) scale = 1e-10f;
  *row_scale = scale;
  *row_offset = mn;
  float inv = 1.0f / scale;
  for (int c = 0; c < n; c++) {
    float r = roundf((v[c] - mn) * inv);
    /* (int) of a NaN is INT_MIN on x86 (cvttss2si); both clamp to code 0 below. */
    int t = (r != r) ? INT32_MIN : (int)r;
    if (t < 0) t = 0;
    if (t > 255) t = 255;
    q[c] = (int8_t)(t - 128);
  }
}

/* ds_quantize.c:49-81. */
int or_quantize_bf16(int8_t *q, float *scale, float *offset, const uint16_t *W, int out_dim, int in_dim) {
  if (!q || !scale || !offset || !W || out_dim <= 0 || in_dim <= 0) return -1;
  float *row = (float *)malloc((size_t)in_dim * sizeof(float));
  if (!row) return -1;
  for (int r = 0; r < out_dim; r++) {
    const uint16_t *w = W + (size_t)r * in_dim;
    for (int c = 0; c < in_dim; c++) row[c] = or_bf16_to_f32(w[c]);
    quantize_row(q + (size_t)r * in_dim, &scale[r], &offset[r], row, in_dim);
  }
  free(row);
  return 0;
}

/* ds_quantize.c:83-105. */
int or_quantize_f32(int8_t *q, float *scale, float *offset, const float *W, int out_dim, int in_dim) {
  if (!q || !scale || !offset || !W || out_dim <= 0 || in_dim <= 0) return -1;
  for (int r = 0; r < out_dim; r++)
    quantize_row(q + (size_t)r * in_dim, &scale[r], &offset[r], W + (size_t)r * in_dim, in_dim);
  return 0;
}

/* ds_quantize.c:115-125: scale*(q+128)+off, contracted to fma(scale, q+128, off). */
void or_dequantize_f32(float *out, const int8_t *q, const float *scale, const float *offset, int out_dim,
                       int in_dim) {
  for (int r = 0; r < out_dim; r++)
    for (int c = 0; c < in_dim; c++) {
      size_t i = (size_t)r * in_dim + c;
      out[i] = fmaf(scale[r], (float)((int)q[i] + 128), offset[r]);
    }
}

/* ds_quantize.c:127-144: double accumulation of f32 differences. d*d is a float product promoted
 * to double after rounding (ssq += d*d with d float). */
float or_quant_error_rms(const int8_t *q, const float *scale, const float *offset, const uint16_t *W,
                         int out_dim, int in_dim) {
  double ssq = 0, sor = 0;
  for (int r = 0; r < out_dim; r++)
    for (int c = 0; c < in_dim; c++) {
      size_t i = (size_t)r * in_dim + c;
      float deq = fmaf(scale[r], (float)((int)q[i] + 128), offset[r]);
      float orig = or_bf16_to_f32(W[i]);
      float d = orig - deq;
      ssq += (double)(d * d);
      sor += (double)(orig * orig);
    }
  return (sor > 0) ? sqrtf((float)(ssq / sor)) : 0.0f;
}

/* ---------------------------------------------------------------- INT8 matvec */

/* ds_quantize.c:154-170 int8_matvec_generic: two sequential chains per row (GCC keeps this loop
 * scalar); the dot chain is contracted (dot = fma(q+128, x, dot)) and the epilogue
 * scale*dot + off*xs becomes fma(scale, dot, off*xs). Both pinned bit-exactly against oracle/_ref. */
void or_int8_matvec_rows(float *y, const float *x, const int8_t *q, const float *scale, const float *offset,
                         int in_dim, int row_start, int nrows) {
  for (int r = row_start; r < row_start + nrows; r++) {
    const int8_t *qr = q + (size_t)r * in_dim;
    float dot = 0.0f, xs = 0.0f;
    for (int c = 0; c < in_dim; c++) {
      dot = fmaf((float)((int)qr[c] + 128), x[c], dot);
      xs += x[c];
    }
    y[r - row_start] = fmaf(scale[r], dot, offset[r] * xs);
  }
}

void or_int8_matvec_f64(double *y, const float *x, const int8_t *q, const float *scale, const float *offset,
                        int in_dim, int out_dim) {
  for (int r = 0; r < out_dim; r++) {
    double acc = 0;
    for (int c = 0; c < in_dim; c++) {
      double w = (double)scale[r] * (double)((int)q[(size_t)r * in_dim + c] + 128) + (double)offset[r];
      acc += w * (double)x[c];
    }
    y[r] = acc;
  }
}

/* ---------------------------------------------------------------- elementwise */

/* ds_kernels.h:296-302 (Schraudolph). 12102203*x + 1064866805 is contracted to an fma; the
 * float->uint32 conversion is done as the scalar x86 code does (via a 64-bit truncation). The
 * constant 1064866805.0f rounds to 1064866816.0f. */
float or_fast_expf(float x) {
  if (x < -88.0f) return 0.0f;
  if (x > 88.0f) return 1e38f;
  float v = fmaf(12102203.0f, x, 1064866805.0f);
  uint32_t i = (v != v) ? 0u : (uint32_t)(int64_t)v;
  float f;
  memcpy(&f, &i, 4);
  return f;
}

/* ds_kernels.c:1768-1773 (non-Apple branch of ds_swiglu_direct_worker). */
void or_swiglu_direct(float *out, const float *gate, const float *up, int n) {
  for (int j = 0; j < n; j++) out[j] = (gate[j] / (1.0f + or_fast_expf(-gate[j]))) * up[j];
}

/* ds_kernels.c:2484-2490: round-half-up on the bit pattern. */
void or_bf16_truncate(float *a, int n) {
  for (int i = 0; i < n; i++) {
    uint32_t u;
    memcpy(&u, &a[i], 4);
    u = (u + 0x8000u) & 0xFFFF0000u;
    memcpy(&a[i], &u, 4);
  }
}

/* ---------------------------------------------------------------- AVX-512 order BF16 */

/* GCC 11 _mm512_reduce_add_ps tree (avx512fintrin.h __MM512_REDUCE_OP):
 * T3[i] = A[8+i] + A[i]; T6[j] = T3[4+j] + T3[j]; (T6[0]+T6[2]) + (T6[1]+T6[3]). */
static float tree16(const float *A) {
  float T3[8], T6[4];
  for (int i = 0; i < 8; i++) T3[i] = A[8 + i] + A[i];
  for (int j = 0; j < 4; j++) T6[j] = T3[4 + j] + T3[j];
  return (T6[0] + T6[2]) + (T6[1] + T6[3]);
}

/* Rows [o, o+nr) processed as one group with two 16-lane accumulators per row (4-row and 2-row
 * groups of ds_kernels_avx.c:29-128 and :162-228 share this per-row order). add_zero reproduces
 * the "+ (bias ? bias[o] : 0.0f)" of the matvec path. The scalar tail (in_dim % 16 columns) is a
 * fused chain except in the matvec's 4-row group, whose tail GCC vectorizes across the four rows
 * with rounded products (vmulss) added by vaddps: fused_tail = 0 there. */
static void group_rows_2acc(float *out, const float *x, const uint16_t *W, int in_dim, int o, int nr,
                            int add_zero, int fused_tail) {
  for (int j = 0; j < nr; j++) {
    const uint16_t *w = W + (size_t)(o + j) * in_dim;
    float a0[16], a1[16];
    for (int l = 0; l < 16; l++) a0[l] = a1[l] = 0.0f;
    int k = 0;
    for (; k + 32 <= in_dim; k += 32)
      for (int l = 0; l < 16; l++) {
        a0[l] = fmaf(or_bf16_to_f32(w[k + l]), x[k + l], a0[l]);
        a1[l] = fmaf(or_bf16_to_f32(w[k + 16 + l]), x[k + 16 + l], a1[l]);
      }
    for (; k + 16 <= in_dim; k += 16)
      for (int l = 0; l < 16; l++) a0[l] = fmaf(or_bf16_to_f32(w[k + l]), x[k + l], a0[l]);
    float A[16];
    for (int l = 0; l < 16; l++) A[l] = a0[l] + a1[l];
    float s = tree16(A);
    if (add_zero) s = s + 0.0f;
    if (fused_tail)
      for (; k < in_dim; k++) s = fmaf(or_bf16_to_f32(w[k]), x[k], s);
    else
      for (; k < in_dim; k++) s = s + or_bf16_to_f32(w[k]) * x[k];
    out[j] = s;
  }
}

/* Single-row path (ds_kernels_avx.c:131-152 matvec, :230-245 argmax): one 16-lane accumulator. */
static float single_row_1acc(const float *x, const uint16_t *w, int in_dim, int add_zero) {
  float a[16];
  for (int l = 0; l < 16; l++) a[l] = 0.0f;
  int k = 0;
  for (; k + 16 <= in_dim; k += 16)
    for (int l = 0; l < 16; l++) a[l] = fmaf(or_bf16_to_f32(w[k + l]), x[k + l], a[l]);
  float s = tree16(a);
  if (add_zero) s = s + 0.0f;
  for (; k < in_dim; k++) s = fmaf(or_bf16_to_f32(w[k]), x[k], s);
  return s;
}

/* ds_bf16_matvec_fused_avx over one contiguous range (4-row groups, then 2-row, then 1-row). */
static void matvec_range_avx512(float *y, const float *x, const uint16_t *W, int in_dim, int start, int end) {
  int o = start;
  for (; o + 3 < end; o += 4) group_rows_2acc(y + (o - start), x, W, in_dim, o, 4, 1, 0);
  for (; o + 1 < end; o += 2) group_rows_2acc(y + (o - start), x, W, in_dim, o, 2, 1, 1);
  for (; o < end; o++) y[o - start] = single_row_1acc(x, W + (size_t)o * in_dim, in_dim, 1);
}

/* ds_bf16_matvec_threaded / ds_matvec_worker chunking (ds_kernels.c:806-828). */
void or_bf16_matvec_avx512(float *y, const float *x, const uint16_t *W, int in_dim, int out_dim,
                           int nthreads) {
  if (nthreads <= 1) {
    matvec_range_avx512(y, x, W, in_dim, 0, out_dim);
    return;
  }
  int chunk = (out_dim + nthreads - 1) / nthreads;
  for (int t = 0; t < nthreads; t++) {
    int s = t * chunk, e = s + chunk;
    if (e > out_dim) e = out_dim;
    if (s >= e) continue;
    matvec_range_avx512(y + s, x, W, in_dim, s, e);
  }
}

/* ds_argmax_bf16_range_avx row order: 4-row groups, then 1-row remainder (no 2-row path). */
static void argmax_logits_range(float *lg, const float *x, const uint16_t *W, int in_dim, int start, int end) {
  int o = start;
  for (; o + 3 < end; o += 4) group_rows_2acc(lg + o, x, W, in_dim, o, 4, 0, 1);
  for (; o < end; o++) lg[o] = single_row_1acc(x, W + (size_t)o * in_dim, in_dim, 0);
}

void or_argmax_logits_avx512(float *logits, const float *x, const uint16_t *W, int in_dim, int out_dim,
                             int nthreads) {
  if (nthreads <= 1) {
    argmax_logits_range(logits, x, W, in_dim, 0, out_dim);
    return;
  }
  int chunk = (out_dim + nthreads - 1) / nthreads;
  for (int t = 0; t < nthreads; t++) {
    int s = t * chunk, e = s + chunk;
    if (e > out_dim) e = out_dim;
    if (s >= e) continue;
    argmax_logits_range(logits, x, W, in_dim, s, e);
  }
}

/* Strict '>' scan from best=start, best_val=-1e30 per chunk; chunk results merged with strict '>'
 * in thread order (ds_kernels.c:965-978, :1054-1068; ds_kernels_avx.c:157-249). */
int or_argmax_bf16(const float *x, const uint16_t *W, int in_dim, int out_dim, int nthreads, float *best_val) {
  float *lg = (float *)malloc((size_t)out_dim * sizeof(float));
  if (!lg) return -1;
  or_argmax_logits_avx512(lg, x, W, in_dim, out_dim, nthreads);
  int T = nthreads <= 1 ? 1 : nthreads;
  int chunk = (out_dim + T - 1) / T;
  int best = 0;
  float bv = -1e30f;
  for (int t = 0; t < T; t++) {
    int s = t * chunk, e = s + chunk;
    if (e > out_dim) e = out_dim;
    int cb = 0;
    float cv = -1e30f;
    if (s < e) {
      cb = s;
      for (int o = s; o < e; o++)
        if (lg[o] > cv) {
          cv = lg[o];
          cb = o;
        }
    }
    if (t == 0) {
      best = cb;
      bv = cv;
    } else if (cv > bv) {
      bv = cv;
      best = cb;
    }
  }
  free(lg);
  if (best_val) *best_val = bv;
  return best;
}

/* ds_kernels.c:1000-1008: sequential contracted chain from 0. */
float or_bf16_dot_row(const float *x, const uint16_t *W, int in_dim, int row) {
  const uint16_t *w = W + (size_t)row * in_dim;
  float s = 0.0f;
  for (int k = 0; k < in_dim; k++) s = fmaf(or_bf16_to_f32(w[k]), x[k], s);
  return s;
}

/* The reference's penalty (ds_moe_decoder.c:1048, :1058, :1191-1195): divide positive logits,
 * multiply the others. */
static float or_penalize(float v, float rp) { return v > 0 ? v / rp : v * rp; }

/* 1 if the last (n-1)-token prefix of hist occurs at position i with hist[i + n - 1] == tok. */
static int or_ngram_bans(const int *hist, int hist_len, int p, int i, int tok) {
  for (int j = 0; j < p; j++)
    if (hist[i + j] != hist[hist_len - p + j]) return 0;
  return hist[i + p] == tok;
}

/* ds_moe_decoder.c:1036-1095 (fast path) and :1105-1237 (full path, temperature 0). The full
 * path's logits come from ds_bf16_matvec_pub (the reference's branch without an F32 copy of the
 * head; with one it calls a BLAS sgemm, whose summation order is the BLAS library's). */
int or_lm_sample_greedy(const float *x, const uint16_t *W, int in_dim, int vocab, const int *hist, int hist_len,
                        float rp, int ngram_n, int nthreads, int *used_full) {
  int best = or_argmax_bf16(x, W, in_dim, vocab, nthreads, NULL);
  float best_val = or_bf16_dot_row(x, W, in_dim, best);
  if (rp > 1.0f && hist && hist_len > 0) {
    for (int i = 0; i < hist_len; i++)
      if (hist[i] == best) {
        best_val = or_penalize(best_val, rp);
        break;
      }
    for (int i = 0; i < hist_len; i++) {
      int tid = hist[i];
      if (tid >= 0 && tid < vocab && tid != best) {
        float v = or_penalize(or_bf16_dot_row(x, W, in_dim, tid), rp);
        if (v > best_val) {
          best_val = v;
          best = tid;
        }
      }
    }
  }
  int full = 0;
  if (ngram_n > 0 && hist_len >= ngram_n - 1) {
    int p = ngram_n - 1;
    for (int i = 0; i <= hist_len - p - 1 && !full; i++) full = or_ngram_bans(hist, hist_len, p, i, best);
  }
  if (used_full) *used_full = full;
  if (!full) return best;
  float *lg = (float *)malloc((size_t)vocab * sizeof(float));
  if (!lg) return -1;
  or_bf16_matvec_avx512(lg, x, W, in_dim, vocab, nthreads);
  if (rp > 1.0f && hist && hist_len > 0) {
    for (int i = 0; i < hist_len; i++) {
      int tid = hist[i];
      if (tid >= 0 && tid < vocab) lg[tid] = or_penalize(lg[tid], rp);
    }
  }
  if (ngram_n > 0 && hist_len >= ngram_n - 1) {
    int p = ngram_n - 1;
    for (int i = 0; i <= hist_len - p - 1; i++) {
      int m = 1;
      for (int j = 0; j < p && m; j++) m = hist[i + j] == hist[hist_len - p + j];
      if (m) {
        int banned = hist[i + p];
        if (banned >= 0 && banned < vocab) lg[banned] = -1e30f;
      }
    }
  }
  int tok = 0;
  float b = lg[0];
  for (int i = 1; i < vocab; i++)
    if (lg[i] > b) {
      b = lg[i];
      tok = i;
    }
  free(lg);
  return tok;
}

/* ---------------------------------------------------------------- decoder attention block */

/* Sum of squares as the AVX-512 branches of ds_rms_norm / ds_rms_norm_per_head compute it
 * (ds_kernels.c:1387-1440, :1473-1500): 16 lanes of fused squares over the leading multiple of 16,
 * the reduce tree, then the tail added with fused squares (GCC contracts the scalar line). */
static float or_sumsq16(const float *x, int n) {
  float acc[16];
  for (int l = 0; l < 16; l++) acc[l] = 0.0f;
  int i = 0;
  for (; i + 16 <= n; i += 16)
    for (int l = 0; l < 16; l++) acc[l] = fmaf(x[i + l], x[i + l], acc[l]);
  float s = tree16(acc);
  for (; i < n; i++) s = fmaf(x[i], x[i], s);
  return s;
}

/* ds_rms_norm for one row, AVX-512 branch: out = (x*w)*r on the leading multiple of 16, then
 * (x*r)*w on the tail, r = 1/sqrtf(sum/n + eps). */
void or_rms_norm(float *out, const float *x, const float *w, int n, float eps) {
  float r = 1.0f / sqrtf(or_sumsq16(x, n) / n + eps);
  int j = 0;
  for (; j + 16 <= n; j += 16)
    for (int l = 0; l < 16; l++) out[j + l] = (x[j + l] * w[j + l]) * r;
  for (; j < n; j++) out[j] = x[j] * r * w[j];
}

/* ds_residual_rms_norm, AVX-512 branch (ds_kernels.c:1544-1600): out = x + res (rounded), the
 * squares of out summed as above, norm_out as or_rms_norm. */
void or_residual_rms_norm(float *out, float *norm_out, const float *x, const float *res, const float *w, int n,
                          float eps) {
  for (int i = 0; i < n; i++) out[i] = x[i] + res[i];
  or_rms_norm(norm_out, out, w, n, eps);
}

/* ds_compute_rope_neox for one position (ds_kernels.c:2407-2424): the host libm's powf, cosf, sinf. */
void or_rope_row(float *cos_out, float *sin_out, int pos, int head_dim, float theta) {
  int half = head_dim / 2;
  for (int d = 0; d < half; d++) {
    float freq = 1.0f / powf(theta, (float)(2 * d) / (float)head_dim);
    float angle = (float)pos * freq;
    cos_out[d] = cos_out[d + half] = cosf(angle);
    sin_out[d] = sin_out[d + half] = sinf(angle);
  }
}

/* ds_apply_rope_neox for one token (ds_kernels.c:2426-2455); GCC fuses the first product of each
 * line into the subtraction / addition (fmaf(x1, c, -(x2*s)) and fmaf(x1, s, x2*c)). */
void or_apply_rope(float *x, const float *c, const float *sn, int n_heads, int head_dim) {
  int half = head_dim / 2;
  for (int h = 0; h < n_heads; h++) {
    float *v = x + h * head_dim;
    for (int d = 0; d < half; d++) {
      float x1 = v[d], x2 = v[d + half];
      v[d] = fmaf(x1, c[d], -(x2 * sn[d]));
      v[d + half] = fmaf(x1, sn[d + half], x2 * c[d + half]);
    }
  }
}

/* ds_rms_norm_per_head, AVX-512 branch (in place). */
void or_rms_norm_per_head(float *x, const float *w, int n_heads, int head_dim, float eps) {
  for (int h = 0; h < n_heads; h++) or_rms_norm(x + h * head_dim, x + h * head_dim, w, head_dim, eps);
}

/* ds_dot_f32_avx, AVX-512 branch (ds_kernels_avx.c:357-377): four 16-lane accumulators over
 * 64-element blocks, added pairwise, 16-element steps, the reduce tree, fused tail. */
float or_dot_f32(const float *a, const float *b, int n) {
  float a0[16], a1[16], a2[16], a3[16], acc[16];
  for (int l = 0; l < 16; l++) a0[l] = a1[l] = a2[l] = a3[l] = 0.0f;
  int i = 0;
  for (; i + 64 <= n; i += 64)
    for (int l = 0; l < 16; l++) {
      a0[l] = fmaf(a[i + l], b[i + l], a0[l]);
      a1[l] = fmaf(a[i + 16 + l], b[i + 16 + l], a1[l]);
      a2[l] = fmaf(a[i + 32 + l], b[i + 32 + l], a2[l]);
      a3[l] = fmaf(a[i + 48 + l], b[i + 48 + l], a3[l]);
    }
  for (int l = 0; l < 16; l++) acc[l] = (a0[l] + a1[l]) + (a2[l] + a3[l]);
  for (; i + 16 <= n; i += 16)
    for (int l = 0; l < 16; l++) acc[l] = fmaf(a[i + l], b[i + l], acc[l]);
  float s = tree16(acc);
  for (; i < n; i++) s = fmaf(a[i], b[i], s);
  return s;
}

/* One head of single-token MHA decode attention over the KV rows in [r0, r1) then [r2, r3)
 * (ds_kernels.c:2124-2160 causal: one range; :2270-2330 R-SWA: reference then window): online
 * softmax with ds_fast_expf; on a new maximum sum_e = fma(sum_e, corr, 1) and o = o*corr + v
 * (ds_vec_scale_add), otherwise sum_e += wt and o += wt*v (ds_vec_axpy_inplace); then o *= 1/sum_e. */
static void or_attn_head(float *o, const float *q, const float *kh, const float *vh, int head_dim, float scale,
                         int kv_stride, const int *rng, int nrng) {
  float max_s = -1e30f, sum_e = 0.0f;
  for (int d = 0; d < head_dim; d++) o[d] = 0.0f;
  for (int r = 0; r < nrng; r++)
    for (int j = rng[2 * r]; j < rng[2 * r + 1]; j++) {
      const float *kr = kh + (size_t)j * kv_stride, *vr = vh + (size_t)j * kv_stride;
      float score = or_dot_f32(q, kr, head_dim) * scale;
      if (score > max_s) {
        float corr = or_fast_expf(max_s - score);
        sum_e = fmaf(sum_e, corr, 1.0f);  /* GCC contracts the reference's sum_e * corr + 1.0f */
        for (int d = 0; d < head_dim; d++) o[d] = fmaf(o[d], corr, vr[d]);
        max_s = score;
      } else {
        float wt = or_fast_expf(score - max_s);
        sum_e += wt;
        for (int d = 0; d < head_dim; d++) o[d] = fmaf(vr[d], wt, o[d]);
      }
    }
  if (sum_e > 0.0f) {
    float inv = 1.0f / sum_e;
    for (int d = 0; d < head_dim; d++) o[d] = o[d] * inv;
  }
}

/* The KV ranges decoder_layer_forward attends to for the token at cache position pos
 * (ds_moe_decoder.c:396-423): [0, pos+1), or with R-SWA (window > 0, pos >= prefill_len) the
 * reference tokens [0, prefill_len) and the window [max(prefill_len, pos+1-window), pos+1) when
 * they do not touch. Returns the number of ranges. */
int or_attn_ranges(int *rng, int pos, int prefill_len, int window) {
  int kv = pos + 1;
  if (window > 0 && pos >= prefill_len) {
    int ws = prefill_len > kv - window ? prefill_len : kv - window;
    if (ws > prefill_len) {
      rng[0] = 0;
      rng[1] = prefill_len;
      rng[2] = ws;
      rng[3] = kv;
      return 2;
    }
  }
  rng[0] = 0;
  rng[1] = kv;
  return 1;
}

void or_attention_decode(float *out, const float *Q, const float *K, const float *V, int n_heads, int head_dim,
                         float scale, int kv_stride, const int *rng, int nrng) {
  for (int h = 0; h < n_heads; h++)
    or_attn_head(out + h * head_dim, Q + h * head_dim, K + h * head_dim, V + h * head_dim, head_dim, scale,
                 kv_stride, rng, nrng);
}

/* ds_linear_nobias_bf16_qkv (ds_kernels.c:844-915): rows of [q; k; v] chunked over the threads,
 * each thread's part of each matrix one ds_bf16_matvec_fused range. */
void or_qkv(float *q, float *k, float *v, const float *x, const uint16_t *Wq, const uint16_t *Wk, const uint16_t *Wv,
            int in_dim, int q_dim, int kv_dim, int nthreads) {
  if (nthreads <= 1) {
    matvec_range_avx512(q, x, Wq, in_dim, 0, q_dim);
    matvec_range_avx512(k, x, Wk, in_dim, 0, kv_dim);
    matvec_range_avx512(v, x, Wv, in_dim, 0, kv_dim);
    return;
  }
  int total = q_dim + 2 * kv_dim, chunk = (total + nthreads - 1) / nthreads;
  int ends[3] = {q_dim, q_dim + kv_dim, total};
  float *ys[3] = {q, k, v};
  const uint16_t *Ws[3] = {Wq, Wk, Wv};
  for (int t = 0; t < nthreads; t++) {
    int start = t * chunk, end = start + chunk;
    if (end > total) end = total;
    if (start >= end) continue;
    for (int m = 0; m < 3; m++) {
      int base = m ? ends[m - 1] : 0;
      int s = start > base ? start - base : 0;
      int e = (end < ends[m] ? end : ends[m]) - base;
      if (s < e) matvec_range_avx512(ys[m] + s, x, Ws[m], in_dim, s, e);
    }
  }
}

/* The attention half of decoder_layer_forward for one token (ds_moe_decoder.c:339-431, MHA):
 * x_norm = RMSNorm(x); q, k, v; optional per-head q/k norms; RoPE at pos; k and v stored in the
 * caches' row pos; attention over or_attn_ranges; h = x + Wo·attn; n = RMSNorm(h). h and n are
 * what the MLP and its residual take. */
void or_decoder_attn(float *h, float *n, const float *x, const or_attn_t *A, float *Kc, float *Vc, int pos,
                     int prefill_len, int window, int nthreads) {
  int H = A->hidden, qd = A->n_heads * A->head_dim;
  float *xn = (float *)malloc((size_t)H * 4), *q = (float *)malloc((size_t)qd * 4);
  float *k = (float *)malloc((size_t)qd * 4), *v = (float *)malloc((size_t)qd * 4);
  float *att = (float *)malloc((size_t)qd * 4), *proj = (float *)malloc((size_t)H * 4);
  float *c = (float *)malloc((size_t)A->head_dim * 4), *sn = (float *)malloc((size_t)A->head_dim * 4);
  or_rms_norm(xn, x, A->input_norm, H, A->eps);
  or_qkv(q, k, v, xn, A->wq, A->wk, A->wv, H, qd, qd, nthreads);
  if (A->q_norm) or_rms_norm_per_head(q, A->q_norm, A->n_heads, A->head_dim, A->eps);
  if (A->k_norm) or_rms_norm_per_head(k, A->k_norm, A->n_heads, A->head_dim, A->eps);
  or_rope_row(c, sn, pos, A->head_dim, A->theta);
  or_apply_rope(q, c, sn, A->n_heads, A->head_dim);
  or_apply_rope(k, c, sn, A->n_heads, A->head_dim);
  memcpy(Kc + (size_t)pos * A->kv_stride, k, (size_t)qd * 4);
  memcpy(Vc + (size_t)pos * A->kv_stride, v, (size_t)qd * 4);
  int rng[4];
  int nr = or_attn_ranges(rng, pos, prefill_len, window);
  or_attention_decode(att, q, Kc, Vc, A->n_heads, A->head_dim, 1.0f / sqrtf((float)A->head_dim), A->kv_stride,
                      rng, nr);
  or_bf16_matvec_avx512(proj, att, A->wo, qd, H, nthreads);
  or_residual_rms_norm(h, n, x, proj, A->post_norm, H, A->eps);
  free(xn), free(q), free(k), free(v), free(att), free(proj), free(c), free(sn);
}

/* ---------------------------------------------------------------- router */

/* ds_linear without USE_BLAS (ds_kernels.c:639-652), as GCC 11 -O3 (AVX-512) compiles its inner
 * loop: sum starts at 0 (b == NULL); while 16 or more terms remain of the leading multiple of 16,
 * products are rounded (vmulps) and added in index order; then, if 8 or more remain, 8 more rounded
 * products in order; the last terms are fused (vfmadd231ss). Pinned against oracle/_ref. */
void or_linear_f32(float *y, const float *x, const float *W, int in_dim, int out_dim) {
  for (int o = 0; o < out_dim; o++) {
    const float *w = W + (size_t)o * in_dim;
    float s = 0.0f;
    int i = 0;
    if (in_dim >= 16) {
      int m = in_dim & ~15;
      for (; i < m; i++) s = s + x[i] * w[i];
    }
    if (in_dim - i >= 8) {
      int m = i + 8;
      for (; i < m; i++) s = s + x[i] * w[i];
    }
    for (; i < in_dim; i++) s = fmaf(x[i], w[i], s);
    y[o] = s;
  }
}

/* ds_kernels.c:193-243. */
void or_moe_top_k(int *idx, float *w, const float *scores, int n_experts, int top_k) {
  int sel[64];
  float ss[64];
  int ns = 0;
  for (int k = 0; k < top_k; k++) {
    int best = -1;
    float bs = -1e30f;
    for (int e = 0; e < n_experts; e++) {
      int already = 0;
      for (int j = 0; j < ns; j++)
        if (sel[j] == e) {
          already = 1;
          break;
        }
      if (already) continue;
      if (scores[e] > bs) {
        bs = scores[e];
        best = e;
      }
    }
    if (best >= 0) {
      sel[ns] = best;
      ss[ns] = bs;
      ns++;
    }
  }
  float mx = -1e30f;
  for (int k = 0; k < ns; k++)
    if (ss[k] > mx) mx = ss[k];
  float sum = 0.0f;
  for (int k = 0; k < ns; k++) {
    ss[k] = expf(ss[k] - mx);
    sum += ss[k];
  }
  float inv = 1.0f / sum;
  for (int k = 0; k < top_k; k++) {
    if (k < ns) {
      idx[k] = sel[k];
      w[k] = ss[k] * inv;
    } else {
      idx[k] = 0;
      w[k] = 0.0f;
    }
  }
}

/* ds_moe_decoder.c:157-183. */
void or_softmax_topk_decode(int *idx, float *w, float *scores, int n_experts, int top_k) {
  float mx = -1e30f;
  for (int e = 0; e < n_experts; e++)
    if (scores[e] > mx) mx = scores[e];
  float sum = 0.0f;
  for (int e = 0; e < n_experts; e++) {
    scores[e] = or_fast_expf(scores[e] - mx);
    sum += scores[e];
  }
  float inv = 1.0f / sum;
  for (int e = 0; e < n_experts; e++) scores[e] *= inv;
  for (int k = 0; k < top_k; k++) {
    int best = -1;
    float bs = -1e30f;
    for (int e = 0; e < n_experts; e++) {
      int already = 0;
      for (int j = 0; j < k; j++)
        if (idx[j] == e) {
          already = 1;
          break;
        }
      if (already) continue;
      if (scores[e] > bs) {
        bs = scores[e];
        best = e;
      }
    }
    idx[k] = best;
    w[k] = bs;
  }
}

/* ---------------------------------------------------------------- experts */

void or_expert_int8(float *out, const float *x, const or_block_t *gu, const or_block_t *dn, int hidden,
                    int inter, int bf16sim) {
  float *gup = (float *)malloc((size_t)2 * inter * sizeof(float));
  float *h = (float *)malloc((size_t)inter * sizeof(float));
  or_int8_matvec_rows(gup, x, gu->q, gu->scale, gu->offset, gu->in_dim, 0, gu->out_dim);
  if (bf16sim) or_bf16_truncate(gup, 2 * inter);
  or_swiglu_direct(h, gup, gup + inter, inter);
  if (bf16sim) or_bf16_truncate(h, inter);
  or_int8_matvec_rows(out, h, dn->q, dn->scale, dn->offset, dn->in_dim, 0, dn->out_dim);
  if (bf16sim) or_bf16_truncate(out, hidden);
  free(gup);
  free(h);
}

void or_expert_bf16(float *out, const float *x, const uint16_t *gu, const uint16_t *dn, int hidden, int inter,
                    int bf16sim, int nthreads) {
  float *gup = (float *)malloc((size_t)2 * inter * sizeof(float));
  float *h = (float *)malloc((size_t)inter * sizeof(float));
  or_bf16_matvec_avx512(gup, x, gu, hidden, 2 * inter, nthreads);
  if (bf16sim) or_bf16_truncate(gup, 2 * inter);
  or_swiglu_direct(h, gup, gup + inter, inter);
  if (bf16sim) or_bf16_truncate(h, inter);
  or_bf16_matvec_avx512(out, h, dn, inter, hidden, nthreads);
  if (bf16sim) or_bf16_truncate(out, hidden);
  free(gup);
  free(h);
}

/* ds_kernels.c:359-371: out = 0; out[i] += w*e[i] (contracted), k in order. */
void or_expert_combine(float *out, const float *expert_outs, const float *w, int top_k, int hidden) {
  for (int i = 0; i < hidden; i++) out[i] = 0.0f;
  for (int k = 0; k < top_k; k++)
    for (int i = 0; i < hidden; i++) out[i] = fmaf(w[k], expert_outs[(size_t)k * hidden + i], out[i]);
}

/* ---------------------------------------------------------------- MoE layer */

static void route(int *idx, float *w, const float *x, const or_moe_layer_t *L, int mode, int nthreads) {
  float scores[64];
  if (mode == OR_ROUTE_CFG) {
    or_linear_f32(scores, x, L->router_f32, L->hidden, L->n_experts);
    or_moe_top_k(idx, w, scores, L->n_experts, L->top_k);
  } else {
    or_bf16_matvec_avx512(scores, x, L->router_bf16, L->hidden, L->n_experts, nthreads);
    or_softmax_topk_decode(idx, w, scores, L->n_experts, L->top_k);
  }
}

void or_moe_layer_decode(float *out, const float *x, const or_moe_layer_t *L, int route_mode, int bf16sim,
                         int nthreads, int *idx_out, float *w_out) {
  int H = L->hidden, K = L->top_k;
  int idx[64];
  float w[64];
  route(idx, w, x, L, route_mode, nthreads);
  float *eo = (float *)calloc((size_t)K * H, sizeof(float));
  float *sh = (float *)malloc((size_t)H * sizeof(float));
  for (int k = 0; k < K; k++) {
    if (idx[k] < 0) continue; /* all-NaN scores: the reference would index experts[-1] */
    or_expert_int8(eo + (size_t)k * H, x, &L->gu[idx[k]], &L->dn[idx[k]], H, L->inter, bf16sim);
  }
  or_expert_combine(out, eo, w, K, H);
  or_expert_int8(sh, x, &L->sgu, &L->sdn, H, L->shared_inter, bf16sim);
  for (int i = 0; i < H; i++) out[i] = out[i] + sh[i];
  if (idx_out)
    for (int k = 0; k < K; k++) idx_out[k] = idx[k];
  if (w_out)
    for (int k = 0; k < K; k++) w_out[k] = w[k];
  free(eo);
  free(sh);
}

/* ---------------------------------------------------------------- prefill */

/* ds_moe_decoder.c:643-686. CFG mode: f32 router + ds_moe_top_k. DECODE mode (the reference
 * prefill's own routing): scores from the bf16 router widened to f32 through ds_linear, then the
 * fast-exp softmax over all experts and top-k without renormalisation. */
void or_prefill_route(int *idx, float *w, const float *X, int T, const or_moe_layer_t *L, int route_mode) {
  int H = L->hidden, E = L->n_experts, K = L->top_k;
  float *Wf = NULL;
  if (route_mode != OR_ROUTE_CFG) {
    Wf = (float *)malloc((size_t)E * H * sizeof(float));
    for (size_t i = 0; i < (size_t)E * H; i++) Wf[i] = or_bf16_to_f32(L->router_bf16[i]);
  }
  for (int t = 0; t < T; t++) {
    float scores[64];
    if (route_mode == OR_ROUTE_CFG) {
      or_linear_f32(scores, X + (size_t)t * H, L->router_f32, H, E);
      or_moe_top_k(idx + (size_t)t * K, w + (size_t)t * K, scores, E, K);
    } else {
      or_linear_f32(scores, X + (size_t)t * H, Wf, H, E);
      or_softmax_topk_decode(idx + (size_t)t * K, w + (size_t)t * K, scores, E, K);
    }
  }
  free(Wf);
}

/* One expert for one token in f64 from f32-dequantized weights (ds_int4_dequantize_f32 form);
 * SwiGLU in f32 with the fast exp, as the reference applies it to f32 gate/up. */
static void expert_f64(double *out, const float *x, const or_block_t *gu, const or_block_t *dn, int H, int I) {
  float *g = (float *)malloc((size_t)2 * I * sizeof(float));
  float *h = (float *)malloc((size_t)I * sizeof(float));
  for (int r = 0; r < 2 * I; r++) {
    double acc = 0;
    const int8_t *q = gu->q + (size_t)r * H;
    for (int c = 0; c < H; c++)
      acc += (double)fmaf(gu->scale[r], (float)((int)q[c] + 128), gu->offset[r]) * (double)x[c];
    g[r] = (float)acc;
  }
  or_swiglu_direct(h, g, g + I, I);
  for (int r = 0; r < H; r++) {
    double acc = 0;
    const int8_t *q = dn->q + (size_t)r * I;
    for (int c = 0; c < I; c++)
      acc += (double)fmaf(dn->scale[r], (float)((int)q[c] + 128), dn->offset[r]) * (double)h[c];
    out[r] = acc;
  }
  free(g);
  free(h);
}

void or_prefill_moe_f64(double *out, const float *X, int T, const or_moe_layer_t *L, const int *idx,
                        const float *w) {
  int H = L->hidden, K = L->top_k;
  double *tmp = (double *)malloc((size_t)H * sizeof(double));
  for (int t = 0; t < T; t++) {
    double *o = out + (size_t)t * H;
    const float *x = X + (size_t)t * H;
    for (int i = 0; i < H; i++) o[i] = 0.0;
    for (int k = 0; k < K; k++) {
      int e = idx[(size_t)t * K + k];
      if (e < 0) continue;
      expert_f64(tmp, x, &L->gu[e], &L->dn[e], H, L->inter);
      for (int i = 0; i < H; i++) o[i] += (double)w[(size_t)t * K + k] * tmp[i];
    }
    expert_f64(tmp, x, &L->sgu, &L->sdn, H, L->shared_inter);
    for (int i = 0; i < H; i++) o[i] += tmp[i];
  }
  free(tmp);
}
