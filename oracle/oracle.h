/*
 * oracle.h — CPU restatement of ds-ocr's quantized-MoE decode arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product library links, loads or calls this code; only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use it, and only as the
 * checker. Every function names the reference file:line whose arithmetic it restates (reference =
 * vislee/ds-ocr C sources). Operation order, fused multiply-adds (the reference is built by GCC with
 * its default -ffp-contract=fast on an FMA target) and tie rules follow the reference exactly, so
 * that integer outputs (codes, indices) and, where stated, float bits match the reference.
 *
 * Pinning status of each function is listed in the header comment of oracle.c.
 */
#ifndef DS_ORACLE_H
#define DS_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------- seeded generators ---------------- */
uint64_t or_splitmix64(uint64_t *state);
/* out[i] = mean + std * N(0,1); SplitMix64 -> Box–Muller in double -> rounded to f32. */
void or_fill_normal_f32(float *out, size_t n, uint64_t seed, float mean, float std_);
/* bf16 = round-to-nearest-even of the f32 sample above. */
void or_fill_normal_bf16(uint16_t *out, size_t n, uint64_t seed, float std_);
/* test_int4.c:39-41 LCG: seed = seed*1103515245+12345; lo+(hi-lo)*((seed&0x7fffffff)/2^31). */
float or_lcg_rand(unsigned *seed, float lo, float hi);
/* test_int4.c:57: bf16 by keeping the top 16 bits of the f32 LCG sample. */
void or_fill_lcg_bf16(uint16_t *out, size_t n, unsigned *seed, float lo, float hi);
void or_fill_lcg_f32(float *out, size_t n, unsigned *seed, float lo, float hi);
uint16_t or_f32_to_bf16_rne(float f);
float or_bf16_to_f32(uint16_t b);

/* ---------------- per-row INT8 quantizer (ds_quantize.c:29-105) ---------------- */
int or_quantize_bf16(int8_t *q, float *scale, float *offset, const uint16_t *W, int out_dim, int in_dim);
int or_quantize_f32(int8_t *q, float *scale, float *offset, const float *W, int out_dim, int in_dim);
void or_dequantize_f32(float *out, const int8_t *q, const float *scale, const float *offset, int out_dim,
                       int in_dim);
float or_quant_error_rms(const int8_t *q, const float *scale, const float *offset, const uint16_t *W,
                         int out_dim, int in_dim);

/* ---------------- INT8 matvec (ds_quantize.c:154-170) ---------------- */
void or_int8_matvec_rows(float *y, const float *x, const int8_t *q, const float *scale, const float *offset,
                         int in_dim, int row_start, int nrows);
/* Brute force: dequantize in double, double dot. */
void or_int8_matvec_f64(double *y, const float *x, const int8_t *q, const float *scale, const float *offset,
                        int in_dim, int out_dim);

/* ---------------- elementwise (ds_kernels.h:296-302, ds_kernels.c:1739-1789, :2464-2492) -------- */
float or_fast_expf(float x);
void or_swiglu_direct(float *out, const float *gate, const float *up, int n);
void or_bf16_truncate(float *a, int n);

/* ---------------- BF16 matvec / argmax in the reference's AVX-512 order ---------------- */
/* ds_bf16_matvec_fused_avx (ds_kernels_avx.c:25-155) applied per thread chunk as
 * ds_bf16_matvec_threaded does (ds_kernels.c:806-828). bias is not supported (NULL in all callers
 * on the path). */
void or_bf16_matvec_avx512(float *y, const float *x, const uint16_t *W, int in_dim, int out_dim,
                           int nthreads);
/* Per-row logits exactly as ds_argmax_bf16_range_avx (ds_kernels_avx.c:157-249) computes them,
 * for the thread chunking of ds_argmax_worker (ds_kernels.c:965-978). */
void or_argmax_logits_avx512(float *logits, const float *x, const uint16_t *W, int in_dim, int out_dim,
                             int nthreads);
/* ds_argmax_matvec_bf16 (ds_kernels.c:1013-1099 with n_exclude=0). */
int or_argmax_bf16(const float *x, const uint16_t *W, int in_dim, int out_dim, int nthreads,
                   float *best_val);
/* ds_bf16_dot_row non-NEON branch (ds_kernels.c:1000-1008). */
float or_bf16_dot_row(const float *x, const uint16_t *W, int in_dim, int row);
/* Greedy token choice of ds_decoder_forward at temperature 0 (ds_moe_decoder.c:1036-1095): argmax,
 * then the repetition penalty over the history (the argmax's own logit once, every other history
 * token's logit from ds_bf16_dot_row), then the n-gram ban; a banned choice falls to the full-logits
 * path (:1105-1237) with logits in ds_bf16_matvec_pub's order, the penalty per history occurrence,
 * banned tokens at -1e30 and the first maximum. *used_full (optional) tells which path chose. */
int or_lm_sample_greedy(const float *x, const uint16_t *W, int in_dim, int vocab, const int *hist, int hist_len,
                        float repeat_penalty, int ngram_n, int nthreads, int *used_full);

/* ---------------- decoder attention block (single-token decode, MHA) ---------------- */
typedef struct {
  int hidden, n_heads, head_dim, kv_stride; /* kv_stride: floats between cache rows (>= n_heads*head_dim) */
  float eps, theta;
  const uint16_t *wq, *wk, *wv, *wo;        /* bf16 [n_heads*head_dim][hidden] x3, [hidden][n_heads*head_dim] */
  const float *input_norm, *post_norm;      /* [hidden] */
  const float *q_norm, *k_norm;             /* [head_dim] or NULL */
} or_attn_t;
void or_rms_norm(float *out, const float *x, const float *w, int n, float eps);
void or_residual_rms_norm(float *out, float *norm_out, const float *x, const float *res, const float *w, int n,
                          float eps);
void or_rope_row(float *cos_out, float *sin_out, int pos, int head_dim, float theta);
void or_apply_rope(float *x, const float *c, const float *sn, int n_heads, int head_dim);
void or_rms_norm_per_head(float *x, const float *w, int n_heads, int head_dim, float eps);
float or_dot_f32(const float *a, const float *b, int n);
int or_attn_ranges(int *rng, int pos, int prefill_len, int window);
void or_attention_decode(float *out, const float *Q, const float *K, const float *V, int n_heads, int head_dim,
                         float scale, int kv_stride, const int *rng, int nrng);
void or_qkv(float *q, float *k, float *v, const float *x, const uint16_t *Wq, const uint16_t *Wk, const uint16_t *Wv,
            int in_dim, int q_dim, int kv_dim, int nthreads);
void or_decoder_attn(float *h, float *n, const float *x, const or_attn_t *A, float *Kc, float *Vc, int pos,
                     int prefill_len, int window, int nthreads);

/* ---------------- router ---------------- */
/* ds_linear without BLAS, seq=1 (ds_kernels.c:639-652): sequential fused chain per row. */
void or_linear_f32(float *y, const float *x, const float *W, int in_dim, int out_dim);
/* ds_moe_top_k (ds_kernels.c:193-243): select on raw scores, then expf softmax over the k. */
void or_moe_top_k(int *idx, float *w, const float *scores, int n_experts, int top_k);
/* moe_forward inline softmax/top-k (ds_moe_decoder.c:157-183): fast-exp softmax over all experts,
 * then select top-k of the probabilities, no renormalisation. scores is overwritten with probs. */
void or_softmax_topk_decode(int *idx, float *w, float *scores, int n_experts, int top_k);

/* ---------------- expert forward ---------------- */
typedef struct {
  const int8_t *q;
  const float *scale;
  const float *offset;
  int out_dim, in_dim;
} or_block_t;

/* ds_expert_forward_fused_int4 (ds_quantize.c:301-321). */
void or_expert_int8(float *out, const float *x, const or_block_t *gu, const or_block_t *dn, int hidden,
                    int inter, int bf16sim);
/* ds_expert_forward_fused (ds_kernels.c:322-357): BF16 weights through the AVX-512 matvec order. */
void or_expert_bf16(float *out, const float *x, const uint16_t *gu, const uint16_t *dn, int hidden,
                    int inter, int bf16sim, int nthreads);
/* ds_expert_combine (ds_kernels.c:359-371). */
void or_expert_combine(float *out, const float *expert_outs, const float *w, int top_k, int hidden);

/* ---------------- MoE layer (decode, ds_moe_decoder.c:131-333 INT8 branches) ---------------- */
enum { OR_ROUTE_DECODE = 0, OR_ROUTE_CFG = 1 };
typedef struct {
  int hidden, inter, n_experts, top_k, shared_inter;
  const float *router_f32;     /* [n_experts, hidden], OR_ROUTE_CFG */
  const uint16_t *router_bf16; /* [n_experts, hidden], OR_ROUTE_DECODE */
  const or_block_t *gu;        /* [n_experts] routed gate_up (2*inter x hidden) */
  const or_block_t *dn;        /* [n_experts] routed down (hidden x inter) */
  or_block_t sgu, sdn;         /* shared gate_up (2*shared_inter x hidden), down (hidden x shared_inter) */
} or_moe_layer_t;

/* out = combine(routed) + shared (the MoE block output; the caller adds the residual). */
void or_moe_layer_decode(float *out, const float *x, const or_moe_layer_t *L, int route_mode, int bf16sim,
                         int nthreads, int *idx_out, float *w_out);

/* ---------------- prefill MoE block (ds_moe_decoder.c:629-809), f64 brute force ---------------- */
/* Routing is taken from the caller (idx/w per token) so that GPU and oracle compare expert math on
 * the same routing; or_prefill_route computes the reference routing separately. */
void or_prefill_route(int *idx, float *w, const float *X, int T, const or_moe_layer_t *L, int route_mode);
void or_prefill_moe_f64(double *out, const float *X, int T, const or_moe_layer_t *L, const int *idx,
                        const float *w);

#ifdef __cplusplus
}
#endif
#endif
