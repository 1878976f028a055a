// k_core.h — launcher entry points of the gfx950 kernels (C linkage, device pointers, one stream).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define DSH_ROUTE_DECODE 0 /* bf16 router, fast-exp softmax over all experts, top-k, no renorm */
#define DSH_ROUTE_CFG 1    /* f32 router, top-k on raw scores, expf softmax over the k (renorm) */

#ifdef __cplusplus
extern "C" {
#endif

hipError_t dsh_launch_quantize_bf16(const uint16_t *W, int8_t *q, float *scale, float *offset, int out_dim, int in_dim,
                                    hipStream_t s);
hipError_t dsh_launch_quantize_f32(const float *W, int8_t *q, float *scale, float *offset, int out_dim, int in_dim,
                                   hipStream_t s);
/* Quantizes into a code array and an interleaved (scale, offset) array. */
hipError_t dsh_launch_quantize_bf16_so(const uint16_t *W, int8_t *q, float *so, int out_dim, int in_dim, hipStream_t s);
/* work: >= 2*1024 + 2 doubles; work[0] = Σ(w-deq)^2, work[1] = Σw^2. */
hipError_t dsh_launch_quant_rms(const int8_t *q, const float *scale, const float *offset, const uint16_t *W,
                                int out_dim, int in_dim, double *work, hipStream_t s);
hipError_t dsh_launch_gemm_bf16w(const float *X, const uint16_t *W, float *Y, int M, int K, int N, hipStream_t s);
/* Reads bytes (a multiple of 16) of src once; sink: [1024] words, written only on an impossible
 * value. The roofline reference for the HBM-bound kernels. */
hipError_t dsh_launch_stream_read(const void *src, size_t bytes, unsigned *sink, hipStream_t s);
hipError_t dsh_launch_fill_normal_bf16(uint16_t *dst, size_t n, uint64_t seed, float std_, hipStream_t s);
hipError_t dsh_launch_fill_normal_f32(float *dst, size_t n, uint64_t seed, float mean, float std_, hipStream_t s);
hipError_t dsh_launch_dequantize(const int8_t *q, const float *scale, const float *offset, float *out, int out_dim,
                                 int in_dim, hipStream_t s);
/* The reference's own per-row order (bit-identical to int8_matvec_generic); in_dim <= 16384. */
hipError_t dsh_launch_int8_matvec_exact(const int8_t *q, const float *scale, const float *offset, const float *x,
                                        float *y, int in_dim, int row_start, int nrows, hipStream_t s);
hipError_t dsh_launch_int8_matvec(const int8_t *q, const float *scale, const float *offset, const float *x, float *y,
                                  int in_dim, int row_start, int nrows, hipStream_t s);
hipError_t dsh_launch_swiglu(float *out, const float *g, const float *u, size_t n, hipStream_t s);
hipError_t dsh_launch_bf16_trunc(float *a, size_t n, hipStream_t s);
hipError_t dsh_launch_vec_add(float *dst, const float *a, const float *b, int n, hipStream_t s);
hipError_t dsh_launch_expert_combine(float *out, const float *eo, const float *w, int top_k, int hidden,
                                     hipStream_t s);
hipError_t dsh_launch_split_swiglu(float *h, const float *gu, int inter, int bf16sim, hipStream_t s);
/* One expert (gate_up, SwiGLU, down) in the reference's per-row order in one launch: the gate
 * blocks write h into hbuf (I device 64-bit words) tagged with epoch, which must differ from the
 * previous launch's on the same hbuf; the down blocks wait (bounded by spin polls; *derr set on
 * expiry) until every word carries it. xcache (optional, H device floats): receives x for later
 * calls on the same input. done (optional): down block d stores epoch to done[d] (system scope,
 * release) after its output rows. 0 blocks: shape not supported. */
int dsh_expert_exact_blocks(int H, int I);
hipError_t dsh_launch_expert_exact(const int8_t *gq, const float *gs, const float *go, const int8_t *dq, const float *dsc,
                                   const float *dof, const float *x, float *xcache, unsigned long long *hbuf, float *y,
                                   unsigned *done, int H, int I, unsigned epoch, int bf16sim, int spin, int *derr,
                                   hipStream_t s);
/* Down blocks of dsh_launch_expert_exact (one completion word each when done is given). */
int dsh_expert_exact_down_blocks(int H);
hipError_t dsh_launch_bf16_matvec_avx(const uint16_t *W, const float *x, const float *bias, float *y, int in_dim,
                                      int out_dim, int nthreads, hipStream_t s);
/* The _done variants: block b stores epoch to done[b] (system scope, release) after its outputs, for
 * a host polling those words (dsr_pin_out_done); _blocks gives the number of words. */
int dsh_bf16_matvec_avx_blocks(int out_dim);
hipError_t dsh_launch_bf16_matvec_avx_done(const uint16_t *W, const float *x, const float *bias, float *y, int in_dim,
                                           int out_dim, int nthreads, unsigned *done, unsigned epoch, hipStream_t s);
int dsh_vec_add_blocks(int n);
hipError_t dsh_launch_vec_add_done(float *dst, const float *a, const float *b, int n, unsigned *done, unsigned epoch,
                                   hipStream_t s);
int dsh_expert_combine_blocks(int hidden);
hipError_t dsh_launch_expert_combine_done(float *out, const float *eo, const float *w, int top_k, int hidden,
                                          unsigned *done, unsigned epoch, hipStream_t s);
int dsh_argmax_avx_blocks(int out_dim);
/* Candidate keys in the file-scope device array of k_core.hip: DSH_STATIC_CAND entries (out_dim up
 * to 64 * DSH_STATIC_CAND rows). _init looks its address up for the current device (once per
 * device; 0 or -1); dsh_static_scratch returns the current device's address (NULL before _init). */
#define DSH_STATIC_CAND 4096
int dsh_static_scratch_init(void);
unsigned long long *dsh_static_scratch(void);
hipError_t dsh_launch_argmax_avx(const uint16_t *W, const float *x, unsigned long long *cand, float *logits,
                                 int in_dim, int out_dim, int nthreads, int *out_idx, float *out_val, hipStream_t s);
hipError_t dsh_launch_argmax_avx_partial(const uint16_t *W, const float *x, unsigned long long *cand, float *logits,
                                         int in_dim, int out_dim, int chunk, hipStream_t s);
/* lg, lg2: [out_dim] scratch; excl: device ids. */
hipError_t dsh_launch_argmax_excluding(const uint16_t *W, const float *x, unsigned long long *cand, float *lg,
                                       float *lg2, int in_dim, int out_dim, int nthreads, const int *excl, int n_excl,
                                       int *out_idx, hipStream_t s);
hipError_t dsh_launch_bf16_dot_row(const uint16_t *W, const float *x, int in_dim, int row, float *out, hipStream_t s);
hipError_t dsh_launch_linear_f32_exact(const float *W, const float *x, float *y, int in_dim, int out_dim,
                                       hipStream_t s);
hipError_t dsh_launch_topk(const float *scores, int n, int k, int mode, int *idx, float *w, hipStream_t s);

/* ---- decode MoE layer (k_moe.hip) ---- */
typedef struct {
  const int8_t *gu_q;   /* [E][2I][H] routed gate_up codes (gate rows, then up rows, per expert) */
  const float *gu_so;   /* [E][2I] (scale, offset) */
  const int8_t *dn_q;   /* [E][H][I] routed down codes */
  const float *dn_so;   /* [E][H] */
  const int8_t *sgu_q;  /* [2SI][H] shared gate_up */
  const float *sgu_so;  /* [2SI] */
  const int8_t *sdn_q;  /* [H][SI] shared down */
  const float *sdn_so;  /* [H] */
  const float *router_f32;     /* [E][H] */
  const float *router_f32_t;   /* [H][E]: the same f32 router transposed (partial scores read rows) */
  const uint16_t *router_bf16; /* [E][H] */
  const float *router_norm;    /* [E]: ||router_f32 row||_2, rounded up (bounds on score rounding) */
  int H, I, E, K, SI;
} dsh_layer_t;

/* Certified CFG routing (dsh_cert.h): counters and an optional log of the routings. stats[0] counts
 * the routings made, stats[1] those whose selection needed ds_linear's order recomputed (the bound
 * could not separate the ranks). The log (a test aid) holds log[0] = entries written, then from word
 * 64 entries of DSH_RLOG_STRIDE(H) words: idx[8], w[8] (f32 bits), flags (bit 0: recomputed in
 * ds_linear's order; bit 1: the one-kernel layer's verdict replaced the speculative selection),
 * tag, 14 spare words, then the H floats of the routed input. One entry per routing, written by one
 * thread per layer launch. */
typedef struct {
  unsigned long long *stats;
  int *log;
  int log_cap;
  int tag;
} dsh_rcert_t;
#define DSH_RLOG_STRIDE(H) (32 + (H))

/* Work buffers of one decode layer. */
typedef struct {
  float *scores; /* [E] router scores */
  int *idx;      /* [K] selected experts */
  float *w;      /* [K] routing weights */
  float *h;      /* [K*I + SI] SwiGLU outputs (routed slots, then shared) */
  float *eo;     /* [K+1][H] expert outputs: routed slots, then shared (bf16 simulation) */
} dsh_layer_work_t;

/* ---- prefill MoE block (k_prefill.hip) ---- */
int dsh_pf_supported(const dsh_layer_t *L);
size_t dsh_pf_workspace_bytes(const dsh_layer_t *L, int T);
/* Outside stream capture: sizes the fused GEMM grid and checks (once) that its blocks cover every
 * XCD. force: 1 / 0 selects the fused or the two-kernel path, -1 the check's choice, -2 keeps the
 * current choice. */
hipError_t dsh_pf_init(int force);
int dsh_pf_fused(void);
/* 1 if a probe grid's blocks were dealt evenly over all 8 XCDs (runs the probe once, outside stream
 * capture): the fused prefill GEMM and the one-kernel layers' per-XCD verifiers rely on it. */
int dsh_xcd_even(void);
/* 1 if a fused launch's bounded wait expired (its output is then not valid), 0 if not; synchronous. */
int dsh_pf_wait_error(const void *ws, const dsh_layer_t *L, int T);
/* out[T][H] = (residual ? X : 0) + MoE(X); ws: dsh_pf_workspace_bytes(L, T) device bytes. derr (may be
 * NULL): a device word the fused kernel sets (and never clears) when a down tile's bounded wait for its
 * gate_up tiles gives up, after spin_max sleeps (DSH_PF_SPIN_MAX normally; < 0: every such wait gives up
 * at once, a test mode). */
#define DSH_PF_SPIN_MAX (1 << 22)
hipError_t dsh_launch_prefill(const dsh_layer_t *L, const float *X, int T, int route_mode, int nthreads, int residual,
                              int bf16sim, float *out, void *ws, int *idx_out, float *w_out, int *derr, int spin_max,
                              hipStream_t s);
/* The prefill SwiGLU against the correctly rounded division over every 32-bit gate value: counts[0]
 * = finite g with a zero or normal quotient whose results differ, counts[1] = those with a
 * subnormal quotient (2 device words, cleared here). */
hipError_t dsh_launch_pf_swiglu_check(unsigned long long *counts, hipStream_t s);

/* Final reduction of per-block argmax candidates: writes tokens[*step] (tokens[0] when step is
 * NULL) and advances *step. Also clears zero_p[0..zero_n) (16-byte aligned, zero_n % 4 == 0; 0 for
 * none) and, when emb_out != NULL, writes the chosen token's bf16 embedding row emb[token][0..H)
 * widened to f32 into emb_out (the next step's input; H % 8 == 0). */
hipError_t dsh_launch_lm_argmax_final(const unsigned long long *cand, int n, int *tokens, int *step, float *zero_p,
                                      int zero_n, const uint16_t *emb, int emb_vocab, int H, float *emb_out,
                                      hipStream_t s);
/* The final reduction fused with the next step's router partials (CFG): *step already advanced
 * (by the LM head's step_inc); writes tokens[*step - 1], clears zero_p like the kernel above, then
 * the next step's input (emb_out != NULL: the token's embedding widened into emb_out, unchanged for
 * a token outside the table; else row *step of x_in, skipped when *step >= rows) and its router
 * partials[H / R][64] as dsh_launch_dec_partial_scores computes them. */
hipError_t dsh_launch_lm_final_scores(const unsigned long long *cand, int n, int *tokens, const int *step,
                                      float *zero_p, int zero_n, const uint16_t *emb, int emb_vocab, float *emb_out,
                                      const float *x_in, int stride, int rows, const float *WrT, int H, int E,
                                      float *partials, hipStream_t s);
/* After the last step of a run whose steps end with the LM head (dsh_split_t fin_cand / nx_partials):
 * when *pending, the argmax of cand[0..n) into tokens[*step - 1] and *pending cleared; zero_p[0..zero_n)
 * cleared (16-byte aligned, zero_n % 4 == 0). */
hipError_t dsh_launch_lm_token_pending(const unsigned long long *cand, int n, int *tokens, const int *step,
                                       int *pending, float *zero_p, int zero_n, hipStream_t s);
/* Router partial rows per partial (dsh_launch_dec_partial_scores): 8 or 16. */
int dsh_dec_partial_rows(int H);
/* emb[tokens[*step - 1]][0..H) widened to f32 into out (a token outside [0, emb_vocab): unchanged). */
hipError_t dsh_launch_embed_next(const int *tokens, const int *step, const uint16_t *emb, int emb_vocab, int H,
                                 float *out, hipStream_t s);

/* ---- latency-oriented decode kernels (k_dec.hip) ---- */
int dsh_dec_supported(int H, int I, int E, int K, int SI);
int dsh_dec_partials(int H); /* partial score rows written per layer in CFG mode */
/* ---- attention half of a decoder layer, one token (k_attn.hip) ---- */
#define DSH_ATTN_MAX_HD 256
typedef struct {
  const uint16_t *wq, *wk, *wv, *wo;         /* bf16 [qd][H] x3, [H][qd] (qd = n_heads*head_dim) */
  const float *in_norm, *post_norm;          /* [H] */
  const float *q_norm, *k_norm;              /* [head_dim] or NULL */
  const float *rope_cos, *rope_sin;          /* [max_seq][head_dim] */
  float *kc, *vc;                            /* [max_seq][kv_stride] */
  float *q, *k, *att, *proj;                 /* scratch: [qd] x3, [H] */
  float *sc, *part, *se;                     /* [n_heads][max_seq], [n_heads][max_seq/32+1][head_dim], [n_heads] */
  int H, n_heads, head_dim, kv_stride, max_seq;
  float eps;
} dsh_attn_t;
int dsh_attn_supported(int H, int n_heads, int head_dim);
size_t dsh_attn_core_lds(int max_kv);
/* h_out = x + Wo·attention(...), n_out = RMSNorm(h_out) for the token at cache position
 * (pos_ptr ? *pos_ptr : 0) + pos_add; x = x_in + (*step)*stride when step != NULL; ncopies > 1:
 * x = Σ of the copies [ncopies][H] at x_in in copy order (step NULL), also written to x_plain ([H]) for the
 * residual kernel. */
/* With WrT_next ([H][E_next] f32), the last kernel also writes the following MoE layer's router
 * partials from n (dsh_dec_partials(H) rows of 64). */
hipError_t dsh_launch_attn(const dsh_attn_t *A, const float *x_in, const int *step, int stride, int ncopies,
                           float *x_plain, const int *pos_ptr, int pos_add, int prefill_len, int window, int nthreads,
                           float *h_out, float *n_out, const float *WrT_next, int E_next, float *partials_next,
                           hipStream_t s);
/* out = ds_rms_norm(x) (AVX-512 order), then bf16 truncation when trunc; x = Σ of ncopies copies
 * [ncopies][H] (1: plain), also written to x_out when given. */
hipError_t dsh_launch_final_norm(const float *x, int ncopies, const float *w, int H, float eps, int trunc, float *out,
                                 float *x_out, hipStream_t s);
/* ---- greedy token choice with repetition penalty and n-gram ban (k_sample.hip) ---- */
int dsh_sample_supported(int H);
/* After the argmax. Stack form (step != NULL): history tokens[0..min(*step - 1, hist_len)), token
 * tokens[*step - 1]. Explicit form (step == NULL): history hist[0..hist_len), token tokens[0].
 * vals: [hist_len + 1] floats, lg: [vocab] floats, flag: one int (device workspace). */
hipError_t dsh_launch_sample(const uint16_t *W, const float *x, int H, int vocab, int nthreads, float rp, int ngram_n,
                             const int *step, int *tokens, const int *hist, int hist_len, float *vals, float *lg,
                             int *flag, hipStream_t s);
/* ---- dense SwiGLU FFN (k_dense.hip) ---- */
int dsh_dense_supported(int H, int I);
hipError_t dsh_launch_dense_gate_up(const uint16_t *Wg, const uint16_t *Wu, const float *x_in, const int *step,
                                    int stride, int H, int I, float *h, hipStream_t s);
/* x_out[H] = (residual ? x : 0) + Wd·h; with WrT_next ([H][E_next] f32), the next MoE layer's router
 * partial scores over 8-row blocks (H / 8 rows of 64, the format k_dec_down writes). */
hipError_t dsh_launch_dense_down(const uint16_t *Wd, const float *h, const float *x_in, const int *step, int stride,
                                 int H, int I, int residual, const float *resid, float *x_out, const float *WrT_next,
                                 int E_next, float *partials_next, hipStream_t s);
hipError_t dsh_launch_transpose_f32(const float *src, float *dst, int rows, int cols, hipStream_t s);
/* out[r] = ||A[r][0..cols)||_2 in f64, rounded up to f32. */
hipError_t dsh_launch_row_norms(const float *A, int rows, int cols, float *out, hipStream_t s);
hipError_t dsh_launch_dec_partial_scores(const float *WrT, const float *x_in, const int *step, int stride, int H, int E,
                                         float *partials, hipStream_t s);
hipError_t dsh_launch_dec_scores_bf16(const uint16_t *Wr, const float *x_in, const int *step, int stride, int H, int E,
                                      int nthreads, float *partials, hipStream_t s);
/* ncopies == 8: x = Σ of the 8 copies [8][H] at x_in (in copy order; step must be NULL). */
hipError_t dsh_launch_dec_scores_bf16_copies(const uint16_t *Wr, const float *x_in, const int *step, int stride,
                                             int ncopies, int H, int E, int nthreads, float *partials, hipStream_t s);
/* CFG router scores of x in ds_linear's exact order (no BLAS), written as one partial (np = 1). */
hipError_t dsh_launch_dec_scores_f32_exact(const float *WrT, const float *x_in, const int *step, int stride, int H,
                                          int E, float *partials, hipStream_t s);
hipError_t dsh_launch_dec_gate_up(const dsh_layer_t *L, const float *x_in, const int *step, int stride,
                                  const float *partials, int np, int route_mode, int bf16sim,
                                  const dsh_layer_work_t *wk, const dsh_rcert_t *rc, hipStream_t s);
/* x_out = (residual ? (resid ? resid : x) : 0) + MoE(x) rows. */
hipError_t dsh_launch_dec_down(const dsh_layer_t *L, const float *x_in, const int *step, int stride, float *x_out,
                               int residual, const float *resid, int bf16sim, const dsh_layer_work_t *wk,
                               const float *WrT_next, int E_next, float *partials_next, hipStream_t s);
int dsh_dec_lm_blocks(int vocab);
int dsh_dec_lm_supported(int in_dim);
int dsh_dec_lm_eligible(const void *W, int in_dim, int vocab, int nthreads);
hipError_t dsh_launch_dec_lm_argmax_depth(const uint16_t *W, const float *x, int in_dim, int vocab,
                                          unsigned long long *cand, int depth, hipStream_t s);
hipError_t dsh_launch_dec_lm_argmax(const uint16_t *W, const float *x, int in_dim, int vocab,
                                    unsigned long long *cand, hipStream_t s);
/* The same head on x = Σ of ncopies (8) copies [ncopies][in_dim] (in_dim <= 2048); x_out (optional)
 * receives that sum; step_inc (optional) is advanced by one. */
hipError_t dsh_launch_dec_lm_argmax_copies(const uint16_t *W, const float *xc, int ncopies, int in_dim, int vocab,
                                           unsigned long long *cand, float *x_out, int *step_inc, hipStream_t s);

/* ---- the LM-head argmax over an int8 copy of the head with bounds (k_lm.hip) ---- */
typedef struct {
  int8_t *q;   /* [vocab][H] codes rint(w / s) */
  float *sab;  /* [vocab][3]: s, α (bound per ||x||_2), β (bound per half grid step), both rounded up */
  int H, vocab;
} dsh_lm_q8_t;
/* H % 256 == 0, H <= 2048. */
int dsh_lm_q8_supported(int H, int vocab);
/* Device bytes of the copy; dsh_lm_q8_carve lays it out from base (256-byte aligned). */
size_t dsh_lm_q8_bytes(int H, int vocab);
void dsh_lm_q8_carve(void *base, int H, int vocab, dsh_lm_q8_t *Q);
/* Builds the codes and the per-row constants from the bf16 head W [vocab][H]. */
hipError_t dsh_launch_lm_q8_build(const uint16_t *W, const dsh_lm_q8_t *Q, hipStream_t s);
/* Blocks of the kernel (512 rows each). */
int dsh_lm_q8_blocks(int vocab);
/* cand[dsh_lm_q8_blocks(vocab)] receives each block's (max, lowest index) key. ncopies 0:
 * x is the input; 8: x holds 8 copies, whose sum block 0 writes to x_out (optional). step_inc
 * (optional) is advanced by one. */
hipError_t dsh_launch_lm_q8(const uint16_t *W, const dsh_lm_q8_t *Q, const float *x, int ncopies, float *x_out,
                            unsigned long long *cand, int *step_inc, hipStream_t s);

/* ---- one kernel per MoE layer, down split over intermediate units (k_layer.hip) ---- */
typedef struct {
  const int8_t *dnT, *sdnT; /* down tiles of the routed experts [E][I/32], of the shared expert [SI/32] */
  const float *M, *sM;      /* next router x down products, tiles as the down tiles; NULL: last layer */
  const float *z, *sz;      /* next router x down offsets: [E][64], [64] */
  const float *WrT_next;    /* [H][E_next]; NULL: last layer */
  int E_next;
  /* the next layer's shared-expert data, read ahead by extra blocks of this layer's kernel on the
   * XCDs whose blocks read it next (pf_gu NULL: none): gate/up codes and their (scale, offset), down
   * tiles, next-router products (may be NULL); pf_SI: its width */
  const int8_t *pf_gu, *pf_dnT;
  const float *pf_guso, *pf_M;
  int pf_SI;
  /* DECODE routing: the router's bf16 rows [E][H], from which the routed blocks compute the exact
   * scores of their input themselves (partials unused); NULL: the scores come in as partials.
   * Only where dsh_layer_dec_scores_fusable holds. */
  const uint16_t *Wr_dec;
  /* CFG routing, certified (dsh_cert.h): the verdict area of this layer, DSH_SPLIT_VD_INTS ints that
   * are zero when the kernel starts (they sit in the layer's output region). The routed blocks
   * select from the scores as given and add their shares at once; 32 extra blocks compute the
   * layer's exact router scores from its input (1/32 of the rows each, with the running-error bound
   * of ds_linear's order); the last to finish certifies the selection (or recomputes the open
   * experts in ds_linear's order) and, where the certified experts differ from the ones used, all of
   * them add the difference. NULL: no certification (the selection from the scores as
   * given). */
  unsigned *vd;
  int *derr;       /* set (system scope) when an extra block's wait for the verdict gives up */
  dsh_rcert_t rc;  /* counters and log (CFG: the verdict's block records; DECODE: the log only) */
  /* A step with no kernel after the LM head (bound input, no embedding feed). fin_cand (first
   * layer): its last extra block turns the previous step's LM-head keys (fin_n of them) into that
   * step's token, tokens[*fin_step - 1], when *fin_pending, and clears the flag. nx_partials (last
   * layer): its extra blocks write the next step's router partials, from row *nx_step + 1 of nx_in
   * (stride nx_stride) when that is below nx_rows, in k_dec_partial_scores' order (nx_R rows each
   * of the transposed router nx_WrT, nx_E experts), and set *nx_pending. Both jobs run in the
   * DL_PF extra blocks, which they add where the layer reads nothing ahead. */
  const unsigned long long *fin_cand;
  int *fin_tokens, *fin_pending;
  const int *fin_step;
  int fin_n;
  const float *nx_in, *nx_WrT;
  const int *nx_step;
  float *nx_partials;
  int *nx_pending;
  int nx_stride, nx_rows, nx_R, nx_E;
} dsh_split_t;
#define DSH_SPLIT_VD_INTS (64 + 256 * 32)
int dsh_layer_split_supported(const dsh_layer_t *L);
/* Whether the layer kernel can compute DECODE scores itself: H <= 1280 and every router row in a
 * 4- or 2-row group of the reference's chunks of nthreads (no single-row path). */
int dsh_layer_dec_scores_fusable(int H, int E, int nthreads);
int dsh_layer_split_blocks(const dsh_layer_t *L);
/* Whether the one-kernel layer can certify its CFG selection (dsh_split_t.vd): E % 4 == 0, K <= 8,
 * both f32 router layouts present. */
int dsh_layer_cert_supported(const dsh_layer_t *L);
int dsh_layer_split_copies(void);
size_t dsh_layer_split_tile_bytes(const dsh_layer_t *L); /* routed + shared down tiles */
size_t dsh_layer_split_m_floats(const dsh_layer_t *L);   /* routed + shared M tiles */
/* Fills the tiles (and, with WrT_next, M and z) of layer L from its arena. */
hipError_t dsh_launch_layer_build(const dsh_layer_t *L, const float *WrT_next, int E_next, int8_t *dnT, int8_t *sdnT,
                                  float *M, float *sM, float *z, float *sz, hipStream_t s);
/* x_out ([copies][H]) += (resid ? resid : x) + MoE(x); lg_out ([copies][64]) += the next layer's router scores (when F->M).
 * Input: ncopies == 1: x = x_in + (*step)*stride (step may be NULL), router partials [np <= 160][64];
 * ncopies == copies: x = Σ copies of x_in, router partials [np <= 8][64] (CFG: the score copies).
 * route_mode: DSH_ROUTE_CFG or DSH_ROUTE_DECODE (then np == 1: the exact scores; empty slots add
 * nothing). Clears zero_p[0..zero_n). */
hipError_t dsh_launch_dec_layer(const dsh_layer_t *L, const dsh_split_t *F, const float *x_in, const int *step,
                                int stride, int ncopies, const float *partials, int np, int route_mode,
                                const float *resid, float *x_out, float *lg_out, float *zero_p, int zero_n,
                                hipStream_t s);
/* out = Σ copies of X ([copies][H]); clears X and zero_p[0..zero_n). */
hipError_t dsh_launch_dec_copy_sum(float *X, int H, float *out, float *zero_p, int zero_n, hipStream_t s);

#ifdef __cplusplus
}
#endif
