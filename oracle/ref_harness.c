/*
 * ref_harness.c — drives the reference's own hot-path functions (compiled from /root/reference by
 * oracle/build_ref.sh) for the oracle pinning tests, the golden-fixture writer and the CPU baseline.
 * Test infrastructure only.
 *
 * ds_verbose / ds_bf16_simulate_python are the two mode globals the reference defines in
 * ds_ocr.c:26-27 (not compiled here; it needs the Darwin-only Metal backend).
 *
 * ref_moe_layer() composes the public reference functions in the order of moe_forward's INT8
 * branch (ds_moe_decoder.c:145-278). moe_forward itself is static; its inline fast-exp softmax and
 * top-k (ds_moe_decoder.c:157-183) are restated here.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "ds_kernels.h"
#include "ds_quantize.h"

int ds_verbose = 0;
int ds_bf16_simulate_python = 0;

void ref_set_bf16sim(int on) { ds_bf16_simulate_python = on; }
int ref_get_bf16sim(void) { return ds_bf16_simulate_python; }

/* Builds a block that borrows caller arrays (no copy). */
void ref_block_wrap(ds_int4_block_t *b, int8_t *q, float *scale, float *offset, int out_dim, int in_dim) {
  memset(b, 0, sizeof(*b));
  b->qweight = q;
  b->scale = scale;
  b->offset = offset;
  b->out_dim = out_dim;
  b->in_dim = in_dim;
  b->bytes = (size_t)out_dim * in_dim + (size_t)out_dim * 8;
}

size_t ref_block_sizeof(void) { return sizeof(ds_int4_block_t); }

/* ds_int4_quantize_bf16 + copy out + free, for ctypes callers. */
int ref_quantize_bf16_copy(int8_t *q, float *scale, float *offset, const uint16_t *W, int out_dim, int in_dim,
                           size_t *bytes) {
  ds_int4_block_t b;
  int rc = ds_int4_quantize_bf16(&b, W, out_dim, in_dim);
  if (rc != 0) return rc;
  memcpy(q, b.qweight, (size_t)out_dim * in_dim);
  memcpy(scale, b.scale, (size_t)out_dim * 4);
  memcpy(offset, b.offset, (size_t)out_dim * 4);
  if (bytes) *bytes = b.bytes;
  ds_int4_block_free(&b);
  return 0;
}

int ref_quantize_f32_copy(int8_t *q, float *scale, float *offset, const float *W, int out_dim, int in_dim) {
  ds_int4_block_t b;
  int rc = ds_int4_quantize_f32(&b, W, out_dim, in_dim);
  if (rc != 0) return rc;
  memcpy(q, b.qweight, (size_t)out_dim * in_dim);
  memcpy(scale, b.scale, (size_t)out_dim * 4);
  memcpy(offset, b.offset, (size_t)out_dim * 4);
  ds_int4_block_free(&b);
  return 0;
}

typedef struct {
  int hidden, inter, n_experts, top_k, shared_inter;
  const float *router_f32;
  const uint16_t *router_bf16;
  ds_int4_block_t gu[64], dn[64], sgu, sdn;
} ref_layer_t;

size_t ref_layer_sizeof(void) { return sizeof(ref_layer_t); }

void ref_layer_init(ref_layer_t *L, int hidden, int inter, int n_experts, int top_k, int shared_inter,
                    const float *router_f32, const uint16_t *router_bf16) {
  memset(L, 0, sizeof(*L));
  L->hidden = hidden;
  L->inter = inter;
  L->n_experts = n_experts;
  L->top_k = top_k;
  L->shared_inter = shared_inter;
  L->router_f32 = router_f32;
  L->router_bf16 = router_bf16;
}

/* e in [0, n_experts) for routed experts, e == -1 for the shared expert. */
void ref_layer_set_expert(ref_layer_t *L, int e, int8_t *gq, float *gs, float *go, int8_t *dq, float *ds,
                          float *dofs) {
  int H = L->hidden;
  int I = e < 0 ? L->shared_inter : L->inter;
  ds_int4_block_t *g = e < 0 ? &L->sgu : &L->gu[e];
  ds_int4_block_t *d = e < 0 ? &L->sdn : &L->dn[e];
  ref_block_wrap(g, gq, gs, go, 2 * I, H);
  ref_block_wrap(d, dq, ds, dofs, H, I);
}

/* route_mode 0: decode (bf16 router, fast-exp softmax over all experts, no renorm);
 * route_mode 1: cfg (f32 ds_moe_router + ds_moe_top_k). Scratch is allocated per call. */
void ref_moe_layer(float *out, const float *x, const ref_layer_t *L, int route_mode, int *idx_out,
                   float *w_out) {
  int H = L->hidden, E = L->n_experts, K = L->top_k;
  float scores[64];
  int idx[64];
  float w[64];
  if (route_mode == 1) {
    ds_moe_router(scores, x, L->router_f32, H, E);
    ds_moe_top_k(idx, w, scores, E, K);
  } else {
    ds_moe_router_bf16(scores, x, L->router_bf16, H, E);
    float max_s = -1e30f;
    for (int e = 0; e < E; e++)
      if (scores[e] > max_s) max_s = scores[e];
    float sum_exp = 0.0f;
    for (int e = 0; e < E; e++) {
      scores[e] = ds_fast_expf(scores[e] - max_s);
      sum_exp += scores[e];
    }
    float inv = 1.0f / sum_exp;
    for (int e = 0; e < E; e++) scores[e] *= inv;
    for (int k = 0; k < K; k++) {
      int best = -1;
      float bs = -1e30f;
      for (int e = 0; e < E; e++) {
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
  int SI = L->shared_inter, I = L->inter;
  int maxI = SI > I ? SI : I;
  float *eo = (float *)calloc((size_t)K * H, sizeof(float));
  float *gub = (float *)malloc((size_t)2 * maxI * sizeof(float));
  float *gb = (float *)malloc((size_t)maxI * sizeof(float));
  float *ub = (float *)malloc((size_t)maxI * sizeof(float));
  float *hb = (float *)malloc((size_t)maxI * sizeof(float));
  float *sh = (float *)malloc((size_t)H * sizeof(float));
  for (int k = 0; k < K; k++) {
    if (idx[k] < 0) continue;
    ds_expert_forward_fused_int4(eo + (size_t)k * H, x, &L->gu[idx[k]], &L->dn[idx[k]], H, I, gub, gb, ub, hb);
  }
  ds_expert_combine(out, eo, idx, w, K, H);
  ds_expert_forward_fused_int4(sh, x, &L->sgu, &L->sdn, H, SI, gub, gb, ub, hb);
  ds_vec_add(out, out, sh, H);
  if (idx_out)
    for (int k = 0; k < K; k++) idx_out[k] = idx[k];
  if (w_out)
    for (int k = 0; k < K; k++) w_out[k] = w[k];
  free(eo);
  free(gub);
  free(gb);
  free(ub);
  free(hb);
  free(sh);
}

static double now_sec(void) {
  struct timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return ts.tv_sec + ts.tv_nsec * 1e-9;
}

/* Decode steps: per step, x <- xs[step]; for each layer x <- x + MoE(x); token <- argmax(W_lm x).
 * Returns wall seconds for the steps; tokens[] receives each step's index. */
double ref_decode_steps(const ref_layer_t *layers, int n_layers, const uint16_t *lm_w, int vocab,
                        const float *xs, int n_steps, int route_mode, int *tokens) {
  int H = layers[0].hidden;
  float *x = (float *)malloc((size_t)H * sizeof(float));
  float *o = (float *)malloc((size_t)H * sizeof(float));
  double t0 = now_sec();
  for (int s = 0; s < n_steps; s++) {
    memcpy(x, xs + (size_t)s * H, (size_t)H * sizeof(float));
    for (int l = 0; l < n_layers; l++) {
      ref_moe_layer(o, x, &layers[l], route_mode, NULL, NULL);
      ds_vec_add(x, x, o, H);
    }
    tokens[s] = ds_argmax_matvec_bf16(x, lm_w, H, vocab);
  }
  double t1 = now_sec();
  free(x);
  free(o);
  return t1 - t0;
}

/* Final hidden state of one decode step (for parity checks of the stack). */
void ref_decode_hidden(float *x_out, const ref_layer_t *layers, int n_layers, const float *x_in, int route_mode) {
  int H = layers[0].hidden;
  float *o = (float *)malloc((size_t)H * sizeof(float));
  memcpy(x_out, x_in, (size_t)H * sizeof(float));
  for (int l = 0; l < n_layers; l++) {
    ref_moe_layer(o, x_out, &layers[l], route_mode, NULL, NULL);
    ds_vec_add(x_out, x_out, o, H);
  }
  free(o);
}
