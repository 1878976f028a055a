/* moe_forward_dropin.c — an integration example: the reference's decode step at batch 1 written
 * against the per-function drop-in API (include/ds_quantize.h, include/ds_kernels.h) in the order
 * the unchanged reference code calls it. Per MoE layer (moe_forward, ds_moe_decoder.c:131-278, INT8
 * branch): ds_moe_router_bf16 (:152), then the caller's own softmax over all experts with
 * ds_fast_expf and strict-> top-k selection on the host (:157-183), ds_expert_forward_fused_int4
 * per selected expert (:237-243), ds_expert_combine (:263), the shared expert through
 * ds_expert_forward_fused_int4 and ds_vec_add (:269-278); the decoder layer's residual add
 * (ds_vec_add, :468); then the greedy head ds_argmax_matvec_bf16 (:1041). Every call is synchronous
 * and moves its activations between host and device, as the drop-in boundary must.
 *
 * Built as examples/libdropin_example.so against libds_ocr_hip.so; bench.py times it beside the
 * reference CPU path. */
#define _POSIX_C_SOURCE 199309L
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "ds_hip.h"
#include "ds_kernels.h"
#include "ds_quantize.h"

typedef struct {
  int hidden, inter, n_experts, top_k, shared_inter;
  const uint16_t *router_bf16;            /* [n_experts][hidden] */
  const ds_int4_block_t *gate_up, *down;  /* [n_experts] each: fused gate_up [2*inter][hidden], down [hidden][inter] */
  const ds_int4_block_t *shared_gate_up, *shared_down;
} dropin_layer_t;

typedef struct {
  float *out, *experts, *shared, *gu, *g, *u, *h;
} dropin_bufs_t;

/* Host wall time and count of each kind of library call during the last dropin_decode_steps run
 * (clock_gettime around every call; the caller's own routing on the host is in none of them). */
enum { K_ROUTER, K_EXPERT, K_COMBINE, K_SHARED, K_VEC_ADD, K_ARGMAX, K_NKIND };
static double g_secs[K_NKIND];
static long g_calls[K_NKIND];

static double now_s(void) {
  struct timespec t;
  clock_gettime(CLOCK_MONOTONIC, &t);
  return (double)t.tv_sec + 1e-9 * (double)t.tv_nsec;
}

#define TIMED(kind, call)             \
  do {                                \
    const double t0_ = now_s();       \
    call;                             \
    g_secs[kind] += now_s() - t0_;    \
    g_calls[kind]++;                  \
  } while (0)

/* secs[k], calls[k] for the kinds router, routed expert, combine, shared expert, vec_add, argmax. */
void dropin_call_times(double *secs, long *calls) {
  for (int k = 0; k < K_NKIND; k++) {
    secs[k] = g_secs[k];
    calls[k] = g_calls[k];
  }
}

/* The caller's routing (ds_moe_decoder.c:157-183): softmax of all router scores with the bit-trick
 * exponent, then the top_k largest probabilities, the first of equal ones, unnormalised. */
static void route(int *idx, float *w, float *scores, int n, int k) {
  float mx = -1e30f;
  for (int e = 0; e < n; e++) mx = scores[e] > mx ? scores[e] : mx;
  float sum = 0.0f;
  for (int e = 0; e < n; e++) {
    scores[e] = ds_fast_expf(scores[e] - mx);
    sum += scores[e];
  }
  const float inv = 1.0f / sum;
  for (int e = 0; e < n; e++) scores[e] *= inv;
  for (int j = 0; j < k; j++) {
    int best = -1;
    float bv = -1e30f;
    for (int e = 0; e < n; e++) {
      int taken = 0;
      for (int i = 0; i < j; i++) taken |= idx[i] == e;
      if (!taken && scores[e] > bv) {
        bv = scores[e];
        best = e;
      }
    }
    idx[j] = best;
    w[j] = bv;
  }
}

static void moe_block(const dropin_layer_t *ly, const float *x, dropin_bufs_t *b) {
  const int H = ly->hidden, I = ly->inter;
  float scores[DS_MAX_EXPERTS], w[DS_MAX_EXPERTS];
  int idx[DS_MAX_EXPERTS];
  TIMED(K_ROUTER, ds_moe_router_bf16(scores, x, ly->router_bf16, H, ly->n_experts));
  route(idx, w, scores, ly->n_experts, ly->top_k);
  for (int k = 0; k < ly->top_k; k++)
    TIMED(K_EXPERT, ds_expert_forward_fused_int4(b->experts + (size_t)k * H, x, &ly->gate_up[idx[k]],
                                                 &ly->down[idx[k]], H, I, b->gu, b->g, b->u, b->h));
  TIMED(K_COMBINE, ds_expert_combine(b->out, b->experts, idx, w, ly->top_k, H));
  TIMED(K_SHARED, ds_expert_forward_fused_int4(b->shared, x, ly->shared_gate_up, ly->shared_down, H,
                                               ly->shared_inter, b->gu, b->g, b->u, b->h));
  TIMED(K_VEC_ADD, ds_vec_add(b->out, b->out, b->shared, H));
}

/* Registers every block and the routers and the head with the device (one upload each), so the
 * timed steps see steady state. Returns 0 or -1. */
int dropin_register(const dropin_layer_t *layers, int n_layers, const uint16_t *lm_w, int vocab) {
  for (int l = 0; l < n_layers; l++) {
    const dropin_layer_t *ly = &layers[l];
    for (int e = 0; e < ly->n_experts; e++)
      if (ds_hip_register_block(&ly->gate_up[e]) || ds_hip_register_block(&ly->down[e])) return -1;
    if (ds_hip_register_block(ly->shared_gate_up) || ds_hip_register_block(ly->shared_down)) return -1;
    if (ds_hip_register_weights(ly->router_bf16, (size_t)ly->n_experts * ly->hidden * 2)) return -1;
  }
  return ds_hip_register_weights(lm_w, (size_t)vocab * layers[0].hidden * 2);
}

/* n_steps decode steps, step s on input row xs[s]; tokens[s] receives the greedy token. Returns the
 * elapsed wall time in seconds (or -1 on allocation failure). */
double dropin_decode_steps(const dropin_layer_t *layers, int n_layers, const uint16_t *lm_w, int vocab,
                           const float *xs, int n_steps, int *tokens) {
  const int H = layers[0].hidden;
  int imax = 0, kmax = 0;
  for (int l = 0; l < n_layers; l++) {
    imax = layers[l].shared_inter > imax ? layers[l].shared_inter : imax;
    imax = layers[l].inter > imax ? layers[l].inter : imax;
    kmax = layers[l].top_k > kmax ? layers[l].top_k : kmax;
  }
  dropin_bufs_t b;
  float *x = (float *)malloc(sizeof(float) * (size_t)H);
  b.out = (float *)malloc(sizeof(float) * (size_t)H);
  b.shared = (float *)malloc(sizeof(float) * (size_t)H);
  b.experts = (float *)malloc(sizeof(float) * (size_t)H * kmax);
  b.gu = (float *)malloc(sizeof(float) * 2 * (size_t)imax);
  b.g = (float *)malloc(sizeof(float) * (size_t)imax);
  b.u = (float *)malloc(sizeof(float) * (size_t)imax);
  b.h = (float *)malloc(sizeof(float) * (size_t)imax);
  double secs = -1.0;
  if (x && b.out && b.shared && b.experts && b.gu && b.g && b.u && b.h) {
    struct timespec t0, t1;
    memset(g_secs, 0, sizeof g_secs);
    memset(g_calls, 0, sizeof g_calls);
    clock_gettime(CLOCK_MONOTONIC, &t0);
    for (int s = 0; s < n_steps; s++) {
      memcpy(x, xs + (size_t)s * H, sizeof(float) * (size_t)H);
      for (int l = 0; l < n_layers; l++) {
        moe_block(&layers[l], x, &b);
        TIMED(K_VEC_ADD, ds_vec_add(x, x, b.out, H));
      }
      TIMED(K_ARGMAX, tokens[s] = ds_argmax_matvec_bf16(x, lm_w, H, vocab));
    }
    clock_gettime(CLOCK_MONOTONIC, &t1);
    secs = (double)(t1.tv_sec - t0.tv_sec) + 1e-9 * (double)(t1.tv_nsec - t0.tv_nsec);
  }
  free(x);
  free(b.out);
  free(b.shared);
  free(b.experts);
  free(b.gu);
  free(b.g);
  free(b.u);
  free(b.h);
  return secs;
}
