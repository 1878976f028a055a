/* ds_hip_layer.c — device-resident MoE layers and the decode stack (ds_hip.h).
 *
 * Layer arena (one hipMalloc per MoE layer, every region 256-byte aligned):
 *   routed gate_up codes [E][2I][H] | routed down codes [E][H][I] | shared gate_up [2SI][H] |
 *   shared down [H][SI] | (scale, offset) pairs for each of those row sets | router f32 [E][H] |
 *   router bf16 [E][H] | work: scores[E], idx[K], w[K], h[K*I+SI], x[H]
 * Expert e's rows sit at a fixed offset, so the kernels index experts from the device-side top-k
 * without any host round trip. The reference allocates every block separately
 * (ds_quantize.c:57-59) and gathers experts through ds_dec_layer_t.experts_int4[64].
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "dsr.h"
#include "ds_hip.h"
#include "ds_kernels.h"

struct ds_hip_layer {
  int H, I, E, K, SI;
  void *arena;
  size_t bytes;
  size_t wbytes; /* the weight regions 0-9: the arena's prefix that a saved arena holds */
  dsh_layer_t d;          /* device pointers into the arena */
  dsh_layer_work_t wk;    /* work buffers (in the arena) */
  float *partials;        /* [H/8][64] router partial scores */
  int np;                 /* number of partial rows in CFG mode */
  int have_f32, have_bf16;
  /* prefill: the launch sequence as a graph, reused while the call's pointers and sizes repeat */
  hipGraphExec_t pf_exec;
  struct pf_key {
    const void *out, *x, *ws, *idx, *w;
    int T, mode, residual, bf16sim, threads, fused, spin_max;
  } pf_key;
};

static size_t al(size_t n) { return (n + 255) & ~(size_t)255; }

ds_hip_layer_t *ds_hip_layer_create(int hidden, int inter, int n_experts, int top_k, int shared_inter) {
  if (dsr_init()) return NULL;
  if (hidden <= 0 || inter <= 0 || n_experts <= 0 || top_k <= 0 || shared_inter <= 0 || n_experts > 64 ||
      top_k > n_experts) {
    dsr_failf("ds_hip_layer_create: invalid shape H=%d I=%d E=%d K=%d SI=%d", hidden, inter, n_experts, top_k,
              shared_inter);
    return NULL;
  }
  if (!dsh_dec_supported(hidden, inter, n_experts, top_k, shared_inter)) {
    dsr_failf("ds_hip_layer_create: shape H=%d I=%d E=%d K=%d SI=%d not supported by the fused decode kernels "
              "(need H %% 256 == 0 and H <= 2048, I %% 16 == 0 and I <= 1024, SI %% I == 0, K + SI/I == 8)",
              hidden, inter, n_experts, top_k, shared_inter);
    return NULL;
  }
  ds_hip_layer_t *L = (ds_hip_layer_t *)calloc(1, sizeof *L);
  if (!L) return NULL;
  size_t H = hidden, I = inter, E = n_experts, K = top_k, SI = shared_inter;
  size_t off[18], n = 0, k = 0;
#define REGION(bytes) (off[k++] = n, n += al(bytes))
  REGION(E * 2 * I * H);          /* 0 gu_q */
  REGION(E * H * I);              /* 1 dn_q */
  REGION(2 * SI * H);             /* 2 sgu_q */
  REGION(H * SI);                 /* 3 sdn_q */
  REGION(E * 2 * I * 8);          /* 4 gu_so */
  REGION(E * H * 8);              /* 5 dn_so */
  REGION(2 * SI * 8);             /* 6 sgu_so */
  REGION(H * 8);                  /* 7 sdn_so */
  REGION(E * H * 4);              /* 8 router f32 */
  REGION(E * H * 2);              /* 9 router bf16 */
  REGION(E * 4);                  /* 10 scores */
  REGION(K * 4);                  /* 11 idx */
  REGION(K * 4);                  /* 12 w */
  REGION((K * I + SI) * 4);       /* 13 h */
  REGION((H / 8) * 64 * 4);       /* 14 router partial scores */
  REGION(E * H * 4);              /* 15 router f32, transposed [H][E] */
  REGION((K + 1) * H * 4);        /* 16 expert outputs (bf16 simulation) */
  REGION(E * 4);                  /* 17 f32 router row norms */
#undef REGION
  hipError_t e = hipMalloc(&L->arena, n);
  if (e != hipSuccess) {
    dsr_fail("layer arena allocation", e);
    free(L);
    return NULL;
  }
  hipMemsetAsync(L->arena, 0, n, dsr_stream);
  char *b = (char *)L->arena;
  L->bytes = n;
  L->wbytes = off[10];
  L->H = hidden;
  L->I = inter;
  L->E = n_experts;
  L->K = top_k;
  L->SI = shared_inter;
  L->d.gu_q = (const int8_t *)(b + off[0]);
  L->d.dn_q = (const int8_t *)(b + off[1]);
  L->d.sgu_q = (const int8_t *)(b + off[2]);
  L->d.sdn_q = (const int8_t *)(b + off[3]);
  L->d.gu_so = (const float *)(b + off[4]);
  L->d.dn_so = (const float *)(b + off[5]);
  L->d.sgu_so = (const float *)(b + off[6]);
  L->d.sdn_so = (const float *)(b + off[7]);
  L->d.router_f32 = (const float *)(b + off[8]);
  L->d.router_bf16 = (const uint16_t *)(b + off[9]);
  L->d.router_f32_t = (const float *)(b + off[15]);
  L->d.router_norm = (const float *)(b + off[17]);
  L->d.H = hidden;
  L->d.I = inter;
  L->d.E = n_experts;
  L->d.K = top_k;
  L->d.SI = shared_inter;
  L->wk.scores = (float *)(b + off[10]);
  L->wk.idx = (int *)(b + off[11]);
  L->wk.w = (float *)(b + off[12]);
  L->wk.h = (float *)(b + off[13]);
  L->wk.eo = (float *)(b + off[16]);
  L->partials = (float *)(b + off[14]);
  L->np = dsh_dec_partials(hidden);
  return L;
}

void ds_hip_layer_destroy(ds_hip_layer_t *L) {
  if (!L) return;
  hipStreamSynchronize(dsr_stream);
  if (L->pf_exec) hipGraphExecDestroy(L->pf_exec);
  hipFree(L->arena);
  free(L);
}

size_t ds_hip_layer_bytes(const ds_hip_layer_t *L) { return L ? L->bytes : 0; }

int ds_hip_layer_set_router(ds_hip_layer_t *L, const float *router_f32, const uint16_t *router_bf16) {
  if (!L) return dsr_failf("ds_hip_layer_set_router: NULL layer");
  size_t n = (size_t)L->E * L->H;
  if (router_f32) {
    if (dsr_h2d((void *)L->d.router_f32, router_f32, n * 4)) return -1;
    DSR_TRY(dsh_launch_transpose_f32(L->d.router_f32, (float *)L->d.router_f32_t, L->E, L->H, dsr_stream),
            "router transpose");
    DSR_TRY(dsh_launch_row_norms(L->d.router_f32, L->E, L->H, (float *)L->d.router_norm, dsr_stream), "router norms");
    L->have_f32 = 1;
  }
  if (router_bf16) {
    if (dsr_h2d((void *)L->d.router_bf16, router_bf16, n * 2)) return -1;
    L->have_bf16 = 1;
  }
  DSR_TRY(hipStreamSynchronize(dsr_stream), "set router");
  return 0;
}

int ds_hip_layer_set_router_dev(ds_hip_layer_t *L, const float *router_f32_dev, const uint16_t *router_bf16_dev) {
  if (!L) return dsr_failf("ds_hip_layer_set_router_dev: NULL layer");
  size_t n = (size_t)L->E * L->H;
  if (router_f32_dev) {
    DSR_TRY(hipMemcpyAsync((void *)L->d.router_f32, router_f32_dev, n * 4, hipMemcpyDeviceToDevice, dsr_stream),
            "router copy");
    DSR_TRY(dsh_launch_transpose_f32(L->d.router_f32, (float *)L->d.router_f32_t, L->E, L->H, dsr_stream),
            "router transpose");
    DSR_TRY(dsh_launch_row_norms(L->d.router_f32, L->E, L->H, (float *)L->d.router_norm, dsr_stream), "router norms");
    L->have_f32 = 1;
  }
  if (router_bf16_dev) {
    DSR_TRY(hipMemcpyAsync((void *)L->d.router_bf16, router_bf16_dev, n * 2, hipMemcpyDeviceToDevice, dsr_stream),
            "router copy");
    L->have_bf16 = 1;
  }
  return 0;
}

/* Device destinations of expert e's rows (e == -1: shared). */
static int expert_dst(const ds_hip_layer_t *L, int e, int8_t **gq, float **gso, int8_t **dq, float **dso, int *I) {
  size_t H = L->H;
  if (e == -1) {
    *I = L->SI;
    *gq = (int8_t *)L->d.sgu_q;
    *gso = (float *)L->d.sgu_so;
    *dq = (int8_t *)L->d.sdn_q;
    *dso = (float *)L->d.sdn_so;
    return 0;
  }
  if (e < 0 || e >= L->E) return dsr_failf("expert index %d outside [-1, %d)", e, L->E);
  size_t In = L->I;
  *I = L->I;
  *gq = (int8_t *)L->d.gu_q + (size_t)e * 2 * In * H;
  *gso = (float *)L->d.gu_so + (size_t)e * 2 * In * 2;
  *dq = (int8_t *)L->d.dn_q + (size_t)e * H * In;
  *dso = (float *)L->d.dn_so + (size_t)e * H * 2;
  return 0;
}

static int upload_block(int8_t *q, float *so, const ds_int4_block_t *b, int out_dim, int in_dim) {
  if (!b || !b->qweight || !b->scale || !b->offset || b->out_dim != out_dim || b->in_dim != in_dim)
    return dsr_failf("ds_hip_layer_set_expert: block shape %dx%d, expected %dx%d", b ? b->out_dim : -1,
                     b ? b->in_dim : -1, out_dim, in_dim);
  float *pairs = (float *)malloc((size_t)out_dim * 8);
  if (!pairs) return dsr_failf("host allocation failed");
  for (int r = 0; r < out_dim; r++) {
    pairs[2 * r] = b->scale[r];
    pairs[2 * r + 1] = b->offset[r];
  }
  int rc = dsr_h2d(q, b->qweight, (size_t)out_dim * in_dim) || dsr_h2d(so, pairs, (size_t)out_dim * 8);
  if (!rc) rc = hipStreamSynchronize(dsr_stream) != hipSuccess;
  free(pairs);
  return rc ? -1 : 0;
}

int ds_hip_layer_set_expert(ds_hip_layer_t *L, int e, const ds_int4_block_t *gate_up, const ds_int4_block_t *down) {
  if (!L) return dsr_failf("ds_hip_layer_set_expert: NULL layer");
  int8_t *gq, *dq;
  float *gso, *dso;
  int I;
  if (expert_dst(L, e, &gq, &gso, &dq, &dso, &I)) return -1;
  if (upload_block(gq, gso, gate_up, 2 * I, L->H)) return -1;
  return upload_block(dq, dso, down, L->H, I);
}

int ds_hip_layer_quantize_expert(ds_hip_layer_t *L, int e, const uint16_t *gate_up_bf16_dev,
                                 const uint16_t *down_bf16_dev) {
  if (!L || !gate_up_bf16_dev || !down_bf16_dev) return dsr_failf("ds_hip_layer_quantize_expert: NULL argument");
  int8_t *gq, *dq;
  float *gso, *dso;
  int I;
  if (expert_dst(L, e, &gq, &gso, &dq, &dso, &I)) return -1;
  hipError_t err = dsh_launch_quantize_bf16_so(gate_up_bf16_dev, gq, gso, 2 * I, L->H, dsr_stream);
  if (err == hipSuccess) err = dsh_launch_quantize_bf16_so(down_bf16_dev, dq, dso, L->H, I, dsr_stream);
  if (err != hipSuccess) return dsr_fail("quantize expert", err);
  return 0;
}

static int export_block(int8_t *q, float *sc, float *of, const int8_t *dq, const float *dso, int out_dim, int in_dim) {
  if (q && dsr_d2h(q, dq, (size_t)out_dim * in_dim)) return -1;
  if (sc || of) {
    float *pairs = (float *)malloc((size_t)out_dim * 8);
    if (!pairs) return dsr_failf("host allocation failed");
    if (dsr_d2h(pairs, dso, (size_t)out_dim * 8)) {
      free(pairs);
      return -1;
    }
    for (int r = 0; r < out_dim; r++) {
      if (sc) sc[r] = pairs[2 * r];
      if (of) of[r] = pairs[2 * r + 1];
    }
    free(pairs);
  }
  return 0;
}

int ds_hip_layer_export_expert(const ds_hip_layer_t *L, int e, int8_t *gu_q, float *gu_scale, float *gu_offset,
                               int8_t *dn_q, float *dn_scale, float *dn_offset) {
  if (!L) return dsr_failf("ds_hip_layer_export_expert: NULL layer");
  int8_t *gq, *dq;
  float *gso, *dso;
  int I;
  if (expert_dst(L, e, &gq, &gso, &dq, &dso, &I)) return -1;
  if (export_block(gu_q, gu_scale, gu_offset, gq, gso, 2 * I, L->H)) return -1;
  return export_block(dn_q, dn_scale, dn_offset, dq, dso, L->H, I);
}

static int check_router(const ds_hip_layer_t *L, int route_mode) {
  if (route_mode == DS_HIP_ROUTE_CFG && !L->have_f32) return dsr_failf("layer has no f32 router (route_mode CFG)");
  if (route_mode == DS_HIP_ROUTE_DECODE && !L->have_bf16)
    return dsr_failf("layer has no bf16 router (route_mode DECODE)");
  if (route_mode != DS_HIP_ROUTE_CFG && route_mode != DS_HIP_ROUTE_DECODE)
    return dsr_failf("unknown route_mode %d", route_mode);
  return 0;
}

/* Event marks between a step's launch groups: ev == NULL records nothing; otherwise mark i records
 * ev[i] when that entry is non-NULL (so a caller can bracket any range of kernels) and always
 * advances the count. */
static hipError_t mark(hipEvent_t *ev, int *n) {
  if (!ev) return hipSuccess;
  hipEvent_t x = ev[(*n)++];
  return x ? hipEventRecord(x, dsr_stream) : hipSuccess;
}

/* Router partial scores of layer L for input x (CFG: f32 partials, or with the bf16 simulation the
 * exact full scores as one partial; DECODE: exact full scores as one partial). Returns the number of
 * partial rows through *np. */
static hipError_t scores_enqueue(const ds_hip_layer_t *L, const float *x_in, const int *step, int stride,
                                 int route_mode, int bf16sim, int threads, float *partials, int *np) {
  if (route_mode == DS_HIP_ROUTE_CFG && bf16sim) { /* exact: ds_linear's own order */
    *np = 1;
    return dsh_launch_dec_scores_f32_exact(L->d.router_f32_t, x_in, step, stride, L->H, L->E, partials, dsr_stream);
  }
  if (route_mode == DS_HIP_ROUTE_CFG) {
    *np = L->np;
    return dsh_launch_dec_partial_scores(L->d.router_f32_t, x_in, step, stride, L->H, L->E, partials, dsr_stream);
  }
  *np = 1;
  return dsh_launch_dec_scores_bf16(L->d.router_bf16, x_in, step, stride, L->H, L->E, threads, partials,
                                    dsr_stream);
}

/* DECODE routing in the one-kernel layers: the router rows from which layer L's kernel computes its
 * own exact scores, or NULL where the scores kernel runs before it (an odd chunk of the reference's
 * threads puts a router row on the single-row path, or H is past the kernel's register budget). */
static const uint16_t *dec_fused_router(const ds_hip_layer_t *L, int route_mode, int split, int threads) {
  return split && route_mode == DS_HIP_ROUTE_DECODE && dsh_layer_dec_scores_fusable(L->H, L->E, threads)
             ? L->d.router_bf16
             : NULL;
}

/* One layer: [scores], gate_up, down. In CFG mode with next != NULL, down also writes the partial
 * scores of layer "next" and the next layer's scores kernel is skipped by the caller. */
static hipError_t layer_enqueue(const ds_hip_layer_t *L, const dsh_layer_work_t *wk, float *partials,
                                int have_scores, int np, const float *x_in, const int *step, int stride, float *x_out,
                                int route_mode, int residual, int bf16sim, const ds_hip_layer_t *next,
                                hipEvent_t *ev, int *nev) {
  hipError_t e = hipSuccess;
  const dsh_rcert_t rc = dsr_rcert(0);
  if (!have_scores) {
    e = scores_enqueue(L, x_in, step, stride, route_mode, bf16sim, dsr_threads(), partials, &np);
    if (e == hipSuccess) e = mark(ev, nev);
  }
  if (e == hipSuccess)
    e = dsh_launch_dec_gate_up(&L->d, x_in, step, stride, partials, np, route_mode, bf16sim, wk, &rc, dsr_stream);
  if (e == hipSuccess) e = mark(ev, nev);
  int chain = next && route_mode == DS_HIP_ROUTE_CFG && !bf16sim;
  if (e == hipSuccess)
    e = dsh_launch_dec_down(&L->d, x_in, step, stride, x_out, residual, NULL, bf16sim, wk,
                            chain ? next->d.router_f32_t : NULL, chain ? next->E : 0, chain ? partials : NULL,
                            dsr_stream);
  if (e == hipSuccess) e = mark(ev, nev);
  return e;
}

int ds_hip_layer_forward(ds_hip_layer_t *L, float *out_dev, const float *x_dev, int route_mode, int residual,
                         int *idx_dev, float *w_dev) {
  if (!L || !out_dev || !x_dev) return dsr_failf("ds_hip_layer_forward: NULL argument");
  if (check_router(L, route_mode)) return -1;
  int bf16sim = ds_bf16_simulate_python;
  hipError_t e = layer_enqueue(L, &L->wk, L->partials, 0, 0, x_dev, NULL, 0, out_dev, route_mode, residual, bf16sim,
                               NULL, NULL, NULL);
  if (e != hipSuccess) return dsr_fail("layer kernels", e);
  if (idx_dev)
    DSR_TRY(hipMemcpyAsync(idx_dev, L->wk.idx, (size_t)L->K * 4, hipMemcpyDeviceToDevice, dsr_stream), "idx copy");
  if (w_dev)
    DSR_TRY(hipMemcpyAsync(w_dev, L->wk.w, (size_t)L->K * 4, hipMemcpyDeviceToDevice, dsr_stream), "w copy");
  return 0;
}

/* Sleeps before a fused prefill tile's wait for its gate_up tiles gives up (ds_hip_prefill_set_wait_limit). */
static int g_pf_spin_max = DSH_PF_SPIN_MAX;

int ds_hip_prefill_set_wait_limit(int spins) {
  g_pf_spin_max = spins == DS_HIP_PREFILL_WAIT_DEFAULT ? DSH_PF_SPIN_MAX : spins;
  return 0;
}

/* Prefill MoE block (ds_moe_decoder.c:629-809) for T tokens already on the device. The workspace
 * (activations split to bf16, routing, the expert-sorted pair list, h and per-pair outputs; about
 * 65 KB per token at DeepSeek-OCR's shape) is a library staging buffer that grows to the largest T. */
int ds_hip_layer_prefill(ds_hip_layer_t *L, float *out_dev, const float *x_dev, int T, int route_mode, int residual,
                         int *idx_dev, float *w_dev) {
  if (!L || !out_dev || !x_dev || T <= 0) return dsr_failf("ds_hip_layer_prefill: invalid arguments");
  if (check_router(L, route_mode)) return -1;
  /* a bounded wait that gave up in an earlier call (already finished) voids that call's output */
  if (dsr_derr_check()) return -1;
  if (!dsh_pf_supported(&L->d))
    return dsr_failf("ds_hip_layer_prefill: shape H=%d I=%d SI=%d not supported (needs H %% 256 == 0, I and SI %% 128 == 0)",
                     L->H, L->I, L->SI);
  DSR_TRY(dsh_pf_init(-2), "prefill init");
  void *ws = dsr_scratch(DSR_SLOT_PF, dsh_pf_workspace_bytes(&L->d, T));
  if (!ws) return -1;
  struct pf_key key;
  memset(&key, 0, sizeof key);
  key.out = out_dev;
  key.x = x_dev;
  key.ws = ws;
  key.idx = idx_dev;
  key.w = w_dev;
  key.T = T;
  key.mode = route_mode;
  key.residual = residual;
  key.bf16sim = ds_bf16_simulate_python;
  key.threads = dsr_threads();
  key.fused = dsh_pf_fused();
  key.spin_max = g_pf_spin_max;
  if (!L->pf_exec || memcmp(&key, &L->pf_key, sizeof key) != 0) {
    /* the seven kernels (and the idx/w copies) captured once, then one graph launch per call */
    if (L->pf_exec) { /* an earlier call's launch of it may still run on the stream */
      DSR_TRY(hipStreamSynchronize(dsr_stream), "prefill graph");
      hipGraphExecDestroy(L->pf_exec);
      L->pf_exec = NULL;
    }
    DSR_TRY(hipStreamBeginCapture(dsr_stream, hipStreamCaptureModeThreadLocal), "prefill capture begin");
    hipError_t e = dsh_launch_prefill(&L->d, x_dev, T, route_mode, key.threads, residual, key.bf16sim, out_dev, ws,
                                      idx_dev, w_dev, dsr_derr_dev(DSR_DERR_PREFILL_WAIT), key.spin_max, dsr_stream);
    hipGraph_t g = NULL;
    hipError_t ec = hipStreamEndCapture(dsr_stream, &g);
    if (e != hipSuccess || ec != hipSuccess || !g) {
      if (g) hipGraphDestroy(g);
      return dsr_fail("prefill kernels", e != hipSuccess ? e : ec);
    }
    e = hipGraphInstantiate(&L->pf_exec, g, NULL, NULL, 0);
    hipGraphDestroy(g);
    if (e != hipSuccess) {
      L->pf_exec = NULL;
      return dsr_fail("prefill graph instantiate", e);
    }
    L->pf_key = key;
  }
  DSR_TRY(hipGraphLaunch(L->pf_exec, dsr_stream), "prefill graph launch");
  return 0;
}

/* Prefill GEMM path: 1 the fused persistent kernel, 0 the two-kernel path, -1 automatic (fused when
 * a grid's blocks cover every XCD). Returns the path now in use (or -1 on error). */
int ds_hip_prefill_path(int mode) {
  if (dsr_init()) return -1;
  if (dsh_pf_init(mode < 0 ? -1 : mode) != hipSuccess) return dsr_failf("ds_hip_prefill_path: init failed");
  return dsh_pf_fused();
}

/* The prefill SwiGLU against the correctly rounded division over all 2^32 gate values (u = 1):
 * n_differ[0] = finite g with a zero or normal quotient whose results differ in any bit,
 * n_differ[1] = finite g with a subnormal quotient whose results differ. Synchronous. */
int ds_hip_check_prefill_swiglu(uint64_t *n_differ) {
  if (dsr_init()) return -1;
  if (!n_differ) return dsr_failf("ds_hip_check_prefill_swiglu: invalid arguments");
  unsigned long long *c = (unsigned long long *)dsr_scratch(DSR_SLOT_IDX, 2 * sizeof(unsigned long long));
  if (!c) return -1;
  unsigned long long h[2];
  DSR_TRY(dsh_launch_pf_swiglu_check(c, dsr_stream), "swiglu check");
  DSR_TRY(hipMemcpyAsync(h, c, sizeof h, hipMemcpyDeviceToHost, dsr_stream), "copy");
  DSR_TRY(hipStreamSynchronize(dsr_stream), "sync");
  n_differ[0] = h[0];
  n_differ[1] = h[1];
  return 0;
}

/* After a prefill call of T tokens on layer L: 1 if the fused kernel's bounded wait expired (the
 * output is then not valid), 0 if not. Synchronises the library stream. */
int ds_hip_prefill_wait_error(ds_hip_layer_t *L, int T) {
  if (!L || T <= 0) return dsr_failf("ds_hip_prefill_wait_error: invalid arguments");
  DSR_TRY(hipStreamSynchronize(dsr_stream), "sync");
  void *ws = dsr_scratch(DSR_SLOT_PF, dsh_pf_workspace_bytes(&L->d, T));
  if (!ws) return -1;
  const int v = dsh_pf_wait_error(ws, &L->d, T);
  if (v == 1) (void)dsr_derr_check(); /* reported here: the caller asked */
  return v;
}

/* Average device time of n back-to-back prefill calls (HIP events on the library stream). */
int ds_hip_time_prefill(ds_hip_layer_t *L, float *out_dev, const float *x_dev, int T, int route_mode, int n, float *ms) {
  if (!ms || n <= 0) return dsr_failf("ds_hip_time_prefill: invalid arguments");
  if (ds_hip_layer_prefill(L, out_dev, x_dev, T, route_mode, 0, NULL, NULL)) return -1; /* sizes the workspace */
  hipEvent_t a, b;
  DSR_TRY(hipEventCreate(&a), "event");
  DSR_TRY(hipEventCreate(&b), "event");
  int rc = 0;
  if (hipEventRecord(a, dsr_stream) != hipSuccess) rc = -1;
  for (int i = 0; i < n && rc == 0; i++) rc = ds_hip_layer_prefill(L, out_dev, x_dev, T, route_mode, 0, NULL, NULL);
  if (rc == 0 && (hipEventRecord(b, dsr_stream) != hipSuccess || hipEventSynchronize(b) != hipSuccess ||
                  hipEventElapsedTime(ms, a, b) != hipSuccess))
    rc = dsr_failf("ds_hip_time_prefill: timing failed");
  if (rc == 0) *ms /= (float)n;
  hipEventDestroy(a);
  hipEventDestroy(b);
  return rc;
}

int ds_hip_time_layer(ds_hip_layer_t *L, float *out_dev, const float *x_dev, int route_mode, int n, float *ms) {
  if (!ms || n <= 0) return dsr_failf("ds_hip_time_layer: invalid arguments");
  if (ds_hip_layer_forward(L, out_dev, x_dev, route_mode, 0, NULL, NULL)) return -1; /* warm-up */
  hipEvent_t a, b;
  DSR_TRY(hipEventCreate(&a), "event");
  DSR_TRY(hipEventCreate(&b), "event");
  int rc = 0;
  if (hipEventRecord(a, dsr_stream) != hipSuccess) rc = -1;
  for (int i = 0; i < n && rc == 0; i++) rc = ds_hip_layer_forward(L, out_dev, x_dev, route_mode, 0, NULL, NULL);
  if (rc == 0 && (hipEventRecord(b, dsr_stream) != hipSuccess || hipEventSynchronize(b) != hipSuccess ||
                  hipEventElapsedTime(ms, a, b) != hipSuccess))
    rc = dsr_failf("ds_hip_time_layer: timing failed");
  if (rc == 0) *ms /= (float)n;
  hipEventDestroy(a);
  hipEventDestroy(b);
  return rc == 0 ? dsr_derr_check() : rc;
}

/* ================================================================ persisted arena
 * File (little-endian): a 256-byte header
 *   [0,8) magic "DSI8ARNA"  [8,12) version (1)  [12,16) n_layers  [16,36) hidden, inter, n_experts,
 *   top_k, shared_inter  [36,40) vocab (0: no LM head)  [40,48) layer_bytes  [48,56) lm_bytes
 *   [56,64) checksum of everything after the header  [64,256) zero
 * then per layer a 64-byte record (u32 has f32 router, u32 has bf16 router, zero) and layer_bytes
 * bytes: the arena's weight regions exactly as they sit in device memory (routed gate_up codes,
 * routed down codes, shared gate_up, shared down, the four (scale, offset) pair arrays, f32 router,
 * bf16 router; each region 256-byte aligned), then lm_bytes of the bf16 LM head [vocab][hidden].
 * The transposed f32 router is rebuilt on load. The checksum folds 8-byte words four at a time. */
#define ARENA_MAGIC "DSI8ARNA"
#define ARENA_VERSION 1u
#define ARENA_CHUNK ((size_t)64 << 20)

typedef struct {
  char magic[8];
  uint32_t version, n_layers, hidden, inter, n_experts, top_k, shared_inter, vocab;
  uint64_t layer_bytes, lm_bytes, checksum;
  uint8_t zero[192];
} arena_header_t;
typedef struct {
  uint32_t have_f32, have_bf16;
  uint8_t zero[56];
} arena_record_t;

_Static_assert(sizeof(arena_header_t) == 256, "arena header layout");
_Static_assert(sizeof(arena_record_t) == 64, "arena layer record layout");

typedef struct {
  uint64_t h[4];
  uint8_t tail[8];
  int ntail;
} arena_sum_t;

static void sum_init(arena_sum_t *c) {
  memset(c, 0, sizeof *c);
  c->h[0] = 0x9E3779B97F4A7C15ull;
  c->h[1] = 0xC2B2AE3D27D4EB4Full;
  c->h[2] = 0x165667B19E3779F9ull;
  c->h[3] = 0x27D4EB2F165667C5ull;
}
static inline uint64_t sum_mix(uint64_t h, uint64_t w) {
  h ^= w;
  h *= 0x100000001B3ull;
  return (h << 29) | (h >> 35);
}
static void sum_add(arena_sum_t *c, const void *p, size_t n) {
  const uint8_t *b = (const uint8_t *)p;
  while (n && c->ntail) {  // finish a partial word
    c->tail[c->ntail++] = *b++;
    n--;
    if (c->ntail == 8) {
      uint64_t w;
      memcpy(&w, c->tail, 8);
      c->h[0] = sum_mix(c->h[0], w);
      c->ntail = 0;
    }
  }
  size_t nw = n / 32;
  for (size_t i = 0; i < nw; i++, b += 32) {
    uint64_t w[4];
    memcpy(w, b, 32);
    for (int k = 0; k < 4; k++) c->h[k] = sum_mix(c->h[k], w[k]);
  }
  n -= nw * 32;
  while (n >= 8) {
    uint64_t w;
    memcpy(&w, b, 8);
    c->h[0] = sum_mix(c->h[0], w);
    b += 8;
    n -= 8;
  }
  while (n--) c->tail[c->ntail++] = *b++;
}
static uint64_t sum_final(arena_sum_t *c) {
  if (c->ntail) {
    memset(c->tail + c->ntail, 0, 8 - c->ntail);
    uint64_t w;
    memcpy(&w, c->tail, 8);
    c->h[0] = sum_mix(c->h[0], w ^ (uint64_t)c->ntail);
  }
  return c->h[0] ^ (c->h[1] * 3) ^ (c->h[2] * 5) ^ (c->h[3] * 7);
}

/* Writes n bytes at device address src to f through the host buffer buf (ARENA_CHUNK bytes). */
static int arena_write_dev(FILE *f, const void *src, size_t n, void *buf, arena_sum_t *c) {
  for (size_t o = 0; o < n; o += ARENA_CHUNK) {
    size_t k = n - o < ARENA_CHUNK ? n - o : ARENA_CHUNK;
    if (dsr_d2h(buf, (const char *)src + o, k)) return -1;
    sum_add(c, buf, k);
    if (fwrite(buf, 1, k, f) != k) return dsr_failf("ds_hip_arena_save: write failed");
  }
  return 0;
}
static int arena_read_dev(FILE *f, void *dst, size_t n, void *buf, arena_sum_t *c) {
  for (size_t o = 0; o < n; o += ARENA_CHUNK) {
    size_t k = n - o < ARENA_CHUNK ? n - o : ARENA_CHUNK;
    if (fread(buf, 1, k, f) != k) return dsr_failf("ds_hip_arena_load: file is truncated");
    sum_add(c, buf, k);
    DSR_TRY(hipMemcpyAsync((char *)dst + o, buf, k, hipMemcpyHostToDevice, dsr_stream), "arena upload");
    DSR_TRY(hipStreamSynchronize(dsr_stream), "arena upload");
  }
  return 0;
}

int ds_hip_arena_save(const char *path, ds_hip_layer_t *const *layers, int n_layers, const uint16_t *lm_head_dev,
                      int vocab) {
  if (!path || !layers || n_layers <= 0 || (lm_head_dev && vocab <= 0))
    return dsr_failf("ds_hip_arena_save: invalid arguments");
  const ds_hip_layer_t *L0 = layers[0];
  if (!L0) return dsr_failf("ds_hip_arena_save: NULL layer");
  for (int i = 1; i < n_layers; i++) {
    const ds_hip_layer_t *L = layers[i];
    if (!L || L->H != L0->H || L->I != L0->I || L->E != L0->E || L->K != L0->K || L->SI != L0->SI)
      return dsr_failf("ds_hip_arena_save: layer %d has another shape than layer 0", i);
  }
  if (dsr_init()) return -1;
  arena_header_t hd;
  memset(&hd, 0, sizeof hd);
  memcpy(hd.magic, ARENA_MAGIC, 8);
  hd.version = ARENA_VERSION;
  hd.n_layers = (uint32_t)n_layers;
  hd.hidden = (uint32_t)L0->H;
  hd.inter = (uint32_t)L0->I;
  hd.n_experts = (uint32_t)L0->E;
  hd.top_k = (uint32_t)L0->K;
  hd.shared_inter = (uint32_t)L0->SI;
  hd.vocab = lm_head_dev ? (uint32_t)vocab : 0u;
  hd.layer_bytes = L0->wbytes;
  hd.lm_bytes = lm_head_dev ? (uint64_t)vocab * (uint64_t)L0->H * 2u : 0u;
  FILE *f = fopen(path, "wb");
  if (!f) return dsr_failf("ds_hip_arena_save: cannot open %s", path);
  void *buf = NULL;
  int rc = 0;
  if (hipHostMalloc(&buf, ARENA_CHUNK, hipHostMallocDefault) != hipSuccess) {
    buf = NULL;
    rc = dsr_failf("ds_hip_arena_save: pinned staging allocation failed");
  }
  arena_sum_t c;
  sum_init(&c);
  if (!rc && fwrite(&hd, sizeof hd, 1, f) != 1) rc = dsr_failf("ds_hip_arena_save: write failed");
  if (!rc) rc = hipStreamSynchronize(dsr_stream) == hipSuccess ? 0 : dsr_failf("ds_hip_arena_save: stream error");
  for (int i = 0; i < n_layers && !rc; i++) {
    arena_record_t r;
    memset(&r, 0, sizeof r);
    r.have_f32 = (uint32_t)layers[i]->have_f32;
    r.have_bf16 = (uint32_t)layers[i]->have_bf16;
    sum_add(&c, &r, sizeof r);
    if (fwrite(&r, sizeof r, 1, f) != 1) rc = dsr_failf("ds_hip_arena_save: write failed");
    if (!rc) rc = arena_write_dev(f, layers[i]->arena, layers[i]->wbytes, buf, &c);
  }
  if (!rc && lm_head_dev) rc = arena_write_dev(f, lm_head_dev, hd.lm_bytes, buf, &c);
  if (!rc) {
    hd.checksum = sum_final(&c);
    if (fseek(f, 0, SEEK_SET) || fwrite(&hd, sizeof hd, 1, f) != 1) rc = dsr_failf("ds_hip_arena_save: write failed");
  }
  if (fclose(f) && !rc) rc = dsr_failf("ds_hip_arena_save: close failed");
  if (buf) hipHostFree(buf);
  return rc;
}

int ds_hip_arena_load(const char *path, ds_hip_layer_t **layers, int max_layers, uint16_t **lm_head_dev, int *vocab) {
  if (!path || !layers || max_layers <= 0) return dsr_failf("ds_hip_arena_load: invalid arguments");
  if (lm_head_dev) *lm_head_dev = NULL;
  if (vocab) *vocab = 0;
  FILE *f = fopen(path, "rb");
  if (!f) return dsr_failf("ds_hip_arena_load: cannot open %s", path);
  arena_header_t hd;
  int rc = 0, made = 0;
  void *buf = NULL;
  uint16_t *lm = NULL;
  if (fread(&hd, sizeof hd, 1, f) != 1 || memcmp(hd.magic, ARENA_MAGIC, 8)) {
    rc = dsr_failf("ds_hip_arena_load: %s is not a packed INT8 arena", path);
  } else if (hd.version != ARENA_VERSION) {
    rc = dsr_failf("ds_hip_arena_load: format version %u, expected %u", hd.version, ARENA_VERSION);
  } else if (hd.n_layers == 0 || (int)hd.n_layers > max_layers) {
    rc = dsr_failf("ds_hip_arena_load: %u layers in the file, room for %d", hd.n_layers, max_layers);
  } else if (hd.lm_bytes != (uint64_t)hd.vocab * hd.hidden * 2u) {
    rc = dsr_failf("ds_hip_arena_load: inconsistent LM head size");
  }
  if (!rc && fseek(f, 0, SEEK_END) == 0) {
    const uint64_t want = sizeof hd + (uint64_t)hd.n_layers * (sizeof(arena_record_t) + hd.layer_bytes) + hd.lm_bytes;
    const long got = ftell(f);
    if (got < 0 || (uint64_t)got != want)
      rc = dsr_failf("ds_hip_arena_load: file size %ld, the header describes %llu", got, (unsigned long long)want);
    else if (fseek(f, (long)sizeof hd, SEEK_SET))
      rc = dsr_failf("ds_hip_arena_load: seek failed");
  }
  if (!rc && hipHostMalloc(&buf, ARENA_CHUNK, hipHostMallocDefault) != hipSuccess) {
    buf = NULL;
    rc = dsr_failf("ds_hip_arena_load: pinned staging allocation failed");
  }
  arena_sum_t c;
  sum_init(&c);
  for (uint32_t i = 0; i < hd.n_layers && !rc; i++) {
    ds_hip_layer_t *L = ds_hip_layer_create((int)hd.hidden, (int)hd.inter, (int)hd.n_experts, (int)hd.top_k,
                                            (int)hd.shared_inter);
    if (!L) {
      rc = -1;
      break;
    }
    layers[made++] = L;
    if (L->wbytes != hd.layer_bytes) {
      rc = dsr_failf("ds_hip_arena_load: layer section of %llu bytes, this build lays out %zu",
                     (unsigned long long)hd.layer_bytes, L->wbytes);
      break;
    }
    arena_record_t r;
    if (fread(&r, sizeof r, 1, f) != 1) {
      rc = dsr_failf("ds_hip_arena_load: file is truncated");
      break;
    }
    sum_add(&c, &r, sizeof r);
    rc = arena_read_dev(f, L->arena, L->wbytes, buf, &c);
    if (rc) break;
    L->have_f32 = r.have_f32 != 0;
    L->have_bf16 = r.have_bf16 != 0;
    if (L->have_f32) {
      hipError_t e = dsh_launch_transpose_f32(L->d.router_f32, (float *)L->d.router_f32_t, L->E, L->H, dsr_stream);
      if (e != hipSuccess) rc = dsr_fail("router transpose", e);
    }
  }
  if (!rc && hd.lm_bytes) {
    if (hipMalloc((void **)&lm, hd.lm_bytes) != hipSuccess) {
      lm = NULL;
      rc = dsr_failf("ds_hip_arena_load: LM head allocation failed");
    } else {
      rc = arena_read_dev(f, lm, hd.lm_bytes, buf, &c);
    }
  }
  if (!rc && sum_final(&c) != hd.checksum) rc = dsr_failf("ds_hip_arena_load: checksum mismatch (corrupt file)");
  if (!rc && hipStreamSynchronize(dsr_stream) != hipSuccess) rc = dsr_failf("ds_hip_arena_load: stream error");
  fclose(f);
  if (buf) hipHostFree(buf);
  if (rc) {
    for (int i = 0; i < made; i++) ds_hip_layer_destroy(layers[i]);
    for (int i = 0; i < made; i++) layers[i] = NULL;
    if (lm) hipFree(lm);
    return -1;
  }
  if (lm_head_dev) *lm_head_dev = lm;
  else if (lm) hipFree(lm);
  if (vocab) *vocab = (int)hd.vocab;
  return (int)hd.n_layers;
}

/* ================================================================ dense FFN (layer 0) */
struct ds_hip_dense {
  int H, I;
  void *arena; /* gate [I][H] | up [I][H] | down [H][I] bf16 | h [I] f32 */
  const uint16_t *wg, *wu, *wd;
  float *h;
};

ds_hip_dense_t *ds_hip_dense_create(int hidden, int inter, const uint16_t *gate, const uint16_t *up,
                                    const uint16_t *down) {
  if (dsr_init()) return NULL;
  if (!gate || !up || !down || !dsh_dense_supported(hidden, inter)) {
    dsr_failf("ds_hip_dense_create: invalid arguments or shape H=%d I=%d (need H %% 128 == 0, H <= 2048, I %% 8 == 0, "
              "I <= 16384)", hidden, inter);
    return NULL;
  }
  ds_hip_dense_t *D = (ds_hip_dense_t *)calloc(1, sizeof *D);
  if (!D) return NULL;
  const size_t w = (size_t)hidden * inter * 2, wa = al(w);
  hipError_t e = hipMalloc(&D->arena, 3 * wa + al((size_t)inter * 4));
  if (e != hipSuccess) {
    dsr_fail("dense FFN allocation", e);
    free(D);
    return NULL;
  }
  char *b = (char *)D->arena;
  D->H = hidden;
  D->I = inter;
  D->wg = (const uint16_t *)b;
  D->wu = (const uint16_t *)(b + wa);
  D->wd = (const uint16_t *)(b + 2 * wa);
  D->h = (float *)(b + 3 * wa);
  if (dsr_h2d((void *)D->wg, gate, w) || dsr_h2d((void *)D->wu, up, w) || dsr_h2d((void *)D->wd, down, w) ||
      hipStreamSynchronize(dsr_stream) != hipSuccess) {
    hipFree(D->arena);
    free(D);
    return NULL;
  }
  return D;
}

void ds_hip_dense_destroy(ds_hip_dense_t *D) {
  if (!D) return;
  hipStreamSynchronize(dsr_stream);
  hipFree(D->arena);
  free(D);
}

static hipError_t dense_enqueue(const ds_hip_dense_t *D, float *out, const float *x, const int *step, int stride,
                                int residual, const ds_hip_layer_t *next, float *partials_next) {
  hipError_t e = dsh_launch_dense_gate_up(D->wg, D->wu, x, step, stride, D->H, D->I, D->h, dsr_stream);
  if (e == hipSuccess)
    e = dsh_launch_dense_down(D->wd, D->h, x, step, stride, D->H, D->I, residual, NULL, out,
                              next ? next->d.router_f32_t : NULL, next ? next->E : 0, partials_next, dsr_stream);
  return e;
}

int ds_hip_dense_forward(ds_hip_dense_t *D, float *out_dev, const float *x_dev, int residual) {
  if (!D || !out_dev || !x_dev) return dsr_failf("ds_hip_dense_forward: invalid arguments");
  DSR_TRY(dense_enqueue(D, out_dev, x_dev, NULL, 0, residual, NULL, NULL), "dense FFN");
  return 0;
}

/* ================================================================ decode stack */

struct ds_hip_stack {
  ds_hip_layer_t **layers;
  int n_layers;
  const ds_hip_dense_t *dense; /* optional dense FFN layer before the MoE layers */
  const uint16_t *lm;
  int vocab, H;
  int route_mode, bf16sim;
  /* the reference's thread count when the stack was created (ds_set_threads): the row chunks the
   * stack's exact kernels emulate (DECODE scores, the head's row order, sampling) all follow it, so
   * a later ds_set_threads does not change a created stack or its captured graph */
  int threads;
  int lm_fast;
  /* the argmax over an int8 copy of the head with exact bounds (same tokens; lm_fast heads only) */
  void *lmq_mem;
  dsh_lm_q8_t lmq;
  int lm_cert;
  void *work;              /* step counter, x buffer, candidates, partials */
  size_t work_bytes;
  int *step;
  float *xbuf;
  unsigned long long *cand;
  int ncand;
  float *partials[2];      /* router partial scores, by layer parity */
  const float *xs;
  int stride;
  int *tokens;
  /* what the step's first kernels read: xs + (*step)*stride, or the embedding feed's row */
  const float *in;
  const int *in_step;
  int in_stride;
  /* steps launched since the bind or the last reset, and how many the bound buffers allow */
  int done, cap;
  int rows; /* rows of the bound input */
  /* the step's final kernel also computes the next step's first router partials (one-kernel layers,
   * CFG routing, no dense layer, attention or sampling rules, the head on the layer copies): the
   * partials always belong to the current step's input (reset and every run call compute them) */
  int merged;
  /* the step ends with the LM head (merged, the bound input without the embedding feed, at least 3
   * layers): the first layer's extra block turns the previous step's LM-head keys into its token,
   * the first two layers clear the last two copies regions, and the last layer's extra blocks
   * compute the next step's router partials; one kernel after a run's steps (tail_enqueue) finishes
   * its last token and clears those regions */
  int tailed;
  int *pending; /* the last step's token is still in the LM-head keys (in work, beside step) */
  /* autoregressive input (ds_hip_stack_set_embedding): step s >= 1 reads the widened embedding of
   * token s - 1, which the step before wrote into ebuf */
  const uint16_t *emb;
  int emb_vocab;
  float *ebuf;
  hipGraph_t graph;
  hipGraphExec_t exec;
  /* runs of several steps launch a graph of gk steps at a time (step_enqueue captured gk times:
   * every step's kernels take the step from the device counter), then the 1-step graph */
  hipGraphExec_t exec_k;
  int gk;
  int bound;
  /* full decoder step (ds_hip_stack_set_attention): one attention block per decoder layer */
  ds_hip_attn_t **attn;
  int n_attn, pos0, trunc_final;
  float final_eps;
  void *att_work;          /* h [H], n [H], the LM head's input [H], final norm weights [H] */
  float *hbuf, *nbuf, *fbuf, *final_norm;
  /* greedy sampling rules after the argmax (ds_hip_stack_set_sampling) */
  float rp;
  int ngram, hist_cap;
  void *smp_work; /* [hist_cap + 1] dots, [vocab] logits, flag */
  /* one kernel per MoE layer (k_layer.hip): per-layer down tiles and next-router products, and the
   * layer outputs kept as per-XCD copies; built by ds_hip_stack_bind */
  int split_want, split;
  void *split_arena;
  dsh_split_t *sp;   /* [n_layers] */
  float *xc;         /* layer l's output (l = 1..n_layers): region l-1 of [copies][H] + [copies][64] */
  size_t xc_region;  /* floats per region */
};

int ds_hip_lm_head_sample(const float *x_dev, const uint16_t *lm_head_dev, int hidden, int vocab, const int *history_dev,
                          int history_len, float repeat_penalty, int no_repeat_ngram_size, int *token_dev) {
  if (!x_dev || !lm_head_dev || !token_dev || hidden <= 0 || vocab <= 0 || history_len < 0 ||
      (history_len > 0 && !history_dev) || no_repeat_ngram_size < 0 || !(repeat_penalty == repeat_penalty))
    return dsr_failf("ds_hip_lm_head_sample: invalid arguments");
  if (!dsh_sample_supported(hidden)) return dsr_failf("ds_hip_lm_head_sample: hidden %d not supported", hidden);
  if (dsr_init()) return -1;
  const int T = dsr_threads();
  const int nb = dsh_argmax_avx_blocks(vocab);
  unsigned long long *cand = (unsigned long long *)dsr_scratch(DSR_SLOT_C, sizeof(unsigned long long) * (size_t)nb);
  float *vals = (float *)dsr_scratch(DSR_SLOT_A, (size_t)(history_len + 1) * 4);
  float *lg = (float *)dsr_scratch(DSR_SLOT_B, (size_t)vocab * 4);
  int *flag = (int *)dsr_scratch(DSR_SLOT_IDX, 16);
  if (!cand || !vals || !lg || !flag) return -1;
  DSR_TRY(dsh_launch_argmax_avx(lm_head_dev, x_dev, cand, NULL, hidden, vocab, T, token_dev, NULL, dsr_stream),
          "LM-head argmax");
  DSR_TRY(dsh_launch_sample(lm_head_dev, x_dev, hidden, vocab, T, repeat_penalty, no_repeat_ngram_size, NULL,
                            token_dev, history_dev, history_len, vals, lg, flag, dsr_stream),
          "sampling rules");
  return 0;
}

/* The int8 copy of the head and its bound constants (k_lm.hip), built from the head's contents.
 * Without device memory for it the stack keeps the one-pass head (the same tokens). */
static int lm_cert_build(ds_hip_stack_t *S) {
  if (!S->lmq_mem) {
    if (hipMalloc(&S->lmq_mem, dsh_lm_q8_bytes(S->H, S->vocab)) != hipSuccess) {
      (void)hipGetLastError();
      S->lmq_mem = NULL;
      S->lm_cert = 0;
      return 0;
    }
    dsh_lm_q8_carve(S->lmq_mem, S->H, S->vocab, &S->lmq);
  }
  DSR_TRY(dsh_launch_lm_q8_build(S->lm, &S->lmq, dsr_stream), "LM head int8 copy");
  S->lm_cert = 1;
  return 0;
}

int ds_hip_stack_set_lm_certified(ds_hip_stack_t *S, int on) {
  if (!S) return dsr_failf("ds_hip_stack_set_lm_certified: NULL stack");
  if (S->bound) return dsr_failf("ds_hip_stack_set_lm_certified: call before ds_hip_stack_bind");
  if (!on) {
    S->lm_cert = 0;
    return 0;
  }
  if (!S->lm_fast || !dsh_lm_q8_supported(S->H, S->vocab))
    return dsr_failf("ds_hip_stack_set_lm_certified: head %d x %d not supported", S->vocab, S->H);
  if (lm_cert_build(S)) return -1;
  if (!S->lm_cert) return dsr_failf("ds_hip_stack_set_lm_certified: no device memory for the int8 copy");
  return 0;
}

int ds_hip_stack_lm_certified(const ds_hip_stack_t *S) { return S && S->lm_fast && S->lm_cert ? 1 : 0; }

ds_hip_stack_t *ds_hip_stack_create(ds_hip_layer_t *const *layers, int n_layers, const uint16_t *lm_head_dev,
                                    int vocab, int route_mode) {
  if (dsr_init()) return NULL;
  if (!layers || n_layers <= 0 || !lm_head_dev || vocab <= 0) {
    dsr_failf("ds_hip_stack_create: invalid arguments");
    return NULL;
  }
  int H = layers[0]->H;
  for (int l = 0; l < n_layers; l++) {
    if (!layers[l] || layers[l]->H != H) {
      dsr_failf("ds_hip_stack_create: layer %d missing or hidden size differs", l);
      return NULL;
    }
    if (check_router(layers[l], route_mode)) return NULL;
  }
  ds_hip_stack_t *S = (ds_hip_stack_t *)calloc(1, sizeof *S);
  if (!S) return NULL;
  S->layers = (ds_hip_layer_t **)malloc(sizeof(ds_hip_layer_t *) * (size_t)n_layers);
  memcpy(S->layers, layers, sizeof(ds_hip_layer_t *) * (size_t)n_layers);
  S->n_layers = n_layers;
  S->lm = lm_head_dev;
  S->vocab = vocab;
  S->H = H;
  S->gk = DS_HIP_GRAPH_STEPS_DEFAULT;
  S->route_mode = route_mode;
  S->bf16sim = ds_bf16_simulate_python;
  S->threads = dsr_threads();
  S->lm_fast = dsh_dec_lm_eligible(lm_head_dev, H, vocab, S->threads);
  S->ncand = S->lm_fast ? dsh_dec_lm_blocks(vocab) : dsh_argmax_avx_blocks(vocab);
  if (S->lm_fast && dsh_lm_q8_supported(H, vocab)) lm_cert_build(S);
  const size_t np_bytes = al((size_t)layers[0]->np * 64 * 4);
  size_t off_x = 256, off_c = off_x + al((size_t)H * 4), off_p = off_c + al((size_t)S->ncand * 8);
  size_t off_e = off_p + 2 * np_bytes, bytes = off_e + al((size_t)H * 4);
  hipError_t e = hipMalloc(&S->work, bytes);
  if (e != hipSuccess) {
    dsr_fail("stack allocation", e);
    free(S->layers);
    free(S);
    return NULL;
  }
  S->work_bytes = bytes;
  hipMemsetAsync(S->work, 0, bytes, dsr_stream);
  S->step = (int *)S->work;
  S->pending = S->step + 1;
  S->xbuf = (float *)((char *)S->work + off_x);
  S->cand = (unsigned long long *)((char *)S->work + off_c);
  S->partials[0] = (float *)((char *)S->work + off_p);
  S->partials[1] = (float *)((char *)S->work + off_p + np_bytes);
  S->ebuf = (float *)((char *)S->work + off_e);
  S->split_want = 1;
  return S;
}

void ds_hip_stack_destroy(ds_hip_stack_t *S) {
  if (!S) return;
  hipStreamSynchronize(dsr_stream);
  if (S->exec) hipGraphExecDestroy(S->exec);
  if (S->exec_k) hipGraphExecDestroy(S->exec_k);
  if (S->graph) hipGraphDestroy(S->graph);
  hipFree(S->work);
  if (S->lmq_mem) hipFree(S->lmq_mem);
  if (S->smp_work) hipFree(S->smp_work);
  if (S->att_work) hipFree(S->att_work);
  if (S->split_arena) hipFree(S->split_arena);
  free(S->sp);
  free(S->attn);
  free(S->layers);
  free(S);
}

static int smp_active(const ds_hip_stack_t *S) { return S->rp > 1.0f || S->ngram > 0; }
static float *smp_vals(const ds_hip_stack_t *S) { return (float *)S->smp_work; }
static float *smp_logits(const ds_hip_stack_t *S) { return (float *)S->smp_work + al((size_t)(S->hist_cap + 1) * 4) / 4; }
static int *smp_flag(const ds_hip_stack_t *S) { return (int *)(smp_logits(S) + al((size_t)S->vocab * 4) / 4); }

int ds_hip_stack_set_sampling(ds_hip_stack_t *S, float repeat_penalty, int no_repeat_ngram_size, int history_cap) {
  if (!S) return dsr_failf("ds_hip_stack_set_sampling: NULL stack");
  if (S->bound) return dsr_failf("ds_hip_stack_set_sampling: call before ds_hip_stack_bind");
  if (no_repeat_ngram_size < 0 || history_cap < 0 || !(repeat_penalty == repeat_penalty))
    return dsr_failf("ds_hip_stack_set_sampling: invalid arguments");
  if (!dsh_sample_supported(S->H)) return dsr_failf("ds_hip_stack_set_sampling: hidden %d not supported", S->H);
  if (S->smp_work) {
    hipFree(S->smp_work);
    S->smp_work = NULL;
  }
  S->rp = repeat_penalty;
  S->ngram = no_repeat_ngram_size;
  S->hist_cap = history_cap;
  if (!smp_active(S)) return 0;
  size_t bytes = al((size_t)(history_cap + 1) * 4) + al((size_t)S->vocab * 4) + 256;
  DSR_TRY(hipMalloc(&S->smp_work, bytes), "sampling workspace");
  return 0;
}

/* The LM head's input: the final RMSNorm's output in a full decoder step, else the last layer's. */
static const float *lm_in(const ds_hip_stack_t *S) { return S->attn ? S->fbuf : S->xbuf; }

int ds_hip_stack_set_attention(ds_hip_stack_t *S, ds_hip_attn_t *const *attn, int n_attn, const float *final_norm,
                               float final_eps, int pos0, int trunc_final) {
  if (!S) return dsr_failf("ds_hip_stack_set_attention: NULL stack");
  if (S->bound) return dsr_failf("ds_hip_stack_set_attention: call before ds_hip_stack_bind");
  if (!attn && n_attn == 0) { /* back to MoE layers only */
    free(S->attn);
    S->attn = NULL;
    S->n_attn = 0;
    return 0;
  }
  const int want = (S->dense ? 1 : 0) + S->n_layers;
  if (!attn || n_attn != want || !final_norm || pos0 < 0)
    return dsr_failf("ds_hip_stack_set_attention: need %d attention blocks (dense layer, then each MoE layer), the "
                     "final norm and pos0 >= 0", want);
  for (int i = 0; i < n_attn; i++)
    if (!attn[i] || ds_hip_attn_hidden(attn[i]) != S->H)
      return dsr_failf("ds_hip_stack_set_attention: block %d missing or hidden size differs", i);
  if (!S->att_work) DSR_TRY(hipMalloc(&S->att_work, (size_t)4 * al((size_t)S->H * 4)), "decoder step buffers");
  char *b = (char *)S->att_work;
  const size_t r = al((size_t)S->H * 4);
  S->hbuf = (float *)b;
  S->nbuf = (float *)(b + r);
  S->fbuf = (float *)(b + 2 * r);
  S->final_norm = (float *)(b + 3 * r);
  if (dsr_h2d(S->final_norm, final_norm, (size_t)S->H * 4)) return -1;
  free(S->attn);
  S->attn = (ds_hip_attn_t **)malloc(sizeof(ds_hip_attn_t *) * (size_t)n_attn);
  if (!S->attn) return dsr_failf("ds_hip_stack_set_attention: out of memory");
  memcpy(S->attn, attn, sizeof(ds_hip_attn_t *) * (size_t)n_attn);
  S->n_attn = n_attn;
  S->pos0 = pos0;
  S->final_eps = final_eps;
  S->trunc_final = trunc_final ? 1 : 0;
  return 0;
}

int ds_hip_stack_set_dense(ds_hip_stack_t *S, ds_hip_dense_t *D) {
  if (!S) return dsr_failf("ds_hip_stack_set_dense: NULL stack");
  if (S->bound) return dsr_failf("ds_hip_stack_set_dense: call before ds_hip_stack_bind");
  if (D && D->H != S->H) return dsr_failf("ds_hip_stack_set_dense: hidden %d, the stack has %d", D->H, S->H);
  if (S->attn) return dsr_failf("ds_hip_stack_set_dense: call before ds_hip_stack_set_attention");
  S->dense = D;
  return 0;
}

size_t ds_hip_stack_bytes_per_step(const ds_hip_stack_t *S) {
  if (!S) return 0;
  size_t per_layer = 0;
  const ds_hip_layer_t *L = S->layers[0];
  size_t H = L->H, I = L->I, K = L->K, SI = L->SI, E = L->E;
  per_layer += K * (2 * I * H + 2 * I * 8) + K * (H * I + H * 8); /* routed experts */
  per_layer += 2 * SI * H + 2 * SI * 8 + H * SI + H * 8;          /* shared expert */
  per_layer += E * H * (S->route_mode == DS_HIP_ROUTE_CFG ? 4 : 2); /* router */
  size_t dense = S->dense ? (size_t)3 * S->dense->H * S->dense->I * 2 : 0;
  for (int i = 0; i < S->n_attn; i++) dense += ds_hip_attn_weight_bytes(S->attn[i]); /* KV reads not counted */
  /* the head: the bf16 rows, or (bounded) the int8 codes and 12 bytes of constants per row (the few
   * candidate rows read again in bf16 are not counted) */
  const size_t head = S->lm_fast && S->lm_cert ? (size_t)S->vocab * ((size_t)S->H + 12) : (size_t)S->vocab * S->H * 2;
  return per_layer * (size_t)S->n_layers + dense + head;
}

/* Kernels launched per decode step (for profiling). */
/* Kernels per step: CFG routing: the first layer's partial scores, then gate_up and down per layer;
 * DECODE routing: scores, gate_up and down per layer. Then the LM head (2 kernels). */
/* The launch groups of one step, in the order step_enqueue records an event after each; names may
 * be NULL. Returns the count. */
static int stack_names(const ds_hip_stack_t *S, const char **names) {
  const int cfg = S->route_mode == DS_HIP_ROUTE_CFG;
  int n = 0;
#define NM(str)                   \
  do {                            \
    if (names) names[n] = (str);  \
    n++;                          \
  } while (0)
  if (S->attn) {
    if (S->dense) {
      NM("attention");
      NM("dense.gate_up");
      NM("dense.down");
    }
    for (int l = 0; l < S->n_layers; l++) {
      NM("attention");
      if ((!cfg || S->bf16sim) && !dec_fused_router(S->layers[l], S->route_mode, S->split, S->threads)) NM("scores");
      if (S->split) {
        NM("layer");
      } else {
        NM("gate_up");
        NM("down");
      }
    }
    NM("final_norm");
  } else if (S->split) {
    if (S->dense) {
      NM("dense.gate_up");
      NM("dense.down");
    }
    for (int l = 0; l < S->n_layers; l++) {
      if (cfg ? l == 0 && !S->dense && !S->merged : !dec_fused_router(S->layers[l], S->route_mode, 1, S->threads)) NM("scores");
      NM("layer");
    }
    if (!S->lm_fast) NM("copy_sum");
  } else {
    if (S->dense) {
      NM("dense.gate_up");
      NM("dense.down");
    }
    for (int l = 0; l < S->n_layers; l++) {
      /* with a dense layer first, its down kernel writes the first MoE layer's CFG partials; the bf16
       * simulation computes every layer's scores exactly */
      if (!cfg || S->bf16sim || (l == 0 && !S->dense)) NM("scores");
      NM("gate_up");
      NM("down");
    }
  }
  NM("lm_head.argmax");
  if (!S->tailed) NM(S->merged ? "lm_head.final+scores" : "lm_head.final");
  if (smp_active(S)) NM("sample");
#undef NM
  return n;
}

static int stack_kernel_count(const ds_hip_stack_t *S) { return stack_names(S, NULL); }

/* One decode step; ev (optional) receives an event before the first kernel and after each one.
 * Layer l reads router partials from partials[l & 1]; in CFG mode its down kernel writes layer
 * l+1's into partials[(l + 1) & 1]. */
/* A full decoder step's layers (ds_moe_decoder.c:339-474 per layer): the attention half, then the
 * MLP on n with h as its residual. In CFG routing the attention's last kernel writes the MoE
 * layer's router partials from n; in DECODE routing the scores kernel reads n. */
static float *xc_region(const ds_hip_stack_t *S, int l);

static hipError_t layers_full_enqueue(ds_hip_stack_t *S, hipEvent_t *ev, int *nev) {
  hipError_t e = hipSuccess;
  const int cfg = S->route_mode == DS_HIP_ROUTE_CFG, C = dsh_layer_split_copies();
  /* CFG scores as partials from the kernel before (the bf16 simulation computes them exactly instead) */
  const int cfgp = cfg && !S->bf16sim;
  const dsh_layer_work_t *wk = &S->layers[0]->wk;
  const float *xin = S->in;
  const int *st = S->in_step;
  int stride = S->in_stride, a = 0, nc = 1; /* nc: copies of xin (one-kernel layers: the per-XCD copies) */
  if (S->dense) {
    e = ds_hip_attn_enqueue(S->attn[a++], xin, st, stride, 1, NULL, S->step, S->pos0, S->hbuf, S->nbuf, NULL, 0,
                            NULL, S->threads);
    if (e == hipSuccess) e = mark(ev, nev);
    if (e == hipSuccess)
      e = dsh_launch_dense_gate_up(S->dense->wg, S->dense->wu, S->nbuf, NULL, 0, S->dense->H, S->dense->I,
                                   S->dense->h, dsr_stream);
    if (e == hipSuccess) e = mark(ev, nev);
    if (e == hipSuccess)
      e = dsh_launch_dense_down(S->dense->wd, S->dense->h, S->nbuf, NULL, 0, S->dense->H, S->dense->I, 1, S->hbuf,
                                S->xbuf, NULL, 0, NULL, dsr_stream);
    if (e == hipSuccess) e = mark(ev, nev);
    xin = S->xbuf;
    st = NULL;
    stride = 0;
  }
  for (int l = 0; l < S->n_layers && e == hipSuccess; l++) {
    const ds_hip_layer_t *L = S->layers[l];
    float *pin = S->partials[l & 1];
    int np = L->np;
    /* with the copies, the attention's first kernel also writes their sum to xbuf for its residual */
    e = ds_hip_attn_enqueue(S->attn[a++], xin, st, stride, nc, nc > 1 ? S->xbuf : NULL, S->step, S->pos0, S->hbuf,
                            S->nbuf,
                            cfgp ? L->d.router_f32_t : NULL, cfgp ? L->E : 0, cfgp ? pin : NULL, S->threads);
    if (e == hipSuccess) e = mark(ev, nev);
    const uint16_t *wr_dec = dec_fused_router(L, S->route_mode, S->split, S->threads);
    if (S->split) S->sp[l].Wr_dec = wr_dec;
    if (e == hipSuccess && !cfgp && !wr_dec) {
      e = scores_enqueue(L, S->nbuf, NULL, 0, S->route_mode, S->bf16sim, S->threads, pin, &np);
      if (e == hipSuccess) e = mark(ev, nev);
    }
    if (S->split) { /* one kernel: MoE(n) + h into the copies region l, clearing region l - 2 */
      float *out = xc_region(S, l), *zp = l >= 2 ? xc_region(S, l - 2) : NULL;
      if (e == hipSuccess)
        e = dsh_launch_dec_layer(&L->d, &S->sp[l], S->nbuf, NULL, 0, 1, pin, np,
                                 cfg ? DSH_ROUTE_CFG : DSH_ROUTE_DECODE, S->hbuf, out, out + (size_t)C * S->H, zp,
                                 zp ? (int)S->xc_region : 0, dsr_stream);
      if (e == hipSuccess) e = mark(ev, nev);
      xin = out;
      nc = C;
    } else {
      const dsh_rcert_t rc = dsr_rcert(l);
      if (e == hipSuccess)
        e = dsh_launch_dec_gate_up(&L->d, S->nbuf, NULL, 0, pin, np, S->route_mode, S->bf16sim, wk, &rc, dsr_stream);
      if (e == hipSuccess) e = mark(ev, nev);
      if (e == hipSuccess)
        e = dsh_launch_dec_down(&L->d, S->nbuf, NULL, 0, S->xbuf, 1, S->hbuf, S->bf16sim, wk, NULL, 0, NULL,
                                dsr_stream);
      if (e == hipSuccess) e = mark(ev, nev);
      xin = S->xbuf;
      nc = 1;
    }
    st = NULL;
    stride = 0;
  }
  /* the final norm; with the copies it also writes their sum (the hidden state) to xbuf */
  if (e == hipSuccess)
    e = dsh_launch_final_norm(xin, nc, S->final_norm, S->H, S->final_eps, S->trunc_final && S->bf16sim, S->fbuf,
                              nc > 1 ? S->xbuf : NULL, dsr_stream);
  if (e == hipSuccess) e = mark(ev, nev);
  return e;
}

/* The MoE layers as one kernel each (CFG routing): layer l reads its input (the step's input or the
 * dense layer's output for l = 0, else the copies region l - 1 with its router scores) and adds
 * into region l; it also clears region l - 2, read by layer l - 2. The last two regions are cleared
 * by the step's final kernel, or, where the step ends with the LM head, by the next step's first
 * two layers and after a run's last step by tail_enqueue; so every region is zero when a step
 * writes it. The copy sum then writes the plain output for the LM head. */
static float *xc_region(const ds_hip_stack_t *S, int l) { return S->xc + (size_t)l * S->xc_region; }
static int lm_keys(const ds_hip_stack_t *S);

static hipError_t split_layers_enqueue(ds_hip_stack_t *S, hipEvent_t *ev, int *nev) {
  hipError_t e = hipSuccess;
  const int dense = S->dense != NULL, NL = S->n_layers, H = S->H, C = dsh_layer_split_copies();
  const int cfg = S->route_mode == DS_HIP_ROUTE_CFG, mode = cfg ? DSH_ROUTE_CFG : DSH_ROUTE_DECODE;
  const int zn = (int)S->xc_region;
  int np0 = S->layers[0]->np;
  for (int l = 0; l < NL; l++) S->sp[l].Wr_dec = dec_fused_router(S->layers[l], S->route_mode, 1, S->threads);
  if ((cfg ? !dense : !S->sp[0].Wr_dec) && !S->merged) {
    e = scores_enqueue(S->layers[0], dense ? S->xbuf : S->in, dense ? NULL : S->in_step, dense ? 0 : S->in_stride,
                       S->route_mode, S->bf16sim, S->threads, S->partials[0], &np0);
    if (e == hipSuccess) e = mark(ev, nev);
  }
  /* a step that ends with the LM head: the first layer finishes the previous step's token, the last
   * computes the next step's router partials (the step counter is still this step's there) */
  dsh_split_t *F0 = &S->sp[0], *FL = &S->sp[NL - 1];
  F0->fin_cand = S->tailed ? S->cand : NULL;
  F0->fin_n = S->tailed ? lm_keys(S) : 0;
  F0->fin_tokens = S->tailed ? S->tokens : NULL;
  F0->fin_step = S->tailed ? S->step : NULL;
  F0->fin_pending = S->tailed ? S->pending : NULL;
  FL->nx_partials = S->tailed ? S->partials[0] : NULL;
  FL->nx_in = S->tailed ? S->in : NULL;
  FL->nx_step = S->tailed ? S->in_step : NULL;
  FL->nx_stride = S->in_stride;
  FL->nx_rows = S->rows;
  FL->nx_R = dsh_dec_partial_rows(H);
  FL->nx_E = S->layers[0]->E;
  FL->nx_WrT = S->tailed ? S->layers[0]->d.router_f32_t : NULL;
  FL->nx_pending = S->tailed ? S->pending : NULL;
  for (int l = 0; l < NL && e == hipSuccess; l++) {
    const ds_hip_layer_t *L = S->layers[l];
    float *out = xc_region(S, l);
    /* layer l clears region l - 2; with the step ending at the LM head, layers 0 and 1 clear the
     * last two regions, which the final kernel clears otherwise */
    float *zp = l >= 2 ? xc_region(S, l - 2) : S->tailed && l < 2 ? xc_region(S, NL - 2 + l) : NULL;
    if (l == 0) {
      e = dsh_launch_dec_layer(&L->d, &S->sp[l], dense ? S->xbuf : S->in, dense ? NULL : S->in_step,
                               dense ? 0 : S->in_stride, 1, S->partials[0], np0, mode, NULL, out, out + (size_t)C * H, zp,
                               zp ? zn : 0, dsr_stream);
    } else {
      float *in = xc_region(S, l - 1);
      const float *pin = in + (size_t)C * H;  /* CFG: the score copies the previous layer accumulated */
      int np = C;
      if (!cfg && !S->sp[l].Wr_dec) { /* DECODE: the exact scores of the summed input */
        e = dsh_launch_dec_scores_bf16_copies(L->d.router_bf16, in, NULL, 0, C, H, L->E, S->threads,
                                              S->partials[l & 1], dsr_stream);
        if (e == hipSuccess) e = mark(ev, nev);
        pin = S->partials[l & 1];
        np = 1;
      }
      if (e == hipSuccess)
        e = dsh_launch_dec_layer(&L->d, &S->sp[l], in, NULL, 0, C, pin, np, mode, NULL, out, out + (size_t)C * H, zp,
                                 zp ? zn : 0, dsr_stream);
    }
    if (e == hipSuccess) e = mark(ev, nev);
  }
  if (!S->lm_fast) { /* the plain output for the general LM-head path (the fast head sums the copies) */
    if (e == hipSuccess)
      e = dsh_launch_dec_copy_sum(xc_region(S, NL - 1), H, S->xbuf, NL >= 2 ? xc_region(S, NL - 2) : NULL,
                                  NL >= 2 ? zn : 0, dsr_stream);
    if (e == hipSuccess) e = mark(ev, nev);
  }
  return e;
}

/* The fast LM head on the last layer's copies (its block 0 writes the plain output, the hidden
 * state); the final kernel after it then clears the last two copies regions. */
static hipError_t split_lm_enqueue(ds_hip_stack_t *S) {
  return dsh_launch_dec_lm_argmax_copies(S->lm, xc_region(S, S->n_layers - 1), dsh_layer_split_copies(), S->H,
                                         S->vocab, S->cand, S->xbuf, S->merged ? S->step : NULL, dsr_stream);
}

/* The step's final kernel: the token into tokens[step], the step counter advanced, the last copies
 * regions cleared (one-kernel layers) and, with the embedding feed and no sampling rules after it,
 * the next step's input row. */
/* Keys the step's head writes: one per block of the kernel in use. */
static int lm_keys(const ds_hip_stack_t *S) { return S->lm_fast && S->lm_cert ? dsh_lm_q8_blocks(S->vocab) : S->ncand; }

static hipError_t final_enqueue(ds_hip_stack_t *S, int clear) {
  const int NL = S->n_layers, embed = S->emb && !smp_active(S);
  float *zp = clear ? xc_region(S, NL >= 2 ? NL - 2 : 0) : NULL;
  const int zn = clear ? (int)S->xc_region * (NL >= 2 ? 2 : 1) : 0;
  if (S->merged) {
    const ds_hip_layer_t *L0 = S->layers[0];
    return dsh_launch_lm_final_scores(S->cand, lm_keys(S), S->tokens, S->step, zp, zn, embed ? S->emb : NULL,
                                      S->emb_vocab, embed ? S->ebuf : NULL, S->xs, S->stride, S->rows,
                                      L0->d.router_f32_t, S->H, L0->E, S->partials[0], dsr_stream);
  }
  return dsh_launch_lm_argmax_final(S->cand, lm_keys(S), S->tokens, S->step, zp, zn, embed ? S->emb : NULL,
                                    S->emb_vocab, S->H, embed ? S->ebuf : NULL, dsr_stream);
}

/* Whether the one-kernel layers apply: no bf16 simulation, no attention, supported shapes (in
 * DECODE routing each layer keeps its exact scores kernel before it). */
static int split_eligible(const ds_hip_stack_t *S) {
  if (!S->split_want || S->bf16sim) return 0;
  const int cfg = S->route_mode == DS_HIP_ROUTE_CFG;
  for (int l = 0; l < S->n_layers; l++)
    if (!dsh_layer_split_supported(&S->layers[l]->d) || (cfg && !dsh_layer_cert_supported(&S->layers[l]->d)))
      return 0;
  return 1;
}

/* Whether the final kernel also computes the next step's first router partials. */
static int merged_eligible(const ds_hip_stack_t *S) {
  return S->split && S->route_mode == DS_HIP_ROUTE_CFG && !S->bf16sim && !S->dense && !S->attn && S->lm_fast &&
         !smp_active(S);
}

/* The current step's first router partials, where the step's final kernel computes the next ones
 * (after a reset, and at every run call: the caller may have rewritten the bound input since). */
static int scores_refresh(ds_hip_stack_t *S) {
  if (!S->merged) return 0;
  const ds_hip_layer_t *L0 = S->layers[0];
  DSR_TRY(dsh_launch_dec_partial_scores(L0->d.router_f32_t, S->in, S->in_step, S->in_stride, S->H, L0->E,
                                        S->partials[0], dsr_stream),
          "router partials");
  return 0;
}

/* Sleeps after which a routed block of a one-kernel layer stops waiting for its rank's verdict (the
 * verifier's work takes a few microseconds, its exact fallback some more). */

/* Allocates and fills the per-layer tiles and products and the copies regions. */
static int split_build(ds_hip_stack_t *S) {
  if (S->split_arena) {
    hipFree(S->split_arena);
    S->split_arena = NULL;
  }
  free(S->sp);
  S->sp = NULL;
  const int NL = S->n_layers, C = dsh_layer_split_copies();
  size_t bytes = 0;
  for (int l = 0; l < NL; l++) {
    const dsh_layer_t *d = &S->layers[l]->d;
    bytes += al(dsh_layer_split_tile_bytes(d));
    if (l + 1 < NL && S->route_mode == DS_HIP_ROUTE_CFG && !S->attn)
      bytes += al(dsh_layer_split_m_floats(d) * 4) + al((size_t)(d->E + 1) * 64 * 4);
  }
  /* per layer: the output copies, the next router's score copies, the routing verdict area */
  S->xc_region = (size_t)C * S->H + (size_t)C * 64 + DSH_SPLIT_VD_INTS;
  bytes += al((size_t)NL * S->xc_region * 4);
  S->sp = (dsh_split_t *)calloc((size_t)NL, sizeof(dsh_split_t));
  if (!S->sp) return dsr_failf("split layer tables: out of memory");
  hipError_t e = hipMalloc(&S->split_arena, bytes);
  if (e != hipSuccess) {
    S->split_arena = NULL;
    return dsr_fail("one-kernel layer arena allocation", e);
  }
  char *b = (char *)S->split_arena;
  S->xc = (float *)b; /* the regions first (their verdict areas are 128-byte aligned) */
  b += al((size_t)NL * S->xc_region * 4);
  for (int l = 0; l < NL && e == hipSuccess; l++) {
    const dsh_layer_t *d = &S->layers[l]->d;
    dsh_split_t *F = &S->sp[l];
    int8_t *tiles = (int8_t *)b;
    const size_t routed = (size_t)d->E * d->I * d->H;
    b += al(dsh_layer_split_tile_bytes(d));
    float *M = NULL, *z = NULL;
    /* the next router's products: CFG routing only (DECODE scores come from the exact kernel) */
    const dsh_layer_t *nx = l + 1 < NL && S->route_mode == DS_HIP_ROUTE_CFG && !S->attn ? &S->layers[l + 1]->d : NULL;
    if (nx) {
      M = (float *)b;
      b += al(dsh_layer_split_m_floats(d) * 4);
      z = (float *)b;
      b += al((size_t)(d->E + 1) * 64 * 4);
    }
    F->dnT = tiles;
    F->sdnT = tiles + routed;
    F->M = M;
    F->sM = M ? M + (size_t)d->E * d->I * 64 : NULL;
    F->z = z;
    F->sz = z ? z + (size_t)d->E * 64 : NULL;
    F->WrT_next = nx ? nx->router_f32_t : NULL;
    F->E_next = nx ? nx->E : 0;
    /* CFG routing: the selection certified against ds_linear's order by a verifier block per XCD */
    if (S->route_mode == DS_HIP_ROUTE_CFG) {
      F->vd = (unsigned *)(S->xc + (size_t)l * S->xc_region + (size_t)C * S->H + (size_t)C * 64);
      F->derr = dsr_derr_dev(DSR_DERR_ROUTE_WAIT);
      F->rc = dsr_rcert(l);
    } else {
      F->rc = dsr_rcert(l); /* DECODE: the routing log only (one routed block records each layer's selection) */
    }
    e = dsh_launch_layer_build(d, F->WrT_next, F->E_next, tiles, tiles + routed, M, (float *)F->sM, z, (float *)F->sz,
                               dsr_stream);
  }
  /* each layer's kernel reads the next layer's shared-expert data ahead, where its grid has no
   * verifier blocks (DECODE routing): with them (certified CFG routing) the grid holds more blocks
   * than there are CUs, the read-ahead blocks start only as others finish, and the step ran
   * 148.43-148.54 us without them against 148.62-148.72 us with them */
  for (int l = 0; l + 1 < NL && S->route_mode != DS_HIP_ROUTE_CFG; l++) {
    const dsh_layer_t *nd = &S->layers[l + 1]->d;
    if (nd->H != S->layers[l]->d.H) continue;
    S->sp[l].pf_gu = nd->sgu_q;
    S->sp[l].pf_guso = nd->sgu_so;
    S->sp[l].pf_dnT = S->sp[l + 1].sdnT;
    S->sp[l].pf_M = S->sp[l + 1].sM;
    S->sp[l].pf_SI = nd->SI;
  }
  if (e == hipSuccess) e = hipMemsetAsync(S->xc, 0, (size_t)NL * S->xc_region * 4, dsr_stream);
  if (e == hipSuccess) e = hipStreamSynchronize(dsr_stream);
  if (e != hipSuccess) return dsr_fail("one-kernel layer tables", e);
  return 0;
}

int ds_hip_stack_set_layer_kernels(ds_hip_stack_t *S, int one_kernel) {
  if (!S || S->bound) return dsr_failf("ds_hip_stack_set_layer_kernels: NULL stack or already bound");
  S->split_want = one_kernel != 0;
  return 0;
}

int ds_hip_stack_layer_kernels(const ds_hip_stack_t *S) { return S && S->split ? 1 : 2; }

static hipError_t step_enqueue(ds_hip_stack_t *S, hipEvent_t *ev) {
  hipError_t e = hipSuccess;
  int n = 0;
  const int cfg = S->route_mode == DS_HIP_ROUTE_CFG;
  const int cfgp = cfg && !S->bf16sim; /* CFG scores as partials from the kernel before */
  const dsh_layer_work_t *wk = &S->layers[0]->wk;
  e = mark(ev, &n);
  if (S->attn) {
    e = layers_full_enqueue(S, ev, &n);
  } else {
    const int dense = S->dense != NULL;
    if (dense) {  /* layer 0: x = x + FFN(x); in CFG mode also the first MoE layer's router partials */
      e = dsh_launch_dense_gate_up(S->dense->wg, S->dense->wu, S->in, S->in_step, S->in_stride, S->dense->H, S->dense->I,
                                   S->dense->h, dsr_stream);
      if (e == hipSuccess) e = mark(ev, &n);
      if (e == hipSuccess)
        e = dsh_launch_dense_down(S->dense->wd, S->dense->h, S->in, S->in_step, S->in_stride, S->dense->H, S->dense->I, 1, NULL,
                                  S->xbuf, cfgp ? S->layers[0]->d.router_f32_t : NULL, cfgp ? S->layers[0]->E : 0,
                                  cfgp ? S->partials[0] : NULL, dsr_stream);
      if (e == hipSuccess) e = mark(ev, &n);
    }
    if (S->split && e == hipSuccess) {
      e = split_layers_enqueue(S, ev, &n);
    } else
    for (int l = 0; l < S->n_layers && e == hipSuccess; l++) {
      const ds_hip_layer_t *L = S->layers[l];
      const int first = l == 0 && !dense; /* reads the step's input directly */
      const float *xin = first ? S->in : S->xbuf;
      const int *st = first ? S->in_step : NULL;
      int stride = first ? S->in_stride : 0;
      float *pin = S->partials[l & 1], *pout = S->partials[(l + 1) & 1];
      int np = L->np;
      if (!cfgp || first) {
        e = scores_enqueue(L, xin, st, stride, S->route_mode, S->bf16sim, S->threads, pin, &np);
        if (e == hipSuccess) e = mark(ev, &n);
        if (e != hipSuccess) break;
      }
      const ds_hip_layer_t *next = cfgp && l + 1 < S->n_layers ? S->layers[l + 1] : NULL;
      const dsh_rcert_t rc = dsr_rcert(l);
      e = dsh_launch_dec_gate_up(&L->d, xin, st, stride, pin, np, S->route_mode, S->bf16sim, wk, &rc, dsr_stream);
      if (e == hipSuccess) e = mark(ev, &n);
      if (e == hipSuccess)
        e = dsh_launch_dec_down(&L->d, xin, st, stride, S->xbuf, 1, NULL, S->bf16sim, wk, next ? next->d.router_f32_t : NULL,
                                next ? next->E : 0, next ? pout : NULL, dsr_stream);
      if (e == hipSuccess) e = mark(ev, &n);
    }
  }
  if (e != hipSuccess) return e;
  const int lm_copies = S->split && S->lm_fast && !S->attn;
  const int clear_in_final = S->split && (S->lm_fast || S->attn); /* else copy_sum cleared them */
  if (S->lm_fast && S->lm_cert) {
    /* on the layer copies (block 0 writes the plain output, the hidden state) or on the head's input */
    e = dsh_launch_lm_q8(S->lm, &S->lmq, lm_copies ? xc_region(S, S->n_layers - 1) : lm_in(S),
                         lm_copies ? dsh_layer_split_copies() : 0, lm_copies ? S->xbuf : NULL, S->cand,
                         lm_copies && S->merged ? S->step : NULL, dsr_stream);
  } else if (lm_copies) {
    e = split_lm_enqueue(S);
  } else if (S->lm_fast) {
    e = dsh_launch_dec_lm_argmax(S->lm, lm_in(S), S->H, S->vocab, S->cand, dsr_stream);
  } else {
    int T = S->threads;
    e = dsh_launch_argmax_avx_partial(S->lm, lm_in(S), S->cand, NULL, S->H, S->vocab,
                                      T > 1 ? (S->vocab + T - 1) / T : S->vocab, dsr_stream);
  }
  if (e == hipSuccess) e = mark(ev, &n);
  if (!S->tailed) {
    if (e == hipSuccess) e = final_enqueue(S, clear_in_final);
    if (e == hipSuccess) e = mark(ev, &n);
  }
  if (e == hipSuccess && smp_active(S)) {
    /* the repetition penalty and the n-gram ban over this stack's earlier tokens, then (embedding
     * feed) the final token's row; one event after all of these kernels */
    e = dsh_launch_sample(S->lm, lm_in(S), S->H, S->vocab, S->threads, S->rp, S->ngram, S->step, S->tokens, NULL,
                          S->hist_cap, smp_vals(S), smp_logits(S), smp_flag(S), dsr_stream);
    if (e == hipSuccess && S->emb)
      e = dsh_launch_embed_next(S->tokens, S->step, S->emb, S->emb_vocab, S->H, S->ebuf, dsr_stream);
    if (e == hipSuccess) e = mark(ev, &n);
  }
  return e;
}

int ds_hip_stack_capacity_for(int n_rows, int stride, int n_tokens, int kv_room) {
  if (n_rows < 1 || n_tokens < 1 || stride < 0) return -1;
  int cap = n_tokens;
  if (stride > 0 && n_rows < cap) cap = n_rows;
  if (kv_room >= 0 && kv_room < cap) cap = kv_room;
  return cap;
}

int ds_hip_steps_fit(int capacity, int steps_done, int n) {
  return capacity >= 0 && steps_done >= 0 && n >= 0 && steps_done <= capacity && n <= capacity - steps_done;
}

/* KV positions left for the stack's steps: min over its attention blocks of max_seq - pos0 (-1:
 * no attention). */
static int stack_kv_room(const ds_hip_stack_t *S) {
  if (!S->attn) return -1;
  int room = -1;
  for (int i = 0; i < S->n_attn; i++) {
    int r = ds_hip_attn_max_seq(S->attn[i]) - S->pos0;
    if (r < 0) r = 0;
    if (room < 0 || r < room) room = r;
  }
  return room;
}

int ds_hip_stack_set_embedding(ds_hip_stack_t *S, const uint16_t *tok_embeddings_dev, int vocab) {
  if (!S) return dsr_failf("ds_hip_stack_set_embedding: NULL stack");
  if (S->bound) return dsr_failf("ds_hip_stack_set_embedding: call before ds_hip_stack_bind");
  if (!tok_embeddings_dev) {
    S->emb = NULL;
    S->emb_vocab = 0;
    return 0;
  }
  if (vocab <= 0 || S->H % 8 || ((uintptr_t)tok_embeddings_dev & 15))
    return dsr_failf("ds_hip_stack_set_embedding: need vocab > 0, hidden %% 8 == 0 and a 16-byte aligned table");
  S->emb = tok_embeddings_dev;
  S->emb_vocab = vocab;
  return 0;
}

/* One graph of k steps (step_enqueue captured k times), instantiated into *out. */
static int capture_steps(ds_hip_stack_t *S, int k, hipGraphExec_t *out) {
  DSR_TRY(hipStreamBeginCapture(dsr_stream, hipStreamCaptureModeThreadLocal), "graph capture begin");
  hipError_t e = hipSuccess;
  for (int i = 0; i < k && e == hipSuccess; i++) e = step_enqueue(S, NULL);
  hipGraph_t g = NULL;
  hipError_t e2 = hipStreamEndCapture(dsr_stream, &g);
  if (e != hipSuccess || e2 != hipSuccess || !g) {
    if (g) hipGraphDestroy(g);
    return dsr_fail("graph capture", e != hipSuccess ? e : e2);
  }
  e = hipGraphInstantiate(out, g, NULL, NULL, 0);
  hipGraphDestroy(g);
  if (e != hipSuccess) {
    *out = NULL;
    return dsr_fail("graph instantiate", e);
  }
  return 0;
}

int ds_hip_stack_bind(ds_hip_stack_t *S, const float *xs_dev, int stride, int n_rows, int *tokens_dev,
                      int n_tokens) {
  if (!S || !xs_dev || !tokens_dev || stride < 0 || n_rows < 1 || n_tokens < 1)
    return dsr_failf("ds_hip_stack_bind: invalid arguments (need xs_dev, tokens_dev, stride >= 0, n_rows >= 1, "
                     "n_tokens >= 1)");
  /* an earlier launch of the old graph may still run on the stream: let it finish first */
  DSR_TRY(hipStreamSynchronize(dsr_stream), "bind");
  if (S->exec) {
    hipGraphExecDestroy(S->exec);
    S->exec = NULL;
  }
  if (S->exec_k) {
    hipGraphExecDestroy(S->exec_k);
    S->exec_k = NULL;
  }
  if (S->graph) {
    hipGraphDestroy(S->graph);
    S->graph = NULL;
  }
  S->bound = 0;
  S->xs = xs_dev;
  S->stride = stride;
  S->tokens = tokens_dev;
  /* with the embedding feed only row 0 of xs is read (at reset, into ebuf) */
  S->in = S->emb ? S->ebuf : xs_dev;
  S->in_step = S->emb ? NULL : S->step;
  S->in_stride = S->emb ? 0 : stride;
  S->cap = ds_hip_stack_capacity_for(n_rows, S->emb ? 0 : stride, n_tokens, stack_kv_room(S));
  DSR_TRY(hipStreamSynchronize(dsr_stream), "bind");
  S->rows = n_rows;
  S->split = split_eligible(S);
  if (S->split && split_build(S)) return -1;
  S->merged = merged_eligible(S);
  S->tailed = S->merged && !S->emb && S->n_layers >= 3;
  DSR_TRY(hipStreamBeginCapture(dsr_stream, hipStreamCaptureModeThreadLocal), "graph capture begin");
  hipError_t e = step_enqueue(S, NULL);
  hipGraph_t g = NULL;
  hipError_t e2 = hipStreamEndCapture(dsr_stream, &g);
  if (e != hipSuccess) {
    if (g) hipGraphDestroy(g);
    return dsr_fail("graph capture", e);
  }
  if (e2 != hipSuccess) return dsr_fail("graph capture end", e2);
  S->graph = g;
  DSR_TRY(hipGraphInstantiate(&S->exec, g, NULL, NULL, 0), "graph instantiate");
  if (S->gk > 1 && capture_steps(S, S->gk, &S->exec_k)) return -1;
  S->bound = 1;
  return ds_hip_stack_reset(S);
}

int ds_hip_stack_set_graph_steps(ds_hip_stack_t *S, int k) {
  if (!S || k < 1 || k > DS_HIP_GRAPH_STEPS_MAX)
    return dsr_failf("ds_hip_stack_set_graph_steps: steps per graph must be 1..%d", DS_HIP_GRAPH_STEPS_MAX);
  if (k == S->gk) return 0;
  DSR_TRY(hipStreamSynchronize(dsr_stream), "graph steps"); /* a launch of the old graph may still run */
  if (S->exec_k) {
    hipGraphExecDestroy(S->exec_k);
    S->exec_k = NULL;
  }
  S->gk = k;
  return S->bound && k > 1 ? capture_steps(S, k, &S->exec_k) : 0;
}

int ds_hip_stack_capacity(const ds_hip_stack_t *S) { return S && S->bound ? S->cap : 0; }

int ds_hip_stack_steps_left(const ds_hip_stack_t *S) { return S && S->bound ? S->cap - S->done : 0; }

/* Zeroes the step counter (and the work buffers with it); with the embedding feed, row 0 of the
 * bound input becomes the first step's input. */
int ds_hip_stack_reset(ds_hip_stack_t *S) {
  if (!S || !S->bound) return dsr_failf("ds_hip_stack_reset: stack not bound");
  DSR_TRY(hipMemsetAsync(S->work, 0, S->work_bytes, dsr_stream), "reset stack");
  if (S->split && S->xc)
    DSR_TRY(hipMemsetAsync(S->xc, 0, (size_t)S->n_layers * S->xc_region * 4, dsr_stream), "reset stack");
  if (S->emb)
    DSR_TRY(hipMemcpyAsync(S->ebuf, S->xs, (size_t)S->H * 4, hipMemcpyDeviceToDevice, dsr_stream), "reset stack");
  S->done = 0;
  return scores_refresh(S);
}

/* Refuses, before anything is launched, n more steps than the bound buffers hold. */
static int steps_check(const ds_hip_stack_t *S, int n, const char *who) {
  if (!S || !S->bound) return dsr_failf("%s: stack not bound", who);
  if (!ds_hip_steps_fit(S->cap, S->done, n))
    return dsr_failf("%s: %d more steps after %d would pass the stack's capacity of %d (rows of the bound input, "
                     "length of the token array, KV positions); reset or bind larger buffers",
                     who, n, S->done, S->cap);
  return 0;
}

/* After a run's steps when they end with the LM head: the last step's token (if still pending) and
 * the last two copies regions cleared. */
static hipError_t tail_enqueue(ds_hip_stack_t *S) {
  if (!S->tailed) return hipSuccess;
  const int NL = S->n_layers;
  return dsh_launch_lm_token_pending(S->cand, lm_keys(S), S->tokens, S->step, S->pending, xc_region(S, NL - 2),
                                     (int)(2 * S->xc_region), dsr_stream);
}

static int graph_steps(ds_hip_stack_t *S, int n_steps) {
  int i = 0;
  for (; S->exec_k && i + S->gk <= n_steps; i += S->gk) {
    DSR_TRY(hipGraphLaunch(S->exec_k, dsr_stream), "graph launch");
    S->done += S->gk;
  }
  for (; i < n_steps; i++) {
    DSR_TRY(hipGraphLaunch(S->exec, dsr_stream), "graph launch");
    S->done++;
  }
  DSR_TRY(tail_enqueue(S), "run tail");
  return 0;
}

int ds_hip_stack_run(ds_hip_stack_t *S, int n_steps) {
  if (steps_check(S, n_steps, "ds_hip_stack_run") || scores_refresh(S)) return -1;
  return graph_steps(S, n_steps);
}

int ds_hip_stack_run_eager(ds_hip_stack_t *S, int n_steps) {
  if (steps_check(S, n_steps, "ds_hip_stack_run_eager") || scores_refresh(S)) return -1;
  for (int i = 0; i < n_steps; i++) {
    hipError_t e = step_enqueue(S, NULL);
    S->done++;
    if (e != hipSuccess) return dsr_fail("decode step", e);
  }
  DSR_TRY(tail_enqueue(S), "run tail");
  return 0;
}

int ds_hip_stack_hidden(ds_hip_stack_t *S, float *x_host) {
  if (!S || !x_host) return -1;
  return dsr_d2h(x_host, S->xbuf, (size_t)S->H * 4);
}

int ds_hip_time_stack(ds_hip_stack_t *S, int n_steps, float *ms) {
  if (!ms) return dsr_failf("ds_hip_time_stack: invalid arguments");
  if (steps_check(S, n_steps, "ds_hip_time_stack") || scores_refresh(S)) return -1;
  hipEvent_t a, b;
  DSR_TRY(hipEventCreate(&a), "event");
  DSR_TRY(hipEventCreate(&b), "event");
  int rc = 0;
  if (hipEventRecord(a, dsr_stream) != hipSuccess || graph_steps(S, n_steps) ||
      hipEventRecord(b, dsr_stream) != hipSuccess || hipEventSynchronize(b) != hipSuccess ||
      hipEventElapsedTime(ms, a, b) != hipSuccess)
    rc = dsr_failf("ds_hip_time_stack: timing failed");
  hipEventDestroy(a);
  hipEventDestroy(b);
  return rc;
}

/* Creates n events (all or none). */
static int events_create(hipEvent_t *ev, int n) {
  for (int i = 0; i < n; i++)
    if (hipEventCreate(&ev[i]) != hipSuccess) {
      while (i--) hipEventDestroy(ev[i]);
      return dsr_failf("event creation failed");
    }
  return 0;
}

static void events_destroy(hipEvent_t *ev, int n) {
  for (int i = 0; i < n; i++)
    if (ev[i]) hipEventDestroy(ev[i]);
}

int ds_hip_time_stack_each(ds_hip_stack_t *S, int n_steps, float *ms_each) {
  if (!ms_each || n_steps <= 0) return dsr_failf("ds_hip_time_stack_each: invalid arguments");
  if (steps_check(S, n_steps, "ds_hip_time_stack_each") || scores_refresh(S)) return -1;
  hipEvent_t *ev = (hipEvent_t *)calloc((size_t)n_steps + 1, sizeof(hipEvent_t));
  if (!ev || events_create(ev, n_steps + 1)) {
    free(ev);
    return dsr_failf("ds_hip_time_stack_each: events");
  }
  hipError_t e = hipEventRecord(ev[0], dsr_stream);
  for (int i = 0; i < n_steps && e == hipSuccess; i++) {
    e = hipGraphLaunch(S->exec, dsr_stream);
    S->done++;
    if (e == hipSuccess) e = hipEventRecord(ev[i + 1], dsr_stream);
  }
  if (e == hipSuccess) e = tail_enqueue(S);
  if (e == hipSuccess) e = hipEventSynchronize(ev[n_steps]);
  for (int i = 0; i < n_steps && e == hipSuccess; i++) e = hipEventElapsedTime(&ms_each[i], ev[i], ev[i + 1]);
  events_destroy(ev, n_steps + 1);
  free(ev);
  if (e != hipSuccess) return dsr_fail("ds_hip_time_stack_each", e);
  return 0;
}

int ds_hip_time_stack_span(ds_hip_stack_t *S, int n_steps, int k0, int k1, float *ms_each) {
  if (!ms_each || n_steps <= 0) return dsr_failf("ds_hip_time_stack_span: invalid arguments");
  if (steps_check(S, n_steps, "ds_hip_time_stack_span") || scores_refresh(S)) return -1;
  const int nk = stack_kernel_count(S);
  if (k0 < 0 || k1 <= k0 || k1 > nk) return dsr_failf("ds_hip_time_stack_span: kernel range [%d, %d) of %d", k0, k1, nk);
  hipEvent_t *marks = (hipEvent_t *)calloc((size_t)nk + 1, sizeof(hipEvent_t));
  hipEvent_t *ev = (hipEvent_t *)calloc(2 * (size_t)n_steps, sizeof(hipEvent_t));
  if (!marks || !ev || events_create(ev, 2 * n_steps)) {
    free(marks);
    free(ev);
    return dsr_failf("ds_hip_time_stack_span: events");
  }
  hipError_t e = hipSuccess;
  for (int i = 0; i < n_steps && e == hipSuccess; i++) {
    marks[k0] = ev[2 * i];
    marks[k1] = ev[2 * i + 1];
    e = step_enqueue(S, marks);
    S->done++;
  }
  if (e == hipSuccess) e = tail_enqueue(S);
  if (e == hipSuccess) e = hipEventSynchronize(ev[2 * n_steps - 1]);
  for (int i = 0; i < n_steps && e == hipSuccess; i++) e = hipEventElapsedTime(&ms_each[i], ev[2 * i], ev[2 * i + 1]);
  events_destroy(ev, 2 * n_steps);
  free(ev);
  free(marks);
  if (e != hipSuccess) return dsr_fail("ds_hip_time_stack_span", e);
  return 0;
}

/* LM-head argmax kernel alone on the stack's current hidden state: n launches back to back
 * between two events (kernel time plus the launch gaps). */
int ds_hip_time_lm_head(ds_hip_stack_t *S, int n, float *ms) {
  if (!S || !S->bound || !ms || n <= 0) return dsr_failf("ds_hip_time_lm_head: invalid arguments");
  hipEvent_t a, b;
  DSR_TRY(hipEventCreate(&a), "event");
  DSR_TRY(hipEventCreate(&b), "event");
  int rc = 0;
  hipError_t e = hipEventRecord(a, dsr_stream);
  for (int i = 0; i < n && e == hipSuccess; i++) {
    if (S->lm_fast && S->lm_cert) {
      /* on the step's head input (the layer copies are cleared after a step; the last hidden state
       * is the same vector, so the candidates are those of the last step) */
      e = dsh_launch_lm_q8(S->lm, &S->lmq, lm_in(S), 0, NULL, S->cand, NULL, dsr_stream);
    } else if (S->split && S->lm_fast && !S->attn) {  /* the head kernel of the step (on the layer copies) */
      e = dsh_launch_dec_lm_argmax_copies(S->lm, xc_region(S, S->n_layers - 1), dsh_layer_split_copies(), S->H,
                                          S->vocab, S->cand, NULL, NULL, dsr_stream);
    } else if (S->lm_fast) {
      e = dsh_launch_dec_lm_argmax(S->lm, lm_in(S), S->H, S->vocab, S->cand, dsr_stream);
    } else {
      int T = S->threads;
      e = dsh_launch_argmax_avx_partial(S->lm, lm_in(S), S->cand, NULL, S->H, S->vocab,
                                        T > 1 ? (S->vocab + T - 1) / T : S->vocab, dsr_stream);
    }
  }
  if (e == hipSuccess) e = hipEventRecord(b, dsr_stream);
  if (e == hipSuccess) e = hipEventSynchronize(b);
  if (e == hipSuccess) e = hipEventElapsedTime(ms, a, b);
  if (e != hipSuccess) rc = dsr_fail("ds_hip_time_lm_head", e);
  else *ms /= (float)n;
  hipEventDestroy(a);
  hipEventDestroy(b);
  return rc;
}

int ds_hip_stack_kernel_count(const ds_hip_stack_t *S) { return S ? stack_kernel_count(S) : 0; }

const char *ds_hip_stack_kernel_name(const ds_hip_stack_t *S, int i) {
  if (!S || i < 0 || i >= stack_kernel_count(S)) return NULL;
  const char **names = (const char **)malloc(sizeof(const char *) * (size_t)stack_kernel_count(S));
  if (!names) return NULL;
  stack_names(S, names);
  const char *r = names[i];
  free(names);
  return r;
}

int ds_hip_profile_stack(ds_hip_stack_t *S, int n_steps, float *ms_out) {
  if (!ms_out || n_steps <= 0) return dsr_failf("ds_hip_profile_stack: invalid arguments");
  if (steps_check(S, n_steps, "ds_hip_profile_stack") || scores_refresh(S)) return -1;
  int nk = stack_kernel_count(S);
  hipEvent_t *ev = (hipEvent_t *)calloc((size_t)(nk + 1), sizeof(hipEvent_t));
  double *acc = (double *)calloc((size_t)nk, sizeof(double));
  int rc = 0;
  for (int i = 0; i <= nk; i++)
    if (hipEventCreate(&ev[i]) != hipSuccess) rc = -1;
  for (int s = 0; s < n_steps && rc == 0; s++) {
    hipError_t e = step_enqueue(S, ev);
    S->done++;
    if (e != hipSuccess || hipEventSynchronize(ev[nk]) != hipSuccess) {
      rc = -1;
      break;
    }
    for (int i = 0; i < nk; i++) {
      float m = 0;
      hipEventElapsedTime(&m, ev[i], ev[i + 1]);
      acc[i] += m;
    }
  }
  if (rc == 0 && tail_enqueue(S) != hipSuccess) rc = -1;
  for (int i = 0; i < nk; i++) ms_out[i] = (float)(acc[i] / n_steps);
  for (int i = 0; i <= nk; i++)
    if (ev[i]) hipEventDestroy(ev[i]);
  free(ev);
  free(acc);
  return rc ? dsr_failf("ds_hip_profile_stack failed") : 0;
}

/* ================================================================ device-pointer kernels */

int ds_hip_quantize_bf16(int8_t *q_dev, float *scale_dev, float *offset_dev, const uint16_t *W_dev, int out_dim,
                         int in_dim) {
  if (dsr_init()) return -1;
  if (!q_dev || !scale_dev || !offset_dev || !W_dev || out_dim <= 0 || in_dim <= 0)
    return dsr_failf("ds_hip_quantize_bf16: invalid arguments");
  DSR_TRY(dsh_launch_quantize_bf16(W_dev, q_dev, scale_dev, offset_dev, out_dim, in_dim, dsr_stream), "quantize");
  return 0;
}

int ds_hip_int8_matvec(float *y_dev, const float *x_dev, const int8_t *q_dev, const float *scale_dev,
                       const float *offset_dev, int in_dim, int row_start, int nrows) {
  if (dsr_init()) return -1;
  if (!y_dev || !x_dev || !q_dev || !scale_dev || !offset_dev || in_dim <= 0 || row_start < 0 || nrows < 0)
    return dsr_failf("ds_hip_int8_matvec: invalid arguments");
  DSR_TRY(dsh_launch_int8_matvec(q_dev, scale_dev, offset_dev, x_dev, y_dev, in_dim, row_start, nrows, dsr_stream),
          "int8 matvec");
  return 0;
}

int ds_hip_argmax_bf16(int *idx_dev, const float *x_dev, const uint16_t *W_dev, int in_dim, int out_dim) {
  if (dsr_init()) return -1;
  if (!idx_dev || !x_dev || !W_dev || in_dim <= 0 || out_dim <= 0)
    return dsr_failf("ds_hip_argmax_bf16: invalid arguments");
  int nb = dsh_argmax_avx_blocks(out_dim);
  unsigned long long *cand = (unsigned long long *)dsr_scratch(DSR_SLOT_C, (size_t)nb * 8);
  if (!cand) return -1;
  DSR_TRY(dsh_launch_argmax_avx(W_dev, x_dev, cand, NULL, in_dim, out_dim, dsr_threads(), idx_dev, NULL, dsr_stream),
          "argmax");
  return 0;
}

int ds_hip_argmax_bf16_noalloc(int *idx_dev, const float *x_dev, const uint16_t *W_dev, int in_dim, int out_dim) {
  if (!dsr_ready()) return dsr_failf("ds_hip_argmax_bf16_noalloc: call ds_hip_init first");
  if (!idx_dev || !x_dev || !W_dev || in_dim <= 0 || out_dim <= 0)
    return dsr_failf("ds_hip_argmax_bf16_noalloc: invalid arguments");
  if (dsh_argmax_avx_blocks(out_dim) > DSH_STATIC_CAND)
    return dsr_failf("ds_hip_argmax_bf16_noalloc: out_dim %d exceeds the maximum of %d rows", out_dim,
                     64 * DSH_STATIC_CAND);
  unsigned long long *cand = dsh_static_scratch();
  if (!cand) return dsr_failf("ds_hip_argmax_bf16_noalloc: no static scratch on this device");
  DSR_TRY(dsh_launch_argmax_avx(W_dev, x_dev, cand, NULL, in_dim, out_dim, dsr_threads(), idx_dev, NULL, dsr_stream),
          "argmax");
  return 0;
}

int ds_hip_fill_normal_bf16(uint16_t *dst_dev, size_t n, uint64_t seed, float std_) {
  if (dsr_init()) return -1;
  DSR_TRY(dsh_launch_fill_normal_bf16(dst_dev, n, seed, std_, dsr_stream), "fill normal");
  return 0;
}

int ds_hip_fill_normal_f32(float *dst_dev, size_t n, uint64_t seed, float mean, float std_) {
  if (dsr_init()) return -1;
  DSR_TRY(dsh_launch_fill_normal_f32(dst_dev, n, seed, mean, std_, dsr_stream), "fill normal");
  return 0;
}
