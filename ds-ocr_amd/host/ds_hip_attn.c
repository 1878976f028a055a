/* ds_hip_attn.c — the attention half of a decoder layer (decoder_layer_forward,
 * ds_moe_decoder.c:339-431) on the device: one arena per layer holds the bf16 projections, the
 * norms, the RoPE cos/sin table, the F32 KV caches and the per-token scratch. */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "ds_hip.h"
#include "dsr.h"

struct ds_hip_attn {
  dsh_attn_t d;
  void *arena;
  size_t bytes;
  int prefill_len, window; /* R-SWA (window 0: causal) */
};

static size_t al256(size_t n) { return (n + 255) & ~(size_t)255; }

/* ds_compute_rope_neox (ds_kernels.c:2407-2424) for positions 0..max_seq-1: the same expressions
 * on the same host libm, so the table equals the reference's cache. */
static void rope_table(float *c, float *s, int max_seq, int head_dim, float theta) {
  int half = head_dim / 2;
  for (int p = 0; p < max_seq; p++)
    for (int d = 0; d < half; d++) {
      float freq = 1.0f / powf(theta, (float)(2 * d) / (float)head_dim);
      float angle = (float)p * freq;
      float cv = cosf(angle), sv = sinf(angle);
      c[(size_t)p * head_dim + d] = c[(size_t)p * head_dim + d + half] = cv;
      s[(size_t)p * head_dim + d] = s[(size_t)p * head_dim + d + half] = sv;
    }
}

ds_hip_attn_t *ds_hip_attn_create(int hidden, int n_heads, int head_dim, int max_seq, float rms_eps, float rope_theta,
                                  const uint16_t *wq, const uint16_t *wk, const uint16_t *wv, const uint16_t *wo,
                                  const float *input_norm, const float *post_attn_norm, const float *q_norm,
                                  const float *k_norm) {
  if (dsr_init()) return NULL;
  if (!wq || !wk || !wv || !wo || !input_norm || !post_attn_norm || max_seq <= 0 || max_seq > DS_HIP_ATTN_MAX_SEQ ||
      !dsh_attn_supported(hidden, n_heads, head_dim)) {
    dsr_failf("ds_hip_attn_create: invalid arguments or shape (hidden %d, %d heads x %d, max_seq %d; need hidden and "
              "heads*head_dim multiples of 256 up to 2048, head_dim a multiple of 64 up to 256, max_seq <= %d)",
              hidden, n_heads, head_dim, max_seq, DS_HIP_ATTN_MAX_SEQ);
    return NULL;
  }
  ds_hip_attn_t *A = (ds_hip_attn_t *)calloc(1, sizeof *A);
  if (!A) return NULL;
  const size_t H = hidden, qd = (size_t)n_heads * head_dim, hd = head_dim;
  const size_t kv_stride = (qd + 15) & ~(size_t)15; /* rows 64-byte aligned, as the reference's cache */
  size_t off[17], n = 0;
  int k = 0;
#define REGION(b) (off[k++] = n, n += al256(b))
  REGION(qd * H * 2);                       /* 0 wq */
  REGION(qd * H * 2);                       /* 1 wk */
  REGION(qd * H * 2);                       /* 2 wv */
  REGION(H * qd * 2);                       /* 3 wo */
  REGION(H * 4);                            /* 4 input norm */
  REGION(H * 4);                            /* 5 post-attention norm */
  REGION(hd * 4);                           /* 6 q norm */
  REGION(hd * 4);                           /* 7 k norm */
  REGION((size_t)max_seq * hd * 4);         /* 8 cos */
  REGION((size_t)max_seq * hd * 4);         /* 9 sin */
  REGION((size_t)max_seq * kv_stride * 4);  /* 10 K cache */
  REGION((size_t)max_seq * kv_stride * 4);  /* 11 V cache */
  REGION(qd * 4 * 3 + H * 4);               /* 12 scratch: q, k, att, proj */
  REGION((size_t)n_heads * max_seq * 4);    /* 13 scores, then coefficients */
  REGION((size_t)n_heads * (max_seq / 32 + 1) * hd * 4); /* 14 per-chunk V sums */
  REGION((size_t)n_heads * 4);              /* 15 softmax sums */
#undef REGION
  hipError_t e = hipMalloc(&A->arena, n);
  if (e != hipSuccess) {
    dsr_fail("attention arena allocation", e);
    free(A);
    return NULL;
  }
  A->bytes = n;
  char *b = (char *)A->arena;
  float *c = (float *)malloc((size_t)max_seq * hd * 4), *s = (float *)malloc((size_t)max_seq * hd * 4);
  int rc = !c || !s;
  if (!rc) {
    rope_table(c, s, max_seq, head_dim, rope_theta);
    rc = hipMemsetAsync(A->arena, 0, n, dsr_stream) != hipSuccess || dsr_h2d(b + off[0], wq, qd * H * 2) ||
         dsr_h2d(b + off[1], wk, qd * H * 2) || dsr_h2d(b + off[2], wv, qd * H * 2) ||
         dsr_h2d(b + off[3], wo, H * qd * 2) || dsr_h2d(b + off[4], input_norm, H * 4) ||
         dsr_h2d(b + off[5], post_attn_norm, H * 4) || (q_norm && dsr_h2d(b + off[6], q_norm, hd * 4)) ||
         (k_norm && dsr_h2d(b + off[7], k_norm, hd * 4)) || dsr_h2d(b + off[8], c, (size_t)max_seq * hd * 4) ||
         dsr_h2d(b + off[9], s, (size_t)max_seq * hd * 4);
  }
  free(c);
  free(s);
  if (rc) {
    dsr_failf("ds_hip_attn_create: upload failed");
    hipFree(A->arena);
    free(A);
    return NULL;
  }
  dsh_attn_t *d = &A->d;
  d->wq = (const uint16_t *)(b + off[0]);
  d->wk = (const uint16_t *)(b + off[1]);
  d->wv = (const uint16_t *)(b + off[2]);
  d->wo = (const uint16_t *)(b + off[3]);
  d->in_norm = (const float *)(b + off[4]);
  d->post_norm = (const float *)(b + off[5]);
  d->q_norm = q_norm ? (const float *)(b + off[6]) : NULL;
  d->k_norm = k_norm ? (const float *)(b + off[7]) : NULL;
  d->rope_cos = (const float *)(b + off[8]);
  d->rope_sin = (const float *)(b + off[9]);
  d->kc = (float *)(b + off[10]);
  d->vc = (float *)(b + off[11]);
  d->q = (float *)(b + off[12]);
  d->k = d->q + qd;
  d->att = d->k + qd;
  d->proj = d->att + qd;
  d->sc = (float *)(b + off[13]);
  d->part = (float *)(b + off[14]);
  d->se = (float *)(b + off[15]);
  d->H = hidden;
  d->n_heads = n_heads;
  d->head_dim = head_dim;
  d->kv_stride = (int)kv_stride;
  d->max_seq = max_seq;
  d->eps = rms_eps;
  return A;
}

void ds_hip_attn_destroy(ds_hip_attn_t *A) {
  if (!A) return;
  hipStreamSynchronize(dsr_stream);
  hipFree(A->arena);
  free(A);
}

int ds_hip_attn_set_window(ds_hip_attn_t *A, int prefill_len, int sliding_window) {
  if (!A || prefill_len < 0 || sliding_window < 0) return dsr_failf("ds_hip_attn_set_window: invalid arguments");
  A->prefill_len = prefill_len;
  A->window = sliding_window;
  return 0;
}

int ds_hip_attn_kv(const ds_hip_attn_t *A, float **k_cache_dev, float **v_cache_dev, int *kv_stride) {
  if (!A) return dsr_failf("ds_hip_attn_kv: NULL");
  if (k_cache_dev) *k_cache_dev = A->d.kc;
  if (v_cache_dev) *v_cache_dev = A->d.vc;
  if (kv_stride) *kv_stride = A->d.kv_stride;
  return 0;
}

int ds_hip_attn_load_kv(ds_hip_attn_t *A, const float *k_host, const float *v_host, int n_pos, int host_stride) {
  if (!A || !k_host || !v_host || n_pos < 0 || n_pos > A->d.max_seq || host_stride < A->d.n_heads * A->d.head_dim)
    return dsr_failf("ds_hip_attn_load_kv: invalid arguments");
  const size_t row = (size_t)A->d.n_heads * A->d.head_dim * 4;
  DSR_TRY(hipMemcpy2DAsync(A->d.kc, (size_t)A->d.kv_stride * 4, k_host, (size_t)host_stride * 4, row, n_pos,
                           hipMemcpyHostToDevice, dsr_stream),
          "K cache upload");
  DSR_TRY(hipMemcpy2DAsync(A->d.vc, (size_t)A->d.kv_stride * 4, v_host, (size_t)host_stride * 4, row, n_pos,
                           hipMemcpyHostToDevice, dsr_stream),
          "V cache upload");
  DSR_TRY(hipStreamSynchronize(dsr_stream), "KV upload");
  return 0;
}

/* The launch sequence, also used inside captured decode steps; threads: the reference thread count
 * whose split of the QKV rows the kernels follow. */
hipError_t ds_hip_attn_enqueue(const ds_hip_attn_t *A, const float *x_in, const int *step, int stride,
                               int ncopies, float *x_plain, const int *pos_ptr, int pos_add, float *h_out,
                               float *n_out, const float *WrT_next, int E_next, float *partials_next, int threads) {
  return dsh_launch_attn(&A->d, x_in, step, stride, ncopies, x_plain, pos_ptr, pos_add, A->prefill_len, A->window, threads,
                         h_out, n_out, WrT_next, E_next, partials_next, dsr_stream);
}

int ds_hip_attn_hidden(const ds_hip_attn_t *A) { return A ? A->d.H : 0; }

int ds_hip_attn_max_seq(const ds_hip_attn_t *A) { return A ? A->d.max_seq : 0; }

size_t ds_hip_attn_weight_bytes(const ds_hip_attn_t *A) {
  return A ? (size_t)4 * A->d.H * A->d.n_heads * A->d.head_dim * 2 + (size_t)2 * A->d.H * 4 : 0;
}

int ds_hip_attn_forward(ds_hip_attn_t *A, float *h_dev, float *n_dev, const float *x_dev, int pos) {
  if (!A || !h_dev || !n_dev || !x_dev || pos < 0 || pos >= A->d.max_seq)
    return dsr_failf("ds_hip_attn_forward: invalid arguments (pos %d, max_seq %d)", pos, A ? A->d.max_seq : 0);
  DSR_TRY(ds_hip_attn_enqueue(A, x_dev, NULL, 0, 1, NULL, NULL, pos, h_dev, n_dev, NULL, 0, NULL, dsr_threads()),
          "attention kernels");
  return 0;
}
