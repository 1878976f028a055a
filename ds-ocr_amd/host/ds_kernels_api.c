/* ds_kernels_api.c — the MoE-decode subset of ds_kernels.h on the GPU. Each function keeps the
 * reference's argument meaning and no-op/error behaviour (cited per function). */
#include <stdlib.h>
#include <string.h>

#include "dsr.h"
#include "ds_kernels.h"

#define F4(n) ((size_t)(n) * sizeof(float))

/* ds_kernels.c:917-927. seq_len == 1 -> AVX-512-order matvec (reference ds_bf16_matvec_threaded);
 * seq_len > 1 -> f32 GEMM on widened weights (reference: f32 view + sgemm). */
void ds_linear_nobias_bf16(float *y, const float *x, const uint16_t *W_bf16, int seq_len, int in_dim, int out_dim) {
  if (!y || !x || !W_bf16 || seq_len <= 0 || in_dim <= 0 || out_dim <= 0) return;
  const uint16_t *Wd = (const uint16_t *)dsr_weight_device(W_bf16, (size_t)out_dim * in_dim * 2);
  if (!Wd) return;
  if (seq_len == 1) { /* the input and scores through pinned staging the kernel reads and writes */
    const float *xp = (const float *)dsr_pin_in(DSR_PIN_X, x, F4(in_dim));
    float *yp = (float *)dsr_pin_buf(DSR_PIN_Y, F4(out_dim));
    const int nb = dsh_bf16_matvec_avx_blocks(out_dim);
    unsigned *done = (unsigned *)dsr_pin_buf(DSR_PIN_DONE, sizeof(unsigned) * (size_t)nb);
    if (!xp || !yp || !done) return;
    const unsigned epoch = dsr_expert_epoch();
    hipError_t e = dsh_launch_bf16_matvec_avx_done(Wd, xp, NULL, yp, in_dim, out_dim, dsr_threads(), done, epoch,
                                                   dsr_stream);
    if (e != hipSuccess) {
      dsr_fail("ds_linear_nobias_bf16", e);
      return;
    }
    dsr_pin_out_done(y, DSR_PIN_Y, F4(out_dim), nb, epoch);
    return;
  }
  float *xd = (float *)dsr_scratch(DSR_SLOT_X, F4((size_t)seq_len * in_dim));
  float *yd = (float *)dsr_scratch(DSR_SLOT_Y, F4((size_t)seq_len * out_dim));
  if (!xd || !yd || dsr_h2d(xd, x, F4((size_t)seq_len * in_dim))) return;
  hipError_t e = dsh_launch_gemm_bf16w(xd, Wd, yd, seq_len, in_dim, out_dim, dsr_stream);
  if (e != hipSuccess) {
    dsr_fail("ds_linear_nobias_bf16", e);
    return;
  }
  dsr_d2h(y, yd, F4((size_t)seq_len * out_dim));
}

/* ds_kernels.c:942-945 (ds_bf16_matvec_threaded with an optional bias). */
void ds_bf16_matvec_pub(float *y, const float *x, const uint16_t *W_bf16, const float *b, int in_dim, int out_dim) {
  if (!y || !x || !W_bf16 || in_dim <= 0 || out_dim <= 0) return;
  const uint16_t *Wd = (const uint16_t *)dsr_weight_device(W_bf16, (size_t)out_dim * in_dim * 2);
  if (!Wd) return;
  float *xd = (float *)dsr_scratch(DSR_SLOT_X, F4(in_dim));
  float *yd = (float *)dsr_scratch(DSR_SLOT_Y, F4(out_dim));
  float *bd = b ? (float *)dsr_scratch(DSR_SLOT_A, F4(out_dim)) : NULL;
  if (!xd || !yd || (b && !bd) || dsr_h2d(xd, x, F4(in_dim)) || (b && dsr_h2d(bd, b, F4(out_dim)))) return;
  hipError_t e = dsh_launch_bf16_matvec_avx(Wd, xd, bd, yd, in_dim, out_dim, dsr_threads(), dsr_stream);
  if (e != hipSuccess) {
    dsr_fail("ds_bf16_matvec_pub", e);
    return;
  }
  dsr_d2h(y, yd, F4(out_dim));
}

/* ds_kernels.c:1621-1642. */
void ds_vec_add(float *dst, const float *a, const float *b, int n) {
  if (!dst || !a || !b || n <= 0) return;
  const float *ap = (const float *)dsr_pin_in(DSR_PIN_A, a, F4(n));
  const float *bp = (const float *)dsr_pin_in(DSR_PIN_B, b, F4(n));
  float *yp = (float *)dsr_pin_buf(DSR_PIN_Y, F4(n));
  const int nb = dsh_vec_add_blocks(n);
  unsigned *done = (unsigned *)dsr_pin_buf(DSR_PIN_DONE, sizeof(unsigned) * (size_t)nb);
  if (!ap || !bp || !yp || !done) return;
  const unsigned epoch = dsr_expert_epoch();
  hipError_t e = dsh_launch_vec_add_done(yp, ap, bp, n, done, epoch, dsr_stream);
  if (e != hipSuccess) {
    dsr_fail("ds_vec_add", e);
    return;
  }
  dsr_pin_out_done(dst, DSR_PIN_Y, F4(n), nb, epoch);
}

/* ds_kernels.c:1739-1789 (fast-exp branch): out[s*inter + j] = silu(g) * u. */
void ds_swiglu_direct(float *out, const float *gate_buf, const float *up_buf, int seq_len, int intermediate) {
  if (!out || !gate_buf || !up_buf || seq_len <= 0 || intermediate <= 0) return;
  size_t n = (size_t)seq_len * intermediate;
  float *gd = (float *)dsr_scratch(DSR_SLOT_A, F4(n)), *ud = (float *)dsr_scratch(DSR_SLOT_B, F4(n));
  if (!gd || !ud || dsr_h2d(gd, gate_buf, F4(n)) || dsr_h2d(ud, up_buf, F4(n))) return;
  hipError_t e = dsh_launch_swiglu(gd, gd, ud, n, dsr_stream);
  if (e != hipSuccess) {
    dsr_fail("ds_swiglu_direct", e);
    return;
  }
  dsr_d2h(out, gd, F4(n));
}

/* ds_kernels.c:2464-2492. */
void ds_bf16_truncate_array(float *data, int n) {
  if (!data || n <= 0) return;
  float *d = (float *)dsr_scratch(DSR_SLOT_A, F4(n));
  if (!d || dsr_h2d(d, data, F4(n))) return;
  hipError_t e = dsh_launch_bf16_trunc(d, (size_t)n, dsr_stream);
  if (e != hipSuccess) {
    dsr_fail("ds_bf16_truncate_array", e);
    return;
  }
  dsr_d2h(data, d, F4(n));
}

/* ds_kernels.c:181-185 -> ds_linear (no-BLAS order). */
void ds_moe_router(float *scores, const float *x, const float *gate_weight, int hidden, int n_experts) {
  if (!scores || !x || !gate_weight || hidden <= 0 || n_experts <= 0) return;
  const float *Wd = (const float *)dsr_weight_device(gate_weight, F4((size_t)n_experts * hidden));
  float *xd = (float *)dsr_scratch(DSR_SLOT_X, F4(hidden)), *yd = (float *)dsr_scratch(DSR_SLOT_Y, F4(n_experts));
  if (!Wd || !xd || !yd || dsr_h2d(xd, x, F4(hidden))) return;
  hipError_t e = dsh_launch_linear_f32_exact(Wd, xd, yd, hidden, n_experts, dsr_stream);
  if (e != hipSuccess) {
    dsr_fail("ds_moe_router", e);
    return;
  }
  dsr_d2h(scores, yd, F4(n_experts));
}

/* ds_kernels.c:187-191. */
void ds_moe_router_bf16(float *scores, const float *x, const uint16_t *gate_weight_bf16, int hidden, int n_experts) {
  ds_linear_nobias_bf16(scores, x, gate_weight_bf16, 1, hidden, n_experts);
}

/* ds_kernels.c:193-243. */
void ds_moe_top_k(int *top_indices, float *top_weights, const float *scores, int n_experts, int top_k) {
  if (!top_indices || !top_weights || !scores || top_k <= 0) return;
  if (n_experts <= 0 || n_experts > DS_MAX_EXPERTS || top_k > n_experts) {
    dsr_failf("ds_moe_top_k: n_experts=%d top_k=%d outside 1..%d", n_experts, top_k, DS_MAX_EXPERTS);
    return;
  }
  float *sd = (float *)dsr_scratch(DSR_SLOT_A, F4(n_experts));
  int *id = (int *)dsr_scratch(DSR_SLOT_IDX, sizeof(int) * (size_t)top_k);
  float *wd = (float *)dsr_scratch(DSR_SLOT_B, F4(top_k));
  if (!sd || !id || !wd || dsr_h2d(sd, scores, F4(n_experts))) return;
  hipError_t e = dsh_launch_topk(sd, n_experts, top_k, DSH_ROUTE_CFG, id, wd, dsr_stream);
  if (e != hipSuccess) {
    dsr_fail("ds_moe_top_k", e);
    return;
  }
  if (dsr_d2h(top_indices, id, sizeof(int) * (size_t)top_k)) return;
  dsr_d2h(top_weights, wd, F4(top_k));
}

/* ds_kernels.c:359-371. top_indices is unused by the reference too. */
void ds_expert_combine(float *output, const float *expert_outputs, const int *top_indices, const float *top_weights,
                       int top_k, int hidden) {
  (void)top_indices;
  if (!output || !expert_outputs || !top_weights || top_k <= 0 || hidden <= 0) return;
  const float *eo = (const float *)dsr_pin_in(DSR_PIN_A, expert_outputs, F4((size_t)top_k * hidden));
  const float *wd = (const float *)dsr_pin_in(DSR_PIN_B, top_weights, F4(top_k));
  float *od = (float *)dsr_pin_buf(DSR_PIN_Y, F4(hidden));
  const int nb = dsh_expert_combine_blocks(hidden);
  unsigned *done = (unsigned *)dsr_pin_buf(DSR_PIN_DONE, sizeof(unsigned) * (size_t)nb);
  if (!eo || !wd || !od || !done) return;
  const unsigned epoch = dsr_expert_epoch();
  hipError_t e = dsh_launch_expert_combine_done(od, eo, wd, top_k, hidden, done, epoch, dsr_stream);
  if (e != hipSuccess) {
    dsr_fail("ds_expert_combine", e);
    return;
  }
  dsr_pin_out_done(output, DSR_PIN_Y, F4(hidden), nb, epoch);
}

/* ds_kernels.c:322-357: BF16 fused expert; both matvecs in the AVX-512 order. */
void ds_expert_forward_fused(float *out, const float *x, const uint16_t *gate_up_fused_bf16, const uint16_t *down_bf16,
                             int hidden, int intermediate, float *gate_up_buf, float *gate_buf, float *up_buf,
                             float *hidden_buf) {
  (void)gate_up_buf;
  (void)gate_buf;
  (void)up_buf;
  (void)hidden_buf;
  if (!out || !x || !gate_up_fused_bf16 || !down_bf16 || hidden <= 0 || intermediate <= 0) return;
  const uint16_t *gu = (const uint16_t *)dsr_weight_device(gate_up_fused_bf16, (size_t)2 * intermediate * hidden * 2);
  const uint16_t *dn = (const uint16_t *)dsr_weight_device(down_bf16, (size_t)hidden * intermediate * 2);
  float *xd = (float *)dsr_scratch(DSR_SLOT_X, F4(hidden));
  float *gd = (float *)dsr_scratch(DSR_SLOT_A, F4(2 * (size_t)intermediate));
  float *hd = (float *)dsr_scratch(DSR_SLOT_B, F4(intermediate));
  float *od = (float *)dsr_scratch(DSR_SLOT_Y, F4(hidden));
  if (!gu || !dn || !xd || !gd || !hd || !od || dsr_h2d(xd, x, F4(hidden))) return;
  int bf16sim = ds_bf16_simulate_python, T = dsr_threads();
  hipError_t e = dsh_launch_bf16_matvec_avx(gu, xd, NULL, gd, hidden, 2 * intermediate, T, dsr_stream);
  if (e == hipSuccess) e = dsh_launch_split_swiglu(hd, gd, intermediate, bf16sim, dsr_stream);
  if (e == hipSuccess) e = dsh_launch_bf16_matvec_avx(dn, hd, NULL, od, intermediate, hidden, T, dsr_stream);
  if (e == hipSuccess && bf16sim) e = dsh_launch_bf16_trunc(od, (size_t)hidden, dsr_stream);
  if (e != hipSuccess) {
    dsr_fail("ds_expert_forward_fused", e);
    return;
  }
  dsr_d2h(out, od, F4(hidden));
}

/* ds_kernels.c:981-1011 (non-NEON branch). The row is staged from the caller's array at every call
 * (2 bytes per column): a registered head is keyed by address, and a row read from it could belong
 * to an older array at the same address. */
float ds_bf16_dot_row(const float *x, const uint16_t *W_bf16, int in_dim, int tok_id) {
  if (!x || !W_bf16 || in_dim <= 0 || tok_id < 0) return 0.0f;
  if (dsr_init()) return 0.0f;
  const size_t row_bytes = (size_t)in_dim * 2;
  const uint16_t *Wd = (const uint16_t *)dsr_scratch(DSR_SLOT_D, row_bytes);
  float *xd = (float *)dsr_scratch(DSR_SLOT_X, F4(in_dim)), *od = (float *)dsr_scratch(DSR_SLOT_Y, F4(1));
  if (!Wd || !xd || !od || dsr_h2d(xd, x, F4(in_dim))) return 0.0f;
  if (dsr_h2d((void *)Wd, W_bf16 + (size_t)tok_id * in_dim, row_bytes)) return 0.0f;
  hipError_t e = dsh_launch_bf16_dot_row(Wd, xd, in_dim, 0, od, dsr_stream);
  if (e != hipSuccess) {
    dsr_fail("ds_bf16_dot_row", e);
    return 0.0f;
  }
  float v = 0.0f;
  dsr_d2h(&v, od, sizeof v);
  return v;
}

/* ds_kernels.c:1013-1016. */
int ds_argmax_matvec_bf16(const float *x, const uint16_t *W_bf16, int in_dim, int out_dim) {
  return ds_argmax_matvec_bf16_excluding(x, W_bf16, in_dim, out_dim, NULL, 0);
}

/* ds_kernels.c:1020-1099. The argmax itself, and the exclusion fallbacks of both the single-thread
 * branch (rescan in 8192-row chunks, a chunk whose best is excluded is skipped) and the threaded
 * branch (best non-excluded per-thread winner; the excluded best if none) run on the device.
 * The reference's CPU path always returns an index its caller may use as a row
 * (ds_moe_decoder.c:1041-1043 reads that row at once); on a device error (reported on stderr and in
 * ds_hip_last_error) or invalid arguments this returns 0, never an index outside [0, out_dim). */
static int argmax_excluding(const float *x, const uint16_t *W_bf16, int in_dim, int out_dim, const int *exclude_ids,
                            int n_exclude);

int ds_argmax_matvec_bf16_excluding(const float *x, const uint16_t *W_bf16, int in_dim, int out_dim,
                                    const int *exclude_ids, int n_exclude) {
  int idx = argmax_excluding(x, W_bf16, in_dim, out_dim, exclude_ids, n_exclude);
  return idx >= 0 && idx < out_dim ? idx : 0;
}

int ds_hip_argmax_int8_copy(const uint16_t *W_bf16) { return W_bf16 && dsr_weight_aux(W_bf16) ? 1 : 0; }

static int argmax_excluding(const float *x, const uint16_t *W_bf16, int in_dim, int out_dim, const int *exclude_ids,
                            int n_exclude) {
  if (!x || !W_bf16 || in_dim <= 0 || out_dim <= 0) return dsr_failf("ds_argmax_matvec_bf16: invalid arguments");
  if (n_exclude < 0 || (n_exclude > 0 && !exclude_ids)) n_exclude = 0;
  const uint16_t *Wd = (const uint16_t *)dsr_weight_device(W_bf16, (size_t)out_dim * in_dim * 2);
  float *xd = (float *)dsr_scratch(DSR_SLOT_X, F4(in_dim));
  int nb = dsh_argmax_avx_blocks(out_dim);
  unsigned long long *cand = (unsigned long long *)dsr_scratch(DSR_SLOT_C, sizeof(unsigned long long) * (size_t)nb);
  int *res = (int *)dsr_scratch(DSR_SLOT_IDX, sizeof(int) * 4);
  float *lg = n_exclude ? (float *)dsr_scratch(DSR_SLOT_A, F4(out_dim)) : NULL;
  float *lg2 = n_exclude ? (float *)dsr_scratch(DSR_SLOT_B, F4(out_dim)) : NULL;
  int *exd = n_exclude ? (int *)dsr_scratch(DSR_SLOT_D, sizeof(int) * (size_t)n_exclude) : NULL;
  if (!Wd || !xd || !cand || !res || (n_exclude && (!lg || !lg2 || !exd)) || dsr_h2d(xd, x, F4(in_dim))) return -1;
  int T = dsr_threads();
  hipError_t e;
  if (!n_exclude && dsh_dec_lm_eligible(Wd, in_dim, out_dim, T) && dsh_lm_q8_supported(in_dim, out_dim) &&
      dsh_lm_q8_blocks(out_dim) <= nb) {
    /* every row in the reference's 4-row-group order: the argmax over the head's int8 copy with
     * exact bounds (k_lm.hip; the same index), the copy built at the first call and kept with the
     * registered weights */
    dsh_lm_q8_t Q;
    void *aux = dsr_weight_aux(W_bf16);
    if (!aux) {
      if (hipMalloc(&aux, dsh_lm_q8_bytes(in_dim, out_dim)) != hipSuccess) {
        (void)hipGetLastError();
        aux = NULL;
      } else {
        dsh_lm_q8_carve(aux, in_dim, out_dim, &Q);
        if (dsh_launch_lm_q8_build(Wd, &Q, dsr_stream) != hipSuccess || dsr_weight_set_aux(W_bf16, aux)) {
          hipFree(aux);
          aux = NULL;
        }
      }
    }
    if (aux) {
      dsh_lm_q8_carve(aux, in_dim, out_dim, &Q);
      e = dsh_launch_lm_q8(Wd, &Q, xd, 0, NULL, cand, NULL, dsr_stream);
      if (e == hipSuccess)
        e = dsh_launch_lm_argmax_final(cand, dsh_lm_q8_blocks(out_dim), res, NULL, NULL, 0, NULL, 0, in_dim, NULL,
                                       dsr_stream);
    } else {
      e = dsh_launch_argmax_avx(Wd, xd, cand, NULL, in_dim, out_dim, T, res, NULL, dsr_stream);
    }
  } else if (!n_exclude) {
    e = dsh_launch_argmax_avx(Wd, xd, cand, NULL, in_dim, out_dim, T, res, NULL, dsr_stream);
  } else {
    if (dsr_h2d(exd, exclude_ids, sizeof(int) * (size_t)n_exclude)) return -1;
    e = dsh_launch_argmax_excluding(Wd, xd, cand, lg, lg2, in_dim, out_dim, T, exd, n_exclude, res, dsr_stream);
  }
  if (e != hipSuccess) {
    dsr_fail("ds_argmax_matvec_bf16", e);
    return -1;
  }
  int idx = -1;
  if (dsr_d2h(&idx, res, sizeof idx)) return -1;
  return idx;
}
