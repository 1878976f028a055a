/* ds_quantize_api.c — ds_quantize.h on the GPU: same semantics and error conventions as the
 * reference ds_quantize.c (cited per function); compute is done by the gfx950 kernels. */
#include <stdlib.h>
#include <string.h>

#include "dsr.h"
#include "ds_kernels.h"
#include "ds_quantize.h"

/* ds_quantize.c:107-113. */
void ds_int4_block_free(ds_int4_block_t *block) {
  if (!block) return;
  dsr_block_forget(block->qweight);
  free(block->qweight);
  block->qweight = NULL;
  free(block->scale);
  block->scale = NULL;
  free(block->offset);
  block->offset = NULL;
  block->bytes = 0;
}

static int alloc_host(ds_int4_block_t *b, int out_dim, int in_dim) {
  memset(b, 0, sizeof *b);
  b->out_dim = out_dim;
  b->in_dim = in_dim;
  b->qweight = (int8_t *)malloc((size_t)out_dim * in_dim);
  b->scale = (float *)malloc((size_t)out_dim * sizeof(float));
  b->offset = (float *)malloc((size_t)out_dim * sizeof(float));
  if (!b->qweight || !b->scale || !b->offset) {
    ds_int4_block_free(b);
    return -1;
  }
  return 0;
}

/* Uploads W (elem bytes per value), quantizes on the device into the block's registered device
 * arrays and copies the codes/scales/offsets to the host arrays. */
static int quantize_common(ds_int4_block_t *b, const void *W, size_t elem) {
  size_t n = (size_t)b->out_dim * b->in_dim;
  dsr_dblock_t db;
  if (dsr_init() || dsr_block_new(b, &db)) return -1;
  void *Wd = dsr_scratch(DSR_SLOT_A, n * elem);
  if (!Wd || dsr_h2d(Wd, W, n * elem)) return -1;
  hipError_t e = elem == 2
                     ? dsh_launch_quantize_bf16((const uint16_t *)Wd, db.q, db.scale, db.offset, b->out_dim, b->in_dim,
                                                dsr_stream)
                     : dsh_launch_quantize_f32((const float *)Wd, db.q, db.scale, db.offset, b->out_dim, b->in_dim,
                                               dsr_stream);
  if (e != hipSuccess) return dsr_fail("quantize kernel", e);
  if (dsr_d2h(b->qweight, db.q, n) || dsr_d2h(b->scale, db.scale, (size_t)b->out_dim * 4) ||
      dsr_d2h(b->offset, db.offset, (size_t)b->out_dim * 4))
    return -1;
  b->bytes = n + (size_t)b->out_dim * sizeof(float) * 2;
  return dsr_block_adopt(b, db.q, db.scale, db.offset);
}

/* ds_quantize.c:49-81. */
int ds_int4_quantize_bf16(ds_int4_block_t *block, const uint16_t *W_bf16, int out_dim, int in_dim) {
  if (!block || !W_bf16 || out_dim <= 0 || in_dim <= 0) return -1;
  if (alloc_host(block, out_dim, in_dim)) return -1;
  if (quantize_common(block, W_bf16, 2)) {
    ds_int4_block_free(block);
    return -1;
  }
  return 0;
}

/* ds_quantize.c:83-105. */
int ds_int4_quantize_f32(ds_int4_block_t *block, const float *W_f32, int out_dim, int in_dim) {
  if (!block || !W_f32 || out_dim <= 0 || in_dim <= 0) return -1;
  if (alloc_host(block, out_dim, in_dim)) return -1;
  if (quantize_common(block, W_f32, 4)) {
    ds_int4_block_free(block);
    return -1;
  }
  return 0;
}

/* ds_quantize.c:115-125. */
void ds_int4_dequantize_f32(float *out, const ds_int4_block_t *block) {
  if (!out || !block || !block->qweight) return;
  dsr_dblock_t db;
  if (dsr_block_device(block, &db)) return;
  size_t n = (size_t)block->out_dim * block->in_dim;
  float *od = (float *)dsr_scratch(DSR_SLOT_A, n * 4);
  if (!od) return;
  hipError_t e = dsh_launch_dequantize(db.q, db.scale, db.offset, od, block->out_dim, block->in_dim, dsr_stream);
  if (e != hipSuccess) {
    dsr_fail("dequantize kernel", e);
    return;
  }
  dsr_d2h(out, od, n * 4);
}

/* ds_quantize.c:127-144: sqrt(Σ(w-deq)^2 / Σw^2) with double sums; -1 on error. */
float ds_int4_quant_error_rms(const ds_int4_block_t *block, const uint16_t *W_bf16) {
  if (!block || !W_bf16 || !block->qweight) return -1.0f;
  dsr_dblock_t db;
  if (dsr_block_device(block, &db)) return -1.0f;
  size_t n = (size_t)block->out_dim * block->in_dim;
  uint16_t *Wd = (uint16_t *)dsr_scratch(DSR_SLOT_A, n * 2);
  double *sums = (double *)dsr_scratch(DSR_SLOT_B, 2 * sizeof(double) * 1024);
  if (!Wd || !sums || dsr_h2d(Wd, W_bf16, n * 2)) return -1.0f;
  hipError_t e = dsh_launch_quant_rms(db.q, db.scale, db.offset, Wd, block->out_dim, block->in_dim, sums, dsr_stream);
  if (e != hipSuccess) {
    dsr_fail("rms kernel", e);
    return -1.0f;
  }
  double h[2];
  if (dsr_d2h(h, sums, sizeof h)) return -1.0f;
  return h[1] > 0 ? sqrtf((float)(h[0] / h[1])) : 0.0f;
}

/* The matvec of the per-function API: the reference's own per-row order (bit-identical results);
 * rows longer than the exact kernel stages in LDS use the lane-parallel kernel (f32 rounding). */
static hipError_t int8_mv(const dsr_dblock_t *db, const float *xd, float *yd, int in_dim, int row_start, int nrows) {
  if ((size_t)in_dim * 4 <= 64 * 1024)
    return dsh_launch_int8_matvec_exact(db->q, db->scale, db->offset, xd, yd, in_dim, row_start, nrows, dsr_stream);
  return dsh_launch_int8_matvec(db->q, db->scale, db->offset, xd, yd, in_dim, row_start, nrows, dsr_stream);
}

static int matvec_dev(float *y, const float *x, const ds_int4_block_t *block, int row_start, int nrows) {
  dsr_dblock_t db;
  if (dsr_block_device(block, &db)) return -1;
  const float *xp = (const float *)dsr_pin_in(DSR_PIN_X, x, (size_t)block->in_dim * 4);
  float *yp = (float *)dsr_pin_buf(DSR_PIN_Y, (size_t)nrows * 4);
  if (!xp || !yp) return -1;
  hipError_t e = int8_mv(&db, xp, yp, block->in_dim, row_start, nrows);
  if (e != hipSuccess) return dsr_fail("int8 matvec kernel", e);
  return dsr_pin_out(y, DSR_PIN_Y, (size_t)nrows * 4);
}

/* ds_quantize.c:260-274. */
void ds_int4_matvec(float *y, const float *x, const ds_int4_block_t *block) {
  if (!y || !x || !block || block->out_dim <= 0) return;
  matvec_dev(y, x, block, 0, block->out_dim);
}

/* ds_quantize.c:276-292. The reference does not check the range; here a range outside the block
 * is reported and ignored. */
void ds_int4_matvec_rows(float *y, const float *x, const ds_int4_block_t *block, int row_start, int nrows) {
  if (!y || !x || !block || nrows <= 0) return;
  if (row_start < 0 || row_start + nrows > block->out_dim) {
    dsr_failf("ds_int4_matvec_rows: rows [%d, %d) outside [0, %d)", row_start, row_start + nrows, block->out_dim);
    return;
  }
  matvec_dev(y, x, block, row_start, nrows);
}

/* ds_quantize.c:301-321: gate_up matvec -> split -> [bf16] -> SwiGLU -> [bf16] -> down -> [bf16];
 * every step in the reference's order, so the output is bit-identical in both modes. */
int ds_hip_time_expert(const ds_int4_block_t *gate_up_int4, const ds_int4_block_t *down_int4, int hidden,
                       int intermediate, const float *x, int n, float *ms) {
  if (dsr_init()) return -1;
  if (!gate_up_int4 || !down_int4 || !x || n <= 0 || !ms) return dsr_failf("ds_hip_time_expert: invalid arguments");
  if (gate_up_int4->out_dim != 2 * intermediate || down_int4->in_dim != intermediate ||
      down_int4->out_dim != hidden || gate_up_int4->in_dim != hidden)
    return dsr_failf("ds_hip_time_expert: block shapes do not match hidden=%d intermediate=%d", hidden, intermediate);
  if (!dsh_expert_exact_blocks(hidden, intermediate))
    return dsr_failf("ds_hip_time_expert: hidden=%d intermediate=%d has no one-launch expert kernel", hidden,
                     intermediate);
  dsr_dblock_t g, d;
  if (dsr_block_device(gate_up_int4, &g) || dsr_block_device(down_int4, &d)) return -1;
  const size_t xb = (size_t)hidden * 4;
  const int nd = dsh_expert_exact_down_blocks(hidden);
  unsigned long long *hb = (unsigned long long *)dsr_expert_hbuf((size_t)intermediate);
  if (!hb) return -1;
  float *xd = NULL, *yd = NULL;
  unsigned *done = NULL;
  hipEvent_t a = NULL, b = NULL;
  int rc = 0;
  if (hipMalloc((void **)&xd, xb) != hipSuccess || hipMalloc((void **)&yd, xb) != hipSuccess ||
      hipMalloc((void **)&done, sizeof(unsigned) * (size_t)nd) != hipSuccess || hipEventCreate(&a) != hipSuccess ||
      hipEventCreate(&b) != hipSuccess)
    rc = dsr_failf("ds_hip_time_expert: allocation failed");
  if (rc == 0 && dsr_h2d(xd, x, xb)) rc = -1;
  for (int i = -1; i < n && rc == 0; i++) { /* i = -1: warm-up launch */
    if (i == 0 && hipEventRecord(a, dsr_stream) != hipSuccess) rc = -1;
    const hipError_t e = dsh_launch_expert_exact(g.q, g.scale, g.offset, d.q, d.scale, d.offset, xd, NULL, hb, yd,
                                                 done, hidden, intermediate, dsr_expert_epoch(),
                                                 ds_bf16_simulate_python, 1 << 22, dsr_derr_dev(DSR_DERR_EXPERT_WAIT),
                                                 dsr_stream);
    if (e != hipSuccess) rc = dsr_fail("expert kernel", e);
  }
  if (rc == 0 && (hipEventRecord(b, dsr_stream) != hipSuccess || hipEventSynchronize(b) != hipSuccess ||
                  hipEventElapsedTime(ms, a, b) != hipSuccess))
    rc = dsr_failf("ds_hip_time_expert: timing failed");
  if (rc == 0) *ms /= (float)n;
  (void)hipStreamSynchronize(dsr_stream);
  if (a) hipEventDestroy(a);
  if (b) hipEventDestroy(b);
  hipFree(xd);
  hipFree(yd);
  hipFree(done);
  return rc == 0 ? dsr_derr_check() : rc;
}

void ds_expert_forward_fused_int4(float *out, const float *x, const ds_int4_block_t *gate_up_int4,
                                  const ds_int4_block_t *down_int4, int hidden, int intermediate, float *gate_up_buf,
                                  float *gate_buf, float *up_buf, float *hidden_buf) {
  (void)gate_up_buf;
  (void)gate_buf;
  (void)up_buf;
  (void)hidden_buf;
  if (!out || !x || !gate_up_int4 || !down_int4) return;
  if (gate_up_int4->out_dim != 2 * intermediate || down_int4->in_dim != intermediate ||
      down_int4->out_dim != hidden || gate_up_int4->in_dim != hidden) {
    dsr_failf("ds_expert_forward_fused_int4: block shapes do not match hidden=%d intermediate=%d", hidden,
              intermediate);
    return;
  }
  dsr_dblock_t g, d;
  if (dsr_block_device(gate_up_int4, &g) || dsr_block_device(down_int4, &d)) return;
  int bf16sim = ds_bf16_simulate_python;
  if (dsh_expert_exact_blocks(hidden, intermediate)) {
    /* one launch (gate_up, SwiGLU, down) writing out to pinned staging; x from pinned staging, or from
     * the device copy the previous call left when x is the same input (the routed experts and the
     * shared expert of a layer share it) */
    const size_t xb = (size_t)hidden * 4;
    float *xc = (float *)dsr_scratch(DSR_SLOT_XC, xb);
    unsigned long long *hb = (unsigned long long *)dsr_expert_hbuf((size_t)intermediate);
    float *op = (float *)dsr_pin_buf(DSR_PIN_Y, xb);
    if (!xc || !hb || !op) return;
    const float *xsrc = xc;
    float *xcache = NULL;
    if (!dsr_input_cached(x, xb)) {
      xsrc = (const float *)dsr_pin_in(DSR_PIN_X, x, xb);
      xcache = xc;
      if (!xsrc) return;
    }
    const int nd = dsh_expert_exact_down_blocks(hidden);
    unsigned *done = (unsigned *)dsr_pin_buf(DSR_PIN_DONE, sizeof(unsigned) * (size_t)nd);
    if (!done) return;
    const unsigned epoch = dsr_expert_epoch();
    hipError_t e = dsh_launch_expert_exact(g.q, g.scale, g.offset, d.q, d.scale, d.offset, xsrc, xcache, hb, op, done,
                                           hidden, intermediate, epoch, bf16sim, 1 << 22,
                                           dsr_derr_dev(DSR_DERR_EXPERT_WAIT), dsr_stream);
    if (e != hipSuccess) {
      dsr_input_forget();
      dsr_fail("expert kernel", e);
      return;
    }
    if (dsr_pin_out_done(out, DSR_PIN_Y, xb, nd, epoch) || dsr_derr_check()) dsr_input_forget();
    return;
  }
  float *gu = (float *)dsr_scratch(DSR_SLOT_A, (size_t)2 * intermediate * 4);
  if (!gu) return;
  float *xd = (float *)dsr_scratch(DSR_SLOT_X, (size_t)hidden * 4);
  float *hd = (float *)dsr_scratch(DSR_SLOT_B, (size_t)intermediate * 4);
  float *od = (float *)dsr_scratch(DSR_SLOT_Y, (size_t)hidden * 4);
  if (!xd || !hd || !od || dsr_h2d(xd, x, (size_t)hidden * 4)) return;
  hipError_t e = int8_mv(&g, xd, gu, hidden, 0, 2 * intermediate);
  if (e == hipSuccess) e = dsh_launch_split_swiglu(hd, gu, intermediate, bf16sim, dsr_stream);
  if (e == hipSuccess) e = int8_mv(&d, hd, od, intermediate, 0, hidden);
  if (e == hipSuccess && bf16sim) e = dsh_launch_bf16_trunc(od, (size_t)hidden, dsr_stream);
  if (e != hipSuccess) {
    dsr_fail("expert kernels", e);
    return;
  }
  dsr_d2h(out, od, (size_t)hidden * 4);
}
