/*
 * ds_quantize.h — per-row asymmetric INT8 expert weights, MI355X implementation.
 *
 * Drop-in for the reference's ds_quantize.h (vislee/ds-ocr): same type layout, same function
 * names, argument meaning and error behaviour, so ds_moe_decoder.c / ds_ocr.c compile and link
 * unchanged against libds_ocr_hip.so. All compute runs on the GPU (gfx950); host pointers are
 * accepted and results are returned in host memory, synchronously, as the reference does.
 *
 * Format (reference ds_quantize.c:29-47), per output row r:
 *   min = min_c W[r,c], max = max_c W[r,c]
 *   scale[r] = max((max-min)/255, 1e-10), offset[r] = min
 *   u = clamp(roundf((W[r,c]-min) * (1/scale)), 0, 255), stored as int8 q = u - 128
 *   W[r,c] ~= scale[r] * (q + 128) + offset[r]
 * Storage: out_dim*in_dim code bytes + 8 bytes per row.
 *
 * Device residency: the first GPU use of a block uploads its codes/scales/offsets once and keeps
 * them (keyed by the qweight host pointer) until ds_int4_block_free(); a block's host arrays must
 * not be modified after that first use.
 */
#ifndef DS_QUANTIZE_H
#define DS_QUANTIZE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Reference ds_quantize.h:30-37. The name says int4; the format is INT8. */
typedef struct {
  int8_t *qweight; /* [out_dim, in_dim] row-major, stores u - 128 */
  float *scale;    /* [out_dim] */
  float *offset;   /* [out_dim] row minimum */
  int out_dim;
  int in_dim;
  size_t bytes;    /* out_dim*in_dim + 8*out_dim */
} ds_int4_block_t;

/* Reference ds_quantize.h:42-44 / ds_quantize.c:49-81. Quantizes on the GPU; the block's host
 * arrays are malloc'd (free with ds_int4_block_free) and filled with the codes, bit-identical to the
 * reference. Returns 0, or -1 on NULL / non-positive dims / allocation or device failure (the block
 * is then zeroed). */
int ds_int4_quantize_bf16(ds_int4_block_t *block, const uint16_t *W_bf16, int out_dim, int in_dim);

/* Reference ds_quantize.h:47-49 / ds_quantize.c:83-105. */
int ds_int4_quantize_f32(ds_int4_block_t *block, const float *W_f32, int out_dim, int in_dim);

/* Reference ds_quantize.h:52 / ds_quantize.c:107-113. Frees host arrays and the device copy;
 * idempotent; NULL-safe. */
void ds_int4_block_free(ds_int4_block_t *block);

/* Reference ds_quantize.h:55 / ds_quantize.c:115-125. out[out_dim*in_dim] (host). */
void ds_int4_dequantize_f32(float *out, const ds_int4_block_t *block);

/* Reference ds_quantize.h:59-60 / ds_quantize.c:260-274. y[out_dim] = dequant(W) x[in_dim].
 * No-op on NULL arguments or out_dim <= 0. */
void ds_int4_matvec(float *y, const float *x, const ds_int4_block_t *block);

/* Reference ds_quantize.h:63-65 / ds_quantize.c:276-292. y[nrows] = rows [row_start,
 * row_start+nrows) of dequant(W) x. No-op on NULL, nrows <= 0, or a range outside the block. */
void ds_int4_matvec_rows(float *y, const float *x, const ds_int4_block_t *block, int row_start, int nrows);

/* Reference ds_quantize.h:69-75 / ds_quantize.c:301-321: out[hidden] = down(SwiGLU(gate, up)) with
 * gate/up = rows [0,inter) / [inter,2*inter) of gate_up x; honours ds_bf16_simulate_python. The
 * four scratch buffers are accepted for signature compatibility; their contents afterwards are
 * unspecified (the reference leaves intermediates there). */
void ds_expert_forward_fused_int4(float *out, const float *x, const ds_int4_block_t *gate_up_int4,
                                  const ds_int4_block_t *down_int4, int hidden, int intermediate,
                                  float *gate_up_buf, float *gate_buf, float *up_buf, float *hidden_buf);

/* Reference ds_quantize.h:78-79 / ds_quantize.c:127-144. Relative RMS error; -1 on error. */
float ds_int4_quant_error_rms(const ds_int4_block_t *block, const uint16_t *W_bf16);

#ifdef __cplusplus
}
#endif

#endif /* DS_QUANTIZE_H */
