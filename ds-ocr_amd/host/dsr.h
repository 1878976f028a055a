/* dsr.h — internal host runtime of libds_ocr_hip (C): device, stream, errors, staging, registry. */
#ifndef DSR_H
#define DSR_H

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

#include "../csrc/k_core.h"
#include "ds_quantize.h"

extern hipStream_t dsr_stream;

/* Initialises device 0 and the library stream once. Returns 0, or -1 (message printed). */
int dsr_init(void);
/* 1 once dsr_init has succeeded (no side effects). */
int dsr_ready(void);
/* Records and prints a failure; returns -1. */
int dsr_fail(const char *what, hipError_t e);
int dsr_failf(const char *fmt, ...);
#define DSR_TRY(call, what)                          \
  do {                                               \
    hipError_t dsr_e_ = (call);                      \
    if (dsr_e_ != hipSuccess) return dsr_fail((what), dsr_e_); \
  } while (0)

/* Errors that kernels report from the device: a word of mapped, coherent host memory per kind, which
 * a kernel sets (a system-scope store) when one of its bounded waits gives up, and the host reads
 * without a copy. dsr_derr_dev(kind) is the device address to pass to the kernel (NULL before
 * dsr_init). dsr_derr_check() reports (and clears) any word that is set: -1 with ds_hip_last_error
 * naming the failure, else 0. It runs after every synchronisation the library API offers
 * (ds_hip_sync) and at the entry of the calls whose results such a failure voids. */
enum { DSR_DERR_PREFILL_WAIT, DSR_DERR_ROUTE_WAIT, DSR_DERR_EXPERT_WAIT, DSR_DERR_N };
int *dsr_derr_dev(int kind);
int dsr_derr_check(void);

/* The certified CFG routing's counters and optional log (ds_hip_route_stats, ds_hip_set_route_log)
 * for a launch: tag identifies the layer in the log entries. */
dsh_rcert_t dsr_rcert(int tag);

/* Grow-only device staging buffer per slot (not thread-safe, like the reference API). */
enum { DSR_SLOT_X, DSR_SLOT_Y, DSR_SLOT_A, DSR_SLOT_B, DSR_SLOT_C, DSR_SLOT_D, DSR_SLOT_IDX, DSR_SLOT_PF, DSR_SLOT_XC, DSR_NSLOTS };
void *dsr_scratch(int slot, size_t bytes);

/* The per-function path's one-launch expert kernels: the device buffer of epoch-tagged h words (at
 * least n 64-bit words, zeroed when it is allocated). dsr_expert_epoch: the next launch epoch (never
 * 0; a new one per launch), also for the completion words of DSR_PIN_DONE. */
void *dsr_expert_hbuf(size_t n);
unsigned dsr_expert_epoch(void);
/* Whether the expert kernel's device copy of its input (DSR_SLOT_XC) holds these n bytes of host
 * input from the previous call (compared by content); if not, remembers them as the copy the coming
 * launch writes. dsr_input_forget() drops the record (any other use of the slot, a failed launch). */
int dsr_input_cached(const void *x, size_t n);
void dsr_input_forget(void);

/* Pinned, mapped host staging per slot that kernels read and write directly (the per-function API's
 * activations: a call copies its host inputs in, launches, synchronises and copies its outputs out,
 * with no copy commands). dsr_pin_in copies n bytes of src into the slot and returns the device
 * address; dsr_pin_buf returns a slot's device address (and its host address in *host); dsr_pin_out
 * synchronises the stream and copies n bytes of a slot out. Grow-only, not thread-safe. */
enum { DSR_PIN_X, DSR_PIN_A, DSR_PIN_B, DSR_PIN_Y, DSR_PIN_DONE, DSR_NPIN };
const void *dsr_pin_in(int slot, const void *src, size_t n);
void *dsr_pin_buf(int slot, size_t n);
int dsr_pin_out(void *dst, int slot, size_t n);
/* Like dsr_pin_out, for a launch whose blocks store epoch into the n_words completion words of
 * DSR_PIN_DONE when their outputs are written: polls those words instead of synchronising the
 * stream (after about a second without them, synchronises and reports failure). */
int dsr_pin_out_done(void *dst, int slot, size_t n, int n_words, unsigned epoch);

int dsr_h2d(void *dst, const void *src, size_t n);
int dsr_d2h(void *dst, const void *src, size_t n); /* synchronises the stream */

/* Device copy of an INT8 block, uploaded on first use (keyed by the qweight host pointer plus a
 * sampled fingerprint of the host arrays, so a new block at a reused address is detected; in-place
 * edits need ds_hip_weights_changed). */
typedef struct {
  int8_t *q;
  float *scale;
  float *offset;
  int out_dim, in_dim;
} dsr_dblock_t;
int dsr_block_device(const ds_int4_block_t *b, dsr_dblock_t *out);
/* Allocates and registers device arrays for a block the device is about to produce; after the host
 * arrays are filled, dsr_block_adopt() records their fingerprint. */
int dsr_block_new(const ds_int4_block_t *b, dsr_dblock_t *out);
int dsr_block_adopt(const ds_int4_block_t *b, int8_t *q, float *scale, float *offset);
void dsr_block_forget(const void *qweight);

/* Device copy of a host weight array (bf16 / f32), uploaded on first use, same keying. */
const void *dsr_weight_device(const void *host, size_t bytes);
/* A device allocation derived from registered weights (e.g. the LM head's int8 copy): NULL until
 * set; dsr_weight_set_aux hands it to the registry, which frees it with the weights' entry (when
 * the weights change or are replaced). */
void *dsr_weight_aux(const void *host);
int dsr_weight_set_aux(const void *host, void *aux_dev);

/* Emulated reference CPU thread count (ds_set_threads). */
int dsr_threads(void);

/* Attention half of a decoder layer (ds_hip_attn.c): its launches for one token at cache position
 * (pos_ptr ? *pos_ptr : 0) + pos_add, input x_in (+ (*step)*stride when step != NULL). */
struct ds_hip_attn;
hipError_t ds_hip_attn_enqueue(const struct ds_hip_attn *A, const float *x_in, const int *step, int stride,
                               int ncopies, float *x_plain, const int *pos_ptr, int pos_add, float *h_out, float *n_out,
                               const float *WrT_next, int E_next, float *partials_next, int threads);
int ds_hip_attn_hidden(const struct ds_hip_attn *A);
int ds_hip_attn_max_seq(const struct ds_hip_attn *A); /* KV positions the caches hold */
size_t ds_hip_attn_weight_bytes(const struct ds_hip_attn *A); /* projections and norms read per token */

#endif
