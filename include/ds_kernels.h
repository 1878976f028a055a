/*
 * ds_kernels.h — the MoE-decode subset of the reference's ds_kernels.h, MI355X implementation.
 *
 * Same names, signatures and argument meaning as the reference (vislee/ds-ocr ds_kernels.h), so the
 * reference's call sites in ds_moe_decoder.c (MoE block, LM head) link unchanged. Every function
 * computes on the GPU; host pointers in, host results out, synchronous.
 *
 * Bit-exactness: functions marked [exact] return the same bits as the reference x86 build for the
 * same inputs and the same ds_set_threads() count (the count decides which rows the reference's
 * AVX-512 kernels process in the single-row order). The rest are within 1e-3 relative error.
 */
#ifndef DS_KERNELS_H
#define DS_KERNELS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DS_MAX_EXPERTS 64

/* Mode globals (reference ds_kernels.h:269-270, defined in ds_ocr.c:26-27). The library provides
 * weak definitions (both 0) so it also links without ds_ocr.c. */
extern int ds_verbose;
extern int ds_bf16_simulate_python;

/* ---- matrix ---- */
/* Reference ds_kernels.h:45-46 / ds_kernels.c:917-927. seq_len == 1: [exact] AVX-512-order BF16
 * matvec. seq_len > 1: f32 GEMM on the widened weights (the reference calls sgemm). */
void ds_linear_nobias_bf16(float *y, const float *x, const uint16_t *W_bf16, int seq_len, int in_dim, int out_dim);

/* Reference ds_kernels.h:86 / ds_kernels.c:1621-1642. [exact] */
void ds_vec_add(float *dst, const float *a, const float *b, int n);

/* ---- activations ---- */
/* Reference ds_kernels.h:107-108 / ds_kernels.c:1739-1789 (fast-exp SiLU). [exact] */
void ds_swiglu_direct(float *out, const float *gate_buf, const float *up_buf, int seq_len, int intermediate);

/* ---- MoE ---- */
/* Reference ds_kernels.h:189-190 / ds_kernels.c:181-185. f32 router scores[n_experts]. [exact]
 * against the reference built without BLAS (the BLAS build's sgemm order is not reproducible). */
void ds_moe_router(float *scores, const float *x, const float *gate_weight, int hidden, int n_experts);
/* Reference ds_kernels.h:191-192 / ds_kernels.c:187-191. [exact] */
void ds_moe_router_bf16(float *scores, const float *x, const uint16_t *gate_weight_bf16, int hidden, int n_experts);
/* Reference ds_kernels.h:195-196 / ds_kernels.c:193-243. Indices [exact]; weights use the device
 * expf (within 1 ulp of glibc's). n_experts <= 64. */
void ds_moe_top_k(int *top_indices, float *top_weights, const float *scores, int n_experts, int top_k);
/* Reference ds_kernels.h:209-214 / ds_kernels.c:322-357 (BF16 experts). [exact] */
void ds_expert_forward_fused(float *out, const float *x, const uint16_t *gate_up_fused_bf16, const uint16_t *down_bf16,
                             int hidden, int intermediate, float *gate_up_buf, float *gate_buf, float *up_buf,
                             float *hidden_buf);
/* Reference ds_kernels.h:230-232 / ds_kernels.c:359-371. [exact] */
void ds_expert_combine(float *output, const float *expert_outputs, const int *top_indices, const float *top_weights,
                       int top_k, int hidden);

/* ---- sampling ---- */
/* Reference ds_kernels.h:239-240 / ds_kernels.c:1013-1016. [exact] index (lowest index among equal
 * maxima, NaN rows never chosen, 0 when no logit exceeds -1e30). */
int ds_argmax_matvec_bf16(const float *x, const uint16_t *W_bf16, int in_dim, int out_dim);
/* Reference ds_kernels.h:244-246 / ds_kernels.c:1020-1099, including its thread-count-dependent
 * fallback when the best token is excluded. [exact] */
int ds_argmax_matvec_bf16_excluding(const float *x, const uint16_t *W_bf16, int in_dim, int out_dim,
                                    const int *exclude_ids, int n_exclude);
/* Reference ds_kernels.h:250-251 / ds_kernels.c:981-1011 (non-NEON branch). [exact] */
float ds_bf16_dot_row(const float *x, const uint16_t *W_bf16, int in_dim, int tok_id);
/* Reference ds_kernels.h:254-255 / ds_kernels.c:942-945. [exact] (bias NULL). */
void ds_bf16_matvec_pub(float *y, const float *x, const uint16_t *W_bf16, const float *b, int in_dim, int out_dim);

/* ---- BF16 simulation ---- */
/* Reference ds_kernels.h:330 / ds_kernels.c:2464-2492. [exact] */
void ds_bf16_truncate_array(float *data, int n);

/* ---- threading (reference ds_kernels.h:262-276, ds_kernels.c:517-582) ----
 * The GPU replaces the CPU pool. ds_set_threads keeps the reference's clamp to [1, 16] and records
 * the count, which selects the reference row order the [exact] BF16 kernels reproduce.
 * ds_parallel_for runs fn(0, 1, arg) on the calling thread. */
typedef void (*ds_parallel_fn_t)(int tid, int n_threads, void *arg);
void ds_set_threads(int n);
int ds_get_threads(void);
int ds_get_num_cpus(void);
void ds_dispatch_ensure_init(void);
void ds_parallel_for(ds_parallel_fn_t fn, void *arg);

/* Reference ds_kernels.h:296-302 (Schraudolph fast exp), kept inline as in the reference. */
static inline float ds_fast_expf(float x) {
  if (x < -88.0f) return 0.0f;
  if (x > 88.0f) return 1e38f;
  union {
    uint32_t i;
    float f;
  } u;
  u.i = (uint32_t)(12102203.0f * x + 1064866805.0f);
  return u.f;
}

#ifdef __cplusplus
}
#endif

#endif /* DS_KERNELS_H */
