/*
 * ds_hip.h — device-resident extension of the ds-ocr MoE decode API (MI355X / gfx950).
 *
 * The per-function API of ds_quantize.h / ds_kernels.h takes host pointers and synchronises on
 * every call, like the reference. A decode step at batch 1 moves ~640 MB in ~100 us on MI355X, so
 * the fast path keeps weights and activations in HBM: a layer handle owns one contiguous arena per
 * MoE layer (all experts' codes, scales/offsets, routers), and a stack handle runs all MoE layers
 * plus the argmax LM head as one captured HIP graph per decode step. This has no counterpart in the
 * reference (whose MoE block, ds_moe_decoder.c:131-333 moe_forward, is a static function); it is
 * the additive C-ABI entry the integration calls instead of the per-expert functions.
 *
 * Conventions: functions returning int return 0 on success and -1 on failure, with the message in
 * ds_hip_last_error() (also printed to stderr). "_dev" pointers are device pointers. All work is
 * ordered on the library's single stream; ds_hip_sync() waits for it.
 */
#ifndef DS_HIP_H
#define DS_HIP_H

#include <stddef.h>
#include <stdint.h>

#include "ds_quantize.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------- runtime ---------------- */
int ds_hip_init(void);
const char *ds_hip_last_error(void);
void *ds_hip_malloc(size_t bytes);
void ds_hip_free(void *p_dev);
int ds_hip_memcpy_h2d(void *dst_dev, const void *src, size_t bytes);
int ds_hip_memcpy_d2h(void *dst, const void *src_dev, size_t bytes);
int ds_hip_memcpy_d2d(void *dst_dev, const void *src_dev, size_t bytes);
/* Average time of n back-to-back launches of a plain streaming read of bytes of src_dev (the
 * achievable-bandwidth reference for the HBM-bound kernels; no counterpart in the reference). */
int ds_hip_time_stream_read(const void *src_dev, size_t bytes, int n, float *ms);
/* Average device time (ms) of n back-to-back launches of the kernel behind
 * ds_expert_forward_fused_int4 (gate_up, SwiGLU and down in one launch, each row in the reference's
 * order) with the input x (host, copied once) and the output in device memory: one expert on its own,
 * without the per-call host transfers (a measurement hook, no counterpart in the reference). The
 * blocks are registered like the per-function API's. */
int ds_hip_time_expert(const ds_int4_block_t *gate_up_int4, const ds_int4_block_t *down_int4, int hidden,
                       int intermediate, const float *x, int n, float *ms);
/* Waits for the library stream. Returns -1 (message in ds_hip_last_error) if a kernel reported since
 * the last check that one of its bounded waits gave up (the prefill's down tiles waiting for their
 * gate_up tiles, the one-kernel decode layers' extra blocks waiting for the verdict on the expert
 * selection): the output of that call or step is not valid. The report is given once. */
int ds_hip_sync(void);
/* Certified CFG routing (no counterpart in the reference; it makes the decode and prefill paths pick
 * exactly the experts ds_moe_router + ds_moe_top_k pick, ds_kernels.c:181-243, on the same input):
 * each MoE layer selects on router scores summed in its own order, checks the selection against a
 * rigorous bound on the difference to ds_linear's sequential order, and recomputes the scores of
 * the experts the bound leaves open in that order. In the stacks' one-kernel layers the routed
 * blocks select from the accumulated scores and add their shares at once, while 32 extra blocks
 * compute the exact scores' intervals and certify that selection, or add the difference to the one
 * certified (rare: a near tie the accumulated scores ranked otherwise). counts[0] = decode routings made since the last
 * reset, counts[1] = those that needed the recomputation, counts[2] = one-kernel layers whose output
 * was corrected to the certified selection (their routed blocks had used another). Synchronises;
 * reset = 1 zeroes them. */
int ds_hip_route_stats(unsigned long long *counts, int reset);
/* Test aid: a device buffer that receives one entry per decode routing (CFG: every layer kind;
 * DECODE: the stacks' one-kernel layers) (log_dev[0] = entries
 * written, then from int 64 entries of 32 + hidden ints: idx[8], w[8] (f32 bits), flags (bit 0:
 * recomputed in ds_linear's order; bit 1: a one-kernel layer's verdict replaced its speculative
 * selection), the layer index, 14 spare ints, the routed input [hidden] (f32 bits)). Kernels record
 * into the buffer set when they are launched or captured (ds_hip_stack_bind); NULL, 0 switches it
 * off. The caller zeroes log_dev[0]. */
int ds_hip_set_route_log(int *log_dev, int capacity);
/* Seeded synthetic data generated on the device (counter-based SplitMix64 + Box–Muller). */
int ds_hip_fill_normal_bf16(uint16_t *dst_dev, size_t n, uint64_t seed, float std_);
int ds_hip_fill_normal_f32(float *dst_dev, size_t n, uint64_t seed, float mean, float std_);

/* The per-function API (ds_quantize.h, ds_kernels.h) keeps one device copy per host weight array and
 * INT8 block, registered on first use and keyed by its address (plus a sampled fingerprint that
 * catches a new array at a freed one's address). Weights edited in place after they were used must
 * be announced: host_ptr is the array (or a block's qweight); its device copy is dropped and
 * uploaded again at the next use. Returns the number of copies dropped (0 if none), -1 on error.
 * No counterpart in the reference, whose weights are read-only mmaps (ds_ocr.c:611-622). */
int ds_hip_weights_changed(const void *host_ptr);
/* Diagnostic: 1 when ds_argmax_matvec_bf16 serves the registered head W_bf16 through its int8 copy
 * with exact bounds (built at the first call when every row is in the reference's 4-row-group
 * order for the current thread count and the head's shape is supported), 0 when it streams the bf16
 * head. No counterpart in the reference. */
int ds_hip_argmax_int8_copy(const uint16_t *W_bf16);
/* Registers (uploads) a block or a weight array now rather than at its first use, e.g. at load time
 * so the first tokens do not pay for the uploads. 0 or -1. */
int ds_hip_register_block(const ds_int4_block_t *block);
int ds_hip_register_weights(const void *host, size_t bytes);

/* ---------------- device-pointer kernels ---------------- */
int ds_hip_quantize_bf16(int8_t *q_dev, float *scale_dev, float *offset_dev, const uint16_t *W_dev, int out_dim,
                         int in_dim);
int ds_hip_int8_matvec(float *y_dev, const float *x_dev, const int8_t *q_dev, const float *scale_dev,
                       const float *offset_dev, int in_dim, int row_start, int nrows);
/* Argmax of W x (bf16 W [out_dim, in_dim]) in the reference's order for ds_get_threads() threads;
 * writes the index to *idx_dev. */
int ds_hip_argmax_bf16(int *idx_dev, const float *x_dev, const uint16_t *W_dev, int in_dim, int out_dim);
/* ds_hip_argmax_bf16 without any allocation: no counterpart in the reference; for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). The per-block candidate keys live in a static device array of the library
 * (262144 rows at most: out_dim beyond that is refused with an error); ds_hip_init must have been
 * called. Same result as ds_hip_argmax_bf16. Every call on a device shares that device's array, so
 * calls that overlap on one device (several host threads or streams) race. */
int ds_hip_argmax_bf16_noalloc(int *idx_dev, const float *x_dev, const uint16_t *W_dev, int in_dim, int out_dim);

/* ---------------- device-resident MoE layer ---------------- */
enum { DS_HIP_ROUTE_DECODE = 0, DS_HIP_ROUTE_CFG = 1 };
/* DS_HIP_ROUTE_DECODE: the reference decode router (bf16 weights, fast-exp softmax over all
 *   experts, top-k, weights = probabilities; ds_moe_decoder.c:145-183).
 * DS_HIP_ROUTE_CFG: f32 router + ds_moe_top_k (top-k on raw scores, softmax over the k). */

typedef struct ds_hip_layer ds_hip_layer_t;

/* shared_inter = n_shared * inter (the shared experts' fused gate_up is [2*shared_inter, hidden]). */
ds_hip_layer_t *ds_hip_layer_create(int hidden, int inter, int n_experts, int top_k, int shared_inter);
void ds_hip_layer_destroy(ds_hip_layer_t *L);
size_t ds_hip_layer_bytes(const ds_hip_layer_t *L);
/* Host router weights [n_experts, hidden]; either may be NULL. */
int ds_hip_layer_set_router(ds_hip_layer_t *L, const float *router_f32, const uint16_t *router_bf16);
/* Router weights already on the device (copied into the arena). */
int ds_hip_layer_set_router_dev(ds_hip_layer_t *L, const float *router_f32_dev, const uint16_t *router_bf16_dev);
/* Copies host INT8 blocks into the arena. e in [0, n_experts) or -1 for the shared expert.
 * gate_up is [2*I, hidden] (gate rows then up rows), down is [hidden, I]. */
int ds_hip_layer_set_expert(ds_hip_layer_t *L, int e, const ds_int4_block_t *gate_up, const ds_int4_block_t *down);
/* Quantizes device BF16 weights straight into the arena (bit-identical to ds_int4_quantize_bf16). */
int ds_hip_layer_quantize_expert(ds_hip_layer_t *L, int e, const uint16_t *gate_up_bf16_dev,
                                 const uint16_t *down_bf16_dev);
/* Copies an expert's codes/scales/offsets back to host arrays (any pointer may be NULL). */
int ds_hip_layer_export_expert(const ds_hip_layer_t *L, int e, int8_t *gu_q, float *gu_scale, float *gu_offset,
                               int8_t *dn_q, float *dn_scale, float *dn_offset);
/* out_dev[hidden] = (residual ? x : 0) + MoE(x_dev). idx_dev/w_dev (optional, [top_k]) receive the
 * routing. bf16sim follows ds_bf16_simulate_python. Asynchronous. out_dev may equal x_dev. */
int ds_hip_layer_forward(ds_hip_layer_t *L, float *out_dev, const float *x_dev, int route_mode, int residual,
                         int *idx_dev, float *w_dev);

/* Prefill MoE block for T tokens (ds_moe_decoder.c:629-809, on this layer's INT8 blocks):
 * out_dev[T][hidden] = (residual ? x : 0) + MoE(x_dev[T][hidden]). Routing per token as
 * ds_hip_layer_forward (route_mode), experts as an expert-sorted grouped GEMM on the int8 MFMA
 * (each f32 activation row as two 8-bit limbs, exact integer sums), routed outputs added in
 * ascending expert order, then the shared expert. idx_dev/w_dev (optional,
 * [T][top_k]) receive the routing. Asynchronous; out_dev must not alias x_dev. The reference's block
 * is synchronous and always complete: if the persistent GEMM kernel's bounded wait gives up (its
 * gate_up tiles not done after the wait limit), the next ds_hip_sync, ds_hip_prefill_wait_error or
 * ds_hip_layer_prefill call returns -1 with ds_hip_last_error saying so, and that output is not
 * valid. */
int ds_hip_layer_prefill(ds_hip_layer_t *L, float *out_dev, const float *x_dev, int T, int route_mode, int residual,
                         int *idx_dev, float *w_dev);

/* Average device time (ms) of n back-to-back ds_hip_layer_prefill calls (no residual). */
int ds_hip_time_prefill(ds_hip_layer_t *L, float *out_dev, const float *x_dev, int T, int route_mode, int n, float *ms);
/* Average device time (ms) of n back-to-back ds_hip_layer_forward calls (no residual): one MoE layer
 * on its own with its input in device memory (a measurement hook, no counterpart in the reference). */
int ds_hip_time_layer(ds_hip_layer_t *L, float *out_dev, const float *x_dev, int route_mode, int n, float *ms);

/* Prefill GEMM path (no counterpart in the reference): 1 = one persistent kernel with a work queue
 * per XCD, 0 = separate gate_up and down kernels, -1 = automatic (persistent when a grid's blocks
 * cover every XCD). Returns the path in use, -1 on error. */
int ds_hip_prefill_path(int mode);

/* After a prefill call of T tokens on L: 1 if the persistent kernel's bounded wait for a gate_up
 * tile expired (that call's output is not valid), 0 if not, -1 on error. Synchronises. */
int ds_hip_prefill_wait_error(ds_hip_layer_t *L, int T);
/* Test hook (no counterpart in the reference): the sleeps after which a persistent prefill tile's
 * wait for its gate_up tiles gives up. DS_HIP_PREFILL_WAIT_DEFAULT restores the default (2^22);
 * spins < 0 makes every such wait give up at once (every kernel still runs to its end; the output is
 * then not valid and the failure is reported as above). Takes effect at the next call. */
#define DS_HIP_PREFILL_WAIT_DEFAULT (-2147483647 - 1)
int ds_hip_prefill_set_wait_limit(int spins);

/* Self-check of the prefill SwiGLU (no counterpart in the reference): the GEMM epilogue's
 * reciprocal-based (g / (1 + fast_exp(-g))) * u against the correctly rounded division of
 * ds_swiglu_direct (ds_kernels.c:1771) over all 2^32 gate values, u = 1. n_differ[0]: finite g
 * with a zero or normal quotient whose results differ in any bit (0 expected), n_differ[1]: finite
 * g with a subnormal quotient (|g| < 2.4e-38) whose results differ. About a second; synchronous. */
int ds_hip_check_prefill_swiglu(uint64_t *n_differ);

/* ---------------- dense FFN layer (layer 0 of the decoder) ---------------- */
/* The decoder's dense SwiGLU FFN (ds_moe_decoder.c:75-105, dense_ffn_forward): gate [inter, hidden],
 * up [inter, hidden], down [hidden, inter] BF16 host arrays, uploaded once. Needs hidden % 128 == 0
 * (<= 2048) and inter % 8 == 0 (<= 16384). f32 dots of the exact bf16 values in a lane-parallel order
 * (the reference's AVX-512 chains differ by f32 rounding), fast-exp SwiGLU as ds_swiglu_direct. */
typedef struct ds_hip_dense ds_hip_dense_t;
ds_hip_dense_t *ds_hip_dense_create(int hidden, int inter, const uint16_t *gate, const uint16_t *up,
                                    const uint16_t *down);
void ds_hip_dense_destroy(ds_hip_dense_t *D);
/* out_dev[hidden] = (residual ? x : 0) + FFN(x_dev); out_dev may equal x_dev. Asynchronous. */
int ds_hip_dense_forward(ds_hip_dense_t *D, float *out_dev, const float *x_dev, int residual);

/* ---------------- weights: checkpoints and the persisted INT8 arena ---------------- */
/* Tensor dtypes reported by ds_hip_safetensors_info. */
enum { DS_HIP_ST_BF16 = 0, DS_HIP_ST_F32 = 1, DS_HIP_ST_F16 = 2, DS_HIP_ST_OTHER = 3 };
/* Looks a tensor up in a set of safetensors shards (the reference reads them through
 * ds_safetensors.h:50-75 / multi_safetensors_find); writes its dtype and up to max_dims extents and
 * returns its rank, or -1. Host only (no GPU needed). */
int ds_hip_safetensors_info(const char *const *files, int n_files, const char *name, int *dtype, int64_t *shape,
                            int max_dims);
/* Builds n_layers device MoE layers from DeepSeek-OCR safetensors shards, layers first_layer ..
 * first_layer + n_layers - 1, with the reference's tensor names (ds_ocr.c:653-680):
 * model.layers.{l}.mlp.gate.weight (router, BF16 or F32), ...mlp.experts.{e}.{gate,up,down}_proj.weight
 * and ...mlp.shared_experts.{gate,up,down}_proj.weight (BF16). Shapes come from the tensors; top_k
 * from the model config. gate and up rows are fused as the reference does (ds_ocr.c:696-768) and
 * quantized on the device, bit-identical to ds_quantize_moe_int4 (ds_ocr.c:781-841). A BF16 router
 * also gives the f32 router (its values widened); an F32 router gives no bf16 router. Returns
 * n_layers (layers[0..n) filled) or -1 (nothing left allocated). Synchronous. */
int ds_hip_load_moe_layers(const char *const *files, int n_files, int first_layer, int n_layers, int top_k,
                           ds_hip_layer_t **layers);
/* The dense FFN of layer `layer` (model.layers.{l}.mlp.{gate,up,down}_proj.weight, BF16;
 * ds_ocr.c:653-657) as a device handle. Returns 0 or -1. */
int ds_hip_load_dense(const char *const *files, int n_files, int layer, ds_hip_dense_t **dense);
/* Uploads lm_head.weight (BF16 [vocab, hidden]; ds_ocr.c:686) to a new device buffer (free with
 * ds_hip_free). Returns 0 or -1. */
int ds_hip_load_lm_head(const char *const *files, int n_files, uint16_t **lm_head_dev, int *vocab, int *hidden);
/* Persisted packed INT8 arena. No counterpart in the reference, which re-quantizes every expert at
 * each load (ds_quantize_moe_int4, ds_ocr.c:781-841); for integrations that keep the packed weights
 * instead of the BF16 checkpoint. Saves the layers (same shape) -- INT8 codes, (scale, offset)
 * pairs, routers -- and optionally the bf16 LM head (lm_head_dev NULL: none) to path, versioned and
 * checksummed. Returns 0 or -1. */
int ds_hip_arena_save(const char *path, ds_hip_layer_t *const *layers, int n_layers, const uint16_t *lm_head_dev,
                      int vocab);
/* Reads a file written by ds_hip_arena_save into new layers (layers[0..n), n <= max_layers) and, if
 * it holds an LM head, a new device buffer (*lm_head_dev, free with ds_hip_free; *vocab). Checks the
 * format version, shapes, size and checksum. Returns the number of layers or -1 (nothing left
 * allocated). */
int ds_hip_arena_load(const char *path, ds_hip_layer_t **layers, int max_layers, uint16_t **lm_head_dev, int *vocab);

/* ---------------- attention half of a decoder layer, one token ---------------- */
/* decoder_layer_forward up to the MLP (ds_moe_decoder.c:339-431; MHA): x_norm = ds_rms_norm(x),
 * q/k/v = ds_linear_nobias_bf16_qkv, optional per-head q/k norms, RoPE (ds_compute_rope_neox /
 * ds_apply_rope_neox), k and v into the F32 KV cache, causal or R-SWA attention
 * (ds_causal_attention_aligned / ds_rswa_attention_aligned), O projection, then
 * ds_residual_rms_norm: h = x + proj and n = RMSNorm(h) -- the MLP's input and residual. Every step
 * but the attention's output sum is bit-exact with the reference; that sum differs by f32 rounding.
 * No counterpart object in the reference (its layer keeps these in ds_ctx_t). */
typedef struct ds_hip_attn ds_hip_attn_t;
#define DS_HIP_ATTN_MAX_SEQ 7680 /* KV positions per layer (the softmax keeps 2 floats per position in LDS) */
/* Weights: bf16 [n_heads*head_dim][hidden] for wq, wk, wv, bf16 [hidden][n_heads*head_dim] for wo;
 * norms f32 [hidden] (q_norm, k_norm: [head_dim] or NULL). Host arrays, uploaded. */
ds_hip_attn_t *ds_hip_attn_create(int hidden, int n_heads, int head_dim, int max_seq, float rms_eps, float rope_theta,
                                  const uint16_t *wq, const uint16_t *wk, const uint16_t *wv, const uint16_t *wo,
                                  const float *input_norm, const float *post_attn_norm, const float *q_norm,
                                  const float *k_norm);
void ds_hip_attn_destroy(ds_hip_attn_t *A);
/* R-SWA (Unlimited-OCR): tokens at positions >= prefill_len attend to [0, prefill_len) and the last
 * sliding_window positions (ds_moe_decoder.c:396-423); sliding_window 0: causal. */
int ds_hip_attn_set_window(ds_hip_attn_t *A, int prefill_len, int sliding_window);
/* The device KV caches ([max_seq][kv_stride] f32 each; k rows roped). */
int ds_hip_attn_kv(const ds_hip_attn_t *A, float **k_cache_dev, float **v_cache_dev, int *kv_stride);
/* Uploads n_pos cached rows (e.g. from a prefill) from host arrays with row stride host_stride. */
int ds_hip_attn_load_kv(ds_hip_attn_t *A, const float *k_host, const float *v_host, int n_pos, int host_stride);
/* One token at cache position pos: writes its k, v into the caches, h_dev = x + O(attention),
 * n_dev = RMSNorm(h) (device [hidden] each). Asynchronous. */
int ds_hip_attn_forward(ds_hip_attn_t *A, float *h_dev, float *n_dev, const float *x_dev, int pos);

/* ---------------- decode stack: n MoE layers + argmax LM head ---------------- */
typedef struct ds_hip_stack ds_hip_stack_t;

/* Greedy sampling rules of ds_decoder_forward at temperature 0 (ds_moe_decoder.c:1036-1095 and the
 * full-logits path :1105-1237) applied after each step's argmax, on the device: the repetition
 * penalty (> 1 enables it) over the stack's earlier tokens (the first history_cap of them, as the
 * reference's capped token_history) and the n-gram ban (no_repeat_ngram_size > 0). Call before
 * ds_hip_stack_bind; (1.0, 0, 0) turns them off. The full-logits path computes the logits in
 * ds_bf16_matvec_pub's order. */
int ds_hip_stack_set_sampling(ds_hip_stack_t *S, float repeat_penalty, int no_repeat_ngram_size, int history_cap);
/* The same rules for one hidden state, device pointers: token_dev[0] receives the chosen token
 * (argmax, penalty over history_dev[0..history_len), n-gram ban). Asynchronous. */
int ds_hip_lm_head_sample(const float *x_dev, const uint16_t *lm_head_dev, int hidden, int vocab, const int *history_dev,
                          int history_len, float repeat_penalty, int no_repeat_ngram_size, int *token_dev);

/* Steps per graph launch in ds_hip_stack_run and the timed runs (no counterpart in the reference; a
 * launch setting): runs of several steps launch a graph of k steps at a time (the step's kernels
 * captured k times; each step takes its index from the device step counter), then 1-step graphs
 * for the rest. Results are the same for every k. Any time; 1..DS_HIP_GRAPH_STEPS_MAX. */
#define DS_HIP_GRAPH_STEPS_MAX 16
#define DS_HIP_GRAPH_STEPS_DEFAULT 8
int ds_hip_stack_set_graph_steps(ds_hip_stack_t *S, int k);


/* Makes each step a whole decoder step (ds_decoder_forward for one token, ds_moe_decoder.c:339-474
 * and :1000): attn[i] is decoder layer i's attention half (the dense layer's first when one is set,
 * then one per MoE layer; call after ds_hip_stack_set_dense), each followed by its MLP on the
 * post-attention RMSNorm with the attention's output as the residual; then ds_rms_norm with
 * final_norm ([hidden] host array, final_eps) -- bf16-truncated when trunc_final and the bf16
 * simulation are on (model version 3) -- feeds the LM head. Step s is cache position pos0 + s.
 * Before ds_hip_stack_bind; (NULL, 0, ...) returns to MoE layers only. Blocks are borrowed. */
int ds_hip_stack_set_attention(ds_hip_stack_t *S, ds_hip_attn_t *const *attn, int n_attn, const float *final_norm,
                               float final_eps, int pos0, int trunc_final);
/* lm_head_dev: bf16 [vocab, hidden] on the device (borrowed). Layers are borrowed. The reference
 * thread count current here (ds_set_threads, ds_kernels.c:123-175) is the one the stack emulates for
 * as long as it lives (the row chunks of the DECODE router, the LM head's row order, the attention's
 * QKV split, the sampling rules); a later ds_set_threads does not change it. */
ds_hip_stack_t *ds_hip_stack_create(ds_hip_layer_t *const *layers, int n_layers, const uint16_t *lm_head_dev,
                                    int vocab, int route_mode);
/* Puts a dense FFN layer before the MoE layers (the decoder's layer 0): a step then runs
 * x = x + FFN(x) on the step's input first, and in CFG routing its down kernel also writes the first
 * MoE layer's router partials (no separate scores kernel). Call before ds_hip_stack_bind; the dense
 * handle must outlive the stack. D = NULL removes it. */
int ds_hip_stack_set_dense(ds_hip_stack_t *S, ds_hip_dense_t *D);
/* MoE layer kernels of the stack's steps (the default, one_kernel = 1): one kernel per layer, the
 * down product split over the intermediate units with the layer output added up in per-XCD copies
 * (device tables built by ds_hip_stack_bind: the down weights in unit tiles, ~76 MB per layer at
 * DeepSeek's shape, and in CFG routing the next router's products with them, ~15 MB); DECODE
 * routing keeps its exact scores kernel before each layer. The low bits of the output then depend
 * on the order of the device's atomic adds. one_kernel = 0: two kernels per layer (gate_up, then
 * down with the combine in top-k order; deterministic). The bf16 simulation always uses two.
 * Call before ds_hip_stack_bind; the tables copy the layers' weights at bind time, so bind again
 * after changing a layer's experts or router. */
int ds_hip_stack_set_layer_kernels(ds_hip_stack_t *S, int one_kernel);
/* Kernels per MoE layer of the bound stack (1 or 2). */
int ds_hip_stack_layer_kernels(const ds_hip_stack_t *S);
/* LM-head argmax over an int8 copy of the head (no counterpart in the reference; the tokens are
 * the reference's, ds_argmax_matvec_bf16's, ds_kernels_avx.c:162-245). Each block of 512 rows
 * (one block per CU) streams the int8 rows (half the bytes) with a rigorous bound on every row's
 * exact logit, then
 * recomputes in the reference's order only its rows whose upper bound reaches the block's largest
 * lower bound, which always include the block's argmax and every row tied with it. On by default
 * where the one-pass head applies and hidden is a multiple of 256 (<= 2048); ds_hip_stack_create
 * builds the copy (vocab x hidden bytes + 12 bytes per row) from the head's contents then. on = 1
 * rebuilds it (call after rewriting the head's weights), 0 returns to the one-pass head. Call
 * before ds_hip_stack_bind. */
int ds_hip_stack_set_lm_certified(ds_hip_stack_t *S, int on);
/* 1 if the stack's steps use the int8 copy of the head. */
int ds_hip_stack_lm_certified(const ds_hip_stack_t *S);
void ds_hip_stack_destroy(ds_hip_stack_t *S);
/* Autoregressive input (ds_ocr.c:2271-2278, the decode loop's "embedding for next token"): with a
 * table set, step s >= 1 reads the BF16 embedding row of the token step s - 1 chose (after the
 * sampling rules, when set), widened to f32 by << 16, and step 0 reads row 0 of the bound input
 * (the caller's first input, e.g. the embedding of the prefill's token). A token outside
 * [0, vocab) leaves the input as it was, as the reference's guard does. The row is written on the
 * device by the step that chose the token, so n steps run with no host round trip.
 * tok_embeddings_dev: bf16 [vocab][hidden] on the device, 16-byte aligned, borrowed; hidden % 8 == 0.
 * Call before ds_hip_stack_bind; NULL turns the feed off. */
int ds_hip_stack_set_embedding(ds_hip_stack_t *S, const uint16_t *tok_embeddings_dev, int vocab);
/* Binds the steps' input and output and captures the graph. Step s (counted from the bind or the
 * last reset) reads its input hidden state from xs_dev + s*stride (stride 0: always xs_dev; the
 * embedding feed reads only row 0, at reset) and writes its token to tokens_dev[s]. n_rows is the
 * number of rows xs_dev holds and n_tokens the length of tokens_dev: the stack then runs at most
 * ds_hip_stack_capacity(S) steps between resets -- the smaller of n_tokens, n_rows (when rows are
 * read per step) and, for whole decoder steps, the KV positions left (max_seq - pos0) -- and every
 * call that launches steps refuses, before launching anything, to go past it. */
int ds_hip_stack_bind(ds_hip_stack_t *S, const float *xs_dev, int stride, int n_rows, int *tokens_dev,
                      int n_tokens);
/* Steps a bound stack may run between resets, and how many of them are left. */
int ds_hip_stack_capacity(const ds_hip_stack_t *S);
int ds_hip_stack_steps_left(const ds_hip_stack_t *S);
/* The capacity rule on its own (host arithmetic, no device): n_rows rows of input read per step
 * when stride > 0, n_tokens token slots, kv_room KV positions left (-1: no attention). Returns the
 * capacity, or -1 for invalid arguments. */
int ds_hip_stack_capacity_for(int n_rows, int stride, int n_tokens, int kv_room);
/* 1 if n more steps fit after steps_done of a capacity, else 0 (host arithmetic). */
int ds_hip_steps_fit(int capacity, int steps_done, int n);
/* Zeroes the step counter and the step's work buffers (with the embedding feed, row 0 of the bound
 * input becomes the next step's input). */
int ds_hip_stack_reset(ds_hip_stack_t *S);
/* Launches n_steps decode steps (one graph launch each), asynchronously. Every step's token is in
 * tokens_dev once the launched work completes. (With one-kernel layers in CFG routing, at least 3
 * layers and the bound input, a step ends with the LM head: the next step's first layer writes the
 * previous step's token, and one kernel after the run's last step writes its token.) */
int ds_hip_stack_run(ds_hip_stack_t *S, int n_steps);
/* Same steps launched kernel by kernel, without the graph. */
int ds_hip_stack_run_eager(ds_hip_stack_t *S, int n_steps);
/* Final hidden state (after the last MoE layer) of the most recent step, to the host. */
int ds_hip_stack_hidden(ds_hip_stack_t *S, float *x_host);
size_t ds_hip_stack_bytes_per_step(const ds_hip_stack_t *S);

/* ---------------- timing (HIP events on the library stream) ---------------- */
/* Every timing call that runs steps counts them against the stack's capacity, like ds_hip_stack_run. */
/* Wall time of n_steps graph launches. */
int ds_hip_time_stack(ds_hip_stack_t *S, int n_steps, float *ms);
/* n_steps graph launches with an event between consecutive launches: ms_each[i] is step i's
 * launch-to-launch time (for medians and percentiles). */
int ds_hip_time_stack_each(ds_hip_stack_t *S, int n_steps, float *ms_each);
/* n_steps eager steps, each with one event before kernel group k0 and one after group k1 - 1
 * (groups as ds_hip_stack_kernel_name numbers them): ms_each[i] is that span in step i, on the
 * step's real inputs. E.g. the MoE layers of a step, for their average launch duration. */
int ds_hip_time_stack_span(ds_hip_stack_t *S, int n_steps, int k0, int k1, float *ms_each);
/* Average time of the LM-head argmax kernel over n back-to-back launches on the stack's current
 * hidden state (no token written; includes the launch gaps). */
int ds_hip_time_lm_head(ds_hip_stack_t *S, int n, float *ms);
/* Kernels one decode step launches, and the kind of kernel i ("scores", "gate_up", "down", "layer",
 * "lm_head.argmax", "lm_head.final", "lm_head.final+scores"; no final kernel where the step ends with
 * the LM head). */
int ds_hip_stack_kernel_count(const ds_hip_stack_t *S);
const char *ds_hip_stack_kernel_name(const ds_hip_stack_t *S, int i);
/* Per-kernel durations over n_steps eager steps, HIP events around every kernel; ms_out receives
 * ds_hip_stack_kernel_count(S) averages in launch order. */
int ds_hip_profile_stack(ds_hip_stack_t *S, int n_steps, float *ms_out);

#ifdef __cplusplus
}
#endif

#endif /* DS_HIP_H */
