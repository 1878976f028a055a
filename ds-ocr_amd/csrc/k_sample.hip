// k_sample.hip — the decoder's greedy token choice with its repetition penalty and n-gram ban, on the
// device (ds_moe_decoder.c:1036-1095, the fast path; :1105-1237, the full-logits path at temperature
// 0). The argmax comes from the LM-head kernels; these kernels then
//   k_sample_dots   : ds_bf16_dot_row (one sequential fused chain, ds_kernels.c:1000-1008) of the
//                     argmax token and of every history token, one wave per token;
//   k_sample_select : the penalty on the argmax's own logit if it is in the history, the best
//                     penalised history logit (the reference's in-order scan keeps the first of equal
//                     values and replaces only on a strictly greater one, so it is the maximum over
//                     the history with the lowest index, compared to the argmax's value), then the
//                     n-gram ban of the chosen token; a banned choice sets the full-path flag;
//   k_sample_full_logits, k_sample_full_pick : only when the flag is set (otherwise they return at
//                     once): all logits in ds_bf16_matvec_pub's order, the penalty once per history
//                     occurrence, banned tokens at -1e30, then the first maximum.
// The history and the token live either in a stack's token array (tokens[0..s) is the history and
// tokens[s] the argmax, s = *step - 1, after the argmax's final kernel advanced the step) or in
// explicit arrays.
#include "dsh.h"
#include "dsh_avx.h"
#include "k_core.h"

struct smp_io {
  const int *step;  // stack: the advanced step counter; NULL: explicit history
  int *tokens;      // stack: token array; explicit: token[0] holds the argmax, then the choice
  const int *hist;  // explicit history (step == NULL)
  int hist_len;     // explicit: its length; stack: the history capacity (the reference keeps the
                    // first token_history_cap tokens, ds_ocr.c:2246-2248)
};

__device__ __forceinline__ void smp_resolve(const smp_io &io, const int *&hist, int &n, int *&tok) {
  if (io.step) {
    const int s = *io.step - 1;
    hist = io.tokens;
    n = min(s, io.hist_len);
    tok = io.tokens + s;
  } else {
    hist = io.hist;
    n = io.hist_len;
    tok = io.tokens;
  }
}

// ds_moe_decoder.c:1048, :1058, :1191-1195 (a true division, as the reference's)
__device__ __forceinline__ float smp_penalize(float v, float rp) { return v > 0.0f ? v / rp : v * rp; }

// 1 if the history's last p tokens also occur at position i and are followed there by tok.
__device__ __forceinline__ bool smp_bans(const int *hist, int n, int p, int i, int tok) {
  for (int j = 0; j < p; j++)
    if (hist[i + j] != hist[n - p + j]) return false;
  return hist[i + p] == tok;
}

// Item j of the dots: 0 is the argmax token, j >= 1 the history entry j - 1; one 64-lane block per
// item. The block stages x and the row in LDS as f32 (every lane's 16-byte pieces in flight
// together, converted by all lanes), then lane 0 runs the chain: a pure dependent FMA chain reading
// LDS (~1280 steps at H 1280, the kernel's latency). vals[j] = NaN for an id outside [0, vocab).
#define SMP_MAX_H 4096
__global__ void __launch_bounds__(64) k_sample_dots(const uint16_t *__restrict__ W, const float *__restrict__ x,
                                                    int H, int vocab, smp_io io, float *__restrict__ vals) {
  extern __shared__ __attribute__((aligned(16))) float s_x[];  // H floats of x, then H floats of the row
  float *s_r = s_x + H;
  const int lane = threadIdx.x;
  const int nx = H / 4, nw = H / 8;  // 16-byte pieces
  constexpr int XP = SMP_MAX_H / 4 / 64, WP = SMP_MAX_H / 8 / 64;
  {  // x's pieces, all in flight, before anything that waits
    f32x4 xr[XP];
#pragma unroll
    for (int q = 0; q < XP; q++)
      if (64 * q < nx) xr[q] = ((const f32x4 *)x)[min(lane + 64 * q, nx - 1)];
#pragma unroll
    for (int q = 0; q < XP; q++)
      if (64 * q < nx && lane + 64 * q < nx) ((f32x4 *)s_x)[lane + 64 * q] = xr[q];
  }
  const int *hist;
  int n;
  int *tok;
  smp_resolve(io, hist, n, tok);
  for (int j = blockIdx.x; j <= n; j += gridDim.x) {
    const int t = j == 0 ? *tok : hist[j - 1];
    if (t < 0 || t >= vocab) {
      if (lane == 0) vals[j] = __builtin_nanf("");
      continue;
    }
    const u32x4 *row = (const u32x4 *)(W + (size_t)t * H);
    u32x4 pc[WP];
#pragma unroll
    for (int q = 0; q < WP; q++)
      if (64 * q < nw) pc[q] = row[min(lane + 64 * q, nw - 1)];
#pragma unroll
    for (int q = 0; q < WP; q++) {
      const int c = lane + 64 * q;
      if (64 * q < nw && c < nw) {
        ((f32x4 *)s_r)[2 * c] = f32x4{dsh_bf16lo(pc[q][0]), dsh_bf16hi(pc[q][0]), dsh_bf16lo(pc[q][1]),
                                      dsh_bf16hi(pc[q][1])};
        ((f32x4 *)s_r)[2 * c + 1] = f32x4{dsh_bf16lo(pc[q][2]), dsh_bf16hi(pc[q][2]), dsh_bf16lo(pc[q][3]),
                                          dsh_bf16hi(pc[q][3])};
      }
    }
    __syncthreads();  // one wave: x and the row are in LDS
    if (lane == 0) {  // the chain in column order
      float s = 0.0f;
      const f32x4 *w4 = (const f32x4 *)s_r, *x4 = (const f32x4 *)s_x;
#pragma unroll 8
      for (int c = 0; c < nx; c++) {
        const f32x4 w = w4[c], xv = x4[c];
        s = __builtin_fmaf(w[0], xv[0], s);
        s = __builtin_fmaf(w[1], xv[1], s);
        s = __builtin_fmaf(w[2], xv[2], s);
        s = __builtin_fmaf(w[3], xv[3], s);
      }
      vals[j] = s;
    }
    __syncthreads();  // lane 0's reads are done before the next row
  }
}

// (value, index) order of the history scan: larger value first, then lower index; NaN never wins.
__device__ __forceinline__ bool smp_better(float v, int i, float bv, int bi) {
  return v > bv || (v == bv && i < bi);
}

__global__ void __launch_bounds__(1024) k_sample_select(int vocab, float rp, int ngram_n, smp_io io,
                                                        const float *__restrict__ vals, int *__restrict__ full_flag) {
  __shared__ float s_v[16];
  __shared__ int s_i[16];
  const int *hist;
  int n;
  int *tok;
  smp_resolve(io, hist, n, tok);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int best = *tok;
  if (rp > 1.0f && n > 0) {
    float bv = vals[0];
    int in_hist = 0;
    for (int i = threadIdx.x; i < n; i += 1024) in_hist |= hist[i] == best;
    if (__syncthreads_or(in_hist)) bv = smp_penalize(bv, rp);
    float mv = -__builtin_huge_valf();
    int mi = 0x7fffffff;
    for (int i = threadIdx.x; i < n; i += 1024) {
      const int t = hist[i];
      if (t < 0 || t >= vocab || t == best) continue;
      const float v = smp_penalize(vals[1 + i], rp);
      if (v == v && smp_better(v, i, mv, mi)) {
        mv = v;
        mi = i;
      }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const float ov = __shfl_xor(mv, o);
      const int oi = __shfl_xor(mi, o);
      if (smp_better(ov, oi, mv, mi)) {
        mv = ov;
        mi = oi;
      }
    }
    if (lane == 0) {
      s_v[wave] = mv;
      s_i[wave] = mi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      for (int w = 1; w < 16; w++)
        if (smp_better(s_v[w], s_i[w], mv, mi)) {
          mv = s_v[w];
          mi = s_i[w];
        }
      s_i[0] = mi < n && mv > bv ? hist[mi] : best;
    }
    __syncthreads();
    best = s_i[0];
  }
  int full = 0;
  if (ngram_n > 0 && n >= ngram_n - 1) {
    const int p = ngram_n - 1;
    for (int i = threadIdx.x; i <= n - p - 1; i += 1024) full |= smp_bans(hist, n, p, i, best);
  }
  full = __syncthreads_or(full);
  if (threadIdx.x == 0) {
    if (!full) *tok = best;
    *full_flag = full;
  }
}

// Full path, step 1: every logit in ds_bf16_matvec_pub's order (4 lanes per row, as the matvec
// kernel), x staged in LDS.
__global__ void __launch_bounds__(256) k_sample_full_logits(const uint16_t *__restrict__ W, const float *__restrict__ x,
                                                            int H, int vocab, int chunk,
                                                            const int *__restrict__ full_flag, float *__restrict__ lg) {
  __shared__ __attribute__((aligned(16))) float s_x[SMP_MAX_H];
  if (!*full_flag) return;
  for (int i = threadIdx.x; i < H / 4; i += 256) ((f32x4 *)s_x)[i] = ((const f32x4 *)x)[i];
  __syncthreads();
  const int L = threadIdx.x & 3;
  for (int r = blockIdx.x * 64 + (threadIdx.x >> 2); r < vocab; r += gridDim.x * 64) {  // 4-lane groups
    const int path = row_path(r, vocab, chunk, false);
    const float v = avx_row<true>(W + (size_t)r * H, s_x, H, L, path == DSH_ROW_SINGLE, true, 0.0f,
                                  path != DSH_ROW_GROUP4);
    if (L == 0) lg[r] = v;
  }
}

// Full path, step 2: the penalty per history occurrence (the first occurrence of a token applies it
// as many times as the token occurs, in the reference's sequential order), the bans, then the first
// maximum (a NaN logit 0 keeps token 0, as the reference's scan does).
__global__ void __launch_bounds__(1024) k_sample_full_pick(int vocab, float rp, int ngram_n, smp_io io,
                                                           const int *__restrict__ full_flag, float *__restrict__ lg) {
  __shared__ float s_v[16];
  __shared__ int s_i[16];
  if (!*full_flag) return;
  const int *hist;
  int n;
  int *tok;
  smp_resolve(io, hist, n, tok);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (rp > 1.0f) {
    for (int i = threadIdx.x; i < n; i += 1024) {
      const int t = hist[i];
      if (t < 0 || t >= vocab) continue;
      bool first = true;
      for (int j = 0; j < i && first; j++) first = hist[j] != t;
      if (!first) continue;
      int c = 1;
      for (int j = i + 1; j < n; j++) c += hist[j] == t;
      float v = lg[t];
      for (int k = 0; k < c; k++) v = smp_penalize(v, rp);
      lg[t] = v;
    }
    __syncthreads();
  }
  if (ngram_n > 0 && n >= ngram_n - 1) {
    const int p = ngram_n - 1;
    for (int i = threadIdx.x; i <= n - p - 1; i += 1024) {
      bool m = true;
      for (int j = 0; j < p && m; j++) m = hist[i + j] == hist[n - p + j];
      const int b = hist[i + p];
      if (m && b >= 0 && b < vocab) lg[b] = -1e30f;
    }
    __syncthreads();
  }
  float mv = -__builtin_huge_valf();
  int mi = 0x7fffffff;
  for (int i = threadIdx.x; i < vocab; i += 1024) {
    const float v = lg[i];
    if (v == v && smp_better(v, i, mv, mi)) {
      mv = v;
      mi = i;
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float ov = __shfl_xor(mv, o);
    const int oi = __shfl_xor(mi, o);
    if (smp_better(ov, oi, mv, mi)) {
      mv = ov;
      mi = oi;
    }
  }
  if (lane == 0) {
    s_v[wave] = mv;
    s_i[wave] = mi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 16; w++)
      if (smp_better(s_v[w], s_i[w], mv, mi)) {
        mv = s_v[w];
        mi = s_i[w];
      }
    const float l0 = lg[0];
    *tok = (l0 != l0 || mi >= vocab) ? 0 : mi;
  }
}

extern "C" {

int dsh_sample_supported(int H) { return H > 0 && H % 8 == 0 && H <= SMP_MAX_H; }

// After the argmax. Stack form (step != NULL): the history is tokens[0..min(s, hist_len)) and the
// token tokens[s], s = *step - 1. Explicit form: hist[0..hist_len), the token tokens[0]. vals:
// [hist_len + 1] floats; lg: [vocab] floats; flag: one int.
hipError_t dsh_launch_sample(const uint16_t *W, const float *x, int H, int vocab, int nthreads, float rp, int ngram_n,
                             const int *step, int *tokens, const int *hist, int hist_len, float *vals, float *lg,
                             int *flag, hipStream_t s) {
  if (!dsh_sample_supported(H) || vocab <= 0 || hist_len < 0 || (!step && hist_len > 0 && !hist))
    return hipErrorInvalidValue;
  smp_io io{step, tokens, hist, hist_len};
  if (rp > 1.0f) k_sample_dots<<<min(hist_len + 1, 4096), 64, (size_t)H * 8, s>>>(W, x, H, vocab, io, vals);
  k_sample_select<<<1, 1024, 0, s>>>(vocab, rp, ngram_n, io, vals, flag);
  if (ngram_n > 0) {
    const int chunk = dsh_chunk_len(vocab, nthreads);
    // a small grid: on most steps the kernel returns at once
    k_sample_full_logits<<<min((vocab + 63) / 64, 512), 256, 0, s>>>(W, x, H, vocab, chunk, flag, lg);
    k_sample_full_pick<<<1, 1024, 0, s>>>(vocab, rp, ngram_n, io, flag, lg);
  }
  return hipGetLastError();
}

}  // extern "C"
