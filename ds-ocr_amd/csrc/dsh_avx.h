// dsh_avx.h — BF16 row dot products in the reference's AVX-512 order (shared by the kernels).
#pragma once
#include "dsh.h"

// ============================================================================ BF16 rows in AVX-512 order
// Reproduces ds_bf16_matvec_fused_avx / ds_argmax_bf16_range_avx (ds_kernels_avx.c:25-249) bit for
// bit: a row in a 4-row or 2-row group accumulates 32 chains (a0: columns k..k+15, a1: k+16..k+31,
// k += 32) with fused multiply-adds, then 16-column steps on a0 only, then a0+a1 and GCC 11's
// _mm512_reduce_add_ps tree, then (matvec only) "+ bias" (0.0f when absent), then a sequential
// tail over the last in_dim % 16 columns. A row taking the single-row path accumulates 16 chains in
// 16-column steps. Four lanes cooperate on one row: in the 2-accumulator order lane L owns chains
// 8L..8L+7, in the 1-accumulator order chains 4L..4L+3.
// The tail is a fused chain everywhere except in the matvec's 4-row groups, where GCC 11 (-O3,
// AVX-512) vectorizes it across the four rows as rounded products (vmulss) added with vaddps.
//
// Which rows take which path depends on how the reference chunks rows over its CPU threads: see
// row_path().

// Row chunk length of the reference's threaded kernels: the whole range for one thread, else
// ceil(out_dim / nthreads) (ds_kernels.c:806-818, :965-978).
__host__ __device__ __forceinline__ int dsh_chunk_len(int out_dim, int nthreads) {
  return nthreads > 1 ? (out_dim + nthreads - 1) / nthreads : out_dim;
}

enum { DSH_ROW_GROUP4 = 0, DSH_ROW_GROUP2 = 1, DSH_ROW_SINGLE = 2 };

// Path of row r when rows are processed in chunks of "chunk" rows: argmax
// (ds_kernels_avx.c:162-245) does 4-row groups, then single rows; matvec (ds_kernels_avx.c:29-152)
// does 4-row groups, then 2-row groups, then one single row if the count is odd.
__device__ __forceinline__ int row_path(int r, int out_dim, int chunk, bool argmax_mode) {
  if (chunk <= 0) chunk = out_dim;
  int s = (r / chunk) * chunk;
  int len = min(chunk, out_dim - s);
  int off = r - s;
  int n4 = len & ~3;
  if (off < n4) return DSH_ROW_GROUP4;
  if (argmax_mode) return DSH_ROW_SINGLE;
  return off < (len & ~1) ? DSH_ROW_GROUP2 : DSH_ROW_SINGLE;
}

// Loads 8 consecutive bf16 at W[k..k+7] (ALIGNED: one 16-byte load) as floats.
template <bool ALIGNED>
__device__ __forceinline__ void load_bf16x8(const uint16_t *w, float *o) {
  if (ALIGNED) {
    u32x4 v = *(const u32x4 *)w;
#pragma unroll
    for (int d = 0; d < 4; d++) {
      o[2 * d] = dsh_bf16lo(v[d]);
      o[2 * d + 1] = dsh_bf16hi(v[d]);
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; j++) o[j] = dsh_bf16_to_f32(w[j]);
  }
}

// The 2-accumulator reduction: a0 + a1, then _mm512_reduce_add_ps's tree, from the 32 chains held
// as 8 per lane (lane L of the 4-lane group owns chains 8L..8L+7). Lane 0 returns the sum.
__device__ __forceinline__ float avx_tree32(const float *a) {
  // A[i] = a0[i] + a1[i]: lane 0 gets A[0..7] (+lane 2), lane 1 gets A[8..15] (+lane 3).
  float A[8];
#pragma unroll
  for (int j = 0; j < 8; j++) A[j] = a[j] + __shfl_down(a[j], 2, 4);
  // T3[i] = A[8+i] + A[i] (lane 1 holds A[8..15]).
  float T3[8];
#pragma unroll
  for (int j = 0; j < 8; j++) T3[j] = __shfl_down(A[j], 1, 4) + A[j];
  float T6[4];
#pragma unroll
  for (int j = 0; j < 4; j++) T6[j] = T3[4 + j] + T3[j];
  return (T6[0] + T6[2]) + (T6[1] + T6[3]);
}

// With add set (matvec path), "addend" is the bias term added after the tree and before the scalar
// tail (ds_kernels_avx.c:84-87: "+ (bias ? bias[o] : 0.0f)"); the argmax path adds nothing.

// Full row value at lane L (0..3) of its 4-lane group; only L == 0 returns the value.
// x: the input vector (LDS or global). Requires all 4 lanes of the group to call it together.
template <bool ALIGNED>
__device__ float avx_row(const uint16_t *__restrict__ w, const float *x, int in_dim, int L, bool single, bool add,
                        float addend, bool fused_tail) {
  float res;
  if (!single) {
    float a[8];
#pragma unroll
    for (int j = 0; j < 8; j++) a[j] = 0.0f;
    int k = 0;
    for (; k + 32 <= in_dim; k += 32) {
      float wv[8];
      load_bf16x8<ALIGNED>(w + k + 8 * L, wv);
#pragma unroll
      for (int j = 0; j < 8; j++) a[j] = __builtin_fmaf(wv[j], x[k + 8 * L + j], a[j]);
    }
    if (k + 16 <= in_dim) {
      if (L < 2) {  // a0 only: chains 0..15 live in lanes 0 and 1
        float wv[8];
        load_bf16x8<ALIGNED>(w + k + 8 * L, wv);
#pragma unroll
        for (int j = 0; j < 8; j++) a[j] = __builtin_fmaf(wv[j], x[k + 8 * L + j], a[j]);
      }
      k += 16;
    }
    res = avx_tree32(a);
    if (add) res = res + addend;
    if (L == 0) {
      if (fused_tail)
        for (; k < in_dim; k++) res = __builtin_fmaf(dsh_bf16_to_f32(w[k]), x[k], res);
      else
        for (; k < in_dim; k++) res = res + dsh_bf16_to_f32(w[k]) * x[k];
    }
  } else {
    float a[4];
#pragma unroll
    for (int j = 0; j < 4; j++) a[j] = 0.0f;
    int k = 0;
    for (; k + 16 <= in_dim; k += 16) {
#pragma unroll
      for (int j = 0; j < 4; j++) a[j] = __builtin_fmaf(dsh_bf16_to_f32(w[k + 4 * L + j]), x[k + 4 * L + j], a[j]);
    }
    // A[i] = chain i; lanes 0,1 hold A[0..7], lanes 2,3 hold A[8..15].
    float T3[4];  // lane 0: T3[0..3] = A[8..11] + A[0..3]; lane 1: T3[4..7] = A[12..15] + A[4..7]
#pragma unroll
    for (int j = 0; j < 4; j++) T3[j] = __shfl_down(a[j], 2, 4) + a[j];
    float T6[4];  // T6[j] = T3[4+j] + T3[j]
#pragma unroll
    for (int j = 0; j < 4; j++) T6[j] = __shfl_down(T3[j], 1, 4) + T3[j];
    res = (T6[0] + T6[2]) + (T6[1] + T6[3]);
    if (add) res = res + addend;
    if (L == 0)
      for (; k < in_dim; k++) res = __builtin_fmaf(dsh_bf16_to_f32(w[k]), x[k], res);
  }
  return res;
}


// avx_row's 4-row / 2-row group path for in_dim == 32*N32 (no 16-column step and no tail), with the
// lane's 16-byte pieces (columns 32i + 8L .. 32i + 8L + 7) already in registers: wv[i]. x: 16-byte
// aligned. Same chains, order and tree as avx_row.
template <int N32>
__device__ __forceinline__ float avx_row_regs32(const u32x4 *wv, const float *x, int L, bool add, float addend) {
  float a[8];
#pragma unroll
  for (int j = 0; j < 8; j++) a[j] = 0.0f;
#pragma unroll
  for (int i = 0; i < N32; i++) {
    const f32x4 x0 = ((const f32x4 *)x)[8 * i + 2 * L], x1 = ((const f32x4 *)x)[8 * i + 2 * L + 1];
    const float xv[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
#pragma unroll
    for (int d = 0; d < 4; d++) {
      a[2 * d] = __builtin_fmaf(dsh_bf16lo(wv[i][d]), xv[2 * d], a[2 * d]);
      a[2 * d + 1] = __builtin_fmaf(dsh_bf16hi(wv[i][d]), xv[2 * d + 1], a[2 * d + 1]);
    }
  }
  float res = avx_tree32(a);
  if (add) res = res + addend;
  return res;
}
