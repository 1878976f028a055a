// k_dense.hip — the decoder's dense SwiGLU FFN (layer 0 of DeepSeek-OCR; ds_moe_decoder.c:75-105)
// on device-resident BF16 weights, as two kernels on the library stream:
//   gate_up : h[i] = SwiGLU(gate[i]·x, up[i]·x) for the I intermediate units
//             (ds_linear_nobias_bf16 twice + ds_swiglu_direct, ds_moe_decoder.c:89-97)
//   down    : x_out[r] = (residual ? x[r] : 0) + down[r]·h (ds_moe_decoder.c:100), and, when the next
//             layer is a MoE layer with an f32 router, that layer's router partial scores for these
//             rows (the same 8-row partials as k_dec_down writes; scores are linear in x).
// The dots are f32 fused multiply-adds of the exact bf16 values in a lane-parallel order (the
// reference sums each row sequentially per AVX-512 chain; the difference is f32 rounding, ~1e-6).
#include "dsh.h"
#include "k_core.h"

__device__ __forceinline__ const float *dn_at_step(const float *x, const int *step, int stride) {
  return step ? x + (size_t)(*step) * stride : x;
}

// One unit (gate row i, up row i) per 16 lanes: lane sub reads the 16-byte chunks sub + 16m
// (m < CPL, H == 128*CPL) of both rows, all loads issued before the first use; x is staged once per
// block in LDS, its loads issued ahead of the rows. UPB units per block (16*UPB threads).
#ifndef DENSE_UPB
#define DENSE_UPB 16
#endif
template <int CPL, int UPB>
__global__ void __launch_bounds__(16 * UPB) k_dense_gate_up(const uint16_t *__restrict__ Wg, const uint16_t *__restrict__ Wu,
                                                            const float *x_in, const int *__restrict__ step, int stride,
                                                            int I, float *__restrict__ h) {
  __shared__ __attribute__((aligned(16))) float s_x[128 * CPL];
  const float *x = dn_at_step(x_in, step, stride);
  const int lane = threadIdx.x & 63, sub = lane & 15;
  const int unit = blockIdx.x * UPB + (threadIdx.x >> 4);
  const int uc = unit < I ? unit : I - 1;
  const int H = 128 * CPL;
  // x first (in-order returns: the LDS stores wait for x only), then both rows
  constexpr int XP = (32 * CPL + 16 * UPB - 1) / (16 * UPB);  // 16-byte pieces of x per thread
  f32x4 xr[XP];
#pragma unroll
  for (int j = 0; j < XP; j++) xr[j] = ((const f32x4 *)x)[min((int)threadIdx.x + 16 * UPB * j, 32 * CPL - 1)];
  asm volatile("" ::: "memory");
  u32x4 wg[CPL], wu[CPL];
  const uint8_t *gr = (const uint8_t *)Wg + (size_t)uc * H * 2;
  const uint8_t *ur = (const uint8_t *)Wu + (size_t)uc * H * 2;
#pragma unroll
  for (int m = 0; m < CPL; m++) {
    wg[m] = dsh_load_nt(gr + 16 * (sub + 16 * m));
    wu[m] = dsh_load_nt(ur + 16 * (sub + 16 * m));
  }
#pragma unroll
  for (int j = 0; j < XP; j++) {
    const int i = threadIdx.x + 16 * UPB * j;
    if (i < 32 * CPL) ((f32x4 *)s_x)[i] = xr[j];
  }
  __syncthreads();
  float dg = 0.0f, du = 0.0f;
#pragma unroll
  for (int m = 0; m < CPL; m++) {
    const int c = sub + 16 * m;  // 8 elements
    const f32x4 x0 = ((const f32x4 *)s_x)[2 * c], x1 = ((const f32x4 *)s_x)[2 * c + 1];
    const float xv[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
#pragma unroll
    for (int d = 0; d < 4; d++) {
      dg = __builtin_fmaf(dsh_bf16lo(wg[m][d]), xv[2 * d], dg);
      dg = __builtin_fmaf(dsh_bf16hi(wg[m][d]), xv[2 * d + 1], dg);
      du = __builtin_fmaf(dsh_bf16lo(wu[m][d]), xv[2 * d], du);
      du = __builtin_fmaf(dsh_bf16hi(wu[m][d]), xv[2 * d + 1], du);
    }
  }
  dg = dsh_row16_sum(dg);
  du = dsh_row16_sum(du);
  if (sub == 0 && unit < I) h[unit] = dsh_swiglu(dg, du);
}

// 8 output rows per 512-thread block, one per wave: lane l reads the 16-byte chunks l, l+64, ... of
// its row (8 bf16 each; I % 8 == 0) in segments of DENSE_NB chunks per lane; h (staged in LDS once
// per block) and the first segment are loaded together. Wave 0 then adds the residual, writes the rows
// and, given the next MoE layer's transposed f32 router WrT_next ([H][E]), its partial scores over
// these 8 rows (one partial per block, in row order).
#define DENSE_ROWS 8
#define DENSE_NB 16
__global__ void __launch_bounds__(512) k_dense_down(const uint16_t *__restrict__ Wd, const float *__restrict__ h,
                                                    const float *x_in, const int *__restrict__ step, int stride,
                                                    int H, int I, int residual, const float *__restrict__ resid,
                                                    float *__restrict__ x_out,
                                                    const float *__restrict__ WrT_next, int E_next,
                                                    float *__restrict__ partials_next) {
  extern __shared__ __attribute__((aligned(16))) float s_h[];  // I floats
  __shared__ float s_y[DENSE_ROWS];
  const float *x = dn_at_step(x_in, step, stride);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r0 = blockIdx.x * DENSE_ROWS, r = r0 + wave;
  const int nch = I >> 3;  // 16-byte chunks per row
  const uint8_t *row = (const uint8_t *)Wd + (size_t)r * I * 2;
  // h, the router columns and the residual first (in-order returns: the LDS stores wait for those
  // only), then the row's first segment; every load address is clamped in range so that the loads
  // issue back to back without branches
  constexpr int HP = (2 * 16384 / 8 + 511) / 512;  // 16-byte pieces of h per thread at the largest I
  const int nhp = nch * 2;
  f32x4 hr[HP];
#pragma unroll
  for (int j = 0; j < HP; j++)
    if (512 * j < nhp) hr[j] = ((const f32x4 *)h)[min((int)threadIdx.x + 512 * j, nhp - 1)];
  float wr[DENSE_ROWS];
  if (WrT_next && wave == 0 && lane < E_next) {
#pragma unroll
    for (int j = 0; j < DENSE_ROWS; j++) wr[j] = WrT_next[(size_t)(r0 + j) * E_next + lane];
  }
  const float xres = residual && wave == 0 && lane < DENSE_ROWS ? (resid ? resid : x)[r0 + lane] : 0.0f;
  asm volatile("" ::: "memory");
  u32x4 w[DENSE_NB];
  auto load_segment = [&](int c0) {
#pragma unroll
    for (int k = 0; k < DENSE_NB; k++) w[k] = dsh_load_nt(row + 16 * min(c0 + lane + 64 * k, nch - 1));
  };
  load_segment(0);
#pragma unroll
  for (int j = 0; j < HP; j++) {
    const int i = threadIdx.x + 512 * j;
    if (512 * j < nhp && i < nhp) ((f32x4 *)s_h)[i] = hr[j];
  }
  __syncthreads();
  float acc = 0.0f;
  for (int c0 = 0;;) {
#pragma unroll
    for (int k = 0; k < DENSE_NB; k++) {
      const int c = c0 + lane + 64 * k;
      if (c < nch) {
        const f32x4 h0 = ((const f32x4 *)s_h)[2 * c], h1 = ((const f32x4 *)s_h)[2 * c + 1];
        const float hv[8] = {h0[0], h0[1], h0[2], h0[3], h1[0], h1[1], h1[2], h1[3]};
#pragma unroll
        for (int d = 0; d < 4; d++) {
          acc = __builtin_fmaf(dsh_bf16lo(w[k][d]), hv[2 * d], acc);
          acc = __builtin_fmaf(dsh_bf16hi(w[k][d]), hv[2 * d + 1], acc);
        }
      }
    }
    c0 += 64 * DENSE_NB;
    if (c0 >= nch) break;
    load_segment(c0);
  }
  acc = dsh_wave_sum(acc);
  if (lane == 0) s_y[wave] = acc;
  __syncthreads();
  if (wave == 0) {
    float xo = 0.0f;
    if (lane < DENSE_ROWS) {
      xo = residual ? xres + s_y[lane] : s_y[lane];
      x_out[r0 + lane] = xo;
    }
    if (WrT_next) {
      float p = 0.0f;
#pragma unroll
      for (int j = 0; j < DENSE_ROWS; j++) {
        const float xj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(xo), j));
        p = lane < E_next ? __builtin_fmaf(wr[j], xj, p) : 0.0f;
      }
      partials_next[(size_t)blockIdx.x * 64 + lane] = lane < E_next ? p : 0.0f;
    }
  }
}

extern "C" {

int dsh_dense_supported(int H, int I) { return H > 0 && H % 128 == 0 && H / 128 <= 16 && H % DENSE_ROWS == 0 && I > 0 && I % 8 == 0 && I <= 16384; }

hipError_t dsh_launch_dense_gate_up(const uint16_t *Wg, const uint16_t *Wu, const float *x_in, const int *step,
                                    int stride, int H, int I, float *h, hipStream_t s) {
  if (!dsh_dense_supported(H, I)) return hipErrorInvalidValue;
  const int blocks = (I + DENSE_UPB - 1) / DENSE_UPB;
#define DG(N)                                                                                        \
  case N:                                                                                            \
    k_dense_gate_up<N, DENSE_UPB><<<blocks, 16 * DENSE_UPB, 0, s>>>(Wg, Wu, x_in, step, stride, I, h);  \
    break;
  switch (H / 128) {
    DG(1) DG(2) DG(3) DG(4) DG(5) DG(6) DG(7) DG(8) DG(9) DG(10) DG(11) DG(12) DG(13) DG(14) DG(15) DG(16)
    default:
      return hipErrorInvalidValue;
  }
#undef DG
  return hipGetLastError();
}

hipError_t dsh_launch_dense_down(const uint16_t *Wd, const float *h, const float *x_in, const int *step, int stride,
                                 int H, int I, int residual, const float *resid, float *x_out, const float *WrT_next,
                                 int E_next, float *partials_next, hipStream_t s) {
  if (!dsh_dense_supported(H, I) || (WrT_next && (E_next <= 0 || E_next > 64))) return hipErrorInvalidValue;
  k_dense_down<<<H / DENSE_ROWS, 512, (size_t)I * 4, s>>>(Wd, h, x_in, step, stride, H, I, residual, resid, x_out, WrT_next,
                                                          E_next, partials_next);
  return hipGetLastError();
}

}  // extern "C"
