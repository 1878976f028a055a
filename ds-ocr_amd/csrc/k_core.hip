// k_core.hip — gfx950 kernels behind the per-function C API of ds_quantize.h / ds_kernels.h.
//
// Each kernel states the reference arithmetic it reproduces (reference = vislee/ds-ocr C sources).
// Bit-exact kernels reproduce the reference's operation order; the others keep its formula and are
// held to 1e-3 relative error.
#include "dsh.h"
#include "k_core.h"
#include "dsh_avx.h"

// ============================================================================ quantizer
// ds_quantize.c:29-47 (int8_quantize_row) per row, one wave per row.
// min/max keep the reference's first-occurrence semantics under '<' / '>' (so -0 vs +0 ties resolve
// to the lowest column, NaN never enters); scale = (max-min)/255 clamped to 1e-10, inv = 1/scale,
// code = clamp(roundf((w-min)*inv), 0, 255) - 128 with roundf = half away from zero.

struct MinMax {
  float mn, mx;
  int imn, imx;
};

__device__ __forceinline__ void mm_take(MinMax &m, float v, int c) {
  if (v < m.mn) { m.mn = v; m.imn = c; }
  if (v > m.mx) { m.mx = v; m.imx = c; }
}

__device__ __forceinline__ void mm_merge(MinMax &a, float omn, int oimn, float omx, int oimx) {
  if (omn < a.mn || (omn == a.mn && oimn < a.imn)) { a.mn = omn; a.imn = oimn; }
  if (omx > a.mx || (omx == a.mx && oimx < a.imx)) { a.mx = omx; a.imx = oimx; }
}

__device__ __forceinline__ int8_t quant_code(float v, float mn, float inv) {
  float r = roundf((v - mn) * inv);
  int t = (r != r) ? 0 : (int)fminf(fmaxf(r, -1.0f), 256.0f);
  t = t < 0 ? 0 : (t > 255 ? 255 : t);
  return (int8_t)(t - 128);
}

template <typename T>
__device__ __forceinline__ float load_w(const T *p, size_t i);
template <>
__device__ __forceinline__ float load_w<uint16_t>(const uint16_t *p, size_t i) { return dsh_bf16_to_f32(p[i]); }
template <>
__device__ __forceinline__ float load_w<float>(const float *p, size_t i) { return p[i]; }

template <typename T>
__global__ void __launch_bounds__(256) k_quantize_rows(const T *__restrict__ W, int8_t *__restrict__ q,
                                                       float *__restrict__ scale, float *__restrict__ offset,
                                                       int so_stride, int out_dim, int in_dim) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= out_dim) return;
  const T *w = W + (size_t)row * in_dim;
  MinMax m{1e30f, -1e30f, 0x7FFFFFFF, 0x7FFFFFFF};
  for (int c = lane; c < in_dim; c += 64) mm_take(m, load_w(w, c), c);
  for (int o = 32; o >= 1; o >>= 1) {
    float omn = __shfl_xor(m.mn, o), omx = __shfl_xor(m.mx, o);
    int oimn = __shfl_xor(m.imn, o), oimx = __shfl_xor(m.imx, o);
    mm_merge(m, omn, oimn, omx, oimx);
  }
  float range = m.mx - m.mn;
  float sc = range / 255.0f;
  if (sc < 1e-10f) sc = 1e-10f;
  float inv = 1.0f / sc;
  if (lane == 0) {
    scale[(size_t)row * so_stride] = sc;
    offset[(size_t)row * so_stride] = m.mn;
  }
  int8_t *qr = q + (size_t)row * in_dim;
  for (int c = lane; c < in_dim; c += 64) qr[c] = quant_code(load_w(w, c), m.mn, inv);
}

// ds_quantize.c:115-125: out = scale*(q+128) + off, contracted by GCC to one fused multiply-add.
__global__ void k_dequantize(const int8_t *__restrict__ q, const float *__restrict__ scale,
                             const float *__restrict__ offset, float *__restrict__ out, int out_dim, int in_dim) {
  size_t n = (size_t)out_dim * in_dim;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    int r = (int)(i / in_dim);
    out[i] = __builtin_fmaf(scale[r], (float)((int)q[i] + 128), offset[r]);
  }
}

// ============================================================================ INT8 matvec
// y[r - row_start] = scale*Σ(q+128)x + off*Σx (ds_quantize.c:154-170), epilogue fma(scale, dot, off*xs)
// as the reference build evaluates it. Summation order is the GPU's (16-byte chunks, DPP tree).
// LPR lanes per row, each lane walks 16-byte chunks ch = sub, sub+LPR, ...
template <int LPR>
__global__ void __launch_bounds__(256) k_int8_matvec16(const int8_t *__restrict__ q, const float *__restrict__ scale,
                                                       const float *__restrict__ offset, const float *__restrict__ x,
                                                       float *__restrict__ y, int in_dim, int row_start, int nrows) {
  constexpr int RPW = 64 / LPR;
  const int lane = threadIdx.x & 63;
  const int sub = lane % LPR;
  const int rr = blockIdx.x * (4 * RPW) + (threadIdx.x >> 6) * RPW + lane / LPR;
  const bool active = rr < nrows;
  const int r = row_start + (active ? rr : 0);
  const int C = in_dim >> 4;
  const int8_t *qr = q + (size_t)r * in_dim;
  float dot = 0.0f, xs = 0.0f;
  if (active) {
    for (int ch = sub; ch < C; ch += LPR) {
      u32x4 w = dsh_load_nt(qr + 16 * ch);
      float xv[16];
#pragma unroll
      for (int d = 0; d < 4; d++) {
        f32x4 t = dsh_load_f4(x + 16 * ch + 4 * d);
        xv[4 * d] = t[0];
        xv[4 * d + 1] = t[1];
        xv[4 * d + 2] = t[2];
        xv[4 * d + 3] = t[3];
      }
      dot = dsh_dot16_u8(w, xv, dot);
      float s = 0.0f;
#pragma unroll
      for (int k = 0; k < 16; k++) s += xv[k];
      xs += s;
    }
  }
  if (LPR == 16) {
    dot = dsh_row16_sum(dot);
    xs = dsh_row16_sum(xs);
  } else if (LPR == 8) {
    dot = dsh_row8_sum(dot);
    xs = dsh_row8_sum(xs);
  } else if (LPR == 4) {
    dot = dsh_row4_sum(dot);
    xs = dsh_row4_sum(xs);
  }
  if (active && sub == 0) y[rr] = __builtin_fmaf(scale[r], dot, offset[r] * xs);
}

// Any in_dim: one wave per row, byte loads.
__global__ void __launch_bounds__(256) k_int8_matvec_any(const int8_t *__restrict__ q, const float *__restrict__ scale,
                                                         const float *__restrict__ offset, const float *__restrict__ x,
                                                         float *__restrict__ y, int in_dim, int row_start, int nrows) {
  const int lane = threadIdx.x & 63;
  const int rr = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (rr >= nrows) return;
  const int r = row_start + rr;
  const int8_t *qr = q + (size_t)r * in_dim;
  float dot = 0.0f, xs = 0.0f;
  for (int c = lane; c < in_dim; c += 64) {
    float xv = x[c];
    dot = __builtin_fmaf((float)((int)qr[c] + 128), xv, dot);
    xs += xv;
  }
  dot = dsh_wave_sum(dot);
  xs = dsh_wave_sum(xs);
  if (lane == 0) y[rr] = __builtin_fmaf(scale[r], dot, offset[r] * xs);
}

// The reference's per-row order exactly (int8_matvec_generic, ds_quantize.c:154-170): one lane per
// row runs the row's two sequential chains, dot = fma(u_j, x_j, dot) and xs += x_j, then
// y = fma(scale, dot, offset * xs) (GCC's contraction of the epilogue), so y is bit-identical to the
// reference's. x is staged in LDS (dynamic, in_dim floats). ALIGNED: in_dim % 16 == 0 and q 16-byte
// aligned (dsh_row_chain); otherwise one byte at a time.
template <bool ALIGNED>
__global__ void __launch_bounds__(256) k_int8_matvec_chain(const int8_t *__restrict__ q,
                                                           const float *__restrict__ scale,
                                                           const float *__restrict__ offset,
                                                           const float *__restrict__ x, float *__restrict__ y,
                                                           int in_dim, int row_start, int nrows) {
  extern __shared__ __attribute__((aligned(16))) float s_x[];
  for (int i = threadIdx.x; i < in_dim; i += 256) s_x[i] = x[i];
  __syncthreads();
  const int rr = blockIdx.x * 256 + threadIdx.x;
  if (rr >= nrows) return;
  const int r = row_start + rr;
  const int8_t *qr = q + (size_t)r * in_dim;
  float dot, xs = 0.0f;
  if (ALIGNED) {
    dot = dsh_row_chain<true>(qr, s_x, in_dim, xs);
  } else {
    dot = 0.0f;
    for (int c = 0; c < in_dim; c++) {
      dot = __builtin_fmaf((float)((int)qr[c] + 128), s_x[c], dot);
      xs += s_x[c];
    }
  }
  y[rr] = __builtin_fmaf(scale[r], dot, offset[r] * xs);
}

// The same order from LDS: a block stages its MV_RB rows as f32 codes u = q + 128 (coalesced
// 16-byte loads, all in flight at once, converted on the way into LDS; row stride in_dim + 4
// floats) and x; then wave 0 runs one row per lane, dot = fma(u_j, x_j, dot) in order (one LDS-fed
// fused multiply-add per step), while wave 1 forms xs = Σ x_j in order once (it is the same for
// every row: the reference adds it in the same loop, int8_matvec_generic, ds_quantize.c:154-170),
// and y = fma(scale, dot, offset * xs). in_dim % 16 == 0, q 16-byte aligned, in_dim <= MV_MAX_DIM.
#define MV_RB 16           // rows per block
#define MV_PB 7            // 16-byte row chunks per thread (16 rows x 1792 bytes)
#define MV_MAX_DIM 1792

// Staged rows 0 .. na - 1 are rows a0 .., staged rows na .. na + nb - 1 are rows b0 .. of q (stride
// in_dim), as f32 codes into s_rows (stride in_dim + 4 floats); PB * 256 >= (na + nb) * in_dim / 16.
template <int PB>
__device__ __forceinline__ void mv_stage_rows(float *s_rows, const int8_t *q, size_t a0, int na, size_t b0, int nb,
                                              int in_dim) {
  const int t = threadIdx.x, C = in_dim >> 4, n = (na + nb) * C, RS = in_dim + 4;
  u32x4 v[PB];
#pragma unroll
  for (int j = 0; j < PB; j++) {
    const int k = min(t + 256 * j, n - 1), r = k / C, c = k - r * C;
    const size_t g = r < na ? a0 + r : b0 + (r - na);
    v[j] = dsh_load_nt(q + g * in_dim + 16 * c);
  }
  asm volatile("" ::: "memory");
#pragma unroll
  for (int j = 0; j < PB; j++) {
    const int k = t + 256 * j, r = k / C, c = k - r * C;
    if (k < n) {
      float *d = s_rows + (size_t)r * RS + 16 * c;
#pragma unroll
      for (int w = 0; w < 4; w++) {
        float f0, f1, f2, f3;
        dsh_u8x4_to_f32(v[j][w], f0, f1, f2, f3);
        *(f32x4 *)(d + 4 * w) = f32x4{f0, f1, f2, f3};
      }
    }
  }
}

// 16 steps of the chain (4 f32x4 of row values and inputs).
__device__ __forceinline__ float mv_steps16(const f32x4 (&w)[4], const f32x4 (&x)[4], float dot) {
#pragma unroll
  for (int k = 0; k < 4; k++) {
    dot = __builtin_fmaf(w[k][0], x[k][0], dot);
    dot = __builtin_fmaf(w[k][1], x[k][1], dot);
    dot = __builtin_fmaf(w[k][2], x[k][2], dot);
    dot = __builtin_fmaf(w[k][3], x[k][3], dot);
  }
  return dot;
}

__device__ __forceinline__ void mv_load16(const f32x4 *p, f32x4 (&v)[4]) {
#pragma unroll
  for (int k = 0; k < 4; k++) v[k] = p[k];
}

// Wave 0, lane l < nr: the chain of staged row l over s_x; wave 1 lane 0: xs into *s_xs. Returns dot.
// The LDS reads of the next 16 steps go out before the current 16 run (two register sets), so the
// chain waits only for its fused multiply-adds. in_dim % 16 == 0.
__device__ __forceinline__ float mv_chain(const float *s_rows, const float *s_x, float *s_xs, int in_dim, int nr) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, n16 = in_dim >> 4;
  const f32x4 *x4 = (const f32x4 *)s_x;
  float dot = 0.0f;
  if (wave == 0 && lane < nr && (n16 & 3) == 0) {
    // a ring of four register sets: each set's LDS reads go out 48 steps before its fused
    // multiply-adds (the loads past the row's end re-read its last 16 values, unused)
    const f32x4 *r4 = (const f32x4 *)(s_rows + (size_t)lane * (in_dim + 4));
    f32x4 w[4][4], xv[4][4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      mv_load16(r4 + 4 * k, w[k]);
      mv_load16(x4 + 4 * k, xv[k]);
    }
    __builtin_amdgcn_sched_barrier(0);
    for (int i = 0; i < n16; i += 4) {
#pragma unroll
      for (int k = 0; k < 4; k++) {
        dot = mv_steps16(w[k], xv[k], dot);
        const int nx = min(i + k + 4, n16 - 1);
        mv_load16(r4 + 4 * nx, w[k]);
        mv_load16(x4 + 4 * nx, xv[k]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  } else if (wave == 0 && lane < nr) {
    const f32x4 *r4 = (const f32x4 *)(s_rows + (size_t)lane * (in_dim + 4));
    f32x4 wa[4], xa[4], wb[4], xb[4];
    mv_load16(r4, wa);
    mv_load16(x4, xa);
    int i = 0;
    for (; i + 2 <= n16; i += 2) {  // the scheduling barriers keep each set's reads ahead of its use
      mv_load16(r4 + 4 * (i + 1), wb);
      mv_load16(x4 + 4 * (i + 1), xb);
      __builtin_amdgcn_sched_barrier(0);
      dot = mv_steps16(wa, xa, dot);
      const int in = min(i + 2, n16 - 1);
      mv_load16(r4 + 4 * in, wa);
      mv_load16(x4 + 4 * in, xa);
      __builtin_amdgcn_sched_barrier(0);
      dot = mv_steps16(wb, xb, dot);
    }
    if (i < n16) dot = mv_steps16(wa, xa, dot);  // odd n16: the last 16
  } else if (wave == 1 && lane == 0) {
    f32x4 xa[4], xb[4];
    mv_load16(x4, xa);
    float xs = 0.0f;
    int i = 0;
    for (; i + 2 <= n16; i += 2) {
      mv_load16(x4 + 4 * (i + 1), xb);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int k = 0; k < 4; k++) {
        xs += xa[k][0];
        xs += xa[k][1];
        xs += xa[k][2];
        xs += xa[k][3];
      }
      mv_load16(x4 + 4 * min(i + 2, n16 - 1), xa);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int k = 0; k < 4; k++) {
        xs += xb[k][0];
        xs += xb[k][1];
        xs += xb[k][2];
        xs += xb[k][3];
      }
    }
    if (i < n16) {
#pragma unroll
      for (int k = 0; k < 4; k++) {
        xs += xa[k][0];
        xs += xa[k][1];
        xs += xa[k][2];
        xs += xa[k][3];
      }
    }
    *s_xs = xs;
  }
  return dot;
}

__global__ void __launch_bounds__(256) k_int8_mv_rows(const int8_t *__restrict__ q, const float *__restrict__ scale,
                                                      const float *__restrict__ offset, const float *x,
                                                      float *y, int in_dim, int row_start, int nrows) {
  extern __shared__ __attribute__((aligned(16))) float mv_smem[];
  float *s_rows = mv_smem, *s_x = mv_smem + (size_t)MV_RB * (in_dim + 4), *s_xs = s_x + in_dim;
  const int t = threadIdx.x, lane = t & 63, r0 = blockIdx.x * MV_RB, nr = min(MV_RB, nrows - r0);
  f32x4 xv[2];
  const int NX = in_dim >> 2;
#pragma unroll
  for (int j = 0; j < 2; j++) xv[j] = ((const f32x4 *)x)[min(t + 256 * j, NX - 1)];
  mv_stage_rows<MV_PB>(s_rows, q, (size_t)row_start + r0, nr, 0, 0, in_dim);
#pragma unroll
  for (int j = 0; j < 2; j++)
    if (t + 256 * j < NX) *(f32x4 *)(s_x + 4 * (t + 256 * j)) = xv[j];
  __syncthreads();
  const float dot = mv_chain(s_rows, s_x, s_xs, in_dim, nr);
  __syncthreads();
  if (t < nr) {
    const int r = row_start + r0 + lane;
    y[r0 + lane] = __builtin_fmaf(scale[r], dot, offset[r] * *s_xs);
  }
}

// One expert of the per-function path (ds_expert_forward_fused_int4) in one launch. Gate blocks
// (the first nG = I / 8) each take units i0 .. i0 + 7 (i0 = 8 b): gate rows i and up rows I + i (16
// rows, staged as above), h_i = SwiGLU(gate_i, up_i) (bf16sim: inputs and h rounded to bf16, as
// k_split_swiglu), written to hbuf as (epoch << 32 | bits of h_i) with one device-scope 64-bit
// store each. Down blocks (16 output rows each) stage their rows, poll hbuf until every entry
// carries this launch's epoch (the host's running count, different for every launch; a bounded wait
// that sets *derr when it gives up) and run their rows over h (bf16sim: y rounded to bf16). Blocks
// are dispatched in index order, so every gate block is running or done before a down block waits.
// done (optional): down block d stores epoch to done[d] after its output rows (a system-scope
// release store), so a host polling those words knows the outputs are there. xcache: when not NULL, gate block
// 0 also writes x there (device memory) for a later call on the same input.
__global__ void __launch_bounds__(256) k_expert_exact(const int8_t *__restrict__ gq, const float *__restrict__ gs,
                                                      const float *__restrict__ go, const int8_t *__restrict__ dq,
                                                      const float *__restrict__ dsc, const float *__restrict__ dof,
                                                      const float *x, float *xcache,
                                                      unsigned long long *hbuf, float *y, unsigned *done, int H,
                                                      int I, int nG, unsigned epoch, int bf16sim, int spin,
                                                      int *derr) {
  extern __shared__ __attribute__((aligned(16))) float mv_smem[];
  const int t = threadIdx.x, lane = t & 63, b = blockIdx.x;
  const bool gate = b < nG;
  const int in_dim = gate ? H : I;
  float *s_rows = mv_smem, *s_x = mv_smem + (size_t)MV_RB * (in_dim + 4), *s_xs = s_x + in_dim;
  __shared__ float s_g[MV_RB];
  if (gate) {
    const int i0 = 8 * b, NX = H >> 2;
    f32x4 xv[2];
#pragma unroll
    for (int j = 0; j < 2; j++) xv[j] = ((const f32x4 *)x)[min(t + 256 * j, NX - 1)];
    mv_stage_rows<MV_PB>(s_rows, gq, (size_t)i0, 8, (size_t)I + i0, 8, H);  // gate rows 0..7, up rows 8..15
#pragma unroll
    for (int j = 0; j < 2; j++)
      if (t + 256 * j < NX) {
        *(f32x4 *)(s_x + 4 * (t + 256 * j)) = xv[j];
        if (xcache && b == 0) *(f32x4 *)(xcache + 4 * (t + 256 * j)) = xv[j];
      }
    __syncthreads();
    const float dot = mv_chain(s_rows, s_x, s_xs, H, MV_RB);
    __syncthreads();
    if (t < MV_RB) {
      const int r = t < 8 ? i0 + t : I + i0 + (t - 8);
      float v = __builtin_fmaf(gs[r], dot, go[r] * *s_xs);
      if (bf16sim) v = dsh_bf16_round_half_up(v);
      s_g[t] = v;
    }
    __syncthreads();
    if (t < 8) {  // h out, each value with this launch's epoch
      float hv = dsh_swiglu(s_g[t], s_g[8 + t]);
      if (bf16sim) hv = dsh_bf16_round_half_up(hv);
      __hip_atomic_store(hbuf + i0 + t, ((unsigned long long)epoch << 32) | __float_as_uint(hv), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    }
    return;
  }
  const int r0 = (b - nG) * MV_RB, nr = min(MV_RB, H - r0);
  mv_stage_rows<MV_PB>(s_rows, dq, (size_t)r0, nr, 0, 0, I);
  {  // h: poll this thread's entries (I <= 8 * 256 here) until every one of the block's carries the
     // epoch; zeros when the wait gave up (the output is then reported invalid)
    unsigned long long hv[8];
    int ok = 0;
    for (int n = 0; n < spin && !ok; n++) {
      bool mine = true;
#pragma unroll
      for (int j = 0; j < 8; j++) {
        hv[j] = __hip_atomic_load(hbuf + min(t + 256 * j, I - 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        mine &= (unsigned)(hv[j] >> 32) == epoch;
      }
      ok = __syncthreads_and(mine);
      if (!ok) __builtin_amdgcn_s_sleep(2);
    }
    if (!ok && t == 0 && derr) __hip_atomic_store(derr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
#pragma unroll
    for (int j = 0; j < 8; j++)
      if (t + 256 * j < I) s_x[t + 256 * j] = ok ? __uint_as_float((unsigned)hv[j]) : 0.0f;
  }
  __syncthreads();
  const float dot = mv_chain(s_rows, s_x, s_xs, I, nr);
  __syncthreads();
  if (t < 64) {
    if (t < nr) {
      const int r = r0 + lane;
      const float v = __builtin_fmaf(dsc[r], dot, dof[r] * *s_xs);
      y[r] = bf16sim ? dsh_bf16_round_half_up(v) : v;
    }
    if (done && t == 0) __hip_atomic_store(done + (b - nG), epoch, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
  }
}

// ============================================================================ elementwise
// ds_swiglu_direct (ds_kernels.c:1739-1789), fast-exp branch, for seq rows of inter.
__global__ void k_swiglu(float *__restrict__ out, const float *__restrict__ g, const float *__restrict__ u, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    out[i] = dsh_swiglu(g[i], u[i]);
}

__global__ void k_bf16_trunc(float *__restrict__ a, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    a[i] = dsh_bf16_round_half_up(a[i]);
}

// done (optional): after the block's stores, thread 0 stores epoch to done[blockIdx.x] (system scope,
// release), for a host that polls those words instead of synchronising.
__device__ __forceinline__ void block_done(unsigned *done, unsigned epoch) {
  if (!done) return;
  __syncthreads();
  if (threadIdx.x == 0) __hip_atomic_store(done + blockIdx.x, epoch, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

__global__ void k_vec_add(float *__restrict__ dst, const float *__restrict__ a, const float *__restrict__ b, int n,
                          unsigned *done, unsigned epoch) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) dst[i] = a[i] + b[i];
  block_done(done, epoch);
}

// ds_expert_combine (ds_kernels.c:359-371): out = 0; out[i] = fma(w_k, e_k[i], out[i]) for k in order.
// The expert outputs (which may sit in host memory) are loaded 8 at a time, all in flight at once;
// the fused multiply-adds run in k order as before.
__global__ void k_expert_combine(float *__restrict__ out, const float *__restrict__ eo, const float *__restrict__ w,
                                 int top_k, int hidden, unsigned *done, unsigned epoch) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < hidden; i += gridDim.x * blockDim.x) {
    float acc = 0.0f;
    for (int k0 = 0; k0 < top_k; k0 += 8) {
      float v[8], wk[8];
#pragma unroll
      for (int k = 0; k < 8; k++) {
        const int kk = min(k0 + k, top_k - 1);
        v[k] = eo[(size_t)kk * hidden + i];
        wk[k] = w[kk];
      }
#pragma unroll
      for (int k = 0; k < 8; k++)
        if (k0 + k < top_k) acc = __builtin_fmaf(wk[k], v[k], acc);
    }
    out[i] = acc;
  }
  block_done(done, epoch);
}

// Split of a fused [2*inter] gate_up vector + optional truncation + SwiGLU (ds_quantize.c:308-318).
__global__ void k_split_swiglu(float *__restrict__ h, const float *__restrict__ gu, int inter, int bf16sim) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < inter; i += gridDim.x * blockDim.x) {
    float g = gu[i], u = gu[inter + i];
    if (bf16sim) {
      g = dsh_bf16_round_half_up(g);
      u = dsh_bf16_round_half_up(u);
    }
    float v = dsh_swiglu(g, u);
    h[i] = bf16sim ? dsh_bf16_round_half_up(v) : v;
  }
}

// Stages x (in_dim floats) into LDS.
// (x may sit in host memory: 16-byte loads, four per thread in flight at once when aligned.)
__device__ __forceinline__ void stage_x(float *xs, const float *x, int in_dim) {
  if ((in_dim & 3) == 0 && ((uintptr_t)x & 15) == 0) {
    const int n4 = in_dim >> 2, nt = blockDim.x;
    for (int base = 0; base < n4; base += 4 * nt) {
      f32x4 v[4];
#pragma unroll
      for (int j = 0; j < 4; j++) v[j] = ((const f32x4 *)x)[min(base + (int)threadIdx.x + j * nt, n4 - 1)];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int i = base + threadIdx.x + j * nt;
        if (i < n4) ((f32x4 *)xs)[i] = v[j];
      }
    }
  } else {
    for (int i = threadIdx.x; i < in_dim; i += blockDim.x) xs[i] = x[i];
  }
  __syncthreads();
}

// y = W x for rows [0, out_dim), 64 rows per 256-thread block.
template <bool ALIGNED>
__global__ void __launch_bounds__(256) k_bf16_matvec_avx(const uint16_t *__restrict__ W, const float *__restrict__ x,
                                                         const float *__restrict__ bias, float *__restrict__ y,
                                                         int in_dim, int out_dim, int chunk, unsigned *done,
                                                         unsigned epoch) {
  extern __shared__ float xs_lds[];
  stage_x(xs_lds, x, in_dim);
  const int L = threadIdx.x & 3;
  const int r = blockIdx.x * 64 + (threadIdx.x >> 2);
  if (r < out_dim) {  // whole 4-lane groups
    int path = row_path(r, out_dim, chunk, false);
    float v = avx_row<ALIGNED>(W + (size_t)r * in_dim, xs_lds, in_dim, L, path == DSH_ROW_SINGLE, true,
                               bias ? bias[r] : 0.0f, path != DSH_ROW_GROUP4);
    if (L == 0) y[r] = v;
  }
  block_done(done, epoch);
}

// Per-row logits in argmax order plus per-block (max, lowest index) candidates.
template <bool ALIGNED>
__global__ void __launch_bounds__(256) k_argmax_avx(const uint16_t *__restrict__ W, const float *__restrict__ x,
                                                    unsigned long long *__restrict__ cand, float *__restrict__ logits,
                                                    int in_dim, int out_dim, int chunk) {
  extern __shared__ float xs_lds[];
  __shared__ unsigned long long wbest[4];
  stage_x(xs_lds, x, in_dim);
  const int L = threadIdx.x & 3;
  const int r = blockIdx.x * 64 + (threadIdx.x >> 2);
  unsigned long long key = 0ull;
  if (r < out_dim) {
    bool single = row_path(r, out_dim, chunk, true) == DSH_ROW_SINGLE;
    float v = avx_row<ALIGNED>(W + (size_t)r * in_dim, xs_lds, in_dim, L, single, false, 0.0f, true);
    if (L == 0) {
      key = dsh_argmax_key(v, r);
      if (logits) logits[r] = v;
    }
  }
  key = dsh_wave_max_u64(key);
  if ((threadIdx.x & 63) == 0) wbest[threadIdx.x >> 6] = key;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long b = wbest[0];
    for (int i = 1; i < 4; i++) b = dsh_umax64(b, wbest[i]);
    cand[blockIdx.x] = b;
  }
}

// Reduces n candidate keys to one index (and value); 4 candidates per thread loaded together
// (clamped addresses), one round trip per 1024 candidates.
__global__ void __launch_bounds__(256) k_argmax_final(const unsigned long long *__restrict__ cand, int n,
                                                      int *__restrict__ out_idx, float *__restrict__ out_val) {
  __shared__ unsigned long long wbest[4];
  unsigned long long b = 0ull;
  for (int i0 = 0; i0 < n; i0 += 1024) {
    unsigned long long c[4];
#pragma unroll
    for (int j = 0; j < 4; j++) c[j] = cand[min(i0 + (int)threadIdx.x + 256 * j, n - 1)];  // duplicates are harmless
#pragma unroll
    for (int j = 0; j < 4; j++) b = dsh_umax64(b, c[j]);
  }
  b = dsh_wave_max_u64(b);
  if ((threadIdx.x & 63) == 0) wbest[threadIdx.x >> 6] = b;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int i = 1; i < 4; i++) wbest[0] = dsh_umax64(wbest[0], wbest[i]);
    *out_idx = dsh_key_index(wbest[0]);
    if (out_val) *out_val = dsh_key_value(wbest[0]);
  }
}

// ds_bf16_dot_row non-NEON branch (ds_kernels.c:1000-1008): one sequential fused chain.
__global__ void k_bf16_dot_row(const uint16_t *__restrict__ W, const float *__restrict__ x, int in_dim, int row,
                               float *__restrict__ out) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  const uint16_t *w = W + (size_t)row * in_dim;
  float s = 0.0f;
  for (int k = 0; k < in_dim; k++) s = __builtin_fmaf(dsh_bf16_to_f32(w[k]), x[k], s);
  *out = s;
}

// ============================================================================ f32 linear (router)
// ds_linear without BLAS, seq = 1 (ds_kernels.c:639-652) as GCC 11 -O3 compiles it for AVX-512:
// rounded products of the leading multiple of 16 (and then of 8) added in index order, fused tail.
// One lane per output row; bit-exact with that build.
__global__ void k_linear_f32_exact(const float *__restrict__ W, const float *__restrict__ x, float *__restrict__ y,
                                   int in_dim, int out_dim) {
  int o = blockIdx.x * blockDim.x + threadIdx.x;
  if (o >= out_dim) return;
  const float *w = W + (size_t)o * in_dim;
  float s = 0.0f;
  int i = 0;
  if (in_dim >= 16) {
    int m = in_dim & ~15;
    for (; i < m; i++) s = __fadd_rn(s, __fmul_rn(x[i], w[i]));
  }
  if (in_dim - i >= 8) {
    int m = i + 8;
    for (; i < m; i++) s = __fadd_rn(s, __fmul_rn(x[i], w[i]));
  }
  for (; i < in_dim; i++) s = __builtin_fmaf(x[i], w[i], s);
  y[o] = s;
}

// ============================================================================ top-k
// Wave-level routing helpers. All per-expert state lives in lanes (lane e = expert e, n <= 64);
// the selections of round t live in lane t. Sequential sums use readlane in index order so they
// round exactly like the reference's loops.

// ds_moe_top_k (ds_kernels.c:193-243): selection on raw scores (strict '>', lowest index on ties,
// -1e30 floor), then expf softmax over the selected k (renormalised).
__device__ void topk_cfg_wave(const float *scores, int n, int k, int *idx, float *w) {
  const int lane = threadIdx.x & 63;
  float s = lane < n ? scores[lane] : 0.0f;
  bool taken = false;
  int my_sel = 0;
  float my_ss = 0.0f;
  int ns = 0;
  for (int t = 0; t < k; t++) {
    unsigned long long key = (lane < n && !taken) ? dsh_argmax_key(s, lane) : 0ull;
    key = dsh_wave_max_u64(key);
    if (key == 0ull) continue;  // nothing strictly above -1e30 left
    int e = dsh_key_index(key);
    if (lane == e) taken = true;
    if (lane == ns) {
      my_sel = e;
      my_ss = dsh_key_value(key);
    }
    ns++;
  }
  float mx = -1e30f;
  for (int j = 0; j < ns; j++) {
    float v = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_ss), j));
    if (v > mx) mx = v;
  }
  float ev = lane < ns ? dsh_expf_cr(my_ss - mx) : 0.0f;
  float sum = 0.0f;
  for (int j = 0; j < ns; j++) sum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ev), j));
  float inv = 1.0f / sum;
  if (lane < k) {
    idx[lane] = lane < ns ? my_sel : 0;
    w[lane] = lane < ns ? ev * inv : 0.0f;
  }
}

// moe_forward inline routing (ds_moe_decoder.c:157-183): fast-exp softmax over all n experts
// (max, sequential sum, one reciprocal), then top-k of the probabilities with strict '>' and the
// lowest index on ties; weights are the probabilities (no renormalisation). idx = -1 when no
// probability exceeds -1e30 (all-NaN input).
__device__ void topk_decode_wave(const float *scores, int n, int k, int *idx, float *w) {
  const int lane = threadIdx.x & 63;
  float s = lane < n ? scores[lane] : 0.0f;
  // max with '>' from -1e30: NaN never wins; equals the max over non-NaN values floored at -1e30.
  float m = (lane < n && s > -1e30f) ? s : -1e30f;
  m = dsh_wave_max(m);
  float p = lane < n ? dsh_fast_expf(s - m) : 0.0f;
  float sum = 0.0f;
  for (int e = 0; e < n; e++) sum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), e));
  float inv = 1.0f / sum;
  p = p * inv;
  bool taken = false;
  int my_sel = -1;
  float my_w = -1e30f;
  for (int t = 0; t < k; t++) {
    unsigned long long key = (lane < n && !taken) ? dsh_argmax_key(p, lane) : 0ull;
    key = dsh_wave_max_u64(key);
    int e = key == 0ull ? -1 : dsh_key_index(key);
    if (lane == e) taken = true;
    if (lane == t) {
      my_sel = e;
      my_w = key == 0ull ? -1e30f : dsh_key_value(key);
    }
  }
  if (lane < k) {
    idx[lane] = my_sel;
    w[lane] = my_w;
  }
}

__global__ void __launch_bounds__(64) k_topk(const float *__restrict__ scores, int n, int k, int mode,
                                             int *__restrict__ idx, float *__restrict__ w) {
  if (mode == DSH_ROUTE_CFG)
    topk_cfg_wave(scores, n, k, idx, w);
  else
    topk_decode_wave(scores, n, k, idx, w);
}

// ============================================================================ argmax with exclusions
// ds_argmax_matvec_bf16_excluding (ds_kernels.c:1020-1099) on precomputed logits. lg: logits in the
// order of the reference's own chunking (one chunk for 1 thread, ceil(n/T) rows otherwise); lg2
// (single-thread branch only): logits in the order of the 8192-row rescan.
#define EXCL_MAX_CHUNKS 1024

__device__ bool excl_has(const int *excl, int n, int id) {
  for (int i = 0; i < n; i++)
    if (excl[i] == id) return true;
  return false;
}

// Per-chunk argmax as ds_argmax_bf16_range_avx returns it: (best, val) with best = start and
// val = -1e30 when no logit exceeds -1e30. Block-wide; result valid in every thread.
__device__ void chunk_best(const float *lg, int s, int e, int *idx, float *val, unsigned long long *wb) {
  unsigned long long k = 0ull;
  for (int r = s + (int)threadIdx.x; r < e; r += 256) k = dsh_umax64(k, dsh_argmax_key(lg[r], r));
  k = dsh_wave_max_u64(k);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) wb[threadIdx.x >> 6] = k;
  __syncthreads();
  k = dsh_umax64(dsh_umax64(wb[0], wb[1]), dsh_umax64(wb[2], wb[3]));
  *idx = k == 0ull ? s : dsh_key_index(k);
  *val = dsh_key_value(k);
}

__global__ void __launch_bounds__(256) k_argmax_excl_select(const float *__restrict__ lg, const float *__restrict__ lg2,
                                                            int out_dim, int nthreads, const int *__restrict__ excl,
                                                            int n_excl, int *__restrict__ out) {
  __shared__ unsigned long long wb[4];
  __shared__ int cb[EXCL_MAX_CHUNKS];
  __shared__ float cv[EXCL_MAX_CHUNKS];
  const int T = nthreads > 1 ? nthreads : 1;
  const int chunk = dsh_chunk_len(out_dim, nthreads);
  for (int t = 0; t < T; t++) {
    int s = t * chunk, e = min(s + chunk, out_dim);
    int bi;
    float bv;
    if (s < e) {
      chunk_best(lg, s, e, &bi, &bv, wb);
    } else {
      bi = 0;
      bv = -1e30f;
    }
    if (threadIdx.x == 0) {
      cb[t] = bi;
      cv[t] = bv;
    }
  }
  int nres = 0;
  if (T == 1) {
    nres = (out_dim + 8191) / 8192;
    for (int c = 0; c < nres; c++) {
      int s = c * 8192, e = min(s + 8192, out_dim);
      int bi;
      float bv;
      chunk_best(lg2, s, e, &bi, &bv, wb);
      if (threadIdx.x == 0) {
        cb[T + c] = bi;
        cv[T + c] = bv;
      }
    }
  }
  __syncthreads();
  if (threadIdx.x != 0) return;
  int best = cb[0];
  float best_val = cv[0];
  for (int t = 1; t < T; t++)
    if (cv[t] > best_val) {
      best_val = cv[t];
      best = cb[t];
    }
  int result = best;
  if (excl_has(excl, n_excl, best)) {
    if (T == 1) {
      int sb = 0;
      float sv = -1e30f;
      for (int c = 0; c < nres; c++) {
        if (excl_has(excl, n_excl, cb[1 + c])) continue;
        if (cv[1 + c] > sv) {
          sv = cv[1 + c];
          sb = cb[1 + c];
        }
      }
      result = sb;
    } else {
      bool found = false;
      int sb = -1;
      float sv = -1e30f;
      for (int t = 0; t < T; t++) {
        if (excl_has(excl, n_excl, cb[t])) continue;
        if (!found || cv[t] > sv) {
          sv = cv[t];
          sb = cb[t];
          found = true;
        }
      }
      if (found) result = sb;
    }
  }
  *out = result;
}

// ============================================================================ quantization RMS
// ds_quantize.c:127-144: Σ(w - deq)^2 and Σ w^2 accumulated in double (deq as ds_int4_dequantize_f32).
__global__ void __launch_bounds__(256) k_quant_rms(const int8_t *__restrict__ q, const float *__restrict__ scale,
                                                   const float *__restrict__ offset, const uint16_t *__restrict__ W,
                                                   int out_dim, int in_dim, double *__restrict__ partial) {
  __shared__ double sa[256], sb[256];
  size_t n = (size_t)out_dim * in_dim;
  double a = 0.0, b = 0.0;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
    int r = (int)(i / in_dim);
    float deq = __builtin_fmaf(scale[r], (float)((int)q[i] + 128), offset[r]);
    float orig = dsh_bf16_to_f32(W[i]);
    float d = orig - deq;
    a += (double)(d * d);
    b += (double)(orig * orig);
  }
  sa[threadIdx.x] = a;
  sb[threadIdx.x] = b;
  __syncthreads();
  for (int o = 128; o >= 1; o >>= 1) {
    if (threadIdx.x < o) {
      sa[threadIdx.x] += sa[threadIdx.x + o];
      sb[threadIdx.x] += sb[threadIdx.x + o];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    partial[2 * blockIdx.x] = sa[0];
    partial[2 * blockIdx.x + 1] = sb[0];
  }
}

__global__ void __launch_bounds__(256) k_sum_pairs_f64(const double *__restrict__ partial, int n,
                                                       double *__restrict__ out) {
  __shared__ double sa[256], sb[256];
  double a = 0.0, b = 0.0;
  for (int i = threadIdx.x; i < n; i += 256) {
    a += partial[2 * i];
    b += partial[2 * i + 1];
  }
  sa[threadIdx.x] = a;
  sb[threadIdx.x] = b;
  __syncthreads();
  for (int o = 128; o >= 1; o >>= 1) {
    if (threadIdx.x < o) {
      sa[threadIdx.x] += sa[threadIdx.x + o];
      sb[threadIdx.x] += sb[threadIdx.x + o];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    out[0] = sa[0];
    out[1] = sb[0];
  }
}

// ============================================================================ f32 GEMM, bf16 weights
// Y[M,N] = X[M,K] * W[N,K]^T with W widened from bf16 (ds_linear_nobias_bf16, seq_len > 1: the
// reference converts W to f32 and calls sgemm, ds_kernels.c:917-927). 64x64 tile, 16-wide K steps.
__global__ void __launch_bounds__(256) k_gemm_bf16w(const float *__restrict__ X, const uint16_t *__restrict__ W,
                                                    float *__restrict__ Y, int M, int K, int N) {
  __shared__ float xs[16][65], ws[16][65];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
  float acc[4][4] = {};
  for (int k0 = 0; k0 < K; k0 += 16) {
    for (int i = threadIdx.x; i < 16 * 64; i += 256) {
      int kk = i & 15, rr = i >> 4;
      int m = m0 + rr, nn = n0 + rr, k = k0 + kk;
      xs[kk][rr] = (m < M && k < K) ? X[(size_t)m * K + k] : 0.0f;
      ws[kk][rr] = (nn < N && k < K) ? dsh_bf16_to_f32(W[(size_t)nn * K + k]) : 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; kk++) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        a[i] = xs[kk][ty * 4 + i];
        b[i] = ws[kk][tx * 4 + i];
      }
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = __builtin_fmaf(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) {
      int m = m0 + ty * 4 + i, nn = n0 + tx * 4 + j;
      if (m < M && nn < N) Y[(size_t)m * N + nn] = acc[i][j];
    }
}

// ============================================================================ synthetic data
// Counter-based: pair p draws two SplitMix64 outputs of (seed, p) and maps them through Box–Muller.
__device__ __forceinline__ uint64_t dsh_splitmix(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

template <typename T>
__device__ __forceinline__ T to_out(float v);
template <>
__device__ __forceinline__ float to_out<float>(float v) { return v; }
template <>
__device__ __forceinline__ uint16_t to_out<uint16_t>(float v) {
  uint32_t u = __float_as_uint(v);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

template <typename T>
__global__ void k_fill_normal(T *__restrict__ dst, size_t n, uint64_t seed, float mean, float std_) {
  size_t pairs = (n + 1) / 2;
  for (size_t p = (size_t)blockIdx.x * blockDim.x + threadIdx.x; p < pairs; p += (size_t)gridDim.x * blockDim.x) {
    uint64_t a = dsh_splitmix(seed * 0x632BE59BD9B4E019ull + 2 * p);
    uint64_t b = dsh_splitmix(seed * 0x632BE59BD9B4E019ull + 2 * p + 1);
    float u1 = ((float)(a >> 40) + 1.0f) * (1.0f / 16777216.0f);
    float u2 = (float)(b >> 40) * (1.0f / 16777216.0f);
    float r = sqrtf(-2.0f * logf(u1));
    float sn, cs;
    sincosf(6.283185307f * u2, &sn, &cs);
    dst[2 * p] = to_out<T>(mean + std_ * r * cs);
    if (2 * p + 1 < n) dst[2 * p + 1] = to_out<T>(mean + std_ * r * sn);
  }
}

// Streaming-read reference for the rooflines: every 16-byte piece of src read once with
// nontemporal loads, 4 per lane in flight (the fastest of the depths and grids measured on MI355X),
// folded into one word that is stored only on an impossible value (so the loads are not removed).
__global__ void __launch_bounds__(256) k_stream_read(const u32x4 *__restrict__ src, size_t n16,
                                                     unsigned *__restrict__ sink) {
  unsigned acc = 0;
  const size_t stride = (size_t)gridDim.x * 256 * 4;
  for (size_t base = (size_t)blockIdx.x * 256 * 4 + threadIdx.x; base < n16; base += stride) {
    u32x4 v[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const size_t i = base + (size_t)k * 256;
      v[k] = i < n16 ? dsh_load_nt(src + i) : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int k = 0; k < 4; k++) acc ^= v[k][0] ^ v[k][1] ^ v[k][2] ^ v[k][3];
  }
  if (acc == 0x9E3779B9u && sink) sink[blockIdx.x] = acc;
}

// ============================================================================ launchers

#define LAUNCH_CHECK() (hipGetLastError())

extern "C" {

hipError_t dsh_launch_stream_read(const void *src, size_t bytes, unsigned *sink, hipStream_t s) {
  k_stream_read<<<1024, 256, 0, s>>>((const u32x4 *)src, bytes / 16, sink);
  return LAUNCH_CHECK();
}

hipError_t dsh_launch_quantize_bf16(const uint16_t *W, int8_t *q, float *scale, float *offset, int out_dim, int in_dim,
                                    hipStream_t s) {
  k_quantize_rows<uint16_t><<<(out_dim + 3) / 4, 256, 0, s>>>(W, q, scale, offset, 1, out_dim, in_dim);
  return LAUNCH_CHECK();
}

hipError_t dsh_launch_quantize_f32(const float *W, int8_t *q, float *scale, float *offset, int out_dim, int in_dim,
                                   hipStream_t s) {
  k_quantize_rows<float><<<(out_dim + 3) / 4, 256, 0, s>>>(W, q, scale, offset, 1, out_dim, in_dim);
  return LAUNCH_CHECK();
}

hipError_t dsh_launch_quantize_bf16_so(const uint16_t *W, int8_t *q, float *so, int out_dim, int in_dim, hipStream_t s) {
  k_quantize_rows<uint16_t><<<(out_dim + 3) / 4, 256, 0, s>>>(W, q, so, so + 1, 2, out_dim, in_dim);
  return LAUNCH_CHECK();
}

hipError_t dsh_launch_quant_rms(const int8_t *q, const float *scale, const float *offset, const uint16_t *W,
                                int out_dim, int in_dim, double *work, hipStream_t s) {
  k_quant_rms<<<1024, 256, 0, s>>>(q, scale, offset, W, out_dim, in_dim, work + 2);
  hipError_t e = LAUNCH_CHECK();
  if (e != hipSuccess) return e;
  k_sum_pairs_f64<<<1, 256, 0, s>>>(work + 2, 1024, work);
  return LAUNCH_CHECK();
}

hipError_t dsh_launch_gemm_bf16w(const float *X, const uint16_t *W, float *Y, int M, int K, int N, hipStream_t s) {
  dim3 grid((N + 63) / 64, (M + 63) / 64);
  k_gemm_bf16w<<<grid, 256, 0, s>>>(X, W, Y, M, K, N);
  return LAUNCH_CHECK();
}

hipError_t dsh_launch_fill_normal_bf16(uint16_t *dst, size_t n, uint64_t seed, float std_, hipStream_t s) {
  size_t pairs = (n + 1) / 2;
  int blocks = (int)((pairs + 255) / 256);
  if (blocks > 65536) blocks = 65536;
  k_fill_normal<uint16_t><<<blocks, 256, 0, s>>>(dst, n, seed, 0.0f, std_);
  return LAUNCH_CHECK();
}

hipError_t dsh_launch_fill_normal_f32(float *dst, size_t n, uint64_t seed, float mean, float std_, hipStream_t s) {
  size_t pairs = (n + 1) / 2;
  int blocks = (int)((pairs + 255) / 256);
  if (blocks > 65536) blocks = 65536;
  k_fill_normal<float><<<blocks, 256, 0, s>>>(dst, n, seed, mean, std_);
  return LAUNCH_CHECK();
}

hipError_t dsh_launch_dequantize(const int8_t *q, const float *scale, const float *offset, float *out, int out_dim,
                                 int in_dim, hipStream_t s) {
  size_t n = (size_t)out_dim * in_dim;
  int blocks = (int)((n + 255) / 256);
  if (blocks > 8192) blocks = 8192;
  k_dequantize<<<blocks, 256, 0, s>>>(q, scale, offset, out, out_dim, in_dim);
  return LAUNCH_CHECK();
}

static size_t mv_lds_host(int in_dim) { return ((size_t)MV_RB * (in_dim + 4) + (size_t)in_dim + 4) * 4; }

hipError_t dsh_launch_int8_matvec_exact(const int8_t *q, const float *scale, const float *offset, const float *x,
                                        float *y, int in_dim, int row_start, int nrows, hipStream_t s) {
  if (nrows <= 0) return hipSuccess;
  const size_t lds = (size_t)in_dim * sizeof(float);
  if (in_dim <= 0 || lds > 64 * 1024) return hipErrorInvalidValue;
  const bool aligned = in_dim % 16 == 0 && ((uintptr_t)q & 15) == 0;
  if (aligned && in_dim <= MV_MAX_DIM && ((uintptr_t)x & 15) == 0) {  // rows staged in LDS
    k_int8_mv_rows<<<(nrows + MV_RB - 1) / MV_RB, 256, mv_lds_host(in_dim), s>>>(q, scale, offset, x, y, in_dim,
                                                                               row_start, nrows);
    return LAUNCH_CHECK();
  }
  if (aligned)
    k_int8_matvec_chain<true><<<(nrows + 255) / 256, 256, lds, s>>>(q, scale, offset, x, y, in_dim, row_start, nrows);
  else
    k_int8_matvec_chain<false><<<(nrows + 255) / 256, 256, lds, s>>>(q, scale, offset, x, y, in_dim, row_start, nrows);
  return LAUNCH_CHECK();
}

hipError_t dsh_launch_int8_matvec(const int8_t *q, const float *scale, const float *offset, const float *x, float *y,
                                  int in_dim, int row_start, int nrows, hipStream_t s) {
  if (nrows <= 0) return hipSuccess;
  int C = in_dim / 16;
  bool aligned = (in_dim % 16 == 0) && (((uintptr_t)q & 15) == 0) && (((uintptr_t)x & 15) == 0);
  if (aligned && C >= 64) {
    k_int8_matvec16<16><<<(nrows + 15) / 16, 256, 0, s>>>(q, scale, offset, x, y, in_dim, row_start, nrows);
  } else if (aligned && C >= 16) {
    k_int8_matvec16<8><<<(nrows + 31) / 32, 256, 0, s>>>(q, scale, offset, x, y, in_dim, row_start, nrows);
  } else if (aligned) {
    k_int8_matvec16<4><<<(nrows + 63) / 64, 256, 0, s>>>(q, scale, offset, x, y, in_dim, row_start, nrows);
  } else {
    k_int8_matvec_any<<<(nrows + 3) / 4, 256, 0, s>>>(q, scale, offset, x, y, in_dim, row_start, nrows);
  }
  return LAUNCH_CHECK();
}

hipError_t dsh_launch_swiglu(float *out, const float *g, const float *u, size_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  int blocks = (int)((n + 255) / 256);
  if (blocks > 4096) blocks = 4096;
  k_swiglu<<<blocks, 256, 0, s>>>(out, g, u, n);
  return LAUNCH_CHECK();
}

hipError_t dsh_launch_bf16_trunc(float *a, size_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  int blocks = (int)((n + 255) / 256);
  if (blocks > 4096) blocks = 4096;
  k_bf16_trunc<<<blocks, 256, 0, s>>>(a, n);
  return LAUNCH_CHECK();
}

int dsh_vec_add_blocks(int n) { return n <= 0 ? 0 : ((n + 255) / 256 > 4096 ? 4096 : (n + 255) / 256); }

hipError_t dsh_launch_vec_add(float *dst, const float *a, const float *b, int n, hipStream_t s) {
  return dsh_launch_vec_add_done(dst, a, b, n, NULL, 0, s);
}

hipError_t dsh_launch_vec_add_done(float *dst, const float *a, const float *b, int n, unsigned *done, unsigned epoch,
                                   hipStream_t s) {
  if (n <= 0) return hipSuccess;
  k_vec_add<<<dsh_vec_add_blocks(n), 256, 0, s>>>(dst, a, b, n, done, epoch);
  return LAUNCH_CHECK();
}

int dsh_expert_combine_blocks(int hidden) { return hidden <= 0 ? 0 : (hidden + 255) / 256; }

hipError_t dsh_launch_expert_combine(float *out, const float *eo, const float *w, int top_k, int hidden,
                                     hipStream_t s) {
  return dsh_launch_expert_combine_done(out, eo, w, top_k, hidden, NULL, 0, s);
}

hipError_t dsh_launch_expert_combine_done(float *out, const float *eo, const float *w, int top_k, int hidden,
                                          unsigned *done, unsigned epoch, hipStream_t s) {
  if (hidden <= 0) return hipSuccess;
  k_expert_combine<<<dsh_expert_combine_blocks(hidden), 256, 0, s>>>(out, eo, w, top_k, hidden, done, epoch);
  return LAUNCH_CHECK();
}

int dsh_expert_exact_down_blocks(int H) { return (H + MV_RB - 1) / MV_RB; }

int dsh_expert_exact_blocks(int H, int I) {
  if (H <= 0 || I <= 0 || H % 16 || I % 16 || H > MV_MAX_DIM || I > MV_MAX_DIM) return 0;
  return I / 8 + (H + MV_RB - 1) / MV_RB;
}

hipError_t dsh_launch_expert_exact(const int8_t *gq, const float *gs, const float *go, const int8_t *dq, const float *dsc,
                                   const float *dof, const float *x, float *xcache, unsigned long long *hbuf, float *y,
                                   unsigned *done, int H, int I, unsigned epoch, int bf16sim, int spin, int *derr,
                                   hipStream_t s) {
  const int nb = dsh_expert_exact_blocks(H, I), nG = I / 8;
  if (!nb || ((uintptr_t)gq & 15) || ((uintptr_t)dq & 15) || ((uintptr_t)x & 15) || ((uintptr_t)xcache & 15) ||
      spin <= 0)
    return hipErrorInvalidValue;
  const size_t lds = mv_lds_host(H > I ? H : I);
  k_expert_exact<<<nb, 256, lds, s>>>(gq, gs, go, dq, dsc, dof, x, xcache, hbuf, y, done, H, I, nG, epoch, bf16sim,
                                      spin, derr);
  return LAUNCH_CHECK();
}

hipError_t dsh_launch_split_swiglu(float *h, const float *gu, int inter, int bf16sim, hipStream_t s) {
  if (inter <= 0) return hipSuccess;
  k_split_swiglu<<<(inter + 255) / 256, 256, 0, s>>>(h, gu, inter, bf16sim);
  return LAUNCH_CHECK();
}

static bool bf16_aligned(const uint16_t *W, int in_dim) { return (in_dim % 8 == 0) && (((uintptr_t)W & 15) == 0); }

hipError_t dsh_launch_bf16_matvec_avx(const uint16_t *W, const float *x, const float *bias, float *y, int in_dim,
                                      int out_dim, int nthreads, hipStream_t s) {
  return dsh_launch_bf16_matvec_avx_done(W, x, bias, y, in_dim, out_dim, nthreads, NULL, 0, s);
}

int dsh_bf16_matvec_avx_blocks(int out_dim) { return out_dim <= 0 ? 0 : (out_dim + 63) / 64; }

hipError_t dsh_launch_bf16_matvec_avx_done(const uint16_t *W, const float *x, const float *bias, float *y, int in_dim,
                                           int out_dim, int nthreads, unsigned *done, unsigned epoch, hipStream_t s) {
  if (out_dim <= 0) return hipSuccess;
  size_t lds = (size_t)in_dim * sizeof(float);
  if (lds > 64 * 1024) return hipErrorInvalidValue;
  int blocks = (out_dim + 63) / 64;
  int chunk = dsh_chunk_len(out_dim, nthreads);
  if (bf16_aligned(W, in_dim))
    k_bf16_matvec_avx<true><<<blocks, 256, lds, s>>>(W, x, bias, y, in_dim, out_dim, chunk, done, epoch);
  else
    k_bf16_matvec_avx<false><<<blocks, 256, lds, s>>>(W, x, bias, y, in_dim, out_dim, chunk, done, epoch);
  return LAUNCH_CHECK();
}

int dsh_argmax_avx_blocks(int out_dim) { return (out_dim + 63) / 64; }

hipError_t dsh_launch_argmax_avx_partial(const uint16_t *W, const float *x, unsigned long long *cand, float *logits,
                                         int in_dim, int out_dim, int chunk, hipStream_t s) {
  if (out_dim <= 0) return hipSuccess;
  size_t lds = (size_t)in_dim * sizeof(float);
  if (lds > 64 * 1024) return hipErrorInvalidValue;
  int blocks = dsh_argmax_avx_blocks(out_dim);
  if (bf16_aligned(W, in_dim))
    k_argmax_avx<true><<<blocks, 256, lds, s>>>(W, x, cand, logits, in_dim, out_dim, chunk);
  else
    k_argmax_avx<false><<<blocks, 256, lds, s>>>(W, x, cand, logits, in_dim, out_dim, chunk);
  return LAUNCH_CHECK();
}

hipError_t dsh_launch_argmax_avx(const uint16_t *W, const float *x, unsigned long long *cand, float *logits,
                                 int in_dim, int out_dim, int nthreads, int *out_idx, float *out_val, hipStream_t s) {
  if (out_dim <= 0) return hipSuccess;
  if (!logits && dsh_dec_lm_eligible(W, in_dim, out_dim, nthreads)) {
    // full-line streaming kernel (k_dec.hip); its candidate count is at most dsh_argmax_avx_blocks
    hipError_t e = dsh_launch_dec_lm_argmax(W, x, in_dim, out_dim, cand, s);
    if (e != hipSuccess) return e;
    k_argmax_final<<<1, 256, 0, s>>>(cand, dsh_dec_lm_blocks(out_dim), out_idx, out_val);
    return LAUNCH_CHECK();
  }
  hipError_t e = dsh_launch_argmax_avx_partial(W, x, cand, logits, in_dim, out_dim, dsh_chunk_len(out_dim, nthreads), s);
  if (e != hipSuccess) return e;
  k_argmax_final<<<1, 256, 0, s>>>(cand, dsh_argmax_avx_blocks(out_dim), out_idx, out_val);
  return LAUNCH_CHECK();
}

hipError_t dsh_launch_argmax_excluding(const uint16_t *W, const float *x, unsigned long long *cand, float *lg,
                                       float *lg2, int in_dim, int out_dim, int nthreads, const int *excl, int n_excl,
                                       int *out_idx, hipStream_t s) {
  if (out_dim <= 0) return hipSuccess;
  // chunk slots: up to 16 thread chunks, then (one thread) the rescan's 8192-row chunks after slot 0
  if (nthreads > 16 || 1 + (out_dim + 8191) / 8192 > EXCL_MAX_CHUNKS) return hipErrorInvalidValue;
  int chunk = dsh_chunk_len(out_dim, nthreads);
  hipError_t e = dsh_launch_argmax_avx_partial(W, x, cand, lg, in_dim, out_dim, chunk, s);
  if (e == hipSuccess && nthreads <= 1) e = dsh_launch_argmax_avx_partial(W, x, cand, lg2, in_dim, out_dim, 8192, s);
  if (e != hipSuccess) return e;
  k_argmax_excl_select<<<1, 256, 0, s>>>(lg, lg2, out_dim, nthreads, excl, n_excl, out_idx);
  return LAUNCH_CHECK();
}

hipError_t dsh_launch_bf16_dot_row(const uint16_t *W, const float *x, int in_dim, int row, float *out, hipStream_t s) {
  k_bf16_dot_row<<<1, 64, 0, s>>>(W, x, in_dim, row, out);
  return LAUNCH_CHECK();
}

hipError_t dsh_launch_linear_f32_exact(const float *W, const float *x, float *y, int in_dim, int out_dim,
                                       hipStream_t s) {
  if (out_dim <= 0) return hipSuccess;
  k_linear_f32_exact<<<(out_dim + 63) / 64, 64, 0, s>>>(W, x, y, in_dim, out_dim);
  return LAUNCH_CHECK();
}

hipError_t dsh_launch_topk(const float *scores, int n, int k, int mode, int *idx, float *w, hipStream_t s) {
  if (n <= 0 || n > 64 || k <= 0 || k > n) return hipErrorInvalidValue;
  k_topk<<<1, 64, 0, s>>>(scores, n, k, mode, idx, w);
  return LAUNCH_CHECK();
}

}  // extern "C"

// ============================================================================ static scratch
// The candidate keys of the allocation-free argmax entry point live in this file-scope device
// array (one (value, index) key per 64-row block of the matrix), so that entry point needs no
// hipMalloc. Each GPU holds its own copy for the life of the process. In host code `scratch` is
// only a stand-in for the symbol: its device address, per device, comes from hipGetSymbolAddress
// at set-up (dsh_static_scratch_init, with that device current) and only that address is passed to
// kernels. Every block of the argmax writes its key before the final kernel reads them, so nothing
// has to start at zero; calls that overlap on one device share the array and race.
static __device__ __align__(256) unsigned long long scratch[DSH_STATIC_CAND];

#define DSH_MAX_DEVICES 64
static unsigned long long *g_scratch_dev[DSH_MAX_DEVICES];

extern "C" {

int dsh_static_scratch_init(void) {
  int d = -1;
  if (hipGetDevice(&d) != hipSuccess || d < 0 || d >= DSH_MAX_DEVICES) return -1;
  if (g_scratch_dev[d]) return 0;
  void *p = nullptr;
  if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return -1;
  g_scratch_dev[d] = (unsigned long long *)p;
  return 0;
}

unsigned long long *dsh_static_scratch(void) {
  int d = -1;
  if (hipGetDevice(&d) != hipSuccess || d < 0 || d >= DSH_MAX_DEVICES) return nullptr;
  return g_scratch_dev[d];
}

}  // extern "C"
