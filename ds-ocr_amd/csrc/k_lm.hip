// k_lm.hip — the decode step's LM-head argmax over an int8 copy of the head, with the same result
// as the one-pass kernel (k_dec_lm_argmax, the reference's 4-row-group AVX-512 order,
// ds_kernels_avx.c:162-245).
//
// The argmax needs every row's logit only to decide which row is largest. A per-row int8 copy of
// the bf16 head (q = rint(w / s), s = max|w| / 127) gives an approximate logit A_r for half the
// bytes, and a rigorous bound |L_r - A_r| <= B_r on the logit L_r the exact order computes:
//   L_r - A_r = (L_r - Σ w x)                    rounding of the exact order: <= γ_n ||w||_2 ||x||_2
//             + Σ (w - s q) x                     quantization:  <= ||w - s q||_2 ||x||_2
//             + s Σ q (x - x~)                    the input on a 2^(e-14) grid: <= s ||q||_1 2^(e-15)
//             + (s Σ q x~ - A_r)                  one rounding of A_r: <= 2^-22 |A_r| (generous)
// with |x| < 2^e and γ_n = n u / (1 - n u), u = 2^-24, n = H/32 + 5: in the exact order each
// product is rounded by its own fused multiply-add and by every later one of its chain (H/32 per
// chain, H % 32 == 0), then by a0 + a1 and by the 4 levels of the 16-lane reduction tree, so no
// term passes through more than H/32 + 5 roundings and |L_r - Σ w x| <= γ_n Σ|w x| (Cauchy-Schwarz
// for the last step). Per row, α_r = γ_n ||w||_2 + ||w - s q||_2 and β_r = s ||q||_1 are computed
// once (f64, rounded up to f32); per step B_r = α_r ||x||_2 + β_r 2^(e-15) + 2^-22 |A_r|.
// k_lm_q8_argmax streams the int8 rows of its block of 512, computes A_r from exact integer dot
// products of the codes with the input's two 8-bit limbs, and takes LB = the largest A_r - B_r
// over the block. The row holding the block's largest exact logit has A_r + B_r >= its logit >= LB,
// and so does every row tied with it, while a row with A_r + B_r < LB has a logit below another
// row's of the block. So the block recomputes only its rows with A_r + B_r >= LB in the exact order
// and writes the block's (max, lowest index) key, the one-pass kernel's key for its rows; the
// final reduction is unchanged. NaN or infinite bounds make a row a candidate (the test is
// !(A_r + B_r < LB)), so such inputs fall back to the exact computation of every row they touch.
#include "dsh.h"
#include "k_core.h"

#define LM_Q8_ROWS 512  // rows per block: 8 waves, one block per CU

namespace {

template <int CTRL>
__device__ __forceinline__ int lm_dppi(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}

// exact integer sum over each aligned group of 16 lanes (every lane of the group gets it)
__device__ __forceinline__ int lm_row16_sum_i(int v) {
  v += lm_dppi<0xB1>(v);   // quad_perm [1,0,3,2]
  v += lm_dppi<0x4E>(v);   // quad_perm [2,3,0,1]
  v += lm_dppi<0x141>(v);  // row_half_mirror
  v += lm_dppi<0x140>(v);  // row_mirror
  return v;
}

__device__ __forceinline__ double lm_wave_max_d(double v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmax(v, __shfl_xor(v, o));
  return v;
}
__device__ __forceinline__ double lm_wave_sum_d(double v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// the next float above f (f finite)
__device__ __forceinline__ float lm_next_up(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) == 0u) return __uint_as_float(1u);  // ±0: the smallest positive subnormal
  return __uint_as_float((int32_t)u >= 0 ? u + 1u : u - 1u);
}

// the smallest float >= d (d finite or infinite, not NaN)
__device__ __forceinline__ float lm_f32_up(double d) {
  float f = (float)d;
  if ((double)f < d) f = lm_next_up(f);
  return f;
}

// γ_n for the exact order's roundings at hidden size H (n = H/32 + 5, the count derived above)
__host__ __device__ constexpr double lm_gamma(int H) {
  return (H / 32 + 5) * 0x1p-24 / (1.0 - (H / 32 + 5) * 0x1p-24);
}

}  // namespace

// One wave per row: q (int8, [vocab][H]) and sab[3 r .. 3 r + 2] = (s, α_r, β_r). A row with a
// non-finite weight gets α = β = +inf (always a candidate).
__global__ void __launch_bounds__(256) k_lm_q8_build(const uint16_t *__restrict__ W, int H, int vocab,
                                                     int8_t *__restrict__ q, float *__restrict__ sab) {
  const int lane = threadIdx.x & 63, row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= vocab) return;  // wave-uniform
  const uint16_t *w = W + (size_t)row * H;
  float amax = 0.0f;
  bool bad = false;
  for (int j = lane; j < H; j += 64) {
    const float v = __uint_as_float((uint32_t)w[j] << 16);
    bad |= !__builtin_isfinite(v);
    amax = fmaxf(amax, fabsf(v));
  }
  amax = dsh_wave_max(amax);
  bad = __ballot(bad) != 0ull;
  const float s = amax / 127.0f, inv = amax > 0.0f ? 1.0f / s : 0.0f;
  double r2 = 0.0, w2 = 0.0, q1 = 0.0;
  int8_t *qr = q + (size_t)row * H;
  for (int j = lane; j < H; j += 64) {
    const float v = __uint_as_float((uint32_t)w[j] << 16);
    int qi = 0;
    if (!bad && amax > 0.0f) qi = max(-127, min(127, (int)__builtin_rintf(v * inv)));
    qr[j] = (int8_t)qi;
    const double d = (double)v - (double)s * (double)qi;
    r2 += d * d;
    w2 += (double)v * (double)v;
    q1 += (double)abs(qi);
  }
  r2 = lm_wave_sum_d(r2);
  w2 = lm_wave_sum_d(w2);
  q1 = lm_wave_sum_d(q1);
  if (lane == 0) {
    const double a = (lm_gamma(H) * sqrt(w2) + sqrt(r2)) * (1.0 + 1e-12);
    const double b = (double)s * q1 * (1.0 + 1e-12);
    sab[3 * (size_t)row] = s;
    sab[3 * (size_t)row + 1] = bad ? __builtin_inff() : lm_f32_up(a);
    sab[3 * (size_t)row + 2] = bad ? __builtin_inff() : lm_f32_up(b);
  }
}

// Block = 512 rows, one block per CU (wave w: rows 64w .. 64w + 63 of the block, four per round:
// lanes 16g .. 16g + 15
// take row 4k + g of round k, lane s of them the 16-byte pieces 16s + 256m of the row, m < NM =
// H / 256, so each load instruction reads 4 rows x 256 contiguous bytes). The input (XC > 0: the
// sum of XC copies in copy order, as the one-pass kernel forms it; block 0 writes it to x_out) is
// put on the grid 2^(e-14) (|x| < 2^e) as two 8-bit limbs (converted once per block in LDS, then
// held by each lane for its own columns); the row's dot products are exact int32 sums, kept in LDS
// per row. D rounds of loads stay in flight. After the stream each thread turns one row's sums into
// its bound and the block takes its largest lower bound. Then each
// half-wave recomputes a candidate row (staged in LDS by 16-byte loads, all in flight at once):
// lane c < 32 runs chain c (columns j = c mod 32 in
// increasing order, fma(w_j, x_j, acc) from 0) and lane 0 of the half adds the chains as
// _mm512_reduce_add_ps(a0 + a1) does (the one-pass kernel's tree). step_inc: advanced by block 0,
// as the one-pass kernel does, for the final kernel after it.
template <int NM, int XC>
// (W, q, sab and x are deliberately not __restrict__: the memory clobbers then keep their loads in
// issue order)
__global__ void __launch_bounds__(512) k_lm_q8_argmax(const uint16_t *W, const int8_t *q, const float *sab,
                                                      const float *x,
                                                      int vocab, float *__restrict__ x_out,
                                                      unsigned long long *__restrict__ cand, int *__restrict__ step_inc) {
  if (step_inc && blockIdx.x == 0 && threadIdx.x == 0) *step_inc += 1;
  constexpr int H = 256 * NM, D = 4, NR = 16;  // rounds of 4 rows per wave
  __shared__ __attribute__((aligned(16))) float s_x[H];
  __shared__ __attribute__((aligned(16))) int8_t s_xq[2][H];  // the input's low and high limbs
  __shared__ int2 s_d[LM_Q8_ROWS];                             // per row: Σ q·lo, Σ q·hi
  __shared__ float s_mx[8];
  __shared__ double s_sq[8], s_lb[8];
  __shared__ int s_n;
  __shared__ int s_list[LM_Q8_ROWS];
  __shared__ float s_acc[16][32];
  __shared__ __attribute__((aligned(16))) uint16_t s_row[16][H];  // a candidate row per half-wave
  __shared__ unsigned long long s_best[16];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, sub = lane & 15, grp = lane >> 4;
  const int rb = blockIdx.x * LM_Q8_ROWS;
  auto src = [&](int k) { return q + (size_t)min(rb + 64 * wave + 4 * k + grp, vocab - 1) * H + 16 * sub; };
  // the input first (it gates the limbs; a wave's loads complete in issue order), then this
  // thread's row's constants, then the first D rounds of rows
  constexpr int NPC = H / 4;  // 4-float pieces of x (<= 512: one per thread)
  f32x4 xa;
  {
    const int p = min(t, NPC - 1);
    if constexpr (XC > 0) {
      f32x4 c4[XC];
#pragma unroll
      for (int c = 0; c < XC; c++) c4[c] = ((const f32x4 *)(x + (size_t)c * H))[p];
      f32x4 s4 = c4[0];
#pragma unroll
      for (int c = 1; c < XC; c++) s4 += c4[c];
      xa = s4;
    } else {
      xa = ((const f32x4 *)x)[p];
    }
  }
  float cs[3];
#pragma unroll
  for (int c = 0; c < 3; c++) cs[c] = sab[3 * (size_t)min(rb + t, vocab - 1) + c];
  asm volatile("" ::: "memory");
  u32x4 ring[D][NM];
#pragma unroll
  for (int k = 0; k < D; k++) {
    const int8_t *p = src(k);
#pragma unroll
    for (int m = 0; m < NM; m++) ring[k][m] = dsh_load_nt(p + 256 * m);
    asm volatile("" ::: "memory");
  }
  float mx = 0.0f;
  double sq = 0.0;
  {
    const bool own = t < NPC;
    if (own) {
      *(f32x4 *)(s_x + 4 * t) = xa;
      if (XC > 0 && x_out && blockIdx.x == 0) *(f32x4 *)(x_out + 4 * t) = xa;
    }
    // the statistics take the piece through selects, so its loads are not moved into a branch
    // (where the wait for them would also wait for the rows issued after them)
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const float v = own ? xa[c] : 0.0f;
      mx = fmaxf(mx, fabsf(v));
      sq += (double)v * (double)v;
    }
  }
  // a NaN input leaves mx NaN-free but makes sq, and so every bound, NaN: every row a candidate
  mx = dsh_wave_max(mx);
  sq = lm_wave_sum_d(sq);
  if (lane == 0) {
    s_mx[wave] = mx;
    s_sq[wave] = sq;
  }
  if (t == 0) s_n = 0;
  __syncthreads();
  float xmax = s_mx[0];
  double sq_all = s_sq[0];
#pragma unroll
  for (int w = 1; w < 8; w++) {
    xmax = fmaxf(xmax, s_mx[w]);
    sq_all += s_sq[w];
  }
  const double x2 = sqrt(sq_all * (1.0 + 1e-12));
  const int e = __builtin_amdgcn_frexp_expf(xmax);  // xmax < 2^e
  const double grid = ldexp(1.0, e - 14), half_grid = ldexp(1.0, e - 15);
  // the limbs: X = rint(x 2^(14-e)) (|X| <= 2^14) = 256 hi + lo, lo in [-128, 127], hi in [-64, 64]
  for (int j = t; j < H; j += LM_Q8_ROWS) {
    const int X = (int)__builtin_rintf(__builtin_ldexpf(s_x[j], 14 - e));
    const int l = __builtin_amdgcn_sbfe(X, 0, 8);
    s_xq[0][j] = (int8_t)l;
    s_xq[1][j] = (int8_t)((X - l) >> 8);
  }
  __syncthreads();
  // this lane's columns 16 sub + 256 m .. + 15
  u32x4 xlo[NM], xhi[NM];
#pragma unroll
  for (int m = 0; m < NM; m++) {
    xlo[m] = *(const u32x4 *)&s_xq[0][16 * sub + 256 * m];
    xhi[m] = *(const u32x4 *)&s_xq[1][16 * sub + 256 * m];
  }
#pragma unroll
  for (int k = 0; k < NR; k++) {
    const int sl = k % D;
    int dlo = 0, dhi = 0;
#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
      for (int w = 0; w < 4; w++) {
        dlo = __builtin_amdgcn_sdot4((int)ring[sl][m][w], (int)xlo[m][w], dlo, false);
        dhi = __builtin_amdgcn_sdot4((int)ring[sl][m][w], (int)xhi[m][w], dhi, false);
      }
    if (k + D < NR) {
      const int8_t *p = src(k + D);
#pragma unroll
      for (int m = 0; m < NM; m++) ring[sl][m] = dsh_load_nt(p + 256 * m);
      asm volatile("" ::: "memory");
    }
    dlo = lm_row16_sum_i(dlo);
    dhi = lm_row16_sum_i(dhi);
    if (sub == 0) s_d[64 * wave + 4 * k + grp] = int2{dlo, dhi};
  }
  __syncthreads();
  // row rb + t: A = s 2^(e-14) (256 Σ q·hi + Σ q·lo), its bound B, the upper bound U = A + B
  const int2 dd = s_d[t];
  const double A = (double)cs[0] * grid * (256.0 * (double)dd.y + (double)dd.x);
  const double B = (double)cs[1] * x2 + (double)cs[2] * half_grid + 0x1p-22 * fabs(A);
  const double u = A + B;
  const double lbmax = lm_wave_max_d(rb + t < vocab ? A - B : -__builtin_inf());
  if (lane == 0) s_lb[wave] = lbmax;
  __syncthreads();
  double lb = s_lb[0];
#pragma unroll
  for (int w = 1; w < 8; w++) lb = fmax(lb, s_lb[w]);
  if (rb + t < vocab && !(u < lb)) s_list[atomicAdd(&s_n, 1)] = rb + t;
  __syncthreads();
  const int n = s_n;
  const int half = t >> 5, c = t & 31;
  unsigned long long best = 0ull;
  for (int k = half; k < n; k += 16) {
    const int r = s_list[k];
    // the row into LDS: NM 16-byte pieces per lane of the half, all in flight at once
    const u32x4 *wr = (const u32x4 *)(W + (size_t)r * H);
    u32x4 pc[NM];
#pragma unroll
    for (int i = 0; i < NM; i++) pc[i] = wr[c + 32 * i];
#pragma unroll
    for (int i = 0; i < NM; i++) *(u32x4 *)&s_row[half][8 * (c + 32 * i)] = pc[i];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float acc = 0.0f;
#pragma unroll 8
    for (int j = c; j < H; j += 32) acc = __builtin_fmaf(__uint_as_float((uint32_t)s_row[half][j] << 16), s_x[j], acc);
    s_acc[half][c] = acc;
    // the half's chains are read by its lane 0: LDS executes a wave's operations in order, the
    // fences keep the compiler from reordering
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (c == 0) {
      const float *a = s_acc[half];
      float A[16], T3[8], T6[4];
#pragma unroll
      for (int i = 0; i < 16; i++) A[i] = a[i] + a[16 + i];
#pragma unroll
      for (int i = 0; i < 8; i++) T3[i] = A[8 + i] + A[i];
#pragma unroll
      for (int i = 0; i < 4; i++) T6[i] = T3[4 + i] + T3[i];
      const float v = (T6[0] + T6[2]) + (T6[1] + T6[3]);
      best = dsh_umax64(best, dsh_argmax_key(v, r));
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  if (c == 0) s_best[half] = best;
  __syncthreads();
  if (t == 0) {
    unsigned long long b = s_best[0];
#pragma unroll
    for (int i = 1; i < 16; i++) b = dsh_umax64(b, s_best[i]);
    cand[blockIdx.x] = b;
  }
}

extern "C" {

int dsh_lm_q8_supported(int H, int vocab) { return H > 0 && H % 256 == 0 && H <= 2048 && vocab > 0; }

int dsh_lm_q8_blocks(int vocab) { return (vocab + LM_Q8_ROWS - 1) / LM_Q8_ROWS; }

size_t dsh_lm_q8_bytes(int H, int vocab) {
  const size_t al = 256;
  auto up = [&](size_t n) { return (n + al - 1) / al * al; };
  return up((size_t)vocab * H) + up((size_t)vocab * 12);
}

void dsh_lm_q8_carve(void *base, int H, int vocab, dsh_lm_q8_t *Q) {
  const size_t al = 256;
  auto up = [&](size_t n) { return (n + al - 1) / al * al; };
  char *p = (char *)base;
  Q->H = H;
  Q->vocab = vocab;
  Q->q = (int8_t *)p;
  p += up((size_t)vocab * H);
  Q->sab = (float *)p;
}

hipError_t dsh_launch_lm_q8_build(const uint16_t *W, const dsh_lm_q8_t *Q, hipStream_t s) {
  if (!W || !Q || !dsh_lm_q8_supported(Q->H, Q->vocab)) return hipErrorInvalidValue;
  k_lm_q8_build<<<(Q->vocab + 3) / 4, 256, 0, s>>>(W, Q->H, Q->vocab, Q->q, Q->sab);
  return hipGetLastError();
}

// ncopies: 0 (x is the input) or 8 (x holds 8 copies whose sum is the input; block 0 writes the sum
// to x_out when given).
hipError_t dsh_launch_lm_q8(const uint16_t *W, const dsh_lm_q8_t *Q, const float *x, int ncopies, float *x_out,
                            unsigned long long *cand, int *step_inc, hipStream_t s) {
  if (!W || !Q || !x || !cand || !dsh_lm_q8_supported(Q->H, Q->vocab) || (ncopies != 0 && ncopies != 8) ||
      ((uintptr_t)x & 15) || (x_out && ((uintptr_t)x_out & 15)))
    return hipErrorInvalidValue;
  const int nb = dsh_lm_q8_blocks(Q->vocab);
#define LM_Q8_CASE(nm)                                                                                           \
  case nm:                                                                                                       \
    if (ncopies)                                                                                                 \
      k_lm_q8_argmax<nm, 8><<<nb, 512, 0, s>>>(W, Q->q, Q->sab, x, Q->vocab, x_out, cand, step_inc);             \
    else                                                                                                         \
      k_lm_q8_argmax<nm, 0><<<nb, 512, 0, s>>>(W, Q->q, Q->sab, x, Q->vocab, nullptr, cand, step_inc);           \
    break;
  switch (Q->H / 256) {
    LM_Q8_CASE(1)
    LM_Q8_CASE(2)
    LM_Q8_CASE(3)
    LM_Q8_CASE(4)
    LM_Q8_CASE(5)
    LM_Q8_CASE(6)
    LM_Q8_CASE(7)
    LM_Q8_CASE(8)
    default:
      return hipErrorInvalidValue;
  }
#undef LM_Q8_CASE
  return hipGetLastError();
}

}  // extern "C"
