// k_dec.hip — latency-oriented decode kernels (batch 1) for the device-resident MoE layer and stack.
//
// Per MoE layer two kernels run back to back on one stream:
//   gate_up : routing (reduction of router partial scores, softmax/top-k) + fused gate_up INT8
//             dequant-matvec + SwiGLU for the top-k routed experts and the shared expert
//             (ds_moe_decoder.c:145-183 routing, ds_quantize.c:301-318 first half of the expert)
//   down    : down INT8 dequant-matvec of every selected expert and the shared expert, combine in
//             top-k order, shared add, residual (ds_quantize.c:319-320, ds_kernels.c:359-371,
//             ds_moe_decoder.c:278, :468); it also emits the next layer's router partial scores
//             (scores are linear in x, so Wr·x = Σ_blocks Wr[:, rows]·x[rows]).
// The first layer's partial scores come from a small kernel; in DECODE routing mode (bf16 router in
// the reference's exact AVX-512 order) a scores kernel writes the full scores as a single partial.
//
// Every load phase is branch-free with all of its loads issued before the first use, so each
// kernel costs one memory round trip plus its transfer time.
#include "dsh_avx.h"
#include "dsh_cert.h"
#include "dsh_route.h"
#include "k_core.h"

__device__ __forceinline__ float2 so_pair(const float *so, size_t i) { return ((const float2 *)so)[i]; }

__device__ __forceinline__ const float *at_step(const float *x, const int *step, int stride) {
  return step ? x + (size_t)(*step) * stride : x;
}

__device__ __forceinline__ void load_f16x(const float *p, float *o) {
#pragma unroll
  for (int d = 0; d < 4; d++) {
    f32x4 t = *(const f32x4 *)(p + 4 * d);
    o[4 * d] = t[0];
    o[4 * d + 1] = t[1];
    o[4 * d + 2] = t[2];
    o[4 * d + 3] = t[3];
  }
}

// ============================================================================ routing in a block
// Routing of one MoE layer from the NP partial score vectors, done by every block that needs it:
// route_load issues the ROUTE_BATCH partial loads of each wave (wave v: the contiguous range
// v*P .. v*P + P - 1, P = ceil(NP / 4) <= ROUTE_BATCH, checked by dsh_dec_supported), route_reduce
// sums them in that order from 0 and stores the wave sums, with (s_lam) the sum of |running sum|
// before each partial, the prefix sizes the certified CFG selection bounds its rounding with
// (dsh_cert.h). route_select (every wave, for itself) adds the four wave sums in wave order and
// selects the experts (same semantics as k_core.hip's top-k helpers); in CFG routing from row
// partials, route_select_cert certifies the selection against ds_linear's order first. Results in
// s_idx/s_w (LDS), visible after the next barrier.
#define ROUTE_BATCH 40

__device__ __forceinline__ int route_span(int np) { return (np + 3) >> 2; }

__device__ __forceinline__ void route_load(const float *partials, int np, float *v) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, b0 = wave * route_span(np);
#pragma unroll
  for (int j = 0; j < ROUTE_BATCH; j++) v[j] = partials[(size_t)min(b0 + j, np - 1) * 64 + lane];
}

__device__ __forceinline__ void route_reduce(int np, int E, const float *v, float (*s_red)[64], float (*s_lam)[64]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, P = route_span(np), b0 = wave * P;
  float acc = 0.0f, lam = 0.0f;
#pragma unroll
  for (int j = 0; j < ROUTE_BATCH; j++)
    if (j < P && b0 + j < np) {
      lam += fabsf(acc);
      acc += v[j];
    }
  s_red[wave][lane] = lane < E ? acc : 0.0f;
  if (s_lam) s_lam[wave][lane] = lane < E ? lam : 0.0f;
}

// partials per wave row of route_reduce
__device__ __forceinline__ void route_counts(int np, int nb[4]) {
  const int P = route_span(np);
#pragma unroll
  for (int v = 0; v < 4; v++) nb[v] = max(0, min(P, np - v * P));
}

// ============================================================================ partial scores
// partials[b][e] = Σ_{r in rows of block b} Wr[e][r] * x[r] for R consecutive rows per block
// (f32 router, CFG mode); the row order inside a block is sequential. WrT is the router
// transposed ([H][E]), so a block reads R contiguous rows of E floats.
template <int R>
__global__ void __launch_bounds__(64) k_dec_partial_scores(const float *__restrict__ WrT, const float *__restrict__ x_in,
                                                           const int *__restrict__ step, int stride, int H, int E,
                                                           float *__restrict__ partials) {
  const float *x = at_step(x_in, step, stride);
  const int lane = threadIdx.x, r0 = blockIdx.x * R;
  float p = 0.0f;
  if (lane < E) {
    float w[R], xv[R];
#pragma unroll
    for (int j = 0; j < R; j++) {
      w[j] = WrT[(size_t)(r0 + j) * E + lane];
      xv[j] = x[r0 + j];
    }
#pragma unroll
    for (int j = 0; j < R; j++) p = __builtin_fmaf(w[j], xv[j], p);
  }
  partials[(size_t)blockIdx.x * 64 + lane] = lane < E ? p : 0.0f;
}

// CFG mode, exact: the full f32 router scores in ds_linear's order (no BLAS, seq 1, ds_kernels.c:639-652,
// as GCC compiles it: rounded products added in index order, the tail past the last multiple of 8
// fused), written as the single partial. One wave, lane = expert, reading the transposed router
// row k (E floats, one coalesced load) PF rows ahead; x staged in LDS. Used where routing must
// match the reference bit for bit (the bf16 simulation); about one 2*H-long dependent chain.
__global__ void __launch_bounds__(64) k_dec_scores_f32_exact(const float *__restrict__ WrT, const float *__restrict__ x_in,
                                                             const int *__restrict__ step, int stride, int H, int E,
                                                             float *__restrict__ partials) {
  constexpr int PF = 32;
  __shared__ __attribute__((aligned(16))) float s_x[2048];
  const float *x = at_step(x_in, step, stride);
  const int lane = threadIdx.x, ec = min(lane, E - 1);
  for (int i = lane; i < H; i += 64) s_x[i] = x[i];
  __syncthreads();
  float ring[PF];
#pragma unroll
  for (int j = 0; j < PF; j++) ring[j] = WrT[(size_t)min(j, H - 1) * E + ec];
  const int m = H >= 16 ? (H & ~15) + ((H - (H & ~15)) >= 8 ? 8 : 0) : (H >= 8 ? 8 : 0);
  float sc = 0.0f;
  for (int k0 = 0; k0 < H; k0 += PF) {
    float w[PF];
#pragma unroll
    for (int j = 0; j < PF; j++) {
      w[j] = ring[j];
      ring[j] = WrT[(size_t)min(k0 + PF + j, H - 1) * E + ec];
    }
#pragma unroll
    for (int j = 0; j < PF; j++) {
      const int k = k0 + j;
      if (k < m)
        sc = __fadd_rn(sc, __fmul_rn(s_x[k], w[j]));
      else if (k < H)
        sc = __builtin_fmaf(s_x[k], w[j], sc);
    }
  }
  partials[lane] = lane < E ? sc : 0.0f;
}

// out[r] = the Euclidean norm of row r, summed in f64 and rounded up to f32 (one block per row).
__global__ void __launch_bounds__(256) k_row_norms(const float *__restrict__ A, int cols, float *__restrict__ out) {
  __shared__ double s[4];
  const float *a = A + (size_t)blockIdx.x * cols;
  double acc = 0.0;
  for (int i = threadIdx.x; i < cols; i += 256) acc += (double)a[i] * (double)a[i];
  for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
  if ((threadIdx.x & 63) == 0) s[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    const double n = sqrt(((s[0] + s[1]) + s[2]) + s[3]);
    float f = (float)n;
    if ((double)f < n) f = __uint_as_float(__float_as_uint(f) + 1u);  // next float up (n >= 0, finite)
    out[blockIdx.x] = f;
  }
}

// dst[c][r] = src[r][c] for a rows x cols f32 matrix (32x32 tiles through LDS).
__global__ void __launch_bounds__(256) k_transpose_f32(const float *__restrict__ src, float *__restrict__ dst, int rows,
                                                       int cols) {
  __shared__ float t[32][33];
  const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  for (int i = ty; i < 32; i += 8)
    if (r0 + i < rows && c0 + tx < cols) t[i][tx] = src[(size_t)(r0 + i) * cols + c0 + tx];
  __syncthreads();
  for (int i = ty; i < 32; i += 8)
    if (c0 + i < cols && r0 + tx < rows) dst[(size_t)(c0 + i) * rows + r0 + tx] = t[tx][i];
}

// DECODE mode: full scores in the reference's AVX-512 order, written as the single partial. 16 rows
// per 64-lane block, 4 lanes per row (H == 32*N32): each lane loads its 16-byte pieces of the row
// (N32 of them) straight into registers, all in flight with x's pieces, which are staged in LDS. Rows
// on the reference's single-row path (an odd thread chunk) read theirs in avx_row's loop.
template <int N32>
__global__ void __launch_bounds__(64) k_dec_scores_bf16(const uint16_t *__restrict__ Wr, const float *__restrict__ x_in,
                                                        const int *__restrict__ step, int stride, int E, int chunk,
                                                        float *__restrict__ partials, int ncopies) {
  constexpr int H = 32 * N32, NX = H / 4, XP = (NX + 63) / 64;
  __shared__ __attribute__((aligned(16))) float xs[H];
  const float *x = at_step(x_in, step, stride);
  const int L = threadIdx.x & 3, e = blockIdx.x * 16 + (threadIdx.x >> 2);
  const int ec = min(e, E - 1);
  f32x4 xr[XP];
#pragma unroll
  for (int j = 0; j < XP; j++) xr[j] = ((const f32x4 *)x)[min((int)threadIdx.x + 64 * j, NX - 1)];
  if (ncopies > 1) {  // x = Σ of 8 copies [8][H], added in copy order (as the one-kernel layer does)
    f32x4 xc[XP][7];
#pragma unroll
    for (int j = 0; j < XP; j++)
#pragma unroll
      for (int c = 0; c < 7; c++) xc[j][c] = ((const f32x4 *)(x + (size_t)(c + 1) * H))[min((int)threadIdx.x + 64 * j, NX - 1)];
#pragma unroll
    for (int j = 0; j < XP; j++)
#pragma unroll
      for (int c = 0; c < 7; c++) xr[j] += xc[j][c];
  }
  asm volatile("" ::: "memory");  // x first: its LDS stores wait for x only
  const u32x4 *row = (const u32x4 *)(Wr + (size_t)ec * H);
  u32x4 wv[N32];
#pragma unroll
  for (int i = 0; i < N32; i++) wv[i] = row[4 * i + L];
#pragma unroll
  for (int j = 0; j < XP; j++) {
    const int i = threadIdx.x + 64 * j;
    if (i < NX) ((f32x4 *)xs)[i] = xr[j];
  }
  __syncthreads();
  if (e >= E) return;
  const int path = row_path(e, E, chunk, false);
  float v;
  if (path == DSH_ROW_SINGLE)
    v = avx_row<true>(Wr + (size_t)e * H, xs, H, L, true, true, 0.0f, true);
  else
    v = avx_row_regs32<N32>(wv, xs, L, true, 0.0f);
  if (L == 0) partials[e] = v;
}

// ============================================================================ gate_up + SwiGLU
// A unit is one row pair (gate row, up row) handled by 16 lanes; lane sub reads the 16-byte chunks
// sub + 16m (m < CPL) of both rows (H == 256*CPL). Block b: wave 0 takes the shared expert's units
// 4b + g (lane group g = lane / 16; rows u and SI + u), waves 1-3 the routed units 12b + 4(w-1) + g
// of the K*I routed ones (slot k = u/I, intermediate i = u%I). The shared wave loads its rows at
// once and never routes; the routed waves select the experts (each for itself) and then load.
//
// The dots run on the integer dot unit: x is split once per block into four signed 8-bit limbs,
// X = rint(x * 2^(29-e)) = L3*2^24 + L2*2^16 + L1*2^8 + L0 with 2^e > max|x| (|X| <= 2^29, so L3
// fits), and a row's dot is sum_j q_j X_j (q = u - 128, the stored signed code) in int32 per limb,
// scaled back by 2^(e-29). X is exact for every x_j within 2^6 of max|x| (a 24-bit mantissa fits in
// 30 bits); smaller ones are rounded by at most 2^(e-30), far below the f32 rounding of a dot. The
// products and sums are exact; the only rounding is the final f32 combination of the limb sums. The +128 of
// the unsigned codes moves into the offset term: scale*Σu*x + off*Σx = scale*Σq*x + (off +
// 128*scale)*Σx (ds_quantize.c:163-166), with Σx summed once per block.
// Every lane of a wave issues the same loads in the same order (x, the routing partials, then its
// rows); all stores happen at the end. The empty asm statements keep the compiler from reordering
// the load groups (x and partials are not __restrict__ so that they cannot be moved across them).
template <int CPL>
__device__ __forceinline__ void gate_up_body(const dsh_layer_t &L, const float *x, const float *partials, int np,
                                             int mode, int bf16sim, const dsh_layer_work_t &wk, const dsh_rcert_t &rc,
                                             int blk, int *s_idx, float *s_w, float (*s_red)[64],
                                             float (*s_lam)[64], float (*s_tmp)[4][64], float *s_stat,
                                             unsigned *s_lq) {
  constexpr int XV = (64 * CPL + 255) / 256;  // 16-byte pieces of x per thread
  constexpr int NP = 64 * CPL;                // pieces (4 elements) of x, = words per limb array
  constexpr int NL = 4;                       // limbs
  const int H = L.H, I = L.I, K = L.K, SI = L.SI;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, sub = lane & 15, grp = lane >> 4;
  const int KI = K * I;
  const bool shared_wave = wave == 0;
  // CFG from row partials (not the bf16 simulation's exact scores): the selection is certified
  // against ds_linear's order (dsh_cert.h)
  const bool cert = mode == DSH_ROUTE_CFG && !bf16sim && np > 1 && H % np == 0;

  f32x4 xr[XV];
#pragma unroll
  for (int j = 0; j < XV; j++) xr[j] = ((const f32x4 *)x)[min((int)threadIdx.x + 256 * j, NP - 1)];
  asm volatile("" ::: "memory");  // keeps the issue order: x, partials, shared rows
  float pv[ROUTE_BATCH];
  route_load(partials, np, pv);
  const float wn = cert && !shared_wave ? L.router_norm[min(lane, L.E - 1)] : 0.0f;
  asm volatile("" ::: "memory");
  const int su = blk * 4 + grp;
  const int suc = su < SI ? su : 0;
  u32x4 wg[CPL], wu[CPL];
  if (shared_wave) {
    const int8_t *grow = L.sgu_q + (size_t)suc * H;
    const int8_t *urow = L.sgu_q + (size_t)(SI + suc) * H;
#pragma unroll
    for (int m = 0; m < CPL; m++) {
      wg[m] = dsh_load_nt(grow + 16 * (sub + 16 * m));
      wu[m] = dsh_load_nt(urow + 16 * (sub + 16 * m));
    }
  }
  asm volatile("" ::: "memory");
  {  // max|x|, Σx and Σx² of the pieces this thread owns (clamped duplicates skipped), per wave
    float mx = 0.0f, sx = 0.0f, ss = 0.0f;
#pragma unroll
    for (int j = 0; j < XV; j++) {
      const bool own = (int)threadIdx.x + 256 * j < NP;
#pragma unroll
      for (int c = 0; c < 4; c++) {
        mx = own ? fmaxf(mx, fabsf(xr[j][c])) : mx;
        sx += own ? xr[j][c] : 0.0f;
        ss = own ? __builtin_fmaf(xr[j][c], xr[j][c], ss) : ss;
      }
    }
    mx = dsh_wave_max(mx);
    sx = dsh_wave_sum(sx);
    if (cert) ss = dsh_wave_sum(ss);
    if (lane == 0) {
      s_stat[wave] = mx;
      s_stat[4 + wave] = sx;
      s_stat[8 + wave] = ss;
    }
  }
  route_reduce(np, L.E, pv, s_red, cert ? s_lam : nullptr);
  __syncthreads();  // s_red, s_lam, s_stat
  const float xmax = fmaxf(fmaxf(s_stat[0], s_stat[1]), fmaxf(s_stat[2], s_stat[3]));
  const float xsum = ((s_stat[4] + s_stat[5]) + s_stat[6]) + s_stat[7];
  const int ex = __builtin_amdgcn_frexp_expf(xmax);  // xmax < 2^ex

  int ru = 0, r = 0, e = 0;
  float2 sog, sou;
  bool recomputed = false;
  if (!shared_wave) {
    if (cert) {
      // ||x|| from the f32 sum of squares: relative error below (H + 3) u, which 2^-10 covers
      const float xn = __builtin_sqrtf(((s_stat[8] + s_stat[9]) + s_stat[10]) + s_stat[11]) * (1.0f + 0x1p-10f);
      int nb[4];
      route_counts(np, nb);
      recomputed = route_select_cert(L.E, K, s_idx + 64 * wave, s_w + 64 * wave, s_red, s_lam, nb, H / np, H, wn, xn,
                                     L.router_f32, x, s_tmp[wave]);
    } else {
      route_select(L.E, K, mode, s_idx + 64 * wave, s_w + 64 * wave, s_red);
    }
    s_idx += 64 * wave;
    s_w += 64 * wave;
    ru = blk * 12 + (wave - 1) * 4 + grp;
    r = ru < KI ? ru : 0;
    const int k = r / I, i = r - k * I;
    e = s_idx[k];
    const size_t base = (size_t)max(e, 0) * 2 * I;
    const int8_t *grow = L.gu_q + (base + i) * H;
    const int8_t *urow = L.gu_q + (base + I + i) * H;
#pragma unroll
    for (int m = 0; m < CPL; m++) {
      wg[m] = dsh_load_nt(grow + 16 * (sub + 16 * m));
      wu[m] = dsh_load_nt(urow + 16 * (sub + 16 * m));
    }
    sog = so_pair(L.gu_so, base + i);
    sou = so_pair(L.gu_so, base + I + i);
  } else {
    sog = so_pair(L.sgu_so, suc);
    sou = so_pair(L.sgu_so, SI + suc);
  }
  // x → limbs, piece p (elements 4p..4p+3) into word p of each limb array
#pragma unroll
  for (int j = 0; j < XV; j++) {
    const int p = min((int)threadIdx.x + 256 * j, NP - 1);  // duplicates store identical words
    unsigned wl[NL] = {};
#pragma unroll
    for (int c = 0; c < 4; c++) {
      int X = (int)__builtin_rintf(__builtin_ldexpf(xr[j][c], 29 - ex));
#pragma unroll
      for (int l = 0; l < NL; l++) {
        const int d = l < NL - 1 ? __builtin_amdgcn_sbfe(X, 0, 8) : X;  // balanced digit; the top one is the rest
        wl[l] |= ((unsigned)d & 255u) << (8 * c);
        X = (X - d) >> 8;
      }
    }
#pragma unroll
    for (int l = 0; l < NL; l++) s_lq[l * NP + p] = wl[l];
  }
  __syncthreads();  // limbs
  int ag[NL] = {}, au[NL] = {};  // |sum| <= 16*CPL * 128 * 128 < 2^21
#pragma unroll
  for (int m = 0; m < CPL; m++) {
    const int c = sub + 16 * m;  // 16-element chunk = 4 words
#pragma unroll
    for (int l = 0; l < NL; l++) {
      const u32x4 lw = *(const u32x4 *)(s_lq + l * NP + 4 * c);
#pragma unroll
      for (int d = 0; d < 4; d++) {
        ag[l] = __builtin_amdgcn_sdot4((int)wg[m][d], (int)lw[d], ag[l], false);
        au[l] = __builtin_amdgcn_sdot4((int)wu[m][d], (int)lw[d], au[l], false);
      }
    }
  }
  float dg = (float)ag[NL - 1], du = (float)au[NL - 1];
#pragma unroll
  for (int l = NL - 2; l >= 0; l--) {
    dg = __builtin_fmaf(dg, 256.0f, (float)ag[l]);
    du = __builtin_fmaf(du, 256.0f, (float)au[l]);
  }
  dg = __builtin_ldexpf(dsh_row16_sum(dg), ex - 29);
  du = __builtin_ldexpf(dsh_row16_sum(du), ex - 29);
  const float og = __builtin_fmaf(128.0f, sog.x, sog.y), ou = __builtin_fmaf(128.0f, sou.x, sou.y);
  float g = __builtin_fmaf(sog.x, dg, og * xsum);
  float up = __builtin_fmaf(sou.x, du, ou * xsum);
  if (bf16sim) {
    g = dsh_bf16_round_half_up(g);
    up = dsh_bf16_round_half_up(up);
  }
  float hv = dsh_swiglu(g, up);
  if (bf16sim) hv = dsh_bf16_round_half_up(hv);
  // stores: shared unit (KI + su), routed unit r (0 when DECODE routing left slot k empty)
  if (sub == 0) {
    float *dst = nullptr;
    float val = hv;
    if (shared_wave) {
      if (su < SI) dst = wk.h + KI + su;
    } else if (ru < KI) {
      dst = wk.h + r;
      val = e >= 0 ? hv : 0.0f;
    }
    if (dst) *dst = val;
  }
  if (blk == 0 && wave == 1 && lane < K) {  // block 0 publishes the routing (read by the down kernel)
    wk.idx[lane] = s_idx[lane];
    wk.w[lane] = s_w[lane];
  }
  if (cert && blk == 0 && wave == 1 && lane == 0) cert_record(rc, s_idx, s_w, K, recomputed ? 1 : 0, x, H);
}

template <int CPL>
__global__ void __launch_bounds__(256) k_dec_gate_up(dsh_layer_t L, const float *x_in, const int *__restrict__ step,
                                                     int stride, const float *partials, int np, int mode, int bf16sim,
                                                     dsh_layer_work_t wk, dsh_rcert_t rc) {
  __shared__ int s_idx[4 * 64];
  __shared__ float s_w[4 * 64];
  __shared__ float s_red[4][64];
  __shared__ float s_lam[4][64];
  __shared__ float s_tmp[4][4][64];
  __shared__ float s_stat[12];
  __shared__ __attribute__((aligned(16))) unsigned s_lq[4 * 64 * CPL];
  gate_up_body<CPL>(L, at_step(x_in, step, stride), partials, np, mode, bf16sim, wk, rc, blockIdx.x, s_idx, s_w,
                    s_red, s_lam, s_tmp, s_stat, s_lq);
}

// ============================================================================ down + combine
// One 512-thread block per R output rows (R = 8 or 16); wave s (0..7) owns segment s: routed slot s
// for s < K (expert idx[s]), else the shared expert's I-wide column block s-K. Lane c < I/16 holds
// the 16 h values of chunk c in registers and streams chunk c of each of its R rows (one 16-byte
// load per row, all issued together). The R row dots of a wave are summed over its lanes by one
// transposed butterfly (row j lands in lanes j*64/R..), Σh by a wave sum; wave 0 then combines the 8
// segments per row in the reference's order (routed slots in top-k order with their weights, then
// the shared expert), adds the residual and, when WrT_next (the next layer's f32 router, transposed
// to [H][E]) is given, writes this block's partial
// router scores for the next layer. Requires I % 16 == 0, I/16 <= 64, K + SI/I == 8, H % R == 0.
template <int R>
__global__ void __launch_bounds__(512) k_dec_down(dsh_layer_t L, const float *__restrict__ x_in,
                                                  const int *__restrict__ step, int stride, float *__restrict__ x_out,
                                                  int residual, const float *__restrict__ resid, int bf16sim,
                                                  dsh_layer_work_t wk,
                                                  const float *__restrict__ WrT_next, int E_next,
                                                  float *__restrict__ partials_next) {
  static_assert(R == 8 || R == 16, "row butterfly for 8 or 16 rows");
  constexpr int LPR = 64 / R;  // lanes holding one row's sum
  __shared__ float s_val[8][R];
  __shared__ float s_hs[8];
  __shared__ float s_x[R];
  const float *x = at_step(x_in, step, stride);
  const int H = L.H, I = L.I, K = L.K, SI = L.SI;
  const int lane = threadIdx.x & 63, seg = threadIdx.x >> 6;
  const int CI = I >> 4;
  const int r0 = blockIdx.x * R;
  const bool lane_on = lane < CI;
  const int ch = lane_on ? lane : 0;
  const int myrow = lane / LPR;  // the row whose sum this lane holds after the butterfly

  // next layer's router columns for these rows (independent of everything else)
  float wr[R];
  if (WrT_next && seg == 0 && lane < E_next) {
#pragma unroll
    for (int j = 0; j < R; j++) wr[j] = WrT_next[(size_t)(r0 + j) * E_next + lane];
  }
  int e = -2;
  const int8_t *wbase;
  size_t so_base;
  int row_stride;
  if (seg < K) {
    e = wk.idx[seg];
    int ee = e < 0 ? 0 : e;
    wbase = L.dn_q + (size_t)ee * H * I;
    so_base = (size_t)ee * H;
    row_stride = I;
  } else {
    wbase = L.sdn_q + (size_t)(seg - K) * I;
    so_base = 0;
    row_stride = SI;
  }
  // weights of the R rows, then this lane's h chunk
  u32x4 wv[R];
#pragma unroll
  for (int j = 0; j < R; j++) wv[j] = dsh_load_nt(wbase + (size_t)(r0 + j) * row_stride + 16 * ch);
  const int hbase = seg < K ? seg * I : K * I + (seg - K) * I;
  float hv[16];
  load_f16x(wk.h + hbase + 16 * ch, hv);
  const float2 so = so_pair(seg < K ? L.dn_so : L.sdn_so, so_base + r0 + myrow);
  // what the combine needs, issued with the loads above so that it costs no round trip after the
  // barrier: the top-k weights, the shared expert's scale/offset and the residual of row r0 + lane % R
  float cw[8];
#pragma unroll
  for (int k = 0; k < 8; k++) cw[k] = wk.w[min(k, K - 1)];
  const int crow = r0 + (lane & (R - 1));
  const float2 sso = so_pair(L.sdn_so, crow);
  const float xres = resid ? resid[crow] : x[crow];  // the residual: the layer input unless given

  float hp = 0.0f;
  if (lane_on) {
#pragma unroll
    for (int j = 0; j < 16; j++) hp += hv[j];
  }
  const float hs = dsh_wave_sum(hp);
  float dots[R];
#pragma unroll
  for (int j = 0; j < R; j++) dots[j] = lane_on ? dsh_dot16_u8(wv[j], hv, 0.0f) : 0.0f;
  const float mine = R == 8 ? dsh_wave_tsum8(dots) : dsh_wave_tsum16(dots);
  if (lane % LPR == 0) {
    float v;
    if (seg < K)
      v = e >= 0 ? __builtin_fmaf(so.x, mine, so.y * hs) : 0.0f;  // e_k = scale*dot + off*Σh
    else
      v = mine;  // shared: raw dot, combined below with its sibling segments
    s_val[seg][myrow] = v;
  }
  if (lane == 0) s_hs[seg] = hs;
  __syncthreads();
  if (seg == 0) {
    float outv = 0.0f;
    if (lane < R) {
#pragma unroll
      for (int k = 0; k < 8; k++) {
        if (k < K) {
          float v = s_val[k][lane];
          if (bf16sim) v = dsh_bf16_round_half_up(v);
          outv = __builtin_fmaf(cw[k], v, outv);
        }
      }
      float sdot = 0.0f, shs = 0.0f;
#pragma unroll
      for (int k = 0; k < 8; k++) {
        if (k >= K) {
          sdot += s_val[k][lane];
          shs += s_hs[k];
        }
      }
      float sh = __builtin_fmaf(sso.x, sdot, sso.y * shs);
      if (bf16sim) sh = dsh_bf16_round_half_up(sh);
      outv = outv + sh;
      float xo = residual ? xres + outv : outv;
      x_out[crow] = xo;
      s_x[lane] = xo;
    }
    if (WrT_next) {
      // wave-local: lanes < R wrote s_x; make it visible to the other lanes of this wave
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      float p = 0.0f;
      if (lane < E_next) {
#pragma unroll
        for (int j = 0; j < R; j++) p = __builtin_fmaf(wr[j], s_x[j], p);
      }
      partials_next[(size_t)blockIdx.x * 64 + lane] = lane < E_next ? p : 0.0f;
    }
  }
}

// ============================================================================ bf16 simulation
// With ds_bf16_simulate_python the reference rounds gate, up, the SwiGLU output and every expert's
// output to bf16 (ds_quantize.c:311-320). A value summed in any order other than the reference's
// lands on the other side of a rounding boundary now and then, so these kernels compute every
// rounded value in the reference's own order (dsh_row_chain: one lane per row, the row's
// sequential fused chain, ds_quantize.c:163-166; Σx and Σh as sequential sums): for the same routing
// the layer output is bit-identical to the reference's. One lane per row makes them latency-bound
// (one 1280-long chain per projection); the unrounded mode keeps the fast kernels above.
//
// k_sim_gate_up: block b owns units 128b .. 128b+127 (the routed units k*I + i, then the shared
// expert's); threads 0-127 run the units' gate rows, 128-255 their up rows, and lane 0 of a fifth
// wave sums x. Waves 0-3 route as k_dec_gate_up does (each for itself). h = bf16(SwiGLU(bf16(g),
// bf16(u))); block 0 publishes the routing.
__global__ void __launch_bounds__(320) k_sim_gate_up(dsh_layer_t L, const float *x_in, const int *__restrict__ step,
                                                     int stride, const float *partials, int np, int mode,
                                                     dsh_layer_work_t wk) {
  __shared__ __attribute__((aligned(16))) float s_x[2048];
  __shared__ int s_idx[4 * 64];
  __shared__ float s_w[4 * 64];
  __shared__ float s_red[4][64];
  __shared__ float s_up[128];
  __shared__ float s_xsum;
  const float *x = at_step(x_in, step, stride);
  const int H = L.H, I = L.I, K = L.K, SI = L.SI, KI = K * I;
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
  for (int i = t; i < H; i += 320) s_x[i] = x[i];
  if (wave < 4) {
    float pv[ROUTE_BATCH];
    route_load(partials, np, pv);
    route_reduce(np, L.E, pv, s_red, nullptr);
  }
  __syncthreads();  // s_x, s_red
  const int u = blockIdx.x * 128 + (t & 127), part = (t >> 7) & 1;
  const bool active = wave < 4 && u < KI + SI;
  float dot = 0.0f;
  float2 so = make_float2(0.0f, 0.0f);
  int e = 0;
  if (wave == 4) {
    if (lane == 0) {  // Σx, added in element order as the reference's loop does
      float xs = 0.0f;
      for (int i = 0; i < H; i += 4) {
        const f32x4 v = *(const f32x4 *)(s_x + i);
        xs += v[0];
        xs += v[1];
        xs += v[2];
        xs += v[3];
      }
      s_xsum = xs;
    }
  } else {
    route_select(L.E, K, mode, s_idx + 64 * wave, s_w + 64 * wave, s_red);
    if (active) {
      const int8_t *row;
      if (u < KI) {
        const int k = u / I, i = u - k * I;
        e = s_idx[64 * wave + k];
        const size_t r = (size_t)max(e, 0) * 2 * I + (size_t)part * I + i;
        row = L.gu_q + r * H;
        so = so_pair(L.gu_so, r);
      } else {
        const size_t r = (size_t)part * SI + (u - KI);
        row = L.sgu_q + r * H;
        so = so_pair(L.sgu_so, r);
      }
      float unused = 0.0f;
      dot = dsh_row_chain<false>(row, s_x, H, unused);
    }
  }
  __syncthreads();  // s_xsum
  float y = 0.0f;
  if (active) {
    y = dsh_bf16_round_half_up(__builtin_fmaf(so.x, dot, so.y * s_xsum));
    if (part) s_up[t & 127] = y;
  }
  __syncthreads();  // s_up
  if (active && !part) {
    const float hv = dsh_bf16_round_half_up(dsh_swiglu(y, s_up[t]));
    wk.h[u] = (u < KI && e < 0) ? 0.0f : hv;
  }
  if (blockIdx.x == 0 && wave == 0 && lane < K) {
    wk.idx[lane] = s_idx[lane];
    wk.w[lane] = s_w[lane];
  }
}

// k_sim_down: block (64-row tile, segment seg): lane r of wave 0 runs output row 64*tile + r of routed
// slot seg (seg < K: expert idx[seg] on its I SwiGLU outputs) or of the shared expert (seg == K, on
// its SI outputs); lane 0 of wave 1 sums h. e = bf16(fma(scale, dot, offset * Σh)) into eo[seg][row]
// (0 for a DECODE slot left empty).
__global__ void __launch_bounds__(128) k_sim_down(dsh_layer_t L, dsh_layer_work_t wk) {
  __shared__ __attribute__((aligned(16))) float s_h[7 * 1024];
  __shared__ float s_hsum;
  const int H = L.H, I = L.I, K = L.K, SI = L.SI;
  const int seg = blockIdx.y, t = threadIdx.x, wave = t >> 6, lane = t & 63;
  const int n = seg < K ? I : SI;
  const float *h = wk.h + (seg < K ? seg * I : K * I);
  for (int i = t; i < n; i += 128) s_h[i] = h[i];
  const int e = seg < K ? wk.idx[seg] : 0;
  __syncthreads();  // s_h
  const int r = blockIdx.x * 64 + lane;
  float dot = 0.0f;
  float2 so = make_float2(0.0f, 0.0f);
  if (wave == 0) {
    const int8_t *row;
    if (seg < K) {
      const size_t rr = (size_t)max(e, 0) * H + r;
      row = L.dn_q + rr * I;
      so = so_pair(L.dn_so, rr);
    } else {
      row = L.sdn_q + (size_t)r * SI;
      so = so_pair(L.sdn_so, r);
    }
    float unused = 0.0f;
    dot = dsh_row_chain<false>(row, s_h, n, unused);
  } else if (lane == 0) {
    float hs = 0.0f;
    for (int i = 0; i < n; i += 4) {
      const f32x4 v = *(const f32x4 *)(s_h + i);
      hs += v[0];
      hs += v[1];
      hs += v[2];
      hs += v[3];
    }
    s_hsum = hs;
  }
  __syncthreads();  // s_hsum
  if (wave == 0)
    wk.eo[(size_t)seg * H + r] =
        (seg < K && e < 0) ? 0.0f : dsh_bf16_round_half_up(__builtin_fmaf(so.x, dot, so.y * s_hsum));
}

// k_sim_combine: R rows per 64-lane block, as k_dec_down's combine: out = Σ_k fma(w_k, e_k, out) in
// top-k order (ds_expert_combine, ds_kernels.c:359-371), + the shared output, + the residual; then
// (WrT_next) this block's partial router scores for the next layer.
template <int R>
__global__ void __launch_bounds__(64) k_sim_combine(dsh_layer_t L, const float *__restrict__ x_in,
                                                    const int *__restrict__ step, int stride, float *x_out,
                                                    int residual, const float *__restrict__ resid,
                                                    dsh_layer_work_t wk, const float *__restrict__ WrT_next,
                                                    int E_next, float *__restrict__ partials_next) {
  __shared__ float s_x[R];
  const float *x = at_step(x_in, step, stride);
  const int H = L.H, K = L.K, lane = threadIdx.x, r0 = blockIdx.x * R;
  float wr[R];
  if (WrT_next && lane < E_next) {
#pragma unroll
    for (int j = 0; j < R; j++) wr[j] = WrT_next[(size_t)(r0 + j) * E_next + lane];
  }
  if (lane < R) {
    const int r = r0 + lane;
    float out = 0.0f;
    for (int k = 0; k < K; k++) out = __builtin_fmaf(wk.w[k], wk.eo[(size_t)k * H + r], out);
    out = out + wk.eo[(size_t)K * H + r];
    const float xo = residual ? (resid ? resid[r] : x[r]) + out : out;
    x_out[r] = xo;
    s_x[lane] = xo;
  }
  if (WrT_next) {
    __syncthreads();
    float p = 0.0f;
    if (lane < E_next) {
#pragma unroll
      for (int j = 0; j < R; j++) p = __builtin_fmaf(wr[j], s_x[j], p);
    }
    partials_next[(size_t)blockIdx.x * 64 + lane] = lane < E_next ? p : 0.0f;
  }
}

// ============================================================================ LM-head argmax
// One row per lane, bit-exact 2-accumulator AVX-512 order (ds_kernels_avx.c:162-245, 4-row group
// path; the stack only takes this kernel when every row of the reference's thread chunks is on that
// path). A wave owns 64 consecutive rows. For each 128-byte line t of its rows (64 elements: two
// AVX iterations, chains 0..31 twice) it issues 8 loads in which 8 adjacent lanes read one row's
// full line, stores the 64 x 128 B tile in a wave-private LDS buffer (row pitch 144 B, so the
// 16-byte reads of 64 different rows are bank-conflict free), and each lane then reads its own row
// and accumulates its 32 chains in registers; x is uniform across the wave (scalar loads). A ring of
// D lines of loads is kept in flight. Requires in_dim % 64 == 0. Each block writes its
// (max, lowest index) key.
// XC > 0: x is XC copies [XC][in_dim] whose sum (in copy order) is the input; each block forms it
// in LDS after issuing its first line of loads (block 0 also stores it to x_out when given).
// (Finishing the argmax in the last block to arrive, with an acquire-release counter, was measured
// ~20 us slower than the separate final kernel: every block's release writes back its XCD's L2.)
template <int D, int XC>
__global__ void __launch_bounds__(256) k_dec_lm_argmax(const uint16_t *W, const float *__restrict__ x,
                                                       int in_dim, int vocab, unsigned long long *__restrict__ cand,
                                                       float *__restrict__ x_out, int *__restrict__ step_inc) {
  // step_inc: the step counter, advanced here (no block of this kernel reads it) so that every
  // block of the final kernel after it reads the same, already advanced value
  if (step_inc && blockIdx.x == 0 && threadIdx.x == 0) *step_inc += 1;
  constexpr int PITCH = 144;
  __shared__ __attribute__((aligned(16))) uint8_t tile[4][64 * PITCH];
  __shared__ unsigned long long wbest[4];
  __shared__ __attribute__((aligned(16))) float s_xs[XC ? 2048 : 4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r0 = (blockIdx.x * 4 + wave) * 64;
  const size_t row_bytes = (size_t)in_dim * 2;
  const int lrow = lane >> 3, piece = lane & 7;
  const uint8_t *src[8];
#pragma unroll
  for (int j = 0; j < 8; j++) {
    int r = min(r0 + 8 * j + lrow, vocab - 1);
    src[j] = (const uint8_t *)W + (size_t)r * row_bytes + 16 * piece;
  }
  uint8_t *wtile = tile[wave];
  const uint8_t *xdummy = (const uint8_t *)x + 16 * (lane % (in_dim / 4));  // in bounds: in_dim*4 bytes
  float acc[32];
#pragma unroll
  for (int c = 0; c < 32; c++) acc[c] = 0.0f;
  const int NT = in_dim >> 6;  // a multiple of D (launcher)
  u32x4 ring[D][8];
  // issue order = stage order, so that waiting for stage s leaves the later stages in flight (W is
  // deliberately not __restrict__: the memory clobber then keeps these loads in place)
#pragma unroll
  for (int s = 0; s < D; s++) {
#pragma unroll
    for (int j = 0; j < 8; j++) ring[s][j] = dsh_load_nt(src[j] + 128 * s);
    asm volatile("" ::: "memory");
  }
  if constexpr (XC > 0) {  // the input: sum of the copies, two 4-float pieces per thread at most
    const int npc = in_dim >> 2;
    const int p0 = threadIdx.x, p1 = min((int)threadIdx.x + 256, npc - 1);
    f32x4 a[XC], b[XC];
#pragma unroll
    for (int c = 0; c < XC; c++) {
      a[c] = ((const f32x4 *)(x + (size_t)c * in_dim))[min(p0, npc - 1)];
      b[c] = ((const f32x4 *)(x + (size_t)c * in_dim))[p1];
    }
    f32x4 sa = a[0], sb = b[0];
#pragma unroll
    for (int c = 1; c < XC; c++) {
      sa += a[c];
      sb += b[c];
    }
    if (p0 < npc) *(f32x4 *)(s_xs + 4 * p0) = sa;
    if ((int)threadIdx.x + 256 < npc) *(f32x4 *)(s_xs + 4 * p1) = sb;
    if (x_out && blockIdx.x == 0) {
      if (p0 < npc) *(f32x4 *)(x_out + 4 * p0) = sa;
      if ((int)threadIdx.x + 256 < npc) *(f32x4 *)(x_out + 4 * p1) = sb;
    }
    __syncthreads();
  }
  for (int t0 = 0; t0 < NT; t0 += D) {
#pragma unroll
    for (int s = 0; s < D; s++) {
      const int t = t0 + s;
#pragma unroll
      for (int j = 0; j < 8; j++) *(u32x4 *)(wtile + (8 * j + lrow) * PITCH + 16 * piece) = ring[s][j];
      // refill; past the last line the refill reads x instead (a few L2-resident bytes), so no line
      // of W is fetched twice
      const bool more = t + D < NT;
#pragma unroll
      for (int j = 0; j < 8; j++) ring[s][j] = dsh_load_nt(more ? src[j] + 128 * (t + D) : xdummy);
      // the tile is wave-private and LDS executes a wave's operations in order: these fences only
      // keep the compiler from moving the reads above the writes (and the next writes above them)
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const uint8_t *mine = wtile + lane * PITCH;
      const float *xt = (XC > 0 ? s_xs : x) + 64 * t;
#pragma unroll
      for (int p = 0; p < 8; p++) {
        u32x4 v = *(const u32x4 *)(mine + 16 * p);
        const int c0 = (8 * p) & 31;
#pragma unroll
        for (int d = 0; d < 4; d++) {
          acc[c0 + 2 * d] = __builtin_fmaf(dsh_bf16lo(v[d]), xt[8 * p + 2 * d], acc[c0 + 2 * d]);
          acc[c0 + 2 * d + 1] = __builtin_fmaf(dsh_bf16hi(v[d]), xt[8 * p + 2 * d + 1], acc[c0 + 2 * d + 1]);
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  }
  // _mm512_reduce_add_ps(a0 + a1) as GCC 11 expands it (see dsh_avx.h)
  float A[16], T3[8], T6[4];
#pragma unroll
  for (int i = 0; i < 16; i++) A[i] = acc[i] + acc[16 + i];
#pragma unroll
  for (int i = 0; i < 8; i++) T3[i] = A[8 + i] + A[i];
#pragma unroll
  for (int i = 0; i < 4; i++) T6[i] = T3[4 + i] + T3[i];
  const float v = (T6[0] + T6[2]) + (T6[1] + T6[3]);
  const int row = r0 + lane;
  unsigned long long key = row < vocab ? dsh_argmax_key(v, row) : 0ull;
  key = dsh_wave_max_u64(key);
  if (lane == 0) wbest[wave] = key;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long b = wbest[0];
    for (int i = 1; i < 4; i++) b = dsh_umax64(b, wbest[i]);
    cand[blockIdx.x] = b;
  }
}

// Final reduction of the candidates; writes tokens[*step] (or tokens[0]) and advances *step.
// The step index and a batch of 4 candidates per thread are loaded together (clamped addresses, no
// branches), so the kernel waits for one round trip per 1024 candidates. Also clears
// zero_p[0..zero_n) (16-byte aligned, zero_n % 4 == 0).
// The next decode step's input (ds_ocr.c:2271-2278): the BF16 embedding row of token tok widened
// by << 16; a token outside [0, emb_vocab) leaves the row as it was, as the reference's guard does.
// Called by all threads of the block with the same tok; H % 8 == 0.
__device__ __forceinline__ void embed_row(const uint16_t *__restrict__ emb, int emb_vocab, int H, int tok,
                                          float *__restrict__ out) {
  if (tok < 0 || tok >= emb_vocab) return;
  const uint16_t *r = emb + (size_t)tok * H;
  for (int i = 8 * (int)threadIdx.x; i < H; i += 8 * (int)blockDim.x) {
    const uint4 u = *(const uint4 *)(r + i);
    const unsigned w[4] = {u.x, u.y, u.z, u.w};
    f32x4 lo, hi;
    lo[0] = __uint_as_float(w[0] << 16), lo[1] = __uint_as_float(w[0] & 0xFFFF0000u);
    lo[2] = __uint_as_float(w[1] << 16), lo[3] = __uint_as_float(w[1] & 0xFFFF0000u);
    hi[0] = __uint_as_float(w[2] << 16), hi[1] = __uint_as_float(w[2] & 0xFFFF0000u);
    hi[2] = __uint_as_float(w[3] << 16), hi[3] = __uint_as_float(w[3] & 0xFFFF0000u);
    *(f32x4 *)(out + i) = lo;
    *(f32x4 *)(out + i + 4) = hi;
  }
}

// tokens[*step - 1]'s embedding into out (after the sampling rules changed the step's token).
__global__ void __launch_bounds__(256) k_embed_next(const int *__restrict__ tokens, const int *__restrict__ step,
                                                    const uint16_t *__restrict__ emb, int emb_vocab, int H,
                                                    float *__restrict__ out) {
  const int s = *step - 1;
  if (s >= 0) embed_row(emb, emb_vocab, H, tokens[s], out);
}

__global__ void __launch_bounds__(256) k_lm_argmax_final(const unsigned long long *__restrict__ cand, int n,
                                                         int *__restrict__ tokens, int *__restrict__ step,
                                                         float *__restrict__ zero_p, int zero_n,
                                                         const uint16_t *__restrict__ emb, int emb_vocab, int H,
                                                         float *__restrict__ emb_out) {
  for (int i = 4 * threadIdx.x; i < zero_n; i += 1024) *(f32x4 *)(zero_p + i) = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  __shared__ unsigned long long wbest[4];
  const int s = step ? *step : 0;
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
  __shared__ int s_tok;
  if (threadIdx.x == 0) {
    unsigned long long best = wbest[0];
    for (int i = 1; i < 4; i++) best = dsh_umax64(best, wbest[i]);
    const int tok = dsh_key_index(best);
    tokens[s] = tok;
    s_tok = tok;
    if (step) *step = s + 1;
  }
  if (emb_out) {
    __syncthreads();
    embed_row(emb, emb_vocab, H, s_tok, emb_out);
  }
}

// The step's final kernel fused with the next step's router partials (CFG routing, one-kernel
// layers). The LM head has advanced the step counter, so sn = *step is the next step and sn - 1
// the token's slot, the same in every block. Each block: the argmax of the LM head's candidates
// (redundantly, as k_lm_argmax_final: n is the head's block count), its share of the regions to
// clear, and R rows r0 .. r0 + R - 1 of the next step's input with their router partials in
// k_dec_partial_scores' order. The input is the token's embedding, widened and written to emb_out
// (emb_out left as it is for a token outside the table, as embed_row), or row sn of x_in; with
// sn >= rows there is no next step in the bound input and no partials are written.
template <int R>
__global__ void __launch_bounds__(64) k_lm_final_scores(const unsigned long long *__restrict__ cand, int n,
                                                        int *__restrict__ tokens, const int *__restrict__ step,
                                                        float *__restrict__ zero_p, int zero_n,
                                                        const uint16_t *__restrict__ emb, int emb_vocab,
                                                        float *__restrict__ emb_out, const float *__restrict__ x_in,
                                                        int stride, int rows, const float *__restrict__ WrT, int E,
                                                        float *__restrict__ partials) {
  const int lane = threadIdx.x, sn = *step, r0 = blockIdx.x * R;
  unsigned long long b = 0ull;
  for (int i0 = 0; i0 < n; i0 += 512) {
    unsigned long long c[8];
#pragma unroll
    for (int j = 0; j < 8; j++) c[j] = cand[min(i0 + lane + 64 * j, n - 1)];  // duplicates are harmless
#pragma unroll
    for (int j = 0; j < 8; j++) b = dsh_umax64(b, c[j]);
  }
  const int tok = dsh_key_index(dsh_wave_max_u64(b));
  if (blockIdx.x == 0 && lane == 0) tokens[sn - 1] = tok;
  for (int i = 4 * (blockIdx.x * 64 + lane); i < zero_n; i += 4 * 64 * (int)gridDim.x)
    *(f32x4 *)(zero_p + i) = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float xv[R];
  if (emb_out) {
    if (tok >= 0 && tok < emb_vocab) {
      const uint16_t *er = emb + (size_t)tok * (size_t)(gridDim.x * R) + r0;
#pragma unroll
      for (int j = 0; j < R; j++) xv[j] = __uint_as_float((unsigned)er[j] << 16);
      if (lane < R) emb_out[r0 + lane] = xv[lane];
    } else {
#pragma unroll
      for (int j = 0; j < R; j++) xv[j] = emb_out[r0 + j];
    }
  } else {
    if (sn >= rows) return;
    const float *x = x_in + (size_t)sn * stride + r0;
#pragma unroll
    for (int j = 0; j < R; j++) xv[j] = x[j];
  }
  float p = 0.0f;
  if (lane < E) {
    float w[R];
#pragma unroll
    for (int j = 0; j < R; j++) w[j] = WrT[(size_t)(r0 + j) * E + lane];
#pragma unroll
    for (int j = 0; j < R; j++) p = __builtin_fmaf(w[j], xv[j], p);
  }
  partials[(size_t)blockIdx.x * 64 + lane] = lane < E ? p : 0.0f;
}

// After the last step of a run whose steps end with the LM head: the pending token (the argmax of
// the last step's keys; the LM head has advanced the step counter) and the last copies regions.
__global__ void __launch_bounds__(256) k_lm_token_pending(const unsigned long long *__restrict__ cand, int n,
                                                         int *__restrict__ tokens, const int *__restrict__ step,
                                                         int *__restrict__ pending, float *__restrict__ zero_p,
                                                         int zero_n) {
  for (int i = 4 * (blockIdx.x * 256 + threadIdx.x); i < zero_n; i += 4 * 256 * (int)gridDim.x)
    *(f32x4 *)(zero_p + i) = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  if (blockIdx.x != 0 || threadIdx.x >= 64 || *pending == 0) return;
  const int lane = threadIdx.x;
  unsigned long long b = 0ull;
  for (int i = lane; i < n; i += 64) b = dsh_umax64(b, cand[i]);
  b = dsh_wave_max_u64(b);
  if (lane == 0) {
    tokens[*step - 1] = dsh_key_index(b);
    *pending = 0;
  }
}

// ============================================================================ launchers
// Rows per down block (and per router partial): keeps the partial count within 4 * ROUTE_BATCH.
static inline int dec_rows(int H) { return H <= 32 * ROUTE_BATCH ? 8 : 16; }
#define LM_D 1

extern "C" {

int dsh_dec_supported(int H, int I, int E, int K, int SI) {
  if (H % 256 || H / 256 > 8) return 0;           // gate_up: H == 256*CPL
  if (I % 16 || I / 16 > 64 || SI % I) return 0;  // down: one chunk per lane
  if (K + SI / I != 8 || H % dec_rows(H) || H / dec_rows(H) > 4 * ROUTE_BATCH) return 0;
  if (E > 64 || K > E) return 0;
  return 1;
}

int dsh_dec_partials(int H) { return H / dec_rows(H); }

int dsh_dec_partial_rows(int H) { return dec_rows(H); }

hipError_t dsh_launch_lm_token_pending(const unsigned long long *cand, int n, int *tokens, const int *step,
                                       int *pending, float *zero_p, int zero_n, hipStream_t s) {
  if (!cand || n <= 0 || !tokens || !step || !pending || ((uintptr_t)zero_p & 15) || zero_n % 4 || zero_n < 0)
    return hipErrorInvalidValue;
  k_lm_token_pending<<<max(1, min(16, (zero_n + 1023) / 1024)), 256, 0, s>>>(cand, n, tokens, step, pending, zero_p,
                                                                            zero_n);
  return hipGetLastError();
}

hipError_t dsh_launch_row_norms(const float *A, int rows, int cols, float *out, hipStream_t s) {
  if (rows <= 0 || cols <= 0) return hipErrorInvalidValue;
  k_row_norms<<<rows, 256, 0, s>>>(A, cols, out);
  return hipGetLastError();
}

hipError_t dsh_launch_transpose_f32(const float *src, float *dst, int rows, int cols, hipStream_t s) {
  k_transpose_f32<<<dim3((cols + 31) / 32, (rows + 31) / 32), 256, 0, s>>>(src, dst, rows, cols);
  return hipGetLastError();
}

hipError_t dsh_launch_dec_partial_scores(const float *WrT, const float *x_in, const int *step, int stride, int H, int E,
                                         float *partials, hipStream_t s) {
  if (dec_rows(H) == 8)
    k_dec_partial_scores<8><<<H / 8, 64, 0, s>>>(WrT, x_in, step, stride, H, E, partials);
  else
    k_dec_partial_scores<16><<<H / 16, 64, 0, s>>>(WrT, x_in, step, stride, H, E, partials);
  return hipGetLastError();
}

hipError_t dsh_launch_dec_scores_bf16_copies(const uint16_t *Wr, const float *x_in, const int *step, int stride,
                                             int ncopies, int H, int E, int nthreads, float *partials, hipStream_t s) {
  const int blocks = (E + 15) / 16, chunk = dsh_chunk_len(E, nthreads);
  if (ncopies != 1 && (ncopies != 8 || step)) return hipErrorInvalidValue;
#define SC(N)                                                                                             \
  case N:                                                                                                 \
    k_dec_scores_bf16<8 * N><<<blocks, 64, 0, s>>>(Wr, x_in, step, stride, E, chunk, partials, ncopies); \
    break;
  if (H % 256) return hipErrorInvalidValue;
  switch (H / 256) {
    SC(1) SC(2) SC(3) SC(4) SC(5) SC(6) SC(7) SC(8)
    default:
      return hipErrorInvalidValue;
  }
#undef SC
  return hipGetLastError();
}

hipError_t dsh_launch_dec_scores_bf16(const uint16_t *Wr, const float *x_in, const int *step, int stride, int H, int E,
                                      int nthreads, float *partials, hipStream_t s) {
  return dsh_launch_dec_scores_bf16_copies(Wr, x_in, step, stride, 1, H, E, nthreads, partials, s);
}

static int dec_gate_up_blocks(const dsh_layer_t *L) {
  return max((L->SI + 3) / 4, (L->K * L->I + 11) / 12);
}

hipError_t dsh_launch_dec_scores_f32_exact(const float *WrT, const float *x_in, const int *step, int stride, int H,
                                          int E, float *partials, hipStream_t s) {
  if (H <= 0 || H > 2048 || E <= 0 || E > 64) return hipErrorInvalidValue;
  k_dec_scores_f32_exact<<<1, 64, 0, s>>>(WrT, x_in, step, stride, H, E, partials);
  return hipGetLastError();
}

hipError_t dsh_launch_dec_gate_up(const dsh_layer_t *L, const float *x_in, const int *step, int stride,
                                  const float *partials, int np, int route_mode, int bf16sim,
                                  const dsh_layer_work_t *wk, const dsh_rcert_t *rc, hipStream_t s) {
  const dsh_rcert_t rc0 = {nullptr, nullptr, 0, 0};
  if (!rc) rc = &rc0;
  if (route_mode == DSH_ROUTE_CFG && !bf16sim && np > 1 && (!L->router_norm || !L->router_f32))
    return hipErrorInvalidValue;
  if (bf16sim) {  // every rounded value in the reference's order
    if (L->H > 2048 || L->H % 16) return hipErrorInvalidValue;
    k_sim_gate_up<<<(L->K * L->I + L->SI + 127) / 128, 320, 0, s>>>(*L, x_in, step, stride, partials, np, route_mode,
                                                                    *wk);
    return hipGetLastError();
  }
  const int blocks = dec_gate_up_blocks(L);
#define GU(N)                                                                                                  \
  case N:                                                                                                      \
    k_dec_gate_up<N><<<blocks, 256, 0, s>>>(*L, x_in, step, stride, partials, np, route_mode, bf16sim, *wk, *rc); \
    break;
  switch (L->H / 256) {
    GU(1) GU(2) GU(3) GU(4) GU(5) GU(6) GU(7) GU(8)
    default:
      return hipErrorInvalidValue;
  }
#undef GU
  return hipGetLastError();
}

hipError_t dsh_launch_dec_down(const dsh_layer_t *L, const float *x_in, const int *step, int stride, float *x_out,
                               int residual, const float *resid, int bf16sim, const dsh_layer_work_t *wk,
                               const float *WrT_next, int E_next, float *partials_next, hipStream_t s) {
  if (bf16sim) {  // every rounded value in the reference's order, then the combine
    if (L->H % 64 || L->I % 16 || L->SI % 16 || L->SI > 7 * 1024 || !wk->eo) return hipErrorInvalidValue;
    k_sim_down<<<dim3(L->H / 64, L->K + 1), 128, 0, s>>>(*L, *wk);
    if (dec_rows(L->H) == 8)
      k_sim_combine<8><<<L->H / 8, 64, 0, s>>>(*L, x_in, step, stride, x_out, residual, resid, *wk, WrT_next, E_next,
                                                partials_next);
    else
      k_sim_combine<16><<<L->H / 16, 64, 0, s>>>(*L, x_in, step, stride, x_out, residual, resid, *wk, WrT_next,
                                                  E_next, partials_next);
    return hipGetLastError();
  }
  if (dec_rows(L->H) == 8)
    k_dec_down<8><<<L->H / 8, 512, 0, s>>>(*L, x_in, step, stride, x_out, residual, resid, bf16sim, *wk, WrT_next,
                                           E_next, partials_next);
  else
    k_dec_down<16><<<L->H / 16, 512, 0, s>>>(*L, x_in, step, stride, x_out, residual, resid, bf16sim, *wk, WrT_next,
                                             E_next, partials_next);
  return hipGetLastError();
}

int dsh_dec_lm_blocks(int vocab) { return (vocab + 255) / 256; }

int dsh_dec_lm_supported(int in_dim) { return in_dim > 0 && in_dim % 64 == 0; }

// The one-row-per-lane kernel computes every row in the 4-row-group order; the reference takes
// that order only for rows inside a whole group of 4 of its thread's chunk.
int dsh_dec_lm_eligible(const void *W, int in_dim, int vocab, int nthreads) {
  if (!dsh_dec_lm_supported(in_dim) || ((uintptr_t)W & 15) || vocab <= 0) return 0;
  const int chunk = dsh_chunk_len(vocab, nthreads);
  for (int s0 = 0; s0 < vocab; s0 += chunk)
    if (min(chunk, vocab - s0) % 4) return 0;
  return 1;
}

hipError_t dsh_launch_lm_final_scores(const unsigned long long *cand, int n, int *tokens, const int *step,
                                      float *zero_p, int zero_n, const uint16_t *emb, int emb_vocab, float *emb_out,
                                      const float *x_in, int stride, int rows, const float *WrT, int H, int E,
                                      float *partials, hipStream_t s) {
  if (((uintptr_t)zero_p & 15) || zero_n % 4 || zero_n < 0 || n <= 0 || E <= 0 || E > 64 || H % dec_rows(H))
    return hipErrorInvalidValue;
  if (emb_out ? (!emb || emb_vocab <= 0) : (!x_in || rows <= 0 || stride < 0)) return hipErrorInvalidValue;
  if (dec_rows(H) == 8)
    k_lm_final_scores<8><<<H / 8, 64, 0, s>>>(cand, n, tokens, step, zero_p, zero_n, emb, emb_vocab, emb_out, x_in,
                                             stride, rows, WrT, E, partials);
  else
    k_lm_final_scores<16><<<H / 16, 64, 0, s>>>(cand, n, tokens, step, zero_p, zero_n, emb, emb_vocab, emb_out, x_in,
                                               stride, rows, WrT, E, partials);
  return hipGetLastError();
}

hipError_t dsh_launch_lm_argmax_final(const unsigned long long *cand, int n, int *tokens, int *step, float *zero_p,
                                      int zero_n, const uint16_t *emb, int emb_vocab, int H, float *emb_out,
                                      hipStream_t s) {
  if (((uintptr_t)zero_p & 15) || zero_n % 4 || zero_n < 0 || n <= 0) return hipErrorInvalidValue;
  if (emb_out && (!emb || emb_vocab <= 0 || H <= 0 || H % 8 || ((uintptr_t)emb & 15) || ((uintptr_t)emb_out & 15)))
    return hipErrorInvalidValue;
  k_lm_argmax_final<<<1, 256, 0, s>>>(cand, n, tokens, step, zero_p, zero_n, emb, emb_vocab, H, emb_out);
  return hipGetLastError();
}

hipError_t dsh_launch_embed_next(const int *tokens, const int *step, const uint16_t *emb, int emb_vocab, int H,
                                 float *out, hipStream_t s) {
  if (!tokens || !step || !emb || !out || emb_vocab <= 0 || H <= 0 || H % 8 || ((uintptr_t)emb & 15) ||
      ((uintptr_t)out & 15))
    return hipErrorInvalidValue;
  k_embed_next<<<1, 256, 0, s>>>(tokens, step, emb, emb_vocab, H, out);
  return hipGetLastError();
}

// depth: lines of loads in flight per lane (1, 2 or 4; must divide in_dim/64).
hipError_t dsh_launch_dec_lm_argmax_depth(const uint16_t *W, const float *x, int in_dim, int vocab,
                                          unsigned long long *cand, int depth, hipStream_t s) {
  if (!dsh_dec_lm_supported(in_dim) || ((uintptr_t)W & 15) || vocab <= 0) return hipErrorInvalidValue;
  if ((in_dim / 64) % depth) return hipErrorInvalidValue;
  const int nb = dsh_dec_lm_blocks(vocab);
  switch (depth) {
    case 1:
      k_dec_lm_argmax<1, 0><<<nb, 256, 0, s>>>(W, x, in_dim, vocab, cand, nullptr, nullptr);
      break;
    case 2:
      k_dec_lm_argmax<2, 0><<<nb, 256, 0, s>>>(W, x, in_dim, vocab, cand, nullptr, nullptr);
      break;
    case 4:
      k_dec_lm_argmax<4, 0><<<nb, 256, 0, s>>>(W, x, in_dim, vocab, cand, nullptr, nullptr);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t dsh_launch_dec_lm_argmax_copies(const uint16_t *W, const float *xc, int ncopies, int in_dim, int vocab,
                                           unsigned long long *cand, float *x_out, int *step_inc, hipStream_t s) {
  if (!dsh_dec_lm_supported(in_dim) || in_dim > 2048 || ((uintptr_t)W & 15) || vocab <= 0 || ncopies != 8)
    return hipErrorInvalidValue;
  k_dec_lm_argmax<1, 8><<<dsh_dec_lm_blocks(vocab), 256, 0, s>>>(W, xc, in_dim, vocab, cand, x_out, step_inc);
  return hipGetLastError();
}

hipError_t dsh_launch_dec_lm_argmax(const uint16_t *W, const float *x, int in_dim, int vocab,
                                    unsigned long long *cand, hipStream_t s) {
  const int nt = in_dim / 64;
  const int depth = nt % LM_D == 0 ? LM_D : (nt % 2 == 0 ? 2 : 1);
  return dsh_launch_dec_lm_argmax_depth(W, x, in_dim, vocab, cand, depth, s);
}

}  // extern "C"
