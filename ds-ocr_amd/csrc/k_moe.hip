// k_moe.hip — device-resident decode MoE layer (batch 1) and the streaming LM-head argmax.
//
// One layer is three kernels on one stream (captured into a hipGraph by the decode stack):
//   scores  : router scores for all experts (ds_moe_router / ds_moe_router_bf16)
//   gate_up : routing (softmax/top-k) + fused gate_up INT8 dequant-matvec + SwiGLU for the top-k
//             routed experts and the shared expert (ds_expert_forward_fused_int4 first half)
//   down    : down INT8 dequant-matvec for every selected expert and the shared expert, weighted
//             combine in top-k order, shared add and residual (ds_expert_combine, ds_vec_add)
// Reference: moe_forward INT8 branch, ds_moe_decoder.c:131-278.
//
// Numerics: codes are read as u = q+128 bytes (XOR 0x80) and multiplied in f32; each row is
// scale*Σu·x + offset*Σx with Σx computed once per vector (the reference recomputes it per row,
// ds_quantize.c:163-169). Routing, the fast-exp SiLU, BF16 truncation and the combine/shared/
// residual arithmetic follow the reference operation by operation; only the dot-product
// summation order differs (GPU tree instead of one sequential chain).
#include "dsh_avx.h"
#include "k_core.h"

// ============================================================================ routing (wave 0)
// Same semantics as k_core.hip's topk helpers, writing to LDS for the block.
__device__ void route_wave(const float *scores, int n, int k, int mode, int *s_idx, float *s_w) {
  const int lane = threadIdx.x & 63;
  float s = lane < n ? scores[lane] : 0.0f;
  bool taken = false;
  if (mode == DSH_ROUTE_CFG) {
    int my_sel = 0;
    float my_ss = 0.0f;
    int ns = 0;
    for (int t = 0; t < k; t++) {
      unsigned long long key = (lane < n && !taken) ? dsh_argmax_key(s, lane) : 0ull;
      key = dsh_wave_max_u64(key);
      if (key == 0ull) continue;
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
    float ev = lane < ns ? expf(my_ss - mx) : 0.0f;
    float sum = 0.0f;
    for (int j = 0; j < ns; j++) sum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ev), j));
    float inv = 1.0f / sum;
    if (lane < k) {
      s_idx[lane] = lane < ns ? my_sel : 0;
      s_w[lane] = lane < ns ? ev * inv : 0.0f;
    }
  } else {
    float m = (lane < n && s > -1e30f) ? s : -1e30f;
    m = dsh_wave_max(m);
    float p = lane < n ? dsh_fast_expf(s - m) : 0.0f;
    float sum = 0.0f;
    for (int e = 0; e < n; e++) sum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), e));
    float inv = 1.0f / sum;
    p = p * inv;
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
      s_idx[lane] = my_sel;
      s_w[lane] = my_w;
    }
  }
}

// (scale, offset) pair i of an interleaved array.
__device__ __forceinline__ float2 SO(const float *so, size_t i) { return ((const float2 *)so)[i]; }

__device__ __forceinline__ const float *step_ptr(const float *x, const int *step, int stride) {
  return step ? x + (size_t)(*step) * stride : x;
}

// ============================================================================ scores
// CFG mode: f32 router rows, 16 lanes per expert, float4 chunks (own summation order).
__global__ void __launch_bounds__(256) k_moe_scores_f32(const float *__restrict__ Wr, const float *__restrict__ x_in,
                                                        const int *__restrict__ step, int stride, int H, int E,
                                                        float *__restrict__ scores) {
  const float *x = step_ptr(x_in, step, stride);
  const int lane = threadIdx.x & 63, sub = lane & 15;
  const int e = blockIdx.x * 16 + (threadIdx.x >> 4);
  float acc = 0.0f;
  if (e < E) {
    const float *w = Wr + (size_t)e * H;
    for (int c = sub; c < (H >> 2); c += 16) {
      f32x4 wv = __builtin_nontemporal_load((const f32x4 *)(w + 4 * c));
      f32x4 xv = dsh_load_f4(x + 4 * c);
      acc = __builtin_fmaf(wv[0], xv[0], acc);
      acc = __builtin_fmaf(wv[1], xv[1], acc);
      acc = __builtin_fmaf(wv[2], xv[2], acc);
      acc = __builtin_fmaf(wv[3], xv[3], acc);
    }
  }
  acc = dsh_row16_sum(acc);
  if (e < E && sub == 0) scores[e] = acc;
}

// DECODE mode: bf16 router in the reference's AVX-512 order (bit-exact scores), 16 experts per
// 64-thread block, x staged in LDS.
__global__ void __launch_bounds__(64) k_moe_scores_bf16(const uint16_t *__restrict__ Wr, const float *__restrict__ x_in,
                                                        const int *__restrict__ step, int stride, int H, int E,
                                                        int chunk, float *__restrict__ scores) {
  extern __shared__ float xs[];
  const float *x = step_ptr(x_in, step, stride);
  for (int i = threadIdx.x; i < H; i += 64) xs[i] = x[i];
  __syncthreads();
  const int L = threadIdx.x & 3;
  const int e = blockIdx.x * 16 + (threadIdx.x >> 2);
  if (e >= E) return;
  int path = row_path(e, E, chunk, false);
  float v = avx_row<true>(Wr + (size_t)e * H, xs, H, L, path == DSH_ROW_SINGLE, true, 0.0f, path != DSH_ROW_GROUP4);
  if (L == 0) scores[e] = v;
}

// ============================================================================ gate_up + SwiGLU
// Units: one SwiGLU output h[u] = silu(gate_row·x) * (up_row·x). Shared-expert units come first
// (they need no routing and start streaming at once), then routed slot k, intermediate i.
// 16 lanes per unit; lane sub reads 16-byte chunks sub, sub+16, ... of both rows (CPL chunks).
template <int CPL>
__global__ void __launch_bounds__(256) k_moe_gate_up(dsh_layer_t L, const float *__restrict__ x_in,
                                                     const int *__restrict__ step, int stride, int mode, int bf16sim,
                                                     dsh_layer_work_t wk) {
  __shared__ int s_idx[64];
  __shared__ float s_w[64];
  const float *x = step_ptr(x_in, step, stride);
  const int H = L.H, I = L.I, K = L.K, SI = L.SI;
  const int C = H >> 4;
  const int lane = threadIdx.x & 63, sub = lane & 15;
  const int unit0 = blockIdx.x * 16;  // first unit of the block
  const int total = K * I + SI;
  const bool need_route = unit0 + 15 >= SI;
  if (need_route && threadIdx.x < 64) {
    route_wave(wk.scores, L.E, K, mode, s_idx, s_w);
    if (unit0 <= SI && SI < unit0 + 16 && lane < K) {  // the block holding routed unit 0 publishes
      wk.idx[lane] = s_idx[lane];
      wk.w[lane] = s_w[lane];
    }
  }
  // x chunks of this lane (same for every unit) and the vector sum Σx.
  float xv[CPL][16];
  float xpart = 0.0f;
#pragma unroll
  for (int m = 0; m < CPL; m++) {
    int ch = sub + 16 * m;
    if (ch < C) {
#pragma unroll
      for (int d = 0; d < 4; d++) {
        f32x4 t = dsh_load_f4(x + 16 * ch + 4 * d);
        xv[m][4 * d] = t[0];
        xv[m][4 * d + 1] = t[1];
        xv[m][4 * d + 2] = t[2];
        xv[m][4 * d + 3] = t[3];
      }
      float s = 0.0f;
#pragma unroll
      for (int j = 0; j < 16; j++) s += xv[m][j];
      xpart += s;
    } else {
#pragma unroll
      for (int j = 0; j < 16; j++) xv[m][j] = 0.0f;
    }
  }
  const float xsum = dsh_row16_sum(xpart);
  if (need_route) __syncthreads();

  const int u = unit0 + (threadIdx.x >> 4);
  if (u >= total) return;
  const int8_t *grow, *urow;
  float2 sog, sou;
  int hpos;
  if (u < SI) {
    grow = L.sgu_q + (size_t)u * H;
    urow = L.sgu_q + (size_t)(SI + u) * H;
    sog = SO(L.sgu_so, u);
    sou = SO(L.sgu_so, SI + u);
    hpos = K * I + u;
  } else {
    int r = u - SI, k = r / I, i = r - k * I;
    int e = s_idx[k];
    hpos = r;
    if (e < 0) {
      if (sub == 0) wk.h[hpos] = 0.0f;
      return;
    }
    size_t base = (size_t)e * 2 * I;
    grow = L.gu_q + (base + i) * H;
    urow = L.gu_q + (base + I + i) * H;
    sog = SO(L.gu_so, base + i);
    sou = SO(L.gu_so, base + I + i);
  }
  u32x4 wg[CPL], wu[CPL];
#pragma unroll
  for (int m = 0; m < CPL; m++) {
    int ch = sub + 16 * m;
    if (ch < C) {
      wg[m] = dsh_load_nt(grow + 16 * ch);
      wu[m] = dsh_load_nt(urow + 16 * ch);
    }
  }
  float dg = 0.0f, du = 0.0f;
#pragma unroll
  for (int m = 0; m < CPL; m++) {
    int ch = sub + 16 * m;
    if (ch < C) {
      dg = dsh_dot16_u8(wg[m], xv[m], dg);
      du = dsh_dot16_u8(wu[m], xv[m], du);
    }
  }
  dg = dsh_row16_sum(dg);
  du = dsh_row16_sum(du);
  if (sub == 0) {
    float g = __builtin_fmaf(sog.x, dg, sog.y * xsum);
    float up = __builtin_fmaf(sou.x, du, sou.y * xsum);
    if (bf16sim) {
      g = dsh_bf16_round_half_up(g);
      up = dsh_bf16_round_half_up(up);
    }
    float hv = dsh_swiglu(g, up);
    if (bf16sim) hv = dsh_bf16_round_half_up(hv);
    wk.h[hpos] = hv;
  }
}

// ============================================================================ down + combine
// One wave per RPW output rows; 8 segments of 8 lanes: segments 0..K-1 are the routed slots,
// K..7 the shared expert's I-wide column blocks. Lane sub reads chunks sub, sub+8, ... (CPLD).
// Combine (ds_kernels.c:359-371), shared add (ds_vec_add) and residual follow the reference order.
template <int CPLD, int RPW>
__global__ void __launch_bounds__(64) k_moe_down(dsh_layer_t L, const float *__restrict__ x_in,
                                                 const int *__restrict__ step, int stride, float *__restrict__ x_out,
                                                 int residual, int bf16sim, dsh_layer_work_t wk) {
  const float *x = step_ptr(x_in, step, stride);
  const int H = L.H, I = L.I, K = L.K, SI = L.SI;
  const int lane = threadIdx.x & 63, seg = lane >> 3, sub = lane & 7;
  const int CI = I >> 4;
  const int hbase = seg < K ? seg * I : K * I + (seg - K) * I;
  const int e = seg < K ? wk.idx[seg] : -2;
  // h chunks of this lane and the segment sum Σh.
  float hv[CPLD][16];
  float hpart = 0.0f;
#pragma unroll
  for (int m = 0; m < CPLD; m++) {
    int ch = sub + 8 * m;
    if (ch < CI) {
#pragma unroll
      for (int d = 0; d < 4; d++) {
        f32x4 t = dsh_load_f4(wk.h + hbase + 16 * ch + 4 * d);
        hv[m][4 * d] = t[0];
        hv[m][4 * d + 1] = t[1];
        hv[m][4 * d + 2] = t[2];
        hv[m][4 * d + 3] = t[3];
      }
      float s = 0.0f;
#pragma unroll
      for (int j = 0; j < 16; j++) s += hv[m][j];
      hpart += s;
    } else {
#pragma unroll
      for (int j = 0; j < 16; j++) hv[m][j] = 0.0f;
    }
  }
  const float hsum = dsh_row8_sum(hpart);
  float wgt[8];
#pragma unroll
  for (int k = 0; k < 8; k++) wgt[k] = k < K ? wk.w[k] : 0.0f;

  const int r0 = blockIdx.x * RPW;
#pragma unroll
  for (int rr = 0; rr < RPW; rr++) {
    const int r = r0 + rr;
    if (r >= H) break;
    const int8_t *wrow = nullptr;
    float2 so = make_float2(0.0f, 0.0f);
    if (seg < K) {
      if (e >= 0) {
        wrow = L.dn_q + ((size_t)e * H + r) * I;
        so = SO(L.dn_so, (size_t)e * H + r);
      }
    } else {
      wrow = L.sdn_q + (size_t)r * SI + (size_t)(seg - K) * I;
      so = SO(L.sdn_so, r);
    }
    float dot = 0.0f;
    if (wrow) {
      u32x4 wv[CPLD];
#pragma unroll
      for (int m = 0; m < CPLD; m++) {
        int ch = sub + 8 * m;
        if (ch < CI) wv[m] = dsh_load_nt(wrow + 16 * ch);
      }
#pragma unroll
      for (int m = 0; m < CPLD; m++) {
        int ch = sub + 8 * m;
        if (ch < CI) dot = dsh_dot16_u8(wv[m], hv[m], dot);
      }
    }
    dot = dsh_row8_sum(dot);
    // Routed slot value e_k = scale*dot + off*Σh on lanes 8k; shared parts summed below.
    float ek = (seg < K && e >= 0) ? __builtin_fmaf(so.x, dot, so.y * hsum) : 0.0f;
    float out = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; k++) {
      float v = __shfl(ek, 8 * k);
      if (k < K) {
        if (bf16sim) v = dsh_bf16_round_half_up(v);
        out = __builtin_fmaf(wgt[k], v, out);
      }
    }
    float sdot = 0.0f, shs = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; k++) {
      float d = __shfl(dot, 8 * k), hsv = __shfl(hsum, 8 * k);
      if (k >= K) {
        sdot += d;
        shs += hsv;
      }
    }
    float2 sso = make_float2(__shfl(so.x, 8 * K), __shfl(so.y, 8 * K));
    float sh = __builtin_fmaf(sso.x, sdot, sso.y * shs);
    if (bf16sim) sh = dsh_bf16_round_half_up(sh);
    out = out + sh;
    if (lane == 0) x_out[r] = residual ? x[r] + out : out;
  }
}

// ============================================================================ LM-head argmax
// Streaming argmax_r (W_r · x) over bf16 rows in the reference's AVX-512 2-accumulator order
// (bit-exact logits, ds_kernels_avx.c:157-228), never materialising logits. Requirements checked
// by the host: in_dim % 32 == 0, 16-byte aligned rows, and every CPU chunk length a multiple of 4
// (so every row takes the 2-accumulator path). A 4-lane group owns R rows and walks them in
// lockstep so each x chunk read from LDS serves R rows; lane L owns chains 8L..8L+7.
template <int R>
__global__ void __launch_bounds__(256) k_lm_argmax(const uint16_t *__restrict__ W, const float *__restrict__ x,
                                                   int in_dim, int vocab, unsigned long long *__restrict__ cand) {
  extern __shared__ float xs[];
  __shared__ unsigned long long wbest[4];
  for (int i = threadIdx.x; i < in_dim; i += 256) xs[i] = x[i];
  __syncthreads();
  const int L = threadIdx.x & 3;
  const int g = threadIdx.x >> 2;
  // Rows of group g: rbase + j*64 for j < R (adjacent groups read adjacent rows).
  const int rbase = blockIdx.x * (64 * R) + g;
  float acc[R][8];
#pragma unroll
  for (int j = 0; j < R; j++)
#pragma unroll
    for (int c = 0; c < 8; c++) acc[j][c] = 0.0f;
  const uint16_t *wp[R];
  bool ok[R];
#pragma unroll
  for (int j = 0; j < R; j++) {
    int r = rbase + j * 64;
    ok[j] = r < vocab;
    wp[j] = W + (size_t)(ok[j] ? r : 0) * in_dim + 8 * L;
  }
  const int T = in_dim >> 5;
  constexpr int U = 4;
  int t = 0;
  for (; t + U <= T; t += U) {
    u32x4 wv[U][R];
#pragma unroll
    for (int u = 0; u < U; u++)
#pragma unroll
      for (int j = 0; j < R; j++) wv[u][j] = dsh_load_nt(wp[j] + 32 * (t + u));
#pragma unroll
    for (int u = 0; u < U; u++) {
      const float *xp = xs + 32 * (t + u) + 8 * L;
      f32x4 x0 = *(const f32x4 *)xp, x1 = *(const f32x4 *)(xp + 4);
      float xf[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
#pragma unroll
      for (int j = 0; j < R; j++)
#pragma unroll
        for (int d = 0; d < 4; d++) {
          acc[j][2 * d] = __builtin_fmaf(dsh_bf16lo(wv[u][j][d]), xf[2 * d], acc[j][2 * d]);
          acc[j][2 * d + 1] = __builtin_fmaf(dsh_bf16hi(wv[u][j][d]), xf[2 * d + 1], acc[j][2 * d + 1]);
        }
    }
  }
  for (; t < T; t++) {
    const float *xp = xs + 32 * t + 8 * L;
    f32x4 x0 = *(const f32x4 *)xp, x1 = *(const f32x4 *)(xp + 4);
    float xf[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
#pragma unroll
    for (int j = 0; j < R; j++) {
      u32x4 wv = dsh_load_nt(wp[j] + 32 * t);
#pragma unroll
      for (int d = 0; d < 4; d++) {
        acc[j][2 * d] = __builtin_fmaf(dsh_bf16lo(wv[d]), xf[2 * d], acc[j][2 * d]);
        acc[j][2 * d + 1] = __builtin_fmaf(dsh_bf16hi(wv[d]), xf[2 * d + 1], acc[j][2 * d + 1]);
      }
    }
  }
  unsigned long long key = 0ull;
#pragma unroll
  for (int j = 0; j < R; j++) {
    float A[8], T3[8], T6[4];
#pragma unroll
    for (int c = 0; c < 8; c++) A[c] = acc[j][c] + __shfl_down(acc[j][c], 2, 4);
#pragma unroll
    for (int c = 0; c < 8; c++) T3[c] = __shfl_down(A[c], 1, 4) + A[c];
#pragma unroll
    for (int c = 0; c < 4; c++) T6[c] = T3[4 + c] + T3[c];
    float v = (T6[0] + T6[2]) + (T6[1] + T6[3]);
    if (L == 0 && ok[j]) key = dsh_umax64(key, dsh_argmax_key(v, rbase + j * 64));
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

// Final reduction of the candidates; writes tokens[*step] (or tokens[0]) and advances *step.
__global__ void __launch_bounds__(256) k_lm_argmax_final(const unsigned long long *__restrict__ cand, int n,
                                                         int *__restrict__ tokens, int *__restrict__ step) {
  __shared__ unsigned long long wbest[4];
  unsigned long long b = 0ull;
  for (int i = threadIdx.x; i < n; i += 256) b = dsh_umax64(b, cand[i]);
  b = dsh_wave_max_u64(b);
  if ((threadIdx.x & 63) == 0) wbest[threadIdx.x >> 6] = b;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int i = 1; i < 4; i++) wbest[0] = dsh_umax64(wbest[0], wbest[i]);
    int s = step ? *step : 0;
    tokens[s] = dsh_key_index(wbest[0]);
    if (step) *step = s + 1;
  }
}

// ============================================================================ launchers
#define LM_R 4

extern "C" {

int dsh_moe_fast_shape(int H, int I, int E, int K, int SI) {
  if (H % 16 || I % 128 || SI % I) return 0;
  if (K + SI / I != 8) return 0;
  if (H / 16 > 16 * 8) return 0;   // CPL <= 8
  if (I / 16 / 8 > 8) return 0;    // CPLD <= 8
  if (E > 64 || K > E || H > 16384) return 0;
  return 1;
}

hipError_t dsh_launch_moe_scores(const dsh_layer_t *L, const float *x_in, const int *step, int step_stride,
                                 int route_mode, int nthreads, float *scores, hipStream_t s) {
  if (route_mode == DSH_ROUTE_CFG) {
    k_moe_scores_f32<<<(L->E + 15) / 16, 256, 0, s>>>(L->router_f32, x_in, step, step_stride, L->H, L->E, scores);
  } else {
    k_moe_scores_bf16<<<(L->E + 15) / 16, 64, (size_t)L->H * 4, s>>>(L->router_bf16, x_in, step, step_stride, L->H,
                                                                       L->E, dsh_chunk_len(L->E, nthreads), scores);
  }
  return hipGetLastError();
}

hipError_t dsh_launch_moe_gate_up(const dsh_layer_t *L, const float *x_in, const int *step, int step_stride,
                                  int route_mode, int bf16sim, const dsh_layer_work_t *wk, hipStream_t s) {
  int total = L->K * L->I + L->SI;
  int blocks = (total + 15) / 16;
  int cpl = (L->H / 16 + 15) / 16;
#define GU(N)                                                                                                  \
  case N:                                                                                                      \
    k_moe_gate_up<N><<<blocks, 256, 0, s>>>(*L, x_in, step, step_stride, route_mode, bf16sim, *wk);            \
    break;
  switch (cpl) {
    GU(1) GU(2) GU(3) GU(4) GU(5) GU(6) GU(7) GU(8)
    default:
      return hipErrorInvalidValue;
  }
#undef GU
  return hipGetLastError();
}

hipError_t dsh_launch_moe_down(const dsh_layer_t *L, const float *x_in, const int *step, int step_stride,
                               float *x_out, int residual, int bf16sim, const dsh_layer_work_t *wk, hipStream_t s) {
  constexpr int RPW = 2;
  int blocks = (L->H + RPW - 1) / RPW;
  int cpld = (L->I / 16 + 7) / 8;
#define DN(N)                                                                                                       \
  case N:                                                                                                           \
    k_moe_down<N, RPW><<<blocks, 64, 0, s>>>(*L, x_in, step, step_stride, x_out, residual, bf16sim, *wk);           \
    break;
  switch (cpld) {
    DN(1) DN(2) DN(3) DN(4) DN(5) DN(6) DN(7) DN(8)
    default:
      return hipErrorInvalidValue;
  }
#undef DN
  return hipGetLastError();
}

int dsh_lm_argmax_blocks(int vocab) { return (vocab + 64 * LM_R - 1) / (64 * LM_R); }

hipError_t dsh_launch_lm_argmax_partial(const uint16_t *W, const float *x, int in_dim, int vocab,
                                        unsigned long long *cand, hipStream_t s) {
  if (in_dim % 32 || ((uintptr_t)W & 15) || in_dim * 4 > 64 * 1024) return hipErrorInvalidValue;
  int blocks = dsh_lm_argmax_blocks(vocab);
  k_lm_argmax<LM_R><<<blocks, 256, (size_t)in_dim * 4, s>>>(W, x, in_dim, vocab, cand);
  return hipGetLastError();
}

hipError_t dsh_launch_lm_argmax_final(const unsigned long long *cand, int n, int *tokens, int *step, hipStream_t s) {
  k_lm_argmax_final<<<1, 256, 0, s>>>(cand, n, tokens, step);
  return hipGetLastError();
}

}  // extern "C"
