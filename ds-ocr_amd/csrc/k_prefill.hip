// k_prefill.hip — prefill MoE block (T tokens) for the device-resident layer: routing, an
// expert-sorted grouped GEMM on bf16 MFMA with INT8 weights dequantized in registers, SwiGLU, the
// down projection and a deterministic combine (ds_moe_decoder.c:629-809 is the reference block; it
// runs sgemm on bf16 weights, this build runs the same layer's INT8 blocks).
//
// Numerics. Codes u = q + 128 (0..255) are exact in bf16. Each f32 activation a is split into
// hi = bf16(a) and lo = bf16(a - hi), so a = hi + lo to about 2^-17 relative, and
// Σ u·a = Σ u·hi + Σ u·lo is accumulated by the MFMA in f32 (products exact). The epilogue folds the
// row's scale and offset exactly as the decode path does: y = scale · Σu·a + offset · Σa.
//
// Kernels (one launch each, all sizes fixed by T, so a graph can hold them):
//   k_pf_split   X → Xhi, Xlo (bf16), Σx per token
//   k_pf_route   router scores in the decode path's order + top-k per token → idx, w
//   k_pf_plan    per-expert counts and offsets, the GEMM work list (expert, 64-row chunk)
//   k_pf_scatter expert-sorted (token, slot) pairs, tokens in increasing order per expert
//   k_pf_gate_up grouped GEMM + SwiGLU → H (bf16 hi/lo) for routed pairs and for the shared expert
//   k_pf_down    grouped GEMM → Y (f32) per routed pair and per token for the shared expert
//   k_pf_combine out[t] = (residual ? x : 0) + (Σ_k w_k·Y_k in ascending expert order + Y_shared)
#include "dsh_avx.h"
#include "dsh_route.h"
#include "k_core.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

#define PF_MT 64   // tokens (rows of A) per work item
#define PF_GU_N 128 // gate_up: intermediate units per block (128 gate + 128 up weight rows)
#define PF_DN_N 256 // down: output rows per block

struct pf_item {
  int seg;   // expert 0..E-1, or E for the shared expert
  int m0;    // first row of the chunk within the segment
  int mcnt;  // rows in the chunk (1..PF_MT)
  int pos0;  // first routed pair position of the segment (routed only)
};

// ---------------------------------------------------------------------------------- helpers
__device__ __forceinline__ bf16x8 codes_to_bf16(u32x2 v) {
  // stored codes are q = u - 128; u = byte ^ 0x80 is exact in bf16
  const uint32_t a = v[0] ^ 0x80808080u, b = v[1] ^ 0x80808080u;
  bf16x8 r;
  r[0] = (__bf16)(float)(a & 0xFF);
  r[1] = (__bf16)(float)((a >> 8) & 0xFF);
  r[2] = (__bf16)(float)((a >> 16) & 0xFF);
  r[3] = (__bf16)(float)(a >> 24);
  r[4] = (__bf16)(float)(b & 0xFF);
  r[5] = (__bf16)(float)((b >> 8) & 0xFF);
  r[6] = (__bf16)(float)((b >> 16) & 0xFF);
  r[7] = (__bf16)(float)(b >> 24);
  return r;
}

__device__ __forceinline__ bf16x8 ld_bf16x8(const __bf16 *p) { return *(const bf16x8 *)p; }

// D[m][n] of a 32x32 MFMA tile held by lane l, register j: n = l % 32, m = 8*(j/4) + 4*(l/32) + j%4
__device__ __forceinline__ int mfma_row(int lane, int j) { return 8 * (j >> 2) + 4 * (lane >> 5) + (j & 3); }

// ---------------------------------------------------------------------------------- split
// One wave per token: hi/lo bf16 split of x and Σx (lanes sum strided elements, then a wave sum).
__global__ void __launch_bounds__(256) k_pf_split(const float *__restrict__ X, int T, int H, __bf16 *__restrict__ Xhi,
                                                  __bf16 *__restrict__ Xlo, float *__restrict__ xsum) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (t >= T) return;
  const float *x = X + (size_t)t * H;
  float s = 0.0f;
  for (int c = lane; c < H; c += 64) {
    const float v = x[c];
    const __bf16 hi = (__bf16)v;
    Xhi[(size_t)t * H + c] = hi;
    Xlo[(size_t)t * H + c] = (__bf16)(v - (float)hi);
    s += v;
  }
  s = dsh_wave_sum(s);
  if (lane == 0) xsum[t] = s;
}

// ---------------------------------------------------------------------------------- routing
// One 256-thread block per token. CFG: the f32 router as the decode path sums it (partials of 8
// rows Σ_j WrT[r0+j][e]·x[r0+j]; wave w adds partials w, w+4, ... in order; the four wave sums are
// added in wave order), top-k on raw scores, softmax over the k. DECODE: the bf16 router in the
// reference's AVX-512 order (as k_dec_scores_bf16), fast-exp softmax over all experts, top-k.
template <int MODE>
__global__ void __launch_bounds__(256) k_pf_route(dsh_layer_t L, const float *__restrict__ X, int nthreads,
                                                  int *__restrict__ idx, float *__restrict__ w) {
  extern __shared__ float xs[];
  __shared__ int s_idx[64];
  __shared__ float s_w[64];
  __shared__ float s_red[4][64];
  const int t = blockIdx.x, H = L.H, E = L.E, K = L.K;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int i = threadIdx.x; i < H; i += 256) xs[i] = X[(size_t)t * H + i];
  __syncthreads();
  if (MODE == DSH_ROUTE_CFG) {
    float acc = 0.0f;
    if (lane < E) {
      for (int b = wave; b < H / 8; b += 4) {
        float p = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++) p = __builtin_fmaf(L.router_f32_t[(size_t)(8 * b + j) * E + lane], xs[8 * b + j], p);
        acc += p;
      }
    }
    s_red[wave][lane] = lane < E ? acc : 0.0f;
  } else {
    // 64 groups of 4 lanes: group g computes expert g's score in the AVX-512 order
    const int Lq = threadIdx.x & 3, g = threadIdx.x >> 2;
    const int chunk = dsh_chunk_len(E, nthreads);
    float v = 0.0f;
    if (g < E) {
      const int path = row_path(g, E, chunk, false);
      v = avx_row<true>(L.router_bf16 + (size_t)g * H, xs, H, Lq, path == DSH_ROW_SINGLE, true, 0.0f,
                        path != DSH_ROW_GROUP4);
    }
    // the full score goes to s_red[0][g]; the other wave rows are zero (0 + ... keeps the value)
    if (Lq == 0) s_red[0][g] = g < E ? v : 0.0f;
    if (threadIdx.x < 192) s_red[1 + threadIdx.x / 64][threadIdx.x & 63] = 0.0f;
  }
  __syncthreads();
  if (wave == 0) route_select(E, K, MODE, s_idx, s_w, s_red);
  __syncthreads();
  if (threadIdx.x < K) {
    idx[(size_t)t * K + threadIdx.x] = s_idx[threadIdx.x];
    w[(size_t)t * K + threadIdx.x] = s_w[threadIdx.x];
  }
}

// ---------------------------------------------------------------------------------- plan
// One block: counts per expert (slots with no expert, idx < 0, are skipped), exclusive offsets,
// and the work list: each expert's pairs in chunks of PF_MT, then the shared expert's T tokens.
__global__ void __launch_bounds__(256) k_pf_plan(const int *__restrict__ idx, int T, int K, int E,
                                                 int *__restrict__ seg_off, pf_item *__restrict__ items,
                                                 int *__restrict__ n_items) {
  __shared__ int cnt[64];
  if (threadIdx.x < 64) cnt[threadIdx.x] = 0;
  __syncthreads();
  for (int i = threadIdx.x; i < T * K; i += 256) {
    const int e = idx[i];
    if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int off = 0, ni = 0;
    for (int e = 0; e < E; e++) {
      seg_off[e] = off;
      for (int m0 = 0; m0 < cnt[e]; m0 += PF_MT) items[ni++] = pf_item{e, m0, min(PF_MT, cnt[e] - m0), off};
      off += cnt[e];
    }
    seg_off[E] = off;
    for (int m0 = 0; m0 < T; m0 += PF_MT) items[ni++] = pf_item{E, m0, min(PF_MT, T - m0), 0};
    *n_items = ni;
  }
}

// One wave per expert: walks the (token, slot) entries in token order and appends those routed
// to its expert (ballot + prefix count), so each expert's tokens are in increasing order.
__global__ void __launch_bounds__(256) k_pf_scatter(const int *__restrict__ idx, int T, int K, int E,
                                                    const int *__restrict__ seg_off, int *__restrict__ pair_tok,
                                                    int *__restrict__ pos_of) {
  const int e = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (e >= E) return;
  int pos = seg_off[e];
  for (int base = 0; base < T * K; base += 64) {
    const int i = base + lane;
    const bool mine = i < T * K && idx[i] == e;
    const unsigned long long m = __ballot(mine);
    if (mine) {
      const int p = pos + __popcll(m & ((1ull << lane) - 1ull));
      pair_tok[p] = i / K;
      pos_of[i] = p;
    }
    pos += __popcll(m);
  }
}

// ---------------------------------------------------------------------------------- gate_up
// Block (work item, n-tile): 64 rows of A (the item's tokens) x 128 intermediate units. Wave w
// owns units i0 + 32w .. +31 of both the gate rows and the up rows, so SwiGLU pairs sit in the same
// lane and register. K (= H) runs in blocks of 32 columns: lane half h = lane/32 reads 16 bytes of
// a weight row at columns k0 + 16h .. +15 and the matching 16 activations of its A row as two
// MFMA k-slices (any permutation of k applied to both operands leaves the product unchanged).
template <bool SHARED>
__device__ __forceinline__ void gate_up_tile(const dsh_layer_t &L, const pf_item &it, int nt, const __bf16 *Xhi,
                                             const __bf16 *Xlo, const float *xsum, const int *pair_tok,
                                             int bf16sim, __bf16 *Hhi, __bf16 *Hlo) {
  const int H = L.H;
  const int Iseg = SHARED ? L.SI : L.I;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, half = lane >> 5, l32 = lane & 31;
  const int unit = nt * PF_GU_N + wave * 32 + l32;  // this lane's B column (intermediate unit)
  const int8_t *wq = SHARED ? L.sgu_q : L.gu_q + (size_t)it.seg * 2 * L.I * H;
  const float *wso = SHARED ? L.sgu_so : L.gu_so + (size_t)it.seg * 2 * L.I * 2;
  const int8_t *grow = wq + (size_t)unit * H;
  const int8_t *urow = wq + (size_t)(Iseg + unit) * H;
  // A rows of the two 32-row halves of the chunk (rows past mcnt repeat row 0: loaded, never stored)
  int tok[2];
#pragma unroll
  for (int ms = 0; ms < 2; ms++) {
    const int r = ms * 32 + l32;
    const int rr = r < it.mcnt ? r : 0;
    tok[ms] = SHARED ? it.m0 + rr : pair_tok[it.pos0 + it.m0 + rr];
  }
  f32x16 acc[2][2];
#pragma unroll
  for (int ms = 0; ms < 2; ms++)
#pragma unroll
    for (int q = 0; q < 2; q++)
#pragma unroll
      for (int j = 0; j < 16; j++) acc[ms][q][j] = 0.0f;
  for (int k0 = 0; k0 < H; k0 += 32) {
    const int kc = k0 + 16 * half;
    const u32x4 gb = *(const u32x4 *)(grow + kc), ub = *(const u32x4 *)(urow + kc);
    bf16x8 ahi[2][2], alo[2][2];
#pragma unroll
    for (int ms = 0; ms < 2; ms++)
#pragma unroll
      for (int s = 0; s < 2; s++) {
        ahi[ms][s] = ld_bf16x8(Xhi + (size_t)tok[ms] * H + kc + 8 * s);
        alo[ms][s] = ld_bf16x8(Xlo + (size_t)tok[ms] * H + kc + 8 * s);
      }
#pragma unroll
    for (int s = 0; s < 2; s++) {
      const bf16x8 bg = codes_to_bf16(u32x2{gb[2 * s], gb[2 * s + 1]});
      const bf16x8 bu = codes_to_bf16(u32x2{ub[2 * s], ub[2 * s + 1]});
#pragma unroll
      for (int ms = 0; ms < 2; ms++) {
        acc[ms][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ahi[ms][s], bg, acc[ms][0], 0, 0, 0);
        acc[ms][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(alo[ms][s], bg, acc[ms][0], 0, 0, 0);
        acc[ms][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ahi[ms][s], bu, acc[ms][1], 0, 0, 0);
        acc[ms][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(alo[ms][s], bu, acc[ms][1], 0, 0, 0);
      }
    }
  }
  const float2 sog = ((const float2 *)wso)[unit], sou = ((const float2 *)wso)[Iseg + unit];
#pragma unroll
  for (int ms = 0; ms < 2; ms++)
#pragma unroll
    for (int j = 0; j < 16; j++) {
      const int r = ms * 32 + mfma_row(lane, j);
      if (r >= it.mcnt) continue;
      const int t = SHARED ? it.m0 + r : pair_tok[it.pos0 + it.m0 + r];
      const float xs = xsum[t];
      float g = __builtin_fmaf(sog.x, acc[ms][0][j], sog.y * xs);
      float up = __builtin_fmaf(sou.x, acc[ms][1][j], sou.y * xs);
      if (bf16sim) {
        g = dsh_bf16_round_half_up(g);
        up = dsh_bf16_round_half_up(up);
      }
      float hv = dsh_swiglu(g, up);
      if (bf16sim) hv = dsh_bf16_round_half_up(hv);
      const size_t row = SHARED ? (size_t)(it.m0 + r) : (size_t)(it.pos0 + it.m0 + r);
      const __bf16 hi = (__bf16)hv;
      Hhi[row * Iseg + unit] = hi;
      Hlo[row * Iseg + unit] = (__bf16)(hv - (float)hi);
    }
}

__global__ void __launch_bounds__(256) k_pf_gate_up(dsh_layer_t L, const pf_item *__restrict__ items,
                                                    const int *__restrict__ n_items, const __bf16 *__restrict__ Xhi,
                                                    const __bf16 *__restrict__ Xlo, const float *__restrict__ xsum,
                                                    const int *__restrict__ pair_tok, int bf16sim,
                                                    __bf16 *__restrict__ Hhi, __bf16 *__restrict__ Hlo,
                                                    __bf16 *__restrict__ Shi, __bf16 *__restrict__ Slo) {
  if ((int)blockIdx.x >= *n_items) return;
  const pf_item it = items[blockIdx.x];
  const int nt = blockIdx.y;
  if (it.seg == L.E) {
    if (nt * PF_GU_N >= L.SI) return;
    gate_up_tile<true>(L, it, nt, Xhi, Xlo, xsum, pair_tok, bf16sim, Shi, Slo);
  } else {
    if (nt * PF_GU_N >= L.I) return;
    gate_up_tile<false>(L, it, nt, Xhi, Xlo, xsum, pair_tok, bf16sim, Hhi, Hlo);
  }
}

// ---------------------------------------------------------------------------------- down
// Block (work item, n-tile): 64 rows of A (h of the item's pairs, or of tokens for the shared
// expert) x 256 output rows. Wave w owns output rows n0 + 64w .. +63 (two 32-column MFMA tiles).
// Σh of each A row is summed from hi + lo along the K loop (lanes l and l+32 hold the two column
// halves of a row) and combined across the halves at the end.
template <bool SHARED>
__device__ __forceinline__ void down_tile(const dsh_layer_t &L, const pf_item &it, int nt, const __bf16 *Hhi,
                                          const __bf16 *Hlo, float *Y) {
  const int H = L.H;
  const int Kd = SHARED ? L.SI : L.I;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, half = lane >> 5, l32 = lane & 31;
  const int8_t *wq = SHARED ? L.sdn_q : L.dn_q + (size_t)it.seg * H * L.I;
  const float *wso = SHARED ? L.sdn_so : L.dn_so + (size_t)it.seg * H * 2;
  int nrow[2];
  const int8_t *brow[2];
#pragma unroll
  for (int q = 0; q < 2; q++) {
    nrow[q] = nt * PF_DN_N + wave * 64 + q * 32 + l32;
    brow[q] = wq + (size_t)nrow[q] * Kd;
  }
  size_t arow[2];
#pragma unroll
  for (int ms = 0; ms < 2; ms++) {
    const int r = ms * 32 + l32;
    const int rr = r < it.mcnt ? r : 0;
    arow[ms] = SHARED ? (size_t)(it.m0 + rr) : (size_t)(it.pos0 + it.m0 + rr);
  }
  f32x16 acc[2][2];
#pragma unroll
  for (int ms = 0; ms < 2; ms++)
#pragma unroll
    for (int q = 0; q < 2; q++)
#pragma unroll
      for (int j = 0; j < 16; j++) acc[ms][q][j] = 0.0f;
  float hsum[2] = {0.0f, 0.0f};
  for (int k0 = 0; k0 < Kd; k0 += 32) {
    const int kc = k0 + 16 * half;
    u32x4 braw[2];
#pragma unroll
    for (int q = 0; q < 2; q++) braw[q] = *(const u32x4 *)(brow[q] + kc);
    bf16x8 ahi[2][2], alo[2][2];
#pragma unroll
    for (int ms = 0; ms < 2; ms++)
#pragma unroll
      for (int s = 0; s < 2; s++) {
        ahi[ms][s] = ld_bf16x8(Hhi + arow[ms] * Kd + kc + 8 * s);
        alo[ms][s] = ld_bf16x8(Hlo + arow[ms] * Kd + kc + 8 * s);
      }
#pragma unroll
    for (int ms = 0; ms < 2; ms++)
#pragma unroll
      for (int s = 0; s < 2; s++)
#pragma unroll
        for (int i = 0; i < 8; i++) hsum[ms] += (float)ahi[ms][s][i] + (float)alo[ms][s][i];
#pragma unroll
    for (int s = 0; s < 2; s++) {
      bf16x8 b[2];
#pragma unroll
      for (int q = 0; q < 2; q++) b[q] = codes_to_bf16(u32x2{braw[q][2 * s], braw[q][2 * s + 1]});
#pragma unroll
      for (int ms = 0; ms < 2; ms++)
#pragma unroll
        for (int q = 0; q < 2; q++) {
          acc[ms][q] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ahi[ms][s], b[q], acc[ms][q], 0, 0, 0);
          acc[ms][q] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(alo[ms][s], b[q], acc[ms][q], 0, 0, 0);
        }
    }
  }
  // Σh of row l32 (+32 ms): lanes l and l+32 hold the two column halves
  __shared__ float s_hsum[4][2][32];
#pragma unroll
  for (int ms = 0; ms < 2; ms++) {
    const float other = __shfl_xor(hsum[ms], 32);
    if (half == 0) s_hsum[wave][ms][l32] = hsum[ms] + other;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
  for (int q = 0; q < 2; q++) {
    const float2 so = ((const float2 *)wso)[nrow[q]];
#pragma unroll
    for (int ms = 0; ms < 2; ms++)
#pragma unroll
      for (int j = 0; j < 16; j++) {
        const int r = ms * 32 + mfma_row(lane, j);
        if (r >= it.mcnt) continue;
        const float hs = s_hsum[wave][ms][mfma_row(lane, j)];
        const size_t row = SHARED ? (size_t)(it.m0 + r) : (size_t)(it.pos0 + it.m0 + r);
        Y[row * H + nrow[q]] = __builtin_fmaf(so.x, acc[ms][q][j], so.y * hs);
      }
  }
}

__global__ void __launch_bounds__(256) k_pf_down(dsh_layer_t L, const pf_item *__restrict__ items,
                                                 const int *__restrict__ n_items, const __bf16 *__restrict__ Hhi,
                                                 const __bf16 *__restrict__ Hlo, const __bf16 *__restrict__ Shi,
                                                 const __bf16 *__restrict__ Slo, float *__restrict__ Y,
                                                 float *__restrict__ Ysh) {
  if ((int)blockIdx.x >= *n_items) return;
  const pf_item it = items[blockIdx.x];
  const int nt = blockIdx.y;
  if (it.seg == L.E)
    down_tile<true>(L, it, nt, Shi, Slo, Ysh);
  else
    down_tile<false>(L, it, nt, Hhi, Hlo, Y);
}

// ---------------------------------------------------------------------------------- combine
// One block per token: routed slots in ascending expert order (the reference's scatter-add order,
// ds_moe_decoder.c:781-795), weights w_k, then the shared output and the residual.
__global__ void __launch_bounds__(256) k_pf_combine(const float *__restrict__ X, const int *__restrict__ idx,
                                                    const float *__restrict__ w, const int *__restrict__ pos_of,
                                                    const float *__restrict__ Y, const float *__restrict__ Ysh,
                                                    int H, int K, int residual, int bf16sim, float *__restrict__ out) {
  __shared__ int s_pos[64];
  __shared__ float s_w[64];
  __shared__ int e_sorted[64];
  __shared__ int s_n;
  const int t = blockIdx.x;
  if (threadIdx.x == 0) {
    int n = 0;
    for (int k = 0; k < K; k++) {
      const int e = idx[(size_t)t * K + k];
      if (e < 0) continue;
      int j = n++;
      while (j > 0 && e_sorted[j - 1] > e) {
        e_sorted[j] = e_sorted[j - 1];
        s_pos[j] = s_pos[j - 1];
        s_w[j] = s_w[j - 1];
        j--;
      }
      e_sorted[j] = e;
      s_pos[j] = pos_of[(size_t)t * K + k];
      s_w[j] = w[(size_t)t * K + k];
    }
    s_n = n;
  }
  __syncthreads();
  for (int c = threadIdx.x; c < H; c += 256) {
    float routed = 0.0f;
    for (int j = 0; j < s_n; j++) {
      float v = Y[(size_t)s_pos[j] * H + c];
      if (bf16sim) v = dsh_bf16_round_half_up(v);
      routed = __builtin_fmaf(s_w[j], v, routed);
    }
    float sh = Ysh[(size_t)t * H + c];
    if (bf16sim) sh = dsh_bf16_round_half_up(sh);
    const float o = routed + sh;
    out[(size_t)t * H + c] = residual ? X[(size_t)t * H + c] + o : o;
  }
}

// ---------------------------------------------------------------------------------- launchers
namespace {
struct pf_ws {
  __bf16 *Xhi, *Xlo;
  float *xsum;
  int *idx;
  float *w;
  int *seg_off, *n_items;
  pf_item *items;
  int *pair_tok, *pos_of;
  __bf16 *Hhi, *Hlo, *Shi, *Slo;
  float *Y, *Ysh;
};

size_t al256(size_t n) { return (n + 255) & ~(size_t)255; }

int pf_max_items(const dsh_layer_t *L, int T) {
  return (T * L->K + PF_MT - 1) / PF_MT + L->E + (T + PF_MT - 1) / PF_MT;
}

// Carves the workspace; returns its size (ws may be NULL to size it).
size_t pf_carve(const dsh_layer_t *L, int T, void *base, pf_ws *w) {
  const size_t H = L->H, I = L->I, SI = L->SI, K = L->K, E = L->E, TK = (size_t)T * K;
  size_t off = 0;
  char *b = (char *)base;
#define TAKE(field, type, count)                          \
  do {                                                    \
    if (w) w->field = (type *)(b + off);                  \
    off += al256(sizeof(type) * (size_t)(count));         \
  } while (0)
  TAKE(Xhi, __bf16, T * H);
  TAKE(Xlo, __bf16, T * H);
  TAKE(xsum, float, T);
  TAKE(idx, int, TK);
  TAKE(w, float, TK);
  TAKE(seg_off, int, E + 1);
  TAKE(n_items, int, 1);
  TAKE(items, pf_item, pf_max_items(L, T));
  TAKE(pair_tok, int, TK);
  TAKE(pos_of, int, TK);
  TAKE(Hhi, __bf16, TK * I);
  TAKE(Hlo, __bf16, TK * I);
  TAKE(Shi, __bf16, T * SI);
  TAKE(Slo, __bf16, T * SI);
  TAKE(Y, float, TK * H);
  TAKE(Ysh, float, T * H);
#undef TAKE
  return off;
}
}  // namespace

extern "C" {

int dsh_pf_supported(const dsh_layer_t *L) {
  if (L->H % PF_DN_N || L->I % PF_GU_N || L->SI % PF_GU_N) return 0;
  if (L->E > 64 || L->K > 64 || L->K > L->E) return 0;
  return 1;
}

size_t dsh_pf_workspace_bytes(const dsh_layer_t *L, int T) { return pf_carve(L, T, NULL, NULL); }

hipError_t dsh_launch_prefill(const dsh_layer_t *L, const float *X, int T, int route_mode, int nthreads, int residual,
                              int bf16sim, float *out, void *ws, int *idx_out, float *w_out, hipStream_t s) {
  if (T <= 0 || !dsh_pf_supported(L)) return hipErrorInvalidValue;
  if (route_mode == DSH_ROUTE_CFG ? !L->router_f32_t : !L->router_bf16) return hipErrorInvalidValue;
  pf_ws w;
  pf_carve(L, T, ws, &w);
  const int H = L->H, K = L->K, E = L->E;
  k_pf_split<<<(T + 3) / 4, 256, 0, s>>>(X, T, H, w.Xhi, w.Xlo, w.xsum);
  if (route_mode == DSH_ROUTE_CFG)
    k_pf_route<DSH_ROUTE_CFG><<<T, 256, (size_t)H * 4, s>>>(*L, X, nthreads, w.idx, w.w);
  else
    k_pf_route<DSH_ROUTE_DECODE><<<T, 256, (size_t)H * 4, s>>>(*L, X, nthreads, w.idx, w.w);
  k_pf_plan<<<1, 256, 0, s>>>(w.idx, T, K, E, w.seg_off, w.items, w.n_items);
  k_pf_scatter<<<(E + 3) / 4, 256, 0, s>>>(w.idx, T, K, E, w.seg_off, w.pair_tok, w.pos_of);
  const int mi = pf_max_items(L, T);
  k_pf_gate_up<<<dim3(mi, max(L->I, L->SI) / PF_GU_N), 256, 0, s>>>(*L, w.items, w.n_items, w.Xhi, w.Xlo, w.xsum,
                                                                   w.pair_tok, bf16sim, w.Hhi, w.Hlo, w.Shi, w.Slo);
  k_pf_down<<<dim3(mi, H / PF_DN_N), 256, 0, s>>>(*L, w.items, w.n_items, w.Hhi, w.Hlo, w.Shi, w.Slo, w.Y, w.Ysh);
  k_pf_combine<<<T, 256, 0, s>>>(X, w.idx, w.w, w.pos_of, w.Y, w.Ysh, H, K, residual, bf16sim, out);
  hipError_t e = hipGetLastError();
  if (e == hipSuccess && idx_out)
    e = hipMemcpyAsync(idx_out, w.idx, sizeof(int) * (size_t)T * K, hipMemcpyDeviceToDevice, s);
  if (e == hipSuccess && w_out)
    e = hipMemcpyAsync(w_out, w.w, sizeof(float) * (size_t)T * K, hipMemcpyDeviceToDevice, s);
  return e;
}

}  // extern "C"
