// k_attn.hip — the attention half of one decoder layer for one token (decoder_layer_forward,
// ds_moe_decoder.c:339-431; MHA, single-token decode) on the device:
//   k_attn_qkv     : x_norm = ds_rms_norm(x) in its AVX-512 order (recomputed by every block), then
//                    the rows of [Wq; Wk; Wv] in ds_linear_nobias_bf16_qkv's AVX-512 order with its
//                    split of the rows over the reference's threads (ds_kernels.c:844-915); v goes
//                    straight into the V cache row pos;
//   k_attn_scores  : per head x chunk of positions, the optional per-head q/k norms and RoPE
//                    (ds_apply_rope_neox, recomputed by every block), the roped k into the K cache row
//                    pos, and the scores;
//   k_attn_coef, k_attn_av, k_attn_combine : the online-softmax attention over the causal or R-SWA
//                    positions (below), spread over heads x position chunks;
//   k_attn_oproj   : proj = Wo·att in ds_bf16_matvec_threaded's order;
//   k_attn_post    : h = x + proj and n = ds_rms_norm(h) (ds_residual_rms_norm, AVX-512 order).
// Everything except the attention's output sum is bit-exact with the reference. The reference's
// attention is a sequential online softmax with ds_fast_expf (ds_kernels.c:2124-2160,
// :2270-2330). Its branch at each position depends only on the running maximum, so these kernels
// take the same branches with the same exp arguments: a prefix-max scan gives each position's
// running maximum P, its factor f = fast_exp(P - s) on a new maximum (the correction) or
// fast_exp(s - P) (its weight), and a suffix product of the later corrections gives each V row's
// final coefficient c; o = sum c*v and sum_e = sum c are then sums in any order. The result differs
// from the reference's sequential recurrence by f32 rounding only.
#include "dsh.h"
#include "dsh_avx.h"
#include "k_core.h"

__device__ __forceinline__ int attn_pos(const int *pos_ptr, int pos_add) { return (pos_ptr ? *pos_ptr : 0) + pos_add; }

// ds_rms_norm's sum of squares (AVX-512 branch): 16 lanes of fused squares over n/16 steps, then
// the reduce tree. Called by all threads; x in LDS, n % 16 == 0. Returns r = 1/sqrtf(sum/n + eps)
// to every thread (s_r: one LDS float).
__device__ float attn_rms_scale(const float *x, int n, float eps, float *s_r) {
  if (threadIdx.x < 16) {
    float acc = 0.0f;
    for (int i = 0; i < n; i += 16) acc = __builtin_fmaf(x[i + threadIdx.x], x[i + threadIdx.x], acc);
    // tree16: T3[i] = A[8+i] + A[i]; T6[j] = T3[4+j] + T3[j]; (T6[0]+T6[2]) + (T6[1]+T6[3])
    const float t3 = __shfl_down(acc, 8, 16) + acc;
    const float t6 = __shfl_down(t3, 4, 16) + t3;
    const float t02 = __shfl_down(t6, 2, 16) + t6;  // lane 0: T6[0]+T6[2]; lane 1: T6[1]+T6[3]
    const float s = t02 + __shfl_down(t02, 1, 16);
    if (threadIdx.x == 0) *s_r = 1.0f / __builtin_sqrtf(s / (float)n + eps);
  }
  __syncthreads();
  return *s_r;
}

// Path of global row R of [q; k; v] under ds_linear_nobias_bf16_qkv's split: thread t takes rows
// [t*chunk, min((t+1)*chunk, total)) and runs one ds_bf16_matvec_fused per matrix over its part.
__device__ __forceinline__ int qkv_row_path(int R, int q_dim, int kv_dim, int nthreads) {
  const int total = q_dim + 2 * kv_dim;
  const int m = R < q_dim ? 0 : (R < q_dim + kv_dim ? 1 : 2);
  const int base = m == 0 ? 0 : (m == 1 ? q_dim : q_dim + kv_dim);
  const int mend = m == 0 ? q_dim : (m == 1 ? q_dim + kv_dim : total);
  int s = base, e = mend;
  if (nthreads > 1) {
    const int chunk = (total + nthreads - 1) / nthreads;
    const int t = R / chunk;
    s = max(t * chunk, base);
    e = min(min((t + 1) * chunk, total), mend);
  }
  const int len = e - s, off = R - s;
  if (off < (len & ~3)) return DSH_ROW_GROUP4;
  return off < (len & ~1) ? DSH_ROW_GROUP2 : DSH_ROW_SINGLE;
}

// One bf16 row of length 32*N32 against x (LDS) at lane L of its 4-lane group, in the path's order.
template <int N32>
__device__ __forceinline__ float attn_row(const uint16_t *w, const u32x4 *wv, const float *x, int L, int path) {
  if (path == DSH_ROW_SINGLE) return avx_row<true>(w, x, 32 * N32, L, true, true, 0.0f, true);
  return avx_row_regs32<N32>(wv, x, L, true, 0.0f);
}

// Every lane's 16-byte pieces of its row (columns 32i + 8L .. +7), issued together.
template <int N32>
__device__ __forceinline__ void attn_row_load(u32x4 *wv, const uint16_t *w, int L) {
#pragma unroll
  for (int i = 0; i < N32; i++) wv[i] = ((const u32x4 *)w)[4 * i + L];
}

// ---------------------------------------------------------------------------- QKV
// 64 rows of [q; k; v] per 256-thread block (4 lanes per row). H == 32*N32.
// Pieces i0 and i1 (f32x4; i1 < 0: none) of x into LDS dst, x summed over ncopies (1 or 8) copies
// [ncopies][H] in copy order; every load is issued before the first add. Also to x_out when given.
__device__ __forceinline__ void attn_x_pieces(const float *x, int H, int ncopies, int i0, int i1, float *dst,
                                              float *x_out) {
  const f32x4 *x4 = (const f32x4 *)x;
  const int H4 = H / 4, j0 = i0 < 0 ? 0 : i0, j1 = i1 < 0 ? j0 : i1;
  f32x4 a = x4[j0], b = x4[j1];
  if (ncopies == 8) {
    f32x4 ca[7], cb[7];
#pragma unroll
    for (int c = 0; c < 7; c++) {
      ca[c] = x4[(size_t)(c + 1) * H4 + j0];
      cb[c] = x4[(size_t)(c + 1) * H4 + j1];
    }
#pragma unroll
    for (int c = 0; c < 7; c++) {
      a += ca[c];
      b += cb[c];
    }
  }
  if (i0 >= 0) {
    ((f32x4 *)dst)[i0] = a;
    if (x_out) ((f32x4 *)x_out)[i0] = a;
  }
  if (i1 >= 0) {
    ((f32x4 *)dst)[i1] = b;
    if (x_out) ((f32x4 *)x_out)[i1] = b;
  }
}

template <int N32>
__global__ void __launch_bounds__(256) k_attn_qkv(dsh_attn_t A, const float *x_in, const int *step, int stride,
                                                  int ncopies, float *x_plain, const int *pos_ptr, int pos_add,
                                                  int nthreads) {
  constexpr int H = 32 * N32;
  __shared__ __attribute__((aligned(16))) float s_x[H];
  __shared__ float s_r;
  const int qd = A.n_heads * A.head_dim, total = 3 * qd;
  const int L = threadIdx.x & 3;
  const int R = blockIdx.x * 64 + (threadIdx.x >> 2);
  const int Rc = R < total ? R : total - 1;
  const int m = Rc < qd ? 0 : (Rc < 2 * qd ? 1 : 2), r = Rc - m * qd;
  const uint16_t *w = (m == 0 ? A.wq : (m == 1 ? A.wk : A.wv)) + (size_t)r * H;
  const int path = qkv_row_path(Rc, qd, qd, nthreads);
  u32x4 wv[N32];
  if (path != DSH_ROW_SINGLE) attn_row_load<N32>(wv, w, L);
  const float *x = step ? x_in + (size_t)(*step) * stride : x_in;
  // H/4 <= 512 pieces: at most two per thread (block 0 also writes x for the residual kernel)
  attn_x_pieces(x, H, ncopies, (int)threadIdx.x < H / 4 ? (int)threadIdx.x : -1,
                (int)threadIdx.x + 256 < H / 4 ? (int)threadIdx.x + 256 : -1, s_x, blockIdx.x == 0 ? x_plain : nullptr);
  __syncthreads();
  const float rs = attn_rms_scale(s_x, H, A.eps, &s_r);
  float xn[(H + 255) / 256];
#pragma unroll
  for (int k = 0; k < (H + 255) / 256; k++) {
    const int i = threadIdx.x + 256 * k;
    if (i < H) xn[k] = (s_x[i] * A.in_norm[i]) * rs;
  }
  __syncthreads();  // every thread has read s_x
#pragma unroll
  for (int k = 0; k < (H + 255) / 256; k++) {
    const int i = threadIdx.x + 256 * k;
    if (i < H) s_x[i] = xn[k];
  }
  __syncthreads();
  const float v = attn_row<N32>(w, wv, s_x, L, path);
  if (L == 0 && R < total) {
    if (m == 0)
      A.q[r] = v;
    else if (m == 1)
      A.k[r] = v;
    else
      A.vc[(size_t)attn_pos(pos_ptr, pos_add) * A.kv_stride + r] = v;
  }
}

// ---------------------------------------------------------------------------- attention core
#define ATTN_THREADS 256

// Inclusive scan over the block's threads (ATTN_THREADS) with an associative op; s_w: 4 floats.
template <typename Op>
__device__ __forceinline__ float attn_block_scan(float v, Op op, float *s_w) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const float u = __shfl_up(v, o);
    if (lane >= o) v = op(u, v);
  }
  if (lane == 63) s_w[wave] = v;
  __syncthreads();
  for (int w = 0; w < wave; w++) v = op(s_w[w], v);
  __syncthreads();
  return v;
}

// ds_dot_f32 in its AVX-512 order for n % 64 == 0 (ds_kernels_avx.c:357-377): four 16-lane
// accumulators over 64-element blocks, added pairwise, then the reduce tree. q in LDS, k global.
__device__ __forceinline__ float attn_dot(const float *q, const float *k, int n) {
  float a[4][16];
#pragma unroll
  for (int m = 0; m < 4; m++)
#pragma unroll
    for (int l = 0; l < 16; l++) a[m][l] = 0.0f;
#pragma unroll
  for (int i = 0; i < n; i += 64) {
#pragma unroll
    for (int m = 0; m < 4; m++) {
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const f32x4 kv = ((const f32x4 *)(k + i + 16 * m))[c];
        const f32x4 qv = ((const f32x4 *)(q + i + 16 * m))[c];
#pragma unroll
        for (int e = 0; e < 4; e++) a[m][4 * c + e] = __builtin_fmaf(qv[e], kv[e], a[m][4 * c + e]);
      }
    }
  }
  float A16[16];
#pragma unroll
  for (int l = 0; l < 16; l++) A16[l] = (a[0][l] + a[1][l]) + (a[2][l] + a[3][l]);
  float T3[8], T6[4];
#pragma unroll
  for (int i = 0; i < 8; i++) T3[i] = A16[8 + i] + A16[i];
#pragma unroll
  for (int j = 0; j < 4; j++) T6[j] = T3[4 + j] + T3[j];
  return (T6[0] + T6[2]) + (T6[1] + T6[3]);
}

// The attended positions of the token at cache position pos: p < r1 is position p, then r2 + (p - r1)
// ([0, pos+1), or R-SWA's reference tokens [0, prefill_len) and window [ws, pos+1)).
struct attn_span {
  int r1, r2, n;
  __device__ __forceinline__ int j(int p) const { return p < r1 ? p : r2 + (p - r1); }
};
__device__ __forceinline__ attn_span attn_positions(int pos, int prefill_len, int window) {
  const int kv = pos + 1;
  attn_span sp{kv, kv, kv};
  if (window > 0 && pos >= prefill_len) {
    const int ws = prefill_len > kv - window ? prefill_len : kv - window;
    if (ws > prefill_len) sp = attn_span{prefill_len, ws, prefill_len + (kv - ws)};
  }
  return sp;
}

// The optional per-head norms (ds_rms_norm_per_head) and RoPE of one head's q and k (in LDS, hd
// threads of the block active). Called by every thread of the block.
__device__ void attn_rope_head(const dsh_attn_t &A, int h, int pos, float *s_q, float *s_k, float *s_r) {
  const int hd = A.head_dim, half = hd / 2, tid = threadIdx.x;
  const float *cs = A.rope_cos + (size_t)pos * hd, *sn = A.rope_sin + (size_t)pos * hd;
  for (int d = tid; d < hd; d += blockDim.x) {
    s_q[d] = A.q[h * hd + d];
    s_k[d] = A.k[h * hd + d];
  }
  __syncthreads();
  for (int which = 0; which < 2; which++) {
    const float *nw = which ? A.k_norm : A.q_norm;
    float *v = which ? s_k : s_q;
    if (nw) {
      const float r = attn_rms_scale(v, hd, A.eps, s_r);
      float y[DSH_ATTN_MAX_HD / 64];
      for (int d = tid, i = 0; d < hd; d += blockDim.x, i++) y[i] = (v[d] * nw[d]) * r;
      __syncthreads();
      for (int d = tid, i = 0; d < hd; d += blockDim.x, i++) v[d] = y[i];
      __syncthreads();
    }
  }
  float rq[DSH_ATTN_MAX_HD / 64], rk[DSH_ATTN_MAX_HD / 64];
  for (int t = tid, i = 0; t < hd; t += blockDim.x, i++) {
    const int d = t < half ? t : t - half;
    const float q1 = s_q[d], q2 = s_q[d + half], k1 = s_k[d], k2 = s_k[d + half];
    if (t < half) {
      rq[i] = __builtin_fmaf(q1, cs[d], -(q2 * sn[d]));
      rk[i] = __builtin_fmaf(k1, cs[d], -(k2 * sn[d]));
    } else {
      rq[i] = __builtin_fmaf(q1, sn[t], q2 * cs[t]);
      rk[i] = __builtin_fmaf(k1, sn[t], k2 * cs[t]);
    }
  }
  __syncthreads();
  for (int t = tid, i = 0; t < hd; t += blockDim.x, i++) {
    s_q[t] = rq[i];
    s_k[t] = rk[i];
  }
  __syncthreads();
}

// Scores, bit-exact: 64 attended positions per 64-thread block (grid: heads x chunks of the cache),
// one thread per position; sc[h][p] = ds_dot_f32(q, k_j) * (1/sqrtf(head_dim)). Every block ropes
// the head's q (and k) itself; the block holding the token's own position writes its roped k into
// the K cache row pos and uses it from LDS.
template <int HD>
__global__ void __launch_bounds__(64) k_attn_scores(dsh_attn_t A, const int *pos_ptr, int pos_add, int prefill_len,
                                                    int window) {
  __shared__ __attribute__((aligned(16))) float s_q[HD], s_k[HD];
  __shared__ float s_r;
  const int h = blockIdx.x, p = blockIdx.y * 64 + threadIdx.x;
  const int pos = attn_pos(pos_ptr, pos_add);
  const attn_span sp = attn_positions(pos, prefill_len, window);
  if ((int)blockIdx.y * 64 >= sp.n) return;  // whole block
  attn_rope_head(A, h, pos, s_q, s_k, &s_r);
  const bool own = ((int)blockIdx.y + 1) * 64 >= sp.n;  // this block holds position n-1 == pos
  if (own)
    for (int d = threadIdx.x; d < HD; d += 64) A.kc[(size_t)pos * A.kv_stride + h * HD + d] = s_k[d];
  if (p < sp.n) {
    const int j = sp.j(p);
    const float scale = 1.0f / __builtin_sqrtf((float)HD);
    A.sc[(size_t)h * A.max_seq + p] =
        attn_dot(s_q, j == pos ? s_k : A.kc + (size_t)j * A.kv_stride + h * HD, HD) * scale;
  }
}

// Per head: the reference's sequence of branches (see the top of this file) as coefficients:
// sc[h][p] <- c_p, se[h] <- sum_e. Dynamic LDS: 2 * max_seq floats.
__global__ void __launch_bounds__(ATTN_THREADS) k_attn_coef(dsh_attn_t A, const int *pos_ptr, int pos_add,
                                                            int prefill_len, int window) {
  extern __shared__ __attribute__((aligned(16))) float s_dyn[];
  __shared__ float s_w[4];
  __shared__ __attribute__((aligned(16))) float s_o[ATTN_THREADS];
  float *s_s = s_dyn, *s_c = s_dyn + A.max_seq;
  const int h = blockIdx.x, tid = threadIdx.x;
  const int n = attn_positions(attn_pos(pos_ptr, pos_add), prefill_len, window).n;
  float *sc = A.sc + (size_t)h * A.max_seq;
  for (int p = tid; p < n; p += ATTN_THREADS) s_s[p] = sc[p];
  __syncthreads();
  // running maximum before each position: exclusive prefix max over contiguous segments
  const int seg = (n + ATTN_THREADS - 1) / ATTN_THREADS;
  const int p0 = min(tid * seg, n), p1 = min(p0 + seg, n);
  float sm = -__builtin_huge_valf();
  for (int p = p0; p < p1; p++) sm = fmaxf(sm, s_s[p]);
  const float incl = attn_block_scan(sm, [](float a, float b) { return fmaxf(a, b); }, s_w);
  s_o[tid] = incl;
  __syncthreads();
  // the reference starts from max_s = -1e30 (a NaN score is never a new maximum: fmaxf skips it)
  float P = fmaxf(-1e30f, tid ? s_o[tid - 1] : -__builtin_huge_valf());
  __syncthreads();
  // factors: a = correction on a new maximum (else 1), g = 1 on a new maximum (else the weight);
  // s_s[p] <- a, s_c[p] <- g
  float prod = 1.0f;
  for (int p = p0; p < p1; p++) {
    const float s = s_s[p];
    const bool nm = s > P;
    const float f = dsh_fast_expf(nm ? P - s : s - P);
    s_s[p] = nm ? f : 1.0f;
    s_c[p] = nm ? 1.0f : f;
    prod *= nm ? f : 1.0f;
    P = nm ? s : P;
  }
  // product of the corrections after each segment: a scan over the threads in reverse order
  // (thread t holds segment ATTN_THREADS-1-t's product; the exclusive suffix of segment tid is the
  // inclusive value of thread ATTN_THREADS-2-tid)
  s_o[tid] = prod;
  __syncthreads();
  const float rprod = s_o[ATTN_THREADS - 1 - tid];
  __syncthreads();
  const float rincl = attn_block_scan(rprod, [](float a, float b) { return a * b; }, s_w);
  s_o[tid] = rincl;
  __syncthreads();
  float after = tid < ATTN_THREADS - 1 ? s_o[ATTN_THREADS - 2 - tid] : 1.0f;
  float csum = 0.0f;
  for (int p = p1 - 1; p >= p0; p--) {
    const float c = s_c[p] * after;  // c = g * (product of the later corrections)
    sc[p] = c;
    csum += c;
    after *= s_s[p];
  }
  const float tot = attn_block_scan(csum, [](float a, float b) { return a + b; }, s_w);
  if (tid == ATTN_THREADS - 1) A.se[h] = tot;
}

// V: 32 attended positions per block of head_dim threads (grid: heads x chunks), every v load of a
// thread in flight together; part[h][chunk][d] = sum over the chunk of c_p * v_p[d].
#define ATTN_VCH 32
__global__ void __launch_bounds__(DSH_ATTN_MAX_HD) k_attn_av(dsh_attn_t A, const int *pos_ptr, int pos_add,
                                                             int prefill_len, int window) {
  __shared__ float s_c[ATTN_VCH];
  const int h = blockIdx.x, hd = A.head_dim, d = threadIdx.x, p0 = blockIdx.y * ATTN_VCH;
  const attn_span sp = attn_positions(attn_pos(pos_ptr, pos_add), prefill_len, window);
  if (p0 >= sp.n) return;  // whole block
  const int cnt = min(ATTN_VCH, sp.n - p0);
  if (d < ATTN_VCH) s_c[d] = d < cnt ? A.sc[(size_t)h * A.max_seq + p0 + d] : 0.0f;
  float v[ATTN_VCH];
#pragma unroll
  for (int q = 0; q < ATTN_VCH; q++) v[q] = A.vc[(size_t)sp.j(p0 + min(q, cnt - 1)) * A.kv_stride + h * hd + d];
  __syncthreads();
  float acc = 0.0f;
#pragma unroll
  for (int q = 0; q < ATTN_VCH; q++) acc = __builtin_fmaf(s_c[q], v[q], acc);  // s_c is 0 past cnt
  A.part[((size_t)h * (A.max_seq / ATTN_VCH + 1) + blockIdx.y) * hd + d] = acc;
}

// Per head: the chunk sums in chunk order, times 1/sum_e (ds_vec_scale_inplace; sum_e > 0).
__global__ void __launch_bounds__(DSH_ATTN_MAX_HD) k_attn_combine(dsh_attn_t A, const int *pos_ptr, int pos_add,
                                                                  int prefill_len, int window) {
  const int h = blockIdx.x, hd = A.head_dim, d = threadIdx.x;
  const int n = attn_positions(attn_pos(pos_ptr, pos_add), prefill_len, window).n;
  const int nch = (n + ATTN_VCH - 1) / ATTN_VCH;
  const float *pt = A.part + (size_t)h * (A.max_seq / ATTN_VCH + 1) * hd + d;
  float o = 0.0f;
  for (int c0 = 0; c0 < nch; c0 += 16) {  // 16 loads in flight, then the adds in chunk order
    float v[16];
#pragma unroll
    for (int q = 0; q < 16; q++) v[q] = pt[(size_t)min(c0 + q, nch - 1) * hd];
#pragma unroll
    for (int q = 0; q < 16; q++)
      if (c0 + q < nch) o += v[q];
  }
  const float se = A.se[h];
  if (se > 0.0f) o = o * (1.0f / se);
  A.att[h * hd + d] = o;
}

// ---------------------------------------------------------------------------- O projection
// 16 output rows per 64-thread block; att (q_dim == 32*N32) staged in LDS.
template <int N32>
__global__ void __launch_bounds__(64) k_attn_oproj(dsh_attn_t A, int chunk) {
  constexpr int QD = 32 * N32;
  __shared__ __attribute__((aligned(16))) float s_a[QD];
  const int L = threadIdx.x & 3;
  const int r = blockIdx.x * 16 + (threadIdx.x >> 2);
  const int rc = r < A.H ? r : A.H - 1;
  const uint16_t *w = A.wo + (size_t)rc * QD;
  const int path = row_path(rc, A.H, chunk, false);
  u32x4 wv[N32];
  if (path != DSH_ROW_SINGLE) attn_row_load<N32>(wv, w, L);
  for (int i = threadIdx.x; i < QD / 4; i += 64) ((f32x4 *)s_a)[i] = ((const f32x4 *)A.att)[i];
  __syncthreads();
  const float v = attn_row<N32>(w, wv, s_a, L, path);
  if (L == 0 && r < A.H) A.proj[r] = v;
}

// ---------------------------------------------------------------------------- residual RMSNorm
// R rows per 256-thread block (H / R blocks): every block forms h = x + proj (rounded) in LDS and
// the RMSNorm scale (ds_residual_rms_norm, AVX-512 order), writes its rows of h and n = (h*w)*r
// and, given the next MoE layer's transposed f32 router WrT ([H][E]), the partial router scores of
// its rows (the format of k_dec_partial_scores: one row of 64 per block, its rows added in order).
template <int N32, int R>
__global__ void __launch_bounds__(256) k_attn_post(dsh_attn_t A, const float *x_in, const int *step, int stride,
                                                   float *h_out, float *n_out,
                                                   const float *__restrict__ WrT, int E, float *__restrict__ partials) {
  constexpr int H = 32 * N32;
  __shared__ __attribute__((aligned(16))) float s_h[H];
  __shared__ float s_r, s_n[R];
  const float *x = step ? x_in + (size_t)(*step) * stride : x_in;
  const int r0 = blockIdx.x * R;
  float wr[R];
  if (WrT && (int)threadIdx.x < E) {
#pragma unroll
    for (int j = 0; j < R; j++) wr[j] = WrT[(size_t)(r0 + j) * E + threadIdx.x];
  }
  for (int i = threadIdx.x; i < H / 4; i += 256) {
    const f32x4 xv = ((const f32x4 *)x)[i], pv = ((const f32x4 *)A.proj)[i];
    ((f32x4 *)s_h)[i] = xv + pv;
  }
  __syncthreads();
  const float r = attn_rms_scale(s_h, H, A.eps, &s_r);
  if (threadIdx.x < R) {
    const int i = r0 + threadIdx.x;
    const float nv = (s_h[i] * A.post_norm[i]) * r;
    h_out[i] = s_h[i];
    n_out[i] = nv;
    s_n[threadIdx.x] = nv;
  }
  __syncthreads();
  if (WrT && threadIdx.x < 64) {
    float p = 0.0f;
    if ((int)threadIdx.x < E) {
#pragma unroll
      for (int j = 0; j < R; j++) p = __builtin_fmaf(wr[j], s_n[j], p);
    }
    partials[(size_t)blockIdx.x * 64 + threadIdx.x] = (int)threadIdx.x < E ? p : 0.0f;
  }
}

// ds_rms_norm of the last hidden state before the LM head (ds_moe_decoder.c:1000), AVX-512 order;
// trunc: ds_bf16_truncate_array after it (:1016-1018, bf16 simulation of model version 3).
template <int N32>
__global__ void __launch_bounds__(256) k_final_norm(const float *__restrict__ x, int ncopies,
                                                    const float *__restrict__ w, float eps, int trunc,
                                                    float *__restrict__ out, float *__restrict__ x_out) {
  constexpr int H = 32 * N32;
  __shared__ __attribute__((aligned(16))) float s_x[H];
  __shared__ float s_r;
  attn_x_pieces(x, H, ncopies, (int)threadIdx.x < H / 4 ? (int)threadIdx.x : -1,
                (int)threadIdx.x + 256 < H / 4 ? (int)threadIdx.x + 256 : -1, s_x, x_out);
  __syncthreads();
  const float r = attn_rms_scale(s_x, H, eps, &s_r);
  for (int i = threadIdx.x; i < H; i += 256) {
    const float v = (s_x[i] * w[i]) * r;
    out[i] = trunc ? dsh_bf16_round_half_up(v) : v;
  }
}

extern "C" {

int dsh_attn_supported(int H, int n_heads, int head_dim) {
  const int qd = n_heads * head_dim;
  return H % 256 == 0 && H / 256 >= 1 && H / 256 <= 8 && head_dim % 64 == 0 && head_dim <= DSH_ATTN_MAX_HD &&
         head_dim <= ATTN_THREADS && qd % 256 == 0 && qd / 256 >= 1 && qd / 256 <= 8;
}

// scores/factors and coefficients; at least 8 floats (the per-part sums reuse the first ones)
size_t dsh_attn_core_lds(int max_kv) { return (size_t)2 * max_kv * sizeof(float); }

hipError_t dsh_launch_attn(const dsh_attn_t *A, const float *x_in, const int *step, int stride, int ncopies,
                           float *x_plain, const int *pos_ptr, int pos_add, int prefill_len, int window, int nthreads,
                           float *h_out, float *n_out, const float *WrT_next, int E_next, float *partials_next,
                           hipStream_t s) {
  if (!dsh_attn_supported(A->H, A->n_heads, A->head_dim)) return hipErrorInvalidValue;
  if ((ncopies != 1 && ncopies != 8) || (ncopies > 1 && (step || !x_plain))) return hipErrorInvalidValue;
  const float *x_post = ncopies > 1 ? x_plain : x_in;  // the residual kernel reads one plain vector
  const int qd = A->n_heads * A->head_dim;
#define QKV(N)                                                                                     \
  case N:                                                                                          \
    k_attn_qkv<8 * N><<<(3 * qd + 63) / 64, 256, 0, s>>>(*A, x_in, step, stride, ncopies,            \
                                                          ncopies > 1 ? x_plain : nullptr, pos_ptr, \
                                                          pos_add, nthreads);                      \
    break;
  switch (A->H / 256) {
    QKV(1) QKV(2) QKV(3) QKV(4) QKV(5) QKV(6) QKV(7) QKV(8)
    default:
      return hipErrorInvalidValue;
  }
#undef QKV
  const dim3 gs(A->n_heads, (A->max_seq + 63) / 64), gv(A->n_heads, (A->max_seq + ATTN_VCH - 1) / ATTN_VCH);
  switch (A->head_dim) {
    case 64:
      k_attn_scores<64><<<gs, 64, 0, s>>>(*A, pos_ptr, pos_add, prefill_len, window);
      break;
    case 128:
      k_attn_scores<128><<<gs, 64, 0, s>>>(*A, pos_ptr, pos_add, prefill_len, window);
      break;
    case 192:
      k_attn_scores<192><<<gs, 64, 0, s>>>(*A, pos_ptr, pos_add, prefill_len, window);
      break;
    case 256:
      k_attn_scores<256><<<gs, 64, 0, s>>>(*A, pos_ptr, pos_add, prefill_len, window);
      break;
    default:
      return hipErrorInvalidValue;
  }
  k_attn_coef<<<A->n_heads, ATTN_THREADS, dsh_attn_core_lds(A->max_seq), s>>>(*A, pos_ptr, pos_add, prefill_len,
                                                                             window);
  k_attn_av<<<gv, A->head_dim, 0, s>>>(*A, pos_ptr, pos_add, prefill_len, window);
  k_attn_combine<<<A->n_heads, A->head_dim, 0, s>>>(*A, pos_ptr, pos_add, prefill_len, window);
  const int chunk = dsh_chunk_len(A->H, nthreads);
#define OP(N)                                                             \
  case N:                                                                 \
    k_attn_oproj<8 * N><<<(A->H + 15) / 16, 64, 0, s>>>(*A, chunk);       \
    break;
  switch (qd / 256) {
    OP(1) OP(2) OP(3) OP(4) OP(5) OP(6) OP(7) OP(8)
    default:
      return hipErrorInvalidValue;
  }
#undef OP
#define PO(N, RR)                                                                                           \
  case N:                                                                                                   \
    k_attn_post<8 * N, RR><<<A->H / RR, 256, 0, s>>>(*A, x_post, ncopies > 1 ? nullptr : step, stride,        \
                                                     h_out, n_out, WrT_next, E_next, partials_next);        \
    break;
  if (WrT_next && (E_next <= 0 || E_next > 64)) return hipErrorInvalidValue;
  if (A->H / dsh_dec_partials(A->H) == 8) {
    switch (A->H / 256) {
      PO(1, 8) PO(2, 8) PO(3, 8) PO(4, 8) PO(5, 8)
      default:
        return hipErrorInvalidValue;
    }
  } else {
    switch (A->H / 256) {
      PO(6, 16) PO(7, 16) PO(8, 16)
      default:
        return hipErrorInvalidValue;
    }
  }
#undef PO
  return hipGetLastError();
}

hipError_t dsh_launch_final_norm(const float *x, int ncopies, const float *w, int H, float eps, int trunc, float *out,
                                 float *x_out, hipStream_t s) {
#define FN(N)                                                                         \
  case N:                                                                             \
    k_final_norm<8 * N><<<1, 256, 0, s>>>(x, ncopies, w, eps, trunc, out, x_out);     \
    break;
  if (H % 256 || (ncopies != 1 && ncopies != 8)) return hipErrorInvalidValue;
  switch (H / 256) {
    FN(1) FN(2) FN(3) FN(4) FN(5) FN(6) FN(7) FN(8)
    default:
      return hipErrorInvalidValue;
  }
#undef FN
  return hipGetLastError();
}

}  // extern "C"
