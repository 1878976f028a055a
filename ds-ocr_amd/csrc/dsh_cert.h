// dsh_cert.h — certified CFG expert selection: the experts ds_moe_top_k picks on ds_linear's scores
// (ds_moe_router → ds_linear_nobias → ds_linear, ds_kernels.c:181-185, :639-652; ds_moe_top_k,
// :193-243), established from scores summed in another order plus a rigorous bound on the
// difference, with ds_linear's own order recomputed for the experts the bound leaves open.
//
// The reference's score of expert e is a sequential f32 sum ŝ of the rounded products
// p_k = fl(w_k x_k) (GCC vectorizes the products and adds them in index order; the scalar tail past
// the last multiple of 8 is fused), starting from 0: ŝ_1 = p_1 exactly, ŝ_k = fl(ŝ_{k-1} + p_k). With
// P_k = Σ_{j<=k} p_j, each addition errs by at most u|P_k + (error so far)| (u = 2^-24), so the
// running-error bound is
//     |ŝ_n - P_n| <= u Σ_{k=2..n} |P_k| / (1 - (n-1)u).
// For random data Σ|P_k| behaves like (2/3) n^1.5 σ_p (a random walk), some 40 times below the
// worst case n Σ|p_k| behind γ_n: the bound needs the prefix sums' sizes, not only the terms'.
//
// cert_radius_partials bounds |ŝ_n - c| for a score c summed from partials: R rows per partial (any
// order inside a partial: at most R roundings per term), the partials of the contiguous range of
// row v added sequentially from 0 (r[v]), then c = ((r0 + r1) + r2) + r3. With T_k the exact prefix
// of w_k x_k, A = Σ|w_k x_k| <= ||w|| ||x||, and lam[v] = Σ over row v's partials of |its running sum
// before that partial|:
//   |c - T_n|   <= e_C = γ_R A + u Σ_v (lam[v] + |r[v]|) + u (|r0 + r1| + |r0 + r1 + r2| + |c|)
//   Σ_k |T_k|   <= R Σ_v (nb[v] |O_v| + lam[v]) + R nb e_C + R A     (O_v: the rows before v)
//   |P_k - T_k| <= u A,   so  Σ_k |P_k| <= Σ_k |T_k| + n u A  and  |P_n - T_n| <= u A
//   |ŝ - c|     <= e_C + u A + u (1 + 2^-10) (R Σ_v (nb[v] |O_v| + lam[v]) + R nb e_C + R A + n u A)
// (n = H <= 2048, so 1 / (1 - (n-1)u) < 1 + 2^-10). Every term is a sum of non-negative f32 values
// computed with at most ~25 roundings, which the final factor 1 + 2^-16 covers.
//
// cert_check takes the selection made on c (route_rounds) and the radii: the selection and its rank
// order are the reference's when the intervals [c - eps, c + eps] of the selected experts, in rank
// order, and of the best unselected one are disjoint (strictly). Otherwise the candidates are the
// experts whose interval reaches the lowest selected lower bound (K experts are surely above it, so
// no other expert can be in the top K), and cert_exact_chain computes their scores in ds_linear's
// order; selecting on those (others set to -inf) is then ds_moe_top_k's selection, and the CFG
// softmax over them (route_finish) gives the reference's weights as well.
#pragma once
#include "dsh_route.h"

#define DSH_U 5.9604644775390625e-8f  // 2^-24

__device__ __forceinline__ float cert_radius_partials(const float r[4], const float lam[4], const int nb[4], int R,
                                                      int H, float wn, float xn) {
  const float u = DSH_U, g10 = 1.0f + 0x1p-10f;
  const float A = wn * xn * (1.0f + 0x1p-20f);
  const float O2 = r[0] + r[1], O3 = O2 + r[2], c = O3 + r[3];
  const float eC = (float)R * u * g10 * A +
                   u * ((((lam[0] + lam[1]) + (lam[2] + lam[3])) + (fabsf(r[0]) + fabsf(r[1]))) +
                        (fabsf(r[2]) + fabsf(r[3]))) +
                   u * ((fabsf(O2) + fabsf(O3)) + fabsf(c));
  const float S1 = (float)R * (((float)nb[1] * fabsf(r[0]) + (float)nb[2] * fabsf(O2)) + (float)nb[3] * fabsf(O3) +
                               ((lam[0] + lam[1]) + (lam[2] + lam[3])));
  const float nbt = (float)(nb[0] + nb[1] + nb[2] + nb[3]);
  const float run = S1 + (float)R * nbt * eC + (float)R * A + (float)H * u * A;
  return (eC + u * A + u * g10 * run) * (1.0f + 0x1p-16f);
}

// The next float below / above f (f finite): with round-to-nearest, next_down(fl(a - b)) <= a - b and
// next_up(fl(a + b)) >= a + b, so intervals built that way contain the exact ones.
__device__ __forceinline__ float cert_next_down(float f) {
  const unsigned u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) == 0u) return -__uint_as_float(1u);
  return __uint_as_float((int)u >= 0 ? u - 1u : u + 1u);
}
__device__ __forceinline__ float cert_next_up(float f) { return -cert_next_down(-f); }

// After route_rounds(st, 0, st.ns) on the scores c (lane = expert, radius eps): true (wave-uniform)
// when the selection and its rank order are certain; otherwise cand gets the candidate experts (all
// E experts when a score or radius is not finite, or fewer than K are selectable). The interval
// ends are rounded outward in f32, so the strict comparisons hold for the exact ends as well.
__device__ __forceinline__ bool cert_check(const route_state &st, float c, float eps, int E, int K,
                                           unsigned long long &cand) {
  const int lane = threadIdx.x & 63;
  const bool valid = lane < E;
  const bool finite = !valid || (__builtin_isfinite(c) && __builtin_isfinite(eps) &&
                                 __builtin_isfinite(c - eps) && __builtin_isfinite(c + eps));
  const unsigned long long all = E >= 64 ? ~0ull : ((1ull << E) - 1ull);
  cand = all;
  if (__ballot(!finite) != 0ull || st.ns < K) return false;
  const bool selectable = valid && c > -1e30f;
  const bool in_sel = selectable && st.key == -__builtin_huge_valf();  // selected keys drop out
  const float lo_me = valid ? cert_next_down(c - eps) : 0.0f, hi_me = valid ? cert_next_up(c + eps) : 0.0f;
  const int er = lane < K ? st.sel : 0;
  const float lo = __shfl(lo_me, er), hi = __shfl(hi_me, er);
  const float hi_next = __shfl(hi, min(lane + 1, 63));
  const float hi_out = dsh_wave_max(selectable && !in_sel ? hi_me : -__builtin_huge_valf());
  const float lo_last = __shfl(lo, K - 1);
  const bool bad = (lane < K - 1 && !(lo > hi_next)) || (lane == 0 && !(lo_last > hi_out));
  if (__ballot(bad) == 0ull) {
    cand = 0ull;
    return true;
  }
  const float lmin = -dsh_wave_max(lane < K ? -lo : -__builtin_huge_valf());
  cand = __ballot(valid && hi_me >= lmin);
  return false;
}

// ds_linear's score (ds_kernels.c:639-652 without BLAS, seq 1, as GCC 11 compiles it: rounded
// products added in index order from 0, the tail past the last multiple of 8 (16 when H >= 16)
// fused) of expert `lane` for each lane whose bit is set in cand; Wr is the row-major router
// [E][H], x (H floats, 16-byte aligned) in LDS or global memory. Other lanes return +0 and read row 0.
// One wave; every lane's loads are issued PF float4s ahead of its chain.
__device__ __forceinline__ float cert_exact_chain(const float *__restrict__ Wr, const float *x, int H,
                                                  unsigned long long cand) {
  constexpr int PF = 8;
  const int lane = threadIdx.x & 63;
  const bool on = (cand >> lane) & 1ull;
  const f32x4 *row = (const f32x4 *)(Wr + (size_t)(on ? lane : 0) * H);
  const int m = H >= 16 ? (H & ~15) + ((H - (H & ~15)) >= 8 ? 8 : 0) : (H >= 8 ? 8 : 0);
  const int n4 = H / 4;  // H % 4 == 0 (H % 256 == 0 for every kernel that calls this)
  f32x4 ring[PF];
#pragma unroll
  for (int j = 0; j < PF; j++) ring[j] = row[min(j, n4 - 1)];
  float s = 0.0f;
  for (int q0 = 0; q0 < n4; q0 += PF) {
#pragma unroll
    for (int j = 0; j < PF; j++) {
      const int q = q0 + j;
      const f32x4 w = ring[j];
      ring[j] = row[min(q + PF, n4 - 1)];
      if (q < n4) {
        const f32x4 xv = *(const f32x4 *)(x + 4 * q);
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int k = 4 * q + i;
          s = k < m ? __fadd_rn(s, __fmul_rn(xv[i], w[i])) : __builtin_fmaf(xv[i], w[i], s);
        }
      }
    }
  }
  return on ? s : 0.0f;
}

// CFG routing of one wave (lane = expert) from partial rows: s_red[v] the row sums and s_lam[v]
// the prefix sizes of cert_radius_partials (nb[v] partials of R rows in row v), wn = ||router row||
// (rounded up), xn >= ||x||; Wr the row-major f32 router and x the routed input for
// ds_linear's order where the bound leaves the selection open; s_tmp: 4 x 64 floats of LDS private
// to this wave. Writes s_idx[0..K) and s_w[0..K) as route_select does (visible to this wave after it
// returns); returns true when ds_linear's order was recomputed.
__device__ __forceinline__ bool route_select_cert(int E, int K, int *s_idx, float *s_w, const float (*s_red)[64],
                                                  const float (*s_lam)[64], const int nb[4], int R, int H, float wn,
                                                  float xn, const float *__restrict__ Wr, const float *x,
                                                  float (*s_tmp)[64]) {
  const int lane = threadIdx.x & 63;
  route_state st;
  route_init(E, K, DSH_ROUTE_CFG, s_red, st);
  route_rounds(st, 0, st.ns);
  const float r[4] = {s_red[0][lane], s_red[1][lane], s_red[2][lane], s_red[3][lane]};
  const float lam[4] = {s_lam[0][lane], s_lam[1][lane], s_lam[2][lane], s_lam[3][lane]};
  const float c = ((r[0] + r[1]) + r[2]) + r[3];
  const float eps = lane < E ? cert_radius_partials(r, lam, nb, R, H, wn, xn) : 0.0f;
  unsigned long long cand;
  bool exact = false;
  if (!cert_check(st, c, eps, E, K, cand)) {
    const float ex = cert_exact_chain(Wr, x, H, cand);
    s_tmp[0][lane] = ((cand >> lane) & 1ull) ? ex : -__builtin_huge_valf();
    s_tmp[1][lane] = 0.0f;
    s_tmp[2][lane] = 0.0f;
    s_tmp[3][lane] = 0.0f;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    route_init(E, K, DSH_ROUTE_CFG, s_tmp, st);
    route_rounds(st, 0, st.ns);
    exact = true;
  }
  int idx;
  float w;
  route_finish(DSH_ROUTE_CFG, st, idx, w);
  if (lane < K) {
    s_idx[lane] = idx;
    s_w[lane] = w;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  return exact;
}

// One routing's record (dsh_rcert_t): the counters, and the log entry when a log is set. Called by
// one lane; x: the routed input (H floats).
__device__ __forceinline__ void cert_record(const dsh_rcert_t &rc, const int *idx, const float *w, int K, int flags,
                                            const float *x, int H) {
  if (rc.stats) {
    __hip_atomic_fetch_add(rc.stats, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (flags & 1) __hip_atomic_fetch_add(rc.stats + 1, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (!rc.log) return;
  const int n = __hip_atomic_fetch_add(rc.log, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (n >= rc.log_cap) return;
  int *e = rc.log + 64 + (size_t)n * DSH_RLOG_STRIDE(H);
  for (int k = 0; k < 8; k++) {
    e[k] = k < K ? idx[k] : -1;
    e[8 + k] = k < K ? __float_as_int(w[k]) : 0;
  }
  e[16] = flags;
  e[17] = rc.tag;
  for (int i = 0; i < H; i++) e[32 + i] = __float_as_int(x[i]);
}
