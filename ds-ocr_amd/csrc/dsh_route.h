// dsh_route.h — expert selection of one MoE layer from per-wave partial score sums, shared by the
// decode kernels (k_dec.hip) and the prefill kernels (k_prefill.hip) so both route identically.
#pragma once
#include "dsh.h"
#include "k_core.h"

// The selection's state in one wave (lane = expert): the scores or DECODE probabilities v, the keys
// still in play, the number of experts selected (ns), and for lane r < rounds done the expert of rank
// r and its value. route_select is route_init, route_rounds(0, ns), route_finish; a wave that needs
// only rank r runs the rounds up to r, and the rest later (the order of the rounds is the same).
struct route_state {
  float v, key;
  int ns, sel;
  float val;
};

__device__ __forceinline__ void route_init(int E, int K, int mode, const float (*s_red)[64], route_state &st) {
  const int lane = threadIdx.x & 63;
  const float s = ((s_red[0][lane] + s_red[1][lane]) + s_red[2][lane]) + s_red[3][lane];
  float v = s;
  if (mode != DSH_ROUTE_CFG) {
    float m = (lane < E && s > -1e30f) ? s : -1e30f;
    m = dsh_wave_max(m);
    const float p = lane < E ? dsh_fast_expf(s - m) : 0.0f;
    // sequential sum in expert order; lanes >= E hold +0, which leaves the (non-negative) sum as is
    float sum = 0.0f;
#pragma unroll
    for (int e = 0; e < 64; e++) sum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), e));
    const float inv = 1.0f / sum;
    v = p * inv;
  }
  const bool selectable = lane < E && v > -1e30f;  // false for NaN
  st.v = v;
  st.key = selectable ? v : -__builtin_huge_valf();
  const int nsel = __popcll(__ballot(selectable));
  st.ns = nsel < K ? nsel : K;  // experts selected
  st.sel = 0;
  st.val = -1e30f;
}

// Rounds r0 .. r1 - 1 (r1 <= ns): round r takes the wave maximum of the keys in play; the lowest lane
// holding a key equal to it (ballot; -0 and +0 compare equal) is rank r, and its key drops out.
__device__ __forceinline__ void route_rounds(route_state &st, int r0, int r1) {
  const int lane = threadIdx.x & 63;
  for (int r = r0; r < r1; r++) {  // r < nsel: a selectable key (> -inf) is still in play
    const float m = dsh_wave_max(st.key);
    const unsigned long long eq = __ballot(st.key == m);
    const int win = __builtin_ctzll(eq);
    const float wv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(st.v), win));
    if (lane == r) {
      st.sel = win;
      st.val = wv;
    }
    if (lane == win) st.key = -__builtin_huge_valf();
  }
}

// After all ns rounds: lane r < K gets its slot's expert and weight. CFG: softmax over the selected
// values in selection order (correctly rounded expf, max first, sequential sum); slots past ns get
// expert 0 and weight 0. DECODE: the probabilities; slots past ns get expert -1 and weight -1e30.
__device__ __forceinline__ void route_finish(int mode, const route_state &st, int &idx, float &w) {
  const int lane = threadIdx.x & 63, ns = st.ns;
  const bool mine = lane < ns;
  const int my_sel = mine ? st.sel : 0;
  const float my_val = mine ? st.val : -1e30f;
  if (mode == DSH_ROUTE_CFG) {
    // the first selected is the largest; lanes past ns hold +0, which leaves the sum as is
    const float mx = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(my_val)));
    const float ev = mine ? dsh_expf_cr(my_val - mx) : 0.0f;
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++) sum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ev), j));
    for (int j = 8; j < ns; j++) sum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ev), j));
    const float inv = 1.0f / sum;
    idx = mine ? my_sel : 0;
    w = mine ? ev * inv : 0.0f;
  } else {
    idx = mine ? my_sel : -1;
    w = my_val;
  }
}

// One wave, lane = expert; s_red (LDS, visible to the wave) holds four partial score rows, added
// in row order. Writes s_idx[0..K) and s_w[0..K) (visible to this wave after it returns).
//
// Order: larger value first, lower index on equal values, NaN and values <= -1e30 never selected,
// ±0 equal (the reference's strict '>' scans, ds_kernels.c:193-243, ds_moe_decoder.c:160-183): the
// rounds of route_rounds give the same order as K successive arg-max scans.
// CFG (ds_moe_top_k): top-K on the raw scores, then softmax over the K chosen in selection order.
// DECODE (ds_moe_decoder.c:145-183): fast-exp softmax over all experts (max, sequential sum in
// expert order, 1/sum), top-K on the probabilities, weights = those probabilities.
__device__ __forceinline__ void route_select(int E, int K, int mode, int *s_idx, float *s_w, float (*s_red)[64]) {
  const int lane = threadIdx.x & 63;
  route_state st;
  route_init(E, K, mode, s_red, st);
  route_rounds(st, 0, st.ns);
  int idx;
  float w;
  route_finish(mode, st, idx, w);
  if (lane < K) {
    s_idx[lane] = idx;
    s_w[lane] = w;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}
