// dsh_route.h — expert selection of one MoE layer from per-wave partial score sums, shared by the
// decode kernels (k_dec.hip) and the prefill kernels (k_prefill.hip) so both route identically.
#pragma once
#include "dsh.h"
#include "k_core.h"

// One wave, lane = expert; s_red (LDS, visible to the wave) holds four partial score rows, added
// in row order. Writes s_idx[0..K) and s_w[0..K) (visible to this wave after it returns).
//
// Order: larger value first, lower index on equal values, NaN and values <= -1e30 never selected,
// ±0 equal (the reference's strict '>' scans, ds_kernels.c:193-243, ds_moe_decoder.c:160-183).
// Selection runs in registers: round r takes the wave maximum of the keys still in play, the
// lowest lane holding a key equal to it (ballot; -0 and +0 compare equal) becomes rank r, and its
// key drops out; the same order as K successive arg-max scans.
// CFG (ds_moe_top_k): top-K on the raw scores, then softmax over the K chosen in selection order
// (correctly rounded expf, max first, sequential sum); slots past the selectable count get expert 0
// and weight 0.
// DECODE (ds_moe_decoder.c:145-183): fast-exp softmax over all experts (max, sequential sum in
// expert order, 1/sum), top-K on the probabilities, weights = those probabilities; empty slots get
// expert -1 and weight -1e30.
__device__ __forceinline__ void route_select(int E, int K, int mode, int *s_idx, float *s_w, float (*s_red)[64]) {
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
  float key = selectable ? v : -__builtin_huge_valf();
  const int nsel = __popcll(__ballot(selectable));
  const int ns = nsel < K ? nsel : K;  // experts selected
  const bool mine = lane < ns;
  int my_sel = 0;           // lane r < ns: the expert of rank r
  float my_val = -1e30f;    // and its value
  for (int r = 0; r < ns; r++) {  // r < nsel: a selectable key (> -inf) is still in play
    const float m = dsh_wave_max(key);
    const unsigned long long eq = __ballot(key == m);
    const int win = __builtin_ctzll(eq);
    const float wv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), win));
    if (lane == r) {
      my_sel = win;
      my_val = wv;
    }
    if (lane == win) key = -__builtin_huge_valf();
  }
  my_sel = mine ? my_sel : 0;
  my_val = mine ? my_val : -1e30f;
  if (mode == DSH_ROUTE_CFG) {
    // the first selected is the largest; lanes past ns hold +0, which leaves the sum as is
    const float mx = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(my_val)));
    const float ev = mine ? dsh_expf_cr(my_val - mx) : 0.0f;
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++) sum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ev), j));
    for (int j = 8; j < ns; j++) sum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ev), j));
    const float inv = 1.0f / sum;
    if (lane < K) {
      s_idx[lane] = mine ? my_sel : 0;
      s_w[lane] = mine ? ev * inv : 0.0f;
    }
  } else if (lane < K) {
    s_idx[lane] = mine ? my_sel : -1;
    s_w[lane] = my_val;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}
