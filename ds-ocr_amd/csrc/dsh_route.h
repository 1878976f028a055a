// dsh_route.h — expert selection of one MoE layer from per-wave partial score sums, shared by the
// decode kernels (k_dec.hip) and the prefill kernels (k_prefill.hip) so both route identically.
#pragma once
#include "dsh.h"
#include "k_core.h"

// LDS scratch of one selecting wave.
struct route_scratch {
  unsigned long long key[64];  // each expert's order key (0: not selectable)
  int sel[64];                 // expert at each rank
  float val[64];               // its score (CFG) or probability (DECODE), as the key orders it
};

// One wave, lane = expert; s_red (LDS, visible to the wave) holds four partial score rows, added
// in row order. Writes s_idx[0..K) and s_w[0..K) (visible to this wave after it returns).
//
// Order keys (dsh_argmax_key) compare as the reference's selection does: larger value first, lower
// index on equal values, NaN and values <= -1e30 never selected, ±0 equal. Each selectable lane
// counts the keys above its own (64 reads of the wave's keys in LDS): that is its selection round,
// the same as K successive arg-max rounds, without their chain of dependent wave reductions.
// CFG (ds_moe_top_k, ds_kernels.c:193-243): top-K on the raw scores, then softmax over the K
// chosen in selection order (expf, max first, sequential sum); slots past the selectable count get
// expert 0 and weight 0. DECODE (ds_moe_decoder.c:145-183): fast-exp softmax over all experts
// (max, sequential sum in expert order, 1/sum), top-K on the probabilities, weights = those
// probabilities; empty slots get expert -1 and weight -1e30.
__device__ __forceinline__ void route_select(int E, int K, int mode, int *s_idx, float *s_w, float (*s_red)[64],
                                             route_scratch *scr) {
  const int lane = threadIdx.x & 63;
  const float s = ((s_red[0][lane] + s_red[1][lane]) + s_red[2][lane]) + s_red[3][lane];
  float v = s;
  if (mode != DSH_ROUTE_CFG) {
    float m = (lane < E && s > -1e30f) ? s : -1e30f;
    m = dsh_wave_max(m);
    float p = lane < E ? dsh_fast_expf(s - m) : 0.0f;
    float sum = 0.0f;
    for (int e = 0; e < E; e++) sum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), e));
    const float inv = 1.0f / sum;
    v = p * inv;
  }
  const unsigned long long key = lane < E ? dsh_argmax_key(v, lane) : 0ull;
  scr->key[lane] = key;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  int rank = 0;
#pragma unroll 16
  for (int j = 0; j < 64; j++) rank += scr->key[j] > key ? 1 : 0;
  const int nsel = __popcll(__ballot(key != 0ull));
  const int ns = nsel < K ? nsel : K;  // experts selected
  if (key != 0ull && rank < K) {
    scr->sel[rank] = lane;
    scr->val[rank] = dsh_key_value(key);
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const bool mine = lane < ns;
  const int my_sel = mine ? scr->sel[lane] : 0;
  const float my_val = mine ? scr->val[lane] : -1e30f;
  if (mode == DSH_ROUTE_CFG) {
    const float mx = ns > 0 ? scr->val[0] : -1e30f;  // the first selected is the largest
    const float ev = mine ? expf(my_val - mx) : 0.0f;
    float sum = 0.0f;
    for (int j = 0; j < ns; j++) sum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ev), j));
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
