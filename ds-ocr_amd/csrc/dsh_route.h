// dsh_route.h — expert selection of one MoE layer from per-wave partial score sums, shared by the
// decode kernels (k_dec.hip) and the prefill kernels (k_prefill.hip) so both route identically.
#pragma once
#include "dsh.h"
#include "k_core.h"

// LDS scratch of one selecting wave.
struct route_scratch {
  alignas(16) float key[64];  // each expert's order value (-inf: not selectable)
  int sel[64];                // expert at each rank
  float val[64];              // its score (CFG) or probability (DECODE)
};

// One wave, lane = expert; s_red (LDS, visible to the wave) holds four partial score rows, added
// in row order. Writes s_idx[0..K) and s_w[0..K) (visible to this wave after it returns).
//
// Order: larger value first, lower index on equal values, NaN and values <= -1e30 never selected,
// ±0 equal (the reference's strict '>' scans, ds_kernels.c:193-243, ds_moe_decoder.c:160-183).
// Each selectable lane counts the values above its own (64 broadcast reads of the wave's values in
// LDS, one f32 compare each): with no equal values that count is its selection round, the same as
// K successive arg-max rounds. Lanes whose count is below K write their slot and read it back; two
// equal values give two lanes the same count, which that read-back detects, and then every lane
// recounts with the index tie-break (values above its own, plus equal values at lower indices).
// CFG (ds_moe_top_k): top-K on the raw scores, then softmax over the K chosen in selection order
// (correctly rounded expf, max first, sequential sum); slots past the selectable count get expert 0
// and weight 0.
// DECODE (ds_moe_decoder.c:145-183): fast-exp softmax over all experts (max, sequential sum in
// expert order, 1/sum), top-K on the probabilities, weights = those probabilities; empty slots get
// expert -1 and weight -1e30.
__device__ __forceinline__ void route_select(int E, int K, int mode, int *s_idx, float *s_w, float (*s_red)[64],
                                             route_scratch *scr) {
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
  const float vk = selectable ? v : -__builtin_huge_valf();
  scr->key[lane] = vk;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  int rank = 0;
#pragma unroll
  for (int j = 0; j < 64; j++) rank += scr->key[j] > vk ? 1 : 0;
  const int nsel = __popcll(__ballot(selectable));
  const int ns = nsel < K ? nsel : K;  // experts selected
  bool put = selectable && rank < K;
  if (put) {
    scr->sel[rank] = lane;
    scr->val[rank] = v;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const bool mine = lane < ns;
  int my_sel = scr->sel[lane];
  float my_val = scr->val[lane];
  if (__ballot(put && scr->sel[rank] != lane)) {  // equal values among the first K: index tie-break
    rank = 0;
    for (int j = 0; j < 64; j++) {
      const float kj = scr->key[j];
      rank += (kj > vk || (kj == vk && j < lane)) ? 1 : 0;
    }
    put = selectable && rank < K;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // the reads above are done
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (put) {
      scr->sel[rank] = lane;
      scr->val[rank] = v;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    my_sel = scr->sel[lane];
    my_val = scr->val[lane];
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
