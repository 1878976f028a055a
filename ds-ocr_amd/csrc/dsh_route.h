// dsh_route.h — expert selection of one MoE layer from per-wave partial score sums, shared by the
// decode kernels (k_dec.hip) and the prefill kernels (k_prefill.hip) so both route identically.
#pragma once
#include "dsh.h"
#include "k_core.h"

// Wave 0 only, after a barrier that made s_red visible.
__device__ __forceinline__ void route_select(int E, int K, int mode, int *s_idx, float *s_w, float (*s_red)[64]) {
  const int lane = threadIdx.x & 63;
  {
    const float s = ((s_red[0][lane] + s_red[1][lane]) + s_red[2][lane]) + s_red[3][lane];
    bool taken = false;
    if (mode == DSH_ROUTE_CFG) {
      int my_sel = 0, ns = 0;
      float my_ss = 0.0f;
      for (int t = 0; t < K; t++) {
        unsigned long long key = (lane < E && !taken) ? dsh_argmax_key(s, lane) : 0ull;
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
      if (lane < K) {
        s_idx[lane] = lane < ns ? my_sel : 0;
        s_w[lane] = lane < ns ? ev * inv : 0.0f;
      }
    } else {
      float m = (lane < E && s > -1e30f) ? s : -1e30f;
      m = dsh_wave_max(m);
      float p = lane < E ? dsh_fast_expf(s - m) : 0.0f;
      float sum = 0.0f;
      for (int e = 0; e < E; e++) sum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), e));
      float inv = 1.0f / sum;
      p = p * inv;
      int my_sel = -1;
      float my_w = -1e30f;
      for (int t = 0; t < K; t++) {
        unsigned long long key = (lane < E && !taken) ? dsh_argmax_key(p, lane) : 0ull;
        key = dsh_wave_max_u64(key);
        int e = key == 0ull ? -1 : dsh_key_index(key);
        if (lane == e) taken = true;
        if (lane == t) {
          my_sel = e;
          my_w = key == 0ull ? -1e30f : dsh_key_value(key);
        }
      }
      if (lane < K) {
        s_idx[lane] = my_sel;
        s_w[lane] = my_w;
      }
    }
  }
}
