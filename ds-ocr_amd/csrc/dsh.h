// dsh.h — device helpers shared by the gfx950 kernels of the ds-ocr INT8 MoE decode path.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

#define DSH_WAVE 64

// ---------------------------------------------------------------- scalar semantics

__device__ __forceinline__ float dsh_bf16_to_f32(uint32_t b16) { return __uint_as_float(b16 << 16); }
__device__ __forceinline__ float dsh_bf16lo(uint32_t packed) { return __uint_as_float(packed << 16); }
__device__ __forceinline__ float dsh_bf16hi(uint32_t packed) { return __uint_as_float(packed & 0xFFFF0000u); }

// Schraudolph fast exp of ds_kernels.h:296-302, as the reference build evaluates it: the affine map
// is one fused multiply-add (GCC contracts 12102203*x + 1064866805), the float->uint32 conversion
// goes through a signed integer (the scalar x86 code), so a negative result wraps instead of
// saturating. The fmaf here is an explicit fused op, independent of contraction flags.
__device__ __forceinline__ float dsh_fast_expf(float x) {
  if (x < -88.0f) return 0.0f;
  if (x > 88.0f) return 1e38f;
  float v = __builtin_fmaf(12102203.0f, x, 1064866805.0f);
  uint32_t i = (v != v) ? 0u : (uint32_t)(int32_t)v;
  return __uint_as_float(i);
}

// expf rounded correctly (exp in double precision, then one rounding to float). The reference's
// ds_moe_top_k calls the host's expf (ds_kernels.c:233), glibc 2.35's on the benchmark hosts; over
// every float in [-104, 0] (the softmax's arguments, x - max) that agrees with the correctly rounded
// value except on 97,052 of 1,120,927,745 arguments (8.7e-5), where glibc is 1 ulp off.
__device__ __forceinline__ float dsh_expf_cr(float x) { return (float)exp((double)x); }

// ds_swiglu_direct element (ds_kernels.c:1771): (g / (1 + fe(-g))) * u. Division is IEEE
// correctly rounded (hipcc default), matching the x86 divss.
__device__ __forceinline__ float dsh_swiglu(float g, float u) { return (g / (1.0f + dsh_fast_expf(-g))) * u; }

// ds_bf16_truncate_array element (ds_kernels.c:2484-2490): round-half-up on the bit pattern.
__device__ __forceinline__ float dsh_bf16_round_half_up(float f) {
  return __uint_as_float((__float_as_uint(f) + 0x8000u) & 0xFFFF0000u);
}

// ---------------------------------------------------------------- wave helpers

template <int CTRL>
__device__ __forceinline__ float dsh_dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over each aligned group of 16 lanes (one DPP row); every lane of the row gets the sum.
__device__ __forceinline__ float dsh_row16_sum(float v) {
  v += dsh_dpp<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dsh_dpp<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dsh_dpp<0x141>(v);  // row_half_mirror
  v += dsh_dpp<0x140>(v);  // row_mirror
  return v;
}

// Sum over each aligned group of 8 lanes; every lane of the group gets the sum.
__device__ __forceinline__ float dsh_row8_sum(float v) {
  v += dsh_dpp<0xB1>(v);
  v += dsh_dpp<0x4E>(v);
  v += dsh_dpp<0x141>(v);
  return v;
}

// Sum over each aligned group of 4 lanes.
__device__ __forceinline__ float dsh_row4_sum(float v) {
  v += dsh_dpp<0xB1>(v);
  v += dsh_dpp<0x4E>(v);
  return v;
}

__device__ __forceinline__ float dsh_readlane(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Sum over the wave, (r0 + r1) + (r2 + r3) of the four 16-lane row sums; the result is uniform.
// Row sums by DPP, rows combined through readlane (no LDS permutes on the critical path).
__device__ __forceinline__ float dsh_wave_sum(float v) {
  v = dsh_row16_sum(v);
  return (dsh_readlane(v, 0) + dsh_readlane(v, 16)) + (dsh_readlane(v, 32) + dsh_readlane(v, 48));
}

__device__ __forceinline__ float dsh_wave_max(float v) {
  v = fmaxf(v, dsh_dpp<0xB1>(v));
  v = fmaxf(v, dsh_dpp<0x4E>(v));
  v = fmaxf(v, dsh_dpp<0x141>(v));
  v = fmaxf(v, dsh_dpp<0x140>(v));
  return fmaxf(fmaxf(dsh_readlane(v, 0), dsh_readlane(v, 16)), fmaxf(dsh_readlane(v, 32), dsh_readlane(v, 48)));
}

// ---------------------------------------------------------------- INT8 code helpers

// Stored codes are int8 q = u - 128 (ds_quantize.c:45); as bytes that is u ^ 0x80, so one XOR per
// dword recovers u and one conversion per byte (v_cvt_f32_ubyteN) gives it exactly as a float.
__device__ __forceinline__ void dsh_u8x4_to_f32(uint32_t w, float &a, float &b, float &c, float &d) {
  uint32_t u = w ^ 0x80808080u;
  a = (float)(u & 0xFFu);  // selected as v_cvt_f32_ubyte0..3
  b = (float)((u >> 8) & 0xFFu);
  c = (float)((u >> 16) & 0xFFu);
  d = (float)(u >> 24);
}

// dot += Σ u_j * x_j over 16 codes in one 128-bit word.
__device__ __forceinline__ float dsh_dot16_u8(u32x4 w, const float *x, float acc) {
#pragma unroll
  for (int d = 0; d < 4; d++) {
    float a, b, c, e;
    dsh_u8x4_to_f32(w[d], a, b, c, e);
    acc = __builtin_fmaf(a, x[4 * d + 0], acc);
    acc = __builtin_fmaf(b, x[4 * d + 1], acc);
    acc = __builtin_fmaf(c, x[4 * d + 2], acc);
    acc = __builtin_fmaf(e, x[4 * d + 3], acc);
  }
  return acc;
}

__device__ __forceinline__ u32x4 dsh_load_nt(const void *p) {
  return __builtin_nontemporal_load((const u32x4 *)p);
}

// The reference's INT8 row loop in its own order (int8_matvec_generic, ds_quantize.c:163-166, which
// GCC keeps scalar and contracts): dot = fma(u_j, x_j, dot) for j = 0, 1, ... with the exact code
// u = q + 128, and with XS also xs += x_j in the same loop. One lane runs one row, so the result
// is bit-identical to the reference's. row: 16-byte aligned, n % 16 == 0; x in LDS (the lanes of a
// wave read the same x_j at once: a broadcast). Loads run PF 16-byte chunks ahead in registers.
template <bool XS>
__device__ __forceinline__ float dsh_row_chain(const int8_t *row, const float *x, int n, float &xs) {
  constexpr int PF = 16;
  const int C = n >> 4;
  u32x4 buf[PF];
#pragma unroll
  for (int j = 0; j < PF; j++) buf[j] = j < C ? dsh_load_nt(row + 16 * j) : u32x4{0u, 0u, 0u, 0u};
  float dot = 0.0f;
  for (int g = 0; g < C; g += PF) {
    u32x4 cur[PF];
#pragma unroll
    for (int j = 0; j < PF; j++) cur[j] = buf[j];
#pragma unroll
    for (int j = 0; j < PF; j++)
      if (g + PF + j < C) buf[j] = dsh_load_nt(row + 16 * (g + PF + j));
#pragma unroll
    for (int j = 0; j < PF; j++) {
      if (g + j < C) {
        const float *xc = x + 16 * (g + j);
#pragma unroll
        for (int d = 0; d < 4; d++) {
          float u[4];
          dsh_u8x4_to_f32(cur[j][d], u[0], u[1], u[2], u[3]);
          const f32x4 xv = *(const f32x4 *)(xc + 4 * d);
#pragma unroll
          for (int c = 0; c < 4; c++) {
            dot = __builtin_fmaf(u[c], xv[c], dot);
            if (XS) xs += xv[c];
          }
        }
      }
    }
  }
  return dot;
}

__device__ __forceinline__ f32x4 dsh_load_f4(const float *p) { return *(const f32x4 *)p; }

// ---------------------------------------------------------------- argmax key

// Orderable key for (value, index): larger value wins, then smaller index. Only values strictly
// greater than -1e30 and not NaN can win (ds_kernels_avx.c:159-160 initial best_val = -1e30 with
// strict '>'); key 0 means "no candidate". -0 and +0 compare equal in the reference, so both map
// to the +0 key and the index decides.
__device__ __forceinline__ unsigned long long dsh_argmax_key(float v, int idx) {
  if (!(v > -1e30f)) return 0ull;
  uint32_t u = __float_as_uint(v);
  if ((u << 1) == 0u) u = 0u;
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((unsigned long long)u << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)idx);
}
__device__ __forceinline__ int dsh_key_index(unsigned long long k) {
  return k == 0ull ? 0 : (int)(0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFull));
}
__device__ __forceinline__ float dsh_key_value(unsigned long long k) {
  if (k == 0ull) return -1e30f;
  uint32_t u = (uint32_t)(k >> 32);
  u = (u & 0x80000000u) ? (u & 0x7FFFFFFFu) : ~u;
  return __uint_as_float(u);
}
__device__ __forceinline__ unsigned long long dsh_umax64(unsigned long long a, unsigned long long b) {
  return a > b ? a : b;
}
// Transposed butterfly sums of V per-lane values over the wave (V = 8 or 16). Each exchange halves
// the values a lane carries: lanes whose partner bit is 0 keep the lower half of the pairs (j, j+V/2)
// and lanes with the bit set the upper half (v_permlane32_swap for lane bit 5, v_permlane16_swap for
// bit 4, a DPP row rotation or mirror with a select for bits 3 (and 2)); the last lane bits are
// summed by DPP. On return lane l holds the sum of value l >> (6 - log2 V), i.e. value j sits in
// lanes j*64/V .. j*64/V + 64/V - 1, all with the same bits.
__device__ __forceinline__ void dsh_pl32_add(float *v, int half) {
  for (int j = 0; j < half; j++) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[j]), __float_as_uint(v[j + half]), false, false);
    v[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
}
__device__ __forceinline__ void dsh_pl16_add(float *v, int half) {
  for (int j = 0; j < half; j++) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[j]), __float_as_uint(v[j + half]), false, false);
    v[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
}
// lanes with bit B keep value "hi", the others "lo"; the partner (CTRL) has the opposite bit B
template <int CTRL>
__device__ __forceinline__ float dsh_halve(float lo, float hi, bool bit) {
  const float keep = bit ? hi : lo, send = bit ? lo : hi;
  return keep + dsh_dpp<CTRL>(send);
}
__device__ __forceinline__ float dsh_wave_tsum8(const float *in) {
  const int lane = threadIdx.x & 63;
  float v[8];
#pragma unroll
  for (int j = 0; j < 8; j++) v[j] = in[j];
  dsh_pl32_add(v, 4);
  dsh_pl16_add(v, 2);
  float z = dsh_halve<0x128>(v[0], v[1], lane & 8);  // row_ror:8 pairs lane l with l ^ 8
  z += dsh_dpp<0x141>(z);                            // row_half_mirror
  z += dsh_dpp<0x4E>(z);
  z += dsh_dpp<0xB1>(z);
  return z;
}
__device__ __forceinline__ float dsh_wave_tsum16(const float *in) {
  const int lane = threadIdx.x & 63;
  float v[16];
#pragma unroll
  for (int j = 0; j < 16; j++) v[j] = in[j];
  dsh_pl32_add(v, 8);
  dsh_pl16_add(v, 4);
  float y0 = dsh_halve<0x128>(v[0], v[2], lane & 8);
  float y1 = dsh_halve<0x128>(v[1], v[3], lane & 8);
  float z = dsh_halve<0x141>(y0, y1, lane & 4);  // row_half_mirror pairs l with 7 - l (bit 2 flipped)
  z += dsh_dpp<0x4E>(z);
  z += dsh_dpp<0xB1>(z);
  return z;
}

template <int CTRL>
__device__ __forceinline__ unsigned long long dsh_dpp64(unsigned long long v) {
  uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
  lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)lo, CTRL, 0xF, 0xF, false);
  hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)hi, CTRL, 0xF, 0xF, false);
  return ((unsigned long long)hi << 32) | lo;
}
__device__ __forceinline__ unsigned long long dsh_readlane64(unsigned long long v, int lane) {
  uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, lane);
  uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), lane);
  return ((unsigned long long)hi << 32) | lo;
}
// Maximum over the wave (uniform result): DPP within each 16-lane row, readlane across rows.
__device__ __forceinline__ unsigned long long dsh_wave_max_u64(unsigned long long v) {
  v = dsh_umax64(v, dsh_dpp64<0xB1>(v));
  v = dsh_umax64(v, dsh_dpp64<0x4E>(v));
  v = dsh_umax64(v, dsh_dpp64<0x141>(v));
  v = dsh_umax64(v, dsh_dpp64<0x140>(v));
  return dsh_umax64(dsh_umax64(dsh_readlane64(v, 0), dsh_readlane64(v, 16)),
                    dsh_umax64(dsh_readlane64(v, 32), dsh_readlane64(v, 48)));
}
