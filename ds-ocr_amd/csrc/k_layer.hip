// k_layer.hip — one kernel per MoE layer for the decode stacks (CFG routing with the f32 router;
// DECODE routing with the exact bf16 scores computed before each layer).
//
// The two-kernel layer (k_dec.hip) needs a grid-wide boundary between gate_up and down because
// every down row reads all of h. Here the down product is split over the intermediate dimension
// instead: a block owns DL_UB intermediate units of one expert (unit i = gate row i, up row i,
// down column i), computes their h values itself and adds its share of the down output,
// w_e * (scale[r] * Σ_{i in block} u[r][i] h_i + offset[r] * Σ_{i in block} h_i) for every output
// row r, into the layer output with float atomics (ds_quantize.c:301-320 per expert,
// ds_kernels.c:359-371 combine, ds_moe_decoder.c:278 shared add, :468 residual). The output is kept
// as DL_REP copies, one per XCD (the block adds into the copy of the XCD it runs on, which divides
// the atomics per address by DL_REP); its value is the sum of the copies in copy order, which the
// next layer's blocks form for themselves.
//
// The next layer's router scores are linear in this layer's output, so they accumulate the same
// way: Wr'·x_out = Wr'·x + Σ_blocks w_e (M_e[:, units]·h_units + z_e Σh_units) with
// M_e = Wr' diag(scale_e) U_e and z_e = Wr'·offset_e precomputed from the weights
// (k_layer_build_m), and Wr'·x split over the blocks by rows of x.
//
// The sums differ from the reference's order by f32 rounding (the combine adds the experts' shares
// in an order set by the atomics, so the low bits of the output may differ from run to run).
#include "dsh_avx.h"
#include "dsh_route.h"
#include "k_core.h"

#define DL_UB 32  // intermediate units per block
#define DL_REP 8  // copies of each accumulated output
#define DL_PF 32  // blocks that read the next layer's shared-expert data ahead

// The XCD this wave runs on: s_getreg_b32 hwreg(HW_REG_XCC_ID, 0, 4) (register id 20, 4 bits at
// offset 0). It only picks which copy the block adds into (every copy is summed), so any value is
// correct; the id spreads the atomics of different XCDs over different addresses.
__device__ __forceinline__ int dl_copy() { return __builtin_amdgcn_s_getreg((3 << 11) | 20) & (DL_REP - 1); }

// Loads of one block's units (512 threads, 8 waves): gate and up rows of four units per wave (16
// lanes per unit, CPL 16-byte pieces per lane); the thread's part of the down tile: rows t' + 256k
// (t' = t % 256) of the block's unit half t / 256 (16 columns: one 16-byte piece per row; piece
// q = 2k + half of all t' is one contiguous 4 KB run, so a wave's load reads 1 KB in one piece); the
// down (scale, offset) of those rows; and lane a's M row (a = router row) for the wave's four units.
template <int CPL>
struct dl_regs {
  u32x4 wg[CPL], wu[CPL];
  u32x4 wd[CPL];
  float2 sog, sou;
  float2 dso[CPL];
  f32x4 mv;
  float zv;
};

template <int CPL>
__device__ __forceinline__ void dl_issue(dl_regs<CPL> &R, const int8_t *gu, const float *guso, size_t gate0,
                                         size_t up0, const int8_t *tile, const float *dso, const float *mt,
                                         const float *z) {
  constexpr int H = 256 * CPL;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, sub = lane & 15, grp = lane >> 4;
  const int th = t & 255, half = t >> 8;
  const size_t u = 4 * wave + grp;
  const int8_t *grow = gu + (gate0 + u) * H, *urow = gu + (up0 + u) * H;
#pragma unroll
  for (int m = 0; m < CPL; m++) {
    R.wg[m] = dsh_load_nt(grow + 16 * (sub + 16 * m));
    R.wu[m] = dsh_load_nt(urow + 16 * (sub + 16 * m));
  }
#pragma unroll
  for (int k = 0; k < CPL; k++) R.wd[k] = dsh_load_nt(tile + ((size_t)(2 * k + half) * 256 + th) * 16);
  R.sog = ((const float2 *)guso)[gate0 + u];
  R.sou = ((const float2 *)guso)[up0 + u];
#pragma unroll
  for (int k = 0; k < CPL; k++) R.dso[k] = ((const float2 *)dso)[th + 256 * k];
  if (mt) {
    R.mv = *(const f32x4 *)(mt + (size_t)wave * 256 + lane * 4);
    R.zv = z[lane];
  }
}

// LDS of one layer block.
template <int CPL>
struct dl_smem {
  static constexpr int H = 256 * CPL, NP = 64 * CPL, NL = 4;
  float s_w[1];  // routed blocks: the expert weight
  float s_red[4][64];
  float s_stat[16];
  __attribute__((aligned(16))) unsigned s_lq[NL * NP];
  __attribute__((aligned(16))) float s_x[H];
  __attribute__((aligned(16))) float s_h[DL_UB];
  float s_dn[H];
  float s_lg[8][64];
};

// The block's work; SH: a shared-expert block (a compile-time split, so each kind of block runs
// straight-line code and every wait for a load counts only that kind's own loads). DS: DECODE routing
// with the router's rows (F.Wr_dec): a routed block computes the exact scores of its input itself,
// in the reference's order for rows in 4- and 2-row groups (avx_row_regs32, as k_dec_scores_bf16),
// instead of reading them as partials.
template <int CPL, int NREP, int RB, bool SH, bool DS>
__device__ __forceinline__ void dl_body(const dsh_layer_t &L, const dsh_split_t &F, const float *x_in,
                                        const int *__restrict__ step, int stride, const float *partials, int np,
                                        int mode, const float *__restrict__ resid, float *x_out, float *lg_out,
                                        float *zero_p, int zero_n, dl_smem<CPL> &S) {
  // x pieces (4 values each): piece p belongs to thread XO + p % XT of round p / XT
  constexpr int XO = 0, XT = 512 - XO;
  constexpr int H = 256 * CPL, NP = 64 * CPL, XV = (NP + XT - 1) / XT, NL = 4;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, sub = lane & 15, grp = lane >> 4;
  const int th = t & 255, half = t >> 8;
  const int I = L.I, SI = L.SI, NS = SI / DL_UB, NSL = I / DL_UB, blk = blockIdx.x;
  constexpr bool shared_blk = SH;
  const int rb = blk - NS, slot = shared_blk ? 0 : rb / NSL, sl = shared_blk ? blk : rb - slot * NSL;
  const float *x = step ? x_in + (size_t)(*step) * stride : x_in;

  for (int i = blk * 512 + t; i < zero_n; i += gridDim.x * 512) zero_p[i] = 0.0f;

  // Loads in the order they are needed (a wave's loads complete in issue order): the router
  // partials, then the input copies, the residual rows and the next router's rows.
  float pv[RB];
  if (!shared_blk && !DS && wave < 4) {
#pragma unroll
    for (int j = 0; j < RB; j++) pv[j] = partials[(size_t)min(wave + 4 * j, np - 1) * 64 + lane];
  }
  asm volatile("" ::: "memory");
  f32x4 xr[XV][NREP];
#pragma unroll
  for (int j = 0; j < XV; j++)
#pragma unroll
    for (int c = 0; c < NREP; c++) xr[j][c] = ((const f32x4 *)(x + (size_t)c * H))[min(max(t - XO, 0) + XT * j, NP - 1)];
  asm volatile("" ::: "memory");
  // DS: waves 0-3 of a routed block load router row 16 * wave + lane / 4 (4 lanes a row; lane
  // L = lane % 4 holds columns 32i + 8L .. 32i + 8L + 7 in piece i), used once x is in LDS
  constexpr int N32 = DS ? 8 * CPL : 1;
  u32x4 wv[N32];
  if constexpr (DS && !SH) {
    if (wave < 4) {
      const u32x4 *row = (const u32x4 *)(F.Wr_dec + (size_t)min(16 * wave + (lane >> 2), L.E - 1) * H);
#pragma unroll
      for (int i = 0; i < N32; i++) wv[i] = row[4 * i + (lane & 3)];
    }
    asm volatile("" ::: "memory");
  }
  float rv[CPL];  // block 0: the residual rows it adds (when it is not the input)
  if (blk == 0 && resid && !half) {
#pragma unroll
    for (int k = 0; k < CPL; k++) rv[k] = resid[th + 256 * k];
  }
  const bool base_blk = F.WrT_next && blk < H / 8;  // adds Wr'·x over rows 8*blk .. 8*blk + 7
  float wr[8];
  if (base_blk && wave == 0 && lane < F.E_next) {
#pragma unroll
    for (int j = 0; j < 8; j++) wr[j] = F.WrT_next[(size_t)(blk * 8 + j) * F.E_next + lane];
  }
  asm volatile("" ::: "memory");

  // A wave that issues its weight rows (15 loads per lane, 120 KB per block) cannot execute past
  // them until the memory system has accepted them, which takes about as long as they take to
  // arrive; whatever the wave does after the issue, and any barrier after it, waits that long. So
  // each block finishes its preparation (x summed and converted to limbs, the selection) first and
  // issues last, with no barrier between the issue and the dot products: each wave starts its gate
  // and up products as its own rows arrive. Shared-expert blocks need no selection and issue right
  // behind their input loads (which return first: a wave's loads complete in issue order). In a
  // routed block every wave runs the selection's rounds up to the block's slot itself; wave 0 then
  // finishes the rounds and the expert weight (the CFG softmax over all selected experts) while
  // its rows stream, and passes it through LDS.
  dl_regs<CPL> R;
  float wexp = 1.0f;  // this block's expert weight (1 for the shared expert)
  if constexpr (shared_blk) {
    dl_issue<CPL>(R, L.sgu_q, L.sgu_so, (size_t)sl * DL_UB, (size_t)SI + sl * DL_UB,
                  F.sdnT + (size_t)sl * DL_UB * H, L.sdn_so, F.sM ? F.sM + (size_t)sl * 2048 : nullptr, F.sz);
    asm volatile("" ::: "memory");
  }
  if (!shared_blk && wave < 4) {
    if constexpr (DS) {  // the scores go to row 0 (below); rows 1-3 add zeros, as a single partial's do
      if (wave > 0) S.s_red[wave][lane] = 0.0f;
    } else {
      float acc = 0.0f;
#pragma unroll
      for (int j = 0; j < RB; j++)
        if (wave + 4 * j < np) acc += pv[j];
      S.s_red[wave][lane] = lane < L.E ? acc : 0.0f;
    }
  }
  // x: the copies summed in copy order; max|x| and Σx per wave
  f32x4 xs[XV];
  {
    float mx = 0.0f, sx = 0.0f;
#pragma unroll
    for (int j = 0; j < XV; j++) {
      xs[j] = xr[j][0];
#pragma unroll
      for (int c = 1; c < NREP; c++) xs[j] += xr[j][c];
      const int p = t - XO + XT * j;
      const bool own = t >= XO && p < NP;
      if (own) *(f32x4 *)(S.s_x + 4 * p) = xs[j];
#pragma unroll
      for (int c = 0; c < 4; c++) {
        mx = own ? fmaxf(mx, fabsf(xs[j][c])) : mx;
        sx += own ? xs[j][c] : 0.0f;
      }
    }
    mx = dsh_wave_max(mx);
    sx = dsh_wave_sum(sx);
    if (lane == 0) {
      S.s_stat[wave] = mx;
      S.s_stat[8 + wave] = sx;
    }
  }
  __syncthreads();  // s_red, s_stat, s_x
  float xmax = S.s_stat[0], xsum = S.s_stat[8];
#pragma unroll
  for (int w = 1; w < 8; w++) {
    xmax = fmaxf(xmax, S.s_stat[w]);
    xsum += S.s_stat[8 + w];
  }
  const int ex = __builtin_amdgcn_frexp_expf(xmax);  // xmax < 2^ex
  if constexpr (DS && !SH) {  // the scores of x (s_x), row e into s_red[0][e]; read after the next barrier
    if (wave < 4) {
      const float v = avx_row_regs32<N32>(wv, S.s_x, lane & 3, true, 0.0f);
      const int e = 16 * wave + (lane >> 2);
      if ((lane & 3) == 0) S.s_red[0][e] = e < L.E ? v : 0.0f;
    }
  }

  // x → limbs, piece p (elements 4p..4p+3) into word p of each limb array
#pragma unroll
  for (int j = 0; j < XV; j++) {
    const int p = t - XO + XT * j;
    unsigned wl[NL] = {};
#pragma unroll
    for (int c = 0; c < 4; c++) {
      int X = (int)__builtin_rintf(__builtin_ldexpf(xs[j][c], 29 - ex));
#pragma unroll
      for (int l = 0; l < NL; l++) {
        const int d = l < NL - 1 ? __builtin_amdgcn_sbfe(X, 0, 8) : X;
        wl[l] |= ((unsigned)d & 255u) << (8 * c);
        X = (X - d) >> 8;
      }
    }
    if (t >= XO && p < NP) {
#pragma unroll
      for (int l = 0; l < NL; l++) S.s_lq[l * NP + p] = wl[l];
    }
  }
  __syncthreads();  // limbs
  if constexpr (!shared_blk) {
    route_state st;
    route_init(L.E, L.K, mode, S.s_red, st);
    const int r1 = min(slot + 1, st.ns);
    route_rounds(st, 0, r1);
    // the slot's expert: rank `slot` (an empty slot streams expert 0's rows, added with weight 0)
    const int e = slot < st.ns ? __builtin_amdgcn_readlane(st.sel, slot) : 0;
    const size_t g0 = (size_t)e * 2 * I + (size_t)sl * DL_UB;
    const size_t tile = (size_t)e * NSL + sl;
    dl_issue<CPL>(R, L.gu_q, L.gu_so, g0, g0 + I, F.dnT + tile * DL_UB * H, L.dn_so + (size_t)e * H * 2,
                  F.M ? F.M + tile * 2048 : nullptr, F.z ? F.z + (size_t)e * 64 : nullptr);
    asm volatile("" ::: "memory");
    if (wave == 0) {
      route_rounds(st, r1, st.ns);
      int idx;
      float w;
      route_finish(mode, st, idx, w);
      const float ws = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), slot));
      if (lane == 0) S.s_w[0] = slot < st.ns ? ws : 0.0f;  // DECODE: an empty slot adds with weight 0
    }
  }
  {
    int ag[NL] = {}, au[NL] = {};
#pragma unroll
    for (int m = 0; m < CPL; m++) {
      const int c = sub + 16 * m;
#pragma unroll
      for (int l = 0; l < NL; l++) {
        const u32x4 lw = *(const u32x4 *)(S.s_lq + l * NP + 4 * c);
#pragma unroll
        for (int d = 0; d < 4; d++) {
          ag[l] = __builtin_amdgcn_sdot4((int)R.wg[m][d], (int)lw[d], ag[l], false);
          au[l] = __builtin_amdgcn_sdot4((int)R.wu[m][d], (int)lw[d], au[l], false);
        }
      }
    }
    float dg = (float)ag[NL - 1], du = (float)au[NL - 1];
#pragma unroll
    for (int l = NL - 2; l >= 0; l--) {
      dg = __builtin_fmaf(dg, 256.0f, (float)ag[l]);
      du = __builtin_fmaf(du, 256.0f, (float)au[l]);
    }
    dg = __builtin_ldexpf(dsh_row16_sum(dg), ex - 29);
    du = __builtin_ldexpf(dsh_row16_sum(du), ex - 29);
    const float og = __builtin_fmaf(128.0f, R.sog.x, R.sog.y), ou = __builtin_fmaf(128.0f, R.sou.x, R.sou.y);
    const float g = __builtin_fmaf(R.sog.x, dg, og * xsum);
    const float up = __builtin_fmaf(R.sou.x, du, ou * xsum);
    if (sub == 0) S.s_h[4 * wave + grp] = dsh_swiglu(g, up);
  }
  __syncthreads();  // s_h, s_w
  if constexpr (!shared_blk) wexp = S.s_w[0];
  float hv[16];
#pragma unroll
  for (int j = 0; j < 16; j += 4) {
    const f32x4 v = *(const f32x4 *)(S.s_h + 16 * half + j);
    hv[j] = v[0];
    hv[j + 1] = v[1];
    hv[j + 2] = v[2];
    hv[j + 3] = v[3];
  }
  float dk[CPL];
#pragma unroll
  for (int k = 0; k < CPL; k++) dk[k] = dsh_dot16_u8(R.wd[k], hv, 0.0f);
  if (half) {
#pragma unroll
    for (int k = 0; k < CPL; k++) S.s_dn[th + 256 * k] = dk[k];
  }
  if (F.M) {  // the next layer's router scores: this wave's four units
    const f32x4 h4 = *(const f32x4 *)(S.s_h + 4 * wave);
    float pm = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; j++) pm = __builtin_fmaf(R.mv[j], h4[j], pm);
    S.s_lg[wave][lane] = pm;
  }
  __syncthreads();  // s_dn, s_lg
  float hs = 0.0f;  // Σh over the block's units
#pragma unroll
  for (int j = 0; j < DL_UB; j += 4) {
    const f32x4 v = *(const f32x4 *)(S.s_h + j);
    hs += v[0];
    hs += v[1];
    hs += v[2];
    hs += v[3];
  }
  const int cp = dl_copy();
  if (!half) {
    float *xo = x_out + (size_t)cp * H;
#pragma unroll
    for (int k = 0; k < CPL; k++) {
      const int r = th + 256 * k;
      const float d = dk[k] + S.s_dn[r];
      float c = wexp * __builtin_fmaf(R.dso[k].x, d, R.dso[k].y * hs);
      if (blk == 0) c += resid ? rv[k] : S.s_x[r];  // the residual, added once
      __hip_atomic_fetch_add(xo + r, c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  if (F.M && wave == 0 && lane < F.E_next) {
    float v = S.s_lg[0][lane];
#pragma unroll
    for (int w = 1; w < 8; w++) v += S.s_lg[w][lane];
    v = wexp * __builtin_fmaf(R.zv, hs, v);
    if (base_blk) {
#pragma unroll
      for (int j = 0; j < 8; j++) v = __builtin_fmaf(wr[j], S.s_x[blk * 8 + j], v);
    }
    __hip_atomic_fetch_add(lg_out + (size_t)cp * 64 + lane, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// The extra blocks: their share of the region to clear, then the next layer's shared-expert data
// (F.pf_*) read with ordinary loads while this layer's routed blocks are still selecting, so that
// layer's kernel reads it back faster (measured: its shared blocks finish ~1 us earlier; the L2
// does not keep the lines across the kernel boundary, the cache behind it does) and leaves more of
// HBM to its routed rows. Blocks are dealt to the 8 XCDs in turn, the same way in every launch of
// the same grid, so prefetch block p (XCD residue p % 8) reads the data of the shared blocks
// sl = p % 8 + 8 (p / 8 + 4 i), which run on that XCD in the next kernel. Nothing is written (the
// loaded words feed a condition that never holds, which keeps the loads).
template <int CPL>
__device__ __forceinline__ void dl_prefetch(const dsh_split_t &F, int nwork, float *x_out, float *zero_p, int zero_n) {
  constexpr int H = 256 * CPL;
  const int t = threadIdx.x, blk = blockIdx.x;
  for (int i = blk * 512 + t; i < zero_n; i += gridDim.x * 512) zero_p[i] = 0.0f;
  const int p = blk - nwork, ns = F.pf_SI / DL_UB;
  unsigned acc = 0;
  for (int sl = (p & 7) + 8 * (p >> 3); sl < ns; sl += 8 * (DL_PF / 8)) {
    const u32x4 *g = (const u32x4 *)(F.pf_gu + (size_t)sl * DL_UB * H);
    const u32x4 *u = (const u32x4 *)(F.pf_gu + (size_t)(F.pf_SI + sl * DL_UB) * H);
    const u32x4 *d = (const u32x4 *)(F.pf_dnT + (size_t)sl * DL_UB * H);
    u32x4 v[3 * CPL + 2];
#pragma unroll
    for (int k = 0; k < CPL; k++) {  // each region DL_UB x H bytes: CPL 16-byte pieces per thread
      v[k] = g[t + 512 * k];
      v[CPL + k] = u[t + 512 * k];
      v[2 * CPL + k] = d[t + 512 * k];
    }
    v[3 * CPL] = F.pf_M ? ((const u32x4 *)(F.pf_M + (size_t)sl * DL_UB * 64))[t] : u32x4{0, 0, 0, 0};
    v[3 * CPL + 1] = u32x4{0, 0, 0, 0};
    if (t < 16) v[3 * CPL + 1] = ((const u32x4 *)(F.pf_guso + 2 * (size_t)sl * DL_UB))[t];
    else if (t < 32) v[3 * CPL + 1] = ((const u32x4 *)(F.pf_guso + 2 * (size_t)(F.pf_SI + sl * DL_UB)))[t - 16];
#pragma unroll
    for (int k = 0; k < 3 * CPL + 2; k++) acc ^= v[k][0] ^ v[k][1] ^ v[k][2] ^ v[k][3];
  }
  if (acc == 0x9E3779B9u && F.pf_SI < 0) x_out[0] = 0.0f;
}

// x_out copies [DL_REP][H] and lg_out copies [DL_REP][64] must be zero when the kernel starts
// (the kernel of the layer after next, or the final sum, clears them: zero_p/zero_n).
// NREP: copies of the input (1: a plain vector at x_in + step*stride); RB: router partial rows
// loaded per wave by waves 0-3 (np <= 4 * RB). Blocks 0 .. SI/DL_UB - 1 run the shared expert.
template <int CPL, int NREP, int RB>
__global__ void __launch_bounds__(512) k_dec_layer(dsh_layer_t L, dsh_split_t F, const float *x_in,
                                                   const int *__restrict__ step, int stride,
                                                   const float *partials, int np, int mode,
                                                   const float *__restrict__ resid, float *x_out, float *lg_out,
                                                   float *zero_p, int zero_n) {
  __shared__ dl_smem<CPL> S;
  const int nwork = (L.SI + L.K * L.I) / DL_UB;
  if ((int)blockIdx.x >= nwork) {
    dl_prefetch<CPL>(F, nwork, x_out, zero_p, zero_n);
    return;
  }
  if ((int)blockIdx.x < L.SI / DL_UB)
    dl_body<CPL, NREP, RB, true, false>(L, F, x_in, step, stride, partials, np, mode, resid, x_out, lg_out, zero_p,
                                        zero_n, S);
  else
    dl_body<CPL, NREP, RB, false, false>(L, F, x_in, step, stride, partials, np, mode, resid, x_out, lg_out, zero_p,
                                         zero_n, S);
}

// DECODE routing with the scores computed in the routed blocks (F.Wr_dec; CPL <= 5, so a lane's
// router pieces fit in registers next to the input copies).
template <int CPL, int NREP>
__global__ void __launch_bounds__(512) k_dec_layer_ds(dsh_layer_t L, dsh_split_t F, const float *x_in,
                                                      const int *__restrict__ step, int stride,
                                                      const float *__restrict__ resid, float *x_out, float *lg_out,
                                                      float *zero_p, int zero_n) {
  __shared__ dl_smem<CPL> S;
  const int nwork = (L.SI + L.K * L.I) / DL_UB;
  if ((int)blockIdx.x >= nwork) {
    dl_prefetch<CPL>(F, nwork, x_out, zero_p, zero_n);
    return;
  }
  if ((int)blockIdx.x < L.SI / DL_UB)
    dl_body<CPL, NREP, 1, true, true>(L, F, x_in, step, stride, nullptr, 1, DSH_ROUTE_DECODE, resid, x_out, lg_out,
                                      zero_p, zero_n, S);
  else
    dl_body<CPL, NREP, 1, false, true>(L, F, x_in, step, stride, nullptr, 1, DSH_ROUTE_DECODE, resid, x_out, lg_out,
                                       zero_p, zero_n, S);
}

// out[i] = Σ_c X[c][i] in copy order, then X is cleared; zero_p[0..zero_n) is cleared too.
__global__ void __launch_bounds__(256) k_dec_copy_sum(float *X, int H, float *out, float *zero_p, int zero_n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < H) {
    float v[DL_REP];
#pragma unroll
    for (int c = 0; c < DL_REP; c++) v[c] = X[(size_t)c * H + i];
    float s = v[0];
#pragma unroll
    for (int c = 1; c < DL_REP; c++) s += v[c];
    out[i] = s;
#pragma unroll
    for (int c = 0; c < DL_REP; c++) X[(size_t)c * H + i] = 0.0f;
  }
  for (int j = i; j < zero_n; j += gridDim.x * 256) zero_p[j] = 0.0f;
}

// ============================================================================ derived weights
// Down tiles: for expert e and unit block s, tile[2k + j/16][t][j % 16] = dn[e][t + 256k][DL_UB*s + j]
// (bytes): piece q = 2k + j/16 of thread t's rows sits at (q*256 + t)*16.
__global__ void __launch_bounds__(256) k_layer_build_tiles(const int8_t *__restrict__ dn, int H, int I, int n_mat,
                                                           int8_t *__restrict__ tiles) {
  const int CPL = H / 256;
  const size_t per_mat = (size_t)H * I / 16;  // 16-byte pieces
  const size_t n = per_mat * n_mat;
  for (size_t g = (size_t)blockIdx.x * 256 + threadIdx.x; g < n; g += (size_t)gridDim.x * 256) {
    const size_t mat = g / per_mat, w = g - mat * per_mat;
    // w enumerates the tile pieces in order: s, q = 2k + half, t
    const int t = (int)(w % 256);
    size_t rest = w / 256;
    const int q = (int)(rest % (2 * CPL));
    const int s = (int)(rest / (2 * CPL));
    const int k = q >> 1, half = q & 1;
    const int r = t + 256 * k, i = DL_UB * s + 16 * half;
    const u32x4 v = *(const u32x4 *)(dn + (mat * H + r) * (size_t)I + i);
    *(u32x4 *)(tiles + g * 16) = v;
  }
}

// M tiles for expert e and unit block s: m[w][jj/4][a][jj%4] = Σ_r WrT[r][a] * scale[r] * u[r][DL_UB*s + 8w + jj]
// (u = stored code ^ 0x80, 0..255), accumulated in double; rows a >= E are 0. One block per tile.
__global__ void __launch_bounds__(256) k_layer_build_m(const int8_t *__restrict__ dn, const float *__restrict__ so,
                                                       const float *__restrict__ WrT, int H, int I, int E,
                                                       float *__restrict__ M) {
  const int NSL = I / DL_UB, tile = blockIdx.x, mat = tile / NSL, s = tile - mat * NSL;
  const int a = threadIdx.x & 63, w = threadIdx.x >> 6;
  double acc[8] = {};
  if (a < E) {
    const int8_t *base = dn + (size_t)mat * H * I + DL_UB * s + 8 * w;
    for (int r = 0; r < H; r++) {
      const double c = (double)WrT[(size_t)r * E + a] * (double)so[((size_t)mat * H + r) * 2];
      const uint2 q = *(const uint2 *)(base + (size_t)r * I);
#pragma unroll
      for (int jj = 0; jj < 8; jj++) {
        const unsigned word = jj < 4 ? q.x : q.y;
        const double u = (double)(((word >> (8 * (jj & 3))) & 255u) ^ 128u);
        acc[jj] += c * u;
      }
    }
  }
  float *dst = M + ((size_t)tile * 4 + w) * 512 + a * 4;
#pragma unroll
  for (int jj = 0; jj < 8; jj++) dst[(jj >> 2) * 256 + (jj & 3)] = (float)acc[jj];
}

// z[mat][a] = Σ_r WrT[r][a] * offset[r] (double accumulation); one 64-lane block per matrix.
__global__ void __launch_bounds__(64) k_layer_build_z(const float *__restrict__ so, const float *__restrict__ WrT,
                                                      int H, int E, float *__restrict__ z) {
  const int mat = blockIdx.x, a = threadIdx.x;
  double acc = 0.0;
  if (a < E)
    for (int r = 0; r < H; r++) acc += (double)WrT[(size_t)r * E + a] * (double)so[((size_t)mat * H + r) * 2 + 1];
  z[(size_t)mat * 64 + a] = (float)acc;
}

extern "C" {

int dsh_layer_split_supported(const dsh_layer_t *L) {
  return L->H % 256 == 0 && L->H / 256 <= 8 && L->I % DL_UB == 0 && L->SI % DL_UB == 0 && L->E <= 64 &&
         L->K <= L->E && L->H / 8 <= dsh_layer_split_blocks(L);
}

int dsh_layer_split_blocks(const dsh_layer_t *L) { return (L->SI + L->K * L->I) / DL_UB; }

int dsh_layer_split_copies(void) { return DL_REP; }

int dsh_layer_dec_scores_fusable(int H, int E, int nthreads) {
  if (H <= 0 || H > 1280 || H % 256 || E <= 0 || E > 64) return 0;
  const int chunk = dsh_chunk_len(E, nthreads);
  for (int s0 = 0; s0 < E; s0 += chunk)
    if (min(chunk, E - s0) % 2) return 0;  // an odd chunk ends in a single row
  return 1;
}

size_t dsh_layer_split_tile_bytes(const dsh_layer_t *L) { return (size_t)(L->E * L->I + L->SI) * L->H; }

size_t dsh_layer_split_m_floats(const dsh_layer_t *L) { return (size_t)(L->E * L->I + L->SI) * 64; }

hipError_t dsh_launch_layer_build(const dsh_layer_t *L, const float *WrT_next, int E_next, int8_t *dnT, int8_t *sdnT,
                                  float *M, float *sM, float *z, float *sz, hipStream_t s) {
  const int H = L->H, I = L->I, SI = L->SI, E = L->E;
  k_layer_build_tiles<<<2048, 256, 0, s>>>(L->dn_q, H, I, E, dnT);
  k_layer_build_tiles<<<256, 256, 0, s>>>(L->sdn_q, H, SI, 1, sdnT);
  if (WrT_next) {
    k_layer_build_m<<<E * (I / DL_UB), 256, 0, s>>>(L->dn_q, L->dn_so, WrT_next, H, I, E_next, M);
    k_layer_build_m<<<SI / DL_UB, 256, 0, s>>>(L->sdn_q, L->sdn_so, WrT_next, H, SI, E_next, sM);
    k_layer_build_z<<<E, 64, 0, s>>>(L->dn_so, WrT_next, H, E_next, z);
    k_layer_build_z<<<1, 64, 0, s>>>(L->sdn_so, WrT_next, H, E_next, sz);
  }
  return hipGetLastError();
}

hipError_t dsh_launch_dec_layer(const dsh_layer_t *L, const dsh_split_t *F, const float *x_in, const int *step,
                                int stride, int ncopies, const float *partials, int np, int route_mode,
                                const float *resid, float *x_out, float *lg_out, float *zero_p, int zero_n,
                                hipStream_t s) {
  const int nb = dsh_layer_split_blocks(L) + (F->pf_gu ? DL_PF : 0);
  if (ncopies != 1 && ncopies != DL_REP) return hipErrorInvalidValue;
  if (F->pf_gu && (!F->pf_dnT || !F->pf_guso || F->pf_SI <= 0 || F->pf_SI % DL_UB)) return hipErrorInvalidValue;
  if (F->Wr_dec) {  // the scores from the router rows: partials and np are not read
    if (route_mode != DSH_ROUTE_DECODE || F->M || L->H > 1280 || L->E > 64) return hipErrorInvalidValue;
#define DLS(N)                                                                                                   \
  case N:                                                                                                        \
    if (ncopies == 1)                                                                                            \
      k_dec_layer_ds<N, 1><<<nb, 512, 0, s>>>(*L, *F, x_in, step, stride, resid, x_out, lg_out, zero_p, zero_n); \
    else                                                                                                         \
      k_dec_layer_ds<N, DL_REP><<<nb, 512, 0, s>>>(*L, *F, x_in, step, stride, resid, x_out, lg_out, zero_p,     \
                                                   zero_n);                                                      \
    break;
    switch (L->H / 256) {
      DLS(1) DLS(2) DLS(3) DLS(4) DLS(5)
      default:
        return hipErrorInvalidValue;
    }
#undef DLS
    return hipGetLastError();
  }
  if (np < 1 || (ncopies == 1 ? np > 160 : np > 8)) return hipErrorInvalidValue;
  if (route_mode != DSH_ROUTE_CFG && (route_mode != DSH_ROUTE_DECODE || np != 1 || F->M)) return hipErrorInvalidValue;
#define DLK(N)                                                                                                   \
  case N:                                                                                                        \
    if (ncopies == 1)                                                                                            \
      k_dec_layer<N, 1, 40><<<nb, 512, 0, s>>>(*L, *F, x_in, step, stride, partials, np, route_mode, resid,    \
                                               x_out, lg_out, zero_p, zero_n);                                                          \
    else                                                                                                         \
      k_dec_layer<N, DL_REP, 2><<<nb, 512, 0, s>>>(*L, *F, x_in, step, stride, partials, np, route_mode, resid, \
                                                   x_out, lg_out, zero_p, zero_n);                                              \
    break;
  switch (L->H / 256) {
    DLK(1) DLK(2) DLK(3) DLK(4) DLK(5) DLK(6) DLK(7) DLK(8)
    default:
      return hipErrorInvalidValue;
  }
#undef DLK
  return hipGetLastError();
}

hipError_t dsh_launch_dec_copy_sum(float *X, int H, float *out, float *zero_p, int zero_n, hipStream_t s) {
  k_dec_copy_sum<<<(H + 255) / 256, 256, 0, s>>>(X, H, out, zero_p, zero_n);
  return hipGetLastError();
}

}  // extern "C"
