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
#include "dsh_cert.h"
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
  // certified CFG routing: the verdict state and arrival rank; the verifier's segment sums / offsets
  // (s_vS), running sizes (s_vA), rows for the selection (s_vr) and its result, the gathered sums
  int s_ev, s_claim;
  float s_vS[8][64], s_vA[8][64];
  float s_vr[4][64];
  int s_vi[8], s_si[8];
  float s_vw[8], s_sw[8];
  double s_vG[8][64], s_vT[3][8][64];
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
                                        float *zero_p, int zero_n, int blk, dl_smem<CPL> &S) {
  // x pieces (4 values each): piece p belongs to thread XO + p % XT of round p / XT
  constexpr int XO = 0, XT = 512 - XO;
  constexpr int H = 256 * CPL, NP = 64 * CPL, XV = (NP + XT - 1) / XT, NL = 4;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, sub = lane & 15, grp = lane >> 4;
  const int th = t & 255, half = t >> 8;
  const int I = L.I, SI = L.SI, NS = SI / DL_UB, NSL = I / DL_UB;
  constexpr bool shared_blk = SH;
  const int rb = blk - NS, slot = shared_blk ? 0 : rb / NSL, sl = shared_blk ? blk : rb - slot * NSL;
  const float *x = step ? x_in + (size_t)(*step) * stride : x_in;

  for (int i = blockIdx.x * 512 + t; i < zero_n; i += gridDim.x * 512) zero_p[i] = 0.0f;

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
      if (mode == DSH_ROUTE_DECODE && F.rc.log && rb == 0) {  // the routing log (a test aid): one block
        if (lane < 8) {
          S.s_vi[lane] = lane < L.K ? idx : -1;
          S.s_vw[lane] = lane < L.K ? w : 0.0f;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (lane == 0) {
          dsh_rcert_t r = F.rc;
          r.stats = nullptr;  // the counters count CFG routings only
          cert_record(r, S.s_vi, S.s_vw, L.K, 0, S.s_x, H);
        }
      }
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

// Certified CFG routing in the one-kernel layer (dsh_split_t.vd). The routed blocks select from the
// accumulated scores and add their shares at once; meanwhile the DL_NPART extra blocks compute the
// layer's exact router scores from its input, a slice of the router rows each (so the router is
// read once per layer), with the running-error bound of ds_linear's order, and the last to finish
// certifies the selection (dsh_cert.h). Should the certified set of experts differ from the one the
// routed blocks used (a near tie that the accumulated scores ranked otherwise), the extra blocks add
// the difference, Δw_e (h_e → down) for every expert in either set, so the layer's output is the
// one of the certified selection.
//
// The verdict area (DL_VX ints, zero when the kernel starts): [0] parts done, [2] verdict (1: the
// selection stands, 2: corrected), [3] experts to correct, [16..27] their indices, [32..43] their
// Δw; from DL_VP, per part j: [256 j ..] the part's sum S_j (64 f64), [+128] its bound sum U_j (64
// f32), [+192] its own rounding sum A_j (64 f32). Written and read with device-scope atomics; a
// writer waits for its stores before it counts itself done or publishes the verdict.
#ifndef DL_NPART
#define DL_NPART 32  // extra blocks that verify: H / DL_NPART router rows each (a multiple of 8, <= 32)
#endif
#define DL_VP 64     // first int of the parts' results
#define DL_VX (DL_VP + 256 * DL_NPART)
#define DL_VD_SPIN (1 << 18)  // polls of the verdict word before a waiting extra block gives up

// The next layer's shared-expert data (F.pf_*) read ahead by the extra blocks while this layer's
// routed blocks are still at work, so that layer's kernel reads it back faster (measured: its
// shared blocks finish ~1 us earlier; the L2 does not keep the lines across the kernel boundary,
// the cache behind it does, which all XCDs share) and leaves more of HBM to its routed rows. Extra
// block p reads the data of the shared blocks sl = p + DL_PF i. Nothing is written (the loaded
// words feed a condition that never holds, which keeps the loads). dl_pf_load issues one slice's
// loads (its gate, up and transposed down rows, M rows, scales), dl_pf_fold consumes them.
#define DL_PFV(CPL) (3 * (CPL) + 2)
template <int CPL>
__device__ __forceinline__ void dl_pf_load(const dsh_split_t &F, int sl, u32x4 (&v)[DL_PFV(CPL)]) {
  constexpr int H = 256 * CPL;
  const int t = threadIdx.x;
  const u32x4 *g = (const u32x4 *)(F.pf_gu + (size_t)sl * DL_UB * H);
  const u32x4 *u = (const u32x4 *)(F.pf_gu + (size_t)(F.pf_SI + sl * DL_UB) * H);
  const u32x4 *d = (const u32x4 *)(F.pf_dnT + (size_t)sl * DL_UB * H);
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
}

template <int CPL>
__device__ __forceinline__ unsigned dl_pf_fold(const u32x4 (&v)[DL_PFV(CPL)]) {
  unsigned acc = 0;
#pragma unroll
  for (int k = 0; k < DL_PFV(CPL); k++) acc ^= v[k][0] ^ v[k][1] ^ v[k][2] ^ v[k][3];
  return acc;
}

// The next step's router partials (F.nx_partials; the last layer's extra block p): wave w of the
// block takes partials 8 p + w, 8 p + w + 8 DL_PF, ... of R rows each, lane = expert, as
// k_dec_partial_scores computes them (a fused multiply-add chain over the rows in order from 0).
// The step counter is still this step's (the LM head advances it after this kernel).
template <int CPL, int R>
__device__ __forceinline__ void dl_next_partials_r(const dsh_split_t &F, int p, const float *x) {
  constexpr int H = 256 * CPL;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, E = F.nx_E;
  for (int g = 8 * p + wave; g < H / R; g += 8 * DL_PF) {
    const int r0 = g * R;
    float acc = 0.0f;
    if (lane < E) {
      float w[R], xv[R];
#pragma unroll
      for (int j = 0; j < R; j++) {
        w[j] = F.nx_WrT[(size_t)(r0 + j) * E + lane];
        xv[j] = x[r0 + j];
      }
#pragma unroll
      for (int j = 0; j < R; j++) acc = __builtin_fmaf(w[j], xv[j], acc);
    }
    F.nx_partials[(size_t)g * 64 + lane] = lane < E ? acc : 0.0f;
  }
}
template <int CPL>
__device__ __forceinline__ void dl_next_partials(const dsh_split_t &F, int p) {
  const int sn = *F.nx_step + 1;
  if (p == 0 && threadIdx.x == 0) *F.nx_pending = 1;  // this step's token: the LM head's keys, turned later
  if (sn >= F.nx_rows) return;                        // no next row in the bound input
  const float *x = F.nx_in + (size_t)sn * F.nx_stride;
  if (F.nx_R == 8)
    dl_next_partials_r<CPL, 8>(F, p, x);
  else
    dl_next_partials_r<CPL, 16>(F, p, x);
}

// The previous step's token from its LM-head keys, when one is pending (F.fin_cand; one wave of
// the first layer's last extra block).
__device__ __forceinline__ void dl_finish_token(const dsh_split_t &F) {
  const int lane = threadIdx.x & 63;
  if (*F.fin_pending == 0) return;
  unsigned long long b = 0ull;
  for (int i = lane; i < F.fin_n; i += 64) b = dsh_umax64(b, F.fin_cand[i]);
  b = dsh_wave_max_u64(b);
  if (lane == 0) {
    F.fin_tokens[*F.fin_step - 1] = dsh_key_index(b);
    *F.fin_pending = 0;
  }
}

// Extra block p's share (after clearing its share of the region to clear).
template <int CPL>
__device__ __forceinline__ void dl_prefetch(const dsh_split_t &F, int p, float *x_out, float *zero_p, int zero_n) {
  const int t = threadIdx.x;
  for (int i = blockIdx.x * 512 + t; i < zero_n; i += gridDim.x * 512) zero_p[i] = 0.0f;
  if (F.nx_partials) dl_next_partials<CPL>(F, p);
  if (F.fin_cand && p == DL_PF - 1 && t < 64) dl_finish_token(F);
  const int ns = F.pf_gu ? F.pf_SI / DL_UB : 0;
  unsigned acc = 0;
  for (int sl = p; sl < ns; sl += DL_PF) {
    u32x4 v[DL_PFV(CPL)];
    dl_pf_load<CPL>(F, sl, v);
    acc ^= dl_pf_fold<CPL>(v);
  }
  if (acc == 0x9E3779B9u && F.pf_SI < 0) x_out[0] = 0.0f;
}

// Part j of the verification: rows RP j .. RP j + RP - 1 (RP = H / DL_NPART) of all experts, from
// the transposed router (lane = expert, a row's 64 scores are contiguous). Wave w: segment w, rows
// RP j + SR w .. + SR - 1 (SR = RP / 8). Pass 1 adds each expert's products p_k = fl(x_k w_k) sequentially in f32
// (t_i) with Σ|t_i| (its own rounding); per expert, the segment offsets O (the f64 prefix of the
// segment sums, kept in f32) and the part's sum S_j (f64); pass 2 adds |O + t_i| over the part's
// rows. Published per expert: S_j, U_j = Σ|O + t| (1 + 2^-12) + u SR Σ|O| (1 + 2^-16) (the offsets'
// rounding to f32), A_j = Σ_segments Σ|t_i|. The verdict bounds Σ_k |P_k| by Σ_j (RP |B_j| + U_j)
// (B_j: the f64 sum of the parts before j, whose own error is far below the terms).
template <int CPL, int NREP>
__device__ __forceinline__ void dl_verify_part(const dsh_layer_t &L, const float *x, int *A, int j,
                                               dl_smem<CPL> &S) {
  constexpr int H = 256 * CPL, RP = H / DL_NPART, SR = RP / 8;
  static_assert(DL_NPART % 8 == 0 && DL_NPART <= 32 && RP % 8 == 0, "parts");
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, E = L.E, e = min(lane, E - 1);
  const int r0 = RP * j + SR * wave;
  float wv[SR];
#pragma unroll
  for (int i = 0; i < SR; i++) wv[i] = L.router_f32_t[(size_t)(r0 + i) * E + e];
  f32x4 xr[NREP];  // every thread loads (a clamped piece: no branch around the loads)
  const int xp = min(t, RP / 4 - 1);
#pragma unroll
  for (int c = 0; c < NREP; c++) xr[c] = ((const f32x4 *)(x + (size_t)c * H + RP * j))[xp];
  asm volatile("" ::: "memory");
  if (t < RP / 4) {  // the part's input: the copies summed in copy order, as the routed blocks do
    f32x4 xs = xr[0];
#pragma unroll
    for (int c = 1; c < NREP; c++) xs += xr[c];
    *(f32x4 *)(S.s_x + 4 * t) = xs;
  }
  __syncthreads();  // s_x: this part's RP values
  float tt = 0.0f, la = 0.0f;
#pragma unroll
  for (int i = 0; i < SR; i++) {
    tt = __fadd_rn(tt, __fmul_rn(S.s_x[SR * wave + i], wv[i]));
    la += fabsf(tt);
  }
  S.s_vS[wave][lane] = tt;
  S.s_vA[wave][lane] = la;
  __syncthreads();
  double off = 0.0, tot = 0.0;
  float eA = 0.0f;
#pragma unroll
  for (int w = 0; w < 8; w++) {  // every wave forms the same sums in the same order
    const double g = (double)S.s_vS[w][lane];
    if (w < wave) off += g;
    tot += g;
    eA += S.s_vA[w][lane];
  }
  const float O = (float)off;  // this segment's offset
  float U = 0.0f;
  tt = 0.0f;
#pragma unroll
  for (int i = 0; i < SR; i++) {
    tt = __fadd_rn(tt, __fmul_rn(S.s_x[SR * wave + i], wv[i]));
    U += fabsf(O + tt);
  }
  __syncthreads();  // every wave has read s_vS, s_vA
  S.s_vS[wave][lane] = fabsf(O);
  S.s_vA[wave][lane] = U;
  __syncthreads();
  if (wave == 0 && lane < E) {
    float Ut = 0.0f, Oabs = 0.0f;
#pragma unroll
    for (int w = 0; w < 8; w++) {
      Ut += S.s_vA[w][lane];
      Oabs += S.s_vS[w][lane];
    }
    const float Uj = Ut * (1.0f + 0x1p-12f) + DSH_U * (float)SR * Oabs * (1.0f + 0x1p-16f);
    int *P = A + DL_VP + 256 * j;
    __hip_atomic_store((unsigned long long *)P + lane, (unsigned long long)__double_as_longlong(tot),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(P + 128 + lane, __float_as_int(Uj), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(P + 192 + lane, __float_as_int(eA), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// The routed blocks' selection from the accumulated scores, restated by lane = expert of one wave
// with the same loads, sums and rounds (so the same experts and weights bit for bit): idx/w of rank
// lane < K, idx -1 for an empty slot (fewer than K scores above -1e30). dl_spec_load issues the loads (partial rows v + 4 j, lane's column), dl_spec_finish
// adds them in the routed blocks' order and selects.
template <int RB>
__device__ __forceinline__ void dl_spec_load(const float *partials, int np, float (&pv)[4][RB]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int v = 0; v < 4; v++)
#pragma unroll
    for (int j = 0; j < RB; j++) pv[v][j] = partials[(size_t)min(v + 4 * j, np - 1) * 64 + lane];
}

template <int RB>
__device__ __forceinline__ void dl_spec_finish(int E, int K, int np, const float (&pv)[4][RB], float (*s_red)[64],
                                               int &idx, float &w) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int v = 0; v < 4; v++) {
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < RB; j++)
      if (v + 4 * j < np) acc += pv[v][j];
    s_red[v][lane] = lane < E ? acc : 0.0f;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  route_state st;
  route_init(E, K, DSH_ROUTE_CFG, s_red, st);
  route_rounds(st, 0, st.ns);
  route_finish(DSH_ROUTE_CFG, st, idx, w);
  if (lane >= st.ns) idx = -1;  // an empty slot (the routed blocks use expert 0 with weight 0 there)
}

// The parts' sums, gathered by the whole block of the last part to finish (wave w: parts PW w ..
// PW w + PW - 1, PW = DL_NPART / 8; lane = expert), into S.s_vG (group sums G_w = Σ S_j, f64 in part order) and S.s_vT
// ([0] Σ (RP |B_j| + U_j), [1] Σ A_j, [2] Σ |S_j|, f64, over the group's parts). The prefix B_j is
// the group's own prefix on top of the sum of the groups before: an f64 regrouping of the same
// terms whose rounding is far below the margins of the bound (dl_verdict_select).
template <int CPL>
__device__ __forceinline__ void dl_verdict_gather(const dsh_layer_t &L, const int *A, dl_smem<CPL> &S) {
  constexpr int H = 256 * CPL, RP = H / DL_NPART;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const bool valid = lane < L.E;
  constexpr int PW = DL_NPART / 8;
  double Sj[PW];
  float Uj[PW], Aj[PW];
#pragma unroll
  for (int i = 0; i < PW; i++) {
    Sj[i] = 0.0;
    Uj[i] = Aj[i] = 0.0f;
  }
  if (valid) {
#pragma unroll
    for (int i = 0; i < PW; i++) {
      const int *P = A + DL_VP + 256 * (PW * wave + i);
      Sj[i] = __longlong_as_double((long long)__hip_atomic_load((const unsigned long long *)P + lane,
                                                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
      Uj[i] = __int_as_float(__hip_atomic_load(P + 128 + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
      Aj[i] = __int_as_float(__hip_atomic_load(P + 192 + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    }
  }
  double b[PW], g = 0.0;
#pragma unroll
  for (int i = 0; i < PW; i++) {
    b[i] = g;
    g += Sj[i];
  }
  S.s_vG[wave][lane] = g;
  __syncthreads();
  double B = 0.0;
#pragma unroll
  for (int w = 0; w < 8; w++)
    if (w < wave) B += S.s_vG[w][lane];
  double T = 0.0, ea = 0.0, sa = 0.0;
#pragma unroll
  for (int i = 0; i < PW; i++) {
    T += (double)RP * fabs(B + b[i]) + (double)Uj[i];
    ea += (double)Aj[i];
    sa += fabs(Sj[i]);
  }
  S.s_vT[0][wave][lane] = T;
  S.s_vT[1][wave][lane] = ea;
  S.s_vT[2][wave][lane] = sa;
  __syncthreads();
}

// The whole input into sx (LDS) by one wave: the copies summed in copy order, as the routed blocks
// do; visible to the wave when it returns.
template <int CPL, int NREP>
__device__ __forceinline__ void dl_input_wave(const float *x, float *sx) {
  constexpr int H = 256 * CPL, NP = 64 * CPL;
  for (int p = threadIdx.x & 63; p < NP; p += 64) {
    f32x4 xs = ((const f32x4 *)x)[p];
#pragma unroll
    for (int c = 1; c < NREP; c++) xs += ((const f32x4 *)(x + (size_t)c * H))[p];
    *(f32x4 *)(sx + 4 * p) = xs;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The centre and radius of expert lane's score (wave 0 of the last part to finish, after
// dl_verdict_gather): the radius
//   eps = (e_C + u (1 + 2^-10) (Σ_j (RP |B_j| + U_j) + H e_C)) (1 + 2^-16),
//   e_C = u (1 + 2^-10) Σ_j A_j + 2^-40 Σ_j |S_j|   (B_j = Σ_{j' < j} S_j'),
// rounded up to f32, around the centre C = Σ_j S_j rounded to f32, widened by that rounding: the
// reference's score lies in [c - epsr, c + epsr]. Lanes >= E: 0 and 0.
template <int CPL>
__device__ __forceinline__ void dl_verdict_bounds(const dsh_layer_t &L, const dl_smem<CPL> &S, float &c,
                                                  float &epsr) {
  constexpr int H = 256 * CPL;
  const int lane = threadIdx.x & 63;
  const bool valid = lane < L.E;
  double C = 0.0, Ut = 0.0, eA = 0.0, sa = 0.0;
#pragma unroll
  for (int w = 0; w < 8; w++) {
    C += S.s_vG[w][lane];
    Ut += S.s_vT[0][w][lane];
    eA += S.s_vT[1][w][lane];
    sa += S.s_vT[2][w][lane];
  }
  float eps = 0.0f;
  if (valid) {
    const double u = 0x1p-24;
    const double eC = u * (1.0 + 0x1p-10) * eA + 0x1p-40 * sa;
    const double e = (eC + u * (1.0 + 0x1p-10) * (Ut + (double)H * eC)) * (1.0 + 0x1p-16);
    eps = (float)e;
    if ((double)eps < e) eps = __uint_as_float(__float_as_uint(eps) + 1u);
  }
  c = valid ? (float)C : 0.0f;
  const double ed = (double)eps + fabs((double)c - C);
  epsr = (float)ed;
  if ((double)epsr < ed) epsr = __uint_as_float(__float_as_uint(epsr) + 1u);  // rounded up (>= 0)
  if (!valid) epsr = 0.0f;
}

// Whether the intervals certify the routed blocks' own selection (S.s_si, ranks 0 .. K-1) as it
// stands: its K experts distinct (no empty slot), their intervals strictly ordered in its rank order, the last one's
// above every other expert's interval and above -1e30. Then the reference's selection is that one,
// in that order (wave-uniform result). Interval ends rounded outward as in cert_check.
template <int CPL>
__device__ __forceinline__ bool dl_spec_certified(int E, int K, float c, float epsr, const dl_smem<CPL> &S) {
  const int lane = threadIdx.x & 63;
  const bool valid = lane < E;
  const bool finite = !valid || (__builtin_isfinite(c) && __builtin_isfinite(epsr) &&
                                 __builtin_isfinite(c - epsr) && __builtin_isfinite(c + epsr));
  if (__ballot(!finite) != 0ull) return false;
  bool in_s = false;
  for (int k = 0; k < K; k++) in_s |= S.s_si[k] == lane;
  if (__popcll(__ballot(valid && in_s)) != K) return false;  // K distinct experts (all < E)
  const float lo_me = valid ? cert_next_down(c - epsr) : 0.0f, hi_me = valid ? cert_next_up(c + epsr) : 0.0f;
  const int er = lane < K ? S.s_si[lane] : 0;
  const float lo = __shfl(lo_me, er), hi = __shfl(hi_me, er);
  const float hi_next = __shfl(hi, min(lane + 1, 63));
  const float hi_out = dsh_wave_max(valid && !in_s ? hi_me : -__builtin_huge_valf());
  const float lo_last = __shfl(lo, K - 1);
  const bool bad = (lane < K - 1 && !(lo > hi_next)) || (lane == 0 && !(lo_last > hi_out && lo_last > -1e30f));
  return __ballot(bad) == 0ull;
}

// The verdict, part 1, where dl_spec_certified does not hold (wave 0): the selection certified on
// the intervals (route_rounds on c, cert_check) or recomputed in ds_linear's order: rank lane's
// expert and weight (vi, vw; vi -1 for an empty slot); flags bit 0 when recomputed.
template <int CPL, int NREP>
__device__ __forceinline__ void dl_verdict_select(const dsh_layer_t &L, const float *x, bool need_x, float c,
                                                  float epsr, dl_smem<CPL> &S, int &vi, float &vw, int &flags) {
  constexpr int H = 256 * CPL;
  const int lane = threadIdx.x & 63, E = L.E, K = L.K;
  const bool valid = lane < E;
  S.s_vr[0][lane] = valid ? c : 0.0f;
  S.s_vr[1][lane] = 0.0f;
  S.s_vr[2][lane] = 0.0f;
  S.s_vr[3][lane] = 0.0f;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  route_state st;
  route_init(E, K, DSH_ROUTE_CFG, S.s_vr, st);
  route_rounds(st, 0, st.ns);
  unsigned long long cand;
  flags = 0;
  const bool certain = cert_check(st, valid ? c : 0.0f, valid ? epsr : 0.0f, E, K, cand);
  if (!certain || need_x) dl_input_wave<CPL, NREP>(x, S.s_x);
  if (!certain) {
    const float ex = cert_exact_chain(L.router_f32, S.s_x, H, cand);
    S.s_vr[0][lane] = ((cand >> lane) & 1ull) ? ex : -__builtin_huge_valf();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    route_init(E, K, DSH_ROUTE_CFG, S.s_vr, st);
    route_rounds(st, 0, st.ns);
    flags = 1;
  }
  route_finish(DSH_ROUTE_CFG, st, vi, vw);
  if (lane >= st.ns) vi = -1;  // an empty slot: no expert (weight 0)
}

// The verdict, part 2 (wave 0; the routed blocks' own selection, restated by wave 1, in S.s_si /
// S.s_sw): compared with the certified one, empty slots (-1) in neither set. Returns the state word (1: it stands, 2: the experts in
// A[16..] need their Δw added; flags bit 1 then) and leaves the record in S.s_vi / S.s_vw: the
// certified experts in rank order with the weights the layer's output carries.
template <int CPL>
__device__ __forceinline__ int dl_verdict_compare(const dsh_layer_t &L, int *A, int vi, float vw, int &flags,
                                                  dl_smem<CPL> &S) {
  const int lane = threadIdx.x & 63, E = L.E, K = L.K;
  const bool valid = lane < E;
  // the weight of each expert in either selection (lane = expert), from the ranks in LDS
  if (lane < 8) {
    S.s_vi[lane] = lane < K ? vi : -1;
    S.s_vw[lane] = lane < K ? vw : 0.0f;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float wv = 0.0f, ws = 0.0f;
  bool in_v = false, in_s = false;
  for (int k = 0; k < K; k++) {
    const int a = S.s_vi[k], b = S.s_si[k];
    if (a == lane) {
      in_v = true;
      wv = S.s_vw[k];
    }
    if (b == lane) {
      in_s = true;
      ws = S.s_sw[k];
    }
  }
  const bool differ = __ballot(valid && in_v != in_s) != 0ull;
  int state = 1;
  if (differ) {  // every expert in either set gets Δw = w_certified - w_used
    const unsigned long long m = __ballot(valid && (in_v || in_s));
    const int pos = __popcll(m & ((1ull << lane) - 1ull));
    if ((m >> lane) & 1ull) {
      __hip_atomic_store(A + 16 + pos, lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(A + 32 + pos, __float_as_int(wv - ws), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (lane == 0) __hip_atomic_store(A + 3, __popcll(m), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    state = 2;
    flags |= 2;
  }
  // the record: the routed blocks' weights for the same experts when the set stands; an empty slot
  // as ds_moe_top_k fills it (expert 0, weight 0)
  if (lane < K) {
    const int a = S.s_vi[lane];
    if (!differ) {
      float w_used = 0.0f;
      for (int k = 0; k < K; k++)
        if (a >= 0 && S.s_si[k] == a) w_used = S.s_sw[k];
      S.s_vw[lane] = w_used;
    }
    S.s_vi[lane] = max(a, 0);
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  return state;
}

// One correction job: Δw (h → down) of expert e's units 32 sl .. 32 sl + 31 added to this XCD's
// output copy (and to the next layer's score copy through M, z), h from f32 dot products of the
// codes with x (s_x, xsum): y = scale Σ u x + offset Σ x, then the reference's SwiGLU.
template <int CPL>
__device__ __forceinline__ void dl_correct_job(const dsh_layer_t &L, const dsh_split_t &F, int e, int sl, float dw,
                                               float xsum, float *x_out, float *lg_out, int cp, dl_smem<CPL> &S) {
  constexpr int H = 256 * CPL, PL = H / 8 / 16;  // 16-byte pieces per lane (8 lanes per row)
  const int t = threadIdx.x, I = L.I, NSL = I / DL_UB;
  {  // 64 rows (32 gate, 32 up), 8 lanes each
    const int r = t >> 3, q = t & 7, i = DL_UB * sl + (r & 31);
    const size_t grow = (size_t)e * 2 * I + (size_t)(r < 32 ? 0 : I) + i;
    const u32x4 *src = (const u32x4 *)(L.gu_q + grow * H);
    float acc = 0.0f;
#pragma unroll
    for (int m = 0; m < PL; m++) {
      const int pc = q + 8 * m;
      const u32x4 wq = src[pc];
      acc = dsh_dot16_u8(wq, S.s_x + 16 * pc, acc);
    }
    acc += __shfl_xor(acc, 1);
    acc += __shfl_xor(acc, 2);
    acc += __shfl_xor(acc, 4);
    if (q == 0) {
      const float2 so = ((const float2 *)L.gu_so)[grow];
      S.s_dn[r] = __builtin_fmaf(so.x, acc, so.y * xsum);
    }
  }
  __syncthreads();
  if (t < DL_UB) S.s_h[t] = dsh_swiglu(S.s_dn[t], S.s_dn[DL_UB + t]);
  __syncthreads();
  float hs = 0.0f;
  for (int j = 0; j < DL_UB; j++) hs += S.s_h[j];
  for (int r = t; r < H; r += 512) {  // down rows: 32 codes of this unit block
    const u32x4 *d = (const u32x4 *)(L.dn_q + ((size_t)e * H + r) * I + DL_UB * sl);
    float a = dsh_dot16_u8(d[0], S.s_h, 0.0f);
    a = dsh_dot16_u8(d[1], S.s_h + 16, a);
    const float2 so = ((const float2 *)L.dn_so)[(size_t)e * H + r];
    __hip_atomic_fetch_add(x_out + (size_t)cp * H + r, dw * __builtin_fmaf(so.x, a, so.y * hs), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
  }
  if (F.M && t < 64 && t < F.E_next) {  // m[w][jj/4][a][jj%4] for unit 8w + jj
    const float *m = F.M + ((size_t)e * NSL + sl) * 2048;
    float v = 0.0f;
    for (int j = 0; j < DL_UB; j++) v = __builtin_fmaf(m[(j >> 3) * 512 + ((j & 7) >> 2) * 256 + t * 4 + (j & 3)], S.s_h[j], v);
    v = __builtin_fmaf(F.z[(size_t)e * 64 + t], hs, v);
    __hip_atomic_fetch_add(lg_out + (size_t)cp * 64 + t, dw * v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();  // s_dn, s_h reused by the next job
}


// An extra block of a certified CFG layer (b < DL_NPART): part b of the verification; then wave 1
// restates the routed blocks' selection while wave 0 counts the part done. The last part to finish
// forms the verdict (the block gathers the parts; wave 0 certifies the routed blocks' selection as
// it stands, or selects and compares) and publishes it; the other parts wait for it (a bounded
// wait: on expiry the device error word is set). Rarely, all add their share of the correction
// (jobs j with j % DL_NPART == the block's arrival rank).
template <int CPL, int NREP, int RB>
__device__ __forceinline__ void dl_verify(const dsh_layer_t &L, const dsh_split_t &F, const float *x_in,
                                          const int *__restrict__ step, int stride, const float *partials, int np,
                                          float *x_out, float *lg_out, dl_smem<CPL> &S) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  int *A = (int *)F.vd;
  const float *x = step ? x_in + (size_t)(*step) * stride : x_in;
  constexpr bool pre = RB <= 2;  // the restatement's loads go out with the part's (few partial rows)
  float pv[4][RB];
  if (pre && wave == 1) dl_spec_load<RB>(partials, np, pv);
  dl_verify_part<CPL, NREP>(L, x, A, blockIdx.x, S);
  if (t == 0) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this part's sums are out
    S.s_claim = __hip_atomic_fetch_add(A, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else if (wave == 1) {  // meanwhile (every part: which one finishes last is not known yet)
    if (!pre) dl_spec_load<RB>(partials, np, pv);
    int si;
    float sw;
    dl_spec_finish<RB>(L.E, L.K, np, pv, S.s_red, si, sw);
    if (lane < 8) {
      S.s_si[lane] = si;
      S.s_sw[lane] = sw;
    }
  }
  __syncthreads();  // s_claim, s_si, s_sw
  const int rank = S.s_claim;
  if (rank == DL_NPART - 1) {  // every part is out: the verdict
    dl_verdict_gather<CPL>(L, A, S);
    if (wave == 0) {
      constexpr int H = 256 * CPL;
      const bool log = F.rc.log != nullptr;
      float c, epsr;
      dl_verdict_bounds<CPL>(L, S, c, epsr);
      int state = 1, flags = 0;
      if (dl_spec_certified<CPL>(L.E, L.K, c, epsr, S)) {  // the usual case: it stands as used
        if (lane < 8) {
          S.s_vi[lane] = lane < L.K ? S.s_si[lane] : -1;
          S.s_vw[lane] = lane < L.K ? S.s_sw[lane] : 0.0f;
        }
        if (log) dl_input_wave<CPL, NREP>(x, S.s_x);  // the record's input
      } else {
        int vi = 0;
        float vw = 0.0f;
        dl_verdict_select<CPL, NREP>(L, x, log, c, epsr, S, vi, vw, flags);
        state = dl_verdict_compare<CPL>(L, A, vi, vw, flags, S);
      }
      if (lane == 0) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the correction list is out
        __hip_atomic_store(A + 2, state, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        S.s_ev = state;
        cert_record(F.rc, S.s_vi, S.s_vw, L.K, flags, S.s_x, H);
        if ((flags & 2) && F.rc.stats)
          __hip_atomic_fetch_add(F.rc.stats + 2, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  } else {  // the verdict: a bounded wait
    if (t == 0) {
      int v = 0;
      for (int n = 0; n < DL_VD_SPIN; n++) {
        v = __hip_atomic_load(A + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (v != 0) break;
        __builtin_amdgcn_s_sleep(2);
      }
      if (v == 0 && F.derr) __hip_atomic_store(F.derr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      S.s_ev = v;
    }
  }
  __syncthreads();
  if (S.s_ev == 2) {  // rare: add Δw of every expert in either selection
    constexpr int H = 256 * CPL, NP = 64 * CPL;
    float sx = 0.0f;
    for (int p = t; p < NP; p += 512) {  // the whole input in s_x (the copies summed in copy order)
      f32x4 xs = ((const f32x4 *)x)[p];
#pragma unroll
      for (int c = 1; c < NREP; c++) xs += ((const f32x4 *)(x + (size_t)c * H))[p];
      *(f32x4 *)(S.s_x + 4 * p) = xs;
      sx += (xs[0] + xs[1]) + (xs[2] + xs[3]);
    }
    sx = dsh_wave_sum(sx);
    if (lane == 0) S.s_stat[wave] = sx;
    __syncthreads();
    float xsum = 0.0f;
#pragma unroll
    for (int w = 0; w < 8; w++) xsum += S.s_stat[w];
    const int n = __hip_atomic_load(A + 3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int NSL = L.I / DL_UB, njob = min(n, 16) * NSL, cp = dl_copy();
    for (int j = rank; j < njob; j += DL_NPART) {
      const int k = j / NSL, sl = j - k * NSL;
      const int e = min(max(__hip_atomic_load(A + 16 + k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT), 0), L.E - 1);
      const float dw = __int_as_float(__hip_atomic_load(A + 32 + k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
      dl_correct_job<CPL>(L, F, e, sl, dw, xsum, x_out, lg_out, cp, S);
    }
  }
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
  const int nwork = (L.SI + L.K * L.I) / DL_UB, b = blockIdx.x;
  if (F.vd) {  // certified CFG routing: the extra blocks that verify come first (their loads go out first)
    if (b < DL_NPART) {
      for (int i = b * 512 + threadIdx.x; i < zero_n; i += gridDim.x * 512) zero_p[i] = 0.0f;
      dl_verify<CPL, NREP, RB>(L, F, x_in, step, stride, partials, np, x_out, lg_out, S);
      return;
    }
    const int w = b - DL_NPART;
    if (w >= nwork) {  // after the routed blocks: the next layer's shared-expert data read ahead
      dl_prefetch<CPL>(F, w - nwork, x_out, zero_p, zero_n);
      return;
    }
    if (w < L.SI / DL_UB)
      dl_body<CPL, NREP, RB, true, false>(L, F, x_in, step, stride, partials, np, mode, resid, x_out, lg_out, zero_p,
                                          zero_n, w, S);
    else
      dl_body<CPL, NREP, RB, false, false>(L, F, x_in, step, stride, partials, np, mode, resid, x_out, lg_out,
                                           zero_p, zero_n, w, S);
    return;
  }
  if (b >= nwork) {
    dl_prefetch<CPL>(F, b - nwork, x_out, zero_p, zero_n);
    return;
  }
  if (b < L.SI / DL_UB)
    dl_body<CPL, NREP, RB, true, false>(L, F, x_in, step, stride, partials, np, mode, resid, x_out, lg_out, zero_p,
                                        zero_n, b, S);
  else
    dl_body<CPL, NREP, RB, false, false>(L, F, x_in, step, stride, partials, np, mode, resid, x_out, lg_out, zero_p,
                                         zero_n, b, S);
}

// DECODE routing with the scores computed in the routed blocks (F.Wr_dec; CPL <= 5, so a lane's
// router pieces fit in registers next to the input copies).
template <int CPL, int NREP>
__global__ void __launch_bounds__(512) k_dec_layer_ds(dsh_layer_t L, dsh_split_t F, const float *x_in,
                                                      const int *__restrict__ step, int stride,
                                                      const float *__restrict__ resid, float *x_out, float *lg_out,
                                                      float *zero_p, int zero_n) {
  __shared__ dl_smem<CPL> S;
  const int nwork = (L.SI + L.K * L.I) / DL_UB, b = blockIdx.x;
  if (b >= nwork) {
    dl_prefetch<CPL>(F, b - nwork, x_out, zero_p, zero_n);
    return;
  }
  if (b < L.SI / DL_UB)
    dl_body<CPL, NREP, 1, true, true>(L, F, x_in, step, stride, nullptr, 1, DSH_ROUTE_DECODE, resid, x_out, lg_out,
                                      zero_p, zero_n, b, S);
  else
    dl_body<CPL, NREP, 1, false, true>(L, F, x_in, step, stride, nullptr, 1, DSH_ROUTE_DECODE, resid, x_out, lg_out,
                                       zero_p, zero_n, b, S);
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

int dsh_layer_cert_supported(const dsh_layer_t *L) {
  return dsh_layer_split_supported(L) && L->E % 4 == 0 && L->K <= 8 && L->router_f32 && L->router_f32_t &&
         L->router_norm;
}

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
  static_assert(DL_VX <= DSH_SPLIT_VD_INTS, "verdict area");
  const int extra = F->pf_gu || F->nx_partials || F->fin_cand;
  const int nb = dsh_layer_split_blocks(L) + (F->vd ? DL_NPART : 0) + (extra ? DL_PF : 0);
  if (ncopies != 1 && ncopies != DL_REP) return hipErrorInvalidValue;
  if (F->nx_partials && (!F->nx_in || !F->nx_WrT || !F->nx_step || !F->nx_pending || F->nx_stride < 0 ||
                         (F->nx_R != 8 && F->nx_R != 16) || L->H % F->nx_R || L->H / F->nx_R > 8 * DL_PF ||
                         F->nx_E <= 0 || F->nx_E > 64))
    return hipErrorInvalidValue;
  if (F->fin_cand && (!F->fin_tokens || !F->fin_step || !F->fin_pending || F->fin_n <= 0)) return hipErrorInvalidValue;
  if (F->vd && (route_mode != DSH_ROUTE_CFG || F->Wr_dec || !dsh_layer_cert_supported(L) ||
                ((uintptr_t)F->vd & 127)))
    return hipErrorInvalidValue;
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
