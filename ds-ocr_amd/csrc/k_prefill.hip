// k_prefill.hip — prefill MoE block (T tokens) for the device-resident layer: routing, an
// expert-sorted grouped GEMM on bf16 MFMA with INT8 weights dequantized in registers, SwiGLU, the
// down projection and a deterministic combine (ds_moe_decoder.c:629-809 is the reference block; it
// runs sgemm on bf16 weights, this build runs the same layer's INT8 blocks).
//
// Numerics. The stored codes q = u - 128 (-128..127) are exact in bf16. Each f32 activation a is
// split into hi = bf16(a) and lo = bf16(a - hi), so a = hi + lo to about 2^-17 relative, and
// Σ q·a = Σ q·hi + Σ q·lo is accumulated by the MFMA in f32 (products exact). The epilogue folds the
// row's scale and offset: y = scale·Σu·a + offset·Σa = scale·Σq·a + (offset + 128·scale)·Σa.
//
// Kernels (one launch each, all sizes fixed by T, so a graph can hold them):
//   k_pf_scores  router scores in the decode path's order, as four partial sums per token
//   k_pf_select  per token: X → Xhi, Xlo (bf16), Σx; expert selection → idx, w
//   k_pf_plan    expert-sorted (token, slot) pairs (stable: tokens in increasing order per expert),
//                per-expert offsets and the GEMM work items (expert, up-to-PF_MT-row chunk)
//   k_pf_gate_up grouped GEMM + SwiGLU → H (bf16 hi/lo) for routed pairs and for the shared expert
//   k_pf_down    grouped GEMM → Y (f32) per routed pair and per token for the shared expert
//   k_pf_combine out[t] = (residual ? x : 0) + (Σ_k w_k·Y_k in ascending expert order + Y_shared)
#include "dsh_avx.h"
#include "dsh_route.h"
#include "k_core.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

#define PF_MT 64    // rows of A per work item: one or two MFMA sub-tiles of 32 rows
#define PF_GU_N 128 // gate_up: intermediate units per block (128 gate + 128 up weight rows)
#define PF_DN_N 256 // down: output rows per block
#define PF_TB 8     // tokens per DECODE-mode scores block
#define PF_PLAN_LDS 8192  // (token, slot) entries the plan kernel caches in LDS
#define PF_NQ 8           // work queues of the fused GEMM kernel: one per XCD
#define PF_DN_TILE 0x80000000u  // tile word: down tile flag | item << 8 | n-tile

// Work queues of the fused GEMM kernel (k_pf_moe), built by the plan kernel.
struct pf_queues {
  int *tiles;    // [PF_NQ][cap] tile words in claim order
  int *count;    // [PF_NQ] tiles per queue
  int *next;     // [PF_NQ] claim counters (zeroed by the plan)
  int *gu_done;  // [items] finished gate_up tiles per item (zeroed by the plan)
  int *err;      // set when a bounded wait expires (zeroed by the plan)
  int cap;
  int ngu_r, ngu_s, ndn;      // n-tiles: gate_up routed / shared, down
  int nk_gu, nk_dr, nk_ds;    // 128-column stages: gate_up, routed down, shared down
  int enable;
};

struct pf_item {
  int seg;   // expert 0..E-1, or E for the shared expert
  int m0;    // first row of the chunk within the segment
  int mcnt;  // rows in the chunk (1..PF_MT)
  int pos0;  // first routed pair position of the segment (routed only)
};

// ---------------------------------------------------------------------------------- helpers
__device__ __forceinline__ unsigned pk_bf16(float x, float y) {
  return __builtin_bit_cast(unsigned, __builtin_convertvector(f32x2{x, y}, bf16x2));
}

// 8 stored codes q (signed bytes, q = u - 128) → 8 exact bf16 values (one sign-extending byte
// conversion per code and one pack per pair)
__device__ __forceinline__ bf16x8 codes_to_bf16(u32x2 v) {
  const int a = (int)v[0], b = (int)v[1];
  u32x4 r;
  r[0] = pk_bf16((float)((a << 24) >> 24), (float)((a << 16) >> 24));
  r[1] = pk_bf16((float)((a << 8) >> 24), (float)(a >> 24));
  r[2] = pk_bf16((float)((b << 24) >> 24), (float)((b << 16) >> 24));
  r[3] = pk_bf16((float)((b << 8) >> 24), (float)(b >> 24));
  return __builtin_bit_cast(bf16x8, r);
}

__device__ __forceinline__ bf16x8 ld_bf16x8(const __bf16 *p) { return *(const bf16x8 *)p; }

// D[m][n] of a 32x32 MFMA tile held by lane l, register j: n = l % 32, m = 8*(j/4) + 4*(l/32) + j%4
__device__ __forceinline__ int mfma_row(int lane, int j) { return 8 * (j >> 2) + 4 * (lane >> 5) + (j & 3); }

// ---------------------------------------------------------------------------------- routing
// Router scores in the decode path's order, kept as four partial sums per token and expert:
// ps[t][v][e] = Σ_jb p[v + 4·jb] added sequentially from 0, where p[b] = Σ_j WrT[R·b+j][e]·x[R·b+j]
// is a chain of fused multiply-adds over j (the decode path's partials and per-wave sums, wave v
// taking partials v, v+4, ...); k_pf_select adds them as ((ps0 + ps1) + ps2) + ps3 (route_select).
// CFG (f32 router): block = (PF_SC_TOK tokens, residue v); the residue's router rows and the tokens'
// matching x values are staged in LDS PF_SC_JB partials at a time; wave w runs tokens 4w..4w+3,
// lane = expert.
#define PF_SC_TOK 16
#define PF_SC_JB 20
template <int R>
__global__ void __launch_bounds__(256) k_pf_scores_cfg(const float *__restrict__ WrT, const float *__restrict__ X,
                                                       int T, int H, int E, float *__restrict__ ps) {
  __shared__ __attribute__((aligned(16))) float wv[PF_SC_JB][R][64];
  __shared__ __attribute__((aligned(16))) float xv[PF_SC_TOK][PF_SC_JB][R];
  constexpr int NW = PF_SC_JB * R * 64 / 256;            // router values per thread per pass
  constexpr int NX = PF_SC_TOK * PF_SC_JB * (R / 4);      // x float4s per pass
  constexpr int NXT = (NX + 255) / 256;
  const int v = blockIdx.y, t0 = blockIdx.x * PF_SC_TOK;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nbv = (H / R - v + 3) / 4;
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int jb0 = 0; jb0 < nbv; jb0 += PF_SC_JB) {
    const int nj = min(PF_SC_JB, nbv - jb0);
    // every load of the pass in flight at once (partials past the last repeat it, unused)
    float wr_[NW];
    f32x4 xr_[NXT];
#pragma unroll
    for (int k = 0; k < NW; k++) {
      const int i = threadIdx.x + 256 * k;
      const int row = i >> 6, e = i & 63;
      const int jj = row / R, j = row - jj * R;
      const int b = v + 4 * min(jb0 + jj, nbv - 1);
      const float val = WrT[(size_t)(R * b + j) * E + min(e, E - 1)];  // branch-free load
      wr_[k] = e < E ? val : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < NXT; k++) {
      const int i = min((int)threadIdx.x + 256 * k, NX - 1);
      const int tb = i / (PF_SC_JB * (R / 4)), rem = i - tb * (PF_SC_JB * (R / 4));
      const int jj = rem / (R / 4), q = rem - jj * (R / 4);
      const int t = min(t0 + tb, T - 1);
      const int b = v + 4 * min(jb0 + jj, nbv - 1);
      xr_[k] = *(const f32x4 *)(X + (size_t)t * H + R * b + 4 * q);
    }
    __syncthreads();  // the previous pass's reads are done
#pragma unroll
    for (int k = 0; k < NW; k++) {
      const int i = threadIdx.x + 256 * k;
      (&wv[0][0][0])[i] = wr_[k];
    }
#pragma unroll
    for (int k = 0; k < NXT; k++) {
      const int i = threadIdx.x + 256 * k;
      if (i < NX) ((f32x4 *)&xv[0][0][0])[i] = xr_[k];
    }
    __syncthreads();
    for (int jj = 0; jj < nj; jj++) {
      float wr[R];
#pragma unroll
      for (int j = 0; j < R; j++) wr[j] = wv[jj][j][lane];
#pragma unroll
      for (int tk = 0; tk < 4; tk++) {
        const f32x4 *x4 = (const f32x4 *)xv[4 * wave + tk][jj];
        float p = 0.0f;
#pragma unroll
        for (int q = 0; q < R / 4; q++) {
          const f32x4 xq = x4[q];
#pragma unroll
          for (int i = 0; i < 4; i++) p = __builtin_fmaf(wr[4 * q + i], xq[i], p);
        }
        acc[tk] += p;
      }
    }
  }
#pragma unroll
  for (int tk = 0; tk < 4; tk++) {
    const int t = t0 + 4 * wave + tk;
    if (t < T) ps[((size_t)t * 4 + v) * 64 + lane] = lane < E ? acc[tk] : 0.0f;
  }
}

// DECODE (bf16 router in the reference's AVX-512 order, as k_dec_scores_bf16): one block per PF_TB
// tokens, 64 groups of 4 lanes, group g computes expert g's score; the full score is partial 0, the
// other three are zero (0 + ... keeps it).
__global__ void __launch_bounds__(256) k_pf_scores_bf16(const uint16_t *__restrict__ Wr, const float *__restrict__ X,
                                                        int T, int H, int E, int nthreads, float *__restrict__ ps) {
  extern __shared__ __attribute__((aligned(16))) float xs[];  // [PF_TB][H]
  const int t0 = blockIdx.x * PF_TB, nt = min(PF_TB, T - t0);
  for (int i = threadIdx.x; i < nt * H; i += 256) xs[i] = X[(size_t)t0 * H + i];
  __syncthreads();
  const int Lq = threadIdx.x & 3, g = threadIdx.x >> 2;
  const int chunk = dsh_chunk_len(E, nthreads);
  const int path = g < E ? row_path(g, E, chunk, false) : DSH_ROW_SINGLE;
  for (int tb = 0; tb < nt; tb++) {
    float v = 0.0f;
    if (g < E)
      v = avx_row<true>(Wr + (size_t)g * H, xs + (size_t)tb * H, H, Lq, path == DSH_ROW_SINGLE, true, 0.0f,
                        path != DSH_ROW_GROUP4);
    if (Lq == 0) {
      float *o = ps + (size_t)(t0 + tb) * 4 * 64;
      o[g] = g < E ? v : 0.0f;
      o[64 + g] = 0.0f;
      o[128 + g] = 0.0f;
      o[192 + g] = 0.0f;
    }
  }
}

// One wave per token: the bf16 hi/lo split of x and Σx, then the expert selection from the four
// partial score rows (route_select: CFG top-k on raw scores + softmax over the k; DECODE fast-exp
// softmax over all experts + top-k).
#define PF_SEL_U 8  // x float4 loads per lane in flight
template <int MODE>
__global__ void __launch_bounds__(256) k_pf_select(const float *__restrict__ X, int T, int H, int E, int K,
                                                   const float *__restrict__ ps, __bf16 *__restrict__ Xhi,
                                                   __bf16 *__restrict__ Xlo, float *__restrict__ xsum,
                                                   int *__restrict__ idx, float *__restrict__ w) {
  __shared__ float s_red[4][4][64];
  __shared__ int s_idx[4][64];
  __shared__ float s_w[4][64];
  __shared__ route_scratch s_scr[4];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + wave;
  if (t >= T) return;  // no block-wide barriers below
#pragma unroll
  for (int r = 0; r < 4; r++) s_red[wave][r][lane] = ps[((size_t)t * 4 + r) * 64 + lane];
  const f32x4 *src = (const f32x4 *)(X + (size_t)t * H);
  float s = 0.0f;
  for (int c0 = 0; c0 < H / 4; c0 += 64 * PF_SEL_U) {
    f32x4 xv[PF_SEL_U];
#pragma unroll
    for (int u = 0; u < PF_SEL_U; u++) xv[u] = src[min(c0 + 64 * u + lane, H / 4 - 1)];
#pragma unroll
    for (int u = 0; u < PF_SEL_U; u++) {
      const int c = c0 + 64 * u + lane;
      if (c >= H / 4) continue;
      const f32x4 v = xv[u];
      bf16x4 hi, lo;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        hi[i] = (__bf16)v[i];
        lo[i] = (__bf16)(v[i] - (float)hi[i]);
      }
      *(bf16x4 *)(Xhi + (size_t)t * H + 4 * c) = hi;
      *(bf16x4 *)(Xlo + (size_t)t * H + 4 * c) = lo;
      s += (v[0] + v[1]) + (v[2] + v[3]);
    }
  }
  s = dsh_wave_sum(s);
  if (lane == 0) xsum[t] = s;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  route_select(E, K, MODE, s_idx[wave], s_w[wave], s_red[wave], s_scr + wave);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (lane < K) {
    idx[(size_t)t * K + lane] = s_idx[wave][lane];
    w[(size_t)t * K + lane] = s_w[wave][lane];
  }
}

// ---------------------------------------------------------------------------------- plan
// One 1024-thread block. Wave v owns a contiguous range of the T·K (token, slot) entries. Per-wave
// expert counts give each expert's segment offset and each wave's start inside it, so a pair's
// position is (segment offset) + (pairs of the expert in earlier waves) + (earlier pairs of the
// expert in this wave): expert segments hold their tokens in increasing order. Within a wave, 64
// entries at a time, the entries routed to the same expert are found with 7 ballots over the
// expert's bits. Entries with no expert (idx < 0 or >= E) get pos_of = -1.
// Work items: each expert's pairs in chunks of PF_MT (items 0 .. n_routed-1), then the shared
// expert's T tokens in chunks of PF_MT; counts = {n_routed, n_shared}; and the routed GEMM tile
// lists of both projections.
__global__ void __launch_bounds__(1024) k_pf_plan(const int *__restrict__ idx, int T, int K, int E, int nt_gu,
                                                  int nt_dn, int *__restrict__ seg_off, pf_item *__restrict__ items,
                                                  int *__restrict__ counts, int *__restrict__ tiles_gu,
                                                  int *__restrict__ tiles_dn, int *__restrict__ pair_tok,
                                                  int *__restrict__ pos_of, pf_queues Q) {
  __shared__ int cnt[16][64];
  __shared__ int s_nch[64], s_ich[64];
  __shared__ int s_nr;
  __shared__ int run[16][64];
  __shared__ int cache[PF_PLAN_LDS];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int TK = T * K;
  const bool cached = TK <= PF_PLAN_LDS;
  const int per = (TK + 15) / 16;
  const int lo = min(wave * per, TK), hi = min(lo + per, TK);
  cnt[wave][lane] = 0;
  __syncthreads();
  for (int base = lo; base < hi; base += 64 * 8) {  // 8 loads per lane in flight
    int ev[8];
#pragma unroll
    for (int u = 0; u < 8; u++) ev[u] = idx[min(base + 64 * u + lane, hi - 1)];
#pragma unroll
    for (int u = 0; u < 8; u++) {
      const int i = base + 64 * u + lane;
      if (i >= hi) continue;
      if (cached) cache[i] = ev[u];
      if (ev[u] >= 0 && ev[u] < E) atomicAdd(&cnt[wave][ev[u]], 1);
    }
  }
  __syncthreads();
  if (wave == 0) {  // lane = expert
    int c = 0;
    for (int v = 0; v < 16; v++) {
      run[v][lane] = c;
      c += lane < E ? cnt[v][lane] : 0;
    }
    int incl = c;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int o = __shfl_up(incl, d);
      if (lane >= d) incl += o;
    }
    const int off = incl - c;
    for (int v = 0; v < 16; v++) run[v][lane] += off;
    if (lane < E) seg_off[lane] = off;
    const int total = __shfl(incl, 63);
    if (lane == 0) seg_off[E] = total;
    const int nch = (c + PF_MT - 1) / PF_MT;
    int ich = nch;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int o = __shfl_up(ich, d);
      if (lane >= d) ich += o;
    }
    const int nr = __shfl(ich, 63);
    ich -= nch;
    for (int j = 0; j < nch; j++) items[ich + j] = pf_item{lane, j * PF_MT, min(PF_MT, c - j * PF_MT), off};
    // routed GEMM tiles, expert by expert: n-tile major, the expert's chunks adjacent, so the
    // blocks that stream the same weight rows run side by side (item << 8 | n-tile)
    for (int nt = 0; nt < nt_gu; nt++)
      for (int j = 0; j < nch; j++) tiles_gu[ich * nt_gu + nt * nch + j] = ((ich + j) << 8) | nt;
    for (int nt = 0; nt < nt_dn; nt++)
      for (int j = 0; j < nch; j++) tiles_dn[ich * nt_dn + nt * nch + j] = ((ich + j) << 8) | nt;
    const int ns = (T + PF_MT - 1) / PF_MT;
    for (int j = lane; j < ns; j += 64) items[nr + j] = pf_item{E, j * PF_MT, min(PF_MT, T - j * PF_MT), 0};
    if (lane == 0) {
      counts[0] = nr;
      counts[1] = ns;
      s_nr = nr;
    }
    s_nch[lane] = lane < E ? nch : 0;
    s_ich[lane] = ich;
  }
  if (threadIdx.x == 0) *Q.err = 0;
  __syncthreads();
  if (Q.enable) {
    // Queue units are the work items: the routed items (cost cost_r in 128-column weight stages)
    // and the shared-expert items (cost_s). Items are ranked by cost, costlier kind first, then
    // by item number, and dealt to the queues in snake order (rank 16k + j goes to queue j for
    // j < 8, to queue 15 - j otherwise), so no queue holds more than ceil(items / PF_NQ) of them.
    // Each queue lists all its gate_up tiles (item by item, n-tiles adjacent: they share the item's
    // A rows), then its down tiles, in rank order. Ranks and offsets have closed forms.
    const int ns = (T + PF_MT - 1) / PF_MT, nr = s_nr, nu = nr + ns;
    const int cost_s = Q.ngu_s * Q.nk_gu + Q.ndn * Q.nk_ds, cost_r = Q.ngu_r * Q.nk_gu + Q.ndn * Q.nk_dr;
    const bool sh_first = cost_s > cost_r;
    const int s0 = sh_first ? 0 : nr, s1 = s0 + ns;  // rank range of the shared items
    // units of queue q among ranks [0, lim)
    auto cnt = [](int q, int lim) {
      const int r = lim & (2 * PF_NQ - 1);
      return 2 * (lim / (2 * PF_NQ)) + (r > q) + (r > 2 * PF_NQ - 1 - q);
    };
    // gate_up tiles of queue q among ranks [0, lim)
    auto gtiles = [&](int q, int lim) {
      const int sh = cnt(q, min(lim, s1)) - cnt(q, min(lim, s0));
      return sh * Q.ngu_s + (cnt(q, lim) - sh) * Q.ngu_r;
    };
    if (threadIdx.x < PF_NQ) {
      const int q = threadIdx.x;
      Q.count[q] = gtiles(q, nu) + cnt(q, nu) * Q.ndn;
      Q.next[q] = 0;
    }
    for (int u = threadIdx.x; u < nu; u += 1024) {
      Q.gu_done[u] = 0;
      const bool shared = u >= nr;
      const int rank = sh_first ? (shared ? u - nr : ns + u) : u;
      const int pos = rank & (2 * PF_NQ - 1);
      const int q = pos < PF_NQ ? pos : 2 * PF_NQ - 1 - pos;
      const int gu0 = gtiles(q, rank), dn0 = gtiles(q, nu) + cnt(q, rank) * Q.ndn;
      int *qt = Q.tiles + (size_t)q * Q.cap;
      const int ngu = shared ? Q.ngu_s : Q.ngu_r;
      for (int nt = 0; nt < ngu; nt++) qt[gu0 + nt] = (u << 8) | nt;
      for (int nt = 0; nt < Q.ndn; nt++) qt[dn0 + nt] = (int)(PF_DN_TILE | (u << 8) | nt);
    }
  }
  __syncthreads();
  for (int base = lo; base < hi; base += 64) {
    const int i = base + lane;
    const int e = i < hi ? (cached ? cache[i] : idx[i]) : -1;
    const bool valid = e >= 0 && e < E;
    const int key = valid ? e : 127;
    unsigned long long same = ~0ull;
#pragma unroll
    for (int b = 0; b < 7; b++) {
      const bool bit = (key >> b) & 1;
      const unsigned long long m = __ballot(bit);
      same &= bit ? m : ~m;
    }
    const int rank = __popcll(same & ((1ull << lane) - 1ull));
    const int p = valid ? run[wave][e] + rank : -1;
    __builtin_amdgcn_wave_barrier();
    if (valid && rank == 0) run[wave][e] = p + __popcll(same);
    __builtin_amdgcn_wave_barrier();
    if (i < hi) {
      if (valid) pair_tok[p] = i / K;
      pos_of[i] = p;
    }
  }
}

// ---------------------------------------------------------------------------------- grouped GEMM
// Work tiles: the shared expert's first (n-tile major, its items adjacent), then the routed tiles in
// the plan's order (per expert: n-tile major, chunks adjacent): blocks that read the same weight rows
// are neighbours. Physical block b runs logical tile (b % 8)·C + b / 8 with C = ceil(tiles / 8):
// blocks are handed to the 8 XCDs in turn, so each XCD gets a contiguous run of tiles and
// neighbouring tiles share that XCD's L2.
__device__ __forceinline__ bool pf_tile(const int *counts, const int *tiles, int ntS, int ntR, int &item, int &nt) {
  const int nr = counts[0], ns = counts[1];
  const int nshared = ns * ntS, total = nshared + nr * ntR;
  const int C = (total + 7) / 8;
  const int b = blockIdx.x;
  if (b >= 8 * C) return false;
  const int lg = (b & 7) * C + (b >> 3);
  if (lg >= total) return false;
  if (lg < nshared) {
    nt = lg / ns;
    item = nr + (lg - nt * ns);
  } else {
    const int t = tiles[lg - nshared];
    item = t >> 8;
    nt = t & 255;
  }
  return true;
}

// One block computes C[NSUB·32 A rows][4 waves x 2 tiles x 32 weight rows] = A · B^T over K columns:
// A = activations split to bf16 (hi, lo), B = INT8 weight rows (codes → bf16 in registers).
// K runs in stages of PF_KS = 128 columns, one 128-byte line of each weight row:
// - weights: each wave streams its own 64 rows; per stage 8 loads in which 8 adjacent lanes read one
//   row's full line (full lines keep HBM at its streaming rate), held in a PF_D-stage register ring
//   and written to the wave's own LDS tile when the stage begins;
// - A: the block's rows are copied in 64-column half-stages (8 adjacent lanes read one row's 128
//   bytes of hi or lo; two half-stages ahead in registers) into a double-buffered LDS tile;
// - both LDS tiles have 128-byte rows whose 16-byte chunks are XOR-swizzled by pf_swz(row), so the
//   full-row writes and the MFMA reads (16 lanes, 16 rows, one chunk) are free of bank conflicts;
// - per 32-column block, lane half h takes columns 16h..16h+15 as two MFMA k-slices of 8 (the same
//   permutation of k for A and B leaves the product unchanged): one 16-byte LDS read gives a lane its
//   16 codes of a weight row, one 16-byte read its 8 values of an A row.
// One barrier per half-stage. The load order is the same in every stage and the first group of
// PF_D stages is peeled, so the wait counts the compiler derives keep the rings full. Stages past
// the last (K rounded up to PF_D stages) load a valid line and skip the math. A rows past the item's
// count repeat a valid row; their results are never stored.
#define PF_KS 128
#ifndef PF_D
#define PF_D 1   // weight-line stages in flight per wave
#endif
#ifndef PF_OCC
#define PF_OCC 2  // GEMM blocks per CU the register budget is sized for
#endif

struct pf_smem {
  union {
    struct {
      __bf16 A[2][2][PF_MT][64];      // [half-stage parity][hi, lo][row][column, swizzled]
      unsigned char B[4][64][PF_KS];  // per wave: its 64 weight rows x the stage's codes, swizzled
    } t;
    float red[4][64][33];  // gate_up epilogue: h values per wave for the row sums
  } u;
  float hsum[4][2][32];  // Σh of the block's A rows (per wave, per 32-row sub-tile)
  float xs[PF_MT];       // gate_up: Σx of the block's A rows (their tokens)
};

// 16-byte chunk c of LDS row r sits at chunk c ^ pf_swz(r): 16 consecutive rows map one chunk to 16
// distinct bank groups, and two consecutive rows fill 256 contiguous bytes
__device__ __forceinline__ int pf_swz(int r) { return (r ^ (r >> 3)) & 7; }

template <int NSUB>
__device__ __forceinline__ void pf_mainloop(const __bf16 *Ahi, const __bf16 *Alo, const size_t *arow, int K,
                                            const int8_t *brow0, const int8_t *brow1, f32x16 (&acc)[NSUB][2],
                                            pf_smem &sm) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, half = lane >> 5, l32 = lane & 31;
  const int ar = threadIdx.x >> 3, ac = threadIdx.x & 7;  // A copy: rows ar and ar + 32, chunk ac
  const int nk = K / PF_KS, nkp = (nk + PF_D - 1) / PF_D * PF_D, nh = 2 * nk;
#pragma unroll
  for (int ms = 0; ms < NSUB; ms++)
#pragma unroll
    for (int q = 0; q < 2; q++)
#pragma unroll
      for (int j = 0; j < 16; j++) acc[ms][q][j] = 0.0f;
  // The weight addresses take a zero offset from an asm that depends on the A rows, so the
  // prologue's weight loads are issued after the row indices are known, in the loop's order.
  int zero = 0;
  asm volatile("" : "+v"(zero) : "v"((int)arow[0]), "v"((int)arow[1]));
  const size_t K8 = (size_t)8 * K;
  const int brow = lane >> 3, bch = lane & 7;
  const int8_t *p0 = brow0 + zero + (size_t)brow * K + 16 * bch;
  const int8_t *p1 = brow1 + zero + (size_t)brow * K + 16 * bch;
  const int aw0 = 8 * (ac ^ pf_swz(ar)), aw1 = 8 * (ac ^ pf_swz(ar + 32));
  u32x4 bR[PF_D][8];
  bf16x8 aR[2][4];  // [half-stage parity][hi row ar, hi row ar+32, lo row ar, lo row ar+32]
  auto load_b = [&](u32x4(&dst)[8], int k) {
#pragma unroll
    for (int i = 0; i < 8; i++) dst[i] = *(const u32x4 *)((i < 4 ? p0 : p1) + (i & 3) * K8 + (size_t)k * PF_KS);
  };
  auto load_a = [&](bf16x8(&dst)[4], int hs) {
    const size_t o = (size_t)hs * 64 + 8 * ac;
    dst[0] = ld_bf16x8(Ahi + arow[0] + o);
    dst[1] = ld_bf16x8(Ahi + arow[1] + o);
    dst[2] = ld_bf16x8(Alo + arow[0] + o);
    dst[3] = ld_bf16x8(Alo + arow[1] + o);
  };
#pragma unroll
  for (int s = 0; s < PF_D; s++) {
    load_b(bR[s], min(s, nk - 1));
    asm volatile("" ::: "memory");
  }
  load_a(aR[0], 0);
  asm volatile("" ::: "memory");
  load_a(aR[1], min(1, nh - 1));
  asm volatile("" ::: "memory");

  auto group = [&](int kb0) {
#pragma unroll
    for (int s = 0; s < PF_D; s++) {
      const int k = kb0 + s;
      // the stage's weight lines → the wave's tile (the wave's reads of the previous stage are
      // done: a wave's LDS operations complete in order)
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const int r = 8 * i + brow;
        *(u32x4 *)&sm.u.t.B[wave][r][16 * (bch ^ pf_swz(r))] = bR[s][i];
      }
      load_b(bR[s], min(k + PF_D, nk - 1));
      asm volatile("" ::: "memory");
#pragma unroll
      for (int a = 0; a < 2; a++) {
        *(bf16x8 *)&sm.u.t.A[a][0][ar][aw0] = aR[a][0];
        *(bf16x8 *)&sm.u.t.A[a][0][ar + 32][aw1] = aR[a][1];
        *(bf16x8 *)&sm.u.t.A[a][1][ar][aw0] = aR[a][2];
        *(bf16x8 *)&sm.u.t.A[a][1][ar + 32][aw1] = aR[a][3];
        load_a(aR[a], min(2 * k + a + 2, nh - 1));
        asm volatile("" ::: "memory");
        __syncthreads();
        if (k < nk) {
#pragma unroll
          for (int s2 = 0; s2 < 2; s2++) {
            const int cb = 2 * (2 * a + s2) + half;  // weight chunk of this lane half
            const u32x4 b0 = *(const u32x4 *)&sm.u.t.B[wave][l32][16 * (cb ^ pf_swz(l32))];
            const u32x4 b1 = *(const u32x4 *)&sm.u.t.B[wave][32 + l32][16 * (cb ^ pf_swz(32 + l32))];
            bf16x8 c0[2], c1[2];
#pragma unroll
            for (int u = 0; u < 2; u++) {
              c0[u] = codes_to_bf16(u32x2{b0[2 * u], b0[2 * u + 1]});
              c1[u] = codes_to_bf16(u32x2{b1[2 * u], b1[2 * u + 1]});
            }
#pragma unroll
            for (int ms = 0; ms < NSUB; ms++)
#pragma unroll
              for (int u = 0; u < 2; u++) {
                const int m = 32 * ms + l32;
                const int ch = 4 * s2 + 2 * half + u;  // A chunk (8 columns) within the half-stage
                const bf16x8 ah = *(const bf16x8 *)&sm.u.t.A[a][0][m][8 * (ch ^ pf_swz(m))];
                const bf16x8 al = *(const bf16x8 *)&sm.u.t.A[a][1][m][8 * (ch ^ pf_swz(m))];
                acc[ms][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, c0[u], acc[ms][0], 0, 0, 0);
                acc[ms][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, c1[u], acc[ms][1], 0, 0, 0);
                acc[ms][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, c0[u], acc[ms][0], 0, 0, 0);
                acc[ms][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, c1[u], acc[ms][1], 0, 0, 0);
              }
          }
        }
      }
    }
  };
  group(0);
  for (int kb0 = PF_D; kb0 < nkp; kb0 += PF_D) group(kb0);
}

// gate_up: block = (work item, n-tile): the item's A rows (tokens) x 128 intermediate units; wave w
// owns units i0 + 32w .. +31, tile 0 = their gate rows, tile 1 = their up rows, so the SwiGLU pairs
// sit in the same lane and register.
template <bool SHARED, int NSUB>
__device__ __forceinline__ void gate_up_tile(const dsh_layer_t &L, const pf_item &it, int nt, const __bf16 *Xhi,
                                             const __bf16 *Xlo, const float *xsum, const int *pair_tok,
                                             int bf16sim, __bf16 *Hhi, __bf16 *Hlo, float *hpart,
                                             pf_smem &sm) {
  const int H = L.H;
  const int Iseg = SHARED ? L.SI : L.I, ntK = Iseg / PF_GU_N;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, l32 = lane & 31;
  const int u0 = nt * PF_GU_N + wave * 32, unit = u0 + l32;
  const int8_t *wq = SHARED ? L.sgu_q : L.gu_q + (size_t)it.seg * 2 * L.I * H;
  const float *wso = SHARED ? L.sgu_so : L.gu_so + (size_t)it.seg * 2 * L.I * 2;
  size_t arow[2];
  int tok[2];
#pragma unroll
  for (int c = 0; c < 2; c++) {
    const int r = (threadIdx.x >> 3) + 32 * c;
    const int rr = r < it.mcnt ? r : 0;
    tok[c] = SHARED ? it.m0 + rr : pair_tok[it.pos0 + it.m0 + rr];
    arow[c] = (size_t)tok[c] * H;
  }
  // the rows' Σx for the epilogue, staged in LDS (visible after the main loop's first barrier)
  if ((threadIdx.x & 7) == 0) {
    const float x0 = xsum[tok[0]], x1 = xsum[tok[1]];
    sm.xs[threadIdx.x >> 3] = x0;
    sm.xs[(threadIdx.x >> 3) + 32] = x1;
  }
  f32x16 acc[NSUB][2];
  pf_mainloop<NSUB>(Xhi, Xlo, arow, H, wq + (size_t)u0 * H, wq + (size_t)(Iseg + u0) * H, acc, sm);
  // signed codes: offset + 128·scale multiplies Σa
  float2 sog = ((const float2 *)wso)[unit], sou = ((const float2 *)wso)[Iseg + unit];
  sog.y = __builtin_fmaf(128.0f, sog.x, sog.y);
  sou.y = __builtin_fmaf(128.0f, sou.x, sou.y);
  const size_t rbase = SHARED ? (size_t)it.m0 : (size_t)(it.pos0 + it.m0);
  // The tile's h values (as the down GEMM sees them, hi + lo) also go to LDS for the row sums
  // Σh over the block's 128 units, which the down epilogue needs for the offset term.
  // The tile's h values go to LDS (per wave: 64 rows x its 32 units), from where each lane stores
  // 16-byte runs of 8 units (hi and lo) and sums a row for Σh (over the block's 128 units, for the
  // down epilogue's offset term; summed as the down GEMM sees the values, hi + lo).
  float(*red)[64][33] = sm.u.red;
  __syncthreads();  // every wave is done with the main loop's tiles
#pragma unroll
  for (int ms = 0; ms < NSUB; ms++)
#pragma unroll
    for (int j = 0; j < 16; j++) {
      const int m = ms * 32 + mfma_row(lane, j);
      float hv = 0.0f;
      if (m < it.mcnt) {
        const float xs = sm.xs[m];
        float g = __builtin_fmaf(sog.x, acc[ms][0][j], sog.y * xs);
        float up = __builtin_fmaf(sou.x, acc[ms][1][j], sou.y * xs);
        if (bf16sim) {
          g = dsh_bf16_round_half_up(g);
          up = dsh_bf16_round_half_up(up);
        }
        hv = dsh_swiglu(g, up);
        if (bf16sim) hv = dsh_bf16_round_half_up(hv);
      }
      red[wave][m][l32] = hv;
    }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  {  // stores: lane → rows (lane / 4) + 16k, units 8·(lane % 4) .. +7 of the wave's 32
    const int g8 = 8 * (lane & 3);
#pragma unroll
    for (int k = 0; k < 2 * NSUB; k++) {
      const int m = (lane >> 2) + 16 * k;
      if (m >= it.mcnt) continue;
      bf16x8 hi8, lo8;
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const float hv = red[wave][m][g8 + i];
        hi8[i] = (__bf16)hv;
        lo8[i] = (__bf16)(hv - (float)hi8[i]);
      }
      const size_t o = (rbase + m) * Iseg + u0 + g8;
      *(bf16x8 *)(Hhi + o) = hi8;
      *(bf16x8 *)(Hlo + o) = lo8;
    }
  }
  float part = 0.0f;  // lane = row: its sum over the wave's 32 units, in unit order
  if (lane < 32 * NSUB) {
#pragma unroll 8
    for (int u = 0; u < 32; u++) {
      const float hv = red[wave][lane][u];
      const __bf16 hi = (__bf16)hv;
      part += (float)hi + (float)(__bf16)(hv - (float)hi);
    }
  }
  sm.hsum[wave][lane >> 5][lane & 31] = part;
  __syncthreads();
  if (threadIdx.x < it.mcnt) {
    const int m = threadIdx.x;
    const float tot = ((sm.hsum[0][m >> 5][m & 31] + sm.hsum[1][m >> 5][m & 31]) + sm.hsum[2][m >> 5][m & 31]) +
                      sm.hsum[3][m >> 5][m & 31];
    hpart[(rbase + m) * ntK + nt] = tot;
  }
}

template <bool SHARED>
__device__ __forceinline__ void gate_up_dispatch(const dsh_layer_t &L, const pf_item &it, int nt, const __bf16 *Xhi,
                                                 const __bf16 *Xlo, const float *xsum, const int *pair_tok,
                                                 int bf16sim, __bf16 *Hhi, __bf16 *Hlo, float *hpart,
                                                 pf_smem &sm) {
  if (it.mcnt <= 32)
    gate_up_tile<SHARED, 1>(L, it, nt, Xhi, Xlo, xsum, pair_tok, bf16sim, Hhi, Hlo, hpart, sm);
  else
    gate_up_tile<SHARED, 2>(L, it, nt, Xhi, Xlo, xsum, pair_tok, bf16sim, Hhi, Hlo, hpart, sm);
}

__global__ void __launch_bounds__(256, PF_OCC) k_pf_gate_up(dsh_layer_t L, const pf_item *__restrict__ items,
                                                       const int *__restrict__ counts, const __bf16 *Xhi,
                                                       const __bf16 *Xlo, const float *__restrict__ xsum,
                                                       const int *__restrict__ pair_tok, int bf16sim,
                                                       __bf16 *__restrict__ Hhi, __bf16 *__restrict__ Hlo,
                                                       __bf16 *__restrict__ Shi, __bf16 *__restrict__ Slo,
                                                       float *__restrict__ hpr, float *__restrict__ hps,
                                                       const int *__restrict__ tiles) {
  __shared__ __attribute__((aligned(16))) pf_smem sm;
  int item, nt;
  if (!pf_tile(counts, tiles, L.SI / PF_GU_N, L.I / PF_GU_N, item, nt)) return;
  const pf_item it = items[item];
  if (it.seg == L.E)
    gate_up_dispatch<true>(L, it, nt, Xhi, Xlo, xsum, pair_tok, bf16sim, Shi, Slo, hps, sm);
  else
    gate_up_dispatch<false>(L, it, nt, Xhi, Xlo, xsum, pair_tok, bf16sim, Hhi, Hlo, hpr, sm);
}

// down: block = (work item, n-tile): the item's A rows (h of its pairs, or of tokens for the shared
// expert) x 256 output rows; wave w owns rows n0 + 64w .. +63 as two 32-row tiles. Σh of each A row
// is the sum, in n-tile order, of the per-n-tile row sums the gate_up epilogue wrote.
template <bool SHARED, int NSUB>
__device__ __forceinline__ void down_tile(const dsh_layer_t &L, const pf_item &it, int nt, const __bf16 *Hhi,
                                          const __bf16 *Hlo, const float *hpart, float *Y, pf_smem &sm) {
  const int H = L.H;
  const int Kd = SHARED ? L.SI : L.I, ntK = Kd / PF_GU_N;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, half = lane >> 5, l32 = lane & 31;
  const int8_t *wq = SHARED ? L.sdn_q : L.dn_q + (size_t)it.seg * H * L.I;
  const float *wso = SHARED ? L.sdn_so : L.dn_so + (size_t)it.seg * H * 2;
  const int nw = nt * PF_DN_N + wave * 64, n0 = nw + l32;
  const size_t rbase = SHARED ? (size_t)it.m0 : (size_t)(it.pos0 + it.m0);
  size_t arow[2];
#pragma unroll
  for (int c = 0; c < 2; c++) {
    const int r = (threadIdx.x >> 3) + 32 * c;
    arow[c] = (rbase + (r < it.mcnt ? r : 0)) * Kd;
  }
  f32x16 acc[NSUB][2];
  pf_mainloop<NSUB>(Hhi, Hlo, arow, Kd, wq + (size_t)nw * Kd, wq + (size_t)(nw + 32) * Kd, acc, sm);
  {  // lane = row of the block: Σh from the gate_up partials (each wave for itself)
    float hs = 0.0f;
    if (lane < it.mcnt) {
      // agent-scope atomic loads read the partials at L2 (in the fused kernel other CUs of this
      // XCD wrote them, and lines of this CU's L1 may mix them with older data)
      const float *hp = hpart + (rbase + lane) * ntK;
      for (int k = 0; k < ntK; k++) hs += __hip_atomic_load(hp + k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    sm.hsum[wave][half][l32] = hs;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
  for (int q = 0; q < 2; q++) {
    float2 so = ((const float2 *)wso)[n0 + 32 * q];
    so.y = __builtin_fmaf(128.0f, so.x, so.y);  // signed codes: offset + 128·scale multiplies Σh
#pragma unroll
    for (int ms = 0; ms < NSUB; ms++)
#pragma unroll
      for (int j = 0; j < 16; j++) {
        const int m = ms * 32 + mfma_row(lane, j);
        if (m >= it.mcnt) continue;
        const float hs = sm.hsum[wave][ms][mfma_row(lane, j)];
        Y[(rbase + m) * H + n0 + 32 * q] = __builtin_fmaf(so.x, acc[ms][q][j], so.y * hs);
      }
  }
}

template <bool SHARED>
__device__ __forceinline__ void down_dispatch(const dsh_layer_t &L, const pf_item &it, int nt, const __bf16 *Hhi,
                                              const __bf16 *Hlo, const float *hpart, float *Y, pf_smem &sm) {
  if (it.mcnt <= 32)
    down_tile<SHARED, 1>(L, it, nt, Hhi, Hlo, hpart, Y, sm);
  else
    down_tile<SHARED, 2>(L, it, nt, Hhi, Hlo, hpart, Y, sm);
}

__global__ void __launch_bounds__(256, PF_OCC) k_pf_down(dsh_layer_t L, const pf_item *__restrict__ items,
                                                    const int *__restrict__ counts, const __bf16 *Hhi,
                                                    const __bf16 *Hlo, const __bf16 *Shi, const __bf16 *Slo,
                                                    const float *__restrict__ hpr, const float *__restrict__ hps,
                                                    float *__restrict__ Y, float *__restrict__ Ysh,
                                                    const int *__restrict__ tiles) {
  __shared__ __attribute__((aligned(16))) pf_smem sm;
  int item, nt;
  if (!pf_tile(counts, tiles, L.H / PF_DN_N, L.H / PF_DN_N, item, nt)) return;
  const pf_item it = items[item];
  if (it.seg == L.E)
    down_dispatch<true>(L, it, nt, Shi, Slo, hps, Ysh, sm);
  else
    down_dispatch<false>(L, it, nt, Hhi, Hlo, hpr, Y, sm);
}

// Fused grouped GEMM: one launch runs every gate_up and down tile, one tile per block. A block
// serves the work queue of its own XCD (hardware XCC id) and claims the queue's next tile; the
// grid holds more blocks per XCD than any queue has tiles, and blocks that find their queue empty
// exit. A queue lists all its gate_up tiles, then its down tiles; a down tile needs all gate_up
// tiles of its item, which sit earlier in the same queue: they were claimed by blocks that run
// (blocks are dispatched in order, so they are resident or done) and wait on nothing, so the
// down block's bounded wait always ends. As gate_up tiles finish, down tiles start in their place
// (no tail between the two projections). Coherence is XCD-local: a gate_up block drains its stores
// to the XCD's L2 (vmcnt(0) in every thread, then a barrier) before one thread bumps the item's
// counter with an L2 atomic; the down block reads the counter at L2, and the h rows it then loads
// were written by this XCD (each 128-byte line by one block) and never read here before. Claim
// counters and item counters are zeroed by the plan kernel.
#define PF_SPIN_MAX (1 << 22)
#define PF_PROBE 4096  // blocks of the XCD placement check
__global__ void __launch_bounds__(256, PF_OCC) k_pf_moe(dsh_layer_t L, const pf_item *__restrict__ items,
                                                    pf_queues Q, const __bf16 *Xhi, const __bf16 *Xlo,
                                                    const float *__restrict__ xsum, const int *__restrict__ pair_tok,
                                                    int bf16sim, __bf16 *Hhi, __bf16 *Hlo, __bf16 *Shi, __bf16 *Slo,
                                                    float *hpr, float *hps, float *__restrict__ Y,
                                                    float *__restrict__ Ysh) {
  __shared__ __attribute__((aligned(16))) pf_smem sm;
  __shared__ int s_tile;
  unsigned xcc;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
  const int q = xcc & (PF_NQ - 1);
  if (threadIdx.x == 0) s_tile = __hip_atomic_fetch_add(Q.next + q, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  const int t = s_tile;
  if (t >= Q.count[q]) return;
  const unsigned d = (unsigned)Q.tiles[(size_t)q * Q.cap + t];
  const int item = (int)((d & ~PF_DN_TILE) >> 8), nt = (int)(d & 255);
  const pf_item it = items[item];
  if (!(d & PF_DN_TILE)) {
    if (it.seg == L.E)
      gate_up_dispatch<true>(L, it, nt, Xhi, Xlo, xsum, pair_tok, bf16sim, Shi, Slo, hps, sm);
    else
      gate_up_dispatch<false>(L, it, nt, Xhi, Xlo, xsum, pair_tok, bf16sim, Hhi, Hlo, hpr, sm);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's h stores are in L2
    __syncthreads();
    if (threadIdx.x == 0) __hip_atomic_fetch_add(Q.gu_done + item, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    if (threadIdx.x == 0) {
      const int need = it.seg == L.E ? L.SI / PF_GU_N : L.I / PF_GU_N;
      int spins = 0;
      while (__hip_atomic_load(Q.gu_done + item, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < need) {
        if (++spins > PF_SPIN_MAX) {
          __hip_atomic_store(Q.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
    }
    __syncthreads();
    if (it.seg == L.E)
      down_dispatch<true>(L, it, nt, Shi, Slo, hps, Ysh, sm);
    else
      down_dispatch<false>(L, it, nt, Hhi, Hlo, hpr, Y, sm);
  }
}

// XCC id of each block, to check that a grid's blocks cover all PF_NQ XCDs before the fused kernel
// is used.
__global__ void __launch_bounds__(64) k_pf_xcc_probe(int *__restrict__ out) {
  unsigned xcc;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
  if (threadIdx.x == 0) out[blockIdx.x] = (int)xcc;
}

// ---------------------------------------------------------------------------------- combine
// One block per token: routed slots in ascending expert order (the reference's scatter-add order,
// ds_moe_decoder.c:781-795; equal experts keep slot order), weights w_k, then the shared output
// and the residual.
__global__ void __launch_bounds__(256) k_pf_combine(const float *__restrict__ X, const int *__restrict__ idx,
                                                    const float *__restrict__ w, const int *__restrict__ pos_of,
                                                    const float *__restrict__ Y, const float *__restrict__ Ysh,
                                                    int H, int K, int residual, int bf16sim, float *__restrict__ out) {
  __shared__ int s_pos[64];
  __shared__ float s_w[64];
  __shared__ int s_n;
  const int t = blockIdx.x;
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    const int e = lane < K ? idx[(size_t)t * K + lane] : -1;
    const int pos = lane < K ? pos_of[(size_t)t * K + lane] : -1;
    const float wt = lane < K ? w[(size_t)t * K + lane] : 0.0f;
    const bool valid = e >= 0 && pos >= 0;
    int rank = 0;
    for (int j = 0; j < K; j++) {
      const int ej = __shfl(e, j), pj = __shfl(pos, j);
      if (ej >= 0 && pj >= 0 && (ej < e || (ej == e && j < lane))) rank++;
    }
    if (valid) {
      s_pos[rank] = pos;
      s_w[rank] = wt;
    }
    const int n = __popcll(__ballot(valid));
    if (lane == 0) s_n = n;
  }
  __syncthreads();
  const int n = s_n;
  for (int c = threadIdx.x; c < H / 4; c += 256) {
    f32x4 routed = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int j = 0; j < n; j++) {
      f32x4 v = ((const f32x4 *)(Y + (size_t)s_pos[j] * H))[c];
      const float wj = s_w[j];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        if (bf16sim) v[i] = dsh_bf16_round_half_up(v[i]);
        routed[i] = __builtin_fmaf(wj, v[i], routed[i]);
      }
    }
    f32x4 sh = ((const f32x4 *)(Ysh + (size_t)t * H))[c];
    f32x4 o;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      if (bf16sim) sh[i] = dsh_bf16_round_half_up(sh[i]);
      o[i] = routed[i] + sh[i];
    }
    if (residual) {
      const f32x4 x = ((const f32x4 *)(X + (size_t)t * H))[c];
#pragma unroll
      for (int i = 0; i < 4; i++) o[i] = x[i] + o[i];
    }
    ((f32x4 *)(out + (size_t)t * H))[c] = o;
  }
}

// ---------------------------------------------------------------------------------- launchers
namespace {
struct pf_ws {
  __bf16 *Xhi, *Xlo;
  float *xsum;
  int *idx;
  float *w;
  int *seg_off, *counts;
  pf_item *items;
  int *pair_tok, *pos_of;
  __bf16 *Hhi, *Hlo, *Shi, *Slo;
  float *Y, *Ysh;
  float *ps;        // [T][4][64] partial router scores
  float *hpr, *hps; // Σh partials per (row, gate_up n-tile): routed [TK][I/128], shared [T][SI/128]
  int *tiles_gu, *tiles_dn;  // routed GEMM tiles (item << 8 | n-tile) in launch order
  int *qtiles, *qcount, *qnext, *gu_done, *err;  // fused kernel: work queues, counters, wait error
};

size_t al256(size_t n) { return (n + 255) & ~(size_t)255; }

int pf_max_routed_items(const dsh_layer_t *L, int T) { return (T * L->K + PF_MT - 1) / PF_MT + L->E; }
int pf_shared_items(int T) { return (T + PF_MT - 1) / PF_MT; }

// Blocks of a GEMM launch: every tile of the largest possible work list, rounded up to 8.
int pf_grid(const dsh_layer_t *L, int T, int ntS, int ntR) {
  const int n = pf_shared_items(T) * ntS + pf_max_routed_items(L, T) * ntR;
  return (n + 7) & ~7;
}

// Tiles one fused-kernel queue can hold: every gate_up and down tile of the largest work list.
size_t pf_queue_cap(const dsh_layer_t *L, int T) {
  const size_t r = pf_max_routed_items(L, T), sh = pf_shared_items(T);
  return r * (L->I / PF_GU_N) + sh * (L->SI / PF_GU_N) + (r + sh) * (L->H / PF_DN_N);
}

int g_pf_xcd_min = 0;  // fewest blocks any XCD received out of a probe grid of PF_PROBE blocks
int g_pf_auto = -1;   // -1 unchecked, 1 the grid's blocks cover all PF_NQ XCDs, 0 not
int g_pf_fused = -1;  // path in use

// Carves the workspace; returns its size (ws may be NULL to size it).
size_t pf_carve(const dsh_layer_t *L, int T, void *base, pf_ws *w) {
  const size_t H = L->H, I = L->I, SI = L->SI, K = L->K, E = L->E, TK = (size_t)T * K;
  size_t off = 0;
  char *b = (char *)base;
#define TAKE(field, type, count)                          \
  do {                                                    \
    if (w) w->field = (type *)(b + off);                  \
    off += al256(sizeof(type) * (size_t)(count));         \
  } while (0)
  TAKE(Xhi, __bf16, T * H);
  TAKE(Xlo, __bf16, T * H);
  TAKE(xsum, float, T);
  TAKE(idx, int, TK);
  TAKE(w, float, TK);
  TAKE(seg_off, int, E + 1);
  TAKE(counts, int, 2);
  TAKE(items, pf_item, pf_max_routed_items(L, T) + pf_shared_items(T));
  TAKE(pair_tok, int, TK);
  TAKE(pos_of, int, TK);
  TAKE(Hhi, __bf16, TK * I);
  TAKE(Hlo, __bf16, TK * I);
  TAKE(Shi, __bf16, T * SI);
  TAKE(Slo, __bf16, T * SI);
  TAKE(Y, float, TK * H);
  TAKE(Ysh, float, T * H);
  TAKE(ps, float, (size_t)T * 4 * 64);
  TAKE(hpr, float, TK * (I / PF_GU_N));
  TAKE(hps, float, (size_t)T * (SI / PF_GU_N));
  TAKE(tiles_gu, int, (size_t)pf_max_routed_items(L, T) * (I / PF_GU_N));
  TAKE(tiles_dn, int, (size_t)pf_max_routed_items(L, T) * (H / PF_DN_N));
  TAKE(qtiles, int, (size_t)PF_NQ * pf_queue_cap(L, T));
  TAKE(qcount, int, PF_NQ);
  TAKE(qnext, int, PF_NQ);
  TAKE(gu_done, int, pf_max_routed_items(L, T) + pf_shared_items(T));
  TAKE(err, int, 1);
#undef TAKE
  return off;
}
}  // namespace

extern "C" {

int dsh_pf_supported(const dsh_layer_t *L) {
  if (L->H % PF_DN_N || L->I % PF_GU_N || L->SI % PF_GU_N) return 0;
  if (L->H % PF_KS || L->I % PF_KS || L->SI % PF_KS) return 0;
  if (L->E > 64 || L->K > 64 || L->K > L->E) return 0;
  if ((size_t)PF_TB * L->H * sizeof(float) > 96 * 1024) return 0;  // DECODE scores: x rows in LDS
  return 1;
}

size_t dsh_pf_workspace_bytes(const dsh_layer_t *L, int T) { return pf_carve(L, T, NULL, NULL); }

// Checks, once, that a grid's blocks are dealt evenly over all PF_NQ XCDs (each XCD's work queue is
// served only by its own blocks); otherwise the two-kernel path is used.
// Synchronous: call outside stream capture. force: 1 fused, 0 two kernels, -1 decide by the check,
// -2 only make sure the check has run (keeps a path chosen earlier).
hipError_t dsh_pf_init(int force) {
  if (g_pf_auto < 0) {
    int *d = NULL;
    hipError_t e = hipMalloc(&d, sizeof(int) * PF_PROBE);
    if (e != hipSuccess) return e;
    k_pf_xcc_probe<<<PF_PROBE, 64>>>(d);
    int *h = (int *)malloc(sizeof(int) * PF_PROBE);
    e = hipGetLastError();
    if (e == hipSuccess && h) e = hipMemcpy(h, d, sizeof(int) * PF_PROBE, hipMemcpyDeviceToHost);
    (void)hipFree(d);
    int per[PF_NQ] = {0}, bad = 0;
    if (e == hipSuccess && h)
      for (int i = 0; i < PF_PROBE; i++) {
        if (h[i] >= 0 && h[i] < PF_NQ)
          per[h[i]]++;
        else
          bad = 1;
      }
    free(h);
    if (e != hipSuccess) return e;
    g_pf_xcd_min = PF_PROBE;
    for (int q = 0; q < PF_NQ; q++) g_pf_xcd_min = per[q] < g_pf_xcd_min ? per[q] : g_pf_xcd_min;
    // the fused launch gives each XCD its share of a grid sized for the longest queue: blocks
    // must be dealt evenly over all PF_NQ XCDs
    g_pf_auto = g_pf_fused = !bad && g_pf_xcd_min * PF_NQ >= PF_PROBE - PF_NQ ? 1 : 0;
  }
  if (force >= 0)
    g_pf_fused = force ? 1 : 0;
  else if (force == -1 || g_pf_fused < 0)
    g_pf_fused = g_pf_auto;
  return hipSuccess;
}

int dsh_pf_fused(void) { return g_pf_fused == 1; }

int dsh_pf_wait_error(const void *ws, const dsh_layer_t *L, int T) {
  pf_ws w;
  pf_carve(L, T, (void *)ws, &w);
  int v = 0;
  if (hipMemcpy(&v, w.err, sizeof v, hipMemcpyDeviceToHost) != hipSuccess) return -1;
  return v;
}

hipError_t dsh_launch_prefill(const dsh_layer_t *L, const float *X, int T, int route_mode, int nthreads, int residual,
                              int bf16sim, float *out, void *ws, int *idx_out, float *w_out, hipStream_t s) {
  if (T <= 0 || !dsh_pf_supported(L)) return hipErrorInvalidValue;
  if (route_mode == DSH_ROUTE_CFG ? !L->router_f32_t : !L->router_bf16) return hipErrorInvalidValue;
  pf_ws w;
  pf_carve(L, T, ws, &w);
  const int H = L->H, K = L->K, E = L->E;
  // CFG partial sums over the same row blocks as the decode path (8 rows, 16 past 1280 columns)
  const int R = H / dsh_dec_partials(H);
  if (route_mode == DSH_ROUTE_CFG) {
    const dim3 g((T + PF_SC_TOK - 1) / PF_SC_TOK, 4);
    if (R == 16)
      k_pf_scores_cfg<16><<<g, 256, 0, s>>>(L->router_f32_t, X, T, H, E, w.ps);
    else
      k_pf_scores_cfg<8><<<g, 256, 0, s>>>(L->router_f32_t, X, T, H, E, w.ps);
    k_pf_select<DSH_ROUTE_CFG><<<(T + 3) / 4, 256, 0, s>>>(X, T, H, E, K, w.ps, w.Xhi, w.Xlo, w.xsum, w.idx, w.w);
  } else {
    k_pf_scores_bf16<<<(T + PF_TB - 1) / PF_TB, 256, (size_t)PF_TB * H * sizeof(float), s>>>(
        L->router_bf16, X, T, H, E, nthreads, w.ps);
    k_pf_select<DSH_ROUTE_DECODE><<<(T + 3) / 4, 256, 0, s>>>(X, T, H, E, K, w.ps, w.Xhi, w.Xlo, w.xsum, w.idx,
                                                                w.w);
  }
  const int n_items_max = pf_max_routed_items(L, T) + pf_shared_items(T);
  const bool fused = g_pf_fused == 1 && n_items_max < (1 << 22);
  pf_queues Q{w.qtiles, w.qcount, w.qnext, w.gu_done, w.err, (int)pf_queue_cap(L, T), L->I / PF_GU_N, L->SI / PF_GU_N,
              H / PF_DN_N, H / PF_KS, L->I / PF_KS, L->SI / PF_KS, fused ? 1 : 0};
  k_pf_plan<<<1, 1024, 0, s>>>(w.idx, T, K, E, L->I / PF_GU_N, H / PF_DN_N, w.seg_off, w.items, w.counts,
                               w.tiles_gu, w.tiles_dn, w.pair_tok, w.pos_of, Q);
  if (fused) {
    // blocks per XCD >= tiles of the longest queue (at most ceil(items / PF_NQ) items)
    const int per_item = max(L->I / PF_GU_N, L->SI / PF_GU_N) + H / PF_DN_N;
    const int blocks = PF_NQ * ((n_items_max + PF_NQ - 1) / PF_NQ) * per_item;
    k_pf_moe<<<blocks, 256, 0, s>>>(*L, w.items, Q, w.Xhi, w.Xlo, w.xsum, w.pair_tok, bf16sim, w.Hhi,
                                         w.Hlo, w.Shi, w.Slo, w.hpr, w.hps, w.Y, w.Ysh);
  } else {
    k_pf_gate_up<<<pf_grid(L, T, L->SI / PF_GU_N, L->I / PF_GU_N), 256, 0, s>>>(
        *L, w.items, w.counts, w.Xhi, w.Xlo, w.xsum, w.pair_tok, bf16sim, w.Hhi, w.Hlo, w.Shi, w.Slo, w.hpr, w.hps,
        w.tiles_gu);
    k_pf_down<<<pf_grid(L, T, H / PF_DN_N, H / PF_DN_N), 256, 0, s>>>(*L, w.items, w.counts, w.Hhi, w.Hlo, w.Shi,
                                                                       w.Slo, w.hpr, w.hps, w.Y, w.Ysh, w.tiles_dn);
  }
  k_pf_combine<<<T, 256, 0, s>>>(X, w.idx, w.w, w.pos_of, w.Y, w.Ysh, H, K, residual, bf16sim, out);
  hipError_t e = hipGetLastError();
  if (e == hipSuccess && idx_out)
    e = hipMemcpyAsync(idx_out, w.idx, sizeof(int) * (size_t)T * K, hipMemcpyDeviceToDevice, s);
  if (e == hipSuccess && w_out)
    e = hipMemcpyAsync(w_out, w.w, sizeof(float) * (size_t)T * K, hipMemcpyDeviceToDevice, s);
  return e;
}

}  // extern "C"
