// k_prefill.hip — prefill MoE block (T tokens) for the device-resident layer: routing, an
// expert-sorted grouped GEMM on the int8 MFMA with the INT8 weights as stored, SwiGLU, the down
// projection and a deterministic combine (ds_moe_decoder.c:629-809 is the reference block; it runs
// sgemm on bf16 weights, this build runs the same layer's INT8 blocks).
//
// Numerics. The stored codes q = u - 128 (-128..127) are the MFMA's B operand as they are. Each
// activation row (x per token for gate_up, h per pair or token for down) is two signed 8-bit limbs
// of X = rint(a·2^(15-e)) = 256·X1 + X0 with 2^e > max|a|·(1 + 2^-7) (|X0|, |X1| <= 128; a to 2^-15
// of the row's maximum), so Σ q·a = 2^(e-15)·(256·Σ q·X1 + Σ q·X0) with exact int32 sums. x takes
// one exponent per token. h is written by the gate_up tiles, each 128-unit n-tile of a row at its
// own exponent (the tile's max |h|); the down GEMM aligns every n-tile to the row's largest exponent
// (a right shift, ties to even) as it stages the limbs, so tiles below the row's exponent are
// rounded twice. The epilogues fold the row's scale and offset: y = scale·Σu·a + offset·Σa =
// scale·Σq·a + (offset + 128·scale)·Σa, with Σa of the f32 values.
//
// Kernels (one launch each, all sizes fixed by T, so a graph can hold them):
//   k_pf_route_cfg  CFG: per token, the router scores in ds_linear's order, x → the two int8 limbs
//                and their scale, Σx; expert selection → idx, w
//   k_pf_scores_bf16, k_pf_select_dec  DECODE: the bf16 router's scores in the reference's AVX-512
//                order, then the limbs and the selection
//   k_pf_plan    expert-sorted (token, slot) pairs (stable: tokens in increasing order per expert),
//                per-expert offsets and the GEMM work items (expert, up-to-PF_MT-row chunk)
//   k_pf_gate_up grouped GEMM + SwiGLU → h as limbs, its per-(row, n-tile) sums and maxima, for
//                routed pairs and for the shared expert
//   k_pf_down    grouped GEMM → Y (f32) per routed pair and per token for the shared expert
//   k_pf_moe     both GEMMs in one launch (per-XCD work queues), in place of the two above
//   k_pf_combine out[t] = (residual ? x : 0) + (Σ_k w_k·Y_k in ascending expert order + Y_shared)
#include "dsh_avx.h"
#include "dsh_route.h"
#include "k_core.h"
#include <type_traits>

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

#define PF_MT 64    // rows of A per work item: one or two MFMA sub-tiles of 32 rows
#define PF_GU_N 128 // gate_up: intermediate units per block (128 gate + 128 up weight rows)
#define PF_DN_N 256 // down: output rows per block
#define PF_NT_MAX 16  // down: 128-column stages per A row (I, SI <= 2048)
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
  int *derr;     // the library's device error word for this failure (host memory; never cleared here)
  int spin_max;  // sleeps before a wait gives up; < 0: every wait gives up at once (test mode)
  int cap;
  int ngu_r, ngu_s, ndn;      // n-tiles: gate_up routed / shared, down
  int nk_gu, nk_dr, nk_ds;    // 128-column stages: gate_up, routed down, shared down
  int enable;
};

// h as int8 limbs (low 0, high 1), each 128-column n-tile of a row at its own exponent: routed
// [TK][I], shared [T][SI].
struct pf_hq {
  int8_t *r0, *r1, *s0, *s1;
};

struct pf_item {
  int seg;   // expert 0..E-1, or E for the shared expert
  int m0;    // first row of the chunk within the segment
  int mcnt;  // rows in the chunk (1..PF_MT)
  int pos0;  // first routed pair position of the segment (routed only)
};

// ---------------------------------------------------------------------------------- routing
// One token's x as two int8 limbs (X0 low, X1 high) with their scale 2^(e-15) and Σx, for the
// GEMM's activations: one wave, lane-strided float4s (H <= 256·PF_SEL_U, the whole row in
// registers). xrow (optional, LDS) receives the row itself. Stores only when own.
#define PF_SEL_U 8  // x float4 loads per lane
__device__ __forceinline__ void pf_x_limbs(const float *__restrict__ X, int t, int H, bool own, int8_t *X0, int8_t *X1,
                                           float *xsc, float *xsum, float *xrow) {
  const int lane = threadIdx.x & 63;
  const f32x4 *src = (const f32x4 *)(X + (size_t)t * H);
  const int nc = H / 4;
  f32x4 xv[PF_SEL_U];
#pragma unroll
  for (int u = 0; u < PF_SEL_U; u++) xv[u] = src[min(64 * u + lane, nc - 1)];
  float s = 0.0f, mx = 0.0f;
#pragma unroll
  for (int u = 0; u < PF_SEL_U; u++) {
    if (64 * u + lane >= nc) continue;
    const f32x4 v = xv[u];
    if (xrow) *(f32x4 *)(xrow + 4 * (64 * u + lane)) = v;
    s += (v[0] + v[1]) + (v[2] + v[3]);
    mx = fmaxf(fmaxf(mx, fmaxf(fabsf(v[0]), fabsf(v[1]))), fmaxf(fabsf(v[2]), fabsf(v[3])));
  }
  s = dsh_wave_sum(s);
  mx = dsh_wave_max(mx);
  if (!own) return;
  const int ex = __builtin_amdgcn_frexp_expf(mx * 1.0078125f);  // 2^ex > max|x|·(1 + 2^-7)
#pragma unroll
  for (int u = 0; u < PF_SEL_U; u++) {
    const int c = 64 * u + lane;
    if (c >= nc) continue;
    unsigned w0 = 0u, w1 = 0u;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int q = (int)__builtin_rintf(__builtin_ldexpf(xv[u][i], 15 - ex));  // |q| < 2^15 / (1 + 2^-7)
      const int lo = __builtin_amdgcn_sbfe(q, 0, 8);                            // balanced low digit
      const int hi = (q - lo) >> 8;                                              // |hi| <= 127
      w0 |= ((unsigned)lo & 255u) << (8 * i);
      w1 |= ((unsigned)hi & 255u) << (8 * i);
    }
    *(unsigned *)(X0 + (size_t)t * H + 4 * c) = w0;
    *(unsigned *)(X1 + (size_t)t * H + 4 * c) = w1;
  }
  if (lane == 0) {
    xsum[t] = s;
    xsc[t] = __builtin_ldexpf(1.0f, ex - 15);
  }
}

// CFG (f32 router: ds_moe_router → ds_linear_nobias → ds_linear, ds_kernels.c:181-185, :639-652):
// every score in ds_linear's own order, so the selection is ds_moe_top_k's (:193-243) by
// construction. ds_linear (no BLAS, seq 1, as GCC 11 compiles it) adds the rounded products
// fl(x_k·w_ek) in index order from 0; the tail past the last multiple of 8 (16 when H >= 16) would be
// fused, and H is a multiple of 256 here, so there is none. One wave per token, lane = expert: each
// lane runs its own chain of H dependent adds, all T·E chains at once (one chain's latency for the
// whole batch). The block's 4 tokens share the transposed router rows [H][E], staged in LDS
// PF_RC_KC rows at a time with row stride 64 (double-buffered: the next chunk's loads are in flight
// during the current chunk's chain, one barrier per chunk); each token's x stays in LDS, read as a
// broadcast. The wave also writes its token's x limbs (pf_x_limbs), then selects and weights the
// experts (route_select: top-k with strict >, softmax over the k).
#define PF_RC_KC 128
#define PF_RC_WARM 2  // router lines a thread touches to fill its XCD's L2
#define PF_RC_D 5     // groups of 4 chain steps whose LDS reads are in flight
template <bool E64>
__global__ void __launch_bounds__(256) k_pf_route_cfg(const float *__restrict__ WrT, const float *__restrict__ X,
                                                      int T, int H, int E, int K, int8_t *__restrict__ X0,
                                                      int8_t *__restrict__ X1, float *__restrict__ xsc,
                                                      float *__restrict__ xsum, int *__restrict__ idx,
                                                      float *__restrict__ w) {
  __shared__ __attribute__((aligned(16))) float s_wr[2][PF_RC_KC * 64];
  __shared__ __attribute__((aligned(16))) float s_x[4][256 * PF_SEL_U];
  __shared__ float s_red[4][4][64];
  __shared__ int s_idx[4][64];
  __shared__ float s_w[4][64];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const bool own = (int)blockIdx.x * 4 + wave < T;
  const int t = min((int)blockIdx.x * 4 + wave, T - 1);  // past T: the last token again, nothing stored
  const int nch = H / PF_RC_KC;
  // Every XCD's L2 gets the whole router first: block b touches lines (b / 8) + n8·j (n8 = blocks per
  // XCD when the grid is dealt to the 8 XCDs in turn; any other dealing only makes this prefetch
  // partial). The loaded words feed a condition that never holds, which keeps the loads.
  // At most PF_RC_WARM lines per thread, all loads issued before any is used (small grids warm part
  // of the router; the chunk pipeline below covers the rest).
  unsigned warm = 0;
  {
    const int lines = (H * E + 31) / 32, n8 = ((int)gridDim.x + 7) >> 3, r = (int)blockIdx.x >> 3;
    unsigned v[PF_RC_WARM];
#pragma unroll
    for (int j = 0; j < PF_RC_WARM; j++)
      v[j] = __float_as_uint(WrT[32 * (size_t)min(r + n8 * ((int)threadIdx.x + 256 * j), lines - 1)]);
#pragma unroll
    for (int j = 0; j < PF_RC_WARM; j++) warm ^= v[j];
  }
  // chunk c = router rows c·KC .. +KC-1 (KC·E contiguous floats) into LDS rows of 64 (zeros past E),
  // through two register sets: a chunk's loads are issued two chunks before it is stored
  constexpr int NQ = PF_RC_KC * 64 / 4 / 256;  // float4 slots per thread
  static_assert(4 * NQ == PF_RC_KC / 4, "one piece per four groups of the chain");
  f32x4 ra[NQ], rb[NQ];
  auto load_chunk = [&](f32x4 (&r)[NQ], int c) {
    const float *src = WrT + (size_t)min(c, nch - 1) * PF_RC_KC * E;
#pragma unroll
    for (int j = 0; j < NQ; j++) {
      const int i = threadIdx.x + 256 * j;  // slot: row i / 16, experts 4 (i % 16) .. +3
      if (E64) {
        r[j] = ((const f32x4 *)src)[i];
      } else {
        const int row = i >> 4, e0 = 4 * (i & 15);
#pragma unroll
        for (int q = 0; q < 4; q++) r[j][q] = src[(size_t)row * E + min(e0 + q, E - 1)];
      }
    }
  };
  auto store_chunk = [&](const f32x4 (&r)[NQ], int buf) {
#pragma unroll
    for (int j = 0; j < NQ; j++) {
      const int i = threadIdx.x + 256 * j;
      f32x4 v = r[j];
      if (!E64) {
        const int e0 = 4 * (i & 15);
#pragma unroll
        for (int q = 0; q < 4; q++) v[q] = e0 + q < E ? v[q] : 0.0f;
      }
      ((f32x4 *)s_wr[buf])[i] = v;
    }
  };
  // piece j of a chunk (every thread's register slot j) into LDS buffer buf: the chain of one chunk
  // stores the next chunk piece by piece between its groups, so the stores overlap the adds
  auto store_piece = [&](const f32x4 (&r)[NQ], int buf, int j) {
    const int i = threadIdx.x + 256 * j;
    f32x4 v = r[j];
    if (!E64) {
      const int e0 = 4 * (i & 15);
#pragma unroll
      for (int q = 0; q < 4; q++) v[q] = e0 + q < E ? v[q] : 0.0f;
    }
    ((f32x4 *)s_wr[buf])[i] = v;
  };
  load_chunk(ra, 0);
  load_chunk(rb, 1);
  asm volatile("" ::: "memory");
  pf_x_limbs(X, t, H, own, X0, X1, xsc, xsum, s_x[wave]);
  store_chunk(ra, 0);
  load_chunk(ra, 2);
  __syncthreads();
  float s = 0.0f;
  // chunk c from LDS buffer c & 1; meanwhile chunk c + 1 (in r) goes to the other buffer, which every
  // wave finished before the last barrier, one piece after every fourth group; then r is reloaded with
  // chunk c + 3. Unconditional (after the last chunk a copy of it goes to a buffer that is not read
  // again), so the waits before the stores leave the other register set's loads in flight.
  // The chain reads its operands from LDS through a ring of PF_RC_D groups of 4 steps, issued PF_RC_D
  // groups ahead: per group two ds_read2st64 for the router values (lane = expert) and one 16-byte
  // read of the token's x values at one address for every lane (a broadcast; a DPP row broadcast
  // per step instead cost ~3.7 ns a step more in a microbenchmark). The products run one group
  // ahead of the adds, one between consecutive adds; the scheduling barriers keep that order, so
  // each group waits only for its own reads.
  auto step = [&](int c, f32x4 (&r)[NQ]) {
    const float *wr = s_wr[c & 1] + lane;
    const float *xs = s_x[wave] + c * PF_RC_KC;
    constexpr int G = PF_RC_KC / 4;
    float wq[PF_RC_D][4];
    f32x4 xq[PF_RC_D];
    auto ld = [&](int g, int slot) {
#pragma unroll
      for (int i = 0; i < 4; i++) wq[slot][i] = wr[64 * (4 * g + i)];
      xq[slot] = *(const f32x4 *)(xs + 4 * g);  // one address for every lane: a broadcast read
    };
#pragma unroll
    for (int g = 0; g < PF_RC_D; g++) ld(g, g);
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; i++) p[i] = __fmul_rn(xq[0][i], wq[0][i]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int g = 0; g < G; g++) {
      float pn[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {  // one product of the next group between consecutive adds
        if (g + 1 < G) pn[i] = __fmul_rn(xq[(g + 1) % PF_RC_D][i], wq[(g + 1) % PF_RC_D][i]);
        s = __fadd_rn(s, p[i]);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (g + PF_RC_D < G) ld(g + PF_RC_D, g % PF_RC_D);  // group g's values were used by the last products
      if ((g & 3) == 3) store_piece(r, (c + 1) & 1, g >> 2);
#pragma unroll
      for (int i = 0; i < 4; i++) p[i] = pn[i];
      __builtin_amdgcn_sched_barrier(0);
    }
    load_chunk(r, c + 3);
    __syncthreads();
  };
  for (int c = 0; c < nch; c += 2) {  // nch is even (H is a multiple of 256)
    step(c, rb);
    step(c + 1, ra);
  }
  if (warm == 0x9E3779B9u && T < 0) w[0] = 0.0f;
  s_red[wave][0][lane] = lane < E ? s : 0.0f;
  s_red[wave][1][lane] = 0.0f;
  s_red[wave][2][lane] = 0.0f;
  s_red[wave][3][lane] = 0.0f;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  route_select(E, K, DSH_ROUTE_CFG, s_idx[wave], s_w[wave], s_red[wave]);
  if (own && lane < K) {
    idx[(size_t)t * K + lane] = s_idx[wave][lane];
    w[(size_t)t * K + lane] = s_w[wave][lane];
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


// The same scores with each lane's share of its router row held in registers, for H = 32·N32 when
// every row takes the reference's 4- or 2-row group path (no single rows): a block loads its 64
// rows once (group g of 4 lanes = expert g; lane L holds columns 32i + 8L .. + 7 for every i) and
// runs its tpb tokens from LDS, one token row per pass (double-buffered: the next token's loads are
// in flight during the current pass), with the chains, order and tree of avx_row
// (avx_row_regs32). The rows stream from L2 once per block instead of once per token.
template <int N32>
__global__ void __launch_bounds__(256) k_pf_scores_bf16r(const uint16_t *__restrict__ Wr, const float *__restrict__ X,
                                                         int T, int E, int tpb, float *__restrict__ ps) {
  constexpr int H = 32 * N32, NX = H / 4, XL = (NX + 255) / 256;
  __shared__ __attribute__((aligned(16))) float xs[2][H];
  const int L = threadIdx.x & 3, g = threadIdx.x >> 2, e = min(g, E - 1);
  const int t0 = blockIdx.x * tpb, nt = min(tpb, T - t0);
  if (nt <= 0) return;  // uniform per block: no barrier is skipped by part of a block
  u32x4 wv[N32];
  const u32x4 *wrow = (const u32x4 *)(Wr + (size_t)e * H) + L;
#pragma unroll
  for (int i = 0; i < N32; i++) wv[i] = wrow[4 * i];
  f32x4 xr[XL];
  auto load_x = [&](int t) {
#pragma unroll
    for (int j = 0; j < XL; j++) xr[j] = ((const f32x4 *)(X + (size_t)t * H))[min((int)threadIdx.x + 256 * j, NX - 1)];
  };
  auto store_x = [&](int b) {
#pragma unroll
    for (int j = 0; j < XL; j++) {
      const int i = threadIdx.x + 256 * j;
      if (i < NX) ((f32x4 *)xs[b])[i] = xr[j];
    }
  };
  load_x(t0);
  store_x(0);
  if (nt > 1) load_x(t0 + 1);
  __syncthreads();
  for (int k = 0; k < nt; k++) {
    const float v = avx_row_regs32<N32>(wv, xs[k & 1], L, true, 0.0f);
    if (k + 1 < nt) {
      store_x((k + 1) & 1);  // the buffer of token k - 1, which every wave finished before the last barrier
      if (k + 2 < nt) load_x(t0 + k + 2);
    }
    if (L == 0) {
      float *o = ps + (size_t)(t0 + k) * 4 * 64;
      o[g] = g < E ? v : 0.0f;
      o[64 + g] = 0.0f;
      o[128 + g] = 0.0f;
      o[192 + g] = 0.0f;
    }
    __syncthreads();
  }
}

// DECODE: one wave per token, x's limbs (pf_x_limbs), then the fast-exp softmax over all experts
// and top-k (route_select) on the scores of k_pf_scores_bf16.
__global__ void __launch_bounds__(256) k_pf_select_dec(const float *__restrict__ X, int T, int H, int E, int K,
                                                       const float *__restrict__ ps, int8_t *__restrict__ X0,
                                                       int8_t *__restrict__ X1, float *__restrict__ xsc,
                                                       float *__restrict__ xsum, int *__restrict__ idx,
                                                       float *__restrict__ w) {
  __shared__ float s_red[4][4][64];
  __shared__ int s_idx[4][64];
  __shared__ float s_w[4][64];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + wave;
  if (t >= T) return;  // no block-wide barriers below
#pragma unroll
  for (int r = 0; r < 4; r++) s_red[wave][r][lane] = ps[((size_t)t * 4 + r) * 64 + lane];
  pf_x_limbs(X, t, H, true, X0, X1, xsc, xsum, nullptr);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  route_select(E, K, DSH_ROUTE_DECODE, s_idx[wave], s_w[wave], s_red[wave]);
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
    int cv[16], c = 0;  // the waves' counts, all read before the prefix
#pragma unroll
    for (int v = 0; v < 16; v++) cv[v] = lane < E ? cnt[v][lane] : 0;
#pragma unroll
    for (int v = 0; v < 16; v++) c += cv[v];
    int incl = c;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int o = __shfl_up(incl, d);
      if (lane >= d) incl += o;
    }
    const int off = incl - c;
    int r = off;
#pragma unroll
    for (int v = 0; v < 16; v++) {
      run[v][lane] = r;
      r += cv[v];
    }
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
    // routed GEMM tiles of the two-launch path, expert by expert: n-tile major, the expert's chunks
    // adjacent, so the blocks that stream the same weight rows run side by side (item << 8 |
    // n-tile); the fused kernel takes its queues instead
    if (!Q.enable) {
      for (int nt = 0; nt < nt_gu; nt++)
        for (int j = 0; j < nch; j++) tiles_gu[ich * nt_gu + nt * nch + j] = ((ich + j) << 8) | nt;
      for (int nt = 0; nt < nt_dn; nt++)
        for (int j = 0; j < nch; j++) tiles_dn[ich * nt_dn + nt * nch + j] = ((ich + j) << 8) | nt;
    }
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
  // the pair positions (no barrier: they read only run and the cached entries, both complete)
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

// One block computes C[MB·16 A rows][4 waves x 64 weight rows] = A · B^T over K columns on the
// int8 MFMA (v_mfma_i32_16x16x64_i8): A = activations as two int8 limbs, B = the weights' stored
// codes. K runs in stages of PF_KS = 128 columns (one 128-byte line of each weight row), two
// 64-column MFMA slices each; pf_mainloop_i8 below gives the details.
#define PF_KS 128
#ifndef PF_OCC
#define PF_OCC 2  // GEMM blocks per CU the register budget is sized for
#endif

struct pf_smem {
  union {
    struct {
      int8_t A[2][2][PF_MT][PF_KS];  // [stage parity][low, high limb][row][column, swizzled]
    } q;                             // main loop
    float red[4][64][33];  // gate_up epilogue: h values per wave for the row sums
  } u;
  float hsum[4][2][32];  // Σh of the block's A rows (per wave, per 32-row half)
  float hmx[4][2][32];   // gate_up: max |h| of the block's A rows (per wave, per 32-row half)
  float xs[PF_MT];       // gate_up: Σx of the block's A rows (their tokens)
  float xsc[PF_MT];      // the A rows' limb scale 2^(e-15)
  short ek[PF_MT][PF_NT_MAX];  // down: exponent of each A row's n-tiles
  float hp[PF_MT][PF_NT_MAX];  // down: Σh of each A row's n-tiles (the gate_up partials)
  int erow[PF_MT];             // down: the A rows' common exponent (max over their n-tiles)
};

// Limb exponent of a set of values with max |v| = mx: 2^e > mx·(1 + 2^-7), so rint(v·2^(15-e)) + 128
// stays within 16 bits and both limbs within 8.
// A set whose max |v| is at most 2^-101 (zero, in practice: a tile of zero h) takes e = -100: its
// limbs are zero on that grid (or within 2^-116 of its values), so it neither raises the exponent
// a down row aligns its n-tiles to (which would cost the other tiles' low bits) nor overflows the
// factor 2^(15-e).
__device__ __forceinline__ int pf_limb_exp(float mx) {
  return mx > 0x1p-101f ? __builtin_amdgcn_frexp_expf(mx * 1.0078125f) : -100;
}

// Four values to limbs: fma(v, f, 1.5·2^23 + 128) rounds v·f to the nearest integer (ties to even)
// and leaves t = rint(v·f) + 128 in the low 16 bits of the result's bits (|t| < 2^22); two byte
// permutes gather the four low bytes (xor 0x80: (t & 255) - 128) and the four high bytes (t >> 8).
__device__ __forceinline__ void pf_limbs4(f32x4 v, float f, unsigned &lo, unsigned &hi) {
  const float magic = 12583040.0f;  // 1.5·2^23 + 128
  unsigned w[4];
#pragma unroll
  for (int b = 0; b < 4; b++) w[b] = __float_as_uint(__builtin_fmaf(v[b], f, magic));
  const unsigned p01 = __builtin_amdgcn_perm(w[1], w[0], 0x05040100u);  // t0 b0, t0 b1, t1 b0, t1 b1
  const unsigned p23 = __builtin_amdgcn_perm(w[3], w[2], 0x05040100u);
  lo = __builtin_amdgcn_perm(p23, p01, 0x06040200u) ^ 0x80808080u;
  hi = __builtin_amdgcn_perm(p23, p01, 0x07050301u);
}

// 16 values of one row (low limbs lo, high limbs hi) shifted right by d (1..31), rounded to nearest
// with ties to even (with d = 1 every odd X is a tie; rounding those one way would bias the sums):
// X = 256·hi + lo, X' = (X + 2^(d-1) - 1 + ((X >> d) & 1)) >> d, stored back as limbs of X' + 128
// (as pf_limbs4).
__device__ __forceinline__ void pf_align16(u32x4 &lo, u32x4 &hi, int d) {
  const int r = (1 << (d - 1)) - 1;
#pragma unroll
  for (int w = 0; w < 4; w++) {
    unsigned t[4];
#pragma unroll
    for (int b = 0; b < 4; b++) {
      const int x = __builtin_amdgcn_sbfe((int)hi[w], 8 * b, 8) * 256 + __builtin_amdgcn_sbfe((int)lo[w], 8 * b, 8);
      t[b] = (unsigned)(((x + r + ((x >> d) & 1)) >> d) + 128);
    }
    const unsigned p01 = __builtin_amdgcn_perm(t[1], t[0], 0x05040100u);
    const unsigned p23 = __builtin_amdgcn_perm(t[3], t[2], 0x05040100u);
    lo[w] = __builtin_amdgcn_perm(p23, p01, 0x06040200u) ^ 0x80808080u;
    hi[w] = __builtin_amdgcn_perm(p23, p01, 0x07050301u);
  }
}

// SwiGLU of the prefill GEMM: (g / (1 + fast_exp(-g))) * u (ds_kernels.c:1771) with the quotient
// from the hardware reciprocal refined by one Newton step. The reciprocal flushes a subnormal
// result and g * r can fall below the normal range, so a denominator above 2^126 (g < -87) is
// scaled, with g, by 2^-64, and |g| < 2^-96 is scaled by 2^64 and the quotient scaled back
// (exact while the quotient is normal); the quotient takes g's sign (the Newton step turns -0 into
// +0). k_pf_swiglu_check compares it with the correctly rounded division over every 32-bit g:
// equal for every finite g whose quotient is zero or a normal float, so it can differ only where
// |g| < 2.4e-38 (a gate value is an integer sum times two scales, never that small).
__device__ __forceinline__ float pf_swiglu(float g, float u) {
  // dsh_fast_expf(-g) without branches: the same bits for every input (0 below -88, 1e38 above
  // 88, 0 for NaN; the argument clamped so the integer conversion stays in range)
  const float x = -g, xc = __builtin_fminf(__builtin_fmaxf(x, -88.0f), 88.0f);
  float ex = __uint_as_float((uint32_t)(int32_t)__builtin_fmaf(12102203.0f, xc, 1064866805.0f));
  ex = x < -88.0f ? 0.0f : ex;
  ex = x > 88.0f ? 1e38f : ex;
  ex = x != x ? 0.0f : ex;
  const float d0 = 1.0f + ex;
  const bool big = d0 > 0x1p126f, tiny = __builtin_fabsf(g) < 0x1p-96f;
  const float d = big ? d0 * 0x1p-64f : d0;
  const float gs = g * (big ? 0x1p-64f : (tiny ? 0x1p64f : 1.0f));
  const float r = __builtin_amdgcn_rcpf(d);
  float q = gs * r;
  q = __builtin_fmaf(__builtin_fmaf(-d, q, gs), r, q);
  return __builtin_copysignf(tiny ? q * 0x1p-64f : q, g) * u;
}

// pf_swiglu(g, 1) against dsh_swiglu(g, 1) for the 2^30 bit patterns g = base + i of one launch
// (65536 blocks x 64 iterations x 256 threads; four launches cover every 32-bit g). counts[0] gets
// the finite g whose correctly rounded quotient is zero or normal and whose results differ in any
// bit, counts[1] the finite g with a subnormal quotient whose results differ. Two NaNs count as
// equal: for 87.9895 < g <= 88 the fast exp's affine value is negative and its signed conversion
// wraps to a NaN bit pattern, so both forms (and the reference) give NaN there.
__global__ void __launch_bounds__(256) k_pf_swiglu_check(uint32_t base, unsigned long long *counts) {
  unsigned long long n0 = 0, n1 = 0;
  for (int it = 0; it < 64; it++) {
    const uint32_t bits = base + ((uint32_t)(blockIdx.x * 64 + it) << 8) + threadIdx.x;
    const float g = __uint_as_float(bits);
    const float a = dsh_swiglu(g, 1.0f), b = pf_swiglu(g, 1.0f);
    const bool differ = __builtin_isfinite(g) && !(a != a && b != b) && __float_as_uint(a) != __float_as_uint(b);
    const bool sub = a != 0.0f && __builtin_fabsf(a) < 0x1p-126f;
    n0 += __popcll(__ballot(differ && !sub));
    n1 += __popcll(__ballot(differ && sub));
  }
  if ((threadIdx.x & 63) == 0) {
    if (n0) atomicAdd(&counts[0], n0);
    if (n1) atomicAdd(&counts[1], n1);
  }
}

hipError_t dsh_launch_pf_swiglu_check(unsigned long long *counts, hipStream_t s) {
  hipError_t e = hipMemsetAsync(counts, 0, 2 * sizeof(unsigned long long), s);
  for (uint32_t ch = 0; ch < 4 && e == hipSuccess; ch++) {
    k_pf_swiglu_check<<<65536, 256, 0, s>>>(ch << 30, counts);
    e = hipGetLastError();
  }
  return e;
}

// 16-byte chunk c of LDS row r sits at chunk c ^ pf_swz(r): 16 consecutive rows map one chunk to 16
// distinct bank groups, and two consecutive rows fill 256 contiguous bytes
__device__ __forceinline__ int pf_swz(int r) { return (r ^ (r >> 3)) & 7; }

// The int8 main loop (both projections). Per 128-column stage:
// - weights go from HBM straight into the MFMA's B operand registers: for n-block j (16 weight
//   rows: j = 0, 1 from brow0, 2, 3 from brow1) and slice s, lane l loads bytes 64s + 16(l/16) .. +15
//   of the stage in row 16j + l%16 (each load instruction reads 16 rows x 64 contiguous bytes); a
//   slice's registers are reloaded with the next stage's slice as soon as its MFMAs are issued;
// - A: the block's rows are copied (8 adjacent lanes per row's 128 bytes, one stage ahead in
//   registers) into a double-buffered LDS tile with 128-byte rows whose 16-byte chunks are
//   XOR-swizzled by pf_swz(row); lane l reads chunk 4s + l/16 of row 16mb + l%16, the same columns
//   as its weight bytes, so each MFMA adds the exact products over the slice (A and B share the
//   order of k inside the instruction, which leaves the sum unchanged);
// - one barrier per stage.
// acc[mb][j][l]: A rows 16mb .. +15, n-block j, limb l (low, high), exact int32 sums; lane l,
// register i holds A row 16mb + 4(l/16) + i, weight row 16j + l%16. A rows past the item's count
// repeat a valid row; their results are never stored.
// A is two int8 limb arrays, A0 low and A1 high (gate_up: x at one exponent per row; down: h at
// one exponent per row and 128-column stage). ALIGN (down): before a stage's A values go to LDS,
// each is brought to its row's common exponent (pf_align16 with d = erow - ek of the row's stage;
// sm.ek, sm.erow; trow: the table rows of this thread's two A rows).
// pre() runs once the first stage's loads are issued (down: building the alignment table), so its
// waits leave them in flight.
template <int MB, bool ALIGN, typename Pre>
__device__ __forceinline__ void pf_mainloop_i8(const int8_t *A0, const int8_t *A1, const size_t *arow,
                                               const int *trow, int K, const int8_t *brow0, const int8_t *brow1,
                                               i32x4 (&acc)[MB][4][2], pf_smem &sm, Pre &&pre) {
  const int lane = threadIdx.x & 63, r16 = lane & 15, kg = lane >> 4;
  const int ar = threadIdx.x >> 3, ac = threadIdx.x & 7;  // A copy: rows ar and ar + 32, chunk ac
  const int nk = K / PF_KS;
#pragma unroll
  for (int mb = 0; mb < MB; mb++)
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int l = 0; l < 2; l++) acc[mb][j][l] = i32x4{0, 0, 0, 0};
  int zero = 0;
  asm volatile("" : "+v"(zero) : "v"((int)arow[0]), "v"((int)arow[1]));
  const size_t K16 = (size_t)16 * K;
  const int8_t *p0 = brow0 + zero + (size_t)r16 * K + 16 * kg;
  const int8_t *p1 = brow1 + zero + (size_t)r16 * K + 16 * kg;
  const int aw0 = 16 * (ac ^ pf_swz(ar)), aw1 = 16 * (ac ^ pf_swz(ar + 32));
  i32x4 bR[2][4];  // [slice][n-block] of the stage
  u32x4 aR[4];     // X0 rows ar, ar+32, X1 rows ar, ar+32
  auto load_b = [&](int sl, int k) {
#pragma unroll
    for (int j = 0; j < 4; j++)
      bR[sl][j] = *(const i32x4 *)((j < 2 ? p0 : p1) + (j & 1) * K16 + (size_t)k * PF_KS + 64 * sl);
  };
  auto load_a = [&](int k) {
    const size_t o = (size_t)k * PF_KS + 16 * ac;
    aR[0] = *(const u32x4 *)(A0 + arow[0] + o);
    aR[1] = *(const u32x4 *)(A0 + arow[1] + o);
    aR[2] = *(const u32x4 *)(A1 + arow[0] + o);
    aR[3] = *(const u32x4 *)(A1 + arow[1] + o);
  };
  auto store_a = [&](int a, int k) {
    if (ALIGN) {
#pragma unroll
      for (int c = 0; c < 2; c++) {
        const int d = min(sm.erow[trow[c]] - (int)sm.ek[trow[c]][k], 31);
        if (d > 0) pf_align16(aR[c], aR[2 + c], d);
      }
    }
    *(u32x4 *)&sm.u.q.A[a][0][ar][aw0] = aR[0];
    *(u32x4 *)&sm.u.q.A[a][0][ar + 32][aw1] = aR[1];
    *(u32x4 *)&sm.u.q.A[a][1][ar][aw0] = aR[2];
    *(u32x4 *)&sm.u.q.A[a][1][ar + 32][aw1] = aR[3];
  };
  // the same issue order as in the loop (A, then slice 0, then slice 1), so the wait counts the
  // compiler derives at the loop head leave the weight loads in flight
  load_a(0);
  asm volatile("" ::: "memory");
  load_b(0, 0);
  asm volatile("" ::: "memory");
  load_b(1, 0);
  asm volatile("" ::: "memory");
  pre();
#pragma unroll 1
  for (int k = 0; k < nk; k++) {
    const int a = k & 1, kn = min(k + 1, nk - 1);
    store_a(a, k);
    load_a(kn);
    asm volatile("" ::: "memory");
    __syncthreads();
#pragma unroll
    for (int sl = 0; sl < 2; sl++) {
      i32x4 x0[MB], x1[MB];
#pragma unroll
      for (int mb = 0; mb < MB; mb++) {
        const int m = 16 * mb + r16, c = 16 * ((4 * sl + kg) ^ pf_swz(m));
        x0[mb] = *(const i32x4 *)&sm.u.q.A[a][0][m][c];
        x1[mb] = *(const i32x4 *)&sm.u.q.A[a][1][m][c];
      }
#pragma unroll
      for (int mb = 0; mb < MB; mb++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
          acc[mb][j][0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(x0[mb], bR[sl][j], acc[mb][j][0], 0, 0, 0);
          acc[mb][j][1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(x1[mb], bR[sl][j], acc[mb][j][1], 0, 0, 0);
        }
      load_b(sl, kn);
      asm volatile("" ::: "memory");
    }
  }
}

// gate_up: block = (work item, n-tile): the item's A rows (tokens) x 128 intermediate units; wave w
// owns units i0 + 32w .. +31: n-blocks 0, 1 = their gate rows, 2, 3 = their up rows, so each SwiGLU
// pair sits in the same lane and register (n-blocks h and 2 + h).
template <bool SHARED, int MB>
__device__ __forceinline__ void gate_up_tile(const dsh_layer_t &L, const pf_item &it, int nt, const int8_t *X0,
                                             const int8_t *X1, const float *xsc, const float *xsum,
                                             const int *pair_tok, int bf16sim, int8_t *Hq0, int8_t *Hq1,
                                             float *hpart, float *hmaxp, pf_smem &sm) {
  const int H = L.H;
  const int Iseg = SHARED ? L.SI : L.I, ntK = Iseg / PF_GU_N;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, r16 = lane & 15, kg = lane >> 4;
  const int u0 = nt * PF_GU_N + wave * 32;
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
  // the rows' Σx and limb scales for the epilogue, staged in LDS (visible after the main loop's
  // first barrier)
  if ((threadIdx.x & 7) == 0) {
    const float x0 = xsum[tok[0]], x1 = xsum[tok[1]], c0 = xsc[tok[0]], c1 = xsc[tok[1]];
    sm.xs[threadIdx.x >> 3] = x0;
    sm.xs[(threadIdx.x >> 3) + 32] = x1;
    sm.xsc[threadIdx.x >> 3] = c0;
    sm.xsc[(threadIdx.x >> 3) + 32] = c1;
  }
  // the lane's units' scales and offsets (units u0 + 16h + l%16), loaded before the main loop so
  // the epilogue does not wait for them
  float2 sog[2], sou[2];
#pragma unroll
  for (int h = 0; h < 2; h++) {
    const int unit = u0 + 16 * h + r16;
    sog[h] = ((const float2 *)wso)[unit];
    sou[h] = ((const float2 *)wso)[Iseg + unit];
  }
  i32x4 acc[MB][4][2];
  pf_mainloop_i8<MB, false>(X0, X1, arow, nullptr, H, wq + (size_t)u0 * H, wq + (size_t)(Iseg + u0) * H, acc, sm,
                            [] {});
  // signed codes: offset + 128·scale multiplies Σa
#pragma unroll
  for (int h = 0; h < 2; h++) {
    sog[h].y = __builtin_fmaf(128.0f, sog[h].x, sog[h].y);
    sou[h].y = __builtin_fmaf(128.0f, sou[h].x, sou[h].y);
  }
  const size_t rbase = SHARED ? (size_t)it.m0 : (size_t)(it.pos0 + it.m0);
  // The tile's h values go to LDS (per wave: 64 rows x its 32 units); each lane sums a row (Σh over
  // the block's 128 units, for the down epilogue's offset term) and takes its max |h|; the rows'
  // maxima over the block's 128 units give each row's limb exponent for this n-tile, from which the
  // lanes store 8-unit runs of both limbs.
  float(*red)[64][33] = sm.u.red;
  __syncthreads();  // every wave is done with the main loop's tiles
  // rows past the item's count repeat row 0 (valid values, never stored); the bf16 simulation is
  // one branch around the loop
  auto h_out = [&](auto sim) {
#pragma unroll
    for (int mb = 0; mb < MB; mb++)
#pragma unroll
      for (int h = 0; h < 2; h++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int m = 16 * mb + 4 * kg + i;
          const float xs = sm.xs[m], sc = sm.xsc[m];
          // Σ q·x = 2^(e-15)·(256·Σ q·X1 + Σ q·X0)
          const float dg = sc * __builtin_fmaf(256.0f, (float)acc[mb][h][1][i], (float)acc[mb][h][0][i]);
          const float du = sc * __builtin_fmaf(256.0f, (float)acc[mb][2 + h][1][i], (float)acc[mb][2 + h][0][i]);
          float g = __builtin_fmaf(sog[h].x, dg, sog[h].y * xs);
          float up = __builtin_fmaf(sou[h].x, du, sou[h].y * xs);
          if (decltype(sim)::value) {
            g = dsh_bf16_round_half_up(g);
            up = dsh_bf16_round_half_up(up);
          }
          float hv = pf_swiglu(g, up);
          if (decltype(sim)::value) hv = dsh_bf16_round_half_up(hv);
          red[wave][m][16 * h + r16] = hv;
        }
  };
  if (bf16sim)
    h_out(std::true_type{});
  else
    h_out(std::false_type{});
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float part = 0.0f, pmax = 0.0f;  // lane = row: its sum (in unit order) and max |h| over the wave's 32 units
  if (lane < 16 * MB) {
#pragma unroll 8
    for (int u = 0; u < 32; u++) {
      const float hv = red[wave][lane][u];
      part += hv;
      pmax = fmaxf(pmax, fabsf(hv));
    }
  }
  sm.hsum[wave][lane >> 5][lane & 31] = part;
  sm.hmx[wave][lane >> 5][lane & 31] = pmax;
  __syncthreads();
  {  // stores: lane → rows (lane / 4) + 16k, units 8·(lane % 4) .. +7 of the wave's 32, as limbs
    const int g8 = 8 * (lane & 3);
#pragma unroll
    for (int k = 0; k < MB; k++) {
      const int m = (lane >> 2) + 16 * k;
      if (m >= it.mcnt) continue;
      const int a = m >> 5, b = m & 31;
      const float mx = fmaxf(fmaxf(sm.hmx[0][a][b], sm.hmx[1][a][b]), fmaxf(sm.hmx[2][a][b], sm.hmx[3][a][b]));
      const float f = __builtin_ldexpf(1.0f, 15 - pf_limb_exp(mx));
      f32x4 v0, v1;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        v0[i] = red[wave][m][g8 + i];
        v1[i] = red[wave][m][g8 + 4 + i];
      }
      unsigned l0, h0, l1, h1;
      pf_limbs4(v0, f, l0, h0);
      pf_limbs4(v1, f, l1, h1);
      const size_t o = (rbase + m) * Iseg + u0 + g8;
      *(u32x2 *)(Hq0 + o) = u32x2{l0, l1};
      *(u32x2 *)(Hq1 + o) = u32x2{h0, h1};
    }
  }
  if (threadIdx.x < it.mcnt) {
    const int m = threadIdx.x, a = m >> 5, b = m & 31;
    const float tot = ((sm.hsum[0][a][b] + sm.hsum[1][a][b]) + sm.hsum[2][a][b]) + sm.hsum[3][a][b];
    const float mx = fmaxf(fmaxf(sm.hmx[0][a][b], sm.hmx[1][a][b]), fmaxf(sm.hmx[2][a][b], sm.hmx[3][a][b]));
    hpart[(rbase + m) * ntK + nt] = tot;
    hmaxp[(rbase + m) * ntK + nt] = mx;
  }
}

template <bool SHARED>
__device__ __forceinline__ void gate_up_dispatch(const dsh_layer_t &L, const pf_item &it, int nt, const int8_t *X0,
                                                 const int8_t *X1, const float *xsc, const float *xsum,
                                                 const int *pair_tok, int bf16sim, int8_t *Hq0, int8_t *Hq1,
                                                 float *hpart, float *hmaxp, pf_smem &sm) {
  if (it.mcnt <= 32)
    gate_up_tile<SHARED, 2>(L, it, nt, X0, X1, xsc, xsum, pair_tok, bf16sim, Hq0, Hq1, hpart, hmaxp, sm);
  else
    gate_up_tile<SHARED, 4>(L, it, nt, X0, X1, xsc, xsum, pair_tok, bf16sim, Hq0, Hq1, hpart, hmaxp, sm);
}

__global__ void __launch_bounds__(256, PF_OCC) k_pf_gate_up(dsh_layer_t L, const pf_item *__restrict__ items,
                                                       const int *__restrict__ counts, const int8_t *X0,
                                                       const int8_t *X1, const float *__restrict__ xsc,
                                                       const float *__restrict__ xsum,
                                                       const int *__restrict__ pair_tok, int bf16sim,
                                                       pf_hq hq, float *__restrict__ hpr, float *__restrict__ hps,
                                                       float *__restrict__ hmr, float *__restrict__ hms,
                                                       const int *__restrict__ tiles) {
  __shared__ __attribute__((aligned(16))) pf_smem sm;
  int item, nt;
  if (!pf_tile(counts, tiles, L.SI / PF_GU_N, L.I / PF_GU_N, item, nt)) return;
  const pf_item it = items[item];
  if (it.seg == L.E)
    gate_up_dispatch<true>(L, it, nt, X0, X1, xsc, xsum, pair_tok, bf16sim, hq.s0, hq.s1, hps, hms, sm);
  else
    gate_up_dispatch<false>(L, it, nt, X0, X1, xsc, xsum, pair_tok, bf16sim, hq.r0, hq.r1, hpr, hmr, sm);
}

// down: block = (work item, n-tile): the item's A rows (h of its pairs, or of tokens for the shared
// expert, as limbs) x 256 output rows; wave w owns rows n0 + 64w .. +63 as four 16-row n-blocks. Each A
// row's exponent is the largest of its n-tiles' (from the max |h| per (row, n-tile) the gate_up
// epilogues wrote; read at L2); the main loop aligns every stage to it. Σh of each A row is the sum,
// in n-tile order, of the per-n-tile row sums the gate_up epilogue wrote.
template <bool SHARED, int MB>
__device__ __forceinline__ void down_tile(const dsh_layer_t &L, const pf_item &it, int nt, const int8_t *Hq0,
                                          const int8_t *Hq1, const float *hpart, const float *hmaxp, float *Y,
                                          pf_smem &sm) {
  const int H = L.H;
  const int Kd = SHARED ? L.SI : L.I, ntK = Kd / PF_GU_N;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, r16 = lane & 15, kg = lane >> 4;
  const int8_t *wq = SHARED ? L.sdn_q : L.dn_q + (size_t)it.seg * H * L.I;
  const float *wso = SHARED ? L.sdn_so : L.dn_so + (size_t)it.seg * H * 2;
  const int nw = nt * PF_DN_N + wave * 64;
  const size_t rbase = SHARED ? (size_t)it.m0 : (size_t)(it.pos0 + it.m0);
  // The gate_up partials of the A rows (max |h| and Σh per row and n-tile; at most PF_MT x
  // PF_NT_MAX = 4 per thread), read at L2 and all issued at once, then the output rows' scales
  // and offsets; all are in flight while the main loop issues its first stage.
  const int ntot = it.mcnt * ntK;
  float mxv[4], hpv[4];
#pragma unroll
  for (int c = 0; c < 4; c++) {
    const int i = threadIdx.x + 256 * c;
    mxv[c] = 0.0f;
    hpv[c] = 0.0f;
    if (i < ntot) {
      mxv[c] = __hip_atomic_load(hmaxp + rbase * ntK + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      hpv[c] = __hip_atomic_load(hpart + rbase * ntK + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  float2 so[4];
#pragma unroll
  for (int j = 0; j < 4; j++) so[j] = ((const float2 *)wso)[nw + 16 * j + r16];
  if (threadIdx.x < PF_MT) sm.erow[threadIdx.x] = -1024;
  // each A row's exponent (the largest of its n-tiles'), its limb scale and its Σh (n-tile order)
  auto table = [&] {
    __syncthreads();
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const int i = threadIdx.x + 256 * c;
      if (i < ntot) {
        const int r = i / ntK, k = i - r * ntK, e = pf_limb_exp(mxv[c]);
        sm.ek[r][k] = (short)e;
        sm.hp[r][k] = hpv[c];
        atomicMax(&sm.erow[r], e);
      }
    }
    __syncthreads();
    if (threadIdx.x < it.mcnt) {
      const int r = threadIdx.x;
      sm.xsc[r] = __builtin_ldexpf(1.0f, sm.erow[r] - 15);
      float hs = 0.0f;
      for (int k = 0; k < ntK; k++) hs += sm.hp[r][k];
      sm.hsum[0][r >> 5][r & 31] = hs;
    }
  };
  size_t arow[2];
  int trow[2];
#pragma unroll
  for (int c = 0; c < 2; c++) {
    const int r = (threadIdx.x >> 3) + 32 * c;
    trow[c] = r < it.mcnt ? r : 0;
    arow[c] = (rbase + trow[c]) * Kd;
  }
  i32x4 acc[MB][4][2];
  pf_mainloop_i8<MB, true>(Hq0, Hq1, arow, trow, Kd, wq + (size_t)nw * Kd, wq + (size_t)(nw + 32) * Kd, acc, sm,
                           table);
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int n = nw + 16 * j + r16;
    so[j].y = __builtin_fmaf(128.0f, so[j].x, so[j].y);  // signed codes: offset + 128·scale multiplies Σh
#pragma unroll
    for (int mb = 0; mb < MB; mb++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int m = 16 * mb + 4 * kg + i;
        if (m >= it.mcnt) continue;
        const float hs = sm.hsum[0][m >> 5][m & 31];
        // Σ q·h = 2^(erow-15)·(256·Σ q·H1 + Σ q·H0)
        const float dot = sm.xsc[m] * __builtin_fmaf(256.0f, (float)acc[mb][j][1][i], (float)acc[mb][j][0][i]);
        Y[(rbase + m) * H + n] = __builtin_fmaf(so[j].x, dot, so[j].y * hs);
      }
  }
}

template <bool SHARED>
__device__ __forceinline__ void down_dispatch(const dsh_layer_t &L, const pf_item &it, int nt, const int8_t *Hq0,
                                              const int8_t *Hq1, const float *hpart, const float *hmaxp, float *Y,
                                              pf_smem &sm) {
  if (it.mcnt <= 32)
    down_tile<SHARED, 2>(L, it, nt, Hq0, Hq1, hpart, hmaxp, Y, sm);
  else
    down_tile<SHARED, 4>(L, it, nt, Hq0, Hq1, hpart, hmaxp, Y, sm);
}

__global__ void __launch_bounds__(256, PF_OCC) k_pf_down(dsh_layer_t L, const pf_item *__restrict__ items,
                                                    const int *__restrict__ counts, pf_hq hq,
                                                    const float *__restrict__ hpr, const float *__restrict__ hps,
                                                    const float *__restrict__ hmr, const float *__restrict__ hms,
                                                    float *__restrict__ Y, float *__restrict__ Ysh,
                                                    const int *__restrict__ tiles) {
  __shared__ __attribute__((aligned(16))) pf_smem sm;
  int item, nt;
  if (!pf_tile(counts, tiles, L.H / PF_DN_N, L.H / PF_DN_N, item, nt)) return;
  const pf_item it = items[item];
  if (it.seg == L.E)
    down_dispatch<true>(L, it, nt, hq.s0, hq.s1, hps, hms, Ysh, sm);
  else
    down_dispatch<false>(L, it, nt, hq.r0, hq.r1, hpr, hmr, Y, sm);
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
// counter with an L2 atomic; the down block reads the counter at L2, and the h limbs it then loads
// were written by this XCD (each 128-byte line by one block) and never read here before (the
// per-row partials, which share lines across items, are read with L2 atomics). Claim counters and
// item counters are zeroed by the plan kernel.
#define PF_PROBE 4096  // blocks of the XCD placement check
__global__ void __launch_bounds__(256, PF_OCC) k_pf_moe(dsh_layer_t L, const pf_item *__restrict__ items,
                                                    pf_queues Q, const int8_t *X0, const int8_t *X1,
                                                    const float *__restrict__ xsc, const float *__restrict__ xsum,
                                                    const int *__restrict__ pair_tok,
                                                    int bf16sim, pf_hq hq, float *hpr, float *hps, float *hmr,
                                                    float *hms, float *__restrict__ Y,
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
      gate_up_dispatch<true>(L, it, nt, X0, X1, xsc, xsum, pair_tok, bf16sim, hq.s0, hq.s1, hps, hms, sm);
    else
      gate_up_dispatch<false>(L, it, nt, X0, X1, xsc, xsum, pair_tok, bf16sim, hq.r0, hq.r1, hpr, hmr, sm);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's limb and partial stores are in L2
    __syncthreads();
    if (threadIdx.x == 0) __hip_atomic_fetch_add(Q.gu_done + item, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    if (threadIdx.x == 0) {
      const int need = it.seg == L.E ? L.SI / PF_GU_N : L.I / PF_GU_N;
      int spins = 0;
      bool gave_up = Q.spin_max < 0;
      while (!gave_up && __hip_atomic_load(Q.gu_done + item, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < need) {
        if (++spins > Q.spin_max) gave_up = true;
        else __builtin_amdgcn_s_sleep(2);
      }
      if (gave_up) {  // the tile computes on h as it is; the call's output is reported as not valid
        __hip_atomic_store(Q.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (Q.derr) __hip_atomic_store(Q.derr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      }
    }
    __syncthreads();
    if (it.seg == L.E)
      down_dispatch<true>(L, it, nt, hq.s0, hq.s1, hps, hms, Ysh, sm);
    else
      down_dispatch<false>(L, it, nt, hq.r0, hq.r1, hpr, hmr, Y, sm);
  }
}

// XCC id of each block, to check that a grid's blocks cover all PF_NQ XCDs before the fused kernel
// is used.
__global__ void __launch_bounds__(64) k_pf_xcc_probe(int *__restrict__ out) {
  unsigned xcc;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
  if (threadIdx.x == 0) out[blockIdx.x] = (int)xcc;
}

// The same for a 512-thread grid (the one-kernel decode layers' block size).
__global__ void __launch_bounds__(512) k_pf_xcc_probe512(int *__restrict__ out) {
  unsigned xcc;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
  if (threadIdx.x == 0) out[blockIdx.x] = (int)xcc;
}

// ---------------------------------------------------------------------------------- combine
#define PF_CB 8  // routed slots whose rows a combine thread loads before adding them
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
  // a thread's (up to) two 4-float columns (H <= 2048), every row's load of a group of PF_CB slots
  // issued before the adds, which keep the slot order; clamped duplicates are loaded, not stored
  const int n = s_n, nc = H / 4;
  int cc[2];
  f32x4 routed[2], sh[2], xr[2];
#pragma unroll
  for (int h = 0; h < 2; h++) {
    cc[h] = min((int)threadIdx.x + 256 * h, nc - 1);
    routed[h] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    sh[h] = ((const f32x4 *)(Ysh + (size_t)t * H))[cc[h]];
    xr[h] = residual ? ((const f32x4 *)(X + (size_t)t * H))[cc[h]] : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }
  for (int j0 = 0; j0 < n; j0 += PF_CB) {
    f32x4 v[2][PF_CB];
#pragma unroll
    for (int j = 0; j < PF_CB; j++) {
      const float *row = Y + (size_t)s_pos[min(j0 + j, n - 1)] * H;
#pragma unroll
      for (int h = 0; h < 2; h++) v[h][j] = ((const f32x4 *)row)[cc[h]];
    }
    // every load issued before the adds (their early exit would otherwise pull the loads in)
    asm volatile("" : "+v"(v[0][0]), "+v"(v[0][1]), "+v"(v[0][2]), "+v"(v[0][3]), "+v"(v[0][4]), "+v"(v[0][5]),
                 "+v"(v[0][6]), "+v"(v[0][7]), "+v"(v[1][0]), "+v"(v[1][1]), "+v"(v[1][2]), "+v"(v[1][3]),
                 "+v"(v[1][4]), "+v"(v[1][5]), "+v"(v[1][6]), "+v"(v[1][7]));
#pragma unroll
    for (int j = 0; j < PF_CB; j++) {
      if (j0 + j >= n) break;
      const float wj = s_w[j0 + j];
#pragma unroll
      for (int h = 0; h < 2; h++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          float vv = v[h][j][i];
          if (bf16sim) vv = dsh_bf16_round_half_up(vv);
          routed[h][i] = __builtin_fmaf(wj, vv, routed[h][i]);
        }
    }
  }
#pragma unroll
  for (int h = 0; h < 2; h++) {
    if ((int)threadIdx.x + 256 * h >= nc) break;
    f32x4 o;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      float s2 = sh[h][i];
      if (bf16sim) s2 = dsh_bf16_round_half_up(s2);
      o[i] = routed[h][i] + s2;
      if (residual) o[i] = xr[h][i] + o[i];
    }
    ((f32x4 *)(out + (size_t)t * H))[cc[h]] = o;
  }
}

// ---------------------------------------------------------------------------------- launchers
namespace {
struct pf_ws {
  int8_t *X0, *X1;  // x as two int8 limbs [T][H]
  float *xsc;       // their scale per token
  float *xsum;
  int *idx;
  float *w;
  int *seg_off, *counts;
  pf_item *items;
  int *pair_tok, *pos_of;
  pf_hq hq;         // SwiGLU outputs h as int8 limbs: routed [TK][I], shared [T][SI]
  float *Y, *Ysh;
  float *ps;        // [T][4][64] router scores (DECODE: the full score in row 0, rows 1-3 zero)
  float *hpr, *hps; // Σh partials per (row, gate_up n-tile): routed [TK][I/128], shared [T][SI/128]
  float *hmr, *hms; // max |h| per (row, gate_up n-tile), same layout
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
  TAKE(X0, int8_t, T * H);
  TAKE(X1, int8_t, T * H);
  TAKE(xsc, float, T);
  TAKE(xsum, float, T);
  TAKE(idx, int, TK);
  TAKE(w, float, TK);
  TAKE(seg_off, int, E + 1);
  TAKE(counts, int, 2);
  TAKE(items, pf_item, pf_max_routed_items(L, T) + pf_shared_items(T));
  TAKE(pair_tok, int, TK);
  TAKE(pos_of, int, TK);
  TAKE(hq.r0, int8_t, TK * I);
  TAKE(hq.r1, int8_t, TK * I);
  TAKE(hq.s0, int8_t, T * SI);
  TAKE(hq.s1, int8_t, T * SI);
  TAKE(Y, float, TK * H);
  TAKE(Ysh, float, T * H);
  TAKE(ps, float, (size_t)T * 4 * 64);
  TAKE(hpr, float, TK * (I / PF_GU_N));
  TAKE(hps, float, (size_t)T * (SI / PF_GU_N));
  TAKE(hmr, float, TK * (I / PF_GU_N));
  TAKE(hms, float, (size_t)T * (SI / PF_GU_N));
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
  if (L->H > 256 * PF_SEL_U) return 0;  // a wave holds a token's x row (pf_x_limbs, k_pf_route_cfg's LDS)
  if (L->I > PF_KS * PF_NT_MAX || L->SI > PF_KS * PF_NT_MAX) return 0;  // down: exponent table per row
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

// 1 when a 512-thread grid's blocks are dealt to the 8 XCDs in turn (blocks 8 r .. 8 r + 7 on 8
// different XCDs), as the one-kernel layers' verifier parts assume (they check it again on every
// launch); probed once (outside stream capture).
static int g_xcd_rr = -1;

int dsh_xcd_even(void) {
  if (g_pf_auto < 0 && dsh_pf_init(-2) != hipSuccess) return 0;
  if (g_xcd_rr < 0) {
    const int n = 256;
    int *d = NULL;
    int h[256];
    g_xcd_rr = 0;
    if (hipMalloc(&d, sizeof(int) * n) == hipSuccess) {
      k_pf_xcc_probe512<<<n, 512>>>(d);
      if (hipGetLastError() == hipSuccess && hipMemcpy(h, d, sizeof(int) * n, hipMemcpyDeviceToHost) == hipSuccess) {
        g_xcd_rr = 1;
        for (int r = 0; r < n / PF_NQ; r++) {
          unsigned m = 0;
          for (int i = 0; i < PF_NQ; i++) m |= 1u << (h[PF_NQ * r + i] & 31);
          g_xcd_rr &= m == (1u << PF_NQ) - 1u;
        }
      }
      (void)hipFree(d);
    }
  }
  return g_pf_auto == 1 && g_xcd_rr == 1;
}

int dsh_pf_wait_error(const void *ws, const dsh_layer_t *L, int T) {
  pf_ws w;
  pf_carve(L, T, (void *)ws, &w);
  int v = 0;
  if (hipMemcpy(&v, w.err, sizeof v, hipMemcpyDeviceToHost) != hipSuccess) return -1;
  return v;
}

hipError_t dsh_launch_prefill(const dsh_layer_t *L, const float *X, int T, int route_mode, int nthreads, int residual,
                              int bf16sim, float *out, void *ws, int *idx_out, float *w_out, int *derr, int spin_max,
                              hipStream_t s) {
  if (T <= 0 || !dsh_pf_supported(L)) return hipErrorInvalidValue;
  if (route_mode == DSH_ROUTE_CFG ? !L->router_f32_t : !L->router_bf16) return hipErrorInvalidValue;
  pf_ws w;
  pf_carve(L, T, ws, &w);
  const int H = L->H, K = L->K, E = L->E;
  if (route_mode == DSH_ROUTE_CFG) {
    if (E == 64)
      k_pf_route_cfg<true><<<(T + 3) / 4, 256, 0, s>>>(L->router_f32_t, X, T, H, E, K, w.X0, w.X1, w.xsc, w.xsum,
                                                        w.idx, w.w);
    else
      k_pf_route_cfg<false><<<(T + 3) / 4, 256, 0, s>>>(L->router_f32_t, X, T, H, E, K, w.X0, w.X1, w.xsc, w.xsum,
                                                         w.idx, w.w);
  } else {
    // every row on a group path: the chunks of the reference's threads all have an even length
    const int chunk = dsh_chunk_len(E, nthreads);
    bool grouped = true;
    for (int s0 = 0; s0 < E; s0 += chunk) grouped = grouped && (min(chunk, E - s0) % 2 == 0);
    const int tpb = (T + 255) / 256, nbr = (T + tpb - 1) / tpb;
#define PFR(N)                                                                                                      \
  case N:                                                                                                           \
    k_pf_scores_bf16r<N><<<nbr, 256, 0, s>>>(L->router_bf16, X, T, E, tpb, w.ps);                                 \
    break;
    if (grouped && H % 256 == 0 && H <= 1280) {
      switch (H / 32) { PFR(8) PFR(16) PFR(24) PFR(32) PFR(40) }
    } else {
      k_pf_scores_bf16<<<(T + PF_TB - 1) / PF_TB, 256, (size_t)PF_TB * H * sizeof(float), s>>>(
          L->router_bf16, X, T, H, E, nthreads, w.ps);
    }
#undef PFR
    k_pf_select_dec<<<(T + 3) / 4, 256, 0, s>>>(X, T, H, E, K, w.ps, w.X0, w.X1, w.xsc, w.xsum, w.idx, w.w);
  }
  const int n_items_max = pf_max_routed_items(L, T) + pf_shared_items(T);
  const bool fused = g_pf_fused == 1 && n_items_max < (1 << 22);
  pf_queues Q{w.qtiles, w.qcount, w.qnext, w.gu_done, w.err, derr, spin_max, (int)pf_queue_cap(L, T),
              L->I / PF_GU_N, L->SI / PF_GU_N,
              H / PF_DN_N, H / PF_KS, L->I / PF_KS, L->SI / PF_KS, fused ? 1 : 0};
  k_pf_plan<<<1, 1024, 0, s>>>(w.idx, T, K, E, L->I / PF_GU_N, H / PF_DN_N, w.seg_off, w.items, w.counts,
                               w.tiles_gu, w.tiles_dn, w.pair_tok, w.pos_of, Q);
  if (fused) {
    // blocks per XCD >= tiles of the longest queue (at most ceil(items / PF_NQ) items)
    const int per_item = max(L->I / PF_GU_N, L->SI / PF_GU_N) + H / PF_DN_N;
    const int blocks = PF_NQ * ((n_items_max + PF_NQ - 1) / PF_NQ) * per_item;
    k_pf_moe<<<blocks, 256, 0, s>>>(*L, w.items, Q, w.X0, w.X1, w.xsc, w.xsum, w.pair_tok, bf16sim, w.hq, w.hpr,
                                    w.hps, w.hmr, w.hms, w.Y, w.Ysh);
  } else {
    k_pf_gate_up<<<pf_grid(L, T, L->SI / PF_GU_N, L->I / PF_GU_N), 256, 0, s>>>(
        *L, w.items, w.counts, w.X0, w.X1, w.xsc, w.xsum, w.pair_tok, bf16sim, w.hq, w.hpr, w.hps, w.hmr, w.hms,
        w.tiles_gu);
    k_pf_down<<<pf_grid(L, T, H / PF_DN_N, H / PF_DN_N), 256, 0, s>>>(*L, w.items, w.counts, w.hq, w.hpr, w.hps,
                                                                       w.hmr, w.hms, w.Y, w.Ysh, w.tiles_dn);
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
