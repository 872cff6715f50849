// Weight-streaming bf16 GEMM for decode-sized M on gfx950 (MI355X).
//
//   Y[M, N] = X[M, K] . W[N, K]^T      (nn.Linear without the transpose copy)
//
// Design (HBM-bound: every weight byte is read exactly once per call):
// * W is pre-packed once into MFMA-native tiles: tile (nb, kb) holds rows
//   [16nb, 16nb+16) x k [32kb, 32kb+32) as 64 lanes x 8 bf16, in the order the
//   v_mfma_f32_16x16x32_bf16 A operand wants it. A wave's load of one tile is
//   one fully contiguous 1 KiB request (16 B per lane). Rows are padded to 64.
// * A workgroup owns NSUB 16-row tiles of N and the whole K; its KS waves split
//   K (k-block pairs dealt round-robin) and are summed through LDS in wave order. Each
//   wave streams its NSUB weight tiles against one X fragment per k-block, so
//   activation traffic from L2 is CT/NSUB of the weight traffic (CT = 16-row
//   column tiles of M), and issues 4 k-blocks of loads (4*NSUB KiB of weights)
//   before it waits: HBM is kept busy by bytes in flight, not by instruction
//   count. Wide N uses NSUB=4 / 4 waves; narrow N (o, down, qkv) NSUB=1 with up
//   to 16 waves so that every CU still streams. (K is never split across
//   workgroups: an agent-scope fence between them costs a write-back and
//   invalidate of the whole L2 on this chip.)
// * Batch invariance: instruction, NSUB, KS and every summation order
//   depend only on (N, K), never on M, so a row's result is bit-identical
//   whether it is computed alone (autoregressive step) or inside a 25-row
//   verify batch. This is what keeps speculative greedy output identical to
//   plain greedy decoding in bf16.
// * Epilogues mirror the reference's bf16 rounding points (linear output
//   rounded to bf16, then each elementwise op rounded): plain store, bias +
//   activation, residual add, SwiGLU (gate rows 0-7 / up rows 8-15 of a tile),
//   and QKV + RoPE + KV-cache write (rotary pair dims in rows r and r+8).
#include "gemm_epi.h"
#include "topk.h"

#include <algorithm>

namespace ssd {

template <int KS, int NSUB, int CT>
struct GemmLds {
  // [wave][sub-tile][column tile][element e][lane]; the e stride of 68 words puts the 64 values
  // one wave reads in the epilogue (4 rows m x 16 tile rows r) in 64 different banks
  float red[KS][NSUB][CT][4][68];
  float ss[KS][CT][16];  // per-wave sums of x^2 per row (folded RMSNorm)
  float rn[CT * 16];     // per-row rsqrt(mean(x^2) + eps)
};

// X staged through LDS (gemm_kernel<..., XS = true>): K = 4096 (8 rounds of 16 k-blocks), 8 waves.
// Each round's rows are copied memory -> LDS by DMA as whole 1 KiB row segments (full 128-byte
// lines, once per workgroup) instead of each wave loading its 64-byte row pieces itself; rows are
// XS_ROW bytes apart so the 8 lanes a b128 read serves at a time fall in different banks.
constexpr int XS_ROUNDS = 8, XS_SLOTS = 2, XS_AHEAD = 3, XS_ROW = 16 * 64 + 16;

template <int KS, int NSUB, int CT, bool XS>
union GemmSmem {
  GemmLds<KS, NSUB, CT> g;
  unsigned char ring[XS ? XS_SLOTS * CT * 16 * XS_ROW : 16];
};

template <int CT, int NSUB, int KS, int U, int EPI, int NORM, bool XS = false>
__global__ __launch_bounds__(64 * KS) void gemm_kernel(GemmArgs a) {
  static_assert(!XS || KS == 8, "the staged path deals 16 k-blocks per round to 8 waves");
  __shared__ GemmSmem<KS, NSUB, CT, XS> smem;
  auto& lds = smem.g;
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int tile = blockIdx.x;
  const int kbt = a.kb_total;
  const int j = lane & 15, g = lane >> 4;

  f32x4_t acc[NSUB][CT];
#pragma unroll
  for (int s = 0; s < NSUB; ++s)
#pragma unroll
    for (int c = 0; c < CT; ++c) acc[s][c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float ss[CT];  // folded RMSNorm: this lane's sum of x^2 for row c*16 + j
#pragma unroll
  for (int c = 0; c < CT; ++c) ss[c] = 0.f;

  const u32x4_t* wp[NSUB];
#pragma unroll
  for (int s = 0; s < NSUB; ++s) wp[s] = (const u32x4_t*)a.W + (size_t)tile * kbt * NSUB * 64 + s * 64 + lane;  // grouped layout
  // Rows past M load row M-1 (always valid, no per-lane branch); their columns are never stored.
  const bf16_t* xp[CT];
#pragma unroll
  for (int c = 0; c < CT; ++c) xp[c] = a.X + (size_t)min(c * 16 + j, a.M - 1) * a.ldx + g * 8;

  // q/k/v: thread t owns pair t (token t / 8, pair row t % 8) of every sub-tile when the
  // workgroup has enough threads; its cache slot and position are loaded now (clamped, so the
  // loads are unconditional) and arrive while the weights stream.
  const int Mv = a.M < CT * 16 ? a.M : CT * 16;
  const bool qkv_pre = EPI == EPI_QKV && 8 * Mv <= 64 * KS;
  int pre_m = 0, pre_r = 0, pre_slot = 0, pre_pos = 0;
  int64_t pre_off = 0;
  if constexpr (EPI == EPI_QKV) {
    pre_m = min((int)threadIdx.x >> 3, Mv - 1);
    pre_r = threadIdx.x & 7;
    pre_slot = a.row_slot[pre_m];
    pre_pos = min(max(a.row_pos[pre_m], 0), (int)a.rope_rows - 1);
    if (a.row_kv_off) pre_off = a.row_kv_off[pre_m];
  }

  // plain store: thread t owns output (token t / 16, tile row t % 16) of every sub-tile when the
  // workgroup has enough threads; its residual and bias values are loaded now (clamped
  // addresses) and arrive while the weights stream.
  const bool st_pre = EPI == EPI_STORE && 16 * Mv <= 64 * KS;
  float pre_res[NSUB], pre_bias[NSUB];
  if constexpr (EPI == EPI_STORE) {
    const int pm = min((int)threadIdx.x >> 4, Mv - 1);
#pragma unroll
    for (int s = 0; s < NSUB; ++s) {
      const int n = min((tile * NSUB + s) * 16 + ((int)threadIdx.x & 15), a.N - 1);
      pre_res[s] = a.residual ? bf2f(a.residual[(size_t)pm * a.ldr + n]) : 0.f;
      pre_bias[s] = a.bias ? bf2f(a.bias[n]) : 0.f;
    }
  }

  // The wave's k-blocks: pairs dealt round-robin to the KS waves (pair i to wave i % KS), so the
  // waves stream neighbouring weight regions at the same time and finish together; the k-blocks
  // left after whole rounds go one by one. The sequence depends on (N, K) only.
  // Every workgroup reads all of X: the sequence is rotated by a tile-dependent, even number of
  // k-blocks ((tile / 8) % 8 eighths of K) so that the workgroups of one XCD (tiles 8 apart) read
  // different X lines at any moment instead of all the same ones.
  const int n_full = (kbt / (KS * 2)) * 2;
  const int rot = ((((tile >> 3) & 7) * kbt) >> 3) & ~1;
  auto wrap = [&](int kb) { return kb >= kbt ? kb - kbt : kb; };
  auto kb_at = [&](int t) { return wrap(((t >> 1) * KS + w) * 2 + (t & 1) + rot); };
  const int kb_rest = (kbt / (KS * 2)) * KS * 2 + w;
  if constexpr (XS) {
    // Round r = k-blocks kb_at(2r), kb_at(2r + 1) of every wave, i.e. 16 consecutive (rotated)
    // k-blocks. The wave loads its CT*2 rows of round r (one 1 KiB row segment per instruction)
    // and its weight tiles of round r XS_AHEAD rounds ahead, stores the rows into LDS slot r % 2
    // one round ahead, and every wave reads its fragments back after the barrier that opens
    // round r.
    // The MFMAs and the x^2 sums see the same fragments in the same order as the loop below.
    constexpr int RPW = CT * 2;  // rows each wave stages per round
    u32x4_t wv[XS_ROUNDS][2][NSUB], xv[XS_ROUNDS][RPW];
    auto issue = [&](int r) {
      const int kb = wrap(r * 16 + (lane >> 2) + rot);
#pragma unroll
      for (int i = 0; i < RPW; ++i)
        xv[r][i] = *(const u32x4_t*)(a.X + (size_t)min(w * RPW + i, a.M - 1) * a.ldx + kb * 32 + (lane & 3) * 8);
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int s = 0; s < NSUB; ++s)
          wv[r][u][s] = __builtin_nontemporal_load(wp[s] + (size_t)kb_at(2 * r + u) * NSUB * 64);
    };
    auto stage = [&](int r) {
      unsigned char* slot = smem.ring + (r % XS_SLOTS) * CT * 16 * XS_ROW;
#pragma unroll
      for (int i = 0; i < RPW; ++i) *(u32x4_t*)(slot + (w * RPW + i) * XS_ROW + lane * 16) = xv[r][i];
    };
#pragma unroll
    for (int r = 0; r < XS_AHEAD; ++r) issue(r);
    stage(0);
#pragma unroll
    for (int r = 0; r < XS_ROUNDS; ++r) {
      // round r's rows are in LDS (every wave's stores done before the barrier); no memory wait
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      if (r + XS_AHEAD < XS_ROUNDS) issue(r + XS_AHEAD);
      const unsigned char* slot = smem.ring + (r % XS_SLOTS) * CT * 16 * XS_ROW;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        u32x4_t xr[CT];
#pragma unroll
        for (int c = 0; c < CT; ++c) xr[c] = *(const u32x4_t*)(slot + (c * 16 + j) * XS_ROW + (2 * w + u) * 64 + g * 16);
#pragma unroll
        for (int s = 0; s < NSUB; ++s)
#pragma unroll
          for (int c = 0; c < CT; ++c) acc[s][c] = mfma16x16x32(bits_bf16x8(wv[r][u][s]), bits_bf16x8(xr[c]), acc[s][c]);
        if constexpr (NORM) {
#pragma unroll
          for (int c = 0; c < CT; ++c) ss[c] += sumsq8(xr[c]);
        }
      }
      // slot (r + 1) % 2 last held round r - 1, which every wave finished before this barrier
      if (r + 1 < XS_ROUNDS) stage(r + 1);
    }
    __syncthreads();  // the ring is reused for the partial sums below
  } else {
  int t = 0;
  for (; t + U <= n_full; t += U) {
    u32x4_t wr[U][NSUB], xr[U][CT];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int s = 0; s < NSUB; ++s) wr[u][s] = __builtin_nontemporal_load(wp[s] + (size_t)kb_at(t + u) * NSUB * 64);
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int c = 0; c < CT; ++c)
        xr[u][c] = *(const u32x4_t*)(xp[c] + kb_at(t + u) * 32);
    // Keep every load of the trip ahead of its MFMAs: left alone, the scheduler sinks the later
    // k-blocks' loads below the first MFMAs to save registers, leaving one k-block in flight.
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int s = 0; s < NSUB; ++s)
#pragma unroll
        for (int c = 0; c < CT; ++c) acc[s][c] = mfma16x16x32(bits_bf16x8(wr[u][s]), bits_bf16x8(xr[u][c]), acc[s][c]);
    if constexpr (NORM) {
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int c = 0; c < CT; ++c) ss[c] += sumsq8(xr[u][c]);
    }
  }
  for (int tt = t;; ++tt) {  // the rest of the whole rounds, then the leftover k-blocks
    const int kb0 = tt < n_full ? ((tt >> 1) * KS + w) * 2 + (tt & 1) : kb_rest + (tt - n_full) * KS;
    if (kb0 >= kbt) break;
    const int kb = wrap(kb0 + rot);
    u32x4_t wr[NSUB], xr[CT];
#pragma unroll
    for (int s = 0; s < NSUB; ++s) wr[s] = __builtin_nontemporal_load(wp[s] + (size_t)kb * NSUB * 64);
#pragma unroll
    for (int c = 0; c < CT; ++c) xr[c] = *(const u32x4_t*)(xp[c] + kb * 32);
#pragma unroll
    for (int s = 0; s < NSUB; ++s)
#pragma unroll
      for (int c = 0; c < CT; ++c) acc[s][c] = mfma16x16x32(bits_bf16x8(wr[s]), bits_bf16x8(xr[c]), acc[s][c]);
    if constexpr (NORM) {
#pragma unroll
      for (int c = 0; c < CT; ++c) ss[c] += sumsq8(xr[c]);
    }
  }
  }

  // rotary cos/sin of this thread's pairs (issued before the reduction so they overlap it)
  float pre_cs[NSUB], pre_sn[NSUB];
  if constexpr (EPI == EPI_QKV) {
    const int half = a.head_dim >> 1;
#pragma unroll
    for (int s = 0; s < NSUB; ++s) {
      const QkvTile q = qkv_tile(a, min(tile * NSUB + s, (a.N >> 4) - 1));
      const size_t at = (size_t)pre_pos * half + min(q.p * 8 + pre_r, half - 1);
      pre_cs[s] = bf2f(a.cos_tab[at]);
      pre_sn[s] = bf2f(a.sin_tab[at]);
    }
  }

#pragma unroll
  for (int s = 0; s < NSUB; ++s)
#pragma unroll
    for (int c = 0; c < CT; ++c)
#pragma unroll
      for (int e = 0; e < 4; ++e) lds.red[w][s][c][e][lane] = acc[s][c][e];
  if constexpr (NORM) {
    // row sums: the 4 k-groups of the wave (lanes j, j+16, j+32, j+48), then the waves in order
#pragma unroll
    for (int c = 0; c < CT; ++c) {
      float v = ss[c];
      v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 32);
      if (g == 0) lds.ss[w][c][j] = v;
    }
  }
  __syncthreads();
  if constexpr (NORM) {
    if ((int)threadIdx.x < CT * 16) {
      const int c = threadIdx.x >> 4, jj = threadIdx.x & 15;
      float v = lds.ss[0][c][jj];
#pragma unroll
      for (int ww = 1; ww < KS; ++ww) v += lds.ss[ww][c][jj];
      lds.rn[threadIdx.x] = rsqrtf(v / (float)(kbt * 32) + a.norm_eps);
    }
    __syncthreads();
  }

  // Tile row r (0..15) of sub-tile s, token m, summed over the waves in wave order (then scaled
  // by the row's folded RMSNorm factor).
#pragma unroll
  for (int s = 0; s < NSUB; ++s) {
    auto val = [&](int r, int m) -> float {
      const int c = m >> 4;
      const int ln = (m & 15) + 16 * (r >> 2);
      const int e = r & 3;
      float v = lds.red[0][s][c][e][ln];
#pragma unroll
      for (int ww = 1; ww < KS; ++ww) v += lds.red[ww][s][c][e][ln];
      if constexpr (NORM) v *= lds.rn[m];
      return v;
    };
    if constexpr (EPI == EPI_STORE) {
      if (st_pre) {
        const int m = threadIdx.x >> 4, r = threadIdx.x & 15;
        const int n = (tile * NSUB + s) * 16 + r;
        if (m < Mv && n < a.N) epi_store_pre(a, n, m, val(r, m), pre_bias[s], pre_res[s]);
        continue;
      }
    }
    if constexpr (EPI == EPI_QKV) {
      if (qkv_pre) {
        const int nb = tile * NSUB + s;
        if (nb * 16 < a.N && (int)threadIdx.x < 8 * Mv)
          epi_qkv_pre(a, qkv_tile(a, nb), pre_m, pre_r, val(pre_r, pre_m), val(pre_r + 8, pre_m), pre_slot,
                      pre_cs[s], pre_sn[s], pre_off);
        continue;
      }
    }
    gemm_epilogue<EPI, 64 * KS>(a, tile * NSUB + s, Mv, val, threadIdx.x);
  }
}

// ------------------------------------------------------------ wide outputs (vocabulary heads)
// One 8-wave workgroup per CU streams whole 8-tile groups g = blockIdx.x, + gridDim.x, ... (the
// NSUB = 8 packing); the waves take each group's k-block pairs round-robin (pair i to wave i % 8),
// so all eight walk one contiguous weight region together and finish together, and their
// partial sums meet in LDS in wave order. The folded RMSNorm scale comes from the first group's
// X fragments. Order of every sum: a function of (N, K) only.
constexpr int WIDE_WAVES = 8, WIDE_DEAL = 2;

template <int CT>
struct WideCfg {
  static constexpr int SC0 = 17408 / (WIDE_WAVES * CT * 4 * 68);
  static constexpr int SC = SC0 < 8 ? SC0 : 8;  // sub-tiles reduced per LDS pass
};

// Top-k records of a vocabulary head (ssd_gemm_topk_bf16). The 8-tile groups are cut into S slabs
// of G consecutive groups (a function of N only); a workgroup walks slabs blockIdx.x, + gridDim.x,
// ..., the groups of a slab in order, and leaves one TopkPart per (row, slab): the slab's k best
// (value, column) keys, its maximum and (mode 1) its sum of exp(x - max), accumulated group by group
// (the sum rescaled when the maximum grows). Values are the bf16-rounded logits, exactly what the
// plain head would store.
struct WideTopk {
  TopkPart* parts;  // [M][S]
  int k, mode;      // k <= TOPK_MAX; mode 1 adds the sum of exp
  int G, S;
  int pg;           // tiles per packing group of W (the layout ssd_gemm_bf16 reads for this N)
};

__device__ __forceinline__ uint64_t shfl_u64(uint64_t v, int src) {
  const uint32_t lo = __shfl((uint32_t)v, src), hi = __shfl((uint32_t)(v >> 32), src);
  return ((uint64_t)hi << 32) | lo;
}

// PG: W packed in 8-tile groups (8), or (0) in tk.pg-tile groups, pg in {1, 2, 4, 8}: tile t, k-block kb at
// ((t / pg) * kb_total * pg + kb * pg + t % pg) * 64 lanes.
template <int CT, int U, int NORM, int TOPK, int PG>
__global__ __launch_bounds__(64 * WIDE_WAVES) void gemm_wide_kernel(GemmArgs a, int n_groups, WideTopk tk) {
  constexpr int SC = WideCfg<CT>::SC;
  constexpr int TR = TOPK ? CT * 16 : 1;  // rows of the top-k state
  __shared__ float red[WIDE_WAVES][SC][CT][4][68];
  __shared__ float ssw[WIDE_WAVES][CT][16];
  __shared__ float rn[CT * 16];
  __shared__ float tv[TR][128];                // one group's bf16-rounded logits per row
  __shared__ uint64_t tkey[TR][TOPK_MAX];      // running k best per row (0: none)
  __shared__ float tmx[TR], tse[TR];           // running max / sum of exp per row
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int kbt = a.kb_total;
  const int Mv = a.M < CT * 16 ? a.M : CT * 16;
  const bf16_t* xp[CT];
#pragma unroll
  for (int c = 0; c < CT; ++c) xp[c] = a.X + (size_t)min(c * 16 + j, a.M - 1) * a.ldx + g * 8;
  const int n_full = (kbt / (WIDE_WAVES * WIDE_DEAL)) * WIDE_DEAL;  // this wave's k-blocks in whole rounds
  auto kb_at = [&](int t) { return ((t / WIDE_DEAL) * WIDE_WAVES + w) * WIDE_DEAL + t % WIDE_DEAL; };
  const int kb_rest = (kbt / (WIDE_WAVES * WIDE_DEAL)) * WIDE_WAVES * WIDE_DEAL + w;
  // plain logits: two adjacent outputs per 4-byte store
  const bool pair_store = !a.bias && !a.act && !a.residual && a.ldy % 2 == 0 && ((uintptr_t)a.Y & 3) == 0;
  const bool store = a.Y != nullptr;  // the top-k head stores its logits only when asked
  const int G = TOPK ? tk.G : 1, n_slabs = TOPK ? tk.S : n_groups;
  bool first = true;
  for (int slab = blockIdx.x; slab < n_slabs; slab += gridDim.x) {
  if constexpr (TOPK) {
    for (int i = threadIdx.x; i < TR * TOPK_MAX; i += 64 * WIDE_WAVES) tkey[i / TOPK_MAX][i % TOPK_MAX] = 0ull;
    if ((int)threadIdx.x < TR) { tmx[threadIdx.x] = -INFINITY; tse[threadIdx.x] = 0.f; }
    // the first group's epilogue barriers order these writes before the state is read
  }
  const int g_end = min((slab + 1) * G, n_groups);
  for (int grp = slab * G; grp < g_end; ++grp, first = false) {
    f32x4_t acc[8][CT];
#pragma unroll
    for (int s = 0; s < 8; ++s)
#pragma unroll
      for (int c = 0; c < CT; ++c) acc[s][c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    float ss[CT];
#pragma unroll
    for (int c = 0; c < CT; ++c) ss[c] = 0.f;
    const u32x4_t* wp = (const u32x4_t*)a.W + (size_t)grp * kbt * 8 * 64 + lane;
    uint32_t wq[8];  // PG == 0: 16-byte offset of tile s of the group (packed heads stay below 2^32 of them)
    uint32_t wstride = 0;
    if constexpr (PG == 0) {
      const int pg = tk.pg;
      wstride = (uint32_t)pg * 64;
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const int t = grp * 8 + s;
        wq[s] = ((uint32_t)(t / pg) * kbt * pg + t % pg) * 64 + lane;
      }
    }
    auto wload = [&](int kb, int s) -> u32x4_t {
      if constexpr (PG == 8) return __builtin_nontemporal_load(wp + ((size_t)kb * 8 + s) * 64);
      else return __builtin_nontemporal_load((const u32x4_t*)a.W + (wq[s] + (uint32_t)kb * wstride));
    };
    int t = 0;
    for (; t + U <= n_full; t += U) {
      u32x4_t wr[U][8], xr[U][CT];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int kb = kb_at(t + u);
#pragma unroll
        for (int s = 0; s < 8; ++s) wr[u][s] = wload(kb, s);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int kb = kb_at(t + u);
#pragma unroll
        for (int c = 0; c < CT; ++c) xr[u][c] = *(const u32x4_t*)(xp[c] + kb * 32);
      }
      __builtin_amdgcn_sched_barrier(0);  // every load of the trip ahead of its MFMAs
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int s = 0; s < 8; ++s)
#pragma unroll
          for (int c = 0; c < CT; ++c)
            acc[s][c] = mfma16x16x32(bits_bf16x8(wr[u][s]), bits_bf16x8(xr[u][c]), acc[s][c]);
      if (NORM && first) {
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int c = 0; c < CT; ++c) ss[c] += sumsq8(xr[u][c]);
      }
    }
    for (int tt = t;; ++tt) {  // the rest of the whole rounds, then the leftover k-blocks
      const int kb = tt < n_full ? kb_at(tt) : kb_rest + (tt - n_full) * WIDE_WAVES;
      if (kb >= kbt) break;
      u32x4_t wr[8], xr[CT];
#pragma unroll
      for (int s = 0; s < 8; ++s) wr[s] = wload(kb, s);
#pragma unroll
      for (int c = 0; c < CT; ++c) xr[c] = *(const u32x4_t*)(xp[c] + kb * 32);
#pragma unroll
      for (int s = 0; s < 8; ++s)
#pragma unroll
        for (int c = 0; c < CT; ++c) acc[s][c] = mfma16x16x32(bits_bf16x8(wr[s]), bits_bf16x8(xr[c]), acc[s][c]);
      if (NORM && first) {
#pragma unroll
        for (int c = 0; c < CT; ++c) ss[c] += sumsq8(xr[c]);
      }
    }
    if (NORM && first) {
#pragma unroll
      for (int c = 0; c < CT; ++c) {
        float v = ss[c];
        v += __shfl_xor(v, 16);
        v += __shfl_xor(v, 32);
        if (g == 0) ssw[w][c][j] = v;
      }
    }
    // sub-tiles in passes of SC through LDS; item (sub-tile, row m, column pair q): outputs
    // 16 (8 grp + s) + 2q and + 2q + 1
#pragma unroll
    for (int s0 = 0; s0 < 8; s0 += SC) {
#pragma unroll
      for (int s = 0; s < 8; ++s)
        if (s >= s0 && s < s0 + SC)
#pragma unroll
          for (int c = 0; c < CT; ++c)
#pragma unroll
            for (int e = 0; e < 4; ++e) red[w][s - s0][c][e][lane] = acc[s][c][e];
      __syncthreads();
      if (NORM && first && s0 == 0) {
        if ((int)threadIdx.x < CT * 16) {
          const int c = threadIdx.x >> 4, jj = threadIdx.x & 15;
          float v = ssw[0][c][jj];
#pragma unroll
          for (int ww = 1; ww < WIDE_WAVES; ++ww) v += ssw[ww][c][jj];
          rn[threadIdx.x] = rsqrtf(v / (float)(kbt * 32) + a.norm_eps);
        }
        __syncthreads();
      }
      const int nsc = 8 - s0 < SC ? 8 - s0 : SC;
      for (int o = threadIdx.x; o < nsc * 8 * Mv; o += 64 * WIDE_WAVES) {
        const int q = o & 7;
        const int m = (o >> 3) % Mv, sl = (o >> 3) / Mv;
        const int c = m >> 4;
        auto val = [&](int r) -> float {
          const int ln = (m & 15) + 16 * (r >> 2), e = r & 3;
          float v = red[0][sl][c][e][ln];
#pragma unroll
          for (int ww = 1; ww < WIDE_WAVES; ++ww) v += red[ww][sl][c][e][ln];
          if constexpr (NORM) v *= rn[m];
          return v;
        };
        const int n = (grp * 8 + s0 + sl) * 16 + 2 * q;
        if (n >= a.N) continue;
        const float v0 = val(2 * q), v1 = val(2 * q + 1);
        if constexpr (TOPK) {
          tv[m][(s0 + sl) * 16 + 2 * q] = rbf(v0);
          tv[m][(s0 + sl) * 16 + 2 * q + 1] = rbf(v1);  // past N: never read
          if (!store) continue;
        }
        if (pair_store && n + 1 < a.N) {
          *(uint32_t*)(a.Y + (size_t)m * a.ldy + n) = pack_bf16x2(rbf(v0), rbf(v1));
        } else {
          epi_store(a, n, m, v0);
          if (n + 1 < a.N) epi_store(a, n + 1, m, v1);
        }
      }
      __syncthreads();  // the next pass (or group) overwrites red
    }
    if constexpr (TOPK) {
      // wave w updates rows w, w + 8, ...: lane l holds columns 2l, 2l + 1 of the group
      const int n0 = grp * 128 + 2 * lane;
      const bool ok0 = n0 < a.N, ok1 = n0 + 1 < a.N;
      for (int m = w; m < Mv; m += WIDE_WAVES) {
        const float va = tv[m][2 * lane], vb = tv[m][2 * lane + 1];
        float gm = fmaxf(ok0 ? va : -INFINITY, ok1 ? vb : -INFINITY);
        for (int off = 32; off >= 1; off >>= 1) gm = fmaxf(gm, __shfl_xor(gm, off));
        const float om = tmx[m], nm = fmaxf(om, gm);
        if (tk.mode == 1) {
          float e = (ok0 ? __expf(va - nm) : 0.f) + (ok1 ? __expf(vb - nm) : 0.f);
          for (int off = 32; off >= 1; off >>= 1) e += __shfl_xor(e, off);
          const float os = tse[m];
          if (lane == 0) tse[m] = (om == -INFINITY ? 0.f : os * __expf(om - nm)) + e;
        }
        if (lane == 0) tmx[m] = nm;
        const uint64_t ka = ok0 ? rank_key(va, n0) : 0ull, kb = ok1 ? rank_key(vb, n0 + 1) : 0ull;
        uint64_t c0 = lane < TOPK_MAX ? tkey[m][lane] : 0ull;
        const uint64_t kth = shfl_u64(c0, tk.k - 1);
        if (!__any(ka > kth || kb > kth)) continue;  // nothing in this group enters the row's k best
        // the k best of (list, group): k rounds of a wave maximum (keys are distinct)
        uint64_t c1 = ka, c2 = kb, nk = 0ull;
        for (int q = 0; q < tk.k; ++q) {
          uint64_t b = c0 > c1 ? c0 : c1;
          b = b > c2 ? b : c2;
          const uint64_t mq = wave_max_u64(b);
          if (mq != 0ull) {
            if (c0 == mq) c0 = 0ull;
            else if (c1 == mq) c1 = 0ull;
            else if (c2 == mq) c2 = 0ull;
          }
          if (lane == q) nk = mq;
        }
        if (lane < TOPK_MAX) tkey[m][lane] = nk;
      }
      // the next group's first barrier orders these updates before tv is rewritten
    }
  }
  if constexpr (TOPK) {
    // each row's state was last written by its own wave: no barrier needed to read it here
    for (int m = w; m < Mv; m += WIDE_WAVES) {
      const TopkRec o = topk_rec(tk.parts, (size_t)m * tk.S + slab, tk.k);
      if (lane < tk.k) o.key[lane] = tkey[m][lane];
      if (lane == 0) {
        *o.mx = tmx[m];
        *o.se = tk.mode == 1 ? tse[m] : 0.f;
      }
    }
    __syncthreads();  // the next slab's reset follows every wave's record
  }
  }
}

// ------------------------------------------------------------ split-K partials
// P[s][m][n] = sum over the s-th K range of X[m, k] W[n, k], fp32 (s < S). Workgroup = (NW*NSUB
// 16-row tiles of N, one K range); wave w streams its NSUB weight tiles over the whole range,
// and all waves share the activations, staged once per workgroup in LDS (k-block major, KC
// k-blocks per pass, the next pass's weights and activations loaded while this one computes).
// Splitting K over workgroups keeps narrow-N GEMMs (o, down, qkv) at >= 256 workgroups with
// NSUB = 1 while each activation byte leaves L2 once per workgroup instead of once per wave.
// The S partials are reduced in a fixed order by the consumer (gemm_finalize_kernel,
// add_rmsnorm_kernel); S depends only on (N, K), so results stay batch-invariant.
template <int CT>
struct PartCfg {
  static constexpr int KC = CT <= 2 ? 16 : 8;  // k-blocks of activations per LDS pass (KC * CT KiB)
};

template <int CT, int NSUB, int NW>
__global__ __launch_bounds__(64 * NW) void gemm_part_kernel(GemmArgs a, float* __restrict__ P, int64_t ldp,
                                                            int64_t sstride, int S) {
  constexpr int KC = PartCfg<CT>::KC;
  constexpr int XCH = KC * CT * 64;                    // 16-byte activation chunks per pass
  constexpr int XIT = (XCH + 64 * NW - 1) / (64 * NW); // per thread
  __shared__ u32x4_t xs[XCH];                          // [kb][m][4 x 16 B]
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int kbt = a.kb_total;
  const int split = blockIdx.y;
  const int kb0 = (int)(((int64_t)kbt * split) / S), kb1 = (int)(((int64_t)kbt * (split + 1)) / S);
  const int tile0 = (blockIdx.x * NW + w) * NSUB;
  const bool active = tile0 * 16 < a.N;  // packed rows are padded to 64, so whole sub-tiles exist
  const u32x4_t* W = (const u32x4_t*)a.W;
  const u32x4_t* wp[NSUB];
#pragma unroll
  for (int s = 0; s < NSUB; ++s) wp[s] = W + ((size_t)(tile0 + s) * kbt) * 64 + lane;

  f32x4_t acc[NSUB][CT];
#pragma unroll
  for (int s = 0; s < NSUB; ++s)
#pragma unroll
    for (int c = 0; c < CT; ++c) acc[s][c] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  u32x4_t xv[XIT], wr[KC][NSUB];
  // Loads of one pass [c0, c0 + nk): indices are clamped (no per-lane branches around loads).
  auto load_pass = [&](int c0, int nk, u32x4_t (&xo)[XIT], u32x4_t (&wo)[KC][NSUB]) {
    const int nx = nk * CT * 64;
#pragma unroll
    for (int it = 0; it < XIT; ++it) {
      const int idx = min((int)threadIdx.x + it * 64 * NW, nx - 1);
      const int kb = idx / (CT * 64), rem = idx % (CT * 64);
      const int m = min(rem >> 2, a.M - 1);
      xo[it] = *(const u32x4_t*)(a.X + (size_t)m * a.ldx + (size_t)(c0 + kb) * 32 + (rem & 3) * 8);
    }
    if (active) {
#pragma unroll
      for (int u = 0; u < KC; ++u)
#pragma unroll
        for (int s = 0; s < NSUB; ++s) wo[u][s] = __builtin_nontemporal_load(wp[s] + (size_t)(c0 + min(u, nk - 1)) * 64);
    }
  };
  int c0 = kb0;
  int nk = min(KC, kb1 - c0);
  if (nk > 0) load_pass(c0, nk, xv, wr);
  while (nk > 0) {
    __syncthreads();  // the previous pass's readers are done with xs
#pragma unroll
    for (int it = 0; it < XIT; ++it) {
      const int idx = threadIdx.x + it * 64 * NW;
      if (idx < nk * CT * 64) xs[idx] = xv[it];
    }
    __syncthreads();
    const int c1 = c0 + nk;
    const int nk1 = min(KC, kb1 - c1);
    u32x4_t wn[KC][NSUB];
    if (nk1 > 0) load_pass(c1, nk1, xv, wn);
    if (active) {
#pragma unroll
      for (int u = 0; u < KC; ++u) {
        if (u < nk) {
          u32x4_t xr[CT];
#pragma unroll
          for (int c = 0; c < CT; ++c) xr[c] = xs[(u * CT * 16 + c * 16 + j) * 4 + g];
#pragma unroll
          for (int s = 0; s < NSUB; ++s)
#pragma unroll
            for (int c = 0; c < CT; ++c)
              acc[s][c] = mfma16x16x32(bits_bf16x8(wr[u][s]), bits_bf16x8(xr[c]), acc[s][c]);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < KC; ++u)
#pragma unroll
      for (int s = 0; s < NSUB; ++s) wr[u][s] = wn[u][s];
    c0 = c1;
    nk = nk1;
  }
  // Lane (j, g) holds rows n = 16 tile + 4g + e of column m = 16c + j.
  if (active) {
#pragma unroll
    for (int s = 0; s < NSUB; ++s)
#pragma unroll
      for (int c = 0; c < CT; ++c) {
        const int m = c * 16 + j;
        if (m < a.M) *(f32x4_t*)(P + split * sstride + (size_t)m * ldp + (tile0 + s) * 16 + 4 * g) = acc[s][c];
      }
  }
}

// Epilogue over split-K partials: one thread per (row m, tile nb, pair r) -- r and r + 8 for the
// SwiGLU / RoPE pairings, both for the plain store -- so the grid covers every output at once.
// The S partials (S a template constant, loads issued together) are summed in order s = 0..S-1,
// then the single-pass kernel's bf16 epilogue runs on the sums.
template <int EPI, int S>
__global__ __launch_bounds__(256) void gemm_finalize_kernel(GemmArgs a, const float* __restrict__ P, int64_t ldp,
                                                            int64_t sstride) {
  const int tiles = (a.N + 15) / 16;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)a.M * tiles * 8) return;
  const int r = (int)(idx & 7);
  const int nb = (int)((idx >> 3) % tiles);
  const int m = (int)((idx >> 3) / tiles);
  const float* p = P + (size_t)m * ldp + nb * 16 + r;
  float lo[S], hi[S];
#pragma unroll
  for (int s = 0; s < S; ++s) {
    lo[s] = p[s * sstride];
    hi[s] = p[s * sstride + 8];
  }
  float vlo = lo[0], vhi = hi[0];
#pragma unroll
  for (int s = 1; s < S; ++s) {
    vlo += lo[s];
    vhi += hi[s];
  }
  if constexpr (EPI == EPI_STORE) {
    if (nb * 16 + r < a.N) epi_store(a, nb * 16 + r, m, vlo);
    if (nb * 16 + r + 8 < a.N) epi_store(a, nb * 16 + r + 8, m, vhi);
  } else {
    epi_qkv(a, nb, m, r, vlo, vhi);
  }
}

template <int EPI>
static int launch_finalize(const GemmArgs& a, const float* P, int64_t ldp, int64_t sstride, int S, hipStream_t s) {
  const int64_t threads = (int64_t)a.M * ((a.N + 15) / 16) * 8;
  const dim3 grid((unsigned)((threads + 255) / 256)), block(256);
  switch (S) {
    case 1: SSD_LAUNCH((gemm_finalize_kernel<EPI, 1>), grid, block, 0, s, a, P, ldp, sstride); break;
    case 2: SSD_LAUNCH((gemm_finalize_kernel<EPI, 2>), grid, block, 0, s, a, P, ldp, sstride); break;
    case 4: SSD_LAUNCH((gemm_finalize_kernel<EPI, 4>), grid, block, 0, s, a, P, ldp, sstride); break;
    case 8: SSD_LAUNCH((gemm_finalize_kernel<EPI, 8>), grid, block, 0, s, a, P, ldp, sstride); break;
    case 16: SSD_LAUNCH((gemm_finalize_kernel<EPI, 16>), grid, block, 0, s, a, P, ldp, sstride); break;
    default: return set_error(SSD_EINVAL, "finalize: split count %d not in {1, 2, 4, 8, 16}", S);
  }
  return SSD_OK;
}

struct PartPlan {
  int nsub, nw, S;
};

// Split count as a function of (N, K) only: enough workgroups for the chip (~256), each with at
// least 8 k-blocks.
static PartPlan part_plan(int N, int K) {
  PartPlan p;
  p.nsub = 1;
  p.nw = 8;
  const int kbt = K / 32;
  const int groups = (N + 16 * p.nw * p.nsub - 1) / (16 * p.nw * p.nsub);
  p.S = 1;
  while (groups * p.S < 256 && p.S * 2 * 8 <= kbt && p.S < 16) p.S *= 2;
  return p;
}

static int launch_part(const GemmArgs& a, float* P, int64_t ldp, int64_t sstride, hipStream_t s) {
  const PartPlan p = part_plan(a.N, a.kb_total * 32);
  const int groups = (a.N + 16 * p.nw * p.nsub - 1) / (16 * p.nw * p.nsub);
  for (int m0 = 0; m0 < a.M; m0 += 64) {
    GemmArgs b = a;
    b.M = std::min(64, a.M - m0);
    b.X = a.X + (size_t)m0 * a.ldx;
    float* Pm = P + (size_t)m0 * ldp;
    const int ct = (b.M + 15) / 16;
    dim3 grid(groups, p.S);
    switch (ct) {
      case 1: SSD_LAUNCH((gemm_part_kernel<1, 1, 8>), grid, dim3(512), 0, s, b, Pm, ldp, sstride, p.S); break;
      case 2: SSD_LAUNCH((gemm_part_kernel<2, 1, 8>), grid, dim3(512), 0, s, b, Pm, ldp, sstride, p.S); break;
      case 3: SSD_LAUNCH((gemm_part_kernel<3, 1, 8>), grid, dim3(512), 0, s, b, Pm, ldp, sstride, p.S); break;
      default: SSD_LAUNCH((gemm_part_kernel<4, 1, 8>), grid, dim3(512), 0, s, b, Pm, ldp, sstride, p.S); break;
    }
    const int rc = check_launch("gemm_part");
    if (rc) return rc;
  }
  return SSD_OK;
}

// ---------------------------------------------------------------- packing
// dst tile (nb, kb), lane l, element t  <-  W[row_map[16 nb + l%16]][32 kb + 8 (l/16) + t]
// (row_map entry < 0 or beyond K -> zero). Tiles are stored grouped: the `group` tiles
// nb = g*group .. g*group+group-1 of one k-block sit next to each other ([g][kb][nb % group]), so
// a workgroup that owns a group streams one contiguous region.
__global__ void pack_kernel(const bf16_t* __restrict__ src, int64_t ld, int K, const int* __restrict__ row_map,
                            int n_tiles_n, int kb_total, int group, const bf16_t* __restrict__ col_scale,
                            uint4* __restrict__ dst) {
  const int64_t tile = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (tile >= (int64_t)n_tiles_n * kb_total) return;
  const int nb = (int)(tile / kb_total), kb = (int)(tile % kb_total);
  const int row = row_map[nb * 16 + (lane & 15)];
  const int k0 = kb * 32 + (lane >> 4) * 8;
  Pack8 p;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const bf16_t v = (row >= 0 && k0 + t < K) ? src[(size_t)row * ld + k0 + t] : (bf16_t)0;
    // folded RMSNorm weight: column k scaled by col_scale[k], rounded once to bf16
    p.h[t] = (col_scale && k0 + t < K) ? f2bf(bf2f(v) * bf2f(col_scale[k0 + t])) : v;
  }
  const int64_t dst_tile = ((int64_t)(nb / group) * kb_total + kb) * group + nb % group;
  dst[dst_tile * 64 + lane] = p.u;
}

struct GemmPlan {
  int nsub, ks, tiles;
};

// Launch geometry as a function of (N, K) only (never of M): that is what keeps every row's
// arithmetic identical for any batch size (a row's sum runs over the k-blocks of each of the ks
// waves in order, then over the waves in order; the tile grouping nsub does not enter it). The
// per-trip unroll U may follow M: it does not change the order. Measured on MI355X with every
// launch streaming its weights from HBM: vocabulary-wide heads stream best as 8-tile groups (run by
// gemm_wide_kernel for plain stores, else by gemm_kernel as 8 tiles x 2 waves),
// gate/up-wide outputs as 4 tiles x 2 waves, q/k/v-wide outputs as 2 tiles x 8 waves, narrow
// outputs as 1 tile x 8 waves (16 waves left the workgroup waiting ≈ 3 us for its slowest wave).
static GemmPlan plan_for(int N, int K) {
  const int kbt = K / 32;
  GemmPlan p;
  if (N >= 65536) {
    p.nsub = 8; p.ks = 2;
  } else if (N >= 16384) {
    p.nsub = 4; p.ks = 2;
  } else if (N >= 6144) {
    p.nsub = 2; p.ks = 8;
  } else {
    p.nsub = 1; p.ks = 8;
  }
  while (p.ks > 1 && kbt / p.ks < 4) p.ks >>= 1;  // at least 4 k-blocks per wave
  p.tiles = (N + 16 * p.nsub - 1) / (16 * p.nsub);
  return p;
}

// Wide plain-store GEMMs (N >= 65536: vocabulary heads) use gemm_wide_kernel on the same 8-tile
// packing (a function of the shape only).
static bool use_wide(const GemmPlan& p) { return p.nsub == 8; }

template <int EPI>
static int launch_wide(GemmArgs a, int n_groups, hipStream_t s, const WideTopk* tk = nullptr) {
  // one workgroup per CU (the CU count is read once per device)
  static int cus_of[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return set_error(SSD_EHIP, "gemm_wide: no current device");
  int cus = dev >= 0 && dev < 64 ? cus_of[dev] : 0;
  if (cus <= 0) {
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    if (dev >= 0 && dev < 64) cus_of[dev] = cus;
  }
  const dim3 grid((unsigned)std::min(tk ? tk->S : n_groups, cus)), block(64 * WIDE_WAVES);
  const int ct = (a.M + 15) / 16;
  const WideTopk t = tk ? *tk : WideTopk{};
  const bool pg8 = !tk || tk->pg == 8;
#define SSD_WIDE_K(CT_, U_, NORM_, TOPK_)                                                                \
  if (pg8) SSD_LAUNCH((gemm_wide_kernel<CT_, U_, NORM_, TOPK_, 8>), grid, block, 0, s, a, n_groups, t); \
  else SSD_LAUNCH((gemm_wide_kernel<CT_, (U_ > 2 ? 2 : U_), NORM_, TOPK_, 0>), grid, block, 0, s, a, n_groups, t);
#define SSD_WIDE(CT_, U_)                                                                            \
  if (tk) {                                                                                          \
    if (a.norm_eps > 0.f) { SSD_WIDE_K(CT_, U_, 1, 1) } else { SSD_WIDE_K(CT_, U_, 0, 1) }           \
  } else if (a.norm_eps > 0.f) SSD_LAUNCH((gemm_wide_kernel<CT_, U_, 1, 0, 8>), grid, block, 0, s, a, n_groups, t); \
  else SSD_LAUNCH((gemm_wide_kernel<CT_, U_, 0, 0, 8>), grid, block, 0, s, a, n_groups, t);
  switch (ct) {
    case 1: SSD_WIDE(1, 4) break;
    case 2: SSD_WIDE(2, 2) break;
    case 3: SSD_WIDE(3, 2) break;
    default: SSD_WIDE(4, 1) break;
  }
#undef SSD_WIDE
#undef SSD_WIDE_K
  return check_launch("gemm_wide");
}

// Slabs of the top-k head: G consecutive 8-tile groups each, at most TOPK_MAX_PARTS of them; a
// function of N only, so a row's records do not depend on M or on the device.
static void topk_slabs(int N, int& G, int& S) {
  const int groups = (N + 127) / 128;
  G = (groups + TOPK_MAX_PARTS - 1) / TOPK_MAX_PARTS;
  S = (groups + G - 1) / G;
}

template <int EPI>
static int launch_gemm(GemmArgs a, hipStream_t s) {
  const GemmPlan p = plan_for(a.N, a.kb_total * 32);
  // Rows beyond 64 are processed in chunks of 64; each chunk is computed exactly as it would be alone.
  for (int m0 = 0; m0 < a.M; m0 += 64) {
    GemmArgs b = a;
    b.M = std::min(64, a.M - m0);
    b.X = a.X + (size_t)m0 * a.ldx;
    if (a.Y) b.Y = a.Y + (size_t)m0 * a.ldy;
    if (a.residual) b.residual = a.residual + (size_t)m0 * a.ldr;
    if (a.row_pos) b.row_pos = a.row_pos + m0;
    if (a.row_slot) b.row_slot = a.row_slot + m0;
    if constexpr (EPI == EPI_STORE) {
      if (use_wide(p)) {
        const int rc = launch_wide<EPI>(b, p.tiles, s);
        if (rc) return rc;
        continue;
      }
    }
    const int ct = (b.M + 15) / 16;
    dim3 grid(p.tiles);
    if (b.kb_total == XS_ROUNDS * 16 && p.ks == 8 && p.nsub <= 2 && ct <= 2) {
      // K = 4096 narrow projections: x staged through LDS
#define SSD_GEMM_XS(CT_, NS_)                                                                             \
  if (ct == CT_ && p.nsub == NS_) {                                                                       \
    if (b.norm_eps > 0.f)                                                                                 \
      SSD_LAUNCH((gemm_kernel<CT_, NS_, 8, (CT_ == 1 ? 4 : 2), EPI, 1, true>), grid, dim3(512), 0, s, b); \
    else                                                                                                  \
      SSD_LAUNCH((gemm_kernel<CT_, NS_, 8, (CT_ == 1 ? 4 : 2), EPI, 0, true>), grid, dim3(512), 0, s, b); \
  }
      SSD_GEMM_XS(1, 1) SSD_GEMM_XS(1, 2) SSD_GEMM_XS(2, 1) SSD_GEMM_XS(2, 2)
#undef SSD_GEMM_XS
      int rc = check_launch("gemm");
      if (rc) return rc;
      continue;
    }
#define SSD_GEMM_CASE(CT_, NS_, KS_) \
  if (ct == CT_ && p.nsub == NS_ && p.ks == KS_) {                                                             \
    if (b.norm_eps > 0.f)                                                                                      \
      SSD_LAUNCH((gemm_kernel<CT_, NS_, KS_, (CT_ == 1 ? 4 : 2), EPI, 1>), grid, dim3(64 * KS_), 0, s, b); \
    else                                                                                                       \
      SSD_LAUNCH((gemm_kernel<CT_, NS_, KS_, (CT_ == 1 ? 4 : 2), EPI, 0>), grid, dim3(64 * KS_), 0, s, b); \
  }
#define SSD_GEMM_PLANS(CT_)                                                                                \
  SSD_GEMM_CASE(CT_, 8, 2) SSD_GEMM_CASE(CT_, 8, 1) SSD_GEMM_CASE(CT_, 4, 2) SSD_GEMM_CASE(CT_, 4, 1)     \
  SSD_GEMM_CASE(CT_, 2, 8) SSD_GEMM_CASE(CT_, 2, 4) SSD_GEMM_CASE(CT_, 2, 2) SSD_GEMM_CASE(CT_, 2, 1)     \
  SSD_GEMM_CASE(CT_, 1, 16) SSD_GEMM_CASE(CT_, 1, 8) SSD_GEMM_CASE(CT_, 1, 4) SSD_GEMM_CASE(CT_, 1, 2)    \
  SSD_GEMM_CASE(CT_, 1, 1)
    SSD_GEMM_PLANS(1) SSD_GEMM_PLANS(2) SSD_GEMM_PLANS(3) SSD_GEMM_PLANS(4)
#undef SSD_GEMM_PLANS
#undef SSD_GEMM_CASE
    int rc = check_launch("gemm");
    if (rc) return rc;
  }
  return SSD_OK;
}

static int check_common(const bf16_t* X, int64_t ldx, int M, const void* W, int N, int K) {
  if (!X || !W) return set_error(SSD_EINVAL, "gemm: null X or W");
  if (M < 0 || N <= 0 || K <= 0) return set_error(SSD_EINVAL, "gemm: bad shape M=%d N=%d K=%d", M, N, K);
  if (K % 32) return set_error(SSD_EINVAL, "gemm: K=%d must be a multiple of 32", K);
  if (((uintptr_t)X & 15) || (ldx % 8)) return set_error(SSD_EINVAL, "gemm: X must be 16-byte aligned with ldx %% 8 == 0");
  if (((uintptr_t)W & 15)) return set_error(SSD_EINVAL, "gemm: packed W must be 16-byte aligned");
  return SSD_OK;
}

}  // namespace ssd

using namespace ssd;

SSD_API int64_t ssd_packed_weight_elems(int N, int K) {
  return (int64_t)((N + 127) / 128) * 128 * (int64_t)((K + 31) / 32) * 32;
}

SSD_API int ssd_gemm_weight_group(int N, int K) {
  if (N <= 0 || K <= 0 || K % 32) {
    set_error(SSD_EINVAL, "weight_group: bad shape N=%d K=%d", N, K);
    return 0;
  }
  return plan_for(N, K).nsub;
}


SSD_API int ssd_pack_weight_bf16(const uint16_t* src, int64_t ld, int N_src, int K, const int32_t* row_map,
                                 int N_packed, int group, const uint16_t* col_scale, uint16_t* dst,
                                 hipStream_t stream) {
  if (!src || !dst || !row_map) return set_error(SSD_EINVAL, "pack: null pointer");
  if (N_packed <= 0 || N_packed % 128 || K <= 0 || N_src <= 0)
    return set_error(SSD_EINVAL, "pack: N_packed=%d must be a positive multiple of 128 (K=%d)", N_packed, K);
  const int n_tiles_n = N_packed / 16, kb_total = (K + 31) / 32;
  if (group < 1 || group > 16 || n_tiles_n % group)
    return set_error(SSD_EINVAL, "pack: group %d must be in [1, 16] and divide the %d row tiles", group, n_tiles_n);
  const int64_t tiles = (int64_t)n_tiles_n * kb_total;
  SSD_LAUNCH(pack_kernel, dim3((unsigned)((tiles + 3) / 4)), dim3(256), 0, stream, src, ld, K, row_map,
                     n_tiles_n, kb_total, group, col_scale, (uint4*)dst);
  return check_launch("pack");
}

// Y = act(X W^T + bias) [+ residual], bf16 rounding after each step. Y may alias residual.
// norm_eps > 0: X is the residual stream h and W was packed with the RMSNorm weight as col_scale;
// each row's outputs are scaled by rsqrt(mean(h^2) + norm_eps) (RMSNorm folded into the GEMM).
SSD_API int ssd_gemm_bf16(const uint16_t* X, int64_t ldx, int M, const uint16_t* W_packed, int N, int K,
                          float norm_eps, uint16_t* Y, int64_t ldy, const uint16_t* bias, int act,
                          const uint16_t* residual, int64_t ldr, hipStream_t stream) {
  int rc = check_common(X, ldx, M, W_packed, N, K);
  if (rc) return rc;
  if (!Y) return set_error(SSD_EINVAL, "gemm: null Y");
  if (act < 0 || act > 3) return set_error(SSD_EINVAL, "gemm: bad activation %d", act);
  if (residual && act) return set_error(SSD_EINVAL, "gemm: residual and activation are exclusive");
  if (M == 0) return SSD_OK;
  GemmArgs a{};
  a.X = X; a.ldx = ldx; a.M = M; a.W = (const uint4*)W_packed; a.N = N; a.kb_total = K / 32;
  a.Y = Y; a.ldy = ldy; a.bias = bias; a.act = act; a.residual = residual; a.ldr = ldr;
  a.norm_eps = norm_eps > 0.f ? norm_eps : 0.f;
  return launch_gemm<EPI_STORE>(a, stream);
}

SSD_API int ssd_gemm_topk_parts(int N) {
  if (N <= 0) return set_error(SSD_EINVAL, "gemm_topk_parts: N=%d", N);
  int G, S;
  topk_slabs(N, G, S);
  return S;
}

// The vocabulary head with its per-row top-k chunk pass in the epilogue: parts[m * S + s] (S =
// ssd_gemm_topk_parts(N)) gets slab s's k best keys, max and (mode 1) sum of exp of row m of
// X W^T (final norm folded when norm_eps > 0), for a merge (ssd_tree_level_topk,
// ssd_row_topk_merge_bf16). The logits themselves are stored only when Y is not null.
SSD_API int ssd_gemm_topk_bf16(const uint16_t* X, int64_t ldx, int M, const uint16_t* W_packed, int N, int K,
                               float norm_eps, int k, int mode, void* parts, int64_t parts_bytes, uint16_t* Y,
                               int64_t ldy, hipStream_t stream) {
  int rc = check_common(X, ldx, M, W_packed, N, K);
  if (rc) return rc;
  if (k < 1 || k > TOPK_MAX || k > N) return set_error(SSD_EINVAL, "gemm_topk: k=%d outside [1, min(%d, N)]", k, TOPK_MAX);
  if (mode != 0 && mode != 1) return set_error(SSD_EINVAL, "gemm_topk: mode %d", mode);
  if (!parts || ((uintptr_t)parts & 7)) return set_error(SSD_EINVAL, "gemm_topk: parts must be 8-byte aligned");
  if (Y && ldy < N) return set_error(SSD_EINVAL, "gemm_topk: ldy %lld < N=%d", (long long)ldy, N);
  WideTopk t{};
  topk_slabs(N, t.G, t.S);
  if (parts_bytes < (int64_t)M * t.S * (int64_t)sizeof(TopkPart))
    return set_error(SSD_EINVAL, "gemm_topk: parts of %lld bytes < %lld", (long long)parts_bytes,
                     (long long)M * t.S * (long long)sizeof(TopkPart));
  t.k = k;
  t.mode = mode;
  t.pg = plan_for(N, K).nsub;  // W is packed as ssd_gemm_bf16 reads it for this shape
  if (t.pg != 8 && ((N + 127) / 128 * 128) * (int64_t)K / 8 >= ((int64_t)1 << 32))
    return set_error(SSD_ERANGE, "gemm_topk: packed head of %d x %d too large", N, K);
  const int n_groups = (N + 127) / 128;
  for (int m0 = 0; m0 < M; m0 += 64) {
    GemmArgs a{};
    a.X = X + (size_t)m0 * ldx; a.ldx = ldx; a.M = std::min(64, M - m0); a.W = (const uint4*)W_packed;
    a.N = N; a.kb_total = K / 32;
    a.Y = Y ? Y + (size_t)m0 * ldy : nullptr; a.ldy = ldy;
    a.norm_eps = norm_eps > 0.f ? norm_eps : 0.f;
    t.parts = (TopkPart*)((char*)parts + (size_t)m0 * t.S * (size_t)(8 + 8 * k));
    if ((rc = launch_wide<EPI_STORE>(a, n_groups, stream, &t))) return rc;
  }
  return SSD_OK;
}

// Y[M, I] = silu(X Wg^T + bg) * (X Wu^T + bu); W_packed holds, per 16-row tile i, gate rows
// [8i, 8i+8) then up rows [8i, 8i+8). N = 2 I.
SSD_API int ssd_gemm_swiglu_bf16(const uint16_t* X, int64_t ldx, int M, const uint16_t* W_packed, int I, int K,
                                 float norm_eps, uint16_t* Y, int64_t ldy, const uint16_t* bias_gate,
                                 const uint16_t* bias_up, hipStream_t stream) {
  int rc = check_common(X, ldx, M, W_packed, 2 * I, K);
  if (rc) return rc;
  if (!Y || I % 8) return set_error(SSD_EINVAL, "gemm_swiglu: null Y or I=%d not a multiple of 8", I);
  if (M == 0) return SSD_OK;
  GemmArgs a{};
  a.X = X; a.ldx = ldx; a.M = M; a.W = (const uint4*)W_packed; a.N = 2 * I; a.kb_total = K / 32;
  a.Y = Y; a.ldy = ldy; a.bias = bias_gate; a.bias2 = bias_up;
  a.norm_eps = norm_eps > 0.f ? norm_eps : 0.f;
  return launch_gemm<EPI_SWIGLU>(a, stream);
}

// Fused q/k/v projection + RoPE + KV-cache write. W_packed: q heads, k heads, v heads; each
// head as head_dim/16 tiles whose rows 0-7 are dims [8p, 8p+8) and rows 8-15 dims
// [hd/2 + 8p, hd/2 + 8p + 8). q -> Q[m, heads*hd]; k and v -> slot row_slot[m] of the cache in
// its 64-slot block layout (k_off / v_off).
SSD_API int ssd_gemm_qkv_rope_bf16(const uint16_t* X, int64_t ldx, int M, const uint16_t* W_packed, int K,
                                   float norm_eps, int heads, int kv_heads, int head_dim, const uint16_t* cos_tab,
                                   const uint16_t* sin_tab, int64_t rope_rows, const int32_t* row_pos,
                                   const int32_t* row_slot,
                                   uint16_t* Q, int64_t ldq, uint16_t* k_cache, uint16_t* vt_cache,
                                   int64_t max_len, hipStream_t stream) {
  return ssd::qkv_rope_gemm(X, ldx, M, W_packed, K, norm_eps, heads, kv_heads, head_dim, cos_tab, sin_tab, rope_rows,
                            row_pos, row_slot, nullptr, Q, ldq, k_cache, vt_cache, max_len, stream);
}

// The q/k/v GEMM with per-row KV arena offsets (rows of several sequences in one launch).
int ssd::qkv_rope_gemm(const uint16_t* X, int64_t ldx, int M, const uint16_t* W_packed, int K, float norm_eps,
                       int heads, int kv_heads, int head_dim, const uint16_t* cos_tab, const uint16_t* sin_tab,
                       int64_t rope_rows, const int32_t* row_pos, const int32_t* row_slot, const int64_t* row_kv_off,
                       uint16_t* Q, int64_t ldq, uint16_t* k_cache, uint16_t* vt_cache, int64_t max_len,
                       hipStream_t stream) {
  const int N = (heads + 2 * kv_heads) * head_dim;
  int rc = check_common(X, ldx, M, W_packed, N, K);
  if (rc) return rc;
  if (head_dim % 32 || head_dim > 256) return set_error(SSD_EINVAL, "qkv: head_dim=%d unsupported", head_dim);
  if (!Q || !k_cache || !vt_cache || !cos_tab || !sin_tab || !row_pos || !row_slot)
    return set_error(SSD_EINVAL, "qkv: null pointer");
  if (max_len <= 0 || max_len % 64) return set_error(SSD_EINVAL, "qkv: max_len %lld not a multiple of 64", (long long)max_len);
  if (M == 0) return SSD_OK;
  GemmArgs a{};
  a.X = X; a.ldx = ldx; a.M = M; a.W = (const uint4*)W_packed; a.N = N; a.kb_total = K / 32;
  a.Y = Q; a.ldy = ldq; a.heads = heads; a.kv_heads = kv_heads; a.head_dim = head_dim;
  if (rope_rows <= 0) return set_error(SSD_EINVAL, "qkv: empty rope table");
  a.cos_tab = cos_tab; a.sin_tab = sin_tab; a.rope_rows = rope_rows; a.row_pos = row_pos; a.row_slot = row_slot;
  a.k_cache = k_cache; a.vt_cache = vt_cache; a.max_len = max_len; a.row_kv_off = row_kv_off;
  a.norm_eps = norm_eps > 0.f ? norm_eps : 0.f;
  return launch_gemm<EPI_QKV>(a, stream);
}

// ------------------------------------------------------------ split-K entry points
SSD_API int ssd_gemm_splits(int N, int K) {
  if (N <= 0 || K <= 0 || K % 32) return set_error(SSD_EINVAL, "gemm_splits: bad shape N=%d K=%d", N, K);
  return part_plan(N, K).S;
}

static int check_partials(const void* P, int64_t ldp, int64_t sstride, int M, int N) {
  if (!P) return set_error(SSD_EINVAL, "partials: null buffer");
  if (((uintptr_t)P & 15) || ldp % 4 || ldp < (N + 63) / 64 * 64 || sstride < (int64_t)M * ldp || sstride % 4)
    return set_error(SSD_EINVAL, "partials: need 16-byte alignment, ldp >= %d (multiple of 4), split stride >= M*ldp",
                     (N + 63) / 64 * 64);
  return SSD_OK;
}

// P[s][m][n] (s < ssd_gemm_splits(N, K)) = sum over the s-th K range of X W^T, fp32.
SSD_API int ssd_gemm_partial_bf16(const uint16_t* X, int64_t ldx, int M, const uint16_t* W_packed, int N, int K,
                                  float* P, int64_t ldp, int64_t split_stride, hipStream_t stream) {
  int rc = check_common(X, ldx, M, W_packed, N, K);
  if (rc) return rc;
  if ((rc = check_partials(P, ldp, split_stride, M, N))) return rc;
  if (M == 0) return SSD_OK;
  GemmArgs a{};
  a.X = X; a.ldx = ldx; a.M = M; a.W = (const uint4*)W_packed; a.N = N; a.kb_total = K / 32;
  return launch_part(a, P, ldp, split_stride, stream);
}

// The ssd_gemm_bf16 epilogue (bias, activation, residual) over S split-K partials.
SSD_API int ssd_gemm_finalize_bf16(const float* P, int64_t ldp, int64_t split_stride, int S, int M, int N, uint16_t* Y,
                                   int64_t ldy, const uint16_t* bias, int act, const uint16_t* residual, int64_t ldr,
                                   hipStream_t stream) {
  int rc = check_partials(P, ldp, split_stride, M, N);
  if (rc) return rc;
  if (!Y || S < 1 || M < 0 || N <= 0) return set_error(SSD_EINVAL, "gemm_finalize: null Y or bad S=%d M=%d N=%d", S, M, N);
  if (act < 0 || act > 3 || (residual && act)) return set_error(SSD_EINVAL, "gemm_finalize: bad activation %d", act);
  if (M == 0) return SSD_OK;
  GemmArgs a{};
  a.M = M; a.N = N; a.Y = Y; a.ldy = ldy; a.bias = bias; a.act = act; a.residual = residual; a.ldr = ldr;
  rc = launch_finalize<EPI_STORE>(a, P, ldp, split_stride, S, stream);
  return rc ? rc : check_launch("gemm_finalize");
}

// q/k/v RoPE + KV-cache write (as ssd_gemm_qkv_rope_bf16) over S split-K partials of the packed
// q/k/v projection.
SSD_API int ssd_qkv_rope_finalize_bf16(const float* P, int64_t ldp, int64_t split_stride, int S, int M, int heads,
                                       int kv_heads, int head_dim, const uint16_t* cos_tab, const uint16_t* sin_tab,
                                       int64_t rope_rows, const int32_t* row_pos, const int32_t* row_slot, uint16_t* Q,
                                       int64_t ldq, uint16_t* k_cache, uint16_t* vt_cache, int64_t max_len,
                                       hipStream_t stream) {
  const int N = (heads + 2 * kv_heads) * head_dim;
  int rc = check_partials(P, ldp, split_stride, M, N);
  if (rc) return rc;
  if (S < 1 || M < 0 || heads <= 0 || kv_heads <= 0) return set_error(SSD_EINVAL, "qkv_finalize: bad S/M/heads");
  if (head_dim % 32 || head_dim > 256) return set_error(SSD_EINVAL, "qkv_finalize: head_dim=%d unsupported", head_dim);
  if (max_len <= 0 || max_len % 64)
    return set_error(SSD_EINVAL, "qkv_finalize: max_len %lld not a multiple of 64", (long long)max_len);
  if (!Q || !k_cache || !vt_cache || !cos_tab || !sin_tab || !row_pos || !row_slot || rope_rows <= 0)
    return set_error(SSD_EINVAL, "qkv_finalize: null pointer or empty rope table");
  if (M == 0) return SSD_OK;
  GemmArgs a{};
  a.M = M; a.N = N; a.Y = Q; a.ldy = ldq; a.heads = heads; a.kv_heads = kv_heads; a.head_dim = head_dim;
  a.cos_tab = cos_tab; a.sin_tab = sin_tab; a.rope_rows = rope_rows; a.row_pos = row_pos; a.row_slot = row_slot;
  a.k_cache = k_cache; a.vt_cache = vt_cache; a.max_len = max_len;
  rc = launch_finalize<EPI_QKV>(a, P, ldp, split_stride, S, stream);
  return rc ? rc : check_launch("qkv_finalize");
}


// ------------------------------------------------------- residual projection
// Measured on MI355X at decode shapes (M = 25, weights streamed from HBM): a K <= 4096 projection
// (o_proj, bridge out_proj) is fastest as one direct GEMM with the residual add in its epilogue;
// a long-K projection (down_proj, K = intermediate) as split-K partials plus a finalize that only
// adds (the direct GEMM would re-read the long activation rows in every workgroup).
static bool residual_split(int N, int K) { return K > 4096; }

SSD_API int ssd_gemm_residual_group(int N, int K) {
  if (N <= 0 || K <= 0 || K % 32) {
    set_error(SSD_EINVAL, "residual_group: bad shape N=%d K=%d", N, K);
    return 0;
  }
  return residual_split(N, K) ? 1 : plan_for(N, K).nsub;
}

SSD_API int64_t ssd_gemm_residual_floats(int M, int N, int K) {
  if (M < 0 || N <= 0 || K <= 0 || K % 32) return -1;
  return residual_split(N, K) ? (int64_t)part_plan(N, K).S * M * ((N + 63) / 64 * 64) : 0;
}

SSD_API int ssd_gemm_residual_bf16(const uint16_t* X, int64_t ldx, int M, const uint16_t* W_packed, int N, int K,
                                   const uint16_t* bias, uint16_t* h, int64_t ldh, float* part, int64_t part_floats,
                                   hipStream_t stream) {
  int rc = check_common(X, ldx, M, W_packed, N, K);
  if (rc) return rc;
  if (!h) return set_error(SSD_EINVAL, "gemm_residual: null h");
  if (M == 0) return SSD_OK;
  GemmArgs a{};
  a.X = X; a.ldx = ldx; a.M = M; a.W = (const uint4*)W_packed; a.N = N; a.kb_total = K / 32;
  a.Y = h; a.ldy = ldh; a.bias = bias; a.residual = h; a.ldr = ldh;
  if (!residual_split(N, K)) return launch_gemm<EPI_STORE>(a, stream);
  const int64_t ldp = (N + 63) / 64 * 64;
  const int S = part_plan(N, K).S;
  if (part_floats < (int64_t)S * M * ldp)
    return set_error(SSD_EINVAL, "gemm_residual: scratch of %lld floats < %lld", (long long)part_floats,
                     (long long)S * M * ldp);
  if ((rc = check_partials(part, ldp, (int64_t)M * ldp, M, N))) return rc;
  if ((rc = launch_part(a, part, ldp, (int64_t)M * ldp, stream))) return rc;
  rc = launch_finalize<EPI_STORE>(a, part, ldp, (int64_t)M * ldp, S, stream);
  return rc ? rc : check_launch("gemm_residual");
}
