// Fused decoder MLP for decode-sized M on gfx950 (MI355X):
//
//   h <- h + down( silu(gate(RMSNorm(h))) * up(RMSNorm(h)) )
//
// as ONE launch of 256 workgroups (one per CU, all resident at once) in three phases, instead of
// three launches (gate/up, down partials, finalize). Each launch boundary costs 4-7 us of ramp-up
// and tail on this chip. Between phases there is no grid-wide barrier: a workgroup waits only for
// the workgroups whose output it reads (each publishes a per-call flag when a phase is done), and
// it issues the loads of its next phase's weight tiles (which do not depend on the previous
// phase) before it waits, so HBM keeps streaming while it waits.
//
//   phase 1  act = SwiGLU(RMSNorm(h) . Wgu^T). Workgroup b owns the T1 = I / 2048 gate/up tiles
//            [b T1, b T1 + T1) with the whole K; its 8 waves split K (TG1 tile groups of KS1
//            waves). Wgu is packed with group T1 so a workgroup streams one contiguous region.
//   phase 2  P[s] = act[:, K_s] . Wd[:, K_s]^T: workgroup b = (group b % G, split b / G) as
//            gemm_part_kernel (8 waves x one down tile each, activations staged in LDS).
//            It waits for the phase-1 workgroups that produced act columns K_s.
//   phase 3  h = rbf(h + rbf(sum_s P[s])), s = 0..S-1 in order (gemm_finalize_kernel's order):
//            workgroup (g, s) adds up its group's 8 tiles for rows m = s mod S, after waiting for
//            the S workgroups (g, 0..S-1).
//
// Cross-phase data (act, P) moves between XCDs, whose L2s are not coherent with each other. It
// is written with device-scope stores (write-through past L2), and every wave waits for its
// stores (vmcnt 0) before its workgroup publishes its flag; flags are written and polled with
// device-scope accesses. The consumers read the data with plain loads, through their L2: the
// kernel starts with invalidated caches and no workgroup touches a line of act or P before the
// workgroups that write every byte of that line have published their flags (each down split's
// act columns and each partial row segment are whole 128-byte lines, checked on the host), so
// the first read of a line in an XCD fetches the written data and later reads share it. No
// agent-scope fence is used (that would write back and invalidate every L2).
//
// Flags: every call advances each workgroup's flag by 2: sync[b] = F + 1 once workgroup b finished
// phase 1, F + 2 after phase 2, where F is the value sync[b] held when the call started (2 E for the
// E-th call on a zeroed buffer, modulo 2^32). Only workgroup b writes sync[b], so it reads F at
// its start without a race, and since every call leaves all flags equal, F is every producer's
// start value too. Waits compare for equality, so a flag left by the previous call (F) never
// matches. The call count lives in the flags themselves, not in a host counter baked into the
// kernel arguments, so a launch captured in a HIP graph stays correct on every replay. Every wait
// is bounded; one that gives up counts a timeout in sync[MLP_WGS + 1] and lets the workgroup go
// on (its results are then wrong, and the count says so; the host reads the count and fails the
// call's results). The waits need all 256 workgroups resident at once: one per CU (123 KiB of LDS
// each).
//
// The order of every sum depends only on (I, H): results are batch-invariant (a row computed
// alone equals the same row inside a 64-row batch).
#include "common.h"

#include <mutex>
#include <unordered_map>

namespace ssd {

constexpr int MLP_WGS = 256;                    // workgroups (one per CU), fixed: the plan depends on it
constexpr int MLP_THREADS = 512;                // 8 waves
constexpr int MLP_SYNC_WORDS = MLP_WGS + 64;    // flags [0, 256), timeouts [257]
constexpr uint32_t MLP_SPIN_LIMIT = 1u << 21;   // polls before a barrier gives up (~seconds)
constexpr int MLP_RED_FLOATS = 30464;           // phase-1 reduction buffer (119 KiB of LDS)
constexpr int MLP_DEAL = 2;                     // phase-1 k-blocks dealt to a wave at a time

struct MlpArgs {
  const bf16_t* h_in;  // phase-1 input rows and phase-3 residual (may equal h_out)
  bf16_t* h_out;
  int64_t ldh;
  int M;
  const u32x4_t* wgu;  // packed gate/up, group T1
  const u32x4_t* wd;   // packed down, group 1
  int hidden, inter;
  float eps;
  bf16_t* act;         // [M, lda]
  int64_t lda;
  float* part;         // [S][M][ldp]
  int64_t ldp, sstride;
  int groups;          // down: hidden / 128 tile groups; groups * S == MLP_WGS
  uint32_t* sync;
};

// Publish this workgroup's flag: every wave has waited for its own cross-phase stores
// (wait_vmem) before the workgroup barrier, so the data is visible device-wide before the flag.
__device__ __forceinline__ void publish_flag(uint32_t* sync, uint32_t value) {
  __syncthreads();
  if (threadIdx.x == 0) st_agent_u32(&sync[blockIdx.x], value);
}

// Wave-level wait (call from one whole wave) until each of flags [b0, b0 + n) equals v1 or v2.
// Bounded: gives up after MLP_SPIN_LIMIT polls and counts a timeout.
__device__ __forceinline__ void wait_flags(uint32_t* sync, int b0, int n, uint32_t v1, uint32_t v2) {
  const int lane = threadIdx.x & 63;
  uint32_t spins = 0;
  for (;;) {
    bool done = true;
    for (int b = lane; b < n; b += 64) {
      const uint32_t f = ld_agent_u32(&sync[b0 + b]);
      done &= f == v1 || f == v2;
    }
    if (__all(done)) return;
    if (++spins >= MLP_SPIN_LIMIT) {
      if (lane == 0) __hip_atomic_fetch_add(&sync[MLP_WGS + 1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// Wave-level wait until the flags of workgroups b0 + k * stride, k < n, equal `value`.
__device__ __forceinline__ void wait_flags_strided(uint32_t* sync, int b0, int stride, int n, uint32_t value) {
  const int lane = threadIdx.x & 63;
  uint32_t spins = 0;
  for (;;) {
    bool done = true;
    for (int k = lane; k < n; k += 64) done &= ld_agent_u32(&sync[b0 + k * stride]) == value;
    if (__all(done)) return;
    if (++spins >= MLP_SPIN_LIMIT) {
      if (lane == 0) __hip_atomic_fetch_add(&sync[MLP_WGS + 1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

__device__ __forceinline__ float mlp_sumsq8(u32x4_t v) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float lo = __uint_as_float(v[i] << 16), hi = __uint_as_float(v[i] & 0xffff0000u);
    s = fmaf(lo, lo, s);
    s = fmaf(hi, hi, s);
  }
  return s;
}

template <int CT, int NS1>
struct MlpCfg {
  static constexpr int SC0 = MLP_RED_FLOATS / (MLP_THREADS / 64 * CT * 4 * 68);
  static constexpr int SC = SC0 < NS1 ? SC0 : NS1;        // sub-tiles reduced per LDS pass
  static constexpr int KC = CT <= 2 ? 16 : 8;             // phase-2 k-blocks per activation pass
  static constexpr int XCH = KC * CT * 64;                // 16-byte activation chunks per pass
  static constexpr int XIT = XCH / MLP_THREADS;           // per thread
  static_assert(XCH % MLP_THREADS == 0, "activation pass must split evenly over the threads");
};

template <int CT, int NS1>
union MlpLds {
  struct {
    float red[MLP_THREADS / 64][MlpCfg<CT, NS1>::SC][CT][4][68];
    float ss[MLP_THREADS / 64][CT][16];
    float rn[CT * 16];
  } p1;
  u32x4_t xs[MlpCfg<CT, NS1>::XCH];
};

// CT: 16-row column tiles of M; NS1 x TG1: gate/up tiles per workgroup (TG1 groups of 8 / TG1
// waves); S: down splits.
template <int CT, int NS1, int TG1, int S>
__global__ __launch_bounds__(MLP_THREADS) void mlp_kernel(MlpArgs a) {
  constexpr int KS1 = 8 / TG1;
  constexpr int T1 = NS1 * TG1;
  constexpr int U1 = CT == 1 ? 4 : CT == 2 ? 2 : 1;
  using Cfg = MlpCfg<CT, NS1>;
  constexpr int SC = Cfg::SC, KC = Cfg::KC, XIT = Cfg::XIT;
  __shared__ MlpLds<CT, NS1> lds;

  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int Mv = a.M < CT * 16 ? a.M : CT * 16;
  const uint32_t flag0 = ld_agent_u32(&a.sync[blockIdx.x]);  // all flags hold this value now
  const uint32_t flag1 = flag0 + 1u, flag2 = flag0 + 2u;

  // ---------------------------------------------------------------- phase 1: gate/up + SwiGLU
  {
    const int tg = w / KS1, kw = w % KS1;
    const int kbt = a.hidden >> 5;
    f32x4_t acc[NS1][CT];
#pragma unroll
    for (int s = 0; s < NS1; ++s)
#pragma unroll
      for (int c = 0; c < CT; ++c) acc[s][c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    float ss[CT];
#pragma unroll
    for (int c = 0; c < CT; ++c) ss[c] = 0.f;
    const u32x4_t* wp = a.wgu + ((size_t)blockIdx.x * kbt * T1 + tg * NS1) * 64 + lane;
    const bf16_t* xp[CT];
#pragma unroll
    for (int c = 0; c < CT; ++c) xp[c] = a.h_in + (size_t)min(c * 16 + j, a.M - 1) * a.ldh + g * 8;

    // The wave's k-blocks: pairs dealt round-robin to the KS1 waves (pair i to wave i % KS1), so
    // the waves stream neighbouring weight regions at the same time and finish together; the
    // k-blocks left after whole rounds go one by one. The sequence depends on the shape only
    // (never on M), and each wave accumulates it in order.
    const int n_full = (kbt / (KS1 * MLP_DEAL)) * MLP_DEAL;  // this wave's k-blocks in whole rounds
    auto kb_at = [&](int t) { return ((t / MLP_DEAL) * KS1 + kw) * MLP_DEAL + t % MLP_DEAL; };
    int t = 0;
    for (; t + U1 <= n_full; t += U1) {
      u32x4_t wr[U1][NS1], xr[U1][CT];
#pragma unroll
      for (int u = 0; u < U1; ++u) {
        const int kb = kb_at(t + u);
#pragma unroll
        for (int s = 0; s < NS1; ++s) wr[u][s] = __builtin_nontemporal_load(wp + ((size_t)kb * T1 + s) * 64);
      }
#pragma unroll
      for (int u = 0; u < U1; ++u) {
        const int kb = kb_at(t + u);
#pragma unroll
        for (int c = 0; c < CT; ++c) xr[u][c] = *(const u32x4_t*)(xp[c] + kb * 32);
      }
      __builtin_amdgcn_sched_barrier(0);  // every load of the trip ahead of its MFMAs
#pragma unroll
      for (int u = 0; u < U1; ++u)
#pragma unroll
        for (int s = 0; s < NS1; ++s)
#pragma unroll
          for (int c = 0; c < CT; ++c)
            acc[s][c] = mfma16x16x32(bits_bf16x8(wr[u][s]), bits_bf16x8(xr[u][c]), acc[s][c]);
#pragma unroll
      for (int u = 0; u < U1; ++u)
#pragma unroll
        for (int c = 0; c < CT; ++c) ss[c] += mlp_sumsq8(xr[u][c]);
    }
    // the rest of the whole rounds, then the leftover k-blocks (kb = rounds end + kw + KS1 i)
    const int kb_rest = (kbt / (KS1 * MLP_DEAL)) * KS1 * MLP_DEAL + kw;
    for (int tt = t;; ++tt) {
      const int kb = tt < n_full ? kb_at(tt) : kb_rest + (tt - n_full) * KS1;
      if (kb >= kbt) break;
      u32x4_t wr[NS1], xr[CT];
#pragma unroll
      for (int s = 0; s < NS1; ++s) wr[s] = __builtin_nontemporal_load(wp + ((size_t)kb * T1 + s) * 64);
#pragma unroll
      for (int c = 0; c < CT; ++c) xr[c] = *(const u32x4_t*)(xp[c] + kb * 32);
#pragma unroll
      for (int s = 0; s < NS1; ++s)
#pragma unroll
        for (int c = 0; c < CT; ++c) acc[s][c] = mfma16x16x32(bits_bf16x8(wr[s]), bits_bf16x8(xr[c]), acc[s][c]);
#pragma unroll
      for (int c = 0; c < CT; ++c) ss[c] += mlp_sumsq8(xr[c]);
    }

    // Per-wave sums of x^2 (the 4 k-groups of the wave), then the row scale from tile group 0's
    // waves in order.
#pragma unroll
    for (int c = 0; c < CT; ++c) {
      float v = ss[c];
      v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 32);
      if (g == 0) lds.p1.ss[w][c][j] = v;
    }
    // Sub-tiles in passes of SC through LDS: wave w's partial of sub-tile s, then the epilogue
    // sums the KS1 waves of each tile group in order. Thread item: (tile group, sub-tile, row m,
    // column pair q) -> intermediate columns 2q, 2q + 1 of the tile (gate rows 2q, 2q + 1, up
    // rows 2q + 8, 2q + 9), stored as one 4-byte device-scope store.
#pragma unroll
    for (int s0 = 0; s0 < NS1; s0 += SC) {
      const int nsc = NS1 - s0 < SC ? NS1 - s0 : SC;
#pragma unroll
      for (int s = 0; s < NS1; ++s)
        if (s >= s0 && s < s0 + SC)
#pragma unroll
          for (int c = 0; c < CT; ++c)
#pragma unroll
            for (int e = 0; e < 4; ++e) lds.p1.red[w][s - s0][c][e][lane] = acc[s][c][e];
      __syncthreads();
      if (s0 == 0) {
        if ((int)threadIdx.x < CT * 16) {
          const int c = threadIdx.x >> 4, jj = threadIdx.x & 15;
          float v = lds.p1.ss[0][c][jj];
#pragma unroll
          for (int ww = 1; ww < KS1; ++ww) v += lds.p1.ss[ww][c][jj];
          lds.p1.rn[threadIdx.x] = rsqrtf(v / (float)a.hidden + a.eps);
        }
        __syncthreads();
      }
      const int items = TG1 * nsc * 4 * Mv;
      for (int o = threadIdx.x; o < items; o += MLP_THREADS) {
        const int q = o & 3;
        int rest = o >> 2;
        const int m = rest % Mv;
        rest /= Mv;
        const int sl = rest % nsc, gi = rest / nsc;
        const int c = m >> 4;
        auto val = [&](int r) -> float {
          const int ln = (m & 15) + 16 * (r >> 2), e = r & 3;
          float v = lds.p1.red[gi * KS1][sl][c][e][ln];
#pragma unroll
          for (int ww = 1; ww < KS1; ++ww) v += lds.p1.red[gi * KS1 + ww][sl][c][e][ln];
          return v * lds.p1.rn[m];
        };
        const float g0 = val(2 * q), g1 = val(2 * q + 1), u0 = val(2 * q + 8), u1 = val(2 * q + 9);
        const float a0 = rbf(silu_f(rbf(g0))) * rbf(u0);
        const float a1 = rbf(silu_f(rbf(g1))) * rbf(u1);
        const int nb = blockIdx.x * T1 + gi * NS1 + s0 + sl;
        st_agent_u32((uint32_t*)(a.act + (size_t)m * a.lda + nb * 8 + 2 * q), pack_bf16x2(a0, a1));
      }
      __syncthreads();  // the next pass overwrites red
    }
  }
  wait_vmem();  // this wave's act stores are complete before its workgroup arrives

  // ---------------------------------------------------------------- phase 2: down partials
  const int grp = blockIdx.x % a.groups, split = blockIdx.x / a.groups;
  const int kbt2 = a.inter >> 5;
  const int kb0 = (kbt2 * split) / S, kb1 = (kbt2 * (split + 1)) / S;
  const int tile2 = grp * 8 + w;
  const u32x4_t* wp2 = a.wd + (size_t)tile2 * kbt2 * 64 + lane;
  f32x4_t acc2[CT];
#pragma unroll
  for (int c = 0; c < CT; ++c) acc2[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  u32x4_t xv[XIT], wr2[KC];
  auto load_w = [&](int c0, int nk, u32x4_t (&wo)[KC]) {
#pragma unroll
    for (int u = 0; u < KC; ++u) wo[u] = __builtin_nontemporal_load(wp2 + (size_t)(c0 + min(u, nk - 1)) * 64);
  };
  auto load_x = [&](int c0, int nk, u32x4_t (&xo)[XIT]) {
    const int nx = nk * CT * 64;
#pragma unroll
    for (int it = 0; it < XIT; ++it) {
      const int idx = min((int)threadIdx.x + it * MLP_THREADS, nx - 1);
      const int kb = idx / (CT * 64), rem = idx % (CT * 64);
      const int m = min(rem >> 2, a.M - 1);
      xo[it] = *(const u32x4_t*)(a.act + (size_t)m * a.lda + (size_t)(c0 + kb) * 32 + (rem & 3) * 8);
    }
  };
  int c0 = kb0;
  int nk = min(KC, kb1 - c0);
  publish_flag(a.sync, flag1);
  // The first pass's weights stream while this workgroup waits for the phase-1 workgroups that
  // produced act columns [32 kb0, 32 kb1) (8 T1 columns each); wave 0 polls, and issues its own
  // weight loads after polling (its polls wait for every load the wave has in flight).
  if (w != 0) load_w(c0, nk, wr2);
  if (w == 0) {
    const int p0 = (kb0 * 32) / (8 * T1), p1 = (kb1 * 32 - 1) / (8 * T1);
    wait_flags(a.sync, p0, p1 - p0 + 1, flag1, flag2);  // a producer may be past phase 2 already
    load_w(c0, nk, wr2);
  }
  __syncthreads();
  load_x(c0, nk, xv);
  while (nk > 0) {
    __syncthreads();  // the previous pass's readers are done with xs
#pragma unroll
    for (int it = 0; it < XIT; ++it) {
      const int idx = threadIdx.x + it * MLP_THREADS;
      if (idx < nk * CT * 64) lds.xs[idx] = xv[it];
    }
    __syncthreads();
    const int c1 = c0 + nk;
    const int nk1 = min(KC, kb1 - c1);
    u32x4_t wn[KC];
    if (nk1 > 0) {
      load_x(c1, nk1, xv);
      load_w(c1, nk1, wn);
    }
#pragma unroll
    for (int u = 0; u < KC; ++u) {
      if (u < nk) {
        u32x4_t xr[CT];
#pragma unroll
        for (int c = 0; c < CT; ++c) xr[c] = lds.xs[(u * CT * 16 + c * 16 + j) * 4 + g];
#pragma unroll
        for (int c = 0; c < CT; ++c) acc2[c] = mfma16x16x32(bits_bf16x8(wr2[u]), bits_bf16x8(xr[c]), acc2[c]);
      }
    }
#pragma unroll
    for (int u = 0; u < KC; ++u) wr2[u] = wn[u];
    c0 = c1;
    nk = nk1;
  }
  // lane (j, g) holds rows n = 16 tile2 + 4g + e of column m = 16c + j
#pragma unroll
  for (int c = 0; c < CT; ++c) {
    const int m = c * 16 + j;
    if (m < a.M) {
      float* p = a.part + split * a.sstride + (size_t)m * a.ldp + tile2 * 16 + 4 * g;
      st_agent_u64((uint64_t*)p, ((uint64_t)__float_as_uint(acc2[c][1]) << 32) | __float_as_uint(acc2[c][0]));
      st_agent_u64((uint64_t*)p + 1, ((uint64_t)__float_as_uint(acc2[c][3]) << 32) | __float_as_uint(acc2[c][2]));
    }
  }
  wait_vmem();

  // ---------------------------------------------------------------- phase 3: h += sum_s P[s]
  // Workgroup (grp, split) finishes its group's 8 tiles for rows m = split, split + S, ...;
  // thread item (row, tile, pair r): outputs 16 tile + r and 16 tile + r + 8, summed over the S
  // splits in order as gemm_finalize_kernel does. The first item's residual is loaded before
  // the wait.
  publish_flag(a.sync, flag2);
  const int rows = (a.M - split + S - 1) / S;  // rows m = split + S i < M
  const int items = rows * 64;
  int it = threadIdx.x;
  float res_lo, res_hi;
  auto item_at = [&](int i, int& m, int& n) {
    m = split + S * (i >> 6);
    n = (grp * 8 + ((i >> 3) & 7)) * 16 + (i & 7);
  };
  {
    int m, n;
    item_at(min(it, max(items - 1, 0)), m, n);
    m = min(m, a.M - 1);
    res_lo = bf2f(a.h_in[(size_t)m * a.ldh + n]);
    res_hi = bf2f(a.h_in[(size_t)m * a.ldh + n + 8]);
  }
  if (w == 0) wait_flags_strided(a.sync, grp, a.groups, S, flag2);
  __syncthreads();
  for (bool first = true; it < items; it += MLP_THREADS, first = false) {
    int m, n;
    item_at(it, m, n);
    const float* p = a.part + (size_t)m * a.ldp + n;
    float lo[S], hi[S];
#pragma unroll
    for (int s = 0; s < S; ++s) {
      lo[s] = p[s * a.sstride];
      hi[s] = p[s * a.sstride + 8];
    }
    if (!first) {
      res_lo = bf2f(a.h_in[(size_t)m * a.ldh + n]);
      res_hi = bf2f(a.h_in[(size_t)m * a.ldh + n + 8]);
    }
    float vlo = lo[0], vhi = hi[0];
#pragma unroll
    for (int s = 1; s < S; ++s) {
      vlo += lo[s];
      vhi += hi[s];
    }
    a.h_out[(size_t)m * a.ldh + n] = f2bf(rbf(res_lo + rbf(vlo)));
    a.h_out[(size_t)m * a.ldh + n + 8] = f2bf(rbf(res_hi + rbf(vhi)));
  }
}

struct MlpPlan {
  int ns1, tg1, S, groups;  // ns1 == 0: no fused plan for this shape
};

// Fused plans exist for shapes whose work splits evenly over 256 workgroups: I / 2048 gate/up
// tiles per workgroup and (hidden / 128) x S down workgroups; the down split count S is the
// one the split-K path uses for (hidden, I) (a function of the shape only).
static MlpPlan mlp_plan(int inter, int hidden) {
  MlpPlan p{0, 0, 0, 0};
  if (inter <= 4096 || inter % 2048 || hidden % 128 || hidden < 128) return p;
  const int t1 = inter / 2048;
  const int groups = hidden / 128;
  const int kbt = inter / 32;
  int S = 1;
  while (groups * S < MLP_WGS && S * 2 * 8 <= kbt && S < 16) S *= 2;
  if (groups * S != MLP_WGS) return p;
  if (t1 == 4 && S == 16) p = MlpPlan{4, 1, 16, groups};
  else if (t1 == 7 && S == 8) p = MlpPlan{7, 1, 8, groups};
  else if (t1 == 14 && S == 4) p = MlpPlan{7, 2, 4, groups};
  return p;
}

template <int NS1, int TG1, int S>
static hipError_t launch_mlp_ct(int ct, const MlpArgs& a, hipStream_t s) {
  const dim3 grid(MLP_WGS), block(MLP_THREADS);
  switch (ct) {
    case 1: SSD_LAUNCH((mlp_kernel<1, NS1, TG1, S>), grid, block, 0, s, a); break;
    case 2: SSD_LAUNCH((mlp_kernel<2, NS1, TG1, S>), grid, block, 0, s, a); break;
    case 3: SSD_LAUNCH((mlp_kernel<3, NS1, TG1, S>), grid, block, 0, s, a); break;
    default: SSD_LAUNCH((mlp_kernel<4, NS1, TG1, S>), grid, block, 0, s, a); break;
  }
  return hipGetLastError();
}

// The waits between workgroups need all MLP_WGS workgroups resident at once (one per CU): checked
// once per (device, kernel instantiation) from the CU count and that instantiation's occupancy.
// (A cooperative launch would guarantee it too, but costs ~17 us more per launch on this runtime.)
static int check_residency(int dev, const void* fn) {
  static std::mutex mu;
  static std::unordered_map<uint64_t, int> ok;
  std::lock_guard<std::mutex> lock(mu);
  const uint64_t key = ((uint64_t)(uint32_t)dev << 48) ^ (uint64_t)(uintptr_t)fn;
  auto it = ok.find(key);
  if (it != ok.end()) return it->second;
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, MLP_THREADS, 0) != hipSuccess)
    return set_error(SSD_EHIP, "mlp: cannot query device %d", dev);
  const int rc = (int64_t)cus * per_cu >= MLP_WGS
                     ? SSD_OK
                     : set_error(SSD_ERANGE, "mlp: device %d holds %d x %d workgroups at once, needs %d", dev, cus,
                                 per_cu, MLP_WGS);
  ok[key] = rc;
  return rc;
}

template <int NS1, int TG1, int S>
static const void* mlp_fn(int ct) {
  switch (ct) {
    case 1: return (const void*)mlp_kernel<1, NS1, TG1, S>;
    case 2: return (const void*)mlp_kernel<2, NS1, TG1, S>;
    case 3: return (const void*)mlp_kernel<3, NS1, TG1, S>;
    default: return (const void*)mlp_kernel<4, NS1, TG1, S>;
  }
}

static const void* mlp_fn_for(const MlpPlan& p, int ct) {
  if (p.ns1 == 4) return mlp_fn<4, 1, 16>(ct);
  if (p.tg1 == 1) return mlp_fn<7, 1, 8>(ct);
  return mlp_fn<7, 2, 4>(ct);
}

}  // namespace ssd

using namespace ssd;

SSD_API int ssd_mlp_group(int inter, int hidden) {
  const MlpPlan p = mlp_plan(inter, hidden);
  return p.ns1 * p.tg1;
}

SSD_API int64_t ssd_mlp_sync_words(void) { return MLP_SYNC_WORDS; }

SSD_API int ssd_mlp_timeout_word(void) { return MLP_WGS + 1; }

SSD_API int ssd_mlp_bf16(uint16_t* h, int64_t ldh, int M, const uint16_t* wgu, const uint16_t* wd, int inter,
                         int hidden, float eps, uint16_t* act, int64_t lda, float* part, int64_t part_floats,
                         uint32_t* sync, hipStream_t stream) {
  const MlpPlan p = mlp_plan(inter, hidden);
  if (!p.ns1) return set_error(SSD_EINVAL, "mlp: no fused plan for inter=%d hidden=%d", inter, hidden);
  if (!h || !wgu || !wd || !act || !part || !sync) return set_error(SSD_EINVAL, "mlp: null pointer");
  if (M < 0) return set_error(SSD_EINVAL, "mlp: M=%d", M);
  if (((uintptr_t)h & 15) || ldh % 8 || ldh < hidden)
    return set_error(SSD_EINVAL, "mlp: h must be 16-byte aligned with ldh %% 8 == 0 and ldh >= hidden");
  if (((uintptr_t)act & 15) || lda % 8 || lda < inter)
    return set_error(SSD_EINVAL, "mlp: act must be 16-byte aligned with lda %% 8 == 0 and lda >= inter");
  if (((uintptr_t)wgu & 15) || ((uintptr_t)wd & 15) || ((uintptr_t)part & 15) || ((uintptr_t)sync & 3))
    return set_error(SSD_EINVAL, "mlp: misaligned weights, partials or sync words");
  if (!(eps > 0.f)) return set_error(SSD_EINVAL, "mlp: eps must be > 0");
  // consumers read act and P through L2: every line they read must be written by the
  // workgroups they wait for (whole 128-byte lines per down split and per partial segment)
  if (((uintptr_t)act & 127) || lda % 64 || (inter / p.S) % 64 || ((uintptr_t)part & 127))
    return set_error(SSD_EINVAL, "mlp: act and part must be 128-byte aligned with lda %% 64 == 0");
  const int64_t ldp = (hidden + 63) / 64 * 64;
  const int mc = M < 64 ? M : 64;
  if (part_floats < (int64_t)p.S * mc * ldp)
    return set_error(SSD_EINVAL, "mlp: partials of %lld floats < %lld", (long long)part_floats,
                     (long long)p.S * mc * ldp);
  if (M == 0) return SSD_OK;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return set_error(SSD_EHIP, "mlp: no current device");
  for (int m0 = 0; m0 < M; m0 += 64) {
    const int mc0 = M - m0 < 64 ? M - m0 : 64;
    if (int rc = check_residency(dev, mlp_fn_for(p, (mc0 + 15) / 16))) return rc;
  }
  for (int m0 = 0; m0 < M; m0 += 64) {
    MlpArgs a{};
    a.M = M - m0 < 64 ? M - m0 : 64;
    a.h_in = h + (size_t)m0 * ldh;
    a.h_out = h + (size_t)m0 * ldh;
    a.ldh = ldh;
    a.wgu = (const u32x4_t*)wgu;
    a.wd = (const u32x4_t*)wd;
    a.hidden = hidden;
    a.inter = inter;
    a.eps = eps;
    a.act = act + (size_t)m0 * lda;
    a.lda = lda;
    a.part = part;
    a.ldp = ldp;
    a.sstride = (int64_t)a.M * ldp;
    a.groups = p.groups;
    a.sync = sync;
    const int ct = (a.M + 15) / 16;
    hipError_t e;
    if (p.ns1 == 4) e = launch_mlp_ct<4, 1, 16>(ct, a, stream);
    else if (p.tg1 == 1) e = launch_mlp_ct<7, 1, 8>(ct, a, stream);
    else e = launch_mlp_ct<7, 2, 4>(ct, a, stream);
    if (e != hipSuccess) return set_error(SSD_EHIP, "mlp: launch failed: %s", hipGetErrorString(e));
  }
  return SSD_OK;
}
