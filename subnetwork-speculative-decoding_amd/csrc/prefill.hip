// Prefill on gfx950: the target forward over a long prompt chunk (hundreds to thousands of rows),
// where every projection is a compute-bound GEMM and attention is causal.
//
// The decode kernels stream each weight once per call and suit M <= 64 rows; a 4096-token prompt
// through them re-reads every weight 64 times. Here (reference ssd/engine/speculative.py:149-151,
// the target's forward over the prompt):
//
// * prefill_gemm_kernel: Y = X W^T over the same packed weights as the decode GEMMs (16 x 32
//   MFMA A-operand tiles, any tile grouping), as an LDS-tiled MFMA GEMM: a workgroup of 8 waves
//   (one per CU, two per SIMD) owns a 256 (N) x 128 (M) output tile, stages 256 x 64 of W and
//   128 x 64 of X per step in LDS (double buffered, the next step's global loads in flight while the
//   MFMAs run), and each wave computes a 64 x 64 sub-tile with v_mfma_f32_16x16x32_bf16 (against
//   two 4-wave 128 x 128 workgroups per CU, a quarter fewer bytes staged per MFMA). X is staged in the MFMA B-operand lane order so
//   every LDS read is one contiguous 1 KiB per wave. The decode epilogues run on the accumulators:
//   the folded RMSNorm scale (sum of x^2 accumulated by the threads that stage X), RoPE + KV-cache
//   write for q/k/v, SwiGLU for gate/up (rotary / gate-up row pairs r and r + 8 meet through one
//   v_permlane32_swap), residual add for o and down. The launch is persistent and XCD-aware: the
//   workgroups resident on one XCD sweep blocks of output tiles together, so the weight and
//   activation tiles they share are fetched into that XCD's L2 once per block.
// * prefill_gemm4_kernel: the plain and SwiGLU projections (o, down, gate/up) on one 4-wave
//   workgroup per CU with a 256 x 256 output tile and 128 x 128 per wave (accumulators pinned to
//   the accumulator registers), operands loaded straight into a five-slot LDS ring, outputs staged
//   through LDS and stored as whole rows; q/k/v stays on prefill_gemm_kernel.
// * prefill_attention_kernel: causal flash attention, one wave per (q head, 32 tokens), K/V read
//   in the cache's 64-slot MFMA-operand blocks; S^T = K Q^T and O^T = V^T P^T on MFMA with the
//   running max / sum rescaled per 64-key block.
// * ssd_prefill: the whole target forward for one chunk of prompt rows in one C call.
//
// Prefill rows are not required to be bit-identical to the same rows decoded one by one: greedy
// speculative decoding and greedy autoregressive decoding both start from the same prefill, and
// the decode kernels keep their batch invariance among themselves.
#include "gemm_epi.h"

#include <math.h>

#include <type_traits>

namespace ssd {

constexpr int PF_WN = 4;    // waves along N (x 2 along M): 64 * PF_WN = 256 output rows of W per workgroup
constexpr int PF_BM = 128;  // tokens per workgroup
constexpr int PF_KB = 2;    // 32-wide k-blocks per pipeline step

// Tile (nb, kb) of a packed weight with `group` row tiles per k-block group: 64 lanes x 16 B.
__device__ __forceinline__ size_t packed_tile(int nb, int kb, int kbt, int group) {
  return ((size_t)(nb / group) * kbt + kb) * group + nb % group;
}

// Epilogue of one 16 x 16 accumulator tile: lane (g, j) holds rows n = 16 nb + 4 g + e of token m
// (scaled by the folded RMSNorm factor sc). Every lane must call it (the q/k/v and SwiGLU pairs meet
// through a cross-lane swap).
template <int EPI>
__device__ __forceinline__ void pf_tile_epilogue(const GemmArgs& a, const f32x4_t& acc, int nb, int m, float sc,
                                                 int g, int pos0) {
  const bool mv = m < a.M;
  float v[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = acc[e] * sc;
  if constexpr (EPI == EPI_STORE) {
    const int n = nb * 16 + 4 * g;
    if (mv) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (n + e < a.N) {
          float r = rbf(v[e]);
          if (a.residual) r = rbf(bf2f(a.residual[(size_t)m * a.ldr + n + e]) + r);
          a.Y[(size_t)m * a.ldy + n + e] = f2bf(r);
        }
    }
  } else {
    // rows r (lanes g < 2) and r + 8 (lanes g >= 2) of the tile meet: r[0] = the lower
    // half's value, r[1] = the upper half's, on every lane
    float lo[4], hi[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[e]), __float_as_uint(v[e]), false, false);
      lo[e] = __uint_as_float(p[0]);
      hi[e] = __uint_as_float(p[1]);
    }
    if (mv && g < 2 && nb * 16 < a.N) {
      if constexpr (EPI == EPI_SWIGLU) {
#pragma unroll
        for (int e = 0; e < 4; ++e) epi_swiglu(a, nb * 8 + 4 * g + e, m, lo[e], hi[e]);
      } else {
        const QkvTile q = qkv_tile(a, nb);
        const int pos = min(max(pos0 + m, 0), (int)a.rope_rows - 1), half = a.head_dim >> 1;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int pr = 4 * g + e;
          const size_t at = (size_t)pos * half + q.p * 8 + pr;
          epi_qkv_pre(a, q, m, pr, lo[e], hi[e], pos0 + m, bf2f(a.cos_tab[at]), bf2f(a.sin_tab[at]), 0);
        }
      }
    }
  }
}

template <int EPI, int NORM>
__global__ __launch_bounds__(128 * PF_WN, 4 / PF_WN) void prefill_gemm_kernel(GemmArgs a, int group, int n_mt,
                                                                              int n_nt, int pos0, int sb_n, int sb_m) {
  constexpr int WN = PF_WN;
  constexpr int NT = 128 * WN;   // threads
  constexpr int RT = 4 * WN;     // 16-row tiles of W per workgroup
  constexpr int XL = 8 / WN;     // X chunks each thread stages per step
  __shared__ u32x4_t As[2][PF_KB][RT][64];
  __shared__ u32x4_t Bs[2][PF_KB][8][64];
  __shared__ float rn_s[PF_BM];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int wn = w % WN, wm = w / WN;
  const int n_rt = (a.N + 127) / 128 * 8;  // row tiles of the packed weight (rows padded to 128)
  const int kbt = a.kb_total;

  // Persistent, XCD-aware schedule: the workgroups resident on one XCD (ids x, x + 8, ...) sweep
  // blocks of sb_n x sb_m output tiles together -- workgroup j takes tile (j % sb_n, j / sb_n)
  // of the block -- so each weight tile is read by sb_m and each activation tile by sb_n
  // workgroups that run in step through K, and the block's k slices stay in that XCD's L2.
  // Blocks are dealt to the 8 XCDs round-robin, M-fastest (consecutive blocks of an XCD keep
  // their activation band).
  const int xcd = blockIdx.x % 8, jw = blockIdx.x / 8;
  const int n_bn = (n_nt + sb_n - 1) / sb_n, n_bm = (n_mt + sb_m - 1) / sb_m;
  for (int blk = xcd; blk < n_bn * n_bm; blk += 8) {
  const int bn = (blk / n_bm) * sb_n + jw % sb_n, bm = (blk % n_bm) * sb_m + jw / sb_n;
  if (bn >= n_nt || bm >= n_mt || jw >= sb_n * sb_m) continue;  // uniform per workgroup
  const int nb0 = bn * RT, m0 = bm * PF_BM;

  // Staging assignment: 512 WN 16-byte chunks of W and 1024 of X per step, 4 and XL per thread.
  // W chunk i: k-block i / (64 RT) of the step, row tile (i >> 6) % RT, lane i & 63 (one tile =
  // 1 KiB; row tiles past the weight's last load that one, their outputs are never stored).
  // X: a wave's load covers 8 rows x the step's 8 16-byte columns (whole 128-byte lines); thread
  // t, load r: row 8 (t >> 6) + 16 WN r + (t & 7), column c = lane >> 3 (k-block c >> 2, B-operand
  // lane group c & 3). The 8 lanes that the LDS serves together hold 8 consecutive rows of one
  // column: 8 consecutive 16-byte slots of the operand layout, free of bank conflicts.
  const u32x4_t* W = (const u32x4_t*)a.W;
  size_t wbase[4];
  int wkb[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int i = t + NT * r;
    wkb[r] = i / (64 * RT);
    const int nb = min(nb0 + ((i >> 6) % RT), n_rt - 1);
    wbase[r] = packed_tile(nb, 0, kbt, group) * 64 + (i & 63);
  }
  const int xc = lane >> 3;
  auto xrow_of = [&](int r) { return (t >> 6) * 8 + 16 * WN * r + (t & 7); };
  const bf16_t* xrow[XL];
#pragma unroll
  for (int r = 0; r < XL; ++r) xrow[r] = a.X + (size_t)min(m0 + xrow_of(r), a.M - 1) * a.ldx + xc * 8;
  const int xkb = xc >> 2, xg = xc & 3;

  // Two register sets of staged chunks: a step's global loads are issued two compute steps before
  // they are written to LDS, so their latency is covered by two steps of MFMAs.
  struct Stage {
    u32x4_t a[4], b[XL];
  };
  Stage s0, s1;
  float ss[XL] = {};
  auto gload = [&](int st, Stage& r) {
    const int k0 = st * PF_KB;
#pragma unroll
    for (int i = 0; i < 4; ++i) r.a[i] = W[wbase[i] + (size_t)(k0 + wkb[i]) * group * 64];  // shared by sb_m workgroups: cached
#pragma unroll
    for (int i = 0; i < XL; ++i) r.b[i] = *(const u32x4_t*)(xrow[i] + (size_t)k0 * 32);
  };
  // real == false stores zeros (the padding step of an odd step count): a mask, not a branch,
  // so every path through the loop has the same loads in flight
  auto lstore = [&](int buf, const Stage& r, bool real) {
    const uint32_t keep = real ? 0xffffffffu : 0u;
#pragma unroll
    for (int i = 0; i < 4; ++i) (&As[buf][0][0][0])[t + NT * i] = r.a[i] & keep;
#pragma unroll
    for (int i = 0; i < XL; ++i) {
      const int row = xrow_of(i);
      Bs[buf][xkb][row >> 4][xg * 16 + (row & 15)] = r.b[i] & keep;
    }
    if constexpr (NORM) {
      if (real) {
#pragma unroll
        for (int i = 0; i < XL; ++i) ss[i] += sumsq8(r.b[i]);
      }
    }
  };

  f32x4_t acc[4][4];
#pragma unroll
  for (int x = 0; x < 4; ++x)
#pragma unroll
    for (int y = 0; y < 4; ++y) acc[x][y] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int buf) {
#pragma unroll
    for (int kb = 0; kb < PF_KB; ++kb) {
      u32x4_t af[4], bf[4];
#pragma unroll
      for (int x = 0; x < 4; ++x) af[x] = As[buf][kb][wn * 4 + x][lane];
#pragma unroll
      for (int y = 0; y < 4; ++y) bf[y] = Bs[buf][kb][wm * 4 + y][lane];
#pragma unroll
      for (int x = 0; x < 4; ++x)
#pragma unroll
        for (int y = 0; y < 4; ++y) acc[x][y] = mfma16x16x32(bits_bf16x8(af[x]), bits_bf16x8(bf[y]), acc[x][y]);
    }
  };
  // step st: issue the loads of step st + 2 into `nxt`, compute step st from LDS, store step
  // st + 1 (held in `cur`) into the other LDS buffer. Loads and stores are unconditional: the
  // last steps re-load the final k slice, and an odd step count runs one more step over zeros.
  // A load skipped on some path makes the compiler's wait counting assume fewer loads in flight,
  // and the waits before the LDS stores would then also drain the loads issued at the top of the
  // same step (the two-step prefetch would shrink to one).
  const int n_st = kbt / PF_KB, n_run = (n_st + 1) & ~1;
  // The scheduling barriers keep the three phases in this order (left free, the scheduler hoists
  // the stores' masking, which waits for data, above the issue of the next loads).
  auto step = [&](int st, Stage& cur, Stage& nxt) {
    gload(min(st + 2, n_st - 1), nxt);
    __builtin_amdgcn_sched_barrier(0);
    compute(st & 1);
    __builtin_amdgcn_sched_barrier(0);
    lstore((st + 1) & 1, cur, st + 1 < n_st);
    __syncthreads();
  };
  gload(0, s0);
  gload(min(1, n_st - 1), s1);
  lstore(0, s0, true);
  __syncthreads();
  for (int st = 0; st < n_run; st += 2) {
    step(st, s1, s0);
    step(st + 1, s0, s1);
  }

  if constexpr (NORM) {
    // the 8 lanes that staged one row hold its partial sums (lanes l, l ^ 8, ..., l ^ 56)
#pragma unroll
    for (int r = 0; r < XL; ++r) {
      float v = ss[r];
      v += __shfl_xor(v, 8);
      v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 32);
      if (xc == 0) rn_s[xrow_of(r)] = rsqrtf(v / (float)(kbt * 32) + a.norm_eps);
    }
    __syncthreads();
  }

  // Lane (g, j) of acc[x][y] holds rows n = 16 (nb0 + 4 wn + x) + 4 g + e of token m = m0 + 64 wm
  // + 16 y + j.
#pragma unroll
  for (int y = 0; y < 4; ++y) {
    const int mr = wm * 64 + y * 16 + j;
    const float sc = NORM ? rn_s[mr] : 1.f;
#pragma unroll
    for (int x = 0; x < 4; ++x) pf_tile_epilogue<EPI>(a, acc[x][y], nb0 + wn * 4 + x, m0 + mr, sc, g, pos0);
  }
  }  // tile loop
}
// ------------------------------------------------------------------ 4-wave variant
// One workgroup of 4 waves per CU (one per SIMD) owns a 256 (N) x 256 (M) output tile; wave (wn,
// wm) computes 128 x 128 of it (64 accumulator tiles, held in the accumulator registers), so each
// k-block it reads 16 KiB of operands from LDS for 64 MFMAs -- half the LDS bytes per MFMA of the
// 8-wave 64 x 64 layout, whose LDS reads matched the LDS bandwidth at full MFMA rate. Operands
// reach LDS by direct global-to-LDS loads (16 bytes per lane, one contiguous KiB per wave
// instruction: a packed W tile, or 16 tokens x 32 k of X gathered into the MFMA B-operand lane
// order) into a ring of five k-block slots (all 160 KiB of LDS). Step kb: wait until this wave's
// loads of k-block kb + 1 have landed (those of kb + 2 and kb + 3 may still run) and pass one
// barrier; issue the loads of kb + 4 into the slot k-block kb - 1 used; read k-block kb + 1's
// fragments; run k-block kb's 64 MFMAs on the fragments read one step earlier. The step body takes
// its LDS slots as restrict pointers, which lets the compiler see that the fragment reads do not
// touch the slot being loaded (otherwise it waits for every load in flight before each LDS read).
// The folded RMSNorm's sums of squares come from the X fragments the waves already hold (wave wn
// sums fragments 4 wn .. 4 wn + 3 of its 8). Plain and SwiGLU outputs are staged through LDS after
// the k loop and leave as whole 16-byte row pieces (residual read the same way); q/k/v keeps the
// per-element RoPE / KV-cache epilogue.
constexpr int P4_BM = 256, P4_SLOTS = 5, P4_AHEAD = 4;
constexpr int P4_SLOT_BYTES = 32768;                 // 16 W tiles + 16 X tiles of one k-block
constexpr int P4_ROW = 264;                           // staged output row: 256 (or 128) bf16 + 8 of pad
constexpr int P4_RN_OFF = P4_BM * P4_ROW * 2;         // norm scales after the staged tile
typedef __attribute__((address_space(3))) u32x4_t lds_u32x4;

// The k loop's MFMAs are written as inline assembly with the accumulators bound to the accumulator
// registers ("a"): left to the register allocator, some of the 256 accumulator values land in vector
// registers and are copied in and out around their MFMAs, which costs up to half the loop's rate
// depending on the epilogue compiled after it. The first k-block uses srcC = 0 (no read of
// uninitialised accumulators, no VALU-write-to-MFMA-read hazard); accumulator reuse is 64 MFMAs
// apart, and p4_drain() puts the wait states before the epilogue reads them.
template <bool INIT>
__device__ __forceinline__ void mfma_acc(f32x4_t& c, const u32x4_t& a, const u32x4_t& b) {
  if constexpr (INIT) asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, 0" : "=a"(c) : "v"(a), "v"(b));
  else asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
}

__device__ __forceinline__ void p4_drain(f32x4_t (&acc)[8][8]) {
  // the epilogue's reads of every accumulator depend on these statements, which follow the wait
  // states (more than the 16x16x32 MFMA's write latency) in program order
  asm volatile("s_nop 15\n\ts_nop 15" : "+a"(acc[0][0]));
#pragma unroll
  for (int x = 0; x < 8; ++x)
#pragma unroll
    for (int y = 0; y < 8; ++y)
      if (x | y) asm volatile("" : "+a"(acc[x][y]));
}

template <int NORM, bool INIT = false>
__device__ __forceinline__ void p4_step(const u32x4_t* const (&wsrc)[4], const bf16_t* const (&xsrc)[4], size_t woff,
                                        size_t xoff, bool issue, lds_u32x4* __restrict__ dA,
                                        lds_u32x4* __restrict__ dB, const lds_u32x4* __restrict__ nA,
                                        const lds_u32x4* __restrict__ nB, bool fetch, const u32x4_t (&fa)[8],
                                        const u32x4_t (&fb)[8], u32x4_t (&na)[8], u32x4_t (&nb)[8],
                                        f32x4_t (&acc)[8][8], float (&ss)[4], int y0, int lane) {
  if (issue) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      __builtin_amdgcn_global_load_lds((const void*)(wsrc[r] + woff), (__attribute__((address_space(3))) void*)(dA + r * 64),
                                       16, 0, 0);
#pragma unroll
    for (int r = 0; r < 4; ++r)
      __builtin_amdgcn_global_load_lds((const void*)(xsrc[r] + xoff), (__attribute__((address_space(3))) void*)(dB + r * 64),
                                       16, 0, 0);
  }
  if (fetch) {
#pragma unroll
    for (int y = 0; y < 8; ++y) nb[y] = nB[y * 64 + lane];
#pragma unroll
    for (int x = 0; x < 8; ++x) na[x] = nA[x * 64 + lane];
  }
  if constexpr (NORM == 1) {
#pragma unroll
    for (int y = 0; y < 4; ++y) ss[y] += sumsq8(y0 ? fb[4 + y] : fb[y]);
  }
#pragma unroll
  for (int x = 0; x < 8; ++x)
#pragma unroll
    for (int y = 0; y < 8; ++y) mfma_acc<INIT>(acc[x][y], fa[x], fb[y]);
}

// this wave's loads of k-block kb + 1 have landed (the 8 each of up to `later` later k-blocks may
// still run), then the workgroup barrier (no wait for other memory operations)
__device__ __forceinline__ void p4_wait(int later) {
  if (later >= 2) asm volatile("s_waitcnt vmcnt(16)\n\ts_barrier" ::: "memory");
  else if (later == 1) asm volatile("s_waitcnt vmcnt(8)\n\ts_barrier" ::: "memory");
  else asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
}

template <int EPI, int NORM>
__global__ __launch_bounds__(256, 1) void prefill_gemm4_kernel(GemmArgs a, int group, int n_mt, int n_nt, int pos0,
                                                               int sb_n, int sb_m) {
  __shared__ __align__(16) unsigned char smem[P4_SLOTS * P4_SLOT_BYTES];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int wn = w & 1, wm = w >> 1;
  const int n_rt = (a.N + 127) / 128 * 8;
  const int kbt = a.kb_total;
  const u32x4_t* W = (const u32x4_t*)a.W;
  // slot s: W tiles at s * 32 KiB, X tiles 16 KiB further; tile i is 64 lanes x 16 bytes
  auto slotA = [&](int kb, int tile) { return (lds_u32x4*)(smem + (kb % P4_SLOTS) * P4_SLOT_BYTES) + tile * 64; };
  auto slotB = [&](int kb, int tile) {
    return (lds_u32x4*)(smem + (kb % P4_SLOTS) * P4_SLOT_BYTES + 16384) + tile * 64;
  };
  float* rn_s = (float*)(smem + P4_RN_OFF);
  bf16_t* stage = (bf16_t*)smem;  // [256 tokens][P4_ROW] after the k loop
  // the same XCD-aware persistent schedule as prefill_gemm_kernel
  const int xcd = blockIdx.x % 8, jw = blockIdx.x / 8;
  const int n_bn = (n_nt + sb_n - 1) / sb_n, n_bm = (n_mt + sb_m - 1) / sb_m;
  for (int blk = xcd; blk < n_bn * n_bm; blk += 8) {
  const int bn = (blk / n_bm) * sb_n + jw % sb_n, bm = (blk % n_bm) * sb_m + jw / sb_n;
  if (bn >= n_nt || bm >= n_mt || jw >= sb_n * sb_m) continue;  // uniform per workgroup
  const int nb0 = bn * 16, m0 = bm * P4_BM;
  // wave w loads W tiles 4w .. 4w + 3 and X tiles 4w .. 4w + 3 of every k-block (row tiles past
  // the weight's last load that one; tokens past M load the last row: neither is stored)
  const u32x4_t* wsrc[4];
  const bf16_t* xsrc[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int nb = min(nb0 + 4 * w + r, n_rt - 1);
    wsrc[r] = W + packed_tile(nb, 0, kbt, group) * 64 + lane;
    xsrc[r] = a.X + (size_t)min(m0 + 16 * (4 * w + r) + j, a.M - 1) * a.ldx + g * 8;
  }
  const size_t wstep = (size_t)group * 64;

  f32x4_t acc[8][8];  // written first by k-block 0's srcC = 0 MFMAs
  float ss[4] = {};

  // prologue: loads of k-blocks 0 .. 3, fragments of k-block 0
  u32x4_t a0[8], b0[8], a1[8], b1[8];
  for (int p = 0; p < P4_AHEAD; ++p)
    if (p < kbt) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        __builtin_amdgcn_global_load_lds((const void*)(wsrc[r] + p * wstep),
                                         (__attribute__((address_space(3))) void*)(slotA(p, 4 * w) + r * 64), 16, 0, 0);
#pragma unroll
      for (int r = 0; r < 4; ++r)
        __builtin_amdgcn_global_load_lds((const void*)(xsrc[r] + (size_t)p * 32),
                                         (__attribute__((address_space(3))) void*)(slotB(p, 4 * w) + r * 64), 16, 0, 0);
    }
  // k-block 0 landed (up to three later ones may still run), fragments of 0
  if (kbt >= 4) asm volatile("s_waitcnt vmcnt(24)\n\ts_barrier" ::: "memory");
  else if (kbt == 3) asm volatile("s_waitcnt vmcnt(16)\n\ts_barrier" ::: "memory");
  else asm volatile("s_waitcnt vmcnt(8)\n\ts_barrier" ::: "memory");
#pragma unroll
  for (int y = 0; y < 8; ++y) b0[y] = slotB(0, wm * 8)[y * 64 + lane];
#pragma unroll
  for (int x = 0; x < 8; ++x) a0[x] = slotA(0, wn * 8)[x * 64 + lane];

  auto step = [&](auto init, int kb, const u32x4_t (&fa)[8], const u32x4_t (&fb)[8], u32x4_t (&na)[8],
                  u32x4_t (&nb)[8]) {
    p4_wait(min(kbt - 2 - kb, 2));  // loads of kb + 2 .. kb + 3 may still run
    const int ki = kb + P4_AHEAD;
    p4_step<NORM, decltype(init)::value>(wsrc, xsrc, (size_t)ki * wstep, (size_t)ki * 32, ki < kbt, slotA(ki, 4 * w),
                                         slotB(ki, 4 * w), slotA(kb + 1, wn * 8), slotB(kb + 1, wm * 8), kb + 1 < kbt,
                                         fa, fb, na, nb, acc, ss, wn, lane);
  };
  using first_t = std::integral_constant<bool, true>;
  using rest_t = std::integral_constant<bool, false>;
  // kbt is even (K % 64 == 0): step 0, pairs (1, 2) .. (kbt - 3, kbt - 2), step kbt - 1
  step(first_t{}, 0, a0, b0, a1, b1);
  for (int kb = 1; kb + 1 < kbt; kb += 2) {
    step(rest_t{}, kb, a1, b1, a0, b0);
    step(rest_t{}, kb + 1, a0, b0, a1, b1);
  }
  step(rest_t{}, kbt - 1, a1, b1, a0, b0);
  p4_drain(acc);
  __syncthreads();  // every wave is done with the slots: the staged tile and the scales reuse LDS

  if constexpr (NORM == 1) {
    // lanes j, j + 16, j + 32, j + 48 hold the four k-chunks of token 16 y + j
#pragma unroll
    for (int y = 0; y < 4; ++y) {
      float v = ss[y];
      v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 32);
      if (g == 0) rn_s[wm * 128 + 16 * (4 * wn + y) + j] = rsqrtf(v / (float)(kbt * 32) + a.norm_eps);
    }
    __syncthreads();
  } else if constexpr (NORM == 2) {
    rn_s[t] = a.row_scale[min(m0 + t, a.M - 1)];  // 256 threads, 256 rows
    __syncthreads();
  }
  static_assert(EPI != EPI_QKV, "q/k/v runs on prefill_gemm_kernel");
  {
    // stage: lane (g, j) of tile (x, y) holds output rows 16 (wn 8 + x) + 4 g + e of token
    // wm 128 + 16 y + j -- four consecutive columns (plain) or, for SwiGLU, rows r (gate) and
    // r + 8 (up) meeting through a lane swap, four consecutive intermediate columns on lanes g < 2
    constexpr int COLS = EPI == EPI_SWIGLU ? 128 : 256;
#pragma unroll
    for (int y = 0; y < 8; ++y) {
      const int mr = wm * 128 + y * 16 + j;
      const float sc = NORM ? rn_s[mr] : 1.f;
#pragma unroll
      for (int x = 0; x < 8; ++x) {
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[x][y][e] * sc;
        uint32_t lo2, hi2;
        int col;
        if constexpr (EPI == EPI_SWIGLU) {
          float o[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[e]), __float_as_uint(v[e]), false, false);
            const float gt = __uint_as_float(p[0]), up = __uint_as_float(p[1]);
            o[e] = rbf(silu_f(rbf(gt))) * rbf(up);
          }
          lo2 = pack_bf16x2(o[0], o[1]);
          hi2 = pack_bf16x2(o[2], o[3]);
          col = (wn * 8 + x) * 8 + 4 * g;
        } else {
          lo2 = pack_bf16x2(v[0], v[1]);
          hi2 = pack_bf16x2(v[2], v[3]);
          col = (wn * 8 + x) * 16 + 4 * g;
        }
        if (EPI != EPI_SWIGLU || g < 2) *(uint2*)(stage + mr * P4_ROW + col) = make_uint2(lo2, hi2);
      }
    }
    __syncthreads();
    // write out: 8 columns (16 bytes) per item, a row's items on consecutive threads
    const int n_out = EPI == EPI_SWIGLU ? a.N / 2 : a.N;
    const int c0 = (EPI == EPI_SWIGLU ? nb0 * 8 : nb0 * 16);
    const bool vec = a.ldy % 8 == 0 && ((uintptr_t)a.Y & 15) == 0 &&
                     (!a.residual || (a.ldr % 8 == 0 && ((uintptr_t)a.residual & 15) == 0));
    for (int it = t; it < P4_BM * (COLS / 8); it += 256) {
      const int row = it / (COLS / 8), c8 = (it % (COLS / 8)) * 8;
      const int m = m0 + row, n = c0 + c8;
      if (m >= a.M || n >= n_out) continue;
      Pack8 v;
      v.u = *(const uint4*)(stage + row * P4_ROW + c8);
      if (vec && n + 8 <= n_out) {
        if (EPI == EPI_STORE && a.residual) {
          Pack8 r;
          r.u = *(const uint4*)(a.residual + (size_t)m * a.ldr + n);
#pragma unroll
          for (int e = 0; e < 8; ++e) v.h[e] = f2bf(bf2f(r.h[e]) + bf2f(v.h[e]));
        }
        *(uint4*)(a.Y + (size_t)m * a.ldy + n) = v.u;
      } else {
        for (int e = 0; e < 8 && n + e < n_out; ++e) {
          float r = bf2f(v.h[e]);
          if (EPI == EPI_STORE && a.residual) r = rbf(bf2f(a.residual[(size_t)m * a.ldr + n + e]) + r);
          a.Y[(size_t)m * a.ldy + n + e] = f2bf(r);
        }
      }
    }
  }
  __syncthreads();  // the next tile's loads reuse LDS
  }  // tile loop
}

// ------------------------------------------------------------------ causal flash attention
// Row (token t, q head h) at position pos0 + t attends cache slots [0, pos0 + t] (the prompt rows
// before it and itself, whose K/V the q/k/v GEMM of this chunk already wrote).
__device__ __forceinline__ int pf_perm_key(int kt, int i) {
  return (kt >> 1) * 32 + (i >> 2) * 8 + (kt & 1) * 4 + (i & 3);
}

__device__ __forceinline__ float pf_max_lanes(float v) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pf_sum_lanes(float v) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

constexpr int PF_TOK = 32;  // tokens per wave (two 16-row tiles)

template <int HD>
__global__ __launch_bounds__(256, 2) void prefill_attention_kernel(const bf16_t* __restrict__ Q, int64_t ldq, int M,
                                                                   int pos0, int heads, int kv_heads,
                                                                   const bf16_t* __restrict__ Kc,
                                                                   const bf16_t* __restrict__ Vt, int64_t max_len,
                                                                   float scale_log2, bf16_t* __restrict__ out,
                                                                   int64_t ldo, int n_tt) {
  constexpr int KS = HD / 32, DT = HD / 16, NT = PF_TOK / 16;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int n_hg = (heads + 3) / 4;
  // the longest token tiles first (their rows attend the most keys)
  const int tt = n_tt - 1 - (int)blockIdx.x / n_hg;
  const int h = ((int)blockIdx.x % n_hg) * 4 + w;
  if (h >= heads) return;
  const int kvh = h / (heads / kv_heads);
  const int t0 = tt * PF_TOK;
  const bf16_t* kb = Kc + (size_t)kvh * max_len * HD + lane * 8;
  const bf16_t* vb = Vt + (size_t)kvh * max_len * HD + lane * 8;

  u32x4_t qf[NT][KS];
  int lim[NT];  // last attended key of this lane's row in tile rt
#pragma unroll
  for (int rt = 0; rt < NT; ++rt) {
    const int tok = min(t0 + rt * 16 + j, M - 1);
    lim[rt] = pos0 + t0 + rt * 16 + j;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qf[rt][ks] = *(const u32x4_t*)(Q + (size_t)tok * ldq + (size_t)h * HD + ks * 32 + g * 8);
  }
  float m_run[NT], l_run[NT];
  f32x4_t o[NT][DT];
#pragma unroll
  for (int rt = 0; rt < NT; ++rt) {
    m_run[rt] = -INFINITY;
    l_run[rt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[rt][dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  const int last = pos0 + min(t0 + PF_TOK, M) - 1;  // the tile's last attended key
  const int n_blk = last / 64 + 1;
  const int full_blk = (pos0 + t0) / 64;  // blocks every row of the tile attends entirely
  for (int b = 0; b < n_blk; ++b) {
    // K first: the scores of both row tiles; V is loaded while the softmax runs (K and V are not
    // live together, which keeps the wave inside 256 registers)
    u32x4_t kf[4][KS];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) kf[kt][ks] = *(const u32x4_t*)(kb + (size_t)b * 64 * HD + (kt * KS + ks) * 512);
    // k-step outer: consecutive MFMAs go to different accumulators (each sum keeps its ks order)
    f32x4_t s[NT][4];
#pragma unroll
    for (int rt = 0; rt < NT; ++rt)
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) s[rt][kt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int rt = 0; rt < NT; ++rt)
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) s[rt][kt] = mfma16x16x32(bits_bf16x8(kf[kt][ks]), bits_bf16x8(qf[rt][ks]), s[rt][kt]);
    u32x4_t vf[DT][2];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      vf[dt][0] = *(const u32x4_t*)(vb + (size_t)b * 64 * HD + (dt * 2) * 512);
      vf[dt][1] = *(const u32x4_t*)(vb + (size_t)b * 64 * HD + (dt * 2 + 1) * 512);
    }
    if (b == n_blk - 1) {
      // slots past the tile's last key hold whatever the cache held (not yet written): their
      // probabilities are 0, and 0 * V must stay 0, so V is zeroed there. Lane (g, i) of V tile
      // (dt, c) holds slots 64 b + 32 c + 8 g .. + 8.
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const int s0 = b * 64 + c * 32 + g * 8;
        u32x4_t keep;
#pragma unroll
        for (int w2 = 0; w2 < 4; ++w2)
          keep[w2] = (s0 + 2 * w2 <= last ? 0x0000ffffu : 0u) | (s0 + 2 * w2 + 1 <= last ? 0xffff0000u : 0u);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) vf[dt][c] &= keep;
      }
    }
    const bool masked = b >= full_blk;
#pragma unroll
    for (int rt = 0; rt < NT; ++rt) {
      float sv[16], mx = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float v = s[rt][kt][e] * scale_log2;
          if (masked && b * 64 + pf_perm_key(kt, 4 * g + e) > lim[rt]) v = -INFINITY;
          sv[kt * 4 + e] = v;
          mx = fmaxf(mx, v);
        }
      mx = pf_max_lanes(mx);
      const float m_new = fmaxf(m_run[rt], mx);
      // every row attends key 0, so m_new is finite from the first block on
      const float alpha = __builtin_amdgcn_exp2f(m_run[rt] - m_new);
      float l = 0.f;
      uint32_t pw[2][4];
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int e = 0; e < 4; e += 2) {
          const float p0 = __builtin_amdgcn_exp2f(sv[kt * 4 + e] - m_new);
          const float p1 = __builtin_amdgcn_exp2f(sv[kt * 4 + e + 1] - m_new);
          l += p0 + p1;
          pw[kt >> 1][(kt & 1) * 2 + e / 2] = pack_bf16x2(p0, p1);
        }
      l = pf_sum_lanes(l);
      l_run[rt] = l_run[rt] * alpha + l;
      m_run[rt] = m_new;
      const u32x4_t pb0 = {pw[0][0], pw[0][1], pw[0][2], pw[0][3]};
      const u32x4_t pb1 = {pw[1][0], pw[1][1], pw[1][2], pw[1][3]};
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) o[rt][dt] = mfma16x16x32(bits_bf16x8(vf[dt][0]), bits_bf16x8(pb0), o[rt][dt] * alpha);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) o[rt][dt] = mfma16x16x32(bits_bf16x8(vf[dt][1]), bits_bf16x8(pb1), o[rt][dt]);
    }
  }
  // lane (g, j) of o[rt][dt] holds dims 16 dt + 4 g + e of row j
#pragma unroll
  for (int rt = 0; rt < NT; ++rt) {
    const int tok = t0 + rt * 16 + j;
    if (tok >= M) continue;
    const float inv = 1.f / l_run[rt];
    bf16_t* dst = out + (size_t)tok * ldo + (size_t)h * HD;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const uint32_t lo = pack_bf16x2(o[rt][dt][0] * inv, o[rt][dt][1] * inv);
      const uint32_t hi = pack_bf16x2(o[rt][dt][2] * inv, o[rt][dt][3] * inv);
      *(uint2*)(dst + dt * 16 + 4 * g) = make_uint2(lo, hi);
    }
  }
}

// Row scales of the folded RMSNorm, rn[m] = rsqrt(mean(X[m, :K]^2) + eps), one wave per row: lane l
// sums its 8-element pieces l, l + 64, ... of the row in order, then a fixed butterfly (the order
// depends only on K, so a row's scale does not depend on M or on the chunking).
__global__ __launch_bounds__(256) void prefill_rowscale_kernel(const bf16_t* __restrict__ X, int64_t ldx, int M,
                                                               int K, float eps, float* __restrict__ rn) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= M) return;
  const bf16_t* x = X + (size_t)row * ldx;
  float acc = 0.f;
  for (int c = lane * 8; c < K; c += 512) acc += sumsq8(*(const u32x4_t*)(x + c));
  for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off);
  if (lane == 0) rn[row] = rsqrtf(acc / (float)K + eps);
}

static int launch_prefill_gemm4(GemmArgs a, int group, int pos0, int epi, int cus, hipStream_t s) {
  const int n_mt = (a.M + P4_BM - 1) / P4_BM;
  const int n_nt = (a.N + 255) / 256;
  const int per_xcd = max((cus / 8) & ~3, 4);  // one workgroup per CU
  const int sb_m = n_mt < 4 ? n_mt : 4;
  const int sb_n = per_xcd / sb_m;
  const int grid = 8 * sb_n * sb_m;
  const bool norm = a.norm_eps > 0.f;
#define PF4_LAUNCH(E)                                                                                             \
  if (norm) SSD_LAUNCH((prefill_gemm4_kernel<E, 1>), dim3(grid), dim3(256), 0, s, a, group, n_mt, n_nt, pos0, sb_n, sb_m); \
  else SSD_LAUNCH((prefill_gemm4_kernel<E, 0>), dim3(grid), dim3(256), 0, s, a, group, n_mt, n_nt, pos0, sb_n, sb_m);
  if (epi == EPI_SWIGLU) {
    if (a.row_scale)
      SSD_LAUNCH((prefill_gemm4_kernel<EPI_SWIGLU, 2>), dim3(grid), dim3(256), 0, s, a, group, n_mt, n_nt, pos0, sb_n,
                 sb_m);
    else
      PF4_LAUNCH(EPI_SWIGLU);
  } else {
    PF4_LAUNCH(EPI_STORE);
  }
#undef PF4_LAUNCH
  return check_launch("prefill_gemm4");
}

static int launch_prefill_gemm(GemmArgs a, int group, int pos0, int epi, hipStream_t s) {
  const int n_mt = (a.M + PF_BM - 1) / PF_BM;
  const int n_nt = (a.N + 64 * PF_WN - 1) / (64 * PF_WN);
  // 4 / PF_WN workgroups per CU, all resident: 8 XCDs x per_xcd workgroups
  static int cus_of[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return set_error(SSD_EHIP, "prefill gemm: no current device");
  int cus = dev >= 0 && dev < 64 ? cus_of[dev] : 0;
  if (cus <= 0) {
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    if (dev >= 0 && dev < 64) cus_of[dev] = cus;
  }
  // plain and SwiGLU outputs: the 4-wave 256 x 256 kernel (measured at 4096 tokens, 8B shapes: gate/up
  // 1295 against 1440 us, o_proj 160 against 226, down 481 against 602); q/k/v keeps the 8-wave
  // kernel (its RoPE / KV-cache epilogue, and 384 256 x 256 tiles would leave half the CUs idle in a
  // second round)
  if (epi != EPI_QKV) return launch_prefill_gemm4(a, group, pos0, epi, cus, s);
  // 32 on MI355X; at least one block row of 8 M-tiles, so a device reporting fewer CUs (a compute
  // partition) still gets a nonempty grid (the schedule loops, so any grid size is correct)
  const int per_xcd = max((4 / PF_WN * cus / 8) & ~7, 8);
  const int sb_m = n_mt < 8 ? n_mt : 8;
  const int sb_n = per_xcd / sb_m;
  const int grid = 8 * sb_n * sb_m;
  const bool norm = a.norm_eps > 0.f;
#define PF_LAUNCH(E)                                                                                                   \
  if (norm) SSD_LAUNCH((prefill_gemm_kernel<E, 1>), dim3(grid), dim3(128 * PF_WN), 0, s, a, group, n_mt, n_nt, pos0, sb_n, sb_m); \
  else SSD_LAUNCH((prefill_gemm_kernel<E, 0>), dim3(grid), dim3(128 * PF_WN), 0, s, a, group, n_mt, n_nt, pos0, sb_n, sb_m);
  switch (epi) {
    case EPI_STORE: PF_LAUNCH(EPI_STORE); break;
    case EPI_SWIGLU: PF_LAUNCH(EPI_SWIGLU); break;
    default: PF_LAUNCH(EPI_QKV); break;
  }
#undef PF_LAUNCH
  return check_launch("prefill_gemm");
}

static int check_packed(int N, int K, int group) {
  if (N <= 0 || K <= 0 || K % (32 * PF_KB)) return set_error(SSD_EINVAL, "prefill gemm: N=%d K=%d (K %% 64 == 0)", N, K);
  const int tiles = (N + 127) / 128 * 8;  // packed row tiles (rows padded to 128)
  if (group < 1 || group > 16 || tiles % group)
    return set_error(SSD_EINVAL, "prefill gemm: group %d does not divide the %d row tiles", group, tiles);
  return SSD_OK;
}

}  // namespace ssd

using namespace ssd;

static int prefill_gemm(const uint16_t* X, int64_t ldx, int M, const uint16_t* W_packed, int group, int N, int K,
                        float norm_eps, int epi, uint16_t* Y, int64_t ldy, const uint16_t* residual, int64_t ldr,
                        const SsdQkvEpilogue* qkv, const float* row_scale, hipStream_t stream);

SSD_API int ssd_prefill_gemm_bf16(const uint16_t* X, int64_t ldx, int M, const uint16_t* W_packed, int group, int N,
                                  int K, float norm_eps, int epi, uint16_t* Y, int64_t ldy, const uint16_t* residual,
                                  int64_t ldr, const SsdQkvEpilogue* qkv, hipStream_t stream) {
  return prefill_gemm(X, ldx, M, W_packed, group, N, K, norm_eps, epi, Y, ldy, residual, ldr, qkv, nullptr, stream);
}

// ssd_prefill_gemm_bf16 with the folded RMSNorm's row scales given (row_scale, [M] floats, with
// norm_eps > 0; used by the 4-wave kernel's plain and SwiGLU outputs instead of in-loop sums).
static int prefill_gemm(const uint16_t* X, int64_t ldx, int M, const uint16_t* W_packed, int group, int N, int K,
                        float norm_eps, int epi, uint16_t* Y, int64_t ldy, const uint16_t* residual, int64_t ldr,
                        const SsdQkvEpilogue* qkv, const float* row_scale, hipStream_t stream) {
  if (!X || !W_packed || !Y) return set_error(SSD_EINVAL, "prefill gemm: null pointer");
  if (M <= 0) return set_error(SSD_EINVAL, "prefill gemm: M=%d", M);
  int rc = check_packed(N, K, group);
  if (rc) return rc;
  if (ldx < K || ldx % 8 || ((uintptr_t)X & 15)) return set_error(SSD_EINVAL, "prefill gemm: X rows must be 16-byte aligned");
  if (epi != SSD_EPI_STORE && epi != SSD_EPI_SWIGLU && epi != SSD_EPI_QKV)
    return set_error(SSD_EINVAL, "prefill gemm: epilogue %d", epi);
  if (epi == SSD_EPI_STORE && ldy < N) return set_error(SSD_EINVAL, "prefill gemm: ldy %lld < N", (long long)ldy);
  if (epi == SSD_EPI_SWIGLU && (N % 16 || ldy < N / 2)) return set_error(SSD_EINVAL, "prefill gemm: swiglu N=%d", N);
  if (epi != SSD_EPI_STORE && residual) return set_error(SSD_EINVAL, "prefill gemm: residual only with a plain store");
  GemmArgs a{};
  a.X = X; a.ldx = ldx; a.M = M; a.W = (const uint4*)W_packed; a.N = N; a.kb_total = K / 32;
  a.Y = Y; a.ldy = ldy; a.residual = residual; a.ldr = ldr; a.norm_eps = norm_eps;
  a.row_scale = norm_eps > 0.f ? row_scale : nullptr;
  int pos0 = 0;
  if (epi == SSD_EPI_QKV) {
    if (!qkv || !qkv->cos || !qkv->sin || !qkv->k_cache || !qkv->vt_cache)
      return set_error(SSD_EINVAL, "prefill gemm: q/k/v epilogue needs rotary tables and the cache");
    const int hd = qkv->head_dim;
    if ((hd != 32 && hd != 64 && hd != 128) || qkv->heads <= 0 || qkv->kv_heads <= 0 ||
        N != (qkv->heads + 2 * qkv->kv_heads) * hd || ldy < (int64_t)qkv->heads * hd)
      return set_error(SSD_EINVAL, "prefill gemm: q/k/v shape N=%d heads=%d kv=%d hd=%d", N, qkv->heads,
                       qkv->kv_heads, hd);
    if (qkv->pos0 < 0 || qkv->pos0 + M > qkv->max_len || qkv->pos0 + M > qkv->rope_rows || qkv->max_len % 64)
      return set_error(SSD_EINVAL, "prefill gemm: rows [%d, %d) outside the cache (%lld) or rotary table (%lld)",
                       qkv->pos0, qkv->pos0 + M, (long long)qkv->max_len, (long long)qkv->rope_rows);
    a.heads = qkv->heads; a.kv_heads = qkv->kv_heads; a.head_dim = hd;
    a.cos_tab = qkv->cos; a.sin_tab = qkv->sin; a.rope_rows = qkv->rope_rows;
    a.k_cache = qkv->k_cache; a.vt_cache = qkv->vt_cache; a.max_len = qkv->max_len;
    pos0 = qkv->pos0;
  }
  return launch_prefill_gemm(a, group, pos0, epi, stream);
}

SSD_API int ssd_prefill_attention_bf16(const uint16_t* q, int64_t ldq, int M, int pos0, int heads, int kv_heads,
                                       int head_dim, const uint16_t* k_cache, const uint16_t* vt_cache,
                                       int64_t max_len, float scale, uint16_t* out, int64_t ldo,
                                       hipStream_t stream) {
  if (!q || !k_cache || !vt_cache || !out) return set_error(SSD_EINVAL, "prefill attention: null pointer");
  if (M <= 0 || pos0 < 0 || heads <= 0 || kv_heads <= 0 || heads % kv_heads)
    return set_error(SSD_EINVAL, "prefill attention: M=%d pos0=%d heads=%d kv_heads=%d", M, pos0, heads, kv_heads);
  if (pos0 + M > max_len || max_len % 64 || ldq % 8 || ((uintptr_t)q & 15) || ((uintptr_t)k_cache & 15) ||
      ((uintptr_t)vt_cache & 15) || ldo % 4 || ((uintptr_t)out & 7))
    return set_error(SSD_EINVAL, "prefill attention: rows [%d, %d) vs cache %lld, or misaligned operands", pos0,
                     pos0 + M, (long long)max_len);
  const int n_tt = (M + PF_TOK - 1) / PF_TOK;
  const dim3 grid((unsigned)(n_tt * ((heads + 3) / 4))), block(256);
  const float sl2 = scale * 1.4426950408889634f;
  switch (head_dim) {
    case 64:
      SSD_LAUNCH((prefill_attention_kernel<64>), grid, block, 0, stream, (const bf16_t*)q, ldq, M, pos0, heads,
                         kv_heads, (const bf16_t*)k_cache, (const bf16_t*)vt_cache, max_len, sl2, (bf16_t*)out, ldo, n_tt);
      break;
    case 128:
      SSD_LAUNCH((prefill_attention_kernel<128>), grid, block, 0, stream, (const bf16_t*)q, ldq, M, pos0,
                         heads, kv_heads, (const bf16_t*)k_cache, (const bf16_t*)vt_cache, max_len, sl2, (bf16_t*)out,
                         ldo, n_tt);
      break;
    default:
      return set_error(SSD_EINVAL, "prefill attention: head_dim %d unsupported (64, 128)", head_dim);
  }
  return check_launch("prefill_attention");
}

// The target forward over prompt rows [pos0, pos0 + m): embed -> per layer q/k/v (+RoPE, KV
// write) -> causal attention -> o_proj + residual -> gate/up + SwiGLU -> down + residual; then the
// full-vocabulary head (head_w, final norm folded; NULL = none) on the last row. Buffers are
// [m_cap] rows.
SSD_API int ssd_prefill(const SsdModel* md, const uint16_t* head_w, const SsdPrefillBuffers* pb, const int32_t* ids,
                        int m, int pos0, hipStream_t s) {
  if (!md || !pb || !ids) return set_error(SSD_EINVAL, "prefill: null descriptor");
  if (m <= 0 || m > pb->m_cap) return set_error(SSD_EINVAL, "prefill: m=%d outside [1, %d]", m, pb->m_cap);
  if (!md->layers) return set_error(SSD_EINVAL, "prefill: null layer table");
  if (!(md->eps > 0.f)) return set_error(SSD_EINVAL, "prefill: norm eps must be > 0");
  if (pos0 < 0 || pos0 + m > pb->cache_cap)
    return set_error(SSD_EINVAL, "prefill: rows [%d, %d) beyond the cache (%lld)", pos0, pos0 + m,
                     (long long)pb->cache_cap);
  if (head_w && !pb->logits) return set_error(SSD_EINVAL, "prefill: no logits buffer");
  const int d = md->hidden, hd = md->head_dim, H = md->heads, KV = md->kv_heads, I = md->inter;
  const int64_t qdim = (int64_t)H * hd;
  const int nqkv = (H + 2 * KV) * hd;
  const size_t layer_elems = (size_t)KV * pb->cache_cap * hd;
  const int g_qkv = ssd_gemm_weight_group(nqkv, d), g_o = ssd_gemm_residual_group(d, (int)qdim);
  const int g_gu = md->mlp_fused ? ssd_mlp_group(I, d) : ssd_gemm_weight_group(2 * I, d);
  const int g_d = ssd_gemm_residual_group(d, I);
  if (g_qkv < 1 || g_o < 1 || g_gu < 1 || g_d < 1) return set_error(SSD_EINVAL, "prefill: no packing plan for this shape");
  int rc = ssd_embed_bf16(ids, m, md->embed, md->vocab, d, pb->h, d, s);
  if (rc) return rc;
  for (int li = 0; li < md->n_layers; ++li) {
    const SsdLayerW& L = md->layers[li];
    SsdQkvEpilogue qe{H, KV, hd, md->cos, md->sin, md->rope_rows, pos0, pb->k_arena + li * layer_elems,
                      pb->vt_arena + li * layer_elems, pb->cache_cap};
    if ((rc = ssd_prefill_gemm_bf16(pb->h, d, m, L.wqkv, g_qkv, nqkv, d, md->eps, SSD_EPI_QKV, pb->q, qdim, nullptr, 0,
                                    &qe, s)))
      return rc;
    if ((rc = ssd_prefill_attention_bf16(pb->q, qdim, m, pos0, H, KV, hd, qe.k_cache, qe.vt_cache, pb->cache_cap,
                                         md->attn_scale, pb->attn, qdim, s)))
      return rc;
    if ((rc = ssd_prefill_gemm_bf16(pb->attn, qdim, m, L.wo, g_o, d, (int)qdim, 0.f, SSD_EPI_STORE, pb->h, d, pb->h, d,
                                    nullptr, s)))
      return rc;
    // gate/up's norm scales computed once per row into the q buffer (free after the attention)
    float* rs = (float*)pb->q;
    SSD_LAUNCH(prefill_rowscale_kernel, dim3((m + 3) / 4), dim3(256), 0, s, pb->h, (int64_t)d, m, d, md->eps, rs);
    if ((rc = check_launch("prefill_rowscale"))) return rc;
    if ((rc = prefill_gemm(pb->h, d, m, L.wgu, g_gu, 2 * I, d, md->eps, SSD_EPI_SWIGLU, pb->act, I, nullptr, 0, nullptr,
                           rs, s)))
      return rc;
    if ((rc = ssd_prefill_gemm_bf16(pb->act, I, m, L.wd, g_d, d, I, 0.f, SSD_EPI_STORE, pb->h, d, pb->h, d, nullptr, s)))
      return rc;
  }
  if (head_w)
    return ssd_gemm_bf16(pb->h + (size_t)(m - 1) * d, d, 1, head_w, md->vocab, d, md->eps, pb->logits, md->vocab,
                         nullptr, 0, nullptr, 0, s);
  return SSD_OK;
}
