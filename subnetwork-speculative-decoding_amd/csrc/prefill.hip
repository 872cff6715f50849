// Prefill on gfx950: the target forward over a long prompt chunk (hundreds to thousands of rows),
// where every projection is a compute-bound GEMM and attention is causal.
//
// The decode kernels stream each weight once per call and suit M <= 64 rows; a 4096-token prompt
// through them re-reads every weight 64 times. Here (reference ssd/engine/speculative.py:149-151,
// the target's forward over the prompt):
//
// * prefill_gemm4_kernel: Y = X W^T over the same packed weights as the decode GEMMs (16 x 32 MFMA
//   A-operand tiles, any tile grouping) with v_mfma_f32_16x16x32_bf16: one 4-wave workgroup per CU
//   with a 256 x 256 (o, down, gate/up) or 192 x 256 (q/k/v) output tile, accumulators pinned to the
//   accumulator registers, operands loaded straight into a five-slot LDS ring, outputs staged through
//   LDS and stored as 16-byte pieces. The decode epilogues run on the staged tile: SwiGLU for gate/up
//   (gate / up rows r and r + 8 meet through one v_permlane32_swap), residual add for o and down,
//   RoPE + KV-cache write for q/k/v; the folded RMSNorm scale comes from a row-scale pass. The launch
//   is persistent and XCD-aware: the workgroups resident on one XCD sweep blocks of output tiles
//   together, so the weight and activation tiles they share are fetched into that XCD's L2 once per
//   block.
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

// Tile (nb, kb) of a packed weight with `group` row tiles per k-block group: 64 lanes x 16 B.
__device__ __forceinline__ size_t packed_tile(int nb, int kb, int kbt, int group) {
  return ((size_t)(nb / group) * kbt + kb) * group + nb % group;
}

// ------------------------------------------------------------------ 4-wave variant
// One workgroup of 4 waves per CU (one per SIMD) owns a 32 XT (N) x 256 (M) output tile; wave (wn,
// wm) computes 16 XT x 128 of it (8 XT accumulator tiles, held in the accumulator registers), so
// with XT = 8 each k-block it reads 16 KiB of operands from LDS for 64 MFMAs -- half the LDS bytes
// per MFMA of a 64 x 64-per-wave layout, whose LDS reads would match the LDS bandwidth at full MFMA
// rate. XT = 8 (256 x 256 tiles) serves the plain and SwiGLU projections; q/k/v uses XT = 6
// (192 x 256 tiles), which at the 8B shape (N 6144) makes 512 tiles, two full rounds of 256 CUs
// instead of 384 tiles whose second round leaves half the CUs idle. Operands reach LDS by direct
// global-to-LDS loads (16 bytes per lane, one contiguous KiB per wave instruction: a packed W tile,
// or 16 tokens x 32 k of X gathered into the MFMA B-operand lane order) into a ring of five k-block
// slots (all 160 KiB of LDS). Step kb: wait until this wave's loads of k-block kb + 1 have landed
// (those of kb + 2 and kb + 3 may still run) and pass one barrier; issue the loads of kb + 4 into
// the slot k-block kb - 1 used; read k-block kb + 1's fragments; run k-block kb's MFMAs on the
// fragments read one step earlier. The step body takes its LDS slots as restrict pointers, which
// lets the compiler see that the fragment reads do not touch the slot being loaded (otherwise it
// waits for every load in flight before each LDS read). The folded RMSNorm's row scales come either
// from the caller (a row-scale pass) or from sums of squares of the X fragments the waves already
// hold (wave wn sums fragments 4 wn .. 4 wn + 3 of its 8). Outputs are staged through LDS after the
// k loop and leave as whole 16-byte pieces: rows of Y (residual read the same way); for q/k/v, rows
// of q and K-cache slots with RoPE applied on the way out, and 8-slot runs of the V^T cache.
constexpr int P4_BM = 256, P4_SLOTS = 5, P4_AHEAD = 4;
constexpr int P4_SLOT_BYTES = 32768;                 // up to 16 W tiles + 16 X tiles of one k-block
constexpr int P4_ROW = 264;                           // staged output row: up to 256 bf16 + 8 of pad
constexpr int P4_RN_OFF = P4_BM * P4_ROW * 2;         // norm scales after the staged tile
typedef __attribute__((address_space(3))) u32x4_t lds_u32x4;

// The k loop's MFMAs are written as inline assembly with the accumulators bound to the accumulator
// registers ("a"): left to the register allocator, some of the accumulator values land in vector
// registers and are copied in and out around their MFMAs, which costs up to half the loop's rate
// depending on the epilogue compiled after it. The first k-block uses srcC = 0 (no read of
// uninitialised accumulators, no VALU-write-to-MFMA-read hazard); accumulator reuse is 8 XT MFMAs
// apart, and p4_drain() puts the wait states before the epilogue reads them.
template <bool INIT>
__device__ __forceinline__ void mfma_acc(f32x4_t& c, const u32x4_t& a, const u32x4_t& b) {
  if constexpr (INIT) asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, 0" : "=a"(c) : "v"(a), "v"(b));
  else asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
}

template <int XT>
__device__ __forceinline__ void p4_drain(f32x4_t (&acc)[XT][8]) {
  // the epilogue's reads of every accumulator depend on these statements, which follow the wait
  // states (more than the 16x16x32 MFMA's write latency) in program order
  asm volatile("s_nop 15\n\ts_nop 15" : "+a"(acc[0][0]));
#pragma unroll
  for (int x = 0; x < XT; ++x)
#pragma unroll
    for (int y = 0; y < 8; ++y)
      if (x | y) asm volatile("" : "+a"(acc[x][y]));
}

template <bool INIT, int XT>
__device__ __forceinline__ void p4_step(const u32x4_t* const (&wsrc)[XT / 2], const bf16_t* const (&xsrc)[4],
                                        size_t woff, size_t xoff, bool issue, lds_u32x4* __restrict__ dA,
                                        lds_u32x4* __restrict__ dB, const lds_u32x4* __restrict__ nA,
                                        const lds_u32x4* __restrict__ nB, bool fetch, const u32x4_t (&fa)[XT],
                                        const u32x4_t (&fb)[8], u32x4_t (&na)[XT], u32x4_t (&nb)[8],
                                        f32x4_t (&acc)[XT][8], int lane) {
  if (issue) {
#pragma unroll
    for (int r = 0; r < XT / 2; ++r)
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
    for (int x = 0; x < XT; ++x) na[x] = nA[x * 64 + lane];
  }
#pragma unroll
  for (int x = 0; x < XT; ++x)
#pragma unroll
    for (int y = 0; y < 8; ++y) mfma_acc<INIT>(acc[x][y], fa[x], fb[y]);
}

// this wave's loads of k-block kb + 1 have landed (the PER = XT / 2 + 4 each of up to `later`
// later k-blocks may still run), then the workgroup barrier (no wait for other memory operations)
template <int PER>
__device__ __forceinline__ void p4_wait(int later) {
  static_assert(PER == 8 || PER == 7, "XT = 8 or 6");
  if constexpr (PER == 8) {
    if (later >= 3) asm volatile("s_waitcnt vmcnt(24)\n\ts_barrier" ::: "memory");
    else if (later == 2) asm volatile("s_waitcnt vmcnt(16)\n\ts_barrier" ::: "memory");
    else if (later == 1) asm volatile("s_waitcnt vmcnt(8)\n\ts_barrier" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
  } else {
    if (later >= 3) asm volatile("s_waitcnt vmcnt(21)\n\ts_barrier" ::: "memory");
    else if (later == 2) asm volatile("s_waitcnt vmcnt(14)\n\ts_barrier" ::: "memory");
    else if (later == 1) asm volatile("s_waitcnt vmcnt(7)\n\ts_barrier" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
  }
}

// SiLU of the prefill's SwiGLU staging: x sigma(x) with the logistic function through the hardware
// base-2 exponential and reciprocal, 1 / (1 + 2^(-x log2 e)) (a few ulp of fp32, then rounded to
// bf16; the exact division and exponential of silu_f cost half of the gate/up tile's staging).
// exp2 overflows to +inf for x < -88 (sigma = 0, silu = -0) and underflows to 0 for large x (silu = x).
__device__ __forceinline__ float pf_silu(float x) {
  return x * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(x * -1.4426950408889634f));
}

// q/k/v write-out of one staged tile: rows of q and K-cache slots (RoPE applied here), then 8-slot
// runs of V^T. Staged column 16 t + i holds weight tile nb0 + t's row i: rotary dim p 8 + i
// (i < 8) or hd / 2 + p 8 + i - 8 (i >= 8) of its head -- both halves of each rotary pair. Thread
// t's q/k items are (token, weight tile) = divmod(t + 256 i, 2 XT), i < 2 XT; their rotary cos / sin
// pieces are loaded by p4_qkv_rope() before the tile is staged (clamped addresses for items that
// are not q/k, so the loads are unconditional), so their latency overlaps the staging.
template <int XT>
struct P4Rope {
  Pack8 cs[2 * XT], sn[2 * XT];
};

template <int XT>
__device__ __forceinline__ void p4_qkv_rope(const GemmArgs& a, int nb0, int m0, int pos0, int t, P4Rope<XT>& r) {
  constexpr int NWT = 2 * XT;
  const int half = a.head_dim >> 1;
#pragma unroll
  for (int i = 0; i < NWT; ++i) {
    const int it = t + 256 * i, row = it / NWT, tt = it % NWT;
    const QkvTile q = qkv_tile(a, nb0 + tt);
    const int pos = min(max(pos0 + m0 + row, 0), (int)a.rope_rows - 1);
    const size_t at = (size_t)pos * half + (q.p & (half / 8 - 1)) * 8;
    r.cs[i].u = *(const uint4*)(a.cos_tab + at);
    r.sn[i].u = *(const uint4*)(a.sin_tab + at);
  }
}

template <int XT>
__device__ __forceinline__ void p4_qkv_out(const GemmArgs& a, const bf16_t* stage, int nb0, int m0, int pos0, int t,
                                           const P4Rope<XT>& r) {
  constexpr int NWT = 2 * XT;  // weight tiles of the workgroup tile
  const int hd = a.head_dim, half = hd >> 1;
  const int n_wt = min(NWT, a.N / 16 - nb0);  // N is a multiple of 16 (q/k/v shape)
  const bool qvec = a.ldy % 8 == 0 && ((uintptr_t)a.Y & 15) == 0;
  // q and K: one (token, weight tile) per item, two 16-byte pieces (the pair's halves)
#pragma unroll
  for (int i = 0; i < NWT; ++i) {
    const int it = t + 256 * i, row = it / NWT, tt = it % NWT, m = m0 + row;
    if (tt >= n_wt || m >= a.M) continue;
    const QkvTile q = qkv_tile(a, nb0 + tt);
    if (q.region == 2) continue;
    Pack8 lo, hi, olo, ohi;
    lo.u = *(const uint4*)(stage + row * P4_ROW + tt * 16);
    hi.u = *(const uint4*)(stage + row * P4_ROW + tt * 16 + 8);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float xl = bf2f(lo.h[e]), xh = bf2f(hi.h[e]), c = bf2f(r.cs[i].h[e]), s = bf2f(r.sn[i].h[e]);
      olo.h[e] = f2bf(rbf(rbf(xl * c) - rbf(xh * s)));
      ohi.h[e] = f2bf(rbf(rbf(xh * c) + rbf(xl * s)));
    }
    if (q.region == 0) {
      bf16_t* qo = a.Y + (size_t)m * a.ldy + (size_t)q.head * hd + q.p * 8;
      if (qvec) {
        *(uint4*)qo = olo.u;
        *(uint4*)(qo + half) = ohi.u;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          qo[e] = olo.h[e];
          qo[half + e] = ohi.h[e];
        }
      }
    } else {
      const int slot = pos0 + m;  // inside the cache (checked on the host)
      bf16_t* kc = a.k_cache + (size_t)q.head * a.max_len * hd;
      *(uint4*)(kc + k_off(slot, q.p * 8, hd)) = olo.u;
      *(uint4*)(kc + k_off(slot, half + q.p * 8, hd)) = ohi.u;
    }
  }
  // V^T: one (8-slot run, staged column) per item; runs cut by the tile's first or last token, or by
  // M, are written element by element (the neighbouring tile writes the rest of such a run)
  const int s_lo = pos0 + m0, s_hi = pos0 + min(m0 + P4_BM, a.M);  // slots [s_lo, s_hi)
  const int g_lo = s_lo >> 3, n_runs = ((s_hi + 7) >> 3) - g_lo;
  for (int it = t; it < n_runs * NWT * 16; it += 256) {
    const int run = it / (NWT * 16), c = it % (NWT * 16), tt = c >> 4, i = c & 15;
    if (tt >= n_wt) continue;
    const QkvTile q = qkv_tile(a, nb0 + tt);
    if (q.region != 2) continue;
    const int d = q.p * 8 + (i & 7) + (i >= 8 ? half : 0);
    const int s0 = (g_lo + run) * 8;
    bf16_t* vt = a.vt_cache + (size_t)q.head * hd * a.max_len;
    if (s0 >= s_lo && s0 + 8 <= s_hi) {
      Pack8 v;
#pragma unroll
      for (int e = 0; e < 8; ++e) v.h[e] = stage[(s0 + e - s_lo) * P4_ROW + c];
      *(uint4*)(vt + v_off(s0, d, hd)) = v.u;
    } else {
      for (int e = 0; e < 8; ++e) {
        const int s = s0 + e;
        if (s >= s_lo && s < s_hi) vt[v_off(s, d, hd)] = stage[(s - s_lo) * P4_ROW + c];
      }
    }
  }
}

template <int EPI, bool RS, int XT>
__global__ __launch_bounds__(256, 1) void prefill_gemm4_kernel(GemmArgs a, int group, int n_mt, int n_nt, int pos0,
                                                               int sb_n, int sb_m) {
  static_assert(XT == 8 || XT == 6, "8 or 6 weight tiles per wave");
  static_assert(EPI != EPI_SWIGLU || XT == 8, "SwiGLU pairs need whole 16-column output groups");
  constexpr int WR = XT / 2, PER = WR + 4;  // W tiles each wave loads per k-block; loads per k-block
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
  // persistent and XCD-aware: the workgroups resident on one XCD sweep blocks of sb_n x sb_m output
  // tiles together, so the weight and activation tiles they share are fetched into that XCD's L2
  // once per block
  const int xcd = blockIdx.x % 8, jw = blockIdx.x / 8;
  const int n_bn = (n_nt + sb_n - 1) / sb_n, n_bm = (n_mt + sb_m - 1) / sb_m;
  for (int blk = xcd; blk < n_bn * n_bm; blk += 8) {
  const int bn = (blk / n_bm) * sb_n + jw % sb_n, bm = (blk % n_bm) * sb_m + jw / sb_n;
  if (bn >= n_nt || bm >= n_mt || jw >= sb_n * sb_m) continue;  // uniform per workgroup
  const int nb0 = bn * 2 * XT, m0 = bm * P4_BM;
  // wave w loads W tiles WR w .. WR w + WR - 1 and X tiles 4w .. 4w + 3 of every k-block (row tiles
  // past the weight's last load that one; tokens past M load the last row: neither is stored)
  const u32x4_t* wsrc[WR];
  const bf16_t* xsrc[4];
#pragma unroll
  for (int r = 0; r < WR; ++r) {
    const int nb = min(nb0 + WR * w + r, n_rt - 1);
    wsrc[r] = W + packed_tile(nb, 0, kbt, group) * 64 + lane;
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) xsrc[r] = a.X + (size_t)min(m0 + 16 * (4 * w + r) + j, a.M - 1) * a.ldx + g * 8;
  const size_t wstep = (size_t)group * 64;

  f32x4_t acc[XT][8];  // written first by k-block 0's srcC = 0 MFMAs

  // prologue: loads of k-blocks 0 .. 3, fragments of k-block 0
  u32x4_t a0[XT], b0[8], a1[XT], b1[8];
  for (int p = 0; p < P4_AHEAD; ++p)
    if (p < kbt) {
#pragma unroll
      for (int r = 0; r < WR; ++r)
        __builtin_amdgcn_global_load_lds((const void*)(wsrc[r] + p * wstep),
                                         (__attribute__((address_space(3))) void*)(slotA(p, WR * w) + r * 64), 16, 0, 0);
#pragma unroll
      for (int r = 0; r < 4; ++r)
        __builtin_amdgcn_global_load_lds((const void*)(xsrc[r] + (size_t)p * 32),
                                         (__attribute__((address_space(3))) void*)(slotB(p, 4 * w) + r * 64), 16, 0, 0);
    }
  // k-block 0 landed (up to three later ones may still run), fragments of 0
  p4_wait<PER>(min(kbt, P4_AHEAD) - 1);
#pragma unroll
  for (int y = 0; y < 8; ++y) b0[y] = slotB(0, wm * 8)[y * 64 + lane];
#pragma unroll
  for (int x = 0; x < XT; ++x) a0[x] = slotA(0, wn * XT)[x * 64 + lane];

  auto step = [&](auto init, int kb, const u32x4_t (&fa)[XT], const u32x4_t (&fb)[8], u32x4_t (&na)[XT],
                  u32x4_t (&nb)[8]) {
    p4_wait<PER>(min(kbt - 2 - kb, 2));  // loads of kb + 2 .. kb + 3 may still run
    const int ki = kb + P4_AHEAD;
    p4_step<decltype(init)::value, XT>(wsrc, xsrc, (size_t)ki * wstep, (size_t)ki * 32, ki < kbt, slotA(ki, WR * w),
                                       slotB(ki, 4 * w), slotA(kb + 1, wn * XT), slotB(kb + 1, wm * 8), kb + 1 < kbt,
                                       fa, fb, na, nb, acc, lane);
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
  p4_drain<XT>(acc);
  __syncthreads();  // every wave is done with the slots: the staged tile and the scales reuse LDS

  if constexpr (RS) {
    rn_s[t] = a.row_scale[min(m0 + t, a.M - 1)];  // 256 threads, 256 rows
    __syncthreads();
  }
  {
    // the epilogue's thread indices pass through an empty asm statement, so that nothing computed
    // from them is hoisted above the k loop and kept live (spilled) across it
    int te = t;
    asm volatile("" : "+v"(te));
    const int je = te & 15, ge = (te >> 4) & 3, we = te >> 6, wne = we & 1, wme = we >> 1;
    constexpr int COLS = EPI == EPI_SWIGLU ? 16 * XT : 32 * XT;  // staged columns
    constexpr int NIT = COLS / 8;                                   // write-out items per thread
    const int n_out = EPI == EPI_SWIGLU ? a.N / 2 : a.N;
    const int c0 = (EPI == EPI_SWIGLU ? nb0 * 8 : nb0 * 16);
    // The residual joins in the staging: lane (g, j)'s four columns of tile (x, y) are one 8-byte
    // residual piece, loaded two token tiles ahead (clamped addresses, so the loads are
    // unconditional; columns past N are never stored). The rotary tables of the q/k/v write-out are
    // loaded before the staging. Either way the loads' latency overlaps the staging.
    const bool res = EPI == EPI_STORE && a.residual && a.ldr % 4 == 0 && ((uintptr_t)a.residual & 7) == 0 &&
                     n_out % 4 == 0;  // uniform
    // 16-byte stores of staged rows (with a residual, only when the staging added it)
    const bool vec = a.ldy % 8 == 0 && ((uintptr_t)a.Y & 15) == 0 && (!a.residual || res);
    [[maybe_unused]] uint2 rq[3][EPI == EPI_STORE ? XT : 1];
    auto load_res = [&](int y, uint2 (&dst)[EPI == EPI_STORE ? XT : 1]) {
      if constexpr (EPI == EPI_STORE) {
        const int m = min(m0 + wme * 128 + y * 16 + je, a.M - 1);
#pragma unroll
        for (int x = 0; x < XT; ++x) {
          const int n = min(c0 + (wne * XT + x) * 16 + 4 * ge, n_out - 4);
          dst[x] = *(const uint2*)(a.residual + (size_t)m * a.ldr + n);
        }
      }
    };
    [[maybe_unused]] P4Rope<EPI == EPI_QKV ? XT : 1> rope;
    if constexpr (EPI == EPI_STORE) {
      if (res) {
        load_res(0, rq[0]);
        load_res(1, rq[1]);
      }
    } else if constexpr (EPI == EPI_QKV) {
      p4_qkv_rope<XT>(a, nb0, m0, pos0, te, rope);
    }
    // stage: lane (g, j) of tile (x, y) holds output rows 16 (wn XT + x) + 4 g + e of token
    // wm 128 + 16 y + j -- four consecutive columns (plain, q/k/v). For SwiGLU, rows r (gate) and
    // r + 8 (up) meet through a lane swap, after which lanes g and g + 2 hold the same four pairs:
    // lanes g < 2 finish pairs 0, 1 and lanes g >= 2 pairs 2, 3 of them (intermediate columns
    // 8 (wn XT + x) + 4 (g & 1) + 2 (g >> 1) + 0, 1).
#pragma unroll
    for (int y = 0; y < 8; ++y) {
      const int mr = wme * 128 + y * 16 + je;
      const float sc = RS ? rn_s[mr] : 1.f;
      if constexpr (EPI == EPI_STORE) {
        __builtin_amdgcn_sched_barrier(0);  // keep each row's loads two rows ahead (not all hoisted)
        if (res && y + 2 < 8) load_res(y + 2, rq[(y + 2) % 3]);
      }
#pragma unroll
      for (int x = 0; x < XT; ++x) {
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[x][y][e] * sc;
        if constexpr (EPI == EPI_SWIGLU) {
          float gt[4], up[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[e]), __float_as_uint(v[e]), false, false);
            gt[e] = __uint_as_float(p[0]);
            up[e] = __uint_as_float(p[1]);
          }
          const bool hi = ge >= 2;
          const float g0 = hi ? gt[2] : gt[0], g1 = hi ? gt[3] : gt[1];
          const float u0 = hi ? up[2] : up[0], u1 = hi ? up[3] : up[1];
          const float o0 = rbf(pf_silu(rbf(g0))) * rbf(u0), o1 = rbf(pf_silu(rbf(g1))) * rbf(u1);
          const int col = (wne * XT + x) * 8 + 4 * (ge & 1) + 2 * (ge >> 1);
          *(uint32_t*)(stage + mr * P4_ROW + col) = pack_bf16x2(o0, o1);
        } else {
          if constexpr (EPI == EPI_STORE) {
            if (res) {
              // out = bf16(residual + bf16(acc sc)), the order of the decode epilogue
              const uint2 r = rq[y % 3][x];
              const uint32_t rw[2] = {r.x, r.y};
#pragma unroll
              for (int e = 0; e < 4; ++e) v[e] = bf2f((bf16_t)(rw[e >> 1] >> (16 * (e & 1)))) + rbf(v[e]);
            }
          }
          const int col = (wne * XT + x) * 16 + 4 * ge;
          *(uint2*)(stage + mr * P4_ROW + col) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
        }
      }
    }
    __syncthreads();
    if constexpr (EPI == EPI_QKV) {
      p4_qkv_out<XT>(a, stage, nb0, m0, pos0, te, rope);
    } else {
      // write out: 8 columns (16 bytes) per item, a row's items on consecutive threads
      if (vec && n_out % 8 == 0) {  // uniform: every item is one whole 16-byte piece
        for (int i = 0; i < NIT; ++i) {
          const int it = te + 256 * i, row = it / NIT, c8 = (it % NIT) * 8;
          const int m = m0 + row, n = c0 + c8;
          if (m >= a.M || n >= n_out) continue;
          *(uint4*)(a.Y + (size_t)m * a.ldy + n) = *(const uint4*)(stage + row * P4_ROW + c8);
        }
      } else {  // element by element (unaligned output or residual, or N not a multiple of 8)
        for (int i = 0; i < NIT; ++i) {
          const int it = te + 256 * i, row = it / NIT, c8 = (it % NIT) * 8;
          const int m = m0 + row, n = c0 + c8;
          if (m >= a.M || n >= n_out) continue;
          Pack8 v;
          v.u = *(const uint4*)(stage + row * P4_ROW + c8);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            if (n + e >= n_out) continue;
            float r = bf2f(v.h[e]);  // the staged value already holds the residual when res
            if (EPI == EPI_STORE && a.residual && !res) r = rbf(bf2f(a.residual[(size_t)m * a.ldr + n + e]) + r);
            a.Y[(size_t)m * a.ldy + n + e] = f2bf(r);
          }
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

// Per-wave state of the causal attention: the query fragments of two 16-row tiles, their running
// max / sum and output accumulators, and each lane's last attended key.
template <int HD>
struct PfAttnState {
  static constexpr int KS = HD / 32, DT = HD / 16, NT = PF_TOK / 16;
  u32x4_t qf[NT][KS];
  float m_run[NT], l_run[NT];
  f32x4_t o[NT][DT];
  int lim[NT];
};

// One 64-key block b for both row tiles. K / V fragments come from `ck` / `cv` (the block in LDS,
// SHARED) or from the cache rows `kb` / `vb`; with SHARED the copy of block b + 1 into `nk` / `nv`
// is issued first. The LDS pointers are restrict, so the compiler sees that the fragment reads do
// not touch the buffer being filled and does not wait for that copy before them.
template <int HD, bool SHARED>
__device__ __forceinline__ void pf_attend_block(PfAttnState<HD>& st, int b, int n_blk, int full_blk, int last,
                                                float scale_log2, int lane, const bf16_t* kb, const bf16_t* vb,
                                                const u32x4_t* ksrc, const u32x4_t* vsrc,
                                                const lds_u32x4* __restrict__ ck, const lds_u32x4* __restrict__ cv,
                                                lds_u32x4* __restrict__ nk, lds_u32x4* __restrict__ nv) {
  constexpr int KS = HD / 32, DT = HD / 16, NT = PF_TOK / 16;
  constexpr int PIECES = 64 * HD / 8;  // 16-byte pieces of one block's K (and of its V^T)
  const int g = lane >> 4, w = threadIdx.x >> 6;
  if constexpr (SHARED) {
    // this block's copy landed (the only loads in flight: an explicit wait, since a workgroup
    // barrier does not wait for global-to-LDS loads) and every wave is done with the buffer the next
    // copy overwrites (it held block b - 1). The barrier is __syncthreads (not inline assembly) so
    // the compiler sees it and places its own wait for the copy there, not before the fragment reads.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (b + 1 < n_blk) {
      // wave w, load i copies pieces 256 i + 64 w + lane of block b + 1's K and V^T
      const size_t off = (size_t)(b + 1) * PIECES + 64 * w;
#pragma unroll
      for (int i = 0; i < PIECES / 256; ++i) {
        __builtin_amdgcn_global_load_lds((const void*)(ksrc + off + 256 * i),
                                         (__attribute__((address_space(3))) void*)(nk + 256 * i + 64 * w), 16, 0, 0);
        __builtin_amdgcn_global_load_lds((const void*)(vsrc + off + 256 * i),
                                         (__attribute__((address_space(3))) void*)(nv + 256 * i + 64 * w), 16, 0, 0);
      }
    }
  }
  // K first: the scores of both row tiles; V is read while the softmax runs (K and V are not live
  // together, which keeps the wave inside 256 registers)
  u32x4_t kf[4][KS];
#pragma unroll
  for (int kt = 0; kt < 4; ++kt)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if constexpr (SHARED) kf[kt][ks] = ck[(kt * KS + ks) * 64 + lane];
      else kf[kt][ks] = *(const u32x4_t*)(kb + (size_t)b * 64 * HD + (kt * KS + ks) * 512);
    }
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
      for (int kt = 0; kt < 4; ++kt) s[rt][kt] = mfma16x16x32(bits_bf16x8(kf[kt][ks]), bits_bf16x8(st.qf[rt][ks]), s[rt][kt]);
  u32x4_t vf[DT][2];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    if constexpr (SHARED) {
      vf[dt][0] = cv[(dt * 2) * 64 + lane];
      vf[dt][1] = cv[(dt * 2 + 1) * 64 + lane];
    } else {
      vf[dt][0] = *(const u32x4_t*)(vb + (size_t)b * 64 * HD + (dt * 2) * 512);
      vf[dt][1] = *(const u32x4_t*)(vb + (size_t)b * 64 * HD + (dt * 2 + 1) * 512);
    }
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
    // Softmax in base 2 with the score scale folded into the exponent: p = 2^(s c - m), m a running
    // reference in scaled units. The reference only moves up when a block's maximum exceeds it by
    // more than 8 (so p <= 2^8 stays exact enough in fp32 and in the bf16 P operand); otherwise O
    // and l keep their scale and O is not rescaled -- for the whole wave when no row of it moved.
    // Every row attends key 0, so the first block sets a finite reference.
    float sv[16], mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float v = s[rt][kt][e];
        if (masked && b * 64 + pf_perm_key(kt, 4 * g + e) > st.lim[rt]) v = -INFINITY;
        sv[kt * 4 + e] = v;
        mx = fmaxf(mx, v);
      }
    mx = pf_max_lanes(mx) * scale_log2;
    const bool grow = mx > st.m_run[rt] + 8.f;  // true in the first block (m_run = -inf)
    const float m_use = grow ? mx : st.m_run[rt];
    const float alpha = grow ? __builtin_amdgcn_exp2f(st.m_run[rt] - mx) : 1.f;
    float l = 0.f;
    uint32_t pw[2][4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int e = 0; e < 4; e += 2) {
        const float p0 = __builtin_amdgcn_exp2f(fmaf(sv[kt * 4 + e], scale_log2, -m_use));
        const float p1 = __builtin_amdgcn_exp2f(fmaf(sv[kt * 4 + e + 1], scale_log2, -m_use));
        l += p0 + p1;
        pw[kt >> 1][(kt & 1) * 2 + e / 2] = pack_bf16x2(p0, p1);
      }
    l = pf_sum_lanes(l);
    st.l_run[rt] = st.l_run[rt] * alpha + l;
    st.m_run[rt] = m_use;
    if (__builtin_amdgcn_ballot_w64(grow)) {  // wave-uniform: multiplying by alpha = 1 is exact
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) st.o[rt][dt] = st.o[rt][dt] * alpha;
    }
    const u32x4_t pb0 = {pw[0][0], pw[0][1], pw[0][2], pw[0][3]};
    const u32x4_t pb1 = {pw[1][0], pw[1][1], pw[1][2], pw[1][3]};
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) st.o[rt][dt] = mfma16x16x32(bits_bf16x8(vf[dt][0]), bits_bf16x8(pb0), st.o[rt][dt]);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) st.o[rt][dt] = mfma16x16x32(bits_bf16x8(vf[dt][1]), bits_bf16x8(pb1), st.o[rt][dt]);
  }
}

// SHARED: the workgroup's four waves are four q heads of one kv head, so each 64-key block of K and
// V^T is copied once per workgroup into LDS (direct global-to-LDS loads, 16 bytes per lane, the
// cache layout kept) one block ahead of its use, and the waves read their MFMA fragments from there;
// otherwise every wave loads its block's K and V straight into registers when it needs them. The
// fragments and their order are the same either way, so the outputs are bit-identical.
template <int HD, bool SHARED>
__global__ __launch_bounds__(256, 2) void prefill_attention_kernel(const bf16_t* __restrict__ Q, int64_t ldq, int M,
                                                                   int pos0, int heads, int kv_heads,
                                                                   const bf16_t* __restrict__ Kc,
                                                                   const bf16_t* __restrict__ Vt, int64_t max_len,
                                                                   float scale_log2, bf16_t* __restrict__ out,
                                                                   int64_t ldo, int n_tt) {
  constexpr int KS = HD / 32, DT = HD / 16, NT = PF_TOK / 16;
  constexpr int PIECES = 64 * HD / 8;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int n_hg = (heads + 3) / 4;
  // the longest token tiles first (their rows attend the most keys)
  const int tt = n_tt - 1 - (int)blockIdx.x / n_hg;
  const int h = ((int)blockIdx.x % n_hg) * 4 + w;
  if (!SHARED && h >= heads) return;  // SHARED launches have heads % 4 == 0 (no wave leaves early)
  const int kvh = h / (heads / kv_heads);
  const int t0 = tt * PF_TOK;
  const bf16_t* kb = Kc + (size_t)kvh * max_len * HD + lane * 8;
  const bf16_t* vb = Vt + (size_t)kvh * max_len * HD + lane * 8;
  // this kv head's blocks as 16-byte pieces (per lane) for the LDS copies
  const u32x4_t* ksrc = (const u32x4_t*)(Kc + (size_t)kvh * max_len * HD) + lane;
  const u32x4_t* vsrc = (const u32x4_t*)(Vt + (size_t)kvh * max_len * HD) + lane;

  PfAttnState<HD> st;
#pragma unroll
  for (int rt = 0; rt < NT; ++rt) {
    const int tok = min(t0 + rt * 16 + j, M - 1);
    st.lim[rt] = pos0 + t0 + rt * 16 + j;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      st.qf[rt][ks] = *(const u32x4_t*)(Q + (size_t)tok * ldq + (size_t)h * HD + ks * 32 + g * 8);
    st.m_run[rt] = -INFINITY;
    st.l_run[rt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) st.o[rt][dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  const int last = pos0 + min(t0 + PF_TOK, M) - 1;  // the tile's last attended key
  const int n_blk = last / 64 + 1;
  const int full_blk = (pos0 + t0) / 64;  // blocks every row of the tile attends entirely

  // two K / V^T buffers (SHARED): blocks alternate between them
  constexpr int BUF = SHARED ? PIECES : 1;
  [[maybe_unused]] __shared__ __align__(16) u32x4_t kA[BUF], vA[BUF], kB[BUF], vB[BUF];
  typedef __attribute__((address_space(3))) u32x4_t* lp;
  if constexpr (SHARED) {
#pragma unroll
    for (int i = 0; i < PIECES / 256; ++i) {
      __builtin_amdgcn_global_load_lds((const void*)(ksrc + 256 * i + 64 * w),
                                       (__attribute__((address_space(3))) void*)((lp)kA + 256 * i + 64 * w), 16, 0, 0);
      __builtin_amdgcn_global_load_lds((const void*)(vsrc + 256 * i + 64 * w),
                                       (__attribute__((address_space(3))) void*)((lp)vA + 256 * i + 64 * w), 16, 0, 0);
    }
  }
  // blocks in pairs: each instance of the body reads one buffer and fills the other
  for (int b = 0; b < n_blk; b += 2) {
    pf_attend_block<HD, SHARED>(st, b, n_blk, full_blk, last, scale_log2, lane, kb, vb, ksrc, vsrc, (lp)kA, (lp)vA,
                                (lp)kB, (lp)vB);
    if (b + 1 < n_blk)
      pf_attend_block<HD, SHARED>(st, b + 1, n_blk, full_blk, last, scale_log2, lane, kb, vb, ksrc, vsrc, (lp)kB,
                                  (lp)vB, (lp)kA, (lp)vA);
  }
  // lane (g, j) of o[rt][dt] holds dims 16 dt + 4 g + e of row j
#pragma unroll
  for (int rt = 0; rt < NT; ++rt) {
    const int tok = t0 + rt * 16 + j;
    if (tok >= M) continue;
    const float inv = 1.f / st.l_run[rt];
    bf16_t* dst = out + (size_t)tok * ldo + (size_t)h * HD;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const uint32_t lo = pack_bf16x2(st.o[rt][dt][0] * inv, st.o[rt][dt][1] * inv);
      const uint32_t hi = pack_bf16x2(st.o[rt][dt][2] * inv, st.o[rt][dt][3] * inv);
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
  const int xt = epi == EPI_QKV ? 6 : 8;  // weight tiles per wave: 192- or 256-column workgroup tiles
  const int n_mt = (a.M + P4_BM - 1) / P4_BM;
  const int n_nt = (a.N + 32 * xt - 1) / (32 * xt);
  const int per_xcd = max((cus / 8) & ~3, 4);  // one workgroup per CU
  const int sb_m = n_mt < 4 ? n_mt : 4;
  const int sb_n = per_xcd / sb_m;
  const int grid = 8 * sb_n * sb_m;
#define PF4_LAUNCH(E, R, X)                                                                                     \
  SSD_LAUNCH((prefill_gemm4_kernel<E, R, X>), dim3(grid), dim3(256), 0, s, a, group, n_mt, n_nt, pos0, sb_n, sb_m)
#define PF4_SCALES(E, X)                   \
  if (a.row_scale) PF4_LAUNCH(E, true, X); \
  else PF4_LAUNCH(E, false, X);
  if (epi == EPI_SWIGLU) {
    PF4_SCALES(EPI_SWIGLU, 8);
  } else if (epi == EPI_QKV) {
    PF4_SCALES(EPI_QKV, 6);
  } else {
    PF4_SCALES(EPI_STORE, 8);
  }
#undef PF4_SCALES
#undef PF4_LAUNCH
  return check_launch("prefill_gemm4");
}

static int launch_prefill_gemm(GemmArgs a, int group, int pos0, int epi, hipStream_t s) {
  static int cus_of[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return set_error(SSD_EHIP, "prefill gemm: no current device");
  int cus = dev >= 0 && dev < 64 ? cus_of[dev] : 0;
  if (cus <= 0) {
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    if (dev >= 0 && dev < 64) cus_of[dev] = cus;
  }
  return launch_prefill_gemm4(a, group, pos0, epi, cus, s);
}

static int check_packed(int N, int K, int group) {
  if (N <= 0 || K <= 0 || K % 64) return set_error(SSD_EINVAL, "prefill gemm: N=%d K=%d (K %% 64 == 0)", N, K);
  const int tiles = (N + 127) / 128 * 8;  // packed row tiles (rows padded to 128)
  if (group < 1 || group > 16 || tiles % group)
    return set_error(SSD_EINVAL, "prefill gemm: group %d does not divide the %d row tiles", group, tiles);
  return SSD_OK;
}

}  // namespace ssd

using namespace ssd;

static int launch_row_scale(const uint16_t* X, int64_t ldx, int M, int K, float eps, float* rs, hipStream_t s) {
  SSD_LAUNCH(prefill_rowscale_kernel, dim3((M + 3) / 4), dim3(256), 0, s, (const bf16_t*)X, ldx, M, K, eps, rs);
  return check_launch("prefill_row_scale");
}

// Row scales of the RMSNorm folded into a prefill GEMM's packed weight: rs[m] = rsqrt(mean(X[m, :K]^2)
// + eps), one wave per row in a fixed order (a row's scale does not depend on M).
SSD_API int ssd_prefill_row_scale_bf16(const uint16_t* X, int64_t ldx, int M, int K, float eps, float* row_scale,
                                       hipStream_t stream) {
  if (!X || !row_scale) return set_error(SSD_EINVAL, "prefill row scale: null pointer");
  if (M <= 0 || K <= 0 || K % 8 || ldx < K || ldx % 8 || ((uintptr_t)X & 15) || !(eps > 0.f))
    return set_error(SSD_EINVAL, "prefill row scale: M=%d K=%d ldx=%lld eps=%g (16-byte rows, eps > 0)", M, K,
                     (long long)ldx, (double)eps);
  return launch_row_scale(X, ldx, M, K, eps, row_scale, stream);
}

// Y = epilogue(X W^T) with the folded RMSNorm's row scales (row_scale, [M] floats from
// ssd_prefill_row_scale_bf16) applied to the products, or none (row_scale null).
SSD_API int ssd_prefill_gemm_bf16(const uint16_t* X, int64_t ldx, int M, const uint16_t* W_packed, int group, int N,
                                  int K, const float* row_scale, int epi, uint16_t* Y, int64_t ldy,
                                  const uint16_t* residual, int64_t ldr, const SsdQkvEpilogue* qkv,
                                  hipStream_t stream) {
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
  a.Y = Y; a.ldy = ldy; a.residual = residual; a.ldr = ldr;
  a.row_scale = row_scale;
  int pos0 = 0;
  if (epi == SSD_EPI_QKV) {
    if (!qkv || !qkv->cos || !qkv->sin || !qkv->k_cache || !qkv->vt_cache)
      return set_error(SSD_EINVAL, "prefill gemm: q/k/v epilogue needs rotary tables and the cache");
    const int hd = qkv->head_dim;
    if ((hd != 32 && hd != 64 && hd != 128) || qkv->heads <= 0 || qkv->kv_heads <= 0 ||
        N != (qkv->heads + 2 * qkv->kv_heads) * hd || ldy < (int64_t)qkv->heads * hd)
      return set_error(SSD_EINVAL, "prefill gemm: q/k/v shape N=%d heads=%d kv=%d hd=%d", N, qkv->heads,
                       qkv->kv_heads, hd);
    if (((uintptr_t)qkv->k_cache & 15) || ((uintptr_t)qkv->vt_cache & 15) || ((uintptr_t)qkv->cos & 15) ||
        ((uintptr_t)qkv->sin & 15))
      return set_error(SSD_EINVAL, "prefill gemm: caches and rotary tables must be 16-byte aligned");
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
  // a workgroup's four waves share one kv head's K/V when 4 divides the q heads per kv head
  const bool shared = (heads / kv_heads) % 4 == 0;
#define PF_ATT(D, SH)                                                                                         \
  SSD_LAUNCH((prefill_attention_kernel<D, SH>), grid, block, 0, stream, (const bf16_t*)q, ldq, M, pos0, heads, \
             kv_heads, (const bf16_t*)k_cache, (const bf16_t*)vt_cache, max_len, sl2, (bf16_t*)out, ldo, n_tt)
  switch (head_dim) {
    case 64:
      if (shared) PF_ATT(64, true);
      else PF_ATT(64, false);
      break;
    case 128:
      if (shared) PF_ATT(128, true);
      else PF_ATT(128, false);
      break;
    default:
      return set_error(SSD_EINVAL, "prefill attention: head_dim %d unsupported (64, 128)", head_dim);
  }
#undef PF_ATT
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
    // the input norm's row scales, computed once per row into the attention buffer (free until the
    // attention writes it)
    float* rs_qkv = (float*)pb->attn;
    if ((rc = launch_row_scale(pb->h, d, m, d, md->eps, rs_qkv, s))) return rc;
    if ((rc = ssd_prefill_gemm_bf16(pb->h, d, m, L.wqkv, g_qkv, nqkv, d, rs_qkv, SSD_EPI_QKV, pb->q, qdim, nullptr, 0,
                                    &qe, s)))
      return rc;
    if ((rc = ssd_prefill_attention_bf16(pb->q, qdim, m, pos0, H, KV, hd, qe.k_cache, qe.vt_cache, pb->cache_cap,
                                         md->attn_scale, pb->attn, qdim, s)))
      return rc;
    if ((rc = ssd_prefill_gemm_bf16(pb->attn, qdim, m, L.wo, g_o, d, (int)qdim, nullptr, SSD_EPI_STORE, pb->h, d, pb->h,
                                    d, nullptr, s)))
      return rc;
    // gate/up's norm scales computed once per row into the q buffer (free after the attention)
    float* rs = (float*)pb->q;
    if ((rc = launch_row_scale(pb->h, d, m, d, md->eps, rs, s))) return rc;
    if ((rc = ssd_prefill_gemm_bf16(pb->h, d, m, L.wgu, g_gu, 2 * I, d, rs, SSD_EPI_SWIGLU, pb->act, I, nullptr, 0,
                                    nullptr, s)))
      return rc;
    if ((rc = ssd_prefill_gemm_bf16(pb->act, I, m, L.wd, g_d, d, I, nullptr, SSD_EPI_STORE, pb->h, d, pb->h, d, nullptr,
                                    s)))
      return rc;
  }
  if (head_w)
    return ssd_gemm_bf16(pb->h + (size_t)(m - 1) * d, d, 1, head_w, md->vocab, d, md->eps, pb->logits, md->vocab,
                         nullptr, 0, nullptr, 0, s);
  return SSD_OK;
}
