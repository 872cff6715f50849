// Tree attention for decode on gfx950: a small block of query rows (tree nodes,
// the root, or one autoregressive token) against the single shared KV cache.
//
// Row model. Query token t attends, in *logical* key order:
//   logical positions [0, P_t)        -> cache slots [0, P_t)            (prefix)
//   logical positions [P_t, P_t + D_t) -> cache slots anc[t][0..D_t)     (ancestors
//                                         in depth order, self included)
// so its logical length is L_t = P_t + D_t. An autoregressive step is P = L,
// D = 0; a verify node at depth k is P = committed + 1, D = k; a causal prefill
// chunk row is P = past + t + 1, D = 0. This is the reference's boolean mask
// (ssd/models/subnetwork_draft.py:165-191, ssd/engine/verify.py:37-41,
// ssd/engine/tree_drafter.py:189-196) written as a gather list.
//
// Canonical arithmetic (what makes greedy speculative output bit-identical to
// plain greedy decoding): keys are cut into 64-key blocks by logical position.
// Each block gives a partial (m, l, O) with its own max; the blocks of a
// 256-key superblock are folded left to right, then the superblocks are folded
// left to right. That structure depends only on (q, the row's logical keys),
// never on how many rows share the call or where the tree slots sit, so a
// verify row reproduces the autoregressive step at the same position exactly.
//
// Kernel structure: attn_partial computes one (m, l, O) partial per (row, superblock) into a
// workspace -- superblocks below min(P) by workgroups that serve every row at once, the rest by
// one workgroup per token -- and attn_combine folds the superblocks of each row. S^T = K Q^T and
// O^T = V^T P^T both run on v_mfma_f32_16x16x32_bf16; the key order inside a block is permuted so
// the score accumulators are already the P^T operand (no LDS transpose). Row max/sum use
// cross-lane shuffles of the wave64.
#include "common.h"

#include <math.h>

namespace ssd {

constexpr int ATT_BLK = 64;
constexpr int ATT_SB = 4;        // blocks per superblock
constexpr int ATT_MAXD = 32;     // gathered tree slots per row

struct AttnArgs {
  const bf16_t* Q;  // [M, heads*hd] (row stride ldq)
  int64_t ldq;
  const bf16_t* K;   // this layer: kv_heads x (max_len x hd), 64-slot block layout (k_off in common.h)
  const bf16_t* Vt;  // this layer: kv_heads x (max_len x hd), 64-slot block layout (v_off in common.h)
  int64_t max_len;
  int M, heads, kv_heads;
  const int* prefix;  // [M]
  const int* depth;   // [M]
  const int* anc;     // [M, ATT_MAXD]
  const int64_t* kv_off;  // [M] element offset of token t's sequence in the K / V arenas, or null
  int p_min, l_max;
  float scale_log2;
  float* ws;  // fp16 O / l [kv_heads][M*rep][n_sb_cap][hd], then fp32 (m, l) [kv_heads][M*rep][n_sb_cap]
  int n_sb_cap;
  // launch geometry (set by launch_attn)
  int n_full;         // superblocks entirely below p_min (shared by every row)
  int n_tail_sb;      // superblocks from n_full up to l_max (built per token)
  int tail_slots;     // workgroup ids [0, tail_slots) are tail workgroups
  int groups, tiles_per_group;  // row tile groups of the shared workgroups
  uint32_t rep_magic;  // ceil(2^32 / (heads / kv_heads)): R / rep == umulhi(R, rep_magic) for R < 2^16
};

typedef _Float16 h16x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int perm_key(int kt, int i) {
  // key offset (within a 64-key block) that sits in row i of key tile kt
  return (kt >> 1) * 32 + (i >> 2) * 8 + (kt & 1) * 4 + (i & 3);
}

template <int HD>
struct Frags {
  static constexpr int KS = HD / 32;  // k-steps over head_dim for Q K^T
  static constexpr int DT = HD / 16;  // 16-wide d tiles for P V
  u32x4_t k[4][KS];
  u32x4_t v[DT][2];
};

// The block's operand tiles are stored in lane order (cache block layout), so each tile is one
// contiguous 1 KiB load: lane l gets elements [8l, 8l + 8) of the tile.
template <int HD>
__device__ __forceinline__ void load_shared_frags(Frags<HD>& f, const AttnArgs& a, int kvh, int key0, int lane) {
  constexpr int KS = Frags<HD>::KS, DT = Frags<HD>::DT;
  const bf16_t* kb = a.K + (size_t)kvh * a.max_len * HD + (size_t)(key0 >> 6) * 64 * HD + lane * 8;
#pragma unroll
  for (int kt = 0; kt < 4; ++kt)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) f.k[kt][ks] = *(const u32x4_t*)(kb + (kt * KS + ks) * 512);
  const bf16_t* vb = a.Vt + (size_t)kvh * HD * a.max_len + (size_t)(key0 >> 6) * 64 * HD + lane * 8;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    f.v[dt][0] = *(const u32x4_t*)(vb + (dt * 2) * 512);
    f.v[dt][1] = *(const u32x4_t*)(vb + (dt * 2 + 1) * 512);
  }
}

// Logical key -> cache slot for token t (-1 = not attended; out-of-range slots are dropped).
__device__ __forceinline__ int logical_slot(int jpos, int P, int L, const int* anc_t, int64_t max_len) {
  int s = -1;
  if (jpos < P) s = jpos;
  else if (jpos < L && jpos - P < ATT_MAXD) s = anc_t[jpos - P];
  return (s >= 0 && s < max_len) ? s : -1;
}

// One token's block at logical positions [key0, key0 + 64): positions < P are cache slots
// themselves, positions in [P, L) are the ancestor slots anc[pos - P], the rest is empty (zero).
// K rows are loaded per key. V^T is loaded as for a prefix block (one 16-byte run of 8 positions
// per lane, positions >= P masked to zero); the ancestor positions are patched in afterwards by
// patch_ancestors. Loads are unconditional (clamped, valid addresses; values masked
// afterwards): a load under a per-lane condition compiles to a branch after which the compiler
// waits for the value, serialising the loads.
template <int HD>
__device__ __forceinline__ void load_virtual_frags(Frags<HD>& f, const AttnArgs& a, const bf16_t* K,
                                                   const bf16_t* Vt, int kvh, int key0, int P, int L,
                                                   const int* anc_t, int lane) {
  const int i = lane & 15, g = lane >> 4;
  const bf16_t* kb = K + (size_t)kvh * a.max_len * HD;
#pragma unroll
  for (int kt = 0; kt < 4; ++kt) {
    const int slot = logical_slot(key0 + perm_key(kt, i), P, L, anc_t, a.max_len);
    const int sl = slot < 0 ? 0 : slot;
    const uint32_t keep = slot >= 0 ? 0xffffffffu : 0u;
#pragma unroll
    for (int ks = 0; ks < Frags<HD>::KS; ++ks) f.k[kt][ks] = *(const u32x4_t*)(kb + k_off(sl, ks * 32 + g * 8, HD)) & keep;
  }
  const bf16_t* vb = Vt + (size_t)kvh * HD * a.max_len;
  const int lim = P < a.max_len ? P : (int)a.max_len;  // prefix positions that exist
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int pos0 = key0 + c * 32 + g * 8;
    const int base = pos0 + 8 <= a.max_len ? pos0 : 0;
    u32x4_t keep;
#pragma unroll
    for (int w2 = 0; w2 < 4; ++w2)
      keep[w2] = (pos0 + 2 * w2 < lim ? 0x0000ffffu : 0u) | (pos0 + 2 * w2 + 1 < lim ? 0xffff0000u : 0u);
#pragma unroll
    for (int dt = 0; dt < Frags<HD>::DT; ++dt)
      f.v[dt][c] = *(const u32x4_t*)(vb + v_off(base, dt * 16 + i, HD)) & keep;
  }
}

// Patch the ancestor positions of this block into the V^T operands from the ancestors' V^T
// columns staged in LDS (avt[a][d], a < D): wave-uniform loop over the ancestors in the block.
template <int HD>
__device__ __forceinline__ void patch_ancestors(Frags<HD>& f, const bf16_t (*avt)[HD], int key0, int P, int L,
                                                int lane) {
  const int i = lane & 15, g = lane >> 4;
  const int a_lo = (key0 > P ? key0 : P) - P;
  const int a_hi = (L < key0 + ATT_BLK ? L : key0 + ATT_BLK) - P;
  for (int an = a_lo; an < a_hi; ++an) {
    const int off = P + an - key0;  // 0..63, uniform
    const int c = off >> 5, grp = (off >> 3) & 3, t = off & 7;
    const uint32_t sel = g == grp ? ((t & 1) ? 0xffff0000u : 0x0000ffffu) : 0u;
#pragma unroll
    for (int dt = 0; dt < Frags<HD>::DT; ++dt) {
      const uint32_t h = avt[an][dt * 16 + i];
      const uint32_t v = (h | (h << 16)) & sel;
#pragma unroll
      for (int w2 = 0; w2 < 4; ++w2) {
        const uint32_t m = (t >> 1) == w2 ? sel : 0u;
        if (c == 0) f.v[dt][0][w2] = (f.v[dt][0][w2] & ~m) | (v & m);
        else f.v[dt][1][w2] = (f.v[dt][1][w2] & ~m) | (v & m);
      }
    }
  }
}

// Reductions over lanes j, j ^ 16 (and j ^ 32) with gfx950's v_permlane16/32_swap (VALU, no LDS
// round trip): swapping a value with itself leaves {own, partner} in the pair, in the same order
// on both lanes, so both get the same result.
__device__ __forceinline__ float pair_max16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_max32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float pair_sum32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// One 64-key block for a 16-row tile. valid_bits: bit (kt*4+e) says whether key perm_key(kt, 4g+e)
// is attended (same for every row of the pass). Outputs per lane (row j = lane%16): m (log2 units,
// -inf if nothing attended), l, and O[row j][dt*16 + 4g + e] in o[dt][e].
// exp2 for the softmax: the bare hardware instruction (results below 2^-126 flush to zero, which
// every path shares).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

template <int HD, bool MASKED>
__device__ __forceinline__ void block_attend(const Frags<HD>& f, const u32x4_t (&qf)[HD / 32], uint32_t valid_bits,
                                             float scale_log2, float& m_out, float& l_out,
                                             f32x4_t (&o)[HD / 16]) {
  // No multiply-add contraction: the masked instance has a select between s * scale_log2 and the
  // exponent's subtraction, the unmasked one does not, and a fused multiply-subtract in one of them
  // only would give the two kinds of workgroup p values an ulp apart.
#pragma clang fp contract(off)
  constexpr int KS = HD / 32, DT = HD / 16;
  // k-step outer: consecutive MFMAs go to different accumulators (each sum keeps its ks order)
  f32x4_t s[4];
#pragma unroll
  for (int kt = 0; kt < 4; ++kt) s[kt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < KS; ++ks)
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) s[kt] = mfma16x16x32(bits_bf16x8(f.k[kt][ks]), bits_bf16x8(qf[ks]), s[kt]);
  float sv[16];
  float mx = -INFINITY;
#pragma unroll
  for (int kt = 0; kt < 4; ++kt)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float v = s[kt][e] * scale_log2;
      if (MASKED) v = ((valid_bits >> (kt * 4 + e)) & 1u) ? v : -INFINITY;
      sv[kt * 4 + e] = v;
      mx = fmaxf(mx, v);
    }
  mx = pair_max16(mx);
  mx = pair_max32(mx);
  m_out = mx;
  // A row with nothing attended gets p = 0 everywhere (m stays -inf and marks it absent).
  // No early exit: every lane must stay active for the MFMAs below.
  const float msafe = (MASKED && mx == -INFINITY) ? 0.f : mx;
  float l = 0.f;
  // P^T operand: key tile kt, element e goes to half (kt & 1) * 4 + e of operand kt >> 1.
  uint32_t pw[2][4];
#pragma unroll
  for (int kt = 0; kt < 4; ++kt)
#pragma unroll
    for (int e = 0; e < 4; e += 2) {
      const float p0 = fast_exp2(sv[kt * 4 + e] - msafe), p1 = fast_exp2(sv[kt * 4 + e + 1] - msafe);
      l += p0;
      l += p1;
      pw[kt >> 1][(kt & 1) * 2 + e / 2] = pack_bf16x2(p0, p1);
    }
  l = pair_sum16(l);
  l = pair_sum32(l);
  l_out = l;
  const u32x4_t pb0 = {pw[0][0], pw[0][1], pw[0][2], pw[0][3]};
  const u32x4_t pb1 = {pw[1][0], pw[1][1], pw[1][2], pw[1][3]};
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) o[dt] = mfma16x16x32(bits_bf16x8(f.v[dt][0]), bits_bf16x8(pb0), f32x4_t{0.f, 0.f, 0.f, 0.f});
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) o[dt] = mfma16x16x32(bits_bf16x8(f.v[dt][1]), bits_bf16x8(pb1), o[dt]);
}

// The four block partials of a row tile meet in LDS; two such areas alternate between consecutive
// tiles, so one barrier per tile suffices (see the tile loop).
template <int HD>
struct alignas(16) AttnLds {
  float o[2][ATT_SB][16][HD + 4];
  float m[2][ATT_SB][16];
  float l[2][ATT_SB][16];
  bf16_t avt[ATT_MAXD][HD];  // tail: the token's ancestors' V^T columns
};

// One launch holds two kinds of workgroups (4 waves; wave w owns block 4*sb + w):
//  * tail:   (superblock at or beyond min(P), kv head, one token), dispatched first. The wave
//    builds its block from the token's logical keys (prefix slots, then ancestor slots) and
//    processes the token's GQA rows.
//  * shared: (superblock below min(P), kv head, tile group). Every row attends every key of the
//    superblock; the wave loads its block's K and V^T into MFMA operand registers once and runs
//    every 16-row tile of its group against them. The groups of a superblock sit on one XCD, so
//    K/V bytes come from HBM once and the other groups read them from that XCD's L2.
// Each wave loads the query fragments of a row tile straight from memory, one tile ahead (the first
// tile's loads are issued before the K/V loads). Both kinds end in the same code: the four block
// partials of a tile meet in LDS and are folded left to right into the superblock partial, so a
// superblock's result does not depend on which kind of workgroup produced it. Ids are decoded XCD-aware: the workgroups that read one (superblock, kv head)
// -- its tokens (tail) or tile groups (shared) -- get ids 8 apart, i.e. one XCD (workgroups are
// dealt to the 8 XCDs round-robin), so their re-reads of that K/V hit the XCD's L2.
//
// Workspace: normalised O partials (O / l, fp16) [kv_heads][M*rep][n_sb_cap][HD], then fp32 (m, l) pairs
// [kv_heads][M*rep][n_sb_cap].
// Every (row, superblock < n_sb) pair of the call is written; m = -inf marks "no keys".
template <int HD>
__global__ __launch_bounds__(256, 2) void attn_partial_kernel(AttnArgs a) {
  constexpr int KS = HD / 32, DT = HD / 16;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int rep = a.heads / a.kv_heads;
  const int n_rows = a.M * rep;
  const bool tail = (int)blockIdx.x < a.tail_slots;
  int sb, kvh, tok = 0, grp = 0;
  if (tail) {
    const int bid = blockIdx.x, xcd = bid & 7, rest = bid >> 3;
    const int u = (rest / a.M) * 8 + xcd;
    tok = rest % a.M;
    if (u >= a.n_tail_sb * a.kv_heads) return;
    sb = a.n_full + u / a.kv_heads;
    kvh = u % a.kv_heads;
  } else {
    const int bid = blockIdx.x - a.tail_slots, xcd = bid & 7, rest = bid >> 3;
    const int u = (rest / a.groups) * 8 + xcd;
    grp = rest % a.groups;
    if (u >= a.n_full * a.kv_heads) return;
    sb = u / a.kv_heads;
    kvh = u % a.kv_heads;
  }
  const int key0 = (sb * ATT_SB + w) * ATT_BLK;
  _Float16* ws_o = (_Float16*)a.ws;
  float2* ws_ml = (float2*)(a.ws + (size_t)a.kv_heads * n_rows * a.n_sb_cap * (HD / 2));

  __shared__ AttnLds<HD> lds;
  __shared__ int s_anc[ATT_MAXD];
  int r_begin, r_end, P = 0, L = 0, anc_v = 0;
  const bf16_t* Kt = a.K;  // this token's sequence (tail workgroups of a multi-sequence call)
  const bf16_t* Vtt = a.Vt;
  if (tail) {
    if (a.kv_off) {
      const int64_t off = a.kv_off[tok];
      Kt += off;
      Vtt += off;
    }
    anc_v = a.anc[(size_t)tok * ATT_MAXD + (threadIdx.x & (ATT_MAXD - 1))];
    P = a.prefix[tok];
    L = P + min(max(a.depth[tok], 0), ATT_MAXD);
    r_begin = tok * rep;
    r_end = r_begin + rep;
  } else {
    r_begin = grp * a.tiles_per_group * 16;
    r_end = min(n_rows, r_begin + a.tiles_per_group * 16);
  }

  // Query fragments of the 16-row tile starting at row t0 (R = token * rep + GQA head within the kv
  // group): lane (j, g) holds row t0 + j, dims ks * 32 + 8g ... + 8 -- the MFMA B operand. Rows at
  // or past r_end load row r_begin (a valid address): every score, softmax and output column
  // belongs to one row, so a padding row only produces its own partial, which is never stored.
  auto load_qf = [&](int t0, u32x4_t (&qf)[KS]) {
    const int R = t0 + j < r_end ? t0 + j : r_begin;
    const int qt = (int)__umulhi((uint32_t)R, a.rep_magic);
    const bf16_t* qp = a.Q + (size_t)qt * a.ldq + (size_t)(kvh * rep + R - qt * rep) * HD + g * 8;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qf[ks] = *(const u32x4_t*)(qp + ks * 32);
  };
  u32x4_t qn[KS];
  load_qf(r_begin, qn);

  Frags<HD> f;
  uint32_t bits = 0xffffu;
  bool have = true;
  if (tail) {
    if (sb * ATT_SB * ATT_BLK >= L) {  // the token's keys end before this superblock
      for (int r = threadIdx.x; r < rep; r += 256)
        ws_ml[((size_t)kvh * n_rows + r_begin + r) * a.n_sb_cap + sb] = make_float2(-INFINITY, 0.f);
      return;
    }
    if (threadIdx.x < ATT_MAXD) s_anc[threadIdx.x] = anc_v;
    __syncthreads();
    // The ancestors' V^T columns (L - P of them) go to LDS; their loads are issued before the
    // block's K/V loads and land while those are in flight.
    const bool patch = L > P;
    constexpr int AIT = ATT_MAXD * HD / 256;
    uint32_t av[AIT];
    const int n_av = (L - P) * HD;  // (ancestor, d) pairs to stage
    if (patch) {
      const bf16_t* vb = Vtt + (size_t)kvh * HD * a.max_len;
#pragma unroll
      for (int it = 0; it < AIT; ++it) {
        if (it * 256 >= n_av) break;  // uniform
        const int idx = threadIdx.x + it * 256;
        const int an = min(idx / HD, L - P - 1), d = idx % HD;
        const int slot = s_anc[an];
        const bool ok = slot >= 0 && slot < a.max_len;
        const uint32_t h = vb[v_off(ok ? slot : 0, d, HD)];
        av[it] = ok ? h : 0u;
      }
    }
    have = key0 < L;
    if (have) {
      load_virtual_frags<HD>(f, a, Kt, Vtt, kvh, key0, P, L, s_anc, lane);
      bits = 0;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (logical_slot(key0 + perm_key(kt, 4 * g + e), P, L, s_anc, a.max_len) >= 0) bits |= 1u << (kt * 4 + e);
    }
    if (patch) {
#pragma unroll
      for (int it = 0; it < AIT; ++it) {
        if (it * 256 >= n_av) break;  // uniform
        const int idx = threadIdx.x + it * 256;
        lds.avt[idx / HD][idx % HD] = (bf16_t)av[it];
      }
      __syncthreads();
      if (have) patch_ancestors<HD>(f, lds.avt, key0, P, L, lane);
    }
  } else {
    load_shared_frags<HD>(f, a, kvh, key0, lane);
  }

  // Row tiles in turn. Tile i's block partials go to LDS area i % 2; one barrier makes them visible
  // and the fold reads them. Area i % 2 is written next by tile i + 2, which no wave starts before
  // it has passed tile i + 1's barrier, i.e. before every wave has finished folding tile i. Query
  // fragments alternate between two register sets (a copy would wait for the previous tile's
  // stores when it reuses their registers).
  auto publish = [&](int buf, float m, float l, const f32x4_t (&o)[DT]) {
    lds.m[buf][w][j] = m;  // the four lanes of row j write the same value
    lds.l[buf][w][j] = l;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) *(f32x4_t*)&lds.o[buf][w][j][dt * 16 + 4 * g] = o[dt];
    __syncthreads();
  };
  // Fold the 4 block partials of each row of the tile at t0: superblock max first, then the
  // weighted sums in block order -> superblock partial. Branch-free, and every thread stores (threads of padding rows fold row nv - 1 again and
  // write the same values; a superblock without keys gets O = 0, which the combine never reads
  // since its m is -inf), so the number of stores per tile is fixed and the next tile's query
  // loads, issued before them, are waited for without waiting for the stores.
  auto fold = [&](int t0, int buf) {
    const int nv = min(16, r_end - t0);
    const int rr = min((int)threadIdx.x >> 4, nv - 1);  // tile row
    const int dc = threadIdx.x & 15;                    // d chunk
    constexpr int DPT = HD / 16;                        // d per thread
    float mb[ATT_SB], mS = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < ATT_SB; ++ww) {
      mb[ww] = lds.m[buf][ww][rr];
      mS = fmaxf(mS, mb[ww]);
    }
    float lS = 0.f, oS[DPT];
#pragma unroll
    for (int d = 0; d < DPT; ++d) oS[d] = 0.f;
    // A block without keys gets weight 0: its l and O in LDS are finite zeros (published by every
    // wave), and adding an exact zero leaves a sum that is never -0 unchanged, so this equals
    // skipping the block.
#pragma unroll
    for (int ww = 0; ww < ATT_SB; ++ww) {
      const float wgt = mb[ww] != -INFINITY ? fast_exp2(mb[ww] - mS) : 0.f;
      lS = fmaf(lds.l[buf][ww][rr], wgt, lS);
#pragma unroll
      for (int d = 0; d < DPT; ++d) oS[d] = fmaf(lds.o[buf][ww][rr][dc * DPT + d], wgt, oS[d]);
    }
    const size_t rec = ((size_t)kvh * n_rows + t0 + rr) * a.n_sb_cap + sb;
    // the superblock's normalised output O / l in fp16 (|O / l| <= max |v|; 0 without keys)
    const float inv = lS > 0.f ? 1.f / lS : 0.f;
    _Float16* dst = ws_o + rec * HD + dc * DPT;
    if constexpr (DPT % 4 == 0) {
#pragma unroll
      for (int d = 0; d < DPT; d += 4) {
        const h16x4_t q = {(_Float16)(oS[d] * inv), (_Float16)(oS[d + 1] * inv), (_Float16)(oS[d + 2] * inv),
                           (_Float16)(oS[d + 3] * inv)};
        *(h16x4_t*)(dst + d) = q;
      }
    } else {
#pragma unroll
      for (int d = 0; d < DPT; ++d) dst[d] = (_Float16)(oS[d] * inv);
    }
    ws_ml[rec] = make_float2(mS, lS);  // the same pair from each of the row's 16 threads
  };
  u32x4_t qa[KS];
  float m, l;
  f32x4_t o[DT];
  if (tail) {
    // one token's rows (rep <= 16 at every supported shape: one tile, at most a few): in turn
    for (int t0 = r_begin; t0 < r_end; t0 += 32) {
      load_qf(t0 + 16, qa);
      if (have) {
        block_attend<HD, true>(f, qn, bits, a.scale_log2, m, l, o);
      } else {
        m = -INFINITY;
        l = 0.f;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      }
      publish(0, m, l, o);
      fold(t0, 0);
      if (t0 + 16 >= r_end) break;  // uniform
      load_qf(t0 + 32, qn);
      if (have) {
        block_attend<HD, true>(f, qa, bits, a.scale_log2, m, l, o);
      } else {
        m = -INFINITY;
        l = 0.f;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      }
      publish(1, m, l, o);
      fold(t0 + 16, 1);
    }
  } else {
    // Shared workgroups run many tiles: software-pipelined, each wave folds tile i in the same
    // straight-line code that computes tile i + 1 (fold first, so its LDS reads and record stores
    // are issued before the next query loads and the MFMAs they overlap).
    load_qf(r_begin + 16, qa);
    block_attend<HD, false>(f, qn, bits, a.scale_log2, m, l, o);
    publish(0, m, l, o);
    // Nothing outstanding on entry to the loop: the compiler's wait counts at the loop head then
    // follow the loop's own order (query loads, then the fold's stores) and wait for the query
    // fragments only. With the prologue's loads still counted, its merged state placed a wait for
    // the previous tile's record stores in front of every other tile's MFMAs.
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0), lgkmcnt and expcnt not waited for
    for (int t0 = r_begin;; t0 += 32) {
      // tile t0 is in area 0, tile t0 + 16's query fragments in qa
      fold(t0, 0);
      if (t0 + 16 >= r_end) break;  // uniform
      load_qf(t0 + 32, qn);
      block_attend<HD, false>(f, qa, bits, a.scale_log2, m, l, o);
      publish(1, m, l, o);
      fold(t0 + 16, 1);
      if (t0 + 32 >= r_end) break;
      load_qf(t0 + 48, qa);
      block_attend<HD, false>(f, qn, bits, a.scale_log2, m, l, o);
      publish(0, m, l, o);
    }
  }
}

// Cross-superblock combine, one wave per (token, q head). Canonical arithmetic for a row with
// superblocks s = 0..n-1 (record: m_s, l_s and the normalised output o_s = O_s / l_s in fp16):
// M = max_s m_s; w_s = l_s 2^(m_s - M) (0 where m_s = -inf); L = sum_s w_s and O = sum_s o_s w_s,
// both summed in increasing s; out = O / L. The partials of up to 32 superblocks (a batch divides
// the 64-superblock window) are loaded in one batch, issued before the max is reduced.
template <int HD>
__global__ __launch_bounds__(256) void attn_combine_kernel(const float* __restrict__ ws, int n_sb_cap, int M,
                                                           int heads, int kv_heads, bf16_t* __restrict__ out,
                                                           int64_t ldo, int n) {
  constexpr int PER = (HD + 63) / 64;
  constexpr int CH = 32;
  const int wid = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (wid >= M * heads) return;
  const int tok = wid / heads, hq = wid % heads;
  const int rep = heads / kv_heads, kvh = hq / rep;
  const int n_rows = M * rep;
  const size_t row = (size_t)kvh * n_rows + tok * rep + hq % rep;
  const _Float16* O = (const _Float16*)ws + row * n_sb_cap * HD;
  const float2* ml = (const float2*)(ws + (size_t)kv_heads * n_rows * n_sb_cap * (HD / 2)) + row * n_sb_cap;
  // Lane s of a 64-superblock window holds record (m, l) of superblock window + s; the fold reads
  // it back with readlane (no registers per superblock).
  float v[CH][PER];
  // Unconditional loads from clamped indices (a per-lane conditional load would be waited for
  // one by one); entries past n are masked where they are used. At head_dim 128 lane l owns dims
  // 2l and 2l + 1 (one 4-byte load per record), otherwise dims l + 64 i.
  constexpr bool PAIRS = HD == 128;
  auto dim = [&](int i) { return PAIRS ? 2 * lane + i : min(lane + 64 * i, HD - 1); };
  auto load_chunk = [&](int s0) {
#pragma unroll
    for (int q = 0; q < CH; ++q) {
      const int sq = min(s0 + q, n - 1);
      if constexpr (PAIRS) {
        const uint32_t w = *(const uint32_t*)(O + (size_t)sq * HD + 2 * lane);
        v[q][0] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
        v[q][1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
      } else {
#pragma unroll
        for (int i = 0; i < PER; ++i) v[q][i] = (float)O[(size_t)sq * HD + dim(i)];
      }
    }
  };
  float2 win = ml[min(lane, n - 1)];
  load_chunk(0);
  float mx = win.x;
  for (int s = lane + 64; s < n; s += 64) mx = fmaxf(mx, ml[s].x);
  for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
  float l = 0.f, o[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) o[i] = 0.f;
  for (int s0 = 0;;) {
#pragma unroll
    for (int q = 0; q < CH; ++q) {
      const int ln = (s0 & 63) + q;
      const float mq = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(win.x), ln));
      const float lq = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(win.y), ln));
      const float wq = (s0 + q >= n || mq == -INFINITY) ? 0.f : lq * fast_exp2(mq - mx);
      if (wq != 0.f) {
        l += wq;
#pragma unroll
        for (int i = 0; i < PER; ++i) o[i] += v[q][i] * wq;
      }
    }
    s0 += CH;
    if (s0 >= n) break;
    if ((s0 & 63) == 0) win = ml[min(s0 + lane, n - 1)];
    load_chunk(s0);
  }
  bf16_t* dst = out + (size_t)tok * ldo + (size_t)hq * HD;
  if constexpr (PAIRS) {
    *(uint32_t*)(dst + 2 * lane) = pack_bf16x2(l > 0.f ? o[0] / l : 0.f, l > 0.f ? o[1] / l : 0.f);
  } else {
#pragma unroll
    for (int i = 0; i < PER; ++i)
      if (lane + 64 * i < HD) dst[lane + 64 * i] = f2bf(l > 0.f ? o[i] / l : 0.f);
  }
}

template <int HD>
static int launch_attn(AttnArgs a, bf16_t* out, int64_t ldo, hipStream_t s) {
  constexpr int SBK = ATT_BLK * ATT_SB;
  const int n_sb = (a.l_max + SBK - 1) / SBK;
  if (n_sb > a.n_sb_cap) return set_error(SSD_ERANGE, "attention: length %d needs %d superblocks > workspace %d",
                                          a.l_max, n_sb, a.n_sb_cap);
  // rows of several sequences share no keys: every superblock is built per token
  a.n_full = a.kv_off ? 0 : (a.p_min / SBK < n_sb ? a.p_min / SBK : n_sb);
  a.n_tail_sb = n_sb - a.n_full;
  a.tail_slots = (a.n_tail_sb * a.kv_heads + 7) / 8 * 8 * a.M;
  const uint32_t rep = (uint32_t)(a.heads / a.kv_heads);
  a.rep_magic = (uint32_t)((((uint64_t)1 << 32) + rep - 1) / rep);
  // Shared workgroups split their rows into tile groups when the chip has room for more
  // workgroups (about 2 per CU resident at once); the groups of one superblock share an XCD.
  const int units8 = (a.n_full * a.kv_heads + 7) / 8 * 8;
  const int n_tiles = (a.M * (a.heads / a.kv_heads) + 15) / 16;
  int groups = units8 ? (512 - a.tail_slots) / units8 : 1;
  groups = groups < 1 ? 1 : (groups > n_tiles ? n_tiles : groups);
  a.tiles_per_group = (n_tiles + groups - 1) / groups;
  a.groups = (n_tiles + a.tiles_per_group - 1) / a.tiles_per_group;
  const int grid = a.tail_slots + units8 * a.groups;
  if (grid > 0) {
    SSD_LAUNCH((attn_partial_kernel<HD>), dim3(grid), dim3(256), 0, s, a);
    const int rc = check_launch("attn_partial");
    if (rc) return rc;
  }
  const int waves = a.M * a.heads;
  SSD_LAUNCH((attn_combine_kernel<HD>), dim3((waves + 3) / 4), dim3(256), 0, s, a.ws, a.n_sb_cap, a.M,
                     a.heads, a.kv_heads, out, ldo, n_sb);
  return check_launch("attn_combine");
}

}  // namespace ssd

using namespace ssd;

SSD_API int ssd_attn_workspace_floats(int M, int heads, int head_dim, int64_t max_len) {
  const int64_t n_sb = (max_len + ATT_BLK * ATT_SB - 1) / (ATT_BLK * ATT_SB);
  return (int)((int64_t)M * heads * n_sb * (head_dim / 2 + 2));  // fp16 O / l, then fp32 (m, l)
}

SSD_API int ssd_attn_max_depth(void) { return ATT_MAXD; }

// out[t, h*hd:(h+1)*hd] = softmax over row t's logical keys (see header) of q.k/sqrt(hd), times v.
// q: [M, heads*hd] bf16 (post-RoPE); k_cache / vt_cache: kv_heads x (max_len x hd) each, in the
// 64-slot block layout (k_off / v_off in common.h).
// prefix/depth: [M] int32; anc: [M, 32] int32 slots; p_min <= min(prefix); l_max >= max(prefix+depth).
// ws: fp32 workspace of ssd_attn_workspace_floats(M, heads, hd, max_len) floats.
SSD_API int ssd_tree_attention_bf16(const uint16_t* q, int64_t ldq, int M, int heads, int kv_heads, int head_dim,
                                    const uint16_t* k_cache, const uint16_t* vt_cache, int64_t max_len,
                                    const int32_t* prefix, const int32_t* depth, const int32_t* anc, int p_min,
                                    int l_max, float scale, float* ws, int64_t ws_floats, uint16_t* out,
                                    int64_t ldo, hipStream_t stream) {
  return ssd::tree_attention(q, ldq, M, heads, kv_heads, head_dim, k_cache, vt_cache, max_len, prefix, depth, anc,
                             nullptr, p_min, l_max, scale, ws, ws_floats, out, ldo, stream);
}

// Tree attention whose rows may belong to several sequences: row t's K / V are at kv_off[t]
// elements past k_cache / vt_cache (same layout and capacity for every sequence).
int ssd::tree_attention(const uint16_t* q, int64_t ldq, int M, int heads, int kv_heads, int head_dim,
                        const uint16_t* k_cache, const uint16_t* vt_cache, int64_t max_len, const int32_t* prefix,
                        const int32_t* depth, const int32_t* anc, const int64_t* kv_off, int p_min, int l_max,
                        float scale, float* ws, int64_t ws_floats, uint16_t* out, int64_t ldo, hipStream_t stream) {
  if (!q || !k_cache || !vt_cache || !prefix || !depth || !anc || !ws || !out)
    return set_error(SSD_EINVAL, "attention: null pointer");
  if (M <= 0 || heads <= 0 || kv_heads <= 0 || heads % kv_heads)
    return set_error(SSD_EINVAL, "attention: bad M=%d heads=%d kv_heads=%d", M, heads, kv_heads);
  if (max_len % 64 || ((uintptr_t)vt_cache & 15) || ((uintptr_t)k_cache & 15) || ((uintptr_t)q & 15) || ldq % 8)
    return set_error(SSD_EINVAL, "attention: caches/q must be 16-byte aligned, max_len %% 64 == 0");
  if (((uintptr_t)out & 3) || ldo % 2 || ldo < (int64_t)heads * head_dim)
    return set_error(SSD_EINVAL, "attention: out must be 4-byte aligned with an even row stride >= heads * head_dim");
  if (l_max > max_len || p_min < 0 || l_max < 1 || p_min > l_max)
    return set_error(SSD_EINVAL, "attention: bad bounds p_min=%d l_max=%d max_len=%lld", p_min, l_max,
                     (long long)max_len);
  const int64_t n_sb_cap = (max_len + ATT_BLK * ATT_SB - 1) / (ATT_BLK * ATT_SB);
  if (ws_floats < (int64_t)M * heads * n_sb_cap * (head_dim / 2 + 2))
    return set_error(SSD_EINVAL, "attention: workspace too small");
  AttnArgs a{};
  a.Q = q; a.ldq = ldq; a.K = k_cache; a.Vt = vt_cache; a.max_len = max_len;
  a.M = M; a.heads = heads; a.kv_heads = kv_heads; a.prefix = prefix; a.depth = depth; a.anc = anc;
  a.kv_off = kv_off;
  a.p_min = p_min; a.l_max = l_max; a.scale_log2 = scale * 1.4426950408889634f; a.ws = ws;
  a.n_sb_cap = (int)n_sb_cap;
  switch (head_dim) {
    case 32: return launch_attn<32>(a, out, ldo, stream);
    case 64: return launch_attn<64>(a, out, ldo, stream);
    case 128: return launch_attn<128>(a, out, ldo, stream);
    default: return set_error(SSD_EINVAL, "attention: head_dim %d unsupported (32, 64, 128)", head_dim);
  }
}
