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
// Kernel structure (attn_partial): workgroup = (superblock, kv head, row-tile
// group), 4 waves, wave w owns block 4s+w. Blocks entirely below min(P) are
// "shared": the wave loads K and V^T for its block once into MFMA operand
// registers (16-byte HBM loads, no LDS staging) and reuses them for every
// 16-row tile (rows = token x GQA head). Other blocks are built per token from
// gathered slots. S^T = K Q^T and O^T = V^T P^T both run on
// v_mfma_f32_16x16x32_bf16; the key order inside a block is permuted so the
// score accumulators are already the P^T operand (no LDS transpose). Row
// max/sum use cross-lane shuffles of the wave64. Block partials meet in LDS and
// are folded; superblock partials go to a workspace and attn_combine folds them.
#include "common.h"

#include <math.h>

namespace ssd {

constexpr int ATT_BLK = 64;
constexpr int ATT_SB = 4;        // blocks per superblock
constexpr int ATT_MAXD = 32;     // gathered tree slots per row

struct AttnArgs {
  const bf16_t* Q;  // [M, heads*hd] (row stride ldq)
  int64_t ldq;
  const bf16_t* K;   // this layer: [kv_heads, max_len, hd]
  const bf16_t* Vt;  // this layer: [kv_heads, hd, max_len]
  int64_t max_len;
  int M, heads, kv_heads;
  const int* prefix;  // [M]
  const int* depth;   // [M]
  const int* anc;     // [M, ATT_MAXD]
  int p_min, l_max;
  float scale_log2;
  int tiles_per_group;
  float* ws;  // [kv_heads][M*rep][n_sb_cap][hd + 2]
  int n_sb_cap;
};

__device__ __forceinline__ int perm_key(int kt, int i) {
  // key offset (within a 64-key block) that sits in row i of key tile kt
  return (kt >> 1) * 32 + (i >> 2) * 8 + (kt & 1) * 4 + (i & 3);
}

template <int HD>
struct Frags {
  static constexpr int KS = HD / 32;  // k-steps over head_dim for Q K^T
  static constexpr int DT = HD / 16;  // 16-wide d tiles for P V
  uint4 k[4][KS];
  uint4 v[DT][2];
};

template <int HD>
__device__ __forceinline__ void load_shared_frags(Frags<HD>& f, const AttnArgs& a, int kvh, int key0, int lane) {
  const int i = lane & 15, g = lane >> 4;
  const bf16_t* kb = a.K + (size_t)kvh * a.max_len * HD;
#pragma unroll
  for (int kt = 0; kt < 4; ++kt) {
    const bf16_t* row = kb + (size_t)(key0 + perm_key(kt, i)) * HD + g * 8;
#pragma unroll
    for (int ks = 0; ks < Frags<HD>::KS; ++ks) f.k[kt][ks] = *(const uint4*)(row + ks * 32);
  }
  const bf16_t* vb = a.Vt + (size_t)kvh * HD * a.max_len;
#pragma unroll
  for (int dt = 0; dt < Frags<HD>::DT; ++dt) {
    const bf16_t* row = vb + (size_t)(dt * 16 + i) * a.max_len + key0 + g * 8;
    f.v[dt][0] = *(const uint4*)(row);
    f.v[dt][1] = *(const uint4*)(row + 32);
  }
}

// Logical key -> cache slot for token t (-1 = not attended; out-of-range slots are dropped).
__device__ __forceinline__ int logical_slot(int jpos, int P, int L, const int* anc_t, int64_t max_len) {
  int s = -1;
  if (jpos < P) s = jpos;
  else if (jpos < L && jpos - P < ATT_MAXD) s = anc_t[jpos - P];
  return (s >= 0 && s < max_len) ? s : -1;
}

template <int HD>
__device__ __forceinline__ void load_virtual_frags(Frags<HD>& f, const AttnArgs& a, int kvh, int key0, int P,
                                                   int L, const int* anc_t, int lane) {
  const int i = lane & 15, g = lane >> 4;
  const bf16_t* kb = a.K + (size_t)kvh * a.max_len * HD;
#pragma unroll
  for (int kt = 0; kt < 4; ++kt) {
    const int slot = logical_slot(key0 + perm_key(kt, i), P, L, anc_t, a.max_len);
    const bf16_t* row = kb + (size_t)(slot < 0 ? 0 : slot) * HD + g * 8;
#pragma unroll
    for (int ks = 0; ks < Frags<HD>::KS; ++ks)
      f.k[kt][ks] = slot >= 0 ? *(const uint4*)(row + ks * 32) : make_uint4(0, 0, 0, 0);
  }
  const bf16_t* vb = a.Vt + (size_t)kvh * HD * a.max_len;
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    int slots[8];
    bool contiguous = true;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      slots[t] = logical_slot(key0 + c * 32 + g * 8 + t, P, L, anc_t, a.max_len);
      contiguous = contiguous && slots[t] >= 0 && slots[t] == slots[0] + t;
    }
    contiguous = contiguous && (slots[0] % 8 == 0);
#pragma unroll
    for (int dt = 0; dt < Frags<HD>::DT; ++dt) {
      const bf16_t* row = vb + (size_t)(dt * 16 + i) * a.max_len;
      if (contiguous) {
        f.v[dt][c] = *(const uint4*)(row + slots[0]);
      } else {
        Pack8 p;
#pragma unroll
        for (int t = 0; t < 8; ++t) p.h[t] = slots[t] >= 0 ? row[slots[t]] : (bf16_t)0;
        f.v[dt][c] = p.u;
      }
    }
  }
}

// One 64-key block for a 16-row tile. valid_bits: bit (kt*4+e) says whether key perm_key(kt, 4g+e)
// is attended (same for every row of the pass). Outputs per lane (row j = lane%16): m (log2 units,
// -inf if nothing attended), l, and O[row j][dt*16 + 4g + e] in o[dt][e].
template <int HD>
__device__ __forceinline__ void block_attend(const Frags<HD>& f, const uint4 (&qf)[HD / 32], uint32_t valid_bits,
                                             float scale_log2, float& m_out, float& l_out,
                                             f32x4_t (&o)[HD / 16]) {
  constexpr int KS = HD / 32, DT = HD / 16;
  f32x4_t s[4];
#pragma unroll
  for (int kt = 0; kt < 4; ++kt) {
    s[kt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) s[kt] = mfma16x16x32(as_bf16x8(f.k[kt][ks]), as_bf16x8(qf[ks]), s[kt]);
  }
  float sv[16];
  float mx = -INFINITY;
#pragma unroll
  for (int kt = 0; kt < 4; ++kt)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float v = ((valid_bits >> (kt * 4 + e)) & 1u) ? s[kt][e] * scale_log2 : -INFINITY;
      sv[kt * 4 + e] = v;
      mx = fmaxf(mx, v);
    }
  mx = fmaxf(mx, __shfl_xor(mx, 16));
  mx = fmaxf(mx, __shfl_xor(mx, 32));
  m_out = mx;
  // A row with nothing attended gets p = 0 everywhere (m stays -inf and marks it absent).
  // No early exit: every lane must stay active for the MFMAs below.
  const float msafe = mx == -INFINITY ? 0.f : mx;
  float l = 0.f;
  Pack8 pb[2];
#pragma unroll
  for (int kt = 0; kt < 4; ++kt)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float p = exp2f(sv[kt * 4 + e] - msafe);
      l += p;
      pb[kt >> 1].h[(kt & 1) * 4 + e] = f2bf(p);
    }
  l += __shfl_xor(l, 16);
  l += __shfl_xor(l, 32);
  l_out = l;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    f32x4_t acc = f32x4_t{0.f, 0.f, 0.f, 0.f};
    acc = mfma16x16x32(as_bf16x8(f.v[dt][0]), pb[0].v, acc);
    acc = mfma16x16x32(as_bf16x8(f.v[dt][1]), pb[1].v, acc);
    o[dt] = acc;
  }
}

template <int HD>
struct AttnLds {
  float o[ATT_SB][16][HD + 4];
  float m[ATT_SB][16];
  float l[ATT_SB][16];
};

template <int HD>
__global__ __launch_bounds__(256) void attn_partial_kernel(AttnArgs a) {
  constexpr int KS = HD / 32, DT = HD / 16;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int sb = blockIdx.x, kvh = blockIdx.y, grp = blockIdx.z;
  const int rep = a.heads / a.kv_heads;
  const int n_rows = a.M * rep;
  const int n_tiles = (n_rows + 15) / 16;
  const int t_lo = grp * a.tiles_per_group;
  const int t_hi = min(n_tiles, t_lo + a.tiles_per_group);
  const int key0 = (sb * ATT_SB + w) * ATT_BLK;
  const bool active = key0 < a.l_max;
  const bool shared = key0 + ATT_BLK <= a.p_min;
  const int j = lane & 15, g = lane >> 4;
  // Blocks of this superblock that must be built per token (they reach past min(P)).
  int tail_blocks[ATT_SB];
  int n_tail = 0;
#pragma unroll
  for (int ww = 0; ww < ATT_SB; ++ww) {
    const int k0 = (sb * ATT_SB + ww) * ATT_BLK;
    if (k0 < a.l_max && k0 + ATT_BLK > a.p_min) tail_blocks[n_tail++] = ww;
  }

  __shared__ AttnLds<HD> lds;
  __shared__ int s_anc[16][ATT_MAXD];  // ancestor slots of the tile's tokens
  __shared__ int s_P[16], s_L[16];
  Frags<HD> f;
  if (active && shared) load_shared_frags<HD>(f, a, kvh, key0, lane);

  for (int t = t_lo; t < t_hi; ++t) {
    const int tok_first = (t * 16) / rep;
    const int tok_last = min(a.M - 1, (t * 16 + 15) / rep);
    const int ntok = tok_last - tok_first + 1;
    if (n_tail) {
      for (int idx = threadIdx.x; idx < ntok * ATT_MAXD; idx += 256)
        s_anc[idx / ATT_MAXD][idx % ATT_MAXD] = a.anc[(size_t)(tok_first + idx / ATT_MAXD) * ATT_MAXD + idx % ATT_MAXD];
      if (threadIdx.x < ntok) {
        const int P = a.prefix[tok_first + threadIdx.x];
        s_P[threadIdx.x] = P;
        s_L[threadIdx.x] = P + min(a.depth[tok_first + threadIdx.x], ATT_MAXD);
      }
      __syncthreads();
    }
    const int r = t * 16 + j;
    const bool rv = r < n_rows;
    const int tok = rv ? r / rep : 0;
    const int hq = kvh * rep + (rv ? r % rep : 0);
    uint4 qf[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      qf[ks] = rv ? *(const uint4*)(a.Q + (size_t)tok * a.ldq + (size_t)hq * HD + ks * 32 + g * 8)
                  : make_uint4(0, 0, 0, 0);

    if (!active) {
      if (g == 0) { lds.m[w][j] = -INFINITY; lds.l[w][j] = 0.f; }
    } else if (shared) {
      float m, l;
      f32x4_t o[DT];
      block_attend<HD>(f, qf, 0xffffu, a.scale_log2, m, l, o);
      if (g == 0) { lds.m[w][j] = m; lds.l[w][j] = l; }
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int e = 0; e < 4; ++e) lds.o[w][j][dt * 16 + 4 * g + e] = o[dt][e];
    }
    // Per-token virtual blocks, spread over the four waves.
    const int units = n_tail * ntok;
    for (int u = w; u < units; u += ATT_SB) {
      const int wb = tail_blocks[u / ntok];
      const int tl = u % ntok, tk = tok_first + tl;
      const int kb0 = (sb * ATT_SB + wb) * ATT_BLK;
      const int P = s_P[tl], L = s_L[tl];
      const int* anc_t = s_anc[tl];
      Frags<HD> fv;
      load_virtual_frags<HD>(fv, a, kvh, kb0, P, L, anc_t, lane);
      uint32_t bits = 0;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (logical_slot(kb0 + perm_key(kt, 4 * g + e), P, L, anc_t, a.max_len) >= 0) bits |= 1u << (kt * 4 + e);
      float m, l;
      f32x4_t o[DT];
      block_attend<HD>(fv, qf, bits, a.scale_log2, m, l, o);
      if (rv && tok == tk) {
        if (g == 0) { lds.m[wb][j] = m; lds.l[wb][j] = l; }
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int e = 0; e < 4; ++e) lds.o[wb][j][dt * 16 + 4 * g + e] = o[dt][e];
      }
    }
    __syncthreads();

    // Fold the 4 block partials of each row left to right -> superblock partial.
    {
      const int rr = threadIdx.x >> 4;       // tile row
      const int dc = threadIdx.x & 15;       // d chunk
      constexpr int DPT = HD / 16;           // d per thread
      const int R = t * 16 + rr;
      if (R < n_rows) {
        float mS = -INFINITY, lS = 0.f, oS[DPT];
        bool first = true;
#pragma unroll
        for (int ww = 0; ww < ATT_SB; ++ww) {
          const float mb = lds.m[ww][rr];
          if (mb == -INFINITY) continue;
          const float lb = lds.l[ww][rr];
          if (first) {
            mS = mb; lS = lb;
#pragma unroll
            for (int d = 0; d < DPT; ++d) oS[d] = lds.o[ww][rr][dc * DPT + d];
            first = false;
          } else {
            const float mN = fmaxf(mS, mb);
            const float a1 = exp2f(mS - mN), a2 = exp2f(mb - mN);
            lS = lS * a1 + lb * a2;
#pragma unroll
            for (int d = 0; d < DPT; ++d) oS[d] = oS[d] * a1 + lds.o[ww][rr][dc * DPT + d] * a2;
            mS = mN;
          }
        }
        float* dst = a.ws + (((size_t)kvh * n_rows + R) * a.n_sb_cap + sb) * (HD + 2);
        if (!first) {
#pragma unroll
          for (int d = 0; d < DPT; ++d) dst[dc * DPT + d] = oS[d];
        }
        if (dc == 0) { dst[HD] = mS; dst[HD + 1] = lS; }
      }
    }
    __syncthreads();
  }
}

// Cross-superblock combine, one wave per (token, q head). Canonical arithmetic for a row of
// length L with superblocks s = 0..n-1: M = max_s m_s; w_s = 2^(m_s - M); l = sum_s l_s w_s and
// O = sum_s O_s w_s, both summed in increasing s; out = O / l. All loads are independent of
// the running sums, so they are issued ahead of the arithmetic.
template <int HD>
__global__ __launch_bounds__(256) void attn_combine_kernel(const float* __restrict__ ws, int n_sb_cap, int M,
                                                           int heads, int kv_heads, const int* __restrict__ prefix,
                                                           const int* __restrict__ depth, bf16_t* __restrict__ out,
                                                           int64_t ldo, int n_sb_run) {
  constexpr int PER = (HD + 63) / 64;
  const int wid = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (wid >= M * heads) return;
  const int tok = wid / heads, hq = wid % heads;
  const int rep = heads / kv_heads, kvh = hq / rep;
  const int R = tok * rep + hq % rep;
  const int L = prefix[tok] + min(depth[tok], ATT_MAXD);
  const int nsb = min(n_sb_run, (L + ATT_BLK * ATT_SB - 1) / (ATT_BLK * ATT_SB));
  const float* base = ws + ((size_t)kvh * M * rep + R) * n_sb_cap * (HD + 2);
  // pass 1: row max over superblocks (lanes own superblocks)
  float mx = -INFINITY;
  for (int s0 = 0; s0 < nsb; s0 += 64) {
    const int s = s0 + lane;
    if (s < nsb) mx = fmaxf(mx, base[(size_t)s * (HD + 2) + HD]);
  }
  for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
  float l = 0.f, o[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) o[i] = 0.f;
  for (int s0 = 0; s0 < nsb; s0 += 64) {
    const int s = s0 + lane;
    float wgt = 0.f, ls = 0.f;
    if (s < nsb) {
      const float ms = base[(size_t)s * (HD + 2) + HD];
      ls = base[(size_t)s * (HD + 2) + HD + 1];
      wgt = ms == -INFINITY ? 0.f : exp2f(ms - mx);
    }
    const int cnt = min(64, nsb - s0);
    for (int q = 0; q < cnt; ++q) {
      const float wq = __shfl(wgt, q);
      const float lq = __shfl(ls, q);
      l += lq * wq;
      const float* p = base + (size_t)(s0 + q) * (HD + 2);
#pragma unroll
      for (int i = 0; i < PER; ++i)
        if (lane + 64 * i < HD && wq != 0.f) o[i] += p[lane + 64 * i] * wq;
    }
  }
  bf16_t* dst = out + (size_t)tok * ldo + (size_t)hq * HD;
#pragma unroll
  for (int i = 0; i < PER; ++i)
    if (lane + 64 * i < HD) dst[lane + 64 * i] = f2bf(l > 0.f ? o[i] / l : 0.f);
}

template <int HD>
static int launch_attn(AttnArgs a, bf16_t* out, int64_t ldo, hipStream_t s) {
  const int rep = a.heads / a.kv_heads;
  const int n_tiles = (a.M * rep + 15) / 16;
  const int n_sb = (a.l_max + ATT_BLK * ATT_SB - 1) / (ATT_BLK * ATT_SB);
  if (n_sb > a.n_sb_cap) return set_error(SSD_ERANGE, "attention: length %d needs %d superblocks > workspace %d",
                                          a.l_max, n_sb, a.n_sb_cap);
  // Tile groups: enough workgroups to cover the chip, never changing the arithmetic.
  const int units = n_sb * a.kv_heads;
  int groups = (512 + units - 1) / units;
  groups = groups < 1 ? 1 : (groups > n_tiles ? n_tiles : groups);
  a.tiles_per_group = (n_tiles + groups - 1) / groups;
  groups = (n_tiles + a.tiles_per_group - 1) / a.tiles_per_group;
  hipLaunchKernelGGL((attn_partial_kernel<HD>), dim3(n_sb, a.kv_heads, groups), dim3(256), 0, s, a);
  int rc = check_launch("attn_partial");
  if (rc) return rc;
  const int waves = a.M * a.heads;
  hipLaunchKernelGGL((attn_combine_kernel<HD>), dim3((waves + 3) / 4), dim3(256), 0, s, a.ws, a.n_sb_cap, a.M,
                     a.heads, a.kv_heads, a.prefix, a.depth, out, ldo, n_sb);
  return check_launch("attn_combine");
}

}  // namespace ssd

using namespace ssd;

SSD_API int ssd_attn_workspace_floats(int M, int heads, int head_dim, int64_t max_len) {
  const int64_t n_sb = (max_len + ATT_BLK * ATT_SB - 1) / (ATT_BLK * ATT_SB);
  return (int)((int64_t)M * heads * n_sb * (head_dim + 2));
}

SSD_API int ssd_attn_max_depth(void) { return ATT_MAXD; }

// out[t, h*hd:(h+1)*hd] = softmax over row t's logical keys (see header) of q.k/sqrt(hd), times v.
// q: [M, heads*hd] bf16 (post-RoPE); k_cache: [kv_heads, max_len, hd]; vt_cache: [kv_heads, hd, max_len].
// prefix/depth: [M] int32; anc: [M, 32] int32 slots; p_min <= min(prefix); l_max >= max(prefix+depth).
// ws: fp32 workspace of ssd_attn_workspace_floats(M, heads, hd, max_len) floats.
SSD_API int ssd_tree_attention_bf16(const uint16_t* q, int64_t ldq, int M, int heads, int kv_heads, int head_dim,
                                    const uint16_t* k_cache, const uint16_t* vt_cache, int64_t max_len,
                                    const int32_t* prefix, const int32_t* depth, const int32_t* anc, int p_min,
                                    int l_max, float scale, float* ws, int64_t ws_floats, uint16_t* out,
                                    int64_t ldo, hipStream_t stream) {
  if (!q || !k_cache || !vt_cache || !prefix || !depth || !anc || !ws || !out)
    return set_error(SSD_EINVAL, "attention: null pointer");
  if (M <= 0 || heads <= 0 || kv_heads <= 0 || heads % kv_heads)
    return set_error(SSD_EINVAL, "attention: bad M=%d heads=%d kv_heads=%d", M, heads, kv_heads);
  if (max_len % 8 || ((uintptr_t)vt_cache & 15) || ((uintptr_t)k_cache & 15) || ((uintptr_t)q & 15) || ldq % 8)
    return set_error(SSD_EINVAL, "attention: caches/q must be 16-byte aligned, max_len %% 8 == 0");
  if (l_max > max_len || p_min < 0 || l_max < 1 || p_min > l_max)
    return set_error(SSD_EINVAL, "attention: bad bounds p_min=%d l_max=%d max_len=%lld", p_min, l_max,
                     (long long)max_len);
  const int64_t n_sb_cap = (max_len + ATT_BLK * ATT_SB - 1) / (ATT_BLK * ATT_SB);
  if (ws_floats < (int64_t)M * heads * n_sb_cap * (head_dim + 2))
    return set_error(SSD_EINVAL, "attention: workspace too small");
  AttnArgs a{};
  a.Q = q; a.ldq = ldq; a.K = k_cache; a.Vt = vt_cache; a.max_len = max_len;
  a.M = M; a.heads = heads; a.kv_heads = kv_heads; a.prefix = prefix; a.depth = depth; a.anc = anc;
  a.p_min = p_min; a.l_max = l_max; a.scale_log2 = scale * 1.4426950408889634f; a.ws = ws;
  a.n_sb_cap = (int)n_sb_cap;
  switch (head_dim) {
    case 32: return launch_attn<32>(a, out, ldo, stream);
    case 64: return launch_attn<64>(a, out, ldo, stream);
    case 128: return launch_attn<128>(a, out, ldo, stream);
    default: return set_error(SSD_EINVAL, "attention: head_dim %d unsupported (32, 64, 128)", head_dim);
  }
}
