// Sampling path: temperature + nucleus warp, Gumbel top-k draft proposals,
// speculative-sampling acceptance over the verify tree, and categorical draws.
//
// Reference semantics (restated, not transcribed):
// * warp_probs  ssd/engine/tree_drafter.py:34-45: p = softmax(logits / T); with
//   top_p < 1 an entry survives when the mass of the entries sorted before it is
//   <= top_p; survivors are renormalised.
// * _propose    ssd/engine/tree_drafter.py:124-145 (sampling branch): q is the warped
//   draft distribution over the full vocabulary (zero outside a draft-vocab subset);
//   children are min(k, |support|) draws without replacement, in draw order, via the
//   Gumbel top-k trick; their log-probs are log q.
// * sample_verify ssd/engine/verify.py:60-95: walk root -> children in rank order;
//   accept child x with probability min(1, p(x) / q(x)); on rejection
//   p <- (p - q)+ / sum (when the sum is positive), q(x) <- 0, q <- q / sum(q), stop when
//   q has no mass left; the bonus token is drawn from the final p.
// * torch.multinomial (ssd/engine/speculative.py:81-84, verify.py:94): one categorical
//   draw, here as argmax_y p(y) / E(y) with E(y) ~ Exp(1) (the Gumbel-max trick).
//
// Randomness: Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as
// easy as 1, 2, 3", SC 2011). Key = 64-bit seed; counter = (element or step index,
// row | level << 16, round counter low word, round counter high bits << 8 | purpose tag),
// so every draw of a generation has its own counter and the result does not depend on
// launch shapes or on how many rows share a launch.
//
// Tie rules (where the reference leaves the order to torch's sort): equal probabilities
// rank lower column first in the nucleus cut; equal Gumbel keys rank lower token first.
//
// Each row is one 1024-thread workgroup making several passes over its row (fp32,
// L2-resident after the first). Thread t always owns elements 4t + 4096 j, so a value a
// thread stores in one pass is read back by the same thread in the next.
#include "common.h"

#include <math.h>

namespace ssd {

constexpr int SMP_THREADS = 1024;
constexpr int SMP_MAXK = 16;      // children per node considered by the acceptance walk
constexpr int SMP_MAXDEPTH = 32;  // tree depth (matches the tree kernels)
constexpr int SMP_BINS = 1024;

enum SmpTag { TAG_PROPOSE = 1, TAG_ACCEPT = 2, TAG_BONUS = 3, TAG_DRAW = 4 };

struct Rng {
  uint32_t k0, k1;        // key: seed
  uint32_t c2, c3_base;   // counter words 2 and 3 (round counter; tag is or-ed into c3)
};

static Rng make_rng(uint64_t seed, uint64_t ctr) {
  return Rng{(uint32_t)seed, (uint32_t)(seed >> 32), (uint32_t)ctr, (uint32_t)((ctr >> 32) << 8)};
}

struct U4 {
  uint32_t x, y, z, w;
};

// Philox4x32 with 10 rounds: multipliers 0xD2511F53 / 0xCD9E8D57, Weyl key increments
// 0x9E3779B9 / 0xBB67AE85 (the published constants of the generator).
__device__ __forceinline__ U4 philox(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3, uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint32_t lo0 = 0xD2511F53u * c0, hi0 = __umulhi(0xD2511F53u, c0);
    const uint32_t lo1 = 0xCD9E8D57u * c2, hi1 = __umulhi(0xCD9E8D57u, c2);
    c0 = hi1 ^ c1 ^ k0;
    c1 = lo1;
    c2 = hi0 ^ c3 ^ k1;
    c3 = lo0;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  return U4{c0, c1, c2, c3};
}

__device__ __forceinline__ U4 rng_block(const Rng& g, uint32_t c0, uint32_t c1, int tag) {
  return philox(c0, c1, g.c2, g.c3_base | (uint32_t)tag, g.k0, g.k1);
}

// Standard exponential -log(U) from 32 random bits, U = (b + 1/2) / 2^32 in (0, 1). The lower
// half of U is taken directly and the upper half through 1 - U, so both tails keep 24 bits.
__device__ __forceinline__ float exp1_from_bits(uint32_t b) {
  if (b < 0x80000000u) return -logf(((float)b + 0.5f) * 0x1p-32f);
  return -log1pf(-(((float)(~b) + 0.5f) * 0x1p-32f));
}

__device__ __forceinline__ double uniform_from_bits(uint32_t b) { return ((double)b + 0.5) * 0x1p-32; }

__device__ __forceinline__ uint32_t u4_get(const U4& r, int e) {
  return e == 0 ? r.x : e == 1 ? r.y : e == 2 ? r.z : r.w;
}

// ----------------------------------------------------------- block reductions (1024 threads)
__device__ __forceinline__ float block_max(float v, float* sh) {
#pragma unroll
  for (int o = 32; o; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = sh[0];
  for (int i = 1; i < 16; ++i) r = fmaxf(r, sh[i]);
  __syncthreads();
  return r;
}

// Fixed-order sums: butterfly inside each wave, then the 16 wave sums in order.
template <typename T>
__device__ __forceinline__ T block_sum(T v, T* sh) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) v += __shfl_xor(v, o);
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  T r = sh[0];
  for (int i = 1; i < 16; ++i) r += sh[i];
  __syncthreads();
  return r;
}

struct KeyIdx {
  float key;
  int idx;
};

__device__ __forceinline__ bool better(float ka, int ia, float kb, int ib) {
  return ka > kb || (ka == kb && ia < ib);
}

// Largest key, lowest index among equal keys. Every thread gets the result.
__device__ __forceinline__ KeyIdx block_argmax(float key, int idx, KeyIdx* sh) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const float k2 = __shfl_xor(key, o);
    const int i2 = __shfl_xor(idx, o);
    if (better(k2, i2, key, idx)) {
      key = k2;
      idx = i2;
    }
  }
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = KeyIdx{key, idx};
  __syncthreads();
  KeyIdx r = sh[0];
  for (int i = 1; i < 16; ++i)
    if (better(sh[i].key, sh[i].idx, r.key, r.idx)) r = sh[i];
  __syncthreads();
  return r;
}

// Inclusive prefix sum over the 1024 threads (thread order).
__device__ __forceinline__ uint32_t block_scan(uint32_t v, uint32_t* sh) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t n = __shfl_up(v, o);
    if (lane >= o) v += n;
  }
  if (lane == 63) sh[w] = v;
  __syncthreads();
  uint32_t add = 0;
  for (int i = 0; i < w; ++i) add += sh[i];
  __syncthreads();
  return v + add;
}

// ------------------------------------------------------------------------ warp
struct WarpArgs {
  const bf16_t* logits;
  int64_t ld;
  int rows, n;           // logit rows and columns
  const int* vocab;      // column -> token (draft-vocab subset), or null (column = token)
  const int* inv;        // token -> column or -1 (with vocab), length V
  int V;                 // output row length (full vocabulary)
  float temp, top_p;
  const int* meta;       // tree meta: rows are the frontier proposing `level`; null: plain rows
  int level;
  float* out;
  int64_t ldo;
};

// Frontier size and first output row of a proposal step (tree meta layout: [0] nodes,
// [1 + d] start of level d, [1 + SMP_MAXDEPTH + d] its size). Level 0 proposes the root's
// children (q row 0); level d > 0 proposes children of level d - 1, whose node i keeps its
// q in row 1 + i.
__device__ __forceinline__ void frontier_rows(const int* meta, int level, int rows, int& F, int& base) {
  if (!meta) {
    F = rows;
    base = 0;
  } else if (level == 0) {
    F = 1;
    base = 0;
  } else {
    F = min(rows, meta[1 + SMP_MAXDEPTH + level - 1]);
    base = 1 + meta[1 + level - 1];
  }
}

struct Cut {
  int bin;
  uint32_t above;  // fixed-point mass ranked before the bin
};

// The bin holding the first entry whose preceding mass exceeds T, scanning bins from the
// largest value down; `base` is the mass ranked before every bin of this histogram.
// Returns bin -1 when the whole histogram fits under T.
__device__ __forceinline__ Cut find_cut(const uint32_t* hist, uint32_t base, uint32_t T, uint32_t* scan_sh,
                                        Cut* cut_sh) {
  const int b = SMP_BINS - 1 - (int)threadIdx.x;
  const uint32_t v = hist[b];
  const uint32_t incl = block_scan(v, scan_sh);
  if (threadIdx.x == 0) *cut_sh = Cut{-1, 0};
  __syncthreads();
  const uint32_t above = base + incl - v;
  if (v > 0 && above <= T && T < base + incl) *cut_sh = Cut{b, above};
  __syncthreads();
  const Cut c = *cut_sh;
  __syncthreads();
  return c;
}

__device__ __forceinline__ uint32_t mass_fixed(float p) { return __float2uint_rn(p * 0x1p31f); }

__global__ __launch_bounds__(SMP_THREADS) void warp_kernel(WarpArgs a) {
  __shared__ uint32_t hist_m[SMP_BINS];
  __shared__ uint32_t hist_c[SMP_BINS];
  __shared__ uint32_t scan_sh[16];
  __shared__ float red_f[16];
  __shared__ Cut cut_sh;
  __shared__ int idx_cut_sh;
  int F, base;
  frontier_rows(a.meta, a.level, a.rows, F, base);
  const int f = blockIdx.x;
  if (f >= F) return;
  const bf16_t* lg = a.logits + (size_t)f * a.ld;
  float* out = a.out + (size_t)(base + f) * a.ldo;
  const int t = threadIdx.x;
  const int n = a.n;
  const float temp = a.temp;
  if (t == 0) idx_cut_sh = 0x7fffffff;

  // Pass 1: max and sum of exp (online per thread, fixed-order combine).
  float m = -INFINITY, s = 0.f;
  for (int i = t * 4; i < n; i += 4 * SMP_THREADS) {
    const uint2 raw = *(const uint2*)(lg + i);
    const bf16_t h[4] = {(bf16_t)(raw.x & 0xffff), (bf16_t)(raw.x >> 16), (bf16_t)(raw.y & 0xffff),
                         (bf16_t)(raw.y >> 16)};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (i + e >= n) break;
      const float x = bf2f(h[e]) / temp;
      if (x > m) {
        s = s * expf(m - x) + 1.f;
        m = x;
      } else {
        s += expf(x - m);
      }
    }
  }
  const float M = block_max(m, red_f);
  const float S = block_sum<float>(m == -INFINITY ? 0.f : s * expf(m - M), red_f);
  const bool nucleus = a.top_p < 1.f;
  const uint32_t T = nucleus ? (uint32_t)fmin(fmax((double)a.top_p, 0.0) * 2147483648.0, 4294967295.0) : 0u;

  if (nucleus) {
    hist_m[t] = 0;
    __syncthreads();
  }
  // Pass 2: probabilities into the output row; mass histogram of the top 12 value bits.
  for (int i = t * 4; i < n; i += 4 * SMP_THREADS) {
    const uint2 raw = *(const uint2*)(lg + i);
    const bf16_t h[4] = {(bf16_t)(raw.x & 0xffff), (bf16_t)(raw.x >> 16), (bf16_t)(raw.y & 0xffff),
                         (bf16_t)(raw.y >> 16)};
    float p[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) p[e] = expf(bf2f(h[e]) / temp - M) / S;
    if (!a.vocab && i + 3 < n) {
      *(float4*)(out + i) = make_float4(p[0], p[1], p[2], p[3]);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (i + e < n) out[a.vocab ? a.vocab[i + e] : i + e] = p[e];
    }
    if (nucleus) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (i + e < n) atomicAdd(&hist_m[min(__float_as_uint(p[e]) >> 20, 1023u)], mass_fixed(p[e]));
    }
  }
  if (a.vocab) {  // tokens outside the subset have probability 0
    for (int y = t; y < a.V; y += SMP_THREADS)
      if (a.inv[y] < 0) out[y] = 0.f;
  }
  if (!nucleus) return;
  __syncthreads();

  auto load_p = [&](int i, float p[4]) {
    if (!a.vocab && i + 3 < n) {
      const float4 v = *(const float4*)(out + i);
      p[0] = v.x;
      p[1] = v.y;
      p[2] = v.z;
      p[3] = v.w;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) p[e] = i + e < n ? out[a.vocab ? a.vocab[i + e] : i + e] : 0.f;
    }
  };

  // Radix search for the cut: 12 + 10 + 10 value bits (probabilities are <= 1, so the top
  // 12 bits of a float are < 1024).
  const Cut cA = find_cut(hist_m, 0u, T, scan_sh, &cut_sh);
  uint32_t vbits = 0, kept_mass = 0;
  int idx_cut = 0x7fffffff;
  if (cA.bin < 0) {  // everything fits under top_p: keep all
    vbits = 0;
    kept_mass = 0xffffffffu;
  } else {
    hist_m[t] = 0;
    __syncthreads();
    for (int i = t * 4; i < n; i += 4 * SMP_THREADS) {
      float p[4];
      load_p(i, p);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t b = __float_as_uint(p[e]);
        if (i + e < n && (int)(b >> 20) == cA.bin) atomicAdd(&hist_m[(b >> 10) & 1023], mass_fixed(p[e]));
      }
    }
    __syncthreads();
    const Cut cB = find_cut(hist_m, cA.above, T, scan_sh, &cut_sh);
    const uint32_t hiB = ((uint32_t)cA.bin << 10) | (uint32_t)max(cB.bin, 0);
    hist_m[t] = 0;
    hist_c[t] = 0;
    __syncthreads();
    for (int i = t * 4; i < n; i += 4 * SMP_THREADS) {
      float p[4];
      load_p(i, p);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t b = __float_as_uint(p[e]);
        if (i + e < n && (b >> 10) == hiB) {
          atomicAdd(&hist_m[b & 1023], mass_fixed(p[e]));
          atomicAdd(&hist_c[b & 1023], 1u);
        }
      }
    }
    __syncthreads();
    const Cut cC = find_cut(hist_m, cB.above, T, scan_sh, &cut_sh);
    // cB / cC cannot miss when cA hit (the bin's mass straddles T); guard anyway.
    const int binC = max(cC.bin, 0);
    vbits = (hiB << 10) | (uint32_t)binC;
    const uint32_t n_t = hist_c[binC];
    const uint32_t w_v = n_t ? hist_m[binC] / n_t : 0u;
    const uint32_t C3 = cC.bin < 0 ? cB.above : cC.above;
    uint32_t c = n_t;
    if (w_v > 0 && T >= C3) c = min(n_t, (T - C3) / w_v + 1u);
    kept_mass = C3 + c * w_v;
    if (c < n_t) {
      // Equal probabilities straddle the cut: keep the c lowest columns among them.
      int sh = 0;
      while (((n - 1) >> sh) >= SMP_BINS) ++sh;
      __syncthreads();
      hist_c[t] = 0;
      __syncthreads();
      for (int i = t * 4; i < n; i += 4 * SMP_THREADS) {
        float p[4];
        load_p(i, p);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (i + e < n && __float_as_uint(p[e]) == vbits) atomicAdd(&hist_c[(i + e) >> sh], 1u);
      }
      __syncthreads();
      const uint32_t cnt = hist_c[t];
      const uint32_t incl = block_scan(cnt, scan_sh);
      if (cnt > 0 && incl - cnt < c && c <= incl) {
        cut_sh = Cut{t, c - (incl - cnt)};  // bin t holds the c-th tie, the `above`-th inside it
      }
      __syncthreads();
      const Cut cd = cut_sh;
      __syncthreads();
      // One element per thread inside the bin (bins span at most 2^sh <= 1024 columns).
      const int col = (cd.bin << sh) + t;
      int tie = 0;
      if (t < (1 << sh) && col < n) {
        const float pv = a.vocab ? out[a.vocab[col]] : out[col];
        tie = __float_as_uint(pv) == vbits;
      }
      const uint32_t rk = block_scan((uint32_t)tie, scan_sh);
      if (tie && rk == cd.above) idx_cut_sh = col;
      __syncthreads();
      idx_cut = idx_cut_sh;
    }
  }
  const float inv_sum = kept_mass == 0xffffffffu ? -1.f : (float)(1.0 / ((double)kept_mass * 0x1p-31));
  float keep_sum_f = 0.f;
  if (kept_mass == 0xffffffffu) {  // keep all: renormalise by the plain sum
    for (int i = t * 4; i < n; i += 4 * SMP_THREADS) {
      float p[4];
      load_p(i, p);
#pragma unroll
      for (int e = 0; e < 4; ++e) keep_sum_f += i + e < n ? p[e] : 0.f;
    }
    keep_sum_f = block_sum<float>(keep_sum_f, red_f);
  }
  // Final pass: survivors renormalised, the rest zeroed.
  for (int i = t * 4; i < n; i += 4 * SMP_THREADS) {
    float p[4];
    load_p(i, p);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t b = __float_as_uint(p[e]);
      const bool keep = b > vbits || (b == vbits && i + e <= idx_cut);
      p[e] = keep ? (inv_sum < 0.f ? p[e] / keep_sum_f : p[e] * inv_sum) : 0.f;
    }
    if (!a.vocab && i + 3 < n) {
      *(float4*)(out + i) = make_float4(p[0], p[1], p[2], p[3]);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (i + e < n) out[a.vocab ? a.vocab[i + e] : i + e] = p[e];
    }
  }
}

// ------------------------------------------------------------------- Gumbel top-k
struct TopkArgs {
  const float* q;
  int64_t ldq;
  int rows, V, k;
  const int* meta;
  int level;
  Rng rng;
  int* out_tok;   // [rows][k], -1 past min(k, support)
  float* out_lp;  // log q of each drawn token
};

// Draws min(k, |support|) tokens without replacement from each row of q: the k largest keys
// q(y) / E(y), E(y) ~ Exp(1) i.i.d. (equivalently log q(y) + Gumbel), in decreasing key
// order, which is the order of the sequential draws.
template <int K>
__global__ __launch_bounds__(SMP_THREADS) void gumbel_topk_kernel(TopkArgs a) {
  __shared__ KeyIdx red[16];
  __shared__ int red_i[16];
  int F, base;
  frontier_rows(a.meta, a.level, a.rows, F, base);
  const int f = blockIdx.x;
  if (f >= F) return;
  const float* q = a.q + (size_t)(base + f) * a.ldq;
  const int t = threadIdx.x;
  float kk[K];
  int ki[K];
#pragma unroll
  for (int j = 0; j < K; ++j) {
    kk[j] = -1.f;
    ki[j] = 0x7fffffff;
  }
  int supp = 0;
  const uint32_t c1 = (uint32_t)f | ((uint32_t)a.level << 16);
  for (int i = t * 4; i < a.V; i += 4 * SMP_THREADS) {
    float p[4];
    if (i + 3 < a.V) {
      const float4 v = *(const float4*)(q + i);
      p[0] = v.x;
      p[1] = v.y;
      p[2] = v.z;
      p[3] = v.w;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) p[e] = i + e < a.V ? q[i + e] : 0.f;
    }
    const U4 r = rng_block(a.rng, (uint32_t)(i >> 2), c1, TAG_PROPOSE);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (!(p[e] > 0.f)) continue;
      ++supp;
      const float key = p[e] / exp1_from_bits(u4_get(r, e));
      if (key > kk[K - 1]) {  // insert, keeping earlier (lower) tokens first among equal keys
        float ck = key;
        int ci = i + e;
#pragma unroll
        for (int j = 0; j < K; ++j) {
          if (ck > kk[j]) {
            const float tk = kk[j];
            const int ti = ki[j];
            kk[j] = ck;
            ki[j] = ci;
            ck = tk;
            ci = ti;
          }
        }
      }
    }
  }
  const int support = block_sum<int>(supp, red_i);
  const int take = min(a.k, support);
  for (int r = 0; r < a.k; ++r) {
    int tok = -1;
    if (r < take) {
      const KeyIdx w = block_argmax(kk[0], ki[0], red);
      tok = w.idx;
      if (ki[0] == w.idx) {  // owner pops its head
#pragma unroll
        for (int j = 0; j + 1 < K; ++j) {
          kk[j] = kk[j + 1];
          ki[j] = ki[j + 1];
        }
        kk[K - 1] = -1.f;
        ki[K - 1] = 0x7fffffff;
      }
    }
    if (t == 0) {
      a.out_tok[f * a.k + r] = tok;
      a.out_lp[f * a.k + r] = tok >= 0 ? logf(q[tok]) : 0.f;
    }
  }
}

// ------------------------------------------------------------- categorical draws
// One draw per row from p (any nonnegative row; normalisation is irrelevant to the argmax):
// argmax_y p(y) / E(y), E from the DRAW stream with counter (y / 4, row).
__global__ __launch_bounds__(SMP_THREADS) void sample_rows_kernel(const float* __restrict__ P, int64_t ldp, int V,
                                                                  Rng rng, int* __restrict__ out_tok) {
  __shared__ KeyIdx red[16];
  const int row = blockIdx.x;
  const float* p = P + (size_t)row * ldp;
  float best = -1.f;
  int bi = 0x7fffffff;
  for (int i = threadIdx.x * 4; i < V; i += 4 * SMP_THREADS) {
    const U4 r = rng_block(rng, (uint32_t)(i >> 2), (uint32_t)row, TAG_DRAW);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (i + e >= V) break;
      const float pv = p[i + e];
      if (!(pv > 0.f)) continue;
      const float key = pv / exp1_from_bits(u4_get(r, e));
      if (key > best) {
        best = key;
        bi = i + e;
      }
    }
  }
  const KeyIdx w = block_argmax(best, bi, red);
  if (threadIdx.x == 0) out_tok[row] = w.idx == 0x7fffffff ? 0 : w.idx;
}

// ----------------------------------------------------------- speculative acceptance
// Per verify row (node `cur`, row cur + 1): the states the walk can reach at that node.
// State j = after the first j children (rank order, q0(x) > 0) were rejected:
//   q_0 = q0, q_j(y) = q0(y) [y not rejected] / zq[j] (zq[j] = sum q0 - sum of rejected q0),
//   p_0 = p,  p_j = (p_{j-1} - q_{j-1})+ / zr[j] when zr[j] = sum (p_{j-1} - q_{j-1})+ > 0,
//             p_j = p_{j-1} otherwise,
// and bonus[j] = the categorical draw from p_j (one shared Exp(1) vector per round: only one
// state's draw is ever used, and which one is decided by the acceptance uniforms alone).
struct SampleState {
  int n;     // children considered
  int supp;  // |support of q0|
  int kid[SMP_MAXK];
  int bonus[SMP_MAXK + 1];
  float zr[SMP_MAXK + 1];
  float zq[SMP_MAXK + 1];
};

// p_j(y) for the state arrays above, evaluated at one column. `rej` holds the rejected
// tokens x_1..x_{j} (only the first j entries are read); the walk and the state pass share
// this code, so both see the same fp32 values.
__device__ __forceinline__ float chain_p(float p0, float q0, int y, int j, const float* zr, const float* zq,
                                         const int* rej) {
  float pv = p0;
  for (int i = 1; i <= j; ++i) {
    float qv = q0;  // q_{i-1}(y)
    if (i - 1 > 0) {
      bool r = false;
      for (int u = 0; u < i - 1; ++u) r |= rej[u] == y;
      qv = r ? 0.f : q0 / zq[i - 1];
    }
    if (zr[i] > 0.f) pv = fmaxf(pv - qv, 0.f) / zr[i];
  }
  return pv;
}

struct AcceptArgs {
  SsdTree tree;
  const float* P;
  int64_t ldp;
  const float* Q;
  int64_t ldq;
  int V;
  Rng rng;
  SampleState* st;
  int rows;
};

__global__ __launch_bounds__(SMP_THREADS) void sample_state_kernel(AcceptArgs a) {
  __shared__ KeyIdx red[16];
  __shared__ double red_d[16];
  __shared__ int red_i[16];
  __shared__ int kid_sh[SMP_MAXK];
  __shared__ int tok_sh[SMP_MAXK];
  __shared__ int n_sh;
  __shared__ float zr_sh[SMP_MAXK + 1], zq_sh[SMP_MAXK + 1];
  __shared__ int bonus_sh[SMP_MAXK + 1];
  const int r = blockIdx.x;
  const int vn = a.tree.vmeta[0];
  if (r > vn) return;
  const int cur = r - 1;
  const int t = threadIdx.x;
  // Children of cur in rank order (ranks are distinct among siblings: they are draw order).
  if (t == 0) n_sh = 0;
  __syncthreads();
  int n_all = 0;
  for (int v0 = 0; v0 < vn; v0 += SMP_THREADS) {
    const int v = v0 + t;
    const bool kid = v < vn && a.tree.vparents[v] == cur;
    int pos = 0;
    if (kid) {
      const int rk = a.tree.vranks[v];
      for (int o = 0; o < vn; ++o) pos += a.tree.vparents[o] == cur && a.tree.vranks[o] < rk;
      if (pos < SMP_MAXK) kid_sh[pos] = v;
    }
    n_all += block_sum<int>(kid ? 1 : 0, red_i);
  }
  n_all = min(n_all, SMP_MAXK);
  const float* p = a.P + (size_t)r * a.ldp;
  const float* q0 = a.Q + (size_t)(cur < 0 ? 0 : 1 + a.tree.vorig[cur]) * a.ldq;
  if (t == 0) {
    int n = 0;
    for (int i = 0; i < n_all; ++i) {
      const int v = kid_sh[i];
      const int x = a.tree.vtokens[v];
      if (q0[x] > 0.f) {
        kid_sh[n] = v;
        tok_sh[n] = x;
        ++n;
      }
    }
    n_sh = n;
  }
  __syncthreads();
  const int n = n_sh;
  // Pass 0: draw from p_0; the support and mass of q0.
  double s0 = 0.0;
  int supp = 0;
  {
    float best = -1.f;
    int bi = 0x7fffffff;
    for (int i = t * 4; i < a.V; i += 4 * SMP_THREADS) {
      const U4 rb = rng_block(a.rng, (uint32_t)(i >> 2), 0u, TAG_BONUS);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int y = i + e;
        if (y >= a.V) break;
        const float pv = p[y];
        if (pv > 0.f) {
          const float key = pv / exp1_from_bits(u4_get(rb, e));
          if (key > best) {
            best = key;
            bi = y;
          }
        }
        if (n > 0) {
          const float qv = q0[y];
          s0 += qv;
          supp += qv > 0.f;
        }
      }
    }
    const KeyIdx w = block_argmax(best, bi, red);
    if (t == 0) {
      bonus_sh[0] = w.idx == 0x7fffffff ? 0 : w.idx;
      zr_sh[0] = 0.f;
      zq_sh[0] = 1.f;
    }
  }
  if (n > 0) {
    s0 = block_sum<double>(s0, red_d);
    supp = block_sum<int>(supp, red_i);
  }
  if (t == 0 && n > 0) {
    double zq = s0;
    for (int j = 1; j <= n; ++j) {
      zq -= (double)q0[tok_sh[j - 1]];
      zq_sh[j] = (float)zq;
    }
  }
  __syncthreads();
  // Pass j: residual of state j-1 -> zr[j] and the draw from p_j.
  for (int j = 1; j <= n; ++j) {
    double zs = 0.0;
    float best = -1.f;
    int bi = 0x7fffffff;
    for (int i = t * 4; i < a.V; i += 4 * SMP_THREADS) {
      const U4 rb = rng_block(a.rng, (uint32_t)(i >> 2), 0u, TAG_BONUS);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int y = i + e;
        if (y >= a.V) break;
        const float qy = q0[y];
        const float pprev = chain_p(p[y], qy, y, j - 1, zr_sh, zq_sh, tok_sh);
        float qprev = qy;
        if (j - 1 > 0) {
          bool rj = false;
          for (int u = 0; u < j - 1; ++u) rj |= tok_sh[u] == y;
          qprev = rj ? 0.f : qy / zq_sh[j - 1];
        }
        const float res = fmaxf(pprev - qprev, 0.f);
        zs += res;
        if (res > 0.f) {
          const float key = res / exp1_from_bits(u4_get(rb, e));
          if (key > best) {
            best = key;
            bi = y;
          }
        }
      }
    }
    zs = block_sum<double>(zs, red_d);
    const KeyIdx w = block_argmax(best, bi, red);
    if (t == 0) {
      zr_sh[j] = zs > 0.0 ? (float)zs : 0.f;
      bonus_sh[j] = zs > 0.0 && w.idx != 0x7fffffff ? w.idx : bonus_sh[j - 1];
    }
    __syncthreads();
  }
  if (t == 0) {
    SampleState* s = a.st + r;
    s->n = n;
    s->supp = n > 0 ? supp : 0;
    for (int i = 0; i < SMP_MAXK; ++i) s->kid[i] = i < n ? kid_sh[i] : -1;
    for (int j = 0; j <= SMP_MAXK; ++j) {
      s->bonus[j] = j <= n ? bonus_sh[j] : 0;
      s->zr[j] = j <= n ? zr_sh[j] : 0.f;
      s->zq[j] = j <= n ? zq_sh[j] : 1.f;
    }
  }
}

// The walk of sample_verify over the precomputed states, then the same bookkeeping as the
// greedy walk: result = [n_new, tokens...], compaction sources, next root token.
__global__ void sample_walk_kernel(AcceptArgs a, int committed, int* result, int* keep_src, int* n_keep,
                                   int* root_token) {
  if (threadIdx.x != 0) return;
  int cur = -1, n_acc = 0, bonus = 0;
  int rej[SMP_MAXK];
  for (int step = 0; step <= SMP_MAXDEPTH; ++step) {
    const int r = cur + 1;
    const SampleState& s = a.st[r];
    const float* p = a.P + (size_t)r * a.ldp;
    const float* q0 = a.Q + (size_t)(cur < 0 ? 0 : 1 + a.tree.vorig[cur]) * a.ldq;
    int chosen = -1, j = 0;
    for (int i = 0; i < s.n; ++i) {
      const int v = s.kid[i];
      const int x = a.tree.vtokens[v];
      const float q0x = q0[x];
      const float pj = chain_p(p[x], q0x, x, j, s.zr, s.zq, rej);
      const float qj = j == 0 ? q0x : q0x / s.zq[j];
      const U4 rb = rng_block(a.rng, (uint32_t)j, (uint32_t)r, TAG_ACCEPT);
      const double u = uniform_from_bits(rb.x);
      const float ratio = pj / qj;
      if (u < (double)fminf(1.f, ratio)) {
        chosen = v;
        break;
      }
      rej[j] = x;
      ++j;
      if (j >= s.supp) break;  // no draft mass left
    }
    if (chosen < 0) {
      bonus = s.bonus[j];
      break;
    }
    result[1 + n_acc] = a.tree.vtokens[chosen];
    keep_src[1 + n_acc] = committed + 1 + chosen;
    ++n_acc;
    cur = chosen;
  }
  result[1 + n_acc] = bonus;
  result[0] = n_acc + 1;
  keep_src[0] = committed;
  *n_keep = n_acc + 1;
  *root_token = bonus;
}

}  // namespace ssd

using namespace ssd;

SSD_API int ssd_sample_limits(int32_t* out2) {
  if (!out2) return set_error(SSD_EINVAL, "sample_limits: null");
  out2[0] = SMP_MAXK;
  out2[1] = (int)sizeof(SampleState);
  return SSD_OK;
}

SSD_API int ssd_warp_probs_bf16(const uint16_t* logits, int64_t ld, int rows, int n, const int32_t* vocab_ids,
                                const int32_t* vocab_inv, int V, float temperature, float top_p,
                                const int32_t* tree_meta, int level, float* probs, int64_t ldp, hipStream_t stream) {
  if (!logits || !probs || (vocab_ids && !vocab_inv)) return set_error(SSD_EINVAL, "warp_probs: null pointer");
  if (rows < 0 || n <= 0 || V <= 0 || (!vocab_ids && n != V) || n > V || n > SMP_BINS * SMP_THREADS)
    return set_error(SSD_EINVAL, "warp_probs: bad shape rows=%d n=%d V=%d", rows, n, V);
  if (ld % 4 || ld < (n + 3) / 4 * 4 || ldp % 4 || ldp < V)
    return set_error(SSD_EINVAL, "warp_probs: ld %lld / ldp %lld must be multiples of 4 covering the row",
                     (long long)ld, (long long)ldp);
  if (!(temperature > 0.f)) return set_error(SSD_EINVAL, "warp_probs: temperature must be > 0");
  if (tree_meta && (level < 0 || level >= SMP_MAXDEPTH)) return set_error(SSD_ERANGE, "warp_probs: level %d", level);
  if (rows == 0) return SSD_OK;
  WarpArgs a{logits, ld, rows, n, vocab_ids, vocab_inv, V, temperature, top_p, tree_meta, level, probs, ldp};
  hipLaunchKernelGGL(warp_kernel, dim3(rows), dim3(SMP_THREADS), 0, stream, a);
  return check_launch("warp_probs");
}

SSD_API int ssd_gumbel_topk(const float* probs, int64_t ldp, int rows, int V, int k, const int32_t* tree_meta,
                            int level, uint64_t seed, uint64_t counter, int32_t* out_tok, float* out_lp,
                            hipStream_t stream) {
  if (!probs || !out_tok || !out_lp) return set_error(SSD_EINVAL, "gumbel_topk: null pointer");
  if (rows < 0 || V <= 0 || ldp % 4 || ldp < V) return set_error(SSD_EINVAL, "gumbel_topk: bad shape");
  if (k < 1 || k > SMP_MAXK) return set_error(SSD_ERANGE, "gumbel_topk: k=%d not in [1, %d]", k, SMP_MAXK);
  if (tree_meta && (level < 0 || level >= SMP_MAXDEPTH)) return set_error(SSD_ERANGE, "gumbel_topk: level %d", level);
  if (rows > 65535) return set_error(SSD_ERANGE, "gumbel_topk: %d rows", rows);
  if (rows == 0) return SSD_OK;
  TopkArgs a{probs, ldp, rows, V, k, tree_meta, level, make_rng(seed, counter), out_tok, out_lp};
  if (k <= 1)
    hipLaunchKernelGGL(gumbel_topk_kernel<1>, dim3(rows), dim3(SMP_THREADS), 0, stream, a);
  else if (k <= 2)
    hipLaunchKernelGGL(gumbel_topk_kernel<2>, dim3(rows), dim3(SMP_THREADS), 0, stream, a);
  else if (k <= 4)
    hipLaunchKernelGGL(gumbel_topk_kernel<4>, dim3(rows), dim3(SMP_THREADS), 0, stream, a);
  else if (k <= 8)
    hipLaunchKernelGGL(gumbel_topk_kernel<8>, dim3(rows), dim3(SMP_THREADS), 0, stream, a);
  else
    hipLaunchKernelGGL(gumbel_topk_kernel<16>, dim3(rows), dim3(SMP_THREADS), 0, stream, a);
  return check_launch("gumbel_topk");
}

SSD_API int ssd_sample_rows(const float* probs, int64_t ldp, int rows, int V, uint64_t seed, uint64_t counter,
                            int32_t* out_tok, hipStream_t stream) {
  if (!probs || !out_tok) return set_error(SSD_EINVAL, "sample_rows: null pointer");
  if (rows < 0 || V <= 0 || ldp < V) return set_error(SSD_EINVAL, "sample_rows: bad shape");
  if (rows == 0) return SSD_OK;
  hipLaunchKernelGGL(sample_rows_kernel, dim3(rows), dim3(SMP_THREADS), 0, stream, probs, ldp, V,
                     make_rng(seed, counter), out_tok);
  return check_launch("sample_rows");
}

SSD_API int64_t ssd_sample_state_bytes(int rows) {
  return rows < 0 ? -1 : (int64_t)rows * (int64_t)sizeof(SampleState);
}

SSD_API int ssd_accept_sample(const SsdTree* tree, const float* P, int64_t ldp, const float* Q, int64_t ldq, int V,
                              int rows, uint64_t seed, uint64_t counter, void* state, int64_t state_bytes,
                              int committed, int32_t* result, int32_t* keep_src, int32_t* n_keep,
                              int32_t* root_token, hipStream_t stream) {
  if (!tree || !P || !Q || !state || !result || !keep_src || !n_keep || !root_token)
    return set_error(SSD_EINVAL, "accept_sample: null pointer");
  if (V <= 0 || ldp < V || ldq < V || rows < 1) return set_error(SSD_EINVAL, "accept_sample: bad shape");
  if (state_bytes < ssd_sample_state_bytes(rows))
    return set_error(SSD_EINVAL, "accept_sample: state workspace %lld < %lld bytes", (long long)state_bytes,
                     (long long)ssd_sample_state_bytes(rows));
  AcceptArgs a{*tree, P, ldp, Q, ldq, V, make_rng(seed, counter), (SampleState*)state, rows};
  hipLaunchKernelGGL(sample_state_kernel, dim3(rows), dim3(SMP_THREADS), 0, stream, a);
  if (int rc = check_launch("accept_sample/state")) return rc;
  hipLaunchKernelGGL(sample_walk_kernel, dim3(1), dim3(64), 0, stream, a, committed, result, keep_src, n_keep,
                     root_token);
  return check_launch("accept_sample/walk");
}
