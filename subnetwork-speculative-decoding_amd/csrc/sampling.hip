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
// easy as 1, 2, 3", SC 2011). Key = 64-bit seed; counter = (element / 4 or step index,
// row | level << 16, round counter low word, round counter high bits << 8 | purpose tag),
// so every draw of a generation has its own counter and no result depends on launch
// shapes or on how many rows share a launch.
//
// Work layout: a row is cut into chunks of 4096 columns, one 1024-thread workgroup per
// (chunk, row), 4 consecutive columns per thread. Cross-chunk results go through a
// caller-provided workspace between launches: integer histograms built with atomics
// (order-independent), or per-chunk partials combined afterwards in chunk order, so every
// result is deterministic.
//
// Nucleus cut: the order of a row's probabilities is the order of its bf16 logits, so the
// cut is searched over the 16-bit logit keys: a 256-bin mass histogram of the key's high
// byte (mass = round(p * 2^52), exact integer sums), then a 256-bin count histogram of the
// low byte inside the cut bin, which fixes the cut key; equal logits rank lower column first
// (per-chunk counts of the cut key give each tie its column rank).
#include "common.h"

#include <math.h>

namespace ssd {

constexpr int SMP_THREADS = 1024;
constexpr int SMP_CHUNK = 4096;
constexpr int SMP_MAXK = 16;      // children per node / draws per row
constexpr int SMP_MAXC = 256;     // chunks per row (rows up to 1M columns)
constexpr int SMP_MAXDEPTH = 32;  // tree depth (matches the tree kernels)

enum SmpTag { TAG_PROPOSE = 1, TAG_ACCEPT = 2, TAG_BONUS = 3, TAG_DRAW = 4, TAG_TOP64 = 5 };

struct Rng {
  uint32_t k0, k1;       // key: seed
  uint32_t c2, c3_base;  // counter words 2 and 3 (round counter; tag is or-ed into c3)
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

constexpr int NO_IDX = 0x7fffffff;

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

__device__ __forceinline__ uint64_t block_scan64(uint64_t v, uint64_t* sh) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint64_t n = __shfl_up(v, o);
    if (lane >= o) v += n;
  }
  if (lane == 63) sh[w] = v;
  __syncthreads();
  uint64_t add = 0;
  for (int i = 0; i < w; ++i) add += sh[i];
  __syncthreads();
  return v + add;
}

// ------------------------------------------------------------------------ workspace
// One caller-provided buffer, carved per (rows, chunks). Histograms are cleared by the first
// launch of each warp; every other array is fully written before it is read.
struct SmpWs {
  float2* stats;      // [rows][C] chunk (max, sum exp) of logits / T
  uint64_t* coarse;   // [rows][256] mass by key high byte
  uint32_t* fine;     // [rows][256] count by key low byte inside the cut bin
  uint32_t* finec;    // [rows][C][256] the same per chunk (column rank of ties)
  KeyIdx* cand;       // [rows][C][SMP_MAXK] per-chunk Gumbel top-k candidates
  int* csupp;         // [rows][C] per-chunk support size
  KeyIdx* arg;        // [rows][C] per-chunk categorical draw
  double* zr;         // [rows][SMP_MAXK + 1][C] residual mass partials per rejection state
  KeyIdx* bon;        // [rows][SMP_MAXK + 1][C] bonus draw partials per rejection state
  double* s0;         // [rows][C] mass of q0 per chunk
  int* supp;          // [rows][C] support of q0 per chunk
  int C;
};

static int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

static int64_t smp_layout(int rows, int C, char* base, SmpWs* ws) {
  int64_t off = 0;
  auto take = [&](int64_t bytes) -> char* {
    char* p = base ? base + off : nullptr;
    off += align256(bytes);
    return p;
  };
  const int64_t R = rows, CC = C;
  SmpWs w;
  w.stats = (float2*)take(R * CC * sizeof(float2));
  w.coarse = (uint64_t*)take(R * 256 * 8);
  w.fine = (uint32_t*)take(R * 256 * 4);
  w.finec = (uint32_t*)take(R * CC * 256 * 4);
  w.cand = (KeyIdx*)take(R * CC * SMP_MAXK * sizeof(KeyIdx));
  w.csupp = (int*)take(R * CC * 4);
  w.arg = (KeyIdx*)take(R * CC * sizeof(KeyIdx));
  w.zr = (double*)take(R * (SMP_MAXK + 1) * CC * 8);
  w.bon = (KeyIdx*)take(R * (SMP_MAXK + 1) * CC * sizeof(KeyIdx));
  w.s0 = (double*)take(R * CC * 8);
  w.supp = (int*)take(R * CC * 4);
  w.C = C;
  if (ws) *ws = w;
  return off;
}

static int chunks_of(int n) { return (n + SMP_CHUNK - 1) / SMP_CHUNK; }

// ------------------------------------------------------------------------ warp
struct WarpArgs {
  const bf16_t* logits;
  int64_t ld;
  int rows, n;        // logit rows and columns
  const int* vocab;   // column -> token (draft-vocab subset), or null (column = token)
  const int* inv;     // token -> column or -1 (with vocab), length V
  int V;              // output row length (full vocabulary)
  float temp, top_p;
  uint64_t T;         // top_p in units of 2^-52
  const int* meta;    // tree meta: rows are the frontier proposing `level`; null: plain rows
  int level;
  float* out;
  int64_t ldo;
  SmpWs ws;
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

// Monotone 16-bit key of a bf16 value (ascending key = ascending value) and its inverse.
__device__ __forceinline__ uint32_t bf_key(uint32_t h) { return h ^ ((h & 0x8000u) ? 0xffffu : 0x8000u); }
__device__ __forceinline__ uint32_t key_bf(uint32_t k) { return k ^ ((k & 0x8000u) ? 0x8000u : 0xffffu); }

// The probability of a logit and its fixed-point mass: one code path for every use, so a
// value and the mass accumulated for it always agree bit for bit.
__device__ __forceinline__ float prob_of(uint32_t h, float temp, float M, float S) {
  return expf(bf2f((bf16_t)h) / temp - M) / S;
}
__device__ __forceinline__ uint64_t mass_of(float p) { return __double2ull_rn((double)p * 0x1p52); }

__device__ __forceinline__ void load4_bf16(const bf16_t* row, int i, int n, uint32_t h[4]) {
  if (i + 3 < n) {
    const uint2 raw = *(const uint2*)(row + i);
    h[0] = raw.x & 0xffff;
    h[1] = raw.x >> 16;
    h[2] = raw.y & 0xffff;
    h[3] = raw.y >> 16;
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) h[e] = i + e < n ? row[i + e] : 0xff80u;  // -inf pads
  }
}

struct WarpShared {
  float red_f[16];
  uint32_t red_u[16];
  uint64_t red_l[16];
  uint64_t histm[256];
  uint32_t histc[256];
  float M, S;
  int cut;
  uint64_t above, total;
};

// Row max and sum exp from the chunk partials (fixed order: block reduction over chunk index).
__device__ __forceinline__ void row_stats(const float2* st, int C, WarpShared& sh, float& M, float& S) {
  const int t = threadIdx.x;
  const float2 v = t < C ? st[t] : make_float2(-INFINITY, 0.f);
  M = block_max(v.x, sh.red_f);
  S = block_sum<float>(t < C && v.x != -INFINITY ? v.y * expf(v.x - M) : 0.f, sh.red_f);
}

// Scan a 256-bin histogram (bin masses from mass_fn(bin)) from the largest key down: the bin
// holding the first entry whose preceding mass exceeds T. Sets sh.cut (-1 when the whole
// histogram fits under T), sh.above (mass of the bins above the cut bin, plus `base`) and
// sh.total.
template <typename MassFn>
__device__ __forceinline__ void cut_scan(MassFn mass_fn, uint64_t base, uint64_t T, WarpShared& sh) {
  const int t = threadIdx.x;
  const int b = 255 - t;
  const uint64_t v = t < 256 ? mass_fn(b) : 0ull;
  const uint64_t incl = block_scan64(v, sh.red_l);
  if (t == 0) sh.cut = -1;
  if (t == 255) sh.total = base + incl;
  __syncthreads();
  if (t < 256 && v > 0 && base + incl - v <= T && T < base + incl) {
    sh.cut = b;
    sh.above = base + incl - v;
  }
  __syncthreads();
}

// L0: chunk max / sum exp; the first chunk of each row clears the row's histograms.
__global__ __launch_bounds__(SMP_THREADS) void warp_stats_kernel(WarpArgs a) {
  __shared__ WarpShared sh;
  int F, base;
  frontier_rows(a.meta, a.level, a.rows, F, base);
  const int f = blockIdx.y, c = blockIdx.x, t = threadIdx.x;
  if (f >= F) return;
  if (c == 0 && a.top_p < 1.f) {
    if (t < 256) a.ws.coarse[(size_t)f * 256 + t] = 0;
    if (t < 256) a.ws.fine[(size_t)f * 256 + t] = 0;
  }
  const int i = c * SMP_CHUNK + t * 4;
  uint32_t h[4];
  load4_bf16(a.logits + (size_t)f * a.ld, i, a.n, h);
  float x[4], m = -INFINITY;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    x[e] = i + e < a.n ? bf2f((bf16_t)h[e]) / a.temp : -INFINITY;
    m = fmaxf(m, x[e]);
  }
  const float M = block_max(m, sh.red_f);
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) s += i + e < a.n ? expf(x[e] - M) : 0.f;
  const float S = block_sum<float>(s, sh.red_f);
  if (t == 0) a.ws.stats[(size_t)f * a.ws.C + c] = make_float2(M, S);
}

// L1: mass / count histogram of the key high byte.
__global__ __launch_bounds__(SMP_THREADS) void warp_coarse_kernel(WarpArgs a) {
  __shared__ WarpShared sh;
  int F, base;
  frontier_rows(a.meta, a.level, a.rows, F, base);
  const int f = blockIdx.y, c = blockIdx.x, t = threadIdx.x;
  if (f >= F) return;
  float M, S;
  row_stats(a.ws.stats + (size_t)f * a.ws.C, a.ws.C, sh, M, S);
  if (t < 256) sh.histm[t] = 0;
  __syncthreads();
  const int i = c * SMP_CHUNK + t * 4;
  uint32_t h[4];
  load4_bf16(a.logits + (size_t)f * a.ld, i, a.n, h);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if (i + e >= a.n) continue;
    const uint32_t bin = bf_key(h[e]) >> 8;
    atomicAdd((unsigned long long*)&sh.histm[bin], (unsigned long long)mass_of(prob_of(h[e], a.temp, M, S)));
  }
  __syncthreads();
  if (t < 256 && sh.histm[t])
    atomicAdd((unsigned long long*)&a.ws.coarse[(size_t)f * 256 + t], (unsigned long long)sh.histm[t]);
}

// L2: inside the coarse cut bin, count histogram of the key low byte (row total and per chunk).
__global__ __launch_bounds__(SMP_THREADS) void warp_fine_kernel(WarpArgs a) {
  __shared__ WarpShared sh;
  int F, base;
  frontier_rows(a.meta, a.level, a.rows, F, base);
  const int f = blockIdx.y, c = blockIdx.x, t = threadIdx.x;
  if (f >= F) return;
  const uint64_t* coarse = a.ws.coarse + (size_t)f * 256;
  cut_scan([&](int b) { return coarse[b]; }, 0ull, a.T, sh);
  const int cut = sh.cut;
  if (cut < 0) return;  // everything fits under top_p (uniform per block)
  if (t < 256) sh.histc[t] = 0;
  __syncthreads();
  const int i = c * SMP_CHUNK + t * 4;
  uint32_t h[4];
  load4_bf16(a.logits + (size_t)f * a.ld, i, a.n, h);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t k = bf_key(h[e]);
    if (i + e < a.n && (int)(k >> 8) == cut) atomicAdd(&sh.histc[k & 255], 1u);
  }
  __syncthreads();
  if (t < 256) {
    const uint32_t v = sh.histc[t];
    a.ws.finec[((size_t)f * a.ws.C + c) * 256 + t] = v;
    if (v) atomicAdd(&a.ws.fine[(size_t)f * 256 + t], v);
  }
}

// L3: probabilities out (renormalised survivors when top_p < 1); zeros outside a subset.
__global__ __launch_bounds__(SMP_THREADS) void warp_final_kernel(WarpArgs a) {
  __shared__ WarpShared sh;
  __shared__ uint32_t cut_key_sh, c_keep_sh, prefix_sh;
  __shared__ uint64_t kept_sh;
  int F, base;
  frontier_rows(a.meta, a.level, a.rows, F, base);
  const int f = blockIdx.y, c = blockIdx.x, t = threadIdx.x;
  if (f >= F) return;
  float* out = a.out + (size_t)(base + f) * a.ldo;
  if (a.vocab) {  // tokens outside the subset have probability 0
    const int y0 = c * SMP_CHUNK + t * 4;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (y0 + e < a.V && a.inv[y0 + e] < 0) out[y0 + e] = 0.f;
  }
  if (c * SMP_CHUNK >= a.n) return;  // a zero-fill-only chunk (uniform per block)
  float M, S;
  row_stats(a.ws.stats + (size_t)f * a.ws.C, a.ws.C, sh, M, S);
  uint32_t cut_key = 0, c_keep = 0xffffffffu, prefix = 0;
  float scale = 1.f;
  if (a.top_p < 1.f) {
    const uint64_t* coarse = a.ws.coarse + (size_t)f * 256;
    cut_scan([&](int b) { return coarse[b]; }, 0ull, a.T, sh);
    if (sh.cut < 0) {  // keep all: renormalise by the total mass
      scale = (float)(1.0 / ((double)sh.total * 0x1p-52));
    } else {
      const int cb = sh.cut;
      const uint64_t above = sh.above;
      const uint32_t* fine = a.ws.fine + (size_t)f * 256;
      // mass of fine bin b = count * mass of that exact logit
      cut_scan([&](int b) {
        const uint32_t n = fine[b];
        return n ? (uint64_t)n * mass_of(prob_of(key_bf(((uint32_t)cb << 8) | (uint32_t)b), a.temp, M, S)) : 0ull;
      }, above, a.T, sh);
      if (t == 0) {
        const int fb = sh.cut < 0 ? 0 : sh.cut;  // always found: the coarse bin's mass straddles T
        const uint32_t key = ((uint32_t)cb << 8) | (uint32_t)fb;
        const uint32_t n_t = fine[fb];
        const uint64_t w = mass_of(prob_of(key_bf(key), a.temp, M, S));
        const uint64_t C3 = sh.cut < 0 ? above : sh.above;
        uint64_t keep = n_t;
        if (w > 0 && a.T >= C3) keep = min((uint64_t)n_t, (a.T - C3) / w + 1ull);
        cut_key_sh = key;
        c_keep_sh = (uint32_t)keep;
        kept_sh = C3 + keep * w;
      }
      __syncthreads();
      cut_key = cut_key_sh;
      c_keep = c_keep_sh;
      scale = (float)(1.0 / ((double)kept_sh * 0x1p-52));
      // ties of the cut key in earlier chunks
      const uint32_t fb = cut_key & 255;
      const uint32_t v = t < c ? a.ws.finec[((size_t)f * a.ws.C + t) * 256 + fb] : 0u;
      const uint32_t pre = block_sum<uint32_t>(v, (uint32_t*)sh.red_u);
      if (t == 0) prefix_sh = pre;
      __syncthreads();
      prefix = prefix_sh;
    }
  }
  const int i = c * SMP_CHUNK + t * 4;
  uint32_t h[4];
  load4_bf16(a.logits + (size_t)f * a.ld, i, a.n, h);
  // column rank of this thread's ties of the cut key
  uint32_t ties = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) ties += (i + e < a.n && bf_key(h[e]) == cut_key) ? 1u : 0u;
  uint32_t rank = 0;
  if (a.top_p < 1.f && c_keep != 0xffffffffu) rank = prefix + block_scan(ties, sh.red_u) - ties;
  float p[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t k = bf_key(h[e]);
    bool keep = true;
    if (a.top_p < 1.f && c_keep != 0xffffffffu) {
      keep = k > cut_key;
      if (k == cut_key && i + e < a.n) keep = rank++ < c_keep;
    }
    const float pv = prob_of(h[e], a.temp, M, S);
    p[e] = keep ? (a.top_p < 1.f ? pv * scale : pv) : 0.f;
  }
  if (!a.vocab && i + 3 < a.n) {
    *(float4*)(out + i) = make_float4(p[0], p[1], p[2], p[3]);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (i + e < a.n) out[a.vocab ? a.vocab[i + e] : i + e] = p[e];
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
  SmpWs ws;
};

__device__ __forceinline__ void load4_f32(const float* row, int i, int n, float v[4]) {
  if (i + 3 < n) {
    const float4 q = *(const float4*)(row + i);
    v[0] = q.x;
    v[1] = q.y;
    v[2] = q.z;
    v[3] = q.w;
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = i + e < n ? row[i + e] : 0.f;
  }
}

// Per chunk: the k largest keys q(y) / E(y) (E ~ Exp(1) from the PROPOSE stream) and the
// support size. Keys of one thread are its 4 columns; the chunk's top k are popped one at a
// time by block argmax.
__global__ __launch_bounds__(SMP_THREADS) void gumbel_chunk_kernel(TopkArgs a) {
  __shared__ KeyIdx red[16];
  __shared__ int red_i[16];
  int F, base;
  frontier_rows(a.meta, a.level, a.rows, F, base);
  const int f = blockIdx.y, c = blockIdx.x, t = threadIdx.x;
  if (f >= F) return;
  const float* q = a.q + (size_t)(base + f) * a.ldq;
  const int i = c * SMP_CHUNK + t * 4;
  float v[4];
  load4_f32(q, i, a.V, v);
  const U4 r = rng_block(a.rng, (uint32_t)(i >> 2), (uint32_t)f | ((uint32_t)a.level << 16), TAG_PROPOSE);
  float kk[4];
  int ki[4];
  int supp = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const bool on = i + e < a.V && v[e] > 0.f;
    supp += on;
    kk[e] = on ? v[e] / exp1_from_bits(u4_get(r, e)) : -1.f;
    ki[e] = on ? i + e : NO_IDX;
  }
  const int support = block_sum<int>(supp, red_i);
  KeyIdx* cand = a.ws.cand + ((size_t)f * a.ws.C + c) * SMP_MAXK;
  for (int j = 0; j < a.k; ++j) {
    // this thread's best remaining column
    int b = 0;
#pragma unroll
    for (int e = 1; e < 4; ++e)
      if (better(kk[e], ki[e], kk[b], ki[b])) b = e;
    float bk = kk[0];
    int bi = ki[0];
#pragma unroll
    for (int e = 1; e < 4; ++e)
      if (e == b) {
        bk = kk[e];
        bi = ki[e];
      }
    const KeyIdx w = block_argmax(bk, bi, red);
    if (t == 0) cand[j] = w;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (ki[e] == w.idx) {
        kk[e] = -1.f;
        ki[e] = NO_IDX;
      }
  }
  if (t == 0) a.ws.csupp[(size_t)f * a.ws.C + c] = support;
}

// Per row: merge the chunks' candidates in chunk order; write min(k, support) tokens in draw
// order and log q of each.
__global__ __launch_bounds__(SMP_THREADS) void gumbel_merge_kernel(TopkArgs a) {
  __shared__ KeyIdx red[16];
  __shared__ int red_i[16];
  int F, base;
  frontier_rows(a.meta, a.level, a.rows, F, base);
  const int f = blockIdx.x, t = threadIdx.x;
  if (f >= F) return;
  const int C = a.ws.C;
  const int total = C * a.k;
  const float* q = a.q + (size_t)(base + f) * a.ldq;
  int support = block_sum<int>(t < C ? a.ws.csupp[(size_t)f * C + t] : 0, red_i);
  const int take = min(a.k, support);
  // each thread holds up to 4 candidates (C * k <= 256 * 16 = 4096)
  float kk[4];
  int ki[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int j = t * 4 + e;
    if (j < total) {
      const KeyIdx v = a.ws.cand[((size_t)f * C + j / a.k) * SMP_MAXK + j % a.k];
      kk[e] = v.key;
      ki[e] = v.idx;
    } else {
      kk[e] = -1.f;
      ki[e] = NO_IDX;
    }
  }
  for (int r = 0; r < a.k; ++r) {
    int tok = -1;
    if (r < take) {
      int b = 0;
#pragma unroll
      for (int e = 1; e < 4; ++e)
        if (better(kk[e], ki[e], kk[b], ki[b])) b = e;
      float bk = kk[0];
      int bi = ki[0];
#pragma unroll
      for (int e = 1; e < 4; ++e)
        if (e == b) {
          bk = kk[e];
          bi = ki[e];
        }
      const KeyIdx w = block_argmax(bk, bi, red);
      tok = w.idx == NO_IDX ? -1 : w.idx;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (ki[e] == w.idx) {
          kk[e] = -1.f;
          ki[e] = NO_IDX;
        }
    }
    if (t == 0) {
      a.out_tok[f * a.k + r] = tok;
      a.out_lp[f * a.k + r] = tok >= 0 ? logf(q[tok]) : 0.f;
    }
  }
}

// ------------------------------------------------------------- categorical draws
// One draw per row: argmax_y p(y) / E(y), E from the DRAW stream with counter (y / 4, row).
__global__ __launch_bounds__(SMP_THREADS) void draw_chunk_kernel(const float* __restrict__ P, int64_t ldp, int V,
                                                                 Rng rng, SmpWs ws) {
  __shared__ KeyIdx red[16];
  const int row = blockIdx.y, c = blockIdx.x, t = threadIdx.x;
  const int i = c * SMP_CHUNK + t * 4;
  float v[4];
  load4_f32(P + (size_t)row * ldp, i, V, v);
  const U4 r = rng_block(rng, (uint32_t)(i >> 2), (uint32_t)row, TAG_DRAW);
  float best = -1.f;
  int bi = NO_IDX;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if (i + e < V && v[e] > 0.f) {
      const float key = v[e] / exp1_from_bits(u4_get(r, e));
      if (better(key, i + e, best, bi)) {
        best = key;
        bi = i + e;
      }
    }
  }
  const KeyIdx w = block_argmax(best, bi, red);
  if (t == 0) ws.arg[(size_t)row * ws.C + c] = w;
}

__device__ __forceinline__ KeyIdx merge_chunks(const KeyIdx* part, int C) {
  KeyIdx b{-1.f, NO_IDX};
  for (int c = 0; c < C; ++c)
    if (better(part[c].key, part[c].idx, b.key, b.idx)) b = part[c];
  return b;
}

__global__ void draw_merge_kernel(int rows, SmpWs ws, int* __restrict__ out_tok) {
  const int row = blockIdx.x * blockDim.x + threadIdx.x;
  if (row >= rows) return;
  const KeyIdx b = merge_chunks(ws.arg + (size_t)row * ws.C, ws.C);
  out_tok[row] = b.idx == NO_IDX ? 0 : b.idx;
}

// ----------------------------------------------------------- speculative acceptance
// Verify row r holds node cur = r - 1 (root: r = 0). State j of a node = after its first j
// children (rank order, q0(x) > 0) were rejected:
//   q_0 = q0, q_j(y) = q0(y) [y not rejected] / zq[j]  (zq[j] = sum q0 - sum of rejected q0),
//   p_0 = p,  p_j = (p_{j-1} - q_{j-1})+ / zr[j] when zr[j] = sum (p_{j-1} - q_{j-1})+ > 0,
//             p_j = p_{j-1} otherwise,
// and bonus[j] = the categorical draw from p_j (one shared Exp(1) vector per round: only one
// state's draw is ever used, and which one is decided by the acceptance uniforms alone).
// Pass j (one launch over all rows and chunks) produces the chunk partials of zr[j] and
// bonus[j]; partials are combined by whoever needs them (the next pass, the walk), always by
// the same wave reduction (combine_states), so every reader sees the same values.
struct AcceptArgs {
  SsdTree tree;
  const float* P;
  int64_t ldp;
  const float* Q;
  int64_t ldq;
  int V;
  int rows;      // verify rows in P and in the workspace
  int max_kids;  // children considered per node (the launch runs this many rejection passes)
  Rng rng;
  SmpWs ws;
};

constexpr int SMP_MAXNODES = 63;  // verify nodes (rows = nodes + 1 <= 64)

__device__ __forceinline__ int verify_nodes(const SsdTree& t) { return min(t.vmeta[0], SMP_MAXNODES); }

struct NodeKids {
  int n;
  int kid[SMP_MAXK];
  int tok[SMP_MAXK];
};

__device__ __forceinline__ const float* q_row(const AcceptArgs& a, int cur) {
  return a.Q + (size_t)(cur < 0 ? 0 : 1 + a.tree.vorig[cur]) * a.ldq;
}

// Children of cur in rank order (ranks are distinct among siblings: they are draw order),
// skipping those with q0(x) <= 0 (verify.py:77-78), built by a whole workgroup of at least 64
// threads (tree nodes staged in LDS; each child finds its position by counting siblings of lower
// rank). Result in `k` (shared), valid after return.
__device__ __forceinline__ void node_kids_block(const AcceptArgs& a, int cur, NodeKids& k, int* sh_par,
                                                int* sh_rank, int* sh_pos) {
  const int vn = verify_nodes(a.tree);
  const int t = threadIdx.x;
  if (t < vn) {
    sh_par[t] = a.tree.vparents[t];
    sh_rank[t] = a.tree.vranks[t];
  }
  if (t < SMP_MAXK) sh_pos[t] = -1;
  __syncthreads();
  if (t < vn && sh_par[t] == cur) {
    int pos = 0;
    for (int o = 0; o < vn; ++o) pos += sh_par[o] == cur && sh_rank[o] < sh_rank[t];
    if (pos < SMP_MAXK) sh_pos[pos] = t;
  }
  __syncthreads();
  if (t < 64) {  // wave 0: lane i takes rank position i (positions are dense from 0), loads in parallel
    const float* q0 = q_row(a, cur);
    int pos = t < a.max_kids && t < SMP_MAXK ? sh_pos[t] : -1;
    // the list ends at the first empty position, as a rank-order scan would stop there
    const uint64_t filled = __ballot(pos >= 0);
    if (t >= __ffsll((unsigned long long)~filled) - 1) pos = -1;
    const int x = pos >= 0 ? a.tree.vtokens[pos] : 0;
    const bool keep = pos >= 0 && q0[x] > 0.f;
    const uint64_t m = __ballot(keep);
    if (keep) {
      const int slot = __popcll(m & ((1ull << t) - 1));  // kept children of lower rank
      k.kid[slot] = pos;
      k.tok[slot] = x;
    }
    if (t == 0) k.n = __popcll(m);
  }
  __syncthreads();
}

// Wave reductions: a butterfly of exchanges, so every lane ends with the same value (each step adds
// the same two partials on both lanes, and floating-point addition is commutative) and the order
// of the additions is fixed.
__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) v += __shfl_xor(v, o);
  return v;
}
__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) v += __shfl_xor(v, o);
  return v;
}
__device__ __forceinline__ KeyIdx wave_argmax(float k, int i) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const float ok = __shfl_xor(k, o);
    const int oi = __shfl_xor(i, o);
    if (better(ok, oi, k, i)) {
      k = ok;
      i = oi;
    }
  }
  return KeyIdx{k, i};
}

struct StateScalars {
  double s0;
  int supp;
  float zr[SMP_MAXK + 1];  // zr[j] for j >= 1 (0 when the residual had no mass)
  float zq[SMP_MAXK + 1];  // zq[0] = 1
};

// Combine the chunk partials of row r: q0's mass and support, and states 1..upto. Called by a
// whole wave: lane l sums chunks l, l + 64, ..., then the wave reduces; every lane returns the
// same values, and every reader (the passes and the walk) uses this code, so all see the same.
__device__ __forceinline__ void combine_states(const AcceptArgs& a, int r, const float* q0, const NodeKids& k,
                                               int upto, StateScalars& s) {
  const int C = a.ws.C, lane = threadIdx.x & 63;
  double s0 = 0.0;
  int supp = 0;
  for (int c = lane; c < C; c += 64) {
    s0 += a.ws.s0[(size_t)r * C + c];
    supp += a.ws.supp[(size_t)r * C + c];
  }
  double z[SMP_MAXK + 1];
#pragma unroll
  for (int j = 1; j <= SMP_MAXK; ++j) {
    z[j] = 0.0;
    if (j <= upto)
      for (int c = lane; c < C; c += 64) z[j] += a.ws.zr[((size_t)r * (SMP_MAXK + 1) + j) * C + c];
  }
  s0 = wave_sum_d(s0);
  s.s0 = s0;
  s.supp = wave_sum_i(supp);
  s.zr[0] = 0.f;
  s.zq[0] = 1.f;
  double zq = s0;
#pragma unroll
  for (int j = 1; j <= SMP_MAXK; ++j) {
    if (j <= upto) {  // uniform
      const double zj = wave_sum_d(z[j]);
      s.zr[j] = zj > 0.0 ? (float)zj : 0.f;
      zq -= (double)q0[k.tok[j - 1]];
      s.zq[j] = (float)zq;
    }
  }
}

// p_j(y) for the state scalars, evaluated at one column. `rej` holds the rejected tokens
// x_1..x_j (only the first j entries are read); the passes and the walk share this code.
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

// Pass 0: bonus draw from p_0 per chunk; q0's mass and support per chunk.
__global__ __launch_bounds__(SMP_THREADS) void state0_kernel(AcceptArgs a) {
  __shared__ KeyIdx red[16];
  __shared__ double red_d[16];
  __shared__ int red_i[16];
  __shared__ int sh_par[64], sh_rank[64], sh_pos[SMP_MAXK];
  __shared__ NodeKids kids;
  const int r = blockIdx.y, c = blockIdx.x, t = threadIdx.x;
  if (r > verify_nodes(a.tree)) return;
  const int cur = r - 1;
  node_kids_block(a, cur, kids, sh_par, sh_rank, sh_pos);
  const int i = c * SMP_CHUNK + t * 4;
  float p[4];
  load4_f32(a.P + (size_t)r * a.ldp, i, a.V, p);
  const U4 rb = rng_block(a.rng, (uint32_t)(i >> 2), 0u, TAG_BONUS);
  float best = -1.f;
  int bi = NO_IDX;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if (i + e < a.V && p[e] > 0.f) {
      const float key = p[e] / exp1_from_bits(u4_get(rb, e));
      if (better(key, i + e, best, bi)) {
        best = key;
        bi = i + e;
      }
    }
  }
  const KeyIdx w = block_argmax(best, bi, red);
  double s0 = 0.0;
  int supp = 0;
  if (kids.n > 0) {
    float q[4];
    load4_f32(q_row(a, cur), i, a.V, q);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      s0 += (double)q[e];
      supp += q[e] > 0.f;
    }
    s0 = block_sum<double>(s0, red_d);
    supp = block_sum<int>(supp, red_i);
  }
  if (t == 0) {
    const int C = a.ws.C;
    a.ws.bon[((size_t)r * (SMP_MAXK + 1) + 0) * C + c] = w;
    a.ws.s0[(size_t)r * C + c] = s0;
    a.ws.supp[(size_t)r * C + c] = supp;
  }
}

// Pass j >= 1: residual of state j-1 -> chunk partials of zr[j] and of the draw from p_j.
__global__ __launch_bounds__(SMP_THREADS) void statej_kernel(AcceptArgs a, int j) {
  __shared__ KeyIdx red[16];
  __shared__ double red_d[16];
  __shared__ int sh_par[64], sh_rank[64], sh_pos[SMP_MAXK];
  __shared__ NodeKids kids;
  __shared__ StateScalars st;
  const int r = blockIdx.y, c = blockIdx.x, t = threadIdx.x;
  if (r > verify_nodes(a.tree)) return;
  const int cur = r - 1;
  node_kids_block(a, cur, kids, sh_par, sh_rank, sh_pos);
  if (kids.n < j) return;  // uniform: this node has fewer children
  const float* q0 = q_row(a, cur);
  if (t < 64) combine_states(a, r, q0, kids, j - 1, st);  // wave 0; its lanes store the same values
  __syncthreads();
  const int i = c * SMP_CHUNK + t * 4;
  float p[4], q[4];
  load4_f32(a.P + (size_t)r * a.ldp, i, a.V, p);
  load4_f32(q0, i, a.V, q);
  const U4 rb = rng_block(a.rng, (uint32_t)(i >> 2), 0u, TAG_BONUS);
  double zs = 0.0;
  float best = -1.f;
  int bi = NO_IDX;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int y = i + e;
    if (y >= a.V) continue;
    const float pprev = chain_p(p[e], q[e], y, j - 1, st.zr, st.zq, kids.tok);
    float qprev = q[e];
    if (j - 1 > 0) {
      bool rj = false;
      for (int u = 0; u < j - 1; ++u) rj |= kids.tok[u] == y;
      qprev = rj ? 0.f : q[e] / st.zq[j - 1];
    }
    const float res = fmaxf(pprev - qprev, 0.f);
    zs += (double)res;
    if (res > 0.f) {
      const float key = res / exp1_from_bits(u4_get(rb, e));
      if (better(key, y, best, bi)) {
        best = key;
        bi = y;
      }
    }
  }
  zs = block_sum<double>(zs, red_d);
  const KeyIdx w = block_argmax(best, bi, red);
  if (t == 0) {
    const int C = a.ws.C;
    a.ws.zr[((size_t)r * (SMP_MAXK + 1) + j) * C + c] = zs;
    a.ws.bon[((size_t)r * (SMP_MAXK + 1) + j) * C + c] = w;
  }
}

// The walk of sample_verify over the state scalars, then the same bookkeeping as the greedy
// walk: result = [n_new, tokens...], compaction sources, next root token. One wave: every lane
// walks the same path with the same values (the child lists, the state sums and the bonus merge
// are wave-wide operations), lane 0 writes the result.
__global__ __launch_bounds__(64) void sample_walk_kernel(AcceptArgs a, int committed, int* result, int* keep_src,
                                                        int* n_keep, int* root_token) {
  __shared__ int sh_par[64], sh_rank[64], sh_pos[SMP_MAXK];
  __shared__ NodeKids kids;
  const int lane = threadIdx.x;
  const int C = a.ws.C;
  int cur = -1, n_acc = 0, bonus = 0;
  int rej[SMP_MAXK];
  StateScalars s;
  for (int step = 0; step <= SMP_MAXDEPTH; ++step) {
    const int r = cur + 1;
    if (r >= a.rows) break;  // a tree larger than the launch's rows (the engine never makes one)
    node_kids_block(a, cur, kids, sh_par, sh_rank, sh_pos);
    const int kn = kids.n;
    const float* q0 = q_row(a, cur);
    const float* p = a.P + (size_t)r * a.ldp;
    s.supp = 0;
    s.zr[0] = 0.f;
    s.zq[0] = 1.f;
    if (kn > 0) combine_states(a, r, q0, kids, kn, s);
    int chosen = -1, j = 0;
    for (int i = 0; i < kn; ++i) {
      const int x = kids.tok[i];
      const float q0x = q0[x];
      const float pj = chain_p(p[x], q0x, x, j, s.zr, s.zq, rej);
      const float qj = j == 0 ? q0x : q0x / s.zq[j];
      const double u = uniform_from_bits(rng_block(a.rng, (uint32_t)j, (uint32_t)r, TAG_ACCEPT).x);
      if (u < (double)fminf(1.f, pj / qj)) {
        chosen = kids.kid[i];
        break;
      }
      rej[j] = x;
      ++j;
      if (j >= s.supp) break;  // no draft mass left
    }
    if (chosen < 0) {
      int jj = j;
      while (jj > 0 && !(s.zr[jj] > 0.f)) --jj;  // p_j == p_{j-1} when the residual had no mass
      // the categorical draw from p_jj: the best of the chunks' records (a strict order on
      // (key, column), so any merge order gives the same record)
      const KeyIdx* part = a.ws.bon + ((size_t)r * (SMP_MAXK + 1) + jj) * C;
      KeyIdx b{-1.f, NO_IDX};
      for (int c = lane; c < C; c += 64)
        if (better(part[c].key, part[c].idx, b.key, b.idx)) b = part[c];
      b = wave_argmax(b.key, b.idx);
      bonus = b.idx == NO_IDX ? 0 : b.idx;
      break;
    }
    if (lane == 0) {
      result[1 + n_acc] = a.tree.vtokens[chosen];
      keep_src[1 + n_acc] = committed + 1 + chosen;
    }
    ++n_acc;
    cur = chosen;
  }
  if (lane == 0) {
    result[1 + n_acc] = bonus;
    result[0] = n_acc + 1;
    keep_src[0] = committed;
    *n_keep = n_acc + 1;
    *root_token = bonus;
  }
}

// ------------------------------------------------------ batched acceptance trials
// Many independent rounds of proposal + acceptance over one fixed set of per-node distributions
// (row 0 the root, row 1 + v node v; P = warped target, Q = warped draft of the node's
// children), one wave per trial, trial t drawing with round counter counter0 + t. The tree is
// unpruned with branch[d] children per node at level d, numbered level by level (level L node with
// in-level index f has children start[L + 1] + f * branch[L + 1] + i, i = draw order). Each trial
// draws only the children on its walk; every draw and decision uses the engine's streams,
// counters and formulas (gumbel_chunk / state0 / statej / sample_walk above): Gumbel keys
// q / Exp(1) from the PROPOSE stream at (column / 4, f | level << 16), acceptance uniforms at
// (rejections, row), residual states through chain_p, the bonus race on the unnormalised
// residual at (column / 4, 0). Sums run over each row's support list (columns where P or Q is
// nonzero; every other column contributes nothing) in double, in lane-strided order. Only the
// sums' rounding order differs from the per-round kernels, so a trial reproduces the engine's
// round with the same counter decision for decision.
constexpr int TRIAL_MAXD = 8;

struct TrialArgs {
  const float* P;
  int64_t ldp;
  const float* Q;
  int64_t ldq;
  const int* cols;  // support columns of row r: cols[off[r] .. off[r + 1]), ascending
  const int* off;
  int depth;
  int branch[TRIAL_MAXD];
  int start[TRIAL_MAXD + 1];
  uint64_t seed, counter0;
  int trials;
  int* out_tok;  // [trials][depth + 1]: accepted tokens, then the bonus
  int* out_n;    // [trials]
};


// q_{j-1}(y) as statej_kernel computes it: rejected tokens have no draft mass left.
__device__ __forceinline__ float trial_qprev(float q0, int y, int j, const float* zq, const int* rej) {
  if (j - 1 <= 0) return q0;
  bool r = false;
  for (int u = 0; u < j - 1; ++u) r |= rej[u] == y;
  return r ? 0.f : q0 / zq[j - 1];
}

__global__ __launch_bounds__(256) void accept_trials_kernel(TrialArgs a) {
  const int lane = threadIdx.x & 63;
  const int trial = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (trial >= a.trials) return;  // whole wave
  const uint64_t ctr = a.counter0 + (uint64_t)trial;
  const Rng rng{(uint32_t)a.seed, (uint32_t)(a.seed >> 32), (uint32_t)ctr, (uint32_t)((ctr >> 32) << 8)};
  int cur = -1, lv = 0, f = 0, n_out = 0, bonus = 0;
  for (;;) {
    const int r = cur + 1;
    const float* p = a.P + (size_t)r * a.ldp;
    const float* q = a.Q + (size_t)r * a.ldq;
    const int* cs = a.cols + a.off[r];
    const int ns = a.off[r + 1] - a.off[r];
    int rej[SMP_MAXK];
    float zr[SMP_MAXK + 1], zq[SMP_MAXK + 1];
    zr[0] = 0.f;
    zq[0] = 1.f;
    int j = 0, chosen = -1;
    if (lv < a.depth) {
      const int k = a.branch[lv];
      // q0's mass and support count, then min(k, support) children by Gumbel top-k
      double s0 = 0.0;
      int supp = 0;
      for (int e = lane; e < ns; e += 64) {
        const float qv = q[cs[e]];
        s0 += (double)qv;
        supp += qv > 0.f;
      }
      s0 = wave_sum_d(s0);
      supp = wave_sum_i(supp);
      int take = min(k, supp);
      int tok[SMP_MAXK];
      for (int c = 0; c < take; ++c) {
        float bk = -1.f;
        int bi = NO_IDX;
        for (int e = lane; e < ns; e += 64) {
          const int y = cs[e];
          const float qv = q[y];
          if (!(qv > 0.f)) continue;
          bool taken = false;
          for (int u = 0; u < c; ++u) taken |= tok[u] == y;
          if (taken) continue;
          const U4 rb = rng_block(rng, (uint32_t)(y >> 2), (uint32_t)f | ((uint32_t)lv << 16), TAG_PROPOSE);
          const float key = qv / exp1_from_bits(u4_get(rb, y & 3));
          if (better(key, y, bk, bi)) {
            bk = key;
            bi = y;
          }
        }
        const KeyIdx w = wave_argmax(bk, bi);
        if (w.idx == NO_IDX) {  // no candidate left (cannot happen below the support count)
          take = c;
          break;
        }
        tok[c] = w.idx;
      }
      // the walk over the children in draw order (sample_walk_kernel)
      double zqd = s0;
      for (int i = 0; i < take; ++i) {
        const int x = tok[i];
        const float q0x = q[x];
        const float pj = chain_p(p[x], q0x, x, j, zr, zq, rej);
        const float qj = j == 0 ? q0x : q0x / zq[j];
        const double u = uniform_from_bits(rng_block(rng, (uint32_t)j, (uint32_t)r, TAG_ACCEPT).x);
        if (u < (double)fminf(1.f, pj / qj)) {
          chosen = i;
          break;
        }
        rej[j] = x;
        ++j;
        zqd -= (double)q0x;
        zq[j] = (float)zqd;
        // residual mass of state j (statej_kernel with its first j children rejected)
        double z = 0.0;
        for (int e = lane; e < ns; e += 64) {
          const int y = cs[e];
          const float pprev = chain_p(p[y], q[y], y, j - 1, zr, zq, rej);
          z += (double)fmaxf(pprev - trial_qprev(q[y], y, j, zq, rej), 0.f);
        }
        z = wave_sum_d(z);
        zr[j] = z > 0.0 ? (float)z : 0.f;
        if (j >= supp) break;  // no draft mass left
      }
      if (chosen >= 0) {
        const int fc = f * k + chosen;  // in-level index of the accepted child
        if (lane == 0) a.out_tok[(size_t)trial * (a.depth + 1) + n_out] = tok[chosen];
        ++n_out;
        cur = a.start[lv] + fc;
        f = fc;
        ++lv;
        continue;
      }
    }
    // bonus: the categorical draw from the last state with residual mass (state 0 at a leaf)
    int jj = j;
    while (jj > 0 && !(zr[jj] > 0.f)) --jj;
    float bk = -1.f;
    int bi = NO_IDX;
    for (int e = lane; e < ns; e += 64) {
      const int y = cs[e];
      float w;
      if (jj == 0) {
        w = p[y];
      } else {
        const float pprev = chain_p(p[y], q[y], y, jj - 1, zr, zq, rej);
        w = fmaxf(pprev - trial_qprev(q[y], y, jj, zq, rej), 0.f);
      }
      if (!(w > 0.f)) continue;
      const float key = w / exp1_from_bits(u4_get(rng_block(rng, (uint32_t)(y >> 2), 0u, TAG_BONUS), y & 3));
      if (better(key, y, bk, bi)) {
        bk = key;
        bi = y;
      }
    }
    const KeyIdx b = wave_argmax(bk, bi);
    bonus = b.idx == NO_IDX ? 0 : b.idx;
    break;
  }
  if (lane == 0) {
    a.out_tok[(size_t)trial * (a.depth + 1) + n_out] = bonus;
    a.out_n[trial] = n_out + 1;
  }
}

// ------------------------------------------------- top-64 draws (batched generation)
// sample_next of ssd/data/generate_selfdistill.py:50-60: the 64 largest logits of a row, the
// temperature + nucleus warp of those 64 alone, one categorical draw among them.
// Candidates are 64-bit records key << 32 | ~column (key = the bf16 logit's monotone key), so
// a larger record is a larger logit or, among equal logits, a lower column; 0 marks no entry.
constexpr int T64 = 64;
constexpr int T64_MAXC = 64;  // chunks per row (rows up to 262144 columns)

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int o) {
  const uint32_t lo = __shfl_xor((uint32_t)v, o), hi = __shfl_xor((uint32_t)(v >> 32), o);
  return ((uint64_t)hi << 32) | lo;
}

// Chunk pass: the chunk's min(64, columns) best records, sorted best first, into
// parts[row][chunk][64] (0-padded). The 64th-best key is found by two 256-bin count histograms
// (key high byte, then low byte inside the cut bin); the records above it are collected in any
// order, its ties by column rank (a block scan of per-thread tie counts: thread order is column
// order), then one wave sorts the 64 (bitonic network over the lanes).
__global__ __launch_bounds__(SMP_THREADS) void top64_chunk_kernel(const bf16_t* __restrict__ logits, int64_t ld,
                                                                  int n, int C, uint64_t* __restrict__ parts) {
  __shared__ uint32_t hist[256];
  __shared__ uint32_t red[16];
  __shared__ uint64_t list[T64];
  __shared__ uint32_t cut_sh, above_sh, cnt_sh;
  const int row = blockIdx.y, c = blockIdx.x, t = threadIdx.x;
  const int i = c * SMP_CHUNK + t * 4;
  uint32_t h[4], k[4];
  load4_bf16(logits + (size_t)row * ld, i, n, h);
#pragma unroll
  for (int e = 0; e < 4; ++e) k[e] = bf_key(h[e]);
  const uint32_t want = (uint32_t)min(T64, n - c * SMP_CHUNK);
  if (t < 256) hist[t] = 0;
  if (t == 0) cnt_sh = 0;
  __syncthreads();
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (i + e < n) atomicAdd(&hist[k[e] >> 8], 1u);
  __syncthreads();
  // bins from the largest key down: the bin holding the want-th record
  uint32_t hv = t < 256 ? hist[255 - t] : 0u;
  uint32_t incl = block_scan(hv, red);
  if (t < 256 && hv > 0 && incl - hv < want && incl >= want) {
    cut_sh = 255u - (uint32_t)t;
    above_sh = incl - hv;
  }
  __syncthreads();
  const uint32_t cb = cut_sh, above1 = above_sh;
  if (t < 256) hist[t] = 0;
  __syncthreads();
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (i + e < n && (k[e] >> 8) == cb) atomicAdd(&hist[k[e] & 255u], 1u);
  __syncthreads();
  hv = t < 256 ? hist[255 - t] : 0u;
  incl = above1 + block_scan(hv, red);
  __syncthreads();
  if (t < 256 && hv > 0 && incl - hv < want && incl >= want) {
    cut_sh = (cb << 8) | (255u - (uint32_t)t);
    above_sh = incl - hv;
  }
  __syncthreads();
  const uint32_t ck = cut_sh, above = above_sh, ties_keep = want - above;
  uint32_t nt = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) nt += (i + e < n && k[e] == ck) ? 1u : 0u;
  uint32_t rank = block_scan(nt, red) - nt;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if (i + e >= n) continue;
    const uint64_t rec = ((uint64_t)k[e] << 32) | (uint32_t)~(uint32_t)(i + e);
    if (k[e] > ck) {
      list[atomicAdd(&cnt_sh, 1u)] = rec;  // exactly `above` of these
    } else if (k[e] == ck) {
      if (rank < ties_keep) list[above + rank] = rec;
      ++rank;
    }
  }
  __syncthreads();
  if (t < T64) {
    uint64_t x = (uint32_t)t < want ? list[t] : 0ull;
#pragma unroll
    for (int size = 2; size <= T64; size <<= 1) {
#pragma unroll
      for (int stride = size >> 1; stride > 0; stride >>= 1) {
        const uint64_t y = shfl_xor_u64(x, stride);
        const bool desc = (t & size) == 0, lo = (t & stride) == 0;
        x = (lo == desc) ? (x > y ? x : y) : (x < y ? x : y);
      }
    }
    parts[((size_t)row * C + c) * T64 + t] = x;
  }
}

// Merge + warp + draw, one wave per row: the 64 best of the chunk lists (lane c walks list c;
// each round takes the wave's largest head), then in rank order p = softmax(v / T), the
// nucleus cut of warp_probs (an entry is dropped when the sequential fp32 cumulative mass before
// it exceeds top_p; none with top_p >= 1) and a Gumbel-max draw over the kept ranks, Exp(1) of
// rank j from the draw stream (counter (j / 4, row), tag TAG_TOP64).
__global__ __launch_bounds__(64) void top64_draw_kernel(const uint64_t* __restrict__ parts, int C, float temp,
                                                        float top_p, Rng rng, int* __restrict__ out_tok) {
  __shared__ uint64_t L[T64_MAXC * T64];
  const int row = blockIdx.x, lane = threadIdx.x;
  const uint64_t* P = parts + (size_t)row * C * T64;
  for (int j = lane; j < C * T64; j += 64) L[j] = P[j];
  __syncthreads();
  int head = 0;
  uint64_t cur = lane < C ? L[lane * T64] : 0ull, mine = 0ull;
  for (int r = 0; r < T64; ++r) {
    uint64_t best = cur;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint64_t y = shfl_xor_u64(best, o);
      best = y > best ? y : best;
    }
    if (r == lane) mine = best;
    if (best != 0ull && cur == best) {  // records are distinct: exactly one lane advances
      ++head;
      cur = head < T64 ? L[lane * T64 + head] : 0ull;
    }
  }
  const bool has = mine != 0ull;
  const float x = has ? bf2f((bf16_t)key_bf((uint32_t)(mine >> 32))) / temp : -INFINITY;
  const float M = __shfl(x, 0);  // rank 0 holds the largest logit
  const float e = has ? expf(x - M) : 0.f;
  float S = e;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) S += __shfl_xor(S, o);
  const float p = e / S;
  float acc = 0.f, cum = 0.f;
  for (int j = 0; j < 64; ++j) {  // torch.cumsum order: rank 0 first
    acc += __shfl(p, j);
    if (j == lane) cum = acc;
  }
  const bool keep = has && p > 0.f && (top_p >= 1.f || !(cum - p > top_p));
  const U4 rb = rng_block(rng, (uint32_t)(lane >> 2), (uint32_t)row, TAG_TOP64);
  const float key = keep ? p / exp1_from_bits(u4_get(rb, lane & 3)) : -1.f;
  const KeyIdx w = wave_argmax(key, lane);
  const int col = (int)~(uint32_t)mine;
  const int pick = __shfl(col, w.idx == NO_IDX ? 0 : w.idx);
  if (lane == 0) out_tok[row] = pick;
}

}  // namespace ssd

using namespace ssd;

SSD_API int ssd_sample_limits(int32_t* out2) {
  if (!out2) return set_error(SSD_EINVAL, "sample_limits: null");
  out2[0] = SMP_MAXK;
  out2[1] = SMP_CHUNK * SMP_MAXC;
  return SSD_OK;
}

SSD_API int64_t ssd_sample_ws_bytes(int rows, int n) {
  if (rows < 0 || n <= 0 || chunks_of(n) > SMP_MAXC) return -1;
  return smp_layout(rows, chunks_of(n), nullptr, nullptr);
}

static int carve(void* ws, int64_t ws_bytes, int rows, int n, SmpWs* out, const char* what) {
  const int64_t need = ssd_sample_ws_bytes(rows, n);
  if (need < 0) return set_error(SSD_ERANGE, "%s: %d columns > %d", what, n, SMP_CHUNK * SMP_MAXC);
  if (!ws || ws_bytes < need)
    return set_error(SSD_EINVAL, "%s: workspace %lld < %lld bytes", what, (long long)ws_bytes, (long long)need);
  smp_layout(rows, chunks_of(n), (char*)ws, out);
  return SSD_OK;
}

SSD_API int ssd_warp_probs_bf16(const uint16_t* logits, int64_t ld, int rows, int n, const int32_t* vocab_ids,
                                const int32_t* vocab_inv, int V, float temperature, float top_p,
                                const int32_t* tree_meta, int level, float* probs, int64_t ldp, void* ws,
                                int64_t ws_bytes, hipStream_t stream) {
  if (!logits || !probs || (vocab_ids && !vocab_inv)) return set_error(SSD_EINVAL, "warp_probs: null pointer");
  if (rows < 0 || n <= 0 || V <= 0 || (!vocab_ids && n != V) || n > V)
    return set_error(SSD_EINVAL, "warp_probs: bad shape rows=%d n=%d V=%d", rows, n, V);
  if (ld % 4 || ld < (n + 3) / 4 * 4 || ldp % 4 || ldp < V)
    return set_error(SSD_EINVAL, "warp_probs: ld %lld / ldp %lld must be multiples of 4 covering the row",
                     (long long)ld, (long long)ldp);
  if (!(temperature > 0.f)) return set_error(SSD_EINVAL, "warp_probs: temperature must be > 0");
  if (tree_meta && (level < 0 || level >= SMP_MAXDEPTH)) return set_error(SSD_ERANGE, "warp_probs: level %d", level);
  if (rows > 65535) return set_error(SSD_ERANGE, "warp_probs: %d rows", rows);
  if (rows == 0) return SSD_OK;
  SmpWs w;
  if (int rc = carve(ws, ws_bytes, rows, V, &w, "warp_probs")) return rc;
  const int C = chunks_of(n), CV = chunks_of(V);
  w.C = C;  // stats / histograms are per logit chunk (the layout was sized for V >= n chunks)
  const double tp = top_p < 0.f ? 0.0 : (double)top_p;
  WarpArgs a{logits, ld, rows, n, vocab_ids, vocab_inv, V, temperature, top_p,
             (uint64_t)fmin(tp * 0x1p52, 0x1p63), tree_meta, level, probs, ldp, w};
  SSD_LAUNCH(warp_stats_kernel, dim3(C, rows), dim3(SMP_THREADS), 0, stream, a);
  if (top_p < 1.f) {
    SSD_LAUNCH(warp_coarse_kernel, dim3(C, rows), dim3(SMP_THREADS), 0, stream, a);
    SSD_LAUNCH(warp_fine_kernel, dim3(C, rows), dim3(SMP_THREADS), 0, stream, a);
  }
  SSD_LAUNCH(warp_final_kernel, dim3(vocab_ids ? max(C, CV) : C, rows), dim3(SMP_THREADS), 0, stream, a);
  return check_launch("warp_probs");
}

SSD_API int ssd_gumbel_topk(const float* probs, int64_t ldp, int rows, int V, int k, const int32_t* tree_meta,
                            int level, uint64_t seed, uint64_t counter, int32_t* out_tok, float* out_lp, void* ws,
                            int64_t ws_bytes, hipStream_t stream) {
  if (!probs || !out_tok || !out_lp) return set_error(SSD_EINVAL, "gumbel_topk: null pointer");
  if (rows < 0 || V <= 0 || ldp % 4 || ldp < V) return set_error(SSD_EINVAL, "gumbel_topk: bad shape");
  if (k < 1 || k > SMP_MAXK) return set_error(SSD_ERANGE, "gumbel_topk: k=%d not in [1, %d]", k, SMP_MAXK);
  if (tree_meta && (level < 0 || level >= SMP_MAXDEPTH)) return set_error(SSD_ERANGE, "gumbel_topk: level %d", level);
  if (rows > 65535) return set_error(SSD_ERANGE, "gumbel_topk: %d rows", rows);
  if (rows == 0) return SSD_OK;
  SmpWs w;
  if (int rc = carve(ws, ws_bytes, rows, V, &w, "gumbel_topk")) return rc;
  TopkArgs a{probs, ldp, rows, V, k, tree_meta, level, make_rng(seed, counter), out_tok, out_lp, w};
  SSD_LAUNCH(gumbel_chunk_kernel, dim3(w.C, rows), dim3(SMP_THREADS), 0, stream, a);
  SSD_LAUNCH(gumbel_merge_kernel, dim3(rows), dim3(SMP_THREADS), 0, stream, a);
  return check_launch("gumbel_topk");
}

SSD_API int ssd_sample_rows(const float* probs, int64_t ldp, int rows, int V, uint64_t seed, uint64_t counter,
                            int32_t* out_tok, void* ws, int64_t ws_bytes, hipStream_t stream) {
  if (!probs || !out_tok) return set_error(SSD_EINVAL, "sample_rows: null pointer");
  if (rows < 0 || V <= 0 || ldp % 4 || ldp < V) return set_error(SSD_EINVAL, "sample_rows: bad shape");
  if (rows > 65535) return set_error(SSD_ERANGE, "sample_rows: %d rows", rows);
  if (rows == 0) return SSD_OK;
  SmpWs w;
  if (int rc = carve(ws, ws_bytes, rows, V, &w, "sample_rows")) return rc;
  SSD_LAUNCH(draw_chunk_kernel, dim3(w.C, rows), dim3(SMP_THREADS), 0, stream, probs, ldp, V,
                     make_rng(seed, counter), w);
  SSD_LAUNCH(draw_merge_kernel, dim3((rows + 63) / 64), dim3(64), 0, stream, rows, w, out_tok);
  return check_launch("sample_rows");
}

SSD_API int64_t ssd_sample_top64_ws_bytes(int rows, int V) {
  if (rows < 0 || V < T64 || chunks_of(V) > T64_MAXC) return -1;
  return (int64_t)rows * chunks_of(V) * T64 * (int64_t)sizeof(uint64_t);
}

SSD_API int ssd_sample_top64_bf16(const uint16_t* logits, int64_t ld, int rows, int V, float temperature, float top_p,
                                  uint64_t seed, uint64_t counter, int32_t* out_tok, void* ws, int64_t ws_bytes,
                                  hipStream_t stream) {
  if (!logits || !out_tok) return set_error(SSD_EINVAL, "sample_top64: null pointer");
  if (rows < 0 || V < T64 || chunks_of(V) > T64_MAXC)
    return set_error(SSD_ERANGE, "sample_top64: V=%d outside [%d, %d]", V, T64, SMP_CHUNK * T64_MAXC);
  if (ld % 4 || ld < (V + 3) / 4 * 4)
    return set_error(SSD_EINVAL, "sample_top64: ld %lld must be a multiple of 4 covering the row", (long long)ld);
  if (!(temperature > 0.f) || !(top_p > 0.f))
    return set_error(SSD_EINVAL, "sample_top64: temperature and top_p must be > 0");
  if (rows > 65535) return set_error(SSD_ERANGE, "sample_top64: %d rows", rows);
  if (rows == 0) return SSD_OK;
  const int64_t need = ssd_sample_top64_ws_bytes(rows, V);
  if (!ws || ws_bytes < need || ((uintptr_t)ws & 7))
    return set_error(SSD_EINVAL, "sample_top64: workspace %lld < %lld bytes or misaligned", (long long)ws_bytes,
                     (long long)need);
  const int C = chunks_of(V);
  SSD_LAUNCH(top64_chunk_kernel, dim3(C, rows), dim3(SMP_THREADS), 0, stream, (const bf16_t*)logits, ld, V, C,
             (uint64_t*)ws);
  SSD_LAUNCH(top64_draw_kernel, dim3(rows), dim3(64), 0, stream, (const uint64_t*)ws, C, temperature, top_p,
             make_rng(seed, counter), out_tok);
  return check_launch("sample_top64");
}

SSD_API int ssd_accept_sample(const SsdTree* tree, const float* P, int64_t ldp, const float* Q, int64_t ldq, int V,
                              int rows, int max_kids, uint64_t seed, uint64_t counter, void* ws, int64_t ws_bytes,
                              int committed, int32_t* result, int32_t* keep_src, int32_t* n_keep,
                              int32_t* root_token, hipStream_t stream) {
  if (!tree || !P || !Q || !result || !keep_src || !n_keep || !root_token)
    return set_error(SSD_EINVAL, "accept_sample: null pointer");
  if (V <= 0 || ldp % 4 || ldq % 4 || ldp < V || ldq < V || rows < 1 || rows > 64)
    return set_error(SSD_EINVAL, "accept_sample: bad shape (rows %d must be in [1, 64])", rows);
  if (max_kids < 0 || max_kids > SMP_MAXK)
    return set_error(SSD_ERANGE, "accept_sample: max_kids %d not in [0, %d]", max_kids, SMP_MAXK);
  SmpWs w;
  if (int rc = carve(ws, ws_bytes, rows, V, &w, "accept_sample")) return rc;
  AcceptArgs a{*tree, P, ldp, Q, ldq, V, rows, max_kids, make_rng(seed, counter), w};
  SSD_LAUNCH(state0_kernel, dim3(w.C, rows), dim3(SMP_THREADS), 0, stream, a);
  for (int j = 1; j <= max_kids; ++j)
    SSD_LAUNCH(statej_kernel, dim3(w.C, rows), dim3(SMP_THREADS), 0, stream, a, j);
  SSD_LAUNCH(sample_walk_kernel, dim3(1), dim3(64), 0, stream, a, committed, result, keep_src, n_keep,
                     root_token);
  return check_launch("accept_sample");
}

// Batched acceptance trials (accept_trials_kernel): trials independent rounds over fixed per-node
// distributions P/Q ([rows][ld] fp32, rows >= 1 + nodes of the unpruned tree given by branch[0 ..
// depth)), support lists cols/col_off (CSR over rows: ascending columns where P or Q > 0).
SSD_API int ssd_accept_sample_trials(const float* P, int64_t ldp, const float* Q, int64_t ldq, int rows,
                                     const int32_t* cols, const int32_t* col_off, int depth, const int32_t* branch,
                                     uint64_t seed, uint64_t counter0, int trials, int32_t* out_tokens,
                                     int32_t* out_n, hipStream_t stream) {
  if (!P || !Q || !cols || !col_off || !branch || !out_tokens || !out_n)
    return set_error(SSD_EINVAL, "accept_trials: null pointer");
  if (depth < 1 || depth > TRIAL_MAXD) return set_error(SSD_ERANGE, "accept_trials: depth %d not in [1, %d]", depth, TRIAL_MAXD);
  if (trials < 0 || ldp % 4 || ldq % 4 || rows < 1) return set_error(SSD_EINVAL, "accept_trials: bad shape");
  TrialArgs a{};
  a.P = P; a.ldp = ldp; a.Q = Q; a.ldq = ldq; a.cols = cols; a.off = col_off; a.depth = depth;
  int64_t level = 1, nodes = 0;
  for (int d = 0; d < depth; ++d) {
    if (branch[d] < 1 || branch[d] > SMP_MAXK)
      return set_error(SSD_ERANGE, "accept_trials: branch[%d]=%d not in [1, %d]", d, branch[d], SMP_MAXK);
    a.branch[d] = branch[d];
    a.start[d] = (int)nodes;
    level *= branch[d];
    nodes += level;
    if (nodes > (1 << 20)) return set_error(SSD_ERANGE, "accept_trials: tree too large");
  }
  a.start[depth] = (int)nodes;
  if (rows < 1 + nodes) return set_error(SSD_EINVAL, "accept_trials: %d rows for a tree of %lld nodes", rows, (long long)nodes);
  a.seed = seed; a.counter0 = counter0; a.trials = trials; a.out_tok = out_tokens; a.out_n = out_n;
  if (trials == 0) return SSD_OK;
  SSD_LAUNCH(accept_trials_kernel, dim3((trials + 3) / 4), dim3(256), 0, stream, a);
  return check_launch("accept_trials");
}

