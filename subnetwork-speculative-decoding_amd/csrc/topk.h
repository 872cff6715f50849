// Row top-k over a vocabulary in two passes, shared by the top-k entry points (rows.hip) and the
// level expansion that merges its candidates itself (tree.hip): a partial pass keeps the k best
// (value, column) keys and the max / sum of exp of each 4096-column chunk (TopkPart), and a merge
// takes a row's k best over its chunks.
#pragma once

#include "common.h"

#include <math.h>

namespace ssd {

constexpr int TOPK_MAX = 16;
constexpr int TOPK_CHUNK = 4096;  // columns per partial workgroup: 256 threads x 16 columns
constexpr int TOPK_PER = TOPK_CHUNK / 256;

// Ranking key of a (value, column) pair: a larger key ranks first, i.e. larger value, then
// lower column (the oracle's stable-sort order). The value maps to its order-preserving
// unsigned image; NaN ranks below every number; key 0 is "no candidate".
__device__ __forceinline__ uint64_t rank_key(float v, int col) {
  uint32_t b = __float_as_uint(v);
  b = (v != v) ? 0u : ((b & 0x80000000u) ? ~b : (b | 0x80000000u));
  return ((uint64_t)b << 32) | (uint32_t)(~(uint32_t)col);
}
__device__ __forceinline__ float key_value(uint64_t key) {
  const uint32_t b = (uint32_t)(key >> 32);
  return __uint_as_float((b & 0x80000000u) ? (b & 0x7fffffffu) : ~b);
}
__device__ __forceinline__ int key_col(uint64_t key) { return (int)~(uint32_t)key; }

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const uint32_t lo = __shfl_xor((uint32_t)v, off), hi = __shfl_xor((uint32_t)(v >> 32), off);
    const uint64_t o = ((uint64_t)hi << 32) | lo;
    v = o > v ? o : v;
  }
  return v;
}

struct TopkPart {
  float mx;  // chunk maximum
  float se;  // sum of exp(x - mx) over the chunk (mode 1)
  uint64_t key[TOPK_MAX];  // the chunk's k best, best first
};

// Records are stored packed for the k of the call: 8 + 8 k bytes each (the maximum, the sum of exp,
// then the k keys, 8-byte aligned), so a merge reads the bytes it uses (32 B a record at k = 3
// instead of a 136-byte TopkPart's line). Buffers stay sized for sizeof(TopkPart) records, which
// covers every k <= TOPK_MAX.
struct TopkRec {
  float* mx;
  float* se;
  uint64_t* key;
};
__device__ __forceinline__ TopkRec topk_rec(void* parts, size_t idx, int k) {
  char* r = (char*)parts + idx * (size_t)(8 + 8 * k);
  return TopkRec{(float*)r, (float*)r + 1, (uint64_t*)(r + 8)};
}
__device__ __forceinline__ TopkRec topk_rec(const void* parts, size_t idx, int k) {
  return topk_rec(const_cast<void*>(parts), idx, k);
}

constexpr int TOPK_MAX_PARTS = 256;  // records per row a merge takes (S * k <= 64 * TOPK_MAX as well)

// Merge of one row's S <= 256 partial records (each the k best keys and the max / sum of exp of a
// disjoint column range) by one wave: global max M; logsumexp = M + log(sum_s se_s exp(mx_s - M))
// (lane l sums its records l, l + 64, ... in that order, then a fixed butterfly); the k best of
// the S*k keys, held in registers (lane l: candidates l + 64*j, S*k <= 64 * TOPK_MAX), in k rounds
// of a wave maximum. Lane 0 writes token q (vocab_ids[column] when vocab_ids is set) to tok[q]
// and, when val is set, its value to val[q]: mode 0 the raw value, mode 1 the log-softmax value
// (x - M) - log(sum); lse (mode 1, when set) gets M + log(sum).
__device__ __forceinline__ void topk_merge_row(const void* __restrict__ p, int S, int k, int mode,
                                               const int* __restrict__ vocab_ids, int lane, int* tok, float* val,
                                               float* lse_out) {
  // Every load is issued up front from a clamped index (one memory round trip instead of one per
  // step); values past S and past S*k are masked afterwards.
  const int total = S * k;  // <= 64 * TOPK_MAX
  constexpr int PER = TOPK_MAX_PARTS / 64;
  float mx_o[PER], se_o[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const TopkRec own = topk_rec(p, min(lane + 64 * i, S - 1), k);
    mx_o[i] = *own.mx;
    se_o[i] = *own.se;
  }
  uint64_t key[TOPK_MAX];
#pragma unroll
  for (int j = 0; j < TOPK_MAX; ++j) {
    const int c = min(lane + 64 * j, total - 1);
    key[j] = topk_rec(p, c / k, k).key[c % k];
  }
#pragma unroll
  for (int j = 0; j < TOPK_MAX; ++j)
    if (lane + 64 * j >= total) key[j] = 0ull;
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < PER; ++i)
    if (lane + 64 * i < S) mx = fmaxf(mx, mx_o[i]);
  for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
  float lse = 0.f;
  if (mode == 1) {
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < PER; ++i)
      if (lane + 64 * i < S) acc += se_o[i] * __expf(mx_o[i] - mx);
    for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off);
    lse = logf(acc);
  }
  uint32_t taken = 0;
  for (int q = 0; q < k; ++q) {
    uint64_t b = 0;
    int bj = -1;
#pragma unroll
    for (int j = 0; j < TOPK_MAX; ++j)
      if (!((taken >> j) & 1u) && key[j] > b) { b = key[j]; bj = j; }
    const uint64_t m = wave_max_u64(b);
    if (bj >= 0 && b == m) taken |= 1u << bj;
    if (lane == 0) {
      const int col = key_col(m);
      const float v = key_value(m);
      tok[q] = vocab_ids ? vocab_ids[col] : col;
      if (val) val[q] = mode == 1 ? (v - mx) - lse : v;
    }
  }
  if (lane == 0 && mode == 1 && lse_out) *lse_out = mx + lse;
}

}  // namespace ssd
