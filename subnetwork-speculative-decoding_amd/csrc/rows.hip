// Row kernels: RMSNorm, embedding gather, KV compaction, and the vocabulary
// reductions that close the lm_head (argmax / log-softmax top-k).
//
// Every reduction runs in a fixed order that depends only on the row length,
// so each row's result is independent of how many rows share the launch.
#include "common.h"
#include "topk.h"

#include <math.h>

#include <mutex>

namespace ssd {

// Deterministic 256-thread sum: butterfly inside each wave, then waves in order.
__device__ __forceinline__ float block_sum_256(float v, float* sh) {
  v += __shfl_xor(v, 1);
  v += __shfl_xor(v, 2);
  v += __shfl_xor(v, 4);
  v += __shfl_xor(v, 8);
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  const float r = ((sh[0] + sh[1]) + sh[2]) + sh[3];
  __syncthreads();
  return r;
}

// HF LlamaRMSNorm / bridge RMSNorm: y = w * bf16(x * rsqrt(mean(x^2) + eps)) (ssd/models/bridges.py:33-37).
__global__ __launch_bounds__(256) void rmsnorm_kernel(const bf16_t* __restrict__ x, int64_t ldx,
                                                      const bf16_t* __restrict__ w, bf16_t* __restrict__ y,
                                                      int64_t ldy, int D, float eps) {
  __shared__ float sh[4];
  const bf16_t* xr = x + (size_t)blockIdx.x * ldx;
  bf16_t* yr = y + (size_t)blockIdx.x * ldy;
  float ss = 0.f;
  for (int k = threadIdx.x * 8; k < D; k += 256 * 8) {
    Pack8 p;
    p.u = *(const uint4*)(xr + k);
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const float f = bf2f(p.h[t]);
      ss += f * f;
    }
  }
  const float tot = block_sum_256(ss, sh);
  const float r = rsqrtf(tot / (float)D + eps);
  for (int k = threadIdx.x * 8; k < D; k += 256 * 8) {
    Pack8 p, q, o;
    p.u = *(const uint4*)(xr + k);
    q.u = *(const uint4*)(w + k);
#pragma unroll
    for (int t = 0; t < 8; ++t) o.h[t] = f2bf(bf2f(q.h[t]) * rbf(bf2f(p.h[t]) * r));
    *(uint4*)(yr + k) = o.u;
  }
}

// Deterministic 1024-thread sum: butterfly inside each wave, then the 16 wave sums in order.
__device__ __forceinline__ float block_sum_1024(float v, float* sh) {
  v += __shfl_xor(v, 1);
  v += __shfl_xor(v, 2);
  v += __shfl_xor(v, 4);
  v += __shfl_xor(v, 8);
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = sh[0];
#pragma unroll
  for (int i = 1; i < 16; ++i) r += sh[i];
  __syncthreads();
  return r;
}

// Residual update from split-K partials, then RMSNorm of the new residual:
//   h <- bf16(h + bf16(sum_s P[s] + bias));  y <- w * bf16(h * rsqrt(mean(h^2) + eps))
// (the o_proj / down_proj / bridge out_proj residual add of the reference, followed by the next
// RMSNorm; ssd/models/subnetwork_draft.py:243-245, ssd/models/bridges.py:131-135). One 1024-thread
// workgroup per row, 4 columns per thread per pass; the S partials (a template constant, loads
// issued together) are summed in order s = 0..S-1. S = 0: y = RMSNorm(h) only.
template <int S>
__global__ __launch_bounds__(1024) void add_rmsnorm_kernel(const float* __restrict__ P, int64_t ldp, int64_t sstride,
                                                           const bf16_t* __restrict__ bias, bf16_t* __restrict__ h,
                                                           int64_t ldh, const bf16_t* __restrict__ w,
                                                           bf16_t* __restrict__ y, int64_t ldy, int D, float eps) {
  __shared__ float sh[16];
  const int m = blockIdx.x;
  bf16_t* hr = h + (size_t)m * ldh;
  float ss = 0.f;
  for (int k = threadIdx.x * 4; k < D; k += 1024 * 4) {
    const uint2 hv = *(const uint2*)(hr + k);
    float v[4] = {bf2f((bf16_t)(hv.x & 0xffff)), bf2f((bf16_t)(hv.x >> 16)), bf2f((bf16_t)(hv.y & 0xffff)),
                  bf2f((bf16_t)(hv.y >> 16))};
    if constexpr (S > 0) {
      const float* pr = P + (size_t)m * ldp + k;
      f32x4_t part[S];
#pragma unroll
      for (int s = 0; s < S; ++s) part[s] = *(const f32x4_t*)(pr + s * sstride);
      f32x4_t o = part[0];
#pragma unroll
      for (int s = 1; s < S; ++s) o += part[s];
      float bv[4] = {0.f, 0.f, 0.f, 0.f};
      if (bias) {
        const uint2 b = *(const uint2*)(bias + k);
        bv[0] = bf2f((bf16_t)(b.x & 0xffff)); bv[1] = bf2f((bf16_t)(b.x >> 16));
        bv[2] = bf2f((bf16_t)(b.y & 0xffff)); bv[3] = bf2f((bf16_t)(b.y >> 16));
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) v[t] = rbf(v[t] + rbf(bias ? o[t] + bv[t] : o[t]));
      *(uint2*)(hr + k) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) ss += v[t] * v[t];
  }
  const float tot = block_sum_1024(ss, sh);
  if (!y) return;
  const float r = rsqrtf(tot / (float)D + eps);
  bf16_t* yr = y + (size_t)m * ldy;
  for (int k = threadIdx.x * 4; k < D; k += 1024 * 4) {
    const uint2 hv = *(const uint2*)(hr + k), wv = *(const uint2*)(w + k);
    const uint32_t hw[2] = {hv.x, hv.y}, ww[2] = {wv.x, wv.y};
    uint32_t o[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const float a0 = bf2f((bf16_t)(ww[q] & 0xffff)) * rbf(bf2f((bf16_t)(hw[q] & 0xffff)) * r);
      const float a1 = bf2f((bf16_t)(ww[q] >> 16)) * rbf(bf2f((bf16_t)(hw[q] >> 16)) * r);
      o[q] = pack_bf16x2(a0, a1);
    }
    *(uint2*)(yr + k) = make_uint2(o[0], o[1]);
  }
}

__global__ __launch_bounds__(256) void embed_kernel(const int* __restrict__ ids, const bf16_t* __restrict__ table,
                                                    int64_t V, int D, bf16_t* __restrict__ out, int64_t ldo) {
  const int m = blockIdx.x;
  int id = ids[m];
  id = id < 0 ? 0 : (id >= V ? (int)V - 1 : id);
  const uint4* src = (const uint4*)(table + (size_t)id * D);
  uint4* dst = (uint4*)(out + (size_t)m * ldo);
  for (int k = threadIdx.x; k < D / 8; k += 256) dst[k] = src[k];
}

// Move cache entries src[0..n) to [start, start+n) in every layer and kv head
// (ssd/engine/kv_cache.py:54-70), in 16-byte runs. All sources are read before any destination
// is written: a destination may be the source of a later entry (start=10, src=[10,12,13]).
// Every (layer, kv head) holds max_len slots of K and of V in the 64-slot block layout (k_off,
// v_off in common.h). K: each entry is hd/8 runs of 8 dims (contiguous in the layout), copied
// whole. V: the layout keeps 8 consecutive slots of one dim together, so each 16-byte run of
// the destination range's 8-slot groups is read, the moved entries are put into it, and it is
// written back whole. n is read from device memory (n_ptr) so the launch needs no host round
// trip; n <= n_max. An out-of-range source leaves its slot as it is.
__global__ __launch_bounds__(256) void kv_compact_kernel(bf16_t* __restrict__ kc, bf16_t* __restrict__ vt, int kv_heads,
                                                         int hd, int64_t max_len, int start, const int* __restrict__ src,
                                                         const int* __restrict__ n_ptr, int n_max,
                                                         const int* __restrict__ pos_base) {
  extern __shared__ u32x4_t stage16[];  // K runs [n_max][hd / 8], then V runs [groups][hd]
  const int lh = blockIdx.x;            // layer * kv_heads + head
  if (pos_base) start += *pos_base;
  // a destination range outside the cache moves nothing (the host checks absolute starts itself)
  const int n = (start < 0 || start + n_max > max_len) ? 0 : max(0, min(*n_ptr, n_max));
  bf16_t* kbase = kc + (size_t)lh * max_len * hd;
  bf16_t* vbase = vt + (size_t)lh * hd * max_len;
  const int hq = hd >> 3;
  const int g0 = start >> 3, ng = n > 0 ? ((start + n + 7) >> 3) - g0 : 0;
  u32x4_t* kst = stage16;
  u32x4_t* vst = stage16 + (size_t)n_max * hq;
  auto src_of = [&](int i) {
    const int s = src[i];
    return (s >= 0 && s < max_len) ? s : start + i;
  };
  for (int e = threadIdx.x; e < n * hq; e += 256) {
    const int i = e / hq, q = e - i * hq;
    kst[e] = *(const u32x4_t*)(kbase + k_off(src_of(i), q * 8, hd));
  }
  for (int e = threadIdx.x; e < ng * hd; e += 256) {
    const int g = e / hd, d = e - g * hd;
    const int s0 = (g0 + g) * 8;
    u32x4_t run = *(const u32x4_t*)(vbase + v_off(s0, d, hd));
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int i = s0 + t - start;
      if (i >= 0 && i < n) {
        const uint32_t h = (uint32_t)vbase[v_off(src_of(i), d, hd)];
        const int w = t >> 1;
        run[w] = (t & 1) ? ((run[w] & 0x0000ffffu) | (h << 16)) : ((run[w] & 0xffff0000u) | h);
      }
    }
    vst[e] = run;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < n * hq; e += 256) {
    const int i = e / hq, q = e - i * hq;
    *(u32x4_t*)(kbase + k_off(start + i, q * 8, hd)) = kst[e];
  }
  for (int e = threadIdx.x; e < ng * hd; e += 256) {
    const int g = e / hd, d = e - g * hd;
    *(u32x4_t*)(vbase + v_off((g0 + g) * 8, d, hd)) = vst[e];
  }
}

// Partial pass: workgroup (s, row) holds columns [s*4096, (s+1)*4096) of one row of bf16 logits
// in registers (thread t: columns t*8 + [0, 8) and 2048 + t*8 + [0, 8) of the chunk) and takes
// its k best keys in k rounds of a block-wide maximum, each round retiring the winner; it also
// writes the chunk maximum and (mode 1) the sum of exp(x - max).
__global__ __launch_bounds__(256) void row_topk_partial_kernel(const bf16_t* __restrict__ logits, int64_t ld, int N,
                                                               int k, int mode, TopkPart* __restrict__ parts) {
  __shared__ uint64_t wbest[2][4];
  __shared__ float sh[4];
  const int s = blockIdx.x, row = blockIdx.y, S = gridDim.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const bf16_t* x = logits + (size_t)row * ld;
  float val[TOPK_PER];
  uint64_t key[TOPK_PER];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int col = s * TOPK_CHUNK + h * 2048 + threadIdx.x * 8;
    Pack8 p;
    if (col + 8 <= N) {
      p.u = *(const uint4*)(x + col);
    } else {
#pragma unroll
      for (int t = 0; t < 8; ++t) p.h[t] = col + t < N ? x[col + t] : (bf16_t)0;
    }
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const bool ok = col + t < N;
      val[h * 8 + t] = ok ? bf2f(p.h[t]) : -INFINITY;
      key[h * 8 + t] = ok ? rank_key(val[h * 8 + t], col + t) : 0ull;
    }
  }
  const TopkRec out = topk_rec(parts, (size_t)row * S + s, k);
  uint32_t taken = 0;
  float mx = -INFINITY;
  for (int q = 0; q < k; ++q) {
    uint64_t b = 0;
    int bj = -1;
#pragma unroll
    for (int j = 0; j < TOPK_PER; ++j)
      if (!((taken >> j) & 1u) && key[j] > b) { b = key[j]; bj = j; }
    const uint64_t wm = wave_max_u64(b);
    if (lane == 0) wbest[q & 1][wave] = wm;
    __syncthreads();  // one barrier per round: rounds alternate between the two slots
    uint64_t m = wbest[q & 1][0];
#pragma unroll
    for (int w = 1; w < 4; ++w) m = wbest[q & 1][w] > m ? wbest[q & 1][w] : m;
    if (bj >= 0 && b == m) taken |= 1u << bj;  // keys are distinct: one thread retires it
    if (threadIdx.x == 0) out.key[q] = m;
    if (q == 0) mx = m ? key_value(m) : -INFINITY;
  }
  float se = 0.f;
  if (mode == 1) {
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < TOPK_PER; ++j) acc += __expf(val[j] - mx);
    se = block_sum_256(acc, sh);
  }
  if (threadIdx.x == 0) { *out.mx = mx; *out.se = se; }
}

// Merge pass, one wave per row (topk_merge_row).
__global__ __launch_bounds__(64) void row_topk_merge_kernel(const TopkPart* __restrict__ parts, int S, int k, int mode,
                                                            const int* __restrict__ vocab_ids, int* __restrict__ out_tok,
                                                            float* __restrict__ out_val, float* __restrict__ out_lse) {
  const int row = blockIdx.x;
  topk_merge_row((const char*)parts + (size_t)row * S * (size_t)(8 + 8 * k), S, k, mode, vocab_ids, threadIdx.x,
                 out_tok + row * k,
                 out_val ? out_val + row * k : nullptr, out_lse ? out_lse + row : nullptr);
}

}  // namespace ssd

using namespace ssd;

SSD_API int ssd_rmsnorm_bf16(const uint16_t* x, int64_t ldx, int M, int D, const uint16_t* w, float eps,
                             uint16_t* y, int64_t ldy, hipStream_t stream) {
  if (!x || !w || !y || M < 0 || D <= 0 || D % 8 || ldx % 8 || ldy % 8)
    return set_error(SSD_EINVAL, "rmsnorm: bad arguments (D=%d must be a multiple of 8)", D);
  if (M == 0) return SSD_OK;
  SSD_LAUNCH(rmsnorm_kernel, dim3(M), dim3(256), 0, stream, x, ldx, w, y, ldy, D, eps);
  return check_launch("rmsnorm");
}

SSD_API int ssd_embed_bf16(const int32_t* ids, int M, const uint16_t* table, int64_t V, int D, uint16_t* out,
                           int64_t ldo, hipStream_t stream) {
  if (!ids || !table || !out || M < 0 || D % 8 || ldo % 8) return set_error(SSD_EINVAL, "embed: bad arguments");
  if (M == 0) return SSD_OK;
  SSD_LAUNCH(embed_kernel, dim3(M), dim3(256), 0, stream, ids, table, V, D, out, ldo);
  return check_launch("embed");
}

SSD_API int ssd_kv_compact_bf16(uint16_t* k_arena, uint16_t* vt_arena, int layers, int kv_heads, int head_dim,
                                int64_t max_len, int start, const int32_t* src, const int32_t* n_dev, int n_max,
                                const int32_t* pos_base, hipStream_t stream) {
  if (!k_arena || !vt_arena || !src || !n_dev || layers <= 0 || kv_heads <= 0 || head_dim <= 0 || n_max < 0)
    return set_error(SSD_EINVAL, "kv_compact: bad arguments");
  if (head_dim % 32 || max_len % 64)
    return set_error(SSD_EINVAL, "kv_compact: head_dim %d / max_len %lld must be multiples of 32 / 64", head_dim,
                     (long long)max_len);
  if (!pos_base && (start < 0 || start + n_max > max_len))
    return set_error(SSD_EINVAL, "kv_compact: start %d + %d > max_len", start, n_max);
  if (n_max == 0) return SSD_OK;
  const size_t lds = ((size_t)n_max * (head_dim / 8) + (size_t)((n_max + 7) / 8 + 1) * head_dim) * 16;
  if (lds > 64 * 1024) return set_error(SSD_ERANGE, "kv_compact: n_max=%d too large", n_max);
  SSD_LAUNCH(kv_compact_kernel, dim3(layers * kv_heads), dim3(256), lds, stream, (bf16_t*)k_arena,
                     (bf16_t*)vt_arena, kv_heads, head_dim, max_len, start, src, n_dev, n_max, pos_base);
  return check_launch("kv_compact");
}

// Merge pass alone, over S records per row written by ssd_row_topk_partial_bf16 (S = ceil(N / 4096))
// or ssd_gemm_topk_bf16 (S = ssd_gemm_topk_parts(N)).
SSD_API int ssd_row_topk_merge(const void* parts, int64_t parts_bytes, int M, int S, int k, int mode,
                               const int32_t* vocab_ids, int32_t* out_tok, float* out_val, float* out_lse,
                               hipStream_t stream) {
  if (!parts || !out_tok) return set_error(SSD_EINVAL, "row_topk_merge: null pointer");
  if ((uintptr_t)parts & 7) return set_error(SSD_EINVAL, "row_topk_merge: parts must be 8-byte aligned");
  if (M < 0 || k < 1 || k > TOPK_MAX || (mode != 0 && mode != 1))
    return set_error(SSD_EINVAL, "row_topk_merge: M=%d k=%d mode=%d", M, k, mode);
  if (S < 1 || S > TOPK_MAX_PARTS || S * k > 64 * TOPK_MAX)
    return set_error(SSD_EINVAL, "row_topk_merge: %d records of %d keys per row", S, k);
  if (parts_bytes < (int64_t)M * S * (int64_t)sizeof(TopkPart))
    return set_error(SSD_EINVAL, "row_topk_merge: parts of %lld bytes < %lld", (long long)parts_bytes,
                     (long long)M * S * (long long)sizeof(TopkPart));
  if (M == 0) return SSD_OK;
  SSD_LAUNCH(row_topk_merge_kernel, dim3(M), dim3(64), 0, stream, (const TopkPart*)parts, S, k, mode, vocab_ids,
             out_tok, out_val, out_lse);
  return check_launch("row_topk_merge");
}

SSD_API int64_t ssd_row_topk_ws_bytes(int M, int N) {
  const int S = (N + TOPK_CHUNK - 1) / TOPK_CHUNK;
  return (int64_t)M * S * (int64_t)sizeof(TopkPart);
}

static int row_topk_launch(const uint16_t* logits, int64_t ld, int M, int N, int k, int mode,
                           const int32_t* vocab_ids, int32_t* out_tok, float* out_val, float* out_lse, TopkPart* parts,
                           hipStream_t stream) {
  const int S = (N + TOPK_CHUNK - 1) / TOPK_CHUNK;
  SSD_LAUNCH(row_topk_partial_kernel, dim3(S, M), dim3(256), 0, stream, logits, ld, N, k, mode, parts);
  int rc = check_launch("row_topk_partial");
  if (rc) return rc;
  SSD_LAUNCH(row_topk_merge_kernel, dim3(M), dim3(64), 0, stream, (const TopkPart*)parts, S, k, mode,
                     vocab_ids, out_tok, out_val, out_lse);
  return check_launch("row_topk_merge");
}

static int row_topk_check(const uint16_t* logits, int64_t ld, int N, int k, int mode, const int32_t* out_tok) {
  if (!logits || !out_tok || N <= 0 || k < 1 || k > TOPK_MAX || k > N || (mode != 0 && mode != 1))
    return set_error(SSD_EINVAL, "row_topk: bad arguments (k=%d, N=%d, mode=%d)", k, N, mode);
  if (ld % 8 || ((uintptr_t)logits & 15)) return set_error(SSD_EINVAL, "row_topk: logits must be 16-byte aligned");
  if ((N + TOPK_CHUNK - 1) / TOPK_CHUNK > 64)
    return set_error(SSD_ERANGE, "row_topk: N=%d above %d columns", N, 64 * TOPK_CHUNK);
  return SSD_OK;
}

// The partial pass alone: the chunk records of ssd_row_topk_bf16's workspace, for a consumer that
// merges them itself (ssd_tree_level_topk).
SSD_API int ssd_row_topk_partial_bf16(const uint16_t* logits, int64_t ld, int M, int N, int k, int mode, void* ws,
                                      int64_t ws_bytes, hipStream_t stream) {
  if (M < 0 || !ws) return set_error(SSD_EINVAL, "row_topk_partial: bad arguments (M=%d, workspace %p)", M, ws);
  if (!logits || N <= 0 || k < 1 || k > TOPK_MAX || k > N || (mode != 0 && mode != 1))
    return set_error(SSD_EINVAL, "row_topk_partial: bad arguments (k=%d, N=%d, mode=%d)", k, N, mode);
  if (ld % 8 || ((uintptr_t)logits & 15))
    return set_error(SSD_EINVAL, "row_topk_partial: logits must be 16-byte aligned");
  const int S = (N + TOPK_CHUNK - 1) / TOPK_CHUNK;
  if (S > 64) return set_error(SSD_ERANGE, "row_topk_partial: N=%d above %d columns", N, 64 * TOPK_CHUNK);
  if (ws_bytes < ssd_row_topk_ws_bytes(M, N)) return set_error(SSD_EINVAL, "row_topk_partial: workspace too small");
  if (M == 0) return SSD_OK;
  SSD_LAUNCH(row_topk_partial_kernel, dim3(S, M), dim3(256), 0, stream, (const bf16_t*)logits, ld, N, k, mode,
             (TopkPart*)ws);
  return check_launch("row_topk_partial");
}

SSD_API int ssd_row_topk_bf16(const uint16_t* logits, int64_t ld, int M, int N, int k, int mode,
                              const int32_t* vocab_ids, int32_t* out_tok, float* out_val, float* out_lse, void* ws,
                              int64_t ws_bytes, hipStream_t stream) {
  if (M < 0 || !ws) return set_error(SSD_EINVAL, "row_topk: bad arguments (M=%d, workspace %p)", M, ws);
  if (int rc = row_topk_check(logits, ld, N, k, mode, out_tok)) return rc;
  if (ws_bytes < ssd_row_topk_ws_bytes(M, N)) return set_error(SSD_EINVAL, "row_topk: workspace too small");
  if (M == 0) return SSD_OK;
  return row_topk_launch(logits, ld, M, N, k, mode, vocab_ids, out_tok, out_val, out_lse, (TopkPart*)ws, stream);
}

// ---- the same reduction without a caller workspace: the chunk partials live in a file-scope
// device array (one copy per GPU, held until the process ends). Host code never passes the
// array's name to a kernel (on the host it is only a stand-in symbol): its device address is
// looked up once per device with hipGetSymbolAddress, with that device current, and kept.
constexpr int TOPK_STATIC_PARTS = 64 * 64;  // rows x 4096-column chunks: 64 rows of up to 262144 columns
static __device__ __align__(256) TopkPart scratch[TOPK_STATIC_PARTS];  // 544 KiB per GPU

constexpr int MAX_DEVICES = 64;
static TopkPart* scratch_ptr[MAX_DEVICES];
static std::mutex scratch_mu;

static int topk_scratch(TopkPart** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return set_error(SSD_EHIP, "row_topk_noalloc: no current device");
  if (dev < 0 || dev >= MAX_DEVICES) return set_error(SSD_ERANGE, "row_topk_noalloc: device %d", dev);
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (!scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_error(SSD_EHIP, "row_topk_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                       hipGetErrorString(e));
    scratch_ptr[dev] = (TopkPart*)p;
  }
  *out = scratch_ptr[dev];
  return SSD_OK;
}

SSD_API int ssd_row_topk_bf16_noalloc(const uint16_t* logits, int64_t ld, int M, int N, int k, int mode,
                                      const int32_t* vocab_ids, int32_t* out_tok, float* out_val, float* out_lse,
                                      hipStream_t stream) {
  if (M < 0) return set_error(SSD_EINVAL, "row_topk_noalloc: M=%d", M);
  if (int rc = row_topk_check(logits, ld, N, k, mode, out_tok)) return rc;
  const int64_t parts = (int64_t)M * ((N + TOPK_CHUNK - 1) / TOPK_CHUNK);
  if (parts > TOPK_STATIC_PARTS)
    return set_error(SSD_ERANGE,
                     "row_topk_noalloc: M=%d rows x %d-column chunks of N=%d need %lld partials, the static "
                     "scratch holds %d (use ssd_row_topk_bf16 with a workspace)",
                     M, TOPK_CHUNK, N, (long long)parts, TOPK_STATIC_PARTS);
  if (M == 0) return SSD_OK;
  TopkPart* ws = nullptr;
  if (int rc = topk_scratch(&ws)) return rc;
  return row_topk_launch(logits, ld, M, N, k, mode, vocab_ids, out_tok, out_val, out_lse, ws, stream);
}

SSD_API int ssd_add_rmsnorm_bf16(const float* P, int64_t ldp, int64_t split_stride, int S, const uint16_t* bias,
                                 uint16_t* h, int64_t ldh, int M, int D, const uint16_t* w, float eps, uint16_t* y,
                                 int64_t ldy, hipStream_t stream) {
  if (!h || (y && !w) || (S > 0 && !P) || S < 0 || S > 16 || M < 0 || D <= 0 || D % 8)
    return set_error(SSD_EINVAL, "add_rmsnorm: null pointer or bad S=%d M=%d D=%d", S, M, D);
  if (((uintptr_t)h & 15) || ldh % 8 || (y && (((uintptr_t)y & 15) || ldy % 8)) || (w && ((uintptr_t)w & 15)) ||
      (bias && ((uintptr_t)bias & 15)))
    return set_error(SSD_EINVAL, "add_rmsnorm: bf16 tensors must be 16-byte aligned with strides %% 8 == 0");
  if (S > 0 && (((uintptr_t)P & 15) || ldp % 4 || ldp < D || split_stride < (int64_t)M * ldp || split_stride % 4))
    return set_error(SSD_EINVAL, "add_rmsnorm: partials need 16-byte alignment, ldp >= D, split stride >= M*ldp");
  if (M == 0) return SSD_OK;
#define SSD_ADD_RMS(S_)                                                                                       \
  SSD_LAUNCH((add_rmsnorm_kernel<S_>), dim3(M), dim3(1024), 0, stream, P, ldp, split_stride,          \
                     (const bf16_t*)bias, (bf16_t*)h, ldh, (const bf16_t*)w, (bf16_t*)y, ldy, D, eps)
  switch (S) {
    case 0: SSD_ADD_RMS(0); break;
    case 1: SSD_ADD_RMS(1); break;
    case 2: SSD_ADD_RMS(2); break;
    case 4: SSD_ADD_RMS(4); break;
    case 8: SSD_ADD_RMS(8); break;
    case 16: SSD_ADD_RMS(16); break;
    default: return set_error(SSD_EINVAL, "add_rmsnorm: split count %d not in {0, 1, 2, 4, 8, 16}", S);
  }
#undef SSD_ADD_RMS
  return check_launch("add_rmsnorm");
}

