// GEMM arguments and the bf16 epilogues shared by the decode GEMMs (gemm.hip) and the prefill
// GEMM (prefill.hip): per-element functions from fp32 dot products to the reference's bf16
// rounding points -- plain store with bias / activation / residual add, SwiGLU of a gate/up
// tile pair, and q/k/v with RoPE and the KV-cache write.
#pragma once

#include "common.h"

namespace ssd {

enum Epi { EPI_STORE = 0, EPI_SWIGLU = 1, EPI_QKV = 2 };

struct GemmArgs {
  const bf16_t* X;
  int64_t ldx;
  int M;
  const uint4* W;  // packed tiles
  int N;           // logical output columns (rows of W)
  int kb_total;    // K / 32
  // EPI_STORE
  bf16_t* Y;
  int64_t ldy;
  const bf16_t* bias;      // [N] or null
  int act;                 // Act
  const bf16_t* residual;  // [M, ldr] or null (Y may alias it)
  int64_t ldr;
  // EPI_SWIGLU: bias for gate / up (null ok); output columns = N / 2
  const bf16_t* bias2;
  // EPI_QKV
  int heads, kv_heads, head_dim;
  const bf16_t* cos_tab;  // [rope_rows, head_dim/2]
  const bf16_t* sin_tab;
  const int* row_pos;     // [M]
  const int* row_slot;    // [M]
  int64_t rope_rows;
  bf16_t* k_cache;        // this layer: kv_heads x (max_len x head_dim) in the block layout (k_off)
  bf16_t* vt_cache;       // this layer: kv_heads x (max_len x head_dim) in the block layout (v_off)
  int64_t max_len;
  const int64_t* row_kv_off;  // [M] element offset of row m's sequence in the cache arena, or null
  // RMSNorm of the rows of X folded into the GEMM (> 0: X is the residual stream h; the norm's
  // weight is already folded into W's columns; each output is scaled by rsqrt(mean(h^2) + eps))
  float norm_eps;
  // prefill: the folded RMSNorm's row scales, computed beforehand (rsqrt(mean(x^2) + eps) per row of
  // X, [M] floats); used instead of norm_eps's in-loop sums where a kernel supports it
  const float* row_scale;
};


// Per-element epilogues (fp32 dot products in, bf16 rounding points of the reference out).
// Plain store: output column n of row m.
__device__ __forceinline__ void epi_store(const GemmArgs& a, int n, int m, float t) {
  if (a.bias) t += bf2f(a.bias[n]);
  t = rbf(t);
  if (a.act) t = rbf(apply_act(a.act, t));
  if (a.residual) t = rbf(bf2f(a.residual[(size_t)m * a.ldr + n]) + t);
  a.Y[(size_t)m * a.ldy + n] = f2bf(t);
}

// epi_store with the bias and residual values already loaded (bias_v / res_v are read only when
// the corresponding pointer is set).
__device__ __forceinline__ void epi_store_pre(const GemmArgs& a, int n, int m, float t, float bias_v, float res_v) {
  if (a.bias) t += bias_v;
  t = rbf(t);
  if (a.act) t = rbf(apply_act(a.act, t));
  if (a.residual) t = rbf(res_v + t);
  a.Y[(size_t)m * a.ldy + n] = f2bf(t);
}

// SwiGLU: intermediate column col of row m from its gate and up dot products.
__device__ __forceinline__ void epi_swiglu(const GemmArgs& a, int col, int m, float gt, float up) {
  if (a.bias) gt += bf2f(a.bias[col]);
  if (a.bias2) up += bf2f(a.bias2[col]);
  const float gs = rbf(silu_f(rbf(gt)));
  a.Y[(size_t)m * a.ldy + col] = f2bf(gs * rbf(up));
}

// q/k/v tile nb, pair r (rows r and r + 8 = rotary dims p*8 + r and hd/2 + p*8 + r) of row m:
// RoPE for q/k, then Q store or KV-cache write (block layout, k_off / v_off).
__device__ __forceinline__ void epi_qkv(const GemmArgs& a, int nb, int m, int r, float vlo, float vhi) {
  const int hd = a.head_dim, half = hd >> 1, tiles_per_head = hd >> 4;
  const int q_tiles = a.heads * tiles_per_head, k_tiles = a.kv_heads * tiles_per_head;
  int region, head, p;
  if (nb < q_tiles) {
    region = 0; head = nb / tiles_per_head; p = nb % tiles_per_head;
  } else if (nb < q_tiles + k_tiles) {
    region = 1; head = (nb - q_tiles) / tiles_per_head; p = (nb - q_tiles) % tiles_per_head;
  } else {
    region = 2; head = (nb - q_tiles - k_tiles) / tiles_per_head; p = (nb - q_tiles - k_tiles) % tiles_per_head;
  }
  const int dlo = p * 8 + r, dhi = dlo + half;
  const float xlo = rbf(vlo), xhi = rbf(vhi);
  const int slot = a.row_slot[m];
  if (region != 0 && (slot < 0 || slot >= a.max_len)) return;  // never write outside the cache
  const int64_t off = a.row_kv_off ? a.row_kv_off[m] : 0;
  if (region == 2) {
    bf16_t* vt = a.vt_cache + off + (size_t)head * hd * a.max_len;
    vt[v_off(slot, dlo, hd)] = f2bf(xlo);
    vt[v_off(slot, dhi, hd)] = f2bf(xhi);
    return;
  }
  const int pos = min(max(a.row_pos[m], 0), (int)a.rope_rows - 1);
  const float cs = bf2f(a.cos_tab[(size_t)pos * half + dlo]);
  const float sn = bf2f(a.sin_tab[(size_t)pos * half + dlo]);
  const float olo = rbf(rbf(xlo * cs) - rbf(xhi * sn));
  const float ohi = rbf(rbf(xhi * cs) + rbf(xlo * sn));
  if (region == 0) {
    bf16_t* q = a.Y + (size_t)m * a.ldy + (size_t)head * hd;
    q[dlo] = f2bf(olo);
    q[dhi] = f2bf(ohi);
  } else {
    bf16_t* kc = a.k_cache + off + (size_t)head * a.max_len * hd;
    kc[k_off(slot, dlo, hd)] = f2bf(olo);
    kc[k_off(slot, dhi, hd)] = f2bf(ohi);
  }
}

// Where tile nb of the fused q/k/v weight lands: region 0 q / 1 k / 2 v, its head, and the
// rotary pair block p (tile rows r and r + 8 are dims p*8 + r and hd/2 + p*8 + r).
struct QkvTile {
  int region, head, p;
};
__device__ __forceinline__ QkvTile qkv_tile(const GemmArgs& a, int nb) {
  const int tph = a.head_dim >> 4;  // tiles per head (head_dim is a power of two)
  const int sh = __ffs(tph) - 1;
  const int q_tiles = a.heads * tph, k_tiles = a.kv_heads * tph;
  const int region = nb < q_tiles ? 0 : nb < q_tiles + k_tiles ? 1 : 2;
  const int rel = nb - (region == 0 ? 0 : region == 1 ? q_tiles : q_tiles + k_tiles);
  return QkvTile{region, rel >> sh, rel & (tph - 1)};
}

// epi_qkv with the row's cache slot and rotary cos/sin already loaded (prefetched before the
// main loop, so the epilogue issues no dependent loads).
__device__ __forceinline__ void epi_qkv_pre(const GemmArgs& a, const QkvTile& q, int m, int r, float vlo,
                                            float vhi, int slot, float cs, float sn, int64_t kv_off) {
  const int hd = a.head_dim, half = hd >> 1;
  const int dlo = q.p * 8 + r, dhi = dlo + half;
  const float xlo = rbf(vlo), xhi = rbf(vhi);
  if (q.region != 0 && (slot < 0 || slot >= a.max_len)) return;  // never write outside the cache
  if (q.region == 2) {
    bf16_t* vt = a.vt_cache + kv_off + (size_t)q.head * hd * a.max_len;
    vt[v_off(slot, dlo, hd)] = f2bf(xlo);
    vt[v_off(slot, dhi, hd)] = f2bf(xhi);
    return;
  }
  const float olo = rbf(rbf(xlo * cs) - rbf(xhi * sn));
  const float ohi = rbf(rbf(xhi * cs) + rbf(xlo * sn));
  if (q.region == 0) {
    bf16_t* qo = a.Y + (size_t)m * a.ldy + (size_t)q.head * hd;
    qo[dlo] = f2bf(olo);
    qo[dhi] = f2bf(ohi);
  } else {
    bf16_t* kc = a.k_cache + kv_off + (size_t)q.head * a.max_len * hd;
    kc[k_off(slot, dlo, hd)] = f2bf(olo);
    kc[k_off(slot, dhi, hd)] = f2bf(ohi);
  }
}

// Epilogue of one 16-row tile `nb` for rows m < Mv; val(r, m) is the fp32 dot product of tile
// row r and token m. Threads tid, tid + NTHREADS, ... of the caller share the work.
template <int EPI, int NTHREADS, class Val>
__device__ __forceinline__ void gemm_epilogue(const GemmArgs& a, int nb, int Mv, Val val, int tid) {
  if (nb * 16 >= a.N) return;
  if constexpr (EPI == EPI_STORE) {
    for (int o = tid; o < 16 * Mv; o += NTHREADS) {
      const int m = o >> 4, r = o & 15;
      const int n = nb * 16 + r;
      if (n < a.N) epi_store(a, n, m, val(r, m));
    }
  } else if constexpr (EPI == EPI_SWIGLU) {
    for (int o = tid; o < 8 * Mv; o += NTHREADS) {
      const int m = o >> 3, r = o & 7;
      const int col = nb * 8 + r;  // intermediate index
      if (col * 2 < a.N) epi_swiglu(a, col, m, val(r, m), val(r + 8, m));
    }
  } else {  // EPI_QKV
    for (int o = tid; o < 8 * Mv; o += NTHREADS) {
      const int m = o >> 3, r = o & 7;
      epi_qkv(a, nb, m, r, val(r, m), val(r + 8, m));
    }
  }
}

// Sum of squares of the 8 bf16 values in a 16-byte fragment.
__device__ __forceinline__ float sumsq8(u32x4_t v) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float lo = __uint_as_float(v[i] << 16), hi = __uint_as_float(v[i] & 0xffff0000u);
    s = fmaf(lo, lo, s);
    s = fmaf(hi, hi, s);
  }
  return s;
}

}  // namespace ssd
