// Host-side sequencer of one model forward (draft sub-network or full target): every kernel of
// the forward is enqueued from here in one C-ABI call, so a decode round costs a handful of
// host calls instead of one per kernel.
//
// Order per selected layer (ssd/models/subnetwork_draft.py:193-246 and :315-351 in the
// reference). Every RMSNorm is folded into the projection that consumes it (its weight is in the
// packed columns, the row scale is computed inside the GEMM from the rows it streams), and every
// residual add is fused into the projection that produces it, so h is the only activation that
// moves between sub-layers (a long-K projection runs as split-K partials plus a finalize that adds):
//   [bridge: body GEMMs (bridge norm folded) -> out_proj, h += out]
//   q/k/v GEMM (ln1 folded) with RoPE + KV write in its epilogue -> tree attention (+ combine)
//   -> o_proj, h += o -> gate/up GEMM (ln2 folded) + SwiGLU -> down_proj, h += down
//   (the last three as one cooperative launch, ssd_mlp_bf16, when the model's gate/up weights
//   are packed for it)
// then the head over h (final norm folded).
#include "common.h"

namespace ssd {

struct Fwd {
  const SsdModel* md;
  const SsdBuffers* buf;
  int m, d;
  hipStream_t s;

  // h += X W^T (+ bias), one launch.
  int residual(const uint16_t* X, int64_t ldx, const uint16_t* W, int K, const uint16_t* bias) {
    return ssd_gemm_residual_bf16(X, ldx, m, W, d, K, bias, buf->h, d, buf->part, buf->part_floats, s);
  }

  // Bridge: body on RMSNorm(h) (folded into its first GEMM), then h += out_proj(...).
  int bridge(const SsdBridgeW* b) {
    const int widest = b->swiglu ? b->hidden : (b->n_body > 0 ? b->body_n[b->n_body - 1] : 0);
    if (b->n_body < 0 || b->n_body > 2 || (!b->swiglu && b->n_body == 0))
      return set_error(SSD_EINVAL, "forward: bridge with %d body linears", b->n_body);
    if (!(b->eps > 0.f)) return set_error(SSD_EINVAL, "forward: bridge norm eps must be > 0");
    for (int i = 0; i < (b->swiglu ? 0 : b->n_body); ++i)
      if (b->body_n[i] > buf->mid_cols) return set_error(SSD_EINVAL, "forward: bridge width %d > %d", b->body_n[i], buf->mid_cols);
    if (widest > buf->mid_cols) return set_error(SSD_EINVAL, "forward: bridge width %d > %d", widest, buf->mid_cols);
    const uint16_t* cur = buf->h;
    int64_t ldc = d;
    int kin = d, rc;
    if (b->swiglu) {
      rc = ssd_gemm_swiglu_bf16(buf->h, d, m, b->gu, b->hidden, d, b->eps, buf->mid0, buf->mid_cols, b->bg, b->bu, s);
      if (rc) return rc;
      cur = buf->mid0;
      ldc = buf->mid_cols;
      kin = b->hidden;
    } else {
      for (int i = 0; i < b->n_body; ++i) {
        uint16_t* dst = (i % 2) ? buf->mid1 : buf->mid0;
        rc = ssd_gemm_bf16(cur, ldc, m, b->body_w[i], b->body_n[i], kin, i == 0 ? b->eps : 0.f, dst, buf->mid_cols,
                           b->body_b[i], b->body_act[i], nullptr, 0, s);
        if (rc) return rc;
        cur = dst;
        ldc = buf->mid_cols;
        kin = b->body_n[i];
      }
    }
    return residual(cur, ldc, b->out, kin, b->out_b);
  }
};

}  // namespace ssd

using namespace ssd;

SSD_API int ssd_forward(const SsdModel* md, const SsdPlan* plan, const SsdBuffers* buf, const SsdRows* rows, int m,
                        int p_min, int l_max, int head_first, int head_rows, hipStream_t s) {
  if (!md || !plan || !buf || !rows) return set_error(SSD_EINVAL, "forward: null descriptor");
  if (m <= 0 || m > buf->m_cap || m > rows->cap) return set_error(SSD_EINVAL, "forward: m=%d outside [1, %d]", m, buf->m_cap);
  if (head_rows < 0 || head_first < 0 || head_first + head_rows > m)
    return set_error(SSD_EINVAL, "forward: head rows [%d, %d) outside [0, %d)", head_first, head_first + head_rows, m);
  if (l_max > buf->cache_cap) return set_error(SSD_EINVAL, "forward: l_max %d > cache %lld", l_max, (long long)buf->cache_cap);
  if (head_rows > 0 && plan->head_w && (!buf->logits || plan->head_n > buf->ld_logits))
    return set_error(SSD_EINVAL, "forward: head of %d columns into logits rows of %lld", plan->head_n,
                     (long long)buf->ld_logits);
  if (!md->layers || (plan->n_steps > 0 && !plan->layer_ids)) return set_error(SSD_EINVAL, "forward: null layer table");
  if (!(md->eps > 0.f)) return set_error(SSD_EINVAL, "forward: norm eps must be > 0");
  for (int st = 0; st < plan->n_steps; ++st)
    if (plan->layer_ids[st] < 0 || plan->layer_ids[st] >= md->n_layers)
      return set_error(SSD_EINVAL, "forward: layer %d", plan->layer_ids[st]);
  const int d = md->hidden, hd = md->head_dim, H = md->heads, KV = md->kv_heads;
  const int64_t qdim = (int64_t)H * hd;
  const size_t layer_elems = (size_t)KV * buf->cache_cap * hd;
  Fwd f{md, buf, m, d, s};
  int rc = ssd_embed_bf16(rows->ids, m, md->embed, md->vocab, d, buf->h, d, s);
  if (rc) return rc;
  for (int st = 0; st < plan->n_steps; ++st) {
    const int li = plan->layer_ids[st];
    const SsdLayerW& L = md->layers[li];
    if (plan->pre_bridge && plan->pre_bridge[st] && (rc = f.bridge(plan->pre_bridge[st]))) return rc;
    uint16_t* kc = buf->k_arena + li * layer_elems;
    uint16_t* vt = buf->vt_arena + li * layer_elems;
    if ((rc = qkv_rope_gemm(buf->h, d, m, L.wqkv, d, md->eps, H, KV, hd, md->cos, md->sin, md->rope_rows, rows->pos,
                            rows->slot, rows->kv_off, buf->q, qdim, kc, vt, buf->cache_cap, s)))
      return rc;
    if ((rc = tree_attention(buf->q, qdim, m, H, KV, hd, kc, vt, buf->cache_cap, rows->prefix, rows->depth, rows->anc,
                             rows->kv_off, p_min, l_max, md->attn_scale, buf->attn_ws, buf->attn_ws_floats, buf->attn,
                             qdim, s)))
      return rc;
    if ((rc = f.residual(buf->attn, qdim, L.wo, (int)qdim, nullptr))) return rc;
    if (md->mlp_fused) {
      if ((rc = ssd_mlp_bf16(buf->h, d, m, L.wgu, L.wd, md->inter, d, md->eps, buf->mlp, md->inter, buf->part,
                             buf->part_floats, buf->sync, s)))
        return rc;
      continue;
    }
    if ((rc = ssd_gemm_swiglu_bf16(buf->h, d, m, L.wgu, md->inter, d, md->eps, buf->mlp, md->inter, nullptr, nullptr,
                                   s)))
      return rc;
    if ((rc = f.residual(buf->mlp, md->inter, L.wd, md->inter, nullptr))) return rc;
  }
  if (plan->pre_norm && (rc = f.bridge(plan->pre_norm))) return rc;
  if (head_rows > 0 && plan->head_w) {
    rc = ssd_gemm_bf16(buf->h + (size_t)head_first * d, d, head_rows, plan->head_w, plan->head_n, d, md->eps,
                       buf->logits, buf->ld_logits, nullptr, 0, nullptr, 0, s);
    if (rc) return rc;
  }
  return SSD_OK;
}
