// Host-side sequencer of one model forward (draft sub-network or full target): every kernel of
// the forward is enqueued from here in one C-ABI call, so a decode round costs a handful of
// host calls instead of one per kernel.
//
// Order per selected layer (ssd/models/subnetwork_draft.py:193-246 and :315-351 in the
// reference): [bridge] -> RMSNorm -> q/k/v GEMM + RoPE + KV write -> tree attention (+ combine)
// -> o GEMM + residual -> RMSNorm -> gate/up GEMM + SwiGLU -> down GEMM + residual; then
// [pre-norm bridge] -> final RMSNorm -> lm_head (or the vocabulary-subset head).
#include "common.h"

namespace ssd {

static int bridge_forward(const SsdBridgeW* b, const SsdBuffers* buf, int m, int d, hipStream_t s) {
  const int64_t ld = d;
  const int widest = b->swiglu ? b->hidden : (b->n_body > 0 ? b->body_n[b->n_body - 1] : 0);
  if (b->n_body < 0 || b->n_body > 2 || (!b->swiglu && b->n_body == 0))
    return set_error(SSD_EINVAL, "forward: bridge with %d body linears", b->n_body);
  for (int i = 0; i < (b->swiglu ? 0 : b->n_body); ++i)
    if (b->body_n[i] > buf->mid_cols) return set_error(SSD_EINVAL, "forward: bridge width %d > %d", b->body_n[i], buf->mid_cols);
  if (widest > buf->mid_cols) return set_error(SSD_EINVAL, "forward: bridge width %d > %d", widest, buf->mid_cols);
  int rc = ssd_rmsnorm_bf16(buf->h, ld, m, d, b->norm, b->eps, buf->x, ld, s);
  if (rc) return rc;
  const uint16_t* cur = buf->x;
  int64_t ldc = ld;
  int kin = d;
  if (b->swiglu) {
    rc = ssd_gemm_swiglu_bf16(buf->x, ld, m, b->gu, b->hidden, d, buf->mid0, buf->mid_cols, b->bg, b->bu, s);
    if (rc) return rc;
    cur = buf->mid0;
    ldc = buf->mid_cols;
    kin = b->hidden;
  } else {
    for (int i = 0; i < b->n_body; ++i) {
      uint16_t* dst = (i % 2) ? buf->mid1 : buf->mid0;
      rc = ssd_gemm_bf16(cur, ldc, m, b->body_w[i], b->body_n[i], kin, dst, buf->mid_cols, b->body_b[i], b->body_act[i],
                         nullptr, 0, s);
      if (rc) return rc;
      cur = dst;
      ldc = buf->mid_cols;
      kin = b->body_n[i];
    }
  }
  return ssd_gemm_bf16(cur, ldc, m, b->out, d, kin, buf->h, ld, b->out_b, 0, buf->h, ld, s);
}

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
  const int d = md->hidden, hd = md->head_dim, H = md->heads, KV = md->kv_heads;
  const int64_t qdim = (int64_t)H * hd;
  const size_t layer_elems = (size_t)KV * buf->cache_cap * hd;
  int rc = ssd_embed_bf16(rows->ids, m, md->embed, md->vocab, d, buf->h, d, s);
  if (rc) return rc;
  for (int st = 0; st < plan->n_steps; ++st) {
    const int li = plan->layer_ids[st];
    if (li < 0 || li >= md->n_layers) return set_error(SSD_EINVAL, "forward: layer %d", li);
    if (plan->pre_bridge && plan->pre_bridge[st]) {
      rc = bridge_forward(plan->pre_bridge[st], buf, m, d, s);
      if (rc) return rc;
    }
    const SsdLayerW& L = md->layers[li];
    uint16_t* kc = buf->k_arena + li * layer_elems;
    uint16_t* vt = buf->vt_arena + li * layer_elems;
    if ((rc = ssd_rmsnorm_bf16(buf->h, d, m, d, L.ln1, md->eps, buf->x, d, s))) return rc;
    if ((rc = ssd_gemm_qkv_rope_bf16(buf->x, d, m, L.wqkv, d, H, KV, hd, md->cos, md->sin, md->rope_rows, rows->pos,
                                     rows->slot, buf->q, qdim, kc, vt, buf->cache_cap, s)))
      return rc;
    if ((rc = ssd_tree_attention_bf16(buf->q, qdim, m, H, KV, hd, kc, vt, buf->cache_cap, rows->prefix, rows->depth,
                                      rows->anc, p_min, l_max, md->attn_scale, buf->attn_ws, buf->attn_ws_floats,
                                      buf->attn, qdim, s)))
      return rc;
    if ((rc = ssd_gemm_bf16(buf->attn, qdim, m, L.wo, d, (int)qdim, buf->h, d, nullptr, 0, buf->h, d, s))) return rc;
    if ((rc = ssd_rmsnorm_bf16(buf->h, d, m, d, L.ln2, md->eps, buf->x, d, s))) return rc;
    if ((rc = ssd_gemm_swiglu_bf16(buf->x, d, m, L.wgu, md->inter, d, buf->mlp, md->inter, nullptr, nullptr, s))) return rc;
    if ((rc = ssd_gemm_bf16(buf->mlp, md->inter, m, L.wd, d, md->inter, buf->h, d, nullptr, 0, buf->h, d, s))) return rc;
  }
  if (plan->pre_norm && (rc = bridge_forward(plan->pre_norm, buf, m, d, s))) return rc;
  if ((rc = ssd_rmsnorm_bf16(buf->h, d, m, d, md->norm, md->eps, buf->x, d, s))) return rc;
  if (head_rows > 0 && plan->head_w) {
    rc = ssd_gemm_bf16(buf->x + (size_t)head_first * d, d, head_rows, plan->head_w, plan->head_n, d, buf->logits,
                       buf->ld_logits, nullptr, 0, nullptr, 0, s);
    if (rc) return rc;
  }
  return SSD_OK;
}
