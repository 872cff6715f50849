// Device-resident speculation tree: level expansion, max_nodes pruning, verify
// inputs and greedy acceptance. These replace the host loops of
// ssd/engine/tree_drafter.py:147-208 and ssd/engine/verify.py:32-57 so that a
// round needs no host round trip until its committed tokens are read back.
//
// Ordering rules are the reference's, restated:
// * candidates of a level sort by cumulative score (double), ties keeping the
//   order (frontier position, proposal rank) -- Python's stable sort of
//   tree_drafter.py:172;
// * the final cut sorts by (-score, depth), ties keeping node index order
//   (tree_drafter.py:203), then closes the kept set under ancestors and
//   renumbers it in original order (tree_drafter.py:80-95, 204-207);
// * greedy acceptance walks root -> children in rank order, taking the child
//   whose token equals the target argmax (verify.py:45-57).
// Each step is one small workgroup: ranks are computed by counting (every
// thread compares its candidate against all others), which is exact and
// deterministic.
#include "common.h"
#include "topk.h"

#include <math.h>

namespace ssd {

constexpr int TREE_MAXDEPTH = 32;
constexpr int TREE_CAP = 1024;
constexpr int ROW_MAXD = 32;  // ancestors per row (matches the attention gather list)

}  // namespace ssd

namespace ssd {

// Level d's expansion from its candidates (cand_tok / cand_lp: frontier node f's k proposals at
// f*k .. f*k + k - 1, in global memory or LDS). The tree's parents, draft slots and scores are
// staged in LDS at the start (one load per thread, with the level counts), and the new nodes are
// mirrored there, so the parents' scores and the fed rows' ancestor walks read LDS instead of
// chains of dependent global loads. tree_level_stage must run first (before a barrier).
struct TreeLevelLds {
  double sc[TREE_CAP];   // candidate scores
  int vd[TREE_CAP];      // candidate valid
  double tsc[TREE_CAP];  // tree node scores
  int par[TREE_CAP];     // tree node parents
  int dpos[TREE_CAP];    // tree node draft slots
  int tok[TREE_CAP];     // new node j's token (this level)
  int nvalid;
};

__device__ __forceinline__ void tree_level_stage(const SsdTree& t, TreeLevelLds& L) {
  const int i = threadIdx.x, li = min(i, t.cap - 1);
  L.tsc[i] = t.scores[li];
  L.par[i] = t.parents[li];
  L.dpos[i] = t.draft_pos[li];
  if (i == 0) L.nvalid = 0;
}

__device__ __forceinline__ void tree_level_body(SsdTree t, int d, const int* cand_tok, const float* cand_lp, int k,
                                                int width, int feed, int root_pos, int tree_start, int past,
                                                SsdRows rows, int rows_max, int n0, int F, int prev_start,
                                                TreeLevelLds& L) {
  const int C = F * k;
  const int c = threadIdx.x;
  int parent = -1, tok = -1;
  double score = -INFINITY;
  if (c < C) {
    const int f = c / k;
    parent = d == 0 ? -1 : prev_start + f;
    tok = cand_tok[c];
    if (tok >= 0) score = (parent < 0 ? 0.0 : L.tsc[parent]) + (double)cand_lp[c];
    L.sc[c] = score;
    L.vd[c] = tok >= 0;
  }
  __syncthreads();
  if (c < C && tok >= 0) atomicAdd(&L.nvalid, 1);
  int rank = 0;
  if (c < C && tok >= 0) {
    for (int o = 0; o < C; ++o)
      if (L.vd[o] && (L.sc[o] > score || (L.sc[o] == score && o < c))) ++rank;
  }
  __syncthreads();
  const int nvalid = L.nvalid;
  const int n_level = (width > 0 && width < nvalid) ? width : nvalid;
  if (c < C && tok >= 0 && rank < n_level && n0 + rank < t.cap) {
    const int node = n0 + rank;
    const int dp = feed ? past + rank : -1;
    t.tokens[node] = tok;
    t.parents[node] = parent;
    t.depths[node] = d + 1;
    t.scores[node] = score;
    t.ranks[node] = c % k;
    t.draft_pos[node] = dp;
    L.par[node] = parent;
    L.dpos[node] = dp;
    L.tok[rank] = tok;
  }
  __syncthreads();
  if (c == 0) {
    t.meta[0] = min(n0 + n_level, t.cap);
    t.meta[1 + d] = n0;
    t.meta[1 + TREE_MAXDEPTH + d] = n_level;
  }
  if (feed && c < rows_max) {
    const int j = c;
    rows.pos[j] = root_pos + d + 1;
    rows.slot[j] = past + j;
    rows.prefix[j] = tree_start;
    int* anc = rows.anc + (size_t)j * ROW_MAXD;
    if (j < n_level && n0 + j < t.cap) {
      int cur = n0 + j;
      rows.ids[j] = L.tok[j];
      rows.depth[j] = d + 1;
      for (int i = d; i >= 0 && cur >= 0; --i) {
        anc[i] = L.dpos[cur];
        cur = L.par[cur];
      }
    } else {  // padding row (fewer candidates than the launch assumed): attends the prefix only
      rows.ids[j] = 0;
      rows.depth[j] = 0;
    }
  }
}

// Level counts: n0 nodes so far, F frontier nodes (level d - 1) starting at prev_start.
__device__ __forceinline__ void tree_level_counts(const SsdTree& t, int d, int& n0, int& F, int& prev_start) {
  n0 = t.meta[0];
  F = d == 0 ? 1 : t.meta[1 + TREE_MAXDEPTH + (d - 1)];
  prev_start = d == 0 ? 0 : t.meta[1 + (d - 1)];
}

__global__ __launch_bounds__(1024) void tree_level_kernel(SsdTree t, int d, const int* __restrict__ cand_tok,
                                                          const float* __restrict__ cand_lp, int k, int width,
                                                          int feed, int root_pos, int tree_start, int past,
                                                          SsdRows rows, int rows_max, const int* pos_base) {
  __shared__ TreeLevelLds L;
  if (pos_base) {
    const int b = *pos_base;
    root_pos += b;
    tree_start += b;
    past += b;
  }
  int n0, F, prev_start;
  tree_level_counts(t, d, n0, F, prev_start);
  tree_level_stage(t, L);
  __syncthreads();
  tree_level_body(t, d, cand_tok, cand_lp, k, width, feed, root_pos, tree_start, past, rows, rows_max, n0, F,
                  prev_start, L);
}

// The same expansion with the proposals' top-k merge in front: wave w merges the chunk partials
// of frontier rows w, w + 16, ... (topk_merge_row, log-softmax values, vocab_ids mapping) into
// LDS, exactly as row_topk_merge_kernel would write them to memory.
__global__ __launch_bounds__(1024) void tree_level_topk_kernel(SsdTree t, int d, const TopkPart* __restrict__ parts,
                                                               int S, int f_rows, const int* __restrict__ vocab_ids,
                                                               int k, int width, int feed, int root_pos,
                                                               int tree_start, int past, SsdRows rows, int rows_max,
                                                               const int* pos_base) {
  __shared__ int s_tok[TREE_CAP];
  __shared__ float s_lp[TREE_CAP];
  __shared__ TreeLevelLds L;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (pos_base) {
    const int b = *pos_base;
    root_pos += b;
    tree_start += b;
    past += b;
  }
  int n0, F, prev_start;
  tree_level_counts(t, d, n0, F, prev_start);
  tree_level_stage(t, L);
  for (int f = w; f < f_rows; f += 16)
    topk_merge_row((const char*)parts + (size_t)f * S * (size_t)(8 + 8 * k), S, k, 1, vocab_ids, lane, s_tok + f * k,
                   s_lp + f * k, nullptr);
  __syncthreads();
  tree_level_body(t, d, s_tok, s_lp, k, width, feed, root_pos, tree_start, past, rows, rows_max, n0, F, prev_start,
                  L);
}

// The tree (scores, depths, parents: at most TREE_CAP entries) is staged in LDS with one load per
// field and thread, issued together with the node count's, so the rank, the ancestor closure and the
// renumbering run on LDS instead of chains of dependent global loads.
__global__ __launch_bounds__(1024) void tree_finalize_kernel(SsdTree t, int max_nodes, int committed,
                                                             const int* __restrict__ root_token, SsdRows rows,
                                                             int rows_max, const int* pos_base) {
  if (pos_base) committed += *pos_base;
  __shared__ int keep[TREE_CAP];
  __shared__ int newidx[TREE_CAP];
  __shared__ double s_sc[TREE_CAP];
  __shared__ int s_dep[TREE_CAP], s_par[TREE_CAP], s_vdep[TREE_CAP], s_vpar[TREE_CAP], s_vtok[TREE_CAP];
  const int i = threadIdx.x;
  const int li = min(i, t.cap - 1);  // valid index for every thread (values past n are unused)
  const int root = *root_token;
  const int n = min(t.meta[0], t.cap);
  const double sc_i = t.scores[li];
  const int dep_i = t.depths[li], par_i = t.parents[li], tok_i = t.tokens[li], rank_i = t.ranks[li];
  s_sc[i] = sc_i;
  s_dep[i] = dep_i;
  s_par[i] = par_i;
  __syncthreads();
  const bool prune = max_nodes > 0 && n > max_nodes;
  if (i < n) {
    int k = 1;
    if (prune) {
      int rank = 0;
      for (int o = 0; o < n; ++o) {
        const double so = s_sc[o];
        const int dpo = s_dep[o];
        if (so > sc_i || (so == sc_i && (dpo < dep_i || (dpo == dep_i && o < i)))) ++rank;
      }
      k = rank < max_nodes;
    }
    keep[i] = k;
  }
  __syncthreads();
  // Ancestor closure (a no-op unless float ties broke it; kept for parity with the reference).
  if (i < n && keep[i]) {
    int p = par_i;
    for (int step = 0; p >= 0 && p < n && step < TREE_MAXDEPTH; ++step) {
      keep[p] = 1;
      p = s_par[p];
    }
  }
  __syncthreads();
  if (i < n) {
    int idx = 0;
    for (int o = 0; o < i; ++o) idx += keep[o];
    newidx[i] = idx;
  }
  __syncthreads();
  int vn = 0;
  for (int o = 0; o < n; ++o) vn += keep[o];
  if (i < n && keep[i]) {
    const int v = newidx[i];
    const int vp = par_i < 0 ? -1 : newidx[par_i];
    t.vtokens[v] = tok_i;
    t.vparents[v] = vp;
    t.vdepths[v] = dep_i;
    t.vranks[v] = rank_i;
    t.vorig[v] = i;
    s_vpar[v] = vp;
    s_vdep[v] = dep_i;
    s_vtok[v] = tok_i;
  }
  if (i == 0) t.vmeta[0] = vn;
  __syncthreads();
  // Verify rows (verify.py:32-42): row 0 is the root; row 1+v is verify node v.
  if (i < rows_max) {
    rows.slot[i] = committed + i;
    rows.prefix[i] = committed + 1;
    int* anc = rows.anc + (size_t)i * ROW_MAXD;
    if (i == 0) {
      rows.ids[0] = root;
      rows.pos[0] = committed;
      rows.depth[0] = 0;
    } else if (i <= vn) {
      const int v = i - 1;
      const int dep = s_vdep[v];
      rows.ids[i] = s_vtok[v];
      rows.pos[i] = committed + dep;
      rows.depth[i] = dep;
      int cur = v;
      for (int q = min(dep, ROW_MAXD) - 1; q >= 0 && cur >= 0; --q) {
        anc[q] = committed + 1 + cur;
        cur = s_vpar[cur];
      }
    } else {
      rows.ids[i] = 0;
      rows.pos[i] = committed;
      rows.depth[i] = 0;
    }
  }
}

// Greedy acceptance over the verify tree. argmax[r] is the target's first-index argmax
// for verify row r. Writes result = [n_new, tok_0..tok_{n_new-1}], keep_src = compaction
// sources ([committed] + [committed + 1 + accepted]), n_keep, and the next root token.
__global__ void accept_greedy_kernel(SsdTree t, const int* __restrict__ argmax, int committed, int* result,
                                     int* keep_src, int* n_keep, int* root_token, const int* pos_base) {
  if (threadIdx.x != 0) return;
  if (pos_base) committed += *pos_base;
  const int vn = t.vmeta[0];
  int cur = -1, n_acc = 0;
  int want;
  for (int step = 0; step <= TREE_MAXDEPTH; ++step) {  // one accepted node per depth at most
    want = argmax[cur + 1];
    int best = -1, best_rank = 0x7fffffff;
    for (int v = 0; v < vn; ++v)
      if (t.vparents[v] == cur && t.vtokens[v] == want && t.vranks[v] < best_rank) {
        best = v;
        best_rank = t.vranks[v];
      }
    if (best < 0) break;
    result[1 + n_acc] = t.vtokens[best];
    keep_src[1 + n_acc] = committed + 1 + best;
    ++n_acc;
    cur = best;
  }
  result[1 + n_acc] = want;
  result[0] = n_acc + 1;
  keep_src[0] = committed;
  *n_keep = n_acc + 1;
  *root_token = want;
}

// Start of a round: empty tree (level counts zero) and the root's draft row (position and slot
// root_pos = base + n_new[0] + pos_base[0], each term present when its pointer is; prefix
// root_pos + 1, no ancestors); the root token stays as the last round left it. With pos_base the
// new root position is stored back there: the round's other kernels read it as their base.
__global__ void round_begin_kernel(SsdTree t, SsdRows r, int base, const int32_t* n_new, int32_t* pos_base) {
  const int i = threadIdx.x;
  if (i < 1 + 2 * TREE_MAXDEPTH) t.meta[i] = 0;
  if (i == 0) {
    const int root_pos = base + (n_new ? n_new[0] : 0) + (pos_base ? pos_base[0] : 0);
    if (pos_base) pos_base[0] = root_pos;
    r.pos[0] = root_pos;
    r.slot[0] = root_pos;
    r.prefix[0] = root_pos + 1;
    r.depth[0] = 0;
  }
}

}  // namespace ssd

using namespace ssd;

SSD_API int ssd_round_begin(const SsdTree* tree, const SsdRows* root, int base, const int32_t* n_new,
                            int32_t* pos_base, hipStream_t stream) {
  if (!tree || !root || !tree->meta || !root->pos || root->cap < 1) return set_error(SSD_EINVAL, "round_begin: null");
  if (base < 0) return set_error(SSD_EINVAL, "round_begin: base %d < 0", base);
  SSD_LAUNCH(round_begin_kernel, dim3(1), dim3(128), 0, stream, *tree, *root, base, n_new, pos_base);
  return check_launch("round_begin");
}

SSD_API int ssd_tree_limits(int32_t* out) {
  if (!out) return set_error(SSD_EINVAL, "tree_limits: null");
  out[0] = TREE_CAP;
  out[1] = TREE_MAXDEPTH;
  out[2] = ROW_MAXD;
  return SSD_OK;
}

SSD_API int ssd_tree_level_topk(const SsdTree* tree, int d, const void* parts, int64_t parts_bytes, int N, int S,
                                const int32_t* vocab_ids, int F_max, int k, int width, int feed, int root_pos,
                                int tree_start, int past, const SsdRows* rows, int rows_max, const int32_t* pos_base,
                                hipStream_t stream) {
  if (!tree || !parts || (feed && !rows)) return set_error(SSD_EINVAL, "tree_level_topk: null pointer");
  if ((uintptr_t)parts & 7) return set_error(SSD_EINVAL, "tree_level_topk: parts must be 8-byte aligned");
  if (d < 0 || d >= TREE_MAXDEPTH || d + 1 > ROW_MAXD)
    return set_error(SSD_ERANGE, "tree_level_topk: depth %d too deep", d);
  if (F_max < 1 || k < 1 || k > TOPK_MAX || F_max * k > TREE_CAP)
    return set_error(SSD_ERANGE, "tree_level_topk: %d x %d candidates (k <= %d, total <= %d)", F_max, k, TOPK_MAX,
                     TREE_CAP);
  if (N < k || S < 1 || S > TOPK_MAX_PARTS || S > N || S * k > 64 * TOPK_MAX)
    return set_error(SSD_EINVAL, "tree_level_topk: N=%d with %d records of %d keys per row", N, S, k);
  if (parts_bytes < (int64_t)F_max * S * (int64_t)sizeof(TopkPart))
    return set_error(SSD_EINVAL, "tree_level_topk: partials of %lld bytes < %lld", (long long)parts_bytes,
                     (long long)F_max * S * (long long)sizeof(TopkPart));
  if (tree->cap > TREE_CAP || tree->cap < 1)
    return set_error(SSD_ERANGE, "tree_level_topk: capacity %d outside [1, %d]", tree->cap, TREE_CAP);
  if (feed && (rows_max > rows->cap || rows_max > TREE_CAP))
    return set_error(SSD_ERANGE, "tree_level_topk: rows_max too big");
  SsdRows r = feed ? *rows : SsdRows{};
  SSD_LAUNCH(tree_level_topk_kernel, dim3(1), dim3(1024), 0, stream, *tree, d, (const TopkPart*)parts, S, F_max,
             vocab_ids, k, width, feed, root_pos, tree_start, past, r, feed ? rows_max : 0, pos_base);
  return check_launch("tree_level_topk");
}

SSD_API int ssd_tree_level(const SsdTree* tree, int d, const int32_t* cand_tok, const float* cand_lp, int F_max,
                           int k, int width, int feed, int root_pos, int tree_start, int past, const SsdRows* rows,
                           int rows_max, const int32_t* pos_base, hipStream_t stream) {
  if (!tree || !cand_tok || !cand_lp || (feed && !rows)) return set_error(SSD_EINVAL, "tree_level: null pointer");
  if (d < 0 || d >= TREE_MAXDEPTH || d + 1 > ROW_MAXD) return set_error(SSD_ERANGE, "tree_level: depth %d too deep", d);
  if (F_max * k > TREE_CAP || k < 1) return set_error(SSD_ERANGE, "tree_level: %d x %d candidates > %d", F_max, k, TREE_CAP);
  if (tree->cap > TREE_CAP || tree->cap < 1)
    return set_error(SSD_ERANGE, "tree_level: capacity %d outside [1, %d]", tree->cap, TREE_CAP);
  if (feed && (rows_max > rows->cap || rows_max > TREE_CAP)) return set_error(SSD_ERANGE, "tree_level: rows_max too big");
  SsdRows r = feed ? *rows : SsdRows{};
  SSD_LAUNCH(tree_level_kernel, dim3(1), dim3(1024), 0, stream, *tree, d, cand_tok, cand_lp, k, width, feed,
                     root_pos, tree_start, past, r, feed ? rows_max : 0, pos_base);
  return check_launch("tree_level");
}

SSD_API int ssd_tree_finalize(const SsdTree* tree, int max_nodes, int committed, const int32_t* root_token,
                              const SsdRows* rows, int rows_max, const int32_t* pos_base, hipStream_t stream) {
  if (!tree || !root_token || !rows) return set_error(SSD_EINVAL, "tree_finalize: null pointer");
  if (tree->cap < 1) return set_error(SSD_EINVAL, "tree_finalize: tree capacity %d", tree->cap);
  if (rows_max > rows->cap || rows_max > TREE_CAP + 1 || tree->cap > TREE_CAP)
    return set_error(SSD_ERANGE, "tree_finalize: rows_max %d too big", rows_max);
  SSD_LAUNCH(tree_finalize_kernel, dim3(1), dim3(1024), 0, stream, *tree, max_nodes, committed, root_token,
                     *rows, rows_max, pos_base);
  return check_launch("tree_finalize");
}

SSD_API int ssd_accept_greedy(const SsdTree* tree, const int32_t* argmax, int committed, int32_t* result,
                              int32_t* keep_src, int32_t* n_keep, int32_t* root_token, const int32_t* pos_base,
                              hipStream_t stream) {
  if (!tree || !argmax || !result || !keep_src || !n_keep || !root_token)
    return set_error(SSD_EINVAL, "accept_greedy: null pointer");
  SSD_LAUNCH(accept_greedy_kernel, dim3(1), dim3(64), 0, stream, *tree, argmax, committed, result, keep_src,
                     n_keep, root_token, pos_base);
  return check_launch("accept_greedy");
}
