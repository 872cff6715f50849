/* C ABI of the MI355X (gfx950) speculative-decoding hot path: libssd_mi355x.so.
 *
 * Conventions
 *  - Every pointer argument is a device pointer unless stated; bf16 tensors are passed as
 *    uint16_t bit patterns; shapes are plain integers; strides are in elements.
 *  - Every entry point enqueues work on `stream` and returns 0 on success, or a nonzero
 *    code (1 bad argument, 2 beyond a compiled limit, 3 HIP runtime error) with a message
 *    from ssd_last_error(). No entry point allocates device memory or synchronises the
 *    host; workspaces are caller-provided.
 *  - Thread-compatible: concurrent calls on different streams must not share buffers.
 *
 * The reference (yotamabramson/subnetwork-speculative-decoding) is pure Python/PyTorch;
 * each function below replaces the PyTorch op call site cited beside it.
 */
#ifndef SSD_MI355X_H
#define SSD_MI355X_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif
#if defined(__GNUC__) || defined(__clang__)
#pragma GCC visibility push(default)
#endif

typedef struct ihipStream_t* hipStream_t;

/* ------------------------------------------------------------------ library */
const char* ssd_last_error(void);
int ssd_abi_version(void);
/* Kernels this library has enqueued since it was loaded (all devices and streams): the number
 * of launches a caller's step costs is the difference around it. No counterpart in the
 * reference. */
uint64_t ssd_launch_count(void);
/* Hash of the csrc/ and include/ sources the library was built from (16 hex digits; "unknown" for a
 * build without it); the Python package refuses a library whose hash differs from its sources. */
const char* ssd_build_hash(void);
int ssd_device_arch(char* buf, int len); /* host buffer; gcnArchName of the current device */

/* ------------------------------------------------------------ weight format
 * Packs a row-major bf16 matrix W[N_src, K] (row stride ld) into MFMA tiles: tile (nb, kb) =
 * rows row_map[16nb .. 16nb+16) x k [32kb, 32kb+32), 64 lanes x 8 bf16. N_packed is a multiple
 * of 128 (ssd_packed_weight_elems pads rows to 128 and K to 32). row_map[N_packed]
 * (device int32) names the source row of each packed row (-1 = zero row); it fuses q/k/v,
 * interleaves gate/up and pairs rotary dims. Tiles are stored in groups of `group` row tiles
 * per k-block ([nb / group][kb][nb % group]) so that a workgroup streams one contiguous region:
 * weights for ssd_gemm_bf16 / ssd_gemm_swiglu_bf16 / ssd_gemm_qkv_rope_bf16 use
 * group = ssd_gemm_weight_group(N, K); weights for ssd_gemm_partial_bf16 use group = 1.
 * Replaces holding nn.Linear weights as-is (ssd/models/subnetwork_draft.py:80-89 references HF
 * modules). */
int64_t ssd_packed_weight_elems(int N, int K);
int ssd_gemm_weight_group(int N, int K); /* 1, 2, 4 or 8; 0 on a bad shape */
/* col_scale [K] (may be NULL): each column k is multiplied by col_scale[k] and rounded once to
 * bf16 -- the RMSNorm weight folded into the projection that consumes the norm
 * (modeling_llama RMSNorm `weight * hidden` at :66-67; bridge RMSNorm ssd/models/bridges.py:33-37). */
int ssd_pack_weight_bf16(const uint16_t* src, int64_t ld, int N_src, int K, const int32_t* row_map, int N_packed,
                         int group, const uint16_t* col_scale, uint16_t* dst, hipStream_t stream);

/* ---------------------------------------------------------------- GEMMs
 * Y = act(X W^T + bias) [+ residual] with bf16 rounding after each step; Y may alias residual.
 * Replaces F.linear / nn.Linear at ssd/models/subnetwork_draft.py:243 (o_proj + residual),
 * :349 (lm_head and vocab-subset head) and the bridge linears ssd/models/bridges.py:53-54,131-135.
 * act: 0 none, 1 silu, 2 gelu, 3 relu. Batch-invariant: a row's result does not depend on M.
 * norm_eps > 0 folds the RMSNorm that precedes the projection (modeling_llama.py:53-67,
 * ssd/models/bridges.py:27-37): X is the un-normalised residual stream h, W was packed with the
 * norm weight as col_scale, and every output of row m is scaled by rsqrt(mean(h_m^2) + norm_eps)
 * (the row's sum of squares is accumulated from the X fragments the GEMM streams anyway).
 * norm_eps = 0: plain GEMM. The same flag exists on the SwiGLU and q/k/v GEMMs. */
int ssd_gemm_bf16(const uint16_t* X, int64_t ldx, int M, const uint16_t* W_packed, int N, int K, float norm_eps,
                  uint16_t* Y, int64_t ldy, const uint16_t* bias, int act, const uint16_t* residual, int64_t ldr,
                  hipStream_t stream);

/* The vocabulary head fused with its per-row top-k chunk pass: the draft head's logits
 * (ssd/models/subnetwork_draft.py:345-349) reduced in the GEMM's epilogue to the records that the
 * proposal's top-k (ssd/engine/tree_drafter.py:129-133) merges, so the logits never make a round trip
 * through memory. parts (8-byte aligned, >= M * ssd_gemm_topk_parts(N) * 136 bytes) gets, for row m
 * and slab s (consecutive 128-column groups, the slabs a function of N only), the slab's k best
 * (value, column) keys of the bf16-rounded logits, its maximum and (mode 1) its sum of exp(x - max);
 * merge them with ssd_tree_level_topk or ssd_row_topk_merge (S = ssd_gemm_topk_parts(N), the same
 * k: records are stored packed for k, 8 + 8 k bytes each). The keys
 * are exact; the sums of exp differ from ssd_row_topk_partial_bf16's only in summation order.
 * W_packed as for ssd_gemm_bf16 (tiles grouped by ssd_gemm_weight_group(N, K)). Y (NULL or ldy >= N)
 * also receives the logits, bit-identical to ssd_gemm_bf16's for N >= 65536.
 * k in [1, 16], mode 0 (raw values) or 1 (log-softmax). */
int ssd_gemm_topk_parts(int N);
int ssd_gemm_topk_bf16(const uint16_t* X, int64_t ldx, int M, const uint16_t* W_packed, int N, int K,
                       float norm_eps, int k, int mode, void* parts, int64_t parts_bytes, uint16_t* Y, int64_t ldy,
                       hipStream_t stream);

/* Y[M, I] = silu(X Wg^T + bg) * (X Wu^T + bu), gate/up interleaved per 16-row tile.
 * Replaces LlamaMLP's gate/up/act (modeling_llama MLP called at ssd/models/subnetwork_draft.py:245)
 * and the swiglu bridge (ssd/models/bridges.py:57-65). */
int ssd_gemm_swiglu_bf16(const uint16_t* X, int64_t ldx, int M, const uint16_t* W_packed, int I, int K,
                         float norm_eps, uint16_t* Y, int64_t ldy, const uint16_t* bias_gate,
                         const uint16_t* bias_up, hipStream_t stream);

/* q/k/v projection + RoPE + KV-cache write, fused. Replaces ssd/models/subnetwork_draft.py:209-222
 * (q/k/v_proj, rotate_half RoPE, KVCache.update at ssd/engine/kv_cache.py:32-43). Row m is at
 * rotary position row_pos[m] (cos/sin tables [rope_rows, hd/2]) and writes cache slot row_slot[m]
 * (rows whose slot is outside [0, max_len) are not written); K and V go to the cache block layout
 * below. */
int ssd_gemm_qkv_rope_bf16(const uint16_t* X, int64_t ldx, int M, const uint16_t* W_packed, int K, float norm_eps,
                           int heads, int kv_heads, int head_dim, const uint16_t* cos_tab, const uint16_t* sin_tab,
                           int64_t rope_rows, const int32_t* row_pos, const int32_t* row_slot, uint16_t* Q, int64_t ldq,
                           uint16_t* k_cache, uint16_t* vt_cache, int64_t max_len, hipStream_t stream);

/* ---------------------------------------------------------- split-K GEMMs
 * For narrow outputs (o_proj, down_proj, q/k/v, bridge out_proj) K is split over workgroups
 * (weights packed with group 1):
 * P[s][m][n] = sum over the s-th K range of X W^T in fp32, s < ssd_gemm_splits(N, K) (a function
 * of the shape only, so results stay batch-invariant). P: 16-byte aligned fp32, row stride
 * ldp >= N rounded up to 64 (multiple of 4), split stride >= M * ldp. A consumer sums the S
 * partials in order s = 0..S-1 and applies the epilogue of the op it replaces. */
int ssd_gemm_splits(int N, int K);
int ssd_gemm_partial_bf16(const uint16_t* X, int64_t ldx, int M, const uint16_t* W_packed, int N, int K, float* P,
                          int64_t ldp, int64_t split_stride, hipStream_t stream);
/* The ssd_gemm_bf16 epilogue (bias, activation, residual; Y may alias residual) over S partials. */
int ssd_gemm_finalize_bf16(const float* P, int64_t ldp, int64_t split_stride, int S, int M, int N, uint16_t* Y,
                           int64_t ldy, const uint16_t* bias, int act, const uint16_t* residual, int64_t ldr,
                           hipStream_t stream);
/* The RoPE + KV-cache-write epilogue of ssd_gemm_qkv_rope_bf16 over S partials of the packed q/k/v
 * projection (ssd/models/subnetwork_draft.py:209-222). */
int ssd_qkv_rope_finalize_bf16(const float* P, int64_t ldp, int64_t split_stride, int S, int M, int heads,
                               int kv_heads, int head_dim, const uint16_t* cos_tab, const uint16_t* sin_tab,
                               int64_t rope_rows, const int32_t* row_pos, const int32_t* row_slot, uint16_t* Q,
                               int64_t ldq, uint16_t* k_cache, uint16_t* vt_cache, int64_t max_len, hipStream_t stream);
/* Residual add of a projection's partials, then the next RMSNorm (ssd/models/subnetwork_draft.py:243-245,
 * ssd/models/bridges.py:131-135):  h <- bf16(h + bf16(sum_s P[s] + bias));  y <- w * bf16(h * rsqrt(mean(h^2)
 * + eps)). S = 0: y = RMSNorm(h) only; y = NULL: residual update only. D = row length (P's N). */
int ssd_add_rmsnorm_bf16(const float* P, int64_t ldp, int64_t split_stride, int S, const uint16_t* bias, uint16_t* h,
                         int64_t ldh, int M, int D, const uint16_t* w, float eps, uint16_t* y, int64_t ldy,
                         hipStream_t stream);
/* Projection + residual add (ssd/models/subnetwork_draft.py:243, :245 residual adds;
 * ssd/models/bridges.py:131-135 bridge residual): h[:M] <- bf16(h + bf16(X W^T + bias)). By shape:
 * one direct GEMM with the add in its epilogue, or (long K) split-K partials plus a finalize that
 * adds -- W packed with group = ssd_gemm_residual_group(N, K); part: fp32 scratch of
 * ssd_gemm_residual_floats(M, N, K) floats (0 when the direct form is used). */
int ssd_gemm_residual_group(int N, int K);
int64_t ssd_gemm_residual_floats(int M, int N, int K);
int ssd_gemm_residual_bf16(const uint16_t* X, int64_t ldx, int M, const uint16_t* W_packed, int N, int K,
                           const uint16_t* bias, uint16_t* h, int64_t ldh, float* part, int64_t part_floats,
                           hipStream_t stream);

/* Decoder MLP with its RMSNorm and residual add, fused into one launch of 256 workgroups (one per
 * CU; the workgroups wait on each other's flags, so the device must hold all of them at once,
 * which is checked per kernel instantiation before the first launch):
 * h[:M] <- bf16(h + bf16(down(act))), act = bf16(silu(bf16(g))) * bf16(u) rounded to
 * bf16, [g | u] = RMSNorm(h) . Wgu^T. Replaces the post-attention half of the decoder layer
 * (ssd/models/subnetwork_draft.py:244-246: post_attention_layernorm, LlamaMLP, residual add).
 * ssd_mlp_group(I, H) = the packing group of Wgu for this path (gate/up interleaved per 16-row
 * tile, ln2 folded in as col_scale), 0 when the shape has no fused plan; Wd is packed with
 * group ssd_gemm_residual_group(H, I). act: [M][lda] bf16 scratch (lda >= I); part: fp32 scratch
 * of ssd_gemm_residual_floats(min(M, 64), H, I) floats; sync: ssd_mlp_sync_words() uint32 words,
 * zero before the first call and then left to the kernel. Word ssd_mlp_timeout_word() counts
 * flag waits that gave up (a workgroup another process kept off the GPU): nonzero means the
 * results of every call since it was last zero are invalid, and the caller must check it (the
 * waits are bounded, so a failure never hangs). Calls sharing sync must run in stream order; the
 * call count is kept in the flags themselves, so a launch captured in a HIP graph replays
 * correctly. */
int ssd_mlp_group(int I, int H);
int64_t ssd_mlp_sync_words(void);
int ssd_mlp_timeout_word(void); /* index of the timeout count in sync */
int ssd_mlp_bf16(uint16_t* h, int64_t ldh, int M, const uint16_t* Wgu_packed, const uint16_t* Wd_packed, int I, int H,
                 float eps, uint16_t* act, int64_t lda, float* part, int64_t part_floats, uint32_t* sync,
                 hipStream_t stream);

/* ------------------------------------------------------------ KV-cache layout
 * k_cache / vt_cache (one layer, as passed to the q/k/v GEMM and the attention; the compaction
 * takes all layers back to back) are kv_heads regions of max_len * head_dim bf16 each, max_len a
 * multiple of 64 and head_dim a multiple of 32. A region is a sequence of 64-slot blocks, each
 * stored as the tree-attention MFMA operands in lane order (64 lanes x 8 bf16 per 1 KiB tile):
 *   K[s][d] at ((((s/64)*4 + kt)*(hd/32) + d/32)*64 + ((d/8)%4)*16 + i)*8 + d%8, with o = s%64,
 *     kt = (o/32)*2 + (o/4)%2, i = ((o/8)%4)*4 + o%4;
 *   V[s][d] at ((((s/64)*(hd/16) + d/16)*2 + o/32)*64 + ((o/8)%4)*16 + d%16)*8 + o%8.
 * (Python: ssd.ops.kv_block_index / kv_tile / kv_untile.) The attention reads every tile of a
 * block as one contiguous 1 KiB load; the reference's cache is [1, kv_heads, max_len, hd] per
 * layer (ssd/engine/kv_cache.py:38-43). */

/* ------------------------------------------------------------ tree attention
 * Row t attends cache slots [0, prefix[t]) then anc[t][0..depth[t]) (ancestors in depth order,
 * self included), i.e. the reference's boolean tree mask (ssd/models/subnetwork_draft.py:165-191,
 * ssd/engine/verify.py:37-41, ssd/engine/tree_drafter.py:189-196) as a gather list. Replaces the
 * SDPA call at ssd/models/subnetwork_draft.py:236-241 (GQA, scale 1/sqrt(hd)). Keys are folded in
 * a canonical logical order, so a verify row equals the autoregressive step at its position. */
int ssd_attn_workspace_floats(int M, int heads, int head_dim, int64_t max_len);
int ssd_attn_max_depth(void);
int ssd_tree_attention_bf16(const uint16_t* q, int64_t ldq, int M, int heads, int kv_heads, int head_dim,
                            const uint16_t* k_cache, const uint16_t* vt_cache, int64_t max_len,
                            const int32_t* prefix, const int32_t* depth, const int32_t* anc, int p_min, int l_max,
                            float scale, float* ws, int64_t ws_floats, uint16_t* out, int64_t ldo,
                            hipStream_t stream);

/* ---------------------------------------------------------------- rows */
/* HF LlamaRMSNorm / bridge RMSNorm (ssd/models/bridges.py:33-37; subnetwork_draft.py:216,245,344). */
int ssd_rmsnorm_bf16(const uint16_t* x, int64_t ldx, int M, int D, const uint16_t* w, float eps, uint16_t* y,
                     int64_t ldy, hipStream_t stream);
/* embed_tokens gather (ssd/models/subnetwork_draft.py:290-291). */
int ssd_embed_bf16(const int32_t* ids, int M, const uint16_t* table, int64_t V, int D, uint16_t* out, int64_t ldo,
                   hipStream_t stream);
/* KVCache.keep_positions (ssd/engine/kv_cache.py:54-70): move src[0..*n_dev) to [start, ...) in every
 * layer in one launch; all sources are read before any destination is written. pos_base (NULL or a
 * device word): start is relative to *pos_base, read on the device (a destination range outside
 * the cache then moves nothing). */
int ssd_kv_compact_bf16(uint16_t* k_arena, uint16_t* vt_arena, int layers, int kv_heads, int head_dim,
                        int64_t max_len, int start, const int32_t* src, const int32_t* n_dev, int n_max,
                        const int32_t* pos_base, hipStream_t stream);
/* Row top-k over bf16 logits. mode 0: raw values (k=1 is the first-index argmax of
 * ssd/engine/verify.py:47, speculative.py:83). mode 1: log_softmax values + logsumexp
 * (ssd/engine/tree_drafter.py:129-133); columns map through vocab_ids (subset head,
 * ssd/models/subnetwork_draft.py:136-144). Equal values rank lower column first. Each row is scanned
 * in 4096-column chunks by separate workgroups, merged in a fixed order; workspace of
 * ssd_row_topk_ws_bytes(M, N) bytes. */
int64_t ssd_row_topk_ws_bytes(int M, int N);
int ssd_row_topk_bf16(const uint16_t* logits, int64_t ld, int M, int N, int k, int mode, const int32_t* vocab_ids,
                      int32_t* out_tok, float* out_val, float* out_lse, void* ws, int64_t ws_bytes,
                      hipStream_t stream);
/* ssd_row_topk_bf16 without the workspace argument: no counterpart in the reference; for callers
 * that cannot allocate device memory (code under HIP graph capture, serving loops or harnesses
 * that forbid hipMalloc). The chunk partials live in a static device array of the library, one
 * per GPU (544 KiB, held until the process ends): M * ceil(N / 4096) must be <= 4096 (e.g. 64
 * rows of a 128256-column vocabulary), larger calls fail with code 2. The call allocates nothing
 * and needs nothing cleared. All calls on one GPU share that array: calls that overlap in time on
 * one GPU (other streams or threads) race and must be serialised by the caller. Results are
 * bit-identical to ssd_row_topk_bf16. */
int ssd_row_topk_bf16_noalloc(const uint16_t* logits, int64_t ld, int M, int N, int k, int mode,
                              const int32_t* vocab_ids, int32_t* out_tok, float* out_val, float* out_lse,
                              hipStream_t stream);
/* The chunk pass of ssd_row_topk_bf16 alone: fills ws (ssd_row_topk_ws_bytes(M, N) bytes) with each
 * row's 4096-column chunk records, for ssd_tree_level_topk to merge (the first half of the
 * proposal step, ssd/engine/tree_drafter.py:129-133). */
int ssd_row_topk_partial_bf16(const uint16_t* logits, int64_t ld, int M, int N, int k, int mode, void* ws,
                              int64_t ws_bytes, hipStream_t stream);
/* The merge pass of ssd_row_topk_bf16 alone, over S records per row (S = ceil(N / 4096) from
 * ssd_row_topk_partial_bf16, ssd_gemm_topk_parts(N) from ssd_gemm_topk_bf16; S <= 256 and
 * S * k <= 1024): out_tok[M * k], out_val (NULL or M * k), out_lse (NULL or M, mode 1). */
int ssd_row_topk_merge(const void* parts, int64_t parts_bytes, int M, int S, int k, int mode,
                       const int32_t* vocab_ids, int32_t* out_tok, float* out_val, float* out_lse,
                       hipStream_t stream);

/* ------------------------------------------------------------------ tree
 * Device-resident DraftTree (ssd/engine/tree_drafter.py:48-95). All members are device
 * pointers of `cap` entries except meta (1 + 2*32 ints) and vmeta (1 int). */
typedef struct SsdTree {
  int32_t* tokens;
  int32_t* parents;
  int32_t* depths;
  int32_t* ranks;
  int32_t* draft_pos;
  double* scores;
  int32_t* meta; /* [0] nodes, [1+d] level start, [33+d] level size */
  int32_t* vtokens;
  int32_t* vparents;
  int32_t* vdepths;
  int32_t* vranks;
  int32_t* vorig;
  int32_t* vmeta; /* [0] verify nodes */
  int32_t cap;
} SsdTree;

/* Per-row inputs of one forward: token ids, rotary positions, cache slots, and the
 * attention rows (prefix, depth, anc[cap][32]); with kv_off, each row reads and writes the KV
 * arena of its own sequence (every sequence's arena has the layout and capacity of SsdBuffers'). */
typedef struct SsdRows {
  int32_t* ids;
  int32_t* pos;
  int32_t* slot;
  int32_t* prefix;
  int32_t* depth;
  int32_t* anc;
  int32_t cap;
  const int64_t* kv_off;  /* [cap] element offset of each row's sequence in the KV arenas (rows of several
                             sequences in one forward: batched generation), or NULL (one sequence) */
} SsdRows;

int ssd_tree_limits(int32_t* out3); /* host: {node capacity, max depth, max ancestors per row} */

/* Start of a draft phase (ssd/engine/tree_drafter.py:147-160: a fresh DraftTree and the root fed
 * at root_pos): tree level counts to zero and root row 0 = position/slot root_pos, prefix
 * root_pos + 1, depth 0, on the device (no host copy). root_pos = base + n_new[0] + pos_base[0],
 * read on the device (n_new: the committed count of the previous round's record; pos_base: a
 * device word holding the previous round's root position; either may be NULL), so a round can
 * start before the host has read the previous one. With pos_base, root_pos is stored back into
 * *pos_base: the round's other calls given the same pos_base take their positions relative to
 * it, so the whole round has no host-side position and can be captured once and replayed. */
int ssd_round_begin(const SsdTree* tree, const SsdRows* root, int base, const int32_t* n_new, int32_t* pos_base,
                    hipStream_t stream);

/* One level of TreeDrafter.build (ssd/engine/tree_drafter.py:165-200): candidates of the current
 * frontier (cand_tok/cand_lp [F, k]; tok < 0 = none) -> score = parent score + lp, stable sort,
 * width cut, append; if feed, write the next draft forward's rows (positions root_pos+d+1, slots
 * past+j, prefix tree_start, ancestors' draft slots). pos_base (NULL or a device word): root_pos,
 * tree_start and past are relative to *pos_base. */
int ssd_tree_level(const SsdTree* tree, int d, const int32_t* cand_tok, const float* cand_lp, int F_max, int k,
                   int width, int feed, int root_pos, int tree_start, int past, const SsdRows* rows, int rows_max,
                   const int32_t* pos_base, hipStream_t stream);
/* ssd_tree_level whose candidates are merged in the same launch from the F_max rows of S records
 * each that ssd_row_topk_partial_bf16 (S = ceil(N / 4096)) or ssd_gemm_topk_bf16 (S =
 * ssd_gemm_topk_parts(N)) left in parts (k, mode 1: log-softmax; S <= 256, S * k <= 1024): the
 * greedy proposal's merge (ssd/engine/tree_drafter.py:129-133) and the level expansion (:165-183) in
 * one launch; identical results to ssd_row_topk_bf16 followed by ssd_tree_level.
 * N: the logits' columns; vocab_ids as for ssd_row_topk_bf16 (null: identity). */
int ssd_tree_level_topk(const SsdTree* tree, int d, const void* parts, int64_t parts_bytes, int N, int S,
                        const int32_t* vocab_ids, int F_max, int k, int width, int feed, int root_pos, int tree_start,
                        int past, const SsdRows* rows, int rows_max, const int32_t* pos_base, hipStream_t stream);

/* max_nodes cut by (-score, depth), ancestor closure and renumbering (ssd/engine/tree_drafter.py:202-207),
 * then the verify rows of verify_inputs (ssd/engine/verify.py:32-42); root token read from device.
 * pos_base (NULL or a device word): committed is relative to *pos_base. */
int ssd_tree_finalize(const SsdTree* tree, int max_nodes, int committed, const int32_t* root_token,
                      const SsdRows* rows, int rows_max, const int32_t* pos_base, hipStream_t stream);

/* greedy_verify (ssd/engine/verify.py:45-57) plus the bookkeeping of speculative.py:166-171:
 * result = [n_new, tokens...], keep_src/n_keep for ssd_kv_compact_bf16, next root token.
 * pos_base (NULL or a device word): committed is relative to *pos_base. */
int ssd_accept_greedy(const SsdTree* tree, const int32_t* argmax, int committed, int32_t* result,
                      int32_t* keep_src, int32_t* n_keep, int32_t* root_token, const int32_t* pos_base,
                      hipStream_t stream);

/* ---------------------------------------------------------------- sampling
 * Randomness is Philox4x32-10 keyed by a 64-bit seed; `counter` separates draws (one value per
 * round / decode step). Reproducible for a given (seed, counter), independent of launch shape.
 * Rows are processed in 4096-column chunks (one workgroup each); chunk results meet in a
 * caller workspace of ssd_sample_ws_bytes(rows, columns) bytes (no clearing needed). */
int ssd_sample_limits(int32_t* out2); /* host: {max children per node / draws per row, max columns} */
int64_t ssd_sample_ws_bytes(int rows, int n);

/* warp_probs (ssd/engine/tree_drafter.py:34-45) and the scatter of a draft-vocab subset back to
 * the full vocabulary (tree_drafter.py:134-137): probs[r][V] fp32 = softmax(logits / T), and with
 * top_p < 1 only the entries whose preceding (descending) mass is <= top_p, renormalised; equal
 * logits rank lower column first. vocab_ids (n columns -> tokens, with vocab_inv[V] the inverse,
 * -1 outside) may be NULL when n == V. With tree_meta, the rows are the frontier that proposes
 * `level` and row f is written at probs row 1 + (start of level-1) + f (row 0 for the root) so
 * each tree node keeps the q its children were drawn from. */
int ssd_warp_probs_bf16(const uint16_t* logits, int64_t ld, int rows, int n, const int32_t* vocab_ids,
                        const int32_t* vocab_inv, int V, float temperature, float top_p, const int32_t* tree_meta,
                        int level, float* probs, int64_t ldp, void* ws, int64_t ws_bytes, hipStream_t stream);

/* _propose, sampling branch (ssd/engine/tree_drafter.py:138-144): per row of q, min(k, |support|)
 * tokens without replacement in draw order (largest q(y)/E(y), E ~ Exp(1)) and their log q;
 * out_tok[r][k] is -1 past the support. tree_meta/level address q rows as ssd_warp_probs_bf16. */
int ssd_gumbel_topk(const float* probs, int64_t ldp, int rows, int V, int k, const int32_t* tree_meta, int level,
                    uint64_t seed, uint64_t counter, int32_t* out_tok, float* out_lp, void* ws, int64_t ws_bytes,
                    hipStream_t stream);

/* torch.multinomial(p, 1) per row (ssd/engine/speculative.py:81-84): a categorical draw from
 * each nonnegative row (need not be normalised). */
int ssd_sample_rows(const float* probs, int64_t ldp, int rows, int V, uint64_t seed, uint64_t counter,
                    int32_t* out_tok, void* ws, int64_t ws_bytes, hipStream_t stream);

/* sample_next at temperature > 0 (ssd/data/generate_selfdistill.py:50-60): per row of bf16 logits,
 * the 64 largest values (equal values: lower column first), warp_probs over those 64 alone
 * (softmax(v / T), an entry dropped when the fp32 cumulative mass before it exceeds top_p), one
 * categorical draw among them; out_tok[r] is the drawn column. Needs 64 <= V <= 262144 (the
 * reference's topk(64) needs V >= 64), temperature > 0, top_p > 0, and a workspace of
 * ssd_sample_top64_ws_bytes(rows, V) bytes, 8-byte aligned. */
int64_t ssd_sample_top64_ws_bytes(int rows, int V);
int ssd_sample_top64_bf16(const uint16_t* logits, int64_t ld, int rows, int V, float temperature, float top_p,
                          uint64_t seed, uint64_t counter, int32_t* out_tok, void* ws, int64_t ws_bytes,
                          hipStream_t stream);

/* sample_verify (ssd/engine/verify.py:60-95) over the finalized tree plus the bookkeeping of
 * ssd_accept_greedy. P[rows][V]: warped target rows (row 0 root, 1 + v verify node v; rows <= 64);
 * Q: warped draft rows as written by ssd_warp_probs_bf16 with tree_meta (row 1 + draft index).
 * max_kids: the most children any node has (<= 16); that many rejection passes are launched. */
int ssd_accept_sample(const SsdTree* tree, const float* P, int64_t ldp, const float* Q, int64_t ldq, int V,
                      int rows, int max_kids, uint64_t seed, uint64_t counter, void* ws, int64_t ws_bytes,
                      int committed, int32_t* result, int32_t* keep_src, int32_t* n_keep, int32_t* root_token,
                      hipStream_t stream);

/* Batched acceptance trials for the statistical check of the acceptance rule at scale (no
 * counterpart in the reference, whose loop is verify.py:60-95 on the CPU): `trials` independent
 * rounds over fixed per-node distributions P / Q ([rows][ld] fp32; row 0 the root, row 1 + v node v
 * of the unpruned tree with branch[d] children per level-d node, numbered level by level, children
 * in draw order), each drawing its children on the walk by Gumbel top-k and accepting / rejecting
 * exactly as ssd_gumbel_topk + ssd_accept_sample would with round counter counter0 + trial.
 * cols / col_off: per-row support (CSR, ascending columns where P or Q > 0). Outputs per trial:
 * out_tokens[trial][depth + 1] (accepted tokens, then the bonus) and out_n[trial]. */
int ssd_accept_sample_trials(const float* P, int64_t ldp, const float* Q, int64_t ldq, int rows, const int32_t* cols,
                             const int32_t* col_off, int depth, const int32_t* branch, uint64_t seed,
                             uint64_t counter0, int trials, int32_t* out_tokens, int32_t* out_n, hipStream_t stream);

/* ---------------------------------------------------------------- forward
 * Descriptors of one model forward; every pointer is device memory in the formats above
 * (weights packed by ssd_pack_weight_bf16). Host structs, read during the call only. */
typedef struct SsdLayerW {    /* one decoder layer */
  const uint16_t* wqkv;       /* q/k/v fused, rotary-paired rows, ln1 folded in (col_scale) */
  const uint16_t* wo;
  const uint16_t* wgu;        /* gate/up interleaved per 16-row tile, ln2 folded in */
  const uint16_t* wd;
  const uint16_t* ln1;        /* input RMSNorm weight [hidden] */
  const uint16_t* ln2;        /* post-attention RMSNorm weight [hidden] */
} SsdLayerW;

typedef struct SsdModel {     /* base model shared by target and draft */
  int32_t hidden, heads, kv_heads, head_dim, inter, vocab, n_layers;
  float eps, attn_scale;
  const uint16_t* embed;      /* [vocab][hidden] row-major */
  const uint16_t* norm;       /* final RMSNorm weight */
  const uint16_t* cos;        /* bf16 rotary tables [rope_rows][head_dim/2] */
  const uint16_t* sin;
  int64_t rope_rows;
  const SsdLayerW* layers;    /* host array [n_layers] */
  int32_t mlp_fused;          /* 1: wgu packed with group ssd_mlp_group(inter, hidden) -> ssd_mlp_bf16 */
} SsdModel;

typedef struct SsdBridgeW {   /* x + MLP(RMSNorm(x)) */
  const uint16_t* norm;
  float eps;
  int32_t hidden, swiglu, n_body;
  const uint16_t* body_w[2];  /* plain MLP: n_body linears with bias + activation; the norm is
                                 folded into body_w[0] (or into gu for swiglu) */
  const uint16_t* body_b[2];
  int32_t body_n[2], body_act[2];
  const uint16_t* gu;         /* swiglu: packed gate/up and biases */
  const uint16_t* bg;
  const uint16_t* bu;
  const uint16_t* out;        /* output projection [hidden -> model hidden] and bias */
  const uint16_t* out_b;
} SsdBridgeW;

typedef struct SsdPlan {      /* which layers run, with which bridges, and which head */
  int32_t n_steps;
  const int32_t* layer_ids;          /* host [n_steps] */
  const SsdBridgeW* const* pre_bridge; /* host [n_steps], NULL entries = none; NULL = no bridges */
  const SsdBridgeW* pre_norm;        /* bridge before the final norm, or NULL */
  const uint16_t* head_w;            /* packed lm_head (full or vocabulary subset) with the final
                                        norm folded in, or NULL */
  int32_t head_n;
} SsdPlan;

typedef struct SsdBuffers {   /* activations [m_cap][...] and the layer-major KV arena */
  uint16_t *h, *x, *q, *attn, *mlp, *mid0, *mid1;
  int32_t m_cap, mid_cols;
  uint16_t* k_arena;          /* [n_layers][kv_heads][cache_cap * head_dim], 64-slot block layout */
  uint16_t* vt_arena;         /* [n_layers][kv_heads][cache_cap * head_dim], 64-slot block layout */
  int64_t cache_cap;
  float* attn_ws;
  int64_t attn_ws_floats;
  uint16_t* logits;           /* [head_rows][ld_logits] */
  int64_t ld_logits;
  float* part;                /* split-K partials of one GEMM (fp32) */
  int64_t part_floats;
  uint32_t* sync;             /* ssd_mlp_sync_words() words, zeroed once (used when mlp_fused) */
} SsdBuffers;

/* Embedding, the plan's decoder layers with their bridges, final norm and the head over rows
 * [head_first, head_first + head_rows) — one call per forward (m <= m_cap rows, attention rows
 * as for ssd_tree_attention_bf16). Replaces SubnetworkDraftModel.forward
 * (ssd/models/subnetwork_draft.py:249-358, layer body :193-246) and the target's forward. */
int ssd_forward(const SsdModel* model, const SsdPlan* plan, const SsdBuffers* buf, const SsdRows* rows, int m,
                int p_min, int l_max, int head_first, int head_rows, hipStream_t stream);

/* ---- Prefill: the target's forward over a long prompt chunk (reference
 * ssd/engine/speculative.py:149-151, the target called on the prompt; its layers
 * ssd/models/subnetwork_draft.py:193-246). Compute-bound MFMA GEMMs tiled 128 x 128 through LDS
 * and causal flash attention; rows are prompt positions pos0 .. pos0 + m - 1 written to cache
 * slots of the same index. Results match the decode kernels within bf16 rounding (not bit for
 * bit); greedy speculative and greedy autoregressive decoding share one prefill. */
#define SSD_EPI_STORE 0   /* Y = XW^T (+ residual) */
#define SSD_EPI_SWIGLU 1  /* Y[:, i] = silu(gate_i) * up_i, gate/up interleaved 8 + 8 rows per tile */
#define SSD_EPI_QKV 2     /* q -> Y with RoPE; k (RoPE), v -> the cache at slot pos0 + row */

typedef struct SsdQkvEpilogue {
  int32_t heads, kv_heads, head_dim;
  const uint16_t* cos;        /* bf16 rotary tables [rope_rows][head_dim/2] */
  const uint16_t* sin;
  int64_t rope_rows;
  int32_t pos0;               /* position (= cache slot) of row 0 */
  uint16_t* k_cache;          /* this layer: kv_heads x (max_len x head_dim), 64-slot block layout */
  uint16_t* vt_cache;
  int64_t max_len;
} SsdQkvEpilogue;

/* Row scales of an RMSNorm folded into a prefill GEMM's packed weight (the LlamaRMSNorm before the
 * target layers' q/k/v and gate/up projections, ssd/models/subnetwork_draft.py:209-212, :243-245):
 * row_scale[m] = rsqrt(mean(X[m, :K]^2) + eps), [M] floats; K % 8 == 0, 16-byte rows. */
int ssd_prefill_row_scale_bf16(const uint16_t* X, int64_t ldx, int M, int K, float eps, float* row_scale,
                               hipStream_t stream);

/* Y = epilogue(X[M, K] W^T) for any M (W packed by ssd_pack_weight_bf16 with `group`, K % 64 == 0);
 * row_scale ([M] floats from ssd_prefill_row_scale_bf16, or NULL) multiplies row m's products, which
 * with the RMSNorm weight folded into W's columns is the RMSNorm of X's rows. Replaces the
 * prompt-length F.linear / nn.Linear calls of the target layers (ssd/models/subnetwork_draft.py:209-212,
 * :243-245). */
int ssd_prefill_gemm_bf16(const uint16_t* X, int64_t ldx, int M, const uint16_t* W_packed, int group, int N, int K,
                          const float* row_scale, int epi, uint16_t* Y, int64_t ldy, const uint16_t* residual,
                          int64_t ldr, const SsdQkvEpilogue* qkv, hipStream_t stream);

/* Causal attention of prompt rows: row t (position pos0 + t) attends cache slots [0, pos0 + t],
 * scale * q.k, GQA (heads / kv_heads q heads per kv head). Replaces the causal SDPA of the prompt
 * forward (ssd/models/subnetwork_draft.py:236-241 with no tree mask). head_dim 64 or 128. */
int ssd_prefill_attention_bf16(const uint16_t* q, int64_t ldq, int M, int pos0, int heads, int kv_heads,
                               int head_dim, const uint16_t* k_cache, const uint16_t* vt_cache, int64_t max_len,
                               float scale, uint16_t* out, int64_t ldo, hipStream_t stream);

typedef struct SsdPrefillBuffers {  /* activations [m_cap][...] and the KV arena */
  int32_t m_cap;
  uint16_t *h, *q, *attn, *act;     /* [m_cap][hidden], [m_cap][heads*hd] x 2, [m_cap][inter] */
  uint16_t* k_arena;                /* as SsdBuffers */
  uint16_t* vt_arena;
  int64_t cache_cap;
  uint16_t* logits;                 /* [vocab]: the last row's logits */
} SsdPrefillBuffers;

/* The whole target forward over rows [pos0, pos0 + m), m <= m_cap, in one call; head_w (the packed
 * full lm_head with the final norm folded, NULL = no head) gives the last row's logits. */
int ssd_prefill(const SsdModel* model, const uint16_t* head_w, const SsdPrefillBuffers* buf, const int32_t* ids,
                int m, int pos0, hipStream_t stream);

#if defined(__GNUC__) || defined(__clang__)
#pragma GCC visibility pop
#endif
#ifdef __cplusplus
}
#endif

#endif /* SSD_MI355X_H */
