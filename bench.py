"""Benchmark: speculative decoding rounds of a Llama-3-8B-shaped bf16 model on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME] [--no-cpu]

A *step* is one speculative round (draft tree -> verify -> commit) of the hot path. The
workload (default ``llama3_8b_tree``): random-init Llama-3-8B shapes (hidden 4096, 32 layers,
32/8 heads, head_dim 128, SwiGLU 14336, vocab 128256) in bf16, draft_layers [0, 15, 31] with
two untrained bridges, tree depth 4 / branch [3, 2, 2, 1] / max_nodes 24, greedy, a 4096-token
uniform random prompt, full-vocabulary draft head. W untimed rounds, then exactly K timed
rounds bracketed by device synchronisation. ``value`` = committed tokens / timed seconds.

Per-kernel figures are measured live with HIP events on the launch stream (same shapes as in
the timed rounds: verify M = 25 rows at the reached context). ``cpu_baseline`` times the CPU
oracle (this repo's PyTorch restatement of the reference path) on the host cores for a few
rounds of the same model shape and tree after a shortened prompt.

Prints one JSON line. More than one GPU is not supported: --gpus > 1 exits.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
for _p in (REPO, os.path.join(REPO, "subnetwork-speculative-decoding_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
METRIC = "decode tokens/s + ms/round, Llama-3-8B bf16 tree spec; tree-attn HBM GB/s"

WORKLOADS = {
    # name: (shape, draft_layers, drafting kwargs, prompt, draft_vocab)
    "llama3_8b_tree": ("llama3_8b", [0, 15, 31], dict(depth=4, branch=[3, 2, 2, 1], max_nodes=24), 4096, None),
    "llama3_8b_c": ("llama3_8b", [0, 15, 31], dict(depth=6, branch=[4, 2, 2, 1, 1, 1], max_nodes=32), 4096, None),
    "llama32_1b_b": ("llama32_1b", [0, 7, 15], dict(depth=4, branch=[3, 2, 2, 1], width=8, max_nodes=24), 512, 32768),
    "llama3_8b_sampled": ("llama3_8b", [0, 15, 31], dict(depth=3, branch=[3, 2, 1], temperature=0.7, top_p=0.9),
                          4096, None),
    "llama3_70b_tree": ("llama3_70b", [0, 40, 79], dict(depth=4, branch=[3, 2, 2, 1], max_nodes=24), 16384, None),
}
# Sampled decoding measured beside the default workload (same model, draft and prompt).
SAMPLED = dict(depth=3, branch=[3, 2, 1], temperature=0.7, top_p=0.9)


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def time_launches(fn, n: int, reps: int = 3) -> float:
    """Average duration (ms) of one launch of fn(i), i = 0..n-1: the n launches are captured once in
    a HIP graph and replayed between two HIP events on the launching stream (no host time between
    kernels), best of reps. Callers pass a different layer's weights per i, so every launch
    streams its weights from HBM as in a decode round (a repeat of one layer would be served from
    the 256 MB Infinity Cache)."""
    import torch

    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        for i in range(n):  # warm up outside the capture
            fn(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        for i in range(n):
            fn(i)
    best = float("inf")
    with torch.cuda.stream(st):
        g.replay()
        for _ in range(reps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(st)
            g.replay()
            b.record(st)
            b.synchronize()
            best = min(best, a.elapsed_time(b) / n)
    torch.cuda.synchronize()
    return best


def kernel_figures(gen, sess) -> dict:
    """Live per-kernel timings at the verify shape of the last timed round (M = verify rows,
    context = the committed length), each kernel launched once per layer like in the round."""
    import torch

    from ssd import ops

    target, cache, ws = gen.target, sess.cache, sess.ws
    model = target.model
    s = model.shape
    L = model.layers
    nl = s.layers
    m = gen.drafter.max_verify_nodes() + 1
    aws = ws.attn_ws(model, cache.capacity)
    rows = sess.verify_rows  # the last round's verify rows (the next round's draft only touches the root row)
    p = int(rows.prefix[0])  # that round's committed length + 1
    committed = p - 1
    part = ws.part
    out = {}

    def fig(name, t, b, **kw):
        out[name] = dict(ms=t, bytes=b, gbs=b / t / 1e6, frac=b / t / 1e6 / HBM_PEAK_GBS, rows=m, **kw)

    def attn(i):
        kc, vt = cache.layer(i)
        ops.tree_attention(ws.q, m, s.heads, s.kv_heads, s.head_dim, kc, vt, cache.capacity, rows.prefix, rows.depth,
                           rows.anc, p, p + gen.cfg.depth, aws, ws.attn)

    kv_bytes = 2 * s.kv_heads * (p + m) * s.head_dim * 2
    fig("tree_attention", time_launches(attn, nl), kv_bytes + 2 * m * s.heads * s.head_dim * 2 + m * 32 * 4,
        context=p)
    n_qkv = (s.heads + 2 * s.kv_heads) * s.head_dim
    cos, sin = model.rope(cache.capacity)

    def qkv(i):
        kc, vt = cache.layer(i)
        ops.qkv_rope(ws.h, m, L[i].wqkv, s.hidden, s.heads, s.kv_heads, s.head_dim, cos, sin, rows.pos, rows.slot,
                     ws.q, kc, vt, cache.capacity, norm_eps=s.eps)

    fig("gemm_qkv_rope", time_launches(qkv, nl), n_qkv * s.hidden * 2 + m * s.hidden * 2 + m * n_qkv * 2)

    h_scratch = ws.h.clone()  # the residual projections update h in place
    qdim = s.heads * s.head_dim

    def o_proj(i):
        ops.gemm_residual(ws.attn, m, L[i].wo, s.hidden, qdim, h_scratch, ws.part)

    fig("o_proj", time_launches(o_proj, nl), s.hidden * qdim * 2 + m * qdim * 2 + 2 * m * s.hidden * 2)
    sp = ops.gemm_splits(s.hidden, s.inter)
    if model.mlp_fused:
        # gate/up + SwiGLU + down + residual in one launch: weights, h read and written, act and
        # the down partials written once and read once
        sync = ops.mlp_sync(model.device)

        def mlp(i):
            ops.mlp(h_scratch, m, L[i].wgu, L[i].wd, s.inter, s.hidden, s.eps, ws.mlp, part, sync)

        fig("mlp", time_launches(mlp, nl), 3 * s.inter * s.hidden * 2 + 2 * m * s.hidden * 2 + 2 * m * s.inter * 2
            + 2 * sp * m * s.hidden * 4, flops=2 * m * 3 * s.inter * s.hidden, splits=sp)
    else:
        def gateup(i):
            ops.gemm_swiglu(ws.h, m, L[i].wgu, s.inter, s.hidden, ws.mlp, norm_eps=s.eps)

        fig("gemm_gate_up", time_launches(gateup, nl),
            2 * s.inter * s.hidden * 2 + m * s.hidden * 2 + m * s.inter * 2, flops=2 * m * 2 * s.inter * s.hidden)

        def down(i):
            ops.gemm_residual(ws.mlp, m, L[i].wd, s.hidden, s.inter, h_scratch, part)

        fig("gemm_down_residual", time_launches(down, nl),
            s.hidden * s.inter * 2 + m * s.inter * 2 + 2 * m * s.hidden * 2, splits=sp)
    logits = ws.logits_buf(m, s.vocab)

    def head(i):
        ops.gemm(ws.h, m, model.lm_head, s.vocab, s.hidden, logits, norm_eps=s.eps)

    fig("lm_head", time_launches(head, 4), s.vocab * s.hidden * 2 + m * s.hidden * 2 + m * s.vocab * 2)
    n = gen.cfg.depth + 1
    src = torch.arange(committed, committed + n, dtype=torch.int32, device=model.device) + torch.tensor(
        [0] + [1] * (n - 1), dtype=torch.int32, device=model.device)
    nd = torch.tensor([n], dtype=torch.int32, device=model.device)

    def compact(i):
        cache.compact_device(committed, src, nd, n)

    fig("kv_compact", time_launches(compact, 8), 2 * n * s.layers * 2 * s.kv_heads * s.head_dim * 2)
    out["kv_compact"]["rows"] = n
    return out


BF16_MFMA_PEAK_TFLOPS = 2500.0


def prefill_figures(target, ids: list, reps: int = 3) -> dict:
    """The prompt's target forward alone (ssd_prefill: MFMA GEMMs + causal flash attention), best
    of ``reps`` into fresh caches: ms, achieved TFLOP/s (2 flop per weight per token for the
    projections, 4 * hd per (query, key) pair for attention, the causal half) and the fraction of
    the MI355X dense bf16 MFMA peak."""
    import torch

    from ssd.engine.speculative import _prefill_logits

    s = target.model.shape
    P = len(ids)
    ws = target.workspace()
    best = float("inf")
    for _ in range(reps):
        cache = target.new_cache(P + 64)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        _prefill_logits(target, ids, cache, ws)
        torch.cuda.synchronize()
        best = min(best, time.perf_counter() - t0)
        del cache
    per_layer = (s.hidden * (s.heads + 2 * s.kv_heads) * s.head_dim + s.hidden * s.heads * s.head_dim
                 + 3 * s.hidden * s.inter)
    flops = 2 * P * s.layers * per_layer + 2 * s.vocab * s.hidden + 4 * (P * (P + 1) / 2) * s.heads * s.head_dim * s.layers
    tf = flops / best / 1e12
    return {"tokens": P, "ms": round(1000 * best, 3), "tflops": round(tf, 1),
            "mfma_frac": round(tf / BF16_MFMA_PEAK_TFLOPS, 4), "flops": flops}


def batch_generation_figures(target, batch: int, prompt: int, new: int) -> dict:
    """Greedy batched generation (ssd.data.generate_selfdistill.generate_batch): ``batch`` prompts
    of ``prompt`` uniform random tokens, ``new`` tokens each; decode tokens/s over the whole batch
    (prefill of the batch timed separately as a one-token run)."""
    import torch

    from ssd.data.generate_selfdistill import generate_batch

    V = target.model.shape.vocab
    g = torch.Generator().manual_seed(11)
    prompts = [torch.randint(0, V, (prompt,), generator=g).tolist() for _ in range(batch)]
    generate_batch(target, prompts, 2, {-1}, 0.0, 1.0, 0)  # warm-up
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    generate_batch(target, prompts, 1, {-1}, 0.0, 1.0, 0)
    torch.cuda.synchronize()
    t_pre = time.perf_counter() - t0
    t0 = time.perf_counter()
    rows = generate_batch(target, prompts, new, {-1}, 0.0, 1.0, 0)
    torch.cuda.synchronize()
    t_all = time.perf_counter() - t0
    toks = sum(len(r) for r in rows)
    dec = max(t_all - t_pre, 1e-9)
    return {"batch": batch, "prompt_tokens": prompt, "new_tokens": new, "seconds": round(t_all, 4),
            "decode_tokens_per_s": round((toks - batch) / dec, 1), "ms_per_step": round(1000 * dec / (new - 1), 4)}


def load_traffic(kernel_key: str):
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3 --pmc summary
    (profiles/*_traffic.json: FETCH_SIZE + WRITE_SIZE per dispatch, scaled by the same counters'
    reading for a plain copy of known size), or None if absent."""
    path = os.path.join(REPO, "profiles", f"{kernel_key}_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("traffic_bytes")


def cpu_baseline(model, layers: list, dcfg: dict, rounds: int, prompt_len: int) -> dict:
    """The CPU oracle (PyTorch restatement of the reference path) on the host cores. Its weights
    are the GPU model's packed tensors copied to the host and viewed as row-major matrices of the
    same shapes (a permutation of the same N(0, 0.02) values): the timing does not depend on
    which permutation is used, and the copy takes seconds instead of minutes of CPU sampling."""
    import torch

    from oracle import engine as oe
    from oracle import model as om

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    s = model.shape
    shape = om.LlamaShape(s.hidden, s.layers, s.heads, s.kv_heads, s.head_dim, s.inter, s.vocab, s.eps, s.theta,
                          s.rope_scaling)
    t0 = time.perf_counter()
    host = lambda t, n, k: t[: n * k].view(n, k).cpu()
    sd = {"model.embed_tokens.weight": model.embed.cpu(), "model.norm.weight": model.norm.cpu(),
          "lm_head.weight": host(model.lm_head, s.vocab, s.hidden)}
    nq, nkv = s.heads * s.head_dim, s.kv_heads * s.head_dim
    for i, L in enumerate(model.layers):
        p = f"model.layers.{i}."
        qkv = host(L.wqkv, nq + 2 * nkv, s.hidden)
        sd[p + "self_attn.q_proj.weight"] = qkv[:nq]
        sd[p + "self_attn.k_proj.weight"] = qkv[nq:nq + nkv]
        sd[p + "self_attn.v_proj.weight"] = qkv[nq + nkv:]
        sd[p + "self_attn.o_proj.weight"] = host(L.wo, s.hidden, nq)
        gu = host(L.wgu, 2 * s.inter, s.hidden)
        sd[p + "mlp.gate_proj.weight"], sd[p + "mlp.up_proj.weight"] = gu[:s.inter], gu[s.inter:]
        sd[p + "mlp.down_proj.weight"] = host(L.wd, s.hidden, s.inter)
        sd[p + "input_layernorm.weight"] = L.ln1.cpu()
        sd[p + "post_attention_layernorm.weight"] = L.ln2.cpu()
    base = om.Llama(sd, shape, torch.bfloat16)
    del sd
    specs = om.plan_bridges(layers, s.layers)
    draft = om.Subnetwork(base, layers, om.random_bridges(specs, s.hidden, seed=1, dtype=torch.bfloat16))
    target = om.Target(base)
    log(f"cpu oracle ready in {time.perf_counter() - t0:.1f}s on {cores} threads")
    gen = oe.SpeculativeGenerator(target, draft, oe.Drafting(**dcfg), s.vocab)
    ids = torch.randint(0, s.vocab, (prompt_len,), generator=torch.Generator().manual_seed(1)).tolist()
    res = gen.generate(ids, 10 ** 6, {-1}, max_rounds=rounds)
    toks = sum(res.accepted_per_round)
    secs = res.decode_seconds
    log(f"cpu oracle: {rounds} rounds, {toks} tokens in {secs:.2f}s")
    return dict(value=round(toks / secs, 4), unit="tokens/s", cores=cores, kind="port",
                sample=f"{rounds} speculative rounds of the same model shape and tree after a {prompt_len}-token "
                       f"prompt (the GPU run uses the full prompt), bf16 PyTorch CPU oracle; "
                       f"{1000 * secs / rounds:.0f} ms/round")


def sampled_rounds(model, draft, target, ids: list, steps: int, warmup: int = 5) -> dict:
    """Sampled speculative rounds (SAMPLED drafting) after the same prompt: ms/round, tokens/s,
    mean tokens per round and phase split; Philox seed 0."""
    import torch

    from ssd.config import DraftingConfig
    from ssd.engine.speculative import SpeculativeGenerator

    cfg = DraftingConfig(**SAMPLED)
    gen = SpeculativeGenerator(model, draft, cfg, target)
    sess = gen.session(len(ids) + (warmup + steps) * (cfg.depth + 1) + gen.capacity(0, 0), seed=0)
    sess.prefill(ids)
    for _ in range(warmup):
        sess.step()
    sess.phases.totals.clear()
    n0 = len(sess.accepted_per_round)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    toks = sum(len(sess.step()) for _ in range(steps))
    torch.cuda.synchronize()
    secs = time.perf_counter() - t0
    acc = sess.accepted_per_round[n0:]
    return {"drafting": SAMPLED, "rounds": steps, "tokens_per_s": round(toks / secs, 3),
            "ms_per_round": round(1000 * secs / steps, 4), "mean_accepted": round(sum(acc) / len(acc), 4),
            "ms_per_round_phases": {k: round(1000 * v / steps, 4) for k, v in sess.phases.totals.items()}}


# Standalone tree-attention shapes (--attention): (kv heads, q heads, head_dim, prefix slots, rows, depth,
# layers rotated so every call streams its K/V from HBM).
ATTN_SHAPES = {
    "8b_verify": (8, 32, 128, 4097, 25, 4, 32),
    "8b_draft": (8, 32, 128, 4098, 12, 4, 32),
    "8b_ar": (8, 32, 128, 4100, 1, 0, 32),
    "70b_verify": (8, 64, 128, 16385, 25, 4, 8),
    "70b_draft": (8, 64, 128, 16386, 12, 4, 8),
}


def attention_figures(name: str, reps: int = 20) -> dict:
    """One tree-attention call (partial + combine) at a decode shape: the root row attends the prefix,
    the tree rows the prefix plus 1..depth ancestors among the tree slots; best of `reps` passes over
    the rotated layers, us per call, and the algorithmic bytes (K/V over P + depth slots, queries,
    outputs)."""
    import torch

    from ssd import ops

    kvh, heads, hd, P, M, depth, layers = ATTN_SHAPES[name]
    dev = "cuda"
    cap = (P + 2 * 64 + 63) // 64 * 64
    g = torch.Generator().manual_seed(0)
    ks = [ops.kv_tile(torch.randn(kvh, cap, hd, generator=g).to(torch.bfloat16).to(dev), "k") for _ in range(layers)]
    vs = [ops.kv_tile(torch.randn(kvh, cap, hd, generator=g).to(torch.bfloat16).to(dev), "v") for _ in range(layers)]
    q = torch.randn(M, heads * hd, generator=g).to(torch.bfloat16).to(dev)
    pre = torch.full((M,), P, dtype=torch.int32, device=dev)
    dep = torch.tensor([0] + [min(depth, 1 + i % depth) for i in range(M - 1)], dtype=torch.int32, device=dev)
    an = torch.zeros(M, 32, dtype=torch.int32)
    for t in range(1, M):
        an[t, :int(dep[t])] = torch.arange(P + 1, P + 1 + int(dep[t])) + (t % 3)
    an = an.to(dev)
    ws = torch.zeros(ops.attn_workspace_floats(M, heads, hd, cap), dtype=torch.float32, device=dev)
    out = torch.zeros(M, heads * hd, dtype=torch.bfloat16, device=dev)

    def call(i):
        ops.tree_attention(q, M, heads, kvh, hd, ks[i], vs[i], cap, pre, dep, an, P, P + depth + 3, ws, out)

    for i in range(layers):
        call(i)
    torch.cuda.synchronize()
    best = float("inf")
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for i in range(layers):
            call(i)
        b.record()
        b.synchronize()
        best = min(best, a.elapsed_time(b) * 1000 / layers)
    byts = 2 * kvh * (P + depth) * hd * 2 + 2 * M * heads * hd * 2
    return {"shape": name, "us": round(best, 2), "bytes": byts, "gbs": round(byts / best / 1e3, 1),
            "frac": round(byts / best / 1e3 / HBM_PEAK_GBS, 4)}


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="llama3_8b_tree", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--graphs", action="store_true", help="replay captured greedy rounds (HIP graphs)")
    ap.add_argument("--cpu-rounds", type=int, default=40)
    ap.add_argument("--cpu-prompt", type=int, default=128)
    ap.add_argument("--ar-tokens", type=int, default=128)
    ap.add_argument("--sampled-rounds", type=int, default=30,
                    help="also time this many sampled rounds (T 0.7, top_p 0.9, d3 [3,2,1]); 0 = skip")
    ap.add_argument("--batch-gen", type=int, default=32,
                    help="also time greedy batched generation (generate_batch) of this many prompts; 0 = skip")
    ap.add_argument("--batch-gen-prompt", type=int, default=512)
    ap.add_argument("--batch-gen-tokens", type=int, default=64)
    ap.add_argument("--copy-probe-mb", type=int, default=0,
                    help="also run one plain device copy of this many MiB (calibrates rocprofv3 byte counters)")
    ap.add_argument("--attention", default="",
                    help=f"only time tree attention at these shapes (comma list of {', '.join(ATTN_SHAPES)}), "
                         "one JSON line each")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: bench.py runs on exactly one GPU (got --gpus {args.gpus}); multi-GPU runs are not supported",
              file=sys.stderr)
        sys.exit(3)

    import torch

    if args.attention:
        torch.cuda.set_device(0)
        for name in args.attention.split(","):
            print(json.dumps(attention_figures(name)), flush=True)
        if args.copy_probe_mb:
            src = torch.ones(args.copy_probe_mb << 20, dtype=torch.uint8, device="cuda")
            torch.empty_like(src).copy_(src)
            torch.cuda.synchronize()
            log(f"copy probe: {args.copy_probe_mb} MiB read + {args.copy_probe_mb} MiB written")
        return

    from ssd import _lib
    from ssd.config import BridgeConfig, DraftingConfig
    from ssd.data.token_freq import top_vocab, zipf_counts
    from ssd.engine.speculative import SpeculativeGenerator, TargetRunner, autoregressive_generate
    from ssd.models.llama import MI355XLlama
    from ssd.models.subnetwork_draft import SubnetworkDraftModel
    from ssd.runtime import SHAPES

    torch.cuda.set_device(0)
    shape_name, layers, dkw, n_prompt, draft_vocab = WORKLOADS[args.workload]
    shape = SHAPES[shape_name]
    t0 = time.perf_counter()
    model = MI355XLlama.synthetic(shape, seed=0)
    target = TargetRunner(model)
    torch.manual_seed(0)
    draft = SubnetworkDraftModel(model, layers, BridgeConfig())
    draft.bridges.to(torch.bfloat16)
    if draft_vocab:
        draft.set_vocab_subset(top_vocab(zipf_counts(shape.vocab, 1.1, seed=0), draft_vocab))
    cfg = DraftingConfig(**dkw)
    gen = SpeculativeGenerator(model, draft, cfg, target)
    ids = torch.randint(0, shape.vocab, (n_prompt,), generator=torch.Generator().manual_seed(1)).tolist()
    rounds = args.warmup + args.steps
    sess = gen.session(n_prompt + rounds * (cfg.depth + 1) + gen.capacity(0, 0), seed=0,
                       graphs=args.graphs)
    log(f"model + draft ready in {time.perf_counter() - t0:.1f}s")
    t0 = time.perf_counter()
    sess.prefill(ids)
    torch.cuda.synchronize()
    log(f"prefill {n_prompt} tokens: {time.perf_counter() - t0:.2f}s")
    # exactly `steps` rounds in the timed region: nothing of a later round is enqueued by the last
    # warm-up step or by the last timed step (graph rounds otherwise keep one round queued)
    for i in range(args.warmup):
        sess.step(lookahead=i < args.warmup - 1)
    sess.phases.totals.clear()
    n_warm = len(sess.accepted_per_round)
    torch.cuda.synchronize()
    launches0 = int(_lib.load().ssd_launch_count())
    t0 = time.perf_counter()
    toks = 0
    for i in range(args.steps):
        toks += len(sess.step(lookahead=i < args.steps - 1))
    torch.cuda.synchronize()
    secs = time.perf_counter() - t0
    launches = (int(_lib.load().ssd_launch_count()) - launches0) / args.steps
    if sess.graph_rounds:  # replays do not pass through the library's launch counter
        launches = sess.graph_launches
    graph_info = {"enabled": sess.graphs, "rounds_replayed": sess.graph_rounds, "captures": sess.captures}
    acc = sess.accepted_per_round[n_warm:]
    phases = {k: 1000 * v / args.steps for k, v in sess.phases.totals.items()}
    log(f"{args.steps} rounds: {toks} tokens in {secs:.3f}s ({toks / secs:.1f} tok/s, {1000 * secs / args.steps:.3f} "
        f"ms/round), phases {phases}")
    kf = kernel_figures(gen, sess)
    log(f"kernels: { {k: (round(v['ms'] * 1000, 1), round(v['gbs'])) for k, v in kf.items()} } (us, GB/s)")
    del sess
    torch.cuda.empty_cache()
    sampled = None
    if args.sampled_rounds and "temperature" not in dkw:
        sampled = sampled_rounds(model, draft, target, ids, args.sampled_rounds)
        log(f"sampled {SAMPLED}: {sampled}")
        torch.cuda.empty_cache()
    ar = autoregressive_generate(target, torch.tensor([ids]), args.ar_tokens, {-1})
    ar_tps = (len(ar.tokens) - 1) / ar.times["decode"]
    log(f"autoregressive baseline: {ar_tps:.1f} tok/s")
    pre = prefill_figures(target, ids)
    log(f"prefill: {pre}")
    batch = batch_generation_figures(target, args.batch_gen, args.batch_gen_prompt, args.batch_gen_tokens) \
        if args.batch_gen else None
    if batch:
        log(f"batched generation: {batch}")

    bytes_round = model.weight_bytes() + 4 * model.weight_bytes(layers)
    fused = "mlp" in kf
    g = kf["mlp" if fused else "gemm_gate_up"]
    kname = ("mlp (verify: gate/up + SwiGLU + down + residual in one launch, M=%d)" if fused
             else "gemm_swiglu (verify gate/up, M=%d)") % g["rows"]
    tkey = "mlp_llama3_8b_verify" if fused else "gemm_gate_up_llama3_8b_verify"
    line = {
        "metric": METRIC,
        "value": round(toks / secs, 3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1000 * secs / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: random-init weights N(0, 0.02) generated on the GPU, uniform random prompt ids",
        "config": {"workload": args.workload, "shape": shape_name, "draft_layers": layers, "drafting": dkw,
                   "prompt_tokens": n_prompt, "draft_vocab": draft_vocab or "full", "batch": 1,
                   "parallelism": "single GPU"},
        "mean_accepted": round(sum(acc) / len(acc), 4),
        "ms_per_round_phases": {k: round(v, 4) for k, v in phases.items()},
        # kernels the library enqueues per round (the engine adds two small torch ops and the
        # result copy)
        "launches_per_round": round(launches, 2),
        "graph": graph_info,
        "ar_tokens_per_s": round(ar_tps, 3),
        "speedup_vs_ar": round((toks / secs) / ar_tps, 4),
        "round_weight_bytes": bytes_round,
        "round_hbm_lower_bound_ms": round(bytes_round / HBM_PEAK_GBS / 1e6, 4),
        "roofline": {"bound": "hbm", "kernel": kname,
                     "achieved": round(g["gbs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(g["frac"], 4),
                     # the committed PMC summary covers the default workload's kernel only
                     "traffic": load_traffic(tkey) if args.workload == "llama3_8b_tree" else None},
        "kernels": {k: {kk: (round(vv, 5) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                    for k, v in kf.items()},
    }
    if sampled is not None:
        line["sampled"] = sampled
    line["prefill"] = pre
    if batch:
        line["batch_generation"] = batch
    if args.copy_probe_mb:
        src = torch.ones(args.copy_probe_mb << 20, dtype=torch.uint8, device=model.device)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy probe: {args.copy_probe_mb} MiB read + {args.copy_probe_mb} MiB written")
        del src, dst
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(model, layers, dkw, args.cpu_rounds, args.cpu_prompt)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
