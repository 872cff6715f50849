"""Prefill kernels (MFMA GEMM over prompt-length M, causal flash attention, the one-call target
forward ssd_prefill) against the CPU oracle and the decode kernels.

* GEMM epilogues (plain, residual add, folded RMSNorm, SwiGLU, q/k/v + RoPE + KV write) against
  the fp32 product of the same bf16 operands (outputs within one bf16 rounding step, >= 97% equal)
  and against the decode kernels on the same rows; every output row is independent of how many
  rows share the call (bitwise).
* Causal attention against the oracle's exact softmax attention, with cache slots past the
  prompt holding NaN (they must not leak into the result).
* The whole prefill forward: logits against the oracle's fp32 evaluation and bf16 chain, chunked
  prompts bit-identical to one call, the decode forward's logits within the per-node tolerance.
"""

import pytest
import torch

from oracle import kernels as ok
from oracle import model as om

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = dict(atol=1e-2, rtol=2e-2)


def _ops():
    from ssd import ops
    return ops


def bf(t):
    return t.to(torch.bfloat16)


def rand(*shape, std=1.0, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g) * std


def close_bf16(got, ref, frac=0.97, rtol=1.6e-2, atol=1e-2):
    """bf16 results of fp32 sums in different orders (values of order 1): within two rounding
    steps (absolute where a residual add cancels), mostly equal."""
    got, ref = got.float().cpu(), ref.float().cpu()
    torch.testing.assert_close(got, ref, atol=atol, rtol=rtol)
    exact = (got == ref).float().mean().item()
    assert exact >= frac, f"only {exact:.3f} of outputs are equal"


@pytest.mark.parametrize("m", [1, 77, 300])
# N = 384 and 640: the last 256-row workgroup tile reaches past the weight's (128-row padded) tiles
@pytest.mark.parametrize("n,k,residual", [(256, 256, False), (6144, 4096, False), (4096, 4096, True),
                                          (4096, 14336, True), (384, 512, False), (640, 1024, True)])
def test_prefill_gemm_store_and_residual(m, n, k, residual):
    ops = _ops()
    x, w = bf(rand(m, k, seed=1)), bf(rand(n, k, std=0.02, seed=2))
    grp = ops.residual_group(n, k) if residual else ops.weight_group(n, k)
    wp = ops.pack_weight(w.to(DEV), residual=residual)
    res = bf(rand(m, n, seed=3)) if residual else None
    y = res.to(DEV).clone() if residual else torch.zeros(m, n, dtype=torch.bfloat16, device=DEV)
    ops.prefill_gemm(x.to(DEV), m, wp, grp, n, k, y, "store", residual=y if residual else None)
    ref = bf(x.float() @ w.float().T)
    if residual:
        ref = bf(res.float() + ref.float())
    close_bf16(y, ref)


def test_prefill_gemm_rows_do_not_depend_on_m():
    """A row's result is the same whether it is computed in a call of 1000 rows or of 37."""
    ops = _ops()
    n, k = 4096, 4096
    x, w = bf(rand(1000, k, seed=4)).to(DEV), bf(rand(n, k, std=0.02, seed=5)).to(DEV)
    wp = ops.pack_weight(w)
    grp = ops.weight_group(n, k)
    a = torch.zeros(1000, n, dtype=torch.bfloat16, device=DEV)
    b = torch.zeros(37, n, dtype=torch.bfloat16, device=DEV)
    ops.prefill_gemm(x, 1000, wp, grp, n, k, a, "store", norm_eps=1e-5)
    ops.prefill_gemm(x[500:537].contiguous(), 37, wp, grp, n, k, b, "store", norm_eps=1e-5)
    assert torch.equal(a[500:537], b)


@pytest.mark.parametrize("hidden,inter,m", [(256, 512, 200), (4096, 14336, 300)])
def test_prefill_gemm_norm_swiglu_matches_decode(hidden, inter, m):
    """Folded RMSNorm + SwiGLU (gate/up interleaved 8 + 8 rows per tile, the fused-MLP grouping
    where the shape has one) against the decode GEMM in 64-row chunks and the fp32 formula."""
    from ssd.models.llama import gate_up_row_map
    ops = _ops()
    h = bf(rand(m, hidden, seed=6))
    ln = bf(1 + 0.1 * rand(hidden, seed=7))
    wg, wu = bf(rand(inter, hidden, std=0.02, seed=8)), bf(rand(inter, hidden, std=0.02, seed=9))
    gu = torch.cat([wg, wu]).to(DEV)
    g_mlp = ops.mlp_group(inter, hidden)
    grp = g_mlp or ops.weight_group(2 * inter, hidden)
    wp = ops.pack_weight(gu, gate_up_row_map(inter), col_scale=ln.to(DEV), group=grp)
    hd = h.to(DEV)
    got = torch.zeros(m, inter, dtype=torch.bfloat16, device=DEV)
    ops.prefill_gemm(hd, m, wp, grp, 2 * inter, hidden, got, "swiglu", norm_eps=1e-5)
    if not g_mlp:  # the decode swiglu GEMM reads the single-pass grouping
        dec = torch.zeros(m, inter, dtype=torch.bfloat16, device=DEV)
        for c0 in range(0, m, 64):
            c1 = min(m, c0 + 64)
            ops.gemm_swiglu(hd[c0:c1], c1 - c0, wp, inter, hidden, dec[c0:c1], norm_eps=1e-5)
        close_bf16(got, dec)
    # fp32 formula on the same bf16 operands: x * rsqrt(mean x^2 + eps) against W * ln (rounded
    # once, as packed), bf16 rounding at the linear outputs and the SwiGLU product
    wgf = bf(wg.float() * ln.float()).float()
    wuf = bf(wu.float() * ln.float()).float()
    r = torch.rsqrt(h.float().pow(2).mean(1, keepdim=True) + 1e-5)
    g32, u32 = (h.float() @ wgf.T) * r, (h.float() @ wuf.T) * r
    ref = bf(bf(torch.nn.functional.silu(bf(g32).float())).float() * bf(u32).float())
    close_bf16(got, ref, frac=0.95, rtol=1.6e-2)


@pytest.mark.parametrize("heads,kv,hd,hidden,m,pos0", [(4, 2, 64, 256, 150, 70), (32, 8, 128, 4096, 150, 70),
                                                      (8, 2, 128, 512, 600, 37)])
def test_prefill_gemm_qkv_rope_matches_decode(heads, kv, hd, hidden, m, pos0):
    """q/k/v + RoPE + KV-cache write at positions pos0 + row against the decode q/k/v GEMM. Unaligned
    pos0: the V^T cache's 8-slot runs are cut at the first and last row and, with m > 256, between
    the two row tiles' workgroups."""
    from ssd.models.llama import qkv_row_map, rope_tables
    ops = _ops()
    cap = (pos0 + m + 63) // 64 * 64 + 64
    n = (heads + 2 * kv) * hd
    h = bf(rand(m, hidden, seed=10)).to(DEV)
    ln = bf(1 + 0.1 * rand(hidden, seed=11)).to(DEV)
    w = bf(rand(n, hidden, std=0.02, seed=12)).to(DEV)
    wp = ops.pack_weight(w, qkv_row_map(heads, kv, hd), col_scale=ln)
    cos, sin = rope_tables(cap, hd, 500000.0, DEV)
    caches = []
    for path in ("prefill", "decode"):
        q = torch.zeros(m, heads * hd, dtype=torch.bfloat16, device=DEV)
        kc = torch.zeros(kv, cap * hd, dtype=torch.bfloat16, device=DEV)
        vt = torch.zeros(kv, cap * hd, dtype=torch.bfloat16, device=DEV)
        if path == "prefill":
            ops.prefill_gemm(h, m, wp, ops.weight_group(n, hidden), n, hidden, q, "qkv", norm_eps=1e-5,
                             qkv=dict(heads=heads, kv_heads=kv, head_dim=hd, cos=cos, sin=sin, pos0=pos0, k_cache=kc,
                                      vt_cache=vt, max_len=cap))
        else:
            for c0 in range(0, m, 64):
                c1 = min(m, c0 + 64)
                pos = torch.arange(pos0 + c0, pos0 + c1, dtype=torch.int32, device=DEV)
                ops.qkv_rope(h[c0:c1], c1 - c0, wp, hidden, heads, kv, hd, cos, sin, pos, pos, q[c0:c1], kc, vt, cap,
                             norm_eps=1e-5)
        caches.append((q, ops.kv_untile(kc, cap, hd, "k"), ops.kv_untile(vt, cap, hd, "v")))
    (qa, ka, va), (qb, kb, vb) = caches
    close_bf16(qa, qb)
    close_bf16(ka[:, pos0:pos0 + m], kb[:, pos0:pos0 + m])
    close_bf16(va[:, pos0:pos0 + m], vb[:, pos0:pos0 + m])
    assert not ka[:, :pos0].any() and not ka[:, pos0 + m:].any()  # nothing written outside the rows
    assert not va[:, :pos0].any() and not va[:, pos0 + m:].any()


@pytest.mark.parametrize("heads,kv,hd", [(4, 2, 64), (32, 8, 128), (64, 8, 128)])
@pytest.mark.parametrize("m,pos0", [(300, 0), (161, 77), (1, 500)])
def test_prefill_attention_matches_oracle(heads, kv, hd, m, pos0):
    ops = _ops()
    L = pos0 + m
    cap = (L + 63) // 64 * 64 + 64
    q = bf(rand(m, heads, hd, seed=13))
    k = bf(rand(kv, cap, hd, seed=14))
    v = bf(rand(kv, cap, hd, seed=15))
    k[:, L:] = float("nan")  # not yet written: must not reach any output
    v[:, L:] = float("nan")
    kd, vd = ops.kv_tile(k.to(DEV), "k"), ops.kv_tile(v.to(DEV), "v")
    out = torch.zeros(m, heads * hd, dtype=torch.bfloat16, device=DEV)
    ops.prefill_attention(q.reshape(m, -1).to(DEV), m, pos0, heads, kv, hd, kd, vd, cap, out)
    got = out.view(m, heads, hd).float().cpu()
    assert torch.isfinite(got).all()
    ref = ok.tree_attention(q, k[:, :L], v[:, :L], [pos0 + t + 1 for t in range(m)], [[] for _ in range(m)])
    scale = ref.abs().max().item()
    torch.testing.assert_close(got, ref, atol=1e-2 * scale, rtol=2e-2)


@pytest.mark.parametrize("heads,kv,hd,m,pos0", [(32, 8, 128, 300, 0), (64, 8, 128, 161, 77), (16, 4, 64, 97, 40),
                                               (32, 8, 128, 1, 500)])
def test_prefill_attention_shared_kv_equals_per_wave_loads(heads, kv, hd, m, pos0):
    """With 4 | (q heads per kv head) a workgroup's four waves share their kv head's K/V blocks
    through LDS (copied one block ahead); the same heads run as 2-head, 1-kv-head problems take the
    kernel whose waves load their own K/V. The fragments and their order are the same, so every
    head's output is bit-identical (unwritten cache slots hold NaN, as in the test above)."""
    ops = _ops()
    L = pos0 + m
    cap = (L + 63) // 64 * 64 + 64
    q = bf(rand(m, heads, hd, seed=21))
    k = bf(rand(kv, cap, hd, seed=22))
    v = bf(rand(kv, cap, hd, seed=23))
    k[:, L:] = float("nan")
    v[:, L:] = float("nan")
    kd, vd = ops.kv_tile(k.to(DEV), "k"), ops.kv_tile(v.to(DEV), "v")
    out = torch.zeros(m, heads * hd, dtype=torch.bfloat16, device=DEV)
    ops.prefill_attention(q.reshape(m, -1).to(DEV), m, pos0, heads, kv, hd, kd, vd, cap, out)
    out = out.view(m, heads, hd)
    assert torch.isfinite(out.float()).all()
    rep = heads // kv
    for kvh in range(kv):
        kh, vh = kd[kvh:kvh + 1].contiguous(), vd[kvh:kvh + 1].contiguous()
        for h0 in range(kvh * rep, (kvh + 1) * rep, 2):
            o2 = torch.zeros(m, 2 * hd, dtype=torch.bfloat16, device=DEV)
            ops.prefill_attention(q[:, h0:h0 + 2].reshape(m, -1).contiguous().to(DEV), m, pos0, 2, 1, hd, kh, vh, cap,
                                  o2)
            assert torch.equal(o2.view(m, 2, hd), out[:, h0:h0 + 2]), (kvh, h0)


def _small_hf(layers=4):
    from transformers import LlamaConfig, LlamaForCausalLM
    torch.manual_seed(0)
    m = LlamaForCausalLM(LlamaConfig(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=layers,
                                     num_attention_heads=4, num_key_value_heads=2, rope_theta=500000.0,
                                     max_position_embeddings=4096)).eval()
    return m.to(torch.bfloat16)


def test_prefill_forward_logits_match_oracle():
    """A 300-token prompt through the target (prefill path) against the oracle's fp32 evaluation
    (every element within the per-node tolerance) and its bf16 chain (>= 99.9%)."""
    import ssd.engine.speculative as sp
    hf = _small_hf()
    target = sp.TargetRunner(hf)
    ids = torch.randint(0, 512, (1, 300), generator=torch.Generator().manual_seed(2))
    got = target(ids).logits[0].float().cpu()
    base = om.Llama.from_hf(hf)
    ref = om.Target(base)(ids[0])[0].float()
    exact = om.Target(om.Llama({k: v.float() for k, v in base.sd.items()}, base.shape, torch.float32))(ids[0])[0]
    torch.testing.assert_close(got, exact, **TOL)
    err = (got - ref).abs()
    lim = TOL["atol"] + TOL["rtol"] * ref.abs()
    assert (err <= lim).float().mean() >= 0.999


def test_prefill_chunks_bitwise_equal_one_call_and_decode_path_close(monkeypatch):
    """A 700-token prompt in chunks of 256 rows gives the same logits and cache bits as one call
    (prefill rows depend only on their own keys); the decode forward (64-row causal chunks) agrees
    within the per-node tolerance."""
    import ssd.engine.speculative as sp
    import ssd.models.subnetwork_draft as sdm
    hf = _small_hf()
    target = sp.TargetRunner(hf)
    ids = torch.randint(0, 512, (1, 700), generator=torch.Generator().manual_seed(3))
    runs = {}
    for name in ("one", "chunked", "decode"):
        cache = target.new_cache(768)
        if name == "chunked":
            monkeypatch.setattr(sdm, "PREFILL_CHUNK", 256)
        if name == "decode":
            monkeypatch.setattr(target, "prefill_capable", lambda: False)
        runs[name] = (target(ids, past_key_values=cache).logits[0].clone(), cache.k.clone(), cache.vt.clone())
        monkeypatch.undo()
    assert torch.equal(runs["one"][0], runs["chunked"][0])
    assert torch.equal(runs["one"][1], runs["chunked"][1]) and torch.equal(runs["one"][2], runs["chunked"][2])
    torch.testing.assert_close(runs["one"][0].float(), runs["decode"][0].float(), **TOL)


def test_prefill_engine_first_token_and_sd_equals_ar():
    """The engine's prefill runs on the prefill kernels for a 600-token prompt: the first token is
    the argmax of the prefill logits, and greedy SD == greedy AR after it."""
    import ssd.engine.speculative as sp
    from ssd.config import BridgeConfig, DraftingConfig
    from ssd.models.subnetwork_draft import SubnetworkDraftModel
    hf = _small_hf(6)
    target = sp.TargetRunner(hf)
    ids = torch.randint(0, 512, (1, 600), generator=torch.Generator().manual_seed(4))
    logits = target(ids).logits[0, -1].float()
    ar = sp.autoregressive_generate(target, ids, 24, {-1}).tokens
    assert ar[0] == int(torch.argmax(logits))
    torch.manual_seed(1)
    draft = SubnetworkDraftModel(hf, [0, 3, 5], BridgeConfig(init_std=0.02))
    res = sp.SpeculativeGenerator(hf, draft, DraftingConfig(depth=4, branch=[3, 2, 2, 1], max_nodes=24),
                                  target).generate(ids, 24, {-1})
    assert res.tokens == ar
