"""ssd_row_topk_bf16_noalloc (no caller workspace: chunk partials in the library's static device
array) against ssd_row_topk_bf16 with a workspace, through the C ABI: bit-identical tokens,
values and log-sum-exps on two calls in a row, the second smaller (fewer rows, a narrower
vocabulary subset, another mode and k), plus the size limit rejected on the host."""

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _noalloc(logits, m, n, k, mode, vocab_ids, tok, val, lse):
    from ssd import _lib, ops

    _lib.call("ssd_row_topk_bf16_noalloc", logits.data_ptr(), logits.stride(0), m, n, k, mode,
              vocab_ids.data_ptr() if vocab_ids is not None else None, tok.data_ptr(),
              val.data_ptr() if val is not None else None, lse.data_ptr() if lse is not None else None, ops.stream())


def _case(m, n, k, mode, subset, seed):
    from ssd import ops

    g = torch.Generator(device="cpu").manual_seed(seed)
    logits = (torch.randn(m, n, generator=g) * 3).to(torch.bfloat16)
    logits[:, 5] = logits[:, 9] = logits.max()  # exact ties: lower column first
    logits = logits.to(DEV)
    vocab_ids = None
    if subset:
        vocab_ids = torch.randperm(128256, generator=g)[:n].sort().values.to(torch.int32).to(DEV)
    outs = []
    for fn in ("ws", "noalloc"):
        tok = torch.full((m * k,), -7, dtype=torch.int32, device=DEV)
        val = torch.full((m * k,), -7.0, dtype=torch.float32, device=DEV)
        lse = torch.full((m,), -7.0, dtype=torch.float32, device=DEV) if mode == 1 else None
        if fn == "ws":
            ops.row_topk(logits, m, n, k, mode, vocab_ids, tok, val, lse)
        else:
            _noalloc(logits, m, n, k, mode, vocab_ids, tok, val, lse)
        torch.cuda.synchronize()
        outs.append((tok.cpu(), val.cpu(), None if lse is None else lse.cpu()))
    (t0, v0, l0), (t1, v1, l1) = outs
    assert torch.equal(t0, t1), f"tokens differ (m={m}, n={n}, k={k}, mode={mode})"
    assert torch.equal(v0, v1)
    assert (l0 is None) == (l1 is None) and (l0 is None or torch.equal(l0, l1))
    assert int(t1.min()) >= 0
    return t1


def test_noalloc_topk_matches_workspace_entry_point():
    print("noalloc topk: 64 x 128256, k 4, log-softmax", flush=True)
    big = _case(64, 128256, 4, 1, False, seed=1)
    assert int(big[0]) == 5  # the tied maximum at columns 5 and 9: lower column first
    print("noalloc topk: 9 x 32768 subset, k 1, raw argmax", flush=True)
    _case(9, 32768, 1, 0, True, seed=2)


def test_noalloc_topk_rejects_sizes_beyond_its_scratch():
    from ssd import _lib

    logits = torch.zeros(100, 262144, dtype=torch.bfloat16, device=DEV)
    tok = torch.zeros(100, dtype=torch.int32, device=DEV)
    with pytest.raises(_lib.SsdError, match="static scratch holds 4096"):
        _noalloc(logits, 100, 262144, 1, 0, None, tok, None, None)
    _noalloc(logits, 16, 262144, 1, 0, None, tok, None, None)  # 16 x 64 partials fit
    torch.cuda.synchronize()
    assert int(tok[:16].max()) == 0
