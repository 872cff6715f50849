"""Model loading, draft construction and the bridge-checkpoint layout (reference ssd/runtime.py).

* ``build_draft`` keeps the reference's behaviour (ssd/runtime.py:101-138): bridges from a
  checkpoint path or ``"latest"`` (online > stage2 > stage1 under
  ``{output_dir}/{L-profile}/``), cast to the base dtype at inference, and the draft vocabulary
  from ``draft_vocab.pt`` or ``top_vocab(token_freq.pt, N, eos)``.
* ``load_base_model`` loads a *local* HF checkpoint directory (no network here) and packs it
  into HBM, or builds a seeded random-init model of a named Llama shape when
  ``model.base_model`` is ``synthetic:<shape>`` (``llama32_1b``, ``llama3_8b``, ``llama3_70b``).
"""

from __future__ import annotations

import logging
import os
from pathlib import Path
from typing import Optional

import torch

from ssd.config import SSDConfig, profile_name
from ssd.models.llama import LlamaShape, MI355XLlama
from ssd.models.subnetwork_draft import SubnetworkDraftModel, as_device_model

log = logging.getLogger("ssd")

SHAPES = {
    "llama32_1b": LlamaShape(hidden=2048, layers=16, heads=32, kv_heads=8, head_dim=64, inter=8192, vocab=128256,
                             eps=1e-5, theta=500000.0),
    "llama3_8b": LlamaShape(hidden=4096, layers=32, heads=32, kv_heads=8, head_dim=128, inter=14336, vocab=128256,
                            eps=1e-5, theta=500000.0),
    "llama3_70b": LlamaShape(hidden=8192, layers=80, heads=64, kv_heads=8, head_dim=128, inter=28672, vocab=128256,
                             eps=1e-5, theta=500000.0),
}


def setup_env(level: int = logging.INFO) -> None:
    """Configure logging (the reference also reads a .env for HF tokens; nothing is fetched here)."""
    logging.basicConfig(level=level, format="%(asctime)s %(levelname)s %(message)s", datefmt="%H:%M:%S")


def resolve_device(name: str = "auto") -> torch.device:
    if name != "auto":
        return torch.device(name)
    if not torch.cuda.is_available():
        raise RuntimeError("no HIP device: this package runs on MI355X (gfx950) only")
    return torch.device("cuda", torch.cuda.current_device())


def device_memory_gb(device: torch.device) -> float:
    return torch.cuda.memory_reserved(device) / 2**30 if device.type == "cuda" else 0.0


def load_base_model(cfg: SSDConfig, device: Optional[torch.device] = None, seed: int = 0) -> MI355XLlama:
    name = cfg.model.base_model
    dev = device or resolve_device(cfg.model.device)
    if cfg.model.torch_dtype != "bfloat16":
        raise ValueError("this package runs bf16 models (model.torch_dtype: bfloat16)")
    if name.startswith("synthetic:"):
        shape = SHAPES[name.split(":", 1)[1]]
        base = MI355XLlama.synthetic(shape, seed=seed, device=dev)
    elif os.path.isdir(name):
        from transformers import AutoModelForCausalLM

        hf = AutoModelForCausalLM.from_pretrained(name, dtype=torch.bfloat16, local_files_only=True)
        base = MI355XLlama.from_hf(hf, dev)
        gc = getattr(hf, "generation_config", None)
        base.generation_config.eos_token_id = getattr(gc, "eos_token_id", None)
        del hf
    else:
        raise FileNotFoundError(f"{name!r} is neither a local checkpoint directory nor synthetic:<shape> "
                                f"({', '.join(SHAPES)}); there is no network access to the model hub")
    cfg.validate_against(base.shape.layers)
    return base


def checkpoint_path(cfg: SSDConfig, stage) -> Path:
    """stage: 1, 2 or "online" -> {output_dir}/{L-profile}/stage{1,2}.pt | online.pt."""
    name = f"stage{stage}.pt" if isinstance(stage, int) else f"{stage}.pt"
    return Path(cfg.training.output_dir) / profile_name(cfg.draft_layers) / name


def latest_checkpoint(cfg: SSDConfig) -> Optional[Path]:
    for stage in ("online", 2, 1):
        p = checkpoint_path(cfg, stage)
        if p.exists():
            return p
    return None


def eos_ids_of(base) -> set:
    eos = getattr(getattr(base, "generation_config", None), "eos_token_id", None)
    if eos is None:
        return set()
    return set(eos if isinstance(eos, list) else [eos])


def build_draft(cfg: SSDConfig, base, checkpoint="latest", inference: bool = False) -> SubnetworkDraftModel:
    draft = SubnetworkDraftModel(base, cfg.draft_layers, cfg.bridge)
    name = profile_name(cfg.draft_layers)
    if checkpoint == "latest":
        checkpoint = latest_checkpoint(cfg)
        if checkpoint is None and draft.bridge_specs:
            log.warning("no trained bridges for %s under %s; using untrained bridges", name, cfg.training.output_dir)
    if checkpoint is not None:
        draft.load_bridges(str(checkpoint))
        log.info("loaded bridges for %s from %s", name, checkpoint)
    if inference:
        draft.bridges.to(torch.bfloat16)
    if inference and cfg.drafting.draft_vocab:
        from ssd.data.token_freq import token_freq_path, top_vocab

        explicit = Path(cfg.training.output_dir) / "draft_vocab.pt"
        if explicit.exists():
            ids = torch.load(explicit, weights_only=True)[: cfg.drafting.draft_vocab]
            draft.set_vocab_subset(ids.sort().values)
        else:
            path = token_freq_path(cfg)
            if not path.exists():
                raise FileNotFoundError(f"{path} missing: write token frequencies there (torch.save of a [V] tensor)")
            counts = torch.load(path, weights_only=True)
            draft.set_vocab_subset(top_vocab(counts, cfg.drafting.draft_vocab, eos_ids_of(as_device_model(base))))
    return draft
