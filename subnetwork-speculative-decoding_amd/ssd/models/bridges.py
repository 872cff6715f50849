"""Transition bridges ``out = x + MLP(RMSNorm(x))`` (ssd/models/bridges.py in the reference).

The module tree (``norm.weight``, ``mlp.body.{0,2}.*``, ``mlp.out_proj.*``; or
``mlp.{gate,up,out}_proj.*`` for swiglu) matches the reference's, so bridge checkpoints
written by it load unchanged. Parameters live in ``dtype`` (fp32 by default) for training
compatibility; at inference the bridge is cast to bf16 (ssd/runtime.py:120-121 in the
reference) and packed once for the gfx950 kernels (``packed()``): RMSNorm kernel, then the
weight-streaming GEMMs with bias + activation and a final bias + residual epilogue, each
result rounded to bf16 like the reference's bf16 ``nn.Linear`` chain.
"""

from __future__ import annotations

import math
from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from ssd import _lib, ops
from ssd.config import BridgeConfig

_ACTS = {"silu": nn.SiLU, "gelu": nn.GELU, "relu": nn.ReLU}


class RMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float = 1e-5):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        xf = x.float()
        return self.weight * (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)).to(x.dtype)


class _PlainMLP(nn.Module):
    def __init__(self, d_model: int, hidden: int, num_layers: int, activation: str, bias: bool):
        super().__init__()
        if num_layers not in (2, 3):
            raise ValueError(f"mlp bridge supports 2 or 3 layers, got {num_layers}")
        dims = [d_model] + [hidden] * (num_layers - 1)
        mods: list = []
        for a, b in zip(dims[:-1], dims[1:]):
            mods += [nn.Linear(a, b, bias=bias), _ACTS[activation]()]
        self.body = nn.Sequential(*mods)
        self.out_proj = nn.Linear(hidden, d_model, bias=bias)

    def forward(self, x):
        return self.out_proj(self.body(x))


class _SwiGLU(nn.Module):
    def __init__(self, d_model: int, hidden: int, bias: bool):
        super().__init__()
        self.gate_proj = nn.Linear(d_model, hidden, bias=bias)
        self.up_proj = nn.Linear(d_model, hidden, bias=bias)
        self.out_proj = nn.Linear(hidden, d_model, bias=bias)

    def forward(self, x):
        return self.out_proj(F.silu(self.gate_proj(x)) * self.up_proj(x))


class PackedBridge:
    """bf16 packed form run by the kernels."""

    def __init__(self, bridge: "TransitionBridge", device):
        def bf(t):
            return None if t is None else t.detach().to(device=device, dtype=torch.bfloat16).contiguous()

        self.d = bridge.d_model
        self.hidden = bridge.hidden
        self.eps = bridge.norm.eps
        self.norm = bf(bridge.norm.weight)
        self.swiglu = isinstance(bridge.mlp, _SwiGLU)
        if self.swiglu:
            from ssd.models.llama import gate_up_row_map

            m = bridge.mlp
            w = torch.cat([bf(m.gate_proj.weight), bf(m.up_proj.weight)], 0)
            self.gu = ops.pack_weight(w, gate_up_row_map(self.hidden), col_scale=self.norm)  # norm folded
            self.bg, self.bu = bf(m.gate_proj.bias), bf(m.up_proj.bias)
            self.body = []
        else:
            self.body = []
            lins = [mod for mod in bridge.mlp.body if isinstance(mod, nn.Linear)]
            acts = [mod for mod in bridge.mlp.body if not isinstance(mod, nn.Linear)]
            for i, (lin, act) in enumerate(zip(lins, acts)):
                name = {nn.SiLU: "silu", nn.GELU: "gelu", nn.ReLU: "relu"}[type(act)]
                w = ops.pack_weight(bf(lin.weight), col_scale=self.norm if i == 0 else None)  # norm folded in first
                self.body.append((w, bf(lin.bias), lin.out_features, lin.in_features, name))
        out = bridge.mlp.out_proj
        self.out = ops.pack_weight(bf(out.weight), residual=True)
        self.out_bias = bf(out.bias)
        self._native: Optional[_lib.SsdBridgeW] = None

    def native(self) -> "_lib.SsdBridgeW":
        """C descriptor (SsdBridgeW) for ssd_forward; the tensors it points at live on this object."""
        if self._native is None:
            def p(t):
                return None if t is None else t.data_ptr()

            st = _lib.SsdBridgeW()
            st.norm, st.eps, st.hidden, st.swiglu, st.n_body = p(self.norm), self.eps, self.hidden, int(self.swiglu), \
                len(self.body)
            for i, (w, b, n, _, act) in enumerate(self.body):
                st.body_w[i], st.body_b[i], st.body_n[i], st.body_act[i] = p(w), p(b), n, ops.ACT[act]
            if self.swiglu:
                st.gu, st.bg, st.bu = p(self.gu), p(self.bg), p(self.bu)
            st.out, st.out_b = p(self.out), p(self.out_bias)
            self._native = st
        return self._native

    def body_(self, h: torch.Tensor, m: int, mids: list) -> tuple:
        """MLP body over RMSNorm(h[:m]) (the norm folded into the first GEMM); returns (output,
        its width)."""
        if self.swiglu:
            ops.gemm_swiglu(h, m, self.gu, self.hidden, self.d, mids[0], self.bg, self.bu, norm_eps=self.eps)
            return mids[0], self.hidden
        cur, k = h, self.d
        for i, (w, b, n, kin, act) in enumerate(self.body):
            dst = mids[i % 2]
            ops.gemm(cur, m, w, n, kin, dst, bias=b, act=act, norm_eps=self.eps if i == 0 else 0.0)
            cur, k = dst, n
        return cur, k

    def apply_(self, h: torch.Tensor, m: int, mids: list, part: torch.Tensor) -> None:
        """h[:m] <- h + MLP(RMSNorm(h)) with the kernels of ssd_forward (body GEMMs, then the
        out_proj with the residual add in its epilogue)."""
        cur, k = self.body_(h, m, mids)
        ops.gemm_residual(cur, m, self.out, self.d, k, h, part, bias=self.out_bias)


class TransitionBridge(nn.Module):
    """Residual MLP bridge ``out = x + MLP(RMSNorm(x))`` (reference ssd/models/bridges.py:68-135)."""

    def __init__(self, d_model: int, hidden_dim: Optional[int] = None, num_layers: int = 2, mlp_type: str = "mlp",
                 activation: str = "silu", bias: bool = True, init_std: float = 1e-3, norm_eps: float = 1e-5,
                 dtype: torch.dtype = torch.float32):
        super().__init__()
        self.d_model = d_model
        self.hidden = hidden_dim or d_model
        self.norm = RMSNorm(d_model, eps=norm_eps)
        if mlp_type == "mlp":
            if activation not in _ACTS:
                raise ValueError(f"unknown activation {activation!r}")
            self.mlp = _PlainMLP(d_model, self.hidden, num_layers, activation, bias)
        elif mlp_type == "swiglu":
            if num_layers != 2:
                raise ValueError("swiglu bridge is a fixed gate/up + down block; set num_layers=2")
            self.mlp = _SwiGLU(d_model, self.hidden, bias)
        else:
            raise ValueError(f"unknown mlp_type {mlp_type!r}")
        self.reset_parameters(init_std)
        self.to(dtype)
        self._packed: Optional[PackedBridge] = None

    @classmethod
    def from_config(cls, d_model: int, cfg: BridgeConfig) -> "TransitionBridge":
        return cls(d_model, cfg.hidden_dim, cfg.num_layers, cfg.mlp_type, cfg.activation, cfg.bias, cfg.init_std,
                   cfg.norm_eps, getattr(torch, cfg.dtype))

    @torch.no_grad()
    def reset_parameters(self, init_std: float = 1e-3) -> None:
        """Output projection N(0, init_std) (zeros when init_std == 0), inner projections
        N(0, 1/sqrt(fan_in)), zero biases, unit norm (reference bridges.py:118-129)."""
        for name, mod in self.mlp.named_modules():
            if not isinstance(mod, nn.Linear):
                continue
            if name == "out_proj":
                if init_std > 0:
                    nn.init.normal_(mod.weight, std=init_std)
                else:
                    mod.weight.zero_()
            else:
                nn.init.normal_(mod.weight, std=1.0 / math.sqrt(mod.in_features))
            if mod.bias is not None:
                mod.bias.zero_()
        self.norm.weight.fill_(1.0)
        self._packed = None

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """Torch form, kept for training-time use and API compatibility; decoding uses ``packed()``."""
        p = self.norm.weight
        xi = x.to(device=p.device, dtype=p.dtype)
        return (xi + self.mlp(self.norm(xi))).to(x.dtype)

    def packed(self, device) -> PackedBridge:
        if self._packed is None:
            if self.hidden % 32 or self.d_model % 32:
                raise ValueError("bridge dims must be multiples of 32 for the packed kernels")
            self._packed = PackedBridge(self, device)
        return self._packed

    def _apply(self, fn, *args, **kwargs):  # .to()/.cuda(): drop the packed copy if parameters changed
        before = [(p.data_ptr(), p.dtype, p.device) for p in self.parameters()]
        out = super()._apply(fn, *args, **kwargs)
        if [(p.data_ptr(), p.dtype, p.device) for p in self.parameters()] != before:
            self._packed = None
        return out

    def load_state_dict(self, *args, **kwargs):
        self._packed = None
        return super().load_state_dict(*args, **kwargs)
