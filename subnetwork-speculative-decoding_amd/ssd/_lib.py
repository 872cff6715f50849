"""Loader for the gfx950 C-ABI library (``libssd_mi355x.so``, declared in include/ssd_mi355x.h).

There is no fallback: if the library is missing or cannot be loaded, every hot-path call
raises. Build it with ``python subnetwork-speculative-decoding_amd/build.py``.
"""

from __future__ import annotations

import ctypes as C
import hashlib
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libssd_mi355x.so")
_PKG = os.path.dirname(_HERE)
SOURCE_DIRS = (os.path.join(_PKG, "csrc"), os.path.join(os.path.dirname(_PKG), "include"))


def source_hash() -> str:
    """First 16 hex digits of a sha256 over the HIP sources and C headers the library is built
    from (file names and contents, sorted); build.py compiles it into the library, and load()
    refuses a library whose hash differs from the sources beside it (a stale build)."""
    h = hashlib.sha256()
    for d in SOURCE_DIRS:
        for f in sorted(os.listdir(d)):
            if f.endswith((".hip", ".h")):
                h.update(f.encode() + b"\0")
                with open(os.path.join(d, f), "rb") as fh:
                    h.update(fh.read())
                h.update(b"\0")
    return h.hexdigest()[:16]

P = C.c_void_p
I32 = C.c_int
I64 = C.c_int64
F32 = C.c_float
U64 = C.c_uint64


class SsdTree(C.Structure):
    _fields_ = [(n, P) for n in ("tokens", "parents", "depths", "ranks", "draft_pos", "scores", "meta", "vtokens",
                                 "vparents", "vdepths", "vranks", "vorig", "vmeta")] + [("cap", C.c_int32)]


class SsdRows(C.Structure):
    _fields_ = [(n, P) for n in ("ids", "pos", "slot", "prefix", "depth", "anc")] + [("cap", C.c_int32),
                                                                                      ("kv_off", P)]


class SsdLayerW(C.Structure):
    _fields_ = [(n, P) for n in ("wqkv", "wo", "wgu", "wd", "ln1", "ln2")]


class SsdModel(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("hidden", "heads", "kv_heads", "head_dim", "inter", "vocab", "n_layers")] + [
        ("eps", F32), ("attn_scale", F32), ("embed", P), ("norm", P), ("cos", P), ("sin", P), ("rope_rows", I64),
        ("layers", C.POINTER(SsdLayerW)), ("mlp_fused", C.c_int32)]


class SsdBridgeW(C.Structure):
    _fields_ = [("norm", P), ("eps", F32), ("hidden", C.c_int32), ("swiglu", C.c_int32), ("n_body", C.c_int32),
                ("body_w", P * 2), ("body_b", P * 2), ("body_n", C.c_int32 * 2), ("body_act", C.c_int32 * 2),
                ("gu", P), ("bg", P), ("bu", P), ("out", P), ("out_b", P)]


class SsdPlan(C.Structure):
    _fields_ = [("n_steps", C.c_int32), ("layer_ids", C.POINTER(C.c_int32)),
                ("pre_bridge", C.POINTER(C.POINTER(SsdBridgeW))), ("pre_norm", C.POINTER(SsdBridgeW)),
                ("head_w", P), ("head_n", C.c_int32)]


class SsdBuffers(C.Structure):
    _fields_ = [(n, P) for n in ("h", "x", "q", "attn", "mlp", "mid0", "mid1")] + [
        ("m_cap", C.c_int32), ("mid_cols", C.c_int32), ("k_arena", P), ("vt_arena", P), ("cache_cap", I64),
        ("attn_ws", P), ("attn_ws_floats", I64), ("logits", P), ("ld_logits", I64), ("part", P), ("part_floats", I64),
        ("sync", P)]


class SsdQkvEpilogue(C.Structure):
    _fields_ = [("heads", C.c_int32), ("kv_heads", C.c_int32), ("head_dim", C.c_int32), ("cos", P), ("sin", P),
                ("rope_rows", I64), ("pos0", C.c_int32), ("k_cache", P), ("vt_cache", P), ("max_len", I64)]


class SsdPrefillBuffers(C.Structure):
    _fields_ = [("m_cap", C.c_int32)] + [(n, P) for n in ("h", "q", "attn", "act", "k_arena", "vt_arena")] + [
        ("cache_cap", I64), ("logits", P)]


_PROTOS = {
    "ssd_last_error": (C.c_char_p, []),
    "ssd_abi_version": (I32, []),
    "ssd_launch_count": (U64, []),
    "ssd_build_hash": (C.c_char_p, []),
    "ssd_device_arch": (I32, [C.c_char_p, I32]),
    "ssd_packed_weight_elems": (I64, [I32, I32]),
    "ssd_gemm_weight_group": (I32, [I32, I32]),
    "ssd_mlp_group": (I32, [I32, I32]),
    "ssd_mlp_sync_words": (I64, []),
    "ssd_mlp_timeout_word": (I32, []),
    "ssd_mlp_bf16": (I32, [P, I64, I32, P, P, I32, I32, F32, P, I64, P, I64, P, P]),
    "ssd_pack_weight_bf16": (I32, [P, I64, I32, I32, P, I32, I32, P, P, P]),
    "ssd_gemm_bf16": (I32, [P, I64, I32, P, I32, I32, F32, P, I64, P, I32, P, I64, P]),
    "ssd_gemm_swiglu_bf16": (I32, [P, I64, I32, P, I32, I32, F32, P, I64, P, P, P]),
    "ssd_gemm_qkv_rope_bf16": (I32, [P, I64, I32, P, I32, F32, I32, I32, I32, P, P, I64, P, P, P, I64, P, P, I64, P]),
    "ssd_attn_workspace_floats": (I32, [I32, I32, I32, I64]),
    "ssd_attn_max_depth": (I32, []),
    "ssd_tree_attention_bf16": (I32, [P, I64, I32, I32, I32, I32, P, P, I64, P, P, P, I32, I32, F32, P, I64, P,
                                      I64, P]),
    "ssd_rmsnorm_bf16": (I32, [P, I64, I32, I32, P, F32, P, I64, P]),
    "ssd_embed_bf16": (I32, [P, I32, P, I64, I32, P, I64, P]),
    "ssd_kv_compact_bf16": (I32, [P, P, I32, I32, I32, I64, I32, P, P, I32, P, P]),
    "ssd_row_topk_ws_bytes": (I64, [I32, I32]),
    "ssd_row_topk_bf16": (I32, [P, I64, I32, I32, I32, I32, P, P, P, P, P, I64, P]),
    "ssd_row_topk_bf16_noalloc": (I32, [P, I64, I32, I32, I32, I32, P, P, P, P, P]),
    "ssd_row_topk_partial_bf16": (I32, [P, I64, I32, I32, I32, I32, P, I64, P]),
    "ssd_row_topk_merge": (I32, [P, I64, I32, I32, I32, I32, P, P, P, P, P]),
    "ssd_gemm_topk_parts": (I32, [I32]),
    "ssd_gemm_topk_bf16": (I32, [P, I64, I32, P, I32, I32, F32, I32, I32, P, I64, P, I64, P]),
    "ssd_tree_limits": (I32, [P]),
    "ssd_round_begin": (I32, [C.POINTER(SsdTree), C.POINTER(SsdRows), I32, P, P, P]),
    "ssd_tree_level": (I32, [C.POINTER(SsdTree), I32, P, P, I32, I32, I32, I32, I32, I32, I32, C.POINTER(SsdRows),
                             I32, P, P]),
    "ssd_tree_level_topk": (I32, [C.POINTER(SsdTree), I32, P, I64, I32, I32, P, I32, I32, I32, I32, I32, I32,
                                  I32, C.POINTER(SsdRows), I32, P, P]),
    "ssd_tree_finalize": (I32, [C.POINTER(SsdTree), I32, I32, P, C.POINTER(SsdRows), I32, P, P]),
    "ssd_accept_greedy": (I32, [C.POINTER(SsdTree), P, I32, P, P, P, P, P, P]),
    "ssd_gemm_splits": (I32, [I32, I32]),
    "ssd_gemm_partial_bf16": (I32, [P, I64, I32, P, I32, I32, P, I64, I64, P]),
    "ssd_gemm_finalize_bf16": (I32, [P, I64, I64, I32, I32, I32, P, I64, P, I32, P, I64, P]),
    "ssd_qkv_rope_finalize_bf16": (I32, [P, I64, I64, I32, I32, I32, I32, I32, P, P, I64, P, P, P, I64, P, P, I64, P]),
    "ssd_add_rmsnorm_bf16": (I32, [P, I64, I64, I32, P, P, I64, I32, I32, P, F32, P, I64, P]),
    "ssd_gemm_residual_group": (I32, [I32, I32]),
    "ssd_gemm_residual_floats": (I64, [I32, I32, I32]),
    "ssd_gemm_residual_bf16": (I32, [P, I64, I32, P, I32, I32, P, P, I64, P, I64, P]),
    "ssd_sample_limits": (I32, [P]),
    "ssd_sample_ws_bytes": (I64, [I32, I32]),
    "ssd_warp_probs_bf16": (I32, [P, I64, I32, I32, P, P, I32, F32, F32, P, I32, P, I64, P, I64, P]),
    "ssd_gumbel_topk": (I32, [P, I64, I32, I32, I32, P, I32, U64, U64, P, P, P, I64, P]),
    "ssd_sample_rows": (I32, [P, I64, I32, I32, U64, U64, P, P, I64, P]),
    "ssd_sample_top64_ws_bytes": (I64, [I32, I32]),
    "ssd_sample_top64_bf16": (I32, [P, I64, I32, I32, F32, F32, U64, U64, P, P, I64, P]),
    "ssd_accept_sample": (I32, [C.POINTER(SsdTree), P, I64, P, I64, I32, I32, I32, U64, U64, P, I64, I32, P, P, P, P,
                                P]),
    "ssd_accept_sample_trials": (I32, [P, I64, P, I64, I32, P, P, I32, C.POINTER(C.c_int32), U64, U64, I32, P, P, P]),
    "ssd_forward": (I32, [C.POINTER(SsdModel), C.POINTER(SsdPlan), C.POINTER(SsdBuffers), C.POINTER(SsdRows), I32,
                          I32, I32, I32, I32, P]),
    "ssd_prefill_row_scale_bf16": (I32, [P, I64, I32, I32, F32, P, P]),
    "ssd_prefill_gemm_bf16": (I32, [P, I64, I32, P, I32, I32, I32, P, I32, P, I64, P, I64,
                                    C.POINTER(SsdQkvEpilogue), P]),
    "ssd_prefill_attention_bf16": (I32, [P, I64, I32, I32, I32, I32, I32, P, P, I64, F32, P, I64, P]),
    "ssd_prefill": (I32, [C.POINTER(SsdModel), P, C.POINTER(SsdPrefillBuffers), P, I32, I32, P]),
}

EXPORTED = tuple(_PROTOS)
ABI_VERSION = 6  # descriptor struct layouts (SsdModel.mlp_fused, SsdBuffers.sync, SsdRows.kv_off); pos_base
# arguments; ssd_tree_level_topk's record count S; ssd_prefill_gemm_bf16 takes row scales

_lib = None


class SsdError(RuntimeError):
    pass


def load(path: str = LIB_PATH):
    """Load the library (once). Raises if it is absent: there is no non-HIP path."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise ImportError(f"{path} not found: build it with `python subnetwork-speculative-decoding_amd/build.py`")
    lib = C.CDLL(path)
    for name, (res, args) in _PROTOS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.ssd_abi_version() != ABI_VERSION:
        raise ImportError(f"{path} has ABI {lib.ssd_abi_version()}, this package needs {ABI_VERSION}: rebuild it")
    if all(os.path.isdir(d) for d in SOURCE_DIRS):
        built, now = lib.ssd_build_hash().decode(), source_hash()
        if built != now:
            raise ImportError(f"{path} was built from other sources (hash {built}, sources {now}): rebuild it with "
                              "`python subnetwork-speculative-decoding_amd/build.py`")
    _lib = lib
    return lib


def call(name: str, *args) -> int:
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.ssd_last_error().decode(errors="replace")
        if rc == 1:
            raise ValueError(f"{name}: {msg}")
        raise SsdError(f"{name}: {msg}")
    return rc
