"""The C-ABI library loads and exports every entry point include/ssd_mi355x.h declares (CPU only,
no compute calls), and the Python binding covers exactly that set."""

import ctypes
import os
import re

import pytest

from conftest import REPO

HEADER = os.path.join(REPO, "include", "ssd_mi355x.h")


def declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+char\s*\*|u?int64_t|int)\s+(ssd_\w+)\s*\(", text, re.M)))


def test_header_declares_entry_points():
    names = declared()
    assert "ssd_tree_attention_bf16" in names and "ssd_kv_compact_bf16" in names and len(names) >= 18


def test_library_exports_every_declared_symbol():
    from ssd import _lib

    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail("libssd_mi355x.so is not built (run subnetwork-speculative-decoding_amd/build.py)")
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"


def test_binding_matches_header():
    from ssd import _lib

    assert sorted(_lib.EXPORTED) == declared()


def test_host_only_entry_points():
    from ssd import _lib

    lib = _lib.load()
    assert lib.ssd_abi_version() == _lib.ABI_VERSION == 6
    assert lib.ssd_packed_weight_elems(17, 40) == 128 * 64  # rows padded to 128, K to 32
    assert [lib.ssd_gemm_weight_group(n, 4096) for n in (4096, 8192, 28672, 128256)] == [1, 2, 4, 8]
    assert lib.ssd_gemm_weight_group(4096, 100) == 0
    # fused MLP plans: Llama-3.2-1B, -3-8B, -3-70B shapes; none for a small MLP
    assert [lib.ssd_mlp_group(i, h) for i, h in ((8192, 2048), (14336, 4096), (28672, 8192), (1024, 256))] == [
        4, 7, 14, 0]
    assert lib.ssd_mlp_sync_words() >= 258 and 0 <= lib.ssd_mlp_timeout_word() < lib.ssd_mlp_sync_words()
    assert lib.ssd_build_hash().decode() == _lib.source_hash()  # built from the sources beside it
    lim = (ctypes.c_int32 * 3)()
    assert lib.ssd_tree_limits(lim) == 0 and list(lim) == [1024, 32, 32]
    assert lib.ssd_attn_max_depth() == 32
    # argument validation happens on the host, before any launch
    rc = lib.ssd_gemm_bf16(None, 0, 1, None, 16, 32, 0.0, None, 0, None, 0, None, 0, None)
    assert rc == 1 and b"null" in lib.ssd_last_error()


def test_descriptor_structs_match_c_layout(tmp_path):
    """The ctypes mirrors of the descriptor structs have the C compiler's sizes and offsets."""
    import ctypes as C
    import subprocess

    from ssd import _lib

    structs = {name: getattr(_lib, name) for name in ("SsdTree", "SsdRows", "SsdLayerW", "SsdModel", "SsdBridgeW",
                                                       "SsdPlan", "SsdBuffers", "SsdQkvEpilogue",
                                                       "SsdPrefillBuffers")}
    lines = ["#include <stdio.h>", "#include <stddef.h>", f'#include "{HEADER}"', "int main(void) {"]
    for name, T in structs.items():
        lines.append(f'printf("{name} %zu\\n", sizeof({name}));')
        for field, *_ in T._fields_:
            lines.append(f'printf("{name}.{field} %zu\\n", offsetof({name}, {field}));')
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-o", str(exe), str(src)], check=True)
    got = dict(line.split() for line in subprocess.run([str(exe)], capture_output=True, text=True,
                                                       check=True).stdout.splitlines())
    for name, T in structs.items():
        assert int(got[name]) == C.sizeof(T), name
        for field, *_ in T._fields_:
            assert int(got[f"{name}.{field}"]) == getattr(T, field).offset, f"{name}.{field}"


def test_unpack_rows_inverts_grouped_packing():
    """The tile layout written by ssd_pack_weight_bf16 (restated here from its documentation) is
    inverted by ssd.models.llama.unpack_rows for every tile grouping."""
    import torch

    from ssd.models.llama import unpack_rows

    n, k = 256, 96
    w = torch.arange(n * k, dtype=torch.float32).view(n, k).to(torch.bfloat16)
    kb = k // 32
    for group in (1, 2, 4, 8):
        packed = torch.zeros(n // 16, kb, 64, 8, dtype=torch.bfloat16)
        for nb in range(n // 16):
            for b in range(kb):
                for lane in range(64):
                    packed[nb, b, lane] = w[nb * 16 + lane % 16, b * 32 + (lane // 16) * 8: b * 32 + (lane // 16) * 8 + 8]
        grouped = packed.view(n // 16 // group, group, kb, 64, 8).transpose(1, 2).reshape(-1)  # [g][kb][nb%g]
        ids = torch.tensor([0, 5, 17, 100, 255])
        assert torch.equal(unpack_rows(grouped, n, k, ids, group), w[ids])



def test_every_call_site_passes_the_declared_argument_count():
    """Each _lib.call("ssd_x", ...) in the package, bench.py and the tests passes exactly as many
    arguments as the ctypes prototype of ssd_x declares (caught on the CPU, before a GPU run)."""
    import ast
    import glob

    from ssd import _lib

    files = glob.glob(os.path.join(REPO, "subnetwork-speculative-decoding_amd", "ssd", "**", "*.py"), recursive=True)
    files += glob.glob(os.path.join(REPO, "tests", "*.py")) + [os.path.join(REPO, "bench.py")]
    checked = 0
    for f in files:
        for node in ast.walk(ast.parse(open(f).read())):
            if not (isinstance(node, ast.Call) and isinstance(node.func, ast.Attribute) and node.func.attr == "call"
                    and isinstance(node.func.value, ast.Name) and node.func.value.id == "_lib"):
                continue
            if not node.args or not isinstance(node.args[0], ast.Constant) or any(
                    isinstance(a, ast.Starred) for a in node.args):
                continue
            name = node.args[0].value
            assert name in _lib._PROTOS, f"{f}:{node.lineno}: {name} has no prototype"
            want = len(_lib._PROTOS[name][1])
            assert len(node.args) - 1 == want, f"{f}:{node.lineno}: {name} given {len(node.args) - 1} args, takes {want}"
            checked += 1
    assert checked > 30
