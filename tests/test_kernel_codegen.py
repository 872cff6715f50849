"""Code-generation guard for the prefill GEMM (csrc/prefill.hip, prefill_gemm4_kernel).

Its k loop issues the MFMAs as inline assembly, with the accumulators bound to the accumulator
registers, and waits for its own global-to-LDS loads with hand-counted ``s_waitcnt vmcnt(N)``. Both
are sound only while the loop holds nothing else, because the compiler treats inline assembly as
opaque:

* it inserts no wait states between its own VALU write of a register and an asm MFMA that reads
  it (a register copy or an accumulator-register move right before an MFMA gives that MFMA stale
  operands: wrong results, no error);
* a spill store or reload is a vector-memory operation that ``vmcnt`` also counts, so the
  hand-counted wait would let the barrier pass before the operands it waits for have landed.

Register pressure decides whether the allocator adds such instructions, and an epilogue change far
from the loop can tip it. This test compiles the file for gfx950 with the library's own flags and
checks every instantiation: between its first and last MFMA there is no accumulator-register move,
no vector-memory instruction other than the global-to-LDS loads, and no copy into a register that
one of the next few MFMAs reads; and the kernel has no scratch (private segment) at all.
"""

import os
import re
import shutil
import subprocess
import sys
import tempfile

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "subnetwork-speculative-decoding_amd")
SRC = os.path.join(PKG, "csrc", "prefill.hip")
KERNEL = "prefill_gemm4_kernel"

VMEM = re.compile(r"^\s*(global_|buffer_|scratch_|flat_)")
VREG = re.compile(r"v\[(\d+):(\d+)\]|v(\d+)\b")


def _regs(text):
    out = set()
    for a, b, one in VREG.findall(text):
        if one:
            out.add(int(one))
        else:
            out.update(range(int(a), int(b) + 1))
    return out


@pytest.fixture(scope="module")
def asm():
    sys.path.insert(0, PKG)
    import build

    if not os.path.exists(build.HIPCC) and not shutil.which("hipcc"):
        pytest.skip("hipcc not available")
    with tempfile.TemporaryDirectory() as d:
        out = os.path.join(d, "prefill.s")
        cmd = [build.HIPCC, *build.FLAGS, "-I", os.path.join(REPO, "include"), "--offload-device-only", "-S", SRC,
               "-o", out]
        r = subprocess.run(cmd, capture_output=True, text=True)
        assert r.returncode == 0, r.stderr[-2000:]
        return open(out).read()


def _kernels(asm_text):
    names = re.findall(rf"^(_ZN3ssd\d+{KERNEL}\w*):", asm_text, re.M)
    for name in names:
        body = asm_text[asm_text.index(name + ":"):]
        body = body[:body.index("s_endpgm")]
        meta = asm_text[asm_text.index(f".amdhsa_kernel {name}"):]
        private = int(re.search(r"\.amdhsa_private_segment_fixed_size (\d+)", meta).group(1))
        yield name, body.splitlines(), private


def test_prefill_gemm_k_loop_holds_only_its_loads_and_mfmas(asm):
    found = list(_kernels(asm))
    assert len(found) >= 6, [n for n, _, _ in found]  # {store, swiglu, q/k/v} x {row scales, none}
    for name, lines, private in found:
        assert private == 0, f"{name}: {private} bytes of scratch"
        idx = [i for i, l in enumerate(lines) if "v_mfma" in l]
        loop = lines[idx[0]:idx[-1] + 1]
        bad = [l.strip() for l in loop if "v_accvgpr" in l]
        assert not bad, f"{name}: accumulator-register moves in the k loop: {bad[:4]}"
        bad = [l.strip() for l in loop if VMEM.match(l) and "global_load_lds" not in l]
        assert not bad, f"{name}: vector-memory instructions besides the operand loads in the k loop: {bad[:4]}"
        # a VALU copy whose destination one of the next 4 instructions' MFMAs reads
        for i, l in enumerate(loop):
            s = l.strip()
            if not s.startswith("v_mov_b"):
                continue
            dst = _regs(s.split(None, 1)[1].split(",")[0])
            for nxt in loop[i + 1:i + 5]:
                if "v_mfma" in nxt:
                    srcs = _regs(",".join(nxt.split(",")[1:3]))
                    assert not (dst & srcs), f"{name}: {s} feeds {nxt.strip()} without wait states"
