"""Code-generation guard for tree attention's shared tile loop (csrc/attention.hip, attn_partial_kernel).

Each iteration of that loop issues the query-fragment loads of a later tile and, in the fold, two
record stores per thread, and later waits (``s_waitcnt vmcnt(N)``) for the query fragments. The
counter is in order, so a wait whose N is smaller than the number of operations issued after the
fragment loads also waits for whatever came before them. The compiler derives N from the state it
merges at the loop head; when the prologue's loads were still counted there, it chose N so small
that every other tile waited for the stores issued just before it -- a full store round trip in
the middle of the loop, ~1 us per call at the 8B verify shape, with identical results.

The test compiles the file for gfx950 with the library's own flags, finds the shared loop of the
head_dim-128 kernel (the loop with MFMAs and stores whose softmax has no key mask, i.e. the fewest
``v_cndmask``), walks its instructions cyclically and checks that no vmcnt wait requires a store
issued fewer than MIN_DIST instructions before it. The kernel before the fix had such a wait 60
instructions after the stores; the fixed one's nearest is ~200.
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
SRC = os.path.join(PKG, "csrc", "attention.hip")
KERNEL = "_ZN3ssd19attn_partial_kernelILi128EEEvNS_8AttnArgsE"
MIN_DIST = 120

LABEL = re.compile(r"^(\.LBB\d+_\d+):|^; %bb\.(\d+):")
VMEM = re.compile(r"^\s*(global_|buffer_|scratch_|flat_)")


@pytest.fixture(scope="module")
def kernel_lines():
    sys.path.insert(0, PKG)
    import build

    if not os.path.exists(build.HIPCC) and not shutil.which("hipcc"):
        pytest.skip("hipcc not available")
    with tempfile.TemporaryDirectory() as d:
        out = os.path.join(d, "attention.s")
        cmd = [build.HIPCC, *build.FLAGS, "-I", os.path.join(REPO, "include"), "--offload-device-only", "-S", SRC,
               "-o", out]
        r = subprocess.run(cmd, capture_output=True, text=True)
        assert r.returncode == 0, r.stderr[-2000:]
        text = open(out).read()
    body = text[text.index(KERNEL + ":"):]
    return body[:body.index("s_endpgm")].splitlines()


def _loops(lines):
    """Loop header -> the instructions of its blocks, in layout order (from the compiler's block
    comments: a header block says "Inner Loop Header", its other blocks "in Loop: Header=...")."""
    blocks, cur = [], None
    for i, line in enumerate(lines):
        m = LABEL.match(line)
        if not m:
            continue
        if cur:
            blocks.append((cur[0], i, cur[1]))
        name = m.group(1) or f"bb.{m.group(2)}"
        hm = re.search(r"Header=BB(\d+_\d+)", line)
        header = name[1:].replace("LBB", "BB") if "Inner Loop Header" in line else (f"BB{hm.group(1)}" if hm else None)
        cur = (i, header)
    if cur:
        blocks.append((cur[0], len(lines), cur[1]))
    loops = {}
    for s, e, header in blocks:
        if header:
            loops.setdefault(header, []).extend(
                l for l in lines[s:e] if l.strip() and not l.strip().startswith(";") and not LABEL.match(l))
    return loops


def test_shared_tile_loop_waits_never_cover_fresh_stores(kernel_lines):
    loops = {h: ins for h, ins in _loops(kernel_lines).items()
             if sum("v_mfma" in l for l in ins) >= 32 and any("global_store" in l for l in ins)}
    assert len(loops) >= 2, sorted(loops)  # shared and tail tile loops
    header = min(loops, key=lambda h: sum("v_cndmask" in l for l in loops[h]))
    ins = loops[header]
    n, waits = len(ins), 0
    for p, line in enumerate(ins):
        m = re.search(r"s_waitcnt\s.*vmcnt\((\d+)\)", line)
        if not m:
            continue
        waits += 1
        allowed, seen = int(m.group(1)), 0
        for back in range(1, n):  # cyclically: through the back edge into the previous iteration
            q = (p - back) % n
            if VMEM.match(ins[q]):
                seen += 1
                if seen > allowed:
                    # the oldest operation this wait may leave outstanding is behind us: everything
                    # from here back must be complete
                    if "global_store" in ins[q]:
                        assert back >= MIN_DIST, (f"{header}: '{line.strip()}' waits for a store issued {back} "
                                                  f"instructions earlier")
    assert waits > 0, f"{header}: no vmcnt waits found; the loop no longer loads its query fragments"
