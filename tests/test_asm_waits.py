"""The decode GEMV kernels hand a wave its LDS activation copies
(buffer_load ... lds, issued before its weight / scale / zero loads) with a
counted wait: s_waitcnt vmcnt(n) lets the n loads issued after the copies stay
in flight.  The count is written in the source, the loads are emitted by the
compiler: if it merges two of them (two tiles reading one zero word), fewer
than n follow the copies and the wait no longer covers them -- a race on the
LDS slot that no numeric test catches reliably.

This compiles the library's own HIP sources to gfx950 assembly (the build's
flags) and checks, for every kernel that issues LDS copies and is not a
software-pipelined GEMM (those drain with vmcnt(0) and a barrier per stage),
that the first vmcnt wait after the last copy is at most the number of loads
issued after it, and that no LDS read comes before that wait.
"""
import os
import re
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "fastllm-py_amd")
SOURCES = ("int4_marlin.hip", "moe_int4.hip", "fp8.hip")


def _flags():
    sys.path.insert(0, PKG)
    try:
        import build_native
    finally:
        sys.path.remove(PKG)
    return build_native.HIPCC, build_native.CFLAGS


def _functions(asm: str) -> dict:
    funcs, cur = {}, None
    for line in asm.split("\n"):
        m = re.match(r"^(_Z\S+):", line)
        if m:
            cur = m.group(1)
            funcs[cur] = []
            continue
        if cur and ".Lfunc_end" in line:
            cur = None
            continue
        if cur:
            funcs[cur].append(line.strip().split(";")[0])
    return funcs


def copy_wait_violations(asm: str) -> tuple[list, int]:
    """(violations, kernels checked) for one assembly file."""
    bad, checked = [], 0
    for name, body in _functions(asm).items():
        if "gemm" in name:
            continue
        copies = [i for i, s in enumerate(body) if re.match(r"(buffer|global)_load\S* .*\blds\b", s)]
        if not copies:
            continue
        checked += 1
        after, verdict = 0, None
        for s in body[copies[-1] + 1:]:
            if re.match(r"(global|buffer)_(load|atomic)", s):
                after += 1
            m = re.match(r"s_waitcnt vmcnt\((\d+)\)", s)
            if m:
                verdict = (int(m.group(1)), after)
                break
            if s.startswith(("ds_read", "ds_load")):
                verdict = ("LDS read before any vmcnt wait", after)
                break
        if verdict is None or verdict[0] == "LDS read before any vmcnt wait" or verdict[0] > verdict[1]:
            bad.append((name, verdict))
    return bad, checked


@pytest.mark.skipif(not os.path.exists("/opt/rocm/bin/hipcc"), reason="hipcc not installed")
def test_lds_copy_waits_cover_the_copies(tmp_path):
    hipcc, cflags = _flags()
    if not shutil.which(hipcc) and not os.path.exists(hipcc):
        pytest.skip("hipcc not found")

    def compile_one(src):
        out = os.path.join(tmp_path, src.replace(".hip", ".s"))
        cmd = [hipcc, *[f for f in cflags if f != "-fPIC"], "--cuda-device-only", "-S",
               os.path.join(PKG, "csrc", src), "-o", out]
        r = subprocess.run(cmd, capture_output=True, text=True)
        assert r.returncode == 0, r.stderr[-2000:]
        return open(out).read()

    with ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        asms = list(ex.map(compile_one, SOURCES))
    total, problems = 0, []
    for src, asm in zip(SOURCES, asms):
        bad, checked = copy_wait_violations(asm)
        total += checked
        problems += [(src, n, v) for n, v in bad]
    assert total >= 40, total  # the decode GEMV / MoE instantiations were found
    assert not problems, problems


def test_checker_flags_a_short_count():
    """The rule itself on hand-written sequences: a wait above the loads that
    follow the copies, and an LDS read with no wait, are both flagged."""
    ok = "\n".join(["_Zk1:", "buffer_load_dwordx4 v1, s[0:3], 0 offen lds", "global_load_dwordx4 v[2:5], v1, s[4:5]",
                    "global_load_dword v6, v[2:3], off", "s_waitcnt vmcnt(2)", "ds_read_b128 v[8:11], v0",
                    ".Lfunc_end0:"])
    short = ok.replace("vmcnt(2)", "vmcnt(3)").replace("_Zk1", "_Zk2")
    none = ok.replace("s_waitcnt vmcnt(2)\n", "").replace("_Zk1", "_Zk3")
    assert copy_wait_violations(ok) == ([], 1)
    assert copy_wait_violations(short)[0] == [("_Zk2", (3, 2))]
    assert copy_wait_violations(none)[0][0][0] == "_Zk3"
