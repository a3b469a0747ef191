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

Two more properties of the emitted waits, which no numeric test sees (they
only cost time):
  * the hot decode kernels issue all their weight loads up front and compute
    each block as it lands, so no wait between their first weight load and
    their first MFMA may drain the vector memory counter (vmcnt(0) there
    means every block is waited for before any is computed);
  * the MFMA GEMMs' copy rings (copies from inline asm) are never drained
    before a block's LDS reads inside the main loop.
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
        # the copies issued before the kernel's first other load (a ring's
        # later refills are waited for by counts of their own, checked by the
        # kernel's parity tests)
        others = [i for i, s in enumerate(body) if i > copies[0] and re.match(r"(global|buffer)_(load|atomic)", s)
                  and not re.search(r"\blds\b", s)]
        first_other = others[0] if others else len(body)
        last = max(i for i in copies if i < first_other)
        after, verdict = 0, None
        for s in body[last + 1:]:
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


def first_mfma_drains(asm: str) -> dict:
    """{kernel: min vmcnt between its first non-temporal (weight) load and its
    first MFMA} for every kernel that has both."""
    out = {}
    for name, body in _functions(asm).items():
        idx = [i for i, s in enumerate(body) if re.match(r"(global|buffer)_load_dwordx4 .*\bnt\b", s)]
        if not idx:
            continue
        mf = [i for i, s in enumerate(body) if s.startswith("v_mfma") and i > idx[0]]
        if not mf:
            continue
        waits = [int(m.group(1)) for s in body[idx[0]:mf[0]]
                 for m in [re.search(r"vmcnt\((\d+)\)", s)] if m]
        out[name] = (min(waits) if waits else None, sum(1 for i in idx if i < mf[0]))
    return out


def ring_drains(asm: str, pattern: str) -> dict:
    """{kernel: number of vmcnt(0) waits that follow an LDS copy and precede
    an LDS read within 40 instructions} for kernels whose name matches."""
    out = {}
    for name, body in _functions(asm).items():
        if not re.search(pattern, name):
            continue
        n, seen = 0, False
        for i, s in enumerate(body):
            if re.match(r"buffer_load\S* .*\blds\b", s):
                seen = True
            if seen and s.startswith("s_waitcnt") and "vmcnt(0)" in s:
                if any(t.startswith("ds_read") for t in body[i + 1:i + 40]):
                    n += 1
        out[name] = n
    return out


@pytest.fixture(scope="module")
def asms(tmp_path_factory):
    if not os.path.exists("/opt/rocm/bin/hipcc"):
        pytest.skip("hipcc not installed")
    hipcc, cflags = _flags()
    if not shutil.which(hipcc) and not os.path.exists(hipcc):
        pytest.skip("hipcc not found")
    tmp = tmp_path_factory.mktemp("asm")

    def compile_one(src):
        out = os.path.join(tmp, src.replace(".hip", ".s"))
        cmd = [hipcc, *[f for f in cflags if f != "-fPIC"], "--cuda-device-only", "-S",
               os.path.join(PKG, "csrc", src), "-o", out]
        r = subprocess.run(cmd, capture_output=True, text=True)
        assert r.returncode == 0, r.stderr[-2000:]
        return open(out).read()

    with ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        return dict(zip(SOURCES, ex.map(compile_one, SOURCES)))


def test_lds_copy_waits_cover_the_copies(asms):
    total, problems = 0, []
    for src, asm in asms.items():
        bad, checked = copy_wait_violations(asm)
        total += checked
        problems += [(src, n, v) for n, v in bad]
    assert total >= 40, total  # the decode GEMV / MoE instantiations were found
    assert not problems, problems


# the launch shapes the library picks for the benchmark's decode shapes
# (mangled-name fragments): Marlin GEMV at M <= 4 and above, row-major
# whole-line GEMV, FP8 GEMVs, decode MoE
HOT_DECODE = [
    ("int4_marlin.hip", "int4_gemv_nbILi2ELi4ELb0ELi0ELb0E"),
    ("int4_marlin.hip", "int4_gemv_nbILi1ELi4ELb0ELi0ELb0E"),
    ("int4_marlin.hip", "int4_gemv_nbILi1ELi6ELb0ELi0ELb0E"),
    ("int4_marlin.hip", "int4_gemv_nbILi2ELi2ELb0ELi3ELb0E"),
    ("int4_marlin.hip", "int4_gemv_nbILi1ELi4ELb0ELi3ELb0E"),
    ("int4_marlin.hip", "int4_gemv_nbILi2ELi4ELb0ELi3ELb0E"),
    ("int4_marlin.hip", "int4_gemv_nbILi2ELi3ELb0ELi3ELb0E"),
    ("int4_marlin.hip", "int4_gemv_normILi2ELi4ELb0ELb1E"),
    ("moe_int4.hip", "rm_gemv_lineILi2ELi2ELi0ELb0E"),
    ("moe_int4.hip", "rm_gemv_lineILi1ELi3ELi0ELb0E"),
    ("moe_int4.hip", "moe_gate_up_kILi0ELb1ELi2ELi4E"),
    ("moe_int4.hip", "moe_gate_up_kILi1ELb1ELi2ELi2E"),
    ("moe_int4.hip", "moe_down_kILi0ELb1ELi2ELi2E"),
    ("fp8.hip", "fp8_gemv_q2ILi3ELb0ELb1ELb1E"),
    ("fp8.hip", "fp8_gemv_q2ILi3ELb0ELb1ELb0E"),
    ("fp8.hip", "fp8_gemv_q4ILi3ELb0ELb1E"),
    ("fp8.hip", "fp8_gemv_nbILi1ELi4ELb0ELb1ELi3E"),
]


def test_hot_decode_kernels_compute_blocks_as_they_land(asms):
    found, drained = 0, []
    for src, frag in HOT_DECODE:
        hits = {n: v for n, v in first_mfma_drains(asms[src]).items() if frag in n}
        assert hits, (src, frag)
        found += 1
        for n, (mn, nl) in hits.items():
            if mn == 0 and nl > 2:
                drained.append((n, nl))
    assert found == len(HOT_DECODE)
    assert not drained, drained


def test_gemm_rings_are_not_drained(asms):
    # the FP8 GEMM's three-ahead instance keeps three blocks in flight; its
    # split-K epilogue drains once or twice after the ring, nothing in the
    # ring may.  (The one-ahead instance's own wait is vmcnt(0) by design:
    # only the block about to be read is in flight there.)
    res = ring_drains(asms["fp8.hip"], r"fp8_gemm_mfmaILb1ELi3E")
    assert res
    for name, n in res.items():
        assert n <= 2, (name, n)
    for src, pat in (("int4_marlin.hip", "int4_gemm_mfma"), ("moe_int4.hip", "moe_gemm_k")):
        res = ring_drains(asms[src], pat)
        assert res, pat
        for name, n in res.items():
            assert n == 0, (name, n)


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
