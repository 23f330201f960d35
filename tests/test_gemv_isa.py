"""The GEMV prologue's untracked loads, checked in the gfx950 assembly.

gemv.hip issues the activation, norm, residual-update and partial-sum loads
(and a residual-add producer's norm weights) as inline-asm global loads, so
that the compiler does not wait for them with
vmcnt(0) (which would also wait for the weight copies issued after them);
the kernel waits with its own s_waitcnt.  That is only correct if no other
instruction reads or writes a destination register of those loads before
the wait: the compiler does not know the loads are in flight.  The wait
also counts on the loads being older than every weight copy
(global_load_lds) issued before it, so a load the compiler moved after a
copy would make the wait too weak.  This test compiles gemv.hip to assembly
and checks both for every gemv_kernel and gemv_wide_kernel instantiation.
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = os.environ.get("HIPCC") or ("/opt/rocm/bin/hipcc" if os.path.exists("/opt/rocm/bin/hipcc") else
                                    shutil.which("hipcc"))


def vregs(tok):
    m = re.match(r"v\[(\d+):(\d+)\]$", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", tok)
    return {int(m.group(1))} if m else set()


def check_kernel(body):
    """Problems in one kernel's text: a pending load's register used before
    the first inline-asm s_waitcnt vmcnt, a pending load issued after a weight
    copy, or no such loads / wait at all."""
    pending = set()
    in_asm = False
    waited = False
    copied = False
    problems = []
    for line in body.split("\n"):
        s = line.strip()
        if s.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if s.startswith(";;#ASMEND"):
            in_asm = False
            continue
        if not s or s.startswith(";") or s.endswith(":"):
            continue
        if in_asm and s.startswith("s_waitcnt vmcnt"):
            waited = True
            break
        toks = re.findall(r"v\[\d+:\d+\]|v\d+\b", s)
        if not in_asm and s.startswith("global_load_lds"):
            copied = True
        if in_asm and s.startswith("global_load_dword"):
            if copied:
                problems.append("prologue load after a weight copy: " + s)
            if vregs(toks[1]) & pending:
                problems.append("address register of a pending load: " + s)
            pending |= vregs(toks[0])
            continue
        if any(vregs(t) & pending for t in toks):
            problems.append("pending register touched: " + s)
    if not pending:
        problems.append("no prologue loads found")
    if not waited:
        problems.append("no prologue wait found")
    return problems


@pytest.mark.skipif(not HIPCC, reason="hipcc not found")
def test_gemv_prologue_loads_untouched_until_waited(tmp_path):
    out = tmp_path / "gemv.s"
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off", "-Xclang",
           "-target-feature", "-Xclang", "-packed-fp32-ops", f"-I{os.path.join(ROOT, 'include')}",
           "--cuda-device-only", "-S", "-x", "hip", os.path.join(ROOT, "llama3pure_amd", "csrc", "gemv.hip"),
           "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    src = out.read_text()
    kernels = re.findall(r"^(_ZN\S*gemv_(?:wide_)?kernel\S+):[^\n]*\n(.*?)s_endpgm", src, re.S | re.M)
    assert len(kernels) >= 100, len(kernels)
    bad = {name: p for name, body in kernels if (p := check_kernel(body))}
    assert not bad, {k: v[:3] for k, v in list(bad.items())[:5]}


def test_checker_flags_early_use():
    """The checker itself: a read of a pending register before the wait, an
    address register overwritten by an earlier pending load, a prologue load
    after a weight copy and a missing wait are reported; a clean sequence is
    not."""
    load = ";;#ASMSTART\n\tglobal_load_dwordx4 v[10:13], v[2:3], off offset:0\n;;#ASMEND\n"
    wait = ";;#ASMSTART\n\ts_waitcnt vmcnt(6)\n;;#ASMEND\n"
    clean = load + "\tv_add_u32 v20, v21, v22\n\tglobal_load_lds_dwordx4 v[30:31], off nt\n" + wait + "\tv_mov_b32 v1, v11\n"
    assert check_kernel(clean) == []
    early = load + "\tv_mov_b32 v1, v12\n" + wait
    assert any("pending register" in p for p in check_kernel(early))
    clobbered = load + ";;#ASMSTART\n\tglobal_load_dwordx4 v[14:17], v[10:11], off offset:16\n;;#ASMEND\n" + wait
    assert any("address register" in p for p in check_kernel(clobbered))
    assert "no prologue wait found" in check_kernel(load + "\tv_mov_b32 v1, v2\n")
    late = load + "\tglobal_load_lds_dwordx4 v[30:31], off nt\n" + load.replace("v[10:13]", "v[40:43]") + wait
    assert any("after a weight copy" in p for p in check_kernel(late))
