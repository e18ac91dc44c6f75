"""Assembly checks of the MFMA kernels (CPU: hipcc cross-compiles gfx950; no GPU needed).

The compiler inserts the wait states between a VALU write and an MFMA read of the written VGPR
only for instructions it can see. A value built by inline-asm VALU code (the library's v_bfi_b32
helpers) and read by an MFMA a few instructions later gets none, and the MFMA can read stale
bytes (this happened in the Q6_K batch kernel). Every kernel source that uses MFMAs is compiled to
assembly with the library's flags, and no MFMA may read an inline-asm VALU result within 24 issue
slots of the write.
"""
import os
import re
import shutil
import subprocess
import tempfile
from concurrent.futures import ThreadPoolExecutor

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "..", "densecore_amd", "csrc")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-mllvm", "-amdgpu-kernarg-preload-count=16", "--cuda-device-only", "-S"]
WINDOW = 24


def _regs(tok):
    m = re.match(r"v\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", tok)
    return {int(m.group(1))} if m else set()


def asm_valu_to_mfma(asm_text, window=WINDOW):
    """(kernel, slots) for every inline-asm VALU write read by an MFMA within `window` issue slots
    (s_nop n counts n + 1), unless a compiler-visible VALU instruction rewrites the register first."""
    insts, cur, inasm = [], None, False
    for ln in asm_text.splitlines():
        s = ln.strip()
        m = re.match(r"^(_Z\w+):", s)
        if m:
            cur = m.group(1)
            continue
        if s.startswith(";;#ASMSTART"):
            inasm = True
            continue
        if s.startswith(";;#ASMEND"):
            inasm = False
            continue
        if not s or s.startswith(";") or s.startswith(".") or s.endswith(":"):
            continue
        insts.append((cur, s, inasm))
    hits = []
    for i, (k, s, in_asm) in enumerate(insts):
        if not in_asm or not s.startswith("v_") or len(s.split(None, 1)) < 2:
            continue
        dst = _regs(s.split(None, 1)[1].split(",")[0].strip())
        slots = 0
        for k2, s2, _ in insts[i + 1:i + 80]:
            if k2 != k:
                break
            op = s2.split()[0]
            slots += int(s2.split()[1]) + 1 if op == "s_nop" else 1
            if slots > window:
                break
            parts = s2.split(None, 1)
            if op.startswith("v_mfma") and len(parts) > 1:
                ops = [o.strip() for o in parts[1].split(",")]
                if dst & set().union(*[_regs(o) for o in ops[1:]]):
                    hits.append((k, slots))
                    break
            if op.startswith("v_") and len(parts) > 1 and _regs(parts[1].split(",")[0].strip()) & dst:
                break
    return hits


def test_scan_flags_the_known_pattern():
    """The checker itself: a v_bfi_b32 from inline asm read as an MFMA operand three slots later."""
    text = """_ZN3dcq1kEv:
	;;#ASMSTART
	v_bfi_b32 v101, v143, v31, v1
	;;#ASMEND
	v_perm_b32 v102, 0, v144, v2
	s_waitcnt lgkmcnt(8)
	v_mfma_i32_32x32x16_i8 v[0:15], v[92:93], v[100:101], 0
"""
    assert asm_valu_to_mfma(text) == [("_ZN3dcq1kEv", 3)]
    # a compiler-visible rewrite in between clears it; so does distance beyond the window
    assert asm_valu_to_mfma(text.replace("v_perm_b32 v102", "v_mov_b32 v101")) == []
    assert asm_valu_to_mfma(text.replace("s_waitcnt lgkmcnt(8)", "s_nop 7\n\ts_nop 7\n\ts_nop 7")) == []


@pytest.mark.skipif(not shutil.which(HIPCC) and not os.path.exists(HIPCC), reason="hipcc not available")
def test_no_inline_asm_valu_result_feeds_an_mfma():
    srcs = sorted(f for f in os.listdir(CSRC) if f.endswith(".hip")
                  and "mfma" in open(os.path.join(CSRC, f)).read())
    assert srcs, "no MFMA kernel sources found"
    with tempfile.TemporaryDirectory() as tmp:
        def compile_one(f):
            out = os.path.join(tmp, f + ".s")
            r = subprocess.run([HIPCC] + FLAGS + [os.path.join(CSRC, f), "-o", out], capture_output=True, text=True,
                               cwd=CSRC)
            assert r.returncode == 0, f"{f}: {r.stderr[-2000:]}"
            return f, open(out).read()
        with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
            results = list(ex.map(compile_one, srcs))
    bad = [(f, k, n) for f, text in results for k, n in asm_valu_to_mfma(text)]
    assert not bad, f"inline-asm VALU results read by an MFMA without wait states: {bad[:5]}"
