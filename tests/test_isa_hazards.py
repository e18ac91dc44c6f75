"""Assembly checks of the hand-scheduled kernels (CPU: hipcc cross-compiles gfx950; no GPU needed).

Every kernel source that uses MFMAs or direct-to-LDS loads is compiled to gfx950 assembly with the
library's flags, once per session, and scanned for four hazards the compiler cannot see:

1. Inline-asm VALU results read by an MFMA. The compiler inserts the wait states between a VALU
   write and an MFMA read of the written VGPR only for instructions it can see. A value built by
   inline-asm VALU code (the library's v_bfi_b32 helpers) and read by an MFMA a few instructions
   later gets none, and the MFMA can read stale bytes (this happened in the Q6_K batch kernel). No
   MFMA may read an inline-asm VALU result within 24 issue slots of the write.
2. Untracked register loads. An inline-asm global load into VGPRs (the fused Q6_K decode's
   activation loads) is taken by the compiler as complete when the asm issues. If the register
   allocator copies, spills or reuses its destination registers before the kernel's explicit wait,
   the load lands on live values (a variant of the Q4_K batch kernel faulted the GPU this way). On
   every control-flow path from such a load, no instruction may read or write its destination
   registers before an s_waitcnt vmcnt(0) or the end of the kernel's counted wait (the
   ";dcq counted wait" marker after its binary search over s_waitcnt immediates).
3. Direct-to-LDS loads before a barrier. Data a workgroup publishes with s_barrier must have
   landed: on every path from a global_load_lds, an s_waitcnt vmcnt(0) or a counted wait must come
   before the next s_barrier. Loads into a wave's own row image ("; wave-private" in their asm),
   read only by that wave after its own counted wait, may stay in flight across a barrier.
4. MFMA operand overlap. The compiler gives some MFMAs a result range overlapping their A or B
   operand (the operand's last use). The scan checks the forms in which it does so: the
   accumulator input C is then the inline constant 0, and a register C is either the result range
   itself or disjoint from it (never a partial overlap).
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
MARK = "dcq counted wait"
PRIVATE = "wave-private"


def _regs(tok):
    m = re.match(r"v\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", tok)
    return {int(m.group(1))} if m else set()


def _refs(inst):
    """Every VGPR an instruction names (operands, not the mnemonic; comments stripped)."""
    parts = inst.split(";")[0].split(None, 1)
    out = set()
    if len(parts) > 1:
        for tok in re.findall(r"v\[\d+:\d+\]|\bv\d+\b", parts[1]):
            out |= _regs(tok)
    return out


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


# ---------------------------------------------------------------- control-flow scan (hazards 2, 3)
def functions(asm_text):
    """{kernel: (instructions [(text, from inline asm)], labels {label: instruction index})}.
    The counted-wait marker and sched_barrier comments are kept as pseudo-instructions."""
    funcs, cur, inasm = {}, None, False
    for ln in asm_text.splitlines():
        s = ln.strip()
        m = re.match(r"^(_Z\w+):", s)
        if m:
            cur = m.group(1)
            funcs[cur] = ([], {})
            continue
        if cur is None:
            continue
        if s.startswith(";;#ASMSTART"):
            inasm = True
            continue
        if s.startswith(";;#ASMEND"):
            inasm = False
            continue
        m = re.match(r"^(\.LBB\w+):", s)
        if m:
            funcs[cur][1][m.group(1)] = len(funcs[cur][0])
            continue
        if MARK in s:
            funcs[cur][0].append((MARK, True))
            continue
        if not s or s.startswith(";") or s.startswith(".") or s.endswith(":"):
            continue
        funcs[cur][0].append((s, inasm))
        if s.startswith("s_endpgm"):
            cur = None
    return funcs


def _succ(insts, labels, i):
    s = insts[i][0]
    op = s.split()[0]
    if op == "s_endpgm":
        return []
    if op == "s_branch":
        return [labels[s.split()[1]]]
    if op.startswith("s_cbranch"):
        return [i + 1, labels[s.split()[1]]]
    return [i + 1] if i + 1 < len(insts) else []


def _covering_wait(s):
    return s == MARK or re.match(r"s_waitcnt\b.*vmcnt\(0\)", s) is not None or s == "s_waitcnt 0"


def _first_on_a_path(insts, labels, i, hit):
    """The first instruction, on some control-flow path from instruction i, for which hit() holds
    before a covering wait; None if every path reaches a covering wait (or the end) first."""
    seen, stack = set(), _succ(insts, labels, i)
    while stack:
        j = stack.pop()
        if j in seen:
            continue
        seen.add(j)
        s = insts[j][0]
        if _covering_wait(s):
            continue
        if hit(s):
            return s
        stack.extend(_succ(insts, labels, j))
    return None


def load_hazards(asm_text):
    """(untracked register loads, direct-to-LDS loads, hits) over every kernel in the assembly."""
    n_reg = n_dma = 0
    hits = []
    for f, (insts, labels) in functions(asm_text).items():
        for i, (s, in_asm) in enumerate(insts):
            if in_asm and re.match(r"global_load_(dword|ubyte|sbyte|ushort|short)", s) and "_lds" not in s:
                n_reg += 1
                dst = _regs(s.split(None, 1)[1].split(",")[0].strip())
                r = _first_on_a_path(insts, labels, i, lambda t: bool(_refs(t) & dst))
                if r:
                    hits.append(("register load touched before its wait", f, s, r))
            if re.match(r"(global|buffer)_load_lds_", s):
                n_dma += 1
                if PRIVATE in s:
                    continue
                r = _first_on_a_path(insts, labels, i, lambda t: t.startswith("s_barrier"))
                if r:
                    hits.append(("barrier before the direct-to-LDS load's wait", f, s, r))
    return n_reg, n_dma, hits


def mfma_overlaps(asm_text):
    """(MFMAs, overlaps of the result with A or B, violations): a violation is an overlap of the
    result with A or B while C is not the inline constant 0, or a register C that partly overlaps
    the result."""
    n = n_ab = 0
    bad = []
    for ln in asm_text.splitlines():
        s = ln.strip()
        if not s.startswith("v_mfma"):
            continue
        n += 1
        ops = [o.strip() for o in s.split(";")[0].split(None, 1)[1].split(",")]
        d = _regs(ops[0].replace("a[", "v[") if ops[0].startswith("a") else ops[0])
        dkind = ops[0][0]
        a, b, c = ops[1], ops[2], ops[3]
        if any(o[0] == dkind and _regs(o.replace("a", "v", 1)) & d for o in (a, b)):
            n_ab += 1
            if c != "0":
                bad.append(s)
        if c[0] in "va":
            rc = _regs(c.replace("a", "v", 1))
            if c[0] == dkind and rc & d and rc != d:
                bad.append(s)
    return n, n_ab, bad


# ---------------------------------------------------------------- the checkers on known patterns
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


_REG_LOAD = """_ZN3dcq1kEv:
	;;#ASMSTART
	global_load_dwordx4 v[2:5], v[14:15], off
	;;#ASMEND
	s_cmp_lt_i32 s4, 3
	s_cbranch_scc1 .LBB0_2
	v_mov_b32_e32 v9, 0
.LBB0_2:
	s_waitcnt vmcnt(1)
	;;#ASMSTART
	;dcq counted wait
	;;#ASMEND
	v_max3_f32 v18, v2, 0, v3
	s_endpgm
"""


def test_register_load_scan_on_known_patterns():
    """Planted mistakes: a copy of a pending register, a reuse on one branch only, a path that skips
    the wait; the clean form and a full wait pass."""
    assert load_hazards(_REG_LOAD) == (1, 0, [])
    copy = _REG_LOAD.replace("v_mov_b32_e32 v9, 0", "v_mov_b32_e32 v9, v3")
    assert [h[3] for h in load_hazards(copy)[2]] == ["v_mov_b32_e32 v9, v3"]
    reuse = _REG_LOAD.replace("v_mov_b32_e32 v9, 0", "v_mbcnt_lo_u32_b32 v2, -1, 0")
    assert len(load_hazards(reuse)[2]) == 1
    skip = _REG_LOAD.replace("\ts_cbranch_scc1 .LBB0_2\n", "\ts_cbranch_scc1 .LBB0_3\n").replace(
        "\tv_max3_f32", ".LBB0_3:\n\tv_max3_f32")
    assert [h[3] for h in load_hazards(skip)[2]] == ["v_max3_f32 v18, v2, 0, v3"]
    full = _REG_LOAD.replace("s_waitcnt vmcnt(1)", "s_waitcnt vmcnt(0)").replace(";dcq counted wait", "")
    assert load_hazards(full)[2] == []
    no_wait = _REG_LOAD.replace(";dcq counted wait", "")
    assert len(load_hazards(no_wait)[2]) == 1  # a partial vmcnt wait alone does not count


_DMA = """_ZN3dcq1kEv:
	s_mov_b32 m0, s43
	;;#ASMSTART
	global_load_lds_dwordx4 v[18:19], off
	;;#ASMEND
	v_add_u32_e32 v1, 64, v1
	s_waitcnt vmcnt(0) expcnt(0) lgkmcnt(0)
	s_barrier
	s_endpgm
"""


def test_lds_load_scan_on_known_patterns():
    """Planted mistakes: a barrier with no wait, or only a partial one; a wave-private load is exempt."""
    assert load_hazards(_DMA) == (0, 1, [])
    assert len(load_hazards(_DMA.replace("\ts_waitcnt vmcnt(0) expcnt(0) lgkmcnt(0)\n", ""))[2]) == 1
    assert len(load_hazards(_DMA.replace("vmcnt(0) expcnt(0)", "vmcnt(3) expcnt(0)"))[2]) == 1
    private = _DMA.replace("off\n", "off ; wave-private\n").replace("\ts_waitcnt vmcnt(0) expcnt(0) lgkmcnt(0)\n", "")
    assert load_hazards(private) == (0, 1, [])


def test_mfma_overlap_scan_on_known_patterns():
    ok = "\tv_mfma_i32_32x32x32_i8 v[0:15], v[32:35], v[0:3], 0\n\tv_mfma_i32_32x32x32_i8 v[0:15], v[32:35], v[36:39], v[0:15]\n"
    assert mfma_overlaps(ok) == (2, 1, [])
    assert len(mfma_overlaps("\tv_mfma_i32_32x32x32_i8 v[0:15], v[32:35], v[0:3], v[0:15]\n")[2]) == 1
    assert len(mfma_overlaps("\tv_mfma_i32_32x32x32_i8 v[0:15], v[32:35], v[36:39], v[8:23]\n")[2]) == 1


# ---------------------------------------------------------------- the library's kernels
@pytest.fixture(scope="module")
def kernel_asm():
    if not shutil.which(HIPCC) and not os.path.exists(HIPCC):
        pytest.skip("hipcc not available")
    srcs = sorted(f for f in os.listdir(CSRC) if f.endswith(".hip")
                  and re.search(r"mfma|load_lds", open(os.path.join(CSRC, f)).read()))
    assert srcs, "no MFMA or direct-to-LDS kernel sources found"
    with tempfile.TemporaryDirectory() as tmp:
        def compile_one(f):
            out = os.path.join(tmp, f + ".s")
            r = subprocess.run([HIPCC] + FLAGS + [os.path.join(CSRC, f), "-o", out], capture_output=True, text=True,
                               cwd=CSRC)
            assert r.returncode == 0, f"{f}: {r.stderr[-2000:]}"
            return f, open(out).read()
        with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
            return dict(ex.map(compile_one, srcs))


def test_no_inline_asm_valu_result_feeds_an_mfma(kernel_asm):
    bad = [(f, k, n) for f, text in kernel_asm.items() for k, n in asm_valu_to_mfma(text)]
    assert not bad, f"inline-asm VALU results read by an MFMA without wait states: {bad[:5]}"


def test_untracked_loads_and_lds_loads_are_waited_for(kernel_asm):
    totals = {f: load_hazards(text) for f, text in kernel_asm.items()}
    bad = [(f,) + h for f, (_, _, hits) in totals.items() for h in hits]
    assert not bad, f"{len(bad)} load hazards, e.g. {bad[:3]}"
    # the scan saw what it is for: the fused Q6_K decode's activation loads, and direct-to-LDS
    # loads in every staged kernel
    assert totals["dcq_decode_q6.hip"][0] > 0
    for f in ("dcq_prefill.hip", "dcq_prefill_kq.hip", "dcq_batch.hip", "dcq_batch_q8.hip", "dcq_batch_q6.hip",
              "dcq_decode_q6.hip"):
        assert totals[f][1] > 0, f


def test_mfma_operand_overlaps_are_of_the_checked_forms(kernel_asm):
    res = {f: mfma_overlaps(text) for f, text in kernel_asm.items()}
    bad = [(f, s) for f, (_, _, b) in res.items() for s in b]
    assert not bad, f"MFMA operand overlaps outside the checked forms: {bad[:3]}"
    assert sum(n for n, _, _ in res.values()) > 0
