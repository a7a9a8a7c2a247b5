"""Static check of the gfx950 device assembly (CPU, hipcc only): a register written by an
inline-asm LDS read (lds_read16 / gv_read) is neither read nor overwritten by any other
instruction before an `s_waitcnt lgkmcnt(N)` that covers the read.

The compiler does not know that the value of such an asm statement arrives later: a copy
it makes before the wait (for instance of a fragment assigned to a second variable) holds
the registers' old contents, and the MFMAs that use the copy get wrong data with no error.
LDS operations return in order, so `lgkmcnt(N)` leaves at most the N most recent of them
outstanding (scalar loads share the counter but only make the wait stricter). The scan is
linear over each kernel; reads issued by the compiler itself are counted for the wait
positions but not checked (the compiler places their waits)."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "prune_path_openpangu-embedded-1b_amd", "csrc")
BUILD = os.path.join(ROOT, "prune_path_openpangu-embedded-1b_amd", "_build")
SOURCES = ("route", "decode", "prefill", "dense", "masked")


def _regs(tok):
    m = re.match(r"([va])\[(\d+):(\d+)\]", tok)
    if m:
        return {f"{m.group(1)}{i}" for i in range(int(m.group(2)), int(m.group(3)) + 1)}
    return {tok} if re.match(r"[va]\d+$", tok) else set()


def _operands(rest):
    return [o.strip().split()[0] for o in rest.split(",") if o.strip()]


def scan(lines):
    """(kernel, line number, instruction, registers) of every violation in an .s text."""
    bad, pend, kernel, in_asm = [], [], None, False
    for ln, raw in enumerate(lines, 1):
        t = raw.strip()
        if t.startswith("_Z") and t.endswith(":") or re.match(r"^_Z\S*:", t):
            kernel, pend = t.split(":")[0], []
            continue
        if t.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if t.startswith(";;#ASMEND"):
            in_asm = False
            continue
        if not t or t[0] in ";." or t.endswith(":"):
            continue
        if t.startswith("s_endpgm"):
            pend = []
            continue
        op, _, rest = t.partition(" ")
        if op == "s_waitcnt":
            m = re.search(r"lgkmcnt\((\d+)\)", rest)
            if m:
                n = int(m.group(1))
                pend = pend[len(pend) - n:] if 0 < n < len(pend) else ([] if n == 0 else pend)
            continue
        ops = _operands(rest)
        used = set().union(*(_regs(o) for o in ops)) if ops else set()
        live = set().union(*pend) if pend else set()
        if used & live:
            bad.append((kernel, ln, t, sorted(used & live)))
        if op.startswith("ds_read") or op.startswith("ds_load"):
            pend.append(_regs(ops[0]) if in_asm else set())
        elif op.startswith("ds_"):
            pend.append(set())
    return bad


def test_scan_finds_a_copy_before_the_wait():
    # a fragment copied (v_mov) before its wait, as the compiler emitted for a second
    # variable holding the same fragment
    s = """_Zkernel:
;;#ASMSTART
ds_read_b128 v[36:39], v35
;;#ASMEND
ds_read_b32 v2, v3
v_mov_b64_e32 v[64:65], v[36:37]
;;#ASMSTART
s_waitcnt lgkmcnt(0)
;;#ASMEND
v_mfma_f32_16x16x4_f32 v[10:13], v64, v40, v[10:13]
s_endpgm
"""
    bad = scan(s.splitlines())
    assert [b[1] for b in bad] == [6] and bad[0][3] == ["v36", "v37"]


def test_scan_accepts_partial_waits_in_order():
    # lgkmcnt(1) after two reads covers the first one only
    s = """_Zkernel:
;;#ASMSTART
ds_read_b128 v[0:3], v20
;;#ASMEND
;;#ASMSTART
ds_read_b128 v[4:7], v21
;;#ASMEND
s_waitcnt lgkmcnt(1)
v_mfma_f32_32x32x16_bf16 v[32:47], v[0:3], v[8:11], v[32:47]
v_mov_b32_e32 v30, v4
s_endpgm
"""
    bad = scan(s.splitlines())
    assert [b[1] for b in bad] == [10]


@pytest.mark.skipif(shutil.which("hipcc") is None and not os.path.exists("/opt/rocm/bin/hipcc"),
                    reason="hipcc is not installed")
def test_no_asm_lds_read_is_used_before_its_wait():
    targets = [os.path.join(BUILD, f"{s}.s") for s in SOURCES]
    r = subprocess.run(["make", "-s", "-C", CSRC, "-j8"] + [os.path.relpath(t, CSRC) for t in targets],
                       capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    bad = []
    for t in targets:
        with open(t) as f:
            bad += [(os.path.basename(t),) + b for b in scan(f.read().splitlines())]
    assert not bad, "\n".join(f"{b[0]}:{b[2]} {b[1]}: {b[3]} uses {b[4]} before its wait" for b in bad[:20])
