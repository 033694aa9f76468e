"""A vector-memory store of more than 8 bytes (buffer_/global_/flat_/scratch_store_dwordx3,
_dwordx4) reads its data VGPRs after it issues, so a VALU instruction that
overwrites those VGPRs must not follow it directly: the hardware needs one wait
state between them.  The compiler does not always keep that gap.  A build of the
48-wide kept-scores forward with 64-key sub-tiles placed `v_sub_f32 v103, ...`
right after `buffer_store_dwordx4 v[100:103]` (and `v_or_b32 v100, ...` after the
last store).  The stored scores then came out wrong in exactly those elements,
only in blocks that shared a CU with another block.  Every kernel of the library
is compiled to device assembly here and scanned for a store whose next
instruction writes one of its data VGPRs.

The compiler inserts the wait states an MFMA result needs before a VALU
instruction reads it (about a dozen for v_mfma_f32_16x16x4_f32), and before an
instruction overwrites a register an MFMA still reads, only for instructions it
generates itself: inline assembly is invisible to that bookkeeping.  An
inline-asm v_max3_f32 over a score chain's accumulators once came directly
after the chain's last MFMA and read stale values (the running maximum of
whole waves came out wrong).  The kernels therefore contain no inline
assembly; the second check keeps it that way.  No GPU needed."""
import re
import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "wave-engine_amd"

STORE = re.compile(r"^\s*(buffer|global|flat|scratch)_store_(dwordx3|dwordx4|b96|b128)\s+(.*)$")
SKIP = re.compile(r"^\s*($|;|\.|\S+:)")


def vgprs(spec):
    spec = spec.strip()
    m = re.match(r"v\[(\d+):(\d+)\]", spec)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)\b", spec)
    return {int(m.group(1))} if m else set()


def written_vgprs(line):
    """VGPRs a VALU instruction writes (its first operand); none for other instructions."""
    parts = line.strip().split(None, 1)
    if len(parts) < 2 or not parts[0].startswith("v_") or parts[0].startswith(("v_cmp", "v_readfirstlane", "v_readlane")):
        return set()
    return vgprs(parts[1].split(",")[0])


def scan(text):
    """(line number, store, next instruction) for every store followed directly by a write of its data."""
    lines = text.splitlines()
    found = []
    for i, line in enumerate(lines):
        m = STORE.match(line)
        if not m:
            continue
        ops = m.group(3).split(",")
        # buffer stores name their data first; global/flat/scratch stores name the address first
        data = vgprs(ops[0]) if m.group(1) == "buffer" else vgprs(ops[1]) if len(ops) > 1 else set()
        j = i + 1
        while j < len(lines) and SKIP.match(lines[j]):
            j += 1
        if j < len(lines) and data & written_vgprs(lines[j]):
            found.append((i + 1, line.strip(), lines[j].strip()))
    return found


def test_scanner_finds_the_pattern():
    """The scanner itself, on the sequence that corrupted the kept scores and on safe variants."""
    bad = "\tbuffer_store_dwordx4 v[100:103], v86, s[52:55], s16 offen\n\tv_sub_f32_e32 v103, v27, v15\n"
    assert len(scan(bad)) == 1
    bad_global = "\tglobal_store_dwordx4 v[4:5], v[10:13], off\n\tv_mov_b32_e32 v10, 0\n"
    assert len(scan(bad_global)) == 1
    gap = "\tbuffer_store_dwordx4 v[100:103], v86, s[52:55], s16 offen\n\ts_nop 0\n\tv_sub_f32_e32 v103, v27, v15\n"
    other = "\tbuffer_store_dwordx4 v[100:103], v86, s[52:55], s16 offen\n\tv_sub_f32_e32 v104, v27, v15\n"
    spill = "\tscratch_store_dwordx4 off, v[20:23], s33 offset:16\n\tv_mov_b32_e32 v21, 0\n"
    assert len(scan(spill)) == 1
    small = "\tbuffer_store_dwordx2 v[100:101], v86, s[52:55], s16 offen\n\tv_sub_f32_e32 v101, v27, v15\n"
    assert scan(gap) == [] and scan(other) == [] and scan(small) == []


def test_no_store_data_overwritten_by_the_next_instruction():
    subprocess.run(["make", "-s", "-C", str(PKG), "-j8", "isa"], check=True, timeout=900)
    files = sorted((PKG / "_build" / "isa").glob("*.s"))
    assert len(files) >= 10
    hits = [(f.name, *h) for f in files for h in scan(f.read_text())]
    assert hits == [], "\n".join(f"{f}:{n}: {s} / {nx}" for f, n, s, nx in hits)


def asm_instructions(text):
    """(line number, instruction) of every instruction inside an inline-asm
    block; empty blocks (compiler barriers, asm volatile("" ::: "memory"))
    emit nothing and are not reported."""
    found, inside = [], False
    for n, line in enumerate(text.splitlines()):
        if ";;#ASMSTART" in line:
            inside = True
        elif ";;#ASMEND" in line:
            inside = False
        elif inside and not SKIP.match(line):
            found.append((n + 1, line.strip()))
    return found


def test_asm_scanner():
    barrier = "\t;;#ASMSTART\n\t;;#ASMEND\n\tv_add_f32_e32 v1, v2, v3\n"
    asm_max = "\tv_mfma_f32_16x16x4_f32 v[48:51], v51, v121, v[44:47]\n\t;;#ASMSTART\n\tv_max_f32 v4, v48, v49\n\t;;#ASMEND\n"
    assert asm_instructions(barrier) == []
    assert asm_instructions(asm_max) == [(3, "v_max_f32 v4, v48, v49")]


def test_no_inline_assembly_in_kernels():
    """Inline asm bypasses the compiler's MFMA hazard handling (module docstring)."""
    subprocess.run(["make", "-s", "-C", str(PKG), "-j8", "isa"], check=True, timeout=900)
    files = sorted((PKG / "_build" / "isa").glob("*.s"))
    assert len(files) >= 10
    hits = [(f.name, *h) for f in files for h in asm_instructions(f.read_text())]
    assert hits == [], f"inline assembly in device code: {hits[:10]}"
