"""The attention kernels' scalar inline assembly must not break the compiler's own register
use: its 64-bit address arithmetic (SCC) and m0.

A 64-bit scalar add is s_add_u32 (low word, carry out in SCC) followed by s_addc_u32 (high word,
carry in from SCC).  An inline-assembly statement that writes SCC (s_max_i32, s_min_i32, ...)
without declaring it clobbered can be scheduled between the two, and the high word then takes the
statement's SCC as its carry: a load address off by 4 GiB.  This test compiles the kernels for
gfx950 and checks that the SCC read by every s_addc_u32 / s_subb_u32 was written by the matching
add / subtract.

m0 likewise: the LDS-load statement writes m0 (the LDS destination of buffer_load ... lds), which
the compiler treats as reserved and so cannot be declared clobbered.  The compiler sets m0 right
before each of its own uses; the check is that every instruction outside the assembly that reads
m0 finds it last written outside the assembly too.  Needs hipcc (compile only, no GPU)."""
import re
import shutil
import subprocess
from pathlib import Path

import pytest

CSRC = Path(__file__).resolve().parents[1] / "my-inference-engine_amd" / "csrc"
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
         "-packed-fp32-ops", "--cuda-device-only", "-S", "-o", "-"]

# scalar instructions that write SCC
_SCC_WRITERS = re.compile(
    r"\s+(s_add_u32|s_addc_u32|s_sub_u32|s_subb_u32|s_add_i32|s_sub_i32|s_(max|min)_[iu]32|"
    r"s_cmp\w*|s_(and|or|xor|andn2|orn2|nand|nor|xnor|not)_b\d+|s_(lshl|lshr)_b\d+|s_ashr_i\d+|"
    r"s_bfe_\w+|s_abs_i32|s_bcnt\w+|s_lshl\d_add_u32)\b")


def carry_hazards(asm):
    """(line, consumer, scc writer) for every carry consumer whose SCC was last written by an
    inline-assembly statement (between the compiler's ;;#ASMSTART / ;;#ASMEND markers).  The
    compiler's own SCC producers (the add of the pair, or an s_cmp it uses as a carry on purpose)
    are not reported."""
    lines = asm.split("\n")
    bad = []
    for i, line in enumerate(lines):
        m = re.match(r"\s+(s_addc_u32|s_subb_u32)\b", line)
        if not m:
            continue
        in_asm = False
        for j in range(i - 1, -1, -1):
            t = lines[j]
            if ";;#ASMEND" in t:
                in_asm = True
                continue
            if ";;#ASMSTART" in t:
                in_asm = False
                continue
            if t.startswith(".LBB") or re.match(r"\s+s_cbranch", t):
                break
            if _SCC_WRITERS.match(t):
                if in_asm:
                    bad.append((i, line.strip(), t.strip()))
                break
    return bad


_M0_WRITE = re.compile(r"\s+\w+\s+m0\s*,")
# instructions that read m0: an explicit m0 source operand, or an implicit use (LDS-destination
# loads, messages, relative moves, GWS, interpolation)
_M0_IMPLICIT = re.compile(r"\s+(s_sendmsg\w*|s_movrel\w*|v_movrel\w*|ds_gws\w*|v_interp\w*)\b"
                          r"|.*\blds\s*$")


def _reads_m0(line):
    if _M0_IMPLICIT.match(line):
        return True
    m = re.match(r"\s+\w+\s+(.*)", line)
    if not m:
        return False
    ops = [o.strip() for o in m.group(1).split(",")]
    return any(re.search(r"\bm0\b", o) for o in ops[1:])


_LABEL = re.compile(r"^([.\w$]+):")
_BRANCH = re.compile(r"\s+(s_branch|s_cbranch_\w+)\s+([.\w$]+)")
_END_OF_FLOW = re.compile(r"\s+(s_branch|s_endpgm|s_setpc_b64)\b")


def m0_hazards(asm):
    """(line, reader, writer) for every m0 read outside the inline assembly that some control-flow
    path reaches with its last m0 write inside an inline-assembly statement.  From each read the
    code is scanned backwards; at a basic-block label the scan follows every predecessor: the
    fall-through from the line above (unless that ends the flow: s_branch, s_endpgm, s_setpc) and
    every branch that targets the label (loop back edges included).  A function's own entry label
    (not a local .L label) ends a path with no write."""
    lines = asm.split("\n")
    in_asm = [False] * len(lines)
    state = False
    for i, t in enumerate(lines):
        if ";;#ASMSTART" in t:
            state = True
        elif ";;#ASMEND" in t:
            state = False
        in_asm[i] = state
    branches_to = {}
    for i, t in enumerate(lines):
        m = _BRANCH.match(t)
        if m:
            branches_to.setdefault(m.group(2), []).append(i)

    def last_writes(start):
        """Indices of the last m0 write on every path ending just above line `start`."""
        found, seen, todo = set(), set(), [start]
        while todo:
            j = todo.pop() - 1
            while j >= 0:
                t = lines[j]
                if _M0_WRITE.match(t):
                    found.add(j)
                    break
                lm = _LABEL.match(t)
                if lm:
                    label = lm.group(1)
                    if not label.startswith(".L"):
                        break  # a function's entry: no write on this path
                    if label in seen:
                        break
                    seen.add(label)
                    todo.extend(b for b in branches_to.get(label, []))
                    k = j - 1
                    while k >= 0 and (not lines[k].strip() or lines[k].lstrip().startswith(";")):
                        k -= 1
                    if k >= 0 and _END_OF_FLOW.match(lines[k]):
                        break  # no fall-through into this label
                j -= 1
        return found

    bad = []
    for i, line in enumerate(lines):
        if in_asm[i] or not _reads_m0(line):
            continue
        for j in sorted(last_writes(i)):
            if in_asm[j]:
                bad.append((i, line.strip(), lines[j].strip()))
                break
    return bad


def test_checker_flags_a_clobbered_carry():
    asm = ("\ts_add_u32 s4, s0, s2\n\t;;#ASMSTART\n\ts_max_i32 s6, s7, 0\n\t;;#ASMEND\n"
           "\ts_addc_u32 s5, s1, s3\n")
    assert carry_hazards(asm) == [(4, "s_addc_u32 s5, s1, s3", "s_max_i32 s6, s7, 0")]
    # the compiler's own patterns: the add of the pair, an s_cmp used as a carry, asm without SCC
    assert carry_hazards("\ts_add_u32 s4, s0, s2\n\t;;#ASMSTART\n\ts_mov_b32 m0, s6\n"
                         "\t;;#ASMEND\n\ts_addc_u32 s5, s1, s3\n") == []
    assert carry_hazards("\ts_cmp_lg_u64 s[12:13], 0\n\ts_addc_u32 s15, s15, s16\n") == []


@pytest.mark.skipif(not Path(HIPCC).exists(), reason="hipcc not available")
@pytest.mark.parametrize("src", ["fa2_prefill.hip", "fa2_decode.hip"])
def test_no_inline_asm_between_a_carry_and_its_use(src):
    asm = subprocess.run([HIPCC, *FLAGS, str(CSRC / src)], capture_output=True, text=True,
                         check=True, timeout=600).stdout
    assert "s_addc_u32" in asm
    assert carry_hazards(asm) == []


def test_checker_flags_m0_set_by_inline_assembly():
    asm = ("\ts_mov_b32 m0, s2\n\tbuffer_load_dword v1, v2, s[4:7], 0 offen lds\n"
           "\t;;#ASMSTART\n\ts_mov_b32 m0, s9\n\t;;#ASMEND\n"
           "\tv_readlane_b32 s3, v4, m0\n\tbuffer_load_dword v1, v2, s[4:7], 0 offen lds\n")
    assert [b[0] for b in m0_hazards(asm)] == [5, 6]
    # the compiler resets m0 before its own use: fine; m0 as a destination is not a read
    assert m0_hazards("\t;;#ASMSTART\n\ts_mov_b32 m0, s9\n\t;;#ASMEND\n\ts_mov_b32 m0, s2\n"
                      "\tbuffer_load_dword v1, v2, s[4:7], 0 offen lds\n") == []
    # a loop: the read at the loop head is preceded in text by the compiler's own write, but the
    # back edge brings it the value the inline assembly at the loop's end wrote
    loop = ("kern:\n\ts_mov_b32 m0, s2\n.LBB0_1:\n"
            "\tbuffer_load_dword v1, v2, s[4:7], 0 offen lds\n"
            "\t;;#ASMSTART\n\ts_mov_b32 m0, s9\n\t;;#ASMEND\n"
            "\ts_cbranch_scc1 .LBB0_1\n\ts_endpgm\n")
    assert [b[0] for b in m0_hazards(loop)] == [3]
    # the same loop with the compiler's write inside it, ahead of the read: fine
    assert m0_hazards(loop.replace(".LBB0_1:\n", ".LBB0_1:\n\ts_mov_b32 m0, s2\n")) == []
    # a branch target reached only by a jump from code whose last write is the compiler's: fine,
    # even though the text right above the label ends with an assembly write and an s_branch
    jump = ("kern:\n\ts_mov_b32 m0, s2\n\ts_cbranch_scc0 .LBB0_2\n"
            "\t;;#ASMSTART\n\ts_mov_b32 m0, s9\n\t;;#ASMEND\n\ts_branch .LBB0_3\n"
            ".LBB0_2:\n\tbuffer_load_dword v1, v2, s[4:7], 0 offen lds\n"
            ".LBB0_3:\n\ts_endpgm\n")
    assert m0_hazards(jump) == []
    assert [b[0] for b in m0_hazards(jump.replace("s_branch .LBB0_3", "s_nop 0"))] == [8]


@pytest.mark.skipif(not Path(HIPCC).exists(), reason="hipcc not available")
@pytest.mark.parametrize("src", ["fa2_prefill.hip", "fa2_decode.hip"])
def test_no_compiler_m0_read_sees_an_inline_assembly_write(src):
    asm = subprocess.run([HIPCC, *FLAGS, str(CSRC / src)], capture_output=True, text=True,
                         check=True, timeout=600).stdout
    assert m0_hazards(asm) == []
