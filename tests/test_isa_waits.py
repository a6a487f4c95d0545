"""The Q8_0 product kernels' untracked loads against their waits, on this build's own AMD
assembly (ex-nihilo_amd/_build/gemm.o's gfx950 code object, disassembled with ROCm's
llvm-objdump; no GPU needed).

k_gemm_q8_tall and k_gemm_bt<..., true> load the codes and scales with inline-assembly buffer
loads the compiler does not see as loads: it inserts no wait for them, and only the kernels'
own vmcnt waits (counted from the operations' positions) cover them.  That holds only while the
register allocator neither reads nor copies a load's destination before the covering wait.
This checks it on the machine code: in every main loop of those kernels (and of k_gemm_few,
whose loads the compiler tracks), walking the loop body cyclically from each vector-memory load
into registers, no instruction touches the load's destination registers before an s_waitcnt
whose vmcnt leaves out no more operations than were issued after the load."""
import os
import re
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
OBJ = os.path.join(HERE, "..", "ex-nihilo_amd", "_build", "gemm.o")
LLVM = "/opt/rocm/llvm/bin"
KERNELS = ("k_gemm_q8_tall", "k_gemm_few", "k_gemm_bt")

FUNC = re.compile(r"^([0-9a-f]+) <(\S+)>:$")
INSN = re.compile(r"^\s+(\S+)\s*(.*?)\s*//\s*([0-9A-F]+):(.*)$")
TARGET = re.compile(r"<(\S+)\+0x([0-9a-f]+)>")
VREG = re.compile(r"\b([va])(\d+)\b|\b([va])\[(\d+):(\d+)\]")


def disassemble(tmp):
    fat = os.path.join(tmp, "fat.bin")
    co = os.path.join(tmp, "gemm.co")
    subprocess.run([os.path.join(LLVM, "llvm-objcopy"), "--dump-section", ".hip_fatbin=" + fat, OBJ, os.devnull],
                   check=True)
    subprocess.run([os.path.join(LLVM, "clang-offload-bundler"), "--unbundle", "--type=o", "--input=" + fat,
                    "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", "--output=" + co], check=True)
    out = subprocess.run([os.path.join(LLVM, "llvm-objdump"), "-d", "--mcpu=gfx950", co], check=True,
                         capture_output=True, text=True).stdout
    funcs, cur = {}, None
    for line in out.splitlines():
        m = FUNC.match(line)
        if m:
            cur = (int(m.group(1), 16), [])
            funcs[m.group(2)] = cur
            continue
        m = INSN.match(line)
        if m and cur is not None:
            # a branch's operand is its target, which the comment names as symbol + offset
            t = TARGET.search(m.group(4))
            ops = "<%s+0x%s>" % t.groups() if t and m.group(1).startswith("s_") else m.group(2)
            cur[1].append((int(m.group(3), 16), m.group(1), ops))
    return funcs


def regs(operands):
    """The vector registers an operand list names (v and a, single or ranges)."""
    s = set()
    for m in VREG.finditer(operands.split("//")[0]):
        if m.group(1):
            s.add((m.group(1), int(m.group(2))))
        else:
            s.update((m.group(3), r) for r in range(int(m.group(4)), int(m.group(5)) + 1))
    return s


def vmcnt(operands):
    m = re.search(r"vmcnt\((\d+)\)", operands)
    return int(m.group(1)) if m else None


def is_vmem(op):
    return op.startswith(("buffer_", "global_", "flat_", "scratch_", "tbuffer_"))


def loops(base, insns):
    """(first, last) index ranges of the straight-line loops: a backward branch to an earlier
    instruction of the function, with no other branch between."""
    index = {a: i for i, (a, _, _) in enumerate(insns)}
    for i, (a, op, ops) in enumerate(insns):
        if not op.startswith("s_cbranch") and op != "s_branch":
            continue
        t = TARGET.search(ops)
        if not t:
            continue
        tgt = base + int(t.group(2), 16)
        if tgt < a and tgt in index:
            first = index[tgt]
            if not any(o.startswith("s_cbranch") or o == "s_branch" for _, o, _ in insns[first:i]):
                yield first, i


def violations(insns, first, last):
    body = insns[first:last + 1]
    bad = []
    for k, (a, op, ops) in enumerate(body):
        if not (is_vmem(op) and "load" in op) or " lds" in " " + ops:
            continue
        dest = regs(ops.split(",")[0])
        after = 0
        for step in range(1, len(body) + 1):
            a2, op2, ops2 = body[(k + step) % len(body)]
            if op2 == "s_waitcnt":
                n = vmcnt(ops2)
                if n is not None and n <= after:
                    break   # covered
                continue
            if regs(ops2) & dest:
                bad.append("%x %s %s: %s %s at %x before its wait" % (a, op, ops, op2, ops2, a2))
                break
            if is_vmem(op2):
                after += 1
        else:
            bad.append("%x %s %s: no wait covers it in the loop" % (a, op, ops))
    return bad


@pytest.mark.skipif(not os.path.exists(OBJ), reason="gemm.o not built (__graft_entry__.build())")
@pytest.mark.skipif(not shutil.which(os.path.join(LLVM, "llvm-objdump")), reason="no ROCm llvm-objdump")
def test_untracked_loads_are_waited_for(tmp_path):
    funcs = disassemble(str(tmp_path))
    checked = 0
    for name, (base, insns) in funcs.items():
        if not any(k in name for k in KERNELS):
            continue
        q8_bt = "k_gemm_bt" in name and "Lb1E" in name
        if "k_gemm_bt" in name and not q8_bt:
            continue
        for first, last in loops(base, insns):
            body = insns[first:last + 1]
            if not any(is_vmem(op) and "load" in op and " lds" not in " " + ops for _, op, ops in body):
                continue
            assert not violations(insns, first, last), (name, violations(insns, first, last))
            checked += 1
    # the tall kernel's 7 epilogues, the few-row kernel's and the 256 x 256 Q8_0 instances all
    # have a main loop with register loads in it
    assert checked >= 20, checked


def test_the_check_sees_an_early_use():
    """A planted read of a load's register before its wait is reported; after it, not."""
    ins = [(0x0, "buffer_load_dword", "v5, v1, s[0:3], s4 offen"),
           (0x8, "v_add_u32_e32", "v7, v5, v6"),
           (0x10, "s_waitcnt", "vmcnt(0)"),
           (0x14, "s_cbranch_scc1", "<f+0x0>")]
    assert violations(ins, 0, 3)
    ins[1], ins[2] = ins[2], ins[1]
    assert not violations(ins, 0, 3)
    # a wait that leaves the load out (one operation issued after it, vmcnt(2)) does not cover it
    ins = [(0x0, "buffer_load_dword", "v5, v1, s[0:3], s4 offen"),
           (0x8, "buffer_load_dwordx4", "v1, s[8:11], s4 offen lds"),
           (0x10, "s_waitcnt", "vmcnt(2)"),
           (0x14, "v_mov_b32_e32", "v9, v5"),
           (0x18, "s_cbranch_scc1", "<f+0x0>")]
    assert violations(ins, 0, 4)
    ins[2] = (0x10, "s_waitcnt", "vmcnt(1)")
    assert not violations(ins, 0, 4)
