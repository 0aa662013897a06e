"""Checks on the gfx950 machine code of the built library (CPU only).

The GEMM issues its direct global->LDS loads (`global_load_lds_dwordx4`) as
inline asm (`dma16` in csrc/mnb_device.h), and the compiler's hazard
recognizer does not look inside inline asm.  gfx9 requires:
  - 5 wait states between a VALU write of an SGPR (v_readlane reloading a
    spilled SGPR, v_readfirstlane, a VOP3 carry-out) and a vector memory
    instruction that reads that SGPR (the load's scalar base);
  - 1 wait state between an SALU write of M0 and an LDS DMA.
A build that broke the first rule read a stale base and faulted.  These
tests disassemble the library's code objects with llvm-objdump and walk
back from every such load along every path into it (fall-through and
branches), counting wait states (1 per instruction, N + 1 for s_nop N).
"""
import os
import re
import shutil
import subprocess
import tempfile

import pytest

import mnb_hip

OBJDUMP = "/opt/rocm/llvm/bin/llvm-objdump"

_INST = re.compile(r"^\s+([a-z_0-9]+)(?:\s+([^/]*?))?\s*//\s*([0-9A-Fa-f]+):")
_FUNC = re.compile(r"^[0-9a-f]+ <(.+)>:$")
_SREG = re.compile(r"^s\[(\d+):(\d+)\]$|^s(\d+)$")


def _sgprs(tok):
    m = _SREG.match(tok.strip())
    if not m:
        return set()
    if m.group(3) is not None:
        return {int(m.group(3))}
    return set(range(int(m.group(1)), int(m.group(2)) + 1))


def parse(text):
    """{function: [(addr, mnemonic, [operands])]} from llvm-objdump -d output."""
    funcs, cur = {}, None
    for line in text.splitlines():
        m = _FUNC.match(line.strip())
        if m:
            cur = funcs.setdefault(m.group(1), [])
            continue
        m = _INST.match(line)
        if m and cur is not None:
            ops = [o.strip() for o in (m.group(2) or "").split(",") if o.strip()]
            cur.append((int(m.group(3), 16), m.group(1), ops))
    return funcs


def _wait_states(mn, ops):
    if mn == "s_nop":
        return int(ops[0], 0) + 1
    return 1


def _valu_sgpr_writes(mn, ops):
    """SGPRs a VALU instruction writes: its first operand when that is an
    SGPR (v_readlane, v_readfirstlane, v_cmp_*_e64), and the carry-out or
    second destination of the two-destination forms."""
    if not mn.startswith("v_") or not ops:
        return set()
    out = _sgprs(ops[0])
    if len(ops) > 1 and ("_co_" in mn or mn.startswith(("v_mad_u64", "v_mad_i64", "v_div_scale"))):
        out |= _sgprs(ops[1])
    return out


def _writes_m0(mn, ops):
    return mn.startswith("s_") and bool(ops) and ops[0] == "m0"


_ENDS = ("s_branch", "s_endpgm", "s_setpc_b64")


def _preds(insts, index_of, q):
    """Instructions that can execute right before instruction q."""
    out = []
    if q > 0 and not insts[q - 1][1].startswith(_ENDS):
        out.append(q - 1)
    out.extend(index_of.get(insts[q][0], ()))
    return out


def hazards(funcs):
    """Violations as (function, load address, offending instruction, wait states between)."""
    bad = []
    for name, insts in funcs.items():
        addr_idx = {a: i for i, (a, _, _) in enumerate(insts)}
        branch_to = {}
        for i, (a, mn, ops) in enumerate(insts):
            if mn.startswith(("s_branch", "s_cbranch")) and ops:
                t = a + 4 + 4 * int(ops[0], 0)
                if t in addr_idx:
                    branch_to.setdefault(t, []).append(i)
        for i, (a, mn, ops) in enumerate(insts):
            if not mn.startswith("global_load_lds"):
                continue
            base = _sgprs(ops[1]) if len(ops) > 1 else set()
            # walk back: (instruction before which we stand, wait states since)
            stack, seen = [(i, 0)], set()
            while stack:
                q, ws = stack.pop()
                for p in _preds(insts, branch_to, q):
                    if (p, ws) in seen:
                        continue
                    seen.add((p, ws))
                    _, pmn, pops = insts[p]
                    if ws < 5 and base & _valu_sgpr_writes(pmn, pops):
                        bad.append((name, hex(a), pmn + " " + ", ".join(pops), ws))
                    if ws < 1 and _writes_m0(pmn, pops):
                        bad.append((name, hex(a), pmn + " " + ", ".join(pops), ws))
                    w = ws + _wait_states(pmn, pops)
                    if w < 5:
                        stack.append((p, w))
    return bad


def _disassemble(lib):
    with tempfile.TemporaryDirectory() as d:
        so = os.path.join(d, "lib.so")
        shutil.copy(lib, so)
        subprocess.run([OBJDUMP, "--offloading", so], cwd=d, check=True, capture_output=True)
        objs = sorted(f for f in os.listdir(d) if "gfx950" in f)
        assert objs, "no gfx950 code object in %s" % lib
        return "\n".join(
            subprocess.run([OBJDUMP, "-d", "--mcpu=gfx950", os.path.join(d, f)], check=True, capture_output=True,
                           text=True).stdout for f in objs)


@pytest.fixture(scope="module")
def library_code():
    lib = mnb_hip.library_path()
    if not os.path.exists(lib):
        pytest.skip("library not built: " + lib)
    if not os.path.exists(OBJDUMP):
        pytest.skip("llvm-objdump not found")
    return parse(_disassemble(lib))


def test_direct_lds_loads_keep_their_wait_states(library_code):
    loads = sum(1 for insts in library_code.values() for (_, mn, _) in insts if mn.startswith("global_load_lds"))
    assert loads > 100, "expected the GEMM's direct-to-LDS loads in the library, found %d" % loads
    bad = hazards(library_code)
    assert not bad, "direct-to-LDS loads too close to a write of their base or M0: %s" % bad[:10]


# A listing in llvm-objdump's format: the hazards a build of the GEMM
# without MFMAs had (a spilled SGPR reloaded by v_readlane right before the
# load, a second load with the same base 4 wait states later), an M0 write
# right before a load, a branch into the window, and a form that must pass.
_PLANTED = """
0000000000001000 <k_bad>:
\tv_readlane_b32 s36, v173, 44                               // 000000001000: D2890024 00015
\tv_lshl_add_u32 v62, v62, 1, v157                           // 000000001008: D1FD003E 0676033E
\ts_mov_b32 m0, s48                                          // 000000001010: BEFC0030
\tv_readlane_b32 s37, v173, 45                               // 000000001014: D2890025 00015
\tglobal_load_lds_dwordx4 v62, s[36:37]                      // 00000000101C: DDF48000 0024003E
\tv_or_b32_e32 v62, s58, v130                                // 000000001024: 287D043A
\tv_lshl_add_u32 v62, v62, 1, v158                           // 000000001028: D1FD003E 067A033E
\ts_add_i32 m0, s48, 0x400                                   // 000000001030: 817CFF30 00000400
\tglobal_load_lds_dwordx4 v62, s[36:37]                      // 000000001038: DDF48000 0024003E
\ts_endpgm                                                   // 000000001040: BF810000
0000000000002000 <k_branch>:
\tv_readfirstlane_b32 s9, v3                                 // 000000002000: 7E120503
\ts_branch 3                                                 // 000000002004: BF820003
\ts_nop 7                                                    // 000000002008: BF800007
\ts_nop 7                                                    // 00000000200C: BF800007
\ts_nop 7                                                    // 000000002010: BF800007
\ts_mov_b32 m0, s2                                           // 000000002014: BEFC0002
\ts_nop 0                                                    // 000000002018: BF800000
\tglobal_load_lds_dwordx4 v4, s[8:9]                         // 00000000201C: DDF48000 00080004
\ts_endpgm                                                   // 000000002024: BF810000
0000000000003000 <k_good>:
\tv_readlane_b32 s37, v173, 45                               // 000000003000: D2890025 00015
\tv_or_b32_e32 v62, s58, v130                                // 000000003008: 287D043A
\ts_nop 2                                                    // 00000000300C: BF800002
\ts_mov_b32 m0, s48                                          // 000000003010: BEFC0030
\ts_nop 0                                                    // 000000003014: BF800000
\tglobal_load_lds_dwordx4 v62, s[36:37]                      // 000000003018: DDF48000 0024003E
\ts_endpgm                                                   // 000000003020: BF810000
"""


def test_the_checker_finds_planted_hazards():
    funcs = parse(_PLANTED)
    assert set(funcs) == {"k_bad", "k_branch", "k_good"}
    bad = hazards(funcs)
    found = {(f, a, ws) for (f, a, _, ws) in bad}
    # k_bad: the first load right after the v_readlane of s37 and 3 wait
    # states after that of s36; the second load right after an M0 write and
    # 4 wait states after the v_readlane of s37
    assert ("k_bad", "0x101c", 0) in found
    assert ("k_bad", "0x101c", 3) in found
    assert ("k_bad", "0x1038", 4) in found
    assert any(f == "k_bad" and a == "0x1038" and "m0" in i and ws == 0 for (f, a, i, ws) in bad)
    assert not any(f == "k_bad" and a == "0x101c" and "m0" in i for (f, a, i, _) in bad)
    # k_branch: the s_branch skips the padding, so the v_readfirstlane of s9
    # reaches the load after 1 (branch) + 2 (s_mov, s_nop 0) wait states
    assert ("k_branch", "0x201c", 3) in found
    # k_good: 1 + 3 + 1 + 1 = 6 wait states after the v_readlane, 1 after M0
    assert not any(f == "k_good" for (f, _, _, _) in bad)
