"""Static check of one wait-state rule in the gfx950 code of this build's own kernels.

A VALU instruction that writes a VGPR must be followed by at least 2 wait states before a DPP
instruction reads that VGPR as its DPP source (src0): the CDNA3/CDNA4 ISA's manually inserted
wait states ("VALU write VGPR -> VALU DPP read of that VGPR: 2"). The compiler inserts them for the
DPP instructions it emits itself; the inline-asm v_fmac_f32_dpp of the forward scan relies on an
`s_nop 1` tied to its source registers, which holds only as long as the compiler puts nothing that
rewrites the source between that s_nop and the DPP read. This module checks the rule on the
disassembly of the built objects, for every DPP instruction, whoever emitted it.

Input: the device code object of a hipcc object file (`.hip_fatbin` section, unbundled with
clang-offload-bundler for gfx950) disassembled by llvm-objdump. Wait states: `s_nop N` provides
N + 1, every other instruction 1. Across basic blocks the walk follows both the fall-through
predecessor and every branch that targets the block.
"""
from __future__ import annotations

import os
import re
import subprocess
import tempfile

LLVM_BIN = "/opt/rocm/llvm/bin"
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"
NEED_WS = 2

_FUNC = re.compile(r"^([0-9a-f]+) <(.+)>:$")
_INST = re.compile(r"^\s+(\S+)\s*(.*?)\s*//\s*([0-9A-F]+):")
_TARGET = re.compile(r"<(.+)\+0x([0-9a-f]+)>")
_VREG = re.compile(r"^v(\d+)$")
_VRANGE = re.compile(r"^v\[(\d+):(\d+)\]$")


def disassemble(obj_path: str) -> str:
    """llvm-objdump text of the gfx950 device code inside a hipcc object file."""
    with tempfile.TemporaryDirectory() as tmp:
        fat = os.path.join(tmp, "fatbin")
        dev = os.path.join(tmp, "dev.co")
        subprocess.run([f"{LLVM_BIN}/llvm-objcopy", f"--dump-section=.hip_fatbin={fat}", obj_path, os.devnull],
                       check=True, capture_output=True)
        subprocess.run([f"{LLVM_BIN}/clang-offload-bundler", "--unbundle", "--type=o", f"--input={fat}",
                        f"--targets={TARGET}", f"--output={dev}"], check=True, capture_output=True)
        out = subprocess.run([f"{LLVM_BIN}/llvm-objdump", "-d", "--mcpu=gfx950", dev], check=True,
                             capture_output=True, text=True)
        return out.stdout


def _regs(tok: str):
    tok = tok.strip().rstrip(",")
    m = _VREG.match(tok)
    if m:
        return {int(m.group(1))}
    m = _VRANGE.match(tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    return set()


class Inst:
    __slots__ = ("addr", "op", "args", "ws", "vwrites", "dpp_src", "target", "ends_block")

    def __init__(self, addr, op, args, line, func_start, func_name):
        self.addr, self.op, self.args = addr, op, args
        self.ws = int(args.split()[0], 0) + 1 if op == "s_nop" else 1
        toks = [t for t in args.replace(",", " ").split()]
        valu = op.startswith("v_") and not op.startswith(("v_readlane", "v_readfirstlane", "v_cmp"))
        self.vwrites = _regs(toks[0]) if (valu and toks) else set()
        is_dpp = op.endswith("_dpp") or any(k in args for k in ("row_newbcast", "quad_perm", "row_shl",
                                                                  "row_shr", "row_ror", "row_mirror",
                                                                  "row_half_mirror", "row_bcast",
                                                                  "wave_shl", "wave_shr", "wave_rol",
                                                                  "wave_ror", "row_share", "row_xmask"))
        self.dpp_src = None
        if is_dpp and op.startswith("v_") and len(toks) >= 2:
            r = _regs(toks[1])
            self.dpp_src = r if r else None
        self.target = None
        if op.startswith(("s_branch", "s_cbranch")):
            m = _TARGET.search(line)   # llvm-objdump prints the target after the encoding
            if m and m.group(1) == func_name:
                self.target = func_start + int(m.group(2), 16)
        self.ends_block = op in ("s_branch", "s_endpgm", "s_setpc_b64")


def parse(text: str):
    """{function name: [Inst, ...]} in address order."""
    funcs, cur, name, start = {}, None, None, 0
    for line in text.splitlines():
        m = _FUNC.match(line)
        if m:
            start, name = int(m.group(1), 16), m.group(2)
            cur = funcs.setdefault(name, [])
            continue
        if cur is None:
            continue
        m = _INST.match(line)
        if m:
            cur.append(Inst(int(m.group(3), 16), m.group(1), m.group(2), line, start, name))
    return funcs


def check_function(insts):
    """Violations [(dpp address, dpp text, writer address, writer text, wait states between)]."""
    index = {ins.addr: i for i, ins in enumerate(insts)}
    preds = {}   # block-start index -> indices of branch instructions targeting it
    for i, ins in enumerate(insts):
        if ins.target is not None and ins.target in index:
            preds.setdefault(index[ins.target], []).append(i)
    bad = []

    def walk(i, regs, ws, dpp, seen):
        # instruction i precedes the DPP instruction with `ws` wait states between them
        if ws >= NEED_WS or i < 0 or (i, ws) in seen:
            return
        seen.add((i, ws))
        ins = insts[i]
        if ins.vwrites & regs:
            bad.append((dpp.addr, f"{dpp.op} {dpp.args}", ins.addr, f"{ins.op} {ins.args}", ws))
        nws = ws + ins.ws
        # predecessors of instruction i: i - 1 unless it ends a block, and branches to i
        if i - 1 >= 0 and not insts[i - 1].ends_block:
            walk(i - 1, regs, nws, dpp, seen)
        for b in preds.get(i, ()):
            walk(b, regs, nws, dpp, seen)   # the branch itself is the instruction before i

    for i, ins in enumerate(insts):
        if ins.dpp_src:
            seen = set()
            if i - 1 >= 0 and not insts[i - 1].ends_block:
                walk(i - 1, ins.dpp_src, 0, ins, seen)
            for b in preds.get(i, ()):
                walk(b, ins.dpp_src, 0, ins, seen)
    return bad


def check_object(obj_path: str):
    """(number of DPP instructions checked, violations by function)."""
    funcs = parse(disassemble(obj_path))
    n_dpp, out = 0, {}
    for name, insts in funcs.items():
        n_dpp += sum(1 for x in insts if x.dpp_src)
        v = check_function(insts)
        if v:
            out[name] = v
    return n_dpp, out
