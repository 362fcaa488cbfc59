"""The DPP wait-state rule (a VALU write of a VGPR needs 2 wait states before a DPP instruction
reads it as its DPP source) checked on the gfx950 code of the built objects, after the checker
itself is shown to catch planted violations in synthetic disassembly.

The forward scan's inline-asm v_fmac_f32_dpp (row_newbcast broadcasts of B and C) is guarded by an
`s_nop 1` tied to its source registers; that guard is only as good as the compiler's placement of
the instructions around it, which this test reads back from every build."""
import glob
import os

import pytest

from tests import isa_hazards as H

OBJ_DIR = os.path.join(os.path.dirname(__file__), "..", "motif-mamba_amd", "motif_mamba_amd", "_obj")


def _fn(body):
    """A one-function disassembly in llvm-objdump's layout; body = [(mnemonic, args, target offset)]."""
    lines = ["0000000000001000 <f>:"]
    for k, (op, args, tgt) in enumerate(body):
        addr = 0x1000 + 4 * k
        tail = f" <f+0x{tgt:x}>" if tgt is not None else ""
        lines.append(f"\t{op} {args}    // {addr:012X}: 00000000{tail}")
    return "\n".join(lines)


def _violations(body):
    insts = H.parse(_fn(body))["f"]
    return H.check_function(insts)


DPP = ("v_fmac_f32_dpp", "v0, v5, v2 row_newbcast:1 row_mask:0xf bank_mask:0xf", None)


def test_checker_flags_a_write_right_before_the_dpp_read():
    assert len(_violations([("v_mov_b32_e32", "v5, v1", None), DPP])) == 1


def test_checker_flags_one_wait_state():
    assert len(_violations([("v_mul_f32_e32", "v5, v1, v3", None), ("s_nop", "0", None), DPP])) == 1
    assert len(_violations([("v_mul_f32_e32", "v5, v1, v3", None), ("v_add_f32_e32", "v7, v1, v3", None), DPP])) == 1


def test_checker_accepts_two_wait_states():
    assert not _violations([("v_mul_f32_e32", "v5, v1, v3", None), ("s_nop", "1", None), DPP])
    assert not _violations([("v_mul_f32_e32", "v5, v1, v3", None), ("v_add_f32_e32", "v7, v1, v3", None),
                            ("v_add_f32_e32", "v8, v1, v3", None), DPP])


def test_checker_reads_register_ranges_and_ignores_other_registers():
    assert len(_violations([("v_lshl_add_u64", "v[4:5], v[0:1], 0, v[2:3]", None), DPP])) == 1
    assert not _violations([("v_mov_b32_e32", "v6, v1", None), DPP])
    # the DPP read is of src0 only: a write of src1 (v2) right before is no hazard
    assert not _violations([("v_mov_b32_e32", "v2, v1", None), DPP])


def test_checker_follows_branches_into_a_block():
    # block 0: write v5, branch to the DPP at offset 0x10 (the branch is one wait state)
    body = [("v_mov_b32_e32", "v5, v1", None), ("s_branch", "2", 0x10),
            ("v_mov_b32_e32", "v9, v1", None), ("s_nop", "4", None), DPP]
    assert len(_violations(body)) == 1
    # the fall-through path alone (s_nop 4 before the DPP) would have been fine
    assert not _violations(body[2:])


def _objects():
    return sorted(glob.glob(os.path.join(OBJ_DIR, "*.o")))


@pytest.mark.skipif(not _objects() or not os.path.exists(os.path.join(H.LLVM_BIN, "llvm-objdump")),
                    reason="no built objects (run __graft_entry__.build()) or no ROCm LLVM tools")
def test_built_kernels_respect_dpp_wait_states():
    total = 0
    for obj in _objects():
        n, bad = H.check_object(obj)
        total += n
        assert not bad, f"{os.path.basename(obj)}: {sum(len(v) for v in bad.values())} DPP reads within " \
                        f"{H.NEED_WS} wait states of a VALU write, e.g. {next(iter(bad.items()))}"
        if os.path.basename(obj).startswith("mm_scan_tiled"):
            assert n > 1000, f"{obj}: only {n} DPP instructions found (disassembly not parsed?)"
    assert total > 0
