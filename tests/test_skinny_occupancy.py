"""The skinny forward path's planner charges a kernel shape extra when its registers or LDS leave
one 8-wave workgroup per CU (`skinny_slots` in nf4_gemm.hip).  That table is written from the
compiler's register counts; this test compiles nf4_gemm.hip for gfx950 to assembly (hipcc
cross-compiles without a GPU) and recomputes, for every skinny kernel the planner can launch
without the in-launch LoRA down-projection, the workgroups per CU from the kernel metadata
(`.vgpr_count` + `.agpr_count` rounded to the 8-register granule of a 512-register SIMD lane,
at most 8 waves per SIMD, 2 waves per SIMD for each 8-wave workgroup; LDS from
`.group_segment_fixed_size` against 160 KB), and checks it against the table."""

import re

import pytest



def table_slots(mt, rt, dks):
    """Mirror of skinny_slots() in nf4_gemm.hip."""
    return 1 if (dks == 256 and rt <= 2) or (mt == 2 and rt == 1) or (mt == 4 and rt <= 4) else 2


def _metadata(asm: str):
    """{kernel name: {field: int}} from the amdhsa.kernels metadata of an assembly file."""
    meta = asm[asm.index("amdhsa.kernels:"):]
    out = {}
    for block in re.split(r"\n  - ", meta)[1:]:
        name = re.search(r"\.name:\s+(\S+)", block)
        if not name:
            continue
        fields = {}
        for key in ("vgpr_count", "agpr_count", "group_segment_fixed_size"):
            m = re.search(rf"\.{key}:\s+(\d+)", block)
            fields[key] = int(m.group(1)) if m else 0
        out[name.group(1)] = fields
    return out


@pytest.mark.timeout(600)
def test_skinny_slots_match_the_compiled_kernels(gemm_asm):
    checked = 0
    for name, f in _metadata(gemm_asm).items():
        m = re.search(r"skinny_kernelILi(\d)ELi(\d)ELi(\d)ELi(\d)ELi(\d+)ELb([01])E", name)
        if not m or m.group(6) == "1":
            continue
        mt, rt, dks = int(m.group(2)), int(m.group(3)), int(m.group(5))
        regs = -(-(f["vgpr_count"] + f["agpr_count"]) // 8) * 8
        waves = min(8, 512 // regs)
        by_lds = (160 * 1024) // max(1, f["group_segment_fixed_size"])
        slots = max(1, min(waves // 2, by_lds))
        assert min(slots, 2) == table_slots(mt, rt, dks), (name, f, slots)
        checked += 1
    assert checked >= 15, checked
