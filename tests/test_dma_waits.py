"""The fused GEMMs stage their activation / dY tile by LDS DMA written as inline assembly, which
the compiler does not count, and wait for it with an explicit `s_waitcnt vmcnt(3)`: that is
right only if at least 3 other vector-memory loads are issued after a step's DMA and before the
wait (loads complete in order, so vmcnt(N) leaves only the N youngest in flight).  The kernel
source places exactly one weight register stage (3 loads) there; this test compiles
nf4_gemm.hip for gfx950 to assembly (hipcc cross-compiles without a GPU) and checks, in every
forward and input-gradient kernel, that after each group of `buffer_load_dwordx4 ... lds`
instructions the first wait that covers them comes before the next barrier or DMA: a wait
vmcnt(N) covers them once at least N loads have been issued after the group's last DMA."""

import re
import subprocess

import pytest

from tests.conftest import PKG


def _hipcc():
    import build

    try:
        return build.hipcc()
    except RuntimeError:
        return None


def _kernels(asm: str):
    """(name, lines) of every function in the assembly text."""
    out, name, body = [], None, []
    for line in asm.split("\n"):
        m = re.match(r"^(_Z\S+):", line)
        if m:
            name, body = m.group(1), []
            continue
        if name is None:
            continue
        if line.startswith(".Lfunc_end"):
            out.append((name, body))
            name = None
            continue
        t = line.split(";")[0].strip()
        if t:
            body.append(t)
    return out


def _is_dma(t):
    return t.startswith("buffer_load_dwordx4") and t.endswith(" lds")


def _check(lines):
    """Number of DMA groups checked; raises AssertionError on an uncovered group."""
    groups, i, n = 0, 0, len(lines)
    while i < n:
        if not _is_dma(lines[i]):
            i += 1
            continue
        # the group: DMA instructions with no other load, wait, barrier or branch between them
        j, k = i, i + 1
        while k < n and (_is_dma(lines[k]) or not (
                lines[k].startswith(("buffer_load", "global_load", "s_barrier", "s_cbranch",
                                     "s_branch", "s_endpgm", "."))
                or lines[k].startswith("s_waitcnt") and "vmcnt" in lines[k])):
            if _is_dma(lines[k]):
                j = k
            k += 1
        groups += 1
        loads, covered = 0, False
        for t in lines[j + 1:]:
            if t.startswith(("buffer_load", "global_load")):
                assert not t.endswith(" lds"), "a second DMA group before the first one's wait"
                loads += 1
            elif t.startswith("s_waitcnt") and "vmcnt(" in t:
                if int(re.search(r"vmcnt\((\d+)\)", t).group(1)) <= loads:
                    covered = True
                    break
            elif t.startswith("s_barrier"):
                break
        assert covered, f"DMA group ending at line {j} is not waited for before the next barrier"
        i = j + 1
    return groups


@pytest.mark.timeout(600)
def test_dma_is_waited_for_before_the_barrier(tmp_path):
    hipcc = _hipcc()
    if hipcc is None:
        pytest.skip("hipcc not available")
    import build

    out = tmp_path / "nf4_gemm.s"
    cmd = [hipcc, *build.FLAGS, "--offload-device-only", "-S", str(PKG / "csrc" / "nf4_gemm.hip"),
           "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    kernels = [(k, b) for k, b in _kernels(out.read_text())
               if re.search(r"(fwd|dx)_(head_tail_|rw_)?kernel", k)]
    assert len(kernels) >= 8
    checked = 0
    for name, body in kernels:
        g = _check(body)
        assert g >= 3, f"{name}: expected the prologue's and the loop's DMA groups, found {g}"
        checked += g
    assert checked > 0
