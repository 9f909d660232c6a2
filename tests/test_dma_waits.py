"""The fused GEMMs stage their activation / dY tile by LDS DMA written as inline assembly, which
the compiler does not count, and wait for it with an explicit `s_waitcnt vmcnt(N)`: that is
right only if at least N other vector-memory loads are issued after a step's DMA and before the
wait (loads complete in order, so vmcnt(N) leaves only the N youngest in flight).  This test
compiles nf4_gemm.hip for gfx950 to assembly (hipcc cross-compiles without a GPU) and checks,
in every forward and input-gradient kernel, that after each group of `buffer_load_dwordx4 ...
lds` instructions a wait that covers it comes before the next barrier.

A load written as inline assembly is not known to the compiler at all: it neither waits for it
nor knows that its destination registers are busy until the explicit wait.  A second test
replays every kernel's instruction stream (each loop body twice, the second pass starting with
the loads still in flight at the end of the first; a forward branch hands its state to its
target) through an in-order model of the vmcnt counter and checks that no instruction reads or
writes a register that an inline-assembly load still in flight is to write."""

import re

import pytest



def _kernels(asm: str):
    """(name, lines) of every function in the assembly text; an instruction written as inline
    assembly in the source (between the compiler's ASMSTART / ASMEND markers) gets the prefix
    "@asm ".  """
    out, name, body, in_asm = [], None, [], False
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
        if ";;#ASMSTART" in line:
            in_asm = True
        elif ";;#ASMEND" in line:
            in_asm = False
        t = line.split(";")[0].strip()
        if t:
            body.append(("@asm " + t) if in_asm else t)
    return out


def _strip(lines):
    return [t[5:] if t.startswith("@asm ") else t for t in lines]


def _is_dma(t):
    return t.startswith("buffer_load_dwordx4") and t.endswith(" lds")


def _check(lines, barriers_allowed=0):
    """Number of DMA groups checked; raises AssertionError on a group not covered by a wait
    before barrier number barriers_allowed + 1 after it."""
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
        loads, covered, barriers = 0, False, 0
        for t in lines[j + 1:]:
            if t.startswith(("buffer_load", "global_load")):
                loads += 1
            elif t.startswith("s_waitcnt") and "vmcnt(" in t:
                if int(re.search(r"vmcnt\((\d+)\)", t).group(1)) <= loads:
                    covered = True
                    break
            elif t.startswith("s_barrier"):
                barriers += 1
                if barriers > barriers_allowed:
                    break
        assert covered, f"DMA group ending at line {j} is not waited for in time"
        i = j + 1
    return groups


@pytest.fixture(scope="module")
def kernels(gemm_asm):
    """(name, lines) of every forward and input-gradient kernel of nf4_gemm.hip."""
    ks = [(k, b) for k, b in _kernels(gemm_asm) if re.search(r"(fwd|dx)_(head_tail_|rw_)?kernel", k)]
    assert len(ks) >= 8
    return ks


_REG = re.compile(r"\bv\[(\d+):(\d+)\]|\bv(\d+)\b")


def _regs(text):
    out = set()
    for m in _REG.finditer(text):
        if m.group(3) is not None:
            out.add(int(m.group(3)))
        else:
            out.update(range(int(m.group(1)), int(m.group(2)) + 1))
    return out


def _replay(lines):
    """In-order vmcnt model over the instruction stream.  Loads written as inline assembly
    ("@asm " lines) are tracked with their destination registers (the compiler waits for its own
    loads before their registers are touched); every load and store counts in vmcnt.  Control
    flow: a forward branch hands its states (the possible queues of loads in flight) to its
    target label, an unconditional one ends the fall-through path, and a backward branch (a loop)
    replays the loop body once with the states its first pass ends in.  Returns the hazards
    (line, instruction, register): an instruction that reads or writes a register an assembly
    load still in flight is to write."""
    labels = {t[:-1]: i for i, t in enumerate(lines) if t.startswith(".L") and t.endswith(":")}
    hazards = []

    def flag(i, t, regs, queues):
        for r in regs:
            if any(r in q for qu in queues for q in qu):
                hazards.append((i, t, r))

    def step(i, queues):
        """Apply line i to every possible queue; returns the new list of queues."""
        t = lines[i]
        is_asm = t.startswith("@asm ")
        if is_asm:
            t = t[5:]
        op = t.split()[0] if t else ""
        if op.startswith("s_waitcnt") and "vmcnt(" in t:
            keep = int(re.search(r"vmcnt\((\d+)\)", t).group(1))
            return [qu[max(0, len(qu) - keep):] for qu in queues]
        if op.startswith(("buffer_load", "global_load", "buffer_store", "global_store",
                          "buffer_atomic", "global_atomic")):
            ops = t[len(op):]
            dst = frozenset()
            src_txt = ops
            if op.startswith(("buffer_load", "global_load")) and not t.endswith(" lds"):
                dst_txt, src_txt = ops.split(",", 1)
                flag(i, t, _regs(dst_txt), queues)
                if is_asm:
                    dst = frozenset(_regs(dst_txt))
            flag(i, t, _regs(src_txt), queues)
            return [qu + (dst,) for qu in queues]
        flag(i, t, _regs(t), queues)
        return queues

    def dedup(queues):
        return list(dict.fromkeys(queues))

    pending = {}
    states = [()]
    looped = set()
    for i, t in enumerate(lines):
        if t.startswith(".L") and t.endswith(":"):
            states = dedup(states + pending.pop(t[:-1], []))
            continue
        if not states:
            continue
        states = step(i, states)
        if t.startswith(("s_cbranch", "s_branch")):
            target = t.split()[-1]
            start = labels.get(target)
            if start is not None and start > i:
                pending[target] = dedup(pending.get(target, []) + states)
            elif start is not None and target not in looped:
                looped.add(target)
                for k in range(start + 1, i + 1):
                    if not (lines[k].startswith(".L") and lines[k].endswith(":")):
                        states = step(k, states)
                states = dedup(states)
            if t.startswith("s_branch"):
                states = []
        elif t.startswith("s_endpgm"):
            states = []
    return hazards


@pytest.mark.timeout(600)
def test_dma_is_waited_for_before_the_barrier(kernels):
    checked = 0
    for name, body in kernels:
        g = _check(_strip(body))
        assert g >= 3, f"{name}: expected the prologue's and the loop's DMA groups, found {g}"
        checked += g
    assert checked > 0


@pytest.mark.timeout(600)
def test_no_register_of_a_load_in_flight_is_touched(kernels):
    for name, body in kernels:
        hz = _replay(body)
        assert not hz, f"{name}: {hz[:3]}"


def test_replay_model_flags_a_register_used_before_its_wait():
    """The model itself: a load whose register is read before a wait covers it is flagged; the
    same read after vmcnt(0), or after a vmcnt(1) that leaves only a younger load in flight, is
    not."""
    base = ["@asm buffer_load_dwordx4 v[4:7], v1, s[0:3], 0 offen",
            "@asm buffer_load_dword v9, v2, s[0:3], 0 offen"]
    assert _replay(base + ["v_add_u32_e32 v10, v5, v3"])
    assert not _replay(base + ["s_waitcnt vmcnt(1)", "v_add_u32_e32 v10, v5, v3"])
    assert _replay(base + ["s_waitcnt vmcnt(1)", "v_add_u32_e32 v10, v9, v3"])
    assert not _replay(base + ["s_waitcnt vmcnt(0)", "v_add_u32_e32 v10, v9, v3"])
    # a loop body replayed: the load issued at its end is in flight at its start
    loop = [".LBB0_1:", "v_mov_b32_e32 v20, v8", "s_waitcnt vmcnt(0)",
            "@asm buffer_load_dword v8, v2, s[0:3], 0 offen", "s_cbranch_scc1 .LBB0_1"]
    assert _replay(loop)
    # the DMA form writes no register (its first operand is the address)
    assert not _replay(["@asm buffer_load_dwordx4 v3, s[0:3], s4 offen lds", "v_mov_b32_e32 v5, v3"])
    # a load the compiler issued is not tracked (the compiler waits for it itself)
    assert not _replay(["buffer_load_dword v9, v2, s[0:3], 0 offen", "v_mov_b32_e32 v5, v9"])
