"""Host model of the key split's merge protocols (no GPU).

The split kernels (attn_fwd_pipe16.h, attn_fwd_mfma16.h, attn_fwd_mfma32.hip)
let the parts of a query block hand their partial (O, m, l) to one merging
part through per-(block, wave) counters in an exchange space.  A protocol in
which a part waits for another workgroup can hang the GPU when two launches
share the counters (the allocation-free entry point's fixed scratch, or a
workspace handed to two streams at once).  This module models each part as a
sequence of atomic steps on shared counters and explores every interleaving
of the parts of one or two launches:

* the former two-part protocol (ticket, then the second part spins on a
  "written" flag) reaches a state where the parts still running can only
  spin: it blocks forever;
* the protocols the kernels use now never wait, so every interleaving ends
  with every part finished.  With one launch at a time exactly one part
  merges, it sees every other part's state written, and the counters are
  back at zero; with two overlapping launches the result may be mixed (the
  documented contract) but nothing blocks.
"""
from __future__ import annotations

# ---------------------------------------------------------------- the model
#
# Each part is a small state machine: step(pc, me, mem) performs one atomic
# action on the shared memory and returns the next program point, or a
# finished record ("done", merged, states seen by the merger).  A wait whose
# condition is false returns the same program point and leaves memory
# untouched (a spin).  Memory is (c0, c1, states written); c0 and c1 are the
# two counters of one (block, wave), shared by every launch that uses the same
# exchange space.


def old_two_part(pc, me, mem):
    """The former protocol: ticket first; the first writes and raises the
    flag, the second spins until the flag is up, then resets and merges."""
    c0, c1, written = mem
    if pc == 0:
        return (1 if c0 == 0 else 3), (c0 + 1, c1, written)
    if pc == 1:
        return 2, (c0, c1, written | {me})
    if pc == 2:
        return ("done", False, None), (c0, 1, written)
    if pc == 3:
        return (3 if c1 == 0 else 4), mem          # spin until the flag is up
    if pc == 4:
        return ("done", True, written), (0, 0, written)
    raise AssertionError(pc)


def new_two_part(pc, me, mem):
    """attn_fwd_pipe16.h, two parts: count arrivals; the first always leaves
    its state, the second only if the first has not finished writing; whoever
    completes the pair merges and resets both counters.  No step waits."""
    c0, c1, written = mem
    if pc == 0:                                     # arrivals
        return (1 if c0 == 0 else 4), (c0 + 1, c1, written)
    if pc == 1:                                     # first: leave state
        return 2, (c0, c1, written | {me})
    if pc == 2:                                     # first: count the write
        return (("done", False, None) if c1 == 0 else 7), (c0, c1 + 1, written)
    if pc == 4:                                     # second: is the first's state in?
        return (5 if c1 == 0 else 7), mem
    if pc == 5:                                     # second: leave state too
        return 6, (c0, c1, written | {me})
    if pc == 6:
        return (("done", False, None) if c1 == 0 else 7), (c0, c1 + 1, written)
    if pc == 7:                                     # merge, reset
        return ("done", True, written), (0, 0, written)
    raise AssertionError(pc)


def count_in(nparts):
    """Every split kernel, more than two parts: every part writes, then
    counts itself in; the one that brings the count to nparts merges."""
    def step(pc, me, mem):
        c0, c1, written = mem
        if pc == 0:
            return 1, (c0, c1, written | {me})
        if pc == 1:
            return (("done", False, None) if c0 != nparts - 1 else 2), (c0 + 1, c1, written)
        if pc == 2:
            return ("done", True, written), (0, c1, written)
        raise AssertionError(pc)
    return step


def explore(step, parts_per_launch, launches):
    """Every interleaving of the parts of `launches` launches sharing one
    counter pair.  Returns (final states, blocked): a final state maps each
    part to its finished record, plus the final memory; blocked is True when
    some reachable state has live parts that can only spin."""
    procs = tuple((l, p) for l in range(launches) for p in range(parts_per_launch))
    start = ((0, 0, frozenset()), tuple(0 for _ in procs))
    seen, stack, finals, blocked = {start}, [start], [], False
    while stack:
        mem, pcs = stack.pop()
        live = [i for i, pc in enumerate(pcs) if not isinstance(pc, tuple)]
        if not live:
            finals.append(({procs[i]: pcs[i] for i in range(len(procs))}, mem))
            continue
        moved = False
        for i in live:
            npc, nmem = step(pcs[i], procs[i], mem)
            nxt = (nmem, pcs[:i] + (npc,) + pcs[i + 1:])
            if nxt == (mem, pcs):
                continue                            # a spin: nothing changes
            moved = True
            if nxt not in seen:
                seen.add(nxt)
                stack.append(nxt)
        if not moved:
            blocked = True
    return finals, blocked


# ---------------------------------------------------------------- the tests

def _merged(final):
    parts, _ = final
    return [pp for pp, rec in parts.items() if rec[1]]


def test_old_two_part_protocol_blocks_when_two_launches_share_counters():
    # e.g. arrivals A0, B0, A1, B1: A0 writes and raises the flag, B0 merges
    # and lowers it, A1 and B1 then spin for a writer that never comes
    _, blocked = explore(old_two_part, 2, 2)
    assert blocked, "the former protocol should reach a state where every live part spins"


def test_old_two_part_protocol_is_fine_alone():
    finals, blocked = explore(old_two_part, 2, 1)
    assert not blocked and finals


def test_new_two_part_protocol_never_blocks_and_merges_once():
    finals, blocked = explore(new_two_part, 2, 1)
    assert not blocked and finals
    for final in finals:
        parts, mem = final
        merged = _merged(final)
        assert len(merged) == 1
        other = [pp for pp in parts if pp not in merged][0]
        assert other in parts[merged[0]][2]        # the merger reads a written state
        assert mem[0] == 0 and mem[1] == 0         # counters back at zero


def test_new_two_part_protocol_usually_writes_once():
    """Both parts write only when the second arrives while the first is
    still writing; in the other orders one state is written."""
    finals, _ = explore(new_two_part, 2, 1)
    assert {len(mem[2]) for _, mem in finals} == {1, 2}


def test_new_protocols_never_block_with_overlapping_launches():
    for step, n in ((new_two_part, 2), (count_in(2), 2), (count_in(3), 3)):
        finals, blocked = explore(step, n, 2)
        assert not blocked, step
        assert finals and all(len(parts) == 2 * n for parts, _ in finals)


def test_count_in_merges_once_with_every_state():
    for n in (2, 3, 4):
        finals, blocked = explore(count_in(n), n, 1)
        assert not blocked
        for final in finals:
            parts, mem = final
            merged = _merged(final)
            assert len(merged) == 1
            assert parts[merged[0]][2] == {(0, p) for p in range(n)}
            assert mem[0] == 0


def test_planted_mistake_is_caught():
    """A count-in variant that counts itself in before writing lets the
    merger miss a state: the model must notice (so the checks above mean
    something)."""
    def early_count(pc, me, mem):
        c0, c1, written = mem
        if pc == 0:
            return (1 if c0 != 1 else 2), (c0 + 1, c1, written)
        if pc == 1:
            return ("done", False, None), (c0, c1, written | {me})
        if pc == 2:
            return ("done", True, written), (0, c1, written | {me})
        raise AssertionError(pc)
    finals, _ = explore(early_count, 2, 1)
    assert any(len(parts[m][2]) < 2 for parts, _ in finals for m in _merged((parts, _)))
