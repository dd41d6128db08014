"""CPU: the early exit of the ping-pong kernel's unchecked run (csrc/flash_fwd.hip,
flash_fwd_pingpong16: the chunked loop over steps of three unchecked tiles and the pp_flags
slots).

Phases are the intervals between workgroup barriers, numbered by the barriers passed. Group 0
(waves 0-3) runs the softmax phase S_t of steady tile t in phase 2t + 1 and its matrix phase M_t
in 2t + 2; group 1 (waves 4-7) runs each one phase later. The unchecked run starts at tile 1 and
goes in steps of three tiles, in chunks of 1, 2, 4, ... steps, at most `cap` steps (the
kernel's FA_PP16_EXIT_STEPS): chunk c starts at step start_c, tile jj = 1 + 3 start_c. At that
boundary (the phase of S_jj) every wave first reads flag (c - 1) % 2 (from the second boundary
on) and leaves the run if it is set, then sets flag c % 2 if its row sums are no longer finite.
An LDS write completes before its wave's next barrier, so a read in a later phase sees it; a
read in the same phase as a write to the same slot could see either value (a race that could
split the workgroup between leaving and staying, and hang it at the next barrier). All eight
waves must take part: the kernel sets no flag where some wave skips the run (a causal wave
that starts past the end of the sequence has no active tile and spends the run in the
idle-tile loop; leaving without it would put its refills and barriers into the second pass --
a planted mistake below).

This model replays every wave's reads and writes for a sample of overflow patterns and
checks: no read shares a phase with a write to its slot; all eight waves read the same values
and so leave at the same boundary, i.e. after the same number of barriers (group 0 then adds
its one closing barrier, as after a full run); and a wave that overflows by step b makes the
workgroup leave at the second boundary from b on (the one after the boundary that sees it).
The first tile's wide-spread vote (pp_flags[3]) is checked the same way at the end: every wave
reads it after every write, so all of them run the item checked or none does.
"""

from __future__ import annotations

import random

import pytest

WAVES = 8


def _group(w: int) -> int:
    return w // 4


def chunk_starts(n_steps: int, cap: int) -> list[int]:
    """First step of every chunk: chunks of 1, 2, 4, ... steps, at most cap."""
    starts, step, size = [], 0, 1
    while step < n_steps:
        starts.append(step)
        step += size
        size = min(2 * size, cap)
    return starts


def boundary_phase(g: int, start: int) -> int:
    jj = 1 + 3 * start
    return 2 * jj + 1 + g


def simulate(n_steps: int, cap: int, bad_at: list, read_slot=lambda c: (c - 1) % 2,
             write_slot=lambda c: c % 2, idle=()) -> int | None:
    """Replay the run for overflow onsets bad_at[w] (the first step by whose head wave w's row
    sums are not finite, or None). Returns the step at which the waves leave, or None if they
    complete all n_steps. Raises AssertionError on a race or on waves that leave apart."""
    starts = chunk_starts(n_steps, cap)
    events: dict[int, list] = {}  # phase -> [(wave, chunk)]
    for w in range(WAVES):
        if w in idle:  # no step, no flag: such a wave stays for the whole run
            continue
        for c, st in enumerate(starts):
            events.setdefault(boundary_phase(_group(w), st), []).append((w, c))
    writes: dict[int, list[int]] = {}  # slot -> phases of its writes
    left = [None] * WAVES  # step at which the wave left the run
    for ph in sorted(events):
        now = [(w, c) for w, c in sorted(events[ph]) if left[w] is None]
        reads = [(w, c, read_slot(c)) for w, c in now if c > 0]  # none at the first boundary
        new_writes = [(w, c, write_slot(c)) for w, c in now
                      if bad_at[w] is not None and starts[c] >= bad_at[w]]
        for w, c, slot in reads:
            assert all(ws != slot for _, _, ws in new_writes), ("read and write of a slot in "
                                                                "one phase", c, w)
            assert ph not in writes.get(slot, []), ("read and write of a slot in one phase", c, w)
            if any(p < ph for p in writes.get(slot, [])):
                left[w] = starts[c]
        for w, c, slot in new_writes:
            if left[w] is None:
                writes.setdefault(slot, []).append(ph)
    assert len(set(left)) == 1, ("waves leave at different steps", left)
    return left[0]


def _patterns(n_steps: int, count: int, seed: int):
    rng = random.Random(seed)
    yield [None] * WAVES
    for _ in range(count):
        waves = rng.sample(range(WAVES), rng.randint(1, WAVES))
        yield [rng.randrange(n_steps) if w in waves else None for w in range(WAVES)]


@pytest.mark.parametrize("cap", [1, 2, 8, 16, 32])
@pytest.mark.parametrize("n_steps", [1, 3, 7, 20, 42, 170])
def test_waves_leave_together_and_promptly(n_steps, cap):
    starts = chunk_starts(n_steps, cap)
    for bad_at in _patterns(n_steps, 300, seed=31 * n_steps + cap):
        exit_step = simulate(n_steps, cap, bad_at)
        onsets = [b for b in bad_at if b is not None]
        if not onsets:
            assert exit_step is None
            continue
        # the first boundary at or after the onset writes, the next one reads and leaves
        seen = [c for c, st in enumerate(starts) if st >= min(onsets)]
        leave = starts[seen[0] + 1] if seen and seen[0] + 1 < len(starts) else None
        assert exit_step == leave, (bad_at, exit_step)


def test_schedule_and_phases_match_the_kernel():
    """Chunks of 1, 2, 4, ... steps up to the cap; group 0 runs S_t in phase 2t + 1, group 1
    one phase later, and chunk c's boundary is the phase of the softmax phase of tile
    1 + 3 start_c."""
    assert chunk_starts(170, 16) == [0, 1, 3, 7, 15, 31, 47, 63, 79, 95, 111, 127, 143, 159]
    assert chunk_starts(42, 16) == [0, 1, 3, 7, 15, 31]
    assert boundary_phase(0, 0) == 3 and boundary_phase(1, 0) == 4    # S_1
    assert boundary_phase(0, 3) == 21 and boundary_phase(1, 3) == 22  # S_10


@pytest.mark.parametrize("mistake", ["one slot", "read the slot being written",
                                     "a wave past the end of the sequence left out"])
def test_model_catches_a_broken_protocol(mistake):
    """Planted mistakes must be caught as a race or a split decision: one slot for all chunks
    (read and written at every boundary); reading the slot this boundary writes; and an exit
    while one wave (past the end of a causal sequence) takes no part in the run."""
    kwargs = {"one slot": dict(read_slot=lambda c: 0, write_slot=lambda c: 0),
              "read the slot being written": dict(read_slot=lambda c: c % 2),
              "a wave past the end of the sequence left out": dict(idle=(7,))}[mistake]
    with pytest.raises(AssertionError):
        for bad_at in _patterns(12, 200, seed=1):
            simulate(12, 2, bad_at, **kwargs)


# ---- the first tile's wide-spread vote (pp_flags[3], FA_PP16_SPREAD) ---------------------------
# A wave that finds a wide row in its item's first steady tile (tile 0, exact) sets the flag in
# that tile's softmax phase S_0 (phase 1 + g); the flag was cleared before the prologue's
# barrier (phase 0). Every wave that ran tile 0 reads it once tile 0 returns, i.e. in the phase of
# its S_1 (3 + g), and runs the item checked if it is set. Waves without an active first tile
# (a causal wave whose rows all precede its first keys) neither vote nor read: their unchecked
# run is empty anyway.


def vote_decisions(voters, read_phase) -> list:
    """Each reading wave's decision for the set of voting waves; asserts that no read shares a
    phase with a write (a race)."""
    writes = [1 + _group(w) for w in voters]
    out = []
    for w in range(WAVES):
        ph = read_phase(_group(w))
        assert ph not in writes, ("read and write of the vote in one phase", w, ph)
        out.append(any(p < ph for p in writes))
    return out


def _subsets():
    for mask in range(1 << WAVES):
        yield {w for w in range(WAVES) if mask >> w & 1}


def test_spread_vote_is_read_alike_by_every_wave():
    """All 256 sets of voting waves: every wave reads after every write (no race), so all eight
    take the same decision, and it is 'checked' exactly when some wave voted."""
    assert boundary_phase(0, 0) - 2 == 1 and boundary_phase(1, 0) - 2 == 2  # S_0 of each group
    for voters in _subsets():
        d = vote_decisions(voters, lambda g: boundary_phase(g, 0))  # the phase of S_1
        assert len(set(d)) == 1 and d[0] == bool(voters), (voters, d)


@pytest.mark.parametrize("mistake", ["read in the voting phase", "read in the first matrix phase"])
def test_vote_model_catches_an_early_read(mistake):
    """Reading the vote in S_0 itself, or in M_0 (the phase of group 1's S_0), races with a
    write: both planted mistakes must be caught."""
    read = {"read in the voting phase": lambda g: 1 + g,
            "read in the first matrix phase": lambda g: 2 + g}[mistake]
    with pytest.raises(AssertionError):
        for voters in _subsets():
            d = vote_decisions(voters, read)
            assert len(set(d)) == 1
