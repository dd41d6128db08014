"""CPU: the K/V buffer protocol of the ping-pong kernel (csrc/flash_fwd.hip, flash_fwd_pingpong16).

The kernel's steady state is a sequence of global phases separated by workgroup barriers.
Group 0 runs the softmax phase S_j in phase 2j and the matrix phase M_j in 2j+1; group 1 runs
one phase later (its M_{-1}, phase 0, only issues requests). K_t and V_t live in LDS buffer
t mod 3. S_j reads the K_{j+1} and V_j fragments; in M_j group 0 requests K_{j+3} and V_{j+2},
group 1 requests K_{j+4} and V_{j+3}; at the end of every odd phase each wave waits until at
most its two newest requests are in flight (vmcnt(2)). The prologue leaves K_0, K_1, K_2, V_0
and V_1 resident, and general_tiles16 takes over at tile n_steady after a full wait.

This model replays that schedule for every steady length and checks what the kernel relies on:
each fragment read finds its tile landed, no request is in flight into a buffer some wave reads
in the same phase, two requests for different tiles never overlap in one buffer, and the state
handed to general_tiles16 is the one it expects.
"""

from __future__ import annotations

import pytest


def _requests(group: int, j: int):
    if group == 0:
        return [(("k", (j + 3) % 3), j + 3), (("v", (j + 2) % 3), j + 2)]
    return [(("k", (j + 4) % 3), j + 4), (("v", (j + 3) % 3), j + 3)]


def simulate(n_steady: int) -> dict:
    landed = {("k", 0): 0, ("k", 1): 1, ("k", 2): 2, ("v", 0): 0, ("v", 1): 1}
    pending = {0: [], 1: []}  # per group, in issue order: (phase, buffer, tile)
    for phase in range(2 * n_steady + 1):
        for g in (0, 1):  # requests of M_j, which group g runs in phase 2j + 1 + g
            if (phase - 1 - g) % 2 == 0:
                j = (phase - 1 - g) // 2
                if (g == 0 and 0 <= j < n_steady) or (g == 1 and -1 <= j < n_steady):
                    for buf, tile in _requests(g, j):
                        for gg in (0, 1):
                            for (_, b2, t2) in pending[gg]:
                                assert not (b2 == buf and t2 != tile), (
                                    "two tiles in flight into one buffer", n_steady, phase, buf)
                        pending[g].append((phase, buf, tile))
        for g in (0, 1):  # fragment reads of S_j, which group g runs in phase 2j + g
            if (phase - g) % 2 == 0 and 0 <= (phase - g) // 2 < n_steady:
                j = (phase - g) // 2
                for kind, tile in (("k", j + 1), ("v", j)):
                    buf = (kind, tile % 3)
                    assert landed.get(buf) == tile, ("read before landing", n_steady, phase, g,
                                                     buf, tile, landed.get(buf))
                    for gg in (0, 1):
                        for (_, b2, _) in pending[gg]:
                            assert b2 != buf, ("request in flight into a buffer being read",
                                               n_steady, phase, g, buf)
        if phase % 2 == 1:  # vmcnt(2) at the end of odd phases, then the barrier
            for g in (0, 1):
                for (_, buf, tile) in pending[g][:-2]:
                    landed[buf] = tile
                pending[g] = pending[g][-2:]
    for g in (0, 1):  # general_tiles16 starts with a full wait
        for (_, buf, tile) in pending[g]:
            landed[buf] = tile
    return landed


@pytest.mark.parametrize("n_steady", list(range(1, 40)))
def test_protocol_invariants(n_steady):
    landed = simulate(n_steady)
    # general_tiles16 at j0 = n_steady reads K_{j0+1} and V_{j0}
    assert landed[("k", (n_steady + 1) % 3)] == n_steady + 1
    assert landed[("v", n_steady % 3)] == n_steady


def test_model_catches_a_short_wait():
    """A planted mistake (waiting with vmcnt(4), i.e. one more phase of slack) must fail."""
    def broken(n_steady):
        landed = {("k", 0): 0, ("k", 1): 1, ("k", 2): 2, ("v", 0): 0, ("v", 1): 1}
        pending = []
        for phase in range(2 * n_steady + 1):
            for g in (0, 1):
                if (phase - 1 - g) % 2 == 0:
                    j = (phase - 1 - g) // 2
                    if (g == 0 and 0 <= j < n_steady) or (g == 1 and -1 <= j < n_steady):
                        pending.extend(_requests(g, j))
            for g in (0, 1):
                if (phase - g) % 2 == 0 and 0 <= (phase - g) // 2 < n_steady:
                    j = (phase - g) // 2
                    for kind, tile in (("k", j + 1), ("v", j)):
                        assert landed.get((kind, tile % 3)) == tile
            if phase % 2 == 1:
                for buf, tile in pending[:-8]:
                    landed[buf] = tile
                pending = pending[-8:]

    with pytest.raises(AssertionError):
        for n in range(1, 12):
            broken(n)
