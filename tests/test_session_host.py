"""Host logic of the request layer that runs without a GPU: decide's state_boundary
(forward.rs:1503-1515), restated in decide_amd/csrc/session.cpp and reached through the C ABI.

Pinned against the definition itself: one past the first occurrence of the marker inside
ids[prefix:min(limit, len)], computed here by brute force over every window."""

import itertools
import random

import pytest

from decide_amd.forward import STATE_MARKER, state_boundary


def _brute(ids, prefix, marker, limit):
    hay = ids[prefix:min(limit, len(ids))] if prefix <= min(limit, len(ids)) else None
    if hay is None:
        return None
    for i in range(len(hay) - len(marker) + 1):
        if hay[i:i + len(marker)] == marker:
            return prefix + i + len(marker)
    return None


def test_examples():
    m = list(STATE_MARKER)
    ids = [7] * 10 + m + [9] * 5
    assert state_boundary(ids, 3, m, len(ids)) == 14
    assert state_boundary(ids, 3, m, 14) == 14  # the state may end exactly at the limit
    assert state_boundary(ids, 3, m, 13) is None  # but not past it
    assert state_boundary(ids, 11, m, len(ids)) is None  # the marker starts before the search does
    assert state_boundary(ids, 10, m, len(ids)) == 14
    assert state_boundary(ids + m, 3, m, 100) == 14  # the first occurrence
    assert state_boundary(ids, 20, m, 5) is None  # prefix past the limit


@pytest.mark.parametrize("seed", range(4))
def test_matches_brute_force(seed):
    rnd = random.Random(seed)
    for _ in range(300):
        ids = [rnd.randrange(3) for _ in range(rnd.randrange(0, 14))]
        marker = [rnd.randrange(3) for _ in range(rnd.randrange(1, 4))]
        prefix, limit = rnd.randrange(0, 16), rnd.randrange(0, 16)
        assert state_boundary(ids, prefix, marker, limit) == _brute(ids, prefix, marker, limit), (ids, prefix, marker,
                                                                                                 limit)


def test_every_window_position():
    m = [5, 6]
    for n, at in itertools.product(range(2, 9), range(0, 7)):
        if at + 2 > n:
            continue
        ids = [0] * n
        ids[at:at + 2] = m
        assert state_boundary(ids, 0, m, n) == at + 2
