"""The prefill split-K work list, on the CPU (host-side planner, no device work).

Invariants every plan must keep, over a grid of chunk shapes: the items of a
query block partition its causal key range [0, nkt) exactly; no part starts
after the block's first diagonal tile (so every query row sees a key in every
part); partial slots are contiguous per split block, distinct across blocks,
and -1 exactly for unsplit blocks; the item list and the partial buffer stay
within their caps; items go out costliest first under the documented cost
model (int8 tile 1, exact or mixed tile 1.4, workgroup start-up 2.1).
"""
import itertools

import pytest

BQ = BK = 64
MAX_ITEMS = 384
MAX_PARTS = (16 << 20) // (8 * (4 * 16 * 64 * 4 + 4 * 64 * 2))   # partial buffer / (8 kv heads x slot)


def nkt(qt, m, P):
    return (P + min(qt * BQ + BQ, m) + BK - 1) // BK


def exact(P, qt32, kt, near, sink):
    # reference prefill.cu:1381-1382, on 64-key tiles
    return kt * 64 + 64 > P + qt32 * 32 - near or (sink and kt == 0)


def cost(qt, lo, hi, P, near, sink, int8):
    return 2.1 + sum(1.4 if (not int8 or exact(P, 2 * qt, kt, near, sink)) else 1.0 for kt in range(lo, hi))


def check_plan(items, m, P, near, sink, int8):
    nq = (m + BQ - 1) // BQ
    assert len(items) <= MAX_ITEMS
    by_block = {}
    for qt, lo, hi, slot in items:
        assert 0 <= qt < nq
        assert 0 <= lo < hi <= nkt(qt, m, P)
        by_block.setdefault(qt, []).append((lo, hi, slot))
    assert sorted(by_block) == list(range(nq)), "every query block appears"
    used, parts = set(), 0
    for qt, pieces in by_block.items():
        pieces.sort()
        assert pieces[0][0] == 0 and pieces[-1][1] == nkt(qt, m, P)
        for (l0, h0, _), (l1, _, _) in zip(pieces, pieces[1:]):
            assert h0 == l1, "pieces are contiguous"
        if len(pieces) == 1:
            assert pieces[0][2] == -1
            continue
        parts += len(pieces)
        kdiag = (P + qt * BQ) // BK
        assert all(lo <= kdiag for lo, _, _ in pieces), "no part starts past the first diagonal tile"
        slots = [s for _, _, s in pieces]
        assert slots == list(range(slots[0], slots[0] + len(slots))), "slots contiguous, in key order"
        assert not used & set(slots)
        used |= set(slots)
    assert parts <= MAX_PARTS
    costs = [cost(qt, lo, hi, P, near, sink, int8) for qt, lo, hi, _ in items]
    assert all(a >= b - 1e-4 for a, b in zip(costs, costs[1:])), "costliest first"
    return by_block


SHAPES = list(itertools.product([1, 63, 64, 65, 1000, 4096, 8192], [0, 1, 777, 4096, 126976],
                                [0, 256, 1024, 1 << 20], [0, 1], [True, False]))


@pytest.mark.parametrize("m,P,near,sink,int8", SHAPES[::3])
def test_plan_invariants(lk_host, m, P, near, sink, int8):
    items = lk_host.pf_plan_items(m, P, near, sink, int8)
    if items:
        check_plan(items, m, P, near, sink, int8)


def test_c4_chunk_is_split_and_c5_last_chunk_is_not(lk_host):
    items = lk_host.pf_plan_items(4096, 0, 1024, 1, True)
    by_block = check_plan(items, 4096, 0, 1024, 1, True)
    assert any(len(p) > 1 for p in by_block.values())
    # the long blocks are cut, the short ones are whole
    assert len(by_block[63]) > 1 and len(by_block[0]) == 1
    # a chunk deep in the prompt has near-equal blocks: no split
    assert lk_host.pf_plan_items(4096, 126976, 1024, 1, True) == []


def test_override(lk_host):
    try:
        lk_host.pf_split_override(-1)
        assert lk_host.pf_plan_items(4096, 0, 1024, 1, True) == []
        lk_host.pf_split_override(8)
        items = lk_host.pf_plan_items(2048, 0, 0, 0, True)
        by_block = check_plan(sorted(items, key=lambda t: -cost(t[0], t[1], t[2], 0, 0, 0, True)), 2048, 0, 0, 0, True)
        # equal parts of at most 8 tiles (doubled while the partial buffer would overflow)
        sizes = {hi - lo for p in by_block.values() if len(p) > 1 for lo, hi, _ in p}
        assert max(sizes) <= 16
    finally:
        lk_host.pf_split_override(0)


def test_bad_arguments(lk_host):
    with pytest.raises(Exception):
        lk_host.pf_plan_items(0, 0, 0, 0, True)
