"""The paged block-input restatement against a brute-force walk of the pages."""
from __future__ import annotations

import numpy as np

from oracle import paged


def _walk(pages, pos, page_size):
    # Physical slots of a sequence's logical positions, built page by page.
    phys = []
    for p in pages:
        phys.extend(p * page_size + o for o in range(page_size))
    return phys[pos] if pos < len(phys) else -1


def test_slots_match_a_page_walk():
    rng = np.random.default_rng(0)
    for page_size in (1, 4, 16, 24):
        lists = [list(rng.permutation(200)[: rng.integers(1, 12)]) for _ in range(5)]
        starts = [int(rng.integers(0, len(l) * page_size)) for l in lists]
        Q = 9
        width = 12
        tab, slots, pos, lens = paged.block_inputs(lists, starts, Q, page_size, width)
        for b, l in enumerate(lists):
            assert list(tab[b, : len(l)]) == l and not tab[b, len(l):].any()
            assert lens[b] == starts[b] + Q
            for i in range(Q):
                assert pos[b, i] == starts[b] + i
                assert slots[b, i] == _walk(l, starts[b] + i, page_size)


def test_width_bound_and_negative_pages():
    tab, slots, _, _ = paged.block_inputs([[3, -1, 5]], [0], 12, 4, 2)
    assert list(tab[0]) == [3, 0]
    assert list(slots[0, :4]) == [12, 13, 14, 15]
    assert (slots[0, 4:] == -1).all()  # page -1, then past the width
