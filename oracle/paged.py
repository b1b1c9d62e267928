"""ORACLE -- test infrastructure only.

Integer restatement of the paged-KV block inputs the reference builds on the
host every step:

* Runner._tables, serving/backend.py:73-76 -- one row per sequence, its page
  list padded with 0 to the table width;
* Runner.forward, serving/backend.py:123-124 -- the slot of logical position
  pos is table[pos // PAGE] * PAGE + pos % PAGE, for pos = start .. start+Q-1;
* context length = start + Q (the block's keys are appended first).

Positions whose page index falls past the table width, or whose page id is
negative, get slot -1 (the KV append skips such tokens); the reference never
forms them because it reserves the pages first.
"""
from __future__ import annotations

from typing import List, Sequence

import numpy as np


def tables(page_lists: Sequence[List[int]], width: int) -> np.ndarray:
    """Page lists padded with 0 to ``width``; a negative id (no page) reads as 0 too."""
    out = np.zeros((len(page_lists), width), np.int32)
    for b, pages in enumerate(page_lists):
        n = min(len(pages), width)
        out[b, :n] = np.maximum(np.asarray(pages[:n], np.int64), 0)
    return out


def block_inputs(page_lists: Sequence[List[int]], starts: Sequence[int], Q: int, page_size: int, width: int):
    """(tables [B, width] int32, slots [B, Q] int64, positions [B, Q] int64, lens [B] int32)."""
    tab = tables(page_lists, width)
    B = len(page_lists)
    pos = np.asarray(starts, np.int64)[:, None] + np.arange(Q, dtype=np.int64)[None, :]
    slots = np.full((B, Q), -1, np.int64)
    for b in range(B):
        for i in range(Q):
            pi = pos[b, i] // page_size
            if 0 <= pos[b, i] and pi < width and pi < len(page_lists[b]) and page_lists[b][pi] >= 0:
                slots[b, i] = page_lists[b][pi] * page_size + pos[b, i] % page_size
    lens = (np.asarray(starts, np.int64) + Q).astype(np.int32)
    return tab, slots, pos, lens
