"""Host-side logic of the engine step (CPU): branch specs and acceptance lists."""
from __future__ import annotations

import random

import pytest

from d3d_amd.engine import Engine, branch_specs


def _reference_specs(K, A, current, top):
    """serving/engine.py:98-105 (non-shallow branches), restated."""
    branches = []
    for accepted in range(1, K):
        anchors = [v for v in top[accepted] if v != current[accepted]][:A]
        assert len(anchors) == A
        branches.extend((accepted, a) for a in anchors)
    branches.append((K, None))
    return branches


@pytest.mark.parametrize("A", [1, 2, 3])
def test_branch_specs_follow_engine_predict(A):
    rng = random.Random(A)
    K = 16
    for _ in range(50):
        top = [rng.sample(range(40), A + 1) for _ in range(K)]
        # current agrees with the draft's greedy token at some positions only
        current = [t[0] if rng.random() < 0.5 else rng.randrange(40) for t in top]
        assert branch_specs(K, A, current, top) == _reference_specs(K, A, current, top)
    assert len(branch_specs(K, A, current, top)) == A * (K - 1) + 1


def test_branch_specs_need_enough_alternatives():
    with pytest.raises(RuntimeError):
        branch_specs(3, 2, [1, 2, 3], [[1, 2, 3], [2, 2, 2], [5, 6, 7]])


def test_accepted_lists_follow_engine_accepted():
    """Engine._accepted keeps serving/engine.py:138-145's list semantics."""
    assert Engine._accepted([[5, 1, 2, 9]], [[1, 2, 7, 8]]) == [(3, 7)]
    assert Engine._accepted([[5, 1, 2]], [[1, 2, 4]]) == [(3, 4)]
    assert Engine._accepted([[5, 0, 0]], [[1, 2, 4]]) == [(1, 1)]
