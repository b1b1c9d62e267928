"""Process-exit teardown of the HIP objects this package creates (GPU).

streams.teardown() -- registered with atexit when the first dedicated
stream or captured graph appears -- drains the device, drops every
BlockStep's captured graph and workspaces, and destroys the dedicated
streams, so none is left to the runtime's static destruction.  Checked in
process: after a graph-replayed engine run, teardown empties both
registries, is idempotent, and a new engine afterwards works.
"""
from __future__ import annotations

import atexit

import pytest
import torch

from d3d_amd import streams
from d3d_amd.engine import Engine
from d3d_amd.model import ModelShape

pytestmark = pytest.mark.gpu

TARGET = ModelShape(layers=1, hidden=256, heads=8, kv_heads=2, head_dim=128, mlp=512, vocab=1000)
DRAFT = ModelShape(layers=1, hidden=256, heads=4, kv_heads=2, head_dim=128, mlp=256, vocab=1000)


def _run(seed):
    eng = Engine(TARGET, DRAFT, pages=8, seed=seed, mask_id=999)
    prompts = torch.randint(0, 999, (2, 20), generator=torch.Generator().manual_seed(seed)).tolist()
    res = eng.generate(prompts, 2, max_new_tokens=8, ignore_eos=True)
    return eng, [o["tokens"] for o in res["outputs"]]


def test_teardown_releases_graphs_and_streams():
    eng, first = _run(31)
    steps = list(eng.target._steps.values()) + list(eng.draft._steps.values())
    assert steps and all(s.graph is not None for s in steps)
    assert len(streams._streams) >= 2 and len(streams._graph_owners) >= len(steps)
    del eng
    streams.teardown()
    assert streams._streams == [] and len(streams._graph_owners) == 0
    assert all(s.graph is None and s.out is None and not s.workspaces for s in steps)
    streams.teardown()  # idempotent
    eng2, again = _run(31)  # new streams, new captures
    assert again == first
    del eng2
    streams.teardown()


def test_teardown_is_registered_at_exit():
    # atexit keeps no public registry; unregister returns silently whether or
    # not the function was there, so re-register to leave the state as found.
    assert streams._hook_registered
    atexit.unregister(streams.teardown)
    atexit.register(streams.teardown)
