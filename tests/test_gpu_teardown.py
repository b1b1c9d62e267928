"""Process-exit teardown of the HIP objects this package creates (GPU).

streams._teardown() -- the private hook registered with atexit when the
first dedicated stream or captured graph appears -- drains the devices that
hold them, drops every BlockStep's captured graph and workspaces, drops the
workspaces cached for the dedicated streams and destroys the streams, so
none is left to the runtime's static destruction.  Checked in process, with
no engine left alive (as at exit): after a graph-replayed engine run, the
hook empties every registry, is idempotent, and a new engine afterwards
works.
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
    assert streams._used_devices() == [torch.device("cuda:0").index or 0]
    handles = set(streams._streams)
    del eng
    streams._teardown()
    assert streams._streams == [] and len(streams._graph_owners) == 0 and not streams._pool
    assert all(s.graph is None and s.out is None and not s.workspaces for s in steps)
    from d3d_amd import _lib
    assert not any(k[1] in handles for k in _lib._workspaces)
    streams._teardown()  # idempotent
    eng2, again = _run(31)  # new streams, new captures
    assert again == first
    del eng2
    streams._teardown()


def test_teardown_is_registered_at_exit():
    # atexit keeps no public registry; unregister returns silently whether or
    # not the function was there, so re-register to leave the state as found.
    assert streams._hook_registered
    assert not hasattr(streams, "teardown")
    atexit.unregister(streams._teardown)
    atexit.register(streams._teardown)
