"""Graph captures run with Python's cyclic garbage collector off.

A collection that starts in the middle of a HIP graph capture runs the
finalizers of unreachable objects (an earlier step's graph, events, pinned
buffers), whose HIP calls are not allowed while a stream captures; an error
in a finalizer aborts the process.  CPU only: the context managers every
capture in the package, the bench and the tests enters."""
import gc

import pytest

from d3d_amd import _lib


@pytest.fixture
def gc_on():
    was = gc.isenabled()
    gc.enable()
    yield
    (gc.enable if was else gc.disable)()


def test_collection_is_paused_inside_and_restored_after(gc_on):
    with _lib.collection_paused():
        assert not gc.isenabled()
        with _lib.collection_paused():  # nested: the outer pause holds
            assert not gc.isenabled()
        assert not gc.isenabled()
    assert gc.isenabled()


def test_a_pause_keeps_a_disabled_collector_disabled(gc_on):
    gc.disable()
    with _lib.collection_paused():
        assert not gc.isenabled()
    assert not gc.isenabled()


def test_capture_workspaces_pause_collection_and_restore_on_error(gc_on):
    owner = []
    with pytest.raises(KeyError):
        with _lib.capture_workspaces(owner) as got:
            assert got is owner and not gc.isenabled()
            assert _lib._capture_owner is owner
            raise KeyError("inside the capture")
    assert gc.isenabled() and _lib._capture_owner is None
