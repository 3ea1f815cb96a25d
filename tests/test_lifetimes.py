"""Lifetimes of the Python objects made from a Context (CPU only: a fake library stands in for
libzwgpu.so and records the calls the bindings make).

A KVCache or Q8Resident holds device memory that belongs to its context.  Closing the context
(explicitly or by `with`) must destroy them first, and a child collected after its context
closed must not call into the library with a freed handle.
"""
from __future__ import annotations

import ctypes
import gc

import numpy as np
import pytest

from zwhisper_amd import _lib, ops


class FakeLib:
    """Enough of the C ABI for Context, KVCache and Q8Resident, with every call logged."""

    def __init__(self):
        self.calls: list[tuple[str, int]] = []
        self.live: set[int] = set()
        self._next = 0x1000

    def _new(self) -> int:
        self._next += 0x10
        self.live.add(self._next)
        return self._next

    @staticmethod
    def _out(ref):
        return ref._obj  # the object ctypes.byref() wraps

    def zwg_open(self, device, lim, out):
        h = self._new()
        self._out(out).value = h
        self.calls.append(("open", h))
        return _lib.ZWG_OK

    def zwg_close(self, h):
        h = h.value if isinstance(h, ctypes.c_void_p) else h
        assert h in self.live, "close of a dead context"
        self.live.discard(h)
        self.calls.append(("close", h))

    def zwg_kv_create(self, ctx, desc, out):
        h = self._new()
        self._out(out).value = h
        self.calls.append(("kv_create", h))
        return _lib.ZWG_OK

    def zwg_kv_get_info(self, h, info):
        return _lib.ZWG_OK

    def zwg_kv_destroy(self, h):
        h = h.value if isinstance(h, ctypes.c_void_p) else h
        assert h in self.live, "destroy of a dead kv cache"
        self.live.discard(h)
        self.calls.append(("kv_destroy", h))

    def zwg_q8w_create(self, ctx, q, sc, n, k, flags, out):
        h = self._new()
        self._out(out).value = h
        self.calls.append(("q8w_create", h))
        return _lib.ZWG_OK

    def zwg_q8w_destroy(self, h):
        assert h in self.live, "destroy of dead int8 weights"
        self.live.discard(h)
        self.calls.append(("q8w_destroy", h))

    def zwg_last_error(self, ctx):
        return b""


@pytest.fixture
def fake(monkeypatch):
    f = FakeLib()
    monkeypatch.setattr(_lib, "_lib", f)
    return f


def _children(ctx):
    kv = ops.KVCache(ctx, 1, 2, 16, 2, 64)
    q = np.zeros((32, 64), np.int8)
    sc = np.ones((32, 2), np.float32)
    w = ops.Q8(q, sc, 32, 64).resident(ctx)
    return kv, w


def test_context_close_destroys_children_first(fake):
    ctx = ops.Context(0)
    kv, w = _children(ctx)
    ctx.close()
    names = [c for c, _ in fake.calls]
    assert names.index("kv_destroy") < names.index("close")
    assert names.index("q8w_destroy") < names.index("close")
    assert not fake.live, "something outlived its context"
    # collecting the children afterwards calls nothing more
    n = len(fake.calls)
    del kv, w
    gc.collect()
    assert len(fake.calls) == n


def test_with_block_then_collect(fake):
    with ops.Context(0) as ctx:
        kv, w = _children(ctx)
    assert not fake.live
    del kv, w, ctx
    gc.collect()
    assert [c for c, _ in fake.calls].count("close") == 1


def test_children_closed_early_are_not_closed_twice(fake):
    ctx = ops.Context(0)
    kv, w = _children(ctx)
    kv.close()
    w.close()
    ctx.close()
    names = [c for c, _ in fake.calls]
    assert names.count("kv_destroy") == 1 and names.count("q8w_destroy") == 1
    assert names[-1] == "close"


def test_closed_context_handle_raises(fake):
    ctx = ops.Context(0)
    ctx.close()
    with pytest.raises(ops.ZwgError):
        _ = ctx.handle
