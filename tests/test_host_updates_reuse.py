"""The native host's update-only outputs (``_rfhost.updates_out``): an
earlier call's buffer is written again only when nothing outside the cache
references it -- not the tree the caller still holds, not a leaf taken out
of it, not an alias of its storage -- and the table rows point into the
buffer the returned views use.  CPU tensors: the function only allocates
like the grads and writes pointers, it launches nothing."""

from __future__ import annotations

import ctypes
import gc

import torch

from rollfast_amd import _lib


def _call(host, grads, table, cache):
    names = sorted(grads)
    lg = [grads[k] for k in names]
    lm = [object() for _ in names]
    rows = [(i,) for i in range(len(names))]
    return host.updates_out(grads, lg, lm, rows, ctypes.addressof(table), cache)


def _ptrs(table, n):
    return [table[j].updates for j in range(n)]


def test_updates_buffers_reused_only_when_unreferenced():
    host = _lib.pyhost()
    grads = {"a": torch.zeros(3, 5), "b": torch.zeros(7), "c": torch.zeros(2, 2, 2)}
    n = len(grads)
    table = (_lib.Adam8Leaf * n)()
    for j, k in enumerate(sorted(grads)):
        table[j].size = grads[k].numel()
    cache = []
    t1 = _call(host, grads, table, cache)
    p1 = _ptrs(table, n)
    assert [t1[k].data_ptr() for k in sorted(grads)] == p1
    assert tuple(t1["a"].shape) == (3, 5) and tuple(t1["c"].shape) == (2, 2, 2)
    t2 = _call(host, grads, table, cache)          # t1 still held: a new buffer
    p2 = _ptrs(table, n)
    assert set(p1).isdisjoint(p2)
    del t1
    gc.collect()
    t3 = _call(host, grads, table, cache)          # t1 dropped: its buffer again
    assert _ptrs(table, n) == p1 and [t3[k].data_ptr() for k in sorted(grads)] == p1
    assert len(cache) == 2
    # a leaf taken out of the tree keeps its buffer from reuse
    keep = t2["b"]
    del t2
    gc.collect()
    t4 = _call(host, grads, table, cache)
    p4 = _ptrs(table, n)
    assert set(p4).isdisjoint(p1) and set(p4).isdisjoint(p2)
    del keep, t3
    gc.collect()
    # an alias of the storage (a view of a leaf) keeps it from reuse too
    alias = t4["a"].view(-1)
    del t4
    gc.collect()
    t5 = _call(host, grads, table, cache)
    assert set(_ptrs(table, n)).isdisjoint(p4)
    assert alias.numel() == 15 and len(cache) == 2
    del t5


def test_updates_out_without_cache_allocates_each_call():
    host = _lib.pyhost()
    grads = {"w": torch.zeros(4)}
    table = (_lib.Adam8Leaf * 1)()
    table[0].size = 4
    names = ["w"]
    a = host.updates_out(grads, [grads["w"]], [object()], [(0,)], ctypes.addressof(table))
    pa = table[0].updates
    del a
    gc.collect()
    host.updates_out(grads, [grads["w"]], [object()], [(0,)], ctypes.addressof(table))
    assert len(names) == 1 and isinstance(pa, int)


def test_tree_walks_leave_no_reference_cycles():
    """flatten / unflatten / flatten_up_to hold no leaf past their return: a
    self-calling nested walk would be a reference cycle keeping every leaf
    (an update tree's views) alive until the cyclic collector runs, and the
    output buffer of the next update-only step could not be reused."""
    import weakref

    from rollfast_amd import _tree

    was = gc.isenabled()
    gc.disable()
    try:
        tree = {"a": [torch.zeros(2), torch.zeros(3)], "b": (torch.zeros(1), {"c": torch.zeros(4)})}
        leaves, td = _tree.flatten(tree)
        w_leaf = weakref.ref(leaves[0])
        rebuilt = _tree.unflatten(td, [torch.ones(1) for _ in leaves])
        w_rebuilt = weakref.ref(rebuilt["b"][1]["c"])
        ups = _tree.flatten_up_to(td, rebuilt)
        w_up = weakref.ref(ups[-1])
        del leaves, tree, rebuilt, ups
        assert w_leaf() is None and w_rebuilt() is None and w_up() is None
    finally:
        if was:
            gc.enable()
