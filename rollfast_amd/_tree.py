"""Minimal pytree utilities with JAX's flattening rules.

The reference (rollfast) walks parameter and state trees with
``jax.tree.flatten`` / ``jax.tree.map`` and an ``is_leaf`` predicate
(``src/rollfast/optim/adam8.py:584``, ``:644``; ``src/rollfast/utils.py:679``).
Leaf order decides which PRNG subkey each leaf receives, so this module
reproduces JAX's order exactly:

* ``dict``: children in sorted key order (``OrderedDict``: insertion order);
* ``list`` / ``tuple``: in order; ``NamedTuple``: in field order;
* ``None``: a node with no children (so not a leaf) unless ``is_leaf``
  says otherwise;
* registered node classes (``register_node``): their ``tree_flatten``;
* anything else is a leaf.
"""

from __future__ import annotations

from collections import OrderedDict
from typing import Any, Callable, Optional

_NODES: dict[type, tuple[Callable, Callable]] = {}


def register_node(cls, flatten: Callable, unflatten: Callable) -> None:
    """Register ``cls`` as an internal node: ``flatten(x) -> (children, aux)``,
    ``unflatten(aux, children) -> x``."""
    _NODES[cls] = (flatten, unflatten)
    _TYPE_KIND.pop(cls, None)


class TreeDef:
    __slots__ = ("kind", "aux", "children", "num_leaves")

    def __init__(self, kind, aux=None, children=()):
        self.kind = kind
        self.aux = aux
        self.children = tuple(children)
        self.num_leaves = 1 if kind == "leaf" else sum(c.num_leaves for c in self.children)

    def __eq__(self, other):
        return self is other or (
            isinstance(other, TreeDef)
            and self.kind == other.kind
            and self.num_leaves == other.num_leaves
            and self.aux == other.aux
            and self.children == other.children
        )

    def __hash__(self):
        return hash((self.kind, repr(self.aux), self.children))

    def __repr__(self):
        if self.kind == "leaf":
            return "*"
        return f"{self.kind}({self.aux!r}, {list(self.children)!r})"


_LEAF = TreeDef("leaf")

# Node classification per concrete type (computed once per type): "leaf",
# "none", "custom", "dict", "odict", "namedtuple", "tuple", "list".
_TYPE_KIND: dict[type, str] = {type(None): "none"}


def _type_kind(t: type) -> str:
    k = _TYPE_KIND.get(t)
    if k is None:
        if t in _NODES:
            k = "custom"
        elif issubclass(t, OrderedDict):
            k = "odict"
        elif issubclass(t, dict):
            k = "dict"
        elif issubclass(t, tuple) and hasattr(t, "_fields"):
            k = "namedtuple"
        elif issubclass(t, tuple):
            k = "tuple"
        elif issubclass(t, list):
            k = "list"
        else:
            k = "leaf"
        _TYPE_KIND[t] = k
    return k


def _children(x):
    """(kind, aux, children) of an internal node, or None for a leaf."""
    t = type(x)
    k = _TYPE_KIND.get(t) or _type_kind(t)
    if k == "leaf":
        return None
    if k == "none":
        return ("none", None, [])
    if k == "dict":
        keys = sorted(x.keys())
        return ("dict", (t, tuple(keys)), [x[key] for key in keys])
    if k == "odict":
        keys = tuple(x.keys())
        return ("odict", (t, keys), [x[key] for key in keys])
    if k == "custom":
        children, aux = _NODES[t][0](x)
        return ("custom", (t, aux), list(children))
    if k == "namedtuple":
        return ("namedtuple", t, list(x))
    if k == "tuple":
        return ("tuple", None, list(x))
    return ("list", None, list(x))


# The walks below are module-level functions that take their accumulator as
# an argument.  A nested function that calls itself is a reference cycle
# (the function, its closure cell, the function again) holding everything it
# closes over -- here the leaves, often device tensors -- until the cyclic
# garbage collector runs; a caller's update tree would then outlive its last
# reference by an unpredictable number of steps.


def _flatten_rec(x, is_leaf, leaves_: list):
    if is_leaf is not None and is_leaf(x):
        leaves_.append(x)
        return _LEAF
    node = _children(x)
    if node is None:
        leaves_.append(x)
        return _LEAF
    kind, aux, children = node
    return TreeDef(kind, aux, [_flatten_rec(c, is_leaf, leaves_) for c in children])


def flatten(tree, is_leaf: Optional[Callable[[Any], bool]] = None):
    """Return ``(leaves, treedef)``."""
    leaves_: list = []
    td = _flatten_rec(tree, is_leaf, leaves_)
    return leaves_, td


def leaves(tree, is_leaf=None) -> list:
    return flatten(tree, is_leaf)[0]


def _build(td: TreeDef, children):
    if td.kind == "none":
        return None
    if td.kind == "dict":
        cls, keys = td.aux
        d = dict(zip(keys, children))
        return d if cls is dict else cls(d)
    if td.kind == "odict":
        cls, keys = td.aux
        return cls(zip(keys, children))
    if td.kind == "namedtuple":
        return td.aux(*children)
    if td.kind == "tuple":
        return tuple(children)
    if td.kind == "list":
        return list(children)
    if td.kind == "custom":
        cls, aux = td.aux
        return _NODES[cls][1](aux, children)
    raise ValueError(f"unknown node kind {td.kind!r}")


def _unflatten_rec(t: TreeDef, it):
    if t.kind == "leaf":
        return next(it)
    return _build(t, [_unflatten_rec(c, it) for c in t.children])


def unflatten(td: TreeDef, leaves_) -> Any:
    it = iter(leaves_)
    out = _unflatten_rec(td, it)
    rest = list(it)
    if rest:
        raise ValueError(f"too many leaves for the tree structure ({len(rest)} left over)")
    return out


def _flatten_up_to_rec(t: TreeDef, x, out: list) -> None:
    if t.kind == "leaf":
        out.append(x)
        return
    node = _children(x)
    if node is None:
        raise ValueError(f"tree structure mismatch: expected a {t.kind} node, got a leaf {type(x)}")
    kind, aux, children = node
    if kind != t.kind or len(children) != len(t.children):
        raise ValueError(f"tree structure mismatch: {t.kind} vs {kind}")
    if kind in ("dict", "odict") and aux[1] != t.aux[1]:
        raise ValueError(f"dict keys differ: {t.aux[1]} vs {aux[1]}")
    for ct, cx in zip(t.children, children):
        _flatten_up_to_rec(ct, cx, out)


def flatten_up_to(td: TreeDef, tree) -> list:
    """Subtrees of ``tree`` at the leaf positions of ``td`` (``td`` must be a
    prefix of ``tree``'s structure), as ``jax`` does for ``tree.map`` rests."""
    out: list = []
    _flatten_up_to_rec(td, tree, out)
    return out


def tree_map(fn: Callable, tree, *rest, is_leaf=None):
    """``jax.tree.map``: ``tree`` gives the structure, ``rest`` are flattened up
    to it."""
    leaves_, td = flatten(tree, is_leaf)
    others = [flatten_up_to(td, r) for r in rest]
    return unflatten(td, [fn(*xs) for xs in zip(leaves_, *others)])
