"""Minimal pytree utilities with JAX's flattening rules.

The reference (rollfast) walks parameter and state trees with
``jax.tree.flatten`` / ``jax.tree.map`` and an ``is_leaf`` predicate
(``src/rollfast/optim/adam8.py:584``, ``:644``; ``src/rollfast/utils.py:679``).
Leaf order decides which PRNG subkey each leaf receives, so this module
reproduces JAX's order exactly:

* ``dict``: children in sorted key order;
* ``list`` / ``tuple``: in order; ``NamedTuple``: in field order;
* ``None``: a node with no children (so not a leaf) unless ``is_leaf``
  says otherwise;
* registered node classes (``register_node``): their ``tree_flatten``;
* anything else is a leaf.
"""

from __future__ import annotations

from typing import Any, Callable, Optional

_NODES: dict[type, tuple[Callable, Callable]] = {}


def register_node(cls, flatten: Callable, unflatten: Callable) -> None:
    """Register ``cls`` as an internal node: ``flatten(x) -> (children, aux)``,
    ``unflatten(aux, children) -> x``."""
    _NODES[cls] = (flatten, unflatten)


def _is_namedtuple(x) -> bool:
    return isinstance(x, tuple) and hasattr(type(x), "_fields")


class TreeDef:
    __slots__ = ("kind", "aux", "children")

    def __init__(self, kind, aux=None, children=()):
        self.kind = kind
        self.aux = aux
        self.children = tuple(children)

    @property
    def num_leaves(self) -> int:
        if self.kind == "leaf":
            return 1
        return sum(c.num_leaves for c in self.children)

    def __eq__(self, other):
        return (
            isinstance(other, TreeDef)
            and self.kind == other.kind
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


def _children(x):
    """(kind, aux, children) of an internal node, or None for a leaf."""
    if x is None:
        return ("none", None, [])
    t = type(x)
    if t in _NODES:
        children, aux = _NODES[t][0](x)
        return ("custom", (t, aux), list(children))
    if isinstance(x, dict):
        keys = sorted(x.keys())
        return ("dict", (type(x), tuple(keys)), [x[k] for k in keys])
    if _is_namedtuple(x):
        return ("namedtuple", type(x), list(x))
    if isinstance(x, tuple):
        return ("tuple", None, list(x))
    if isinstance(x, list):
        return ("list", None, list(x))
    return None


def flatten(tree, is_leaf: Optional[Callable[[Any], bool]] = None):
    """Return ``(leaves, treedef)``."""
    leaves: list = []

    def rec(x):
        if is_leaf is not None and is_leaf(x):
            leaves.append(x)
            return _LEAF
        node = _children(x)
        if node is None:
            leaves.append(x)
            return _LEAF
        kind, aux, children = node
        return TreeDef(kind, aux, [rec(c) for c in children])

    td = rec(tree)
    return leaves, td


def leaves(tree, is_leaf=None) -> list:
    return flatten(tree, is_leaf)[0]


def _build(td: TreeDef, children):
    if td.kind == "none":
        return None
    if td.kind == "dict":
        cls, keys = td.aux
        d = dict(zip(keys, children))
        return d if cls is dict else cls(d)
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


def unflatten(td: TreeDef, leaves_) -> Any:
    it = iter(leaves_)

    def rec(t: TreeDef):
        if t.kind == "leaf":
            return next(it)
        return _build(t, [rec(c) for c in t.children])

    out = rec(td)
    rest = list(it)
    if rest:
        raise ValueError(f"too many leaves for the tree structure ({len(rest)} left over)")
    return out


def flatten_up_to(td: TreeDef, tree) -> list:
    """Subtrees of ``tree`` at the leaf positions of ``td`` (``td`` must be a
    prefix of ``tree``'s structure), as ``jax`` does for ``tree.map`` rests."""
    out: list = []

    def rec(t: TreeDef, x):
        if t.kind == "leaf":
            out.append(x)
            return
        node = _children(x)
        if node is None:
            raise ValueError(f"tree structure mismatch: expected a {t.kind} node, got a leaf {type(x)}")
        kind, aux, children = node
        if kind != t.kind or len(children) != len(t.children):
            raise ValueError(f"tree structure mismatch: {t.kind} vs {kind}")
        if kind == "dict" and aux[1] != t.aux[1]:
            raise ValueError(f"dict keys differ: {t.aux[1]} vs {aux[1]}")
        for ct, cx in zip(t.children, children):
            rec(ct, cx)

    rec(td, tree)
    return out


def tree_map(fn: Callable, tree, *rest, is_leaf=None):
    """``jax.tree.map``: ``tree`` gives the structure, ``rest`` are flattened up
    to it."""
    leaves_, td = flatten(tree, is_leaf)
    others = [flatten_up_to(td, r) for r in rest]
    return unflatten(td, [fn(*xs) for xs in zip(leaves_, *others)])
