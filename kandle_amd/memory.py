"""Scoped lifetime of intermediate tensors: tidy() and keep(), the contract of Kandle's
packages/core/src/memory.ts:83-119 (tidy), :150-182 (tidyAsync), :190-193 (keep), :219-260
(scope end).

Every Tensor created while a tidy scope is active is recorded in that scope.  When the scope ends,
each recorded tensor that is neither returned by the function nor marked with keep() is disposed
(its device storage returns to the caching allocator once no view shares it).  Tensors in the
return value (a Tensor, or Tensors inside lists, tuples and dict values, searched recursively)
move to the enclosing scope, if any, so an outer tidy still owns them.  If the function raises,
every tensor of the scope is disposed and the exception propagates.  The reference's tidyAsync
exists because its forward passes are async; Python's are synchronous, so tidy covers both.
"""
from __future__ import annotations

from contextlib import contextmanager
from typing import Any, Callable, Iterator, List, Optional, TypeVar, Union

T = TypeVar("T")


class _Scope:
    __slots__ = ("name", "tracked")

    def __init__(self, name: str):
        self.name = name
        self.tracked: List[Any] = []


_stack: List[_Scope] = []


def _track(tensor) -> None:
    """Called by Tensor.__init__: records a new tensor in the innermost active scope."""
    if _stack:
        _stack[-1].tracked.append(tensor)
        tensor._scope = _stack[-1]


def is_in_tidy_scope() -> bool:
    return bool(_stack)


def keep(tensor):
    """Marks `tensor` to survive the tidy scope it was created in (and every enclosing one)."""
    tensor._kept = True
    return tensor


def _tensors_in(value, out: list, seen: set) -> list:
    from .tensor import Tensor

    if isinstance(value, Tensor):
        if id(value) not in seen:
            seen.add(id(value))
            out.append(value)
    elif isinstance(value, (list, tuple, set, frozenset)):
        for v in value:
            _tensors_in(v, out, seen)
    elif isinstance(value, dict):
        for v in value.values():
            _tensors_in(v, out, seen)
    return out


def _end(scope: _Scope, result, failed: bool) -> None:
    returned = [] if failed else _tensors_in(result, [], set())
    keep_ids = {id(t) for t in returned}
    popped = _stack.pop()
    assert popped is scope, "tidy scopes ended out of order"
    for t in scope.tracked:
        if getattr(t, "_kept", False) or id(t) in keep_ids or t.is_disposed:
            continue
        t.dispose()
    if _stack:   # returned tensors of this scope now belong to the enclosing one
        parent = _stack[-1]
        for t in returned:
            if not getattr(t, "_kept", False) and getattr(t, "_scope", None) is scope:
                parent.tracked.append(t)
                t._scope = parent


def tidy(name_or_fn: Union[str, Callable[[], T]], fn: Optional[Callable[[], T]] = None) -> T:
    """Runs fn() in a new scope and disposes the tensors it created except those it returns or that
    were kept: tidy(fn) or tidy(name, fn)."""
    if callable(name_or_fn):
        name, func = "unnamed scope", name_or_fn
    else:
        if fn is None:
            raise ValueError("When calling tidy with a name, the second argument must be a function")
        name, func = str(name_or_fn), fn
    scope = _Scope(name)
    _stack.append(scope)
    try:
        result = func()
    except BaseException:
        _end(scope, None, failed=True)
        raise
    _end(scope, result, failed=False)
    return result


@contextmanager
def scope(name: str = "unnamed scope") -> Iterator[None]:
    """`with scope(): ...` -- a tidy scope around a block; nothing is returned from a block, so
    every tensor it creates is disposed at its end unless kept."""
    s = _Scope(name)
    _stack.append(s)
    try:
        yield
    except BaseException:
        _end(s, None, failed=True)
        raise
    _end(s, None, failed=False)
