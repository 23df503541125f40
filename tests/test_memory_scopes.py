"""tidy / keep (packages/core/src/memory.ts:83-119, :190-193, :219-260) on the host: which tensors a
scope disposes, what moves to the enclosing scope, and failure handling.  Tensors wrap a stub
handle here (no device memory); tests/test_gpu_support.py runs the same contract on the device."""
import pytest

from kandle_amd import Tensor, is_in_tidy_scope, keep, tidy
from kandle_amd.memory import scope


class _Handle:
    def __init__(self):
        self.disposed = False

    def dispose(self):
        self.disposed = True

    @property
    def is_disposed(self):
        return self.disposed


def _t():
    return Tensor(handle=_Handle())


def test_tidy_disposes_intermediates_keeps_returned_and_kept():
    made = {}

    def body():
        made["a"], made["b"], made["k"] = _t(), _t(), keep(_t())
        made["r"] = _t()
        return {"out": [made["r"]], "n": 3}

    res = tidy(body)
    assert res["out"][0] is made["r"] and not made["r"].is_disposed
    assert made["a"].is_disposed and made["b"].is_disposed and not made["k"].is_disposed
    assert not is_in_tidy_scope()


def test_nested_scopes_move_returned_tensors_to_the_parent():
    inner = {}

    def outer():
        x = tidy("inner", lambda: inner.setdefault("t", _t()))
        assert not x.is_disposed
        return None          # the outer scope returns nothing: x is disposed at its end

    tidy("outer", outer)
    assert inner["t"].is_disposed


def test_failure_disposes_everything_and_reraises():
    made = []

    def body():
        made.append(_t())
        raise RuntimeError("boom")

    with pytest.raises(RuntimeError, match="boom"):
        tidy(body)
    assert made[0].is_disposed and not is_in_tidy_scope()


def test_named_tidy_needs_a_function_and_scope_block():
    with pytest.raises(ValueError, match="second argument must be a function"):
        tidy("name")
    with scope():
        a = _t()
        b = keep(_t())
    assert a.is_disposed and not b.is_disposed
    outside = _t()       # no scope: untracked, never disposed implicitly
    assert not outside.is_disposed
