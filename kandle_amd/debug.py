"""Debug mode of the HIP backend: synchronous launches and a NaN/Inf scan of every kernel's output.

enable() sets the library's debug flag (kh_set_debug: each entry point waits for its kernels and
reports a device fault at the call that launched it) and wraps every kernel registered on the
backend so that, after it returns, its floating-point outputs are copied to the host and checked
for NaN/Inf; the first kernel producing one raises KandleHipError naming it.  disable() restores
both.  It costs a synchronisation and a readback per kernel: a debugging aid, not for timing.
Kernels recorded into a HIP graph (generate(use_graph=True)) are not scanned: while the capture is
open they have not run, and a replay launches the whole graph without calling the host wrappers.
The reference proposes the same per-dispatch check (knownIssues/shader.md:151-175); its kernels
run asynchronously on WebGPU and a fault or a NaN surfaces only at the next readback.
"""
from __future__ import annotations

from typing import Callable, Dict, Optional

import numpy as np

from . import _lib
from .dtypes import BFLOAT16, FLOAT32
from .tensor import HipTensorHandle

_saved: Dict[str, Callable] = {}
_state = {"backend": None, "check_finite": True}


def _outputs(name: str, args, kwargs, ret):
    """The tensor handles a kernel wrote, by its registered signature."""
    outs = []
    if isinstance(ret, HipTensorHandle):
        outs.append(ret)
    elif isinstance(ret, (tuple, list)):
        outs += [r for r in ret if isinstance(r, HipTensorHandle)]
    if name in ("matmul", "mm", "bmm", "addmm", "baddbmm") and args:
        outs.append(args[0].output)
    elif args and hasattr(args[0], "output") and callable(getattr(args[0], "output")):   # TensorIterator ops
        outs.append(args[0].output())
    elif name in ("flash_attention", "sdpa_masked", "index_select", "linear_swiglu", "silu_mul", "gemv_fused"):
        pos = {"flash_attention": 3, "sdpa_masked": 4, "index_select": 3, "linear_swiglu": 2, "silu_mul": 2,
               "gemv_fused": 3}[name]
        if len(args) > pos and isinstance(args[pos], HipTensorHandle):
            outs.append(args[pos])
    elif name == "decode_attention" and len(args) > 4:
        outs.append(args[4])
    elif name in ("rms_norm",) and len(args) > 1 and isinstance(args[1], dict) and args[1].get("out") is not None:
        outs.append(args[1]["out"])
    return [o for o in outs if isinstance(o, HipTensorHandle) and o.dtype in (FLOAT32, BFLOAT16)
            and not o.is_disposed]


def _wrap(name: str, fn: Callable) -> Callable:
    def checked(*args, **kwargs):
        ret = fn(*args, **kwargs)
        # under graph capture the kernels are only recorded: nothing has run and the runtime
        # refuses the readback, so the scan is skipped (replays are not scanned)
        if _state["check_finite"] and not _lib.is_capturing():
            for o in _outputs(name, args, kwargs, ret):
                vals = o.data_async()
                if not np.all(np.isfinite(vals)):
                    bad = int(np.size(vals) - np.count_nonzero(np.isfinite(vals)))
                    raise _lib.KandleHipError(
                        f"debug: kernel {name!r} wrote {bad} non-finite value(s) into its {tuple(o.shape)} output")
        return ret
    checked.__wrapped__ = fn
    return checked


def enable(backend=None, check_finite: bool = True) -> None:
    """Turns debug mode on for `backend` (default: the registered hip backend)."""
    from . import env

    b = backend or env.get_backend("hip")
    _lib.call("kh_set_debug", 1)
    _state["check_finite"] = check_finite
    if _state["backend"] is b:
        return
    disable()
    _state["backend"] = b
    reg = b.operators
    for name in list(reg.names()):
        fn = reg.find(name)
        _saved[name] = fn
        reg.register(name, _wrap(name, fn))


def disable() -> None:
    """Turns debug mode off and restores the unwrapped kernels."""
    b: Optional[object] = _state["backend"]
    if _lib.is_initialized():
        _lib.call("kh_set_debug", 0)
    if b is not None:
        for name, fn in _saved.items():
            b.operators.register(name, fn)
    _saved.clear()
    _state["backend"] = None
