"""CPU tests of the host side: the C-ABI library loads and exports every declared symbol, dtype
conversions, the registry/backend surface and view arithmetic.  No compute calls (no GPU here)."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

import oracle
from kandle_amd import _lib, dtypes, kernels
from kandle_amd.registry import SimpleOperatorRegistry
from kandle_amd.tensor import _coalesce, contiguous_strides

ROOT = Path(__file__).resolve().parent.parent


def declared_symbols():
    text = (ROOT / "include" / "kandle_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kh_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    if not _lib.LIB_PATH.exists():
        from kandle_amd.build import build_library

        build_library(verbose=False)
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    syms = declared_symbols()
    assert len(syms) >= 25
    missing = [s for s in syms if not hasattr(lib, s)]
    assert not missing, missing
    # every declared entry point has a ctypes signature in the binding (kh_last_error is special)
    assert set(syms) - {"kh_last_error"} == set(_lib.SIGNATURES)


def test_no_device_means_loud_errors():
    lib = _lib.load()
    n = ctypes.c_int(-1)
    assert lib.kh_device_count(ctypes.byref(n)) == 0
    if n.value == 0:
        assert lib.kh_init(0) != 0
        assert b"not available" in lib.kh_last_error()
        p = ctypes.c_void_p()
        assert lib.kh_alloc(ctypes.byref(p), 16) == 3  # KH_ERR_NOT_INIT
        with pytest.raises(_lib.KandleHipError):
            _lib.init_check()


def test_bf16_conversion_matches_oracle_all_patterns():
    allb = np.arange(65536, dtype=np.uint16)
    f = dtypes.bf16_bits_to_f32(allb)
    np.testing.assert_array_equal(f.view(np.uint32), oracle.from_bf16_bits(allb).view(np.uint32))
    r = np.random.default_rng(0)
    x = np.concatenate([r.standard_normal(100000).astype(np.float32) * 10.0 ** r.integers(-30, 30, 100000),
                        np.array([np.inf, -np.inf, 0.0, -0.0, 1 + 2 ** -8, 65504.0], np.float32)]).astype(np.float32)
    np.testing.assert_array_equal(dtypes.f32_to_bf16_bits(x), oracle.to_bf16_bits(x))


def test_registry_and_kernel_names():
    reg = SimpleOperatorRegistry()
    assert not reg.has("flash_attention") and reg.find("flash_attention") is None
    for name, fn in kernels.KERNELS.items():
        reg.register(name, fn)
    for name in ("flash_attention", "matmul", "rms_norm", "silu", "mul", "add", "copy", "contiguous",
                 "index_select", "argmax", "rms_norm_rope", "silu_mul", "decode_attention"):
        assert reg.has(name), name


def test_view_helpers():
    assert contiguous_strides([2, 3, 4]) == [12, 4, 1]
    # a [B, H, S, D] view of a [B, S, H, D] buffer does not coalesce; a contiguous one does
    assert _coalesce([2, 3, 4], [12, 4, 1]) == ([24], [1])
    assert _coalesce([2, 4, 3, 8], [96, 8, 32, 1]) == ([2, 4, 3, 8], [96, 8, 32, 1])
    assert _coalesce([1, 5, 1, 8], [40, 8, 8, 1]) == ([40], [1])


def test_mask_strides_follow_numpy_broadcasting():
    """The explicit-mask route broadcasts attn_mask to the [B, Hq, Lq, Lk] scores by element
    strides (0 for a broadcast axis), and rejects shapes that do not broadcast, as add_Tensor does
    (packages/core/src/dispatch/handlers/composite.ts:279-300)."""
    from types import SimpleNamespace as NS
    tgt = (2, 4, 5, 7)
    ms = kernels._mask_strides
    assert ms(NS(shape=(5, 7), strides=(7, 1)), tgt) == [0, 0, 7, 1]
    assert ms(NS(shape=(2, 1, 5, 7), strides=(35, 35, 7, 1)), tgt) == [35, 0, 7, 1]
    assert ms(NS(shape=(2, 4, 5, 7), strides=(140, 35, 7, 1)), tgt) == [140, 35, 7, 1]
    assert ms(NS(shape=(1, 7), strides=(7, 1)), tgt) == [0, 0, 0, 1]          # one row for all queries
    assert ms(NS(shape=(7, 5), strides=(1, 7)), (1, 1, 7, 5)) == [0, 0, 1, 7]  # transposed view
    assert ms(NS(shape=(1, 1, 1, 1), strides=(1, 1, 1, 1)), (1, 1, 1, 1)) == [0, 0, 0, 0]
    for bad in ((3, 7), (5, 6), (3, 1, 5, 7), (1, 1, 2, 5, 7)):
        with pytest.raises(ValueError):
            ms(NS(shape=bad, strides=(1,) * len(bad)), tgt)


def test_generic_kernel_names_registered():
    """Kandle's composite RoPE and factories look these up by name (rope.ts:546-644)."""
    for name in ("neg", "cos", "sin", "arange", "sdpa_masked", "copy", "copy_", "add", "mul", "index_select",
                 "argmax", "zeros", "cast", "contiguous"):
        assert name in kernels.KERNELS, name
