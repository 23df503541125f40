"""kh_decode_attention_noalloc (the allocation-free variant of kh_decode_attention) against
kh_decode_attention through the C ABI: identical outputs bit for bit (the same kernels on the same
inputs) on two calls in a row, the second smaller; no device allocation during the calls (the
caching allocator's counters do not move); and the size limit rejected with a clear error."""
import ctypes as C

import numpy as np
import pytest

from helpers import seeded
from kandle_amd import HipTensorHandle, Tensor, _lib
from kandle_amd import synthetic as syn

pytestmark = pytest.mark.gpu


def _args(q, kc, vc, o, sl, scale):
    B, Hq, D = q.shape
    _, Hkv, L, _ = kc.shape
    h = lambda t: t.handle if hasattr(t, "handle") else t  # noqa: E731
    strides = _lib.i64_array(list(h(q).strides[:2]) + list(h(kc).strides[:3]) + list(h(vc).strides[:3]) +
                             list(h(o).strides[:2]))
    vp = lambda t: C.c_void_p(h(t).data_ptr())  # noqa: E731
    return (vp(q), vp(kc), vp(vc), vp(o), vp(sl), B, Hq, Hkv, D, L, strides, C.c_float(scale), h(q).kh_dtype)


def _stats():
    s = _lib.AllocStats()
    _lib.call("kh_get_alloc_stats", C.byref(s))
    return s.live_bytes, s.cached_bytes, s.n_device_allocs, s.n_cache_hits


@pytest.mark.parametrize("dtype,D,cases", [
    ("bfloat16", 128, [(8, 16, 8, 32768, 2024), (2, 16, 2, 1500, 7)]),   # the C4 shape, then a smaller call
    ("float32", 128, [(4, 16, 8, 4096, 31), (1, 8, 8, 300, 37)]),
    ("bfloat16", 64, [(4, 16, 4, 5000, 41), (1, 8, 8, 700, 43)]),        # head dim 64: 512-key chunks
    ("float32", 64, [(2, 16, 2, 3000, 47), (1, 4, 4, 200, 53)]),
    ("bfloat16", 128, [(2, 10, 2, 3000, 61), (1, 24, 2, 500, 67)])])      # GQA 5, then 12 (2 groups of 6)
def test_noalloc_decode_matches_allocating_entry_point(hip, dtype, D, cases):
    for B, Hq, Hkv, ML, seed in cases:
        lens = syn.randint(seed, (B,), 1, ML + 1)
        q, _ = seeded(seed + 1, (B, Hq, D), dtype)
        kc, _ = seeded(seed + 2, (B, Hkv, ML, D), dtype)
        vc, _ = seeded(seed + 3, (B, Hkv, ML, D), dtype)
        sl = Tensor(lens, dtype="int32")
        o_ref = HipTensorHandle.create_new((B, Hq, D), dtype)
        o_na = HipTensorHandle.create_new((B, Hq, D), dtype)
        _lib.call("kh_decode_attention", *_args(q, kc, vc, o_ref, sl, 1 / np.sqrt(D)))
        _lib.synchronize()
        before = _stats()
        _lib.call("kh_decode_attention_noalloc", *_args(q, kc, vc, o_na, sl, 1 / np.sqrt(D)))
        _lib.synchronize()
        assert _stats() == before, "the allocation-free entry point touched the caching allocator"
        a, b = o_ref.data_async(), o_na.data_async()
        assert np.all(np.isfinite(a)) and np.array_equal(a.view(np.uint32), b.view(np.uint32)), (dtype, D, B, ML)
        for t in (q, kc, vc, sl):
            t.dispose()
        o_ref.dispose()
        o_na.dispose()


def test_noalloc_decode_rejects_oversize(hip):
    """64 sequences x 32 heads x 65536 keys need 272 MB of partials: rejected before any launch."""
    q, _ = seeded(1, (1, 32, 128), "bfloat16")
    kc, _ = seeded(2, (1, 8, 256, 128), "bfloat16")
    o = HipTensorHandle.create_new((1, 32, 128), "bfloat16")
    sl = Tensor(np.array([1], np.int32), dtype="int32")
    args = list(_args(q, kc, kc, o, sl, 0.1))
    args[5], args[9] = 64, 65536   # batch, max_len
    with pytest.raises(_lib.KandleHipError, match="scratch array"):
        _lib.call("kh_decode_attention_noalloc", *args)
    for t in (q, kc, sl):
        t.dispose()
    o.dispose()
