"""Debug mode (kandle_amd.debug, kh_set_debug): launches synchronise and a kernel whose output holds a
NaN or Inf raises, naming the kernel; healthy kernels run unchanged; disable() restores the plain
kernels.  (No test faults the device on purpose: the synchronous error path is exercised by every
healthy launch returning KH_OK.)"""
import numpy as np
import pytest

import oracle
from helpers import seeded
from kandle_amd import KandleHipError, Tensor
from kandle_amd import debug
from kandle_amd import functional as F

pytestmark = pytest.mark.gpu


def test_debug_mode_flags_non_finite_outputs(hip):
    q, qh = seeded(80, (1, 4, 64, 128), "bfloat16")
    k, kh = seeded(81, (1, 2, 64, 128), "bfloat16")
    v, vh = seeded(82, (1, 2, 64, 128), "bfloat16")
    debug.enable()
    try:
        o = F.scaled_dot_product_attention(q, k, v, is_causal=True).numpy()   # healthy: passes the scan
        assert np.max(np.abs(o - oracle.sdpa(qh, kh, vh, causal=True))) < 2e-2
        bad = vh.copy()
        bad[0, 1, 5, 7] = np.nan
        vb = Tensor(bad, dtype="bfloat16")
        with pytest.raises(KandleHipError, match="flash_attention.*non-finite"):
            F.scaled_dot_product_attention(q, k, vb, is_causal=True)
        x = Tensor(np.array([[1.0, np.inf]], np.float32))
        with pytest.raises(KandleHipError, match="non-finite"):
            F.rms_norm(x, [2], None, 1e-6)
    finally:
        debug.disable()
    # off again: the same NaN input flows through without a check
    vb2 = Tensor(bad, dtype="bfloat16")
    out = F.scaled_dot_product_attention(q, k, vb2, is_causal=True).numpy()
    assert np.isnan(out).any()
