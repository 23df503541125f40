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


def test_debug_mode_with_graph_capture(hip):
    """Debug mode with generate(use_graph=True): the kernels recorded while the prefill and decode
    graphs are captured are not scanned (they have not run; the runtime refuses a readback into a
    capturing stream), and the tokens and logits equal those of an eager generation with debug mode
    off."""
    from kandle_amd import synthetic as syn
    from kandle_amd.model_utils import Qwen3Config, Qwen3ForCausalLM, init_qwen3_weights

    cfg = Qwen3Config(vocab_size=4096, num_hidden_layers=2)
    w = init_qwen3_weights(cfg, seed=5)
    prompt = syn.randint(6, (24,), 0, cfg.vocab_size)
    model = Qwen3ForCausalLM(cfg, w, max_seq_len=48)
    try:
        debug.enable()
        try:
            toks, log = model.generate(prompt, 4, return_logits=True, use_graph=True)   # captures both graphs
        finally:
            debug.disable()
        ref_toks, ref_log = model.generate(prompt, 4, return_logits=True, use_graph=False)
    finally:
        model.dispose()
    assert toks == ref_toks
    for a, b in zip(log, ref_log):
        assert np.array_equal(a, b)
