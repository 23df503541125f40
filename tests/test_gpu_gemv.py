"""GPU parity of the one-row projections with fused producers (kh_gemv_fused) and of the two-pass
argmax, against the CPU oracle.

The fused prologues must equal the unfused sequence: rms_norm (or silu*mul) rounded to bf16, then
the linear.  Bars: bf16 outputs within one bf16 rounding plus fp32 accumulation noise; fp32
outputs within 1e-3 of the output scale (the bf16 activation row may differ by one ulp in rare
elements where the fp32 norm lands on a rounding boundary).
"""
import numpy as np
import pytest

import oracle
from helpers import seeded
from kandle_amd import Tensor
from kandle_amd import functional as F
from kandle_amd import synthetic as syn

pytestmark = pytest.mark.gpu


def _close_bf16(y, ref, K):
    err = np.abs(y - ref)
    return bool(np.all(err <= 2 ** -8 * np.abs(ref) + 1e-4 * np.sqrt(K) * 0.02 * 4)), float(err.max())


def _close_f32(y, ref):
    err = float(np.max(np.abs(y - ref)))
    return err <= 1e-3 * max(1.0, float(np.max(np.abs(ref)))), err


@pytest.mark.parametrize("N,K", [(3000, 1024), (37, 200), (1024, 2048), (6144, 1024), (151936, 1024)])
def test_gemv_plain_bf16(hip, N, K):
    x, xh = seeded(300, (1, K), "bfloat16")
    w, wh = seeded(301, (N, K), "bfloat16", std=0.02)
    y = F.linear_fused("none", x, w).numpy()
    ok, err = _close_bf16(y, oracle.linear(xh, wh), K)
    assert ok, err


def test_gemv_rms_norm_prologue_matches_unfused(hip):
    K, N = 1024, 4096
    x, xh = seeded(310, (1, K), std=3.0)                    # fp32 residual row
    nw = oracle.bf16_round(syn.uniform(311, (K,), 0.5, 1.5))
    w, wh = seeded(312, (N, K), "bfloat16", std=0.02)
    y = F.linear_fused("rms_norm", x, w, Tensor(nw, dtype="bfloat16"), 1e-6).numpy()
    h = oracle.bf16_round(oracle.rms_norm(xh, nw, 1e-6))
    ok, err = _close_bf16(y, oracle.linear(h, wh), K)
    assert ok, err


def test_gemv_rms_norm_prologue_fp32_logits(hip):
    """The lm_head form: final norm fused into the vocab projection, fp32 logits."""
    K, N = 1024, 151936
    x, xh = seeded(320, (1, K), std=2.0)
    nw = oracle.bf16_round(syn.uniform(321, (K,), 0.5, 1.5))
    w, wh = seeded(322, (N, K), "bfloat16", std=0.02)
    y = F.linear_fused("rms_norm", x, w, Tensor(nw, dtype="bfloat16"), 1e-6, out_dtype="float32").numpy()
    h = oracle.bf16_round(oracle.rms_norm(xh, nw, 1e-6))
    ok, err = _close_f32(y, oracle.linear(h, wh))
    assert ok, err


def test_gemv_silu_mul_prologue_residual(hip):
    """down_proj form: silu(gate) * up as the input, added into an fp32 residual row in place."""
    I, H = 3072, 1024
    gu, guh = seeded(330, (1, 2 * I), "bfloat16")
    w, wh = seeded(331, (H, I), "bfloat16", std=0.02)
    r, rh = seeded(332, (1, H))
    g, u = F.narrow(gu, 1, 0, I), F.narrow(gu, 1, I, I)
    out = F.linear_fused("silu_mul", g, w, x2=u, residual=r)
    assert out is r
    a = oracle.bf16_round(oracle.silu_mul(guh[:, :I], guh[:, I:]))
    ok, err = _close_f32(r.numpy(), oracle.linear(a, wh) + rh)
    assert ok, err


def test_gemv_strided_weight_rows_ignore_padding(hip):
    """Weight rows with padding past k (ldw > k) filled with NaN: the padding is never used."""
    N, K, LD = 300, 520, 528
    full = np.full((N, LD), np.nan, np.float32)
    wv = syn.bf16(syn.normal(341, (N, K), 0.02))[1]
    full[:, :K] = wv
    wt = Tensor(full, dtype="bfloat16")
    w = F.narrow(wt, 1, 0, K)
    x, xh = seeded(340, (1, K), "bfloat16")
    y = F.linear_fused("none", x, w).numpy()
    assert np.all(np.isfinite(y))
    ok, err = _close_bf16(y, oracle.linear(xh, wv), K)
    assert ok, err


def test_argmax_ties_across_chunks_and_rows(hip):
    """Two-pass argmax: ties in different 4096-column chunks keep the lowest index; a row without
    a candidate above -FLT_MAX gives 0; bf16 rows; more rows than one launch's grid.y when batched."""
    x = syn.normal(350, (4, 151936))
    x[0, 4100] = x[0, 150000] = 1e3
    x[1, 140000] = 1e3
    x[2, :] = -np.inf
    x[3, 77] = np.nan
    a = F.argmax(Tensor(x)).numpy()
    np.testing.assert_array_equal(a, oracle.argmax(x))
    assert a[0] == 4100 and a[1] == 140000 and a[2] == 0
    xb = syn.bf16(syn.normal(351, (3, 9000)))[1]
    ab = F.argmax(Tensor(xb, dtype="bfloat16")).numpy()
    np.testing.assert_array_equal(ab, oracle.argmax(xb))
