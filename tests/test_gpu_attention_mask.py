"""GPU parity of scaled_dot_product_attention with an explicit additive attn_mask against the CPU
oracle (oracle.sdpa_masked, the reference's matmul -> add -> softmax -> matmul route of
packages/core/src/dispatch/handlers/composite.ts:279-300).

Tolerances: bf16 inputs with fp32 accumulation within 2e-2 absolute on the outputs; fp32 within
1e-4 relative (max-abs error over max-abs value).  Rows whose every score is -inf are NaN in the
reference softmax (0 / 0) and must be NaN here.
"""
import numpy as np
import pytest

import oracle
from helpers import dev, max_rel, seeded
from kandle_amd import functional as F
from kandle_amd import synthetic as syn

pytestmark = pytest.mark.gpu

BF16_ATOL = 2e-2
F32_RTOL = 1e-4


def _run(q, k, v, mask, scale=None, causal=False):
    o = F.scaled_dot_product_attention(q, k, v, attn_mask=mask, is_causal=causal, scale=scale)
    out = o.numpy()
    o.dispose()
    return out


def _mask(seed, shape, drop=0.25, std=2.0):
    """N(0, std^2) additive mask with a fraction of -inf entries; key 0 always finite."""
    m = syn.normal(seed, shape, std)
    r = np.random.default_rng(seed)
    m[r.random(shape) < drop] = -np.inf
    m[..., 0] = np.where(np.isinf(m[..., 0]), 0.0, m[..., 0])
    return m.astype(np.float32)


@pytest.mark.parametrize("B,Hq,Hkv,L,S,D", [(2, 8, 4, 128, 128, 128), (1, 4, 2, 77, 77, 128), (1, 8, 8, 40, 300, 128),
                                            (1, 4, 1, 1, 200, 128), (1, 6, 2, 100, 128, 128), (2, 10, 1, 64, 200, 128),
                                            (2, 8, 4, 128, 128, 64), (1, 6, 2, 77, 300, 64)])
def test_mfma_full_mask_matches_oracle(hip, B, Hq, Hkv, L, S, D):
    """bf16 q/k/v, D = 128 or 64 (MFMA kernel), a full [B, Hq, L, S] float32 mask with -inf entries;
    ragged S (77, 300) takes the packed-mask path, S = 128 reads the mask in place; L = 1 is a
    decode-shaped call; GQA 3 and 10 run as groups of one query head per workgroup."""
    q, qh = seeded(101, (B, Hq, L, D), "bfloat16")
    k, kh = seeded(102, (B, Hkv, S, D), "bfloat16")
    v, vh = seeded(103, (B, Hkv, S, D), "bfloat16")
    m = _mask(104, (B, Hq, L, S))
    out = _run(q, k, v, dev(m))
    ref = oracle.sdpa_masked(qh, kh, vh, m)
    assert np.max(np.abs(out - ref)) < BF16_ATOL


def test_mfma_broadcast_bottom_right_mask_and_causal_flag_ignored(hip):
    """A broadcast [L, S] mask with the capture path's bottom-right causal pattern
    (packages/model-utils/src/attention/gqa.ts:374: key j > i + (S - L) masked); is_causal=True is
    ignored when a mask is given (composite.ts:279-300 returns before the causal route)."""
    L, S = 100, 300
    q, qh = seeded(111, (2, 4, L, 128), "bfloat16")
    k, kh = seeded(112, (2, 2, S, 128), "bfloat16")
    v, vh = seeded(113, (2, 2, S, 128), "bfloat16")
    br = np.where(np.arange(S)[None, :] > np.arange(L)[:, None] + (S - L), -np.inf, 0.0).astype(np.float32)
    out = _run(q, k, v, dev(br), causal=True)
    ref = oracle.sdpa_masked(qh, kh, vh, br)
    assert np.max(np.abs(out - ref)) < BF16_ATOL
    # with L == S the bottom-right mask is the top-left causal attention
    qs_, qsh = seeded(114, (1, 4, 256, 128), "bfloat16")
    tri = np.where(np.arange(256)[None, :] > np.arange(256)[:, None], -np.inf, 0.0).astype(np.float32)
    k0, v0 = F.narrow(F.narrow(k, 0, 0, 1), 2, 0, 256), F.narrow(F.narrow(v, 0, 0, 1), 2, 0, 256)
    out2 = _run(qs_, k0, v0, dev(tri))
    ref2 = oracle.sdpa(qsh, kh[:1, :, :256], vh[:1, :, :256], causal=True)
    assert np.max(np.abs(out2 - ref2[:1])) < BF16_ATOL


def test_mfma_bf16_mask_head_broadcast(hip):
    """bfloat16 mask [B, 1, L, S] broadcast over the query heads."""
    q, qh = seeded(121, (2, 8, 64, 128), "bfloat16")
    k, kh = seeded(122, (2, 4, 192, 128), "bfloat16")
    v, vh = seeded(123, (2, 4, 192, 128), "bfloat16")
    m = _mask(124, (2, 1, 64, 192))
    bits, mvals = syn.bf16(np.where(np.isinf(m), 0.0, m).astype(np.float32))
    mvals = np.where(np.isinf(m), -np.inf, mvals).astype(np.float32)
    out = _run(q, k, v, dev(mvals, "bfloat16"))
    ref = oracle.sdpa_masked(qh, kh, vh, mvals)
    assert np.max(np.abs(out - ref)) < BF16_ATOL


def test_mfma_strided_mask_view_is_packed(hip):
    """A transposed view (key stride != 1) is packed before the MFMA kernel reads it."""
    L, S = 96, 160
    q, qh = seeded(131, (1, 4, L, 128), "bfloat16")
    k, kh = seeded(132, (1, 2, S, 128), "bfloat16")
    v, vh = seeded(133, (1, 2, S, 128), "bfloat16")
    m = _mask(134, (L, S))
    m_dev = F.transpose(dev(np.ascontiguousarray(m.T)), 0, 1)  # device [L, S] view, strides (1, L)
    assert m_dev.strides[-1] != 1
    out = _run(q, k, v, m_dev)
    ref = oracle.sdpa_masked(qh, kh, vh, m)
    assert np.max(np.abs(out - ref)) < BF16_ATOL


def test_fully_masked_rows_are_nan(hip):
    """Rows whose every score is -inf are 0 / 0 = NaN (reference softmax); other rows are exact."""
    for dtype, L, S, D in (("bfloat16", 70, 130, 128), ("float32", 20, 33, 64)):
        q, qh = seeded(141, (1, 4, L, D), dtype)
        k, kh = seeded(142, (1, 2, S, D), dtype)
        v, vh = seeded(143, (1, 2, S, D), dtype)
        m = _mask(144, (1, 4, L, S))
        m[0, 1, 5, :] = -np.inf
        m[0, 3, L - 1, :] = -np.inf
        out = _run(q, k, v, dev(m))
        ref = oracle.sdpa_masked(qh, kh, vh, m)
        nan_ref = np.isnan(ref)
        assert nan_ref[0, 1, 5].all() and nan_ref[0, 3, L - 1].all()
        assert np.array_equal(np.isnan(out), nan_ref)
        ok = ~nan_ref
        if dtype == "bfloat16":
            assert np.max(np.abs(out[ok] - ref[ok])) < BF16_ATOL
        else:
            assert max_rel(out[ok], ref[ok]) < F32_RTOL


def test_fp32_masked_c1_size(hip):
    """fp32 at config C1's shape (B=1, Hq=16, Hkv=8, S=256, D=128) with a full mask: the fp32-math
    kernel, 1e-4 relative."""
    q, qh = seeded(151, (1, 16, 256, 128))
    k, kh = seeded(152, (1, 8, 256, 128))
    v, vh = seeded(153, (1, 8, 256, 128))
    m = _mask(154, (256, 256))
    out = _run(q, k, v, dev(m))
    ref = oracle.sdpa_masked(qh, kh, vh, m)
    assert max_rel(out, ref) < F32_RTOL


def test_mask_errors(hip):
    q, _ = seeded(161, (1, 2, 8, 128), "bfloat16")
    k, _ = seeded(162, (1, 2, 8, 128), "bfloat16")
    with pytest.raises(ValueError, match="cannot be broadcast"):
        F.scaled_dot_product_attention(q, k, k, attn_mask=dev(np.zeros((3, 8), np.float32)))
    with pytest.raises(TypeError, match="attn_mask dtype"):
        F.scaled_dot_product_attention(q, k, k, attn_mask=dev(np.zeros((8, 8), np.int32), "int32"))


@pytest.mark.parametrize("B,Hq,Hkv,L,S,D", [(1, 8, 4, 100, 300, 96), (2, 4, 2, 77, 77, 48), (1, 4, 4, 128, 128, 80)])
def test_mfma_mask_staged_head_dims(hip, B, Hq, Hkv, L, S, D):
    """Head dims without MFMA tiles: Q, K and V are staged as rows zero-padded to 64 or 128 columns
    and the masked MFMA kernel runs on them (the packed-mask path for S = 77 and 300)."""
    q, qh = seeded(111, (B, Hq, L, D), "bfloat16")
    k, kh = seeded(112, (B, Hkv, S, D), "bfloat16")
    v, vh = seeded(113, (B, Hkv, S, D), "bfloat16")
    m = _mask(114, (B, Hq, L, S))
    out = _run(q, k, v, dev(m))
    ref = oracle.sdpa_masked(qh, kh, vh, m)
    assert np.max(np.abs(out - ref)) < BF16_ATOL
