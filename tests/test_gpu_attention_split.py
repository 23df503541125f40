"""GPU parity of the split-bf16 fp32 attention (kh_flash_attention_split, registered as
flash_attention_split): each fp32 operand value x is taken as hi = bf16(x) plus lo = bf16(x - hi),
and every product of S = Q K^T and O = P V as hi*hi + hi*lo + lo*hi in fp32.

Two bars per case:
- against a float64 numpy emulation of that arithmetic (split Q, K; softmax of the split scores;
  P split the same way; l the sum of P): 6e-5 of the output scale, so a wrong operand layout, a
  dropped term or a mis-merged key split fails.  (The emulation's P is relative to the row maximum,
  the kernel's to its running reference maximum, so the two split P differently, each within 2^-16
  of every weight);
- against the fp32 oracle (the reference's f32 attention): 4e-4 of the output scale.  Each dropped
  lo*lo term and each lo rounding is below 2^-16 of its product, so a score moves by up to about
  2^-15 * scale * sum|q||k| (~3e-4 at D = 128 with unit-variance q, k) and the output by about that
  relative; measured errors are well inside.
Semantics (causal top-left mask, GQA h -> h / G, scale) as flash_attention
(packages/backend-webgpu/src/kernels/attention/builder.ts:138-329)."""
import numpy as np
import pytest

import oracle
from helpers import assert_close_elem, max_rel, seeded
from kandle_amd import HipTensorHandle, Tensor, kernels

pytestmark = pytest.mark.gpu

EMU_RTOL = 6e-5
F32_RTOL = 4e-4


def _split(a):
    a = np.asarray(a, np.float32)
    hi = oracle.bf16_round(a)
    lo = oracle.bf16_round(a - hi)
    return hi.astype(np.float64), lo.astype(np.float64)


def _emulate(q, k, v, scale, causal):
    """float64 split-bf16 attention over [B, H, L, D] arrays (GQA by head index)."""
    B, Hq, Lq, D = q.shape
    Hkv, Lk = k.shape[1], k.shape[2]
    G = Hq // Hkv
    out = np.empty((B, Hq, Lq, D), np.float64)
    mask = np.arange(Lk)[None, :] > np.arange(Lq)[:, None] if causal else None
    for b in range(B):
        for h in range(Hq):
            qh, ql = _split(q[b, h])
            kh, kl = _split(k[b, h // G])
            vh, vl = _split(v[b, h // G])
            s = (qh @ kh.T + qh @ kl.T + ql @ kh.T) * scale
            if causal:
                s[mask] = -np.inf
            p = np.exp(s - s.max(axis=1, keepdims=True)).astype(np.float32)
            ph, pl = _split(p)
            out[b, h] = (ph @ vh + ph @ vl + pl @ vh) / p.astype(np.float64).sum(axis=1, keepdims=True)
    return out


def _run(q, k, v, causal, scale):
    B, Hq, Lq, D = q.shape
    o = HipTensorHandle.create_new((B, Hq, Lq, D), "float32")
    kernels.flash_attention_split(q.handle, k.handle, v.handle, o, scale, causal)
    out = o.data_async()
    o.dispose()
    return out


@pytest.mark.parametrize("B,Hq,Hkv,Lq,Lk,causal", [
    (1, 16, 8, 512, 512, True),    # the C5 prefill
    (1, 16, 8, 256, 256, True),    # C1's shape
    (1, 4, 4, 300, 300, True),     # GQA 1, a partial last block
    (2, 16, 4, 257, 257, False),   # GQA 4, a ragged key chunk
    (1, 8, 4, 100, 300, True),     # Lq < Lk (top-left: row i sees keys 0..i)
    (1, 8, 8, 300, 100, True),     # Lq > Lk: rows past Lk see every key
    (1, 4, 2, 77, 77, False),
    (2, 8, 8, 33, 1000, False),    # many stages, one query block
    (1, 16, 1, 130, 130, True),    # GQA 16 (one kv head for all query heads)
    (1, 12, 4, 200, 200, True),    # GQA 3
])
def test_split_attention_matches_emulation_and_fp32(hip, B, Hq, Hkv, Lq, Lk, causal):
    D = 128
    q, qv = seeded(70, (B, Hq, Lq, D))
    k, kv = seeded(71, (B, Hkv, Lk, D))
    v, vv = seeded(72, (B, Hkv, Lk, D))
    scale = 1.0 / np.sqrt(D)
    out = _run(q, k, v, causal, scale)
    assert np.all(np.isfinite(out))
    emu = _emulate(qv, kv, vv, scale, causal)
    e_emu = max_rel(out, emu)
    e_f32 = max_rel(out, oracle.sdpa(qv, kv, vv, scale=scale, causal=causal))
    print(f"[split attention] {B, Hq, Hkv, Lq, Lk, causal}: vs emulation {e_emu:.2e}, vs fp32 {e_f32:.2e}")
    assert e_emu < EMU_RTOL
    assert e_f32 < F32_RTOL
    assert_close_elem(out, oracle.sdpa(qv, kv, vv, scale=scale, causal=causal), rtol=4e-4, atol=4e-5,
                      what="split vs fp32")


def test_split_attention_softmax_raises_and_strided_views(hip):
    """q, k ~ N(0, 2^2) spread the scores over tens of nats, so the reference maximum is raised in
    the middle of the key loop of every key split; the operands are [B, S, H, D] storage read
    through permuted views (no copy)."""
    B, S, Hq, Hkv, D = 1, 400, 8, 4, 128
    qs, qv = seeded(73, (B, S, Hq, D), std=2.0)
    ks, kv = seeded(74, (B, S, Hkv, D), std=2.0)
    vs, vv = seeded(75, (B, S, Hkv, D))
    perm = (0, 2, 1, 3)

    def view(t, shape):
        Bn, Sn, Hn, Dn = shape
        return Tensor(handle=HipTensorHandle.create_view(t.handle.storage, (Bn, Hn, Sn, Dn), "float32",
                                                         (Sn * Hn * Dn, Dn, Hn * Dn, 1), 0))

    q, k, v = view(qs, qs.shape), view(ks, ks.shape), view(vs, vs.shape)
    qp, kp, vp = (np.ascontiguousarray(np.transpose(a, perm)) for a in (qv, kv, vv))
    scale = 1.0 / np.sqrt(D)
    out = _run(q, k, v, True, scale)
    assert max_rel(out, _emulate(qp, kp, vp, scale, True)) < EMU_RTOL
    assert max_rel(out, oracle.sdpa(qp, kp, vp, scale=scale, causal=True)) < F32_RTOL


def test_split_attention_8k_tokens(hip):
    """An 8192-token causal call (8/4 heads): long-sequence offsets; the last 32 rows of every head
    and one row per 256-row block of every head against the fp32 oracle."""
    B, Hq, Hkv, S, D = 1, 8, 4, 8192, 128
    q, qv = seeded(83, (B, Hq, S, D))
    k, kv = seeded(84, (B, Hkv, S, D))
    v, vv = seeded(85, (B, Hkv, S, D))
    scale = 1.0 / np.sqrt(D)
    out = _run(q, k, v, True, scale)
    assert np.all(np.isfinite(out))
    G = Hq // Hkv
    for h in range(Hq):
        rows = np.concatenate([np.array([blk * 256 + (29 * blk + 7 * h) % 256 for blk in range(S // 256)]),
                               np.arange(S - 32, S)])
        mask = np.where(np.arange(S)[None, :] > rows[:, None], -np.inf, 0.0).astype(np.float32)
        ref = oracle.sdpa_masked(qv[:, h:h + 1, rows], kv[:, h // G:h // G + 1], vv[:, h // G:h // G + 1], mask,
                                 scale=scale)
        assert max_rel(out[:, h:h + 1, rows], ref) < F32_RTOL, h


def test_split_attention_gqa_8(hip):
    """GQA 8 (query head h reads kv head h / 8)."""
    q, qv = seeded(80, (1, 16, 130, 128))
    k, kv = seeded(81, (1, 2, 130, 128))
    v, vv = seeded(82, (1, 2, 130, 128))
    scale = 1.0 / np.sqrt(128)
    out = _run(q, k, v, True, scale)
    assert max_rel(out, _emulate(qv, kv, vv, scale, True)) < EMU_RTOL
    assert max_rel(out, oracle.sdpa(qv, kv, vv, scale=scale, causal=True)) < F32_RTOL


def test_split_attention_other_head_dims_take_the_fp32_kernel(hip):
    """head_dim 64 is outside the split kernel: the call runs the fp32 kernel (1e-4)."""
    q, qv = seeded(76, (1, 4, 130, 64))
    k, kv = seeded(77, (1, 2, 130, 64))
    v, vv = seeded(78, (1, 2, 130, 64))
    scale = 1.0 / np.sqrt(64)
    out = _run(q, k, v, True, scale)
    assert max_rel(out, oracle.sdpa(qv, kv, vv, scale=scale, causal=True)) < 1e-4


def test_split_attention_rejects_bf16(hip):
    q, _ = seeded(79, (1, 4, 16, 128), "bfloat16")
    o = HipTensorHandle.create_new((1, 4, 16, 128), "bfloat16")
    with pytest.raises(TypeError):
        kernels.flash_attention_split(q.handle, q.handle, q.handle, o, 0.1, True)
    o.dispose()
