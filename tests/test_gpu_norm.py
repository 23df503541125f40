"""GPU parity of RMSNorm and the fused qk-norm + RoPE kernel against the CPU oracle."""
import numpy as np
import pytest

import oracle
from helpers import max_rel, seeded
from kandle_amd import Tensor
from kandle_amd import functional as F
from kandle_amd import kernels
from kandle_amd import synthetic as syn

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows,n", [(37, 1024), (5, 128), (3, 4096), (2, 6000), (4, 33)])
def test_rms_norm_fp32(hip, rows, n):
    x, xh = seeded(101, (rows, n))
    w = syn.uniform(102, (n,), 0.5, 1.5)
    y = F.rms_norm(x, [n], Tensor(w), eps=1e-6).numpy()
    assert max_rel(y, oracle.rms_norm(xh, w, 1e-6)) < 1e-4


def test_rms_norm_bf16_no_weight_default_eps(hip):
    x, xh = seeded(103, (64, 1024), "bfloat16")
    y = F.rms_norm(x, [1024]).numpy()  # kernel default eps 1e-5 (normalize/executor.ts:58)
    ref = oracle.bf16_round(oracle.rms_norm(xh, None, 1e-5))
    assert np.max(np.abs(y - ref)) <= 2 ** -7 * np.max(np.abs(ref))


@pytest.mark.parametrize("rows,n", [(9, 1024), (3, 130)])
def test_rms_norm_fp32_in_bf16_out(hip, rows, n):
    """A float32 residual row normalised straight into bf16 with a bf16 weight: exactly the oracle's
    fp32 result rounded once (within one bf16 ulp of rounding-boundary noise)."""
    x, xh = seeded(105, (rows, n))
    w = oracle.bf16_round(syn.uniform(106, (n,), 0.5, 1.5))
    y = F.rms_norm(x, [n], Tensor(w, dtype="bfloat16"), eps=1e-6, out_dtype="bfloat16")
    assert y.dtype == "bfloat16"
    ref = oracle.bf16_round(oracle.rms_norm(xh, w, 1e-6))
    assert np.max(np.abs(y.numpy() - ref)) <= 2 ** -7 * np.max(np.abs(ref))


def test_rms_norm_on_permuted_view(hip):
    """Strided input is materialised; the output is contiguous (normalize/executor.ts:121-122)."""
    x, xh = seeded(104, (6, 4, 128))
    xt = F.permute(x, (1, 0, 2))
    y = F.rms_norm(xt, [128]).numpy()
    assert max_rel(y, oracle.rms_norm(np.transpose(xh, (1, 0, 2)), None, 1e-5)) < 1e-4


def _qk_case(T, Hq, Hkv, D, dtype, seed, theta=1e6, eps=1e-6):
    q, qh = seeded(seed, (1, T, Hq, D), dtype)
    k, kh = seeded(seed + 1, (1, T, Hkv, D), dtype)
    wq = syn.uniform(seed + 2, (D,), 0.5, 1.5)
    wk = syn.uniform(seed + 3, (D,), 0.5, 1.5)
    if dtype == "bfloat16":
        wq, wk = oracle.bf16_round(wq), oracle.bf16_round(wk)
    inv = oracle.rope_inv_freq(D, theta)
    pos = np.arange(T, dtype=np.int32)
    params = {"q_weight": Tensor(wq, dtype=dtype).handle, "k_weight": Tensor(wk, dtype=dtype).handle,
              "inv_freq": Tensor(inv).handle, "positions": Tensor(pos, dtype="int32").handle, "eps": eps}
    qo, ko = kernels.rms_norm_rope(q.handle, k.handle, params)
    rq = oracle.qk_norm_rope(qh[0], wq, pos, inv, eps)      # [T, Hq, D]
    rk = oracle.qk_norm_rope(kh[0], wk, pos, inv, eps)
    gq = qo.data_async()[0].transpose(1, 0, 2)             # [Hq, T, D] -> [T, Hq, D]
    gk = ko.data_async()[0].transpose(1, 0, 2)
    return gq, gk, rq, rk


def test_qk_norm_rope_fp32_matches_oracle(hip):
    gq, gk, rq, rk = _qk_case(300, 16, 8, 128, "float32", 110)
    assert max_rel(gq, rq) < 1e-4 and max_rel(gk, rk) < 1e-4


@pytest.mark.parametrize("D", [64, 128, 256])
def test_qk_norm_rope_head_dims(hip, D):
    gq, gk, rq, rk = _qk_case(40, 4, 2, D, "float32", 120, theta=1e4)
    assert max_rel(gq, rq) < 1e-4 and max_rel(gk, rk) < 1e-4


def test_c2_full_size_bf16(hip):
    """Config C2: 8192 tokens, hidden 1024 RMSNorm + 16/8-head qk-norm + RoPE, theta 1e6, eps 1e-6,
    bf16 in/out with fp32 math: every output within one bf16 rounding of the oracle."""
    T = 8192
    x, xh = seeded(130, (T, 1024), "bfloat16")
    wh = oracle.bf16_round(syn.uniform(131, (1024,), 0.5, 1.5))
    y = F.rms_norm(x, [1024], Tensor(wh, dtype="bfloat16"), eps=1e-6).numpy()
    ry = oracle.rms_norm(xh, wh, 1e-6)
    assert np.all(np.abs(y - ry) <= 2 ** -8 * np.abs(ry) + 1e-6)
    gq, gk, rq, rk = _qk_case(T, 16, 8, 128, "bfloat16", 140)
    for g, r in ((gq, rq), (gk, rk)):
        assert np.all(np.abs(g - r) <= 2 ** -8 * np.abs(r) + 1e-5), float(np.max(np.abs(g - r)))


def test_qk_norm_rope_fused_v_copy(hip):
    """The fused V cache write copies V rows unchanged into a heads-first cache slice."""
    T, Hq, Hkv, D = 20, 4, 2, 128
    q, _ = seeded(150, (1, T, Hq, D), "bfloat16")
    k, _ = seeded(151, (1, T, Hkv, D), "bfloat16")
    v, vh = seeded(152, (1, T, Hkv, D), "bfloat16")
    cache = F.zeros((1, Hkv, 64, D), "bfloat16")
    v_out = F.narrow(cache, 2, 10, T)
    ones = Tensor(np.ones(D, np.float32), dtype="bfloat16").handle
    params = {"q_weight": ones, "k_weight": ones, "inv_freq": Tensor(oracle.rope_inv_freq(D, 1e6)).handle,
              "positions": Tensor(np.arange(T, dtype=np.int32) + 10, dtype="int32").handle, "eps": 1e-6,
              "v": v.handle, "v_out": v_out.handle}
    kernels.rms_norm_rope(q.handle, k.handle, params)
    c = cache.numpy()
    np.testing.assert_array_equal(c[0, :, 10:10 + T], vh[0].transpose(1, 0, 2))
    assert np.all(c[0, :, :10] == 0) and np.all(c[0, :, 10 + T:] == 0)


def test_qk_norm_rope_cache_positions(hip):
    """Cache addressing: K/V of token t land in cache row positions[t]; a position outside the
    cache writes nothing; rows no token names keep their contents; q keeps token order."""
    T, Hq, Hkv, D, L = 5, 4, 2, 128, 8
    pos = np.array([3, 0, 7, 9, 1], np.int32)
    q, qh = seeded(130, (1, T, Hq, D))
    k, kh = seeded(131, (1, T, Hkv, D))
    v, vh = seeded(132, (1, T, Hkv, D))
    wq = syn.uniform(133, (D,), 0.5, 1.5)
    wk = syn.uniform(134, (D,), 0.5, 1.5)
    inv = oracle.rope_inv_freq(D, 1e6)
    kc = Tensor(np.full((1, Hkv, L, D), 7.0, np.float32))
    vc = Tensor(np.full((1, Hkv, L, D), 7.0, np.float32))
    params = {"q_weight": Tensor(wq).handle, "k_weight": Tensor(wk).handle, "inv_freq": Tensor(inv).handle,
              "positions": Tensor(pos, dtype="int32").handle, "eps": 1e-6, "k_out": kc.handle,
              "v": v.handle, "v_out": vc.handle, "cache_positions": True}
    qo, _ = kernels.rms_norm_rope(q.handle, k.handle, params)
    rq = oracle.qk_norm_rope(qh[0], wq, pos, inv, 1e-6)          # [T, Hq, D]
    rk = oracle.qk_norm_rope(kh[0], wk, pos, inv, 1e-6)          # [T, Hkv, D]
    assert max_rel(qo.data_async()[0].transpose(1, 0, 2), rq) < 1e-4
    gk, gv = kc.numpy()[0], vc.numpy()[0]                          # [Hkv, L, D]
    written = {int(p_): t for t, p_ in enumerate(pos) if 0 <= p_ < L}
    for row in range(L):
        if row in written:
            t = written[row]
            assert max_rel(gk[:, row], rk[t]) < 1e-4
            np.testing.assert_array_equal(gv[:, row], vh[0, t])
        else:
            assert np.all(gk[:, row] == 7.0) and np.all(gv[:, row] == 7.0)
