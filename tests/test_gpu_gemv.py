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


@pytest.mark.parametrize("N,K", [(300, 17408), (1000, 25600), (64, 32768)])
def test_gemv_long_rows(hip, N, K):
    """Rows longer than 16384 (the down projections of 14B- and 32B-class models: intermediate sizes
    17408 and 25600): x' staged in more than 64 KiB of LDS; fp32 residual row out, bf16 weights."""
    x, xh = seeded(305, (1, K), "bfloat16")
    w, wh = seeded(306, (N, K), "bfloat16", std=0.02)
    y = F.linear_fused("none", x, w).numpy()
    ok, err = _close_bf16(y, oracle.linear(xh, wh), K)
    assert ok, err
    r, rh = seeded(307, (1, N))
    F.linear_fused("none", x, w, residual=r)          # r += x W^T, fp32
    ok, err = _close_f32(r.numpy(), rh + oracle.linear(xh, wh))
    assert ok, err


def test_gemv_rejects_rows_past_32768(hip):
    x, _ = seeded(308, (1, 32776), "bfloat16")
    w, _ = seeded(309, (8, 32776), "bfloat16")
    with pytest.raises(Exception, match="32768"):
        F.linear_fused("none", x, w)


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


def test_gemv_interleaved_silu_mul_prologue_matches_split_halves(hip):
    """Prologue 'silu_mul_interleaved' reads gate/up interleaved in blocks of 8 from one row; it
    equals prologue 'silu_mul' on the same values split into gate and up rows, bit for bit."""
    I, N = 3072, 1024
    g, gh = seeded(330, (1, I), "bfloat16", std=2.0)
    u, uh = seeded(331, (1, I), "bfloat16", std=2.0)
    from kandle_amd.kernels import interleave_gate_up
    gu_vals = interleave_gate_up(gh.reshape(I, 1), uh.reshape(I, 1)).reshape(1, 2 * I)
    gu = Tensor(syn.bf16(gu_vals)[0], dtype="bfloat16")
    w, wh = seeded(332, (N, I), "bfloat16", std=0.02)
    res0 = Tensor(np.zeros((1, N), np.float32))
    res1 = Tensor(np.zeros((1, N), np.float32))
    a = F.linear_fused("silu_mul", g, w, x2=u, residual=res0).numpy()
    b = F.linear_fused("silu_mul_interleaved", gu, w, residual=res1).numpy()
    assert np.array_equal(a, b)
    ref = oracle.linear(oracle.bf16_round(oracle.silu_mul(gh, uh)), wh)
    ok, err = _close_f32(b, ref)
    assert ok, err


@pytest.mark.parametrize("prologue", ["rms_norm", "none"])
@pytest.mark.parametrize("I,K", [(3072, 1024), (64, 256), (8, 520)])
def test_gemv_swiglu_matches_gate_up_row_and_silu_mul_prologue(hip, prologue, I, K):
    """kh_gemv_swiglu (one wave per gate/up row pair of the interleaved weight, silu * mul in the
    epilogue) equals the gate/up projection row (kh_gemv_fused) followed by the interleaved
    silu * mul, bit for bit; so does the down projection fed from either."""
    from kandle_amd.kernels import interleave_gate_up
    N = 1024
    if prologue == "rms_norm":
        x = Tensor(syn.normal(340, (1, K), 3.0))
        nw, _ = seeded(341, (K,), "bfloat16")
    else:
        x, _ = seeded(340, (1, K), "bfloat16")
        nw = None
    _, gh = seeded(342, (I, K), "bfloat16", std=0.05)
    _, uh = seeded(343, (I, K), "bfloat16", std=0.05)
    w_gu = Tensor(syn.bf16(interleave_gate_up(gh, uh))[0], dtype="bfloat16")
    a = F.linear_swiglu_row(prologue, x, w_gu, nw, 1e-6)
    gu = F.linear_fused(prologue, x, w_gu, nw, 1e-6)                    # [1, 2I] interleaved
    gv = gu.numpy().reshape(I // 8, 2, 8)
    ref = oracle.silu_mul(gv[:, 0].reshape(-1), gv[:, 1].reshape(-1))
    av = a.numpy().reshape(-1)
    assert np.all(np.abs(av - ref) <= 2 ** -8 * np.abs(ref) + 1e-30)      # one bf16 rounding
    w_d, _ = seeded(344, (N, I), "bfloat16", std=0.02)
    res0 = Tensor(np.ones((1, N), np.float32))
    res1 = Tensor(np.ones((1, N), np.float32))
    y0 = F.linear_fused("silu_mul_interleaved", gu, w_d, residual=res0).numpy()
    y1 = F.linear_fused("none", a, w_d, residual=res1).numpy()
    np.testing.assert_array_equal(y0, y1)


@pytest.mark.parametrize("M,I,K", [(512, 3072, 1024), (130, 96, 64), (1, 3072, 1024), (7, 40, 200), (600, 3072, 1024)])
def test_linear_swiglu_matches_unfused_gemm_and_silu_mul(hip, M, I, K):
    """kh_gemm_swiglu (gate/up GEMM with silu*mul in the epilogue, interleaved weight) against the
    unfused sequence -- the GEMM over the plain [gate; up] weight stored in bf16, then silu_mul --
    bit for bit where that GEMM runs the same MFMA tiles (M > 8), and against the oracle within a
    bound for one bf16 rounding of g, u and h."""
    from kandle_amd.kernels import interleave_gate_up
    x, xh = seeded(340, (M, K), "bfloat16")
    wg_bits, wg = syn.bf16(syn.normal(341, (I, K), 0.05))
    wu_bits, wu = syn.bf16(syn.normal(342, (I, K), 0.05))
    w_cat = Tensor(np.concatenate([wg_bits, wu_bits]), dtype="bfloat16")
    w_il = Tensor(interleave_gate_up(wg_bits, wu_bits), dtype="bfloat16")
    fused = F.linear_swiglu(x, w_il).numpy()
    gu = F.linear(x, w_cat)
    unfused = F.silu_mul(F.narrow(gu, 1, 0, I), F.narrow(gu, 1, I, I)).numpy()
    if M > 8:   # the unfused GEMM takes the same MFMA tiles (M <= 8: the one-row / skinny paths)
        assert np.array_equal(fused.view(np.uint32), unfused.view(np.uint32))
    g = oracle.bf16_round(oracle.linear(xh, wg)).astype(np.float64)
    u = oracle.bf16_round(oracle.linear(xh, wu)).astype(np.float64)
    ref = oracle.silu_mul(g.astype(np.float32), u.astype(np.float32)).astype(np.float64)
    # g and u are fp32 sums rounded to bf16, so either may sit one bf16 rounding (2^-8 relative) away
    # from the f64 oracle's; silu' <= 1.1, and h itself is rounded once more.
    silu = g / (1.0 + np.exp(-np.clip(g, -88, 88)))
    bound = 2.0 ** -8 * (1.1 * np.abs(g) * np.abs(u) + np.abs(silu) * np.abs(u) + np.abs(ref)) + 1e-6
    assert np.all(np.abs(fused - ref) <= bound), float(np.max(np.abs(fused - ref) - bound))


def test_linear_swiglu_rejects_bad_layouts(hip):
    x, _ = seeded(350, (4, 64), "bfloat16")
    w, _ = seeded(351, (2 * 12, 64), "bfloat16")   # intermediate 12: not a multiple of 8
    with pytest.raises(Exception, match="multiple of 8"):
        F.linear_swiglu(x, w)


@pytest.mark.parametrize("M,N,K,rows", [(512, 1024, 2048, None), (512, 1024, 3072, None), (512, 1024, 3072, (511, 512)),
                                        (130, 1024, 2048, (7, 100)), (600, 1024, 3072, None), (64, 96, 40, None)])
def test_linear_add_rms_norm_matches_separate_launches(hip, M, N, K, rows):
    """The projection + residual add + RMSNorm of linear_add_rms_norm (split-K partials summed by
    kh_add_rms_norm when kh_gemm splits the shape, else kh_gemm then kh_rms_norm) against the
    separate launches -- kh_gemm with the residual as C (beta = 1), then kh_rms_norm -- bit for bit
    in both the residual and the normed rows, rows outside `rows` untouched; and against the oracle
    (fp32 residual within the accumulation-order allowance, the bf16 norm within one rounding)."""
    from kandle_amd import kernels
    x, xh = seeded(360, (M, K), "bfloat16")
    w, wh = seeded(361, (N, K), "bfloat16", std=0.02)
    nw_bits, nwh = syn.bf16(1.0 + syn.normal(362, (N,), 0.1))
    nw = Tensor(nw_bits, dtype="bfloat16")
    r0 = syn.normal(363, (M, N))
    lo, hi = rows if rows is not None else (0, M)
    res = Tensor(r0.copy())
    h = F.linear_add_rms_norm(x, w, res, nw, 1e-6, rows=rows)
    fused_res, fused_h = res.numpy(), h.numpy()
    ref_res = Tensor(r0.copy())
    F.dispatch_matmul(x, w, c=ref_res, beta=1.0, out=ref_res, transpose_b=True)
    sep_h = F.rms_norm(F.narrow(ref_res, 0, lo, hi - lo), [N], nw, 1e-6, out_dtype="bfloat16").numpy()
    sep_res = ref_res.numpy()
    assert fused_h.shape == (hi - lo, N)
    assert np.array_equal(fused_res[lo:hi].view(np.uint32), sep_res[lo:hi].view(np.uint32))
    assert np.array_equal(fused_h.view(np.uint32), sep_h.view(np.uint32))
    assert np.array_equal(fused_res[:lo], r0[:lo]) and np.array_equal(fused_res[hi:], r0[hi:])
    ref = oracle.linear(xh, wh) + r0
    ok, err = _close_f32(fused_res[lo:hi], ref[lo:hi])
    assert ok, err
    ok, err = _close_bf16(fused_h, oracle.rms_norm(ref[lo:hi], nwh, 1e-6), N)
    assert ok, err
    if (M, N, K) == (512, 1024, 2048):
        assert kernels.gemm_split_count(M, N, K) > 1     # the fused split path is what ran


@pytest.mark.parametrize("S,H,Hq,Hkv,L,pos0", [(512, 1024, 16, 8, 640, 0), (200, 1024, 16, 8, 204, 10),
                                              (40, 256, 4, 2, 64, 30), (9, 256, 4, 2, 64, 60)])
def test_linear_qk_norm_rope_matches_projection_then_rms_norm_rope(hip, S, H, Hq, Hkv, L, pos0):
    """kh_gemm_qk_norm_rope (QKV projection with qk-norm, RoPE and the K/V cache write in its
    epilogue; again with the angles from kh_rope_table) against the two launches it replaces --
    kh_gemm into [S, (Hq + 2 Hkv) 128], then kh_qk_norm_rope with cache addressing -- bit for bit
    in q and in both whole caches, on shapes
    kh_gemm does not split over K (where the model fuses); a ragged last tile (200 rows); positions
    past the cache (pos0 + S > L) write no K/V row, as in the unfused kernel."""
    from kandle_amd import kernels
    from kandle_amd.tensor import HipTensorHandle

    D = 128
    N = (Hq + 2 * Hkv) * D
    assert kernels.gemm_split_count(S, N, H) == 1
    x, _ = seeded(360, (S, H), "bfloat16")
    w, _ = seeded(361, (N, H), "bfloat16", std=0.05)
    wq = Tensor(syn.bf16(syn.uniform(362, (D,), 0.5, 1.5))[0], dtype="bfloat16")
    wk = Tensor(syn.bf16(syn.uniform(363, (D,), 0.5, 1.5))[0], dtype="bfloat16")
    inv = Tensor(oracle.rope_inv_freq(D, 1e6))
    pos = Tensor(np.arange(pos0, pos0 + S, dtype=np.int32), dtype="int32")
    cache0 = syn.bf16(syn.normal(364, (1, Hkv, L, D)))[0]    # rows the launches must leave alone

    def caches():
        return (Tensor(cache0.copy(), dtype="bfloat16"), Tensor(cache0.copy(), dtype="bfloat16"))

    # unfused: the projection, then qk-norm + RoPE with the cache write
    qkv = F.linear(x, w)
    k1, v1 = caches()
    q1 = HipTensorHandle.create_new((1, Hq, S, D), "bfloat16")

    def heads(col, n):
        return HipTensorHandle.create_view(qkv.handle.storage, (1, S, n, D), "bfloat16", (S * N, N, D, 1), col)

    kernels.rms_norm_rope(heads(0, Hq), heads(Hq * D, Hkv), {
        "q_weight": wq.handle, "k_weight": wk.handle, "inv_freq": inv.handle, "positions": pos.handle, "eps": 1e-6,
        "q_out": q1, "k_out": k1.handle, "v": heads((Hq + Hkv) * D, Hkv), "v_out": v1.handle, "cache_positions": True})
    # fused
    k2, v2 = caches()
    q2 = HipTensorHandle.create_new((1, Hq, S, D), "bfloat16")
    kernels.linear_qk_norm_rope(x.handle, w.handle, {
        "q_weight": wq.handle, "k_weight": wk.handle, "inv_freq": inv.handle, "positions": pos.handle, "eps": 1e-6,
        "q_out": q2, "k_out": k2.handle, "v_out": v2.handle})
    for a, b in ((Tensor(handle=q1), Tensor(handle=q2)), (k1, k2), (v1, v2)):
        assert np.array_equal(a.numpy().view(np.uint32), b.numpy().view(np.uint32))
    # fused, the angles read from the per-forward table (kh_rope_table): the same bits again
    tab = kernels.rope_table(pos.handle, inv.handle)
    angles = np.arange(pos0, pos0 + S, dtype=np.float32)[:, None] * inv.numpy()[None, :]   # f32 products
    t = tab.data_async()
    assert t.shape == (S, D // 2, 2)
    assert np.max(np.abs(t[..., 0] - np.cos(angles.astype(np.float64)))) < 2e-6
    assert np.max(np.abs(t[..., 1] - np.sin(angles.astype(np.float64)))) < 2e-6
    k3, v3 = caches()
    q3 = HipTensorHandle.create_new((1, Hq, S, D), "bfloat16")
    kernels.linear_qk_norm_rope(x.handle, w.handle, {
        "q_weight": wq.handle, "k_weight": wk.handle, "inv_freq": inv.handle, "positions": pos.handle, "eps": 1e-6,
        "q_out": q3, "k_out": k3.handle, "v_out": v3.handle, "rope_table": tab})
    for a, b in ((Tensor(handle=q1), Tensor(handle=q3)), (k1, k3), (v1, v3)):
        assert np.array_equal(a.numpy().view(np.uint32), b.numpy().view(np.uint32))
    tab.dispose()
    if pos0 + S > L:   # rows past the cache were not written
        assert np.array_equal(k2.numpy()[:, :, :pos0].view(np.uint32),
                              oracle.from_bf16_bits(cache0[:, :, :pos0]).view(np.uint32))


def test_linear_qk_norm_rope_rejects_bad_shapes(hip):
    from kandle_amd import kernels
    from kandle_amd.tensor import HipTensorHandle

    x, _ = seeded(370, (16, 64), "bfloat16")
    w, _ = seeded(371, (4 * 64, 64), "bfloat16")   # head_dim 64: not fused
    q = HipTensorHandle.create_new((1, 2, 16, 64), "bfloat16")
    kc = HipTensorHandle.create_new((1, 1, 32, 64), "bfloat16")
    with pytest.raises(ValueError, match="head_dim 128"):
        kernels.linear_qk_norm_rope(x.handle, w.handle, {"q_out": q, "k_out": kc, "v_out": kc})
