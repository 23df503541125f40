"""GPU parity of the float32-activation paths: float32 activations multiplied by bfloat16 weights,
the reference's float32 arithmetic (its bf16 checkpoints are widened to float32 on load,
packages/core/src/io/safetensor/dtypes.ts:17-31, and matmul runs in f32,
packages/core/src/dispatch/matmulOps.ts:136-144).

Bars.  On MFMA tiles each fp32 activation a enters as bf16 hi = bf16(a) plus lo = bf16(a - hi), so
|a - hi - lo| <= 2^-16 |a| and every product carries at most 2^-16 |a w| of error; fp32 accumulation
over K terms adds at most K 2^-24 sum|a w| (a worst-case bound, far above typical).  Outputs are
checked element by element against the oracle's double-accumulated products within
(2^-16 + K 2^-24) sum_k |a_k w_k|.  The one-row and skinny kernels multiply in fp32 and meet the
same bound.  Fused epilogues are checked against the unfused launches on the same inputs (bit for
bit where both sum in the same order), and the fused chain against the oracle.
"""
import numpy as np
import pytest

import oracle
from helpers import seeded
from kandle_amd import Tensor
from kandle_amd import functional as F
from kandle_amd import synthetic as syn

pytestmark = pytest.mark.gpu


def _gemm_bound(xh, wh, K):
    """(2^-16 + K 2^-24) * (|x| |w|^T): the split-operand plus fp32-accumulation bound."""
    return (2.0 ** -16 + K * 2.0 ** -24) * (np.abs(xh).astype(np.float64) @ np.abs(wh).astype(np.float64).T) + 1e-30


@pytest.mark.parametrize("M,N,K", [(512, 4096, 1024), (512, 1024, 2048), (512, 6144, 1024), (2048, 4096, 1024),
                                   (130, 96, 64), (600, 1024, 3072), (1, 3000, 1024), (7, 40, 200), (33, 24, 520)])
def test_gemm_f32_activations_bf16_weights(hip, M, N, K):
    """kh_gemm_ex: fp32 x [M, K] times bf16 W [N, K]^T, fp32 out -- MFMA tiles with the hi/lo split
    (M > 8: 64-, 128- and split-K tiles), the one-row GEMV (M = 1) and the skinny kernel (M <= 8) --
    within the split + accumulation bound of the oracle's double sums; a bf16 activation would miss
    it by ~2^-9 relative."""
    x, xh = seeded(600, (M, K), std=1.5)
    w, wh = seeded(601, (N, K), "bfloat16", std=0.05)
    y = F.linear(x, w).numpy()
    assert y.dtype == np.float32 and y.shape == (M, N)
    ref = oracle.linear(xh, wh).astype(np.float64)
    bound = _gemm_bound(xh, wh, K)
    assert np.all(np.abs(y - ref) <= bound), float(np.max(np.abs(y - ref) / bound))
    # the bar separates fp32 activations from bf16 ones: rounding x to bf16 moves the product about a
    # thousand times further from the oracle than the kernel's error
    yb = oracle.linear(oracle.bf16_round(xh), wh).astype(np.float64)
    assert np.max(np.abs(y - ref)) < 0.02 * np.max(np.abs(yb - ref))


def test_gemm_f32_activations_residual_epilogue(hip):
    """alpha / beta / C epilogue with an fp32 residual (the o_proj and down form, split over K)."""
    from kandle_amd import kernels

    M, N, K = 512, 1024, 3072
    assert kernels.gemm_split_count(M, N, K) > 1
    x, xh = seeded(610, (M, K))
    w, wh = seeded(611, (N, K), "bfloat16", std=0.02)
    r0 = syn.normal(612, (M, N))
    res = Tensor(r0.copy())
    F.dispatch_matmul(x, w, c=res, beta=1.0, out=res, transpose_b=True)
    ref = oracle.linear(xh, wh).astype(np.float64) + r0
    bound = _gemm_bound(xh, wh, K) + 2.0 ** -23 * np.abs(ref)
    assert np.all(np.abs(res.numpy() - ref) <= bound)


def test_gemm_f32_activations_rejects_bf16_a_with_f32_b(hip):
    x, _ = seeded(615, (16, 64), "bfloat16")
    w, _ = seeded(616, (32, 64))
    with pytest.raises(Exception):
        F.linear(x, w)


@pytest.mark.parametrize("M,N,K,rows", [(512, 1024, 2048, None), (512, 1024, 3072, (511, 512)),
                                        (130, 1024, 2048, (7, 100)), (64, 96, 40, None)])
def test_linear_add_rms_norm_f32_matches_separate_launches(hip, M, N, K, rows):
    """linear_add_rms_norm with fp32 activations and an fp32 norm (split-K partials summed by
    kh_add_rms_norm, or kh_gemm_ex then kh_rms_norm) against the separate launches bit for bit, and
    the residual against the oracle within the GEMM bound."""
    x, xh = seeded(620, (M, K))
    w, wh = seeded(621, (N, K), "bfloat16", std=0.02)
    nwh = oracle.bf16_round(1.0 + syn.normal(622, (N,), 0.1))
    nw = Tensor(nwh)                           # fp32 holding the bf16 values exactly
    r0 = syn.normal(623, (M, N))
    lo, hi = rows if rows is not None else (0, M)
    res = Tensor(r0.copy())
    h = F.linear_add_rms_norm(x, w, res, nw, 1e-6, rows=rows)
    assert h.dtype == "float32"
    ref_res = Tensor(r0.copy())
    F.dispatch_matmul(x, w, c=ref_res, beta=1.0, out=ref_res, transpose_b=True)
    sep_h = F.rms_norm(F.narrow(ref_res, 0, lo, hi - lo), [N], nw, 1e-6, out_dtype="float32").numpy()
    fused_res = res.numpy()
    assert np.array_equal(fused_res[lo:hi].view(np.uint32), ref_res.numpy()[lo:hi].view(np.uint32))
    assert np.array_equal(h.numpy().view(np.uint32), sep_h.view(np.uint32))
    ref = oracle.linear(xh, wh).astype(np.float64) + r0
    bound = _gemm_bound(xh, wh, K) + 2.0 ** -23 * np.abs(ref)
    assert np.all(np.abs(fused_res[lo:hi] - ref[lo:hi]) <= bound[lo:hi])
    rn = oracle.rms_norm(fused_res[lo:hi], nwh, 1e-6)
    assert np.max(np.abs(h.numpy() - rn)) <= 1e-5 * max(1.0, float(np.max(np.abs(rn))))


@pytest.mark.parametrize("M,I,K", [(512, 3072, 1024), (130, 96, 64), (600, 3072, 1024), (2048, 3072, 1024)])
def test_linear_swiglu_f32_matches_gemm_then_silu_mul(hip, M, I, K):
    """kh_gemm_swiglu with fp32 activations: the gate and up sums are the GEMM's over the plain
    [gate; up] weight bit for bit (same tiles, same k order), and h = silu(g) * u in fp32 without
    rounding g, u or h to bf16 (checked in double from the GEMM's g and u)."""
    from kandle_amd.kernels import interleave_gate_up
    x, _ = seeded(630, (M, K), std=2.0)
    wg_bits, _ = syn.bf16(syn.normal(631, (I, K), 0.05))
    wu_bits, _ = syn.bf16(syn.normal(632, (I, K), 0.05))
    w_cat = Tensor(np.concatenate([wg_bits, wu_bits]), dtype="bfloat16")
    w_il = Tensor(interleave_gate_up(wg_bits, wu_bits), dtype="bfloat16")
    h = F.linear_swiglu(x, w_il)
    assert h.dtype == "float32"
    gu = F.linear(x, w_cat).numpy().astype(np.float64)
    g, u = gu[:, :I], gu[:, I:]
    ref = g / (1.0 + np.exp(-np.clip(g, -88, 88))) * u
    err = np.abs(h.numpy() - ref)
    assert np.all(err <= 2.0 ** -20 * np.abs(ref) + 1e-12), float(np.max(err / (np.abs(ref) + 1e-12)))


@pytest.mark.parametrize("S,H,Hq,Hkv,L,pos0", [(512, 1024, 16, 8, 640, 0), (200, 1024, 16, 8, 204, 10),
                                              (40, 256, 4, 2, 64, 30)])
def test_linear_qk_norm_rope_f32_matches_projection_then_rms_norm_rope(hip, S, H, Hq, Hkv, L, pos0):
    """kh_gemm_qk_norm_rope with fp32 activations (the projection kept in fp32 into qk-norm + RoPE,
    fp32 q rows and caches) against kh_gemm_ex into [S, (Hq + 2 Hkv) 128] then kh_qk_norm_rope in
    fp32 with cache addressing, bit for bit; positions past the cache write no row."""
    from kandle_amd import kernels
    from kandle_amd.tensor import HipTensorHandle

    D = 128
    N = (Hq + 2 * Hkv) * D
    assert kernels.gemm_split_count(S, N, H) == 1
    x, _ = seeded(640, (S, H))
    w, _ = seeded(641, (N, H), "bfloat16", std=0.05)
    wq_bits, wqv = syn.bf16(syn.uniform(642, (D,), 0.5, 1.5))
    wk_bits, wkv = syn.bf16(syn.uniform(643, (D,), 0.5, 1.5))
    wq, wk = Tensor(wq_bits, dtype="bfloat16"), Tensor(wk_bits, dtype="bfloat16")
    wq32, wk32 = Tensor(wqv), Tensor(wkv)
    inv = Tensor(oracle.rope_inv_freq(D, 1e6))
    pos = Tensor(np.arange(pos0, pos0 + S, dtype=np.int32), dtype="int32")
    cache0 = syn.normal(644, (1, Hkv, L, D))

    def caches():
        return Tensor(cache0.copy()), Tensor(cache0.copy())

    qkv = F.linear(x, w)
    assert qkv.dtype == "float32"
    k1, v1 = caches()
    q1 = HipTensorHandle.create_new((1, Hq, S, D), "float32")

    def heads(col, n):
        return HipTensorHandle.create_view(qkv.handle.storage, (1, S, n, D), "float32", (S * N, N, D, 1), col)

    kernels.rms_norm_rope(heads(0, Hq), heads(Hq * D, Hkv), {
        "q_weight": wq32.handle, "k_weight": wk32.handle, "inv_freq": inv.handle, "positions": pos.handle,
        "eps": 1e-6, "q_out": q1, "k_out": k1.handle, "v": heads((Hq + Hkv) * D, Hkv), "v_out": v1.handle,
        "cache_positions": True})
    k2, v2 = caches()
    q2 = HipTensorHandle.create_new((1, Hq, S, D), "float32")
    kernels.linear_qk_norm_rope(x.handle, w.handle, {
        "q_weight": wq.handle, "k_weight": wk.handle, "inv_freq": inv.handle, "positions": pos.handle, "eps": 1e-6,
        "q_out": q2, "k_out": k2.handle, "v_out": v2.handle})
    for a, b in ((Tensor(handle=q1), Tensor(handle=q2)), (k1, k2), (v1, v2)):
        assert np.array_equal(a.numpy().view(np.uint32), b.numpy().view(np.uint32))
    if pos0 + S > L:
        assert np.array_equal(k2.numpy()[:, :, :pos0], cache0[:, :, :pos0])


@pytest.mark.parametrize("prologue", ["none", "rms_norm", "silu_mul", "silu_mul_interleaved"])
@pytest.mark.parametrize("N,K", [(4096, 1024), (1024, 3072), (151936, 1024), (37, 200)])
def test_gemv_fused_f32_activations(hip, prologue, N, K):
    """One-row projections with act_dtype float32: x' formed in fp32 (never rounded to bf16) from
    fp32 inputs, times the bf16 weight, against the oracle's double sums within (2^-20 + K 2^-24)
    sum |x' w| (x' itself carries a few fp32 roundings)."""
    w, wh = seeded(650, (N, K), "bfloat16", std=0.02)
    params = {}
    if prologue == "rms_norm":
        x, xh = seeded(651, (1, K), std=3.0)
        nw_bits, nwv = syn.bf16(syn.uniform(652, (K,), 0.5, 1.5))
        args = dict(norm_weight=Tensor(nw_bits, dtype="bfloat16"), eps=1e-6)
        xp = oracle.rms_norm(xh, nwv, 1e-6)
    elif prologue == "silu_mul":
        x, xh = seeded(651, (1, K), std=2.0)
        x2, x2h = seeded(653, (1, K), std=2.0)
        args = dict(x2=x2)
        xp = (xh / (1.0 + np.exp(-np.clip(xh.astype(np.float64), -88, 88))) * x2h)
    elif prologue == "silu_mul_interleaved":
        if K % 8:
            pytest.skip("interleaved gate/up rows need k % 8 == 0")
        x, xh = seeded(651, (1, 2 * K), std=2.0)
        g = xh.reshape(K // 8, 2, 8)[:, 0].reshape(1, K).astype(np.float64)
        u = xh.reshape(K // 8, 2, 8)[:, 1].reshape(1, K)
        args = {}
        xp = g / (1.0 + np.exp(-np.clip(g, -88, 88))) * u
    else:
        x, xh = seeded(651, (1, K), std=2.0)
        args = {}
        xp = xh
    del params
    y = F.linear_fused(prologue, x, w, out_dtype="float32", act_dtype="float32", **args).numpy()
    ref = (np.asarray(xp, np.float64) @ wh.astype(np.float64).T)
    bound = (2.0 ** -20 + K * 2.0 ** -24) * (np.abs(np.asarray(xp, np.float64)) @ np.abs(wh.astype(np.float64)).T)
    assert np.all(np.abs(y - ref) <= bound + 1e-30), float(np.max(np.abs(y - ref) / (bound + 1e-30)))


@pytest.mark.parametrize("prologue", ["rms_norm", "none"])
def test_gemv_swiglu_f32_matches_gate_up_row(hip, prologue):
    """kh_gemv_swiglu with fp32 activations: h = silu(g) * u of the same fp32 gate / up sums the
    one-row projection forms (bit for bit), unrounded; the down projection reads h as an fp32 row."""
    from kandle_amd.kernels import interleave_gate_up
    I, K = 3072, 1024
    if prologue == "rms_norm":
        x = Tensor(syn.normal(660, (1, K), 3.0))
        nw = Tensor(syn.bf16(syn.uniform(661, (K,), 0.5, 1.5))[0], dtype="bfloat16")
    else:
        x, _ = seeded(660, (1, K), std=2.0)
        nw = None
    _, gh = seeded(662, (I, K), "bfloat16", std=0.05)
    _, uh = seeded(663, (I, K), "bfloat16", std=0.05)
    w_gu = Tensor(syn.bf16(interleave_gate_up(gh, uh))[0], dtype="bfloat16")
    a = F.linear_swiglu_row(prologue, x, w_gu, nw, 1e-6, act_dtype="float32")
    assert a.dtype == "float32"
    gu = F.linear_fused(prologue, x, w_gu, nw, 1e-6, act_dtype="float32")       # [1, 2I] interleaved, fp32
    gv = gu.numpy().reshape(I // 8, 2, 8).astype(np.float64)
    g, u = gv[:, 0].reshape(-1), gv[:, 1].reshape(-1)
    ref = g / (1.0 + np.exp(-np.clip(g, -88, 88))) * u
    av = a.numpy().reshape(-1)
    assert np.all(np.abs(av - ref) <= 2.0 ** -20 * np.abs(ref) + 1e-12)
    w_d, wdh = seeded(664, (1024, I), "bfloat16", std=0.02)
    y = F.linear_fused("none", a, w_d, out_dtype="float32", act_dtype="float32").numpy()
    r = av.astype(np.float64) @ wdh.astype(np.float64).T
    bound = (2.0 ** -20 + I * 2.0 ** -24) * (np.abs(av).astype(np.float64) @ np.abs(wdh).astype(np.float64).T)
    assert np.all(np.abs(y - r) <= bound + 1e-30)
