"""GPU parity of the support kernels (pointwise, copies, gather, argmax, GEMM) and the allocator."""
import numpy as np
import pytest

import oracle
from helpers import max_rel, seeded
from kandle_amd import HipBackend, Tensor
from kandle_amd import functional as F
from kandle_amd import synthetic as syn

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_add_mul_broadcast(hip, dtype):
    a, ah = seeded(201, (3, 5, 64), dtype)
    b, bh = seeded(202, (5, 64), dtype)
    s = F.add(a, b).numpy()
    m = F.mul(a, b).numpy()
    rs, rm = ah + bh, ah * bh
    if dtype == "bfloat16":
        rs, rm = oracle.bf16_round(rs), oracle.bf16_round(rm)
    np.testing.assert_allclose(s, rs, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(m, rm, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_silu_mul(hip, dtype):
    g, gh = seeded(210, (7, 3072), dtype, std=4.0)
    u, uh = seeded(211, (7, 3072), dtype)
    y = F.silu_mul(g, u).numpy()
    ref = oracle.silu_mul(gh, uh)
    if dtype == "float32":
        assert max_rel(y, ref) < 1e-5
    else:
        assert np.all(np.abs(y - ref) <= 2 ** -8 * np.abs(ref) + 1e-6)
    s = F.silu(g).numpy()
    refs = oracle.silu_mul(gh)
    tol = 1e-5 if dtype == "float32" else 2 ** -8
    assert np.all(np.abs(s - refs) <= tol * np.abs(refs) + 1e-6)


def test_silu_mul_strided_halves_of_fused_gate_up(hip):
    gu, guh = seeded(212, (5, 2 * 256), "bfloat16")
    g = F.narrow(gu, 1, 0, 256)
    u = F.narrow(gu, 1, 256, 256)
    y = F.silu_mul(g, u).numpy()
    ref = oracle.silu_mul(guh[:, :256], guh[:, 256:])
    assert np.all(np.abs(y - ref) <= 2 ** -8 * np.abs(ref) + 1e-6)


def test_cast_to_bf16_rounding_edge_cases(hip):
    """The device float32 -> bf16 conversion (one v_cvt_pk_bf16_f32 per pair) rounds to nearest even
    bit for bit like the oracle: ties both ways, carries into the exponent, overflow to infinity,
    subnormals, signed zeros; NaN stays NaN."""
    tie = np.float32(1.0) + np.float32(2.0 ** -8)            # exactly half an ulp above 1 -> 1
    vals = np.array([0.0, -0.0, 1.0, tie, 1.0 + 3 * 2.0 ** -8, 1.0 + 2 ** -8 + 2 ** -20, -tie,
                     1.9999999, 3.3895e38, 3.4028235e38, -3.4028235e38, np.inf, -np.inf,
                     1e-40, -3e-39, 9.18e-41, 1.1754942e-38, 1.17549435e-38, 5.9e-39, 65504.0, 1e10,
                     np.nan, -np.nan], np.float32)
    x = np.concatenate([vals, syn.normal(225, (997,)) * np.float32(1e3)]).astype(np.float32)
    y = F.cast(Tensor(x), "bfloat16").numpy()
    ref = oracle.bf16_round(x)
    nan = np.isnan(x)
    np.testing.assert_array_equal(np.isnan(y), nan)
    np.testing.assert_array_equal(y[~nan].view(np.uint32), ref[~nan].view(np.uint32))


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_contiguous_cast_of_permuted_view(hip, dtype):
    x, xh = seeded(220, (2, 3, 4, 8), dtype)
    p = F.permute(x, (0, 2, 1, 3))
    np.testing.assert_array_equal(F.contiguous(p).numpy(), np.transpose(xh, (0, 2, 1, 3)))
    other = "float32" if dtype == "bfloat16" else "bfloat16"
    c = F.cast(p, other).numpy()
    ref = np.transpose(xh, (0, 2, 1, 3))
    np.testing.assert_array_equal(c, oracle.bf16_round(ref) if other == "bfloat16" else ref)


def test_copy_into_strided_cache_slice(hip):
    cache = F.zeros((1, 2, 16, 8), "float32")
    src, sh = seeded(221, (1, 2, 3, 8))
    F.copy_(F.narrow(cache, 2, 5, 3), src)
    c = cache.numpy()
    np.testing.assert_array_equal(c[:, :, 5:8], sh)
    assert np.all(c[:, :, :5] == 0) and np.all(c[:, :, 8:] == 0)


def test_embedding_and_argmax(hip):
    V, H = 1000, 64
    table, th = seeded(230, (V, H), "bfloat16")
    ids = syn.randint(231, (2, 7), 0, V)
    e = F.embedding(Tensor(ids, dtype="int32"), table).numpy()
    np.testing.assert_array_equal(e, th[ids])
    ids_bad = np.array([3, -1, V, 0], np.int32)      # ids outside the table give zero rows
    e32 = F.embedding(Tensor(ids_bad, dtype="int32"), table, out_dtype="float32")
    assert e32.dtype == "float32"
    ref = th[np.clip(ids_bad, 0, V - 1)].copy()
    ref[1:3] = 0.0
    np.testing.assert_array_equal(e32.numpy(), ref)
    x = syn.normal(232, (3, 151936))
    x[1, 5] = x[1, 77] = 100.0  # tie: lowest index wins
    x[2, :] = -np.inf
    x[2, 9] = np.nan
    a = F.argmax(Tensor(x)).numpy()
    np.testing.assert_array_equal(a, oracle.argmax(x))
    assert a[1] == 5 and a[2] == 0


@pytest.mark.parametrize("M,N,K", [(512, 1024, 1024), (130, 200, 72), (8, 3000, 1024), (1, 151936, 1024),
                                   (3, 100, 30), (600, 4096, 2048), (2048, 2048, 256), (1000, 4100, 136)])
def test_linear_bf16(hip, M, N, K):
    x, xh = seeded(240, (M, K), "bfloat16")
    w, wh = seeded(241, (N, K), "bfloat16", std=0.02)
    y = F.linear(x, w).numpy()
    ref = oracle.linear(xh, wh)
    err = np.abs(y - ref)
    # one bf16 rounding of the output plus fp32 accumulation-order noise
    assert np.all(err <= 2 ** -8 * np.abs(ref) + 1e-4 * np.sqrt(K) * 0.02 * 4), float(err.max())


@pytest.mark.parametrize("M,N,K", [(512, 1024, 3072), (100, 520, 2048)])
def test_linear_split_k_residual_deterministic(hip, M, N, K):
    """Few output tiles and a long K: workgroups split K and write fp32 partials, and a second
    kernel adds them in split order to the residual in place -- bit-identical results over four
    runs, with another split GEMM of a different tile count between them (the partial buffer is
    reused with another layout)."""
    x, xh = seeded(245, (M, K), "bfloat16")
    w, wh = seeded(246, (N, K), "bfloat16", std=0.02)
    x2, _ = seeded(248, (64, 2048), "bfloat16")
    w2, _ = seeded(249, (96, 2048), "bfloat16", std=0.02)
    r0 = syn.normal(247, (M, N))
    outs, others = [], []
    for _ in range(4):
        r = Tensor(r0.copy())
        F.dispatch_matmul(x, w, c=r, beta=1.0, out=r, transpose_b=True)
        outs.append(r.numpy())
        r.dispose()
        others.append(F.dispatch_matmul(x2, w2, transpose_b=True).numpy())
    assert all(np.array_equal(outs[0], o) for o in outs[1:])
    assert all(np.array_equal(others[0], o) for o in others[1:])
    ref = oracle.linear(xh, wh) + r0
    assert max_rel(outs[0], ref) < 1e-4


def test_linear_fp32_bias_and_residual_epilogue(hip):
    x, xh = seeded(250, (33, 96))
    w, wh = seeded(251, (40, 96))
    b, bh = seeded(252, (40,))
    c, ch = seeded(253, (33, 40))
    y = F.linear(x, w, b).numpy()
    assert max_rel(y, oracle.linear(xh, wh, bias=bh)) < 1e-5
    z = F.dispatch_matmul(x, w, c=c, alpha=0.5, beta=2.0, transpose_b=True).numpy()
    assert max_rel(z, oracle.linear(xh, wh, cin=ch, alpha=0.5, beta=2.0)) < 1e-5


def test_matmul_batched_fp32(hip):
    a, ah = seeded(260, (3, 17, 24))
    b, bh = seeded(261, (3, 24, 9))
    y = F.matmul(a, b).numpy()
    assert max_rel(y, np.einsum("bmk,bkn->bmn", ah.astype(np.float64), bh)) < 1e-5


@pytest.mark.parametrize("dim", [0, 1, 2, -1])
@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_index_select_any_dim(hip, dim, dtype):
    """index_select along every dim of a 3-d tensor (gather.ts:121,190), ids out of range giving zeros,
    and a permuted (non-contiguous) source."""
    x, xh = seeded(60, (5, 7, 9), dtype)
    n = xh.shape[dim]
    idx = np.array([n - 1, 0, 2, 2, n, -1], np.int32)
    out = F.index_select(x, dim, Tensor(idx, dtype="int32")).numpy()
    ref = np.take(xh, np.clip(idx, 0, n - 1), axis=dim)
    bad = (idx < 0) | (idx >= n)
    sl = [slice(None)] * 3
    sl[dim] = bad
    ref[tuple(sl)] = 0.0
    assert np.array_equal(out, ref)
    xp = F.permute(x, [2, 0, 1])
    out2 = F.index_select(xp, 1, Tensor(np.array([4, 1], np.int32), dtype="int32")).numpy()
    assert np.array_equal(out2, np.take(np.transpose(xh, (2, 0, 1)), [4, 1], axis=1))


@pytest.mark.parametrize("dim", [0, 1, 2])
def test_argmax_any_dim(hip, dim):
    """argmax over a non-last dim (moved last and materialised), lowest index on ties."""
    xh = np.round(syn.normal(61, (6, 50, 33)) * 2).astype(np.float32)   # many ties
    out = F.argmax(Tensor(xh), dim).numpy()
    assert np.array_equal(out, np.argmax(xh, axis=dim).astype(np.int32))


def test_matmul_transpose_a_and_detected_transpose_b(hip):
    """The matmul kernel with config.transpose_a (A stored [K, M]) and with B passed as a transposed
    view of a row-major [N, K] weight (taken as the transposed operand, not copied), bf16 and fp32."""
    from kandle_amd import kernels
    for dtype in ("float32", "bfloat16"):
        M, K, N = 130, 256, 72
        at, ath = seeded(62, (K, M), dtype)           # A^T stored
        w, wh = seeded(63, (N, K), dtype, std=0.05)   # B^T stored, passed as the view w^T [K, N]
        out = F.dispatch_matmul(at, F.transpose(w, 0, 1), transpose_a=True).numpy()
        ref = oracle.linear(np.ascontiguousarray(ath.T), wh)
        tol = 1e-4 if dtype == "float32" else 2e-2
        assert max_rel(out, ref) < tol, dtype
        # the kernel called as a dispatcher would with MatmulDispatchResult.transposeA set
        o = F.zeros((M, N), dtype)
        cfg = kernels.MatmulDispatchResult(variant="mm", output=o.handle, M=M, K=K, N=N, batch_shape=(),
                                           batch_size=1, transpose_a=True, transpose_b=True, alpha=1.0, beta=0.0)
        kernels.matmul(cfg, at.handle, w.handle)
        assert max_rel(o.numpy(), ref) < tol, dtype


def test_allocator_reuses_freed_blocks(hip):
    before = HipBackend.memory_stats()
    t = Tensor(np.zeros(1 << 20, np.float32))
    live = HipBackend.memory_stats()["live_bytes"]
    t.dispose()
    t2 = Tensor(np.zeros(1 << 20, np.float32))
    after = HipBackend.memory_stats()
    assert after["n_cache_hits"] > before["n_cache_hits"]
    assert after["live_bytes"] == live
    t2.dispose()


def test_tidy_returns_intermediate_device_memory(hip):
    """tidy around real ops: the intermediates' blocks go back to the allocator (live bytes return
    to the level before the scope plus the returned tensor), the returned and kept tensors stay
    usable (memory.ts:83-119, :190-193)."""
    from kandle_amd import _lib, keep, tidy

    x, xh = seeded(70, (256, 256))
    base = _lib.alloc_stats()["live_bytes"]
    kept = {}

    def body():
        kept["y"] = F.silu(x)                           # intermediate
        kept["z"] = F.add(kept["y"], x)                 # intermediate
        kept["k"] = keep(F.mul(kept["z"], kept["z"]))
        return F.mul(kept["z"], x)

    out = tidy(body)
    assert kept["y"].is_disposed and kept["z"].is_disposed
    assert not out.is_disposed and not kept["k"].is_disposed
    # The allocator hands out a cached block of up to twice the request, so the two survivors hold
    # between 2 and 4 times 256 KiB; the two intermediates' blocks are back in the cache.
    live = _lib.alloc_stats()["live_bytes"]
    assert 2 * 256 * 256 * 4 <= live - base <= 4 * 256 * 256 * 4, (live, base)
    silu = xh / (1 + np.exp(-np.clip(xh, -88, 88)))
    np.testing.assert_allclose(out.numpy(), (silu + xh) * xh, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(kept["k"].numpy(), (silu + xh) ** 2, rtol=1e-5, atol=1e-5)
    out.dispose()
    kept["k"].dispose()
    assert _lib.alloc_stats()["live_bytes"] == base
