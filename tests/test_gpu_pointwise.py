"""GPU parity of the pointwise/factory kernels Kandle's composite RoPE calls by name (neg, cos, sin,
arange; cat is copies into slices), and of that composite against the fused qk-norm + RoPE kernel.

References: packages/backend-webgpu/src/kernels/pointwise/ops.ts:168 neg, :201 sin, :202 cos;
packages/backend-webgpu/src/kernels/factory/arangeShaderBuilder.ts:66-78 (start + f32(i) * step);
packages/model-utils/src/rope.ts:159-255, 546-644 (the composite).  Bars: neg exact; cos/sin in
fp32 within 2e-6 of float64 cos/sin of the stored input, bf16 within one bf16 rounding (2^-8
relative of a value in [-1, 1]); arange bit-exact in f32 (two roundings), bf16 and int32.
"""
import numpy as np
import pytest

import oracle
from helpers import dev
from kandle_amd import HipTensorHandle, Tensor, kernels
from kandle_amd import functional as F
from kandle_amd import synthetic as syn

pytestmark = pytest.mark.gpu


def test_neg_cos_sin_f32_and_bf16(hip):
    x = syn.normal(801, (4099,), 4.0)
    x[:6] = [0.0, -0.0, 1000.5, -8191.0, 3.14159265, 1e-30]
    for dtype in ("float32", "bfloat16"):
        t = dev(x, dtype)
        xs = t.numpy().astype(np.float64)  # the stored values
        n, c, s = F.neg(t).numpy(), F.cos(t).numpy(), F.sin(t).numpy()
        assert np.array_equal(n, -t.numpy())
        tol = 2e-6 if dtype == "float32" else 2.0 ** -8
        assert float(np.max(np.abs(c - np.cos(xs)))) <= tol
        assert float(np.max(np.abs(s - np.sin(xs)))) <= tol


def test_arange_matches_reference_formula(hip):
    for dtype, start, step, n in (("float32", 0.5, 0.25, 5000), ("float32", -3.0, 0.1, 777),
                                  ("bfloat16", 2.0, 0.5, 300), ("int32", -5, 3, 1000)):
        t = F.arange(start, start + step * n, step, dtype=dtype)
        got = t.numpy()
        assert got.shape == (n,)
        i = np.arange(n)
        if dtype == "int32":
            ref = (start + i * step).astype(np.int32)
        else:
            ref = np.float32(start) + np.float32(i).astype(np.float32) * np.float32(step)  # two f32 roundings
            if dtype == "bfloat16":
                ref = oracle.bf16_round(ref)
        assert np.array_equal(got, ref), dtype
    assert F.arange(0.0, 0.0).shape == (0,)


def test_composite_rope_from_registered_ops_matches_fused_kernel(hip):
    """Kandle's RotaryEmbedding + applyRotaryPosEmbDirect composite (rope.ts:159-255, 546-644) built
    from the registered kernels (arange, mul, copy into slices for cat, cos, sin, neg, add) equals
    the fused qk-norm + RoPE kernel with unit norm weights applied to already-normalised rows."""
    T, H, D, theta = 96, 4, 128, 1e6
    x = syn.normal(802, (T, H, D))
    x /= np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + 1e-6)   # unit RMS: the norm is ~identity
    inv = oracle.rope_inv_freq(D, theta)
    # composite on the device, fp32
    pos = F.arange(0.0, float(T))                                  # [T]
    freqs = F.mul(F.view(pos, (T, 1)), F.view(Tensor(inv), (1, D // 2)))  # [T, 64], f32 product
    emb = Tensor(handle=HipTensorHandle.create_new((T, D), "float32"))
    F.copy_(F.narrow(emb, 1, 0, D // 2), freqs)                    # cat(freqs, freqs)
    F.copy_(F.narrow(emb, 1, D // 2, D // 2), freqs)
    cos_t, sin_t = F.cos(emb), F.sin(emb)                          # [T, D]
    xt = dev(x)
    x1, x2 = F.narrow(xt, 2, 0, D // 2), F.narrow(xt, 2, D // 2, D // 2)
    rot = Tensor(handle=HipTensorHandle.create_new((T, H, D), "float32"))
    F.copy_(F.narrow(rot, 2, 0, D // 2), F.neg(x2))                # cat(-x2, x1)
    F.copy_(F.narrow(rot, 2, D // 2, D // 2), x1)
    c3, s3 = F.view(cos_t, (T, 1, D)), F.view(sin_t, (T, 1, D))
    out = F.add(F.mul(xt, c3), F.mul(rot, s3)).numpy()
    # the oracle's fused restatement (norm + rope) with unit weights on unit-RMS rows
    ref = oracle.qk_norm_rope(x, None, np.arange(T, dtype=np.int32), inv, 1e-6)
    assert float(np.max(np.abs(out - ref))) < 1e-4
    # and the fused kernel in fp32 through the backend
    qo, _ = kernels.rms_norm_rope(Tensor(x.reshape(1, T, H, D)).handle, Tensor(x[:, :1].reshape(1, T, 1, D)).handle, {
        "q_weight": Tensor(np.ones(D, np.float32)).handle, "k_weight": Tensor(np.ones(D, np.float32)).handle,
        "inv_freq": Tensor(inv).handle, "positions": Tensor(np.arange(T, dtype=np.int32), dtype="int32").handle,
        "eps": 1e-6})
    fused = qo.data_async()[0].transpose(1, 0, 2)
    assert float(np.max(np.abs(out - fused))) < 1e-4
