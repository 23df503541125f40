"""GPU parity of the iterator kernels under Kandle's calling convention (register.ts:9: (iter) => void):
operands carry element strides aligned to the output shape (0 on broadcast axes) and element
offsets (packages/types/src/tensor.ts:282-378, built as core/src/dispatch/TensorIterator.ts builds
them), and the kernel writes iter.output().tensor_handle.

Kernels: add / sub (alpha) / mul / div / neg / cos / sin / silu (pointwise/ops.ts), copy / cast /
contiguous / clone / copy_ (copy/index.ts:13-33), zeros / ones / full / empty / arange (factory
handlers, arangeExecutor.ts:37-44) and argmax (reduction/index.ts:20-22) over any axis.
Bars: copies, casts, int32 arithmetic and argmax bit-exact; fp32 arithmetic equal to numpy's fp32
result (one rounding per op, the same op order); transcendental ops within 2e-6 of float64.
"""
import numpy as np
import pytest

import oracle
from kandle_amd import HipTensorHandle, Tensor, kernels
from kandle_amd import synthetic as syn
from kandle_amd.kernels import TensorIterator

pytestmark = pytest.mark.gpu


def _view(t, shape, strides, offset):
    return HipTensorHandle.create_view(t.handle.storage, shape, t.dtype, strides, offset)


def _np_view(a, shape, strides, offset):
    flat = a.reshape(-1)
    return np.lib.stride_tricks.as_strided(flat[offset:], shape=shape, strides=[s * flat.itemsize for s in strides])


def test_binary_broadcast_strided_and_offset_operands(hip):
    """a: a permuted [2, 5, 4, 3] view of a [2, 3, 4, 5] buffer; b: [4, 1] broadcast over the rest,
    read through a view with an element offset; add with alpha 2, sub with alpha 0.5, mul, div."""
    base = syn.normal(900, (2, 3, 4, 5))
    tb = Tensor(base)
    a = _view(tb, (2, 5, 4, 3), (60, 1, 5, 20), 0)              # permute(0, 3, 2, 1)
    an = base.transpose(0, 3, 2, 1)
    braw = syn.normal(901, (10,)) + 3.0
    tbr = Tensor(braw)
    b = _view(tbr, (4, 1), (2, 1), 1)                              # elements 1, 3, 5, 7
    bn = braw[1:9:2].reshape(4, 1)
    for name, alpha, ref in (("add", 2.0, an + np.float32(2.0) * bn), ("sub", 0.5, an - np.float32(0.5) * bn),
                             ("mul", None, an * bn), ("div", None, an / bn)):
        it = TensorIterator.binary_op(a, b, scalar_args=None if alpha is None else {"alpha": alpha})
        assert it.output_shape == (2, 5, 4, 3) and it.input(1).strides == (0, 0, 2, 0)
        kernels.KERNELS[name](it)
        got = it.output().tensor_handle.data_async()
        assert np.array_equal(got, ref.astype(np.float32)), name


def test_mixed_dtypes_promote_and_bf16(hip):
    """bf16 * f32 -> f32 (promotion); bf16 + bf16 -> bf16 rounded once."""
    x = syn.normal(902, (7, 33))
    xb_bits, xb = syn.bf16(x)
    y = syn.normal(903, (33,))
    tx = Tensor(xb_bits, dtype="bfloat16")
    ty = Tensor(y)
    it = TensorIterator.binary_op(tx.handle, ty.handle)
    kernels.mul(it)
    assert it.output().tensor_handle.dtype == "float32"
    assert np.array_equal(it.output().tensor_handle.data_async(), xb * y)
    it2 = TensorIterator.binary_op(tx.handle, tx.handle)
    kernels.add(it2)
    assert it2.output().tensor_handle.dtype == "bfloat16"
    assert np.array_equal(it2.output().tensor_handle.data_async(), oracle.bf16_round(xb + xb))


def test_unary_ops_on_strided_views(hip):
    base = syn.normal(904, (64, 48), 3.0)
    tb = Tensor(base)
    v = _view(tb, (48, 32), (1, 48), 96)                           # a transposed window
    vn = _np_view(base, (48, 32), (1, 48), 96).astype(np.float64)
    for name, fn, tol in (("neg", np.negative, 0.0), ("cos", np.cos, 2e-6), ("sin", np.sin, 2e-6),
                          ("silu", lambda z: z / (1.0 + np.exp(-np.clip(z, -88, 88))), 2e-6)):
        it = TensorIterator.unary_op(v)
        kernels.KERNELS[name](it)
        got = it.output().tensor_handle.data_async()
        assert np.max(np.abs(got - fn(vn))) <= tol * max(1.0, float(np.max(np.abs(fn(vn))))), name


def test_copy_family_casts_and_strided_outputs(hip):
    """cast f32 -> bf16 (RNE) / bf16 -> f32 (exact) / f32 -> int32 (truncation toward zero) /
    int32 -> f32; contiguous of a permuted view; clone; copy_ into a strided window with an offset,
    the rest of the buffer untouched."""
    x = syn.normal(905, (6, 10), 50.0)
    x[0, :4] = [2.5, -2.5, 0.99, -0.99]
    tx = Tensor(x)
    outs = {}
    for dt in ("bfloat16", "int32"):
        o = HipTensorHandle.create_new((6, 10), dt)
        kernels.cast(TensorIterator.unary_op(tx.handle, o))
        outs[dt] = o.data_async()
    assert np.array_equal(outs["bfloat16"], oracle.bf16_round(x))
    assert np.array_equal(outs["int32"], np.trunc(x).astype(np.int32))
    ti = Tensor(np.arange(-30, 30, dtype=np.int32).reshape(6, 10), dtype="int32")
    of = HipTensorHandle.create_new((6, 10), "float32")
    kernels.cast(TensorIterator.unary_op(ti.handle, of))
    assert np.array_equal(of.data_async(), np.arange(-30, 30, dtype=np.float32).reshape(6, 10))
    perm = _view(tx, (10, 6), (1, 10), 0)
    oc = HipTensorHandle.create_new((10, 6), "float32")
    kernels.contiguous(TensorIterator.unary_op(perm, oc))
    assert np.array_equal(oc.data_async(), x.T)
    ocl = HipTensorHandle.create_new((6, 10), "float32")
    kernels.clone(TensorIterator.unary_op(tx.handle, ocl))
    assert np.array_equal(ocl.data_async(), x)
    buf = np.full((8, 16), -7.0, np.float32)
    tbuf = Tensor(buf)
    win = _view(tbuf, (6, 10), (16, 1), 17)                        # rows 1..6, cols 1..10
    kernels.copy_(TensorIterator.unary_op(tx.handle, win))
    want = buf.copy()
    want[1:7, 1:11] = x
    assert np.array_equal(tbuf.numpy(), want)
    # a source broadcast into the window (copy_ of a row vector)
    row = Tensor(np.arange(10, dtype=np.float32))
    kernels.copy_(TensorIterator.unary_op(row.handle, win))
    want[1:7, 1:11] = np.arange(10, dtype=np.float32)
    assert np.array_equal(tbuf.numpy(), want)


def test_factories_and_int32_arithmetic(hip):
    for name, sc, val in (("zeros", None, 0.0), ("ones", None, 1.0), ("full", {"fill_value": -2.5}, -2.5)):
        it = TensorIterator.nullary_op((3, 5), "float32", scalar_args=sc)
        kernels.KERNELS[name](it)
        assert np.array_equal(it.output().tensor_handle.data_async(), np.full((3, 5), val, np.float32))
    it = TensorIterator.nullary_op((1000,), "float32", scalar_args={"start": 0.5, "end": 250.5, "step": 0.25})
    kernels.arange(it)
    i = np.arange(1000)
    assert np.array_equal(it.output().tensor_handle.data_async(), np.float32(0.5) + i.astype(np.float32) * np.float32(0.25))
    it = TensorIterator.nullary_op((100,), "int32", scalar_args={"start": -7, "step": 3})
    kernels.arange(it)
    assert np.array_equal(it.output().tensor_handle.data_async(), (-7 + 3 * np.arange(100)).astype(np.int32))
    a = Tensor(np.array([2147483647, -5, 7, 1 << 20], np.int32), dtype="int32")
    b = Tensor(np.array([1, 3, -2, 1 << 12], np.int32), dtype="int32")
    with np.errstate(over="ignore"):
        for name, ref in (("add", a.numpy() + b.numpy()), ("sub", a.numpy() - b.numpy()),
                          ("mul", a.numpy() * b.numpy())):
            it = TensorIterator.binary_op(a.handle, b.handle)
            kernels.KERNELS[name](it)
            assert np.array_equal(it.output().tensor_handle.data_async(), ref.astype(np.int32)), name


@pytest.mark.parametrize("axes,keep", [([0], False), ([1], True), ([2], False), ([-1], False), (None, False), ([0, 2], False)])
def test_argmax_reduction_iterator_any_axis(hip, axes, keep):
    """argmax over any axes of a [5, 7, 300] input read through a permuted view (no materialised
    copy by the caller), ties resolved to the lowest index, keepdim."""
    x = syn.normal(906, (300, 7, 5))
    x[3, 2, 1] = x[200, 2, 1] = 50.0                     # a tie along axis 0 of the permuted view
    tx = Tensor(x)
    v = _view(tx, (5, 7, 300), (1, 5, 35), 0)            # x.transpose(2, 1, 0)
    vn = x.transpose(2, 1, 0)
    it = TensorIterator.reduction_op(v, axes, keep, out_dtype="int32")
    kernels.argmax(it)
    got = it.output().tensor_handle.data_async()
    nd = 3
    red = list(range(nd)) if not axes else sorted(a % nd for a in axes)
    kept = [i for i in range(nd) if i not in red]
    rows = vn.transpose(kept + red).reshape(int(np.prod([vn.shape[i] for i in kept])) if kept else 1, -1)
    ref = oracle.argmax(np.ascontiguousarray(rows))
    assert np.array_equal(got.reshape(-1), ref)
    if keep:
        assert got.shape == tuple(1 if i in red else vn.shape[i] for i in range(nd))


def test_iterator_rejects_bad_geometry(hip):
    x = Tensor(np.zeros((4, 4), np.float32))
    with pytest.raises(ValueError, match="broadcasts"):
        kernels.copy_(TensorIterator([Tensor(np.zeros(4, np.float32)).handle],
                                     [_view(x, (4, 4), (0, 1), 0)]))   # the output repeats a row
    with pytest.raises(ValueError, match="reaches elements"):
        _view(x, (4, 5), (4, 1), 0)                                   # runs past the storage
