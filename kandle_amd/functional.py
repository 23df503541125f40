"""User-facing ops for the hot path (Tensor in, Tensor out), restating Kandle's dispatch layer.

Each op validates and routes exactly as the reference dispatcher does, allocates its output through
the active backend and calls the kernel it finds BY NAME in the backend's registry (a missing kernel
raises: there is no fallback implementation here):
  scaled_dot_product_attention  packages/core/src/dispatch/handlers/composite.ts:247-348
  linear                        packages/core/src/dispatch/handlers/composite.ts:55-77
  matmul                        packages/core/src/dispatch/matmulOps.ts:408-496, :649-814
  rms_norm                      packages/core/src/dispatch/handlers/normalize.ts:46-95
  silu / mul / add              packages/core/src/dispatch/handlers/iterator.ts:24-135
  contiguous / cast / copy_     packages/core/src/dispatch/handlers/copy.ts:40-71, :123-138
  embedding                     packages/core/src/dispatch/handlers/composite.ts:149-245
  views                         packages/core/src/dispatch/handlers/shape.ts (metadata only)
"""
from __future__ import annotations

import math
import warnings
from typing import Optional, Sequence

import numpy as np

from . import env
from .kernels import MatmulDispatchResult, TensorIterator
from .tensor import HipTensorHandle, Tensor, contiguous_strides, numel_of


def _backend(t: Tensor):
    return env.get_backend(t.device)


def _kernel(t: Tensor, name: str):
    k = _backend(t).operators.find(name)
    if k is None:
        raise RuntimeError(f"kernel {name!r} is not registered for device {t.device}")
    return k


def _new(t: Tensor, shape, dtype=None) -> HipTensorHandle:
    return _backend(t).create_tensor_handle(tuple(shape), dtype or t.dtype)


def _wrap(h: HipTensorHandle) -> Tensor:
    return Tensor(handle=h)


# ---------------------------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------------------------
def scaled_dot_product_attention(query: Tensor, key: Tensor, value: Tensor, attn_mask: Optional[Tensor] = None,
                                 dropout_p: float = 0.0, is_causal: bool = False,
                                 scale: Optional[float] = None, out: Optional[Tensor] = None) -> Tensor:
    """softmax(scale * Q K^T [+ causal | + attn_mask]) V.  q (..., L, E), k (..., S, E),
    v (..., S, Ev) -> (..., L, Ev).

    Like the reference: dropout_p > 0 is warned about and ignored (inference), the default scale is
    1/sqrt(E), the `flash_attention` kernel is found by name, and an explicit attn_mask takes the
    masked route (added to the scaled scores, is_causal ignored, composite.ts:279-300), which this
    backend runs as the fused `sdpa_masked` kernel instead of matmul -> add -> softmax -> matmul."""
    if dropout_p > 0:
        warnings.warn("SDPA: dropout_p > 0 is not supported in inference mode, ignoring")
    E = query.shape[-1]
    if scale is None:
        scale = 1.0 / math.sqrt(E)
    out_shape = tuple(query.shape[:-1]) + (value.shape[-1],)
    output = out.handle if out is not None else _new(query, out_shape)
    if attn_mask is not None:
        _kernel(query, "sdpa_masked")(query.handle, key.handle, value.handle, attn_mask.handle, output,
                                      float(scale))
    else:
        _kernel(query, "flash_attention")(query.handle, key.handle, value.handle, output, float(scale),
                                          bool(is_causal))
    return out if out is not None else _wrap(output)


def decode_attention(q: Tensor, k_cache: Tensor, v_cache: Tensor, seq_lens: Tensor,
                     scale: Optional[float] = None) -> Tensor:
    """Varlen 1-token decode: q [B, Hq, D] against caches [B, Hkv, max_len, D] with seq_lens [B]."""
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    output = _new(q, q.shape)
    _kernel(q, "decode_attention")(q.handle, k_cache.handle, v_cache.handle, seq_lens.handle, output, float(scale))
    return _wrap(output)


# ---------------------------------------------------------------------------------------------
# matmul / linear
# ---------------------------------------------------------------------------------------------
def dispatch_matmul(a: Tensor, b: Tensor, c: Optional[Tensor] = None, alpha: float = 1.0, beta: float = 0.0,
                    out: Optional[Tensor] = None, transpose_a: bool = False, transpose_b: bool = False,
                    bias: Optional[Tensor] = None, out_dtype: Optional[str] = None) -> Tensor:
    """out = alpha * a @ op(b) + beta * c (+ bias).  With transpose_b, b is stored [..., N, K].
    out_dtype (default: the input dtype) may be float32 for bfloat16 inputs."""
    if a.device != b.device:
        raise RuntimeError(f"matmul requires tensors on same device, got {a.device} and {b.device}")
    for t, nm in ((a, "a"), (b, "b")):
        if t.dtype not in ("float32", "bfloat16"):
            raise TypeError(f"matmul does not support dtype {t.dtype}")
    if beta != 0.0 and c is None:
        raise ValueError(f"matmul: beta={beta} requires inputC to be provided")
    if transpose_a:
        a = transpose(a, -1, -2)
    ash, bsh = list(a.shape), list(b.shape)
    if len(ash) < 1 or len(bsh) < 1:
        raise ValueError("matmul: scalars are not matrices")
    a2 = ash if len(ash) >= 2 else [1] + ash
    if transpose_b:
        b2 = bsh if len(bsh) >= 2 else bsh + [1]
        N, Kb = b2[-2], b2[-1]
    else:
        b2 = bsh if len(bsh) >= 2 else bsh + [1]
        Kb, N = b2[-2], b2[-1]
    M, K = a2[-2], a2[-1]
    if K != Kb:
        raise ValueError(f"matmul: inner dimensions differ ({K} vs {Kb}) for {tuple(ash)} @ {tuple(bsh)}")
    batch_shape = list(np.broadcast_shapes(tuple(a2[:-2]), tuple(b2[:-2])))
    out_shape = batch_shape + [M, N]
    if len(ash) == 1:
        out_shape.pop(-2)
    if len(bsh) == 1:
        out_shape.pop(-1)
    if out is not None:
        if tuple(out.shape) != tuple(out_shape):
            raise ValueError(f"matmul: out shape {out.shape} != {tuple(out_shape)}")
        output = out.handle
    else:
        output = _new(a, out_shape, out_dtype)
    variant = "mm" if not batch_shape else "bmm"
    cfg = MatmulDispatchResult(variant=variant, output=output, M=M, K=K, N=N, batch_shape=tuple(batch_shape),
                               batch_size=int(np.prod(batch_shape)) if batch_shape else 1, transpose_a=False,
                               transpose_b=bool(transpose_b), alpha=float(alpha), beta=float(beta),
                               input_c=c.handle if c is not None else None,
                               bias=bias.handle if bias is not None else None)
    ah = a.handle if len(ash) >= 2 else _view_handle(a.handle, [1] + ash, [0] + list(a.strides))
    bh = b.handle
    if len(bsh) == 1:
        bh = _view_handle(b.handle, bsh + [1], list(b.strides) + [1]) if not transpose_b else \
            _view_handle(b.handle, [1] + bsh, [0] + list(b.strides))
    try:
        _kernel(a, "matmul")(cfg, ah, bh)
    finally:
        if ah is not a.handle:
            ah.dispose()
        if bh is not b.handle:
            bh.dispose()
    return out if out is not None else _wrap(output)


def matmul(a: Tensor, b: Tensor) -> Tensor:
    return dispatch_matmul(a, b)


def linear(input: Tensor, weight: Tensor, bias: Optional[Tensor] = None, out_dtype: Optional[str] = None) -> Tensor:
    """y = input @ weight^T + bias with weight [out_features, in_features] (nn.Linear layout)."""
    return dispatch_matmul(input, weight, transpose_b=True, bias=bias, out_dtype=out_dtype)


def linear_fused(prologue: str, x: Tensor, weight: Tensor, norm_weight: Optional[Tensor] = None,
                 eps: float = 1e-6, x2: Optional[Tensor] = None, residual: Optional[Tensor] = None,
                 out_dtype: Optional[str] = None, act_dtype: str = "bfloat16") -> Tensor:
    """One-row linear with its producer fused in front (decode).  prologue 'rms_norm': x is the
    fp32 residual row and the input is rms_norm(x, norm_weight, eps); 'silu_mul': the input is
    silu(x) * x2; 'silu_mul_interleaved': x is a gate/up row interleaved in blocks of 8 and the
    input is silu(gate) * up; 'none': the input is x.  act_dtype is the activations' dtype: bfloat16
    (the input rounded to bf16 as the unfused producer stores it) or float32 (kept in fp32).  With
    `residual` the result is added into it in place (residual += input @ weight^T) and returned;
    otherwise a new [1, out_features] tensor of out_dtype (default act_dtype)."""
    params = {"eps": eps, "act_dtype": act_dtype}
    if norm_weight is not None:
        params["norm_weight"] = norm_weight.handle
    if x2 is not None:
        params["x2"] = x2.handle
    if residual is not None:
        params["cin"] = residual.handle
        params["beta"] = 1.0
        out = residual.handle
    else:
        out = _new(weight, (1, weight.shape[0]), out_dtype or act_dtype)
    _kernel(weight, "gemv_fused")(prologue, x.handle, weight.handle, out, params)
    if residual is not None:
        return residual
    return _wrap(out)


def linear_swiglu_row(prologue: str, x: Tensor, w_gu: Tensor, norm_weight: Optional[Tensor] = None,
                      eps: float = 1e-6, act_dtype: str = "bfloat16") -> Tensor:
    """One-row SwiGLU (decode): silu(x' W_gate^T) * (x' W_up^T) as a new [1, I] tensor of act_dtype
    (bfloat16: x', gate and up rounded to bf16; float32: all kept in fp32) from the interleaved
    gate/up weight [2I, H]; prologue 'rms_norm' (x the fp32 residual row, x' its RMSNorm) or 'none'
    (x' = x, of act_dtype)."""
    out = _new(w_gu, (1, w_gu.shape[0] // 2), act_dtype)
    params = {"eps": eps}
    if norm_weight is not None:
        params["norm_weight"] = norm_weight.handle
    _kernel(w_gu, "gemv_swiglu")(prologue, x.handle, w_gu.handle, out, params)
    return _wrap(out)


# ---------------------------------------------------------------------------------------------
# normalisation and pointwise
# ---------------------------------------------------------------------------------------------
def rms_norm(input: Tensor, normalized_shape: Sequence[int], weight: Optional[Tensor] = None,
             eps: Optional[float] = None, out_dtype: Optional[str] = None) -> Tensor:
    """RMSNorm over the trailing normalized_shape dims; out_dtype (default: the input dtype) is the
    dtype of the result and of the weight."""
    params = {"normalized_shape": list(normalized_shape), "eps": eps,
              "weight": weight.handle if weight is not None else None, "out_dtype": out_dtype}
    return _wrap(_kernel(input, "rms_norm")([input.handle], params))


def _binary(name: str, a: Tensor, b: Tensor, alpha: Optional[float] = None) -> Tensor:
    """A binary map op through its iterator kernel (handlers/iterator.ts:24-135): broadcast and
    strided operands are read in place through their iterator strides; the result is a new tensor
    of the promoted dtype."""
    it = TensorIterator.binary_op(a.handle, b.handle, scalar_args=None if alpha is None else {"alpha": alpha})
    _kernel(a, name)(it)
    return _wrap(it.output().tensor_handle)


def add(a: Tensor, b: Tensor, alpha: Optional[float] = None) -> Tensor:
    """a + alpha * b (ops.ts:437)."""
    return _binary("add", a, b, alpha)


def mul(a: Tensor, b: Tensor) -> Tensor:
    return _binary("mul", a, b)


def sub(a: Tensor, b: Tensor, alpha: Optional[float] = None) -> Tensor:
    return _binary("sub", a, b, alpha)


def div(a: Tensor, b: Tensor) -> Tensor:
    return _binary("div", a, b)


def _map(x: Tensor, name: str) -> Tensor:
    """A one-input pointwise op found by name (the reference's IteratorHandler route,
    packages/core/src/dispatch/handlers/iterator.ts:24-135): the input read through its strides,
    a new output."""
    it = TensorIterator.unary_op(x.handle)
    _kernel(x, name)(it)
    return _wrap(it.output().tensor_handle)


def silu(x: Tensor) -> Tensor:
    return _map(x, "silu")


def neg(x: Tensor) -> Tensor:
    return _map(x, "neg")


def cos(x: Tensor) -> Tensor:
    return _map(x, "cos")


def sin(x: Tensor) -> Tensor:
    return _map(x, "sin")


def arange(start: float, end: Optional[float] = None, step: float = 1.0, dtype: str = "float32") -> Tensor:
    """[start, end) with step (arange(n) = [0, n)); n = ceil((end - start) / step) elements, values
    start + i * step from the `arange` factory kernel."""
    if end is None:
        start, end = 0.0, start
    if step == 0:
        raise ValueError("arange: step must be nonzero")
    n = max(0, int(math.ceil((end - start) / step)))
    from .env import get_backend, get_default_device
    it = TensorIterator.nullary_op((n,), dtype, scalar_args={"start": float(start), "end": float(end),
                                                             "step": float(step)})
    get_backend(get_default_device()).operators.find("arange")(it)
    return _wrap(it.output().tensor_handle)


def linear_swiglu(input: Tensor, weight_gu: Tensor) -> Tensor:
    """silu(input W_gate^T) * (input W_up^T) in one launch from the interleaved gate/up weight
    [2 I, H] (kernels.interleave_gate_up); returns [..., I] of input's dtype (bf16, or float32 with
    float32 activations) (swiglu.ts:119-134)."""
    out = _new(input, tuple(input.shape[:-1]) + (weight_gu.shape[0] // 2,), input.dtype)
    _kernel(input, "linear_swiglu")(input.handle, weight_gu.handle, out)
    return _wrap(out)


def linear_add_rms_norm(input: Tensor, weight: Tensor, residual: Tensor, norm_weight: Tensor, eps: float,
                        rows=None) -> Tensor:
    """residual += input W^T in place (fp32) and returns rms_norm(residual) * norm_weight in
    norm_weight's dtype -- a decoder sub-block's closing projection, its residual add and the next
    RMSNorm (decoder_layer.ts:224-238, RMSNorm.ts:92-99).  rows = (r0, r1) limits the add and the
    norm to those residual rows (the result has r1 - r0 rows)."""
    r0, r1 = rows if rows is not None else (0, residual.shape[0])
    out = _new(residual, (r1 - r0, residual.shape[1]), norm_weight.dtype)
    _kernel(input, "linear_add_rms_norm")(input.handle, weight.handle, residual.handle, norm_weight.handle,
                                          float(eps), out, rows)
    return _wrap(out)


def silu_mul(gate: Tensor, up: Tensor) -> Tensor:
    out = _new(gate, gate.shape)
    _kernel(gate, "silu_mul")(gate.handle, up.handle, out)
    return _wrap(out)


# ---------------------------------------------------------------------------------------------
# copies, gathers, reductions
# ---------------------------------------------------------------------------------------------
def contiguous(x: Tensor) -> Tensor:
    """Zero-copy when already contiguous at its offset (copy.ts:123-138), else a materialising copy."""
    if x.handle.is_contiguous():
        x.handle.storage.inc_ref()
        return _wrap(HipTensorHandle(x.handle.storage, x.shape, x.dtype, x.strides, x.offset))
    out = _new(x, x.shape)
    _kernel(x, "contiguous")(TensorIterator.unary_op(x.handle, out))
    return _wrap(out)


def cast(x: Tensor, dtype: str) -> Tensor:
    """x in another dtype (handlers/copy.ts cast: the same tensor when the dtype matches)."""
    if x.dtype == dtype:
        x.handle.storage.inc_ref()
        return _wrap(HipTensorHandle(x.handle.storage, x.shape, x.dtype, x.strides, x.offset))
    out = _new(x, x.shape, dtype)
    _kernel(x, "cast")(TensorIterator.unary_op(x.handle, out))
    return _wrap(out)


def clone(x: Tensor) -> Tensor:
    out = _new(x, x.shape)
    _kernel(x, "clone")(TensorIterator.unary_op(x.handle, out))
    return _wrap(out)


def copy_(dst: Tensor, src: Tensor) -> Tensor:
    """dst (any view) takes src's values (handlers/copy.ts copyInplace: shapes must match)."""
    if tuple(dst.shape) != tuple(src.shape):
        raise ValueError(f"copy_: shape mismatch {tuple(dst.shape)} vs {tuple(src.shape)}")
    _kernel(dst, "copy_")(TensorIterator.unary_op(src.handle, dst.handle))
    return dst


def embedding(input_ids: Tensor, weight: Tensor, out_dtype: Optional[str] = None) -> Tensor:
    """weight[input_ids] with ids int32 of any shape -> ids.shape + [hidden], in out_dtype
    (default: the table's dtype); ids outside the table give zero rows."""
    ids = input_ids if input_ids.handle.is_contiguous() else contiguous(input_ids)
    out = _new(weight, tuple(input_ids.shape) + tuple(weight.shape[1:]), out_dtype)
    _kernel(weight, "index_select")(weight.handle, ids.handle, {"dim": 0}, out)
    if ids is not input_ids:
        ids.dispose()
    return _wrap(out)


def index_select(x: Tensor, dim: int, index: Tensor) -> Tensor:
    """x with the entries of `index` (int32, 1-d) taken along `dim` (gather.ts:121,190)."""
    nd = len(x.shape)
    d = dim + nd if dim < 0 else dim
    if not 0 <= d < nd or len(index.shape) != 1:
        raise ValueError("index_select: dim out of range or index not 1-d")
    ids = index if index.handle.is_contiguous() else contiguous(index)
    out = _new(x, tuple(x.shape[:d]) + (index.shape[0],) + tuple(x.shape[d + 1:]))
    _kernel(x, "index_select")(x.handle, ids.handle, {"dim": d}, out)
    if ids is not index:
        ids.dispose()
    return _wrap(out)


def argmax(x: Tensor, dim: Optional[int] = -1, keepdim: bool = False) -> Tensor:
    """Index of the maximum along `dim` (all elements when None), lowest index among maxima, int32,
    through the reduction iterator (handlers/iterator.ts buildReduceIterator; the kernel reads the
    input through its strides, reduction/argShaderBuilder.ts:205-240 reduces any dim)."""
    nd = len(x.shape)
    axes = None if dim is None else [dim]
    if axes is not None and not -nd <= dim < nd:
        raise ValueError(f"argmax: dim {dim} out of range for a {nd}-d tensor")
    it = TensorIterator.reduction_op(x.handle, axes, keepdim, out_dtype="int32")
    _kernel(x, "argmax")(it)
    return _wrap(it.output().tensor_handle)


def zeros(shape, dtype: str = "float32") -> Tensor:
    """The zeros factory (handlers/factory.ts:50-61): a nullary iterator over a new tensor."""
    it = TensorIterator.nullary_op(tuple(shape), dtype)
    env.get_backend("hip").operators.find("zeros")(it)
    return _wrap(it.output().tensor_handle)


# ---------------------------------------------------------------------------------------------
# views (metadata only; the storage is shared and incRef'd)
# ---------------------------------------------------------------------------------------------
def _view_handle(h: HipTensorHandle, shape, strides, offset=None) -> HipTensorHandle:
    return HipTensorHandle.create_view(h.storage, shape, h.dtype, strides, h.offset if offset is None else offset)


def view(x: Tensor, shape) -> Tensor:
    shape = list(shape)
    if -1 in shape:
        i = shape.index(-1)
        rest = numel_of([s for j, s in enumerate(shape) if j != i])
        shape[i] = x.numel // rest if rest else 0
    if numel_of(shape) != x.numel:
        raise ValueError(f"view: {tuple(x.shape)} cannot become {tuple(shape)}")
    if not x.handle.is_contiguous():
        raise ValueError("view: input must be contiguous (use reshape)")
    return _wrap(_view_handle(x.handle, shape, contiguous_strides(shape)))


def reshape(x: Tensor, shape) -> Tensor:
    if x.handle.is_contiguous():
        return view(x, shape)
    c = contiguous(x)
    try:
        return view(c, shape)
    finally:
        c.dispose()


def permute(x: Tensor, dims) -> Tensor:
    nd = len(x.shape)
    dims = [d % nd for d in dims]
    return _wrap(_view_handle(x.handle, [x.shape[d] for d in dims], [x.strides[d] for d in dims]))


def transpose(x: Tensor, d0: int, d1: int) -> Tensor:
    nd = len(x.shape)
    dims = list(range(nd))
    dims[d0 % nd], dims[d1 % nd] = dims[d1 % nd], dims[d0 % nd]
    return permute(x, dims)


def narrow(x: Tensor, dim: int, start: int, length: int) -> Tensor:
    dim %= len(x.shape)
    if start < 0 or start + length > x.shape[dim]:
        raise ValueError(f"narrow: [{start}, {start + length}) outside dim {dim} of size {x.shape[dim]}")
    shape = list(x.shape)
    shape[dim] = length
    return _wrap(_view_handle(x.handle, shape, x.strides, x.offset + start * x.strides[dim]))


def unsqueeze(x: Tensor, dim: int) -> Tensor:
    nd = len(x.shape) + 1
    dim %= nd
    shape, strides = list(x.shape), list(x.strides)
    inner = strides[dim] * shape[dim] if dim < len(shape) else 1
    shape.insert(dim, 1)
    strides.insert(dim, inner)
    return _wrap(_view_handle(x.handle, shape, strides))


def expand(x: Tensor, shape) -> Tensor:
    shape = list(shape)
    pad = len(shape) - len(x.shape)
    xs, xst = [1] * pad + list(x.shape), [0] * pad + list(x.strides)
    strides = []
    for s, xs_i, st in zip(shape, xs, xst):
        if xs_i == s:
            strides.append(st)
        elif xs_i == 1:
            strides.append(0)
        else:
            raise ValueError(f"expand: cannot expand {tuple(x.shape)} to {tuple(shape)}")
    return _wrap(_view_handle(x.handle, shape, strides))
