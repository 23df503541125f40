"""Kernel implementations registered by HipBackend, with the reference kernel signatures.

Each function validates shapes on the host, materialises views the kernels cannot take, and calls
one C-ABI entry point of libkandle_hip.so.  There is no CPU or WebGPU fallback: a shape or dtype the
HIP kernels do not take raises.

Signatures follow packages/types/src/backend/register.ts:
  flash_attention(query, key, value, output, scale, is_causal) -> None            (:102-109)
  matmul(config, a, b) -> None  (config = MatmulDispatchResult)                   (core/src/dispatch/matmulOps.ts:486-493)
  rms_norm(inputs, params) -> handle  (NormalizeKernelImpl)                        (:52-55)
  silu / mul / add / sub (iter) -> None  (IteratorKernelImpl)                       (:9)
  copy(input, options) -> handle  (CopyKernelImpl: contiguous / cast)              (:14-25)
  index_select(self, index, params, output) -> None  (GatherKernelImpl)            (:64-69)
  argmax(iter) -> None
New fused names (no reference schema; the reference composes them from the ops above):
  rms_norm_rope(q, k, params) -> (q_out, k_out)   qk-norm + RoPE (+ V cache write)
  silu_mul(gate, up, output) -> None              SwiGLU activation
  decode_attention(q, k_cache, v_cache, seq_lens, output, scale) -> None   varlen split-K decode
"""
from __future__ import annotations

import ctypes as C
import dataclasses
from dataclasses import dataclass, field
from typing import Optional, Sequence

import numpy as np

from . import _lib
from .dtypes import BFLOAT16, FLOAT32, INT32, KH_CODE
from .tensor import HipTensorHandle, check_extent, copy_into, contiguous_strides

_vp = C.c_void_p


def _materialize(h: HipTensorHandle, dtype: Optional[str] = None) -> HipTensorHandle:
    """Contiguous handle with the same logical data (a new one unless already contiguous)."""
    dtype = dtype or h.dtype
    if h.is_contiguous() and dtype == h.dtype:
        h.storage.inc_ref()
        return HipTensorHandle(h.storage, h.shape, h.dtype, h.strides, h.offset)
    out = HipTensorHandle.create_new(h.shape, dtype)
    copy_into(h, out)
    return out


def _last_dim_contiguous(h: HipTensorHandle) -> bool:
    return h.strides[-1] == 1 or h.shape[-1] == 1


def _as_4d(h: HipTensorHandle):
    """[B,H,L,D] view parameters (shape, strides) of a 2/3/4-D handle (attention/executor.ts:198-220)."""
    shape, strides = list(h.shape), list(h.strides)
    if len(shape) == 4:
        return shape, strides
    if len(shape) == 3:
        return [1] + shape, [0] + strides
    if len(shape) == 2:
        return [1, 1] + shape, [0, 0] + strides
    raise ValueError(f"attention expects a 2-D, 3-D or 4-D tensor, got shape {tuple(h.shape)}")


# ---------------------------------------------------------------------------------------------
# flash_attention
# ---------------------------------------------------------------------------------------------
def flash_attention(query, key, value, output, scale: float, is_causal: bool) -> None:
    """O = softmax(scale * Q K^T + causal) V with native GQA; output preallocated by the caller."""
    _flash(query, key, value, output, scale, is_causal, split=False)


def flash_attention_split(query, key, value, output, scale: float, is_causal: bool) -> None:
    """flash_attention's signature for fp32 operands, computed in split-bf16 form (each fp32 value as
    bf16 hi + lo, every product as three bf16 MFMAs: within about 2^-15 relative of the fp32
    products; kh_flash_attention_split): the float32-activation prefill's attention.  Shapes the
    split kernel does not take run the fp32 kernel."""
    _flash(query, key, value, output, scale, is_causal, split=True)


def _flash(query, key, value, output, scale: float, is_causal: bool, split: bool) -> None:
    for name, h in (("query", query), ("key", key), ("value", value), ("output", output)):
        if h.dtype not in (FLOAT32, BFLOAT16):
            raise TypeError(f"flash_attention: {name} dtype {h.dtype} not supported")
    if not (query.dtype == key.dtype == value.dtype == output.dtype):
        raise TypeError("flash_attention: query/key/value/output dtypes differ")
    tmp = []
    try:
        hs = []
        for h in (query, key, value):
            if not _last_dim_contiguous(h):
                h = _materialize(h)
                tmp.append(h)
            hs.append(h)
        q, k, v = hs
        qs, qst = _as_4d(q)
        ks, kst = _as_4d(k)
        vs, vst = _as_4d(v)
        os_, ost = _as_4d(output)
        B, Hq, Lq, D = qs
        Bk, Hkv, Lk, Dk = ks
        if Bk != B or vs[0] != B or Dk != D or vs[1] != Hkv or vs[2] != Lk:
            raise ValueError(f"flash_attention: incompatible shapes q{qs} k{ks} v{vs}")
        if vs[3] != D:
            raise ValueError("flash_attention: value head_dim must equal query head_dim")
        if Hq % Hkv != 0:
            raise ValueError(f"flash_attention: numHeadsQ ({Hq}) must be divisible by numHeadsKV ({Hkv})")
        if tuple(os_) != (B, Hq, Lq, D) or ost[3] != 1:
            raise ValueError(f"flash_attention: output must be [B,Hq,Lq,D] with a contiguous last dim, got {os_}")
        strides = _lib.i64_array(qst[:3] + kst[:3] + vst[:3] + ost[:3])
        args = (_vp(q.data_ptr()), _vp(k.data_ptr()), _vp(v.data_ptr()), _vp(output.data_ptr()),
                B, Hq, Hkv, Lq, Lk, D, strides, C.c_float(scale), int(bool(is_causal)))
        if split:
            if q.dtype != FLOAT32:
                raise TypeError("flash_attention_split: float32 operands expected")
            _lib.call("kh_flash_attention_split", *args)
        else:
            _lib.call("kh_flash_attention", *args, q.kh_dtype)
    finally:
        for t in tmp:
            t.dispose()


def _mask_strides(mask, target) -> list:
    """Element strides of `mask` broadcast (numpy rules, trailing axes aligned) to the 4-D score
    shape `target` = [B, Hq, Lq, Lk]; 0 for a broadcast axis.  Shapes that do not broadcast raise,
    as the reference's add_Tensor does."""
    shape, strides = list(mask.shape), list(mask.strides)
    if len(shape) > 4:
        raise ValueError(f"sdpa_masked: attn_mask has {len(shape)} dims, scores have 4")
    shape = [1] * (4 - len(shape)) + shape
    strides = [0] * (4 - len(strides)) + strides
    out = []
    for n, st, t in zip(shape, strides, target):
        if n == t:
            out.append(st if t > 1 else 0)
        elif n == 1:
            out.append(0)
        else:
            raise ValueError(f"sdpa_masked: attn_mask shape {tuple(mask.shape)} cannot be broadcast to the "
                             f"attention scores {tuple(target)}")
    return out


def sdpa_masked(query, key, value, mask, output, scale: float) -> None:
    """O = softmax(scale * Q K^T + mask) V, the reference's explicit-mask route
    (packages/core/src/dispatch/handlers/composite.ts:279-300) in one kernel: the mask is added to
    the scaled scores (broadcast over [B, Hq, Lq, Lk]), causal masking is not applied, and a row
    whose exponentials sum to 0 (every score far below -1e38, e.g. all -inf) is NaN, as the
    reference softmax's 0 / 0 (normalize/shaderBuilder.ts:143-213).  GQA as flash_attention."""
    for name, h in (("query", query), ("key", key), ("value", value), ("output", output)):
        if h.dtype not in (FLOAT32, BFLOAT16):
            raise TypeError(f"sdpa_masked: {name} dtype {h.dtype} not supported")
    if not (query.dtype == key.dtype == value.dtype == output.dtype):
        raise TypeError("sdpa_masked: query/key/value/output dtypes differ")
    if mask.dtype not in (FLOAT32, BFLOAT16):
        raise TypeError(f"sdpa_masked: attn_mask dtype {mask.dtype} not supported (additive float32 or bfloat16)")
    tmp = []
    try:
        hs = []
        for h in (query, key, value):
            if not _last_dim_contiguous(h):
                h = _materialize(h)
                tmp.append(h)
            hs.append(h)
        q, k, v = hs
        qs, qst = _as_4d(q)
        ks, kst = _as_4d(k)
        vs, vst = _as_4d(v)
        os_, ost = _as_4d(output)
        B, Hq, Lq, D = qs
        Bk, Hkv, Lk, Dk = ks
        if Bk != B or vs[0] != B or Dk != D or vs[1] != Hkv or vs[2] != Lk or vs[3] != D:
            raise ValueError(f"sdpa_masked: incompatible shapes q{qs} k{ks} v{vs}")
        if Hq % Hkv != 0:
            raise ValueError(f"sdpa_masked: numHeadsQ ({Hq}) must be divisible by numHeadsKV ({Hkv})")
        if tuple(os_) != (B, Hq, Lq, D) or ost[3] != 1:
            raise ValueError(f"sdpa_masked: output must be [B,Hq,Lq,D] with a contiguous last dim, got {os_}")
        ms = _mask_strides(mask, (B, Hq, Lq, Lk))
        strides = _lib.i64_array(qst[:3] + kst[:3] + vst[:3] + ost[:3])
        _lib.call(
            "kh_flash_attention_masked",
            _vp(q.data_ptr()), _vp(k.data_ptr()), _vp(v.data_ptr()), _vp(output.data_ptr()),
            B, Hq, Hkv, Lq, Lk, D, strides, C.c_float(scale), _vp(mask.data_ptr()), _lib.i64_array(ms),
            mask.kh_dtype, q.kh_dtype,
        )
    finally:
        for t in tmp:
            t.dispose()


def decode_attention(q, k_cache, v_cache, seq_lens, output, scale: float) -> None:
    """One query token per sequence against [B, Hkv, max_len, D] caches with per-sequence lengths.

    q/output: [B, Hq, D] or [B, Hq, 1, D]; seq_lens: int32 device handle [B] (values in [1, max_len])."""
    qs, qst = list(q.shape), list(q.strides)
    os_, ost = list(output.shape), list(output.strides)
    if len(qs) == 4:
        qs, qst = qs[:2] + qs[3:], qst[:2] + qst[3:]
    if len(os_) == 4:
        os_, ost = os_[:2] + os_[3:], ost[:2] + ost[3:]
    B, Hq, D = qs
    _, Hkv, L, Dk = k_cache.shape
    if seq_lens.dtype != INT32 or seq_lens.shape != (B,):
        raise ValueError("decode_attention: seq_lens must be an int32 tensor of shape [B]")
    if Dk != D or tuple(v_cache.shape) != tuple(k_cache.shape) or os_ != [B, Hq, D]:
        raise ValueError("decode_attention: incompatible shapes")
    if qst[2] != 1 or ost[2] != 1 or k_cache.strides[3] != 1 or v_cache.strides[3] != 1:
        raise ValueError("decode_attention: the head_dim axis must be contiguous")
    strides = _lib.i64_array(qst[:2] + list(k_cache.strides[:3]) + list(v_cache.strides[:3]) + ost[:2])
    _lib.call(
        "kh_decode_attention",
        _vp(q.data_ptr()), _vp(k_cache.data_ptr()), _vp(v_cache.data_ptr()), _vp(output.data_ptr()),
        _vp(seq_lens.data_ptr()), B, Hq, Hkv, D, L, strides, C.c_float(scale), q.kh_dtype,
    )


def decode_attention_block(qkv, params: dict) -> None:
    """The attention block of one decode step (kh_decode_attention_block): qkv [1, hq*D + 2*hkv*D]
    raw projections of the new token; params: q_norm, k_norm (bf16 [D]), inv_freq (fp32 [D/2]), eps,
    position (int32 [1], device), k_cache / v_cache ([1, hkv, max_len, D], qkv's dtype), w_o (bf16
    [hidden, hq*D]), x (fp32 residual row [1, hidden], updated in place), scale.  qkv and the caches
    are bfloat16 (values rounded to bf16 where the unfused launches store them) or float32 (every
    activation kept in fp32)."""
    kc, vc, wo, x = params["k_cache"], params["v_cache"], params["w_o"], params["x"]
    _, hkv, max_len, D = kc.shape
    n_in = qkv.numel
    hq = (n_in - 2 * hkv * D) // D
    if D != 128 or hq <= 0 or hq * D + 2 * hkv * D != n_in:
        raise ValueError(f"decode_attention_block: qkv of {n_in} values does not split into q/k/v heads of 128")
    if qkv.dtype not in (FLOAT32, BFLOAT16):
        raise TypeError("decode_attention_block: qkv must be float32 or bfloat16")
    for name, h in (("k_cache", kc), ("v_cache", vc)):
        if h.dtype != qkv.dtype:
            raise TypeError(f"decode_attention_block: {name} must have qkv's dtype {qkv.dtype}")
    for name, h in (("q_norm", params["q_norm"]), ("k_norm", params["k_norm"]), ("w_o", wo)):
        if h.dtype != BFLOAT16:
            raise TypeError(f"decode_attention_block: {name} must be bfloat16")
    if not qkv.is_contiguous() or x.dtype != FLOAT32 or not x.is_contiguous():
        raise TypeError("decode_attention_block: qkv and x (fp32) must be contiguous")
    n_out = x.numel
    if tuple(wo.shape) != (n_out, hq * D) or wo.strides[1] != 1:
        raise ValueError(f"decode_attention_block: w_o must be [{n_out}, {hq * D}] with contiguous rows")
    pos = params["position"]
    if pos.dtype != INT32 or pos.numel < 1:
        raise TypeError("decode_attention_block: position must be an int32 device tensor")
    strides = _lib.i64_array([kc.strides[1], kc.strides[2], vc.strides[1], vc.strides[2]])
    _lib.call("kh_decode_attention_block", _vp(qkv.data_ptr()), _vp(params["q_norm"].data_ptr()),
              _vp(params["k_norm"].data_ptr()), _vp(params["inv_freq"].data_ptr()), C.c_float(params["eps"]),
              _vp(pos.data_ptr()), _vp(kc.data_ptr()), _vp(vc.data_ptr()), hq, hkv, max_len, strides,
              C.c_float(params["scale"]), _vp(wo.data_ptr()), wo.strides[0], n_out, _vp(x.data_ptr()), qkv.kh_dtype)


# ---------------------------------------------------------------------------------------------
# matmul
# ---------------------------------------------------------------------------------------------
@dataclass
class MatmulDispatchResult:
    """Subset of the reference MatmulDispatchResult (packages/core/src/dispatch/matmulOps.ts:32-125)
    the kernel reads, plus `bias` (fused linear bias)."""

    variant: str
    output: HipTensorHandle
    M: int
    K: int
    N: int
    batch_shape: Sequence[int] = field(default_factory=tuple)
    batch_size: int = 1
    transpose_a: bool = False
    transpose_b: bool = False
    alpha: float = 1.0
    beta: float = 0.0
    input_c: Optional[HipTensorHandle] = None
    bias: Optional[HipTensorHandle] = None


def matmul(config: MatmulDispatchResult, a: HipTensorHandle, b: HipTensorHandle) -> None:
    """out[..., M, N] = alpha * A[..., M, K] op(B) + beta * C (+ bias), one GEMM per batch entry.

    `b` is [..., K, N] (transpose_b False) or [..., N, K] (transpose_b True, the nn.Linear weight).
    Operands share a dtype (float32 or bfloat16), except that float32 activations may meet bfloat16
    weights: the reference's float32 matmul of a checkpoint it widens to float32 on load
    (io/safetensor/dtypes.ts:17-31), computed from the bf16 weights directly (kh_gemm_ex)."""
    out = config.output
    mixed = a.dtype == FLOAT32 and b.dtype == BFLOAT16
    if a.dtype != b.dtype and not mixed:
        raise TypeError(f"matmul: dtype mismatch {a.dtype} vs {b.dtype}")
    if a.dtype not in (FLOAT32, BFLOAT16):
        raise TypeError(f"matmul does not support dtype {a.dtype}")
    if out.dtype != a.dtype and not (a.dtype == BFLOAT16 and out.dtype == FLOAT32):
        raise TypeError(f"matmul: {a.dtype} inputs cannot produce a {out.dtype} output")
    M, K, N = config.M, config.K, config.N
    tmp = []
    try:
        if config.transpose_a:
            # A stored [..., K, M]: op(A) = A^T, materialised as contiguous [..., M, K]
            a = HipTensorHandle.create_view(a.storage, list(a.shape[:-2]) + [a.shape[-1], a.shape[-2]], a.dtype,
                                            list(a.strides[:-2]) + [a.strides[-1], a.strides[-2]], a.offset)
            tmp.append(a)
        A = a if (a.strides[-1] == 1 or K == 1) else _materialize(a)
        if A is not a:
            tmp.append(A)
        if (not config.transpose_b and len(b.shape) >= 2 and b.strides[-2] == 1 and b.shape[-1] > 1
                and b.strides[-1] >= K):
            # B [..., K, N] stored column-major is B^T [..., N, K] stored row-major: use it as the
            # transposed operand instead of copying (matmulOps.ts:171-181 detects this from strides)
            b = HipTensorHandle.create_view(b.storage, list(b.shape[:-2]) + [N, K], b.dtype,
                                            list(b.strides[:-2]) + [b.strides[-1], 1], b.offset)
            tmp.append(b)
            config = dataclasses.replace(config, transpose_b=True)
        Bm = b if (b.strides[-1] == 1 or b.shape[-1] == 1) else _materialize(b)
        if Bm is not b:
            tmp.append(Bm)
        if not out.is_contiguous():
            raise ValueError("matmul: output must be contiguous")
        batch = int(np.prod(config.batch_shape)) if len(config.batch_shape) else 1
        a_rows = A.numel // K if K else 0
        # Fold batch into M when A is a contiguous stack and B is shared (x W^T of a 3-D activation).
        b_batched = len(Bm.shape) > 2 and int(np.prod(Bm.shape[:-2])) > 1
        if not b_batched and A.is_contiguous():
            _gemm_call(A, K, Bm, out, N, config, rows=a_rows, a_off=0, b_off=0, c_off=0)
            return
        a_bs = _batch_offsets(A, config.batch_shape, 2)
        b_bs = _batch_offsets(Bm, config.batch_shape, 2)
        for i in range(batch):
            _gemm_call(A, A.strides[-2], Bm, out, N, config, rows=M, a_off=a_bs[i], b_off=b_bs[i], c_off=i * M * N)
    finally:
        for t in tmp:
            t.dispose()


def _batch_offsets(h: HipTensorHandle, batch_shape, mat_dims: int):
    """Element offsets of each broadcast batch entry of h over batch_shape."""
    bshape = list(batch_shape)
    hb_shape = list(h.shape[:-mat_dims])
    hb_str = list(h.strides[:-mat_dims])
    pad = len(bshape) - len(hb_shape)
    hb_shape = [1] * pad + hb_shape
    hb_str = [0] * pad + hb_str
    offs = []
    for idx in np.ndindex(*bshape) if bshape else [()]:
        off = 0
        for d, i in enumerate(idx):
            off += (0 if hb_shape[d] == 1 else i) * hb_str[d]
        offs.append(off)
    return offs


def _gemm_call(A, lda, Bm, out, N, config, rows, a_off, b_off, c_off):
    K = config.K
    isz, bsz = A.itemsize, Bm.itemsize
    osz = out.itemsize
    # [.., N, K] (transpose_b) or [.., K, N]: either way the row stride of the stored matrix.
    ldb = Bm.strides[-2] if len(Bm.shape) >= 2 else Bm.shape[-1]
    cin = config.input_c
    cin_ptr, ldcin = None, N
    if cin is not None and config.beta != 0.0:
        if tuple(cin.shape[-2:]) != (config.M, N) or not cin.is_contiguous() or cin.dtype != out.dtype:
            raise ValueError("matmul: inputC must be a contiguous [.., M, N] tensor of the output dtype")
        cin_ptr = cin.data_ptr() + c_off * osz
    bias_ptr = None
    if config.bias is not None:
        if config.bias.shape != (N,) or not config.bias.is_contiguous() or config.bias.dtype != out.dtype:
            raise ValueError("matmul: bias must be a contiguous [N] tensor of the output dtype")
        bias_ptr = config.bias.data_ptr()
    lda_eff = lda if lda else K
    _lib.call(
        "kh_gemm_ex",
        _vp(A.data_ptr() + a_off * isz), lda_eff, A.kh_dtype,
        _vp(Bm.data_ptr() + b_off * bsz), ldb, Bm.kh_dtype,
        _vp(out.data_ptr() + c_off * osz), N,
        _vp(cin_ptr) if cin_ptr else None, ldcin,
        _vp(bias_ptr) if bias_ptr else None,
        rows, N, K, C.c_float(config.alpha), C.c_float(config.beta), int(bool(config.transpose_b)), out.kh_dtype,
    )


# ---------------------------------------------------------------------------------------------
# normalisation / fused qk-norm + RoPE
# ---------------------------------------------------------------------------------------------
def rms_norm(inputs, params) -> HipTensorHandle:
    """NormalizeKernelImpl: inputs = [x], params = {normalized_shape, eps, weight?, out?, out_dtype?}.

    Normalises over the trailing dims given by normalized_shape; output is contiguous
    (packages/backend-webgpu/src/kernels/normalize/executor.ts:121-122).  The kernel default eps is
    1e-5 (executor.ts:58).  out_dtype (default: the input dtype) lets a float32 residual stream be
    normalised straight into a bfloat16 activation; the weight then has out_dtype."""
    x = inputs[0]
    ns = params.get("normalized_shape") or params.get("normalizedShape")
    if ns is None:
        raise ValueError("rms_norm: normalized_shape is required")
    ns = [int(v) for v in (ns if isinstance(ns, (list, tuple)) else [ns])]
    if list(x.shape[len(x.shape) - len(ns):]) != ns:
        raise ValueError(f"rms_norm: normalized_shape {ns} does not match input shape {x.shape}")
    eps = params.get("eps")
    eps = 1e-5 if eps is None else float(eps)
    w = params.get("weight")
    if params.get("bias") is not None:
        raise ValueError("rms_norm: bias is not part of RMSNorm")
    n = int(np.prod(ns))
    xs = x if x.is_contiguous() else _materialize(x)
    try:
        rows = xs.numel // n if n else 0
        out_dtype = params.get("out").dtype if params.get("out") is not None else (params.get("out_dtype") or x.dtype)
        if out_dtype not in (FLOAT32, BFLOAT16) or x.dtype not in (FLOAT32, BFLOAT16):
            raise TypeError(f"rms_norm: unsupported dtypes {x.dtype} -> {out_dtype}")
        out = params.get("out") or HipTensorHandle.create_new(x.shape, out_dtype)
        if not out.is_contiguous() or tuple(out.shape) != tuple(x.shape):
            raise ValueError("rms_norm: out must be a contiguous tensor of the input's shape")
        if w is not None:
            if w.numel != n or w.dtype != out_dtype:
                raise ValueError("rms_norm: weight must have normalized_shape elements and the output dtype")
            wc = w if w.is_contiguous() else _materialize(w)
        else:
            wc = None
        try:
            _lib.call(
                "kh_rms_norm", _vp(xs.data_ptr()), n, _vp(wc.data_ptr()) if wc is not None else None,
                _vp(out.data_ptr()), n, rows, n, C.c_float(eps), x.kh_dtype, out.kh_dtype,
            )
        finally:
            if wc is not None and wc is not w:
                wc.dispose()
        return out
    finally:
        if xs is not x:
            xs.dispose()


def rms_norm_rope(q, k, params):
    """Fused per-head RMSNorm + RoPE (+ optional V cache write) for q [B,S,Hq,D] and k [B,S,Hkv,D].

    params: q_weight, k_weight (handles [D]), inv_freq (float32 handle [D/2]), positions (int32 handle
    [B*S]), eps, and optional q_out / k_out (default: new [B,Hq,S,D] / [B,Hkv,S,D] tensors, i.e. the
    heads-first layout the attention consumes), v / v_out.  With cache_positions=True, k_out and
    v_out are whole KV caches [B, Hkv, max_seq, D] and token t is written at sequence index
    positions[t] (positions outside [0, max_seq) write nothing), so the write location can live on
    the device (kv-cache.ts:164-212 writes the slice [pos, pos+S)).  Returns (q_out, k_out)."""
    if q.dtype != k.dtype or q.dtype not in (FLOAT32, BFLOAT16):
        raise TypeError("rms_norm_rope: q and k must share a float dtype")
    if len(q.shape) != 4 or len(k.shape) != 4:
        raise ValueError("rms_norm_rope: q and k must be [B, S, H, D]")
    B, S, Hq, D = q.shape
    _, _, Hkv, _ = k.shape
    q_out = params.get("q_out") or HipTensorHandle.create_new((B, Hq, S, D), q.dtype)
    k_out = params.get("k_out") or HipTensorHandle.create_new((B, Hkv, S, D), k.dtype)

    def bsh(h, heads_first):
        st = h.strides
        if h.strides[-1] != 1:
            raise ValueError("rms_norm_rope: head_dim must be contiguous")
        # heads_first tensors are [B, H, S, D]; the kernel wants (batch, seq, head) strides
        return [st[0], st[2], st[1]] if heads_first else [st[0], st[1], st[2]]

    v, v_out = params.get("v"), params.get("v_out")
    kv_cache_len = 0
    if params.get("cache_positions"):
        kv_cache_len = k_out.shape[2]
        if v_out is not None and v_out.shape[2] != kv_cache_len:
            raise ValueError("rms_norm_rope: K and V caches must have the same length")
    s = bsh(q, False) + bsh(k, False) + bsh(q_out, True) + bsh(k_out, True)
    if v is not None:
        s += bsh(v, False) + bsh(v_out, True)
    pos, inv_freq = params["positions"], params["inv_freq"]
    if pos.dtype != INT32 or pos.numel != B * S:
        raise ValueError("rms_norm_rope: positions must be int32 with B*S entries")
    if inv_freq.dtype != FLOAT32 or inv_freq.numel != D // 2:
        raise ValueError("rms_norm_rope: inv_freq must be float32 [D/2]")
    _lib.call(
        "kh_qk_norm_rope",
        _vp(q.data_ptr()), _vp(k.data_ptr()), _vp(q_out.data_ptr()), _vp(k_out.data_ptr()),
        _vp(v.data_ptr()) if v is not None else None, _vp(v_out.data_ptr()) if v is not None else None,
        _vp(params["q_weight"].data_ptr()), _vp(params["k_weight"].data_ptr()),
        _vp(inv_freq.data_ptr()), _vp(pos.data_ptr()),
        B, S, Hq, Hkv, D, _lib.i64_array(s), C.c_float(float(params.get("eps", 1e-6))), q.kh_dtype,
        kv_cache_len,
    )
    return q_out, k_out


# ---------------------------------------------------------------------------------------------
# Iterators: the operand geometry Kandle's dispatcher hands an iterator kernel
# (packages/core/src/dispatch/TensorIterator.ts), and the kernels that consume it
# ---------------------------------------------------------------------------------------------
def broadcast_strides(shape, strides, target) -> tuple:
    """computeBroadcastStrides (packages/utils/src/shape.ts:57-100): the strides of a view of
    shape / strides read at every index of `target` (right-aligned; 0 on new axes and on broadcast
    extents of 1)."""
    if len(target) < len(shape):
        raise ValueError("broadcast: the target shape has fewer dimensions")
    out = [0] * len(target)
    for i in range(len(target)):
        si = len(shape) - len(target) + i
        if si < 0:
            continue
        if shape[si] == target[i]:
            out[i] = strides[si]
        elif shape[si] != 1:
            raise ValueError(f"broadcast: {tuple(shape)} does not broadcast to {tuple(target)}")
    return tuple(out)


def _promote(dtypes) -> str:
    """The dtype an elementwise op computes and stores in: float32 over bfloat16, floats over int32."""
    if FLOAT32 in dtypes:
        return FLOAT32
    if BFLOAT16 in dtypes:
        return BFLOAT16
    return INT32


@dataclass
class IteratorOperand:
    """TensorIteratorOperand (packages/types/src/tensor.ts:282-378): strides are element strides
    aligned to the iterator's output shape (0 on broadcast axes), or for a reduction input to its
    kept axes with reduction_strides over the reduced ones; offset is in elements."""

    tensor_handle: HipTensorHandle
    dtype: str
    shape: tuple
    strides: tuple
    offset: int
    is_output: bool
    reduction_strides: Optional[tuple] = None


class TensorIterator:
    """ITensorIterator (packages/types/src/tensor.ts:395-569) over this backend's handles, built as
    Kandle's TensorIterator factories build one (TensorIterator.ts: build / unaryOp / binaryOp /
    nullaryOp / reductionOp): outputs first, input strides aligned to the output shape, scalar
    arguments (get_scalar_args).  TensorIterator(inputs, outputs) is the elementwise form (the
    inputs broadcast to the first output's shape)."""

    def __init__(self, inputs, outputs, scalar_args: Optional[dict] = None, _operands=None, _shapes=None,
                 _reduction=None):
        if _operands is None:
            out = outputs[0]
            shape = tuple(out.shape)
            ops = [IteratorOperand(o, o.dtype, tuple(o.shape), tuple(o.strides), o.offset, True) for o in outputs]
            ops += [IteratorOperand(h, h.dtype, tuple(h.shape), broadcast_strides(h.shape, h.strides, shape), h.offset,
                                    False) for h in inputs]
            _operands, _shapes = ops, (shape, shape)
        self.operands = list(_operands)
        self.num_outputs = len(outputs)
        self.num_inputs = len(self.operands) - self.num_outputs
        self.input_shape, self.output_shape = _shapes
        self.output_numel = int(np.prod(self.output_shape)) if self.output_shape else 1
        axes, keep = _reduction if _reduction is not None else ((), False)
        self.reduction_axes = tuple(axes)
        self.is_reduction = bool(axes)
        self.keep_dims = bool(keep)
        self.reduction_shape = tuple(self.input_shape[a] for a in self.reduction_axes)
        self._scalars = dict(scalar_args or {})

    def output(self, i: int = 0) -> IteratorOperand:
        return self.operands[i]

    def input(self, i: int = 0) -> IteratorOperand:
        return self.operands[self.num_outputs + i]

    def set_scalar_args(self, args: dict) -> None:
        self._scalars = dict(args)

    def get_scalar_args(self) -> dict:
        return dict(self._scalars)

    def get_scalar_arg(self, name: str):
        return self._scalars.get(name)

    # -- factories ----------------------------------------------------------------------------
    @classmethod
    def build(cls, inputs, output: Optional[HipTensorHandle] = None, out_dtype: Optional[str] = None,
              scalar_args: Optional[dict] = None) -> "TensorIterator":
        """Elementwise: the inputs broadcast to one shape; the output (allocated, in out_dtype or the
        promoted input dtype, when not given) has that shape."""
        if output is None:
            shape = tuple(np.broadcast_shapes(*[tuple(h.shape) for h in inputs])) if inputs else ()
            output = HipTensorHandle.create_new(shape, out_dtype or _promote([h.dtype for h in inputs]))
        else:
            np.broadcast_shapes(tuple(output.shape), *[tuple(h.shape) for h in inputs])
        return cls(list(inputs), [output], scalar_args)

    @classmethod
    def unary_op(cls, x, output=None, scalar_args=None) -> "TensorIterator":
        return cls.build([x], output, scalar_args=scalar_args)

    @classmethod
    def binary_op(cls, a, b, output=None, scalar_args=None) -> "TensorIterator":
        return cls.build([a, b], output, scalar_args=scalar_args)

    @classmethod
    def nullary_op(cls, shape, dtype: str, output: Optional[HipTensorHandle] = None,
                   scalar_args: Optional[dict] = None) -> "TensorIterator":
        """A factory's iterator: no inputs, a new contiguous output of shape and dtype (or `output`)."""
        out = output if output is not None else HipTensorHandle.create_new(tuple(shape), dtype)
        return cls([], [out], scalar_args)

    @classmethod
    def reduction_op(cls, x: HipTensorHandle, axes=None, keep_dims: bool = False,
                     output: Optional[HipTensorHandle] = None, out_dtype: Optional[str] = None,
                     scalar_args: Optional[dict] = None) -> "TensorIterator":
        """A reduction over `axes` (all axes when None or empty): the output holds the kept axes (and
        extent-1 reduced axes with keep_dims); the input's strides split into the kept axes' and the
        reduced axes' (reduction_strides), as splitStridesForReduction does."""
        nd = len(x.shape)
        red = sorted(range(nd)) if not axes else sorted(a + nd if a < 0 else a for a in axes)
        if any(not 0 <= a < nd for a in red):
            raise ValueError(f"reduction: axis out of range for a {nd}-d tensor")
        kept = [i for i in range(nd) if i not in red]
        out_shape = tuple(1 if i in red else x.shape[i] for i in range(nd)) if keep_dims else \
            tuple(x.shape[i] for i in kept)
        out = output if output is not None else HipTensorHandle.create_new(out_shape, out_dtype or x.dtype)
        if out.numel != (int(np.prod(out_shape)) if out_shape else 1):
            raise ValueError(f"reduction: output {tuple(out.shape)} for a result of {out_shape}")
        ops = [IteratorOperand(out, out.dtype, tuple(out.shape), tuple(out.strides), out.offset, True),
               IteratorOperand(x, x.dtype, tuple(x.shape), tuple(x.strides[i] for i in kept), x.offset, False,
                               tuple(x.strides[i] for i in red))]
        return cls(None, [out], scalar_args, _operands=ops, _shapes=(tuple(x.shape), out_shape),
                   _reduction=(red, keep_dims))


def _operand_geometry(op, shape, is_output: bool, name: str):
    """(device pointer, strides over `shape`, dtype code) of an iterator operand: the strides the
    dispatcher aligned (or, for an operand without them, its handle broadcast to `shape`), checked to
    stay inside its storage.  A bare handle is taken as an operand with its own geometry."""
    h = op.tensor_handle if isinstance(op, IteratorOperand) else op
    dtype = op.dtype if isinstance(op, IteratorOperand) else h.dtype
    if dtype != h.dtype:
        raise TypeError(f"{name}: operand dtype {dtype} differs from its handle's {h.dtype}")
    offset = op.offset if isinstance(op, IteratorOperand) else h.offset
    st = op.strides if isinstance(op, IteratorOperand) and len(op.strides) == len(shape) else \
        broadcast_strides(h.shape, h.strides, shape)
    if is_output and any(n > 1 and s == 0 for n, s in zip(shape, st)):
        raise ValueError(f"{name}: the output broadcasts an axis")
    check_extent(h.storage, shape, st, offset, dtype, f"{name} operand")
    return h.storage.ptr + offset * h.itemsize, tuple(st), KH_CODE[dtype]


MAP_OPS = {"copy": 0, "add": 1, "sub": 2, "mul": 3, "div": 4, "neg": 5, "cos": 6, "sin": 7, "silu": 8, "fill": 9,
           "arange": 10}
_MAP_NIN = {0: 1, 1: 2, 2: 2, 3: 2, 4: 2, 5: 1, 6: 1, 7: 1, 8: 1, 9: 0, 10: 0}


def map_strided(op: int, shape, out, a=None, b=None, s0: float = 0.0, s1: float = 0.0, name: str = "map") -> None:
    """kh_map_strided over `shape`: out and the inputs are IteratorOperands (or handles read with
    their own strides broadcast to `shape`)."""
    shape = tuple(int(n) for n in shape)
    if len(shape) > 8:
        raise ValueError(f"{name}: at most 8 dimensions")
    po, so, do = _operand_geometry(out, shape, True, name)
    args = [op, len(shape), _lib.i64_array(shape or [1]), _vp(po), _lib.i64_array(so or [1]), do]
    for x in (a, b):
        if x is None:
            args += [None, None, 0]
        else:
            px, sx, dx = _operand_geometry(x, shape, False, name)
            args += [_vp(px), _lib.i64_array(sx or [1]), dx]
    _lib.call("kh_map_strided", *args, C.c_double(s0), C.c_double(s1))


def _map_kernel(name: str, op: int, scalars=None):
    """An iterator kernel (register.ts:9: (iter) => None, the output preallocated as
    iter.output().tensor_handle) over kh_map_strided: inputs read through their strides, broadcast
    included; the output written through its own (a view for copy_).  scalars(args) -> (s0, s1)
    from the iterator's scalar arguments: add / sub alpha (default 1), a fill value, arange's start
    and step (arangeExecutor.ts:37-44)."""
    nin = _MAP_NIN[op]

    def kernel(it: TensorIterator) -> None:
        if it.num_inputs < nin:
            raise ValueError(f"{name}: {nin} inputs expected")
        s0, s1 = scalars(it.get_scalar_args()) if scalars is not None else (0.0, 0.0)
        map_strided(op, it.output_shape, it.output(0), it.input(0) if nin >= 1 else None,
                    it.input(1) if nin >= 2 else None, s0, s1, name)

    kernel.__name__ = name
    return kernel


def _alpha(sc):
    return float(sc.get("alpha", 1.0)), 0.0


add = _map_kernel("add", MAP_OPS["add"], _alpha)
sub = _map_kernel("sub", MAP_OPS["sub"], _alpha)
mul = _map_kernel("mul", MAP_OPS["mul"])
div = _map_kernel("div", MAP_OPS["div"])
neg = _map_kernel("neg", MAP_OPS["neg"])
cos = _map_kernel("cos", MAP_OPS["cos"])
sin = _map_kernel("sin", MAP_OPS["sin"])
silu = _map_kernel("silu", MAP_OPS["silu"])
# copy / cast / contiguous / clone / copy_ are one kernel: the output (possibly a strided view, or a
# new tensor in the target dtype) takes the input's values (copy/index.ts:13-33, handlers/copy.ts)
copy = _map_kernel("copy", MAP_OPS["copy"])
cast = _map_kernel("cast", MAP_OPS["copy"])
contiguous = _map_kernel("contiguous", MAP_OPS["copy"])
clone = _map_kernel("clone", MAP_OPS["copy"])
copy_ = _map_kernel("copy_", MAP_OPS["copy"])
zeros = _map_kernel("zeros", MAP_OPS["fill"], lambda sc: (0.0, 0.0))
ones = _map_kernel("ones", MAP_OPS["fill"], lambda sc: (1.0, 0.0))
full = _map_kernel("full", MAP_OPS["fill"],
                   lambda sc: (float(sc["fill_value"] if "fill_value" in sc else sc["fillValue"]), 0.0))
arange = _map_kernel("arange", MAP_OPS["arange"],
                     lambda sc: (float(sc.get("start", 0.0)), float(sc.get("step", 1.0))))


def empty(it: TensorIterator) -> None:
    """empty: the output is left as allocated."""


def fill(output: HipTensorHandle, value: float) -> None:
    """Every element of `output` (any view) set to value."""
    map_strided(MAP_OPS["fill"], output.shape, output, s0=float(value), name="fill")


def silu_mul(gate: HipTensorHandle, up: HipTensorHandle, output: HipTensorHandle) -> None:
    """output = silu(gate) * up over [..., n]; rows may be strided (e.g. halves of a fused gate/up)."""
    n = gate.shape[-1]
    if up.shape != gate.shape or output.shape != gate.shape:
        raise ValueError("silu_mul: shapes differ")
    for h in (gate, up, output):
        if h.strides[-1] != 1:
            raise ValueError("silu_mul: last dim must be contiguous")
    rows = gate.numel // n if n else 0

    def row_stride(h):
        if len(h.shape) == 1:
            return n
        # rows must be evenly spaced: all leading dims flatten into one row index
        lead = [(s, st) for s, st in zip(h.shape[:-1], h.strides[:-1]) if s != 1]
        rs = lead[-1][1] if lead else n
        acc = rs
        for s, st in reversed(lead):
            if st != acc:
                raise ValueError("silu_mul: leading dims must flatten to one row stride")
            acc = st * s
        return rs

    _lib.call(
        "kh_silu_mul", _vp(gate.data_ptr()), row_stride(gate), _vp(up.data_ptr()), row_stride(up),
        _vp(output.data_ptr()), row_stride(output), rows, n, output.kh_dtype,
    )


# ---------------------------------------------------------------------------------------------
# copy / gather / argmax / factory
# ---------------------------------------------------------------------------------------------
def index_select(self_: HipTensorHandle, index: HipTensorHandle, params: dict, output: HipTensorHandle) -> None:
    """GatherKernelImpl (gather.ts:121,190): output = self_ with the entries of `index` taken along
    params['dim'] (default 0: rows of an embedding table); output holds self_'s shape with that dim
    replaced by len(index) (dim 0 also accepts index.shape + self_.shape[1:], the embedding form).
    A non-contiguous table is materialised first; ids outside the dim give zeros."""
    nd = len(self_.shape)
    dim = int((params or {}).get("dim", 0))
    if dim < 0:
        dim += nd
    if not 0 <= dim < max(nd, 1):
        raise ValueError(f"index_select: dim {dim} out of range for a {nd}-d tensor")
    if index.dtype != INT32 or not index.is_contiguous():
        raise TypeError("index_select: index must be a contiguous int32 tensor")
    if not output.is_contiguous() or output.dtype not in (FLOAT32, BFLOAT16) or self_.dtype not in (FLOAT32, BFLOAT16):
        raise TypeError("index_select: table and output must be float tensors; output contiguous")
    t = self_ if self_.is_contiguous() else _materialize(self_)
    try:
        shape = list(t.shape) if nd else [1]
        outer = int(np.prod(shape[:dim])) if dim else 1
        inner = int(np.prod(shape[dim + 1:])) if dim + 1 < len(shape) else 1
        if output.numel != outer * index.numel * inner:
            raise ValueError("index_select: output must hold len(index) entries along dim")
        _lib.call(
            "kh_index_select_dim", _vp(t.data_ptr()), outer, shape[dim], inner, _vp(index.data_ptr()), index.numel,
            _vp(output.data_ptr()), t.kh_dtype, output.kh_dtype,
        )
    finally:
        if t is not self_:
            t.dispose()


def argmax(it: TensorIterator) -> None:
    """argmax (reduction/index.ts:20-22; argShaderBuilder.ts:205-240) over the iterator's reduction
    axes (the dispatcher's dim; all axes without one, or the scalar argument 'dim'): the input's
    rows are gathered into [kept, reduced] order with one strided copy and each row's maximum taken
    with the lowest index among maxima (sampling/index.ts:132,138; NaN never wins), int32 output."""
    x = it.input(0).tensor_handle
    nd = len(x.shape)
    if it.is_reduction:
        axes = list(it.reduction_axes)
    else:
        dim = it.get_scalar_arg("dim")
        axes = list(range(nd)) if dim is None else [int(dim[0] if isinstance(dim, (list, tuple)) else dim)]
    axes = [a + nd if a < 0 else a for a in axes]
    if any(not 0 <= a < nd for a in axes):
        raise ValueError(f"argmax: axis out of range for a {nd}-d tensor")
    kept = [i for i in range(nd) if i not in axes]
    perm = kept + axes
    R = int(np.prod([x.shape[a] for a in axes])) if axes else 1
    P = int(np.prod([x.shape[i] for i in kept])) if kept else 1
    if R == 0:
        raise ValueError("argmax: reduction over an empty axis")
    out = it.output(0)
    if out.tensor_handle.dtype != INT32:
        raise TypeError("argmax: the output must be int32")
    if it.output_numel != P:
        raise ValueError(f"argmax: an output of {tuple(it.output_shape)} for {P} rows")
    # rows already contiguous in [kept, reduced] order (the last axis of a contiguous input) into a
    # contiguous int32 output: one launch, no gather or copy
    o = out.tensor_handle if isinstance(out, IteratorOperand) else out
    if axes == list(range(len(kept), nd)) and x.is_contiguous() and o.is_contiguous() and o.numel == P and \
            (not isinstance(out, IteratorOperand) or out.offset == o.offset):
        _lib.call("kh_argmax", _vp(x.data_ptr()), P, R, _vp(o.data_ptr()), x.kh_dtype)
        return
    pshape = tuple(x.shape[i] for i in perm)
    rows = HipTensorHandle.create_new(pshape, x.dtype)
    idx = HipTensorHandle.create_new(tuple(it.output_shape), INT32)
    try:
        src = IteratorOperand(x, x.dtype, pshape, tuple(x.strides[i] for i in perm), x.offset, False)
        map_strided(MAP_OPS["copy"], pshape, rows, src, name="argmax")
        _lib.call("kh_argmax", _vp(rows.data_ptr()), P, R, _vp(idx.data_ptr()), rows.kh_dtype)
        map_strided(MAP_OPS["copy"], it.output_shape, out, idx, name="argmax")
    finally:
        rows.dispose()
        idx.dispose()


GEMV_PROLOGUES = {"none": 0, "rms_norm": 1, "silu_mul": 2, "silu_mul_interleaved": 3}


def interleave_gate_up(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """The fused gate/up weight of linear_swiglu: rows 16i .. 16i + 7 are gate rows 8i .. 8i + 7 and
    rows 16i + 8 .. 16i + 15 the matching up rows (both [I, H], I % 8 == 0)."""
    I, H = gate.shape
    if up.shape != gate.shape or I % 8:
        raise ValueError("interleave_gate_up: gate and up must share a shape [I, H] with I % 8 == 0")
    return np.stack([gate.reshape(I // 8, 8, H), up.reshape(I // 8, 8, H)], axis=1).reshape(2 * I, H)


def linear_swiglu(x, w_gu, output) -> None:
    """output [..., I] = silu(x W_gate^T) * (x W_up^T) from the interleaved bf16 weight w_gu [2I, H]
    (interleave_gate_up); x [..., H] with contiguous rows, x and output bf16 (gate, up and the
    product rounded to bf16) or float32 (all kept in fp32).  The gate/up projections, silu and mul
    of SwiGLUMLP.forward (swiglu.ts:119-134) in one launch (kh_gemm_swiglu)."""
    two_i, H = w_gu.shape
    I = two_i // 2
    if x.dtype not in (BFLOAT16, FLOAT32) or w_gu.dtype != BFLOAT16 or output.dtype != x.dtype:
        raise TypeError("linear_swiglu: a bf16 weight with bf16 or float32 x and output of x's dtype expected")
    if x.shape[-1] != H or tuple(output.shape) != tuple(x.shape[:-1]) + (I,):
        raise ValueError(f"linear_swiglu: x [..., {H}] and output [..., {I}] expected for w_gu {tuple(w_gu.shape)}")
    if x.strides[-1] != 1 or w_gu.strides[1] != 1 or output.strides[-1] != 1:
        raise ValueError("linear_swiglu: rows must be contiguous")
    m = int(np.prod(x.shape[:-1])) if len(x.shape) > 1 else 1
    if len(x.shape) > 2 and not (x.is_contiguous() and output.is_contiguous()):
        raise ValueError("linear_swiglu: batched operands must be contiguous")
    ldx = x.strides[-2] if len(x.shape) >= 2 else H
    ldh = output.strides[-2] if len(output.shape) >= 2 else I
    _lib.call("kh_gemm_swiglu", _vp(x.data_ptr()), ldx, _vp(w_gu.data_ptr()), w_gu.strides[0],
              _vp(output.data_ptr()), ldh, m, I, H, x.kh_dtype)


def linear_qk_norm_rope(x, w_qkv, params) -> None:
    """The QKV projection of a multi-token chunk fused with qk-norm, RoPE and the K/V cache write
    (kh_gemm_qk_norm_rope): x [S, H] bf16 or float32 (contiguous rows; q_out and the caches of the
    same dtype), w_qkv [(Hq + 2 Hkv) D, H] bf16 (q, k, v projection rows concatenated), D = 128.
    params: q_weight, k_weight ([D] bf16), inv_freq
    (float32 [D/2]), positions (int32 [S]), eps, q_out ([1, Hq, S, D] or any [1, Hq, S, D] view with
    a contiguous head dim), k_out / v_out (the KV caches [1, Hkv, max_seq, D]; token t lands in row
    positions[t], rows outside the cache write nothing).  The same values as linear() followed by
    rms_norm_rope(..., cache_positions=True) (gqa.ts:269-309, rope.ts:546-644,
    kv-cache.ts:164-212), without the [S, (Hq + 2 Hkv) D] projection output."""
    q_out, k_out, v_out = params["q_out"], params["k_out"], params["v_out"]
    _, Hq, S, D = q_out.shape
    _, Hkv, L, _ = k_out.shape
    N, H = w_qkv.shape
    if D != 128 or N != (Hq + 2 * Hkv) * D:
        raise ValueError(f"linear_qk_norm_rope: head_dim 128 and w_qkv [(Hq + 2 Hkv) D, H] expected, got D = {D}, "
                         f"w_qkv {tuple(w_qkv.shape)} for Hq = {Hq}, Hkv = {Hkv}")
    if tuple(x.shape) != (S, H) or x.strides[-1] != 1 or w_qkv.strides[1] != 1:
        raise ValueError(f"linear_qk_norm_rope: x [{S}, {H}] with contiguous rows expected, got {tuple(x.shape)}")
    if x.dtype not in (BFLOAT16, FLOAT32) or any(t.dtype != x.dtype for t in (q_out, k_out, v_out)):
        raise TypeError("linear_qk_norm_rope: x, q_out and the caches must share a dtype (bf16 or float32)")
    if w_qkv.dtype != BFLOAT16 or params["q_weight"].dtype != BFLOAT16 or params["k_weight"].dtype != BFLOAT16:
        raise TypeError("linear_qk_norm_rope: the projection and norm weights must be bfloat16")
    if tuple(v_out.shape) != tuple(k_out.shape):
        raise ValueError("linear_qk_norm_rope: K and V caches must have the same shape")
    pos, inv_freq = params["positions"], params["inv_freq"]
    if pos.dtype != INT32 or pos.numel != S:
        raise ValueError("linear_qk_norm_rope: positions must be int32 with S entries")
    if inv_freq.dtype != FLOAT32 or inv_freq.numel != D // 2:
        raise ValueError("linear_qk_norm_rope: inv_freq must be float32 [D/2]")
    for t in (q_out, k_out, v_out):
        if t.strides[-1] != 1:
            raise ValueError("linear_qk_norm_rope: head_dim must be contiguous")
    # (batch, seq, head) strides of the heads-first outputs
    st = []
    for t in (q_out, k_out, v_out):
        st += [t.strides[0], t.strides[2], t.strides[1]]
    table = params.get("rope_table")
    if table is not None and (table.dtype != FLOAT32 or table.numel != S * D or not table.is_contiguous()):
        raise ValueError("linear_qk_norm_rope: rope_table must be rope_table(positions, inv_freq): float32 [S, D/2, 2]")
    _lib.call("kh_gemm_qk_norm_rope_table", _vp(x.data_ptr()), x.strides[0], _vp(w_qkv.data_ptr()),
              w_qkv.strides[0], 1, S, H, Hq, Hkv, D, _vp(params["q_weight"].data_ptr()),
              _vp(params["k_weight"].data_ptr()), _vp(inv_freq.data_ptr()), _vp(pos.data_ptr()),
              _vp(q_out.data_ptr()), _vp(k_out.data_ptr()), _vp(v_out.data_ptr()), _lib.i64_array(st),
              C.c_float(float(params.get("eps", 1e-6))), L, x.kh_dtype,
              _vp(table.data_ptr() if table is not None else None))


def rope_table(positions: HipTensorHandle, inv_freq: HipTensorHandle,
               output: Optional[HipTensorHandle] = None) -> HipTensorHandle:
    """The RoPE angles of a chunk once per forward (kh_rope_table): output [S, D/2, 2] float32 =
    (cos, sin) of float(positions[t]) * inv_freq[i] (rope.ts:193-255); linear_qk_norm_rope reads it
    (params["rope_table"]) in every layer instead of evaluating the angles in each head tile."""
    if positions.dtype != INT32 or not positions.is_contiguous():
        raise TypeError("rope_table: positions must be a contiguous int32 tensor")
    if inv_freq.dtype != FLOAT32 or not inv_freq.is_contiguous():
        raise TypeError("rope_table: inv_freq must be a contiguous float32 tensor")
    S, half = positions.numel, inv_freq.numel
    out = output if output is not None else HipTensorHandle.create_new((S, half, 2), FLOAT32)
    if out.dtype != FLOAT32 or out.numel != S * half * 2 or not out.is_contiguous():
        raise ValueError("rope_table: output must be a contiguous float32 [S, D/2, 2] tensor")
    _lib.call("kh_rope_table", _vp(positions.data_ptr()), S, _vp(inv_freq.data_ptr()), half, _vp(out.data_ptr()))
    return out


def gemm_split_count(m: int, n: int, k: int) -> int:
    """The K split kh_gemm uses for a contiguous bf16 [m, k] x [n, k]^T product (1: none)."""
    out = C.c_int(0)
    _lib.call("kh_gemm_split_count", int(m), int(n), int(k), C.byref(out))
    return out.value


def linear_add_rms_norm(x, w, residual, norm_weight, eps, output, rows=None) -> None:
    """residual += x W^T (fp32, in place) and output = rms_norm(residual) * norm_weight: the
    projection that closes a decoder sub-block, its residual add and the RMSNorm that opens the next
    (decoder_layer.ts:224-238 with RMSNorm.ts:92-99).  x [M, K] (bf16, or float32 activations) and w
    bf16 [N, K] with contiguous rows, residual fp32 [M, N] contiguous, norm_weight [N] and output
    [R, N] of one dtype (bf16 or fp32).  rows = (r0, r1) restricts the add and the norm to residual rows r0 .. r1 - 1
    (output has r1 - r0 rows; the other residual rows are left as they were), default all rows.
    When kh_gemm would split K for this shape, the partials go straight into kh_add_rms_norm
    (two launches instead of GEMM + split reduction + RMSNorm); the values are those of the
    separate launches bit for bit either way."""
    M, K = x.shape
    N = w.shape[0]
    r0, r1 = rows if rows is not None else (0, M)
    if x.dtype not in (BFLOAT16, FLOAT32) or w.dtype != BFLOAT16 or residual.dtype != FLOAT32:
        raise TypeError("linear_add_rms_norm: bf16 or float32 x and a bf16 w with an fp32 residual expected")
    if w.shape[1] != K or tuple(residual.shape) != (M, N) or tuple(output.shape) != (r1 - r0, N):
        raise ValueError("linear_add_rms_norm: shapes do not match")
    if norm_weight.numel != N or norm_weight.dtype != output.dtype:
        raise ValueError("linear_add_rms_norm: norm_weight must have N elements and the output dtype")
    if not (0 <= r0 < r1 <= M):
        raise ValueError(f"linear_add_rms_norm: bad row range {rows} for {M} rows")
    for h, nm in ((x, "x"), (w, "w"), (residual, "residual"), (output, "output"), (norm_weight, "norm_weight")):
        if not h.is_contiguous():
            raise ValueError(f"linear_add_rms_norm: {nm} must be contiguous")
    splits = gemm_split_count(M, N, K)
    aligned = all(h.data_ptr() % 16 == 0 for h in (x, w, residual, output, norm_weight))
    if splits > 1 and aligned and N % 8 == 0 and N <= 2048:
        part = HipTensorHandle.create_new((splits, M, N), FLOAT32)
        try:
            _lib.call("kh_gemm_splitk_partials", _vp(x.data_ptr()), K, _vp(w.data_ptr()), K, _vp(part.data_ptr()),
                      M, N, K, splits, x.kh_dtype)
            _lib.call("kh_add_rms_norm", _vp(part.data_ptr() + r0 * N * 4), splits, M * N,
                      _vp(residual.data_ptr() + r0 * N * 4), _vp(norm_weight.data_ptr()), _vp(output.data_ptr()),
                      r1 - r0, N, C.c_float(eps), output.kh_dtype)
        finally:
            part.dispose()
        return
    _lib.call("kh_gemm_ex", _vp(x.data_ptr()), K, x.kh_dtype, _vp(w.data_ptr()), K, w.kh_dtype,
              _vp(residual.data_ptr()), N, _vp(residual.data_ptr()), N, None, M, N, K, C.c_float(1.0), C.c_float(1.0),
              1, residual.kh_dtype)
    _lib.call("kh_rms_norm", _vp(residual.data_ptr() + r0 * N * 4), N, _vp(norm_weight.data_ptr()),
              _vp(output.data_ptr()), N, r1 - r0, N, C.c_float(eps), residual.kh_dtype, output.kh_dtype)


def gemv_fused(prologue: str, x, w, out, params=None) -> None:
    """One-row projection with its producer fused in front (decode): out[1, n] = alpha * x' W^T
    + beta * cin (+ bias) for the bf16 weight W [n, k] (nn.Linear layout), where x' is
      'none'     -> x ([k]);
      'rms_norm' -> rms_norm(x, norm_weight, eps) of the fp32 residual row x;
      'silu_mul' -> silu(x) * x2 of the gate/up rows;
      'silu_mul_interleaved' -> the same product read from one row [2k] holding gate and up
                    interleaved in blocks of 8 (the output of a linear with interleave_gate_up's weight).
    params: act_dtype (the activations' dtype, default bfloat16: x' rounded to bf16 and x, x2 of
    'none' / 'silu_mul*' bf16; float32: x' kept in fp32 and x, x2 float32), norm_weight, eps, x2,
    cin, alpha, beta, bias.  out may alias cin (residual add).
    Fuses RMSNorm.ts:92-99 or swiglu.ts:119-134 into Linear.ts:135-137."""
    params = params or {}
    code = GEMV_PROLOGUES[prologue]
    n, k = w.shape
    if w.dtype != BFLOAT16 or w.strides[1] != 1:
        raise TypeError("gemv_fused: the weight must be bf16 with contiguous rows")
    act = params.get("act_dtype") or BFLOAT16
    if act not in (BFLOAT16, FLOAT32):
        raise TypeError(f"gemv_fused: act_dtype must be bfloat16 or float32, not {act}")
    want = FLOAT32 if prologue == "rms_norm" else act
    x2 = params.get("x2")
    for h, nm in ((x, "x"), (x2, "x2")):
        if h is None:
            continue
        kx = 2 * k if prologue == "silu_mul_interleaved" else k
        if h.dtype != want or h.numel != kx or (len(h.shape) > 0 and h.strides[-1] != 1):
            raise ValueError(f"gemv_fused: {nm} must be one contiguous {want} row of {kx} elements")
    if prologue == "silu_mul" and x2 is None:
        raise ValueError("gemv_fused: silu_mul needs x2")
    nw = params.get("norm_weight")
    if prologue == "rms_norm" and (nw is None or nw.dtype != BFLOAT16 or nw.numel != k):
        raise ValueError("gemv_fused: rms_norm needs a bf16 norm_weight of k elements")
    if out.numel != n or not out.is_contiguous() or out.dtype not in (FLOAT32, BFLOAT16):
        raise ValueError("gemv_fused: out must be a contiguous float row of n elements")
    cin, bias = params.get("cin"), params.get("bias")
    for h, nm in ((cin, "cin"), (bias, "bias")):
        if h is not None and (h.numel != n or not h.is_contiguous() or h.dtype != out.dtype):
            raise ValueError(f"gemv_fused: {nm} must be a contiguous row of n elements in the output dtype")
    beta = float(params.get("beta", 1.0 if cin is not None else 0.0))
    _lib.call(
        "kh_gemv_fused", code, _vp(x.data_ptr()), _vp(x2.data_ptr()) if x2 is not None else None,
        _vp(nw.data_ptr()) if nw is not None else None, C.c_float(float(params.get("eps", 1e-6))),
        _vp(w.data_ptr()), w.strides[0], _vp(out.data_ptr()), _vp(cin.data_ptr()) if cin is not None else None,
        _vp(bias.data_ptr()) if bias is not None else None, n, k, C.c_float(float(params.get("alpha", 1.0))),
        C.c_float(beta), out.kh_dtype, KH_CODE[act],
    )


def gemv_swiglu(prologue: str, x, w_gu, out, params=None) -> None:
    """One-row SwiGLU projection (decode): out[1, I] = silu(x' W_gate^T) * (x' W_up^T), from the
    gate/up weight w_gu [2I, H] interleaved in blocks of 8 rows (interleave_gate_up), where x' is
    'none' -> x ([H]) or 'rms_norm' -> rms_norm(x, norm_weight, eps) of the fp32 residual row.
    out's dtype is the activations': bfloat16 (x' and gate and up rounded to bf16 before the
    product, as gemv_fused's gate/up row followed by the 'silu_mul_interleaved' prologue forms it;
    x of 'none' bf16) or float32 (all kept in fp32; x of 'none' float32) (swiglu.ts:119-134 for
    one token).  params: norm_weight, eps."""
    params = params or {}
    if prologue not in ("none", "rms_norm"):
        raise ValueError(f"gemv_swiglu: prologue must be 'none' or 'rms_norm', not {prologue!r}")
    two_i, k = w_gu.shape
    n_half = two_i // 2
    if w_gu.dtype != BFLOAT16 or w_gu.strides[1] != 1:
        raise TypeError("gemv_swiglu: the weight must be bf16 with contiguous rows")
    act = out.dtype
    if act not in (BFLOAT16, FLOAT32) or out.numel != n_half or not out.is_contiguous():
        raise ValueError(f"gemv_swiglu: out must be a contiguous bf16 or float32 row of {n_half} elements")
    want = FLOAT32 if prologue == "rms_norm" else act
    if x.dtype != want or x.numel != k or not x.is_contiguous():
        raise ValueError(f"gemv_swiglu: x must be one contiguous {want} row of {k} elements")
    nw = params.get("norm_weight")
    if prologue == "rms_norm" and (nw is None or nw.dtype != BFLOAT16 or nw.numel != k):
        raise ValueError("gemv_swiglu: rms_norm needs a bf16 norm_weight of k elements")
    _lib.call("kh_gemv_swiglu", GEMV_PROLOGUES[prologue], _vp(x.data_ptr()),
              _vp(nw.data_ptr()) if nw is not None else None, C.c_float(float(params.get("eps", 1e-6))),
              _vp(w_gu.data_ptr()), w_gu.strides[0], _vp(out.data_ptr()), n_half, k, out.kh_dtype)


def greedy_advance(next_token, position, seq_len, token_log, log_base: int) -> None:
    """Device-side step of the greedy loop (for_causal_lm.ts:475-508): with p = position[0],
    token_log[p + 1 - log_base] = next_token[0] (when inside the log), position = p + 1,
    seq_len = p + 2.  All operands are int32 device tensors."""
    for h in (next_token, position, seq_len, token_log):
        if h.dtype != INT32 or not h.is_contiguous():
            raise TypeError("greedy_advance: operands must be contiguous int32 tensors")
    _lib.call("kh_greedy_advance", _vp(next_token.data_ptr()), _vp(position.data_ptr()), _vp(seq_len.data_ptr()),
              _vp(token_log.data_ptr()), int(log_base), token_log.numel)


def sample(logits, params: dict):
    """Choose one token from a [vocab] (or [1, vocab]) float32 logits row on the device
    (sampling/index.ts:103-243).  params: do_sample (True; False = greedy), temperature (1.0),
    top_k (0 = off), top_p (1.0 = off), seed (int), counter (int32 device tensor [1]; r comes from
    philox4x32-10(seed, counter); unused when greedy), display_k (0), and the outputs token (int32 [1]),
    logprob (float32 [1], optional), display_ids (int32 [display_k], optional) and display_probs
    (float32 [display_k], optional)."""
    if logits.dtype != FLOAT32 or not logits.is_contiguous():
        raise TypeError("sample: logits must be a contiguous float32 tensor")
    vocab = logits.shape[-1]
    if logits.numel != vocab:
        raise ValueError(f"sample: one row of logits expected, got shape {list(logits.shape)}")
    do_sample = bool(params.get("do_sample", True))
    ctr, tok = params.get("counter"), params["token"]
    for name, h in (("counter", ctr), ("token", tok)):
        if h is None and name == "counter" and not do_sample:
            continue
        if h is None or h.dtype != INT32 or h.numel < 1:
            raise TypeError(f"sample: {name} must be an int32 tensor with one element")
    dk = int(params.get("display_k", 0))
    ptr = lambda h: _vp(h.data_ptr()) if h is not None else _vp(0)  # noqa: E731
    dids, dprobs = params.get("display_ids"), params.get("display_probs")
    if dk and ((dids is not None and dids.numel < dk) or (dprobs is not None and dprobs.numel < dk)):
        raise ValueError("sample: display outputs shorter than display_k")
    _lib.call("kh_sample", _vp(logits.data_ptr()), vocab, int(do_sample), float(params.get("temperature", 1.0)),
              int(params.get("top_k", 0)), float(params.get("top_p", 1.0)), C.c_uint64(int(params.get("seed", 0))),
              ptr(ctr), _vp(tok.data_ptr()), ptr(params.get("logprob")), dk, ptr(dids), ptr(dprobs))


def sample_set_path(path: int) -> None:
    """Select kh_sample's implementation: 0 the selection path where it applies (default), 1 the
    full sort for every call (both give the same results; used by tests)."""
    _lib.call("kh_sample_set_path", int(path))


def philox4x32_10(seed: int, counters, out) -> None:
    """out[i] = philox4x32-10(counters[i], key = seed) for uint32 [n, 4] device tensors (int32 storage)."""
    if counters.numel % 4 or out.numel != counters.numel:
        raise ValueError("philox4x32_10: counters and out must be [n, 4]")
    _lib.call("kh_philox4x32_10", C.c_uint64(int(seed)), _vp(counters.data_ptr()), counters.numel // 4,
              _vp(out.data_ptr()))


KERNELS = {
    "sample": sample,
    "decode_attention_block": decode_attention_block,
    "flash_attention": flash_attention,
    "flash_attention_split": flash_attention_split,
    "sdpa_masked": sdpa_masked,
    "decode_attention": decode_attention,
    "matmul": matmul,
    "mm": matmul,
    "bmm": matmul,
    "addmm": matmul,
    "baddbmm": matmul,
    "rms_norm": rms_norm,
    "rms_norm_rope": rms_norm_rope,
    "silu": silu,
    "neg": neg,
    "cos": cos,
    "sin": sin,
    "arange": arange,
    "mul": mul,
    "add": add,
    "sub": sub,
    "silu_mul": silu_mul,
    "linear_swiglu": linear_swiglu,
    "linear_qk_norm_rope": linear_qk_norm_rope,
    "rope_table": rope_table,
    "linear_add_rms_norm": linear_add_rms_norm,
    "copy": copy,
    "contiguous": contiguous,
    "cast": cast,
    "clone": clone,
    "copy_": copy_,
    "div": div,
    "ones": ones,
    "full": full,
    "empty": empty,
    "index_select": index_select,
    "argmax": argmax,
    "greedy_advance": greedy_advance,
    "gemv_fused": gemv_fused,
    "gemv_swiglu": gemv_swiglu,
    "zeros": zeros,
}
