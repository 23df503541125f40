"""CPU oracle for Kandle's transformer hot path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() (as the checker) and bench.py's cpu_baseline leg may import
this package.  The product (kandle_amd) never imports, links or calls it.

The math lives in oracle.c (a C restatement of the reference algorithms, each function citing the
reference file:line it follows); this module builds it with the Makefile beside it and wraps it with
numpy.  Parity pinning of every function is done in tests/test_oracle.py against closed forms,
invariants, brute force on tiny inputs and the torch-generated golden vectors in tests/golden/.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

_lib = None


def build(force: bool = False) -> Path:
    """Compile oracle.c into liboracle.so with gcc (via the Makefile)."""
    if force or not LIB_PATH.exists() or LIB_PATH.stat().st_mtime < (HERE / "oracle.c").stat().st_mtime:
        subprocess.run(["make", "-s", "-C", str(HERE), "-B" if force else "all"], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        build()
        L = C.CDLL(str(LIB_PATH))
        f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
        u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
        i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
        f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
        i64 = C.c_int64
        L.or_f32_to_bf16.argtypes = [f32p, u16p, i64]
        L.or_bf16_to_f32.argtypes = [u16p, f32p, i64]
        L.or_sdpa.argtypes = [f32p, f32p, f32p, f32p, C.c_int, C.c_int, C.c_int, i64, i64, C.c_int, C.c_float,
                              C.c_int, C.c_void_p, f64p]
        L.or_rms_norm.argtypes = [f32p, C.c_void_p, f32p, i64, i64, C.c_float]
        L.or_rope_inv_freq.argtypes = [f32p, C.c_int, C.c_double]
        L.or_qk_norm_rope.argtypes = [f32p, C.c_void_p, f32p, i64, C.c_int, C.c_int, i32p, f32p, C.c_float, C.c_int]
        L.or_silu_mul.argtypes = [f32p, C.c_void_p, f32p, i64]
        L.or_linear.argtypes = [f32p, f32p, C.c_void_p, C.c_void_p, f32p, i64, i64, i64, C.c_float, C.c_float]
        L.or_argmax.argtypes = [f32p, i64, i64, i32p]
        L.or_sdpa_masked.argtypes = [f32p, f32p, f32p, f32p, C.c_int, C.c_int, C.c_int, i64, i64, C.c_int,
                                     C.c_float, C.c_void_p, i64, i64, i64, i64, f64p]
        L.or_flash_f32.argtypes = [f32p, f32p, f32p, f32p, C.c_int, C.c_int, C.c_int, i64, i64, C.c_int, C.c_float,
                                   C.c_int, i64]
        for fn in ("or_f32_to_bf16", "or_bf16_to_f32", "or_sdpa", "or_rms_norm", "or_rope_inv_freq",
                   "or_qk_norm_rope", "or_silu_mul", "or_linear", "or_argmax", "or_flash_f32"):
            getattr(L, fn).restype = None
        _lib = L
    return _lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a):
    return None if a is None else a.ctypes.data


# ---- bf16 -----------------------------------------------------------------------------------
def to_bf16_bits(x) -> np.ndarray:
    x = _f32(x)
    out = np.empty(x.shape, np.uint16)
    lib().or_f32_to_bf16(x.reshape(-1), out.reshape(-1), x.size)
    return out


def from_bf16_bits(b) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint16)
    out = np.empty(b.shape, np.float32)
    lib().or_bf16_to_f32(b.reshape(-1), out.reshape(-1), b.size)
    return out


def bf16_round(x) -> np.ndarray:
    """float32 values rounded to the nearest bf16 (ties to even), returned as float32."""
    return from_bf16_bits(to_bf16_bits(x))


# ---- ops ------------------------------------------------------------------------------------
def sdpa(q, k, v, scale=None, causal=False, kv_len=None) -> np.ndarray:
    """q [B,Hq,Lq,D], k/v [B,Hkv,Lk,D] -> o [B,Hq,Lq,D] (double accumulation)."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    B, Hq, Lq, D = q.shape
    _, Hkv, Lk, _ = k.shape
    if scale is None:
        scale = 1.0 / np.sqrt(D)
    o = np.zeros((B, Hq, Lq, D), np.float32)
    work = np.zeros(max(Lk, 1), np.float64)
    kl = None if kv_len is None else np.ascontiguousarray(kv_len, dtype=np.int32)
    lib().or_sdpa(q, k, v, o, B, Hq, Hkv, Lq, Lk, D, float(scale), int(bool(causal)), _ptr(kl), work)
    return o


def sdpa_masked(q, k, v, mask, scale=None) -> np.ndarray:
    """softmax(scale * Q K^T + mask) V with the reference's softmax (row max floored at -1e38, a
    row summing to 0 gives NaN); mask broadcasts to [B, Hq, Lq, Lk] (numpy rules)."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    B, Hq, Lq, D = q.shape
    _, Hkv, Lk, _ = k.shape
    if scale is None:
        scale = 1.0 / np.sqrt(D)
    m = np.broadcast_to(np.asarray(mask, dtype=np.float32), (B, Hq, Lq, Lk))
    ms = [st // 4 for st in m.strides]
    o = np.zeros((B, Hq, Lq, D), np.float32)
    work = np.zeros(max(Lk, 1), np.float64)
    lib().or_sdpa_masked(q, k, v, o, B, Hq, Hkv, Lq, Lk, D, float(scale), C.c_void_p(m.ctypes.data),
                         ms[0], ms[1], ms[2], ms[3], work)
    return o


def flash_f32(q, k, v, scale=None, causal=False, heads_limit=0) -> np.ndarray:
    """The reference's blockwise online-softmax algorithm in float32 (the timed CPU baseline).
    heads_limit > 0 processes only the first heads_limit (b, h) pairs (a bounded sample)."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    B, Hq, Lq, D = q.shape
    _, Hkv, Lk, _ = k.shape
    if scale is None:
        scale = 1.0 / np.sqrt(D)
    o = np.zeros((B, Hq, Lq, D), np.float32)
    lib().or_flash_f32(q, k, v, o, B, Hq, Hkv, Lq, Lk, D, float(scale), int(bool(causal)), int(heads_limit))
    return o


def node_available() -> bool:
    """True when a `node` executable runs here (the JS restatement needs it)."""
    import shutil
    import subprocess
    exe = shutil.which("node")
    if exe is None:
        return False
    try:
        return subprocess.run([exe, "--version"], capture_output=True, timeout=30).returncode == 0
    except (OSError, subprocess.SubprocessError):
        return False


def flash_js(q, k, v, scale=None, causal=False, heads_limit=0):
    """The reference flash algorithm restated in JavaScript (oracle/js/flash_sdpa.js), run by Node:
    (o [B,Hq,Lq,D] float32, wall ms of the computation inside Node).  heads_limit > 0 computes only
    the first heads_limit (b, h) pairs (a bounded sample; the other rows stay zero)."""
    import json
    import subprocess
    import tempfile
    q, k, v = _f32(q), _f32(k), _f32(v)
    B, Hq, Lq, D = q.shape
    _, Hkv, Lk, _ = k.shape
    if scale is None:
        scale = 1.0 / np.sqrt(D)
    script = os.path.join(os.path.dirname(os.path.abspath(__file__)), "js", "flash_sdpa.js")
    with tempfile.TemporaryDirectory() as d:
        for name, a in (("q", q), ("k", k), ("v", v)):
            a.tofile(os.path.join(d, name + ".f32"))
        out = subprocess.run(["node", script, d, str(B), str(Hq), str(Hkv), str(Lq), str(Lk), str(D), repr(float(scale)),
                              "1" if causal else "0", str(int(heads_limit))], capture_output=True, text=True, check=True)
        o = np.fromfile(os.path.join(d, "o.f32"), dtype=np.float32).reshape(B, Hq, Lq, D)
    return o, float(json.loads(out.stdout.strip().splitlines()[-1])["ms"])


def js_bench(op, inputs, args, repeat=1, outputs=()):
    """Runs oracle/js/bench_cpu.js OP on float32 inputs {name: array} with numeric ARGS: one untimed
    run, then `repeat` timed runs on one Node thread.  Returns ({name: float32 array} for the
    requested output files, [ms of each timed run])."""
    import json
    import subprocess
    import tempfile
    script = os.path.join(os.path.dirname(os.path.abspath(__file__)), "js", "bench_cpu.js")
    with tempfile.TemporaryDirectory() as d:
        for name, a in inputs.items():
            _f32(a).tofile(os.path.join(d, name + ".f32"))
        cmd = ["node", script, op, d, str(int(repeat))] + [repr(float(x)) if isinstance(x, float) else str(x)
                                                           for x in args]
        out = subprocess.run(cmd, capture_output=True, text=True, check=True)
        res = {name: np.fromfile(os.path.join(d, name + ".f32"), dtype=np.float32) for name in outputs}
    return res, [float(x) for x in json.loads(out.stdout.strip().splitlines()[-1])["runs_ms"]]


def js_qwen3_timing(cfg, prompt_len: int, decode_steps: int, seed: int = 7) -> dict:
    """oracle/js/bench_cpu.js qwen3: ONE decoder layer of `cfg`'s shapes (seeded weights) in Node on
    one thread -- the prefill of prompt_len ids, then decode_steps greedy one-token forwards, and the
    lm_head row alone.  Returns {"prefill_ms", "decode_ms" (per step), "head_ms", "last_token"}."""
    import json
    import subprocess
    script = os.path.join(os.path.dirname(os.path.abspath(__file__)), "js", "bench_cpu.js")
    args = [cfg.hidden_size, cfg.intermediate_size, cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim,
            cfg.vocab_size, int(prompt_len), int(decode_steps), repr(float(cfg.rms_norm_eps)),
            repr(float(cfg.rope_theta)), int(seed)]
    out = subprocess.run(["node", script, "qwen3", ".", "1"] + [str(a) for a in args], capture_output=True,
                         text=True, check=True)
    return json.loads(out.stdout.strip().splitlines()[-1])


def rms_norm(x, w=None, eps=1e-6) -> np.ndarray:
    x = _f32(x)
    n = x.shape[-1]
    rows = x.size // n
    wv = None if w is None else _f32(w)
    y = np.empty_like(x)
    lib().or_rms_norm(x.reshape(-1), _ptr(wv), y.reshape(-1), rows, n, float(eps))
    return y


def rope_inv_freq(head_dim: int, theta: float) -> np.ndarray:
    out = np.empty(head_dim // 2, np.float32)
    lib().or_rope_inv_freq(out, head_dim, float(theta))
    return out


def qk_norm_rope(x, w, positions, inv_freq, eps=1e-6, do_norm=True) -> np.ndarray:
    """x [T, H, D] -> RoPE(rms_norm(x) * w) with per-token positions [T]."""
    x = _f32(x)
    T, H, D = x.shape
    wv = None if w is None else _f32(w)
    out = np.empty_like(x)
    pos = np.ascontiguousarray(positions, dtype=np.int32)
    lib().or_qk_norm_rope(x, _ptr(wv), out, T, H, D, pos, _f32(inv_freq), float(eps), int(bool(do_norm)))
    return out


def silu_mul(g, u=None) -> np.ndarray:
    g = _f32(g)
    uv = None if u is None else _f32(u)
    out = np.empty_like(g)
    lib().or_silu_mul(g.reshape(-1), _ptr(uv), out.reshape(-1), g.size)
    return out


def linear(a, w, cin=None, bias=None, alpha=1.0, beta=0.0) -> np.ndarray:
    """a [M, K], w [N, K] -> alpha * a w^T + beta * cin + bias, double accumulation."""
    a, w = _f32(a), _f32(w)
    M, K = a.shape
    N = w.shape[0]
    c = np.empty((M, N), np.float32)
    ci = None if cin is None else _f32(cin)
    bi = None if bias is None else _f32(bias)
    lib().or_linear(a, w, _ptr(ci), _ptr(bi), c, M, N, K, float(alpha), float(beta))
    return c


def argmax_workgroup_rule(x, wg=256) -> np.ndarray:
    """The reference argmax kernel's tie rule, restated for comparison only, by simulating the
    kernel: thread t of a workgroup of wg threads (a power of two) keeps the first strict maximum of
    indices t, t + wg, t + 2 wg, ... (packages/backend-webgpu/src/kernels/reduction/
    argShaderBuilder.ts:214-228); then for stride = wg/2, wg/4, ..., 1 position p < stride takes
    position p + stride's value only when it is strictly greater (:86-98), and position 0 is the
    result.  Among tied maxima the result depends on wg and is not the lowest index in general."""
    x = np.asarray(x, np.float32)
    x2 = x.reshape(-1, x.shape[-1])
    out = np.zeros(x2.shape[0], np.int32)
    lowest = -np.float32(3.4028234663852886e38)
    for r, row in enumerate(x2):
        vals = [lowest] * wg
        idxs = [0] * wg
        for t in range(wg):
            for i in range(t, row.size, wg):
                if row[i] > vals[t]:
                    vals[t], idxs[t] = row[i], i
        stride = wg // 2
        while stride >= 1:
            for p in range(stride):
                if vals[p + stride] > vals[p]:
                    vals[p], idxs[p] = vals[p + stride], idxs[p + stride]
            stride //= 2
        out[r] = idxs[0]
    return out.reshape(x.shape[:-1])


def argmax(x) -> np.ndarray:
    x = _f32(x)
    n = x.shape[-1]
    rows = x.size // n
    out = np.empty(rows, np.int32)
    lib().or_argmax(x.reshape(-1), rows, n, out)
    return out.reshape(x.shape[:-1])


__all__ = [n for n in dir() if not n.startswith("_")]
