"""Benchmark of the Kandle hot path on one MI355X.

Headline (BASELINE.json metric): causal GQA flash-attention prefill TFLOP/s on config C3
(B=4, Hq=16, Hkv=8, S=4096, D=128, bf16, fp32 accumulate).  A "step" is one prefill call over that
batch with inputs resident in HBM.  The same run also measures decode attention (config C4: B=8,
Hq=16, Hkv=8, D=128, per-sequence KV lengths ~ U[8192, 32768]) in HBM GB/s and the fused RMSNorm +
qk-norm + RoPE (config C2) in GB/s, each against its roofline, and times the CPU oracle's flash
algorithm on a bounded sample as the CPU baseline.

It also runs the full Qwen3-0.6B model of config C5 (512-token prefill, 128 greedy decode steps)
and reports prefill tokens/s and TFLOP/s and decode tokens/s and GB/s against their rooflines.
`--only copy` runs the 1 GiB copy that calibrates the HBM traffic counters; `--only mask` times the
explicit-mask SDPA route at C3 shapes; `--only prefill_b1` the causal prefill of one sequence at
512 to 4096 tokens.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu-baseline]
                    [--only prefill|decode|norm|model|copy|load|sample|stream|gemm|gemv|vendor|mask|prefill_b1]
Prints ONE JSON line.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402

METRIC = "flash-attn prefill TFLOP/s (%MFMA peak) S=4096; decode-attn HBM GB/s @32k KV"
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_HBM_GBPS = 8000.0     # MI355X HBM3E


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def bf16_tensor(seed, shape):
    from kandle_amd import Tensor
    from kandle_amd import synthetic as syn

    bits, _ = syn.bf16(syn.normal(seed, shape))
    return Tensor(bits, dtype="bfloat16")


def time_calls(fn, steps, warmup, lead=None):
    """(wall ms per call, device ms per call from HIP events on the library stream): `warmup` untimed
    calls, a synchronisation, `steps` calls bracketed by events, a synchronisation.  `lead`, when
    given, is enqueued right before the warm-up calls with no synchronisation in between (see
    main: the explicit-mask leg leads the headline)."""
    from kandle_amd import _lib

    if lead is not None:
        lead()
    for _ in range(warmup):
        fn()
    _lib.synchronize()
    e0, e1 = _lib.Event(), _lib.Event()
    t0 = time.perf_counter()
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    _lib.synchronize()
    t1 = time.perf_counter()
    return (t1 - t0) * 1e3 / steps, e0.elapsed_ms(e1) / steps


def enqueue_timed(fn, steps, warmup):
    """Enqueues `warmup` calls, a synchronisation, then `steps` calls bracketed by events, and returns
    without waiting for them; read the device ms per call with finish_timed after a later sync."""
    from kandle_amd import _lib

    for _ in range(warmup):
        fn()
    _lib.synchronize()
    e0, e1 = _lib.Event(), _lib.Event()
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    return e0, e1, steps


def finish_timed(handle):
    e0, e1, steps = handle
    return e0.elapsed_ms(e1) / steps


# Each prep_* function uploads its inputs and returns run(steps, warmup) -> result dict (the run
# frees what the prep allocated).  main() prepares every leg first and then runs the GPU legs back
# to back, the headline last: the GPU reaches its steady clock only after several ms of sustained
# load (C3 prefill measured 0.34 ms per call over 20 calls after 3 warm-up calls from idle, 0.296 ms
# once the clock has settled), so the headline is timed at the clock a loaded GPU runs at, with no
# input generation or CPU work between the legs.

def prep_prefill():
    from kandle_amd import HipTensorHandle, kernels

    B, Hq, Hkv, S, D = 4, 16, 8, 4096, 128
    q = bf16_tensor(301, (B, Hq, S, D))
    k = bf16_tensor(302, (B, Hkv, S, D))
    v = bf16_tensor(303, (B, Hkv, S, D))
    o = HipTensorHandle.create_new((B, Hq, S, D), "bfloat16")
    scale = 1.0 / np.sqrt(D)

    def run(steps, warmup, lead=None):
        fn = lambda: kernels.flash_attention(q.handle, k.handle, v.handle, o, scale, True)  # noqa: E731
        wall_ms, dev_ms = time_calls(fn, steps, warmup, lead=lead)
        flops = 4.0 * B * Hq * S * S * D / 2.0
        out = o.data_async()
        assert np.all(np.isfinite(out)), "prefill produced non-finite values"
        for t in (q, k, v):
            t.dispose()
        o.dispose()
        return {"B": B, "Hq": Hq, "Hkv": Hkv, "S": S, "D": D, "flops": flops, "wall_ms": wall_ms, "dev_ms": dev_ms}
    return run


def prep_c1():
    """Config C1 on the GPU: SDPA in fp32, B=1, Hq=16, Hkv=8, S=256, D=128, causal, scale 1/sqrt(128)
    (the fp32 MFMA flash kernel)."""
    from kandle_amd import HipTensorHandle, Tensor, kernels
    from kandle_amd import synthetic as syn

    B, Hq, Hkv, S, D = 1, 16, 8, 256, 128
    q = Tensor(syn.normal(11, (B, Hq, S, D)))
    k = Tensor(syn.normal(12, (B, Hkv, S, D)))
    v = Tensor(syn.normal(13, (B, Hkv, S, D)))
    o = HipTensorHandle.create_new((B, Hq, S, D), "float32")
    scale = 1.0 / np.sqrt(D)

    def run(steps, warmup):
        fn = lambda: kernels.flash_attention(q.handle, k.handle, v.handle, o, scale, True)  # noqa: E731
        wall_ms, dev_ms = time_calls(fn, steps, warmup)
        # the same call in split-bf16 form (kh_flash_attention_split: three bf16 MFMAs per product,
        # within about 2^-15 of the fp32 products), the float32-activation model's prefill attention
        fs = lambda: kernels.flash_attention_split(q.handle, k.handle, v.handle, o, scale, True)  # noqa: E731
        split_wall, split_dev = time_calls(fs, steps, warmup)
        for t in (q, k, v):
            t.dispose()
        o.dispose()
        flops = 4.0 * B * Hq * S * S * D / 2.0
        return {"flops": flops, "wall_ms": wall_ms, "dev_ms": dev_ms, "split_wall_ms": split_wall,
                "split_dev_ms": split_dev}
    return run


def prep_mask():
    """C3 shapes with an explicit [S, S] float32 mask (the top-left causal pattern as -inf / 0):
    the masked route scores every (query, key) pair, so the work is the full 4 B Hq S^2 D."""
    from kandle_amd import HipTensorHandle, Tensor, kernels

    B, Hq, Hkv, S, D = 4, 16, 8, 4096, 128
    q = bf16_tensor(301, (B, Hq, S, D))
    k = bf16_tensor(302, (B, Hkv, S, D))
    v = bf16_tensor(303, (B, Hkv, S, D))
    m = Tensor(np.where(np.arange(S)[None, :] > np.arange(S)[:, None], -np.inf, 0.0).astype(np.float32))
    o = HipTensorHandle.create_new((B, Hq, S, D), "bfloat16")
    scale = 1.0 / np.sqrt(D)

    fn = lambda: kernels.sdpa_masked(q.handle, k.handle, v.handle, m.handle, o, scale)  # noqa: E731

    def result(dev_ms, wall_ms=None):
        flops = 4.0 * B * Hq * S * S * D
        out = o.data_async()
        assert np.all(np.isfinite(out)), "masked prefill produced non-finite values"
        for t in (q, k, v, m):
            t.dispose()
        o.dispose()
        tf = flops / (dev_ms * 1e-3) / 1e12
        return {"workload": "C3 shapes with an explicit [4096, 4096] float32 mask (causal pattern), all pairs scored",
                "flops": flops, "ms": round(dev_ms, 4), "wall_ms": None if wall_ms is None else round(wall_ms, 4),
                "TFLOP/s": round(tf, 1),
                "roofline": {"bound": "mfma", "achieved": round(tf, 1), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                             "frac": round(tf / PEAK_BF16_TFLOPS, 4)},
                "kernel": "flash_fwd_kernel<64, 8, 1, false, 1>"}

    def run(steps, warmup):
        wall_ms, dev_ms = time_calls(fn, steps, warmup)
        return result(dev_ms, wall_ms)

    def enqueue(steps, warmup):
        return enqueue_timed(fn, steps, warmup)

    run.enqueue, run.result = enqueue, result
    return run


C4_SHAPE = dict(B=8, Hq=16, Hkv=8, D=128, ML=32768)


def c4_lengths():
    """The per-sequence KV lengths of config C4: 8 draws from U[8192, 32768] (seed 2024)."""
    from kandle_amd import synthetic as syn
    return syn.randint(2024, (C4_SHAPE["B"],), 8192, 32769)


def prep_decode():
    from kandle_amd import HipTensorHandle, Tensor, kernels

    B, Hq, Hkv, D, ML = (C4_SHAPE[x] for x in ("B", "Hq", "Hkv", "D", "ML"))
    lens = c4_lengths()
    q = bf16_tensor(401, (B, Hq, D))
    kc = bf16_tensor(402, (B, Hkv, ML, D))
    vc = bf16_tensor(403, (B, Hkv, ML, D))
    sl = Tensor(lens, dtype="int32")
    o = HipTensorHandle.create_new((B, Hq, D), "bfloat16")
    scale = 1.0 / np.sqrt(D)

    def run(steps, warmup):
        fn = lambda: kernels.decode_attention(q.handle, kc.handle, vc.handle, sl.handle, o, scale)  # noqa: E731
        wall_ms, dev_ms = time_calls(fn, steps, warmup)
        kv_bytes = float(lens.sum()) * Hkv * D * 2 * 2
        # Head dim 64 over the same K/V bytes: the caches' storage read as [B, Hkv, 2 ML, 64] rows
        # (a view, no copy) with twice the C4 lengths.
        D64 = 64
        q64 = bf16_tensor(404, (B, Hq, D64))
        sl64 = Tensor((2 * lens).astype(np.int32), dtype="int32")
        o64 = HipTensorHandle.create_new((B, Hq, D64), "bfloat16")
        st64 = (Hkv * 2 * ML * D64, 2 * ML * D64, D64, 1)
        kc64 = HipTensorHandle.create_view(kc.handle.storage, (B, Hkv, 2 * ML, D64), "bfloat16", st64, 0)
        vc64 = HipTensorHandle.create_view(vc.handle.storage, (B, Hkv, 2 * ML, D64), "bfloat16", st64, 0)
        fn64 = lambda: kernels.decode_attention(q64.handle, kc64, vc64, sl64.handle, o64,  # noqa: E731
                                                1.0 / np.sqrt(D64))
        wall64, dev64 = time_calls(fn64, steps, warmup)
        for t in (q, kc, vc, sl, q64, sl64):
            t.dispose()
        for h in (o, o64, kc64, vc64):
            h.dispose()
        return {"B": B, "sum_len": int(lens.sum()), "bytes": kv_bytes, "wall_ms": wall_ms, "dev_ms": dev_ms,
                "d64": {"sum_len": int(2 * lens.sum()), "wall_ms": wall64, "dev_ms": dev64}}
    return run


def prep_norm_rope():
    from kandle_amd import HipTensorHandle, Tensor, kernels
    from kandle_amd import synthetic as syn

    T, Hq, Hkv, D, H = 8192, 16, 8, 128, 1024
    x = bf16_tensor(501, (T, H))
    q = bf16_tensor(502, (1, T, Hq, D))
    k = bf16_tensor(503, (1, T, Hkv, D))
    w = Tensor(syn.bf16(syn.uniform(504, (H,), 0.5, 1.5))[0], dtype="bfloat16")
    wq = Tensor(syn.bf16(syn.uniform(505, (D,), 0.5, 1.5))[0], dtype="bfloat16")
    wk = Tensor(syn.bf16(syn.uniform(506, (D,), 0.5, 1.5))[0], dtype="bfloat16")
    half = D // 2
    inv = np.array([1.0 / (1e6 ** (i / half)) for i in range(half)], np.float64).astype(np.float32)
    invt = Tensor(inv)
    pos = Tensor(np.arange(T, dtype=np.int32), dtype="int32")
    y = HipTensorHandle.create_new((T, H), "bfloat16")
    qo = HipTensorHandle.create_new((1, Hq, T, D), "bfloat16")
    ko = HipTensorHandle.create_new((1, Hkv, T, D), "bfloat16")
    params = {"q_weight": wq.handle, "k_weight": wk.handle, "inv_freq": invt.handle, "positions": pos.handle,
              "eps": 1e-6, "q_out": qo, "k_out": ko}
    norm_params = {"normalized_shape": [H], "eps": 1e-6, "weight": w.handle, "out": y}

    def fn():
        kernels.rms_norm([x.handle], norm_params)
        kernels.rms_norm_rope(q.handle, k.handle, params)

    def run(steps, warmup):
        wall_ms, dev_ms = time_calls(fn, steps, warmup)
        bytes_ = 2 * T * H * 2 + H * 2 + 2 * (T * Hq * D + T * Hkv * D) * 2 + 2 * D * 2
        for t in (x, q, k, w, wq, wk, invt, pos):
            t.dispose()
        for h in (y, qo, ko):
            h.dispose()
        return {"T": T, "bytes": float(bytes_), "wall_ms": wall_ms, "dev_ms": dev_ms}
    return run


TS_EXAMPLE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "packages", "backend-hip", "examples",
                          "generate.js")


def _ts_host_ready():
    """Node, the built N-API addon and the stripped TypeScript model are all present."""
    import shutil

    pkg = os.path.dirname(os.path.dirname(TS_EXAMPLE))
    return (shutil.which("node") is not None and os.path.exists(os.path.join(pkg, "native", "kandle_hip.node"))
            and all(os.path.exists(os.path.join(pkg, "dist", m + ".js")) for m in ("index", "qwen3")))


def _write_ts_inputs(cfg, weights, prompt):
    """The C5 weights, a Hugging Face style config and the prompt ids in a temporary directory, the
    input of packages/backend-hip/examples/generate.js."""
    import tempfile

    from kandle_amd.io import save_safetensors

    d = tempfile.mkdtemp(prefix="kandle_c5_")
    save_safetensors(os.path.join(d, "model.safetensors"), weights)
    hf = {"vocab_size": cfg.vocab_size, "hidden_size": cfg.hidden_size, "intermediate_size": cfg.intermediate_size,
          "num_hidden_layers": cfg.num_hidden_layers, "num_attention_heads": cfg.num_attention_heads,
          "num_key_value_heads": cfg.num_key_value_heads, "head_dim": cfg.head_dim, "rms_norm_eps": cfg.rms_norm_eps,
          "rope_theta": cfg.rope_theta, "tie_word_embeddings": True}
    with open(os.path.join(d, "config.json"), "w") as f:
        json.dump(hf, f)
    with open(os.path.join(d, "prompt.json"), "w") as f:
        json.dump([int(t) for t in prompt], f)
    return d


def _run_ts_host(d, new_tokens, py_tokens, activations="float32"):
    """C5 generation driven from Node through the TypeScript model and the N-API addon: one warm-up
    generation of 8 tokens (captures the prefill and decode graphs), then the timed one.  Its tokens
    must equal the Python host's."""
    import shutil
    import subprocess

    try:
        out = subprocess.run(["node", TS_EXAMPLE, os.path.join(d, "config.json"), os.path.join(d, "model.safetensors"),
                              os.path.join(d, "prompt.json"), str(new_tokens), "--activations", activations],
                             capture_output=True, text=True, timeout=300)
    finally:
        shutil.rmtree(d, ignore_errors=True)
    if out.returncode != 0:
        raise RuntimeError(f"TypeScript host generation failed: {out.stderr[-2000:]}")
    r = json.loads(out.stdout.strip().splitlines()[-1])
    toks = r.pop("tokens")
    r["tokens_match_python_host"] = toks == [int(t) for t in py_tokens]
    r["first_tokens"] = toks[:8]
    return r


def c5_weights():
    """(config, weights) of C5: Qwen3-0.6B architecture, random N(0, 0.02) bf16 weights (seed 7)."""
    from kandle_amd.model_utils import Qwen3Config, init_qwen3_weights

    cfg = Qwen3Config()
    t0 = time.perf_counter()
    w = init_qwen3_weights(cfg, seed=7)
    log(f"model weights generated in {time.perf_counter() - t0:.1f} s")
    return cfg, w


def prep_model(cfg, w, new_tokens=128, prompt_len=512, use_graph=True, ts_host=False, activations="float32"):
    """Config C5: Qwen3-0.6B architecture, random N(0, 0.02) bf16 weights, a 512-token prefill of
    uniform-random ids, then 128 greedy decode steps (the decode step captured once as a HIP graph
    and replayed), with the given activation dtype (float32: the reference's arithmetic;
    bfloat16: activations rounded to bf16 between kernels).  One warm-up generation of 8 tokens
    precedes the timed one; it runs the prefill eagerly (reported as prefill_eager_ms) and
    captures it, so the timed prefill is a graph replay, as in a server that captures one prefill
    graph per prompt-length bucket."""
    from kandle_amd.model_utils import Qwen3ForCausalLM
    from kandle_amd import synthetic as syn

    prompt = syn.randint(8, (prompt_len,), 0, cfg.vocab_size)
    model = Qwen3ForCausalLM(cfg, w, max_seq_len=prompt_len + new_tokens, activations=activations)
    ts_dir = _write_ts_inputs(cfg, w, prompt) if ts_host else None

    def run(steps, warmup):
        try:
            warm = {}
            model.generate(prompt, 8, use_graph=use_graph, timing=warm)   # eager prefill (then captured)
            timing = {}
            toks = model.generate(prompt, new_tokens, timing=timing, use_graph=use_graph)
        except BaseException:
            if ts_dir is not None:   # the checkpoint written for the TypeScript host (1.2 GB)
                import shutil
                shutil.rmtree(ts_dir, ignore_errors=True)
            raise
        if not use_graph:  # every step eager: time all of them
            timing["replay_ms"], timing["replay_steps"] = timing["decode_ms"], new_tokens
        model.dispose()
        ts = _run_ts_host(ts_dir, new_tokens, toks, activations) if ts_dir is not None else None   # removes ts_dir
        H, I, D = cfg.hidden_size, cfg.intermediate_size, cfg.head_dim
        Hq, Hkv, Lyr = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.num_hidden_layers
        layer_w = H * (Hq + 2 * Hkv) * D + Hq * D * H + 3 * H * I            # projection weights per layer
        prefill_flops = (2.0 * prompt_len * layer_w * Lyr                      # projections, all rows
                         + 2.0 * cfg.vocab_size * H                            # lm_head, last row
                         + Lyr * 4.0 * Hq * prompt_len * prompt_len * D / 2)   # causal attention
        # bytes a decode step must read: every weight once (tied embedding as lm_head), plus the KV
        # cache rows attended; the mean attended length over the timed replays
        weight_bytes = 2.0 * (Lyr * (layer_w + 2 * H + 2 * D) + cfg.vocab_size * H + H)
        steps_r = timing.get("replay_steps", 0)
        mean_len = prompt_len + 1 + (new_tokens + 1) / 2.0
        kv_bytes = Lyr * 2 * Hkv * D * (4 if activations == "float32" else 2) * mean_len
        return {"activations": activations, "prefill_ms": timing["prefill_ms"], "prefill_issue": timing["prefill_issue"],
                "prefill_eager_ms": warm["prefill_ms"], "prefill_flops": prefill_flops, "prompt_len": prompt_len,
                "new_tokens": new_tokens, "replay_ms": timing.get("replay_ms"), "replay_steps": steps_r,
                "decode_ms": timing["decode_ms"], "step_bytes": weight_bytes + kv_bytes, "tokens": toks[:8],
                "ts_host": ts}
    return run


def bench_prefill_one_sequence(steps, warmup):
    """Causal bf16 flash prefill of ONE sequence (B = 1, Hq = 16, Hkv = 8, D = 128) at several prompt
    lengths: the shapes whose query blocks are too few to fill the CUs as C3's four sequences do
    (the key-split persistent form runs S >= 1024), and at S = 4096 two head dims the kernel has no
    tiles for (96, 80: staged as zero-padded 128-column rows; FLOPs counted at the true D)."""
    from kandle_amd import HipTensorHandle, kernels

    out = {}
    Hq, Hkv = 16, 8
    # D = 96 and 80: head dims without tiles of their own, run on rows staged with zero padding to 128.
    for S, D in ((512, 128), (1024, 128), (2048, 128), (4096, 128), (4096, 96), (4096, 80)):
        q = bf16_tensor(311, (1, Hq, S, D))
        k = bf16_tensor(312, (1, Hkv, S, D))
        v = bf16_tensor(313, (1, Hkv, S, D))
        o = HipTensorHandle.create_new((1, Hq, S, D), "bfloat16")
        fn = lambda: kernels.flash_attention(q.handle, k.handle, v.handle, o, 1.0 / np.sqrt(D), True)  # noqa: E731
        wall_ms, dev_ms = time_calls(fn, steps, warmup)
        flops = 4.0 * Hq * S * S * D / 2.0
        tf = flops / (dev_ms * 1e-3) / 1e12
        key = f"S{S}" if D == 128 else f"S{S}_D{D}_staged"
        out[key] = {"ms": round(dev_ms, 4), "TFLOP/s": round(tf, 1), "frac": round(tf / PEAK_BF16_TFLOPS, 4)}
        for t in (q, k, v):
            t.dispose()
        o.dispose()
    return out


def bench_copy(steps, warmup):
    """Calibration workload for the HBM-traffic counters: a contiguous 1 GiB device-to-device copy
    through the library's strided-copy kernel (1 GiB read + 1 GiB written per call)."""
    from kandle_amd import HipTensorHandle, kernels

    n = 1 << 29  # bf16 elements = 1 GiB
    src = HipTensorHandle.create_new((n,), "bfloat16")
    kernels.zeros(src)
    dst = HipTensorHandle.create_new((n,), "bfloat16")
    from kandle_amd.tensor import copy_into

    wall_ms, dev_ms = time_calls(lambda: copy_into(src, dst), steps, warmup)
    src.dispose()
    dst.dispose()
    return {"bytes": float(2 * n * 2), "wall_ms": wall_ms, "dev_ms": dev_ms}


def bench_load():
    """Native-bf16 checkpoint load: the C5 Qwen3-0.6B weights (random N(0, 0.02) bf16) written as a
    two-shard safetensors checkpoint with config.json into a temporary directory, then
    Qwen3ForCausalLM.from_pretrained timed from the call to the last weight resident in HBM (the
    files were just written, so they are read from the page cache).  A short greedy generation
    checks the loaded model against one built from the same in-memory weights."""
    import dataclasses
    import tempfile

    import torch
    from safetensors.torch import save_file

    from kandle_amd import _lib
    from kandle_amd.model_utils import Qwen3Config, Qwen3ForCausalLM, init_qwen3_weights
    from kandle_amd import synthetic as syn

    cfg = Qwen3Config()
    w = init_qwen3_weights(cfg, seed=7)
    names = list(w)
    nbytes = sum(v.nbytes for v in w.values())
    with tempfile.TemporaryDirectory() as d:
        half = len(names) // 2
        wm = {}
        for i, keys in enumerate((names[:half], names[half:])):
            shard = f"model-0000{i + 1}-of-00002.safetensors"
            save_file({k: torch.from_numpy(w[k].astype(np.int16)).view(torch.bfloat16) for k in keys},
                      os.path.join(d, shard))
            wm.update({k: shard for k in keys})
        with open(os.path.join(d, "model.safetensors.index.json"), "w") as fh:
            json.dump({"metadata": {"total_size": nbytes}, "weight_map": wm}, fh)
        with open(os.path.join(d, "config.json"), "w") as fh:
            json.dump(dataclasses.asdict(cfg), fh)
        log(f"checkpoint written ({nbytes / 1e9:.2f} GB)")
        _lib.synchronize()
        t0 = time.perf_counter()
        model = Qwen3ForCausalLM.from_pretrained(d, max_seq_len=64)
        _lib.synchronize()
        load_s = time.perf_counter() - t0
    prompt = syn.randint(8, (16,), 0, cfg.vocab_size)
    toks = model.generate(prompt, 4)
    model.dispose()
    ref = Qwen3ForCausalLM(cfg, w, max_seq_len=64)
    rtoks = ref.generate(prompt, 4)
    ref.dispose()
    return {"bytes": nbytes, "load_s": load_s, "tokens_match": toks == rtoks}


# (name, N, K, output): "swiglu" is the gate/up projection with silu * mul in the epilogue (N = 2 I
# interleaved weight rows, output [M, I] bf16), as the model's prefill runs it.
GEMM_SHAPES = (("qkv", 4096, 1024, "bf16"), ("o_proj", 1024, 2048, "f32"), ("gate_up_swiglu", 6144, 1024, "swiglu"),
               ("down", 1024, 3072, "f32"))


def bench_gemm(steps, warmup, M=512, eager=False, act="bfloat16"):
    """The four projection GEMMs of a C5 prefill layer (M = 512 tokens, bf16 weights [N, K], fp32
    accumulate): y = x W^T, the activation dtype out for qkv and gate/up, fp32 out plus the fp32
    residual (beta = 1) for o_proj and down, as in the model.  act: the activations' dtype
    (bfloat16, or float32: x fp32, split into bf16 hi + lo on the MFMA tiles).  Per shape: device
    time (calls replayed from a graph, as the model's prefill runs them; with eager, launched one by
    one from the host, the form a kernel tracer or counter run takes) and TFLOP/s of the algorithmic
    2 M N K."""
    import ctypes as C

    from kandle_amd import Tensor, _lib

    f32 = act == "float32"
    a_code = 0 if f32 else 1
    out = {}
    for name, N, K, odt in GEMM_SHAPES:
        x = Tensor(np.random.default_rng(701).normal(size=(M, K)).astype(np.float32)) if f32 else \
            bf16_tensor(701, (M, K))
        w = bf16_tensor(702, (N, K))
        ny = N // 2 if odt == "swiglu" else N
        y = Tensor(np.zeros((M, ny), np.float32), dtype="float32" if (odt == "f32" or f32) else "bfloat16")
        res = Tensor(np.zeros((M, N), np.float32), dtype="float32") if odt == "f32" else None
        vp = lambda t: C.c_void_p(t.handle.data_ptr() if t is not None else 0)  # noqa: E731
        if odt == "swiglu":
            call = lambda: _lib.call("kh_gemm_swiglu", vp(x), K, vp(w), K, vp(y), ny, M, ny, K, a_code)  # noqa: E731
        else:
            call = lambda: _lib.call("kh_gemm_ex", vp(x), K, a_code, vp(w), K, 1, vp(y), N, vp(res), N,  # noqa: E731
                                     vp(None), M, N, K, C.c_float(1.0), C.c_float(1.0 if res is not None else 0.0), 1,
                                     0 if (odt == "f32" or f32) else 1)
        # Device time: 20 calls captured as one graph and replayed (no host launch cost per call).
        from kandle_amd.graphs import HipGraph

        call()
        if eager:
            wall, dev = time_calls(call, steps, warmup)
        else:
            g = HipGraph()
            with g.capture():
                for _ in range(20):
                    call()
            wall, dev = time_calls(g.replay, max(1, steps // 4), warmup)
            g.dispose()
            dev /= 20.0
        flops = 2.0 * M * N * K
        out[name] = {"M": M, "N": N, "K": K, "us": round(dev * 1e3, 2),
                     "TFLOP/s": round(flops / (dev * 1e-3) / 1e12, 1)}
        for t in (x, w, y, res):
            if t is not None:
                t.dispose()
    tot = sum(v["us"] for v in out.values())
    out["activations"] = act
    out["layer_us"] = round(tot, 2)
    out["layer_TFLOP/s"] = round(sum(2.0 * M * n * k for _, n, k, _ in GEMM_SHAPES) / (tot * 1e-6) / 1e12, 1)
    return out


GEMV_SHAPES = (  # (name, N, K, prologue 0 none / 1 RMSNorm / 3 silu*mul of interleaved gate/up, fp32 out + residual)
    ("qkv", 4096, 1024, 1, False), ("o_proj", 1024, 2048, 0, True), ("gate_up", 6144, 1024, 1, False),
    ("down", 1024, 3072, 3, True), ("lm_head", 151936, 1024, 1, True), ("launch_floor", 64, 64, 0, False))


def bench_gemv(steps, warmup):
    """The one-row GEMVs of a C5 decode step (bf16 weights [N, K], fp32 accumulate) through
    kh_gemv_fused with the prologue the model uses, 20 calls captured in a graph and replayed: device
    time per call and weight GB/s against the HBM roofline.  launch_floor is a 64 x 64 GEMV: the
    per-kernel cost of a launch inside a graph."""
    import ctypes as C

    from kandle_amd import Tensor, _lib
    from kandle_amd.graphs import HipGraph

    out = {}
    for name, N, K, pro, res in GEMV_SHAPES:
        w = bf16_tensor(711, (N, K))
        kx = 2 * K if pro == 3 else K
        x = (Tensor(np.random.default_rng(5).normal(size=kx).astype(np.float32), dtype="float32") if pro == 1
             else bf16_tensor(712, (kx,)))
        x2 = bf16_tensor(713, (K,)) if pro == 2 else None
        nw = bf16_tensor(714, (K,)) if pro == 1 else None
        y = Tensor(np.zeros(N, np.float32), dtype="float32" if res else "bfloat16")
        cin = Tensor(np.zeros(N, np.float32), dtype="float32") if res else None
        vp = lambda t: C.c_void_p(t.handle.data_ptr() if t is not None else 0)  # noqa: E731
        call = lambda: _lib.call("kh_gemv_fused", pro, vp(x), vp(x2), vp(nw), C.c_float(1e-6), vp(w), K, vp(y),  # noqa
                                 vp(cin), vp(None), N, K, C.c_float(1.0), C.c_float(1.0 if res else 0.0),
                                 0 if res else 1, 1)
        call()
        g = HipGraph()
        with g.capture():
            for _ in range(20):
                call()
        _, dev = time_calls(g.replay, max(1, steps // 4), warmup)
        g.dispose()
        us = dev * 1e3 / 20.0
        out[name] = {"N": N, "K": K, "us": round(us, 2), "GB/s": round(2.0 * N * K / (us * 1e-6) / 1e9, 1)}
        for t in (w, x, x2, nw, y, cin):
            if t is not None:
                t.dispose()
    layer = sum(out[n]["us"] for n in ("qkv", "o_proj", "gate_up", "down"))
    out["layer_gemv_us"] = round(layer, 2)
    return out


def bench_vendor(steps):
    """Reference points from the vendor stack in this image, on the same shapes (not part of this
    backend): torch's scaled_dot_product_attention on C3 (each backend torch offers here, with the
    KV heads expanded to Hq since GQA is not taken natively), and torch.matmul (hipBLASLt) on the
    C5 prefill projection GEMMs, 20 calls captured in a CUDA graph and replayed."""
    import torch
    import torch.nn.functional as TF

    dev = "cuda"
    out = {}
    B, Hq, Hkv, S, D = 4, 16, 8, 4096, 128
    g = torch.Generator(device=dev).manual_seed(0)
    q = torch.randn(B, Hq, S, D, device=dev, dtype=torch.bfloat16, generator=g)
    k = torch.randn(B, Hkv, S, D, device=dev, dtype=torch.bfloat16, generator=g)
    v = torch.randn(B, Hkv, S, D, device=dev, dtype=torch.bfloat16, generator=g)
    kk = k.repeat_interleave(Hq // Hkv, dim=1).contiguous()
    vv = v.repeat_interleave(Hq // Hkv, dim=1).contiguous()
    flops = 4.0 * B * Hq * S * S * D / 2
    from torch.nn.attention import SDPBackend, sdpa_kernel

    for name, be in (("flash", SDPBackend.FLASH_ATTENTION), ("efficient", SDPBackend.EFFICIENT_ATTENTION)):
        try:
            with sdpa_kernel(be):
                for _ in range(3):
                    TF.scaled_dot_product_attention(q, kk, vv, is_causal=True)
                torch.cuda.synchronize()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(steps):
                    TF.scaled_dot_product_attention(q, kk, vv, is_causal=True)
                e1.record()
                torch.cuda.synchronize()
            ms = e0.elapsed_time(e1) / steps
            out[f"sdpa_{name}"] = {"ms": round(ms, 4), "TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 1)}
        except Exception as ex:  # a backend torch does not offer for these inputs
            out[f"sdpa_{name}"] = {"unavailable": str(ex)[:160]}
    out["gemm_hipblaslt"] = _vendor_gemms(torch, dev, g, torch.bfloat16)
    # the reference's own arithmetic: float32 activations times float32 weights (the bf16 weights
    # widened on load), as torch.matmul runs it in float32
    out["gemm_hipblaslt_f32"] = _vendor_gemms(torch, dev, g, torch.float32)
    return out


def _vendor_gemms(torch, dev, g, dtype):
    """torch.matmul (hipBLASLt / rocBLAS) on the C5 prefill projection shapes in `dtype`: x [512, K]
    times w [N, K] transposed, 20 calls captured in a graph and replayed 5 times."""
    gem = {}
    for name, N, K, _ in GEMM_SHAPES:
        x = torch.randn(512, K, device=dev, dtype=dtype, generator=g)
        w = torch.randn(N, K, device=dev, dtype=dtype, generator=g)
        s2 = torch.cuda.Stream()
        s2.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s2):
            for _ in range(3):
                x @ w.t()
        torch.cuda.current_stream().wait_stream(s2)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(20):
                x @ w.t()
        graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(5):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) / 100 * 1e3
        gem[name] = {"us": round(us, 2), "TFLOP/s": round(2.0 * 512 * N * K / (us * 1e-6) / 1e12, 1)}
    gem["layer_us"] = round(sum(v["us"] for v in gem.values()), 2)
    gem["dtype"] = str(dtype).replace("torch.", "")
    return gem


def bench_sample(steps, warmup):
    """On-device sampling of one token from a Qwen3 logits row (vocab 151936, float32): kh_sample
    per call for greedy, an unfiltered draw, and temperature 0.7 with top-k 50 and top-p 0.9 (the
    counter stays in device memory; its value changes r, not the work)."""
    from kandle_amd import Tensor
    from kandle_amd.model_utils.sampling import SamplerConfig, sample_device

    V = 151936
    x = (np.random.default_rng(21).normal(size=V) * 3).astype(np.float32)
    lg = Tensor(x, dtype="float32")
    ctr = Tensor(np.zeros(1, np.int32), dtype="int32")
    tok = Tensor(np.zeros(1, np.int32), dtype="int32")
    out = {"vocab": V}
    from kandle_amd.graphs import HipGraph

    for name, cfg in (("greedy", SamplerConfig(do_sample=False)), ("plain", SamplerConfig()),
                      ("t0.7_k50_p0.9", SamplerConfig(temperature=0.7, top_k=50, top_p=0.9)),
                      ("t0.7_p0.9_fullsort", SamplerConfig(temperature=0.7, top_p=0.9))):
        wall, dev = time_calls(lambda cfg=cfg: sample_device(lg, cfg, 1234, ctr, tok), steps, warmup)
        out[name] = {"wall_us": round(wall * 1e3, 2), "dev_us": round(dev * 1e3, 2)}
        if "fullsort" in name:
            continue
        # device time without the host: one draw captured in a graph, replayed
        g = HipGraph()
        with g.capture():
            sample_device(lg, cfg, 1234, ctr, tok)
        _, gdev = time_calls(g.replay, steps, warmup)
        g.dispose()
        out[name]["graph_replay_us"] = round(gdev * 1e3, 2)
    for t in (lg, ctr, tok):
        t.dispose()
    return out


def bench_stream(new_tokens=64, prompt_len=512):
    """Config C5 model driven through generate_stream with Qwen3's sampling settings (temperature
    0.6, top-k 20, top-p 0.95, 10 display candidates): per-token wall time of the whole interactive
    step -- device sampling, the host reading the step back, and the captured one-token forward --
    beside greedy generate()'s replayed step."""
    from kandle_amd.model_utils import GeneratorConfig, Qwen3Config, Qwen3ForCausalLM, init_qwen3_weights
    from kandle_amd import synthetic as syn

    cfg = Qwen3Config()
    w = init_qwen3_weights(cfg, seed=7)
    prompt = syn.randint(8, (prompt_len,), 0, cfg.vocab_size)
    model = Qwen3ForCausalLM(cfg, w, max_seq_len=prompt_len + new_tokens + 8)
    del w
    gc = GeneratorConfig(max_new_tokens=new_tokens, temperature=0.6, top_k=20, top_p=0.95, display_top_k=10)
    for _ in model.generate_stream(prompt, GeneratorConfig(max_new_tokens=4)):   # capture the prefill
        pass
    times = []
    t = time.perf_counter()
    for _ in model.generate_stream(prompt, gc, seed=1):
        now = time.perf_counter()
        times.append(now - t)
        t = now
    timing = {}
    model.generate(prompt, new_tokens, timing=timing)
    model.dispose()
    steady = times[2:]   # after the prefill step and the step that captures the forward
    return {"new_tokens": new_tokens, "first_step_ms": round(times[0] * 1e3, 3),
            "stream_ms_per_token": round(float(np.mean(steady)) * 1e3, 4),
            "greedy_replay_ms_per_token": round(timing["replay_ms"] / timing["replay_steps"], 4)}


def cpu_baseline_sample(reps=20):
    """The oracle's numpy restatement of sample() (temperature 0.7, top-k 50, top-p 0.9) on the same
    row, single thread: the reference's per-token host work (sort, softmax, filters, draw)."""
    from oracle.sampling import sample_reference

    x = (np.random.default_rng(21).normal(size=151936) * 3).astype(np.float32)
    t0 = time.perf_counter()
    for i in range(reps):
        sample_reference(x, 0.7, 50, 0.9, (i + 0.5) / reps, 10)
    return (time.perf_counter() - t0) * 1e6 / reps


def measured_traffic(workload):
    """HBM bytes per launch from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE measurements
    (profiles/traffic.json), scaled by the copy-kernel calibration factors; None if absent."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)
        k = t["kernels"][workload]
        cal = t["calibration"]
        return float(k["fetch_kib"] * 1024 * cal["fetch_factor"] + k["write_kib"] * 1024 * cal["write_factor"])
    except (OSError, KeyError, ValueError):
        return None


def _node_version():
    import subprocess
    try:
        return subprocess.run(["node", "--version"], capture_output=True, text=True, timeout=30).stdout.strip()
    except (OSError, subprocess.SubprocessError):
        return "?"


def _one_thread():
    """Context that limits numpy's BLAS to one thread (the CPU baselines state cores = 1)."""
    try:
        from threadpoolctl import threadpool_limits
        return threadpool_limits(1)
    except ImportError:  # pragma: no cover
        import contextlib
        return contextlib.nullcontext()


MASK_LEAD_WARMUP = 40  # warm-up calls of the explicit-mask leg that leads the headline
JS_REPEAT = 5   # timed runs of each JavaScript baseline after one untimed run; the median is reported


def _js_leg(op, inputs, args, work, unit, sample, scale_to_full=1.0):
    """One JavaScript CPU baseline: oracle/js/bench_cpu.js OP run by Node on one thread, one untimed
    run then JS_REPEAT timed runs; value = work / median time (x scale_to_full for a sample)."""
    import oracle

    _, runs = oracle.js_bench(op, inputs, args, JS_REPEAT)
    med = float(np.median(runs))
    return {"value": round(work * scale_to_full / (med * 1e-3), 6), "unit": unit, "cores": 1, "kind": "port",
            "runtime": f"JavaScript, Node {_node_version()}, one thread (host has {os.cpu_count()} cores)",
            "sample": sample + f"; median of {JS_REPEAT} timed runs after 1 warm-up "
                               f"({', '.join(f'{r / 1e3:.2f}' for r in runs)} s)",
            "median_s": round(med / 1e3, 4)}


def cpu_baseline_prefill():
    """The reference flash algorithm on CPU for C3, restated in JavaScript and run by Node (the
    stand-in for Kandle's pure-JS CPU backend, which the reference does not ship): one (batch,
    q-head) slice at full S = 4096, causal, extrapolated x64 to the whole batch.  The oracle's
    float32 C port on the same slice rides along."""
    import oracle
    from kandle_amd import synthetic as syn

    S, D = 4096, 128
    q = syn.normal(601, (1, 1, S, D))
    k = syn.normal(602, (1, 1, S, D))
    v = syn.normal(603, (1, 1, S, D))
    slice_flops = 4.0 * S * S * D / 2.0
    t0 = time.perf_counter()
    oracle.flash_f32(q, k, v, causal=True)
    dt = time.perf_counter() - t0
    c_port = {"value": slice_flops / dt / 1e12, "unit": "TFLOP/s", "cores": 1, "kind": "port",
              "sample": f"C port (oracle/oracle.c), 1 of 64 (batch, q-head) slices of C3 at full S=4096, causal, "
                        f"fp32, single thread ({dt:.2f} s)"}
    if not oracle.node_available():
        c_port["sample"] += f"; host has {os.cpu_count()} cores (Node not installed: no JavaScript baseline)"
        return c_port
    js = _js_leg("flash", {"q": q, "k": k, "v": v}, [1, 1, 1, S, S, D, 1.0 / np.sqrt(D), 1, 0],
                 slice_flops / 1e12, "TFLOP/s",
                 "JavaScript restatement of the reference flash algorithm (oracle/js/flash_sdpa.js: Br=8 Bc=4 tiles, "
                 "Float32Array storage) on 1 of the 64 (batch, q-head) slices of C3 at full S=4096, causal; "
                 "extrapolated x64 (throughput of the slice = throughput of the batch)")
    js["extrapolated"] = "x64"
    js["c_port"] = c_port
    return js


def cpu_baseline_c1():
    """Config C1 at full size in JavaScript: SDPA fp32, B=1, Hq=16, Hkv=8, S=256, D=128, causal."""
    import oracle
    from kandle_amd import synthetic as syn

    if not oracle.node_available():
        return None
    B, Hq, Hkv, S, D = 1, 16, 8, 256, 128
    q = syn.normal(11, (B, Hq, S, D))
    k = syn.normal(12, (B, Hkv, S, D))
    v = syn.normal(13, (B, Hkv, S, D))
    return _js_leg("flash", {"q": q, "k": k, "v": v}, [B, Hq, Hkv, S, S, D, 1.0 / np.sqrt(D), 1, 0],
                   4.0 * B * Hq * S * S * D / 2.0 / 1e9, "GFLOP/s",
                   "full C1 (B=1, Hq=16, Hkv=8, S=256, D=128, causal, fp32), oracle/js/flash_sdpa.js")


def cpu_baseline_decode():
    """C4 at full size in JavaScript: one L = 1 SDPA per sequence over its whole cache (the caller's
    decode step, gqa.ts:333-336), float32 caches; GB/s of the bf16 K/V bytes the GPU kernel reads.
    Without Node, the oracle's C SDPA (double accumulation) times the same work."""
    import oracle
    from kandle_amd import synthetic as syn

    B, Hq, Hkv, D = (C4_SHAPE[x] for x in ("B", "Hq", "Hkv", "D"))
    lens = c4_lengths()
    nbytes = float(lens.sum()) * Hkv * D * 2 * 2
    q = syn.normal(3000, (B, Hq, D))
    ks = [syn.normal(4000 + b, (Hkv, int(L), D)) for b, L in enumerate(lens)]
    vs = [syn.normal(5000 + b, (Hkv, int(L), D)) for b, L in enumerate(lens)]
    if oracle.node_available():
        inputs = {"q": q}
        for b in range(B):
            inputs[f"k_{b}"], inputs[f"v_{b}"] = ks[b], vs[b]
        return _js_leg("decode", inputs, [Hq, Hkv, D, 1.0 / np.sqrt(D)] + [int(L) for L in lens], nbytes / 1e9, "GB/s",
                       f"full C4 (sum L = {int(lens.sum())}), oracle/js/flash_sdpa.js with one query per sequence")
    dt = 0.0
    for b in range(B):
        t0 = time.perf_counter()
        oracle.sdpa(q[b][None, :, None, :], ks[b][None], vs[b][None])
        dt += time.perf_counter() - t0
    return {"value": round(nbytes / dt / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"full C4 (sum L = {int(lens.sum())}), oracle SDPA in C, one thread, {dt:.2f} s "
                      "(Node not installed: no JavaScript baseline)"}


def cpu_baseline_norm():
    """C2 at full size in JavaScript: RMSNorm over [8192, 1024], qk-norm + RoPE over q [8192, 16, 128]
    and k [8192, 8, 128] (the composite's cos/sin tables included); GB/s of the bf16 bytes the GPU
    kernels move.  Without Node, the oracle's C functions time the same work."""
    import oracle
    from kandle_amd import synthetic as syn

    T, H, Hq, Hkv, D = 8192, 1024, 16, 8, 128
    x = syn.normal(501, (T, H))
    q = syn.normal(502, (T, Hq, D))
    k = syn.normal(503, (T, Hkv, D))
    w = syn.uniform(504, (H,), 0.5, 1.5)
    wq = syn.uniform(505, (D,), 0.5, 1.5)
    wk = syn.uniform(506, (D,), 0.5, 1.5)
    nbytes = 134220288.0
    if oracle.node_available():
        return _js_leg("normrope", {"x": x, "q": q, "k": k, "w": w, "wq": wq, "wk": wk},
                       [T, H, Hq, Hkv, D, 1e-6, 1e6], nbytes / 1e9, "GB/s",
                       "full C2 (8192 tokens), oracle/js/cpu_ops.js")
    inv = oracle.rope_inv_freq(D, 1e6)
    pos = np.arange(T, dtype=np.int32)
    t0 = time.perf_counter()
    oracle.rms_norm(x, w, 1e-6)
    oracle.qk_norm_rope(q, wq, pos, inv, 1e-6)
    oracle.qk_norm_rope(k, wk, pos, inv, 1e-6)
    dt = time.perf_counter() - t0
    return {"value": round(nbytes / dt / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"full C2 (8192 tokens), oracle in C, one thread, {dt:.2f} s (Node not installed)"}


def cpu_baseline_model(prompt_len=512, decode_steps=4):
    """C5 on the CPU, extrapolated from ONE decoder layer of the 0.6B architecture over the 512-token
    prompt and `decode_steps` one-token steps after it: times 28 layers, plus the lm_head row, as
    tokens/s for prefill and decode.  The leg reported is the JavaScript restatement run by Node on
    one thread (oracle/js/qwen3_cpu.js, checked against the numpy oracle in tests/test_oracle_js.py);
    the numpy oracle (one BLAS thread) rides along as "numpy_oracle"."""
    import oracle

    js = None
    if oracle.node_available():
        from kandle_amd.model_utils import Qwen3Config

        t = oracle.js_qwen3_timing(Qwen3Config(), prompt_len, decode_steps)
        L = Qwen3Config().num_hidden_layers
        pre_s = ((t["prefill_ms"] - t["head_ms"]) * L + t["head_ms"]) * 1e-3
        dec_s = ((t["decode_ms"] - t["head_ms"]) * L + t["head_ms"]) * 1e-3
        js = {"prefill_tokens_per_s": round(prompt_len / pre_s, 3), "decode_tokens_per_s": round(1.0 / dec_s, 4),
              "cores": 1, "kind": "port",
              "runtime": f"JavaScript, Node {_node_version()}, one thread (host has {os.cpu_count()} cores)",
              "sample": f"extrapolated x28 layers: 1 layer measured once (prefill of {prompt_len} tokens "
                        f"{t['prefill_ms'] / 1e3:.2f} s, decode {t['decode_ms']:.0f} ms/step over {decode_steps} "
                        f"steps, both incl. the lm_head row {t['head_ms']:.0f} ms, counted once)"}
    npy = _cpu_baseline_model_numpy(prompt_len, decode_steps)
    if js is None:
        return npy
    js["numpy_oracle"] = npy
    return js


def _cpu_baseline_model_numpy(prompt_len=512, decode_steps=4):
    """The numpy oracle (one BLAS thread) of one decoder layer, extrapolated as cpu_baseline_model."""
    import dataclasses

    from kandle_amd import synthetic as syn
    from kandle_amd.model_utils import Qwen3Config, init_qwen3_weights
    from oracle.qwen3 import Qwen3Oracle

    full = Qwen3Config()
    cfg = dataclasses.replace(full, num_hidden_layers=1)
    w = init_qwen3_weights(cfg, seed=7)
    prompt = syn.randint(8, (prompt_len,), 0, cfg.vocab_size)
    with _one_thread():
        ref = Qwen3Oracle(cfg, w, max_seq_len=prompt_len + decode_steps + 1)
        t0 = time.perf_counter()
        logits = ref.forward(prompt, 0)
        t_pre = time.perf_counter() - t0
        t0 = time.perf_counter()
        pos = prompt_len
        for _ in range(decode_steps):
            logits = ref.forward([int(np.argmax(logits))], pos)
            pos += 1
        t_dec = (time.perf_counter() - t0) / decode_steps
        # lm_head share, measured on its own and not multiplied by the layer count
        e = ref.embed
        hrow = np.zeros((1, cfg.hidden_size), np.float32)
        t0 = time.perf_counter()
        for _ in range(3):
            hrow @ e.T
        t_head = (time.perf_counter() - t0) / 3
    L = full.num_hidden_layers
    pre_s = (t_pre - t_head) * L + t_head
    dec_s = (t_dec - t_head) * L + t_head
    return {"prefill_tokens_per_s": round(prompt_len / pre_s, 2), "decode_tokens_per_s": round(1.0 / dec_s, 3),
            "cores": 1, "kind": "port",
            "sample": f"extrapolated: 1 of 28 layers measured (prefill {t_pre:.2f} s, decode {t_dec * 1e3:.1f} ms/step "
                      f"incl. lm_head {t_head * 1e3:.1f} ms), numpy oracle, one BLAS thread"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # Single-leg runs (--only) start from an idle GPU: these defaults time enough calls for its clock
    # to settle.  The default run times the headline after the other GPU legs.
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--eager-decode", action="store_true",
                    help="C5: issue every decode step's kernels from the host instead of replaying a HIP graph")
    ap.add_argument("--no-ts-host", action="store_true",
                    help="C5: skip the generation driven from Node through the TypeScript model")
    ap.add_argument("--eager-gemm", action="store_true",
                    help="--only gemm: launch each GEMM from the host instead of replaying a HIP graph")
    ap.add_argument("--only", choices=["prefill", "c1", "decode", "norm", "model", "copy", "load", "sample", "stream",
                                       "gemm", "gemv", "vendor", "mask", "prefill_b1"], default=None)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); this build has no multi-GPU path",
              file=sys.stderr)
        sys.exit(2)

    res = {}
    if args.only == "vendor":
        # torch carries its own HIP runtime: it must be the only one to open the device in this process
        log("vendor reference points (torch SDPA, hipBLASLt) ...")
        res["vendor"] = bench_vendor(args.steps)
    else:
        from kandle_amd import HipBackend

        HipBackend.create(0)
    # Inputs of every GPU leg first (host generation and upload), then the legs back to back with
    # the headline (C3 prefill) last, then the CPU baselines.
    legs = []
    if args.only in (None, "model"):
        log("C5 model weights ...")
        ts_host = not args.no_ts_host and _ts_host_ready()
        if not ts_host:
            log("C5 from the TypeScript host: skipped (" + ("--no-ts-host" if args.no_ts_host else
                "node, the N-API addon or the stripped TypeScript is missing: run __graft_entry__.build()") + ")")
        cfg5, w5 = c5_weights()
        # float32 activations (the reference's arithmetic, the C5 parity mode) and, as a separately
        # labelled line, bfloat16 activations
        legs.append(("model", "Qwen3-0.6B C5 (float32 activations)",
                     prep_model(cfg5, w5, use_graph=not args.eager_decode, ts_host=ts_host and not args.eager_decode,
                                activations="float32")))
        legs.append(("model_bf16", "Qwen3-0.6B C5 (bfloat16 activations)",
                     prep_model(cfg5, w5, use_graph=not args.eager_decode, activations="bfloat16")))
        del w5
    if args.only in (None, "decode"):
        legs.append(("decode", "decode C4", prep_decode()))
    if args.only in (None, "norm"):
        legs.append(("norm", "norm+rope C2", prep_norm_rope()))
    if args.only in (None, "c1"):
        legs.append(("c1", "SDPA fp32 C1", prep_c1()))
    if args.only == "mask":
        legs.append(("mask", "explicit-mask SDPA at C3 shapes", prep_mask()))
    lead_mask = prep_mask() if args.only is None else None
    if args.only in (None, "prefill"):
        legs.append(("prefill", "prefill C3", prep_prefill()))
    for key, label, run in legs:
        if key == "prefill" and args.only is None:
            log("sampling ...")
            res["sample"] = bench_sample(args.steps, args.warmup)
            # The explicit-mask leg (the same C3 inputs with a float mask, every pair scored: a
            # measurement of its own) leads the headline: its timed calls and the headline's warm-up
            # calls are enqueued back to back, so the headline starts on a GPU that is already under
            # sustained MFMA load instead of one coming out of the sampling leg's short calls.  The
            # GPU's clock needs tens of ms of such load to settle (per call from idle: 0.315 ms for
            # calls 2-5, 0.36 ms for calls 6-20, then 0.278 ms after about 150 calls; a constant
            # cycle count per call, profiles/flash_prefill_c3.md).  The headline itself is still W
            # warm-up calls, a synchronisation, then K timed calls and a synchronisation.
            # The mask leg takes at least MASK_LEAD_WARMUP warm-up calls (~0.9 ms each), so that with
            # its timed calls some 50 ms of load precede the headline at any --steps / --warmup.
            log("explicit-mask SDPA at C3 shapes, leading the headline ...")
            handle = {}
            lead = lambda: handle.setdefault("h", lead_mask.enqueue(  # noqa: E731
                args.steps, max(args.warmup, MASK_LEAD_WARMUP)))
            log(f"{label} ...")
            res[key] = run(args.steps, args.warmup, lead=lead)
            res["mask"] = lead_mask.result(finish_timed(handle["h"]))
            res["lead_calls"] = max(args.warmup, MASK_LEAD_WARMUP) + args.steps
            continue
        log(f"{label} ...")
        res[key] = run(args.steps, args.warmup)
    if args.only == "sample":
        log("sampling ...")
        res["sample"] = bench_sample(args.steps, args.warmup)
        if not args.no_cpu_baseline:
            res["sample"]["cpu_oracle_us"] = round(cpu_baseline_sample(), 1)
    if args.only == "prefill_b1":
        log("one-sequence causal prefill ...")
        res["prefill_b1"] = bench_prefill_one_sequence(args.steps, args.warmup)
    if args.only == "copy":
        log("copy calibration ...")
        res["copy"] = bench_copy(args.steps, args.warmup)
    if args.only == "load":
        log("checkpoint load ...")
        res["load"] = bench_load()
    if args.only == "stream":
        log("generate_stream ...")
        res["stream"] = bench_stream()
    if args.only == "gemm":
        log("C5 prefill GEMMs ...")
        res["gemm"] = bench_gemm(args.steps, args.warmup, eager=args.eager_gemm)
        res["gemm_f32"] = bench_gemm(args.steps, args.warmup, eager=args.eager_gemm, act="float32")
    if args.only == "gemv":
        log("C5 decode GEMVs ...")
        res["gemv"] = bench_gemv(args.steps, args.warmup)
    cpu = None
    if not args.no_cpu_baseline and args.only in (None, "prefill"):
        log("cpu baseline (C3) ...")
        with _one_thread():
            cpu = cpu_baseline_prefill()
    cpu_more = {}
    if not args.no_cpu_baseline and args.only in (None, "c1"):
        log("cpu baseline (C1) ...")
        cpu_more["c1"] = cpu_baseline_c1()
    if not args.no_cpu_baseline and args.only is None:
        log("cpu baselines of C4, C2, C5 ...")
        with _one_thread():
            cpu_more["decode"] = cpu_baseline_decode()
            cpu_more["norm_rope"] = cpu_baseline_norm()
        cpu_more["model"] = cpu_baseline_model()

    line = {"metric": METRIC, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seeded Philox N(0,1))"}
    if "lead_calls" in res and "mask" in res:
        # the load that precedes the headline's warm-up with no synchronisation in between: the
        # explicit-mask leg's warm-up and timed calls (the settled-clock condition of the headline)
        line["lead"] = {"what": "explicit-mask SDPA at C3 shapes, enqueued right before the headline's warm-up",
                        "calls": res["lead_calls"], "device_ms": round(res["lead_calls"] * res["mask"]["ms"], 2)}
    if "prefill" in res:
        p = res["prefill"]
        tflops = p["flops"] / (p["wall_ms"] * 1e-3) / 1e12
        achieved = p["flops"] / (p["dev_ms"] * 1e-3) / 1e12
        line.update({
            "value": round(tflops, 2), "unit": "TFLOP/s", "ms_per_step": round(p["wall_ms"], 4),
            "config": {"workload": "C3 causal GQA flash-attention prefill", "batch": p["B"], "q_heads": p["Hq"],
                       "kv_heads": p["Hkv"], "seq_len": p["S"], "head_dim": p["D"]},
            "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                         "traffic": measured_traffic("prefill"),
                         "kernel": "flash_fwd_persistent_kernel<true, 128, 1, false>", "kernel_ms": round(p["dev_ms"], 4)},
        })
    if "decode" in res:
        d = res["decode"]
        gbps = d["bytes"] / (d["dev_ms"] * 1e-3) / 1e9
        line["decode"] = {"workload": "C4 decode attention, B=8, Hq=16, Hkv=8, D=128, L~U[8192,32768]",
                          "sum_len": d["sum_len"], "bytes": d["bytes"], "ms": round(d["dev_ms"], 4),
                          "wall_ms": round(d["wall_ms"], 4), "GB/s": round(gbps, 1),
                          "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": PEAK_HBM_GBPS,
                                       "unit": "GB/s", "frac": round(gbps / PEAK_HBM_GBPS, 4),
                                       "traffic": measured_traffic("decode")}}
        d64 = d["d64"]
        line["decode"]["head_dim_64"] = {
            "workload": "B=8, Hq=16, Hkv=8, D=64, L = 2 x the C4 lengths (the same K/V bytes)",
            "sum_len": d64["sum_len"], "ms": round(d64["dev_ms"], 4),
            "GB/s": round(d["bytes"] / (d64["dev_ms"] * 1e-3) / 1e9, 1)}
        if "value" not in line:
            line.update({"value": round(gbps, 1), "unit": "GB/s", "ms_per_step": round(d["wall_ms"], 4),
                         "config": {"workload": "C4 decode attention"}})
    if "norm" in res:
        n = res["norm"]
        gbps = n["bytes"] / (n["dev_ms"] * 1e-3) / 1e9
        line["norm_rope"] = {"workload": "C2 RMSNorm + qk-norm + RoPE, T=8192, bf16", "bytes": n["bytes"],
                             "ms": round(n["dev_ms"], 4), "GB/s": round(gbps, 1),
                             "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": PEAK_HBM_GBPS,
                                          "unit": "GB/s", "frac": round(gbps / PEAK_HBM_GBPS, 4),
                                          "traffic": measured_traffic("norm")}}
        if "value" not in line:
            line.update({"value": round(gbps, 1), "unit": "GB/s", "ms_per_step": round(n["wall_ms"], 4),
                         "config": {"workload": "C2 norm + rope"}})
    if "c1" in res:
        c1 = res["c1"]
        gf = c1["flops"] / (c1["dev_ms"] * 1e-3) / 1e9
        line["c1"] = {"workload": "C1 SDPA fp32, B=1, Hq=16, Hkv=8, S=256, D=128, causal (fp32 MFMA flash kernel)",
                      "flops": c1["flops"], "ms": round(c1["dev_ms"], 4), "wall_ms": round(c1["wall_ms"], 4),
                      "GFLOP/s": round(gf, 1),
                      "roofline": {"bound": "mfma fp32", "achieved": round(gf / 1e3, 3), "peak": 157.3,
                                   "unit": "TFLOP/s", "frac": round(gf / 1e3 / 157.3, 4), "traffic": None}}
        if "split_dev_ms" in c1:
            sg = c1["flops"] / (c1["split_dev_ms"] * 1e-3) / 1e9
            line["c1"]["split_bf16"] = {
                "what": "the same call as kh_flash_attention_split: fp32 operands as bf16 hi + lo, three bf16 MFMAs "
                        "per product (within about 2^-15 of the fp32 products)",
                "ms": round(c1["split_dev_ms"], 4), "wall_ms": round(c1["split_wall_ms"], 4), "GFLOP/s": round(sg, 1),
                "roofline": {"bound": "mfma bf16, 3 products per fp32 product", "achieved": round(3 * sg / 1e3, 2),
                             "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                             "frac": round(3 * sg / 1e3 / PEAK_BF16_TFLOPS, 4), "traffic": None}}
        if "value" not in line:
            line.update({"value": round(gf, 1), "unit": "GFLOP/s", "ms_per_step": round(c1["wall_ms"], 4),
                         "config": {"workload": "C1 SDPA fp32"}})
    for mkey in ("model", "model_bf16"):
        if mkey not in res:
            continue
        m = res[mkey]
        p_tps = m["prompt_len"] / (m["prefill_ms"] * 1e-3)
        p_tf = m["prefill_flops"] / (m["prefill_ms"] * 1e-3) / 1e12
        d_ms = m["replay_ms"] / m["replay_steps"]
        d_gbps = m["step_bytes"] / (d_ms * 1e-3) / 1e9
        line[mkey] = {
            "workload": "C5 Qwen3-0.6B (28 layers, hidden 1024, 16/8 heads, vocab 151936, random bf16 weights): "
                        f"{m['prompt_len']}-token prefill + {m['new_tokens']} greedy decode steps",
            "activations": m["activations"] + (" (the reference's float32 arithmetic; bf16 weights, fp32 "
                                               "activations and KV cache)" if m["activations"] == "float32" else
                                               " (activations and KV cache rounded to bf16 between kernels)"),
            "prefill_ms": round(m["prefill_ms"], 3), "prefill_tokens_per_s": round(p_tps, 1),
            "prefill": {"bound": "mfma", "achieved": round(p_tf, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                        "frac": round(p_tf / PEAK_BF16_TFLOPS, 4), "flops": m["prefill_flops"]},
            "decode_ms_per_token": round(d_ms, 4), "decode_tokens_per_s": round(1e3 / d_ms, 1),
            "decode": {"bound": "hbm", "achieved": round(d_gbps, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                       "frac": round(d_gbps / PEAK_HBM_GBPS, 4),
                       "bytes_per_step": m["step_bytes"]},
            "decode_steps_timed": m["replay_steps"], "decode_total_ms": round(m["decode_ms"], 3),
            "decode_issue": "eager" if args.eager_decode else "hip graph replay",
            "prefill_issue": m["prefill_issue"], "prefill_eager_ms": round(m["prefill_eager_ms"], 3),
            "first_tokens": m["tokens"]}
        if m.get("ts_host") is not None:
            t = m["ts_host"]
            line[mkey]["ts_host"] = {
                "workload": "the same generation driven from Node (packages/backend-hip/examples/generate.js: the "
                            "TypeScript Qwen3 model over the N-API addon)",
                "prefill_ms": round(t["prefill_ms"], 3), "prefill_issue": "hip graph replay",
                "prefill_eager_ms": round(t["prefill_eager_ms"], 3) if t["prefill_eager_ms"] is not None else None,
                "decode_tokens_per_s": round(t["decode_tokens_per_s"], 1), "decode_steps_timed": t["decode_steps_timed"],
                "decode_issue": t["issue"], "load_ms": round(t["load_ms"], 1),
                "tokens_match_python_host": t["tokens_match_python_host"], "first_tokens": t["first_tokens"]}
        if "value" not in line:
            line.update({"value": round(1e3 / d_ms, 1), "unit": "tokens/s", "ms_per_step": round(d_ms, 4),
                         "config": {"workload": "C5 Qwen3-0.6B greedy decode"}})
    if "load" in res:
        ld = res["load"]
        line.update({"value": round(ld["bytes"] / ld["load_s"] / 1e9, 2), "unit": "GB/s", "ms_per_step": round(ld["load_s"] * 1e3, 1),
                     "config": {"workload": "Qwen3-0.6B bf16 safetensors (2 shards, page cache) -> HBM via from_pretrained",
                                "bytes": ld["bytes"], "tokens_match_in_memory_model": ld["tokens_match"]}})
    if "copy" in res:
        c = res["copy"]
        gbps = c["bytes"] / (c["dev_ms"] * 1e-3) / 1e9
        line.update({"value": round(gbps, 1), "unit": "GB/s", "ms_per_step": round(c["wall_ms"], 4),
                     "config": {"workload": "1 GiB device copy (traffic-counter calibration)"}})
    if "sample" in res:
        line["sample"] = dict(res["sample"], workload="kh_sample, one float32 logits row, vocab 151936")
        if "value" not in line:
            sm = res["sample"]["t0.7_k50_p0.9"]
            line.update({"value": round(1e6 / sm["wall_us"], 1), "unit": "draws/s",
                         "ms_per_step": round(sm["wall_us"] * 1e-3, 4),
                         "config": {"workload": "on-device sampling, T=0.7, top-k 50, top-p 0.9, vocab 151936"}})
    if "prefill_b1" in res:
        pb = res["prefill_b1"]
        line.update({"value": pb["S4096"]["TFLOP/s"], "unit": "TFLOP/s", "ms_per_step": pb["S4096"]["ms"],
                     "config": {"workload": "causal bf16 flash prefill of one sequence, Hq=16, Hkv=8, D=128", **pb}})
    if "gemm" in res:
        gm = res["gemm"]
        line.update({"value": gm["layer_TFLOP/s"], "unit": "TFLOP/s", "ms_per_step": round(gm["layer_us"] * 1e-3, 4),
                     "config": {"workload": "C5 prefill projection GEMMs of one layer, M=512", **gm,
                                **({"float32_activations": res["gemm_f32"]} if "gemm_f32" in res else {})},
                     "roofline": {"bound": "mfma", "achieved": gm["layer_TFLOP/s"], "peak": PEAK_BF16_TFLOPS,
                                  "unit": "TFLOP/s", "frac": round(gm["layer_TFLOP/s"] / PEAK_BF16_TFLOPS, 4),
                                  "traffic": None}})
    if "vendor" in res:
        vd = res["vendor"]
        best = max((v.get("TFLOP/s", 0.0) for k2, v in vd.items() if k2.startswith("sdpa_")), default=0.0)
        line.update({"value": best, "unit": "TFLOP/s", "ms_per_step": None,
                     "config": {"workload": "vendor stack reference points on C3 and the C5 prefill GEMMs "
                                            "(torch SDPA, hipBLASLt); not this backend", **vd}})
    if "gemv" in res:
        gv = res["gemv"]
        lm = gv["lm_head"]
        line.update({"value": lm["GB/s"], "unit": "GB/s", "ms_per_step": round(gv["layer_gemv_us"] * 1e-3, 4),
                     "config": {"workload": "C5 decode one-row GEMVs (bf16 weights), graph-replayed", **gv},
                     "roofline": {"bound": "hbm", "achieved": lm["GB/s"], "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                                  "frac": round(lm["GB/s"] / PEAK_HBM_GBPS, 4), "traffic": None}})
    if "mask" in res:
        mk = res["mask"]
        if "value" in line:   # the default run: a sub-object beside the headline it leads
            line["mask"] = dict(mk, roofline=dict(mk["roofline"], traffic=None),
                                note="timed immediately before the headline, which follows it with no idle gap")
        else:
            line.update({"value": mk["TFLOP/s"], "unit": "TFLOP/s", "ms_per_step": mk["wall_ms"],
                         "config": {"workload": mk["workload"], "batch": 4, "q_heads": 16, "kv_heads": 8,
                                    "seq_len": 4096, "head_dim": 128},
                         "roofline": dict(mk["roofline"], traffic=None, kernel=mk["kernel"], kernel_ms=mk["ms"])})
    if "stream" in res:
        st = res["stream"]
        line.update({"value": round(1e3 / st["stream_ms_per_token"], 1), "unit": "tokens/s",
                     "ms_per_step": st["stream_ms_per_token"],
                     "config": {"workload": "C5 Qwen3-0.6B generate_stream, T=0.6 top-k 20 top-p 0.95, 512-token "
                                            "prompt", **st}})
    for key, val in cpu_more.items():
        if key in line:
            line[key]["cpu_baseline"] = val
    line["cpu_baseline"] = cpu
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
