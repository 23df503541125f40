"""Kandle's kernels driven from Node through the TypeScript HipBackend (packages/backend-hip/src/
index.ts, stripped to dist/index.js by strip-types.js): tests/node/backend_ops.js creates the backend,
looks each kernel up in its operator registry by the name Kandle's dispatcher uses and calls it with
the reference kernel signature -- flash_attention, sdpa_masked, rms_norm, matmul (linear plus a
residual), silu_mul, the iterator kernels silu / mul on a transposed view, index_select, argmax,
neg / cos / sin, arange, rms_norm_rope writing KV caches at device positions, decode_attention over
ragged cache lengths, the fused gemv_fused / gemv_swiglu / linear_swiglu / linear_qk_norm_rope / linear_add_rms_norm /
decode_attention_block, sample, greedy_advance, copy_ into a strided view and zeros -- then disposes
every handle.  This test writes the inputs and checks each output against the CPU oracle (the fused
ops bit for bit against the Python binding), that the backend's live device bytes return to where
they started, and that a storage dropped without dispose() is freed by the garbage collector."""
import json
import math
import os
import shutil
import subprocess

import numpy as np
import pytest

import oracle
from kandle_amd import synthetic as syn

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "packages", "backend-hip")
ADDON = os.path.join(PKG, "native", "kandle_hip.node")
SCRIPT = os.path.join(ROOT, "tests", "node", "backend_ops.js")


def _ensure_dist():
    src = os.path.join(PKG, "src", "index.ts")
    dist = os.path.join(PKG, "dist", "index.js")
    if not os.path.exists(dist) or os.path.getmtime(dist) < os.path.getmtime(src):
        os.makedirs(os.path.dirname(dist), exist_ok=True)
        subprocess.run(["node", os.path.join(PKG, "strip-types.js"), src, dist], check=True, timeout=60)


def test_typescript_backend_runs_registered_kernels(hip, tmp_path):
    if shutil.which("node") is None or not os.path.exists(ADDON):
        pytest.skip("node or the built addon is not available")
    _ensure_dist()
    f = dict(B=1, Hq=8, Hkv=2, S=200, D=128)
    r = dict(rows=5, n=1000, eps=1e-6)
    m = dict(M=37, K=256, N=96)
    e = dict(V=50, H=64, n=7)
    A = {}

    def put_bf16(name, seed, shape, std=1.0):
        bits, vals = syn.bf16(syn.normal(seed, shape, std))
        bits.astype(np.uint16).tofile(str(tmp_path / name))
        A[name] = vals

    def put_f32(name, arr):
        arr = np.ascontiguousarray(arr, np.float32)
        arr.tofile(str(tmp_path / name))
        A[name] = arr

    put_bf16("fq", 11, (f["B"], f["Hq"], f["S"], f["D"]))
    put_bf16("fk", 12, (f["B"], f["Hkv"], f["S"], f["D"]))
    put_bf16("fv", 13, (f["B"], f["Hkv"], f["S"], f["D"]))
    bias = syn.uniform(14, (f["S"], f["S"]), -1.0, 1.0)
    bias[np.triu_indices(f["S"], 1)] = -np.inf
    put_f32("fmask", bias)
    put_f32("nx", syn.normal(15, (r["rows"], r["n"]), 3.0))
    put_bf16("nw", 16, (r["n"],))
    put_bf16("ma", 17, (m["M"], m["K"]))
    put_bf16("mb", 18, (m["N"], m["K"]))
    put_f32("mc", syn.normal(19, (m["M"], m["N"]), 2.0))
    put_bf16("et", 20, (e["V"], e["H"]))
    ids = syn.randint(21, (e["n"],), 0, e["V"])
    ids[0], ids[-1] = 0, e["V"] - 1
    ids.tofile(str(tmp_path / "ei"))
    p = dict(T=5, Hq=4, Hkv=2, D=128, L=8, eps=1e-6)
    put_bf16("rq", 22, (1, p["T"], p["Hq"], p["D"]))
    put_bf16("rk", 23, (1, p["T"], p["Hkv"], p["D"]))
    put_bf16("rv", 24, (1, p["T"], p["Hkv"], p["D"]))
    for name, seed in (("rwq", 25), ("rwk", 26)):
        bits, vals = syn.bf16(syn.uniform(seed, (p["D"],), 0.5, 1.5))
        bits.astype(np.uint16).tofile(str(tmp_path / name))
        A[name] = vals
    put_f32("rinv", oracle.rope_inv_freq(p["D"], 1e6))
    rpos = np.array([3, 0, 7, 9, 1], np.int32)            # 9 is outside the 8-row cache: writes nothing
    rpos.tofile(str(tmp_path / "rpos"))
    dd = dict(B=3, Hq=8, Hkv=2, D=128, L=96, lens=[1, 50, 96])
    put_bf16("dq", 27, (dd["B"], dd["Hq"], dd["D"]))
    put_bf16("dk", 28, (dd["B"], dd["Hkv"], dd["L"], dd["D"]))
    put_bf16("dv", 29, (dd["B"], dd["Hkv"], dd["L"], dd["D"]))
    # fused ops (run again through the Python binding below, on the same inputs)
    fu = dict(gvN=512, gvK=1024, swM=37, swH=256, swI=96, lM=64, lN=1024, lK=2048)
    put_f32("gvx", syn.normal(30, (fu["gvK"],), 2.0))
    put_bf16("gvw", 31, (fu["gvN"], fu["gvK"]), 0.05)
    put_bf16("gvn", 32, (fu["gvK"],))
    put_bf16("gvb", 33, (fu["gvK"],))
    put_f32("gvc", syn.normal(34, (1, fu["gvN"])))
    put_bf16("swx", 35, (fu["swM"], fu["swH"]))
    put_bf16("swg", 36, (2 * fu["swI"], fu["swH"]), 0.1)
    put_bf16("lax", 37, (fu["lM"], fu["lK"]))
    put_bf16("law", 38, (fu["lN"], fu["lK"]), 0.05)
    put_f32("lar", syn.normal(39, (fu["lM"], fu["lN"])))
    put_bf16("lan", 40, (fu["lN"],))
    blk = dict(Hq=16, Hkv=8, L=64, hidden=1024, pos=20, qS=40, qPos0=30)
    put_bf16("bqkv", 41, (1, (blk["Hq"] + 2 * blk["Hkv"]) * 128))
    put_bf16("bqn", 42, (128,))
    put_bf16("bkn", 43, (128,))
    put_f32("binv", oracle.rope_inv_freq(128, 1e6))
    put_bf16("bkc", 44, (1, blk["Hkv"], blk["L"], 128))
    put_bf16("bvc", 45, (1, blk["Hkv"], blk["L"], 128))
    put_bf16("bwo", 46, (blk["hidden"], blk["Hq"] * 128), 0.02)
    put_f32("bx", syn.normal(47, (1, blk["hidden"])))
    put_bf16("qx", 50, (blk["qS"], blk["hidden"]))
    put_bf16("qw", 51, ((blk["Hq"] + 2 * blk["Hkv"]) * 128, blk["hidden"]), 0.05)
    smp = dict(V=1000, seed=1234, counter=7)
    put_f32("slg", syn.normal(48, (smp["V"],), 3.0))
    put_f32("cps", syn.normal(49, (4, 3)))
    (tmp_path / "meta.json").write_text(json.dumps({"flash": f, "norm": r, "mm": m, "emb": e, "rope": p,
                                                    "decode": dd, "fused": fu, "block": blk, "sample": smp}))

    out = subprocess.run(["node", "--expose-gc", SCRIPT, str(tmp_path)], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr[-2000:]
    res = json.loads(out.stdout.strip().splitlines()[-1])
    assert res["ok"]
    assert res["liveAfter"] == res["liveBefore"], res
    assert res["gcFreed"]["held"] >= 4 << 20 and res["gcFreed"]["left"] == 0, res["gcFreed"]   # GC safety net

    def f32_file(name, shape, dtype=np.float32):
        return np.fromfile(str(tmp_path / name), dtype).reshape(shape)

    fshape = (f["B"], f["Hq"], f["S"], f["D"])
    err = float(np.max(np.abs(f32_file("fo", fshape) - oracle.sdpa(A["fq"], A["fk"], A["fv"], causal=True))))
    assert err < 2e-2, ("flash_attention", err)
    ref = oracle.sdpa_masked(A["fq"], A["fk"], A["fv"], A["fmask"])
    err = float(np.max(np.abs(f32_file("fmo", fshape) - ref)))
    assert err < 2e-2, ("sdpa_masked", err)

    # rms_norm: fp32 arithmetic, one bf16 rounding of the output
    y = f32_file("ny", (r["rows"], r["n"]))
    ref = oracle.rms_norm(A["nx"], A["nw"], r["eps"])
    np.testing.assert_allclose(y, ref, rtol=2 ** -8, atol=1e-6)

    c = A["mc"]
    np.testing.assert_allclose(f32_file("mo", (m["M"], m["N"])), oracle.linear(A["ma"], A["mb"], cin=c, beta=1.0),
                               rtol=1e-5, atol=1e-4)
    np.testing.assert_allclose(f32_file("sm", (m["M"], m["N"])), oracle.silu_mul(c, np.full_like(c, 0.5)),
                               rtol=1e-5, atol=1e-6)
    st = f32_file("st", (m["N"], m["M"]))
    np.testing.assert_allclose(st, oracle.silu_mul(c.T.copy()), rtol=1e-5, atol=1e-6)
    np.testing.assert_array_equal(f32_file("pt", (m["N"], m["M"])), c.T * st)
    np.testing.assert_array_equal(f32_file("eo", (e["n"], e["H"])), A["et"][ids])
    np.testing.assert_array_equal(f32_file("am", (m["M"],), np.int32), oracle.argmax(c))
    for name, fn in (("neg", np.negative), ("cos", np.cos), ("sin", np.sin)):
        np.testing.assert_allclose(f32_file("u_" + name, (m["M"], m["N"])), fn(c), rtol=0, atol=2e-6)
    np.testing.assert_array_equal(f32_file("ar", (10,)), 0.5 + 2.0 * np.arange(10, dtype=np.float32))

    # rms_norm_rope: one bf16 rounding of the fp32 result; cache rows no in-range token names keep 7
    bar = lambda g, ref: np.all(np.abs(g - ref) <= 2 ** -8 * np.abs(ref) + 1e-5)
    rq = oracle.qk_norm_rope(A["rq"][0], A["rwq"], rpos, A["rinv"], p["eps"])        # [T, Hq, D]
    rk = oracle.qk_norm_rope(A["rk"][0], A["rwk"], rpos, A["rinv"], p["eps"])        # [T, Hkv, D]
    qo = f32_file("rqo", (p["Hq"], p["T"], p["D"])).transpose(1, 0, 2)
    assert bar(qo, rq), float(np.max(np.abs(qo - rq)))
    kc = f32_file("rkc", (p["Hkv"], p["L"], p["D"]))
    vc = f32_file("rvc", (p["Hkv"], p["L"], p["D"]))
    written = set()
    for t, row in enumerate(rpos):
        if row < p["L"]:
            written.add(int(row))
            assert bar(kc[:, row], rk[t]), (t, float(np.max(np.abs(kc[:, row] - rk[t]))))
            np.testing.assert_array_equal(vc[:, row], A["rv"][0, t])
    for row in set(range(p["L"])) - written:
        assert np.all(kc[:, row] == 7) and np.all(vc[:, row] == 7), row

    do = f32_file("do", (dd["B"], dd["Hq"], dd["D"]))
    ref = oracle.sdpa(A["dq"][:, :, None, :], A["dk"], A["dv"], kv_len=np.array(dd["lens"], np.int32))[:, :, 0, :]
    err = float(np.max(np.abs(do - ref)))
    assert err < 2e-2, ("decode_attention", err)

    # The fused ops: bit for bit what the Python binding computes from the same inputs.
    from kandle_amd import HipTensorHandle, Tensor, kernels

    T = lambda name, dt="bfloat16": Tensor(A[name], dtype=dt)  # noqa: E731
    gx, gw, gn, gb, gc = T("gvx", "float32"), T("gvw"), T("gvn"), T("gvb"), T("gvc", "float32")
    go = HipTensorHandle.create_new((1, fu["gvN"]), "bfloat16")
    kernels.gemv_fused("rms_norm", gx.handle, gw.handle, go, {"norm_weight": gn.handle, "eps": 1e-6})
    np.testing.assert_array_equal(f32_file("gvo", (1, fu["gvN"])), go.data_async())
    gs = HipTensorHandle.create_new((1, fu["gvN"] // 2), "bfloat16")
    kernels.gemv_swiglu("rms_norm", gx.handle, gw.handle, gs, {"norm_weight": gn.handle, "eps": 1e-6})
    np.testing.assert_array_equal(f32_file("gvs", (1, fu["gvN"] // 2)), gs.data_async())
    kernels.gemv_fused("none", gb.handle, gw.handle, gc.handle, {"cin": gc.handle})
    np.testing.assert_array_equal(f32_file("gvr", (1, fu["gvN"])), gc.numpy())
    sx, sg = T("swx"), T("swg")
    so = HipTensorHandle.create_new((fu["swM"], fu["swI"]), "bfloat16")
    kernels.linear_swiglu(sx.handle, sg.handle, so)
    np.testing.assert_array_equal(f32_file("swo", (fu["swM"], fu["swI"])), so.data_async())
    assert kernels.gemm_split_count(fu["lM"], fu["lN"], fu["lK"]) > 1   # the partials + add-norm route
    lx, lw, lr, ln = T("lax"), T("law"), T("lar", "float32"), T("lan")
    lo = HipTensorHandle.create_new((fu["lM"] - 1, fu["lN"]), "bfloat16")
    kernels.linear_add_rms_norm(lx.handle, lw.handle, lr.handle, ln.handle, 1e-6, lo, rows=(1, fu["lM"]))
    np.testing.assert_array_equal(f32_file("lao", (fu["lM"] - 1, fu["lN"])), lo.data_async())
    np.testing.assert_array_equal(f32_file("lar2", (fu["lM"], fu["lN"])), lr.numpy())

    bk, bv, bx = T("bkc"), T("bvc"), T("bx", "float32")
    bpos = Tensor(np.array([blk["pos"]], np.int32), dtype="int32")
    kernels.decode_attention_block(T("bqkv").handle, {
        "q_norm": T("bqn").handle, "k_norm": T("bkn").handle, "inv_freq": T("binv", "float32").handle, "eps": 1e-6,
        "position": bpos.handle, "k_cache": bk.handle, "v_cache": bv.handle, "w_o": T("bwo").handle,
        "x": bx.handle, "scale": 1.0 / math.sqrt(128)})
    np.testing.assert_array_equal(f32_file("bxo", (1, blk["hidden"])), bx.numpy())
    np.testing.assert_array_equal(f32_file("bkco", bk.shape), bk.numpy())
    np.testing.assert_array_equal(f32_file("bvco", bv.shape), bv.numpy())
    assert not np.array_equal(bx.numpy(), A["bx"])                 # the block did add into x

    qpos = Tensor(np.arange(blk["qPos0"], blk["qPos0"] + blk["qS"], dtype=np.int32), dtype="int32")
    qkc, qvc = T("bkc"), T("bvc")
    qq = HipTensorHandle.create_new((1, blk["Hq"], blk["qS"], 128), "bfloat16")
    kernels.linear_qk_norm_rope(T("qx").handle, T("qw").handle, {
        "q_weight": T("bqn").handle, "k_weight": T("bkn").handle, "inv_freq": T("binv", "float32").handle,
        "positions": qpos.handle, "eps": 1e-6, "q_out": qq, "k_out": qkc.handle, "v_out": qvc.handle})
    np.testing.assert_array_equal(f32_file("qqo", (1, blk["Hq"], blk["qS"], 128)), qq.data_async())
    np.testing.assert_array_equal(f32_file("qkco", qkc.shape), qkc.numpy())
    np.testing.assert_array_equal(f32_file("qvco", qvc.shape), qvc.numpy())
    assert not np.array_equal(qkc.numpy(), A["bkc"])               # rows 30..63 were written

    lg = T("slg", "float32")
    tok = Tensor(np.zeros(1, np.int32), dtype="int32")
    kernels.sample(lg.handle, {"do_sample": False, "token": tok.handle})
    assert res["greedyTok"] == int(tok.numpy()[0]) == int(np.argmax(A["slg"]))
    ctr = Tensor(np.array([smp["counter"]], np.int32), dtype="int32")
    lp = Tensor(np.zeros(1, np.float32))
    kernels.sample(lg.handle, {"do_sample": True, "temperature": 0.8, "top_k": 50, "top_p": 0.9, "seed": smp["seed"],
                               "counter": ctr.handle, "token": tok.handle, "logprob": lp.handle})
    assert res["sampledTok"] == int(tok.numpy()[0])
    assert np.float32(res["sampledLp"]) == lp.numpy()[0]

    assert res["adv"] == {"pos": 6, "len": 7, "log": [0, 0, 0, 42, 0, 0, 0, 0, 0, 0]}
    buf = np.zeros((4, 8), np.float32)
    buf[:, 2:5] = A["cps"]
    np.testing.assert_array_equal(f32_file("cpo", (4, 8)), buf)
    assert res["zsum"] == 0
