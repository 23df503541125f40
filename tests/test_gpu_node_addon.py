"""The HIP kernels driven from Node through the N-API addon (packages/backend-hip/native/kandle_hip.node):
a child `node` process allocates, uploads, runs a causal GQA flash-attention prefill and a varlen
decode attention through the addon's flashAttention / decodeAttention, and reads the results back;
this test writes the inputs and compares the outputs with the CPU oracle (2e-2 absolute, bf16)."""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

import oracle
from kandle_amd import synthetic as syn

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ADDON = os.path.join(ROOT, "packages", "backend-hip", "native", "kandle_hip.node")
SCRIPT = os.path.join(ROOT, "tests", "node", "addon_ops.js")


def test_node_drives_flash_and_decode_through_the_addon(hip, tmp_path):
    if shutil.which("node") is None or not os.path.exists(ADDON):
        pytest.skip("node or the built addon is not available")
    f = dict(B=2, Hq=8, Hkv=4, S=300, D=128, causal=True)
    d = dict(B=3, Hq=16, Hkv=8, D=128, ML=2000, lens=[1, 777, 2000])
    arrays = {}
    for name, seed, shape in (("fq", 1, (f["B"], f["Hq"], f["S"], 128)), ("fk", 2, (f["B"], f["Hkv"], f["S"], 128)),
                              ("fv", 3, (f["B"], f["Hkv"], f["S"], 128)), ("dq", 4, (d["B"], d["Hq"], 128)),
                              ("dk", 5, (d["B"], d["Hkv"], d["ML"], 128)), ("dv", 6, (d["B"], d["Hkv"], d["ML"], 128))):
        bits, vals = syn.bf16(syn.normal(900 + seed, shape))
        bits.astype(np.uint16).tofile(str(tmp_path / name))
        arrays[name] = vals
    (tmp_path / "meta.json").write_text(json.dumps({"flash": f, "decode": d}))
    out = subprocess.run(["node", SCRIPT, str(tmp_path)], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr[-2000:]
    res = json.loads(out.stdout.strip().splitlines()[-1])
    assert res["ok"] and "must be divisible" in res["gqaError"]

    def bf16_file(name, shape):
        return (np.fromfile(str(tmp_path / name), np.uint16).astype(np.uint32) << 16).view(np.float32).reshape(shape)

    fo = bf16_file("fo", (f["B"], f["Hq"], f["S"], 128))
    ref = oracle.sdpa(arrays["fq"], arrays["fk"], arrays["fv"], causal=True)
    err = float(np.max(np.abs(fo - ref)))
    assert err < 2e-2, err
    do = bf16_file("do", (d["B"], d["Hq"], 128))
    lens = np.array(d["lens"], np.int32)
    ref = oracle.sdpa(arrays["dq"][:, :, None, :], arrays["dk"], arrays["dv"], kv_len=lens)[:, :, 0, :]
    err = float(np.max(np.abs(do - ref)))
    assert err < 2e-2, err
