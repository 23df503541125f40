"""The N-API addon (packages/backend-hip/native/kandle_hip.node) under the image's Node (v12) on the
CPU: it loads, exports one function per entry point the C ABI header declares, reports the devices
the host has, and turns library errors into JS Errors carrying kh_last_error() (the reference's
throw-from-kernel convention, packages/core/src/dispatch/handlers/normalize.ts:57-59).  Skipped
where Node or the built addon is absent."""
import json
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ADDON = os.path.join(ROOT, "packages", "backend-hip", "native", "kandle_hip.node")


def _node(script):
    import shutil
    if shutil.which("node") is None or not os.path.exists(ADDON):
        pytest.skip("node or the built addon is not available")
    out = subprocess.run(["node", "-e", script], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    return json.loads(out.stdout.strip().splitlines()[-1])


def _camel(sym):
    parts = sym[len("kh_"):].split("_")
    return parts[0] + "".join(p[:1].upper() + p[1:] for p in parts[1:])


def test_addon_exports_every_entry_point():
    header = open(os.path.join(ROOT, "include", "kandle_hip.h")).read()
    syms = sorted(set(re.findall(r"^(?:int|const char\*)\s+(kh_\w+)\(", header, re.M)))
    # kh_get_alloc_stats is allocStats, kh_device_count deviceCount, kh_memcpy_h2d memcpyH2D, ...
    special = {"kh_get_alloc_stats": "allocStats", "kh_memcpy_h2d": "memcpyH2D", "kh_memcpy_d2h": "memcpyD2H",
               "kh_memcpy_d2d": "memcpyD2D", "kh_philox4x32_10": "philox4x32_10"}
    want = sorted(special.get(s, _camel(s)) for s in syms)
    got = _node(f"const a = require({json.dumps(ADDON)}); "
                "console.log(JSON.stringify(Object.keys(a).filter(k => typeof a[k] === 'function')))")
    missing = [w for w in want if w not in got]
    assert not missing, missing
    assert len(want) >= 40


def test_addon_errors_and_device_count():
    r = _node(f"""
      const a = require({json.dumps(ADDON)});
      const n = a.deviceCount();
      const res = {{n: n, codes: [a.F32, a.BF16, a.I32]}};
      if (n === 0) {{
        try {{ a.init(0); }} catch (e) {{ res.init = [e.constructor.name, e.code, e.message, a.lastError()]; }}
      }}
      try {{ a.alloc(16); }} catch (e) {{ res.alloc = [e.constructor.name, e.message]; }}
      try {{ a.flashAttention(1n, 2n); }} catch (e) {{ res.arity = [e.constructor.name, e.message]; }}
      try {{ a.fill('x', 1, 0, 0); }} catch (e) {{ res.type = [e.constructor.name, e.message]; }}
      try {{ a.copyStrided(0n, 0, 0n, [1, 2, 3, 4, 5, 6, 7], [1], 0, 0); }} catch (e) {{ res.list = e.message; }}
      // freeOwned / ownedPtr take only blocks from allocOwned
      try {{ a.freeOwned({{}}); }} catch (e) {{ res.owned = [e.constructor.name, e.message]; }}
      res.capturing = a.isCapturing();
      // the longest bindings: every argument reaches the C call (which then reports the missing
      // init), and surplus arguments past the binding's capacity are ignored, never read
      const qknr = [16n, 8, 32n, 8, 1, 4, 8, 1, 1, 128, 48n, 64n, 80n, 96n, 112n, 128n, 144n,
                    [0, 0, 0, 0, 0, 0, 0, 0, 0], 1e-6, 8, 0];
      try {{ a.gemmQkNormRope(...qknr); }} catch (e) {{ res.long = [e.constructor.name, e.message]; }}
      try {{ a.gemmQkNormRope(...qknr, 1, 2, 3, 4, 5); }} catch (e) {{ res.surplus = [e.constructor.name, e.message]; }}
      try {{ a.gemmEx(16n, 8, 0, 32n, 8, 1, 48n, 8, null, 8, null, 1, 1, 8, 1, 0, true, 0); }}
      catch (e) {{ res.ex = [e.constructor.name, e.message]; }}
      console.log(JSON.stringify(res));""")
    assert r["codes"] == [0, 1, 2]
    if r["n"] == 0:
        assert r["init"][0] == "Error" and r["init"][1] == "KH_1"
        assert "device 0 not available" in r["init"][2] and r["init"][2] == r["init"][3]
        assert r["alloc"][0] == "Error" and "kh_init has not been called" in r["alloc"][1]
    assert r["arity"] == ["TypeError", "kandle_hip.flashAttention: expected 14 arguments, got 2"]
    assert r["type"][0] == "TypeError" and "argument 0 must be a device pointer" in r["type"][1]
    assert "at most 6 extents" in r["list"]
    assert r["owned"][0] == "TypeError" and "an owned block" in r["owned"][1]
    assert r["capturing"] is False
    if r["n"] == 0:
        for key in ("long", "surplus", "ex"):
            assert r[key][0] == "Error" and "kh_init has not been called" in r[key][1], (key, r[key])
