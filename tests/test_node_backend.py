"""The TypeScript HipBackend (packages/backend-hip/src/index.ts) on the CPU: strip-types.js erases
its type syntax into JavaScript that the image's Node (v12, no TypeScript compiler) parses and
loads; the module exports the plugin surface and registers the kernels under the names Kandle's
dispatcher looks up (packages/types/src/backend/register.ts:128-144).  The stripper itself is
checked on a snippet of every construct it handles, by running the output.  Skipped without Node
or the built addon."""
import json
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "packages", "backend-hip")
ADDON = os.path.join(PKG, "native", "kandle_hip.node")
STRIP = os.path.join(PKG, "strip-types.js")


def _need_node():
    if shutil.which("node") is None or not os.path.exists(ADDON):
        pytest.skip("node or the built addon is not available")


def _strip(src_path, out_path):
    subprocess.run(["node", STRIP, str(src_path), str(out_path)], check=True, capture_output=True, timeout=60)


def test_backend_source_strips_to_loadable_javascript(tmp_path):
    _need_node()
    out = tmp_path / "index.js"
    _strip(os.path.join(PKG, "src", "index.ts"), out)
    chk = subprocess.run(["node", "--check", str(out)], capture_output=True, text=True)
    assert chk.returncode == 0, chk.stderr
    # dist/index.js requires ../native/kandle_hip.node relative to itself: load the built copy
    script = f"""
      const m = require({json.dumps(os.path.join(PKG, 'dist', 'index.js'))});
      const reg = new m.SimpleOperatorRegistry();
      m.registerHipKernels(reg);
      console.log(JSON.stringify({{exports: Object.keys(m).sort(), names: reg.names().sort(),
                                  strides: m.contiguousStrides([2, 3, 4]),
                                  bf16: Array.from(m.toBf16Bits(new Float32Array([1, -2.5, 3.14159, 65504]))),
                                  back: Array.from(m.fromBf16Bits(new Uint16Array([0x3f80, 0xc020])))}}));"""
    res = subprocess.run(["node", "-e", script], capture_output=True, text=True, timeout=60)
    assert res.returncode == 0, res.stderr
    r = json.loads(res.stdout.strip().splitlines()[-1])
    assert {"HipBackend", "HipStorage", "HipTensorHandle", "HipTensorIterator", "SimpleOperatorRegistry",
            "registerHipKernels"} <= set(r["exports"])
    for name in ("flash_attention", "flash_attention_split", "rope_table", "sdpa_masked", "rms_norm", "matmul", "mm", "bmm", "addmm", "baddbmm", "add",
                 "mul", "sub", "div", "silu", "silu_mul", "index_select", "argmax", "copy", "contiguous", "cast", "clone",
                 "copy_", "zeros", "ones", "full", "empty", "neg", "cos", "sin", "arange", "decode_attention",
                 "rms_norm_rope", "gemv_fused", "gemv_swiglu", "linear_swiglu", "linear_qk_norm_rope",
                 "linear_add_rms_norm", "decode_attention_block", "greedy_advance", "sample"):
        assert name in r["names"], name
    assert r["strides"] == [12, 4, 1]
    assert r["bf16"] == [0x3F80, 0xC020, 0x4049, 0x4780]   # RNE: 3.14159 -> 0x4049, 65504 -> 65536
    assert r["back"] == [1.0, -2.5]


SNIPPET = r'''
export type Pair = [number, number];
type Fn = (a: number, b: number) => number;
interface Box {
  value: number;
  label?: string;
}
export interface Wide<T> {
  items: T[];
}
interface Named {
  name: string;
}
export class Counter<T> implements Named {
  private count: number = 0;
  readonly name: string;
  items: Map<string, number> = new Map<string, number>();
  constructor(name: string, quiet?: boolean) {
    this.name = name;
  }
  add(n: number = 1): number {
    this.count += n;
    return this.count;
  }
  get total(): number {
    return this.count;
  }
  static make(name: string): Counter<number> {
    return new Counter<number>(name);
  }
}
export function pick(flag: boolean, a?: number, ...rest: number[]): number | undefined {
  const obj: { [k: string]: number } = { x: 1, y: flag ? 2 : 3 };
  const v = (flag ? (a as number) : obj.y) as number;
  const add: Fn = (p: number, q: number): number => p + q;
  let s: number = 0;
  for (const r of rest) s = add(s, r);
  if (s > 0) { return s; }
  const t = `sum ${s as number} ${flag ? 'yes: x' : 'no'}`;
  return t.length > 100 ? undefined : v + obj.x;
}
export const twice = (x: number): number => x * 2;
export function longest(xs: readonly (readonly number[])[], f?: (sc: { [k: string]: any }) => number[]): number {
  let best = 0;
  for (const x of xs) best = Math.max(best, x.length);
  return f === undefined ? best : best + f({ k: 1 })[0];
}
export function wrapped(n: number): number {
  const o = { first: n, second: 2,
              third: 3 };
  return o.first + o.second + o.third;
}
function lessThan(a: number, b: number): boolean { return a < b && b > a; }
export { lessThan };
'''


def test_type_stripper_handles_each_construct(tmp_path):
    _need_node()
    src = tmp_path / "snippet.ts"
    src.write_text(SNIPPET)
    out = tmp_path / "snippet.js"
    _strip(src, out)
    js = out.read_text()
    for leftover in ("interface", "implements", "type Pair", "type Fn", ": number", "private", "readonly", " as ",
                     "<string"):
        assert leftover not in js, (leftover, js)
    script = f"""
      const m = require({json.dumps(str(out))});
      const c = m.Counter.make('k');
      c.add(); c.add(4);
      console.log(JSON.stringify({{total: c.total, name: c.name, size: c.items.size,
                                  p1: m.pick(true, 7), p2: m.pick(false), p3: m.pick(true, 1, 2, 3),
                                  tw: m.twice(21), lt: m.lessThan(1, 2), wr: m.wrapped(1),
                                  lg: m.longest([[1, 2], [3]]), lg2: m.longest([[1]], (o) => [o.k + 1]),
                                  keys: Object.keys(m).sort()}}));"""
    res = subprocess.run(["node", "-e", script], capture_output=True, text=True, timeout=60)
    assert res.returncode == 0, (res.stderr, js)
    r = json.loads(res.stdout.strip().splitlines()[-1])
    assert r == {"total": 5, "name": "k", "size": 0, "p1": 8, "p2": 4, "p3": 5, "tw": 42, "lt": True, "wr": 6,
                 "lg": 2, "lg2": 3, "keys": ["Counter", "lessThan", "longest", "pick", "twice", "wrapped"]}


def test_typescript_safetensors_reader(tmp_path):
    """qwen3.ts's readSafetensors on a file the safetensors package wrote: names, dtypes, shapes and
    the bytes of every tensor; a truncated file is rejected."""
    _need_node()
    import numpy as np
    torch = pytest.importorskip("torch")
    from safetensors.torch import save_file

    a = np.arange(24, dtype=np.float32).reshape(2, 3, 4)
    b = (np.arange(10, dtype=np.int16) * 37).reshape(5, 2)
    save_file({"a.weight": torch.from_numpy(a), "b": torch.from_numpy(b).view(torch.bfloat16)},
              str(tmp_path / "m.safetensors"), metadata={"format": "pt"})
    (tmp_path / "bad.safetensors").write_bytes((tmp_path / "m.safetensors").read_bytes()[:40])
    script = f"""
      const m = require({json.dumps(os.path.join(PKG, 'dist', 'qwen3.js'))});
      const t = m.readSafetensors({json.dumps(str(tmp_path / 'm.safetensors'))});
      const out = {{}};
      for (const k of Object.keys(t)) out[k] = [t[k].dtype, t[k].shape, Array.from(t[k].bytes)];
      let err = null;
      try {{ m.readSafetensors({json.dumps(str(tmp_path / 'bad.safetensors'))}); }} catch (e) {{ err = e.message; }}
      console.log(JSON.stringify({{t: out, err}}));"""
    res = subprocess.run(["node", "-e", script], capture_output=True, text=True, timeout=60)
    assert res.returncode == 0, res.stderr
    r = json.loads(res.stdout.strip().splitlines()[-1])
    assert sorted(r["t"]) == ["a.weight", "b"]
    assert r["t"]["a.weight"][:2] == ["F32", [2, 3, 4]] and bytes(r["t"]["a.weight"][2]) == a.tobytes()
    assert r["t"]["b"][:2] == ["BF16", [5, 2]] and bytes(r["t"]["b"][2]) == b.tobytes()
    assert r["err"] is not None and "outside the file" in r["err"]


def test_generate_example_checks_and_prints_usage(tmp_path):
    """packages/backend-hip/examples/generate.js (the Node generation CLI that bench.py drives on the
    GPU box) parses, and without its four arguments prints its usage and exits with status 2 before
    touching a device; the stripped Qwen3 module it loads exports the model and the reader."""
    _need_node()
    out = tmp_path / "qwen3.js"
    _strip(os.path.join(PKG, "src", "qwen3.ts"), out)
    for js in (str(out), os.path.join(PKG, "examples", "generate.js")):
        chk = subprocess.run(["node", "--check", js], capture_output=True, text=True)
        assert chk.returncode == 0, (js, chk.stderr)
    res = subprocess.run(["node", os.path.join(PKG, "examples", "generate.js")], capture_output=True, text=True,
                         timeout=60)
    assert res.returncode == 2 and "usage: node examples/generate.js CONFIG.json MODEL.safetensors" in res.stderr
    script = f"const m = require({json.dumps(os.path.join(PKG, 'dist', 'qwen3.js'))}); " \
             "console.log(JSON.stringify(Object.keys(m).sort()));"
    r = subprocess.run(["node", "-e", script], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    assert {"Qwen3ForCausalLM", "readSafetensors"} <= set(json.loads(r.stdout.strip().splitlines()[-1]))
