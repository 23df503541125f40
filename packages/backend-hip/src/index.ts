// @kandle/backend-hip — Kandle's IBackend for AMD MI355X (gfx950), host side in TypeScript.
//
// The plugin surface mirrors packages/backend-webgpu/src/index.ts:15-87: a backend object with a
// name, createTensorHandle(options | shape, dtype, data) and an operator registry that Kandle's
// dispatcher queries by name (packages/types/src/backend/register.ts:128-144).  Every kernel is one
// call into the N-API addon (../native/kandle_hip.node), which forwards to the C ABI of
// libkandle_hip.so (include/kandle_hip.h): hand-written HIP kernels enqueued on one stream.
// Device pointers travel as BigInt.  Strided inputs are materialised to contiguous storage before a
// kernel sees them, except attention, whose kernels take (batch, head, seq) strides.
//
// Node 12 has no TypeScript compiler here: strip-types.js (next to this package's src/) erases the
// type syntax into dist/index.js, which tests run.  The code keeps to ES2019 for the same reason.

const path = require('path');
const addon = require(path.join(__dirname, '..', 'native', 'kandle_hip.node'));

// ---------------------------------------------------------------------------------------------
// Types mirrored from @kandle/types (tensor.ts:6-55, backend/index.ts:9-55, register.ts:9-144,
// matmulOps.ts:32-125); only the members this backend reads or provides.
// ---------------------------------------------------------------------------------------------
export type DType = 'float32' | 'bfloat16' | 'int32';
export type Shape = number[];
type TypedData = Float32Array | Int32Array | Uint16Array;
type KernelFn = (...args: any[]) => any;

export interface CreateTensorOptions {
  shape: Shape;
  dtype: DType;
  storage?: HipStorage;
  data?: TypedData | number[];
  strides?: number[];
  offset?: number;
}

export interface MatmulConfig {
  output: HipTensorHandle;
  M: number;
  K: number;
  N: number;
  batchSize: number;
  transposeA: boolean;
  transposeB: boolean;
  alpha: number;
  beta: number;
  inputC?: HipTensorHandle;
}

export interface IteratorOperand {
  tensorHandle: HipTensorHandle;
}

export interface TensorIterator {
  numInputs: number;
  output(idx?: number): IteratorOperand;
  input(idx: number): IteratorOperand;
}

const DTYPE_CODE: { [name: string]: number } = { float32: 0, bfloat16: 1, int32: 2 };
const ITEMSIZE: { [name: string]: number } = { float32: 4, bfloat16: 2, int32: 4 };

function contiguousStrides(shape: Shape): number[] {
  const strides = new Array(shape.length).fill(1);
  for (let i = shape.length - 2; i >= 0; --i) strides[i] = strides[i + 1] * shape[i + 1];
  return strides;
}

function numelOf(shape: Shape): number {
  return shape.reduce((a: number, b: number) => a * b, 1);
}

// f32 -> bf16 bits, round to nearest even (NaN kept quiet), and back.
function toBf16Bits(values: Float32Array): Uint16Array {
  const u32 = new Uint32Array(values.buffer, values.byteOffset, values.length);
  const out = new Uint16Array(values.length);
  for (let i = 0; i < values.length; ++i) {
    const x = u32[i];
    if ((x & 0x7fffffff) > 0x7f800000) out[i] = ((x >>> 16) | 0x40) & 0xffff;
    else out[i] = ((x + 0x7fff + ((x >>> 16) & 1)) >>> 16) & 0xffff;
  }
  return out;
}

function fromBf16Bits(bits: Uint16Array): Float32Array {
  const u32 = new Uint32Array(bits.length);
  for (let i = 0; i < bits.length; ++i) u32[i] = bits[i] << 16;
  return new Float32Array(u32.buffer);
}

// ---------------------------------------------------------------------------------------------
// Storage and tensor handles (base/storage.ts:60-245, base/tensor.ts:55-156 semantics)
// ---------------------------------------------------------------------------------------------
let nextId = 1;

export class HipStorage {
  ptr: bigint;
  byteLength: number;
  refCount: number;
  id: number;

  constructor(byteLength: number) {
    this.ptr = addon.alloc(Math.max(byteLength, 1));
    this.byteLength = byteLength;
    this.refCount = 1;
    this.id = nextId++;
  }

  incRef(): void {
    this.refCount += 1;
  }

  // Returns the block to the library's caching allocator once the last view lets go.
  decRef(): void {
    this.refCount -= 1;
    if (this.refCount === 0) addon.free(this.ptr);
  }
}

export class HipTensorHandle {
  readonly shape: Shape;
  readonly dtype: DType;
  readonly strides: number[];
  readonly offset: number;
  readonly storage: HipStorage;
  readonly id: number;
  readonly device: string = 'hip';
  isDisposed: boolean = false;

  constructor(storage: HipStorage, shape: Shape, dtype: DType, strides: number[], offset: number) {
    if (!(dtype in DTYPE_CODE)) throw new TypeError(`backend-hip: unsupported dtype ${dtype}`);
    this.storage = storage;
    this.shape = shape.slice();
    this.dtype = dtype;
    this.strides = strides.slice();
    this.offset = offset;
    this.id = nextId++;
  }

  static createNew(shape: Shape, dtype: DType, data?: TypedData | number[]): HipTensorHandle {
    const n = numelOf(shape);
    const storage = new HipStorage(n * ITEMSIZE[dtype]);
    const h = new HipTensorHandle(storage, shape, dtype, contiguousStrides(shape), 0);
    if (data !== undefined) h.upload(data);
    return h;
  }

  get numel(): number {
    return numelOf(this.shape);
  }

  get storageId(): number {
    return this.storage.id;
  }

  get kh(): number {
    return DTYPE_CODE[this.dtype];
  }

  // Device address of element 0 of this view.
  get ptr(): bigint {
    return this.storage.ptr + BigInt(this.offset * ITEMSIZE[this.dtype]);
  }

  isContiguous(): boolean {
    const want = contiguousStrides(this.shape);
    for (let i = 0; i < this.shape.length; ++i) if (this.shape[i] > 1 && this.strides[i] !== want[i]) return false;
    return true;
  }

  upload(data: TypedData | number[]): void {
    if (!this.isContiguous()) throw new Error('backend-hip: upload into a strided view');
    let host: TypedData;
    if (this.dtype === 'bfloat16') {
      host = data instanceof Uint16Array ? data : toBf16Bits(Float32Array.from(data as number[]));
    } else if (this.dtype === 'int32') {
      host = data instanceof Int32Array ? data : Int32Array.from(data as number[]);
    } else {
      host = data instanceof Float32Array ? data : Float32Array.from(data as number[]);
    }
    if (host.length !== this.numel) throw new Error(`backend-hip: ${host.length} values for ${this.numel} elements`);
    addon.memcpyH2D(this.ptr, host);
  }

  // Logical contiguous values (bf16 widened to float32), after the stream's pending work.
  dataAsync(): Promise<Float32Array | Int32Array> {
    const src = this.isContiguous() ? this : contiguous(this);
    const n = this.numel;
    let out: Float32Array | Int32Array;
    if (this.dtype === 'bfloat16') {
      const bits = new Uint16Array(n);
      addon.memcpyD2H(bits, src.ptr);
      out = fromBf16Bits(bits);
    } else if (this.dtype === 'int32') {
      out = new Int32Array(n);
      addon.memcpyD2H(out, src.ptr);
    } else {
      out = new Float32Array(n);
      addon.memcpyD2H(out, src.ptr);
    }
    if (src !== this) src.dispose();
    return Promise.resolve(out);
  }

  dispose(): void {
    if (this.isDisposed) return;
    this.isDisposed = true;
    this.storage.decRef();
  }
}

function viewOf(base: HipTensorHandle, shape: Shape, strides: number[], offset: number): HipTensorHandle {
  base.storage.incRef();
  return new HipTensorHandle(base.storage, shape, base.dtype, strides, offset);
}

// contiguous()/copy kernel (copy.ts:102-138): a fresh contiguous copy of any view.
function contiguous(x: HipTensorHandle, dtype?: DType): HipTensorHandle {
  const outDtype = dtype === undefined ? x.dtype : dtype;
  const out = HipTensorHandle.createNew(x.shape, outDtype);
  if (x.numel > 0) {
    addon.copyStrided(x.storage.ptr, x.offset, out.ptr, x.shape.length > 0 ? x.shape : [1],
                      x.shape.length > 0 ? x.strides : [1], x.kh, out.kh);
  }
  return out;
}

function materialize(x: HipTensorHandle): HipTensorHandle {
  if (x.isContiguous()) return viewOf(x, x.shape, x.strides, x.offset);
  return contiguous(x);
}

// ---------------------------------------------------------------------------------------------
// Registry (packages/utils/src/registry/index.ts:3-17)
// ---------------------------------------------------------------------------------------------
export class SimpleOperatorRegistry {
  private kernels: Map<string, KernelFn> = new Map<string, KernelFn>();

  register(opName: string, kernelFunc: KernelFn): void {
    this.kernels.set(opName, kernelFunc);
  }

  find(opName: string): KernelFn | undefined {
    return this.kernels.get(opName);
  }

  has(opName: string): boolean {
    return this.kernels.has(opName);
  }

  names(): string[] {
    return Array.from(this.kernels.keys());
  }
}

// ---------------------------------------------------------------------------------------------
// Kernels
// ---------------------------------------------------------------------------------------------

// (batch, head, seq) element strides of a [B, H, L, D] handle whose last axis is contiguous.
function bhlStrides(h: HipTensorHandle, name: string): number[] {
  if (h.shape.length !== 4) throw new Error(`flash_attention: ${name} must be [batch, heads, seq, head_dim]`);
  if (h.strides[3] !== 1) throw new Error(`flash_attention: ${name} needs a contiguous head_dim axis`);
  return [h.strides[0], h.strides[1], h.strides[2]];
}

// flash_attention(query, key, value, output, scale, isCausal) — register.ts:102-109.
function flashAttention(q: HipTensorHandle, k: HipTensorHandle, v: HipTensorHandle, out: HipTensorHandle,
                        scale: number, isCausal: boolean): void {
  const st = bhlStrides(q, 'query').concat(bhlStrides(k, 'key'), bhlStrides(v, 'value'), bhlStrides(out, 'output'));
  addon.flashAttention(q.ptr, k.ptr, v.ptr, out.ptr, q.shape[0], q.shape[1], k.shape[1], q.shape[2], k.shape[2],
                       q.shape[3], st, scale, isCausal, q.kh);
}

// sdpa_masked(query, key, value, mask, output, scale): the attnMask route of composite.ts:279-300 in
// one kernel; the mask broadcasts to [B, Hq, Lq, Lk] (a stride of 0 on a broadcast axis).
function sdpaMasked(q: HipTensorHandle, k: HipTensorHandle, v: HipTensorHandle, mask: HipTensorHandle,
                    out: HipTensorHandle, scale: number): void {
  const st = bhlStrides(q, 'query').concat(bhlStrides(k, 'key'), bhlStrides(v, 'value'), bhlStrides(out, 'output'));
  const target = [q.shape[0], q.shape[1], q.shape[2], k.shape[2]];
  const nd = mask.shape.length;
  const ms: number[] = [];
  for (let i = 0; i < 4; ++i) {
    const j = i - (4 - nd);
    const extent = j >= 0 ? mask.shape[j] : 1;
    if (extent !== 1 && extent !== target[i]) throw new Error('sdpa_masked: the mask does not broadcast to the scores');
    ms.push(j >= 0 && extent !== 1 ? mask.strides[j] : 0);
  }
  addon.flashAttentionMasked(q.ptr, k.ptr, v.ptr, out.ptr, q.shape[0], q.shape[1], k.shape[1], q.shape[2],
                             k.shape[2], q.shape[3], st, scale, mask.ptr, ms, mask.kh, q.kh);
}

// rms_norm(inputs, params) — NormalizeKernelImpl (register.ts:52-55, normalize.ts:46-95): params
// normalizedShape, eps (kernel default 1e-5, executor.ts:58), weight?, out?, outDtype?.
function rmsNorm(inputs: HipTensorHandle[], params: { [key: string]: any }): HipTensorHandle {
  const x = materialize(inputs[0]);
  const ns = (params.normalizedShape || params.normalized_shape) as number[];
  const n = numelOf(ns);
  const eps = params.eps === undefined ? 1e-5 : (params.eps as number);
  const w = params.weight as HipTensorHandle | undefined;
  const outDtype = (params.out ? (params.out as HipTensorHandle).dtype : (params.outDtype || x.dtype)) as DType;
  const out = (params.out as HipTensorHandle | undefined) || HipTensorHandle.createNew(x.shape, outDtype);
  const rows = x.numel / n;
  const wc = w === undefined ? undefined : materialize(w);
  addon.rmsNorm(x.ptr, n, wc === undefined ? null : wc.ptr, out.ptr, n, rows, n, eps, x.kh, out.kh);
  x.dispose();
  if (wc !== undefined) wc.dispose();
  return out;
}

// matmul(config, a, b) — out = alpha * a @ op(b) + beta * inputC (matmulOps.ts:32-125, 486-493).
// a [..., M, K] and out [..., M, N] row-major; b [N, K] with transposeB (nn.Linear weights) or
// [K, N]; batches loop over the leading dims of a (b shared or batched alike).
function matmul(config: MatmulConfig, a: HipTensorHandle, b: HipTensorHandle): void {
  if (config.transposeA) throw new Error('backend-hip matmul: transposeA operands must be materialised first');
  const ac = materialize(a);
  const bc = materialize(b);
  const out = config.output;
  const M = config.M, N = config.N, K = config.K;
  const batch = config.batchSize || 1;
  const bBatched = bc.numel === batch * N * K && batch > 1;
  const c = config.inputC === undefined ? undefined : materialize(config.inputC);
  for (let i = 0; i < batch; ++i) {
    const aPtr = ac.ptr + BigInt(i * M * K * ITEMSIZE[ac.dtype]);
    const bPtr = bc.ptr + BigInt((bBatched ? i * N * K : 0) * ITEMSIZE[bc.dtype]);
    const oPtr = out.ptr + BigInt(i * M * N * ITEMSIZE[out.dtype]);
    const cPtr = c === undefined ? null : c.ptr + BigInt((c.numel === batch * M * N ? i * M * N : 0) * ITEMSIZE[c.dtype]);
    addon.gemm(aPtr, K, bPtr, config.transposeB ? K : N, oPtr, N, cPtr, N, null, M, N, K, config.alpha,
               config.beta, config.transposeB, ac.kh, out.kh);
  }
  ac.dispose();
  bc.dispose();
  if (c !== undefined) c.dispose();
}

function sameShapeContiguous(hs: HipTensorHandle[], name: string): void {
  for (const h of hs) {
    if (h.numel !== hs[0].numel) throw new Error(`${name}: broadcasting operands must be expanded first`);
  }
}

const BINARY_OP: { [name: string]: number } = { add: 0, mul: 1, sub: 2 };

// Pointwise iterator kernels (register.ts:9; ops.ts:299 silu, :329 mul, :437 add): same-shape
// operands, materialised when strided; the output is preallocated by the dispatcher.
function binaryKernel(name: string): KernelFn {
  return (iter: TensorIterator): void => {
    const out = iter.output().tensorHandle;
    const a = materialize(iter.input(0).tensorHandle);
    const b = materialize(iter.input(1).tensorHandle);
    sameShapeContiguous([out, a, b], name);
    addon.binary(BINARY_OP[name], a.ptr, b.ptr, out.ptr, out.numel, out.kh);
    a.dispose();
    b.dispose();
  };
}

function silu(iter: TensorIterator): void {
  const out = iter.output().tensorHandle;
  const x = materialize(iter.input(0).tensorHandle);
  sameShapeContiguous([out, x], 'silu');
  addon.silu(x.ptr, out.ptr, out.numel, out.kh);
  x.dispose();
}

const UNARY_OP: { [name: string]: number } = { neg: 0, cos: 1, sin: 2 };

// neg / cos / sin: what Kandle's composite RoPE (rope.ts:546-644) looks up besides mul and add.
function unaryKernel(name: string): KernelFn {
  return (iter: TensorIterator): void => {
    const out = iter.output().tensorHandle;
    const x = materialize(iter.input(0).tensorHandle);
    sameShapeContiguous([out, x], name);
    if (x.dtype !== out.dtype) throw new Error(`${name}: input and output dtypes differ`);
    addon.unary(UNARY_OP[name], x.ptr, out.ptr, out.numel, out.kh);
    x.dispose();
  };
}

// arange(output, start, step): output[i] = start + i * step (the factory kernel the RoPE tables use).
function arange(out: HipTensorHandle, start?: number, step?: number): void {
  if (!out.isContiguous()) throw new Error('arange: contiguous output expected');
  addon.arange(out.ptr, out.numel, start === undefined ? 0 : start, step === undefined ? 1 : step, out.kh);
}

// decode_attention(query, kCache, vCache, seqLens, output, scale): one query token per sequence
// against [B, Hkv, maxLen, D] caches, each sequence reading its first seqLens[b] (int32, on the
// device) rows — the per-token attention of gqa.ts:246-430 once the KV cache holds the new row.
function decodeAttention(q: HipTensorHandle, kCache: HipTensorHandle, vCache: HipTensorHandle,
                         seqLens: HipTensorHandle, out: HipTensorHandle, scale: number): void {
  const drop = (h: HipTensorHandle): number[][] => (h.shape.length === 4
    ? [[h.shape[0], h.shape[1], h.shape[3]], [h.strides[0], h.strides[1], h.strides[3]]]
    : [h.shape, h.strides]);
  const qv = drop(q);
  const ov = drop(out);
  const B = qv[0][0], Hq = qv[0][1], D = qv[0][2];
  if (kCache.shape.length !== 4 || kCache.shape[3] !== D || vCache.shape.join() !== kCache.shape.join())
    throw new Error('decode_attention: caches must both be [batch, kv_heads, max_len, head_dim]');
  if (ov[0].join() !== qv[0].join()) throw new Error('decode_attention: output shape differs from the query');
  if (seqLens.dtype !== 'int32' || seqLens.numel !== B) throw new Error('decode_attention: seqLens must be int32 [batch]');
  if (qv[1][2] !== 1 || ov[1][2] !== 1 || kCache.strides[3] !== 1 || vCache.strides[3] !== 1)
    throw new Error('decode_attention: the head_dim axis must be contiguous');
  const st = [qv[1][0], qv[1][1]].concat(kCache.strides.slice(0, 3), vCache.strides.slice(0, 3), [ov[1][0], ov[1][1]]);
  addon.decodeAttention(q.ptr, kCache.ptr, vCache.ptr, out.ptr, seqLens.ptr, B, Hq, kCache.shape[1], D,
                        kCache.shape[2], st, scale, q.kh);
}

// rms_norm_rope(q, k, params): per-head RMSNorm with q_norm / k_norm weights and RoPE at int32
// positions, for q [B, S, Hq, D] and k [B, S, Hkv, D] (gqa.ts:279-309 then rope.ts:590-630), written
// heads-first ([B, H, S, D]).  params: qWeight, kWeight, invFreq (float32 [D/2]), positions (int32
// [B*S]), eps, and optional qOut / kOut, v / vOut.  With cachePositions, kOut and vOut are whole KV
// caches [B, Hkv, maxLen, D] and token t lands at row positions[t] (kv-cache.ts:164-212), so the
// write position can live on the device.  Returns [qOut, kOut].
function rmsNormRope(q: HipTensorHandle, k: HipTensorHandle, params: { [key: string]: any }): HipTensorHandle[] {
  if (q.dtype !== k.dtype || q.dtype === 'int32') throw new Error('rms_norm_rope: q and k must share a float dtype');
  if (q.shape.length !== 4 || k.shape.length !== 4) throw new Error('rms_norm_rope: q and k must be [B, S, H, D]');
  const B = q.shape[0], S = q.shape[1], Hq = q.shape[2], D = q.shape[3];
  const Hkv = k.shape[2];
  const qOut = (params.qOut as HipTensorHandle | undefined) || HipTensorHandle.createNew([B, Hq, S, D], q.dtype);
  const kOut = (params.kOut as HipTensorHandle | undefined) || HipTensorHandle.createNew([B, Hkv, S, D], k.dtype);
  const v = params.v as HipTensorHandle | undefined;
  const vOut = params.vOut as HipTensorHandle | undefined;
  const bsh = (h: HipTensorHandle, headsFirst: boolean): number[] => {
    if (h.strides[3] !== 1) throw new Error('rms_norm_rope: head_dim must be contiguous');
    return headsFirst ? [h.strides[0], h.strides[2], h.strides[1]] : [h.strides[0], h.strides[1], h.strides[2]];
  };
  let st = bsh(q, false).concat(bsh(k, false), bsh(qOut, true), bsh(kOut, true));
  if (v !== undefined) {
    if (vOut === undefined) throw new Error('rms_norm_rope: v needs vOut');
    st = st.concat(bsh(v, false), bsh(vOut, true));
  }
  let cacheLen = 0;
  if (params.cachePositions) {
    cacheLen = kOut.shape[2];
    if (vOut !== undefined && vOut.shape[2] !== cacheLen) throw new Error('rms_norm_rope: K and V caches must have the same length');
  }
  const pos = params.positions as HipTensorHandle;
  const invFreq = params.invFreq as HipTensorHandle;
  if (pos.dtype !== 'int32' || pos.numel !== B * S) throw new Error('rms_norm_rope: positions must be int32 with B*S entries');
  if (invFreq.dtype !== 'float32' || invFreq.numel !== D / 2) throw new Error('rms_norm_rope: invFreq must be float32 [D/2]');
  addon.qkNormRope(q.ptr, k.ptr, qOut.ptr, kOut.ptr, v === undefined ? null : v.ptr,
                   vOut === undefined ? null : vOut.ptr, (params.qWeight as HipTensorHandle).ptr,
                   (params.kWeight as HipTensorHandle).ptr, invFreq.ptr, pos.ptr, B, S, Hq, Hkv, D, st,
                   params.eps === undefined ? 1e-6 : (params.eps as number), q.kh, cacheLen);
  return [qOut, kOut];
}

// silu_mul(gate, up, output): SwiGLU's silu(gate) * up in one pass (swiglu.ts:119-134).
function siluMul(gate: HipTensorHandle, up: HipTensorHandle, out: HipTensorHandle): void {
  const g = materialize(gate);
  const u = materialize(up);
  const n = g.shape[g.shape.length - 1];
  const rows = g.numel / n;
  addon.siluMul(g.ptr, n, u.ptr, n, out.ptr, n, rows, n, g.kh);
  g.dispose();
  u.dispose();
}

// index_select(self, index, params, output) — gather/index.ts:16-23; params.dim (default 0).
function indexSelect(self: HipTensorHandle, index: HipTensorHandle, params: { [key: string]: any },
                     output: HipTensorHandle): void {
  const t = materialize(self);
  const idx = materialize(index);
  const nd = t.shape.length;
  const dim = params.dim === undefined ? 0 : ((params.dim as number) + nd) % nd;
  const outer = numelOf(t.shape.slice(0, dim));
  const inner = numelOf(t.shape.slice(dim + 1));
  addon.indexSelectDim(t.ptr, outer, t.shape[dim], inner, idx.ptr, idx.numel, output.ptr, t.kh, output.kh);
  t.dispose();
  idx.dispose();
}

// argmax over the last axis of x into int32 out (lowest index among maxima, NaN never wins).
function argmax(x: HipTensorHandle, out: HipTensorHandle): void {
  const xc = materialize(x);
  const n = xc.shape[xc.shape.length - 1];
  addon.argmax(xc.ptr, xc.numel / n, n, out.ptr, xc.kh);
  xc.dispose();
}

// copy / contiguous / cast (CopyKernelImpl: (input, options) => handle).
function copyKernel(input: HipTensorHandle, options: { [key: string]: any }): HipTensorHandle {
  return contiguous(input, options && options.dtype ? (options.dtype as DType) : undefined);
}

function fill(out: HipTensorHandle, value: number): void {
  if (!out.isContiguous()) throw new Error('fill: contiguous output expected');
  addon.fill(out.ptr, out.numel, value, out.kh);
}

// ---------------------------------------------------------------------------------------------
// The backend (backend-webgpu/src/index.ts:15-87 surface)
// ---------------------------------------------------------------------------------------------
export class HipBackend {
  readonly name: string = 'hip';
  readonly operators: SimpleOperatorRegistry = new SimpleOperatorRegistry();
  readonly device: number;

  private constructor(device: number) {
    this.device = device;
  }

  static async create(device: number = 0): Promise<HipBackend> {
    addon.init(device);
    const b = new HipBackend(device);
    registerHipKernels(b.operators);
    return b;
  }

  // createTensorHandle(options) or the deprecated (shape, dtype, data) form (backend/index.ts:33-55).
  createTensorHandle(optionsOrShape: CreateTensorOptions | Shape, dtype?: DType, data?: TypedData | number[]): HipTensorHandle {
    if (Array.isArray(optionsOrShape)) return HipTensorHandle.createNew(optionsOrShape, dtype as DType, data);
    const o = optionsOrShape as CreateTensorOptions;
    if (o.storage !== undefined) {
      o.storage.incRef();
      return new HipTensorHandle(o.storage, o.shape, o.dtype, o.strides || contiguousStrides(o.shape), o.offset || 0);
    }
    return HipTensorHandle.createNew(o.shape, o.dtype, o.data);
  }

  synchronize(): void {
    addon.synchronize();
  }

  memoryStats(): { [key: string]: number } {
    return addon.allocStats();
  }
}

export function registerHipKernels(reg: SimpleOperatorRegistry): void {
  reg.register('flash_attention', flashAttention);
  reg.register('sdpa_masked', sdpaMasked);
  reg.register('rms_norm', rmsNorm);
  for (const name of ['matmul', 'mm', 'bmm', 'addmm', 'baddbmm']) reg.register(name, matmul);
  reg.register('add', binaryKernel('add'));
  reg.register('mul', binaryKernel('mul'));
  reg.register('sub', binaryKernel('sub'));
  reg.register('silu', silu);
  for (const name of ['neg', 'cos', 'sin']) reg.register(name, unaryKernel(name));
  reg.register('arange', arange);
  reg.register('decode_attention', decodeAttention);
  reg.register('rms_norm_rope', rmsNormRope);
  reg.register('silu_mul', siluMul);
  reg.register('index_select', indexSelect);
  reg.register('argmax', argmax);
  for (const name of ['copy', 'contiguous', 'cast']) reg.register(name, copyKernel);
  reg.register('fill', fill);
}

export { contiguousStrides, toBf16Bits, fromBf16Bits };
