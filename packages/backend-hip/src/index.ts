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
// int64 is stored as int32 on the device, as backend-webgpu stores it (base/DTypeResolver.ts:331-350:
// uploads narrow BigInt64 values to i32, downloads widen them back to BigInt64Array).
export type DType = 'float32' | 'bfloat16' | 'int32' | 'int64';
export type Shape = number[];
type TypedData = Float32Array | Int32Array | Uint16Array | BigInt64Array;
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

// TensorIteratorOperand / ITensorIterator (types/src/tensor.ts:282-569): what an iterator kernel
// reads.  strides are element strides aligned to outputShape (0 on broadcast axes) and offset is in
// elements; for a reduction input, strides cover the kept axes and reductionStrides the reduced ones.
export interface IteratorOperand {
  tensorHandle: HipTensorHandle;
  dtype?: DType;
  shape?: readonly number[];
  strides?: readonly number[];
  offset?: number;
  isOutput?: boolean;
  reductionStrides?: readonly number[];
}

export interface TensorIterator {
  numInputs: number;
  numOutputs?: number;
  inputShape?: readonly number[];
  outputShape?: readonly number[];
  outputNumel?: number;
  isReduction?: boolean;
  reductionAxes?: readonly number[];
  reductionShape?: readonly number[];
  keepDims?: boolean;
  output(idx?: number): IteratorOperand;
  input(idx?: number): IteratorOperand;
  getScalarArgs?(): { [key: string]: any };
}

const DTYPE_CODE: { [name: string]: number } = { float32: 0, bfloat16: 1, int32: 2, int64: 2 };
const ITEMSIZE: { [name: string]: number } = { float32: 4, bfloat16: 2, int32: 4, int64: 4 };

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

// The device block is an addon-owned object: dispose() frees it through the last view's decRef, and
// a storage that is dropped without dispose() is freed by the object's finalizer when the garbage
// collector reclaims it (the role of backend-webgpu's FinalizationRegistry, storage.ts:6-14, which
// Node 12 lacks).
export class HipStorage {
  ptr: bigint;
  byteLength: number;
  refCount: number;
  id: number;
  private block: any;

  constructor(byteLength: number) {
    this.block = addon.allocOwned(Math.max(byteLength, 1));
    this.ptr = addon.ownedPtr(this.block);
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
    if (this.refCount === 0) addon.freeOwned(this.block);
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
    if (strides.length !== shape.length) throw new Error(`backend-hip: ${strides.length} strides for a ${shape.length}-d shape`);
    checkExtent(storage, shape, strides, offset, dtype, 'view');
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
    } else if (this.dtype === 'int64') {
      // narrowed to the int32 storage (DTypeResolver.ts:331-340)
      const src = data as any;
      host = new Int32Array(src.length);
      for (let i = 0; i < src.length; ++i) (host as Int32Array)[i] = Number(src[i]);
    } else {
      host = data instanceof Float32Array ? data : Float32Array.from(data as number[]);
    }
    if (host.length !== this.numel) throw new Error(`backend-hip: ${host.length} values for ${this.numel} elements`);
    addon.memcpyH2D(this.ptr, host);
  }

  // Logical contiguous values (bf16 widened to float32, int64 widened to BigInt64Array from its
  // int32 storage), after the stream's pending work.
  dataAsync(): Promise<Float32Array | Int32Array | BigInt64Array> {
    const src = this.isContiguous() ? this : contiguous(this);
    const n = this.numel;
    let out: Float32Array | Int32Array | BigInt64Array;
    if (this.dtype === 'bfloat16') {
      const bits = new Uint16Array(n);
      addon.memcpyD2H(bits, src.ptr);
      out = fromBf16Bits(bits);
    } else if (this.dtype === 'int32') {
      out = new Int32Array(n);
      addon.memcpyD2H(out, src.ptr);
    } else if (this.dtype === 'int64') {
      const narrow = new Int32Array(n);
      addon.memcpyD2H(narrow, src.ptr);
      out = new BigInt64Array(n);
      for (let i = 0; i < n; ++i) (out as BigInt64Array)[i] = BigInt(narrow[i]);
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

// The element offsets a view of `shape` with `strides` from `offset` reaches must lie inside its
// storage: every kernel addresses memory from these numbers, so a view running past the block (or
// before it) is refused here rather than read or written on the device.
function checkExtent(storage: HipStorage, shape: readonly number[], strides: readonly number[], offset: number,
                     dtype: string, what: string): void {
  if (!Number.isInteger(offset) || offset < 0) throw new Error(`backend-hip: ${what} offset ${offset} is not a non-negative integer`);
  let lo = offset, hi = offset, empty = false;
  for (let i = 0; i < shape.length; ++i) {
    if (!Number.isInteger(shape[i]) || shape[i] < 0) throw new Error(`backend-hip: ${what} extent ${shape[i]} is invalid`);
    if (shape[i] === 0) empty = true;
    const span = (shape[i] - 1) * strides[i];
    if (span < 0) lo += span; else hi += span;
  }
  if (empty) return;
  const capacity = Math.floor(storage.byteLength / ITEMSIZE[dtype]);
  if (lo < 0 || hi >= capacity)
    throw new Error(`backend-hip: ${what} reaches elements [${lo}, ${hi}] of a storage holding ${capacity}`);
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

// flash_attention_split(query, key, value, output, scale, isCausal): flash_attention's signature for
// fp32 operands in split-bf16 form (each fp32 value as bf16 hi + lo, every product as three bf16
// MFMAs, within about 2^-15 relative of the fp32 products); the float32-activation prefill's
// attention.  Shapes the split kernel does not take run the fp32 kernel.
function flashAttentionSplit(q: HipTensorHandle, k: HipTensorHandle, v: HipTensorHandle, out: HipTensorHandle,
                             scale: number, isCausal: boolean): void {
  if (q.dtype !== 'float32' || k.dtype !== 'float32' || v.dtype !== 'float32' || out.dtype !== 'float32')
    throw new Error('flash_attention_split: float32 operands expected');
  const st = bhlStrides(q, 'query').concat(bhlStrides(k, 'key'), bhlStrides(v, 'value'), bhlStrides(out, 'output'));
  addon.flashAttentionSplit(q.ptr, k.ptr, v.ptr, out.ptr, q.shape[0], q.shape[1], k.shape[1], q.shape[2], k.shape[2],
                            q.shape[3], st, scale, isCausal);
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
  if (params.bias !== undefined && params.bias !== null) throw new Error('rms_norm: bias is not part of RMSNorm');
  const outDtype = (params.out ? (params.out as HipTensorHandle).dtype : (params.outDtype || x.dtype)) as DType;
  const out = (params.out as HipTensorHandle | undefined) || HipTensorHandle.createNew(x.shape, outDtype);
  const rows = x.numel / n;
  const wc = w === undefined ? undefined : materialize(w);
  addon.rmsNorm(x.ptr, n, wc === undefined ? null : wc.ptr, out.ptr, n, rows, n, eps, x.kh, out.kh);
  x.dispose();
  if (wc !== undefined) wc.dispose();
  return out;
}

// matmul(config, a, b) — out = alpha * op(a) @ op(b) + beta * inputC (matmulOps.ts:32-125, 486-493).
// op(a) [..., M, K]: a itself, or with transposeA a stored [..., K, M] (the dispatcher's transpose
// detection from strides, matmulOps.ts:171-181), materialised as [..., M, K]; out [..., M, N]
// row-major; b [N, K] with transposeB (nn.Linear weights) or [K, N]; batches loop over the leading
// dims of a (b shared or batched alike).  float32 activations may meet bfloat16 weights.
function matmul(config: MatmulConfig, a: HipTensorHandle, b: HipTensorHandle): void {
  let at = a;
  if (config.transposeA) {
    const nd = a.shape.length;
    if (nd < 2) throw new Error('matmul: transposeA needs a matrix');
    const sh = a.shape.slice(), st = a.strides.slice();
    [sh[nd - 2], sh[nd - 1]] = [sh[nd - 1], sh[nd - 2]];
    [st[nd - 2], st[nd - 1]] = [st[nd - 1], st[nd - 2]];
    at = viewOf(a, sh, st, a.offset);
  }
  const ac = materialize(at);
  if (at !== a) at.dispose();
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
    addon.gemmEx(aPtr, K, ac.kh, bPtr, config.transposeB ? K : N, bc.kh, oPtr, N, cPtr, N, null, M, N, K,
                 config.alpha, config.beta, config.transposeB, out.kh);
  }
  ac.dispose();
  bc.dispose();
  if (c !== undefined) c.dispose();
}

// ---------------------------------------------------------------------------------------------
// Iterators: the operand geometry Kandle's dispatcher hands an iterator kernel
// (core/src/dispatch/TensorIterator.ts), and the kernels that consume it
// ---------------------------------------------------------------------------------------------

// computeBroadcastStrides (utils/src/shape.ts:57-100): the strides of a view of `shape` / `strides`
// read at every index of `target` (right-aligned; 0 on new axes and on broadcast extents of 1).
function broadcastStrides(shape: readonly number[], strides: readonly number[], target: readonly number[]): number[] {
  if (target.length < shape.length) throw new Error('broadcast: the target shape has fewer dimensions');
  const out: number[] = new Array(target.length).fill(0);
  for (let i = 0; i < target.length; ++i) {
    const si = shape.length - target.length + i;
    if (si < 0) continue;
    if (shape[si] === target[i]) out[i] = strides[si];
    else if (shape[si] !== 1) throw new Error(`broadcast: [${shape}] does not broadcast to [${target}]`);
  }
  return out;
}

function broadcastShapes(shapes: readonly (readonly number[])[]): number[] {
  let nd = 0;
  for (const sh of shapes) nd = Math.max(nd, sh.length);
  const out: number[] = new Array(nd).fill(1);
  for (const sh of shapes) {
    for (let i = 0; i < sh.length; ++i) {
      const j = nd - sh.length + i;
      if (sh[i] === out[j] || sh[i] === 1) continue;
      if (out[j] !== 1) throw new Error(`broadcast: shapes ${shapes.map((x) => '[' + x + ']').join(', ')} do not broadcast`);
      out[j] = sh[i];
    }
  }
  return out;
}

// The dtype an elementwise op computes and stores in (the dispatcher's type promotion, reduced to
// this backend's dtypes): float32 over bfloat16, floats over integers.
function promoteTypes(dtypes: readonly DType[]): DType {
  if (dtypes.indexOf('float32') >= 0) return 'float32';
  if (dtypes.indexOf('bfloat16') >= 0) return 'bfloat16';
  if (dtypes.indexOf('int64') >= 0) return 'int64';
  return 'int32';
}

// An ITensorIterator over this backend's handles, built the way Kandle's TensorIterator factories
// build one (unaryOp / binaryOp / nullaryOp / reductionOp / build, TensorIterator.ts): outputs first,
// input strides aligned to the output shape, outputs allocated when not given, scalar arguments.
export class HipTensorIterator implements TensorIterator {
  readonly inputShape: number[];
  readonly outputShape: number[];
  readonly outputNumel: number;
  readonly operands: IteratorOperand[];
  readonly numOutputs: number;
  readonly numInputs: number;
  readonly isReduction: boolean;
  readonly reductionAxes: number[];
  readonly reductionShape: number[];
  readonly keepDims: boolean;
  private scalarArgs: { [key: string]: any } = {};

  private constructor(inputShape: number[], outputShape: number[], operands: IteratorOperand[], numOutputs: number,
                      reductionAxes: number[], keepDims: boolean) {
    this.inputShape = inputShape;
    this.outputShape = outputShape;
    this.outputNumel = numelOf(outputShape);
    this.operands = operands;
    this.numOutputs = numOutputs;
    this.numInputs = operands.length - numOutputs;
    this.isReduction = reductionAxes.length > 0;
    this.reductionAxes = reductionAxes;
    this.reductionShape = reductionAxes.map((a) => inputShape[a]);
    this.keepDims = keepDims;
  }

  output(idx: number = 0): IteratorOperand {
    return this.operands[idx];
  }

  input(idx: number = 0): IteratorOperand {
    return this.operands[this.numOutputs + idx];
  }

  setScalarArgs(args: { [key: string]: any }): void {
    this.scalarArgs = Object.assign({}, args);
  }

  getScalarArgs(): { [key: string]: any } {
    return Object.assign({}, this.scalarArgs);
  }

  getScalarArg(name: string): any {
    return this.scalarArgs[name];
  }

  private static operand(h: HipTensorHandle, strides: readonly number[], isOutput: boolean): IteratorOperand {
    return { tensorHandle: h, dtype: h.dtype, shape: h.shape, strides: strides.slice(), offset: h.offset, isOutput };
  }

  // An elementwise iterator: the inputs broadcast to one shape; the output (allocated in outDtype,
  // default the promoted input dtype, when not given) has that shape.
  static build(inputs: HipTensorHandle[], output?: HipTensorHandle, outDtype?: DType): HipTensorIterator {
    const shape = output !== undefined ? output.shape.slice() : broadcastShapes(inputs.map((h) => h.shape));
    if (output !== undefined) broadcastShapes([output.shape as readonly number[]].concat(inputs.map((h) => h.shape)));
    const out = output !== undefined ? output
      : HipTensorHandle.createNew(shape, outDtype || promoteTypes(inputs.map((h) => h.dtype)));
    const ops = [HipTensorIterator.operand(out, out.strides, true)].concat(
      inputs.map((h) => HipTensorIterator.operand(h, broadcastStrides(h.shape, h.strides, shape), false)));
    return new HipTensorIterator(shape, shape, ops, 1, [], false);
  }

  static unaryOp(x: HipTensorHandle, output?: HipTensorHandle): HipTensorIterator {
    return HipTensorIterator.build([x], output);
  }

  static binaryOp(a: HipTensorHandle, b: HipTensorHandle, output?: HipTensorHandle): HipTensorIterator {
    return HipTensorIterator.build([a, b], output);
  }

  // A factory's iterator: no inputs, a new contiguous output of `shape` and `dtype`, or `output`.
  static nullaryOp(shape: number[], dtype: DType, output?: HipTensorHandle): HipTensorIterator {
    const out = output !== undefined ? output : HipTensorHandle.createNew(shape, dtype);
    return new HipTensorIterator(out.shape.slice(), out.shape.slice(),
                                 [HipTensorIterator.operand(out, out.strides, true)], 1, [], false);
  }

  // A reduction over `axes` (all axes when empty or undefined): the output has the kept axes (and
  // extent-1 reduced axes with keepDims); the input's strides split into the kept axes' and the
  // reduced axes' (reductionStrides), as splitStridesForReduction does.
  static reductionOp(x: HipTensorHandle, axes: number[] | undefined, keepDims: boolean, output?: HipTensorHandle,
                     outDtype?: DType): HipTensorIterator {
    const nd = x.shape.length;
    const red = (axes === undefined || axes.length === 0 ? x.shape.map((_: number, i: number) => i)
      : axes.map((a) => (a < 0 ? a + nd : a))).sort((p, q) => p - q);
    for (const a of red) if (a < 0 || a >= nd) throw new Error(`reduction: axis out of range for a ${nd}-d tensor`);
    const kept = x.shape.map((_: number, i: number) => i).filter((i: number) => red.indexOf(i) < 0);
    const outShape = keepDims ? x.shape.map((e: number, i: number) => (red.indexOf(i) >= 0 ? 1 : e))
      : kept.map((i: number) => x.shape[i]);
    const out = output !== undefined ? output : HipTensorHandle.createNew(outShape, outDtype || x.dtype);
    if (out.numel !== numelOf(outShape)) throw new Error(`reduction: output [${out.shape}] for a result of [${outShape}]`);
    const inOp = HipTensorIterator.operand(x, kept.map((i: number) => x.strides[i]), false);
    inOp.reductionStrides = red.map((i: number) => x.strides[i]);
    return new HipTensorIterator(x.shape.slice(), outShape, [HipTensorIterator.operand(out, out.strides, true), inOp],
                                 1, red, keepDims);
  }
}

// Device address, element strides over `shape` and dtype code of an iterator operand: the strides
// the dispatcher aligned (or, when an operand carries none, the handle's own broadcast to `shape`)
// and the element offset, checked to stay inside the operand's storage.
function operandGeometry(op: IteratorOperand, shape: readonly number[], isOutput: boolean, name: string):
    { ptr: bigint; strides: number[]; kh: number } {
  const h = op.tensorHandle;
  const dtype = (op.dtype || h.dtype) as DType;
  if (dtype !== h.dtype) throw new Error(`${name}: operand dtype ${dtype} differs from its handle's ${h.dtype}`);
  const offset = op.offset === undefined ? h.offset : op.offset;
  const strides = op.strides !== undefined && op.strides.length === shape.length ? op.strides.slice()
    : broadcastStrides(h.shape, h.strides, shape);
  if (isOutput) {
    for (let i = 0; i < shape.length; ++i)
      if (shape[i] > 1 && strides[i] === 0) throw new Error(`${name}: the output broadcasts axis ${i}`);
  }
  checkExtent(h.storage, shape, strides, offset, dtype, `${name} operand`);
  return { ptr: h.storage.ptr + BigInt(offset * ITEMSIZE[dtype]), strides, kh: DTYPE_CODE[dtype] };
}

function iteratorShape(iter: TensorIterator): number[] {
  return (iter.outputShape !== undefined ? iter.outputShape : iter.output(0).tensorHandle.shape).slice();
}

function scalarArgsOf(iter: TensorIterator): { [key: string]: any } {
  return iter.getScalarArgs !== undefined ? iter.getScalarArgs() : {};
}

// kh_map_strided op codes (include/kandle_hip.h)
const MAP = { copy: 0, add: 1, sub: 2, mul: 3, div: 4, neg: 5, cos: 6, sin: 7, silu: 8, fill: 9, arange: 10 };

// An iterator kernel over kh_map_strided (register.ts:9: (iter) => void, the output preallocated in
// iter.output().tensorHandle): `nin` inputs read through their strides, broadcast included, the
// output written through its own strides (a view for copy_, channels-last for contiguous).  s0/s1
// come from the op's scalar arguments: add/sub alpha (ops.ts:437; default 1), a fill value,
// arange's start and step (arangeExecutor.ts:37-44).
function mapKernel(name: string, op: number, nin: number,
                   scalars?: (sc: { [key: string]: any }) => number[]): KernelFn {
  return (iter: TensorIterator): void => {
    const shape = iteratorShape(iter);
    if (shape.length > 8) throw new Error(`${name}: at most 8 dimensions`);
    if (iter.numInputs < nin) throw new Error(`${name}: ${nin} inputs expected`);
    const o = operandGeometry(iter.output(0), shape, true, name);
    const a = nin >= 1 ? operandGeometry(iter.input(0), shape, false, name) : null;
    const b = nin >= 2 ? operandGeometry(iter.input(1), shape, false, name) : null;
    const sv = scalars === undefined ? [0, 0] : scalars(scalarArgsOf(iter));
    addon.mapStrided(op, shape, o.ptr, o.strides, o.kh, a === null ? null : a.ptr, a === null ? [] : a.strides,
                     a === null ? 0 : a.kh, b === null ? null : b.ptr, b === null ? [] : b.strides,
                     b === null ? 0 : b.kh, sv[0], sv[1]);
  };
}

function alphaOf(sc: { [key: string]: any }): number[] {
  return [sc.alpha === undefined ? 1 : Number(sc.alpha), 0];
}

// argmax(iter): a reduction iterator (reduction/index.ts:20-22; argShaderBuilder.ts:205-240) over
// iter.reductionAxes (the dispatcher's dim; all axes when it has none): the input is gathered into
// [kept, reduced] rows (one strided copy) and each row's maximum found with the lowest index among
// maxima (sampling/index.ts:132,138; NaN never wins); indices are stored as int32 (an int64 output
// included, as backend-webgpu stores it).
function argmaxKernel(iter: TensorIterator): void {
  const x = iter.input(0).tensorHandle;
  const nd = x.shape.length;
  let axes: number[];
  if (iter.reductionAxes !== undefined && iter.reductionAxes.length > 0) {
    axes = iter.reductionAxes.slice();
  } else {
    const dim = scalarArgsOf(iter).dim;
    axes = dim === undefined || dim === null ? x.shape.map((_: number, i: number) => i)
      : [Array.isArray(dim) ? dim[0] : (dim as number)];
  }
  axes = axes.map((a) => (a < 0 ? a + nd : a));
  for (const a of axes) if (!(a >= 0 && a < nd)) throw new Error(`argmax: axis out of range for a ${nd}-d tensor`);
  const kept = x.shape.map((_: number, i: number) => i).filter((i: number) => axes.indexOf(i) < 0);
  const perm = kept.concat(axes);
  if (perm.length > 8) throw new Error('argmax: at most 8 dimensions');
  const R = numelOf(axes.map((i) => x.shape[i]));
  const P = numelOf(kept.map((i) => x.shape[i]));
  if (R === 0) throw new Error('argmax: reduction over an empty axis');
  const out = iter.output(0);
  const dt = out.tensorHandle.dtype;
  if (dt !== 'int32' && dt !== 'int64') throw new Error('argmax: the output must be an integer tensor');
  const oshape = iteratorShape(iter);
  if (numelOf(oshape) !== P) throw new Error(`argmax: an output of [${oshape}] for ${P} rows`);
  // rows already contiguous in [kept, reduced] order (the last axes of a contiguous input) into a
  // contiguous output: one launch, no gather or copy
  const oh = out.tensorHandle;
  const trailing = axes.slice().sort((p, q) => p - q).every((a: number, i: number) => a === kept.length + i);
  if (trailing && x.isContiguous() && oh.isContiguous() && oh.numel === P &&
      (out.offset === undefined || out.offset === oh.offset)) {
    addon.argmax(x.ptr, P, R, oh.ptr, x.kh);
    return;
  }
  // the input's rows in [kept..., reduced...] order
  const pshape = perm.map((i) => x.shape[i]);
  const g = operandGeometry({ tensorHandle: x, strides: perm.map((i) => x.strides[i]), offset: x.offset }, pshape,
                            false, 'argmax');
  const rows = HipTensorHandle.createNew(pshape, x.dtype);
  addon.mapStrided(MAP.copy, pshape, rows.ptr, rows.strides, rows.kh, g.ptr, g.strides, g.kh, null, [], 0, 0, 0);
  const og = operandGeometry(out, oshape, true, 'argmax');
  const idx = HipTensorHandle.createNew(oshape, 'int32');
  addon.argmax(rows.ptr, P, R, idx.ptr, rows.kh);
  addon.mapStrided(MAP.copy, oshape, og.ptr, og.strides, og.kh, idx.ptr, idx.strides, idx.kh, null, [], 0, 0, 0);
  idx.dispose();
  rows.dispose();
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

const GEMV_PROLOGUE: { [name: string]: number } = { none: 0, rms_norm: 1, silu_mul: 2, silu_mul_interleaved: 3 };

// gemv_fused(prologue, x, w, out, params): one-row projection (decode) out[1, n] = alpha * x' W^T
// + beta * cin (+ bias) with the producer of x' fused in front: 'none' x' = x; 'rms_norm'
// x' = rms_norm(x, normWeight, eps) of the fp32 residual row; 'silu_mul' x' = silu(x) * x2;
// 'silu_mul_interleaved' the same product from one gate/up row interleaved in blocks of 8
// (RMSNorm.ts:92-99 or swiglu.ts:119-134 fused into Linear.ts:135-137).  params: actDtype (the
// activations' dtype: 'bfloat16', the default, rounds x' to bf16 and takes bf16 x / x2 for
// 'none' / 'silu_mul*'; 'float32' keeps x' in fp32 and takes float32 x / x2), normWeight, eps,
// x2, cin, bias, alpha, beta; out may alias cin (residual add).
function gemvFused(prologue: string, x: HipTensorHandle, w: HipTensorHandle, out: HipTensorHandle,
                   params?: { [key: string]: any }): void {
  const p = params || {};
  const code = GEMV_PROLOGUE[prologue];
  if (code === undefined) throw new Error(`gemv_fused: unknown prologue ${prologue}`);
  if (w.dtype !== 'bfloat16' || w.shape.length !== 2 || w.strides[1] !== 1)
    throw new Error('gemv_fused: the weight must be bf16 [n, k] with contiguous rows');
  const n = w.shape[0], k = w.shape[1];
  if (out.numel !== n || !out.isContiguous()) throw new Error('gemv_fused: out must be a contiguous row of n elements');
  const act = (p.actDtype || 'bfloat16') as DType;
  if (act !== 'bfloat16' && act !== 'float32') throw new Error('gemv_fused: actDtype must be bfloat16 or float32');
  const want = prologue === 'rms_norm' ? 'float32' : act;
  const kx = prologue === 'silu_mul_interleaved' ? 2 * k : k;
  const x2 = p.x2 as HipTensorHandle | undefined;
  for (const h of x2 === undefined ? [x] : [x, x2]) {
    if (h.dtype !== want || h.numel !== kx || !h.isContiguous())
      throw new Error(`gemv_fused: inputs must be contiguous ${want} rows of ${kx} elements`);
  }
  const nw = p.normWeight as HipTensorHandle | undefined;
  const cin = p.cin as HipTensorHandle | undefined;
  const bias = p.bias as HipTensorHandle | undefined;
  const beta = p.beta !== undefined ? (p.beta as number) : cin !== undefined ? 1 : 0;
  addon.gemvFused(code, x.ptr, x2 === undefined ? null : x2.ptr, nw === undefined ? null : nw.ptr,
                  p.eps === undefined ? 1e-6 : (p.eps as number), w.ptr, w.strides[0], out.ptr,
                  cin === undefined ? null : cin.ptr, bias === undefined ? null : bias.ptr, n, k,
                  p.alpha === undefined ? 1 : (p.alpha as number), beta, out.kh, DTYPE_CODE[act]);
}

// gemv_swiglu(prologue, x, wGu, out, params): one-row SwiGLU (decode): out[1, I] = silu(x' W_gate^T)
// * (x' W_up^T) from the gate/up weight interleaved in blocks of 8 rows; out's dtype is the
// activations' (bf16: x', gate and up rounded to bf16; float32: kept in fp32); prologue 'none'
// (x' = x, of out's dtype) or 'rms_norm' (x the fp32 residual row; params normWeight, eps).
function gemvSwiglu(prologue: string, x: HipTensorHandle, wGu: HipTensorHandle, out: HipTensorHandle,
                    params?: { [key: string]: any }): void {
  const p = params || {};
  if (prologue !== 'none' && prologue !== 'rms_norm') throw new Error(`gemv_swiglu: unknown prologue ${prologue}`);
  const k = wGu.shape[1], nHalf = wGu.shape[0] / 2;
  if (wGu.dtype !== 'bfloat16' || wGu.strides[1] !== 1) throw new Error('gemv_swiglu: bf16 weight with contiguous rows');
  if ((out.dtype !== 'bfloat16' && out.dtype !== 'float32') || out.numel !== nHalf || !out.isContiguous())
    throw new Error(`gemv_swiglu: out must be a contiguous bf16 or float32 row of ${nHalf} elements`);
  const want = prologue === 'rms_norm' ? 'float32' : out.dtype;
  if (x.dtype !== want || x.numel !== k || !x.isContiguous())
    throw new Error(`gemv_swiglu: x must be a contiguous ${want} row of ${k} elements`);
  const nw = p.normWeight as HipTensorHandle | undefined;
  addon.gemvSwiglu(GEMV_PROLOGUE[prologue], x.ptr, nw === undefined ? null : nw.ptr,
                   p.eps === undefined ? 1e-6 : (p.eps as number), wGu.ptr, wGu.strides[0], out.ptr, nHalf, k,
                   out.kh);
}

// linear_swiglu(x, wGu, output): output [.., I] = silu(x W_gate^T) * (x W_up^T) from the bf16
// gate/up weight [2I, H] interleaved in blocks of 8 rows (swiglu.ts:119-134 in one GEMM); x and
// output bf16 (gate, up and the product rounded to bf16) or float32 (kept in fp32).
function linearSwiglu(x: HipTensorHandle, wGu: HipTensorHandle, out: HipTensorHandle): void {
  const H = wGu.shape[1], I = wGu.shape[0] / 2;
  if ((x.dtype !== 'bfloat16' && x.dtype !== 'float32') || wGu.dtype !== 'bfloat16' || out.dtype !== x.dtype)
    throw new Error('linear_swiglu: a bf16 weight with bf16 or float32 x and output of x\'s dtype expected');
  if (x.shape[x.shape.length - 1] !== H || out.shape[out.shape.length - 1] !== I)
    throw new Error(`linear_swiglu: x [.., ${H}] and output [.., ${I}] expected`);
  if (!x.isContiguous() || !out.isContiguous() || wGu.strides[1] !== 1)
    throw new Error('linear_swiglu: contiguous operands expected');
  const m = x.numel / H;
  addon.gemmSwiglu(x.ptr, H, wGu.ptr, wGu.strides[0], out.ptr, I, m, I, H, x.kh);
}

// linear_qk_norm_rope(x, wQkv, params): the QKV projection of a chunk of S tokens with qk-norm, RoPE
// and the K/V cache write in its epilogue (gqa.ts:269-309, rope.ts:546-644, kv-cache.ts:164-212);
// x [S, H] bf16 or float32 (qOut and the caches of x's dtype), wQkv [(Hq + 2 Hkv) 128, H] bf16;
// params: qWeight, kWeight (bf16), invFreq, positions (int32 [S]),
// eps, qOut ([1, Hq, S, 128]), kOut / vOut (the caches [1, Hkv, maxSeq, 128], token t at row
// positions[t]).  The values of matmul followed by rms_norm_rope with cachePositions.
function linearQkNormRope(x: HipTensorHandle, wQkv: HipTensorHandle, p: { [key: string]: any }): void {
  const qOut: HipTensorHandle = p.qOut;
  const kOut: HipTensorHandle = p.kOut;
  const vOut: HipTensorHandle = p.vOut;
  const Hq = qOut.shape[1], S = qOut.shape[2], D = qOut.shape[3], Hkv = kOut.shape[1], L = kOut.shape[2];
  const H = wQkv.shape[1];
  if (D !== 128 || wQkv.shape[0] !== (Hq + 2 * Hkv) * D)
    throw new Error('linear_qk_norm_rope: head_dim 128 and wQkv [(Hq + 2 Hkv) D, H] expected');
  if (x.shape.join() !== [S, H].join() || x.strides[1] !== 1 || wQkv.strides[1] !== 1)
    throw new Error(`linear_qk_norm_rope: x [${S}, ${H}] with contiguous rows expected`);
  if (x.dtype !== 'bfloat16' && x.dtype !== 'float32') throw new Error('linear_qk_norm_rope: bf16 or float32 x expected');
  for (const t of [qOut, kOut, vOut]) {
    if (t.dtype !== x.dtype) throw new Error('linear_qk_norm_rope: qOut and the caches must have x\'s dtype');
  }
  if (wQkv.dtype !== 'bfloat16') throw new Error('linear_qk_norm_rope: the projection weight must be bf16');
  if (vOut.shape.join() !== kOut.shape.join()) throw new Error('linear_qk_norm_rope: K and V caches differ in shape');
  const st: number[] = [];
  for (const t of [qOut, kOut, vOut]) st.push(t.strides[0], t.strides[2], t.strides[1]);
  const tab = p.ropeTable as HipTensorHandle | undefined;
  if (tab !== undefined && (tab.dtype !== 'float32' || tab.numel !== S * D || !tab.isContiguous()))
    throw new Error('linear_qk_norm_rope: ropeTable must be rope_table(positions, invFreq): float32 [S, D/2, 2]');
  addon.gemmQkNormRopeTable(x.ptr, x.strides[0], wQkv.ptr, wQkv.strides[0], 1, S, H, Hq, Hkv, D, p.qWeight.ptr,
                            p.kWeight.ptr, p.invFreq.ptr, p.positions.ptr, qOut.ptr, kOut.ptr, vOut.ptr, st,
                            p.eps === undefined ? 1e-6 : p.eps, L, x.kh, tab === undefined ? null : tab.ptr);
}

// rope_table(positions, invFreq, output?): the RoPE angles of a chunk once per forward, [S, D/2, 2]
// float32 (cos, sin) of float(positions[t]) * invFreq[i] (rope.ts:193-255); linear_qk_norm_rope
// reads it (params.ropeTable) in every layer instead of evaluating the angles in each head tile.
function ropeTable(positions: HipTensorHandle, invFreq: HipTensorHandle, output?: HipTensorHandle): HipTensorHandle {
  if (positions.dtype !== 'int32' || !positions.isContiguous()) throw new Error('rope_table: contiguous int32 positions expected');
  if (invFreq.dtype !== 'float32' || !invFreq.isContiguous()) throw new Error('rope_table: contiguous float32 invFreq expected');
  const S = positions.numel, half = invFreq.numel;
  const out = output || HipTensorHandle.createNew([S, half, 2], 'float32');
  if (out.dtype !== 'float32' || out.numel !== S * half * 2 || !out.isContiguous())
    throw new Error('rope_table: output must be a contiguous float32 [S, D/2, 2] tensor');
  addon.ropeTable(positions.ptr, S, invFreq.ptr, half, out.ptr);
  return out;
}

// linear_add_rms_norm(x, w, residual, normWeight, eps, output, rows?): residual += x W^T (fp32, in
// place), then output = rms_norm(residual rows) * normWeight (decoder_layer.ts:224-238 with
// RMSNorm.ts:92-99).  When the GEMM splits K, its fp32 partials go straight into the fused
// add + RMSNorm kernel; the values are those of the separate launches bit for bit.
function linearAddRmsNorm(x: HipTensorHandle, w: HipTensorHandle, residual: HipTensorHandle,
                          normWeight: HipTensorHandle, eps: number, out: HipTensorHandle, rows?: number[]): void {
  const M = x.shape[0], K = x.shape[1], N = w.shape[0];
  const r0 = rows === undefined ? 0 : rows[0], r1 = rows === undefined ? M : rows[1];
  if ((x.dtype !== 'bfloat16' && x.dtype !== 'float32') || w.dtype !== 'bfloat16' || residual.dtype !== 'float32')
    throw new Error('linear_add_rms_norm: bf16 or float32 x and a bf16 w with an fp32 residual expected');
  if (w.shape[1] !== K || residual.shape.join() !== [M, N].join() || out.shape.join() !== [r1 - r0, N].join())
    throw new Error('linear_add_rms_norm: shapes do not match');
  if (normWeight.numel !== N || normWeight.dtype !== out.dtype)
    throw new Error('linear_add_rms_norm: normWeight must have N elements and the output dtype');
  if (!(r0 >= 0 && r0 < r1 && r1 <= M)) throw new Error('linear_add_rms_norm: bad row range');
  for (const h of [x, w, residual, out, normWeight])
    if (!h.isContiguous()) throw new Error('linear_add_rms_norm: contiguous operands expected');
  const splits = addon.gemmSplitCount(M, N, K) as number;
  const aligned = [x, w, residual, out, normWeight].every((h) => h.ptr % 16n === 0n);
  const rowOff = BigInt(r0 * N * 4);
  if (splits > 1 && aligned && N % 8 === 0 && N <= 2048) {
    const part = HipTensorHandle.createNew([splits, M, N], 'float32');
    addon.gemmSplitkPartials(x.ptr, K, w.ptr, K, part.ptr, M, N, K, splits, x.kh);
    addon.addRmsNorm(part.ptr + rowOff, splits, M * N, residual.ptr + rowOff, normWeight.ptr, out.ptr, r1 - r0, N,
                     eps, out.kh);
    part.dispose();  // stream ordered: reused only by later work on the same stream
    return;
  }
  addon.gemmEx(x.ptr, K, x.kh, w.ptr, K, w.kh, residual.ptr, N, residual.ptr, N, null, M, N, K, 1, 1, true,
               residual.kh);
  addon.rmsNorm(residual.ptr + rowOff, N, normWeight.ptr, out.ptr, N, r1 - r0, N, eps, residual.kh, out.kh);
}

// decode_attention_block(qkv, params): one decode step's attention block after the QKV projection
// of the new token (gqa.ts:246-430): qk-norm, RoPE at the device position, the K/V cache row write,
// attention over cache rows [0, position], o_proj and the residual add into x, in two kernels.
// params: qNorm, kNorm (bf16 [128]), invFreq (fp32 [64]), eps, position (int32 [1]), kCache,
// vCache ([1, Hkv, maxLen, 128] of qkv's dtype: bf16, or float32 activations), wO (bf16
// [hidden, Hq * 128]), x (fp32 [1, hidden]), scale.
function decodeAttentionBlock(qkv: HipTensorHandle, params: { [key: string]: any }): void {
  const kc = params.kCache as HipTensorHandle, vc = params.vCache as HipTensorHandle;
  const wo = params.wO as HipTensorHandle, x = params.x as HipTensorHandle;
  const hkv = kc.shape[1], maxLen = kc.shape[2], D = kc.shape[3];
  const hq = (qkv.numel - 2 * hkv * D) / D;
  if (D !== 128 || !(hq > 0) || hq !== Math.floor(hq))
    throw new Error(`decode_attention_block: qkv of ${qkv.numel} values does not split into heads of 128`);
  for (const h of [params.qNorm as HipTensorHandle, params.kNorm as HipTensorHandle, wo])
    if (h.dtype !== 'bfloat16') throw new Error('decode_attention_block: bf16 norm and projection weights expected');
  if (qkv.dtype !== 'bfloat16' && qkv.dtype !== 'float32') throw new Error('decode_attention_block: bf16 or float32 qkv');
  for (const h of [kc, vc])
    if (h.dtype !== qkv.dtype) throw new Error('decode_attention_block: the caches must have qkv\'s dtype');
  if (!qkv.isContiguous() || x.dtype !== 'float32' || !x.isContiguous())
    throw new Error('decode_attention_block: qkv and x (fp32) must be contiguous');
  if (wo.shape.join() !== [x.numel, hq * D].join() || wo.strides[1] !== 1)
    throw new Error(`decode_attention_block: wO must be [${x.numel}, ${hq * D}] with contiguous rows`);
  const pos = params.position as HipTensorHandle;
  if (pos.dtype !== 'int32') throw new Error('decode_attention_block: position must be int32');
  addon.decodeAttentionBlock(qkv.ptr, (params.qNorm as HipTensorHandle).ptr, (params.kNorm as HipTensorHandle).ptr,
                             (params.invFreq as HipTensorHandle).ptr, params.eps === undefined ? 1e-6 : params.eps,
                             pos.ptr, kc.ptr, vc.ptr, hq, hkv, maxLen,
                             [kc.strides[1], kc.strides[2], vc.strides[1], vc.strides[2]], params.scale as number,
                             wo.ptr, wo.strides[0], x.numel, x.ptr, qkv.kh);
}

// greedy_advance(nextToken, position, seqLen, tokenLog, logBase): the device-side step of the greedy
// loop (for_causal_lm.ts:475-508): tokenLog[p + 1 - logBase] = nextToken, position = p + 1,
// seqLen = p + 2, with p = position[0].  int32 operands.
function greedyAdvance(nextToken: HipTensorHandle, position: HipTensorHandle, seqLen: HipTensorHandle,
                       tokenLog: HipTensorHandle, logBase: number): void {
  for (const h of [nextToken, position, seqLen, tokenLog])
    if (h.dtype !== 'int32' || !h.isContiguous()) throw new Error('greedy_advance: contiguous int32 operands expected');
  addon.greedyAdvance(nextToken.ptr, position.ptr, seqLen.ptr, tokenLog.ptr, logBase, tokenLog.numel);
}

// sample(logits, params): one token from a float32 logits row on the device (sampling/index.ts:
// 103-243).  params: doSample (true), temperature (1), topK (0 = off), topP (1 = off), seed, counter
// (int32 [1]: r = philox4x32-10(seed, counter)), displayK (0), and the outputs token (int32 [1]),
// logprob (float32 [1]), displayIds (int32 [displayK]) and displayProbs (float32 [displayK]).
function sample(logits: HipTensorHandle, params: { [key: string]: any }): void {
  if (logits.dtype !== 'float32' || !logits.isContiguous())
    throw new Error('sample: logits must be a contiguous float32 tensor');
  const vocab = logits.shape[logits.shape.length - 1];
  if (logits.numel !== vocab) throw new Error('sample: one row of logits expected');
  const opt = (name: string): HipTensorHandle | undefined => params[name] as HipTensorHandle | undefined;
  const ptrOf = (h: HipTensorHandle | undefined): bigint | null => (h === undefined ? null : h.ptr);
  const doSample = params.doSample === undefined ? true : !!params.doSample;
  const token = opt('token');
  if (token === undefined || token.dtype !== 'int32') throw new Error('sample: token must be an int32 tensor');
  if (doSample && (opt('counter') === undefined || (opt('counter') as HipTensorHandle).dtype !== 'int32'))
    throw new Error('sample: counter must be an int32 tensor');
  addon.sample(logits.ptr, vocab, doSample, params.temperature === undefined ? 1 : params.temperature,
               params.topK || 0, params.topP === undefined ? 1 : params.topP, BigInt(params.seed || 0),
               ptrOf(opt('counter')), token.ptr, ptrOf(opt('logprob')), params.displayK || 0,
               ptrOf(opt('displayIds')), ptrOf(opt('displayProbs')));
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

  // HIP graphs of library launches: between graphBegin() and graphEnd() kernels are recorded instead
  // of run (allocations made meanwhile belong to the graph until graphDestroy); graphLaunch replays.
  graphBegin(): void {
    addon.graphBeginCapture();
  }

  graphEnd(): bigint {
    return addon.graphEndCapture() as bigint;
  }

  graphLaunch(graph: bigint): void {
    addon.graphLaunch(graph);
  }

  graphDestroy(graph: bigint): void {
    addon.graphDestroy(graph);
  }

  // The K split matmul (kh_gemm) uses for a contiguous bf16 [m, k] x [n, k]^T product (1: none).
  gemmSplitCount(m: number, n: number, k: number): number {
    return addon.gemmSplitCount(m, n, k);
  }

  memoryStats(): { [key: string]: number } {
    return addon.allocStats();
  }
}

export function registerHipKernels(reg: SimpleOperatorRegistry): void {
  reg.register('flash_attention', flashAttention);
  reg.register('flash_attention_split', flashAttentionSplit);
  reg.register('sdpa_masked', sdpaMasked);
  reg.register('rms_norm', rmsNorm);
  for (const name of ['matmul', 'mm', 'bmm', 'addmm', 'baddbmm']) reg.register(name, matmul);
  // Iterator kernels, (iter: ITensorIterator) => void with broadcast / strided operands
  // (register.ts:9; pointwise ops.ts:168-437, copy/index.ts:13-33, factory/index.ts:27-29,
  // reduction/index.ts:20-22): the output is iter.output().tensorHandle.
  reg.register('add', mapKernel('add', MAP.add, 2, alphaOf));
  reg.register('sub', mapKernel('sub', MAP.sub, 2, alphaOf));
  reg.register('mul', mapKernel('mul', MAP.mul, 2));
  reg.register('div', mapKernel('div', MAP.div, 2));
  for (const name of ['neg', 'cos', 'sin', 'silu']) reg.register(name, mapKernel(name, (MAP as any)[name], 1));
  for (const name of ['copy', 'cast', 'contiguous', 'clone', 'copy_']) reg.register(name, mapKernel(name, MAP.copy, 1));
  reg.register('zeros', mapKernel('zeros', MAP.fill, 0, () => [0, 0]));
  reg.register('ones', mapKernel('ones', MAP.fill, 0, () => [1, 0]));
  reg.register('full', mapKernel('full', MAP.fill, 0, (sc: { [key: string]: any }) =>
    [Number(sc.fill_value !== undefined ? sc.fill_value : sc.fillValue), 0]));
  reg.register('empty', (_iter: TensorIterator): void => undefined);
  reg.register('arange', mapKernel('arange', MAP.arange, 0, (sc: { [key: string]: any }) =>
    [sc.start === undefined ? 0 : Number(sc.start), sc.step === undefined ? 1 : Number(sc.step)]));
  reg.register('argmax', argmaxKernel);
  reg.register('decode_attention', decodeAttention);
  reg.register('rms_norm_rope', rmsNormRope);
  reg.register('silu_mul', siluMul);
  reg.register('index_select', indexSelect);
  reg.register('gemv_fused', gemvFused);
  reg.register('gemv_swiglu', gemvSwiglu);
  reg.register('linear_swiglu', linearSwiglu);
  reg.register('linear_qk_norm_rope', linearQkNormRope);
  reg.register('rope_table', ropeTable);
  reg.register('linear_add_rms_norm', linearAddRmsNorm);
  reg.register('decode_attention_block', decodeAttentionBlock);
  reg.register('greedy_advance', greedyAdvance);
  reg.register('sample', sample);
}

export { contiguousStrides, toBf16Bits, fromBf16Bits };
