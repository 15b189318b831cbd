/**
 * A ruNNtime Executor whose kernels are this repository's HIP library,
 * reached through the N-API addon next to this file (runntime_moe.node).
 *
 * It implements the reference's executor contract — Executor and Readback,
 * packages/runntime/src/core/graph/evalCore.ts:14-43 — for the ops of the
 * MoE path: topk, moeUp, moeDown (src/core/graph/ops/reduce.ts:93-100,
 * ops/matmul.ts:220-272), rmsNorm (ops/reduce.ts:61-92) and the router's
 * f32 matmul (ops/matmul.ts:35-97; nn.Linear → linear(), graph/
 * compose.ts:45-53). Each dispatch reads the node's `pending` record in the
 * operand order its op builder wrote it and makes one C-ABI call:
 *
 *   moeUp   inputs [x, route, glu.w, glu.scales, lin.w, lin.scales,
 *                   cat([glu.bias, lin.bias])], attrs [bits, groupSize,
 *                   experts] (ops/matmul.ts:236-242)
 *   moeDown inputs [act, route, w, scales, bias, residual], attrs [bits,
 *                   groupSize, experts] (ops/matmul.ts:265-270)
 *   topk    inputs [x]; k = out cols / 2 (ops/reduce.ts:95-100)
 *   rmsNorm inputs [x, weight, residual?], scalar eps, attrs [group, scale]
 *   matmul  inputs [a, b, bias?, addend?], attrs [hasBias, hasAddend, act,
 *                   baseRow, baseRowSet] (f32, no activation, baseRow 0)
 *
 * Any other op throws: the rest of a graph stays on the reference's WebGPU
 * executor. Device buffers are plain HIP allocations held as BigInt
 * pointers; the op builders' checks (checkExpertWeight and the rest) have
 * run before dispatch, and the library re-checks what pointers allow.
 *
 * Written in erasable TypeScript (types only: no enums, namespaces or
 * parameter properties), so Node ≥ 22 loads it by stripping the types.
 * Place it at packages/runntime/src/core/gpu/hip/hipExecutor.ts; the type
 * imports below are relative to that place.
 */
import type { DispatchExtras, Executor, Readback } from '../../graph/evalCore.ts';
import type { GpuBufferRef, Value, ValueMeta } from '../../graph/value.ts';

/** The addon's functions this executor calls (runntime_moe_addon.cc). */
export interface RunntimeMoeAddon {
  version(): number;
  ctxCreate(device: number, stream?: bigint | null): bigint;
  ctxDestroy(ctx: bigint): void;
  sync(ctx: bigint): void;
  bufferAlloc(ctx: bigint, bytes: number): bigint;
  bufferFree(ctx: bigint, ptr: bigint): void;
  bufferWrite(ctx: bigint, dst: bigint, host: ArrayBufferView | ArrayBuffer): void;
  bufferRead(ctx: bigint, src: bigint, host: ArrayBufferView | ArrayBuffer): void;
  topk(ctx: bigint, logits: bigint, dtype: number, t: number, e: number, k: number,
    route: bigint): void;
  moeUp(ctx: bigint, x: bigint, dtype: number, route: bigint, gluW: bigint, gluScales: bigint,
    gluBias: bigint, linW: bigint, linScales: bigint, linBias: bigint, t: number, k: number,
    n: number, experts: number, slots: number, bits: number, groupSize: number,
    act: bigint): void;
  moeDown(ctx: bigint, act: bigint, route: bigint, w: bigint, scales: bigint, bias: bigint,
    residual: bigint, t: number, k: number, n: number, experts: number, slots: number,
    bits: number, groupSize: number, out: bigint): void;
  rmsNorm(ctx: bigint, x: bigint, dtype: number, rows: number, cols: number, weight: bigint,
    weightLen: number, eps: number, group: number, residual: bigint, scale: number,
    out: bigint): void;
  linear(ctx: bigint, x: bigint, w: bigint, bias: bigint, addend: bigint, t: number, k: number,
    n: number, out: bigint): void;
}

/** What a GpuBufferRef is on this backend: a device allocation. */
export interface HipBuffer {
  readonly ptr: bigint;
  readonly bytes: number;
}

const F32 = 0;
const F16 = 1;

function dtypeCode(shape: ValueMeta): number {
  if (shape.dtype === 'f32') return F32;
  if (shape.dtype === 'f16') return F16;
  throw new Error(`HipExecutor: a ${shape.dtype} value is not a float tensor`);
}

/** Bytes of a value: 2 per f16 element, 4 per f32 element or quantW word
 *  (elemBytes, src/core/graph/value.ts:9-13). */
function valueBytes(shape: ValueMeta): number {
  return shape.elems * (shape.dtype === 'f16' ? 2 : 4);
}

/** A HipBuffer record. */
function hipBuffer(ptr: bigint, bytes: number): HipBuffer {
  return { ptr, bytes };
}

function dims2(shape: ValueMeta, what: string): readonly number[] {
  const d = shape.dims;
  if (!d || d.length !== 2) throw new Error(`HipExecutor: ${what} must be 2D`);
  return d;
}

/** f16 bits → f32 (readback of an f16 value as the reference returns it,
 *  a Float32Array). */
function halfToFloat(h: number): number {
  const s = h & 0x8000 ? -1 : 1;
  const e = (h >> 10) & 0x1f;
  const m = h & 0x3ff;
  if (e === 0) return s * m * 2 ** -24;
  if (e === 31) return m ? NaN : s * Infinity;
  return s * (1 + m / 1024) * 2 ** (e - 15);
}

export class HipExecutor implements Executor, Readback {
  readonly #addon: RunntimeMoeAddon;
  readonly #ctx: bigint;
  // Released outputs by byte size, handed out again (the reference's
  // BufferPool, src/core/gpu/bufferPool.ts:1-25).
  readonly #free: Map<number, HipBuffer[]> = new Map();

  constructor(addon: RunntimeMoeAddon, device = 0) {
    if (addon.version() !== 1) throw new Error(`HipExecutor: addon version ${addon.version()}`);
    this.#addon = addon;
    this.#ctx = addon.ctxCreate(device, null);
  }

  /** The library context (for direct calls such as moeLayer). */
  get context(): bigint {
    return this.#ctx;
  }

  acquireOutput(shape: ValueMeta): GpuBufferRef {
    const bytes = valueBytes(shape);
    const list = this.#free.get(bytes);
    const buf: HipBuffer = list !== undefined && list.length > 0
      ? list.pop() as HipBuffer
      : hipBuffer(this.#addon.bufferAlloc(this.#ctx, bytes), bytes);
    return buf as unknown as GpuBufferRef;
  }

  releaseOutput(buffer: GpuBufferRef, _shape: ValueMeta): void {
    const b = buffer as unknown as HipBuffer;
    const list = this.#free.get(b.bytes);
    if (list) list.push(b);
    else this.#free.set(b.bytes, [b]);
  }

  /** A host array as a device value (the reference's upload()). */
  upload(data: ArrayBufferView, shape: ValueMeta): GpuBufferRef {
    const out = this.acquireOutput(shape);
    this.#addon.bufferWrite(this.#ctx, (out as unknown as HipBuffer).ptr, data);
    return out;
  }

  dispatch(node: Value, inputs: readonly GpuBufferRef[], out: GpuBufferRef,
    extras?: DispatchExtras): void {
    const pend = node.pending;
    if (!pend) throw new Error('HipExecutor: dispatch of a materialized value');
    if (extras && (extras.addend || extras.outBase || extras.outElems)) {
      throw new Error(`HipExecutor: '${pend.op}' with fused extras is not supported`);
    }
    const a = this.#addon;
    const ctx = this.#ctx;
    const p = (i: number): bigint => (inputs[i] as unknown as HipBuffer).ptr;
    const o = (out as unknown as HipBuffer).ptr;
    const attrs: readonly number[] = pend.attrs === undefined ? [] : pend.attrs;
    switch (pend.op) {
      case 'topk': {
        const [m, n] = dims2(pend.inputs[0]!.shape, 'topk input');
        const k = dims2(node.shape, 'topk output')[1]! / 2;
        a.topk(ctx, p(0), dtypeCode(pend.inputs[0]!.shape), m!, n!, k, o);
        return;
      }
      case 'moeUp': {
        const [bits, groupSize, experts] = attrs;
        const [t, k] = dims2(pend.inputs[0]!.shape, 'moeUp x');
        const n = dims2(pend.inputs[2]!.shape, 'moeUp glu.w')[1]!;
        const slots = dims2(pend.inputs[1]!.shape, 'moeUp route')[1]! / 2;
        // the concatenated bias [2E, N]: glu rows, then lin rows
        const linBias = p(6) + BigInt(experts! * n * 4);
        a.moeUp(ctx, p(0), dtypeCode(pend.inputs[0]!.shape), p(1), p(2), p(3), p(6), p(4), p(5),
          linBias, t!, k!, n, experts!, slots, bits!, groupSize!, o);
        return;
      }
      case 'moeDown': {
        const [bits, groupSize, experts] = attrs;
        const [rows, k] = dims2(pend.inputs[0]!.shape, 'moeDown act');
        const slots = dims2(pend.inputs[1]!.shape, 'moeDown route')[1]! / 2;
        const n = dims2(pend.inputs[2]!.shape, 'moeDown w')[1]!;
        a.moeDown(ctx, p(0), p(1), p(2), p(3), p(4), p(5), rows! / slots, k!, n, experts!, slots,
          bits!, groupSize!, o);
        return;
      }
      case 'rmsNorm': {
        const [group, scale] = attrs;
        const [m, n] = dims2(pend.inputs[0]!.shape, 'rmsNorm x');
        const residual = pend.inputs.length > 2 ? p(2) : 0n;
        a.rmsNorm(ctx, p(0), dtypeCode(pend.inputs[0]!.shape), m!, n!, p(1),
          pend.inputs[1]!.shape.elems, pend.scalar!, group!, residual, scale!, o);
        return;
      }
      case 'matmul': {
        const [hasBias, hasAddend, act, baseRow] = attrs;
        if (pend.inputs[0]!.shape.dtype !== 'f32' || act || baseRow) {
          throw new Error('HipExecutor: matmul is f32 without activation or baseRow here');
        }
        const [m, k] = dims2(pend.inputs[0]!.shape, 'matmul a');
        const n = dims2(pend.inputs[1]!.shape, 'matmul b')[1]!;
        const bias = hasBias ? p(2) : 0n;
        const addend = hasAddend ? p(hasBias ? 3 : 2) : 0n;
        a.linear(ctx, p(0), p(1), bias, addend, m!, k!, n, o);
        return;
      }
      default:
        throw new Error(`HipExecutor: op '${pend.op}' is not on the MoE path`);
    }
  }

  submit(): void {
    // Kernels are enqueued as dispatched; nothing is batched here.
  }

  async readback(buffer: GpuBufferRef, shape: ValueMeta): Promise<Float32Array> {
    const b = buffer as unknown as HipBuffer;
    this.#addon.sync(this.#ctx);
    if (shape.dtype === 'f16') {
      const raw = new Uint16Array(shape.elems);
      this.#addon.bufferRead(this.#ctx, b.ptr, raw);
      return Float32Array.from(raw, halfToFloat);
    }
    const out = new Float32Array(shape.elems);
    this.#addon.bufferRead(this.#ctx, b.ptr, out);
    return out;
  }

  /** Frees every pooled buffer and the context. */
  dispose(): void {
    for (const list of this.#free.values()) {
      for (const b of list) this.#addon.bufferFree(this.#ctx, b.ptr);
    }
    this.#free.clear();
    this.#addon.ctxDestroy(this.#ctx);
  }
}
