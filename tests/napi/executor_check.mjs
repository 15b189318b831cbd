// Runs the type-stripped HipExecutor (runntime_amd/napi/hipExecutor.ts)
// against a recording mock of the addon and prints, per dispatched node,
// the addon call it made. Nodes are shaped like the reference's pending
// records (op, inputs, scalar, attrs; src/core/graph/value.ts:186-196) in
// the operand order of their op builders.
const execPath = process.argv[2];

const calls = [];
const mock = {
  version: () => 1,
  ctxCreate: (device, stream) => { calls.push(['ctxCreate', device, stream]); return 7n; },
  ctxDestroy: (ctx) => calls.push(['ctxDestroy', ctx]),
  sync: (ctx) => calls.push(['sync', ctx]),
  bufferAlloc: (ctx, bytes) => { calls.push(['bufferAlloc', ctx, bytes]); return 4096n * BigInt(calls.length); },
  bufferFree: (ctx, ptr) => calls.push(['bufferFree', ctx, ptr]),
  bufferWrite: (ctx, dst, host) => calls.push(['bufferWrite', ctx, dst, host.byteLength]),
  bufferRead: (ctx, src, host) => { calls.push(['bufferRead', ctx, src, host.byteLength]); if (host instanceof Uint16Array) host.set([0x3c00, 0xc000, 0x0001]); else host.fill(1.5); },
};
for (const name of ['topk', 'moeUp', 'moeDown', 'rmsNorm', 'linear']) mock[name] = (...args) => calls.push([name, ...args]);

const meta = (dtype, dims) => ({ elems: dims.reduce((a, b) => a * b, 1), dtype, dims });
const leaf = (shape) => ({ shape, pending: undefined });
const node = (shape, op, inputs, scalar, attrs) => ({ shape, pending: { op, inputs, scalar, attrs } });
const buf = (ptr) => ({ ptr: BigInt(ptr), bytes: 0 });

(async () => {
  const { HipExecutor } = await import(execPath);
  const ex = new HipExecutor(mock, 0);
  const out = [];
  const record = (label, fn) => {
    const before = calls.length;
    try {
      fn();
      out.push([label, calls.slice(before).map((c) => c.map((x) => (typeof x === 'bigint' ? `${x}n` : x)))]);
    } catch (e) {
      out.push([label, { error: e.message }]);
    }
  };
  // T = 3 tokens, K = 8, N = 16, E = 2 experts, 4 slots, int8, groupSize 8.
  const x = leaf(meta('f32', [3, 8])), route = leaf(meta('f32', [3, 8]));
  const w = leaf(meta('quantW', [16, 16])), sc = leaf(meta('f32', [2, 16]));
  const bcat = leaf(meta('f32', [4, 16]));
  record('moeUp', () => ex.dispatch(
    node(meta('f32', [12, 16]), 'moeUp', [x, route, w, sc, w, sc, bcat], undefined, [8, 8, 2]),
    [100, 200, 300, 400, 500, 600, 700].map(buf), buf(900)));
  const act = leaf(meta('f32', [12, 16])), dw = leaf(meta('quantW', [32, 8]));
  const dsc = leaf(meta('f32', [2, 8])), db = leaf(meta('f32', [2, 8])), res = leaf(meta('f32', [3, 8]));
  record('moeDown', () => ex.dispatch(
    node(meta('f32', [3, 8]), 'moeDown', [act, route, dw, dsc, db, res], undefined, [8, 16, 2]),
    [110, 210, 310, 410, 510, 610].map(buf), buf(910)));
  record('topk', () => ex.dispatch(node(meta('f32', [3, 8]), 'topk', [leaf(meta('f16', [3, 32]))]),
    [buf(120)], buf(920)));
  record('rmsNorm', () => ex.dispatch(
    node(meta('f32', [3, 8]), 'rmsNorm', [x, leaf(meta('f32', [8])), res], 1e-5, [8, 1]),
    [130, 230, 330].map(buf), buf(930)));
  record('matmul', () => ex.dispatch(
    node(meta('f32', [3, 2]), 'matmul', [x, leaf(meta('f32', [8, 2])), leaf(meta('f32', [2]))], undefined, [1, 0, 0, 0, 0]),
    [140, 240, 340].map(buf), buf(940)));
  record('add', () => ex.dispatch(node(meta('f32', [3, 8]), 'add', [x, x]), [buf(1), buf(2)], buf(3)));
  record('pool', () => {
    const a = ex.acquireOutput(meta('f32', [3, 8]));
    ex.releaseOutput(a, meta('f32', [3, 8]));
    const b = ex.acquireOutput(meta('f32', [3, 8]));
    if (a !== b) throw new Error('released buffer not reused');
  });
  const f16 = await ex.readback(buf(5), meta('f16', [3]));
  out.push(['readback f16', Array.from(f16)]);
  console.log(JSON.stringify(out));
})().catch((e) => { console.log(JSON.stringify({ fatal: e.message })); process.exit(1); });
