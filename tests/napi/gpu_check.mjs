// Runs the reference's op chain of one routed MoE layer — the router's f32
// matmul, topk, moeUp, moeDown (src/zoo/privacy-filter/moeMlp.ts:82-117) —
// through the type-stripped HipExecutor (runntime_amd/napi/hipExecutor.ts)
// and the real N-API addon on the GPU. Inputs are raw little-endian files
// written by the Python test (meta.json gives the sizes); the logits, the
// route, act and the output are written back the same way for it to check.
// Nodes are shaped like the reference's pending records (op, inputs, scalar,
// attrs; src/core/graph/value.ts:186-196) in their op builders' operand
// order (ops/matmul.ts:86-96, :236-242, :265-270; ops/reduce.ts:95-100).
import { createRequire } from 'module';
import fs from 'fs';
import path from 'path';

const require = createRequire(import.meta.url);
const [execPath, addonPath, dir] = process.argv.slice(2);
const addon = require(addonPath);
const m = JSON.parse(fs.readFileSync(path.join(dir, 'meta.json'), 'utf8'));
const { T, d, E, k, I } = m;

const load = (name, Ctor) => {
  const b = fs.readFileSync(path.join(dir, name));
  return new Ctor(b.buffer.slice(b.byteOffset, b.byteOffset + b.byteLength));
};
const meta = (dtype, dims) => ({ elems: dims.reduce((a, b) => a * b, 1), dtype, dims });
const quant = (rows, cols) => ({ elems: (rows * cols) / 4, dtype: 'quantW', dims: [rows, cols] });
const leaf = (shape) => ({ shape, pending: undefined });
const node = (shape, op, inputs, scalar, attrs) => ({ shape, pending: { op, inputs, scalar, attrs } });

(async () => {
  const { HipExecutor } = await import(execPath);
  const ex = new HipExecutor(addon, 0);
  const v = {
    x: [meta('f32', [T, d]), load('x.bin', Float32Array)],
    rw: [meta('f32', [d, E]), load('rw.bin', Float32Array)],
    gw: [quant(E * d, I), load('gw.bin', Uint32Array)],
    gs: [meta('f32', [E, I]), load('gs.bin', Float32Array)],
    lw: [quant(E * d, I), load('lw.bin', Uint32Array)],
    ls: [meta('f32', [E, I]), load('ls.bin', Float32Array)],
    bcat: [meta('f32', [2 * E, I]), load('bcat.bin', Float32Array)],
    dw: [quant(E * I, d), load('dw.bin', Uint32Array)],
    ds: [meta('f32', [E, d]), load('ds.bin', Float32Array)],
    db: [meta('f32', [E, d]), load('db.bin', Float32Array)],
    res: [meta('f32', [T, d]), load('res.bin', Float32Array)],
  };
  const buf = {}, val = {};
  for (const [name, [shape, data]] of Object.entries(v)) {
    buf[name] = ex.upload(data, shape);
    val[name] = leaf(shape);
  }
  const run = (n, inputs) => {
    const out = ex.acquireOutput(n.shape);
    ex.dispatch(n, inputs, out);
    return out;
  };
  const logitsN = node(meta('f32', [T, E]), 'matmul', [val.x, val.rw], undefined, [0, 0, 0, 0, 0]);
  const logits = run(logitsN, [buf.x, buf.rw]);
  const routeN = node(meta('f32', [T, 2 * k]), 'topk', [leaf(logitsN.shape)]);
  const route = run(routeN, [logits]);
  const actN = node(meta('f32', [T * k, I]), 'moeUp',
    [val.x, leaf(routeN.shape), val.gw, val.gs, val.lw, val.ls, val.bcat], undefined, [8, d, E]);
  const act = run(actN, [buf.x, route, buf.gw, buf.gs, buf.lw, buf.ls, buf.bcat]);
  const outN = node(meta('f32', [T, d]), 'moeDown',
    [leaf(actN.shape), leaf(routeN.shape), val.dw, val.ds, val.db, val.res], undefined, [8, I, E]);
  const out = run(outN, [act, route, buf.dw, buf.ds, buf.db, buf.res]);
  ex.submit();
  for (const [name, b, shape] of [['logits', logits, logitsN.shape], ['route', route, routeN.shape],
    ['act', act, actN.shape], ['out', out, outN.shape]]) {
    const host = await ex.readback(b, shape);
    fs.writeFileSync(path.join(dir, `${name}.out`), Buffer.from(host.buffer));
  }
  ex.dispose();
  console.log(JSON.stringify({ ok: true }));
})().catch((e) => { console.log(JSON.stringify({ fatal: e.message, stack: e.stack })); process.exit(1); });
