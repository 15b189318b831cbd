// Loads the N-API addon with Node and exercises what runs without a GPU:
// the exports, the error shape, checkExpertWeight's messages (the cases of
// the reference's test/core/graph/ops/matmul.test.ts:276-409) and a
// context refused when no device is visible. Prints one JSON object.
import { createRequire } from 'module';

const require = createRequire(import.meta.url);
const addon = require(process.argv[2]);
const res = { exports: Object.keys(addon).sort(), version: addon.version(), checks: [] };

function caught(fn) {
  try {
    return { ok: true, value: fn() };
  } catch (e) {
    return { ok: false, name: e.name, code: e.code, message: e.message };
  }
}

res.ctxCreate = caught(() => String(addon.ctxCreate(0, null)));
res.nullCtxUp = caught(() => addon.moeUp(0n, 0n, 0, 0n, 0n, 0n, 0n, 0n, 0n, 0n, 1, 8, 8, 2, 4, 8, 8, 0n));
res.badPointer = caught(() => addon.sync('not a pointer'));

// One routed layer of 2 experts of [K=8, N=16] (matmul.test.ts:283-287).
const quant = (r, c, bits = 8) => ({ elems: (r * c * bits) / 32, dtype: 'quantW', dims: [r, c] });
const f32 = (dims) => ({ elems: dims.reduce((a, b) => a * b, 1), dtype: 'f32', dims });
const base = { w: quant(16, 16), scales: f32([4, 16]), bias: f32([2, 16]), route: f32([3, 8]), bits: 8, g: 4 };
const cases = [
  ['good', {}],
  ['bits', { bits: 5 }],
  ['w not quantW', { w: f32([16, 16]) }],
  ['w rows', { w: quant(12, 16) }],
  ['elems', { w: { elems: 32, dtype: 'quantW', dims: [16, 16] } }],
  ['K N multiple of 4', { w: quant(16, 6), scales: f32([4, 6]), bias: f32([2, 6]) }],
  ['groupSize', { g: 3 }],
  ['scales', { scales: f32([2, 16]) }],
  ['bias', { bias: f32([16]) }],
  ['route', { route: f32([3, 3]) }],
];
for (const [name, over] of cases) {
  const c = Object.assign({}, base, over);
  res.checks.push([name, caught(() => addon.checkExpertWeight('moeUp', c.w, c.scales, c.bias, c.route, 8, 3, 4, c.bits, c.g))]);
}
// Malformed ValueMeta and integers past int64 are refused before any shape
// check runs.
res.malformed = [
  ['rank 5', caught(() => addon.checkExpertWeight('moeUp', { elems: 64, dtype: 'quantW', dims: [16, 16, 1, 1, 1] }, base.scales, base.bias, base.route, 8, 3, 4, 8, 4))],
  ['fractional dim', caught(() => addon.checkExpertWeight('moeUp', { elems: 64, dtype: 'quantW', dims: [16.5, 16] }, base.scales, base.bias, base.route, 8, 3, 4, 8, 4))],
  ['string elems', caught(() => addon.checkExpertWeight('moeUp', { elems: '64', dtype: 'quantW', dims: [16, 16] }, base.scales, base.bias, base.route, 8, 3, 4, 8, 4))],
  ['int64 overflow', caught(() => addon.checkExpertWeight('moeUp', base.w, base.scales, base.bias, base.route, 2n ** 70n, 3, 4, 8, 4))],
];
console.log(JSON.stringify(res));
