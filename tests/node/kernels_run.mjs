// Drives the addon's buffer and launcher bindings (one per C-ABI entry point) on inputs the
// pytest wrapper wrote into <dir> (raw little-endian .bin files, shapes in spec.json), and
// writes each result back as <name>.out.bin for the wrapper to check against the oracle.
import { createRequire } from 'module';
import fs from 'fs';
import path from 'path';

const require = createRequire(import.meta.url);
const a = require('../../webgpu_amd/node/wgd_napi.node');
const dir = process.argv[2];
const spec = JSON.parse(fs.readFileSync(path.join(dir, 'spec.json'), 'utf8'));

const bytesOf = (name) => new Uint8Array(fs.readFileSync(path.join(dir, name + '.bin')));
const f32 = (name) => { const b = bytesOf(name); return new Float32Array(b.buffer, b.byteOffset, b.byteLength / 4); };
const i32 = (name) => { const b = bytesOf(name); return new Int32Array(b.buffer, b.byteOffset, b.byteLength / 4); };
const save = (name, arr) => fs.writeFileSync(path.join(dir, name + '.out.bin'), Buffer.from(arr.buffer, arr.byteOffset, arr.byteLength));

const ctx = a.create(0, null);
const errors = {};
try {
  const up = (arr, label) => { const b = a.bufferCreate(ctx, arr.byteLength, label); a.write(ctx, b, 0, arr); return b; };
  const out = (floats, label) => a.bufferCreate(ctx, floats * 4, label);
  const get = (buf, floats) => a.read(ctx, buf, 0, new Float32Array(floats));

  // weights: the GGUF bytes (generic kernels) and the planar upload (fast kernels)
  const { type, cols, rows, batch } = spec.matmul;
  const wBytes = bytesOf('w');
  const wRaw = up(wBytes, 'w raw');
  const wPlanar = a.uploadWeights(ctx, type, cols, rows, wBytes, 'w planar');
  const x = up(f32('x'), 'x');
  const stride = rows + 3, base = 2;
  const y = out(stride * batch, 'y');
  a.clear(ctx, y);
  a.matmul(ctx, type, wPlanar, x, y, cols, rows, stride, base, 1, batch);   // prompt GEMM, input offset 1
  save('gemm', get(y, stride * batch));
  const y1 = out(rows, 'y1');
  a.matmul(ctx, type, wRaw, x, y1, cols, rows, rows, 0, 0, 1);              // GGUF-layout matvec
  save('matvec_raw', get(y1, rows));
  const qx = a.bufferCreate(ctx, a.quantizedBytes(cols), 'qx');
  const nw = up(f32('nw'), 'norm weight');
  a.quantize(ctx, x, cols, nw, spec.eps, qx);                              // RMSNorm(x row 0) * nw, quantized
  const y2 = out(rows, 'y2');
  a.matvec(ctx, type, wPlanar, qx, y2, cols, rows, 0);
  save('matvec_normed', get(y2, rows));
  const deq = out(cols * rows, 'deq');
  a.dequant(ctx, type, wRaw, deq, cols * rows);
  save('dequant', get(deq, cols * rows));

  // norm, rope (three forms), elementwise
  const n = spec.norm.n, nb = spec.norm.batch;
  const xn = up(f32('xn'), 'xn'), wn = up(f32('wn'), 'wn'), yn = out(n * nb, 'yn');
  a.norm(ctx, xn, wn, yn, n, spec.eps, nb);
  save('norm', get(yn, n * nb));
  const r = spec.rope;
  const qk = f32('rope_x');
  const rq = up(qk, 'rope'), rw = up(f32('rope_w'), 'rope w');
  a.ropeNorm(ctx, rq, rw, r.heads, r.hd, r.start, r.theta, 1, spec.eps, 0, r.batch);
  save('rope_norm', get(rq, qk.length));
  a.write(ctx, rq, 0, qk);
  a.ropeNeox(ctx, rq, r.heads, r.hd, r.start, r.theta, 1, r.rot, r.batch);
  save('rope_neox', get(rq, qk.length));
  a.write(ctx, rq, 0, qk);
  a.ropeAdjacent(ctx, rq, r.heads, r.hd, r.start, r.theta, 1, 0, r.batch);
  save('rope_adjacent', get(rq, qk.length));
  const g = up(f32('g'), 'g'), u = up(f32('u'), 'u'), e = spec.elementwise.n;
  const o = out(e, 'o');
  a.silu(ctx, g, u, o, e); save('silu', get(o, e));
  a.gelu(ctx, g, u, o, e); save('gelu', get(o, e));
  a.copy(ctx, u, o, e * 4, 0, 0);
  a.add(ctx, g, o, e); save('add', get(o, e));
  const bias = up(f32('bias'), 'bias');
  a.biasAdd(ctx, o, bias, e, spec.elementwise.width); save('bias_add', get(o, e));
  a.activate(ctx, o, e); save('activate', get(o, e));

  // attention over a wrapped ring, both entry points
  const t = spec.attention;
  const q = up(f32('q'), 'q'), k = up(f32('k'), 'k'), v = up(f32('v'), 'v');
  const ya = out(t.batch * t.heads * t.hd, 'ya'), yb = out(t.batch * t.heads * t.hd, 'yb');
  a.attention(ctx, q, k, v, ya, t.heads, t.kvHeads, t.hd, t.start, t.scale, t.window, t.capacity, t.context, t.batch);
  a.attentionNoalloc(ctx, q, k, v, yb, t.heads, t.kvHeads, t.hd, t.start, t.scale, t.window, t.capacity, t.context, t.batch);
  save('attention', get(ya, t.batch * t.heads * t.hd));
  save('attention_noalloc', get(yb, t.batch * t.heads * t.hd));

  // token pick and embedding
  const logits = up(f32('logits'), 'logits');
  const idx = a.bufferCreate(ctx, 4, 'index');
  const am = a.argmax(ctx, logits, spec.vocab, idx);
  const s = spec.sample;
  const drawn = a.sample(ctx, logits, spec.vocab, s.temperature, s.topK, s.topP, s.seedHi, s.seedLo, s.index);
  save('picks', new Int32Array([am, a.read(ctx, idx, 0, new Int32Array(1))[0], drawn]));
  const table = up(f32('table'), 'table'), ids = up(i32('ids'), 'ids');
  const emb = out(spec.embed.hidden * spec.embed.n, 'embedded');
  a.embed(ctx, 0, table, ids, emb, spec.embed.hidden, spec.embed.n, spec.embed.scale);
  save('embed', get(emb, spec.embed.hidden * spec.embed.n));

  // error paths: statuses become thrown Errors with the library's message and code
  const grab = (f) => { try { f(); return null; } catch (err) { return [err.code, err.message]; } };
  errors.overrun = grab(() => a.write(ctx, idx, 0, new Float32Array(2)));
  errors.badType = grab(() => a.matmul(ctx, 99, wRaw, x, y1, cols, rows, rows, 0, 0, 1));
  errors.negative = grab(() => a.norm(ctx, xn, wn, yn, -1, spec.eps, 1));
  errors.wrongHandle = grab(() => a.clear(ctx, ctx));
  a.bufferDestroy(ctx, idx);
  errors.destroyed = grab(() => a.clear(ctx, idx));
  errors.bufferSize = a.bufferSize(ctx, y1);
  const mem = a.memory(ctx);
  errors.memory = mem.allocated > 0 && mem.peak >= mem.allocated;
  a.done(ctx);
} finally {
  a.destroy(ctx);
}
console.log(JSON.stringify({ ok: true, errors }));
