// gguf.mjs — GGUF tensor/quant-type descriptors, header parser and model configuration for
// the Node host: the rules of src/core/gguf.ts (QUANTS :6-11, parseGGUFHeader :48-77,
// readGGUF :78-83, modelConfig :108-213) for the dense families and Gemma 3, with the
// reference's error messages.
import fs from 'fs';

/** GGUF quantization type id -> block layout (gguf.ts:6-11). */
export const QUANTS = Object.freeze({
  0: { name: 'F32', block: 1, bytes: 4 },
  1: { name: 'F16', block: 1, bytes: 2 },
  2: { name: 'Q4_0', block: 32, bytes: 18 },
  8: { name: 'Q8_0', block: 32, bytes: 34 },
  12: { name: 'Q4_K', block: 256, bytes: 144 },
  13: { name: 'Q5_K', block: 256, bytes: 176 },
  14: { name: 'Q6_K', block: 256, bytes: 210 },
});

const MAGIC = 0x46554747;
const MAX_HEADER = 64 * 1024 * 1024;

export class NeedMore extends Error {}

class Reader {
  constructor(bytes) {
    this.b = bytes;
    this.v = new DataView(bytes.buffer, bytes.byteOffset, bytes.byteLength);
    this.offset = 0;
  }
  need(n) { if (this.offset + n > this.b.byteLength) throw new NeedMore('header continues'); }
  u32() { this.need(4); const x = this.v.getUint32(this.offset, true); this.offset += 4; return x; }
  u64() {
    this.need(8);
    const x = this.v.getBigUint64(this.offset, true);
    this.offset += 8;
    if (x > BigInt(Number.MAX_SAFE_INTEGER)) throw new Error('GGUF integer exceeds safe file addressing.');
    return Number(x);
  }
  string() {
    const n = this.u64();
    if (n > 16 * 1024 * 1024) throw new Error('Oversized GGUF string.');
    this.need(n);
    const s = Buffer.from(this.b.buffer, this.b.byteOffset + this.offset, n).toString('utf8');
    this.offset += n;
    return s;
  }
  value(type, depth = 0) {
    if (depth > 2) throw new Error('Invalid nested metadata.');
    const fixed = { 0: [1, 'getUint8'], 1: [1, 'getInt8'], 2: [2, 'getUint16'], 3: [2, 'getInt16'], 4: [4, 'getUint32'],
      5: [4, 'getInt32'], 6: [4, 'getFloat32'], 7: [1, 'getUint8'], 12: [8, 'getFloat64'] };
    if (type === 8) return this.string();
    if (type === 9) {
      const t = this.u32(), n = this.u64();
      if (n > 2000000) throw new Error('Oversized GGUF array.');
      const out = new Array(n);
      for (let i = 0; i < n; i++) out[i] = this.value(t, depth + 1);
      return out;
    }
    if (type === 10) return this.u64();
    if (type === 11) {
      this.need(8);
      const x = Number(this.v.getBigInt64(this.offset, true));
      this.offset += 8;
      return x;
    }
    const f = fixed[type];
    if (!f) throw new Error(`Unknown GGUF metadata type ${type}.`);
    this.need(f[0]);
    const x = this.v[f[1]](this.offset, true);
    this.offset += f[0];
    return type === 7 ? x !== 0 : x;
  }
}

/** parseGGUFHeader (gguf.ts:48-77); throws NeedMore when `bytes` ends inside the header. */
export function parseGGUFHeader(bytes, fileSize) {
  const r = new Reader(bytes);
  if (r.u32() !== MAGIC) throw new Error('Select a GGUF model file.');
  const version = r.u32();
  if (version !== 2 && version !== 3) throw new Error(`GGUF version ${version} is unsupported.`);
  const count = r.u64(), kvCount = r.u64();
  if (count > 100000 || kvCount > 100000) throw new Error('Invalid GGUF counts.');
  const metadata = {};
  for (let i = 0; i < kvCount; i++) {
    const key = r.string();
    metadata[key] = r.value(r.u32());
  }
  const tensors = new Map();
  let parameters = 0;
  for (let i = 0; i < count; i++) {
    const name = r.string();
    const nd = r.u32();
    if (nd < 1 || nd > 4 || tensors.has(name)) throw new Error('Invalid tensor directory.');
    const dims = [];
    for (let j = 0; j < nd; j++) dims.push(r.u64());
    const type = r.u32(), offset = r.u64();
    const q = QUANTS[type];
    if (!q) throw new Error(`Unsupported tensor quantization ${type} in ${name}. Use Q4_K_M, Q5_K_M, Q6_K or Q8_0.`);
    const n = dims.reduce((a, b) => a * b, 1);
    if (n > Number.MAX_SAFE_INTEGER || dims.some((d) => d < 1) || dims[0] % q.block !== 0) throw new Error(`Invalid shape for ${name}.`);
    tensors.set(name, { name, dims, type, offset, bytes: (n / q.block) * q.bytes, rowBytes: (dims[0] / q.block) * q.bytes });
    parameters += n;
  }
  const alignment = metadata['general.alignment'] === undefined ? 32 : metadata['general.alignment'];
  if (!Number.isInteger(alignment) || alignment < 1 || alignment > 4096 || (alignment & (alignment - 1)))
    throw new Error('Invalid GGUF alignment.');
  const dataOffset = Math.ceil(r.offset / alignment) * alignment;
  for (const t of tensors.values()) {
    t.offset += dataOffset;
    if (t.offset + t.bytes > fileSize) throw new Error(`Truncated model: ${t.name}.`);
  }
  return { metadata, tensors, dataOffset, parameters };
}

/** A GGUF file opened for random reads (the resident form of source.ts's FileSource). */
export class FileSource {
  constructor(path) {
    this.fd = fs.openSync(path, 'r');
    this.size = fs.fstatSync(this.fd).size;
    this.name = path.split('/').pop();
    if (this.size < 24) throw new Error('Invalid model file size.');
  }
  read(offset, length) {
    if (offset < 0 || length < 1 || offset + length > this.size) throw new Error('Invalid model byte range.');
    const out = new Uint8Array(length);
    let done = 0;
    while (done < length) {
      const n = fs.readSync(this.fd, out, done, length - done, offset + done);
      if (n <= 0) throw new Error('Short read of the model file.');
      done += n;
    }
    return out;
  }
  close() { if (this.fd !== null) { fs.closeSync(this.fd); this.fd = null; } }
}

/** readGGUF (gguf.ts:78-83): doubling header reads from 4 MiB up to 64 MiB. */
export function readGGUF(source) {
  let n = Math.min(source.size, 4 * 1024 * 1024);
  for (;;) {
    try {
      return parseGGUFHeader(source.read(0, n), source.size);
    } catch (e) {
      if (!(e instanceof NeedMore)) throw e;
      if (n >= source.size || n >= MAX_HEADER) throw new Error('GGUF header exceeds 64 MiB or is truncated.');
      n = Math.min(source.size, n * 2);
    }
  }
}

const DENSE = new Set(['llama', 'qwen2', 'qwen3']);

/** modelConfig (gguf.ts:108-213) for llama/qwen2/qwen3 (family 'llama') and gemma3. */
export function modelConfig(g) {
  const arch = g.metadata['general.architecture'];
  if (typeof arch !== 'string' || !arch) throw new Error('The GGUF file has no architecture metadata.');
  const family = arch === 'gemma3' ? 'gemma3' : DENSE.has(arch) ? 'llama' : null;
  if (!family)
    throw new Error(`Supported text architectures: Gemma 3, Llama 3.x and Mistral (llama), Qwen2 and Qwen3. The ${arch} architecture is not supported.`);
  const meta = (key) => g.metadata[`${arch}.${key}`];
  const num = (key, fallback) => {
    let v = meta(key);
    if (v === undefined || v === null) v = fallback;
    if (typeof v === 'boolean') v = v ? 1 : 0;
    if (typeof v !== 'number' || !Number.isFinite(v) || v <= 0) throw new Error(`Missing or invalid ${arch} metadata: ${key}.`);
    return v;
  };
  const opt = (key, fallback) => (meta(key) === undefined || meta(key) === null ? fallback : num(key));
  const layers = num('block_count'), hidden = num('embedding_length'), heads = num('attention.head_count');
  const headDim = family === 'llama' ? opt('attention.key_length', hidden / heads) : num('attention.key_length');
  const embd = g.tensors.get('token_embd.weight');
  const vocab = embd && embd.dims.length > 1 ? embd.dims[1] : 0;
  const c = {
    architecture: arch, family, hidden, layers, heads, headDim, vocab,
    kvHeads: family === 'llama' ? opt('attention.head_count_kv', heads) : num('attention.head_count_kv'),
    intermediate: num('feed_forward_length'),
    epsilon: num('attention.layer_norm_rms_epsilon', 1e-6),
    theta: family === 'llama' ? opt('rope.freq_base', 10000) : num('rope.freq_base', 1000000),
    localTheta: family === 'llama' ? opt('rope.freq_base', 10000) : num('rope.local.freq_base', 10000),
    window: family === 'llama' ? 0 : num('attention.sliding_window', 1024),
    period: family === 'gemma3' ? 6 : 0,
    attentionScale: 1 / Math.sqrt(family === 'gemma3' && layers === 62 ? hidden / heads : headDim),
    ropeScale: 1,
    name: String(g.metadata['general.name'] === undefined ? arch : g.metadata['general.name']),
    parameters: g.parameters,
    rotaryDim: family === 'llama' ? opt('rope.dimension_count', headDim) : headDim,
    maxContext: num('context_length', 32768),
    rope: arch === 'llama' ? 'norm' : 'neox',
    slidingWindow: family === 'llama' ? Math.floor(opt('attention.sliding_window', 0)) : num('attention.sliding_window', 1024),
    qkNorm: true, ffnGate: true, activation: family === 'gemma3' ? 'gelu' : 'silu',
    bias: { q: false, k: false, v: false, output: false },
  };
  // a linear RoPE factor is a plain position divisor; llama3/yarn keep unscaled positions
  const scaling = meta('rope.scaling.type');
  if (String(scaling === undefined ? 'linear' : scaling) === 'linear') c.ropeScale = 1 / num('rope.scaling.factor', 1);
  if (!Number.isInteger(c.maxContext)) throw new Error('Invalid model context length.');
  const ints = [layers, hidden, heads, headDim, c.kvHeads, c.intermediate, c.rotaryDim];
  if (ints.some((n) => !Number.isInteger(n) || n < 1) || c.period < 0 || heads % c.kvHeads || headDim % 2 || c.rotaryDim % 2 ||
      c.rotaryDim > headDim || !c.vocab || layers > 128 || heads > 256 || headDim > 512 || hidden > 16384 ||
      c.intermediate > 131072 || c.vocab > 1000000)
    throw new Error('Unsupported model dimensions.');
  const shape = (name, dims) => {
    const t = g.tensors.get(name);
    if (!t || t.dims.length !== dims.length || t.dims.some((d, i) => d !== dims[i])) throw new Error(`Missing or invalid tensor ${name}.`);
  };
  const H = c.hidden, L = c.layers;
  shape('token_embd.weight', [H, c.vocab]);
  shape('output_norm.weight', [H]);
  if (g.tensors.has('output.weight')) shape('output.weight', [H, c.vocab]);
  if (family === 'llama') {
    if (g.tensors.has('blk.0.ffn_gate_inp.weight') || g.tensors.has('blk.0.ffn_gate_exps.weight'))
      throw new Error('Mixture-of-experts models are not supported.');
    c.ffnGate = g.tensors.has('blk.0.ffn_gate.weight');
    c.qkNorm = g.tensors.has('blk.0.attn_q_norm.weight');
    for (const k of ['q', 'k', 'v', 'output']) c.bias[k] = g.tensors.has(`blk.0.attn_${k}.bias`);
    const attn = c.heads * c.headDim, kv = c.kvHeads * c.headDim;
    for (let l = 0; l < L; l++) {
      const p = `blk.${l}.`;
      shape(p + 'attn_norm.weight', [H]);
      shape(p + 'ffn_norm.weight', [H]);
      shape(p + 'attn_q.weight', [H, attn]);
      shape(p + 'attn_k.weight', [H, kv]);
      shape(p + 'attn_v.weight', [H, kv]);
      shape(p + 'attn_output.weight', [attn, H]);
      if (c.bias.q) shape(p + 'attn_q.bias', [attn]);
      if (c.bias.k) shape(p + 'attn_k.bias', [kv]);
      if (c.bias.v) shape(p + 'attn_v.bias', [kv]);
      if (c.bias.output) shape(p + 'attn_output.bias', [H]);
      if (c.qkNorm) for (const k of ['attn_q_norm', 'attn_k_norm']) shape(p + k + '.weight', [c.headDim]);
      if (c.ffnGate) shape(p + 'ffn_gate.weight', [H, c.intermediate]);
      shape(p + 'ffn_up.weight', [H, c.intermediate]);
      shape(p + 'ffn_down.weight', [c.intermediate, H]);
    }
    return c;
  }
  for (let l = 0; l < L; l++) {
    const p = `blk.${l}.`;
    for (const k of ['attn_norm', 'post_attention_norm', 'ffn_norm', 'post_ffw_norm']) shape(p + k + '.weight', [H]);
    for (const k of ['attn_q_norm', 'attn_k_norm']) shape(p + k + '.weight', [c.headDim]);
    shape(p + 'attn_q.weight', [H, c.heads * c.headDim]);
    for (const k of ['attn_k', 'attn_v']) shape(p + k + '.weight', [H, c.kvHeads * c.headDim]);
    shape(p + 'attn_output.weight', [c.heads * c.headDim, H]);
    for (const k of ['ffn_gate', 'ffn_up']) shape(p + k + '.weight', [H, c.intermediate]);
    shape(p + 'ffn_down.weight', [c.intermediate, H]);
  }
  return c;
}
