// engine.mjs — PagedEngine for the Node host (src/core/engine.ts:26-324) over the libwgd
// N-API addon: load(path, options) -> ModelInfo, async generate(prompt ids, options) ->
// TokenEvents, forward, reset, dispose, info and the device token pick. GGUF parsing,
// modelConfig and ring sizing run here as in gguf.ts / context.ts; weights are uploaded
// once and stay resident (the weight pager collapses), and every forward and decode
// step runs in libwgd on the GPU. The Node host has no tokenizer of its own: prompts are ids,
// or any object with chat(messages) -> ids, decode(ids) -> string and eos passed as
// `tokenizer`, which is where the reference's TypeScript tokenizers plug in.
import { createRequire } from 'module';
import { readGGUF, modelConfig, FileSource } from './gguf.mjs';
import { attentionMemory, validateContext, outputLimit, MAX_CONTEXT } from './context.mjs';

const require = createRequire(import.meta.url);
const addon = require('./wgd_napi.node');

const BATCHES = [1, 8, 16, 32, 64, 128];
// engine.ts:14-18: the prompt batch of each performance mode (the budget and page size of
// the reference presets belong to its weight pager; every weight is resident here).
export const PRESETS = { lite: 8, 'low-memory': 16, fast: 128 };

/** The wgd_model_config fields for a ModelConfig (field names of include/wgd.h). */
export function configStruct(c, context, batch, tied, kvF16 = false) {
  const gemma = c.family === 'gemma3';
  return {
    family: gemma ? 1 : 0, rope_adjacent: c.rope === 'norm' ? 1 : 0,
    hidden: c.hidden, intermediate: c.intermediate, layers: c.layers, heads: c.heads, kv_heads: c.kvHeads,
    head_dim: c.headDim, vocab: c.vocab, rotary_dim: c.rotaryDim, window: gemma ? c.window : c.slidingWindow,
    period: c.period, qk_norm: c.qkNorm ? 1 : 0, ffn_gate: c.ffnGate ? 1 : 0, gelu: c.activation === 'gelu' ? 1 : 0,
    bias_q: c.bias.q ? 1 : 0, bias_k: c.bias.k ? 1 : 0, bias_v: c.bias.v ? 1 : 0, bias_output: c.bias.output ? 1 : 0,
    tied_output: tied ? 1 : 0, context, batch,
    epsilon: c.epsilon, theta: c.theta, local_theta: c.localTheta, attention_scale: c.attentionScale,
    rope_scale: c.ropeScale, embed_scale: c.architecture === 'gemma3' ? Math.sqrt(c.hidden) : 1,
    kv_f16: kvF16 ? 1 : 0,
  };
}

/** Throws an Error named AbortError (worker.ts:8) once `signal.aborted` is set; any object
 * with that flag serves (an AbortSignal where the runtime has one). */
function checkAbort(signal) {
  if (signal && signal.aborted) {
    const e = new Error('Stopped by user');
    e.name = 'AbortError';
    throw e;
  }
}

export class PagedEngine {
  constructor(progress) {
    this.progress = progress || (() => {});
    this.ctx = null; this.model = null; this.source = null; this.gguf = null; this.config = null;
    this.context = 512; this.batch = 16; this.kvCapacities = []; this.kvCacheType = 'f32';
    this.budget = null; this.performance = 'low-memory';
    this.busy = false; this.disposed = false; this.tokensInCache = [];
  }

  /** PagedEngine.load (engine.ts:51-114): parse, configure, upload, seal. */
  load(path, options = {}, signal) {
    // kvCacheType 'f16' keeps the K/V rings in half precision (rounded to nearest even when
    // cached, attention math in f32); the reference's rings are f32 (engine.ts:98-101)
    const o = Object.assign({ contextLength: 512, gpuBudgetMiB: null, performance: 'low-memory', device: 0, kvCacheType: 'f32' }, options);
    if (o.kvCacheType !== 'f32' && o.kvCacheType !== 'f16') throw new Error('KV cache type must be f32 or f16.');
    this.kvCacheType = o.kvCacheType;
    if (!(o.performance in PRESETS)) throw new Error('Performance must be lite, low-memory or fast.');
    this.performance = o.performance; this.budget = o.gpuBudgetMiB;
    this.context = o.contextLength; this.batch = o.batchSize === undefined || o.batchSize === null ? PRESETS[o.performance] : o.batchSize;
    validateContext(this.context);
    if (!BATCHES.includes(this.batch)) throw new Error('Batch size must be 1, 8, 16, 32, 64 or 128.');
    if (o.gpuBudgetMiB !== null && (!Number.isInteger(o.gpuBudgetMiB) || o.gpuBudgetMiB < 512))
      throw new Error('GPU budget must be at least 512 MiB.');
    this.source = new FileSource(path);
    this.progress({ phase: 'loading', detail: 'Reading GGUF metadata', fraction: 0.05 });
    this.gguf = readGGUF(this.source);
    const c = this.config = modelConfig(this.gguf);
    validateContext(this.context, c.maxContext);
    this.kvCapacities = attentionMemory(c, this.context, this.batch, o.kvCacheType === 'f16' ? 2 : 4).capacities;
    this.ctx = addon.create(o.device, o.gpuBudgetMiB);
    try {
      const tied = !this.gguf.tensors.has('output.weight');
      this.model = addon.modelCreate(this.ctx, configStruct(c, this.context, this.batch, tied, o.kvCacheType === 'f16'),
        Int32Array.from(this.kvCapacities));
      const tensors = [...this.gguf.tensors.values()].filter((t) => (t.dims.length === 1 || t.dims.length === 2) &&
        (!t.name.startsWith('blk.') || Number(t.name.split('.')[1]) < c.layers));
      tensors.forEach((t, i) => {
        checkAbort(signal);
        addon.modelTensor(this.model, t.name, t.type, t.dims, this.source.read(t.offset, t.bytes));
        if (i % 64 === 0) this.progress({ phase: 'loading', detail: 'Uploading weights', fraction: 0.1 + (0.85 * i) / tensors.length });
      });
      addon.modelReady(this.model);
      this.progress({ phase: 'ready', detail: 'Ready.', fraction: 1 });
      return this.info();
    } catch (e) {
      this.dispose();
      throw e;
    }
  }

  info() {
    return { config: this.config, fileBytes: this.source ? this.source.size : 0, adapter: this.ctx ? addon.adapterName(this.ctx) : '',
      contextLength: this.context, gpuBudgetMiB: this.budget, batchSize: this.batch, performance: this.performance,
      stats: this.stats() };
  }

  stats() {
    if (!this.ctx) return { gpuBytes: 0, peakGpuBytes: 0 };
    const m = addon.memory(this.ctx);
    return { gpuBytes: m.allocated, peakGpuBytes: m.peak };
  }

  /** forward(ids, start, logits) (engine.ts:138-180): the last row's logits, or null. */
  forward(ids, start, logits) {
    if (!this.model) throw new Error('Load a model first.');
    const out = logits ? new Float32Array(this.config.vocab) : null;
    addon.modelForward(this.model, Int32Array.from(ids), start, out);
    return out;
  }

  /** forward + the token pick on the device (greedy, or sampled: setSampling). */
  forwardArgmax(ids, start) {
    if (!this.model) throw new Error('Load a model first.');
    return addon.modelForward(this.model, Int32Array.from(ids), start, null);
  }

  /** The token pick of forwardArgmax and decode: greedy at temperature 0, else top-k /
   * top-p sampling on the device with the uniforms of `seed` (an integer below 2^53). */
  setSampling(temperature, topK = 40, topP = 0.9, seed = 0) {
    addon.modelSampling(this.model, temperature, topK, topP, Math.floor(seed / 4294967296) >>> 0, seed >>> 0);
  }

  /** `count` decode steps on the device from `token` at position `start`. */
  decode(token, start, count) {
    return Array.from(addon.modelDecode(this.model, token, start, count));
  }

  /** PagedEngine.generate (engine.ts:257-301), greedy or sampled on the device (the
   * reference's GenerationOptions defaults, plus `seed`): prefix reuse, output limit, chunked
   * prefill and the busy guard; the decode loop runs on the device `chunk` tokens at a time.
   * A chunk may run past an end-of-turn token; a sliding ring keeps the window plus one
   * prompt batch, so on models with one the chunk is capped to the batch. An aborted
   * `signal` stops at the next prompt batch or token and drops the cached prefix. */
  async *generate(prompt, options = {}, tokenizer = null, chunk = 32, signal = undefined) {
    if (this.busy) throw new Error('A generation is already running.');
    if (this.disposed || !this.model) throw new Error('Load a model first.');
    const o = Object.assign({ maxTokens: 128, temperature: 0.7, topK: 40, topP: 0.9, seed: null }, options);
    if (!Number.isInteger(o.maxTokens) || o.maxTokens < 1 || o.maxTokens > MAX_CONTEXT) throw new Error(`maxTokens must be 1–${MAX_CONTEXT}.`);
    if (!Number.isFinite(o.temperature) || o.temperature < 0 || o.temperature > 2 || !Number.isInteger(o.topK) || o.topK < 1 ||
        o.topK > 200 || !Number.isFinite(o.topP) || o.topP <= 0 || o.topP > 1) throw new Error('Invalid sampling settings.');
    const ids = tokenizer ? Array.from(tokenizer.chat(prompt)) : Array.from(prompt, Number);
    if (!ids.length) throw new Error('Provide a non-empty prompt.');
    const eos = new Set((tokenizer && tokenizer.eos) || []);
    if (this.kvCapacities.some((cap) => cap < this.context)) chunk = Math.min(chunk, this.batch);
    this.busy = true;
    try {
      const limit = outputLimit(o.maxTokens, ids.length, this.context);
      this.setSampling(o.temperature, o.topK, o.topP, o.seed === null ? Math.floor(Math.random() * 2 ** 53) : o.seed);
      let shared = 0;
      while (shared < ids.length && shared < this.tokensInCache.length && ids[shared] === this.tokensInCache[shared]) shared++;
      shared = Math.min(shared, ids.length - 1);
      if (shared < this.tokensInCache.length && this.kvCapacities.some((cap) => cap < this.context)) shared = 0;
      const started = Date.now();
      this.tokensInCache = this.tokensInCache.slice(0, shared);
      let token = -1;
      for (let i = shared; i < ids.length; i += this.batch) {
        checkAbort(signal);
        const part = ids.slice(i, i + this.batch);
        if (i + part.length === ids.length) token = this.forwardArgmax(part, i);
        else this.forward(part, i, false);
        this.tokensInCache.push(...part);
      }
      const generated = [];
      let text = '';
      let pending = [];
      for (let i = 0; i < limit; i++) {
        checkAbort(signal);
        if (i > 0) {
          if (!pending.length) pending = this.decode(token, this.tokensInCache.length, Math.min(chunk, limit - i));
          this.tokensInCache.push(token);
          token = pending.shift();
        }
        if (eos.has(token)) break;
        generated.push(token);
        const full = tokenizer ? tokenizer.decode(generated) : '';
        const delta = full.slice(text.length);
        text = full;
        yield { token, text, delta, tokens: generated.length, promptTokens: ids.length, contextLength: this.context,
          seconds: (Date.now() - started) / 1000, stats: this.stats() };
      }
    } catch (e) {
      this.tokensInCache = [];
      throw e;
    } finally {
      this.busy = false;
    }
  }

  reset() {
    if (this.busy) throw new Error('Stop generation first.');
    this.tokensInCache = [];
  }

  dispose() {
    this.disposed = true;
    if (this.model) addon.modelDestroy(this.model);
    this.model = null;
    if (this.ctx) addon.destroy(this.ctx);
    this.ctx = null;
    if (this.source) this.source.close();
    this.source = null;
    this.tokensInCache = [];
  }
}
