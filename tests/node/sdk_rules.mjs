// sdk_rules.mjs — the WebGPU class (webgpu_amd/node/sdk.mjs) and its worker against the rules
// of src/sdk.ts / src/worker.ts, with a scripted engine in the worker (no GPU). Prints JSON.
import { WebGPU } from '../../webgpu_amd/node/sdk.mjs';

const engineModule = new URL('./scripted_engine.mjs', import.meta.url).href;

async function collect(it) { const out = []; for await (const e of it) out.push(e.token); return out; }
async function error(p) { try { await p; return null; } catch (e) { return [e.name, e.message]; } }

async function main() {
  const r = {};
  let rt = new WebGPU({ engineModule });
  const progress = [];
  rt.onProgress = (p) => progress.push(p.fraction);
  r.noModel = await error(collect(rt.generate([1])));
  r.badLoad = await error(rt.load('bad'));
  r.info = await rt.load('model.gguf');
  r.progress = progress;
  r.tokens = await collect(rt.generate([1, 2], { maxTokens: 5 }));
  // a second request while one runs
  const it = rt.generate([1], { maxTokens: 50 });
  const first = await it.next();
  r.busy = await error(rt.reset());
  // stop: AbortError after the tokens already sent
  rt.stop();
  r.stopped = await error((async () => { for await (const e of it) { void e; } })());
  r.afterStop = (await collect(rt.generate([1], { maxTokens: 3 }))).length;
  // early exit: no error, the runtime is free afterwards
  for await (const e of rt.generate([1], { maxTokens: 1000 })) { if (e.token === 2) break; }
  r.afterBreak = (await collect(rt.generate([1], { maxTokens: 4 }))).length;
  r.first = first.value.token;
  // dispose: pending request and later calls fail
  const pending = rt.generate([1], { maxTokens: 1000 });
  await pending.next();
  const rest = (async () => { for await (const e of pending) { void e; } })();
  rt.dispose();
  r.pending = await error(rest);
  r.disposed = await error(rt.load('model.gguf'));
  console.log(JSON.stringify(r));
}

main().catch((e) => { console.error(e && e.stack ? e.stack : e); process.exit(1); });
