// engine_rules.mjs — the Node PagedEngine's generate rules with the device calls scripted
// (no GPU): device chunks capped to the batch on a sliding ring, an aborted signal that
// stops the loop and drops the cached prefix, and the sampling-settings validation.
// Prints one JSON line.
import { PagedEngine } from '../../webgpu_amd/node/engine.mjs';

function scripted(context, batch, caps) {
  const eng = new PagedEngine();
  Object.assign(eng, { context, batch, kvCapacities: caps, model: {}, counts: [] });
  eng.forward = () => null;
  eng.forwardArgmax = () => 7;
  eng.decode = (token, start, count) => { eng.counts.push(count); return new Array(count).fill(7); };
  eng.stats = () => ({});
  eng.setSampling = () => {};
  return eng;
}

async function drain(it) { const out = []; for await (const e of it) out.push(e.token); return out; }

async function main() {
  const result = {};
  let eng = scripted(256, 8, [31, 256]);
  result.slidingTokens = (await drain(eng.generate([1, 2, 3], { maxTokens: 100 }))).length;
  result.slidingMaxChunk = Math.max(...eng.counts);
  eng = scripted(256, 8, [256, 256]);
  await drain(eng.generate([1, 2, 3], { maxTokens: 100 }));
  result.fullMaxChunk = Math.max(...eng.counts);

  eng = scripted(512, 16, [512]);
  const signal = { aborted: false };
  const seen = [];
  try {
    for await (const e of eng.generate([1, 2, 3], { maxTokens: 50 }, null, 32, signal)) {
      seen.push(e.token);
      if (seen.length === 3) signal.aborted = true;
    }
    result.abortError = null;
  } catch (e) { result.abortError = e.name; }
  result.abortSeen = seen.length;
  result.abortCache = eng.tokensInCache.length;
  result.abortBusy = eng.busy;

  result.invalid = [];
  for (const bad of [{ temperature: -1 }, { topK: 0 }, { topK: 201 }, { topP: 0 }, { topP: 1.5 }]) {
    try { await drain(scripted(512, 16, [512]).generate([1], bad)); result.invalid.push('accepted'); }
    catch (e) { result.invalid.push(e.message); }
  }
  console.log(JSON.stringify(result));
}
main().catch((e) => { console.error(e); process.exit(1); });
