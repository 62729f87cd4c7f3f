// Drives the Node host end to end and prints JSON for the pytest wrapper: argv is
// <gguf path> <mode> [prompt ids comma-separated] [max tokens] [temperature:seed].
//   config: modelConfig + attentionMemory of the file (no GPU)
//   greedy: load, last-row logits of forward(ids, 0), then generate(ids, maxTokens) ids
//           (sampled with the given temperature and seed when the last argument is set)
import { readGGUF, modelConfig, FileSource } from '../../webgpu_amd/node/gguf.mjs';
import { attentionMemory } from '../../webgpu_amd/node/context.mjs';

const [path, mode, idsArg, maxArg, sampleArg] = process.argv.slice(2);

async function main() {
  if (mode === 'config') {
    const src = new FileSource(path);
    const g = readGGUF(src);
    const c = modelConfig(g);
    src.close();
    const tensors = [...g.tensors.values()].map((t) => [t.name, t.type, t.offset, t.bytes]);
    console.log(JSON.stringify({ config: c, capacities: attentionMemory(c, 512, 128).capacities, tensors, dataOffset: g.dataOffset }));
    return;
  }
  const { PagedEngine } = await import('../../webgpu_amd/node/engine.mjs');
  const ids = idsArg.split(',').map(Number);
  const eng = new PagedEngine();
  const info = eng.load(path, { contextLength: 512, batchSize: 128 });
  try {
    const logits = eng.forward(ids, 0, true);
    eng.reset();
    const tokens = [];
    const [temperature, seed] = sampleArg ? sampleArg.split(':').map(Number) : [0, 0];
    for await (const ev of eng.generate(ids, { maxTokens: Number(maxArg), temperature, seed })) tokens.push(ev.token);
    console.log(JSON.stringify({ adapter: info.adapter, logits: Array.from(logits), tokens, gpuBytes: info.stats.gpuBytes }));
  } finally {
    eng.dispose();
  }
}

main().catch((e) => { console.error(e && e.stack ? e.stack : e); process.exit(1); });
