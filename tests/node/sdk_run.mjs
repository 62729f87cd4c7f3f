// sdk_run.mjs — the Node WebGPU class with the real engine in its worker: load a GGUF, one
// greedy reply to prompt ids. argv: <gguf path> <ids comma-separated> <max tokens>. Prints JSON.
import { WebGPU } from '../../webgpu_amd/node/sdk.mjs';

async function main() {
  const [path, idsArg, maxArg] = process.argv.slice(2);
  const rt = new WebGPU();
  try {
    const info = await rt.load(path, { contextLength: 512, batchSize: 128 });
    const tokens = [];
    for await (const e of rt.generate(idsArg.split(',').map(Number), { maxTokens: Number(maxArg), temperature: 0 }))
      tokens.push(e.token);
    console.log(JSON.stringify({ batchSize: info.batchSize, tokens }));
  } finally {
    rt.dispose();
  }
}

main().catch((e) => { console.error(e && e.stack ? e.stack : e); process.exit(1); });
