// worker.mjs — the runtime worker of src/worker.ts:1-25 on a Node worker thread: it owns the
// PagedEngine (and so the libwgd context) and answers the WebGPU class (sdk.mjs) with the
// same messages: progress, token, done, error (with `aborted` for a stopped request). A
// request while another runs fails with "The runtime is busy."; a cancel message aborts the
// running one. The addon's calls block this thread, so after each token the loop yields to
// the event loop once, which lets a cancel message in (the reference's awaits do the same).
// workerData.engineModule replaces the engine module (tests drive the rules without a GPU).
import { parentPort, workerData } from 'worker_threads';

const engineModule = (workerData && workerData.engineModule) || './engine.mjs';
let engine = null;
let current = null;
const turn = () => new Promise((resolve) => setImmediate(resolve));

async function handle(m) {
  const { id, action } = m;
  if (action === 'cancel') {
    if (current) current.aborted = true;
    return;
  }
  if (current) {
    parentPort.postMessage({ id, type: 'error', error: 'The runtime is busy.' });
    return;
  }
  const signal = { aborted: false };
  current = signal;
  try {
    const { PagedEngine } = await import(engineModule);
    if (action === 'load') {
      if (engine) engine.dispose();
      engine = new PagedEngine((value) => parentPort.postMessage({ id, type: 'progress', value }));
      const info = engine.load(m.source, m.options || {}, signal);
      parentPort.postMessage({ id, type: 'done', value: info });
    } else if (action === 'generate') {
      if (!engine) throw new Error('Load a model first.');
      for await (const token of engine.generate(m.messages, m.options || {}, null, 32, signal)) {
        parentPort.postMessage({ id, type: 'token', value: token });
        await turn();
      }
      parentPort.postMessage({ id, type: 'done' });
    } else if (action === 'reset') {
      if (engine) engine.reset();
      parentPort.postMessage({ id, type: 'done' });
    } else {
      throw new Error('Unknown runtime action.');
    }
  } catch (e) {
    parentPort.postMessage({ id, type: 'error', error: e instanceof Error ? e.message : String(e), aborted: signal.aborted });
  } finally {
    current = null;
  }
}

parentPort.on('message', (m) => { handle(m); });
