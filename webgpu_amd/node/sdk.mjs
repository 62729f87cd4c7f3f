// sdk.mjs — the runtime API of src/sdk.ts:6-49 for Node: a worker thread (worker.mjs) owns
// every GPU resource; this class sends it requests and turns its messages into promises
// and an async generator, with the reference's rules: one request at a time ("The runtime
// is busy."), stop() cancels the running one (an Error named AbortError), leaving a
// generate loop early stops it and waits without an error, and dispose() ends the worker
// (a pending request fails with "Runtime disposed.", later calls with the disposed error).
import { Worker } from 'worker_threads';

export class WebGPU {
  constructor(options = {}) {
    this.worker = new Worker(new URL('./worker.mjs', import.meta.url),
      { workerData: { engineModule: options.engineModule || null } });
    this.sequence = 0;
    this.busy = false;
    this.disposed = false;
    this.rejectPending = null;
    this.onProgress = null;
  }

  request(action, payload, token) {
    if (this.disposed) return Promise.reject(new Error('This runtime was disposed. Create a new WebGPU instance.'));
    if (this.busy) return Promise.reject(new Error('The runtime is busy.'));
    this.busy = true;
    const id = ++this.sequence;
    return new Promise((resolve, reject) => {
      this.rejectPending = reject;
      const finish = () => {
        this.busy = false;
        this.rejectPending = null;
        this.worker.off('message', listener);
        this.worker.off('error', error);
      };
      const error = (e) => { finish(); reject(new Error(e.message || 'The runtime worker could not start.')); };
      const listener = (m) => {
        if (m.id !== id) return;
        if (m.type === 'progress' && this.onProgress) this.onProgress(m.value);
        if (m.type === 'token' && token) token(m.value);
        if (m.type === 'done') { finish(); resolve(m.value); }
        if (m.type === 'error') {
          finish();
          const e = new Error(m.error);
          if (m.aborted) e.name = 'AbortError';
          reject(e);
        }
      };
      this.worker.on('message', listener);
      this.worker.on('error', error);
      this.worker.postMessage(Object.assign({ id, action }, payload));
    });
  }

  load(source, options = {}) { return this.request('load', { source, options }); }

  async *generate(messages, options = {}) {
    const queue = [];
    let ended = false;
    let failure = null;
    let wake = () => {};
    const task = this.request('generate', { messages, options }, (t) => { queue.push(t); wake(); })
      .catch((e) => { failure = e; })
      .then(() => { ended = true; wake(); });
    try {
      while (!ended || queue.length) {
        if (queue.length) yield queue.shift();
        else await new Promise((resolve) => { wake = resolve; });
      }
      if (failure) throw failure;
    } finally {
      if (!ended) this.stop();
      await task;
    }
  }

  stop() { this.worker.postMessage({ action: 'cancel' }); }

  async reset() { await this.request('reset', {}); }

  dispose() {
    this.disposed = true;
    this.worker.terminate();
    if (this.rejectPending) this.rejectPending(new Error('Runtime disposed.'));
    this.rejectPending = null;
    this.busy = false;
  }
}
