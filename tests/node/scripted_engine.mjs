// A PagedEngine stand-in with the surface worker.mjs drives and no device: ids count up,
// every token yields to the event loop, the abort flag is checked per token.
export class PagedEngine {
  constructor(progress) { this.progress = progress; this.cache = []; }
  load(source, options, signal) {
    if (source === 'bad') throw new Error('Unsupported GGUF version.');
    this.progress({ phase: 'loading', detail: 'Uploading weights', fraction: 0.5 });
    return { fileBytes: 123, contextLength: 512, batchSize: 16, performance: 'low-memory' };
  }
  async *generate(messages, options, tokenizer, chunk, signal) {
    if (!messages || !messages.length) throw new Error('Provide user/assistant text messages.');
    this.cache = [1, 2, 3];
    const n = options.maxTokens || 5;
    try {
      for (let i = 0; i < n; i++) {
        await new Promise((r) => setTimeout(r, 2));
        if (signal.aborted) { const e = new Error('Stopped by user'); e.name = 'AbortError'; throw e; }
        yield { token: i, text: 'x'.repeat(i + 1), delta: 'x', tokens: i + 1 };
      }
    } catch (e) { this.cache = []; throw e; }
  }
  reset() { this.cache = []; }
  dispose() {}
}
