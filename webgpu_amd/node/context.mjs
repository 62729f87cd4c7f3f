// context.mjs — context limits and KV-ring sizing for the Node host: validateContext /
// outputLimit (src/core/context.ts:5-13) and attentionMemory (context.ts:16-24). Weights are
// resident in HBM, so the paging budget helper has no counterpart.
export const MAX_CONTEXT = 32768;

export function validateContext(context, modelLimit = MAX_CONTEXT) {
  if (!Number.isInteger(context) || context < 256 || context > MAX_CONTEXT)
    throw new Error(`Context must be an integer from 256 to ${MAX_CONTEXT} tokens.`);
  if (context > modelLimit)
    throw new Error(`This model declares a ${modelLimit.toLocaleString('en-US')}-token context. Choose a smaller context.`);
}

export function outputLimit(requested, promptTokens, context) {
  if (!Number.isInteger(requested) || requested < 1 || requested > MAX_CONTEXT)
    throw new Error(`maxTokens must be 1–${MAX_CONTEXT}.`);
  if (promptTokens >= context)
    throw new Error(`The prompt has ${promptTokens.toLocaleString('en-US')} tokens; the context limit is ` +
      `${context.toLocaleString('en-US')}. Start a new chat or reload with a longer context.`);
  return Math.min(requested, context - promptTokens);
}

/** Per-layer ring capacities: Gemma local layers and sliding-window models keep the window
 * plus the rest of the current prompt batch. kvBytes counts K and V at `elementBytes` each
 * (4 as the reference's f32 rings, 2 for f16 rings). */
export function attentionMemory(c, context, batch, elementBytes = 4) {
  const capacities = [];
  for (let l = 0; l < c.layers; l++) {
    if (c.family === 'gemma3') capacities.push(l % c.period !== c.period - 1 ? Math.min(context, c.window + batch - 1) : context);
    else if (c.slidingWindow > 0) capacities.push(Math.min(context, c.slidingWindow + batch - 1));
    else capacities.push(context);
  }
  const kvBytes = capacities.reduce((a, b) => a + b, 0) * c.kvHeads * c.headDim * 2 * elementBytes;
  return { capacities, kvBytes, stateBytes: 0, totalBytes: kvBytes };
}
