"""Context limits and KV-ring sizing: host mirror of ``src/core/context.ts``.

``validate_context`` / ``output_limit`` follow context.ts:5-13, ``attention_memory``
sizes each layer's K/V ring (context.ts:16-24) and ``cache_copies`` splits a ring
append at the wrap point (context.ts:34-37). The paging budget helper
(``suggestBudget``) has no counterpart: weights are resident in HBM.
"""
from __future__ import annotations

from typing import Dict, List

MAX_CONTEXT = 32768
MAX_MESSAGE_CHARS = 1048576


def _is_int(v) -> bool:
    return isinstance(v, int) and not isinstance(v, bool) or (isinstance(v, float) and v.is_integer())


def validate_context(context, model_limit: int = MAX_CONTEXT) -> None:
    if not _is_int(context) or context < 256 or context > MAX_CONTEXT:
        raise ValueError(f"Context must be an integer from 256 to {MAX_CONTEXT} tokens.")
    if context > model_limit:
        raise ValueError(f"This model declares a {model_limit:,}-token context. Choose a smaller context.")


def output_limit(requested, prompt_tokens: int, context: int) -> int:
    if not _is_int(requested) or requested < 1 or requested > MAX_CONTEXT:
        raise ValueError(f"maxTokens must be 1–{MAX_CONTEXT}.")
    if prompt_tokens >= context:
        raise ValueError(f"The prompt has {prompt_tokens:,} tokens; the context limit is {context:,}. "
                         "Start a new chat or reload with a longer context.")
    return int(min(requested, context - prompt_tokens))


def attention_memory(c, context: int, batch: int, element_bytes: int = 4) -> Dict[str, object]:
    """Per-layer ring capacities: Gemma local layers and sliding-window models keep the
    window plus the rest of the current prompt batch (context.ts:14-19). kvBytes counts
    K and V at ``element_bytes`` each: 4 as the reference's f32 rings, 2 for f16 rings."""
    caps: List[int] = []
    for l in range(c.layers):
        if c.family == "gemma3":
            caps.append(min(context, c.window + batch - 1) if l % c.period != c.period - 1 else context)
        elif c.slidingWindow > 0:
            caps.append(min(context, c.slidingWindow + batch - 1))
        else:
            caps.append(context)
    kv_bytes = sum(caps) * c.kvHeads * c.headDim * 2 * element_bytes
    return {"capacities": caps, "kvBytes": kv_bytes, "stateBytes": 0, "totalBytes": kv_bytes}


def cache_copies(start: int, count: int, capacity: int) -> List[Dict[str, int]]:
    """Consecutive ring copies, split at the wrap (context.ts:34-37)."""
    offset = start % capacity
    first = min(count, capacity - offset)
    copies = [{"source": 0, "target": offset, "count": first}]
    if first < count:
        copies.append({"source": first, "target": 0, "count": count - first})
    return copies
