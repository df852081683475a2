"""Greedy generation over the quantized Qwen3 model (batch 1).

Callers' interface as in the reference (``ondeviceinfer/generation.py:15-70``):
``greedy_generate(model, input_ids, *, max_new_tokens, cache, eos_token_id)``
returns ``GenerationResult`` (``token_ids``, ``generated_ids``,
``prefill_seconds``, ``decode_seconds``, ``decode_tokens_per_second`` =
(generated - 1) / decode seconds, the first token being the prefill's).

The loop is built around the decode graph: each step's greedy token stays on
the device (the LM-head kernel picks it, ``CausalLMOutput.next_token``), is
fed straight back as the next input and is written into a preallocated
device row of generated ids, so without an ``eos_token_id`` the host waits
only once, at the end of the decode phase.  With one, every step has to
read the token back to decide whether to stop.
"""
from __future__ import annotations

import time
from dataclasses import dataclass

import torch
from torch import Tensor


@dataclass
class GenerationResult:
    token_ids: Tensor
    generated_ids: Tensor
    prefill_seconds: float
    decode_seconds: float

    @property
    def decode_tokens_per_second(self) -> float:
        """Tokens of the decode phase per second; the first generated token
        belongs to the prefill."""
        steps = self.generated_ids.shape[1] - 1
        return steps / self.decode_seconds if steps > 0 and self.decode_seconds > 0 else 0.0


def greedy_token(output) -> Tensor:
    """The greedy next token ``[batch, 1]`` of a model output: the decode
    graph's in-kernel pick when present (the first index of the largest fp16
    logit, ``torch.argmax``'s rule), else the argmax of the last position."""
    picked = getattr(output, 'next_token', None)
    if picked is not None:
        return picked
    return torch.argmax(output.logits[:, -1], dim=-1, keepdim=True)


def _wait(device: torch.device) -> None:
    if device.type == 'cuda':
        torch.cuda.synchronize(device)


@torch.inference_mode()
def greedy_generate(model, input_ids: Tensor, *, max_new_tokens: int, cache, eos_token_id: int | None = None
                    ) -> GenerationResult:
    """Prefill ``input_ids [1, S]`` into ``cache``, then decode greedily until
    ``max_new_tokens`` tokens exist (at least the prefill's one) or the last
    one equals ``eos_token_id``."""
    if input_ids.dim() != 2:
        raise ValueError(f'input_ids must be [batch, sequence], got shape {tuple(input_ids.shape)}')
    if input_ids.shape[0] != 1:
        raise NotImplementedError(f'greedy_generate runs batch size 1, got {input_ids.shape[0]}')
    device = input_ids.device
    budget = max(1, max_new_tokens)

    _wait(device)
    t_prefill = time.perf_counter()
    token = greedy_token(model(input_ids, cache=cache, logits_to_keep=1))
    generated = torch.empty((1, budget), dtype=torch.long, device=token.device)
    generated[:, :1].copy_(token)
    _wait(device)
    prefill_seconds = time.perf_counter() - t_prefill

    count = 1
    t_decode = time.perf_counter()
    while count < budget:
        if eos_token_id is not None and bool((token == eos_token_id).all()):
            break
        token = greedy_token(model(token, cache=cache, logits_to_keep=1))
        generated[:, count:count + 1].copy_(token)
        count += 1
    _wait(device)
    decode_seconds = time.perf_counter() - t_decode

    generated = generated[:, :count]
    return GenerationResult(token_ids=torch.cat((input_ids, generated.to(input_ids.dtype)), dim=1),
                            generated_ids=generated, prefill_seconds=prefill_seconds,
                            decode_seconds=decode_seconds)
