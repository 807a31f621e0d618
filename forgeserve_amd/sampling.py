"""Token sampling and the plain greedy/sampling generator (sampling.py:1-35 in the reference).

A categorical draw is argmax(p / E) with E ~ Exp(1): this is what torch.multinomial(p, 1) computes
(one exponential_ over the probability tensor, then a divide and an argmax). The noise is drawn from
the caller's generator exactly as torch.multinomial would draw it, then the kernel does the rest on
the GPU, so a seeded run reproduces the reference's tokens.
"""

from typing import Optional

import torch

from . import ops
from .kv import new_contiguous_cache


def exp_noise(shape, generator: Optional[torch.Generator], device) -> torch.Tensor:
    """Exp(1) noise from `generator` (torch's default CPU generator when None), on `device`."""
    gen = generator if generator is not None else torch.default_generator
    e = torch.empty(shape, dtype=torch.float32, device=gen.device).exponential_(generator=gen)
    return e.to(device, non_blocking=True)


def probs_from_logits(logits: torch.Tensor, temperature: float) -> torch.Tensor:
    """softmax(f32(logits) / T); at T == 0 the one-hot of the argmax in the logits dtype."""
    return ops.probs_from_logits(logits, temperature)


def sample(logits: torch.Tensor, temperature: float = 0.0, generator=None) -> torch.Tensor:
    """logits (..., V) -> token ids (...,), int64 on the logits' device."""
    if temperature == 0:
        return ops.sample_logits(logits, 0.0)
    v = logits.shape[-1]
    rows = logits.numel() // v
    noise = exp_noise((rows, v), generator, logits.device)
    return ops.sample_logits(logits, float(temperature), noise)


@torch.no_grad()
def generate(model, prompt: torch.Tensor, max_new_tokens: int, temperature: float = 0.0, generator=None):
    """Prefill, then one token at a time on a contiguous cache; rows of equal length (sampling.py:24-35)."""
    kv = new_contiguous_cache(model.cfg.n_layers)
    max_new_tokens = min(max_new_tokens, model.cfg.max_seq_len - prompt.shape[1])
    dev = model.device
    out = [prompt.to(dev)]
    logits = model(prompt, kv=kv, last_only=True)
    for i in range(max_new_tokens):
        nxt = sample(logits[:, -1], temperature, generator)[:, None]
        out.append(nxt)
        if i + 1 < max_new_tokens:
            logits = model(nxt, kv=kv, last_only=True)
    return torch.cat(out, dim=1).to(prompt.device)
