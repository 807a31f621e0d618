"""Speculative decoding on the GPU (speculative.py:1-86 in the reference).

Two entry points:

* `verify_draft` / `speculative_generate`: the reference's single-sequence API. The forwards, the
  draft draws and the acceptance run as HIP kernels; the random numbers are drawn from the caller's
  generator in exactly the order the reference draws them (draft Exp(1) vectors, then one uniform per
  examined proposal, then one Exp(1) vector for the final draw), so a seeded run reproduces the
  reference's tokens.

* `SpeculativeBatch` / `speculative_generate_batch`: batched speculation over paged KV pools, the
  throughput path. Per round it runs k draft decode steps (T = 2 for the first step, which re-feeds
  the previous token so a fully accepted round needs no separate catch-up forward), one target
  verify pass over the k+1 window, and one fused acceptance launch that also advances the cached
  lengths on the device. Randomness comes from the device generator as tensors (u, E) handed to the
  kernels; the only device-to-host copy per round is (n_accepted, out_tokens).
"""

from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np
import torch

from . import ops
from ._lib import to_device
from .kv import new_contiguous_cache
from .paged import BlockList, OutOfBlocks, PagedKVPool, block_table
from .sampling import exp_noise, probs_from_logits

I32 = torch.int32


def _clone_generator(gen: torch.Generator) -> torch.Generator:
    g = torch.Generator(device=gen.device)
    g.set_state(gen.get_state())
    return g


def verify_draft(p: torch.Tensor, q: torch.Tensor, draft_tokens: List[int], generator=None) -> Tuple[List[int], int]:
    """p (k+1, V) target probabilities, q (k, V) draft probabilities, k draft tokens ->
    (accepted draft tokens, one extra token from the target) (speculative.py:20-33)."""
    k = len(draft_tokens)
    v = p.shape[-1]
    dev = p.device
    gen = generator if generator is not None else torch.default_generator
    # the reference draws u_i lazily, one per examined proposal; a clone yields the same values
    peek = _clone_generator(gen)
    u = torch.tensor([float(torch.rand((), generator=peek, device=gen.device)) for _ in range(k)],
                     dtype=torch.float32)
    u = u.to(dev)
    xs = torch.tensor(list(draft_tokens), dtype=I32).to(dev)
    qq = q if k else p[:0]
    # decisions do not depend on the noise: find the first rejection, then draw the noise the
    # reference would draw after exactly that many uniforms
    _, n = ops.verify_probs(p, qq, xs, u, torch.ones(v, dtype=torch.float32, device=dev))
    j = int(n[0])
    for _ in range(min(j + 1, k)):
        torch.rand((), generator=gen, device=gen.device)
    noise = exp_noise((v,), gen, dev)
    out, _ = ops.verify_probs(p, qq, xs, u, noise)
    toks = out[: j + 1].tolist()
    return toks[:j], toks[j]


@torch.no_grad()
def speculative_generate(target, draft, prompt: List[int], max_new_tokens: int, k: int = 4,
                         temperature: float = 0.0, generator=None):
    """Generate with `target`, drafting k tokens at a time with `draft` (speculative.py:36-86).

    Returns (new tokens, {"rounds", "proposed", "accepted"}). One sequence."""
    if target.cfg.vocab_size != draft.cfg.vocab_size:
        raise ValueError("target and draft must share a vocabulary")
    limit = min(target.cfg.max_seq_len, draft.cfg.max_seq_len)
    tokens = list(prompt)
    kv_t, kv_d = new_contiguous_cache(target.cfg.n_layers), new_contiguous_cache(draft.cfg.n_layers)
    if len(tokens) > 1:
        target(torch.tensor([tokens[:-1]]), kv=kv_t, last_only=True)
        draft(torch.tensor([tokens[:-1]]), kv=kv_d, last_only=True)
    stats = {"rounds": 0, "proposed": 0, "accepted": 0}
    start = len(tokens)
    dev = target.device
    v = target.cfg.vocab_size

    while len(tokens) - start < max_new_tokens and len(tokens) < limit:
        remaining = min(max_new_tokens - (len(tokens) - start), limit - len(tokens))
        k_eff = min(k, remaining - 1)
        cached = kv_t[0].length

        xs, qs, cur = [], [], tokens[-1]
        for _ in range(k_eff):
            logits = draft(torch.tensor([[cur]]), kv=kv_d)[0, -1]
            q = probs_from_logits(logits, temperature)
            if temperature == 0:
                cur = int(ops.sample_logits(logits, 0.0))
            else:
                cur = int(ops.sample_logits(logits, float(temperature), exp_noise((1, v), generator, dev)))
            xs.append(cur)
            qs.append(q)

        p = probs_from_logits(target(torch.tensor([[tokens[-1]] + xs]), kv=kv_t)[0], temperature)
        accepted, extra = verify_draft(p, torch.stack(qs) if qs else p[:0], xs, generator)
        tokens += accepted + [extra]
        stats["rounds"] += 1
        stats["proposed"] += k_eff
        stats["accepted"] += len(accepted)

        want = cached + 1 + len(accepted)
        for view in kv_t:
            view.truncate(want)
        have = kv_d[0].length
        if have > want:
            for view in kv_d:
                view.truncate(want)
        elif have < want:
            draft(torch.tensor([tokens[have:want]]), kv=kv_d, last_only=True)
    return tokens[start:], stats


# ------------------------------------------------------------------------------------------------
# one round over a batch of sequences held in paged pools
# ------------------------------------------------------------------------------------------------
class _GeneratorDraws:
    """The round's random numbers from one generator, in the batch loop's order: per draft step a
    (b, V) Exp(1) block, then u (b, k), then the final Exp(1) block."""

    def __init__(self, gen, b, k, v, dev):
        self.gen, self.b, self.k, self.v, self.dev = gen, b, k, v, dev

    def draft(self, i):
        return torch.empty((self.b, self.v), dtype=torch.float32, device=self.dev).exponential_(generator=self.gen)

    def accept(self):
        u = torch.rand((self.b, max(self.k, 1)), dtype=torch.float32, device=self.dev, generator=self.gen)
        e = torch.empty((self.b, self.v), dtype=torch.float32, device=self.dev).exponential_(generator=self.gen)
        return u[:, : self.k].contiguous(), e


@torch.no_grad()
def spec_round(target, draft, pool_t: PagedKVPool, pool_d: PagedKVPool, tokens: List[List[int]],
               blocks_t: List[List[int]], blocks_d: List[List[int]], k_eff: List[int], temps: List[float],
               draws) -> torch.Tensor:
    """One draft-then-verify round (speculative.py:53-85) for b sequences whose caches hold positions
    0..n-2 (n = len(tokens[r])) and whose block lists cover positions up to n-1+k_eff[r].

    Per round: k draft decode steps (step 0 re-feeds (tokens[-2], tokens[-1]) at (n-2, n-1), so a fully
    accepted round needs no catch-up forward; step i feeds x_{i-1} at n-1+i), one target verify pass
    over the k+1 window, one fused acceptance. `draws` supplies the randomness: draft(i) -> (b, V)
    Exp(1) noise of draft step i, accept() -> (u (b, k), E (b, V)); rows of greedy sequences are
    ignored. Returns (b, k+2) int32 on the host: n_accepted, then the committed tokens (-1 padded)."""
    b = len(tokens)
    k = max(k_eff)
    dev, dtype = target.device, target.dtype
    n = np.array([len(t) for t in tokens], dtype=np.int64)
    keff = np.array(k_eff, dtype=np.int64)
    tab_t = block_table(blocks_t, dev)
    tab_d = block_table(blocks_d, dev)
    v = target.cfg.vocab_size
    temps_dev = to_device(torch.tensor(temps, dtype=torch.float32), dev)
    sampling = any(t > 0 for t in temps)
    # The LM heads emit the logits' softmax statistics (sampling.py:13) as they write them, so the
    # acceptance does not read the 2k+1 logit rows back to normalise them.
    d = target.cfg.d_model
    fused = (dtype == torch.bfloat16 and k > 0 and ops.row_stats_parts(b, v, d) > 0
             and ops.row_stats_parts(b * (k + 1), v, d) > 0)
    if fused:
        inv_t = torch.tensor([1.0 / t if t > 0 else 0.0 for t in temps], dtype=torch.float32)
        inv_t_d = to_device(inv_t, dev)
        inv_t_t = to_device(inv_t.repeat_interleave(k + 1), dev)
        # draft step i writes its rows' records into parts_d[:, i]; one merge after the last step
        parts_d = torch.empty((b, k, ops.row_stats_parts(b, v, d), 4), dtype=I32, device=dev)
        parts_t = torch.empty((b * (k + 1), ops.row_stats_parts(b * (k + 1), v, d), 4), dtype=I32, device=dev)
        row_stats = torch.empty((b, 2 * k + 1, 4), dtype=I32, device=dev)

    # 1. draft
    dft_logits = torch.empty((b, k, v), dtype=dtype, device=dev)
    draft_tok = torch.empty((b, k), dtype=I32, device=dev)
    last = torch.tensor([t[-1] for t in tokens], dtype=torch.int64)
    prev = torch.tensor([t[-2] if len(t) > 1 else 0 for t in tokens], dtype=torch.int64)
    cur = None
    for i in range(k):
        if i == 0:
            idx = to_device(torch.stack([prev, last], 1), dev)
            p = np.stack([np.where(n > 1, n - 2, -1), n - 1], 1)
            pos = torch.from_numpy(np.where(keff[:, None] > 0, p, -1))
        else:
            idx = cur.to(torch.int64)[:, None]
            pos = torch.from_numpy(np.where(i < keff, n - 1 + i, -1)[:, None])
        logits = draft(idx, pos, pool_d.views(tab_d, pos), last_only=True,
                       head_stats=(inv_t_d, parts_d[:, i]) if fused else None)[:, 0]
        dft_logits[:, i].copy_(logits)
        ops.sample_logits(logits, temps_dev, draws.draft(i) if sampling else None, out32=draft_tok[:, i])
        cur = draft_tok[:, i]
    if fused:   # draft row (b, i) is record b*k + i: sequence b's draft rows k+1 .. 2k
        ops.row_stats_merge(parts_d.view(b * k, -1, 4), row_stats, k, 2 * k + 1, k + 1)

    # 2. target verify over [tokens[-1], x_0 .. x_{k-1}] at n-1 .. n-1+k
    last_dev = to_device(last, dev)
    idx = torch.cat([last_dev[:, None], draft_tok.to(torch.int64)], 1) if k else last_dev[:, None]
    t_ = np.arange(k + 1)[None, :]
    pos = torch.from_numpy(np.where(t_ <= keff[:, None], n[:, None] - 1 + t_, -1))
    tgt_logits = target(idx, pos, pool_t.views(tab_t, pos), head_stats=(inv_t_t, parts_t) if fused else None)
    if fused:
        ops.row_stats_merge(parts_t, row_stats, k + 1, 2 * k + 1, 0)

    # 3. acceptance
    u, noise = draws.accept()
    keff_dev = to_device(torch.tensor(k_eff, dtype=I32), dev)
    out_tok, n_acc = ops.spec_accept(tgt_logits, dft_logits, draft_tok, keff_dev, temps_dev, u, noise,
                                     row_stats=row_stats if fused else None)
    return torch.cat([n_acc[:, None], out_tok], 1).cpu()


# ------------------------------------------------------------------------------------------------
# batched speculation over paged pools
# ------------------------------------------------------------------------------------------------
class _Seq:
    __slots__ = ("tokens", "start", "max_new", "temperature", "blocks_t", "blocks_d", "done", "eos_id")

    def __init__(self, tokens, max_new, temperature, eos_id=None):
        self.tokens = list(tokens)
        self.start = len(tokens)
        self.max_new = max_new
        self.temperature = float(temperature)
        self.blocks_t = BlockList()
        self.blocks_d = BlockList()
        self.done = False
        self.eos_id = eos_id


class SpeculativeBatch:
    """Batched draft-then-verify rounds over paged KV pools (one pool for the target, one for the draft).

    Sequence state lives on the host (token lists, block lists); KV, logits, draft tokens, random
    numbers and acceptance results live on the GPU. `round()` advances every active sequence by
    1 + (accepted proposals) tokens."""

    def __init__(self, target, draft, num_blocks: int, block_size: int = 16, k: int = 4,
                 draft_num_blocks: Optional[int] = None, generator: Optional[torch.Generator] = None):
        if target.cfg.vocab_size != draft.cfg.vocab_size:
            raise ValueError("target and draft must share a vocabulary")
        self.target, self.draft, self.k = target, draft, k
        self.dev, self.dtype = target.device, target.dtype
        self.pool_t = PagedKVPool(target.cfg, num_blocks, block_size, dtype=self.dtype, device=self.dev)
        self.pool_d = PagedKVPool(draft.cfg, draft_num_blocks or num_blocks, block_size, dtype=self.dtype,
                                  device=self.dev)
        self.block_size = block_size
        self.limit = min(target.cfg.max_seq_len, draft.cfg.max_seq_len)
        self.gen = generator
        self.seqs: List[_Seq] = []
        self.stats = {"rounds": 0, "proposed": 0, "accepted": 0}

    # ---- sequences ------------------------------------------------------------------------------
    def _grow(self, seq: _Seq, n_tokens: int) -> None:
        for pool, blocks in ((self.pool_t, seq.blocks_t), (self.pool_d, seq.blocks_d)):
            need = pool.blocks_for(n_tokens) - len(blocks)
            if need > 0:
                blocks += pool.allocator.allocate(need)

    def release(self, seq: _Seq) -> None:
        self.pool_t.allocator.release(seq.blocks_t)
        self.pool_d.allocator.release(seq.blocks_d)
        seq.blocks_t, seq.blocks_d = BlockList(), BlockList()

    def add(self, prompt: Sequence[int], max_new_tokens: int, temperature: float = 0.0, eos_id=None,
            prefill: bool = True) -> _Seq:
        """Add a sequence; with prefill, its prompt (all but the last token) is run through both models."""
        if not 0 < len(prompt) < self.limit:
            raise ValueError(f"prompt length must be in 1..{self.limit - 1}")
        seq = _Seq(prompt, max_new_tokens, temperature, eos_id)
        self._grow(seq, len(seq.tokens))
        if prefill and len(seq.tokens) > 1:
            n = len(seq.tokens) - 1
            idx = torch.tensor([seq.tokens[:-1]])
            pos = torch.arange(n)[None]
            for model, pool, blocks in ((self.target, self.pool_t, seq.blocks_t),
                                        (self.draft, self.pool_d, seq.blocks_d)):
                model(idx, pos, pool.views(torch.tensor([blocks]), pos), last_only=True)
        self.seqs.append(seq)
        return seq

    def active(self) -> List[_Seq]:
        return [s for s in self.seqs if not s.done]

    # ---- one round --------------------------------------------------------------------------------
    def _remaining(self, s: _Seq) -> int:
        return min(s.max_new - (len(s.tokens) - s.start), self.limit - len(s.tokens))

    def _finish_check(self, s: _Seq) -> None:
        if self._remaining(s) <= 0 or (s.eos_id is not None and s.eos_id in s.tokens[s.start:]):
            if s.eos_id is not None and s.eos_id in s.tokens[s.start:]:
                cut = s.tokens.index(s.eos_id, s.start) + 1
                del s.tokens[cut:]
            s.done = True
            self.release(s)

    @torch.no_grad()
    def round(self) -> int:
        """One draft-then-verify round for every active sequence. Returns the tokens committed."""
        seqs = self.active()
        if not seqs:
            return 0
        b = len(seqs)
        k_eff = [max(0, min(self.k, self._remaining(s) - 1)) for s in seqs]
        k = max(k_eff)
        for s in seqs:
            self._grow(s, len(s.tokens) + k)
        res = spec_round(self.target, self.draft, self.pool_t, self.pool_d, [s.tokens for s in seqs],
                         [s.blocks_t for s in seqs], [s.blocks_d for s in seqs], k_eff,
                         [s.temperature for s in seqs], _GeneratorDraws(self.gen, b, k, self.target.cfg.vocab_size,
                                                                        self.dev))
        committed = 0
        rows = res.tolist()
        for r, s in enumerate(seqs):
            a = rows[r][0]
            new = rows[r][1: a + 2]
            s.tokens += new
            committed += len(new)
            self.stats["proposed"] += k_eff[r]
            self.stats["accepted"] += a
            self._finish_check(s)
        self.stats["rounds"] += 1
        return committed

    def run(self) -> None:
        while self.active():
            self.round()


@torch.no_grad()
def speculative_generate_batch(target, draft, prompts: List[List[int]], max_new_tokens, k: int = 4,
                               temperature=0.0, generator: Optional[torch.Generator] = None,
                               block_size: int = 16, num_blocks: Optional[int] = None):
    """Batched speculative decoding; returns (list of new-token lists, stats)."""
    n = len(prompts)
    max_new = list(max_new_tokens) if isinstance(max_new_tokens, (list, tuple)) else [max_new_tokens] * n
    temps = list(temperature) if isinstance(temperature, (list, tuple)) else [temperature] * n
    if num_blocks is None:
        limit = min(target.cfg.max_seq_len, draft.cfg.max_seq_len)
        num_blocks = sum(-(-min(len(p) + m + k + 1, limit + k) // block_size) + 1 for p, m in zip(prompts, max_new))
    sb = SpeculativeBatch(target, draft, num_blocks, block_size, k, generator=generator)
    seqs = [sb.add(p, m, t) for p, m, t in zip(prompts, max_new, temps)]
    sb.run()
    return [s.tokens[s.start:] for s in seqs], sb.stats
