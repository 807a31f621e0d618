"""Continuous batching over the paged KV pool (engine.py:1-139 in the reference).

Each step prefills one waiting request or decodes one token for every running request in one
batched forward; when the pool runs out during decoding the most recently started request is
preempted (its blocks are freed, it is re-prefilled later from prompt + output). Scheduling and the
order of random draws are the reference's; the forwards, the KV writes and the sampling are HIP
kernels, and a decode step samples every row in one launch with a single device-to-host copy.

With a draft model (`Engine(..., draft=..., k=...)`) a decode step is one batched draft-then-verify
round over the running requests instead (speculative.py:53-85 for a batch): each request proposes up
to k_eff = min(k, remaining - 1) tokens, the k+1 window is reserved in both pools before the round
(preempting as above when a pool runs out), and EOS, max_new_tokens and max_seq_len stop a request
exactly where one-token decoding would. The random numbers of a request come from its own stream,
keyed by (seed, request id, position) and drawn on the device by a counter-based generator
(ops.keyed_noise): each use has a fixed slot (draft step i, the uniforms, the final draw, the
prefill draw), so a request's tokens do not depend on which other requests share the batch nor on
the round's k. (A recompute preemption re-prefills and samples the next token from the prefill
logits, as one-token decoding does; that moves the request's round boundaries, so at T > 0 a
preempted request continues with a different, equally valid sample.)
"""

from collections import deque
from dataclasses import dataclass, field
from typing import Deque, Dict, List, Optional

import torch

from . import ops
from ._lib import to_device
from .model import ForgeModel, prefill_packed
from .paged import BlockList, PagedKVPool, block_table
from .sampling import exp_noise
from .speculative import _bucket, _launch_round, _round_state, shared_layers, spec_round


@dataclass
class Request:
    id: int
    prompt: List[int]
    max_new_tokens: int
    eos_id: Optional[int] = None
    temperature: float = 0.0
    output: List[int] = field(default_factory=list)
    blocks: List[int] = field(default_factory=BlockList)
    cached: int = 0
    finished: bool = False
    blocks_d: List[int] = field(default_factory=BlockList)   # draft pool blocks (speculative engine)
    preempted: int = 0                                        # times this request was preempted
    stream: int = -1                                          # id of its random stream (speculative engine)


class _TokenTail:
    """What a round reads of a request's tokens (prompt + output): their number and the last two."""

    __slots__ = ("n", "tail")

    def __init__(self, req: "Request"):
        self.n = len(req.prompt) + len(req.output)
        self.tail = (req.prompt + req.output)[-2:] if len(req.output) < 2 else req.output[-2:]

    def __len__(self) -> int:
        return self.n

    def __getitem__(self, i: int) -> int:
        if not -len(self.tail) <= i < 0:
            raise IndexError("only the last two tokens are kept")
        return self.tail[i]


def _stream_key(seed: int, rid: int, pos: int) -> int:
    """Key of request `rid`'s random stream for the round (or prefill) that starts at position `pos`."""
    return ((seed * 1_000_003 + rid) * 1_000_033 + pos) % (1 << 62)


# Slots of a key's stream: draft step i uses slot i; the acceptance's uniforms and its final Exp(1)
# row, and the draw after a (re)prefill, have slots of their own past any draft step.
SLOT_U, SLOT_FINAL, SLOT_PREFILL = 1 << 20, (1 << 20) + 1, (1 << 20) + 2


class _KeyedDraws:
    """A speculative round's random numbers, one stream per request keyed by (seed, request id,
    position): the draft steps' Exp(1) rows (slot i for step i), the uniforms u (slot SLOT_U, column i
    for proposal i) and the final Exp(1) row (SLOT_FINAL). Every value depends only on the request's
    key, the slot and the column, never on the batch or the round's k. Greedy requests get numbers too;
    the kernels ignore them. The round draws them on the device in its own kernels (and so inside its
    HIP graph): the key of a round that starts at length n is base(seed, request id) + n modulo 2^62
    (_stream_key), formed from the bases staged with the round's tables and the lengths the round
    holds, staged by the host or advanced on the device (fs_spec_advance) for a queued round."""

    def __init__(self, reqs, seed):
        self.kbase = [_stream_key(seed, r.stream, 0) for r in reqs]

    @staticmethod
    def fill_in_round(st) -> None:
        """Keys of st's rows from their staged bases and lengths, then their numbers (rows past the
        batch have base 0 and length 0; the kernels ignore their numbers)."""
        torch.add(st.d["kbase"], st.d["n"], out=st.keys)
        st.keys.bitwise_and_((1 << 62) - 1)
        if st.k:
            ops.keyed_noise(st.keys, 0, st.noise_d[: st.k], ops.RNG_EXP)
        ops.keyed_noise(st.keys, SLOT_U, st.u, ops.RNG_UNIFORM)
        ops.keyed_noise(st.keys, SLOT_FINAL, st.e, ops.RNG_EXP)


class Engine:
    """key_layout: the pools' key storage (`PagedKVPool`): "slots" keeps `pool.k` in the reference's
    shape; "groups" streams faster in attention, with the same tokens."""

    def __init__(self, model: ForgeModel, num_blocks: int, block_size: int = 16, max_batch: int = 8, seed: int = 0,
                 draft: Optional[ForgeModel] = None, k: int = 4, draft_num_blocks: Optional[int] = None,
                 graphs: bool = True, share_kv: Optional[bool] = None, key_layout: str = "slots"):
        self.model, self.cfg = model, model.cfg
        self.pool = PagedKVPool(self.cfg, num_blocks, block_size, tp=model.tp, dtype=model.dtype, device=model.device,
                                key_layout=key_layout)
        self.max_batch = max_batch
        self.generator = torch.Generator().manual_seed(seed)
        self.waiting: Deque[Request] = deque()
        self.running: List[Request] = []
        self.requests: Dict[int, Request] = {}
        self.steps = self.preemptions = self.peak_running = self.peak_blocks = 0
        # speculative decoding (optional): the draft keeps its own pool, as speculative.py:46 keeps kv_d,
        # unless it is an early-exit draft of the model (share_kv None or True): then it uses the model's
        # pool for the blocks they share (SpeculativeBatch's share_kv; the tokens are the same)
        self.draft, self.k, self.seed = draft, k, seed
        self.shared = False
        self.graphs = graphs   # speculative rounds: replay each round shape from a captured HIP graph
        self.limit = self.cfg.max_seq_len
        self.stats = {"rounds": 0, "proposed": 0, "accepted": 0}
        if draft is not None:
            if draft.cfg.vocab_size != self.cfg.vocab_size:
                raise ValueError("target and draft must share a vocabulary")
            if k < 1:
                raise ValueError("k must be at least 1")
            n_shared = shared_layers(model, draft)
            if share_kv and not n_shared:
                raise ValueError("share_kv needs an early-exit draft of the model (early_exit_draft)")
            self.shared = bool(n_shared) if share_kv is None else bool(share_kv)
            self.pool_d = self.pool if self.shared else PagedKVPool(
                draft.cfg, draft_num_blocks or num_blocks, block_size, dtype=model.dtype, device=model.device,
                key_layout=key_layout)
            self.limit = min(self.cfg.max_seq_len, draft.cfg.max_seq_len)

    # ---- public API ---------------------------------------------------------------------------------
    def add_request(self, prompt: List[int], max_new_tokens: int, eos_id: Optional[int] = None,
                    temperature: float = 0.0, stream_id: Optional[int] = None) -> int:
        """Queue a request (engine.py:48-55); returns its id. stream_id (speculative engine, optional):
        the id its random numbers are keyed by, default the request id; two requests with the same
        stream id, prompt and settings sample the same tokens in any engine (absent preemption)."""
        if not 0 < len(prompt) < self.limit:
            raise ValueError(f"prompt length must be in 1..{self.limit - 1}")
        if self.pool.blocks_for(len(prompt) + 1) > self.pool.allocator.num_blocks or (
                self.draft is not None and self.pool_d.blocks_for(len(prompt) + 1) > self.pool_d.allocator.num_blocks):
            raise ValueError("prompt does not fit in the block pool")
        req = Request(len(self.requests), list(prompt), max_new_tokens, eos_id, temperature)
        req.stream = req.id if stream_id is None else int(stream_id)
        self.requests[req.id] = req
        self.waiting.append(req)
        return req.id

    def has_work(self) -> bool:
        return bool(self.waiting or self.running)

    def run(self) -> Dict[int, List[int]]:
        """Steps until every request has finished (engine.py:57-60). With a draft, a run of speculative
        rounds whose successors are known in advance is queued back to back (_queued_rounds): the same
        steps, tokens, preemptions and counters as calling step() each time."""
        while self.has_work():
            if not (self.draft is not None and self._queued_rounds()):
                self.step()
        return {rid: r.output for rid, r in self.requests.items()}

    def step(self) -> None:
        """One engine step (engine.py:62-77); when the reference would prefill several waiting requests
        in consecutive steps, those steps run here at once (_prefill_run)."""
        if self.waiting and len(self.running) < self.max_batch and self._prefill_run():
            return
        self.steps += 1
        if self.running:
            if self.draft is not None:
                self._spec_decode()
            else:
                self._decode()
        elif self.waiting:
            raise RuntimeError("the head request cannot be scheduled: the block pool is too small")
        self._note_peaks()

    def _note_peaks(self, held_back: int = 0) -> None:
        """Peak running requests and peak blocks in use after a step; held_back: blocks allocated ahead
        for requests whose prefill steps come later."""
        used = self.pool.allocator.num_blocks - self.pool.allocator.num_free - held_back
        self.peak_running, self.peak_blocks = max(self.peak_running, len(self.running)), max(self.peak_blocks, used)

    # ---- scheduling ---------------------------------------------------------------------------------
    PACK_TOKENS = 32768   # tokens per packed prefill forward

    def _prefill_run(self) -> int:
        """The prefill steps the reference would take one after another from here (engine.py:80-95): the
        head request is prefilled while fewer than max_batch requests run and its blocks fit; each one
        is a step of its own. They are admitted in the reference's order, computed in packed forwards
        (model.prefill_packed, bit-identical to one forward per request), then each request's first
        token is sampled in order and the step's counters updated as if it had run alone. Admission
        counts every admitted request as running and its blocks as held, so a request the reference
        would admit only because an earlier one finished at its first token is left to the next call.
        Returns the number of steps taken (0: the head request does not fit)."""
        spec = self.draft is not None
        admitted = []
        while self.waiting and len(self.running) + len(admitted) < self.max_batch:
            req = self.waiting[0]
            tokens = req.prompt + req.output
            need = self.pool.blocks_for(len(tokens))
            need_d = self.pool_d.blocks_for(len(tokens)) if spec and not self.shared else 0
            if need > self.pool.allocator.num_free or (spec and need_d > self.pool_d.allocator.num_free):
                break
            self.waiting.popleft()
            req.blocks = BlockList(self.pool.allocator.allocate(need))
            if need_d:
                req.blocks_d = BlockList(self.pool_d.allocator.allocate(need_d))
            admitted.append((req, tokens))
        if not admitted:
            return 0
        logits = []
        i = 0
        while i < len(admitted):   # packed forwards of up to PACK_TOKENS tokens
            chunk, total = [], 0
            while i < len(admitted) and (not chunk or total + len(admitted[i][1]) <= self.PACK_TOKENS):
                chunk.append(admitted[i])
                total += len(admitted[i][1])
                i += 1
            toks = [t for _, t in chunk]
            logits.append(prefill_packed(self.model, self.pool, toks, [r.blocks for r, _ in chunk]))
            if spec and not self.shared:   # (a shared draft's blocks were written by the model's prefill)
                prefill_packed(self.draft, self.pool_d, toks, [r.blocks_d for r, _ in chunk])
        logits = torch.cat(logits, 0)
        held = sum(len(r.blocks) for r, _ in admitted)
        # the first tokens of a speculative engine's requests come from their own streams: drawn for all
        # of them at once (each row's numbers depend only on its key)
        firsts = self._first_tokens([r for r, _ in admitted], logits) if spec else None
        for j, (req, tokens) in enumerate(admitted):
            self.steps += 1
            held -= len(req.blocks)
            req.cached = len(tokens)
            if spec:
                self._push(req, firsts[j])
            else:
                self._append([req], logits[j: j + 1])
            if not req.finished:
                self.running.append(req)
            self._note_peaks(held)
        return len(admitted)

    # ---- speculative decoding ---------------------------------------------------------------------
    def _remaining(self, req: Request) -> int:
        return min(req.max_new_tokens - len(req.output), self.limit - len(req.prompt) - len(req.output))

    def _k_eff(self, req: Request) -> int:
        return max(0, min(self.k, self._remaining(req) - 1))

    def _release(self, req: Request) -> None:
        self.pool.allocator.release(req.blocks)
        req.blocks = BlockList()
        if self.draft is not None and not self.shared:
            self.pool_d.allocator.release(req.blocks_d)
            req.blocks_d = BlockList()

    def _spec_decode(self) -> None:
        """One draft-then-verify round over the running requests. Every request first gets the blocks
        of its k+1 window (positions up to n-1+k_eff) in both pools; when a pool runs out the most
        recently started request is preempted (engine.py:100-118)."""
        i = 0
        while i < len(self.running):
            req = self.running[i]
            span = len(req.prompt) + len(req.output) + self._k_eff(req)
            need_t = self.pool.blocks_for(span) - len(req.blocks)
            need_d = 0 if self.shared else self.pool_d.blocks_for(span) - len(req.blocks_d)
            if need_t > self.pool.allocator.num_free or need_d > self.pool_d.allocator.num_free:
                if len(self.running) == 1:
                    raise RuntimeError("the block pool is too small to hold even one sequence of this length")
                victim = self.running.pop()
                self._release(victim)
                victim.cached = 0
                victim.preempted += 1
                self.waiting.appendleft(victim)
                self.preemptions += 1
                continue   # retry (or, if the victim was this request, the loop ends or moves on)
            if need_t > 0:
                req.blocks += self.pool.allocator.allocate(need_t)
            if need_d > 0:
                req.blocks_d += self.pool_d.allocator.allocate(need_d)
            i += 1
        if not self.running:
            return
        batch = list(self.running)
        k_eff = [self._k_eff(r) for r in batch]
        tokens = [_TokenTail(r) for r in batch]
        temps = [float(r.temperature) for r in batch]
        draws = _KeyedDraws(batch, self.seed)
        res = spec_round(self.model, self.draft, self.pool, self.pool_d, tokens, [r.blocks for r in batch],
                         [r.blocks_d for r in batch], k_eff, temps, draws, graphs=self.graphs, k=self.k)
        self.stats["rounds"] += 1
        for r, (req, row) in enumerate(zip(batch, res.tolist())):
            a = row[0]
            self.stats["proposed"] += k_eff[r]
            self.stats["accepted"] += a
            for token in row[1: a + 2]:
                self._push(req, token)
                if req.finished:
                    break
            req.cached = len(req.prompt) + len(req.output) - 1
            if req.finished:
                self.running.remove(req)

    # ---- speculative rounds queued back to back ---------------------------------------------------
    def _next_round_known(self, batch: List[Request]) -> bool:
        """Whether, from the state at the start of a round over `batch`, the step after it is known to
        be another round over the same requests: no row can finish in the round (each has at least
        k + 2 tokens left and no EOS id; a round commits at most k + 1 tokens) and step() would not try
        a prefill first (no request waits, or every batch slot is taken)."""
        if self.waiting and len(self.running) < self.max_batch:
            return False
        return all(r.eos_id is None and self._remaining(r) >= self.k + 2 for r in batch)

    def _reserve(self, batch: List[Request], spans: List[int]) -> Optional[int]:
        """Blocks for `spans[i]` tokens of each request in both pools, taken in batch order, if they all
        fit (else nothing is taken and None returned): the number taken from the model's pool."""
        need_t = [max(0, self.pool.blocks_for(s) - len(r.blocks)) for r, s in zip(batch, spans)]
        need_d = [] if self.shared else [max(0, self.pool_d.blocks_for(s) - len(r.blocks_d))
                                         for r, s in zip(batch, spans)]
        if sum(need_t) > self.pool.allocator.num_free or (need_d and sum(need_d) > self.pool_d.allocator.num_free):
            return None
        for r, n in zip(batch, need_t):
            if n:
                r.blocks += self.pool.allocator.allocate(n)
        for r, n in zip(batch, need_d):
            if n:
                r.blocks_d += self.pool_d.allocator.allocate(n)
        return sum(need_t)

    def _trim(self, batch: List[Request], base: List[tuple]) -> None:
        """Give back what a reservation took beyond the blocks _spec_decode would hold now: each
        request keeps max(its blocks before the reservation, the blocks of its next window)."""
        for r, (n_t, n_d) in zip(batch, base):
            span = len(r.prompt) + len(r.output) + self._k_eff(r)
            for pool, blocks, n0 in ((self.pool, r.blocks, n_t),) + (
                    () if self.shared else ((self.pool_d, r.blocks_d, n_d),)):
                keep = max(n0, pool.blocks_for(span))
                if len(blocks) > keep:
                    extra = blocks[keep:]
                    del blocks[keep:]
                    pool.allocator.release(extra)

    def _queued_rounds(self) -> int:
        """Speculative rounds queued back to back. While the step after the current round is known to
        be another round over the same requests (_next_round_known), that round is launched before the
        current one's tokens are read back: fs_spec_advance writes its inputs on the device, where its
        keys are formed too (_KeyedDraws), so the GPU does not wait for the host between rounds. A
        queued round's blocks are reserved for the most tokens the round before it can commit; once
        those are known the excess goes back (_trim), so each step leaves the pools' counts, the tokens
        and the counters as step() leaves them (block ids may differ). Returns the steps taken; 0 when
        the current step is not such a round (or its blocks would need a preemption): step() takes it."""
        batch = list(self.running)
        if not batch or not self._next_round_known(batch):
            return 0
        k, b = self.k, len(batch)
        # the first round's blocks exactly as _spec_decode takes them (all fit: no preemption)
        if self._reserve(batch, [len(r.prompt) + len(r.output) + k for r in batch]) is None:
            return 0
        blocks_t = [r.blocks for r in batch]
        blocks_d = blocks_t if self.shared else [r.blocks_d for r in batch]
        temps = [float(r.temperature) for r in batch]
        draws = _KeyedDraws(batch, self.seed)
        st = _round_state(self.model, self.draft, self.pool, self.pool_d, b, k, blocks_t, blocks_d,
                          any(t > 0 for t in temps), keyed=True)
        st.stage([_TokenTail(r) for r in batch], [k] * b, temps, blocks_t, blocks_d, slot=0,
                 budget=[self._remaining(r) for r in batch], eos=[-1] * b, kbase=draws.kbase)
        st.dev.copy_(st.hosts[0], non_blocking=True)

        def launch(j):
            _launch_round(self.model, self.draft, self.pool, self.pool_d, st, b, draws, self.graphs)
            st.res_hosts[j % 2].copy_(st.res, non_blocking=True)
            ev = torch.cuda.Event()
            ev.record()
            return j, ev

        pending = [launch(0)]
        steps = 0
        while pending:
            j, ev = pending.pop(0)
            held, base = 0, None
            if self._next_round_known(batch):   # the host state is round j's start
                # round j+1 starts at most k+1 tokens later and writes k past its start
                spans = [min(len(r.prompt) + len(r.output) + 2 * k + 1, self.limit) for r in batch]
                wt = _bucket(max(max(len(r.blocks), self.pool.blocks_for(x)) for r, x in zip(batch, spans)), 64)
                wd = wt if self.shared else _bucket(
                    max(max(len(r.blocks_d), self.pool_d.blocks_for(x)) for r, x in zip(batch, spans)), 64)
                if (wt, wd) == (st.wt, st.wd):
                    base = [(len(r.blocks), len(r.blocks_d)) for r in batch]
                    held = self._reserve(batch, spans)
                if held is not None and base is not None:
                    slot = (j + 1) % 2
                    st.stage_host(temps, blocks_t, blocks_d, slot, draws.kbase)
                    st.dev[st.host_off:].copy_(st.hosts[slot][st.host_off:], non_blocking=True)
                    pending.append(launch(j + 1))
                else:
                    held, base = 0, None
            # round j's tokens, as _spec_decode takes them (a request can finish only in a round with
            # no successor queued)
            ev.synchronize()
            rows = st.res_hosts[j % 2][:b].tolist()
            self.steps += 1
            for req, row in zip(batch, rows):
                a = row[0]
                self.stats["proposed"] += self._k_eff(req)
                self.stats["accepted"] += a
                for token in row[1: a + 2]:
                    self._push(req, token)
                    if req.finished:
                        break
                req.cached = len(req.prompt) + len(req.output) - 1
                if req.finished:
                    if pending:
                        raise RuntimeError("internal error: a request finished in a round with a successor queued")
                    self.running.remove(req)
            self.stats["rounds"] += 1
            self._note_peaks(held)
            if base is not None:
                self._trim(batch, base)
            steps += 1
        return steps

    def _first_tokens(self, reqs: List[Request], logits: torch.Tensor) -> List[int]:
        """The token after each request's (re)prefill (logits row i for reqs[i]), from the request's own
        stream at its current length (slot SLOT_PREFILL), in one launch; greedy rows take the argmax."""
        v, dev = logits.shape[-1], logits.device
        temps = [float(r.temperature) for r in reqs]
        noise = None
        if any(t > 0 for t in temps):
            keys = [_stream_key(self.seed, r.stream, len(r.prompt) + len(r.output)) for r in reqs]
            noise = ops.keyed_noise(to_device(torch.tensor(keys, dtype=torch.int64), dev), SLOT_PREFILL,
                                    torch.empty((len(reqs), v), device=dev), ops.RNG_EXP)
        t_dev = to_device(torch.tensor(temps, dtype=torch.float32), dev)
        return ops.sample_logits(logits, t_dev, noise).tolist()

    def _push(self, req: Request, token: int) -> None:
        """Append one token; finish the request at max_new_tokens, EOS or max_seq_len (engine.py:132-139)."""
        req.output.append(token)
        total = len(req.prompt) + len(req.output)
        if len(req.output) >= req.max_new_tokens or token == req.eos_id or total >= self.limit:
            req.finished = True
            self._release(req)

    def _decode(self) -> None:
        bs = self.pool.block_size
        i = 0
        while i < len(self.running):
            req = self.running[i]
            if req.cached % bs == 0 and req.cached // bs == len(req.blocks):
                if self.pool.allocator.num_free == 0:
                    if len(self.running) == 1:
                        raise RuntimeError("the block pool is too small to hold even one sequence of this length")
                    victim = self.running.pop()
                    self.pool.allocator.release(victim.blocks)
                    victim.blocks, victim.cached = BlockList(), 0
                    victim.preempted += 1
                    self.waiting.appendleft(victim)
                    self.preemptions += 1
                    if victim is req:
                        continue
                    if not self.running:
                        return
                    continue
                req.blocks += self.pool.allocator.allocate(1)
            i += 1
        if not self.running:
            return
        tables = block_table([r.blocks for r in self.running], self.pool.device)
        positions = torch.tensor([[r.cached] for r in self.running])
        idx = torch.tensor([[r.output[-1]] for r in self.running])
        logits = self.model(idx, positions, self.pool.views(tables, positions), last_only=True)
        batch = list(self.running)
        for req in batch:
            req.cached += 1
        self._append(batch, logits[:, -1])
        for req in batch:
            if req.finished:
                self.running.remove(req)

    def _append(self, reqs: List[Request], logits: torch.Tensor) -> None:
        """Sample one token per request in one launch. Noise rows are drawn from the engine's generator
        in request order, only for sampled (T > 0) requests, as per-row torch.multinomial calls would."""
        v = logits.shape[-1]
        temps = [float(r.temperature) for r in reqs]
        noise = None
        if any(t > 0 for t in temps):
            rows = [exp_noise((v,), self.generator, "cpu") if t > 0 else torch.ones(v) for t in temps]
            noise = to_device(torch.stack(rows), logits.device)
        t_dev = to_device(torch.tensor(temps, dtype=torch.float32), logits.device)
        toks = ops.sample_logits(logits, t_dev, noise).tolist()
        for req, token in zip(reqs, toks):
            self._push(req, token)
