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

from collections import OrderedDict
from typing import List, Optional, Sequence, Tuple

import numpy as np
import torch

from . import ops
from .kv import new_contiguous_cache
from .model import prefill_packed
from .paged import BlockList, OutOfBlocks, PagedKVPool
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

    # the same numbers drawn straight into the round's buffers (contiguous (b, V) / (b, max(k, 1)) slices)
    def draft_into(self, i, out):
        out.exponential_(generator=self.gen)

    def accept_into(self, u, e):
        u.uniform_(generator=self.gen)
        e.exponential_(generator=self.gen)


def shared_layers(target, draft) -> int:
    """How many leading blocks an early-exit draft shares with its target (the same modules, with the
    same embedding), 0 if it is not such a draft. Those blocks compute the same keys, values and
    residual streams for the same tokens in either model, so the draft can read and write the target's
    cache for them instead of keeping its own (the reference keeps a separate cache, speculative.py:46:
    the tokens do not change, only the memory and the work)."""
    n = draft.cfg.n_layers
    if (n > target.cfg.n_layers or draft.tok_emb is not target.tok_emb or draft.cfg.d_model != target.cfg.d_model
            or draft.cfg.max_seq_len != target.cfg.max_seq_len):
        return 0
    return n if all(draft.layers[i] is target.layers[i] for i in range(n)) else 0


def _bucket(x: int, q: int) -> int:
    return max(q, -(-x // q) * q)


class _RoundState:
    """What one shape of round keeps between rounds: the pinned host staging and the device copy of
    the round's inputs (one host-to-device copy per round), the buffers that pass results between the
    round's phases, the random-number buffers, and, from its second use on, one HIP graph per phase
    (each draft step, then the verify pass with the acceptance), replayed on those fixed addresses.

    The shape is (b, k, table widths, sampling, statistics path); b is padded to a multiple of 8 and
    the table widths to multiples of 64 blocks, so that growing contexts and a changing batch reuse a
    few graphs. Padding rows have k_eff 0 and only -1 positions (no KV write, no keys), temperature
    0, and their results are dropped."""

    def __init__(self, dev, dtype, b, k, wt, wd, v, sampling, fused, parts_d, parts_t, n_shared=0, d_model=0,
                 keyed=False):
        self.b, self.k, self.wt, self.wd, self.v = b, k, wt, wd, v
        self.sampling, self.fused = sampling, fused
        # keyed: the round's random numbers are drawn inside its kernels (and graph) from per-row key
        # bases staged with the tables and the rows' lengths (the Engine's keyed streams)
        self.keyed = keyed
        # a draft sharing the target's first n_shared blocks and their cache leaves its residual
        # streams after them here, one per fed token (the verify pass continues from them)
        self.n_shared = n_shared
        self.hidden = torch.empty((b, max(k, 1), d_model), dtype=dtype, device=dev) if n_shared else None
        # staging: int64 ids [b, 2] (prev, last) and last [b]; int32 k_eff [b], draft positions [b, 2] (step 0)
        # then [k-1, b] (steps 1..k-1; [k, b], steps 0..k-1, with a shared cache), verify positions
        # [b, k+1], tables [b, wt] and [b, wd];
        # float32 temperatures [b]; int64 key bases [b] (keyed rounds)
        # a draft on the target's cache feeds only `last` in step 0 (the verify pass has cached every
        # position before it), so its step 0 is staged with the others
        km = k if n_shared else max(k - 1, 0)
        self.km = km
        # The spans up to `temps` are what a round computes from the previous one (fs_spec_advance
        # writes them on the device when rounds are queued back to back, with each row's length n,
        # token budget, EOS id and done flag); the tables and temperatures after them always come from
        # the host. Two pinned host buffers: a queued round's copy may still be pending while the next
        # is staged.
        spans = [("ids", np.int64, (b, 2)), ("last", np.int64, (b,)), ("keff", np.int32, (b,)), ("pos0", np.int32, (b, 2)),
                 ("posd", np.int32, (km, b)), ("posv", np.int32, (b, k + 1)), ("n", np.int32, (b,)),
                 ("budget", np.int32, (b,)), ("eos", np.int32, (b,)), ("done", np.int32, (b,)),
                 ("temps", np.float32, (b,)), ("kbase", np.int64, (b,)), ("tab_t", np.int32, (b, wt))]
        if not n_shared:   # a draft on the target's cache reads the target's table
            spans.append(("tab_d", np.int32, (b, wd)))
        off, lay = 0, {}
        for name, dt, shape in spans:
            nbytes = int(np.prod(shape)) * np.dtype(dt).itemsize
            lay[name] = (off, nbytes, dt, shape)
            off += -(-nbytes // 16) * 16
        self.host_off = lay["temps"][0]
        self.hosts = [torch.empty(max(off, 16), dtype=torch.uint8, pin_memory=True) for _ in range(2)]
        self.dev = torch.empty(max(off, 16), dtype=torch.uint8, device=dev)
        tdt = {np.int64: torch.int64, np.int32: torch.int32, np.float32: torch.float32}
        self.hs, self.d = [{}, {}], {}
        for name, (o, nbytes, dt, shape) in lay.items():
            for i in range(2):
                self.hs[i][name] = self.hosts[i].numpy()[o: o + nbytes].view(dt).reshape(shape)
            self.d[name] = self.dev[o: o + nbytes].view(tdt[dt]).view(shape)
        if n_shared:
            self.d["tab_d"] = self.d["tab_t"]
        for h in self.hs:
            h["tab_t"].fill(0)
            if "tab_d" in lay:
                h["tab_d"].fill(0)
        # what each table row of each host buffer holds: (block list, its version, entries copied)
        self._staged = [{}, {}]
        kk = max(k, 1)
        self.keys = torch.zeros((b,), dtype=torch.int64, device=dev)
        self.u = torch.zeros((b, kk), dtype=torch.float32, device=dev)
        self.e = torch.ones((b, v), dtype=torch.float32, device=dev)
        self.noise_d = torch.ones((kk, b, v), dtype=torch.float32, device=dev) if sampling else None
        # results passed between phases
        self.dft_logits = torch.empty((b, k, v), dtype=dtype, device=dev)
        self.draft_tok = torch.empty((b, k), dtype=I32, device=dev)
        self.tok64 = torch.empty((max(k, 1), b), dtype=torch.int64, device=dev)   # step i's tokens, as ids
        if fused:
            # draft step i writes its rows' records into parts_d[:, i]; one merge after the last step
            self.parts_d = torch.empty((b, k, parts_d, 4), dtype=I32, device=dev)
            self.parts_t = torch.empty((b * (k + 1), parts_t, 4), dtype=I32, device=dev)
            self.row_stats = torch.empty((b, 2 * k + 1, 4), dtype=I32, device=dev)
        self.res_hosts = [torch.empty((b, k + 2), dtype=torch.int32, pin_memory=True) for _ in range(2)]
        self.res = torch.empty((b, k + 2), dtype=I32, device=dev)   # the verify phase's output
        self.graph = None          # the round's kernels (k+1 phases, fs_spec_advance) in one graph
        self.phase_graphs = None   # one graph per phase, captured on request (phase timing)
        self.uses = 0

    def stage(self, tokens, k_eff, temps, blocks_t, blocks_d, slot=0, budget=None, eos=None, kbase=None) -> None:
        """Write one round's inputs into pinned staging buffer `slot` (rows past len(tokens) are padding,
        and done). budget, eos: each row's remaining tokens and EOS id (-1: none), for rounds whose
        successors are advanced on the device. kbase: each row's key base (keyed rounds)."""
        b, k = len(tokens), self.k
        h = self.hs[slot]
        n = np.array([len(t) for t in tokens], dtype=np.int64)
        keff = np.array(k_eff, dtype=np.int64)
        ids = h["ids"]
        ids.fill(0)
        ids[:b, 0] = [t[-2] if len(t) > 1 else 0 for t in tokens]
        ids[:b, 1] = [t[-1] for t in tokens]
        h["last"][:] = ids[:, 1]
        h["keff"].fill(0)
        h["keff"][:b] = keff
        # step 0 re-feeds (prev, last) at (n-2, n-1); step i feeds x_{i-1} at n-1+i; the verify pass
        # feeds [last, x_0 .. x_{k-1}] at n-1 .. n-1+k; positions past a row's k_eff are -1
        h["pos0"].fill(-1)
        h["pos0"][:b] = np.where(keff[:, None] > 0, np.stack([np.where(n > 1, n - 2, -1), n - 1], 1), -1)
        h["posd"].fill(-1)
        first = 0 if self.n_shared else 1
        for i in range(first, k):
            h["posd"][i - first, :b] = np.where(keff > i, n - 1 + i, -1)
        t_ = np.arange(k + 1)[None, :]
        h["posv"].fill(-1)
        h["posv"][:b] = np.where(t_ <= keff[:, None], n[:, None] - 1 + t_, -1)
        h["n"].fill(0)
        h["n"][:b] = n
        # (without a budget the rows stay live in the round's device-side advance: its next-round
        # inputs are then the real round's successor, which a host-staged next round overwrites)
        h["budget"].fill(0)
        h["budget"][:b] = budget if budget is not None else 1 << 30
        h["eos"].fill(-1)
        h["eos"][:b] = eos if eos is not None else -1
        h["done"].fill(1)
        h["done"][:b] = 0
        self.stage_host(temps, blocks_t, blocks_d, slot, kbase)

    def stage_host(self, temps, blocks_t, blocks_d, slot, kbase=None) -> None:
        """The host-owned spans of staging buffer `slot`: temperatures, key bases and block tables."""
        h, b = self.hs[slot], len(temps)
        h["temps"].fill(0)
        h["temps"][:b] = temps
        h["kbase"].fill(0)
        if kbase is not None:
            h["kbase"][:b] = kbase
        tables = (("tab_t", blocks_t),) if self.n_shared else (("tab_t", blocks_t), ("tab_d", blocks_d))
        for name, lists in tables:
            # rows keep last round's entries: a row whose block list only grew gets its new blocks
            tab, prev, rows = h[name], self._staged[slot].get(name, ()), []
            for r, x in enumerate(lists):
                p = prev[r] if r < len(prev) else None
                if isinstance(x, BlockList):
                    a, ver = x.array(), x.version
                    m = a.shape[0]
                    if p is not None and p[0] is x and p[1] == ver and p[2] <= m:
                        if m > p[2]:
                            tab[r, p[2]: m] = a[p[2]:]
                    else:
                        tab[r, :m] = a
                        tab[r, m:] = 0
                    rows.append((x, ver, m))
                else:
                    a = np.asarray(x, dtype=np.int32)
                    tab[r, : a.shape[0]] = a
                    tab[r, a.shape[0]:] = 0
                    rows.append((None, 0, a.shape[0]))
            for r in range(len(lists), len(prev)):   # rows of sequences that left the batch
                if prev[r][2]:
                    tab[r] = 0
            self._staged[slot][name] = rows


def _round_phase(target, draft, pool_t: PagedKVPool, pool_d: PagedKVPool, st: _RoundState, phase: int):
    """The kernels of one phase of a round, reading only st's device buffers (no host copies, no host
    syncs): phase i < k is draft step i, phase k the target's verify pass over the k+1 window and the
    fused acceptance, which returns (b, k+2) int32: n_accepted, then the committed tokens (-1 padded)."""
    b, k = st.b, st.k
    d = st.d
    temps = d["temps"]
    if phase < k:
        i = phase
        if i == 0 and st.n_shared:   # the shared cache holds every position before `last`
            idx, pos = d["last"][:, None], d["posd"][0][:, None]
        elif i == 0:                  # re-feed (prev, last): the draft's own cache may lack prev
            idx, pos = d["ids"], d["pos0"]
        else:
            idx = st.tok64[i - 1][:, None]
            pos = d["posd"][i if st.n_shared else i - 1][:, None]
        logits = draft._run(idx, pos, pool_d.views(d["tab_d"], pos), last_only=True,
                            head_stats=(temps, st.parts_d[:, i]) if st.fused else None, out=st.dft_logits[:, i],
                            hidden_out=st.hidden[:, i] if st.n_shared else None)
        ops.sample_logits(logits, temps, st.noise_d[i] if st.sampling else None, out32=st.draft_tok[:, i],
                          out64=st.tok64[i])
        if st.fused and i == k - 1:   # draft row (b, i) is record b*k + i: sequence b's draft rows k+1 .. 2k
            ops.row_stats_merge(st.parts_d.view(b * k, -1, 4), st.row_stats, k, 2 * k + 1, k + 1)
        return None
    last = d["last"]
    idx = torch.cat([last[:, None], st.tok64[:k].t()], 1) if k else last[:, None]
    pos = d["posv"]
    temps_t = temps.repeat_interleave(k + 1) if st.fused else None
    views = pool_t.views(d["tab_t"], pos)
    stats = (temps_t, st.parts_t) if st.fused else None
    if st.n_shared and k:   # the draft has run the shared blocks for all but token k_eff of each row
        tgt_logits = target._run_verify_reusing(st.n_shared, idx, pos, views, d["keff"], st.hidden[:, :k], stats)
    else:
        tgt_logits = target._run(idx, pos, views, head_stats=stats)
    if st.fused:
        ops.row_stats_merge(st.parts_t, st.row_stats, k + 1, 2 * k + 1, 0)
    out_tok, n_acc = ops.spec_accept(tgt_logits, st.dft_logits, st.draft_tok, d["keff"], temps, st.u[:, :k], st.e,
                                     row_stats=st.row_stats if st.fused else None)
    return torch.cat([n_acc[:, None], out_tok], 1, out=st.res)


def _graph_key(model) -> tuple:
    """Which weights a captured round reads: the model object and a few parameter addresses (a model
    whose parameters were replaced by new tensors gets new graphs)."""
    blk = model.layers
    return (id(model), model.tok_emb.weight.data_ptr(), blk[0].attn.wq.weight.data_ptr(),
            blk[-1].mlp.w_down.weight.data_ptr())


_MAX_GRAPHS = 8


def _round_state(target, draft, pool_t: PagedKVPool, pool_d: PagedKVPool, b: int, k: int, blocks_t, blocks_d,
                 sampling: bool, keyed: bool = False) -> "_RoundState":
    """The _RoundState of a round's shape (created on first use; at most _MAX_GRAPHS kept per pool).
    keyed: the round draws its random numbers in its own kernels from staged key bases."""
    dev, dtype = target.device, target.dtype
    v = target.cfg.vocab_size
    n_shared = 0
    if pool_d is pool_t:   # the draft reads and writes the target's cache for the blocks they share
        n_shared = shared_layers(target, draft)
        if not n_shared:
            raise ValueError("only an early-exit draft of the target can share the target's pool")
        blocks_d = blocks_t
    bp = _bucket(b, 8)
    wt = _bucket(max(len(x) for x in blocks_t), 64)
    wd = _bucket(max(len(x) for x in blocks_d), 64)
    # The LM heads emit the logits' softmax statistics (sampling.py:13) as they write them, so the
    # acceptance does not read the 2k+1 logit rows back to normalise them.
    d = target.cfg.d_model
    pd, pt = ops.row_stats_parts(bp, v, d), ops.row_stats_parts(bp * (k + 1), v, d)
    fused = dtype == torch.bfloat16 and k > 0 and pd > 0 and pt > 0
    cache = pool_t.__dict__.setdefault("_rounds", OrderedDict())
    keyed = bool(keyed and sampling)
    key = (bp, k, wt, wd, sampling, fused, keyed, _graph_key(target), _graph_key(draft), id(pool_d))
    st = cache.get(key)
    if st is None:
        st = _RoundState(dev, dtype, bp, k, wt, wd, v, sampling, fused, pd, pt, n_shared, target.cfg.d_model, keyed)
        cache[key] = st
        while len(cache) > _MAX_GRAPHS:
            cache.popitem(last=False)
    cache.move_to_end(key)
    st.key = key
    return st


def _launch_round(target, draft, pool_t, pool_d, st: "_RoundState", b: int, draws, graphs: bool) -> None:
    """Queue one round on the current stream: the random numbers (drawn in the reference loop's order,
    or, for a keyed round, by its own first kernels), then the k+1 phases and fs_spec_advance, which
    writes the next round's inputs from this round's acceptance into the same device buffers (used by
    a round queued behind this one; a round staged by the host overwrites them). The kernels run
    eagerly on the shape's first round and are captured in one graph on its second, replayed after.
    The round's result is st.res: (b, k+2) int32, n_accepted then the committed tokens."""
    k = st.k
    if st.sampling and not st.keyed:
        if hasattr(draws, "draft_into"):
            for i in range(k):
                draws.draft_into(i, st.noise_d[i, :b])
            draws.accept_into(st.u[:b], st.e[:b])
        else:
            for i in range(k):
                st.noise_d[i, :b].copy_(draws.draft(i))
            u, e = draws.accept()
            st.u[:b, :k].copy_(u)
            st.e[:b].copy_(e)

    def kernels():
        if st.keyed:   # the round's numbers from the staged key bases and the rows' lengths
            draws.fill_in_round(st)
        for phase in range(k + 1):
            _round_phase(target, draft, pool_t, pool_d, st, phase)
        d = st.d
        ops.spec_advance(st.res, st.b, k, 0 if st.n_shared else 1, d["n"], d["budget"], d["eos"], d["done"],
                         d["ids"], d["last"], d["keff"], d["pos0"], d["posd"], d["posv"])

    if not graphs or st.uses == 0:
        kernels()
    else:
        if st.graph is None:   # the whole round in one graph: no launch gap between its phases
            torch.cuda.current_stream().synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                kernels()
            st.graph = g
        st.graph.replay()
    st.uses += 1


def capture_phase_graphs(target, draft, pool_t, pool_d, st: "_RoundState") -> list:
    """One HIP graph per phase of st's round (draft steps 0..k-1, then the verify phase), for timing a
    phase alone. Their replays rewrite what the round graph's last replay wrote: the same inputs give
    the same keys, values, logits and outputs (st.res included)."""
    if st.phase_graphs is None:
        torch.cuda.current_stream().synchronize()
        gs = []
        for phase in range(st.k + 1):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                _round_phase(target, draft, pool_t, pool_d, st, phase)
            gs.append(g)
        st.phase_graphs = gs
    return st.phase_graphs


@torch.no_grad()
def spec_round(target, draft, pool_t: PagedKVPool, pool_d: PagedKVPool, tokens: List[List[int]],
               blocks_t: List[List[int]], blocks_d: List[List[int]], k_eff: List[int], temps: List[float],
               draws, graphs: bool = True, k: Optional[int] = None) -> torch.Tensor:
    """One draft-then-verify round (speculative.py:53-85) for b sequences whose caches hold positions
    0..n-2 (n = len(tokens[r])) and whose block lists cover positions up to n-1+k_eff[r].

    Per round: k draft decode steps (step 0 re-feeds (tokens[-2], tokens[-1]) at (n-2, n-1), so a fully
    accepted round needs no catch-up forward; step i feeds x_{i-1} at n-1+i), one target verify pass
    over the k+1 window, one fused acceptance. `draws` supplies the randomness: draft(i) -> (b, V)
    Exp(1) noise of draft step i, accept() -> (u (b, k), E (b, V)); rows of greedy sequences are
    ignored, and a round with no sampled row draws nothing. Draws with a `kbase` list instead have the
    round draw its numbers in its own kernels: the bases are staged with the tables and
    `draws.fill_in_round(st)` runs first in the round (captured with it). With `graphs`, the round's kernels are
    captured in a HIP graph on the second round of a shape and replayed from then on (the same kernels
    on the same inputs: results are identical to running them one by one).
    k: the round's number of draft steps (its graph shape), at least max(k_eff); default max(k_eff).
    A caller whose rows' k_eff vary from round to round passes a fixed k so that its rounds share one
    shape: rows with k_eff < k take no part in the steps past their k_eff.
    Returns (b, k+2) int32 on the host: n_accepted, then the committed tokens (-1 padded)."""
    b = len(tokens)
    k = max(k_eff) if k is None else k
    if k < max(k_eff):
        raise ValueError(f"k = {k} < max(k_eff) = {max(k_eff)}")
    n = np.array([len(t) for t in tokens], dtype=np.int64)
    keff = np.array(k_eff, dtype=np.int64)
    limit = min(target.cfg.max_seq_len, draft.cfg.max_seq_len)
    if int((n - 1 + keff).max()) >= limit:
        raise ValueError(f"a round would write position {int((n - 1 + keff).max())} >= max_seq_len {limit}")
    sampling = any(t > 0 for t in temps)
    kbase = getattr(draws, "kbase", None)   # draws made inside the round from staged key bases
    st = _round_state(target, draft, pool_t, pool_d, b, k, blocks_t, blocks_d, sampling, keyed=kbase is not None)
    if st.n_shared:
        blocks_d = blocks_t
    # host staging -> one copy, then the round
    st.stage(tokens, k_eff, temps, blocks_t, blocks_d, kbase=kbase)
    st.dev.copy_(st.hosts[0], non_blocking=True)
    _launch_round(target, draft, pool_t, pool_d, st, b, draws, graphs)
    st.res_hosts[0].copy_(st.res, non_blocking=True)
    torch.cuda.current_stream().synchronize()
    return st.res_hosts[0][:b].clone()


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
    """Batched draft-then-verify rounds over paged KV pools.

    Sequence state lives on the host (token lists, block lists); KV, logits, draft tokens, random
    numbers and acceptance results live on the GPU. `round()` advances every active sequence by
    1 + (accepted proposals) tokens.

    share_kv: an early-exit draft (`early_exit_draft`) computes exactly the keys and values of the
    target's first blocks, so by default (None) it uses the target's pool for them instead of a pool of
    its own, needs no prefill of its own, and the verify pass continues from the draft's residual
    streams instead of re-running those blocks for the drafted tokens. The tokens are the same either
    way; False keeps the separate draft pool of the reference (speculative.py:46).

    key_layout: the pools' key storage (`PagedKVPool`); "groups" (the default here: the pools are
    internal) streams faster in attention than the reference-shaped "slots", with the same results."""

    def __init__(self, target, draft, num_blocks: int, block_size: int = 16, k: int = 4,
                 draft_num_blocks: Optional[int] = None, generator: Optional[torch.Generator] = None,
                 graphs: bool = True, share_kv: Optional[bool] = None, key_layout: str = "groups"):
        if target.cfg.vocab_size != draft.cfg.vocab_size:
            raise ValueError("target and draft must share a vocabulary")
        self.target, self.draft, self.k = target, draft, k
        self.dev, self.dtype = target.device, target.dtype
        shared = shared_layers(target, draft)
        if share_kv and not shared:
            raise ValueError("share_kv needs an early-exit draft of the target (early_exit_draft)")
        self.shared = bool(shared) if share_kv is None else bool(share_kv)
        self.pool_t = PagedKVPool(target.cfg, num_blocks, block_size, dtype=self.dtype, device=self.dev,
                                  key_layout=key_layout)
        self.pool_d = self.pool_t if self.shared else PagedKVPool(draft.cfg, draft_num_blocks or num_blocks,
                                                                  block_size, dtype=self.dtype, device=self.dev,
                                                                  key_layout=key_layout)
        self.block_size = block_size
        self.limit = min(target.cfg.max_seq_len, draft.cfg.max_seq_len)
        self.gen = generator
        self.graphs = graphs   # replay each round shape's kernels from a captured HIP graph
        self.seqs: List[_Seq] = []
        self.stats = {"rounds": 0, "proposed": 0, "accepted": 0}

    # ---- sequences ------------------------------------------------------------------------------
    def _grow(self, seq: _Seq, n_tokens: int) -> None:
        pools = ((self.pool_t, seq.blocks_t),) if self.shared else ((self.pool_t, seq.blocks_t),
                                                                     (self.pool_d, seq.blocks_d))
        for pool, blocks in pools:
            need = pool.blocks_for(n_tokens) - len(blocks)
            if need > 0:
                blocks += pool.allocator.allocate(need)

    def release(self, seq: _Seq) -> None:
        self.pool_t.allocator.release(seq.blocks_t)
        if not self.shared:
            self.pool_d.allocator.release(seq.blocks_d)
        seq.blocks_t, seq.blocks_d = BlockList(), BlockList()

    def add(self, prompt: Sequence[int], max_new_tokens: int, temperature: float = 0.0, eos_id=None,
            prefill: bool = True) -> _Seq:
        """Add a sequence; with prefill, its prompt (all but the last token) is run through the target
        (and through the draft when it keeps its own pool)."""
        if not 0 < len(prompt) < self.limit:
            raise ValueError(f"prompt length must be in 1..{self.limit - 1}")
        seq = _Seq(prompt, max_new_tokens, temperature, eos_id)
        self._grow(seq, len(seq.tokens))
        if prefill and len(seq.tokens) > 1:
            n = len(seq.tokens) - 1
            idx = torch.tensor([seq.tokens[:-1]])
            pos = torch.arange(n)[None]
            runs = [(self.target, self.pool_t, seq.blocks_t)]
            if not self.shared:   # a shared draft's blocks were written by the target's prefill
                runs.append((self.draft, self.pool_d, seq.blocks_d))
            for model, pool, blocks in runs:
                model(idx, pos, pool.views(torch.tensor([blocks]), pos), last_only=True)
        self.seqs.append(seq)
        return seq

    def add_many(self, prompts: Sequence[Sequence[int]], max_new_tokens, temperature=0.0, eos_id=None,
                 max_prefill_tokens: int = 32768) -> List[_Seq]:
        """Add several sequences and prefill their prompts (all but each last token) packed: a few
        forwards of up to max_prefill_tokens tokens each through both models, instead of one forward per
        prompt. max_new_tokens, temperature, eos_id: one value, or one per prompt. The caches end up
        exactly as add() would leave them."""
        n = len(prompts)
        per = lambda x: list(x) if isinstance(x, (list, tuple)) else [x] * n
        max_new, temps, eos = per(max_new_tokens), per(temperature), per(eos_id)
        for p in prompts:
            if not 0 < len(p) < self.limit:
                raise ValueError(f"prompt length must be in 1..{self.limit - 1}")
        seqs = [_Seq(p, m, t, e) for p, m, t, e in zip(prompts, max_new, temps, eos)]
        for s in seqs:
            self._grow(s, len(s.tokens))
        todo = [s for s in seqs if len(s.tokens) > 1]
        i = 0
        while i < len(todo):
            chunk, total = [], 0
            while i < len(todo) and (not chunk or total + len(todo[i].tokens) - 1 <= max_prefill_tokens):
                chunk.append(todo[i])
                total += len(todo[i].tokens) - 1
                i += 1
            toks = [s.tokens[:-1] for s in chunk]
            prefill_packed(self.target, self.pool_t, toks, [s.blocks_t for s in chunk])
            if not self.shared:
                prefill_packed(self.draft, self.pool_d, toks, [s.blocks_d for s in chunk])
        self.seqs.extend(seqs)
        return seqs

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
                                                                        self.dev), graphs=self.graphs)
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

    @torch.no_grad()
    def run_rounds(self, n_rounds: int) -> int:
        """n_rounds rounds (fewer once every sequence has finished); returns the tokens committed.
        Tokens and stats are exactly those of n_rounds calls of round(). Where it is safe, each round is
        queued before the previous round's tokens are read back (fs_spec_advance computes its inputs
        on the GPU), so the GPU does not wait for the host between rounds: for a greedy batch always,
        for a sampled one while no sequence can finish inside the queue and none has an EOS id (the
        random numbers a round draws depend on the batch, which a finishing sequence changes)."""
        committed, left = 0, n_rounds
        while left > 0 and self.active():
            n_run, c = self._queued_rounds(left) if self.graphs else (0, 0)
            if n_run == 0:
                c, n_run = self.round(), 1
            committed += c
            left -= n_run
        return committed

    def _queued_rounds(self, max_rounds: int):
        """Up to max_rounds rounds of the current batch, each queued before the previous one's tokens
        are read: (rounds run, tokens committed); (0, 0) when the batch does not allow it."""
        seqs = self.active()
        b, k = len(seqs), self.k
        temps = [s.temperature for s in seqs]
        sampled = any(t > 0 for t in temps)
        rem = [self._remaining(s) for s in seqs]
        if k == 0 or min(rem) <= 0:
            return 0, 0
        n_max = max_rounds
        if sampled:
            if any(s.eos_id is not None for s in seqs):
                return 0, 0
            # every queued round must see k_eff = k in every row (the round's k and batch fix its draws):
            # round j has at least rem - j*(k+1) tokens left
            n_max = min(n_max, (min(rem) - k - 1) // (k + 1) + 1)
        if n_max < 2:
            return 0, 0
        limit = self.limit
        eos = [s.eos_id if s.eos_id is not None else -1 for s in seqs]
        st, pending, run, committed = None, [], 0, 0

        def process(j, ev):
            nonlocal run, committed
            ev.synchronize()
            rows = st.res_hosts[j % 2][:b].tolist()
            live = False
            for r, s in enumerate(seqs):
                if s.done:
                    continue
                live = True
                ke = max(0, min(k, self._remaining(s) - 1))
                a = rows[r][0]
                new = rows[r][1: a + 2]
                s.tokens += new
                committed += len(new)
                self.stats["proposed"] += ke
                self.stats["accepted"] += a
                self._finish_check(s)
            if live:
                self.stats["rounds"] += 1
                run += 1

        for j in range(n_max):
            if not any(not s.done for s in seqs):
                break
            # blocks for every position round j can write: its rows start at most k+1 tokens past the
            # lengths the host knows (those of round j-1's start), and write k past their start
            try:
                for s in seqs:
                    if not s.done:
                        self._grow(s, min(len(s.tokens) + (k if j == 0 else 2 * k + 1), limit))
            except OutOfBlocks:
                break
            blocks_t = [s.blocks_t for s in seqs]
            blocks_d = blocks_t if self.shared else [s.blocks_d for s in seqs]
            if j == 0:
                st = _round_state(self.target, self.draft, self.pool_t, self.pool_d, b, k, blocks_t, blocks_d, sampled)
                k_eff = [max(0, min(k, r_ - 1)) for r_ in rem]
                st.stage([s.tokens for s in seqs], k_eff, temps, blocks_t, blocks_d, slot=0, budget=rem, eos=eos)
                st.dev.copy_(st.hosts[0], non_blocking=True)
            else:
                wt = _bucket(max(len(x) for x in blocks_t), 64)
                wd = _bucket(max(len(x) for x in blocks_d), 64)
                if (wt, wd) != (st.wt, st.wd):   # the tables outgrew the shape: finish what is queued
                    break
                slot = j % 2
                st.stage_host(temps, blocks_t, blocks_d, slot)
                o = st.host_off
                st.dev[o:].copy_(st.hosts[slot][o:], non_blocking=True)
            draws = _GeneratorDraws(self.gen, b, k, self.target.cfg.vocab_size, self.dev) if sampled else None
            _launch_round(self.target, self.draft, self.pool_t, self.pool_d, st, b, draws, True)
            st.res_hosts[j % 2].copy_(st.res, non_blocking=True)
            ev = torch.cuda.Event()
            ev.record()
            pending.append((j, ev))
            if len(pending) == 2:
                process(*pending.pop(0))
        while pending:
            process(*pending.pop(0))
        return run, committed

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
    seqs = sb.add_many(prompts, max_new, temps)
    sb.run()
    return [s.tokens[s.start:] for s in seqs], sb.stats
