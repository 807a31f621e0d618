"""CPU restatement of the reference hot path (TEST INFRASTRUCTURE ONLY; see oracle/__init__.py).

Weights are a dict keyed by the reference's state_dict names. Every function cites the reference
lines it restates. Arithmetic follows the reference's dtype/cast order so the restatement agrees
with the reference to float32 rounding (pinned against its own outputs in tests/golden/).
"""

import math
from collections import deque
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple

import torch

Weights = Dict[str, torch.Tensor]


# ------------------------------------------------------------------------------------------------
# configuration and synthetic weights
# ------------------------------------------------------------------------------------------------
@dataclass
class Shape:
    """The fields of config.py:8-17 the math needs."""
    vocab_size: int
    d_model: int
    n_layers: int
    n_heads: int
    n_kv_heads: int
    ffn_dim: int
    max_seq_len: int
    rope_theta: float = 10000.0
    norm_eps: float = 1e-5

    @property
    def head_dim(self) -> int:
        return self.d_model // self.n_heads

    @staticmethod
    def of(cfg) -> "Shape":
        return Shape(cfg.vocab_size, cfg.d_model, cfg.n_layers, cfg.n_heads, cfg.n_kv_heads, cfg.ffn_dim,
                     cfg.max_seq_len, cfg.rope_theta, cfg.norm_eps)


def param_names(s: Shape) -> List[Tuple[str, Tuple[int, ...]]]:
    """Parameters in the reference's registration order (model.py:96-120; lm_head is tok_emb)."""
    hd = s.head_dim
    out = [("tok_emb.weight", (s.vocab_size, s.d_model))]
    for i in range(s.n_layers):
        p = f"layers.{i}."
        out += [(p + "attn_norm.weight", (s.d_model,)),
                (p + "attn.wq.weight", (s.n_heads * hd, s.d_model)),
                (p + "attn.wk.weight", (s.n_kv_heads * hd, s.d_model)),
                (p + "attn.wv.weight", (s.n_kv_heads * hd, s.d_model)),
                (p + "attn.wo.weight", (s.d_model, s.n_heads * hd)),
                (p + "mlp_norm.weight", (s.d_model,)),
                (p + "mlp.w_gate.weight", (s.ffn_dim, s.d_model)),
                (p + "mlp.w_up.weight", (s.ffn_dim, s.d_model)),
                (p + "mlp.w_down.weight", (s.d_model, s.ffn_dim))]
    out.append(("norm.weight", (s.d_model,)))
    return out


def synthetic_weights(s: Shape, seed: int, std: float) -> Weights:
    """Matrices ~ N(0, std^2) drawn in registration order from Generator().manual_seed(seed), norms = 1
    (the recipe of the reference's tests/conftest.py:18-27, which the golden script also applies)."""
    g = torch.Generator().manual_seed(seed)
    w = {}
    for name, shape in param_names(s):
        w[name] = torch.randn(shape, generator=g) * std if len(shape) >= 2 else torch.ones(shape)
    return w


# ------------------------------------------------------------------------------------------------
# caches
# ------------------------------------------------------------------------------------------------
class ContiguousCache:
    """kv.py:10-29: keys/values of all rows, appended along the sequence axis."""

    def __init__(self):
        self.k = None
        self.v = None

    @property
    def length(self) -> int:
        return 0 if self.k is None else self.k.shape[2]

    def update(self, k, v):
        self.k = k if self.k is None else torch.cat((self.k, k), 2)
        self.v = v if self.v is None else torch.cat((self.v, v), 2)
        return self.k, self.v

    def truncate(self, n: int) -> None:
        if self.k is not None:
            self.k = self.k[:, :, :n]
            self.v = self.v[:, :, :n]


def contiguous_caches(n: int) -> List[ContiguousCache]:
    return [ContiguousCache() for _ in range(n)]


class Allocator:
    """paged.py:24-39: LIFO stack of free block ids, block 0 first."""

    def __init__(self, num_blocks: int):
        self.num_blocks = num_blocks
        self.free = list(reversed(range(num_blocks)))

    @property
    def num_free(self) -> int:
        return len(self.free)

    def allocate(self, n: int) -> List[int]:
        if n > len(self.free):
            raise RuntimeError(f"need {n} blocks, {len(self.free)} free")
        return [self.free.pop() for _ in range(n)]

    def release(self, blocks: List[int]) -> None:
        self.free += blocks


class PagedPool:
    """paged.py:42-58: per-layer (num_blocks, n_kv_heads, block_size, head_dim) tensors."""

    def __init__(self, s: Shape, num_blocks: int, block_size: int, dtype=torch.float32):
        shp = (num_blocks, s.n_kv_heads, block_size, s.head_dim)
        self.k = [torch.zeros(shp, dtype=dtype) for _ in range(s.n_layers)]
        self.v = [torch.zeros(shp, dtype=dtype) for _ in range(s.n_layers)]
        self.block_size = block_size
        self.allocator = Allocator(num_blocks)

    def blocks_for(self, n: int) -> int:
        return (n + self.block_size - 1) // self.block_size

    def views(self, tables, positions):
        return [PagedView(self, i, tables, positions) for i in range(len(self.k))]


class PagedView:
    """paged.py:61-82: scatter the step's k/v at (table[pos // bs], pos % bs), then gather every block."""

    def __init__(self, pool: PagedPool, layer: int, tables, positions):
        self.pool, self.layer, self.tables, self.positions = pool, layer, tables.long(), positions.long()

    def update(self, k, v):
        bs = self.pool.block_size
        kp, vp = self.pool.k[self.layer], self.pool.v[self.layer]
        b, h, t, d = k.shape
        for r in range(b):
            for j in range(t):
                pos = int(self.positions[r, j])
                blk = int(self.tables[r, pos // bs])
                kp[blk, :, pos % bs] = k[r, :, j]
                vp[blk, :, pos % bs] = v[r, :, j]
        nb = self.tables.shape[1]
        k_all = torch.stack([torch.cat([kp[int(self.tables[r, i])] for i in range(nb)], 1) for r in range(b)])
        v_all = torch.stack([torch.cat([vp[int(self.tables[r, i])] for i in range(nb)], 1) for r in range(b)])
        return k_all, v_all


# ------------------------------------------------------------------------------------------------
# model
# ------------------------------------------------------------------------------------------------
def rope_tables(s: Shape):
    """model.py:34-37: inv_freq = theta^(-2i/D); angles = outer(position, inv_freq) in f32."""
    i = torch.arange(0, s.head_dim, 2).float()
    inv = 1.0 / (s.rope_theta ** (i / s.head_dim))
    ang = torch.arange(s.max_seq_len).float()[:, None] * inv[None, :]
    return ang.cos(), ang.sin()


def rms_norm(x, w, eps):
    """model.py:29-31: normalise in f32, round to x's dtype, multiply by the weight."""
    xf = x.float()
    inv = torch.rsqrt((xf * xf).mean(dim=-1, keepdim=True) + eps)
    return (xf * inv).to(x.dtype) * w


def rotate(x, cos, sin, positions):
    """model.py:40-45: half-split rotation with cos/sin cast to x's dtype; x (B, H, T, D)."""
    half = x.shape[-1] // 2
    c = cos[positions].unsqueeze(1).to(x.dtype)
    s_ = sin[positions].unsqueeze(1).to(x.dtype)
    a, b = x[..., :half], x[..., half:]
    return torch.cat((a * c - b * s_, b * c + a * s_), -1)


def attention_math(q, k_all, v_all, positions, rep):
    """model.py:70-76: GQA by repeating KV heads, key index <= query position, softmax(q k^T / sqrt(D)) v.

    Written as explicit f32 math (no SDPA): q (B, H, T, D), k_all/v_all (B, Hkv, S, D)."""
    k_all = k_all.repeat_interleave(rep, dim=1).float()
    v_all = v_all.repeat_interleave(rep, dim=1).float()
    scale = 1.0 / math.sqrt(q.shape[-1])
    scores = torch.matmul(q.float(), k_all.transpose(-1, -2)) * scale
    key_idx = torch.arange(k_all.shape[2])
    visible = key_idx[None, None, :] <= positions[:, :, None]        # (B, T, S)
    scores = scores.masked_fill(~visible[:, None], float("-inf"))
    probs = torch.softmax(scores, dim=-1)
    return torch.matmul(probs, v_all).to(q.dtype)


def block(lw: Weights, s: Shape, x, positions, cache, rope):
    """model.py:104-106 with Attention.forward (62-78) and SwiGLU (92-93): one pre-norm block on the
    residual stream x (B, T, d). lw holds the block's weights under their names inside the block
    ("attn_norm.weight", "attn.wq.weight", ...); cache is the block's cache view."""
    b, t, _ = x.shape
    cos, sin = rope
    hd, nh, nkv = s.head_dim, s.n_heads, s.n_kv_heads
    h = rms_norm(x, lw["attn_norm.weight"], s.norm_eps)
    q = (h @ lw["attn.wq.weight"].T).view(b, t, nh, hd).transpose(1, 2)
    k = (h @ lw["attn.wk.weight"].T).view(b, t, nkv, hd).transpose(1, 2)
    v = (h @ lw["attn.wv.weight"].T).view(b, t, nkv, hd).transpose(1, 2)
    q, k = rotate(q, cos, sin, positions), rotate(k, cos, sin, positions)
    k_all, v_all = cache.update(k, v)
    o = attention_math(q, k_all, v_all, positions, nh // nkv)
    x = x + o.transpose(1, 2).reshape(b, t, nh * hd) @ lw["attn.wo.weight"].T
    h = rms_norm(x, lw["mlp_norm.weight"], s.norm_eps)
    g = h @ lw["mlp.w_gate.weight"].T
    u = h @ lw["mlp.w_up.weight"].T
    return x + (torch.nn.functional.silu(g) * u) @ lw["mlp.w_down.weight"].T


def _positions(s: Shape, kv, idx, positions):
    b, t = idx.shape
    if positions is None:
        positions = (kv[0].length + torch.arange(t))[None].expand(b, t)
    positions = positions.long()
    if int(positions.max()) >= s.max_seq_len:
        raise ValueError("position exceeds max_seq_len")
    return positions


def forward(w: Weights, s: Shape, idx, positions=None, kv=None, rope=None):
    """model.py:141-159: logits (B, T, V) for token ids idx (B, T); kv: one cache view per layer."""
    if kv is None:
        kv = contiguous_caches(s.n_layers)
    positions = _positions(s, kv, idx, positions)
    rope = rope if rope is not None else rope_tables(s)
    x = w["tok_emb.weight"][idx]
    for i in range(s.n_layers):
        p = f"layers.{i}."
        lw = {name[len(p):]: t for name, t in w.items() if name.startswith(p)}
        x = block(lw, s, x, positions, kv[i], rope)
    return rms_norm(x, w["norm.weight"], s.norm_eps) @ w["tok_emb.weight"].T


def forward_streamed(layer_weights, emb, norm_w, s: Shape, idx, positions=None, hidden=None):
    """forward() (model.py:141-159) with one block's weights on the host at a time, for models too
    large to hold whole in host memory: layer_weights(i) returns block i's weights (the names inside
    the block, as block() takes them) and may build them on demand; emb is the tied embedding/head,
    norm_w the final norm's weight. A fresh contiguous cache. hidden: optional list that receives the
    residual stream after each block. Identical arithmetic to forward()."""
    kv = contiguous_caches(s.n_layers)
    positions = _positions(s, kv, idx, positions)
    rope = rope_tables(s)
    x = emb[idx]
    for i in range(s.n_layers):
        x = block(layer_weights(i), s, x, positions, kv[i], rope)
        kv[i] = None
        if hidden is not None:
            hidden.append(x)
    return rms_norm(x, norm_w, s.norm_eps) @ emb.T


def draft_weights(w: Weights, n_layers: int) -> Weights:
    """An early-exit draft: embedding/head/final norm plus the first n_layers blocks of the target."""
    out = {}
    for name, t in w.items():
        if name.startswith("layers."):
            if int(name.split(".")[1]) < n_layers:
                out[name] = t
        else:
            out[name] = t
    return out


# ------------------------------------------------------------------------------------------------
# sampling
# ------------------------------------------------------------------------------------------------
def probs_from_logits(logits, temperature):
    """sampling.py:9-13."""
    if temperature == 0:
        hot = torch.zeros_like(logits)
        return hot.scatter_(-1, logits.argmax(-1, keepdim=True), 1.0)
    return torch.softmax(logits.float() / temperature, dim=-1)


def draw(w, noise):
    """torch.multinomial(w, 1) as the library computes it: argmax(w / noise), first index on ties."""
    return int(torch.argmax(w / noise))


def exp_noise(n: int, gen) -> torch.Tensor:
    g = gen if gen is not None else torch.default_generator
    return torch.empty(n, dtype=torch.float32).exponential_(generator=g)


def sample(logits, temperature, gen=None):
    """sampling.py:16-21 for one row (V,)."""
    if temperature == 0:
        return int(logits.argmax())
    p = probs_from_logits(logits, temperature)
    return draw(p, exp_noise(p.shape[-1], gen))


def generate(w: Weights, s: Shape, prompt: List[int], n: int, temperature=0.0, gen=None) -> List[int]:
    """sampling.py:24-35 for one row: prefill, then one token per step."""
    kv = contiguous_caches(s.n_layers)
    n = min(n, s.max_seq_len - len(prompt))
    out = list(prompt)
    logits = forward(w, s, torch.tensor([prompt]), kv=kv)[0, -1]
    for i in range(n):
        tok = sample(logits, temperature, gen)
        out.append(tok)
        if i + 1 < n:
            logits = forward(w, s, torch.tensor([[tok]]), kv=kv)[0, -1]
    return out


# ------------------------------------------------------------------------------------------------
# speculative decoding
# ------------------------------------------------------------------------------------------------
def verify_with_noise(p, q, xs: List[int], u, noise) -> Tuple[List[int], int]:
    """speculative.py:20-33 with the randomness given: u[i] is the uniform of proposal i, noise the Exp(1)
    vector of the final draw. Returns (accepted, extra)."""
    acc = []
    for i, x in enumerate(xs):
        qx = q[i, x]
        ratio = float(p[i, x] / qx) if qx > 0 else 1.0
        if float(u[i]) < min(1.0, ratio):
            acc.append(x)
            continue
        r = torch.clamp(p[i] - q[i], min=0)
        tot = r.sum()
        r = r / tot if tot > 0 else p[i]
        return acc, draw(r, noise)
    return acc, draw(p[len(xs)], noise)


def verify_draft(p, q, xs: List[int], gen=None) -> Tuple[List[int], int]:
    """speculative.py:20-33 with its generator stream: a uniform per examined proposal (lazily, stopping
    at the first rejection), then one Exp(1) vector for the final draw."""
    g = gen if gen is not None else torch.default_generator
    acc = []
    for i, x in enumerate(xs):
        qx = q[i, x]
        ratio = float(p[i, x] / qx) if qx > 0 else 1.0
        if float(torch.rand((), generator=g)) < min(1.0, ratio):
            acc.append(x)
            continue
        r = torch.clamp(p[i] - q[i], min=0)
        tot = r.sum()
        r = r / tot if tot > 0 else p[i]
        return acc, draw(r, exp_noise(r.shape[-1], g))
    last = p[len(xs)]
    return acc, draw(last, exp_noise(last.shape[-1], g))


def speculative_generate(wt: Weights, st: Shape, wd: Weights, sd: Shape, prompt: List[int], n: int, k: int = 4,
                         temperature=0.0, gen=None):
    """speculative.py:36-86, one sequence, contiguous caches, the reference's draw order."""
    if st.vocab_size != sd.vocab_size:
        raise ValueError("target and draft must share a vocabulary")
    limit = min(st.max_seq_len, sd.max_seq_len)
    toks = list(prompt)
    kt, kd = contiguous_caches(st.n_layers), contiguous_caches(sd.n_layers)
    if len(toks) > 1:
        forward(wt, st, torch.tensor([toks[:-1]]), kv=kt)
        forward(wd, sd, torch.tensor([toks[:-1]]), kv=kd)
    stats = {"rounds": 0, "proposed": 0, "accepted": 0}
    start = len(toks)
    while len(toks) - start < n and len(toks) < limit:
        left = min(n - (len(toks) - start), limit - len(toks))
        ke = min(k, left - 1)
        cached = kt[0].length
        xs, qs, cur = [], [], toks[-1]
        for _ in range(ke):
            qrow = probs_from_logits(forward(wd, sd, torch.tensor([[cur]]), kv=kd)[0, -1], temperature)
            cur = int(qrow.argmax()) if temperature == 0 else draw(qrow, exp_noise(qrow.shape[-1], gen))
            xs.append(cur)
            qs.append(qrow)
        p = probs_from_logits(forward(wt, st, torch.tensor([[toks[-1]] + xs]), kv=kt)[0], temperature)
        acc, extra = verify_draft(p, torch.stack(qs) if qs else p[:0], xs, gen)
        toks += acc + [extra]
        stats["rounds"] += 1
        stats["proposed"] += ke
        stats["accepted"] += len(acc)
        want = cached + 1 + len(acc)
        for c in kt:
            c.truncate(want)
        have = kd[0].length
        if have > want:
            for c in kd:
                c.truncate(want)
        elif have < want:
            forward(wd, sd, torch.tensor([toks[have:want]]), kv=kd)
    return toks[start:], stats


# ------------------------------------------------------------------------------------------------
# continuous batching
# ------------------------------------------------------------------------------------------------
@dataclass
class Req:
    id: int
    prompt: List[int]
    max_new: int
    eos_id: Optional[int] = None
    temperature: float = 0.0
    output: List[int] = field(default_factory=list)
    blocks: List[int] = field(default_factory=list)
    cached: int = 0
    finished: bool = False


class Engine:
    """engine.py:36-139: prefill-or-decode steps, newest-first recompute preemption, one generator."""

    def __init__(self, w: Weights, s: Shape, num_blocks: int, block_size: int = 16, max_batch: int = 8, seed: int = 0):
        self.w, self.s = w, s
        self.pool = PagedPool(s, num_blocks, block_size)
        self.max_batch = max_batch
        self.gen = torch.Generator().manual_seed(seed)
        self.waiting = deque()
        self.running: List[Req] = []
        self.requests: Dict[int, Req] = {}
        self.preemptions = 0
        self.rope = rope_tables(s)

    def add(self, prompt, max_new, eos_id=None, temperature=0.0) -> int:
        r = Req(len(self.requests), list(prompt), max_new, eos_id, temperature)
        self.requests[r.id] = r
        self.waiting.append(r)
        return r.id

    def run(self) -> Dict[int, List[int]]:
        while self.waiting or self.running:
            if self.waiting and len(self.running) < self.max_batch and self._prefill():
                continue
            if self.running:
                self._decode()
            elif self.waiting:
                raise RuntimeError("pool too small")
        return {i: r.output for i, r in self.requests.items()}

    def _prefill(self) -> bool:
        r = self.waiting[0]
        toks = r.prompt + r.output
        need = self.pool.blocks_for(len(toks))
        if need > self.pool.allocator.num_free:
            return False
        self.waiting.popleft()
        r.blocks = self.pool.allocator.allocate(need)
        pos = torch.arange(len(toks))[None]
        logits = forward(self.w, self.s, torch.tensor([toks]), pos, self.pool.views(torch.tensor([r.blocks]), pos),
                         rope=self.rope)
        r.cached = len(toks)
        self._emit(r, logits[0, -1])
        if not r.finished:
            self.running.append(r)
        return True

    def _decode(self) -> None:
        bs = self.pool.block_size
        i = 0
        while i < len(self.running):
            r = self.running[i]
            if r.cached % bs == 0 and r.cached // bs == len(r.blocks):
                if self.pool.allocator.num_free == 0:
                    if len(self.running) == 1:
                        raise RuntimeError("pool too small for one sequence")
                    victim = self.running.pop()
                    self.pool.allocator.release(victim.blocks)
                    victim.blocks, victim.cached = [], 0
                    self.waiting.appendleft(victim)
                    self.preemptions += 1
                    if victim is r or not self.running:
                        if not self.running:
                            return
                    continue
                r.blocks += self.pool.allocator.allocate(1)
            i += 1
        width = max(len(r.blocks) for r in self.running)
        tables = torch.tensor([r.blocks + [0] * (width - len(r.blocks)) for r in self.running])
        pos = torch.tensor([[r.cached] for r in self.running])
        idx = torch.tensor([[r.output[-1]] for r in self.running])
        logits = forward(self.w, self.s, idx, pos, self.pool.views(tables, pos), rope=self.rope)
        for row, r in enumerate(list(self.running)):
            r.cached += 1
            self._emit(r, logits[row, -1])
            if r.finished:
                self.running.remove(r)

    def _emit(self, r: Req, logits) -> None:
        tok = sample(logits, r.temperature, self.gen)
        r.output.append(tok)
        if len(r.output) >= r.max_new or tok == r.eos_id or len(r.prompt) + len(r.output) >= self.s.max_seq_len:
            r.finished = True
            self.pool.allocator.release(r.blocks)
            r.blocks = []
