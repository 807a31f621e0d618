"""LLaMA-style decoder on gfx950 kernels (model.py:23-159 in the reference).

Same modules, parameter names and state_dict keys as the reference (RMSNorm, Attention with GQA and
half-split rotary, SwiGLU, pre-norm blocks, tied embedding/head), so weights load interchangeably.
The forward runs on the GPU only, as one chain of HIP kernels per layer:

    gemm(qkv) -> qkv_rope_write (rotary + KV write; a split-K projection is reduced here)
      -> paged_attention -> gemm(wo) -> residual add + mlp RMSNorm
      -> gemm(gate|up) with the SwiGLU gate in its epilogue -> gemm(w_down) -> residual add + next RMSNorm

q/k/v and gate/up use one fused weight each; the per-projection parameters are re-pointed at slices
of the fused buffer, so no weight is stored twice.
"""

import math
from typing import List, Optional

import torch
import torch.nn as nn

from . import ops
from ._lib import to_device
from .config import ModelConfig
from .parallel import SINGLE, TPContext


def precompute_rope(head_dim: int, max_len: int, theta: float):
    """cos/sin tables (max_len, head_dim/2) in f32 (model.py:34-37)."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2).float() / head_dim))
    angles = torch.outer(torch.arange(max_len).float(), inv_freq)
    return angles.cos(), angles.sin()


def _fused_weight(owner: nn.Module, params: List[nn.Parameter]) -> torch.Tensor:
    """One (sum of rows, cols) weight whose row slices are `params`; re-points them if needed. The
    result is kept on `owner` and reused while the parameters still hold the same storage."""
    key = tuple((p.data.data_ptr(), tuple(p.shape), p.dtype) for p in params)
    hit = owner.__dict__.get("_fused")
    if hit is not None and hit[1] == key:
        return hit[0]
    fused = _build_fused(params)
    owner.__dict__["_fused"] = (fused, tuple((p.data.data_ptr(), tuple(p.shape), p.dtype) for p in params))
    return fused


def _build_fused(params: List[nn.Parameter]) -> torch.Tensor:
    first = params[0].data
    rows = sum(p.shape[0] for p in params)
    cols = first.shape[1]
    ok = all(p.data.is_contiguous() and p.dtype == first.dtype and p.device == first.device and p.shape[1] == cols
             for p in params)
    if ok:
        off = first.data_ptr()
        for p in params:
            if p.data.data_ptr() != off or p.data.untyped_storage().data_ptr() != first.untyped_storage().data_ptr():
                ok = False
                break
            off += p.numel() * p.element_size()
    if ok:
        return first.new_empty(0).set_(first.untyped_storage(), first.storage_offset(), (rows, cols), (cols, 1))
    buf = torch.cat([p.data for p in params], 0).contiguous()
    r = 0
    for p in params:
        n = p.shape[0]
        p.data = buf[r: r + n]
        r += n
    return buf


class RMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float = 1e-5):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x):
        shape = x.shape
        y = ops.add_rmsnorm(x.reshape(-1, shape[-1]), self.weight, self.eps)
        return y.reshape(shape)


class Attention(nn.Module):
    """GQA attention: query head h reads KV head h // (n_heads // n_kv_heads) (model.py:48-78)."""

    def __init__(self, cfg: ModelConfig, tp: TPContext):
        super().__init__()
        self.tp = tp
        self.hd = cfg.head_dim
        self.nh, self.nkv = cfg.n_heads // tp.size, cfg.n_kv_heads // tp.size
        self.rep = cfg.n_heads // cfg.n_kv_heads
        self.wq = nn.Linear(cfg.d_model, self.nh * self.hd, bias=False)
        self.wk = nn.Linear(cfg.d_model, self.nkv * self.hd, bias=False)
        self.wv = nn.Linear(cfg.d_model, self.nkv * self.hd, bias=False)
        self.wo = nn.Linear(self.nh * self.hd, cfg.d_model, bias=False)

    def qkv_weight(self) -> torch.Tensor:
        return _fused_weight(self, [self.wq.weight, self.wk.weight, self.wv.weight])

    def attend(self, h: torch.Tensor, b: int, t: int, pos32: torch.Tensor, view, rope) -> torch.Tensor:
        """h (B*T, d) normed input -> attention output (B*T, n_heads*head_dim), before wo."""
        if getattr(view, "packed", False):   # packed prefill: rows are the step's tokens, no padding
            st = view.step
            q = ops.qkv_rope_write_varlen(ops.gemm(h, self.qkv_weight()), st.pos_tok, st.token_row, self.nh,
                                          rope[0], rope[1], st.tables, view.layout)
            o = ops.paged_attention_varlen(q.view(-1, self.nh, self.hd), view.layout, st.tables, st.pos_pad, st.cu,
                                           1.0 / math.sqrt(self.hd), plan_key=st)
            return o.view(-1, self.nh * self.hd)
        layout, tables, slots, mask = view.prepare(b, t, self.nkv, self.hd, h.dtype, h.device, pos32)
        q = ops.qkv_rope_gemm(h, self.qkv_weight(), pos32.reshape(-1), t, self.nh, rope[0], rope[1], tables, layout,
                              slots=slots)
        # the layers of one step share its positions: the attention work plan is built once per step
        o = ops.paged_attention(q.view(b, t, self.nh, self.hd), layout, tables, mask, 1.0 / math.sqrt(self.hd),
                                plan_key=getattr(view, "plan_key", None))
        view.commit(t)
        return o.view(b * t, self.nh * self.hd)


class SwiGLU(nn.Module):
    def __init__(self, cfg: ModelConfig, tp: TPContext):
        super().__init__()
        self.tp = tp
        hidden = cfg.ffn_dim // tp.size
        self.w_gate = nn.Linear(cfg.d_model, hidden, bias=False)
        self.w_up = nn.Linear(cfg.d_model, hidden, bias=False)
        self.w_down = nn.Linear(hidden, cfg.d_model, bias=False)

    def gate_up_weight(self) -> torch.Tensor:
        return _fused_weight(self, [self.w_gate.weight, self.w_up.weight])

    def forward(self, x, residual: Optional[torch.Tensor] = None):
        shape = x.shape
        x2 = x.reshape(-1, shape[-1])
        h = ops.gemm_swiglu(x2, self.gate_up_weight())
        r = None if residual is None else residual.reshape(-1, shape[-1])
        return ops.gemm(h, self.w_down.weight, residual=r).reshape(shape)


class Block(nn.Module):
    def __init__(self, cfg: ModelConfig, tp: TPContext):
        super().__init__()
        self.attn_norm = RMSNorm(cfg.d_model, cfg.norm_eps)
        self.attn = Attention(cfg, tp)
        self.mlp_norm = RMSNorm(cfg.d_model, cfg.norm_eps)
        self.mlp = SwiGLU(cfg, tp)

    def step(self, x: torch.Tensor, b: int, t: int, pos32: torch.Tensor, view, rope, h=None, next_norm=None,
             x_out=None):
        """x (B*T, d) -> x + attn(norm(x)), then + mlp(norm(.)) (model.py:104-106). h: norm(x) by this
        block's attention norm when the caller has it. Returns (x_out, next_norm(x_out) or None): a
        projection that splits K is reduced inside the residual-add + norm kernel that follows it. x_out:
        where the block's output goes (a new tensor when None)."""
        if h is None:
            h = ops.add_rmsnorm(x, self.attn_norm.weight, self.attn_norm.eps)
        a = self.attn.attend(h, b, t, pos32, view, rope)
        x1, h2 = ops.gemm_add_rmsnorm(a, self.attn.wo.weight, x, self.mlp_norm.weight, self.mlp_norm.eps)
        g = ops.gemm_swiglu(h2, self.mlp.gate_up_weight())
        if next_norm is None:
            return ops.gemm(g, self.mlp.w_down.weight, out=x_out, residual=x1), None
        return ops.gemm_add_rmsnorm(g, self.mlp.w_down.weight, x1, next_norm.weight, next_norm.eps, x_out=x_out)


class ForgeModel(nn.Module):
    """Embedding and head are shared (tied), as in model.py:109-159."""

    def __init__(self, cfg: ModelConfig, tp: TPContext = SINGLE):
        super().__init__()
        cfg.check_tensor_parallel(tp.size)
        self.cfg, self.tp = cfg, tp
        self.tok_emb = nn.Embedding(cfg.vocab_size, cfg.d_model)
        self.layers = nn.ModuleList(Block(cfg, tp) for _ in range(cfg.n_layers))
        self.norm = RMSNorm(cfg.d_model, cfg.norm_eps)
        self.lm_head = nn.Linear(cfg.d_model, cfg.vocab_size, bias=False)
        self.lm_head.weight = self.tok_emb.weight
        cos, sin = precompute_rope(cfg.head_dim, cfg.max_seq_len, cfg.rope_theta)
        self.register_buffer("rope_cos", cos, persistent=False)
        self.register_buffer("rope_sin", sin, persistent=False)
        self._rope_cache = None
        self.apply(self._init_weights)

    @staticmethod
    def _init_weights(m):
        if isinstance(m, (nn.Linear, nn.Embedding)):
            nn.init.normal_(m.weight, mean=0.0, std=0.02)

    def num_params(self) -> int:
        return sum(p.numel() for p in self.parameters())

    @property
    def device(self) -> torch.device:
        return self.tok_emb.weight.device

    @property
    def dtype(self) -> torch.dtype:
        return self.tok_emb.weight.dtype

    def _rope(self):
        """f32 copies of the rotary tables on the model's device (a bf16 model rounds them once)."""
        c, s = self.rope_cos, self.rope_sin
        key = (c.data_ptr(), s.data_ptr(), c.dtype, c.device)
        if self._rope_cache is None or self._rope_cache[0] != key:
            self._rope_cache = (key, (c.float().contiguous(), s.float().contiguous()))
        return self._rope_cache[1]

    def embed(self, idx):
        return ops.embedding(to_device(idx, self.device), self.tok_emb.weight).reshape(*idx.shape, self.cfg.d_model)

    def head_normed(self, y, stats=None, out=None):
        """The tied head (model.py:138) on rows already normalised by the final norm: (rows, vocab)."""
        if stats is not None:
            return ops.gemm_row_stats(y, self.lm_head.weight, stats[0], stats[1], out=out)
        return ops.gemm(y, self.lm_head.weight, out=out)

    def head(self, x, stats=None, out=None):
        """Final norm + tied head (model.py:137-138). stats = (temperature (rows,), parts): also emit
        the logits' per-row softmax statistics (ops.gemm_row_stats). out: optional (rows, vocab) view
        (contiguous rows, any row stride) that receives the logits."""
        shape = x.shape
        y = ops.add_rmsnorm(x.reshape(-1, shape[-1]), self.norm.weight, self.norm.eps)
        if stats is not None:
            logits = ops.gemm_row_stats(y, self.lm_head.weight, stats[0], stats[1], out=out)
        else:
            logits = ops.gemm(y, self.lm_head.weight, out=out)
        return logits if out is not None else logits.reshape(*shape[:-1], self.cfg.vocab_size)

    @torch.no_grad()
    def forward(self, idx, positions: Optional[torch.Tensor] = None, kv: Optional[List] = None,
                last_only: bool = False, head_stats=None):
        """idx (B, T) token ids -> logits (B, T, vocab) (model.py:141-159).

        positions (B, T): absolute positions; default continues after what `kv` holds.
        kv: one cache view per layer (ContiguousKV or PagedLayerView); None uses a fresh cache.
        last_only: return only the logits of the last position, (B, 1, vocab).
        head_stats: (temperature, parts) for the head's rows: see head()."""
        dev = self.device
        if dev.type != "cuda":
            raise RuntimeError("ForgeModel runs on the GPU: move it with .to('cuda') first")
        b, t = idx.shape
        if kv is None:
            from .kv import new_contiguous_cache
            kv = new_contiguous_cache(self.cfg.n_layers)
        if positions is None:
            start = kv[0].length
            positions = (start + torch.arange(t))[None, :].expand(b, t)
        pmax = int(positions.max())
        if pmax >= self.cfg.max_seq_len:
            raise ValueError(f"position {pmax} exceeds max_seq_len {self.cfg.max_seq_len}")
        pos32 = to_device(positions.reshape(b, t).contiguous(), dev, torch.int32)
        return self._run(to_device(idx, dev), pos32, kv, last_only, head_stats)

    def _run(self, idx: torch.Tensor, pos32: torch.Tensor, kv: List, last_only: bool = False, head_stats=None,
             out=None, hidden_out=None):
        """The forward's kernels alone: idx (B, T) int64 and pos32 (B, T) int32 already on the device,
        no argument checks and no host synchronisation, so that a caller can capture it in a HIP graph
        (positions < max_seq_len is the caller's to guarantee). With last_only, `out` (B, vocab) may
        receive the logits (then it is returned as is) and `hidden_out` (B, d_model) the last
        position's residual stream after the last layer (the head's input before its norm)."""
        b, t = idx.shape
        direct = last_only and t == 1 and hidden_out is not None   # the last block writes hidden_out
        x, y = self._layers(ops.embedding(idx, self.tok_emb.weight), 0, len(self.layers), b, t, pos32, kv,
                            last_norm=self.norm, x_out=hidden_out if direct else None)
        if last_only:
            if hidden_out is not None and x is not hidden_out:
                hidden_out.copy_(x.view(b, t, -1)[:, -1])
            y = y.view(b, t, -1)[:, -1].contiguous()
            if out is not None:
                return self.head_normed(y, head_stats, out=out)
            return self.head_normed(y, head_stats).view(b, 1, -1)
        return self.head_normed(y, head_stats).view(b, t, -1)

    def _layers(self, x: torch.Tensor, start: int, stop: int, b: int, t: int, pos32: torch.Tensor, kv: List,
                last_norm=None, x_out=None):
        """Blocks start..stop-1 on the residual stream x (B*T, d); kv[i] is block i's cache view.
        Returns (x, last_norm(x)): each block's output is normalised by the next block's attention
        norm in the same kernel as its last projection's reduction; after block stop-1 by last_norm
        (None: not normalised). x_out: where block stop-1 writes its output (then returned as x)."""
        rope = self._rope()
        h = None
        for i in range(start, stop):
            nxt = self.layers[i + 1].attn_norm if i + 1 < stop else last_norm
            x, h = self.layers[i].step(x, b, t, pos32, kv[i], rope, h=h, next_norm=nxt,
                                       x_out=x_out if i == stop - 1 else None)
        if start >= stop and last_norm is not None:   # no block ran (a draft that is the whole model)
            h = ops.add_rmsnorm(x, last_norm.weight, last_norm.eps)
        return x, h

    def _run_verify_reusing(self, n_shared: int, window: torch.Tensor, pos32: torch.Tensor, kv: List,
                            keff: torch.Tensor, hidden: torch.Tensor, head_stats=None):
        """The verify pass over window (B, T) at pos32 when blocks 0..n_shared-1 have already run for
        the first keff[r] tokens of row r (an early-exit draft sharing those blocks and their cache):
        hidden (B, T-1, d) holds their residual streams after block n_shared-1. Only token keff[r] of
        each row goes through blocks 0..n_shared-1 here (one row each, at its own position); then
        all T tokens run the remaining blocks and the head. Every row's result is bit-identical to the
        full pass: the blocks compute a row the same way whatever else is in the batch."""
        b, t = window.shape
        d = self.cfg.d_model
        k1 = keff.to(torch.int64)[:, None]
        tail_idx = window.gather(1, k1)
        tail_pos = pos32.gather(1, k1)
        h_tail, _ = self._layers(ops.embedding(tail_idx, self.tok_emb.weight), 0, n_shared, b, 1, tail_pos, kv)
        x = torch.empty((b, t, d), dtype=h_tail.dtype, device=h_tail.device)
        x[:, : t - 1].copy_(hidden)
        x.scatter_(1, k1[:, :, None].expand(b, 1, d), h_tail.view(b, 1, d))
        _, y = self._layers(x.view(b * t, d), n_shared, len(self.layers), b, t, pos32, kv, last_norm=self.norm)
        return self.head_normed(y, head_stats).view(b, t, -1)


@torch.no_grad()
def prefill_packed(model: ForgeModel, pool, tokens: List[List[int]], block_lists: List[List[int]],
                   starts: Optional[List[int]] = None) -> torch.Tensor:
    """Run several sequences' new tokens through `model` in one packed forward (no padding rows),
    writing their keys/values into `pool` (a PagedKVPool of the model's layers) through block_lists.
    Sequence s's tokens sit at positions starts[s] .. (default 0 ..). Returns the logits of each
    sequence's last token, (S, vocab). Each sequence's cache contents and logits are bit-identical to
    prefilling it alone (model(tokens, positions, pool.views(...)), engine.py:80-95)."""
    from .paged import PackedPrefill

    if len(pool.k) != model.cfg.n_layers:
        raise ValueError(f"pool has {len(pool.k)} layers, the model {model.cfg.n_layers}")
    starts = [0] * len(tokens) if starts is None else list(starts)
    step = PackedPrefill(pool, block_lists, starts, [len(t) for t in tokens])
    if step.max_position >= model.cfg.max_seq_len:
        raise ValueError(f"position {step.max_position} exceeds max_seq_len {model.cfg.max_seq_len}")
    flat = torch.tensor([x for t in tokens for x in t], dtype=torch.int64)
    if flat.numel() and (int(flat.min()) < 0 or int(flat.max()) >= model.cfg.vocab_size):
        raise ValueError("token ids must be in [0, vocab_size)")
    ids = to_device(flat, model.device)
    x = ops.embedding(ids, model.tok_emb.weight)
    _, y = model._layers(x, 0, len(model.layers), 1, step.n_tokens, None, step.views(), last_norm=model.norm)
    return model.head_normed(y.index_select(0, step.last_rows))


def early_exit_draft(target: ForgeModel, n_layers: int) -> ForgeModel:
    """A draft that is the target's embedding, first n_layers blocks, final norm and head, sharing the
    target's weight tensors (no copy). Its KV cache is separate from the target's."""
    from dataclasses import replace

    cfg = replace(target.cfg, n_layers=n_layers)
    d = ForgeModel.__new__(ForgeModel)
    nn.Module.__init__(d)
    d.cfg, d.tp = cfg, target.tp
    d.tok_emb = target.tok_emb
    d.layers = nn.ModuleList(list(target.layers)[:n_layers])
    d.norm = target.norm
    d.lm_head = target.lm_head
    d.register_buffer("rope_cos", target.rope_cos, persistent=False)
    d.register_buffer("rope_sin", target.rope_sin, persistent=False)
    d._rope_cache = None
    return d
