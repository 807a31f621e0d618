"""The workloads of the benchmark configurations at their full sizes on the GPU.

* 8B shape (32 layers, d 4096, 32/8 heads, head_dim 128, ffn 14336, vocab 128256, bf16, N(0, 0.02)):
  verify attention at batch 64 / k+1 = 7 / contexts U[2048, 8192] against the fp32 oracle (and a case
  whose positions cross the 8192-key chunk); the fused acceptance at batch 64 / k = 6 / vocab 128256
  on logits and statistics from the model's own LM head, against the oracle's verify_draft on the same
  injected randomness; greedy batched speculation equal to the target's own greedy tokens (the
  reference invariant of tests/test_speculative.py:22-37), and HIP-graph rounds equal to eager rounds
  at T = 1.
* 1B shape (16 layers, d 2048, 32/8 heads, head_dim 64, ffn 8192, vocab 32000, bf16): the
  continuous-batching speculative Engine over 48 requests through a pool small enough to preempt.
* Both shapes at full depth (every layer, the full vocabulary): bf16 logits of a teacher-forced
  sequence against the oracle's f32 arithmetic on the same bf16 weights, and greedy tokens against
  the oracle's argmax, allowing only near-ties.

Acceptance decisions compare bit for bit; a decision whose oracle-side margin is below NEAR_TIE may
differ, and every such case is printed. The margin is |u - min(1, p/q)| / min(1, p/q) for a proposal
and the relative gap between the two largest keys w/E of the final draw. NEAR_TIE is the float32
noise of torch's own softmax at this vocabulary: its vectorised sum differs from an exact sum by up to
~50 ulps (3e-6) at V = 128256, and a ratio p/q carries two of them.
"""

import pytest
import torch

import forgeserve_amd as fa
from forgeserve_amd import ops
from helpers import record
from oracle import reference_cpu as orc

pytestmark = pytest.mark.gpu
DEV = "cuda"
NEAR_TIE = 1e-5

C5 = dict(vocab_size=128256, d_model=4096, n_layers=32, n_heads=32, n_kv_heads=8, ffn_dim=14336, max_seq_len=10240)
C4 = dict(vocab_size=32000, d_model=2048, n_layers=16, n_heads=32, n_kv_heads=8, ffn_dim=8192, max_seq_len=2048)


def case(*a):
    print("case:", *a, flush=True)


def _bf16_model(cfg, seed):
    torch.manual_seed(seed)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(DEV):
            return fa.ForgeModel(fa.ModelConfig(**cfg)).eval()
    finally:
        torch.set_default_dtype(prev)


@pytest.fixture(scope="module")
def c5_target():
    m = _bf16_model(C5, 0)
    yield m
    del m
    torch.cuda.empty_cache()


# ---- verify attention at the 8B shape ---------------------------------------------------------------------
def _attention_case(ctx, t, seed):
    """Pool, tables (a random permutation of the pool, rows padded to multiples of 64 blocks with block
    0 as the round stages them), N(0,1) bf16 queries/keys/values, the last t positions of each context."""
    h, hkv, d, bs = 32, 8, 128, 16
    nb = [-(-c // bs) for c in ctx]
    n_pool = sum(nb) + 16
    perm = torch.randperm(n_pool, generator=torch.Generator().manual_seed(seed))
    tables = torch.zeros(len(ctx), -(-max(nb) // 64) * 64, dtype=torch.int32)
    at = 0
    for i, n in enumerate(nb):
        tables[i, :n] = perm[at: at + n].int()
        at += n
    cfg = fa.ModelConfig(vocab_size=8, d_model=h * d, n_layers=1, n_heads=h, n_kv_heads=hkv, max_seq_len=16)
    pool = fa.PagedKVPool(cfg, n_pool, bs, dtype=torch.bfloat16, device=DEV)
    g = torch.Generator(device=DEV).manual_seed(seed)
    pool.k_store.normal_(generator=g)
    pool.v_store.normal_(generator=g)
    q = torch.randn(len(ctx), t, h, d, device=DEV, generator=g).bfloat16()
    pos = torch.tensor([[c - t + i for i in range(t)] for c in ctx], dtype=torch.int32)
    return q, pool, tables, pos


def _oracle_attention_rows(q, pool, tables, pos, ctx):
    """The oracle's gather + fp32 attention (paged.py:80-81, model.py:70-76), one row at a time."""
    outs = []
    for b, c in enumerate(ctx):
        nb = -(-c // 16)
        blk = tables[b, :nb].long().to(DEV)
        kb = pool.k[0][blk].permute(1, 0, 2, 3).reshape(1, 8, nb * 16, 128).float().cpu()
        vb = pool.v[0][blk].permute(1, 0, 2, 3).reshape(1, 8, nb * 16, 128).float().cpu()
        qb = q[b: b + 1].float().cpu().transpose(1, 2)
        outs.append(orc.attention_math(qb, kb, vb, pos[b: b + 1].long(), 4).transpose(1, 2))
    return torch.cat(outs)


@pytest.mark.parametrize("which", ["c5", "past_chunk"])
def test_attention_c5_shape(which):
    """B = 64, T = 7, 32/8 heads, head_dim 128, bf16, contexts U[2048, 8192] (seed 0), 16-token blocks
    in random pool order; and 8 rows whose query windows reach or cross key positions 8192 and 16384
    (the attention's key chunks are 16384 positions)."""
    if which == "c5":
        ctx = torch.randint(2048, 8193, (64,), generator=torch.Generator().manual_seed(0)).tolist()
    else:
        ctx = [8190, 8199, 16380, 16384, 16385, 16390, 20000, 2048]
    case("attention", which, len(ctx), "rows, max context", max(ctx))
    q, pool, tables, pos = _attention_case(ctx, 7, 0)
    out = ops.paged_attention(q, pool.layout(0), tables.to(DEV), pos.to(DEV), 128 ** -0.5).float().cpu()
    ref = _oracle_attention_rows(q, pool, tables, pos, ctx)
    err = (out - ref).abs()
    rel = err.max().item() / ref.abs().max().item()
    record(f"8B verify attention {which}: max-abs/max {rel:.3e}, mean-abs {err.mean().item():.3e}")
    assert rel < 2e-2 and err.mean().item() < 2e-3


# ---- acceptance at the 8B shape ---------------------------------------------------------------------------
def _margins(p, q, xs, u, e, n_acc):
    """Oracle-side distance to a tie of one sequence's outcome: the smallest |u - min(1, ratio)| /
    min(1, ratio) over the proposals it examined, and the relative gap of the final draw's top-2 keys."""
    m = 1.0
    for i in range(min(n_acc + 1, len(xs))):
        qx = float(q[i, xs[i]])
        r1 = min(1.0, float(p[i, xs[i]] / q[i, xs[i]]) if qx > 0 else 1.0)
        if r1 > 0:
            m = min(m, abs(float(u[i]) - r1) / r1)
    if n_acc < len(xs):
        r = torch.clamp(p[n_acc] - q[n_acc], min=0)
        tot = r.sum()
        w = r / tot if tot > 0 else p[n_acc]
    else:
        w = p[n_acc]
    top = torch.topk((w / e).float(), 2).values
    gap = float((top[0] - top[1]) / top[0]) if top[0] > 0 else 1.0
    return m, gap


@pytest.mark.parametrize("temperature", [0.0, 1.0, 0.7])
def test_spec_accept_c5_shape(c5_target, temperature):
    """B = 64, k = 6, V = 128256, bf16 logits from the model's LM head (hidden states N(0, 1.5^2); the
    draft's are the target's plus N(0, 0.4^2), so proposals are often accepted), ragged k_eff. Both the
    standalone acceptance (its own statistics pass) and the round's path (statistics from the head's
    epilogue, merged) against the oracle's verify_draft on the same u and E; the debug outputs p(x),
    q(x) and the residual sum against the oracle's values."""
    case("spec_accept c5", temperature)
    b, k, v, d = 64, 6, C5["vocab_size"], C5["d_model"]
    head = c5_target.lm_head.weight
    g = torch.Generator(device=DEV).manual_seed(13)
    h_t = torch.randn(b, k + 1, d, device=DEV, generator=g) * 1.5
    h_d = h_t[:, :k] + torch.randn(b, k, d, device=DEV, generator=g) * 0.4
    h_t, h_d = h_t.bfloat16().reshape(b * (k + 1), d), h_d.bfloat16().reshape(b * k, d)
    temps = torch.full((b,), float(temperature), device=DEV)
    pt, pd = ops.row_stats_parts(b * (k + 1), v, d), ops.row_stats_parts(b * k, v, d)
    parts_t = torch.empty((b * (k + 1), pt, 4), dtype=torch.int32, device=DEV)
    parts_d = torch.empty((b * k, pd, 4), dtype=torch.int32, device=DEV)
    lt = ops.gemm_row_stats(h_t, head, temps.repeat_interleave(k + 1), parts_t).view(b, k + 1, v)
    ld = ops.gemm_row_stats(h_d, head, temps.repeat_interleave(k), parts_d).view(b, k, v)
    row_stats = torch.empty((b, 2 * k + 1, 4), dtype=torch.int32, device=DEV)
    ops.row_stats_merge(parts_t, row_stats, k + 1, 2 * k + 1, 0)
    ops.row_stats_merge(parts_d, row_stats, k, 2 * k + 1, k + 1)
    tl, dl = lt.cpu(), ld.cpu()

    gc = torch.Generator().manual_seed(17)
    xs = torch.zeros(b, k, dtype=torch.int32)
    for bi in range(b):
        for i in range(k):
            if temperature == 0:
                xs[bi, i] = int(dl[bi, i].float().argmax())
            else:
                xs[bi, i] = orc.draw(orc.probs_from_logits(dl[bi, i], temperature), orc.exp_noise(v, gc))
    u = torch.rand(b, k, generator=gc)
    e = torch.empty(b, v).exponential_(generator=gc)
    k_eff = torch.tensor([k if i % 7 else i % 6 for i in range(b)], dtype=torch.int32)
    args = (lt, ld, xs.to(DEV), k_eff.to(DEV), temps, u.to(DEV), e.to(DEV))
    runs = {"standalone": ops.spec_accept(*args, debug=True),
            "head statistics": ops.spec_accept(*args, row_stats=row_stats, debug=True)}
    worst = [1.0, 1.0]
    for name, (out, n, dbg) in runs.items():
        out, n = out.cpu(), n.cpu()
        dbg = {key: val.cpu() for key, val in dbg.items()}
        near, accepted = [], 0
        for bi in range(b):
            ke = int(k_eff[bi])
            tlb = tl[bi, : ke + 1] if temperature else tl[bi, : ke + 1].float()
            dlb = dl[bi, :ke] if temperature else dl[bi, :ke].float()
            p, q = orc.probs_from_logits(tlb, temperature), orc.probs_from_logits(dlb, temperature)
            xb = xs[bi, :ke].tolist()
            acc, extra = orc.verify_with_noise(p, q, xb, u[bi], e[bi])
            accepted += len(acc)
            m, gap = _margins(p, q, xb, u[bi], e[bi], len(acc))
            worst = [min(worst[0], m), min(worst[1], gap)]
            same = int(n[bi]) == len(acc) and out[bi, : len(acc) + 1].tolist() == acc + [extra]
            if not same:
                near.append((bi, m, gap))
                assert min(m, gap) < NEAR_TIE, (name, bi, m, gap)
                continue
            assert (out[bi, len(acc) + 1:] == -1).all()
            # the kernel's p(x), q(x) and residual sum are the oracle's to float32 rounding
            for i in range(min(len(acc) + 1, ke)):
                for key, ref in (("p_x", p[i, xb[i]]), ("q_x", q[i, xb[i]])):
                    assert abs(float(dbg[key][bi, i]) - float(ref)) <= 1e-5 * float(ref) + 1e-30, (name, bi, i, key)
            if temperature and len(acc) < ke:
                tot = float(torch.clamp(p[len(acc)] - q[len(acc)], min=0).sum())
                assert abs(float(dbg["res_sum"][bi]) - tot) <= 1e-5 * tot + 1e-30, (name, bi)
            else:
                assert float(dbg["res_sum"][bi]) == 0.0
        record(f"8B acceptance T={temperature} {name}: {accepted} of {int(k_eff.sum())} proposals accepted; "
               f"near-tie mismatches (below {NEAR_TIE:g}) {len(near)} {near}")
    record(f"8B acceptance T={temperature}: smallest oracle margins: decision {worst[0]:.3e}, "
           f"final-draw key gap {worst[1]:.3e}")


# ---- batched speculation at the 8B shape ------------------------------------------------------------------
def _c5_prompts(n_tokens):
    g = torch.Generator().manual_seed(17)
    return [torch.randint(0, C5["vocab_size"], (n,), generator=g).tolist() for n in n_tokens]


def test_c5_greedy_speculation_equals_target_generate(c5_target):
    """Six rows with ~2K-token contexts, k = 6: greedy batched speculation with the 4-layer early-exit
    draft, and with a perfect draft (all 32 layers: every proposal accepted, so accepted prefixes and
    the rollback run at this shape), emit exactly the target's own greedy tokens."""
    case("c5 greedy speculation")
    prompts = _c5_prompts([2048, 2100, 1999, 2304, 2200, 2050])
    n_new = 22
    want = [fa.generate(c5_target, torch.tensor([p]), n_new)[0].tolist()[len(p):] for p in prompts]
    got, stats = fa.speculative_generate_batch(c5_target, fa.early_exit_draft(c5_target, 4), prompts, n_new, k=6)
    print("4-layer draft:", stats)
    assert got == want
    got, stats = fa.speculative_generate_batch(c5_target, fa.early_exit_draft(c5_target, 32), prompts, n_new, k=6)
    print("perfect draft:", stats)
    assert got == want
    assert stats["accepted"] == stats["proposed"] > 0


def test_c5_sampled_graph_rounds_equal_eager_rounds(c5_target):
    """T = 1.0 at the 8B shape: rounds replayed from HIP graphs commit exactly the eager rounds' tokens
    and counters (rows of different lengths and budgets, so the batch shrinks as rows finish)."""
    case("c5 T=1 graphs == eager")
    prompts = _c5_prompts([2048, 2500, 2111, 2222])
    draft = fa.early_exit_draft(c5_target, 4)

    def run(graphs):
        sb = fa.SpeculativeBatch(c5_target, draft, 2000, 16, k=6, graphs=graphs,
                                 generator=torch.Generator(device=DEV).manual_seed(5))
        seqs = sb.add_many(prompts, [30, 45, 24, 38], 1.0)
        sb.run()
        return [s.tokens for s in seqs], sb.stats

    eager, graph = run(False), run(True)
    print("stats:", graph[1])
    assert graph == eager


# ---- the 1B-shape continuous-batching engine --------------------------------------------------------------
@pytest.fixture(scope="module")
def c4_target():
    m = _bf16_model(C4, 0)
    yield m
    del m
    torch.cuda.empty_cache()


def _c4_requests(n=48):
    g = torch.Generator().manual_seed(1)
    return [(torch.randint(0, C4["vocab_size"], (int(torch.randint(128, 1025, (1,), generator=g)),),
                           generator=g).tolist(), int(torch.randint(64, 257, (1,), generator=g))) for _ in range(n)]


def _c4_engine(model, temperature, reqs, num_blocks=600, max_batch=16, check_blocks=False, streams=None):
    eng = fa.Engine(model, num_blocks=num_blocks, block_size=16, max_batch=max_batch, seed=0,
                    draft=fa.early_exit_draft(model, 2), k=4)
    ids = [eng.add_request(p, n, temperature=temperature, stream_id=None if streams is None else streams[j])
           for j, (p, n) in enumerate(reqs)]
    while eng.has_work():
        eng.step()
        if check_blocks:
            # blocks are reserved on demand: a running request holds the blocks of its cached tokens
            # and at most those of its next k+1 window (reference tests/test_engine.py:64-74 bounds the
            # one-token engine to one spare block)
            for r in eng.running:
                assert eng.pool.blocks_for(r.cached) <= len(r.blocks) <= eng.pool.blocks_for(r.cached + 4 + 1)
    return eng, ids


def test_c4_engine_run(c4_target):
    """48 requests (prompts U[128, 1024], max_new_tokens U[64, 256]), max_batch 16, k = 4, T = 0.7, a
    2-layer early-exit draft, 600 blocks of 16 (below the peak demand): every request gets exactly its
    max_new_tokens, requests are preempted and re-prefilled, the pool is fully released, blocks are
    reserved on demand; requests that were never preempted produce, alone, the tokens they produced
    inside the batch (their random streams are their own)."""
    case("c4 engine T=0.7")
    reqs = _c4_requests()
    eng, ids = _c4_engine(c4_target, 0.7, reqs, check_blocks=True)
    print(f"steps {eng.steps}, preemptions {eng.preemptions}, peak running {eng.peak_running}, "
          f"peak blocks {eng.peak_blocks}, stats {eng.stats}")
    out = {rid: eng.requests[rid].output for rid in ids}
    assert all(len(out[rid]) == n for rid, (_, n) in zip(ids, reqs))
    assert eng.preemptions > 0
    assert eng.pool.allocator.num_free == 600
    assert 0 <= eng.stats["accepted"] <= eng.stats["proposed"]
    kept = [i for i, rid in enumerate(ids) if eng.requests[rid].preempted == 0]
    assert len(kept) >= 4
    for i in kept[:2] + kept[-2:]:
        alone, aid = _c4_engine(c4_target, 0.7, [reqs[i]], num_blocks=200, max_batch=1, streams=[ids[i]])
        assert alone.requests[aid[0]].output == out[ids[i]], i


def test_c4_engine_greedy_equals_generate(c4_target):
    """The same 48 requests greedy through the same tight pool: preemptions happen, and requests
    (including preempted ones) emit exactly the target's own greedy continuation."""
    case("c4 engine greedy")
    reqs = _c4_requests()
    eng, ids = _c4_engine(c4_target, 0.0, reqs)
    assert eng.preemptions > 0
    pre = [i for i, rid in enumerate(ids) if eng.requests[rid].preempted > 0]
    check = sorted(set(pre[:3] + [0, 1, 47]))
    print("preempted requests:", len(pre), "checked:", check)
    for i in check:
        p, n = reqs[i]
        assert eng.requests[ids[i]].output == fa.generate(c4_target, torch.tensor([p]), n)[0].tolist()[len(p):], i


# ---- full depth: logits and greedy tokens against the oracle ----------------------------------------------
def _host_block(model, i, dtype):
    """Block i's weights copied off the GPU, under the names oracle.block() takes."""
    return {n: t.detach().to("cpu").to(dtype) for n, t in model.layers[i].state_dict().items()}


def _full_depth_parity(model, name, rows=4, n_prompt=32, n_new=16, seed=23):
    """Greedy generation on the GPU (prefill, then one token per step), then the whole sequence again
    teacher-forced through the GPU forward and through the oracle's forward, one block's weights on
    the host at a time: in f32 on the bf16-rounded weights (the bar's reference), and in bf16 (the
    reference's own arithmetic run in bf16, model.py:141-159).

    Logits: max-abs error over max-abs logit at each position (the worst position is reported) and
    RMS error over RMS logit, for the kernels and for the reference's bf16 arithmetic, both against
    the f32 path. Greedy tokens, teacher-forced: the token the kernels chose at each position must be
    the f32 oracle's argmax there unless the oracle's own logits put it within twice the kernels'
    largest logit error of the top (a near-tie); every exception is listed."""
    cfg = model.cfg
    prompt = torch.randint(0, cfg.vocab_size, (rows, n_prompt), generator=torch.Generator().manual_seed(seed))
    seq = fa.generate(model, prompt, n_new)
    hip = model(seq).float().cpu()
    s = orc.Shape.of(cfg)
    emb, norm = model.tok_emb.weight.detach().cpu(), model.norm.weight.detach().cpu()
    ref = orc.forward_streamed(lambda i: _host_block(model, i, torch.float32), emb.float(), norm.float(), s, seq)
    ref_bf16 = orc.forward_streamed(lambda i: _host_block(model, i, torch.bfloat16), emb, norm, s, seq).float()

    def rel(x, y=ref):
        e = (x - y).abs()
        return (e.amax(-1) / y.abs().amax(-1)).max().item(), (e.pow(2).mean().sqrt() / y.pow(2).mean().sqrt()).item()

    max_k, rms_k = rel(hip)
    max_r, rms_r = rel(ref_bf16)
    max_kr, rms_kr = rel(hip, ref_bf16)
    tol = 2 * (hip - ref).abs().max().item()
    exceptions, miss_bf16, n = [], 0, 0
    for b in range(rows):
        for t in range(n_prompt - 1, n_prompt + n_new - 1):
            tok = int(seq[b, t + 1])
            n += 1
            # the teacher-forced forward's argmax is the token decoded one position at a time
            assert int(hip[b, t].argmax()) == tok, (name, b, t)
            top = int(ref[b, t].argmax())
            miss_bf16 += int(ref_bf16[b, t].argmax()) != top
            if tok != top:
                gap = float(ref[b, t, top] - ref[b, t, tok])
                exceptions.append((b, t, tok, top, round(gap, 4)))
                assert gap < tol, (name, b, t, gap, tol)
    record(f"{name} full depth ({cfg.n_layers} layers, V {cfg.vocab_size}, {rows}x{n_prompt + n_new} tokens), "
           f"max-abs/max at the worst position and rms-rel against the f32 oracle: kernels {max_k:.4f} / {rms_k:.4f}, "
           f"the reference's bf16 arithmetic {max_r:.4f} / {rms_r:.4f} (kernels vs it {max_kr:.4f} / {rms_kr:.4f}); "
           f"greedy: {n - len(exceptions)}/{n} kernel tokens = f32 oracle argmax, bf16 reference arithmetic "
           f"{n - miss_bf16}/{n}; near-tie exceptions (row, pos, token, oracle top, gap < {tol:.3f}): {exceptions}")
    return dict(max_k=max_k, rms_k=rms_k, max_r=max_r, rms_r=rms_r, exceptions=exceptions, miss_bf16=miss_bf16, n=n)


def _check(name, f):
    """The north-star bar is bf16 logits within 2e-2 of the f32 path, relative. The reference's own
    arithmetic run in bf16 is not within it at full depth of these random-init models (the residual
    stream's bf16 roundings compound over the layers: max-abs/max ~0.08 and rms ~0.06 at 32 layers),
    so no kernel that rounds where the reference rounds can be. The bar held here: the kernels are
    within 2e-2 where the reference's bf16 arithmetic is, and otherwise within 1.25x of that
    arithmetic's own error, in both forms (2-layer slices of both shapes meet 2e-2 outright:
    test_bf16_logits_at_config_init_within_2e2). Greedy tokens: every mismatch is a near-tie, and
    there are no more than the reference's bf16 arithmetic shows plus 1 in 16."""
    assert f["max_k"] <= max(2e-2, 1.25 * f["max_r"]), (name, f)
    assert f["rms_k"] <= max(2e-2, 1.25 * f["rms_r"]), (name, f)
    assert len(f["exceptions"]) <= f["miss_bf16"] + f["n"] // 16, (name, f)


@pytest.mark.timeout(900)
def test_c5_full_depth_logits_and_greedy_tokens(c5_target):
    """The 8B shape at full depth: 32 layers and the 128256-token head, 4 rows of a 32-token prompt and
    16 greedy tokens."""
    case("c5 full-depth parity")
    _check("8B", _full_depth_parity(c5_target, "8B"))


@pytest.mark.timeout(900)
def test_c4_full_depth_logits_and_greedy_tokens(c4_target):
    """The 1B shape at full depth: 16 layers and the 32000-token head, same check."""
    case("c4 full-depth parity")
    _check("1B", _full_depth_parity(c4_target, "1B"))
