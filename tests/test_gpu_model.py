"""The decoder, the caches, generate, speculative decoding and the engine on the GPU against the
reference's own outputs (tests/golden/) and the CPU oracle."""

import numpy as np
import pytest
import torch

import forgeserve_amd as fa
from helpers import C1, SMALL, golden_json, golden_npz, oracle_model, product_model
from oracle import reference_cpu as orc

pytestmark = pytest.mark.gpu


def case(*a):
    print("case:", *a, flush=True)


@pytest.fixture(scope="module")
def small():
    return product_model(SMALL, 1, 0.25)


@pytest.fixture(scope="module")
def small_draft():
    return product_model(SMALL, 7, 0.25)


def _max_abs(got, want):
    err = float(np.abs(np.asarray(got, dtype=np.float64) - np.asarray(want, dtype=np.float64)).max())
    print(f"fp32 logits: max-abs error {err:.3e} (bar 1e-4)")
    return err


def test_small_logits_match_reference(small):
    """fp32 logits within 1e-4 max-abs of the reference's own (golden) logits."""
    case("small logits")
    gold = golden_npz("model_small.npz")
    idx = torch.from_numpy(gold["idx"])
    assert _max_abs(small(idx).cpu().numpy(), gold["logits"]) <= 1e-4
    shifted = small(idx[:1, :5], positions=torch.arange(5)[None] + 11)
    assert _max_abs(shifted.cpu().numpy(), gold["logits_shifted"]) <= 1e-4


def test_cache_one_token_at_a_time_matches_full_forward(small):
    """tests/test_model.py:31-42 of the reference."""
    case("cache equivalence")
    idx = torch.randint(0, 64, (2, 20))
    kv = fa.new_contiguous_cache(3)
    steps = torch.cat([small(idx[:, i: i + 1], kv=kv) for i in range(20)], dim=1)
    torch.testing.assert_close(steps, small(idx), atol=1e-4, rtol=1e-4)
    kv = fa.new_contiguous_cache(3)
    small(idx[:, :10], kv=kv)
    torch.testing.assert_close(small(idx[:, 10:], kv=kv), small(idx)[:, 10:], atol=1e-4, rtol=1e-4)


def test_paged_forward_matches_reference(small):
    case("paged forward")
    gold = golden_npz("model_small.npz")
    seq = torch.from_numpy(gold["paged_seq"])
    table = torch.from_numpy(gold["paged_table"])
    pool = fa.PagedKVPool(small.cfg, num_blocks=16, block_size=4)
    got = [small(seq[:, :12], torch.arange(12)[None], pool.views(table, torch.arange(12)[None]))]
    for i in range(12, 30):
        pos = torch.tensor([[i]])
        got.append(small(seq[:, i: i + 1], pos, pool.views(table, pos)))
    assert _max_abs(torch.cat(got, 1).cpu().numpy(), gold["paged_logits"]) <= 1e-4


@pytest.mark.parametrize("key_layout", ["slots", "groups"])
def test_paged_update_write_then_read_back(key_layout):
    """tests/test_paged.py:20-41 of the reference through PagedLayerView.update (keys slot-major, or
    stored as 8-dim groups: the same values through the reference-shaped reads)."""
    case("paged update", key_layout)
    cfg = fa.ModelConfig(vocab_size=64, d_model=64, n_layers=3, n_heads=8, n_kv_heads=4, max_seq_len=64)
    pool = fa.PagedKVPool(cfg, num_blocks=10, block_size=4, key_layout=key_layout)
    table = torch.tensor([[7, 2, 9]])
    k = torch.randn(1, 4, 10, 8, device="cuda")
    v = torch.randn_like(k)
    k_all, v_all = pool.views(table, torch.arange(10)[None])[0].update(k, v)
    assert k_all.shape == (1, 4, 12, 8)
    assert torch.equal(k_all[:, :, :10], k) and torch.equal(v_all[:, :, :10], v)
    keys = pool.k[0].flatten(-2) if key_layout == "groups" else pool.k[0]
    assert torch.equal(keys[2, :, 1], k[0, :, 5]) and torch.equal(pool.v[0][2, :, 1], v[0, :, 5])
    pool = fa.PagedKVPool(cfg, num_blocks=8, block_size=4, key_layout=key_layout)
    k = torch.randn(2, 4, 6, 8, device="cuda")
    k_all, _ = pool.views(torch.tensor([[0, 1], [2, 3]]), torch.arange(6)[None].expand(2, 6))[0].update(k, k.clone())
    assert torch.equal(k_all[:, :, :6], k)


def test_generate_matches_reference(small):
    case("generate")
    gold = golden_json("model_small.json")
    for i, p in enumerate(gold["prompts"]):
        assert fa.generate(small, torch.tensor([p]), 20)[0].tolist() == gold["generate_greedy"][i]
        got = fa.generate(small, torch.tensor([p]), 20, temperature=1.0, generator=torch.Generator().manual_seed(21 + i))
        assert got[0].tolist() == gold["generate_t1"][i]


def test_speculative_matches_reference_streams(small, small_draft):
    case("speculative golden")
    gold = golden_json("model_small.json")
    for kk in (1, 3, 6):
        for p, want in zip(gold["prompts"], gold["spec"][f"greedy_k{kk}"]):
            assert list(fa.speculative_generate(small, small_draft, p, 20, k=kk)) == want, (kk, p)
    for i, (p, want) in enumerate(zip(gold["prompts"], gold["spec"]["t1_k3"])):
        got = fa.speculative_generate(small, small_draft, p, 20, k=3, temperature=1.0,
                                      generator=torch.Generator().manual_seed(31 + i))
        assert list(got) == want, p
    for i, (p, want) in enumerate(zip(gold["prompts"], gold["spec"]["t07_k4_self"])):
        got = fa.speculative_generate(small, small, p, 25, k=4, temperature=0.7,
                                      generator=torch.Generator().manual_seed(41 + i))
        assert list(got) == want, p


def test_speculative_stopping_and_vocab_checks(small, small_draft):
    """tests/test_speculative.py:46-57 of the reference."""
    case("speculative stopping")
    for n in (1, 2, 7):
        got, _ = fa.speculative_generate(small, small_draft, [1, 2, 3], n, k=5)
        assert len(got) == n
    got, _ = fa.speculative_generate(small, small_draft, list(range(1, 60)), 100, k=4)
    assert 59 + len(got) == small.cfg.max_seq_len
    other = product_model(dict(SMALL, vocab_size=32), 7, 0.25)
    with pytest.raises(ValueError):
        fa.speculative_generate(small, other, [1, 2], 3)


def test_c1_end_to_end_matches_reference():
    """Tiny config: 4 layers, d 256, 8/4 heads, ffn 688, vocab 512, fp32, early-exit draft of 1 layer,
    k=4, 64 new tokens: logits, greedy and seeded T=0.8 speculative tokens + stats equal the reference's."""
    case("c1")
    target = product_model(C1, 0, 0.02)
    draft = fa.early_exit_draft(target, 1)
    gold = golden_json("model_c1.json")
    prompt = gold["prompt"]
    assert _max_abs(target(torch.tensor([prompt]))[0].cpu().numpy(), golden_npz("model_c1.npz")["logits"]) <= 1e-4
    assert fa.generate(target, torch.tensor([prompt]), 64)[0].tolist()[16:] == gold["greedy"]
    assert list(fa.speculative_generate(target, draft, prompt, 64, k=4)) == gold["spec_greedy"]
    got = fa.speculative_generate(target, draft, prompt, 64, k=4, temperature=0.8,
                                  generator=torch.Generator().manual_seed(2))
    assert list(got) == gold["spec_t08"]


def test_engine_matches_reference_runs(small):
    case("engine golden")
    gold = golden_json("engine_runs.json")
    for name, run in gold["runs"].items():
        e = fa.Engine(small, num_blocks=run["num_blocks"], block_size=4, max_batch=5, seed=run["seed"])
        ids = [e.add_request(p, n, temperature=run["temperature"]) for p, n in gold["requests"]]
        out = e.run()
        assert [out[i] for i in ids] == run["outputs"], name
        assert e.preemptions == run["preemptions"], name
        assert e.pool.allocator.num_free == run["num_blocks"]


def test_engine_errors(small):
    """tests/test_engine.py:106-120 of the reference."""
    case("engine errors")
    e = fa.Engine(small, num_blocks=4, block_size=4)
    with pytest.raises(ValueError):
        e.add_request([], 5)
    with pytest.raises(ValueError):
        e.add_request(list(range(1, 40)), 5)
    e = fa.Engine(small, num_blocks=2, block_size=4)
    e.add_request([1, 2, 3, 4, 5], 30)
    with pytest.raises(RuntimeError):
        e.run()


# ---- bf16 models on the MFMA path ------------------------------------------------------------------------
BF = dict(vocab_size=1000, d_model=512, n_layers=3, n_heads=4, n_kv_heads=1, ffn_dim=1024, max_seq_len=512)


@pytest.fixture(scope="module")
def bf_target():
    return product_model(BF, 3, 0.06, dtype=torch.bfloat16)


def _rel(got, ref):
    """(max-abs error / max-abs value, RMS error / RMS value)."""
    e = (got - ref).abs()
    return e.max().item() / ref.abs().max().item(), (e.pow(2).mean().sqrt() / ref.pow(2).mean().sqrt()).item()


def test_bf16_logits_within_tolerance(bf_target):
    """bf16 logits against the reference's f32 math on the same bf16-rounded weights. The bound is the
    error of the reference's own arithmetic run in bf16 (model.py computed in bf16 on the CPU) against
    its f32 path, with 25% headroom: the kernels are no less accurate than the reference in bf16."""
    case("bf16 logits")
    w, s = oracle_model(BF, 3, 0.06)
    wb = {k: v.bfloat16() for k, v in w.items()}
    idx = torch.randint(0, 1000, (2, 40))
    ref = orc.forward({k: v.float() for k, v in wb.items()}, s, idx)
    ref_bf16 = orc.forward(wb, s, idx).float()
    got = bf_target(idx).float().cpu()
    bound_max, bound_rms = _rel(ref_bf16, ref)
    got_max, got_rms = _rel(got, ref)
    print(f"reference bf16 path: {bound_max:.4f} / {bound_rms:.4f}; kernels: {got_max:.4f} / {got_rms:.4f}")
    assert got_max <= 1.25 * bound_max and got_rms <= 1.25 * bound_rms


@pytest.mark.parametrize("shape", ["small", "c4 slice", "c5 slice"])
def test_bf16_logits_at_config_init_within_2e2(shape):
    """With the configs' N(0, 0.02) init, bf16 logits are within 2e-2 of the f32 math on the same
    bf16-rounded weights, as max-abs error over max-abs logit; also on 2-layer
    slices of the 1B shape (d 2048, 32/8 heads, head_dim 64, ffn 8192) and of the 8B shape (d 4096,
    32/8 heads, head_dim 128, ffn 14336), with a 32000-token vocabulary."""
    case("bf16 logits 0.02 init", shape)
    cfg = {"small": dict(vocab_size=2000, d_model=1024, n_layers=4, n_heads=8, n_kv_heads=2, ffn_dim=2816),
           "c4 slice": dict(vocab_size=32000, d_model=2048, n_layers=2, n_heads=32, n_kv_heads=8, ffn_dim=8192),
           "c5 slice": dict(vocab_size=32000, d_model=4096, n_layers=2, n_heads=32, n_kv_heads=8, ffn_dim=14336)}[shape]
    cfg["max_seq_len"] = 512
    w, s = oracle_model(cfg, 5, 0.02)
    wb = {k: v.bfloat16().float() for k, v in w.items()}
    model = product_model(cfg, 5, 0.02, dtype=torch.bfloat16)
    idx = torch.randint(0, cfg["vocab_size"], (3, 33))
    got_max, got_rms = _rel(model(idx).float().cpu(), orc.forward(wb, s, idx))
    print(f"kernels vs f32: max-relative {got_max:.4f}, rms-relative {got_rms:.4f}")
    assert got_max <= 2e-2


def test_bf16_speculative_batch_equals_greedy_generate(bf_target):
    """Batched paged speculation (greedy) emits exactly the target's own greedy tokens, bit for bit,
    for every row: verify, decode and prefill rows are computed identically (batch invariance)."""
    case("bf16 batch == greedy")
    draft = fa.early_exit_draft(bf_target, 1)
    g = torch.Generator().manual_seed(9)
    prompts = [torch.randint(0, 1000, (int(n),), generator=g).tolist() for n in torch.randint(2, 60, (6,), generator=g)]
    want = [fa.generate(bf_target, torch.tensor([p]), 40)[0].tolist()[len(p):] for p in prompts]
    got, stats = fa.speculative_generate_batch(bf_target, draft, prompts, 40, k=4)
    assert got == want
    assert stats["accepted"] <= stats["proposed"]
    single, _ = fa.speculative_generate(bf_target, draft, prompts[0], 40, k=4)
    assert single == want[0]


def test_bf16_batch_perfect_draft_accepts_everything(bf_target):
    case("bf16 perfect draft")
    prompts = [[1, 2, 3], [4, 5, 6, 7, 8]]
    got, stats = fa.speculative_generate_batch(bf_target, bf_target, prompts, 25, k=4)
    assert stats["accepted"] == stats["proposed"]
    assert got == [fa.generate(bf_target, torch.tensor([p]), 25)[0].tolist()[len(p):] for p in prompts]


@pytest.mark.parametrize("which", ["bf16", "f32"])
def test_packed_prefill_equals_per_sequence_prefill(which, bf_target, small):
    """Several prompts prefilled in one packed forward (no padding rows) leave the pool holding exactly
    what one-prompt-per-step prefills (engine.py:80-95) leave, and give the same last-token logits;
    one prompt starts after a cached prefix."""
    case("packed prefill", which)
    model = bf_target if which == "bf16" else small
    cfg, bs = model.cfg, 16 if which == "bf16" else 4
    g = torch.Generator().manual_seed(31)
    prompts = [torch.randint(0, cfg.vocab_size, (int(n),), generator=g).tolist() for n in (23, 1, 40, 9)]
    prefix = torch.randint(0, cfg.vocab_size, (11,), generator=g).tolist()

    def pools():
        pool = fa.PagedKVPool(cfg, 64, bs, dtype=model.dtype, device="cuda")
        lists = [pool.allocator.allocate(pool.blocks_for(len(p) + (11 if i == 2 else 0))) for i, p in enumerate(prompts)]
        # sequence 2 first caches an 11-token prefix, then prefills its prompt after it
        pos = torch.arange(11)[None]
        model(torch.tensor([prefix]), pos, pool.views(torch.tensor([lists[2]]), pos))
        return pool, lists

    alone_pool, lists = pools()
    alone = []
    for i, p in enumerate(prompts):
        st = 11 if i == 2 else 0
        pos = torch.arange(st, st + len(p))[None]
        alone.append(model(torch.tensor([p]), pos, alone_pool.views(torch.tensor([lists[i]]), pos))[0, -1])
    packed_pool, lists2 = pools()
    assert lists2 == lists
    got = fa.prefill_packed(model, packed_pool, prompts, lists, starts=[0, 0, 11, 0])
    assert torch.equal(got, torch.stack(alone))
    assert torch.equal(packed_pool.k_store, alone_pool.k_store) and torch.equal(packed_pool.v_store, alone_pool.v_store)


def test_long_packed_prefill_equals_per_sequence_prefill():
    """At the 8B layer shape (two blocks, d 4096, 32/8 heads, head_dim 128, ffn 14336), a 4400-token
    packed forward runs the qkv and wo projections with their K splits inside each workgroup and the
    long-batch tile order, the one-prompt prefills run them through split-K partials: the pool and the
    last-token logits are the same bit for bit."""
    case("long packed prefill")
    from forgeserve_amd import _lib
    lib = _lib.load()
    assert lib.fs_gemm_serial(4400, 6144, 4096, _lib.BF16) and lib.fs_gemm_serial(4400, 4096, 4096, _lib.BF16)
    assert not lib.fs_gemm_serial(1500, 6144, 4096, _lib.BF16)
    cfg = fa.ModelConfig(vocab_size=32000, d_model=4096, n_layers=2, n_heads=32, n_kv_heads=8, ffn_dim=14336,
                         max_seq_len=2048)
    torch.manual_seed(5)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device("cuda"):
            model = fa.ForgeModel(cfg).eval()
    finally:
        torch.set_default_dtype(prev)
    g = torch.Generator().manual_seed(32)
    prompts = [torch.randint(0, cfg.vocab_size, (n,), generator=g).tolist() for n in (1500, 1200, 1300, 400)]

    def pool_and_lists():
        pool = fa.PagedKVPool(cfg, 300, 16, dtype=model.dtype, device="cuda", key_layout="groups")
        return pool, [pool.allocator.allocate(pool.blocks_for(len(p))) for p in prompts]

    alone_pool, lists = pool_and_lists()
    alone = []
    for i, p in enumerate(prompts):
        pos = torch.arange(len(p))[None]
        alone.append(model(torch.tensor([p]), pos, alone_pool.views(torch.tensor([lists[i]]), pos))[0, -1])
    packed_pool, lists2 = pool_and_lists()
    assert lists2 == lists
    got = fa.prefill_packed(model, packed_pool, prompts, lists)
    assert torch.equal(got, torch.stack(alone))
    assert torch.equal(packed_pool.k_store, alone_pool.k_store) and torch.equal(packed_pool.v_store, alone_pool.v_store)


@pytest.mark.parametrize("which", ["bf16", "f32"])
def test_shared_draft_cache_equals_separate_cache(which, bf_target, small):
    """An early-exit draft that reads and writes the target's cache for the blocks they share (and a
    verify pass that continues from the draft's residual streams) commits exactly the tokens of a draft
    with its own cache: greedy and sampled rows, sequences finishing at different rounds (ragged
    k_eff), graphs on."""
    case("shared draft cache", which)
    model = bf_target if which == "bf16" else small
    draft = fa.early_exit_draft(model, 2 if which == "bf16" else 1)
    cfg = model.cfg
    g = torch.Generator().manual_seed(41)
    prompts = [torch.randint(0, cfg.vocab_size, (int(n),), generator=g).tolist() for n in (5, 17, 2, 30, 9)]
    temps = [0.0, 0.9, 1.0, 0.0, 0.6]
    lim = cfg.max_seq_len

    def run(share):
        sb = fa.SpeculativeBatch(model, draft, 200, 4, k=3, generator=torch.Generator(device="cuda").manual_seed(2),
                                 share_kv=share)
        seqs = sb.add_many(prompts, [min(12 + 5 * i, lim - len(p) - 1) for i, p in enumerate(prompts)], temps)
        sb.run()
        return [s.tokens for s in seqs], sb.stats, sb.pool_d is sb.pool_t

    sep, shared = run(False), run(True)
    assert not sep[2] and shared[2]
    assert shared[0] == sep[0] and shared[1] == sep[1]


def test_spec_engine_shared_cache_equals_separate_cache(small):
    """The speculative engine with the draft on the model's pool gives the separate-pool engine's
    tokens: sampled rows through a roomy pool, greedy rows through a pool tight enough to preempt."""
    case("spec engine shared cache")
    draft = fa.early_exit_draft(small, 1)
    reqs = [([1, 2, 3], 20, 0.8), ([9, 8, 7, 6], 15, 0.0), ([5, 5], 18, 1.0), ([30, 31, 32, 33, 34], 12, 0.6)]

    def run(share, num_blocks, greedy):
        e = fa.Engine(small, num_blocks=num_blocks, block_size=4, max_batch=4, seed=5, draft=draft, k=3,
                      share_kv=share)
        ids = [e.add_request(p, n, temperature=0.0 if greedy else t) for p, n, t in reqs]
        out = e.run()
        return [out[i] for i in ids], e.preemptions, e.pool_d is e.pool

    roomy = run(False, 64, False), run(True, 64, False)
    assert not roomy[0][2] and roomy[1][2]
    assert roomy[1][0] == roomy[0][0]
    tight = run(False, 14, True), run(True, 14, True)
    assert tight[0][1] > 0 and tight[1][1] > 0
    assert tight[1][0] == tight[0][0]


def test_graph_rounds_equal_eager_rounds(bf_target):
    """Rounds replayed from captured HIP graphs commit exactly the eager rounds' tokens. Each shape is
    replayed many times with new inputs (and eager work, host copies and syncs in between); the batch
    shrinks as sequences finish, so several shapes are captured; greedy and sampled rows are mixed."""
    case("graph rounds == eager rounds")
    draft = fa.early_exit_draft(bf_target, 2)
    g = torch.Generator().manual_seed(21)
    prompts = [torch.randint(0, 1000, (int(n),), generator=g).tolist() for n in torch.randint(2, 90, (11,), generator=g)]
    temps = [0.0, 0.7, 1.0, 0.0, 1.3, 0.9, 0.0, 0.5, 1.0, 0.8, 0.0]

    def run(graphs):
        sb = fa.SpeculativeBatch(bf_target, draft, 400, 16, k=4,
                                 generator=torch.Generator(device="cuda").manual_seed(3), graphs=graphs)
        seqs = [sb.add(p, 30 + 3 * i, t) for i, (p, t) in enumerate(zip(prompts, temps))]
        sb.run()
        return [s.tokens for s in seqs], sb.stats

    eager, stats_e = run(False)
    graph, stats_g = run(True)
    assert stats_g["rounds"] >= 10
    assert graph == eager and stats_g == stats_e


@pytest.mark.parametrize("share", [True, False])
def test_queued_rounds_equal_rounds(bf_target, share):
    """run_rounds(n), which queues each round before reading the previous one's tokens (the next
    round's inputs computed on the GPU), commits exactly what n round() calls commit, with the same
    stats: a greedy batch whose sequences finish at different rounds by token budget and by EOS (the
    queue keeps running past them), and a sampled batch (queued while no sequence can finish inside
    the queue, then round by round)."""
    case("queued rounds == rounds", share)
    draft = fa.early_exit_draft(bf_target, 2)
    g = torch.Generator().manual_seed(31)
    prompts = [torch.randint(0, 1000, (int(n),), generator=g).tolist() for n in torch.randint(2, 70, (9,), generator=g)]

    def run(queued, temps, max_new, eos, rounds):
        sb = fa.SpeculativeBatch(bf_target, draft, 900, 16, k=4, share_kv=share,
                                 generator=torch.Generator(device="cuda").manual_seed(4))
        seqs = [sb.add(p, m, t, eos_id=e) for p, t, m, e in zip(prompts, temps, max_new, eos)]
        if queued:
            c = sb.run_rounds(rounds)
        else:
            c = sum(sb.round() for _ in range(rounds))
        return [s.tokens for s in seqs], [s.done for s in seqs], c, sb.stats

    greedy = [0.0] * 9
    budgets = [12, 40, 70, 25, 90, 8, 55, 33, 100]
    free = run(False, greedy, budgets, [None] * 9, 30)
    # EOS ids for three sequences: tokens their greedy continuation produces
    eos = [None] * 9
    for i in (1, 4, 6):
        gen = free[0][i][len(prompts[i]):]
        eos[i] = gen[min(7 + i, len(gen) - 1)]
    a = run(False, greedy, budgets, eos, 30)
    b = run(True, greedy, budgets, eos, 30)
    assert b == a
    assert any(a[1]) and not all(a[1])   # some sequences finished inside the run, some did not
    temps = [0.8, 1.0, 0.0, 1.2, 0.7, 0.0, 1.0, 0.9, 0.6]
    budgets = [60, 80, 70, 90, 200, 75, 65, 85, 120]
    a = run(False, temps, budgets, [None] * 9, 25)
    b = run(True, temps, budgets, [None] * 9, 25)
    assert b == a


def test_graph_engine_equals_eager_engine(small):
    """The speculative engine (f32 model: the generic kernels) gives the same tokens, preemptions and
    counters with graph-replayed rounds as with eager rounds, at T > 0 through a tight pool."""
    case("graph engine == eager engine")
    draft = fa.early_exit_draft(small, 1)
    reqs = [([1, 2, 3], 20, 0.8), ([9, 8, 7, 6], 15, 0.0), ([5, 5], 18, 1.0), ([30, 31, 32, 33, 34], 12, 0.6),
            ([7] * 9, 16, 0.9)]

    def run(graphs):
        e = fa.Engine(small, num_blocks=14, block_size=4, max_batch=4, seed=5, draft=draft, k=3, graphs=graphs)
        ids = [e.add_request(p, n, temperature=t) for p, n, t in reqs]
        out = e.run()
        return [out[i] for i in ids], e.preemptions, e.stats

    eager = run(False)
    graph = run(True)
    assert eager[1] > 0
    assert graph == eager


def _engine_outcome(model, reqs, queued, **kw):
    """Tokens, preemptions, steps, counters, peaks and free blocks of one Engine over `reqs`, driven by
    run() (queued: it may queue rounds back to back) or by step() one call at a time (never queues);
    also the steps run() took inside queued runs."""
    e = fa.Engine(model, **kw)
    ids = [e.add_request(p, n, temperature=t) for p, n, t in reqs]
    taken = []
    if queued:
        inner = e._queued_rounds
        e._queued_rounds = lambda: taken.append(inner()) or taken[-1]
        out = e.run()
    else:
        while e.has_work():
            e.step()
        out = {rid: r.output for rid, r in e.requests.items()}
    free = (e.pool.allocator.num_free, e.pool_d.allocator.num_free)
    return ([out[i] for i in ids], e.preemptions, e.steps, dict(e.stats), e.peak_blocks, e.peak_running, free), taken


@pytest.mark.parametrize("graphs", [True, False])
def test_engine_run_queued_rounds_equal_single_steps(small, graphs):
    """Engine.run() queues a speculative round behind the current one when the step after it is known
    to be another round (no request can finish in it, none is admitted first, the blocks fit). It gives
    what step() called once at a time gives: tokens (greedy and sampled), preemptions, steps, rounds,
    proposals, peaks and free blocks, through a roomy pool, one tight enough to preempt, and a separate
    draft pool; one request runs into max_seq_len."""
    case("engine queued rounds", graphs)
    draft = fa.early_exit_draft(small, 1)
    reqs = [([1, 2, 3], 40, 0.8), ([9, 8, 7, 6], 35, 0.0), ([5, 5], 38, 1.0), ([30, 31, 32, 33, 34], 30, 0.6),
            ([7] * 9, 36, 0.9), ([4, 4, 2], 33, 0.0), (list(range(20)), 60, 0.7)]
    for num_blocks, share in ((96, None), (26, None), (96, False)):
        kw = dict(num_blocks=num_blocks, block_size=4, max_batch=4, seed=5, draft=draft, k=3, graphs=graphs,
                  share_kv=share)
        got, taken = _engine_outcome(small, reqs, True, **kw)
        want, _ = _engine_outcome(small, reqs, False, **kw)
        assert got == want, num_blocks
        assert max(taken) >= 3, taken   # runs of queued rounds did happen
        if num_blocks == 26:
            assert got[1] > 0


def test_engine_run_queued_rounds_equal_single_steps_bf16(bf_target):
    """The same on the bf16 kernels (fused head statistics, grouped keys, a 2-layer draft on the target's
    cache), sampled and greedy requests through a pool that forces preemptions."""
    case("engine queued rounds bf16")
    draft = fa.early_exit_draft(bf_target, 2)
    g = torch.Generator().manual_seed(21)
    reqs = [(torch.randint(0, 1000, (int(n),), generator=g).tolist(), int(m), t)
            for n, m, t in zip(torch.randint(2, 60, (9,), generator=g), torch.randint(20, 70, (9,), generator=g),
                               [0.0, 0.7, 1.0, 0.0, 0.9, 0.5, 0.0, 0.8, 1.0])]
    kw = dict(num_blocks=22, block_size=16, max_batch=5, seed=9, draft=draft, k=4, key_layout="groups")
    got, taken = _engine_outcome(bf_target, reqs, True, **kw)
    want, _ = _engine_outcome(bf_target, reqs, False, **kw)
    assert got == want
    assert max(taken) >= 3 and got[1] > 0, (taken, got[1])


# ---- speculative engine (batched speculation inside Engine) ---------------------------------------------
@pytest.mark.parametrize("key_layout", ["slots", "groups"])
def test_spec_engine_greedy_matches_the_reference_engine(small, key_layout):
    """Greedy: the speculative engine emits the reference Engine's tokens exactly, through a pool small
    enough to force recompute preemptions (engine_runs.json, run greedy_tight), whichever key layout
    its pool uses."""
    case("spec engine greedy", key_layout)
    gold = golden_json("engine_runs.json")
    run = gold["runs"]["greedy_tight"]
    draft = fa.early_exit_draft(small, 1)
    e = fa.Engine(small, num_blocks=run["num_blocks"], block_size=4, max_batch=5, draft=draft, k=4,
                  key_layout=key_layout)
    ids = [e.add_request(p, n) for p, n in gold["requests"]]
    out = e.run()
    assert [out[i] for i in ids] == run["outputs"]
    assert e.preemptions > 0
    assert e.pool.allocator.num_free == run["num_blocks"] and e.pool_d.allocator.num_free == run["num_blocks"]
    assert e.stats["rounds"] > 0 and e.stats["accepted"] <= e.stats["proposed"]


@pytest.mark.parametrize("key_layout", ["slots", "groups"])
def test_spec_engine_bf16_greedy_equals_generate(bf_target, key_layout):
    case("spec engine bf16", key_layout)
    draft = fa.early_exit_draft(bf_target, 1)
    g = torch.Generator().manual_seed(11)
    reqs = [(torch.randint(0, 1000, (int(n),), generator=g).tolist(), int(m))
            for n, m in zip(torch.randint(2, 50, (7,), generator=g), torch.randint(3, 30, (7,), generator=g))]
    e = fa.Engine(bf_target, num_blocks=200, block_size=16, max_batch=4, draft=draft, k=3, key_layout=key_layout)
    ids = [e.add_request(p, m) for p, m in reqs]
    out = e.run()
    for rid, (p, m) in zip(ids, reqs):
        assert out[rid] == fa.generate(bf_target, torch.tensor([p]), m)[0].tolist()[len(p):], rid


def test_spec_engine_stops_at_eos_and_max_seq_len(small):
    case("spec engine stops")
    draft = fa.early_exit_draft(small, 1)
    prompt = [3, 1, 4, 1, 5]
    full = fa.generate(small, torch.tensor([prompt]), 10)[0].tolist()[len(prompt):]
    eos = full[3]
    e = fa.Engine(small, num_blocks=32, block_size=4, draft=draft, k=4)
    rid = e.add_request(prompt, 10, eos_id=eos)
    assert e.run()[rid] == full[: full.index(eos) + 1]
    e = fa.Engine(small, num_blocks=64, block_size=4, draft=draft, k=4)
    rid = e.add_request(list(range(1, 60)), 100)
    assert 59 + len(e.run()[rid]) == small.cfg.max_seq_len


def test_spec_engine_sampling_does_not_depend_on_the_batch(small):
    """At T > 0 a request's tokens come from its own keyed stream: alone or batched with others it
    produces the same tokens. (A recompute preemption re-prefills and samples the next token from the
    prefill logits, as the reference's engine does, which moves the request's round boundaries: a
    preempted request's later tokens are a different valid sample.)"""
    case("spec engine keyed sampling")
    draft = fa.early_exit_draft(small, 1)
    reqs = [([1, 2, 3], 20), ([9, 8, 7, 6], 15), ([5, 5], 18), ([30, 31, 32, 33, 34], 12)]

    def run(subset, num_blocks, streams=None):
        e = fa.Engine(small, num_blocks=num_blocks, block_size=4, max_batch=4, seed=5, draft=draft, k=3)
        ids = [e.add_request(p, n, temperature=0.8, stream_id=None if streams is None else streams[j])
               for j, (p, n) in enumerate(subset)]
        return [e.run()[i] for i in ids], e

    together, e1 = run(reqs, 64)
    assert e1.preemptions == 0
    for i, req in enumerate(reqs):   # every request, whatever its budget (its k_eff shrinks at the end)
        alone, _ = run([req], 64, streams=[i])
        assert together[i] == alone[0], i
    tight, e2 = run(reqs, 14)
    assert e2.preemptions > 0
    for (p, n), out, out2 in zip(reqs, together, tight):
        assert len(out) == n and all(0 <= t < small.cfg.vocab_size for t in out)
        assert len(out2) == n and all(0 <= t < small.cfg.vocab_size for t in out2)
    again, _ = run(reqs, 64)
    assert again == together


def test_spec_engine_errors(small):
    case("spec engine errors")
    other = fa.ForgeModel(fa.ModelConfig(vocab_size=32, d_model=64, n_layers=1, n_heads=8, n_kv_heads=4,
                                         max_seq_len=64))
    with pytest.raises(ValueError):
        fa.Engine(small, num_blocks=8, block_size=4, draft=other)
    with pytest.raises(ValueError):
        fa.Engine(small, num_blocks=8, block_size=4, draft=fa.early_exit_draft(small, 1), k=0)


# ---- sampling statistics of batched speculation ------------------------------------------------------------
TINY = dict(vocab_size=6, d_model=32, n_layers=2, n_heads=4, n_kv_heads=2, max_seq_len=16)


def _tiny_target_draft():
    """The reference's distribution test models (tests/test_speculative.py:84-93): vocabulary 6, weights
    N(0, 0.4^2), target and draft unrelated."""
    return product_model(TINY, 1, 0.4), product_model(TINY, 2, 0.4)


def _next_token_probs(model, prefix):
    return torch.softmax(model(torch.tensor([prefix]))[0, -1].float().cpu(), -1)


def _first_two_marginals(model, prompt):
    p1 = _next_token_probs(model, prompt)
    p2 = sum(p1[x] * _next_token_probs(model, prompt + [x]) for x in range(TINY["vocab_size"]))
    return p1, p2


def test_batched_speculation_follows_the_target_distribution():
    """tests/test_speculative.py:84-99 of the reference for the batched loop: 1,500 identical rows
    speculate together at T = 1 (k = 3, so the first token goes through the draft's proposal and the
    accept/residual test, not just the bonus draw); the frequencies of the first and second emitted
    tokens are within 0.05 of the target's own marginals."""
    case("batched speculation statistics")
    target, draft = _tiny_target_draft()
    prompt, n = [1, 2, 3], 1500
    p1, p2 = _first_two_marginals(target, prompt)
    sb = fa.SpeculativeBatch(target, draft, num_blocks=n, block_size=16, k=3,
                             generator=torch.Generator(device="cuda").manual_seed(5))
    seqs = sb.add_many([prompt] * n, 4, 1.0)
    sb.run()
    toks = torch.tensor([s.tokens[3:5] for s in seqs])
    f1 = torch.bincount(toks[:, 0], minlength=6).float() / n
    f2 = torch.bincount(toks[:, 1], minlength=6).float() / n
    print("first:", f1.tolist(), p1.tolist(), "second:", f2.tolist(), p2.tolist(), sb.stats)
    assert (f1 - p1).abs().max() < 0.05 and (f2 - p2).abs().max() < 0.05
    assert 0 < sb.stats["accepted"] < sb.stats["proposed"]


def test_speculative_engine_keyed_draws_follow_the_target_distribution():
    """The speculative Engine's keyed device draws: 1,500 requests of one prompt at T = 1. The first
    token comes from the prefill logits (keyed Exp(1) noise), the second from a speculation round
    (keyed draft noise, uniforms and final noise); both follow the target's marginals within 0.05."""
    case("keyed engine statistics")
    target, draft = _tiny_target_draft()
    prompt, n = [1, 2, 3], 1500
    p1, p2 = _first_two_marginals(target, prompt)
    e = fa.Engine(target, num_blocks=2 * n, block_size=16, max_batch=n, seed=3, draft=draft, k=3)
    ids = [e.add_request(prompt, 3, temperature=1.0) for _ in range(n)]
    out = e.run()
    toks = torch.tensor([out[i][:2] for i in ids])
    f1 = torch.bincount(toks[:, 0], minlength=6).float() / n
    f2 = torch.bincount(toks[:, 1], minlength=6).float() / n
    print("first:", f1.tolist(), p1.tolist(), "second:", f2.tolist(), p2.tolist(), e.stats)
    assert (f1 - p1).abs().max() < 0.05 and (f2 - p2).abs().max() < 0.05
    assert e.stats["rounds"] > 0
