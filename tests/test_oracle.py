"""Pin the CPU oracle (oracle/reference_cpu.py) before trusting it as the GPU checker.

Each oracle function is checked against what the reference itself produced (tests/golden/, written by
make_golden.py) and/or against a closed form or library identity chosen so that a plausible mistake
(a dropped term, a swapped operand, a wrong sign or index, a lost generator draw) fails.
"""

import math

import numpy as np
import pytest
import torch

from helpers import C1, SMALL, golden_json, golden_npz, oracle_model
from oracle import reference_cpu as orc


# ---- sampling / acceptance --------------------------------------------------------------------------
def test_multinomial_is_argmax_over_exponential_noise():
    """torch.multinomial(w, 1) == argmax(w / Exp(1)) with the same generator advance (the library
    identity the oracle's `draw` and the GPU kernels rely on)."""
    for trial in range(300):
        v = [3, 17, 512, 4096][trial % 4]
        g0 = torch.Generator().manual_seed(trial)
        w = torch.softmax(torch.randn(v, generator=g0) * 3, -1)
        if trial % 5 == 0:
            w[torch.randint(0, v, (v // 3,), generator=g0)] = 0.0
        ga = torch.Generator().manual_seed(10_000 + trial)
        gb = torch.Generator().manual_seed(10_000 + trial)
        want = int(torch.multinomial(w, 1, generator=ga))
        got = orc.draw(w, orc.exp_noise(v, gb))
        assert got == want, trial
        assert torch.equal(ga.get_state(), gb.get_state()), "generator advanced differently"


def test_verify_draft_matches_reference_outcomes():
    cases = golden_json("verify_cases.json")
    assert len(cases) >= 100
    for c in cases:
        p = torch.tensor(c["p"], dtype=torch.float32)
        q = torch.tensor(c["q"], dtype=torch.float32).reshape(c["k"], c["V"])
        acc, extra = orc.verify_draft(p, q, c["xs"], torch.Generator().manual_seed(c["seed"]))
        assert (acc, extra) == (c["accepted"], c["extra"]), c["seed"]


def test_verify_with_noise_equals_stream_version():
    """The injected-randomness verify (the GPU contract) equals the generator version when u and E are
    drawn in the reference's order; u/E drawn up front (no laziness) must give the same result."""
    for c in golden_json("verify_cases.json"):
        k, v = c["k"], c["V"]
        p = torch.tensor(c["p"], dtype=torch.float32)
        q = torch.tensor(c["q"], dtype=torch.float32).reshape(k, v)
        g = torch.Generator().manual_seed(c["seed"])
        peek = torch.Generator().manual_seed(c["seed"])
        u = [float(torch.rand((), generator=peek)) for _ in range(k)]
        acc, extra = orc.verify_draft(p, q, c["xs"], g)
        # replay: the noise comes after exactly min(len(acc) + 1, k) uniforms
        g2 = torch.Generator().manual_seed(c["seed"])
        for _ in range(min(len(acc) + 1, k)):
            torch.rand((), generator=g2)
        noise = orc.exp_noise(v, g2)
        assert orc.verify_with_noise(p, q, c["xs"], u, noise) == (acc, extra)


def test_greedy_verification_known_answer():
    """tests/test_speculative.py:76-81 of the reference."""
    p = torch.eye(5)[[2, 4, 1, 3]]
    assert orc.verify_draft(p, torch.eye(5)[[2, 4, 0]], [2, 4, 0]) == ([2, 4], 1)
    assert orc.verify_draft(p, torch.eye(5)[[2, 4, 1]], [2, 4, 1]) == ([2, 4, 1], 3)


def test_verification_preserves_the_target_distribution():
    """The first emitted token follows p_1 whatever q is (speculative.py:1-9; the reference's
    statistical test, test_speculative.py:60-73, at a smaller trial count and tolerance ~6 SE)."""
    g = torch.Generator().manual_seed(0)
    v, k, n = 4, 3, 20_000
    p = torch.softmax(torch.randn(k + 1, v, generator=g) * 1.5, -1)
    q = torch.softmax(torch.randn(k, v, generator=g) * 1.5, -1)
    first = []
    for _ in range(n):
        xs = [int(torch.multinomial(q[i], 1, generator=g)) for i in range(k)]
        acc, extra = orc.verify_draft(p, q, xs, g)
        first.append((acc + [extra])[0])
    freq = torch.bincount(torch.tensor(first), minlength=v).float() / n
    assert (freq - p[0]).abs().max() < 0.021, (freq, p[0])


def test_probs_from_logits_closed_form():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(6, 300, generator=g) * 4
    for t in (0.3, 1.0, 2.5):
        want = torch.softmax(x.double() / t, -1)
        torch.testing.assert_close(orc.probs_from_logits(x, t).double(), want, atol=1e-6, rtol=1e-5)
    hot = orc.probs_from_logits(x.to(torch.bfloat16), 0)
    assert hot.dtype == torch.bfloat16 and torch.equal(hot.float().argmax(-1), x.to(torch.bfloat16).float().argmax(-1))
    assert torch.equal(hot.float().sum(-1), torch.ones(6))


# ---- model math ------------------------------------------------------------------------------------
def test_rotate_is_a_half_split_complex_rotation():
    """model.py:40-45: pairs (x_i, x_{i+D/2}) rotate by angle pos * theta^(-2i/D)."""
    s = orc.Shape(16, 32, 1, 2, 1, 64, 40)
    cos, sin = orc.rope_tables(s)
    x = torch.randn(1, 2, 3, 16, dtype=torch.float64)
    pos = torch.tensor([[0, 7, 39]])
    got = orc.rotate(x, cos.double(), sin.double(), pos)
    for t in range(3):
        for i in range(8):
            ang = pos[0, t].item() * (10000.0 ** (-2 * i / 16))
            z = complex(x[0, 0, t, i].item(), x[0, 0, t, i + 8].item()) * complex(math.cos(ang), math.sin(ang))
            assert abs(got[0, 0, t, i].item() - z.real) < 1e-5 and abs(got[0, 0, t, i + 8].item() - z.imag) < 1e-5


def test_attention_math_against_brute_force():
    """GQA head h reads KV head h // rep, key index <= query position, softmax scaled by 1/sqrt(D)."""
    g = torch.Generator().manual_seed(5)
    b, h, hkv, t, s_, d = 2, 4, 2, 3, 7, 8
    q = torch.randn(b, h, t, d, generator=g, dtype=torch.float64)
    k = torch.randn(b, hkv, s_, d, generator=g, dtype=torch.float64)
    v = torch.randn(b, hkv, s_, d, generator=g, dtype=torch.float64)
    pos = torch.tensor([[2, 4, 6], [0, 3, 5]])
    got = orc.attention_math(q, k, v, pos, h // hkv)
    for bi in range(b):
        for hi in range(h):
            for ti in range(t):
                p = pos[bi, ti].item()
                sc = [sum(q[bi, hi, ti, e] * k[bi, hi // 2, j, e] for e in range(d)).item() / math.sqrt(d)
                      for j in range(p + 1)]
                m = max(sc)
                w = [math.exp(x - m) for x in sc]
                z = sum(w)
                for e in range(d):
                    ref = sum(w[j] * v[bi, hi // 2, j, e].item() for j in range(p + 1)) / z
                    assert abs(got[bi, hi, ti, e].item() - ref) < 1e-6   # the oracle computes in f32


def test_paged_write_then_read_known_answer():
    """tests/test_paged.py:20-32: table [7, 2, 9], block size 4, position 5 -> pool block 2, slot 1."""
    s = orc.Shape(64, 64, 3, 8, 4, 192, 64)
    pool = orc.PagedPool(s, 10, 4)
    table = torch.tensor([[7, 2, 9]])
    k = torch.randn(1, 4, 10, 8)
    v = torch.randn_like(k)
    k_all, v_all = pool.views(table, torch.arange(10)[None])[0].update(k, v)
    assert k_all.shape == (1, 4, 12, 8)
    assert torch.equal(k_all[:, :, :10], k) and torch.equal(v_all[:, :, :10], v)
    assert torch.equal(pool.k[0][2, :, 1], k[0, :, 5])


def test_allocator_order():
    a = orc.Allocator(4)
    assert a.allocate(3) == [0, 1, 2] and a.num_free == 1
    with pytest.raises(RuntimeError):
        a.allocate(2)


def test_forward_matches_reference_logits():
    w, s = oracle_model(SMALL, 1, 0.25)
    gold = golden_npz("model_small.npz")
    idx = torch.from_numpy(gold["idx"])
    np.testing.assert_allclose(orc.forward(w, s, idx).numpy(), gold["logits"], atol=2e-5, rtol=1e-5)
    shifted = orc.forward(w, s, idx[:1, :5], positions=torch.arange(5)[None] + 11)
    np.testing.assert_allclose(shifted.numpy(), gold["logits_shifted"], atol=2e-5, rtol=1e-5)


def test_forward_c1_matches_reference_logits():
    w, s = oracle_model(C1, 0, 0.02)
    gold = golden_npz("model_c1.npz")
    prompt = golden_json("model_c1.json")["prompt"]
    np.testing.assert_allclose(orc.forward(w, s, torch.tensor([prompt]))[0].numpy(), gold["logits"], atol=1e-5,
                               rtol=1e-5)


def test_streamed_forward_matches_reference_logits():
    """The layer-at-a-time forward (the full-depth GPU checks feed it one block's weights at a time)
    gives the reference's logits, and the whole-dict forward's bit for bit, in float32 and in bf16."""
    for cfg, seed, std, name in ((SMALL, 1, 0.25, "model_small.npz"), (C1, 0, 0.02, "model_c1.npz")):
        w, s = oracle_model(cfg, seed, std)
        gold = golden_npz(name)
        idx = torch.from_numpy(gold["idx"]) if "idx" in gold else torch.tensor([golden_json("model_c1.json")["prompt"]])

        def layer(i, w=w):
            p = f"layers.{i}."
            return {n[len(p):]: t for n, t in w.items() if n.startswith(p)}

        hidden = []
        got = orc.forward_streamed(layer, w["tok_emb.weight"], w["norm.weight"], s, idx, hidden=hidden)
        assert len(hidden) == s.n_layers and hidden[-1].shape == (*idx.shape, s.d_model)
        assert torch.equal(got, orc.forward(w, s, idx))
        want = gold["logits"] if got.shape[0] > 1 or "idx" in gold else gold["logits"][None]
        np.testing.assert_allclose(got.numpy(), want, atol=2e-5, rtol=1e-5)
        wb = {n: t.bfloat16() for n, t in w.items()}
        got_b = orc.forward_streamed(lambda i: {n: t.bfloat16() for n, t in layer(i).items()}, wb["tok_emb.weight"],
                                     wb["norm.weight"], s, idx)
        assert got_b.dtype == torch.bfloat16 and torch.equal(got_b, orc.forward(wb, s, idx))


def test_paged_forward_matches_reference():
    w, s = oracle_model(SMALL, 1, 0.25)
    gold = golden_npz("model_small.npz")
    seq = torch.from_numpy(gold["paged_seq"])
    table = torch.from_numpy(gold["paged_table"])
    pool = orc.PagedPool(s, 16, 4)
    rope = orc.rope_tables(s)
    got = [orc.forward(w, s, seq[:, :12], torch.arange(12)[None], pool.views(table, torch.arange(12)[None]), rope)]
    for i in range(12, 30):
        pos = torch.tensor([[i]])
        got.append(orc.forward(w, s, seq[:, i: i + 1], pos, pool.views(table, pos), rope))
    np.testing.assert_allclose(torch.cat(got, 1).numpy(), gold["paged_logits"], atol=2e-5, rtol=1e-5)


def test_generate_matches_reference_tokens():
    w, s = oracle_model(SMALL, 1, 0.25)
    gold = golden_json("model_small.json")
    for i, p in enumerate(gold["prompts"]):
        assert orc.generate(w, s, p, 20) == gold["generate_greedy"][i]
        assert orc.generate(w, s, p, 20, 1.0, torch.Generator().manual_seed(21 + i)) == gold["generate_t1"][i]


def test_speculative_generate_matches_reference_streams():
    wt, st = oracle_model(SMALL, 1, 0.25)
    wd, sd = oracle_model(SMALL, 7, 0.25)
    gold = golden_json("model_small.json")
    for kk in (1, 3, 6):
        for p, (toks, stats) in zip(gold["prompts"], gold["spec"][f"greedy_k{kk}"]):
            assert list(orc.speculative_generate(wt, st, wd, sd, p, 20, k=kk)) == [toks, stats]
    for i, (p, (toks, stats)) in enumerate(zip(gold["prompts"], gold["spec"]["t1_k3"])):
        got = orc.speculative_generate(wt, st, wd, sd, p, 20, k=3, temperature=1.0,
                                       gen=torch.Generator().manual_seed(31 + i))
        assert list(got) == [toks, stats]
    for i, (p, (toks, stats)) in enumerate(zip(gold["prompts"], gold["spec"]["t07_k4_self"])):
        got = orc.speculative_generate(wt, st, wt, st, p, 25, k=4, temperature=0.7,
                                       gen=torch.Generator().manual_seed(41 + i))
        assert list(got) == [toks, stats]


def test_speculative_c1_matches_reference():
    wt, st = oracle_model(C1, 0, 0.02)
    wd, sd = oracle_model(C1, 0, 0.02, n_layers=1)
    gold = golden_json("model_c1.json")
    prompt = gold["prompt"]
    assert orc.generate(wt, st, prompt, 64)[16:] == gold["greedy"]
    assert list(orc.speculative_generate(wt, st, wd, sd, prompt, 64, k=4)) == gold["spec_greedy"]
    got = orc.speculative_generate(wt, st, wd, sd, prompt, 64, k=4, temperature=0.8,
                                   gen=torch.Generator().manual_seed(2))
    assert list(got) == gold["spec_t08"]


def test_engine_matches_reference_runs():
    w, s = oracle_model(SMALL, 1, 0.25)
    gold = golden_json("engine_runs.json")
    for name, run in gold["runs"].items():
        e = orc.Engine(w, s, run["num_blocks"], block_size=4, max_batch=5, seed=run["seed"])
        ids = [e.add(p, n, temperature=run["temperature"]) for p, n in gold["requests"]]
        out = e.run()
        assert [out[i] for i in ids] == run["outputs"], name
        assert e.preemptions == run["preemptions"], name


def test_a_planted_mistake_is_caught():
    """Flip the sign of the rotary's second half in a copy of the oracle: the golden logits must reject it."""
    w, s = oracle_model(SMALL, 1, 0.25)
    gold = golden_npz("model_small.npz")
    idx = torch.from_numpy(gold["idx"])
    original = orc.rotate

    def wrong(x, cos, sin, positions):
        half = x.shape[-1] // 2
        c = cos[positions].unsqueeze(1).to(x.dtype)
        s_ = sin[positions].unsqueeze(1).to(x.dtype)
        a, b = x[..., :half], x[..., half:]
        return torch.cat((a * c + b * s_, b * c - a * s_), -1)

    orc.rotate = wrong
    try:
        bad = orc.forward(w, s, idx).numpy()
    finally:
        orc.rotate = original
    assert not np.allclose(bad, gold["logits"], atol=1e-3)


def test_philox_known_answers():
    """The Philox4x32-10 restatement against the known-answer vectors published with Random123
    (counter and key all zeros, all ones, and the digits of pi)."""
    from oracle.keyed_noise import philox4x32_10
    kat = [((0, 0, 0, 0, 0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
           ((0xFFFFFFFF,) * 6, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
           ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344, 0xA4093822, 0x299F31D0),
            (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1))]
    for args, want in kat:
        assert tuple(int(w) for w in philox4x32_10(*args)) == want


def test_keyed_noise_distributions():
    """Uniforms on [0, 1) and Exp(1) variates of the keyed stream: Kolmogorov-Smirnov distances small,
    the Exp(1) values never 0 and finite, different slots and keys independent-looking."""
    import numpy as np
    from scipy import stats
    from oracle import keyed_noise as kn
    u = kn.uniform(12345, 7, 200_000)
    e = kn.exponential(12345, 8, 200_000)
    assert u.min() >= 0 and u.max() < 1
    assert (e > 0).all() and np.isfinite(e).all()
    assert stats.kstest(u, "uniform").statistic < 0.005
    assert stats.kstest(e, "expon").statistic < 0.005
    # small values keep their resolution: the exponential's lower tail follows 1 - exp(-x)
    assert abs((e < 1e-3).mean() - (1 - np.exp(-1e-3))) < 3e-4
    other = kn.uniform(12346, 7, 200_000)
    assert abs(np.corrcoef(u, other)[0, 1]) < 0.01
    assert abs(np.corrcoef(u, kn.uniform(12345, 9, 200_000))[0, 1]) < 0.01
