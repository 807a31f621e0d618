"""Write golden vectors by running the reference (forgeserve, pure PyTorch CPU) in this container.

    PYTHONPATH=/root/reference python tests/golden/make_golden.py

Only outputs are committed (JSON / .npz next to this script); weights are regenerated from seeds with
oracle.reference_cpu.synthetic_weights, so fixtures stay small. The reference never runs on the GPU
box: there, tests compare against these files and the CPU oracle.

What only the reference can pin (the oracle restates everything else from the math):
  * its logits at float32 rounding level (SDPA / matmul order),
  * the tokens of its seeded generator streams (verify_draft, speculative_generate, Engine at T > 0).
"""

import json
import os
import sys

import numpy as np
import torch

REF = "/root/reference"
HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REF)
sys.path.insert(0, ROOT)

import forgeserve as ref  # noqa: E402  (the reference)
from forgeserve.model import ForgeModel  # noqa: E402

from oracle.reference_cpu import Shape, synthetic_weights  # noqa: E402

SMALL = dict(vocab_size=64, d_model=64, n_layers=3, n_heads=8, n_kv_heads=4, max_seq_len=64)
C1 = dict(vocab_size=512, d_model=256, n_layers=4, n_heads=8, n_kv_heads=4, ffn_dim=688, max_seq_len=256)


def ref_model(cfg_kw, seed, std, n_layers=None):
    cfg = ref.ModelConfig(**cfg_kw)
    w = synthetic_weights(Shape.of(cfg), seed, std)
    if n_layers is not None:
        cfg = ref.ModelConfig(**{**cfg_kw, "n_layers": n_layers})
        w = {k: v for k, v in w.items() if not k.startswith("layers.") or int(k.split(".")[1]) < n_layers}
    m = ForgeModel(cfg).eval()
    sd = dict(w)
    sd["lm_head.weight"] = w["tok_emb.weight"]
    m.load_state_dict(sd)
    return m


def verify_cases():
    g = torch.Generator().manual_seed(123)
    cases = []
    for c in range(120):
        v = [4, 7, 16, 24][c % 4]
        k = c % 6
        sharp = [0.5, 1.5, 4.0][c % 3]
        p = torch.softmax(torch.randn(k + 1, v, generator=g) * sharp, -1)
        q = torch.softmax(torch.randn(k, v, generator=g) * sharp, -1) if k else p[:0]
        if c % 5 == 0 and k:
            q = q.clone()
            q[0] = p[0]                     # ratio exactly 1 for the first proposal
        xs = [int(torch.multinomial(q[i], 1, generator=g)) for i in range(k)]
        if c % 7 == 3 and k:
            q = q.clone()
            q[0, xs[0]] = 0.0               # q(x) == 0 -> ratio 1.0 (speculative.py:26)
        seed = 1000 + c
        acc, extra = ref.verify_draft(p, q, xs, torch.Generator().manual_seed(seed))
        cases.append({"V": v, "k": k, "p": p.tolist(), "q": q.tolist(), "xs": xs, "seed": seed,
                      "accepted": acc, "extra": extra})
    # greedy KAT of tests/test_speculative.py:76-81 through the reference itself
    p = torch.eye(5)[[2, 4, 1, 3]]
    for q_rows, xs in (([2, 4, 0], [2, 4, 0]), ([2, 4, 1], [2, 4, 1])):
        q = torch.eye(5)[q_rows]
        acc, extra = ref.verify_draft(p, q, xs, torch.Generator().manual_seed(0))
        cases.append({"V": 5, "k": 3, "p": p.tolist(), "q": q.tolist(), "xs": xs, "seed": 0, "accepted": acc,
                      "extra": extra})
    with open(os.path.join(HERE, "verify_cases.json"), "w") as f:
        json.dump(cases, f)


def model_small():
    target = ref_model(SMALL, 1, 0.25)
    draft = ref_model(SMALL, 7, 0.25)
    g = torch.Generator().manual_seed(11)
    idx = torch.randint(0, 64, (2, 12), generator=g)
    out = {"idx": idx.numpy(), "logits": target(idx).detach().numpy()}
    # explicit positions shifted past the cache (model.py:151-155 + mask semantics)
    out["logits_shifted"] = target(idx[:1, :5], positions=torch.arange(5)[None] + 11).detach().numpy()
    # paged forward: prefill 12, then 18 single-token steps over fragmented blocks (test_paged.py:44-61)
    seq = torch.randint(0, 64, (1, 30), generator=g)
    pool = ref.PagedKVPool(target.cfg, num_blocks=16, block_size=4)
    blocks = pool.allocator.allocate(8)
    perm = torch.randperm(8, generator=g).tolist()
    blocks = [blocks[i] for i in perm]
    table = torch.tensor([blocks])
    got = [target(seq[:, :12], torch.arange(12)[None], pool.views(table, torch.arange(12)[None]))]
    for i in range(12, 30):
        pos = torch.tensor([[i]])
        got.append(target(seq[:, i: i + 1], pos, pool.views(table, pos)))
    out["paged_seq"] = seq.numpy()
    out["paged_table"] = table.numpy()
    out["paged_logits"] = torch.cat(got, 1).detach().numpy()
    prompts = [[1, 2, 3], [5], [9, 8, 7, 6, 5, 4], [0, 0, 1]]
    gen_greedy = [ref.generate(target, torch.tensor([p]), 20)[0].tolist() for p in prompts]
    gen_t1 = [ref.generate(target, torch.tensor([p]), 20, temperature=1.0,
                           generator=torch.Generator().manual_seed(21 + i))[0].tolist() for i, p in enumerate(prompts)]
    spec = {}
    for kk in (1, 3, 6):
        spec[f"greedy_k{kk}"] = [list(ref.speculative_generate(target, draft, p, 20, k=kk)) for p in prompts]
    spec["t1_k3"] = [list(ref.speculative_generate(target, draft, p, 20, k=3, temperature=1.0,
                                                   generator=torch.Generator().manual_seed(31 + i)))
                     for i, p in enumerate(prompts)]
    spec["t07_k4_self"] = [list(ref.speculative_generate(target, target, p, 25, k=4, temperature=0.7,
                                                         generator=torch.Generator().manual_seed(41 + i)))
                           for i, p in enumerate(prompts)]
    np.savez(os.path.join(HERE, "model_small.npz"), **out)
    with open(os.path.join(HERE, "model_small.json"), "w") as f:
        json.dump({"prompts": prompts, "generate_greedy": gen_greedy, "generate_t1": gen_t1, "spec": spec}, f)


def model_c1():
    target = ref_model(C1, 0, 0.02)
    draft = ref_model(C1, 0, 0.02, n_layers=1)
    prompt = torch.randint(0, 512, (16,), generator=torch.Generator().manual_seed(1)).tolist()
    logits = target(torch.tensor([prompt]))[0].detach().numpy()
    greedy = ref.generate(target, torch.tensor([prompt]), 64)[0].tolist()[16:]
    s0, st0 = ref.speculative_generate(target, draft, prompt, 64, k=4)
    s1, st1 = ref.speculative_generate(target, draft, prompt, 64, k=4, temperature=0.8,
                                       generator=torch.Generator().manual_seed(2))
    np.savez(os.path.join(HERE, "model_c1.npz"), logits=logits)
    with open(os.path.join(HERE, "model_c1.json"), "w") as f:
        json.dump({"prompt": prompt, "greedy": greedy, "spec_greedy": [s0, st0], "spec_t08": [s1, st1]}, f)


def engine_runs():
    model = ref_model(SMALL, 1, 0.25)
    g = torch.Generator().manual_seed(1)
    reqs = []
    for _ in range(5):
        plen = int(torch.randint(2, 20, (1,), generator=g))
        reqs.append((torch.randint(0, 64, (plen,), generator=g).tolist(), int(torch.randint(3, 15, (1,), generator=g))))
    runs = {}
    for name, temp, nb, seed in (("greedy_tight", 0.0, 12, 0), ("t1_tight", 1.0, 12, 3), ("t1_roomy", 1.0, 64, 4)):
        e = ref.Engine(model, num_blocks=nb, block_size=4, max_batch=5, seed=seed)
        ids = [e.add_request(p, n, temperature=temp) for p, n in reqs]
        out = e.run()
        runs[name] = {"num_blocks": nb, "seed": seed, "temperature": temp, "outputs": [out[i] for i in ids],
                      "preemptions": e.preemptions, "steps": e.steps}
    with open(os.path.join(HERE, "engine_runs.json"), "w") as f:
        json.dump({"requests": reqs, "runs": runs}, f)


if __name__ == "__main__":
    torch.manual_seed(0)
    verify_cases()
    model_small()
    model_c1()
    engine_runs()
    print("golden vectors written to", HERE)
