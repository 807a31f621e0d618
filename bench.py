"""Benchmark: batched speculative decoding at the 8B shape on one MI355X.

Workload (the reference's largest single-GPU configuration): target = LLaMA-style decoder with 32 layers,
d_model 4096, 32 query / 8 KV heads, head_dim 128, SwiGLU ffn 14336, vocab 128256, bf16, weights
N(0, 0.02) from a seed; draft = the target's embedding, head and first 4 layers. 64 running sequences,
k = 6, contexts uniform in [2048, 8192] held in a paged pool with block_size 16. The
contexts come from a packed prefill of uniform random prompt ids through both models (`--synthetic-kv`:
N(0, 1) bf16 keys/values written straight into the pools instead), then `--steps` decode rounds are
timed: k draft decode steps, one target verify pass over k+1 tokens, one fused acceptance.

One "step" = one speculative round for the whole batch, replayed from the HIP graphs captured for its
shape (the first round of a shape runs eagerly, the second captures). The timed rounds are queued back
to back (`SpeculativeBatch.run_rounds`: each round's inputs are computed on the GPU from the previous
round's acceptance, and the host reads a round's tokens while the next one runs). `value` = committed tokens per
second (accepted proposals + one target token per sequence per round), inputs resident in HBM.
`roofline` = the paged verify attention (the unit kernel per layer, + combine when a query spans chunks,
and one work plan per pass): the last timed round's 32 verify-attention launches (each layer's pool,
that round's tables and query positions) replayed from one HIP graph between HIP events on the
launching stream, against 8 TB/s.
`cpu_baseline` = the CPU oracle (oracle/reference_cpu.py) timed on this host on one target layer's
verify pass, one draft layer's decode step, the LM head and the acceptance at the same shapes (one
warm-up, then the median of three runs of each), scaled to a round.
`t1_variant` = the same workload at temperature 1.0 (fresh prefill, same timing), whose acceptance
exercises the residual draws; `verify_pass` = the target's verify pass alone (its k+1-token forward,
head, statistics merge and fused acceptance) and one draft step, replayed from the round's graphs.
`accept_kernel` = the fused acceptance alone at the 8B shape, standalone (every logit row read) and
with the rows' statistics given as the round's LM heads emit them (achieved GB/s on the bytes that
call reads, and the epilogue's marginal cost per head call).
`c3_attention` / `c2_accept` = the paged verify attention (B=32, k+1=5, contexts U[512,4096], a random
12,288-block pool) and the fused acceptance (B=64, k=5, V=32000, f32) alone, each with the CPU oracle
timed at the same shape; `engine_1b` = the 1B-shape continuous-batching Engine over 48 requests.

    python bench.py [--gpus 1] [--steps 128] [--warmup 4] [--temperature 0.0] [--no-t1-variant]

Kernel-only modes (one JSON line each, used for the rocprofv3 counter runs):
    python bench.py --kernel attention   the verify attention alone: B=64, T=7, 32/8 heads, head_dim 128,
                                         bf16, contexts U[2048,8192], block 16, tables a random permutation;
                                         the calls share one work plan (built by the first warm-up call)
    python bench.py --kernel accept      the fused acceptance alone: B=64, k=6, V=128256, bf16 logits
    python bench.py --kernel copy        1 GiB device-to-device copies, f32 and bf16 (counter calibration)
    python bench.py --kernel gemm        the 8B model's four layer GEMMs and the LM head at M = 448 (a verify
                                         pass) and M = 64 (a draft step), each call on the next layer's weights
    python bench.py --kernel prefill_attention
                                         packed causal prefill attention: 8 prompts of 4096 tokens back to
                                         back, 32/8 heads, head_dim 128, bf16, block 16, TFLOP/s vs 2.5 PFLOP/s
    python bench.py --kernel c3          the attention configuration (see c3_attention), both key layouts
    python bench.py --kernel c2          the acceptance configuration (see c2_accept)
    python bench.py --kernel engine_1b   the 1B-shape Engine workload (see engine_1b)
    python bench.py --kernel gemm_prefill
                                         the 8B model's four layer GEMMs at M = 32768 (one packed prefill
                                         forward), each call on the next layer's weights
"""

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0   # dense bf16
CFG = dict(vocab_size=128256, d_model=4096, n_layers=32, n_heads=32, n_kv_heads=8, ffn_dim=14336,
           max_seq_len=10240)
DRAFT_LAYERS = 4
BATCH, K, BLOCK = 64, 6, 16
CTX_LO, CTX_HI = 2048, 8192
PREFILL_TOKENS = 32768   # tokens per packed prefill forward (SpeculativeBatch.add_many's default)
ACCEPT_CALLS_PER_GRAPH = 10


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def build_models(torch, fa):
    cfg = fa.ModelConfig(**CFG)
    torch.manual_seed(0)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device("cuda"):
            target = fa.ForgeModel(cfg).eval()
    finally:
        torch.set_default_dtype(prev)
    draft = fa.early_exit_draft(target, DRAFT_LAYERS)
    return target, draft


CFG_1B = dict(vocab_size=32000, d_model=2048, n_layers=16, n_heads=32, n_kv_heads=8, ffn_dim=8192,
              max_seq_len=2048)


def engine_1b(args):
    """The 1B-shape continuous-batching workload: Engine(max_batch 16, k = 4, T = 0.7) with a 2-layer
    early-exit draft over 48 requests (prompts U[128, 1024], max_new_tokens U[64, 256]), the pool sized
    below the peak demand so that recompute preemptions happen, timed after a short warm-up run on
    another Engine. Returns the figures as a dict."""
    import torch

    import forgeserve_amd as fa

    cfg = fa.ModelConfig(**CFG_1B)
    torch.manual_seed(args.seed)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device("cuda"):
            target = fa.ForgeModel(cfg).eval()
    finally:
        torch.set_default_dtype(prev)
    draft = fa.early_exit_draft(target, 2)
    g = torch.Generator().manual_seed(args.seed + 1)
    reqs = [(torch.randint(0, cfg.vocab_size, (int(torch.randint(128, 1025, (1,), generator=g)),), generator=g).tolist(),
             int(torch.randint(64, 257, (1,), generator=g))) for _ in range(48)]
    # warm-up: a short run of the same engine settings loads every kernel the run uses (the first launch
    # of a kernel loads its code object); the timed engine then captures its own round graphs
    warm = fa.Engine(target, num_blocks=600, block_size=16, max_batch=16, seed=args.seed + 7, draft=draft, k=4,
                     key_layout="groups")
    for p, _ in reqs[:20]:
        warm.add_request(p, 12, temperature=0.7)
    warm.run()
    del warm
    torch.cuda.synchronize()
    time.sleep(0.25)   # an idle gap that marks where the timed run starts in a kernel trace
    eng = fa.Engine(target, num_blocks=600, block_size=16, max_batch=16, seed=args.seed, draft=draft, k=4,
                    key_layout="groups")
    for p, n in reqs:
        eng.add_request(p, n, temperature=0.7)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    out = eng.run()
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    toks = sum(len(v) for v in out.values())
    assert all(len(out[i]) == n for i, (_, n) in enumerate(reqs))
    res = {"workload": "1B-shape continuous batching: 16L d2048 32/8 heads hd64 ffn8192 V32000 bf16, "
                       "2-layer early-exit draft, Engine max_batch 16, k=4, T=0.7, 48 requests, "
                       "prompts U[128,1024], max_new U[64,256], 600 blocks of 16 (keys in 8-dim groups)",
           "generated_tokens": toks, "seconds": round(el, 3), "tok_per_s": round(toks / el, 1),
           "engine_steps": eng.steps, "rounds": eng.stats["rounds"], "preemptions": eng.preemptions,
           "peak_running": eng.peak_running, "peak_blocks": eng.peak_blocks,
           "acceptance": round(eng.stats["accepted"] / max(eng.stats["proposed"], 1), 4),
           "gpu_busy_fraction": profiled_figure("engine_1b_kernel_stats.md", "gpu_busy_fraction", float),
           "gpu_busy_fraction_unprofiled_wall": profiled_figure("engine_1b_kernel_stats.md",
                                                                "gpu_busy_fraction_unprofiled_wall", float),
           "gpu_busy_note": "kernel time / wall time of the same command under rocprofv3 --kernel-trace "
                            "(and kernel time / the wall time without the profiler), "
                            "from profiles/engine_1b_kernel_stats.md"}
    del eng, target, draft
    torch.cuda.empty_cache()
    return res


def attn_bytes(ctxs, t, h, hkv, d, bs):
    kv = sum(ctxs) * hkv * d * 2 * 2
    qo = len(ctxs) * t * h * d * 2 * 2
    tables = 4 * sum(-(-c // bs) for c in ctxs)
    return kv + qo + tables + 4 * len(ctxs) * t


def accept_bytes(b, k, v, s_logit=2):
    return s_logit * b * v * (2 * k + 1) + 4 * b * v + 4 * b * k * 2 + 4 * b * (k + 2)


def time_verify_attention(torch, fa, ops, sb, lens, reps=4):
    """Per-launch duration of the verify attention as the timed rounds ran it: the last timed round's
    32 verify-attention launches (every layer's pool, that round's block tables, and its k+1 query
    positions per sequence, lens = the sequences' lengths before it; one work plan for the 32, as a
    verify pass builds it) captured in one HIP graph, whose replays are bracketed by events on the
    launching stream. Returns (seconds per launch, algorithmic bytes per launch)."""
    dev = sb.dev
    seqs = sb.active()
    tables = fa.paged.block_table([s.blocks_t for s in seqs], dev)
    pos = torch.tensor([[n - 1 + t for t in range(K + 1)] for n in lens], dtype=torch.int32, device=dev)
    h, d = CFG["n_heads"], CFG["d_model"] // CFG["n_heads"]
    q = torch.randn(len(seqs), K + 1, h, d, device=dev).to(torch.bfloat16)
    out = torch.empty_like(q)
    layers = range(CFG["n_layers"])

    def launches():
        step = object()   # the layers of one verify pass share its positions
        for layer in layers:
            ops.paged_attention(q, sb.pool_t.layout(layer), tables, pos, d ** -0.5, out=out, plan_key=step)

    launches()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        launches()
    g.replay()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    for a, b in ev:
        a.record()
        g.replay()
        b.record()
    torch.cuda.synchronize()
    sec = sum(a.elapsed_time(b) for a, b in ev) * 1e-3 / (reps * len(layers))
    return sec, attn_bytes([n + K for n in lens], K + 1, h, CFG["n_kv_heads"], d, BLOCK)


def cpu_baseline(torch, committed_per_round):
    """Time the CPU oracle on one layer of each kind at the benchmark shapes; scale to one round."""
    from oracle import reference_cpu as orc

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(0)
    s = orc.Shape(CFG["vocab_size"], CFG["d_model"], 1, CFG["n_heads"], CFG["n_kv_heads"], CFG["ffn_dim"],
                  CFG["max_seq_len"])
    w = {}
    for name, shape in orc.param_names(s):
        if name == "tok_emb.weight":
            continue
        w[name] = torch.randn(shape, generator=g) * 0.02 if len(shape) > 1 else torch.ones(shape)
    rope = orc.rope_tables(s)
    ctxs = torch.randint(CTX_LO, CTX_HI + 1, (BATCH,), generator=torch.Generator().manual_seed(1)).tolist()
    hd, hkv = s.head_dim, s.n_kv_heads
    # per-row cached keys/values of one layer, generated before any timing
    kcache = [torch.randn(1, hkv, c, hd, generator=g) for c in ctxs]
    vcache = [torch.randn(1, hkv, c, hd, generator=g) for c in ctxs]

    def layer(t):
        """One decoder layer (model.py:104-106) for BATCH rows of t new tokens over their contexts."""
        x = torch.randn(BATCH, t, s.d_model, generator=g) * 0.5
        p = "layers.0."
        h = orc.rms_norm(x, w[p + "attn_norm.weight"], s.norm_eps)
        q = (h @ w[p + "attn.wq.weight"].T).view(BATCH, t, s.n_heads, hd).transpose(1, 2)
        k = (h @ w[p + "attn.wk.weight"].T).view(BATCH, t, hkv, hd).transpose(1, 2)
        v = (h @ w[p + "attn.wv.weight"].T).view(BATCH, t, hkv, hd).transpose(1, 2)
        outs = []
        for b in range(BATCH):          # one row at a time keeps the gathered context in memory
            pos = torch.arange(ctxs[b] - t, ctxs[b])[None]
            qb, kb = orc.rotate(q[b:b + 1], *rope, pos), orc.rotate(k[b:b + 1], *rope, pos)
            kc, vc = kcache[b][:, :, : ctxs[b] - t], vcache[b][:, :, : ctxs[b] - t]
            outs.append(orc.attention_math(qb, torch.cat([kc, kb], 2), torch.cat([vc, v[b:b + 1]], 2), pos,
                                           s.n_heads // hkv))
        o = torch.cat(outs, 0)
        x = x + o.transpose(1, 2).reshape(BATCH, t, -1) @ w[p + "attn.wo.weight"].T
        h = orc.rms_norm(x, w[p + "mlp_norm.weight"], s.norm_eps)
        return x + (torch.nn.functional.silu(h @ w[p + "mlp.w_gate.weight"].T) * (h @ w[p + "mlp.w_up.weight"].T)) \
            @ w[p + "mlp.w_down.weight"].T

    def timed(fn, runs=3):
        """One warm-up, then the median of `runs` timed calls."""
        fn()
        ts = []
        for _ in range(runs):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return sorted(ts)[len(ts) // 2]

    t_verify = timed(lambda: layer(K + 1))
    t_decode = timed(lambda: layer(1))
    head = torch.randn(CFG["vocab_size"], CFG["d_model"], generator=g) * 0.02
    t_head_v = timed(lambda: torch.randn(BATCH * (K + 1), CFG["d_model"]) @ head.T)
    t_head_d = timed(lambda: torch.randn(BATCH, CFG["d_model"]) @ head.T)
    logits_t = torch.randn(BATCH, K + 1, CFG["vocab_size"], generator=g) * 2
    logits_d = logits_t[:, :K] + torch.randn(BATCH, K, CFG["vocab_size"], generator=g) * 0.5

    def accept():
        for b in range(BATCH):
            p = orc.probs_from_logits(logits_t[b], 1.0)
            q = orc.probs_from_logits(logits_d[b], 1.0)
            xs = [int(q[i].argmax()) for i in range(K)]
            orc.verify_with_noise(p, q, xs, torch.rand(K), torch.empty(CFG["vocab_size"]).exponential_())

    t_acc = timed(accept)
    n_t, n_d = CFG["n_layers"], DRAFT_LAYERS
    round_s = n_t * t_verify + K * n_d * t_decode + t_head_v + K * t_head_d + t_acc
    return {
        "value": committed_per_round / round_s,
        "unit": "tok/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"CPU oracle at the bench shapes, each piece warmed up once then the median of 3 runs: "
                   f"1 target layer verify (B={BATCH}, T={K + 1}, per-row "
                   f"contexts U[{CTX_LO},{CTX_HI}]) {t_verify:.2f}s, 1 draft layer decode {t_decode:.2f}s, "
                   f"LM head {t_head_v:.2f}s/{t_head_d:.2f}s, acceptance {t_acc:.2f}s; scaled to one round "
                   f"({n_t} verify layers + {K}x{n_d} draft layers + heads) = {round_s:.1f}s for "
                   f"{committed_per_round:.1f} committed tokens"),
    }


def profiled_figure(name, key, conv=int):
    """A figure measured under rocprofv3 (counters or a kernel trace), from the summary committed under
    profiles/ (its line `key: value`), or None."""
    import re

    path = os.path.join(ROOT, "profiles", name)
    try:
        m = re.search(re.escape(key) + r":\s*([0-9.]+)", open(path).read())
    except OSError:
        return None
    return conv(m.group(1)) if m else None


def profiled_traffic(name):
    """HBM bytes per call measured with rocprofv3 counters (`traffic_bytes_per_call: N`), or None."""
    return profiled_figure(name, "traffic_bytes_per_call")


def time_accept(torch, ops, reps, warmup, with_stats=False):
    """The acceptance kernel alone at the benchmark shape (bf16 logits, V = 128256): (mean seconds per
    call, bytes the call reads). ACCEPT_CALLS_PER_GRAPH calls back to back are captured into a graph and
    replayed between HIP events, so neither the host's launch overhead nor the events' own cost (about
    10 µs per replay) is timed; the launch gaps between and inside the calls are. with_stats: the rows' softmax statistics are given, as the LM head's
    epilogue emits them in the round (they are computed here once, outside the timed calls); the call
    then reads only the rejected position's two logit rows (the target row alone for a bonus token),
    the Exp(1) row, and per sequence the proposals, uniforms, statistics and 2k+1 proposal logits."""
    v = CFG["vocab_size"]
    g = torch.Generator(device="cuda").manual_seed(3)
    tl = torch.randn(BATCH, K + 1, v, device="cuda", generator=g).mul_(2).bfloat16()
    dl = (tl[:, :K].float() + torch.randn(BATCH, K, v, device="cuda", generator=g) * 0.5).bfloat16()
    xs = dl.float().argmax(-1).int()
    temps = torch.ones(BATCH, device="cuda")
    u = torch.rand(BATCH, K, device="cuda", generator=g)
    e = torch.empty(BATCH, v, device="cuda").exponential_(generator=g)
    st = None
    if with_stats:
        rows = torch.cat([tl, dl], 1).float()
        mx = rows.max(-1).values
        f = torch.stack([mx, torch.exp(rows - mx[..., None]).sum(-1), mx], -1).contiguous().view(torch.int32)
        st = torch.cat([f, rows.argmax(-1).to(torch.int32)[..., None]], -1).contiguous()
        del rows
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(max(warmup, 1)):
            ops.spec_accept(tl, dl, xs, None, temps, u, e, row_stats=st)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(ACCEPT_CALLS_PER_GRAPH):
            ops.spec_accept(tl, dl, xs, None, temps, u, e, row_stats=st)
    graph.replay()
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    for a, b in ev:
        a.record()
        graph.replay()
        b.record()
    torch.cuda.synchronize()
    sec = sum(a.elapsed_time(b) for a, b in ev) / len(ev) * 1e-3 / ACCEPT_CALLS_PER_GRAPH
    if not with_stats:
        return sec, accept_bytes(BATCH, K, v)
    _, n = ops.spec_accept(tl, dl, xs, None, temps, u, e, row_stats=st)
    rows = sum(2 if int(x) < K else 1 for x in n.cpu())   # logit rows of the final draw
    small = BATCH * (4 * K * 2 + 16 * (2 * K + 1) + 2 * (2 * K + 1) + 4 * (K + 2))
    return sec, rows * v * 2 + BATCH * v * 4 + small


def time_gemms(torch, ops, model, m, passes=3, head=True):
    """One layer's four GEMMs and the LM head at M rows (the verify pass: M = B*(k+1); a draft step:
    M = B; a packed prefill forward: M = 32768, no head), each as the model runs it: qkv, wo and
    w_down as split-K partials where their (N, K) splits K (the round adds the partials inside the
    rotary + KV write and the residual-add + RMSNorm that follow, kernels counted apart) unless the
    batch is long enough for the splits to run inside each workgroup (fs_gemm_serial), gate|up with the
    SwiGLU gate in its epilogue, the head with its softmax-statistics epilogue. A shape's calls run back
    to back over successive layers' weights (so that, as in a round, the weights stream from HBM rather
    than the 256 MB last-level cache), `passes` times over the layers, between one pair of events:
    {name: (seconds per call, flops)}."""
    from forgeserve_amd import _lib
    lib = _lib.load()
    layers = model.layers
    d = model.cfg.d_model
    shapes = {"qkv": (d, [b.attn.qkv_weight() for b in layers], "gemm"),
              "o": (d, [b.attn.wo.weight for b in layers], "gemm"),
              "gate_up": (d, [b.mlp.gate_up_weight() for b in layers], "swiglu"),
              "down": (layers[0].mlp.w_down.weight.shape[1], [b.mlp.w_down.weight for b in layers], "gemm")}
    if head:
        shapes["head"] = (d, [model.lm_head.weight], "head")
    out = {}
    for name, (kdim, ws, kind) in shapes.items():
        n = ws[0].shape[0]
        x = torch.randn(m, kdim, device="cuda").to(ws[0].dtype)
        if kind == "swiglu":
            def fn(w):
                ops.gemm_swiglu(x, w)
        elif kind == "head":
            stats = torch.empty((m, ops.row_stats_parts(m, n, kdim), 4), dtype=torch.int32, device="cuda")
            logits = torch.empty((m, n), dtype=x.dtype, device="cuda")

            def fn(w):
                ops.gemm_row_stats(x, w, None, stats, out=logits)
        elif lib.fs_gemm_splits(n, kdim, _lib.BF16) > 1 and not lib.fs_gemm_serial(m, n, kdim, _lib.BF16):
            part = torch.empty(lib.fs_gemm_splits(n, kdim, _lib.BF16) * m * n, dtype=torch.float32, device="cuda")

            def fn(w):
                ops.check(lib.fs_gemm_partials(ops.ptr(x), x.stride(0), ops.ptr(w), w.stride(0), m, n, kdim,
                                               _lib.BF16, ops.ptr(part), part.numel() * 4, ops.stream_ptr()),
                          "gemm_partials")
        else:
            c = torch.empty((m, n), dtype=x.dtype, device="cuda")

            def fn(w):
                ops.gemm(x, w, out=c)
        calls = max(passes * len(ws), 8)
        for i in range(2):
            fn(ws[i % len(ws)])
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for i in range(calls):
            fn(ws[i % len(ws)])
        b.record()
        torch.cuda.synchronize()
        out[name] = (a.elapsed_time(b) * 1e-3 / calls, 2.0 * m * kdim * n)
    return out


def head_epilogue_cost(torch, ops, model):
    """Marginal cost of the LM head's softmax-statistics epilogue: graph-replayed head GEMMs with and
    without it at M = B*(k+1) (a verify pass) and M = B (a draft step), in µs per call."""
    w = model.lm_head.weight
    n, d = w.shape
    out = {}
    for name, m in (("m448", BATCH * (K + 1)), ("m64", BATCH)):
        x = torch.randn(m, d, device="cuda").to(w.dtype)
        logits = torch.empty((m, n), dtype=w.dtype, device="cuda")
        parts = torch.empty((m, ops.row_stats_parts(m, n, d), 4), dtype=torch.int32, device="cuda")
        t_plain = graph_time(torch, lambda: ops.gemm(x, w, out=logits), 8)
        t_stats = graph_time(torch, lambda: ops.gemm_row_stats(x, w, None, parts, out=logits), 8)
        out[name] = round((t_stats - t_plain) * 1e6, 1)
    return out


def gemm_summary(times, layers, peak_tflops):
    """Σ flops / Σ time over a pass's GEMMs (the layer GEMMs `layers` times, the head once; the verify
    pass runs blocks L_d..L-1 at M = B*(k+1), a draft step its L_d blocks at M = B)."""
    hd = times.get("head", (0.0, 0))
    t = sum(v[0] for k, v in times.items() if k != "head") * layers + hd[0]
    f = sum(v[1] for k, v in times.items() if k != "head") * layers + hd[1]
    return {"tflops": round(f / t / 1e12, 1), "frac": round(f / t / 1e12 / peak_tflops, 4),
            "ms_per_pass": round(t * 1e3, 3),
            "per_gemm_us": {k: round(v[0] * 1e6, 1) for k, v in times.items()}}


def attention_inputs(torch, fa, seed=0):
    """Verify-attention inputs at the benchmark shape: contexts U[2048,8192] (the round benchmark's
    seed), the k+1 = 7 query positions at the end of each context, block tables a random permutation
    of the pool, N(0,1) bf16 queries, keys and values; keys in 8-dim groups, as the rounds' pools hold
    them."""
    g = torch.Generator().manual_seed(seed)
    ctxs = torch.randint(CTX_LO, CTX_HI + 1, (BATCH,), generator=g).tolist()
    nb = [-(-c // BLOCK) for c in ctxs]
    n_pool = sum(nb) + 16
    perm = torch.randperm(n_pool, generator=g)
    tables = torch.zeros(BATCH, max(nb), dtype=torch.int32)
    at = 0
    for i, n in enumerate(nb):
        tables[i, :n] = perm[at:at + n].int()
        at += n
    cfg = fa.ModelConfig(vocab_size=8, d_model=CFG["n_heads"] * 128, n_layers=1, n_heads=CFG["n_heads"],
                         n_kv_heads=CFG["n_kv_heads"], max_seq_len=16)
    pool = fa.PagedKVPool(cfg, n_pool, BLOCK, dtype=torch.bfloat16, device="cuda", key_layout="groups")
    pool.k_store.normal_()
    pool.v_store.normal_()
    q = torch.randn(BATCH, K + 1, CFG["n_heads"], 128, device="cuda").bfloat16()
    pos = torch.tensor([[c - (K + 1) + i for i in range(K + 1)] for c in ctxs], dtype=torch.int32).cuda()
    return ctxs, pool, q, pos, tables.cuda()


def cpu_timed(fn, runs=3):
    """One warm-up call, then the median of `runs` timed calls (seconds)."""
    fn()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return sorted(ts)[len(ts) // 2]


def graph_time(torch, fn, calls, reps=5):
    """Mean seconds per fn() call: `calls` calls captured in one HIP graph, replayed `reps` times between
    HIP events on the capturing stream (no host launch overhead in the figure)."""
    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(calls):
            fn()
    g.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        g.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e-3 / (reps * calls)


C3 = dict(batch=32, t=5, h=32, hkv=8, d=128, bs=16, pool=12288, lo=512, hi=4096, seed=6)


def c3_attention(torch, fa, ops, cpu=True):
    """The paged verify-attention kernel alone at the attention configuration: 32 sequences, k+1 = 5 query
    tokens each (causal inside the window: the last 5 positions of each context), 32/8 heads, head_dim
    128, bf16 N(0, 1) queries/keys/values (seed 6), contexts U[512, 4096], block 16, block tables the
    first sum(ceil(ctx/16)) entries of a random permutation of a 12,288-block pool (paged.py:80-81,
    model.py:70-76). Two layers' pools, alternated, so that a call does not find the previous call's
    keys in the last-level cache. Per layout (keys slot-major as the reference's pool, and in 8-dim
    groups as the speculative batches' pools): the attention per call with one work plan shared by 16
    calls (a layer of a verify pass) and per standalone call (plan + attention). cpu: the oracle's
    gather + masked softmax attention in f32 on this host (paged.py:80-81, model.py:70-76)."""
    c = C3
    g = torch.Generator().manual_seed(c["seed"])
    ctxs = torch.randint(c["lo"], c["hi"] + 1, (c["batch"],), generator=g).tolist()
    nb = [-(-x // c["bs"]) for x in ctxs]
    perm = torch.randperm(c["pool"], generator=g)
    tables = torch.zeros(c["batch"], max(nb), dtype=torch.int32)
    at = 0
    for i, n in enumerate(nb):
        tables[i, :n] = perm[at:at + n].int()
        at += n
    cfg = fa.ModelConfig(vocab_size=8, d_model=c["h"] * c["d"], n_layers=2, n_heads=c["h"], n_kv_heads=c["hkv"],
                         max_seq_len=16)
    gd = torch.Generator(device="cuda").manual_seed(c["seed"])
    q = torch.randn(c["batch"], c["t"], c["h"], c["d"], device="cuda", generator=gd).bfloat16()
    pos = torch.tensor([[x - c["t"] + i for i in range(c["t"])] for x in ctxs], dtype=torch.int32).cuda()
    tab = tables.cuda()
    byts = attn_bytes(ctxs, c["t"], c["h"], c["hkv"], c["d"], c["bs"])
    out = {"workload": "paged verify attention alone: B=32, k+1=5, 32/8 heads, hd128, bf16, ctx U[512,4096] "
                       "(seed 6), block 16, tables a random permutation of a 12,288-block pool",
           "algorithmic_bytes": byts}
    o = torch.empty_like(q)
    for layout in ("slots", "groups"):
        pool = fa.PagedKVPool(cfg, c["pool"], c["bs"], dtype=torch.bfloat16, device="cuda", key_layout=layout)
        pool.k_store.normal_(generator=gd)
        pool.v_store.normal_(generator=gd)
        lays = [pool.layout(0), pool.layout(1)]
        state = {"i": 0, "key": object()}

        def shared():
            ops.paged_attention(q, lays[state["i"] % 2], tab, pos, c["d"] ** -0.5, out=o, plan_key=state["key"])
            state["i"] += 1

        def alone():
            ops.paged_attention(q, lays[state["i"] % 2], tab, pos, c["d"] ** -0.5, out=o)
            state["i"] += 1

        t_shared = graph_time(torch, shared, 16)
        t_alone = graph_time(torch, alone, 16)
        out[layout] = {"avg_us": round(t_shared * 1e6, 2), "achieved_GBs": round(byts / t_shared / 1e9, 1),
                       "frac": round(byts / t_shared / 1e9 / HBM_PEAK_GBS, 4),
                       "standalone_us": round(t_alone * 1e6, 2)}
        if layout == "slots" and cpu:
            out["cpu"] = c3_cpu(torch, pool, q, tables, pos, ctxs)
        del pool, lays
        torch.cuda.empty_cache()
    return out


def c3_cpu(torch, pool, q, tables, pos, ctxs):
    """The oracle's attention on the host at the attention configuration: the reference's gather of every
    table block (paged.py:80-81), GQA repeat, key <= position mask and softmax attention in f32
    (model.py:70-76), for the 32 rows at once."""
    from oracle import reference_cpu as orc

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    c = C3
    used = tables.unique().long()
    kp = torch.zeros(c["pool"], c["hkv"], c["bs"], c["d"])
    vp = torch.zeros(c["pool"], c["hkv"], c["bs"], c["d"])
    kp[used] = pool.k[0][used.cuda()].float().cpu()
    vp[used] = pool.v[0][used.cuda()].float().cpu()
    qc = q.float().cpu().transpose(1, 2)
    pc = pos.long().cpu()
    tl = tables.long()
    b = c["batch"]

    def run():
        k_all = kp[tl].permute(0, 2, 1, 3, 4).reshape(b, c["hkv"], -1, c["d"])
        v_all = vp[tl].permute(0, 2, 1, 3, 4).reshape(b, c["hkv"], -1, c["d"])
        return orc.attention_math(qc, k_all, v_all, pc, c["h"] // c["hkv"])

    sec = cpu_timed(run)
    byts = attn_bytes(ctxs, c["t"], c["h"], c["hkv"], c["d"], c["bs"])
    return {"seconds": round(sec, 3), "GBs": round(byts / sec / 1e9, 2), "cores": threads, "kind": "port",
            "sample": "the whole call (32 rows), one warm-up then the median of 3"}


C2 = dict(batch=64, k=5, v=32000)


def c2_inputs(torch):
    """The acceptance configuration: target logits 2.0*N(0,1) (B, k+1, V) (seed 3), draft logits = the
    target's first k positions + 0.5*N(0,1) (seed 4), f32, T = 1; draft tokens argmax(q_j / E_j), the
    uniforms u (B, k) and the final Exp(1) row E (B, V) from seed 5."""
    c = C2
    b, k, v = c["batch"], c["k"], c["v"]
    tl = torch.randn(b, k + 1, v, generator=torch.Generator().manual_seed(3)) * 2.0
    dl = tl[:, :k] + torch.randn(b, k, v, generator=torch.Generator().manual_seed(4)) * 0.5
    g5 = torch.Generator().manual_seed(5)
    e_draft = torch.empty(b, k, v).exponential_(generator=g5)
    xs = (torch.softmax(dl, -1) / e_draft).argmax(-1).int()
    u = torch.rand(b, k, generator=g5)
    e = torch.empty(b, v).exponential_(generator=g5)
    return tl, dl, xs, u, e


def c2_accept(torch, ops, cpu=True):
    """The fused acceptance alone at the acceptance configuration (B = 64, k = 5, V = 32000, f32 logits,
    T = 1): graph-replayed standalone calls, and, with cpu, the oracle's softmaxes and verify_draft on
    the same injected randomness on this host (sampling.py:9-13, speculative.py:20-33)."""
    c = C2
    b, k, v = c["batch"], c["k"], c["v"]
    tl, dl, xs, u, e = c2_inputs(torch)
    args = (tl.cuda(), dl.cuda(), xs.cuda(), None, torch.ones(b, device="cuda"), u.cuda(), e.cuda())
    sec = graph_time(torch, lambda: ops.spec_accept(*args), 16)
    byts = accept_bytes(b, k, v, s_logit=4)
    out = {"workload": "fused acceptance alone: B=64, k=5, V=32000, f32 logits, T=1, seeds 3/4/5",
           "avg_us": round(sec * 1e6, 2), "algorithmic_bytes": byts, "achieved_GBs": round(byts / sec / 1e9, 1),
           "frac": round(byts / sec / 1e9 / HBM_PEAK_GBS, 4)}
    got, n = ops.spec_accept(*args)
    out["mean_accepted"] = round(float(n.float().mean()), 3)
    if cpu:
        from oracle import reference_cpu as orc

        threads = len(os.sched_getaffinity(0))
        torch.set_num_threads(threads)

        def run():
            res = []
            for i in range(b):
                p, q = orc.probs_from_logits(tl[i], 1.0), orc.probs_from_logits(dl[i], 1.0)
                res.append(orc.verify_with_noise(p, q, xs[i].tolist(), u[i], e[i]))
            return res

        t = cpu_timed(run)
        res = run()
        out["cpu"] = {"seconds": round(t, 3), "GBs": round(byts / t / 1e9, 2), "cores": threads, "kind": "port",
                      "sample": "the whole call (64 sequences), one warm-up then the median of 3"}
        got, n = got.cpu(), n.cpu()
        out["tokens_equal_oracle"] = all(got[i, : len(a) + 1].tolist() == a + [x] and int(n[i]) == len(a)
                                         for i, (a, x) in enumerate(res))
    return out


def phase_times(torch, sb, reps=8):
    """The round's phases, each captured in a graph of its own, replayed alone between HIP events on the launching
    stream: the target's verify phase (k+1-token forward through the reused draft residual streams,
    LM head with its statistics epilogue, statistics merges, fused acceptance) and the draft steps. The
    replays rewrite what the last round wrote (same keys, values, logits and outputs)."""
    st = next(reversed(sb.pool_t.__dict__.get("_rounds", {}).values()), None)
    if st is None or st.graph is None:
        return None
    from forgeserve_amd.speculative import capture_phase_graphs
    graphs = capture_phase_graphs(sb.target, sb.draft, sb.pool_t, sb.pool_d, st)
    out = {}
    for name, idx in (("verify_ms", [st.k]), ("draft_step_ms", list(range(st.k)))):
        for i in idx:
            graphs[i].replay()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            for i in idx:
                graphs[i].replay()
        b.record()
        torch.cuda.synchronize()
        out[name] = round(a.elapsed_time(b) / reps / len(idx), 3)
    out["what"] = ("verify_ms: the verify phase (28 blocks over the k+1 window from the draft's residual "
                   "streams, 4 shared blocks for the last proposal, head + statistics, merges, acceptance); "
                   "draft_step_ms: one draft decode step (4 blocks, head + statistics, sample), mean of the k")
    return out


def run_rounds(torch, fa, ops, target, draft, args, temperature, timing):
    """Prefill the benchmark's 64 contexts into a fresh SpeculativeBatch at `temperature`, run the warm-up
    rounds, then time args.steps rounds (queued back to back). With timing: also the verify-attention
    launch time of the last round and the round's phases."""
    g = torch.Generator().manual_seed(args.seed)
    ctxs = torch.randint(CTX_LO, CTX_HI + 1, (BATCH,), generator=g).tolist()
    rounds = args.warmup + args.steps
    per_seq = [-(-(c + 2 + rounds * (K + 1) + K) // BLOCK) for c in ctxs]
    nblocks = sum(per_seq) + 8
    sb = fa.SpeculativeBatch(target, draft, nblocks, BLOCK, K,
                             generator=torch.Generator(device="cuda").manual_seed(args.seed))
    prompts = [torch.randint(0, CFG["vocab_size"], (c + 1,), generator=g).tolist() for c in ctxs]
    prefill = None
    if args.synthetic_kv:   # random keys/values in the pools instead of a prefill
        for store in (sb.pool_t.k_store, sb.pool_t.v_store, sb.pool_d.k_store, sb.pool_d.v_store):
            store.normal_()
        for toks in prompts:
            sb.add(toks, max_new_tokens=10 ** 9, temperature=temperature, prefill=False)
    else:                   # the contexts come from the models: packed prefill of every prompt
        torch.cuda.synchronize()
        tp = time.perf_counter()
        sb.add_many(prompts, 10 ** 9, temperature)
        torch.cuda.synchronize()
        tp = time.perf_counter() - tp
        n_tok = sum(len(p) - 1 for p in prompts)
        prefill = {"tokens": n_tok, "seconds": round(tp, 3), "tok_per_s": round(n_tok / tp, 1),
                   "models": ("target (32 layers; the early-exit draft shares its first 4 layers' cache)"
                              if sb.shared else "target (32 layers) and draft (4 layers)") +
                             ", packed 32K-token forwards"}
        log(f"T={temperature}: prefill {n_tok} tokens in {tp:.1f}s")
    torch.cuda.synchronize()
    for i in range(args.warmup):
        sb.round()
    log(f"T={temperature}: {args.warmup} warm-up rounds done")
    torch.cuda.synchronize()

    # timed rounds: each round's kernels replay from the HIP graph captured for its shape, queued back
    # to back (each one's inputs computed on the GPU from the previous one's acceptance, the host's
    # bookkeeping one round behind), in chunks of 32 for the progress lines; the last round on its own,
    # after noting the lengths it starts from
    acc0 = dict(sb.stats)
    torch.cuda.synchronize()
    t_start = time.perf_counter()
    committed = 0
    done_rounds = 0
    while done_rounds < args.steps - 1:
        n = min(32 - done_rounds % 32, args.steps - 1 - done_rounds)
        committed += sb.run_rounds(n)
        done_rounds += n
        if done_rounds % 32 == 0:
            log(f"T={temperature}: round {done_rounds}/{args.steps}: {committed} tokens committed")
    last_lens = [len(s.tokens) for s in sb.active()]
    committed += sb.round()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t_start
    log(f"T={temperature}: round {args.steps}/{args.steps}: {committed} tokens committed in {elapsed:.2f}s")
    out = {"elapsed": elapsed, "committed": committed, "prefill": prefill,
           "proposed": sb.stats["proposed"] - acc0["proposed"], "accepted": sb.stats["accepted"] - acc0["accepted"]}
    if timing:
        out["attn_avg"], out["attn_bytes"] = time_verify_attention(torch, fa, ops, sb, last_lens)
        from forgeserve_amd import _lib

        split = int(_lib.load().fs_paged_attention_split())
        past = sum(1 for n in last_lens for t in range(K + 1) if n - 1 + t >= split)
        out["combine_note"] = (f"{split}-key chunks; {past} of {len(last_lens) * (K + 1)} query positions of the "
                               f"measured round reach past key {split - 1}, so attn_combine_kernel also runs"
                               if past else f"{split}-key chunks; every query of the measured round sees one "
                               "chunk, so no combine launch")
        out["phases"] = phase_times(torch, sb)
    del sb
    torch.cuda.empty_cache()
    return out


def kernel_mode(args):
    import torch

    import forgeserve_amd as fa
    from forgeserve_amd import ops

    assert torch.cuda.is_available(), "bench.py needs a ROCm GPU"
    steps, warmup = args.steps, args.warmup
    if args.kernel == "attention":
        ctxs, pool, q, pos, tab = attention_inputs(torch, fa, args.seed)
        lay = pool.layout(0)
        step = object()   # the calls share one work plan, as the layers of one verify pass do
        for _ in range(max(warmup, 1)):
            ops.paged_attention(q, lay, tab, pos, 128 ** -0.5, plan_key=step)
        torch.cuda.synchronize()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
        for a, b in ev:
            a.record()
            ops.paged_attention(q, lay, tab, pos, 128 ** -0.5, plan_key=step)
            b.record()
        torch.cuda.synchronize()
        sec = sum(a.elapsed_time(b) for a, b in ev) / steps * 1e-3
        byts = attn_bytes(ctxs, K + 1, CFG["n_heads"], CFG["n_kv_heads"], 128, BLOCK)
        out = {"kernel": "paged_attention verify", "calls": steps, "avg_us": round(sec * 1e6, 2),
               "algorithmic_bytes": byts, "achieved_GBs": round(byts / sec / 1e9, 1)}
    elif args.kernel in ("accept", "accept_stats"):
        stats = args.kernel == "accept_stats"
        sec, byts = time_accept(torch, ops, steps, warmup, with_stats=stats)
        out = {"kernel": "spec_accept" + (" (row statistics given)" if stats else ""), "calls": steps,
               "avg_us": round(sec * 1e6, 2), "bytes": byts, "achieved_GBs": round(byts / sec / 1e9, 1)}
    elif args.kernel == "c3":
        out = c3_attention(torch, fa, ops, cpu=False)
    elif args.kernel == "c2":
        out = c2_accept(torch, ops, cpu=False)
    elif args.kernel == "gemm":
        target, draft = build_models(torch, fa)
        out = {"kernel": "gemm", "m448": gemm_summary(time_gemms(torch, ops, target, BATCH * (K + 1)),
                                                      CFG["n_layers"] - draft.cfg.n_layers, MFMA_PEAK_TFLOPS),
               "m64": gemm_summary(time_gemms(torch, ops, draft, BATCH), draft.cfg.n_layers, MFMA_PEAK_TFLOPS)}
    elif args.kernel == "gemm_prefill":
        target, _ = build_models(torch, fa)
        out = {"kernel": "gemm prefill (packed 32768-token forward, the 32 layers' four GEMMs)",
               "m32768": gemm_summary(time_gemms(torch, ops, target, PREFILL_TOKENS, passes=1, head=False),
                                      CFG["n_layers"], MFMA_PEAK_TFLOPS)}
    elif args.kernel == "prefill_attention":
        n_seq, L, h, hkv, d = 8, 4096, CFG["n_heads"], CFG["n_kv_heads"], 128
        g = torch.Generator(device="cuda").manual_seed(args.seed)
        cfg = fa.ModelConfig(vocab_size=8, d_model=h * d, n_layers=1, n_heads=h, n_kv_heads=hkv, max_seq_len=16)
        nb = -(-L // BLOCK)
        pool = fa.PagedKVPool(cfg, n_seq * nb + 8, BLOCK, dtype=torch.bfloat16, device="cuda", key_layout="groups")
        pool.k_store.normal_(generator=g)
        pool.v_store.normal_(generator=g)
        perm = torch.randperm(n_seq * nb, generator=torch.Generator().manual_seed(args.seed))
        tab = perm.view(n_seq, nb).int().cuda()
        pos = torch.arange(L, dtype=torch.int32).repeat(n_seq, 1).cuda()
        cu = torch.arange(0, (n_seq + 1) * L, L, dtype=torch.int32).cuda()
        q = torch.randn(n_seq * L, h, d, device="cuda", generator=g).bfloat16()
        lay = pool.layout(0)
        for _ in range(max(warmup, 1)):
            ops.paged_attention_varlen(q, lay, tab, pos, cu, d ** -0.5)
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(steps):
            ops.paged_attention_varlen(q, lay, tab, pos, cu, d ** -0.5)
        b.record()
        torch.cuda.synchronize()
        sec = a.elapsed_time(b) / steps * 1e-3
        flops = 4.0 * d * h * n_seq * L * (L + 1) / 2   # QK^T and PV over the causal triangle
        out = {"kernel": "paged_attention_varlen prefill", "calls": steps, "prompts": n_seq, "tokens_each": L,
               "avg_us": round(sec * 1e6, 1), "tflops": round(flops / sec / 1e12, 1),
               "frac_of_bf16_peak": round(flops / sec / 1e12 / MFMA_PEAK_TFLOPS, 4)}
    else:
        # 1 GiB device copies: f32 (16 bytes per lane per load) and bf16 (8 bytes per lane per load)
        out = {"kernel": "copy 1 GiB", "calls": steps}
        for name, dt, n in (("f32", torch.float32, 1 << 28), ("bf16", torch.bfloat16, 1 << 29)):
            src = torch.randn(n, device="cuda").to(dt)
            dst = torch.empty_like(src)
            for _ in range(warmup):
                dst.copy_(src)
            torch.cuda.synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(steps):
                dst.copy_(src)
            b.record()
            torch.cuda.synchronize()
            sec = a.elapsed_time(b) / steps * 1e-3
            out[name] = {"avg_us": round(sec * 1e6, 2), "read_bytes": 1 << 30, "write_bytes": 1 << 30,
                         "achieved_GBs": round(2 * (1 << 30) / sec / 1e9, 1)}
            del src, dst
    print(json.dumps(out), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=4)
    ap.add_argument("--temperature", type=float, default=0.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-t1-variant", action="store_true", help="skip the temperature-1.0 run")
    ap.add_argument("--synthetic-kv", action="store_true",
                    help="fill the pools with N(0,1) keys/values instead of prefilling the prompts")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-engine-1b", action="store_true", help="skip the 1B-shape engine workload")
    ap.add_argument("--kernel", choices=("round", "attention", "accept", "accept_stats", "copy", "engine_1b",
                                         "prefill_attention", "gemm", "gemm_prefill", "c2", "c3"),
                    default="round")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus})",
              file=sys.stderr)
        sys.exit(2)
    if args.kernel == "engine_1b":
        print(json.dumps(engine_1b(args)), flush=True)
        return
    if args.kernel != "round":
        kernel_mode(args)
        return

    import torch

    import forgeserve_amd as fa
    from forgeserve_amd import ops

    assert torch.cuda.is_available(), "bench.py needs a ROCm GPU"
    t0 = time.time()
    target, draft = build_models(torch, fa)
    log(f"models built in {time.time() - t0:.1f}s")

    main_run = run_rounds(torch, fa, ops, target, draft, args, args.temperature, timing=True)
    elapsed, committed = main_run["elapsed"], main_run["committed"]
    proposed, accepted = main_run["proposed"], main_run["accepted"]
    attn_avg, attn_bytes_launch = main_run["attn_avg"], main_run["attn_bytes"]
    attn_gbs = attn_bytes_launch / attn_avg / 1e9
    attn_traffic = attn_bytes_launch
    prefill = main_run["prefill"]
    value = committed / elapsed
    t1 = None
    if not args.no_t1_variant and args.temperature != 1.0:
        r = run_rounds(torch, fa, ops, target, draft, args, 1.0, timing=False)
        t1 = {"value": round(r["committed"] / r["elapsed"], 2), "unit": "tok/s", "temperature": 1.0,
              "ms_per_step": round(r["elapsed"] / args.steps * 1e3, 3),
              "acceptance": {"proposed": r["proposed"], "accepted": r["accepted"],
                             "rate": round(r["accepted"] / max(r["proposed"], 1), 4),
                             "committed_per_round": round(r["committed"] / args.steps, 2)}}

    v = CFG["vocab_size"]
    acc_avg, _ = time_accept(torch, ops, 20, 3)
    acc_gbs = accept_bytes(BATCH, K, v) / acc_avg / 1e9
    accs_avg, accs_read = time_accept(torch, ops, 20, 3, with_stats=True)
    head_ep = head_epilogue_cost(torch, ops, target)
    gemm_verify = gemm_summary(time_gemms(torch, ops, target, BATCH * (K + 1)), CFG["n_layers"] - draft.cfg.n_layers,
                               MFMA_PEAK_TFLOPS)
    gemm_draft = gemm_summary(time_gemms(torch, ops, draft, BATCH), draft.cfg.n_layers, MFMA_PEAK_TFLOPS)
    log("timing the attention and acceptance configurations ...")
    c3 = c3_attention(torch, fa, ops, cpu=not args.no_cpu_baseline)
    c2 = c2_accept(torch, ops, cpu=not args.no_cpu_baseline)
    eng = None
    if not args.no_engine_1b:
        del target, draft
        torch.cuda.empty_cache()
        log("running the 1B-shape engine workload ...")
        eng = engine_1b(args)

    result = {
        "metric": "accepted tok/s (8B-shape, k=6, bs=64); verify-attn HBM GB/s vs peak",
        "value": round(value, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed / args.steps * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": ("synthetic (random-init N(0,0.02) weights; " +
                 ("N(0,1) bf16 context KV)" if args.synthetic_kv else
                  "uniform random prompt ids, contexts prefilled through the models)")),
        "config": {"workload": "8B-shape speculative decode: 32L d4096 32/8 heads hd128 ffn14336 V128256 bf16, "
                               "early-exit draft 4 layers, batch 64, k=6, contexts U[2048,8192], block 16",
                   "global_batch": BATCH, "k": K, "temperature": args.temperature, "parallelism": "none (1 GPU)"},
        "acceptance": {"proposed": proposed, "accepted": accepted,
                       "rate": round(accepted / max(proposed, 1), 4),
                       "committed_per_round": round(committed / args.steps, 2)},
        "roofline": {"bound": "hbm", "achieved": round(attn_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(attn_gbs / HBM_PEAK_GBS, 4),
                     "traffic": profiled_traffic("paged_attention_verify_8b.md"),
                     "kernel": "paged_attention verify: attn_unit_kernel<128,16>, one call per layer, after one "
                               "attn_plan_kernel per pass; " + main_run["combine_note"],
                     "avg_launch_us": round(attn_avg * 1e6, 2),
                     "algorithmic_bytes_per_launch": int(attn_traffic)},
        "accept_kernel": {"avg_us": round(acc_avg * 1e6, 2), "achieved_GBs": round(acc_gbs, 1),
                          "algorithmic_bytes": accept_bytes(BATCH, K, v),
                          "traffic": profiled_traffic("spec_accept_8b.md"),
                          # as the round runs it: the rows' statistics come from the LM heads' epilogue,
                          # so the call reads only what its bytes_read says; achieved_GBs is on those bytes
                          "with_head_stats": {"avg_us": round(accs_avg * 1e6, 2), "bytes_read": accs_read,
                                              "achieved_GBs": round(accs_read / accs_avg / 1e9, 1),
                                              "head_epilogue_us": head_ep,
                                              "note": "the statistics pass is not timed here: the LM head's "
                                                      "epilogue computes it (head_epilogue_us: its marginal "
                                                      "cost per head call, with statistics minus without)"}},
        "c3_attention": c3,
        "c2_accept": c2,
        "engine_1b": eng,
        "prefill": prefill,
        "verify_pass": main_run["phases"],
        "t1_variant": t1,
        # MFMA utilisation of the GEMM kernels (bf16 dense peak 2.5 PFLOP/s), each shape run as the round
        # runs it (split-K partials, the SwiGLU and statistics epilogues) back to back over the layers'
        # weights, event-timed after the rounds
        "gemm_verify_m448": gemm_verify,
        "gemm_draft_m64": gemm_draft,
    }
    if not args.no_cpu_baseline:
        log("timing the CPU baseline ...")
        result["cpu_baseline"] = cpu_baseline(torch, committed / args.steps)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
