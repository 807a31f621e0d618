"""CPU oracle of the forgeserve speculative-decoding hot path. TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg may import this package, and
only as the checker (or the timed CPU baseline); the product path (forgeserve_amd) never calls it.

It restates, from scratch and in PyTorch on the CPU (float32, the reference's own arithmetic), the
reference algorithms the GPU kernels must reproduce:

  model.py:23-159     RMSNorm, half-split rotary, GQA attention with the key<=position mask,
                      SwiGLU, pre-norm blocks, tied head           -> oracle.reference_cpu.forward
  kv.py:10-33         contiguous cache append/truncate            -> ContiguousCache
  paged.py:20-82      allocator, pool, scatter + table gather      -> Allocator, PagedPool
  sampling.py:9-35    probs_from_logits, sample, generate         -> probs_from_logits, sample, generate
  speculative.py      verify_draft, speculative_generate          -> verify_with_noise, verify_draft,
                                                                     speculative_generate
  engine.py:36-139    continuous batching with preemption         -> Engine

and, in oracle.keyed_noise, the counter-based (Philox4x32-10) per-request random stream that the
speculative Engine draws instead of the reference's shared generator (engine.py:41, 126-133).

Pinning (tests/test_oracle.py): every function is checked against golden vectors written by the
reference itself (tests/golden/make_golden.py) and/or closed forms and library identities
(torch.multinomial == argmax(p / Exp(1) noise), softmax in float64, brute-force attention).
"""
