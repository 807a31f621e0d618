"""Shared test helpers: golden fixtures, synthetic models for the product and the oracle."""

import json
import os

import numpy as np
import torch

from oracle import reference_cpu as orc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

SMALL = dict(vocab_size=64, d_model=64, n_layers=3, n_heads=8, n_kv_heads=4, max_seq_len=64)
C1 = dict(vocab_size=512, d_model=256, n_layers=4, n_heads=8, n_kv_heads=4, ffn_dim=688, max_seq_len=256)


def golden_json(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


def golden_npz(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def oracle_model(cfg_kw, seed, std, n_layers=None):
    """(weights, shape) of the oracle for a synthetic model."""
    from forgeserve_amd.config import ModelConfig

    s = orc.Shape.of(ModelConfig(**cfg_kw))
    w = orc.synthetic_weights(s, seed, std)
    if n_layers is not None:
        w = orc.draft_weights(w, n_layers)
        s = orc.Shape(**{**s.__dict__, "n_layers": n_layers})
    return w, s


def product_model(cfg_kw, seed, std, dtype=torch.float32, n_layers=None, device="cuda"):
    """A forgeserve_amd.ForgeModel holding the same synthetic weights as the oracle/golden models."""
    from forgeserve_amd import ForgeModel, ModelConfig

    w, _ = oracle_model(cfg_kw, seed, std)
    kw = dict(cfg_kw)
    if n_layers is not None:
        kw["n_layers"] = n_layers
        w = orc.draft_weights(w, n_layers)
    m = ForgeModel(ModelConfig(**kw)).eval()
    sd = dict(w)
    sd["lm_head.weight"] = w["tok_emb.weight"]
    m.load_state_dict(sd)
    return m.to(device=device, dtype=dtype)


# Parity figures the GPU tests measure (errors, margins, near-tie counts). conftest.py prints them in
# pytest's terminal summary, so a quiet (-q) run's output still carries them.
RECORDS = []


def record(line: str) -> None:
    print(line, flush=True)
    RECORDS.append(line)
