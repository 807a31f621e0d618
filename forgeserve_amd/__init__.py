"""forgeserve_amd: the speculative-decoding hot path of forgeserve on MI355X (gfx950) HIP kernels.

The public names match the reference's forgeserve/__init__.py:11 for the hot path (the pipeline
helpers are not part of this build). Batched speculation is added as SpeculativeBatch /
speculative_generate_batch.
"""

from .config import ModelConfig
from .engine import Engine, Request
from .kv import ContiguousKV, new_contiguous_cache
from .model import ForgeModel, early_exit_draft, prefill_packed
from .paged import BlockAllocator, OutOfBlocks, PagedKVPool
from .parallel import SINGLE, TPContext
from .sampling import generate, probs_from_logits, sample
from .speculative import SpeculativeBatch, speculative_generate, speculative_generate_batch, verify_draft

__all__ = ["speculative_generate", "verify_draft", "Engine", "Request", "BlockAllocator", "OutOfBlocks",
           "PagedKVPool", "ModelConfig", "ForgeModel", "TPContext", "SINGLE", "ContiguousKV",
           "new_contiguous_cache", "generate", "sample", "probs_from_logits", "early_exit_draft",
           "SpeculativeBatch", "speculative_generate_batch", "prefill_packed"]
