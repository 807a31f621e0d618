"""ctypes binding of libforgeserve_hip.so (declarations: include/forgeserve_amd.h).

The library is loaded after torch so that it binds to the HIP runtime torch already mapped (both
carry the soname libamdhip64.so.7): device pointers and streams from torch are then valid in it.
There is no fallback: if the library is missing or no ROCm GPU is visible, every op raises.
"""

import ctypes
import os

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libforgeserve_hip.so")

F32, BF16, F16 = 0, 1, 2
DTYPE_CODE = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16}

c_i32, c_i64, c_f32, c_p = ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p


class KVLayout(ctypes.Structure):
    """fs_kv_layout: one layer of a paged pool."""

    _fields_ = [
        ("k", c_p), ("v", c_p),
        ("k_block", c_i64), ("k_head", c_i64), ("k_slot", c_i64), ("k_dim", c_i64),
        ("v_block", c_i64), ("v_head", c_i64), ("v_slot", c_i64), ("v_dim", c_i64),
        ("block_size", c_i32), ("n_kv_heads", c_i32), ("head_dim", c_i32), ("dtype", c_i32),
        ("num_blocks", c_i64), ("k_group", c_i64),
    ]


# name -> (restype, argtypes)
SIGNATURES = {
    "fs_last_error": (ctypes.c_char_p, []),
    "fs_abi_version": (c_i32, []),
    "fs_qkv_rope_write": (c_i32, [c_p, c_i64, c_i64, c_i32, c_i32, c_p, c_p, c_p, c_p, c_i32, c_p, c_i64, c_i32,
                                  ctypes.POINTER(KVLayout), c_p, c_i64, c_p]),
    "fs_qkv_rope_write_varlen": (c_i32, [c_p, c_i64, c_i64, c_i32, c_p, c_p, c_i32, c_p, c_p, c_i32, c_p, c_i64, c_i32,
                                         ctypes.POINTER(KVLayout), c_p, c_i64, c_p]),
    "fs_qkv_rope_write_partials": (c_i32, [c_p, c_i32, c_i64, c_i64, c_i32, c_i32, c_p, c_p, c_p, c_p, c_i32, c_p,
                                           c_i64, c_i32, ctypes.POINTER(KVLayout), c_p, c_i64, c_p]),
    "fs_paged_kv_write": (c_i32, [c_p, c_p, c_i64, c_i64, c_i64, c_i32, c_i32, c_p, c_p, c_i64, c_i32,
                                  ctypes.POINTER(KVLayout), c_p]),
    "fs_paged_gather": (c_i32, [ctypes.POINTER(KVLayout), c_p, c_i64, c_i32, c_i32, c_p, c_p, c_p]),
    "fs_paged_attention": (c_i32, [c_p, c_i64, c_i64, c_i64, ctypes.POINTER(KVLayout), c_p, c_i64, c_i32, c_p,
                                   c_i32, c_i32, c_i32, c_f32, c_p, c_i64, c_i64, c_i64, c_p, c_i64, c_p]),
    "fs_paged_attention_varlen": (c_i32, [c_p, c_i64, c_i64, ctypes.POINTER(KVLayout), c_p, c_i64, c_i32, c_p, c_p,
                                          c_i32, c_i32, c_i32, c_f32, c_p, c_i64, c_i64, c_p, c_i64, c_p]),
    "fs_paged_attention_reuse_plan": (c_i32, [c_p, c_i64, c_i64, c_i64, ctypes.POINTER(KVLayout), c_p, c_i64, c_i32,
                                              c_p, c_i32, c_i32, c_i32, c_f32, c_p, c_i64, c_i64, c_i64, c_p, c_i64,
                                              c_p]),
    "fs_paged_attention_varlen_reuse_plan": (c_i32, [c_p, c_i64, c_i64, ctypes.POINTER(KVLayout), c_p, c_i64, c_i32,
                                                     c_p, c_p, c_i32, c_i32, c_i32, c_f32, c_p, c_i64, c_i64, c_p,
                                                     c_i64, c_p]),
    "fs_paged_attention_workspace_size": (c_i64, [c_i32, c_i32, c_i32, c_i32, c_i32, c_i32]),
    "fs_paged_attention_split": (c_i32, []),
    "fs_gemm": (c_i32, [c_p, c_i64, c_p, c_i64, c_p, c_i64, c_p, c_i64, c_i64, c_i64, c_i64, c_i32, c_p, c_i64,
                        c_p]),
    "fs_gemm_workspace_size": (c_i64, [c_i64, c_i64, c_i64, c_i32]),
    "fs_gemm_splits": (c_i32, [c_i64, c_i64, c_i32]),
    "fs_gemm_serial": (c_i32, [c_i64, c_i64, c_i64, c_i32]),
    "fs_gemm_partials": (c_i32, [c_p, c_i64, c_p, c_i64, c_i64, c_i64, c_i64, c_i32, c_p, c_i64, c_p]),
    "fs_splitk_add_rmsnorm": (c_i32, [c_p, c_i32, c_p, c_i64, c_p, c_i64, c_p, c_p, c_i64, c_i64, c_i64, c_f32, c_i32,
                                      c_p]),
    "fs_gemm_row_stats": (c_i32, [c_p, c_i64, c_p, c_i64, c_p, c_i64, c_i64, c_i64, c_i64, c_p, c_p, c_i64, c_i64,
                                  c_p]),
    "fs_gemm_row_stats_parts": (c_i64, [c_i64, c_i64, c_i64]),
    "fs_row_stats_merge": (c_i32, [c_p, c_i64, c_i64, c_i64, c_p, c_i32, c_i64, c_i64, c_p]),
    "fs_add_rmsnorm": (c_i32, [c_p, c_i64, c_p, c_i64, c_p, c_i64, c_p, c_p, c_i64, c_i64, c_i64, c_f32, c_i32, c_p]),
    "fs_silu_mul": (c_i32, [c_p, c_i64, c_p, c_i64, c_i64, c_i64, c_i32, c_p]),
    "fs_gemm_swiglu": (c_i32, [c_p, c_i64, c_p, c_i64, c_p, c_i64, c_i64, c_i64, c_i64, c_i32, c_p]),
    "fs_spec_advance": (c_i32, [c_p, c_i64, c_i32, c_i32, c_i32, c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_p,
                                c_p]),
    "fs_embedding": (c_i32, [c_p, c_i64, c_p, c_i64, c_i64, c_p, c_i64, c_i32, c_p]),
    "fs_probs_from_logits": (c_i32, [c_p, c_i64, c_i64, c_i64, c_f32, c_i32, c_p, c_i64, c_i32, c_p, c_i64, c_p]),
    "fs_sample_logits": (c_i32, [c_p, c_i64, c_i64, c_i64, c_p, c_f32, c_p, c_i64, c_i32, c_p, c_p, c_i64, c_p,
                                 c_i64, c_p]),
    "fs_sampling_workspace_size": (c_i64, [c_i64, c_i64]),
    "fs_spec_accept": (c_i32, [c_p, c_i64, c_i64, c_p, c_i64, c_i64, c_i32, c_i32, c_i64, c_i32, c_p, c_p, c_p,
                               c_p, c_p, c_i64, c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_i64, c_p]),
    "fs_spec_accept_stats": (c_i32, [c_p, c_i64, c_i64, c_p, c_i64, c_i64, c_i32, c_i32, c_i64, c_i32, c_p, c_p, c_p,
                                     c_p, c_p, c_i64, c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_i64, c_p]),
    "fs_spec_accept_noalloc": (c_i32, [c_p, c_i64, c_i64, c_p, c_i64, c_i64, c_i32, c_i32, c_i64, c_i32, c_p, c_p,
                                       c_p, c_p, c_p, c_i64, c_p, c_p, c_p, c_p, c_p]),
    "fs_verify_probs": (c_i32, [c_p, c_i64, c_p, c_i64, c_i32, c_i64, c_i32, c_p, c_p, c_p, c_p, c_p, c_p, c_i64,
                                c_p]),
    "fs_spec_accept_workspace_size": (c_i64, [c_i32, c_i32, c_i64]),
    "fs_keyed_noise": (c_i32, [c_p, c_i32, c_i32, c_i32, c_i64, c_i32, c_p, c_i64, c_i64, c_p]),
}

_lib = None


def load() -> ctypes.CDLL:
    """Load the library (no GPU needed to load it; launching needs one)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run `python -m forgeserve_amd.build`")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


class FSError(RuntimeError):
    pass


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().fs_last_error().decode(errors="replace")
        if rc < 0:
            raise ValueError(f"{what}: {msg}")
        raise FSError(f"{what}: hip error {rc}: {msg}")


def to_device(t: torch.Tensor, device, dtype=None) -> torch.Tensor:
    """A host tensor on `device` without stalling the host: a copy from pageable memory waits until the
    device has drained its queue, so host tensors are staged through pinned memory and copied
    asynchronously (the pinned block is held until the copy has run)."""
    if dtype is not None and t.dtype != dtype:
        t = t.to(dtype)
    if t.device.type != "cpu":
        return t.to(device)
    return t.pin_memory().to(device, non_blocking=True)


def require_device(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError(
                f"forgeserve_amd runs its kernels on a ROCm GPU; got a tensor on {t.device} "
                "(there is no CPU path)")


def stream_ptr(device=None) -> int:
    """The current HIP stream of `device` (default: the current device) as a raw pointer."""
    idx = torch.cuda.current_device() if device is None else torch.device(device).index
    if idx is None:
        idx = torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(idx)


def ptr(t) -> int:
    return 0 if t is None else t.data_ptr()
