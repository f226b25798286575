"""ctypes binding of libdsv41hip.so (the C ABI declared in include/dsv41_rocm.h).

The library is loaded from this package directory only.  There is no fallback:
if the library is missing or was built for another ABI, every product entry point
raises ``RuntimeError`` naming the file and the build step.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

LIB_PATH = Path(__file__).with_name("libdsv41hip.so")
ABI_VERSION = 6

DTYPE_F32 = 0
DTYPE_BF16 = 1

OK = 0
E_INVALID = -1
E_UNSUPPORTED = -2
E_WORKSPACE = -3
E_HIP = -4
E_ABI = -5

STATUS_NONFINITE = 1
STATUS_BAD_HISTORY = 2
STATUS_BAD_UNIFORM = 4
STATUS_RATIO_ZERO = 8
STATUS_BAD_TARGET = 16
STATUS_BAD_SLICES = 32


class SamplerDesc(ctypes.Structure):
    """Mirror of dsv41_sampler_desc."""

    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("rows", ctypes.c_int32),
        ("vocab", ctypes.c_int32),
        ("logits_dtype", ctypes.c_int32),
        ("logits_row_stride", ctypes.c_int64),
        ("logits", ctypes.c_void_p),
        ("history", ctypes.c_void_p),
        ("history_row_stride", ctypes.c_int64),
        ("hist_len", ctypes.c_int32),
        ("history_lens", ctypes.c_void_p),
        ("uniforms", ctypes.c_void_p),
        ("temperature", ctypes.c_float),
        ("repetition_penalty", ctypes.c_float),
        ("presence_penalty", ctypes.c_float),
        ("frequency_penalty", ctypes.c_float),
        ("top_k", ctypes.c_int32),
        ("top_p", ctypes.c_float),
        ("min_p", ctypes.c_float),
        ("greedy", ctypes.c_int32),
        ("out_ids", ctypes.c_void_p),
        ("out_logprob", ctypes.c_void_p),
        ("out_kept", ctypes.c_void_p),
        ("out_status", ctypes.c_void_p),
        ("exponentials", ctypes.c_void_p),
        ("exponentials_row_stride", ctypes.c_int64),
        ("replay_ids", ctypes.c_void_p),
        ("history_prompt_lens", ctypes.c_void_p),
    ]


class LogprobDesc(ctypes.Structure):
    """Mirror of dsv41_logprob_desc."""

    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("n_tokens", ctypes.c_int32),
        ("hidden", ctypes.c_int32),
        ("vocab", ctypes.c_int32),
        ("x", ctypes.c_void_p),
        ("x_row_stride", ctypes.c_int64),
        ("w", ctypes.c_void_p),
        ("w_row_stride", ctypes.c_int64),
        ("targets", ctypes.c_void_p),
        ("temperature", ctypes.c_float),
        ("behavior", ctypes.c_void_p),
        ("is_cap", ctypes.c_float),
        ("out_logprob", ctypes.c_void_p),
        ("out_entropy", ctypes.c_void_p),
        ("out_ratio", ctypes.c_void_p),
        ("out_status", ctypes.c_void_p),
        ("out_lse", ctypes.c_void_p),
    ]


class LogprobGradDesc(ctypes.Structure):
    """Mirror of dsv41_logprob_grad_desc."""

    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("n_tokens", ctypes.c_int32),
        ("hidden", ctypes.c_int32),
        ("vocab", ctypes.c_int32),
        ("x", ctypes.c_void_p),
        ("x_row_stride", ctypes.c_int64),
        ("w", ctypes.c_void_p),
        ("w_row_stride", ctypes.c_int64),
        ("targets", ctypes.c_void_p),
        ("temperature", ctypes.c_float),
        ("lse", ctypes.c_void_p),
        ("entropy", ctypes.c_void_p),
        ("grad_logprob", ctypes.c_void_p),
        ("grad_entropy", ctypes.c_void_p),
        ("vocab_begin", ctypes.c_int32),
        ("vocab_end", ctypes.c_int32),
        ("out", ctypes.c_void_p),
        ("out_row_stride", ctypes.c_int64),
    ]


class TokenTisDesc(ctypes.Structure):
    """Mirror of dsv41_token_tis_desc."""

    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("n_responses", ctypes.c_int32),
        ("n_tokens", ctypes.c_int64),
        ("offsets", ctypes.c_void_p),
        ("current", ctypes.c_void_p),
        ("native_old", ctypes.c_void_p),
        ("behavior", ctypes.c_void_p),
        ("advantages", ctypes.c_void_p),
        ("clip_eps", ctypes.c_double),
        ("is_cap", ctypes.c_double),
        ("out_loss", ctypes.c_void_p),
        ("out_grad", ctypes.c_void_p),
        ("out_metrics", ctypes.c_void_p),
        ("out_status", ctypes.c_void_p),
    ]


class GrpoDesc(ctypes.Structure):
    """Mirror of dsv41_grpo_desc."""

    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("n_responses", ctypes.c_int32),
        ("n_tokens", ctypes.c_int64),
        ("offsets", ctypes.c_void_p),
        ("current", ctypes.c_void_p),
        ("behavior", ctypes.c_void_p),
        ("reference", ctypes.c_void_p),
        ("advantages", ctypes.c_void_p),
        ("clip_eps", ctypes.c_double),
        ("kl_beta", ctypes.c_double),
        ("out_loss", ctypes.c_void_p),
        ("out_grad", ctypes.c_void_p),
        ("out_metrics", ctypes.c_void_p),
        ("out_status", ctypes.c_void_p),
    ]


class LogprobShardDesc(ctypes.Structure):
    """Mirror of dsv41_logprob_shard_desc."""

    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("n_tokens", ctypes.c_int32),
        ("hidden", ctypes.c_int32),
        ("vocab", ctypes.c_int32),
        ("x", ctypes.c_void_p),
        ("x_row_stride", ctypes.c_int64),
        ("w", ctypes.c_void_p),
        ("w_row_stride", ctypes.c_int64),
        ("targets", ctypes.c_void_p),
        ("vocab_offset", ctypes.c_int64),
        ("temperature", ctypes.c_float),
        ("out_state", ctypes.c_void_p),
    ]


class LogprobCombineDesc(ctypes.Structure):
    """Mirror of dsv41_logprob_combine_desc."""

    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("n_tokens", ctypes.c_int32),
        ("n_shards", ctypes.c_int32),
        ("states", ctypes.c_void_p),
        ("behavior", ctypes.c_void_p),
        ("is_cap", ctypes.c_float),
        ("out_logprob", ctypes.c_void_p),
        ("out_entropy", ctypes.c_void_p),
        ("out_ratio", ctypes.c_void_p),
        ("out_status", ctypes.c_void_p),
        ("out_lse", ctypes.c_void_p),
    ]


class SamplerShardDesc(ctypes.Structure):
    """dsv41_sampler_shard_desc: one vocabulary slice of a sharded sampling batch."""

    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("max_candidates", ctypes.c_int32),
        ("sampler", ctypes.POINTER(SamplerDesc)),
        ("vocab_offset", ctypes.c_int64),
        ("vocab_size", ctypes.c_int64),
        ("out_keys", ctypes.c_void_p),
        ("out_counts", ctypes.c_void_p),
        ("out_status", ctypes.c_void_p),
    ]


class SamplerMergeDesc(ctypes.Structure):
    """dsv41_sampler_merge_desc: the exact finish of a sharded batch."""

    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("rows", ctypes.c_int32),
        ("n_shards", ctypes.c_int32),
        ("max_candidates", ctypes.c_int32),
        ("keys", ctypes.c_void_p),
        ("counts", ctypes.c_void_p),
        ("status", ctypes.c_void_p),
        ("uniforms", ctypes.c_void_p),
        ("top_k", ctypes.c_int32),
        ("top_p", ctypes.c_float),
        ("min_p", ctypes.c_float),
        ("greedy", ctypes.c_int32),
        ("out_ids", ctypes.c_void_p),
        ("out_logprob", ctypes.c_void_p),
        ("out_kept", ctypes.c_void_p),
        ("out_status", ctypes.c_void_p),
    ]


class SamplerFullShardDesc(ctypes.Structure):
    """dsv41_sampler_full_shard_desc: one vocabulary slice of a full-vocabulary draw."""

    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("n_shards", ctypes.c_int32),
        ("sampler", ctypes.POINTER(SamplerDesc)),
        ("vocab_offset", ctypes.c_int64),
        ("vocab_size", ctypes.c_int64),
        ("shard_index", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("states", ctypes.c_void_p),
        ("out_states", ctypes.c_void_p),
        ("out_picks", ctypes.c_void_p),
        ("masses", ctypes.c_void_p),
        ("out_masses", ctypes.c_void_p),
    ]


class SamplerFullFinishDesc(ctypes.Structure):
    """dsv41_sampler_full_finish_desc: the finish of a full-vocabulary draw over slices."""

    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("rows", ctypes.c_int32),
        ("n_shards", ctypes.c_int32),
        ("draw", ctypes.c_int32),
        ("states", ctypes.c_void_p),
        ("picks", ctypes.c_void_p),
        ("uniforms", ctypes.c_void_p),
        ("vocab_size", ctypes.c_int64),
        ("out_ids", ctypes.c_void_p),
        ("out_logprob", ctypes.c_void_p),
        ("out_kept", ctypes.c_void_p),
        ("out_status", ctypes.c_void_p),
    ]


FULL_DRAW_CDF = 0
FULL_DRAW_RACE = 1
FULL_DRAW_GREEDY = 2
SAMPLER_STATIC_SCRATCH_BYTES = 32 << 20  # DSV41_SAMPLER_STATIC_SCRATCH_BYTES
FULL_STATE_BYTES = 32  # dsv41_full_state
FULL_PICK_BYTES = 16   # dsv41_full_pick


EXPORTS = (
    "dsv41_abi_version",
    "dsv41_sampler_desc_size",
    "dsv41_logprob_desc_size",
    "dsv41_logprob_grad_desc_size",
    "dsv41_token_tis_desc_size",
    "dsv41_grpo_desc_size",
    "dsv41_logprob_shard_desc_size",
    "dsv41_logprob_combine_desc_size",
    "dsv41_sampler_shard_desc_size",
    "dsv41_sampler_merge_desc_size",
    "dsv41_sampler_full_shard_desc_size",
    "dsv41_sampler_full_finish_desc_size",
    "dsv41_last_error",
    "dsv41_sampler_workspace_bytes",
    "dsv41_sampler_run",
    "dsv41_sampler_run_static",
    "dsv41_logprob_workspace_bytes",
    "dsv41_logprob_run",
    "dsv41_logprob_grad_run",
    "dsv41_token_tis_workspace_bytes",
    "dsv41_token_tis_run",
    "dsv41_grpo_workspace_bytes",
    "dsv41_grpo_run",
    "dsv41_logprob_shard_workspace_bytes",
    "dsv41_logprob_shard_run",
    "dsv41_logprob_combine_run",
    "dsv41_sampler_shard_run",
    "dsv41_sampler_merge_run",
    "dsv41_sampler_full_state_run",
    "dsv41_sampler_full_mass_run",
    "dsv41_sampler_full_draw_run",
    "dsv41_sampler_full_finish_run",
)

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def _bind(lib: ctypes.CDLL) -> ctypes.CDLL:
    lib.dsv41_abi_version.restype = ctypes.c_int
    lib.dsv41_sampler_desc_size.restype = ctypes.c_size_t
    lib.dsv41_logprob_desc_size.restype = ctypes.c_size_t
    lib.dsv41_logprob_grad_desc_size.restype = ctypes.c_size_t
    lib.dsv41_token_tis_desc_size.restype = ctypes.c_size_t
    lib.dsv41_grpo_desc_size.restype = ctypes.c_size_t
    lib.dsv41_logprob_shard_desc_size.restype = ctypes.c_size_t
    lib.dsv41_logprob_combine_desc_size.restype = ctypes.c_size_t
    lib.dsv41_sampler_shard_desc_size.restype = ctypes.c_size_t
    lib.dsv41_sampler_merge_desc_size.restype = ctypes.c_size_t
    lib.dsv41_sampler_full_shard_desc_size.restype = ctypes.c_size_t
    lib.dsv41_sampler_full_finish_desc_size.restype = ctypes.c_size_t
    lib.dsv41_last_error.restype = ctypes.c_char_p
    lib.dsv41_sampler_workspace_bytes.restype = ctypes.c_size_t
    lib.dsv41_sampler_workspace_bytes.argtypes = [ctypes.POINTER(SamplerDesc)]
    lib.dsv41_sampler_run.restype = ctypes.c_int
    lib.dsv41_sampler_run.argtypes = [ctypes.POINTER(SamplerDesc), ctypes.c_void_p, ctypes.c_size_t,
                                      ctypes.c_void_p]
    lib.dsv41_sampler_run_static.restype = ctypes.c_int
    lib.dsv41_sampler_run_static.argtypes = [ctypes.POINTER(SamplerDesc), ctypes.c_void_p]
    lib.dsv41_logprob_workspace_bytes.restype = ctypes.c_size_t
    lib.dsv41_logprob_workspace_bytes.argtypes = [ctypes.POINTER(LogprobDesc)]
    lib.dsv41_logprob_run.restype = ctypes.c_int
    lib.dsv41_logprob_run.argtypes = [ctypes.POINTER(LogprobDesc), ctypes.c_void_p, ctypes.c_size_t,
                                      ctypes.c_void_p]
    lib.dsv41_logprob_grad_run.restype = ctypes.c_int
    lib.dsv41_logprob_grad_run.argtypes = [ctypes.POINTER(LogprobGradDesc), ctypes.c_void_p]
    lib.dsv41_token_tis_workspace_bytes.restype = ctypes.c_size_t
    lib.dsv41_token_tis_workspace_bytes.argtypes = [ctypes.POINTER(TokenTisDesc)]
    lib.dsv41_token_tis_run.restype = ctypes.c_int
    lib.dsv41_token_tis_run.argtypes = [ctypes.POINTER(TokenTisDesc), ctypes.c_void_p, ctypes.c_size_t,
                                        ctypes.c_void_p]
    lib.dsv41_grpo_workspace_bytes.restype = ctypes.c_size_t
    lib.dsv41_grpo_workspace_bytes.argtypes = [ctypes.POINTER(GrpoDesc)]
    lib.dsv41_grpo_run.restype = ctypes.c_int
    lib.dsv41_grpo_run.argtypes = [ctypes.POINTER(GrpoDesc), ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    lib.dsv41_logprob_shard_workspace_bytes.restype = ctypes.c_size_t
    lib.dsv41_logprob_shard_workspace_bytes.argtypes = [ctypes.POINTER(LogprobShardDesc)]
    lib.dsv41_logprob_shard_run.restype = ctypes.c_int
    lib.dsv41_logprob_shard_run.argtypes = [ctypes.POINTER(LogprobShardDesc), ctypes.c_void_p, ctypes.c_size_t,
                                            ctypes.c_void_p]
    lib.dsv41_logprob_combine_run.restype = ctypes.c_int
    lib.dsv41_logprob_combine_run.argtypes = [ctypes.POINTER(LogprobCombineDesc), ctypes.c_void_p]
    lib.dsv41_sampler_shard_run.restype = ctypes.c_int
    lib.dsv41_sampler_shard_run.argtypes = [ctypes.POINTER(SamplerShardDesc), ctypes.c_void_p]
    lib.dsv41_sampler_merge_run.restype = ctypes.c_int
    lib.dsv41_sampler_merge_run.argtypes = [ctypes.POINTER(SamplerMergeDesc), ctypes.c_void_p]
    for name in ("dsv41_sampler_full_state_run", "dsv41_sampler_full_mass_run", "dsv41_sampler_full_draw_run"):
        getattr(lib, name).restype = ctypes.c_int
        getattr(lib, name).argtypes = [ctypes.POINTER(SamplerFullShardDesc), ctypes.c_void_p]
    lib.dsv41_sampler_full_finish_run.restype = ctypes.c_int
    lib.dsv41_sampler_full_finish_run.argtypes = [ctypes.POINTER(SamplerFullFinishDesc), ctypes.c_void_p]
    return lib


def load() -> ctypes.CDLL:
    """Load and check libdsv41hip.so; raise RuntimeError when it is absent or stale."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.is_file():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `make -C {LIB_PATH.parent.parent}` "
                "(or __graft_entry__.build()); there is no CPU fallback")
        lib = _bind(ctypes.CDLL(os.fspath(LIB_PATH)))
        if lib.dsv41_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH} has ABI {lib.dsv41_abi_version()}, expected {ABI_VERSION}")
        if lib.dsv41_sampler_desc_size() != ctypes.sizeof(SamplerDesc):
            raise RuntimeError("dsv41_sampler_desc layout differs between library and binding")
        if lib.dsv41_logprob_desc_size() != ctypes.sizeof(LogprobDesc):
            raise RuntimeError("dsv41_logprob_desc layout differs between library and binding")
        if lib.dsv41_logprob_grad_desc_size() != ctypes.sizeof(LogprobGradDesc):
            raise RuntimeError("dsv41_logprob_grad_desc layout differs between library and binding")
        if lib.dsv41_token_tis_desc_size() != ctypes.sizeof(TokenTisDesc):
            raise RuntimeError("dsv41_token_tis_desc layout differs between library and binding")
        if lib.dsv41_grpo_desc_size() != ctypes.sizeof(GrpoDesc):
            raise RuntimeError("dsv41_grpo_desc layout differs between library and binding")
        if lib.dsv41_logprob_shard_desc_size() != ctypes.sizeof(LogprobShardDesc):
            raise RuntimeError("dsv41_logprob_shard_desc layout differs between library and binding")
        if lib.dsv41_logprob_combine_desc_size() != ctypes.sizeof(LogprobCombineDesc):
            raise RuntimeError("dsv41_logprob_combine_desc layout differs between library and binding")
        if lib.dsv41_sampler_shard_desc_size() != ctypes.sizeof(SamplerShardDesc):
            raise RuntimeError("dsv41_sampler_shard_desc layout differs between library and binding")
        if lib.dsv41_sampler_merge_desc_size() != ctypes.sizeof(SamplerMergeDesc):
            raise RuntimeError("dsv41_sampler_merge_desc layout differs between library and binding")
        if lib.dsv41_sampler_full_shard_desc_size() != ctypes.sizeof(SamplerFullShardDesc):
            raise RuntimeError("dsv41_sampler_full_shard_desc layout differs between library and binding")
        if lib.dsv41_sampler_full_finish_desc_size() != ctypes.sizeof(SamplerFullFinishDesc):
            raise RuntimeError("dsv41_sampler_full_finish_desc layout differs between library and binding")
        _lib = lib
        return lib


def last_error() -> str:
    msg = load().dsv41_last_error()
    return msg.decode() if msg else ""


def check(rc: int) -> None:
    """Map a negative return code to the Python exception the reference raises."""
    if rc == OK:
        return
    msg = last_error()
    if rc in (E_INVALID, E_WORKSPACE):
        raise ValueError(msg)
    if rc == E_UNSUPPORTED:
        raise NotImplementedError(msg)
    raise RuntimeError(f"libdsv41hip error {rc}: {msg}")
