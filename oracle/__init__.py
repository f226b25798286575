"""CPU oracle for Tiny-DSV41's sampling step and selected-token log-prob.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package, and only as the checker
(or, for bench, as the timed CPU restatement).  The product (``libdsv41hip.so`` and the
``dsv41_rocm`` package) never imports or calls it.

* ``sample`` wraps ``sampler_oracle.c`` (plain C, exact integer/fp arithmetic), the
  restatement of ``dsv41_train/rl/rollout.py:144-150`` plus the vLLM knobs.
* ``logprob_oracle`` (numpy fp64) restates ``dsv41_train/models/dsv4/model.py:679-684``,
  ``dsv41_train/rl/native_lora.py:80-82`` and the Token-TIS weight of
  ``dsv41_train/rl/algorithm.py:293-299``; ``logprob_grad_oracle`` its backward.
* ``token_tis_loss_oracle`` (numpy) restates ``decoupled_token_tis_loss``,
  ``dsv41_train/rl/algorithm.py:249-346``, with its gradient and pooled metrics.

Pinning: tests/test_oracle_sampler.py and tests/test_oracle_logprob.py check every
function here against closed forms, brute force on tiny inputs, libm, torch and the
known answers of the reference's own tests (tests/golden/).
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

from .logprob_oracle import logprob_grad_oracle, logprob_oracle, token_tis_weight  # noqa: F401
from .tis_oracle import grpo_loss_oracle, token_tis_loss_oracle  # noqa: F401

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle_dsv41.so"

_lib = None


def build() -> None:
    """Compile the C restatement (gcc, -ffp-contract=off)."""
    subprocess.run(["make", "-B", "-C", os.fspath(HERE)], check=True, stdout=subprocess.DEVNULL)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.is_file():
            build()
        c = ctypes.CDLL(os.fspath(LIB_PATH))
        c.dsv41_exp_det.restype = ctypes.c_double
        c.dsv41_exp_det.argtypes = [ctypes.c_double]
        c.dsv41_mass.restype = ctypes.c_uint64
        c.dsv41_mass.argtypes = [ctypes.c_float, ctypes.c_float]
        c.dsv41_top_p_threshold.restype = ctypes.c_uint64
        c.dsv41_top_p_threshold.argtypes = [ctypes.c_float, ctypes.c_uint64]
        c.dsv41_draw_target.restype = ctypes.c_uint64
        c.dsv41_draw_target.argtypes = [ctypes.c_float, ctypes.c_uint64]
        c.dsv41_penalize.restype = ctypes.c_float
        c.dsv41_penalize.argtypes = [ctypes.c_float, ctypes.c_uint32, ctypes.c_float, ctypes.c_float,
                                     ctypes.c_float]
        c.dsv41_check_division.restype = ctypes.c_uint64
        c.dsv41_check_division.argtypes = [ctypes.c_float, ctypes.c_uint32, ctypes.c_uint32,
                                           ctypes.POINTER(ctypes.c_uint32)]
        c.dsv41_oracle_sample.restype = ctypes.c_int
        c.dsv41_oracle_full_draw.restype = ctypes.c_int64
        c.dsv41_oracle_full_total.restype = ctypes.c_uint64
        _lib = c
    return _lib


def exp_det(d: float) -> float:
    return lib().dsv41_exp_det(d)


def mass(z: float, zmax: float) -> int:
    return lib().dsv41_mass(z, zmax)


def top_p_threshold(p: float, s: int) -> int:
    return lib().dsv41_top_p_threshold(p, s)


def draw_target(u: float, s: int) -> int:
    return lib().dsv41_draw_target(u, s)


def penalize(x: float, count: int, rp: float, pres: float, freq: float) -> float:
    return lib().dsv41_penalize(x, count, rp, pres, freq)


def process_row(logits, *, temperature=1.0, history=None, history_prompt_len=0, repetition_penalty=1.0,
                presence_penalty=0.0, frequency_penalty=0.0):
    """Processed logits z of one row (penalties, then / T) and the status bits."""
    x = np.ascontiguousarray(np.asarray(logits, dtype=np.float32))
    V = x.shape[0]
    h = np.ascontiguousarray(np.asarray([] if history is None else history, dtype=np.int64))
    counts = np.empty(V, np.uint32)
    z = np.empty(V, np.float32)
    c = lib()
    st = c.dsv41_oracle_process_row(_ptr(x), ctypes.c_int(V), _ptr(h) if h.size else None, ctypes.c_int(h.size),
                                    ctypes.c_int(history_prompt_len), ctypes.c_float(temperature),
                                    ctypes.c_float(repetition_penalty), ctypes.c_float(presence_penalty),
                                    ctypes.c_float(frequency_penalty), _ptr(counts), _ptr(z))
    return z, int(st)


def full_draw(z, U: int, *, history_ids=None, slice_starts=None) -> int:
    """The full-vocabulary inverse-CDF draw of processed logits ``z`` at the 32-bit uniform
    ``U`` (u = U / 2^32); ``history_ids``: the ids the penalties processed."""
    z = np.ascontiguousarray(np.asarray(z, dtype=np.float32))
    counts = None
    if history_ids is not None:
        counts = np.zeros(z.shape[0], np.uint32)
        counts[np.asarray(history_ids, dtype=np.int64)] = 1
    ss = None if slice_starts is None else np.ascontiguousarray(np.asarray(slice_starts, dtype=np.int32))
    return int(lib().dsv41_oracle_full_draw(_ptr(z), ctypes.c_int(z.shape[0]), _ptr(counts), _ptr(ss),
                                            ctypes.c_int(0 if ss is None else ss.size), ctypes.c_uint32(U)))


def full_total(z, *, history_ids=None, slice_starts=None) -> int:
    """The exact total S of the full-vocabulary draw's 2^-43 masses over processed logits
    ``z``: every full-vocabulary draw reports lp = (z_tok - max z) - log(S 2^-43)."""
    z = np.ascontiguousarray(np.asarray(z, dtype=np.float32))
    counts = None
    if history_ids is not None:
        counts = np.zeros(z.shape[0], np.uint32)
        counts[np.asarray(history_ids, dtype=np.int64)] = 1
    ss = None if slice_starts is None else np.ascontiguousarray(np.asarray(slice_starts, dtype=np.int32))
    return int(lib().dsv41_oracle_full_total(_ptr(z), ctypes.c_int(z.shape[0]), _ptr(counts), _ptr(ss),
                                             ctypes.c_int(0 if ss is None else ss.size)))


def check_division(temperature: float, lo: int, hi: int) -> tuple[int, int]:
    first = ctypes.c_uint32(0)
    n = lib().dsv41_check_division(temperature, lo, hi, ctypes.byref(first))
    return int(n), int(first.value)


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def sample(logits, *, temperature=1.0, uniforms=None, history=None, history_lens=None,
           repetition_penalty=1.0, presence_penalty=0.0, frequency_penalty=0.0, top_k=0,
           top_p=1.0, min_p=0.0, greedy=False, history_prompt_lens=None, slice_starts=None):
    """Oracle sampler over fp32 logits [rows, V] (bf16 callers widen exactly first).
    ``history_prompt_lens[r]`` leading history entries of row r are prompt ids (repetition
    penalty only; frequency and presence count the rest).  ``slice_starts`` (ascending,
    starting at 0): the vocabulary slices of a sharded full-vocabulary draw, whose 256-id
    mass chunks restart at each slice start; None is one slice.

    Returns numpy (ids int64, logprobs fp32, kept int32, status int32).
    """
    x = np.ascontiguousarray(np.asarray(logits, dtype=np.float32))
    rows, vocab = x.shape
    u = None if uniforms is None else np.ascontiguousarray(np.asarray(uniforms, dtype=np.float32))
    h = None if history is None else np.ascontiguousarray(np.asarray(history, dtype=np.int64))
    hl = None if history_lens is None else np.ascontiguousarray(np.asarray(history_lens, dtype=np.int32))
    pl = None if history_prompt_lens is None else np.ascontiguousarray(np.asarray(history_prompt_lens, dtype=np.int32))
    ss = None if slice_starts is None else np.ascontiguousarray(np.asarray(slice_starts, dtype=np.int32))
    if ss is not None and (ss.ndim != 1 or ss.size == 0 or ss[0] != 0 or np.any(np.diff(ss) <= 0)):
        raise ValueError("slice_starts must ascend from 0")
    ids = np.empty(rows, np.int64)
    lps = np.empty(rows, np.float32)
    kept = np.empty(rows, np.int32)
    status = np.empty(rows, np.int32)
    c = lib()
    rc = c.dsv41_oracle_sample(
        _ptr(x), ctypes.c_int(rows), ctypes.c_int(vocab), _ptr(h),
        ctypes.c_int64(0 if h is None else h.shape[1]), ctypes.c_int(0 if h is None else h.shape[1]),
        _ptr(hl), _ptr(pl), _ptr(u), ctypes.c_float(temperature), ctypes.c_float(repetition_penalty),
        ctypes.c_float(presence_penalty), ctypes.c_float(frequency_penalty), ctypes.c_int(top_k),
        ctypes.c_float(top_p), ctypes.c_float(min_p), ctypes.c_int(1 if greedy else 0), _ptr(ids),
        _ptr(lps), _ptr(kept), _ptr(status), _ptr(ss), ctypes.c_int(0 if ss is None else ss.size))
    if rc != 0:
        raise MemoryError("oracle scratch allocation failed")
    return ids, lps, kept, status
