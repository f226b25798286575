"""Fused selected-token log-prob on MI355X: the drop-in for the scoring head.

Reference (paths relative to the Tiny-DSV41 tree):

* ``dsv41_train/models/dsv4/model.py:679-684`` — ``_token_log_probs``:
  ``log_softmax(lm_head(hidden[mask]).float() / T).gather(targets[mask])`` scattered into
  zeros of the mask's shape; target ids are validated at ``:725-727``.
* ``dsv41_train/rl/native_lora.py:80-82`` — ``_score_targets``, the same expression on a
  chunk of selected tokens.
* ``dsv41_train/rl/algorithm.py:293-299`` — the Token-TIS weight
  ``float32(min(cap, exp(float64(old - behavior))))``.

The logits never reach HBM: libdsv41hip.so computes them tile by tile on the matrix
cores and keeps only each token's running softmax state.  Logits are accumulated in fp32
from the bf16 operands (the reference rounds ``lm_head``'s output to bf16 first).
"""

from __future__ import annotations

import ctypes
import math
from typing import Optional

import torch

from . import _lib


def _status_error(status: torch.Tensor) -> None:
    bits = 0
    for v in status.cpu().tolist():
        bits |= int(v)
    if bits & _lib.STATUS_NONFINITE:
        raise ValueError("response log probabilities contain non-finite values")
    if bits & _lib.STATUS_RATIO_ZERO:
        raise ValueError("raw rollout importance weights underflowed")


def selected_log_probs(
    hidden: torch.Tensor,
    weight: torch.Tensor,
    targets: torch.Tensor,
    temperature: float = 1.0,
    *,
    behavior: Optional[torch.Tensor] = None,
    is_cap: float = 2.0,
    check: bool = True,
) -> tuple[torch.Tensor, torch.Tensor, Optional[torch.Tensor]]:
    """Log-prob of ``targets[n]`` under ``softmax(hidden[n] @ weight.T / T)``, the entropy of
    that distribution, and (with ``behavior``) the clipped Token-TIS weight.

    ``hidden [N, H]`` and ``weight [V, H]`` are bf16 on the GPU; ``targets [N]`` int64.
    Returns fp32 tensors ``(logprob [N], entropy [N], ratio [N] or None)``.
    """
    if not math.isfinite(temperature) or temperature <= 0:
        raise ValueError("temperature must be finite and positive")
    if hidden.ndim != 2 or weight.ndim != 2 or hidden.shape[1] != weight.shape[1]:
        raise ValueError("hidden must be [tokens, hidden] and weight [vocab, hidden]")
    if not (hidden.is_cuda and weight.is_cuda):
        raise ValueError("hidden and weight must be on the GPU (libdsv41hip has no CPU path)")
    n, h = hidden.shape
    v = weight.shape[0]
    device = hidden.device
    targets = targets.to(device=device, dtype=torch.int64).reshape(-1)
    if targets.numel() != n:
        raise ValueError("one target is required per token")
    if n and bool(((targets < 0) | (targets >= v)).any()):
        raise ValueError("target token ID is outside the model vocabulary")
    hidden = hidden.to(torch.bfloat16)
    weight = weight.to(torch.bfloat16)
    if h % 8:
        raise ValueError("hidden size must be a multiple of 8")
    if hidden.stride(1) != 1 or hidden.stride(0) % 8 or hidden.data_ptr() % 16:
        hidden = hidden.contiguous()
    if weight.stride(1) != 1 or weight.stride(0) % 8 or weight.data_ptr() % 16:
        weight = weight.contiguous()
    lp = torch.empty(n, dtype=torch.float32, device=device)
    ent = torch.empty(n, dtype=torch.float32, device=device)
    ratio = None
    status = torch.empty(n, dtype=torch.int32, device=device)
    d = _lib.LogprobDesc()
    d.struct_size = ctypes.sizeof(_lib.LogprobDesc)
    d.n_tokens, d.hidden, d.vocab = n, h, v
    d.x, d.x_row_stride = hidden.data_ptr(), hidden.stride(0)
    d.w, d.w_row_stride = weight.data_ptr(), weight.stride(0)
    d.targets = targets.data_ptr()
    d.temperature = temperature
    if behavior is not None:
        behavior = behavior.to(device=device, dtype=torch.float32).reshape(-1).contiguous()
        if behavior.numel() != n:
            raise ValueError("one behavior log probability is required per token")
        if not math.isfinite(is_cap) or is_cap <= 0:
            raise ValueError("is_cap must be finite and positive")
        ratio = torch.empty(n, dtype=torch.float32, device=device)
        d.behavior = behavior.data_ptr()
        d.is_cap = is_cap
        d.out_ratio = ratio.data_ptr()
    d.out_logprob, d.out_entropy, d.out_status = lp.data_ptr(), ent.data_ptr(), status.data_ptr()
    lib = _lib.load()
    ws_bytes = lib.dsv41_logprob_workspace_bytes(ctypes.byref(d))
    workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device)
    with torch.cuda.device(device):
        stream = torch.cuda.current_stream(device).cuda_stream
        rc = lib.dsv41_logprob_run(ctypes.byref(d), workspace.data_ptr(), ws_bytes, stream)
    _lib.check(rc)
    if check and n and bool((status != 0).any()):
        _status_error(status)
    return lp, ent, ratio


def score_targets(hidden: torch.Tensor, weight: torch.Tensor, targets: torch.Tensor,
                  temperature: float) -> torch.Tensor:
    """Drop-in for native_lora.py:80-82 (``_score_targets``): fp32 log-probs [N]."""
    return selected_log_probs(hidden, weight, targets, temperature)[0]


def token_log_probs(hidden: torch.Tensor, weight: torch.Tensor, targets: torch.Tensor,
                    mask: torch.Tensor, temperature: float) -> torch.Tensor:
    """Drop-in for model.py:679-684 (``_token_log_probs``): fp32 [B, T] with the selected
    targets' log-probs where ``mask`` is set and zeros elsewhere."""
    mask = mask.to(torch.bool)
    selected = hidden[mask]
    if selected.shape[0] == 0:
        return torch.zeros(mask.shape, dtype=torch.float32, device=hidden.device)
    lp = selected_log_probs(selected, weight, targets[mask], temperature)[0]
    return lp.new_zeros(mask.shape).masked_scatter(mask, lp)
