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

Under autograd the head is differentiable as the reference's is when the learner scores
its ``current`` phase (``dsv41_train/rl/distributed_grpo.py:352-375`` through the
checkpointed ``_score_targets``, ``native_lora.py:120-122``): the backward recomputes the
logits tile by tile and produces their gradient in bf16, then takes the two GEMMs.
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


def _prepare(hidden, weight, targets, temperature):
    if not math.isfinite(temperature) or temperature <= 0:
        raise ValueError("temperature must be finite and positive")
    if hidden.ndim != 2 or weight.ndim != 2 or hidden.shape[1] != weight.shape[1]:
        raise ValueError("hidden must be [tokens, hidden] and weight [vocab, hidden]")
    if not (hidden.is_cuda and weight.is_cuda):
        raise ValueError("hidden and weight must be on the GPU (libdsv41hip has no CPU path)")
    n, h = hidden.shape
    v = weight.shape[0]
    targets = targets.to(device=hidden.device, dtype=torch.int64).reshape(-1)
    if targets.numel() != n:
        raise ValueError("one target is required per token")
    if n and bool(((targets < 0) | (targets >= v)).any()):
        raise ValueError("target token ID is outside the model vocabulary")
    if h % 8:
        raise ValueError("hidden size must be a multiple of 8")
    hidden = hidden.to(torch.bfloat16)
    weight = weight.to(torch.bfloat16)
    if hidden.stride(1) != 1 or hidden.stride(0) % 8 or hidden.data_ptr() % 16:
        hidden = hidden.contiguous()
    if weight.stride(1) != 1 or weight.stride(0) % 8 or weight.data_ptr() % 16:
        weight = weight.contiguous()
    return hidden, weight, targets.contiguous()


def _forward(hidden, weight, targets, temperature, behavior, is_cap):
    """One launch of dsv41_logprob_run; returns (logprob, entropy, ratio or None, lse, status)."""
    n, h = hidden.shape
    v = weight.shape[0]
    device = hidden.device
    lp = torch.empty(n, dtype=torch.float32, device=device)
    ent = torch.empty(n, dtype=torch.float32, device=device)
    lse = torch.empty(n, dtype=torch.float32, device=device)
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
    d.out_lse = lse.data_ptr()
    lib = _lib.load()
    ws_bytes = lib.dsv41_logprob_workspace_bytes(ctypes.byref(d))
    workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device)
    with torch.cuda.device(device):
        stream = torch.cuda.current_stream(device).cuda_stream
        rc = lib.dsv41_logprob_run(ctypes.byref(d), workspace.data_ptr(), ws_bytes, stream)
    _lib.check(rc)
    return lp, ent, ratio, lse, status


def logits_grad(hidden: torch.Tensor, weight: torch.Tensor, targets: torch.Tensor, temperature: float,
                lse: torch.Tensor, entropy: Optional[torch.Tensor], grad_logprob: Optional[torch.Tensor],
                grad_entropy: Optional[torch.Tensor], vocab_begin: int = 0,
                vocab_end: Optional[int] = None) -> torch.Tensor:
    """Gradient with respect to the logits ``hidden @ weight[vocab_begin:vocab_end].T`` of a loss
    whose gradients with respect to the outputs of ``selected_log_probs`` are ``grad_logprob``
    and ``grad_entropy`` (None = zero), as bf16 ``[N, vocab_end - vocab_begin]``: the dtype of
    the reference's ``lm_head`` output, whose autograd gradient it is (model.py:682).

    ``hidden``, ``weight`` and ``targets`` must already be in kernel form (bf16, 16-byte
    aligned rows; see ``_prepare``); ``lse`` and ``entropy`` come from the forward.
    """
    n, h = hidden.shape
    v = weight.shape[0]
    vocab_end = v if vocab_end is None else vocab_end
    width = vocab_end - vocab_begin
    stride = (width + 7) // 8 * 8
    out = torch.empty(n, stride, dtype=torch.bfloat16, device=hidden.device)
    f32 = lambda t: None if t is None else t.to(device=hidden.device, dtype=torch.float32).reshape(-1).contiguous()
    lse, entropy, grad_logprob, grad_entropy = f32(lse), f32(entropy), f32(grad_logprob), f32(grad_entropy)
    d = _lib.LogprobGradDesc()
    d.struct_size = ctypes.sizeof(_lib.LogprobGradDesc)
    d.n_tokens, d.hidden, d.vocab = n, h, v
    d.x, d.x_row_stride = hidden.data_ptr(), hidden.stride(0)
    d.w, d.w_row_stride = weight.data_ptr(), weight.stride(0)
    d.targets = targets.data_ptr()
    d.temperature = temperature
    ptr = lambda t: None if t is None else t.data_ptr()
    d.lse, d.entropy = ptr(lse), ptr(entropy)
    d.grad_logprob, d.grad_entropy = ptr(grad_logprob), ptr(grad_entropy)
    d.vocab_begin, d.vocab_end = vocab_begin, vocab_end
    d.out, d.out_row_stride = out.data_ptr(), stride
    lib = _lib.load()
    with torch.cuda.device(hidden.device):
        stream = torch.cuda.current_stream(hidden.device).cuda_stream
        rc = lib.dsv41_logprob_grad_run(ctypes.byref(d), stream)
    _lib.check(rc)
    return out[:, :width]


# Largest bf16 logit-gradient block the backward materialises at once (bytes); the
# vocabulary is processed in ranges that fit.  1 GiB is about the fp32 logits of one
# 2048-token chunk of the reference's scoring head (native_lora.py:76-77: 2048 x 129280 x 4 B
# = 1.06 GB); at 16384 tokens x 129280 rows it takes four ranges of 32768 rows.
GRAD_BLOCK_BYTES = 1 << 30


def selected_log_probs_backward(hidden, weight, targets, temperature, lse, entropy, grad_logprob,
                                grad_entropy, need_hidden=True, need_weight=True, vocab_chunk=None):
    """dL/dhidden and dL/dweight (bf16, or None when not needed) of the fused log-prob.

    The logit gradient comes from ``dsv41_logprob_grad_run`` (recomputed logits on the
    matrix cores, bf16 like the reference's ``lm_head`` output gradient); the two products
    with it are plain GEMMs (hipBLASLt through torch), as in the reference's ``nn.Linear``
    backward.  Vocabulary ranges of ``vocab_chunk`` rows (default: as many as
    ``GRAD_BLOCK_BYTES`` allows) bound the logit gradient held at once.
    """
    n, _ = hidden.shape
    v = weight.shape[0]
    if vocab_chunk is None:
        vocab_chunk = max(256, GRAD_BLOCK_BYTES // max(1, 2 * n) // 256 * 256)
    ranges = [(b, min(v, b + vocab_chunk)) for b in range(0, v, vocab_chunk)]
    dx = None
    dw = torch.empty_like(weight) if need_weight else None
    for b, e in ranges:
        g = logits_grad(hidden, weight, targets, temperature, lse, entropy, grad_logprob, grad_entropy, b, e)
        if need_hidden:
            part = torch.mm(g, weight[b:e])
            if len(ranges) == 1:
                dx = part
            else:
                dx = part.float() if dx is None else dx.add_(part.float())
        if need_weight:
            torch.mm(g.t(), hidden, out=dw[b:e])
    if dx is not None:
        dx = dx.to(hidden.dtype)
    return dx, dw


class _SelectedLogProbs(torch.autograd.Function):
    """Differentiable fused log-prob: forward = dsv41_logprob_run, backward =
    dsv41_logprob_grad_run + two GEMMs.  The Token-TIS weight carries no gradient (the
    reference computes it from detached old log-probs, algorithm.py:293-299)."""

    @staticmethod
    def forward(ctx, hidden, weight, targets, temperature, behavior, is_cap):
        lp, ent, ratio, lse, status = _forward(hidden, weight, targets, temperature, behavior, is_cap)
        ctx.temperature = temperature
        ctx.save_for_backward(hidden, weight, targets, lse, ent)
        if ratio is None:
            ratio = lp.new_empty(0)
        ctx.mark_non_differentiable(ratio, status)
        return lp, ent, ratio, status

    @staticmethod
    def backward(ctx, g_lp, g_ent, g_ratio, g_status):
        hidden, weight, targets, lse, ent = ctx.saved_tensors
        dx, dw = selected_log_probs_backward(hidden, weight, targets, ctx.temperature, lse, ent, g_lp, g_ent,
                                             need_hidden=ctx.needs_input_grad[0],
                                             need_weight=ctx.needs_input_grad[1])
        return dx, dw, None, None, None, None


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
    Returns fp32 tensors ``(logprob [N], entropy [N], ratio [N] or None)``.  Differentiable
    in ``hidden`` and ``weight`` (log-prob and entropy), like the reference expression under
    autograd.
    """
    hidden, weight, targets = _prepare(hidden, weight, targets, temperature)
    if torch.is_grad_enabled() and (hidden.requires_grad or weight.requires_grad):
        lp, ent, ratio, status = _SelectedLogProbs.apply(hidden, weight, targets, temperature, behavior, is_cap)
        ratio = ratio if behavior is not None else None
    else:
        lp, ent, ratio, _, status = _forward(hidden, weight, targets, temperature, behavior, is_cap)
    if check and hidden.shape[0] and bool((status != 0).any()):
        _status_error(status)
    return lp, ent, ratio


def shard_states(hidden: torch.Tensor, weight_slice: torch.Tensor, targets: torch.Tensor, temperature: float,
                 vocab_offset: int) -> torch.Tensor:
    """One GPU's part of a vocabulary-sharded head: ``weight_slice`` holds the head's rows
    ``[vocab_offset, vocab_offset + rows)``.  Returns fp32 ``[N, 4]`` states
    ``(max z, sum e, sum e*z, z_target or -inf)``, 16 bytes per token: what a tensor-parallel
    head exchanges (one all-gather) before ``combine_states``."""
    if not isinstance(vocab_offset, int) or vocab_offset < 0:
        raise ValueError("vocab_offset must be a nonnegative integer")
    if not math.isfinite(temperature) or temperature <= 0:
        raise ValueError("temperature must be finite and positive")
    if hidden.ndim != 2 or weight_slice.ndim != 2 or hidden.shape[1] != weight_slice.shape[1]:
        raise ValueError("hidden must be [tokens, hidden] and weight [vocab, hidden]")
    if not (hidden.is_cuda and weight_slice.is_cuda):
        raise ValueError("hidden and weight must be on the GPU (libdsv41hip has no CPU path)")
    n, h = hidden.shape
    if h % 8:
        raise ValueError("hidden size must be a multiple of 8")
    hidden = hidden.to(torch.bfloat16)
    weight_slice = weight_slice.to(torch.bfloat16)
    if hidden.stride(1) != 1 or hidden.stride(0) % 8 or hidden.data_ptr() % 16:
        hidden = hidden.contiguous()
    if weight_slice.stride(1) != 1 or weight_slice.stride(0) % 8 or weight_slice.data_ptr() % 16:
        weight_slice = weight_slice.contiguous()
    targets = targets.to(device=hidden.device, dtype=torch.int64).reshape(-1).contiguous()
    if targets.numel() != n:
        raise ValueError("one target is required per token")
    states = torch.empty(n, 4, dtype=torch.float32, device=hidden.device)
    d = _lib.LogprobShardDesc()
    d.struct_size = ctypes.sizeof(_lib.LogprobShardDesc)
    d.n_tokens, d.hidden, d.vocab = n, h, weight_slice.shape[0]
    d.x, d.x_row_stride = hidden.data_ptr(), hidden.stride(0)
    d.w, d.w_row_stride = weight_slice.data_ptr(), weight_slice.stride(0)
    d.targets, d.vocab_offset, d.temperature = targets.data_ptr(), vocab_offset, temperature
    d.out_state = states.data_ptr()
    lib = _lib.load()
    ws_bytes = lib.dsv41_logprob_shard_workspace_bytes(ctypes.byref(d))
    workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=hidden.device)
    with torch.cuda.device(hidden.device):
        rc = lib.dsv41_logprob_shard_run(ctypes.byref(d), workspace.data_ptr(), ws_bytes,
                                         torch.cuda.current_stream(hidden.device).cuda_stream)
    _lib.check(rc)
    return states


def combine_states(states: torch.Tensor, *, behavior: Optional[torch.Tensor] = None, is_cap: float = 2.0,
                   check: bool = True) -> tuple[torch.Tensor, torch.Tensor, Optional[torch.Tensor]]:
    """Exact combine of gathered shard states ``[shards, N, 4]`` into ``(logprob, entropy,
    ratio or None)``, the outputs ``selected_log_probs`` gives for the unsharded head."""
    if states.ndim != 3 or states.shape[2] != 4 or not states.is_cuda:
        raise ValueError("states must be a GPU tensor of shape [shards, tokens, 4]")
    states = states.to(torch.float32).contiguous()
    g, n, _ = states.shape
    dev = states.device
    lp = torch.empty(n, dtype=torch.float32, device=dev)
    ent = torch.empty(n, dtype=torch.float32, device=dev)
    status = torch.empty(n, dtype=torch.int32, device=dev)
    ratio = None
    d = _lib.LogprobCombineDesc()
    d.struct_size = ctypes.sizeof(_lib.LogprobCombineDesc)
    d.n_tokens, d.n_shards, d.states = n, g, states.data_ptr()
    if behavior is not None:
        behavior = behavior.to(device=dev, dtype=torch.float32).reshape(-1).contiguous()
        ratio = torch.empty(n, dtype=torch.float32, device=dev)
        d.behavior, d.is_cap, d.out_ratio = behavior.data_ptr(), is_cap, ratio.data_ptr()
    d.out_logprob, d.out_entropy, d.out_status = lp.data_ptr(), ent.data_ptr(), status.data_ptr()
    lib = _lib.load()
    with torch.cuda.device(dev):
        rc = lib.dsv41_logprob_combine_run(ctypes.byref(d), torch.cuda.current_stream(dev).cuda_stream)
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
