"""Decoupled Token-TIS and GRPO losses on MI355X: the drop-ins for ``decoupled_token_tis_loss``
and ``grpo_loss``.

Reference (paths relative to the Tiny-DSV41 tree):

* ``dsv41_train/rl/algorithm.py:249-346`` — ``decoupled_token_tis_loss(policy_log_probs,
  native_old_log_probs, behavior_log_probs, advantages, clip_eps=0.2, is_cap=2.0)``: the
  loss ``mean_r(-mean_i(w * min(r A, clamp(r) A)))`` with detached weights
  ``w = f32(min(cap, exp(f64(old - behavior))))`` and ``r = exp(current - old)``, plus a
  metric dict; its argument checks and ``ValueError`` messages (``:268-312``).
* ``dsv41_train/rl/algorithm.py:169-246`` — ``grpo_loss(policy_log_probs, behavior_log_probs,
  advantages, clip_eps=0.2, ref_log_probs=None, kl_beta=0.0)``: the mean over responses of
  ``-mean(min(r A, clamp(r) A))`` plus ``kl_beta`` times the mean of the importance-weighted
  k3 KL, with its metric dict and checks.
* ``dsv41_train/rl/distributed_grpo.py:197-222`` — ``aggregate_token_tis_metrics``, the
  pooling of per-response metric rows; one call here over many responses returns the pooled
  values directly.

libdsv41hip.so computes the loss, its gradient with respect to ``current`` and every metric
in two launches with fixed reduction orders; the metrics come back in one host copy
(the reference takes one per metric).  ``current`` stays differentiable.
"""

from __future__ import annotations

import ctypes
import math
from typing import Sequence

import torch

from . import _lib

METRIC_KEYS = (
    "loss", "policy_loss", "response_count", "token_count", "is_cap", "is_weight_sum",
    "is_weight_square_sum", "is_weight_mean", "is_weight_min", "is_weight_max", "is_raw_weight_sum",
    "is_raw_weight_min", "is_raw_weight_max", "is_clipped_tokens", "is_clipped_fraction",
    "is_dropped_weight_mass", "is_dropped_weight_mass_fraction", "is_token_weight_ess",
    "is_token_weight_ess_fraction", "native_old_minus_behavior_mean", "native_old_minus_behavior_max_abs",
    "native_ppo_ratio_mean", "native_ppo_clip_fraction",
)

# per-response status bits (include/dsv41_rocm.h) in the reference's check order, with its messages
_CHECKS = (
    (0x1, "policy log probabilities contains non-finite values"),
    (0x2, "policy log probabilities must be nonpositive"),
    (0x4, "native-old log probabilities contains non-finite values"),
    (0x8, "native-old log probabilities must be nonpositive"),
    (0x10, "behavior log probabilities contains non-finite values"),
    (0x20, "behavior log probabilities must be nonpositive"),
    (0x40, "raw rollout importance weights contains non-finite values"),
    (0x80, "raw rollout importance weights underflowed"),
    (0x100, "training rollout importance weights contains non-finite values"),
    (0x200, "training rollout importance weights underflowed"),
    (0x400, "native PPO ratios contains non-finite values"),
    (0x800, "native PPO ratios underflowed"),
    (0x1000, "each policy log-probability tensor must be a nonempty vector"),
    (0x2000, "advantages contains non-finite values"),
    (0x4000, "response offsets must be nondecreasing and within the token count"),
)


def _run(current, old, behavior, advantages, offsets, clip_eps, is_cap, want_grad):
    R = advantages.numel()
    dev = current.device
    loss = torch.empty(1, dtype=torch.float32, device=dev)
    grad = torch.empty_like(current) if want_grad else None
    metrics = torch.empty(len(METRIC_KEYS), dtype=torch.float64, device=dev)
    status = torch.empty(R, dtype=torch.int32, device=dev)
    d = _lib.TokenTisDesc()
    d.struct_size = ctypes.sizeof(_lib.TokenTisDesc)
    d.n_responses, d.n_tokens = R, current.numel()
    d.offsets = offsets.data_ptr()
    d.current, d.native_old, d.behavior = current.data_ptr(), old.data_ptr(), behavior.data_ptr()
    d.advantages = advantages.data_ptr()
    d.clip_eps, d.is_cap = clip_eps, is_cap
    d.out_loss, d.out_metrics, d.out_status = loss.data_ptr(), metrics.data_ptr(), status.data_ptr()
    d.out_grad = grad.data_ptr() if grad is not None else None
    lib = _lib.load()
    ws_bytes = lib.dsv41_token_tis_workspace_bytes(ctypes.byref(d))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        rc = lib.dsv41_token_tis_run(ctypes.byref(d), ws.data_ptr(), ws_bytes, torch.cuda.current_stream(dev).cuda_stream)
    _lib.check(rc)
    return loss[0], grad, metrics, status


class _TokenTIS(torch.autograd.Function):
    @staticmethod
    def forward(ctx, current, old, behavior, advantages, offsets, clip_eps, is_cap):
        loss, grad, metrics, status = _run(current, old, behavior, advantages, offsets, clip_eps, is_cap, True)
        ctx.save_for_backward(grad)
        ctx.mark_non_differentiable(metrics, status)
        return loss, metrics, status

    @staticmethod
    def backward(ctx, g_loss, g_metrics, g_status):
        (grad,) = ctx.saved_tensors
        return grad * g_loss, None, None, None, None, None, None


def decoupled_token_tis_loss(
    policy_log_probs: Sequence[torch.Tensor],
    native_old_log_probs: Sequence,
    behavior_log_probs: Sequence,
    advantages,
    clip_eps: float = 0.2,
    is_cap: float = 2.0,
) -> tuple[torch.Tensor, dict[str, float]]:
    """Same arguments, checks, loss and metric dict as algorithm.py:249-346; the per-token
    work runs on the GPU holding ``policy_log_probs``."""
    if not math.isfinite(clip_eps) or not 0 <= clip_eps < 1:
        raise ValueError("clip_eps must be finite and in [0, 1)")
    if not math.isfinite(is_cap) or is_cap <= 0:
        raise ValueError("is_cap must be finite and positive")
    size = len(policy_log_probs)
    if size == 0 or len(native_old_log_probs) != size or len(behavior_log_probs) != size:
        raise ValueError("current, native-old and behavior require the same nonzero response count")
    advantage_values = torch.as_tensor(advantages, dtype=torch.float32).detach()
    if advantage_values.ndim != 1 or len(advantage_values) != size:
        raise ValueError("one scalar advantage is required per response")
    if not bool(torch.isfinite(advantage_values).all()):
        raise ValueError("advantages contains non-finite values")
    currents, olds, behaviors, lengths = [], [], [], []
    for index, current in enumerate(policy_log_probs):
        if not isinstance(current, torch.Tensor) or current.ndim != 1 or current.numel() == 0:
            raise ValueError("each policy log-probability tensor must be a nonempty vector")
        current = current.float()
        old = torch.as_tensor(native_old_log_probs[index], dtype=torch.float32, device=current.device).detach()
        behavior = torch.as_tensor(behavior_log_probs[index], dtype=torch.float32, device=current.device).detach()
        if old.shape != current.shape or behavior.shape != current.shape:
            raise ValueError("native-old, behavior and policy response lengths must match")
        currents.append(current)
        olds.append(old)
        behaviors.append(behavior)
        lengths.append(current.numel())
    dev = currents[0].device
    if dev.type != "cuda":
        raise ValueError("log probabilities must be on the GPU (libdsv41hip has no CPU path)")
    offsets = torch.zeros(size + 1, dtype=torch.int64)
    offsets[1:] = torch.cumsum(torch.tensor(lengths, dtype=torch.int64), 0)
    cur = torch.cat(currents)
    old = torch.cat(olds).contiguous()
    beh = torch.cat(behaviors).contiguous()
    adv = advantage_values.to(dev).contiguous()
    offsets = offsets.to(dev)
    if torch.is_grad_enabled() and cur.requires_grad:
        loss, metrics, status = _TokenTIS.apply(cur.contiguous(), old, beh, adv, offsets, clip_eps, is_cap)
    else:
        loss, _, metrics, status = _run(cur.detach().contiguous(), old, beh, adv, offsets, clip_eps, is_cap, False)
    host = torch.cat([metrics, status.double()]).cpu()  # the one host copy
    values, st = host[:len(METRIC_KEYS)].tolist(), [int(v) for v in host[len(METRIC_KEYS):].tolist()]
    for bits in st:
        if bits:
            for bit, message in _CHECKS:
                if bits & bit:
                    raise ValueError(message)
    m = dict(zip(METRIC_KEYS, values))
    if not math.isfinite(m["loss"]):
        raise ValueError("Token-TIS loss contains non-finite values")
    if not math.isfinite(m["is_raw_weight_sum"]):
        raise ValueError("summed raw rollout importance weights contains non-finite values")
    if not math.isfinite(m["is_token_weight_ess"]):
        raise ValueError("token weight ESS contains non-finite values")
    m["is_cap"] = float(is_cap)
    return loss, m


GRPO_METRIC_KEYS = ("loss", "policy_loss", "kl", "clip_fraction", "importance_ratio", "approx_kl")

_GRPO_CHECKS = (
    (0x1, "policy log probabilities contains non-finite values"),
    (0x2, "behavior log probabilities contains non-finite values"),
    (0x4, "importance ratios (reduce policy lag or learning rate) contains non-finite values"),
    (0x8, "reference log probabilities contains non-finite values"),
    (0x10, "importance-weighted reference KL contains non-finite values"),
    (0x20, "each policy log-probability tensor must be a nonempty vector"),
    (0x40, "advantages contains non-finite values"),
    (0x80, "response offsets must be nondecreasing and within the token count"),
)


def _run_grpo(current, behavior, reference, advantages, offsets, clip_eps, kl_beta, want_grad):
    R = advantages.numel()
    dev = current.device
    loss = torch.empty(1, dtype=torch.float32, device=dev)
    grad = torch.empty_like(current) if want_grad else None
    metrics = torch.empty(len(GRPO_METRIC_KEYS), dtype=torch.float64, device=dev)
    status = torch.empty(R, dtype=torch.int32, device=dev)
    d = _lib.GrpoDesc()
    d.struct_size = ctypes.sizeof(_lib.GrpoDesc)
    d.n_responses, d.n_tokens = R, current.numel()
    d.offsets = offsets.data_ptr()
    d.current, d.behavior = current.data_ptr(), behavior.data_ptr()
    d.reference = reference.data_ptr() if reference is not None else None
    d.advantages = advantages.data_ptr()
    d.clip_eps, d.kl_beta = clip_eps, kl_beta
    d.out_loss, d.out_metrics, d.out_status = loss.data_ptr(), metrics.data_ptr(), status.data_ptr()
    d.out_grad = grad.data_ptr() if grad is not None else None
    lib = _lib.load()
    ws_bytes = lib.dsv41_grpo_workspace_bytes(ctypes.byref(d))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        rc = lib.dsv41_grpo_run(ctypes.byref(d), ws.data_ptr(), ws_bytes, torch.cuda.current_stream(dev).cuda_stream)
    _lib.check(rc)
    return loss[0], grad, metrics, status


class _Grpo(torch.autograd.Function):
    @staticmethod
    def forward(ctx, current, behavior, reference, advantages, offsets, clip_eps, kl_beta):
        loss, grad, metrics, status = _run_grpo(current, behavior, reference, advantages, offsets, clip_eps,
                                                kl_beta, True)
        ctx.save_for_backward(grad)
        ctx.mark_non_differentiable(metrics, status)
        return loss, metrics, status

    @staticmethod
    def backward(ctx, g_loss, g_metrics, g_status):
        (grad,) = ctx.saved_tensors
        return grad * g_loss, None, None, None, None, None, None


def grpo_loss(
    policy_log_probs: Sequence[torch.Tensor],
    behavior_log_probs: Sequence,
    advantages,
    clip_eps: float = 0.2,
    ref_log_probs: Sequence | None = None,
    kl_beta: float = 0.0,
) -> tuple[torch.Tensor, dict[str, float]]:
    """Same arguments, checks, loss and metric dict as algorithm.py:169-246; the per-token
    work runs on the GPU holding ``policy_log_probs``."""
    if not math.isfinite(clip_eps) or not 0 <= clip_eps < 1:
        raise ValueError("clip_eps must be finite and in [0, 1)")
    if not math.isfinite(kl_beta) or kl_beta < 0:
        raise ValueError("kl_beta must be finite and nonnegative")
    size = len(policy_log_probs)
    if size == 0 or len(behavior_log_probs) != size:
        raise ValueError("policy and behavior must contain the same nonzero number of responses")
    advantage_values = torch.as_tensor(advantages, dtype=torch.float32).detach()
    if advantage_values.ndim != 1 or len(advantage_values) != size:
        raise ValueError("one scalar advantage is required per response")
    if not bool(torch.isfinite(advantage_values).all()):
        raise ValueError("advantages contains non-finite values")
    if ref_log_probs is not None and len(ref_log_probs) != size:
        raise ValueError("one reference log-probability vector is required per response")
    if kl_beta and ref_log_probs is None:
        raise ValueError("positive kl_beta requires reference log probabilities")
    currents, behaviors, references, lengths = [], [], [], []
    for index, current in enumerate(policy_log_probs):
        if current.ndim != 1 or current.numel() == 0:
            raise ValueError("each policy log-probability tensor must be a nonempty vector")
        current = current.float()
        behavior = torch.as_tensor(behavior_log_probs[index], dtype=torch.float32, device=current.device).detach()
        if behavior.shape != current.shape:
            raise ValueError("behavior and policy response lengths must match")
        if kl_beta:
            reference = ref_log_probs[index].to(device=current.device, dtype=torch.float32).detach()
            if reference.shape != current.shape:
                raise ValueError("reference and policy response lengths must match")
            references.append(reference)
        currents.append(current)
        behaviors.append(behavior)
        lengths.append(current.numel())
    dev = currents[0].device
    if dev.type != "cuda":
        raise ValueError("log probabilities must be on the GPU (libdsv41hip has no CPU path)")
    offsets = torch.zeros(size + 1, dtype=torch.int64)
    offsets[1:] = torch.cumsum(torch.tensor(lengths, dtype=torch.int64), 0)
    cur = torch.cat(currents)
    beh = torch.cat(behaviors).contiguous()
    ref = torch.cat(references).contiguous() if kl_beta else None
    adv = advantage_values.to(dev).contiguous()
    offsets = offsets.to(dev)
    if torch.is_grad_enabled() and cur.requires_grad:
        loss, metrics, status = _Grpo.apply(cur.contiguous(), beh, ref, adv, offsets, clip_eps, kl_beta)
    else:
        loss, _, metrics, status = _run_grpo(cur.detach().contiguous(), beh, ref, adv, offsets, clip_eps, kl_beta,
                                             False)
    host = torch.cat([metrics, status.double()]).cpu()
    values, st = host[:len(GRPO_METRIC_KEYS)].tolist(), [int(v) for v in host[len(GRPO_METRIC_KEYS):].tolist()]
    for bits in st:
        if bits:
            for bit, message in _GRPO_CHECKS:
                if bits & bit:
                    raise ValueError(message)
    m = dict(zip(GRPO_METRIC_KEYS, values))
    if not math.isfinite(m["loss"]):
        raise ValueError("GRPO loss contains non-finite values")
    return loss, m
