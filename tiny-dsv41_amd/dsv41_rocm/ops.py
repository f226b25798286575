"""torch.library custom ops over libdsv41hip.so, in the reference's operator idiom
(``torch.library.custom_op(..., mutates_args=(), device_types="cuda")`` plus
``register_fake``, dsv41_train/models/dsv4/moe/kernels.py:236-281).

* ``dsv41_rocm::sample_rows`` — the row sampler; returns ``(ids, logprobs, kept, status)``.
* ``dsv41_rocm::selected_log_probs`` — the fused log-prob head; returns
  ``(logprob, entropy, ratio, lse)`` with an empty ``ratio`` when no behaviour log-probs are
  given.  Differentiable in ``hidden`` and ``weight`` through ``register_autograd`` (the
  reference registers its Triton ops' backward the same way, moe/kernels.py:283-307);
  ``ratio`` and ``lse`` carry no gradient.

The ops only register a CUDA (HIP) kernel: called on CPU tensors they raise, as the library
has no CPU path.  Status bits are returned, not raised, so the ops stay traceable; the
Python wrappers in ``sampling`` and ``logprob`` raise the reference's errors.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import logprob as _logprob
from . import sampling as _sampling


@torch.library.custom_op("dsv41_rocm::sample_rows", mutates_args=(), device_types="cuda")
def sample_rows(
    logits: torch.Tensor,
    uniforms: Optional[torch.Tensor],
    history: Optional[torch.Tensor],
    history_lens: Optional[torch.Tensor],
    temperature: float,
    repetition_penalty: float,
    presence_penalty: float,
    frequency_penalty: float,
    top_k: int,
    top_p: float,
    min_p: float,
    greedy: bool,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    if not greedy and uniforms is None:
        raise ValueError("sampling requires one uniform per row")
    r = _sampling.sample(logits, temperature=temperature, uniforms=uniforms, history=history,
                         history_lens=history_lens, repetition_penalty=repetition_penalty,
                         presence_penalty=presence_penalty, frequency_penalty=frequency_penalty,
                         top_k=top_k, top_p=top_p, min_p=min_p, greedy=greedy, check=False)
    return r.ids, r.logprobs, r.kept, r.status


@sample_rows.register_fake
def _sample_rows_fake(logits, uniforms, history, history_lens, temperature, repetition_penalty,
                      presence_penalty, frequency_penalty, top_k, top_p, min_p, greedy):
    rows = logits.shape[0]
    dev = logits.device
    return (torch.empty(rows, dtype=torch.int64, device=dev),
            torch.empty(rows, dtype=torch.float32, device=dev),
            torch.empty(rows, dtype=torch.int32, device=dev),
            torch.empty(rows, dtype=torch.int32, device=dev))


@torch.library.custom_op("dsv41_rocm::selected_log_probs", mutates_args=(), device_types="cuda")
def selected_log_probs_op(
    hidden: torch.Tensor,
    weight: torch.Tensor,
    targets: torch.Tensor,
    temperature: float,
    behavior: Optional[torch.Tensor],
    is_cap: float,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    hidden, weight, targets = _logprob._prepare(hidden, weight, targets, temperature)
    lp, ent, ratio, lse, _ = _logprob._forward(hidden, weight, targets, temperature, behavior, is_cap)
    if ratio is None:
        ratio = lp.new_empty(0)
    return lp, ent, ratio, lse


@selected_log_probs_op.register_fake
def _selected_log_probs_fake(hidden, weight, targets, temperature, behavior, is_cap):
    n = hidden.shape[0]
    dev = hidden.device
    lp = torch.empty(n, dtype=torch.float32, device=dev)
    ent = torch.empty(n, dtype=torch.float32, device=dev)
    ratio = torch.empty(n if behavior is not None else 0, dtype=torch.float32, device=dev)
    lse = torch.empty(n, dtype=torch.float32, device=dev)
    return lp, ent, ratio, lse


def _selected_log_probs_setup(ctx, inputs, output):
    hidden, weight, targets, temperature, _, _ = inputs
    _, ent, _, lse = output
    ctx.temperature = temperature
    ctx.hidden_dtype, ctx.weight_dtype = hidden.dtype, weight.dtype
    ctx.save_for_backward(hidden, weight, targets, lse, ent)


def _selected_log_probs_backward(ctx, g_lp, g_ent, g_ratio, g_lse):
    hidden, weight, targets, lse, ent = ctx.saved_tensors
    h, w, t = _logprob._prepare(hidden, weight, targets, ctx.temperature)
    dx, dw = _logprob.selected_log_probs_backward(h, w, t, ctx.temperature, lse, ent, g_lp, g_ent,
                                                  need_hidden=ctx.needs_input_grad[0],
                                                  need_weight=ctx.needs_input_grad[1])
    if dx is not None:
        dx = dx.to(ctx.hidden_dtype)
    if dw is not None:
        dw = dw.to(ctx.weight_dtype)
    return dx, dw, None, None, None, None


selected_log_probs_op.register_autograd(_selected_log_probs_backward, setup_context=_selected_log_probs_setup)


__all__ = ["sample_rows", "selected_log_probs_op"]
