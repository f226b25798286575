"""The autoregressive decode loop with its sampling step on the GPU: the drop-in for the
per-token loop of ``generate_group`` (``dsv41_train/rl/rollout.py:124-157``).

The reference evaluates ``log_softmax(logits.float() / T)`` on the model device, copies the
whole probability row to the host (``.exp().cpu()``, 4V bytes per token) and draws with
``torch.multinomial`` on one CPU thread.  Here the row stays on the GPU: libdsv41hip.so
draws the token and its behaviour log-prob, and two scalars come back.

``draw="exponential_race"`` consumes the CPU generator exactly as the reference does (V
``exponential_`` variates per token) and draws the same token, so a run seeded like the
reference's (``rollout_manager/backends/pytorch_rl.py:70-72``) replays its samples and leaves
the generator state that the reference checkpoints (``rl/checkpoint.py:207-222``).
``draw="inverse_cdf"`` uses one uniform per token instead (no V-sized host work at all).

The model contract, the EOS / stop-sequence rules, the finish reasons and the error
messages are the reference's; building ``Sample`` / ``RolloutGroup`` records and rewards is
left to the caller.
"""

from __future__ import annotations

from typing import Optional, Sequence

import torch

from .sampling import sample_next, validate_temperature


def _token_ids(value, name, allow_empty=False) -> list[int]:
    """Same rules and messages as validate_token_ids (dsv41_train/rl/data.py:14-21)."""
    if not isinstance(value, (list, tuple)):
        raise ValueError(f"{name} must be a list of nonnegative integer token IDs")
    if not value and not allow_empty:
        raise ValueError(f"{name} must not be empty")
    if any(isinstance(token, bool) or not isinstance(token, int) or token < 0 for token in value):
        raise ValueError(f"{name} must contain only nonnegative integer token IDs")
    return list(value)


def _input_device(model) -> torch.device:
    parameter = next(model.parameters(), None) if hasattr(model, "parameters") else None
    if parameter is not None:
        return parameter.device
    buffer = next(model.buffers(), None) if hasattr(model, "buffers") else None
    return buffer.device if buffer is not None else torch.device("cpu")


def _next_logits(model, tokens: torch.Tensor) -> torch.Tensor:
    """rollout.py:128-141: the next_token_logits hook ([1, V]) or the last row of forward."""
    hook = getattr(model, "next_token_logits", None)
    if hook is None:
        out = model(tokens, attention_mask=torch.ones_like(tokens))
        logits = out if isinstance(out, torch.Tensor) else out.logits
        if logits.ndim != 3 or logits.shape[0] != 1 or logits.shape[1] == 0 or logits.shape[2] == 0:
            raise ValueError("model logits must have shape [1, sequence_length, vocabulary_size]")
        if logits.shape[1] != tokens.shape[1]:
            raise ValueError("model must return one logits vector per input token")
        return logits[0, -1]
    if not callable(hook):
        raise ValueError("model next_token_logits hook must be callable")
    logits = hook(tokens, attention_mask=torch.ones_like(tokens))
    if not isinstance(logits, torch.Tensor) or logits.ndim != 2 or logits.shape[0] != 1 or logits.shape[1] == 0:
        raise ValueError("model next_token_logits must return [1, vocabulary_size]")
    return logits[0]


def generate_response(
    model,
    prompt_ids: Sequence[int],
    max_new_tokens: int,
    temperature: float,
    eos_token_id: Optional[int | Sequence[int]] = None,
    stop_token_sequences: Sequence[Sequence[int]] = (),
    generator: Optional[torch.Generator] = None,
    draw: str = "exponential_race",
) -> tuple[list[int], list[float], str, int]:
    """One response: ``(response_ids, behavior_log_probs, finish_reason, stop_token_count)``
    with the reference's semantics (stop tokens stay in the response; finish reason "stop",
    "eos" or "length")."""
    validate_temperature(temperature)
    if isinstance(max_new_tokens, bool) or not isinstance(max_new_tokens, int) or max_new_tokens <= 0:
        raise ValueError("max_new_tokens must be a positive integer")
    if generator is not None and generator.device.type != "cpu":
        raise ValueError("generation requires a CPU torch.Generator")
    prompt = _token_ids(prompt_ids, "prompt_ids")
    eos_ids = [] if eos_token_id is None else _token_ids(
        [eos_token_id] if isinstance(eos_token_id, int) else eos_token_id, "eos_token_id", allow_empty=True)
    stops = sorted((_token_ids(ids, "stop_token_sequences") for ids in stop_token_sequences), key=len, reverse=True)
    device = _input_device(model)
    response: list[int] = []
    behavior: list[float] = []
    finish_reason, stop_count = "length", 0
    with torch.inference_mode():
        for _ in range(max_new_tokens):
            tokens = torch.tensor([prompt + response], dtype=torch.long, device=device)
            logits = _next_logits(model, tokens)
            if any(t >= logits.shape[-1] for t in eos_ids + [t for ids in stops for t in ids]):
                raise ValueError("stop token ID is outside the model vocabulary")
            token, lp = sample_next(logits, temperature, generator=generator, draw=draw)
            response.append(token)
            behavior.append(lp)
            matched = next((ids for ids in stops if response[-len(ids):] == ids), None)
            if matched is not None:
                finish_reason, stop_count = "stop", len(matched)
                break
            if token in eos_ids:
                finish_reason, stop_count = "eos", 1
                break
    return response, behavior, finish_reason, stop_count


def generate_group_responses(model, prompt_ids, group_size: int, max_new_tokens: int, temperature: float,
                             eos_token_id=None, stop_token_sequences=(), generator=None,
                             draw: str = "exponential_race") -> list[tuple[list[int], list[float], str, int]]:
    """``group_size`` responses drawn one after another from one generator, in the order the
    reference draws them (rollout.py:124), so the random stream is consumed identically."""
    if isinstance(group_size, bool) or not isinstance(group_size, int) or group_size <= 0:
        raise ValueError("group_size must be a positive integer")
    was_training = getattr(model, "training", False)
    if hasattr(model, "eval"):
        model.eval()
    try:
        return [generate_response(model, prompt_ids, max_new_tokens, temperature, eos_token_id,
                                  stop_token_sequences, generator, draw) for _ in range(group_size)]
    finally:
        if hasattr(model, "train"):
            model.train(was_training)
