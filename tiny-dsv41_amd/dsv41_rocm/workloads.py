"""Synthetic inputs of the five benchmark configurations (seeded, fixed draw order).

A: sampler 8 x 129280 fp32 logits 3*N(0,1), history 256, T 0.7, rp 1.1, top-k 50, top-p 0.95
   (+ a greedy pass).
B: sampler 256 x 151936 bf16 Zipf-biased logits, history 2048, T 1.0, presence 0.5,
   frequency 0.2, full-vocab draw.
C: log-prob 8192 tokens x hidden 2048 -> vocab 151936 (Qwen3-MoE head shape).
D: log-prob + Token-TIS ratio, 16384 tokens x hidden 7168 -> vocab 129280 (DeepSeek head).
E: sampler 4096 x 151936 fp32 Zipf-biased, history 4096, T 0.6, rp 1.05, top-k 1024,
   top-p 0.98, min-p 0.05.

Zipf bias: ``N(0,1) - 1.1 * log(rank)`` with ranks 1..V assigned through a per-row random
permutation.  Seed ``20261201 + index`` (A=0 ... E=4); draw order: logits, bias
permutation, history, uniforms, then the rest.  ``rows``/``tokens`` may be reduced for
parity tests; the draw order is kept so a reduced batch is a prefix-shaped sample of
the same distribution (not the same numbers).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import torch

SEED_BASE = 20261201


@dataclass
class SamplerConfig:
    name: str
    index: int
    rows: int
    vocab: int
    dtype: torch.dtype
    hist_len: int
    zipf: bool
    knobs: dict = field(default_factory=dict)


SAMPLER_CONFIGS = {
    "A": SamplerConfig("A", 0, 8, 129280, torch.float32, 256, False,
                       dict(temperature=0.7, repetition_penalty=1.1, top_k=50, top_p=0.95)),
    "B": SamplerConfig("B", 1, 256, 151936, torch.bfloat16, 2048, True,
                       dict(temperature=1.0, presence_penalty=0.5, frequency_penalty=0.2)),
    "E": SamplerConfig("E", 4, 4096, 151936, torch.float32, 4096, True,
                       dict(temperature=0.6, repetition_penalty=1.05, top_k=1024, top_p=0.98,
                            min_p=0.05)),
}


@dataclass
class LogprobConfig:
    name: str
    index: int
    tokens: int
    hidden: int
    vocab: int
    ratio: bool


LOGPROB_CONFIGS = {
    "C": LogprobConfig("C", 2, 8192, 2048, 151936, False),
    "D": LogprobConfig("D", 3, 16384, 7168, 129280, True),
}


def _gen(device, seed):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def sampler_inputs(name: str, rows: Optional[int] = None, device="cpu", seed: Optional[int] = None):
    """Returns dict(logits, history, uniforms, knobs) for sampler config A, B or E.  ``seed``
    (default: the config's own) draws other batches of the same distribution."""
    cfg = SAMPLER_CONFIGS[name]
    rows = cfg.rows if rows is None else rows
    g = _gen(device, SEED_BASE + cfg.index if seed is None else seed)
    V = cfg.vocab
    if cfg.zipf:
        noise = torch.randn(rows, V, generator=g, device=device)
        perm = torch.argsort(torch.rand(rows, V, generator=g, device=device), dim=1)
        logits = noise - 1.1 * torch.log((perm + 1).float())
        del noise, perm
    else:
        logits = 3.0 * torch.randn(rows, V, generator=g, device=device)
    logits = logits.to(cfg.dtype)
    history = torch.randint(0, V, (rows, cfg.hist_len), generator=g, device=device)
    uniforms = torch.rand(rows, generator=g, device=device)
    return dict(logits=logits, history=history, uniforms=uniforms, knobs=dict(cfg.knobs))


def logprob_inputs(name: str, tokens: Optional[int] = None, device="cpu", weight=True):
    """Returns dict(x, w, targets, temperature) for log-prob config C or D (bf16 x, w)."""
    cfg = LOGPROB_CONFIGS[name]
    n = cfg.tokens if tokens is None else tokens
    g = _gen(device, SEED_BASE + cfg.index)
    x = torch.randn(n, cfg.hidden, generator=g, device=device).to(torch.bfloat16)
    w = None
    if weight:
        w = torch.empty(cfg.vocab, cfg.hidden, device=device, dtype=torch.bfloat16)
        step = 8192
        for s in range(0, cfg.vocab, step):
            e = min(cfg.vocab, s + step)
            w[s:e] = (0.02 * torch.randn(e - s, cfg.hidden, generator=g, device=device)).to(torch.bfloat16)
    targets = torch.randint(0, cfg.vocab, (n,), generator=g, device=device)
    return dict(x=x, w=w, targets=targets, temperature=1.0, generator=g)
