"""numpy restatement of the decoupled Token-TIS loss, its gradient and its metrics.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Follows ``dsv41_train/rl/algorithm.py:249-346`` (``decoupled_token_tis_loss``) dtype by dtype:
``delta = f32(old - behavior)``, ``raw = exp(f64(delta))``, ``w = f32(min(raw, cap))``,
``ratio = exp(f32(current - old))`` in fp32, the surrogate
``min(ratio * A, clamp(ratio, f32(1 - eps), f32(1 + eps)) * A)`` in fp32, per-response fp32
means, and the metric sums in fp64 over the clamped raw weights.  The gradient with respect to
``current`` is written out from the autograd rules torch applies to that expression:
``minimum`` gives the smaller side the gradient and splits ties in half, ``clamp`` passes it
inside its closed interval, ``mean`` divides by the count.  Metrics are pooled over all
responses, as ``aggregate_token_tis_metrics`` (``dsv41_train/rl/distributed_grpo.py:197-222``)
pools per-response rows.  The per-response loop is deliberately plain.
"""

from __future__ import annotations

import numpy as np

METRIC_KEYS = (
    "loss", "policy_loss", "response_count", "token_count", "is_cap", "is_weight_sum",
    "is_weight_square_sum", "is_weight_mean", "is_weight_min", "is_weight_max", "is_raw_weight_sum",
    "is_raw_weight_min", "is_raw_weight_max", "is_clipped_tokens", "is_clipped_fraction",
    "is_dropped_weight_mass", "is_dropped_weight_mass_fraction", "is_token_weight_ess",
    "is_token_weight_ess_fraction", "native_old_minus_behavior_mean", "native_old_minus_behavior_max_abs",
    "native_ppo_ratio_mean", "native_ppo_clip_fraction",
)


def token_tis_loss_oracle(current, old, behavior, advantages, clip_eps=0.2, is_cap=2.0):
    """current / old / behavior: lists of 1-D arrays (one per response); advantages: [R].

    Returns (loss fp32, [grad fp32 array per response], metrics dict of Python floats).
    """
    f32 = np.float32
    R = len(current)
    adv = np.asarray(advantages, dtype=f32)
    lo, hi = f32(1.0 - clip_eps), f32(1.0 + clip_eps)
    terms, grads = [], []
    wd_all, raw_all, ratio_all, delta_all = [], [], [], []
    for r in range(R):
        c = np.asarray(current[r], dtype=f32)
        o = np.asarray(old[r], dtype=f32)
        b = np.asarray(behavior[r], dtype=f32)
        delta = (o - b).astype(f32)
        raw = np.exp(delta.astype(np.float64))
        wd = np.minimum(raw, np.float64(is_cap))
        w = wd.astype(f32)
        ratio = np.exp((c - o).astype(f32)).astype(f32)
        A = adv[r]
        u = (ratio * A).astype(f32)
        cl = (np.clip(ratio, lo, hi) * A).astype(f32)
        s = np.minimum(u, cl)
        terms.append(-f32(np.mean((w * s).astype(f32), dtype=f32)))
        gu = np.where(u < cl, 1.0, np.where(u == cl, 0.5, 0.0)).astype(f32)
        gc = np.where(cl < u, 1.0, np.where(u == cl, 0.5, 0.0)).astype(f32)
        inside = ((ratio >= lo) & (ratio <= hi)).astype(f32)
        ds = (A * (gu + gc * inside) * ratio).astype(f32)
        grads.append((-(w * ds) / f32(len(c)) / f32(R)).astype(f32))
        wd_all.append(wd)
        raw_all.append(raw)
        ratio_all.append(ratio.astype(np.float64))
        delta_all.append(delta.astype(np.float64))
    loss = f32(np.mean(np.asarray(terms, dtype=f32), dtype=f32))
    wd, raw = np.concatenate(wd_all), np.concatenate(raw_all)
    ratios, deltas = np.concatenate(ratio_all), np.concatenate(delta_all)
    total, squared, raw_total = wd.sum(), (wd * wd).sum(), raw.sum()
    ess = total * total / squared
    n = float(wd.size)
    dropped = max(raw_total - total, 0.0)
    values = (float(loss), float(loss), float(R), n, float(is_cap), float(total), float(squared), float(wd.mean()),
              float(wd.min()), float(wd.max()), float(raw_total), float(raw.min()), float(raw.max()),
              float((raw > is_cap).sum()), float((raw > is_cap).mean()), float(dropped), float(dropped / raw_total),
              float(ess), float(ess / n), float(deltas.mean()), float(np.abs(deltas).max()), float(ratios.mean()),
              float((np.abs(ratios - 1) > clip_eps).mean()))
    return loss, grads, dict(zip(METRIC_KEYS, values))


def grpo_loss_oracle(current, behavior, advantages, clip_eps=0.2, reference=None, kl_beta=0.0, full=False):
    """grpo_loss (algorithm.py:169-246) in fp32 per response: ratio = exp(current - behavior),
    the clipped surrogate mean, and with kl_beta the mean of ratio * (expm1(d) - d),
    d = reference - current.  Returns the loss, or with ``full`` (loss, grads, metrics), the
    gradient written out from torch's minimum / clamp rules and d(k3)/d current =
    ratio * (current - reference)."""
    f32 = np.float32
    R = len(current)
    lo, hi = f32(1.0 - clip_eps), f32(1.0 + clip_eps)
    beta = f32(kl_beta)
    pols, kls, clips, ratios, akls, grads = [], [], [], [], [], []
    for r, (c, b, A) in enumerate(zip(current, behavior, np.asarray(advantages, dtype=f32))):
        c = np.asarray(c, f32)
        lr = (c - np.asarray(b, f32)).astype(f32)
        ratio = np.exp(lr).astype(f32)
        u = (ratio * A).astype(f32)
        cl = (np.clip(ratio, lo, hi) * A).astype(f32)
        s = np.minimum(u, cl)
        pols.append(-f32(np.mean(s, dtype=f32)))
        gu = np.where(u < cl, 1.0, np.where(u == cl, 0.5, 0.0)).astype(f32)
        gc = np.where(cl < u, 1.0, np.where(u == cl, 0.5, 0.0)).astype(f32)
        inside = ((ratio >= lo) & (ratio <= hi)).astype(f32)
        g = (-(A * (gu + gc * inside) * ratio)).astype(f32)
        if kl_beta:
            ref = np.asarray(reference[r], f32)
            d = (ref - c).astype(f32)
            k3 = (ratio * (np.expm1(d).astype(f32) - d)).astype(f32)
            kls.append(f32(np.mean(k3, dtype=f32)))
            g = (g + beta * (ratio * (c - ref))).astype(f32)
        else:
            kls.append(f32(0.0))
        grads.append((g / f32(c.size) / f32(R)).astype(f32))
        clips.append(f32(np.mean((np.abs(ratio - f32(1)) > f32(clip_eps)).astype(f32), dtype=f32)))
        ratios.append(f32(np.mean(ratio, dtype=f32)))
        akls.append(f32(np.mean(-lr, dtype=f32)))
    mean = lambda v: f32(np.mean(np.asarray(v, dtype=f32), dtype=f32))
    policy, kl = mean(pols), mean(kls)
    loss = f32(policy + beta * kl)
    if not full:
        return loss
    metrics = {"loss": float(loss), "policy_loss": float(policy), "kl": float(kl), "clip_fraction": float(mean(clips)),
               "importance_ratio": float(mean(ratios)), "approx_kl": float(mean(akls))}
    return loss, grads, metrics
