"""numpy fp64 restatement of the selected-token log-prob head.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Follows ``dsv41_train/models/dsv4/model.py:679-684`` (``_token_log_probs``:
``log_softmax(lm_head(h).float() / T).gather(targets)``) and
``dsv41_train/rl/native_lora.py:80-82`` (``_score_targets``), with one deliberate
difference: the logits are the exact products of the bf16 inputs accumulated in fp64
(no bf16 rounding of the logits), which is the quantity the fused kernel approximates
in fp32.  Entropy is the closed form ``H = LSE - sum_v p_v z_v``.  The Token-TIS weight
follows ``dsv41_train/rl/algorithm.py:293-299``:
``delta = float32(old - behavior); raw = exp(float64(delta)); w = float32(min(cap, raw))``.

``logprob_grad_oracle`` restates the backward of the same expression as autograd takes it
when the learner differentiates its ``current`` scores (``dsv41_train/rl/distributed_grpo.py:
352-375``): with ``p = softmax(z)``, ``dlp/dz = onehot(t) - p`` and
``dH/dz = p * (LSE - H - z)``; the logit gradient is ``dL/dz / T`` and the input and weight
gradients are its products with ``w`` and ``x`` (fp64 throughout).
"""

from __future__ import annotations

import numpy as np


def logprob_oracle(x, w, targets, temperature=1.0, chunk=256):
    """x [N, H], w [V, H] (any float dtype holding the bf16 values exactly), targets [N].

    Returns (logprob fp64 [N], entropy fp64 [N]).
    """
    x = np.asarray(x, dtype=np.float64)
    w = np.asarray(w, dtype=np.float64)
    targets = np.asarray(targets, dtype=np.int64)
    n = x.shape[0]
    lp = np.empty(n, np.float64)
    ent = np.empty(n, np.float64)
    for s in range(0, n, chunk):
        z = (x[s:s + chunk] @ w.T) / float(temperature)
        m = z.max(axis=1, keepdims=True)
        e = np.exp(z - m)
        tot = e.sum(axis=1, keepdims=True)
        lse = (m + np.log(tot))[:, 0]
        lp[s:s + chunk] = z[np.arange(z.shape[0]), targets[s:s + chunk]] - lse
        ent[s:s + chunk] = lse - (e * z).sum(axis=1) / tot[:, 0]
    return lp, ent


def token_tis_weight(old, behavior, is_cap=2.0):
    """Clipped Token-TIS weight, algorithm.py:293-299 (fp32 result)."""
    delta = (np.asarray(old, dtype=np.float32) - np.asarray(behavior, dtype=np.float32)).astype(np.float32)
    raw = np.exp(delta.astype(np.float64))
    return np.minimum(np.float64(is_cap), raw).astype(np.float32), raw


def logprob_grad_oracle(x, w, targets, temperature, grad_logprob, grad_entropy=None, chunk=256):
    """Returns (dL/dlogits [N, V], dL/dx [N, H], dL/dw [V, H]) in fp64 for the loss
    ``sum(grad_logprob * logprob) + sum(grad_entropy * entropy)``."""
    x = np.asarray(x, dtype=np.float64)
    w = np.asarray(w, dtype=np.float64)
    targets = np.asarray(targets, dtype=np.int64)
    n, v = x.shape[0], w.shape[0]
    glp = np.asarray(grad_logprob, dtype=np.float64)
    gent = np.zeros(n) if grad_entropy is None else np.asarray(grad_entropy, dtype=np.float64)
    gl = np.empty((n, v), np.float64)
    for s in range(0, n, chunk):
        z = (x[s:s + chunk] @ w.T) / float(temperature)
        m = z.max(axis=1, keepdims=True)
        e = np.exp(z - m)
        tot = e.sum(axis=1, keepdims=True)
        p = e / tot
        lse = m + np.log(tot)
        ent = lse[:, 0] - (p * z).sum(axis=1)
        onehot = np.zeros_like(z)
        onehot[np.arange(z.shape[0]), targets[s:s + chunk]] = 1.0
        gz = glp[s:s + chunk, None] * (onehot - p) + gent[s:s + chunk, None] * p * (lse - ent[:, None] - z)
        gl[s:s + chunk] = gz / float(temperature)
    return gl, gl @ w, gl.T @ x
