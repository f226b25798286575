"""Pins the numpy log-prob oracle (oracle/logprob_oracle.py) without a GPU: torch's
log_softmax in fp64, the entropy closed form, and the known answers of the reference's
Token-TIS tests (tests/golden/token_tis_known_answers.json)."""

import json
import math
from pathlib import Path

import numpy as np
import torch

import oracle

GOLDEN = Path(__file__).parent / "golden"


def _bf16_values(shape, scale, seed):
    g = torch.Generator().manual_seed(seed)
    return (scale * torch.randn(*shape, generator=g)).to(torch.bfloat16).float().numpy()


def test_logprob_and_entropy_match_torch_fp64():
    x = _bf16_values((37, 48), 1.0, 1)
    w = _bf16_values((501, 48), 0.3, 2)
    t = np.random.default_rng(3).integers(0, 501, 37)
    for T in (1.0, 0.7, 1.9):
        lp, ent = oracle.logprob_oracle(x, w, t, T, chunk=8)
        z = torch.from_numpy(x).double() @ torch.from_numpy(w).double().T / T
        lsm = torch.log_softmax(z, -1)
        np.testing.assert_allclose(lp, lsm[torch.arange(37), torch.from_numpy(t)].numpy(), atol=1e-12)
        np.testing.assert_allclose(ent, (-(lsm.exp() * lsm).sum(-1)).numpy(), atol=1e-10)


def test_entropy_special_cases():
    # uniform logits: entropy log V and log-prob -log V; one dominant logit: entropy ~ 0
    x = np.zeros((2, 8))
    w = np.zeros((1000, 8))
    lp, ent = oracle.logprob_oracle(x, w, np.array([3, 999]))
    np.testing.assert_allclose(ent, math.log(1000), rtol=1e-12)
    np.testing.assert_allclose(lp, -math.log(1000), rtol=1e-12)
    w2 = np.zeros((5, 8))
    w2[2, 0] = 1000.0
    lp, ent = oracle.logprob_oracle(np.ones((1, 8)), w2, np.array([2]))
    assert abs(ent[0]) < 1e-12 and abs(lp[0]) < 1e-12


def test_token_tis_weight_known_answers_from_reference_tests():
    cases = json.loads((GOLDEN / "token_tis_known_answers.json").read_text())["cases"]
    for c in cases:
        old = np.array(c["old"], np.float32)
        behavior = (old.astype(np.float64) - np.log(np.array(c["behavior_minus_old_logs"]))).astype(np.float32)
        w, raw = oracle.token_tis_weight(old, behavior, c["is_cap"])
        np.testing.assert_allclose(raw, c["raw"], rtol=1e-6)
        np.testing.assert_allclose(w, c["weights"], rtol=1e-6)
        assert w.dtype == np.float32
        if "is_weight_sum" in c:
            assert abs(float(w.astype(np.float64).sum()) - c["is_weight_sum"]) < 1e-6
            assert abs(float(raw.sum()) - c["is_raw_weight_sum"]) < 1e-6
            assert int((raw > c["is_cap"]).sum()) == c["is_clipped_tokens"]
            ws = w.astype(np.float64)
            assert abs(ws.sum() ** 2 / (ws ** 2).sum() - c["is_token_weight_ess"]) < 1e-6
        if "is_weight_min" in c:
            assert abs(w.min() - c["is_weight_min"]) < 1e-6 and w.max() == c["is_weight_max"]
        if "is_clipped_fraction" in c:
            assert (raw > c["is_cap"]).mean() == c["is_clipped_fraction"]


def test_grad_oracle_matches_torch_fp64_autograd():
    """The backward restatement against torch autograd of the reference expression in fp64
    (log_softmax(x @ w.T / T).gather, entropy = -(p * log p).sum), with both upstream
    gradients nonzero and a token whose target is the row maximum."""
    x = _bf16_values((23, 40), 1.0, 11)
    w = _bf16_values((301, 40), 0.4, 12)
    rng = np.random.default_rng(13)
    t = rng.integers(0, 301, 23)
    glp = rng.normal(size=23)
    gent = rng.normal(size=23)
    for T in (1.0, 0.6):
        gl, dx, dw = oracle.logprob_grad_oracle(x, w, t, T, glp, gent, chunk=7)
        xt = torch.from_numpy(x).double().requires_grad_()
        wt = torch.from_numpy(w).double().requires_grad_()
        logits = xt @ wt.T
        logits.retain_grad()
        lsm = torch.log_softmax(logits / T, -1)
        lp = lsm.gather(-1, torch.from_numpy(t)[:, None])[:, 0]
        ent = -(lsm.exp() * lsm).sum(-1)
        ((torch.from_numpy(glp) * lp).sum() + (torch.from_numpy(gent) * ent).sum()).backward()
        np.testing.assert_allclose(gl, logits.grad.numpy(), atol=1e-12)
        np.testing.assert_allclose(dx, xt.grad.numpy(), atol=1e-10)
        np.testing.assert_allclose(dw, wt.grad.numpy(), atol=1e-10)
    # log-prob alone: each logit-gradient row sums to zero and equals (onehot - softmax) / T
    gl, _, _ = oracle.logprob_grad_oracle(x, w, t, 0.8, np.ones(23))
    np.testing.assert_allclose(gl.sum(axis=1), 0.0, atol=1e-12)
    assert np.all(gl[np.arange(23), t] > 0) and np.all(np.delete(gl[0], t[0]) < 0)
