"""Pins the Token-TIS and GRPO oracles (oracle/tis_oracle.py) without a GPU: the reference's
own known answers (tests/test_rl_token_tis.py and tests/test_rl_algorithm.py in the Tiny-DSV41
tree; the Token-TIS ones kept as tests/golden/token_tis_known_answers.json), torch autograd for
the gradients, and the reduction to grpo_loss when native-old equals behaviour."""

import json
import math
from pathlib import Path

import numpy as np
import torch

import oracle

GOLDEN = json.loads((Path(__file__).parent / "golden" / "token_tis_known_answers.json").read_text())


def test_known_answers_of_reference_tests():
    for case in GOLDEN["loss_cases"]:
        loss, grads, m = oracle.token_tis_loss_oracle(case["current"], case["old"], case["behavior"],
                                                      case["advantages"], case["clip_eps"], case["is_cap"])
        if "loss" in case:
            assert abs(float(loss) - case["loss"]) < 1e-6, case["name"]
        if "grads" in case:
            for g, want in zip(grads, case["grads"]):
                np.testing.assert_allclose(g, want, atol=1e-6, err_msg=case["name"])
        if case.get("loss_equals_grpo"):
            want = oracle.grpo_loss_oracle(case["current"], case["behavior"], case["advantages"], case["clip_eps"])
            assert abs(float(loss) - float(want)) < 1e-7
        for k, v in case["metrics"].items():
            assert abs(m[k] - v) < 1e-6, (case["name"], k, m[k], v)


def _torch_expression(current, old, behavior, adv, eps, cap):
    """algorithm.py:275-303 as torch expressions (the loss only), for autograd."""
    terms = []
    for c, o, b, a in zip(current, old, behavior, adv):
        w = (o - b).double().exp().clamp(max=cap).float()
        ratio = (c - o).exp()
        terms.append(-(w * torch.minimum(ratio * a, ratio.clamp(1 - eps, 1 + eps) * a)).mean())
    return torch.stack(terms).mean()


def test_gradient_matches_torch_autograd_including_ties_and_clipping():
    rng = np.random.default_rng(5)
    lens = [1, 7, 33, 2, 64]
    old = [(-rng.uniform(0.1, 5, n)).astype(np.float32) for n in lens]
    behavior = [(o + rng.normal(0, 0.7, o.size)).astype(np.float32).clip(max=0) for o in old]
    current = [(o + rng.normal(0, 0.3, o.size)).astype(np.float32).clip(max=0) for o in old]
    current[1][:3] = old[1][:3]  # ratio exactly 1: the surrogate's two sides tie
    adv = np.array([1.0, -1.0, 0.5, -2.0, 0.0], np.float32)
    for eps, cap in ((0.2, 2.0), (0.05, 1.0), (0.0, 8.0)):
        loss, grads, m = oracle.token_tis_loss_oracle(current, old, behavior, adv, eps, cap)
        cur = [torch.from_numpy(c).requires_grad_() for c in current]
        ref = _torch_expression(cur, [torch.from_numpy(o) for o in old], [torch.from_numpy(b) for b in behavior],
                                torch.from_numpy(adv), eps, cap)
        ref.backward()
        assert abs(float(loss) - ref.item()) <= 1e-6 * max(1.0, abs(ref.item()))
        for g, c in zip(grads, cur):
            np.testing.assert_allclose(g, c.grad.numpy(), rtol=1e-5, atol=1e-8)
        # pooled diagnostics: ESS never exceeds the token count; dropped mass is raw - clamped
        assert m["is_token_weight_ess"] <= m["token_count"] + 1e-9
        assert abs(m["is_dropped_weight_mass"] - (m["is_raw_weight_sum"] - m["is_weight_sum"])) < 1e-9


def test_grpo_known_answers_of_reference_tests():
    # test_rl_algorithm.py:64-75: clipping for both advantage signs, zero gradients, clip fraction 1
    loss, grads, m = oracle.grpo_loss_oracle([[math.log(0.25 * 1.5)], [math.log(0.25 * 0.5)]],
                                             [[math.log(0.25)], [math.log(0.25)]], [1.0, -1.0], full=True)
    assert abs(float(loss) - (-1.2 + 0.8) / 2) < 1e-6 and m["clip_fraction"] == 1.0
    assert all(float(g[0]) == 0.0 for g in grads)
    # :77-81: each response is averaged before the batch
    loss = oracle.grpo_loss_oracle([[math.log(0.25 * 1.1)], [math.log(0.25 * 0.7)] * 3],
                                   [[math.log(0.25)], [math.log(0.25)] * 3], [1.0, 1.0])
    assert abs(float(loss) + 0.9) < 1e-6
    # :83-91: unclipped gradient direction
    _, grads, _ = oracle.grpo_loss_oracle([[-1.0], [-1.0]], [[-1.0], [-1.0]], [1.0, -1.0], full=True)
    assert grads[0][0] < 0 < grads[1][0]
    # :93-112: behaviour-weighted k3 equals KL(pi || ref) exactly
    log_pi = np.log(np.exp([0.3, -0.5]) / np.exp([0.3, -0.5]).sum()).astype(np.float32)
    behavior, reference = np.array([0.7, 0.3]), np.array([0.4, 0.6])
    total = sum(behavior[t] * float(oracle.grpo_loss_oracle([[log_pi[t]]], [[math.log(behavior[t])]], [0.0],
                                                            reference=[[math.log(reference[t])]], kl_beta=1.0))
                for t in range(2))
    exact = float((np.exp(log_pi) * (log_pi - np.log(reference))).sum())
    assert abs(total - exact) < 1e-6


def test_grpo_gradient_and_metrics_match_torch_autograd():
    rng = np.random.default_rng(8)
    lens = [1, 9, 40, 3]
    behavior = [(-rng.uniform(0.1, 4, n)).astype(np.float32) for n in lens]
    current = [np.minimum(b + rng.normal(0, 0.4, b.size), 0).astype(np.float32) for b in behavior]
    reference = [np.minimum(b + rng.normal(0, 0.3, b.size), 0).astype(np.float32) for b in behavior]
    current[1][:2] = behavior[1][:2]  # ratio exactly one
    adv = np.array([1.0, -0.5, 2.0, 0.0], np.float32)
    for eps, beta in ((0.2, 0.0), (0.1, 0.3)):
        loss, grads, m = oracle.grpo_loss_oracle(current, behavior, adv, eps, reference, beta, full=True)
        cur = [torch.from_numpy(c).requires_grad_() for c in current]
        pol, kls, clips, ratios, akls = [], [], [], [], []
        for c, b, rf, a in zip(cur, behavior, reference, torch.from_numpy(adv)):
            lr = c - torch.from_numpy(b)
            ratio = torch.exp(lr)
            pol.append(-torch.minimum(ratio * a, ratio.clamp(1 - eps, 1 + eps) * a).mean())
            d = torch.from_numpy(rf) - c
            kls.append((ratio * (torch.expm1(d) - d)).mean() if beta else c.new_zeros(()))
            clips.append(((ratio - 1).abs() > eps).float().mean())
            ratios.append(ratio.mean())
            akls.append((-lr).mean())
        ref_loss = torch.stack(pol).mean() + beta * torch.stack(kls).mean()
        ref_loss.backward()
        assert abs(float(loss) - ref_loss.item()) <= 1e-6 * max(1.0, abs(ref_loss.item()))
        for g, c in zip(grads, cur):
            np.testing.assert_allclose(g, c.grad.numpy(), rtol=1e-5, atol=1e-8)
        assert abs(m["clip_fraction"] - torch.stack(clips).mean().item()) < 1e-7
        assert abs(m["importance_ratio"] - torch.stack(ratios).mean().item()) < 1e-6
        assert abs(m["approx_kl"] - torch.stack(akls).mean().item()) < 1e-6
