"""GPU parity of the decoupled Token-TIS loss (dsv41_token_tis_run through the C ABI) against
the numpy oracle and the reference's known answers.

Bars: loss within 1e-6 relative (fp32 sums in another order), per-token gradient within
1e-5 relative, fp64 metric sums within 1e-9 relative, counts and extrema exact; the two
metrics built from fp32 PPO ratios (whose exp may differ by an ulp between libraries, as the
reference's CPU and GPU torch do) within 1e-6 relative and two tokens of clip count.
Repeated calls are bitwise equal; errors raise the reference's messages.
"""

import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from dsv41_rocm import decoupled_token_tis_loss

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
GOLDEN = json.loads((Path(__file__).parent / "golden" / "token_tis_known_answers.json").read_text())


def _run(current, old, behavior, adv, eps=0.2, cap=2.0):
    cur = [torch.tensor(c, dtype=torch.float32, device=DEV, requires_grad=True) for c in current]
    loss, m = decoupled_token_tis_loss(cur, old, behavior, adv, clip_eps=eps, is_cap=cap)
    loss.backward()
    return loss, [c.grad.cpu().numpy() for c in cur], m


def test_known_answers_of_reference_tests():
    for case in GOLDEN["loss_cases"]:
        print(f"case: {case['name']}", flush=True)
        loss, grads, m = _run(case["current"], case["old"], case["behavior"], case["advantages"],
                              case["clip_eps"], case["is_cap"])
        if "loss" in case:
            assert abs(loss.item() - case["loss"]) < 1e-6
        if "grads" in case:
            for g, want in zip(grads, case["grads"]):
                np.testing.assert_allclose(g, want, atol=1e-6)
        if case.get("loss_equals_grpo"):
            want = oracle.grpo_loss_oracle(case["current"], case["behavior"], case["advantages"], case["clip_eps"])
            assert abs(loss.item() - float(want)) < 1e-6
        for k, v in case["metrics"].items():
            assert abs(m[k] - v) < 1e-6, (k, m[k], v)


def _batch(lens, seed, scale=0.3):
    rng = np.random.default_rng(seed)
    old = [(-rng.uniform(0.05, 12, n)).astype(np.float32) for n in lens]
    behavior = [np.minimum(o + rng.normal(0, 0.05 if scale < 1 else 1.0, o.size), 0).astype(np.float32) for o in old]
    current = [np.minimum(o + rng.normal(0, scale, o.size), 0).astype(np.float32) for o in old]
    adv = rng.normal(size=len(lens)).astype(np.float32)
    return current, old, behavior, adv


@pytest.mark.parametrize("lens,eps,cap,scale", [([512] * 32, 0.2, 2.0, 0.05), ([1, 3, 700, 257, 1024, 5], 0.1, 1.5, 0.4),
                                                ([300] * 200, 0.28, 4.0, 1.0)])
def test_matches_oracle_on_random_batches(lens, eps, cap, scale):
    print(f"case: {len(lens)} responses, {sum(lens)} tokens, eps {eps}, cap {cap}", flush=True)
    current, old, behavior, adv = _batch(lens, sum(lens), scale)
    loss, grads, m = _run(current, [torch.tensor(o) for o in old], [torch.tensor(b) for b in behavior], adv, eps, cap)
    oloss, ograds, om = oracle.token_tis_loss_oracle(current, old, behavior, adv, eps, cap)
    assert abs(loss.item() - float(oloss)) <= 1e-6 * max(1.0, abs(float(oloss)))
    for g, og in zip(grads, ograds):
        np.testing.assert_allclose(g, og, rtol=1e-5, atol=1e-9)
    for k in om:
        if k in ("loss", "policy_loss"):
            continue
        if k == "native_ppo_ratio_mean":
            assert abs(m[k] - om[k]) <= 1e-6 * abs(om[k]), (k, m[k], om[k])
            continue
        if k == "native_ppo_clip_fraction":
            assert abs(m[k] - om[k]) <= 2.0 / om["token_count"], (k, m[k], om[k])
            continue
        if k in ("response_count", "token_count", "is_clipped_tokens", "is_weight_min", "is_weight_max",
                 "is_raw_weight_min", "is_raw_weight_max", "native_old_minus_behavior_max_abs", "is_cap"):
            assert m[k] == om[k] or abs(m[k] - om[k]) <= 1e-15 * abs(om[k]), k
        else:
            assert abs(m[k] - om[k]) <= 1e-9 * max(1.0, abs(om[k])), (k, m[k], om[k])


def test_repeatable_bitwise_and_no_grad_path():
    current, old, behavior, adv = _batch([100, 200, 50], 3)
    a = _run(current, old, behavior, adv)
    b = _run(current, old, behavior, adv)
    assert a[0].item() == b[0].item() and all(np.array_equal(x, y) for x, y in zip(a[1], b[1]))
    assert a[2] == b[2]
    with torch.no_grad():
        loss, m = decoupled_token_tis_loss([torch.tensor(c, device=DEV) for c in current], old, behavior, adv)
    assert loss.item() == a[0].item() and m == a[2]


@pytest.mark.parametrize("mutate,message", [
    (lambda c, o, b: c[1].__setitem__(2, 0.5), "policy log probabilities must be nonpositive"),
    (lambda c, o, b: o[0].__setitem__(0, float("nan")), "native-old log probabilities contains non-finite values"),
    (lambda c, o, b: b[2].__setitem__(1, 1e-3), "behavior log probabilities must be nonpositive"),
    (lambda c, o, b: (o[1].__setitem__(0, -900.0), b[1].__setitem__(0, -1.0)), "raw rollout importance weights underflowed"),
    (lambda c, o, b: (c[0].__setitem__(0, -200.0), o[0].__setitem__(0, -0.5)), "native PPO ratios underflowed"),
])
def test_errors_raise_reference_messages(mutate, message):
    current, old, behavior, adv = _batch([4, 5, 6], 9)
    mutate(current, old, behavior)
    print(f"case: {message}", flush=True)
    with pytest.raises(ValueError, match=message):
        decoupled_token_tis_loss([torch.tensor(c, device=DEV) for c in current], old, behavior, adv)


def test_argument_checks():
    c = [torch.zeros(3, device=DEV) - 1]
    with pytest.raises(ValueError, match="clip_eps"):
        decoupled_token_tis_loss(c, [[-1.0] * 3], [[-1.0] * 3], [1.0], clip_eps=1.0)
    with pytest.raises(ValueError, match="is_cap"):
        decoupled_token_tis_loss(c, [[-1.0] * 3], [[-1.0] * 3], [1.0], is_cap=math.inf)
    with pytest.raises(ValueError, match="lengths must match"):
        decoupled_token_tis_loss(c, [[-1.0] * 2], [[-1.0] * 3], [1.0])
    with pytest.raises(ValueError, match="nonempty vector"):
        decoupled_token_tis_loss([torch.zeros(0, device=DEV)], [[]], [[]], [1.0])
    with pytest.raises(ValueError, match="advantages contains non-finite"):
        decoupled_token_tis_loss(c, [[-1.0] * 3], [[-1.0] * 3], [math.nan])


# ------------------------------------------------------------------------------- GRPO
from dsv41_rocm import grpo_loss  # noqa: E402


def test_grpo_known_answers_of_reference_tests():
    # test_rl_algorithm.py:64-75
    cur = [torch.tensor([math.log(0.25 * 1.5)], device=DEV, requires_grad=True),
           torch.tensor([math.log(0.25 * 0.5)], device=DEV, requires_grad=True)]
    loss, m = grpo_loss(cur, [[math.log(0.25)], [math.log(0.25)]], [1.0, -1.0])
    assert abs(loss.item() - (-1.2 + 0.8) / 2) < 1e-6 and m["clip_fraction"] == 1.0
    loss.backward()
    assert all(c.grad.item() == 0.0 for c in cur)
    # :77-81
    loss, _ = grpo_loss([torch.tensor([math.log(0.25 * 1.1)], device=DEV),
                         torch.tensor([math.log(0.25 * 0.7)] * 3, device=DEV)],
                        [[math.log(0.25)], [math.log(0.25)] * 3], [1.0, 1.0])
    assert abs(loss.item() + 0.9) < 1e-6
    # :83-91
    cur = [torch.tensor([-1.0], device=DEV, requires_grad=True), torch.tensor([-1.0], device=DEV, requires_grad=True)]
    loss, _ = grpo_loss(cur, [c.detach().clone() for c in cur], torch.tensor([1.0, -1.0]))
    loss.backward()
    assert cur[0].grad.item() < 0 < cur[1].grad.item()
    # :93-112: the behaviour-weighted k3 value and gradient equal KL(pi || ref) and its gradient
    theta = torch.tensor([0.3, -0.5], device=DEV, requires_grad=True)
    log_pi = torch.log_softmax(theta, -1)
    behavior = torch.tensor([0.7, 0.3], device=DEV)
    reference = torch.tensor([0.4, 0.6], device=DEV)
    total = 0
    for t in range(2):
        sampled, _ = grpo_loss([log_pi[t:t + 1]], [behavior[t:t + 1].log()], [0.0],
                               ref_log_probs=[reference[t:t + 1].log()], kl_beta=1.0)
        total = total + behavior[t] * sampled
    exact = (log_pi.exp() * (log_pi - reference.log())).sum()
    torch.testing.assert_close(total, exact)
    g1 = torch.autograd.grad(total, theta, retain_graph=True)[0]
    g2 = torch.autograd.grad(exact, theta)[0]
    torch.testing.assert_close(g1, g2)


@pytest.mark.parametrize("lens,eps,beta", [([512] * 32, 0.2, 0.0), ([1, 3, 700, 257, 1024, 5], 0.1, 0.05)])
def test_grpo_matches_oracle_on_random_batches(lens, eps, beta):
    print(f"case: GRPO {len(lens)} responses, eps {eps}, kl_beta {beta}", flush=True)
    current, old, behavior, adv = _batch(lens, 3 * sum(lens), 0.3)
    reference = [np.minimum(o + np.float32(0.1), 0).astype(np.float32) for o in old]
    cur = [torch.tensor(c, device=DEV, requires_grad=True) for c in current]
    loss, m = grpo_loss(cur, behavior, adv, clip_eps=eps,
                        ref_log_probs=[torch.tensor(r) for r in reference] if beta else None, kl_beta=beta)
    loss.backward()
    oloss, ograds, om = oracle.grpo_loss_oracle(current, behavior, adv, eps, reference, beta, full=True)
    assert abs(loss.item() - float(oloss)) <= 1e-6 * max(1.0, abs(float(oloss)))
    for c, og in zip(cur, ograds):
        np.testing.assert_allclose(c.grad.cpu().numpy(), og, rtol=1e-5, atol=1e-9)
    for k in om:
        tol = 2.0 / sum(lens) if k == "clip_fraction" else 1e-6 * max(1.0, abs(om[k]))
        assert abs(m[k] - om[k]) <= tol, (k, m[k], om[k])


def test_grpo_errors_raise_reference_messages():
    with pytest.raises(ValueError, match="response lengths"):
        grpo_loss([torch.tensor([-1.0, -2.0], device=DEV)], [[-1.0]], [1.0])
    with pytest.raises(ValueError, match="requires reference"):
        grpo_loss([torch.tensor([-1.0], device=DEV)], [[-1.0]], [1.0], kl_beta=0.1)
    with pytest.raises(ValueError, match="importance ratios"):
        grpo_loss([torch.tensor([-1.0], device=DEV)], [[-1000.0]], [1.0])
    with pytest.raises(ValueError, match="policy log probabilities contains non-finite"):
        grpo_loss([torch.tensor([math.nan], device=DEV)], [[-1.0]], [1.0])
