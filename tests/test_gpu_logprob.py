"""GPU parity of the fused selected-token log-prob (libdsv41hip.so through the C ABI).

Reference values: fp64 log-softmax of fp64 logits computed from the same bf16 operands
on the GPU (exact products, fp64 accumulation), plus the numpy fp64 oracle on a subset.
Bar: log-prob, entropy and Token-TIS ratio within 1e-4 absolute.
"""

import numpy as np
import pytest
import torch

import oracle
from dsv41_rocm import score_targets, selected_log_probs, token_log_probs, workloads

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
TOL = 1e-4


def reference(x, w, t, temperature):
    """fp64 log-prob and entropy from bf16 operands (on the GPU, chunked over tokens)."""
    wd = w.double()
    lps, ents = [], []
    for s in range(0, x.shape[0], 256):
        z = (x[s:s + 256].double() @ wd.T) / temperature
        lsm = torch.log_softmax(z, dim=-1)
        lps.append(lsm.gather(1, t[s:s + 256, None])[:, 0])
        ents.append(-(lsm.exp() * lsm).sum(dim=1))
    return torch.cat(lps), torch.cat(ents)


def check(x, w, t, temperature, behavior=None, cap=2.0):
    print(f"case: N={x.shape[0]} H={x.shape[1]} V={w.shape[0]} T={temperature} ratio={behavior is not None}",
          flush=True)
    lp, ent, ratio = selected_log_probs(x, w, t, temperature, behavior=behavior, is_cap=cap)
    torch.cuda.synchronize()
    rlp, rent = reference(x, w, t, temperature)
    assert torch.max(torch.abs(lp.double() - rlp)).item() <= TOL
    assert torch.max(torch.abs(ent.double() - rent)).item() <= TOL
    if behavior is not None:
        w_ref, _ = oracle.token_tis_weight(rlp.float().cpu().numpy(), behavior.cpu().numpy(), cap)
        assert np.max(np.abs(ratio.cpu().numpy() - w_ref)) <= TOL
    return lp, ent, ratio


def test_config_c_shape_reduced_tokens():
    inp = workloads.logprob_inputs("C", tokens=512, device=DEV)
    check(inp["x"], inp["w"], inp["targets"], 1.0)


def test_config_d_shape_reduced_tokens_with_ratio():
    inp = workloads.logprob_inputs("D", tokens=384, device=DEV)
    g = torch.Generator(device=DEV).manual_seed(5)
    rlp, _ = reference(inp["x"], inp["w"], inp["targets"], 1.0)
    behavior = (rlp + 0.05 * torch.randn(rlp.shape, generator=g, device=DEV, dtype=torch.float64)).float()
    check(inp["x"], inp["w"], inp["targets"], 1.0, behavior=behavior)


def test_numpy_oracle_subset_agrees():
    inp = workloads.logprob_inputs("C", tokens=256, device=DEV)
    lp, ent, _ = selected_log_probs(inp["x"], inp["w"], inp["targets"], 0.8)
    idx = torch.arange(0, 256, 37)
    olp, oent = oracle.logprob_oracle(inp["x"][idx].float().cpu().numpy(), inp["w"].float().cpu().numpy(),
                                      inp["targets"][idx].cpu().numpy(), 0.8)
    assert np.max(np.abs(lp[idx].cpu().numpy() - olp)) <= TOL
    assert np.max(np.abs(ent[idx].cpu().numpy() - oent)) <= TOL


@pytest.mark.parametrize("n,h,v", [(1, 8, 1), (5, 40, 3), (130, 72, 257), (257, 136, 1000), (300, 2048, 4099),
                                   (64, 64, 65536 + 17)])
def test_ragged_shapes(n, h, v):
    g = torch.Generator(device=DEV).manual_seed(n * 1000 + v)
    x = torch.randn(n, h, generator=g, device=DEV).to(torch.bfloat16)
    w = (0.3 * torch.randn(v, h, generator=g, device=DEV)).to(torch.bfloat16)
    t = torch.randint(0, v, (n,), generator=g, device=DEV)
    check(x, w, t, 0.7)


def test_strided_hidden_and_empty_and_errors():
    g = torch.Generator(device=DEV).manual_seed(9)
    big = torch.randn(70, 200, generator=g, device=DEV).to(torch.bfloat16)
    x = big[:, :192]  # row stride 200 (multiple of 8), 16-byte aligned rows
    w = (0.2 * torch.randn(999, 192, generator=g, device=DEV)).to(torch.bfloat16)
    t = torch.randint(0, 999, (70,), generator=g, device=DEV)
    check(x, w, t, 1.3)
    lp, ent, _ = selected_log_probs(x[:0], w, t[:0], 1.0)
    assert lp.shape == (0,) and ent.shape == (0,)
    with pytest.raises(ValueError, match="outside the model vocabulary"):
        selected_log_probs(x, w, torch.full_like(t, 999), 1.0)
    with pytest.raises(ValueError, match="temperature"):
        selected_log_probs(x, w, t, 0.0)


def test_drop_ins_match_reference_expression():
    g = torch.Generator(device=DEV).manual_seed(3)
    B, T, H, V = 2, 7, 64, 515
    hidden = torch.randn(B, T, H, generator=g, device=DEV).to(torch.bfloat16)
    w = (0.2 * torch.randn(V, H, generator=g, device=DEV)).to(torch.bfloat16)
    targets = torch.randint(0, V, (B, T), generator=g, device=DEV)
    mask = torch.rand(B, T, generator=g, device=DEV) > 0.3
    out = token_log_probs(hidden, w, targets, mask, 0.8)
    # model.py:682-684 with fp32 logits (the kernel does not round logits to bf16)
    logits = (hidden[mask].double() @ w.double().T) / 0.8
    sel = torch.log_softmax(logits, -1).gather(-1, targets[mask].unsqueeze(-1)).squeeze(-1)
    expect = torch.zeros(B, T, dtype=torch.float64, device=DEV).masked_scatter(mask, sel)
    assert out.dtype == torch.float32 and out.shape == (B, T)
    assert torch.max(torch.abs(out.double() - expect)).item() <= TOL
    assert torch.equal(out[~mask], torch.zeros_like(out[~mask]))
    s = score_targets(hidden[mask], w, targets[mask], 0.8)
    assert torch.equal(s, out[mask])
    empty = token_log_probs(hidden, w, targets, torch.zeros_like(mask), 0.8)
    assert torch.equal(empty, torch.zeros(B, T, device=DEV))


def test_repeatable_bitwise():
    inp = workloads.logprob_inputs("C", tokens=300, device=DEV)
    a = selected_log_probs(inp["x"], inp["w"], inp["targets"], 1.0)
    b = selected_log_probs(inp["x"], inp["w"], inp["targets"], 1.0)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_custom_op_matches_wrapper():
    inp = workloads.logprob_inputs("C", tokens=64, device=DEV)
    x, w, t = inp["x"], inp["w"], inp["targets"]
    print("case: torch.ops.dsv41_rocm.selected_log_probs on config C, 64 tokens", flush=True)
    behavior = torch.full((64,), -12.0, device=DEV)
    lp, ent, ratio, lse = torch.ops.dsv41_rocm.selected_log_probs(x, w, t, 0.9, behavior, 2.0)
    rlp, rent, rratio = selected_log_probs(x, w, t, 0.9, behavior=behavior, is_cap=2.0)
    assert torch.equal(lp, rlp) and torch.equal(ent, rent) and torch.equal(ratio, rratio)
    zt = (x.double() * w[t].double()).sum(-1) / 0.9
    assert torch.max(torch.abs(lse.double() - (zt - lp.double()))).item() <= 1e-4
    lp2, _, empty, _ = torch.ops.dsv41_rocm.selected_log_probs(x, w, t, 0.9, None, 2.0)
    assert torch.equal(lp2, rlp) and empty.numel() == 0


@pytest.mark.parametrize("n,h,v,cuts", [(512, 2048, 20000, [12000]), (300, 136, 1000, [1, 257, 700]),
                                        (384, 7168, 129280, [16160 * k for k in range(1, 8)])])
def test_vocabulary_shards_combine_to_the_unsharded_head(n, h, v, cuts):
    """A vocabulary-sharded head on one GPU: each slice's 16-byte states, stacked as an
    all-gather would deliver them, combine to the unsharded outputs."""
    print(f"case: shards N={n} H={h} V={v} cuts={cuts}", flush=True)
    from dsv41_rocm import combine_states, shard_states

    g = torch.Generator(device=DEV).manual_seed(n + v)
    x = torch.randn(n, h, generator=g, device=DEV).to(torch.bfloat16)
    w = (0.3 * torch.randn(v, h, generator=g, device=DEV) / (h ** 0.5) * 8).to(torch.bfloat16)
    t = torch.randint(0, v, (n,), generator=g, device=DEV)
    behavior = torch.full((n,), -9.0, device=DEV)
    lp, ent, ratio = selected_log_probs(x, w, t, 0.8, behavior=behavior)
    bounds = [0] + cuts + [v]
    states = torch.stack([shard_states(x, w[b:e], t, 0.8, b) for b, e in zip(bounds[:-1], bounds[1:])])
    assert states.shape == (len(bounds) - 1, n, 4)
    owned = torch.isfinite(states[:, :, 3]).sum(dim=0)
    assert torch.equal(owned, torch.ones_like(owned))  # each target logit comes from exactly one slice
    clp, cent, cratio = combine_states(states, behavior=behavior)
    assert torch.max(torch.abs(clp - lp)).item() <= 2e-5
    assert torch.max(torch.abs(cent - ent)).item() <= 2e-5
    assert torch.max(torch.abs(cratio - ratio)).item() <= 2e-5
    rlp, rent = reference(x, w, t, 0.8)
    assert torch.max(torch.abs(clp.double() - rlp)).item() <= TOL
    assert torch.max(torch.abs(cent.double() - rent)).item() <= TOL
