"""GPU parity of the exponential-race draw and of the decode-loop drop-in.

The reference draws with ``torch.multinomial(log_softmax(logits.float() / T).exp().cpu(), 1,
generator=g)`` (dsv41_train/rl/rollout.py:144-148).  Fed ``torch.empty(V).exponential_(1,
generator=g)`` from an identically seeded generator, the race draw must return the same token
on at least 99.9% of rows (ids can differ only where two ratios p/E lie within an ulp), the
behaviour log-prob within 1e-5 of ``log_softmax(...)[token]``, and the generator must end in
the reference's state.
"""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from dsv41_rocm import generate_group_responses, generate_response, sample, workloads

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
GOLDEN = Path(__file__).parent / "golden"


def _reference_draws(logits, T, seed):
    g = torch.Generator().manual_seed(seed)
    ids, lps = [], []
    for r in range(logits.shape[0]):
        lsm = torch.log_softmax(logits[r].float() / T, dim=-1)
        tok = int(torch.multinomial(lsm.exp().cpu(), 1, generator=g).item())
        ids.append(tok)
        lps.append(float(lsm[tok].item()))
    return np.array(ids), np.array(lps), g.get_state()


def _race_draws(logits, T, seed, **knobs):
    g = torch.Generator().manual_seed(seed)
    e = torch.empty(logits.shape, dtype=torch.float32).exponential_(1, generator=g)
    res = sample(logits, temperature=T, exponentials=e, **knobs)
    return res.ids.cpu().numpy(), res.logprobs.cpu().numpy(), g.get_state()


@pytest.mark.parametrize("name,rows,T", [("B", 256, 1.0), ("A", 8, 0.7), ("B", 64, 0.6)])
def test_race_draw_reproduces_torch_multinomial(name, rows, T):
    print(f"case: exponential race config {name} rows {rows} T {T}", flush=True)
    inp = workloads.sampler_inputs(name, rows=rows, device=DEV)
    logits = inp["logits"]
    rid, rlp, rstate = _reference_draws(logits, T, 11)
    oid, olp, ostate = _race_draws(logits, T, 11)
    agree = (rid == oid).mean()
    print(f"agreement {agree:.4f}", flush=True)
    assert agree >= 0.999
    ok = rid == oid
    assert np.max(np.abs(rlp[ok] - olp[ok])) <= 1e-5
    assert torch.equal(rstate, ostate)


def test_race_draw_with_penalties_matches_penalized_multinomial():
    inp = workloads.sampler_inputs("B", rows=32, device=DEV)
    logits, hist = inp["logits"].float(), inp["history"][:, :256]
    rp, pres, freq, T = 1.3, 0.4, 0.25, 0.8
    # the penalties of the sampler specification, as float32 torch ops on the GPU
    x = logits.clone()
    counts = torch.zeros_like(x).scatter_add_(1, hist, torch.ones_like(hist, dtype=torch.float32))
    seen = counts > 0
    x = torch.where(seen, torch.where(x > 0, x / rp, x * rp), x)
    x = torch.where(seen, x - freq * counts, x)
    x = torch.where(seen, x - pres, x)
    rid, rlp, _ = _reference_draws(x, T, 5)
    oid, olp, _ = _race_draws(logits, T, 5, history=hist, repetition_penalty=rp, presence_penalty=pres,
                              frequency_penalty=freq)
    assert (rid == oid).mean() >= 0.999
    ok = rid == oid
    assert np.max(np.abs(rlp[ok] - olp[ok])) <= 1e-5


class TransitionModel(torch.nn.Module):
    """The reference's rollout toy (tests/test_rl_rollout.py:18-29): the next-token logits are
    the row of the last input token."""

    def __init__(self, table):
        super().__init__()
        self.table = torch.nn.Parameter(torch.tensor(table, dtype=torch.float32, device=DEV), requires_grad=False)

    def forward(self, tokens, attention_mask=None):
        return self.table[tokens]


class RandomHead(torch.nn.Module):
    """A small random causal LM: embedding, one tanh layer, vocabulary head."""

    def __init__(self, vocab, width, seed):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        self.emb = torch.nn.Parameter((torch.randn(vocab, width, generator=g)).to(DEV), requires_grad=False)
        self.head = torch.nn.Parameter((torch.randn(vocab, width, generator=g) / width ** 0.5 * 4).to(DEV),
                                       requires_grad=False)

    def forward(self, tokens, attention_mask=None):
        h = torch.tanh(torch.cumsum(self.emb[tokens], dim=1) / tokens.shape[1] ** 0.5)
        return h @ self.head.T


def _reference_loop(model, prompt, max_new, T, eos, stops, g):
    """rollout.py:124-157 restated (sampling step as the reference does it)."""
    stops = sorted(stops, key=len, reverse=True)
    response, behavior, reason, count = [], [], "length", 0
    with torch.inference_mode():
        for _ in range(max_new):
            tokens = torch.tensor([prompt + response], dtype=torch.long, device=DEV)
            logits = model(tokens, attention_mask=torch.ones_like(tokens))[0, -1]
            lsm = torch.log_softmax(logits.float() / T, dim=-1)
            tok = int(torch.multinomial(lsm.exp().cpu(), 1, generator=g).item())
            response.append(tok)
            behavior.append(float(lsm[tok].item()))
            m = next((ids for ids in stops if response[-len(ids):] == ids), None)
            if m is not None:
                reason, count = "stop", len(m)
                break
            if tok in eos:
                reason, count = "eos", 1
                break
    return response, behavior, reason, count


@pytest.mark.parametrize("which", ["transition", "random_head"])
def test_decode_loop_replays_reference_samples(which):
    if which == "transition":
        fixture = json.loads((GOLDEN / "rollout_transition_model.json").read_text())
        model, prompt, T, eos, stops, group = TransitionModel(fixture["transitions"]), [0], fixture["temperature"], [2], [], 12
    else:
        model, prompt, T, eos, stops, group = RandomHead(3000, 64, 3), [5, 17, 400], 0.9, [7], [[11, 12], [13]], 6
    print(f"case: decode loop, {which} model, group {group}", flush=True)
    g_ref, g_ours = torch.Generator().manual_seed(42), torch.Generator().manual_seed(42)
    ref = [_reference_loop(model, prompt, 24, T, eos, stops, g_ref) for _ in range(group)]
    ours = generate_group_responses(model, prompt, group, 24, T, eos_token_id=eos, stop_token_sequences=stops,
                                    generator=g_ours)
    for (rr, rb, rreason, rc), (orr, ob, oreason, oc) in zip(ref, ours):
        assert rr == orr and rreason == oreason and rc == oc
        assert np.max(np.abs(np.array(rb) - np.array(ob))) <= 1e-5
    assert torch.equal(g_ref.get_state(), g_ours.get_state())


def test_decode_loop_finish_reasons_and_errors():
    model = TransitionModel([[-100.0, -100.0, 100.0]] * 3)  # always draws token 2
    resp, beh, reason, count = generate_response(model, [0], 5, 1.0, eos_token_id=2)
    assert resp == [2] and reason == "eos" and count == 1 and beh[0] <= 1e-6
    resp, _, reason, count = generate_response(model, [0], 5, 1.0, stop_token_sequences=[[2, 2]])
    assert resp == [2, 2] and reason == "stop" and count == 2
    resp, _, reason, count = generate_response(model, [0], 3, 1.0, draw="inverse_cdf")
    assert resp == [2, 2, 2] and reason == "length" and count == 0
    with pytest.raises(ValueError, match="outside the model vocabulary"):
        generate_response(model, [0], 3, 1.0, eos_token_id=3)
    with pytest.raises(ValueError, match="non-finite"):
        generate_response(TransitionModel([[float("nan"), 0.0, 0.0]] * 3), [0], 3, 1.0)
    with pytest.raises(ValueError, match="temperature"):
        generate_response(model, [0], 3, 0.0)
    with pytest.raises(ValueError, match="CPU torch.Generator"):
        generate_response(model, [0], 3, 1.0, generator=torch.Generator(device=DEV))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_sample_next_step_equals_sample(dtype):
    """sample_next's batch-1 inverse-CDF step (buffers kept across calls, uniform and outputs
    through a pinned host block, one synchronisation) returns what sample() returns for the
    same row and the same uniform, bit for bit, and leaves the generator where sample()'s
    torch.rand leaves it; a non-finite row raises the reference's message."""
    from dsv41_rocm import sample, sample_next
    g = torch.Generator().manual_seed(99)
    rows = (2.5 * torch.randn(12, 151936, generator=g)).to(dtype).to(DEV)
    ga, gb = torch.Generator().manual_seed(5), torch.Generator().manual_seed(5)
    for i in range(rows.shape[0]):
        T = (0.6, 1.0, 1.3)[i % 3]
        print(f"case: sample_next step {i} dtype={dtype} T={T}", flush=True)
        tok, lp = sample_next(rows[i], T, generator=ga)
        u = torch.rand(1, generator=gb)
        ref = sample(rows[i:i + 1], temperature=T, uniforms=u.to(DEV))
        assert tok == int(ref.ids[0])
        assert torch.tensor([lp], dtype=torch.float32).view(torch.int32) == ref.logprobs.cpu().view(torch.int32)
    assert torch.equal(ga.get_state(), gb.get_state())
    bad = rows[0].clone()
    bad[7] = float("nan")
    with pytest.raises(ValueError, match="generation log probabilities contain non-finite values"):
        sample_next(bad, 1.0, generator=ga)
    with pytest.raises(ValueError, match="temperature must be finite and positive"):
        sample_next(rows[0], 0.0, generator=ga)
