"""Replay of behaviour log-probs (a10): the reference requires the log-prob a policy reports
when it replays an action to equal the one recorded when the action was sampled, bit for bit
(tests/test_qwen_kv_cache.py:76-77 in the Tiny-DSV41 tree).  replay_log_probs on the same
logits, temperature and penalties must return exactly the float that sample reported for the
drawn token, whichever draw produced it; and it must agree with torch's
log_softmax(logits / T)[token] within 1e-5 where no penalties apply.
"""

import numpy as np
import pytest
import torch

import oracle
from dsv41_rocm import replay_log_probs, sample, workloads

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


@pytest.mark.parametrize("name,rows,draw", [("B", 64, "cdf"), ("B", 64, "race"), ("B", 64, "greedy"),
                                            ("E", 32, "cdf"), ("A", 8, "race")])
def test_replay_equals_behaviour_bitwise(name, rows, draw):
    inp = workloads.sampler_inputs(name, rows=rows, device=DEV)
    x, h = inp["logits"], inp["history"]
    pen = {k: v for k, v in inp["knobs"].items()
           if k in ("temperature", "repetition_penalty", "presence_penalty", "frequency_penalty")}
    print(f"case: config {name} rows {rows} draw {draw} knobs {pen}", flush=True)
    g = torch.Generator().manual_seed(rows)
    if draw == "race":
        e = torch.empty(x.shape, dtype=torch.float32).exponential_(1, generator=g)
        res = sample(x, history=h, exponentials=e, **pen)
    elif draw == "greedy":
        res = sample(x, history=h, greedy=True, **pen)
    else:
        res = sample(x, history=h, generator=g, **pen)
    lp = replay_log_probs(x, res.ids, history=h, **pen)
    assert torch.equal(lp, res.logprobs)


@pytest.mark.parametrize("draw", ["cdf", "race", "greedy"])
def test_log_prob_is_against_the_exact_mass_total(draw):
    """Every full-vocabulary draw reports lp = (z_tok - M) - log(S 2^-43), S the exact
    integer total of the draw's 2^-43 masses: the float equals the one formed from the
    oracle's processed row and its S (the fp64 logs of the two sides agree far below the
    float's rounding), on config B's rows with their penalties."""
    inp = workloads.sampler_inputs("B", rows=24)
    x, h, knobs = inp["logits"], inp["history"], inp["knobs"]
    print(f"case: config B rows 24 draw {draw}", flush=True)
    g = torch.Generator().manual_seed(11)
    kw = {}
    if draw == "race":
        kw["exponentials"] = torch.empty(x.shape, dtype=torch.float32).exponential_(1, generator=g).to(DEV)
    elif draw == "greedy":
        kw["greedy"] = True
    else:
        kw["uniforms"] = inp["uniforms"].to(DEV)
    res = sample(x.to(DEV), history=h.to(DEV), **knobs, **kw)
    ids, lps = res.ids.cpu().numpy(), res.logprobs.cpu().numpy()
    assert (res.status.cpu() == 0).all()
    xf = x.float().numpy()
    for r in range(x.shape[0]):
        z, st = oracle.process_row(xf[r], temperature=knobs["temperature"], history=h[r].numpy(),
                                   presence_penalty=knobs["presence_penalty"],
                                   frequency_penalty=knobs["frequency_penalty"])
        assert st == 0
        S = oracle.full_total(z, history_ids=np.unique(h[r].numpy()))
        want = np.float32((np.float64(z[ids[r]]) - np.float64(z.max())) - np.log(float(S) * 2.0**-43))
        assert lps[r] == want, (r, lps[r], want)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("vocab", [1, 255, 256, 257, 151936, 2097151])
def test_log_prob_total_closed_forms(vocab, dtype):
    """The exact total in closed form.  Equal logits: every id weighs 2^43, so S = V 2^43 and
    every draw reports lp = -log V.  Two levels (k ids at 0, the rest at -d): an all-low chunk
    weighs its count times g = floor(2^43 exp32(-d)) exactly, and a mixed chunk holds its
    masses unscaled, so S = k 2^43 + (V - k) g whatever the chunking, and the drawn id reports
    z_tok - log(S 2^-43).  Ids at -60 weigh nothing.  The floats must be those of numpy's fp64
    log, bit for bit, for the inverse CDF, the race, greedy and the replay, on fp32 and bf16
    rows (the three values are exact in both)."""
    g = torch.Generator().manual_seed(vocab)
    rows = 3
    x = torch.zeros(rows, vocab)
    k = max(1, vocab // 1000)
    top = torch.randperm(vocab, generator=g)[:k]
    x[1] = -7.25
    x[1, top] = 0.0
    x[2] = -60.0  # below the 2^-43 resolution: the low ids weigh nothing
    x[2, top] = 0.0
    print(f"case: vocab {vocab} top ids {k} dtype {dtype}", flush=True)
    gm = oracle.mass(-7.25, 0.0)
    totals = [vocab << 43, (k << 43) + (vocab - k) * gm, k << 43]  # S per row, exact integers
    xd = x.to(dtype).to(DEV)
    draws = {
        "cdf": sample(xd, uniforms=torch.rand(rows, generator=g).to(DEV)),
        "race": sample(xd, exponentials=torch.empty(rows, vocab).exponential_(1, generator=g).to(DEV)),
        "greedy": sample(xd, greedy=True),
    }
    for name, res in draws.items():
        ids = res.ids.cpu()
        lp = res.logprobs.cpu().numpy()
        assert (res.status.cpu() == 0).all(), name
        ztok = x.gather(1, ids[:, None])[:, 0].double().numpy()
        assert ztok[2] == 0.0, name  # the ids at -60 carry no mass
        want = np.array([np.float32(z - np.log(float(S) * 2.0**-43)) for z, S in zip(ztok, totals)])
        assert np.array_equal(lp, want), (name, lp, want)
        assert torch.equal(replay_log_probs(xd, res.ids).cpu(), res.logprobs.cpu()), name


def test_replay_matches_torch_log_softmax_and_any_token():
    g = torch.Generator().manual_seed(4)
    x = (3.0 * torch.randn(16, 50021, generator=g)).to(DEV)
    tok = torch.randint(0, 50021, (16,), generator=g).to(DEV)
    for T in (0.6, 1.0, 1.7):
        lp = replay_log_probs(x, tok, temperature=T)
        ref = torch.log_softmax(x.double() / T, dim=-1).gather(1, tok[:, None])[:, 0]
        assert float((lp.double() - ref).abs().max()) <= 1e-5


def test_replay_bad_ids_and_nonfinite_rows():
    x = torch.randn(3, 1000, device=DEV)
    with pytest.raises(ValueError, match="outside the model vocabulary"):
        replay_log_probs(x, torch.tensor([0, 1000, 5]))
    lp = replay_log_probs(x, torch.tensor([0, -1, 5]), check=False)
    assert torch.isnan(lp[1]) and torch.isfinite(lp[0]) and torch.isfinite(lp[2])
    x[2, 7] = float("nan")
    with pytest.raises(ValueError, match="non-finite"):
        replay_log_probs(x, torch.tensor([0, 1, 5]))
    with pytest.raises(ValueError, match="one token ID"):
        replay_log_probs(x, torch.tensor([0, 1]))
