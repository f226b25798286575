"""Pins the C oracle of the sampler (oracle/sampler_oracle.c) without a GPU.

Every check compares the oracle with something it does not share code with: libm's exp,
Python's exact integers and fractions, torch's log_softmax in fp64, hand-derived penalty
values, brute force over every prefix on tiny vocabularies, and the known answers of the
reference's rollout tests (tests/golden/rollout_transition_model.json).
"""

import json
import math
import random
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle

GOLDEN = Path(__file__).parent / "golden"
TWO43 = 1 << 43


def test_exp_det_matches_libm_within_two_ulp():
    rng = random.Random(1)
    pts = [0.0, -1e-300, -0.5, -1.0, -math.log(2), -10.0, -29.9, -39.999] + [-40 * rng.random() for _ in range(20000)]
    for d in pts:
        e, ref = oracle.exp_det(d), math.exp(d)
        assert abs(e - ref) <= 2 * math.ulp(ref), (d, e, ref)
    assert oracle.exp_det(-40.0001) == 0.0 and oracle.exp_det(-1e9) == 0.0
    assert oracle.exp_det(float("nan")) == 0.0
    assert oracle.exp_det(0.25) == 1.0  # positive differences clamp to 0 (z never exceeds zmax)


def test_mass_is_floor_of_2_43_times_exp():
    # the mass is floor(2^43 exp(d)) of the fp32 difference d = z - zmax, evaluated in fp32:
    # against libm's exp of the same d it is within 2^-22 relative plus the floor's unit
    rng = random.Random(2)
    worst = 0.0
    for _ in range(20000):
        z, zmax = np.float32(rng.uniform(-30, 10)), np.float32(rng.uniform(10, 20))
        d = float(np.float32(z - zmax))
        q = oracle.mass(float(z), float(zmax))
        e = math.ldexp(math.exp(d), 43)
        assert abs(q - math.floor(e)) <= e * 2.0 ** -22 + 1, (z, zmax, q, e)
        if e > 1e7:
            worst = max(worst, abs(q - e) / e)
    assert worst <= 2.0 ** -22
    # every integer is exact where no rounding is involved
    assert oracle.mass(3.0, 3.0) == TWO43 and oracle.mass(-7.5, -7.5) == TWO43
    for n in range(0, 40):  # the reduction's edge cases: d = fl(-n ln 2), where r is near 0
        d = float(np.float32(-n * math.log(2)))
        e = math.ldexp(math.exp(d), 43)
        assert abs(oracle.mass(d, 0.0) - e) <= e * 2.0 ** -22 + 1
    # below -40 and for NaN the mass is 0; the masses are non-decreasing in z on a fine grid
    assert oracle.mass(-40.001, 0.0) == 0 and oracle.mass(float("nan"), 0.0) == 0
    assert oracle.mass(float("-inf"), 0.0) == 0
    grid = np.float32(-np.linspace(0, 39.9, 40001))[::-1]
    qs = [oracle.mass(float(v), 0.0) for v in grid]
    assert all(a <= b for a, b in zip(qs, qs[1:]))


def test_top_p_threshold_is_exact_ceiling():
    rng = random.Random(3)
    for _ in range(20000):
        p = float(np.float32(rng.choice([rng.random(), 0.95, 0.98, 0.5, 1e-6, 0.999999, 1.0])))
        if p <= 0.0:
            continue
        s = rng.randrange(1, 1 << 62)
        want = math.ceil(Fraction(p) * s)
        assert oracle.top_p_threshold(p, s) == want, (p, s)


def test_draw_target_is_exact():
    rng = random.Random(4)
    for _ in range(20000):
        u = float(np.float32(rng.random()))
        s = rng.randrange(1, 1 << 62)
        uu = math.floor(Fraction(u) * (1 << 32))
        assert oracle.draw_target(u, s) == (s * uu) >> 32
    assert oracle.draw_target(0.0, 12345) == 0


def test_penalties_hand_derived():
    # vLLM apply_penalties: repetition (divide positive, multiply non-positive), then
    # frequency * count, then presence, each rounded in fp32
    assert oracle.penalize(2.0, 1, 2.0, 0.0, 0.0) == 1.0
    assert oracle.penalize(-2.0, 1, 2.0, 0.0, 0.0) == -4.0
    assert oracle.penalize(0.0, 1, 2.0, 0.0, 0.0) == 0.0
    assert oracle.penalize(1.0, 3, 1.0, 0.0, 0.5) == -0.5
    assert oracle.penalize(1.0, 3, 1.0, 0.25, 0.5) == -0.75
    assert oracle.penalize(3.0, 2, 1.5, 0.5, 0.25) == 1.0  # 3/1.5 = 2; 2 - 0.5 - 0.5
    # an id of the prompt only (count 0 among the generated ids): repetition alone
    assert oracle.penalize(3.0, 0, 1.5, 0.5, 0.25) == 2.0
    assert oracle.penalize(-3.0, 0, 1.5, 0.5, 0.25) == -4.5
    x, c, rp, pres, freq = 1.2345678, 7, 1.1, 0.3, 0.07
    f32 = np.float32
    want = f32(f32(f32(x) / f32(rp)) - f32(f32(freq) * f32(c))) - f32(pres)
    assert oracle.penalize(x, c, rp, pres, freq) == float(want)


def test_prompt_ids_take_repetition_only():
    # vLLM's rule: repetition over prompt and output ids; frequency and presence count the
    # generated ids only.  History = prompt [1, 2, 2, 5] + generated [2, 3, 3], T = 1.
    x = np.array([1.0, 2.0, -1.0, 4.0, 0.5, -2.0, 3.0, 0.25], np.float32)
    hist = [1, 2, 2, 5, 2, 3, 3]
    rp, pres, freq = 2.0, 0.5, 0.25
    z, st = oracle.process_row(x, history=hist, history_prompt_len=4, repetition_penalty=rp,
                               presence_penalty=pres, frequency_penalty=freq)
    want = x.copy()
    want[1] = 2.0 / 2.0                       # prompt only: repetition
    want[5] = -2.0 * 2.0                      # prompt only, negative logit
    want[2] = -1.0 * 2.0 - 0.25 * 1 - 0.5     # prompt and generated once
    want[3] = 4.0 / 2.0 - 0.25 * 2 - 0.5      # generated twice
    assert st == 0 and np.array_equal(z, want), (z, want)
    # without the split every entry counts as generated
    z0, _ = oracle.process_row(x, history=hist, repetition_penalty=rp, presence_penalty=pres, frequency_penalty=freq)
    assert z0[1] == 1.0 - 0.25 - 0.5 and z0[2] == -2.0 - 0.75 - 0.5 and z0[3] == 2.0 - 0.5 - 0.5
    # the whole history as prompt: repetition alone everywhere
    zp, _ = oracle.process_row(x, history=hist, history_prompt_len=7, repetition_penalty=rp, presence_penalty=pres,
                               frequency_penalty=freq)
    zr, _ = oracle.process_row(x, history=hist, repetition_penalty=rp)
    assert np.array_equal(zp, zr)


@pytest.mark.parametrize("T", [0.6, 0.7, 1.3, 0.1, 7.77])
def test_three_operation_division_is_ieee_on_guarded_range(T):
    # the kernel divides by T with q = x*r, e = fma(-q, T, x), z = fma(e, r, q) when
    # 2^-100 <= |x| < 2^100; 256 windows of 65536 consecutive bit patterns spread over
    # that range (both signs, both edges included) must match IEEE division
    win = 65536
    for lo, hi in ((0x0D800000, 0x71800000), (0x8D800000, 0xF1800000)):
        starts = [lo + (hi - lo - win) * i // 255 for i in range(256)]
        bad = sum(oracle.check_division(T, s, s + win)[0] for s in starts)
        assert bad == 0


def test_division_scheme_fails_below_the_guard():
    # the guard exists because the residual underflows for tiny |x|
    n, first = oracle.check_division(0.7, 0x00000001, 0x00800000)
    assert n > 0 and first < 0x00800000


def _row_reference_lp(x, T, tok):
    z = torch.tensor(x, dtype=torch.float32) / T
    return float(torch.log_softmax(z.double(), dim=-1)[tok])


def test_full_vocab_logprob_is_log_softmax_of_scaled_logits():
    rng = np.random.default_rng(5)
    x = (3 * rng.standard_normal((16, 5000))).astype(np.float32)
    u = rng.random(16).astype(np.float32)
    ids, lps, kept, st = oracle.sample(x, uniforms=u, temperature=0.7)
    assert (st == 0).all() and (kept == 5000).all()
    for r in range(16):
        assert abs(lps[r] - _row_reference_lp(x[r], np.float32(0.7), ids[r])) <= 1e-5


def test_draw_is_inverse_cdf_in_vocabulary_order():
    # brute force: with exact integer masses the drawn token is the first whose
    # cumulative mass exceeds floor(u * 2^32) * S >> 32
    rng = np.random.default_rng(6)
    for _ in range(300):
        V = int(rng.integers(1, 9))
        x = rng.standard_normal((1, V)).astype(np.float32)
        u = np.array([rng.random()], np.float32)
        ids, _, _, _ = oracle.sample(x, uniforms=u, temperature=1.0)
        zmax = float(x[0].max())
        q = [oracle.mass(float(v), zmax) for v in x[0]]  # the mass itself is pinned above
        t = (sum(q) * math.floor(Fraction(float(u[0])) * (1 << 32))) >> 32
        cum, want = 0, None
        for i, qi in enumerate(q):
            cum += qi
            if cum > t:
                want = i
                break
        assert ids[0] == want


def _brute_kept(z, k, p, min_p):
    """Independent restatement with Python sorting and exact fractions."""
    V = len(z)
    zmax = max(z)
    order = sorted(range(V), key=lambda i: (-float(z[i]), i))
    if min_p > 0:
        lm = math.log(float(np.float32(min_p)))
        order = [i for i in order if float(z[i]) - zmax >= lm]
    if 0 < k < len(order):
        order = order[:k]
    if p < 1:
        q = [oracle.mass(float(z[i]), float(zmax)) for i in order]  # pinned by the mass test
        thr = math.ceil(Fraction(float(np.float32(p))) * sum(q))
        cum = 0
        for n, qi in enumerate(q):
            cum += qi
            if cum >= thr:
                order = order[:n + 1]
                break
    return sorted(order)


def test_kept_sets_match_brute_force_on_tiny_vocabularies():
    rng = np.random.default_rng(7)
    for trial in range(600):
        V = int(rng.integers(1, 13))
        # coarse values so that ties are common
        x = (np.round(rng.standard_normal(V) * 2) / 2).astype(np.float32)
        k = int(rng.integers(0, V + 2))
        p = float(rng.choice([1.0, 0.9, 0.5, 0.3]))
        mp = float(rng.choice([0.0, 0.0, 0.2, 0.6]))
        T = float(rng.choice([1.0, 0.7]))
        z = (x / np.float32(T)).astype(np.float32)
        want = _brute_kept(z, k, p, mp)
        # greedy reveals nothing about the kept set, so draw with u at each kept item
        _, _, kept, st = oracle.sample(x[None], uniforms=np.array([0.5], np.float32), temperature=T, top_k=k,
                                       top_p=p, min_p=mp)
        assert st[0] == 0 and kept[0] == len(want), (trial, x, k, p, mp)
        # every kept token is drawable and only kept tokens are drawn
        seen = set()
        for u in np.linspace(0, 1, 97, endpoint=False):
            ids, _, _, _ = oracle.sample(x[None], uniforms=np.array([u], np.float32), temperature=T, top_k=k,
                                         top_p=p, min_p=mp)
            seen.add(int(ids[0]))
        assert seen <= set(want)


def test_identities_and_greedy_first_max():
    rng = np.random.default_rng(8)
    x = rng.standard_normal((6, 300)).astype(np.float32)
    x[:, 10] = x[:, 200] = x.max() + 1  # tie: greedy must pick index 10
    u = rng.random(6).astype(np.float32)
    base = oracle.sample(x, uniforms=u)
    for knobs in (dict(top_k=300), dict(top_k=10 ** 6), dict(top_p=1.0), dict(min_p=0.0)):
        got = oracle.sample(x, uniforms=u, **knobs)
        assert np.array_equal(got[0], base[0]) and np.array_equal(got[2], base[2])
    ids, _, _, _ = oracle.sample(x, greedy=True)
    assert (ids == 10).all()
    assert (ids == torch.argmax(torch.from_numpy(x), dim=1).numpy()).all()
    ids, _, kept, _ = oracle.sample(x, uniforms=u, top_k=1)
    assert (ids == 10).all() and (kept == 1).all()


def test_status_rows():
    x = np.zeros((4, 10), np.float32)
    x[1, 3] = np.nan
    x[2, 0] = -np.inf
    h = np.zeros((4, 2), np.int64)
    h[3, 0] = 99
    u = np.array([0.5, 0.5, 0.5, 1.0], np.float32)
    ids, lps, kept, st = oracle.sample(x, uniforms=u, history=h, repetition_penalty=1.2)
    assert list(st) == [0, 1, 1, 2 | 4]
    assert ids[1] == -1 and ids[2] == -1 and np.isnan(lps[1])


def test_reference_rollout_toy_model_known_answers():
    g = json.loads((GOLDEN / "rollout_transition_model.json").read_text())
    T = g["temperature"]
    rows = np.array(g["transitions"], np.float32)
    for r in range(3):
        for u in np.linspace(0, 1, 40, endpoint=False):
            ids, lps, _, _ = oracle.sample(rows[r:r + 1], uniforms=np.array([u], np.float32), temperature=T)
            # behaviour log-prob equals teacher forcing (test_rl_rollout.py:48-57)
            assert abs(lps[0] - _row_reference_lp(rows[r], np.float32(T), ids[0])) <= 1e-6
    eos = np.array([g["always_eos_row"]], np.float32)
    ids, _, _, _ = oracle.sample(eos, uniforms=np.array([0.999], np.float32), temperature=T)
    assert ids[0] == 2
    zeros = np.zeros((1, 3), np.float32)
    seen = {int(oracle.sample(zeros, uniforms=np.array([u], np.float32), temperature=T)[0][0])
            for u in np.linspace(0, 1, 30, endpoint=False)}
    assert seen == {0, 1, 2}  # every vocabulary token is reachable (test_rl_rollout.py:105-110)


def test_torch_multinomial_is_an_exponential_race_on_the_cpu():
    """The library behaviour the exponential-race draw relies on (torch, not the reference):
    torch.multinomial(p, 1, generator=g) on the CPU equals argmax(p / E) with
    E = empty_like(p).exponential_(1, generator=g), leaves g in the same state, and filling
    [rows, V] at once consumes the stream as rows one after another."""
    for V in (3, 1000, 151936):
        for seed in range(20 if V < 151936 else 2):
            p = torch.softmax(3 * torch.randn(V, generator=torch.Generator().manual_seed(100 + seed)), 0)
            g1, g2 = torch.Generator().manual_seed(seed), torch.Generator().manual_seed(seed)
            a = int(torch.multinomial(p, 1, generator=g1))
            b = int(torch.argmax(p / torch.empty_like(p).exponential_(1, generator=g2)))
            assert a == b and torch.equal(g1.get_state(), g2.get_state())
    g1, g2 = torch.Generator().manual_seed(9), torch.Generator().manual_seed(9)
    bulk = torch.empty(4, 5000).exponential_(1, generator=g1)
    rows = torch.stack([torch.empty(5000).exponential_(1, generator=g2) for _ in range(4)])
    assert torch.equal(bulk, rows) and torch.equal(g1.get_state(), g2.get_state())


def _draw_intervals(z, **kw):
    """For every id, how many 32-bit uniforms U draw it: the draw is a non-decreasing step
    function of U, so a binary search finds the first U of each id."""
    V = len(z)
    firsts = []
    lo = 0
    for v in range(V + 1):
        a, b = lo, 1 << 32  # smallest U in [a, b] whose draw is >= v (U = 2^32 stands for "none")
        while a < b:
            mid = (a + b) // 2
            if oracle.full_draw(z, mid, **kw) >= v:
                b = mid
            else:
                a = mid + 1
        firsts.append(a)
        lo = a
    return np.diff(np.array(firsts, dtype=np.int64))


def _softmax64(z):
    z = np.asarray(z, dtype=np.float64)
    e = np.exp(z - z.max())
    return e / e.sum()


@pytest.mark.parametrize("case", ["plain", "history", "slices_aligned", "slices_ragged"])
def test_full_draw_intervals_are_the_softmax(case):
    """The full-vocabulary inverse-CDF draw over 256-id chunk masses (each chunk's masses
    against its own maximum, scaled exactly to the row maximum; history ids against the row
    maximum): the share of the 2^32 uniforms that draws each id equals softmax(z) in fp64
    within fp32 accuracy.  Chunks sit at different heights (+3, 0, -5 and a far chunk at
    -60 that must get nothing), so a missing or wrong chunk scale shows as a factor of
    e^3 or more; the history case puts the row maximum on a history id."""
    g = np.random.default_rng(17)
    z = (2.0 * g.standard_normal(900)).astype(np.float32)
    z[:256] += 3.0
    z[512:768] -= 5.0
    z[768:] -= 60.0
    kw = {}
    if case == "history":
        hist = g.choice(900, size=60, replace=False)
        hist[0] = int(np.argmax(z))
        kw["history_ids"] = hist
    if case == "slices_aligned":
        kw["slice_starts"] = [0, 256, 768]
    if case == "slices_ragged":
        kw["slice_starts"] = [0, 301, 611]
    lengths = _draw_intervals(z, **kw)
    assert lengths.sum() == 1 << 32 and (lengths >= 0).all()
    p = _softmax64(z)
    share = lengths / float(1 << 32)
    assert np.all(np.abs(share - p) <= 2e-6 * p + 5e-10), np.max(np.abs(share - p) / (p + 1e-30))
    assert lengths[768:].sum() == 0  # e^-60 relative to the maximum: below the 2^-43 resolution
    if case == "slices_aligned":
        # chunks restarting at multiples of 256 are the unsliced chunks: the same draw
        assert np.array_equal(lengths, _draw_intervals(z))


@pytest.mark.parametrize("case", ["plain", "history", "slices_aligned", "slices_ragged"])
def test_full_total_is_the_softmax_normalizer(case):
    """The exact total S every full-vocabulary draw reports its log-prob against:
    S 2^-43 = sum exp(z - zmax) within fp32 accuracy on rows whose chunks sit at different
    heights (+3, 0, -5, -60), so a missing or wrong chunk scale is off by a factor e^3 or
    more and a dropped history mass by the history's share (the row maximum is on a history
    id).  Slices cut at multiples of 256 are the unsliced chunks: the same integer."""
    g = np.random.default_rng(23)
    z = (2.0 * g.standard_normal(900)).astype(np.float32)
    z[:256] += 3.0
    z[512:768] -= 5.0
    z[768:] -= 60.0
    kw = {}
    if case == "history":
        hist = g.choice(900, size=60, replace=False)
        hist[0] = int(np.argmax(z))
        kw["history_ids"] = hist
    if case == "slices_aligned":
        kw["slice_starts"] = [0, 256, 768]
    if case == "slices_ragged":
        kw["slice_starts"] = [0, 301, 611]
    S = oracle.full_total(z, **kw)
    e = np.exp(z.astype(np.float64) - float(z.max())).sum()
    assert abs(S * 2.0**-43 - e) <= 2e-6 * e
    if case == "slices_aligned":
        assert S == oracle.full_total(z)


def test_full_total_single_chunk_is_the_sum_of_masses():
    """At most 256 ids without history: one chunk whose maximum is the row maximum, so S is
    the plain sum of floor(2^43 exp32(z - zmax)), and the maximum alone weighs 2^43."""
    g = np.random.default_rng(5)
    for V in (1, 7, 256):
        z = (3.0 * g.standard_normal(V)).astype(np.float32)
        zmax = float(z.max())
        assert oracle.full_total(z) == sum(oracle.mass(float(v), zmax) for v in z)
    assert oracle.full_total(np.array([2.5], np.float32)) == 1 << 43


def test_full_draw_single_chunk_is_the_plain_inverse_cdf():
    """A row of at most 256 ids without history is one chunk whose maximum is the row
    maximum: its masses are floor(2^43 exp32(z - zmax)) in vocabulary order, the
    single-level inverse CDF, for every uniform of a sweep."""
    g = np.random.default_rng(3)
    z = g.standard_normal(200).astype(np.float32)
    zmax = float(z.max())
    q = np.array([oracle.mass(float(v), zmax) for v in z], dtype=object)
    cum = np.cumsum(q)
    S = int(cum[-1])
    for U in list(range(0, 1 << 32, (1 << 32) // 997)) + [(1 << 32) - 1]:
        t = (S * U) >> 32
        want = int(np.argmax(cum > t))
        assert oracle.full_draw(z, U) == want
