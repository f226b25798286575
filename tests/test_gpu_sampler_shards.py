"""GPU parity of vocabulary-sharded sampling: the logits of a batch split into slices of a
tensor-parallel head, each slice's candidate list (dsv41_sampler_shard_run), then the exact
merge (dsv41_sampler_merge_run), all on one GPU.  The merged ids, kept sets and statuses
must equal the unsharded sampler's and the C oracle's; log-probs agree within 1e-6 with the
unsharded sampler (the kept-set sum may run in another order) and 1e-4 with the oracle.

Full-vocabulary draws over slices (dsv41_sampler_full_state_run, _draw_run, _finish_run):
greedy ids equal the unsharded sampler's.  Inverse-CDF ids equal the C oracle's run with the
same slice starts (the exact masses come in 256-id chunks that restart at each slice start),
and the unsharded sampler's whenever the slice starts are multiples of 256; with other
starts, and for the race (whose p / E come from another sum order), they agree on >= 99.9%
of rows.  Log-probs agree within 1e-5 with the unsharded sampler and 1e-4 with the oracle.
"""

import numpy as np
import pytest
import torch

import oracle
from dsv41_rocm import (full_shard_draw, full_shard_finish, full_shard_masses, full_shard_states, merge_shards,
                        sample, sample_shard,
                        workloads)

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def edges(vocab, n, seed, align=1):
    """n ragged slices covering [0, vocab), cut at multiples of ``align``."""
    g = torch.Generator().manual_seed(seed)
    cuts = sorted(torch.randperm((vocab - 1) // align, generator=g)[: n - 1].add(1).mul(align).tolist())
    return [0] + cuts + [vocab]


def run_sharded(logits, bounds, uniforms=None, history=None, greedy=False, **knobs):
    sk = {k: v for k, v in knobs.items() if k != "greedy"}
    shards = []
    for a, b in zip(bounds[:-1], bounds[1:]):
        print(f"case: slice [{a}, {b}) of {logits.shape[1]} knobs={knobs}", flush=True)
        shards.append(sample_shard(logits[:, a:b], vocab_offset=a, vocab_size=logits.shape[1],
                                   history=history, **sk))
    merged = merge_shards(shards, top_k=knobs["top_k"], top_p=knobs.get("top_p", 1.0),
                          min_p=knobs.get("min_p", 0.0), uniforms=uniforms, greedy=greedy, check=False)
    torch.cuda.synchronize()
    return merged, shards


def assert_same(merged, whole, ora=None):
    for name in ("ids", "kept", "status"):
        assert torch.equal(getattr(merged, name), getattr(whole, name)), name
    ok = (whole.status == 0)
    diff = (merged.logprobs - whole.logprobs)[ok].abs()
    assert diff.numel() == 0 or float(diff.max()) <= 1e-6
    if ora is not None:
        oids, olp, okept, ost = ora
        np.testing.assert_array_equal(merged.status.cpu().numpy(), ost)
        okr = ost == 0
        np.testing.assert_array_equal(merged.ids.cpu().numpy()[okr], oids[okr])
        np.testing.assert_array_equal(merged.kept.cpu().numpy()[okr], okept[okr])
        assert np.max(np.abs(merged.logprobs.cpu().numpy()[okr] - olp[okr]), initial=0.0) <= 1e-4


@pytest.mark.parametrize("n_shards", [2, 8])
def test_config_e_split_over_slices(n_shards):
    inp = workloads.sampler_inputs("E", rows=96, device=DEV)
    x, u, h, knobs = inp["logits"], inp["uniforms"], inp["history"], inp["knobs"]
    bounds = edges(x.shape[1], n_shards, seed=n_shards)
    merged, shards = run_sharded(x, bounds, uniforms=u, history=h, **knobs)
    whole = sample(x, uniforms=u, history=h, check=False, **knobs)
    ora = oracle.sample(x.float().cpu().numpy(), uniforms=u.cpu().numpy(), history=h.cpu().numpy(), **knobs)
    assert_same(merged, whole, ora)
    # what crosses the wire: at most top_k keys per row and slice, typically a few dozen
    assert all(int(s.counts.max()) <= knobs["top_k"] for s in shards)


@pytest.mark.parametrize("knobs", [
    dict(temperature=0.7, top_k=40, top_p=0.9, repetition_penalty=1.3),                # lowering, bitmap only
    dict(temperature=1.1, top_k=200, min_p=0.02, presence_penalty=0.5, frequency_penalty=0.2),  # with counts
    dict(temperature=0.8, top_k=30, repetition_penalty=0.8, presence_penalty=-0.3),    # raising: gathered
    dict(temperature=0.9, top_k=1),
    dict(temperature=0.6, top_k=50, greedy=True),
])
def test_knobs_and_penalties_across_slices(knobs):
    g = torch.Generator().manual_seed(17)
    rows, V = 40, 20011
    x = (2.0 * torch.randn(rows, V, generator=g)).to(DEV)
    u = torch.rand(rows, generator=g).to(DEV)
    h = torch.randint(-1, V, (rows, 500), generator=g).to(DEV)
    bounds = edges(V, 5, seed=3)
    greedy = knobs.get("greedy", False)
    merged, _ = run_sharded(x, bounds, uniforms=None if greedy else u, history=h, **knobs)
    whole = sample(x, uniforms=None if greedy else u, history=h, check=False, **knobs)
    ora = oracle.sample(x.cpu().numpy(), uniforms=None if greedy else u.cpu().numpy(), history=h.cpu().numpy(),
                        **knobs)
    assert_same(merged, whole, ora)


def test_bf16_flat_rows_statuses_and_the_block_merge():
    """bf16 slices; flat rows whose merged lists exceed one wave (the block merge); a NaN in
    one slice, an id past the vocabulary and a bad uniform flag their rows as unsharded."""
    g = torch.Generator().manual_seed(29)
    rows, V = 24, 30000
    x = 3.0 * torch.randn(rows, V, generator=g)
    x[::3] = 0.001 * torch.randn((rows + 2) // 3, V, generator=g)
    x[4, 12345] = float("nan")
    x = x.to(torch.bfloat16).to(DEV)
    u = torch.rand(rows, generator=g)
    u[5] = 1.5
    u = u.to(DEV)
    h = torch.randint(0, V, (rows, 64), generator=g)
    h[6, 3] = V + 7
    h = h.to(DEV)
    knobs = dict(temperature=0.9, top_k=400, top_p=0.95, repetition_penalty=1.1)
    bounds = edges(V, 6, seed=5)
    bounds = sorted(set(bounds + [bounds[1] + 100]))  # one slice narrower than top_k
    merged, shards = run_sharded(x, bounds, uniforms=u, history=h, **knobs)
    whole = sample(x, uniforms=u, history=h, check=False, **knobs)
    assert_same(merged, whole)
    st = merged.status.cpu().tolist()
    assert st[4] & 1 and st[5] & 4 and st[6] & 2
    assert int(sum(s.counts for s in shards)[0]) > 256  # row 0 is flat: the block path merged it
    with pytest.raises(ValueError, match="non-finite"):
        merge_shards(shards, top_k=400, top_p=0.95, uniforms=u)


def run_full_sharded(logits, bounds, draw, uniforms=None, exponentials=None, history=None, **knobs):
    """The steps of a full-vocabulary draw over the slices ``bounds`` on one GPU; the lists of
    states, masses and picks stand for what the all-gathers would deliver."""
    V = logits.shape[1]
    slices = list(enumerate(zip(bounds[:-1], bounds[1:])))
    states = []
    for _, (a, b) in slices:
        print(f"case: full-vocabulary slice [{a}, {b}) of {V} draw={draw} knobs={knobs}", flush=True)
        states.append(full_shard_states(logits[:, a:b], vocab_offset=a, vocab_size=V, history=history, **knobs))
    masses = None
    if draw == "inverse_cdf":
        masses = [full_shard_masses(logits[:, a:b], states, shard_index=i, vocab_offset=a, vocab_size=V,
                                    history=history, **knobs) for i, (a, b) in slices]
    picks = None
    if draw != "greedy":
        picks = [full_shard_draw(logits[:, a:b], states, masses, shard_index=i, vocab_offset=a, vocab_size=V,
                                 uniforms=uniforms, history=history,
                                 exponentials=None if exponentials is None else exponentials[:, a:b], **knobs)
                 for i, (a, b) in slices]
    res = full_shard_finish(states, picks, vocab_size=V, draw=draw, uniforms=uniforms, check=False)
    torch.cuda.synchronize()
    return res


def assert_full_close(res, whole, exact_ids, bounds=None):
    """``exact_ids``: an inverse-CDF or greedy draw, whose ids equal the unsharded ones when
    every slice starts at a multiple of 256 (the mass chunks are then the same)."""
    assert torch.equal(res.status, whole.status)
    assert torch.equal(res.kept, whole.kept)
    ok = whole.status == 0
    same = (res.ids == whole.ids) & ok
    if exact_ids and bounds is not None and any(b % 256 for b in bounds[:-1]):
        exact_ids = False
    if exact_ids:
        assert bool(same[ok].all())
    else:
        assert float(same[ok].float().mean()) >= 0.999
    diff = (res.logprobs - whole.logprobs)[same].abs()
    assert diff.numel() == 0 or float(diff.max()) <= 1e-5


@pytest.mark.parametrize("n_shards", [2, 8])
@pytest.mark.parametrize("draw", ["inverse_cdf", "exponential_race", "greedy"])
@pytest.mark.parametrize("where", ["cpu", "gpu"])
def test_config_b_full_vocabulary_draw_over_slices(n_shards, draw, where):
    """Config B over 2 ragged slices and 8 slices cut at multiples of 256, on the
    CPU-generated batch and on a GPU-generated one.  Greedy ids, and inverse-CDF ids over the
    aligned slices, equal the unsharded sampler's; inverse-CDF ids equal the oracle's with
    the same slice starts; the race forms p / E from a different sum order, so its ids may
    differ where two ratios lie within an ulp."""
    inp = workloads.sampler_inputs("B", device="cpu" if where == "cpu" else DEV,
                                   seed=None if where == "cpu" else 4242)
    x, u, h, knobs = inp["logits"].to(DEV), inp["uniforms"].to(DEV), inp["history"].to(DEV), inp["knobs"]
    bounds = edges(x.shape[1], n_shards, seed=10 + n_shards, align=256 if n_shards == 8 else 1)
    e = None
    if draw == "exponential_race":
        g = torch.Generator().manual_seed(77)
        e = torch.empty(x.shape, dtype=torch.float32).exponential_(1, generator=g).to(DEV)
    res = run_full_sharded(x, bounds, draw, uniforms=u if draw == "inverse_cdf" else None, exponentials=e,
                           history=h, **knobs)
    whole = sample(x, uniforms=u, history=h, greedy=draw == "greedy", exponentials=e, check=False, **knobs)
    assert_full_close(res, whole, exact_ids=draw != "exponential_race", bounds=bounds)
    if draw == "inverse_cdf":
        oids, olp, okept, ost = oracle.sample(x.float().cpu().numpy(), uniforms=u.cpu().numpy(),
                                              history=h.cpu().numpy(), slice_starts=bounds[:-1], **knobs)
        np.testing.assert_array_equal(res.status.cpu().numpy(), ost)
        np.testing.assert_array_equal(res.ids.cpu().numpy(), oids)
        assert np.max(np.abs(res.logprobs.cpu().numpy() - olp)) <= 1e-4


@pytest.mark.parametrize("draw", ["inverse_cdf", "exponential_race", "greedy"])
def test_full_vocabulary_slices_fp32_unaligned_and_statuses(draw):
    """fp32 rows over three slices whose edges are not 16-byte aligned; a NaN in one slice, a
    history id past the vocabulary and (inverse CDF) a bad uniform flag their rows."""
    g = torch.Generator().manual_seed(5)
    rows, V = 24, 5003
    x = 2.0 * torch.randn(rows, V, generator=g)
    x[3, 2500] = float("nan")
    h = torch.randint(0, V, (rows, 40), generator=g)
    h[5, 7] = V + 3
    u = torch.rand(rows, generator=g)
    u[7] = 1.5
    e = torch.empty(rows, V).exponential_(1, generator=g).to(DEV) if draw == "exponential_race" else None
    x, h, u = x.to(DEV), h.to(DEV), u.to(DEV)
    knobs = dict(temperature=0.8, repetition_penalty=1.2, presence_penalty=0.3, frequency_penalty=0.1)
    bounds = [0, 1237, 3001, V]
    res = run_full_sharded(x, bounds, draw, uniforms=u if draw == "inverse_cdf" else None, exponentials=e,
                           history=h, **knobs)
    whole = sample(x, uniforms=u, history=h, greedy=draw == "greedy", exponentials=e, check=False, **knobs)
    st = res.status.cpu()
    assert st[3] & 1 and int(res.ids[3]) == -1 and st[5] & 2
    if draw == "inverse_cdf":
        assert st[7] & 4
        oids, olp, okept, ost = oracle.sample(x.cpu().numpy(), uniforms=u.cpu().numpy(), history=h.cpu().numpy(),
                                              slice_starts=bounds[:-1], **knobs)
        np.testing.assert_array_equal(st.numpy(), ost)
        np.testing.assert_array_equal(res.ids.cpu().numpy(), oids)
    assert_full_close(res, whole, exact_ids=draw != "exponential_race", bounds=bounds)



@pytest.mark.parametrize("draw", ["top_k", "inverse_cdf", "greedy"])
def test_prompt_history_split_over_slices(draw):
    """History = prompt ids + generated ids with per-row prompt lengths (repetition for both,
    frequency and presence for the generated ids only): the slices reach the unsharded
    sampler's ids, kept sets and statuses."""
    g = torch.Generator().manual_seed(33)
    rows, V, L = 16, 30011, 300
    x = (2.0 * torch.randn(rows, V, generator=g)).to(DEV)
    h = torch.randint(0, V, (rows, L), generator=g)
    h[:, 200:] = h[:, :100]
    h = h.to(DEV)
    plens = torch.randint(0, L + 1, (rows,), generator=g).to(torch.int32).to(DEV)
    u = torch.rand(rows, generator=g).to(DEV)
    pen = dict(temperature=0.9, repetition_penalty=1.25, presence_penalty=0.5, frequency_penalty=0.2)
    bounds = edges(V, 4, seed=4)
    if draw == "top_k":
        knobs = dict(top_k=40, top_p=0.9, **pen)
        merged, _ = run_sharded(x, bounds, uniforms=u, history=h, history_prompt_lens=plens, **knobs)
        whole = sample(x, uniforms=u, history=h, history_prompt_lens=plens, check=False, **knobs)
        assert_same(merged, whole)
        return
    res = run_full_sharded(x, bounds, draw, uniforms=u if draw == "inverse_cdf" else None, history=h,
                           history_prompt_lens=plens, **pen)
    whole = sample(x, uniforms=u, history=h, history_prompt_lens=plens, greedy=draw == "greedy", check=False, **pen)
    assert_full_close(res, whole, exact_ids=True, bounds=bounds)
    if draw == "inverse_cdf":
        oids, _, _, ost = oracle.sample(x.cpu().numpy(), uniforms=u.cpu().numpy(), history=h.cpu().numpy(),
                                        history_prompt_lens=plens.cpu().numpy(), slice_starts=bounds[:-1], **pen)
        np.testing.assert_array_equal(res.status.cpu().numpy(), ost)
        np.testing.assert_array_equal(res.ids.cpu().numpy(), oids)


def test_masses_that_no_slice_holds_flag_the_row():
    """The inverse-CDF draw step places the token against masses gathered from every slice.
    When they come from other inputs than the draw step's (here slice 0's mass is inflated a
    hundredfold), the slice they name as the owner cannot hold the target in its own masses:
    no id is placed, and the finish flags the row instead of returning the slice's first id."""
    g = torch.Generator().manual_seed(11)
    rows, V = 16, 4096
    x = torch.randn(rows, V, generator=g).to(DEV)
    u = torch.full((rows,), 0.5).to(DEV)
    bounds = [0, V // 2, V]
    slices = list(enumerate(zip(bounds[:-1], bounds[1:])))
    print(f"case: mismatched slice masses rows={rows} V={V}", flush=True)
    states = [full_shard_states(x[:, a:b], vocab_offset=a, vocab_size=V) for _, (a, b) in slices]
    masses = [full_shard_masses(x[:, a:b], states, shard_index=i, vocab_offset=a, vocab_size=V)
              for i, (a, b) in slices]
    # masses of 2^43 per unit of exp(z - M): a 2048-id half stays far below 2^63 / 100
    assert int(masses[0].max()) < (1 << 56)
    bad = [masses[0] * 100, masses[1]]
    picks = [full_shard_draw(x[:, a:b], states, bad, shard_index=i, vocab_offset=a, vocab_size=V, uniforms=u)
             for i, (a, b) in slices]
    res = full_shard_finish(states, picks, vocab_size=V, draw="inverse_cdf", uniforms=u, check=False)
    assert bool((res.status & 32 != 0).all())
    assert bool((res.ids == -1).all()) and bool(torch.isnan(res.logprobs).all())
    with pytest.raises(ValueError, match="slice masses"):
        full_shard_finish(states, picks, vocab_size=V, draw="inverse_cdf", uniforms=u)
    good = [full_shard_draw(x[:, a:b], states, masses, shard_index=i, vocab_offset=a, vocab_size=V, uniforms=u)
            for i, (a, b) in slices]
    ok = full_shard_finish(states, good, vocab_size=V, draw="inverse_cdf", uniforms=u)
    whole = sample(x, uniforms=u)
    assert torch.equal(ok.ids, whole.ids) and bool((ok.status == 0).all())


@pytest.mark.parametrize("shuffle", [False, True])
def test_small_top_k_merge_of_many_lists(shuffle):
    """top_k <= 64 over more than 64 keys: the merge takes the union's 64 largest keys by
    bitonic merges of the sorted lists.  Lists handed over in another order (a caller's own
    gather) fail its sortedness check and take the general merge; both equal the unsharded
    row and the oracle."""
    from dsv41_rocm.sampling import ShardCandidates

    g = torch.Generator().manual_seed(640)
    rows, V = 12, 60000
    x = 2.0 * torch.randn(rows, V, generator=g)
    x[3] = 0.01 * torch.randn(V, generator=g)  # flat row: every list full
    u = torch.rand(rows, generator=g)
    hist = torch.randint(0, V, (rows, 32), generator=g)
    knobs = dict(top_k=40, top_p=0.9, repetition_penalty=1.2)
    bounds = edges(V, 12, 7)
    xd, ud, hd = x.to(DEV), u.to(DEV), hist.to(DEV)
    shards = [sample_shard(xd[:, a:b], vocab_offset=a, vocab_size=V, history=hd, top_k=40,
                           repetition_penalty=1.2) for a, b in zip(bounds[:-1], bounds[1:])]
    if shuffle:
        mixed = []
        for k, sh in enumerate(shards):
            keys = sh.keys.clone()
            perm = torch.randperm(keys.shape[1], generator=torch.Generator().manual_seed(k)).to(DEV)
            for r in range(rows):
                c = int(sh.counts[r])
                if c > 1:
                    keys[r, :c] = keys[r, perm[perm < c]]
            mixed.append(ShardCandidates(keys, sh.counts, sh.status))
        shards = mixed
    print(f"case: 12 lists of top_k=40, shuffled={shuffle}", flush=True)
    merged = merge_shards(shards, top_k=40, top_p=0.9, uniforms=ud, check=False)
    whole = sample(xd, uniforms=ud, history=hd, check=False, **knobs)
    torch.cuda.synchronize()
    ora = oracle.sample(x.numpy(), uniforms=u.numpy(), history=hist.numpy(), **knobs)
    assert_same(merged, whole, ora)
