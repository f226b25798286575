"""Parity at the full benchmark shapes of configs C, D and E.

The reduced-size tests elsewhere take other launch plans than the benchmark does.  Here the
plans of the benchmark runs themselves are checked:
* D (16384 tokens x 7168 -> 129280): 64 token blocks x 4 vocabulary splits, mapped onto
  8 x 4 XCD super-tiles, forward with the Token-TIS ratio and the logit gradient;
* C (8192 tokens x 2048 -> 151936): 32 token blocks x 8 splits;
* E (4096 x 151936 fp32): 256-thread top-k workgroups with the deferred final selection;
  E's logits with top-p 0.9 alone (512-thread top-p workgroups) and top-k 50 alone (the
  seeded top-k instantiation);
* a 2048 x 136 -> 8192 head, small enough to check every logit gradient, on the same 8 x 4
  super-tile mapping (8 token blocks x 32 splits).

Reference values: fp64 log-softmax of fp64 logits from the same bf16 operands (GPU, chunked
over tokens); the C oracle for the sampler.  Bars as in the reduced tests: 1e-4 absolute for
log-prob, entropy and ratio; ids, kept sets and statuses bit-exact; the bf16 logit gradient
within 2^-7 |G| + 1e-3 max|G row| elementwise.

Beside the fp64 reference each log-prob case prints the "reference-rounding" difference: the
reference's literal expression (model.py:682-683: bf16 ``lm_head`` output, then ``.float()``,
``log_softmax``, ``gather``) against the same fp64 values, on a token subset.  It is reported,
not asserted against 1e-4: rounding the logits to bf16 moves log-probs by ~1e-3-1e-2.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from dsv41_rocm import logprob as lpmod
from dsv41_rocm import sample, selected_log_probs, workloads

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
TOL = 1e-4


def reference(x, w, t, temperature, chunk=1024):
    """fp64 log-prob, entropy and lse from bf16 operands, chunked over tokens."""
    wd = w.double()
    lps, ents, lses = [], [], []
    for s in range(0, x.shape[0], chunk):
        z = (x[s:s + chunk].double() @ wd.T) / temperature
        lse = torch.logsumexp(z, dim=-1)
        lsm = z - lse[:, None]
        lps.append(lsm.gather(1, t[s:s + chunk, None])[:, 0])
        ents.append(lse - (lsm.exp() * z).sum(dim=1))
        lses.append(lse)
        del z, lsm
    del wd
    return torch.cat(lps), torch.cat(ents), torch.cat(lses)


def reference_rounding(x, w, t, temperature, rlp, idx):
    """max |literal reference expression - fp64| and the kernel's own, on tokens idx."""
    logits = F.linear(x[idx], w)  # bf16 output, as nn.Linear returns it (model.py:682)
    lit = torch.log_softmax(logits.float() / temperature, dim=-1).gather(-1, t[idx, None])[:, 0]
    return torch.max(torch.abs(lit.double() - rlp[idx])).item()


def logprob_case(name, with_ratio):
    inp = workloads.logprob_inputs(name, device=DEV)
    x, w, t = inp["x"], inp["w"], inp["targets"]
    n = x.shape[0]
    print(f"case: full-size config {name}: N={n} H={x.shape[1]} V={w.shape[0]} ratio={with_ratio}", flush=True)
    rlp, rent, rlse = reference(x, w, t, 1.0)
    behavior = None
    if with_ratio:
        g = torch.Generator(device=DEV).manual_seed(5)
        behavior = (rlp + 0.05 * torch.randn(n, generator=g, device=DEV, dtype=torch.float64)).float()
    lp, ent, ratio = selected_log_probs(x, w, t, 1.0, behavior=behavior, is_cap=2.0)
    torch.cuda.synchronize()
    d_lp = torch.max(torch.abs(lp.double() - rlp)).item()
    d_ent = torch.max(torch.abs(ent.double() - rent)).item()
    idx = torch.arange(0, n, max(1, n // 1024), device=DEV)
    d_lit = reference_rounding(x, w, t, 1.0, rlp, idx)
    print(f"config {name}: max|lp - fp64| {d_lp:.3e}, max|entropy - fp64| {d_ent:.3e}; reference-rounding "
          f"(bf16 logits, model.py:682) max|lp - fp64| {d_lit:.3e} on {idx.numel()} tokens", flush=True)
    assert d_lp <= TOL and d_ent <= TOL
    if with_ratio:
        w_ref, _ = oracle.token_tis_weight(rlp.float().cpu().numpy(), behavior.cpu().numpy(), 2.0)
        d_ratio = np.max(np.abs(ratio.cpu().numpy() - w_ref))
        print(f"config {name}: max|ratio - oracle weight| {d_ratio:.3e}", flush=True)
        assert d_ratio <= TOL
    return inp, rlse


def grad_reference_rows(x, w, t, temperature, glp, gent, rows):
    """fp64 dL/dz / T for the token rows `rows` (log-prob and entropy terms)."""
    z = (x[rows].double() @ w.double().T) / temperature
    lse = torch.logsumexp(z, dim=-1, keepdim=True)
    p = torch.exp(z - lse)
    ent = lse[:, 0] - (p * z).sum(-1)
    onehot = torch.zeros_like(z).scatter_(1, t[rows, None], 1.0)
    g = glp[rows, None].double() * (onehot - p) + gent[rows, None].double() * p * (lse - ent[:, None] - z)
    return g / temperature


def assert_grad_close(got, ref):
    rowmax = ref.abs().amax(dim=1, keepdim=True)
    bad = (got.double() - ref).abs() > 2.0 ** -7 * ref.abs() + 1e-3 * rowmax
    assert not bool(bad.any()), int(bad.sum())


def test_config_d_full_size_forward_ratio_and_gradient():
    inp, _ = logprob_case("D", True)
    x, w, t = inp["x"], inp["w"], inp["targets"]
    n = x.shape[0]
    print("case: full-size config D logit gradient (all 129280 columns, 64 token rows checked)", flush=True)
    g = torch.Generator(device=DEV).manual_seed(11)
    glp = torch.randn(n, generator=g, device=DEV)
    gent = torch.randn(n, generator=g, device=DEV)
    hx, hw, ht = lpmod._prepare(x, w, t, 1.0)
    _, ent, _, lse, _ = lpmod._forward(hx, hw, ht, 1.0, None, 2.0)
    grad = lpmod.logits_grad(hx, hw, ht, 1.0, lse, ent, glp, gent)
    torch.cuda.synchronize()
    rows = torch.arange(0, n, 257, device=DEV)
    assert_grad_close(grad[rows], grad_reference_rows(x, w, t, 1.0, glp, gent, rows))


def test_config_c_full_size_forward():
    logprob_case("C", False)


def test_xcd_super_tile_plan_forward_and_every_logit_gradient():
    # 2048 tokens = 8 token blocks; 8192 rows = 32 vocabulary splits; 8 x 32 = 256 workgroups
    # tile into 8 x 4 super-tiles, the mapping of every C and D launch
    n, h, v, T = 2048, 136, 8192, 0.9
    print(f"case: super-tile plan N={n} H={h} V={v} T={T}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(2048)
    x = torch.randn(n, h, generator=g, device=DEV).to(torch.bfloat16)
    w = (0.3 * torch.randn(v, h, generator=g, device=DEV)).to(torch.bfloat16)
    t = torch.randint(0, v, (n,), generator=g, device=DEV)
    glp = torch.randn(n, generator=g, device=DEV)
    gent = torch.randn(n, generator=g, device=DEV)
    lp, ent, _ = selected_log_probs(x, w, t, T)
    rlp, rent, _ = reference(x, w, t, T)
    assert torch.max(torch.abs(lp.double() - rlp)).item() <= TOL
    assert torch.max(torch.abs(ent.double() - rent)).item() <= TOL
    hx, hw, ht = lpmod._prepare(x, w, t, T)
    _, ent2, _, lse, _ = lpmod._forward(hx, hw, ht, T, None, 2.0)
    grad = lpmod.logits_grad(hx, hw, ht, T, lse, ent2, glp, gent)
    torch.cuda.synchronize()
    for s in range(0, n, 512):
        rows = torch.arange(s, s + 512, device=DEV)
        assert_grad_close(grad[rows], grad_reference_rows(x, w, t, T, glp, gent, rows))


def test_config_e_full_size_sampler():
    inp = workloads.sampler_inputs("E", device=DEV)
    logits, history, uniforms, knobs = inp["logits"], inp["history"], inp["uniforms"], inp["knobs"]
    print(f"case: full-size config E {tuple(logits.shape)} knobs={knobs}", flush=True)
    res = sample(logits, uniforms=uniforms, history=history, check=False, **knobs)
    torch.cuda.synchronize()
    gids, glp, gkept, gst = (r.cpu().numpy() for r in (res.ids, res.logprobs, res.kept, res.status))
    oids, olp, okept, ost = oracle.sample(logits.cpu().numpy(), uniforms=uniforms.cpu().numpy(),
                                          history=history.cpu().numpy(), **knobs)
    np.testing.assert_array_equal(gst, ost)
    assert (ost == 0).all()
    np.testing.assert_array_equal(gkept, okept)
    np.testing.assert_array_equal(gids, oids)
    d_lp = np.max(np.abs(glp - olp))
    print(f"config E: 4096 rows, ids and kept sets identical, max|lp - oracle| {d_lp:.3e}", flush=True)
    assert d_lp <= TOL


@pytest.mark.parametrize("mode", ["top_p", "top_k"])
def test_config_e_shape_serving_mixes(mode):
    """E's 4096 rows in two serving mixes, on the launch plans of the opt-in bench workloads:
    top-p 0.9 alone (topp_kernel with 512 threads, two workgroups per CU) and top-k 50 alone
    (the seeded 256-thread topk_kernel and the deferred selection).  The oracle runs over row
    blocks in threads (ctypes releases the GIL): top-p alone sorts every row."""
    from concurrent.futures import ThreadPoolExecutor

    inp = workloads.sampler_inputs("E", device=DEV)
    logits, uniforms = inp["logits"], inp["uniforms"]
    knobs = dict(temperature=0.6, **(dict(top_p=0.9) if mode == "top_p" else dict(top_k=50)))
    print(f"case: config E's logits {tuple(logits.shape)} knobs={knobs}", flush=True)
    res = sample(logits, uniforms=uniforms, check=False, **knobs)
    torch.cuda.synchronize()
    gids, glp, gkept, gst = (r.cpu().numpy() for r in (res.ids, res.logprobs, res.kept, res.status))
    x, u = logits.cpu().numpy(), uniforms.cpu().numpy()
    cuts = np.linspace(0, x.shape[0], 17).astype(int)
    with ThreadPoolExecutor(16) as ex:
        parts = list(ex.map(lambda ab: oracle.sample(x[ab[0]:ab[1]], uniforms=u[ab[0]:ab[1]], **knobs),
                            zip(cuts[:-1], cuts[1:])))
    oids, olp, okept, ost = (np.concatenate([p[i] for p in parts]) for i in range(4))
    np.testing.assert_array_equal(gst, ost)
    assert (ost == 0).all()
    np.testing.assert_array_equal(gkept, okept)
    np.testing.assert_array_equal(gids, oids)
    d_lp = np.max(np.abs(glp - olp))
    print(f"config E's logits, {mode}: ids and kept sets identical, max|lp - oracle| {d_lp:.3e}", flush=True)
    assert d_lp <= TOL
