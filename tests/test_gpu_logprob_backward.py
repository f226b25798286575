"""GPU parity of the fused log-prob backward (dsv41_logprob_grad_run through the C ABI, and
the autograd path built on it).

Reference values: the numpy fp64 oracle (oracle.logprob_grad_oracle, pinned against torch
fp64 autograd on the CPU), and torch fp64 autograd on the GPU for larger shapes.

Bars (the logit gradient is bf16, as the reference's lm_head output gradient is):
* logit gradient: |G - G64| <= 2^-7 |G64| + 1e-3 * max|G64 row|, elementwise;
* dL/dx and dL/dw: relative Frobenius error <= 1e-2 against fp64, and no more than twice
  the error of the reference expression's own autograd (bf16 linear, fp32 log_softmax)
  plus 1e-3.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from dsv41_rocm import logprob as lpmod
from dsv41_rocm import selected_log_probs, token_log_probs, workloads

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _case(n, h, v, seed, wscale=0.3):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn(n, h, generator=g, device=DEV).to(torch.bfloat16)
    w = (wscale * torch.randn(v, h, generator=g, device=DEV)).to(torch.bfloat16)
    t = torch.randint(0, v, (n,), generator=g, device=DEV)
    glp = torch.randn(n, generator=g, device=DEV)
    gent = torch.randn(n, generator=g, device=DEV)
    return x, w, t, glp, gent


def _rel(a, b):
    a, b = a.double(), b.double()
    return (torch.linalg.norm(a - b) / torch.linalg.norm(b)).item()


def _grads_fp64(x, w, t, T, glp, gent):
    xd = x.double().requires_grad_()
    wd = w.double().requires_grad_()
    lsm = torch.log_softmax((xd @ wd.T) / T, -1)
    lp = lsm.gather(-1, t[:, None])[:, 0]
    ent = -(lsm.exp() * lsm).sum(-1)
    ((glp.double() * lp).sum() + (gent.double() * ent).sum()).backward()
    return xd.grad, wd.grad


def _grads_reference_expression(x, w, t, T, glp, gent):
    """model.py:682-683 under autograd: bf16 linear, fp32 log_softmax (on the CPU)."""
    xr = x.cpu().requires_grad_()
    wr = w.cpu().requires_grad_()
    lsm = F.log_softmax(F.linear(xr, wr).float() / T, dim=-1)
    lp = lsm.gather(-1, t.cpu()[:, None])[:, 0]
    ent = -(lsm.exp() * lsm).sum(-1)
    ((glp.cpu() * lp).sum() + (gent.cpu() * ent).sum()).backward()
    return xr.grad.to(DEV), wr.grad.to(DEV)


@pytest.mark.parametrize("n,h,v,T", [(300, 136, 1000, 1.0), (257, 2048, 4099, 0.7), (5, 40, 3, 1.3),
                                     (64, 64, 65536 + 17, 1.0)])
def test_logits_grad_matches_oracle(n, h, v, T):
    print(f"case: logits_grad N={n} H={h} V={v} T={T}", flush=True)
    x, w, t, glp, gent = _case(n, h, v, n + v)
    hx, hw, ht = lpmod._prepare(x, w, t, T)
    _, ent, _, lse, _ = lpmod._forward(hx, hw, ht, T, None, 2.0)
    g = lpmod.logits_grad(hx, hw, ht, T, lse, ent, glp, gent)
    torch.cuda.synchronize()
    cols = slice(None) if v <= 8192 else slice(0, 8192)
    gl, _, _ = oracle.logprob_grad_oracle(x.float().cpu().numpy(), w.float().cpu().numpy(), t.cpu().numpy(), T,
                                          glp.cpu().numpy(), gent.cpu().numpy())
    ref = torch.from_numpy(gl).to(DEV)[:, cols]
    got = g.double()[:, cols]
    rowmax = ref.abs().amax(dim=1, keepdim=True)
    assert torch.all((got - ref).abs() <= 2.0 ** -7 * ref.abs() + 1e-3 * rowmax)
    # the log-prob part alone: each row of dL/dlogits sums to ~0 over the vocabulary
    g1 = lpmod.logits_grad(hx, hw, ht, T, lse, None, torch.ones_like(glp), None).double()
    assert torch.max(torch.abs(g1.sum(dim=1))).item() <= 1e-2 / T


def test_logits_grad_vocabulary_ranges_are_column_slices():
    x, w, t, glp, gent = _case(130, 72, 1300, 5)
    hx, hw, ht = lpmod._prepare(x, w, t, 0.9)
    _, ent, _, lse, _ = lpmod._forward(hx, hw, ht, 0.9, None, 2.0)
    full = lpmod.logits_grad(hx, hw, ht, 0.9, lse, ent, glp, gent)
    for b, e in [(0, 256), (100, 613), (1299, 1300), (517, 1300)]:
        print(f"case: vocabulary range [{b}, {e})", flush=True)
        part = lpmod.logits_grad(hx, hw, ht, 0.9, lse, ent, glp, gent, b, e)
        assert part.shape == (130, e - b)
        assert torch.equal(part, full[:, b:e])


@pytest.mark.parametrize("n,h,v,T", [(300, 136, 1000, 1.0), (257, 2048, 4099, 0.7)])
def test_autograd_matches_fp64_and_reference_expression(n, h, v, T):
    print(f"case: autograd N={n} H={h} V={v} T={T}", flush=True)
    x, w, t, glp, gent = _case(n, h, v, 7 * n + v)
    xg = x.clone().requires_grad_()
    wg = w.clone().requires_grad_()
    lp, ent, _ = selected_log_probs(xg, wg, t, T)
    ((glp * lp).sum() + (gent * ent).sum()).backward()
    assert xg.grad.dtype == torch.bfloat16 and wg.grad.dtype == torch.bfloat16
    dx64, dw64 = _grads_fp64(x, w, t, T, glp, gent)
    dxr, dwr = _grads_reference_expression(x, w, t, T, glp, gent)
    ex, ew = _rel(xg.grad, dx64), _rel(wg.grad, dw64)
    rx, rw = _rel(dxr, dx64), _rel(dwr, dw64)
    print(f"rel errors: ours dx {ex:.2e} dw {ew:.2e}; reference expression dx {rx:.2e} dw {rw:.2e}", flush=True)
    assert ex <= 1e-2 and ew <= 1e-2
    assert ex <= 2 * rx + 1e-3 and ew <= 2 * rw + 1e-3


def test_chunked_backward_matches_one_block():
    x, w, t, glp, gent = _case(200, 256, 3000, 9)
    hx, hw, ht = lpmod._prepare(x, w, t, 1.0)
    _, ent, _, lse, _ = lpmod._forward(hx, hw, ht, 1.0, None, 2.0)
    dx1, dw1 = lpmod.selected_log_probs_backward(hx, hw, ht, 1.0, lse, ent, glp, gent)
    dx2, dw2 = lpmod.selected_log_probs_backward(hx, hw, ht, 1.0, lse, ent, glp, gent, vocab_chunk=512)
    assert _rel(dx2, dx1) <= 5e-3 and _rel(dw2, dw1) <= 5e-3
    dx3, dw3 = lpmod.selected_log_probs_backward(hx, hw, ht, 1.0, lse, ent, glp, gent, need_weight=False)
    assert dw3 is None and torch.equal(dx3, dx1)


def test_token_log_probs_backward_through_mask():
    g = torch.Generator(device=DEV).manual_seed(21)
    B, T, H, V = 3, 11, 64, 700
    hidden = torch.randn(B, T, H, generator=g, device=DEV).to(torch.bfloat16).requires_grad_()
    w = (0.2 * torch.randn(V, H, generator=g, device=DEV)).to(torch.bfloat16).requires_grad_()
    targets = torch.randint(0, V, (B, T), generator=g, device=DEV)
    mask = torch.rand(B, T, generator=g, device=DEV) > 0.4
    adv = torch.randn(B, T, generator=g, device=DEV)
    out = token_log_probs(hidden, w, targets, mask, 0.8)
    (out * adv).sum().backward()
    # model.py:682-684 in fp64 under autograd
    hd = hidden.detach().double().requires_grad_()
    wd = w.detach().double().requires_grad_()
    sel = torch.log_softmax((hd[mask] @ wd.T) / 0.8, -1).gather(-1, targets[mask][:, None])[:, 0]
    ref = sel.new_zeros(mask.shape).masked_scatter(mask, sel)
    (ref * adv.double()).sum().backward()
    assert torch.equal(hidden.grad[~mask], torch.zeros_like(hidden.grad[~mask]))
    assert _rel(hidden.grad, hd.grad) <= 1e-2 and _rel(w.grad, wd.grad) <= 1e-2


def test_custom_op_autograd_matches_wrapper():
    x, w, t, glp, gent = _case(96, 128, 900, 31)
    print("case: torch.ops.dsv41_rocm.selected_log_probs backward", flush=True)
    xa, wa = x.clone().requires_grad_(), w.clone().requires_grad_()
    lp, ent, _, lse = torch.ops.dsv41_rocm.selected_log_probs(xa, wa, t, 0.9, None, 2.0)
    ((glp * lp).sum() + (gent * ent).sum()).backward()
    xb, wb = x.clone().requires_grad_(), w.clone().requires_grad_()
    lp2, ent2, _ = selected_log_probs(xb, wb, t, 0.9)
    ((glp * lp2).sum() + (gent * ent2).sum()).backward()
    assert torch.equal(xa.grad, xb.grad) and torch.equal(wa.grad, wb.grad)


def test_config_d_shape_reduced_tokens_input_gradient():
    inp = workloads.logprob_inputs("D", tokens=256, device=DEV)
    x, w, t = inp["x"], inp["w"], inp["targets"]
    print("case: backward at the D head shape, 256 tokens", flush=True)
    glp = torch.randn(256, generator=inp["generator"], device=DEV)
    xg = x.clone().requires_grad_()
    lp, _, _ = selected_log_probs(xg, w, t, 1.0)
    (glp * lp).sum().backward()
    xd = x.double().requires_grad_()
    lsm = torch.log_softmax(xd @ w.double().T, -1)
    (glp.double() * lsm.gather(-1, t[:, None])[:, 0]).sum().backward()
    assert _rel(xg.grad, xd.grad) <= 1e-2
