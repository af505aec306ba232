"""The derived fp32 gradient bound (tests/_gradbound.py) on the CPU: it holds for fp32
evaluations of the euclidean, cosine and Minkowski p = 3 gradients in a blocked order (torch's
fp32 matrix products and chunked sums), and mistakes planted in the float64 reference (a dropped
term, a doubled term, a flipped sign, a weight off by one part in 10^4) each break it."""
import pytest
import torch

from tests import _gradbound as GB


def _euclid_case(n=24, m=3000, d=64, seed=0):
    g = torch.Generator().manual_seed(seed)
    x1 = torch.randn(n, d, generator=g)
    x2 = torch.randn(m, d, generator=g)
    gr = torch.randn(n, m, generator=g)
    return x1, x2, gr


def _euclid_fp32_grad(x1, x2, gr, chunk=32):
    """grad_x1 = x1 * rowsum(w) - w @ x2 in fp32, accumulated over chunks of the columns (a
    blocked order like the tile kernel's K chunks), w = g / res from the fp32 forward."""
    res = torch.cdist(x1, x2)
    w = gr / res
    acc = torch.zeros_like(x1)
    rs = torch.zeros(x1.shape[0])
    for j0 in range(0, x2.shape[0], chunk):
        acc = acc + w[:, j0:j0 + chunk] @ x2[j0:j0 + chunk]
        rs = rs + w[:, j0:j0 + chunk].sum(1)
    return rs[:, None] * x1 - acc


def _euclid_ref(x1, x2, gr):
    a = x1.double().requires_grad_()
    out = torch.cdist(a, x2.double())
    out.backward(gr.double())
    w = gr.double() / out.detach()
    return a.grad, w


def test_bound_holds_for_a_blocked_fp32_euclidean_gradient():
    x1, x2, gr = _euclid_case()
    got = _euclid_fp32_grad(x1, x2, gr)
    ref, w = _euclid_ref(x1, x2, gr)
    bound = GB.inner_grad_bound(w, x2, x1, w, None, c_w=5.0)
    worst = GB.check(got, ref, bound, "fp32 euclidean gradient")
    assert worst < 0.5, worst  # with room: the statistical part is a 6-sigma bound
    # tighter than the flat bar it replaces, on the typical element
    flat = 1e-4 * ref.abs() + 1e-4 * ref.abs().max()
    assert float((bound / flat).median()) < 0.5


@pytest.mark.parametrize("mistake", ["drop", "double", "sign", "weight"])
def test_bound_catches_mistakes_planted_in_the_reference(mistake):
    x1, x2, gr = _euclid_case(seed=1)
    got = _euclid_fp32_grad(x1, x2, gr)
    a = x1.double()
    res = torch.cdist(a, x2.double())
    w = gr.double() / res
    wm = w.clone()
    if mistake == "drop":
        wm[:, 1234] = 0.0           # one pair's term left out of every row
    elif mistake == "double":
        wm[:, 77] *= 2.0            # one pair counted twice
    elif mistake == "sign":
        wm[:, 2999] = -wm[:, 2999]  # one pair's sign flipped
    else:
        wm = w * (1.0 + 1e-4)       # every weight off by one part in 10^4
    ref = a * wm.sum(1, keepdim=True) - wm @ x2.double()
    bound = GB.inner_grad_bound(wm, x2, x1, wm, None, c_w=5.0)
    with pytest.raises(AssertionError, match="exceeds the derived bound"):
        GB.check(got, ref, bound, f"planted {mistake}")


def test_bound_holds_for_a_blocked_fp32_minkowski_p3_gradient():
    g = torch.Generator().manual_seed(2)
    x1 = torch.rand(16, 64, generator=g) * 2 - 1
    x2 = torch.rand(4096, 64, generator=g) * 2 - 1
    dist = torch.cdist(x1, x2, 3.0)
    w = 1.0 / (dist * dist)                                     # upstream gradient of ones
    d = x1[:, None, :] - x2[None, :, :]
    t = w[:, :, None] * (d * d.abs())
    got = torch.zeros_like(x1)
    for j0 in range(0, 4096, 1024):                             # four j splits, summed in order
        part = torch.zeros_like(x1)
        for j in range(j0, j0 + 1024, 32):
            part = part + t[:, j:j + 32].sum(1)
        got = got + part
    a = x1.double().requires_grad_()
    out = torch.cdist(a, x2.double(), 3.0)
    out.backward(torch.ones_like(out))
    dd = x1.double()[:, None, :] - x2.double()[None, :, :]
    terms = (1.0 / out.detach() ** 2)[:, :, None] * dd * dd.abs()
    worst = GB.check(got, a.grad, GB.sum_bound(terms, 1, 8.0), "fp32 minkowski p=3 gradient")
    assert worst < 0.5, worst
