"""Per-element error bounds for fp32 gradients that are sums over the other operand's rows.

Every fp32 gradient checked against a float64 reference here has the form

    grad[i, k] = sum_{j=1..K} t_j  (+ a second sum, scaled per row, for the inner-product family)

evaluated in fp32: each term t_j is formed with a few roundings (relative error c_t u each
term, u = 2^-24), and the K terms are accumulated in a blocked order (MFMA accumulators over
K chunks, or VALU accumulators over j splits).  The bound has two parts:

* terms: |sum of the term errors| <= c_t u sum_j |t_j|  (rigorous, first order);
* accumulation: each addition rounds its partial sum s_k with a relative error delta_k,
  |delta_k| <= u, so the accumulated error is sum_k delta_k s_k.  The worst case, u sum_k |s_k|,
  is about sqrt(K) times what a computation ever shows; with delta_k modelled as independent
  and uniform on [-u, u] (the standard statistical model of rounding, Higham, "Accuracy and
  Stability of Numerical Algorithms", 2nd ed., sections 2.8 and 4.2), the error has standard
  deviation u sqrt(sum_k s_k^2 / 3).  The bound takes 6 of them.  The partial sums are taken
  in index order, in float64; a blocked order permutes the terms within a block and restarts
  at a split, which leaves sum_k s_k^2 of the same size or smaller.

So |err| <= u (c_t sum_j |t_j| + 6 sqrt(sum_k s_k^2 / 3)), plus one rounding of each part where
two parts are combined.  For the euclidean gradient with K = 8192 random terms and d = 256 this
is about 6e-5 of a typical element's magnitude, 15 times tighter (median) than the flat bar
rtol 1e-4 + 1e-4 max|ref| it replaces; an fp32 evaluation in a blocked order stays below 4 % of
it.  A single dropped, doubled or sign-flipped term, or weights off by one part in 10^4, exceed
it (tests/test_gradbound.py plants such mistakes in the reference and shows the bound catches
them).
"""
from __future__ import annotations

import torch

U = 2.0 ** -24
Z = 6.0  # standard deviations of the accumulation error


def sum_bound(t: torch.Tensor, dim: int, c_t: float) -> torch.Tensor:
    """Bound of |fp32 sum of t over `dim` - the exact sum|, for terms with relative error
    c_t u each: u (c_t sum |t| + Z sqrt(sum_k s_k^2 / 3)), s_k the partial sums along dim."""
    t = t.double()
    s = torch.cumsum(t, dim)
    return U * (c_t * t.abs().sum(dim) + Z * torch.sqrt((s * s).sum(dim) / 3.0))


def check(got: torch.Tensor, ref: torch.Tensor, bound: torch.Tensor, what: str) -> float:
    """Asserts |got - ref| <= bound elementwise; returns the largest ratio err / bound."""
    err = (got.double() - ref.double()).abs()
    bound = bound.double()
    ratio = err / bound.clamp_min(1e-300)
    worst = float(ratio.max())
    if not worst <= 1.0:
        idx = int(ratio.argmax())
        raise AssertionError(f"{what}: |err| exceeds the derived bound by {worst:.3g}x at flat index {idx} "
                             f"(err {float(err.flatten()[idx]):.3e}, bound {float(bound.flatten()[idx]):.3e}, "
                             f"ref {float(ref.flatten()[idx]):.3e})")
    return worst


def inner_grad_bound(w: torch.Tensor, other: torch.Tensor, own: torch.Tensor, coef_terms: torch.Tensor,
                     coef_scale: torch.Tensor | None, c_w: float, c_coef: torch.Tensor | None = None) -> torch.Tensor:
    """Bound for grad[i, k] = sign * sum_j w[i, j] other[j, k] + coef[i] own[i, k], coef[i] =
    sum_j coef_terms[i, j] * coef_scale[i] (the inner-product family's backward: euclidean with
    coef_terms = w, the cosine family with coef_terms = its row terms and coef_scale = 1 / n1).
    w, coef_terms [R, K] (float64, the reference's values); other [K, D]; own [R, D].  c_w: the
    relative error (units of u) of each computed weight.  c_coef [R, K] (optional): an absolute
    error per coefficient term in units of u (the cosine family's q read back from its output),
    replacing c_w |coef_terms|."""
    w = w.double()
    other, own = other.double(), own.double()
    # the products w_ij other_jk: the weight's error plus one rounding (in row chunks of the
    # [R, K, D] terms, to bound the memory)
    prod = torch.empty_like(own)
    A = torch.empty_like(own)
    step = max(1, (1 << 24) // max(1, other.numel()))
    for r0 in range(0, w.shape[0], step):
        terms = w[r0:r0 + step, :, None] * other[None, :, :]
        prod[r0:r0 + step] = sum_bound(terms, 1, c_w + 1.0)
        A[r0:r0 + step] = terms.sum(1)
        del terms
    ct = coef_terms.double()
    cs = torch.ones(ct.shape[0], dtype=torch.float64) if coef_scale is None else coef_scale.double()
    if c_coef is None:
        cb = sum_bound(ct, 1, c_w)
    else:
        s = torch.cumsum(ct, 1)
        cb = U * (c_coef.double().abs().sum(1) + Z * torch.sqrt((s * s).sum(1) / 3.0))
    coef = ct.sum(1) * cs
    B = coef[:, None] * own
    # coef's error scaled, its own rounding and the product with own, the final add
    bound = prod + (cb * cs.abs())[:, None] * own.abs() + U * (2.0 * B.abs() + A.abs() + (A + B).abs())
    return bound


def euclidean_grad_bound(own: torch.Tensor, other: torch.Tensor, gsl: torch.Tensor) -> torch.Tensor:
    """Bound of the fp32 euclidean gradient of `own`'s rows (a sum over `other`'s rows), gsl
    [rows of own, rows of other] the upstream gradient in that orientation (grad^T for x2's
    rows): w = g / res, grad = own sum_j w - w other.  The weight comes from the fp32 forward
    output and the hardware reciprocal (fast_div): 5 u."""
    own, other, gsl = own.double(), other.double(), gsl.double()
    w = gsl / torch.cdist(own, other)
    return inner_grad_bound(w, other, own, w, None, c_w=5.0)


def cosine_grad_bound(own: torch.Tensor, other: torch.Tensor, gsl: torch.Tensor,
                      similarity: bool = False) -> torch.Tensor:
    """Bound of the fp32 cosine-distance (or, with similarity, cosine-similarity) gradient of
    `own`'s rows: W = gq / den, coef = sum_j (-W q n_other) / n_own.  W: 6 u (the reciprocal,
    the norm product, the norms); each coefficient term 8 u relative, plus 3 u |W| n_other
    absolute for q, which the backward reads back from the fp32 output (1 - out)."""
    own, other, gsl = own.double(), other.double(), gsl.double()
    n_own, n_other = own.norm(dim=1), other.norm(dim=1)
    den = n_own[:, None] * n_other[None, :]
    q = (own @ other.T) / den
    if similarity:
        gq = gsl
    else:
        v = 1.0 - q
        gq = torch.where((v >= 0) & (v <= 2), -gsl, torch.zeros_like(gsl))
    W = gq / den
    rt = -W * q * n_other[None, :]
    c_coef = 8.0 * rt.abs() + 3.0 * W.abs() * n_other[None, :]
    return inner_grad_bound(W, other, own, rt, 1.0 / n_own, c_w=6.0, c_coef=c_coef)
