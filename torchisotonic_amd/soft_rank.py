"""Soft ranks by isotonic regression: a differentiable consumer of the isotonic forward and
backward at scale.

``soft_rank(x, regularization_strength)`` is the L2-regularised soft rank of Blondel et al.,
"Fast Differentiable Sorting and Ranking" (ICML 2020): the projection of the ranks' permutahedron
point, computed per row from one sort and one decreasing isotonic fit with weights of one. It
has the semantics of torchsort's ``soft_rank(..., regularization="l2")`` with this package's
isotonic solver in place of torchsort's, as the reference wires it (reference
paper/soft_rank.py:31-55):

    w = (n, n - 1, ..., 1)                      the ranks of a descending sort
    s, perm = sort(x / eps, descending)
    dual = isotonic(s - w, increasing=False)    (equal means pool: PAVA's rule)
    soft_rank = (s - dual) in x's order

and its gradient is the isotonic step's vector-Jacobian product (block averages over the dual's
blocks) taken through the sort: dx = (g - A g) / eps, A the block-averaging map of the dual's
partition. As eps -> 0 the soft ranks approach the hard ranks (1 for the smallest entry, n for
the largest); as eps grows they approach (n + 1) / 2.

Rows are the last dimension of a 2-D tensor on a ROCm device; the isotonic fit and its backward
run in the package's HIP kernels (float64 sums and hull tests, float32 rounded once).
"""

from __future__ import annotations

import torch
from torch import Tensor

from torchisotonic_amd._api import isotonic


def _ranks_desc(x: Tensor) -> Tensor:
    """(n, n - 1, ..., 1), broadcast over the rows of x."""
    n = x.shape[-1]
    return torch.arange(n, 0, -1, dtype=x.dtype, device=x.device).expand_as(x)


# torch.sort of one row of at most 2^20 elements runs the sort library's merge sort (225 us at
# 2^20 on MI355X), of more its one-sweep radix sort (100 us at 2^20 + 1): a single row of
# _PAD_FROM .. 2^20 elements is sorted padded to 2^20 + 1 with -inf, which a stable descending
# sort puts after every element of the row (its own -inf included), so the first n places and
# their indices are the row's own. (Rows of 2^18 elements: 118 -> 100 us; 1e6: 221 -> 100 us.)
_PAD_TO = (1 << 20) + 1
_PAD_FROM = 1 << 18


def _sort_desc(v: Tensor) -> tuple[Tensor, Tensor]:
    n = v.shape[-1]
    if v.shape[0] == 1 and _PAD_FROM <= n < _PAD_TO:
        padded = torch.full((1, _PAD_TO), float("-inf"), dtype=v.dtype, device=v.device)
        padded[:, :n] = v
        s, perm = torch.sort(padded, dim=-1, descending=True, stable=True)
        return s[:, :n], perm[:, :n]
    return torch.sort(v, dim=-1, descending=True)


class _SoftRank(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x: Tensor, strength: float) -> Tensor:  # type: ignore[override]
        scale = 1.0 / strength
        s, perm = _sort_desc(x * scale)
        inv = torch.empty_like(perm)
        inv.scatter_(-1, perm, torch.arange(x.shape[-1], device=x.device).expand_as(perm))
        with torch.enable_grad():
            z = (s - _ranks_desc(s)).detach().requires_grad_()
            dual = isotonic(z, increasing=False)
        ctx.scale = scale
        ctx.z, ctx.dual = z, dual
        ctx.save_for_backward(perm, inv)
        return (s - dual.detach()).gather(-1, inv)

    @staticmethod
    def backward(ctx, grad_out: Tensor) -> tuple[Tensor, None]:  # type: ignore[override]
        perm, inv = ctx.saved_tensors
        sorted_grad = grad_out.gather(-1, perm)
        # (the graph is kept, as in the reference, so that backward may run more than once)
        (avg,) = torch.autograd.grad(ctx.dual, ctx.z, sorted_grad, retain_graph=True)
        return (grad_out - avg.gather(-1, inv)) * ctx.scale, None


def soft_rank(x: Tensor, regularization_strength: float = 1.0) -> Tensor:
    """Soft ranks of every row of ``x`` ([batch, n], float, on the GPU): a differentiable
    relaxation of the ranks (1 = smallest), exact ranks as ``regularization_strength`` -> 0."""
    if not isinstance(x, Tensor):
        raise TypeError(f"x must be a torch.Tensor, got {type(x).__name__}")
    if x.ndim != 2:
        raise ValueError(f"x must be [batch, n], got shape {tuple(x.shape)}")
    if not x.is_floating_point():
        raise TypeError(f"x must be a float tensor, got {x.dtype}")
    if not regularization_strength > 0:
        raise ValueError("regularization_strength must be positive")
    if x.numel() == 0:
        return x.clone()
    return _SoftRank.apply(x, float(regularization_strength))
