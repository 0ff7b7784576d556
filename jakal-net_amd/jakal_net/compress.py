"""Edge and route compressions of the operators, and their keep-masks.

A compression maps raw scores ``[..., n]`` and a boolean keep-mask to edge or
route weights that are exactly 0 on the dropped entries:

* ``softsign``            x / (1 + |x|) per entry (src/jakal_net/propagation.py:85-88);
* ``signed_abs_softmax``  sign(x) * softmax(|x|) over the kept entries of a row
  (propagation.py:67-82, transition.py:53-67);
* ``signed_entmax15``     sign(x) * entmax15(|x|) over the kept entries of a row
  (kernels.py:221-237);
* ``softmax`` (routes)    softmax over the kept entries, dropped entries held at
  the dtype minimum (kernel_common.py:420-423).

entmax15 is computed here by support refinement rather than by sorting: start
from every kept entry, take the closed-form threshold of that support, keep
the entries above it and repeat until the support is stable.  It solves the
same threshold equation sum (x_i - tau)^2 = 1 over the support as the
reference's sort (kernels.py:155-202); the HIP kernels use the same iteration.

Keep-masks: ``topk_keep_mask`` (the k best entries of each row,
kernel_common.py:433-440) and ``window_keep_mask`` (the causal band
i - window <= j <= i, kernel_common.py:443-456).
"""

from __future__ import annotations

from typing import Callable

import torch
from torch import Tensor
from torch.nn import functional as F

# __name__ values under which the operators recognise an edge compression; the
# names are part of the operator interface (propagation.py:56-64)
_EDGE_NAMES = {
    "softsign": "softsign",
    "signed_abs_softmax": "signed_abs_softmax",
    "signed_abs_softmax_edges": "signed_abs_softmax",
    "_signed_abs_softmax_edges": "signed_abs_softmax",
    "signed_entmax15": "signed_entmax15",
    "_signed_entmax15_edges": "signed_entmax15",
}
ROUTE_COMPRESS_NAMES = ("softmax", "signed_abs_softmax", "signed_entmax15")


def _kept(mask: Tensor | None, like: Tensor) -> Tensor:
    return torch.ones_like(like, dtype=torch.bool) if mask is None else mask.to(torch.bool)


def masked_softmax(logits: Tensor, mask: Tensor, dim: int = -1) -> Tensor:
    """Softmax with the dropped logits held at the dtype's minimum (a row with
    nothing kept therefore comes out uniform, as in the reference)."""
    floor = torch.finfo(logits.dtype).min
    return torch.where(mask, logits, logits.new_full((), floor)).softmax(dim=dim)


def signed_abs_softmax(scores: Tensor, *, dim: int = -1, mask: Tensor | None = None) -> Tensor:
    """sign(x) * softmax(|x|) over the kept entries; 0 elsewhere and on rows with nothing kept."""
    x = torch.nan_to_num(scores)
    keep = _kept(mask, x)
    p = torch.where(keep, x.abs(), x.new_full((), -torch.inf)).softmax(dim=dim)
    return torch.where(keep, torch.sign(x) * p, torch.zeros_like(p)).nan_to_num()


def entmax15(scores: Tensor, *, mask: Tensor | None = None) -> Tensor:
    """1.5-entmax over the kept entries of the last axis (0 elsewhere).

    With x = (z - max z) / 2 the result is max(x - tau, 0)^2, tau chosen so
    that it sums to 1; rows with nothing kept are all 0."""
    z = torch.nan_to_num(scores)
    keep = _kept(mask, z)
    top = torch.where(keep, z, z.new_full((), -torch.inf)).amax(dim=-1, keepdim=True)
    x = torch.where(keep, (z - torch.nan_to_num(top, neginf=0.0)) / 2, torch.zeros_like(z))
    support = keep
    with torch.no_grad():
        for _ in range(z.shape[-1]):
            tau = _entmax_threshold(x, support)
            refined = keep & (x > tau)
            if torch.equal(refined, support):
                break
            support = refined
    tau = _entmax_threshold(x, support)  # differentiable in x on the final support
    p = torch.where(keep, torch.clamp(x - tau, min=0.0).square(), torch.zeros_like(x))
    total = p.sum(dim=-1, keepdim=True)
    return torch.where(total > 0, p / total.clamp_min(torch.finfo(p.dtype).eps), torch.zeros_like(p))


def _entmax_threshold(x: Tensor, support: Tensor) -> Tensor:
    """tau with sum over the support of (x - tau)^2 = 1, the larger root clipped at the mean."""
    n = support.sum(dim=-1, keepdim=True).clamp_min(1).to(x.dtype)
    xs = torch.where(support, x, torch.zeros_like(x))
    mean = xs.sum(dim=-1, keepdim=True) / n
    spread = (xs.square().sum(dim=-1, keepdim=True) - n * mean.square()).clamp_min(0.0)
    return mean - torch.sqrt(((1.0 - spread) / n).clamp_min(0.0))


def signed_entmax15(scores: Tensor, *, dim: int = -1, mask: Tensor | None = None) -> Tensor:
    """sign(x) * entmax15(|x|) over the kept entries of the last axis."""
    if dim not in (-1, scores.dim() - 1):
        raise ValueError("signed_entmax15 normalises over the last axis only.")
    x = torch.nan_to_num(scores)
    out = torch.sign(x) * entmax15(x.abs(), mask=mask)
    return out.nan_to_num()


def edge_compress_name(edge_compress_fn: Callable[[Tensor], Tensor]) -> str | None:
    """Canonical name of a recognised edge compression, None for any other callable."""
    if edge_compress_fn is F.softsign:
        return "softsign"
    return _EDGE_NAMES.get(getattr(edge_compress_fn, "__name__", None))


_ROW_EDGE_COMPRESS = {"signed_abs_softmax": signed_abs_softmax, "signed_entmax15": signed_entmax15}


def compress_edges(scores: Tensor, edge_compress_fn: Callable[[Tensor], Tensor], *,
                   mask: Tensor | None = None) -> Tensor:
    """Edge weights of ``scores``: the row-normalising compressions run over the
    kept entries; any other function is applied entrywise and then masked."""
    row_fn = _ROW_EDGE_COMPRESS.get(edge_compress_name(edge_compress_fn))
    if row_fn is not None:
        return row_fn(scores, mask=mask)
    edges = edge_compress_fn(scores)
    return edges if mask is None else edges * mask.to(edges.dtype)


def compress_routes(logits: Tensor, name: str, *, mask: Tensor | None = None) -> Tensor:
    """Route weights of each source row over its kept destinations."""
    if name == "softmax":
        return logits.softmax(dim=-1) if mask is None else masked_softmax(logits, mask)
    if name == "signed_abs_softmax":
        return signed_abs_softmax(logits, mask=mask)
    if name == "signed_entmax15":
        return signed_entmax15(logits, mask=mask)
    raise ValueError(f"route compression must be one of {ROUTE_COMPRESS_NAMES}, got {name!r}.")


def topk_keep_mask(scores: Tensor, topk: int, *, dim: int = -1) -> Tensor:
    """True on the ``topk`` best entries along ``dim`` (every entry when topk >= the extent)."""
    if topk < 1:
        raise ValueError(f"topk must be at least 1, got {topk}.")
    if topk >= scores.shape[dim]:
        return torch.ones_like(scores, dtype=torch.bool)
    best = torch.topk(scores, topk, dim=dim, sorted=False).indices
    return torch.zeros(scores.shape, dtype=torch.bool, device=scores.device).scatter_(dim, best, True)


def window_keep_mask(t0: int, t1: int, s0: int, s1: int, window: int, *, device=None) -> Tensor:
    """[t1 - t0, s1 - s0] mask of target rows t0..t1 and source columns s0..s1:
    True where 0 <= target - source <= window."""
    if window < 0:
        raise ValueError(f"window must be non-negative, got {window}.")
    lag = torch.arange(t0, t1, device=device)[:, None] - torch.arange(s0, s1, device=device)[None, :]
    return (lag >= 0) & (lag <= window)
