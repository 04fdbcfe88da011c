"""Global-L2 gradient clipping (CPU oracle; test infrastructure only).

Restates the clip branch of ``_prepare_grads`` (``apexw/optimizer.py:242-256``):
per-tensor L2 norms via ``_foreach_norm`` (each norm is returned in the grad's
own dtype, so bf16 grads give bf16-rounded norms; fp32 norms are accumulated in
float64, see ``_norms``), total = L2 norm of those
norms in fp32, ``coef = clip / (total + 1e-6)`` clamped to at most 1, and the
grads are multiplied in place (rounded to their dtype) when ``coef < 1``.
"""

import torch


def _norms(grads):
    """Per-tensor L2 norms in each grad's dtype.  fp32 grads accumulate in float64
    and round once: the reference's device reduction (a tree) is accurate to fp32
    rounding, while torch's CPU fp32 reduction over ~1e5+ elements drifts by
    ~1e-5 relative.  16-bit grads keep _foreach_norm (norms rounded to the dtype)."""
    out = list(torch._foreach_norm(grads, 2.0))
    for i, g in enumerate(grads):
        if g.dtype == torch.float32:
            out[i] = torch.linalg.vector_norm(g.double(), 2.0).to(torch.float32)
    return out


def total_norm(grads):
    norms = _norms(grads)
    return torch.linalg.vector_norm(torch.stack([n.to(torch.float32) for n in norms]), 2.0)


def clip_coef(grads, clip):
    return torch.clamp(clip / (total_norm(grads) + 1e-6), max=1.0)


def clip_grads_(grads, clip):
    coef = clip_coef(grads, clip)
    if float(coef.item()) < 1.0:
        torch._foreach_mul_(grads, coef)
    return coef
