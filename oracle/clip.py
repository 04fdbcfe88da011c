"""Global-L2 gradient clipping (CPU oracle; test infrastructure only).

Restates the clip branch of ``_prepare_grads`` (``apexw/optimizer.py:242-256``):
per-tensor L2 norms via ``_foreach_norm`` (each norm is returned in the grad's
own dtype, so bf16 grads give bf16-rounded norms), total = L2 norm of those
norms in fp32, ``coef = clip / (total + 1e-6)`` clamped to at most 1, and the
grads are multiplied in place (rounded to their dtype) when ``coef < 1``.
"""

import torch


def total_norm(grads):
    norms = torch._foreach_norm(grads, 2.0)
    return torch.linalg.vector_norm(torch.stack([n.to(torch.float32) for n in norms]), 2.0)


def clip_coef(grads, clip):
    return torch.clamp(clip / (total_norm(grads) + 1e-6), max=1.0)


def clip_grads_(grads, clip):
    coef = clip_coef(grads, clip)
    if float(coef.item()) < 1.0:
        torch._foreach_mul_(grads, coef)
    return coef
