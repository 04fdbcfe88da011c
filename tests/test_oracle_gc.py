"""CPU: gradient centralization of the oracle (_prepare_grads,
apexw/optimizer.py:239-243: each dim >= 2 grad minus its mean over dims 1..).

Pinned by closed forms: rows of [[1, 2, 3], [4, 5, 6]] centralize to
[[-1, 0, 1], [-1, 0, 1]]; a 3-D grad centralizes over its last two dims; 1-D
grads are left alone; row-constant grads become zero.  A mean over the wrong
dims, a missing subtraction or centralized biases each fail one of them.  The
power-of-two AMP invariant (test_oracle_amp.py) also runs with centralization.
"""

import torch

from oracle.optim import OracleApexW


def _prepared(grads, **kw):
    ps = [torch.nn.Parameter(torch.zeros_like(g)) for g in grads]
    opt = OracleApexW(ps, grad_centralization=True, **kw)
    out, scale = opt._prepare([g.clone() for g in grads], sanitize=False)
    assert scale is None
    return out


def test_rows_centralize_to_closed_form():
    for dt in (torch.float32, torch.bfloat16):
        g = torch.tensor([[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]], dtype=dt)
        (out,) = _prepared([g])
        assert torch.equal(out, torch.tensor([[-1.0, 0.0, 1.0], [-1.0, 0.0, 1.0]], dtype=dt))


def test_3d_grad_over_last_dims_and_1d_untouched():
    g3 = torch.arange(8.0).reshape(2, 2, 2)                 # rows [0..3] and [4..7], means 1.5 and 5.5
    b = torch.tensor([1.0, 2.0, 4.0])
    out3, outb = _prepared([g3, b])
    assert torch.equal(out3, g3 - torch.tensor([1.5, 5.5]).reshape(2, 1, 1))
    assert torch.equal(outb, b)


def test_row_constant_grads_vanish():
    g = torch.tensor([[0.25] * 5, [-3.0] * 5])
    (out,) = _prepared([g])
    assert torch.equal(out, torch.zeros_like(g))


def test_sanitize_then_centralize():
    g = torch.tensor([[float("nan"), 2.0], [float("inf"), 0.0]])
    (out,) = _prepared([g])
    # NaN -> 0 and +Inf -> 65504 before the mean
    assert torch.equal(out, torch.tensor([[-1.0, 1.0], [32752.0, -32752.0]]))
