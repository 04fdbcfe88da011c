"""CPU: the oracle's AMP grad-scale hand-off (GradScaler sets ``grad_scale`` and
``found_inf`` on optimizers with ``_step_supports_amp_scaling``).

Pinned by an invariant rather than by reference vectors (the reference's tests
hold none for this): GradScaler's scales are powers of two, and multiplying a
grad by 2^k and unscaling by 2^-k is exact in bf16/fp32, so a step on
``g * 2^k`` with ``grad_scale = 2^k`` must equal, bit for bit, the same step on
``g`` -- on every path (compact native / foreach, 8-bit chunked / generic, with
and without the global-norm clip, which must then see the unscaled norm).  A
dropped unscale, an unscale applied twice, or a clip taken on the scaled norm
each break the equality.
"""

import pytest
import torch

from oracle.optim import OracleApexW

SCALE = 1024.0


def _run(shapes, dtype, kw, amp, steps=3):
    gen = torch.Generator().manual_seed(5)
    ps = [torch.nn.Parameter((torch.randn(s, generator=gen) * 0.02).to(dtype)) for s in shapes]
    opt = OracleApexW(ps, **kw)
    ggen = torch.Generator().manual_seed(6)
    for _ in range(steps):
        for p in ps:
            g = (torch.randn(p.shape, generator=ggen) * 1e-3).to(dtype)
            p.grad = g * SCALE if amp else g
        if amp:
            opt.grad_scale = torch.tensor(SCALE)
            opt.found_inf = torch.tensor(0.0)
        opt.step()
    return ps, opt


CASES = [
    ("compact native bf16", [(64,), (32, 16)], torch.bfloat16, dict(precision="compact")),
    ("compact foreach bf16 quad", [(256, 128), (64,)], torch.bfloat16, dict(precision="compact")),
    ("compact foreach fp32", [(256, 128), (1000,)], torch.float32, dict(precision="compact", adamw_compat=True,
                                                                       stochastic_rounding=False)),
    ("8bit chunked + generic", [(1024, 512), (4096,)], torch.bfloat16, dict(precision="8bit")),
]


@pytest.mark.parametrize("gc", [False, True])
@pytest.mark.parametrize("clip", [None, 1e-3])
@pytest.mark.parametrize("name,shapes,dtype,kw", CASES, ids=[c[0] for c in CASES])
def test_pow2_grad_scale_equals_unscaled_step(name, shapes, dtype, kw, clip, gc):
    kw = dict(kw, lr=1e-3, weight_decay=0.1, clip_grad_norm=clip, grad_centralization=gc)
    kw.setdefault("stochastic_rounding", False)
    a, oa = _run(shapes, dtype, kw, amp=True)
    b, ob = _run(shapes, dtype, kw, amp=False)
    for pa, pb in zip(a, b):
        assert torch.equal(pa, pb), name
        for k, v in oa.state[pa].items():
            if torch.is_tensor(v):
                assert torch.equal(v, ob.state[pb][k]), (name, k)


def test_found_inf_skips_the_step():
    shapes = [(64, 32)]
    kw = dict(precision="compact", lr=1e-3, stochastic_rounding=False)
    gen = torch.Generator().manual_seed(1)
    p = torch.nn.Parameter(torch.randn(shapes[0], generator=gen))
    opt = OracleApexW([p], **kw)
    p.grad = torch.randn(shapes[0], generator=gen)
    opt.step()
    before = p.detach().clone()
    step = float(opt.state[p]["step"])
    opt.grad_scale, opt.found_inf = torch.tensor(SCALE), torch.tensor(1.0)
    p.grad = torch.full(shapes[0], float("inf"))
    opt.step()
    assert torch.equal(p.detach(), before) and float(opt.state[p]["step"]) == step
