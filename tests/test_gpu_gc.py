"""GPU: gradient centralization (grad_centralization=True) against the CPU oracle.

Compact, 8-bit and ultra groups fold it into the step and the clip
(apexw_grad_row_means writes one mean per row, the kernels subtract it from the
raw grad: compact descriptors carry the means, 8-bit / ultra ones a side table);
groups with factored tensors read a prepared copy (apexw_grad_prepare).
* the prepared grads (8-bit plan with a factored tensor: sanitized, centralized
  per row of every dim >= 2 grad) vs the oracle's _prepare_grads, and the row
  means (compact plan) vs torch's mean of the sanitized grads: bf16 within 1
  ulp (the row mean is a sum in a different order, rounded to bf16), fp32
  within 1e-6 of the row's largest |g|;
* full steps with bf16 params (compact, 8-bit with and without a full-block
  NF4 tensor, ultra; SR off) at the parity bars of test_gpu_parity.py;
* with AMP and the clip as well: the 2^10-scaled step equals the unscaled one
  bit for bit (unscale before centralizing, clip on centralized grads).
"""

import numpy as np
import pytest
import torch

from golden_replay import bf16_ulp_diff
from test_gpu_edge import _compare

pytestmark = pytest.mark.gpu

SHAPES = [(256, 128), (33, 65), (4, 4, 16), (4096,), (64, 2048)]


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_row_means_match_oracle(dtype):
    _need_gpu()
    from apexw_amd import ApexW
    from oracle.compact import sanitize_grads
    print(f"gc row means {dtype}", flush=True)
    gen = torch.Generator().manual_seed(11)
    host = [(torch.randn(s, generator=gen) * 0.02).to(dtype) for s in SHAPES]
    grads = [(torch.randn(s, generator=gen) * 1e-3 + 5e-4).to(dtype) for s in SHAPES]
    grads[0][3, 7] = float("nan")
    gps = [torch.nn.Parameter(h.cuda()) for h in host]
    for p, g in zip(gps, grads):
        p.grad = g.cuda()
    opt = ApexW(gps, lr=1e-3, grad_centralization=True, stochastic_rounding=False)
    opt.step()
    torch.cuda.synchronize()
    plan = next(iter(opt._plans.values()))
    assert plan.gc_fold
    for i, g in enumerate(sanitize_grads([g.clone() for g in grads])):
        if g.dim() < 2:
            continue
        ref = g.mean(dim=tuple(range(1, g.dim()))).reshape(-1)       # torch's mean in the grad dtype
        got = plan.gc_means[i].cpu()
        assert got.numel() == ref.numel()
        if dtype == torch.bfloat16:
            assert torch.equal(got.bfloat16().float(), got), i          # the means are bf16 values
            d = bf16_ulp_diff(got.bfloat16(), ref)
            assert int(d.max()) <= 1, (i, int(d.max()))
        else:
            tol = 1e-6 * g.reshape(g.shape[0], -1).abs().amax(dim=1)
            assert bool(((got.double() - ref.double()).abs() <= tol.double()).all()), i


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_prepared_grads_match_oracle(dtype):
    _need_gpu()
    from apexw_amd import ApexW
    from oracle.optim import OracleApexW
    print(f"gc prepared {dtype}", flush=True)
    gen = torch.Generator().manual_seed(11)
    # (256, 512) is factored with factored_v=True (>= 65536 elements, >= 128 rows and columns); no
    # thin matrix such as (64, 2048), which would make the group look like an adapter (no factoring)
    shapes = [s for s in SHAPES if s != (64, 2048)] + [(256, 512)]
    host = [(torch.randn(s, generator=gen) * 0.02).to(dtype) for s in shapes]
    grads = [(torch.randn(s, generator=gen) * 1e-3 + 5e-4).to(dtype) for s in shapes]
    grads[0][3, 7] = float("nan")
    gps = [torch.nn.Parameter(h.cuda()) for h in host]
    for p, g in zip(gps, grads):
        p.grad = g.cuda()
    # a group with a factored tensor steps a prepared copy of the grads
    opt = ApexW(gps, lr=1e-3, grad_centralization=True, stochastic_rounding=False, precision="8bit",
                factored_v=True)
    opt.step()
    torch.cuda.synchronize()
    plan = next(iter(opt._plans.values()))
    assert plan.factored.any() and not plan.gc_fold
    cps = [torch.nn.Parameter(h.clone()) for h in host]
    ref, _ = OracleApexW(cps, grad_centralization=True)._prepare([g.clone() for g in grads], sanitize=True)
    for i, (out, r) in enumerate(zip(plan.gc_out, ref)):
        got = out.cpu().reshape(r.shape)
        if dtype == torch.bfloat16:
            d = bf16_ulp_diff(got.reshape(-1), r.reshape(-1))
            assert int(d.max()) <= 1, (i, int(d.max()))
        else:
            rows = r.reshape(r.shape[0], -1) if r.dim() >= 2 else r.reshape(1, -1)
            tol = 1e-6 * rows.abs().amax(dim=1, keepdim=True)
            err = (got.reshape(rows.shape).double() - rows.double()).abs() - tol.double()
            assert float(err.max()) <= 0, (i, float(err.max()))


@pytest.mark.parametrize("precision,extra", [("compact", ()), ("8bit", ()), ("8bit", ((512, 1024), (300, 2048))),
                                             ("ultra", ())], ids=["compact", "8bit", "8bit-fullblock", "ultra"])
def test_gc_steps_match_oracle_bf16(precision, extra):
    """4 steps; "8bit-fullblock" adds tensors of more than 2^18 elements (the
    full-block NF4 kernel, its centralized instantiation) with rows of 1024 and
    2048 elements."""
    _need_gpu()
    from apexw_amd import ApexW
    from oracle.optim import OracleApexW
    print(f"gc steps {precision} {extra}", flush=True)
    kw = dict(lr=1e-3, weight_decay=0.1, precision=precision, stochastic_rounding=False, grad_centralization=True)
    if precision == "ultra":
        kw["threshold"] = 4096
    gen = torch.Generator().manual_seed(12)
    host = [(torch.randn(s, generator=gen) * 0.02).bfloat16() for s in SHAPES + list(extra)]
    gps = [torch.nn.Parameter(h.cuda()) for h in host]
    cps = [torch.nn.Parameter(h.clone()) for h in host]
    gopt, copt = ApexW(gps, **kw), OracleApexW(cps, **kw)
    for _ in range(4):
        for gp, cp in zip(gps, cps):
            g = (torch.randn(gp.shape, generator=gen) * 1e-3).bfloat16()
            gp.grad, cp.grad = g.cuda(), g.clone()
        gopt.step()
        copt.step()
    torch.cuda.synchronize()
    plan = next(iter(gopt._plans.values()))
    assert plan.gc_fold
    if extra:
        assert plan.fast is not None and plan.fast.any(), "no tensor took the full-block kernel"
    _compare(gps, cps, gopt, copt, f"gc {precision}")


@pytest.mark.parametrize("precision,dtype", [("compact", torch.bfloat16), ("compact", torch.float32),
                                             ("8bit", torch.bfloat16), ("8bit", torch.float32),
                                             ("ultra", torch.bfloat16)])
def test_gc_with_amp_and_clip_equals_unscaled(precision, dtype):
    _need_gpu()
    from apexw_amd import ApexW
    print(f"gc amp clip {precision} {dtype}", flush=True)
    kw = dict(lr=1e-3, weight_decay=0.1, precision=precision, stochastic_rounding=False, grad_centralization=True,
              clip_grad_norm=1e-3)
    gen = torch.Generator().manual_seed(13)
    host = [(torch.randn(s, generator=gen) * 0.02).to(dtype) for s in SHAPES]
    pa = [torch.nn.Parameter(h.cuda()) for h in host]
    pb = [torch.nn.Parameter(h.cuda()) for h in host]
    oa, ob = ApexW(pa, **kw), ApexW(pb, **kw)
    for _ in range(3):
        for a, b in zip(pa, pb):
            g = (torch.randn(a.shape, generator=gen) * 1e-3).to(dtype)
            a.grad, b.grad = (g * 1024.0).cuda(), g.cuda()
        oa.grad_scale, oa.found_inf = torch.tensor(1024.0, device="cuda"), torch.zeros((), device="cuda")
        oa.step()
        ob.step()
    torch.cuda.synchronize()
    for a, b in zip(pa, pb):
        assert torch.equal(a, b)
