"""GPU: grads of another dtype than their parameters (torch's Tensor.grad_dtype) in the
compact-kernel precisions.

The reference-written trajectories (gd_*_rne) are replayed by test_gpu_parity.py.
Here, against the CPU oracle at the bars of test_gpu_edge.py (bf16 / fp16 <= 1 ulp,
fp32 1e-6 relative):

* ragged sizes with fp32 grads for bf16 and fp16 parameters and bf16 grads for fp32
  parameters, plain and with nesterov, amsgrad, cautious, AMP's unscale and (bf16 grads)
  the clip;
* the grads' dtype switched mid-run (a new table, in the replay order as the
  reference's replayed plan steps it);
* refusals before any tensor moves: the 8-bit precision, the native fused order
  (torch._fused_adamw_ refuses such grads too), two grad dtypes for one parameter
  dtype.
"""

import pytest
import torch

from test_gpu_edge import RAGGED, _compare, _grads, _need_gpu, _pair

pytestmark = pytest.mark.gpu

RUNS = [("bf16 p fp32 g", torch.bfloat16, torch.float32, dict(precision="compact", fused=False)),
        ("fp32 p bf16 g", torch.float32, torch.bfloat16, dict(precision="compact")),
        ("fp16 p fp32 g", torch.float16, torch.float32, dict(precision="compact", fused=False)),
        ("bf16 p fp32 g full", torch.bfloat16, torch.float32, dict(precision="full")),
        ("bf16 p fp32 g nesterov", torch.bfloat16, torch.float32,
         dict(precision="compact", fused=False, nesterov=True)),
        # the clip on bf16 grads: norms rounded to bf16 (fp32 grads take the fp32-norm drift of
        # the reference's CPU reduction, as compact_fp32_clip_rne in test_gpu_parity.py)
        ("fp32 p bf16 g clip", torch.float32, torch.bfloat16, dict(precision="compact", clip_grad_norm=1e-3)),
        ("fp32 p bf16 g amsgrad cautious", torch.float32, torch.bfloat16,
         dict(precision="compact", amsgrad=True, cautious=True))]


def _with_grad_dtype(ps, gd):
    for p in ps:
        p.grad_dtype = gd
    return ps


@pytest.mark.parametrize("name,pdt,gdt,kw", RUNS, ids=[r[0] for r in RUNS])
def test_grad_dtype_ragged_matches_oracle(name, pdt, gdt, kw):
    _need_gpu()
    from apexw_amd import ApexW
    from oracle.optim import OracleApexW
    print(f"grad dtype ragged {name}", flush=True)
    kw = dict(dict(lr=1e-3, weight_decay=0.1, stochastic_rounding=False), **kw)
    gps, cps = _pair(RAGGED, pdt, 71)
    _with_grad_dtype(gps, gdt)
    _with_grad_dtype(cps, gdt)
    gopt, copt = ApexW(gps, **kw), OracleApexW(cps, **kw)
    for step in range(4):
        for gp, cp, g in zip(gps, cps, _grads(RAGGED, gdt, 1300 + step)):
            gp.grad, cp.grad = g.cuda(), g.clone()
        if step == 2:
            # AMP's unscale (GradScaler read on the host for this plan)
            gopt.grad_scale, copt.grad_scale = torch.tensor(1.0, device="cuda"), torch.tensor(1.0)
        gopt.step()
        copt.step()
    torch.cuda.synchronize()
    _compare(gps, cps, gopt, copt, f"grad dtype {name}")


SHAPES = [(256, 128), (96, 200), (20000,), (300,), (40, 50), (7,)] + [(32, 32)] * 3


def test_grad_dtype_switched_mid_run():
    _need_gpu()
    from apexw_amd import ApexW
    from oracle.optim import OracleApexW
    print("grad dtype switched", flush=True)
    kw = dict(lr=1e-3, weight_decay=0.1, stochastic_rounding=False, threshold=4096)
    gps, cps = _pair(SHAPES, torch.bfloat16, 72)      # 9 tensors: quad v for the large ones
    gopt, copt = ApexW(gps, **kw), OracleApexW(cps, **kw)
    for step in range(5):
        gdt = torch.float32 if step in (2, 3) else torch.bfloat16
        for gp, cp, g in zip(gps, cps, _grads(SHAPES, gdt, 1400 + step)):
            gp.grad = cp.grad = None
            gp.grad_dtype = cp.grad_dtype = gdt
            gp.grad, cp.grad = g.cuda(), g.clone()
        gopt.step()
        copt.step()
    torch.cuda.synchronize()
    _compare(gps, cps, gopt, copt, "grad dtype switched")


@pytest.mark.parametrize("case", ["8bit", "native", "two grad dtypes"])
def test_grad_dtype_refusals(case):
    _need_gpu()
    from apexw_amd import ApexW
    print(f"grad dtype refusal {case}", flush=True)
    shapes = [(256, 128), (300,)]
    gps, _ = _pair(shapes, torch.bfloat16, 73)
    gdts = [torch.float32, torch.float32]
    kw = dict(lr=1e-3, stochastic_rounding=False)
    if case == "8bit":
        kw["precision"] = "8bit"
    elif case == "native":
        kw["precision"] = "compact"       # two tensors, bf16 m / v: the native fused order
    else:
        gdts = [torch.float32, torch.float16]
        kw["fused"] = False
    for p, gd, g in zip(gps, gdts, _grads(shapes, torch.float32, 1500)):
        p.grad_dtype = gd
        p.grad = g.to(gd).cuda()
    opt = ApexW(gps, **kw)
    before = [p.detach().clone() for p in gps]
    with pytest.raises((NotImplementedError, RuntimeError)):
        opt.step()
    torch.cuda.synchronize()
    assert all(torch.equal(a, b) for a, b in zip(before, gps))
