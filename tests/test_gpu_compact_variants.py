"""GPU: nesterov=True and cautious=True in the compact-kernel precisions (compact,
full, auto).

The reference-written trajectories (compact_*/full_*/auto_*_{nesterov,cautious}_rne)
are replayed by test_gpu_parity.py.  Here, against the CPU oracle at the bars of
test_gpu_edge.py (bf16 <= 1 ulp, fp32 1e-6 relative):

* stochastic_rounding=True: the nesterov and cautious updates of non-quad tensors
  are addcdiv passes rounded to nearest (never stochastic), and beta2 = 0.99 keeps
  v on the rounded path, so the step is deterministic and the oracle's SR-on run is
  its exact reference (nesterov gives no tensor quad v; the cautious run uses fewer
  than 8 tensors, which get none either);
* the option switched on mid-run: the replayed plan takes it in place (as the
  reference's does), and the quad-v tensors made before the switch step with
  lerp(g, m, beta1) (nesterov) or the fp32 mask (cautious).
"""

import pytest
import torch

from test_gpu_edge import _compare, _grads, _need_gpu, _pair

pytestmark = pytest.mark.gpu

SHAPES = [(256, 128), (64, 512), (20000,), (300,), (40, 50), (7,)]


SMALL = [(64, 128), (2000,), (300,), (40, 50), (7,)]
VARIANTS = [("nesterov", p, d) for p, d in (("compact", torch.bfloat16), ("compact", torch.float32),
                                             ("full", torch.bfloat16), ("auto", torch.bfloat16))]
VARIANTS += [("cautious", p, d) for p, d in (("compact", torch.bfloat16), ("compact", torch.float32),
                                              ("full", torch.bfloat16), ("full", torch.float32))]


@pytest.mark.parametrize("option,precision,dtype", VARIANTS, ids=[f"{o}-{p}-{d}" for o, p, d in VARIANTS])
def test_variant_with_sr_on_is_deterministic(option, precision, dtype):
    _need_gpu()
    from apexw_amd import ApexW
    from oracle.optim import OracleApexW
    print(f"{option} sr-on {precision} {dtype}", flush=True)
    kw = dict(lr=1e-3, weight_decay=0.1, precision=precision, stochastic_rounding=True, betas=(0.9, 0.99),
              threshold=4096, **{option: True})
    shapes = SHAPES if option == "nesterov" else SMALL
    gps, cps = _pair(shapes, dtype, 31)
    gopt, copt = ApexW(gps, **kw), OracleApexW(cps, **kw)
    for step in range(5):
        for gp, cp, g in zip(gps, cps, _grads(shapes, dtype, 200 + step)):
            gp.grad, cp.grad = g.cuda(), g.clone()
        gopt.step()
        copt.step()
    torch.cuda.synchronize()
    for gp in gps:
        assert not gopt.state[gp].get("is_quad_v", False)
    _compare(gps, cps, gopt, copt, f"{option} sr {precision}")


@pytest.mark.parametrize("option", ["nesterov", "cautious"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_variant_switched_on_mid_run(option, dtype):
    _need_gpu()
    from apexw_amd import ApexW
    from oracle.optim import OracleApexW
    print(f"{option} switched on {dtype}", flush=True)
    kw = dict(lr=1e-3, weight_decay=0.1, stochastic_rounding=False, threshold=4096)
    shapes = SHAPES + [(32, 32)] * 3          # 8 or more tensors: the large ones get quad v
    gps, cps = _pair(shapes, dtype, 32)
    gopt, copt = ApexW(gps, **kw), OracleApexW(cps, **kw)
    for step in range(5):
        if step == 2:
            gopt.param_groups[0][option] = True
            copt.group[option] = True
        for gp, cp, g in zip(gps, cps, _grads(shapes, dtype, 300 + step)):
            gp.grad, cp.grad = g.cuda(), g.clone()
        gopt.step()
        copt.step()
    torch.cuda.synchronize()
    assert any(gopt.state[gp].get("is_quad_v", False) for gp in gps)
    _compare(gps, cps, gopt, copt, f"{option} switched on {dtype}")
