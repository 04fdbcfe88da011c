"""GPU: beta3 (AdEMAMix) in the compact-kernel precisions (compact, full, auto).

The reference-written trajectories (*_beta3_rne) are replayed by test_gpu_parity.py.
Here, against the CPU oracle at the bars of test_gpu_edge.py (bf16 / fp16 <= 1 ulp,
fp32 1e-6 relative), with exp_avg_slow compared too:

* ragged sizes in every dtype pairing, with amsgrad, nesterov (ignored under beta3,
  as in the reference) and the clip;
* fp32 parameters at a floor of 4e-9 instead of 1e-9 (FP32_FLOOR: the reference's CPU
  sqrt against the kernel's IEEE one, under beta3's larger updates);
* stochastic_rounding=True at beta2 = 0.99: the beta3 update is a round-to-nearest
  addcdiv and v stays on the rounded path, so the oracle's SR-on run is exact;
* beta3 set mid-run (a zero slow moment is made, as the reference's _init_group does)
  and cleared again (a new plan each time, as the reference's validity rule gives);
* beta3 set over a quad-v state: refused before any tensor moves.
"""

import pytest
import torch

from test_gpu_edge import RAGGED, _assert_close, _compare, _grads, _need_gpu, _pair

pytestmark = pytest.mark.gpu

RUNS = [("compact bf16", torch.bfloat16, dict(precision="compact", beta3=0.9999)),
        ("compact fp32 p", torch.float32, dict(precision="compact", beta3=0.999, alpha=2.0)),
        ("full bf16 p", torch.bfloat16, dict(precision="full", beta3=0.9999)),
        ("full fp32", torch.float32, dict(precision="full", beta3=0.9999)),
        ("compact fp16", torch.float16, dict(precision="compact", beta3=0.999)),
        ("compact bf16 amsgrad nesterov clip", torch.bfloat16,
         dict(precision="compact", beta3=0.999, amsgrad=True, nesterov=True, clip_grad_norm=1e-3)),
        ("compact bf16 sr on", torch.bfloat16,
         dict(precision="compact", beta3=0.9999, stochastic_rounding=True, betas=(0.9, 0.99)))]


# fp32 parameters: torch's CPU fp32 sqrt is faithfully, not correctly, rounded (1 ulp off
# on ~0.5% of the elements of a vectorised sqrt on AVX512 hosts, against numpy's), where
# the kernel's is IEEE; a one-ulp denominator moves the update by 2^-23 of itself, and
# beta3's update at slow_ratio ~5000 is ~6e-3 per step, so 4 steps may differ by ~2e-9
# in absolute terms where p is near 0: the fp32 floor is 4e-9 here instead of 1e-9
FP32_FLOOR = 4e-9


def _compare_slow(gps, cps, gopt, copt, tag):
    for i, (gp, cp) in enumerate(zip(gps, cps)):
        if gp.dtype == torch.float32:
            got, ref = gp.detach().cpu().double(), cp.detach().double()
            err = (got - ref).abs() - (1e-6 * ref.abs() + FP32_FLOOR)
            assert float(err.max()) <= 0, f"{tag} p{i}: excess {float(err.max()):.3e}"
    keep = [(gp, cp) for gp, cp in zip(gps, cps) if gp.dtype != torch.float32]
    if keep:
        _compare([k[0] for k in keep], [k[1] for k in keep], gopt, copt, tag)
    for i, (gp, cp) in enumerate(zip(gps, cps)):
        gs, cs = gopt.state[gp], copt.state[cp]
        assert set(gs) == set(cs), f"{tag} p{i} state keys"
        for k in ("exp_avg", "exp_avg_sq", "exp_avg_slow", "max_exp_avg_sq"):
            if k in cs:
                assert gs[k].dtype == cs[k].dtype and gs[k].shape == cs[k].shape
                _assert_close(gs[k], cs[k], f"{tag} p{i} {k}")
        assert float(gs["step"]) == float(cs["step"])


@pytest.mark.parametrize("name,dtype,kw", RUNS, ids=[r[0] for r in RUNS])
def test_beta3_ragged_matches_oracle(name, dtype, kw):
    _need_gpu()
    from apexw_amd import ApexW
    from oracle.optim import OracleApexW
    print(f"beta3 ragged {name}", flush=True)
    kw = dict(dict(lr=1e-3, weight_decay=0.1, stochastic_rounding=False), **kw)
    gps, cps = _pair(RAGGED, dtype, 61)
    gopt, copt = ApexW(gps, **kw), OracleApexW(cps, **kw)
    for step in range(4):
        for gp, cp, g in zip(gps, cps, _grads(RAGGED, dtype, 1000 + step)):
            gp.grad, cp.grad = g.cuda(), g.clone()
        gopt.step()
        copt.step()
    torch.cuda.synchronize()
    _compare_slow(gps, cps, gopt, copt, f"beta3 {name}")


SHAPES = [(256, 128), (96, 200), (20000,), (300,), (40, 50), (7,)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_beta3_set_and_cleared_mid_run(dtype):
    _need_gpu()
    from apexw_amd import ApexW
    from oracle.optim import OracleApexW
    print(f"beta3 set / cleared {dtype}", flush=True)
    kw = dict(lr=1e-3, weight_decay=0.1, stochastic_rounding=False, threshold=4096)
    gps, cps = _pair(SHAPES, dtype, 62)            # fewer than 8 tensors: no quad v
    gopt, copt = ApexW(gps, **kw), OracleApexW(cps, **kw)
    for step in range(6):
        if step in (2, 4):
            b3 = 0.999 if step == 2 else None
            gopt.param_groups[0]["beta3"] = b3
            copt.group["beta3"] = b3
        for gp, cp, g in zip(gps, cps, _grads(SHAPES, dtype, 1100 + step)):
            gp.grad, cp.grad = g.cuda(), g.clone()
        gopt.step()
        copt.step()
        if step == 3:
            torch.cuda.synchronize()
            _compare_slow(gps, cps, gopt, copt, f"beta3 set {dtype}")
    torch.cuda.synchronize()
    _compare_slow(gps, cps, gopt, copt, f"beta3 cleared {dtype}")


def test_beta3_over_quad_state_is_refused():
    _need_gpu()
    from apexw_amd import ApexW
    print("beta3 over quad v", flush=True)
    shapes = SHAPES + [(32, 32)] * 3               # 8 or more tensors: the large ones get quad v
    gps, _ = _pair(shapes, torch.bfloat16, 63)
    opt = ApexW(gps, lr=1e-3, stochastic_rounding=False, threshold=4096)
    for gp, g in zip(gps, _grads(shapes, torch.bfloat16, 1200)):
        gp.grad = g.cuda()
    opt.step()
    assert any(opt.state[gp].get("is_quad_v", False) for gp in gps)
    before = [gp.detach().clone() for gp in gps]
    opt.param_groups[0]["beta3"] = 0.999
    with pytest.raises(NotImplementedError):
        opt.step()
    torch.cuda.synchronize()
    assert all(torch.equal(a, b) for a, b in zip(before, gps))
