"""GPU: amsgrad=True in the compact-kernel precisions (compact, full, auto).

The reference-written trajectories (*_amsgrad_*_rne) are replayed by
test_gpu_parity.py.  Here, against the CPU oracle at the bars of test_gpu_edge.py
(bf16 / fp16 <= 1 ulp, fp32 1e-6 relative), with max_exp_avg_sq compared too:

* ragged sizes (the element-wise tails of the 8-element groups) in the native
  fused order, the foreach order (fused=False) and with fp32 moments;
* amsgrad switched on mid-run (a zero max is made, as the reference's
  _init_group does) and off again (a new plan; the max is kept, unused);
* amsgrad switched on over a quad-v state: refused before any tensor moves.

At larger sizes, with stochastic rounding on (no oracle bit pattern to match),
the property amsgrad defines: after every step max_exp_avg_sq is exactly the
running element-wise maximum of v.
"""

import pytest
import torch

from test_gpu_edge import RAGGED, _compare, _grads, _need_gpu, _pair

pytestmark = pytest.mark.gpu

ORDERS = [("native bf16", torch.bfloat16, dict(precision="compact")),
          ("foreach bf16", torch.bfloat16, dict(precision="compact", fused=False)),
          ("foreach fp32 p", torch.float32, dict(precision="compact")),
          ("full bf16 p", torch.bfloat16, dict(precision="full")),
          ("native fp16", torch.float16, dict(precision="compact", betas=(0.9, 0.5))),
          ("foreach fp16", torch.float16, dict(precision="compact", fused=False))]


@pytest.mark.parametrize("name,dtype,kw", ORDERS, ids=[o[0] for o in ORDERS])
def test_amsgrad_ragged_matches_oracle(name, dtype, kw):
    _need_gpu()
    from apexw_amd import ApexW
    from oracle.optim import OracleApexW
    print(f"amsgrad ragged {name}", flush=True)
    kw = dict(kw, lr=1e-3, weight_decay=0.1, stochastic_rounding=False, amsgrad=True)
    gps, cps = _pair(RAGGED, dtype, 41)
    gopt, copt = ApexW(gps, **kw), OracleApexW(cps, **kw)
    for step in range(4):
        for gp, cp, g in zip(gps, cps, _grads(RAGGED, dtype, 400 + step)):
            gp.grad, cp.grad = g.cuda(), g.clone()
        gopt.step()
        copt.step()
    torch.cuda.synchronize()
    assert all("max_exp_avg_sq" in gopt.state[gp] for gp in gps)
    _compare(gps, cps, gopt, copt, f"amsgrad {name}")


SHAPES = [(256, 128), (96, 200), (20000,), (300,), (40, 50), (7,)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_amsgrad_switched_on_and_off_mid_run(dtype):
    _need_gpu()
    from apexw_amd import ApexW
    from oracle.optim import OracleApexW
    print(f"amsgrad switched on / off {dtype}", flush=True)
    kw = dict(lr=1e-3, weight_decay=0.1, stochastic_rounding=False, threshold=4096, fused=False)
    gps, cps = _pair(SHAPES, dtype, 42)            # fewer than 8 tensors: no quad v
    gopt, copt = ApexW(gps, **kw), OracleApexW(cps, **kw)
    for step in range(6):
        if step in (2, 4):
            on = step == 2
            gopt.param_groups[0]["amsgrad"] = on
            copt.group["amsgrad"] = on
        for gp, cp, g in zip(gps, cps, _grads(SHAPES, dtype, 500 + step)):
            gp.grad, cp.grad = g.cuda(), g.clone()
        gopt.step()
        copt.step()
        if step == 3:
            torch.cuda.synchronize()
            _compare(gps, cps, gopt, copt, f"amsgrad on {dtype}")
    torch.cuda.synchronize()
    _compare(gps, cps, gopt, copt, f"amsgrad off {dtype}")


def test_amsgrad_over_quad_state_is_refused():
    _need_gpu()
    from apexw_amd import ApexW
    print("amsgrad over quad v", flush=True)
    shapes = SHAPES + [(32, 32)] * 3               # 8 or more tensors: the large ones get quad v
    gps, _ = _pair(shapes, torch.bfloat16, 43)
    opt = ApexW(gps, lr=1e-3, stochastic_rounding=False, threshold=4096)
    for gp, g in zip(gps, _grads(shapes, torch.bfloat16, 600)):
        gp.grad = g.cuda()
    opt.step()
    assert any(opt.state[gp].get("is_quad_v", False) for gp in gps)
    before = [gp.detach().clone() for gp in gps]
    opt.param_groups[0]["amsgrad"] = True
    with pytest.raises(NotImplementedError):
        opt.step()
    torch.cuda.synchronize()
    assert all(torch.equal(a, b) for a, b in zip(before, gps))


@pytest.mark.parametrize("precision,dtype,betas,fused", [("compact", torch.bfloat16, (0.9, 0.999), False),
                                                         ("compact", torch.bfloat16, (0.9, 0.95), None),
                                                         ("full", torch.float32, (0.9, 0.999), None)])
def test_amsgrad_keeps_the_running_max_of_v(precision, dtype, betas, fused):
    """SR on (the foreach order rounds v stochastically at beta2 0.999), 4 tensors of
    3-17 M elements: max_exp_avg_sq after each step equals the element-wise maximum of
    its value before the step and the new v, bit for bit."""
    _need_gpu()
    from apexw_amd import ApexW
    print(f"amsgrad running max {precision} {dtype} {betas} fused={fused}", flush=True)
    shapes = [(4096, 4096), (1 << 22,), (2048, 2048 + 8), (3001, 1001)]
    gen = torch.Generator(device="cuda").manual_seed(44)
    ps = [torch.nn.Parameter((torch.randn(s, device="cuda", generator=gen) * 0.02).to(dtype)) for s in shapes]
    opt = ApexW(ps, lr=1e-3, weight_decay=0.1, precision=precision, betas=betas, amsgrad=True,
                stochastic_rounding=True, fused=fused)
    prev = None
    for step in range(5):
        # the grad scale shrinks and grows, so v falls below its running max in places
        scale = 1e-3 * (0.1 if step % 2 else 1.0)
        for p in ps:
            p.grad = (torch.randn(p.shape, device="cuda", generator=gen) * scale).to(dtype)
        opt.step()
        cur = [(opt.state[p]["max_exp_avg_sq"].clone(), opt.state[p]["exp_avg_sq"].clone()) for p in ps]
        for i, (mx, v) in enumerate(cur):
            want = v if prev is None else torch.maximum(prev[i][0], v)
            assert torch.equal(mx, want), f"step {step} tensor {i}"
        prev = cur
    assert any(bool((mx != v).any()) for mx, v in prev)
