"""GPU: lion=True in the compact-kernel precisions (compact, full, auto).

The reference-written trajectories (compact_bf16 / compact_fp32 / auto_bf16 / fp16
_lion_rne) are replayed by test_gpu_parity.py.  Here, against the CPU oracle at the
bars of test_gpu_edge.py (bf16 / fp16 <= 1 ulp, fp32 1e-6 relative):

* ragged sizes in every dtype pairing, with weight decay, the clip and maximize
  (fp32 moments included: the reference's step raises IndexError for lion when its
  first tensor's m is fp32, so those runs are checked against the oracle's
  restatement of the lion ops only);
* stochastic_rounding=True changes nothing (lion rounds to nearest);
* lion switched on mid-run over AdamW states, quad v included (v is left as it is),
  and switched back off;
* lion switched off over states made under lion (no second moment): refused
  before any tensor moves.
"""

import pytest
import torch

from test_gpu_edge import RAGGED, _compare, _grads, _need_gpu, _pair

pytestmark = pytest.mark.gpu

RUNS = [("compact bf16", torch.bfloat16, dict(precision="compact", lr=1e-2)),
        ("compact fp32 p", torch.float32, dict(precision="compact")),
        ("compact fp16", torch.float16, dict(precision="compact", lr=1e-2)),
        ("full bf16 p", torch.bfloat16, dict(precision="full", lr=1e-2)),
        ("full fp32", torch.float32, dict(precision="full")),
        ("compact bf16 clip maximize", torch.bfloat16,
         dict(precision="compact", lr=1e-2, clip_grad_norm=1e-3, maximize=True)),
        ("compact bf16 sr on", torch.bfloat16, dict(precision="compact", lr=1e-2, stochastic_rounding=True))]


@pytest.mark.parametrize("name,dtype,kw", RUNS, ids=[r[0] for r in RUNS])
def test_lion_ragged_matches_oracle(name, dtype, kw):
    _need_gpu()
    from apexw_amd import ApexW
    from oracle.optim import OracleApexW
    print(f"lion ragged {name}", flush=True)
    kw = dict(dict(lr=1e-3, weight_decay=0.1, stochastic_rounding=False, lion=True), **kw)
    gps, cps = _pair(RAGGED, dtype, 51)
    # the oracle steps with SR off: lion never rounds stochastically
    gopt, copt = ApexW(gps, **kw), OracleApexW(cps, **dict(kw, stochastic_rounding=False))
    for step in range(4):
        for gp, cp, g in zip(gps, cps, _grads(RAGGED, dtype, 700 + step)):
            gp.grad, cp.grad = g.cuda(), g.clone()
        gopt.step()
        copt.step()
    torch.cuda.synchronize()
    assert all("exp_avg_sq" not in gopt.state[gp] for gp in gps)
    _compare(gps, cps, gopt, copt, f"lion {name}")


SHAPES = [(256, 128), (96, 200), (20000,), (300,), (40, 50), (7,)] + [(32, 32)] * 3


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_lion_switched_on_and_off_mid_run(dtype):
    _need_gpu()
    from apexw_amd import ApexW
    from oracle.optim import OracleApexW
    print(f"lion switched on / off {dtype}", flush=True)
    kw = dict(lr=1e-2, weight_decay=0.1, stochastic_rounding=False, threshold=4096)
    gps, cps = _pair(SHAPES, dtype, 52)            # 9 tensors: the large ones get quad v
    gopt, copt = ApexW(gps, **kw), OracleApexW(cps, **kw)
    for step in range(6):
        if step in (2, 4):
            on = step == 2
            gopt.param_groups[0]["lion"] = on
            copt.group["lion"] = on
        for gp, cp, g in zip(gps, cps, _grads(SHAPES, dtype, 800 + step)):
            gp.grad, cp.grad = g.cuda(), g.clone()
        gopt.step()
        copt.step()
        if step == 3:
            torch.cuda.synchronize()
            _compare(gps, cps, gopt, copt, f"lion on {dtype}")
    torch.cuda.synchronize()
    assert any(gopt.state[gp].get("is_quad_v", False) for gp in gps)
    _compare(gps, cps, gopt, copt, f"lion off {dtype}")


def test_lion_state_switched_to_adamw_is_refused():
    _need_gpu()
    from apexw_amd import ApexW
    print("lion state, lion off", flush=True)
    gps, _ = _pair(SHAPES, torch.bfloat16, 53)
    opt = ApexW(gps, lr=1e-2, stochastic_rounding=False, lion=True)
    for gp, g in zip(gps, _grads(SHAPES, torch.bfloat16, 900)):
        gp.grad = g.cuda()
    opt.step()
    before = [gp.detach().clone() for gp in gps]
    opt.param_groups[0]["lion"] = False
    with pytest.raises(NotImplementedError):
        opt.step()
    torch.cuda.synchronize()
    assert all(torch.equal(a, b) for a, b in zip(before, gps))
