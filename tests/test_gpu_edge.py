"""GPU edge cases of the fused step against the CPU oracle (SR off, the parity bars
of test_gpu_parity.py), plus size-independent properties at maximum sizes.

Covers what the reference's own tests exercise around the step: parameters
without grads, a changing set of active parameters (plan rebuild -> cold step),
several param groups, ragged sizes around unit / block boundaries, zero and
non-finite grads, AMP found_inf skips, checkpoint round trips, and a tensor of
more than 2^31 elements (64-bit indexing).
"""

import copy

import numpy as np
import pytest
import torch

from golden_replay import bf16_ulp_diff
from test_gpu_parity import _cmp_f16

pytestmark = pytest.mark.gpu


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")


def _pair(shapes, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    host = [(torch.randn(s, generator=g) * 0.02).to(dtype) for s in shapes]
    return ([torch.nn.Parameter(h.cuda()) for h in host], [torch.nn.Parameter(h.clone()) for h in host])


def _grads(shapes, dtype, seed, scale=1e-3):
    g = torch.Generator().manual_seed(seed)
    return [(torch.randn(s, generator=g) * scale).to(dtype) for s in shapes]


def _assert_close(gpu, cpu, what):
    got, ref = gpu.detach().cpu(), cpu.detach()
    if got.dtype == torch.bfloat16:
        d = bf16_ulp_diff(got.contiguous().reshape(-1), ref.contiguous().reshape(-1))
        assert int(d.max()) <= 1, f"{what}: {int(d.max())} ulps"
    elif got.dtype == torch.float32:
        err = (got.double() - ref.double()).abs() - (1e-6 * ref.double().abs() + 1e-9)
        assert float(err.max()) <= 0, f"{what}: excess {float(err.max()):.3e}"
    elif got.dtype == torch.float16:
        _cmp_f16(got.reshape(-1), ref.reshape(-1), what=what)
    else:
        a, b = got.reshape(-1).to(torch.int32), ref.reshape(-1).to(torch.int32)
        if got.dtype == torch.uint8:
            a = torch.stack([a >> 4, a & 15], 1).reshape(-1) if what.endswith("exp_avg") else a
            b = torch.stack([b >> 4, b & 15], 1).reshape(-1) if what.endswith("exp_avg") else b
        assert int((a - b).abs().max()) <= 1, f"{what}: codes differ by {int((a - b).abs().max())}"


def _compare(gps, cps, gopt, copt, tag):
    for i, (gp, cp) in enumerate(zip(gps, cps)):
        _assert_close(gp, cp, f"{tag} p{i}")
        gs, cs = gopt.state[gp], copt.state[cp]
        assert set(gs) == set(cs), f"{tag} p{i} state keys"
        for k in ("exp_avg", "exp_avg_sq", "exp_avg_scales", "exp_avg_sq_scales", "max_exp_avg_sq"):
            if k in cs and torch.is_tensor(cs[k]):
                assert gs[k].dtype == cs[k].dtype and gs[k].shape == cs[k].shape
                _assert_close(gs[k], cs[k], f"{tag} p{i} {k}")
        assert float(gs["step"]) == float(cs["step"])


RAGGED = [(1,), (3,), (63,), (64,), (65,), (2047,), (2048,), (2049,), (4095,), (4097,), (33, 65), (128, 129)]


@pytest.mark.parametrize("precision,dtype", [("compact", torch.bfloat16), ("compact", torch.float32),
                                             ("8bit", torch.bfloat16), ("8bit", torch.float32)])
def test_ragged_sizes_none_grads_and_active_set_changes(precision, dtype):
    _need_gpu()
    from apexw_amd import ApexW
    from oracle.optim import OracleApexW
    print(f"ragged {precision} {dtype}", flush=True)
    kw = dict(lr=1e-3, weight_decay=0.1, precision=precision, stochastic_rounding=False, adamw_compat=True)
    gps, cps = _pair(RAGGED, dtype, 1)
    gopt, copt = ApexW(gps, **kw), OracleApexW(cps, **kw)
    for step in range(6):
        grads = _grads(RAGGED, dtype, 100 + step)
        for i, (gp, cp, g) in enumerate(zip(gps, cps, grads)):
            # every third parameter has no grad on odd steps: the active set changes
            if step % 2 == 1 and i % 3 == 0:
                gp.grad, cp.grad = None, None
            else:
                gp.grad, cp.grad = g.cuda(), g.clone()
        gopt.step()
        copt.step()
    torch.cuda.synchronize()
    _compare(gps, cps, gopt, copt, f"{precision}/{dtype}")


def test_param_groups_zero_and_nonfinite_grads():
    _need_gpu()
    from apexw_amd import ApexW
    from oracle.optim import OracleApexW
    shapes = [(256, 64), (512,), (64, 64), (4096,)]
    gps, cps = _pair(shapes, torch.bfloat16, 2)

    def groups(ps):
        return [{"params": ps[:2], "lr": 2e-3, "weight_decay": 0.0},
                {"params": ps[2:], "lr": 5e-4, "weight_decay": 0.05, "betas": (0.8, 0.99)}]
    kw = dict(stochastic_rounding=False)
    gopt = ApexW(groups(gps), **kw)
    # the reference steps every param group independently (its own plan); the
    # oracle restates one group, so it runs one optimizer per group
    copts = [OracleApexW(g["params"], **kw, **{k: v for k, v in g.items() if k != "params"}) for g in groups(cps)]
    for step in range(5):
        grads = _grads(shapes, torch.bfloat16, 200 + step)
        grads[1].zero_()                              # all-zero grad: still stepped (decay, moments)
        if step == 0:                                 # the cold step sanitizes NaN/Inf
            grads[2][0, 0] = float("nan")
            grads[2][1, 1] = float("inf")
            grads[3][7] = float("-inf")
        for gp, cp, g in zip(gps, cps, grads):
            gp.grad, cp.grad = g.cuda(), g.clone()
        gopt.step()
        for o in copts:
            o.step()

    class _Both:
        state = {**copts[0].state, **copts[1].state}
    copt = _Both()
    torch.cuda.synchronize()
    _compare(gps, cps, gopt, copt, "groups")
    for p in gps:
        assert torch.isfinite(p.float()).all()


def test_found_inf_skips_the_step():
    _need_gpu()
    from apexw_amd import ApexW
    p = torch.nn.Parameter(torch.randn(1024, device="cuda"))
    opt = ApexW([p], lr=1e-2)
    p.grad = torch.randn(1024, device="cuda")
    opt.step()
    before = p.detach().clone()
    st = {k: v.clone() if torch.is_tensor(v) else v for k, v in opt.state[p].items()}
    opt.found_inf = torch.ones((), device="cuda")
    opt.step()
    assert torch.equal(p.detach(), before)
    assert float(opt.state[p]["step"]) == float(st["step"])


@pytest.mark.parametrize("precision", ["compact", "8bit"])
def test_checkpoint_resume_matches_oracle(precision):
    _need_gpu()
    from apexw_amd import ApexW
    shapes = [(300, 200), (4096,), (2048, 64)]
    kw = dict(lr=1e-3, weight_decay=0.1, precision=precision, stochastic_rounding=False)
    a, _ = _pair(shapes, torch.bfloat16, 3)
    b = [torch.nn.Parameter(p.detach().clone()) for p in a]
    oa = ApexW(a, **kw)
    grads = [_grads(shapes, torch.bfloat16, 300 + s) for s in range(6)]
    for s in range(6):
        for p, g in zip(a, grads[s]):
            p.grad = g.cuda()
        oa.step()
    ob = ApexW(b, **kw)
    for s in range(3):
        for p, g in zip(b, grads[s]):
            p.grad = g.cuda()
        ob.step()
    sd = copy.deepcopy(ob.state_dict())
    c = [torch.nn.Parameter(p.detach().clone()) for p in b]
    oc = ApexW(c, **kw)
    oc.load_state_dict(sd)
    for k, v in oc.state[c[0]].items():
        if torch.is_tensor(v):
            assert v.dtype == ob.state[b[0]][k].dtype, k
    for s in range(3, 6):
        for p, g in zip(c, grads[s]):
            p.grad = g.cuda()
        oc.step()
    torch.cuda.synchronize()
    # a resumed optimizer has no cached plan, so its first step is a cold step (as
    # the reference's after load_state_dict); the oracle reproduces the break by
    # dropping its plan at the same step
    from oracle.optim import OracleApexW
    r2 = _pair(shapes, torch.bfloat16, 3)[1]
    orf2 = OracleApexW(r2, **kw)
    for s in range(6):
        if s == 3:
            orf2._plan = None
        for p, g in zip(r2, grads[s]):
            p.grad = g.clone()
        orf2.step()
    _compare(c, r2, oc, orf2, f"resume {precision}")


def test_tensor_beyond_2_31_elements():
    """64-bit indexing: the last 2^19 elements (256 blocks) of a 2^31 + 4096-element
    bf16 tensor are updated exactly as the same data stepped alone (elements and
    quantization blocks are independent; both tensors exceed 262144 elements, so
    both take the reference's chunked rounding order)."""
    _need_gpu()
    from apexw_amd import ApexW
    free = torch.cuda.mem_get_info()[0]
    n = 2 ** 31 + 4096
    if free < 24 * 2 ** 30:
        pytest.skip("needs ~24 GiB of free device memory")
    print("big tensor", n, flush=True)
    tail = 2 ** 19
    for precision in ("8bit", "compact"):
        kw = dict(lr=1e-3, weight_decay=0.1, precision=precision, stochastic_rounding=False)
        big = torch.nn.Parameter(torch.zeros(n, dtype=torch.bfloat16, device="cuda"))
        g = torch.zeros(n, dtype=torch.bfloat16, device="cuda")
        gen = torch.Generator(device="cuda").manual_seed(9)
        seg = torch.randn(tail, generator=gen, device="cuda").bfloat16()
        big.data[-tail:] = seg * 0.02
        g[-tail:] = seg * 1e-3
        big.grad = g
        small = torch.nn.Parameter(big.data[-tail:].clone())
        small.grad = g[-tail:].clone()
        ob, osm = ApexW([big], **kw), ApexW([small], **kw)
        for _ in range(2):
            ob.step()
            osm.step()
        torch.cuda.synchronize()
        assert torch.equal(big.data[-tail:], small.data), precision
        if precision == "8bit":
            sb, ss = ob.state[big], osm.state[small]
            nb = tail // 2048
            assert torch.equal(sb["exp_avg_scales"].reshape(-1)[-nb:], ss["exp_avg_scales"].reshape(-1))
            assert torch.equal(sb["exp_avg"][-tail // 2:], ss["exp_avg"])
        del big, g, small, ob, osm
        torch.cuda.empty_cache()
