"""The step's error convention: a refused launch changes nothing and never double-steps.

The reference validates a fused launch before it mutates anything and rolls the
step counters back when the launch is refused (apexw/optimizer.py:3184-3356,
:3806); its test checks that a refused 8-bit launch leaves the step counter at
exactly one increment and the other tensors unmutated
(tests/test_quantization.py:238-263).  Here a step prepares every parameter
group (counters advanced, every launch's arguments checked by the library's
apexw_check_launch) before any group runs.

The refusals are forced on the host: the plan's library handle is wrapped so
that one call returns APEXW_ERR_ARG.  Nothing reaches the device for a refused
launch, so no kernel is disturbed.
"""

import pytest
import torch

from apexw_amd import ApexW
from apexw_amd import _lib as L

pytestmark = pytest.mark.gpu


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")


class _Refuse:
    """Library proxy: `name` returns APEXW_ERR_ARG (1) on its first `after`+1-th call and
    forwards every other call."""

    def __init__(self, lib, name, after=0):
        self._lib, self._name, self._after, self.calls = lib, name, after, 0

    def __getattr__(self, attr):
        fn = getattr(self._lib, attr)
        if attr != self._name:
            return fn

        def wrapped(*args):
            self.calls += 1
            if self.calls == self._after + 1:
                return 1
            return fn(*args)
        return wrapped


def _model(precisions, seed=0):
    g = torch.Generator().manual_seed(seed)
    shapes = [(256, 1024), (4096,), (300, 64)]
    groups = []
    for prec in precisions:
        ps = [torch.nn.Parameter((torch.randn(s, generator=g) * 0.02).bfloat16().cuda()) for s in shapes]
        groups.append({"params": ps, "precision": prec})
    return groups


def _set_grads(groups, seed):
    g = torch.Generator().manual_seed(seed)
    for grp in groups:
        for p in grp["params"]:
            p.grad = (torch.randn(p.shape, generator=g) * 1e-3).bfloat16().cuda()


def _snapshot(opt, groups):
    out = []
    for grp in groups:
        for p in grp["params"]:
            st = opt.state[p]
            out.append((p.detach().clone(), {k: (v.detach().clone() if torch.is_tensor(v) else v)
                                             for k, v in st.items()}))
    return out


def _assert_same(opt, groups, snap, which):
    i = 0
    for gi, grp in enumerate(groups):
        for p in grp["params"]:
            p0, st0 = snap[i]
            i += 1
            if gi not in which:
                continue
            assert torch.equal(p.detach(), p0), f"group {gi}: parameter changed"
            st = opt.state[p]
            for k, v in st0.items():
                if torch.is_tensor(v):
                    assert torch.equal(st[k].detach(), v), f"group {gi}: state {k} changed"


@pytest.mark.parametrize("precisions", [("8bit", "8bit"), ("compact", "8bit"), ("8bit", "compact")])
def test_refused_second_group_changes_nothing(precisions):
    """The second group's launch check refuses: step() raises, and neither group's
    parameters, states nor step counters move; the next step() is an ordinary one."""
    _need_gpu()
    groups = _model(precisions)
    opt = ApexW(groups, lr=1e-3, weight_decay=0.1, stochastic_rounding=False)
    _set_grads(groups, 1)
    opt.step()
    _set_grads(groups, 2)
    torch.cuda.synchronize()
    snap = _snapshot(opt, groups)
    plan2 = opt._plans[id(opt.param_groups[1])]
    lib = plan2._lib
    plan2._lib = _Refuse(lib, "apexw_check_launch")
    with pytest.raises(L.ApexwError):
        opt.step()
    plan2._lib = lib
    torch.cuda.synchronize()
    _assert_same(opt, groups, snap, which={0, 1})
    for grp in groups:
        for p in grp["params"]:
            assert int(opt.state[p]["step"]) == 1
    # not refused: every counter advances by exactly one, and the groups step as a clean
    # optimizer fed the same two steps does
    opt.step()
    torch.cuda.synchronize()
    ref_groups = _model(precisions)
    ref = ApexW(ref_groups, lr=1e-3, weight_decay=0.1, stochastic_rounding=False)
    _set_grads(ref_groups, 1)
    ref.step()
    _set_grads(ref_groups, 2)
    ref.step()
    torch.cuda.synchronize()
    for grp, rgrp in zip(groups, ref_groups):
        for p, rp in zip(grp["params"], rgrp["params"]):
            assert int(opt.state[p]["step"]) == 2
            assert torch.equal(p.detach(), rp.detach())


def test_failed_launch_rolls_back_its_group_only():
    """The second group's step entry point itself returns an error while running: the
    first group has stepped (its counters advance), the second group's counters are
    restored and its tensors untouched."""
    _need_gpu()
    groups = _model(("8bit", "8bit"))
    opt = ApexW(groups, lr=1e-3, weight_decay=0.1, stochastic_rounding=False)
    _set_grads(groups, 1)
    opt.step()
    _set_grads(groups, 2)
    torch.cuda.synchronize()
    snap = _snapshot(opt, groups)
    plan2 = opt._plans[id(opt.param_groups[1])]
    lib = plan2._lib
    plan2._lib = _Refuse(lib, "apexw_q8_step")
    with pytest.raises(L.ApexwError):
        opt.step()
    plan2._lib = lib
    torch.cuda.synchronize()
    _assert_same(opt, groups, snap, which={1})
    for p in groups[0]["params"]:
        assert int(opt.state[p]["step"]) == 2
    for p in groups[1]["params"]:
        assert int(opt.state[p]["step"]) == 1


def test_refused_hook_batch_restores_counters():
    """In-backward 8-bit steps: a refused batch leaves every queued parameter's pass and
    step counters where they were."""
    _need_gpu()
    torch.manual_seed(0)
    layers = torch.nn.Sequential(*[torch.nn.Linear(256, 256, bias=False) for _ in range(10)]).cuda().bfloat16()
    opt = ApexW(layers.parameters(), lr=1e-3, precision="8bit", stochastic_rounding=False)
    if not opt._auto_hook_handles:
        pytest.skip("in-backward steps not enabled for this model")
    x = torch.randn(8, 256, device="cuda", dtype=torch.bfloat16)
    layers(x).float().square().mean().backward()
    opt.step()
    torch.cuda.synchronize()
    params = list(layers.parameters())
    before = {id(p): (opt.state[p].get("_hook_mstep", 0), float(opt.state[p]["step"])) for p in params}
    weights = [p.detach().clone() for p in params]
    orig = opt._hook_plan

    def refusing(group, ps):
        plan = orig(group, ps)
        if not isinstance(plan._lib, _Refuse):
            plan._lib = _Refuse(plan._lib, "apexw_check_launch")
        return plan
    opt._hook_plan = refusing
    with pytest.raises(L.ApexwError):
        layers(x).float().square().mean().backward()
    opt._hook_plan = orig
    torch.cuda.synchronize()
    for p, w in zip(params, weights):
        assert (opt.state[p].get("_hook_mstep", 0), float(opt.state[p]["step"])) == before[id(p)]
        assert torch.equal(p.detach(), w)
