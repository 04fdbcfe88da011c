"""The execution-plan host logic, exercised on the CPU with the kernel launches recorded.

The plan builds device tables from tensor pointers and launches through the
C ABI; here the ABI step functions are replaced by recorders (no GPU), so table
layout, unit splitting, fast/general partition, cold/replay mode and the
host-computed scalars are checked without touching a device.
"""

import ctypes

import numpy as np
import pytest
import torch

from apexw_amd import _lib as L
from apexw_amd import _plan


class _Recorder:
    def __init__(self, real):
        self.real = real
        self.calls = []

    def __getattr__(self, name):
        return getattr(self.real, name)

    def _rec(self, name, args):
        hp = ctypes.cast(args[-2], ctypes.POINTER(L.HParams)).contents if name != "clip" else None
        self.calls.append((name, args, None if hp is None else {f: getattr(hp, f) for f, _ in L.HParams._fields_}))
        return 0

    def apexw_compact_step(self, *a):
        return self._rec("compact", a)

    def apexw_q8_step(self, *a):
        return self._rec("q8", a)

    def apexw_grad_clip_coef(self, *a):
        self.calls.append(("clip", a, None))
        return 0

    def apexw_factored_step(self, *a):
        hp = ctypes.cast(a[-2], ctypes.POINTER(L.HParams)).contents
        self.calls.append(("factored", a, {f: getattr(hp, f) for f, _ in L.HParams._fields_}))
        return 0


@pytest.fixture
def cpu_plans(monkeypatch):
    """Let plans run on CPU tensors: current_stream -> dummy, library step calls recorded."""
    rec = _Recorder(L.load())
    monkeypatch.setattr(_plan.StepPlan, "_lib", property(lambda self: rec, lambda self, v: None), raising=False)

    class _S:
        cuda_stream = 0
    monkeypatch.setattr(torch.cuda, "current_stream", lambda dev=None: _S())
    return rec


def _opt(params, **kw):
    from apexw_amd.optimizer import ApexW
    opt = ApexW(params, **kw)
    opt._build_plan_orig = opt._build_plan
    return opt


def _build(opt):
    group = opt.param_groups[0]
    from apexw_amd import state as S
    group["precision"] = S.normalize_precision(group["precision"])
    params = [p for p in group["params"] if p.grad is not None]
    peft = S.detect_peft_context(opt.param_groups)
    for p in params:
        if len(opt.state[p]) == 0:
            opt.state[p].update(S.init_state(p, group, peft))
    kind = "q8" if group["precision"] == "8bit" else "compact"
    return _plan.StepPlan(opt, group, params, kind), group


def _params(shapes, dtype):
    ps = []
    for s in shapes:
        p = torch.nn.Parameter(torch.zeros(s, dtype=dtype))
        p.grad = torch.zeros(s, dtype=dtype)
        ps.append(p)
    return ps


def test_q8_plan_partitions_fast_tensors_first(cpu_plans):
    shapes = [(4096,), (512, 1024), (100, 300), (50,), (64, 2048)]
    ps = _params(shapes, torch.bfloat16)
    opt = _opt(ps, precision="8bit", lr=1e-3, weight_decay=0.1, adamw_compat=True)
    plan, group = _build(opt)
    plan.execute(group, seed=7)
    name, args, hp = cpu_plans.calls[-1]
    assert name == "q8"
    # fast: (512,1024), (100,300) (short last block) and (64,2048) -- bf16, NF4, quad, block 2048
    fast_counts = [512 * 1024 // 2048, (30000 + 2047) // 2048, 64 * 2048 // 2048]
    assert args[4] == sum(fast_counts)
    assert plan.fast.tolist() == [False, True, True, False, True]
    units = plan.d_units.cpu().numpy().view(L.UNIT_DTYPE)
    assert units["tensor"][: sum(fast_counts)].max() == 2  # first three table rows are the fast tensors
    assert hp["mode"] == L.MODE_COLD and hp["step"] == 1
    assert hp["flags"] & L.HP_SR
    table = plan.d_table.cpu().numpy().view(L.TENSOR_DTYPE)
    assert [int(n) for n in table["n"]] == [512 * 1024, 30000, 64 * 2048, 4096, 50]
    plan.execute(group, seed=7)
    assert cpu_plans.calls[-1][2]["mode"] == L.MODE_REPLAY and cpu_plans.calls[-1][2]["step"] == 2


def test_compact_plan_scalars_and_modes(cpu_plans):
    ps = _params([(128, 256), (300,)], torch.float32)
    opt = _opt(ps, lr=1e-3, weight_decay=0.1, adamw_compat=True, stochastic_rounding=False)
    plan, group = _build(opt)
    plan.execute(group, seed=1)
    name, args, hp = cpu_plans.calls[-1]
    assert name == "compact" and args[3] == 16 + 1
    b1, b2 = 0.9, 0.999
    bc1, bc2 = 1 - b1, 1 - b2
    assert hp["step_size"] == pytest.approx(1e-3 * bc2 ** 0.5 / bc1, rel=1e-6)
    assert hp["eps_scaled"] == pytest.approx(1e-8 * bc2 ** 0.5, rel=1e-6)
    assert hp["wd_factor"] == pytest.approx(1 - 1e-4, rel=1e-7)
    assert hp["flags"] & L.HP_SANITIZE and not hp["flags"] & L.HP_SR
    assert hp["mode"] == L.MODE_COLD
    table = plan.d_table.cpu().numpy().view(L.TENSOR_DTYPE)
    assert all(table["flags"] & L.FLAG_WD)  # adamw_compat decays every tensor
    plan.execute(group, seed=1)
    hp2 = cpu_plans.calls[-1][2]
    assert hp2["mode"] == L.MODE_REPLAY and not hp2["flags"] & L.HP_SANITIZE
    assert [float(s) for s in (opt.state[p]["step"] for p in ps)] == [2.0, 2.0]


def test_step_counters_share_one_buffer(cpu_plans):
    ps = _params([(10,), (20,), (30,)], torch.bfloat16)
    opt = _opt(ps)
    plan, group = _build(opt)
    for _ in range(3):
        plan.execute(group, seed=0)
    steps = [opt.state[p]["step"] for p in ps]
    assert all(float(s) == 3.0 for s in steps)
    assert all(s.untyped_storage().data_ptr() == plan.steps.untyped_storage().data_ptr() for s in steps)


def test_cold_step_splits_by_step_count(cpu_plans):
    ps = _params([(64,), (64,)], torch.bfloat16)
    opt = _opt(ps, precision="8bit")
    plan, group = _build(opt)
    plan.steps[1] = 5.0
    plan.execute(group, seed=0)
    q8 = [c for c in cpu_plans.calls if c[0] == "q8"]
    assert sorted(c[2]["step"] for c in q8[-2:]) == [1, 6]


def _table(plan):
    return plan.d_table.cpu().numpy().view(L.TENSOR_DTYPE)


def test_scan_is_native():
    from apexw_amd import _host  # noqa: F401 -- built by apexw_amd._build
    ps = _params([(8,), (8,)], torch.float32)
    pp, dt = np.zeros(2, np.uint64), np.zeros(2, np.int8)
    _host.snapshot(ps, pp.ctypes.data, dt.ctypes.data)
    assert pp.tolist() == [p.data_ptr() for p in ps]
    with pytest.raises(TypeError):
        _host.snapshot([1], pp.ctypes.data, dt.ctypes.data)


def test_new_grads_are_repointed(cpu_plans):
    ps = _params([(64, 64), (300,)], torch.bfloat16)
    opt = _opt(ps)
    plan, group = _build(opt)
    plan.execute(group, seed=0)
    assert [int(x) for x in _table(plan)["g"]] == [p.grad.data_ptr() for p in ps]
    for p in ps:                       # zero_grad(set_to_none=True) + a new backward
        p.grad = torch.ones_like(p)
    assert plan.valid_for(group)
    plan.execute(group, seed=0)
    assert [int(x) for x in _table(plan)["g"]] == [p.grad.data_ptr() for p in ps]
    # a grad whose storage is swapped in place keeps its Python object
    ps[1].grad.data = torch.full((300,), 2.0, dtype=torch.bfloat16)
    assert plan.valid_for(group)
    plan.execute(group, seed=0)
    assert int(_table(plan)["g"][1]) == ps[1].grad.data_ptr()


def test_noncontiguous_grad_is_copied(cpu_plans):
    ps = _params([(32, 64)], torch.bfloat16)
    opt = _opt(ps)
    plan, group = _build(opt)
    ps[0].grad = torch.ones(64, 32, dtype=torch.bfloat16).t()
    assert plan.valid_for(group)
    keep = plan._refresh_grads()
    assert keep[0].is_contiguous() and int(_table(plan)["g"][0]) == keep[0].data_ptr()
    ps[0].grad_dtype = None                       # torch then accepts a grad of another dtype
    ps[0].grad = torch.ones(64, 32, dtype=torch.float32).t()
    # a grad of another dtype than the table's: a new plan (the table's descriptors change)
    assert not plan.valid_for(group)
    with pytest.raises(RuntimeError):
        plan._refresh_grads()


def test_param_storage_or_dtype_change_invalidates(cpu_plans):
    ps = _params([(64, 64), (300,)], torch.float32)
    opt = _opt(ps)
    plan, group = _build(opt)
    plan.execute(group, seed=0)
    assert plan.valid_for(group)
    ps[0].data = ps[0].data.clone()               # same dtype, new address
    assert not plan.valid_for(group)
    plan, group = _build(opt)
    assert plan.valid_for(group)
    m = torch.nn.Module()
    m.w = ps[1]
    m.to(torch.bfloat16)                           # module cast: same objects, new storage and dtype
    assert ps[1].dtype == torch.bfloat16 and not plan.valid_for(group)


def test_missing_grad_or_inactive_grad_invalidates(cpu_plans):
    ps = _params([(16,), (16,), (16,)], torch.bfloat16)
    g2 = ps[2].grad
    ps[2].grad = None
    opt = _opt(ps)
    plan, group = _build(opt)
    assert plan.valid_for(group)
    ps[2].grad = g2                               # a parameter outside the plan gains a grad
    assert not plan.valid_for(group)
    ps[2].grad = None
    ps[0].grad = None                             # a plan parameter loses its grad
    assert not plan.valid_for(group)


@pytest.mark.parametrize("prec", ["8bit", "compact"])
def test_factored_rows_and_launch(cpu_plans, prec):
    """Factored tensors stay rows of the table (clip and centralization see them),
    flagged so the step kernels skip them; apexw_factored_step gets their table
    rows (ascending), shapes, workspace and units."""
    shapes = [(1024, 512), (300,), (256, 512)] if prec == "compact" else [(256, 512), (300,), (1024, 512)]
    ps = _params(shapes, torch.bfloat16)
    opt = _opt(ps, precision=prec, factored_v=True, six_bit=True, lr=1e-3, weight_decay=0.1)
    plan, group = _build(opt)
    plan.execute(group, seed=0)
    plan.execute(group, seed=0)
    table = _table(plan)
    fac = (table["flags"] & L.FLAG_FACTORED) != 0
    big = [int(n) for n in table["n"][fac]]
    if prec == "compact":
        assert big == [1024 * 512]                  # 256 x 512 is under the compact threshold
    else:
        assert sorted(big) == [256 * 512, 1024 * 512]
        m6 = (table["flags"] & L.FLAG_M6) != 0
        assert [int(n) for n in table["n"][m6]] == [1024 * 512]
    calls = [c for c in cpu_plans.calls if c[0] == "factored"]
    assert len(calls) == 2
    _, args, hp = calls[-1]
    fv = plan.fv["d_fv"].cpu().numpy().view(L.FV_TENSOR_DTYPE)
    assert list(fv["tensor"]) == sorted(fv["tensor"]) and args[3] == len(fv)
    ends = plan.fv["range_ends"]
    assert args[8] == ends.ctypes.data and len(ends) == L.FV_UNIT_RANGES and ends[-1] == plan.fv["n_units"]
    for row in fv:
        d = int(row["tensor"])
        assert fac[d] and int(row["rows"]) * int(row["cols"]) == int(table["n"][d])
        assert int(row["flags"]) == (L.FV_SUM_COLS if int(table["n"][d]) > 262144 else 0)
    units = plan.fv["d_units"].cpu().numpy().view(L.UNIT_DTYPE)
    assert set(units["tensor"].tolist()) == set(range(len(fv)))    # units name their fv entry
    for k in range(len(fv)):
        assert (units["tensor"] == k).sum() == plan.unit_counts[int(fv[k]["tensor"])]
    # groups (bf16 params): INT8 m, then 6-bit m, then bf16 m; no fp32 groups
    begins = np.concatenate([[0], ends[:-1]])
    for r, (b, e) in enumerate(zip(begins, ends)):
        for k in set(units["tensor"][b:e].tolist()):
            row = table[int(fv[k]["tensor"])]
            want = 2 if int(row["block"]) == 0 else (1 if int(row["flags"]) & L.FLAG_M6 else 0)
            assert r == want
    assert ends[2] == plan.fv["n_units"]
    if prec == "compact":
        assert ends[1] == 0
    else:
        assert 0 < ends[0] < ends[1] == ends[2]
    # the step kernels get only the other rows' units (the factored rows' are apexw_factored_step's)
    steps = [c for c in cpu_plans.calls if c[0] in ("compact", "q8")]
    assert len(steps) == 2
    n_fac = sum(int(plan.unit_counts[int(r["tensor"])]) for r in fv)
    assert steps[-1][1][3] == plan.n_units - n_fac == plan.n_step_units
    step_units = plan.d_step_units.cpu().numpy().view(L.UNIT_DTYPE)[:plan.n_step_units]
    assert not fac[step_units["tensor"]].any()
    assert hp["step"] == 2 and hp["flags"] & L.HP_FV_SANITIZE == (L.HP_FV_SANITIZE if prec == "8bit" else 0)
    assert hp["eps"] == pytest.approx(1e-8) and hp["mode"] == L.MODE_COLD
