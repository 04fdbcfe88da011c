"""Host logic of the automatic 8-bit runtime acceleration, on the CPU.

Construction-time downcast and hook registration, the queue of 14, the anchor
flush, the learned accumulation count, AMP detection and the restore rules run
as in the reference (apexw/optimizer.py:1346-1507, :2059-2371).  The kernel
launch of a flushed batch is replaced by a recorder, so no device is needed.
"""

import pytest
import torch
import torch.nn as nn

from apexw_amd import runtime as R
from apexw_amd.optimizer import ApexW


class _Rec:
    def __init__(self):
        self.calls = []

    def make(self, opt):
        rec = self

        class _Plan:
            def __init__(self, group, params):
                self.group, self.params = group, params

            def prepare(self, group, seed, inv, lr=None, wd=None, steps=None):
                call = dict(params=list(self.params), inv=inv, lr=lr, wd=wd, steps=list(steps))

                class _Prog:
                    def run(self):
                        rec.calls.append(call)

                    def rollback(self):
                        pass
                return _Prog()
        return lambda group, params: _Plan(group, params)


@pytest.fixture
def rec(monkeypatch):
    r = _Rec()
    orig_init = ApexW.__init__

    def init(self, *a, **k):
        orig_init(self, *a, **k)
        self._hook_plan = r.make(self)
    monkeypatch.setattr(ApexW, "__init__", init)
    yield r
    R.restore_all_downcast_params()


def _chain(n=16, shape=(64, 512), seed=123):
    torch.manual_seed(seed)
    return [nn.Parameter(torch.randn(*shape) * 0.05) for _ in range(n)]


def _loss(params, x):
    y = x
    for p in params:
        y = (y @ p.t()) @ p
    return (y.float() ** 2).mean()


def test_downcast_and_hooks_registered(rec):
    ps = _chain()
    opt = ApexW(ps, lr=2e-4, precision="8bit")
    assert all(p.dtype == torch.bfloat16 for p in ps)
    assert len(opt._auto_hook_handles) == 16            # 15 layers + the anchor
    assert all(R._is_downcast(p) for p in ps)


@pytest.mark.parametrize("kw", [dict(clip_grad_norm=1.0), dict(grad_centralization=True), dict(precision="compact")])
def test_not_enabled(rec, kw):
    ps = _chain()
    opt = ApexW(ps, lr=2e-4, **{"precision": "8bit", **kw})
    assert all(p.dtype == torch.float32 for p in ps) and not opt._auto_hook_handles


def test_small_models_not_enabled(rec):
    ps = _chain(n=7)
    opt = ApexW(ps, precision="8bit")
    assert all(p.dtype == torch.float32 for p in ps) and not opt._auto_hook_handles


def test_backward_steps_layers_in_batches_of_14(rec):
    """The reference's own case (test_quantization.py:1093-1129)."""
    ps = _chain()
    opt = ApexW(ps, lr=2e-4, precision="8bit")
    x = torch.randn(16, 512, dtype=torch.bfloat16)
    _loss(ps, x).backward()
    assert ps[0].grad is not None                        # the anchor keeps its grad
    assert all(p.grad is None for p in ps[1:])
    assert [len(c["params"]) for c in rec.calls] == [14, 1]
    stepped = [p for c in rec.calls for p in c["params"]]
    assert sorted(map(id, stepped)) == sorted(map(id, ps[1:]))
    assert all(c["lr"] == 2e-4 and c["wd"] == 1e-2 and c["inv"] is None and c["steps"] == [1] * len(c["params"])
               for c in rec.calls)
    assert all(int(opt.state[p]["step"]) == 1 for p in ps[1:])
    assert opt._anchor_backward_count == 1


def test_zero_grad_drops_the_queue(rec):
    ps = _chain()
    opt = ApexW(ps, precision="8bit")
    opt._auto_hook_queue.append((ps[3], opt.param_groups[0]))
    opt.zero_grad()
    assert not opt._auto_hook_queue


def test_accumulation_count_is_learned(rec):
    """Two backward passes before the first step(): the hooks step every pass
    with K = 1, step() learns K = 2; later passes use lr K^-0.4, wd / (K K^-0.4),
    grads scaled by K, and store the step counter (passes - 1) // K + 1."""
    ps = _chain()
    opt = ApexW(ps, lr=2e-4, precision="8bit")
    opt.step = lambda closure=None: _host_step(opt)
    x = torch.randn(16, 512, dtype=torch.bfloat16)
    for _ in range(2):
        _loss(ps, x).backward()
    _host_step(opt)
    assert opt._grad_accum_steps == 2 and opt._grad_accum_steps_known
    n0 = len(rec.calls)
    _loss(ps, x).backward()
    c = rec.calls[n0]
    K, mult = 2, 2 ** -0.4
    assert c["lr"] == pytest.approx(2e-4 * mult, rel=1e-15)
    assert c["wd"] == pytest.approx(1e-2 / (K * mult), rel=1e-15)
    assert c["inv"] == 2.0 and c["steps"] == [3] * len(c["params"])
    p = c["params"][0]
    assert opt.state[p]["_hook_mstep"] == 3 and int(opt.state[p]["step"]) == 2   # (3 - 1) // 2 + 1
    _loss(ps, x).backward()
    assert opt.state[p]["_hook_mstep"] == 4 and int(opt.state[p]["step"]) == 2
    _loss(ps, x).backward()
    assert opt.state[p]["_hook_mstep"] == 5 and int(opt.state[p]["step"]) == 3


def _host_step(opt):
    """The bookkeeping head of ApexW.step without the launch of the anchor's step."""
    opt._has_stepped = True
    if opt._auto_hook_queue:
        opt._flush_auto_8bit_hook_queue()
    if opt._auto_hook_stepped_count > 0:
        if not opt._grad_accum_steps_known and opt._anchor_backward_count > 1:
            opt._grad_accum_steps = opt._anchor_backward_count
            opt._grad_accum_steps_known = True
        opt._auto_hook_stepped_count = 0
        opt._anchor_backward_count = 0
    R.amp_scaled_this_backward = False
    for p in opt.param_groups[0]["params"]:
        p.grad = None


def test_amp_scale_is_read_from_grad_scaler(rec):
    ps = _chain()
    ApexW(ps, lr=2e-4, precision="8bit")
    scaler = torch.amp.GradScaler("cpu", init_scale=1024.0)
    x = torch.randn(16, 512, dtype=torch.bfloat16)
    scaler.scale(_loss(ps, x)).backward()
    assert R.last_amp_scale == 1024.0 and R.amp_scaled_this_backward
    assert all(c["inv"] == 1.0 / 1024.0 for c in rec.calls)
    scaler.update(new_scale=1024.0)
    assert R.last_amp_scale is None and not R.amp_scaled_this_backward


def test_restore_rules(rec):
    ps = _chain()
    opt = ApexW(ps, precision="8bit")
    ApexW(_chain(n=8, seed=1), precision="8bit")       # another 8-bit ApexW before any step: nothing restored
    assert all(p.dtype == torch.bfloat16 for p in ps) and opt._auto_hook_handles
    torch.optim.AdamW(ps, lr=1e-3)                      # any other optimizer restores and unhooks
    assert all(p.dtype == torch.float32 for p in ps) and not opt._auto_hook_handles
    assert not R.DOWNCAST

    m = nn.Sequential(*[nn.Linear(512, 256, bias=False) for _ in range(8)])
    sd = {k: v.clone() for k, v in m.state_dict().items()}
    ApexW(m.parameters(), precision="8bit")
    assert all(p.dtype == torch.bfloat16 for p in m.parameters())
    m.load_state_dict(sd)                              # loading weights restores fp32 first
    assert all(p.dtype == torch.float32 for p in m.parameters())


def test_fused_backward_hooks_count_passes(monkeypatch):
    """enable_fused_backward: one hook per trainable parameter, a step on every
    K-th grad, the grad freed; the automatic 8-bit hooks stand aside."""
    ps = _chain()
    opt = ApexW(ps, lr=2e-4, precision="8bit")
    calls = []

    def fake(p, group):
        calls.append(p)
    monkeypatch.setattr(opt, "_step_single_param_fused", fake)
    monkeypatch.setattr(opt, "_hook_plan", lambda group, params: pytest.fail("auto hooks must stand aside"))
    opt.enable_fused_backward(grad_accum_steps=2)
    assert len(opt._fused_backward_handles) == 16
    x = torch.randn(16, 512, dtype=torch.bfloat16)
    _loss(ps, x).backward()
    assert not calls and all(p.grad is not None for p in ps)
    _loss(ps, x).backward()
    assert sorted(map(id, calls)) == sorted(map(id, ps)) and all(p.grad is None for p in ps)
    opt.disable_fused_backward()
    assert not opt._fused_backward_handles and not opt._fused_backward_enabled
    R.restore_all_downcast_params()


@pytest.mark.parametrize("prec", ["8bit", "compact"])
def test_fused_backward_refuses_factored_state(prec):
    """A parameter that step() gave factored-v state cannot take the per-parameter
    in-backward update (the reference's has no factored branch): a clear error,
    raised before the state or the step counter changes."""
    p = nn.Parameter(torch.randn(256, 512))
    opt = ApexW([p], precision=prec, factored_v=True)
    st = opt.state[p]
    st.update(step=torch.tensor(3.0), is_factored_v=True, exp_avg=torch.zeros(256, 512, dtype=torch.bfloat16),
              exp_avg_sq_row=torch.zeros(256), exp_avg_sq_col=torch.zeros(512))
    p.grad = torch.zeros_like(p)
    with pytest.raises(RuntimeError, match="factored_v"):
        opt._step_single_param_fused(p, opt.param_groups[0])
    assert float(st["step"]) == 3.0
    R.restore_all_downcast_params()
