"""Pins the oracle of the in-backward 8-bit steps (oracle/hooks.py) on the CPU."""

import pytest
import torch

from oracle import hooks as H
from oracle import layout as L
from oracle.optim import OracleApexW


def _group(**kw):
    g = dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.1, decay_norm_only=True,
             precision="8bit", stochastic_rounding=False, block_size=None, int4_m=None)
    g.update(kw)
    return g


def _params(shapes, dtype, seed):
    gen = torch.Generator().manual_seed(seed)
    ps = [torch.nn.Parameter((torch.randn(s, generator=gen) * 0.02).to(dtype)) for s in shapes]
    gs = [(torch.randn(s, generator=gen) * 1e-3).to(dtype) for s in shapes]
    return ps, gs


SHAPES = [(512, 1024), (64, 512), (300, 1000), (16384,), (128, 130), (2048,)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_k1_flush_equals_the_ordinary_step(dtype):
    """K = 1, no AMP: lr, weight decay, grad scale and bias correction reduce to the
    ordinary step's, so three flushes equal three OracleApexW steps bit for bit."""
    group = _group()
    a, grads = _params(SHAPES, dtype, 0)
    b = [torch.nn.Parameter(p.detach().clone()) for p in a]
    states = {}
    ref = OracleApexW(b, lr=1e-3, weight_decay=0.1, precision="8bit", stochastic_rounding=False)
    for it in range(3):
        gs = [g * (1 + it) for g in grads]
        H.flush_8bit(a, gs, states, group)
        for p, g in zip(b, gs):
            p.grad = g.clone()
        ref.step()
    for i, (x, y) in enumerate(zip(a, b)):
        assert torch.equal(x, y), f"param {i}"
        sa, sb = states[x], ref.state[y]
        for k in ("exp_avg", "exp_avg_scales", "exp_avg_sq", "exp_avg_sq_scales"):
            assert torch.equal(sa[k], sb[k]), f"param {i} {k}"
        assert float(sa["step"]) == float(sb["step"]) == 3.0 and sa["_hook_mstep"] == 3


@pytest.mark.parametrize("K", [2, 3])
def test_first_pass_matches_closed_form(K):
    """A first pass from zero state with K accumulation passes: grads scaled by K,
    lr * K^-0.4, decay lr * wd / K.  eps = 1 makes the update proportional to the
    scaled grad (the denominator clamps at eps), so each factor shows."""
    group = _group(eps=1.0, lr=1e-2)
    ps, gs = _params([(40, 50)], torch.float32, 3)
    p0 = ps[0].detach().clone()
    states = {}
    H.flush_8bit(ps, gs, states, group, K=K)
    want = H.first_step_closed_form(p0, gs[0], lr=1e-2, beta1=0.9, beta2=0.999, eps=1.0,
                                    weight_decay=0.1, K=K)
    got = ps[0].detach().double()
    upd = (want - p0.double()).abs()
    assert upd.max() > 1e-5
    tol = 4 * 2.0 ** -24 * p0.double().abs() + 1e-5 * upd + 1e-12
    assert ((got - want).abs() <= tol).all()
    # a wrong scale (1/K instead of K) would move the update by K^2
    assert ((got - p0.double()).abs() - upd).abs().max() < 0.01 * upd.max()


def test_step_counter_advances_once_per_k_passes():
    group = _group()
    ps, gs = _params([(64, 512)], torch.bfloat16, 4)
    states = {}
    for _ in range(6):
        H.flush_8bit(ps, gs, states, group, K=3)
    st = states[ps[0]]
    assert st["_hook_mstep"] == 6 and float(st["step"]) == 2.0


def test_power_of_two_amp_scale_cancels():
    group = _group()
    a, grads = _params(SHAPES[:4], torch.bfloat16, 5)
    b = [torch.nn.Parameter(p.detach().clone()) for p in a]
    sa, sb = {}, {}
    for it in range(2):
        H.flush_8bit(a, [g * 65536.0 for g in grads], sa, group, amp_scale=65536.0)
        H.flush_8bit(b, grads, sb, group)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_partition_and_downcast_rules():
    """The reference's own case (test_quantization.py:1093-1129): 16 fp32 tensors of
    64 x 512 -> all bf16, 15 hooked, the first is the anchor."""
    ps = [torch.nn.Parameter(torch.zeros(64, 512)) for _ in range(16)]
    on, anchor, hooked = H.hook_partition(ps)
    assert on and anchor is ps[0] and hooked == ps[1:]
    assert all(H.downcast_dtype(p) == torch.bfloat16 for p in ps)
    assert H.downcast_dtype(torch.zeros(1023)) == torch.float32
    assert not H.hook_partition(ps[:7])[0]                     # fewer than 8 tensors
    assert not H.hook_partition([torch.nn.Parameter(torch.zeros(1000)) for _ in range(20)])[0]   # < 524,288
    small = [torch.nn.Parameter(torch.zeros(100000)) for _ in range(8)] + [torch.nn.Parameter(torch.zeros(16383))]
    assert H.hook_partition(small)[2] == small[1:8]


@pytest.mark.parametrize("shape", [(16384,), (64, 512), (300, 1000), (4096, 7), (128, 130), (16388,), (20000,)])
def test_lazy_state_matches_init_group_where_rules_coincide(shape):
    """ensure_8bit_state equals the golden-pinned init_state for tensors of >= 16384
    elements unless int4_m is forced on (then _init_group can take NF4 m without quad v)."""
    group = _group()
    p = torch.zeros(shape, dtype=torch.bfloat16)
    a = H.ensure_8bit_state({}, p, group)
    b = L.init_state(p, group, 16, False)
    assert a.keys() == b.keys()
    for k in a:
        if torch.is_tensor(a[k]):
            assert torch.equal(a[k], b[k]) and a[k].dtype == b[k].dtype, k
        else:
            assert a[k] == b[k], k
    forced = H.ensure_8bit_state({}, torch.zeros(16386), _group(int4_m=True))
    assert not forced["is_4bit_m"] and not forced["is_quad_v"]
    assert L.init_state(torch.zeros(16386), _group(int4_m=True), 16, False)["is_4bit_m"]


@pytest.mark.parametrize("prec", ["8bit", "compact"])
def test_fused_first_step_matches_closed_form(prec):
    """enable_fused_backward's update from zero state.  eps = 1 with
    eps_scaled = sqrt(1 - b2) < 1: the 8-bit denominator has no eps floor here
    (the ordinary 8-bit step would clamp it to 1)."""
    group = _group(eps=1.0, lr=1e-2, precision=prec, stochastic_rounding=False)
    ps, gs = _params([(40, 50)], torch.float32, 7)
    gs = [g * 50.0 for g in gs]
    p0 = ps[0].detach().clone()
    st = {}
    H.fused_param_step(ps[0], gs[0], st, group)
    q8, compact = H.fused_first_step_closed_form(p0, gs[0], lr=1e-2, beta1=0.9, beta2=0.999, eps=1.0,
                                                 weight_decay=0.1)
    want = q8 if prec == "8bit" else compact
    got = ps[0].detach().double()
    upd = (want - p0.double() * (1 - 1e-3)).abs()
    assert upd.max() > 1e-4
    tol = 4 * 2.0 ** -24 * p0.double().abs() + 1e-5 * upd + 1e-12
    assert ((got - want).abs() <= tol).all()
    assert float(st["step"]) == 1.0
    if prec == "compact":
        assert set(st) == {"stochastic_rounding", "step", "exp_avg", "exp_avg_sq"}
        assert st["exp_avg"].dtype == st["exp_avg_sq"].dtype == torch.bfloat16
        assert torch.equal(st["exp_avg"], (0.1 * gs[0]).to(torch.bfloat16))


def test_fused_int8_momentum_scale_has_no_ema():
    """Second update with a grad that halves the momentum: the INT8 scale is the
    new absmax / 127, below the 0.9 x old floor the ordinary step keeps."""
    group = _group(precision="8bit", stochastic_rounding=False)
    ps, gs = _params([(32, 128)], torch.float32, 8)
    st = {}
    H.fused_param_step(ps[0], gs[0], st, group)
    bs = st["block_size_8bit"]
    s1 = st["exp_avg_scales"].clone().double()
    m1 = (st["exp_avg"].double().reshape(-1, bs) * s1).reshape(32, 128)
    g2 = (-4.5 * m1).float()                   # m2 = 0.9 m1 + 0.1 g2 = 0.45 m1
    H.fused_param_step(ps[0], g2, st, group)
    m2 = 0.9 * m1 + 0.1 * g2.double()
    want = m2.reshape(-1, bs).abs().amax(dim=1, keepdim=True) / 127.0
    got = st["exp_avg_scales"].double()
    assert torch.allclose(got, want, rtol=1e-6, atol=0)
    assert (got < 0.9 * s1).all()
