"""The CPU oracle reproduces the reference's own outputs bit-for-bit (SR off).

Golden vectors come from tests/golden/make_golden.py, which stepped the reference
implementation on the same seeded inputs.

One deliberate difference: the oracle's fp32 grad norms (global-norm clip) are
accumulated in float64, where the reference's CPU ``torch._foreach_norm`` sums in
fp32 and drifts from the exact norm (9.5e-6 relative on a 2^20-element grad of
the fixture).  The fp32 clip fixtures are therefore replayed twice: with the
reference's own norm reduction swapped in, bit for bit (everything downstream of
the norms is pinned), and with the oracle's, within that drift.
"""

import numpy as np
import pytest
import torch

from golden_replay import (CASES, FUSED_CASES, HOOK_CASES, SD_CASES, fused_inputs, hook_inputs, load, replay,
                           sd_inputs, state_keys, to_torch)
from oracle.clip import clip_grads_
from oracle.optim import OracleApexW


def _state_arrays(opt, p):
    st = opt.state[p]
    out = {"m": st["exp_avg"], "v": st["exp_avg_sq"]}
    if "exp_avg_scales" in st:
        out["ms"] = st["exp_avg_scales"]
        out["vs"] = st["exp_avg_sq_scales"]
    return out


def _as_np(t):
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


# trajectories whose grads go through the clip in fp32
FP32_CLIP_CASES = {"compact_fp32_clip_rne"}


def _torch_norms(grads):
    """The reference's own per-tensor norms (torch's CPU reduction in the grad dtype)."""
    return list(torch._foreach_norm(grads, 2.0))


@pytest.mark.parametrize("name", sorted(CASES))
def test_oracle_matches_reference_trajectory(name, monkeypatch):
    if name in FP32_CLIP_CASES:
        import oracle.clip
        monkeypatch.setattr(oracle.clip, "_norms", _torch_norms)
    params, opt, gold = replay(name, OracleApexW)
    for i, p in enumerate(params):
        np.testing.assert_array_equal(_as_np(p.data).reshape(-1), gold[f"p_{i}"].reshape(-1), err_msg=f"p_{i}")
        if f"flags_{i}" not in gold:
            # every state tensor was recorded (factored layouts)
            keys = state_keys(gold, i)
            assert keys == sorted(k for k, v in opt.state[p].items() if torch.is_tensor(v) and k != "step")
            for k in keys:
                np.testing.assert_array_equal(_as_np(opt.state[p][k]).reshape(-1), gold[f"st_{i}_{k}"].reshape(-1),
                                              err_msg=f"{k}_{i}")
            assert float(opt.state[p]["step"]) == float(gold[f"step_{i}"][0])
            if f"scale_{i}" in gold:
                st = opt.state[p]
                assert [float(st["scale_v"]), float(st["sqrt_scale_v"])] == gold[f"scale_{i}"].tolist()
            continue
        st = _state_arrays(opt, p)
        for key in ("m", "v", "ms", "vs"):
            if key in st:
                np.testing.assert_array_equal(_as_np(st[key]).reshape(-1), gold[f"{key}_{i}"].reshape(-1),
                                              err_msg=f"{key}_{i}")
        fl = gold[f"flags_{i}"]
        s = opt.state[p]
        assert int(bool(s.get("is_quad_v", False))) == fl[0]
        assert int(bool(s.get("is_4bit_m", False))) == fl[1]
        assert int(bool(s.get("is_8bit", False))) == fl[2]
        assert int(s.get("block_size_8bit", 0) or 0) == fl[3]


VARIANT_OPTIONS = ("amsgrad", "lion", "maximize", "nesterov", "cautious")


@pytest.mark.parametrize("name", sorted(n for n in CASES if any(o in n for o in VARIANT_OPTIONS)))
def test_variant_goldens_pin_the_variant(name):
    """Each amsgrad / maximize / nesterov / cautious trajectory tells the variant from
    the plain step: the same run with the option off ends on other parameters (so the
    golden pins the running max, the negated grads, the Nesterov numerator or the
    mask, not only the rest of the step)."""
    option = next(o for o in VARIANT_OPTIONS if o in name)

    def plain(params, **kw):
        return OracleApexW(params, **dict(kw, **{option: False}))
    params, _, gold = replay(name, plain)
    assert any(not np.array_equal(_as_np(p.data).reshape(-1), gold[f"p_{i}"].reshape(-1))
               for i, p in enumerate(params))


AMSGRAD_CASES = sorted(n for n in CASES if "amsgrad" in n)
# homogeneous groups: torch._fused_adamw_ takes the max itself
AMSGRAD_NATIVE = {"compact_bf16_amsgrad_rne", "full_fp32_amsgrad_rne", "fp16_amsgrad_native_rne"}


@pytest.mark.parametrize("name", AMSGRAD_CASES)
def test_amsgrad_goldens_hold_an_active_max(name):
    """The reference's running max ends above v somewhere in every amsgrad trajectory,
    so the max (not v) fed some denominator of the recorded steps."""
    gold = load(name)
    n = len(CASES[name][0])
    assert any((gold[f"st_{i}_max_exp_avg_sq"] != gold[f"st_{i}_exp_avg_sq"]).any() for i in range(n))


@pytest.mark.parametrize("name", AMSGRAD_CASES)
def test_amsgrad_goldens_pin_the_max_in_the_denominator(name, monkeypatch):
    """The foreach-order trajectories tell a step that keeps the max but divides by v
    from the reference's (the native ones take torch._fused_adamw_'s own max)."""
    import oracle.compact as C

    def v_denominator(max_vs, vs):
        if max_vs is not None:
            torch._foreach_maximum_(max_vs, vs)
        return vs
    monkeypatch.setattr(C, "_amsgrad_max", v_denominator)
    params, opt, gold = replay(name, OracleApexW)
    assert (opt._plan["kind"] == "native") == (name in AMSGRAD_NATIVE)
    if name in AMSGRAD_NATIVE:
        return
    assert any(not np.array_equal(_as_np(p.data).reshape(-1), gold[f"p_{i}"].reshape(-1))
               for i, p in enumerate(params))


@pytest.mark.parametrize("name", ["compact_bf16_lion_rne", "fp16_lion_rne"])
def test_lion_goldens_pin_the_rounded_scalar(name, monkeypatch):
    """The 16-bit lion trajectories tell torch's same-dtype add (the scalar -lr rounded to
    the tensors' dtype) from an fp32 scalar: an oracle with the latter ends elsewhere."""
    import oracle.compact as C

    def fp32_alpha(params, grads, ms, *, lr, beta1, beta2):
        target = ms[0].dtype
        gc = [g.to(target) for g in grads] if grads[0].dtype != target else list(grads)
        for p, g, m in zip(params, gc, ms):
            u = torch.lerp(g, m, beta1).sign()
            p.copy_((p.float() - lr * u.float()).to(p.dtype))
        torch._foreach_lerp_(ms, gc, 1.0 - beta2)
    monkeypatch.setattr(C, "lion_update", fp32_alpha)
    params, _, gold = replay(name, OracleApexW)
    assert any(not np.array_equal(_as_np(p.data).reshape(-1), gold[f"p_{i}"].reshape(-1))
               for i, p in enumerate(params))


def _no_upcast(ms, slows, ratio, upcast):
    return torch._foreach_add(ms, slows, alpha=ratio)


def _fp32_ratio(ms, slows, ratio, upcast):
    return [(m.float() + ratio * s.float()).to(torch.float32 if upcast else m.dtype) for m, s in zip(ms, slows)]


@pytest.mark.parametrize("name,mistake", [("compact_fp32_beta3_rne", _no_upcast),
                                          ("compact_bf16_beta3_rne", _fp32_ratio),
                                          ("fp16_beta3_rne", _fp32_ratio)])
def test_beta3_goldens_pin_the_numerator(name, mistake, monkeypatch):
    """The beta3 trajectories tell the reference's numerator m + slow_ratio m_slow from
    a plausible other: the cold order's fp32 upcast for fp32 parameters over bf16 m
    skipped, or the ratio kept in fp32 where torch's same-dtype add rounds it to the
    16-bit dtype; an oracle with either ends elsewhere."""
    import oracle.compact as C
    monkeypatch.setattr(C, "_slow_numerators", mistake)
    params, _, gold = replay(name, OracleApexW)
    assert any(not np.array_equal(_as_np(p.data).reshape(-1), gold[f"p_{i}"].reshape(-1))
               for i, p in enumerate(params))


GD_NAMES = sorted(n for n in CASES if n.startswith("gd_"))


@pytest.mark.parametrize("name", GD_NAMES)
def test_grad_dtype_goldens_pin_the_grad_dtype(name):
    """The trajectories with grads of another dtype tell the reference's handling from
    an optimizer handed the same grads in the parameter dtype (fp32 grads of 16-bit
    parameters rounded, bf16 grads of fp32 parameters widened): such an oracle ends
    elsewhere, so the goldens pin the grads' own precision and their dtype-dependent
    rounding order."""
    class InParamDtype(OracleApexW):
        def step(self):
            for p in self.params:
                if p.grad is not None:
                    g = p.grad
                    p.grad = None
                    p.grad_dtype = None
                    p.grad = g.to(p.dtype)
            super().step()
    params, _, gold = replay(name, InParamDtype)
    assert any(not np.array_equal(_as_np(p.data).reshape(-1), gold[f"p_{i}"].reshape(-1))
               for i, p in enumerate(params))


def test_oracle_clip_matches_reference():
    z = load("clip_bf16")
    n = len([k for k in z if k.startswith("g_")])
    grads = [to_torch(z[f"g_{i}"], torch.bfloat16) for i in range(n)]
    clip_grads_(grads, 1.0)
    for i, g in enumerate(grads):
        np.testing.assert_array_equal(_as_np(g), z[f"gc_{i}"])


def _clip_fp32_inputs():
    from golden.make_golden import CLIP_FP32_SHAPES, CLIP_SCALES, CLIP_SHAPES, _fingerprint, _grad
    z = load("clip_fp32")
    gen = torch.Generator().manual_seed(7)
    for s, sc in zip(CLIP_SHAPES, CLIP_SCALES):   # the bf16 fixture's draws come first
        _grad(s, torch.bfloat16, gen, sc)
    grads = [_grad(s, torch.float32, gen, sc) for s, sc in zip(CLIP_FP32_SHAPES, CLIP_SCALES)]
    np.testing.assert_array_equal(np.array([_fingerprint(g) for g in grads]), z["fingerprint"])
    return grads, z


def test_oracle_fp32_clip_matches_reference(monkeypatch):
    """fp32 grads up to 2^20 elements: with the reference's norm reduction the
    clipped grads are bit-equal; with the oracle's float64 norms the coefficient
    (the ratio of clipped to raw grads) is within 1e-5 relative of the reference's,
    the drift of its fp32 reduction (leaving out one of the large tensors' terms,
    or a wrong power, moves it by 1e-3 or more)."""
    import oracle.clip
    from golden.make_golden import CLIP_FP32_KEEP
    grads, z = _clip_fp32_inputs()
    raw = [g.clone() for g in grads]
    coef = float(clip_grads_(grads, 1.0))
    assert coef < 1.0
    for i, (g, r) in enumerate(zip(grads, raw)):
        ref = z[f"gc_{i}"].astype(np.float64)
        ratio = ref / r.reshape(-1)[:CLIP_FP32_KEEP].numpy().astype(np.float64)
        np.testing.assert_allclose(ratio, coef, rtol=1e-5, err_msg=f"coefficient of gc_{i}")
        np.testing.assert_allclose(g.reshape(-1)[:CLIP_FP32_KEEP].numpy(), z[f"gc_{i}"], rtol=1e-5, atol=0)
    monkeypatch.setattr(oracle.clip, "_norms", _torch_norms)
    grads = [r.clone() for r in raw]
    clip_grads_(grads, 1.0)
    for i, g in enumerate(grads):
        np.testing.assert_array_equal(g.reshape(-1)[:CLIP_FP32_KEEP].numpy(), z[f"gc_{i}"])


@pytest.mark.parametrize("name", sorted(FP32_CLIP_CASES))
def test_oracle_fp32_clip_trajectory_with_exact_norms(name):
    """The product oracle (float64 norms) on the fp32 clip trajectory: the
    reference's norm drift moves the coefficient by ~1e-6 relative, which reaches
    fp32 p as at most 1e-5 relative; the bf16 states absorb it."""
    params, opt, gold = replay(name, OracleApexW)
    for i, p in enumerate(params):
        np.testing.assert_allclose(_as_np(p.data).reshape(-1), gold[f"p_{i}"].reshape(-1), rtol=1e-5, atol=1e-9,
                                   err_msg=f"p_{i}")
        for k, arr in _state_arrays(opt, p).items():
            got = arr.detach()
            ref = gold[f"{k}_{i}"].reshape(-1)
            if got.dtype == torch.bfloat16:
                d = np.abs(_as_np(got).reshape(-1).astype(np.int64) - ref.astype(np.int64))
                assert int(d.max()) <= 1, f"{k}_{i}: {int(d.max())} bf16 ulps"
            else:
                np.testing.assert_allclose(_as_np(got).reshape(-1), ref, rtol=1e-5, atol=1e-12, err_msg=f"{k}_{i}")


@pytest.mark.parametrize("name", sorted(HOOK_CASES))
def test_oracle_hooks_match_reference_trajectory(name):
    """The in-backward path over several steps: the hooked tensors are stepped once per
    backward pass by oracle.hooks.flush_8bit (K = 1 until the first step() has seen
    the anchor's pass count), the anchor and the small tensors accumulate their
    grads and take the ordinary 8-bit step in step()."""
    from oracle import hooks as H
    host, grads, gold = hook_inputs(name)
    params = [torch.nn.Parameter(h.to(H.downcast_dtype(h))) for h in host]
    on, anchor, hooked = H.hook_partition(params)
    assert on and anchor is params[0]
    hooked_ids = {id(p) for p in hooked}
    rest = [p for p in params if id(p) not in hooked_ids]
    kw = dict(lr=1e-3, weight_decay=0.1, adamw_compat=True, precision="8bit", stochastic_rounding=False)
    rest_opt = OracleApexW(rest, **kw)
    group = dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.1, decay_norm_only=False,
                 precision="8bit", stochastic_rounding=False, block_size=None, int4_m=None)
    states = {}
    K = 1
    for per_step in grads:
        acc = {}
        for gs in per_step:
            H.flush_8bit(hooked, [gs[i] for i, p in enumerate(params) if id(p) in hooked_ids], states, group, K=K)
            for i, p in enumerate(params):
                if id(p) not in hooked_ids:
                    acc[i] = gs[i].clone() if i not in acc else acc[i] + gs[i]
        for i, p in enumerate(params):
            if id(p) not in hooked_ids:
                p.grad = acc[i]
        rest_opt.step()
        for p in rest:
            p.grad = None
        K = len(per_step)
    np.testing.assert_array_equal(np.array([{torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}[p.dtype] for p in params]),
                                  gold["dtypes"])
    for i, p in enumerate(params):
        np.testing.assert_array_equal(_as_np(p.data).reshape(-1), gold[f"p_{i}"].reshape(-1), err_msg=f"p_{i}")
        st = states[p] if id(p) in hooked_ids else rest_opt.state[p]
        for k in ("exp_avg", "exp_avg_scales", "exp_avg_sq", "exp_avg_sq_scales"):
            np.testing.assert_array_equal(_as_np(st[k]).reshape(-1), gold[f"st_{i}_{k}"].reshape(-1),
                                          err_msg=f"{k}_{i}")
        assert float(st["step"]) == float(gold[f"step_{i}"][0]), f"step_{i}"


def fused_group(kwargs):
    """The group dict oracle.hooks.fused_param_step reads, from ApexW's constructor
    defaults (8-bit betas (0.9, 0.999), compact (0.9, 0.99), eps 1e-8,
    decay_norm_only on)."""
    prec = kwargs.get("precision", "compact")
    return dict(lr=kwargs["lr"], betas=(0.9, 0.999) if prec == "8bit" else (0.9, 0.99), eps=1e-8,
                weight_decay=kwargs["weight_decay"], decay_norm_only=True, precision=prec,
                stochastic_rounding=kwargs["stochastic_rounding"], block_size=None, int4_m=None)


@pytest.mark.parametrize("name", sorted(FUSED_CASES))
def test_oracle_fused_backward_matches_reference_trajectory(name):
    """enable_fused_backward over 6 steps (bias corrections of steps 1..6, the
    momentum's INT8 scale without the EMA floor from step 2 on), one or two
    backward passes per step: each parameter's grads summed in its own dtype, as
    autograd accumulates them, then oracle.hooks.fused_param_step.  Bit-exact."""
    from oracle import hooks as H
    dtype, kwargs, host, grads, gold = fused_inputs(name)
    group = fused_group(kwargs)
    params = [torch.nn.Parameter(h.clone()) for h in host]
    states = {}
    for per_step in grads:
        for i, p in enumerate(params):
            acc = per_step[0][i].clone()
            for gs in per_step[1:]:
                acc += gs[i]
            H.fused_param_step(p, acc, states.setdefault(p, {}), group)
    for i, p in enumerate(params):
        np.testing.assert_array_equal(_as_np(p.data).reshape(-1), gold[f"p_{i}"].reshape(-1), err_msg=f"p_{i}")
        st = states[p]
        for k in state_keys(gold, i):
            np.testing.assert_array_equal(_as_np(st[k]).reshape(-1), gold[f"st_{i}_{k}"].reshape(-1),
                                          err_msg=f"{k}_{i}")
        assert float(st["step"]) == float(gold[f"step_{i}"][0]) == 6.0


@pytest.mark.parametrize("name", ["sd_compact", "sd_q8"])
def test_oracle_resumes_reference_checkpoint(name):
    """The reference's resume from its own checkpoint: a fresh optimizer loads the
    state_dict written after 3 steps and takes 2 more -- a cold step from non-zero
    state, then a replayed one.  The oracle, given the same state, lands on the
    same bits."""
    shapes, dtype, kwargs, sd, mid, grads, gold = sd_inputs(name)
    params = [torch.nn.Parameter(m.clone()) for m in mid]
    opt = OracleApexW(params, **kwargs)
    for pid, p in zip(sd["param_groups"][0]["params"], params):
        opt.state[p] = {k: (v.clone() if torch.is_tensor(v) else v) for k, v in sd["state"][pid].items()}
    for gs in grads:
        for p, g in zip(params, gs):
            p.grad = g.clone()
        opt.step()
    for i, p in enumerate(params):
        np.testing.assert_array_equal(_as_np(p.data).reshape(-1), gold[f"p_{i}"].reshape(-1), err_msg=f"p_{i}")
        for k in state_keys(gold, i):
            np.testing.assert_array_equal(_as_np(opt.state[p][k]).reshape(-1), gold[f"st_{i}_{k}"].reshape(-1),
                                          err_msg=f"{k}_{i}")
