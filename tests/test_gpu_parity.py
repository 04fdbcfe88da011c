"""GPU parity: the HIP step against the reference's own trajectories and the CPU oracle.

Tolerances (round to nearest, SR off):
  * fp32 params:  |d| <= 1e-6*|ref| + 1e-9 (the absolute floor covers p ~ 0); under
    the global-norm clip 1e-5*|ref| + 2^-8*S*lr + 1e-9 after S steps: the reference's
    CPU fp32 norm reduction drifts from the exact norm (up to ~1e-5 relative), so the
    coefficient differs by that much, which can flip the last bit of a bf16 m or v
    (held to 1 ulp) and so move a step's update (|u| <= ~lr) by 2^-8 of itself
  * bf16 tensors (params, m, v): <= 1 bf16 ulp; fp16 tensors <= 1 fp16 ulp
  * fp32 v (compact):             |d| <= 1e-6*|ref| + 1e-12
  * 8-bit codes: NF4/INT8/log-u8 differ by <= 1 code; block scales within 1e-6 relative
Factored-v trajectories (S steps, no resynchronisation): the row / column EMAs
are sums reduced in another order than torch's CPU kernels, held to 1e-5
relative; m does not depend on them (INT8 and 6-bit codes <= 1, m block scales
1e-5 relative, bf16 m <= 2 ulps).  The denominator carries the EMAs' few-ulp
difference into the update, which is rounded to bf16 before the subtraction:
each step can move bf16 p by one ulp of the update (<= 2^-8 |u|, and
|u| <= |p_before| + |p_after|) plus one ulp of p, so bf16 p is held to 2 ulps
or, where the updates are large against p, 2^-7 S (|p_0| + 2 |p_S|); fp32 p to
1e-5 relative (+1e-9).
"""

import numpy as np
import pytest
import torch

from golden_replay import CASES, bf16_ulp_diff, initial_params, replay, state_keys, to_torch

pytestmark = pytest.mark.gpu

dev = "cuda"
FP32_CLIP_CASES = {"compact_fp32_clip_rne"}   # fp32 grads through the global-norm clip


def _require_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")


def _cmp_f32(got, ref, rel=1e-6, floor=1e-9, what=""):
    got, ref = got.double().cpu(), ref.double()
    err = (got - ref).abs() - (rel * ref.abs() + floor)
    assert float(err.max()) <= 0, f"{what}: max excess {float(err.max()):.3e}"


def _cmp_bf16(got, ref, ulps=1, what=""):
    d = bf16_ulp_diff(got.cpu().contiguous(), ref.contiguous())
    assert int(d.max()) <= ulps, f"{what}: {int(d.max())} bf16 ulps ({int((d > ulps).sum())} elements)"


def _cmp_f16(got, ref, ulps=1, what=""):
    """fp16 tensors within ``ulps`` units in the last place (sign-aware bit distance);
    NaN where the reference has NaN (an fp16 step can divide 0 by a denominator that
    underflowed to 0, in the reference as here), whatever its sign bit."""
    got = got.cpu().contiguous()
    ref = ref.contiguous()
    nan_a, nan_b = torch.isnan(got), torch.isnan(ref)
    assert torch.equal(nan_a, nan_b), f"{what}: NaN at {int((nan_a != nan_b).sum())} elements not matched"
    ia = got.view(torch.int16).to(torch.int32)
    ib = ref.view(torch.int16).to(torch.int32)
    ia = torch.where(ia < 0, -(ia & 0x7FFF), ia)
    ib = torch.where(ib < 0, -(ib & 0x7FFF), ib)
    d = torch.where(nan_b, torch.zeros_like(ia), (ia - ib).abs())
    assert int(d.max()) <= ulps, f"{what}: {int(d.max())} fp16 ulps ({int((d > ulps).sum())} elements)"


def _cmp_tensor(got, gold_arr, what, rel=1e-6, floor=1e-9):
    if got.dtype == torch.bfloat16:
        _cmp_bf16(got.reshape(-1), to_torch(gold_arr, torch.bfloat16).reshape(-1), what=what)
    elif got.dtype == torch.float16:
        _cmp_f16(got.reshape(-1), torch.from_numpy(gold_arr).reshape(-1), what=what)
    elif got.dtype == torch.float32:
        _cmp_f32(got.reshape(-1), torch.from_numpy(gold_arr).reshape(-1), rel=rel,
                 floor=1e-12 if what.startswith("v") else floor, what=what)
    else:
        a = got.cpu().reshape(-1).to(torch.int32)
        b = torch.from_numpy(gold_arr.reshape(-1).astype(np.int32))
        if got.dtype == torch.uint8 and what.startswith("m"):  # packed NF4 nibbles
            a = torch.stack([a >> 4, a & 15], 1).reshape(-1)
            b = torch.stack([b >> 4, b & 15], 1).reshape(-1)
        d = (a - b).abs()
        assert int(d.max()) <= 1, f"{what}: codes differ by {int(d.max())}"


@pytest.mark.parametrize("name", sorted(CASES))
def test_hip_step_matches_reference_trajectory(name):
    _require_gpu()
    from apexw_amd import ApexW
    params, opt, gold = replay(name, ApexW, device=dev)
    torch.cuda.synchronize()
    if "flags_0" not in gold:
        # beta3: torch's CPU fp32 sqrt is faithfully rounded where the kernel's is IEEE, and
        # beta3's updates (slow_ratio up to ~5000) are ~6e-3 per step: fp32 p near 0 may
        # differ by ~1 ulp of the update per step
        _cmp_factored(params, opt, gold, initial_params(name), CASES[name][2],
                      floor=4e-9 if "beta3" in name else 1e-9)
        return
    rel, floor = 1e-6, 1e-9
    if name in FP32_CLIP_CASES:
        steps, kw = CASES[name][2], CASES[name][4]
        rel, floor = 1e-5, 2.0 ** -8 * steps * kw["lr"] + 1e-9
    for i, p in enumerate(params):
        st = opt.state[p]
        _cmp_tensor(p.data, gold[f"p_{i}"], f"p_{i}", rel, floor)
        _cmp_tensor(st["exp_avg"], gold[f"m_{i}"], f"m_{i}", rel)
        _cmp_tensor(st["exp_avg_sq"], gold[f"v_{i}"], f"v_{i}", rel)
        if f"ms_{i}" in gold:
            _cmp_f32(st["exp_avg_scales"].reshape(-1), torch.from_numpy(gold[f"ms_{i}"]).reshape(-1), floor=0,
                     rel=1e-6, what=f"ms_{i}")
            _cmp_f32(st["exp_avg_sq_scales"].reshape(-1), torch.from_numpy(gold[f"vs_{i}"]).reshape(-1), floor=0,
                     rel=1e-6, what=f"vs_{i}")


def _codes6(q):
    w = q.reshape(-1, 3).to(torch.int32)
    word = w[:, 0] | (w[:, 1] << 8) | (w[:, 2] << 16)
    return torch.stack([(word >> (6 * i)) & 63 for i in range(4)], 1).reshape(-1)


def _cmp_factored(params, opt, gold, init, steps, floor=1e-9):
    for i, p in enumerate(params):
        st = opt.state[p]
        keys = state_keys(gold, i)
        assert keys == sorted(k for k, v in st.items() if torch.is_tensor(v) and k != "step"), f"state keys {i}"
        assert float(st["step"]) == float(gold[f"step_{i}"][0])
        if f"scale_{i}" in gold:
            assert [float(st["scale_v"]), float(st["sqrt_scale_v"])] == gold[f"scale_{i}"].tolist(), f"scale_{i}"
        fac = bool(st.get("is_factored_v", False))
        if not fac:
            _cmp_tensor(p.data, gold[f"p_{i}"], f"p_{i}", floor=floor)
            for k in keys:
                g = gold[f"st_{i}_{k}"]
                if k.endswith("scales"):
                    _cmp_f32(st[k].reshape(-1), torch.from_numpy(g).reshape(-1), floor=0, what=f"{k}_{i}")
                else:
                    _cmp_tensor(st[k], g, f"{'m' if k == 'exp_avg' else 'v'}_{i}")
            continue
        if p.dtype == torch.bfloat16:
            got, ref = p.data.cpu().reshape(-1), to_torch(gold[f"p_{i}"], torch.bfloat16).reshape(-1)
            d = bf16_ulp_diff(got, ref)
            g64, r64, p0 = got.double(), ref.double(), init[i].reshape(-1).double()
            tol = 2.0 ** -7 * steps * (p0.abs() + 2.0 * r64.abs())
            bad = (d > 2) & ((g64 - r64).abs() > tol)
            assert not bool(bad.any()), f"p_{i}: {int(bad.sum())} elements beyond the bar (max {int(d.max())} ulps)"
        elif p.dtype == torch.float16:
            # fp32 decay and update, one rounding to fp16 per step: the bf16 bar with fp16's ulp
            got, ref = p.data.cpu().reshape(-1), torch.from_numpy(gold[f"p_{i}"]).reshape(-1)
            d = bf16_ulp_diff(got, ref)
            g64, r64, p0 = got.double(), ref.double(), init[i].reshape(-1).double()
            tol = 2.0 ** -10 * steps * (p0.abs() + 2.0 * r64.abs())
            bad = (d > 2) & ((g64 - r64).abs() > tol)
            assert not bool(bad.any()), f"p_{i}: {int(bad.sum())} elements beyond the bar (max {int(d.max())} ulps)"
        else:
            _cmp_f32(p.data.reshape(-1), torch.from_numpy(gold[f"p_{i}"]).reshape(-1), rel=1e-5, what=f"p_{i}")
        for k in ("exp_avg_sq_row", "exp_avg_sq_col"):
            _cmp_f32(st[k].reshape(-1), torch.from_numpy(gold[f"st_{i}_{k}"]).reshape(-1), rel=1e-5, floor=1e-30,
                     what=f"{k}_{i}")
        m, gm = st["exp_avg"].cpu(), gold[f"st_{i}_exp_avg"]
        if st.get("is_6bit_m", False):
            d = (_codes6(m) - _codes6(torch.from_numpy(gm.astype(np.uint8)))).abs()
            assert int(d.max()) <= 1, f"6-bit m_{i}: codes differ by {int(d.max())}"
        elif m.dtype == torch.int8:
            d = (m.reshape(-1).to(torch.int32) - torch.from_numpy(gm.reshape(-1).astype(np.int32))).abs()
            assert int(d.max()) <= 1, f"int8 m_{i}: codes differ by {int(d.max())}"
        elif m.dtype == torch.float16:
            _cmp_f16(m.reshape(-1), torch.from_numpy(gm).reshape(-1), ulps=2, what=f"fp16 m_{i}")
        else:
            _cmp_bf16(m.reshape(-1), to_torch(gm, torch.bfloat16).reshape(-1), ulps=2, what=f"bf16 m_{i}")
        if "exp_avg_scales" in keys:
            _cmp_f32(st["exp_avg_scales"].reshape(-1), torch.from_numpy(gold[f"st_{i}_exp_avg_scales"]).reshape(-1),
                     rel=1e-5, floor=0, what=f"m scales {i}")
