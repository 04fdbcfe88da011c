"""Reference-written checkpoints and in-backward trajectories, replayed on the GPU.

* Checkpoints (tests/golden/sd_*.npz): the reference stepped 3 times and wrote
  ``state_dict()``; apexw_amd loads that dict into an optimizer over the
  parameters of that moment, steps the same 2 grads the reference stepped
  next, and must land where the reference landed: compact and 8-bit at the
  bars of test_gpu_parity.py (bf16 <= 1 ulp, fp32 1e-6 relative + 1e-9, codes
  <= 1, scales 1e-6 relative); the hybrid's Muon matrices within 3% relative
  Frobenius of the reference's fp32 update over the 2 steps (the bf16
  Newton-Schulz bound of test_gpu_muon.py), its AdamW tensors at the fp32 bar.
* In-backward trajectories (tests/golden/hooks_*.npz): fp32 parameters, an
  8-bit ApexW that converts them to bf16 and steps the large ones inside
  backward, 3 optimizer steps of one or two backward passes each, with no
  resynchronisation between steps; same bars.
* enable_fused_backward trajectories (tests/golden/fused_*.npz): 8-bit and
  compact, bf16 and fp32 parameters, 6 optimizer steps of one or two backward
  passes each (grad_accum_steps), every parameter stepped inside its own
  post-accumulate hook; no resynchronisation; same bars, except fp32
  parameters: 1e-6 relative plus 2^-20 lr per step taken (a few fp32 ulps of
  each step's update, which at lr 1e-2 is as large as p and can cancel it).
"""

import numpy as np
import pytest
import torch
import torch.nn as nn

from golden_replay import FUSED_CASES, HOOK_CASES, SD_CASES, fused_inputs, hook_inputs, sd_inputs, state_keys
from test_gpu_parity import _cmp_f32, _cmp_tensor

pytestmark = pytest.mark.gpu


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")


def _cmp_state(st, gold, i, keys):
    for k in keys:
        g = gold[f"st_{i}_{k}"]
        if k.endswith("scales"):
            _cmp_f32(st[k].reshape(-1), torch.from_numpy(g).reshape(-1), floor=0, what=f"{k}_{i}")
        elif k == "momentum":
            continue
        else:
            _cmp_tensor(st[k], g, f"{'m' if k == 'exp_avg' else 'v'}_{i}")


@pytest.mark.parametrize("name", sorted(HOOK_CASES))
def test_in_backward_matches_reference_trajectory(name):
    _need_gpu()
    from apexw_amd import ApexW
    from golden.make_golden import HOOK_KW
    print(f"reference in-backward trajectory {name}", flush=True)
    host, grads, gold = hook_inputs(name)
    params = [nn.Parameter(h.cuda()) for h in host]
    opt = ApexW(params, **HOOK_KW)
    assert [{torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}[p.dtype] for p in params] == gold["dtypes"].tolist()
    assert opt._auto_hook_handles, "the in-backward path is not on"
    for per_step in grads:
        for gs in per_step:
            torch.autograd.backward([p.view_as(p) for p in params], grad_tensors=[g.cuda() for g in gs])
        opt.step()
        opt.zero_grad(set_to_none=True)
    torch.cuda.synchronize()
    for i, p in enumerate(params):
        _cmp_tensor(p.data, gold[f"p_{i}"], f"p_{i}")
        st = opt.state[p]
        _cmp_state(st, gold, i, ("exp_avg", "exp_avg_scales", "exp_avg_sq", "exp_avg_sq_scales"))
        assert float(st["step"]) == float(gold[f"step_{i}"][0]), f"step_{i}"
    opt._disable_auto_8bit_hooks()


@pytest.mark.parametrize("name", sorted(FUSED_CASES))
def test_fused_backward_matches_reference_trajectory(name):
    _need_gpu()
    from apexw_amd import ApexW
    print(f"reference enable_fused_backward trajectory {name}", flush=True)
    dtype, kwargs, host, grads, gold = fused_inputs(name)
    params = [nn.Parameter(h.cuda()) for h in host]
    opt = ApexW(params, **kwargs)
    opt.enable_fused_backward(grad_accum_steps=len(grads[0]))
    for per_step in grads:
        for gs in per_step:
            torch.autograd.backward([p.view_as(p) for p in params], grad_tensors=[g.cuda() for g in gs])
        assert all(p.grad is None for p in params)
        opt.step()
        opt.zero_grad(set_to_none=True)
    torch.cuda.synchronize()
    steps = len(grads)
    for i, p in enumerate(params):
        _cmp_tensor(p.data, gold[f"p_{i}"], f"p_{i}", floor=2.0 ** -20 * kwargs["lr"] * steps + 1e-9)
        st = opt.state[p]
        keys = state_keys(gold, i)
        assert keys == sorted(k for k, v in st.items() if torch.is_tensor(v) and k != "step"), f"state keys {i}"
        _cmp_state(st, gold, i, keys)
        assert float(st["step"]) == float(gold[f"step_{i}"][0]) == 6.0, f"step_{i}"
    opt.disable_fused_backward()


def _rel_fro(a, b):
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


@pytest.mark.parametrize("name", sorted(SD_CASES))
def test_reference_checkpoint_resumes(name):
    _need_gpu()
    from apexw_amd import ApexW
    print(f"reference checkpoint {name}", flush=True)
    shapes, dtype, kwargs, sd, mid, grads, gold = sd_inputs(name)
    params = [nn.Parameter(m.cuda()) for m in mid]
    opt = ApexW(params, **kwargs)
    opt.load_state_dict(sd)
    hybrid = type(opt).__name__ == "HybridApexW"
    for gs in grads:
        for p, g in zip(params, gs):
            p.grad = g.cuda()
        opt.step()
    torch.cuda.synchronize()
    muon_ids = {id(p) for p in opt.muon_params} if hybrid else set()
    for i, p in enumerate(params):
        keys = state_keys(gold, i)
        st = opt.state[p]
        assert keys == sorted(k for k, v in st.items() if torch.is_tensor(v) and k != "step"), f"state keys {i}"
        if id(p) in muon_ids:
            got, ref, start = p.detach().cpu().double(), torch.from_numpy(gold[f"p_{i}"]).double(), mid[i].double()
            assert _rel_fro(got - start, ref - start) <= 0.03, f"muon p_{i}"
            mom, gmom = st["momentum"].cpu().double(), torch.from_numpy(gold[f"st_{i}_momentum"]).double()
            assert float(((mom - gmom).abs() - (1e-6 * gmom.abs() + 1e-12)).max()) <= 0, f"momentum_{i}"
            continue
        _cmp_tensor(p.data, gold[f"p_{i}"], f"p_{i}")
        _cmp_state(st, gold, i, keys)
