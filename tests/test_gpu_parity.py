"""GPU parity: the HIP step against the reference's own trajectories and the CPU oracle.

Tolerances (round to nearest, SR off):
  * fp32 params:  |d| <= 1e-6*|ref| + 1e-9 (the absolute floor covers p ~ 0)
  * bf16 tensors (params, m, v): <= 1 bf16 ulp
  * fp32 v (compact):             |d| <= 1e-6*|ref| + 1e-12
  * 8-bit codes: NF4/INT8/log-u8 differ by <= 1 code; block scales within 1e-6 relative
"""

import numpy as np
import pytest
import torch

from golden_replay import CASES, bf16_ulp_diff, replay, to_torch

pytestmark = pytest.mark.gpu

dev = "cuda"


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


def _cmp_tensor(got, gold_arr, what):
    if got.dtype == torch.bfloat16:
        _cmp_bf16(got.reshape(-1), to_torch(gold_arr, torch.bfloat16).reshape(-1), what=what)
    elif got.dtype == torch.float32:
        _cmp_f32(got.reshape(-1), torch.from_numpy(gold_arr).reshape(-1), floor=1e-12 if what.startswith("v") else 1e-9,
                 what=what)
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
    for i, p in enumerate(params):
        st = opt.state[p]
        _cmp_tensor(p.data, gold[f"p_{i}"], f"p_{i}")
        _cmp_tensor(st["exp_avg"], gold[f"m_{i}"], f"m_{i}")
        _cmp_tensor(st["exp_avg_sq"], gold[f"v_{i}"], f"v_{i}")
        if f"ms_{i}" in gold:
            _cmp_f32(st["exp_avg_scales"].reshape(-1), torch.from_numpy(gold[f"ms_{i}"]).reshape(-1), floor=0,
                     rel=1e-6, what=f"ms_{i}")
            _cmp_f32(st["exp_avg_sq_scales"].reshape(-1), torch.from_numpy(gold[f"vs_{i}"]).reshape(-1), floor=0,
                     rel=1e-6, what=f"vs_{i}")
