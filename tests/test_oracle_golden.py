"""The CPU oracle reproduces the reference's own outputs bit-for-bit (SR off).

Golden vectors come from tests/golden/make_golden.py, which stepped the reference
implementation on the same seeded inputs.
"""

import numpy as np
import pytest
import torch

from golden_replay import CASES, load, replay, to_torch
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


@pytest.mark.parametrize("name", sorted(CASES))
def test_oracle_matches_reference_trajectory(name):
    params, opt, gold = replay(name, OracleApexW)
    for i, p in enumerate(params):
        np.testing.assert_array_equal(_as_np(p.data).reshape(-1), gold[f"p_{i}"].reshape(-1), err_msg=f"p_{i}")
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


def test_oracle_clip_matches_reference():
    z = load("clip_bf16")
    n = len([k for k in z if k.startswith("g_")])
    grads = [to_torch(z[f"g_{i}"], torch.bfloat16) for i in range(n)]
    clip_grads_(grads, 1.0)
    for i, g in enumerate(grads):
        np.testing.assert_array_equal(_as_np(g), z[f"gc_{i}"])
