"""Checkpoint format fidelity on the CPU: a state_dict written by the reference
(tests/golden/sd_*.npz, after 3 steps) loads into apexw_amd's optimizer with
every state tensor in its saved dtype, shape and bytes, and apexw_amd's own
state_dict() of that optimizer equals the reference's: the same param_groups
(keys and values), the same per-parameter state keys, tensors bit for bit and
scalars equal.  No step runs (stepping needs the GPU); the GPU continuation is
tests/test_gpu_reference_state.py.
"""

import pytest
import torch

from golden.sd_codec import decode, encode
from golden_replay import SD_CASES, sd_inputs


def _same(a, b, where):
    if torch.is_tensor(a):
        assert torch.is_tensor(b), where
        assert a.dtype == b.dtype and a.shape == b.shape, f"{where}: {a.dtype}{tuple(a.shape)} vs {b.dtype}{tuple(b.shape)}"
        assert torch.equal(a.cpu(), b.cpu()), where
    elif isinstance(a, dict):
        assert isinstance(b, dict) and set(a) == set(b), f"{where}: keys {sorted(map(str, a))} vs {sorted(map(str, b))}"
        for k in a:
            _same(a[k], b[k], f"{where}/{k}")
    elif isinstance(a, (list, tuple)):
        assert len(a) == len(b), where
        for i, (x, y) in enumerate(zip(a, b)):
            _same(x, y, f"{where}[{i}]")
    else:
        assert a == b, f"{where}: {a!r} vs {b!r}"


@pytest.mark.parametrize("name", sorted(SD_CASES))
def test_reference_checkpoint_round_trips(name):
    from apexw_amd import ApexW
    shapes, dtype, kwargs, sd, mid, grads, gold = sd_inputs(name)
    params = [torch.nn.Parameter(m.clone()) for m in mid]
    with _quiet():
        opt = ApexW(params, **kwargs)
    opt.load_state_dict(sd)
    ours = opt.state_dict()
    ref = decode(*encode(sd))   # a fresh copy: loading must not have changed the caller's dict
    if "muon_state_dict" in ref:
        for key in ("muon_state_dict", "adamw_state_dict"):
            _same(ref[key]["state"], ours[key]["state"], key)
            _same(ref[key]["param_groups"], ours[key]["param_groups"], key)
    _same(ref["state"], ours["state"], "state")
    _same(ref["param_groups"], ours["param_groups"], "param_groups")
    # the loaded tensors are the saved ones, in their saved dtypes
    for p, st in opt.state.items():
        for k, v in st.items():
            if torch.is_tensor(v):
                assert v.device == p.device


class _quiet:
    def __enter__(self):
        import warnings
        self._cm = warnings.catch_warnings()
        self._cm.__enter__()
        warnings.simplefilter("ignore")

    def __exit__(self, *exc):
        return self._cm.__exit__(*exc)


def test_codec_round_trip():
    """encode/decode keep every tensor's dtype and bytes and every scalar's type."""
    sd = {"state": {0: {"step": torch.tensor(3.0), "exp_avg": torch.randn(5).bfloat16(),
                        "exp_avg_sq": torch.randint(0, 255, (7,), dtype=torch.uint8), "is_8bit": True,
                        "state_dtype": torch.int8, "block_size_8bit": 2048}},
          "param_groups": [{"betas": (0.9, 0.999), "lr": 1e-3, "params": [0], "clip_grad_norm": None}],
          "_dynamic_scaling_meta": {}}
    _same(sd, decode(*encode(sd)), "sd")
