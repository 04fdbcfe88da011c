"""Host logic of HybridApexW / ApexMuon (no GPU): routing, constructor contract, state_dict schema."""

import pytest
import torch

from apexw_amd import ApexW
from apexw_amd.hybrid import HybridApexW, partition_parameters_for_hybrid
from apexw_amd.muon import ApexMuon
from golden_replay import load


def _params(shapes):
    return [torch.nn.Parameter(torch.zeros(s)) for s in shapes]


def test_use_muon_routes_to_hybrid_with_reference_defaults():
    ps = _params([(64, 64), (64, 64), (48, 96), (64,), (4096, 32)])
    with pytest.warns(UserWarning):
        opt = ApexW(ps, lr=1e-3, weight_decay=0.1, use_muon=True, stochastic_rounding=False)
    assert isinstance(opt, HybridApexW)
    assert [1 if any(p is q for q in opt.muon_params) else 0 for p in ps] == load("muon")["h_route"].tolist()
    mg = opt.muon_opt.defaults
    assert mg["lr"] == pytest.approx(5e-3) and mg["ns_steps"] == 5 and mg["momentum"] == 0.95
    assert mg["scale_mode"] == "rms_matched" and mg["ns_method"] == "newtonschulz5"
    assert opt.adamw_opt.defaults["betas"] == (0.9, 0.99)
    with pytest.warns(UserWarning):
        h2 = ApexW(_params([(64, 64), (64,)]), precision="hybrid", stochastic_rounding=False)
    assert isinstance(h2, HybridApexW)


def test_module_partition_uses_names():
    m = torch.nn.ModuleDict({"embed": torch.nn.Embedding(100, 64), "proj": torch.nn.Linear(64, 64),
                             "norm": torch.nn.LayerNorm(64), "lm_head": torch.nn.Linear(64, 100, bias=False)})
    mu, aw = partition_parameters_for_hybrid(m)
    assert [tuple(p.shape) for p in mu] == [(64, 64)]
    assert len(aw) == 5   # embedding, proj bias, norm weight/bias, lm_head


def test_grouped_params_keep_overrides_and_tags():
    a, b, c = _params([(64, 64), (64, 64), (64,)])
    opt = HybridApexW([{"params": [a], "lr": 0.5}, {"params": [b, c], "use_muon": False}], lr=1e-3)
    assert opt.muon_params == [a] and opt.adamw_params == [b, c]
    assert opt.muon_opt.param_groups[0]["lr"] == 0.5


def test_state_dict_schema_and_round_trip():
    ps = _params([(64, 64), (64,)])
    opt = HybridApexW(ps, lr=1e-3)
    opt.muon_opt._init_param_state(ps[0])["step"] = 3
    sd = opt.state_dict()
    assert set(sd) == {"state", "param_groups", "muon_state_dict", "adamw_state_dict", "apexw_state_dict"}
    assert sd["state"][0]["momentum"].dtype == torch.float32 and sd["state"][0]["step"] == 3
    ps2 = [torch.nn.Parameter(torch.zeros(s, dtype=torch.bfloat16)) for s in [(64, 64), (64,)]]
    opt2 = HybridApexW(ps2, lr=1e-3)
    opt2.load_state_dict(sd)
    st = opt2.state[opt2.muon_params[0]]
    assert st["momentum"].dtype == torch.float32 and st["step"] == 3


def test_apexmuon_contract():
    with pytest.raises(ValueError):
        ApexMuon(_params([(64, 64)]), momentum=1.0)
    for kw in (dict(beta3=0.9), dict(cautious=True), dict(ns_method="polar_express"), dict(scale_mode="rms"),
               dict(precision="8bit")):
        with pytest.raises(NotImplementedError):
            ApexMuon(_params([(64, 64)]), **kw)
    p = torch.nn.Parameter(torch.zeros(64, 64))
    p.grad = torch.zeros(64, 64)
    with pytest.raises(RuntimeError):
        ApexMuon([p]).step()   # CPU tensors: the product path is GPU-only


def test_betas_and_lr_precedence():
    """ApexW betas: adamw_betas, else a betas keyword (its third entry is beta3),
    else apexw_betas, else the precision's default; Muon lr 5 x lr only under the
    rms_matched / spectral scale modes (apexw/hybrid.py:222-266)."""
    ps = lambda: _params([(64, 64), (64,)])  # noqa: E731
    assert HybridApexW(ps()).adamw_opt.defaults["betas"] == (0.9, 0.99)
    assert HybridApexW(ps(), apexw_betas=(0.8, 0.9)).adamw_opt.defaults["betas"] == (0.8, 0.9)
    assert HybridApexW(ps(), apexw_betas=(0.8, 0.9), betas=(0.7, 0.95)).adamw_opt.defaults["betas"] == (0.7, 0.95)
    assert HybridApexW(ps(), adamw_betas=(0.6, 0.97), betas=(0.7, 0.95)).adamw_opt.defaults["betas"] == (0.6, 0.97)
    with pytest.raises(NotImplementedError):   # beta3 (AdEMAMix) from betas[2] is outside the hot path
        HybridApexW(ps(), betas=(0.9, 0.99, 0.999))
    assert HybridApexW(ps(), lr=2e-3, scale_mode="none").muon_opt.defaults["lr"] == pytest.approx(2e-3)
    assert HybridApexW(ps(), lr=2e-3, scale_mode="spectral").muon_opt.defaults["lr"] == pytest.approx(1e-2)
    assert HybridApexW(ps(), lr=2e-3, muon_lr=0.05).muon_opt.defaults["lr"] == 0.05
    h = HybridApexW(ps(), weight_decay=0.3, muon_weight_decay=0.01)
    assert h.muon_opt.defaults["weight_decay"] == 0.01 and h.adamw_opt.defaults["weight_decay"] == 0.3


def test_groups_state_view_and_late_groups():
    a, b, c, d = _params([(64, 64), (64,), (96, 64), (32,)])
    opt = HybridApexW([a, b], lr=1e-3)
    assert opt.param_groups[0] is opt.muon_opt.param_groups[0]     # a schedule edits the engines
    opt.param_groups[1]["lr"] = 0.25
    assert opt.adamw_opt.param_groups[0]["lr"] == 0.25
    assert a not in opt.state and len(opt.state) == 0
    opt.muon_opt._init_param_state(a)
    assert a in opt.state and list(opt.state) == [a] and opt.state[a]["momentum"].shape == (64, 64)
    opt.add_param_group({"params": [c, d], "lr": 0.5})
    assert opt.muon_params == [a, c] and opt.adamw_params == [b, d] and opt.apexw_params is opt.adamw_params
    assert [g["lr"] for g in opt.param_groups] == [pytest.approx(5e-3), 0.5, 0.25, 0.5]
    with pytest.raises(KeyError):
        opt.state[torch.nn.Parameter(torch.zeros(3))]


def test_flat_state_dict_loads_into_both_engines():
    ps = _params([(64, 64), (64,)])
    opt = HybridApexW(ps, lr=1e-3)
    opt.muon_opt._init_param_state(ps[0])["step"] = 7
    opt.adamw_opt.state[ps[1]]["step"] = torch.tensor(4.0)
    opt.adamw_opt.state[ps[1]]["exp_avg"] = torch.full((64,), 0.5, dtype=torch.bfloat16)
    sd = opt.state_dict()
    assert [g["params"] for g in sd["param_groups"]] == [[0], [1]] and set(sd["state"]) == {0, 1}
    flat = {"state": sd["state"], "param_groups": sd["param_groups"]}
    ps2 = _params([(64, 64), (64,)])
    opt2 = HybridApexW(ps2, lr=1e-3)
    opt2.load_state_dict(flat)
    assert opt2.state[ps2[0]]["step"] == 7 and float(opt2.state[ps2[1]]["step"]) == 4.0
    assert opt2.state[ps2[1]]["exp_avg"].dtype == torch.bfloat16
