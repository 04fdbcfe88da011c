"""Pins of oracle.muon.coordwise_step (ApexMuon's coordinate-wise fallback,
apexw/muon.py:775-799, :841-858) by what the mathematics fixes."""

import math

import torch

from oracle.muon import coordwise_step


def _first(g, lr=1e-2, mu=0.95, wd=0.0, p=None, nesterov=False):
    p = torch.zeros_like(g) if p is None else p
    buf = torch.zeros_like(g, dtype=torch.float32)
    U = coordwise_step(p, g, buf, lr=lr, momentum=mu, weight_decay=wd, nesterov=nesterov)
    return p, buf, U


def test_two_elements_population_std():
    """s = (1 - mu) g; for two elements the population std is |s0 - s1| / 2, so
    U = +-2 s / |s0 - s1| around the mean -- the unbiased std would give sqrt(2)."""
    g = torch.tensor([3.0, 1.0])
    _, buf, U = _first(g)
    s = buf.double()
    std = abs(float(s[0] - s[1])) / 2.0
    assert torch.allclose(U.double(), s / (std + 1e-7), rtol=1e-6, atol=0)


def test_one_element():
    g = torch.tensor([-2.5])
    _, buf, U = _first(g)
    assert math.isclose(float(U), float(buf) / (abs(float(buf)) + 1e-7), rel_tol=1e-7)
    assert float(U) < 0


def test_scale_invariance_from_zero_momentum():
    torch.manual_seed(0)
    g = torch.randn(300)
    _, _, U1 = _first(g)
    _, _, U2 = _first(g * 64.0)        # a power of two: s scales exactly, std scales exactly
    assert torch.allclose(U1, U2, rtol=1e-5, atol=1e-5)   # the +1e-7 moves U by ~2e-6 relative
    # U has unit population std (std(s) >> 1e-7)
    assert abs(float(U1.std(unbiased=False)) - 1.0) < 1e-5


def test_first_step_update():
    """From zero momentum: p' = p (1 - lr wd) - lr * 0.05 * U in fp32."""
    torch.manual_seed(1)
    g = torch.randn(64)
    p0 = torch.randn(64)
    p, _, U = _first(g, lr=1e-2, wd=0.1, p=p0.clone())
    ref = p0 * (1.0 - 1e-2 * 0.1) - 1e-2 * 0.05 * U
    assert torch.allclose(p, ref, rtol=1e-6, atol=1e-9)


def test_nesterov_source():
    """With nesterov the source is lerp(g, buf, mu): from zero momentum that is
    g (1 - mu (1 - (1 - mu))) = g (1 - mu^2); its normalised form equals g's."""
    torch.manual_seed(2)
    g = torch.randn(100)
    _, _, Un = _first(g, nesterov=True)
    _, _, U = _first(g)
    assert torch.allclose(Un, U, rtol=1e-5, atol=1e-5)
