"""Pin the oracle's quantizers, SR and Muon pieces against closed forms,
brute force, the reference's own known answers and the Muon golden vectors.

Each check is chosen so that a plausible slip in the restatement (a wrong
midpoint, a shifted LUT index, a missing clamp, a transposed Newton-Schulz
product) fails it; none of them retypes the oracle's own formula.
"""

import math

import numpy as np
import pytest
import torch

from golden.make_golden import _fingerprint, _grad, _param
from golden_replay import load
from oracle import quant
from oracle.muon import (OracleHybrid, muon_eligible, newton_schulz5, newton_schulz5_batched,
                         partition_for_hybrid)

DISTINCT_LEVELS = quant.NF4_CODEBOOK[:15].double()


# ----------------------------------------------------------------- NF4 codes
def test_nf4_dequant_of_every_code_is_the_codebook():
    # reference known answer: tests/test_quantization.py:132-135
    codes = torch.arange(16, dtype=torch.uint8)
    packed = (codes << 4) | codes
    out = quant.dequant_nf4(packed, torch.ones(1, 1), 32, 32).view(16, 2)
    assert torch.equal(out[:, 0], quant.NF4_CODEBOOK) and torch.equal(out[:, 1], quant.NF4_CODEBOOK)
    # symmetric levels, exact zero at index 7, index 15 repeats +1
    cb = quant.NF4_CODEBOOK
    assert float(cb[7]) == 0.0 and float(cb[15]) == 1.0 and float(cb[14]) == 1.0
    assert torch.equal(cb[:7], -cb[8:15].flip(0))


def test_nf4_round_to_nearest_is_brute_force_argmin():
    g = torch.Generator().manual_seed(0)
    x = torch.rand(20000, generator=g) * 2 - 1
    x[:15] = quant.NF4_CODEBOOK[:15]                   # exact levels
    x[15:29] = quant.NF4_MIDS                          # exact midpoints: ties go to the lower code
    packed, scale = quant.quant_nf4(x, 20000)
    assert float(scale) == float(x.abs().max())
    codes = torch.stack([packed >> 4, packed & 15], 1).reshape(-1)[:20000].long()
    normed = (x / scale.reshape(())).double()
    dist = (normed[:, None] - DISTINCT_LEVELS[None, :]).abs()
    best = dist.min(1).values
    got = dist.gather(1, codes[:, None]).squeeze(1)
    assert torch.all(got <= best + 1e-7)
    ties = codes[15:29]
    assert torch.equal(ties, torch.arange(14)), "midpoint ties must pick the lower code"


def test_nf4_scale_is_ema_max_and_odd_tail_is_padded_with_zero_code():
    x = torch.tensor([0.5, -0.25, 0.1])
    packed, scale = quant.quant_nf4(x, 4, old_scales=torch.tensor([1.0]))
    assert math.isclose(float(scale), 0.9, rel_tol=1e-7)          # max(0.5, 0.9 * 1.0)
    assert int(packed[1]) & 15 == 7                                 # pad nibble = code of 0.0
    packed2, scale2 = quant.quant_nf4(torch.zeros(4), 4)
    assert float(scale2) == float(np.float32(1e-12)) and torch.all(packed2 == 0x77)


def test_nf4_stochastic_rounding_picks_neighbours_with_the_right_probability():
    torch.manual_seed(3)
    x0 = 0.3 * torch.ones(200000)                      # between 0.2844 (idx 10) and 0.3949 (idx 11)
    x = torch.cat([x0, torch.tensor([1.0])])           # absmax 1 keeps x0 unscaled
    packed, _ = quant.quant_nf4(x, x.numel(), stochastic=True)
    codes = torch.stack([packed >> 4, packed & 15], 1).reshape(-1)[:200000]
    assert set(codes.unique().tolist()) <= {10, 11}
    p_hi = (0.3 - 0.2844) / (0.3949 - 0.2844)
    frac = float((codes == 11).double().mean())
    assert abs(frac - p_hi) < 4 * math.sqrt(p_hi * (1 - p_hi) / 200000)


# ----------------------------------------------------------- INT8 codes
def test_int8_round_trip_and_extremes():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(4096, generator=g)
    q, scale = quant.quant_int8(x, 1024)
    back = quant.dequant_int8(q, scale, 1024)
    assert q.abs().max() == 127
    per_block = scale.view(-1, 1).expand(-1, 1024).reshape(-1)
    assert torch.all((back - x).abs() <= per_block / 2 + 1e-7)
    # the block maximum maps to exactly +-127
    for b in range(4):
        blk = x[b * 1024:(b + 1) * 1024]
        i = int(blk.abs().argmax())
        assert abs(int(q[b * 1024 + i])) == 127


# ------------------------------------------------------------ log-uint8 codes
def test_logu8_lut_closed_form():
    lut = quant.V_LOG_LUT
    assert float(lut[0]) == 0.0 and float(lut[1]) == 2.0 ** -24 and float(lut[255]) == 1.0
    # 254 steps over 24 octaves: every code step is a constant ratio 2^(24/254)
    ratio = (lut[2:].double() / lut[1:-1].double())
    assert torch.allclose(ratio, torch.full_like(ratio, 2.0 ** (24.0 / 254.0)), rtol=1e-6)
    assert float(lut[128]) == np.float32(2.0 ** (127 * 24.0 / 254.0 - 24.0))


def test_logu8_quantizer_rounds_the_log_code():
    g = torch.Generator().manual_seed(2)
    v = torch.exp(torch.rand(8192, generator=g) * 30 - 28)      # spans > 24 octaves below the max
    v[5] = 0.0
    q, vmax = quant.quant_logu8(v, 8192)
    assert float(vmax) == float(v.max())
    assert int(q[5]) == 0 and int(q[int(v.argmax())]) == 255
    r = (v.double() / float(vmax))
    exact = torch.tensor([quant.logu8_code_exact(float(t)) for t in r])
    keep = (v > 0) & (exact > 1.0)
    assert torch.all((q[keep].double() - exact[keep]).abs() <= 0.5 + 1e-4)
    tiny = (v > 0) & (r < 2.0 ** -24)
    assert torch.all(q[tiny] == 1)                               # clamped ratio -> code 1
    back = quant.dequant_logu8(q, vmax, 8192)
    rel = (back[keep].double() / v[keep].double()).log2().abs()
    assert float(rel.max()) <= 0.5 * 24.0 / 254.0 + 1e-4         # half a code step in octaves


# ---------------------------------------------------------------- 16-bit SR
def test_bf16_stochastic_rounding_is_unbiased_and_brackets():
    torch.manual_seed(4)
    x = (torch.rand(400000) * 2 - 1) * 3.0
    out = torch.empty(x.shape, dtype=torch.bfloat16)
    quant.store_16bit(out, x, stochastic=True)
    lo = x.view(torch.int32).bitwise_and(-65536).view(torch.float32)
    hi_bits = x.view(torch.int32).bitwise_and(-65536) + 65536
    hi = hi_bits.view(torch.float32)
    o = out.float()
    assert torch.all((o == lo) | (o == hi))
    gap = (hi - lo).abs()
    err = ((o - x) / gap).double()
    assert abs(float(err.mean())) < 3 * float(err.std()) / math.sqrt(err.numel())
    rne = torch.empty_like(out)
    quant.store_16bit(rne, x, stochastic=False)
    assert torch.equal(rne, x.to(torch.bfloat16))


# ---------------------------------------------------------------- Muon
def test_newton_schulz_matches_reference_vectors():
    z = load("muon")
    for i in range(3):
        G = torch.from_numpy(z[f"ns_in_{i}"])
        U = newton_schulz5(G, steps=5, work_dtype=torch.float32)
        assert torch.allclose(U, torch.from_numpy(z[f"ns_out_{i}"]), rtol=0, atol=2e-6), i


def test_newton_schulz_polar_invariants():
    # reference known answer: with torch.manual_seed(42) and these shapes the singular
    # values land in (0.5, 1.3) (tests/test_muon.py:26-51)
    torch.manual_seed(42)
    for shape in [(64, 64), (128, 64), (64, 128)]:
        G = torch.randn(shape)
        X = newton_schulz5(G, steps=5)
        s = torch.linalg.svdvals(X.double())
        assert float(s.min()) > 0.5 and float(s.max()) < 1.3, shape


def test_newton_schulz_is_the_scalar_quintic_on_each_singular_value():
    # closed form: X_{k+1} = a X + (b A + c A^2) X with A = X X^T keeps G's singular
    # vectors and maps every normalised singular value s to a s + b s^3 + c s^5
    g = torch.Generator().manual_seed(5)
    for shape in [(48, 96), (96, 48), (40, 40)]:
        G = torch.randn(shape, generator=g, dtype=torch.float64).float()
        X = newton_schulz5(G, steps=5).double()
        Ug, sg, Vh = torch.linalg.svd(G.double(), full_matrices=False)
        s = sg / (float(G.norm()) + 1e-7)
        for _ in range(5):
            s = 3.4445 * s - 4.7750 * s ** 3 + 2.0315 * s ** 5
        proj = Ug.T @ X @ Vh.T
        assert torch.allclose(torch.diagonal(proj), s, atol=2e-4), shape
        assert float((proj - torch.diag(torch.diagonal(proj))).abs().max()) < 2e-4, shape


def test_batched_newton_schulz_equals_single():
    # reference known answer: batched == single < 1e-5 (tests/test_muon.py:53-70)
    g = torch.Generator().manual_seed(6)
    Xb = torch.randn(3, 32, 80, generator=g)
    Ub = newton_schulz5_batched(Xb)
    for i in range(3):
        assert torch.allclose(Ub[i], newton_schulz5(Xb[i]), atol=1e-5)


def test_hybrid_routing_matches_reference():
    z = load("muon")
    c5 = [(4096, 4096), (1024, 4096), (1024, 4096), (4096, 4096), (14336, 4096), (14336, 4096), (4096, 14336),
          (4096,), (4096,)]
    params = [torch.nn.Parameter(torch.empty(s, device="meta")) for s in c5]
    mu, _ = partition_for_hybrid(params)
    route = [1 if any(p is q for q in mu) else 0 for p in params]
    assert route == z["route_c5"].tolist()
    assert route == [1, 0, 0, 1, 1, 1, 1, 0, 0]      # k/v (aspect exactly 4) fall back to AdamW
    assert not muon_eligible(torch.nn.Parameter(torch.empty(31, 64, device="meta")))


def test_hybrid_trajectory_matches_reference():
    z = load("muon")
    shapes = [(64, 64), (64, 64), (48, 96), (64,), (4096, 32)]
    gen = torch.Generator().manual_seed(12)
    ps = [torch.nn.Parameter(_param(s, torch.float32, gen)) for s in shapes]
    fp = [_fingerprint(p.data) for p in ps]
    opt = OracleHybrid(ps, lr=1e-3, weight_decay=0.1, stochastic_rounding=False)
    for _ in range(3):
        for p in ps:
            g = _grad(p.shape, torch.float32, gen, 1e-3)
            p.grad = g
            fp.append(_fingerprint(g))
        opt.step()
    np.testing.assert_array_equal(np.array(fp, dtype=np.int64), z["h_fingerprint"])
    assert [1 if any(p is q for q in opt.muon_params) else 0 for p in ps] == z["h_route"].tolist()
    for i, p in enumerate(ps):
        np.testing.assert_allclose(p.data.numpy(), z[f"hp_{i}"], rtol=0, atol=1e-7, err_msg=f"hp_{i}")
