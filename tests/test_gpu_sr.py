"""Stochastic rounding on the GPU is unbiased (|mean error| < 3 sigma over >= 1e7 elements).

At the first step from zero state the pre-rounding values are known exactly:
  m = (1 - b1) g,  v = (1 - b2) g^2 (quad: (1 - b2) mean4(g^2)),
and the parameter before rounding is the fp32 result of the same step on an
fp32 copy of the parameters (the CPU oracle with fp32 params, no rounding).
Each test checks that the rounded outputs straddle those values (floor/ceil
only) and that the mean rounding error, in units of the local rounding gap,
is within 3 standard errors of zero.
"""

import math

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
N = 5120 * 2048  # 10,485,760 elements


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")


def _unbiased(err, what):
    err = err.double()
    mean, sd = float(err.mean()), float(err.std())
    se = sd / math.sqrt(err.numel())
    assert abs(mean) < 3 * se, f"{what}: mean {mean:.3e} vs 3*se {3 * se:.3e}"


def _bf16_gap(x):
    """Spacing of bf16 values at |x| (fp32 input)."""
    e = torch.floor(torch.log2(x.abs().clamp_min(1e-30)))
    return torch.exp2(e - 7)


def test_bf16_param_sr_unbiased_8bit():
    _need_gpu()
    from apexw_amd import ApexW
    from oracle.optim import OracleApexW
    torch.manual_seed(0)
    shape = (5120, 2048)
    p0 = (torch.randn(shape) * 0.02).bfloat16()
    g = (torch.randn(shape) * 1e-3).bfloat16()
    kw = dict(lr=1e-3, weight_decay=0.1, adamw_compat=True, precision="8bit")
    gp = torch.nn.Parameter(p0.cuda())
    gp.grad = g.cuda()
    ApexW([gp], stochastic_rounding=True, **kw).step()
    cp = torch.nn.Parameter(p0.float())
    cp.grad = g.float()
    OracleApexW([cp], stochastic_rounding=False, **kw).step()
    x = cp.detach()
    got = gp.detach().float().cpu()
    # p*decay - update cancels for some elements; there the fp32 rounding of the
    # two sides (one fma on the GPU, two ops on the CPU) exceeds a bf16 gap of x
    keep = x.abs() > 1e-4
    err = ((got - x) / _bf16_gap(x))[keep]
    assert float(err.abs().max()) <= 1.0 + 1e-3
    _unbiased(err, "bf16 param SR (8-bit step)")


def test_nf4_and_logu8_code_sr_unbiased():
    _need_gpu()
    from apexw_amd import ApexW
    from oracle.quant import NF4_CODEBOOK, V_LOG_LUT
    torch.manual_seed(1)
    shape = (5120, 2048)
    g = (torch.randn(shape) * 1e-3).bfloat16()
    p = torch.nn.Parameter(torch.zeros(shape, dtype=torch.bfloat16, device="cuda"))
    p.grad = g.cuda()
    opt = ApexW([p], lr=1e-3, weight_decay=0.0, precision="8bit", stochastic_rounding=True)
    opt.step()
    st = opt.state[p]
    assert st["is_4bit_m"] and st["is_quad_v"]
    gf = g.float().reshape(-1)
    m_exact = torch.tensor(np.float32(1 - 0.9)) * gf  # lerp from zero: fma(w, g - 0, 0)
    ms = st["exp_avg_scales"].cpu().reshape(-1)
    codes = st["exp_avg"].cpu()
    c = torch.stack([codes >> 4, codes & 15], 1).reshape(-1).long()
    deq = NF4_CODEBOOK[c]
    x = (m_exact.view(-1, 2048) / ms[:, None]).reshape(-1).clamp(-1, 1)
    lev = NF4_CODEBOOK[:15]
    hi = torch.searchsorted(lev, x).clamp(0, 14)
    lo = (hi - 1).clamp_min(0)
    gap = (lev[hi] - lev[lo]).clamp_min(1e-12)
    ok = (deq == lev[hi]) | (deq == lev[lo])
    bad = torch.nonzero(~ok).reshape(-1)
    # x within a few ulps of a level may land on the other side of it in the
    # kernel's reciprocal-multiply; only such elements may pick the level below
    near = (x[bad, None] - lev[None, :]).abs().min(1).values < 1e-6 if bad.numel() else torch.zeros(0, dtype=torch.bool)
    assert bad.numel() <= 8 and bool(near.all()), (
        f"NF4 SR picked a non-neighbouring level for {bad.numel()} elements, e.g. "
        f"{[(float(x[i]), int(c[i]), float(deq[i]), float(lev[lo[i]]), float(lev[hi[i]])) for i in bad[:5]]}")
    _unbiased((deq - x) / gap, "NF4 momentum SR")
    # log-uint8 v: SR is unbiased in the code domain
    gq = (gf.view(-1, 4) ** 2).sum(1) / 4
    v_exact = torch.tensor(np.float32(1 - 0.999)) * gq
    vs = st["exp_avg_sq_scales"].cpu().reshape(-1)
    qf = torch.log2((v_exact.view(-1, 512) / vs[:, None]).clamp_min(2.0 ** -24)) * (254.0 / 24.0) + 255.0
    qv = st["exp_avg_sq"].cpu().reshape(-1).float()
    qf = qf.reshape(-1)
    keep = (qf > 1.5) & (qf < 254.5) & (v_exact > 0)
    d = (qv - qf)[keep]
    assert float(d.abs().max()) < 1.0 + 1e-3
    _unbiased(d, "log-uint8 variance SR")


def test_compact_bf16_sr_unbiased():
    """Compact quad-v group (8 tensors): SR of the bf16 params and of the bf16 v EMA."""
    _need_gpu()
    from apexw_amd import ApexW
    torch.manual_seed(2)
    shapes = [(640, 2048)] * 8
    p0 = [(torch.randn(s) * 0.02).bfloat16() for s in shapes]
    g = [(torch.randn(s) * 1e-3).bfloat16() for s in shapes]
    ps = [torch.nn.Parameter(p.cuda()) for p in p0]
    for p, gg in zip(ps, g):
        p.grad = gg.cuda()
    opt = ApexW(ps, lr=1e-3, weight_decay=0.1, adamw_compat=True, stochastic_rounding=True)  # beta2 0.999
    opt.step()
    b2 = np.float32(1 - 0.999)
    es = np.float32(1e-8 * math.sqrt(1 - 0.999))
    ss = np.float32(1e-3 * math.sqrt(1 - 0.999) / (1 - 0.9))
    wd = torch.tensor(np.float32(1 - 1e-4)).bfloat16().float()  # foreach scalar rounded to bf16
    verr, perr = [], []
    for p, pp, gg in zip(ps, p0, g):
        st = opt.state[p]
        assert st.get("is_quad_v", False)
        gf = gg.float().reshape(-1, 4)
        sq = gf * gf
        gq = (((sq[:, 0] + sq[:, 1]) + sq[:, 2]) + sq[:, 3]) * 0.25
        v_exact = torch.tensor(b2) * gq                      # fma(1-b2, gq, 0*b2)
        v_got = st["exp_avg_sq"].float().cpu()
        keep = v_exact > 0
        verr.append(((v_got - v_exact) / _bf16_gap(v_exact))[keep])
        m = st["exp_avg"].float().cpu().reshape(-1, 4)
        d = (torch.sqrt(v_got).bfloat16().float() + torch.tensor(es).bfloat16().float()).bfloat16().float()
        pw = (pp.float() * wd).bfloat16().float().reshape(-1, 4)
        x = (pw - (m / d[:, None]) * torch.tensor(ss)).reshape(-1)
        got = p.detach().float().cpu().reshape(-1)
        k2 = x.abs() > 1e-4
        perr.append(((got - x) / _bf16_gap(x))[k2])
    verr, perr = torch.cat(verr), torch.cat(perr)
    assert float(verr.abs().max()) <= 1.0 + 1e-6 and float(perr.abs().max()) <= 1.0 + 1e-3
    _unbiased(verr, "compact bf16 v SR")
    _unbiased(perr, "compact bf16 param SR")


# ---------------------------------------------------------------------------
# SR beyond the first step, per kernel branch: three round-to-nearest steps, then
# two SR steps from the state they left, each against the oracle run from the
# GPU's pre-step state (tests/sr_inject.py: every SR result in the bracket of the
# exact pre-rounding value, |z| < 3 signed and by magnitude over >= 1e7 elements,
# the deterministic parts at the round-to-nearest bars).
# ---------------------------------------------------------------------------
SR_BRANCHES = [
    # name, precision, param dtype, shapes, extra kwargs, SR outputs with >= 1e7 elements
    ("nf4 fast kernel, partial last blocks", "8bit", torch.bfloat16, [(4000, 1037)] * 10, {},
     ("bf16", "nf4", "logu8")),
    ("nf4 generic-order quad (<= 262144 elements)", "8bit", torch.bfloat16, [(256, 1024)] * 160, {},
     ("bf16", "nf4", "logu8")),
    ("int8 + log-u8, general kernel, generic order", "8bit", torch.bfloat16, [(10240,)] * 1024, {},
     ("int8", "logu8")),
    ("int8 + log-u8, general kernel, chunked order", "8bit", torch.bfloat16, [(1000002,)] * 11, {},
     ("bf16", "int8", "logu8")),
    ("fp32 parameters, nf4 codes", "8bit", torch.float32, [(4096, 10240)], {}, ("nf4", "logu8")),
    # a homogeneous group (every state in the parameter dtype and size) takes the
    # reference's torch._fused_adamw_ path, which has no SR; the quad tensor makes the
    # group mixed, so the non-quad ones (numel % 4 != 0) take the foreach path with SR v
    ("compact non-quad bf16 v with SR", "compact", torch.bfloat16, [(1000001,)] * 10 + [(2048, 1024)],
     {"force_compact_v": True}, ("bf16",)),
]


@pytest.mark.parametrize("name,prec,dtype,shapes,extra,kinds", SR_BRANCHES, ids=[b[0] for b in SR_BRANCHES])
def test_sr_branch_after_rne_steps(name, prec, dtype, shapes, extra, kinds):
    _need_gpu()
    from test_gpu_configs import KW, _drive
    print(f"SR branch: {name}", flush=True)
    kw = dict(KW, precision=prec, **extra)
    stats = _drive(name, shapes, dtype, kw, [(i, None) for i in range(len(shapes))], 5, True,
                   seed=sum(map(ord, name)) % 10007, sr_from=3)
    for k in kinds:
        st = stats[k]
        assert st.n >= 10_000_000 and abs(st.z) < 3 and abs(st.z_mag) < 3, (k, st)
