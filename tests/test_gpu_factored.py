"""Factored second moment (factored_v=True) and packed 6-bit m (six_bit=True) on
the GPU against the CPU oracle, and the reference's own factored-v tests.

Bars: the row / column EMAs are sums over rows and columns, reduced in another
order than torch's CPU kernels, so they are held to 1e-5 relative; everything
downstream is elementwise: codes <= 1, scales 1e-6, m (bf16) bit for bit, and p
within 2^-7 (|p_before| + 2 |p_after|) (bf16: one ulp of the update, which
|p_before| + |p_after| bounds, plus one ulp of the result when the subtraction
lands on a rounding tie), or 1e-6 (fp32) of |p_before| + |p_after|, since the
denominator carries the EMAs' few-ulp difference into the rounding of the update.  Each step starts the oracle from the GPU's state, so a
one-ulp denominator difference is not carried into the next step.
"""

import copy

import numpy as np
import pytest
import torch
import torch.nn as nn

from golden_replay import bf16_ulp_diff

pytestmark = pytest.mark.gpu


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")


def _codes6(q):
    w = q.view(-1, 3).to(torch.int32)
    word = w[:, 0] | (w[:, 1] << 8) | (w[:, 2] << 16)
    return torch.stack([(word >> (6 * i)) & 63 for i in range(4)], 1).reshape(-1)


def _check(gpu_p, cpu_p, prev, gs, cs, tag, scale_rtol=1e-6, m_atol=None):
    got, ref = gpu_p.detach().cpu(), cpu_p.detach()
    if got.dtype == torch.bfloat16:
        # the update u is rounded to bf16 before the subtraction, and a denominator a few
        # fp32 ulps off can move that rounding by one ulp of u (<= 2^-7 |u|); the result
        # round(p_before - u) then moves by up to one more ulp of p_after when p_before - u
        # lands on a rounding tie.  At lr 1e-2 the update can exceed p, and
        # |u| <= |p_before| + |p_after|, so |diff| <= 2^-7 (|p_before| + 2 |p_after|).
        g64, r64, p0 = got.double(), ref.double(), prev.double()
        tol = 2.0 ** -7 * (2.0 * r64.abs() + p0.abs()) + 1e-30
        assert ((g64 - r64).abs() <= tol).all(), f"{tag} p: {int(bf16_ulp_diff(got.reshape(-1), ref.reshape(-1)).max())} ulps"
    elif got.dtype == torch.float16:
        # decay and update in fp32 (the fp32 bound below), then one rounding to fp16: a
        # result on the other side of a tie moves by one fp16 ulp (<= 2^-10 |p_after|,
        # 2^-24 in the subnormal range)
        g64, r64, p0 = got.double(), ref.double(), prev.double()
        tol = 2.0 ** -10 * r64.abs() + 1e-6 * (r64.abs() + p0.abs() + (r64 - p0).abs()) + 2.0 ** -24
        assert ((g64 - r64).abs() <= tol).all(), f"{tag} p: {int(bf16_ulp_diff(got.reshape(-1), ref.reshape(-1)).max())} ulps"
    else:
        g64, r64, p0 = got.double(), ref.double(), prev.double()
        tol = 1e-6 * (r64.abs() + p0.abs() + (r64 - p0).abs()) + 1e-9
        assert ((g64 - r64).abs() <= tol).all(), f"{tag} p"
    for k in ("exp_avg_sq_row", "exp_avg_sq_col"):
        a, b = gs[k].cpu().double(), cs[k].double()
        assert ((a - b).abs() <= 1e-5 * b.abs() + 1e-30).all(), f"{tag} {k}"
    m_g, m_c = gs["exp_avg"].cpu(), cs["exp_avg"]
    if cs.get("is_6bit_m", False):
        assert int((_codes6(m_g) - _codes6(m_c)).abs().max()) <= 1, f"{tag} 6-bit m"
    elif m_c.dtype == torch.int8:
        assert int((m_g.to(torch.int32) - m_c.to(torch.int32)).abs().max()) <= 1, f"{tag} int8 m"
    else:   # the lerp is elementwise and the fp32 result is rounded to nearest-even on both sides
        if m_atol is None:
            assert int(bf16_ulp_diff(m_g.reshape(-1), m_c.reshape(-1)).max()) == 0, f"{tag} bf16 m"
        else:   # a reduction upstream of m: one bf16 ulp, plus its absolute error where it cancels
            a, b = m_g.double(), m_c.double()
            assert ((a - b).abs() <= 2.0 ** -7 * b.abs() + m_atol).all(), f"{tag} bf16 m"
    if "exp_avg_scales" in cs:
        a, b = gs["exp_avg_scales"].cpu().double(), cs["exp_avg_scales"].double()
        assert ((a - b).abs() <= scale_rtol * b.abs()).all(), f"{tag} m scales"


def _sync(gpu_p, cpu_p, gs, cs):
    with torch.no_grad():
        cpu_p.copy_(gpu_p.detach().cpu())
    for k, v in cs.items():
        if torch.is_tensor(v) and k != "step":
            v.copy_(gs[k].cpu())


CASES = [
    ("8bit int8 m, one piece", "8bit", (256, 512), {}),
    ("8bit int8 m, row-chunked stats", "8bit", (1024, 512), {}),
    ("8bit int8 m, ragged cols", "8bit", (200, 333), {}),
    ("8bit 6-bit m", "8bit", (1024, 512), {"six_bit": True}),
    ("8bit 6-bit m, partial last block", "8bit", (1030, 515), {"six_bit": True}),
    ("compact bf16 m", "compact", (1024, 512), {}),
    ("compact bf16 m, ragged", "compact", (1025, 515), {}),
    # rows of 2048+ columns: units inside one row take the single-row update
    ("8bit int8 m, wide rows", "8bit", (128, 4096), {}),
    ("8bit 6-bit m, wide rows", "8bit", (128, 6144), {"six_bit": True}),
    ("8bit int8 m, 3000-col rows", "8bit", (200, 3000), {}),      # units inside and across rows
    ("compact bf16 m, 3000-col rows", "compact", (256, 3000), {}),
]


@pytest.mark.parametrize("name,prec,shape,kw", CASES, ids=[c[0] for c in CASES])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
def test_factored_steps_match_oracle(name, prec, shape, kw, dtype):
    _need_gpu()
    from apexw_amd import ApexW
    from oracle.optim import OracleApexW
    print(f"factored {name} {dtype}", flush=True)
    gen = torch.Generator().manual_seed(sum(map(ord, name)))
    host = (torch.randn(shape, generator=gen) * 0.02).to(dtype)
    small = (torch.randn(300, generator=gen) * 0.02).to(dtype)          # an ordinary tensor beside it
    opts = dict(lr=1e-2, weight_decay=0.1, precision=prec, factored_v=True, stochastic_rounding=False, **kw)
    gps = [nn.Parameter(host.cuda()), nn.Parameter(small.cuda())]
    cps = [nn.Parameter(host.clone()), nn.Parameter(small.clone())]
    gopt, copt = ApexW(gps, **opts), OracleApexW(cps, **opts)
    for step in range(3):
        gs = [(torch.randn(shape, generator=gen) * 1e-3 * (1 + step)).to(dtype), (torch.randn(300, generator=gen) * 1e-3).to(dtype)]
        for gp, cp, g in zip(gps, cps, gs):
            gp.grad, cp.grad = g.cuda(), g.clone()
        prev = cps[0].detach().clone()
        gopt.step()
        copt.step()
        torch.cuda.synchronize()
        st_g, st_c = gopt.state[gps[0]], copt.state[cps[0]]
        assert st_g["is_factored_v"] and st_c["is_factored_v"]
        _check(gps[0], cps[0], prev, st_g, st_c, f"{name} step {step}")
        _sync(gps[0], cps[0], st_g, st_c)


@pytest.mark.parametrize("prec", ["8bit", "compact"])
@pytest.mark.parametrize("clip", [0.5, None])
@pytest.mark.parametrize("shape", [(1024, 512), (128, 4096)])      # 4096 columns: whole-tile statistics
def test_factored_with_clip_and_amp_equals_unscaled(prec, shape, clip):
    """GradScaler's power-of-two scale cancels exactly, also through the clip."""
    _need_gpu()
    from apexw_amd import ApexW
    gen = torch.Generator().manual_seed(5)
    host = (torch.randn(shape, generator=gen) * 0.02).bfloat16()
    pa, pb = nn.Parameter(host.cuda()), nn.Parameter(host.cuda())
    kw = dict(lr=1e-2, precision=prec, factored_v=True, stochastic_rounding=False, clip_grad_norm=clip)
    oa, ob = ApexW([pa], **kw), ApexW([pb], **kw)
    for step in range(3):
        g = (torch.randn(shape, generator=gen) * 1e-2).bfloat16().cuda()
        pa.grad, pb.grad = g * 1024.0, g.clone()
        oa.grad_scale, oa.found_inf = torch.tensor(1024.0, device="cuda"), torch.tensor(0.0, device="cuda")
        oa.step()
        ob.step()
    torch.cuda.synchronize()
    assert torch.equal(pa, pb)
    for k in ("exp_avg", "exp_avg_sq_row", "exp_avg_sq_col"):
        assert torch.equal(oa.state[pa][k], ob.state[pb][k]), k


def test_reference_factored_8bit_routing():
    """test_quantization.py:548-592 on the GPU."""
    _need_gpu()
    from apexw_amd import ApexW
    torch.manual_seed(0)
    model = nn.Sequential(nn.Embedding(1024, 256), nn.Linear(256, 256), nn.Linear(64, 128), nn.LayerNorm(256)).cuda()
    conv = nn.Conv2d(64, 128, 3, bias=False).cuda()
    opt = ApexW(list(model.parameters()) + [conv.weight], lr=1e-3, precision="8bit", factored_v=True)
    idx = torch.randint(0, 1024, (2, 4)).cuda()
    emb_out = model[0](idx).mean(dim=1)
    h = model[3](model[1](emb_out))
    loss = model[2](h[:, :64]).sum() + conv(torch.randn(1, 64, 4, 4).cuda()).sum()
    loss.backward()
    opt.step()
    for p in (model[0].weight, model[1].weight, conv.weight):
        st = opt.state[p]
        assert st["is_factored_v"] and not st["is_4bit_m"] and st["exp_avg"].dtype == torch.int8
        assert st["exp_avg_sq_row"].dtype == torch.float32 and "exp_avg_sq" not in st
        assert torch.isfinite(p).all()
    assert not opt.state[model[2].weight]["is_factored_v"]
    assert not opt.state[model[3].weight]["is_factored_v"]
    big = nn.Linear(512, 512, bias=False).cuda()
    opt_big = ApexW(big.parameters(), lr=1e-3, precision="8bit", factored_v=True)
    big.weight.grad = torch.randn_like(big.weight)
    opt_big.step()
    assert opt_big.get_state_memory_mb() * 1024 * 1024 / big.weight.numel() < 1.05


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_reference_factored_8bit_convergence(dtype):
    """test_quantization.py:594-623 on the GPU (the plain update; cautious, and
    nesterov with factored second moments, are outside this build)."""
    _need_gpu()
    from apexw_amd import ApexW
    torch.manual_seed(7)
    lin = nn.Linear(256, 256, bias=True).to(dtype).cuda()
    target = torch.randn(4, 256, dtype=dtype).cuda()
    x = torch.randn(4, 256, dtype=dtype).cuda()
    opt = ApexW(lin.parameters(), lr=5e-3, weight_decay=0.01, decay_norm_only=True, stochastic_rounding=False,
                precision="8bit", factored_v=True)
    losses = []
    for _ in range(15):
        opt.zero_grad()
        loss = ((lin(x) - target) ** 2).mean()
        loss.backward()
        opt.step()
        losses.append(float(loss.item()))
    assert all(np.isfinite(losses)) and losses[-1] < losses[0] * 0.5
    assert opt.state[lin.weight]["is_factored_v"] and torch.isfinite(lin.weight).all()


def test_reference_factored_checkpoint_roundtrip():
    """test_quantization.py:625-656 on the GPU (bf16)."""
    _need_gpu()
    from apexw_amd import ApexW
    torch.manual_seed(11)
    m1 = nn.Linear(256, 256, bias=False).bfloat16().cuda()
    m2 = nn.Linear(256, 256, bias=False).bfloat16().cuda()
    m2.load_state_dict(m1.state_dict())
    opt1 = ApexW(m1.parameters(), lr=1e-3, precision="8bit", factored_v=True, stochastic_rounding=False)
    m1.weight.grad = torch.randn_like(m1.weight) * 0.1
    opt1.step()
    m2.load_state_dict(m1.state_dict())
    sd = copy.deepcopy(opt1.state_dict())
    opt2 = ApexW(m2.parameters(), lr=1e-3, precision="8bit", factored_v=True, stochastic_rounding=False)
    opt2.load_state_dict(sd)
    st2 = opt2.state[m2.weight]
    assert st2["exp_avg"].dtype == torch.int8 and st2["exp_avg_sq_row"].dtype == torch.float32
    assert torch.equal(st2["exp_avg_sq_row"], opt1.state[m1.weight]["exp_avg_sq_row"])
    assert torch.equal(st2["exp_avg_sq_col"], opt1.state[m1.weight]["exp_avg_sq_col"])
    g2 = torch.randn_like(m1.weight) * 0.1
    m1.weight.grad, m2.weight.grad = g2.clone(), g2.clone()
    opt1.step()
    opt2.step()
    assert torch.equal(m1.weight, m2.weight)


def test_reference_6bit_state_dict_resume():
    """test_quantization.py:1374-1400 on the GPU."""
    _need_gpu()
    from apexw_amd import ApexW
    torch.manual_seed(5)
    p = nn.Parameter(torch.randn(1024, 512, dtype=torch.bfloat16).cuda())
    opt = ApexW([p], lr=1e-3, precision="8bit", factored_v=True, six_bit=True)
    p.grad = torch.randn_like(p) * 0.02
    opt.step()
    st = opt.state[p]
    assert st["is_6bit_m"] and st["is_factored_v"] and st["exp_avg"].dtype == torch.uint8
    tot = sum(v.numel() * v.element_size() for v in st.values() if torch.is_tensor(v))
    assert tot / p.numel() < 0.80
    sd = opt.state_dict()
    p2 = nn.Parameter(p.detach().clone())
    opt2 = ApexW([p2], lr=1e-3, precision="8bit", factored_v=True, six_bit=True)
    opt2.load_state_dict(sd)
    st2 = opt2.state[p2]
    assert st2["is_6bit_m"] and st2["exp_avg"].dtype == torch.uint8 and st2["exp_avg_scales"].dtype == torch.float32
    assert torch.equal(st["exp_avg"], st2["exp_avg"]) and torch.equal(st["exp_avg_scales"], st2["exp_avg_scales"])
    p2.grad = torch.randn_like(p2) * 0.02
    opt2.step()
    torch.cuda.synchronize()
    assert torch.isfinite(p2).all()


def test_reference_compact_factored_threshold_and_convergence():
    """test_quantization.py:1285-1334 on the GPU."""
    _need_gpu()
    from apexw_amd import ApexW
    p_small = nn.Parameter(torch.randn(512, 512, dtype=torch.bfloat16).cuda())
    opt_small = ApexW([p_small], lr=1e-3, betas=(0.9, 0.95), precision="compact", factored_v=True)
    p_small.grad = torch.randn_like(p_small) * 0.01
    opt_small.step()
    assert not opt_small.state[p_small].get("is_factored_v", False)
    p_large = nn.Parameter(torch.randn(1024, 512, dtype=torch.bfloat16).cuda())
    opt_large = ApexW([p_large], lr=1e-3, betas=(0.9, 0.95), precision="compact", factored_v=True)
    p_large.grad = torch.randn_like(p_large) * 0.01
    opt_large.step()
    st = opt_large.state[p_large]
    assert st["is_factored_v"] and st["exp_avg"].dtype == torch.bfloat16
    assert st["exp_avg_sq_row"].numel() == 1024 and st["exp_avg_sq_col"].numel() == 512
    b = sum(v.numel() * v.element_size() for k, v in st.items() if torch.is_tensor(v) and k != "step")
    assert b / p_large.numel() < 2.05

    torch.manual_seed(10)
    x = torch.randn(32, 512, dtype=torch.bfloat16).cuda()
    target = x @ (torch.randn(512, 1024, dtype=torch.bfloat16).cuda() * 0.05)

    def run(use_apex):
        torch.manual_seed(123)
        w = nn.Parameter((torch.randn(512, 1024, dtype=torch.bfloat16) * 0.02).cuda())
        opt = (ApexW([w], lr=1e-2, betas=(0.9, 0.95), precision="compact", factored_v=True) if use_apex
               else torch.optim.AdamW([w], lr=1e-2, betas=(0.9, 0.95)))
        for _ in range(30):
            opt.zero_grad()
            loss = ((x @ w) - target).float().pow(2).mean()
            loss.backward()
            opt.step()
        if use_apex:
            assert opt.state[w]["is_factored_v"]
        return float(loss.item())
    assert run(True) < run(False) * 1.15 + 1e-4


@pytest.mark.parametrize("prec", ["8bit", "compact"])
@pytest.mark.parametrize("shape", [(1024, 512), (128, 4096)])      # 4096 columns: whole-tile statistics
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_factored_with_centralization_and_clip_matches_oracle(prec, shape, dtype):
    """Grad centralization and the global-norm clip prepare the grads of factored
    tensors as of any other (apexw/optimizer.py:204-258), beside an ordinary tensor."""
    _need_gpu()
    from apexw_amd import ApexW
    from oracle.optim import OracleApexW
    gen = torch.Generator().manual_seed(9)
    host = [(torch.randn(shape, generator=gen) * 0.02).to(dtype), (torch.randn(4096, generator=gen) * 0.02).to(dtype)]
    opts = dict(lr=1e-2, weight_decay=0.1, precision=prec, factored_v=True, stochastic_rounding=False,
                grad_centralization=True, clip_grad_norm=0.5)
    gps = [nn.Parameter(h.cuda()) for h in host]
    cps = [nn.Parameter(h.clone()) for h in host]
    gopt, copt = ApexW(gps, **opts), OracleApexW(cps, **opts)
    for step in range(3):
        gs = [(torch.randn(h.shape, generator=gen) * 1e-2).to(dtype) for h in host]
        for gp, cp, g in zip(gps, cps, gs):
            gp.grad, cp.grad = g.cuda(), g.clone()
        prev = cps[0].detach().clone()
        gopt.step()
        copt.step()
        torch.cuda.synchronize()
        st_g, st_c = gopt.state[gps[0]], copt.state[cps[0]]
        # fp32 grads: the clip coefficient (an fp32 norm over 0.5 M elements) and the
        # centralization's row means are reductions in another order than the oracle's:
        # a few fp32 ulps, which every m value and scale carries; where g is close to its
        # row mean the subtraction cancels, so m is held to 1 bf16 ulp plus (1-b1) times
        # the mean's absolute error (~2^-24 * 512 * 1e-2)
        f32 = dtype == torch.float32
        _check(gps[0], cps[0], prev, st_g, st_c, f"{prec} gc+clip step {step}",
               scale_rtol=2e-6 if f32 else 1e-6, m_atol=1e-10 if f32 else None)
        _sync(gps[0], cps[0], st_g, st_c)


@pytest.mark.parametrize("six", [False, True])
def test_factored_m_code_sr_unbiased(six):
    """First step from zero state: m = (1 - b1) g exactly, so the codes must be
    floor or ceil of m / scale, with a mean rounding error within 3 standard
    errors of zero (10.5 M elements, one row per 2048-element unit)."""
    _need_gpu()
    from apexw_amd import ApexW
    torch.manual_seed(2)
    shape = (5120, 2048)
    g = (torch.randn(shape) * 1e-3).bfloat16()
    p = nn.Parameter(torch.zeros(shape, dtype=torch.bfloat16, device="cuda"))
    p.grad = g.cuda()
    opt = ApexW([p], lr=1e-3, weight_decay=0.0, precision="8bit", factored_v=True, six_bit=six,
                stochastic_rounding=True)
    opt.step()
    st = opt.state[p]
    assert st["is_factored_v"] and bool(st.get("is_6bit_m", False)) == six
    m_exact = torch.tensor(np.float32(1 - 0.9)) * g.float().reshape(-1)   # lerp from zero: fma(w, g - 0, 0)
    ms = st["exp_avg_scales"].cpu().reshape(-1)
    codes = (_codes6(st["exp_avg"].cpu()) - 31).float() if six else st["exp_avg"].cpu().reshape(-1).float()
    codes = codes[:m_exact.numel()]
    x = (m_exact.view(ms.numel(), -1) / ms[:, None]).reshape(-1)
    lo = torch.floor(x)
    assert bool(((codes == lo) | (codes == lo + 1)).all()), "SR code is not floor or ceil of m / scale"
    err = codes - x
    mean, se = float(err.double().mean()), float(err.double().std()) / err.numel() ** 0.5
    assert abs(mean) < 3 * se, f"factored m SR: mean {mean:.3e} vs 3*se {3 * se:.3e}"


@pytest.mark.parametrize("prec", ["8bit", "compact"])
def test_all_factored_group_with_uneven_step_counts(prec):
    """A group of factored tensors only, whose second parameter first receives a
    grad on step 2: its step count then trails the first one's, so the step runs
    one factored launch per count and no step-kernel launch at all."""
    _need_gpu()
    from apexw_amd import ApexW
    from oracle.optim import OracleApexW
    print(f"all-factored group {prec}", flush=True)
    gen = torch.Generator().manual_seed(11)
    shapes = [(1024, 512), (512, 1024)]
    host = [(torch.randn(s, generator=gen) * 0.02).bfloat16() for s in shapes]
    opts = dict(lr=1e-2, weight_decay=0.1, precision=prec, factored_v=True, stochastic_rounding=False)
    gps = [nn.Parameter(h.cuda()) for h in host]
    cps = [nn.Parameter(h.clone()) for h in host]
    gopt, copt = ApexW(gps, **opts), OracleApexW(cps, **opts)
    for step in range(4):
        active = [0] if step == 0 else [0, 1]
        for i in range(2):
            g = (torch.randn(shapes[i], generator=gen) * 1e-3).bfloat16() if i in active else None
            gps[i].grad = None if g is None else g.cuda()
            cps[i].grad = None if g is None else g.clone()
        prevs = [c.detach().clone() for c in cps]
        gopt.step()
        copt.step()
        torch.cuda.synchronize()
        for i in active:
            st_g, st_c = gopt.state[gps[i]], copt.state[cps[i]]
            assert st_g["is_factored_v"] and float(st_g["step"]) == float(st_c["step"])
            _check(gps[i], cps[i], prevs[i], st_g, st_c, f"{prec} tensor {i} step {step}")
            _sync(gps[i], cps[i], st_g, st_c)
    assert float(gopt.state[gps[0]]["step"]) == 4.0 and float(gopt.state[gps[1]]["step"]) == 3.0
