"""State conversion between precision modes on the GPU (apexw_state_decode /
apexw_state_encode, ApexW.set_precision) against the CPU oracle (oracle/convert.py).

Bars: decode is bit for bit (one fp32 product per element); encode gives the
same NF4 / INT8 codes and block scales bit for bit (the same fp32 divisions
and comparisons), log-uint8 codes within 1 (log2 on the GPU against torch's
CPU log2 can land on the other side of a half-integer), dense buffers bit for
bit (one rounding to nearest-even).  After set_precision, one step on the GPU
matches the oracle's step from the oracle-converted state at the parity bars
of test_gpu_parity.py (a cold step of the new mode from non-zero state).
"""

import ctypes

import pytest
import torch
import torch.nn as nn

from test_gpu_parity import _cmp_tensor

pytestmark = pytest.mark.gpu


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")


def _group(prec, **kw):
    return dict(dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.1, precision=prec,
                     stochastic_rounding=False, block_size=None, int4_m=None, force_compact_v=False,
                     factored_v=False, six_bit=False), **kw)


def _fresh(p, prec, nparams=10):
    from oracle import layout as Lay
    return Lay.init_state(p, _group(prec), nparams, False)


def _to(st, dev):
    return {k: (v.to(dev) if torch.is_tensor(v) and k != "step" else v) for k, v in st.items()}


SHAPES = [((512, 256), "8bit"), ((16390,), "8bit"), ((300,), "8bit"), ((40, 70), "8bit"), ((6000,), "8bit"),
          ((128, 256), "compact"), ((768,), "compact")]


@pytest.mark.parametrize("shape,prec", SHAPES, ids=[f"{s}-{p}" for s, p in SHAPES])
def test_decode_encode_match_oracle(shape, prec):
    _need_gpu()
    from apexw_amd import _lib as L
    from apexw_amd import convert as CV
    from oracle import convert as C
    print(f"convert {shape} {prec}", flush=True)
    p = torch.zeros(shape, dtype=torch.bfloat16)
    n = p.numel()
    g = torch.Generator().manual_seed(n)
    m = torch.randn(n, generator=g) * 1e-3
    v = (torch.randn(n, generator=g) * 1e-3) ** 2
    v[::97] = 0.0
    ref = C.encode(_fresh(p, prec), m, v)
    got = _to(_fresh(p, prec), "cuda")
    lib = L.load()
    stream = torch.cuda.current_stream().cuda_stream
    md, vd = m.cuda(), v.cuda()
    L.check(lib.apexw_state_encode(ctypes.byref(CV._layout(got, n)), md.data_ptr(), vd.data_ptr(), stream), "encode")
    torch.cuda.synchronize()
    for k in ("exp_avg", "exp_avg_scales", "exp_avg_sq_scales"):
        if k in ref:
            assert torch.equal(got[k].cpu(), ref[k]), k
    a, b = got["exp_avg_sq"].cpu(), ref["exp_avg_sq"]
    if a.dtype == torch.uint8:
        assert int((a.int() - b.int()).abs().max()) <= 1
    else:
        assert torch.equal(a, b)
    # decode the oracle's state (copied to the GPU) and compare with the oracle's decode
    src = _to(ref, "cuda")
    m32 = torch.empty(n, device="cuda")
    v32 = torch.empty(n, device="cuda")
    L.check(lib.apexw_state_decode(ctypes.byref(CV._layout(src, n)), m32.data_ptr(), v32.data_ptr(), stream), "decode")
    rm, rv = C.decode(ref, n)
    torch.cuda.synchronize()
    assert torch.equal(m32.cpu(), rm)
    assert torch.equal(v32.cpu(), rv)


# fp16 parameters with beta2 = 0.99: the compact v is fp16 and holds the moment times
# its dynamic scale (1024), which the conversion divides out or multiplies in
SWITCH = [("8bit", "compact", torch.bfloat16), ("compact", "8bit", torch.bfloat16),
          ("8bit", "compact", torch.float16), ("compact", "8bit", torch.float16)]


@pytest.mark.parametrize("src,dst,dtype", SWITCH, ids=[f"{a}-{b}-{str(d)[6:]}" for a, b, d in SWITCH])
def test_checkpoint_resumes_in_other_precision(src, dst, dtype):
    """Train 3 steps in one mode, save, load into an optimizer, switch it to the
    other mode with set_precision, and step: the converted state equals the
    oracle's conversion, and the step equals the oracle's step from it."""
    _need_gpu()
    from apexw_amd import ApexW
    from oracle import convert as C
    from oracle import layout as Lay
    from oracle.optim import OracleApexW
    print(f"resume {src} -> {dst} {dtype}", flush=True)
    shapes = [(512, 256), (16384,), (4096,), (300,), (64, 33), (40,), (128, 130), (96, 256)]
    gen = torch.Generator().manual_seed(99)
    host = [(torch.randn(s, generator=gen) * 0.02).to(dtype) for s in shapes]
    kw = dict(lr=1e-3, weight_decay=0.1, adamw_compat=True, stochastic_rounding=False)
    if dtype == torch.float16:
        del kw["adamw_compat"]        # which sets beta2 = 0.999, and so an fp32 v
        kw["betas"] = (0.9, 0.99)
    ps = [nn.Parameter(h.cuda()) for h in host]
    opt = ApexW(ps, precision=src, **kw)
    for _ in range(3):
        for p in ps:
            p.grad = (torch.randn(p.shape, generator=gen) * 1e-3).to(dtype).cuda()
        opt.step()
    sd = opt.state_dict()
    ps2 = [nn.Parameter(p.detach().clone()) for p in ps]
    opt2 = ApexW(ps2, precision=dst, **kw)
    opt2.load_state_dict(sd)
    opt2.set_precision(dst)
    assert opt2.param_groups[0]["precision"] == dst
    # the oracle converts the saved state with its own decode / encode
    cps = [nn.Parameter(p.detach().cpu().clone()) for p in ps2]
    copt = OracleApexW(cps, precision=dst, **kw)
    grp = copt.group
    scaled = 0
    for p0, p, cp in zip(ps, ps2, cps):
        saved = {k: (v.detach().cpu().clone() if torch.is_tensor(v) else v) for k, v in opt.state[p0].items()}
        mf, vf = C.decode(saved, p.numel())
        tgt = Lay.init_state(cp, grp, len(cps), False)
        C.encode(tgt, mf, vf)
        tgt["step"] = saved["step"].clone()
        copt.state[cp] = tgt
        gs = opt2.state[p]
        assert bool(gs.get("is_8bit", False)) == bool(tgt.get("is_8bit", False))
        for k in ("exp_avg", "exp_avg_sq", "exp_avg_scales", "exp_avg_sq_scales"):
            if k in tgt:
                a, b = gs[k].cpu(), tgt[k]
                if k == "exp_avg_sq" and tgt[k].dtype == torch.float16:
                    assert gs["scale_v"] == tgt["scale_v"] == 1024.0
                    scaled += 1
                if a.dtype == torch.uint8 and k == "exp_avg_sq":
                    assert int((a.int() - b.int()).abs().max()) <= 1, k
                else:
                    assert torch.equal(a, b), k
                gs[k].copy_(b.to(gs[k].device))   # start the step from the oracle's codes
        assert float(gs["step"]) == 3.0
    if dtype == torch.float16:
        src_scaled = sum(opt.state[p0]["exp_avg_sq"].dtype == torch.float16 for p0 in ps)
        assert (scaled if dst == "compact" else src_scaled) > 0, "no fp16 v with a dynamic scale on either side"
    for p, cp in zip(ps2, cps):
        g = (torch.randn(p.shape, generator=gen) * 1e-3).to(dtype)
        p.grad, cp.grad = g.cuda(), g.clone()
    opt2.step()
    copt.step()
    torch.cuda.synchronize()
    for i, (p, cp) in enumerate(zip(ps2, cps)):
        _cmp_tensor(p.data, _as_np(cp.data), f"p_{i}")
        gs, cs = opt2.state[p], copt.state[cp]
        for k in ("exp_avg", "exp_avg_sq"):
            _cmp_tensor(gs[k], _as_np(cs[k]), f"{'m' if k == 'exp_avg' else 'v'}_{i}")


def _as_np(t):
    import numpy as np
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()
