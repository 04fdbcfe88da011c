"""The reference-side binding shown in INTEGRATION.md, executed as written.

``tests/integration_binding.py`` loads the ``apexw/rocm_extension.py`` code
block of INTEGRATION.md; its ``step_fused`` / ``step_fused_8bit`` (the
reference's ``apexw.cuda_extension`` signatures) then step state laid out as
the reference lays it out, and the results are held to the CPU oracle at the
parity bars of test_gpu_configs.py: the compact call against the cold foreach
step (``_multi_tensor_step``), the 8-bit call against ``_step_ultra`` per
tensor (chunked order above 262,144 elements, generic below; every tensor
generic with cautious=True), SR off.
"""

import pytest
import torch

from integration_binding import load_binding
from oracle import compact as OC
from oracle import layout as OL
from oracle import q8 as OQ
from test_gpu_configs import _cmp, _cmp_p

pytestmark = pytest.mark.gpu

KW = dict(lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.1)


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")


def _group(prec, n):
    return dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.1, precision=prec, stochastic_rounding=False,
                block_size=None, int4_m=None, force_compact_v=False, factored_v=False, six_bit=False,
                params=[None] * n)


def _setup(shapes, dtype, prec, seed):
    gen = torch.Generator().manual_seed(seed)
    ps = [(torch.randn(s, generator=gen) * 0.02).to(dtype) for s in shapes]
    gs = [(torch.randn(s, generator=gen) * 1e-3).to(dtype) for s in shapes]
    grp = _group(prec, len(shapes))
    sts = [OL.init_state(p, grp, len(shapes), False) for p in ps]
    return ps, gs, sts


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_binding_step_fused_matches_oracle(dtype):
    _need_gpu()
    print(f"binding step_fused {dtype}", flush=True)
    rx = load_binding()
    shapes = [(256, 128), (16384,), (300,), (64, 33), (40000,), (8, 2048), (5,), (1000,)]
    ps, gs, sts = _setup(shapes, dtype, "compact", 5)
    for step in (1, 2):
        dp = [p.cuda() for p in ps]
        dm = [st["exp_avg"].cuda() for st in sts]
        dv = [st["exp_avg_sq"].cuda() for st in sts]
        ok = rx.step_fused(dp, [g.cuda() for g in gs], dm, dv, step=step, decay_norm_only=True, stochastic=False,
                           **KW)
        assert ok
        prev = [p.clone() for p in ps]
        # the oracle's cold foreach step, per (quad) subgroup, on the CPU copies
        for quad in (False, True):
            idx = [i for i, st in enumerate(sts) if bool(st.get("is_quad_v", False)) == quad]
            if idx:
                OC.compact_subgroup_step([ps[i] for i in idx], [gs[i] for i in idx],
                                         [sts[i]["exp_avg"] for i in idx], [sts[i]["exp_avg_sq"] for i in idx],
                                         lr=KW["lr"], beta1=KW["beta1"], beta2=KW["beta2"], eps=KW["eps"],
                                         weight_decay=KW["weight_decay"], decay_norm_only=True, step=step,
                                         is_quad=quad, stochastic=False)
        torch.cuda.synchronize()
        for i in range(len(shapes)):
            what = f"step {step} tensor {i} {shapes[i]}"
            v16 = sts[i]["exp_avg_sq"].dtype == torch.bfloat16
            _cmp_p(dp[i], ps[i], prev[i], f"{what} p", 2.0 ** -7 if v16 else 2.0 ** -22)
            _cmp(dm[i], sts[i]["exp_avg"], f"{what} m")
            _cmp(dv[i], sts[i]["exp_avg_sq"], f"{what} v", floor=1e-12)
            ps[i] = dp[i].cpu()
            sts[i]["exp_avg"], sts[i]["exp_avg_sq"] = dm[i].cpu(), dv[i].cpu()
        gs = [g * 0.7 for g in gs]


@pytest.mark.parametrize("dtype,cautious", [(torch.bfloat16, False), (torch.float32, False), (torch.bfloat16, True),
                                            (torch.float32, True)])
def test_binding_step_fused_8bit_matches_oracle(dtype, cautious):
    _need_gpu()
    print(f"binding step_fused_8bit {dtype} cautious={cautious}", flush=True)
    rx = load_binding()
    shapes = [(512, 1024), (256, 256), (4096,), (3000,), (100, 300), (70,)]
    ps, gs, sts = _setup(shapes, dtype, "8bit", 6)
    keys = ("exp_avg", "exp_avg_scales", "exp_avg_sq", "exp_avg_sq_scales")
    dp = [p.cuda() for p in ps]
    dst = [{k: st[k].cuda() for k in keys} for st in sts]
    ok = rx.step_fused_8bit(dp, [g.cuda() for g in gs], [d["exp_avg"] for d in dst],
                            [d["exp_avg_scales"] for d in dst], [d["exp_avg_sq"] for d in dst],
                            [d["exp_avg_sq_scales"] for d in dst], [st["block_size_8bit"] for st in sts],
                            step=1, decay_norm_only=True, stochastic=False, cautious=cautious, **KW)
    assert ok
    prev = [p.clone() for p in ps]
    for p, g, st in zip(ps, gs, sts):
        OQ.q8_param_step(p, g, st, lr=KW["lr"], beta1=KW["beta1"], beta2=KW["beta2"], eps=KW["eps"],
                         weight_decay=KW["weight_decay"], decay_norm_only=True, step=1, cautious=cautious)
    torch.cuda.synchronize()
    for i in range(len(shapes)):
        what = f"tensor {i} {shapes[i]}"
        generic = dtype == torch.bfloat16 and (ps[i].numel() <= OQ.CHUNK or cautious)
        _cmp_p(dp[i], ps[i], prev[i], f"{what} p", 2.0 ** -7 if generic else 2.0 ** -22)
        for k in keys:
            kind = "#nf4" if (k == "exp_avg" and sts[i].get("is_4bit_m")) else ""
            _cmp(dst[i][k], sts[i][k], f"{what} {k}{kind}", floor=0.0 if k.endswith("scales") else 1e-9)


def test_binding_refuses_without_writing():
    """A dtype the kernels do not take: False, and the tensors are untouched (the
    caller's torch path then runs)."""
    _need_gpu()
    rx = load_binding()
    p = torch.zeros(4096, dtype=torch.float16, device="cuda")
    m = torch.zeros(4096, dtype=torch.bfloat16, device="cuda")
    v = torch.zeros(4096, dtype=torch.bfloat16, device="cuda")
    g = torch.ones_like(p)
    assert not rx.step_fused([p], [g], [m], [v], stochastic=False, **KW)
    torch.cuda.synchronize()
    assert not bool(p.any()) and not bool(m.any()) and not bool(v.any())
