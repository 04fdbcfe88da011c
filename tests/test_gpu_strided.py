"""GPU: dense non-contiguous parameters (channels_last convolution weights, transposed
matrices) in the compact-kernel precisions.

The step is element by element, so it walks the parameter, its grad and its state in
the parameter's memory layout; the state is laid out like the parameter (the
reference's zeros_like(p, memory_format=torch.preserve_format)).  Against the CPU
oracle (torch ops on the same strided tensors) at the bars of test_gpu_edge.py:

* channels_last and transposed parameters, bf16 and fp32, with the clip, amsgrad and
  a grad handed over contiguous (copied into the parameter's layout);
* refusals before any tensor moves: a non-dense parameter (a strided slice), a
  non-contiguous tensor with quad v (the reference's `.view(-1, 4)` fails on it too),
  grad centralization, and the 8-bit precision.
"""

import pytest
import torch

from test_gpu_edge import _compare, _need_gpu

pytestmark = pytest.mark.gpu


def _layouts(dtype, seed):
    """Host tensors in their layouts: two channels_last conv weights, a transposed matrix,
    a contiguous vector."""
    g = torch.Generator().manual_seed(seed)
    w1 = (torch.randn(32, 16, 3, 3, generator=g) * 0.02).to(dtype).to(memory_format=torch.channels_last)
    w2 = (torch.randn(64, 32, 3, 3, generator=g) * 0.02).to(dtype).to(memory_format=torch.channels_last)
    t = (torch.randn(96, 40, generator=g) * 0.02).to(dtype).t()
    b = (torch.randn(300, generator=g) * 0.02).to(dtype)
    return [w1, w2, t, b]


def _clone_layout(h, device):
    out = torch.empty_strided(h.shape, h.stride(), dtype=h.dtype, device=device)
    out.copy_(h)
    return out


RUNS = [("bf16 compact", torch.bfloat16, dict(precision="compact")),
        ("bf16 compact foreach clip", torch.bfloat16, dict(precision="compact", fused=False, clip_grad_norm=1e-3)),
        ("fp32 compact amsgrad", torch.float32, dict(precision="compact", amsgrad=True)),
        ("bf16 full", torch.bfloat16, dict(precision="full"))]


@pytest.mark.parametrize("name,dtype,kw", RUNS, ids=[r[0] for r in RUNS])
def test_strided_parameters_match_oracle(name, dtype, kw):
    _need_gpu()
    from apexw_amd import ApexW
    from oracle.optim import OracleApexW
    print(f"strided {name}", flush=True)
    kw = dict(dict(lr=1e-3, weight_decay=0.1, stochastic_rounding=False), **kw)
    host = _layouts(dtype, 81)
    gps = [torch.nn.Parameter(_clone_layout(h, "cuda")) for h in host]
    cps = [torch.nn.Parameter(_clone_layout(h, "cpu")) for h in host]
    assert not gps[0].is_contiguous() and gps[0].stride() == cps[0].stride()
    gopt, copt = ApexW(gps, **kw), OracleApexW(cps, **kw)
    for step in range(4):
        for i, (gp, cp) in enumerate(zip(gps, cps)):
            g = torch.empty_like(cp.detach())
            g.copy_((torch.randn(cp.shape, generator=torch.Generator().manual_seed(900 + 10 * step + i)) * 1e-3)
                    .to(dtype))
            cp.grad = g.clone()
            # step 2 hands the GPU a contiguous grad: copied into the parameter's layout
            gp.grad = g.contiguous().cuda() if step == 2 else _clone_layout(g, "cuda")
        gopt.step()
        copt.step()
    torch.cuda.synchronize()
    for gp in gps:
        st = gopt.state[gp]
        assert st["exp_avg"].stride() == gp.stride()
    _compare(gps, cps, gopt, copt, f"strided {name}")


@pytest.mark.parametrize("case", ["slice", "quad", "centralization", "8bit"])
def test_strided_refusals(case):
    _need_gpu()
    from apexw_amd import ApexW
    print(f"strided refusal {case}", flush=True)
    kw = dict(lr=1e-3, stochastic_rounding=False)
    if case == "slice":
        ps = [torch.nn.Parameter(torch.randn(64, 64, device="cuda")[:, ::2])]
    elif case == "quad":
        # 9 tensors: the transposed 256 x 256 matrix gets quad v
        ps = [torch.nn.Parameter(torch.randn(256, 256, device="cuda", dtype=torch.bfloat16).t())]
        ps += [torch.nn.Parameter(torch.randn(32, 32, device="cuda", dtype=torch.bfloat16)) for _ in range(8)]
    elif case == "centralization":
        ps = [torch.nn.Parameter(torch.randn(32, 16, 3, 3, device="cuda").to(memory_format=torch.channels_last))]
        kw["grad_centralization"] = True
    else:
        ps = [torch.nn.Parameter(torch.randn(256, 64, device="cuda", dtype=torch.bfloat16).t())]
        kw["precision"] = "8bit"
    for p in ps:
        p.grad = torch.empty_like(p).normal_(0, 1e-3)
    opt = ApexW(ps, **kw)
    before = [p.detach().clone() for p in ps]
    with pytest.raises(NotImplementedError):
        opt.step()
    torch.cuda.synchronize()
    assert all(torch.equal(a, b) for a, b in zip(before, ps))
