"""GPU: AMP grad-scale hand-off (torch.amp.GradScaler with
``_step_supports_amp_scaling``): the step kernels unscale the grads.

* kernels vs the CPU oracle with the same ``grad_scale`` on the same scaled
  grads, every path (the parity bars of test_gpu_parity.py, SR off);
* with the global-norm clip: the AMP step equals, bit for bit, the kernels'
  own step on the unscaled grads.  (Against the oracle the clip coefficient, a
  global sum of squares, differs from torch's CPU reduction order by a few
  fp32 ulps; with fp32 grads and bf16 m that flips occasional m roundings, so
  the oracle comparison of clipped fp32 steps is not bit-level);
* a real GradScaler loop equals, bit for bit, the same loop without scaling
  (power-of-two scales are exact in fp32);
* ApexMuon: a power-of-two grad scale gives the step of the unscaled grads.
"""

import pytest
import torch

from test_gpu_edge import _compare

pytestmark = pytest.mark.gpu

SCALE = 1024.0


@pytest.fixture(autouse=True)
def _fresh_fp16_flag(monkeypatch):
    """An 8-bit ApexW over fp16 parameters sets a process-wide flag that clamps
    GradScaler's scale to 256 (as the reference does); tests here start without it,
    whichever tests ran before them in the process."""
    from apexw_amd import runtime as R
    monkeypatch.setattr(R, "fp16_active", False)


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")


CASES = [
    ("compact native bf16", [(64,), (32, 16)], torch.bfloat16, dict(precision="compact")),
    ("compact foreach bf16 quad", [(256, 128), (64,)], torch.bfloat16, dict(precision="compact")),
    ("compact foreach fp32", [(256, 128), (1000,)], torch.float32, dict(precision="compact", adamw_compat=True)),
    ("8bit chunked + generic", [(1024, 512), (4096,)], torch.bfloat16, dict(precision="8bit")),
    ("8bit fp32", [(2048, 256), (100,)], torch.float32, dict(precision="8bit")),
    # maximize: the negative unscale factor carries both (GradScaler read on the host)
    ("8bit maximize", [(1024, 512), (4096,), (40,)], torch.bfloat16, dict(precision="8bit", maximize=True)),
    ("8bit cautious", [(1024, 512), (4096,), (40,)], torch.bfloat16, dict(precision="8bit", cautious=True)),
    ("compact maximize", [(256, 128), (1000,), (64,)], torch.bfloat16, dict(precision="compact", maximize=True)),
    # cautious: the count pass reads the device scalars too (8 tensors: quad v for the large ones)
    ("compact cautious", [(256, 128), (20000,)] + [(64,)] * 6, torch.bfloat16,
     dict(precision="compact", cautious=True)),
    # amsgrad: the running max in the native fused order and in the foreach one
    ("compact amsgrad native", [(256, 128), (1000,), (64,)], torch.bfloat16, dict(precision="compact", amsgrad=True)),
    ("compact amsgrad foreach fp32", [(256, 128), (1000,)], torch.float32,
     dict(precision="compact", amsgrad=True)),
]


@pytest.mark.parametrize("name,shapes,dtype,kw", CASES, ids=[c[0] for c in CASES])
def test_grad_scale_matches_oracle(name, shapes, dtype, kw):
    _need_gpu()
    from apexw_amd import ApexW
    from oracle.optim import OracleApexW
    print(f"amp {name}", flush=True)
    kw = dict(kw, lr=1e-3, weight_decay=0.1, stochastic_rounding=False)
    gen = torch.Generator().manual_seed(3)
    host = [(torch.randn(s, generator=gen) * 0.02).to(dtype) for s in shapes]
    gps = [torch.nn.Parameter(h.cuda()) for h in host]
    cps = [torch.nn.Parameter(h.clone()) for h in host]
    gopt, copt = ApexW(gps, **kw), OracleApexW(cps, **kw)
    ggen = torch.Generator().manual_seed(4)
    for _ in range(4):
        for gp, cp in zip(gps, cps):
            g = (torch.randn(gp.shape, generator=ggen) * 1e-3 * SCALE).to(dtype)
            gp.grad, cp.grad = g.cuda(), g.clone()
        gopt.grad_scale, gopt.found_inf = torch.tensor(SCALE, device="cuda"), torch.zeros((), device="cuda")
        copt.grad_scale, copt.found_inf = torch.tensor(SCALE), torch.tensor(0.0)
        gopt.step()
        copt.step()
    torch.cuda.synchronize()
    _compare(gps, cps, gopt, copt, name)


@pytest.mark.parametrize("name,shapes,dtype,kw", CASES, ids=[c[0] for c in CASES])
def test_grad_scale_with_clip_equals_unscaled_step(name, shapes, dtype, kw):
    """The clip must see the unscaled norm: a 2^10-scaled step with grad_scale
    2^10 is bit-identical to the step on the unscaled grads."""
    _need_gpu()
    from apexw_amd import ApexW
    print(f"amp clip {name}", flush=True)
    kw = dict(kw, lr=1e-3, weight_decay=0.1, clip_grad_norm=1e-3, stochastic_rounding=False)
    gen = torch.Generator().manual_seed(3)
    host = [(torch.randn(s, generator=gen) * 0.02).to(dtype) for s in shapes]
    pa = [torch.nn.Parameter(h.cuda()) for h in host]
    pb = [torch.nn.Parameter(h.cuda()) for h in host]
    oa, ob = ApexW(pa, **kw), ApexW(pb, **kw)
    ggen = torch.Generator().manual_seed(4)
    for _ in range(4):
        for a, b in zip(pa, pb):
            g = (torch.randn(a.shape, generator=ggen) * 1e-3).to(dtype)
            a.grad, b.grad = (g * SCALE).cuda(), g.cuda()
        oa.grad_scale, oa.found_inf = torch.tensor(SCALE, device="cuda"), torch.zeros((), device="cuda")
        oa.step()
        ob.step()
    torch.cuda.synchronize()
    for a, b in zip(pa, pb):
        assert torch.equal(a, b), name
        for k, v in oa.state[a].items():
            if torch.is_tensor(v):
                assert torch.equal(v, ob.state[b][k]), (name, k)


@pytest.mark.parametrize("precision,extra", [("8bit", {}), ("8bit", dict(clip_grad_norm=1e-3)),
                                             ("8bit", dict(grad_centralization=True, clip_grad_norm=1e-3)),
                                             ("ultra", dict(threshold=4096, clip_grad_norm=1e-3)),
                                             ("compact", {}), ("compact", dict(clip_grad_norm=1e-3)),
                                             ("compact", dict(grad_centralization=True, clip_grad_norm=1e-3)),
                                             ("full", dict(clip_grad_norm=1e-3)), ("auto", dict(threshold=4096))],
                         ids=["8bit", "8bit-clip", "8bit-gc-clip", "ultra-clip", "compact", "compact-clip",
                              "compact-gc-clip", "full-clip", "auto"])
def test_maximize_equals_negated_grads(precision, extra):
    """maximize=True on grads g steps exactly as maximize=False on -g (the
    reference negates the grads after nan_to_num, and negation commutes with the
    clip, centralization and AMP's unscale): bit-identical parameters and states,
    with a GradScaler scale of 2^10 on every step.  maximize leaves the native fused
    order of a compact group whose states all match their parameters (as the
    reference's plan does), so the plain run there takes the foreach order too
    (fused=False)."""
    _need_gpu()
    from apexw_amd import ApexW
    print(f"maximize {precision} {extra}", flush=True)
    kw = dict(lr=1e-3, weight_decay=0.1, precision=precision, stochastic_rounding=False, **extra)
    gen = torch.Generator().manual_seed(5)
    shapes = [(1024, 512), (256, 128), (4096,), (40,)]
    host = [(torch.randn(s, generator=gen) * 0.02).bfloat16() for s in shapes]
    pa = [torch.nn.Parameter(h.cuda()) for h in host]
    pb = [torch.nn.Parameter(h.cuda()) for h in host]
    plain = dict(kw, fused=False) if precision in ("compact", "full", "auto") else kw
    oa, ob = ApexW(pa, maximize=True, **kw), ApexW(pb, **plain)
    for _ in range(3):
        for a, b in zip(pa, pb):
            g = (torch.randn(a.shape, generator=gen) * 1e-3 * SCALE).bfloat16()
            a.grad, b.grad = g.cuda(), (-g).cuda()
        for o in (oa, ob):
            o.grad_scale, o.found_inf = torch.tensor(SCALE, device="cuda"), torch.zeros((), device="cuda")
            o.step()
    torch.cuda.synchronize()
    for a, b in zip(pa, pb):
        assert torch.equal(a, b)
        for k, v in oa.state[a].items():
            if torch.is_tensor(v):
                assert torch.equal(v, ob.state[b][k]), k


def _model(seed):
    torch.manual_seed(seed)
    return torch.nn.Sequential(torch.nn.Linear(64, 128), torch.nn.GELU(), torch.nn.Linear(128, 32)).cuda()


@pytest.mark.parametrize("precision", ["compact", "8bit"])
def test_grad_scaler_loop_equals_unscaled_loop(precision):
    _need_gpu()
    from apexw_amd import ApexW
    print(f"grad scaler loop {precision}", flush=True)
    ma, mb = _model(0), _model(0)
    kw = dict(lr=1e-3, weight_decay=0.1, precision=precision, stochastic_rounding=False)
    oa, ob = ApexW(ma.parameters(), **kw), ApexW(mb.parameters(), **kw)
    scaler = torch.amp.GradScaler("cuda", init_scale=2.0 ** 12)
    gen = torch.Generator(device="cuda").manual_seed(1)
    for _ in range(5):
        x = torch.randn(16, 64, device="cuda", generator=gen)
        y = torch.randn(16, 32, device="cuda", generator=gen)
        oa.zero_grad()
        scaler.scale(torch.nn.functional.mse_loss(ma(x), y)).backward()
        scaler.step(oa)
        scaler.update()
        ob.zero_grad()
        torch.nn.functional.mse_loss(mb(x), y).backward()
        ob.step()
    torch.cuda.synchronize()
    for pa, pb in zip(ma.parameters(), mb.parameters()):
        assert torch.equal(pa, pb)


def test_grad_scaler_skips_inf_step():
    _need_gpu()
    from apexw_amd import ApexW
    m = _model(2)
    opt = ApexW(m.parameters(), lr=1e-3)
    scaler = torch.amp.GradScaler("cuda", init_scale=2.0 ** 12)
    x = torch.randn(4, 64, device="cuda")
    scaler.scale(m(x).sum()).backward()
    scaler.step(opt)
    scaler.update()
    before = [p.detach().clone() for p in m.parameters()]
    opt.zero_grad()
    scaler.scale(m(x).sum()).backward()
    next(m.parameters()).grad[0, 0] = float("inf")
    scaler.step(opt)                     # found_inf -> skipped
    scaler.update()
    torch.cuda.synchronize()
    for p, b in zip(m.parameters(), before):
        assert torch.equal(p.detach(), b)
    assert scaler.get_scale() == 2.0 ** 11


def test_muon_grad_scale_equals_unscaled():
    _need_gpu()
    from apexw_amd.muon import ApexMuon
    gen = torch.Generator().manual_seed(9)
    host = [torch.randn(s, generator=gen) * 0.02 for s in [(256, 384), (384, 256)]]
    pa = [torch.nn.Parameter(h.cuda()) for h in host]
    pb = [torch.nn.Parameter(h.cuda()) for h in host]
    oa = ApexMuon(pa, lr=0.02, weight_decay=0.1, scale_mode="rms_matched")
    ob = ApexMuon(pb, lr=0.02, weight_decay=0.1, scale_mode="rms_matched")
    for _ in range(2):
        for a, b in zip(pa, pb):
            g = torch.randn(a.shape, generator=gen) * 1e-3
            a.grad, b.grad = (g * SCALE).cuda(), g.cuda()
        oa.grad_scale, oa.found_inf = torch.tensor(SCALE, device="cuda"), torch.zeros((), device="cuda")
        oa.step()
        ob.step()
    torch.cuda.synchronize()
    for a, b in zip(pa, pb):
        assert torch.equal(a, b)
        assert torch.equal(oa.state[a]["momentum"], ob.state[b]["momentum"])


def test_grad_scaler_step_reads_nothing_on_the_host():
    """Once a plan has taken its first step, a GradScaler step launches without a
    host synchronisation: found_inf and the scale are read by the kernels
    (torch's sync debug mode raises on any synchronising torch call)."""
    _need_gpu()
    from apexw_amd import ApexW
    for precision, clip, gc in (("compact", None, False), ("8bit", None, False), ("compact", 1.0, True)):
        print(f"amp without host reads: {precision} clip={clip} gc={gc}", flush=True)
        m = _model(3)
        opt = ApexW(m.parameters(), lr=1e-3, precision=precision, clip_grad_norm=clip, grad_centralization=gc)
        scaler = torch.amp.GradScaler("cuda", init_scale=2.0 ** 12)
        x = torch.randn(8, 64, device="cuda")
        for it in range(3):
            opt.zero_grad()
            scaler.scale(m(x).square().mean()).backward()
            if it > 0:
                torch.cuda.set_sync_debug_mode("error")
            try:
                scaler.step(opt)
            finally:
                torch.cuda.set_sync_debug_mode("default")
            scaler.update()
        torch.cuda.synchronize()
        assert all(int(opt.state[p]["step"]) == 3 for p in m.parameters())


AMP_PAIR_CASES = [
    ("compact", {}, 0),
    ("8bit", {}, 0),
    # a centralized 8-bit group unscales a prepared copy of its grads: it must read
    # found_inf on the host, or an inf step would be applied to the sanitized grads
    ("8bit", dict(grad_centralization=True), 0),
    ("ultra", dict(threshold=4096), 0),
    # step counts near 5e4: the device's bias corrections (double pow) against the host's
    ("8bit", {}, 49_990),
    ("compact", {}, 49_990),
]


def _restep(opt, start):
    """Set every parameter's step counter to ``start`` through the state mapping,
    as a resumed checkpoint would."""
    sd = opt.state_dict()
    for st in sd["state"].values():
        st["step"] = torch.tensor(float(start))
    opt.load_state_dict(sd)


@pytest.mark.parametrize("precision,extra,start", AMP_PAIR_CASES,
                         ids=[f"{c[0]}{'-gc' if c[1].get('grad_centralization') else ''}-from{c[2]}"
                              for c in AMP_PAIR_CASES])
def test_device_amp_equals_host_amp_with_skipped_steps(precision, extra, start):
    """The same sequence of scaled steps, some with found_inf, through the device
    path (GradScaler's CUDA tensors) and the host path (the same values as CPU
    tensors, read on the host like the reference): identical parameters and
    state, and step counters that count only the steps taken (exact after
    state_dict(), which subtracts the skips the device saw).  ``start``: the
    step counters are first set to it (one unscaled step, then a state_dict
    round trip), so the bias corrections come from large step counts."""
    _need_gpu()
    from apexw_amd import ApexW
    print(f"device vs host amp {precision} {extra} from step {start}", flush=True)
    gen = torch.Generator().manual_seed(21)
    shapes = [(256, 128), (300,), (64, 33), (16384,), (512, 64)]
    host = [(torch.randn(s, generator=gen) * 0.02).bfloat16() for s in shapes]
    pa = [torch.nn.Parameter(h.cuda()) for h in host]
    pb = [torch.nn.Parameter(h.cuda()) for h in host]
    kw = dict(lr=1e-3, weight_decay=0.1, precision=precision, stochastic_rounding=False, **extra)
    oa, ob = ApexW(pa, **kw), ApexW(pb, **kw)
    if start:
        for a, b in zip(pa, pb):
            g = (torch.randn(a.shape, generator=gen) * 1e-3).bfloat16()
            a.grad, b.grad = g.cuda(), g.cuda()
        oa.step()
        ob.step()
        _restep(oa, start)
        _restep(ob, start)
    scale = 1024.0
    infs = [0, 0, 1, 0, 1, 1, 0]
    for it, inf in enumerate(infs):
        for a, b in zip(pa, pb):
            g = (torch.randn(a.shape, generator=gen) * 1e-3 * scale).bfloat16()
            if inf and a.dim() == 2:
                g[0, 0] = float("inf")            # the step GradScaler found an inf in
            a.grad, b.grad = g.cuda(), g.cuda()
        oa.grad_scale, oa.found_inf = torch.tensor(scale, device="cuda"), torch.tensor(float(inf), device="cuda")
        ob.grad_scale, ob.found_inf = torch.tensor(scale), torch.tensor(float(inf))
        oa.step()
        ob.step()
    sd = oa.state_dict()
    torch.cuda.synchronize()
    taken = start + len(infs) - sum(infs)
    for a, b in zip(pa, pb):
        assert torch.equal(a, b)
        assert bool(torch.isfinite(a).all())
        sa, sb = oa.state[a], ob.state[b]
        for k in ("exp_avg", "exp_avg_sq", "exp_avg_scales", "exp_avg_sq_scales"):
            if k in sb:
                assert torch.equal(sa[k], sb[k]), k
        assert float(sa["step"]) == float(sb["step"]) == taken
    assert all(float(st["step"]) == taken for st in sd["state"].values())


def test_device_amp_with_more_step_counts_than_its_table():
    """An 8-bit group whose parameters hold 20 distinct step counts (more launches
    than the device-side AMP table's 16): GradScaler's scale is then read on the
    host for that step, and the results equal the host path's."""
    _need_gpu()
    from apexw_amd import ApexW
    from apexw_amd import _lib as L
    print("device amp, 20 distinct step counts", flush=True)
    gen = torch.Generator().manual_seed(23)
    n = 20
    assert n > L.AMP_MAX_LAUNCHES
    host = [(torch.randn(64, 64, generator=gen) * 0.02).bfloat16() for _ in range(n)]
    pa = [torch.nn.Parameter(h.cuda()) for h in host]
    pb = [torch.nn.Parameter(h.cuda()) for h in host]
    kw = dict(lr=1e-3, weight_decay=0.1, precision="8bit", stochastic_rounding=False)
    oa, ob = ApexW(pa, **kw), ApexW(pb, **kw)
    scale = 256.0
    for it in range(n + 3):
        for i, (a, b) in enumerate(zip(pa, pb)):
            if it < n and i < it:
                a.grad = b.grad = None          # parameter i misses the first i steps
                continue
            g = (torch.randn(a.shape, generator=gen) * 1e-3 * scale).bfloat16()
            a.grad, b.grad = g.cuda(), g.cuda()
        inf = float(it == n + 1)
        oa.grad_scale, oa.found_inf = torch.tensor(scale, device="cuda"), torch.tensor(inf, device="cuda")
        ob.grad_scale, ob.found_inf = torch.tensor(scale), torch.tensor(inf)
        oa.step()
        ob.step()
    torch.cuda.synchronize()
    counts = sorted({int(oa.state[a]["step"]) for a in pa})
    assert len(counts) == n, counts
    for i, (a, b) in enumerate(zip(pa, pb)):
        assert torch.equal(a, b), i
        for k in ("exp_avg", "exp_avg_sq", "exp_avg_scales", "exp_avg_sq_scales"):
            assert torch.equal(oa.state[a][k], ob.state[b][k]), (i, k)
        assert float(oa.state[a]["step"]) == float(ob.state[b]["step"]) == i + 3   # i + 1, then 2 of 3


def test_muon_device_amp_equals_host_amp_with_skipped_steps():
    """ApexMuon under GradScaler: the device path (found_inf and the scale read by
    the kernels) against the host path (the same values as CPU tensors, read on
    the host like the reference, apexw/muon.py:557-577), over steps some of which
    found an inf: identical parameters and momenta, and step counters that count
    only the steps taken.  The parameters cover the grouped Newton-Schulz with its
    fused update (wide, tall, non-contiguous), a group with ns_steps=0 (the
    separate update pass) and the coordinate-wise fallback (a vector, a matrix
    with a dimension under 16)."""
    _need_gpu()
    from apexw_amd.muon import ApexMuon
    print("muon device vs host amp", flush=True)
    gen = torch.Generator().manual_seed(31)
    shapes = [(256, 384), (384, 256), (300,), (8, 40)]
    host = [torch.randn(s, generator=gen) * 0.02 for s in shapes]
    host_t = torch.randn(384, 128, generator=gen) * 0.02
    host_z = torch.randn(128, 256, generator=gen) * 0.02

    def params():
        ps = [torch.nn.Parameter(h.cuda().bfloat16()) for h in host]
        ps.append(torch.nn.Parameter(host_t.cuda().bfloat16().t()))     # non-contiguous [128 x 384]
        return ps, torch.nn.Parameter(host_z.cuda())

    (pa, za), (pb, zb) = params(), params()
    kw = dict(lr=0.02, weight_decay=0.1, scale_mode="rms_matched")
    oa = ApexMuon([{"params": pa}, {"params": [za], "ns_steps": 0}], **kw)
    ob = ApexMuon([{"params": pb}, {"params": [zb], "ns_steps": 0}], **kw)
    scale = 4096.0
    infs = [0, 1, 0, 0, 1, 1, 0]
    for inf in infs:
        for a, b in zip(pa + [za], pb + [zb]):
            g = torch.randn(a.shape, generator=gen) * 1e-3 * scale
            if inf:
                g.view(-1)[7] = float("inf")
            a.grad, b.grad = g.to("cuda", a.dtype), g.to("cuda", b.dtype)
        oa.grad_scale, oa.found_inf = torch.tensor(scale, device="cuda"), torch.tensor(float(inf), device="cuda")
        ob.grad_scale, ob.found_inf = torch.tensor(scale), torch.tensor(float(inf))
        oa.step()
        ob.step()
    sd = oa.state_dict()
    torch.cuda.synchronize()
    taken = len(infs) - sum(infs)
    for a, b in zip(pa + [za], pb + [zb]):
        assert torch.equal(a, b)
        assert torch.equal(oa.state[a]["momentum"], ob.state[b]["momentum"])
        assert oa.state[a]["step"] == ob.state[b]["step"] == taken
    assert all(st["step"] == taken for st in sd["state"].values())


def test_muon_grad_scaler_step_reads_nothing_on_the_host():
    """After its first step, ApexMuon's GradScaler step (momentum, grouped
    Newton-Schulz with the fused update, coordinate-wise vectors) launches without
    a host synchronisation, and its step counters are exact when looked at."""
    _need_gpu()
    from apexw_amd.muon import ApexMuon
    torch.manual_seed(5)
    m = torch.nn.Sequential(torch.nn.Linear(64, 128), torch.nn.GELU(), torch.nn.Linear(128, 64)).cuda()
    opt = ApexMuon(m.parameters(), lr=0.02, weight_decay=0.01)
    scaler = torch.amp.GradScaler("cuda", init_scale=2.0 ** 12)
    x = torch.randn(8, 64, device="cuda")
    for it in range(3):
        opt.zero_grad()
        scaler.scale(m(x).square().mean()).backward()
        if it > 0:
            torch.cuda.set_sync_debug_mode("error")
        try:
            scaler.step(opt)
        finally:
            torch.cuda.set_sync_debug_mode("default")
        scaler.update()
    torch.cuda.synchronize()
    assert all(opt.state[p]["step"] == 3 for p in m.parameters())
