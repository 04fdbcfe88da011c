"""In-backward 8-bit steps on the GPU against the CPU oracle (SR off, the parity
bars of test_gpu_parity.py), through a real autograd backward.

The model is a chain y = (y W_i^T) W_i (+ b) of fp32 weights; an 8-bit ApexW
over it converts the weights to bf16 (the biases, under 1024 elements, stay
fp32) and steps the large ones during backward in
batches of 14 (apexw/optimizer.py:2059-2371).  Every grad is captured by a
tensor hook as autograd produces it, so the oracle steps the same grads:
oracle.hooks.flush_8bit for the hooked weights, OracleApexW (the ordinary
8-bit step) for the anchor and the small tensors that step() takes.
"""

import pytest
import torch
import torch.nn as nn

from test_gpu_edge import _assert_close

pytestmark = pytest.mark.gpu

ROWS = [64, 1024, 32, 64, 128, 64, 64, 1024, 64, 32, 64, 64, 256, 64, 64, 64, 512, 64]


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")


class Chain(nn.Module):
    def __init__(self, rows, seed, lead=False):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        # lead: a 512-element input scale registered first, so the anchor stays fp32
        self.s = nn.Parameter(1.0 + 0.1 * torch.randn(512, generator=g)) if lead else None
        self.w = nn.ParameterList([nn.Parameter(torch.randn(r, 512, generator=g) * 0.05) for r in rows])
        self.b = nn.ParameterList([nn.Parameter(torch.randn(512, generator=g) * 0.01) for _ in range(2)])

    def forward(self, x):
        y = x if self.s is None else x * self.s.to(x.dtype)
        for i, w in enumerate(self.w):
            y = (y @ w.t()) @ w
            if i in (3, 11):
                y = y + self.b[(i > 3)].to(y.dtype)
            y = y / y.float().pow(2).mean().sqrt().to(y.dtype)
        return (y.float() ** 2).mean()


def _setup(seed=0, lead=False, **kw):
    from apexw_amd import ApexW
    from oracle import hooks as H
    from oracle.optim import OracleApexW
    model = Chain(ROWS, seed, lead).cuda()
    params = list(model.parameters())
    kw = dict(dict(lr=1e-3, weight_decay=0.1, precision="8bit", stochastic_rounding=False), **kw)
    before = [H.downcast_dtype(p) for p in params]
    opt = ApexW(params, **kw)
    assert [p.dtype for p in params] == before          # fp32 weights -> bf16; the 512-element biases stay fp32
    on, anchor, hooked = H.hook_partition(params)
    assert on and anchor is params[0]
    assert len(opt._auto_hook_handles) == len(hooked) + 1
    cpu = {p: nn.Parameter(p.detach().cpu().clone()) for p in params}
    hooked_ids = {id(p) for p in hooked}
    rest = [p for p in params if id(p) not in hooked_ids]
    oracle_rest = OracleApexW([cpu[p] for p in rest], **kw)
    group = dict(lr=kw["lr"], betas=(0.9, 0.999), eps=1e-8, weight_decay=kw["weight_decay"], decay_norm_only=True,
                 precision="8bit", stochastic_rounding=False, block_size=None, int4_m=None)
    captured = {}
    for p in params:
        p.register_hook(lambda g, p=p: captured.setdefault(id(p), []).append(g.detach().cpu().clone()))
    return model, params, opt, cpu, hooked, rest, oracle_rest, group, captured


def _batch(seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(16, 512, generator=g)).cuda().bfloat16()


def _compare(params, opt, cpu, hooked_states, oracle_rest, hooked, tag, only=None):
    """One step's parity, then the oracle takes the GPU's values: a log-uint8 code
    may differ by one where log2 lands within rounding of a half-integer (the
    bar allows it), and the next step would carry that into p; starting each
    step from the same values checks every step at the bar."""
    torch.cuda.synchronize()
    hid = {id(p) for p in hooked}
    for i, p in enumerate(params):
        if only is not None and not any(p is q for q in only):
            continue
        _assert_close(p, cpu[p], f"{tag} p{i}")
        cs = hooked_states[cpu[p]] if id(p) in hid else oracle_rest.state[cpu[p]]
        gs = opt.state[p]
        for k in ("exp_avg", "exp_avg_scales", "exp_avg_sq", "exp_avg_sq_scales"):
            _assert_close(gs[k], cs[k], f"{tag} p{i} {k}")
            cs[k].copy_(gs[k].cpu())
        assert float(gs["step"]) == float(cs["step"]), f"{tag} p{i} step"
        with torch.no_grad():
            cpu[p].copy_(p.detach().cpu())


@pytest.mark.parametrize("cautious", [False, True], ids=["plain", "cautious"])
def test_backward_steps_match_oracle(cautious):
    """cautious=True: the in-backward batches take the mask too (the reference's flush
    passes it to _step_ultra, apexw/optimizer.py:2359)."""
    _need_gpu()
    from oracle import hooks as H
    print(f"hooks: K=1, 3 iterations, cautious={cautious}", flush=True)
    kw = dict(cautious=True) if cautious else {}
    model, params, opt, cpu, hooked, rest, oracle_rest, group, captured = _setup(0, **kw)
    group = dict(group, **kw)
    states = {}
    for it in range(3):
        captured.clear()
        model(_batch(it)).backward()
        assert all(p.grad is None for p in hooked) and params[0].grad is not None
        rest_grads = [p.grad.detach().cpu().clone() for p in rest]
        opt.step()
        opt.zero_grad()
        H.flush_8bit([cpu[p] for p in hooked], [captured[id(p)][0] for p in hooked], states, group)
        for p, g in zip(rest, rest_grads):
            cpu[p].grad = g
        oracle_rest.step()
        _compare(params, opt, cpu, states, oracle_rest, hooked, f"iter {it}")
    assert all(int(opt.state[p]["step"]) == 3 for p in params)


def test_accumulation_passes_match_oracle():
    """Two backward passes per step: the first step learns K = 2, later passes step
    with the accumulation scaling; the anchor and small tensors accumulate."""
    _need_gpu()
    from oracle import hooks as H
    print("hooks: K=2 accumulation", flush=True)
    model, params, opt, cpu, hooked, rest, oracle_rest, group, captured = _setup(1)
    states = {}
    K = 1
    for it in range(3):
        captured.clear()
        for micro in range(2):
            model(_batch(10 * it + micro)).backward()
            H.flush_8bit([cpu[p] for p in hooked], [captured[id(p)][micro] for p in hooked], states, group, K=K)
            _compare(params, opt, cpu, states, oracle_rest, hooked, f"iter {it} pass {micro}", only=hooked)
        rest_grads = [p.grad.detach().cpu().clone() for p in rest]
        opt.step()
        opt.zero_grad()
        for p, g in zip(rest, rest_grads):
            cpu[p].grad = g
        oracle_rest.step()
        K = 2
        assert opt._grad_accum_steps == 2
        _compare(params, opt, cpu, states, oracle_rest, hooked, f"iter {it}", only=rest)


def test_grad_scaler_backward_matches_oracle():
    _need_gpu()
    from oracle import hooks as H
    print("hooks: GradScaler", flush=True)
    # GradScaler cannot check bf16 grads on the GPU; the tensors step() takes stay fp32
    model, params, opt, cpu, hooked, rest, oracle_rest, group, captured = _setup(2, lead=True)
    assert all(p.dtype == torch.float32 for p in rest)
    scaler = torch.amp.GradScaler("cuda", init_scale=2.0 ** 16)
    states = {}
    for it in range(2):
        captured.clear()
        scaler.scale(model(_batch(20 + it))).backward()
        rest_grads = [p.grad.detach().cpu().clone() for p in rest]
        scale = float(scaler.get_scale())
        scaler.step(opt)
        scaler.update()
        opt.zero_grad()
        H.flush_8bit([cpu[p] for p in hooked], [captured[id(p)][0] for p in hooked], states, group, amp_scale=scale)
        for p, g in zip(rest, rest_grads):
            cpu[p].grad = g
        oracle_rest.grad_scale = torch.tensor(scale)
        oracle_rest.found_inf = torch.tensor(0.0)
        oracle_rest.step()
        _compare(params, opt, cpu, states, oracle_rest, hooked, f"iter {it}")


def test_reference_in_backward_case():
    """The reference's test_quantization.py:1093-1129 on the GPU."""
    _need_gpu()
    from apexw_amd import ApexW
    print("hooks: reference case", flush=True)
    torch.manual_seed(123)
    params = [nn.Parameter((torch.randn(64, 512) * 0.05).cuda()) for _ in range(16)]
    orig_bytes = sum(p.numel() * p.element_size() for p in params)
    opt = ApexW(params, lr=2e-4, precision="8bit")
    assert sum(p.numel() * p.element_size() for p in params) == orig_bytes // 2
    x = torch.randn(16, 512).cuda().to(params[0].dtype)
    y = x
    for p in params:
        y = (y @ p.t()) @ p
    (y ** 2).mean().backward()
    assert params[0].grad is not None
    for p in params[1:]:
        assert p.grad is None and int(opt.state[p]["step"].item()) == 1
    torch.nn.utils.clip_grad_norm_(params, 1.0)
    opt.step()
    opt.zero_grad(set_to_none=True)
    assert all(int(opt.state[p]["step"].item()) == 1 for p in params)
    torch.optim.AdamW(params, lr=2e-4)
    assert all(p.dtype == torch.float32 for p in params)


@pytest.mark.parametrize("lr", [5e-4, 2e-4, 1e-5])
def test_reference_convergence_vs_adamw(lr):
    """The reference's test_quantization.py:1131-1168 on the GPU: 8-bit ApexW (SR on,
    in-backward steps) reaches a lower mean and final loss than torch AdamW."""
    _need_gpu()
    from apexw_amd import ApexW
    print(f"hooks: convergence lr={lr}", flush=True)
    torch.manual_seed(77)
    w_inits = [torch.randn(64, 512) * 0.05 for _ in range(16)]
    x = torch.randn(32, 512).cuda()
    target = torch.randn(32, 64).cuda()
    w_adamw = [nn.Parameter(w.clone().cuda()) for w in w_inits]
    opt_adamw = torch.optim.AdamW(w_adamw, lr=lr, betas=(0.9, 0.95), weight_decay=0.01)
    losses_adamw = []
    for _ in range(20):
        opt_adamw.zero_grad()
        loss = sum(((x @ w.t() - target) ** 2).mean() for w in w_adamw) / len(w_adamw)
        loss.backward()
        opt_adamw.step()
        losses_adamw.append(loss.item())
    w8 = [nn.Parameter(w.clone().cuda()) for w in w_inits]
    opt8 = ApexW(w8, lr=lr, betas=(0.9, 0.95), weight_decay=0.01, precision="8bit", stochastic_rounding=True)
    losses8 = []
    for _ in range(20):
        opt8.zero_grad()
        xc, tc = x.to(w8[0].dtype), target.to(w8[0].dtype)
        loss = sum(((xc @ w.t() - tc).float() ** 2).mean() for w in w8) / len(w8)
        loss.backward()
        opt8.step()
        losses8.append(loss.item())
    assert sum(losses8) / len(losses8) < sum(losses_adamw) / len(losses_adamw)
    assert losses8[-1] < losses_adamw[-1]


class Small(nn.Module):
    """Varied shapes: 2-D weights, 1-D norms and biases, a tensor under 64 elements."""

    def __init__(self, seed):
        super().__init__()
        torch.manual_seed(seed)
        self.a = nn.Linear(512, 256)
        self.norm = nn.LayerNorm(256)
        self.b = nn.Linear(256, 40)
        self.c = nn.Linear(40, 8)

    def forward(self, x):
        return (self.c(torch.relu(self.b(self.norm(self.a(x))))).float() ** 2).mean()


def _fused_setup(prec, dtype, seed, K=1, sr=False):
    from apexw_amd import ApexW
    model = Small(seed).cuda().to(dtype)
    params = list(model.parameters())
    kw = dict(lr=1e-2, weight_decay=0.1, precision=prec, stochastic_rounding=sr)
    opt = ApexW(params, **kw)
    cpu = {p: nn.Parameter(p.detach().cpu().clone()) for p in params}
    seen = {}
    for p in params:        # registered first: sees each accumulated grad before the fused step frees it
        p.register_post_accumulate_grad_hook(lambda t, p=p: seen.setdefault(id(p), []).append(t.grad.detach().cpu().clone()))
    opt.enable_fused_backward(model, grad_accum_steps=K)
    group = dict(lr=1e-2, betas=(0.9, 0.999) if prec == "8bit" else (0.9, 0.99), eps=1e-8, weight_decay=0.1,
                 decay_norm_only=True, precision=prec, stochastic_rounding=sr, block_size=None, int4_m=None)
    return model, params, opt, cpu, seen, group


def _compare_fused(params, opt, cpu, states, tag, prev):
    """fp32 parameters: the bound is relative to the operands of the last add,
    |p_prev| + |update|, not to the result.  torch's CPU sqrt (the oracle's) is
    one ulp below the IEEE square root for about 0.7% of inputs on its AVX-512
    build; at lr 1e-2 the first update is as large as p, and where it cancels p
    that ulp is large relative to the result."""
    torch.cuda.synchronize()
    for i, p in enumerate(params):
        if p.dtype == torch.float32:
            got, ref, p0 = p.detach().cpu().double(), cpu[p].detach().double(), prev[p].double()
            tol = 1e-6 * (ref.abs() + p0.abs() + (ref - p0).abs()) + 1e-9
            assert ((got - ref).abs() <= tol).all(), f"{tag} p{i}: excess {float(((got - ref).abs() - tol).max()):.3e}"
        else:
            _assert_close(p, cpu[p], f"{tag} p{i}")
        gs, cs = opt.state[p], states[cpu[p]]
        assert set(gs) == set(cs), f"{tag} p{i} keys"
        for k, v in cs.items():
            if torch.is_tensor(v) and k != "step":
                _assert_close(gs[k], v, f"{tag} p{i} {k}")
                v.copy_(gs[k].cpu())
        assert float(gs["step"]) == float(cs["step"])
        with torch.no_grad():
            cpu[p].copy_(p.detach().cpu())


@pytest.mark.parametrize("prec,dtype", [("8bit", torch.float32), ("8bit", torch.bfloat16), ("8bit", torch.float16),
                                        ("compact", torch.float32), ("compact", torch.bfloat16),
                                        ("compact", torch.float16)])
def test_fused_backward_matches_oracle(prec, dtype):
    _need_gpu()
    from oracle import hooks as H
    print(f"fused backward {prec} {dtype}", flush=True)
    model, params, opt, cpu, seen, group = _fused_setup(prec, dtype, 3)
    states = {}
    for it in range(3):
        seen.clear()
        g = torch.Generator().manual_seed(40 + it)
        model(torch.randn(16, 512, generator=g).cuda().to(dtype)).backward()
        assert all(p.grad is None for p in params)
        opt.step()                                   # nothing left to step
        prev = {p: cpu[p].detach().clone() for p in params}
        for p in params:
            H.fused_param_step(cpu[p], seen[id(p)][0], states.setdefault(cpu[p], {}), group)
        _compare_fused(params, opt, cpu, states, f"iter {it}", prev)


def test_fused_backward_accumulates_k_passes():
    _need_gpu()
    from oracle import hooks as H
    print("fused backward K=2", flush=True)
    model, params, opt, cpu, seen, group = _fused_setup("8bit", torch.bfloat16, 4, K=2)
    states = {}
    for it in range(2):
        seen.clear()
        for micro in range(2):
            g = torch.Generator().manual_seed(60 + 2 * it + micro)
            model(torch.randn(16, 512, generator=g).cuda().bfloat16()).backward()
            assert all((p.grad is None) == (micro == 1) for p in params)
        prev = {p: cpu[p].detach().clone() for p in params}
        for p in params:
            H.fused_param_step(cpu[p], seen[id(p)][1], states.setdefault(cpu[p], {}), group)
        _compare_fused(params, opt, cpu, states, f"iter {it}", prev)


@pytest.mark.parametrize("prec", ["compact", "8bit"])
def test_reference_fused_backward_case(prec):
    """The reference's test_quantization.py:794-816 on the GPU."""
    _need_gpu()
    from apexw_amd import ApexW
    print(f"fused backward reference case {prec}", flush=True)
    torch.manual_seed(42)
    model = nn.Sequential(nn.Linear(32, 16), nn.ReLU(), nn.Linear(16, 8)).cuda()
    opt = ApexW(model.parameters(), lr=1e-2, precision=prec)
    opt.enable_fused_backward(model)
    x = torch.randn(4, 32).cuda()
    target = torch.randn(4, 8).cuda()
    losses = []
    for _ in range(10):
        opt.zero_grad()
        loss = ((model(x) - target) ** 2).mean()
        loss.backward()
        assert all(p.grad is None for p in model.parameters())
        opt.step()
        losses.append(loss.item())
    assert losses[-1] < losses[0] * 0.5


def test_reference_fused_backward_disable():
    """The reference's test_quantization.py:818-830 on the GPU."""
    _need_gpu()
    from apexw_amd import ApexW
    torch.manual_seed(42)
    model = nn.Sequential(nn.Linear(32, 8)).cuda()
    opt = ApexW(model.parameters(), lr=1e-2, precision="compact")
    opt.enable_fused_backward(model)
    opt.disable_fused_backward()
    model(torch.randn(4, 32).cuda()).sum().backward()
    assert all(p.grad is not None for p in model.parameters())
    opt.step()
