"""GPU: the bf16 MFMA GEMM, the Muon step and the hybrid optimizer.

Tolerances:
  * GEMM: |O - ref| <= 2^-8 |ref| + 1e-4 max|ref| against an fp32 product of the
    same bf16 inputs (bf16 output rounding is <= 2^-9 relative);
  * Newton-Schulz / Muon update: relative Frobenius error <= 3% against the fp32
    CPU oracle.  The work dtype is bf16 (as the reference's on a bf16-capable
    GPU); the reference's own bf16 path differs from its fp32 path by 0.9-1.5%
    on these shapes (torch CPU bf16 matmuls), so 3% is twice that;
  * fp32 momentum and the AdamW-routed parameters: the fp32 bounds of the
    fused-step parity tests (1e-6 relative).
"""

import math

import numpy as np
import pytest
import torch

from golden.make_golden import _fingerprint, _grad, _param
from golden_replay import load
from oracle.muon import NS_A, NS_B, NS_C, newton_schulz5

pytestmark = pytest.mark.gpu


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")


def _rel_fro(got, ref):
    got, ref = got.double().cpu(), ref.double().cpu()
    return float((got - ref).norm() / ref.norm())


@pytest.mark.parametrize("m,n,k,batch", [(256, 512, 320, 2), (512, 256, 1024, 1), (256, 256, 64, 3)])
def test_gemm_nt_bf16_matches_fp32_product(m, n, k, batch):
    _need_gpu()
    from apexw_amd import _lib
    lib = _lib.load()
    print(f"gemm m={m} n={n} k={k} batch={batch}", flush=True)
    g = torch.Generator().manual_seed(m + n + k)
    A = torch.randn(batch, m, k, generator=g).bfloat16()
    B = torch.randn(batch, n, k, generator=g).bfloat16()
    E = torch.randn(batch, m, n, generator=g).bfloat16()
    alpha, beta = 0.75, -1.25
    ref = alpha * (A.float() @ B.float().transpose(1, 2)) + beta * E.float()   # fp32 on the CPU
    dA, dB, dEt = A.cuda(), B.cuda(), E.transpose(1, 2).contiguous().cuda()
    C = torch.full((batch, m, n), float("nan"), dtype=torch.bfloat16, device="cuda")
    Ct = torch.full((batch, n, m), float("nan"), dtype=torch.bfloat16, device="cuda")
    st = lib.apexw_gemm_nt_bf16(dA.data_ptr(), dB.data_ptr(), dEt.data_ptr(), C.data_ptr(), Ct.data_ptr(),
                                m, n, k, k, k, m, n, m, batch, m * k, n * k, n * m, m * n, n * m, alpha, beta,
                                torch.cuda.current_stream().cuda_stream)
    assert st == 0
    torch.cuda.synchronize()
    got = C.float().cpu()
    err = (got - ref).abs() - (2.0 ** -8 * ref.abs() + 1e-4 * ref.abs().max())
    assert float(err.max()) <= 0, f"max excess {float(err.max()):.3e}"
    assert torch.equal(Ct.cpu().transpose(1, 2), C.cpu())


def test_gemm_rejects_bad_shapes_before_launch():
    _need_gpu()
    from apexw_amd import _lib
    lib = _lib.load()
    x = torch.zeros(256 * 256, dtype=torch.bfloat16, device="cuda")
    p = x.data_ptr()
    s = torch.cuda.current_stream().cuda_stream
    assert lib.apexw_gemm_nt_bf16(p, p, None, None, p, 200, 256, 64, 64, 64, 0, 0, 256, 1, 0, 0, 0, 0, 0,
                                  1.0, 0.0, s) == 1   # m not a tile multiple
    assert lib.apexw_gemm_nt_bf16(p, p, None, None, None, 256, 256, 64, 64, 64, 0, 0, 256, 1, 0, 0, 0, 0, 0,
                                  1.0, 0.0, s) == 1   # no output
    assert lib.apexw_gemm_nt_bf16(p, p, None, None, p, 256, 256, 64, 64, 64, 0, 0, 256, 1, 0, 0, 0, 0, 0,
                                  1.0, 2.0, s) == 1   # beta without addend
    assert lib.apexw_gemm_nt_bf16(p + 2, p, None, None, p, 256, 256, 64, 64, 64, 0, 0, 256, 1, 0, 0, 0, 0, 0,
                                  1.0, 0.0, s) == 4   # misaligned


def _muon_updates(shapes, steps=1, seed=0, dtype=torch.float32, nesterov=False):
    """Run ApexMuon on the GPU and the fp32 oracle recipe on the CPU; return per-param (gpu, cpu) pairs."""
    from apexw_amd.muon import ApexMuon
    g = torch.Generator().manual_seed(seed)
    lr, wd, mu = 0.02, 0.1, 0.95
    host = [(torch.randn(s, generator=g) * 0.02).to(dtype) for s in shapes]
    ps = [torch.nn.Parameter(h.cuda()) for h in host]
    opt = ApexMuon(ps, lr=lr, momentum=mu, weight_decay=wd, ns_steps=5, scale_mode="rms_matched",
                   nesterov=nesterov)
    ref = [h.float().clone() for h in host]
    bufs = [torch.zeros(s) for s in shapes]
    out = []
    for _ in range(steps):
        grads = [(torch.randn(s, generator=g) * 1e-3).to(dtype) for s in shapes]
        before = [p.detach().float().cpu() for p in ps]
        for p, gr in zip(ps, grads):
            p.grad = gr.cuda()
        opt.step()
        torch.cuda.synchronize()
        out = []
        for i, s in enumerate(shapes):
            bufs[i].mul_(mu).add_(grads[i].float(), alpha=1 - mu)
            src = grads[i].float().lerp(bufs[i], mu) if nesterov else bufs[i]
            U = newton_schulz5(src, 5, work_dtype=torch.float32)
            scale = 0.2 * math.sqrt(max(s[0], int(np.prod(s)) // s[0]))
            if dtype == torch.float32:
                d_ref = -lr * scale * U
                d_gpu = ps[i].detach().float().cpu() - before[i] * (1 - lr * wd)
            else:
                # same roundings as p.mul_(1 - lr*wd); p.add_(U, alpha=-lr*scale) on a 16-bit p
                decayed = (before[i] * np.float32(1 - lr * wd)).to(dtype).float()
                p_ref = (decayed + np.float32(-lr * scale) * U.to(dtype).float()).to(dtype).float()
                d_ref = p_ref - before[i]
                d_gpu = ps[i].detach().float().cpu() - before[i]
            out.append((d_gpu, d_ref, opt.state[ps[i]], bufs[i].clone()))
    return out


@pytest.mark.parametrize("shapes", [[(256, 512)], [(512, 256)], [(300, 200)], [(64, 64)], [(256, 512), (256, 512)],
                                    [(33, 50)], [(100, 36), (100, 36)]])
def test_muon_step_matches_fp32_oracle(shapes):
    _need_gpu()
    print(f"muon shapes={shapes}", flush=True)
    for d_gpu, d_ref, st, buf in _muon_updates(shapes, steps=2, seed=len(shapes) + shapes[0][0]):
        assert _rel_fro(d_gpu, d_ref) <= 0.03, _rel_fro(d_gpu, d_ref)
        got = st["momentum"].cpu()
        assert st["momentum"].dtype == torch.float32 and st["step"] == 2
        assert torch.allclose(got, buf, rtol=1e-6, atol=1e-12)


def test_muon_nesterov_and_bf16_params():
    _need_gpu()
    for d_gpu, d_ref, st, _ in _muon_updates([(256, 384), (384, 256)], steps=1, seed=7, nesterov=True):
        assert _rel_fro(d_gpu, d_ref) <= 0.03
    # bf16 params: both sides round the decayed and the updated parameter to bf16;
    # a Newton-Schulz difference flips some of those roundings by one bf16 ulp
    for d_gpu, d_ref, st, _ in _muon_updates([(256, 256)], steps=1, seed=8, dtype=torch.bfloat16):
        assert _rel_fro(d_gpu, d_ref) <= 0.05, _rel_fro(d_gpu, d_ref)


def test_muon_polar_invariant_on_gpu():
    # reference known answer (tests/test_muon.py:26-51): singular values of the NS5 result in (0.5, 1.3)
    _need_gpu()
    from apexw_amd.muon import ApexMuon
    torch.manual_seed(42)
    for shape in [(64, 64), (128, 64), (64, 128)]:
        G = torch.randn(shape)
        p = torch.nn.Parameter(torch.zeros(shape, device="cuda"))
        # one step from zero momentum with mu = 0: the NS input is G itself
        opt = ApexMuon([p], lr=1.0, momentum=0.0, weight_decay=0.0, ns_steps=5, scale_mode="none")
        p.grad = G.cuda()
        opt.step()
        U = -p.detach().double().cpu()
        s = torch.linalg.svdvals(U)
        assert float(s.min()) > 0.5 and float(s.max()) < 1.3, (shape, float(s.min()), float(s.max()))


def test_hybrid_trajectory_matches_reference_vectors():
    _need_gpu()
    from apexw_amd import ApexW
    z = load("muon")
    shapes = [(64, 64), (64, 64), (48, 96), (64,), (4096, 32)]
    gen = torch.Generator().manual_seed(12)
    host = [_param(s, torch.float32, gen) for s in shapes]
    init = [h.clone() for h in host]
    fp = [_fingerprint(h) for h in host]
    ps = [torch.nn.Parameter(h.cuda()) for h in host]
    opt = ApexW(ps, lr=1e-3, weight_decay=0.1, use_muon=True, stochastic_rounding=False)
    assert type(opt).__name__ == "HybridApexW"
    for _ in range(3):
        for p in ps:
            gr = _grad(p.shape, torch.float32, gen, 1e-3)
            fp.append(_fingerprint(gr))
            p.grad = gr.cuda()
        opt.step()
    torch.cuda.synchronize()
    np.testing.assert_array_equal(np.array(fp, dtype=np.int64), z["h_fingerprint"])
    assert [1 if any(p is q for q in opt.muon_params) else 0 for p in ps] == z["h_route"].tolist()
    for i, p in enumerate(ps):
        got = p.detach().cpu().double()
        gold = torch.from_numpy(z[f"hp_{i}"]).double()
        if z["h_route"][i]:
            # Muon: the accumulated update within the bf16 Newton-Schulz bound
            assert _rel_fro(got - init[i].double(), gold - init[i].double()) <= 0.03, i
        else:
            err = (got - gold).abs() - (1e-6 * gold.abs() + 1e-9)
            assert float(err.max()) <= 0, i


def _grouped(lib, rows, cus=0):
    """Schedule and run one grouped launch of host-built problem rows (cus > 0:
    CUs per queue for the schedule, which then splits tail tiles into halves)."""
    from apexw_amd import _lib
    probs = _lib.gemm_problems(rows)
    items, offsets, n_wg, kind = _lib.gemm_schedule(probs, cus)
    if cus:
        assert np.any((items >> 22) & 3), "no half tiles in the schedule"
    dev = lambda a: torch.from_numpy(a.view(np.uint8).copy()).cuda()  # noqa: E731
    dp, di, do = dev(probs), dev(items), dev(offsets)
    st = lib.apexw_gemm_nt_grouped(dp.data_ptr(), di.data_ptr(), do.data_ptr(), n_wg, kind, None,
                                   torch.cuda.current_stream().cuda_stream)
    assert st == 0
    torch.cuda.synchronize()


def _assert_gemm_close(got, ref):
    err = (got.float().cpu() - ref).abs() - (2.0 ** -8 * ref.abs() + 1e-4 * ref.abs().max())
    assert float(err.max()) <= 0, f"max excess {float(err.max()):.3e}"


@pytest.mark.parametrize("cus", [0, 4])
def test_grouped_gemm_symmetric_and_plain_products(cus):
    """One grouped launch per Newton-Schulz product over matrices of two shapes:
    the symmetric products fill both triangles (bitwise symmetric), the plain
    product writes both layouts.  cus=4: a schedule for 4 CUs per queue, which
    splits tiles into 128-row halves (every epilogue kind, the diagonal addend
    and the [K x N] operand through the half-tile path)."""
    _need_gpu()
    from apexw_amd import _lib
    lib = _lib.load()
    print(f"grouped gemm cus={cus}", flush=True)
    g = torch.Generator().manual_seed(11)
    shapes = [(256, 512), (512, 768), (512, 768)]
    X = [(torch.randn(m, n, generator=g) / math.sqrt(n)).bfloat16() for m, n in shapes]
    dX = [x.cuda() for x in X]
    dXt = [x.t().contiguous().cuda() for x in X]
    nan = lambda *s: torch.full(s, float("nan"), dtype=torch.bfloat16, device="cuda")  # noqa: E731
    dA = [nan(m, m) for m, _ in shapes]
    dB = [nan(m, m) for m, _ in shapes]
    dC = [nan(m, n) for m, n in shapes]
    dCt = [nan(n, m) for m, n in shapes]
    SYM = _lib.GEMM_SYM
    # A = X X^T
    _grouped(lib, [(x.data_ptr(), x.data_ptr(), 0, a.data_ptr(), a.data_ptr(), m, m, n, n, n, 0, m, m, 1.0, 0.0,
                    SYM, 0) for x, a, (m, n) in zip(dX, dA, shapes)], cus)
    for x, a in zip(X, dA):
        ref = x.float() @ x.float().t()
        _assert_gemm_close(a, ref)
        assert torch.equal(a.cpu(), a.cpu().t())
    # B = c A A + b A
    _grouped(lib, [(a.data_ptr(), a.data_ptr(), a.data_ptr(), b.data_ptr(), b.data_ptr(), m, m, m, m, m, m, m, m,
                    NS_C, NS_B, SYM, 0) for a, b, (m, _) in zip(dA, dB, shapes)], cus)
    for a, b in zip(dA, dB):
        af = a.float().cpu()
        _assert_gemm_close(b, NS_C * (af @ af) + NS_B * af)
        assert torch.equal(b.cpu(), b.cpu().t())
    # X' = B X + a X, written row-major and transposed
    _grouped(lib, [(b.data_ptr(), xt.data_ptr(), xt.data_ptr(), c.data_ptr(), ct.data_ptr(), m, n, m, m, m, m, n, m,
                    1.0, NS_A, 0, 0) for b, xt, c, ct, (m, n) in zip(dB, dXt, dC, dCt, shapes)], cus)
    for b, x, c, ct in zip(dB, X, dC, dCt):
        _assert_gemm_close(c, b.float().cpu() @ x.float() + NS_A * x.float())
        assert torch.equal(ct.cpu().t(), c.cpu())
    # the same product with X as [K x N] rows (transposing LDS reads) and the
    # addend taken from that operand on the matrix cores (beta within 2^-18)
    for c in dC:
        c.fill_(float("nan"))
    KN = _lib.GEMM_B_KN | _lib.GEMM_ADD_B
    _grouped(lib, [(b.data_ptr(), x.data_ptr(), 0, c.data_ptr(), 0, m, n, m, m, n, 0, n, 0, 1.0, NS_A, KN, 0)
                   for b, x, c, (m, n) in zip(dB, dX, dC, shapes)], cus)
    for b, x, c in zip(dB, X, dC):
        _assert_gemm_close(c, b.float().cpu() @ x.float() + NS_A * x.float())


@pytest.mark.parametrize("cus", [0, 4])
def test_grouped_gemm_panels_equal_row_major(cus):
    """APEXW_GEMM_PANEL: the same products with every matrix in 32 x 32 panels give
    the row-major results bit for bit (only the operand and output addresses
    differ), for each epilogue kind Newton-Schulz uses and the plain product with
    both outputs and a read addend; cus=4 runs the half tiles too."""
    _need_gpu()
    from apexw_amd import _lib
    from apexw_amd.muon import _from_panels, _to_panels
    lib = _lib.load()
    print(f"grouped gemm panels cus={cus}", flush=True)
    g = torch.Generator().manual_seed(12)
    shapes = [(256, 512), (512, 768), (512, 768)]
    X = [(torch.randn(m, n, generator=g) / math.sqrt(n)).bfloat16().cuda() for m, n in shapes]

    def run(panel):
        lay = _to_panels if panel else (lambda t: t.clone())
        back = _from_panels if panel else (lambda t: t)
        pf = _lib.GEMM_PANEL if panel else 0
        dX = [lay(x) for x in X]
        dXt = [lay(x.t().contiguous()) for x in X]
        nan = lambda *s: torch.full(s, float("nan"), dtype=torch.bfloat16, device="cuda")  # noqa: E731
        dA, dB = [nan(m, m) for m, _ in shapes], [nan(m, m) for m, _ in shapes]
        dC, dCt, dK = [nan(m, n) for m, n in shapes], [nan(n, m) for m, n in shapes], [nan(m, n) for m, n in shapes]
        SYM = _lib.GEMM_SYM | pf
        _grouped(lib, [(x.data_ptr(), x.data_ptr(), 0, a.data_ptr(), a.data_ptr(), m, m, n, n, n, 0, m, m, 1.0, 0.0,
                        SYM, 0) for x, a, (m, n) in zip(dX, dA, shapes)], cus)
        _grouped(lib, [(a.data_ptr(), a.data_ptr(), a.data_ptr(), b.data_ptr(), b.data_ptr(), m, m, m, m, m, m, m, m,
                        NS_C, NS_B, SYM, 0) for a, b, (m, _) in zip(dA, dB, shapes)], cus)
        _grouped(lib, [(b.data_ptr(), xt.data_ptr(), xt.data_ptr(), c.data_ptr(), ct.data_ptr(), m, n, m, m, m, m, n,
                        m, 1.0, NS_A, pf, 0) for b, xt, c, ct, (m, n) in zip(dB, dXt, dC, dCt, shapes)], cus)
        KN = _lib.GEMM_B_KN | _lib.GEMM_ADD_B | pf
        _grouped(lib, [(b.data_ptr(), x.data_ptr(), 0, k.data_ptr(), 0, m, n, m, m, n, 0, n, 0, 1.0, NS_A, KN, 0)
                       for b, x, k, (m, n) in zip(dB, dX, dK, shapes)], cus)
        return [[back(t).cpu() for t in ts] for ts in (dA, dB, dC, dCt, dK)]

    rows, panels = run(False), run(True)
    for what, r, p in zip(("X X^T", "c A A + b A", "B X^T + a E (C)", "B X^T + a E (C^T)", "B X + a X"), rows,
                          panels):
        for i, (x, y) in enumerate(zip(r, p)):
            assert not torch.isnan(x).any(), (what, i)
            assert torch.equal(x, y), (what, i)


def test_muon_panels_match_row_major():
    """ApexMuon with its Newton-Schulz work matrices in 32 x 32 panels (the default)
    and row-major (ns_panels = False) gives the same parameters bit for bit over
    two steps: wide, tall and padded shapes, a batched shape, and an ns_steps == 0
    group, whose separate update pass reads the work matrix in its layout."""
    _need_gpu()
    from apexw_amd import ApexMuon
    print("muon panels vs row-major", flush=True)
    shapes = [(300, 700), (700, 300), (256, 512), (256, 512), (96, 160), (160, 96)]
    g = torch.Generator().manual_seed(13)
    init = [(torch.randn(s, generator=g) * 0.02).bfloat16() for s in shapes]
    grads = [[(torch.randn(s, generator=g) * 1e-3).bfloat16() for s in shapes] for _ in range(2)]

    def run(panels):
        ps = [torch.nn.Parameter(h.cuda()) for h in init]
        opt = ApexMuon([{"params": ps[:4], "ns_steps": 5}, {"params": ps[4:], "ns_steps": 0}], lr=0.02,
                       momentum=0.9, weight_decay=0.1, scale_mode="none")
        opt.ns_panels = panels
        for gs in grads:
            for p, gr in zip(ps, gs):
                p.grad = gr.cuda()
            opt.step()
        torch.cuda.synchronize()
        assert opt._ws and all(ws.panel == panels for ws in opt._ws.values())
        return [p.detach().cpu() for p in ps]

    for s, x, y in zip(shapes, run(True), run(False)):
        assert torch.equal(x, y), s


def test_muon_groups_with_different_ns_steps_and_many_matrices():
    """Param groups with different ns_steps share the grouped launches (a group
    leaves them when its iterations are done), and more than 256 matrices split
    into several launches; each parameter matches its own fp32 oracle update."""
    _need_gpu()
    from apexw_amd.muon import ApexMuon
    g = torch.Generator().manual_seed(21)
    big = [(torch.randn(256, 384, generator=g) * 0.02) for _ in range(2)]
    small = [(torch.randn(32, 48, generator=g) * 0.02) for _ in range(260)]
    pb = [torch.nn.Parameter(h.cuda()) for h in big]
    ps = [torch.nn.Parameter(h.cuda()) for h in small]
    lr, mu = 0.02, 0.95
    opt = ApexMuon([{"params": pb, "ns_steps": 5}, {"params": ps, "ns_steps": 3}], lr=lr, momentum=mu,
                   weight_decay=0.0, scale_mode="none")
    grads = [(torch.randn(h.shape, generator=g) * 1e-3) for h in big + small]
    for p, gr in zip(pb + ps, grads):
        p.grad = gr.cuda()
    opt.step()
    torch.cuda.synchronize()
    checks = [(pb[0], big[0], grads[0], 5), (pb[1], big[1], grads[1], 5)]
    checks += [(ps[i], small[i], grads[2 + i], 3) for i in (0, 1, 255, 256, 259)]
    for p, h, gr, steps in checks:
        U = newton_schulz5((1 - mu) * gr, steps, work_dtype=torch.float32)
        d_ref = -lr * U
        d_gpu = p.detach().float().cpu() - h
        assert _rel_fro(d_gpu, d_ref) <= 0.03, (tuple(p.shape), steps, _rel_fro(d_gpu, d_ref))


def test_fused_update_dtypes_layouts_and_zero_steps():
    """The update applied in the last Newton-Schulz product's epilogue, for fp32,
    bf16 and fp16 parameters, wide and tall (transposed work matrix), column
    counts that are not multiples of 8 (per-element path) and padded tiles: p
    equals round(round(p * (1 - lr wd)) + round(-lr) * U) from the kept U within
    one ulp of p's dtype (alpha rounded to p's dtype, as torch's add_ on a
    16-bit tensor does).  A group with ns_steps=0 takes the separate apply pass
    (U = the normalised momentum)."""
    _need_gpu()
    from apexw_amd.muon import ApexMuon
    g = torch.Generator().manual_seed(33)
    specs = [((300, 20), torch.float32), ((40, 100), torch.bfloat16), ((520, 264), torch.float16),
             ((64, 72), torch.float32)]
    init = [(torch.randn(s, generator=g) * 0.02).to(dt) for s, dt in specs]
    ps = [torch.nn.Parameter(h.cuda()) for h in init]
    lr, wd, mu = 0.02, 0.1, 0.9
    opt = ApexMuon([{"params": ps[:3], "ns_steps": 5}, {"params": ps[3:], "ns_steps": 0}], lr=lr, momentum=mu,
                   weight_decay=wd, scale_mode="none")
    opt.keep_ns_result = True
    grads = [(torch.randn(s, generator=g) * 1e-3).to(dt) for s, dt in specs]
    for p, gr in zip(ps, grads):
        p.grad = gr.cuda()
    opt.step()
    torch.cuda.synchronize()
    ws_by_shape = {k[1]: ws for k, ws in opt._ws.items()}
    for p, h, gr, (shape, dt), steps in zip(ps, init, grads, specs, (5, 5, 5, 0)):
        rows, cols = shape
        ws = ws_by_shape[shape]
        wide = ws.rows_of(ws.x[steps % 2][0])[:min(rows, cols), :max(rows, cols)].float().cpu()
        U = wide.T if rows > cols else wide
        if steps:
            U32 = newton_schulz5((1 - mu) * gr.float(), steps, work_dtype=torch.float32)
            assert _rel_fro(U, U32) <= 0.03, (shape, _rel_fro(U, U32))
        decayed = (h.float() * np.float32(1.0 - lr * wd)).to(dt).float()
        # p.add_(U, alpha=-lr) on a 16-bit p takes alpha in p's dtype (torch CPU)
        step = torch.tensor(-lr, dtype=torch.float32).to(dt).float() * U
        p_ref = (decayed + step).to(dt).float()
        got = p.detach().float().cpu()
        # one ulp of the result, plus the fp32 rounding of the product and sum
        # (the kernel fuses them into one fma): relative to the operands, which
        # can exceed the result where they cancel
        eps = 2.0 ** -7 if dt == torch.bfloat16 else 2.0 ** -10 if dt == torch.float16 else 2.0 ** -23
        bar = eps * p_ref.abs() + 2.0 ** -23 * (decayed.abs() + step.abs()) + 1e-30
        ex = (got - p_ref).abs() - bar
        w = int(ex.argmax())
        vals = {k: float(v.reshape(-1)[w]) for k, v in
                (("p0", h.float()), ("got", got), ("ref", p_ref), ("decayed", decayed), ("step", step), ("U", U))}
        assert float(ex.max()) <= 0, f"{shape} {dt} element {w}: {vals}"


def _assert_p_close(got, ref, what, upd):
    """p within one ulp of its dtype (fp32: 1e-6 relative + 1e-9) plus one ulp of
    the update upd = |lr * 0.05 * U|, which U's rounding to p's dtype can move by
    that much where the std differs in its last bits (it dominates where p ~ 0)."""
    dt = got.dtype
    got, ref, upd = got.detach().cpu().double(), ref.detach().double(), upd.detach().double().abs()
    if dt == torch.float32:
        tol = 1e-6 * ref.abs() + 1e-9 + 2.0 ** -23 * upd
    else:
        ulp = torch.finfo(dt).eps
        tol = ulp * (torch.maximum(got.abs(), ref.abs()) + upd) + 1e-30
    assert bool(((got - ref).abs() <= tol).all()), what


COORDWISE = [((64,), torch.bfloat16, torch.bfloat16, False), ((1,), torch.float32, torch.float32, False),
             ((2,), torch.float32, torch.float32, False), ((8, 4096), torch.bfloat16, torch.bfloat16, True),
             ((3000,), torch.bfloat16, torch.float32, False), ((40, 12), torch.float32, torch.bfloat16, True),
             ((15, 15), torch.float16, torch.float16, False)]


@pytest.mark.parametrize("shape,pdt,gdt,nesterov", COORDWISE, ids=[f"{c[0]}-{c[1]}-{c[2]}-{c[3]}" for c in COORDWISE])
def test_coordwise_fallback_matches_oracle(shape, pdt, gdt, nesterov):
    """Vectors and dimensions under 16 take the reference's coordinate-wise update
    (apexw/muon.py:841-858); grads may have another dtype than the parameter.
    Bars: fp32 momentum within 1e-6 relative (the same fmas), p within one ulp of
    its dtype (the std is a reduction in another order, ~1e-7 relative in U);
    each step starts the oracle from the GPU's p."""
    _need_gpu()
    from apexw_amd.muon import ApexMuon
    from oracle.muon import coordwise_step
    print(f"coordwise {shape} {pdt} {gdt} nesterov={nesterov}", flush=True)
    gen = torch.Generator().manual_seed(sum(shape))
    host = (torch.randn(shape, generator=gen) * 0.02).to(pdt)
    p = torch.nn.Parameter(host.cuda())
    if gdt != pdt:
        p.grad_dtype = None          # torch checks a grad's dtype against the parameter's unless told not to
    cp = host.clone()
    buf = torch.zeros(shape, dtype=torch.float32)
    opt = ApexMuon([p], lr=1e-2, momentum=0.95, nesterov=nesterov, weight_decay=0.1, ns_steps=5)
    for step in range(3):
        g = (torch.randn(shape, generator=gen) * 1e-3 * (1 + step)).to(gdt)
        p.grad = g.cuda()
        opt.step()
        U = coordwise_step(cp, g.clone(), buf, lr=1e-2, momentum=0.95, weight_decay=0.1, nesterov=nesterov)
        torch.cuda.synchronize()
        assert p.dtype == cp.dtype
        _assert_p_close(p, cp, f"p step {step}", 1e-2 * 0.05 * U)
        mom = opt.state[p]["momentum"].cpu().double()
        assert float(((mom - buf.double()).abs() - (1e-6 * buf.double().abs() + 1e-12)).max()) <= 0, "momentum"
        cp.copy_(p.detach().cpu())
    assert opt.state[p]["step"] == 3


def test_noncontiguous_matrix_and_grad_dtype():
    """A transposed (non-contiguous) parameter is stepped like its contiguous copy,
    with an fp32 grad on a bf16 parameter."""
    _need_gpu()
    from apexw_amd.muon import ApexMuon
    gen = torch.Generator().manual_seed(5)
    base = (torch.randn(96, 64, generator=gen) * 0.02).bfloat16().cuda()
    p_nc = torch.nn.Parameter(base.t())                  # [64 x 96], strides (1, 64)
    p_c = torch.nn.Parameter(base.t().contiguous())
    assert not p_nc.is_contiguous()
    p_nc.grad_dtype = None
    p_c.grad_dtype = None
    oa = ApexMuon([p_nc], lr=1e-2, weight_decay=0.1, ns_steps=5)
    ob = ApexMuon([p_c], lr=1e-2, weight_decay=0.1, ns_steps=5)
    for _ in range(2):
        g = torch.randn(64, 96, generator=gen).cuda() * 1e-3
        p_nc.grad = g.clone()
        p_c.grad = g.clone()
        oa.step()
        ob.step()
    torch.cuda.synchronize()
    assert torch.equal(p_nc.detach().contiguous(), p_c.detach())
    assert not p_nc.is_contiguous()
