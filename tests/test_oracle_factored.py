"""Pins the factored-v / 6-bit oracle (oracle/factored.py) on the CPU."""

import pytest
import torch

from oracle import factored as F
from oracle import layout as L
from oracle.optim import OracleApexW


def test_reference_6bit_roundtrip():
    """The reference's test_quantization.py:1273-1283."""
    torch.manual_seed(42)
    x = torch.randn(1024, 512, dtype=torch.float32) * 0.25
    q, scales = F.quant_6bit(x, 256)
    assert q.dtype == torch.uint8 and scales.dtype == torch.float32
    assert q.numel() == (x.numel() // 4) * 3
    deq = F.dequant_6bit(q, scales, x.numel(), 256).reshape(x.shape)
    assert ((deq - x).abs().mean() / x.abs().mean()).item() < 0.05


def test_6bit_bit_layout_brute_force():
    """Codes c0..c3 (0..62) occupy bits [6i, 6i+6) of a little-endian 24-bit word."""
    gen = torch.Generator().manual_seed(1)
    codes = torch.randint(0, 63, (256,), generator=gen)
    scale = torch.full((1, 1), 0.5)
    x = (codes.float() - 31.0) * 0.5
    q, s = F.quant_6bit(x, 256)
    assert torch.equal(s, scale)
    for k in range(64):
        word = int(q[3 * k]) | (int(q[3 * k + 1]) << 8) | (int(q[3 * k + 2]) << 16)
        for i in range(4):
            assert (word >> (6 * i)) & 63 == int(codes[4 * k + i])
    assert torch.equal(F.dequant_6bit(q, s, 256, 256), x)
    z, zs = F.quant_6bit(torch.zeros(8), 8)
    assert z.tolist() == [0xDF, 0xF7, 0x7D] * 2 and float(zs) == pytest.approx(1e-12 / 31.0)


def test_6bit_scale_ema_and_padding():
    x = torch.linspace(-1, 1, 300)
    q, s = F.quant_6bit(x, 128, old_scales=torch.tensor([[0.01], [0.01], [0.05]]))
    assert q.numel() == 3 * 384 // 4                     # padded to 3 blocks of 128
    amax = torch.stack([x[:128].abs().max(), x[128:256].abs().max(), x[256:].abs().max()])
    want = torch.maximum(amax / 31.0, torch.tensor([0.009, 0.009, 0.045]))
    assert torch.allclose(s.view(-1), want, rtol=1e-6) and float(s[2]) == pytest.approx(0.045)
    assert torch.equal(F.dequant_6bit(q, s, 384, 128)[300:], torch.zeros(84))


def _group(**kw):
    g = dict(lr=1e-2, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.1)
    g.update(kw)
    return g


@pytest.mark.parametrize("shape", [(256, 512), (1024, 512)])     # one piece; row-chunked statistics
@pytest.mark.parametrize("m_kind", ["int8", "bf16"])
def test_first_step_matches_closed_form(shape, m_kind):
    gen = torch.Generator().manual_seed(3)
    p = torch.randn(shape, generator=gen) * 0.02
    g = torch.randn(shape, generator=gen) * 1e-3
    rows, cols = shape
    st = {"exp_avg_sq_row": torch.zeros(rows), "exp_avg_sq_col": torch.zeros(cols), "is_6bit_m": False}
    if m_kind == "int8":
        st["exp_avg"] = torch.zeros(shape, dtype=torch.int8)
        st["exp_avg_scales"] = torch.full((p.numel() // 2048, 1), 1e-12 / 127)
    else:
        st["exp_avg"] = torch.zeros(shape, dtype=torch.bfloat16)
    p0 = p.clone()
    b2 = 0.999
    F.factored_update(p, g, st, beta1=0.9, beta2=b2, step_size=1e-2 * (1 - b2) ** 0.5 / 0.1,
                      eps_scaled=1e-8 * (1 - b2) ** 0.5, eps=1e-8, stochastic=False, block_size=2048,
                      wd_factor=1 - 1e-3)
    want, r, c = F.first_step_closed_form(p0, g, lr=1e-2, beta1=0.9, beta2=b2, eps=1e-8, weight_decay=0.1)
    assert torch.allclose(st["exp_avg_sq_row"].double(), r, rtol=1e-5, atol=0)
    assert torch.allclose(st["exp_avg_sq_col"].double(), c, rtol=1e-5, atol=0)
    upd = (want - p0.double() * (1 - 1e-3)).abs()
    assert ((p.double() - want).abs() <= 1e-5 * upd + 4 * 2.0 ** -24 * p0.double().abs() + 1e-12).all()


def test_chunked_and_single_piece_statistics_agree():
    gen = torch.Generator().manual_seed(4)
    g = torch.randn(1024, 512, generator=gen) * 1e-3
    outs = []
    for chunk in (F.CHUNK, 1 << 30):
        st = {"exp_avg_sq_row": torch.zeros(1024), "exp_avg_sq_col": torch.zeros(512),
              "exp_avg": torch.zeros(1024, 512, dtype=torch.bfloat16)}
        old, F.CHUNK = F.CHUNK, chunk
        try:
            F.factored_update(torch.zeros(1024, 512), g, st, beta1=0.9, beta2=0.999, step_size=1e-3,
                              eps_scaled=1e-9, eps=1e-8, stochastic=False, block_size=256)
        finally:
            F.CHUNK = old
        outs.append((st["exp_avg_sq_row"].clone(), st["exp_avg_sq_col"].clone()))
    assert torch.equal(outs[0][0], outs[1][0])             # same row formula
    assert torch.allclose(outs[0][1], outs[1][1], rtol=2e-6, atol=0)


def test_layout_matches_reference_cases():
    """test_quantization.py:548-592, :1285-1310, :1374-1395."""
    def st_of(p, **kw):
        grp = dict(precision="8bit", betas=(0.9, 0.999), stochastic_rounding=True, factored_v=True, int4_m=None)
        grp.update(kw)
        return L.init_state(p, grp, 8, False)
    for shape in [(1024, 256), (256, 256), (128, 64, 3, 3)]:
        st = st_of(torch.zeros(shape))
        assert st["is_factored_v"] and not st["is_4bit_m"] and st["exp_avg"].dtype == torch.int8
        assert "exp_avg_sq" not in st and st["exp_avg_sq_row"].dtype == torch.float32
    st = st_of(torch.zeros(128, 64))                        # 8,192 < 65,536
    assert not st["is_factored_v"] and st["exp_avg_sq"].dtype == torch.uint8
    st = st_of(torch.zeros(512, 512))
    b = sum(v.numel() * v.element_size() for k, v in st.items() if torch.is_tensor(v) and k != "step")
    assert b / (512 * 512) < 1.05
    st = st_of(torch.zeros(1024, 512, dtype=torch.bfloat16), six_bit=True)
    assert st["is_6bit_m"] and st["exp_avg"].dtype == torch.uint8
    b = sum(v.numel() * v.element_size() for k, v in st.items() if torch.is_tensor(v))
    assert b / (1024 * 512) < 0.80
    cgrp = dict(precision="compact", betas=(0.9, 0.95), stochastic_rounding=True, factored_v=True, int4_m=None)
    assert not L.init_state(torch.zeros(512, 512, dtype=torch.bfloat16), cgrp, 1, False)["is_factored_v"]
    st = L.init_state(torch.zeros(1024, 512, dtype=torch.bfloat16), cgrp, 1, False)
    assert st["is_factored_v"] and st["exp_avg"].dtype == torch.bfloat16
    assert st["exp_avg_sq_row"].numel() == 1024 and st["exp_avg_sq_col"].numel() == 512
    b = sum(v.numel() * v.element_size() for k, v in st.items() if torch.is_tensor(v) and k != "step")
    assert b / (1024 * 512) < 2.05


@pytest.mark.parametrize("prec,kw", [("8bit", {}), ("8bit", {"six_bit": True}), ("compact", {})])
def test_oracle_optimizer_converges_with_factored_v(prec, kw):
    """The reference's convergence checks (test_quantization.py:594-623, :1312-1334) on the oracle."""
    torch.manual_seed(10)
    x = torch.randn(32, 512, dtype=torch.bfloat16)
    target = x @ (torch.randn(512, 1024, dtype=torch.bfloat16) * 0.05)
    w = torch.nn.Parameter(torch.randn(1024, 512, dtype=torch.bfloat16) * 0.02)
    opt = OracleApexW([w], lr=1e-2, betas=(0.9, 0.95), precision=prec, factored_v=True, **kw)
    losses = []
    for _ in range(15):
        w.grad = None
        loss = ((x.float() @ w.float().t()) - target.float()).pow(2).mean()
        loss.backward()
        opt.step()
        losses.append(float(loss))
    assert opt.state[w]["is_factored_v"]
    assert losses[-1] < losses[0] * 0.5
