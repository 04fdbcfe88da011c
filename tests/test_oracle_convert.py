"""Pins of the state conversion oracle (oracle/convert.py) on the CPU.

The conversion has no counterpart in the reference (its load keeps the saved
layout), so it is pinned by what the mathematics fixes: decode is the
reference's dequantizers; a state built by encode is a fixed point of
encode(decode(.)) -- the same codes, the same NF4 and log-uint8 scales (a
block's largest element decodes to exactly +-scale, and LUT[255] = 1), INT8
scales within one fp32 ulp (127 * (a / 127) / 127 need not round back to
a / 127); decode(encode(x)) stays within half a quantization step of x; the
pairwise quad mean of 4 equal values is that value, bit for bit.
"""

import pytest
import torch

from oracle import convert as C
from oracle import layout as Lay
from oracle import quant as Q


def _state(shape, prec, dtype=torch.bfloat16, nparams=10, **kw):
    p = torch.zeros(shape, dtype=dtype)
    group = dict(lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0, precision=prec, stochastic_rounding=True,
                 block_size=None, int4_m=None, force_compact_v=False, factored_v=False, six_bit=False, **kw)
    return p, Lay.init_state(p, group, nparams, False)


def _moments(n, seed):
    g = torch.Generator().manual_seed(seed)
    m = torch.randn(n, generator=g) * 1e-3
    v = (torch.randn(n, generator=g) * 1e-3) ** 2
    v[::97] = 0.0
    return m, v


CASES = [((512, 256), "8bit"), ((4096,), "8bit"), ((300,), "8bit"), ((40, 70), "8bit"), ((16390,), "8bit"),
         ((128, 256), "compact"), ((768,), "compact")]


@pytest.mark.parametrize("shape,prec", CASES)


def test_encode_decode_fixed_point(shape, prec):
    p, st = _state(shape, prec)
    n = p.numel()
    m, v = _moments(n, n)
    C.encode(st, m, v)
    s0 = {k: t.clone() for k, t in st.items() if torch.is_tensor(t)}
    m1, v1 = C.decode(st, n)
    C.encode(st, m1, v1)
    assert torch.equal(st["exp_avg"], s0["exp_avg"])
    assert torch.equal(st["exp_avg_sq"], s0["exp_avg_sq"])
    if st.get("is_8bit", False):
        assert torch.equal(st["exp_avg_sq_scales"], s0["exp_avg_sq_scales"])
        if st.get("is_4bit_m", False):
            assert torch.equal(st["exp_avg_scales"], s0["exp_avg_scales"])
        else:
            a, b = st["exp_avg_scales"], s0["exp_avg_scales"]
            assert bool(((a - b).abs() <= b.abs() * 2.0 ** -23).all())


@pytest.mark.parametrize("shape,prec", CASES)


def test_decode_encode_error_bound(shape, prec):
    p, st = _state(shape, prec)
    n = p.numel()
    m, v = _moments(n, 7 + n)
    C.encode(st, m, v)
    m1, v1 = C.decode(st, n)
    quad = st["exp_avg_sq"].numel() * 4 == n and st["exp_avg_sq"].numel() != n
    vq = C.quad_mean(v).repeat_interleave(4) if quad else v
    if st.get("is_8bit", False):
        bs = int(st["block_size_8bit"])
        ms = st["exp_avg_scales"].reshape(-1).repeat_interleave(bs)[:n]
        if st.get("is_4bit_m", False):
            gap = float((Q.NF4_CODEBOOK[1:15] - Q.NF4_CODEBOOK[:14]).max())
            assert bool(((m1 - m).abs() <= 0.5 * gap * ms * (1 + 1e-6)).all())
        else:
            assert bool(((m1 - m).abs() <= 0.5 * ms * (1 + 1e-6)).all())
        vs = st["exp_avg_sq_scales"].reshape(-1).repeat_interleave(bs)[:n]
        ratio = 2.0 ** (12.0 / 254.0) * (1 + 1e-5)
        big = vq > vs * 2.0 ** -24
        assert bool(((v1 <= vq * ratio) & (v1 >= vq / ratio) | ~big).all())
        assert bool((v1[vq == 0] == 0).all())
    else:
        assert torch.equal(m1, m.to(st["exp_avg"].dtype).float())
        assert torch.equal(v1, vq.to(st["exp_avg_sq"].dtype).float())


def test_quad_mean_of_equal_values_is_exact():
    g = torch.Generator().manual_seed(3)
    x = torch.rand(4096, generator=g) * 10.0 ** torch.randint(-30, 30, (4096,), generator=g).float()
    assert torch.equal(C.quad_mean(x.repeat_interleave(4)), x)


def test_nf4_encode_known_answers():
    """A block holding +-scale and every codebook level times the scale encodes to
    those codes; a value on a midpoint goes to the lower code; the block scale is
    the absmax (no /127)."""
    p, st = _state((16384,), "8bit")
    assert st["is_4bit_m"] and st["is_quad_v"]
    m = torch.zeros(16384)
    m[:15] = Q.NF4_CODEBOOK[:15] * 0.5
    m[15] = float(Q.NF4_MIDS[9]) * 0.5   # on the midpoint between codes 9 and 10
    C.encode(st, m, torch.zeros(16384))
    assert float(st["exp_avg_scales"].reshape(-1)[0]) == 0.5
    q = st["exp_avg"]
    codes = torch.stack([q >> 4, q & 15], 1).reshape(-1)
    assert codes[:15].tolist() == list(range(15))
    assert int(codes[15]) == 9
    assert bool((codes[16:2048] == 7).all())          # zeros -> code 7 (0.0)
    assert bool((st["exp_avg_sq"] == 0).all())


def test_fp16_scaled_v_decodes_to_the_moment():
    """An fp16 compact v holds the moment times scale_v (1024 for a fresh fp16 state
    with stochastic rounding): decode gives stored / 1024 exactly, and encode writes
    the same fp16 bits back; an 8-bit target gets the unscaled moment."""
    p, st = _state((64, 32), "compact", dtype=torch.float16)
    assert st["exp_avg_sq"].dtype == torch.float16 and st["scale_v"] == 1024.0
    g = torch.Generator().manual_seed(7)
    stored = ((torch.rand(p.numel(), generator=g) * 8.0).to(torch.float16))
    st["exp_avg_sq"].view(-1).copy_(stored)
    mf, vf = C.decode(st, p.numel())
    assert torch.equal(vf, stored.float() / 1024.0)
    assert float(vf.max()) < 8.0 / 1024.0 * 1.001
    _, st2 = _state((64, 32), "compact", dtype=torch.float16)
    C.encode(st2, mf, vf)
    assert torch.equal(st2["exp_avg_sq"].view(torch.int16), st["exp_avg_sq"].view(torch.int16))
    _, q8 = _state((64, 32), "8bit", dtype=torch.float16)
    C.encode(q8, mf, vf)
    _, v8 = C.decode(q8, p.numel())
    # log-uint8 keeps the magnitude: within a factor 2^(12/254) of the unscaled moment
    big = vf > vf.max() * 2.0 ** -20
    ratio = v8[big] / vf[big]
    assert float(ratio.max()) <= 2.0 ** (12 / 254) * 1.0001 and float(ratio.min()) >= 2.0 ** (-12 / 254) / 1.0001
