"""The SR checker (tests/sr_inject.py) pinned on the CPU.

The oracle's own stochastic rounding (torch's RNG) must pass it: every result
in the bracket and |z| < 3.  Mistakes planted in the oracle's rounding must
fail it: always rounding toward zero (biased), always taking the lower code
(biased), and a result two ulps / codes away (outside the bracket).
"""

import pytest
import torch

import oracle.quant as Q
from sr_inject import SRCheck

N = 1 << 20


def _x(seed, n=N):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(n, generator=g) * 0.02


def test_bf16_store_passes_for_oracle_sr():
    torch.manual_seed(1001)   # noise seed distinct from the data generator seed
    x = _x(1)
    gpu = torch.empty(N, dtype=torch.bfloat16)
    Q.store_16bit(gpu, x, True)
    dst = torch.empty(N, dtype=torch.bfloat16)
    with SRCheck() as sr:
        sr.target(dst, gpu)
        Q.store_16bit(dst, x, True)
    assert torch.equal(dst, gpu)            # the GPU's choice is written back
    sr.assert_unbiased(["bf16"], min_n=N // 2)


def test_bf16_store_catches_truncation_and_far_values():
    x = _x(2)
    trunc = (x.view(torch.int32) & -65536).view(torch.float32).to(torch.bfloat16)   # toward zero
    with SRCheck() as sr:
        sr.target(torch.empty(N, dtype=torch.bfloat16), trunc)
        Q.store_16bit(sr.targets[0][0], x, True)
    with pytest.raises(AssertionError, match="biased"):
        sr.assert_unbiased(["bf16"], min_n=N // 2)
    far = (x.view(torch.int32) + 3 * 65536).view(torch.float32).to(torch.bfloat16)
    with SRCheck() as sr:
        sr.target(torch.empty(N, dtype=torch.bfloat16), far)
        with pytest.raises(AssertionError, match="outside the bracket"):
            Q.store_16bit(sr.targets[0][0], x, True)


def _nf4_codes(packed, n):
    p = packed.to(torch.int64)
    return torch.stack([p >> 4, p & 15], 1).reshape(-1)[:n]


def test_nf4_codes_pass_for_oracle_sr_and_catch_floor():
    torch.manual_seed(1003)
    x = _x(3)
    gpu, _ = Q.quant_nf4(x, 2048, None, True)
    with SRCheck() as sr:
        Q.quant_nf4(x, 2048, None, True)
        sr.check_nf4(gpu, N)
    sr.assert_unbiased(["nf4"], min_n=N // 2)
    # planted: always the lower of the two neighbouring codes
    with SRCheck() as sr:
        Q.quant_nf4(x, 2048, None, True)
        b, _ = Q._blocks(x, 2048)
        scale = b.abs().amax(dim=1, keepdim=True).clamp_min(1e-12)
        normed = (b / scale).clamp(-1, 1).reshape(-1)
        lo = (torch.searchsorted(Q.NF4_CODEBOOK[:15], normed).clamp(0, 14) - 1).clamp_min(0)
        lo = torch.where(Q.NF4_CODEBOOK[lo + 1] == normed, lo + 1, lo).clamp_max(14).to(torch.uint8)
        packed = ((lo.view(-1, 2)[:, 0] << 4) | lo.view(-1, 2)[:, 1]).to(torch.uint8)
        sr.check_nf4(packed, N)
    with pytest.raises(AssertionError, match="biased"):
        sr.assert_unbiased(["nf4"], min_n=N // 2)


def test_int8_and_logu8_codes_pass_for_oracle_sr_and_catch_mistakes():
    torch.manual_seed(1004)
    x = _x(4)
    q, _ = Q.quant_int8(x, 2048, None, True)
    v = x.square()
    qv, _ = Q.quant_logu8(v, 512, None, True)
    with SRCheck() as sr:
        Q.quant_int8(x, 2048, None, True)
        sr.check_int8(q)
        Q.quant_logu8(v, 512, None, True)
        sr.check_logu8(qv)
    sr.assert_unbiased(["int8", "logu8"], min_n=N // 2)
    # planted: log-u8 codes rounded down (biased); INT8 codes two away (bracket)
    b, _ = Q._blocks(v, 512)
    c = torch.log2((b / b.amax(dim=1, keepdim=True)).clamp_min(Q.V_MIN_RATIO)) * Q.V_SCALE + 255.0
    floor = c.floor().clamp(1, 255).reshape(-1).to(torch.uint8)
    with SRCheck() as sr:
        Q.quant_logu8(v, 512, None, True)
        sr.check_logu8(floor)
    with pytest.raises(AssertionError, match="biased"):
        sr.assert_unbiased(["logu8"], min_n=N // 2)
    bad = (q.to(torch.int16) + 2).clamp(-127, 127).to(torch.int8)
    with SRCheck() as sr:
        Q.quant_int8(x, 2048, None, True)
        with pytest.raises(AssertionError, match="outside the bracket"):
            sr.check_int8(bad)
