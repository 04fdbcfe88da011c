"""Blockwise quantizers and 16-bit stochastic rounding (CPU oracle; test infrastructure only).

Restates the reference's quantization module (``apexw/quantization.py``) with
torch CPU ops, keeping its arithmetic order:

* NF4 4-bit momentum codes      -- quantization.py:224-357
* INT8 momentum codes           -- quantization.py:66-126
* 24-octave log-uint8 variance  -- quantization.py:360-448
* fp32 -> bf16/fp16 stochastic rounding -- quantization.py:451-482

Noise for stochastic rounding comes from torch's global RNG (fresh draws; the
reference additionally recycles a cached pool for small tensors, which changes
which random numbers are used but not their distribution).
"""

import math

import torch

# NF4 codebook (quantization.py:225-233): symmetric levels, index 7 is exactly 0,
# index 15 repeats +1.0 so that a 4-bit code never decodes out of range.
_NF4_LEVELS = (-1.0, -0.6962, -0.5251, -0.3949, -0.2844, -0.1848, -0.0911, 0.0,
               0.0911, 0.1848, 0.2844, 0.3949, 0.5251, 0.6962, 1.0, 1.0)
NF4_CODEBOOK = torch.tensor(_NF4_LEVELS, dtype=torch.float32)
# Decision boundaries between consecutive codes 0..14, in fp32 (quantization.py:235-236).
NF4_MIDS = ((NF4_CODEBOOK[:15] + NF4_CODEBOOK[1:16]) / 2.0)[:14].clone()
# byte -> (high-nibble value, low-nibble value) (quantization.py:260-263).
NF4_PAIR = torch.stack([NF4_CODEBOOK[torch.arange(256) >> 4], NF4_CODEBOOK[torch.arange(256) & 15]], dim=1)

# log-uint8 variance code q in 1..255 decodes to 2^((q-1)*24/254 - 24) (quantization.py:360-367),
# evaluated in double and stored as fp32; code 0 decodes to 0.
V_BITS = 24.0
V_SCALE = 254.0 / V_BITS
V_MIN_RATIO = 2.0 ** (-V_BITS)
V_LOG_LUT = torch.tensor([0.0] + [2.0 ** ((q - 1) * (V_BITS / 254.0) - V_BITS) for q in range(1, 256)],
                         dtype=torch.float32)


def _blocks(x, block):
    """Flatten to [n_blocks, block] fp32, zero-padding the tail block."""
    n = x.numel()
    pad = (-n) % block
    flat = x.reshape(-1).float()
    if pad:
        flat = torch.nn.functional.pad(flat, (0, pad))
    return flat.view(-1, block), n


def _uniform_pm_half(shape):
    return torch.rand(shape, dtype=torch.float32) - 0.5


def quant_int8(x, block, old_scales=None, stochastic=False):
    """INT8 codes with EMA-max scales: scale = max(absmax/127, 0.9*old)."""
    b, n = _blocks(x, block)
    scale = b.abs().amax(dim=1, keepdim=True).clamp_min(1e-12) / 127.0
    if old_scales is not None:
        scale = torch.maximum(scale, old_scales.view(-1, 1).float() * 0.9)
    y = b / scale
    if stochastic:
        y = y + _uniform_pm_half(y.shape)
    q = y.round().clamp(-127, 127).to(torch.int8)
    return q.view(-1)[:n].view(x.shape), scale


def dequant_int8(q, scales, block):
    b, n = _blocks(q, block)
    return (b * scales.view(-1, 1).float()).view(-1)[:n].view(q.shape)


def quant_nf4(x, block, old_scales=None, stochastic=False):
    """NF4 codes packed two per byte (even element in the high nibble), absmax scales."""
    b, n = _blocks(x, block)
    scale = b.abs().amax(dim=1, keepdim=True).clamp_min(1e-12)
    if old_scales is not None:
        scale = torch.maximum(scale, old_scales.view(-1, 1).float() * 0.9)
    normed = (b / scale).clamp(-1.0, 1.0).reshape(-1)
    if stochastic:
        levels = NF4_CODEBOOK[:15]
        hi = torch.searchsorted(levels, normed).clamp(0, 14)
        lo = (hi - 1).clamp_min(0)
        c_lo, c_hi = levels[lo], levels[hi]
        gap = c_hi - c_lo
        p_hi = torch.where(gap > 0, (normed - c_lo) / gap.clamp_min(1e-12), torch.ones_like(normed))
        u = torch.rand(normed.shape, dtype=torch.float32)
        codes = torch.where(u < p_hi, hi, lo)
    else:
        codes = torch.searchsorted(NF4_MIDS, normed).clamp(0, 14)
    codes = codes.to(torch.uint8)[:n]
    if n % 2:
        codes = torch.nn.functional.pad(codes, (0, 1), value=7)
    pairs = codes.view(-1, 2)
    return ((pairs[:, 0] << 4) | pairs[:, 1]).to(torch.uint8), scale


def dequant_nf4(packed, scales, numel, block):
    flat = NF4_PAIR[packed.long()].reshape(-1)[:numel]
    b, n = _blocks(flat, block)
    return (b * scales.view(-1, 1).float()).view(-1)[:n]


def quant_logu8(v, block, old_scales=None, stochastic=False):
    """24-octave log-uint8 codes of a non-negative tensor, block-max scales (EMA 0.95)."""
    b, n = _blocks(v, block)
    b = torch.nan_to_num(b, nan=0.0, posinf=0.0, neginf=0.0)
    vmax = b.amax(dim=1, keepdim=True).clamp_min(1e-12).nan_to_num(nan=1.0, posinf=1.0)
    if old_scales is not None:
        vmax = torch.maximum(vmax, old_scales.view(-1, 1).float() * 0.95)
    r = (b / vmax).clamp_min(V_MIN_RATIO)
    qf = torch.log2(r).mul_(V_SCALE).add_(255.0)
    if stochastic:
        qf = qf.add_(_uniform_pm_half(qf.shape))
    q = qf.round_().clamp_(1.0, 255.0).to(torch.uint8)
    q.masked_fill_(b <= 0, 0)
    return q.view(-1)[:n].view(v.shape), vmax


def dequant_logu8(q, scales, block):
    b, n = _blocks(q, block)
    return (V_LOG_LUT[b.long()] * scales.view(-1, 1).float()).view(-1)[:n].view(q.shape)


def store_16bit(dst, src_f32, stochastic):
    """Write fp32 values into a bf16/fp16/fp32 tensor; 16-bit targets use SR when asked.

    bf16 SR adds a uniform integer in [0, 2^16) to the fp32 bit pattern and
    truncates the low 16 bits; fp16 SR does the same with 13 bits after clamping to
    the fp16 range (quantization.py:451-482).
    """
    if dst.dtype == torch.float32:
        dst.copy_(src_f32)
        return
    if not stochastic:
        if dst.dtype == torch.float16:
            src_f32 = src_f32.clamp(-65504.0, 65504.0)
        dst.copy_(src_f32.to(dst.dtype))
        return
    x = src_f32.float().clone().contiguous()
    bits = x.view(-1).view(torch.int32)
    if dst.dtype == torch.float16:
        x.clamp_(-65504.0, 65504.0)
        bits.add_(torch.randint(0, 8192, bits.shape, dtype=torch.int32)).bitwise_and_(-8192)
        x.clamp_(-65504.0, 65504.0)
        dst.copy_(x.to(torch.float16))
    else:
        bits.add_(torch.randint(0, 65536, bits.shape, dtype=torch.int32)).bitwise_and_(-65536)
        dst.copy_(x.to(torch.bfloat16))


def nf4_midpoint(k):
    """Decision boundary between NF4 codes k and k+1 (fp32), for known-answer tests."""
    return float(NF4_MIDS[k])


def logu8_code_exact(r):
    """Real-valued log-u8 code of ratio r (double), the closed form the quantizer rounds."""
    return math.log2(max(r, V_MIN_RATIO)) * V_SCALE + 255.0
