"""Factored second moment and packed 6-bit momentum (CPU oracle; test infrastructure only).

Restates, with torch CPU ops in the reference's order:

* ``quant_6bit`` / ``dequant_6bit`` -- ``_quantize_blockwise_6bit`` /
  ``_dequantize_blockwise_6bit`` (apexw/quantization.py:129-222): codes
  round(x / scale) clamped to +-31, stored as code + 31, four codes in three
  bytes (little-endian 24-bit words); scale = max(absmax (>= 1e-12) / 31,
  0.9 * old); the tensor is padded to whole blocks and quads;
* ``factored_update`` -- ``_apply_factored_v_int8_update`` for contiguous
  tensors (apexw/state.py:442-608) with ``_compute_factored_v_denom``
  (:313-337) and ``_apply_factored_v_chunk_body`` (:360-439): the fp32 grad
  (nan_to_num, AMP unscale), row / column EMAs of g^2 (tensors above 262,144
  elements sum the columns over row chunks and scale by (1-b2)/rows),
  den = max(sqrt(row / mean(row)) sqrt(col) + eps_scaled, eps), m = lerp(m, g,
  1-b1) dequantized from INT8 / 6-bit or read from a 16-bit tensor,
  p = p * wd - (m / den) * step_size, and the block requantization.  The
  update chunks of the reference are whole blocks, so stepping the tensor in
  one piece gives the same values.

Parity pins (tests/test_oracle_factored.py): the reference's own 6-bit
round-trip test; pack / unpack against a brute-force bit layout; the zero fill
[0xDF, 0xF7, 0x7D]; a first step from zero state against its closed form
(row / column means, the normalised denominator), for both the one-piece and
the row-chunked statistics; the chunked and one-piece statistics agree to fp32
rounding.
"""

import torch

from . import quant as Q

CHUNK = 262144  # _FACTORED_CHUNK_ELEMS


def _pad_blocks(x, block):
    n = x.numel()
    pad = (block - n % block) % block
    padded = n + pad
    rem4 = (4 - padded % 4) % 4
    return torch.nn.functional.pad(x.reshape(-1).float(), (0, pad + rem4)), n


def quant_6bit(x, block, old_scales=None, stochastic=False):
    flat, n = _pad_blocks(x, block)
    blocks = flat.view(-1, block)
    scale = blocks.abs().amax(dim=1, keepdim=True).clamp_min(1e-12) / 31.0
    if old_scales is not None:
        scale = torch.maximum(scale, old_scales.view(-1, 1).float() * 0.9)
    y = blocks / scale
    if stochastic:
        y = y + (torch.rand(y.shape) - 0.5)
    u = y.round().clamp(-31.0, 31.0).add(31.0).to(torch.uint8).reshape(-1, 4)
    packed = torch.empty((u.shape[0], 3), dtype=torch.uint8)
    u0, u1, u2, u3 = u[:, 0], u[:, 1], u[:, 2], u[:, 3]
    packed[:, 0] = (u0 & 0x3F) | ((u1 & 0x03) << 6)
    packed[:, 1] = ((u1 >> 2) & 0x0F) | ((u2 & 0x0F) << 4)
    packed[:, 2] = ((u2 >> 4) & 0x03) | ((u3 & 0x3F) << 2)
    return packed.view(-1), scale


def dequant_6bit(q, scales, numel, block):
    packed = q.view(-1, 3)
    b0, b1, b2 = packed[:, 0], packed[:, 1], packed[:, 2]
    u = torch.empty((packed.shape[0], 4), dtype=torch.uint8)
    u[:, 0] = b0 & 0x3F
    u[:, 1] = ((b0 >> 6) & 0x03) | ((b1 & 0x0F) << 2)
    u[:, 2] = ((b1 >> 4) & 0x0F) | ((b2 & 0x03) << 4)
    u[:, 3] = (b2 >> 2) & 0x3F
    deq = (u.reshape(-1, block).float() - 31.0) * scales.view(-1, 1).float()
    return deq.reshape(-1)[:numel]


def _prep(g, sanitize, inv_scale):
    gc = g.reshape(-1).float().clone()
    if sanitize:
        gc.nan_to_num_(nan=0.0, posinf=65504.0, neginf=-65504.0)
    if inv_scale is not None:
        gc.mul_(inv_scale)
    return gc


@torch.no_grad()
def factored_update(p, g, st, *, beta1, beta2, step_size, eps_scaled, eps, stochastic, block_size,
                    wd_factor=None, inv_scale=None, sanitize=True):
    """One step of a factored-v parameter ``p`` (contiguous) with grad ``g``."""
    r, c = st["exp_avg_sq_row"], st["exp_avg_sq_col"]
    rows, cols = r.numel(), c.numel()
    n = p.numel()
    gf = _prep(g, sanitize, inv_scale)
    if n <= CHUNK:
        g_sq = gf.view(rows, cols).square()
        r.mul_(beta2).add_(g_sq.mean(dim=1), alpha=1.0 - beta2)
        c.mul_(beta2).add_(g_sq.mean(dim=0), alpha=1.0 - beta2)
    else:
        r_step = max(1, CHUNK // cols)
        c_acc = torch.zeros(cols, dtype=torch.float32)
        for r0 in range(0, rows, r_step):
            r1 = min(r0 + r_step, rows)
            g_sq = gf[r0 * cols:r1 * cols].view(r1 - r0, cols).square()
            r[r0:r1].mul_(beta2).add_(g_sq.mean(dim=1), alpha=1.0 - beta2)
            c_acc.add_(g_sq.sum(dim=0))
        c.mul_(beta2).add_(c_acc, alpha=(1.0 - beta2) / rows)
    r.nan_to_num_(nan=0.0, posinf=0.0, neginf=0.0)
    c.nan_to_num_(nan=0.0, posinf=0.0, neginf=0.0)
    inv_r_mean = 1.0 / r.mean().clamp_min_(1e-30)
    row_norm = (r * inv_r_mean).sqrt()
    den = (row_norm.unsqueeze(1) * c.sqrt().unsqueeze(0)).add_(eps_scaled).clamp_min_(eps).reshape(-1)
    m = st["exp_avg"]
    ms = st.get("exp_avg_scales")
    six = bool(st.get("is_6bit_m", False))
    int8 = not six and m.dtype == torch.int8
    if six:
        mf = dequant_6bit(m, ms, n, block_size)
    elif int8:
        mf = Q.dequant_int8(m.reshape(-1), ms, block_size)
    else:
        mf = m.reshape(-1).float()
    mf.lerp_(gf, 1.0 - beta1)
    upd = torch.div(mf, den).mul_(step_size)
    pf = p.view(-1)
    if p.dtype == torch.float32:
        if wd_factor is not None:
            pf.mul_(wd_factor)
        pf.sub_(upd)
    elif p.dtype == torch.float16:
        # apexw/state.py:405-410: decay and update in fp32, clamped to fp16's range,
        # one rounding
        pw = pf.float()
        if wd_factor is not None:
            pw.mul_(wd_factor)
        pw.sub_(upd).clamp_(-65504.0, 65504.0)
        pf.copy_(pw.to(torch.float16))
    else:
        if wd_factor is not None:
            pf.mul_(wd_factor)
        pf.sub_(upd.to(p.dtype))
    if six:
        q, s = quant_6bit(mf, block_size, ms, stochastic)
        m.copy_(q)
        ms.copy_(s)
    elif int8:
        q, s = Q.quant_int8(mf, block_size, ms, stochastic)
        m.copy_(q.view(m.shape))
        ms.copy_(s)
    else:
        m.copy_(mf.view(m.shape).to(m.dtype))


def first_step_closed_form(p, g, *, lr, beta1, beta2, eps, weight_decay):
    """A first factored step from zero state in float64: row / column means of
    g^2, the mean-normalised row factor, m = (1-b1) g, and decay on (2-D)."""
    G = g.double()
    rows = G.shape[0]
    G2 = G.reshape(rows, -1) ** 2
    r = (1.0 - beta2) * G2.mean(dim=1)
    c = (1.0 - beta2) * G2.mean(dim=0)
    den = ((r / r.mean()).sqrt().unsqueeze(1) * c.sqrt().unsqueeze(0) + eps * (1.0 - beta2) ** 0.5)
    den = den.clamp_min(eps).reshape(G.shape)
    m = (1.0 - beta1) * G
    s = lr * (1.0 - beta2) ** 0.5 / (1.0 - beta1)
    return p.double() * max(1.0 - lr * weight_decay, 0.0) - s * m / den, r, c
