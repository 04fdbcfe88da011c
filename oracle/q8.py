"""8-bit AdamW step (CPU oracle; test infrastructure only).

Restates ``ApexW._step_ultra`` (``apexw/optimizer.py:4313-4735``) for
``precision="8bit"`` with the standard update, ``nesterov=True``,
``cautious=True`` or ``maximize=True`` (no amsgrad / lion / AdEMAMix), per parameter:

* large contiguous quantized tensors (numel > 262144) use the chunked path,
  optimizer.py:4402-4499 -- decay and update fused in fp32, one rounding of p;
* other quantized tensors use the generic path, optimizer.py:4538-4639 -- decay
  rounded into p first, then ``p -= bf16(update)`` (SR only for quad-v);
* tensors with fewer than 64 elements keep 16-bit m/v, optimizer.py:4688-4735.

``precision="ultra"`` runs the same function (optimizer.py:3583-3587): 2-D or
large tensors hold INT8 m and a dense 16-bit (or fp32) v, updated without the
lookahead gain and without the eps floor (:4640-4686); the others keep fp32
m/v and take the dense branch above.

The update is AdamW with the "Nesterov-SNR" lookahead gain: ``m_look =
lerp(g, m, b1)``, gain ``1+0.2*b1`` where ``m*g >= 0`` else ``1-0.35*b1``.
With ``nesterov=True`` the numerator is ``lerp(g, m, b1)`` without the gain in the
quantized branches (optimizer.py:4444-4445, :4581-4582), and replaces ``m`` in the
dense and ultra ones (:4667-4670, :4719-4724).  With ``cautious=True`` no tensor
takes the chunked path (:4402-4414), the numerator is ``m`` and it is multiplied
by ``mask / mask.mean().clamp(min=1e-3)``, ``mask = num * g >= 0`` over the whole
tensor (:4585-4588, :4672-4675, :4726-4729).
"""

import math

import torch

from . import quant as Q
from .factored import factored_update

CHUNK = 262144  # _FACTORED_CHUNK_ELEMS, state.py:44


def _bias(lr, beta1, beta2, eps, step):
    bc1 = 1.0 - beta1 ** step
    bc2 = 1.0 - beta2 ** step
    s = math.sqrt(bc2)
    return lr * s / bc1, eps * s


def _cautious(num, g):
    """num * (mask / mean(mask)), mask = num * g >= 0 as float32 (optimizer.py:4585-4588)."""
    mask = (num * g >= 0).to(torch.float32)
    return num * (mask / mask.mean().clamp(min=1e-3))


def _snr_num(m, g, beta1, nesterov=False, cautious=False):
    if cautious:
        return _cautious(m, g)
    if nesterov:
        return torch.lerp(g, m, beta1)
    gain_hi = 1.0 + 0.20 * beta1
    gain_lo = 1.0 - 0.35 * beta1
    look = torch.lerp(g, m, beta1)
    return look.mul_(torch.where(m * g >= 0.0, gain_hi, gain_lo))


def q8_param_step(p, g, st, *, lr, beta1, beta2, eps, weight_decay, decay_norm_only, step, inv_scale=None,
                  nesterov=False, cautious=False, maximize=False):
    """Update one parameter and its state in place.  ``step`` is already incremented.
    maximize: the grad is negated after nan_to_num, before the unscale
    (optimizer.py:4500-4505; state.py:341-346 in the chunked order)."""
    if maximize:
        # negation is exact and commutes with nan_to_num's +-65504 and the unscale, so the
        # grads can be negated once here for every branch below
        g = -g
    step_size, eps_scaled = _bias(lr, beta1, beta2, eps, step)
    decay = max(1.0 - lr * weight_decay, 0.0) if weight_decay != 0 else 1.0
    apply_wd = weight_decay != 0 and (not decay_norm_only or p.dim() >= 2)
    sr = st.get("stochastic_rounding", True)
    n = p.numel()
    if st.get("is_factored_v", False):              # optimizer.py:4380-4400
        factored_update(p, g, st, beta1=beta1, beta2=beta2, step_size=step_size, eps_scaled=eps_scaled, eps=eps,
                        stochastic=sr, block_size=st.get("block_size_8bit", 256),
                        wd_factor=decay if apply_wd else None, inv_scale=inv_scale, sanitize=True)
        return
    if st.get("is_ultra", False):
        _ultra(p, g, st, beta1, beta2, step_size, eps_scaled, decay if apply_wd else None, sr, inv_scale, nesterov,
               cautious)
        return
    if st.get("is_8bit", False) and n > CHUNK and p.is_contiguous() and not cautious:
        _chunked(p, g, st, beta1, beta2, eps, step_size, eps_scaled, decay if apply_wd else None, sr, inv_scale,
                 nesterov)
        return
    gf = torch.nan_to_num(g, nan=0.0, posinf=65504.0, neginf=-65504.0).float()
    if inv_scale is not None:                           # AMP: optimizer.py:4504-4505
        gf.mul_(inv_scale)
    if apply_wd:
        p.mul_(decay)
    if st.get("is_8bit", False):
        bs = st["block_size_8bit"]
        int4 = st.get("is_4bit_m", False)
        quad = bool(st.get("is_quad_v", False))
        if int4:
            m = Q.dequant_nf4(st["exp_avg"], st["exp_avg_scales"], n, bs).view(p.shape)
        else:
            m = Q.dequant_int8(st["exp_avg"], st["exp_avg_scales"], bs)
        m.lerp_(gf, 1.0 - beta1)
        if quad:
            vbs = max(1, bs // 4)
            v = Q.dequant_logu8(st["exp_avg_sq"], st["exp_avg_sq_scales"], vbs)
            gq = gf.reshape(-1, 4).square().mean(dim=1)
            v.mul_(beta2).add_(gq, alpha=1.0 - beta2)
            v.nan_to_num_(nan=0.0, posinf=0.0, neginf=0.0)
            den = v.sqrt().add_(eps_scaled).clamp_min_(eps).unsqueeze(1).expand(-1, 4).reshape(p.shape)
        else:
            vbs = bs
            v = Q.dequant_logu8(st["exp_avg_sq"], st["exp_avg_sq_scales"], bs)
            v.mul_(beta2).addcmul_(gf, gf, value=1.0 - beta2)
            v.nan_to_num_(nan=0.0, posinf=0.0, neginf=0.0)
            den = v.sqrt().add_(eps_scaled).clamp_min_(eps)
        num = _snr_num(m, gf, beta1, nesterov, cautious)
        if p.dtype == torch.float32:
            p.addcdiv_(num, den, value=-step_size)
        else:
            upd = (num / den).mul_(step_size)
            if quad and sr:
                Q.store_16bit(p, p.float().sub_(upd), True)
            else:
                p.sub_(upd.to(p.dtype))
        if int4:
            q, s = Q.quant_nf4(m, bs, st["exp_avg_scales"], sr)
        else:
            q, s = Q.quant_int8(m, bs, st["exp_avg_scales"], sr)
        st["exp_avg"].copy_(q.view(st["exp_avg"].shape))
        st["exp_avg_scales"].copy_(s)
        qv, sv = Q.quant_logu8(v, vbs, st["exp_avg_sq_scales"], sr)
        st["exp_avg_sq"].copy_(qv.view(st["exp_avg_sq"].shape))
        st["exp_avg_sq_scales"].copy_(sv)
        return
    # tiny tensors: 16-bit (or fp32) m and v, fp32 math
    m, v = st["exp_avg"], st["exp_avg_sq"]
    mf = m.float().lerp_(gf, 1.0 - beta1)
    m.copy_(mf.to(m.dtype))
    vf = v.float().mul_(beta2).addcmul_(gf, gf, value=1.0 - beta2)
    v.copy_(vf.to(v.dtype))
    den = vf.sqrt().add_(eps_scaled)
    num = torch.lerp(gf, mf, beta1) if nesterov else mf
    if cautious:
        num = _cautious(num, gf)
    upd = (num / den).mul_(step_size)
    p.sub_(upd.to(p.dtype))


def _chunked(p, g, st, beta1, beta2, eps, step_size, eps_scaled, decay, sr, inv_scale=None, nesterov=False):
    n = p.numel()
    bs = st["block_size_8bit"]
    int4 = st.get("is_4bit_m", False)
    mbuf, vbuf = st["exp_avg"].reshape(-1), st["exp_avg_sq"].reshape(-1)
    msc, vsc = st["exp_avg_scales"], st["exp_avg_sq_scales"]
    quad = bool(st.get("is_quad_v", False)) or (int4 and n % 4 == 0 and vbuf.numel() * 4 == n)
    vbs = max(1, bs // 4) if quad else bs
    step_elems = max(CHUNK // bs, 1) * bs
    pf_all, gf_all = p.reshape(-1), g.reshape(-1)
    for off in range(0, n, step_elems):
        end = min(off + step_elems, n)
        blk0, last = off // bs, end >= n
        sl = slice(blk0, None) if last else slice(blk0, blk0 + (end - off) // bs)
        sm, sv = msc[sl], vsc[sl]
        gc = gf_all[off:end].float().nan_to_num_(nan=0.0, posinf=65504.0, neginf=-65504.0)
        if inv_scale is not None:                       # AMP: _prep_grad_chunk_fp32, state.py:326-347
            gc.mul_(inv_scale)
        if int4:
            msl = mbuf[off // 2:(end + 1) // 2]
            m = Q.dequant_nf4(msl, sm, end - off, bs)
        else:
            msl = mbuf[off:end]
            m = Q.dequant_int8(msl, sm, bs)
        m.lerp_(gc, 1.0 - beta1)
        num = _snr_num(m, gc, beta1, nesterov)
        if quad:
            vsl = vbuf[off // 4:end // 4]
            v = Q.dequant_logu8(vsl, sv, vbs)
            v.mul_(beta2).add_(gc.view(-1, 4).square().mean(dim=1), alpha=1.0 - beta2)
            v.nan_to_num_(nan=0.0, posinf=0.0, neginf=0.0)
            den = v.sqrt().add_(eps_scaled).clamp_min_(eps)
            num.view(-1, 4).div_(den.unsqueeze(1))
            upd = num.mul_(step_size)
        else:
            vsl = vbuf[off:end]
            v = Q.dequant_logu8(vsl, sv, bs)
            v.mul_(beta2).addcmul_(gc, gc, value=1.0 - beta2)
            v.nan_to_num_(nan=0.0, posinf=0.0, neginf=0.0)
            den = v.sqrt().add_(eps_scaled).clamp_min_(eps)
            upd = torch.div(num, den).mul_(step_size)
        psl = pf_all[off:end]
        if p.dtype == torch.float32:
            if decay is not None:
                psl.mul_(decay)
            psl.sub_(upd)
        else:
            x = psl.float()
            if decay is not None:
                x.mul_(decay)
            Q.store_16bit(psl, x.sub_(upd), sr)
        if int4:
            q, s = Q.quant_nf4(m, bs, sm, sr)
        else:
            q, s = Q.quant_int8(m, bs, sm, sr)
        msl.copy_(q.view(msl.shape))
        sm.copy_(s)
        qv, s2 = Q.quant_logu8(v, vbs, sv, sr)
        vsl.copy_(qv.view(vsl.shape))
        sv.copy_(s2)


def _ultra(p, g, st, beta1, beta2, step_size, eps_scaled, decay, sr, inv_scale, nesterov=False, cautious=False):
    """optimizer.py:4500-4511, :4640-4686: INT8 m (block ``ultra_block_size``,
    EMA-max scales), dense v rounded to its dtype once, the denominator from the
    unrounded fp32 v, p decayed then ``p -= update.to(p.dtype)``."""
    gf = torch.nan_to_num(g, nan=0.0, posinf=65504.0, neginf=-65504.0).float()
    if inv_scale is not None:
        gf.mul_(inv_scale)
    if decay is not None:
        p.mul_(decay)
    bs = st.get("block_size_8bit", st.get("ultra_block_size", 256))
    m = Q.dequant_int8(st["exp_avg"], st["exp_avg_scales"], bs)
    m.lerp_(gf, 1.0 - beta1)
    v = st["exp_avg_sq"]
    vf = v.float().mul_(beta2).addcmul_(gf, gf, value=1.0 - beta2)
    v.copy_(vf.to(v.dtype))
    den = vf.sqrt().add_(eps_scaled)
    num = torch.lerp(gf, m, beta1) if nesterov else m
    if cautious:
        num = _cautious(num, gf)
    upd = (num / den).mul_(step_size)
    p.sub_(upd.to(p.dtype))
    q, s = Q.quant_int8(m, bs, st["exp_avg_scales"], sr)
    st["exp_avg"].copy_(q.view(st["exp_avg"].shape))
    st["exp_avg_scales"].copy_(s)
