"""In-backward steps (CPU oracle; test infrastructure only).

Restates the reference's automatic 8-bit runtime acceleration and its
``enable_fused_backward`` per-parameter update:

* ``hook_partition`` -- which parameters are stepped during backward
  (``_enable_8bit_runtime_acceleration``, apexw/optimizer.py:2076-2133): the
  8-bit trainable tensors, enabled with >= 8 of them and >= 524,288 elements;
  fp32 tensors of >= 1024 elements become bf16; tensors of >= 16384 elements
  other than the first are hooked, the first is the anchor;
* ``ensure_8bit_state`` -- the lazily created state
  (``_ensure_8bit_state_initialized``, optimizer.py:2169-2224);
* ``flush_8bit`` -- one flushed batch (``_flush_auto_8bit_hook_queue``,
  optimizer.py:2226-2371), on the path the reference takes without its CUDA
  extension: ``_step_ultra`` with lr * K^-0.4, weight decay wd / (K * K^-0.4),
  the grad scale 1 / (amp_inv * K) as a float32 tensor, and the step counter set
  so that the bias correction uses the pass count (mstep) and the stored
  counter ends at (mstep - 1) // K + 1;
* ``fused_param_step`` -- ``_step_single_param_fused`` (optimizer.py:2373-2471),
  the update ``enable_fused_backward`` runs per parameter: fp32 moments
  (m = b1 m + (1-b1) g), lookahead b1 m' + (1-b1) g with the new m, no grad
  sanitizing, a denominator sqrt(v) + eps_scaled without the eps floor, INT8 m
  requantised from its own absmax (no EMA, round to nearest); the compact
  branch keeps full-size fp32-math moments rounded once on store.

Parity pins (tests/test_oracle_hooks.py): with K = 1 and no AMP a flush equals
the ordinary 8-bit step of ``OracleApexW`` bit for bit; a first step from zero
state with K = 2 and a large eps matches the closed form of the update (which
depends on the grad scale K, on lr * K^-0.4 and on the decay lr * wd / K); an
AMP scale that is a power of two cancels exactly; the state layout equals the
golden-pinned ``layout.init_state`` wherever the two rules coincide;
``fused_param_step`` matches the closed form of a first step from zero state
(8-bit and compact, where a large eps shows the missing floor) and, on a second
step, the INT8 scale equals the new momentum's absmax / 127 (no EMA).
"""

import numpy as np
import torch

from . import layout as L
from . import quant as Q
from .q8 import q8_param_step

MIN_TENSORS = 8
MIN_NUMEL = 524_288
DOWNCAST_MIN_NUMEL = 1024
HOOK_MIN_NUMEL = 16384
BATCH = 14


def hook_partition(params):
    """(enabled, anchor, hooked) for one 8-bit group's trainable tensors in order."""
    trainable = [p for p in params if p.requires_grad and not torch.is_complex(p) and p.dtype != torch.float64]
    if len(trainable) < MIN_TENSORS or sum(p.numel() for p in trainable) < MIN_NUMEL:
        return False, None, []
    return True, trainable[0], [p for p in trainable[1:] if p.numel() >= HOOK_MIN_NUMEL]


def downcast_dtype(p):
    """bf16 for fp32 tensors of >= 1024 elements (devices with bf16), else unchanged."""
    return torch.bfloat16 if p.dtype == torch.float32 and p.numel() >= DOWNCAST_MIN_NUMEL else p.dtype


def ensure_8bit_state(st, p, group):
    if "exp_avg" in st and "exp_avg_sq" in st:
        return st
    n = p.numel()
    st["stochastic_rounding"] = bool(group.get("stochastic_rounding", True))
    st["step"] = torch.tensor(0.0, dtype=torch.float32)
    st["is_8bit"] = True
    bs = L.block_size_8bit(p, group.get("block_size"))
    st["block_size_8bit"] = bs
    st["is_factored_v"] = False
    st["is_6bit_m"] = False
    raw_int4 = group.get("int4_m")
    pow2 = bs >= 64 and (bs & (bs - 1)) == 0
    sub = (raw_int4 is not False and n >= 16384 and n % 4 == 0 and pow2
           and (p.dim() < 2 or min(p.shape) >= 8))
    st["is_4bit_m"] = sub
    st["is_quad_v"] = sub
    st["m_numel"] = n
    st["state_dtype"] = torch.int8
    st["state_dtype_v"] = torch.uint8
    nblk = (n + bs - 1) // bs
    if sub:
        st["exp_avg"] = torch.full(((n + 1) // 2,), 0x77, dtype=torch.uint8)
        st["exp_avg_scales"] = torch.full((nblk, 1), 1e-12, dtype=torch.float32)
        st["exp_avg_sq"] = torch.zeros((n // 4,), dtype=torch.uint8)
    else:
        st["exp_avg"] = torch.zeros(p.shape, dtype=torch.int8)
        st["exp_avg_scales"] = torch.full((nblk, 1), 1e-12 / 127.0, dtype=torch.float32)
        st["exp_avg_sq"] = torch.zeros(p.shape, dtype=torch.uint8)
    st["exp_avg_sq_scales"] = torch.full((nblk, 1), 1e-12, dtype=torch.float32)
    return st


@torch.no_grad()
def flush_8bit(params, grads, states, group, K=1, amp_scale=None):
    """Step ``params`` (CPU tensors) with their ``grads``; ``states`` maps each
    parameter to its state dict (created when missing)."""
    K = max(1, int(K))
    mult = 1.0 if K == 1 else K ** -0.40
    amp_inv = 1.0 / amp_scale if (amp_scale is not None and amp_scale > 0.0) else 1.0
    inv_scale = amp_inv * float(K)
    lr_eff = float(group["lr"]) * mult
    wd = float(group["weight_decay"])
    wd_eff = wd / (float(K) * mult) if wd != 0.0 else 0.0
    b1, b2 = group["betas"]
    inv = None
    if inv_scale != 1.0:
        grad_scale = torch.tensor(1.0 / inv_scale)          # float32, as _step_ultra receives it
        inv = float(grad_scale.reciprocal().item())
    for p, g in zip(params, grads):
        st = ensure_8bit_state(states.setdefault(p, {}), p, group)
        mstep = st.get("_hook_mstep", 0) + 1
        st["_hook_mstep"] = mstep
        q8_param_step(p, g.to(p.dtype), st, lr=lr_eff, beta1=b1, beta2=b2, eps=float(group["eps"]),
                      weight_decay=wd_eff, decay_norm_only=bool(group.get("decay_norm_only", True)),
                      step=mstep, inv_scale=inv, cautious=bool(group.get("cautious", False)))
        st["step"].fill_(float((mstep - 1) // K + 1))


def first_step_closed_form(p, g, *, lr, beta1, beta2, eps, weight_decay, K, amp_scale=None):
    """The first 8-bit step from zero state of a generic-path tensor (INT8 m, full
    v, fp32 p; no chunking), in float64 from the AdamW + lookahead-gain formulas.
    Zero state dequantizes to exact zeros, so quantization does not enter."""
    mult = 1.0 if K == 1 else K ** -0.40
    G = g.double() * (float(K) / (amp_scale if amp_scale else 1.0))
    lr_eff = lr * mult
    wd_eff = weight_decay / (K * mult)
    decay = 1.0 - lr_eff * wd_eff if weight_decay else 1.0
    m = (1.0 - beta1) * G
    v = (1.0 - beta2) * G * G
    look = beta1 * m + (1.0 - beta1) * G
    gain = np.where((m * G >= 0).numpy(), 1.0 + 0.20 * beta1, 1.0 - 0.35 * beta1)
    bc1, bc2 = 1.0 - beta1, 1.0 - beta2
    step_size = lr_eff * bc2 ** 0.5 / bc1
    den = torch.clamp(v.sqrt() + eps * bc2 ** 0.5, min=eps)
    apply_wd = p.dim() >= 2
    base = p.double() * (decay if apply_wd else 1.0)
    return base - step_size * look * torch.from_numpy(gain) / den


@torch.no_grad()
def fused_param_step(p, g, st, group):
    """One in-backward update of ``p`` with grad ``g``; ``st`` is its state dict."""
    prec = group["precision"]
    if len(st) == 0:
        if prec == "8bit":
            ensure_8bit_state(st, p, group)
        else:
            st["stochastic_rounding"] = bool(group.get("stochastic_rounding", True))
            st["step"] = torch.tensor(0.0, dtype=torch.float32)
            cdt = L.compact_dtype(p) if prec == "compact" else torch.float32
            st["exp_avg"] = torch.zeros_like(p, dtype=cdt)
            st["exp_avg_sq"] = torch.zeros_like(p, dtype=cdt)
    st["step"].add_(1)
    step = int(st["step"].item())
    lr, (b1, b2), wd, eps = group["lr"], group["betas"], group["weight_decay"], group["eps"]
    apply_wd = wd != 0 and (not group.get("decay_norm_only", True) or p.dim() >= 2)
    wd_factor = max(1.0 - lr * wd, 0.0) if apply_wd else 1.0
    bc1 = 1.0 - b1 ** step
    bc2 = 1.0 - b2 ** step
    step_size = lr * bc2 ** 0.5 / bc1
    eps_scaled = eps * bc2 ** 0.5
    if st.get("is_8bit", False):
        m, v = st["exp_avg"], st["exp_avg_sq"]
        ms, vs = st["exp_avg_scales"], st["exp_avg_sq_scales"]
        bs = st["block_size_8bit"]
        stoch = st.get("stochastic_rounding", True)
        int4, quad = st.get("is_4bit_m", False), st.get("is_quad_v", False)
        if int4:
            mf = Q.dequant_nf4(m, ms, p.numel(), bs).view_as(p)
        else:
            mf = Q.dequant_int8(m, ms, bs)
        vbs = max(bs // 4, 1) if quad else bs
        vf = Q.dequant_logu8(v, vs, vbs)
        gf = g.to(torch.float32)
        mf.mul_(b1).add_(gf, alpha=1.0 - b1)
        if quad:
            gq = gf.reshape(-1, 4).square().mean(dim=1)
            vf.mul_(b2).add_(gq, alpha=1.0 - b2)
            den = vf.sqrt().add_(eps_scaled).unsqueeze(1).expand(-1, 4).reshape_as(p)
        else:
            vf.mul_(b2).addcmul_(gf, gf, value=1.0 - b2)
            den = vf.sqrt().add_(eps_scaled)
        look = mf.mul(b1).add_(gf, alpha=1.0 - b1)
        look.mul_(torch.where(mf * gf >= 0, 1.0 + 0.20 * b1, 1.0 - 0.35 * b1))
        if p.dtype == torch.float32:
            if apply_wd:
                p.mul_(wd_factor)
            p.addcdiv_(look, den, value=-step_size)
        else:
            pf = p.float()
            if apply_wd:
                pf.mul_(wd_factor)
            pf.addcdiv_(look, den, value=-step_size)
            Q.store_16bit(p, pf, stoch)
        if int4:
            q, sc = Q.quant_nf4(mf, bs, ms, stoch)
        else:
            q, sc = Q.quant_int8(mf, bs)
        m.copy_(q.view(m.shape))
        ms.copy_(sc)
        qv, sv = Q.quant_logu8(vf, vbs, vs, stoch)
        v.copy_(qv.view(v.shape))
        vs.copy_(sv)
        return
    m, v = st["exp_avg"], st["exp_avg_sq"]
    if v.numel() != p.numel():
        raise RuntimeError("the per-parameter update needs full-size exp_avg_sq (quad-v state)")
    gf, mf, vf = g.to(torch.float32), m.to(torch.float32), v.to(torch.float32)
    if apply_wd:
        p.mul_(wd_factor)
    mf.mul_(b1).add_(gf, alpha=1.0 - b1)
    vf.mul_(b2).addcmul_(gf, gf, value=1.0 - b2)
    den = vf.sqrt().add_(eps_scaled)
    p.addcdiv_(mf, den, value=-step_size)
    m.copy_(mf.to(m.dtype))
    v.copy_(vf.to(v.dtype))


def fused_first_step_closed_form(p, g, *, lr, beta1, beta2, eps, weight_decay):
    """First per-parameter update from zero state in float64 (2-D p, decay on):
    m = (1-b1) g, v = (1-b2) g^2, p' = p (1 - lr wd) - s num / (sqrt(v) + eps
    sqrt(1-b2)) with num = (b1 m + (1-b1) g) times the lookahead gain (8-bit)
    or num = m (compact)."""
    G = g.double()
    m = (1.0 - beta1) * G
    v = (1.0 - beta2) * G * G
    s = lr * (1.0 - beta2) ** 0.5 / (1.0 - beta1)
    den = v.sqrt() + eps * (1.0 - beta2) ** 0.5
    base = p.double() * max(1.0 - lr * weight_decay, 0.0)
    look = beta1 * m + (1.0 - beta1) * G
    gain = torch.where(m * G >= 0, 1.0 + 0.20 * beta1, 1.0 - 0.35 * beta1).double()
    return base - s * look * gain / den, base - s * m / den
