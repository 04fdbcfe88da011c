"""Compact-mode multi-tensor AdamW step (CPU oracle; test infrastructure only).

Restates ``ApexW._multi_tensor_step`` (``apexw/optimizer.py:5297-5887``) for the
AdamW update, its nesterov, cautious, amsgrad and AdEMAMix (beta3) variants and the lion
update with the same torch ops, so every bf16 rounding point of the reference is
reproduced:

1. decoupled weight decay ``p *= 1 - lr*wd`` (dim>=2 tensors when
   decay_norm_only) -- optimizer.py:5585-5592
2. ``m = m*b1``, ``m += (1-b1)*g``                 -- :5760-5761 / quad :5684-5685;
   fp32 m (``full`` / small ``auto`` tensors): ``m = lerp(m, g, 1-b1)`` -- :5780
3. ``v`` EMA: SR path when beta2 >= 0.995 and SR on (fp32 math then SR to 16
   bits, per tensor), else two foreach ops in v's dtype -- :5770-5776 / :5691-5697
4. ``d = sqrt(v) + eps*sqrt(bc2)`` in v's dtype       -- :5799-5816 / :5704-5721
5. parameter update: fp32 p ``addcdiv(p, m, d, -step_size)``; 16-bit p with SR
   ``p = SR(p - (m/d)*step_size)``; quad: ``p -= (m/d_q)*step_size``   -- :5818-5828 / :5722-5745;
   nesterov: two ``addcdiv`` (m with -step_size*b1, g with -step_size*(1-b1)), each rounded
   to p's dtype and never stochastic (:5865-5877); quad: ``lerp(g, m, b1)`` in place of m (:5732-5733);
   cautious: m times the mask ``g m >= 0`` over its mean (clamped at 1e-3), the mask, its mean
   and the product in the parameter's / m's dtype, then one ``addcdiv`` (:5847-5864); quad:
   the same in fp32 (:5728-5731);
   amsgrad: ``max_v = maximum(max_v, v)`` after the v EMA and ``d`` from max_v instead of v
   (:5788-5790; the quad branch :5700-5702 is never reached, quad v being off under amsgrad)

beta3 (AdEMAMix): a slow first moment follows m's update with beta3 (:5763-5765, :5781), and
the numerator is ``m + slow_ratio * m_slow`` (fp32 for an fp32 p over 16-bit m, :5834-5845),
``slow_ratio = alpha (1 - b1^t) / (1 - b3^t)``, then one addcdiv (nesterov ignored); the replay
adds in m's dtype (:1232-1238, :1332-1334)

lion (``lion_update``) replaces steps 2-5 after the weight decay: u = lerp(g', m, b1) with g'
the grads cast to m's dtype, ``p += -lr * sign(u)``, ``m = lerp(m, g', 1-b2)`` -- :5677-5683
(the replayed plan: :1214-1225, the same ops)

That is the *cold* step, taken whenever the optimizer (re)builds its cached
execution plan.  Every later step replays the plan through
``FastExecutionPlan.execute_foreach`` (optimizer.py:1069-1341), which rounds
differently; ``replay_subgroup_step`` restates it:

* no NaN/Inf sanitizing of the grads (only clip/centralization sanitize);
* ``m = lerp(m, g, 1-b1)`` in one op when g and m share a dtype (:1231-1234);
* the non-quad v EMA uses the grads in their own dtype (:1301-1302);
* 16-bit params always take ``p = SR-or-RNE(p - (m/d)*step_size)`` (:1334-1338);
* with fp16 in the subgroup the denominators are clamped below by eps.

fp16 second moments carry a dynamic scale (``scale_v``, 1024 at first): v is
stored times scale_v, the EMA adds (1-b2)*scale_v*g^2 and the denominator is
(sqrt(v) + eps_scaled*sqrt(scale_v)) / sqrt(scale_v); every 100 steps the scale
is recalibrated from max(v) (``rescale_v``).
"""

import math

import torch

from .quant import store_16bit


def sanitize_grads(grads):
    """_sanitize_gradients_fast (optimizer.py:136-201): clone-and-clean only tensors with NaN/Inf."""
    out = []
    for g in grads:
        if not bool(torch.isfinite(g).all()):
            if g.dtype in (torch.float16, torch.bfloat16):
                g = g.clone().clamp_(-65504.0, 65504.0).nan_to_num_(0.0)
            else:
                g = g.clone().nan_to_num_(0.0).clamp_(-65504.0, 65504.0)
        out.append(g)
    return out


def bias_terms(lr, beta1, beta2, eps, step):
    """Host scalars in double, as at optimizer.py:5577-5582."""
    bc1 = 1.0 - beta1 ** step
    bc2 = 1.0 - beta2 ** step
    bc2_sqrt = math.sqrt(bc2)
    return lr * bc2_sqrt / bc1, eps * bc2_sqrt


def slow_ratio(alpha, beta1, beta3, step):
    """AdEMAMix's weight of the slow moment, in double (optimizer.py:5584, :1101)."""
    return alpha * ((1.0 - beta1 ** step) / (1.0 - beta3 ** step))


def _slow_numerators(ms, slows, ratio, upcast):
    """m + ratio * m_slow by one foreach add with alpha, on fp32 copies (upcast) or in
    m's dtype (optimizer.py:5834-5845, :1332-1334)."""
    if upcast:
        ms, slows = [m.float() for m in ms], [m.float() for m in slows]
    return torch._foreach_add(ms, slows, alpha=ratio)


def _denominators(vs, eps_scaled, scale_v, sqrt_scale_v):
    """sqrt(v) + eps_scaled, in v's scaled units when fp16 v carries a dynamic
    scale (optimizer.py:5799-5816, :1303-1308)."""
    dens = torch._foreach_sqrt(vs)
    if scale_v != 1.0:
        torch._foreach_add_(dens, eps_scaled * sqrt_scale_v)
        torch._foreach_div_(dens, sqrt_scale_v)
    else:
        torch._foreach_add_(dens, eps_scaled)
    return dens


def lion_update(params, grads, ms, *, lr, beta1, beta2):
    """The lion update of a subgroup after its weight decay (optimizer.py:5677-5683,
    :1214-1225): grads cast to m's dtype, sign of lerp(g', m, beta1) times -lr added to
    p (one foreach add with alpha), then m = lerp(m, g', 1 - beta2)."""
    target = ms[0].dtype
    gc = [g.to(target) for g in grads] if grads[0].dtype != target else list(grads)
    updates = [u.sign() for u in torch._foreach_lerp(gc, ms, beta1)]
    torch._foreach_add_(params, updates, alpha=-lr)
    torch._foreach_lerp_(ms, gc, 1.0 - beta2)


def _amsgrad_max(max_vs, vs):
    """amsgrad: max_v = maximum(max_v, v) in place and the denominators' source
    (optimizer.py:5788-5790, :1253-1255); plain v otherwise."""
    if max_vs is None:
        return vs
    torch._foreach_maximum_(max_vs, vs)
    return max_vs


def _quad_cautious(g, m):
    """fp32 numerator m * mask / mean(mask) of a quad-v tensor (optimizer.py:5728-5731, :1272-1275)."""
    mask = (g * m >= 0).to(torch.float32)
    mask_mean = mask.mean().clamp(min=1e-3)
    return m.mul(mask.div_(mask_mean))


def _masked(nums, lhs, rhs, params):
    """cautious numerators of the non-quad tensors: nums[i] * mask / mean(mask), the
    mask (lhs[i] * rhs[i] >= 0, the product in their dtype) and its mean and quotient
    in the parameter's dtype, the product with the numerator by torch's promotion
    (optimizer.py:5850-5861, :1321-1327)."""
    out = []
    for num, a, b, p in zip(nums, lhs, rhs, params):
        mask = (a * b >= 0).to(p.dtype)
        mask_mean = mask.mean().clamp(min=1e-3)
        mask.div_(mask_mean)
        out.append(num * mask)
    return out


def compact_subgroup_step(params, grads, ms, vs, *, lr, beta1, beta2, eps, weight_decay,
                          decay_norm_only, step, is_quad, stochastic, scale_v=1.0, sqrt_scale_v=1.0,
                          nesterov=False, cautious=False, max_vs=None, lion=False, slows=None, beta3=None,
                          alpha=5.0):
    """One step over a subgroup sharing (p dtype, m dtype, step count, quad flag).

    ``step`` is the already-incremented step count.  Tensors are updated in place.
    scale_v / sqrt_scale_v: the dynamic scale of fp16 v (optimizer.py:5600-5645;
    1.0 otherwise): v holds scale_v times the second moment.
    """
    grads = sanitize_grads(grads)
    step_size, eps_scaled = bias_terms(lr, beta1, beta2, eps, step)
    if weight_decay != 0:
        decay = [p for p in params if p.dim() >= 2] if decay_norm_only else list(params)
        if decay:
            torch._foreach_mul_(decay, 1.0 - lr * weight_decay)
    if lion:
        lion_update(params, grads, ms, lr=lr, beta1=beta1, beta2=beta2)
        return
    gf = [g if g.dtype == torch.float32 else g.float() for g in grads]
    if ms[0].dtype in (torch.bfloat16, torch.float16):
        torch._foreach_mul_(ms, beta1)
        torch._foreach_add_(ms, gf, alpha=1.0 - beta1)
        if slows is not None:
            torch._foreach_mul_(slows, beta3)
            torch._foreach_add_(slows, gf, alpha=1.0 - beta3)
    elif ms[0].dtype == torch.float32:
        # fp32 moments ("full", small "auto" tensors): the grads cast to m's dtype
        # and one lerp (optimizer.py:5669-5674, :5778-5781)
        torch._foreach_lerp_(ms, gf, 1.0 - beta1)
        if slows is not None:
            torch._foreach_lerp_(slows, gf, 1.0 - beta3)
    else:
        raise NotImplementedError(f"oracle compact step: m dtype {ms[0].dtype}")
    v16 = vs[0].dtype in (torch.bfloat16, torch.float16)
    if is_quad:
        if max_vs is not None or slows is not None:
            raise NotImplementedError("oracle compact step: amsgrad or beta3 with quad v")
        gq = [g.reshape(-1, 4).square().mean(dim=1) for g in gf]
        if beta2 >= 0.995 and stochastic and v16:
            for v, q in zip(vs, gq):
                store_16bit(v, v.float().mul_(beta2).add_(q, alpha=(1.0 - beta2) * scale_v), True)
        else:
            torch._foreach_mul_(vs, beta2)
            torch._foreach_add_(vs, gq, alpha=(1.0 - beta2) * scale_v)
        dens = _denominators(vs, eps_scaled, scale_v, sqrt_scale_v)
        for p, g, m, d in zip(params, gf, ms, dens):
            if cautious:
                num = _quad_cautious(g, m.float())
            else:
                num = torch.lerp(g, m.float(), beta1) if nesterov else m.float()
            delta = num.view(-1, 4).div_(d.float().unsqueeze(1)).mul_(step_size).view(p.shape)
            if p.dtype == torch.float32:
                p.sub_(delta)
            else:
                store_16bit(p, p.float().sub_(delta), stochastic)
        return
    if beta2 >= 0.995 and stochastic and v16:
        for v, g in zip(vs, gf):
            store_16bit(v, v.float().mul_(beta2).addcmul_(g, g, value=(1.0 - beta2) * scale_v), True)
    else:
        torch._foreach_mul_(vs, beta2)
        torch._foreach_addcmul_(vs, gf, gf, value=(1.0 - beta2) * scale_v)
    dens = _denominators(_amsgrad_max(max_vs, vs), eps_scaled, scale_v, sqrt_scale_v)
    if slows is not None:
        # fp32 p with 16-bit m takes both moments upcast (optimizer.py:5834-5845)
        up = params[0].dtype == torch.float32 and ms[0].dtype != torch.float32
        nums = _slow_numerators(ms, slows, slow_ratio(alpha, beta1, beta3, step), up)
        torch._foreach_addcdiv_(params, nums, dens, value=-step_size)
    elif cautious:
        # fp32 p with 16-bit m takes m upcast (optimizer.py:5834-5838); the mask from
        # g.float() * num.float() (:5851-5853)
        mf = [m.float() for m in ms] if params[0].dtype == torch.float32 and ms[0].dtype != torch.float32 else ms
        nums = _masked(mf, gf, [n.float() for n in mf], params)
        torch._foreach_addcdiv_(params, nums, dens, value=-step_size)
    elif nesterov:
        # fp32 p with 16-bit m takes m upcast (optimizer.py:5834-5838)
        mf = [m.float() for m in ms] if params[0].dtype == torch.float32 and ms[0].dtype != torch.float32 else ms
        torch._foreach_addcdiv_(params, mf, dens, value=-step_size * beta1)
        torch._foreach_addcdiv_(params, gf, dens, value=-step_size * (1.0 - beta1))
    elif params[0].dtype in (torch.bfloat16, torch.float16) and stochastic:
        for p, m, d in zip(params, ms, dens):
            delta = (m.float() / d.float()) * step_size
            store_16bit(p, p.float().sub_(delta), True)
    else:
        torch._foreach_addcdiv_(params, ms, dens, value=-step_size)


def replay_subgroup_step(params, grads, ms, vs, *, lr, beta1, beta2, eps, weight_decay,
                         apply_wd_mask, step, is_quad, stochastic, scale_v=1.0, sqrt_scale_v=1.0,
                         nesterov=False, cautious=False, max_vs=None, lion=False, slows=None, beta3=None,
                         alpha=5.0):
    """One replayed step over an (p dtype, compact, quad) subgroup (optimizer.py:1200-1338).

    With an fp16 parameter, m or v the denominators are clamped below by eps
    (:1202, :1264-1265, :1310-1311)."""
    step_size, eps_scaled = bias_terms(lr, beta1, beta2, eps, step)
    if weight_decay != 0.0:
        decay = [p for p, w in zip(params, apply_wd_mask) if w]
        if decay:
            torch._foreach_mul_(decay, 1.0 - lr * weight_decay)
    if lion:
        lion_update(params, grads, ms, lr=lr, beta1=beta1, beta2=beta2)
        return
    has_fp16 = torch.float16 in (params[0].dtype, ms[0].dtype, vs[0].dtype)
    if grads[0].dtype == ms[0].dtype:
        torch._foreach_lerp_(ms, grads, 1.0 - beta1)
        if slows is not None:
            torch._foreach_lerp_(slows, grads, 1.0 - beta3)
    else:
        torch._foreach_mul_(ms, beta1)
        torch._foreach_add_(ms, grads, alpha=1.0 - beta1)
        if slows is not None:
            torch._foreach_mul_(slows, beta3)
            torch._foreach_add_(slows, grads, alpha=1.0 - beta3)
    v16 = vs[0].dtype in (torch.bfloat16, torch.float16)
    sr_v = beta2 >= 0.995 and stochastic and v16
    if is_quad:
        if max_vs is not None or slows is not None:
            raise NotImplementedError("oracle compact replay: amsgrad or beta3 with quad v")
        gf = grads if grads[0].dtype == torch.float32 else [g.float() for g in grads]
        gq = [g.reshape(-1, 4).square().mean(dim=1) for g in gf]
        if sr_v:
            for v, q in zip(vs, gq):
                store_16bit(v, v.float().mul_(beta2).add_(q, alpha=(1.0 - beta2) * scale_v), True)
        else:
            torch._foreach_mul_(vs, beta2)
            torch._foreach_add_(vs, gq, alpha=(1.0 - beta2) * scale_v)
        dens = _denominators(vs, eps_scaled, scale_v, sqrt_scale_v)
        if has_fp16:
            torch._foreach_clamp_min_(dens, eps)
        for p, g, m, d in zip(params, gf, ms, dens):
            if cautious:
                num = _quad_cautious(g, m.float())                             # :1272-1275
            else:
                num = torch.lerp(g, m.float(), beta1) if nesterov else m.float()    # :1276-1277
            delta = num.view(-1, 4).div_(d.float().unsqueeze(1)).mul_(step_size).view(p.shape)
            if p.dtype == torch.float32:
                p.sub_(delta)
            else:
                store_16bit(p, p.float().sub_(delta), stochastic)
        return
    if sr_v:
        for v, g in zip(vs, grads):
            g32 = g.float()
            store_16bit(v, v.float().mul_(beta2).addcmul_(g32, g32, value=(1.0 - beta2) * scale_v), True)
    else:
        torch._foreach_mul_(vs, beta2)
        torch._foreach_addcmul_(vs, grads, grads, value=(1.0 - beta2) * scale_v)
    dens = _denominators(_amsgrad_max(max_vs, vs), eps_scaled, scale_v, sqrt_scale_v)
    if has_fp16:
        torch._foreach_clamp_min_(dens, eps)
    if cautious:
        # m cast to the grads' dtype, the mask from their product in it (optimizer.py:1321-1328)
        nums = [m.to(g.dtype) if m.dtype != g.dtype else m for g, m in zip(grads, ms)]
        torch._foreach_addcdiv_(params, _masked(nums, grads, nums, params), dens, value=-step_size)
    elif nesterov and slows is None:
        # the grads in their own dtype (optimizer.py:1329-1331)
        torch._foreach_addcdiv_(params, ms, dens, value=-step_size * beta1)
        torch._foreach_addcdiv_(params, grads, dens, value=-step_size * (1.0 - beta1))
    elif slows is not None:
        # in m's dtype, no upcast (optimizer.py:1332-1334)
        nums = _slow_numerators(ms, slows, slow_ratio(alpha, beta1, beta3, step), False)
        torch._foreach_addcdiv_(params, nums, dens, value=-step_size)
    elif params[0].dtype in (torch.bfloat16, torch.float16):
        for p, m, d in zip(params, ms, dens):
            delta = (m.float() / d.float()) * step_size
            store_16bit(p, p.float().sub_(delta), stochastic)
    else:
        torch._foreach_addcdiv_(params, ms, dens, value=-step_size)


def rescale_v(vs, cur_scale):
    """The every-100-steps recalibration of fp16 v (optimizer.py:5622-5645,
    :1165-1178): factor 4 when max(v) < 0.25 and the scale is below 65536, 0.25
    when max(v) > 16384 and the scale is above 1, else 1; v is multiplied by it
    (in its dtype).  Returns the factor."""
    v_max = max(v.max().item() for v in vs) if vs else 1.0
    factor = 1.0
    if v_max < 0.25 and cur_scale < 65536.0:
        factor = 4.0
    elif v_max > 16384.0 and cur_scale > 1.0:
        factor = 0.25
    if factor != 1.0:
        torch._foreach_mul_(vs, factor)
    return factor
