"""Oracle optimizer objects driving the CPU restatement (test infrastructure only).

``OracleApexW`` mirrors the reference ``ApexW`` constructor defaults and the CPU
dispatch of ``ApexW.step`` (``apexw/optimizer.py:3359-4094``) for the
``compact``, ``8bit``, ``full``, ``auto`` and ``ultra`` precisions (``ultra``
steps like ``8bit`` through ``_step_ultra``; ``full`` and ``auto`` like
``compact``, their state layouts aside):

* constructor: precision aliases (state.py:94-121), default betas (0.9, 0.999)
  for 8bit and full, (0.9, 0.99) otherwise, ``adamw_compat`` forcing
  ``decay_norm_only=False`` and mapping betas (0.9, 0.95)/(0.9, 0.99) to
  (0.9, 0.999) -- optimizer.py:1672-1714;
* step: grad preparation (sanitize + global-norm clip, optimizer.py:204-258 and
  :3469-3476; an AMP ``grad_scale`` attribute, as GradScaler sets it, is
  unscaled before a clip in the grad dtype, else by the step: in place on the
  grads after sanitizing for compact (:5530-5537), on the fp32 copy after
  nan_to_num for 8bit (:4504-4505, state.py:326-347), inside
  ``torch._fused_adamw_`` for the native path), then for 8bit ``_step_ultra`` per parameter, and for compact
  either ``torch._fused_adamw_`` when every state matches its parameter's dtype
  and size (optimizer.py:3683-3766, ``_fused_step`` :4737-4835) or the foreach
  path over (p dtype, m dtype, step, quad) subgroups (:5369-5381); amsgrad keeps a
  running max of v beside each of them (the 8bit and ultra precisions excepted).

Like the reference, the first step after the set of parameters-with-grad changes
is a *cold* step; it caches a plan and the following steps *replay* it
(``FastExecutionPlan``, optimizer.py:406-1341), which for the compact foreach
path rounds differently (see ``oracle.compact``).  Plan validity follows
``is_valid_for_step`` (optimizer.py:575-621).
"""

import math

import torch

from . import layout as L
from .clip import clip_grads_
from .compact import compact_subgroup_step, replay_subgroup_step, rescale_v, sanitize_grads
from .factored import factored_update
from .q8 import q8_param_step

_PREC = {
    "full": ("full", "fp32", "float32", "float", "fp64", "float64", "double"),
    "compact": ("compact", "bf16", "bfloat16", "fp16", "float16", "half", "16", "16-bit"),
    "8bit": ("8bit", "8-bit", "int8", "uint8", "q8", "adamw_8bit", "bnb_8bit"),
    "ultra": ("ultra", "ultra_stable", "3byte", "hybrid8"),
    "auto": ("auto", "smart", "adaptive"),
}


def normalize_precision(precision):
    if isinstance(precision, torch.dtype):
        if precision in (torch.bfloat16, torch.float16):
            return "compact"
        if precision in (torch.int8, torch.uint8):
            return "8bit"
        return "full"
    key = precision.lower().strip()
    for name, aliases in _PREC.items():
        if key in aliases:
            return name
    if key in ("hybrid", "hybrid_apexw", "hybrid-apexw", "apex_hybrid", "hybrid_compact"):
        return "compact"
    raise NotImplementedError(f"oracle does not cover precision {precision!r}")


class OracleApexW:
    def __init__(self, params, lr=1e-3, betas=None, eps=1e-8, weight_decay=1e-2, decay_norm_only=True,
                 adamw_compat=False, clip_grad_norm=None, precision="compact", stochastic_rounding=True,
                 block_size=None, force_compact_v=False, int4_m=None, grad_centralization=False,
                 factored_v=False, six_bit=False, threshold=65536, amp=None, dynamic_scaling=True, nesterov=False,
                 cautious=False, maximize=False, amsgrad=False, fused=None, lion=False, beta3=None, alpha=5.0):
        precision = normalize_precision(precision)
        if betas is not None and len(betas) > 2 and beta3 is None:
            beta3 = betas[2]
        if betas is None:
            betas = (0.9, 0.999) if precision in ("8bit", "full") else (0.9, 0.99)
        if adamw_compat:
            decay_norm_only = False
            if tuple(betas) in ((0.9, 0.95), (0.9, 0.99)):
                betas = (0.9, 0.999)
        self.params = list(params)
        self.group = dict(lr=lr, betas=tuple(betas[:2]), eps=eps, weight_decay=weight_decay,
                          decay_norm_only=decay_norm_only, clip_grad_norm=clip_grad_norm,
                          precision=precision, stochastic_rounding=stochastic_rounding,
                          block_size=block_size, force_compact_v=force_compact_v, int4_m=int4_m,
                          grad_centralization=grad_centralization, factored_v=factored_v, six_bit=six_bit,
                          threshold=threshold, amp=amp, dynamic_scaling=dynamic_scaling, nesterov=bool(nesterov),
                          cautious=bool(cautious), maximize=bool(maximize), amsgrad=bool(amsgrad),
                          fused=fused, lion=bool(lion), beta3=beta3, alpha=alpha, params=self.params)
        self.state = {}
        self._plan = None
        self.grad_scale = None
        self.found_inf = None

    def _plan_valid(self):
        plan = self._plan
        if plan is None:
            return False
        active = set(plan["params"])
        if any(p.grad is None for p in plan["params"]):
            return False
        # amsgrad switched on or off since the plan was made (optimizer.py:585-586): the
        # plan holds max lists only when made with amsgrad and without lion
        if plan["amsgrad"] != self.group["amsgrad"]:
            return False
        # beta3 set or cleared since the plan was made (optimizer.py:587-588)
        grp = self.group
        if plan.get("slow", False) != (grp["beta3"] is not None):
            return False
        # the native fused plan does not replay the variants (optimizer.py:593-600)
        if plan["kind"] == "native" and (grp["nesterov"] or grp["lion"] or grp["cautious"] or grp["maximize"]):
            return False
        return all(p.grad is None for p in self.params if p.requires_grad and p not in active)

    def _prepare(self, grads, sanitize):
        """_prepare_grads (optimizer.py:204-258): returns (grads, grad scale still
        to apply or None).  Grad centralization forces sanitizing (:3469-3473) and
        unscaling, then subtracts each dim >= 2 grad's mean over dims 1.. (:239-243)."""
        gc = self.group.get("grad_centralization", False)
        clip = self.group["clip_grad_norm"]
        if sanitize or gc:
            grads = sanitize_grads(grads)
        scale = self.grad_scale
        if clip is not None or gc:
            grads = [g.clone() for g in grads]
            if scale is not None:                       # unscale first (:227-237)
                torch._foreach_mul_(grads, scale.reciprocal())
                scale = None
            if gc:
                for g in grads:
                    if g.dim() >= 2:
                        g.sub_(g.mean(dim=tuple(range(1, g.dim())), keepdim=True))
            if clip is not None:
                clip_grads_(grads, clip)
        return grads, scale

    @staticmethod
    def _unscale(grads, scale):
        """In-place unscale of the (cloned) grads in their dtype (:5530-5537)."""
        if scale is None:
            return grads
        grads = [g.clone() for g in grads]
        torch._foreach_mul_(grads, scale.reciprocal())
        return grads

    def _signed(self, grads, quantized):
        """maximize in the compact-kernel precisions: the grads negated before anything
        else (the replayed plan, optimizer.py:1104-1105; the cold step negates inside
        _multi_tensor_step after clip and centralization, :5515-5517, which commute with
        the negation).  The quantized step negates inside q8_param_step."""
        if self.group["maximize"] and not quantized:
            return [-g for g in grads]
        return grads

    @staticmethod
    def _inv(scale):
        return None if scale is None else float(scale.reciprocal().item())

    def _kw(self):
        grp = self.group
        b1, b2 = grp["betas"]
        return dict(lr=grp["lr"], beta1=b1, beta2=b2, eps=grp["eps"], weight_decay=grp["weight_decay"],
                    decay_norm_only=grp["decay_norm_only"])

    @torch.no_grad()
    def step(self):
        if self.found_inf is not None and float(self.found_inf) > 0:
            return
        if self._plan_valid():
            self._replay()
            return
        self._plan = None
        grp = self.group
        plist = [p for p in self.params if p.grad is not None]
        if not plist:
            return
        peft = L.peft_context([grp])
        for p in plist:
            if p not in self.state:
                self.state[p] = L.init_state(p, grp, len(self.params), peft)
            elif grp["amsgrad"] and not grp["lion"] and not grp["precision"] in ("8bit", "ultra"):
                L.ensure_max_v(self.state[p], p)      # amsgrad switched on later (optimizer.py:2917-2922)
            if grp["beta3"] is not None and grp["precision"] not in ("8bit", "ultra"):
                L.ensure_slow(self.state[p], p)       # beta3 set later (optimizer.py:2903-2915)
        prec = grp["precision"]
        ams = grp["amsgrad"]
        if (ams or grp["lion"] or grp["beta3"] is not None) and prec in ("8bit", "ultra"):
            raise NotImplementedError("oracle: amsgrad / lion / beta3 in the 8bit / ultra precisions")
        lion = grp["lion"]
        ams = ams and not lion                  # lion keeps no v, nor its max (optimizer.py:5375-5380)
        slow = grp["beta3"] is not None and not lion
        quantized = prec in ("8bit", "ultra")     # both run _step_ultra (optimizer.py:3583-3587)
        grads, scale = self._prepare(self._signed([p.grad for p in plist], quantized),
                                     sanitize=not quantized or grp["clip_grad_norm"] is not None)
        kw = self._kw()
        if quantized:
            for p, g in zip(plist, grads):
                st = self.state[p]
                st["step"].add_(1)
                q8_param_step(p, g, st, step=st["step"].item(), inv_scale=self._inv(scale), nesterov=grp["nesterov"],
                              cautious=grp["cautious"], maximize=grp["maximize"], **kw)
            self._plan = {"kind": "8bit", "params": plist, "amsgrad": ams}
            return
        sts = [self.state[p] for p in plist]
        homogeneous = all("exp_avg_sq" in st and st["exp_avg"].dtype == st["exp_avg_sq"].dtype == p.dtype
                          and st["exp_avg"].numel() == st["exp_avg_sq"].numel() for p, st in zip(plist, sts))
        if homogeneous and grp["fused"] is not False and not (grp["maximize"] or grp["nesterov"] or grp["cautious"]
                                                              or lion or grp["beta3"] is not None):
            # maximize, nesterov and cautious leave the native fused step (optimizer.py:3733, :593-600),
            # and so does fused=False (:3723)
            self._native_fused(plist, grads, sts, grad_scale=scale, amsgrad=ams, **kw)
            self._plan = {"kind": "native", "params": plist, "amsgrad": ams, "slow": False}
            return
        # factored-v tensors: their own update with their own step (optimizer.py:5382-5432)
        for p, g, st in zip(plist, grads, sts):
            if st.get("is_factored_v", False):
                st["step"].add_(1)
                self._factored(p, g, st, int(st["step"].item()), self._inv(scale), sanitize=True)
        # the cached plan holds every parameter with a grad, factored ones included
        # (FastExecutionPlan(params=params_with_grad, factored_mask=...), optimizer.py:4005-4020)
        plan_params = list(plist)
        keep = [i for i, st in enumerate(sts) if not st.get("is_factored_v", False)]
        plist, grads, sts = [plist[i] for i in keep], [grads[i] for i in keep], [sts[i] for i in keep]
        grads = self._unscale(grads, scale)
        sub = {}
        for p, g, st in zip(plist, grads, sts):
            key = (p.dtype, st["exp_avg"].dtype, int(st["step"].item()), self._is_quad(p))
            sub.setdefault(key, []).append((p, g, st))
        for (_, mdt, _, quad), items in sub.items():
            for _, _, st in items:
                st["step"].add_(1)
            step = int(items[0][2]["step"].item())
            vs = [i[2].get("exp_avg_sq") for i in items]
            scale_v, sqrt_scale_v = 1.0, 1.0
            if grp.get("dynamic_scaling", True) and mdt == torch.float16 and not lion:
                # the subgroup's v scale lives in its parameters' states; every 100 steps
                # it is recalibrated from max(v) (optimizer.py:5600-5645; keyed on m's dtype)
                st0 = items[0][2]
                scale_v = st0["scale_v"]
                sqrt_scale_v = st0.get("sqrt_scale_v", math.sqrt(scale_v))
                if step > 1 and step % 100 == 0:
                    f = rescale_v(vs, scale_v)
                    if f != 1.0:
                        scale_v *= f
                        sqrt_scale_v = math.sqrt(scale_v)
                        for _, _, st in items:
                            st["scale_v"], st["sqrt_scale_v"] = scale_v, sqrt_scale_v
            compact_subgroup_step([i[0] for i in items], [i[1] for i in items],
                                  [i[2]["exp_avg"] for i in items], vs, step=step, is_quad=quad,
                                  stochastic=grp["stochastic_rounding"], scale_v=scale_v,
                                  sqrt_scale_v=sqrt_scale_v, nesterov=grp["nesterov"],
                                  cautious=grp["cautious"], lion=lion,
                                  max_vs=[i[2]["max_exp_avg_sq"] for i in items] if ams else None,
                                  slows=[i[2]["exp_avg_slow"] for i in items] if slow else None,
                                  beta3=grp["beta3"], alpha=grp["alpha"], **kw)
        # the replayed plan's per-subgroup scales start at 1.0 (optimizer.py:546-560)
        self._plan = {"kind": "foreach", "params": plan_params, "sg_scale": {}, "amsgrad": ams,
                      "slow": grp["beta3"] is not None}

    def _is_quad(self, p):
        v = self.state[p].get("exp_avg_sq")
        if v is None:                           # lion: no second moment
            return False
        return p.numel() >= 4 and p.numel() % 4 == 0 and v.numel() * 4 == p.numel()

    def _replay(self):
        grp = self.group
        plan = self._plan
        plist = plan["params"]
        kw = self._kw()
        grads = [p.grad for p in plist]
        if plan["kind"] == "8bit":
            grads, scale = self._prepare(grads, sanitize=False)
            for p, g in zip(plist, grads):
                st = self.state[p]
                st["step"].add_(1)
                q8_param_step(p, g, st, step=st["step"].item(), inv_scale=self._inv(scale), nesterov=grp["nesterov"],
                              cautious=grp["cautious"], maximize=grp["maximize"], **kw)
            return
        grads, scale = self._prepare(self._signed(grads, False), sanitize=grp["clip_grad_norm"] is not None)
        sts = [self.state[p] for p in plist]
        lion = grp["lion"]
        ams = plan["amsgrad"] and not lion
        slow = plan.get("slow", False) and not lion
        if plan["kind"] == "native":
            self._native_fused(plist, grads, sts, sanitize=False, grad_scale=scale, amsgrad=ams, **kw)
            return
        steps = [st["step"] for st in sts]
        torch._foreach_add_(steps, 1)
        step = int(steps[0].item())
        # factored-v entries of the replayed plan: the plan's step, no nan_to_num (optimizer.py:1141-1163)
        for p, g, st in zip(plist, grads, sts):
            if st.get("is_factored_v", False):
                self._factored(p, g, st, step, self._inv(scale), sanitize=False)
        keep = [i for i, st in enumerate(sts) if not st.get("is_factored_v", False)]
        plist, grads, sts = [plist[i] for i in keep], [grads[i] for i in keep], [sts[i] for i in keep]
        grads = self._unscale(sanitize_grads(grads), scale)
        sub = {}
        for p, g, st in zip(plist, grads, sts):
            compact = st["exp_avg"].dtype in (torch.bfloat16, torch.float16)
            sub.setdefault((p.dtype, compact, self._is_quad(p)), []).append((p, g, st))
        dno = kw.pop("decay_norm_only")
        sg_scale = plan["sg_scale"]
        if grp.get("dynamic_scaling", True) and step > 1 and step % 100 == 0:
            # the replay's recalibration scales fp16 v by the factor, but the step below
            # takes its scale from the first parameter's state, which the replay never
            # updates (optimizer.py:1165-1178, :1193-1199)
            for key, items in sub.items():
                vs = [i[2].get("exp_avg_sq") for i in items]
                if vs[0] is not None and vs[0].dtype == torch.float16:
                    rescale_v(vs, sg_scale.get(key, 1.0))
        for key, items in sub.items():
            quad = key[2]
            st0 = items[0][2]
            scale_v = st0.get("scale_v", sg_scale.get(key, 1.0))
            sqrt_scale_v = st0.get("sqrt_scale_v", math.sqrt(scale_v))
            sg_scale[key] = scale_v
            replay_subgroup_step([i[0] for i in items], [i[1] for i in items],
                                 [i[2]["exp_avg"] for i in items], [i[2].get("exp_avg_sq") for i in items],
                                 apply_wd_mask=[(i[0].dim() >= 2) if dno else True for i in items],
                                 step=step, is_quad=quad, stochastic=grp["stochastic_rounding"],
                                 scale_v=scale_v, sqrt_scale_v=sqrt_scale_v, nesterov=grp["nesterov"],
                                 cautious=grp["cautious"], lion=lion,
                                 max_vs=[i[2]["max_exp_avg_sq"] for i in items] if ams else None,
                                 slows=[i[2]["exp_avg_slow"] for i in items] if slow else None,
                                 beta3=grp["beta3"], alpha=grp["alpha"], **kw)

    def _factored(self, p, g, st, step, inv, sanitize):
        grp = self.group
        b1, b2 = grp["betas"]
        lr, wd, eps = grp["lr"], grp["weight_decay"], grp["eps"]
        bc1, bc2 = 1.0 - b1 ** step, 1.0 - b2 ** step
        apply_wd = wd != 0 and (not grp["decay_norm_only"] or p.dim() >= 2)
        factored_update(p, g, st, beta1=b1, beta2=b2, step_size=lr * math.sqrt(bc2) / bc1,
                        eps_scaled=eps * math.sqrt(bc2), eps=eps, stochastic=st.get("stochastic_rounding", True),
                        block_size=st.get("block_size_8bit", 256),
                        wd_factor=max(1.0 - lr * wd, 0.0) if apply_wd else None, inv_scale=inv, sanitize=sanitize)

    @staticmethod
    def _native_fused(params, grads, sts, *, lr, beta1, beta2, eps, weight_decay, decay_norm_only,
                      sanitize=True, grad_scale=None, amsgrad=False):
        if sanitize:
            grads = sanitize_grads(grads)
        steps = [st["step"] for st in sts]
        torch._foreach_add_(steps, 1)
        if decay_norm_only and weight_decay != 0.0:
            parts = [([i for i, p in enumerate(params) if p.dim() >= 2], weight_decay),
                     ([i for i, p in enumerate(params) if p.dim() < 2], 0.0)]
        else:
            parts = [(list(range(len(params))), weight_decay)]
        for idx, wd in parts:
            if idx:
                torch._fused_adamw_([params[i] for i in idx], [grads[i] for i in idx],
                                    [sts[i]["exp_avg"] for i in idx], [sts[i]["exp_avg_sq"] for i in idx],
                                    [sts[i]["max_exp_avg_sq"] for i in idx] if amsgrad else [],
                                    [steps[i] for i in idx], amsgrad=amsgrad, lr=lr, beta1=beta1,
                                    beta2=beta2, weight_decay=wd, eps=eps, maximize=False,
                                    grad_scale=grad_scale)
