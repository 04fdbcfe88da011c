"""ApexW: the optimizer front end (drop-in for the reference ``apexw.ApexW``).

Same constructor (33 keyword arguments in the reference's positional order,
apexw/optimizer.py:1632-1668), defaults, argument validation and precision
aliases; same ``state`` keys and dtypes, ``state_dict()`` /
``load_state_dict()`` schema, and ``use_muon=True`` / ``precision="hybrid"``
routing to ``HybridApexW`` (apexw/optimizer.py:1593-1617).

The step itself runs on the GPU through libapexw_hip.so: one fused
multi-tensor kernel launch per parameter group and step (plus three tiny
launches when global-norm clipping is on).  There is no CPU or torch-op
fallback; options outside the hot path raise ``NotImplementedError`` at
construction.

precision="8bit" on a large model (>= 8 trainable tensors, >= 524,288
elements, no clipping or centralization) turns on the reference's automatic
runtime acceleration (optimizer.py:2059-2167): fp32 parameters of >= 1024
elements are converted to bf16 in place, and parameters of >= 16384 elements
(except the first) are stepped during backward, 14 at a time, by the same
8-bit kernel (``_flush_auto_8bit_hook_queue``, optimizer.py:2226-2371).
"""

import math
import warnings
from collections import defaultdict

import numpy as np
import torch
import torch.nn as nn
from torch.optim.optimizer import Optimizer

from . import runtime as R
from . import state as S
from ._plan import StepPlan

AUTO_8BIT_MIN_TENSORS = 8          # optimizer.py:2087
AUTO_8BIT_MIN_NUMEL = 524_288
DOWNCAST_MIN_NUMEL = 1024          # optimizer.py:2100
HOOK_MIN_NUMEL = 16384             # optimizer.py:2131
HOOK_BATCH = 14                    # optimizer.py:2142

_UNSUPPORTED_FLAGS = ("capturable", "differentiable", "auto_pack")
def _check_variants(precision, factored, nesterov, cautious, maximize=False, amsgrad=False, lion=False,
                    beta3=None):
    """nesterov=True, cautious=True and maximize=True run in every precision: the
    8-bit and ultra steps' lookahead numerator lerp(g, m, beta1) without the SNR gain
    and the compact, full and auto steps' two addcdiv passes (lerp(g, m, beta1) for
    quad v); the numerator m times the sign-agreement mask over its mean; the negated
    grads.  amsgrad=True, lion=True and beta3 (AdEMAMix) run in the compact, full and
    auto precisions (a running max of v beside it, no quad v; the sign update on m
    alone, which takes the place of the AdamW update and of its variants; a slow first
    moment beside m, no quad v).  maximize also runs with factored second moments
    (the negated grads reach the factored kernels through the unscale factor).
    nesterov, cautious and amsgrad with factored second moments, nesterov together with
    cautious, beta3 together with cautious, and amsgrad, lion or beta3 in the 8bit and
    ultra precisions do not."""
    for name, on in (("nesterov", nesterov), ("cautious", cautious), ("amsgrad", amsgrad)):
        if not on:
            continue
        if factored:
            raise NotImplementedError(f"apexw_amd: {name}=True with factored_v")
    if nesterov and cautious:
        raise NotImplementedError("apexw_amd: nesterov=True together with cautious=True")
    if amsgrad and precision in ("8bit", "ultra"):
        raise NotImplementedError(f"apexw_amd: amsgrad=True with precision={precision!r}")
    if lion and precision in ("8bit", "ultra"):
        raise NotImplementedError(f"apexw_amd: lion=True with precision={precision!r}")
    if beta3 is not None and not lion:
        if precision in ("8bit", "ultra"):
            raise NotImplementedError(f"apexw_amd: beta3 with precision={precision!r}")
        if factored:
            raise NotImplementedError("apexw_amd: beta3 with factored_v")
        if cautious:
            raise NotImplementedError("apexw_amd: beta3 together with cautious=True")


class ApexW(Optimizer):
    """Memory-efficient AdamW with compact (bf16) or 8-bit (NF4 + log-uint8) state.

    precision="compact": bf16 first moment, bf16 (or fp32) second moment,
    quad-shared v for large tensors.  precision="8bit": NF4 momentum + quad
    log-uint8 variance with per-block fp32 scales (INT8 + uint8 for small
    tensors).  precision="full": fp32 moments.  precision="auto": compact
    moments for 2-D and large tensors, fp32 for small ones (fp32 for all in
    pure-fp32 training).  precision="ultra": INT8 momentum blocks and a dense
    16-bit (or fp32) variance for 2-D and large tensors, fp32 for small ones.
    Weight decay is decoupled; ``adamw_compat=True`` decays every tensor and
    maps betas (0.9, 0.95)/(0.9, 0.99) to (0.9, 0.999).
    """

    _step_supports_amp_scaling = True

    def __new__(cls, *args, **kwargs):
        first = args[0] if args else kwargs.get("params")
        use_muon = kwargs.get("use_muon", args[26] if len(args) > 26 else False)
        prec = kwargs.get("precision", args[16] if len(args) > 16 else None)
        hybrid = bool(use_muon) or (isinstance(prec, str) and prec.lower().strip() in S.HYBRID_ALIASES)
        if hybrid:
            from .hybrid import HybridApexW
            a = list(args)
            kw = dict(kwargs)
            kw.pop("use_muon", None)
            if len(a) > 26:
                a.pop(26)
            if isinstance(kw.get("precision"), str) and kw["precision"].lower().strip() in S.HYBRID_ALIASES:
                kw["precision"] = "compact"
            if len(a) > 16 and isinstance(a[16], str) and a[16].lower().strip() in S.HYBRID_ALIASES:
                a[16] = "compact"
            return HybridApexW(*a, **kw)
        if isinstance(first, nn.Module):
            for name, p in first.named_parameters():
                if not hasattr(p, "_param_name"):
                    setattr(p, "_param_name", name)
        return super().__new__(cls)

    def __init__(self, params, lr=1e-3, betas=None, eps=1e-8, weight_decay=1e-2, amsgrad=False,
                 nesterov=False, cautious=False, grad_centralization=False, decay_norm_only=True,
                 adamw_compat=False, clip_grad_norm=None, beta3=None, alpha=5.0, lion=False, fused=None,
                 precision="compact", threshold=65536, maximize=False, foreach=None, capturable=False,
                 dynamic_scaling=True, differentiable=False, backend=None, auto_pack=False,
                 pack_threshold=50000, use_muon=False, amp=None, stochastic_rounding=True, block_size=None,
                 force_compact_v=False, factored_v=False, int4_m=None, six_bit=False):
        precision = S.normalize_precision(precision)
        if precision == "hybrid":
            precision = "compact"
        if betas is None:
            betas = (0.9, 0.999) if precision in ("8bit", "full") else (0.9, 0.99)
        if isinstance(params, nn.Module):
            for name, p in params.named_parameters():
                if not hasattr(p, "_param_name"):
                    setattr(p, "_param_name", name)
            trainable = [p for p in params.parameters() if p.requires_grad]
            params = trainable if trainable else list(params.parameters())
        if differentiable:
            raise NotImplementedError("ApexW does not currently support differentiable=True.")
        if not 0.0 <= lr:
            raise ValueError(f"Invalid learning rate: {lr}")
        if not 0.0 <= eps:
            raise ValueError(f"Invalid epsilon value: {eps}")
        if not 0.0 <= betas[0] < 1.0:
            raise ValueError(f"Invalid beta1 parameter: {betas[0]}")
        if not 0.0 <= betas[1] < 1.0:
            raise ValueError(f"Invalid beta2 parameter: {betas[1]}")
        if len(betas) > 2 and beta3 is None:
            beta3 = betas[2]
        if beta3 is not None and not 0.0 <= beta3 < 1.0:
            raise ValueError(f"Invalid beta3 parameter: {beta3}")
        if not 0.0 <= weight_decay:
            raise ValueError(f"Invalid weight_decay value: {weight_decay}")
        if clip_grad_norm is not None and clip_grad_norm <= 0.0:
            raise ValueError(f"Invalid clip_grad_norm value: {clip_grad_norm}")
        if block_size is not None and (isinstance(block_size, bool) or not isinstance(block_size, int) or block_size <= 0):
            raise ValueError(f"Invalid block_size value: {block_size}. Must be a positive integer.")
        if threshold <= 0:
            raise ValueError(f"Invalid threshold value: {threshold}. Must be positive.")
        if alpha < 0.0:
            raise ValueError(f"Invalid alpha value: {alpha}")
        if backend is not None and backend not in ("auto", "triton", "cuda", "mps", "foreach", "_multi_tensor", "xla"):
            raise ValueError(f"Invalid backend '{backend}'. Must be 'auto', 'triton', 'cuda', 'mps', 'foreach', or 'xla'.")
        if adamw_compat:
            decay_norm_only = False
            if tuple(betas[:2]) in ((0.9, 0.95), (0.9, 0.99)):
                betas = (0.9, 0.999)
        opts = dict(amsgrad=amsgrad, nesterov=nesterov, cautious=cautious, grad_centralization=grad_centralization,
                    lion=lion, maximize=maximize, capturable=capturable, differentiable=differentiable,
                    auto_pack=auto_pack, factored_v=factored_v, six_bit=six_bit)
        bad = [k for k in _UNSUPPORTED_FLAGS if opts[k]]
        if bad:
            raise NotImplementedError(f"apexw_amd implements the standard AdamW step; not supported: {', '.join(bad)}")
        if nesterov or cautious or maximize or amsgrad or lion or beta3 is not None:
            # factored_v=True lays out no factored state under amsgrad, lion or beta3
            _check_variants(S.normalize_precision(precision),
                            factored_v and not lion and not amsgrad and beta3 is None,
                            nesterov and not lion, cautious and not lion, maximize, amsgrad and not lion, lion,
                            beta3)
        if precision == "compact" and betas[1] >= 0.99 and not stochastic_rounding and not adamw_compat:
            warnings.warn(
                f"ApexW: beta2={betas[1]} with precision='compact' and stochastic_rounding=False "
                f"{'stores exp_avg_sq in float32' if betas[1] >= S.BETA2_V_FP32_THRESHOLD else 'may lose bf16 second-moment precision'}.",
                UserWarning, stacklevel=2)
        defaults = dict(lr=lr, betas=(betas[0], betas[1]), eps=eps, weight_decay=weight_decay, amsgrad=amsgrad,
                        nesterov=nesterov, cautious=cautious, grad_centralization=grad_centralization,
                        decay_norm_only=decay_norm_only, clip_grad_norm=clip_grad_norm, beta3=beta3, alpha=alpha,
                        lion=lion, fused=fused, precision=precision, threshold=threshold, maximize=maximize,
                        foreach=foreach, capturable=capturable, dynamic_scaling=dynamic_scaling,
                        differentiable=differentiable, backend=backend, auto_pack=auto_pack,
                        pack_threshold=pack_threshold, amp=amp, stochastic_rounding=stochastic_rounding,
                        block_size=block_size, force_compact_v=force_compact_v, factored_v=factored_v,
                        int4_m=int4_m, six_bit=six_bit)
        super().__init__(params, defaults)
        self._amp_unfolded = False
        self.state = R.StateMap(self, self.state)
        self._plans = {}
        # seed of the counter-based rounding RNG (drawn from torch's generator, so
        # torch.manual_seed makes runs reproducible)
        self._seed = int(torch.randint(0, 2 ** 62, (1,)).item())
        self._init_hook_state()
        if precision == "8bit":
            self._enable_8bit_runtime_acceleration()

    def _init_hook_state(self):
        self._has_stepped = False
        self._auto_hook_handles = []
        self._auto_hook_queue = []
        self._auto_hook_stepped_count = 0
        self._anchor_backward_count = 0
        self._grad_accum_steps = 1
        self._grad_accum_steps_known = False
        self._hook_plans = {}
        self._single_plans = {}
        self._fused_backward_enabled = False

    def __setstate__(self, state):
        super().__setstate__(state)
        self._amp_unfolded = False
        self.state = R.StateMap(self, dict.items(self.state))
        for group in self.param_groups:
            group.setdefault("decay_norm_only", True)
            group.setdefault("clip_grad_norm", None)
            group.setdefault("precision", "compact")
            group.setdefault("stochastic_rounding", True)
            group.setdefault("force_compact_v", False)
            group.setdefault("int4_m", False)
            group.setdefault("factored_v", False)
            group.setdefault("six_bit", False)
        self._plans = {}
        if not hasattr(self, "_auto_hook_queue"):
            self._init_hook_state()

    # ------------------------------------------------------------------ step
    @R.step_hooks
    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        # in-backward 8-bit steps: step what is still queued, then learn the
        # accumulation count from the backward passes seen (optimizer.py:3371-3381)
        self._has_stepped = True
        if self._auto_hook_queue:
            self._flush_auto_8bit_hook_queue()
        if self._auto_hook_stepped_count > 0:
            if not self._grad_accum_steps_known and self._anchor_backward_count > 1:
                self._grad_accum_steps = self._anchor_backward_count
                self._grad_accum_steps_known = True
            self._auto_hook_stepped_count = 0
            self._anchor_backward_count = 0
        R.amp_scaled_this_backward = False
        # AMP: GradScaler hands over its scale and found_inf instead of unscaling
        # (_step_supports_amp_scaling); an inf/NaN step is skipped, otherwise the
        # grads are unscaled inside the step kernels (apexw/optimizer.py:3458-3480,
        # :3627-3628).  The reference reads both on the host, which waits for the
        # backward; here the step kernels read them on the device (plan.amp_device_ok)
        # and the host reads them only for a plan whose kernels cannot.
        found_inf = getattr(self, "found_inf", None)
        grad_scale = getattr(self, "grad_scale", None)
        amp = None
        if torch.is_tensor(found_inf) and found_inf.is_cuda and (
                grad_scale is None or (torch.is_tensor(grad_scale) and grad_scale.is_cuda)):
            amp = self._amp_tensors(grad_scale, found_inf)
        self._amp_unfolded = False        # no waits in the lookups of the step itself
        try:
            self._step_groups(amp, grad_scale, found_inf)
        finally:
            self._amp_unfolded = any(pl.amp_dirty for pl in self._plans.values())
        return loss

    def _step_groups(self, amp, grad_scale, found_inf):
        """Two phases, as the reference's fused dispatch orders validation before any
        mutation and rolls its step counters back when a launch is refused
        (apexw/optimizer.py:3184-3356, :3806): every group's plan is built and its
        step prepared (counters advanced, every launch checked by the library), then
        the groups run.  A refusal while preparing restores every counter and leaves
        every parameter and state untouched; a launch that fails while running
        restores the counters of that group and of the groups after it."""
        host_amp = None
        progs = []
        try:
            for group in self.param_groups:
                gid = id(group)
                plan = self._plans.get(gid)
                if plan is None or not plan.valid_for(group):
                    old = self._plans.pop(gid, None)
                    if old is not None:
                        old.amp_fold(sync=True)       # its counters are the states' until the new plan reads them
                    keep = old is not None and getattr(old, "keep_replay", False)
                    plan = self._build_plan(group, foreach=keep)
                    if plan is None:
                        continue
                    if keep:
                        # a lion switch or a grad dtype change over a replayed plan: the next step replays too
                        plan.cold_done = True
                        plan._sg_scale = dict(old._sg_scale)
                    self._plans[gid] = plan
                # a plan's first launch (the cold rounding order) stays on the host read, so that
                # a skipped step cannot use it up: the next real step is the cold one, as in the reference
                if amp is not None and plan.amp_device_ok and plan.cold_done:
                    prog = plan.prepare(group, self._seed, amp=amp)
                    if prog is not None:
                        progs.append(prog)
                        continue
                if host_amp is None:
                    host_amp = self._read_amp(grad_scale, found_inf)
                skip, inv_scale = host_amp
                if skip:
                    continue
                progs.append(plan.prepare(group, self._seed, inv_scale))
        except BaseException:
            for prog in progs:
                prog.rollback()
            raise
        for i, prog in enumerate(progs):
            try:
                prog.run()
            except BaseException:
                for later in progs[i + 1:]:
                    later.rollback()
                raise

    @staticmethod
    def _read_amp(grad_scale, found_inf):
        """(skip, inv_scale) read on the host, as the reference does."""
        if found_inf is not None and float(found_inf.item()) > 0:
            return True, None
        if grad_scale is None:
            return False, None
        return False, (float(grad_scale.reciprocal().item()) if torch.is_tensor(grad_scale)
                       else 1.0 / float(grad_scale))

    def _amp_tensors(self, grad_scale, found_inf):
        """(scale, found_inf) as fp32 device scalars for apexw_amp_prepare."""
        dev = found_inf.device
        if grad_scale is None:
            one = getattr(self, "_amp_one", None)
            if one is None or one.device != dev:
                one = self._amp_one = torch.ones(1, dtype=torch.float32, device=dev)
            grad_scale = one
        return (grad_scale.detach().reshape(1).to(dev, torch.float32).contiguous(),
                found_inf.detach().reshape(1).to(dev, torch.float32).contiguous())

    def _fold_amp_skips(self):
        """Make every step counter exact: subtract the steps GradScaler skipped on the device."""
        self._amp_unfolded = False
        for plan in self._plans.values():
            plan.amp_fold(sync=True)

    def _build_plan(self, group, foreach=False):
        """The group's StepPlan from its parameters with grads (states made as needed);
        foreach: never the native fused order."""
        group["precision"] = S.normalize_precision(group.get("precision", "compact"))
        params = []
        for p in group["params"]:
            if p.grad is None:
                continue
            if p.grad.is_sparse:
                raise RuntimeError("ApexW does not support sparse gradients")
            if torch.is_complex(p) or p.dtype not in (torch.float32, torch.bfloat16, torch.float16):
                raise NotImplementedError(f"apexw_amd steps fp32, bf16 and fp16 parameters, got {p.dtype}")
            if p.device.type != "cuda":
                raise RuntimeError("apexw_amd runs the optimizer step on the GPU; parameters must be on cuda")
            params.append(p)
        if not params:
            return None
        peft = S.detect_peft_context(self.param_groups)
        has16 = any(q.dtype in (torch.float16, torch.bfloat16) for g in self.param_groups for q in g["params"])
        for p in params:
            if len(self.state[p]) == 0:
                self.state[p].update(S.init_state(p, group, peft, has16))
        lion = bool(group.get("lion", False))
        # lion takes the place of the AdamW update and of its variants (optimizer.py:5375-5380,
        # :5677-5683): nesterov, cautious, amsgrad and beta3 do not apply under it
        ams = bool(group.get("amsgrad", False)) and not lion
        beta3 = group.get("beta3") if not lion else None
        if (group.get("nesterov", False) or group.get("cautious", False) or group.get("maximize", False) or ams
                or lion or beta3 is not None):
            _check_variants(group["precision"], any(self.state[p].get("is_factored_v", False) for p in params),
                            bool(group.get("nesterov", False)) and not lion,
                            bool(group.get("cautious", False)) and not lion,
                            bool(group.get("maximize", False)), ams, lion, beta3)
        if beta3 is not None:
            for p in params:
                st = self.state[p]
                if st["exp_avg_sq"].numel() != p.numel():
                    raise NotImplementedError("apexw_amd: beta3 on a tensor whose state holds quad v")
                S.ensure_slow(st, p)          # beta3 set after the first step (optimizer.py:2903-2915)
        if not lion:
            for p in params:
                if "exp_avg_sq" not in self.state[p] and not self.state[p].get("is_factored_v", False):
                    raise NotImplementedError("apexw_amd: lion=False on a tensor whose state holds no second "
                                              "moment (made under lion=True)")
        if ams:
            for p in params:
                st = self.state[p]
                if st["exp_avg_sq"].numel() != p.numel():
                    # quad v laid out before amsgrad was switched on: the reference's
                    # torch._foreach_maximum_ over max_v (numel) and v (numel / 4) fails too
                    raise NotImplementedError("apexw_amd: amsgrad=True on a tensor whose state holds quad v")
                S.ensure_max_v(st, p)         # amsgrad switched on after the first step (optimizer.py:2917-2922)
        for p in params:
            if not p.is_contiguous():
                # a dense non-contiguous parameter (channels_last and the like) is stepped in its
                # memory layout: its full-size state tensors take that layout too (a checkpoint's,
                # or amsgrad's max, may be contiguous)
                st = self.state[p]
                for k in ("exp_avg", "exp_avg_sq", "max_exp_avg_sq", "exp_avg_slow"):
                    t = st.get(k)
                    if torch.is_tensor(t) and t.shape == p.shape and t.stride() != p.stride():
                        st[k] = torch.empty_like(p, dtype=t.dtype).copy_(t)
        if group["precision"] in ("8bit", "ultra"):
            # both run the reference's _step_ultra (optimizer.py:3583-3587)
            return StepPlan(self, group, params, "q8")
        sts = [self.state[p] for p in params]
        # torch._fused_adamw_ when every state matches its parameter's dtype and size,
        # unless fused=False asks for the foreach path (optimizer.py:3676-3720)
        homogeneous = all("exp_avg_sq" in st and st["exp_avg"].dtype == st["exp_avg_sq"].dtype == p.dtype
                          and st["exp_avg"].numel() == st["exp_avg_sq"].numel() for p, st in zip(params, sts))
        # maximize, nesterov and cautious leave the native fused plan (FastExecutionPlan.
        # is_valid_for_step, optimizer.py:593-600): the foreach order instead
        native = (homogeneous and group.get("fused") is not False and not group.get("maximize", False)
                  and not group.get("nesterov", False) and not group.get("cautious", False) and not lion
                  and group.get("beta3") is None and not foreach)
        if native and any(p.grad.dtype != p.dtype for p in params):
            # torch._fused_adamw_ takes grads in their parameters' dtype only (it raises "expected
            # scalar type"), so the reference's native fused step fails on such grads; fused=False
            # steps them in the foreach order
            raise RuntimeError("apexw_amd: the native fused step needs grads in their parameters' dtype "
                               "(as torch._fused_adamw_ does); pass fused=False to step grads of another dtype")
        return StepPlan(self, group, params, "compact", native=native)

    # ------------------------------------------------------------------ checkpoints
    def state_dict(self):
        self._fold_amp_skips()
        sd = super().state_dict()
        meta = {}
        for p, s in self.state.items():
            if "scale_v" in s:
                meta[id(p)] = {"scale_v": s["scale_v"], "sqrt_scale_v": s.get("sqrt_scale_v", math.sqrt(s["scale_v"]))}
        sd["_dynamic_scaling_meta"] = meta
        return sd

    def load_state_dict(self, state_dict):
        """Load, then restore every state tensor in its saved dtype (the base loader
        casts floating state to the parameter dtype)."""
        self._fold_amp_skips()
        sd = dict(state_dict)
        sd.pop("_dynamic_scaling_meta", None)
        saved = sd.get("state", {})
        origin = {}
        for sg, g in zip(sd.get("param_groups", []), self.param_groups):
            for pid, p in zip(sg.get("params", ()), g["params"]):
                if pid in saved:
                    origin[p] = saved[pid]
        super().load_state_dict(sd)
        for p, s in self.state.items():
            src = origin.get(p, {})
            for k, v in src.items():
                if torch.is_tensor(v) and k != "step":
                    s[k] = v.detach().to(device=p.device).clone()
        self._plans = {}

    def set_precision(self, precision):
        """Move every group to ``precision`` ("compact" or "8bit", or an alias) and
        convert each parameter's state whose layout belongs to the other mode on
        the GPU (fp32 decode, then the new mode's quantizers; step counts kept).

        For resuming a checkpoint in another precision: load_state_dict keeps the
        saved groups and layouts, as the reference's does, then this converts them.
        States already in a layout of the new mode are kept as they are."""
        from . import convert as C
        self._fold_amp_skips()
        prec = S.normalize_precision(precision)
        if prec not in ("compact", "8bit"):
            raise NotImplementedError(f"apexw_amd implements the compact and 8-bit AdamW step; not supported: "
                                      f"precision={prec!r}")
        if prec == "8bit" and any(g.get("amsgrad", False) for g in self.param_groups):
            raise NotImplementedError("apexw_amd: amsgrad=True with precision='8bit'")
        peft = S.detect_peft_context(self.param_groups)
        for group in self.param_groups:
            group["precision"] = prec
            for p in group["params"]:
                st = self.state.get(p)
                if not st or "exp_avg" not in st:
                    continue
                if C.family(st) != C.target_family(p, group, peft):
                    self.state[p] = C.convert(p, st, group, peft)
        self._plans = {}

    def zero_grad(self, set_to_none=True):
        super().zero_grad(set_to_none=set_to_none)
        self._auto_hook_queue.clear()

    # ------------------------------------------------------------------ in-backward 8-bit steps
    def _enable_8bit_runtime_acceleration(self, force=False):
        """bf16 parameters and layer-batched in-backward steps for large 8-bit
        models (optimizer.py:2059-2167)."""
        d = self.defaults
        if not force and (d.get("clip_grad_norm") is not None or d.get("grad_centralization", False)
                          or d.get("nesterov", False) or d.get("maximize", False) or d.get("amsgrad", False)
                          or d.get("lion", False) or d.get("beta3") is not None):
            return
        trainable = []
        total = 0
        for group in self.param_groups:
            if S.normalize_precision(group.get("precision", "compact")) != "8bit":
                continue
            for p in group["params"]:
                if (isinstance(p, torch.Tensor) and p.requires_grad and not torch.is_complex(p)
                        and p.dtype != torch.float64):
                    trainable.append((p, group))
                    total += p.numel()
        if not force and (len(trainable) < AUTO_8BIT_MIN_TENSORS or total < AUTO_8BIT_MIN_NUMEL):
            return
        # the restore rules and the AMP scale detection the in-backward steps rely on
        # (torch patches, installed once, only when this path turns on); the reference's
        # process-wide TF32 / cuDNN benchmark settings are not taken over
        R.install()
        converted = False
        with torch.no_grad():
            for p, _ in trainable:
                if p.dtype == torch.float32 and p.numel() >= DOWNCAST_MIN_NUMEL:
                    # fp16 only on devices without bf16 (compute capability < 8); MI355X has bf16
                    target = torch.bfloat16
                    if p.is_cuda and torch.cuda.get_device_capability(p.device)[0] < 8:
                        target = torch.float16
                    R.register_downcast(p, torch.float32)
                    p.data = p.data.to(target)
                    if p.grad is not None and p.grad.dtype != target:
                        p.grad = p.grad.to(target)
                    if target == torch.float16:
                        R.fp16_active = True
                    converted = True
                elif p.dtype == torch.float16:
                    R.fp16_active = True
        if converted and torch.cuda.is_available():
            torch.cuda.empty_cache()
        self._disable_auto_8bit_hooks()
        if len(trainable) >= 2:
            anchor = trainable[0][0]
            hooked = [(p, g) for p, g in trainable[1:] if p.numel() >= HOOK_MIN_NUMEL]
            if hooked:
                for p, g in hooked:
                    self._auto_hook_handles.append(p.register_post_accumulate_grad_hook(self._layer_hook(p, g)))
                self._auto_hook_handles.append(anchor.register_post_accumulate_grad_hook(self._anchor_hook))
        R.register_optimizer(self)

    def _layer_hook(self, param, group):
        def hook(_):
            if self._fused_backward_enabled or param.grad is None:
                return
            self._auto_hook_queue.append((param, group))
            if len(self._auto_hook_queue) >= HOOK_BATCH:
                self._flush_auto_8bit_hook_queue()
        return hook

    def _anchor_hook(self, _):
        # the first parameter's grad comes last in backward: step what is queued
        if self._fused_backward_enabled:
            return
        if self._auto_hook_queue:
            self._flush_auto_8bit_hook_queue()
        self._anchor_backward_count += 1

    def _disable_auto_8bit_hooks(self):
        for h in self._auto_hook_handles:
            h.remove()
        self._auto_hook_handles.clear()
        self._auto_hook_queue.clear()
        self._auto_hook_stepped_count = 0
        self._anchor_backward_count = 0

    @torch.no_grad()
    def _flush_auto_8bit_hook_queue(self):
        """Step the queued parameters with the 8-bit kernel and free their grads
        (optimizer.py:2226-2371).  With K accumulated backward passes per step
        (learned by step()), every pass steps with lr * K^-0.4, weight decay
        wd / (K * K^-0.4) and the grads scaled by K; the stored step counter is
        (passes - 1) // K + 1 and the bias correction uses the pass count."""
        if not self._auto_hook_queue:
            return
        batch = list(self._auto_hook_queue)
        self._auto_hook_queue.clear()
        K = max(1, int(self._grad_accum_steps))
        mult = 1.0 if K == 1 else K ** -0.40
        amp = R.last_amp_scale
        amp_inv = 1.0 / amp if (R.amp_scaled_this_backward and amp is not None and amp > 0.0) else 1.0
        inv_scale = amp_inv * float(K)
        by_group, seen = {}, set()
        for p, group in batch:
            if p.grad is None or id(p) in seen:
                continue
            seen.add(id(p))
            by_group.setdefault(id(group), (group, []))[1].append(p)
        # every batch is prepared (counters advanced, launches checked) before any runs;
        # a refusal restores each parameter's counters, as step() does
        progs, undo = [], []
        try:
            for group, params in by_group.values():
                msteps = []
                for p in params:
                    st = S.ensure_8bit_state(self.state[p], p, group)
                    undo.append((st, st.get("_hook_mstep", 0), float(st["step"])))
                    mstep = st.get("_hook_mstep", 0) + 1
                    st["_hook_mstep"] = mstep
                    # the reference's CPU path stores (mstep - 1) // K + 1 (optimizer.py:2366-2367);
                    # its CUDA path instead adds 1 every K passes, which differs once K changes
                    st["step"].fill_(float((mstep - 1) // K + 1))
                    msteps.append(mstep)
                lr_eff = float(group["lr"]) * mult
                wd_raw = float(group["weight_decay"])
                wd_eff = wd_raw / (float(K) * mult) if wd_raw != 0.0 else 0.0
                # the step takes the grad scale as a float32 tensor and multiplies by its reciprocal
                inv = None if inv_scale == 1.0 else float(np.float32(1.0) / np.float32(1.0 / inv_scale))
                for p in params:
                    if p.grad.dtype != p.dtype:
                        p.grad = p.grad.to(p.dtype)
                plan = self._hook_plan(group, params)
                progs.append((plan.prepare(group, self._hook_seed, inv, lr=lr_eff, wd=wd_eff, steps=msteps),
                              params))
        except BaseException:
            for st, mstep, step in undo:
                st["_hook_mstep"] = mstep
                st["step"].fill_(step)
            raise
        for prog, params in progs:
            prog.run()
            for p in params:
                p.grad = None
            self._auto_hook_stepped_count += len(params)

    def _hook_plan(self, group, params):
        key = (id(group), tuple(map(id, params)))
        plan = self._hook_plans.get(key)
        if plan is None or not plan.valid_for(group):
            group["precision"] = S.normalize_precision(group.get("precision", "compact"))
            for p in params:
                if p.device.type != "cuda":
                    raise RuntimeError("apexw_amd runs the optimizer step on the GPU; parameters must be on cuda")
                if p.dtype not in (torch.float32, torch.bfloat16, torch.float16):
                    raise NotImplementedError(f"apexw_amd steps fp32, bf16 and fp16 parameters, got {p.dtype}")
            plan = StepPlan(self, group, params, "q8", hooked=True)
            self._hook_plans[key] = plan
        return plan

    # ------------------------------------------------------------------ fused backward
    def enable_fused_backward(self, model=None, grad_accum_steps=1):
        """Step every parameter inside backward, as soon as its grad is accumulated,
        and free the grad (optimizer.py:1986-2034).  With grad_accum_steps = K a
        parameter is stepped on every K-th grad it receives; ``step()`` then has
        nothing left to do.  The update is the reference's per-parameter one
        (``_step_single_param_fused``), not the fused multi-tensor step."""
        self._fused_backward_enabled = True
        self._grad_accum_steps = max(1, int(grad_accum_steps))
        self._accum_counter = defaultdict(int)
        self._fused_backward_handles = []
        if model is not None and hasattr(model, "parameters"):
            to_hook = [p for p in model.parameters() if p.requires_grad]
        else:
            to_hook = [p for g in self.param_groups for p in g["params"] if p.requires_grad]
        owner = {id(p): g for g in self.param_groups for p in g["params"]}
        for p in to_hook:
            if id(p) in owner:
                self._fused_backward_handles.append(p.register_post_accumulate_grad_hook(
                    self._fused_hook(p, owner[id(p)])))

    def disable_fused_backward(self):
        """Remove the per-parameter hooks; ``step()`` steps again (optimizer.py:2036-2043)."""
        self._fused_backward_enabled = False
        for h in getattr(self, "_fused_backward_handles", ()):
            h.remove()
        if hasattr(self, "_fused_backward_handles"):
            self._fused_backward_handles.clear()

    def _fused_hook(self, param, group):
        def hook(_):
            if param.grad is None:
                return
            pid = id(param)
            self._accum_counter[pid] += 1
            if self._accum_counter[pid] < self._grad_accum_steps:
                return
            self._accum_counter[pid] = 0
            self._step_single_param_fused(param, group)
            param.grad = None
        return hook

    @torch.no_grad()
    def _step_single_param_fused(self, p, group):
        """One per-parameter update (optimizer.py:2373-2471) on the GPU: the same
        state layouts, APEXW_MODE_SINGLE of the compact or 8-bit kernel."""
        if p.grad is None:
            return
        prec = S.normalize_precision(group.get("precision", "compact"))
        state = self.state[p]
        if state.get("is_factored_v", False):
            # the reference's per-parameter update has no factored branch (it fails on the
            # missing exp_avg_sq); refuse before touching the state or the step counter
            raise RuntimeError("enable_fused_backward cannot step a parameter with factored_v state "
                               "(exp_avg_sq_row / exp_avg_sq_col); use step()")
        if state.get("is_ultra", False):
            # the reference's per-parameter update would treat the INT8 m codes as a dense moment
            raise RuntimeError("enable_fused_backward cannot step a parameter with ultra (INT8 m) state; "
                               "use step()")
        if len(state) == 0:
            if prec == "8bit":
                S.ensure_8bit_state(state, p, group)
            else:
                state["stochastic_rounding"] = bool(group.get("stochastic_rounding", True))
                state["step"] = torch.tensor(0.0, dtype=torch.float32)
                cdt = S.compact_dtype(p) if prec == "compact" else torch.float32
                state["exp_avg"] = torch.zeros_like(p, dtype=cdt)
                state["exp_avg_sq"] = torch.zeros_like(p, dtype=cdt)
        state["step"].add_(1)
        step = int(state["step"].item())
        if p.grad.dtype != p.dtype:
            p.grad = p.grad.to(p.dtype)
        plan = self._single_plans.get(id(p))
        if plan is None or not plan.valid_for(group):
            if p.device.type != "cuda":
                raise RuntimeError("apexw_amd runs the optimizer step on the GPU; parameters must be on cuda")
            if p.dtype not in (torch.float32, torch.bfloat16, torch.float16):
                raise NotImplementedError(f"apexw_amd steps fp32, bf16 and fp16 parameters, got {p.dtype}")
            kind = "q8" if (state.get("is_8bit", False) or prec == "8bit") else "compact"
            if kind == "compact" and "exp_avg_sq" not in state:
                raise RuntimeError("enable_fused_backward needs exp_avg_sq; this parameter has lion state "
                                   "(no second moment) from an earlier step()")
            if kind == "compact" and state["exp_avg_sq"].numel() != p.numel():
                # the reference's update broadcasts a full-size square against it and fails
                raise RuntimeError("enable_fused_backward needs full-size exp_avg_sq; this parameter "
                                   "has quad-v state from an earlier step()")
            group["precision"] = prec
            plan = StepPlan(self, group, [p], kind, single=True)
            self._single_plans[id(p)] = plan
        plan.execute(group, self._seed, None, steps=[step])

    @property
    def _hook_seed(self):
        # in-backward batches restart the tensor index at 0: give them their own RNG stream
        return (self._seed ^ 0x5DEECE66D9E3779B) & (2 ** 64 - 1)

    # ------------------------------------------------------------------ reporting
    def get_state_memory_mb(self):
        total = 0
        for st in self.state.values():
            for k, v in st.items():
                if torch.is_tensor(v) and k != "step":
                    total += v.numel() * v.element_size()
        return total / (1024 * 1024)

    def get_memory_summary(self):
        n = sum(p.numel() for g in self.param_groups for p in g["params"])
        mb = self.get_state_memory_mb()
        adamw_mb = n * 8 / (1024 * 1024)
        return {"num_params": n, "state_mb": mb, "adamw_state_mb": adamw_mb,
                "bytes_per_param": (mb * 1024 * 1024 / n) if n else 0.0,
                "savings_pct": (100.0 * (1 - mb / adamw_mb)) if adamw_mb else 0.0}

    def print_summary(self):
        s = self.get_memory_summary()
        print(f"ApexW: {s['num_params']:,} params, state {s['state_mb']:.2f} MB "
              f"({s['bytes_per_param']:.3f} B/param) vs AdamW {s['adamw_state_mb']:.2f} MB "
              f"({s['savings_pct']:.1f}% saved)")

    def __repr__(self):
        return f"ApexW(precision={self.defaults['precision']!r}, lr={self.defaults['lr']})"
