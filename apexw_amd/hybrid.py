"""HybridApexW: Muon for 2-D weight matrices, ApexW for everything else.

Drop-in for the reference ``apexw.hybrid.HybridApexW`` (apexw/hybrid.py:183-508):
same constructor and defaults (muon lr = 5 x lr under the rms_matched/spectral
scale modes, ns_steps 5, Newton-Schulz quintic), the same routing rule
(``partition_parameters_for_hybrid``, hybrid.py:73-141), the same
``state_dict`` layout (flat ids, plus ``muon_state_dict`` /
``adamw_state_dict`` / ``apexw_state_dict``) and ``load_state_dict``.
``ApexW(..., use_muon=True)`` and ``precision="hybrid"`` construct it.
"""

from collections import defaultdict
from typing import Any, Dict

import torch
import torch.nn as nn
from torch import Tensor
from torch.optim.optimizer import Optimizer

from . import state as S
from .muon import ApexMuon
from . import runtime as R
from .optimizer import ApexW


def is_muon_eligible(p, min_dim=32, exclude_embeddings=True):
    """2-D (or reshaped N-D) with both dims >= min_dim, not an embedding-like slab
    (max dim >= 1000 and aspect ratio >= 4) -- apexw/hybrid.py:73-86."""
    if not p.requires_grad or p.ndim < 2:
        return False
    m = p.shape[0]
    n = p.numel() // m
    if min(m, n) < min_dim:
        return False
    if exclude_embeddings and max(m, n) >= 1000 and max(m / n, n / m) >= 4.0:
        return False
    return True


def _is_fsdp_flat_param(p):
    """FSDP1 FlatParameter (apexw/fsdp.py:38-43): always stepped by ApexW."""
    return bool(getattr(p, "_is_flat_param", False)) or "FlatParameter" in type(p).__name__ \
        or hasattr(p, "_param_infos")


_EMBED_NAMES = ("embed", "wte", "wpe", "shared", "lm_head", "cls_head", "score_head")


def partition_parameters_for_hybrid(params, min_muon_dim=32, exclude_embeddings=True):
    """(muon_params, adamw_params) in input order (apexw/hybrid.py:89-141).

    For an ``nn.Module`` the parameter names also route biases, norms and
    embedding / head matrices to ApexW; for tensors, param-group dicts or
    iterables only the shape rule of ``is_muon_eligible`` applies.
    """
    muon, adamw = [], []
    if isinstance(params, nn.Module):
        for name, p in params.named_parameters():
            if not p.requires_grad:
                continue
            low = name.lower()
            one_d = p.ndim < 2 or low.endswith(".bias") or "norm" in low
            embed = exclude_embeddings and (any(k in low for k in _EMBED_NAMES) or low == "head.weight"
                                            or low.endswith(".head.weight"))
            if one_d or embed or _is_fsdp_flat_param(p):
                adamw.append(p)
                continue
            m = p.shape[0]
            n = p.numel() // m
            extreme = exclude_embeddings and max(m, n) >= 1000 and max(m / n, n / m) >= 4.0
            (muon if min(m, n) >= min_muon_dim and not extreme else adamw).append(p)
        return muon, adamw
    params = list(params)
    if params and isinstance(params[0], dict):
        params = [p for g in params for p in g["params"]]
    for p in params:
        if is_muon_eligible(p, min_muon_dim, exclude_embeddings):
            muon.append(p)
        elif p.requires_grad:
            adamw.append(p)
    return muon, adamw


def _partition_grouped_params(groups, min_muon_dim=32, exclude_embeddings=True):
    """Split each param-group dict into a Muon part and an AdamW part, keeping its
    options (apexw/hybrid.py:144-180).  ``use_muon=True`` sends every >= 2-D
    parameter of the group to Muon, ``use_muon=False`` the whole group to ApexW."""
    muon_groups, adamw_groups = [], []
    for g in groups:
        tag = g.get("use_muon", None)
        mu, aw = [], []
        for p in g["params"]:
            if not p.requires_grad:
                continue
            if tag is True and p.ndim >= 2:
                mu.append(p)
            elif tag is False or p.ndim < 2:
                aw.append(p)
            elif is_muon_eligible(p, min_muon_dim, exclude_embeddings):
                mu.append(p)
            else:
                aw.append(p)
        opts = {k: v for k, v in g.items() if k not in ("params", "use_muon")}
        if mu:
            muon_groups.append(dict(opts, params=mu))
        if aw:
            adamw_groups.append(dict(opts, params=aw))
    return muon_groups, adamw_groups


class CombinedOptimizerState(defaultdict):
    """Per-parameter state of both engines behind one mapping (apexw/hybrid.py:29-70):
    a parameter's state lives in the Muon engine if it has one there, else in ApexW's."""

    def __init__(self, muon_opt, apexw_opt=None, adamw_opt=None):
        super().__init__(dict)
        self._muon_opt = muon_opt
        self._adamw_opt = apexw_opt if apexw_opt is not None else adamw_opt

    @property
    def muon_state(self):
        return self._muon_opt.state if self._muon_opt is not None else {}

    @property
    def adamw_state(self):
        return self._adamw_opt.state if self._adamw_opt is not None else {}

    apexw_state = adamw_state

    def __getitem__(self, p):
        return self.muon_state[p] if p in self.muon_state else self.adamw_state[p]

    def __setitem__(self, p, val):
        if p in self.muon_state:
            self.muon_state[p] = val
        else:
            self.adamw_state[p] = val

    def __contains__(self, p):
        return p in self.muon_state or p in self.adamw_state

    def __len__(self):
        return len(self.muon_state) + len(self.adamw_state)

    def __iter__(self):
        yield from self.muon_state
        yield from self.adamw_state

    def keys(self):
        return list(self.muon_state.keys()) + list(self.adamw_state.keys())

    def values(self):
        return list(self.muon_state.values()) + list(self.adamw_state.values())

    def items(self):
        return list(self.muon_state.items()) + list(self.adamw_state.items())

    def get(self, p, default=None):
        return self[p] if p in self else default


class HybridApexW(Optimizer):
    """Muon on eligible matrices + ApexW (compact/8-bit) on the rest."""

    _step_supports_amp_scaling = True

    def __init__(self, params, lr=1e-3, muon_lr=None, muon_momentum=0.95, adamw_betas=None, apexw_betas=None,
                 weight_decay=1e-2, muon_weight_decay=None, ns_steps=5, scale_mode="rms_matched",
                 ns_method="newtonschulz5", beta3=None, alpha=5.0, cautious=False, min_muon_dim=32,
                 exclude_embeddings=True, precision="compact", batch_bmm=None, nesterov=False, fused=None,
                 capturable=False, compiled=False, muon_compiled=None, **apex_kwargs):
        precision = S.normalize_precision(precision)
        if precision == "hybrid":
            precision = "compact"
        extra_betas = apex_kwargs.pop("betas", None)
        if extra_betas is not None:
            if len(extra_betas) >= 3 and beta3 is None:
                beta3 = extra_betas[2]
            if adamw_betas is None:
                adamw_betas = (float(extra_betas[0]), float(extra_betas[1]))
        if apexw_betas is not None and adamw_betas is None:
            adamw_betas = apexw_betas
        if adamw_betas is None:
            adamw_betas = (0.9, 0.999) if precision in ("8bit", "full") else (0.9, 0.99)
        if muon_lr is None:
            muon_lr = lr * 5.0 if scale_mode in ("rms_matched", "spectral") else lr
        if muon_weight_decay is None:
            muon_weight_decay = weight_decay
        if muon_compiled is not None:
            compiled = muon_compiled
        self._min_muon_dim = min_muon_dim
        self._exclude_embeddings = exclude_embeddings
        self._muon_init_kwargs = dict(lr=muon_lr, momentum=muon_momentum, nesterov=nesterov,
                                      weight_decay=muon_weight_decay, ns_steps=ns_steps, beta3=beta3, alpha=alpha,
                                      cautious=cautious, precision=precision, batch_bmm=batch_bmm, fused=fused,
                                      capturable=capturable, scale_mode=scale_mode, ns_method=ns_method,
                                      compiled=compiled)
        self._adamw_init_kwargs = dict(lr=lr, betas=adamw_betas, weight_decay=weight_decay, beta3=beta3, alpha=alpha,
                                       cautious=cautious, precision=precision, fused=fused, capturable=capturable,
                                       **apex_kwargs)
        if not isinstance(params, nn.Module):
            params = list(params)
        if isinstance(params, list) and params and isinstance(params[0], dict):
            muon_groups, adamw_groups = _partition_grouped_params(params, min_muon_dim, exclude_embeddings)
            self.muon_params = [p for g in muon_groups for p in g["params"]]
            self.adamw_params = [p for g in adamw_groups for p in g["params"]]
            self.muon_opt = ApexMuon(muon_groups, **self._muon_init_kwargs) if self.muon_params else None
            self.adamw_opt = ApexW(adamw_groups, **self._adamw_init_kwargs) if self.adamw_params else None
        else:
            self.muon_params, self.adamw_params = partition_parameters_for_hybrid(params, min_muon_dim,
                                                                                  exclude_embeddings)
            self.muon_opt = ApexMuon(self.muon_params, **self._muon_init_kwargs) if self.muon_params else None
            self.adamw_opt = ApexW(self.adamw_params, **self._adamw_init_kwargs) if self.adamw_params else None
        self.apexw_params = self.adamw_params
        self.apexw_opt = self.adamw_opt
        defaults = dict(lr=lr, muon_lr=muon_lr, weight_decay=weight_decay)
        super().__init__(self.muon_params + self.adamw_params, defaults)
        self._sync_groups()
        self._initialized = True

    def _sync_groups(self):
        groups = []
        for o in (self.muon_opt, self.adamw_opt):
            if o is not None:
                groups.extend(o.param_groups)
        self.param_groups = groups
        self.state = CombinedOptimizerState(self.muon_opt, self.adamw_opt)

    def zero_grad(self, set_to_none: bool = True):
        for o in (self.muon_opt, self.adamw_opt):
            if o is not None:
                o.zero_grad(set_to_none=set_to_none)

    def add_param_group(self, param_group):
        if not getattr(self, "_initialized", False):
            return super().add_param_group(param_group)
        muon_groups, adamw_groups = _partition_grouped_params([param_group], self._min_muon_dim,
                                                              self._exclude_embeddings)
        for g in muon_groups:
            self.muon_params.extend(g["params"])
            if self.muon_opt is not None:
                self.muon_opt.add_param_group(g)
            else:
                self.muon_opt = ApexMuon([g], **self._muon_init_kwargs)
        for g in adamw_groups:
            self.adamw_params.extend(g["params"])
            if self.adamw_opt is not None:
                self.adamw_opt.add_param_group(g)
            else:
                self.adamw_opt = ApexW([g], **self._adamw_init_kwargs)
        self.apexw_params = self.adamw_params
        self.apexw_opt = self.adamw_opt
        self._sync_groups()

    @R.step_hooks
    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        grad_scale = getattr(self, "grad_scale", None)
        found_inf = getattr(self, "found_inf", None)
        try:
            for o in (self.muon_opt, self.adamw_opt):
                if o is None:
                    continue
                if grad_scale is not None:
                    o.grad_scale = grad_scale
                if found_inf is not None:
                    o.found_inf = found_inf
                o.step()
        finally:
            for o in (self.muon_opt, self.adamw_opt):
                if o is not None:
                    o.grad_scale = None
                    o.found_inf = None
            self.grad_scale = None
            self.found_inf = None
        return loss

    def state_dict(self) -> Dict[str, Any]:
        """Flat state/param_groups over both engines (Muon ids first) plus each engine's own dict."""
        muon_sd = self.muon_opt.state_dict() if self.muon_opt else None
        adamw_sd = self.adamw_opt.state_dict() if self.adamw_opt else None
        state, groups, offset = {}, [], 0
        if muon_sd is not None:
            max_id = -1
            for g in muon_sd.get("param_groups", []):
                ids = [pid + offset for pid in g.get("params", [])]
                groups.append(dict(g, params=ids))
                if ids:
                    max_id = max(max_id, max(ids))
            for pid, st in muon_sd.get("state", {}).items():
                state[pid + offset] = st
            if state or max_id >= 0:
                offset = max(max_id + 1, max((k + 1 for k in state), default=0))
        if adamw_sd is not None:
            for g in adamw_sd.get("param_groups", []):
                groups.append(dict(g, params=[pid + offset for pid in g.get("params", [])]))
            for pid, st in adamw_sd.get("state", {}).items():
                state[pid + offset] = st
        return {"state": state, "param_groups": groups, "muon_state_dict": muon_sd, "adamw_state_dict": adamw_sd,
                "apexw_state_dict": adamw_sd}

    def load_state_dict(self, state_dict: Dict[str, Any]):
        apexw_sd = state_dict.get("apexw_state_dict") or state_dict.get("adamw_state_dict")
        if state_dict.get("muon_state_dict") or apexw_sd:
            if self.muon_opt and state_dict.get("muon_state_dict"):
                self.muon_opt.load_state_dict(state_dict["muon_state_dict"])
            if self.adamw_opt and apexw_sd:
                self.adamw_opt.load_state_dict(apexw_sd)
        elif "state" in state_dict and "param_groups" in state_dict:
            n_muon = len(self.muon_opt.param_groups) if self.muon_opt else 0
            groups, flat = state_dict["param_groups"], state_dict["state"]
            if self.muon_opt is not None:
                mg = groups[:n_muon]
                self.muon_opt.load_state_dict({"state": {pid: flat[pid] for g in mg for pid in g.get("params", [])
                                                         if pid in flat}, "param_groups": mg})
            if self.adamw_opt is not None:
                ag = groups[n_muon:]
                self.adamw_opt.load_state_dict({"state": {pid: flat[pid] for g in ag for pid in g.get("params", [])
                                                          if pid in flat}, "param_groups": ag})
        self._sync_groups()
        for p, st in self.state.items():
            if isinstance(p, Tensor):
                for k, v in list(st.items()):
                    if isinstance(v, Tensor) and v.device != p.device:
                        st[k] = v.to(p.device)

    def get_state_memory_mb(self) -> float:
        tot = 0.0
        for o in (self.muon_opt, self.adamw_opt):
            if o is not None and hasattr(o, "get_state_memory_mb"):
                tot += o.get_state_memory_mb()
        return tot
