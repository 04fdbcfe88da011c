"""HybridApexW: Muon for 2-D weight matrices, ApexW for everything else.

A drop-in for the reference's ``apexw.hybrid`` API (apexw/hybrid.py:73-508).
What callers observe is kept:

* the routing rule (``partition_parameters_for_hybrid``, ``is_muon_eligible``);
* the constructor's keywords and defaults: the Muon learning rate is 5 x lr
  under the ``rms_matched`` / ``spectral`` scale modes (lr otherwise), the Muon
  weight decay defaults to ``weight_decay``, and ApexW's betas come from
  ``adamw_betas``, else the first two of a ``betas`` keyword, else
  ``apexw_betas``, else the precision's default;
* the two engines as ``muon_opt`` and ``adamw_opt`` (alias ``apexw_opt``), with
  ``muon_params`` / ``adamw_params`` (alias ``apexw_params``);
* ``param_groups`` is the engines' own group dicts (a learning-rate schedule
  that edits them edits the engines), and ``state`` maps every parameter to
  its engine's state;
* the ``state_dict`` schema: a flat ``state`` / ``param_groups`` pair with the
  Muon engine's parameter ids first and ApexW's after them, plus each engine's
  own dict under ``muon_state_dict``, ``adamw_state_dict`` and
  ``apexw_state_dict``; ``load_state_dict`` takes either form;
* AMP: GradScaler's ``grad_scale`` / ``found_inf`` are handed to both engines.

The design is a thin composite.  Each engine is a complete optimizer of this
package (``ApexMuon`` over the Muon-routed matrices, ``ApexW`` over the rest)
that steps on the GPU by itself; the hybrid owns only the routing, an
ownership map from parameter to engine, and the checkpoint merge.
``ApexW(..., use_muon=True)`` and ``precision="hybrid"`` construct it.
"""

from collections.abc import MutableMapping

import torch
import torch.nn as nn
from torch.optim.optimizer import Optimizer

from . import runtime as R
from . import state as S
from .muon import ApexMuon
from .optimizer import ApexW

# ---------------------------------------------------------------------------
# routing
# ---------------------------------------------------------------------------
_EMBED_NAMES = ("embed", "wte", "wpe", "shared", "lm_head", "cls_head", "score_head")


def _extreme_aspect(m, n):
    """An embedding-like slab: long side >= 1000 and aspect ratio >= 4."""
    return max(m, n) >= 1000 and max(m / n, n / m) >= 4.0


def is_muon_eligible(p, min_dim=32, exclude_embeddings=True):
    """2-D (or N-D viewed as [shape[0], rest]) with both sides >= min_dim and, with
    exclude_embeddings, not an embedding-like slab (apexw/hybrid.py:73-86)."""
    if not p.requires_grad or p.ndim < 2:
        return False
    m = p.shape[0]
    n = p.numel() // m
    if min(m, n) < min_dim:
        return False
    return not (exclude_embeddings and _extreme_aspect(m, n))


def _is_fsdp_flat_param(p):
    """FSDP1 FlatParameter (apexw/fsdp.py:38-43): always stepped by ApexW."""
    return bool(getattr(p, "_is_flat_param", False)) or "FlatParameter" in type(p).__name__ \
        or hasattr(p, "_param_infos")


def _named_goes_to_muon(name, p, min_dim, exclude_embeddings):
    low = name.lower()
    if p.ndim < 2 or low.endswith(".bias") or "norm" in low or _is_fsdp_flat_param(p):
        return False
    if exclude_embeddings and (any(k in low for k in _EMBED_NAMES) or low == "head.weight"
                               or low.endswith(".head.weight")):
        return False
    m = p.shape[0]
    n = p.numel() // m
    return min(m, n) >= min_dim and not (exclude_embeddings and _extreme_aspect(m, n))


def partition_parameters_for_hybrid(params, min_muon_dim=32, exclude_embeddings=True):
    """(muon_params, adamw_params) in input order (apexw/hybrid.py:89-141).

    For an ``nn.Module`` the parameter names also send biases, norms and
    embedding / head matrices to ApexW; for tensors, param-group dicts or
    iterables only the shape rule of ``is_muon_eligible`` applies.
    """
    if isinstance(params, nn.Module):
        named = [(n, p) for n, p in params.named_parameters() if p.requires_grad]
        route = [_named_goes_to_muon(n, p, min_muon_dim, exclude_embeddings) for n, p in named]
        tensors = [p for _, p in named]
    else:
        tensors = list(params)
        if tensors and isinstance(tensors[0], dict):
            tensors = [p for g in tensors for p in g["params"]]
        tensors = [p for p in tensors if p.requires_grad]
        route = [is_muon_eligible(p, min_muon_dim, exclude_embeddings) for p in tensors]
    return ([p for p, r in zip(tensors, route) if r], [p for p, r in zip(tensors, route) if not r])


def _route_group(group, min_dim, exclude_embeddings):
    """Split one param-group dict into (muon group or None, apexw group or None),
    both keeping the group's options.  A ``use_muon`` tag forces the choice for
    every >= 2-D parameter of the group (apexw/hybrid.py:144-180)."""
    tag = group.get("use_muon", None)
    to_muon, to_apexw = [], []
    for p in group["params"]:
        if not p.requires_grad:
            continue
        if p.ndim < 2 or tag is False:
            to_apexw.append(p)
        elif tag is True or is_muon_eligible(p, min_dim, exclude_embeddings):
            to_muon.append(p)
        else:
            to_apexw.append(p)
    opts = {k: v for k, v in group.items() if k not in ("params", "use_muon")}
    return (dict(opts, params=to_muon) if to_muon else None, dict(opts, params=to_apexw) if to_apexw else None)


# ---------------------------------------------------------------------------
# per-parameter state across the two engines
# ---------------------------------------------------------------------------
class _JointState(MutableMapping):
    """``HybridApexW.state``: each parameter's entry is the state dict of the engine
    that steps it (looked up through the hybrid's ownership map)."""

    def __init__(self, hybrid):
        self._hybrid = hybrid

    def _engine(self, p):
        eng = self._hybrid._owner.get(id(p))
        if eng is None:
            raise KeyError("parameter is not stepped by this optimizer")
        return eng

    def __getitem__(self, p):
        return self._engine(p).state[p]

    def __setitem__(self, p, value):
        self._engine(p).state[p] = value

    def __delitem__(self, p):
        del self._engine(p).state[p]

    def __contains__(self, p):
        eng = self._hybrid._owner.get(id(p))
        return eng is not None and p in eng.state

    def __iter__(self):
        for eng in self._hybrid._engines():
            yield from list(eng.state.keys())

    def __len__(self):
        return sum(len(eng.state) for eng in self._hybrid._engines())


# ---------------------------------------------------------------------------
# the optimizer
# ---------------------------------------------------------------------------
def _default_muon_lr(lr, scale_mode):
    # the rms-matched / spectral update has ~0.2 sqrt(max dim) RMS: Muon runs at 5x lr
    return lr * 5.0 if scale_mode in ("rms_matched", "spectral") else lr


class HybridApexW(Optimizer):
    """Muon on eligible matrices + ApexW (compact / 8-bit) on the rest."""

    _step_supports_amp_scaling = True

    def __init__(self, params, lr=1e-3, muon_lr=None, muon_momentum=0.95, adamw_betas=None, apexw_betas=None,
                 weight_decay=1e-2, muon_weight_decay=None, ns_steps=5, scale_mode="rms_matched",
                 ns_method="newtonschulz5", beta3=None, alpha=5.0, cautious=False, min_muon_dim=32,
                 exclude_embeddings=True, precision="compact", batch_bmm=None, nesterov=False, fused=None,
                 capturable=False, compiled=False, muon_compiled=None, **apex_kwargs):
        precision = S.normalize_precision(precision)
        if precision == "hybrid":
            precision = "compact"
        extra = apex_kwargs.pop("betas", None)
        if extra is not None and len(extra) >= 3 and beta3 is None:
            beta3 = extra[2]
        betas = next((tuple(b)[:2] for b in (adamw_betas, extra, apexw_betas) if b is not None),
                     (0.9, 0.999) if precision in ("8bit", "full") else (0.9, 0.99))
        betas = (float(betas[0]), float(betas[1]))
        self._route_opts = (min_muon_dim, exclude_embeddings)
        self._muon_kwargs = dict(
            lr=_default_muon_lr(lr, scale_mode) if muon_lr is None else muon_lr, momentum=muon_momentum,
            nesterov=nesterov, weight_decay=weight_decay if muon_weight_decay is None else muon_weight_decay,
            ns_steps=ns_steps, beta3=beta3, alpha=alpha, cautious=cautious, precision=precision,
            batch_bmm=batch_bmm, fused=fused, capturable=capturable, scale_mode=scale_mode, ns_method=ns_method,
            compiled=compiled if muon_compiled is None else muon_compiled)
        self._apexw_kwargs = dict(lr=lr, betas=betas, weight_decay=weight_decay, beta3=beta3, alpha=alpha,
                                  cautious=cautious, precision=precision, fused=fused, capturable=capturable,
                                  **apex_kwargs)
        self.muon_opt = self.adamw_opt = None
        self.muon_params, self.adamw_params = [], []
        self._owner = {}
        if not isinstance(params, nn.Module):
            params = list(params)
        if isinstance(params, list) and params and isinstance(params[0], dict):
            routed = [_route_group(g, *self._route_opts) for g in params]
            muon_groups = [m for m, _ in routed if m is not None]
            apexw_groups = [a for _, a in routed if a is not None]
        else:
            mu, aw = partition_parameters_for_hybrid(params, *self._route_opts)
            muon_groups = [{"params": mu}] if mu else []
            apexw_groups = [{"params": aw}] if aw else []
        for g in muon_groups:
            self._attach("muon", g)
        for g in apexw_groups:
            self._attach("apexw", g)
        self._ready = False
        super().__init__(self.muon_params + self.adamw_params,
                         dict(lr=lr, muon_lr=self._muon_kwargs["lr"], weight_decay=weight_decay))
        self._ready = True
        self._expose()

    # ------------------------------------------------------------------ engines
    @property
    def apexw_opt(self):
        return self.adamw_opt

    @property
    def apexw_params(self):
        return self.adamw_params

    def _engines(self):
        return [e for e in (self.muon_opt, self.adamw_opt) if e is not None]

    def _attach(self, role, group):
        """Give ``group`` to the engine of ``role``, creating the engine on first use."""
        if role == "muon":
            if self.muon_opt is None:
                self.muon_opt = ApexMuon([group], **self._muon_kwargs)
            else:
                self.muon_opt.add_param_group(group)
            eng, plist = self.muon_opt, self.muon_params
        else:
            if self.adamw_opt is None:
                self.adamw_opt = ApexW([group], **self._apexw_kwargs)
            else:
                self.adamw_opt.add_param_group(group)
            eng, plist = self.adamw_opt, self.adamw_params
        for p in group["params"]:
            plist.append(p)
            self._owner[id(p)] = eng

    def _expose(self):
        """The hybrid's groups are the engines' own dicts; its state reads through to them."""
        self.param_groups = [g for eng in self._engines() for g in eng.param_groups]
        self.state = _JointState(self)

    def add_param_group(self, param_group):
        if not getattr(self, "_ready", False):
            # Optimizer.__init__ registering the routed parameters
            return super().add_param_group(param_group)
        group = dict(param_group)
        if isinstance(group["params"], torch.Tensor):
            group["params"] = [group["params"]]
        else:
            group["params"] = list(group["params"])
        muon_group, apexw_group = _route_group(group, *self._route_opts)
        if muon_group is not None:
            self._attach("muon", muon_group)
        if apexw_group is not None:
            self._attach("apexw", apexw_group)
        self._expose()

    def zero_grad(self, set_to_none: bool = True):
        for eng in self._engines():
            eng.zero_grad(set_to_none=set_to_none)

    @R.step_hooks
    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        handoff = {k: getattr(self, k, None) for k in ("grad_scale", "found_inf")}
        try:
            for eng in self._engines():
                for k, v in handoff.items():
                    if v is not None:
                        setattr(eng, k, v)
                eng.step()
        finally:
            for obj in self._engines() + [self]:
                obj.grad_scale = None
                obj.found_inf = None
        return loss

    # ------------------------------------------------------------------ checkpoints
    def state_dict(self):
        """Flat ``state`` / ``param_groups`` (Muon ids first, ApexW's shifted past them) plus
        each engine's own dict."""
        muon_sd = self.muon_opt.state_dict() if self.muon_opt is not None else None
        apexw_sd = self.adamw_opt.state_dict() if self.adamw_opt is not None else None
        flat_state, flat_groups, base = {}, [], 0
        for sd in (muon_sd, apexw_sd):
            if sd is None:
                continue
            ids = [pid for g in sd["param_groups"] for pid in g["params"]] + list(sd["state"])
            for g in sd["param_groups"]:
                flat_groups.append(dict(g, params=[base + pid for pid in g["params"]]))
            for pid, st in sd["state"].items():
                flat_state[base + pid] = st
            base += (max(ids) + 1) if ids else 0
        return {"state": flat_state, "param_groups": flat_groups, "muon_state_dict": muon_sd,
                "adamw_state_dict": apexw_sd, "apexw_state_dict": apexw_sd}

    def load_state_dict(self, state_dict):
        """Load either form: the engines' own dicts when present, else the flat pair
        (the first groups belong to the Muon engine, the rest to ApexW)."""
        muon_sd = state_dict.get("muon_state_dict")
        apexw_sd = state_dict.get("apexw_state_dict") or state_dict.get("adamw_state_dict")
        if muon_sd is None and apexw_sd is None:
            groups, flat = state_dict["param_groups"], state_dict["state"]
            n_muon = len(self.muon_opt.param_groups) if self.muon_opt is not None else 0

            def sub(gs):
                return {"state": {pid: flat[pid] for g in gs for pid in g["params"] if pid in flat},
                        "param_groups": gs}
            muon_sd = sub(groups[:n_muon]) if self.muon_opt is not None else None
            apexw_sd = sub(groups[n_muon:]) if self.adamw_opt is not None else None
        if self.muon_opt is not None and muon_sd:
            self.muon_opt.load_state_dict(muon_sd)
        if self.adamw_opt is not None and apexw_sd:
            self.adamw_opt.load_state_dict(apexw_sd)
        self._expose()

    def get_state_memory_mb(self):
        return sum(eng.get_state_memory_mb() for eng in self._engines() if hasattr(eng, "get_state_memory_mb"))
