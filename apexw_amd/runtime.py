"""Process-wide runtime state of the automatic 8-bit path.

The reference keeps module-level registries and patches torch when its
optimizer module is imported (apexw/optimizer.py:1346-1507); this module does
the same for ``apexw_amd``:

* ``DOWNCAST``: parameters an 8-bit ApexW converted from fp32 to bf16 at
  construction.  They are converted back (and every optimizer's in-backward
  hooks removed) when another optimizer is constructed -- unless it is another
  8-bit ApexW and no 8-bit ApexW has stepped yet --, when a module owning one
  of them loads a state dict, and when ``torch.cuda.reset_peak_memory_stats``
  is called after a step.
* AMP detection for the in-backward steps: ``GradScaler.scale`` records the
  scale of the running backward (the in-backward steps unscale with it),
  ``GradScaler.update`` forgets it; with fp16 parameters in play the scale is
  clamped to 256.

``install()`` applies these patches once per process, and only when an 8-bit
ApexW turns its in-backward steps on (the reference patches at import); an
application that never takes that path sees torch unchanged.

``StateMap`` is the ``optimizer.state`` of ApexW and ApexMuon under GradScaler
steps read on the device.
"""

import weakref
from collections import defaultdict

import torch
import torch.nn as nn
from torch.optim.optimizer import Optimizer

DOWNCAST = {}      # id(p) -> (weakref to p, dtype before the downcast)
OPTIMIZERS = []    # weakrefs to the ApexW instances holding in-backward hooks

fp16_active = False
amp_scaled_this_backward = False
last_amp_scale = None
_installed = False


class StateMap(defaultdict):
    """``optimizer.state`` with step counters that are exact when looked at
    (ApexW, ApexMuon).

    A step whose GradScaler found_inf is read by the kernels advances the host's
    counters optimistically; the device knows which steps were skipped.  The
    first lookup of a state after such a step has the owner subtract them (its
    ``_fold_amp_skips``, one wait), so ``opt.state[p]["step"]`` reads as the
    reference's, whose skipped steps leave it alone.  Inside ``step()`` the
    lookups do not wait (the owner's ``_amp_unfolded`` is cleared meanwhile)."""

    def __init__(self, owner, items=()):
        super().__init__(dict, items)
        self._owner = owner

    def _fold(self):
        o = self._owner
        if o is not None and o._amp_unfolded:
            o._fold_amp_skips()

    def __getitem__(self, key):
        self._fold()
        return super().__getitem__(key)

    def get(self, key, default=None):
        self._fold()
        return super().get(key, default)

    def items(self):
        self._fold()
        return super().items()

    def values(self):
        self._fold()
        return super().values()

    def __reduce__(self):
        # pickles and deep copies hold a plain defaultdict(dict), as torch's optimizers
        # do, with the step counters made exact first
        self._fold()
        return defaultdict, (dict,), None, None, iter(dict.items(self))


def _is_downcast(p):
    entry = DOWNCAST.get(id(p))
    return entry is not None and entry[0]() is p


def register_downcast(p, orig_dtype):
    if not _is_downcast(p):
        DOWNCAST[id(p)] = (weakref.ref(p), orig_dtype)


def register_optimizer(opt):
    if not any(r() is opt for r in OPTIMIZERS):
        OPTIMIZERS.append(weakref.ref(opt))


def any_stepped():
    return any(r() is not None and getattr(r(), "_has_stepped", False) for r in OPTIMIZERS)


def restore_all_downcast_params():
    """Convert every downcast parameter (and its grad) back to its original dtype
    and remove every optimizer's in-backward hooks (optimizer.py:1352-1382)."""
    global fp16_active, amp_scaled_this_backward
    fp16_active = False
    amp_scaled_this_backward = False
    for ref in list(OPTIMIZERS):
        opt = ref()
        if opt is not None:
            opt._disable_auto_8bit_hooks()
    OPTIMIZERS.clear()
    if not DOWNCAST:
        return
    with torch.no_grad():
        for ref, dtype in list(DOWNCAST.values()):
            p = ref()
            if p is None or p.dtype == dtype:
                continue
            p.data = p.data.to(dtype)
            if p.grad is not None and p.grad.dtype != dtype:
                p.grad = p.grad.to(dtype)
    DOWNCAST.clear()


def install():
    """Patch torch once per process (the patches of optimizer.py:1385-1507 that the
    in-backward steps need)."""
    global _installed
    if _installed:
        return
    _installed = True
    _patch_grad_scaler()
    _patch_optimizer_init()
    _patch_module_load_state_dict()
    _patch_reset_peak_memory_stats()


def _patch_grad_scaler():
    from torch.amp.grad_scaler import GradScaler
    if getattr(GradScaler, "_apexw_amd_patched", False):
        return
    orig_scale, orig_update = GradScaler.scale, GradScaler.update

    def scale(self, outputs):
        global amp_scaled_this_backward, last_amp_scale
        if getattr(self, "_enabled", False):
            if isinstance(outputs, torch.Tensor) and self._scale is None:
                self._lazy_init_scale_growth_tracker(outputs.device)
            if self._scale is not None:
                if fp16_active:
                    with torch.no_grad():
                        self._scale.clamp_(max=256.0)
                if last_amp_scale is None:
                    last_amp_scale = float(self._scale.item())
                amp_scaled_this_backward = True
        return orig_scale(self, outputs)

    def update(self, new_scale=None):
        global amp_scaled_this_backward, last_amp_scale
        res = orig_update(self, new_scale=new_scale)
        amp_scaled_this_backward = False
        last_amp_scale = None
        return res

    GradScaler.scale = scale
    GradScaler.update = update
    GradScaler._apexw_amd_patched = True


def _patch_optimizer_init():
    if getattr(Optimizer, "_apexw_amd_init_patched", False):
        return
    orig_init = Optimizer.__init__

    def __init__(self, params, defaults):
        if DOWNCAST:
            from .optimizer import ApexW
            from .state import normalize_precision
            is_8bit = (isinstance(self, ApexW) and isinstance(defaults, dict)
                       and normalize_precision(defaults.get("precision", "compact")) == "8bit")
            if not is_8bit or any_stepped():
                restore_all_downcast_params()
        return orig_init(self, params, defaults)

    Optimizer.__init__ = __init__
    Optimizer._apexw_amd_init_patched = True


def _patch_module_load_state_dict():
    if getattr(nn.Module, "_apexw_amd_load_sd_patched", False):
        return
    orig_load = nn.Module.load_state_dict

    def load_state_dict(self, state_dict, *args, **kwargs):
        if DOWNCAST and any(_is_downcast(p) for p in self.parameters()):
            restore_all_downcast_params()
        return orig_load(self, state_dict, *args, **kwargs)

    nn.Module.load_state_dict = load_state_dict
    nn.Module._apexw_amd_load_sd_patched = True


def _patch_reset_peak_memory_stats():
    if getattr(torch.cuda, "_apexw_amd_reset_peak_patched", False):
        return
    orig_reset = torch.cuda.reset_peak_memory_stats

    def reset_peak_memory_stats(*args, **kwargs):
        if DOWNCAST:
            if any_stepped():
                restore_all_downcast_params()
            if torch.cuda.is_available():
                torch.cuda.empty_cache()
        return orig_reset(*args, **kwargs)

    torch.cuda.reset_peak_memory_stats = reset_peak_memory_stats
    torch.cuda._apexw_amd_reset_peak_patched = True


def step_hooks(func):
    """torch.optim.Optimizer's step wrapper (``Optimizer.profile_hook_step``) with
    the same hook semantics: global and per-optimizer pre hooks (which may
    replace args / kwargs), ``_optimizer_step_code``, then post hooks.  The
    ``Optimizer.step#<class>.step`` profiler range is opened only while a
    profiler runs: outside one, entering and leaving it is a large share of a
    small model's host time per step.  Marked ``hooked`` so that
    ``Optimizer._patch_step_function`` does not wrap the method again."""
    import functools
    from itertools import chain

    from torch.optim import optimizer as _opt

    def run(self, args, kwargs):
        for pre_hook in chain(_opt._global_optimizer_pre_hooks.values(), self._optimizer_step_pre_hooks.values()):
            result = pre_hook(self, args, kwargs)
            if result is not None:
                if isinstance(result, tuple) and len(result) == 2:
                    args, kwargs = result
                else:
                    raise RuntimeError(f"{func} must return None or a tuple of (new_args, new_kwargs), but got {result}.")
        out = func(*args, **kwargs)
        self._optimizer_step_code()
        for post_hook in chain(self._optimizer_step_post_hooks.values(), _opt._global_optimizer_post_hooks.values()):
            post_hook(self, args, kwargs)
        return out

    @functools.wraps(func)
    def wrapper(*args, **kwargs):
        self = args[0]
        if torch.autograd._profiler_enabled():
            with torch.autograd.profiler.record_function(f"Optimizer.step#{self.__class__.__name__}.step"):
                return run(self, args, kwargs)
        return run(self, args, kwargs)

    wrapper.hooked = True
    return wrapper
