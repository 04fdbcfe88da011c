"""Optimizer state across precision modes, converted on the GPU.

The reference keeps a checkpoint's saved layout when it loads one
(apexw/optimizer.py:2487-2572): its groups take the saved hyperparameters,
precision included, and a state written by one mode cannot be stepped by
another.  ``ApexW.set_precision`` here moves a loaded (or live) state into
another mode's layout: each parameter's moments are decoded to fp32 and
re-encoded in the layout a fresh state of the new mode would have
(``state.init_state``), by the kernels behind ``apexw_state_decode`` /
``apexw_state_encode`` (csrc/convert.hip).  The step counts carry over, so
the bias correction continues where the checkpoint left off.

An fp16 v holds the second moment times its state's dynamic scale (scale_v,
a power of two): decode divides it out and encode multiplies the new state's
scale in, both exactly.  The scale a state records is the one its checkpoint
carries (the reference's _dynamic_scaling_meta).

Factored second moments (row / column EMAs) are not converted: a state with
them, or a target layout that would have them, raises NotImplementedError.
"""

import ctypes

import torch

from . import _lib as L
from . import state as S

_DT = {torch.float32: L.F32, torch.bfloat16: L.BF16, torch.float16: L.F16}


def family(st):
    """(8-bit codes?, factored v?) of a state dict: what decides whether a layout can
    be stepped by a precision mode's kernels."""
    return bool(st.get("is_8bit", False)), bool(st.get("is_factored_v", False))


def target_family(p, group, peft):
    """family() of the fresh state ``group``'s precision would give ``p`` (no allocation)."""
    meta = torch.empty(p.shape, dtype=p.dtype, device="meta")
    return family(S.init_state(meta, dict(group, params=group["params"]), peft or S.is_peft_parameter(p)))


def _layout(st, n):
    m, v = st["exp_avg"], st["exp_avg_sq"]
    lay = L.StateLayout()
    lay.m, lay.v, lay.n = m.data_ptr(), v.data_ptr(), n
    quad = v.numel() != n and v.numel() * 4 == n
    flags = L.FLAG_QUAD if quad else 0
    if st.get("is_8bit", False):
        lay.kind = L.STATE_Q8
        lay.block = int(st["block_size_8bit"])
        lay.m_scale = st["exp_avg_scales"].data_ptr()
        lay.v_scale = st["exp_avg_sq_scales"].data_ptr()
        if st.get("is_4bit_m", False):
            flags |= L.FLAG_NF4
    else:
        if m.dtype not in _DT or v.dtype not in _DT:
            raise NotImplementedError(f"state dtypes {m.dtype} / {v.dtype} cannot be converted")
        lay.kind = L.STATE_DENSE
        flags |= (_DT[m.dtype] << L.MDT_SHIFT) | (_DT[v.dtype] << L.VDT_SHIFT)
    lay.flags = flags
    return lay


def v_scale(st):
    """The dynamic scale an fp16 v of state ``st`` holds (1 for every other v)."""
    v = st.get("exp_avg_sq")
    if torch.is_tensor(v) and v.dtype == torch.float16 and not st.get("is_8bit", False):
        return float(st.get("scale_v", 1.0))
    return 1.0


def convert(p, st, group, peft):
    """A new state for ``p`` in the layout ``group``'s precision gives it, holding the
    moments of ``st`` (another mode's state); the step count carries over."""
    if p.device.type != "cuda":
        raise RuntimeError("apexw_amd converts optimizer state on the GPU; parameters must be on cuda")
    if family(st)[1]:
        raise NotImplementedError("converting a factored second moment (row / column EMAs) is not supported")
    target = S.init_state(p, group, peft or S.is_peft_parameter(p))
    if family(target)[1]:
        raise NotImplementedError("converting into a factored second moment (factored_v=True) is not supported")
    n = p.numel()
    src = {k: (v.to(p.device).contiguous() if torch.is_tensor(v) and k != "step" else v) for k, v in st.items()}
    m32 = torch.empty(n, dtype=torch.float32, device=p.device)
    v32 = torch.empty(n, dtype=torch.float32, device=p.device)
    lib = L.load()
    with torch.cuda.device(p.device):
        stream = torch.cuda.current_stream(p.device).cuda_stream
        L.check(lib.apexw_state_decode(ctypes.byref(_layout(src, n)), m32.data_ptr(), v32.data_ptr(), stream),
                "apexw_state_decode")
        ratio = v_scale(target) / v_scale(st)
        if ratio != 1.0:
            v32.mul_(ratio)               # powers of two: exact
        L.check(lib.apexw_state_encode(ctypes.byref(_layout(target, n)), m32.data_ptr(), v32.data_ptr(), stream),
                "apexw_state_encode")
    if "max_exp_avg_sq" in target and "max_exp_avg_sq" in st:
        # amsgrad's running max carries over, rounded to the new layout's dtype
        target["max_exp_avg_sq"].copy_(src["max_exp_avg_sq"].reshape(target["max_exp_avg_sq"].shape))
    step = st.get("step")
    target["step"] = (step.detach().to("cpu", torch.float32).clone() if torch.is_tensor(step)
                      else torch.tensor(float(step or 0.0), dtype=torch.float32))
    return target
