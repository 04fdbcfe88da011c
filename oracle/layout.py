"""Per-parameter optimizer-state layout (CPU oracle; test infrastructure only).

Restates the decisions of the reference's ``ApexW._init_group``
(``apexw/optimizer.py:2574-2957``) and the dtype resolvers in
``apexw/state.py:62-162`` for the ``compact``, ``8bit``, ``full``, ``auto`` and
``ultra`` precisions.

``auto`` keeps fp32 moments for an fp32 parameter on a CUDA device when no
mixed precision is in sight (optimizer.py:2712-2715); ``cuda=True`` (the
default) takes that branch for the GPU parameters the product steps, whose CPU
copies the oracle updates.
"""

import torch

BETA2_V_FP32 = 0.995  # state.py:43


def is_peft_param(p):
    """state.py:62-78: LoRA/adapter names, or thin 2-D matrices (min<=64, max>=256)."""
    if getattr(p, "_is_lora", False):
        return True
    for attr in ("_param_name", "name"):
        val = getattr(p, attr, None)
        if isinstance(val, str) and any(k in val.lower() for k in ("lora_a", "lora_b", "lora_embedding", "adapter", "lora_", "lora")):
            return True
    return p.dim() == 2 and min(p.shape) <= 64 and max(p.shape) >= 256


def peft_context(param_groups):
    """state.py:81-91."""
    for g in param_groups:
        for p in g["params"]:
            if isinstance(p, torch.Tensor):
                if is_peft_param(p):
                    return True
                if hasattr(p, "quant_state") or hasattr(p, "quant_type") or type(p).__name__ in ("Params4bit", "Linear4bit"):
                    return True
    return False


def compact_dtype(p):
    """state.py:124-136 (CPU/CUDA branch)."""
    if p.dtype == torch.float16:
        return torch.float16
    return torch.bfloat16


def v_dtype(cdt, beta2, force_compact_v, stochastic):
    """state.py:139-162: fp32 v only when SR is off and beta2 >= 0.995."""
    if force_compact_v:
        return cdt
    if not stochastic and cdt in (torch.bfloat16, torch.float16) and beta2 >= BETA2_V_FP32:
        return torch.float32
    return cdt


def block_size_8bit(p, user_bs):
    """optimizer.py:2632-2642: user block, narrow 2-D (128/64), else 2048 halving down to 64."""
    n = p.numel()
    if user_bs is not None:
        return user_bs
    if p.dim() >= 2 and min(p.shape) <= 32 and n < 2048:
        return 128 if n >= 128 else 64
    for bs in (2048, 1024, 512, 256, 128):
        if n >= bs:
            return bs
    return 64


def can_factor(p, is_peft, min_numel, amsgrad=False):
    """state.py:234-281: 2-D+, not amsgrad, not PEFT, >= min_numel (65536 for 8bit,
    524288 for compact), rows = shape[0] >= 128, cols = numel / rows >= 128."""
    if amsgrad or p.dim() < 2 or torch.is_complex(p) or p.dtype == torch.float64 or is_peft or p.numel() < min_numel:
        return False
    return p.shape[0] >= 128 and p.numel() // p.shape[0] >= 128


def amp_active(p, group, has_16bit_params, is_peft):
    """optimizer.py:2699-2708 (autocast outside step() aside)."""
    return (bool(group.get("amp", False)) or has_16bit_params
            or (p.grad is not None and p.grad.dtype in (torch.float16, torch.bfloat16))
            or p.dtype in (torch.float16, torch.bfloat16) or is_peft)


def init_state(p, group, n_params_in_group, peft_ctx, has_16bit_params=None, cuda=True):
    """Allocate and return a fresh state dict for parameter ``p``.

    has_16bit_params: whether any parameter of the optimizer is 16-bit (None:
    this parameter's group decides); cuda: lay out as for a CUDA parameter.
    amsgrad adds ``max_exp_avg_sq``: numel zeros in p's shape, fp32 for quantized v,
    else v's dtype (optimizer.py:2878-2886)."""
    st = _init_state(p, group, n_params_in_group, peft_ctx, has_16bit_params, cuda)
    if group.get("amsgrad", False) and not group.get("lion", False):
        ensure_max_v(st, p)
    if group.get("beta3") is not None:
        ensure_slow(st, p)
    return st


def ensure_slow(st, p):
    """beta3's slow first moment, zeros in p's shape and m's dtype, created when missing
    (optimizer.py:2842-2845, :2903-2915; quantized states aside)."""
    if "exp_avg_slow" in st or st.get("is_8bit", False) or st.get("is_ultra", False):
        return
    st["exp_avg_slow"] = torch.zeros_like(p, dtype=st["exp_avg"].dtype, memory_format=torch.preserve_format)


def ensure_max_v(st, p):
    """amsgrad's running max of v, created when missing (at init, or on the first step
    after amsgrad is switched on: optimizer.py:2917-2922)."""
    if "max_exp_avg_sq" in st:
        return
    quantized = st.get("is_8bit", False) or st.get("is_ultra", False)
    dt = torch.float32 if quantized else st.get("state_dtype_v", st.get("state_dtype", p.dtype))
    st["max_exp_avg_sq"] = torch.zeros(p.numel(), dtype=dt, device=p.device).reshape(p.shape)


def _init_state(p, group, n_params_in_group, peft_ctx, has_16bit_params, cuda):
    prec = group["precision"]
    beta2 = group["betas"][1]
    sr = bool(group["stochastic_rounding"])
    st = {"stochastic_rounding": sr, "step": torch.tensor(0.0, dtype=torch.float32)}
    n = p.numel()
    is_peft = is_peft_param(p) or peft_ctx
    ams = bool(group.get("amsgrad", False))
    lion = bool(group.get("lion", False))
    slow = group.get("beta3") is not None
    threshold = group.get("threshold", 65536)
    massive = p.dim() >= 2 or n >= threshold
    if group.get("fused") is True or prec == "full":
        # fp32 moments whatever the parameter dtype (optimizer.py:2625-2626, :2769-2772)
        st.update(is_factored_v=False, is_6bit_m=False)
        return _dense(st, p, torch.float32, group, is_peft, n_params_in_group, prec)
    if prec == "ultra":
        # INT8 block-quantized m and a dense v for 2-D or large tensors, fp32 m/v
        # for the rest (optimizer.py:2736-2748, :2779-2784, :2816-2834)
        st.update(is_factored_v=False, is_6bit_m=False)
        if not massive:
            st["is_ultra"] = False
            return _dense(st, p, torch.float32, group, is_peft, n_params_in_group, prec)
        bs = 2048 if n >= 2048 else 256
        vdt = v_dtype(compact_dtype(p), beta2, group.get("force_compact_v", False), sr)
        st.update(is_ultra=True, ultra_block_size=bs, state_dtype=torch.int8, state_dtype_v=vdt)
        st["exp_avg"] = torch.zeros(p.shape, dtype=torch.int8)
        st["exp_avg_scales"] = torch.full(((n + bs - 1) // bs, 1), 1e-12 / 127.0, dtype=torch.float32)
        st["exp_avg_sq"] = torch.zeros(p.shape, dtype=vdt)
        return st
    if prec == "auto":
        # optimizer.py:2694-2735: fp32 moments for pure-fp32 CUDA training, else 16-bit
        # for 2-D or large tensors and fp32 for small ones
        st.update(is_factored_v=False, is_6bit_m=False)
        if has_16bit_params is None:
            has_16bit_params = any(q.dtype in (torch.float16, torch.bfloat16) for q in group.get("params", ()))
        if cuda and p.dtype == torch.float32 and not amp_active(p, group, has_16bit_params, is_peft):
            return _dense(st, p, torch.float32, group, is_peft, n_params_in_group, prec)
        if not massive:
            return _dense(st, p, torch.float32, group, is_peft, n_params_in_group, prec)
        cdt = compact_dtype(p)
        if bool(group.get("factored_v", False)) and can_factor(p, is_peft, 524288, ams or lion or slow):
            st["is_factored_v"] = True
            return _factored_compact(st, p, cdt)
        return _dense(st, p, cdt, group, is_peft, n_params_in_group, prec)
    if prec == "8bit" and n >= 64:
        bs = block_size_8bit(p, group.get("block_size"))
        narrow = p.dim() >= 2 and min(p.shape) <= 32 and n < 2048
        raw_int4 = group.get("int4_m")
        pow2 = bs >= 64 and (bs & (bs - 1)) == 0
        fv = bool(group.get("factored_v", False)) and can_factor(p, is_peft, 65536, ams or lion or slow)
        auto_sub = (raw_int4 is not False and not fv and not ams and not lion and not slow and n >= 16384 and n % 4 == 0 and pow2
                    and (p.dim() < 2 or min(p.shape) >= 8))
        six = bool(group.get("six_bit", False)) and fv and n >= 524288 and bs % 4 == 0
        int4 = auto_sub or (bool(raw_int4) and not fv and n >= 512 and n >= bs and not narrow and not is_peft)
        quad = bool(auto_sub and int4)
        st.update(is_8bit=True, block_size_8bit=bs, is_factored_v=fv, is_6bit_m=six,
                  is_4bit_m=int4, is_quad_v=quad, m_numel=n,
                  state_dtype=torch.int8, state_dtype_v=torch.uint8)
        nblk = (n + bs - 1) // bs
        if six:
            padded = n + (bs - n % bs) % bs
            padded += (4 - padded % 4) % 4
            st["exp_avg"] = torch.tensor([0xDF, 0xF7, 0x7D], dtype=torch.uint8).repeat(padded // 4)
            st["exp_avg_scales"] = torch.full((padded // bs, 1), 1e-12 / 31.0, dtype=torch.float32)
        elif int4:
            st["exp_avg"] = torch.full(((n + 1) // 2,), 0x77, dtype=torch.uint8)
            st["exp_avg_scales"] = torch.full((nblk, 1), 1e-12, dtype=torch.float32)
        else:
            st["exp_avg"] = torch.zeros(p.shape, dtype=torch.int8)
            st["exp_avg_scales"] = torch.full((nblk, 1), 1e-12 / 127.0, dtype=torch.float32)
        if fv:
            st["exp_avg_sq_row"] = torch.zeros(p.shape[0], dtype=torch.float32)
            st["exp_avg_sq_col"] = torch.zeros(n // p.shape[0], dtype=torch.float32)
            return st
        st["exp_avg_sq"] = (torch.zeros((n // 4,), dtype=torch.uint8) if quad
                            else torch.zeros(p.shape, dtype=torch.uint8))
        st["exp_avg_sq_scales"] = torch.full((nblk, 1), 1e-12, dtype=torch.float32)
        return st
    if prec == "8bit":
        st.update(is_8bit=False, is_factored_v=False, is_6bit_m=False, is_4bit_m=False, is_quad_v=False)
    elif prec == "compact":
        fv = bool(group.get("factored_v", False)) and can_factor(p, is_peft, 524288, ams or lion or slow)
        st.update(is_6bit_m=False, is_4bit_m=False, is_factored_v=fv)
        if fv:
            return _factored_compact(st, p, compact_dtype(p))
    else:
        raise NotImplementedError(f"oracle does not cover precision {prec!r}")
    return _dense(st, p, compact_dtype(p), group, is_peft, n_params_in_group, prec)


def _factored_compact(st, p, mdt):
    """16-bit m, fp32 row / column v (optimizer.py:2785-2787, :2859-2863)."""
    n = p.numel()
    st["state_dtype"] = mdt
    st["state_dtype_v"] = torch.float32
    st["exp_avg"] = torch.zeros(p.shape, dtype=mdt)
    st["exp_avg_sq_row"] = torch.zeros(p.shape[0], dtype=torch.float32)
    st["exp_avg_sq_col"] = torch.zeros(n // p.shape[0], dtype=torch.float32)
    st["scale_v"] = 1.0
    st["sqrt_scale_v"] = 1.0
    return st


def _dense(st, p, mdt, group, is_peft, n_params_in_group, prec):
    """m in ``mdt``, v in the dtype the beta2 rule gives, quad-shared v for large
    16-bit compact/auto tensors, not under nesterov, amsgrad, lion or beta3; no v under lion
    (optimizer.py:2788-2810, :2838-2872)."""
    n = p.numel()
    vdt = v_dtype(mdt, group["betas"][1], group.get("force_compact_v", False), bool(group["stochastic_rounding"]))
    quad = (prec in ("compact", "auto") and mdt in (torch.bfloat16, torch.float16)
            and vdt in (torch.bfloat16, torch.float16)
            and group.get("int4_m") is not False and not group.get("nesterov", False)
            and not group.get("amsgrad", False) and not group.get("lion", False)
            and group.get("beta3") is None and n >= 16384 and n % 4 == 0
            and (p.dim() < 2 or min(p.shape) >= 8) and (is_peft or n_params_in_group >= 8))
    if quad:
        st["is_quad_v"] = True
    st["state_dtype"] = mdt
    st["state_dtype_v"] = vdt
    # in the parameter's memory layout (zeros_like(p, memory_format=torch.preserve_format),
    # optimizer.py:2848-2850, :2873-2875): torch._fused_adamw_ walks its tensors in memory order
    st["exp_avg"] = torch.zeros_like(p, dtype=mdt, memory_format=torch.preserve_format)
    lion = bool(group.get("lion", False))
    if not lion:                   # lion keeps no second moment (optimizer.py:2857)
        st["exp_avg_sq"] = (torch.zeros((n // 4,), dtype=vdt) if quad
                            else torch.zeros_like(p, dtype=vdt, memory_format=torch.preserve_format))
    # fp16 v starts with a dynamic scale of 1024 (optimizer.py:2889-2898)
    fp16_scaled = bool(group.get("dynamic_scaling", True)) and vdt == torch.float16 and not lion
    st["scale_v"] = 1024.0 if fp16_scaled else 1.0
    st["sqrt_scale_v"] = 32.0 if fp16_scaled else 1.0
    return st
