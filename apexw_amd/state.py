"""Optimizer-state layout rules and precision resolution for ApexW.

Decides, per parameter, how its moments are stored -- the decisions of the
reference's ``ApexW._init_group`` (apexw/optimizer.py:2574-2957) and resolvers
(apexw/state.py:62-162):

compact:
  * m in bf16 (fp16 for fp16 params); v in the same dtype, or fp32 when
    stochastic rounding is off and beta2 >= 0.995; an fp16 v is stored times a
    dynamic scale (scale_v, 1024 at first, recalibrated every 100 steps);
  * quad-v (one v per 4 consecutive elements, numel/4 entries) when m and v are
    16-bit, numel >= 16384, numel % 4 == 0, 1-D or min(shape) >= 8, and the
    group has >= 8 parameters (or the model is a PEFT/LoRA model).
8bit (numel >= 64):
  * block size: user value, else 128/64 for narrow 2-D tensors (min dim <= 32,
    numel < 2048), else 2048 halving down to 64;
  * NF4 m (2 codes per byte) + quad log-uint8 v when numel >= 16384,
    numel % 4 == 0, power-of-two block >= 64 and min(shape) >= 8; otherwise
    INT8 m + full-size log-uint8 v; fp32 scales per block;
  * factored_v=True: 2-D+ tensors of >= 65536 elements with rows, cols >= 128
    keep fp32 row / column second moments and INT8 m (packed 6-bit m with
    six_bit=True from 524,288 elements);
  * tensors under 64 elements keep compact 16-bit m/v.
compact with factored_v=True: the same factored v from 524,288 elements, bf16 m.
full (or fused=True): fp32 m and v for every parameter.
auto: fp32 m/v for an fp32 parameter when nothing points at mixed precision (no
  16-bit parameter in the optimizer, fp32 grad, amp not set, no PEFT); otherwise
  compact m/v (quad v and factored v as for compact) for 2-D tensors and 1-D ones
  of >= threshold elements, fp32 m/v for the other 1-D tensors.
ultra: INT8 m with one fp32 scale per 2048 elements (256 below 2048 elements)
  and a dense v in the compact v dtype, for 2-D tensors and 1-D ones of >=
  threshold elements; fp32 m/v for the rest.
Initial state: NF4 bytes 0x77 (both codes = 0.0), m scales 1e-12 (INT8: 1e-12/127),
v codes 0 with scales 1e-12.
"""

import torch

BETA2_V_FP32_THRESHOLD = 0.995

_ALIASES = {
    "full": ("full", "fp32", "float32", "float", "fp64", "float64", "double"),
    "compact": ("compact", "bf16", "bfloat16", "fp16", "float16", "half", "16", "16-bit"),
    "8bit": ("8bit", "8-bit", "int8", "uint8", "q8", "adamw_8bit", "bnb_8bit"),
    "ultra": ("ultra", "ultra_stable", "3byte", "hybrid8"),
    "hybrid": ("hybrid", "hybrid_apexw", "hybrid-apexw", "apex_hybrid", "hybrid_compact"),
    "auto": ("auto", "smart", "adaptive"),
}
HYBRID_ALIASES = _ALIASES["hybrid"]


def normalize_precision(precision):
    """Precision aliases -> canonical name (apexw/state.py:94-121)."""
    if isinstance(precision, torch.dtype):
        if precision in (torch.float32, torch.float64):
            return "full"
        if precision in (torch.bfloat16, torch.float16):
            return "compact"
        if precision in (torch.int8, torch.uint8):
            return "8bit"
        return "full"
    if isinstance(precision, str):
        key = precision.lower().strip()
        for name, aliases in _ALIASES.items():
            if key in aliases:
                return name
    raise ValueError(
        f"Invalid precision mode '{precision}'. Must be '8bit', 'compact', 'hybrid', 'ultra', 'auto', 'full', "
        f"or a valid torch dtype (e.g. torch.float32, torch.bfloat16, torch.float16, torch.int8).")


def is_peft_parameter(p):
    """LoRA/adapter naming, or a thin 2-D matrix (min dim <= 64, max dim >= 256)."""
    if getattr(p, "_is_lora", False):
        return True
    for attr in ("_param_name", "name"):
        val = getattr(p, attr, None)
        if isinstance(val, str):
            low = val.lower()
            if any(k in low for k in ("lora_a", "lora_b", "lora_embedding", "adapter", "lora_", "lora")):
                return True
    return p.dim() == 2 and min(p.shape) <= 64 and max(p.shape) >= 256


def detect_peft_context(param_groups):
    for g in param_groups:
        for p in g.get("params", []):
            if isinstance(p, torch.Tensor):
                if is_peft_parameter(p):
                    return True
                if hasattr(p, "quant_state") or hasattr(p, "quant_type") or type(p).__name__ in ("Params4bit", "Linear4bit"):
                    return True
    return False


def compact_dtype(p):
    if p.dtype == torch.float16:
        return torch.float16
    return torch.bfloat16


def v_dtype_for_beta2(cdt, beta2, force_compact_v=False, stochastic_rounding=True):
    if force_compact_v:
        return cdt
    if not stochastic_rounding and cdt in (torch.bfloat16, torch.float16) and beta2 >= BETA2_V_FP32_THRESHOLD:
        return torch.float32
    return cdt


def block_size_8bit(p, user_bs):
    n = p.numel()
    if user_bs is not None:
        return int(user_bs)
    if p.dim() >= 2 and min(p.shape) <= 32 and n < 2048:
        return 128 if n >= 128 else 64
    for bs in (2048, 1024, 512, 256, 128):
        if n >= bs:
            return bs
    return 64


def _auto_subbyte(p, group, bs, factored=False):
    """NF4 m + quad v eligibility (optimizer.py:2192-2201, the same rule in _init_group,
    where a factored tensor never takes it; never under amsgrad)."""
    n = p.numel()
    raw_int4 = group.get("int4_m", group.get("four_bit", None))
    pow2 = bs >= 64 and (bs & (bs - 1)) == 0
    return (raw_int4 is not False and not factored and not group.get("amsgrad", False)
            and not group.get("lion", False) and group.get("beta3") is None and n >= 16384 and n % 4 == 0 and pow2
            and (p.dim() < 2 or min(p.shape) >= 8))


FACTORED_MIN_8BIT = 65536       # apexw/state.py:234-256
FACTORED_MIN_COMPACT = 524288   # apexw/state.py:259-281
SIX_BIT_MIN = 524288            # optimizer.py:2667-2673
M6_ZERO = (0xDF, 0xF7, 0x7D)    # four codes of 31 (zero) in three bytes


def _can_factor(p, is_peft, min_numel, amsgrad=False):
    """Factored row/column v: 2-D+ real tensors, not under amsgrad, not PEFT, >= min_numel
    elements, rows = shape[0] >= 128 and cols = numel / rows >= 128 (apexw/state.py:234-281)."""
    if amsgrad or p.dim() < 2 or torch.is_complex(p) or p.dtype == torch.float64:
        return False
    rows = p.shape[0]
    cols = p.numel() // rows
    if is_peft or p.numel() < min_numel:
        return False
    return rows >= 128 and cols >= 128


def _factored_v(st, p):
    rows = p.shape[0]
    st["exp_avg_sq_row"] = torch.zeros(rows, dtype=torch.float32, device=p.device)
    st["exp_avg_sq_col"] = torch.zeros(p.numel() // rows, dtype=torch.float32, device=p.device)


def _q8_buffers(st, p, bs, int4, quad, factored=False, six=False):
    """8-bit state buffers: NF4 (packed, fill code 7), packed 6-bit (fill code 31) or
    INT8 m; quad or full log-u8 v, or factored fp32 row/column v; per-block fp32
    scales (optimizer.py:2798-2871)."""
    n, dev = p.numel(), p.device
    st.update(is_8bit=True, block_size_8bit=bs, is_factored_v=bool(factored), is_6bit_m=bool(six),
              is_4bit_m=bool(int4), is_quad_v=bool(quad), m_numel=n)
    st["state_dtype"] = torch.int8
    st["state_dtype_v"] = torch.uint8
    nblk = (n + bs - 1) // bs
    if six:
        padded = nblk * bs
        padded += (-padded) % 4
        st["exp_avg"] = torch.tensor(M6_ZERO, dtype=torch.uint8, device=dev).repeat(padded // 4)
        st["exp_avg_scales"] = torch.full((padded // bs, 1), 1e-12 / 31.0, dtype=torch.float32, device=dev)
    elif int4:
        st["exp_avg"] = torch.full(((n + 1) // 2,), 0x77, dtype=torch.uint8, device=dev)
        st["exp_avg_scales"] = torch.full((nblk, 1), 1e-12, dtype=torch.float32, device=dev)
    else:
        st["exp_avg"] = torch.zeros(p.shape, dtype=torch.int8, device=dev)
        st["exp_avg_scales"] = torch.full((nblk, 1), 1e-12 / 127.0, dtype=torch.float32, device=dev)
    if factored:
        _factored_v(st, p)
        return
    if quad:
        st["exp_avg_sq"] = torch.zeros((n // 4,), dtype=torch.uint8, device=dev)
    else:
        st["exp_avg_sq"] = torch.zeros(p.shape, dtype=torch.uint8, device=dev)
    st["exp_avg_sq_scales"] = torch.full((nblk, 1), 1e-12, dtype=torch.float32, device=dev)


def ensure_8bit_state(st, p, group):
    """The reference's _ensure_8bit_state_initialized (optimizer.py:2169-2224): the
    state the in-backward steps create lazily.  Unlike _init_group it makes
    8-bit buffers at any size and takes NF4 m exactly when quad v applies."""
    if "exp_avg" in st and "exp_avg_sq" in st:
        if st["exp_avg"].device != p.device:
            st["exp_avg"] = st["exp_avg"].to(p.device)
        if st["exp_avg_sq"].device != p.device:
            st["exp_avg_sq"] = st["exp_avg_sq"].to(p.device)
        return st
    st["stochastic_rounding"] = bool(group.get("stochastic_rounding", True))
    st["step"] = torch.tensor(0.0, dtype=torch.float32)
    bs = block_size_8bit(p, group.get("block_size"))
    sub = _auto_subbyte(p, group, bs)
    _q8_buffers(st, p, bs, sub, sub)
    return st


def _mixed_precision_in_sight(p, group, has_16bit_params, is_peft):
    """The "auto" precision's test for mixed-precision training
    (apexw/optimizer.py:2699-2708)."""
    return (bool(group.get("amp", False)) or has_16bit_params
            or (p.grad is not None and p.grad.dtype in (torch.float16, torch.bfloat16))
            or torch.is_autocast_enabled() or p.dtype in (torch.float16, torch.bfloat16) or is_peft)


def init_state(p, group, peft_ctx, has_16bit_params=False):
    """Fresh state dict for ``p`` (keys and dtypes as the reference's _init_group).

    has_16bit_params: whether any parameter of the optimizer is 16-bit (the
    "auto" precision keeps fp32 moments only when none is).  amsgrad adds
    ``max_exp_avg_sq`` (ensure_max_v)."""
    st = _init_state(p, group, peft_ctx, has_16bit_params)
    if group.get("amsgrad", False) and not group.get("lion", False):
        ensure_max_v(st, p)
    if group.get("beta3") is not None:
        ensure_slow(st, p)
    return st


def ensure_slow(st, p):
    """AdEMAMix's slow first moment (beta3): zeros in p's shape and m's dtype, created
    when missing (at init, or on the first step after beta3 is set: optimizer.py:2842-2845,
    :2903-2915).  Quantized states are not given one here (beta3 is refused there)."""
    if "exp_avg_slow" in st or st.get("is_8bit", False) or st.get("is_ultra", False):
        return
    st["exp_avg_slow"] = torch.zeros_like(p, dtype=st["exp_avg"].dtype, memory_format=torch.preserve_format)


def ensure_max_v(st, p):
    """amsgrad's running max of v: numel zeros in p's shape, fp32 for quantized v, else
    v's dtype (optimizer.py:2878-2886), created when missing (at init, or on the first
    step after amsgrad is switched on: :2917-2922)."""
    if "max_exp_avg_sq" in st:
        return
    quantized = st.get("is_8bit", False) or st.get("is_ultra", False)
    dt = torch.float32 if quantized else st.get("state_dtype_v", st.get("state_dtype", p.dtype))
    st["max_exp_avg_sq"] = torch.zeros(p.numel(), dtype=dt, device=p.device).reshape(p.shape)


def _init_state(p, group, peft_ctx, has_16bit_params):
    prec = group["precision"]
    beta2 = group["betas"][1]
    sr = bool(group.get("stochastic_rounding", True))
    dev = p.device
    n = p.numel()
    st = {"stochastic_rounding": sr, "step": torch.tensor(0.0, dtype=torch.float32)}
    is_peft = is_peft_parameter(p) or peft_ctx
    ams = bool(group.get("amsgrad", False))
    lion = bool(group.get("lion", False))
    slow = group.get("beta3") is not None
    large = p.dim() >= 2 or n >= group.get("threshold", 65536)
    if group.get("fused") is True or prec == "full":
        # optimizer.py:2625-2626, :2769-2772
        st.update(is_factored_v=False, is_6bit_m=False)
        return _moments(st, p, torch.float32, group, is_peft, prec)
    if prec == "ultra":
        # optimizer.py:2736-2748, :2779-2784, :2816-2834
        st.update(is_factored_v=False, is_6bit_m=False)
        if not large:
            st["is_ultra"] = False
            return _moments(st, p, torch.float32, group, is_peft, prec)
        bs = 2048 if n >= 2048 else 256
        vdt = v_dtype_for_beta2(compact_dtype(p), beta2, group.get("force_compact_v", False), sr)
        st.update(is_ultra=True, ultra_block_size=bs, state_dtype=torch.int8, state_dtype_v=vdt)
        st["exp_avg"] = torch.zeros(p.shape, dtype=torch.int8, device=dev)
        st["exp_avg_scales"] = torch.full(((n + bs - 1) // bs, 1), 1e-12 / 127.0, dtype=torch.float32, device=dev)
        st["exp_avg_sq"] = torch.zeros(p.shape, dtype=vdt, device=dev)
        return st
    if prec == "auto":
        # optimizer.py:2694-2735 (the parameters here are on the GPU)
        st.update(is_factored_v=False, is_6bit_m=False)
        fp32_training = p.dtype == torch.float32 and not _mixed_precision_in_sight(p, group, has_16bit_params,
                                                                                   is_peft)
        if fp32_training or not large:
            return _moments(st, p, torch.float32, group, is_peft, prec)
        if bool(group.get("factored_v", False)) and _can_factor(p, is_peft, FACTORED_MIN_COMPACT, ams or lion or slow):
            st["is_factored_v"] = True
            return _factored_compact(st, p)
        return _moments(st, p, compact_dtype(p), group, is_peft, prec)
    if prec == "8bit" and n >= 64:
        bs = block_size_8bit(p, group.get("block_size"))
        narrow = p.dim() >= 2 and min(p.shape) <= 32 and n < 2048
        factored = bool(group.get("factored_v", False)) and _can_factor(p, is_peft, FACTORED_MIN_8BIT, ams or lion or slow)
        auto_sub = _auto_subbyte(p, group, bs, factored)
        raw_int4 = group.get("int4_m", group.get("four_bit", None))
        six = bool(group.get("six_bit", False)) and factored and n >= SIX_BIT_MIN and bs % 4 == 0
        int4 = auto_sub or (bool(raw_int4) and not factored and n >= 512 and n >= bs and not narrow and not is_peft)
        _q8_buffers(st, p, bs, int4, bool(auto_sub and int4), factored, six)
        return st
    if prec == "8bit":
        st.update(is_8bit=False, is_factored_v=False, is_6bit_m=False, is_4bit_m=False, is_quad_v=False)
    else:
        factored = bool(group.get("factored_v", False)) and _can_factor(p, is_peft, FACTORED_MIN_COMPACT, ams or lion or slow)
        st.update(is_6bit_m=False, is_4bit_m=False, is_factored_v=factored)
        if factored:
            return _factored_compact(st, p)
    return _moments(st, p, compact_dtype(p), group, is_peft, prec)


def _factored_compact(st, p):
    """16-bit m, fp32 row/column v (optimizer.py:2749-2767, :2785-2787, :2859-2863)."""
    st["state_dtype"] = compact_dtype(p)
    st["state_dtype_v"] = torch.float32
    st["exp_avg"] = torch.zeros(p.shape, dtype=compact_dtype(p), device=p.device)
    _factored_v(st, p)
    st["scale_v"] = 1.0
    st["sqrt_scale_v"] = 1.0
    return st


def _moments(st, p, mdt, group, is_peft, prec):
    """Dense m in ``mdt``, v in the beta2 rule's dtype, quad v for large 16-bit
    compact / auto tensors, not under nesterov, amsgrad, lion or beta3; no v under lion
    (optimizer.py:2788-2810, :2838-2872)."""
    n, dev = p.numel(), p.device
    vdt = v_dtype_for_beta2(mdt, group["betas"][1], group.get("force_compact_v", False),
                            bool(group.get("stochastic_rounding", True)))
    quad = (prec in ("compact", "auto") and mdt in (torch.bfloat16, torch.float16)
            and vdt in (torch.bfloat16, torch.float16)
            and group.get("int4_m", None) is not False and not group.get("nesterov", False)
            and not group.get("amsgrad", False) and not group.get("lion", False)
            and group.get("beta3") is None and n >= 16384 and n % 4 == 0
            and (p.dim() < 2 or min(p.shape) >= 8)
            and (is_peft or len(group["params"]) >= 8))
    if quad:
        st["is_quad_v"] = True
    st["state_dtype"] = mdt
    st["state_dtype_v"] = vdt
    # in the parameter's layout (channels_last and the like), as zeros_like(p,
    # memory_format=torch.preserve_format) gives it (optimizer.py:2848-2850, :2873-2875)
    st["exp_avg"] = torch.zeros_like(p, dtype=mdt, memory_format=torch.preserve_format)
    lion = bool(group.get("lion", False))
    if lion:
        pass                       # lion keeps no second moment (optimizer.py:2857)
    elif quad:
        st["exp_avg_sq"] = torch.zeros((n // 4,), dtype=vdt, device=dev)
    else:
        st["exp_avg_sq"] = torch.zeros_like(p, dtype=vdt, memory_format=torch.preserve_format)
    # an fp16 v holds the second moment times a dynamic scale, 1024 at first
    # (optimizer.py:2889-2898); every other v is unscaled
    scaled = bool(group.get("dynamic_scaling", True)) and vdt == torch.float16 and not lion
    st["scale_v"] = 1024.0 if scaled else 1.0
    st["sqrt_scale_v"] = 32.0 if scaled else 1.0
    return st


def state_bytes_per_param(state, numel):
    tot = sum(v.numel() * v.element_size() for k, v in state.items()
              if isinstance(v, torch.Tensor) and k != "step")
    return tot / max(numel, 1)
