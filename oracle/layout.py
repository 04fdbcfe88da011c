"""Per-parameter optimizer-state layout (CPU oracle; test infrastructure only).

Restates the decisions of the reference's ``ApexW._init_group``
(``apexw/optimizer.py:2574-2957``) and the dtype resolvers in
``apexw/state.py:62-162`` for the ``compact`` and ``8bit`` precisions.
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


def can_factor(p, is_peft, min_numel):
    """state.py:234-281: 2-D+, not PEFT, >= min_numel (65536 for 8bit, 524288 for
    compact), rows = shape[0] >= 128, cols = numel / rows >= 128."""
    if p.dim() < 2 or torch.is_complex(p) or p.dtype == torch.float64 or is_peft or p.numel() < min_numel:
        return False
    return p.shape[0] >= 128 and p.numel() // p.shape[0] >= 128


def init_state(p, group, n_params_in_group, peft_ctx):
    """Allocate and return a fresh state dict for parameter ``p``."""
    prec = group["precision"]
    beta2 = group["betas"][1]
    sr = bool(group["stochastic_rounding"])
    st = {"stochastic_rounding": sr, "step": torch.tensor(0.0, dtype=torch.float32)}
    n = p.numel()
    is_peft = is_peft_param(p) or peft_ctx
    if prec == "8bit" and n >= 64:
        bs = block_size_8bit(p, group.get("block_size"))
        narrow = p.dim() >= 2 and min(p.shape) <= 32 and n < 2048
        raw_int4 = group.get("int4_m")
        pow2 = bs >= 64 and (bs & (bs - 1)) == 0
        fv = bool(group.get("factored_v", False)) and can_factor(p, is_peft, 65536)
        auto_sub = (raw_int4 is not False and not fv and n >= 16384 and n % 4 == 0 and pow2
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
        fv = bool(group.get("factored_v", False)) and can_factor(p, is_peft, 524288)
        st.update(is_6bit_m=False, is_4bit_m=False, is_factored_v=fv)
        if fv:
            st["state_dtype"] = compact_dtype(p)
            st["state_dtype_v"] = torch.float32
            st["exp_avg"] = torch.zeros(p.shape, dtype=compact_dtype(p))
            st["exp_avg_sq_row"] = torch.zeros(p.shape[0], dtype=torch.float32)
            st["exp_avg_sq_col"] = torch.zeros(n // p.shape[0], dtype=torch.float32)
            st["scale_v"] = 1.0
            st["sqrt_scale_v"] = 1.0
            return st
    else:
        raise NotImplementedError(f"oracle covers compact and 8bit, not {prec!r}")
    mdt = compact_dtype(p)
    vdt = v_dtype(mdt, beta2, group.get("force_compact_v", False), sr)
    quad = (prec == "compact" and mdt in (torch.bfloat16, torch.float16) and vdt in (torch.bfloat16, torch.float16)
            and group.get("int4_m") is not False and n >= 16384 and n % 4 == 0
            and (p.dim() < 2 or min(p.shape) >= 8) and (is_peft or n_params_in_group >= 8))
    if quad:
        st["is_quad_v"] = True
    st["state_dtype"] = mdt
    st["state_dtype_v"] = vdt
    st["exp_avg"] = torch.zeros(p.shape, dtype=mdt)
    st["exp_avg_sq"] = torch.zeros((n // 4,), dtype=vdt) if quad else torch.zeros(p.shape, dtype=vdt)
    st["scale_v"] = 1.0
    st["sqrt_scale_v"] = 1.0
    return st
