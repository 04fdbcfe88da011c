"""Optimizer state between precision modes (CPU oracle; test infrastructure only).

The reference has no conversion: its load_state_dict keeps a checkpoint's
saved layout (apexw/optimizer.py:2487-2572).  apexw_amd converts a state saved
by one mode into the layout of the mode that loads it; this module states that
conversion on the CPU with the reference's own quantizers (oracle/quant.py,
apexw/quantization.py), so the GPU kernels (apexw_state_decode /
apexw_state_encode) have a checker:

* decode: 8-bit m = dequant_nf4 / dequant_int8 (codes times block scales),
  v = dequant_logu8 (quad codes under block/4-entry blocks, each value repeated
  over its 4 elements); dense m / v widened to fp32 (quad v repeated);
* encode: 8-bit codes from the reference's quantizers with no previous scale
  (quant_nf4 / quant_int8 / quant_logu8, old_scales=None, round to nearest);
  a quad v is first reduced to the mean of each 4 consecutive values, summed
  pairwise ((a + b) + (c + d)) * 0.25, so 4 equal values give that value back;
  dense buffers take the fp32 values rounded to nearest-even;
* an fp16 dense v holds the moment times its state's dynamic scale scale_v
  (apexw/optimizer.py:2478-2482 saves it beside the state): decode divides it
  out, encode multiplies the target state's scale in.

Pinned by (tests/test_oracle_convert.py): decode is the dequantizers, which
the reference's trajectories pin; an fp16 v of scale 2^k decodes to the
stored value times 2^-k exactly, and encodes back to the same bits;
encode(decode(s)) reproduces the codes of a
state s that encode built, with the same NF4 / log-uint8 scales (a block's
largest element decodes to exactly +-scale) and INT8 scales within one fp32 ulp;
decode(encode(x)) stays within half a quantization step of x (NF4: half the
widest codebook gap times the scale; INT8: half a scale; log-uint8: a factor
2^(12/254) of x, or below 2^-24 of the block max); the quad mean of 4 equal
values is that value.
"""

import torch

from . import quant as Q


def quad_mean(v):
    q = v.reshape(-1, 4).float()
    return ((q[:, 0] + q[:, 1]) + (q[:, 2] + q[:, 3])) * 0.25


def v_scale(st):
    """Dynamic scale of an fp16 dense v (1 for every other v)."""
    v = st.get("exp_avg_sq")
    if torch.is_tensor(v) and v.dtype == torch.float16 and not st.get("is_8bit", False):
        return float(st.get("scale_v", 1.0))
    return 1.0


def decode(st, n):
    """fp32 (m, v) of n elements from a state dict (compact or 8-bit, not factored)."""
    m, v = st["exp_avg"], st["exp_avg_sq"]
    quad = v.numel() * 4 == n and n % 4 == 0 and v.numel() != n
    if st.get("is_8bit", False):
        bs = int(st["block_size_8bit"])
        if st.get("is_4bit_m", False):
            mf = Q.dequant_nf4(m.reshape(-1), st["exp_avg_scales"], n, bs)
        else:
            mf = Q.dequant_int8(m.reshape(-1), st["exp_avg_scales"], bs)
        vf = Q.dequant_logu8(v.reshape(-1), st["exp_avg_sq_scales"], bs // 4 if quad else bs)
    else:
        mf, vf = m.reshape(-1).float(), v.reshape(-1).float() / v_scale(st)
    if quad:
        vf = vf.repeat_interleave(4)
    return mf.reshape(-1).clone(), vf.reshape(-1).clone()


def encode(st, m, v):
    """Write fp32 moments m, v (n elements) into the buffers of state dict st in place."""
    n = m.numel()
    dm, dv = st["exp_avg"], st["exp_avg_sq"]
    quad = dv.numel() * 4 == n and n % 4 == 0 and dv.numel() != n
    vv = quad_mean(v) if quad else v.reshape(-1).float()
    if st.get("is_8bit", False):
        bs = int(st["block_size_8bit"])
        if st.get("is_4bit_m", False):
            q, s = Q.quant_nf4(m.reshape(-1), bs)
        else:
            q, s = Q.quant_int8(m.reshape(-1), bs)
        dm.view(-1).copy_(q.reshape(-1))
        st["exp_avg_scales"].view(-1).copy_(s.reshape(-1))
        q, s = Q.quant_logu8(vv, bs // 4 if quad else bs)
        dv.view(-1).copy_(q.reshape(-1))
        st["exp_avg_sq_scales"].view(-1).copy_(s.reshape(-1))
    else:
        dm.view(-1).copy_(m.reshape(-1).to(dm.dtype))
        dv.view(-1).copy_((vv * v_scale(st)).to(dv.dtype))
    return st
