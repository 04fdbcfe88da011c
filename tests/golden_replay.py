"""Replay the golden trajectories (tests/golden/*.npz) against any optimizer factory.

Inputs are regenerated with the same seeded generator and call order as
``tests/golden/make_golden.py``; the stored fingerprints prove they match.
"""

import os

import numpy as np
import torch

from golden.make_golden import (FP16_CASES, FUSED_CASES, FUSED_SHAPES, FV_KW, FV_Q8_SHAPES, GRAD_DTYPE_CASES, HOOK_KW,
                                 HOOK_SHAPES, PREC_CASES, SD_CASES, _fingerprint, _grad, _param)
from golden.sd_codec import decode

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

# name -> (shapes, dtype, steps, seed, kwargs, grad_scales, zero_grad_idx); mirrors make_golden.py
SHAPES_BF16 = [(128, 256), (64, 512), (16384,), (256, 96), (768,), (768,), (100,), (8, 4096), (3, 5), (36, 64)]
RAGGED = [(300,), (64, 70), (16384,), (128, 128), (17,), (4, 1024), (1000,), (32, 33), (20000,)]
RAGGED_SCALES = [10.0, 0.1, 1.0, 3.0, 0.5, 7.0, 0.2, 1.5, 0.05]
Q8_SHAPES = [(512, 1024), (256, 256), (100, 300), (4096,), (1000,), (50,), (3000,), (16, 100), (64, 33)]
CASES = {
    "compact_c1_fp32_rne": ([(16384,)], torch.float32, 10, 0,
                            dict(lr=1e-3, weight_decay=0.1, adamw_compat=True, stochastic_rounding=False), None, ()),
    "compact_bf16_quad_rne": (SHAPES_BF16, torch.bfloat16, 10, 1,
                              dict(lr=1e-3, weight_decay=0.1, stochastic_rounding=False), None, ()),
    "compact_bf16_fp32v_rne": (SHAPES_BF16, torch.bfloat16, 10, 2,
                               dict(lr=1e-3, weight_decay=0.1, adamw_compat=True, stochastic_rounding=False), None, ()),
    "compact_fp32_quad_rne": (SHAPES_BF16, torch.float32, 10, 3,
                              dict(lr=1e-3, weight_decay=0.1, stochastic_rounding=False), None, ()),
    "compact_bf16_clip_rne": (RAGGED, torch.bfloat16, 6, 4,
                              dict(lr=1e-3, weight_decay=0.1, stochastic_rounding=False, clip_grad_norm=1.0),
                              RAGGED_SCALES, (4,)),
    "compact_fp32_clip_rne": (RAGGED, torch.float32, 6, 8,
                              dict(lr=1e-3, weight_decay=0.1, stochastic_rounding=False, clip_grad_norm=1.0),
                              RAGGED_SCALES, (4,)),
    "q8_bf16_rne": (Q8_SHAPES, torch.bfloat16, 5, 5,
                    dict(lr=1e-3, weight_decay=0.1, adamw_compat=True, precision="8bit", stochastic_rounding=False),
                    None, ()),
    "q8_fp32_rne": ([(300, 1000), (128, 128), (2048,), (700,)], torch.float32, 4, 6,
                    dict(lr=1e-3, weight_decay=0.1, adamw_compat=True, precision="8bit", stochastic_rounding=False),
                    None, ()),
}


# factored-v trajectories (every state tensor recorded as st_<i>_<key>)
FV_CASES = {
    "fv_q8_bf16_rne": (FV_Q8_SHAPES, torch.bfloat16, 4, 21, dict(FV_KW, precision="8bit"), None, ()),
    "fv_q8_fp32_rne": ([(256, 256), (700,)], torch.float32, 3, 22, dict(FV_KW, precision="8bit"), None, ()),
    "fv_6bit_bf16_rne": ([(512, 1024)], torch.bfloat16, 3, 23, dict(FV_KW, precision="8bit", six_bit=True),
                         None, ()),
    "fv_compact_bf16_rne": ([(512, 1024), (768,)], torch.bfloat16, 3, 24, FV_KW, None, ()),
    "fv_q8_fp16_rne": ([(256, 256), (640, 512), (700,)], torch.float16, 3, 25, dict(FV_KW, precision="8bit"),
                       None, ()),
    "fv_compact_fp16_rne": ([(512, 1024), (768,)], torch.float16, 3, 26, FV_KW, None, ()),
    "fv_q8_bf16_maximize_rne": ([(256, 256), (640, 512), (700,)], torch.bfloat16, 3, 27,
                                dict(FV_KW, precision="8bit", maximize=True), None, ()),
    "fv_compact_bf16_maximize_rne": ([(512, 1024), (768,)], torch.bfloat16, 3, 28, dict(FV_KW, maximize=True),
                                     None, ()),
}
CASES.update(FV_CASES)
# the full / auto / ultra precisions (every state tensor recorded)
PREC_NAMES = sorted(PREC_CASES)
CASES.update({k: (sh, dt, n, seed, kw, None, ()) for k, (sh, dt, n, seed, kw) in PREC_CASES.items()})
# fp16 parameters (every state tensor and the v scales recorded); the eighth entry lists
# (step, parameter) pairs without a grad
FP16_NAMES = sorted(FP16_CASES)
CASES.update({k: (sh, torch.float16, n, seed, kw, None, (), ng) for k, (sh, n, seed, kw, ng) in FP16_CASES.items()})
# grads of another dtype than their parameters: the ninth entry is the grads' dtype
CASES.update({k: (sh, dt, n, seed, kw, None, (), (), gd) for k, (sh, dt, gd, n, seed, kw) in GRAD_DTYPE_CASES.items()})
# in-backward trajectories: name -> (steps, backward passes per step, seed, parameter dtype)
HOOK_CASES = {"hooks_k1_rne": (3, 1, 31, torch.float32), "hooks_k2_rne": (3, 2, 32, torch.float32),
              "hooks_fp16_k2_rne": (3, 2, 33, torch.float16)}


def load(name):
    with np.load(os.path.join(GOLDEN, f"{name}.npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def to_torch(arr, like_dtype):
    if like_dtype == torch.bfloat16:
        return torch.from_numpy(arr.astype(np.uint16).view(np.int16)).view(torch.bfloat16)
    return torch.from_numpy(np.ascontiguousarray(arr))


def replay(name, make_opt, device="cpu", get_state=None):
    """Run case ``name`` with ``make_opt(params, **kwargs)``; return (params, opt, golden dict)."""
    shapes, dtype, steps, seed, kwargs, scales, zidx = CASES[name][:7]
    none_grad = CASES[name][7] if len(CASES[name]) > 7 else ()
    grad_dtype = CASES[name][8] if len(CASES[name]) > 8 else None
    gold = load(name)
    gen = torch.Generator().manual_seed(seed)
    host = [_param(s, dtype, gen) for s in shapes]
    fp = [_fingerprint(p) for p in host]
    params = [torch.nn.Parameter(h.to(device)) for h in host]
    if grad_dtype is not None:
        for p in params:
            p.grad_dtype = grad_dtype
    opt = make_opt(params, **kwargs)
    for step in range(steps):
        for i, p in enumerate(params):
            g = _grad(p.shape, dtype if grad_dtype is None else grad_dtype, gen,
                      1e-3 if scales is None else scales[i])
            if i in zidx:
                g.zero_()
            fp.append(_fingerprint(g))
            p.grad = None if (step, i) in none_grad else g.to(device)
        opt.step()
    np.testing.assert_array_equal(np.array(fp, dtype=np.int64), gold["fingerprint"])
    return params, opt, gold


def bf16_ulp_diff(a, b):
    """Distance in bf16 units-in-the-last-place between two bf16 tensors (sign-aware)."""
    ia = a.view(torch.int16).to(torch.int32)
    ib = b.view(torch.int16).to(torch.int32)
    ia = torch.where(ia < 0, -(ia & 0x7FFF), ia)
    ib = torch.where(ib < 0, -(ib & 0x7FFF), ib)
    return (ia - ib).abs()


def hook_inputs(name):
    """Initial parameters (fp32 or fp16) and, per step, per pass, the grads of the
    in-backward case ``name`` (grads in the dtype each parameter has after the downcast)."""
    from oracle import hooks as H
    steps, passes, seed, dtype = HOOK_CASES[name]
    gold = load(name)
    gen = torch.Generator().manual_seed(seed)
    host = [_param(s, dtype, gen) for s in HOOK_SHAPES]
    fp = [_fingerprint(p) for p in host]
    dts = [H.downcast_dtype(p) for p in host]
    grads = []
    for _ in range(steps):
        per_step = []
        for _ in range(passes):
            gs = [_grad(p.shape, dt, gen) for p, dt in zip(host, dts)]
            fp.extend(_fingerprint(g) for g in gs)
            per_step.append(gs)
        grads.append(per_step)
    np.testing.assert_array_equal(np.array(fp, dtype=np.int64), gold["fingerprint"])
    return host, grads, gold


def fused_inputs(name):
    """enable_fused_backward case ``name``: (dtype, kwargs, initial parameters, per
    step the list of per-pass grads, golden dict)."""
    dtype, steps, passes, seed, kwargs = FUSED_CASES[name]
    gold = load(name)
    gen = torch.Generator().manual_seed(seed)
    host = [_param(s, dtype, gen) for s in FUSED_SHAPES]
    fp = [_fingerprint(p) for p in host]
    grads = []
    for _ in range(steps):
        per_step = []
        for _ in range(passes):
            gs = [_grad(p.shape, dtype, gen) for p in host]
            fp.extend(_fingerprint(g) for g in gs)
            per_step.append(gs)
        grads.append(per_step)
    np.testing.assert_array_equal(np.array(fp, dtype=np.int64), gold["fingerprint"])
    return dtype, kwargs, host, grads, gold


def sd_inputs(name):
    """(shapes, dtype, kwargs, the reference's state_dict after 3 steps, the parameters
    then, the grads of the 2 steps after it, the golden dict) of checkpoint case ``name``."""
    shapes, dtype, kwargs = SD_CASES[name]
    gold = load(name)
    gen = torch.Generator().manual_seed(41 + list(SD_CASES).index(name))
    host = [_param(s, dtype, gen) for s in shapes]
    fp = [_fingerprint(p) for p in host]
    grads = []
    for step in range(5):
        gs = [_grad(p.shape, dtype, gen) for p in host]
        fp.extend(_fingerprint(g) for g in gs)
        if step >= 3:
            grads.append(gs)
    np.testing.assert_array_equal(np.array(fp, dtype=np.int64), gold["fingerprint"])
    sd = decode(str(gold["sd_skeleton"]), {k: v for k, v in gold.items() if k.startswith("sd_")})
    mid = [to_torch(gold[f"pmid_{i}"], dtype).reshape(s) for i, s in enumerate(shapes)]
    return shapes, dtype, kwargs, sd, mid, grads, gold


def state_keys(gold, i):
    """The state tensor names recorded for parameter i."""
    pre = f"st_{i}_"
    return sorted(k[len(pre):] for k in gold if k.startswith(pre))


def initial_params(name):
    """The parameters case ``name`` starts from (the generator's first draws)."""
    shapes, dtype, steps, seed, kwargs, scales, zidx = CASES[name][:7]
    gen = torch.Generator().manual_seed(seed)
    return [_param(s, dtype, gen) for s in shapes]
