"""Write the golden input/output vectors that pin the CPU oracle to the reference.

Run once, in a container that has the reference checkout (read-only) at
``/root/reference``::

    python tests/golden/make_golden.py [--ref /root/reference]

The reference's CPU paths are imported from that checkout and stepped on small,
seeded inputs. Only data is written: ``tests/golden/*.npz`` holds inputs and the
reference's outputs (bf16 tensors stored as their uint16 bit patterns). Nothing
from the reference is copied; the tests never import it.

Functions covered, with the reference entry points they exercise:
  * compact foreach trajectories   -> ApexW._multi_tensor_step (optimizer.py:5297-5887)
  * 8-bit trajectories             -> ApexW._step_ultra         (optimizer.py:4313-4735)
  * global-norm clip               -> _prepare_grads            (optimizer.py:204-258)
  * state layout decisions         -> ApexW._init_group         (optimizer.py:2574-2957)
  * hybrid routing                 -> partition_parameters_for_hybrid (hybrid.py:89-141)
  * Newton-Schulz / Muon step      -> muon.py:102-211, :539-861 (CPU fp32 work dtype)
  * factored-v / 6-bit trajectories -> _apply_factored_v_int8_update (state.py:442-652) through
                                      _step_ultra / _multi_tensor_step, several steps
  * in-backward 8-bit steps        -> _flush_auto_8bit_hook_queue (optimizer.py:2226-2371), K = 1 and 2
  * enable_fused_backward          -> _step_single_param_fused (optimizer.py:1986-2043, :2373-2471),
                                      6 steps, 8-bit and compact, grad_accum_steps 1 and 2
  * checkpoints                    -> ApexW / HybridApexW state_dict (optimizer.py:2473-2485,
                                      hybrid.py:436-472), plus the steps after them
  * full / auto / ultra precisions -> _init_group, _fused_step, _multi_tensor_step, _step_ultra
  * nesterov=True                  -> _step_ultra's Nesterov numerators (optimizer.py:4444-4445,
                                      :4581-4582, :4667-4670, :4719-4724); the compact, full
                                      and auto steps' (:5732-5733, :5865-5877, :1276-1277,
                                      :1329-1331)
  * cautious=True                  -> _step_ultra's cautious mask (optimizer.py:4583-4588, :4672-4675,
                                      :4726-4729); the compact, full and auto steps'
                                      (:5728-5731, :5847-5864, :1272-1275, :1321-1328)
  * maximize=True                  -> _step_ultra's negated grads (optimizer.py:4502-4503,
                                      state.py:341-342); the compact, full and auto steps'
                                      (:1104-1105, :5515-5517)
All runs use stochastic_rounding=False: the reference draws SR noise from torch's
global RNG, so SR outputs cannot be pinned bit-wise and are tested statistically.
"""

import argparse
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)


def _np(t):
    """A copy of the tensor's values (bf16 as uint16 bit patterns): never a view of
    storage that later steps keep updating in place."""
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()
    return t.contiguous().numpy().copy()


def _fingerprint(t):
    """Platform-independent digest of a tensor's bytes (two 31-bit words)."""
    import hashlib
    b = t.detach().cpu().contiguous().view(torch.uint8).numpy().tobytes()
    h = hashlib.sha256(b).digest()
    return [int.from_bytes(h[:4], "little") >> 1, int.from_bytes(h[4:8], "little") >> 1]


def _grad(shape, dtype, gen, scale=1e-3):
    return (torch.randn(shape, generator=gen, dtype=torch.float32) * scale).to(dtype)


def _param(shape, dtype, gen):
    return (torch.randn(shape, generator=gen, dtype=torch.float32) * 0.02).to(dtype)


def _record_state(out, opt, params):
    """Every tensor of every parameter's state (all layouts: compact, 8-bit, factored)."""
    for i, p in enumerate(params):
        for key, val in opt.state[p].items():
            if torch.is_tensor(val) and key != "step":
                out[f"st_{i}_{key}"] = _np(val)
        out[f"step_{i}"] = np.array([float(opt.state[p]["step"])], dtype=np.float64)
        if "scale_v" in opt.state[p]:
            out[f"scale_{i}"] = np.array([float(opt.state[p]["scale_v"]), float(opt.state[p]["sqrt_scale_v"])])


def run_trajectory(ApexW, shapes, dtype, steps, seed, opt_kwargs, grad_scales=None, zero_grad_idx=(),
                   record_all=False, none_grad=(), grad_dtype=None):
    """Step ApexW on CPU and record inputs per step plus the final state
    (record_all: every state tensor, keyed st_<i>_<key>, instead of m / v / scales).
    none_grad: (step, parameter) pairs whose grad is None at that step (its grad is
    still drawn, so the inputs of later steps do not shift).  grad_dtype: the grads'
    dtype when it differs from the parameters' (torch's Tensor.grad_dtype)."""
    gen = torch.Generator().manual_seed(seed)
    params = [torch.nn.Parameter(_param(s, dtype, gen)) for s in shapes]
    if grad_dtype is not None:
        for p in params:
            p.grad_dtype = grad_dtype
    out = {}
    # Inputs are regenerated by the tests from the same seeded generator; only a
    # fingerprint is stored so that a generator change is detected.
    fp = [_fingerprint(p.data) for p in params]
    opt = ApexW(params, **opt_kwargs)
    for step in range(steps):
        for i, p in enumerate(params):
            sc = 1e-3 if grad_scales is None else grad_scales[i]
            g = _grad(p.shape, dtype if grad_dtype is None else grad_dtype, gen, sc)
            if i in zero_grad_idx:
                g.zero_()
            p.grad = None if (step, i) in none_grad else g
            fp.append(_fingerprint(g))
        opt.step()
    out["fingerprint"] = np.array(fp, dtype=np.int64)
    if record_all:
        for i, p in enumerate(params):
            out[f"p_{i}"] = _np(p.data)
        _record_state(out, opt, params)
        return out
    for i, p in enumerate(params):
        st = opt.state[p]
        out[f"p_{i}"] = _np(p.data)
        out[f"m_{i}"] = _np(st["exp_avg"])
        out[f"v_{i}"] = _np(st["exp_avg_sq"])
        if "exp_avg_scales" in st:
            out[f"ms_{i}"] = _np(st["exp_avg_scales"])
            out[f"vs_{i}"] = _np(st["exp_avg_sq_scales"])
        out[f"flags_{i}"] = np.array([
            int(bool(st.get("is_quad_v", False))),
            int(bool(st.get("is_4bit_m", False))),
            int(bool(st.get("is_8bit", False))),
            int(st.get("block_size_8bit", 0) or 0),
        ], dtype=np.int64)
    out["meta_shapes"] = np.array([list(s) + [0] * (2 - len(s)) for s in shapes], dtype=np.int64)
    out["meta_ndim"] = np.array([len(s) for s in shapes], dtype=np.int64)
    out["meta_steps"] = np.array([steps], dtype=np.int64)
    return out


def golden_compact(ApexW):
    cases = {}
    # C1 shape family (one flat fp32 tensor), SR off -> fp32 v (beta2=0.999 via adamw_compat).
    cases["compact_c1_fp32_rne"] = run_trajectory(
        ApexW, [(16384,)], torch.float32, 10, 0,
        dict(lr=1e-3, weight_decay=0.1, adamw_compat=True, stochastic_rounding=False))
    # bf16 list with quad-v (>=8 params, default compact betas -> bf16 v), decay_norm_only.
    shapes_bf16 = [(128, 256), (64, 512), (16384,), (256, 96), (768,), (768,), (100,), (8, 4096), (3, 5), (36, 64)]
    cases["compact_bf16_quad_rne"] = run_trajectory(
        ApexW, shapes_bf16, torch.bfloat16, 10, 1,
        dict(lr=1e-3, weight_decay=0.1, stochastic_rounding=False))
    # bf16 list, adamw_compat + SR off -> bf16 m, fp32 v, no quad; wd on all tensors.
    cases["compact_bf16_fp32v_rne"] = run_trajectory(
        ApexW, shapes_bf16, torch.bfloat16, 10, 2,
        dict(lr=1e-3, weight_decay=0.1, adamw_compat=True, stochastic_rounding=False))
    # fp32 params with bf16 state and quad-v.
    cases["compact_fp32_quad_rne"] = run_trajectory(
        ApexW, shapes_bf16, torch.float32, 10, 3,
        dict(lr=1e-3, weight_decay=0.1, stochastic_rounding=False))
    # Global-norm clipping inside the step (ragged, per-tensor grad scales, some all-zero).
    ragged = [(300,), (64, 70), (16384,), (128, 128), (17,), (4, 1024), (1000,), (32, 33), (20000,)]
    scales = [10.0, 0.1, 1.0, 3.0, 0.5, 7.0, 0.2, 1.5, 0.05]
    cases["compact_bf16_clip_rne"] = run_trajectory(
        ApexW, ragged, torch.bfloat16, 6, 4,
        dict(lr=1e-3, weight_decay=0.1, stochastic_rounding=False, clip_grad_norm=1.0),
        grad_scales=scales, zero_grad_idx=(4,))
    # The same with fp32 parameters and grads: the clip's fp32 norms (torch's CPU
    # reduction) feed fp32 moments and parameters.
    cases["compact_fp32_clip_rne"] = run_trajectory(
        ApexW, ragged, torch.float32, 6, 8,
        dict(lr=1e-3, weight_decay=0.1, stochastic_rounding=False, clip_grad_norm=1.0),
        grad_scales=scales, zero_grad_idx=(4,))
    return cases


Q8_SHAPES = [(512, 1024), (256, 256), (100, 300), (4096,), (1000,), (50,), (3000,), (16, 100), (64, 33)]


def golden_8bit(ApexW):
    cases = {}
    cases["q8_bf16_rne"] = run_trajectory(
        ApexW, Q8_SHAPES, torch.bfloat16, 5, 5,
        dict(lr=1e-3, weight_decay=0.1, adamw_compat=True, precision="8bit", stochastic_rounding=False))
    cases["q8_fp32_rne"] = run_trajectory(
        ApexW, [(300, 1000), (128, 128), (2048,), (700,)], torch.float32, 4, 6,
        dict(lr=1e-3, weight_decay=0.1, adamw_compat=True, precision="8bit", stochastic_rounding=False))
    return cases


FV_Q8_SHAPES = [(256, 256), (640, 512), (4096,), (300,)]
FV_KW = dict(lr=1e-3, weight_decay=0.1, adamw_compat=True, stochastic_rounding=False, factored_v=True)


def golden_factored(ApexW):
    """Factored second moment (row / column fp32 EMAs of g^2) over several steps from
    the state the earlier steps left: INT8 m (one-piece (256, 256) and row-chunked
    (640, 512) statistics), packed 6-bit m, and the compact bf16-m form."""
    cases = {}
    cases["fv_q8_bf16_rne"] = run_trajectory(
        ApexW, FV_Q8_SHAPES, torch.bfloat16, 4, 21, dict(FV_KW, precision="8bit"), record_all=True)
    cases["fv_q8_fp32_rne"] = run_trajectory(
        ApexW, [(256, 256), (700,)], torch.float32, 3, 22, dict(FV_KW, precision="8bit"), record_all=True)
    cases["fv_6bit_bf16_rne"] = run_trajectory(
        ApexW, [(512, 1024)], torch.bfloat16, 3, 23, dict(FV_KW, precision="8bit", six_bit=True), record_all=True)
    cases["fv_compact_bf16_rne"] = run_trajectory(
        ApexW, [(512, 1024), (768,)], torch.bfloat16, 3, 24, FV_KW, record_all=True)
    # fp16 parameters: decay and update in fp32, clamped, one rounding (state.py:405-410); fp16 m
    cases["fv_q8_fp16_rne"] = run_trajectory(
        ApexW, [(256, 256), (640, 512), (700,)], torch.float16, 3, 25, dict(FV_KW, precision="8bit"),
        record_all=True)
    cases["fv_compact_fp16_rne"] = run_trajectory(
        ApexW, [(512, 1024), (768,)], torch.float16, 3, 26, FV_KW, record_all=True)
    # maximize: the grads negated before sanitizing and unscaling (state.py:430-439)
    cases["fv_q8_bf16_maximize_rne"] = run_trajectory(
        ApexW, [(256, 256), (640, 512), (700,)], torch.bfloat16, 3, 27, dict(FV_KW, precision="8bit", maximize=True),
        record_all=True)
    cases["fv_compact_bf16_maximize_rne"] = run_trajectory(
        ApexW, [(512, 1024), (768,)], torch.bfloat16, 3, 28, dict(FV_KW, maximize=True), record_all=True)
    return cases


HOOK_SHAPES = [(256, 1024), (512, 512), (128, 256), (256,), (64, 512), (300, 100), (16384,), (128, 128),
               (1024,), (96, 256)]
HOOK_KW = dict(lr=1e-3, weight_decay=0.1, adamw_compat=True, precision="8bit", stochastic_rounding=False)


def run_hooked(ApexW, shapes, steps, passes, seed, kwargs, dtype=torch.float32):
    """In-backward 8-bit steps: fp32 parameters (the large ones become bf16 at
    construction) or fp16 ones (kept), `passes` backward passes per optimizer step,
    each handing every parameter a fresh grad through p.view_as(p), then step() and
    zero_grad()."""
    gen = torch.Generator().manual_seed(seed)
    params = [torch.nn.Parameter(_param(s, dtype, gen)) for s in shapes]
    fp = [_fingerprint(p.data) for p in params]
    opt = ApexW(params, **kwargs)
    out = {"dtypes": np.array([_dtype_code(p.dtype) for p in params], dtype=np.int64)}
    for _ in range(steps):
        for _ in range(passes):
            grads = [_grad(p.shape, p.dtype, gen) for p in params]
            fp.extend(_fingerprint(g) for g in grads)
            torch.autograd.backward([p.view_as(p) for p in params], grad_tensors=grads)
        opt.step()
        opt.zero_grad(set_to_none=True)
    out["fingerprint"] = np.array(fp, dtype=np.int64)
    for i, p in enumerate(params):
        out[f"p_{i}"] = _np(p.data)
    _record_state(out, opt, params)
    opt._disable_auto_8bit_hooks()
    return out


def golden_hooks(ApexW):
    """The reference's in-backward 8-bit path (_flush_auto_8bit_hook_queue) over
    several steps: one backward per step, and two (gradient accumulation, K = 2)."""
    return {"hooks_k1_rne": run_hooked(ApexW, HOOK_SHAPES, 3, 1, 31, HOOK_KW),
            "hooks_k2_rne": run_hooked(ApexW, HOOK_SHAPES, 3, 2, 32, HOOK_KW),
            "hooks_fp16_k2_rne": run_hooked(ApexW, HOOK_SHAPES, 3, 2, 33, HOOK_KW, dtype=torch.float16)}


FUSED_SHAPES = [(256, 512), (128, 256), (300, 100), (512,), (40, 8), (33,)]
# enable_fused_backward: name -> (dtype, steps, backward passes per step (grad_accum_steps), seed, kwargs);
# six tensors, fewer than the eight the automatic in-backward path needs, so only these hooks run
FUSED_CASES = {
    "fused_8bit_bf16_k1": (torch.bfloat16, 6, 1, 61,
                           dict(lr=1e-2, weight_decay=0.1, precision="8bit", stochastic_rounding=False)),
    "fused_8bit_fp32_k2": (torch.float32, 6, 2, 62,
                           dict(lr=1e-2, weight_decay=0.1, precision="8bit", stochastic_rounding=False)),
    "fused_compact_bf16_k1": (torch.bfloat16, 6, 1, 63, dict(lr=1e-2, weight_decay=0.1, stochastic_rounding=False)),
    "fused_compact_fp32_k2": (torch.float32, 6, 2, 64, dict(lr=1e-2, weight_decay=0.1, stochastic_rounding=False)),
    # fp16 parameters: fp16 moments in the compact precision (state.py:124-129), no dynamic v scale
    "fused_compact_fp16_k2": (torch.float16, 6, 2, 65, dict(lr=1e-2, weight_decay=0.1, stochastic_rounding=False)),
    "fused_8bit_fp16_k1": (torch.float16, 6, 1, 66,
                           dict(lr=1e-2, weight_decay=0.1, precision="8bit", stochastic_rounding=False)),
}


def run_fused(ApexW, dtype, steps, passes, seed, kwargs):
    """enable_fused_backward (_step_single_param_fused inside each parameter's
    post-accumulate hook) over several steps: `passes` backward passes per step,
    each handing every parameter a fresh grad through p.view_as(p); step() then
    finds no grads left."""
    gen = torch.Generator().manual_seed(seed)
    params = [torch.nn.Parameter(_param(s, dtype, gen)) for s in FUSED_SHAPES]
    fp = [_fingerprint(p.data) for p in params]
    opt = ApexW(params, **kwargs)
    opt.enable_fused_backward(grad_accum_steps=passes)
    for _ in range(steps):
        for _ in range(passes):
            grads = [_grad(p.shape, dtype, gen) for p in params]
            fp.extend(_fingerprint(g) for g in grads)
            torch.autograd.backward([p.view_as(p) for p in params], grad_tensors=grads)
        assert all(p.grad is None for p in params)
        opt.step()
        opt.zero_grad(set_to_none=True)
    out = {"fingerprint": np.array(fp, dtype=np.int64)}
    for i, p in enumerate(params):
        out[f"p_{i}"] = _np(p.data)
    _record_state(out, opt, params)
    opt.disable_fused_backward()
    return out


def golden_fused(ApexW):
    return {name: run_fused(ApexW, *case) for name, case in FUSED_CASES.items()}


SD_CASES = {
    "sd_compact": ([(128, 256), (16384,), (768,), (100,), (8, 4096)], torch.bfloat16,
                   dict(lr=1e-3, weight_decay=0.1, stochastic_rounding=False)),
    "sd_q8": ([(512, 256), (4096,), (1000,), (50,), (64, 33)], torch.bfloat16,
              dict(lr=1e-3, weight_decay=0.1, adamw_compat=True, precision="8bit", stochastic_rounding=False)),
    "sd_hybrid": ([(64, 64), (64, 64), (48, 96), (64,), (1024, 32)], torch.float32,
                  dict(lr=1e-3, weight_decay=0.1, use_muon=True, stochastic_rounding=False)),
}


def golden_state_dict(ApexW):
    """Checkpoints written by the reference: 3 steps, state_dict() (stored as a JSON
    skeleton plus arrays, tests/golden/sd_codec.py); then the resume: a new
    optimizer over the parameters of that moment loads the stored dict and takes
    2 more steps, whose results a loader of that checkpoint must reproduce."""
    from sd_codec import decode, encode
    cases = {}
    for name, (shapes, dtype, kwargs) in SD_CASES.items():
        gen = torch.Generator().manual_seed(41 + len(cases))
        params = [torch.nn.Parameter(_param(s, dtype, gen)) for s in shapes]
        fp = [_fingerprint(p.data) for p in params]
        opt = ApexW(params, **kwargs)
        out = {}
        for step in range(5):
            if step == 3:
                skel, arrays = encode(opt.state_dict(), prefix="sd_")
                out["sd_skeleton"] = np.array(skel)
                out.update(arrays)
                for i, p in enumerate(params):
                    out[f"pmid_{i}"] = _np(p.data)
                params = [torch.nn.Parameter(p.detach().clone()) for p in params]
                opt = ApexW(params, **kwargs)
                opt.load_state_dict(decode(skel, arrays))
            for p in params:
                g = _grad(p.shape, dtype, gen)
                fp.append(_fingerprint(g))
                p.grad = g
            opt.step()
        out["fingerprint"] = np.array(fp, dtype=np.int64)
        for i, p in enumerate(params):
            out[f"p_{i}"] = _np(p.data)
        st = opt.state
        for i, p in enumerate(params):
            for key, val in st[p].items():
                if torch.is_tensor(val) and key != "step":
                    out[f"st_{i}_{key}"] = _np(val)
        cases[name] = out
    return cases


CLIP_SHAPES = [(300,), (64, 70), (16384,), (17,), (1000,)]
CLIP_SCALES = [10.0, 0.1, 1.0, 0.5, 7.0]
CLIP_FP32_SHAPES = [(300,), (64, 70), (1 << 20,), (17,), (1000, 300)]
CLIP_FP32_KEEP = 4096


def golden_clip(opt_mod):
    gen = torch.Generator().manual_seed(7)
    shapes, scales = CLIP_SHAPES, CLIP_SCALES
    out = {}
    grads = []
    for i, (s, sc) in enumerate(zip(shapes, scales)):
        g = _grad(s, torch.bfloat16, gen, sc)
        out[f"g_{i}"] = _np(g)
        grads.append(g.clone())
    res, _ = opt_mod._prepare_grads(grads, {"clip_grad_norm": 1.0}, None, sanitize=True)
    for i, g in enumerate(res):
        out[f"gc_{i}"] = _np(g)
    # fp32 grads, up to 2^20 elements: the norms are torch's CPU fp32 reductions.  The
    # grads are regenerated by the test from the generator (their fingerprints are
    # stored); the clipped values are kept for the first CLIP_FP32_KEEP elements.
    out32 = {}
    grads, fps = [], []
    for s, sc in zip(CLIP_FP32_SHAPES, scales):
        g = _grad(s, torch.float32, gen, sc)
        fps.append(_fingerprint(g))
        grads.append(g.clone())
    res, _ = opt_mod._prepare_grads(grads, {"clip_grad_norm": 1.0}, None, sanitize=True)
    for i, g in enumerate(res):
        out32[f"gc_{i}"] = _np(g).reshape(-1)[:CLIP_FP32_KEEP]
    out32["fingerprint"] = np.array(fps, dtype=np.int64)
    return {"clip_bf16": out, "clip_fp32": out32}


def golden_layout(ApexW):
    """Record _init_group's layout for the benchmark parameter sets (meta tensors, no data)."""
    from apexw.optimizer import ApexW as _A  # noqa: F401
    def record(shapes, dtype, kwargs):
        params = [torch.nn.Parameter(torch.empty(s, dtype=dtype, device="meta")) for s in shapes]
        for p in params:
            p.grad = torch.empty_like(p)
        opt = ApexW(params, **kwargs)
        group = opt.param_groups[0]
        lists = [[] for _ in range(7)]
        opt._init_group(group, *lists)
        rows = []
        for p in params:
            st = opt.state[p]
            m, v = st["exp_avg"], st["exp_avg_sq"]
            rows.append([
                p.numel(), int(bool(st.get("is_quad_v", False))), int(bool(st.get("is_4bit_m", False))),
                int(bool(st.get("is_8bit", False))), int(st.get("block_size_8bit", 0) or 0),
                m.numel(), _dtype_code(m.dtype), v.numel(), _dtype_code(v.dtype),
                st["exp_avg_scales"].numel() if "exp_avg_scales" in st else 0,
            ])
        return np.array(rows, dtype=np.int64)

    out = {}
    c2 = gpt2_small_shapes()
    out["c2_compact_sr"] = record(c2, torch.bfloat16, dict(lr=1e-3, weight_decay=0.1, adamw_compat=True))
    out["c2_compact_rne"] = record(c2, torch.bfloat16, dict(lr=1e-3, weight_decay=0.1, adamw_compat=True, stochastic_rounding=False))
    out["c2_compact_default"] = record(c2, torch.bfloat16, dict())
    c3 = llama3_8b_shapes()
    out["c3_8bit"] = record(c3, torch.bfloat16, dict(lr=1e-3, weight_decay=0.1, adamw_compat=True, precision="8bit"))
    misc = [(5,), (63,), (64,), (65,), (127,), (128,), (500,), (1024,), (2047,), (2048,), (4096,),
            (16, 100), (32, 64), (33, 40), (8, 2048), (7, 4096), (16384,), (16383,), (16388,), (128, 130)]
    out["misc_8bit"] = record(misc, torch.bfloat16, dict(precision="8bit"))
    out["misc_compact"] = record(misc, torch.bfloat16, dict())
    out["misc_compact_fp32"] = record(misc, torch.float32, dict(adamw_compat=True, stochastic_rounding=False))
    return {"layout": out}


def _dtype_code(dt):
    return {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2, torch.int8: 3, torch.uint8: 4}[dt]


def gpt2_small_shapes():
    s = [(50257, 768), (1024, 768)]
    for _ in range(12):
        s += [(768,), (768,), (768, 2304), (2304,), (768, 768), (768,), (768,), (768,),
              (768, 3072), (3072,), (3072, 768), (768,)]
    return s


def llama3_8b_shapes():
    s = [(128256, 4096)]
    for _ in range(32):
        s += [(4096, 4096), (1024, 4096), (1024, 4096), (4096, 4096), (14336, 4096), (14336, 4096),
              (4096, 14336), (4096,), (4096,)]
    s += [(4096,), (128256, 4096)]
    return s


def golden_muon(muon_mod, hybrid_mod):
    out = {}
    gen = torch.Generator().manual_seed(11)
    for i, shape in enumerate([(64, 128), (96, 48), (32, 32)]):
        G = torch.randn(shape, generator=gen)
        U = muon_mod.zeropower_via_newtonschulz5(G, steps=5, work_dtype=torch.float32, compiled=False)
        out[f"ns_in_{i}"] = _np(G)
        out[f"ns_out_{i}"] = _np(U)
    # Routing of the C5 layer's matrices (and two RMSNorm vectors).
    c5 = [(4096, 4096), (1024, 4096), (1024, 4096), (4096, 4096), (14336, 4096), (14336, 4096), (4096, 14336), (4096,), (4096,)]
    params = [torch.nn.Parameter(torch.empty(s, device="meta")) for s in c5]
    mu, aw = hybrid_mod.partition_parameters_for_hybrid(params)
    out["route_c5"] = np.array([1 if any(p is q for q in mu) else 0 for p in params], dtype=np.int64)
    # Hybrid Muon trajectory on CPU (fp32 work dtype), small shapes: two same-shape matrices,
    # one single matrix, a vector and an embedding-like matrix (AdamW fallback).
    shapes = [(64, 64), (64, 64), (48, 96), (64,), (4096, 32)]
    gen = torch.Generator().manual_seed(12)
    ps = [torch.nn.Parameter(_param(s, torch.float32, gen)) for s in shapes]
    fp = [_fingerprint(p.data) for p in ps]
    from apexw import ApexW
    opt = ApexW(ps, lr=1e-3, weight_decay=0.1, use_muon=True, stochastic_rounding=False)
    for step in range(3):
        for i, p in enumerate(ps):
            g = _grad(p.shape, torch.float32, gen, 1e-3)
            p.grad = g
            fp.append(_fingerprint(g))
        opt.step()
    out["h_fingerprint"] = np.array(fp, dtype=np.int64)
    for i, p in enumerate(ps):
        out[f"hp_{i}"] = _np(p.data)
    out["h_route"] = np.array([1 if any(p is q for q in opt.muon_params) else 0 for p in ps], dtype=np.int64)
    return {"muon": out}


PREC_SHAPES = [(64, 128), (32, 256), (6000,), (256, 72), (768,), (100,), (8, 2048), (3, 5), (36, 64), (16384,),
               (40, 50)]
# threshold 4096: 1-D tensors from 4096 elements count as large (the default is 65536)
PREC_KW = dict(lr=1e-3, weight_decay=0.1, stochastic_rounding=False, threshold=4096)
# name -> (shapes, dtype, steps, seed, kwargs)
PREC_CASES = {
    # fp32 moments: native fused step for fp32 params, foreach lerp path for bf16 params
    "full_fp32_rne": (PREC_SHAPES, torch.float32, 4, 41, dict(PREC_KW, precision="full")),
    "full_bf16_rne": (PREC_SHAPES, torch.bfloat16, 5, 42, dict(PREC_KW, precision="full")),
    # bf16 moments (quad v where eligible) for 2-D / large tensors, fp32 for small 1-D ones
    "auto_bf16_rne": (PREC_SHAPES, torch.bfloat16, 5, 43, dict(PREC_KW, precision="auto")),
    "auto_bf16_fp32v_rne": (PREC_SHAPES, torch.bfloat16, 5, 44, dict(PREC_KW, precision="auto", adamw_compat=True)),
    # INT8 m + dense v for 2-D / large tensors (2048- and 256-element blocks), fp32 m/v otherwise
    "ultra_bf16_rne": (PREC_SHAPES, torch.bfloat16, 4, 45, dict(PREC_KW, precision="ultra")),
    "ultra_bf16_fp32v_rne": (PREC_SHAPES, torch.bfloat16, 4, 46, dict(PREC_KW, precision="ultra", adamw_compat=True)),
    "ultra_fp32_rne": (PREC_SHAPES, torch.float32, 4, 47, dict(PREC_KW, precision="ultra", adamw_compat=True)),
    # nesterov=True: lerp(g, m, beta1) without the SNR gain (chunked NF4, generic NF4 / INT8, the
    # dense tensors under 64 elements, ultra INT8 blocks and fp32 rows)
    "q8_bf16_nesterov_rne": (Q8_SHAPES, torch.bfloat16, 5, 48,
                             dict(PREC_KW, adamw_compat=True, precision="8bit", nesterov=True)),
    "q8_fp32_nesterov_rne": ([(300, 1000), (128, 128), (2048,), (700,), (40,)], torch.float32, 4, 49,
                             dict(PREC_KW, adamw_compat=True, precision="8bit", nesterov=True)),
    "ultra_bf16_nesterov_rne": (PREC_SHAPES, torch.bfloat16, 4, 50, dict(PREC_KW, precision="ultra", nesterov=True)),
    # cautious=True: numerator m times the sign-agreement mask over its mean, every quantized
    # tensor in the generic order (the large NF4 tensors leave the chunked one)
    "q8_bf16_cautious_rne": (Q8_SHAPES, torch.bfloat16, 5, 65,
                             dict(PREC_KW, adamw_compat=True, precision="8bit", cautious=True)),
    "q8_fp32_cautious_rne": ([(300, 1000), (128, 128), (2048,), (700,), (40,)], torch.float32, 4, 66,
                             dict(PREC_KW, adamw_compat=True, precision="8bit", cautious=True)),
    "ultra_bf16_cautious_rne": (PREC_SHAPES, torch.bfloat16, 4, 67, dict(PREC_KW, precision="ultra", cautious=True)),
    # maximize=True: the grads negated (chunked and generic NF4, INT8, dense, ultra)
    "q8_bf16_maximize_rne": (Q8_SHAPES, torch.bfloat16, 4, 68,
                             dict(PREC_KW, adamw_compat=True, precision="8bit", maximize=True)),
    "ultra_bf16_maximize_rne": (PREC_SHAPES, torch.bfloat16, 4, 70, dict(PREC_KW, precision="ultra", maximize=True)),
    # maximize=True in the compact-kernel precisions: the cold step's foreach order and the
    # replayed plan with the grads negated; fp32 moments on fp32 parameters leave the native
    # fused step for the foreach one
    "compact_bf16_maximize_rne": (PREC_SHAPES, torch.bfloat16, 5, 71, dict(PREC_KW, maximize=True)),
    "full_fp32_maximize_rne": (PREC_SHAPES, torch.float32, 4, 72, dict(PREC_KW, precision="full", maximize=True)),
    "auto_bf16_maximize_rne": (PREC_SHAPES, torch.bfloat16, 4, 73,
                               dict(PREC_KW, precision="auto", adamw_compat=True, maximize=True)),
    # nesterov=True in the compact-kernel precisions: two addcdiv passes (m, then g) rounded to
    # the parameter dtype, lerp(g, m, beta1) for quad v, in the cold and the replayed order
    "compact_bf16_nesterov_rne": (PREC_SHAPES, torch.bfloat16, 5, 74, dict(PREC_KW, nesterov=True)),
    "compact_fp32_nesterov_rne": (PREC_SHAPES, torch.float32, 4, 75, dict(PREC_KW, nesterov=True)),
    "full_bf16_nesterov_rne": (PREC_SHAPES, torch.bfloat16, 4, 76, dict(PREC_KW, precision="full", nesterov=True)),
    "full_fp32_nesterov_rne": (PREC_SHAPES, torch.float32, 4, 77, dict(PREC_KW, precision="full", nesterov=True)),
    "auto_bf16_nesterov_rne": (PREC_SHAPES, torch.bfloat16, 4, 78,
                               dict(PREC_KW, precision="auto", adamw_compat=True, nesterov=True)),
    # cautious=True in the compact-kernel precisions: the mask over its mean in the parameter's
    # dtype (non-quad, cold and replayed orders) or in fp32 (quad v)
    "compact_bf16_cautious_rne": (PREC_SHAPES, torch.bfloat16, 5, 79, dict(PREC_KW, cautious=True)),
    "compact_fp32_cautious_rne": (PREC_SHAPES, torch.float32, 4, 80, dict(PREC_KW, cautious=True)),
    "full_bf16_cautious_rne": (PREC_SHAPES, torch.bfloat16, 4, 81, dict(PREC_KW, precision="full", cautious=True)),
    "full_fp32_cautious_rne": (PREC_SHAPES, torch.float32, 4, 82, dict(PREC_KW, precision="full", cautious=True)),
    "auto_bf16_cautious_rne": (PREC_SHAPES, torch.bfloat16, 4, 83,
                               dict(PREC_KW, precision="auto", adamw_compat=True, cautious=True)),
    # amsgrad=True in the compact-kernel precisions: max_exp_avg_sq beside v, no quad v.
    # bf16 compact and fp32 full groups are homogeneous (torch._fused_adamw_ with its max);
    # fused=False, fp32 parameters with bf16 moments and bf16 parameters with fp32 moments
    # take the foreach order, cold then replayed
    "compact_bf16_amsgrad_rne": (PREC_SHAPES, torch.bfloat16, 5, 84, dict(PREC_KW, amsgrad=True)),
    "compact_bf16_amsgrad_foreach_rne": (PREC_SHAPES, torch.bfloat16, 5, 85,
                                         dict(PREC_KW, amsgrad=True, fused=False)),
    "compact_fp32_amsgrad_rne": (PREC_SHAPES, torch.float32, 4, 86, dict(PREC_KW, amsgrad=True)),
    "full_bf16_amsgrad_rne": (PREC_SHAPES, torch.bfloat16, 4, 87, dict(PREC_KW, precision="full", amsgrad=True)),
    "full_fp32_amsgrad_rne": (PREC_SHAPES, torch.float32, 4, 88, dict(PREC_KW, precision="full", amsgrad=True)),
    "auto_bf16_amsgrad_rne": (PREC_SHAPES, torch.bfloat16, 4, 89,
                              dict(PREC_KW, precision="auto", adamw_compat=True, amsgrad=True)),
    "compact_bf16_amsgrad_cautious_rne": (PREC_SHAPES, torch.bfloat16, 4, 90,
                                          dict(PREC_KW, amsgrad=True, cautious=True)),
    # lion=True in the compact-kernel precisions: m only (no v, no quad), the sign update with
    # -lr rounded to a shared 16-bit dtype, m = lerp(m, g, 1 - beta2); cold then replayed.
    # lr 1e-2 moves bf16 parameters of 0.02 by more than half an ulp.  (The reference's step
    # raises IndexError for lion when the first tensor's m is fp32 -- its fused-path test
    # indexes the empty v list, optimizer.py:3684-3687 -- so "full" has no trajectory.)
    "compact_bf16_lion_rne": (PREC_SHAPES, torch.bfloat16, 5, 91, dict(PREC_KW, lion=True, lr=1e-2)),
    "compact_fp32_lion_rne": (PREC_SHAPES, torch.float32, 4, 92, dict(PREC_KW, lion=True)),
    "auto_bf16_lion_rne": (PREC_SHAPES, torch.bfloat16, 4, 95,
                           dict(PREC_KW, precision="auto", adamw_compat=True, lion=True, lr=1e-2)),
    # beta3 (AdEMAMix) in the compact-kernel precisions: a slow first moment beside m (no quad
    # v), the numerator m + slow_ratio m_slow (fp32 for fp32 parameters over bf16 m in the cold
    # order, m's dtype otherwise), one addcdiv; cold then replayed
    "compact_bf16_beta3_rne": (PREC_SHAPES, torch.bfloat16, 5, 96, dict(PREC_KW, beta3=0.9999, alpha=5.0)),
    "compact_fp32_beta3_rne": (PREC_SHAPES, torch.float32, 4, 97, dict(PREC_KW, beta3=0.999, alpha=2.0)),
    "full_bf16_beta3_rne": (PREC_SHAPES, torch.bfloat16, 4, 98, dict(PREC_KW, precision="full", beta3=0.9999)),
    "full_fp32_beta3_rne": (PREC_SHAPES, torch.float32, 4, 99, dict(PREC_KW, precision="full", beta3=0.9999)),
    "auto_bf16_beta3_rne": (PREC_SHAPES, torch.bfloat16, 4, 100,
                            dict(PREC_KW, precision="auto", adamw_compat=True, beta3=0.9999)),
    "compact_bf16_beta3_amsgrad_rne": (PREC_SHAPES, torch.bfloat16, 4, 101,
                                       dict(PREC_KW, beta3=0.999, amsgrad=True, nesterov=True)),
}


FP16_SHAPES = [(64, 512), (32, 256), (16384,), (256, 72), (768,), (100,), (8, 2048), (3, 5), (36, 64), (40, 50)]
FP16_KW = dict(lr=1e-3, weight_decay=0.1, stochastic_rounding=False)
# fp16 parameters: name -> (shapes, steps, seed, kwargs, none_grad)
FP16_CASES = {
    # fp16 m / v (quad v for the large tensors), the dynamic v scale at 1024
    "fp16_compact_quad_rne": (FP16_SHAPES, 6, 51, FP16_KW, ()),
    # beta2 0.999 with SR off: fp32 v under fp16 m
    "fp16_compact_fp32v_rne": (FP16_SHAPES, 6, 52, dict(FP16_KW, adamw_compat=True), ()),
    # every state matches its parameter: torch._fused_adamw_ (no v scale)
    "fp16_native_rne": ([(64, 48), (300,), (1000,)], 5, 53, FP16_KW, ()),
    # 205 steps: the replay recalibrates v at steps 100 and 200; parameter 1 has no grad
    # at step 98 (0-based), so steps 98 and 99 (the 99th and 100th) are cold steps and
    # the cold step's recalibration runs at the 100th
    "fp16_rescale_rne": ([(64, 256), (24, 16), (48,), (16, 32), (8, 8), (96,), (40,), (12, 12)], 205, 54,
                         FP16_KW, ((98, 1),)),
    "fp16_8bit_rne": ([(512, 1024), (256, 256), (4096,), (1000,), (50,), (100, 300)], 4, 55,
                      dict(FP16_KW, adamw_compat=True, precision="8bit"), ()),
    "fp16_full_rne": (FP16_SHAPES, 4, 56, dict(FP16_KW, precision="full"), ()),
    "fp16_ultra_rne": (FP16_SHAPES, 4, 57, dict(FP16_KW, precision="ultra", threshold=4096), ()),
    # amsgrad: fp16 m / v and their max, natively fused (homogeneous; beta2 0.5 keeps the
    # unscaled fp16 v of 1e-3 grads off zero) or in the foreach order with the dynamic v
    # scale (fused=False)
    "fp16_amsgrad_native_rne": (FP16_SHAPES, 4, 58, dict(FP16_KW, amsgrad=True, betas=(0.9, 0.5)), ()),
    "fp16_amsgrad_foreach_rne": (FP16_SHAPES, 5, 59, dict(FP16_KW, amsgrad=True, fused=False), ()),
    # lion: fp16 m, -lr rounded to fp16
    "fp16_lion_rne": (FP16_SHAPES, 4, 60, dict(FP16_KW, lion=True, lr=1e-2), ()),
    # beta3: fp16 m and slow moment, the dynamic v scale
    "fp16_beta3_rne": (FP16_SHAPES, 5, 61, dict(FP16_KW, beta3=0.999), ()),
}


GD_KW = dict(lr=1e-3, weight_decay=0.1, stochastic_rounding=False, threshold=4096)
# grads of another dtype than their parameters (Tensor.grad_dtype):
# name -> (shapes, param dtype, grad dtype, steps, seed, kwargs); the foreach order
# (the native fused step refuses such grads), cold then replayed
GRAD_DTYPE_CASES = {
    "gd_compact_bf16_g32_rne": (PREC_SHAPES, torch.bfloat16, torch.float32, 5, 110, GD_KW),
    # the clip and centralization on bf16 grads (norms and means rounded to bf16; fp32 grads
    # would take the fp32-norm drift of compact_fp32_clip_rne)
    "gd_compact_fp32_g16_clip_gc_rne": (PREC_SHAPES, torch.float32, torch.bfloat16, 4, 111,
                                        dict(GD_KW, clip_grad_norm=1e-3, grad_centralization=True)),
    "gd_compact_fp32_g16_rne": (PREC_SHAPES, torch.float32, torch.bfloat16, 4, 112, GD_KW),
    "gd_full_bf16_g32_rne": (PREC_SHAPES, torch.bfloat16, torch.float32, 4, 113, dict(GD_KW, precision="full")),
    "gd_auto_bf16_g32_rne": (PREC_SHAPES, torch.bfloat16, torch.float32, 4, 114,
                             dict(GD_KW, precision="auto", adamw_compat=True)),
    "gd_compact_bf16_g32_cautious_rne": (PREC_SHAPES, torch.bfloat16, torch.float32, 4, 115,
                                         dict(GD_KW, cautious=True)),
    "gd_compact_fp32_g16_cautious_rne": (PREC_SHAPES, torch.float32, torch.bfloat16, 4, 116,
                                         dict(GD_KW, cautious=True)),
    "gd_compact_fp16_g32_rne": (FP16_SHAPES, torch.float16, torch.float32, 5, 117, dict(GD_KW, threshold=65536)),
}


def golden_grad_dtypes(ApexW):
    """Parameters stepped with grads of another dtype."""
    return {name: run_trajectory(ApexW, shapes, dt, steps, seed, kw, record_all=True, grad_dtype=gd)
            for name, (shapes, dt, gd, steps, seed, kw) in GRAD_DTYPE_CASES.items()}


def golden_fp16(ApexW):
    """fp16 parameters in every precision mode the product steps them in."""
    return {name: run_trajectory(ApexW, shapes, torch.float16, steps, seed, kw, record_all=True, none_grad=ng)
            for name, (shapes, steps, seed, kw, ng) in FP16_CASES.items()}


def golden_precisions(ApexW):
    """The other precision modes' layouts and steps (full, auto, ultra), several
    steps each so that the replayed plan is covered as well as the cold step."""
    return {name: run_trajectory(ApexW, shapes, dtype, steps, seed, kw, record_all=True)
            for name, (shapes, dtype, steps, seed, kw) in PREC_CASES.items()}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--ref", default="/root/reference")
    ap.add_argument("--only", nargs="*", help="write only these fixture names")
    args = ap.parse_args()
    sys.path.insert(0, args.ref)
    import apexw
    from apexw import ApexW
    import apexw.optimizer as opt_mod
    import apexw.muon as muon_mod
    import apexw.hybrid as hybrid_mod
    torch.manual_seed(0)
    allc = {}
    allc.update(golden_compact(ApexW))
    allc.update(golden_8bit(ApexW))
    allc.update(golden_clip(opt_mod))
    allc.update(golden_layout(ApexW))
    allc.update(golden_muon(muon_mod, hybrid_mod))
    allc.update(golden_factored(ApexW))
    allc.update(golden_hooks(ApexW))
    allc.update(golden_fused(ApexW))
    allc.update(golden_state_dict(ApexW))
    allc.update(golden_precisions(ApexW))
    allc.update(golden_fp16(ApexW))
    allc.update(golden_grad_dtypes(ApexW))
    for name, arrays in allc.items():
        if args.only and name not in args.only:
            continue
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **arrays)
        print(f"wrote {path} ({os.path.getsize(path) / 1024:.1f} KiB)")


if __name__ == "__main__":
    main()
