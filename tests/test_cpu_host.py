"""CPU-side checks: the C-ABI library, the host layout rules and the constructor contract."""

import ctypes
import os
import re

import numpy as np
import pytest
import torch

from golden_replay import load

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_symbols():
    src = open(os.path.join(ROOT, "include", "apexw_hip.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:int|int32_t|int64_t)\s+(apexw_\w+)\s*\(", src, flags=re.M)))


def test_library_exports_every_declared_symbol():
    from apexw_amd import _lib
    lib = _lib.load()
    syms = _declared_symbols()
    assert syms, "no declarations parsed"
    for s in syms:
        assert hasattr(lib, s), s
        assert s in _lib.SIGNATURES, f"{s} has no ctypes signature"
    assert lib.apexw_abi_version() == _lib.ABI_VERSION


def test_struct_layouts_match_header():
    from apexw_amd import _lib
    assert ctypes.sizeof(_lib.Tensor) == 64 == _lib.TENSOR_DTYPE.itemsize
    assert ctypes.sizeof(_lib.HParams) == 144
    assert _lib.GEMM_PROBLEM_DTYPE.itemsize == 120
    assert ctypes.sizeof(_lib.StateLayout) == 56


def test_state_conversion_rejects_bad_layouts():
    """apexw_state_decode / _encode validate the layout before anything is enqueued
    (stand-in pointers: a rejected call never dereferences them; skipped where a GPU
    is present, so that a case the checks let through could not launch on them)."""
    if torch.cuda.is_available():
        pytest.skip("stand-in device pointers: run where no GPU is present")
    from apexw_amd import _lib as L
    lib = L.load()
    A = 1 << 20
    lay = L.StateLayout(A, A, A, A, 1002, L.STATE_Q8, L.FLAG_QUAD, 2048, 0)
    assert lib.apexw_state_encode(ctypes.byref(lay), A, A, None) == 1  # quad, n % 4
    lay.n, lay.flags, lay.block = 1000, 0, 4096
    assert lib.apexw_state_encode(ctypes.byref(lay), A, A, None) == 1      # block > 2048
    lay.block, lay.flags = 1004, L.FLAG_NF4
    assert lib.apexw_state_encode(ctypes.byref(lay), A, A, None) == 1      # NF4 block not a multiple of 8
    lay.block, lay.flags, lay.m_scale = 1024, 0, None
    assert lib.apexw_state_decode(ctypes.byref(lay), A, A, None) == 1      # 8-bit without scales
    lay = L.StateLayout(A, A, None, None, 1000, L.STATE_DENSE, 3 << L.MDT_SHIFT, 0, 0)
    assert lib.apexw_state_decode(ctypes.byref(lay), A, A, None) == 2      # m dtype code 3 (u8) is not dense
    lay.flags, lay.kind = 0, 7
    assert lib.apexw_state_decode(ctypes.byref(lay), A, A, None) == 1      # unknown kind
    lay.kind, lay.reserved = L.STATE_DENSE, 1
    assert lib.apexw_state_decode(ctypes.byref(lay), A, A, None) == 1      # reserved must be 0


def test_check_tensor_rejects_bad_descriptors():
    from apexw_amd import _lib
    lib = _lib.load()
    t = _lib.Tensor(16, 32, 48, 64, 0, 0, 100, (_lib.BF16 << 0) | (_lib.BF16 << 2) | (_lib.BF16 << 4) | (_lib.BF16 << 6), 0)
    assert lib.apexw_check_tensor(ctypes.byref(t), 0) == 0
    t.p = 0
    assert lib.apexw_check_tensor(ctypes.byref(t), 0) == 1
    t.p = 18  # misaligned without the scalar flag
    assert lib.apexw_check_tensor(ctypes.byref(t), 0) == 4
    t.flags |= _lib.FLAG_SCALAR
    assert lib.apexw_check_tensor(ctypes.byref(t), 0) == 0
    t.flags = (_lib.F16 << 0) | (_lib.F16 << 2) | (_lib.BF16 << 4) | (_lib.BF16 << 6)   # fp16 p keeps fp16 m
    assert lib.apexw_check_tensor(ctypes.byref(t), 0) == 2
    # p and g dtypes differ (torch's Tensor.grad_dtype): the compact step takes it, the
    # per-parameter update does not
    t.flags = (_lib.F16 << 0) | (_lib.BF16 << 2) | _lib.FLAG_SCALAR
    assert lib.apexw_check_tensor(ctypes.byref(t), 0) == 0
    assert lib.apexw_check_tensor(ctypes.byref(t), 3) == 2
    q = _lib.Tensor(16, 32, 48, 64, 80, 96, 4096, (_lib.BF16 << 0) | (_lib.BF16 << 2) | _lib.FLAG_NF4 | _lib.FLAG_QUAD,
                    2048)
    assert lib.apexw_check_tensor(ctypes.byref(q), 1) == 0
    q.block = 4096  # blocks above 2048 elements are not supported
    assert lib.apexw_check_tensor(ctypes.byref(q), 1) == 2
    # entry points reject null tables before touching the GPU
    hp = _lib.HParams()
    assert lib.apexw_compact_step(None, 1, None, 1, ctypes.byref(hp), None) == 1
    assert lib.apexw_q8_step(None, 1, None, 1, 0, 0, ctypes.byref(hp), None) == 1
    units = ctypes.c_uint64(0)
    assert lib.apexw_q8_step(ctypes.byref(q), 1, ctypes.byref(units), 1, 1, 1, ctypes.byref(hp), None) == 1
    q.block = 2048
    assert lib.apexw_check_tensor(ctypes.byref(q), 2) == 0
    q.flags = (_lib.F32 << 0) | (_lib.F32 << 2) | _lib.FLAG_NF4 | _lib.FLAG_QUAD   # fp32 params: full-block kernel too
    assert lib.apexw_check_tensor(ctypes.byref(q), 2) == 0
    q.flags = (_lib.F32 << 0) | (_lib.BF16 << 2) | _lib.FLAG_NF4 | _lib.FLAG_QUAD  # mixed p / g dtypes: no
    assert lib.apexw_check_tensor(ctypes.byref(q), 2) == 2
    q.flags = (_lib.BF16 << 0) | (_lib.BF16 << 2)
    assert lib.apexw_check_tensor(ctypes.byref(q), 2) == 2


_CODES = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2, torch.int8: 3, torch.uint8: 4}


def _layout_rows(shapes, dtype, kwargs):
    from apexw_amd import state as S
    from apexw_amd.optimizer import ApexW
    params = [torch.nn.Parameter(torch.empty(s, dtype=dtype, device="meta")) for s in shapes]
    opt = ApexW(params, **kwargs)
    g = opt.param_groups[0]
    peft = S.detect_peft_context(opt.param_groups)
    rows = []
    for p in params:
        st = S.init_state(p, g, peft)
        m, v = st["exp_avg"], st["exp_avg_sq"]
        rows.append([p.numel(), int(bool(st.get("is_quad_v", False))), int(bool(st.get("is_4bit_m", False))),
                     int(bool(st.get("is_8bit", False))), int(st.get("block_size_8bit", 0) or 0),
                     m.numel(), _CODES[m.dtype], v.numel(), _CODES[v.dtype],
                     st["exp_avg_scales"].numel() if "exp_avg_scales" in st else 0])
    return np.array(rows, dtype=np.int64)


def test_state_layout_matches_reference():
    import bench
    from golden.make_golden import gpt2_small_shapes, llama3_8b_shapes
    z = load("layout")
    misc = [(5,), (63,), (64,), (65,), (127,), (128,), (500,), (1024,), (2047,), (2048,), (4096,),
            (16, 100), (32, 64), (33, 40), (8, 2048), (7, 4096), (16384,), (16383,), (16388,), (128, 130)]
    cases = {
        "c2_compact_sr": (gpt2_small_shapes(), torch.bfloat16, dict(lr=1e-3, weight_decay=0.1, adamw_compat=True)),
        "c2_compact_rne": (gpt2_small_shapes(), torch.bfloat16,
                           dict(lr=1e-3, weight_decay=0.1, adamw_compat=True, stochastic_rounding=False)),
        "c2_compact_default": (gpt2_small_shapes(), torch.bfloat16, dict()),
        "c3_8bit": (llama3_8b_shapes(), torch.bfloat16,
                    dict(lr=1e-3, weight_decay=0.1, adamw_compat=True, precision="8bit")),
        "misc_8bit": (misc, torch.bfloat16, dict(precision="8bit")),
        "misc_compact": (misc, torch.bfloat16, dict()),
        "misc_compact_fp32": (misc, torch.float32, dict(adamw_compat=True, stochastic_rounding=False)),
    }
    assert bench.llama3_8b_shapes() == llama3_8b_shapes()
    for name, (shapes, dt, kw) in cases.items():
        np.testing.assert_array_equal(_layout_rows(shapes, dt, kw), z[name], err_msg=name)


def test_constructor_contract():
    from apexw_amd import ApexW
    p = [torch.nn.Parameter(torch.zeros(4))]
    o = ApexW(p)
    assert o.defaults["betas"] == (0.9, 0.99) and o.defaults["precision"] == "compact"
    assert o.defaults["decay_norm_only"] is True
    o = ApexW(p, precision="int8")
    assert o.defaults["betas"] == (0.9, 0.999) and o.defaults["precision"] == "8bit"
    o = ApexW(p, adamw_compat=True, betas=(0.9, 0.95))
    assert o.defaults["betas"] == (0.9, 0.999) and o.defaults["decay_norm_only"] is False
    o = ApexW(p, adamw_compat=True, betas=(0.8, 0.9))
    assert o.defaults["betas"] == (0.8, 0.9)
    with pytest.raises(ValueError):
        ApexW(p, lr=-1.0)
    with pytest.raises(ValueError):
        ApexW(p, betas=(1.0, 0.9))
    with pytest.raises(ValueError):
        ApexW(p, block_size=0)
    with pytest.raises(ValueError):
        ApexW(p, precision="nope")
    # amsgrad, lion and beta3: the compact, full and auto precisions, not 8bit / ultra;
    # factored_v=True is accepted and lays out no factored state under them, as in the reference
    for opt, val in (("amsgrad", True), ("lion", True), ("beta3", 0.999)):
        for prec in ("compact", "full", "auto"):
            assert ApexW(p, precision=prec, **{opt: val}).defaults[opt] == val
        assert ApexW(p, precision="compact", factored_v=True, **{opt: val}).defaults["factored_v"]
        for prec in ("8bit", "ultra"):
            with pytest.raises(NotImplementedError):
                ApexW(p, precision=prec, **{opt: val})
    assert ApexW(p, betas=(0.9, 0.999, 0.9999)).defaults["beta3"] == 0.9999
    with pytest.raises(NotImplementedError):
        ApexW(p, beta3=0.999, cautious=True)
    # nesterov: every precision, without factored second moments
    for prec in ("8bit", "ultra", "3byte", "compact", "full", "auto"):
        assert ApexW(p, precision=prec, nesterov=True).defaults["nesterov"]
    for prec in ("8bit", "compact"):
        with pytest.raises(NotImplementedError):
            ApexW(p, precision=prec, nesterov=True, factored_v=True)
    # cautious: every precision, not with factored second moments nor with nesterov
    for prec in ("8bit", "ultra", "compact", "full", "auto"):
        assert ApexW(p, precision=prec, cautious=True).defaults["cautious"]
    for kw in (dict(precision="8bit", factored_v=True), dict(precision="compact", factored_v=True),
               dict(precision="8bit", nesterov=True), dict(precision="compact", nesterov=True)):
        with pytest.raises(NotImplementedError):
            ApexW(p, cautious=True, **kw)
    # maximize: every precision, factored second moments included
    for prec in ("8bit", "ultra", "compact", "full", "auto"):
        assert ApexW(p, precision=prec, maximize=True).defaults["maximize"]
    for kw in (dict(precision="8bit", factored_v=True), dict(precision="compact", factored_v=True)):
        assert ApexW(p, maximize=True, **kw).defaults["maximize"]
    for prec, betas in (("full", (0.9, 0.999)), ("fp32", (0.9, 0.999)), ("auto", (0.9, 0.99)),
                        ("smart", (0.9, 0.99)), ("ultra", (0.9, 0.99)), ("3byte", (0.9, 0.99))):
        o = ApexW(p, precision=prec)
        assert o.defaults["betas"] == betas, prec
    assert ApexW._step_supports_amp_scaling


def test_step_requires_gpu_tensors():
    from apexw_amd import ApexW
    p = torch.nn.Parameter(torch.zeros(8))
    p.grad = torch.zeros(8)
    with pytest.raises(RuntimeError):
        ApexW([p]).step()


def test_step_hooks_match_torch_semantics():
    """The step wrapper keeps torch.optim's hook contract: global and
    per-optimizer pre hooks (which may replace args), then post hooks, in
    order; torch does not wrap the method a second time."""
    from torch.optim.optimizer import register_optimizer_step_pre_hook
    from apexw_amd import ApexW
    from apexw_amd.hybrid import HybridApexW
    from apexw_amd.muon import ApexMuon
    for cls in (ApexW, ApexMuon, HybridApexW):
        assert getattr(cls.step, "hooked", False)
    p = torch.nn.Parameter(torch.zeros(4))
    opt = ApexW([p], lr=1e-3)
    assert getattr(type(opt).step, "hooked", False) and type(opt).step is ApexW.step
    calls = []
    g = register_optimizer_step_pre_hook(lambda o, a, k: calls.append(("global pre", len(a))))
    h1 = opt.register_step_pre_hook(lambda o, a, k: calls.append(("pre", len(a))))
    h2 = opt.register_step_post_hook(lambda o, a, k: calls.append(("post", len(a))))
    try:
        opt.step()                                   # no grads: nothing to step, hooks still run
    finally:
        g.remove(), h1.remove(), h2.remove()
    assert calls == [("global pre", 1), ("pre", 1), ("post", 1)]
    bad = opt.register_step_pre_hook(lambda o, a, k: 3)
    with pytest.raises(RuntimeError):
        opt.step()
    bad.remove()


def test_bench_contract():
    """bench.py: one GPU only (exit 2 with a message for --gpus N > 1, before any
    device work); C3 is the default workload; every config names its workload and
    the in-backward configs are 8-bit (the precision whose hooks they measure)."""
    import subprocess
    import sys
    import bench
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr and r.stdout == ""
    assert bench.CONFIGS["c3"]["workload"].startswith("C3 8-bit")
    for name, cfg in bench.CONFIGS.items():
        assert cfg["workload"] and cfg["shapes"], name
        if cfg.get("backward"):
            assert cfg["kwargs"]["precision"] == "8bit" and cfg["backward"] in ("hooks", "plain"), name


def test_state_map_pickles_as_plain_defaultdict():
    """optimizer.state folds device-counted AMP skips on lookup; copies and
    pickles of an optimizer hold torch's plain defaultdict(dict) and come back
    as the folding map bound to the new optimizer."""
    import copy
    import pickle
    from collections import defaultdict
    from apexw_amd import ApexW
    p = torch.nn.Parameter(torch.zeros(4))
    opt = ApexW([p], lr=1e-3)
    opt.state[p]["k"] = 1
    assert type(pickle.loads(pickle.dumps(opt.state))) is defaultdict
    twin = copy.deepcopy(opt)
    assert twin.state._owner is twin and list(twin.state.values()) == [{"k": 1}]
    other = ApexW([torch.nn.Parameter(torch.zeros(4))], lr=1e-3)
    other.load_state_dict(opt.state_dict())
    assert other.state._owner is other
    # ApexMuon keeps the same mapping; a copy folds the pending skips first
    from apexw_amd.muon import ApexMuon
    q = torch.nn.Parameter(torch.zeros(32, 32))
    mu = ApexMuon([q], lr=0.02)
    mu.state[q]["step"] = 3
    folds = []
    mu._fold_amp_skips = lambda: (folds.append(1), setattr(mu, "_amp_unfolded", False))
    mu._amp_unfolded = True
    twin = copy.deepcopy(mu)
    assert folds == [1] and twin.state._owner is twin and [st["step"] for st in twin.state.values()] == [3]
    assert type(pickle.loads(pickle.dumps(mu.state))) is defaultdict


@pytest.mark.parametrize("prec", ["full", "auto", "ultra", "compact", "8bit"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
@pytest.mark.parametrize("kw", [dict(), dict(adamw_compat=True, stochastic_rounding=False),
                                dict(threshold=4096, force_compact_v=True), dict(fused=True)])
def test_other_precision_layouts_match_oracle(prec, dtype, kw):
    """The product's state layout for every precision and parameter dtype equals the
    oracle's (pinned bit for bit by the reference-written trajectories, fp16_* for
    fp16 parameters): the same keys, flags, dtypes, shapes, initial values and v scales."""
    from apexw_amd import state as S
    from apexw_amd.optimizer import ApexW
    from oracle import layout as OL
    shapes = [(5,), (63,), (100,), (2047,), (2048,), (4096,), (5000,), (16384,), (70000,), (3, 5), (16, 100),
              (8, 2048), (7, 4096), (256, 256), (40, 50)]
    params = [torch.nn.Parameter(torch.zeros(s, dtype=dtype)) for s in shapes]
    opt = ApexW(params, precision=prec, **kw)
    g = opt.param_groups[0]
    ogroup = dict(g, stochastic_rounding=g["stochastic_rounding"], params=params)
    for p in params:
        a = S.init_state(p, g, False, dtype != torch.float32)
        b = OL.init_state(p, ogroup, len(params), False, has_16bit_params=dtype != torch.float32, cuda=True)
        assert sorted(a) == sorted(b), (p.shape, sorted(a), sorted(b))
        for k in a:
            if torch.is_tensor(a[k]):
                assert a[k].dtype == b[k].dtype and a[k].shape == b[k].shape, (k, p.shape)
                assert torch.equal(a[k], b[k]), (k, p.shape)
            else:
                assert a[k] == b[k], (k, p.shape, a[k], b[k])


def test_integration_binding_loads():
    """The binding module of INTEGRATION.md compiles, loads the library, agrees
    with its ABI version and binds both of the reference's entry points."""
    from integration_binding import load_binding
    rx = load_binding()
    assert callable(rx.step_fused) and callable(rx.step_fused_8bit)
    assert ctypes.sizeof(rx.HParams) == 144 and ctypes.sizeof(rx.Tensor) == 64 and ctypes.sizeof(rx.Unit) == 8
    p = torch.zeros(4)          # CPU tensors: not handled, nothing written
    assert rx.step_fused([p], [p], [p], [p], 1e-3, 0.9, 0.999, 1e-8, 0.0) is False
