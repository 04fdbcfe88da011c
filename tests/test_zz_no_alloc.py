"""The allocation-free clip coefficient (apexw_grad_clip_coef_noalloc) against
apexw_grad_clip_coef, through the C ABI.

Both run the same three kernels in the same order with no atomics, so the
coefficient must agree bit for bit.  Two calls in a row, the second over fewer
tensors and units, check that the shared device array is fully rewritten by
each call.  The per-tensor norms (rounded to bf16, like torch._foreach_norm's)
are held to one bf16 ulp of a float64 norm, and the coefficient to 1e-6 of the
one computed from them in float64.  Sizes beyond the array's limits are refused
on the host before anything is enqueued.
"""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")


def _tables(shapes, seed, dtype=torch.bfloat16, unit=None):
    """Device tensor and unit tables (2048-element units unless `unit`) of one grad per shape."""
    from apexw_amd import _lib as L
    gen = torch.Generator().manual_seed(seed)
    grads = [(torch.randn(s, generator=gen) * (1e-3 * (1 + i % 7))).to(dtype).cuda() for i, s in enumerate(shapes)]
    code = L.BF16 if dtype == torch.bfloat16 else L.F32
    unit = unit or L.COMPACT_UNIT
    tab = np.zeros(len(grads), dtype=L.TENSOR_DTYPE)
    counts = np.array([(g.numel() + unit - 1) // unit for g in grads], dtype=np.int64)
    for i, g in enumerate(grads):
        # the clip reads only g; p/m/v point at the grad so the descriptor is well formed
        tab[i]["p"] = tab[i]["g"] = tab[i]["m"] = tab[i]["v"] = g.data_ptr()
        tab[i]["n"] = g.numel()
        tab[i]["flags"] = (code << L.PDT_SHIFT) | (code << L.GDT_SHIFT)
    begin = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    units = np.zeros(int(begin[-1]), dtype=L.UNIT_DTYPE)
    units["tensor"] = np.repeat(np.arange(len(grads), dtype=np.uint32), counts)
    units["unit"] = (np.arange(len(units)) - np.repeat(begin[:-1], counts)).astype(np.uint32)
    dev = lambda a: torch.from_numpy(a.view(np.uint8).copy()).cuda()  # noqa: E731
    return grads, dev(tab), dev(units), torch.from_numpy(begin).cuda(), len(units)


def _coef_pair(shapes, seed, clip=1.0, unit=None):
    from apexw_amd import _lib as L
    lib = L.load()
    unit = unit or L.COMPACT_UNIT
    grads, tab, units, begin, n_units = _tables(shapes, seed, unit=unit)
    stream = torch.cuda.current_stream().cuda_stream
    part = torch.empty(max(n_units, 1), dtype=torch.float32, device="cuda")
    norms = torch.empty(len(grads), dtype=torch.float32, device="cuda")
    coef_a = torch.full((1,), -1.0, device="cuda")
    coef_b = torch.full((1,), -2.0, device="cuda")
    L.check(lib.apexw_grad_clip_coef(tab.data_ptr(), len(grads), units.data_ptr(), n_units, unit,
                                     begin.data_ptr(), part.data_ptr(), norms.data_ptr(), clip, 1.0, L.HP_SANITIZE,
                                     coef_a.data_ptr(), None, None, stream), "apexw_grad_clip_coef")
    L.check(lib.apexw_grad_clip_coef_noalloc(tab.data_ptr(), len(grads), units.data_ptr(), n_units, unit,
                                             begin.data_ptr(), clip, 1.0, L.HP_SANITIZE, coef_b.data_ptr(), None, stream),
            "apexw_grad_clip_coef_noalloc")
    torch.cuda.synchronize()
    # each tensor norm is rounded to the grad dtype (torch._foreach_norm): within one
    # bf16 ulp of the float64 norm; the coefficient follows from those norms
    n64 = torch.tensor([float(g.double().norm()) for g in grads], dtype=torch.float64)
    got = norms.cpu().double()
    assert ((got - n64).abs() <= 2.0 ** -8 * n64).all(), "per-tensor norms"
    total = float(got.square().sum().sqrt())
    return float(coef_a.item()), float(coef_b.item()), min(clip / (total + 1e-6), 1.0)


def test_noalloc_clip_matches_workspace_entry_point_twice():
    _need_gpu()
    print("noalloc clip: 300 ragged tensors, then 17 smaller ones", flush=True)
    gen = np.random.default_rng(3)
    big = [(int(n),) if i % 2 else (8, int(n) // 8 * 1) for i, n in
           enumerate(np.exp(gen.uniform(np.log(64), np.log(1 << 18), 300)).astype(np.int64) // 8 * 8 + 8)]
    small = [(int(n),) for n in gen.integers(1, 5000, 17)]
    # clips below each set's grad norm, so both coefficients are < 1
    for shapes, seed, clip in ((big, 1, 1.0), (small, 2, 0.05)):
        a, b, ref = _coef_pair(shapes, seed, clip)
        assert a == b, f"noalloc {b!r} != workspace {a!r}"
        assert 0.0 < b < 1.0
        assert abs(b - ref) <= 1e-6 * ref, (b, ref)


def test_noalloc_clip_covers_an_8b_unit_count():
    """More units than an 8B-parameter list has in 2048-element units (3.92 M at
    Llama-3-8B), well above 2^21: here as 64-element units of a 256 M-element list,
    then a smaller list in the same array."""
    _need_gpu()
    print("noalloc clip: 4,000,000 units of 64 elements, then 2^21 + 5", flush=True)
    cases = (([((4_000_000 - 1000) * 64,), (1000 * 64,)], 11), ([(((1 << 21) + 5) * 64,)], 12))
    for shapes, seed in cases:
        a, b, ref = _coef_pair(shapes, seed, clip=1.0, unit=64)
        assert a == b, f"noalloc {b!r} != workspace {a!r}"
        assert 0.0 < b < 1.0
        assert abs(b - ref) <= 1e-6 * ref, (b, ref)


def test_noalloc_clip_uses_the_streams_device_array():
    """A non-default stream of the current device: the stream's device array is used and
    the result equals the workspace entry point's."""
    _need_gpu()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        a, b, ref = _coef_pair([(5000,), (64, 300)], 13, clip=0.01)
    torch.cuda.synchronize()
    assert a == b and abs(b - ref) <= 1e-6 * ref


def test_noalloc_clip_unclipped_is_one():
    """A clip above the norm gives exactly 1 (no clipping), like the workspace entry point."""
    _need_gpu()
    a, b, _ = _coef_pair([(4096,), (33,)], 5, clip=1e6)
    assert a == b == 1.0


def test_noalloc_clip_refuses_oversized_work():
    _need_gpu()
    from apexw_amd import _lib as L
    lib = L.load()
    _, tab, units, begin, n_units = _tables([(4096,)], 7)
    coef = torch.zeros(1, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    st = lib.apexw_grad_clip_coef_noalloc(tab.data_ptr(), 1, units.data_ptr(), L.NOALLOC_CLIP_MAX_UNITS + 1,
                                          L.COMPACT_UNIT, begin.data_ptr(), 1.0, 1.0, 0, coef.data_ptr(), None, stream)
    assert st == L.ERR_SIZE
    st = lib.apexw_grad_clip_coef_noalloc(tab.data_ptr(), L.NOALLOC_CLIP_MAX_TENSORS + 1, units.data_ptr(), n_units,
                                          L.COMPACT_UNIT, begin.data_ptr(), 1.0, 1.0, 0, coef.data_ptr(), None, stream)
    assert st == L.ERR_SIZE
    torch.cuda.synchronize()
    assert float(coef.item()) == 0.0     # nothing was enqueued
