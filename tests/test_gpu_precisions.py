"""The full / auto / ultra precisions on the GPU against the CPU oracle.

The reference-written trajectories (full_*, auto_*, ultra_* under
tests/golden/) are replayed by test_gpu_parity.py; these tests take the same
paths at larger and more ragged sizes -- multi-block ultra tensors with a
partial last block, 256-element ultra blocks, dense fp32 units of 2048
elements, fp32 moments under bf16 parameters in one launch with bf16 moments
-- through the config-test mirror (every tensor re-synced from the GPU before
each step, stepped by ``OracleApexW``, compared at the bars stated in
test_gpu_configs.py).

With stochastic rounding on (from the second step), the bf16 parameter stores
of full / auto, auto's bf16 v, and ultra's INT8 m codes must lie in the bracket
of the oracle's exact pre-rounding values and be unbiased (|z| < 3).
"""

import pytest
import torch

from test_gpu_configs import KW, _drive, _need_gpu, _say

pytestmark = pytest.mark.gpu

SHAPES = [(1000, 1001), (4096,), (5000,), (70000,), (300,), (63,), (16, 100), (3, 5), (256, 768), (131072,),
          (40, 50), (1, 4096), (2047,)]
CASES = [("full", torch.bfloat16), ("full", torch.float32), ("auto", torch.bfloat16), ("auto", torch.float32),
         ("ultra", torch.bfloat16), ("ultra", torch.float32)]


@pytest.mark.parametrize("prec,dtype", CASES, ids=[f"{p}-{str(d)[6:]}" for p, d in CASES])
def test_precision_matches_oracle_rne(prec, dtype):
    """Three steps (the cold step and two replays), every tensor checked, SR off."""
    _need_gpu()
    _say(f"{prec} {dtype} rne")
    _drive(f"{prec}-{dtype}", SHAPES, dtype, dict(KW, precision=prec, threshold=4096),
           [(i, None) for i in range(len(SHAPES))], 3, False, seed=300 + CASES.index((prec, dtype)))


@pytest.mark.parametrize("prec,dtype,stat", [("full", torch.bfloat16, "bf16"), ("auto", torch.bfloat16, "bf16"),
                                             ("ultra", torch.bfloat16, "int8"), ("ultra", torch.float32, "int8")])
def test_precision_sr_is_unbiased(prec, dtype, stat):
    """Stochastic rounding from the second step on, from the state the first left."""
    _need_gpu()
    _say(f"{prec} {dtype} sr")
    kw = dict(KW, precision=prec, threshold=4096)
    if prec == "auto":
        kw["adamw_compat"] = False     # betas (0.9, 0.99) with SR: bf16 v
    stats = _drive(f"{prec}-{dtype}-sr", SHAPES, dtype, kw, [(i, None) for i in range(len(SHAPES))], 3, True,
                   seed=400 + CASES.index((prec, dtype)), sr_from=1)
    s = stats[stat]
    assert s.n >= 1_000_000 and abs(s.z) < 3 and abs(s.z_mag) < 3, stats


FP16_CASES = [("compact", dict()), ("compact", dict(adamw_compat=True)), ("full", dict()), ("auto", dict()),
              ("ultra", dict()), ("8bit", dict())]


@pytest.mark.parametrize("prec,extra", FP16_CASES, ids=[f"{p}-{i}" for i, (p, _) in enumerate(FP16_CASES)])
def test_fp16_parameters_match_oracle_rne(prec, extra):
    """fp16 parameters in every precision, three steps, SR off: fp16 m / v with the
    dynamic v scale (compact, auto), fp32 v (beta2 0.999), fp32 moments (full), INT8
    blocks (ultra), NF4 / INT8 codes (8-bit, on the general kernel)."""
    _need_gpu()
    _say(f"fp16 {prec} {extra}")
    kw = dict(KW, precision=prec, threshold=4096)
    kw.update(extra)
    if prec != "compact" or "adamw_compat" not in extra:
        kw["adamw_compat"] = False
    _drive(f"fp16-{prec}", SHAPES, torch.float16, kw, [(i, None) for i in range(len(SHAPES))], 3, False,
           seed=500 + FP16_CASES.index((prec, extra)))
