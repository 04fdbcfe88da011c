"""BASELINE's five configurations at their own workloads on the GPU, against the CPU oracle.

Each test builds the configuration's full parameter list on the GPU (synthetic
data of the stated shapes) and steps it with ``ApexW``.  A checked subset is
mirrored on the CPU: before every GPU step its parameters and state are
copied out, the oracle (``OracleApexW``, the reference's CPU algorithm)
steps the copies with the same grads, and the results are compared.  Every
element and every quantization block of the fused step is independent of the
other tensors (the clip coefficient aside, which C4 checks on its own), so a
subset stepped alone must give what the full launch gave.

Bars (round to nearest, stochastic rounding off):
  * params: one bf16 ulp, or 1e-6 |ref| + 1e-9 (fp32), plus 2^-22 of the
    update |p_after - p_before| (2^-7 where the reference rounds the
    denominator or the update itself to bf16): the update's last fp32 bits
    differ from torch's CPU kernels (SLEEF's square root is not correctly
    rounded), which matters only where the subtraction cancels to a result far
    smaller than the update, or where a bf16 rounding of the update flips;
  * fp32 v: 1e-6 |ref| + 1e-12; bf16 moments: <= 1 bf16 ulp;
  * 8-bit codes (NF4 / INT8 / log-uint8): <= 1 code; block scales 1e-6 relative.
With stochastic rounding on, every SR result must lie in the bracket of the
oracle's exact pre-rounding value and the rounding must be unbiased over the
checked elements (|z| < 3, signed and by magnitude; ``sr_inject``); the
deterministic parts are held to the bars above.  Hyperparameters: C1's
(lr 1e-3, weight decay 0.1, adamw_compat=True) for every configuration, as
BASELINE.json states them for C1 only.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn as nn

from bench import gpt2_small_shapes, llama3_8b_shapes, ragged_shapes
from golden_replay import bf16_ulp_diff
from oracle import layout as OL
from oracle.optim import OracleApexW
from sr_inject import SRCheck

pytestmark = pytest.mark.gpu
KW = dict(lr=1e-3, weight_decay=0.1, adamw_compat=True)


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")


def _say(msg):
    print(msg, flush=True)


# ---------------------------------------------------------------------- comparisons
def _bf16_ulp(x):
    """Spacing of bf16 values at |x| (fp32 input; the smallest normal spacing at 0)."""
    e = torch.floor(torch.log2(x.abs().clamp_min(2.0 ** -126)))
    return torch.exp2(e - 7)


def _f16_ulp(x):
    """Spacing of fp16 values at |x| (fp32 input; the subnormal spacing 2^-24 below 2^-14)."""
    e = torch.floor(torch.log2(x.abs().clamp_min(2.0 ** -14)))
    return torch.exp2(e - 10)


def _cmp_p(got, ref, prev, what, den_rel):
    """A parameter: one bf16 ulp, or 1e-6 relative (fp32) -- plus den_rel of the
    update |ref - prev|.  The update's last fp32 bits differ between the GPU and
    torch's CPU kernels (torch's SLEEF square root is not correctly rounded), and
    where p_before - update cancels to a tiny result those bits are many ulps of
    it; den_rel = 2^-22 (a few fp32 ulps of the update) when the denominator is
    fp32, 2^-7 (one bf16 ulp of it) when it is rounded to bf16."""
    got = got.detach().cpu().reshape(-1).double()
    ref64, prev64 = ref.detach().reshape(-1).double(), prev.detach().reshape(-1).double()
    upd = den_rel * (ref64 - prev64).abs()
    if ref.dtype in (torch.bfloat16, torch.float16):
        f = _bf16_ulp if ref.dtype == torch.bfloat16 else _f16_ulp
        ulp = torch.maximum(f(ref64.float()), f(got.float())).double()
        err = (got - ref64).abs() - (ulp + upd)
        both_nan = torch.isnan(got) & torch.isnan(ref64)
        err = torch.where(both_nan, torch.full_like(err, -1.0), err)
    else:
        err = (got - ref64).abs() - (1e-6 * ref64.abs() + 1e-9 + upd)
    bad = err > 0
    assert not bool(bad.any()), (f"{what}: {int(bad.sum())} elements beyond the bar, worst excess "
                                 f"{float(err.max()):.3e} at {int(err.argmax())}")


def _cmp(got, ref, what, floor=1e-9):
    """got: GPU tensor (any device), ref: CPU oracle tensor of the same dtype and numel."""
    got = got.detach().cpu().reshape(-1)
    ref = ref.detach().reshape(-1)
    assert got.dtype == ref.dtype and got.numel() == ref.numel(), f"{what}: layout {got.dtype} {ref.dtype}"
    if ref.dtype == torch.bfloat16:
        d = bf16_ulp_diff(got.contiguous(), ref.contiguous())
        assert int(d.max()) <= 1, f"{what}: {int(d.max())} bf16 ulps ({int((d > 1).sum())} elements)"
    elif ref.dtype == torch.float16:
        from test_gpu_parity import _cmp_f16
        _cmp_f16(got, ref, what=what)
    elif ref.dtype == torch.float32:
        err = (got.double() - ref.double()).abs() - (1e-6 * ref.double().abs() + floor)
        assert float(err.max()) <= 0, f"{what}: max excess {float(err.max()):.3e}"
    elif ref.dtype == torch.uint8 and what.endswith("exp_avg#nf4"):
        a, b = got.to(torch.int32), ref.to(torch.int32)
        d = (torch.stack([a >> 4, a & 15], 1) - torch.stack([b >> 4, b & 15], 1)).abs()
        assert int(d.max()) <= 1, f"{what}: NF4 codes differ by {int(d.max())}"
    else:
        d = (got.to(torch.int32) - ref.to(torch.int32)).abs()
        assert int(d.max()) <= 1, f"{what}: codes differ by {int(d.max())}"


def _tensor_keys(st):
    return [k for k, v in st.items() if torch.is_tensor(v) and k != "step"]


# ---------------------------------------------------------------------- the mirror
class Mirror:
    """CPU oracle copies of selected GPU parameters, re-synced from the GPU before
    every step.  An entry is (i, None): the whole tensor i; (i, rows): its last
    ``rows`` rows; or (i, rows, row0): rows row0 .. row0 + rows - 1 -- each with
    the matching slices of its state (the slice must start on a quantization
    block).  ``retarget`` moves the slices between steps (same row counts)."""

    def __init__(self, gps, entries, kw, n_group):
        self.gps, self.entries, self.n_group = gps, list(entries), n_group
        self.cps = [nn.Parameter(self._gpu_p(e).cpu().clone()) for e in self.entries]
        self.copt = OracleApexW(self.cps, **kw)
        self.pre = None

    def retarget(self, entries):
        entries = list(entries)
        assert [(e[0], e[1]) for e in entries] == [(e[0], e[1]) for e in self.entries], "retarget: same tensors and rows"
        self.entries = entries

    def _row0(self, e):
        i, rows = e[0], e[1]
        return self.gps[i].shape[0] - rows if len(e) < 3 else e[2]

    def _gpu_p(self, e):
        i, rows = e[0], e[1]
        p = self.gps[i].detach()
        if rows is None:
            return p
        r0 = self._row0(e)
        assert 0 <= r0 and r0 + rows <= p.shape[0], f"rows {r0}..{r0 + rows} of {tuple(p.shape)}"
        return p[r0:r0 + rows]

    def _gpu_state(self, gopt, e):
        i, rows = e[0], e[1]
        st = gopt.state[self.gps[i]]
        if rows is None:
            return st
        p = self.gps[i]
        n0 = self._row0(e) * (p.numel() // p.shape[0])
        n1 = n0 + rows * (p.numel() // p.shape[0])
        out = {}
        for k, v in st.items():
            if torch.is_tensor(v) and k != "step":
                ratio = v.numel() / p.numel()
                assert float(n0 * ratio).is_integer() and float(n1 * ratio).is_integer(), f"slice of {k} not aligned"
                out[k] = v.reshape(-1)[int(n0 * ratio):int(n1 * ratio)]
            else:
                out[k] = v
        return out

    def grads(self, gpu_grads):
        out = []
        for e in self.entries:
            g = gpu_grads[e[0]]
            out.append((g if e[1] is None else g[self._row0(e):self._row0(e) + e[1]]).cpu().clone())
        return out

    def snapshot(self, gopt):
        """Before the GPU step: the subset's parameters and (existing) state."""
        self.pre = []
        for e, cp in zip(self.entries, self.cps):
            st = gopt.state[self.gps[e[0]]] if self.gps[e[0]] in gopt.state else None
            snap = None
            if st:
                snap = {k: (v.detach().cpu().clone() if torch.is_tensor(v) else v)
                        for k, v in self._gpu_state(gopt, e).items()}
            self.pre.append((self._gpu_p(e).cpu().clone(), snap))

    def load(self):
        """Oracle parameters and state := the snapshot (in place; fresh state on the first step)."""
        for cp, (p0, snap) in zip(self.cps, self.pre):
            with torch.no_grad():
                cp.copy_(p0)
            if cp not in self.copt.state:
                # the PEFT context and the 16-bit test look at the whole GPU list, as the optimizer does
                peft = OL.peft_context([{"params": self.gps}])
                has16 = any(p.dtype in (torch.float16, torch.bfloat16) for p in self.gps)
                self.copt.state[cp] = OL.init_state(cp, self.copt.group, self.n_group, peft, has_16bit_params=has16)
            if snap is None:
                continue
            cst = self.copt.state[cp]
            for k, v in snap.items():
                if torch.is_tensor(v) and k != "step":
                    cst[k].copy_(v.view(cst[k].shape))
                elif k == "step":
                    cst["step"].fill_(float(v))
                else:
                    cst[k] = v

    def check_layout(self, gopt):
        for e, cp in zip(self.entries, self.cps):
            gs, cs = self._gpu_state(gopt, e), self.copt.state[cp]
            assert sorted(_tensor_keys(gs)) == sorted(_tensor_keys(cs)), f"{e}: state keys"
            for k in _tensor_keys(cs):
                assert gs[k].dtype == cs[k].dtype and gs[k].numel() == cs[k].numel(), f"{e} {k} layout"
            for k in ("is_8bit", "is_4bit_m", "is_quad_v", "block_size_8bit", "is_ultra", "ultra_block_size"):
                assert gs.get(k) == cs.get(k), f"{e} {k}"

    def step(self, grads, sr_check=None):
        for cp, g in zip(self.cps, grads):
            cp.grad = g
        if sr_check is None:
            self.copt.step()
            return
        with sr_check:
            self.copt.step()

    def compare(self, gopt, tag, sr=False):
        for j, (e, cp) in enumerate(zip(self.entries, self.cps)):
            gs, cs = self._gpu_state(gopt, e), self.copt.state[cp]
            name = f"{tag} tensor {e}"
            # one bf16 ulp of the update where the reference rounds it (or its denominator) to
            # bf16: compact with bf16 v, and the 8-bit / ultra step's tensors outside the chunked
            # order (p -= bf16(update))
            # (2^-10 for fp16: one ulp of an fp16 update or denominator)
            half = (torch.bfloat16, torch.float16)
            v16_den = not cs.get("is_8bit", False) and cs["exp_avg_sq"].dtype in half
            quantized_mode = self.copt.group["precision"] in ("8bit", "ultra")
            chunked = cs.get("is_8bit", False) and cp.numel() > 262144
            generic_8bit = quantized_mode and cp.dtype in half and not chunked
            fp16 = torch.float16 in (cp.dtype, cs["exp_avg_sq"].dtype)
            den_rel = (2.0 ** -10 if fp16 else 2.0 ** -7) if (v16_den or generic_8bit) else 2.0 ** -22
            _cmp_p(self._gpu_p(e), cp.detach(), self.pre[j][0], f"{name} p", den_rel)
            for k in _tensor_keys(cs):
                if sr and cs[k].dtype in (torch.uint8, torch.int8) and not k.endswith("scales"):
                    continue            # SR codes: checked by the bracket / bias test
                kind = "#nf4" if (k == "exp_avg" and cs.get("is_4bit_m")) else ""
                floor = 0.0 if k.endswith("scales") else (1e-12 if k == "exp_avg_sq" else 1e-9)
                _cmp(gs[k], cs[k], f"{name} {k}{kind}", floor=floor)


def _sr_targets(chk, mirror, gopt):
    """Register the GPU results of every 16-bit SR store the oracle makes."""
    for e, cp in zip(mirror.entries, mirror.cps):
        if cp.dtype == torch.bfloat16:
            chk.target(cp.data, mirror._gpu_p(e), "p")
        cs = mirror.copt.state[cp]
        if not (cs.get("is_8bit", False) or cs.get("is_ultra", False)) and cs["exp_avg_sq"].dtype == torch.bfloat16:
            chk.target(cs["exp_avg_sq"], mirror._gpu_state(gopt, e)["exp_avg_sq"], "v")


def _check_codes(chk, mirror, gopt):
    """8-bit SR codes of each mirrored tensor against the captured pre-rounding values."""
    for e, cp in zip(mirror.entries, mirror.cps):
        cs = mirror.copt.state[cp]
        if cs.get("is_ultra", False):
            chk.check_int8(mirror._gpu_state(gopt, e)["exp_avg"], what=f"{e} ultra int8")
            continue
        if not cs.get("is_8bit", False):
            continue
        gs = mirror._gpu_state(gopt, e)
        if cs.get("is_4bit_m"):
            chk.check_nf4(gs["exp_avg"], cp.numel(), what=f"{e} nf4")
        else:
            chk.check_int8(gs["exp_avg"], what=f"{e} int8")
        chk.check_logu8(gs["exp_avg_sq"], what=f"{e} logu8")


# ---------------------------------------------------------------------- a driver
def _params(shapes, dtype, gen):
    return [nn.Parameter(torch.empty(s, dtype=dtype, device="cuda").normal_(0.0, 0.02, generator=gen))
            for s in shapes]


def _grads(shapes, dtype, gen, scales, zero=()):
    out = []
    for i, s in enumerate(shapes):
        g = torch.empty(s, dtype=dtype, device="cuda")
        if i in zero:
            g.zero_()
        else:
            g.normal_(0.0, 1e-3 * scales[i], generator=gen)
        out.append(g)
    return out


def _set_sr(gopt, mirror, on):
    """Switch stochastic rounding for the group (compact steps) and every parameter's
    state (8-bit steps read the state's flag), on the GPU and in the oracle."""
    for g in gopt.param_groups:
        g["stochastic_rounding"] = on
    for st in gopt.state.values():
        st["stochastic_rounding"] = on
    mirror.copt.group["stochastic_rounding"] = on


def _drive(tag, shapes, dtype, kw, entries, steps, sr, seed, scales=None, zero=(), per_step=None, sr_from=0):
    """Step the full list on the GPU ``steps`` times; mirror ``entries`` on the CPU
    (a list, or a function of the step number returning the step's entries: the
    same tensors and row counts every step, the slices free to move).

    sr: stochastic rounding from step ``sr_from`` on (off before it).
    per_step(step, gopt, gps, grads, cpu_grads) may replace the oracle's grads
    (C4 pre-clips them with the GPU's coefficient)."""
    from apexw_amd import ApexW
    gen = torch.Generator(device="cuda").manual_seed(seed)
    scales = scales or [1.0] * len(shapes)
    gps = _params(shapes, dtype, gen)
    kw = dict(kw, stochastic_rounding=sr and sr_from == 0)
    torch.manual_seed(seed)      # ApexW draws its rounding-noise seed from torch's generator
    gopt = ApexW(gps, **kw)
    okw = {k: v for k, v in kw.items() if k != "clip_grad_norm"}
    entries_at = entries if callable(entries) else (lambda step: entries)
    mirror = Mirror(gps, entries_at(0), okw, len(shapes))
    stats = None
    for step in range(steps):
        if step:
            mirror.retarget(entries_at(step))
        sr_step = sr and step >= sr_from
        if sr and step == sr_from and step > 0:
            _set_sr(gopt, mirror, True)
        grads = _grads(shapes, dtype, gen, scales, zero)
        for p, g in zip(gps, grads):
            p.grad = g
        mirror.snapshot(gopt)
        gopt.step()
        torch.cuda.synchronize()
        cgrads = mirror.grads(grads)
        if per_step is not None:
            cgrads = per_step(step, gopt, gps, grads, cgrads)
        mirror.load()
        if step == 0:
            mirror.check_layout(gopt)
        chk = None
        if sr_step:
            chk = SRCheck()
            if stats is not None:
                chk.stats = stats
            _sr_targets(chk, mirror, gopt)
        mirror.step(cgrads, chk)
        if sr_step:
            _check_codes(chk, mirror, gopt)
            stats = chk.stats
        mirror.compare(gopt, f"{tag} step {step}", sr=sr_step)
        _say(f"{tag}: step {step} ok" + (f" {stats}" if sr_step else ""))
    return stats


# ---------------------------------------------------------------------- C1
@pytest.mark.parametrize("sr", [False, True], ids=["rne", "sr"])
def test_c1_compact_fp32_2e20(sr):
    """C1: one fp32 tensor of 2^20 elements, 10 steps.  SR off: fp32 v; SR on: bf16 v
    with SR (beta2 0.999 >= 0.995), checked for 10 x 2^20 >= 1e7 elements."""
    _need_gpu()
    _say(f"C1 sr={sr}")
    stats = _drive("C1", [(1 << 20,)], torch.float32, KW, [(0, None)], 10, sr, seed=100)
    if sr:
        assert stats["bf16"].n >= 10_000_000 and abs(stats["bf16"].z) < 3 and abs(stats["bf16"].z_mag) < 3, stats


# ---------------------------------------------------------------------- C2
def _gpt2():
    shapes = gpt2_small_shapes()
    g = torch.Generator().manual_seed(22)
    # per-tensor grad scale log-uniform in [0.1, 10]
    scales = torch.exp((torch.rand(len(shapes), generator=g, dtype=torch.float64) * 2 - 1) * math.log(10.0)).tolist()
    return shapes, scales


def test_c2_gpt2_small_rne_10_steps():
    """C2: the GPT-2-small list (146 tensors, 124.4M params), bf16, SR off, 10 steps,
    every tensor checked."""
    _need_gpu()
    _say("C2 rne")
    shapes, scales = _gpt2()
    assert len(shapes) == 146 and sum(math.prod(s) for s in shapes) == 124_438_272
    _drive("C2", shapes, torch.bfloat16, KW, [(i, None) for i in range(len(shapes))], 10, False, seed=200,
           scales=scales)


def test_c2_gpt2_small_sr_3_steps():
    """C2 as benchmarked (SR on: bf16 quad v with SR, bf16 params with SR), 3 steps:
    the second and third start from non-zero state."""
    _need_gpu()
    _say("C2 sr")
    shapes, scales = _gpt2()
    stats = _drive("C2", shapes, torch.bfloat16, KW, [(i, None) for i in range(len(shapes))], 3, True, seed=201,
                   scales=scales)
    assert stats["bf16"].n >= 10_000_000


def _c2_drift_entries(shapes):
    """Every C2 tensor: vectors whole, matrices as 64-row slices (the first rows of
    the even-numbered tensors, the last rows of the odd ones)."""
    out = []
    for i, s in enumerate(shapes):
        if len(s) == 1 or s[0] <= 64:
            out.append((i, None))
        else:
            out.append((i, 64, 0) if i % 2 == 0 else (i, 64))
    return out


def _ulps(got, ref):
    """bf16 distance in ulps (int64) between a GPU tensor and a CPU oracle tensor."""
    return bf16_ulp_diff(got.detach().cpu().reshape(-1).contiguous(), ref.detach().reshape(-1).contiguous()).long()


def test_c2_gpt2_small_drift_100_steps():
    """C2 for BASELINE's 100 steps, SR off, with NO re-sync: the GPU steps the whole
    list, the oracle steps its own copy of every tensor (vectors whole, 64-row
    slices of the matrices, 5.6 M elements) from the same start with the same
    grads, and the two trajectories are compared every 10 steps.

    m and v never read p and both sides see the same grads, so their differences
    come from rounding alone and stay at the per-step bars (bf16 m <= 1 ulp, a
    difference decays by beta1 each step; fp32 v 1e-6 relative).  p carries
    every rounding flip forward: a flip is one bf16 ulp of p where it happened,
    and |p| never exceeded |p_0| + 2 lr t by step t (AdamW's update is about lr
    per step), so a difference is measured in ulps of that magnitude, e = dp /
    ulp(|p_0| + 2 lr t).  A flip needs the GPU's and torch's fp32 update to
    straddle a bf16 rounding boundary, which the per-step tests see on a few
    elements per million; bars: |e| <= 1 anywhere, e != 0 on fewer than 1e-4 of
    the elements, mean signed e under 1e-5 -- a systematic error (a bias
    correction or a decay off after some step count) moves every element the
    same way and fails the last two bars at once."""
    _need_gpu()
    from apexw_amd import ApexW
    _say("C2 drift, 100 steps")
    shapes, scales = _gpt2()
    gen = torch.Generator(device="cuda").manual_seed(202)
    gps = _params(shapes, torch.bfloat16, gen)
    kw = dict(KW, stochastic_rounding=False)
    torch.manual_seed(202)
    gopt = ApexW(gps, **kw)
    entries = _c2_drift_entries(shapes)
    mirror = Mirror(gps, entries, kw, len(shapes))
    p0 = [cp.detach().float().abs().reshape(-1).clone() for cp in mirror.cps]
    n_el = sum(cp.numel() for cp in mirror.cps)
    assert n_el > 5_000_000
    lr = kw["lr"]
    for step in range(100):
        grads = _grads(shapes, torch.bfloat16, gen, scales)
        for p, g in zip(gps, grads):
            p.grad = g
        if step == 0:
            mirror.snapshot(gopt)
        gopt.step()
        cgrads = mirror.grads(grads)
        if step == 0:
            mirror.load()
            torch.cuda.synchronize()
            mirror.check_layout(gopt)
        mirror.step(cgrads)
        if (step + 1) % 10:
            continue
        torch.cuda.synchronize()
        t = step + 1
        diff, signed, worst, worst_at, worst_m, worst_v = 0, 0.0, 0.0, None, 0, 0.0
        for j, (e, cp) in enumerate(zip(mirror.entries, mirror.cps)):
            gp = mirror._gpu_p(e).detach().cpu().float().reshape(-1)
            rp = cp.detach().float().reshape(-1)
            unit = _bf16_ulp(p0[j] + 2.0 * lr * t)
            err = (gp.double() - rp.double()) / unit.double()
            diff += int((err != 0).sum())
            signed += float(err.sum())
            if float(err.abs().max()) > worst:
                worst, worst_at = float(err.abs().max()), e
            gs, cs = mirror._gpu_state(gopt, e), mirror.copt.state[cp]
            worst_m = max(worst_m, int(_ulps(gs["exp_avg"], cs["exp_avg"]).max()))
            v, vr = gs["exp_avg_sq"].detach().cpu().reshape(-1).double(), cs["exp_avg_sq"].reshape(-1).double()
            worst_v = max(worst_v, float(((v - vr).abs() / (vr.abs() + 1e-30)).max()))
            assert float(gs["step"]) == float(cs["step"]) == t
        frac, mean = diff / n_el, signed / n_el
        _say(f"C2 drift step {t}: p differs at {diff} of {n_el} elements ({frac:.2e}), worst {worst:.2f} "
             f"(tensor {worst_at}), mean signed {mean:+.2e}; m worst {worst_m} ulp; v worst {worst_v:.2e} relative")
        assert worst <= 1 and worst_m <= 1 and worst_v <= 1e-6, (t, worst, worst_m, worst_v)
        assert frac < 1e-4 and abs(mean) < 1e-5, (t, frac, mean)


# ---------------------------------------------------------------------- C3
def _c3_slice_rows(shape):
    """Rows of a mirrored C3 matrix slice: more than 262,144 elements (the oracle's
    chunked path, as for the whole tensor) in whole 2048-element blocks."""
    cols = shape[1]
    rows = -(-262145 // cols)
    while (rows * cols) % 2048:
        rows += 1
    return rows


def _c3_entries(shapes, seed):
    """Per step, for every one of the 291 tensors: the 65 RMSNorms whole, and for
    each of the 226 matrices two row slices of more than 2^18 elements (130 or
    133 2048-element blocks) -- one at a random offset, drawn afresh each step,
    and the last rows (the tensor's last block)."""
    norms = [(i, None) for i, s in enumerate(shapes) if len(s) == 1]
    mats = [i for i, s in enumerate(shapes) if len(s) == 2]

    def at(step):
        rng = np.random.default_rng(seed + 7919 * step)
        out = list(norms)
        for i in mats:
            rows = _c3_slice_rows(shapes[i])
            r0 = int(rng.integers(0, shapes[i][0] - 2 * rows + 1))
            out += [(i, rows, r0), (i, rows)]
        return out
    return at


def test_c3_llama3_8b_8bit_rne_2_steps():
    """C3 shapes (8.03B params, 291 tensors), 8-bit, SR off, 2 steps; checked every
    step: all 65 RMSNorms, and for each of the 226 matrices a random slice and
    its last rows (more than 2^18 elements each, 121 M elements per step)."""
    _need_gpu()
    _say("C3 rne")
    shapes = llama3_8b_shapes()
    assert len(shapes) == 291 and sum(math.prod(s) for s in shapes) == 8_030_261_248
    try:
        _drive("C3", shapes, torch.bfloat16, dict(KW, precision="8bit"), _c3_entries(shapes, 300), 2, False, seed=300)
    finally:
        torch.cuda.empty_cache()


def test_c3_llama3_8b_8bit_sr_3_steps():
    """C3 as benchmarked (SR on), 3 steps, the slices of the RNE test: the fast
    full-block NF4 kernel on every matrix, the INT8 + log-u8 general kernel on
    the RMSNorms; steps 2 and 3 start from non-zero state."""
    _need_gpu()
    _say("C3 sr")
    shapes = llama3_8b_shapes()
    try:
        stats = _drive("C3", shapes, torch.bfloat16, dict(KW, precision="8bit"), _c3_entries(shapes, 301), 3, True,
                       seed=301)
    finally:
        torch.cuda.empty_cache()
    for k in ("bf16", "nf4", "logu8"):
        assert stats[k].n >= 10_000_000, stats
    assert stats["int8"].n > 0


# ---------------------------------------------------------------------- C4
def _c4_clip_check(coef_box):
    def per_step(step, gopt, gps, grads, cgrads):
        plan = next(iter(gopt._plans.values()))
        coef = float(plan.clip_ws[2].item())
        norms = plan.clip_ws[1].cpu().double()
        # per-tensor norms (bf16-rounded, as torch._foreach_norm) within one bf16 ulp of
        # float64, in the plan's tensor order; the total and the coefficient in float64
        n64 = torch.stack([g.double().norm() for g in (gps[int(i)].grad for i in plan.perm)]).cpu()
        assert bool(((norms - n64).abs() <= 2.0 ** -8 * n64 + 1e-30).all()), "C4 per-tensor norms"
        ref = min(1.0 / (float(norms.square().sum().sqrt()) + 1e-6), 1.0)
        assert abs(coef - ref) <= 1e-6 * ref, (coef, ref)
        # from the float64 norms rounded to bf16: a norm within fp32 rounding of a bf16
        # midpoint may round the other way on the GPU, each such tensor moving the total
        # by ~2^-8 (norm / total)^2, far below 1e-6 with 20,000 tensors
        n16 = n64.float().bfloat16().double()
        ref64 = min(1.0 / (float(n16.square().sum().sqrt()) + 1e-6), 1.0)
        assert abs(coef - ref64) <= 1e-6 * ref64, (coef, ref64)
        assert coef < 1.0
        coef_box.append(coef)
        # the oracle's clip multiplies the (cloned) grads by the 0-dim coefficient in their dtype
        out = [g.clone() for g in cgrads]
        torch._foreach_mul_(out, torch.tensor(coef, dtype=torch.float32))
        return out
    return per_step


@pytest.mark.parametrize("sr", [False, True], ids=["rne", "sr"])
def test_c4_ragged_20k_clip(sr):
    """C4: 20,000 ragged bf16 tensors (2.16e9 elements, 5% all-zero grads) with
    global-norm clip 1.0, 2 steps.  The coefficient is checked against float64
    norms; 500 tensors (every 40th) are checked against the oracle given it."""
    _need_gpu()
    _say(f"C4 sr={sr}")
    shapes = ragged_shapes()
    zero = set(torch.randperm(len(shapes), generator=torch.Generator().manual_seed(4))[:1000].tolist())
    coefs = []
    try:
        stats = _drive("C4", shapes, torch.bfloat16, dict(KW, clip_grad_norm=1.0),
                       [(i, None) for i in range(0, len(shapes), 40)], 2, sr, seed=400, zero=zero,
                       per_step=_c4_clip_check(coefs))
    finally:
        torch.cuda.empty_cache()
    assert len(coefs) == 2
    if sr:
        assert stats["bf16"].n >= 10_000_000


# ---------------------------------------------------------------------- C5
C5_SHAPES = [(4096, 4096), (1024, 4096), (1024, 4096), (4096, 4096), (14336, 4096), (14336, 4096), (4096, 14336),
             (4096,), (4096,)]


def _rel_fro(a, b):
    a, b = a.double(), b.double()
    return float((a - b).norm() / b.norm())


def _torch_bf16_ns(G, steps=5, eps=1e-7):
    """The reference's Newton-Schulz on a bf16-capable GPU (apexw/muon.py:102-108,
    :135-184): bf16 work matrix, each torch product rounded to bf16.  The
    transposed operand is made contiguous before the product."""
    from apexw_amd.muon import NS_A, NS_B, NS_C
    X = G.to(torch.bfloat16)
    X = X / (X.norm() + eps)
    tall = X.shape[0] > X.shape[1]
    X = X.T.contiguous() if tall else X.contiguous()
    for _ in range(steps):
        A = X @ X.T.contiguous()
        B = torch.addmm(A, A, A, beta=NS_B, alpha=NS_C)
        X = torch.addmm(X, B, X, beta=NS_A, alpha=1.0)
    return X.T if tall else X


def _ns_launch(plan, phase, stream):
    from apexw_amd import _lib
    lib = _lib.load()
    for probs, items, offsets, n_wg, kind, *_ in plan.iters[0][phase]:
        _lib.check(lib.apexw_gemm_nt_grouped(probs.data_ptr(), items.data_ptr(), offsets.data_ptr(), n_wg, kind,
                                             None, stream), "apexw_gemm_nt_grouped")


@pytest.mark.parametrize("rows,cols", [(4096, 4096), (4096, 14336)])
def test_c5_ns_products_full_size(rows, cols):
    """Each Newton-Schulz product at C5's sizes (one grouped launch each, 3200 tiles
    for B X at 4096 x 14336) against fp32 products of the same bf16 operands on the
    GPU: |O - ref| <= 2^-8 |ref| + 1e-4 max|ref| (bf16 output rounding is 2^-9)."""
    _need_gpu()
    from apexw_amd.muon import NS_A, NS_B, NS_C, NSPlan, NSWorkspace
    _say(f"C5 NS products {rows}x{cols}")
    torch.backends.cuda.matmul.allow_tf32 = False
    gen = torch.Generator(device="cuda").manual_seed(500 + cols)
    ws = NSWorkspace(rows, cols, 1, torch.device("cuda"))
    G = torch.randn(rows, cols, generator=gen, device="cuda")
    X0 = torch.zeros(ws.mp, ws.np_, dtype=torch.bfloat16, device="cuda")
    X0[:rows, :cols] = (G / G.norm()).bfloat16()
    ws.x[0][0].copy_(ws.in_layout(X0))   # the work buffers hold 32 x 32 panels
    ws.xt[0][0].copy_(ws.in_layout(X0.t().contiguous()))   # X' = B X + a X reads X^T
    # two iterations: the first (run below) is not the last, so its X' product also
    # writes X'^T for the next one (a last product's X'^T is dropped when no other
    # matrix of the launch needs it)
    plan = NSPlan([ws], [2], torch.device("cuda"))
    stream = torch.cuda.current_stream().cuda_stream

    def bar(got, ref, what):
        err = (got.float() - ref).abs() - (2.0 ** -8 * ref.abs() + 1e-4 * ref.abs().max())
        assert float(err.max()) <= 0, f"{what}: max excess {float(err.max()):.3e}"

    X = ws.rows_of(ws.x[0][0]).float()
    _ns_launch(plan, 0, stream)
    torch.cuda.synchronize()
    bar(ws.rows_of(ws.a[0]), X @ X.T, "A = X X^T")
    A = ws.rows_of(ws.a[0]).float()
    _ns_launch(plan, 1, stream)
    torch.cuda.synchronize()
    bar(ws.rows_of(ws.b[0]), NS_C * (A @ A) + NS_B * A, "B = c A A + b A")
    B = ws.rows_of(ws.b[0]).float()
    _ns_launch(plan, 2, stream)
    torch.cuda.synchronize()
    Xn = ws.rows_of(ws.x[1][0])
    bar(Xn, B @ X + NS_A * X, "X' = B X + a X")
    # and its transpose, for the next iteration's X' product
    assert torch.equal(ws.rows_of(ws.xt[1][0]), Xn.t().contiguous())
    # the zero padding stays zero through the products
    assert float(Xn[rows:].abs().max() if ws.mp > rows else 0.0) == 0.0


def test_c5_hybrid_step_one_llama_layer():
    """C5: one Llama-3-8B layer under HybridApexW (use_muon=True), 2 steps.  Routing:
    q, o, gate, up, down to Muon; k, v (aspect exactly 4) and the RMSNorms to ApexW.
    Muon: fp32 momentum at 1e-6; the bf16 Newton-Schulz result no farther (relative
    Frobenius) from the fp32 polar iteration on the same momentum than torch's bf16
    products of the same iteration (the reference's GPU path) are, plus 0.5%, and
    within 1% of those products; the parameter update from that result at one bf16
    ulp.  ApexW part (SR off): one bf16 ulp
    against the oracle."""
    _need_gpu()
    from apexw_amd import ApexW
    from oracle.muon import newton_schulz5
    _say("C5 hybrid layer")
    torch.backends.cuda.matmul.allow_tf32 = False
    gen = torch.Generator(device="cuda").manual_seed(550)
    gps = _params(C5_SHAPES, torch.bfloat16, gen)
    opt = ApexW(gps, lr=1e-3, weight_decay=0.1, use_muon=True, stochastic_rounding=False)
    opt.muon_opt.keep_ns_result = True   # the fused update's U, kept for the check below
    muon_idx = [0, 3, 4, 5, 6]
    assert [id(p) for p in opt.muon_params] == [id(gps[i]) for i in muon_idx]
    assert [id(p) for p in opt.adamw_params] == [id(gps[i]) for i in (1, 2, 7, 8)]
    mg = opt.muon_opt.param_groups[0]
    lr_m, wd, mu = mg["lr"], mg["weight_decay"], mg["momentum"]
    assert lr_m == 5e-3 and mu == 0.95 and mg["ns_steps"] == 5
    mirror = Mirror(gps, [(i, None) for i in (1, 2, 7, 8)], dict(lr=1e-3, weight_decay=0.1, betas=(0.9, 0.99),
                                                                  stochastic_rounding=False), 4)
    bufs = {i: torch.zeros(C5_SHAPES[i], device="cuda") for i in muon_idx}
    for step in range(2):
        grads = _grads(C5_SHAPES, torch.bfloat16, gen, [1.0] * len(C5_SHAPES))
        for p, g in zip(gps, grads):
            p.grad = g
        before = {i: gps[i].detach().clone() for i in muon_idx}
        mirror.snapshot(opt.adamw_opt)
        opt.step()
        torch.cuda.synchronize()
        # ApexW-routed tensors
        mirror.load()
        mirror.step(mirror.grads(grads))
        mirror.compare(opt.adamw_opt, f"C5 step {step} adamw")
        # Muon: per shape, the workspace slot holding the Newton-Schulz result
        ws_by_shape = {k[1]: ws for k, ws in opt.muon_opt._ws.items()}
        slot = {}
        for i in muon_idx:
            slot.setdefault(C5_SHAPES[i], []).append(i)
        for shape, members in slot.items():
            ws = ws_by_shape[shape]
            rows, cols = shape
            batched = len(members) > 1
            for k, i in enumerate(members):
                bufs[i].mul_(mu).add_(grads[i].float(), alpha=1.0 - mu)
                st = opt.muon_opt.state[gps[i]]
                _cmp(st["momentum"], bufs[i].cpu(), f"C5 step {step} momentum {shape}")
                wide = ws.rows_of(ws.x[5 % 2][k])[:min(rows, cols), :max(rows, cols)]
                U_gpu = wide.T if rows > cols else wide
                U32 = newton_schulz5(bufs[i], 5, work_dtype=torch.float32)
                U16 = _torch_bf16_ns(bufs[i])
                e32, e16 = _rel_fro(U_gpu, U32), _rel_fro(U_gpu, U16.float())
                _say(f"C5 step {step} {shape}[{k}]: |U - U_fp32| {e32:.4f}, |U - U_torch_bf16| {e16:.4f}, "
                     f"torch bf16 vs fp32 {_rel_fro(U16.float(), U32):.4f}")
                # no farther from the fp32 iteration than torch's bf16 products are (plus 0.5%),
                # and within 1% of those products themselves
                e_ref = _rel_fro(U16.float(), U32)
                assert e32 <= e_ref + 0.005 and e32 <= 0.03, (e32, e_ref)
                assert e16 <= 0.01, e16
                # the update from the GPU's own U: p = round(round(p * wd_factor) - lr * scale * U)
                scale = 0.2 * math.sqrt(max(rows, cols))
                wdf, neg = 1.0 - lr_m * wd, -lr_m * scale
                # torch's add_ (and _foreach_add_) on a bf16 p takes alpha in bf16; mul_ keeps
                # its scalar in fp32, the same-dtype _foreach_mul_ of the batched path rounds it
                neg = float(torch.tensor(neg).bfloat16().float())
                if batched:
                    wdf = float(torch.tensor(wdf).bfloat16().float())
                decayed = (before[i].float() * np.float32(wdf)).bfloat16().float()
                p_ref = (decayed + np.float32(neg) * U_gpu.float()).bfloat16()
                _cmp(gps[i], p_ref.cpu(), f"C5 step {step} p {shape}[{k}]")
