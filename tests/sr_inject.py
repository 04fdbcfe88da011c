"""Check stochastic rounding on the GPU against the CPU oracle (test helper).

With stochastic rounding (SR) on, the GPU and the oracle draw different random
numbers, so their results cannot be compared element by element.  Three things
can be, and ``SRCheck`` checks all of them while the oracle runs one step from
the GPU's pre-step state:

* **bracket**: every SR result of the GPU is one of the two representable
  neighbours of the oracle's exact pre-rounding value (bf16 values, NF4 /
  INT8 / log-uint8 codes);
* **unbiasedness**: with d_i = chosen_i - exact_i and
  var_i = (exact_i - lo_i)(hi_i - exact_i), both in units of the gap
  hi_i - lo_i, an unbiased rounding has E[sum d] = 0 and Var[sum d] =
  sum var; ``Stat.z`` is the standardised sum, ``Stat.z_mag`` the same for
  d_i times the sign of exact_i (bias toward or away from zero), and both
  |z| < 3 is the 3-sigma bar;
* **everything downstream**: a 16-bit store that the same step reads again
  (the compact v EMA feeds the denominator) is replaced by the GPU's choice
  in the oracle's tensor, so the rest of the step is deterministic and is
  compared at the round-to-nearest bars by the caller.

The quantizers' codes are not read again within a step, so those calls are
captured (exact pre-rounding values in code units, in call order) and checked
against the GPU's stored codes afterwards with ``check_nf4`` / ``check_int8`` /
``check_logu8``.
"""

import math

import torch

import oracle.compact as OC
import oracle.quant as Q


class Stat:
    """Running standardised sums of rounding offsets (gap units): ``z`` of the
    signed offsets and ``z_mag`` of the offsets times the sign of the exact
    value (a rounding biased toward or away from zero cancels in ``z`` on
    sign-symmetric data, not in ``z_mag``)."""

    def __init__(self):
        self.n = 0
        self.sum_d = 0.0
        self.sum_dm = 0.0
        self.sum_var = 0.0

    def add(self, d, var, sign=None):
        self.n += int(d.numel())
        self.sum_d += float(d.double().sum())
        self.sum_dm += float((d.double() * sign).sum()) if sign is not None else float(d.double().sum())
        self.sum_var += float(var.double().sum())

    @property
    def z(self):
        return self.sum_d / math.sqrt(self.sum_var) if self.sum_var > 0 else 0.0

    @property
    def z_mag(self):
        return self.sum_dm / math.sqrt(self.sum_var) if self.sum_var > 0 else 0.0

    def __repr__(self):
        return f"Stat(n={self.n}, z={self.z:+.3f}, z_mag={self.z_mag:+.3f})"


def bf16_neighbours(x):
    """(toward-zero, away-from-zero) bf16 values around fp32 x, as fp32 (equal when x is a bf16)."""
    x = x.float().contiguous()
    bits = x.view(torch.int32)
    trunc_bits = bits & -65536
    exact = trunc_bits == bits
    away_bits = torch.where(exact, trunc_bits, trunc_bits + 65536)
    return trunc_bits.view(torch.float32), away_bits.view(torch.float32)


def offsets(chosen, exact, lo, hi, what, lo_w=None, hi_w=None, near=None):
    """Bracket check; returns (d, var, sign of exact) in gap units over the elements
    with a nonzero gap.

    ``near`` marks elements whose exact value lies within the GPU's arithmetic
    error of a bracket end: the GPU may see them on the other side, so they are
    checked against the widened bracket [lo_w, hi_w] and left out of the sums
    (they sit at both ends of the gap alike, so leaving them out biases nothing).
    """
    ok = (chosen == lo) | (chosen == hi)
    if near is not None:
        ok = ok | (near & (chosen >= lo_w) & (chosen <= hi_w))
    if not bool(ok.all()):
        j = int(torch.nonzero(~ok)[0])
        detail = dict(index=j, chosen=float(chosen[j]), exact=float(exact[j]), lo=float(lo[j]), hi=float(hi[j]))
        if near is not None:
            detail.update(lo_w=float(lo_w[j]), hi_w=float(hi_w[j]), near=bool(near[j]))
        raise AssertionError(f"{what}: {int((~ok).sum())} SR results outside the bracket of the exact value, "
                             f"first {detail}")
    gap = hi - lo
    live = gap != 0
    if near is not None:
        live = live & ~near
    g = gap[live].double()
    e = exact[live].double()
    d = (chosen[live].double() - e) / g
    var = ((e - lo[live].double()) * (hi[live].double() - e)) / (g * g)
    return d, var, torch.sign(e)


def _bf16_bracket(x):
    a, b = bf16_neighbours(x)
    return torch.minimum(a, b), torch.maximum(a, b)


class SRCheck:
    """Patch the oracle's SR entry points while active (``with SRCheck() as sr: ...``).

    ``target(oracle_tensor, gpu_result)`` registers the GPU's post-step tensor
    for an oracle tensor whose 16-bit SR stores are to be checked and replaced
    (a parameter, a compact v).  Stores into a slice of a registered tensor map
    to the same slice of the GPU result.
    """

    def __init__(self):
        self.targets = []
        self.stats = {k: Stat() for k in ("bf16", "nf4", "int8", "logu8")}
        self.captured = {"nf4": [], "int8": [], "logu8": []}

    def target(self, oracle_tensor, gpu_result, label="bf16"):
        """label: an extra statistic for this target's stores ("bf16/<label>"), beside
        the pooled "bf16" one."""
        assert oracle_tensor.is_contiguous() and oracle_tensor.dtype == gpu_result.dtype
        self.targets.append((oracle_tensor, gpu_result.detach().cpu().contiguous(), label))

    def reset_captures(self):
        self.captured = {"nf4": [], "int8": [], "logu8": []}

    # ---------------------------------------------------------------- patching
    def __enter__(self):
        self._orig = (Q.store_16bit, OC.store_16bit, Q.quant_nf4, Q.quant_int8, Q.quant_logu8)
        Q.store_16bit = OC.store_16bit = self._store
        Q.quant_nf4, Q.quant_int8, Q.quant_logu8 = self._nf4, self._int8, self._logu8
        return self

    def __exit__(self, *exc):
        Q.store_16bit, OC.store_16bit, Q.quant_nf4, Q.quant_int8, Q.quant_logu8 = self._orig
        return False

    def _gpu_for(self, dst):
        esize = dst.element_size()
        for t, gpu, label in self.targets:
            lo = t.data_ptr()
            if t.dtype == dst.dtype and lo <= dst.data_ptr() < lo + t.numel() * esize:
                off = (dst.data_ptr() - lo) // esize
                return gpu.reshape(-1)[off:off + dst.numel()].view(dst.shape), label
        raise AssertionError("an SR store into a tensor with no registered GPU result")

    def _store(self, dst, src_f32, stochastic):
        if not stochastic or dst.dtype == torch.float32:
            return self._orig[0](dst, src_f32, stochastic)
        assert dst.dtype == torch.bfloat16 and dst.is_contiguous()
        gpu, label = self._gpu_for(dst)
        x = src_f32.float().reshape(-1)
        lo, hi = _bf16_bracket(x)
        # the GPU's pre-rounding value may differ by a few fp32 ulps of the operands
        # (its reciprocal, square root and fused operations): dst still holds the value
        # the step starts from (p before the update, v before the EMA), so 2^-19 of
        # |x| + |dst| is 16 fp32 ulps of the larger operand, also where x cancels
        slack = (x.abs() + dst.reshape(-1).float().abs()) * 2.0 ** -19
        lo_w, _ = _bf16_bracket(x - slack)
        _, hi_w = _bf16_bracket(x + slack)
        near = ((x - lo) <= slack) | ((hi - x) <= slack)
        res = offsets(gpu.reshape(-1).float(), x, lo, hi, f"bf16 store (dst {tuple(dst.shape)})", lo_w, hi_w, near)
        self.stats["bf16"].add(*res)
        if label != "bf16":
            self.stats.setdefault(f"bf16/{label}", Stat()).add(*res)
        dst.copy_(gpu)

    def _nf4(self, x, block, old_scales=None, stochastic=False):
        q, s = self._orig[2](x, block, old_scales, False)
        if stochastic:
            b, n = Q._blocks(x, block)
            self.captured["nf4"].append((b / s).clamp(-1.0, 1.0).reshape(-1)[:n].clone())
        return q, s

    def _int8(self, x, block, old_scales=None, stochastic=False):
        q, s = self._orig[3](x, block, old_scales, False)
        if stochastic:
            b, n = Q._blocks(x, block)
            self.captured["int8"].append((b / s).reshape(-1)[:n].clone())
        return q, s

    def _logu8(self, v, block, old_scales=None, stochastic=False):
        q, s = self._orig[4](v, block, old_scales, False)
        if stochastic:
            b, n = Q._blocks(v, block)
            b = torch.nan_to_num(b, nan=0.0, posinf=0.0, neginf=0.0)
            r = (b / s).clamp_min(Q.V_MIN_RATIO)
            c = torch.log2(r).mul_(Q.V_SCALE).add_(255.0)
            c = torch.where(b > 0, c, torch.full_like(c, -1.0))     # -1 marks v <= 0 (code 0)
            self.captured["logu8"].append(c.reshape(-1)[:n].clone())
        return q, s

    # ---------------------------------------------------------------- code checks
    def _take(self, kind, count):
        """The next ``count`` captured values of ``kind`` (the oracle quantizes one tensor
        at a time, in order, so a tensor's values are consecutive)."""
        vals, got = self.captured[kind], []
        n = 0
        while n < count:
            assert vals, f"no SR {kind} quantization was captured for {count - n} more values"
            head = vals.pop(0)
            if n + head.numel() > count:
                vals.insert(0, head[count - n:])
                head = head[:count - n]
            got.append(head)
            n += head.numel()
        return torch.cat(got)

    def check_nf4(self, gpu_packed, numel, what="nf4"):
        """GPU NF4 codes (packed, even element in the high nibble) against the captured normed values."""
        normed = self._take("nf4", numel)
        p = gpu_packed.reshape(-1).cpu().to(torch.int64)
        codes = torch.stack([p >> 4, p & 15], 1).reshape(-1)[:numel]
        levels = Q.NF4_CODEBOOK[:15]

        def bracket(x):
            hi_i = torch.searchsorted(levels, x.clamp(-1.0, 1.0)).clamp(0, 14)
            return levels[(hi_i - 1).clamp_min(0)], levels[hi_i]
        lo, hi = bracket(normed)
        slack = 2e-6       # the GPU's normed value (its scale, reciprocal and dequantized m) vs torch's
        lo_w, _ = bracket(normed - slack)
        _, hi_w = bracket(normed + slack)
        near = ((normed - lo) <= slack) | ((hi - normed) <= slack)
        assert bool((codes <= 14).all()), f"{what}: code 15 written"
        self.stats["nf4"].add(*offsets(Q.NF4_CODEBOOK[codes], normed, lo, hi, what, lo_w, hi_w, near))

    def check_int8(self, gpu_codes, what="int8"):
        codes = gpu_codes.reshape(-1).cpu().to(torch.float32)
        y = self._take("int8", codes.numel())
        y = y.clamp(-127, 127)
        slack = 1e-4       # fp32 error of y = m / scale near |y| = 127 is ~1e-5
        near = ((y - y.round()).abs() <= slack)
        self.stats["int8"].add(*offsets(codes, y, y.floor(), y.ceil(), what, (y - slack).floor(), (y + slack).ceil(),
                                        near))

    def check_logu8(self, gpu_codes, what="logu8", slack=2e-3):
        """log-uint8 codes: 0 where v <= 0, else a neighbour of the exact code c (clamped to
        [1, 255]).  The GPU's log2 differs from torch's by a few fp32 ulps, so a c within
        ``slack`` of an integer may be seen on the other side of it: those elements are
        checked against the widened bracket and left out of the bias sum.  Codes above
        254 clamp to 255, which is c's upper neighbour, so no other clamp is special."""
        codes = gpu_codes.reshape(-1).cpu().to(torch.float32)
        c = self._take("logu8", codes.numel())
        zero = c < 0
        assert bool((codes[zero] == 0).all()), f"{what}: nonzero code where v <= 0"
        c, codes = c[~zero], codes[~zero]
        low = c < 1.0
        assert bool((codes[low] == 1).all()), f"{what}: clamped codes"
        c, codes = c[~low], codes[~low]
        near = (c - c.round()).abs() < slack
        self.stats["logu8"].add(*offsets(codes, c, c.floor(), c.ceil(), what, (c - slack).floor().clamp_min(1.0),
                                         (c + slack).ceil().clamp_max(255.0), near))

    def assert_unbiased(self, kinds, min_n=10_000_000):
        for k in kinds:
            st = self.stats[k]
            assert st.n >= min_n, f"{k}: only {st.n} SR elements"
            assert abs(st.z) < 3.0 and abs(st.z_mag) < 3.0, f"{k}: biased SR, {st}"
