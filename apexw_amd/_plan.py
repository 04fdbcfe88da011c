"""Cached execution plan of one parameter group: device tables + one launch per step.

The reference caches per-group tensor lists in ``FastExecutionPlan``
(apexw/optimizer.py:406-1341) and replays them from the second step on; the
first step after a (re)build runs the uncached path.  Both paths round
differently, and this plan keeps that distinction (``MODE_COLD`` for the first
launch, ``MODE_REPLAY`` afterwards).

What the plan owns, built once and reused every step:
  * the tensor table (64-byte descriptors, device-resident) and the unit
    (chunk) table that splits every tensor into 2048-element units (compact)
    or quantization blocks (8-bit) -- one kernel launch covers the whole group;
  * one shared CPU fp32 buffer holding every parameter's step counter; each
    ``state["step"]`` is a 0-dim view into it, so advancing all counters is one
    op instead of one per tensor;
  * clip workspaces (per-unit partial sums, per-tensor norms, the coefficient);
  * with grad_centralization, one prepared-grad buffer per parameter and the
    preparation table: the reference's _prepare_grads works on a clone, and the
    step and the clip read the prepared copy.
Every step the native scan (csrc/host.cpp) re-reads each parameter's data
pointer and dtype and each grad's pointer: a grad that moved is re-pointed in
the tensor table (one host-to-device copy); a parameter whose storage or dtype
changed in place (``p.data = ...``, ``module.to(dtype)``) invalidates the plan.
"""

import functools
import math
import operator

import numpy as np
import torch

from . import _lib as L



def _upload(a, device):
    """Copy a host array to the device without a host synchronisation.

    The bytes go through a pinned tensor from torch's caching host allocator,
    which holds the block until the asynchronous copy has run, so a step that
    re-uploads a table (grads that moved) does not wait for the device."""
    t = torch.from_numpy(np.array(a, copy=True))
    if torch.device(device).type == "cpu":     # host-only plans of the unit tests
        return t
    return t.pin_memory().to(device, non_blocking=True)


def _host():
    """The native scan module, imported on first use (the build imports this package)."""
    try:
        from . import _host as mod
    except ImportError as exc:
        raise ImportError("apexw_amd/_host*.so is not built; run `python -m apexw_amd._build`") from exc
    return mod

_DT = {torch.float32: L.F32, torch.bfloat16: L.BF16, torch.float16: L.F16, torch.uint8: L.U8, torch.int8: L.I8}
CHUNKED_MIN_NUMEL = 262144  # larger 8-bit tensors take the reference's chunked rounding order
_GRAD = operator.attrgetter("grad")

# status of _host.scan (csrc/host.cpp)
SCAN_SAME, SCAN_GRADS_MOVED, SCAN_MISSING, SCAN_REBUILT, SCAN_SLOW, SCAN_GRAD_DTYPE = range(6)


@functools.lru_cache(maxsize=64)
def _lerp_coef(w):
    w32 = np.float32(w)
    if abs(float(w32)) < 0.5:
        return float(w32), False
    return float(np.float32(w32 - np.float32(1.0))), True


class StepPlan:
    def __init__(self, opt, group, params, kind, native=False, hooked=False, single=False):
        self.kind = kind                  # "compact" or "q8"
        self.native = native              # compact group stepped with torch._fused_adamw_ rounding
        # hooked: a batch of in-backward steps; the caller passes the step counts,
        # and the group's other parameters may hold grads meanwhile
        # single: enable_fused_backward's per-parameter update (APEXW_MODE_SINGLE)
        self.single = single
        self.hooked = hooked or single
        self.params = list(params)
        self.param_ids = tuple(id(p) for p in self.params)
        active = set(self.params)
        self.inactive = [] if self.hooked else [p for p in group["params"]
                                           if getattr(p, "requires_grad", False) and p not in active]
        self.precision = group["precision"]
        self.decay_norm_only = group["decay_norm_only"]
        self.device = self.params[0].device
        self.states = [opt.state[p] for p in self.params]
        self.gc = bool(group.get("grad_centralization", False))
        # cautious=True: a count pass forms the mask's mean before the step
        self.cautious = self._cautious_of(group)
        # maximize=True (not the in-backward flush nor the per-parameter update, which step
        # without it): the grads are negated through a negative unscale factor
        self.maximize = self._maximize_of(group)
        # nesterov=True: a compact group's step scalars come from the host (no device AMP);
        # refreshed from the group each step (valid_for)
        self.nesterov = bool(group.get("nesterov", False))
        # lion=True: the compact step's sign update in place of AdamW's (no v read)
        self.lion = self._lion_of(group)
        # amsgrad=True: the compact step keeps a running max of v (hparams.max_v)
        self.amsgrad = self._amsgrad_of(group)
        # beta3 (AdEMAMix): the compact step keeps a slow first moment (hparams.slow);
        # slow_made: whether the group had beta3 when the plan was made (validity)
        self.slow = self._slow_of(group)
        self.slow_made = group.get("beta3") is not None
        self.beta3, self.alpha = group.get("beta3"), float(group.get("alpha", 5.0))
        self.d_counts = None
        self.cold_done = False
        self._nesterov = False
        self.amp_dirty = False      # skips counted on the device that the host has not folded
        # each grad's dtype as the table is built for it: a parameter's grads may be of another
        # dtype (torch's Tensor.grad_dtype), and a change of it makes a new plan
        self.grad_dtypes = [p.grad.dtype if p.grad is not None else p.dtype for p in self.params]
        self.mixed = any(gd != p.dtype for gd, p in zip(self.grad_dtypes, self.params))
        self._build_steps()
        self._build_tables(group)

    def _cautious_of(self, group):
        """The group's cautious flag as this plan's kernels take it: the 8-bit / ultra
        and compact steps, not enable_fused_backward's per-parameter update (which has
        no cautious branch, optimizer.py:2373-2471); lion takes the place of the AdamW
        update, cautious with it (optimizer.py:5677-5683)."""
        return bool(group.get("cautious", False)) and not self.single and not (
            self.kind == "compact" and self._lion_of(group))

    def _maximize_of(self, group):
        return bool(group.get("maximize", False)) and not self.hooked

    def _amsgrad_of(self, group):
        """The group's amsgrad flag as this plan's kernels take it: the compact step, not
        the in-backward batches nor the per-parameter update (which step without it,
        optimizer.py:2360, :2373-2471)."""
        return (bool(group.get("amsgrad", False)) and self.kind == "compact" and not self.hooked
                and not self._lion_of(group))

    def _slow_of(self, group):
        """beta3 as this plan's kernels take it: the compact step without lion, not the
        in-backward batches nor the per-parameter update (optimizer.py:2360, :2373-2471)."""
        return (group.get("beta3") is not None and self.kind == "compact" and not self.hooked
                and not self._lion_of(group))

    def _lion_of(self, group):
        """The group's lion flag as this plan's kernels take it: the compact step, not the
        per-parameter update, which steps AdamW whatever the group says (optimizer.py:2373-2471)."""
        return bool(group.get("lion", False)) and self.kind == "compact" and not self.hooked

    # ------------------------------------------------------------------ validity
    def valid_for(self, group):
        """The reference's FastExecutionPlan.is_valid_for_step (optimizer.py:575-621):
        every plan parameter has a grad and no other trainable parameter of the
        group has one.  Also invalid when a parameter's storage or dtype changed
        in place, since the table holds its address."""
        if not self.params:
            return False
        if group.get("decay_norm_only", self.decay_norm_only) != self.decay_norm_only:
            return False
        if group.get("precision") != self.precision:
            return False
        if bool(group.get("grad_centralization", False)) != self.gc:
            return False
        if self._maximize_of(group) != self.maximize:
            return False
        # amsgrad switched on or off: a new plan (FastExecutionPlan.is_valid_for_step,
        # optimizer.py:585-586: the plan holds max_exp_avg_sq lists only when it was made
        # with amsgrad and without lion, so lion with amsgrad makes every step a cold one)
        if self.kind == "compact" and not self.hooked and bool(group.get("amsgrad", False)) != self.amsgrad:
            return False
        # beta3 set or cleared: a new plan (optimizer.py:587-588)
        if (group.get("beta3") is not None) != self.slow_made:
            return False
        if self.kind == "q8":
            # cautious keeps every 8-bit tensor in the generic order: another table
            if self._cautious_of(group) != self.cautious:
                return False
        else:
            # compact: the replayed plan takes cautious in place, as the reference's does;
            # the native fused plan does not
            self.cautious = self._cautious_of(group)
            if self.native and self.cautious:
                return False
        # nesterov: the replayed plan takes a change in place (the reference's
        # replayed plan stays valid, optimizer.py:575-621); the native fused plan does not
        self.nesterov = bool(group.get("nesterov", False))
        if self.native and self.nesterov:
            return False
        self._scan_status = self._scan()
        if self._scan_status == SCAN_GRAD_DTYPE:
            # a grad of another dtype than the table's: new descriptors; the reference's replayed
            # foreach plan steps it in place (its validity test reads no dtype), so the new plan
            # keeps this one's replay order
            self.keep_replay = self.cold_done and not self.native
            return False
        ok = self._scan_status in (SCAN_SAME, SCAN_GRADS_MOVED, SCAN_SLOW)
        if ok and self._lion_of(group) != self.lion:
            # lion switched on or off: the descriptors change (no v under lion), so a new
            # plan; the reference's replayed foreach plan stays valid across the switch
            # (optimizer.py:575-621) and its native fused one does not, so the new plan keeps
            # this one's replay order when there is one (keep_replay)
            self.keep_replay = self.cold_done and not self.native
            return False
        return ok

    def _scan(self):
        return self._H.scan(self.params, self.inactive, *self._scan_addrs)

    # ------------------------------------------------------------------ build
    def _build_steps(self):
        vals = [float(st["step"].item()) for st in self.states]
        self.steps = torch.tensor(vals, dtype=torch.float32)
        self._steps_np = self.steps.numpy()   # the same memory: cheap host-side updates
        if self.hooked:
            return
        for i, st in enumerate(self.states):
            st["step"] = self.steps[i]

    def _tensor_flags(self, p, st, wd_on, gdt):
        f = (_DT[p.dtype] << L.PDT_SHIFT) | (_DT[gdt] << L.GDT_SHIFT)
        if wd_on and (not self.decay_norm_only or p.dim() >= 2):
            f |= L.FLAG_WD
        if st.get("is_factored_v", False):
            # row / column v: stepped by apexw_factored_step, skipped by the step kernels
            f |= L.FLAG_FACTORED
            if st.get("is_8bit", False):
                if st.get("is_6bit_m", False):
                    f |= L.FLAG_M6
                return f, int(st["block_size_8bit"])
            return f | (_DT[st["exp_avg"].dtype] << L.MDT_SHIFT), 0
        m = st["exp_avg"]
        # lion reads no v: its descriptors describe m in v's place (never quad, never scaled)
        v = m if self.lion else st["exp_avg_sq"]
        if self.kind == "compact":
            f |= (_DT[m.dtype] << L.MDT_SHIFT) | (_DT[v.dtype] << L.VDT_SHIFT)
            if v.numel() * 4 == p.numel() and p.numel() % 4 == 0:
                f |= L.FLAG_QUAD
            if torch.float16 in (m.dtype, v.dtype) and not self.native and not self.single and not self.lion:
                # the dynamic v scale of fp16 subgroups (set per launch, see _update_vscales)
                f |= L.FLAG_VSCALE
            block = 0
        elif st.get("is_ultra", False):
            # precision "ultra": INT8 m blocks, dense v, the per-parameter rounding order
            block = int(st.get("block_size_8bit", st.get("ultra_block_size", 256)))
            f |= L.FLAG_ULTRA | L.FLAG_GENERIC | (_DT[v.dtype] << L.VDT_SHIFT)
            if block % 8:
                f |= L.FLAG_SCALAR
        elif st.get("is_8bit", False):
            block = int(st["block_size_8bit"])
            if st.get("is_4bit_m", False):
                f |= L.FLAG_NF4
            if st.get("is_quad_v", False):
                f |= L.FLAG_QUAD
            # cautious=True keeps every tensor off the chunked order (optimizer.py:4402-4414)
            if self.cautious or not (p.numel() > CHUNKED_MIN_NUMEL and p.is_contiguous()):
                f |= L.FLAG_GENERIC
            if block % 8:
                f |= L.FLAG_SCALAR
        else:
            # dense m / v, stepped in units of 2048 elements
            f |= L.FLAG_DENSE | (_DT[m.dtype] << L.MDT_SHIFT) | (_DT[v.dtype] << L.VDT_SHIFT)
            block = L.COMPACT_UNIT
        return f, block

    def _check_strided(self, i, p, st):
        """A non-contiguous parameter (channels_last and the like): the compact, full and
        auto steps take it when it is dense and non-overlapping and its state shares its
        layout, since their update is element by element and can walk all four tensors in
        memory order.  Quad v (groups of four logical elements; the reference's
        `.view(-1, 4)` fails on such tensors too), centralization (rows in logical order)
        and the quantized and per-parameter steps are refused."""
        from torch._prims_common import is_non_overlapping_and_dense
        what = f"parameter {i} ({tuple(p.shape)}, strides {p.stride()})"
        if self.kind != "compact" or self.single or not is_non_overlapping_and_dense(p):
            raise NotImplementedError(f"apexw_amd: {what}: the HIP step needs contiguous parameters, or dense "
                                      "non-overlapping ones in the compact, full and auto precisions")
        if self.gc:
            raise NotImplementedError(f"apexw_amd: {what}: grad centralization needs contiguous parameters")
        for k in ("exp_avg", "exp_avg_sq"):
            t = st.get(k)
            if t is None:
                continue
            if t.numel() != p.numel():
                raise NotImplementedError(f"apexw_amd: {what}: quad v needs contiguous parameters")
            if t.stride() != p.stride():
                raise NotImplementedError(f"apexw_amd: {what}: state '{k}' is not in the parameter's layout")

    def _build_tables(self, group):
        wd_on = group["weight_decay"] != 0
        n = len(self.params)
        tab = np.zeros(n, dtype=L.TENSOR_DTYPE)
        counts = np.zeros(n, dtype=np.int64)
        if self.mixed:
            # grads of another dtype than their parameters (Tensor.grad_dtype): the compact,
            # full and auto steps, with one grad dtype per parameter dtype, as the reference's
            # foreach subgroups take them (one conversion rule per subgroup, optimizer.py:5662)
            if self.kind != "compact" or self.single:
                raise NotImplementedError("apexw_amd: grads of another dtype than their parameters in the "
                                          f"{self.precision} precision or the per-parameter update")
            per = {}
            for p, gd in zip(self.params, self.grad_dtypes):
                per.setdefault(p.dtype, set()).add(gd)
            if any(len(v) > 1 for v in per.values()):
                raise NotImplementedError("apexw_amd: the grads of parameters of one dtype must share a dtype")
        for i, (p, st) in enumerate(zip(self.params, self.states)):
            if not p.is_contiguous():
                self._check_strided(i, p, st)
            f, block = self._tensor_flags(p, st, wd_on, self.grad_dtypes[i])
            if f & L.FLAG_FACTORED and self.grad_dtypes[i] != p.dtype:
                raise NotImplementedError("apexw_amd: factored_v with grads of another dtype than the parameter")
            tab[i]["p"] = p.data_ptr()
            tab[i]["m"] = st["exp_avg"].data_ptr()
            if f & L.FLAG_FACTORED:
                tab[i]["v"] = st["exp_avg_sq_row"].data_ptr()
                tab[i]["v_scale"] = st["exp_avg_sq_col"].data_ptr()
                if block:
                    tab[i]["m_scale"] = st["exp_avg_scales"].data_ptr()
            elif self.lion:
                tab[i]["v"] = st["exp_avg"].data_ptr()     # never read under APEXW_HP_LION
            else:
                tab[i]["v"] = st["exp_avg_sq"].data_ptr()
                if "exp_avg_scales" in st and st.get("is_8bit", False):
                    tab[i]["m_scale"] = st["exp_avg_scales"].data_ptr()
                    tab[i]["v_scale"] = st["exp_avg_sq_scales"].data_ptr()
                elif st.get("is_ultra", False):
                    tab[i]["m_scale"] = st["exp_avg_scales"].data_ptr()
            tab[i]["n"] = p.numel()
            tab[i]["flags"] = f
            tab[i]["block"] = block
            if self.kind == "compact":
                counts[i] = (p.numel() + L.COMPACT_UNIT - 1) // L.COMPACT_UNIT
            else:
                counts[i] = (p.numel() + block - 1) // block
        self.host_table = tab          # parameter order
        self.factored = (tab["flags"] & np.uint32(L.FLAG_FACTORED)) != 0
        self.max_v_ptrs = self.d_max_v = None
        if self.amsgrad:
            self.max_v_ptrs = np.zeros(n, dtype=np.uint64)
            for i, (p, st) in enumerate(zip(self.params, self.states)):
                mx, v = st.get("max_exp_avg_sq"), st.get("exp_avg_sq")
                if (mx is None or v is None or tab[i]["flags"] & (L.FLAG_QUAD | L.FLAG_FACTORED)
                        or mx.numel() != p.numel() or mx.dtype != v.dtype or mx.stride() != p.stride()
                        or mx.device != p.device):
                    raise NotImplementedError(f"apexw_amd: amsgrad state of tensor {i} ({tuple(p.shape)}): "
                                              "max_exp_avg_sq must be a contiguous full-size tensor in v's dtype")
                self.max_v_ptrs[i] = mx.data_ptr()
        self.slow_ptrs = self.d_slow = None
        if self.slow:
            self.slow_ptrs = np.zeros(n, dtype=np.uint64)
            for i, (p, st) in enumerate(zip(self.params, self.states)):
                ms, m = st.get("exp_avg_slow"), st["exp_avg"]
                if (ms is None or tab[i]["flags"] & (L.FLAG_QUAD | L.FLAG_FACTORED) or ms.numel() != p.numel()
                        or ms.dtype != m.dtype or ms.stride() != p.stride() or ms.device != p.device):
                    raise NotImplementedError(f"apexw_amd: beta3 state of tensor {i} ({tuple(p.shape)}): "
                                              "exp_avg_slow must be a contiguous full-size tensor in m's dtype")
                self.slow_ptrs[i] = ms.data_ptr()
        # per tensor {scale_v, sqrt(scale_v)} of this launch, for rows flagged APEXW_FLAG_VSCALE
        self.vscaled = (tab["flags"] & np.uint32(L.FLAG_VSCALE)) != 0
        self.d_vscale = self.h_vscale = None
        if self.vscaled.any():
            self.d_vscale = torch.ones((n, 2), dtype=torch.float32, device=self.device)
            self.h_vscale = np.ones((n, 2), dtype=np.float32)
            base = self.d_vscale.data_ptr()
            tab["v_scale"] = np.where(self.vscaled, np.arange(n, dtype=np.uint64) * np.uint64(8) + np.uint64(base),
                                      tab["v_scale"])
        self._sg_scale = {}
        self.fv = None
        self._fv_subsets = {}
        self.p_ptrs = np.zeros(n, dtype=np.uint64)
        self.p_dtypes = np.zeros(n, dtype=np.int8)
        self._H = _host()
        self._H.snapshot(self.params, self.p_ptrs.ctypes.data, self.p_dtypes.ctypes.data)
        self.g_ptrs = np.zeros(n, dtype=np.uint64)     # grad pointers the table was built from
        self.g_scan = np.zeros(n, dtype=np.uint64)     # the scan's current grad pointers
        # the grad dtypes the table was built for (torch's codes, as the scan reads them)
        self.g_dtypes = np.zeros(n, dtype=np.int8)
        grads = [p.grad if p.grad is not None else p for p in self.params]
        g_seen = np.zeros(n, dtype=np.uint64)          # held by name: the snapshot writes into it
        self._H.snapshot(grads, g_seen.ctypes.data, self.g_dtypes.ctypes.data)
        # the arrays never move: their addresses are taken once
        self._scan_addrs = (self.p_ptrs.ctypes.data, self.p_dtypes.ctypes.data, self.g_ptrs.ctypes.data,
                            self.g_scan.ctypes.data, self.g_dtypes.ctypes.data)
        self._scan_status = None
        # centralization: folded into the step kernels and the clip (row means only: compact
        # descriptors hold them in m_scale / block, 8-bit and ultra ones in a side table)
        # unless the plan holds factored tensors, which read a prepared copy of the grads
        self.gc_fold = self.gc and not self.single and not self.factored.any()
        self.host_rows = self.d_rows = None
        if self.gc and not self.single:
            self._build_prep()
        self._fast_static = None
        self.counts = counts
        # the ultra precision's rows run on their own kernel (apexw_ultra_step)
        self.ultra = self.kind == "q8" and self.precision == "ultra"
        self.kind_code = (3 if self.single else 0) if self.kind == "compact" else (5 if self.ultra else 1)
        self._lib = L.load()
        self.clip_ws = None
        self.d_table = None
        self.perm = None

    def _build_prep(self):
        """The preparation table (sources filled per step) and its outputs: per
        centralized tensor the fp32 row means (folded path), or per tensor a
        prepared copy of the grad."""
        n = len(self.params)
        prep = np.zeros(n, dtype=L.GRAD_PREP_DTYPE)
        # the reference centralizes dim >= 2 grads over dims 1.. (optimizer.py:239-243)
        prep["row_len"] = [p.numel() // p.shape[0] if p.dim() >= 2 and p.numel() > 0 else 0 for p in self.params]
        prep["n"] = [p.numel() for p in self.params]
        prep["dtype"] = [_DT[gd] for gd in self.grad_dtypes]
        if self.gc_fold:
            self.gc_means = [torch.empty(max(p.numel() // int(prep["row_len"][i]), 1) if prep["row_len"][i] else 1,
                                         dtype=torch.float32, device=self.device)
                             for i, p in enumerate(self.params)]
            prep["out"] = [m.data_ptr() for m in self.gc_means]
            tab = self.host_table
            rows = prep["row_len"] > 0
            tab["flags"] = np.where(rows, tab["flags"] | np.uint32(L.FLAG_GC), tab["flags"])
            if self.kind == "compact":
                tab["m_scale"] = np.where(rows, prep["out"], tab["m_scale"])
                tab["block"] = np.where(rows, prep["row_len"].astype(np.uint32), tab["block"])
            else:
                # 8-bit / ultra descriptors keep their quantization scales and block: the row
                # means go to the launch's side table (hparams.rows, in device-table order)
                self.host_rows = np.zeros(n, dtype=L.ROW_MEANS_DTYPE)
                self.host_rows["means"] = np.where(rows, prep["out"], 0)
                self.host_rows["row_len"] = prep["row_len"]
        else:
            self.gc_out = [torch.empty(p.numel(), dtype=p.dtype, device=self.device) for p in self.params]
            prep["out"] = [o.data_ptr() for o in self.gc_out]
        self.host_prep = prep
        self.d_prep = None
        counts = []
        for i in range(n):
            row = prep[i:i + 1].copy()
            row["g"] = 256                 # stand-in source, checked for real at upload
            if self.gc_fold and not row["row_len"][0]:
                counts.append(0)          # no centralization: nothing to prepare
                continue
            k = int(L.load().apexw_grad_prep_units(row.ctypes.data))
            if k < 0:
                L.check(-k, f"grad preparation of tensor {i}")
            counts.append(k)
        counts = np.array(counts, dtype=np.int64)
        units = np.zeros(int(counts.sum()), dtype=L.UNIT_DTYPE)
        begin = np.concatenate([[0], np.cumsum(counts)])
        units["tensor"] = np.repeat(np.arange(n, dtype=np.uint32), counts)
        units["unit"] = (np.arange(len(units), dtype=np.int64) - np.repeat(begin[:-1], counts)).astype(np.uint32)
        self.n_prep_units = len(units)
        self.d_prep_units = _upload(units.view(np.uint8), self.device)

    def _prepare_grads(self, inv_scale, stream, amp_dyn=None):
        """Sanitize, unscale and centralize into the prepared-grad buffers, or (folded
        path) only the row means of the sanitized, unscaled grads.  amp_dyn: device
        scalars of a GradScaler step (the unscale factor is read there)."""
        flags = L.HP_SANITIZE | (L.HP_UNSCALE if inv_scale is not None else 0)
        fn = self._lib.apexw_grad_row_means if self.gc_fold else self._lib.apexw_grad_prepare
        st = fn(self.d_prep.data_ptr(), len(self.params), self.d_prep_units.data_ptr(), self.n_prep_units,
                1.0 if inv_scale is None else inv_scale, flags, amp_dyn, stream)
        L.check(st, "apexw_grad_row_means" if self.gc_fold else "apexw_grad_prepare")

    def _layout_units(self, fast):
        """Device table in launch order and its unit table.  8-bit: full-block-kernel
        tensors first (bf16, then fp32), then every other tensor."""
        n = len(self.params)
        if fast is None:
            perm, n_bf, n_f32 = np.arange(n), 0, 0
        else:
            is32 = np.array([p.dtype == torch.float32 for p in self.params], dtype=bool)
            fb, ff = fast & ~is32, fast & is32
            perm = np.concatenate([np.nonzero(fb)[0], np.nonzero(ff)[0], np.nonzero(~fast)[0]])
            n_bf, n_f32 = int(fb.sum()), int(ff.sum())
        counts = self.counts[perm]
        self.unit_begin = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
        total = int(self.unit_begin[-1])
        units = np.zeros(total, dtype=L.UNIT_DTYPE)
        units["tensor"] = np.repeat(np.arange(n, dtype=np.uint32), counts)
        units["unit"] = (np.arange(total, dtype=np.int64) - np.repeat(self.unit_begin[:-1], counts)).astype(np.uint32)
        self.n_units = total
        self._host_units = units
        self.n_fast_units = int(counts[:n_bf].sum())
        self.n_fast_f32_units = int(counts[n_bf:n_bf + n_f32].sum())
        self.unit_counts = counts
        self.perm = perm
        self.fast = fast
        self.d_units = _upload(units.view(np.uint8), self.device)
        if self.max_v_ptrs is not None:
            # hparams.max_v: one pointer per descriptor, in device-table order
            self.d_max_v = _upload(np.ascontiguousarray(self.max_v_ptrs[perm]), self.device)
        if self.slow_ptrs is not None:
            self.d_slow = _upload(np.ascontiguousarray(self.slow_ptrs[perm]), self.device)
        self.d_unit_begin = _upload(self.unit_begin, self.device)
        # the step kernels' units: all but the factored rows' (apexw_factored_step steps
        # those; the clip's norm pass still covers every unit).  Factored tensors are
        # never full-block 8-bit tensors, so the fast prefix is unchanged.
        fac_rows = self.factored[perm]
        if fac_rows.any():
            self._step_keep = ~fac_rows[units["tensor"]]
            step_units = units[self._step_keep]
            self.n_step_units = len(step_units)
            self.d_step_units = _upload(step_units.view(np.uint8), self.device) \
                if len(step_units) else self.d_units
        else:
            self._step_keep, self.n_step_units, self.d_step_units = None, total, self.d_units
        self.clip_ws = None
        self._fv_subsets = {}
        self.fv = self._fv_layout(tuple(int(i) for i in np.nonzero(self.factored[perm])[0])) \
            if self.factored.any() else None

    def _fv_layout(self, rows):
        """Factored-v table, workspace and units for the device-table rows ``rows``."""
        fv = np.zeros(len(rows), dtype=L.FV_TENSOR_DTYPE)
        for k, d in enumerate(rows):
            p = self.params[int(self.perm[d])]
            fv[k]["tensor"] = d
            fv[k]["rows"] = p.shape[0]
            fv[k]["cols"] = p.numel() // p.shape[0]
            fv[k]["flags"] = L.FV_SUM_COLS if p.numel() > 262144 else 0
        nb, ncb = ctypes_int64(), ctypes_int64()
        ws = int(self._lib.apexw_factored_layout(fv.ctypes.data, len(fv), ctypes_ref(nb), ctypes_ref(ncb)))
        if ws < 0:
            L.check(-ws, "apexw_factored_layout")
        sel = np.isin(self._host_units["tensor"], np.array(rows, dtype=np.uint32))
        units = self._host_units[sel]
        # units grouped by (parameter dtype: bf16, fp32, fp16; m kind): each group runs on its own kernel
        tab = self.host_table[self.perm]
        pdt = (tab["flags"] >> L.PDT_SHIFT) & 3
        pk = np.where(pdt == L.F32, 1, np.where(pdt == L.F16, 2, 0)).astype(np.int64)
        mk = np.where(tab["block"] == 0, 2, np.where(tab["flags"] & L.FLAG_M6, 1, 0))
        group = (pk * 3 + mk)[units["tensor"]]
        order = np.argsort(group, kind="stable")
        units = np.ascontiguousarray(units[order])
        ends = np.cumsum(np.bincount(group, minlength=L.FV_UNIT_RANGES)).astype(np.int64)
        # the factored kernels address a unit's tensor through its fv entry (rows ascend)
        units["tensor"] = np.searchsorted(fv["tensor"], units["tensor"]).astype(np.uint32)
        return dict(rows=rows, n=len(fv), d_fv=_upload(fv.view(np.uint8), self.device),
                    ws=torch.empty(max(ws, 1), dtype=torch.float32, device=self.device),
                    n_bands=nb.value, n_cb=ncb.value, n_units=len(units), range_ends=ends,
                    d_units=_upload(units.view(np.uint8), self.device) if len(units) else None)

    def _refresh_grads(self):
        """Point the table at this step's grads; re-upload it if any moved.

        Uses the scan done by ``valid_for`` (or scans now on a new plan).  Grads
        that are non-contiguous are copied contiguous; the copies are returned
        so the caller keeps them alive until the launch is enqueued."""
        st = self._scan_status if self._scan_status is not None else self._scan()
        self._scan_status = None
        if st == SCAN_SAME and self.d_table is not None:
            return None
        if st in (SCAN_MISSING, SCAN_REBUILT, SCAN_GRAD_DTYPE):
            raise RuntimeError("the step plan no longer matches its parameters or grads")
        keep = None
        if st == SCAN_SLOW:
            keep = list(map(_GRAD, self.params))
            for i, (p, g) in enumerate(zip(self.params, keep)):
                if g.dtype != self.grad_dtypes[i]:
                    raise RuntimeError("a grad's dtype changed under the step plan")
                if g.numel() != p.numel():
                    raise RuntimeError(f"grad of parameter {i} has {g.numel()} elements, the parameter {p.numel()}")
                if g.stride() != p.stride():
                    # the step walks memory in the parameter's layout: the grad is copied into it
                    keep[i] = torch.empty_like(p, dtype=g.dtype).copy_(g)
            self.g_scan[:] = [g.data_ptr() for g in keep]
        ptrs = self.g_scan.copy()
        self.g_ptrs[:] = ptrs
        if self.gc and not self.single:
            # the prepared copies feed the clip and the step; the sources feed the preparation
            if self.d_prep is None or not np.array_equal(ptrs, self.host_prep["g"]):
                self.host_prep["g"] = ptrs
                for i in range(len(self.params)):
                    if self.gc_fold:
                        if self.host_prep["row_len"][i]:
                            L.check(self._lib.apexw_check_row_means(self.host_prep[i:i + 1].ctypes.data),
                                    f"row means of tensor {i}")
                        continue
                    L.check(self._lib.apexw_check_grad_prep(self.host_prep[i:i + 1].ctypes.data),
                            f"grad preparation of tensor {i}")
                self.d_prep = _upload(self.host_prep.view(np.uint8), self.device)
            if not self.gc_fold:
                ptrs = np.fromiter((o.data_ptr() for o in self.gc_out), dtype=np.uint64, count=len(self.params))
        if self.d_table is None or not np.array_equal(ptrs, self.host_table["g"]):
            self.host_table["g"] = ptrs
            fast = self._validate_and_align()
            if self.perm is None or (fast is not None and not np.array_equal(fast, self.fast)):
                self._layout_units(fast)
            rows = np.ascontiguousarray(self.host_table[self.perm])
            self.d_table = _upload(rows.view(np.uint8), self.device)
            if self.host_rows is not None:
                self.d_rows = _upload(np.ascontiguousarray(self.host_rows[self.perm]).view(np.uint8), self.device)
        return keep

    def _validate_and_align(self):
        """Mark descriptors with an unaligned pointer element-wise; 8-bit: which take the full-block kernel.

        The C ABI validates every descriptor once per plan (dtypes, flags, block,
        pointers); later grad-pointer changes only move the alignment, which is
        recomputed for all rows at once."""
        tab = self.host_table
        scalar = ((tab["p"] | tab["g"] | tab["m"] | tab["v"]) & np.uint64(15)) != 0
        for extra in (self.max_v_ptrs, self.slow_ptrs):
            if extra is not None:
                scalar |= (extra & np.uint64(15)) != 0
        if self.kind == "q8":
            scalar |= (tab["block"] % 8) != 0
        bit = np.uint32(L.FLAG_SCALAR)
        tab["flags"] = np.where(scalar, tab["flags"] | bit, tab["flags"] & ~bit)
        if self._fast_static is None:
            lib = self._lib
            fast_static = np.zeros(len(self.params), dtype=bool)
            for i in range(len(self.params)):
                row = tab[i]
                t = L.Tensor(*(int(row[k]) for k in ("p", "g", "m", "v", "m_scale", "v_scale", "n", "flags", "block")))
                L.check(lib.apexw_check_tensor(ctypes_ref(t), 4 if self.factored[i] else self.kind_code),
                        f"tensor {i} ({tuple(self.params[i].shape)})")
                if self.kind == "q8" and not self.single and not self.ultra and not self.factored[i]:
                    # full-block eligibility apart from alignment: same descriptor on aligned stand-in pointers
                    t.p = t.g = t.m = t.v = 256
                    t.flags = int(row["flags"]) & ~L.FLAG_SCALAR
                    fast_static[i] = lib.apexw_check_tensor(ctypes_ref(t), 2) == 0
            self._fast_static = fast_static
        return (self._fast_static & ~scalar) if self.kind == "q8" and not self.single else None

    # ------------------------------------------------------------------ launch
    def _clip_buffers(self):
        if self.clip_ws is None:
            self.clip_ws = (torch.empty(max(self.n_units, 1), dtype=torch.float32, device=self.device),
                            torch.empty(len(self.params), dtype=torch.float32, device=self.device),
                            torch.empty(1, dtype=torch.float32, device=self.device))
        return self.clip_ws

    def _clip(self, clip, sanitize, inv_scale, stream, amp_dyn=None):
        part, norms, coef = self._clip_buffers()
        unit = L.COMPACT_UNIT if self.kind == "compact" else 0
        st = self._lib.apexw_grad_clip_coef(
            self.d_table.data_ptr(), len(self.params), self.d_units.data_ptr(), self.n_units, unit,
            self.d_unit_begin.data_ptr(), part.data_ptr(), norms.data_ptr(), float(clip),
            1.0 if inv_scale is None else inv_scale,
            (L.HP_SANITIZE if sanitize else 0) | (L.HP_UNSCALE if inv_scale is not None else 0), coef.data_ptr(),
            amp_dyn, self.d_rows.data_ptr() if self.d_rows is not None else None, stream)
        L.check(st, "apexw_grad_clip_coef")
        return coef

    # ------------------------------------------------------------------ AMP on the device
    @property
    def amp_device_ok(self):
        """Whether GradScaler's scale and found_inf can be read on the device for this
        plan (the compact and 8-bit step kernels; not the factored ones or the
        in-backward batches)."""
        # a prepared copy of the grads (8-bit / factored groups that centralize) is unscaled
        # by apexw_grad_prepare and the step launches then carry no AMP scalars, so they
        # could not skip an inf / NaN step: such plans read found_inf on the host
        return not (self.hooked or self.single or self.factored.any() or self.vscaled.any()
                    or (self.gc and not self.gc_fold) or self.maximize
                    or (self.kind == "compact" and self.nesterov) or self.slow)

    def amp_fold(self, sync=False):
        """Subtract from the step counters the steps GradScaler skipped that the host
        has seen (the device's skip count, copied back asynchronously after each
        step).  sync: wait for the copies first, so every skip is folded."""
        if getattr(self, "_amp_skips", None) is None:
            return
        if sync:
            self._amp_event.synchronize()
            self.amp_dirty = False
        seen = int(self._amp_mirror.numpy()[0])
        if seen > self._amp_folded:
            self._steps_np -= float(seen - self._amp_folded)
            self._amp_folded = seen

    def _amp_buffers(self):
        """The device-side AMP scalars' buffers (allocated once); returns their address."""
        if getattr(self, "_amp_skips", None) is None:
            self._amp_skips = torch.zeros(1, dtype=torch.int32, device=self.device)
            self._amp_mirror = torch.zeros(1, dtype=torch.int32, pin_memory=True)
            self._amp_dyn = torch.empty(L.AMP_MAX_LAUNCHES * L.AMP_DYN_BYTES // 4, dtype=torch.float32,
                                        device=self.device)
            self._amp_folded = 0
            self._amp_event = torch.cuda.Event()
        return self._amp_dyn.data_ptr()

    def _amp_prepare(self, amp, groups, lr, b1, b2, eps, stream):
        """Device-side scalars of every launch of this step (apexw_amp_prepare)."""
        self._amp_buffers()
        launches = np.zeros(len(groups), dtype=L.AMP_LAUNCH_DTYPE)
        launches["lr"], launches["beta1"], launches["beta2"], launches["eps"] = lr, b1, b2, eps
        launches["step"] = [g[1] for g in groups]
        launches["kind"] = 1 if self.native else 0
        scale, found_inf = amp
        L.check(self._lib.apexw_amp_prepare(found_inf.data_ptr(), scale.data_ptr(), self._amp_skips.data_ptr(),
                                            self._amp_folded, launches.ctypes.data, len(groups),
                                            self._amp_dyn.data_ptr(), stream), "apexw_amp_prepare")
        self._amp_mirror.copy_(self._amp_skips, non_blocking=True)
        self._amp_event.record(torch.cuda.current_stream(self.device))
        self.amp_dirty = True
        return self._amp_dyn.data_ptr()

    # ------------------------------------------------------------------ fp16 v scales
    def _subgroups(self, key_fn):
        """The plan's non-factored tensors grouped by key_fn(i), in parameter order."""
        out = {}
        for i in range(len(self.params)):
            if not self.factored[i]:
                out.setdefault(key_fn(i), []).append(i)
        return out

    def _rescale_v(self, idx, cur_scale):
        """Every-100-steps recalibration of a subgroup's v (optimizer.py:5622-5645,
        :1165-1178): read max(v) on the host, as the reference does, and scale v
        by 4 or 1/4 in place.  Returns the factor."""
        vs = [self.states[i]["exp_avg_sq"] for i in idx]
        v_max = float(torch.stack([v.max().float() for v in vs]).max().item())
        factor = 1.0
        if v_max < 0.25 and cur_scale < 65536.0:
            factor = 4.0
        elif v_max > 16384.0 and cur_scale > 1.0:
            factor = 0.25
        if factor != 1.0:
            torch._foreach_mul_(vs, factor)
        return factor

    def _update_vscales(self, group, cold):
        """Each tensor's v scale for this launch, as the reference picks it.

        Cold step (_multi_tensor_step, optimizer.py:5600-5645): per subgroup of
        (p dtype, m dtype, step count, quad), the first parameter's state scale when
        m is fp16, recalibrated on every 100th step and written to every state of the
        subgroup.  Replay (execute_foreach, :1165-1199): per subgroup of (p dtype,
        16-bit m, quad), fp16 v is recalibrated every 100 steps with the subgroup's
        remembered scale, and the step takes the first parameter's state scale,
        which the replay itself never changes."""
        dyn = bool(group.get("dynamic_scaling", True))
        st, steps = self.states, self._steps_np
        h = np.ones_like(self.h_vscale)
        quad = (self.host_table["flags"] & np.uint32(L.FLAG_QUAD)) != 0
        if cold:
            subs = self._subgroups(lambda i: (self.params[i].dtype, st[i]["exp_avg"].dtype, int(steps[i]),
                                              bool(quad[i])))
            for (_, mdt, step, _), idx in subs.items():
                if not (dyn and mdt == torch.float16):
                    continue
                scale = float(st[idx[0]]["scale_v"])
                sqrt_scale = float(st[idx[0]].get("sqrt_scale_v", math.sqrt(scale)))
                if step > 1 and step % 100 == 0:
                    f = self._rescale_v(idx, scale)
                    if f != 1.0:
                        scale *= f
                        sqrt_scale = math.sqrt(scale)
                        for i in idx:
                            st[i]["scale_v"], st[i]["sqrt_scale_v"] = scale, sqrt_scale
                h[idx] = (scale, sqrt_scale)
        else:
            subs = self._subgroups(lambda i: (self.params[i].dtype, st[i]["exp_avg"].dtype != torch.float32,
                                              bool(quad[i])))
            step = int(steps[0])
            if dyn and step > 1 and step % 100 == 0:
                for key, idx in subs.items():
                    if st[idx[0]]["exp_avg_sq"].dtype == torch.float16:
                        self._rescale_v(idx, self._sg_scale.get(key, 1.0))
            for key, idx in subs.items():
                scale = float(st[idx[0]].get("scale_v", self._sg_scale.get(key, 1.0)))
                sqrt_scale = float(st[idx[0]].get("sqrt_scale_v", math.sqrt(scale)))
                self._sg_scale[key] = scale
                h[idx] = (scale, sqrt_scale)
        if not np.array_equal(h, self.h_vscale):
            self.h_vscale = h
            self.d_vscale.copy_(torch.from_numpy(h).pin_memory(), non_blocking=True)

    def execute(self, group, seed, inv_scale=None, lr=None, wd=None, steps=None, amp=None):
        """Run one optimizer step for the group (cold the first time, replay after):
        prepare() then run().  Arguments as prepare()."""
        prog = self.prepare(group, seed, inv_scale, lr, wd, steps, amp)
        if prog is None:
            raise L.ApexwError("device-side AMP is unavailable for this step; pass the host-read scale")
        prog.run()

    def prepare(self, group, seed, inv_scale=None, lr=None, wd=None, steps=None, amp=None):
        """Everything of one step up to its first device launch: the grads are
        re-pointed, the step counters advanced, each launch's scalars built and
        checked by the library (apexw_check_launch, the checks every step entry
        point runs before it enqueues).  Nothing the caller can see changes on the
        device here, and a refusal restores the counters, so a caller that prepares
        every group before running any refuses a whole step before any parameter
        moves -- the reference's validate-before-mutate order and step-counter
        rollback around its fused launches (apexw/optimizer.py:3184-3356, :3806).

        inv_scale: 1 / the AMP grad scale handed over by GradScaler, or None.
        amp: instead, GradScaler's (scale, found_inf) device tensors, read on the
        device (amp_device_ok plans): the kernels unscale with 1 / scale and skip
        the step when found_inf is set; the step counters advance on the host and
        the skips are subtracted once seen (amp_fold).  Returns None, with the
        counters untouched, when this step needs more launches than the device-side
        AMP table holds (APEXW_AMP_MAX_LAUNCHES); the caller then reads the scale on
        the host.
        lr, wd: replace the group's values; steps: each parameter's step count
        for this step (already advanced) instead of advancing the plan's own.
        Returns a _Program whose run() enqueues the step and rollback() undoes the
        counters."""
        if amp is not None:
            self.amp_fold()
        saved = self._steps_np.copy()
        try:
            prog = self._prepare(group, seed, inv_scale, lr, wd, steps, amp)
        except BaseException:
            self._steps_np[:] = saved
            raise
        if prog is None:
            self._steps_np[:] = saved
            return None
        prog.saved = saved
        return prog

    def _prepare(self, group, seed, inv_scale, lr, wd, steps, amp):
        mode_cold = not self.cold_done
        if self.cautious and self.d_counts is None:
            self.d_counts = torch.zeros(len(self.params), dtype=torch.int64, device=self.device)
        # the in-backward flush steps without nesterov whatever the group says (optimizer.py:2358)
        self._nesterov = bool(group.get("nesterov", False)) and not (self.single or self.hooked)
        # beta3's value and alpha are read from the group each step, as the reference's step does
        if self.slow:
            self.beta3, self.alpha = group["beta3"], float(group.get("alpha", 5.0))
        keep = self._refresh_grads()      # contiguous copies of non-contiguous grads, alive until the launch
        if amp is not None:
            inv_scale = 1.0          # a stand-in: the kernels read the factor from the device scalars
        elif self.maximize:
            # maximize: g -> -g, through the unscale factor (exact, and it commutes with
            # nan_to_num, the clip, centralization and AMP's unscale: optimizer.py:4502-4503,
            # :1104-1105, :5515-5517)
            inv_scale = -(1.0 if inv_scale is None else inv_scale)
        (b1, b2), eps = group["betas"], group["eps"]
        lr = group["lr"] if lr is None else lr
        wd = group["weight_decay"] if wd is None else wd
        sr = bool(group.get("stochastic_rounding", True))
        clip = group.get("clip_grad_norm", None)
        if self.kind == "compact":
            sanitize = mode_cold or clip is not None
        else:
            sanitize = mode_cold and clip is not None
        if self.single:
            # the per-parameter update takes the grads as they are (no sanitize, clip, AMP or centralization)
            sanitize, clip, inv_scale, amp = False, None, None, None
        if steps is None:
            self._steps_np += 1.0
        else:
            self._steps_np[:] = np.asarray(steps, dtype=np.float32)
        # The reference's replayed compact step takes the bias correction of the
        # first counter for the whole group (optimizer.py:1082-1090); every other
        # path uses each parameter's own count.  SR: the 8-bit step and the
        # per-parameter update read each parameter's state flag (optimizer.py:4377,
        # :2419), the compact step and the in-backward batches the group's (:3789,
        # :4004, :2286).
        sr_t = self._state_sr() if self.kind == "q8" and (self.single or not self.hooked) else None
        if mode_cold or self.native or self.kind == "q8":
            groups = self._split_launches(sr_t, sr)
        else:
            groups = [(None, int(self._steps_np[0]), sr)]
        if amp is not None and len(groups) > L.AMP_MAX_LAUNCHES:
            return None
        amp_dyn = self._amp_buffers() if amp is not None else None
        prep = None
        if self.single:
            pass
        elif self.gc_fold:
            # _prepare_grads with centralization, folded: the row means first; the clip
            # and the step read the raw grads and sanitize, unscale and subtract them
            prep = (inv_scale, amp_dyn)
            sanitize = True
        elif self.gc:
            # _prepare_grads with centralization: sanitize, unscale, centralize;
            # the clip and the step then see finite, unscaled grads
            prep = (inv_scale, amp_dyn)
            sanitize, inv_scale, amp_dyn = False, None, None
        coef = None
        if clip is not None:
            coef = self._clip_buffers()[2]
        launch_kind = L.LAUNCH_COMPACT if self.kind == "compact" else (L.LAUNCH_ULTRA if self.ultra else L.LAUNCH_Q8)
        launches = []
        for li, (units, step, sr_l) in enumerate(groups):
            hp = self._hparams(lr, b1, b2, eps, wd, step, sr_l, sanitize, coef, seed, mode_cold, inv_scale)
            if amp_dyn is not None:
                hp.flags |= L.HP_AMP
                hp.amp = amp_dyn + li * L.AMP_DYN_BYTES
            if units is None:
                d_units, n_units = self.d_step_units, self.n_step_units
                n_fast, n_fast32 = self.n_fast_units, self.n_fast_f32_units
            else:
                d_units, n_units, n_fast, n_fast32 = units
            if n_units == 0:
                continue
            if self.kind == "compact" or self.ultra:
                n_fast = n_fast32 = 0
            L.check(self._lib.apexw_check_launch(launch_kind, len(self.params), n_units, n_fast, n_fast32,
                                                 ctypes_ref(hp)), "apexw step")
            launches.append((d_units, n_units, n_fast, n_fast32, hp))
        if self.cautious and launches:
            L.check(self._lib.apexw_check_launch(L.LAUNCH_CAUTIOUS, len(self.params), self.n_units, 0, 0,
                                                 ctypes_ref(launches[0][4])), "cautious count")
        fv_launches = []
        if self.fv is not None:
            replay_step = None if (mode_cold or self.native or self.kind == "q8") else groups[0][1]
            fv_launches = self._factored_launches(lr, b1, b2, eps, wd, sanitize, coef, seed, mode_cold, inv_scale,
                                                  replay_step)
        return _Program(self, group=group, mode_cold=mode_cold, keep=keep, amp=amp, amp_groups=groups,
                        amp_scalars=(lr, b1, b2, eps), prep=prep, clip=clip, sanitize=sanitize,
                        inv_scale=inv_scale, amp_dyn=amp_dyn, launches=launches, fv_launches=fv_launches)

    def _run(self, prog):
        """Enqueue one prepared step (prepare())."""
        stream = torch.cuda.current_stream(self.device).cuda_stream
        if self.h_vscale is not None:
            self._update_vscales(prog.group, prog.mode_cold)
        if prog.amp is not None:
            lr, b1, b2, eps = prog.amp_scalars
            self._amp_prepare(prog.amp, prog.amp_groups, lr, b1, b2, eps, stream)
        if prog.prep is not None:
            self._prepare_grads(prog.prep[0], stream, prog.prep[1])
        if prog.clip is not None:
            self._clip(prog.clip, prog.sanitize, prog.inv_scale, stream, prog.amp_dyn)
        table = self.d_table.data_ptr()
        if self.cautious and prog.launches:
            # the mask counts of every tensor, from the grads as prepared above (clip,
            # centralization, AMP), before any launch updates a moment
            count = (self._lib.apexw_compact_cautious_count if self.kind == "compact"
                     else self._lib.apexw_q8_cautious_count)
            L.check(count(table, len(self.params), self.d_units.data_ptr(), self.n_units,
                          ctypes_ref(prog.launches[0][4]), stream), "cautious count")
        for d_units, n_units, n_fast, n_fast32, hp in prog.launches:
            if self.kind == "compact":
                st = self._lib.apexw_compact_step(table, len(self.params), d_units.data_ptr(), n_units,
                                                  ctypes_ref(hp), stream)
            elif self.ultra:
                st = self._lib.apexw_ultra_step(table, len(self.params), d_units.data_ptr(), n_units,
                                                ctypes_ref(hp), stream)
            else:
                st = self._lib.apexw_q8_step(table, len(self.params), d_units.data_ptr(), n_units, n_fast, n_fast32,
                                             ctypes_ref(hp), stream)
            L.check(st, "apexw step")
        for fv, hp in prog.fv_launches:
            st = self._lib.apexw_factored_step(
                table, len(self.params), fv["d_fv"].data_ptr(), fv["n"], fv["n_bands"],
                fv["n_cb"], fv["d_units"].data_ptr() if fv["d_units"] is not None else None, fv["n_units"],
                fv["range_ends"].ctypes.data, fv["ws"].data_ptr(), ctypes_ref(hp), stream)
            L.check(st, "apexw_factored_step")
        self.cold_done = True

    def _state_sr(self):
        return np.fromiter((bool(st.get("stochastic_rounding", True)) for st in self.states), dtype=bool,
                           count=len(self.states))

    def _factored_launches(self, lr, b1, b2, eps, wd, sanitize, coef, seed, cold, inv_scale, replay_step):
        """The factored-v rows' launches, checked: one apexw_factored_step per distinct
        (step count, SR flag).  The replayed compact plan uses its first counter for
        every tensor (optimizer.py:1141-1163); SR follows each parameter's state flag
        (_apply_factored_v_int8_update's callers, optimizer.py:5426, :4377).
        Returns [(layout, hparams)]."""
        rows = self.fv["rows"]
        vals = self.steps.numpy()[self.perm]
        srs = self._state_sr()[self.perm]
        buckets = {}
        for d in rows:
            key = (replay_step if replay_step is not None else int(vals[d]), bool(srs[d]))
            buckets.setdefault(key, []).append(d)
        out = []
        for (step, sr), members in buckets.items():
            if len(members) == len(rows):
                fv = self.fv
            else:
                key = tuple(members)
                fv = self._fv_subsets.get(key)
                if fv is None:
                    fv = self._fv_subsets[key] = self._fv_layout(key)
            hp = self._hparams(lr, b1, b2, eps, wd, step, sr, sanitize, coef, seed, cold, inv_scale)
            hp.mode = L.MODE_COLD
            hp.eps = eps
            hp.wd_factor = max(1.0 - lr * wd, 0.0) if wd != 0 else 1.0
            # nan_to_num on the fp32 grad: always in the 8-bit step, on the cold compact step
            # (_apply_factored_v_int8_update's sanitize_g, optimizer.py:4380-4400, :5414-5432, :1147-1163)
            if self.kind == "q8" or cold:
                hp.flags |= L.HP_FV_SANITIZE
            L.check(self._lib.apexw_check_launch(L.LAUNCH_FACTORED, len(self.params), fv["n_units"], 0, 0,
                                                 ctypes_ref(hp)), "apexw_factored_step")
            out.append((fv, hp))
        return out

    def _split_launches(self, sr_t, sr_default):
        """Step-kernel launches as (units or None for all, step count, SR): one per
        distinct (step count, SR flag) among the plan's tensors.  sr_t: each
        parameter's SR flag, or None when the group's flag applies to all."""
        raw = self._steps_np
        sr_uniform = sr_t is None or bool(sr_t.all()) or not bool(sr_t.any())
        sr0 = sr_default if sr_t is None else bool(sr_t[0])
        if ((raw.size == 1 or raw.min() == raw.max()) and sr_uniform) or self.n_step_units == 0:
            # one launch (or none: every tensor is factored and apexw_factored_step
            # buckets those itself)
            return [(None, int(raw[0]), sr0)]
        vals = raw[self.perm]
        srp = np.full(len(vals), sr_default, dtype=bool) if sr_t is None else sr_t[self.perm]
        keys = list(zip(vals.tolist(), srp.tolist()))
        out = []
        for val, srv in sorted(set(keys), key=keys.index):
            keep = (vals == val) & (srp == srv)
            mask = np.repeat(keep, self.unit_counts)
            if self._step_keep is not None:
                mask = mask[self._step_keep]
            if not mask.any():
                continue
            idx = _upload(np.flatnonzero(mask), self.device)
            sel = self.d_step_units.view(-1, 8).index_select(0, idx).reshape(-1)
            nb, nf = self.n_fast_units, self.n_fast_f32_units
            out.append(((sel, int(mask.sum()), int(mask[:nb].sum()), int(mask[nb:nb + nf].sum())), int(val),
                        bool(srv)))
        return out

    def _hparams(self, lr, b1, b2, eps, wd, step, sr, sanitize, coef, seed, cold, inv_scale=None):
        hp = L.HParams()
        bc1 = 1.0 - b1 ** step
        bc2 = 1.0 - b2 ** step
        bc2s = math.sqrt(bc2)
        hp.beta1, hp.one_minus_beta1 = b1, 1.0 - b1
        hp.beta2, hp.one_minus_beta2 = b2, 1.0 - b2
        flags = 0
        if self.single:
            # _step_single_param_fused's scalars (apexw/optimizer.py:2395-2407)
            hp.wd_factor = max(1.0 - lr * wd, 0.0) if wd != 0 else 1.0
            hp.step_size = lr * bc2s / bc1
            hp.eps_scaled = eps * bc2s
            hp.eps = eps
            hp.gain_hi = 1.0 + 0.20 * b1
            hp.gain_lo = 1.0 - 0.35 * b1
            hp.mode = L.MODE_SINGLE
            hp.seed = seed
            hp.step = step & 0xFFFFFFFF
            hp.flags = L.HP_SR if (sr and self.kind == "q8") else 0
            return hp
        if self.kind == "q8":
            hp.wd_factor = max(1.0 - lr * wd, 0.0) if wd != 0 else 1.0
            hp.step_size = lr * bc2s / bc1
            hp.eps_scaled = eps * bc2s
            hp.eps = eps
            if self._nesterov:
                # nesterov: num = lerp(g, m, beta1) with no SNR gain (optimizer.py:4581-4583,
                # :4444-4445): the blocks multiply by a gain of exactly 1, the dense and
                # ultra rows take the lookahead instead of m
                hp.gain_hi = hp.gain_lo = 1.0
                flags |= L.HP_NESTEROV
            elif self.cautious:
                # cautious: num = m' (no lookahead) times the mask over its mean
                # (optimizer.py:4583-4588); the kernels take each tensor's gains from its count
                hp.gain_hi, hp.gain_lo = 1.0, 0.0
                flags |= L.HP_CAUTIOUS
                hp.counts = self.d_counts.data_ptr()
            else:
                hp.gain_hi = 1.0 + 0.20 * b1
                hp.gain_lo = 1.0 - 0.35 * b1
            hp.mode = L.MODE_COLD if cold else L.MODE_REPLAY
            if sr:
                flags |= L.HP_SR
        elif self.native:
            hp.wd_factor = 1.0 - lr * wd
            hp.step_size = lr / bc1
            hp.bc2_sqrt = bc2s
            hp.eps = eps
            hp.mode = L.MODE_NATIVE
        else:
            hp.wd_factor = 1.0 - lr * wd
            hp.step_size = lr * bc2s / bc1
            hp.eps_scaled = eps * bc2s
            hp.eps = eps                   # the replay's denominator floor with fp16 in the subgroup
            hp.mode = L.MODE_COLD if cold else L.MODE_REPLAY
            if sr and not self.lion:
                flags |= L.HP_SR
                if b2 >= 0.995:
                    flags |= L.HP_SR_V
            if self.lion:
                # lion (optimizer.py:5677-5683, :1214-1225): the sign update with -lr, m
                # toward g with weight 1 - beta2 (lerp_coef below); no SR
                flags |= L.HP_LION
                hp.gain_hi = lr
            elif self.cautious:
                # cautious (optimizer.py:5847-5864, :1321-1328): m times the mask over its mean,
                # the counts from apexw_compact_cautious_count
                flags |= L.HP_CAUTIOUS
                hp.counts = self.d_counts.data_ptr()
            elif self._nesterov and not self.slow:
                # nesterov (optimizer.py:5865-5877, :1329-1331): p += (-step_size*b1) m / d, then
                # p += (-step_size*(1-b1)) g / d, the Python products taken to fp32 by torch;
                # quad tensors take lerp(g, m, b1) as the numerator (look_coef below)
                hp.gain_hi = -(lr * bc2s / bc1) * b1
                hp.gain_lo = -(lr * bc2s / bc1) * (1.0 - b1)
                flags |= L.HP_NESTEROV
        hp.lerp_coef, hi = _lerp_coef(1.0 - (b2 if flags & L.HP_LION else b1))
        if hi:
            flags |= L.HP_LERP_HI
        hp.look_coef, hi = _lerp_coef(b1)
        if hi:
            flags |= L.HP_LOOK_HI
        if flags & L.HP_CAUTIOUS:
            # lerp(g, m', b1) with coefficient 0 in the end-based form is m' itself
            hp.look_coef = 0.0
            flags |= L.HP_LOOK_HI
        if sanitize:
            flags |= L.HP_SANITIZE
        if coef is not None:
            flags |= L.HP_CLIP
            hp.clip_coef = coef.data_ptr()
        if inv_scale is not None:
            flags |= L.HP_UNSCALE
            hp.grad_inv_scale = inv_scale
        if self.d_rows is not None:
            hp.rows = self.d_rows.data_ptr()
        if self.mixed:
            # grads of another dtype than their parameters: the variant instantiation reads them
            flags |= L.HP_GRAD_DTYPES
        if self.amsgrad:
            # amsgrad: the denominators take max(max_v, v) (optimizer.py:5788-5790, :1253-1255;
            # torch._fused_adamw_ for the native plan)
            flags |= L.HP_AMSGRAD
            hp.max_v = self.d_max_v.data_ptr()
        if self.slow:
            # beta3 (AdEMAMix): the slow moment's EMA and its weight alpha (1 - b1^t) / (1 - b3^t)
            # in double, as the reference's (optimizer.py:5584, :1101); nesterov does not apply
            b3 = float(self.beta3)
            flags |= L.HP_SLOW
            hp.slow = self.d_slow.data_ptr()
            hp.beta3, hp.one_minus_beta3 = b3, 1.0 - b3
            hp.lerp3_coef, hi = _lerp_coef(1.0 - b3)
            if hi:
                flags |= L.HP_LERP3_HI
            hp.slow_ratio = self.alpha * ((1.0 - b1 ** step) / (1.0 - b3 ** step))
        hp.seed = seed
        hp.step = step & 0xFFFFFFFF
        hp.flags = flags
        return hp


class _Program:
    """One prepared step of a StepPlan: run() enqueues it, rollback() restores the
    step counters it advanced (when a later group of the same step is refused)."""

    def __init__(self, plan, **kw):
        self.plan = plan
        self.saved = None
        self.__dict__.update(kw)

    def run(self):
        try:
            self.plan._run(self)
        except BaseException:
            self.rollback()
            raise

    def rollback(self):
        if self.saved is not None:
            self.plan._steps_np[:] = self.saved


def ctypes_ref(obj):
    import ctypes
    return ctypes.byref(obj)


def ctypes_int64():
    import ctypes
    return ctypes.c_int64(0)
