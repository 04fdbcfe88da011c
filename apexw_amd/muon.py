"""ApexMuon: momentum + Newton-Schulz orthogonalised updates on the GPU.

Drop-in for the reference ``apexw.muon.ApexMuon`` (apexw/muon.py:344-861) for
the fp32-momentum configuration: same constructor, defaults, ``state`` keys
(``step``, ``work_dtype``, ``momentum``) and ``load_state_dict`` dtype
handling.  The step runs through libapexw_hip.so:

* ``apexw_muon_prepare``: fp32 momentum update, the bf16 work matrix (the
  wide orientation) normalised by its Frobenius norm;
* ``NSPlan``: per iteration three bf16 MFMA GEMMs
  (``A = X X^T``; ``B = c A A + b A``; ``X = B X + a X``), each one grouped
  launch (``apexw_gemm_nt_grouped``) over every Muon matrix of the step; the
  two symmetric products compute only the tiles on and above the diagonal;
* the last ``X`` product of each matrix applies the decoupled weight decay and
  ``p -= lr * scale * U`` in its epilogue (``APEXW_GEMM_APPLY``);
  ``apexw_muon_apply`` does it as a separate pass when ``ns_steps == 0``.

Like the reference on a bf16-capable GPU, the Newton-Schulz work dtype is
bf16 (apexw/muon.py:76-89).  Vectors and matrices with a dimension under 16
take the reference's coordinate-wise update (``apexw_muon_coordwise``);
non-contiguous parameters are stepped in a contiguous copy that is written
back.  Under GradScaler, found_inf and the scale are read by the kernels
(each takes the step's ``apexw_amp_dyn``): a skipped step writes nothing and
the host's step counters are corrected when ``state`` is next looked at.
Quantised momentum (precision "8bit"/"ultra"),
AdEMAMix (beta3), cautious masking, grad centralization, the Polar Express
coefficients and scale_mode="rms" raise ``NotImplementedError``.
"""

import functools
import math
from collections import defaultdict

import numpy as np
import torch
from torch.optim.optimizer import Optimizer

from . import runtime as R
from . import _lib
from . import state as S

NS_A, NS_B, NS_C = 3.4445, -4.7750, 2.0315   # apexw/muon.py:49-52
NS_EPS = 1e-7


def _dtype_code(dt):
    if dt == torch.float32:
        return _lib.F32
    if dt == torch.bfloat16:
        return _lib.BF16
    if dt == torch.float16:
        return _lib.F16
    raise NotImplementedError(f"ApexMuon: unsupported dtype {dt}")


def _pad(x, to):
    return (x + to - 1) // to * to


@functools.lru_cache(maxsize=1024)
def _round_to(dtype, x):
    """A Python scalar as torch's same-dtype foreach ops see it (rounded to dtype);
    cached, since a step asks for the same few values every time."""
    return float(torch.tensor(x, dtype=torch.float32).to(dtype).float()) if dtype != torch.float32 else x


def _to_panels(t):
    """A row-major [R x C] bf16 matrix (R, C multiples of 32) in 32 x 32 panels."""
    r, c = t.shape
    return t.view(r // 32, 32, c // 32, 32).transpose(1, 2).contiguous().view(r, c)


def _from_panels(t):
    """The row-major matrix of a [R x C] buffer stored in 32 x 32 panels."""
    r, c = t.shape
    return t.view(r // 32, c // 32, 32, 32).transpose(1, 2).contiguous().view(r, c)


class NSWorkspace:
    """bf16 Newton-Schulz buffers for `batch` matrices whose wide work shape is m x n.

    Dimensions are padded to the GEMM tile; the padding is zero and stays zero
    through every product.  X and its transpose X^T are kept for two iterations
    (ping-pong), plus the symmetric A and B: X' = B X + a X reads X^T as its [N x K]
    operand (direct fragment reads, measured 3% faster than X as [K x N] rows with
    transposing reads) and writes X' and X'^T.  The buffers hold their matrices in 32 x 32 panels
    (APEXW_GEMM_PANEL): each K stage of a product's operand is then whole
    128-byte lines, which the grouped GEMM reads with fewer L2 requests than
    the 64-byte row pieces of a row-major operand (panel=False keeps row-major).
    """

    def __init__(self, m, n, batch, device, panel=True):
        self.m, self.n, self.batch, self.device = m, n, batch, device
        self.panel = bool(panel)
        self.layout = _lib.LAYOUT_PANEL if self.panel else _lib.LAYOUT_ROWS
        t = _lib.GEMM_TILE
        self.mp, self.np_ = _pad(m, t), _pad(n, t)
        z = lambda *s: torch.zeros(*s, dtype=torch.bfloat16, device=device)  # noqa: E731
        self.x = [z(batch, self.mp, self.np_), z(batch, self.mp, self.np_)]
        self.xt = [z(batch, self.np_, self.mp), z(batch, self.np_, self.mp)]
        self.a = z(batch, self.mp, self.mp)
        self.b = z(batch, self.mp, self.mp)
        lib = _lib.load()
        per = int(lib.apexw_muon_workspace_floats(m, n))
        self.partial = torch.empty(batch, max(per, 1), dtype=torch.float32, device=device)

    def rows_of(self, buf):
        """One matrix of x, a or b as a row-major tensor (a copy when in panels)."""
        return _from_panels(buf) if self.panel else buf

    def in_layout(self, mat):
        """A row-major matrix of a buffer's padded shape in this workspace's layout."""
        return _to_panels(mat) if self.panel else mat


def _ns_problems(ws, phase, cur, out, tag=None, tags=None):
    """Append the GEMM problems of one Newton-Schulz product for every matrix of ws.

    phase 0: A = X X^T (symmetric); phase 1: B = c A A + b A (symmetric);
    phase 2: X' = B X + a X with X^T as the [N x K] operand, the addend a X taken
    from that same operand on the matrix cores, and X' written in both layouts.
    cur is the ping-pong slot holding the current X.  With tags, (tag, entry) is
    appended per row.
    """
    mp, np_ = ws.mp, ws.np_
    pf = _lib.GEMM_PANEL if ws.panel else 0
    for e in range(ws.batch):
        if tags is not None:
            tags.append((tag, e))
        x = ws.x[cur][e].data_ptr()
        a, b = ws.a[e].data_ptr(), ws.b[e].data_ptr()
        if phase == 0:
            out.append((x, x, 0, a, a, mp, mp, np_, np_, np_, 0, mp, mp, 1.0, 0.0, _lib.GEMM_SYM | pf, 0))
        elif phase == 1:
            out.append((a, a, a, b, b, mp, mp, mp, mp, mp, mp, mp, mp, NS_C, NS_B, _lib.GEMM_SYM | pf, 0))
        else:
            xt = ws.xt[cur][e].data_ptr()
            nx, nxt = ws.x[cur ^ 1][e].data_ptr(), ws.xt[cur ^ 1][e].data_ptr()
            out.append((b, xt, 0, nx, nxt, mp, np_, mp, mp, mp, 0, np_, mp, 1.0, NS_A, _lib.GEMM_ADD_B | pf, 0))


class NSPlan:
    """Newton-Schulz for every Muon matrix of a step on one device, as grouped launches.

    Iteration i runs three launches (A, B, X') over all workspaces that still
    have iterations left; each launch covers every matrix of every shape, so the
    GPU is filled by the whole step's work rather than one shape at a time.  The
    problem tables and tile schedules are built once and kept on the device
    (they hold the workspaces' addresses, which never change).

    A workspace's last X' product carries the parameter update
    (APEXW_GEMM_APPLY): its rows of the table are filled in at each run with
    the parameters' addresses and the step's scalars, validated, and uploaded
    ahead of the launch on the same stream.  Those rows write X' itself only
    when keep_result is set.
    """

    def __init__(self, wss, steps, device):
        # algorithmic FLOPs (the reference's three matmuls, unpadded) and the
        # FLOPs the kernels execute (padded; upper-triangle tiles of A and B)
        self.flops = sum(ws.batch * s * (4 * ws.m * ws.m * ws.n + 2 * ws.m ** 3) for ws, s in zip(wss, steps))
        self.exec_flops = 0
        for ws, s in zip(wss, steps):
            t = ws.mp // _lib.GEMM_TILE
            tri = (t + 1) / (2 * t)
            self.exec_flops += ws.batch * s * (tri * (2 * ws.mp ** 2 * ws.np_ + 2 * ws.mp ** 3) + 2 * ws.mp ** 2 * ws.np_)
        self.device = device
        self._applied = {}      # id(host table) -> (applies key, device table with the fused update)
        built = {}
        self.iters = []
        for i in range(max(steps, default=0)):
            active = tuple(j for j, s in enumerate(steps) if s > i)
            final = frozenset(j for j in active if steps[j] == i + 1)
            key = (active, final, i % 2)
            if key not in built:
                built[key] = [self._launches(wss, active, final if phase == 2 else (), phase, i % 2, device)
                              for phase in range(3)]
            self.iters.append(built[key])

    def _launches(self, wss, active, final, phase, cur, device):
        rows, tags = [], []
        for j in active:
            _ns_problems(wss[j], phase, cur, rows, j, tags)
        out = []
        for c0 in range(0, len(rows), _lib.GEMM_MAX_PROBLEMS):
            probs = _lib.gemm_problems(rows[c0:c0 + _lib.GEMM_MAX_PROBLEMS])
            # rows (index in this launch, workspace, entry) whose X' is the final update
            fin = [(r, j, e) for r, (j, e) in enumerate(tags[c0:c0 + _lib.GEMM_MAX_PROBLEMS]) if j in final]
            if fin and len(fin) == len(probs):
                # a launch of final products only: no iteration reads their X'^T (the
                # epilogue kind stays one per launch, so mixed launches keep writing it)
                probs["ct"], probs["ldct"] = 0, 0
            items, offsets, n_wg, kind = _lib.gemm_schedule(probs, _lib.cus_per_queue(device))
            to_dev = lambda a: torch.from_numpy(a.view(np.uint8).copy()).to(device)  # noqa: E731
            out.append((to_dev(probs), to_dev(items), to_dev(offsets), n_wg, kind, probs if fin else None, fin))
        return out

    def run(self, stream, applies=None, keep_result=True, amp=None):
        """Run every launch on `stream`.  applies[j][e] = (p, dtype code, rows, cols,
        transposed, apply_wd, wd_factor, neg_lr) for entry e of workspace j: that
        matrix's final X' updates p in its epilogue.  Without applies the final X'
        is only stored (keep_result is then implied)."""
        lib = _lib.load()
        key = None
        if applies is not None:
            key = (tuple(tuple(a) for a in applies), bool(keep_result))
        for phases in self.iters:
            for launches in phases:
                for probs, items, offsets, n_wg, kind, host, fin in launches:
                    if fin and applies is not None:
                        # the fused update's table changes only with the parameters' addresses
                        # or the step's scalars: reuse the last upload while they hold
                        hit = self._applied.get(id(host))
                        if hit is not None and hit[0] == key:
                            probs = hit[1]
                        else:
                            probs = self._upload_applies(lib, probs, host, fin, applies, keep_result)
                            self._applied[id(host)] = (key, probs)
                    _lib.check(lib.apexw_gemm_nt_grouped(probs.data_ptr(), items.data_ptr(), offsets.data_ptr(),
                                                         n_wg, kind, amp, stream), "apexw_gemm_nt_grouped")

    def _upload_applies(self, lib, dev_probs, host, fin, applies, keep_result):
        tbl = host.copy()
        for r, j, e in fin:
            p, dt, rows, cols, transposed, apply_wd, wd_factor, neg_lr = applies[j][e]
            tbl["flags"][r] |= (_lib.GEMM_APPLY | (_lib.GEMM_APPLY_T if transposed else 0)
                                | (_lib.GEMM_APPLY_WD if apply_wd else 0))
            tbl["p"][r], tbl["p_dtype"][r], tbl["p_rows"][r], tbl["p_cols"][r] = p, dt, rows, cols
            tbl["wd_factor"][r], tbl["neg_lr"][r] = (wd_factor if apply_wd else 0.0), neg_lr
            if not keep_result:
                tbl["c"][r], tbl["ldc"][r] = 0, 0
        n = int(lib.apexw_gemm_grouped_items(tbl.ctypes.data, len(tbl)))
        if n < 0:
            _lib.check(-n, "apexw_gemm_grouped_items (fused Muon update)")
        # the table goes up through pinned memory on the launch stream; the
        # caching host allocator keeps the block until that copy has run
        staged = torch.from_numpy(tbl.view(np.uint8)).pin_memory()
        out = torch.empty_like(dev_probs)
        out.copy_(staged, non_blocking=True)
        return out


class ApexMuon(Optimizer):
    """Muon with fp32 momentum and bf16 Newton-Schulz on the matrix cores."""

    _step_supports_amp_scaling = True

    def __init__(self, params, lr=1e-3, momentum=0.95, nesterov=False, weight_decay=1e-2, ns_steps=4, beta3=None,
                 alpha=5.0, cautious=False, grad_centralization=False, precision="compact", scale_mode="none",
                 ns_method="newtonschulz5", batch_bmm=None, fused=None, capturable=False, compiled=False):
        if lr < 0.0:
            raise ValueError(f"Invalid learning rate: {lr}")
        if not 0.0 <= momentum < 1.0:
            raise ValueError(f"Invalid momentum: {momentum}")
        if weight_decay < 0.0:
            raise ValueError(f"Invalid weight decay: {weight_decay}")
        precision = S.normalize_precision(precision)
        bad = []
        if beta3 is not None:
            bad.append("beta3")
        if cautious:
            bad.append("cautious")
        if grad_centralization:
            bad.append("grad_centralization")
        if precision in ("8bit", "ultra"):
            bad.append(f"precision={precision!r} (quantised momentum)")
        if ns_method != "newtonschulz5":
            bad.append(f"ns_method={ns_method!r}")
        if scale_mode not in ("none", "spectral", "rms_matched", "aspect_ratio"):
            bad.append(f"scale_mode={scale_mode!r}")
        if bad:
            raise NotImplementedError("apexw_amd ApexMuon implements fp32-momentum Newton-Schulz Muon; not supported: "
                                      + ", ".join(bad))
        # True: also store each matrix's final Newton-Schulz result in its
        # workspace (the update is applied to the parameter either way)
        self.keep_ns_result = False
        # work matrices in 32 x 32 panels (False: row-major; same results, read
        # by the products with more L2 requests); read when a workspace is made
        self.ns_panels = True
        defaults = dict(lr=lr, momentum=momentum, nesterov=nesterov, weight_decay=weight_decay, ns_steps=ns_steps,
                        beta3=beta3, alpha=alpha, cautious=cautious, grad_centralization=grad_centralization,
                        precision=precision, scale_mode=scale_mode, ns_method=ns_method, batch_bmm=batch_bmm,
                        fused=fused, capturable=capturable, compiled=compiled)
        super().__init__(params, defaults)
        self._ws = {}
        self._ns_plans = {}
        self._copies = []
        self._amp_init()
        self.state = R.StateMap(self, self.state)

    def __setstate__(self, state):
        super().__setstate__(state)
        self._amp_init()
        self.state = R.StateMap(self, dict.items(self.state))

    def _amp_init(self):
        # GradScaler steps read on the device: per step, the stepped states and a
        # pinned copy of found_inf, until the host has seen the copy (_amp_drain)
        self._amp_unfolded = False
        self._amp_pending = []
        self._amp_stepped = None
        self._amp_dev = None

    # ------------------------------------------------------------------ state
    def _init_param_state(self, p):
        st = self.state[p]
        if len(st) == 0:
            st["step"] = 0
            st["work_dtype"] = torch.bfloat16
            st["momentum"] = torch.zeros_like(p, dtype=torch.float32, memory_format=torch.contiguous_format)
        return st

    def load_state_dict(self, state_dict):
        """Keep fp32 momentum fp32 (the base loader casts floating state to the param dtype)."""
        saved = {}
        for g, sg in zip(self.param_groups, state_dict.get("param_groups", [])):
            for p, pid in zip(g["params"], sg.get("params", [])):
                ent = state_dict.get("state", {}).get(pid, {})
                if isinstance(ent, dict) and isinstance(ent.get("momentum"), torch.Tensor):
                    saved[p] = ent["momentum"].detach().clone()
        super().load_state_dict(state_dict)
        for p, t in saved.items():
            if p in self.state:
                self.state[p]["momentum"] = t.to(device=p.device, dtype=torch.float32)

    # ------------------------------------------------------------------- step
    @staticmethod
    def _scale(mode, m_dim, n_dim):
        if mode == "aspect_ratio":
            return max(1.0, math.sqrt(m_dim / n_dim))
        if mode in ("spectral", "rms_matched"):
            return math.sqrt(max(m_dim, n_dim)) * 0.2
        return 1.0

    def _workspace(self, key, m, n, batch, device):
        # one workspace per (param group, shape): all of a step's work matrices
        # are live together while the grouped Newton-Schulz runs
        ws = self._ws.get(key)
        if ws is None:
            ws = self._ws[key] = NSWorkspace(m, n, batch, device, panel=getattr(self, "ns_panels", True))
        return ws

    def _ns_plan(self, jobs, device):
        key = (device, tuple((id(j["ws"]), j["steps"]) for j in jobs))
        plan = self._ns_plans.get(key)
        if plan is None:
            plan = self._ns_plans[key] = NSPlan([j["ws"] for j in jobs], [j["steps"] for j in jobs], device)
        return plan

    @R.step_hooks
    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        found_inf = getattr(self, "found_inf", None)
        grad_scale = getattr(self, "grad_scale", None)
        self._amp_unfolded = False        # no waits in the lookups of the step itself
        amp = None
        try:
            # AMP: the grads are unscaled inside the momentum kernel (the reference
            # unscales p.grad in place first, apexw/muon.py:566-590).  With found_inf
            # and the scale on the parameters' device, the kernels read both there
            # (the reference reads them on the host, :557-577)
            inv_scale = 1.0
            if self._amp_on_device(grad_scale, found_inf):
                amp = self._amp_prepare(grad_scale, found_inf)
            else:
                if found_inf is not None and float(found_inf) != 0.0:
                    return loss
                if grad_scale is not None:
                    inv_scale = (float(grad_scale.reciprocal().item()) if torch.is_tensor(grad_scale)
                                 else 1.0 / float(grad_scale))
            self._amp_stepped = [] if amp is not None else None
            amp_ptr = amp.data_ptr() if amp is not None else None
            jobs = []
            # a non-contiguous parameter is stepped in a contiguous copy, written back afterwards
            self._copies = []
            for gi, group in enumerate(self.param_groups):
                active = [p for p in group["params"] if p.grad is not None]
                if not active:
                    continue
                matrices = []
                for p in active:
                    if not p.is_cuda:
                        raise RuntimeError("apexw_amd ApexMuon steps CUDA (ROCm) parameters only")
                    if p.dtype not in (torch.float32, torch.bfloat16, torch.float16):
                        raise NotImplementedError(f"ApexMuon: unsupported dtype {p.dtype}")
                    rows = p.shape[0] if p.dim() >= 1 else 1
                    if p.dim() < 2 or min(rows, p.numel() // rows) < 16:
                        # vectors and dimensions under 16: coordinate-wise update (apexw/muon.py:841-847)
                        self._coordwise(p, group, inv_scale, amp_ptr)
                    else:
                        matrices.append(p)
                shapes = defaultdict(list)
                for p in matrices:
                    shapes[tuple(p.shape)].append(p)
                for shape, plist in shapes.items():
                    # the reference batches same-shape matrices on the GPU (apexw/muon.py:593-615)
                    jobs.append(self._prepare(gi, shape, plist, group, inv_scale, amp_ptr))
            # Newton-Schulz of every matrix, grouped per device; matrices are
            # independent, so running all momenta first and all updates last
            # gives each parameter the result of the reference's per-shape loop
            # the last X' product of each matrix applies its update to the
            # parameter (decoupled decay, then p += -lr * scale * U) in its
            # epilogue; with ns_steps == 0 the update is the normalised
            # momentum itself and goes through the separate apply pass
            by_dev = defaultdict(list)
            for j in jobs:
                by_dev[j["ws"].device].append(j)
            for dev, djobs in by_dev.items():
                plan = self._ns_plan(djobs, dev)
                applies = [self._apply_args(j) for j in djobs]
                plan.run(torch.cuda.current_stream(dev).cuda_stream, applies, self.keep_ns_result, amp_ptr)
            for j in jobs:
                if j["steps"] == 0:
                    self._apply(j, amp_ptr)
            for p, work in self._copies:
                p.copy_(work)   # after a skipped step, work still equals p
            if amp is not None:
                self._amp_record(found_inf)
        finally:
            self._copies = []
            self._amp_stepped = None
            self.grad_scale = None
            self.found_inf = None
            self._amp_unfolded = bool(self._amp_pending)
        return loss

    # ------------------------------------------------------- AMP on the device
    def _amp_on_device(self, grad_scale, found_inf):
        """found_inf (and the scale, if any) are one-element tensors on the device
        of every parameter stepped this time: the kernels read them there."""
        if not (torch.is_tensor(found_inf) and found_inf.is_cuda and found_inf.numel() == 1):
            return False
        if grad_scale is not None and not (torch.is_tensor(grad_scale) and grad_scale.is_cuda
                                           and grad_scale.numel() == 1):
            return False
        dev = found_inf.device
        return all(p.device == dev for g in self.param_groups for p in g["params"] if p.grad is not None)

    def _amp_prepare(self, grad_scale, found_inf):
        """This step's skip flag and 1 / scale as a device apexw_amp_dyn
        (apexw_amp_prepare; the Muon kernels read only skip and grad_inv_scale)."""
        self._amp_drain(wait=False)
        dev = found_inf.device
        if self._amp_dev is None or self._amp_dev[0] != dev:
            self._amp_dev = (dev, torch.zeros(1, dtype=torch.int32, device=dev),
                             torch.empty(_lib.AMP_DYN_BYTES // 4, dtype=torch.float32, device=dev),
                             torch.ones(1, dtype=torch.float32, device=dev))
        _, skips, dyn, one = self._amp_dev
        scale = one if grad_scale is None else grad_scale.detach().reshape(1).to(dev, torch.float32).contiguous()
        fi = found_inf.detach().reshape(1).to(dev, torch.float32).contiguous()
        launch = np.zeros(1, dtype=_lib.AMP_LAUNCH_DTYPE)
        launch["beta1"], launch["beta2"], launch["step"] = 0.5, 0.5, 1.0
        lib = _lib.load()
        _lib.check(lib.apexw_amp_prepare(fi.data_ptr(), scale.data_ptr(), skips.data_ptr(), 0, launch.ctypes.data, 1,
                                         dyn.data_ptr(), torch.cuda.current_stream(dev).cuda_stream),
                   "apexw_amp_prepare")
        return dyn

    def _amp_record(self, found_inf):
        """Keep this step's stepped states with an asynchronous copy of found_inf."""
        flag = torch.empty(1, dtype=torch.float32, pin_memory=True)
        flag.copy_(found_inf.detach().reshape(1), non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(found_inf.device))
        self._amp_pending.append((ev, flag, self._amp_stepped))

    def _amp_drain(self, wait):
        """Take back the step counts of the skipped steps whose found_inf copy has
        arrived (wait: of every pending step, after waiting for the copies)."""
        while self._amp_pending:
            ev, flag, stepped = self._amp_pending[0]
            if wait:
                ev.synchronize()
            elif not ev.query():
                break
            self._amp_pending.pop(0)
            if float(flag[0]) != 0.0:
                for st in stepped:
                    st["step"] -= 1

    def _fold_amp_skips(self):
        """Make every step counter exact (StateMap's first lookup after a step)."""
        self._amp_unfolded = False
        self._amp_drain(wait=True)

    def _prepare(self, gi, shape, plist, group, inv_scale=1.0, amp=None):
        """Momentum update and normalised bf16 work matrix (both layouts) of one same-shape batch."""
        lib = _lib.load()
        p0 = plist[0]
        rows, cols = p0.shape[0], p0.numel() // p0.shape[0]
        m, n = min(rows, cols), max(rows, cols)
        dev = p0.device
        stream = torch.cuda.current_stream(dev).cuda_stream
        ws = self._workspace((gi, shape, len(plist), dev), m, n, len(plist), dev)
        mu = float(group["momentum"])
        for i, p in enumerate(plist):
            st = self._init_param_state(p)
            self._count_step(st)
            g = p.grad if p.grad.is_contiguous() else p.grad.contiguous()
            _lib.check(lib.apexw_muon_prepare(
                st["momentum"].data_ptr(), g.data_ptr(), _dtype_code(g.dtype), rows, cols, mu, 1.0 - mu,
                int(bool(group["nesterov"])), NS_EPS, inv_scale, ws.x[0][i].data_ptr(), ws.xt[0][i].data_ptr(),
                ws.np_, ws.mp, ws.layout,
                ws.partial[i].data_ptr(), amp, stream), "apexw_muon_prepare")
        return {"plist": plist, "targets": [self._target(p) for p in plist], "group": group, "ws": ws,
                "rows": rows, "cols": cols, "steps": int(group["ns_steps"]), "batched": len(plist) > 1}

    def _update_scalars(self, job):
        """(wd_factor, neg_lr, apply_wd) of the decoupled decay and the scaled
        orthogonalised update (apexw/muon.py:852-858).  On a 16-bit p, torch's
        add_ (and _foreach_add_) take alpha in p's dtype; mul_ keeps its scalar
        in fp32 and only the same-dtype _foreach_mul_ of the batched path rounds it."""
        group, p0 = job["group"], job["plist"][0]
        lr, wd = float(group["lr"]), float(group["weight_decay"])
        scale = self._scale(group["scale_mode"], job["rows"], job["cols"])
        wd_factor, neg_lr = 1.0 - lr * wd, _round_to(p0.dtype, -lr * scale)
        if job["batched"]:
            wd_factor = _round_to(p0.dtype, wd_factor)
        return wd_factor, neg_lr, wd != 0.0

    def _target(self, p):
        """The tensor the update is written into: p itself, or, when p is not
        contiguous, a contiguous copy that step() writes back into p."""
        if p.is_contiguous():
            return p
        work = p.detach().contiguous()
        self._copies.append((p, work))
        return work

    def _count_step(self, st):
        st["step"] += 1
        if self._amp_stepped is not None:
            self._amp_stepped.append(st)

    def _coordwise(self, p, group, inv_scale, amp=None):
        """The reference's coordinate-wise fallback (apexw/muon.py:841-858): momentum,
        U = s / (std(s) + 1e-7), p -= lr * 0.05 * U after the decoupled decay."""
        lib = _lib.load()
        st = self._init_param_state(p)
        self._count_step(st)
        mu = float(group["momentum"])
        lr, wd = float(group["lr"]), float(group["weight_decay"])
        g = p.grad if p.grad.is_contiguous() else p.grad.contiguous()
        dst = self._target(p)
        stream = torch.cuda.current_stream(p.device).cuda_stream
        _lib.check(lib.apexw_muon_coordwise(
            st["momentum"].data_ptr(), g.data_ptr(), _dtype_code(g.dtype), dst.data_ptr(), _dtype_code(p.dtype),
            p.numel(), mu, 1.0 - mu, int(bool(group["nesterov"])), inv_scale, 1.0 - lr * wd, int(wd != 0.0),
            _round_to(p.dtype, -lr * 0.05), amp, stream), "apexw_muon_coordwise")

    def _apply_args(self, job):
        """Per batch entry, the fused update of the final Newton-Schulz product (NSPlan.run).
        U is the wide work matrix: p's layout when wide, its transpose when tall."""
        wd_factor, neg_lr, apply_wd = self._update_scalars(job)
        rows, cols = job["rows"], job["cols"]
        return [(t.data_ptr(), _dtype_code(t.dtype), rows, cols, rows > cols, apply_wd, wd_factor, neg_lr)
                for t in job["targets"]]

    def _apply(self, job, amp=None):
        """The update as a separate pass over the work matrix (ns_steps == 0)."""
        lib = _lib.load()
        plist, ws, rows, cols = job["plist"], job["ws"], job["rows"], job["cols"]
        stream = torch.cuda.current_stream(plist[0].device).cuda_stream
        wd_factor, neg_lr, apply_wd = self._update_scalars(job)
        u_buf = ws.x[job["steps"] % 2]           # ping-pong slot of the Newton-Schulz result
        for i, p in enumerate(job["targets"]):
            _lib.check(lib.apexw_muon_apply(p.data_ptr(), _dtype_code(p.dtype), u_buf[i].data_ptr(), rows, cols,
                                            ws.np_, ws.layout, int(rows > cols), wd_factor, int(apply_wd), neg_lr, amp,
                                            stream),
                       "apexw_muon_apply")

    def get_state_memory_mb(self):
        tot = 0
        for st in self.state.values():
            for v in st.values():
                if isinstance(v, torch.Tensor):
                    tot += v.numel() * v.element_size()
        return tot / (1024 * 1024)
