"""ApexMuon: momentum + Newton-Schulz orthogonalised updates on the GPU.

Drop-in for the reference ``apexw.muon.ApexMuon`` (apexw/muon.py:344-861) for
the fp32-momentum configuration: same constructor, defaults, ``state`` keys
(``step``, ``work_dtype``, ``momentum``) and ``load_state_dict`` dtype
handling.  The step runs through libapexw_hip.so:

* ``apexw_muon_prepare``: fp32 momentum update, the bf16 work matrix normalised
  by its Frobenius norm, written in both orientations;
* ``newton_schulz``: per iteration three bf16 MFMA GEMMs
  (``A = X X^T``; ``B = c A A + b A``; ``X = B X + a X``) through
  ``apexw_gemm_nt_bf16``, batched over same-shape matrices;
* ``apexw_muon_apply``: decoupled weight decay and ``p -= lr * scale * U``.

Like the reference on a bf16-capable GPU, the Newton-Schulz work dtype is
bf16 (apexw/muon.py:76-89).  Quantised momentum (precision "8bit"/"ultra"),
AdEMAMix (beta3), cautious masking, grad centralization, the Polar Express
coefficients and scale_mode="rms" raise ``NotImplementedError``.
"""

import math
from collections import defaultdict

import torch
from torch.optim.optimizer import Optimizer

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


def _round_to(dtype, x):
    """A Python scalar as torch's same-dtype foreach ops see it (rounded to dtype)."""
    return float(torch.tensor(x, dtype=torch.float32).to(dtype).float()) if dtype != torch.float32 else x


class NSWorkspace:
    """bf16 Newton-Schulz buffers for `batch` matrices whose wide work shape is m x n.

    Dimensions are padded to the GEMM tile; the padding is zero and stays zero
    through every product.  X and its transpose are kept for two iterations
    (ping-pong), plus the symmetric A and B.
    """

    def __init__(self, m, n, batch, device):
        self.m, self.n, self.batch = m, n, batch
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


def _gemm(lib, stream, a, b, et, c, ct, m, n, k, lda, ldb, lde, ldc, ldct, batch, sa, sb, se, sc, sct, alpha, beta):
    st = lib.apexw_gemm_nt_bf16(a, b, et, c, ct, m, n, k, lda, ldb, lde, ldc, ldct, batch, sa, sb, se, sc, sct,
                                alpha, beta, stream)
    _lib.check(st, "apexw_gemm_nt_bf16")


def newton_schulz(ws, steps, stream):
    """Run `steps` quintic iterations on ws.x[0] / ws.xt[0]; returns the index of the result buffer."""
    lib = _lib.load()
    mp, np_, bt = ws.mp, ws.np_, ws.batch
    sx, sa = mp * np_, mp * mp
    cur = 0
    for _ in range(steps):
        x, xt = ws.x[cur].data_ptr(), ws.xt[cur].data_ptr()
        nx, nxt = ws.x[cur ^ 1].data_ptr(), ws.xt[cur ^ 1].data_ptr()
        a, b = ws.a.data_ptr(), ws.b.data_ptr()
        # A = X X^T   (symmetric: stored through the transposed output)
        _gemm(lib, stream, x, x, None, None, a, mp, mp, np_, np_, np_, 0, 0, mp, bt, sx, sx, 0, 0, sa, 1.0, 0.0)
        # B = c A A + b A
        _gemm(lib, stream, a, a, a, None, b, mp, mp, mp, mp, mp, mp, 0, mp, bt, sa, sa, sa, 0, sa, NS_C, NS_B)
        # X' = B X + a X  with X read as X^T rows; written in both orientations
        _gemm(lib, stream, b, xt, xt, nx, nxt, mp, np_, mp, mp, mp, mp, np_, mp, bt, sa, sx, sx, sx, sx, 1.0, NS_A)
        cur ^= 1
    return cur


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
        defaults = dict(lr=lr, momentum=momentum, nesterov=nesterov, weight_decay=weight_decay, ns_steps=ns_steps,
                        beta3=beta3, alpha=alpha, cautious=cautious, grad_centralization=grad_centralization,
                        precision=precision, scale_mode=scale_mode, ns_method=ns_method, batch_bmm=batch_bmm,
                        fused=fused, capturable=capturable, compiled=compiled)
        super().__init__(params, defaults)
        self._ws = {}

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

    def _workspace(self, m, n, batch, device):
        key = (m, n, batch, device)
        ws = self._ws.get(key)
        if ws is None:
            ws = self._ws[key] = NSWorkspace(m, n, batch, device)
        return ws

    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        found_inf = getattr(self, "found_inf", None)
        grad_scale = getattr(self, "grad_scale", None)
        try:
            if found_inf is not None and float(found_inf) != 0.0:
                return loss
            if grad_scale is not None:
                raise NotImplementedError("ApexMuon: GradScaler grad_scale hand-off is not supported; unscale first")
            for group in self.param_groups:
                active = [p for p in group["params"] if p.grad is not None]
                if not active:
                    continue
                for p in active:
                    if not p.is_cuda:
                        raise RuntimeError("apexw_amd ApexMuon steps CUDA (ROCm) parameters only")
                    rows = p.shape[0] if p.dim() >= 1 else 1
                    if p.dim() < 2 or min(rows, p.numel() // rows) < 16:
                        raise NotImplementedError(
                            "ApexMuon: parameters with fewer than 16 rows or columns (the reference's coordinate-wise "
                            "fallback) are not supported; route them to ApexW (HybridApexW does)")
                shapes = defaultdict(list)
                for p in active:
                    shapes[tuple(p.shape)].append(p)
                for shape, plist in shapes.items():
                    # the reference batches same-shape matrices on the GPU (apexw/muon.py:593-615)
                    self._step_matrices(plist, group, batched=len(plist) > 1)
        finally:
            self.grad_scale = None
            self.found_inf = None
        return loss

    def _step_matrices(self, plist, group, batched):
        lib = _lib.load()
        p0 = plist[0]
        rows, cols = p0.shape[0], p0.numel() // p0.shape[0]
        m, n = min(rows, cols), max(rows, cols)
        tall = rows > cols
        dev = p0.device
        stream = torch.cuda.current_stream(dev).cuda_stream
        ws = self._workspace(m, n, len(plist), dev)
        mu = float(group["momentum"])
        for i, p in enumerate(plist):
            st = self._init_param_state(p)
            st["step"] += 1
            g = p.grad if p.grad.is_contiguous() else p.grad.contiguous()
            if g.dtype != p.dtype:
                raise NotImplementedError("ApexMuon: gradient dtype must match the parameter dtype")
            _lib.check(lib.apexw_muon_prepare(
                st["momentum"].data_ptr(), g.data_ptr(), _dtype_code(g.dtype), rows, cols, mu, 1.0 - mu,
                int(bool(group["nesterov"])), NS_EPS, ws.x[0][i].data_ptr(), ws.xt[0][i].data_ptr(), ws.np_, ws.mp,
                ws.partial[i].data_ptr(), stream), "apexw_muon_prepare")
        res = newton_schulz(ws, int(group["ns_steps"]), stream)
        lr, wd = float(group["lr"]), float(group["weight_decay"])
        scale = self._scale(group["scale_mode"], rows, cols)
        wd_factor, neg_lr = 1.0 - lr * wd, -lr * scale
        if batched:
            # torch._foreach_mul_ / _foreach_add_ over same-dtype lists see the scalars in p's dtype
            wd_factor, neg_lr = _round_to(p0.dtype, wd_factor), _round_to(p0.dtype, neg_lr)
        # U in p's layout: the work matrix when wide, its transpose when tall
        u_buf, ldu = (ws.xt[res], ws.mp) if tall else (ws.x[res], ws.np_)
        for i, p in enumerate(plist):
            if not p.is_contiguous():
                raise NotImplementedError("ApexMuon: parameters must be contiguous")
            _lib.check(lib.apexw_muon_apply(p.data_ptr(), _dtype_code(p.dtype), u_buf[i].data_ptr(), rows, cols, ldu,
                                            wd_factor, int(wd != 0.0), neg_lr, stream), "apexw_muon_apply")

    def get_state_memory_mb(self):
        tot = 0
        for st in self.state.values():
            for v in st.values():
                if isinstance(v, torch.Tensor):
                    tot += v.numel() * v.element_size()
        return tot / (1024 * 1024)
