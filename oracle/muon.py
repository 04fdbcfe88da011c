"""Newton-Schulz polar factor, Muon step and hybrid routing (CPU oracle; test infrastructure only).

* ``newton_schulz5`` restates ``zeropower_via_newtonschulz5`` (``apexw/muon.py:135-184``)
  and its loop ``_newton_schulz5_inner`` (:102-108): normalise by the Frobenius
  norm + 1e-7, work on the wide orientation (rows <= cols), then
  ``A = X X^T; B = b A + c A A; X = a X + B X`` with (a, b, c) =
  (3.4445, -4.7750, 2.0315).
* ``newton_schulz5_batched`` restates the batched form (:187-211).
* ``muon_eligible`` / ``partition_for_hybrid`` restate ``hybrid.py:73-141``.
* ``OracleHybrid`` drives ``ApexMuon._step_single`` / ``_step_batched``
  (muon.py:539-861) with the ``HybridApexW`` defaults (hybrid.py:222-321:
  ns_steps 5, scale 0.2*sqrt(max(m, n)), muon lr = 5*lr) and hands the
  remaining parameters to ``OracleApexW``.
* ``coordwise_step`` restates ``_step_single``'s coordinate-wise fallback for
  vectors and dimensions under 16 (muon.py:775-799, :841-858): U = s /
  (std(s, unbiased=False) + 1e-7), scale 0.05.  Pinned by
  tests/test_oracle_muon_coordwise.py: two elements (the population std is
  half their distance, where the unbiased one would be 1/sqrt(2) of it), one
  element (U = s / (|s| + 1e-7)), invariance of U under a positive scaling
  of the grad from zero momentum, and a first step from zero momentum whose
  update is -lr * 0.05 * U after the decay.
"""

import math

import torch

from .optim import OracleApexW

NS_A, NS_B, NS_C = 3.4445, -4.7750, 2.0315


def newton_schulz5(G, steps=5, eps=1e-7, work_dtype=torch.float32):
    shape = G.shape
    if G.ndim > 2:
        G = G.reshape(shape[0], -1)
    X = G.to(work_dtype)
    X = X / (X.norm() + eps)
    tall = X.shape[0] > X.shape[1]
    X = X.T.contiguous() if tall else X.contiguous()
    for _ in range(steps):
        A = X @ X.T
        B = torch.addmm(A, A, A, beta=NS_B, alpha=NS_C)
        X = torch.addmm(X, B, X, beta=NS_A, alpha=1.0)
    if tall:
        X = X.T
    return X.reshape(shape).to(G.dtype)


def newton_schulz5_batched(Xb, steps=5, eps=1e-7, work_dtype=torch.float32):
    X = Xb.to(work_dtype)
    X = X / (torch.linalg.norm(X, dim=(-2, -1), keepdim=True) + eps)
    tall = X.shape[1] > X.shape[2]
    X = X.transpose(-2, -1).contiguous() if tall else X.contiguous()
    for _ in range(steps):
        A = torch.bmm(X, X.transpose(-2, -1).contiguous())
        B = torch.baddbmm(A, A, A, beta=NS_B, alpha=NS_C)
        X = torch.baddbmm(X, B, X, beta=NS_A, alpha=1.0)
    if tall:
        X = X.transpose(-2, -1)
    return X.to(Xb.dtype)


def muon_eligible(p, exclude_embeddings=True, min_dim=32):
    if not p.requires_grad or p.ndim < 2:
        return False
    m = p.shape[0]
    n = p.numel() // m
    if min(m, n) < min_dim:
        return False
    if exclude_embeddings and max(m, n) >= 1000 and max(m / n, n / m) >= 4.0:
        return False
    return True


def partition_for_hybrid(params, exclude_embeddings=True, min_dim=32):
    mu, aw = [], []
    for p in params:
        if muon_eligible(p, exclude_embeddings, min_dim):
            mu.append(p)
        elif p.requires_grad:
            aw.append(p)
    return mu, aw


@torch.no_grad()
def coordwise_step(p, grad, buf, *, lr, momentum, weight_decay, nesterov=False, inv_scale=None):
    """ApexMuon._step_single for a parameter Newton-Schulz does not take (a vector,
    or a dimension under 16): apexw/muon.py:775-799 then :841-858.  Updates p and
    the fp32 momentum buf in place; returns U."""
    g = grad
    if inv_scale is not None:
        g = g.mul(inv_scale)                       # p.grad.mul_(inv_scale) in the grad dtype (:566-590)
    g = torch.nan_to_num(g, nan=0.0, posinf=65504.0, neginf=-65504.0)
    g_fp = g if g.dtype == torch.float32 else g.float()
    buf.mul_(momentum).add_(g_fp, alpha=1.0 - momentum)
    src = g_fp.lerp(buf, momentum) if nesterov else buf
    if src.numel() <= 1:
        std = src.abs() + 1e-7
    else:
        std = src.std(unbiased=False) + 1e-7
    U = src / std
    if weight_decay != 0.0:
        p.mul_(1.0 - lr * weight_decay)
    p.add_(U.to(p.dtype), alpha=-lr * 0.05)
    return U


class OracleHybrid:
    """CPU hybrid optimizer: Muon on eligible matrices, OracleApexW on the rest."""

    def __init__(self, params, lr=1e-3, weight_decay=1e-2, muon_momentum=0.95, ns_steps=5,
                 work_dtype=torch.float32, **apex_kwargs):
        params = list(params)
        self.muon_params, self.adamw_params = partition_for_hybrid(params)
        self.lr_mu = lr * 5.0
        self.wd = weight_decay
        self.momentum = muon_momentum
        self.ns_steps = ns_steps
        self.work_dtype = work_dtype
        self.momenta = {}
        self.adamw = OracleApexW(self.adamw_params, lr=lr, weight_decay=weight_decay, **apex_kwargs) \
            if self.adamw_params else None

    @torch.no_grad()
    def step(self):
        groups = {}
        for p in self.muon_params:
            if p.grad is not None:
                groups.setdefault(tuple(p.shape), []).append(p)
        for shape, plist in groups.items():
            valid = len(shape) >= 2 and min(shape[0], plist[0].numel() // shape[0]) >= 16
            if len(plist) > 1 and valid and plist[0].numel() <= 16384:
                self._batched(plist)
            else:
                for p in plist:
                    self._single(p)
        if self.adamw is not None:
            self.adamw.step()

    def _momentum(self, p, g):
        buf = self.momenta.get(p)
        if buf is None:
            buf = self.momenta[p] = torch.zeros_like(p, dtype=torch.float32)
        buf.mul_(self.momentum).add_(g, alpha=1.0 - self.momentum)
        return buf

    def _apply(self, p, U, dims):
        scale = math.sqrt(max(dims)) * 0.2
        if self.wd != 0.0:
            p.mul_(1.0 - self.lr_mu * self.wd)
        p.add_(U.to(p.dtype), alpha=-self.lr_mu * scale)

    def _single(self, p):
        g = torch.nan_to_num(p.grad, nan=0.0, posinf=65504.0, neginf=-65504.0)
        buf = self._momentum(p, g if g.dtype == torch.float32 else g.float())
        U = newton_schulz5(buf, self.ns_steps, work_dtype=self.work_dtype)
        self._apply(p, U, (U.shape[0], U.numel() // U.shape[0]))

    def _batched(self, plist):
        grads = [torch.nan_to_num(p.grad, nan=0.0, posinf=65504.0, neginf=-65504.0) for p in plist]
        shape2 = (plist[0].shape[0], plist[0].numel() // plist[0].shape[0])
        bufs = [self._momentum(p, g) for p, g in zip(plist, grads)]
        Ub = newton_schulz5_batched(torch.stack([b.reshape(shape2).to(self.work_dtype) for b in bufs]),
                                    self.ns_steps, work_dtype=self.work_dtype)
        scale = math.sqrt(max(shape2)) * 0.2
        for i, p in enumerate(plist):
            if self.wd != 0.0:
                p.mul_(1.0 - self.lr_mu * self.wd)
            p.add_(Ub[i].reshape(p.shape).to(p.dtype), alpha=-self.lr_mu * scale)
