"""CPU oracle for the fused chunked Gated DeltaNet (GDN) forward.

TEST INFRASTRUCTURE ONLY.  This module is the checker, never the product:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it.  The product path (the HIP kernels behind the
C ABI) never calls into this file and has no CPU fallback.

It restates, in plain PyTorch on the CPU, the semantics of the reference's
``gdn_ref.py``:

* ``l2norm``          -- gdn_ref.py:24-25
* ``sigmoid``, ``logsigmoid``, ``prep_inputs`` -- the gate activations of
                         the BASELINE.json input recipe and the fused input
                         preparation built on them (fp64, textbook forms)
* ``recurrent``       -- gdn_ref.py:28-45  (the definition, gdn_ref.py:3-9)
* ``chunked_ut``      -- gdn_ref.py:48-99  (the chunked UT transform; same op
                         order, including the two unit-triangular solves and
                         the K x K state update, so that timing it is a fair
                         CPU baseline)
* ``recurrent_grads`` -- gradients of ``recurrent`` by reverse-mode
                         differentiation (torch.autograd, fp64); the
                         reference has no backward (README.md:259)
* ``chunked_bwd``     -- the chunked backward the HIP kernel implements,
                         restated per head in fp64 (pinned against
                         ``recurrent_grads``)
* ``pad_to_multiple`` -- gdn_ref.py:102-114
* ``rel_err``         -- bench_gdn.py:89-94 (max-norm relative error)
* ``make_inputs_*``   -- bench_gdn.py:33-40 (reference recipe) and the
                         BASELINE.json config recipe (L2-normed q/k,
                         N(0,1) v, sigmoid beta, logsigmoid g, optional h0).

State layout: like the reference, the oracle keeps the per-head state as
``h [B, H, V, K]`` (V x K, K contiguous; gdn_ref.py:29,37).  The product API
uses ``final_state [B, H, K, V]`` (the K x V form S = h^T); ``to_kv`` /
``to_vk`` convert between the two.

How each function is pinned (see ``tests/test_oracle.py``):
closed forms (T=1, beta=0, orthonormal keys, the delta "write" property),
invariants (linearity in (v, h0), scale, segment composability, padding,
head/batch permutation), agreement between the two independent algorithms
(step recurrence vs. chunked UT with triangular solves), exact-rational
golden vectors (``tests/golden``), and the reference's own self-check shape
(gdn_ref.py:117-132).
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional, Tuple

import torch

__all__ = [
    "l2norm", "sigmoid", "logsigmoid", "prep_inputs", "recurrent", "recurrent_grads",
    "chunked_bwd", "chunked_ut", "pad_to_multiple", "rel_err",
    "make_inputs_reference", "make_inputs_baseline", "to_kv", "to_vk",
    "BaselineConfig", "BASELINE_CONFIGS", "algorithmic_bytes",
    "algorithmic_flops",
]


# ---------------------------------------------------------------------------
# semantics
# ---------------------------------------------------------------------------

def l2norm(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """``x / sqrt(sum(x^2) + eps)`` over the last dim (gdn_ref.py:24-25).

    The sum of squares is taken in fp32 and the denominator is cast back to
    ``x.dtype`` before the division, as the reference does.
    """
    denom = torch.sqrt(x.float().pow(2).sum(-1, keepdim=True) + eps)
    return x / denom.to(x.dtype)


def sigmoid(x: torch.Tensor) -> torch.Tensor:
    """``1 / (1 + e^{-x})`` in fp64 (beta of the BASELINE input recipe)."""
    return 1.0 / (1.0 + torch.exp(-x.double()))


def logsigmoid(x: torch.Tensor) -> torch.Tensor:
    """``log(sigmoid(x))`` in fp64, as ``min(x, 0) - log1p(e^{-|x|})`` (finite
    for every x; g of the BASELINE input recipe)."""
    x = x.double()
    return torch.clamp(x, max=0.0) - torch.log1p(torch.exp(-x.abs()))


def prep_inputs(q=None, k=None, beta=None, g=None, eps: float = 1e-6,
                gate_dtype=torch.float32):
    """The fused input preparation: ``l2norm`` of q and k (in their dtype),
    ``sigmoid(beta)`` and ``logsigmoid(g)`` cast to ``gate_dtype``.  Any
    argument may be None."""
    return (None if q is None else l2norm(q, eps), None if k is None else l2norm(k, eps),
            None if beta is None else sigmoid(beta).to(gate_dtype),
            None if g is None else logsigmoid(g).to(gate_dtype))


def recurrent(q, k, v, beta, g, initial_state=None, dtype=torch.float64):
    """Step recurrence, the definition of GDN (gdn_ref.py:3-9, 28-45).

    Per head, with the state ``h`` a V x K matrix::

        h_t = e^{g_t} h_{t-1} + u_t k_t^T
        u_t = beta_t (v_t - e^{g_t} h_{t-1} k_t)
        o_t = h_t q_t

    Args are ``q, k [B,T,H,K]``, ``v [B,T,H,V]``, ``beta, g [B,T,H]``,
    ``initial_state [B,H,V,K]`` or None.  Computed in ``dtype``.
    Returns ``o [B,T,H,V]`` and ``h [B,H,V,K]`` in ``dtype``.
    """
    B, T, H, K = q.shape
    V = v.shape[-1]
    q = q.to(dtype)
    k = k.to(dtype)
    v = v.to(dtype)
    beta = beta.to(dtype)
    g = g.to(dtype)
    if initial_state is None:
        h = torch.zeros(B, H, V, K, dtype=dtype)
    else:
        h = initial_state.to(dtype).clone()
    o = torch.empty(B, T, H, V, dtype=dtype)
    for t in range(T):
        kt = k[:, t]                                   # [B,H,K]
        h = h * torch.exp(g[:, t])[:, :, None, None]   # decay first
        pred = (h @ kt.unsqueeze(-1)).squeeze(-1)      # [B,H,V] = h k_t
        u = beta[:, t].unsqueeze(-1) * (v[:, t] - pred)
        h = h + u.unsqueeze(-1) * kt.unsqueeze(-2)     # rank-1 write
        o[:, t] = (h @ q[:, t].unsqueeze(-1)).squeeze(-1)
    return o, h


def recurrent_grads(q, k, v, beta, g, initial_state, do, dfinal, scale=1.0):
    """Gradients of ``L = <o, do> + <final_state, dfinal>`` with respect to
    (q, k, v, beta, g, initial_state) for ``o = scale * recurrent(...)``,
    by torch.autograd through the fp64 step recurrence.

    Shapes as ``recurrent``; ``initial_state`` and ``dfinal`` in the K x V
    layout ``[B, H, K, V]`` (None = zero).  Returns fp64 tensors
    ``(dq, dk, dv, dbeta, dg, dh0)``.
    """
    B, T, H, K = q.shape
    V = v.shape[-1]
    h0 = torch.zeros(B, H, K, V, dtype=torch.float64) if initial_state is None else initial_state
    xs = [t.detach().double().requires_grad_(True) for t in (q, k, v, beta, g, h0)]
    o, h = recurrent(xs[0], xs[1], xs[2], xs[3], xs[4], to_vk(xs[5]), dtype=torch.float64)
    loss = (scale * o * do.double()).sum()
    if dfinal is not None:
        loss = loss + (to_kv(h) * dfinal.double()).sum()
    return torch.autograd.grad(loss, xs)


def chunked_bwd(q, k, v, beta, g, initial_state, do, dfinal, scale=1.0, C=32):
    """The chunked backward, one head at a time, in fp64: pass 1 stores the
    state at each chunk start, pass 2 walks the chunks backward carrying the
    state gradient (the algebra of csrc/gdn_bwd.hip's header).  Same
    arguments and returns as ``recurrent_grads``."""
    B, T, H, K = q.shape
    V = v.shape[-1]
    f = lambda t: t.double()
    outs = [torch.zeros(B, T, H, K, dtype=torch.float64), torch.zeros(B, T, H, K, dtype=torch.float64),
            torch.zeros(B, T, H, V, dtype=torch.float64), torch.zeros(B, T, H, dtype=torch.float64),
            torch.zeros(B, T, H, dtype=torch.float64), torch.zeros(B, H, K, V, dtype=torch.float64)]
    eye = torch.eye(C, dtype=torch.float64)
    for b in range(B):
        for hh in range(H):
            S = (torch.zeros(K, V, dtype=torch.float64) if initial_state is None
                 else f(initial_state[b, hh]))
            nch = (T + C - 1) // C

            def chunk(c):
                sl = slice(c * C, min(c * C + C, T))
                n = sl.stop - sl.start
                pad = lambda x, w: torch.cat([f(x), torch.zeros((C - n,) + tuple(x.shape[1:]),
                                                                dtype=torch.float64)]) if w else f(x)
                Q = pad(q[b, sl, hh], True)
                Kc = pad(k[b, sl, hh], True)
                Vc = pad(v[b, sl, hh], True)
                dO = pad(do[b, sl, hh], True)
                gg = pad(g[b, sl, hh], True)
                bt = pad(beta[b, sl, hh], True)
                return sl, n, Q, Kc, Vc, dO, gg, bt

            def ut(Kc, Vc, gg, bt, S):
                bb = gg.cumsum(0)
                gam, D, gC = bb.exp(), (bb[-1] - bb).exp(), bb[-1].exp()
                M = torch.tril((bb[:, None] - bb[None, :]).exp())
                KK = Kc @ Kc.T
                A = torch.tril(bt[:, None] * M * KK, -1)
                Tm = torch.linalg.solve_triangular(eye + A, eye, upper=False, unitriangular=True)
                W = Tm @ ((bt * gam)[:, None] * Kc)
                u = Tm @ (bt[:, None] * Vc) - W @ S
                return gam, D, gC, M, KK, A, Tm, W, u

            starts = []
            for c in range(nch):
                sl, n, Q, Kc, Vc, dO, gg, bt = chunk(c)
                starts.append(S)
                gam, D, gC, M, KK, A, Tm, W, u = ut(Kc, Vc, gg, bt, S)
                S = gC * S + Kc.T @ (D[:, None] * u)
            dS = (torch.zeros(K, V, dtype=torch.float64) if dfinal is None else f(dfinal[b, hh]))
            for c in reversed(range(nch)):
                sl, n, Q, Kc, Vc, dO, gg, bt = chunk(c)
                S = starts[c]
                gam, D, gC, M, KK, A, Tm, W, u = ut(Kc, Vc, gg, bt, S)
                QK = Q @ Kc.T
                KdS = Kc @ dS
                du = scale * (M * QK).T @ dO + D[:, None] * KdS
                dQK = M * (scale * dO @ u.T)
                dD = (u * KdS).sum(1)
                dgam = scale * (dO * (Q @ S)).sum(1)
                dgC = (dS * S).sum()
                dW = -du @ S.T
                dT = du @ (bt[:, None] * Vc).T + dW @ ((bt * gam)[:, None] * Kc).T
                dWt, dUt = Tm.T @ dW, Tm.T @ du
                dbt = (Vc * dUt).sum(1) + gam * (Kc * dWt).sum(1)
                dgam = dgam + bt * (Kc * dWt).sum(1)
                dA = torch.tril(-(Tm.T @ dT @ Tm.T), -1)
                dKK = dA * bt[:, None] * M
                dbt = dbt + (dA * M * KK).sum(1)
                dQQ, dAA = dQK * QK, dA * A
                db = dgam * gam - dD * D + dQQ.sum(1) - dQQ.sum(0) + dAA.sum(1) - dAA.sum(0)
                db[C - 1] += (dD * D).sum() + dgC * gC
                dgc = db.flip(0).cumsum(0).flip(0)
                outs[0][b, sl, hh] = (dQK @ Kc + scale * gam[:, None] * (dO @ S.T))[:n]
                outs[1][b, sl, hh] = (dQK.T @ Q + D[:, None] * (u @ dS.T) + (bt * gam)[:, None] * dWt
                                      + (dKK + dKK.T) @ Kc)[:n]
                outs[2][b, sl, hh] = (bt[:, None] * dUt)[:n]
                outs[3][b, sl, hh] = dbt[:n]
                outs[4][b, sl, hh] = dgc[:n]
                dS = scale * Q.T @ (gam[:, None] * dO) + gC * dS - W.T @ du
            outs[5][b, hh] = dS
    return tuple(outs)


def chunked_ut(q, k, v, beta, g, C=64, initial_state=None):
    """Chunked UT transform in fp32 (gdn_ref.py:48-99).

    Within each chunk of ``C`` steps, with ``b = cumsum(g)``::

        A[t,j] = beta_t e^{b_t-b_j} (k_t . k_j)       strictly lower
        U = (I+A)^{-1} (beta v),   W = (I+A)^{-1} (beta e^{b} k)
        u = U - W h^T
        o_t = e^{b_t} q_t . h + sum_{j<=t} e^{b_t-b_j} (q_t . k_j) u_j
        h' = h (e^{b_C} I - Wbar^T K) + Ubar^T K,   Xbar_t = X_t e^{b_C-b_t}

    The op order follows the reference, including the two unit-triangular
    solves (gdn_ref.py:84-85) and the K x K update matrix
    (gdn_ref.py:93-98).  Requires ``T % C == 0`` (gdn_ref.py:62).
    """
    B, T, H, K = q.shape
    V = v.shape[-1]
    if T % C != 0:
        raise ValueError(f"T={T} must be a multiple of C={C}; pad first")
    f32 = torch.float32
    q = q.to(f32)
    k = k.to(f32)
    v = v.to(f32)
    beta = beta.to(f32)
    g = g.to(f32)
    if initial_state is None:
        h = torch.zeros(B, H, V, K, dtype=f32)
    else:
        h = initial_state.to(f32).clone()
    o = torch.empty(B, T, H, V, dtype=f32)
    eye_c = torch.eye(C, dtype=f32)
    eye_k = torch.eye(K, dtype=f32)
    for c0 in range(0, T, C):
        sl = slice(c0, c0 + C)
        qc = q[:, sl].transpose(1, 2)                  # [B,H,C,K]
        kc = k[:, sl].transpose(1, 2)
        vc = v[:, sl].transpose(1, 2)                  # [B,H,C,V]
        bc = beta[:, sl].transpose(1, 2)               # [B,H,C]
        b = g[:, sl].transpose(1, 2).cumsum(-1)        # [B,H,C]
        decay = torch.exp(b[..., :, None] - b[..., None, :])
        gram = kc @ kc.transpose(-1, -2)               # [t,j] = k_t . k_j
        A = torch.tril(gram * decay * bc[..., :, None], -1)
        M = eye_c + A
        rhs_u = vc * bc[..., None]
        rhs_w = kc * (bc * torch.exp(b))[..., None]
        U = torch.linalg.solve_triangular(M, rhs_u, upper=False, unitriangular=True)
        W = torch.linalg.solve_triangular(M, rhs_w, upper=False, unitriangular=True)
        u = U - W @ h.transpose(-1, -2)                # [B,H,C,V]
        scores = torch.tril((qc @ kc.transpose(-1, -2)) * decay)   # j <= t
        oc = scores @ u + (qc * torch.exp(b)[..., None]) @ h.transpose(-1, -2)
        o[:, sl] = oc.transpose(1, 2)
        bC = b[..., -1:]                               # [B,H,1]
        tail = torch.exp(bC - b)[..., None]            # e^{b_C - b_t}
        Wb = W * tail
        Ub = U * tail
        WtK = Wb.transpose(-1, -2) @ kc                # [B,H,K,K]
        P = torch.exp(bC)[..., None] * eye_k - WtK
        h = h @ P + Ub.transpose(-1, -2) @ kc          # [B,H,V,K]
    return o, h


def pad_to_multiple(q, k, v, beta, g, C):
    """Zero-pad T up to a multiple of ``C`` (gdn_ref.py:102-114).

    Pad steps carry q=0 (output 0), beta=0 (state unchanged) and g=0
    (no decay), so outputs on real steps and the final state are unchanged.
    """
    B, T, H, K = q.shape
    V = v.shape[-1]
    Tp = (T + C - 1) // C * C
    if Tp == T:
        return q, k, v, beta, g
    p = Tp - T
    cat = lambda x, shape: torch.cat([x, x.new_zeros(shape)], 1)
    return (cat(q, (B, p, H, K)), cat(k, (B, p, H, K)), cat(v, (B, p, H, V)),
            cat(beta, (B, p, H)), cat(g, (B, p, H)))


def rel_err(ref: torch.Tensor, x: torch.Tensor) -> float:
    """``max|ref - x| / max|ref|`` in float64 (bench_gdn.py:89-94)."""
    ref = ref.detach().to("cpu", torch.float64)
    x = x.detach().to("cpu", torch.float64)
    den = ref.abs().max().item()
    num = (ref - x).abs().max().item()
    if den == 0.0:
        return num
    return num / den


def to_kv(h_vk: torch.Tensor) -> torch.Tensor:
    """[B,H,V,K] (reference layout) -> [B,H,K,V] (product layout)."""
    return h_vk.transpose(-1, -2).contiguous()


def to_vk(h_kv: torch.Tensor) -> torch.Tensor:
    """[B,H,K,V] (product layout) -> [B,H,V,K] (reference layout)."""
    return h_kv.transpose(-1, -2).contiguous()


# ---------------------------------------------------------------------------
# inputs
# ---------------------------------------------------------------------------

def make_inputs_reference(B, T, H, K, V, seed=0, gate_scale=0.1,
                          dtype=torch.float16):
    """The reference harness recipe (bench_gdn.py:33-40), on a CPU generator.

    ``q, k = l2norm(randn)`` cast to ``dtype``; ``v = randn`` cast to
    ``dtype``; ``beta ~ U(0.4, 0.9)`` and ``g ~ -U(0, gate_scale)`` in fp32.
    Draw order q, k, v, beta, g.  (The reference draws on the GPU RNG; a CPU
    generator is used here so the values are reproducible on any host.)
    """
    gen = torch.Generator().manual_seed(seed)
    q = l2norm(torch.randn(B, T, H, K, generator=gen)).to(dtype)
    k = l2norm(torch.randn(B, T, H, K, generator=gen)).to(dtype)
    v = torch.randn(B, T, H, V, generator=gen).to(dtype)
    beta = (torch.rand(B, T, H, generator=gen) * 0.5 + 0.4).float()
    g = (-torch.rand(B, T, H, generator=gen) * gate_scale).float()
    return q, k, v, beta, g


def make_inputs_baseline(B, T, H, K, V, seed=0, dtype=torch.float16,
                         with_h0=False, degenerate=False):
    """The BASELINE.json config recipe, on a CPU generator.

    ``q, k = l2norm(randn)`` then cast to ``dtype``; ``v = randn`` cast to
    ``dtype``; ``beta = sigmoid(randn)``, ``g = logsigmoid(randn)`` (fp32);
    ``h0 = 0.1 randn [B,H,K,V]`` fp32 when ``with_h0``.  Draw order q, k, v,
    beta, g, h0.  ``degenerate`` sets g = 0 and beta = 1 (plain DeltaNet with
    full writes), after the draws.
    Returns ``(q, k, v, g, beta, h0)`` in the product's argument order.
    """
    gen = torch.Generator().manual_seed(seed)
    q = l2norm(torch.randn(B, T, H, K, generator=gen)).to(dtype)
    k = l2norm(torch.randn(B, T, H, K, generator=gen)).to(dtype)
    v = torch.randn(B, T, H, V, generator=gen).to(dtype)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=gen)).float()
    g = torch.nn.functional.logsigmoid(torch.randn(B, T, H, generator=gen)).float()
    h0 = None
    if with_h0:
        h0 = (0.1 * torch.randn(B, H, K, V, generator=gen)).float()
    if degenerate:
        g = torch.zeros_like(g)
        beta = torch.ones_like(beta)
    return q, k, v, g, beta, h0


@dataclass(frozen=True)
class BaselineConfig:
    name: str
    B: int
    T: int
    H: int
    K: int
    V: int
    dtype: torch.dtype
    chunk: int
    with_h0: bool = False


# BASELINE.json "configs", in order.  cfg2 is the headline shape; it is timed
# at C=32 and C=64.
BASELINE_CONFIGS = {
    "cfg0": BaselineConfig("cfg0", 1, 256, 2, 64, 64, torch.float32, 32),
    "cfg1": BaselineConfig("cfg1", 2, 1024, 16, 128, 128, torch.float16, 32),
    "cfg2": BaselineConfig("cfg2", 2, 4096, 16, 128, 128, torch.float16, 32),
    "cfg2_c64": BaselineConfig("cfg2_c64", 2, 4096, 16, 128, 128, torch.float16, 64),
    "cfg3": BaselineConfig("cfg3", 2, 16384, 16, 128, 128, torch.float16, 32),
    "cfg4": BaselineConfig("cfg4", 4, 4096, 16, 128, 128, torch.bfloat16, 32, True),
}


def algorithmic_bytes(B, T, H, K, V, in_bytes, with_h0=False):
    """Compulsory HBM bytes of one forward.

    Per head-token: q, k (K each), v in and o out (V each) at ``in_bytes``,
    plus fp32 beta and g (8 B).  Per (b, h): the fp32 K x V final state,
    and the fp32 h0 when given.
    """
    per_tok = in_bytes * (2 * K + 2 * V) + 8
    per_bh = 4 * K * V * (2 if with_h0 else 1)
    return B * T * H * per_tok + B * H * per_bh


def algorithmic_flops(B, T, H, K, V, C):
    """MFMA-eligible flops of one forward (reassociated state update).

    Per head-token: 4CK (K K^T and Q K^T as full C x C), 2CV (scores x u),
    6KV (W h^T, Q h^T and the K^T u state update).
    """
    return B * T * H * (4 * C * K + 2 * C * V + 6 * K * V)
