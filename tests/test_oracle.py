"""CPU tests that pin the oracle (oracle/gdn_oracle.py) before it is trusted.

Each check is chosen so that a plausible slip in the restatement -- decay
applied after the projection, a dropped beta, a transposed state, a wrong
mask diagonal, a missing e^{b_C} -- fails at least one of them:

* exact-rational golden vectors of the definition (tests/golden),
* closed forms: T=1, beta=0, orthonormal keys with g=0/beta=1, and the delta
  "write" property h_t k_t = v_t for beta=1 and unit keys,
* invariants: joint linearity in (v, h0), segment composability through the
  carried state, zero-padding, head permutation,
* two independent algorithms agree: the step recurrence and the chunked UT
  transform with triangular solves, on the reference's own self-check case
  (gdn_ref.py:117-132) and with a non-zero initial state.
"""

import json
import math
import os

import pytest
import torch

from oracle import gdn_oracle as ref

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "gdn_exact.json")


def _golden_cases():
    with open(GOLDEN) as f:
        return json.load(f)["cases"]


def _as_bthd(rows):
    """[T][D] -> [1, T, 1, D] float64."""
    return torch.tensor(rows, dtype=torch.float64)[None, :, None, :]


def _as_bth(vals):
    return torch.tensor(vals, dtype=torch.float64)[None, :, None]


@pytest.mark.parametrize("case", _golden_cases(), ids=lambda c: c["name"])
def test_recurrent_matches_exact_golden(case):
    q, k, v = _as_bthd(case["q"]), _as_bthd(case["k"]), _as_bthd(case["v"])
    beta, g = _as_bth(case["beta"]), _as_bth(case["g"])
    h0 = torch.tensor(case["h0_vk"], dtype=torch.float64)[None, None]
    o, h = ref.recurrent(q, k, v, beta, g, h0, dtype=torch.float64)
    o_exp = _as_bthd(case["o"])
    h_exp = torch.tensor(case["h_vk"], dtype=torch.float64)[None, None]
    assert torch.allclose(o, o_exp, rtol=1e-12, atol=1e-13)
    assert torch.allclose(h, h_exp, rtol=1e-12, atol=1e-13)


@pytest.mark.parametrize("case", [c for c in _golden_cases() if c["T"] % 2 == 0],
                         ids=lambda c: c["name"])
def test_chunked_matches_exact_golden(case):
    q, k, v = _as_bthd(case["q"]), _as_bthd(case["k"]), _as_bthd(case["v"])
    beta, g = _as_bth(case["beta"]), _as_bth(case["g"])
    h0 = torch.tensor(case["h0_vk"], dtype=torch.float64)[None, None]
    o, h = ref.chunked_ut(q, k, v, beta, g, C=2, initial_state=h0)
    assert ref.rel_err(_as_bthd(case["o"]), o) < 1e-6
    assert ref.rel_err(torch.tensor(case["h_vk"])[None, None], h) < 1e-6


def test_golden_fixture_is_exact_definition():
    """The fixture's generator is pure Python; re-derive one value by hand:
    T=1, h0 given -> o_0 = h_1 q_0 with h_1 = g h0 + beta (v - g h0 k) k^T."""
    c = _golden_cases()[0]
    K, V = c["K"], c["V"]
    gam, b = c["gamma"][0], c["beta"][0]
    h0 = c["h0_vk"]
    k0, v0, q0 = c["k"][0], c["v"][0], c["q"][0]
    hd = [[gam * h0[i][j] for j in range(K)] for i in range(V)]
    u = [b * (v0[i] - sum(hd[i][j] * k0[j] for j in range(K))) for i in range(V)]
    h1 = [[hd[i][j] + u[i] * k0[j] for j in range(K)] for i in range(V)]
    o0 = [sum(h1[i][j] * q0[j] for j in range(K)) for i in range(V)]
    assert all(abs(a - e) < 1e-12 for a, e in zip(o0, c["o"][0]))


# --------------------------------------------------------------------------
# closed forms
# --------------------------------------------------------------------------

def test_single_step_zero_state_closed_form():
    """T=1, h0=0: o_0 = beta (k.q) v and h_1 = beta v k^T (K != V)."""
    gen = torch.Generator().manual_seed(0)
    B, H, K, V = 2, 3, 5, 7
    q = torch.randn(B, 1, H, K, generator=gen, dtype=torch.float64)
    k = torch.randn(B, 1, H, K, generator=gen, dtype=torch.float64)
    v = torch.randn(B, 1, H, V, generator=gen, dtype=torch.float64)
    beta = torch.rand(B, 1, H, generator=gen, dtype=torch.float64)
    g = -torch.rand(B, 1, H, generator=gen, dtype=torch.float64)
    o, h = ref.recurrent(q, k, v, beta, g)
    kq = (k * q).sum(-1, keepdim=True)
    assert torch.allclose(o, beta[..., None] * kq * v, atol=1e-14)
    h_exp = beta[:, 0, :, None, None] * v[:, 0, :, :, None] * k[:, 0, :, None, :]
    assert h.shape == (B, H, V, K)
    assert torch.allclose(h, h_exp, atol=1e-14)


def test_zero_beta_is_pure_decay():
    """beta = 0: h_T = e^{sum g} h0 and o_t = e^{b_t} h0 q_t."""
    gen = torch.Generator().manual_seed(1)
    B, T, H, K, V = 1, 9, 2, 4, 6
    q = torch.randn(B, T, H, K, generator=gen, dtype=torch.float64)
    k = torch.randn(B, T, H, K, generator=gen, dtype=torch.float64)
    v = torch.randn(B, T, H, V, generator=gen, dtype=torch.float64)
    g = -torch.rand(B, T, H, generator=gen, dtype=torch.float64)
    h0 = torch.randn(B, H, V, K, generator=gen, dtype=torch.float64)
    o, h = ref.recurrent(q, k, v, torch.zeros(B, T, H, dtype=torch.float64), g, h0)
    b = g.cumsum(1)
    o_exp = torch.exp(b)[..., None] * torch.einsum("bhvk,bthk->bthv", h0, q)
    assert torch.allclose(o, o_exp, atol=1e-13)
    assert torch.allclose(h, torch.exp(b[:, -1])[..., None, None] * h0, atol=1e-13)


def test_orthonormal_keys_no_gate_full_write():
    """g=0, beta=1, h0=0, k_t = e_t: A = 0, so o_t = sum_{j<=t} v_j q_t[j]
    and h = [v_0 ... v_{T-1} 0 ...] column by column."""
    gen = torch.Generator().manual_seed(2)
    T, K, V = 6, 8, 3
    k = torch.eye(K, dtype=torch.float64)[:T][None, :, None, :]
    q = torch.randn(1, T, 1, K, generator=gen, dtype=torch.float64)
    v = torch.randn(1, T, 1, V, generator=gen, dtype=torch.float64)
    ones = torch.ones(1, T, 1, dtype=torch.float64)
    o, h = ref.recurrent(q, k, v, ones, torch.zeros_like(ones))
    for t in range(T):
        exp = sum(v[0, j, 0] * q[0, t, 0, j] for j in range(t + 1))
        assert torch.allclose(o[0, t, 0], exp, atol=1e-14)
    h_exp = torch.zeros(V, K, dtype=torch.float64)
    h_exp[:, :T] = v[0, :, 0].T
    assert torch.allclose(h[0, 0], h_exp, atol=1e-14)
    # the chunked form agrees on the same closed form
    o2, h2 = ref.chunked_ut(q, k, v, ones, torch.zeros_like(ones), C=3)
    assert ref.rel_err(o, o2) < 1e-6 and ref.rel_err(h, h2) < 1e-6


@pytest.mark.parametrize("algo", ["recurrent", "chunked"])
def test_delta_write_property(algo):
    """beta_t = 1 and |k_t| = 1 make step t write v_t exactly: h_t k_t = v_t.
    With q = k the output is therefore o_t = v_t for any gates and h0."""
    gen = torch.Generator().manual_seed(3)
    B, T, H, K, V = 2, 16, 2, 8, 5
    k = ref.l2norm(torch.randn(B, T, H, K, generator=gen, dtype=torch.float64))
    v = torch.randn(B, T, H, V, generator=gen, dtype=torch.float64)
    g = torch.nn.functional.logsigmoid(torch.randn(B, T, H, generator=gen, dtype=torch.float64))
    h0 = torch.randn(B, H, V, K, generator=gen, dtype=torch.float64)
    ones = torch.ones(B, T, H, dtype=torch.float64)
    if algo == "recurrent":
        o, _ = ref.recurrent(k, k, v, ones, g, h0)
        tol = 1e-6  # l2norm's eps makes |k| = 1 - O(1e-7)
    else:
        o, _ = ref.chunked_ut(k, k, v, ones, g, C=8, initial_state=h0)
        tol = 1e-4
    assert ref.rel_err(v, o) < tol


# --------------------------------------------------------------------------
# invariants
# --------------------------------------------------------------------------

def _rand_case(seed, B=1, T=24, H=2, K=6, V=4):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, K, generator=gen, dtype=torch.float64)
    k = ref.l2norm(torch.randn(B, T, H, K, generator=gen, dtype=torch.float64))
    v = torch.randn(B, T, H, V, generator=gen, dtype=torch.float64)
    beta = torch.rand(B, T, H, generator=gen, dtype=torch.float64)
    g = -0.2 * torch.rand(B, T, H, generator=gen, dtype=torch.float64)
    h0 = torch.randn(B, H, V, K, generator=gen, dtype=torch.float64)
    return q, k, v, beta, g, h0


def test_joint_linearity_in_v_and_h0():
    q, k, v1, beta, g, h01 = _rand_case(4)
    _, _, v2, _, _, h02 = _rand_case(5)
    a, b = 0.7, -1.3
    o1, s1 = ref.recurrent(q, k, v1, beta, g, h01)
    o2, s2 = ref.recurrent(q, k, v2, beta, g, h02)
    o3, s3 = ref.recurrent(q, k, a * v1 + b * v2, beta, g, a * h01 + b * h02)
    assert torch.allclose(o3, a * o1 + b * o2, atol=1e-12)
    assert torch.allclose(s3, a * s1 + b * s2, atol=1e-12)


@pytest.mark.parametrize("algo", ["recurrent", "chunked"])
def test_segment_composability(algo):
    """Running [0, T1) then [T1, T) from the carried state equals one run."""
    q, k, v, beta, g, h0 = _rand_case(6, T=32)
    run = (lambda *a, h=None: ref.recurrent(*a, h)) if algo == "recurrent" else \
        (lambda *a, h=None: ref.chunked_ut(*a, C=8, initial_state=h))
    o, h = run(q, k, v, beta, g, h=h0)
    T1 = 16
    oa, ha = run(q[:, :T1], k[:, :T1], v[:, :T1], beta[:, :T1], g[:, :T1], h=h0)
    ob, hb = run(q[:, T1:], k[:, T1:], v[:, T1:], beta[:, T1:], g[:, T1:], h=ha)
    assert ref.rel_err(o, torch.cat([oa, ob], 1)) < 1e-6
    assert ref.rel_err(h, hb) < 1e-6


def test_zero_padding_is_neutral():
    """Pad steps (q=0, beta=0, g=0) leave outputs and the final state alone
    (gdn_ref.py:102-103)."""
    q, k, v, beta, g, h0 = _rand_case(7, T=21)
    o, h = ref.recurrent(q, k, v, beta, g, h0)
    qp, kp, vp, bp, gp = ref.pad_to_multiple(q, k, v, beta, g, 8)
    assert qp.shape[1] == 24
    op, hp = ref.recurrent(qp, kp, vp, bp, gp, h0)
    assert torch.allclose(op[:, :21], o, atol=1e-13)
    assert torch.all(op[:, 21:] == 0)
    assert torch.allclose(hp, h, atol=1e-13)
    oc, hc = ref.chunked_ut(qp, kp, vp, bp, gp, C=8, initial_state=h0)
    assert ref.rel_err(o, oc[:, :21]) < 1e-6 and ref.rel_err(h, hc) < 1e-6


def test_head_permutation_equivariance():
    q, k, v, beta, g, h0 = _rand_case(8, H=3)
    perm = torch.tensor([2, 0, 1])
    o, h = ref.recurrent(q, k, v, beta, g, h0)
    op, hp = ref.recurrent(q[:, :, perm], k[:, :, perm], v[:, :, perm], beta[:, :, perm],
                           g[:, :, perm], h0[:, perm])
    assert torch.allclose(op, o[:, :, perm], atol=1e-14)
    assert torch.allclose(hp, h[:, perm], atol=1e-14)


# --------------------------------------------------------------------------
# recurrence vs chunked UT (two independent algorithms)
# --------------------------------------------------------------------------

def test_reference_self_check_case():
    """gdn_ref.py:117-132: torch.manual_seed(0), B2 T128 H3 K=V=64, C=32,
    beta ~ U(0.4,0.9), g ~ -U(0,0.1).  The reference asserts max-abs < 1e-3
    and its README reports ~4e-7 agreement; the CPU generator seeded 0
    reproduces the same draws in the same order."""
    q, k, v, beta, g = ref.make_inputs_reference(2, 128, 3, 64, 64, seed=0, gate_scale=0.1,
                                                 dtype=torch.float32)
    torch.manual_seed(0)
    q2 = ref.l2norm(torch.randn(2, 128, 3, 64))
    assert torch.equal(q, q2)
    o1, h1 = ref.recurrent(q, k, v, beta, g, dtype=torch.float32)
    o2, h2 = ref.chunked_ut(q, k, v, beta, g, C=32)
    assert (o1 - o2).abs().max().item() < 1e-5
    assert (h1 - h2).abs().max().item() < 1e-5


@pytest.mark.parametrize("C", [32, 64])
def test_chunked_vs_fp64_recurrence_baseline_inputs(C):
    """configs[0] recipe (fp32, B1 H2 T256 K=V=64) plus a non-zero h0."""
    q, k, v, g, beta, _ = ref.make_inputs_baseline(1, 256, 2, 64, 64, seed=0, dtype=torch.float32)
    h0 = 0.1 * torch.randn(1, 2, 64, 64, generator=torch.Generator().manual_seed(9))
    o64, h64 = ref.recurrent(q, k, v, beta, g, h0, dtype=torch.float64)
    oc, hc = ref.chunked_ut(q, k, v, beta, g, C=C, initial_state=h0)
    assert ref.rel_err(o64, oc) < 1e-5
    assert ref.rel_err(h64, hc) < 1e-5


def test_chunk_sizes_agree_mild_gates_k_ne_v():
    q, k, v, beta, g = ref.make_inputs_reference(1, 128, 2, 32, 48, seed=3, gate_scale=0.1,
                                                 dtype=torch.float32)
    o32, h32 = ref.chunked_ut(q, k, v, beta, g, C=32)
    o64, h64 = ref.chunked_ut(q, k, v, beta, g, C=64)
    assert h32.shape == (1, 2, 48, 32)
    assert ref.rel_err(o32, o64) < 1e-5 and ref.rel_err(h32, h64) < 1e-5


def test_chunked_requires_multiple_of_chunk():
    q, k, v, beta, g, _ = _rand_case(10, T=10)
    with pytest.raises(ValueError):
        ref.chunked_ut(q, k, v, beta, g, C=8)


# --------------------------------------------------------------------------
# metric, inputs, roofline arithmetic
# --------------------------------------------------------------------------

def test_rel_err_metric():
    r = torch.tensor([1.0, -4.0, 2.0])
    x = torch.tensor([1.5, -4.0, 2.0])
    assert ref.rel_err(r, x) == pytest.approx(0.5 / 4.0)
    assert ref.rel_err(torch.zeros(3), torch.zeros(3)) == 0.0


def test_baseline_inputs_recipe():
    q, k, v, g, beta, h0 = ref.make_inputs_baseline(2, 64, 3, 32, 16, seed=0,
                                                    dtype=torch.bfloat16, with_h0=True)
    assert q.dtype == k.dtype == v.dtype == torch.bfloat16
    assert g.dtype == beta.dtype == h0.dtype == torch.float32
    assert h0.shape == (2, 3, 32, 16)
    n = q.float().norm(dim=-1)
    assert torch.allclose(n, torch.ones_like(n), atol=1e-2)
    assert torch.all(g < 0) and torch.all((beta > 0) & (beta < 1))
    *_, gd, bd, _ = ref.make_inputs_baseline(1, 8, 1, 32, 16, degenerate=True)
    assert torch.all(gd == 0) and torch.all(bd == 1)
    # same seed -> same values
    q2 = ref.make_inputs_baseline(2, 64, 3, 32, 16, seed=0, dtype=torch.bfloat16)[0]
    assert torch.equal(q, q2)


def test_roofline_arithmetic_matches_baseline_md():
    """cfg2 moves 137.4 MB (17.17 us at 8 TB/s) and does
    16.11 GFLOP at C=32 (122,880 flop per head-token)."""
    by = ref.algorithmic_bytes(2, 4096, 16, 128, 128, 2)
    assert by == 2 * 4096 * 16 * 1032 + 2 * 16 * 4 * 128 * 128
    assert by / 8e12 * 1e6 == pytest.approx(17.17, abs=0.01)
    assert ref.algorithmic_flops(1, 1, 1, 128, 128, 32) == 122880
    assert ref.algorithmic_flops(1, 1, 1, 128, 128, 64) == 147456
    assert ref.algorithmic_bytes(4, 4096, 16, 128, 128, 2, with_h0=True) / 1e6 == \
        pytest.approx(278.9, abs=0.1)


# --------------------------------------------------------------------------
# input preparation: l2norm (gdn_ref.py:24-25) and the gate activations
# --------------------------------------------------------------------------

def test_l2norm_closed_form_norm():
    """|l2norm(x)| = |x| / sqrt(|x|^2 + eps) (eps inside the sqrt), to fp32
    accuracy: the reference squares and sums in fp32 (``x.float()``) whatever
    x's dtype."""
    x = torch.randn(3, 5, 2, 64, generator=torch.Generator().manual_seed(4), dtype=torch.float64)
    ss = (x * x).sum(-1)
    y = ref.l2norm(x)
    assert torch.allclose(y.norm(dim=-1), ss.sqrt() / (ss + 1e-6).sqrt(), rtol=1e-6, atol=0)
    xs = x * 1e-4   # |x|^2 ~ 6e-7, comparable to eps
    ss = (xs * xs).sum(-1)
    assert torch.allclose(ref.l2norm(xs).norm(dim=-1), ss.sqrt() / (ss + 1e-6).sqrt(),
                          rtol=1e-6, atol=0)


def test_l2norm_eps_inside_sqrt_and_zero_rows():
    """A row with |x|^2 = eps is halved in norm by sqrt(2) (eps under the root,
    not added to the root); an all-zero row stays zero (no NaN)."""
    x = torch.zeros(1, 1, 2, 32, dtype=torch.float64)
    x[0, 0, 0, 0] = 1e-3
    y = ref.l2norm(x)
    assert abs(y[0, 0, 0, 0].item() - 1e-3 / math.sqrt(2e-6)) < 1e-6   # 0.7071, not 0.999
    assert torch.equal(y[0, 0, 1], torch.zeros(32, dtype=torch.float64))


def test_l2norm_fp16_rounds_the_denominator():
    """gdn_ref.py:25 casts sqrt(sum + eps) to x.dtype before dividing.  On
    fp16 rows where that rounding changes the quotient, the oracle matches the
    rounded-denominator quotient and not the fp32 one (values computed here
    with numpy's own float16 arithmetic)."""
    import numpy as np
    gen = torch.Generator().manual_seed(11)
    x = torch.randn(4096, 8, generator=gen).to(torch.float16)
    y = ref.l2norm(x).numpy()
    xn = x.numpy().astype(np.float64)
    den32 = np.sqrt((xn * xn).sum(-1, keepdims=True).astype(np.float32) + np.float32(1e-6))
    rounded = (x.numpy() / den32.astype(np.float16)).astype(np.float16)
    unrounded = (xn / den32.astype(np.float64)).astype(np.float16)
    differ = rounded != unrounded
    assert differ.sum() > 50
    assert np.array_equal(y[differ], rounded[differ])


def test_sigmoid_logsigmoid_closed_forms():
    x = torch.tensor([-1000.0, -30.0, -2.5, -1e-8, 0.0, 1e-8, 0.7, 30.0, 1000.0], dtype=torch.float64)
    s = ref.sigmoid(x)
    ls = ref.logsigmoid(x)
    assert s[4].item() == 0.5 and ls[4].item() == -math.log(2.0)
    assert torch.allclose(s + ref.sigmoid(-x), torch.ones_like(x), rtol=0, atol=1e-15)
    assert torch.allclose(s, torch.sigmoid(x), rtol=1e-15, atol=0)
    assert torch.isfinite(ls).all()
    assert ls[0].item() == -1000.0 and ls[-1].item() == 0.0
    mid = slice(1, 7)   # where log(sigmoid) is itself accurate
    assert torch.allclose(ls[mid], torch.log(s[mid]), rtol=1e-14, atol=1e-300)
    # log sigmoid(x) - log sigmoid(-x) = x
    assert torch.allclose(ls - ref.logsigmoid(-x), x, rtol=1e-14, atol=1e-12)


def test_prep_inputs_matches_baseline_recipe():
    """The BASELINE recipe draws q, k, v, beta, g and applies l2norm, sigmoid
    and logsigmoid; prep_inputs on the same raw draws gives the same values."""
    B, T, H, K, V = 1, 64, 2, 32, 32
    q, k, v, g, beta, _ = ref.make_inputs_baseline(B, T, H, K, V, seed=5, dtype=torch.float32)
    gen = torch.Generator().manual_seed(5)
    qr = torch.randn(B, T, H, K, generator=gen)
    kr = torch.randn(B, T, H, K, generator=gen)
    torch.randn(B, T, H, V, generator=gen)
    br = torch.randn(B, T, H, generator=gen)
    gr = torch.randn(B, T, H, generator=gen)
    qp, kp, bp, gp = ref.prep_inputs(qr, kr, br, gr)
    assert torch.equal(qp, q) and torch.equal(kp, k)
    assert torch.allclose(bp, beta, rtol=2e-7, atol=0)
    assert torch.allclose(gp, g, rtol=2e-7, atol=1e-7)


# --------------------------------------------------------------------------
# backward: the chunked restatement vs reverse-mode differentiation
# --------------------------------------------------------------------------

@pytest.mark.parametrize("T,K,V,gate,seed", [(64, 16, 8, 1.0, 0), (77, 32, 16, 1.0, 1),
                                             (33, 16, 16, 1.0, 2), (96, 32, 8, 3.0, 3),
                                             (5, 8, 4, 1.0, 4)])
def test_chunked_bwd_matches_autograd(T, K, V, gate, seed):
    """Two independent routes to the gradients (the chunked algebra with
    triangular solves, and autograd through the step recurrence) agree to
    fp64 rounding, including partial last chunks and strong decay."""
    gen = torch.Generator().manual_seed(seed)
    B, H = 1, 2
    q = ref.l2norm(torch.randn(B, T, H, K, generator=gen, dtype=torch.float64))
    k = ref.l2norm(torch.randn(B, T, H, K, generator=gen, dtype=torch.float64))
    v = torch.randn(B, T, H, V, generator=gen, dtype=torch.float64)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=gen, dtype=torch.float64))
    g = gate * torch.nn.functional.logsigmoid(torch.randn(B, T, H, generator=gen, dtype=torch.float64))
    h0 = 0.1 * torch.randn(B, H, K, V, generator=gen, dtype=torch.float64)
    do = torch.randn(B, T, H, V, generator=gen, dtype=torch.float64)
    dfin = torch.randn(B, H, K, V, generator=gen, dtype=torch.float64)
    auto = ref.recurrent_grads(q, k, v, beta, g, h0, do, dfin, scale=0.7)
    mine = ref.chunked_bwd(q, k, v, beta, g, h0, do, dfin, scale=0.7)
    for name, a, b in zip(("dq", "dk", "dv", "dbeta", "dg", "dh0"), mine, auto):
        assert ref.rel_err(b, a) < 1e-10, name


def test_recurrent_grads_finite_difference():
    """Spot-check recurrent_grads against central differences (fp64)."""
    gen = torch.Generator().manual_seed(6)
    B, T, H, K, V = 1, 9, 1, 4, 3
    q = torch.randn(B, T, H, K, generator=gen, dtype=torch.float64)
    k = ref.l2norm(torch.randn(B, T, H, K, generator=gen, dtype=torch.float64))
    v = torch.randn(B, T, H, V, generator=gen, dtype=torch.float64)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=gen, dtype=torch.float64))
    g = torch.nn.functional.logsigmoid(torch.randn(B, T, H, generator=gen, dtype=torch.float64))
    do = torch.randn(B, T, H, V, generator=gen, dtype=torch.float64)
    grads = ref.recurrent_grads(q, k, v, beta, g, None, do, None, scale=1.3)

    def loss(gg):
        o, _ = ref.recurrent(q, k, v, beta, gg, dtype=torch.float64)
        return (1.3 * o * do).sum().item()

    eps = 1e-6
    for t in (0, 4, 8):
        gp, gm = g.clone(), g.clone()
        gp[0, t, 0] += eps
        gm[0, t, 0] -= eps
        fd = (loss(gp) - loss(gm)) / (2 * eps)
        assert abs(fd - grads[4][0, t, 0].item()) < 1e-6 * max(1.0, abs(fd))
