"""Write ``gdn_exact.json``: exact-arithmetic GDN vectors for tiny cases.

The reference ships no golden vectors (its checks are tolerances in
gdn_ref.py:117-132 and bench_gdn.py:84-99).  These fixtures evaluate the
definition (gdn_ref.py:3-9; the V x K state h)

    h_t = gamma_t h_{t-1} + u_t k_t^T
    u_t = beta_t (v_t - gamma_t h_{t-1} k_t)
    o_t = h_t q_t

in exact rational arithmetic (``fractions.Fraction``) on dyadic inputs, so
every input is an exact float and every expected value is the correctly
rounded float64 of the exact answer.  The gate is given as
``gamma_t = e^{g_t}``; the fixture stores ``g_t = log(gamma_t)`` (float64)
next to ``gamma_t``.

Run: ``python tests/golden/make_golden.py`` (pure Python, no torch).
"""

import json
import math
import os
import random
from fractions import Fraction as F

HERE = os.path.dirname(os.path.abspath(__file__))


def run_exact(q, k, v, beta, gamma, h0):
    """q, k: [T][K]; v: [T][V]; beta, gamma: [T]; h0: [V][K] (Fractions)."""
    T, K, V = len(q), len(q[0]), len(v[0])
    h = [row[:] for row in h0]
    outs = []
    for t in range(T):
        hd = [[gamma[t] * h[i][j] for j in range(K)] for i in range(V)]
        hk = [sum(hd[i][j] * k[t][j] for j in range(K)) for i in range(V)]
        u = [beta[t] * (v[t][i] - hk[i]) for i in range(V)]
        h = [[hd[i][j] + u[i] * k[t][j] for j in range(K)] for i in range(V)]
        outs.append([sum(h[i][j] * q[t][j] for j in range(K)) for i in range(V)])
    return outs, h


def dyadic(rng, lo=-8, hi=8, den=8):
    return F(rng.randint(lo, hi), den)


def make_case(name, T, K, V, seed, with_h0, gammas=None, betas=None):
    rng = random.Random(seed)
    q = [[dyadic(rng) for _ in range(K)] for _ in range(T)]
    k = [[dyadic(rng, -4, 4, 4) for _ in range(K)] for _ in range(T)]
    v = [[dyadic(rng) for _ in range(V)] for _ in range(T)]
    beta = betas or [F(rng.randint(1, 7), 8) for _ in range(T)]
    gamma = gammas or [F(rng.choice([4, 6, 7, 8]), 8) for _ in range(T)]
    h0 = [[dyadic(rng, -4, 4, 16) if with_h0 else F(0) for _ in range(K)] for _ in range(V)]
    o, h = run_exact(q, k, v, beta, gamma, h0)
    fl = lambda m: [[float(x) for x in row] for row in m]
    return {
        "name": name, "T": T, "K": K, "V": V,
        "q": fl(q), "k": fl(k), "v": fl(v),
        "beta": [float(x) for x in beta],
        "gamma": [float(x) for x in gamma],
        "g": [math.log(float(x)) for x in gamma],
        "h0_vk": fl(h0),
        "o": fl(o), "h_vk": fl(h),
    }


def main():
    cases = [
        make_case("k3v2_t5_h0", T=5, K=3, V=2, seed=1, with_h0=True),
        make_case("k2v3_t4_zero_h0", T=4, K=2, V=3, seed=2, with_h0=False),
        make_case("k4v4_t6_h0", T=6, K=4, V=4, seed=3, with_h0=True),
        make_case("k3v2_t4_nogate_fullwrite", T=4, K=3, V=2, seed=4, with_h0=True,
                  gammas=[F(1)] * 4, betas=[F(1)] * 4),
    ]
    path = os.path.join(HERE, "gdn_exact.json")
    with open(path, "w") as f:
        json.dump({"source": "tests/golden/make_golden.py (exact Fractions, definition "
                             "gdn_ref.py:3-9)", "cases": cases}, f, indent=1)
    print("wrote", path)


if __name__ == "__main__":
    main()
