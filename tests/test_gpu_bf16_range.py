"""bf16 inputs outside fp16's range.

bf16 q, k, v reach the matrix cores as fp16 operands.  Each workgroup scales
its V-slice of v and h0 by a power of two chosen from their largest
magnitude and scales o and final_state back, which is exact because o and
the state are jointly linear in (v, h0) and every state column evolves on
its own.  These cases would overflow fp16 (|v| up to 1e5 > 65504) or sink
into its subnormals (|v| ~ 1e-6) without it.  Every forward kernel that
takes bf16 is covered (the record + scan launches at C = 32 and C = 64, the
fused pipelined kernel at C = 32, the phase-by-phase kernel), against the fp64 step
recurrence at the north star's 1e-3 (max-norm relative error,
bench_gdn.py:89-94), with fp32-stored outputs.
"""

import pytest
import torch

from oracle import gdn_oracle as ref

pytestmark = pytest.mark.gpu

TOL = 1e-3

CASES = [  # (name, chunk, kernel, K)
    ("records + scan C=32", 32, "auto", 128),
    ("pipelined C=32", 32, "fused", 128),
    ("two-launch C=64", 64, "auto", 64),
    ("phased C=32", 32, "phased", 64),
]


def _inputs(B, T, H, K, V, seed, v_scale, h0_scale):
    q, k, v, g, beta, h0 = ref.make_inputs_baseline(B, T, H, K, V, seed=seed, dtype=torch.float32,
                                                    with_h0=True)
    v = v * v_scale.view(1, 1, -1, 1) if torch.is_tensor(v_scale) else v * v_scale
    h0 = h0 * h0_scale.view(1, -1, 1, 1) if torch.is_tensor(h0_scale) else h0 * h0_scale
    bf = lambda t: t.to(torch.bfloat16)
    return bf(q), bf(k), bf(v), g, beta, h0


def _check(pkg, cuda, name, q, k, v, g, beta, h0, chunk, kernel, per_head=False):
    d = lambda t: t.to(cuda)
    print(f"[bf16 range] {name}", flush=True)
    o, fs = pkg.gdn_fwd(d(q), d(k), d(v), d(g), d(beta), d(h0), chunk_size=chunk, kernel=kernel,
                        output_dtype=torch.float32)
    torch.cuda.synchronize()
    o, fs = o.cpu(), fs.cpu()
    assert torch.isfinite(o).all() and torch.isfinite(fs).all()
    o_ref, h_ref = ref.recurrent(q, k, v, beta, g, ref.to_vk(h0), dtype=torch.float64)
    h_ref = ref.to_kv(h_ref)
    if per_head:  # each head against its own magnitude
        for h in range(q.shape[2]):
            eo = ref.rel_err(o_ref[:, :, h], o[:, :, h])
            eh = ref.rel_err(h_ref[:, h], fs[:, h])
            assert eo <= TOL and eh <= TOL, (h, eo, eh)
    eo, eh = ref.rel_err(o_ref, o), ref.rel_err(h_ref, fs)
    print(f"[bf16 range] {name}: o rel={eo:.3e} state rel={eh:.3e}", flush=True)
    assert eo <= TOL and eh <= TOL


@pytest.mark.parametrize("case", range(len(CASES)))
@pytest.mark.parametrize("v_scale,h0_scale", [(1e5, 1e4), (1e-6, 1e-7), (3e4, 1e-6)])
def test_bf16_extreme_scales(pkg, cuda, case, v_scale, h0_scale):
    """v and h0 far outside fp16's comfortable range, one scale for all."""
    name, chunk, kernel, K = CASES[case]
    q, k, v, g, beta, h0 = _inputs(1, 150, 3, K, 32, 90 + case, v_scale, h0_scale)
    _check(pkg, cuda, f"{name} v*{v_scale:g} h0*{h0_scale:g}", q, k, v, g, beta, h0, chunk, kernel)


@pytest.mark.parametrize("case", range(len(CASES)))
def test_bf16_per_head_scales(pkg, cuda, case):
    """Heads whose v and h0 span 1e-6 .. 1e5: each head is checked against its
    own magnitude (a single shift for all heads could not serve them all)."""
    name, chunk, kernel, K = CASES[case]
    H = 6
    sv = torch.logspace(-6, 5, H)
    q, k, v, g, beta, h0 = _inputs(2, 100, H, K, 32, 95 + case, sv, sv * 0.5)
    _check(pkg, cuda, f"{name} heads 1e-6..1e5", q, k, v, g, beta, h0, chunk, kernel, per_head=True)


@pytest.mark.parametrize("kernel", ["auto", "fused"])
def test_bf16_in_range_unchanged(pkg, cuda, kernel):
    """Inside [2^-6, 2^10] the shift is zero, and bf16 values are exact in
    fp16: the record + scan launches and the fused kernel on bf16 inputs
    then give the bits they give on the same values in fp16."""
    q, k, v, g, beta, h0 = _inputs(1, 200, 2, 128, 32, 97, 1.0, 1.0)
    d = lambda t: t.to(cuda)
    o_b, f_b = pkg.gdn_fwd(d(q), d(k), d(v), d(g), d(beta), d(h0), kernel=kernel,
                           output_dtype=torch.float32)
    h = lambda t: d(t.to(torch.float16))
    o_h, f_h = pkg.gdn_fwd(h(q), h(k), h(v), d(g), d(beta), d(h0), kernel=kernel,
                           output_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(o_b.cpu(), o_h.cpu()) and torch.equal(f_b.cpu(), f_h.cpu())


@pytest.mark.parametrize("case", range(len(CASES)))
@pytest.mark.parametrize("rising", [True, False])
def test_bf16_scale_changes_along_t(pkg, cuda, case, rising):
    """v's magnitude changes by eleven decades at row 100 (1e-6 then 1e5, or
    the reverse), inside the fourth 32-row chunk.

    Rising: every kernel meets the max-norm bound on o and the final state.
    The record + scan launches at C = 32 choose their shift chunk by chunk
    (it only goes down along the sequence), so there the first three
    chunks' outputs also meet it against their own magnitude; the other
    kernels take one shift per slice for the whole sequence, which sinks
    those rows into fp16's subnormals.
    Falling: o meets the max-norm bound.  The decayed final state is eleven
    decades below the state's earlier magnitude, the one that set the shift
    (a shift that went down stays down, and a single shift cannot serve
    both), so it is held to that earlier magnitude: max |error| <= 1e-3
    max |h0|."""
    name, chunk, kernel, K = CASES[case]
    T, t_sw = 200, 100
    lo, hi = 1e-6, 1e5
    prof = torch.full((T,), hi if rising else lo)
    prof[:t_sw] = lo if rising else hi
    q, k, v, g, beta, h0 = ref.make_inputs_baseline(1, T, 2, K, 32, seed=99 + case, dtype=torch.float32,
                                                    with_h0=True)
    v = v * prof.view(1, T, 1, 1)
    h0 = h0 * (lo if rising else hi)
    bf = lambda t: t.to(torch.bfloat16)
    q, k, v = bf(q), bf(k), bf(v)
    d = lambda t: t.to(cuda)
    print(f"[bf16 range] {name} v 1e-6/1e5 {'rising' if rising else 'falling'}", flush=True)
    o, fs = pkg.gdn_fwd(d(q), d(k), d(v), d(g), d(beta), d(h0), chunk_size=chunk, kernel=kernel,
                        output_dtype=torch.float32)
    torch.cuda.synchronize()
    o, fs = o.cpu(), fs.cpu()
    assert torch.isfinite(o).all() and torch.isfinite(fs).all()
    o_ref, h_ref = ref.recurrent(q, k, v, beta, g, ref.to_vk(h0), dtype=torch.float64)
    h_ref = ref.to_kv(h_ref)
    eo = ref.rel_err(o_ref, o)
    if rising:
        eh = ref.rel_err(h_ref, fs)
    else:
        eh = ((h_ref - fs.double()).abs().max() / h0.abs().max()).item()
    print(f"[bf16 range] {name}: o rel={eo:.3e} state err={eh:.3e}", flush=True)
    assert eo <= TOL and eh <= TOL
    if rising and chunk == 32 and kernel == "auto":
        e = ref.rel_err(o_ref[:, :96], o[:, :96])
        print(f"[bf16 range] {name} rows before the change: o rel={e:.3e}", flush=True)
        assert e <= TOL
