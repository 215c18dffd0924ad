"""GPU tests of FLA's keyword surface and the packed-sequence (varlen) form.

``chunk_gated_delta_rule`` (FLA 0.6.0's name and keywords, called by the
reference at bench_gdn.py:169-172) and ``gdn_fwd(..., cu_seqlens=...)`` run
the same kernels as ``gdn_fwd``: per sequence the arithmetic is the same, so
packed runs are compared bit for bit with separate runs, and every sequence
with the fp64 step recurrence of the oracle (<= 1e-3, bench_gdn.py:89-94).
"""

import pytest
import torch

from oracle import gdn_oracle as ref

pytestmark = pytest.mark.gpu

TOL_LOWP = 1e-3


def _tol_stored(dtype):
    """1e-3 for the kernel's fp32 result plus one rounding to o's storage dtype."""
    return TOL_LOWP + (2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11)


def _recurrent(q, k, v, g, beta, h0, scale=1.0):
    o, h = ref.recurrent(q, k, v, beta, g, None if h0 is None else ref.to_vk(h0),
                         dtype=torch.float64)
    return o * scale, ref.to_kv(h)


def _packed_inputs(lens, H, K, V, dtype, seed):
    T = sum(lens)
    q, k, v, g, beta, _ = ref.make_inputs_baseline(1, T, H, K, V, seed=seed, dtype=dtype)
    h0 = 0.1 * torch.randn(len(lens), H, K, V, generator=torch.Generator().manual_seed(seed + 1))
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0).tolist()), dtype=torch.int64)
    return q, k, v, g, beta, h0, cu


@pytest.mark.parametrize("kernel,C", [("auto", 32), ("phased", 32), ("auto", 64)])
@pytest.mark.parametrize("dtype,K,V,bv", [(torch.float16, 64, 64, 16), (torch.bfloat16, 128, 32, 32),
                                          (torch.float16, 32, 48, 16)])
def test_varlen_equals_separate_runs(pkg, cuda, kernel, C, dtype, K, V, bv):
    """C=64 'auto' is the two-launch path (record + scan)."""
    lens = [37, 0, 1, 32, 100, 64, 5, 129]
    H = 2
    q, k, v, g, beta, h0, cu = _packed_inputs(lens, H, K, V, dtype, seed=21)
    d = lambda t: t.to(cuda)
    print(f"[varlen] {dtype} K={K} V={V} bv={bv} kernel={kernel} C={C} lens={lens}", flush=True)
    o, fs = pkg.gdn_fwd(d(q), d(k), d(v), d(g), d(beta), d(h0), scale=0.5, block_v=bv,
                        kernel=kernel, cu_seqlens=d(cu), chunk_size=C)
    torch.cuda.synchronize()
    o, fs = o.cpu(), fs.cpu()
    assert o.shape == (1, sum(lens), H, V) and fs.shape == (len(lens), H, K, V)
    for i, (a, b) in enumerate(zip(cu[:-1].tolist(), cu[1:].tolist())):
        sl = lambda t: t[:, a:b].contiguous()
        oi, fi = pkg.gdn_fwd(d(sl(q)), d(sl(k)), d(sl(v)), d(sl(g)), d(sl(beta)),
                             d(h0[i:i + 1].contiguous()), scale=0.5, block_v=bv, kernel=kernel,
                             chunk_size=C)
        torch.cuda.synchronize()
        assert torch.equal(o[:, a:b], oi.cpu()), f"sequence {i}: o differs from a separate run"
        assert torch.equal(fs[i:i + 1], fi.cpu()), f"sequence {i}: state differs"
        o_ref, h_ref = _recurrent(sl(q), sl(k), sl(v), sl(g), sl(beta), h0[i:i + 1], scale=0.5)
        eh = ref.rel_err(h_ref, fs[i:i + 1])
        assert eh <= TOL_LOWP, (i, eh)
        if b > a:
            eo = ref.rel_err(o_ref, o[:, a:b])
            assert eo <= _tol_stored(dtype), (i, eo)


def test_varlen_full_size_equals_batched(pkg, cuda):
    """cfg2's two 4096-token sequences packed into one batch of 8192 rows
    give the batched run's results bit for bit (same kernel, same slices)."""
    q, k, v, g, beta, _ = ref.make_inputs_baseline(2, 4096, 16, 128, 128, seed=0)
    d = lambda t: t.to(cuda)
    print("[varlen] cfg2 packed vs batched", flush=True)
    o_b, fs_b = pkg.gdn_fwd(d(q), d(k), d(v), d(g), d(beta), block_v=16)
    pack = lambda t: t.reshape(1, 2 * 4096, *t.shape[2:])
    cu = torch.tensor([0, 4096, 8192], dtype=torch.int64, device=cuda)
    o_p, fs_p = pkg.gdn_fwd(d(pack(q)), d(pack(k)), d(pack(v)), d(pack(g)), d(pack(beta)),
                            block_v=16, cu_seqlens=cu)
    torch.cuda.synchronize()
    assert torch.equal(o_p.reshape(o_b.shape), o_b)
    assert torch.equal(fs_p, fs_b)


def test_fla_defaults_and_head_first(pkg, cuda):
    B, T, H, K, V = 2, 200, 3, 64, 64
    q, k, v, g, beta, h0 = ref.make_inputs_baseline(B, T, H, K, V, seed=3, with_h0=True)
    d = lambda t: t.to(cuda)
    print("[fla] defaults, head_first", flush=True)
    o, fs = pkg.chunk_gated_delta_rule(q=d(q), k=d(k), v=d(v), g=d(g), beta=d(beta),
                                       initial_state=d(h0), output_final_state=True)
    o2, fs2 = pkg.gdn_fwd(d(q), d(k), d(v), d(g), d(beta), d(h0), scale=K ** -0.5)
    assert torch.equal(o, o2) and torch.equal(fs, fs2)
    o3, none = pkg.chunk_gated_delta_rule(d(q), d(k), d(v), d(g), d(beta), scale=1.0)
    assert none is None
    hf = lambda t: t.transpose(1, 2).contiguous()
    o4, fs4 = pkg.chunk_gated_delta_rule(d(hf(q)), d(hf(k)), d(hf(v)), d(hf(g)), d(hf(beta)),
                                         initial_state=d(h0), output_final_state=True,
                                         head_first=True)
    torch.cuda.synchronize()
    assert o4.shape == (B, H, T, V) and o4.is_contiguous()
    assert torch.equal(o4.transpose(1, 2), o) and torch.equal(fs4, fs)
    o_ref, h_ref = _recurrent(q, k, v, g, beta, h0, scale=K ** -0.5)
    assert ref.rel_err(o_ref, o.cpu()) <= _tol_stored(o.dtype)
    assert ref.rel_err(h_ref, fs.cpu()) <= TOL_LOWP
    o_ref1, _ = _recurrent(q, k, v, g, beta, None)
    assert ref.rel_err(o_ref1, o3.cpu()) <= _tol_stored(o3.dtype)


def test_fla_varlen_with_l2norm_in_kernel(pkg, cuda):
    """FLA's varlen call with use_qk_l2norm_in_kernel: raw q, k are
    normalised by the fused preparation, then the packed forward runs."""
    lens = [50, 96, 33]
    H, K, V = 2, 128, 64
    T = sum(lens)
    gen = torch.Generator().manual_seed(8)
    qr = (3 * torch.randn(1, T, H, K, generator=gen)).half()
    kr = (0.2 * torch.randn(1, T, H, K, generator=gen)).half()
    v = torch.randn(1, T, H, V, generator=gen).half()
    beta = torch.sigmoid(torch.randn(1, T, H, generator=gen))
    g = torch.nn.functional.logsigmoid(torch.randn(1, T, H, generator=gen))
    h0 = 0.1 * torch.randn(len(lens), H, K, V, generator=gen)
    cu = torch.tensor([0, 50, 146, 179], dtype=torch.int64)
    d = lambda t: t.to(cuda)
    print("[fla] varlen + l2norm in kernel", flush=True)
    o, fs = pkg.chunk_gated_delta_rule(d(qr), d(kr), d(v), d(g), d(beta), scale=0.25,
                                       initial_state=d(h0), output_final_state=True,
                                       cu_seqlens=d(cu), use_qk_l2norm_in_kernel=True)
    qn, kn = pkg.l2norm(d(qr)), pkg.l2norm(d(kr))
    o2, fs2 = pkg.gdn_fwd(qn, kn, d(v), d(g), d(beta), d(h0), scale=0.25, cu_seqlens=d(cu))
    torch.cuda.synchronize()
    assert torch.equal(o, o2) and torch.equal(fs, fs2)
    qo, ko = ref.l2norm(qr), ref.l2norm(kr)
    for i, (a, b) in enumerate(zip(cu[:-1].tolist(), cu[1:].tolist())):
        sl = lambda t: t[:, a:b]
        o_ref, h_ref = _recurrent(sl(qo), sl(ko), sl(v), sl(g), sl(beta), h0[i:i + 1], scale=0.25)
        assert ref.rel_err(o_ref, o[:, a:b].cpu()) <= _tol_stored(o.dtype)
        assert ref.rel_err(h_ref, fs[i:i + 1].cpu()) <= TOL_LOWP
