"""GPU parity of the HIP backward (``gdn_bwd``, autograd through ``gdn_fwd``).

The reference has no backward (README.md:259); the gradients are those of
its recurrence (gdn_ref.py:3-9).  They are checked against reverse-mode
differentiation of the oracle's fp64 step recurrence (``recurrent_grads``)
on the same (cast) inputs, with the max-norm relative error of
bench_gdn.py:89-94:
  * fp32 inputs: <= 2e-5 (the kernel computes in fp32);
  * fp16 / bf16 inputs: <= 1e-3 plus one rounding of the gradient to its
    storage dtype (2^-11 / 2^-8).
At the full cfg2 shape one head is compared with the oracle's fp64 chunked
backward, and packed sequences are compared bit for bit with separate runs.
"""

import pytest
import torch

from oracle import gdn_oracle as ref

pytestmark = pytest.mark.gpu

NAMES = ("dq", "dk", "dv", "dbeta", "dg", "dh0")


def _inputs(B, T, H, K, V, dtype, seed, gate=1.0):
    gen = torch.Generator().manual_seed(seed)
    q = ref.l2norm(torch.randn(B, T, H, K, generator=gen)).to(dtype)
    k = ref.l2norm(torch.randn(B, T, H, K, generator=gen)).to(dtype)
    v = torch.randn(B, T, H, V, generator=gen).to(dtype)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=gen))
    g = gate * torch.nn.functional.logsigmoid(torch.randn(B, T, H, generator=gen))
    h0 = 0.1 * torch.randn(B, H, K, V, generator=gen)
    do = torch.randn(B, T, H, V, generator=gen).to(dtype)
    dfin = torch.randn(B, H, K, V, generator=gen)
    return q, k, v, g, beta, h0, do, dfin


def _tol(dtype):
    if dtype == torch.float32:
        return 2e-5
    return 1e-3 + (2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11)


def _compare(got, want, dtype, label):
    errs = {}
    for name, a, b in zip(NAMES, got, want):
        if a is None:
            continue
        errs[name] = ref.rel_err(b, a.cpu().double())
    print(f"[bwd] {label}: " + " ".join(f"{n}={e:.2e}" for n, e in errs.items()), flush=True)
    for name, e in errs.items():
        tol = 2e-5 if name == "dh0" and dtype == torch.float32 else _tol(dtype)
        if name == "dh0" and dtype != torch.float32:
            tol = 1e-3        # dh0 is fp32 for every input dtype
        assert e <= tol, (label, name, e)


@pytest.mark.parametrize("T,K,V,gate", [(64, 32, 16, 1.0), (77, 64, 32, 1.0), (33, 128, 16, 1.0),
                                        (130, 128, 48, 3.0), (5, 32, 16, 1.0), (256, 64, 64, 0.1)])
def test_bwd_fp32_vs_autograd(pkg, cuda, T, K, V, gate):
    B, H = 2, 2
    q, k, v, g, beta, h0, do, dfin = _inputs(B, T, H, K, V, torch.float32, seed=T + K, gate=gate)
    d = lambda t: t.to(cuda)
    print(f"[bwd] fp32 T={T} K={K} V={V} gate={gate}", flush=True)
    got = pkg.gdn_bwd(d(q), d(k), d(v), d(g), d(beta), d(h0), d(do), d(dfin), scale=0.7)
    torch.cuda.synchronize()
    want = ref.recurrent_grads(q, k, v, beta, g, h0, do, dfin, scale=0.7)
    got = (got[0], got[1], got[2], got[4], got[3], got[5])   # -> dq dk dv dbeta dg dh0
    _compare(got, want, torch.float32, f"fp32 T={T} K={K} V={V}")


@pytest.mark.parametrize("T,K,V", [(200, 128, 32), (77, 64, 48), (33, 32, 16),
                                   (1, 64, 16), (32, 128, 16), (96, 128, 32), (97, 32, 48)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_bwd_lowp_vs_autograd(pkg, cuda, dtype, T, K, V):
    """16-bit q, k, v and dO: the recurrences run on fp16 hi / lo pairs.
    Chunk counts 1 to 7, whole and partial last chunks: the walks copy their
    inputs one (backward) or two (forward) chunks ahead and zero a partial
    chunk's rows in LDS."""
    B, H = 1, 3
    q, k, v, g, beta, h0, do, dfin = _inputs(B, T, H, K, V, dtype, seed=5)
    d = lambda t: t.to(cuda)
    print(f"[bwd] {dtype} T={T} K={K} V={V}", flush=True)
    got = pkg.gdn_bwd(d(q), d(k), d(v), d(g), d(beta), d(h0), d(do), d(dfin), scale=1.0)
    torch.cuda.synchronize()
    assert got[0].dtype == dtype and got[2].dtype == dtype and got[3].dtype == torch.float32
    want = ref.recurrent_grads(q, k, v, beta, g, h0, do, dfin)
    _compare((got[0], got[1], got[2], got[4], got[3], got[5]), want, dtype, f"{dtype} K={K} V={V}")


def test_autograd_through_gdn_fwd(pkg, cuda):
    """loss.backward() through gdn_fwd (pipelined forward, HIP backward)
    equals the oracle's gradients; gdn_chunk_fwd's V x K state and FLA's
    head_first layout backpropagate through their strides."""
    B, T, H, K, V = 2, 96, 2, 64, 32
    q, k, v, g, beta, h0, do, dfin = _inputs(B, T, H, K, V, torch.float16, seed=9)
    leaves = [t.to(cuda).requires_grad_(True) for t in (q, k, v, g, beta, h0)]
    print("[bwd] autograd gdn_fwd", flush=True)
    o, fs = pkg.gdn_fwd(*leaves, scale=0.5)
    (o.float() * do.to(cuda).float()).sum().backward(inputs=leaves, retain_graph=False)
    fs_loss = None
    got = [t.grad for t in leaves]
    want = ref.recurrent_grads(q, k, v, beta, g, h0, do, None, scale=0.5)
    _compare((got[0], got[1], got[2], got[4], got[3], got[5]), want, torch.float16, "autograd")

    # gdn_chunk_fwd: h [B,H,V,K]; gradient through the final state only
    leaves2 = [t.to(cuda).requires_grad_(True) for t in (q, k, v, beta, g)]
    o2, hf = pkg.gdn_chunk_fwd(*leaves2)
    (hf * dfin.transpose(2, 3).to(cuda)).sum().backward()
    want2 = ref.recurrent_grads(q, k, v, beta, g, None, torch.zeros_like(do), dfin)
    got2 = [leaves2[0].grad, leaves2[1].grad, leaves2[2].grad, leaves2[3].grad, leaves2[4].grad, None]
    _compare(got2, want2, torch.float16, "gdn_chunk_fwd state grad")

    # FLA head_first: gradients come back in the [B, H, T, *] layout
    hf_ = lambda t: t.transpose(1, 2).contiguous()
    leaves3 = [hf_(t).to(cuda).requires_grad_(True) for t in (q, k, v, g, beta)]
    o3, _ = pkg.chunk_gated_delta_rule(*leaves3, scale=0.5, head_first=True)
    (o3.float() * hf_(do).to(cuda).float()).sum().backward()
    want3 = ref.recurrent_grads(q, k, v, beta, g, None, do, None, scale=0.5)
    got3 = [leaves3[0].grad.transpose(1, 2), leaves3[1].grad.transpose(1, 2),
            leaves3[2].grad.transpose(1, 2), leaves3[4].grad.transpose(1, 2),
            leaves3[3].grad.transpose(1, 2), None]
    _compare(got3, want3, torch.float16, "head_first")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_bwd_varlen_equals_separate_runs(pkg, cuda, dtype):
    lens = [40, 0, 1, 64, 75]
    H, K, V = 2, 64, 32
    T = sum(lens)
    q, k, v, g, beta, _, do, _ = _inputs(1, T, H, K, V, dtype, seed=12)
    n = len(lens)
    gen = torch.Generator().manual_seed(13)
    h0 = 0.1 * torch.randn(n, H, K, V, generator=gen)
    dfin = torch.randn(n, H, K, V, generator=gen)
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int64)
    d = lambda t: t.to(cuda)
    print(f"[bwd] varlen {lens} {dtype}", flush=True)
    got = pkg.gdn_bwd(d(q), d(k), d(v), d(g), d(beta), d(h0), d(do), d(dfin), scale=0.9,
                      cu_seqlens=d(cu))
    torch.cuda.synchronize()
    for i, (a, b) in enumerate(zip(cu[:-1].tolist(), cu[1:].tolist())):
        sl = lambda t: t[:, a:b].contiguous()
        sep = pkg.gdn_bwd(d(sl(q)), d(sl(k)), d(sl(v)), d(sl(g)), d(sl(beta)), d(h0[i:i + 1]),
                          d(sl(do)), d(dfin[i:i + 1]), scale=0.9)
        torch.cuda.synchronize()
        for j in range(5):
            assert torch.equal(got[j][:, a:b].cpu(), sep[j].cpu()), (i, j)
        assert torch.equal(got[5][i:i + 1].cpu(), sep[5].cpu()), (i, "dh0")


def test_bwd_full_size_one_head(pkg, cuda):
    """cfg2 shape (fp16 B2 H16 T4096 K=V=128): the whole backward runs, and
    head (b=1, h=5) matches the oracle's fp64 chunked backward."""
    B, T, H, K, V = 2, 4096, 16, 128, 128
    q, k, v, g, beta, _ = ref.make_inputs_baseline(B, T, H, K, V, seed=0)
    gen = torch.Generator().manual_seed(1)
    do = torch.randn(B, T, H, V, generator=gen).half()
    d = lambda t: t.to(cuda)
    print("[bwd] cfg2 full size", flush=True)
    got = pkg.gdn_bwd(d(q), d(k), d(v), d(g), d(beta), None, d(do), None, scale=1.0,
                      need_dh0=False)
    torch.cuda.synchronize()
    for t in got[:5]:
        assert torch.isfinite(t.float()).all()
    b, h = 1, 5
    sel = lambda t: t[b:b + 1, :, h:h + 1]
    want = ref.chunked_bwd(sel(q), sel(k), sel(v), sel(beta), sel(g), None, sel(do), None)
    mine = (sel(got[0].cpu()), sel(got[1].cpu()), sel(got[2].cpu()), sel(got[4].cpu()),
            sel(got[3].cpu()), None)
    _compare(mine, want, torch.float16, "cfg2 head (1,5)")


@pytest.mark.parametrize("dtype,seg", [(torch.float32, 1), (torch.float32, 3), (torch.float16, 2),
                                       (torch.float16, 4), (torch.bfloat16, 3)])
def test_bwd_segments_vs_autograd(pkg, cuda, dtype, seg):
    """A workspace of `seg` chunks per sequence: T = 300 (10 chunks, the
    last partial) runs as ceil(10 / seg) segments, the states at their
    starts from forward calls and the state gradient carried backwards.
    The gradients match the oracle at the one-pass tolerances, and the
    one-pass call within the same bound."""
    B, H, T, K, V = 2, 2, 300, 64, 32
    q, k, v, g, beta, h0, do, dfin = _inputs(B, T, H, K, V, dtype, seed=11 + seg)
    d = lambda t: t.to(cuda)
    print(f"[bwd] segments of {seg} chunks, {dtype}", flush=True)
    got = pkg.gdn_bwd(d(q), d(k), d(v), d(g), d(beta), d(h0), d(do), d(dfin), scale=0.8,
                      max_segment_chunks=seg)
    one = pkg.gdn_bwd(d(q), d(k), d(v), d(g), d(beta), d(h0), d(do), d(dfin), scale=0.8)
    torch.cuda.synchronize()
    want = ref.recurrent_grads(q, k, v, beta, g, h0, do, dfin, scale=0.8)
    order = lambda r: (r[0], r[1], r[2], r[4], r[3], r[5])   # -> dq dk dv dbeta dg dh0
    _compare(order(got), want, dtype, f"{dtype} segments of {seg}")
    _compare(order(got), tuple(t.cpu().double() for t in order(one)), dtype, f"{dtype} segments vs one pass")


def test_bwd_cfg3_length_segmented(pkg, cuda):
    """cfg3's length (fp16 B2 H16 T16384 K=V=128, 512 chunks): the default
    workspace holds 256 chunks per sequence, so the backward runs as two
    segments.  That workspace is the 8192-row one plus three fp32 states,
    under half the one-pass size; the allocator grows by no more than the
    outputs and that workspace over the call; head (1, 5) matches the
    oracle's fp64 chunked backward."""
    import ctypes
    B, T, H, K, V = 2, 16384, 16, 128, 128
    q, k, v, g, beta, _ = ref.make_inputs_baseline(B, T, H, K, V, seed=0)
    gen = torch.Generator().manual_seed(2)
    do = torch.randn(B, T, H, V, generator=gen).half()
    dq_, dk_, dv_, dg_, db_, do_ = (t.to(cuda) for t in (q, k, v, g, beta, do))
    L = pkg._lib
    lib = L.load_library()

    def ws(rows, seg=None):
        P = L.GdnBwdParams()
        P.B, P.T, P.H, P.K, P.V = B, rows, H, K, V
        P.qkv_dtype, P.g_dtype, P.beta_dtype, P.do_dtype = 1, 0, 0, 1
        P.d_o = do_.data_ptr()
        P.do_stride[:] = do_.stride()[:3]
        if seg is None:
            return lib.gdn_bwd_workspace_size_params(ctypes.byref(P))
        return lib.gdn_bwd_segment_workspace_size(ctypes.byref(P), seg)

    state = B * H * K * V * 4
    bound = ws(8192) + 3 * state
    assert ws(T) == bound and bound < 0.51 * ws(T, 10 ** 6)
    print(f"[bwd] cfg3 length, workspace {bound / 2**20:.0f} MiB", flush=True)
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats(cuda)
    base = torch.cuda.memory_allocated(cuda)
    got = pkg.gdn_bwd(dq_, dk_, dv_, dg_, db_, None, do_, None, scale=1.0, need_dh0=False)
    torch.cuda.synchronize()
    grown = torch.cuda.max_memory_allocated(cuda) - base
    outs = sum(t.numel() * t.element_size() for t in got if t is not None)
    assert grown <= outs + bound + (2 << 20), (grown, outs, bound)
    for t in got[:5]:
        assert torch.isfinite(t.float()).all()
    b, h = 1, 5
    sel = lambda t: t[b:b + 1, :, h:h + 1]
    want = ref.chunked_bwd(sel(q), sel(k), sel(v), sel(beta), sel(g), None, sel(do), None)
    mine = (sel(got[0].cpu()), sel(got[1].cpu()), sel(got[2].cpu()), sel(got[4].cpu()),
            sel(got[3].cpu()), None)
    _compare(mine, want, torch.float16, "cfg3 length head (1,5)")


def test_autograd_fla_varlen_bf16(pkg, cuda):
    """loss.backward() through FLA's varlen call (bf16, initial_state and
    final-state gradient): every sequence's gradients match the oracle's."""
    lens = [45, 70, 13]
    H, K, V = 2, 64, 32
    T = sum(lens)
    q, k, v, g, beta, _, do, _ = _inputs(1, T, H, K, V, torch.bfloat16, seed=21)
    gen = torch.Generator().manual_seed(22)
    h0 = 0.1 * torch.randn(len(lens), H, K, V, generator=gen)
    dfin = torch.randn(len(lens), H, K, V, generator=gen)
    cu = torch.tensor([0, 45, 115, 128], dtype=torch.int64)
    leaves = [t.to(cuda).requires_grad_(True) for t in (q, k, v, g, beta, h0)]
    print("[bwd] FLA varlen bf16 autograd", flush=True)
    o, fs = pkg.chunk_gated_delta_rule(*leaves[:5], scale=0.8, initial_state=leaves[5],
                                       output_final_state=True, cu_seqlens=cu.to(cuda))
    ((o.float() * do.to(cuda).float()).sum() + (fs * dfin.to(cuda)).sum()).backward()
    for i, (a, b) in enumerate(zip(cu[:-1].tolist(), cu[1:].tolist())):
        sl = lambda t: t[:, a:b]
        want = ref.recurrent_grads(sl(q), sl(k), sl(v), sl(beta), sl(g), h0[i:i + 1], sl(do),
                                   dfin[i:i + 1], scale=0.8)
        got = (sl(leaves[0].grad.cpu()), sl(leaves[1].grad.cpu()), sl(leaves[2].grad.cpu()),
               sl(leaves[4].grad.cpu()), sl(leaves[3].grad.cpu()), leaves[5].grad[i:i + 1].cpu())
        _compare(got, want, torch.bfloat16, f"varlen seq {i}")


def test_autograd_sum_losses_expanded_grads(pkg, cuda):
    """o.sum().backward() hands the backward a stride-0 expansion of one
    element as dO (and fs.sum() one as d_final_state): the gradients equal
    the oracle's with dO = ones (dfinal = ones).  Weak gates keep dh0 of
    order one: under the recipe's gates a state gradient that only enters
    through d_final_state decays by about e^-56 over 70 steps, below the
    range of the fp16 image the recurrences carry (as the reference's own
    fp16 cast of the state, gdn_triton.py:87)."""
    B, T, H, K, V = 1, 70, 2, 64, 32
    q, k, v, g, beta, h0, _, _ = _inputs(B, T, H, K, V, torch.float16, seed=31, gate=0.05)
    ones_o = torch.ones(B, T, H, V)
    ones_s = torch.ones(B, H, K, V)
    for which in ("o", "fs"):
        leaves = [t.to(cuda).requires_grad_(True) for t in (q, k, v, g, beta, h0)]
        print(f"[bwd] {which}.sum().backward()", flush=True)
        o, fs = pkg.gdn_fwd(*leaves, scale=0.6)
        (o.sum() if which == "o" else fs.sum()).backward()
        torch.cuda.synchronize()
        if which == "o":
            want = ref.recurrent_grads(q, k, v, beta, g, h0, ones_o, None, scale=0.6)
        else:
            want = ref.recurrent_grads(q, k, v, beta, g, h0, torch.zeros(B, T, H, V), ones_s,
                                       scale=0.6)
        got = [t.grad for t in leaves]
        _compare((got[0], got[1], got[2], got[4], got[3], got[5]), want, torch.float16,
                 f"{which}.sum()")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_bwd_lowp_inputs_fp32_do(pkg, cuda, dtype):
    """16-bit q, k, v with an fp32 dO run the fp32 recurrences, which read
    the record's fp32 W (the path taken when the forward wrote o in fp32)."""
    B, H, T, K, V = 1, 3, 150, 128, 32
    q, k, v, g, beta, h0, do, dfin = _inputs(B, T, H, K, V, dtype, seed=41)
    do32 = torch.randn(B, T, H, V, generator=torch.Generator().manual_seed(42))
    d = lambda t: t.to(cuda)
    print(f"[bwd] {dtype} inputs, fp32 dO", flush=True)
    got = pkg.gdn_bwd(d(q), d(k), d(v), d(g), d(beta), d(h0), d(do32), d(dfin), scale=1.0)
    torch.cuda.synchronize()
    want = ref.recurrent_grads(q, k, v, beta, g, h0, do32, dfin)
    _compare((got[0], got[1], got[2], got[4], got[3], got[5]), want, dtype, f"{dtype} fp32 dO")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_autograd_fp32_output(pkg, cuda, dtype):
    """loss.backward() through gdn_fwd(output_dtype=float32): dO arrives in
    fp32 while q, k, v are 16-bit."""
    B, T, H, K, V = 1, 100, 2, 64, 48
    q, k, v, g, beta, h0, _, dfin = _inputs(B, T, H, K, V, dtype, seed=51)
    do = torch.randn(B, T, H, V, generator=torch.Generator().manual_seed(52))
    leaves = [t.to(cuda).requires_grad_(True) for t in (q, k, v, g, beta, h0)]
    print(f"[bwd] autograd {dtype} output_dtype=float32", flush=True)
    o, fs = pkg.gdn_fwd(*leaves, scale=0.9, output_dtype=torch.float32)
    assert o.dtype == torch.float32
    ((o * do.to(cuda)).sum() + (fs * dfin.to(cuda)).sum()).backward()
    want = ref.recurrent_grads(q, k, v, beta, g, h0, do, dfin, scale=0.9)
    got = [t.grad for t in leaves]
    _compare((got[0], got[1], got[2], got[4], got[3], got[5]), want, dtype, f"{dtype} fp32 o")


@pytest.mark.parametrize("v_scale,d_scale", [(1.0, 1e-6), (1e5, 1.0), (1e-6, 1e-7), (3e4, 1e-6)])
def test_bwd_bf16_extreme_scales(pkg, cuda, v_scale, d_scale):
    """bf16 v / h0 and dO / d_final_state far from fp16's range (|v| up to
    1e5, gradients of 1e-6 as in bf16 training without loss scaling): the
    16-bit state walks run on power-of-two-shifted values and shift their
    outputs back (exact), so every gradient stays within the 16-bit bar of
    the fp64 recurrence's, relative to its own magnitude."""
    B, T, H, K, V = 1, 150, 2, 64, 32
    q, k, v, g, beta, h0, do, dfin = _inputs(B, T, H, K, V, torch.float32, seed=41)
    v, h0, do, dfin = v * v_scale, h0 * v_scale, do * d_scale, dfin * d_scale
    bf = lambda t: t.to(torch.bfloat16)
    q, k, v, do = bf(q), bf(k), bf(v), bf(do)
    d = lambda t: t.to(cuda)
    print(f"[bwd] bf16 v*{v_scale:g} dO*{d_scale:g}", flush=True)
    got = pkg.gdn_bwd(d(q), d(k), d(v), d(g), d(beta), d(h0), d(do), d(dfin), scale=1.0)
    torch.cuda.synchronize()
    for t in got:
        assert t is None or torch.isfinite(t.float()).all()
    want = ref.recurrent_grads(q, k, v, beta, g, h0, do, dfin, scale=1.0)
    got = (got[0], got[1], got[2], got[4], got[3], got[5])   # -> dq dk dv dbeta dg dh0
    _compare(got, want, torch.bfloat16, f"bf16 v*{v_scale:g} dO*{d_scale:g}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_bwd_do_row_offsets(pkg, cuda, dtype):
    """dO as a view into a wider buffer: rows 4-byte aligned (the 16-bit
    walks copy dO slices 4 bytes a lane) give the same bits as a dense dO;
    rows only 2-byte aligned take the fp32 recurrences and still match the
    oracle."""
    B, T, H, K, V = 1, 77, 2, 64, 32
    q, k, v, g, beta, h0, do, dfin = _inputs(B, T, H, K, V, dtype, seed=23)
    d = lambda t: t.to(cuda)
    print(f"[bwd] {dtype} dO row offsets T={T} K={K} V={V}", flush=True)
    dense = pkg.gdn_bwd(d(q), d(k), d(v), d(g), d(beta), d(h0), d(do), d(dfin), scale=1.0)
    wide = torch.zeros(B, T, H, V + 8, dtype=dtype)
    for off in (2, 1):   # elements: 4 bytes, then 2 bytes
        wide.zero_()
        wide[..., off:off + V] = do
        view = d(wide)[..., off:off + V]
        assert view.stride(-1) == 1 and (view.data_ptr() % 4 == 0) == (off == 2)
        got = pkg.gdn_bwd(d(q), d(k), d(v), d(g), d(beta), d(h0), view, d(dfin), scale=1.0)
        torch.cuda.synchronize()
        if off == 2:
            for a, b in zip(got, dense):
                if a is not None:
                    assert torch.equal(a, b)
        else:
            want = ref.recurrent_grads(q, k, v, beta, g, h0, do, dfin)
            _compare((got[0], got[1], got[2], got[4], got[3], got[5]), want, dtype, f"{dtype} dO offset {off}")
