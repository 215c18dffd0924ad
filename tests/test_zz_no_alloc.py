"""gdn_fwd_launch_noalloc on the GPU, through the C ABI: the entry point that
takes its record workspace from the library's static scratch array.  Its
outputs must equal gdn_fwd_launch's (given a caller workspace) bit for bit:
the kernels are the same, and a sequence split into more segments only
passes its fp32 state through final_state between them.  Calls run back to
back on one device, each later one smaller than the one before, so a call
that read records left behind by the previous one would show."""

import ctypes

import pytest
import torch

from oracle import gdn_oracle as ref

pytestmark = pytest.mark.gpu

CODE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}


def _params(L, q, k, v, g, beta, h0, o, fs, chunk):
    B, T, H, K = q.shape
    V = v.shape[-1]
    P = L.GdnFwdParams()
    P.q, P.k, P.v, P.g, P.beta = q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr()
    P.h0 = h0.data_ptr() if h0 is not None else None
    P.o, P.final_state = o.data_ptr(), fs.data_ptr()
    P.q_stride[:] = q.stride()[:3]
    P.k_stride[:] = k.stride()[:3]
    P.v_stride[:] = v.stride()[:3]
    P.g_stride[:] = g.stride()
    P.beta_stride[:] = beta.stride()
    P.o_stride[:] = o.stride()[:3]
    P.h0_stride[:] = h0.stride() if h0 is not None else (0, 0, 0, 0)
    P.fs_stride[:] = fs.stride()
    P.B, P.T, P.H, P.K, P.V = B, T, H, K, V
    P.scale, P.chunk_size, P.block_v = 0.8, chunk, 0
    P.qkv_dtype, P.g_dtype, P.beta_dtype, P.o_dtype = CODE[q.dtype], 0, 0, CODE[o.dtype]
    return P


def _inputs(cuda, B, T, H, K, V, dtype, seed):
    """The BASELINE recipe drawn on the device (both runs read the same
    tensors, so the draw itself needs no oracle)."""
    gen = torch.Generator(device=cuda).manual_seed(seed)
    rn = lambda *s: torch.randn(*s, generator=gen, device=cuda)
    q = torch.nn.functional.normalize(rn(B, T, H, K), dim=-1).to(dtype)
    k = torch.nn.functional.normalize(rn(B, T, H, K), dim=-1).to(dtype)
    v = rn(B, T, H, V).to(dtype)
    beta = torch.sigmoid(rn(B, T, H))
    g = torch.nn.functional.logsigmoid(rn(B, T, H))
    h0 = 0.1 * rn(B, H, K, V)
    return q, k, v, g, beta, h0


def _both(pkg, cuda, B, T, H, K, V, dtype, chunk, seed):
    """(o, fs) of gdn_fwd_launch with a workspace of gdn_fwd_workspace_size
    bytes, and of gdn_fwd_launch_noalloc on fresh NaN-filled outputs."""
    L = pkg._lib
    lib = L.load_library()
    q, k, v, g, beta, h0 = _inputs(cuda, B, T, H, K, V, dtype, seed)
    stream = torch.cuda.current_stream().cuda_stream
    outs = []
    for noalloc in (False, True):
        o = torch.full((B, T, H, V), float("nan"), dtype=dtype, device=cuda)
        fs = torch.full((B, H, K, V), float("nan"), dtype=torch.float32, device=cuda)
        P = _params(L, q, k, v, g, beta, h0, o, fs, chunk)
        ws = None
        if noalloc:
            print(f"[no_alloc] gdn_fwd_launch_noalloc B={B} T={T} H={H} K={K} V={V} "
                  f"{dtype} C={chunk}", flush=True)
            rc = lib.gdn_fwd_launch_noalloc(ctypes.byref(P), stream)
        else:
            n = lib.gdn_fwd_workspace_size(ctypes.byref(P))
            assert n >= 0
            ws = torch.empty(max(n, 256), dtype=torch.uint8, device=cuda)
            P.workspace, P.workspace_bytes = ws.data_ptr(), n
            rc = lib.gdn_fwd_launch(ctypes.byref(P), stream)
        torch.cuda.synchronize()
        assert rc == 0, L.status_string(rc)
        outs.append((o, fs))
    return outs


# (B, T, H, K, V, dtype, chunk): the first call runs 3 segments in the
# scratch (1024 heads x 3 KB per chunk: 10 chunks of 22 fit) against one
# segment with a caller workspace; the second is smaller and runs in one.
# The sixth runs 64-row chunks in 10 segments of one chunk in the scratch
# (512 heads x 33 KB per chunk) against one segment.
CASES = [
    (2, 700, 512, 128, 64, torch.float16, 32),
    (1, 300, 4, 128, 64, torch.float16, 32),
    (2, 1000, 3, 64, 32, torch.float16, 64),
    (1, 200, 2, 128, 48, torch.bfloat16, 64),
    (2, 333, 4, 128, 128, torch.bfloat16, 32),
    (1, 600, 512, 64, 32, torch.float16, 64),
    # bf16 records carry the chunk's k rows in fp16 (11 KB per chunk and
    # head at K = 128): 1024 heads run 7 chunks in 4 segments of 2
    (2, 200, 512, 128, 64, torch.bfloat16, 32),
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_noalloc_matches_launch(pkg, cuda, case):
    B, T, H, K, V, dtype, chunk = CASES[case]
    (o1, fs1), (o2, fs2) = _both(pkg, cuda, B, T, H, K, V, dtype, chunk, seed=40 + case)
    assert torch.isfinite(o1.float()).all() and torch.isfinite(fs1).all()
    assert torch.equal(o1, o2)
    assert torch.equal(fs1, fs2)


def test_noalloc_two_calls_in_a_row(pkg, cuda):
    """A large call (320 heads: 4 segments of 34 chunks in the scratch), then a
    smaller one (one segment), each against gdn_fwd_launch."""
    for seed, (B, T, H) in enumerate(((8, 4000, 40), (1, 700, 3))):
        (o1, fs1), (o2, fs2) = _both(pkg, cuda, B, T, H, 128, 128, torch.float16, 32, seed=60 + seed)
        assert torch.equal(o1, o2)
        assert torch.equal(fs1, fs2)


def test_noalloc_against_oracle(pkg, cuda):
    """A small call against the fp64 step recurrence (1e-3)."""
    B, T, H, K, V = 1, 200, 2, 64, 32
    q, k, v, g, beta, h0 = (t.cpu() for t in _inputs(cuda, B, T, H, K, V, torch.float16, 71))
    (_, _), (o, fs) = _both(pkg, cuda, B, T, H, K, V, torch.float16, 32, seed=71)
    o_ref, h_ref = ref.recurrent(q, k, v, beta, g, ref.to_vk(h0), dtype=torch.float64)
    assert ref.rel_err(0.8 * o_ref, o.float().cpu()) <= 1e-3
    assert ref.rel_err(ref.to_kv(h_ref), fs.cpu()) <= 1e-3


def test_noalloc_bf16_beyond_scratch_runs_fused(pkg, cuda):
    """bf16 at 32-row chunks whose records do not fit the scratch array even
    one chunk per sequence-head (3000 heads x 11 KB > 32 MiB) run on the
    fused kernel instead of failing: checked against the fp64 recurrence."""
    B, T, H, K, V = 1, 40, 3000, 128, 16
    q, k, v, g, beta, h0 = _inputs(cuda, B, T, H, K, V, torch.bfloat16, 81)
    L = pkg._lib
    lib = L.load_library()
    o = torch.full((B, T, H, V), float("nan"), dtype=torch.float32, device=cuda)
    fs = torch.full((B, H, K, V), float("nan"), dtype=torch.float32, device=cuda)
    P = _params(L, q, k, v, g, beta, h0, o, fs, 32)
    print(f"[no_alloc] bf16 B={B} T={T} H={H} beyond the scratch array", flush=True)
    rc = lib.gdn_fwd_launch_noalloc(ctypes.byref(P), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == 0, L.status_string(rc)
    qc, kc, vc, gc, bc, hc = (t.cpu() for t in (q, k, v, g, beta, h0))
    o_ref, h_ref = ref.recurrent(qc, kc, vc, bc, gc, ref.to_vk(hc), dtype=torch.float64)
    assert ref.rel_err(0.8 * o_ref, o.cpu()) <= 1e-3
    assert ref.rel_err(ref.to_kv(h_ref), fs.cpu()) <= 1e-3


@pytest.mark.parametrize("dtype,chunk,H", [(torch.float16, 32, 10923), (torch.float16, 64, 1000)])
def test_noalloc_beyond_scratch_falls_back(pkg, cuda, dtype, chunk, H):
    """fp16 at 32-row chunks (10923 heads x 3 KB) and 64-row chunks (1000
    heads x 33 KB) whose records do not fit the scratch array even one chunk
    per sequence-head run on a kernel without workspace (the fused kernel,
    the phased kernel) instead of failing: checked against the fp64
    recurrence."""
    B, T, K, V = 1, 40 if chunk == 32 else 100, 64, 16
    q, k, v, g, beta, h0 = _inputs(cuda, B, T, H, K, V, dtype, 90 + chunk)
    L = pkg._lib
    lib = L.load_library()
    o = torch.full((B, T, H, V), float("nan"), dtype=torch.float32, device=cuda)
    fs = torch.full((B, H, K, V), float("nan"), dtype=torch.float32, device=cuda)
    P = _params(L, q, k, v, g, beta, h0, o, fs, chunk)
    print(f"[no_alloc] {dtype} C={chunk} B={B} T={T} H={H} beyond the scratch array", flush=True)
    rc = lib.gdn_fwd_launch_noalloc(ctypes.byref(P), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == 0, L.status_string(rc)
    qc, kc, vc, gc, bc, hc = (t.cpu() for t in (q, k, v, g, beta, h0))
    o_ref, h_ref = ref.recurrent(qc, kc, vc, bc, gc, ref.to_vk(hc), dtype=torch.float64)
    assert ref.rel_err(0.8 * o_ref, o.cpu()) <= 1e-3
    assert ref.rel_err(ref.to_kv(h_ref), fs.cpu()) <= 1e-3


@pytest.mark.parametrize("dtype,chunk", [(torch.float16, 32), (torch.bfloat16, 32), (torch.float16, 64)])
def test_noalloc_under_graph_capture(pkg, cuda, dtype, chunk):
    """The use the entry point exists for: after one eager call on the
    device, a call captured into a HIP graph (torch.cuda.graph) replays with
    outputs equal bit for bit to gdn_fwd_launch's, replay after replay, with
    eager work and synchronisations between the replays; and a warmed eager
    call takes no device memory (free bytes unchanged)."""
    B, T, H, K, V = 2, 333, 256, 128, 64   # 512 heads: 3 segments of 21 chunks at C = 32 (fp16)
    (o1, fs1), _ = _both(pkg, cuda, B, T, H, K, V, dtype, chunk, seed=97)
    L = pkg._lib
    lib = L.load_library()
    q, k, v, g, beta, h0 = _inputs(cuda, B, T, H, K, V, dtype, 97)
    o = torch.full((B, T, H, V), float("nan"), dtype=dtype, device=cuda)
    fs = torch.full((B, H, K, V), float("nan"), dtype=torch.float32, device=cuda)
    P = _params(L, q, k, v, g, beta, h0, o, fs, chunk)
    # warmed eager call: no allocation
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    rc = lib.gdn_fwd_launch_noalloc(ctypes.byref(P), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == 0, L.status_string(rc)
    assert torch.cuda.mem_get_info()[0] == free0
    assert torch.equal(o, o1) and torch.equal(fs, fs1)
    print(f"[no_alloc] graph capture {dtype} C={chunk} B={B} T={T} H={H}", flush=True)
    o.fill_(float("nan"))
    fs.fill_(float("nan"))
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            rc = lib.gdn_fwd_launch_noalloc(ctypes.byref(P), torch.cuda.current_stream().cuda_stream)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    assert rc == 0, L.status_string(rc)
    for rep in range(3):
        o.fill_(float("nan"))
        fs.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(o, o1), f"replay {rep}: o differs"
        assert torch.equal(fs, fs1), f"replay {rep}: final state differs"
        # eager work between replays
        (_, _), (o3, fs3) = _both(pkg, cuda, 1, 100, 3, K, V, dtype, chunk, seed=98 + rep)
        assert torch.isfinite(o3.float()).all()
