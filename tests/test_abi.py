"""CPU tests of the C-ABI library and the host-side checks (no GPU needed).

* the library built from v100-attention-lab_amd/csrc loads and exports every
  function declared in include/gdn_mi355x.h;
* the ctypes mirror of GdnFwdParams has the C struct's exact layout (checked
  against offsetof/sizeof from gcc on the header);
* argument errors come back as status codes before anything is enqueued;
* the Python surface rejects bad inputs with ValueError and never falls
  back to a CPU path.
"""

import ctypes
import json
import os
import re
import subprocess

import pytest
import torch

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "gdn_mi355x.h")


@pytest.fixture(scope="module")
def lib(pkg):
    if not os.path.exists(pkg.LIB_PATH):
        from importlib import import_module
        import_module("v100-attention-lab_amd.build").build(verbose=False)
    return pkg.load_library()


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(gdn_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_expected_api(pkg):
    from importlib import import_module
    L = import_module("v100-attention-lab_amd._lib")
    assert _declared_functions() == sorted(L.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol(lib, pkg):
    out = subprocess.run(["nm", "-D", "--defined-only", pkg.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\s[TW]\s+(\S+)$", out, flags=re.M))
    for name in _declared_functions():
        assert name in exported, f"{name} not exported"
        assert hasattr(lib, name)


def test_abi_version(lib):
    assert lib.gdn_fwd_abi_version() == 5


@pytest.mark.parametrize("struct", ["GdnFwdParams", "GdnPrepParams", "GdnBwdParams"])
def test_struct_layout_matches_header(tmp_path, struct):
    """Compile a probe against the header with gcc and compare offsets."""
    from importlib import import_module
    L = import_module("v100-attention-lab_amd._lib")
    S = getattr(L, struct)
    fields = [f for f, _ in S._fields_]
    src = tmp_path / "layout.c"
    body = "\n".join(f'  printf("{f} %zu\\n", offsetof({struct}, {f}));' for f in fields)
    src.write_text(f"#include <stddef.h>\n#include <stdio.h>\n#include \"gdn_mi355x.h\"\n"
                   f"int main(void) {{\n{body}\n  printf(\"sizeof %zu\\n\", sizeof({struct}));\n"
                   f"  return 0;\n}}\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", f"-I{os.path.dirname(HEADER)}", str(src),
                    "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()
    c_layout = dict(zip(out[0::2], map(int, out[1::2])))
    for f in fields:
        assert getattr(S, f).offset == c_layout[f], f
    assert ctypes.sizeof(S) == c_layout["sizeof"]


def _params(L, **kw):
    P = L.GdnFwdParams()
    fake = 0x1000  # never dereferenced: every case below fails validation first
    P.q = P.k = P.v = P.g = P.beta = P.o = P.final_state = fake
    P.q_stride[:] = (4096 * 16 * 128, 16 * 128, 128)
    P.k_stride[:] = P.q_stride[:]
    P.v_stride[:] = P.q_stride[:]
    P.g_stride[:] = (4096 * 16, 16, 1)
    P.beta_stride[:] = P.g_stride[:]
    P.o_stride[:] = P.q_stride[:]
    P.fs_stride[:] = (16 * 128 * 128, 128 * 128, 128, 1)
    P.B, P.T, P.H, P.K, P.V = 2, 4096, 16, 128, 128
    P.scale, P.chunk_size, P.block_v = 1.0, 32, 0
    P.qkv_dtype, P.g_dtype, P.beta_dtype, P.o_dtype = 1, 0, 0, 1
    for k_, v_ in kw.items():
        setattr(P, k_, v_)
    return P


def test_fwd_workspace_size(lib, pkg):
    """Fused kernels need no workspace.  32-row chunks with fp16 or bf16
    q/k/v and K in {64, 128} take one 3 KB record per (sequence, head, chunk) of a
    segment of at most 256 chunks.  64-row chunks with K <= 128 take one
    record per (chunk slot, head).  fp32 inputs: T and P (C x C), W (C x K)
    in fp32, then three gate rows.  16-bit inputs: T diag(beta) and P (C x C)
    as fp16 hi/lo pairs, then four fp32 gate rows."""
    L = pkg._lib
    size = lambda **kw: lib.gdn_fwd_workspace_size(ctypes.byref(_params(L, **kw)))
    H = 16
    assert size() == 2 * H * 128 * 3072                  # C = 32 fp16: records of 128 chunks
    assert size(T=16384) == 2 * H * 256 * 3072           # segments of at most 256 chunks
    assert size(T=100, K=64) == 2 * H * 4 * 3072         # partial last chunk included
    assert size(T=0) == 0
    assert size(B=3, T=100, cu_seqlens=0x2000) == 3 * H * 4 * 3072
    assert size(flags=2) == 0                            # fused kernel forced: none
    # bf16: the record, then the chunk's k rows in fp16
    assert size(qkv_dtype=2) == 2 * H * 128 * (3072 + 32 * 128 * 2)
    assert size(qkv_dtype=2, K=64) == 2 * H * 128 * (3072 + 32 * 64 * 2)
    assert size(qkv_dtype=2, V=2512) == 2 * H * 128 * (3072 + 32 * 128 * 2)  # any V
    assert size(qkv_dtype=0) == 0                        # fp32: phased kernel, none
    assert size(K=32) == 0 and size(K=256) == 0          # phased kernel, none
    assert size(chunk_size=64, K=256) == 0               # phased kernel, none
    assert size(chunk_size=64, flags=1) == 0             # phased forced, none
    C, K, H = 64, 128, 16
    rec32 = 4 * (2 * C * C + C * K + 3 * C)
    rec16 = 2 * 4 * C * C + 4 * 4 * C
    for dt, rec in ((0, rec32), (1, rec16), (2, rec16)):
        want = 2 * (4096 // C) * H * rec                 # 64 chunks: one segment
        assert want <= size(chunk_size=64, qkv_dtype=dt) < want + 256
        # T = 16384: segments of 64 chunks, the same workspace
        assert want <= size(chunk_size=64, qkv_dtype=dt, T=16384) < want + 256
    # the 16-bit record does not depend on K, the fp32 one does (W is C x K)
    for k_ in (32, 64):
        want16 = 2 * (4096 // C) * H * rec16
        want32 = 2 * (4096 // C) * H * 4 * (2 * C * C + C * k_ + 3 * C)
        assert want16 <= size(chunk_size=64, K=k_) < want16 + 256
        assert want32 <= size(chunk_size=64, K=k_, qkv_dtype=0) < want32 + 256
    # packed sequences: ceil(T / C) = 2 chunks of records for each of 3
    got = size(chunk_size=64, B=3, T=100, cu_seqlens=0x2000)
    assert 3 * 2 * H * rec16 <= got < 3 * 2 * H * rec16 + 256
    assert size(chunk_size=64, B=0) == -1
    assert size(chunk_size=64, qkv_dtype=9) == -1
    assert lib.gdn_fwd_workspace_size(None) == -1


@pytest.mark.parametrize("kw,code", [
    (dict(chunk_size=64), 1006), (dict(chunk_size=64, workspace=0x1010, workspace_bytes=1 << 40), 1006),
    (dict(chunk_size=64, workspace=0x1000, workspace_bytes=1024), 1006),
])
def test_fwd_c64_rejects_bad_workspace(lib, pkg, kw, code):
    P = _params(pkg._lib, **kw)
    assert lib.gdn_fwd_launch(ctypes.byref(P), None) == code


@pytest.mark.parametrize("kw,code", [
    (dict(B=0), 1002), (dict(T=-1), 1002), (dict(V=24), 1002),
    (dict(chunk_size=48), 1003), (dict(K=96), 1003), (dict(block_v=128), 1003),
    (dict(block_v=48), 1003), (dict(qkv_dtype=7), 1005), (dict(o_dtype=-1), 1005),
    (dict(q=0x1008), 1004), (dict(final_state=None), 1001), (dict(v=None), 1001),
])
def test_launch_rejects_bad_arguments(lib, kw, code):
    from importlib import import_module
    L = import_module("v100-attention-lab_amd._lib")
    P = _params(L, **kw)
    assert lib.gdn_fwd_launch(ctypes.byref(P), None) == code
    assert lib.gdn_fwd_status_string(code).decode().startswith("gdn_fwd:")


def test_misaligned_stride_rejected(lib):
    from importlib import import_module
    L = import_module("v100-attention-lab_amd._lib")
    P = _params(L)
    P.k_stride[1] = 16 * 128 + 1
    assert lib.gdn_fwd_launch(ctypes.byref(P), None) == 1004
    assert lib.gdn_fwd_launch(None, None) == 1001


def test_auto_block_v(pkg):
    # one workgroup per CU (256) when possible, else the narrowest slice
    assert pkg.auto_block_v(2, 16, 128, 128) == 16
    assert pkg.auto_block_v(4, 16, 128, 128) == 32
    assert pkg.auto_block_v(16, 16, 128, 128) == 32
    assert pkg.auto_block_v(16, 16, 96, 128) == -1
    assert pkg.auto_block_v(1, 2, 128, 128, dtype=torch.float32) == 16
    assert pkg.auto_block_v(1, 2, 64, 48) == 16
    assert pkg.auto_block_v(1, 1, 96, 64) == -1


def test_status_strings(lib):
    assert lib.gdn_fwd_status_string(0).decode() == "success"
    for code in (1001, 1002, 1003, 1004, 1005):
        assert "gdn_fwd" in lib.gdn_fwd_status_string(code).decode()


# --------------------------------------------------------------------------
# Python surface: validation happens before any device work
# --------------------------------------------------------------------------

def _cpu_inputs(B=1, T=64, H=2, K=64, V=32, dtype=torch.float16):
    q = torch.zeros(B, T, H, K, dtype=dtype)
    return q, q.clone(), torch.zeros(B, T, H, V, dtype=dtype), torch.zeros(B, T, H), torch.zeros(B, T, H)


def test_cpu_tensors_are_rejected_no_fallback(pkg):
    q, k, v, g, b = _cpu_inputs()
    with pytest.raises(ValueError, match="no CPU path"):
        pkg.gdn_fwd(q, k, v, g, b)
    with pytest.raises(ValueError, match="no CPU path"):
        pkg.gdn_chunk_fwd(q, k, v, b, g)


@pytest.mark.parametrize("mutate,msg", [
    (lambda a: a.__setitem__(1, a[1][:, :, :, :32]), "k shape"),
    (lambda a: a.__setitem__(2, a[2][:, :10]), "v shape"),
    (lambda a: a.__setitem__(3, a[3][:, :, :1]), "g must be"),
    (lambda a: a.__setitem__(2, a[2].float()), "share a dtype"),
    (lambda a: [a.__setitem__(i, a[i].to(torch.int32)) for i in range(3)], "not supported"),
])
def test_shape_and_dtype_validation(pkg, mutate, msg):
    args = list(_cpu_inputs())
    mutate(args)
    with pytest.raises(ValueError, match=msg):
        pkg.gdn_fwd(*args)


def test_h0_and_option_validation(pkg):
    q, k, v, g, b = _cpu_inputs()
    with pytest.raises(ValueError, match="h0 must be"):
        pkg.gdn_fwd(q, k, v, g, b, torch.zeros(1, 2, 32, 64))
    with pytest.raises(ValueError, match="float32"):
        pkg.gdn_fwd(q, k, v, g, b, torch.zeros(1, 2, 64, 32, dtype=torch.float16))
    with pytest.raises(ValueError, match="chunk_size"):
        pkg.gdn_fwd(q, k, v, g, b, chunk_size=16)
    with pytest.raises(ValueError, match="block_v"):
        pkg.gdn_fwd(q, k, v, g, b, block_v=64)
    q2, k2, _, g2, b2 = _cpu_inputs(K=96)
    with pytest.raises(ValueError, match="K=96"):
        pkg.gdn_fwd(q2, k2, v, g2, b2)


def test_missing_library_raises_importerror(tmp_path):
    from importlib import import_module
    L = import_module("v100-attention-lab_amd._lib")
    saved = L._lib
    L._lib = None
    try:
        with pytest.raises(ImportError, match="not found"):
            L.load_library(str(tmp_path / "nope.so"))
    finally:
        L._lib = saved


# --------------------------------------------------------------------------
# input preparation entry point: argument errors before any launch
# --------------------------------------------------------------------------

def _prep_params(L, **kw):
    P = L.GdnPrepParams()
    fake = 0x1000  # never dereferenced: every case below returns before a launch
    P.q_in = P.q_out = P.k_in = P.k_out = fake
    P.beta_in = P.beta_out = P.g_in = P.g_out = fake
    for name in ("q_in", "q_out", "k_in", "k_out"):
        getattr(P, name + "_stride")[:] = (4096 * 16 * 128, 16 * 128, 128)
    for name in ("beta_in", "beta_out", "g_in", "g_out"):
        getattr(P, name + "_stride")[:] = (4096 * 16, 16, 1)
    P.B, P.T, P.H, P.K = 2, 4096, 16, 128
    P.qk_dtype = 1
    P.eps = 1e-6
    for k_, v_ in kw.items():
        setattr(P, k_, v_)
    return P


@pytest.mark.parametrize("kw,code", [
    (dict(B=-1), 1002), (dict(T=1 << 20, H=4096), 1002), (dict(K=96), 1003),
    (dict(qk_dtype=9), 1005), (dict(g_out_dtype=3), 1005), (dict(q_out=None), 1001),
    (dict(beta_out=None), 1001), (dict(k_in=0x1004), 1004),
])
def test_prep_rejects_bad_arguments(lib, kw, code):
    from importlib import import_module
    L = import_module("v100-attention-lab_amd._lib")
    P = _prep_params(L, **kw)
    assert lib.gdn_prep_launch(ctypes.byref(P), None) == code
    assert lib.gdn_prep_launch(None, None) == 1001


def test_prep_misaligned_stride_and_empty(lib):
    from importlib import import_module
    L = import_module("v100-attention-lab_amd._lib")
    P = _prep_params(L)
    P.q_out_stride[2] = 129
    assert lib.gdn_prep_launch(ctypes.byref(P), None) == 1004
    # nothing to do: success without touching the device
    assert lib.gdn_prep_launch(ctypes.byref(_prep_params(L, T=0)), None) == 0


# --------------------------------------------------------------------------
# FLA surface, varlen and prep: host-side validation
# --------------------------------------------------------------------------

@pytest.mark.parametrize("cu,msg", [
    (torch.tensor([0, 10, 64]), None),
    (torch.tensor([0, 10, 64], dtype=torch.int32), None),
    (torch.tensor([1, 10, 64]), "rise from 0"),
    (torch.tensor([0, 30, 20, 64]), "rise from 0"),
    (torch.tensor([0, 10, 63]), "rise from 0"),
    (torch.tensor([0]), "N \\+ 1"),
    (torch.tensor([[0, 64]]), "N \\+ 1"),
    (torch.tensor([0.0, 64.0]), "int64 or int32"),
])
def test_cu_seqlens_validation(pkg, cu, msg):
    from importlib import import_module
    ops = import_module("v100-attention-lab_amd.ops")
    if msg is None:
        c, n = ops._check_cu_seqlens(cu, 64, torch.device("cpu"))
        assert c.dtype == torch.int64 and n == len(cu) - 1
    else:
        with pytest.raises(ValueError, match=msg):
            ops._check_cu_seqlens(cu, 64, torch.device("cpu"))


def test_varlen_needs_one_packed_batch(pkg):
    q, k, v, g, b = _cpu_inputs(B=2)
    with pytest.raises(ValueError, match="B must be 1"):
        pkg.gdn_fwd(q, k, v, g, b, cu_seqlens=torch.tensor([0, 30, 64]))
    q, k, v, g, b = _cpu_inputs(B=1)
    with pytest.raises(ValueError, match="h0 must be \\[N"):
        pkg.gdn_fwd(q, k, v, g, b, torch.zeros(1, 2, 64, 32), cu_seqlens=torch.tensor([0, 30, 64]))


def test_fla_surface_and_prep_reject_cpu_tensors(pkg):
    q, k, v, g, b = _cpu_inputs()
    with pytest.raises(ValueError, match="no CPU path"):
        pkg.chunk_gated_delta_rule(q=q, k=k, v=v, g=g, beta=b, scale=1.0)
    with pytest.raises(ValueError, match="no CPU path"):
        pkg.gdn_prep(q=q, k=k, beta=b, g=g)
    with pytest.raises(ValueError, match="no CPU path"):
        pkg.l2norm(q)
    with pytest.raises(ValueError, match="head_first"):
        pkg.chunk_gated_delta_rule(q, k, v, g[..., None], b, head_first=True)
    with pytest.raises(ValueError, match="K=96"):
        pkg.gdn_prep(q=torch.zeros(1, 4, 2, 96))


# --------------------------------------------------------------------------
# backward entry points: sizes and argument errors before any launch
# --------------------------------------------------------------------------

def test_bwd_workspace_size(lib):
    # cfg2, per (chunk, head), the larger layout (the fp32 walks): the
    # record (T, P, K K^T as C x C, W as C x K, four gate rows), S and dS'
    # (K x V), u and du (C x V), all fp32; then two state scales per walk
    # unit (sequence, head, 16-column slice)
    C, K, V, nrec = 32, 128, 128, 2 * (4096 // 32) * 16
    want = nrec * 4 * ((3 * C * C + C * K + 4 * C) + 2 * K * V + 2 * C * V)
    want += 2 * (2 * 16 * V // 16) * 4
    got = lib.gdn_bwd_workspace_size(2, 4096, 16, 128, 128, 0)
    assert want <= got <= want + 7 * 256
    assert lib.gdn_bwd_workspace_size(2, 4096, 16, 256, 128, 0) == -1
    assert lib.gdn_bwd_workspace_size(2, 4096, 16, 128, 120, 0) == -1
    # packed sequences: chunk slots ceil(T / C) + N
    assert lib.gdn_bwd_workspace_size(3, 100, 2, 64, 32, 3) > 0


def test_bwd_workspace_size_params(lib, pkg):
    """The workspace of the path the params select: the 16-bit walks keep
    T and the gates in the record (C*C + 4C floats), S and dS' in fp16, and
    add T diag(beta) and P as fp16 pairs; fp32 inputs (or a dO of another
    dtype, or one not 4-byte aligned) take the general size."""
    C, K, V, H = 32, 128, 128, 16
    nrec = 2 * (4096 // C) * H
    want16 = nrec * (4 * (C * C + 4 * C) + 2 * 2 * K * V + 4 * 2 * C * V + 2 * 4 * C * C) + 2 * (2 * H * V // 16) * 4
    general = lib.gdn_bwd_workspace_size(2, 4096, H, K, V, 0)
    P = _bwd_params(pkg._lib, B=2, T=4096, H=H, K=K, V=V, qkv_dtype=1, do_dtype=1)
    got = lib.gdn_bwd_workspace_size_params(ctypes.byref(P))
    assert want16 <= got <= want16 + 8 * 256
    assert got < 0.6 * general
    for kw in (dict(qkv_dtype=0, do_dtype=0), dict(qkv_dtype=1, do_dtype=0), dict(qkv_dtype=1, do_dtype=1, d_o=0x3002)):
        P = _bwd_params(pkg._lib, B=2, T=4096, H=H, K=K, V=V, **kw)
        assert lib.gdn_bwd_workspace_size_params(ctypes.byref(P)) == general
    P = _bwd_params(pkg._lib, B=2, T=4096, H=H, K=256, V=V)
    assert lib.gdn_bwd_workspace_size_params(ctypes.byref(P)) == -1
    assert lib.gdn_bwd_workspace_size_params(None) == -1


def test_bwd_workspace_bounded_in_t(lib, pkg):
    """Without cu_seqlens the default workspace holds at most 256 chunks per
    sequence: at cfg3's length (T = 16384, 512 chunks) it is the 8192-row
    layout plus three fp32 states (the checkpoint at the second segment's
    start and the two carried state gradients); the one-pass layout grows
    with T.  Packed sequences keep the one-pass layout."""
    H, K, V = 16, 128, 128
    state = 2 * H * K * V * 4
    sz = lambda **kw: lib.gdn_bwd_workspace_size_params(ctypes.byref(_bwd_params(pkg._lib, **kw)))
    seg = lambda n, **kw: lib.gdn_bwd_segment_workspace_size(ctypes.byref(_bwd_params(pkg._lib, **kw)), n)
    w8 = sz(B=2, T=8192, H=H, K=K, V=V)
    assert sz(B=2, T=16384, H=H, K=K, V=V) == w8 + 3 * state
    assert sz(B=2, T=65536, H=H, K=K, V=V) == w8 + 9 * state
    assert seg(10 ** 6, B=2, T=16384, H=H, K=K, V=V) > 1.99 * w8
    assert seg(256, B=2, T=16384, H=H, K=K, V=V) == w8 + 3 * state
    # shorter segments take less, until the checkpoints (one state per
    # segment) outweigh the layout
    assert seg(64, B=2, T=16384, H=H, K=K, V=V) < seg(128, B=2, T=16384, H=H, K=K, V=V) < w8
    assert seg(4, B=2, T=16384, H=H, K=K, V=V) > seg(8, B=2, T=16384, H=H, K=K, V=V)
    assert seg(0, B=2, T=16384, H=H, K=K, V=V) == -1
    # the dtype-free size is bounded the same way
    assert lib.gdn_bwd_workspace_size(2, 65536, H, K, V, 0) < 1.03 * lib.gdn_bwd_workspace_size(2, 8192, H, K, V, 0)
    # packed sequences (B of them in T rows): one pass, whatever the
    # segment length asked for
    packed = sz(B=2, T=16384, H=H, K=K, V=V, cu_seqlens=0x2000)
    assert packed > 1.99 * sz(B=1, T=8192, H=H, K=K, V=V)
    assert seg(4, B=2, T=16384, H=H, K=K, V=V, cu_seqlens=0x2000) == packed


def _bwd_params(L, **kw):
    P = L.GdnBwdParams()
    fake = 0x1000  # never dereferenced: every case below returns before a launch
    for n in ("q", "k", "v", "g", "beta", "d_o", "dq", "dk", "dv", "dg", "dbeta"):
        setattr(P, n, fake)
    P.B, P.T, P.H, P.K, P.V = 2, 64, 2, 64, 32
    P.workspace = 0x100000
    P.workspace_bytes = 1 << 40
    P.qkv_dtype, P.g_dtype, P.beta_dtype, P.do_dtype = 1, 0, 0, 1
    P.scale = 1.0
    for k_, v_ in kw.items():
        setattr(P, k_, v_)
    return P


@pytest.mark.parametrize("kw,code", [
    (dict(K=256), 1003), (dict(V=24), 1002), (dict(B=0), 1002), (dict(do_dtype=4), 1005),
    (dict(d_o=None), 1001), (dict(dg=None), 1001), (dict(workspace=None), 1006),
    (dict(workspace=0x100010), 1006), (dict(workspace_bytes=1024), 1006),
    (dict(q=0x1008), 1004),
])
def test_bwd_rejects_bad_arguments(lib, kw, code):
    from importlib import import_module
    L = import_module("v100-attention-lab_amd._lib")
    assert lib.gdn_bwd_launch(ctypes.byref(_bwd_params(L, **kw)), None) == code
    assert lib.gdn_bwd_launch(None, None) == 1001
    assert "workspace" in lib.gdn_fwd_status_string(1006).decode()


def test_bwd_python_validation(pkg):
    q, k, v, g, b = _cpu_inputs(K=256)
    with pytest.raises(ValueError, match="K=256"):
        pkg.gdn_bwd(q, k, v, g, b, None, torch.zeros(1, 64, 2, 32, dtype=torch.float16))
    q, k, v, g, b = _cpu_inputs()
    with pytest.raises(ValueError, match="do must"):
        pkg.gdn_bwd(q, k, v, g, b, None, torch.zeros(1, 64, 2, 16, dtype=torch.float16))
    with pytest.raises(ValueError, match="dfinal"):
        pkg.gdn_bwd(q, k, v, g, b, None, torch.zeros(1, 64, 2, 32, dtype=torch.float16),
                    torch.zeros(1, 2, 64, 32, dtype=torch.float16))


# --------------------------------------------------------------------------
# gdn_fwd_launch_noalloc: argument and size checks come before any HIP call
# --------------------------------------------------------------------------

def test_noalloc_scratch_size(lib):
    assert lib.gdn_fwd_scratch_bytes() == 32 << 20


@pytest.mark.parametrize("kw,code", [
    (dict(B=0), 1002), (dict(V=24), 1002), (dict(K=96), 1003), (dict(qkv_dtype=7), 1005),
    (dict(q=0x1008), 1004), (dict(final_state=None), 1001),
    # (calls whose records do not fit the scratch array run on a kernel
    # without workspace: tests/test_zz_no_alloc.py, on the GPU)
])
def test_noalloc_rejects_before_launch(lib, pkg, kw, code):
    P = _params(pkg._lib, **kw)
    assert lib.gdn_fwd_launch_noalloc(ctypes.byref(P), None) == code
    assert lib.gdn_fwd_launch_noalloc(None, None) == 1001
    assert "scratch" in lib.gdn_fwd_status_string(1007).decode()


def test_auto_block_v_matches_sweep(pkg):
    """The launcher's BV for 32-row chunks is the fastest one measured by
    `bench.py --sweep` at every config (profiles/gdn_fwd_sweep_chunk_block_v.json)."""
    import json
    dt = {"f16": torch.float16, "bf16": torch.bfloat16}
    with open(os.path.join(REPO, "profiles", "gdn_fwd_sweep_chunk_block_v.json")) as f:
        rows = json.load(f)["rows"]
    assert len(rows) >= 4
    for r in rows:
        best = min((t, key) for key, t in r["ms_per_step"].items() if key.startswith("C32_"))[1]
        assert pkg.auto_block_v(r["B"], r["H"], r["K"], r["V"], 32, dt[r["dtype"]]) == int(best.split("BV")[1]), r


def test_traffic_profile_tracks_sources(monkeypatch):
    """bench.py reports roofline.traffic from the committed rocprofv3 profile
    only while the kernel sources hash to the digest recorded in it; a stale
    profile gives null and says so."""
    import importlib.util
    spec = importlib.util.spec_from_file_location("_bench", os.path.join(REPO, "bench.py"))
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    for config in ("cfg1", "cfg2", "cfg3", "cfg4", "cfg2_c64"):
        with open(bench.traffic_path(config)) as f:
            rec = json.load(f)
        assert rec["config"] == config and rec["sources"] and rec["commit"] and rec["kernels"]
        assert rec["kernels"] and all(bench.is_library_kernel(k) for k in rec["kernels"])
        assert rec["dispatches_per_kernel_per_launch"] == bench.segments_per_launch(config)
        nbytes, note = bench.load_traffic(config)
        if rec["sources"] == bench.sources_digest(config):
            assert nbytes == rec["hbm_bytes_per_launch"] and rec["commit"] in note
        else:
            assert nbytes is None and note.startswith("stale")
    # the 64-row path's digest covers its own kernel file, not the 32-row one's
    assert bench.sources_digest("cfg2_c64") != bench.sources_digest("cfg2")
    monkeypatch.setattr(bench, "sources_digest", lambda config: "0" * 16)
    nbytes, note = bench.load_traffic("cfg2")
    assert nbytes is None and note.startswith("stale")
