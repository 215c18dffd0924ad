"""Benchmark of the MI355X fused chunked GDN forward (BASELINE.json metric).

``python bench.py [--gpus 1] [--steps K] [--warmup W]`` times K back-to-back
forwards (after W untimed ones, preceded by 0.3 s of untimed calls that bring
the GPU out of its idle clock) of the headline workload (configs[2]: fp16, B=2, H=16, T=4096,
K=V=128, C=32) with inputs already resident in HBM, and prints ONE JSON line
with tokens/s, ms per step, the roofline position of the kernel and a CPU
baseline (the oracle's chunked-UT restatement of gdn_ref.py:48-99 on this
host's cores).

A "step" is one ``gdn_fwd`` call over the whole batch: one ``gdn_fwd_launch``
(for fp16 at C=32, two kernels: the per-chunk records, then the scan).
Extra fields report the C=64 variant, a cold-cache timing (caches flushed
with a 512 MiB write between launches, each launch timed with its own
events) and the fused input preparation (``gdn_prep``: L2-norm of q and k,
sigmoid beta, logsigmoid g) and the backward (``gdn_bwd``) on the same
shapes.  ``--config`` selects another BASELINE config for exploration;
``--workload prep`` / ``--workload bwd`` time only the input preparation /
the backward; the driver's line is the default.
"""

from __future__ import annotations

import argparse
import importlib
import json
import os
import platform
import statistics
import sys
import time

import torch

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, 8 TB/s
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16/bf16 MFMA

CONFIGS = {
    # name: (B, T, H, K, V, dtype, chunk, with_h0)
    "cfg1": (2, 1024, 16, 128, 128, torch.float16, 32, False),
    "cfg2": (2, 4096, 16, 128, 128, torch.float16, 32, False),
    "cfg2_c64": (2, 4096, 16, 128, 128, torch.float16, 64, False),
    "cfg3": (2, 16384, 16, 128, 128, torch.float16, 32, False),
    "cfg4": (4, 4096, 16, 128, 128, torch.bfloat16, 32, True),
    # exploration only: the configs[4] shape in fp16 (64 heads on the
    # two-launch path)
    "cfg4_f16": (4, 4096, 16, 128, 128, torch.float16, 32, True),
    # sweep only: the reference's own autotune shape (bench_gdn.py:120-121,
    # B2 T2048 H8) and a K = V = 64 shape, both with fewer (b, h, 16-column)
    # units than the 256 CUs
    "ref_sweep": (2, 2048, 8, 128, 128, torch.float16, 32, False),
    "k64": (2, 4096, 16, 64, 64, torch.float16, 32, False),
    "k64_bf16": (2, 4096, 16, 64, 64, torch.bfloat16, 32, False),
    # sweep only: the headline shape in bf16 (where the 16-bit input
    # conversion weighs most)
    "cfg2_bf16": (2, 4096, 16, 128, 128, torch.bfloat16, 32, False),
}
SWEEP_CONFIGS = ("cfg1", "cfg2", "cfg3", "cfg4", "cfg4_f16", "ref_sweep", "k64", "k64_bf16", "cfg2_bf16")

DTYPE_NAME = {torch.float16: "f16", torch.bfloat16: "bf16", torch.float32: "f32"}


def make_inputs(B, T, H, K, V, dtype, with_h0, device, seed=0):
    """BASELINE.json recipe: q, k L2-normalised N(0,1); v N(0,1); beta =
    sigmoid(N(0,1)); g = logsigmoid(N(0,1)); h0 = 0.1 N(0,1) (K x V)."""
    gen = torch.Generator(device=device).manual_seed(seed)

    def l2n(x):
        return x / torch.sqrt(x.float().pow(2).sum(-1, keepdim=True) + 1e-6).to(x.dtype)

    q = l2n(torch.randn(B, T, H, K, generator=gen, device=device)).to(dtype)
    k = l2n(torch.randn(B, T, H, K, generator=gen, device=device)).to(dtype)
    v = torch.randn(B, T, H, V, generator=gen, device=device).to(dtype)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=gen, device=device)).float()
    g = torch.nn.functional.logsigmoid(torch.randn(B, T, H, generator=gen, device=device)).float()
    h0 = (0.1 * torch.randn(B, H, K, V, generator=gen, device=device)).float() if with_h0 else None
    return q, k, v, g, beta, h0


def algorithmic_bytes(B, T, H, K, V, in_bytes, with_h0):
    """Compulsory HBM bytes: per head-token q, k, v in and o out at the input
    width plus fp32 g and beta; per (b, h) the fp32 K x V final state (and
    h0 when given)."""
    return B * T * H * (in_bytes * (2 * K + 2 * V) + 8) + B * H * 4 * K * V * (2 if with_h0 else 1)


def algorithmic_flops(B, T, H, K, V, C):
    """MFMA flops: per head-token 4CK (K K^T, Q K^T) + 2CV (P u) + 6KV
    (W S, Q S, K^T u)."""
    return B * T * H * (4 * C * K + 2 * C * V + 6 * K * V)


def make_raw_inputs(B, T, H, K, dtype, device, seed=0):
    """Un-normalised q, k (``dtype``) and gate logits (fp32): the inputs of
    the fused preparation."""
    gen = torch.Generator().manual_seed(seed)
    qr = torch.randn(B, T, H, K, generator=gen).to(dtype).to(device)
    kr = torch.randn(B, T, H, K, generator=gen).to(dtype).to(device)
    br = torch.randn(B, T, H, generator=gen).to(device)
    gr = torch.randn(B, T, H, generator=gen).to(device)
    return qr, kr, br, gr


def prep_bytes(B, T, H, K, in_bytes):
    """Algorithmic bytes of one preparation launch: q and k read and written
    once, beta and g logits read and written once in fp32."""
    return 4 * B * T * H * K * in_bytes + 4 * B * T * H * 4


def time_prep(pkg, B, T, H, K, dtype, steps, warmup):
    """Times the preparation kernel through the C ABI with a prebuilt
    parameter block (outputs allocated once), so that the events bracket
    back-to-back kernels rather than Python argument handling."""
    import ctypes
    ops = importlib.import_module("v100-attention-lab_amd.ops")
    qr, kr, br, gr = make_raw_inputs(B, T, H, K, dtype, torch.device("cuda:0"))
    outs = pkg.gdn_prep(qr, kr, br, gr)          # validates; allocates the outputs
    params, _ = ops._prep_plan(qr, kr, br, gr, 1e-6, torch.float32, False)
    P = pkg._lib.GdnPrepParams.from_buffer_copy(params)
    for name, t, o in zip(("q", "k", "beta", "g"), (qr, kr, br, gr), outs):
        setattr(P, f"{name}_in", t.data_ptr())
        setattr(P, f"{name}_out", o.data_ptr())
    lib = pkg.load_library()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def launch():
        status = lib.gdn_prep_launch(ctypes.byref(P), stream)
        if status != 0:
            raise RuntimeError(f"gdn_prep_launch failed ({status})")

    ms = time_steps(launch, steps, warmup)
    nb = prep_bytes(B, T, H, K, torch.finfo(dtype).bits // 8)
    gbs = nb / (ms / 1e3) / 1e9
    return {"ms_per_step": round(ms, 5), "bytes_per_launch": nb, "achieved_gbs": round(gbs, 2),
            "peak_gbs": HBM_PEAK_GBS, "frac": round(gbs / HBM_PEAK_GBS, 5)}


def bwd_bytes(B, T, H, K, V, in_bytes):
    """Algorithmic bytes of one backward: q, k, v, dO read and dq, dk, dv
    written in the input dtype, g, beta read and dg, dbeta written in fp32."""
    return B * T * H * (in_bytes * (4 * K + 3 * V) + 16)


def time_bwd(pkg, q, k, v, g, beta, h0, steps, warmup):
    do = torch.randn(v.shape, generator=torch.Generator().manual_seed(1)).to(v.dtype).to(v.device)
    ms = time_steps(lambda: pkg.gdn_bwd(q, k, v, g, beta, h0, do, None, need_dh0=h0 is not None),
                    steps, warmup)
    B, T, H, K = q.shape
    nb = bwd_bytes(B, T, H, K, v.shape[-1], q.element_size())
    gbs = nb / (ms / 1e3) / 1e9
    return {"ms_per_step": round(ms, 5), "tokens_per_s": round(B * T / (ms / 1e3), 1),
            "bytes_per_launch": nb, "achieved_gbs": round(gbs, 2), "frac": round(gbs / HBM_PEAK_GBS, 6)}


PREWARM_S = 0.3


def prewarm(fn, seconds=PREWARM_S):
    """Runs ``fn`` back to back, untimed, for ``seconds`` of wall time.  An
    idle MI355X raises its clock only after tens of milliseconds of sustained
    work: five warmup steps of ~0.1 ms leave the timed steps of a short run
    about 10 % slower than the same steps after this.  Returns the calls
    made."""
    n = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        fn()
        n += 1
        if n % 64 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    return n


def time_steps(fn, steps, warmup):
    """Warm up (the clock pre-warm, then ``warmup`` calls), then time exactly
    ``steps`` back-to-back calls between two events on the current stream
    (the stream the kernel is launched on)."""
    prewarm(fn)
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def time_cold(fn, reps, flush_bytes=512 << 20):
    """Per-launch time with L2/MALL flushed by a 512 MiB write before each
    launch; the flush is outside the events."""
    buf = torch.empty(flush_bytes // 4, dtype=torch.float32, device="cuda")
    ts = []
    for _ in range(reps):
        buf.fill_(1.0)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        fn()
        e1.record()
        torch.cuda.synchronize()
        ts.append(e0.elapsed_time(e1))
    del buf
    return statistics.median(ts)


def cpu_baseline(B, T, H, K, V, dtype, C, budget_s=12.0):
    """The oracle's chunked UT (fp32 PyTorch, same op order as
    gdn_ref.py:48-99) on this host's cores over the full workload; median of
    the runs that fit in ``budget_s`` after one warmup."""
    from oracle import gdn_oracle as ref

    n = len(os.sched_getaffinity(0))
    torch.set_num_threads(n)
    q, k, v, g, beta, _ = ref.make_inputs_baseline(B, T, H, K, V, seed=0, dtype=dtype)
    ref.chunked_ut(q, k, v, beta, g, C=C)  # warmup
    ts = []
    t_start = time.time()
    while len(ts) < 3 or (time.time() - t_start < budget_s and len(ts) < 30):
        t0 = time.perf_counter()
        ref.chunked_ut(q, k, v, beta, g, C=C)
        ts.append(time.perf_counter() - t0)
    ms = 1e3 * statistics.median(ts)
    cpu_model = platform.processor() or ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {
        "value": round(B * T / (ms / 1e3), 1),
        "unit": "tokens/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"oracle chunked_ut (fp32 torch CPU, gdn_ref.py:48-99 op order) on the full "
                   f"workload B{B} H{H} T{T} K{K} V{V} C{C}; median of {len(ts)} runs after 1 "
                   f"warmup; {n} threads on '{cpu_model}'"),
        "ms_per_step": round(ms, 3),
    }


# The sources the 32-row forward's two launches are built from (the record
# and scan kernels, the headers they include, the dispatch that launches
# them): the code a forward traffic profile measures.  64-row chunks run the
# record and scan kernels of gdn_fwd_c64.hip (FWD_SOURCES_C64).
FWD_SOURCES = ("gdn_fwd_api.hip", "gdn_fwd_kernel.h", "gdn_fwd_pipe.h", "gdn_fwd_scan32.hip")
FWD_SOURCES_C64 = ("gdn_fwd_api.hip", "gdn_fwd_kernel.h", "gdn_tiles_f16.h", "gdn_fwd_c64.hip")


def sources_digest(config="cfg2"):
    """sha256 (first 16 hex digits) over the HIP sources of the forward path
    that `config` runs (FWD_SOURCES, or FWD_SOURCES_C64 for 64-row chunks),
    names and bytes: it identifies the build a traffic profile was measured
    on, also on a machine without the git history."""
    import hashlib
    d = os.path.join(REPO, "v100-attention-lab_amd", "csrc")
    h = hashlib.sha256()
    for name in FWD_SOURCES_C64 if CONFIGS[config][6] == 64 else FWD_SOURCES:
        h.update(name.encode())
        with open(os.path.join(d, name), "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def traffic_path(config):
    return os.path.join(REPO, "profiles", f"gdn_fwd_{config}_traffic.json")


def load_traffic(config):
    """HBM bytes per launch measured by rocprofv3 FETCH_SIZE/WRITE_SIZE
    (profiles/gdn_fwd_<config>_traffic.json) and a note on where they come
    from.  The bytes are None when no profile exists or when it was taken on
    other kernel sources than the ones present (its ``sources`` digest differs
    from ``sources_digest(config)``): a stale figure is not reported as this
    build's."""
    try:
        with open(traffic_path(config)) as f:
            rec = json.load(f)
    except (OSError, ValueError):
        return None, "no traffic profile for this config"
    where = f"profiles/gdn_fwd_{config}_traffic.json, commit {rec.get('commit', '?')}"
    if rec.get("sources") != sources_digest(config):
        return None, f"stale: {where} measured other kernel sources"
    return rec.get("hbm_bytes_per_launch"), where


def is_library_kernel(name):
    """A kernel of this library, as rocprofv3 names it (mangled or
    demangled)."""
    return name.startswith("_ZN3gdn") or name.startswith("void gdn::")


def segments_per_launch(config):
    """Segments one forward call at `config` runs in (each launches the
    record and the scan kernel once): the records of at most 256 chunks of
    32 rows, or 64 chunks of 64 rows, per sequence and head
    (gdn_fwd_api.hip kSegChunks, gdn_fwd_kernel.h kSegC64)."""
    B, T, H, K, V, dtype, C, with_h0 = CONFIGS[config]
    nch = -(-T // C)
    return -(-nch // (256 if C == 32 else 64))


def write_traffic(config, fetch_csv, write_csv, copy_fetch_csv, copy_write_csv):
    """Writes profiles/gdn_fwd_<config>_traffic.json from four rocprofv3
    ``--pmc`` CSVs: FETCH_SIZE and WRITE_SIZE of a ``bench.py --steps 5
    --warmup 1 --no-extras --no-cpu-baseline`` run, and the same two counters
    of ``bench.py --calibrate-copy`` (a 256 MiB copy, which gives each
    counter's scale).  Each library kernel (``gdn::`` names, mangled or not)
    runs once per segment of a launch: per kernel the median KiB per
    dispatch times the segments per launch (segments_per_launch), summed
    over the kernels, scaled.  Run where the git history is, after the GPU
    run."""
    import csv
    import subprocess

    def medians(path):
        per = {}
        with open(path) as f:
            for r in csv.DictReader(f):
                per.setdefault(r["Kernel_Name"], []).append(float(r["Counter_Value"]))
        return {k: statistics.median(v) for k, v in per.items()}

    def scale(path):
        copy = [v for k, v in medians(path).items() if "copyBuffer" in k or "copy_kernel" in k]
        return (256 << 10) / max(copy)  # the 256 MiB copy in KiB / the counter's KiB

    fetch, write = medians(fetch_csv), medians(write_csv)
    kernels = sorted(k for k in fetch if is_library_kernel(k))
    fs, ws = scale(copy_fetch_csv), scale(copy_write_csv)
    nseg = segments_per_launch(config)
    per_kernel = {k: {"fetch_kib": fetch[k], "write_kib": write.get(k)} for k in kernels}
    rd = sum(fetch[k] for k in kernels) * nseg * 1024 * fs
    wr = sum(write[k] for k in kernels) * nseg * 1024 * ws
    B, T, H, K, V, dtype, C, with_h0 = CONFIGS[config]
    alg = algorithmic_bytes(B, T, H, K, V, torch.finfo(dtype).bits // 8, with_h0)
    git = lambda *a: subprocess.run(["git", *a], cwd=REPO, capture_output=True, text=True).stdout.strip()
    rec = {"config": config, "commit": git("rev-parse", "--short", "HEAD"),
           "uncommitted_changes": bool(git("status", "--porcelain", "--", "v100-attention-lab_amd/csrc")),
           "sources": sources_digest(config), "kernels": per_kernel, "dispatches_per_kernel_per_launch": nseg,
           "fetch_scale": round(fs, 6), "write_scale": round(ws, 6),
           "bytes_read_per_launch": round(rd), "bytes_written_per_launch": round(wr),
           "hbm_bytes_per_launch": round(rd + wr), "algorithmic_bytes_per_launch": alg,
           "traffic_over_algorithmic": round((rd + wr) / alg, 4)}
    with open(traffic_path(config), "w") as f:
        json.dump(rec, f, indent=1)
        f.write("\n")
    print(json.dumps(rec, indent=1))


def phase_stamps(pkg, config):
    """MFMA utilisation of the contraction phases, from the measurement build
    (``build.py --phase-stamps``: the same kernels with s_memtime stamps around
    each MFMA phase, summed per wave).  Per phase: MFMA count x the cycles one
    MFMA keeps a SIMD busy (measured by the build's probe: 256 workgroups of
    four waves, four independent accumulators each) / the phase's stamped
    cycles, on the SIMDs that run it.  The scan's phases are K S -> u -> state
    update (SCAN), Q S and P u (OUT), Q K^T with the decay mask (P); the record
    kernel's is K K^T with A's gates and mask."""
    import ctypes
    import numpy as np
    bmod = importlib.import_module("v100-attention-lab_amd.build")
    lib = pkg.load_library(bmod.STAMPS_LIB_PATH)  # first load of this process
    lib.gdn_phase_read.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    lib.gdn_phase_mfma_probe.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                         ctypes.c_void_p]
    dev = torch.device("cuda:0")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    out = torch.empty(256 * 256, device=dev)
    cyc = torch.zeros(1024, dtype=torch.int64, device=dev)
    for _ in range(3):
        assert lib.gdn_phase_mfma_probe(out.data_ptr(), cyc.data_ptr(), 256, 2000, stream) == 0
    torch.cuda.synchronize()
    cyc_mfma = float(cyc.double().median()) / (4 * 2000)

    B, T, H, K, V, dtype, C, with_h0 = CONFIGS[config]
    q, k, v, g, beta, h0 = make_inputs(B, T, H, K, V, dtype, with_h0, dev)
    step = lambda: pkg.gdn_fwd(q, k, v, g, beta, h0, scale=1.0, chunk_size=C)
    ms = time_steps(step, 20, 5)
    assert lib.gdn_phase_clear() == 0
    step()
    torch.cuda.synchronize()
    scan = np.zeros(1024 * 8 * 8, dtype=np.uint64)
    rec = np.zeros(16384 * 4, dtype=np.uint64)
    assert lib.gdn_phase_read(scan.ctypes.data, rec.ctypes.data) == 0
    scan = scan.reshape(1024, 8, 8).astype(np.float64)
    rec = rec.reshape(16384, 4).astype(np.float64)
    if not (scan[:, :, 0] > 0).any():
        raise RuntimeError(f"{config}: no stamps recorded (the two-launch 32-row path did not run)")
    phases = {}
    for role, names in ((1, ("SCAN: K S, u, state update", None)), (2, ("OUT: Q S", "OUT: P u")),
                        (3, ("P: Q K^T, decay, mask", None))):
        d = scan[scan[:, :, 0] == role]
        for col, name in enumerate(names):
            if name is None:
                continue
            window = float(d[:, 2 + col].sum())
            mfma = float((d[:, 4 + col] * d[:, 1]).sum())
            phases[name] = {"waves": int(len(d)), "mfma": int(mfma), "busy_cycles": mfma * cyc_mfma,
                            "window_cycles": window}
    r = rec[rec[:, 0] > 0]
    phases["records: K K^T, A"] = {"waves": int(len(r)), "mfma": int(r[:, 2].sum()),
                                   "busy_cycles": float(r[:, 2].sum()) * cyc_mfma,
                                   "window_cycles": float(r[:, 1].sum())}
    for ph in phases.values():
        ph["util"] = round(ph["busy_cycles"] / ph["window_cycles"], 4)
        # the same against the nominal 16 cycles per v_mfma_f32_16x16x32_f16
        # (2.5 PFLOP/s dense fp16 on 256 CUs x 4 SIMDs at 2.4 GHz)
        ph["util_nominal16"] = round(ph["mfma"] * 16.0 / ph["window_cycles"], 4)
    scan_names = [n for n in phases if not n.startswith("records")]
    busy = sum(phases[n]["busy_cycles"] for n in scan_names)
    win = sum(phases[n]["window_cycles"] for n in scan_names)
    busy_all = busy + phases["records: K K^T, A"]["busy_cycles"]
    win_all = win + phases["records: K K^T, A"]["window_cycles"]
    mfma_scan = sum(phases[n]["mfma"] for n in scan_names)
    mfma_all = mfma_scan + phases["records: K K^T, A"]["mfma"]
    for ph in phases.values():
        ph["busy_cycles"] = round(ph["busy_cycles"])
        ph["window_cycles"] = round(ph["window_cycles"])
    # per role of the scan: cycles in barriers (the LDS drain before each
    # s_barrier and the wait for the other waves) and the loop's cycles, per
    # chunk, averaged over the waves of the role
    roles = {}
    for role, name in ((1, "SCAN"), (2, "OUT"), (3, "PQK"), (4, "LOAD")):
        d = scan[(scan[:, :, 0] == role) & (scan[:, :, 1] > 0)]
        if len(d):
            nch = float(d[:, 1].sum())
            roles[name] = {"waves": int(len(d)), "barrier_cycles_per_chunk": round(float(d[:, 6].sum()) / nch, 1),
                           "loop_cycles_per_chunk": round(float(d[:, 7].sum()) / nch, 1)}
    print(json.dumps({"metric": "MFMA utilisation of the contraction phases (s_memtime phase windows)",
                      "config": config, "B": B, "T": T, "H": H, "K": K, "V": V, "chunk_size": C,
                      "mfma_cycles_per_instruction": round(cyc_mfma, 3),
                      "stamped_ms_per_step": round(ms, 5),
                      "scan_contraction_util": round(busy / win, 4),
                      "all_contraction_util": round(busy_all / win_all, 4),
                      "scan_contraction_util_nominal16": round(mfma_scan * 16.0 / win, 4),
                      "all_contraction_util_nominal16": round(mfma_all * 16.0 / win_all, 4),
                      "phases": phases, "roles": roles}), flush=True)


# (C, BV) combinations of the sweep: 32-row chunks take BV 16 or 32 on the
# two-launch path (fp16) or the fused kernel (bf16) and 64 on the phased
# kernel; 64-row chunks run at BV 16.
SWEEP = ((32, 16), (32, 32), (32, 64), (64, 16))


def sweep(pkg, steps, warmup, names=SWEEP_CONFIGS):
    """Times every (C, BV) of SWEEP at every config (configs[2] with C = 64 is
    configs[2] as well) and prints one JSON line per config with the times
    and the launcher's automatic BV for 32-row chunks."""
    dev = torch.device("cuda:0")
    for name in names:
        B, T, H, K, V, dtype, _, with_h0 = CONFIGS[name]
        q, k, v, g, beta, h0 = make_inputs(B, T, H, K, V, dtype, with_h0, dev)
        res = {}
        for C, bv in SWEEP:
            fn = lambda: pkg.gdn_fwd(q, k, v, g, beta, h0, scale=1.0, chunk_size=C, block_v=bv)
            res[f"C{C}_BV{bv}"] = round(time_steps(fn, steps, warmup), 5)
        best = min((t, key) for key, t in res.items() if key.startswith("C32_"))[1]
        print(json.dumps({"config": name, "B": B, "T": T, "H": H, "K": K, "V": V,
                          "dtype": DTYPE_NAME[dtype], "ms_per_step": res,
                          "auto_block_v_c32": pkg.auto_block_v(B, H, K, V, 32, dtype),
                          "best_c32": best}), flush=True)
        del q, k, v, g, beta, h0
        torch.cuda.empty_cache()


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--config", default="cfg2", choices=sorted(CONFIGS))
    ap.add_argument("--block-v", type=int, default=None)
    ap.add_argument("--workload", default="fwd", choices=["fwd", "prep", "bwd"],
                    help="fwd: the GDN forward (default); prep: only the fused input "
                         "preparation; bwd: only the backward (gdn_bwd)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extras", action="store_true", help="skip the C=64 and cold-cache lines")
    ap.add_argument("--sweep-configs", default=None,
                    help="comma-separated configs for --sweep (default: all of SWEEP_CONFIGS)")
    ap.add_argument("--sweep", action="store_true",
                    help="time every (chunk, block_v) at every config (one JSON line per config)")
    ap.add_argument("--phase-stamps", action="store_true",
                    help="MFMA utilisation of the contraction phases from the stamps build "
                         "(lib/libgdn_mi355x_stamps.so, built by build.py --phase-stamps)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run only a plain 256 MiB device copy (scale for rocprof byte counters)")
    ap.add_argument("--write-traffic", nargs=4, metavar=("FETCH_CSV", "WRITE_CSV", "COPY_FETCH_CSV",
                                                          "COPY_WRITE_CSV"),
                    help="no GPU: write profiles/gdn_fwd_<config>_traffic.json from rocprofv3 "
                         "--pmc FETCH_SIZE / WRITE_SIZE CSVs of a bench run and of --calibrate-copy")
    args = ap.parse_args()

    if args.write_traffic:
        write_traffic(args.config, *args.write_traffic)
        return

    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested). The GDN "
              "forward shards over (batch, head) with no communication; multi-GPU runs are not "
              "part of this build.", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py: no ROCm GPU visible", file=sys.stderr)
        sys.exit(1)

    if args.calibrate_copy:
        # A plain copy of known size: rocprofv3 FETCH_SIZE / WRITE_SIZE of this
        # kernel divided by 256 MiB gives the counters' scale on this device.
        n = 256 << 20
        src = torch.ones(n // 4, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibration": "copy", "bytes_read": n, "bytes_written": n, "launches": 3}))
        return

    pkg = importlib.import_module("v100-attention-lab_amd")
    if args.phase_stamps:
        phase_stamps(pkg, args.config)
        return
    if args.sweep:
        sweep(pkg, min(args.steps, 50), min(args.warmup, 10),
              args.sweep_configs.split(",") if args.sweep_configs else SWEEP_CONFIGS)
        return
    dev = torch.device("cuda:0")
    B, T, H, K, V, dtype, C, with_h0 = CONFIGS[args.config]
    if args.workload == "prep":
        r = time_prep(pkg, B, T, H, K, dtype, args.steps, args.warmup)
        print(json.dumps({
            "metric": "GDN input prep bytes/s (l2norm q,k; sigmoid beta; logsigmoid g)",
            "value": round(r["bytes_per_launch"] / (r["ms_per_step"] / 1e3), 1), "unit": "B/s",
            "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": r["ms_per_step"], "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": DTYPE_NAME[dtype], "data": "synthetic (seed 0)",
            "config": {"workload": f"gdn_prep {args.config}", "B": B, "T": T, "H": H, "K": K},
            "roofline": {"bound": "hbm", "achieved": r["achieved_gbs"], "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": r["frac"], "traffic": None}}), flush=True)
        return
    q, k, v, g, beta, h0 = make_inputs(B, T, H, K, V, dtype, with_h0, dev)
    if args.workload == "bwd":
        r = time_bwd(pkg, q, k, v, g, beta, h0, args.steps, args.warmup)
        print(json.dumps({
            "metric": "GDN bwd tokens/sec (dq, dk, dv, dg, dbeta from dO)",
            "value": r["tokens_per_s"], "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": r["ms_per_step"], "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": DTYPE_NAME[dtype],
            "data": "synthetic (BASELINE.json recipe, seed 0)",
            "config": {"workload": f"gdn_bwd {args.config}", "B": B, "T": T, "H": H, "K": K, "V": V},
            "roofline": {"bound": "hbm", "achieved": r["achieved_gbs"], "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": r["frac"], "traffic": None}}), flush=True)
        return

    def step(chunk=C):
        return pkg.gdn_fwd(q, k, v, g, beta, h0, scale=1.0, chunk_size=chunk, block_v=args.block_v)

    ms = time_steps(step, args.steps, args.warmup)
    tokens_per_s = B * T / (ms / 1e3)
    in_bytes = torch.finfo(dtype).bits // 8
    alg_bytes = algorithmic_bytes(B, T, H, K, V, in_bytes, with_h0)
    alg_flops = algorithmic_flops(B, T, H, K, V, C)
    achieved_gbs = alg_bytes / (ms / 1e3) / 1e9
    achieved_tflops = alg_flops / (ms / 1e3) / 1e12
    bv = args.block_v or pkg.auto_block_v(B, H, K, V, C, dtype)
    traffic, traffic_note = load_traffic(args.config)

    line = {
        "metric": "GDN fwd tokens/sec at B2 H16 K=V=128 T=4096; % MFMA/HBM roofline",
        "value": round(tokens_per_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "prewarm_s": PREWARM_S,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": DTYPE_NAME[dtype],
        "data": "synthetic (BASELINE.json recipe, seed 0)",
        "config": {"workload": f"gdn_fwd {args.config}", "B": B, "T": T, "H": H, "K": K, "V": V,
                   "chunk_size": C, "block_v": bv, "h0": with_h0,
                   "inputs": f"q,k,v {DTYPE_NAME[dtype]}; g,beta f32; o {DTYPE_NAME[dtype]}; "
                             "final_state f32 [B,H,K,V]"},
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved_gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved_gbs / HBM_PEAK_GBS, 5),
            "traffic": traffic,
            "traffic_profile": traffic_note,
        },
        "head_tokens_per_s": round(B * T * H / (ms / 1e3), 1),
        "mfma": {"algorithmic_tflops": round(achieved_tflops, 3), "peak_tflops": MFMA_F16_PEAK_TFLOPS,
                 "frac": round(achieved_tflops / MFMA_F16_PEAK_TFLOPS, 6),
                 "flops_per_launch": alg_flops},
        "algorithmic_bytes_per_launch": alg_bytes,
    }

    if not args.no_extras:
        line["cold_cache_ms"] = round(time_cold(step, 5), 5)
        if args.config == "cfg2":
            ms64 = time_steps(lambda: step(64), max(5, args.steps // 2), 3)
            line["c64"] = {"ms_per_step": round(ms64, 5),
                           "tokens_per_s": round(B * T / (ms64 / 1e3), 1)}
        torch.cuda.reset_peak_memory_stats()
        base = torch.cuda.memory_allocated()
        step()
        torch.cuda.synchronize()
        line["peak_hbm_delta_bytes"] = torch.cuda.max_memory_allocated() - base
        line["prep"] = time_prep(pkg, B, T, H, K, dtype, max(5, args.steps // 2), 5)
        line["bwd"] = time_bwd(pkg, q, k, v, g, beta, h0, 5, 1)

    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(B, T, H, K, V, dtype, C)
        if args.config == "cfg2":
            # configs[2] times both chunk sizes; the reference's own default is
            # C = 64 (gdn_ref.py:48)
            line["cpu_baseline"]["c64"] = cpu_baseline(B, T, H, K, V, dtype, 64)

    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
