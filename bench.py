#!/usr/bin/env python3
"""GDN-2 chunked linear attention on one MI355X -- the headline benchmark.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Workload (the metric's shape): B=8, T=8192, H=6,
D=128, bfloat16 q,k,v,w,b, float32 g, float32 state/accumulators, chunk 128.
A step is one ``gdn2_pallas_forward`` call on resident synthetic inputs;
``value`` is forward tokens/s (B*T per step).  The same line carries the
training-path figure (configs[3]: float32, forward + backward) when the
backward library entry point is available, per-kernel HIP-event times, the
roofline of the dominant kernel and a CPU baseline (the numpy restatement of
the reference's chunked algorithm, timed on a bounded sample of the same
shape on this host).

Inputs are synthetic with the BASELINE.json distributions (torch generator,
seed 0): q,k ~ N(0,1) L2-normalised over D, v ~ N(0,1), w,b = sigmoid(N(0,1)),
g = -softplus(N(0,1)).

HBM traffic of the kernels (``roofline.traffic``) comes from two rocprofv3
counter runs over ``--pmc-run`` (forward steps plus a plain 1 GiB copy kernel
that calibrates the counters), reduced on any host by ``--traffic-from``:

    rocprofv3 --pmc FETCH_SIZE --output-format csv -d <F> -- python bench.py --pmc-run
    rocprofv3 --pmc WRITE_SIZE --output-format csv -d <W> -- python bench.py --pmc-run
    python bench.py --traffic-from <F> <W>      # writes profiles/traffic_*.json

The float32 training step's traffic (``train.roofline.traffic``) the same way
over ``--pmc-train-run``, reduced by ``--train-traffic-from <F> <W>``.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "gdn2-jax-kernel_amd"))
sys.path.insert(0, str(ROOT))

B, T, H, D = 8, 8192, 6, 128
CHUNK = 128
HBM_PEAK = 8.0e12            # MI355X HBM3E, bytes/s
MFMA_PEAK = {"bf16": 2.5e15, "f32": 157.3e12}


def make_inputs(dtype, seed=0, g_scale=1.0):
    import torch
    gen = torch.Generator(device="cuda").manual_seed(seed)
    shape = (B, T, H, D)
    r = lambda: torch.randn(shape, generator=gen, device="cuda", dtype=torch.float32)
    q, k, v, w, b, g = r(), r(), r(), r(), r(), r()
    q = q / q.norm(dim=-1, keepdim=True)
    k = k / k.norm(dim=-1, keepdim=True)
    w, b = torch.sigmoid(w), torch.sigmoid(b)
    g = -torch.nn.functional.softplus(g) * g_scale
    return [x.to(dtype) for x in (q, k, v, w, b)] + [g]


def kernel_table(dtype_bytes, chunk):
    """Algorithmic HBM bytes and flops per token-head for each kernel.

    bytes: what the kernel must read and write given the layout (inputs read
    once, each workspace tensor written once and read once); flops: the
    chunked algorithm's MACs x2 with triangular products at half.
    """
    s, C = dtype_bytes, chunk
    nb = C // 16
    aqk = C * s * (nb + 1) / (2 * nb)      # Aqk: only blocks on or below the diagonal
    return {
        "fwd_prep": {"bytes": 5 * D * s + D * 4 + 4 * D * s + aqk + 4 * D / C,
                     "flops": 4 * C * D + C * C / 3},
        "fwd_state": {"bytes": 3 * D * s + 4 * D / C + D * D * s / C + D * s,
                      "flops": 4 * D * D},
        "fwd_out": {"bytes": 2 * D * s + aqk + D * D * s / C + D * 4,
                    "flops": 2 * D * D + C * D},
        # the scan with the outputs formed in it (inference): reads W, u^T, kg^T,
        # g_last, q_g and Aqk, writes out
        "fwd_state_out": {"bytes": 4 * D * s + 4 * D / C + aqk + D * 4,
                          "flops": 6 * D * D + C * D},
    }


# Inference forwards whose state scan forms the outputs itself (no fwd_out
# launch): bfloat16 at D = 128 (chunk 64 or 128) and D = 256 (chunk 64), float32
# at D = 64 -- the scan variants whose LDS holds the staged h / v_new tiles
# (state_out_waves_of in gdn2_layout.h).  Their third launch interval is empty.
def fused_out(dtype_bytes, d):
    return (dtype_bytes == 2 and d >= 128) or (dtype_bytes == 4 and d == 64)


def name_kernels(kms, fused):
    """Launch intervals (prep, state, out) of one forward, named."""
    if fused:
        return {"fwd_prep": kms[0], "fwd_state_out": kms[1]}
    return dict(zip(("fwd_prep", "fwd_state", "fwd_out"), kms))


# Compulsory HBM bytes per token-head of the bf16 forward: q,k,v,w,b bf16 and g
# fp32 read once, out fp32 written once (h_final adds 4*D*D per (b,h), under
# 0.1 % here).  Algorithmic flops per token-head at chunk C.
def compulsory_fwd_bytes():
    return 5 * 2 * D + 4 * D + 4 * D + 4 * D * D / T


def fwd_flops(C):
    return 5 * C * D + 6 * D * D + C * C / 3


def roofline(per, ms):
    """The headline roofline on compulsory bytes: the forward must move
    compulsory_fwd_bytes() per token-head (906 MB at B8 T8192 H6 D128) and is
    HBM-bound (about 80 flop/B against a bf16 ridge of about 315).  `achieved`
    divides those bytes by the dominant kernel's event time; `end_to_end` by
    the whole forward's time (the lower bound 906 MB / 8 TB/s over ms_per_step).
    `kernel_io` keeps the dominant kernel's own algorithmic traffic (its inputs
    and workspace tiles), and `traffic` the counter-measured bytes per launch."""
    th = B * T * H
    comp = compulsory_fwd_bytes() * th
    dom = max(per, key=per.get)
    ksec = per[dom] * 1e-3
    roof = {"bound": "hbm", "achieved": comp / ksec / 1e9, "peak": HBM_PEAK / 1e9,
            "unit": "GB/s", "kernel": dom, "compulsory_bytes": comp}
    roof["frac"] = roof["achieved"] / roof["peak"]
    roof["end_to_end"] = {"lower_bound_ms": comp / HBM_PEAK * 1e3,
                          "frac": comp / HBM_PEAK / (ms * 1e-3)}
    tab = kernel_table(2, CHUNK)
    if dom in tab:
        kb = tab[dom]["bytes"] * th
        roof["kernel_io"] = {"bytes": kb, "GB/s": kb / ksec / 1e9, "frac": kb / ksec / HBM_PEAK}
    roof["traffic"] = None
    pmc = ROOT / "profiles" / f"traffic_{dom}_b8t8192h6d128_bf16.json"
    if pmc.exists():
        roof["traffic"] = json.loads(pmc.read_text()).get("bytes_per_launch")
    return roof


TRAIN_TRAFFIC = ROOT / "profiles" / "traffic_train_b8t8192h6d128_fp32.json"


def train_roofline(tms):
    """configs[3] (float32 fwd+bwd): algorithmic flops per token-head (forward
    5CD + 6D^2 + C^2/3, backward twice that) on the float32 MFMA peak, against
    compulsory bytes (80 D per token-head) on HBM; the larger time is the bound.
    `frac` is the published bound's (C = 128: 219 GFLOP -> 1.392 ms) over the
    step; `executed` the same at the chunk this path runs (C = 64: 166 GFLOP),
    and `achieved_tflops` is that executed algorithmic work per second.
    `traffic` is the counter-measured HBM bytes of one step (the sum over its
    seven launches, profiles/traffic_train_*.json) and `hbm_floor_ms` the time
    those bytes take at 8 TB/s."""
    th = B * T * H
    nbytes = 80 * D * th

    def at(C):
        flops = 3 * fwd_flops(C) * th
        t_mfma, t_hbm = flops / (FP32_MFMA_PEAK * 1e12), nbytes / HBM_PEAK
        lb = max(t_mfma, t_hbm)
        return {"bound": "mfma" if t_mfma >= t_hbm else "hbm", "flops": flops,
                "lower_bound_ms": lb * 1e3, "frac": lb / (tms * 1e-3)}

    r = at(128)
    exe = at(TRAIN_CHUNK)
    exe["chunk"] = TRAIN_CHUNK
    r.update({"bytes": nbytes, "peak_tflops": FP32_MFMA_PEAK,
              "achieved_tflops": exe["flops"] / (tms * 1e-3) / 1e12, "executed": exe,
              "traffic": None, "hbm_floor_ms": None})
    if TRAIN_TRAFFIC.exists():
        tb = json.loads(TRAIN_TRAFFIC.read_text())["bytes_per_step"]
        r.update({"traffic": tb, "hbm_floor_ms": tb / HBM_PEAK * 1e3})
    return r


def time_forward(gp, xs, steps, warmup, chunk):
    import torch
    from gdn2_package import _lib
    L = _lib.lib()
    scale = D ** -0.5
    for _ in range(warmup):
        gp.gdn2_pallas_forward(*xs, scale, chunk_size=chunk)
    stream = torch.cuda.current_stream()
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(4 * steps)]
    for e in evs:
        e.record(stream)                      # creates the underlying hipEvent_t
    handles = [(ctypes_vp(evs[4 * i + j].cuda_event)) for i in range(steps) for j in range(4)]
    import ctypes
    arrs = [(ctypes.c_void_p * 4)(*handles[4 * i:4 * i + 4]) for i in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        L.gdn2_set_launch_events(arrs[i], 4)
        gp.gdn2_pallas_forward(*xs, scale, chunk_size=chunk)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    iv = [sum(evs[4 * i + j].elapsed_time(evs[4 * i + j + 1]) for i in range(steps)) / steps
          for j in range(3)]
    return (t1 - t0) / steps * 1e3, name_kernels(iv, fused_out(xs[0].element_size(), D))


def ctypes_vp(x):
    import ctypes
    return ctypes.c_void_p(int(x))


def time_train(gp, xs, steps, warmup):
    import torch
    scale = D ** -0.5
    xs = [x.detach().requires_grad_(True) for x in xs]
    gen = torch.Generator(device="cuda").manual_seed(1)
    dout = torch.randn((B, T, H, D), generator=gen, device="cuda")

    def step():
        # gradients returned as jax.grad returns them (no accumulation into .grad)
        out, hf = gp.gdn2_pallas_forward_trainable(*xs, scale)
        torch.autograd.grad([out], xs, [dout])

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps * 1e3


# Algorithmic MFMA flops per chunk of the float32 training kernels (chunk 64,
# D = 128; products counted as the kernels run them):
#   bwd_b2:    dAqk, Aqk^T do (2 BT BT D each, only the 10 of 16 16x16 blocks on or
#              below the diagonal), qg^T do (2 D D BT)
#   bwd_state: kg dh and W^T dv_new per chunk (2 BT D D each)
#   bwd_wy:    three (BT, D, D) in full; dA (two (BT, BT, D)) and A^T dW, A^T dv_new
#              (two (BT, D, BT)) on the 10 of 16 16x16 blocks A's triangle and the
#              strict mask leave; dA A^T and A^T (dA A^T) (two (BT, BT, BT)) on 30 and
#              20 of 64 block products
TRAIN_CHUNK = 64
_C = TRAIN_CHUNK
_NB = _C // 16
_TRI = _NB * (_NB + 1) // 2                       # blocks on or below the diagonal
_SQ = _NB * (_NB + 1) * (2 * _NB + 1) // 6        # dA A^T: sum over row blocks of (I+1)^2
TRAIN_FLOPS = {
    "bwd_b2": 2 * 2 * _C * _C * D * (_C // 16 + 1) // (2 * (_C // 16)) + 2 * D * D * _C,
    "bwd_state": 2 * 2 * _C * D * D,
    "bwd_wy": 3 * 2 * _C * D * D + 2 * (2 * 2 * _C * _C * D) * _TRI // (_NB * _NB)
              + 2 * _C ** 3 * (_SQ + ((_NB + 1) * _TRI - _SQ)) // _NB ** 3,
}
FP32_MFMA_PEAK = 157.3   # TFLOP/s, MI355X dense float32 matrix


def train_kernels(gp, xs):
    """Per-kernel times (HIP events at the library's launch marks) of one
    float32 training step: the forward with residuals, then the backward."""
    import ctypes
    import torch
    from gdn2_package import _lib
    from gdn2_package.gdn2_fwd import _Prepared, _run_forward
    from gdn2_package.gdn2_pipeline import _run_backward
    L = _lib.lib()
    p = _Prepared(*xs, D ** -0.5, None, TRAIN_CHUNK)
    dout = torch.randn((B, T, H, D), device="cuda")
    res = {}
    for names, run in ((("fwd_prep", "fwd_state", "fwd_out"),
                        lambda: _run_forward(p, flags=_lib.FWD_SAVE_A)),
                       (("bwd_b2", "bwd_state", "bwd_wy", "gram_bwd"), None)):
        n = len(names) + 1
        for _ in range(2):            # second pass timed
            evs = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
            for e in evs:
                e.record()
            arr = (ctypes.c_void_p * n)(*[ctypes.c_void_p(int(e.cuda_event)) for e in evs])
            torch.cuda.synchronize()
            if run is not None:
                L.gdn2_set_launch_events(arr, n)
                _, _, ws, _ = run()
            else:
                L.gdn2_set_launch_events(arr, n)
                _run_backward(p, ws, dout, None)
            torch.cuda.synchronize()
        res.update({nm: evs[i].elapsed_time(evs[i + 1]) for i, nm in enumerate(names)})
    nc = B * H * (T // TRAIN_CHUNK)
    mfma = {k: {"tflops": f * nc / (res[k] * 1e-3) / 1e12,
                "frac_of_fp32_peak": f * nc / (res[k] * 1e-3) / 1e12 / FP32_MFMA_PEAK}
            for k, f in TRAIN_FLOPS.items()}
    return res, mfma


def pmc_train_run():
    """Float32 training steps (train_kernels: the forward with residuals and the
    backward, each twice), one headline forward and, last, the calibration copy
    of --pmc-run: for the MFMA counters (--mfma-from) and the training step's
    HBM traffic (FETCH_SIZE / WRITE_SIZE runs, --train-traffic-from)."""
    import torch
    import gdn2_package as gp
    xs = make_inputs(torch.float32)
    train_kernels(gp, xs)
    del xs
    xb = make_inputs(torch.bfloat16)
    gp.gdn2_pallas_forward(*xb, D ** -0.5, chunk_size=CHUNK)
    del xb
    src = torch.ones(COPY_BYTES // 4, device="cuda")
    dst = torch.empty_like(src)
    torch.abs(src, out=dst)             # one elementwise kernel: reads and writes 1 GiB
    torch.cuda.synchronize()
    print(json.dumps({"pmc_train_run": 1, "copy_bytes": COPY_BYTES}), flush=True)


TRAIN_KERNELS = ("fwd_prep", "fwd_state", "fwd_out", "bwd_b2", "bwd_state", "bwd_wy",
                 "gram_bwd")


def train_traffic_from(fetch_dir, write_dir):
    """Copy-calibrated HBM bytes of each float32 training kernel (chunk 64) from
    the FETCH_SIZE and WRITE_SIZE runs of --pmc-train-run, their sum per step
    against the step's algorithmic bytes, written to profiles/traffic_train_*."""
    fetch, f_copy = _counter_means(fetch_dir, "FETCH_SIZE")
    write, w_copy = _counter_means(write_dir, "WRITE_SIZE")
    f_scale = COPY_BYTES / (f_copy * 1024)
    w_scale = COPY_BYTES / (w_copy * 1024)
    bf16 = lambda n: "DF16b" in n or "__bf16" in n or "bfloat16" in n
    rows = {}
    for k in TRAIN_KERNELS:
        names = [n for n in fetch if k in n and "gdn2" in n and not bf16(n)
                 and not (k == "fwd_state" and "seg_" in n)]
        if len(names) != 1:
            raise SystemExit(f"{k}: expected one float32 kernel, found {names}")
        n = names[0]
        rows[k] = {"fetch_bytes": fetch[n] * 1024 * f_scale,
                   "write_bytes": write[n] * 1024 * w_scale}
        rows[k]["bytes"] = rows[k]["fetch_bytes"] + rows[k]["write_bytes"]
    total = sum(r["bytes"] for r in rows.values())
    rec = {"workload": "B8 T8192 H6 D128 float32 training step (forward with residuals + "
                       f"backward), chunk {TRAIN_CHUNK}",
           "kernels": rows, "bytes_per_step": total,
           "compulsory_bytes": 80 * D * B * T * H,
           "fetch_scale": f_scale, "write_scale": w_scale,
           "calibration": f"copy kernel reading and writing {COPY_BYTES} bytes"}
    TRAIN_TRAFFIC.write_text(json.dumps(rec, indent=1) + "\n")
    print(json.dumps(rec, indent=1))


def mfma_from(run_dir):
    """Per-kernel MFMA flops (SQ_INSTS_VALU_MFMA_MOPS_* x 512) and utilisation
    (SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE x SIMDs)) of a --pmc-train-run
    counter run; durations from the same run's dispatch timestamps."""
    import csv
    files = sorted(Path(run_dir).rglob("*counter_collection.csv"))
    if len(files) != 1:
        raise SystemExit(f"expected one counter file under {run_dir}, found {len(files)}")
    per = {}
    with open(files[0], newline="") as fh:
        for row in csv.DictReader(fh):
            key = (int(row["Dispatch_Id"]), row["Kernel_Name"])
            d = per.setdefault(key, {"ns": int(row["End_Timestamp"]) - int(row["Start_Timestamp"])})
            d[row["Counter_Name"]] = d.get(row["Counter_Name"], 0.0) + float(row["Counter_Value"])
    # GRBM_GUI_ACTIVE arrives summed over the 8 XCDs: per-XCD active cycles are
    # a eighth of it (rocprof's MfmaUtil takes the maximum over instances)
    simds, xcds = 256 * 4, 8
    out = {}
    for (_, name), d in sorted(per.items()):
        if "gdn2" not in name:
            continue
        short = next((k for k in ("fwd_prep", "fwd_state", "fwd_out", "bwd_b2", "bwd_state",
                                  "bwd_wy", "gram_bwd") if k in name), name)
        dt = "bf16" if ("DF16b" in name or "__bf16" in name or "bool" in name) else "fp32"
        f32 = 512 * d.get("SQ_INSTS_VALU_MFMA_MOPS_F32", 0)
        b16 = 512 * d.get("SQ_INSTS_VALU_MFMA_MOPS_BF16", 0)
        # float32 kernels: products in the split form run three bfloat16 MFMAs per
        # float32 product, so their bfloat16 flops count a third as float32 work
        flops = f32 + b16 / 3 if dt == "fp32" else f32 + b16
        peak = FP32_MFMA_PEAK if dt == "fp32" else 2516.6
        out[f"{short} ({dt})"] = {
            "mfma_flops": flops, "f32_mfma_flops": f32, "bf16_mfma_flops": b16, "ns": d["ns"],
            "tflops": flops / d["ns"] / 1e3, "frac_of_peak": flops / d["ns"] / 1e3 / peak,
            "mfma_busy": d.get("SQ_VALU_MFMA_BUSY_CYCLES", 0)
            / max(1.0, d.get("GRBM_GUI_ACTIVE", 0) / xcds * simds)}
    print(json.dumps(out, indent=1))
    return out


SQ_PASSES = (
    ("SQ_WAVES", "SQ_WAVE_CYCLES", "SQ_BUSY_CYCLES", "SQ_WAIT_ANY", "SQ_WAIT_INST_ANY",
     "SQ_ACTIVE_INST_ANY", "SQ_ACTIVE_INST_VALU", "SQ_WAIT_INST_LDS"),
    ("SQ_WAVES", "SQ_INSTS_VALU", "SQ_INSTS_LDS", "SQ_INSTS_MFMA", "SQ_INSTS_VMEM_RD",
     "SQ_INSTS_VMEM_WR", "SQ_LDS_BANK_CONFLICT", "SQ_ACTIVE_INST_LDS"),
)


def sq_from(run_dirs):
    """Where each kernel's waves spend their cycles, from --pmc-train-run counter
    runs of the SQ_PASSES groups (one rocprofv3 run per group): the wave-cycle
    counters SQ_WAIT_ANY (waiting on anything: a memory counter, a barrier, a
    dependency), SQ_WAIT_INST_ANY (an issued instruction waiting for its
    operands or a free unit), SQ_ACTIVE_INST_ANY / _VALU / _LDS (issuing) as
    fractions of SQ_WAVE_CYCLES, and instructions per wave.  The last dispatch
    of each kernel in the run is the one reported."""
    import csv
    per = {}
    for run_dir in run_dirs:
        files = sorted(Path(run_dir).rglob("*counter_collection.csv"))
        if len(files) != 1:
            raise SystemExit(f"expected one counter file under {run_dir}, found {len(files)}")
        with open(files[0], newline="") as fh:
            rows = [r for r in csv.DictReader(fh) if "gdn2" in r["Kernel_Name"]]

        def key_of(name):
            short = next((k for k in TRAIN_KERNELS if k in name), name)
            return f"{short} ({'bf16' if ('DF16b' in name or '__bf16' in name) else 'fp32'})"
        last = {}
        for r in rows:
            k = key_of(r["Kernel_Name"])
            last[k] = max(last.get(k, -1), int(r["Dispatch_Id"]))
        run = {}
        for r in rows:
            k = key_of(r["Kernel_Name"])
            if int(r["Dispatch_Id"]) == last[k]:
                d = run.setdefault(k, {})
                d[r["Counter_Name"]] = d.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
        for k, d in run.items():
            merged = per.setdefault(k, {})
            for c, v in d.items():
                merged.setdefault(c, v)
    out = {}
    for key, d in per.items():
        wc = max(d.get("SQ_WAVE_CYCLES", 0.0), 1.0)
        waves = max(d.get("SQ_WAVES", 0.0), 1.0)
        out[key] = {
            "wait_any": d.get("SQ_WAIT_ANY", 0.0) / wc,
            "wait_inst_any": d.get("SQ_WAIT_INST_ANY", 0.0) / wc,
            "active_any": d.get("SQ_ACTIVE_INST_ANY", 0.0) / wc,
            "active_valu": d.get("SQ_ACTIVE_INST_VALU", 0.0) / wc,
            "active_lds": d.get("SQ_ACTIVE_INST_LDS", 0.0) / wc,
            "wait_inst_lds": d.get("SQ_WAIT_INST_LDS", 0.0) / wc,
            "valu_per_wave": d.get("SQ_INSTS_VALU", 0.0) / waves,
            "lds_per_wave": d.get("SQ_INSTS_LDS", 0.0) / waves,
            "mfma_per_wave": d.get("SQ_INSTS_MFMA", 0.0) / waves,
            "vmem_rd_per_wave": d.get("SQ_INSTS_VMEM_RD", 0.0) / waves,
            "vmem_wr_per_wave": d.get("SQ_INSTS_VMEM_WR", 0.0) / waves,
            "lds_bank_conflict_per_wave": d.get("SQ_LDS_BANK_CONFLICT", 0.0) / waves,
            "waves": d.get("SQ_WAVES", 0.0)}
    print(json.dumps(out, indent=1))
    return out


def _time(fn, steps, warmup):
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps * 1e3


def _event_ms(fn, nmarks):
    """Run fn once with HIP events recorded at the library's launch marks
    (gdn2_set_launch_events) and return the nmarks-1 intervals in ms."""
    import ctypes
    import torch
    from gdn2_package import _lib
    L = _lib.lib()
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(nmarks)]
    for e in evs:
        e.record()
    arr = (ctypes.c_void_p * nmarks)(*[ctypes.c_void_p(int(e.cuda_event)) for e in evs])
    torch.cuda.synchronize()
    L.gdn2_set_launch_events(arr, nmarks)
    fn()
    torch.cuda.synchronize()
    return [evs[i].elapsed_time(evs[i + 1]) for i in range(nmarks - 1)]


def extras(gp, steps=10, warmup=3):
    """The paths beyond the headline, each timed on the GPU in the same run:
    configs[4] (1 x 131072 x 8 heads, segmented state scan), the forward with
    the input activations fused (vs torch activations + forward), a
    variable-length batch with the headline's token count, D = 256, the bfloat16
    training step, a partial last chunk, and the decode step (state read +
    written per token)."""
    import torch
    f = torch.nn.functional
    res = {}
    gen = torch.Generator(device="cuda").manual_seed(5)
    # configs[4]
    B5, T5, H5 = 1, 131072, 8
    r = lambda shape: torch.randn(shape, generator=gen, device="cuda")
    q, k, v, w, b, g = (r((B5, T5, H5, D)) for _ in range(6))
    q, k = f.normalize(q, dim=-1), f.normalize(k, dim=-1)
    w, b, g = torch.sigmoid(w), torch.sigmoid(b), -f.softplus(g) * 0.1
    xs = [x.to(torch.bfloat16) for x in (q, k, v, w, b)] + [g]
    ms = _time(lambda: gp.gdn2_pallas_forward(*xs, D ** -0.5, chunk_size=CHUNK), steps, warmup)
    kms = _event_ms(lambda: gp.gdn2_pallas_forward(*xs, D ** -0.5, chunk_size=CHUNK), 4)
    res["config5_fwd"] = {"shape": "B1 T131072 H8 D128 bf16, chunk 128 (state scan in 8 "
                                   "segments)", "ms": ms, "tokens_per_s": B5 * T5 / (ms * 1e-3),
                          "kernels_ms": name_kernels(kms, fused_out(2, D))}
    # the same at the library's default chunk for bf16 D = 128 (64)
    ms = _time(lambda: gp.gdn2_pallas_forward(*xs, D ** -0.5, chunk_size=64), steps, warmup)
    kms = _event_ms(lambda: gp.gdn2_pallas_forward(*xs, D ** -0.5, chunk_size=64), 4)
    res["config5_fwd_chunk64"] = {"shape": "B1 T131072 H8 D128 bf16, chunk 64 (state scan in "
                                           "8 segments)", "ms": ms,
                                  "tokens_per_s": B5 * T5 / (ms * 1e-3),
                                  "kernels_ms": name_kernels(kms, fused_out(2, D))}
    del q, k, v, w, b, g, xs
    # fused input preparation at the headline shape
    raw = [r((B, T, H, D)).to(torch.bfloat16) for _ in range(5)] + [r((B, T, H, D))]
    ms_raw = _time(lambda: gp.gdn2_pallas_forward_raw(*raw, D ** -0.5), steps, warmup)

    def torch_prep_then_fwd():
        a = [f.normalize(raw[0].float(), dim=-1).to(torch.bfloat16),
             f.normalize(raw[1].float(), dim=-1).to(torch.bfloat16), raw[2],
             torch.sigmoid(raw[3]), torch.sigmoid(raw[4]), -f.softplus(raw[5])]
        return gp.gdn2_pallas_forward(*a, D ** -0.5)
    ms_sep = _time(torch_prep_then_fwd, steps, warmup)
    res["fused_input_prep"] = {"shape": "B8 T8192 H6 D128 bf16", "fused_ms": ms_raw,
                               "torch_activations_plus_forward_ms": ms_sep}
    # variable length: the headline's 65536 tokens as 16 sequences of uneven length
    lens = torch.randint(1, 2 * (B * T) // 16, (16,), generator=torch.Generator().manual_seed(1))
    lens = (lens.float() * (B * T) / lens.sum()).long().clamp(min=1)
    lens[-1] += B * T - lens.sum()
    cu = torch.cat([torch.zeros(1, dtype=torch.long), lens.cumsum(0)])
    packed = [x.reshape(1, B * T, H, D) for x in raw]
    ms_v = _time(lambda: gp.gdn2_pallas_forward_varlen(*packed, D ** -0.5, cu, raw=True),
                 steps, warmup)
    kms = _event_ms(lambda: gp.gdn2_pallas_forward_varlen(*packed, D ** -0.5, cu, raw=True), 4)
    res["varlen_fwd"] = {"shape": f"1 x {B * T} tokens in 16 sequences ({int(lens.min())}.."
                                  f"{int(lens.max())} tokens), H6 D128 bf16, fused activations",
                         "ms": ms_v, "tokens_per_s": B * T / (ms_v * 1e-3),
                         "kernels_ms": name_kernels(kms, fused_out(2, D)),
                         "note": "ms includes building the chunk tables on the host"}
    del raw, packed
    def dist(shape):   # the headline's input distributions at another shape
        q, k, v, w, b_, g = (r(shape) for _ in range(6))
        return [x.to(torch.bfloat16) for x in (f.normalize(q, dim=-1), f.normalize(k, dim=-1), v,
                                               torch.sigmoid(w), torch.sigmoid(b_))] + \
            [-f.softplus(g)]
    # D = 256 (chunk 64): the headline's B, T and element count with H = 3
    x256 = dist((B, T, 3, 256))
    ms = _time(lambda: gp.gdn2_pallas_forward(*x256, 256 ** -0.5), steps, warmup)
    kms = _event_ms(lambda: gp.gdn2_pallas_forward(*x256, 256 ** -0.5), 4)
    res["d256_fwd"] = {"shape": "B8 T8192 H3 D256 bf16, chunk 64", "ms": ms,
                       "tokens_per_s": B * T / (ms * 1e-3),
                       "kernels_ms": name_kernels(kms, fused_out(2, 256))}
    # D = 256 training step, float32 (chunk 64): forward with residuals + backward
    x256f = [x.float().detach().requires_grad_(True) for x in x256]
    do256 = r((B, T, 3, 256))
    ms = _time(lambda: torch.autograd.grad(
        [gp.gdn2_pallas_forward_trainable(*x256f, 256 ** -0.5)[0]], x256f, [do256]), 3, 1)
    res["d256_train"] = {"shape": "B8 T8192 H3 D256 float32, forward + backward", "ms": ms,
                         "tokens_per_s": B * T / (ms * 1e-3)}
    del x256, x256f, do256
    # bfloat16 training step at the headline shape: float32 arithmetic and residuals
    # on the bfloat16 inputs as they are (GDN2_BF16_F32), as the reference upcasts;
    # gradients in the input dtypes
    xb = [x.detach().requires_grad_(True) for x in dist((B, T, H, D))]
    dob = r((B, T, H, D))
    ms = _time(lambda: torch.autograd.grad(
        [gp.gdn2_pallas_forward_trainable(*xb, D ** -0.5)[0]], xb, [dob]), 5, 2)
    res["bf16_train"] = {"shape": "B8 T8192 H6 D128 bf16 inputs (fp32 g), forward + backward "
                                  "in float32 arithmetic on the bf16 data, bf16 gradients",
                         "ms": ms, "tokens_per_s": B * T / (ms * 1e-3)}
    del xb, dob
    # T % BT != 0: 8100 tokens per sequence, the last chunk of each 36 tokens short
    xp = dist((B, 8100, H, D))
    ms = _time(lambda: gp.gdn2_pallas_forward(*xp, D ** -0.5, chunk_size=128), steps, warmup)
    res["partial_chunk_fwd"] = {"shape": "B8 T8100 H6 D128 bf16, chunk 128 (last chunk 36 "
                                         "tokens)", "ms": ms, "tokens_per_s": B * 8100 / (ms * 1e-3)}
    del xp
    # decode: one token for B*H = 48 states of 128 x 128 fp32
    tok = [r((B, 1, H, D)).to(torch.bfloat16) for _ in range(5)] + [-f.softplus(r((B, 1, H, D)))]
    state = torch.zeros((B, H, D, D), device="cuda")
    ms_d = _time(lambda: gp.gdn2_decode_step(*tok, D ** -0.5, state=state, inplace=True),
                 100, 10)
    # the same step captured in a HIP graph (static token buffers, state updated in
    # place): one step per replay, and 16 steps per replay (time per token)
    st_g = torch.zeros_like(state)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        gp.gdn2_decode_step(*tok, D ** -0.5, state=st_g, inplace=True)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g1, g16 = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
    with torch.cuda.graph(g1):
        gp.gdn2_decode_step(*tok, D ** -0.5, state=st_g, inplace=True)
    with torch.cuda.graph(g16):
        for _ in range(16):
            gp.gdn2_decode_step(*tok, D ** -0.5, state=st_g, inplace=True)
    us_g1 = _time(g1.replay, 200, 20) * 1e3
    us_g16 = _time(g16.replay, 50, 5) * 1e3 / 16
    res["decode_step"] = {"shape": "B8 H6 D128, one token", "call_us": ms_d * 1e3,
                          "graph_replay_us": us_g1, "graph_16_steps_us_per_token": us_g16,
                          "note": "call_us per eager call, Python wrapper and launch included "
                                  "(host-bound); graph_*: the step captured in a HIP graph, "
                                  "one or 16 steps per replay; the kernel (decode_step, 6.3 MB "
                                  "of fp32 state read and written) is timed by rocprofv3 in "
                                  "profiles/"}
    del g1, g16
    return res


def _cpu_model():
    """The host CPU's model name (lscpu's "Model name", read from /proc/cpuinfo)."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(min_seconds=10.0, bwd_tokens=1024, bwd_min_seconds=8.0):
    """The numpy restatement of the reference's chunked algorithm on this host:
    the forward (kernels A-D with the 3-D decay tensor, float32) on one batch
    element of the headline workload (B=1, T, H, D as above), repeated until
    `min_seconds` have passed; and the training step of configs[3] (float32
    forward recompute + B1-B5, oracle.chunked_bwd, chunk 64) on a bounded
    prefix of one batch element (`bwd_tokens` tokens of the 8192, all 6 heads),
    scaled linearly -- the work is linear in T."""
    import numpy as np
    from oracle import gdn2_oracle as O
    try:
        from threadpoolctl import threadpool_info
        cores = max(i.get("num_threads", 1) for i in threadpool_info()) or 1
    except Exception:
        cores = os.cpu_count() or 1
    xs = O.make_inputs(1, T, H, D, seed=0)
    runs, t0 = 0, time.perf_counter()
    while True:
        O.chunked_fwd(*xs, D ** -0.5, BT=CHUNK, clip=True, dtype=np.float32)
        runs += 1
        dt = time.perf_counter() - t0
        if dt >= min_seconds:
            break
    xb = [x[:, :bwd_tokens] for x in xs]
    do = np.random.default_rng(1).standard_normal(xb[0].shape).astype(np.float32)
    bruns, t1 = 0, time.perf_counter()
    while True:
        O.chunked_bwd(*xb, D ** -0.5, do, BT=TRAIN_CHUNK, clip=True, dtype=np.float32)
        bruns += 1
        bdt = time.perf_counter() - t1
        if bdt >= bwd_min_seconds:
            break
    btps = bruns * bwd_tokens / bdt
    return {"value": runs * T / dt, "unit": "tokens/s", "cores": int(cores), "kind": "port",
            "cpu": _cpu_model(), "os_cpu_count": os.cpu_count(),
            "sample": f"{runs} x forward of one batch element (B=1 T={T} H={H} D={D} "
                      f"BT={CHUNK}, float32) of the headline workload, numpy restatement of "
                      f"gdn2_fwd.py kernels A-D (oracle.chunked_fwd), {dt:.1f} s; "
                      f"tokens/s comparable to value (same T, H, D)",
            "fwd_bwd": {"value": btps, "unit": "tokens/s",
                        "ms_per_step_scaled": B * T / btps * 1e3,
                        "sample": f"{bruns} x forward + backward (oracle.chunked_bwd: recompute, "
                                  f"B2, B1, B3, B4, B5; float32, chunk {TRAIN_CHUNK}) of "
                                  f"B=1 T={bwd_tokens} H={H} D={D}, the first {bwd_tokens} "
                                  f"tokens of one batch element of configs[3], {bdt:.1f} s; "
                                  f"tokens/s comparable to train.tokens_per_s"}}


COPY_BYTES = 1 << 30           # calibration copy: reads and writes this many bytes
# the headline's launches (its scan forms the outputs): name matched in the
# kernel symbol -> row of kernel_table
KERNELS = {"fwd_prep": "fwd_prep", "fwd_state": "fwd_state_out"}


def pmc_run(steps, chunk=CHUNK):
    """Forward steps plus one plain copy kernel of COPY_BYTES, for counter runs."""
    import torch
    import gdn2_package as gp
    xs = make_inputs(torch.bfloat16)
    for _ in range(steps):
        gp.gdn2_pallas_forward(*xs, D ** -0.5, chunk_size=chunk)
    src = torch.ones(COPY_BYTES // 4, device="cuda")
    dst = torch.empty_like(src)
    torch.abs(src, out=dst)             # one elementwise kernel: reads and writes 1 GiB
    torch.cuda.synchronize()
    print(json.dumps({"pmc_run": steps, "copy_bytes": COPY_BYTES}), flush=True)


def _counter_means(run_dir, counter):
    """Per-dispatch values of `counter` in a rocprofv3 csv counter-collection
    output directory: (mean per kernel name, value of the last dispatch)."""
    import csv
    files = sorted(Path(run_dir).rglob("*counter_collection.csv"))
    if not files:
        raise SystemExit(f"no *counter_collection.csv under {run_dir}")
    if len(files) > 1:   # dispatch ids restart per run: two runs would be summed
        raise SystemExit(f"{len(files)} counter files under {run_dir}: give each run "
                         f"its own output directory")
    per = {}
    for f in files:
        with open(f, newline="") as fh:
            for row in csv.DictReader(fh):
                if row.get("Counter_Name") != counter:
                    continue
                key = (int(row.get("Dispatch_Id", 0)), row.get("Kernel_Name", ""))
                per[key] = per.get(key, 0.0) + float(row["Counter_Value"])
    by_kernel = {}
    for (_, name), v in per.items():
        by_kernel.setdefault(name, []).append(v)
    last = per[max(per)]
    return {name: sum(v) / len(v) for name, v in by_kernel.items()}, last


def traffic_from(fetch_dir, write_dir, chunk=CHUNK):
    """Copy-calibrated HBM bytes per launch of each forward kernel from the
    FETCH_SIZE and WRITE_SIZE runs (counters in KiB per dispatch).  The
    calibration copy is the last dispatch of a --pmc-run (at the same chunk)."""
    fetch, f_copy = _counter_means(fetch_dir, "FETCH_SIZE")
    write, w_copy = _counter_means(write_dir, "WRITE_SIZE")
    f_scale = COPY_BYTES / (f_copy * 1024)
    w_scale = COPY_BYTES / (w_copy * 1024)
    tab = kernel_table(2, chunk)
    pick = lambda t, k: next(v for n, v in t.items() if k in n)
    sfx = "" if chunk == CHUNK else f"_c{chunk}"   # the headline's files carry no suffix
    out = {}
    for k, row in KERNELS.items():
        fb = pick(fetch, k) * 1024 * f_scale
        wb = pick(write, k) * 1024 * w_scale
        rec = {"kernel": row, "workload": f"B8 T8192 H6 D128 bf16 chunk {chunk}",
               "fetch_bytes": fb, "write_bytes": wb, "bytes_per_launch": fb + wb,
               "algorithmic_bytes": tab[row]["bytes"] * B * T * H,
               "fetch_scale": f_scale, "write_scale": w_scale,
               "calibration": f"copy kernel reading and writing {COPY_BYTES} bytes"}
        (ROOT / "profiles" / f"traffic_{row}_b8t8192h6d128_bf16{sfx}.json").write_text(
            json.dumps(rec, indent=1) + "\n")
        out[k] = rec
    print(json.dumps(out, indent=1))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-train", action="store_true")
    ap.add_argument("--no-extras", action="store_true",
                    help="skip configs[4], fused input prep, varlen and decode timings")
    ap.add_argument("--pmc-run", action="store_true",
                    help="forward steps plus the calibration copy, for rocprofv3 --pmc")
    ap.add_argument("--traffic-from", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="reduce two rocprofv3 counter runs to profiles/traffic_*.json")
    ap.add_argument("--chunk", type=int, default=CHUNK,
                    help="chunk size of --pmc-run / --traffic-from (default: the headline's)")
    ap.add_argument("--pmc-train-run", action="store_true",
                    help="one float32 training step and one headline forward, for MFMA counters")
    ap.add_argument("--mfma-from", metavar="DIR",
                    help="reduce a --pmc-train-run MFMA counter run (per-kernel flops, utilisation)")
    ap.add_argument("--train-traffic-from", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="reduce two --pmc-train-run counter runs to profiles/traffic_train_*")
    ap.add_argument("--sq-from", nargs="+", metavar="DIR",
                    help="reduce --pmc-train-run runs of the SQ_PASSES counter groups "
                         "(wave-cycle shares, instructions per wave)")
    args = ap.parse_args()
    if args.sq_from:
        sq_from(args.sq_from)
        return
    if args.mfma_from:
        mfma_from(args.mfma_from)
        return
    if args.train_traffic_from:
        train_traffic_from(*args.train_traffic_from)
        return
    if args.pmc_train_run:
        pmc_train_run()
        return
    if args.traffic_from:
        traffic_from(*args.traffic_from, chunk=args.chunk)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (the op shards over (batch, head) "
              "pairs with no communication); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    if args.pmc_run:
        pmc_run(max(1, min(args.steps, 5)), chunk=args.chunk)
        return

    import torch
    import gdn2_package as gp

    xs = make_inputs(torch.bfloat16)
    torch.cuda.synchronize()
    ms, per = time_forward(gp, xs, args.steps, args.warmup, CHUNK)
    tokens = B * T
    value = tokens / (ms * 1e-3)

    roof = roofline(per, ms)
    # the same workload at the library's default chunk for bf16 D = 128 (64): not
    # the configuration's BT = 128, reported beside it
    ms64, per64 = time_forward(gp, xs, args.steps, args.warmup, 64)

    del xs
    torch.cuda.empty_cache()
    train, failed = None, None
    if not args.no_train:
        try:
            xs32 = make_inputs(torch.float32)
            # the first steps after the allocation of the gradient and workspace
            # tensors run up to 15 % slower (first touch of fresh memory): warm up as
            # many steps as the forward does
            tms = time_train(gp, xs32, max(1, args.steps // 2), max(1, args.warmup))
            kms, mfma = train_kernels(gp, xs32)
            train = {"config": "B8 T8192 H6 D128 float32, forward + backward (trainable)",
                     "ms_per_step": tms, "tokens_per_s": tokens / (tms * 1e-3),
                     "kernels_ms": kms, "mfma": mfma, "roofline": train_roofline(tms)}
            del xs32
        except Exception as e:   # reported in the line, and the run fails
            failed = f"{type(e).__name__}: {e}"[:300]
            train = {"error": failed}

    line = {
        "metric": "fwd & fwd+bwd ms, tokens/s at B8 T8192 H6 D128; % MFMA/HBM roofline",
        "value": value, "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "gdn2_pallas_forward B8 T8192 H6 D128 bf16 inputs, fp32 g/state, "
                               "chunk 128 (BASELINE configs[2])",
                   "B": B, "T": T, "H": H, "D": D, "chunk": CHUNK},
        "kernels_ms": per,
        "roofline": roof,
        "chunk64": {"ms_per_step": ms64, "tokens_per_s": tokens / (ms64 * 1e-3),
                    "kernels_ms": per64,
                    "roofline_end_to_end_frac": roof["end_to_end"]["lower_bound_ms"] / ms64,
                    "note": "same inputs at chunk 64 (the default chunk for bf16 at D = 128); "
                            "value above is at the configuration's chunk 128"},
        "train": train,
    }
    if not args.no_extras:
        line["extras"] = extras(gp)
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line), flush=True)
    if failed:
        print(f"bench.py: the training step failed: {failed}", file=sys.stderr)
        sys.exit(1)


if __name__ == "__main__":
    main()
