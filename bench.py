"""Benchmark of the INT8 quantized-inference path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-extra] [--no-cpu]
    python bench.py --traffic-probe     (the dominant kernels, for rocprofv3 --pmc counter runs)
    python bench.py --counter-summary DIR   (rocprofv3 CSVs -> profiles/kernel_counters.{json,md})

Headline (`value`): configs[1] of BASELINE.json -- the fused W8A8 linear at M=N=K=4096
(FP16 activations with 8 outlier channels x20, per-token quantize, INT8 MFMA GEMM with
INT32 accumulation, dequant + bias to FP16). One step = one forge_int8_linear call
(quantize kernel + GEMM kernel) on inputs already resident in HBM. value = 2*M*N*K / t.

roofline: the dominant kernel (the GEMM) timed alone with HIP events on the launch stream,
algorithmic ops 2*M*N*K per launch against MI355X's dense INT8 peak (5.0 POP/s).
cpu_baseline: the oracle's INT32 loop + dequant epilogue (oracle/) over the whole configs[1]
workload, split over output rows on up to 16 threads (the box's CPU share per GPU), timed on
this host; the single-threaded rate is in its sample text.
roofline.traffic / roofline.mfma_busy: L2-miss bytes per launch of the GEMM (reads and writes
between the L2s and the memory fabric: HBM plus what the 256 MB MALL serves, so an upper bound
of HBM bytes) and its matrix-core busy fraction, read from COUNTERS_FILE (profiles/kernel_counters.json), which `--counter-summary`
writes from rocprofv3 --pmc runs of `bench.py --traffic-probe` (FETCH_SIZE and WRITE_SIZE scaled
by what the same counters read for a device copy of known size in the same runs; MFMA busy
cycles; see profiles/kernel_counters.md).
extra: configs[2] (2:4 sparse vs dense at 4096x11008x4096), configs[3] (decode
M = 1/4/16, N = K = 8192, dense and 2:4, HBM GB/s with 8 dense / 10 sparse rotating weight
copies so the 256 MB MALL cannot hold them; calls captured into a HIP graph and replayed so host launch
overhead is not timed; the whole int8_linear / sparse_int8_linear, and the GEMM alone on
pre-quantized tokens, *_gemm_*), configs[4] (INT8 NHWC 3x3 conv, INT32 and dequant outputs), and
the rest of the INT8 conv family on NCHW FP16 maps: depthwise 3x3 (1, 64, 540, 960) and
ConvTranspose2d k2s2 (1, 64, 270, 480) -> (1, 32, 540, 960), as time and HBM GB/s of
input + output bytes (rotating over more than 256 MB of inputs and outputs, graph-replayed); the
reference's NCHW FP16 int8_conv2d_forward on a (1, 32, 540, 960) 3x3 layer (one fused launch); and SparseLinear's weight preparation at 11008 x 4096 fp32, one pass
against the reference's separate quantize / prune+compress / pack steps; and
extra.reference_sweep: the reference's own sparse benchmark (bench_int8_sparse.cu shapes and
protocol) with the dense path beside it; extra.vendor_hipblaslt: hipBLASLt (torch._int_mm, INT32
out) next to forge_int8_gemm_s32 at 4096^3 and 8192^3 on the same inputs, checked bit-equal -- a
vendor reference point, not part of the product.
    python bench.py --probes            (the measurement probes of libforge_probes.so, one JSON line)
    python bench.py --probe NAME        (one probe, repeated, for rocprofv3 --pmc runs)
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "INT8 dense/2:4-sparse GEMM TOPS @4096^3 (% MFMA peak); M=16 HBM GB/s"
PEAK_INT8_TOPS = 5000.0      # MI355X dense INT8 MFMA, 5.0 POP/s
PEAK_HBM_GBS = 8000.0        # MI355X HBM3E, 8 TB/s
COPY_PROBE_BYTES = 256 << 20  # calibration copy for the traffic counters
PROBE_REPS = 5


COUNTERS_FILE = os.path.join(ROOT, "profiles", "kernel_counters.json")


def _c2_counters():
    try:
        with open(COUNTERS_FILE) as f:
            return json.load(f)["kernels"]["c2_gemm"]
    except (OSError, ValueError, KeyError, TypeError):
        return {}


def measured_traffic():
    """L2-miss bytes per launch of the configs[1] GEMM (L2 <-> memory fabric, HBM plus MALL
    hits) from the committed counter runs (FETCH_SIZE and WRITE_SIZE, scaled by the counters'
    reading for a device copy of known size), or None."""
    v = _c2_counters().get("traffic_bytes")
    return int(v) if v else None


def measured_mfma_busy():
    """Matrix-core busy fraction of the configs[1] GEMM from the committed counter run
    (SQ_VALU_MFMA_BUSY_CYCLES over 4 x SQ_BUSY_CU_CYCLES), or None."""
    v = _c2_counters().get("mfma_busy")
    return round(float(v), 4) if v is not None else None


def traffic_probe() -> int:
    """Launches for the counter runs (rocprofv3 --pmc, one counter set per run), each kernel
    PROBE_REPS times on its configs' shape with inputs resident on the device:
    c2 = the configs[1] dequant GEMM (4096^3, FP16 out); c3 sparse / dense = configs[2]
    (4096 x 11008 x 4096, INT32 out) on the 2:4 and the dense engine; c5 = configs[4] NHWC
    conv (INT32 out; 256-row and 192-row tiles in one launch); c4 = configs[3] M = 16 decode GEMMs
    (N = K = 8192, pre-quantized tokens, FP16 out) dense and 2:4; f1 = the fused quantize + 2:4
    sparse linear on the reference's example layer (1280 -> 320 at M = 147,456); f2 = the NCHW FP16
    conv API on (1, 32, 540, 960) 3x3 -> 32 (one launch); then a COPY_PROBE_BYTES
    device-to-device copy, the calibration of known size for FETCH_SIZE / WRITE_SIZE."""
    import torch
    import forge_amd
    from forge_amd import ops
    forge_amd.load()
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(9)

    def reps(tag, fn):
        for _ in range(PROBE_REPS):
            fn()
        torch.cuda.synchronize()
        print(f"probe {tag} done", flush=True)

    x, W, ws, b = make_c2(dev)
    M, K = x.shape
    N = W.shape[0]
    sq = torch.empty((M, K), dtype=torch.int8, device=dev)
    ss = torch.empty((M,), dtype=torch.float32, device=dev)
    y = torch.empty((M, N), dtype=torch.float16, device=dev)
    ops.fused_quantize_activation(x, M, K, out=sq, scales=ss)
    reps("c2_gemm", lambda: ops.int8_gemm_dequant(sq, W, ss, ws, b, out=y))
    del x, W, y

    M, K, N = 4096, 4096, 11008
    W = torch.randint(-127, 128, (N, K), generator=g, device=dev, dtype=torch.int8)
    comp, meta = _prep_sparse(ops, W)
    C = torch.empty((M, N), dtype=torch.int32, device=dev)
    reps("c3_sparse", lambda: ops.sparse_int8_gemm_s32(comp, sq, meta, out=C))
    reps("c3_dense", lambda: ops.int8_gemm_s32(sq, W, out=C))
    del W, comp, meta, C

    xc = torch.randint(-127, 128, (32, 56, 56, 256), generator=g, device=dev, dtype=torch.int8)
    wc = torch.randint(-127, 128, (256, 3, 3, 256), generator=g, device=dev, dtype=torch.int8)
    o32 = torch.empty((32, 56, 56, 256), dtype=torch.int32, device=dev)
    reps("c5_conv", lambda: ops.int8_conv2d_nhwc_s32(xc, wc, pad=(1, 1), out=o32))
    del xc, wc, o32

    M, N, K = 16, 8192, 8192
    W = torch.randint(-127, 128, (N, K), generator=g, device=dev, dtype=torch.int8)
    comp, meta = _prep_sparse(ops, W)
    xh = torch.randn((M, K), generator=g, device=dev).half()
    q16 = torch.empty((M, K), dtype=torch.int8, device=dev)
    s16 = torch.empty((M,), dtype=torch.float32, device=dev)
    ops.fused_quantize_activation(xh, M, K, out=q16, scales=s16)
    ws8 = (torch.rand((N,), generator=g, device=dev) * 9e-3 + 1e-3).half()
    b8 = (torch.randn((N,), generator=g, device=dev) * 0.1).half()
    y16 = torch.empty((M, N), dtype=torch.float16, device=dev)
    reps("c4_dense_M16", lambda: ops.int8_gemm_dequant(q16, W, s16, ws8, b8, out=y16))
    reps("c4_sparse_M16", lambda: ops.sparse_int8_gemm(comp, q16, meta, s16, ws8, b8, out=y16))
    del W, comp, meta

    # the reference's fused-quantize example layer: sparse_int8_linear 1280 -> 320 at M = 147,456
    M, K, N = 147456, 1280, 320
    W = torch.randint(-127, 128, (N, K), generator=g, device=dev, dtype=torch.int8)
    comp, meta = _prep_sparse(ops, W)
    xf = torch.randn((M, K), generator=g, device=dev).half()
    wsf = (torch.rand((N,), generator=g, device=dev) * 9e-3 + 1e-3).half()
    bf = (torch.randn((N,), generator=g, device=dev) * 0.1).half()
    qf = torch.empty((M, K), dtype=torch.int8, device=dev)
    sf = torch.empty((M,), dtype=torch.float32, device=dev)
    yf = torch.empty((M, N), dtype=torch.float16, device=dev)
    reps("f1_fq", lambda: ops.sparse_int8_linear(xf, comp, meta, wsf, bf, qf, sf, None, 1, 1, out=yf))
    del W, comp, meta, xf, qf, yf

    # the reference's NCHW FP16 conv API on an upscaler-style 3x3 layer (1, 32, 540, 960) -> 32
    xn = (torch.rand((1, 32, 540, 960), generator=g, device=dev) * 2 - 1).half()
    wn = torch.randint(-127, 128, (32, 32 * 9), generator=g, device=dev, dtype=torch.int8)
    wsn = (torch.rand((32,), generator=g, device=dev) * 0.045 + 0.005).half()
    bn = (torch.rand((32,), generator=g, device=dev) - 0.5).half()
    yn = torch.empty((1, 32, 540, 960), dtype=torch.float16, device=dev)
    wspn = torch.empty((ops.int8_conv2d_workspace_size(32, 540, 960, 32, 3, 3, 1, 1, 1, 1),), dtype=torch.uint8,
                       device=dev)
    reps("f2_conv_nchw", lambda: ops.int8_conv2d_forward(xn, wn, wsn, bn, 3, 3, (1, 1), (1, 1), (1, 1),
                                                         workspace=wspn, out=yn))
    del xn, yn, wspn

    src = torch.empty((COPY_PROBE_BYTES,), dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    src.fill_(1)
    reps("copy", lambda: dst.copy_(src))
    print("traffic probe done", flush=True)
    return 0


def _prep_sparse(ops, W):
    import torch
    N, K = W.shape
    comp = torch.empty((N, K // 2), dtype=torch.int8, device=W.device)
    raw = torch.empty((N * K // 4,), dtype=torch.uint8, device=W.device)
    meta = torch.empty((N * K // 32,), dtype=torch.int32, device=W.device)
    ops.prune_compress_24(W, comp, raw, N, K)
    ops.pack_metadata(raw, meta, N, K)
    return comp, meta


# ---- counter summary (rocprofv3 --pmc runs of --traffic-probe) ---------------------------

PROBE_KERNELS = {
    # probe: (kernel-name substrings, any of which marks a dispatch of the probe)
    "c2_gemm": ("gemm_dma_kernel<256, 256, true, forge_amd::DmaRowMajor>",),
    "c3_sparse": ("sparse_wide_s32_kernel", "sparse_dma32_tail_kernel<false,", "sparse_dma32_kernel<false,"),
    "c3_dense": ("gemm_dma_coltail_kernel<false>", "gemm_dma_kernel<256, 256, false, forge_amd::DmaRowMajor>"),
    "c5_conv": ("conv_window_kernel<7, 2, false>",),
    "c4_dense_M16": ("decode_dense_kernel<true",),
    "c4_sparse_M16": ("decode_sparse_reg_kernel<true",),
    "f1_fq": ("sparse_fq_kernel<5, 48, true",),
    "f2_conv_nchw": ("conv_nchw_cl_kernel",),
    "copy": ("copyBuffer",),
}
_C4_TOK = 16 * 8192
PROBE_WORK = {
    # probe: (algorithmic ops per call, algorithmic bytes per call, MFMA peak TOPS)
    "c2_gemm": (2.0 * 4096 ** 3, 4 * 4096 * 4096 + 4096 * 4 + 4096 * 4, 5000.0),
    "c3_sparse": (2.0 * 4096 * 11008 * 4096, 4096 * 4096 + 11008 * 4096 // 2 + 11008 * 4096 // 8 + 4096 * 11008 * 4,
                  10000.0),
    "c3_dense": (2.0 * 4096 * 11008 * 4096, 4096 * 4096 + 11008 * 4096 + 4096 * 11008 * 4, 5000.0),
    "c5_conv": (2.0 * 100352 * 256 * 2304, 32 * 56 * 56 * 256 + 256 * 2304 + 100352 * 256 * 4, 5000.0),
    "c4_dense_M16": (2.0 * 16 * 8192 * 8192, 8192 * 8192 + _C4_TOK + 16 * 8192 * 2 + 8192 * 4 + 16 * 4, 5000.0),
    "c4_sparse_M16": (2.0 * 16 * 8192 * 8192, 8192 * 8192 // 2 + 8192 * 8192 // 8 + _C4_TOK + 16 * 8192 * 2
                      + 8192 * 4 + 16 * 4, 10000.0),
    "f1_fq": (2.0 * 147456 * 320 * 1280, 2 * 147456 * 1280 + 2 * 147456 * 320 + 320 * 1280 * 5 // 8 + 4 * 320,
              10000.0),
    "f2_conv_nchw": (2.0 * 540 * 960 * 32 * 288, 2 * 2 * 32 * 540 * 960 + 32 * 288 + 4 * 32, 5000.0),
}
SIMDS = 256 * 4          # MI355X: 256 CUs x 4 SIMDs
XCDS = 8


def counter_summary(outdir: str) -> int:
    """Reads the rocprofv3 --pmc CSVs of --traffic-probe runs under outdir (one subdirectory per
    counter set) and writes profiles/kernel_counters.json: per probe, medians over its dispatches
    (one kernel per call)."""
    import csv
    import glob
    import statistics
    rows = {}   # probe -> counter -> list of per-call values
    durs = {}
    gui_floor = []   # smallest GRBM_GUI_ACTIVE per XCD in each run: the dispatch overhead
    for path in sorted(glob.glob(os.path.join(outdir, "*", "*counter_collection.csv"))):
        per_dispatch = {}
        with open(path) as f:
            for r in csv.DictReader(f):
                if r["Counter_Name"] == "GRBM_GUI_ACTIVE" and float(r["Counter_Value"]) > 0:
                    v = float(r["Counter_Value"]) / XCDS
                    if len(gui_floor) <= len(durs.get("_runs", [])):
                        gui_floor.append(v)
                    gui_floor[-1] = min(gui_floor[-1], v)
                probe = next((p for p, subs in PROBE_KERNELS.items() if any(x in r["Kernel_Name"] for x in subs)),
                             None)
                if probe is None:
                    continue
                if probe == "copy" and int(r["Grid_Size"]) < (1 << 16):
                    continue
                d = per_dispatch.setdefault(int(r["Dispatch_Id"]), {"probe": probe, "c": {}})
                d["c"][r["Counter_Name"]] = float(r["Counter_Value"])
                d["t"] = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-3
        # one dispatch per call for every probe
        calls = [{"probe": d["probe"], "c": dict(d["c"]), "t": d["t"], "n": 1}
                 for _, d in sorted(per_dispatch.items())]
        for c in calls:
            for k, v in c["c"].items():
                rows.setdefault(c["probe"], {}).setdefault(k, []).append(v)
            durs.setdefault(c["probe"], []).append(c["t"])
        durs.setdefault("_runs", []).append(path)
    overhead = statistics.median(gui_floor) if gui_floor else 0.0
    med = {p: {k: statistics.median(v) for k, v in cs.items()} for p, cs in rows.items()}
    copy = med.get("copy", {})
    fetch_scale = COPY_PROBE_BYTES / (copy["FETCH_SIZE"] * 1024) if copy.get("FETCH_SIZE") else None
    write_scale = COPY_PROBE_BYTES / (copy["WRITE_SIZE"] * 1024) if copy.get("WRITE_SIZE") else None
    out = {"calibration": {"copy_bytes": COPY_PROBE_BYTES, "copy_fetch_kib": copy.get("FETCH_SIZE"),
                           "copy_write_kib": copy.get("WRITE_SIZE"), "fetch_scale": fetch_scale,
                           "write_scale": write_scale, "gui_overhead_cycles_per_xcd": overhead}, "kernels": {}}
    for p, (ops_, alg_bytes, peak) in PROBE_WORK.items():
        c = med.get(p)
        if not c:
            continue
        e = {"raw": c, "algorithmic_ops": ops_, "algorithmic_bytes": alg_bytes,
             "duration_us_in_counter_run": statistics.median(durs[p])}
        gui = c.get("GRBM_GUI_ACTIVE")
        if gui:
            # GRBM_GUI_ACTIVE is summed over the 8 XCDs and also counts a fixed per-dispatch
            # overhead (its smallest reading in the run, a 256-thread fill kernel's), taken off
            # once per kernel of the call.
            e["clock_ghz"] = (gui / XCDS - overhead) / (e["duration_us_in_counter_run"] * 1e3)
            e["peak_tops_at_clock"] = peak * e["clock_ghz"] / 2.4
        busy, cu_busy = c.get("SQ_VALU_MFMA_BUSY_CYCLES"), c.get("SQ_BUSY_CU_CYCLES")
        if busy is not None and cu_busy:
            # matrix-core busy SIMD-cycles over the SIMD-cycles of CUs with waves resident
            e["mfma_busy"] = busy / (4 * cu_busy)
            e["cu_busy_cycles_per_cu"] = cu_busy / (SIMDS // 4)
        if busy is not None and gui:
            e["mfma_busy_at_clock"] = busy / (SIMDS * e["clock_ghz"] * e["duration_us_in_counter_run"] * 1e3)
        mops = c.get("SQ_INSTS_VALU_MFMA_MOPS_I8")
        if mops is not None:
            e["mfma_ops_counted"] = mops * 512
        if c.get("TCP_TCC_READ_REQ_sum"):
            e["l2_read_latency_cycles"] = c["TCP_TCC_READ_REQ_LATENCY_sum"] / c["TCP_TCC_READ_REQ_sum"]
            e["l2_read_requests"] = c["TCP_TCC_READ_REQ_sum"]
        if c.get("TA_TA_BUSY_sum") and gui:
            e["ta_busy"] = c["TA_TA_BUSY_sum"] / (SIMDS // 4) / (e["clock_ghz"] * e["duration_us_in_counter_run"] * 1e3)
        if c.get("SQ_LDS_IDX_ACTIVE"):
            e["lds_bank_conflict_per_active"] = c.get("SQ_LDS_BANK_CONFLICT", 0.0) / c["SQ_LDS_IDX_ACTIVE"]
        if "FETCH_SIZE" in c and fetch_scale:
            e["read_bytes"] = c["FETCH_SIZE"] * 1024 * fetch_scale
        if "WRITE_SIZE" in c and write_scale:
            e["write_bytes"] = c["WRITE_SIZE"] * 1024 * write_scale
        if "read_bytes" in e and "write_bytes" in e:
            e["traffic_bytes"] = e["read_bytes"] + e["write_bytes"]
            e["traffic_over_algorithmic"] = e["traffic_bytes"] / alg_bytes
        if c.get("TCC_HIT_sum") is not None and c.get("TCC_MISS_sum") is not None:
            tot = c["TCC_HIT_sum"] + c["TCC_MISS_sum"]
            e["l2_hit_rate"] = c["TCC_HIT_sum"] / tot if tot else None
        out["kernels"][p] = e
    path = os.path.join(ROOT, "profiles", "kernel_counters.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)
    with open(os.path.join(ROOT, "profiles", "kernel_counters.md"), "w") as f:
        f.write(_counter_markdown(out))
    print(path)
    return 0


COUNTER_SETS = [
    ("sq", "SQ_VALU_MFMA_BUSY_CYCLES SQ_BUSY_CYCLES SQ_WAVE_CYCLES SQ_LDS_BANK_CONFLICT SQ_LDS_IDX_ACTIVE "
           "SQ_INSTS_VALU_MFMA_MOPS_I8 SQ_BUSY_CU_CYCLES GRBM_GUI_ACTIVE"),
    ("fetch", "FETCH_SIZE GRBM_GUI_ACTIVE"),
    ("write", "WRITE_SIZE TCC_HIT_sum TCC_MISS_sum GRBM_GUI_ACTIVE"),
    ("ta", "TA_TA_BUSY_sum TD_TD_BUSY_sum GRBM_TA_BUSY GRBM_GUI_ACTIVE TCP_TCC_READ_REQ_sum "
           "TCP_TCC_READ_REQ_LATENCY_sum"),
]
PROBE_TITLES = {
    "c2_gemm": "configs[1] GEMM 4096^3, FP16 out (`gemm_dma_kernel<256,256,true>`)",
    "c3_sparse": "configs[2] 2:4 sparse 4096x11008x4096, INT32 out (`sparse_wide_s32_kernel`: 256 tokens x 320-352 weight rows per tile, 2 tiles per CU)",
    "c3_dense": "configs[2] shape dense, INT32 out (`gemm_dma_coltail_kernel<false>`: 256- and 192-row tiles, one launch)",
    "c5_conv": "configs[4] NHWC conv, INT32 out (`conv_window_kernel<7,2,false>`: 224-pixel x 256-channel tiles, input window in LDS once per channel chunk)",
    "c4_dense_M16": "configs[3] M=16 dense decode GEMM (`decode_dense_kernel`)",
    "c4_sparse_M16": "configs[3] M=16 2:4 decode GEMM (`decode_sparse_reg_kernel`)",
    "f1_fq": "fused quantize + 2:4 sparse linear 1280->320 at M=147,456 (`sparse_fq_kernel<5,48,true,3>`)",
    "f2_conv_nchw": "`int8_conv2d_forward` NCHW FP16 (1,32,540,960) 3x3 -> 32 (`conv_nchw_cl_kernel<1,true,8>`: channel-last window, 256-pixel tiles)",
}


def _counter_markdown(out) -> str:
    cal = out["calibration"]
    L = ["# Hardware counters of the dominant kernels (one MI355X)", "",
         "Made by `bench.py --traffic-probe` under `rocprofv3 --pmc`, one counter set per run, then "
         "`python bench.py --counter-summary <out>` (this file and `kernel_counters.json`). Commands, from the "
         "repository root on the GPU box:", "", "```", "cd /tmp && export TMPDIR=/tmp && cd <repo>"]
    for name, counters in COUNTER_SETS:
        L.append(f"rocprofv3 --pmc {counters} --output-format csv -d <out>/{name} -o {name} -- "
                 f"python3 bench.py --traffic-probe")
    L += ["python3 bench.py --counter-summary <out>", "```", "",
          f"Each probe runs its kernel {PROBE_REPS} times; values are medians per call. Definitions:", "",
          "- clock = (GRBM_GUI_ACTIVE / 8 XCDs - the per-dispatch overhead) / kernel duration in the counter "
          f"run; the overhead is the smallest per-XCD GRBM_GUI_ACTIVE of the run ({cal.get('gui_overhead_cycles_per_xcd', 0):.0f} "
          "cycles, a 256-thread fill kernel), taken once per launch.",
          "- MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (4 SIMDs x SQ_BUSY_CU_CYCLES): matrix-core busy cycles over "
          "the SIMD cycles of CUs holding waves. The counter adds 32 cycles per `v_mfma_i32_32x32x32_i8` and per "
          "`v_smfmac_i32_32x32x64_i8` (checked: c2 = 2,097,152 MFMAs x 32); `at clock` divides by 1024 SIMDs x "
          "clock x duration instead.",
          "- peak at clock = the 2.4 GHz peak (dense INT8 5.0 POP/s, 2:4 10.0) scaled to the measured clock.",
          f"- L2-miss bytes = FETCH_SIZE x {cal['fetch_scale']:.3f} + WRITE_SIZE x {cal['write_scale']:.3f} (KiB x 1024), "
          f"the factors that make a {COPY_PROBE_BYTES >> 20} MiB device copy in the same runs read and write its size "
          f"(FETCH_SIZE {cal['copy_fetch_kib']:.1f} KiB, WRITE_SIZE {cal['copy_write_kib']:.1f} KiB). These count "
          "traffic between the L2s and the memory fabric: HBM plus what the 256 MB MALL serves, an upper bound of "
          "HBM bytes; `alg.` is the algorithmic bytes (operands read once, output written once).",
          "- L2 read latency = TCP_TCC_READ_REQ_LATENCY_sum / TCP_TCC_READ_REQ_sum (cycles); TA busy = "
          "TA_TA_BUSY_sum / 256 / (clock x duration).", "",
          "| probe | us (counter run) | clock GHz | MFMA busy (at clock) | peak at clock | L2-miss MB (alg.) | L2 hit | "
          "L2 lat. | TA busy | LDS confl./active |",
          "|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|"]
    for p, e in out["kernels"].items():
        unit = "TOPS"
        L.append(f"| {PROBE_TITLES.get(p, p)} | {e['duration_us_in_counter_run']:.1f} | {e.get('clock_ghz', 0):.2f} | "
                 f"{100 * e.get('mfma_busy', 0):.1f} % ({100 * e.get('mfma_busy_at_clock', 0):.1f} %) | "
                 f"{e.get('peak_tops_at_clock', 0):.0f} {unit} | {e.get('traffic_bytes', 0) / 1e6:.1f} "
                 f"({e['algorithmic_bytes'] / 1e6:.1f}) | {100 * (e.get('l2_hit_rate') or 0):.1f} % | "
                 f"{e.get('l2_read_latency_cycles', 0):.0f} | {100 * e.get('ta_busy', 0):.0f} % | "
                 f"{e.get('lds_bank_conflict_per_active', 0):.3f} |")
    L += ["", "Raw medians per call (counter: value) are in `kernel_counters.json` under each probe's `raw`.", ""]
    return "\n".join(L)


def events_time_ms(fn, reps: int) -> float:
    """Average duration of fn() over reps launches, HIP events on torch's current stream
    (the stream the library launches on)."""
    import torch
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        fn()
    e.record()
    e.synchronize()
    return s.elapsed_time(e) / reps


def graph_time_ms(calls, replays: int = 20) -> float:
    """Average GPU time of one call: the calls (each one library call on torch's current
    stream) are captured into one HIP graph and replayed, so host launch overhead is out of
    the timing (the reference's bench_int8_sparse.cu:41-85 protocol)."""
    import torch
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for c in calls:
            c()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for c in calls:
            c()
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(replays):
        graph.replay()
    e.record()
    e.synchronize()
    return s.elapsed_time(e) / (replays * len(calls))


def graph_median_ms(fn, min_sample_ms: float = 0.2, warmup: int = 50, reps: int = 100) -> float:
    """The reference benchmark's protocol (benchmarks/bench_int8_sparse.cu:41-85): fn is
    captured n times into one graph so that a replay takes >= min_sample_ms, replays are
    warmed up, then each of `reps` replays is bracketed by events; the per-call time is the
    median replay / n. Inputs stay resident (L2/MALL), as in the reference."""
    import math
    import torch
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(10):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(20):
        fn()
    e.record()
    e.synchronize()
    n = max(1, math.ceil(min_sample_ms / max(s.elapsed_time(e) / 20, 1e-3)))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(n):
            fn()
    for _ in range(warmup):
        graph.replay()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    for a, b in evs:
        a.record()
        graph.replay()
        b.record()
    torch.cuda.synchronize()
    ts = sorted(a.elapsed_time(b) for a, b in evs)
    return ts[len(ts) // 2] / n


def spin(fn, seconds: float) -> None:
    """Runs fn back to back for `seconds` of GPU time (clocks up before a measurement)."""
    import torch
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    while True:
        for _ in range(50):
            fn()
        e.record()
        e.synchronize()
        if s.elapsed_time(e) >= seconds * 1e3:
            return


def _probe_lib():
    """libforge_probes.so (forge_amd.build builds it beside the product library)."""
    import ctypes
    path = os.path.join(ROOT, "forge_amd", "lib", "libforge_probes.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} missing: build first (python -m forge_amd.build)")
    return ctypes.CDLL(path)


# The dense engine's loop at 8192^3 work: 1024 workgroups (the 32 x 32 tiles of 256 x 256) x
# 64 stages of 128-deep K each, on one 64 KB stage of operands loaded once per workgroup.
MFMA_PROBE_WGS, MFMA_PROBE_STAGES = 1024, 64
STREAM_PROBE_BYTES, STREAM_PROBE_BUFS = 256 << 20, 3     # 3 x 256 MiB rotate past the 256 MB MALL


def _probe_setup(dev):
    """Device buffers of the probes: random and constant INT8 stages for probe_mfma_lds, the
    rotating streaming buffers, the DMA probe's rows."""
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(11)
    tiles = 64
    rnd = [torch.randint(-127, 128, (tiles * 256 * 128,), generator=g, device=dev, dtype=torch.int8) for _ in range(2)]
    one = torch.ones((tiles * 256 * 128,), dtype=torch.int8, device=dev)
    bufs = [torch.randint(-127, 128, (STREAM_PROBE_BYTES,), generator=g, device=dev, dtype=torch.int8)
            for _ in range(STREAM_PROBE_BUFS)]
    dma = torch.randint(-127, 128, (256 * 256 * 8192,), generator=g, device=dev, dtype=torch.int8)
    out = torch.zeros((4096,), dtype=torch.int32, device=dev)
    return {"rnd": rnd, "one": one, "tiles": tiles, "bufs": bufs, "dma": dma, "out": out}


def _probe_calls(P, bufs):
    """name -> (one launch of the probe, its work: ('ops', n) or ('bytes', n))."""
    import ctypes
    import torch
    st = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    V = ctypes.c_void_p
    A, B = bufs["rnd"]
    one, out, tiles = bufs["one"], bufs["out"], bufs["tiles"]
    ops = 2.0 * MFMA_PROBE_WGS * 256 * 256 * 128 * MFMA_PROBE_STAGES

    def mfma(a, b, reads):
        return lambda: P.probe_mfma_lds(V(a.data_ptr()), V(b.data_ptr()), V(out.data_ptr()), MFMA_PROBE_WGS,
                                        MFMA_PROBE_STAGES, tiles, reads, st())
    calls = {
        "mfma_lds_random": (mfma(A, B, 1), ("ops", ops)),
        "mfma_lds_const": (mfma(one, one, 1), ("ops", ops)),
        "mfma_only_random": (mfma(A, B, 0), ("ops", ops)),
        "mfma_only_const": (mfma(one, one, 0), ("ops", ops)),
    }
    state = {"i": 0}

    def stream():
        b = bufs["bufs"][state["i"] % len(bufs["bufs"])]
        state["i"] += 1
        return P.probe_stream(V(b.data_ptr()), ctypes.c_size_t(b.numel()), 2048, V(out.data_ptr()), st())
    calls["stream"] = (stream, ("bytes", STREAM_PROBE_BYTES))
    dma = bufs["dma"]
    for share in (1, 4, 8, 32):
        for half in (0, 1):
            for ldsr in (0, 1):
                if half and ldsr:
                    continue
                calls[f"dma_s{share}_h{half}_r{ldsr}"] = (
                    lambda share=share, half=half, ldsr=ldsr: P.probe_dma(
                        V(dma.data_ptr()), ctypes.c_uint32(dma.numel()), 4096 if half else 8192, share, half, ldsr,
                        V(out.data_ptr()), st()),
                    ("bytes", 256 * 256 * 8192))
    return calls


def run_probes() -> int:
    """bench.py --probes: every probe timed with HIP events (settled clocks: each runs 0.5 s
    first); one JSON line. MFMA probes in TOPS (the 8192^3 GEMM's work), the streaming read in
    TB/s, the DMA probe in bytes per CU per clock at the clock the rest of the line reports is not
    known, so in GB/s per CU. Also the vendor library (hipBLASLt through torch._int_mm, INT32
    out) at 4096^3 and 8192^3 next to forge_int8_gemm_s32, checked bit-equal."""
    import torch
    import forge_amd
    from forge_amd import ops
    forge_amd.load()
    dev = torch.device("cuda:0")
    P = _probe_lib()
    bufs = _probe_setup(dev)
    res = {}
    for name, (fn, (kind, work)) in _probe_calls(P, bufs).items():
        assert fn() == 0, name
        torch.cuda.synchronize()
        spin(fn, 0.5)
        t = min(events_time_ms(fn, 10) for _ in range(3))
        if kind == "ops":
            res[name] = {"us": round(t * 1e3, 2), "TOPS": round(work / t / 1e9, 1)}
        elif name == "stream":
            res[name] = {"us": round(t * 1e3, 2), "TBs": round(work / t / 1e9, 3)}
        else:
            res[name] = {"us": round(t * 1e3, 2), "GBs_per_CU": round(work / 256 / t / 1e6, 1)}
        print(f"probe {name}: {res[name]}", flush=True)
    res["vendor_hipblaslt"] = vendor_gemm_compare(dev)
    print(json.dumps({"probes": res}), flush=True)
    return 0


def run_one_probe(name: str) -> int:
    """bench.py --probe NAME: that probe PROBE_REPS times (for rocprofv3 --pmc runs)."""
    import torch
    dev = torch.device("cuda:0")
    P = _probe_lib()
    calls = _probe_calls(P, _probe_setup(dev))
    if name not in calls:
        raise SystemExit(f"unknown probe {name}; one of {', '.join(calls)}")
    fn = calls[name][0]
    for _ in range(PROBE_REPS):
        assert fn() == 0
    torch.cuda.synchronize()
    print(f"probe {name} done", flush=True)
    return 0


def vendor_gemm_compare(dev):
    """hipBLASLt (torch._int_mm, INT32 out) next to forge_int8_gemm_s32 at 4096^3 and 8192^3:
    a vendor reference point, not part of the product; outputs checked bit-equal."""
    import torch
    from forge_amd import ops
    g = torch.Generator(device=dev)
    g.manual_seed(13)
    out = {}
    for n in (4096, 8192):
        A = torch.randint(-127, 128, (n, n), generator=g, device=dev, dtype=torch.int8)
        B = torch.randint(-127, 128, (n, n), generator=g, device=dev, dtype=torch.int8)
        Bt = B.t()
        C = torch.empty((n, n), dtype=torch.int32, device=dev)
        ref = torch._int_mm(A, Bt)
        ops.int8_gemm_s32(A, B, out=C)
        torch.cuda.synchronize()
        equal = bool(torch.equal(ref, C))
        f_lt = lambda: torch._int_mm(A, Bt)
        f_fg = lambda: ops.int8_gemm_s32(A, B, out=C)
        spin(lambda: (f_lt(), f_fg()), 0.5)
        t_lt, t_fg = [], []
        for _ in range(3):
            t_lt.append(events_time_ms(f_lt, 10))
            t_fg.append(events_time_ms(f_fg, 10))
        ops_ = 2.0 * n ** 3
        out[str(n)] = {"hipblaslt_us": round(min(t_lt) * 1e3, 2), "forge_us": round(min(t_fg) * 1e3, 2),
                       "hipblaslt_tops": round(ops_ / min(t_lt) / 1e9, 1), "forge_tops": round(ops_ / min(t_fg) / 1e9, 1),
                       "bit_equal": equal}
        del A, B, C, ref
    torch.cuda.empty_cache()
    return out


def bench_reference_sweep(dev):
    """The reference's own sparse benchmark (benchmarks/bench_int8_sparse.cu:113-114, 235-236):
    sparse_int8_gemm with the dequant epilogue, automatic plan and a split-K workspace, on
    K x N in {1536x6144, 6144x1536, 1280x5120, 5120x1280} x M in {64, 1024, 4096, 8192}, the
    dense int8_gemm_dequant beside it; and sparse_int8_linear (FP16 in) at its narrow-N layer
    shapes, two-pass / fused / automatic. Microseconds per call."""
    import torch
    from forge_amd import ops
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    gemm, layers, best = {}, {}, 0.0
    spun = False
    for K, N in ((1536, 6144), (6144, 1536), (1280, 5120), (5120, 1280)):
        W = torch.randint(-127, 128, (N, K), generator=g, device=dev, dtype=torch.int8)
        comp = torch.empty((N, K // 2), dtype=torch.int8, device=dev)
        raw = torch.empty((N * K // 4,), dtype=torch.uint8, device=dev)
        meta = torch.empty((N * K // 32,), dtype=torch.int32, device=dev)
        ops.prune_compress_24(W, comp, raw, N, K)
        ops.pack_metadata(raw, meta, N, K)
        ws = (torch.rand((N,), generator=g, device=dev) * 0.01 + 0.001).half()
        b = (torch.rand((N,), generator=g, device=dev) - 0.5).half()
        xh = torch.randn((8192, K), generator=g, device=dev).half()
        row = {}
        for M in (64, 1024, 4096, 8192):
            xq = torch.empty((M, K), dtype=torch.int8, device=dev)
            xs = torch.empty((M,), dtype=torch.float32, device=dev)
            out = torch.empty((M, N), dtype=torch.float16, device=dev)
            wsp = torch.empty((M, N), dtype=torch.float32, device=dev)
            quant = lambda: ops.fused_quantize_activation(xh[:M], M, K, out=xq, scales=xs)
            quant()
            sp = lambda: ops.sparse_int8_gemm(comp, xq, meta, xs, ws, b, splitk_workspace=wsp, split_k=0, out=out)
            de = lambda: ops.int8_gemm_dequant(xq, W, xs, ws, b, out=out)
            if not spun:   # the reference spins >= 1 s of GEMMs before its first measurement
                spin(sp, 1.0)
                spun = True
            sp()
            plan = ops.sparse_int8_gemm_plan(M, K, N, 0, True)
            route_sp = ops.last_route()
            de()
            route_de = ops.last_route()
            t_sp = graph_median_ms(sp)
            t_de = graph_median_ms(de)
            t_q = graph_median_ms(quant)
            tops = 2.0 * M * N * K / t_sp / 1e9
            best = max(best, tops)
            row[str(M)] = {"sparse_us": round(t_sp * 1e3, 2), "sparse_tops": round(tops, 1),
                           "dense_us": round(t_de * 1e3, 2), "quant_us": round(t_q * 1e3, 2),
                           "plan": f"tile{plan[0]} s{plan[1]}", "sparse_engine": route_sp,
                           "dense_engine": route_de}
        gemm[f"{K}x{N}"] = row
        del W, comp, raw, meta, xh
    for K, N, M in ((1280, 320, 147456), (640, 320, 147456), (640, 640, 36864), (1024, 640, 37008),
                    (1024, 320, 37008), (1280, 1280, 9216)):
        W = torch.randint(-127, 128, (N, K), generator=g, device=dev, dtype=torch.int8)
        comp = torch.empty((N, K // 2), dtype=torch.int8, device=dev)
        raw = torch.empty((N * K // 4,), dtype=torch.uint8, device=dev)
        meta = torch.empty((N * K // 32,), dtype=torch.int32, device=dev)
        ops.prune_compress_24(W, comp, raw, N, K)
        ops.pack_metadata(raw, meta, N, K)
        ws = (torch.rand((N,), generator=g, device=dev) * 0.01 + 0.001).half()
        b = (torch.rand((N,), generator=g, device=dev) - 0.5).half()
        x = (torch.rand((M, K), generator=g, device=dev) * 4 - 2).half()
        sq = torch.empty((M, K), dtype=torch.int8, device=dev)
        ss = torch.empty((M,), dtype=torch.float32, device=dev)
        wsp = torch.empty((M, N), dtype=torch.float32, device=dev)
        t = [graph_median_ms(lambda p=p: ops.sparse_int8_linear(x, comp, meta, ws, b, sq, ss, wsp, 0, p))
             for p in (0, 1, -1)]
        ops.sparse_int8_linear(x, comp, meta, ws, b, sq, ss, wsp, 0, -1)
        layers[f"{K}x{N}@{M}"] = {"two_pass_us": round(t[0] * 1e3, 2), "fused_us": round(t[1] * 1e3, 2),
                                  "auto_us": round(t[2] * 1e3, 2), "auto_engine": ops.last_route()}
        del W, comp, raw, meta, x, sq, ss, wsp
    torch.cuda.empty_cache()
    return {"protocol": "bench_int8_sparse.cu: >= 1 s of GEMMs to reach clock, then per call a graph of n "
                        "calls >= 0.2 ms, 50 warm-up + 100 timed replays, median / n, L2-resident inputs; "
                        "quant_us = the per-token quantize of the M x K activations on the same protocol; "
                        "plan = sparse_int8_gemm_plan (kSparseTile index, split); *_engine = the kernel that ran",
            "gemm": gemm, "layers": layers, "peak_sparse_tops": round(best, 1)}


def make_c2(dev, seed=2):
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    M = N = K = 4096
    x = torch.randn((M, K), generator=g, device=dev, dtype=torch.float32)
    cols = torch.randperm(K, generator=g, device=dev)[:8]
    x[:, cols] *= 20
    x = x.half()
    W = torch.randint(-127, 128, (N, K), generator=g, device=dev, dtype=torch.int8)
    ws = (torch.rand((N,), generator=g, device=dev) * 9e-3 + 1e-3).half()
    b = (torch.randn((N,), generator=g, device=dev) * 0.1).half()
    return x, W, ws, b


def cpu_baseline(target_s: float = 12.0):
    """The oracle's INT32 loop + dequant epilogue (oracle/) on configs[1] (M = N = K = 4096),
    split over output rows on the host's cores up to 16 POSIX threads (the GPU box's CPU share
    per GPU; nproc is recorded), over the whole workload; the single-threaded rate over as many
    rows as fit in about target_s seconds is recorded in the sample text."""
    from oracle import oracle
    oracle.build()
    rng = np.random.default_rng(2)
    M = K = N = 4096
    W = rng.integers(-127, 128, (N, K)).astype(np.int8)
    x = rng.standard_normal((M, K), dtype=np.float32)
    x[:, rng.choice(K, 8, replace=False)] *= 20
    q, s = oracle.quantize_rows(x.astype(np.float16))
    ws = rng.uniform(1e-3, 1e-2, N).astype(np.float16)
    b = (rng.standard_normal(N) * 0.1).astype(np.float16)
    rows = 32
    t, _ = oracle.time_gemm_dequant_rows(q, W, s, ws, b, rows)
    rows = int(max(32, min(M, target_s / max(t, 1e-6) * rows)))
    t1, _ = oracle.time_gemm_dequant_rows(q, W, s, ws, b, rows)
    tops1 = 2.0 * rows * N * K / t1 / 1e12
    nproc = os.cpu_count() or 1
    threads = oracle.cpu_threads()
    tm, _ = oracle.time_gemm_dequant_rows_mt(q, W, s, ws, b, M, threads)
    tops = 2.0 * M * N * K / tm / 1e12
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": tops, "unit": "TOPS", "cores": threads, "kind": "port",
            "sample": f"oracle INT32 loop + dequant epilogue over all 4096 rows of configs[1] (N=K=4096) split "
                      f"over output rows on {threads} threads: {tm:.2f} s; one thread over {rows} rows: "
                      f"{t1:.2f} s = {tops1:.4f} TOPS; gcc -O3, host CPU '{model}', nproc {nproc} (threads capped "
                      f"at 16, the box's CPU share per GPU)"}


def bench_extra(dev):
    import torch
    from forge_amd import ops
    out = {}
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    # 2:4 sparse 4096 x 11008 x 4096 INT32 out, and the same shape dense
    M, K, N = 4096, 4096, 11008
    W = torch.randint(-127, 128, (N, K), generator=g, device=dev, dtype=torch.int8)
    x = torch.randint(-127, 128, (M, K), generator=g, device=dev, dtype=torch.int8)
    comp = torch.empty((N, K // 2), dtype=torch.int8, device=dev)
    raw = torch.empty((N * K // 4,), dtype=torch.uint8, device=dev)
    meta = torch.empty((N * K // 32,), dtype=torch.int32, device=dev)
    ops.prune_compress_24(W, comp, raw, N, K)
    ops.pack_metadata(raw, meta, N, K)
    C = torch.empty((M, N), dtype=torch.int32, device=dev)
    for _ in range(3):
        ops.sparse_int8_gemm_s32(comp, x, meta, out=C)
        ops.int8_gemm_s32(x, W, out=C)
    # The clocks settle over the first ~1 s of this load (both kernels speed up, the dense one
    # more: after the idle CPU-baseline leg a first block of each measured 153 / 208 us against
    # 127 / 174 us settled), so both run for 1 s first, as the reference's own benchmark does
    # before it measures (bench_int8_sparse.cu:198-211); then five alternating rounds of 10
    # calls each, the median per side.
    sp3 = lambda: ops.sparse_int8_gemm_s32(comp, x, meta, out=C)
    de3 = lambda: ops.int8_gemm_s32(x, W, out=C)
    spin(lambda: (sp3(), de3()), 1.0)
    rounds_sp, rounds_de = [], []
    for _ in range(5):
        rounds_sp.append(events_time_ms(sp3, 10))
        rounds_de.append(events_time_ms(de3, 10))
    t_sp = sorted(rounds_sp)[2]
    t_de = sorted(rounds_de)[2]
    ops_ = 2.0 * M * N * K
    out["c3_sparse_tops"] = ops_ / t_sp / 1e9
    out["c3_dense_tops"] = ops_ / t_de / 1e9
    out["c3_sparse_over_dense"] = t_de / t_sp
    del W, x, comp, raw, meta, C
    torch.cuda.empty_cache()

    # decode, N = K = 8192; rotating weight copies so that the 256 MB MALL cannot
    # serve them: 8 dense copies (537 MB), 10 sparse copies (W_comp + index words, 420 MB).
    N = K = 8192
    copies, sp_copies = 8, 10
    Ws = [torch.randint(-127, 128, (N, K), generator=g, device=dev, dtype=torch.int8) for _ in range(sp_copies)]
    comps, metas = [], []
    for Wc in Ws:
        cp = torch.empty((N, K // 2), dtype=torch.int8, device=dev)
        rw = torch.empty((N * K // 4,), dtype=torch.uint8, device=dev)
        mt = torch.empty((N * K // 32,), dtype=torch.int32, device=dev)
        ops.prune_compress_24(Wc, cp, rw, N, K)
        ops.pack_metadata(rw, mt, N, K)
        comps.append(cp)
        metas.append(mt)
    del Ws[copies:]
    ws = (torch.rand((N,), generator=g, device=dev) * 9e-3 + 1e-3).half()
    b = (torch.randn((N,), generator=g, device=dev) * 0.1).half()
    for M in (1, 4, 16):
        xh = torch.randn((M, K), generator=g, device=dev).half()
        sq = torch.empty((M, K), dtype=torch.int8, device=dev)
        ss = torch.empty((M,), dtype=torch.float32, device=dev)
        dense = [lambda c=c: ops.int8_linear(xh, Ws[c], ws, b, sq, ss) for c in range(copies)]
        sparse = [lambda c=c: ops.sparse_int8_linear(xh, comps[c], metas[c], ws, b, sq, ss) for c in range(sp_copies)]
        td = graph_time_ms(dense * 6)
        ts = graph_time_ms(sparse * 5)
        bytes_d = N * K + M * K * 2 + M * N * 2 + N * 2 + N * 2
        bytes_s = N * K // 2 + N * K // 8 + M * K * 2 + M * N * 2 + N * 2 + N * 2
        out[f"c4_M{M}_dense_GBs"] = bytes_d / td / 1e6
        out[f"c4_M{M}_sparse_GBs"] = bytes_s / ts / 1e6
        out[f"c4_M{M}_dense_us"] = td * 1e3
        out[f"c4_M{M}_sparse_us"] = ts * 1e3
        # The decode GEMM alone (the gate's "decode-shape GEMM"): on the quantized tokens left in
        # the scratch, INT8 tokens in its algorithmic bytes.
        ops.fused_quantize_activation(xh, M, K, out=sq, scales=ss)
        y = torch.empty((M, N), dtype=torch.float16, device=dev)
        gd = [lambda c=c: ops.int8_gemm_dequant(sq, Ws[c], ss, ws, b, out=y) for c in range(copies)]
        gs = [lambda c=c: ops.sparse_int8_gemm(comps[c], sq, metas[c], ss, ws, b, out=y) for c in range(sp_copies)]
        tgd = graph_time_ms(gd * 6)
        tgs = graph_time_ms(gs * 5)
        gbytes_d = N * K + M * K + M * N * 2 + N * 4 + M * 4
        gbytes_s = N * K // 2 + N * K // 8 + M * K + M * N * 2 + N * 4 + M * 4
        out[f"c4_M{M}_dense_gemm_us"] = tgd * 1e3
        out[f"c4_M{M}_dense_gemm_GBs"] = gbytes_d / tgd / 1e6
        out[f"c4_M{M}_sparse_gemm_us"] = tgs * 1e3
        out[f"c4_M{M}_sparse_gemm_GBs"] = gbytes_s / tgs / 1e6
    del Ws, comps, metas
    torch.cuda.empty_cache()

    # INT8 NHWC conv 3x3, pad 1, stride 1: (32,56,56,256) x (256,3,3,256) -> INT32,
    # and the same with the per-channel dequant + bias epilogue (FP16 out). Implicit GEMM
    # M = 32*56*56 = 100,352, N = 256, K = 2,304.
    xc = torch.randint(-127, 128, (32, 56, 56, 256), generator=g, device=dev, dtype=torch.int8)
    wc = torch.randint(-127, 128, (256, 3, 3, 256), generator=g, device=dev, dtype=torch.int8)
    Mc = 32 * 56 * 56
    asc = torch.full((Mc,), 0.02, dtype=torch.float32, device=dev)
    wsc = (torch.rand((256,), generator=g, device=dev) * 9e-3 + 1e-3).half()
    bc = (torch.randn((256,), generator=g, device=dev) * 0.1).half()
    o32 = torch.empty((32, 56, 56, 256), dtype=torch.int32, device=dev)
    o16 = torch.empty((32, 56, 56, 256), dtype=torch.float16, device=dev)
    conv32 = lambda: ops.int8_conv2d_nhwc_s32(xc, wc, pad=(1, 1), out=o32)
    conv16 = lambda: ops.int8_conv2d_nhwc_dequant(xc, wc, asc, wsc, bc, pad=(1, 1), out=o16)
    spin(lambda: (conv32(), conv16()), 1.0)     # settled clocks, as for configs[2]
    t32 = events_time_ms(conv32, 10)
    t16 = events_time_ms(conv16, 10)
    ops_c = 2.0 * Mc * 256 * 2304
    out["c5_conv_s32_tops"] = ops_c / t32 / 1e9
    out["c5_conv_s32_us"] = t32 * 1e3
    out["c5_conv_dequant_tops"] = ops_c / t16 / 1e9
    out["c5_conv_dequant_us"] = t16 * 1e3
    del xc, wc, o32, o16
    torch.cuda.empty_cache()

    # The rest of the INT8 conv family (NCHW FP16 in and out), HBM-bound:
    # depthwise 3x3, pad 1: (1, 64, 540, 960) -> same shape; bytes = input + output;
    # ConvTranspose2d k2s2: (1, 64, 270, 480) -> (1, 32, 540, 960); bytes = input + output + weights.
    # Each leg rotates over enough input/output pairs that the 256 MB MALL cannot hold them
    # (depthwise: 3 x 133 MB, transposed conv: 6 x 50 MB), graph-replayed.
    nd, nt = 3, 6
    xds = [(torch.rand((1, 64, 540, 960), generator=g, device=dev) * 2 - 1).half() for _ in range(nd)]
    wd = torch.randint(-127, 128, (64, 9), generator=g, device=dev, dtype=torch.int8)
    wsd = (torch.rand((64,), generator=g, device=dev) * 0.045 + 0.005).half()
    bd = (torch.rand((64,), generator=g, device=dev) - 0.5).half()
    yds = [torch.empty_like(xds[0]) for _ in range(nd)]
    dws = [lambda i=i: ops.int8_depthwise_conv2d_forward(xds[i], wd, wsd, bd, 3, 3, (1, 1), out=yds[i])
           for i in range(nd)]
    xts = [(torch.rand((1, 64, 270, 480), generator=g, device=dev) * 2 - 1).half() for _ in range(nt)]
    wt = torch.randint(-127, 128, (4 * 32, 64), generator=g, device=dev, dtype=torch.int8)
    wst = (torch.rand((32,), generator=g, device=dev) * 0.045 + 0.005).half()
    bt = (torch.rand((32,), generator=g, device=dev) - 0.5).half()
    yts = [torch.empty((1, 32, 540, 960), dtype=torch.float16, device=dev) for _ in range(nt)]
    wsp = torch.empty((ops.int8_conv_transpose2d_k2s2_workspace_size(64, 270, 480, 32),), dtype=torch.uint8,
                      device=dev)
    cts = [lambda i=i: ops.int8_conv_transpose2d_k2s2_forward(xts[i], wt, wst, bt, workspace=wsp, out=yts[i])
           for i in range(nt)]
    t_dw = graph_time_ms(dws * 6)
    t_ct = graph_time_ms(cts * 4)
    out["f2_depthwise_us"] = t_dw * 1e3
    out["f2_depthwise_GBs"] = (xds[0].numel() * 2 + yds[0].numel() * 2) / t_dw / 1e6
    out["f2_convT_us"] = t_ct * 1e3
    out["f2_convT_GBs"] = (xts[0].numel() * 2 + yts[0].numel() * 2 + wt.numel()) / t_ct / 1e6
    del xds, yds, xts, yts, wsp
    torch.cuda.empty_cache()

    # The reference's NCHW FP16 conv API (int8_conv2d_forward) on one launch: per-patch-row
    # quantize, implicit GEMM and NCHW epilogue fused; an upscaler-style 3x3 layer,
    # (1, 32, 540, 960) -> (1, 32, 540, 960), pad 1; HBM GB/s of input + output bytes, rotating
    # over 5 input/output pairs (330 MB) so the MALL cannot hold them, graph-replayed.
    nn_ = 5
    xcs = [(torch.rand((1, 32, 540, 960), generator=g, device=dev) * 2 - 1).half() for _ in range(nn_)]
    wcn = torch.randint(-127, 128, (32, 32 * 9), generator=g, device=dev, dtype=torch.int8)
    wscn = (torch.rand((32,), generator=g, device=dev) * 0.045 + 0.005).half()
    bcn = (torch.rand((32,), generator=g, device=dev) - 0.5).half()
    ycs = [torch.empty((1, 32, 540, 960), dtype=torch.float16, device=dev) for _ in range(nn_)]
    wspn = torch.empty((ops.int8_conv2d_workspace_size(32, 540, 960, 32, 3, 3, 1, 1, 1, 1),), dtype=torch.uint8,
                       device=dev)
    cns = [lambda i=i: ops.int8_conv2d_forward(xcs[i], wcn, wscn, bcn, 3, 3, (1, 1), (1, 1), (1, 1), workspace=wspn,
                                               out=ycs[i]) for i in range(nn_)]
    t_cn = graph_time_ms(cns * 4)
    out["f2_conv_nchw_us"] = t_cn * 1e3
    out["f2_conv_nchw_GBs"] = (xcs[0].numel() * 2 + ycs[0].numel() * 2) / t_cn / 1e6
    out["f2_conv_nchw_tops"] = 2.0 * 540 * 960 * 32 * 288 / t_cn / 1e9
    del xcs, ycs, wspn
    torch.cuda.empty_cache()

    # Weight preparation for SparseLinear at configs[2]'s weight (11008 x 4096, fp32): the one
    # pass (quantize + prune + compress + gfx950 pack) against the reference's sequence of
    # separate steps (quantize rows, prune_compress_24 through a raw-nibble buffer, pack).
    N, K = 11008, 4096
    wf = torch.randn((N, K), generator=g, device=dev) * 0.02
    qw = torch.empty((N, K), dtype=torch.int8, device=dev)
    qs = torch.empty((N,), dtype=torch.float16, device=dev)
    cp = torch.empty((N, K // 2), dtype=torch.int8, device=dev)
    rw = torch.empty((N * K // 4,), dtype=torch.uint8, device=dev)
    mt = torch.empty((N * K // 32,), dtype=torch.int32, device=dev)
    one = lambda: ops.prepare_sparse_weight(wf)
    def steps():
        ops.quantize_weight_rows(wf, qw, qs)
        ops.prune_compress_24(qw, cp, rw, N, K)
        ops.pack_metadata(rw, mt, N, K)
    for _ in range(3):
        one()
        steps()
    t_one = events_time_ms(one, 10)
    t_steps = events_time_ms(steps, 10)
    out["f4_prep_sparse_us"] = t_one * 1e3
    out["f4_prep_sparse_GBs"] = (N * K * 4 + N * K // 2 + N * K // 8 + N * 2) / t_one / 1e6
    out["f4_prep_steps_us"] = t_steps * 1e3
    del wf, qw, qs, cp, rw, mt
    torch.cuda.empty_cache()

    # The reference's fused-quantize example layer (int8_sparse.cuh:82): sparse_int8_linear
    # 1280 -> 320 at M = 147,456, FP16 in/out, on the fused path (path 1) and on the two-pass
    # path (path 0); algorithmic bytes of the fused path = x + out + compressed weights + index
    # words + w_scale and bias.
    M, K, N = 147456, 1280, 320
    W = torch.randint(-127, 128, (N, K), generator=g, device=dev, dtype=torch.int8)
    comp = torch.empty((N, K // 2), dtype=torch.int8, device=dev)
    raw = torch.empty((N * K // 4,), dtype=torch.uint8, device=dev)
    meta = torch.empty((N * K // 32,), dtype=torch.int32, device=dev)
    ops.prune_compress_24(W, comp, raw, N, K)
    ops.pack_metadata(raw, meta, N, K)
    xs = torch.randn((M, K), generator=g, device=dev).half()
    ws = (torch.rand((N,), generator=g, device=dev) * 9e-3 + 1e-3).half()
    bs = (torch.randn((N,), generator=g, device=dev) * 0.1).half()
    sq = torch.empty((M, K), dtype=torch.int8, device=dev)
    ss = torch.empty((M,), dtype=torch.float32, device=dev)
    fq = lambda: ops.sparse_int8_linear(xs, comp, meta, ws, bs, sq, ss, None, 1, 1)
    tp = lambda: ops.sparse_int8_linear(xs, comp, meta, ws, bs, sq, ss, None, 1, 0)
    for _ in range(3):
        fq()
        tp()
    t_fq = events_time_ms(fq, 10)
    t_tp = events_time_ms(tp, 10)
    out["f1_fq_us"] = t_fq * 1e3
    out["f1_twopass_us"] = t_tp * 1e3
    out["f1_fq_GBs"] = (2 * M * K + 2 * M * N + N * K // 2 + N * K // 8 + 4 * N) / t_fq / 1e6
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--traffic-probe", action="store_true")
    ap.add_argument("--counter-summary", metavar="DIR", default=None)
    ap.add_argument("--probes", action="store_true", help="run the measurement probes (libforge_probes.so)")
    ap.add_argument("--probe", metavar="NAME", default=None, help="one probe, PROBE_REPS launches (for rocprofv3)")
    args = ap.parse_args()
    if args.traffic_probe:
        return traffic_probe()
    if args.probes:
        return run_probes()
    if args.probe:
        return run_one_probe(args.probe)
    if args.counter_summary:
        return counter_summary(args.counter_summary)
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the W8A8 kernels shard by token rows or weight columns with no communication).",
              file=sys.stderr)
        return 2

    import torch
    import forge_amd
    from forge_amd import ops
    forge_amd.load()
    dev = torch.device("cuda:0")
    x, W, ws, b = make_c2(dev)
    M, K = x.shape
    N = W.shape[0]
    sq = torch.empty((M, K), dtype=torch.int8, device=dev)
    ss = torch.empty((M,), dtype=torch.float32, device=dev)
    y = torch.empty((M, N), dtype=torch.float16, device=dev)

    def step():
        ops.int8_linear(x, W, ws, b, sq, ss)

    # spin to clocks, then warm up
    t_end = time.time() + 1.0
    while time.time() < t_end:
        for _ in range(20):
            step()
        torch.cuda.synchronize()
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms = (t1 - t0) * 1e3 / args.steps
    tops = 2.0 * M * N * K / (ms * 1e-3) / 1e12

    # dominant kernel alone: the dequantizing GEMM on the quantized activations
    gemm = lambda: ops.int8_gemm_dequant(sq, W, ss, ws, b, out=y)
    for _ in range(5):
        gemm()
    t_gemm = events_time_ms(gemm, 50)
    achieved = 2.0 * M * N * K / (t_gemm * 1e-3) / 1e12
    # quantize is short enough that per-call host launch cost would dominate events: graph replay
    quant = lambda: ops.fused_quantize_activation(x, M, K, out=sq, scales=ss)
    t_q = graph_time_ms([quant] * 20)

    line = {
        "metric": METRIC,
        "value": round(tops, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (configs[1]: N(0,1) fp16 activations with 8 outlier channels x20, "
                "uniform int8 weights, random fp16 scales and bias)",
        "config": {"workload": "configs[1] fused W8A8 linear, M=N=K=4096, fp16 in/out",
                   "M": M, "N": N, "K": K, "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_INT8_TOPS,
                     "unit": "TOPS", "frac": round(achieved / PEAK_INT8_TOPS, 4), "traffic": measured_traffic(),
                     "mfma_busy": measured_mfma_busy(),
                     "kernel": "gemm_dma_kernel<256,256,dequant>", "kernel_ms": round(t_gemm, 5),
                     "quantize_ms": round(t_q, 5)},
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline()
    if not args.no_extra:
        line["extra"] = {k: round(v, 3) for k, v in bench_extra(dev).items()}
        line["extra"]["reference_sweep"] = bench_reference_sweep(dev)
        line["extra"]["vendor_hipblaslt"] = vendor_gemm_compare(dev)
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
