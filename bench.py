"""Benchmark of the CIGN sparse message-passing layer on one MI355X.

One step = the headline layer of BASELINE.json, forward + backward, with all
inputs resident in HBM:
  * collapsed GAT core (c2: H=4 heads x C=16 channels, fp32) on the
    24,492-node / 186,100-edge Chung-Lu graph + self-loops (E = 210,592):
    cign_gat_fwd (which also writes the per-row aggregates the backward
    streams, as the drop-in autograd function runs it) then cign_gat_bwd
    (rows and columns kernels);
  * 3-hop CSR SpMM pipeline (c3: D=64, fp32) on the normalized adjacency of
    the same graph: cign_spmm_fwd3 then cign_spmm_bwd3 (3 + 3 kernels).
value = E * K / t (edges/s over the timed K steps; each step is one replay
of the step captured as a HIP graph, or with --eager the four drop-in API
calls). The roofline object is computed for the dominant kernel from HIP
events recorded on the launch stream in a second timed region, where each
phase is launched back to back (captured as one graph of 20 launches and
replayed), which is the per-kernel average rocprofv3 reports.
The same run then adds
  * cpu_baseline: the reference's CPU path on the same layer (float32 torch
    on the host's cores, oracle/cpu_path.py), a bounded sample;
  * cpu_baseline_c1 / c1_gpu: BASELINE config 1, the full 2-layer model's
    training step on the host and on the GPU;
  * c3_multihop: BASELINE config 3, the 3-hop SpMM pipeline alone at D = 64,
    256 and 512 in fp32 and bf16 (forward3 + backward3, per-hop GB/s);
  * c2c3_bf16: the headline layer with bf16 features;
  * c4_pack: BASELINE config 4's pack and side ops at N = 24,492, D = 256
    (switch pack K=3 forward + backward against its 351.4 / 552.3 MB byte
    model; dropout-LN, add-LN, dropout-gamma-residual at p = 0.5);
  * scale: the layer at BASELINE config 5 (2.4M nodes, 62.4M edges, GAT 4 x
    32 + SpMM D=256, bf16, eager launches) with its roofline and full-size
    invariants (--no-scale skips it).
Every step time also comes as the median of per-step HIP event pairs
(median_gpu_ms_per_step, BASELINE's method) beside the mean.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--cpu-seconds S] [--eager] [--dtype f32|bf16]
                       [--no-scale] [--workload layer|scale|block|train|c3|c4pack]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E vendor peak, GB/s


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="bounded sample of each CPU baseline, seconds (0 disables)")
    ap.add_argument("--workload", choices=["layer", "scale", "block", "train", "c3", "c4pack", "c2proj"],
                    default="layer",
                    help="layer: the headline c2+c3 layer (24,492 nodes); scale: the same layer at c5 size "
                         "(2.4M nodes, ~62M edges, GAT 4x32 + SpMM D=256, bf16 by default); c3: the 3-hop SpMM "
                         "pipeline alone at D = 64, 256, 512 in fp32 and bf16; c4pack: the Clifford pack and the "
                         "side ops of BASELINE config c4 (N=24,492, D=256, p=0.5); c2proj: the c2 step with its "
                         "300 -> 4x16 projection alone (fp32, or bf16 autocast with --dtype bf16); block: the full "
                         "Clifford block forward+backward at the production shape (D=256, 6 GAT heads, hops 1-3) "
                         "with every component kernel timed against its own roofline (bf16 = selective AMP GEMMs)")
    ap.add_argument("--dtype", choices=["f32", "bf16"], default=None)
    ap.add_argument("--layers", type=int, default=2,
                    help="--workload train: GraphCliffordNet layers (2: BASELINE config c4; 4 with --in-dim 300: the "
                         "Amazon-ratings production model of the reference's published step times)")
    ap.add_argument("--in-dim", type=int, default=256, help="--workload train: input feature width")
    ap.add_argument("--dims", default="64,256,512",
                    help="--workload c3: comma-separated feature widths (with --dtype: that dtype only)")
    ap.add_argument("--headline-only", action="store_true",
                    help="default workload: skip the c3, c2+c3 bf16 and c4 rows that follow the headline layer "
                         "(for profiles of the headline alone)")
    ap.add_argument("--no-scale", action="store_true",
                    help="default workload: skip the c5 measurement that follows the headline c2+c3 layer")
    ap.add_argument("--eager", action="store_true",
                    help="launch every step through the Python drop-in API instead of replaying it as a HIP graph")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="before warmup, run 3 plain 256 MiB elementwise copies (x * 1 -> y, fp32) whose "
                         "FETCH_SIZE / WRITE_SIZE counters calibrate the per-kernel traffic figures")
    return ap.parse_args()


def cpu_baseline(w, seconds: float, H: int, C: int, D: int):
    """The reference's CPU path on the same c2+c3 layer (oracle/cpu_path.py:
    float32 torch, GATConv-style scatter softmax and torch.sparse.mm hops,
    autograd backward) on the host's cores, timed for about `seconds`:
    median step time after 3 warmup steps (backend_autotune_cign.py:228-229)."""
    import torch

    from oracle import cpu_path

    threads = cpu_path.host_threads()
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        (rowptr, col), _, _ = w.gat_graph
        csr, csr_t = w.operator.csr, w.operator.csr_t
        host = lambda c: (c.crow_indices().cpu().numpy(), c.col_indices().cpu().numpy(), c.values().cpu().numpy())
        layer = cpu_path.LayerCPU(rowptr.cpu().numpy(), col.cpu().numpy(), host(csr), host(csr_t), w.n, H, C, D)
        med, k = cpu_path.time_steps(layer.step, seconds)
    finally:
        torch.set_num_threads(prev)
    return {"value": w.nnz_gat / med, "unit": "edges/s", "cores": threads, "kind": "port",
            "ms_per_step": round(1e3 * med, 3),
            "sample": f"median of {k} c2+c3 layer fwd+bwd steps (GAT {H}x{C} + 3 hops D={D}) of the reference's CPU "
                      f"path restated in float32 torch (GATConv scatter softmax, torch.sparse.mm, autograd), "
                      f"{threads} threads"}


def invariants(torch, w, ext, plan, H, C, D, dt):
    """Size-independent checks of the full-size run (no oracle at this size):
    * P = D^-1/2 (A+I) D^-1/2 has x_i = sqrt(deg_i) as a fixed point, so
      forward3 returns (x, x, x) and backward3(0, 0, x) returns x;
    * constant features make every per-head aggregate exactly 1 (the softmax
      weights of a row sum to 1), so pre = 1 + bias, and the attention
      gradients vanish (ge' is constant along a row, so ge' - wsum = 0).
    Returns the worst relative errors."""
    n = w.n
    (rowptr, col), (row, colptr), perm = w.gat_graph
    deg = torch.diff(w.operator.csr.crow_indices()).float()
    xs = deg.sqrt()[:, None].expand(n, D).contiguous().to(dt)
    ref = xs.float()
    ys = plan.forward3(xs)
    zero = torch.zeros_like(xs)
    gx = plan.backward3(zero, zero, xs)
    scale = float(ref.abs().max())
    mh_err = max(float((y.float() - ref).abs().max()) for y in (*ys, gx)) / scale
    ones = torch.ones(n, H, C, device=xs.device, dtype=dt)
    g = torch.Generator(device="cpu").manual_seed(1)
    ar = torch.randn(n, H, generator=g).to(xs.device)
    ac = torch.randn(n, H, generator=g).to(xs.device)
    bias = torch.randn(C, generator=g).to(xs.device)
    gy = torch.randn(n, C, generator=g).to(xs.device).to(dt)
    (out, pre, emax, esum, mask), agg = ext.forward_agg(ar, ac, rowptr, col, 0.2, ones, bias, 0.0, 0, True)
    gat_err = float((pre - (1.0 + bias)[None]).abs().max()) / float((1.0 + bias).abs().max())
    gf, gar, gac, gb = ext.backward(0.2, 0.0, rowptr, col, colptr, row, perm, emax, esum, mask, ones, ar, ac, pre, gy,
                                    agg)
    gscale = float(gf.float().abs().max())
    att_err = max(float(gar.abs().max()), float(gac.abs().max())) / gscale
    torch.cuda.synchronize()
    return {"multihop_fixed_point_rel_err": mh_err, "gat_constant_feature_pre_rel_err": gat_err,
            "gat_constant_feature_attention_grad_rel": att_err}


# ---------------------------------------------------------------------------
# rocprofv3 summaries (profiles/): kernel statistics and copy-calibrated
# FETCH_SIZE / WRITE_SIZE traffic per launch.
# ---------------------------------------------------------------------------
PHASE_KERNELS = {"gat_fwd": ("gat_fwd",), "spmm_fwd3": ("spmm_kernel",), "spmm_bwd3": ("spmm_kernel",),
                 "gat_bwd": ("gat_bwd_rows", "gat_bwd_cols")}
COPY_KIB = 256 * 1024  # the --calibrate-copy kernel reads and writes 256 MiB


def _short(name: str) -> str:
    name = name.removeprefix("void ").replace("(anonymous namespace)::", "")
    return name.split("(")[0] if "(" in name else name


def measured_traffic(name: str, phase: str):
    """HBM bytes per launch of `phase` from the committed rocprofv3 --pmc summary
    profiles/<name>_traffic.json, or (None, None)."""
    path = ROOT / "profiles" / f"{name}_traffic.json"
    if not path.exists():
        return None, None
    d = json.loads(path.read_text())
    total = 0.0
    for key in PHASE_KERNELS[phase]:
        hits = [v for k, v in d["kernels"].items() if key in k]
        if not hits:
            return None, None
        total += hits[0]["bytes"]
    return total, f"profiles/{path.name}"


def summarize(prof_dir: str, name: str, command: str) -> None:
    """Writes profiles/<name>_kernel_stats.txt, _traffic.txt and _traffic.json
    from rocprofv3 CSV output: <prof_dir>/kt (--kernel-trace --stats),
    <prof_dir>/fetch (--pmc FETCH_SIZE) and <prof_dir>/write (--pmc WRITE_SIZE),
    each made with --calibrate-copy for the counter runs (kernel statistics
    only when there are no counter runs)."""
    import csv
    import glob
    import statistics

    prof = Path(prof_dir)
    out = ROOT / "profiles"
    out.mkdir(exist_ok=True)
    stats = list(csv.DictReader(open(glob.glob(str(prof / "kt" / "*_kernel_stats.csv"))[0])))
    lines = [f"# rocprofv3 kernel statistics: {name}", "", "Command (from the repository root, GPU box):", "",
             "    " + command.replace("\n", "\n    "), "",
             f"{'kernel':72s} {'calls':>6s} {'avg_us':>9s} {'min_us':>9s} {'max_us':>9s} {'pct':>6s}"]
    for r in stats[:16]:
        lines.append(f"{_short(r['Name'])[:72]:72s} {int(r['Calls']):6d} {float(r['AverageNs']) / 1e3:9.2f} "
                     f"{float(r['MinNs']) / 1e3:9.2f} {float(r['MaxNs']) / 1e3:9.2f} {float(r['Percentage']):6.2f}")
    (out / f"{name}_kernel_stats.txt").write_text("\n".join(lines) + "\n")
    if (prof / "mfma").exists():
        _summarize_mfma(prof, name, command, {_short(r["Name"]): float(r["AverageNs"]) for r in stats})
    if (prof / "valu").exists():
        _summarize_valu(prof, name, command, {_short(r["Name"]): float(r["AverageNs"]) for r in stats})
    if not (prof / "fetch").exists():
        print(f"wrote profiles/{name}_kernel_stats.txt (no traffic counter runs)")
        return

    def counters(sub, counter):
        per = {}
        f = glob.glob(str(prof / sub / "*_counter_collection.csv"))[0]
        for r in csv.DictReader(open(f)):
            if r["Counter_Name"] == counter:
                per.setdefault(r["Kernel_Name"], []).append(float(r["Counter_Value"]))
        return per

    fetch, write = counters("fetch", "FETCH_SIZE"), counters("write", "WRITE_SIZE")
    # The calibration copy is torch.mul(src, 1.0, out=dst) over 256 MiB: the
    # MulFunctor elementwise kernel whose writes are 256 MiB (other elementwise
    # kernels of the run, e.g. dtype conversions, may move more).
    copy = sorted((k for k in write if "MulFunctor" in k and k in fetch
                   and abs(statistics.median(write[k]) - COPY_KIB) < 0.1 * COPY_KIB),
                  key=lambda k: abs(statistics.median(write[k]) - COPY_KIB))
    if not copy:
        raise SystemExit("no calibration copy kernel in the counter runs (run bench.py with --calibrate-copy)")
    fk = COPY_KIB / statistics.median(fetch[copy[0]])
    wk = COPY_KIB / statistics.median(write[copy[0]])
    kern = {}
    for k in fetch:
        if "cign" not in k:
            continue
        f_kib, w_kib = statistics.median(fetch[k]), statistics.median(write.get(k, [0.0]))
        kern[_short(k)] = {"fetch_kib": f_kib, "write_kib": w_kib, "dispatches": len(fetch[k]),
                           "bytes": round((f_kib * fk + w_kib * wk) * 1024)}
    doc = {"command": command, "calibration": {"copy_kernel": _short(copy[0]), "copy_bytes_each_way": COPY_KIB * 1024,
                                               "fetch_factor": round(fk, 4), "write_factor": round(wk, 4)},
           "kernels": kern}
    (out / f"{name}_traffic.json").write_text(json.dumps(doc, indent=1) + "\n")
    lines = [f"# rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE per dispatch: {name}", "",
             "Command (from the repository root, GPU box):", "", "    " + command.replace("\n", "\n    "), "",
             f"Calibration: {_short(copy[0])} copying 256 MiB reads FETCH_SIZE x {fk:.4f} and WRITE_SIZE x {wk:.4f}",
             "of the true bytes; traffic = FETCH_SIZE * fetch_factor + WRITE_SIZE * write_factor (KiB -> bytes).",
             "", f"{'kernel':60s} {'FETCH KiB':>10s} {'WRITE KiB':>10s} {'traffic MB':>11s}"]
    for k, v in kern.items():
        lines.append(f"{k[:60]:60s} {v['fetch_kib']:10.0f} {v['write_kib']:10.0f} {v['bytes'] / 1e6:11.2f}")
    (out / f"{name}_traffic.txt").write_text("\n".join(lines) + "\n")
    print(f"wrote profiles/{name}_kernel_stats.txt, _traffic.txt, _traffic.json")


def _summarize_valu(prof: Path, name: str, command: str, avg_ns: dict) -> None:
    """profiles/<name>_valu.txt from <prof>/valu (rocprofv3 --pmc
    SQ_INSTS_VALU SQ_INSTS_VMEM_RD VALUBusy): per kernel of this library the
    wavefront VALU and vector-memory-read instructions one dispatch issues
    (median over dispatches) and the VALU busy share (VALUBusy: percent of
    SIMD cycles issuing VALU while the kernel ran)."""
    import csv
    import glob
    import statistics

    per = {}
    f = glob.glob(str(prof / "valu" / "*_counter_collection.csv"))[0]
    for r in csv.DictReader(open(f)):
        if "cign" in r["Kernel_Name"]:
            per.setdefault(_short(r["Kernel_Name"]), {}).setdefault(r["Counter_Name"], []).append(
                float(r["Counter_Value"]))
    lines = [f"# rocprofv3 --pmc SQ_INSTS_VALU SQ_INSTS_VMEM_RD VALUBusy: {name}", "",
             "Command (from the repository root, GPU box):", "", "    " + command.replace("\n", "\n    "), "",
             "Per dispatch (median): wavefront instructions issued; VALUBusy = percent of SIMD cycles issuing VALU;",
             "avg_us from the kernel trace.", "",
             f"{'kernel':64s} {'VALU M':>9s} {'VMEM_RD M':>10s} {'VALUBusy%':>9s} {'avg_us':>9s}"]
    for k, c in sorted(per.items()):
        med = {n: statistics.median(v) for n, v in c.items()}
        lines.append(f"{k[:64]:64s} {med.get('SQ_INSTS_VALU', 0) / 1e6:9.2f} {med.get('SQ_INSTS_VMEM_RD', 0) / 1e6:10.3f} "
                     f"{med.get('VALUBusy', float('nan')):9.1f} {avg_ns.get(k, float('nan')) / 1e3:9.2f}")
    (ROOT / "profiles" / f"{name}_valu.txt").write_text("\n".join(lines) + "\n")
    print(f"wrote profiles/{name}_valu.txt")


MFMA_PEAK = {"f32": 157.3, "bf16": 2500.0}  # MI355X dense matrix TFLOP/s


def _summarize_mfma(prof: Path, name: str, command: str, avg_ns: dict) -> None:
    """profiles/<name>_mfma.txt from <prof>/mfma (rocprofv3 --pmc MfmaUtil
    SQ_INSTS_VALU_MFMA_MOPS_BF16 SQ_INSTS_VALU_MFMA_MOPS_F32): per MFMA kernel
    the matrix-core busy share (MfmaUtil, percent of SIMD cycles while the
    kernel ran), the flops it issued (MOPS x 512) and those flops over the
    kernel's average duration from the kernel trace, against the dense peak
    of its operand type."""
    import csv
    import glob
    import statistics

    per = {}
    f = glob.glob(str(prof / "mfma" / "*_counter_collection.csv"))[0]
    for r in csv.DictReader(open(f)):
        per.setdefault(_short(r["Kernel_Name"]), {}).setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
    lines = [f"# rocprofv3 --pmc MfmaUtil SQ_INSTS_VALU_MFMA_MOPS_BF16 SQ_INSTS_VALU_MFMA_MOPS_F32: {name}", "",
             "Command (from the repository root, GPU box):", "", "    " + command.replace("\n", "\n    "), "",
             "MfmaUtil = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE x SIMDs), percent; flops = MOPS x 512 per",
             "dispatch (median); TFLOP/s = flops / the kernel trace's average duration; peak = dense MI355X",
             "(bf16 2500, fp32 157.3 TFLOP/s).", "",
             f"{'kernel':56s} {'MfmaUtil%':>9s} {'GFLOP':>8s} {'avg_us':>8s} {'TFLOP/s':>8s} {'of peak':>8s}"]
    for k, c in sorted(per.items()):
        bf = statistics.median(c.get("SQ_INSTS_VALU_MFMA_MOPS_BF16", [0.0])) * 512
        f32 = statistics.median(c.get("SQ_INSTS_VALU_MFMA_MOPS_F32", [0.0])) * 512
        if bf + f32 == 0 or k not in avg_ns:
            continue
        util = statistics.median(c.get("MfmaUtil", [float("nan")]))
        tf = (bf + f32) / (avg_ns[k] * 1e-9) / 1e12
        peak = MFMA_PEAK["bf16"] if bf >= f32 else MFMA_PEAK["f32"]
        lines.append(f"{k[:56]:56s} {util:9.1f} {(bf + f32) / 1e9:8.2f} {avg_ns[k] / 1e3:8.2f} {tf:8.1f} "
                     f"{100 * tf / peak:7.1f}%")
    (ROOT / "profiles" / f"{name}_mfma.txt").write_text("\n".join(lines) + "\n")
    print(f"wrote profiles/{name}_mfma.txt")


def time_components(comps: dict, dtype: str, torch):
    """Launches each component R=20 times back to back (one HIP graph,
    replayed M=5 times), timed with HIP events on the launch stream, against
    its roofline: algorithmic bytes / HBM peak, or flops / MFMA peak (the
    bound is whichever ideal time is longer). comps: name -> (callable,
    bytes, flops). Returns (per-kernel records, roofline of the dominant)."""
    ev = lambda: torch.cuda.Event(enable_timing=True)
    R = 20
    kernels = []
    for name, (fn, nbytes, flops) in comps.items():
        fn()
        torch.cuda.synchronize()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            fn()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            for _ in range(R):
                fn()
        gr.replay()
        b0, b1 = ev(), ev()
        torch.cuda.synchronize()
        b0.record()
        M = 5
        for _ in range(M):
            gr.replay()
        b1.record()
        torch.cuda.synchronize()
        ms = b0.elapsed_time(b1) / (M * R)
        gbs = nbytes / (ms * 1e-3) / 1e9
        rec = {"kernel": name, "avg_launch_ms": round(ms, 5), "bytes_per_launch": int(nbytes),
               "GB_s": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
        if flops:
            tfs = flops / (ms * 1e-3) / 1e12
            peak = MFMA_PEAK[dtype]
            rec.update({"flops_per_launch": int(flops), "TFLOP_s": round(tfs, 2), "mfma_frac": round(tfs / peak, 4)})
            # the bound is whichever roofline the ideal time hits first
            rec["bound"] = "mfma" if flops / (peak * 1e12) > nbytes / (HBM_PEAK_GBS * 1e9) else "hbm"
        else:
            rec["bound"] = "hbm"
        kernels.append(rec)
        del gr

    dom = max(kernels, key=lambda r: r["avg_launch_ms"])
    if dom["bound"] == "mfma":
        roof = {"bound": "mfma", "kernel": dom["kernel"], "achieved": dom["TFLOP_s"], "peak": MFMA_PEAK[dtype],
                "unit": "TFLOP/s", "frac": dom["mfma_frac"], "traffic": None,
                "avg_launch_ms": dom["avg_launch_ms"], "flops_per_launch": dom["flops_per_launch"]}
    else:
        roof = {"bound": "hbm", "kernel": dom["kernel"], "achieved": dom["GB_s"], "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": dom["hbm_frac"], "traffic": None, "avg_launch_ms": dom["avg_launch_ms"],
                "bytes_per_launch": dom["bytes_per_launch"]}
    return kernels, roof


def cpu_train_baseline(seconds: float, torch):
    """The reference's CPU case (BASELINE config c1): the full CIGN model
    forward + cross-entropy + backward + Adam step, restated in float32 torch
    on the host (oracle/block_oracle.net_forward: the torch/PyG fallback path
    of the reference, eval-mode numerics), on N=2000 nodes with out-degree 8
    uniform-random edges (symmetrised, as the reference's default
    use_undirected) plus self-loops, 64-dim features, 2 layers, 4 heads x 64,
    hops (1, 2), 5 classes, seed 0. Median step time over about `seconds`
    with the host's cores (oracle.cpu_path.host_threads)."""
    import numpy as np

    from cign_amd import workloads
    from oracle import block_oracle as B
    from oracle import cpu_path

    d, hidden, heads, classes = 64, 64, 4, 5
    w = workloads.build(workloads.C1, device="cpu")
    n = w.n
    (rowptr, col), _, _ = w.gat_graph
    rp, cl = rowptr.numpy().astype(np.int64), col.numpy().astype(np.int64)
    Pc = w.operator.csr
    p_np = (Pc.crow_indices().numpy(), Pc.col_indices().numpy(), Pc.values().double().numpy())
    g = torch.Generator().manual_seed(0)
    t = lambda *s: (torch.randn(*s, generator=g) * 0.1).requires_grad_()
    params = {"input_proj_0.weight": t(hidden, d), "input_proj_0.bias": t(hidden), "input_proj_1.weight": t(hidden, d),
              "input_proj_1.bias": t(hidden), "input_eta": torch.tensor(0.1, requires_grad=True),
              "output_norm.weight": t(3 * hidden), "output_norm.bias": t(3 * hidden),
              "classifier.weight": t(classes, 3 * hidden), "classifier.bias": t(classes)}
    for i in range(2):
        for k, shape in {"h_norm.weight": (hidden,), "h_norm.bias": (hidden,), "c_norm.weight": (hidden,),
                         "c_norm.bias": (hidden,), "context_gat.lin.weight": (heads * hidden, hidden),
                         "context_gat.att_src": (1, heads, hidden), "context_gat.att_dst": (1, heads, hidden),
                         "context_gat.bias": (hidden,), "proj.weight": (hidden, 4 * hidden), "proj.bias": (hidden,),
                         "hop_gate_mlp.weight": (2, 2 * hidden), "hop_gate_mlp.bias": (2,), "gamma": (hidden,)}.items():
            params[f"blocks.{i}.{k}"] = t(*shape)
    x = torch.randn(n, d, generator=g)
    y = torch.randint(0, classes, (n,), generator=g)
    mask = torch.rand(n, generator=g) < 0.5
    opt = torch.optim.Adam(list(params.values()), lr=3e-3, weight_decay=1e-5)

    def step():
        opt.zero_grad()
        logits = B.net_forward(params, x, rp, cl, p_np, (1, 2), num_layers=2, dual=True, layer_combine="concat",
                               score_mode=1, interaction=1, weighting=0, gate_mode="node", heads=heads)
        torch.nn.functional.cross_entropy(logits[mask], y[mask]).backward()
        opt.step()

    threads = cpu_path.host_threads()
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        med, k = cpu_path.time_steps(step, seconds)
    finally:
        torch.set_num_threads(prev)
    return {"value": int(col.numel()) / med, "unit": "edges/s", "cores": threads, "kind": "port",
            "ms_per_step": round(1e3 * med, 3),
            "sample": f"median of {k} c1 training steps (N=2000, E_nnz={int(col.numel())}, in 64, hidden 64, 2 layers, "
                      f"4 heads, hops 1-2; float32 torch restatement of the reference's CPU path + Adam), "
                      f"{threads} threads"}


def make_train_step(torch, w, in_dim, hidden, heads, layers, order_set, amp, dev):
    """One training step of GraphCliffordNet (zero_grad, forward,
    cross-entropy over a 50% train mask, backward, Adam lr 3e-3 / weight
    decay 1e-5) on workload w, as generic_engine/train_cign.py:2103-2148
    times it; returns the step callable (it returns the loss)."""
    import torch.nn.functional as F

    from cign_amd.model_cign import GraphCliffordNet
    from cign_amd.multihop_csr_pipeline import prepare_multihop_csr_operator

    torch.manual_seed(0)
    model = GraphCliffordNet(in_dim, hidden, 5, num_layers=layers, order_set=order_set, gat_heads=heads,
                             use_selective_amp=amp).to(dev).train()
    model._fused_gat_graph = w.gat_graph
    # the operator the reference's driver prepares for these hops
    mh = prepare_multihop_csr_operator(w.operator, dense_cols=2 * hidden, powers=order_set)
    g = torch.Generator(device="cpu").manual_seed(0)
    x = torch.randn(w.n, in_dim, generator=g).to(dev)
    y = torch.randint(0, 5, (w.n,), generator=g).to(dev)
    mask = (torch.rand(w.n, generator=g) < 0.5).to(dev)
    opt = torch.optim.Adam(model.parameters(), lr=3e-3, weight_decay=1e-5)

    def step():
        opt.zero_grad()
        logits = model(x, None, mh)
        loss = F.cross_entropy(logits[mask], y[mask])
        loss.backward()
        opt.step()
        return loss

    return step


def time_train(torch, step, steps, warmup):
    """(wall seconds of `steps` steps, GPU ms per step) after `warmup` steps."""
    for _ in range(max(1, warmup)):
        loss = step()
    torch.cuda.synchronize()
    if not torch.isfinite(loss):
        raise SystemExit("non-finite training loss")
    a0, a1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    a0.record()
    for _ in range(steps):
        step()
    a1.record()
    torch.cuda.synchronize()
    return time.perf_counter() - t0, a0.elapsed_time(a1) / steps


def c1_gpu(torch, dev, steps=20):
    """The reference's CPU case c1 (N=2000, 64-dim, 4 heads x 64, hops 1-2,
    2 layers) as a training step on the GPU, fp32."""
    from cign_amd import workloads

    w1 = workloads.build(workloads.C1, device=dev)
    e1, gms = time_train(torch, make_train_step(torch, w1, 64, 64, 4, 2, (1, 2), False, dev), steps, 3)
    return {"ms_per_step": round(1e3 * e1 / steps, 4), "gpu_ms_per_step": round(gms, 4), "edges_nnz": w1.nnz_gat,
            "edges_per_s": w1.nnz_gat * steps / e1}


def run_train(args, torch):
    """A full 2-layer CIGN training step (BASELINE config c4, second half):
    GraphCliffordNet(in 256, hidden 256, 5 classes, 2 layers, 6 GAT heads x
    256, hops 1-3, default dropouts, selective bf16 AMP unless --dtype f32)
    on the c2 graph; one step = zero_grad -> forward -> cross-entropy over a
    50% train mask -> backward -> Adam (lr 3e-3, weight decay 1e-5), as
    generic_engine/train_cign.py:2103-2148 times it. value = GAT edges (with
    self-loops) per second of training. The CPU baseline is the reference's
    own CPU case c1 (cpu_train_baseline); the same model at c1 is also timed
    on the GPU for a like-for-like ratio."""
    from cign_amd import workloads

    dev = torch.device("cuda:0")
    amp = args.dtype != "f32"

    w = workloads.build(workloads.C2, device=dev)
    L, ind = int(args.layers), int(args.in_dim)
    elapsed, gpu_ms = time_train(torch, make_train_step(torch, w, ind, 256, 6, L, (1, 2, 3), amp, dev), args.steps,
                                 args.warmup)
    # The reference's CPU case on the GPU (c1: N=2000, 64-dim, 4 heads, hops 1-2).
    c1 = c1_gpu(torch, dev)
    cpu = cpu_train_baseline(args.cpu_seconds, torch) if args.cpu_seconds > 0 else None
    line = {
        "metric": f"CIGN {L}-layer training step edges/sec (zero_grad, forward, cross-entropy, backward, Adam)",
        "value": w.nnz_gat * args.steps / elapsed,
        "unit": "edges/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": 1e3 * elapsed / args.steps,
        "gpu_ms_per_step": round(gpu_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16-gemm" if amp else "f32",
        "data": "synthetic: seeded Chung-Lu power-law graph (gamma 2.5), N(0,1) features, uniform 5-class labels, "
                "random-init model",
        "config": {"workload": f"{'c4 ' if (L, ind) == (2, 256) else ''}training step: GraphCliffordNet in {ind}, "
                               f"hidden 256, {L} layers, 6 GAT heads x 256, hops 1-3, dropout 0.28 / GAT 0.32, "
                               "concat, Adam",
                   "nodes": w.n, "edges_nnz": w.nnz_gat},
        "c1_gpu": c1,
        "roofline": None,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def run_block(args, torch):
    """The Clifford block of the reference at its production shape on the c2
    graph: GraphCliffordBlock(D=256, gat_heads=6, hops (1,2,3), interaction
    new, weighting old, node hop gate), training mode (dropout 0.28 / GAT
    0.32), forward + backward. One step = one block forward+backward; value =
    edges/s. Then each component's kernels are launched back to back (HIP
    graph of 20 launches) and timed with HIP events against their own
    roofline: algorithmic bytes / HBM peak, or flops / MFMA peak for the
    projections (the lower of the two bounds)."""
    from cign_amd import _lib, workloads
    from cign_amd.model_cign import GraphCliffordBlock
    from cign_amd.multihop_csr_pipeline import MultiHopCSR3GraphOperator

    dev = torch.device("cuda:0")
    amp = args.dtype == "bf16"
    lib = _lib.load_library()
    D, heads, K = 256, 6, 3
    w = workloads.build(workloads.C2, device=dev)
    n, E = w.n, w.nnz_gat
    mh = MultiHopCSR3GraphOperator(w.operator, dense_cols=2 * D)
    torch.manual_seed(0)
    block = GraphCliffordBlock(D, order_set=(1, 2, 3), gat_heads=heads, use_selective_amp=amp,
                               alpha_score_mode="new", interaction_mode="new", alpha_weighting_mode="old",
                               hop_gate_mode="node").to(dev).train()
    g = torch.Generator(device="cpu").manual_seed(0)
    H0 = torch.randn(n, D, generator=g).to(dev).requires_grad_(True)
    G0 = torch.randn(n, D, generator=g).to(dev)

    params = list(block.parameters())

    def step():
        # gradients produced, not accumulated across steps (zero_grad with
        # set_to_none, as the training loop does before each backward)
        for prm in params:
            prm.grad = None
        H0.grad = None
        out = block(H0, None, mh, w.gat_graph)
        out.backward(G0)

    for _ in range(max(1, args.warmup)):
        step()
    torch.cuda.synchronize()
    ev = lambda: torch.cuda.Event(enable_timing=True)
    a0, a1 = ev(), ev()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    a0.record()
    for _ in range(args.steps):
        step()
    a1.record()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    gpu_ms = a0.elapsed_time(a1) / args.steps

    # ---- components -------------------------------------------------------
    st = lambda: _lib.stream_ptr(dev)
    rnd = lambda *s: torch.randn(*s, generator=g).to(dev)
    x, hh, cc = rnd(n, D), rnd(n, D), rnd(n, D)
    lnw, lnb = rnd(D), rnd(D)
    y, y2 = torch.empty(n, D, device=dev), torch.empty(n, D, device=dev)
    mean, rstd = torch.empty(n, device=dev), torch.empty(n, device=dev)
    mask = torch.empty(n, D, dtype=torch.uint8, device=dev)
    gw_, gb_ = torch.empty(D, device=dev), torch.empty(D, device=dev)
    ws = torch.empty(int(lib.cign_colsum_workspace_bytes(n, D, 2)) + 256, dtype=torch.uint8, device=dev)
    props = [rnd(n, 2 * D) for _ in range(K)]
    alpha = torch.softmax(rnd(n, K), 1).contiguous()
    gate_w, gate_b = rnd(K, 2 * D) * 0.05, rnd(K)
    gate_ws = torch.empty(int(lib.cign_hop_gate_bwd_workspace_bytes(n, D, K)) + 256, dtype=torch.uint8, device=dev)
    gH_, gC_ = torch.empty(n, D, device=dev), torch.empty(n, D, device=dev)
    gwt, gbt = torch.empty(K, 2 * D, device=dev), torch.empty(K, device=dev)
    gout = rnd(n, 2 * K * D)
    gprops = [torch.empty(n, 2 * D, device=dev) for _ in range(K)]
    parr = _lib.ptr_array([p.data_ptr() for p in props])
    gparr = _lib.ptr_array([p.data_ptr() for p in gprops])
    Wp, bp = rnd(D, 2 * K * D) * 0.02, rnd(D)
    Wl = rnd(heads * D, D) * 0.05
    gp_out, yp = torch.empty(n, D, device=dev), torch.empty(n, D, device=dev)
    xl = torch.empty(n, heads * D, device=dev)
    lin_ws = torch.empty(int(lib.cign_linear_bwd_workspace_bytes(n, D, 2 * K * D, 1)), dtype=torch.uint8, device=dev)
    gxp, gWp, gbp = torch.empty(n, 2 * K * D, device=dev), torch.empty(D, 2 * K * D, device=dev), torch.empty(D, device=dev)
    math = 1 if amp else 0
    galpha = torch.empty(n, K, device=dev)
    pp_ws = torch.empty(int(lib.cign_pack_proj_bwd_workspace_bytes(n, D, K)), dtype=torch.uint8, device=dev)
    pf_ws = torch.empty(max(1, int(lib.cign_pack_proj_fwd_workspace_bytes(D, K, math))), dtype=torch.uint8,
                        device=dev)
    s4 = 4
    NDb = n * D
    comps = {
        # name: (callable, bytes, flops)
        "dropout_ln_fwd": (lambda: lib.call("cign_dropout_ln_fwd", st(), n, D, x.data_ptr(), lnw.data_ptr(),
                                            lnb.data_ptr(), 0.28, 1e-5, 7, y.data_ptr(), mean.data_ptr(),
                                            rstd.data_ptr(), mask.data_ptr()), 9 * NDb + 8 * n, 0),
        "dropout_ln_bwd": (lambda: lib.call("cign_dropout_ln_bwd", st(), n, D, hh.data_ptr(), x.data_ptr(),
                                            lnw.data_ptr(), mean.data_ptr(), rstd.data_ptr(), mask.data_ptr(),
                                            0.28, y2.data_ptr(), gw_.data_ptr(), gb_.data_ptr(), ws.data_ptr(),
                                            ws.numel()), 13 * NDb + 8 * n, 0),
        "add_ln_fwd": (lambda: lib.call("cign_add_ln_fwd", st(), n, D, x.data_ptr(), hh.data_ptr(), lnw.data_ptr(),
                                        lnb.data_ptr(), 1e-5, y.data_ptr(), mean.data_ptr(), rstd.data_ptr()),
                       12 * NDb + 8 * n, 0),
        "add_ln_bwd": (lambda: lib.call("cign_add_ln_bwd", st(), n, D, cc.data_ptr(), x.data_ptr(), hh.data_ptr(),
                                        lnw.data_ptr(), mean.data_ptr(), rstd.data_ptr(), y2.data_ptr(),
                                        gw_.data_ptr(), gb_.data_ptr(), ws.data_ptr(), ws.numel()),
                       16 * NDb + 8 * n, 0),
        # the node hop gate fused into the pack, as the block runs them
        "pack_gate_fwd": (lambda: lib.call("cign_pack_gate_fwd", st(), n, D, K, 1, 0, 1, hh.data_ptr(), cc.data_ptr(),
                                           ctypes.addressof(parr), 2 * D, gate_w.data_ptr(), gate_b.data_ptr(),
                                           alpha.data_ptr(), gout.data_ptr()),
                          8 * NDb + 16 * K * NDb + 4 * n * K, 0),
        "pack_gate_bwd": (lambda: lib.call("cign_pack_gate_bwd", st(), n, D, K, 1, 0, 1, gout.data_ptr(),
                                           hh.data_ptr(), cc.data_ptr(), ctypes.addressof(parr), 2 * D,
                                           alpha.data_ptr(), gate_w.data_ptr(), gH_.data_ptr(), gC_.data_ptr(),
                                           ctypes.addressof(gparr), 2 * D, gwt.data_ptr(), gbt.data_ptr(),
                                           gate_ws.data_ptr(), gate_ws.numel()),
                          24 * K * NDb + 16 * NDb + 8 * n * K, 0),
        "proj_gamma_fwd": (lambda: lib.call("cign_linear_gamma_fwd", st(), n, D, 2 * K * D, 0, math, gout.data_ptr(),
                                            Wp.data_ptr(), bp.data_ptr(), hh.data_ptr(), lnw.data_ptr(), 0.28, 9,
                                            gp_out.data_ptr(), yp.data_ptr(), mask.data_ptr()),
                           s4 * n * 2 * K * D + 13 * NDb, 2 * n * 2 * K * D * D),
        "proj_bwd": (lambda: lib.call("cign_linear_bwd", st(), n, D, 2 * K * D, math, hh.data_ptr(), gout.data_ptr(),
                                      Wp.data_ptr(), gxp.data_ptr(), gWp.data_ptr(), gbp.data_ptr(),
                                      lin_ws.data_ptr(), lin_ws.numel()),
                     2 * s4 * n * 2 * K * D + 2 * 4 * NDb, 4 * n * 2 * K * D * D),
        # the pack built inside proj (the block's tail as it runs): G_raw never stored
        "pack_proj_fwd": (lambda: lib.call("cign_pack_proj_fwd", st(), n, D, K, 1, math, hh.data_ptr(),
                                           cc.data_ptr(), ctypes.addressof(parr), 2 * D, alpha.data_ptr(), K,
                                           Wp.data_ptr(), bp.data_ptr(), x.data_ptr(), lnw.data_ptr(), 0.28, 9,
                                           gp_out.data_ptr(), yp.data_ptr(), mask.data_ptr(),
                                           pf_ws.data_ptr(), pf_ws.numel()),
                          (21 + 8 * K) * NDb + 4 * n * K, 2 * n * 2 * K * D * D),
        "pack_proj_bwd": (lambda: lib.call("cign_pack_proj_bwd", st(), n, D, K, 1, math, x.data_ptr(),
                                           hh.data_ptr(), cc.data_ptr(), ctypes.addressof(parr), 2 * D,
                                           alpha.data_ptr(), K, Wp.data_ptr(), 1, gate_w.data_ptr(),
                                           gH_.data_ptr(), gC_.data_ptr(), ctypes.addressof(gparr), 2 * D,
                                           galpha.data_ptr(), gWp.data_ptr(), gbp.data_ptr(), gwt.data_ptr(),
                                           gbt.data_ptr(), pp_ws.data_ptr(), pp_ws.numel()),
                          (20 + 16 * K) * NDb + 8 * n * K, 4 * n * 2 * K * D * D),
    }
    # The GAT lin: under AMP its bf16 output is held in bf16 (lin_gat), as the
    # block runs it; fp32 otherwise.
    if amp:
        xl16 = torch.empty(n, heads * D, dtype=torch.bfloat16, device=dev)
        comps["gat_lin_fwd"] = (lambda: lib.call("cign_linear_fwd_bf16y", st(), n, heads * D, D, 0, x.data_ptr(),
                                                 Wl.data_ptr(), None, xl16.data_ptr()),
                                4 * NDb + 2 * n * heads * D, 2 * n * D * heads * D)
    else:
        comps["gat_lin_fwd"] = (lambda: lib.call("cign_linear_fwd", st(), n, heads * D, D, 0, math, x.data_ptr(),
                                                 Wl.data_ptr(), None, xl.data_ptr()),
                                4 * NDb + 4 * n * heads * D, 2 * n * D * heads * D)
    # The block's collapsed GAT (H=6 x C=256; under AMP on the bf16-held
    # projection output with fp32 outputs and gradients, as lin_gat runs it)
    # and one hop of its multihop SpMM (D = 2 x 256), as the block runs them.
    from cign_amd.collapsed_gat import ensure_collapsed_gat_loaded

    ext = ensure_collapsed_gat_loaded()
    (rowptr, col), (row_, colptr), perm = w.gat_graph
    xg = rnd(n, heads, D)
    if amp:
        xg = xg.to(torch.bfloat16)
    ar_, ac_, bg_ = rnd(n, heads) * 0.1, rnd(n, heads) * 0.1, rnd(D)
    gyg = rnd(n, D)
    gat_state = {}

    # the per-row aggregates exactly when lin_gat keeps them
    from cign_amd.lin_gat import _GATHER_MAX_DEGREE

    want_agg = not (amp and E <= _GATHER_MAX_DEGREE * n)

    def gat_fwd():
        gat_state["f"] = ext.forward_agg(ar_, ac_, rowptr, col, 0.2, xg, bg_, 0.32, 5, want_agg, f32_out=amp)

    def gat_bwd():
        (_, pre_, em_, es_, mk_), agg_ = gat_state["f"]
        ext.backward(0.2, 0.32, rowptr, col, colptr, row_, perm, em_, es_, mk_, xg, ar_, ac_, pre_, gyg, agg_,
                     f32_out=amp)

    gat_fwd()
    Bg = workloads.algorithmic_bytes(n, E, heads, D, 2 * D, s_gat=2 if amp else 4, dropout=True)
    sfx = "_agg" if want_agg else ""
    if amp:
        Bg["gat_bwd" + sfx] += 2 * n * heads * D  # grad_feat is written as fp32
    Xs = rnd(n, 2 * D)
    comps["gat_fwd"] = (gat_fwd, Bg["gat_fwd" + sfx], 0)
    comps["gat_bwd"] = (gat_bwd, Bg["gat_bwd" + sfx], 0)
    from cign_amd.multihop_csr_pipeline import _csr_mm

    comps["spmm_hop"] = (lambda: _csr_mm(w.operator.csr, Xs), Bg["spmm"], 0)
    kernels, roof = time_components(comps, args.dtype, torch)
    line = {
        "metric": "Clifford block fwd+bwd edges/sec (production shape); per-kernel roofline fractions",
        "value": E * args.steps / elapsed,
        "unit": "edges/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": 1e3 * elapsed / args.steps,
        "gpu_ms_per_step": round(gpu_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16-gemm" if amp else "f32",
        "data": "synthetic: seeded Chung-Lu power-law graph (gamma 2.5), N(0,1) features, random-init block",
        "config": {"workload": "Clifford block (c4/prod): D=256, 6 GAT heads x 256, hops 1-3, interaction new, "
                               "weighting old, node hop gate, training mode, forward+backward",
                   "nodes": n, "edges_nnz": E},
        "kernels": kernels,
        "roofline": roof,
        "cpu_baseline": None,
    }
    print(json.dumps(line), flush=True)


def main():
    if len(sys.argv) > 1 and sys.argv[1] == "--summarize":
        # python bench.py --summarize <rocprof dir> <name> <command text>
        summarize(sys.argv[2], sys.argv[3], sys.argv[4])
        return
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only; --gpus must be 1 (the path would shard by "
                                   "destination rows with halo exchange; that is designed, not run)"}), flush=True)
        sys.exit(2)
    import torch

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.workload == "block":
        if args.dtype is None:
            args.dtype = "f32"
        run_block(args, torch)
        return
    if args.workload == "train":
        if args.dtype is None:
            args.dtype = "bf16"
        run_train(args, torch)
        return
    if args.workload in ("c3", "c4pack", "c2proj"):
        from cign_amd import workloads

        if args.calibrate_copy:
            calibration_copy(torch, dev)
        if args.workload == "c2proj":
            res = {"c2_with_projection": measure_c2proj(torch, args.dtype or "f32", args.steps, args.warmup)}
        elif args.workload == "c3":
            w = workloads.build(workloads.C2, device=dev)
            dts = (args.dtype,) if args.dtype else ("f32", "bf16")
            res = {"c3_multihop": [measure_multihop(torch, w, int(D), dt) for D in args.dims.split(",") for dt in dts]}
        else:
            res = {"c4_pack": measure_c4_pack(torch)}
        print(json.dumps(res), flush=True)
        return
    layer_only = args.workload == "scale"
    if layer_only:
        line, _ = measure_layer(torch, True, args.dtype or "bf16", args.steps, args.warmup, args.eager,
                                args.calibrate_copy)
        print(json.dumps(line), flush=True)
        return
    line, w = measure_layer(torch, False, args.dtype or "f32", args.steps, args.warmup, args.eager,
                            args.calibrate_copy)
    print(f"c2+c3 layer: {line['ms_per_step']:.4f} ms/step", file=sys.stderr, flush=True)
    # The GPU c1 step is launch-bound host code: time it before the CPU
    # baselines leave their worker threads spinning.
    line["c1_gpu"] = c1_gpu(torch, torch.device("cuda:0"))
    if args.cpu_seconds > 0:
        line["cpu_baseline"] = cpu_baseline(w, args.cpu_seconds, 4, 16, 64)
        print("cpu baseline done", file=sys.stderr, flush=True)
        line["cpu_baseline_c1"] = cpu_train_baseline(args.cpu_seconds, torch)
        print("c1 model step on the host done", file=sys.stderr, flush=True)
    else:
        line["cpu_baseline"] = None
    # The other BASELINE rows in the same run: c3 (the SpMM pipeline alone at
    # D = 64, 256, 512, fp32 and bf16), the c2+c3 layer in bf16, and the c4
    # pack + side ops.
    if not args.headline_only:
        line["c3_multihop"] = [measure_multihop(torch, w, D, dt) for D in (64, 256, 512)
                               for dt in ("f32", "bf16")]
        print("c3 done", file=sys.stderr, flush=True)
    del w
    if not args.headline_only:
        lb, _ = measure_layer(torch, False, "bf16", args.steps, args.warmup, args.eager)
        line["c2c3_bf16"] = {k: lb[k] for k in ("value", "unit", "ms_per_step", "median_gpu_ms_per_step", "dtype",
                                               "layer_GB_s", "layer_roofline_frac", "algorithmic_bytes_per_step",
                                               "layer_own_roofline_frac", "breakdown", "roofline") if k in lb}
        if "c2_with_projection" in lb:
            line["c2c3_bf16"]["c2_with_projection"] = lb["c2_with_projection"]
        line["c4_pack"] = measure_c4_pack(torch)
        print("c2+c3 bf16 and c4 pack done", file=sys.stderr, flush=True)
    if not args.no_scale:
        # BASELINE config 5 in the same run: the layer at 2.4M nodes / 62.4M
        # edges (bf16, 4 x 32 heads, D = 256), the true HBM-bound case.
        sc, _ = measure_layer(torch, True, "bf16", max(3, min(args.steps, 20)), 2)
        line["scale"] = {k: sc[k] for k in ("value", "unit", "ms_per_step", "gpu_ms_per_step",
                                           "median_gpu_ms_per_step", "dtype", "config",
                                           "layer_GB_s", "layer_roofline_frac", "algorithmic_bytes_per_step",
                                           "layer_own_roofline_frac", "breakdown", "roofline", "invariants")}
        line["scale"]["steps"] = max(3, min(args.steps, 20))
    print(json.dumps(line), flush=True)


def calibration_copy(torch, dev):
    """Three plain 256 MiB elementwise copies (x * 1 -> y, fp32) whose
    FETCH_SIZE / WRITE_SIZE counters calibrate the per-kernel traffic."""
    src = torch.ones(64 << 20, dtype=torch.float32, device=dev)  # 256 MiB
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.mul(src, 1.0, out=dst)
    torch.cuda.synchronize()
    del src, dst


def measure_layer(torch, scale: bool, dtype: str, steps: int, warmup: int, eager: bool = False,
                  calibrate_copy: bool = False):
    """The layer step (collapsed GAT + 3-hop SpMM, forward + backward) at c2+c3
    (scale False: H=4 x C=16, D=64) or c5 (scale True: H=4 x C=32, D=256,
    eager launches, full-size invariants), timed over `steps` steps after
    `warmup`, with the per-phase roofline. Returns (JSON line without CPU
    baselines, workload)."""
    from cign_amd import workloads
    from cign_amd.collapsed_gat import ensure_collapsed_gat_loaded
    from cign_amd.multihop_csr_pipeline import MultiHopCSR3GraphOperator

    dev = torch.device("cuda:0")
    H, C, D = (4, 32, 256) if scale else (4, 16, 64)
    dt = torch.float32 if dtype == "f32" else torch.bfloat16
    # Captured graphs would keep one output set per captured launch; at c5
    # the GPU is the bottleneck, so its launches stay eager.
    eager = eager or scale
    t_build = time.perf_counter()
    if scale:
        print("building the c5 graph on the host (under a minute)...", file=sys.stderr, flush=True)
    w = workloads.build(workloads.C5 if scale else workloads.C2, device=dev)
    if scale:
        print(f"graph built in {time.perf_counter() - t_build:.0f} s", file=sys.stderr, flush=True)
    (rowptr, col), (row, colptr), perm = w.gat_graph
    n, E = w.n, w.nnz_gat
    g = torch.Generator(device="cpu").manual_seed(0)
    rnd = lambda *s: torch.randn(*s, generator=g).to(dev)
    x = rnd(n, H, C).to(dt)
    ar, ac, bias = rnd(n, H), rnd(n, H), rnd(C)
    gy = rnd(n, C).to(dt)
    X = rnd(n, D).to(dt)
    g1, g2, g3 = rnd(n, D).to(dt), rnd(n, D).to(dt), rnd(n, D).to(dt)
    ext = ensure_collapsed_gat_loaded()
    mh = MultiHopCSR3GraphOperator(w.operator, dense_cols=D, dense_dtype=dt)
    plan = mh.plan

    ev = lambda: torch.cuda.Event(enable_timing=True)
    phases = ("gat_fwd", "spmm_fwd3", "gat_bwd", "spmm_bwd3")
    fwd_out = {}

    def run_phase(p):
        # The GAT runs as the drop-in autograd function does: the forward
        # also writes the per-row aggregates its backward streams.
        if p == "gat_fwd":
            outs, agg = ext.forward_agg(ar, ac, rowptr, col, 0.2, x, bias, 0.0, 0, True)
            fwd_out["gat"] = outs + ([agg] if agg is not None else [])
        elif p == "spmm_fwd3":
            fwd_out["mh"] = plan.forward3(X)
        elif p == "gat_bwd":
            out, pre, emax, esum, mask = fwd_out["gat"][:5]
            agg = fwd_out["gat"][5] if len(fwd_out["gat"]) > 5 else None
            fwd_out["gat_bwd"] = ext.backward(0.2, 0.0, rowptr, col, colptr, row, perm, emax, esum, mask, x, ar,
                                              ac, pre, gy, agg)
        else:
            fwd_out["mh_bwd"] = [plan.backward3(g1, g2, g3)]

    if calibrate_copy:
        calibration_copy(torch, dev)

    # Eager warmup: builds the row schedules (one host copy of each row
    # pointer) and the workspaces, and gives the reference outputs.
    for _ in range(max(1, warmup)):
        for p in phases:
            run_phase(p)
    torch.cuda.synchronize()

    def capture(fn):
        """HIP graph of fn() (allocations settle in a side-stream run first)."""
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            fn()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            fn()
        return g

    def whole_step():
        for p in phases:
            run_phase(p)

    if eager:
        launch_step = whole_step
    else:
        eager_out = {k: [t.clone() for t in v] for k, v in fwd_out.items()}
        # The step as one HIP graph: its host work is one launch, and every
        # replay recomputes every kernel of the four phases.
        launch_step = capture(whole_step).replay
        for _ in range(max(1, warmup)):
            launch_step()
        torch.cuda.synchronize()
        # Replays reproduce the eager results bit for bit (the GAT forward's
        # edge_mask, output 4, is only written when attn_drop > 0).
        for k, v in fwd_out.items():
            for i, (a_, b_) in enumerate(zip(v, eager_out[k])):
                if not (k == "gat" and i == 4) and not torch.equal(a_, b_):
                    raise SystemExit(f"graph replay of {k}[{i}] differs from the eager result")

    # Timed region: K steps, synchronised on both sides.
    start, stop = ev(), ev()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record()
    for _ in range(steps):
        launch_step()
    stop.record()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    gpu_step_ms = start.elapsed_time(stop) / steps
    # The median step (BASELINE's method: a HIP event pair around each of
    # the K steps), in a second pass after the timed region.
    import statistics

    evs = [(ev(), ev()) for _ in range(steps)]
    for a_, b_ in evs:
        a_.record()
        launch_step()
        b_.record()
    torch.cuda.synchronize()
    median_step_ms = statistics.median(a_.elapsed_time(b_) for a_, b_ in evs)

    # Per-phase kernel durations: each phase launched R times back to back
    # (one HIP graph, or R drop-in calls with --eager) and timed with HIP
    # events on the launch stream.
    R, M = (1, max(2, steps)) if scale else (20, max(2, steps // 10))
    phase_ms = {}
    for p in phases:
        if eager:
            rep = lambda p=p: [run_phase(p) for _ in range(R)]
        else:
            gp = capture(lambda p=p: [run_phase(p) for _ in range(R)])
            rep = gp.replay
        rep()
        a0, a1 = ev(), ev()
        torch.cuda.synchronize()
        a0.record()
        for _ in range(M):
            rep()
        a1.record()
        torch.cuda.synchronize()
        phase_ms[p] = a0.elapsed_time(a1) / (M * R)

    s = 2 if dt == torch.bfloat16 else 4
    B = workloads.algorithmic_bytes(n, E, H, C, D, s_gat=s, s_mh=s)
    ms = 1e3 * elapsed / steps
    # One "launch" of the GAT backward is one cign_gat_bwd call (its rows and
    # columns kernels back to back on the stream).
    launches = {"gat_fwd": 1, "spmm_fwd3": 3, "gat_bwd": 1, "spmm_bwd3": 3}
    agg_path = len(fwd_out["gat"]) > 5
    gkey = "_agg" if agg_path else ""
    bytes_per_launch = {"gat_fwd": B["gat_fwd" + gkey], "spmm_fwd3": B["spmm"], "gat_bwd": B["gat_bwd" + gkey],
                        "spmm_bwd3": B["spmm"] + s * n * D * 2 / 3}
    breakdown = {}
    for p in phases:
        per_launch_ms = phase_ms[p] / launches[p]
        gbs = bytes_per_launch[p] / (per_launch_ms * 1e-3) / 1e9
        breakdown[p] = {"ms": round(phase_ms[p], 4), "launches": launches[p], "GB_s": round(gbs, 1)}
    dom = max(phases, key=lambda p: phase_ms[p])
    dom_ms = phase_ms[dom] / launches[dom]
    achieved = bytes_per_launch[dom] / (dom_ms * 1e-3) / 1e9
    kernel_name = {"gat_fwd": "cign_gat_fwd (gat_fwd_fl_kernel)", "spmm_fwd3": "spmm_kernel (fwd hop)",
                   "gat_bwd": ("cign_gat_bwd (gat_bwd_rows_agg_kernel + gat_bwd_cols_fl_kernel)" if agg_path else
                               "cign_gat_bwd (gat_bwd_rows_fl_kernel + gat_bwd_cols_fl_kernel)"),
                   "spmm_bwd3": "spmm_kernel (bwd hop, fused add)"}[dom]
    traffic, traffic_src = measured_traffic(f"layer_{'c5' if scale else 'c2c3'}_{dtype}", dom)
    layer_gbs = B["layer"] / (ms * 1e-3) / 1e9
    layer_own_gbs = B["layer" + gkey] / (ms * 1e-3) / 1e9

    checks = invariants(torch, w, ext, plan, H, C, D, dt) if scale else None
    projected = None
    if not scale and not eager:
        projected = projected_layer(torch, w, dtype, steps, warmup, plan, X, (g1, g2, g3), capture, ev)

    line = {
        "metric": "GAT+multihop layer fwd+bwd edges/sec; achieved HBM GB/s as % of roofline",
        "value": E * steps / elapsed,
        "unit": "edges/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": ms,
        "gpu_ms_per_step": round(gpu_step_ms, 5),
        "median_gpu_ms_per_step": round(median_step_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "data": (f"synthetic: seeded Chung-Lu power-law graph (gamma {2.2 if scale else 2.5}), N(0,1) features "
                 "and gradient probes"),
        "config": {"workload": (f"{'c5 scale' if scale else 'c2+c3'} layer: collapsed GAT H={H} x C={C} + 3-hop "
                                f"CSR SpMM D={D}, forward+backward"),
                   "launch": "eager" if eager else "hip_graph_per_step",
                   "nodes": n, "edges_nnz": E, "heads": H, "channels": C, "dense_cols": D, "hops": 3,
                   "max_in_degree": int(torch.diff(rowptr.long()).max())},
        "layer_GB_s": round(layer_gbs, 1),
        "layer_roofline_frac": round(layer_gbs / HBM_PEAK_GBS, 4),
        "algorithmic_bytes_per_step": B["layer"],
        # The same step priced with the bytes of the algorithm that runs
        # (per-row aggregates instead of the backward's second gather).
        "layer_own_bytes_per_step": B["layer" + gkey],
        "layer_own_roofline_frac": round(layer_own_gbs / HBM_PEAK_GBS, 4),
        "breakdown": breakdown,
        "roofline": {"bound": "hbm", "kernel": kernel_name, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_source": traffic_src, "bytes_per_launch": bytes_per_launch[dom],
                     "avg_launch_ms": round(dom_ms, 5)},
    }
    if checks is not None:
        line["invariants"] = checks
    if projected is not None:
        line["c2_with_projection"] = projected
    return line, w


def _graph_time(torch, fn, R=10, M=20):
    """Per-call milliseconds of fn(): R calls captured as one HIP graph (its
    allocations settled by an eager call on a side stream first), replayed
    M times with a HIP event pair on the launch stream around each replay.
    Returns (mean, median) over the replays."""
    import statistics

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(R):
            fn()
    g.replay()
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(M)]
    for a, b in evs:
        a.record()
        g.replay()
        b.record()
    torch.cuda.synchronize()
    per = [a.elapsed_time(b) / R for a, b in evs]
    return sum(per) / len(per), statistics.median(per)


def measure_multihop(torch, w, D: int, dtype: str):
    """BASELINE config c3: the 3-hop CSR SpMM pipeline alone (MultiHopCsrPlan
    forward3 then backward3, every hop's output retained) on the c2 graph's
    normalized adjacency at D columns, fp32 or bf16 storage (fp32 math). One
    call of each is timed from HIP graph replays; per-hop GB/s against the
    survey byte model (a hop 4(N+1) + 8E + s E D + s N D; the backward's two
    hops that add g_k read s N D more)."""
    from cign_amd import workloads
    from cign_amd.multihop_csr_pipeline import MultiHopCSR3GraphOperator

    dev = torch.device("cuda:0")
    dt = torch.float32 if dtype == "f32" else torch.bfloat16
    s = 4 if dtype == "f32" else 2
    n, E = w.n, w.nnz_p
    g = torch.Generator(device="cpu").manual_seed(3)
    X, g1, g2, g3 = (torch.randn(n, D, generator=g).to(dev).to(dt) for _ in range(4))
    plan = MultiHopCSR3GraphOperator(w.operator, dense_cols=D, dense_dtype=dt).plan
    plan.forward3(X)
    plan.backward3(g1, g2, g3)
    fwd, fwd_med = _graph_time(torch, lambda: plan.forward3(X))
    bwd, bwd_med = _graph_time(torch, lambda: plan.backward3(g1, g2, g3))
    step, step_med = _graph_time(torch, lambda: (plan.forward3(X), plan.backward3(g1, g2, g3)))
    B = workloads.algorithmic_bytes(n, E, 1, 1, D, s_mh=s)
    hop_f = B["spmm"] / (fwd / 3 * 1e-3) / 1e9
    hop_b = (B["spmm"] + s * n * D * 2 / 3) / (bwd / 3 * 1e-3) / 1e9
    gbs = B["multihop"] / (step * 1e-3) / 1e9
    return {"D": D, "dtype": dtype, "ms_per_step": round(step, 5), "median_ms_per_step": round(step_med, 5),
            "fwd3_ms": round(fwd, 5), "bwd3_ms": round(bwd, 5), "edges_per_s": E / (step * 1e-3),
            "algorithmic_bytes_per_step": B["multihop"], "GB_s": round(gbs, 1),
            "roofline_frac": round(gbs / HBM_PEAK_GBS, 4),
            "hop_fwd_GB_s": round(hop_f, 1), "hop_bwd_GB_s": round(hop_b, 1),
            "hop_roofline_frac": round(max(hop_f, hop_b) / HBM_PEAK_GBS, 4)}


C4_N, C4_D = 24492, 256


def measure_c4_pack(torch):
    """BASELINE config c4's first half at N = 24,492, D = 256 (8 blades x 32
    channels), K = 3, fp32 N(0,1): the production Clifford pack (CIGN switch
    pack, interaction new, weighting old: out [N, 6D]) forward and backward
    through the drop-in extension object, and the block's side ops with
    dropout p = 0.5 (dropout + LayerNorm, add + LayerNorm, dropout-gamma
    residual, each forward and backward). Each call is timed from HIP graph
    replays and priced by its streamed bytes: the pack forward reads H, C
    (4ND each), the three hops (8ND each) and alpha (12N) and writes 24ND
    (351.4 MB); the backward reads grad_out (24ND) and the forward's inputs
    and writes their gradients (552.3 MB)."""
    from cign_amd.fused_block_ops import ensure_fused_block_ops_loaded
    from cign_amd.fused_clifford_cign_pack import ensure_fused_clifford_switch_pack_loaded

    dev = torch.device("cuda:0")
    N, D, K, p = C4_N, C4_D, 3, 0.5
    g = torch.Generator(device="cpu").manual_seed(4)
    r = lambda *sh: torch.randn(*sh, generator=g).to(dev)
    H, C, h2 = r(N, D), r(N, D), r(N, D)
    P = [r(N, 2 * D) for _ in range(K)]
    alpha = torch.softmax(r(N, K), -1).contiguous()
    G6 = r(N, 2 * K * D)
    gy = r(N, D)
    w, b, gamma = r(D), r(D), r(D)
    pack = ensure_fused_clifford_switch_pack_loaded()
    ops = ensure_fused_block_ops_loaded()
    y_ln, mu, rs, m_ln = ops.dropout_layernorm_forward(H, w, b, p, 1e-5, 11)
    y_a, mu_a, rs_a = ops.add_layernorm_forward(H, C, w, b, 1e-5)
    y_g, m_g = ops.dropout_gamma_residual_forward(h2, C, gamma, p, 12)
    ND = N * D
    calls = {
        "pack_fwd": (lambda: pack.forward(H, C, *P, alpha, 1, 0), 4 * N * 14 * D + 12 * N),
        "pack_bwd": (lambda: pack.backward(G6, H, C, *P, alpha, 1, 0), 4 * N * 22 * D + 24 * N),
        "dropout_ln_fwd": (lambda: ops.dropout_layernorm_forward(H, w, b, p, 1e-5, 11), 9 * ND + 8 * N + 8 * D),
        "dropout_ln_bwd": (lambda: ops.dropout_layernorm_backward(gy, H, w, mu, rs, m_ln, p),
                           13 * ND + 8 * N + 12 * D),
        "add_ln_fwd": (lambda: ops.add_layernorm_forward(H, C, w, b, 1e-5), 12 * ND + 8 * N + 8 * D),
        "add_ln_bwd": (lambda: ops.add_layernorm_backward(gy, H, C, w, mu_a, rs_a), 16 * ND + 8 * N + 12 * D),
        "gamma_residual_fwd": (lambda: ops.dropout_gamma_residual_forward(h2, C, gamma, p, 12), 13 * ND + 4 * D),
        "gamma_residual_bwd": (lambda: ops.dropout_gamma_residual_backward(gy, C, gamma, m_g, p), 13 * ND + 8 * D),
    }
    out, total_ms, total_b = {}, 0.0, 0
    for k, (fn, nbytes) in calls.items():
        fn()
        mean, med = _graph_time(torch, fn)
        gbs = nbytes / (mean * 1e-3) / 1e9
        out[k] = {"ms": round(mean, 5), "median_ms": round(med, 5), "bytes": nbytes, "GB_s": round(gbs, 1),
                  "roofline_frac": round(gbs / HBM_PEAK_GBS, 4)}
        total_ms += mean
        total_b += nbytes
    step = total_ms
    return {"workload": "c4 pack + side ops: CIGN switch pack (new interaction, old weighting) K=3 + dropout-LN, "
                        "add-LN, dropout-gamma-residual at p=0.5, forward + backward",
            "nodes": N, "dim": D, "hops": K, "dtype": "f32", "ms_per_step": round(step, 5),
            "algorithmic_bytes_per_step": total_b, "GB_s": round(total_b / (step * 1e-3) / 1e9, 1),
            "roofline_frac": round(total_b / (step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "calls": out}


def measure_c2proj(torch, dtype, steps, warmup):
    """projected_layer on its own: the c2 graph, the 3-hop plan at D = 64 and
    its gradient probes, HIP-graph replays as in the headline run."""
    from cign_amd import workloads
    from cign_amd.multihop_csr_pipeline import MultiHopCSR3GraphOperator

    dev = torch.device("cuda:0")
    dt = torch.float32 if dtype == "f32" else torch.bfloat16
    w = workloads.build(workloads.C2, device=dev)
    g = torch.Generator(device="cpu").manual_seed(0)
    X = torch.randn(w.n, 64, generator=g).to(dev).to(dt)
    grads = tuple(torch.randn(w.n, 64, generator=g).to(dev).to(dt) for _ in range(3))
    plan = MultiHopCSR3GraphOperator(w.operator, dense_cols=64, dense_dtype=dt).plan

    def capture(fn):
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            fn()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            fn()
        return gr

    ev = lambda: torch.cuda.Event(enable_timing=True)
    return projected_layer(torch, w, dtype, steps, warmup, plan, X, grads, capture, ev)


def projected_layer(torch, w, dtype, steps, warmup, plan, X, grads, capture, ev):
    """The c2 layer as BASELINE config 2 states it, the GAT's input 300-dim
    features projected to 4 heads x 16 (the GAT lin on MFMA, fp32 or bf16
    autocast, with the attention logits; backward: the weight and logit
    gradients, the input being data) plus the same 3-hop SpMM, one step per
    HIP graph replay, timed as the headline step. The projection runs as
    CompatibleCollapsedFusedGATConv runs it (lin_gat's forward and backward,
    called without autograd so the step captures as one graph)."""
    from cign_amd.lin_gat import _LinGatFn

    dev = torch.device("cuda:0")
    H, C, K_in = 4, 16, 300
    (rowptr, col), (row, colptr), perm = w.gat_graph
    gen = torch.Generator(device="cpu").manual_seed(1)
    x300 = torch.randn(w.n, K_in, generator=gen).to(dev)
    Wl = (torch.randn(H * C, K_in, generator=gen) / K_in ** 0.5).to(dev)
    att_s = (torch.randn(1, H, C, generator=gen) * 0.1).to(dev)
    att_d = (torch.randn(1, H, C, generator=gen) * 0.1).to(dev)
    bias = (torch.randn(C, generator=gen) * 0.1).to(dev)
    gy = torch.randn(w.n, C, generator=gen).to(dev)
    math = 1 if dtype == "bf16" else 0

    class Ctx:
        needs_input_grad = (False, True, True, True, True) + (False,) * 10

        def save_for_backward(self, *t):
            self.saved_tensors = t

    def step():
        ctx = Ctx()
        _LinGatFn.forward(ctx, x300, Wl, att_s, att_d, bias, rowptr, col, colptr, row, perm, 0.2, 0.0, 0, H, math)
        plan.forward3(X)
        _LinGatFn.backward(ctx, gy)
        plan.backward3(*grads)

    for _ in range(max(1, warmup)):
        step()
    torch.cuda.synchronize()
    replay = capture(step).replay
    for _ in range(max(1, warmup)):
        replay()
    torch.cuda.synchronize()
    a0, a1 = ev(), ev()
    t0 = time.perf_counter()
    a0.record()
    for _ in range(steps):
        replay()
    a1.record()
    torch.cuda.synchronize()
    ms = 1e3 * (time.perf_counter() - t0) / steps
    E = w.nnz_gat
    return {"ms_per_step": round(ms, 5), "gpu_ms_per_step": round(a0.elapsed_time(a1) / steps, 5),
            "edges_per_s": E / (ms * 1e-3),
            "projection": f"GAT lin {K_in} -> {H} x {C} on MFMA ({'bf16 autocast' if math else 'fp32'}) with the "
                          "attention logits, forward + weight and logit gradients"}




if __name__ == "__main__":
    main()
