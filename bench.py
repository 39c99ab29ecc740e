#!/usr/bin/env python3
"""Forward throughput of the HdcMamba LM on one MI355X.

Default workload: the 24-layer d_model=1024 (d_state 128, 16 heads, chunk 64, vocab 50304,
tied head) language model forward at B=1, L=32768 in bf16, uniform random token ids and
random-init weights.  One step = one full forward (embedding, 24 blocks, final norms,
logits), timed as replays of the forward recorded as a HIP graph.  Prints ONE JSON line
with tokens/s, the roofline of the dominant custom kernel (HIP events recorded by each
custom kernel's own dispatch, over a second timed region of eager forwards), per-kernel
figures, and the CPU oracle's throughput on a bounded sample of the same workload.

    python bench.py [--steps K] [--warmup W] [--workload lm_c4|lm_c3|block_c1|block_c2|lm_c5_decode|lm_c4_train]
                    [--graph on|off] [--tuned-gemms on|off] [--cpu-baseline on|off]
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
MFMA_PEAK_TFS = 2500.0  # MI355X dense bf16 MFMA


def _cpu_model():
    """The host CPU as /proc/cpuinfo names it, with its family/model/stepping numbers and the
    logical CPU count (a virtual machine may report only a short model name)."""
    fields = {}
    n_logical = 0
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if ":" not in line:
                    continue
                k, v = (t.strip() for t in line.split(":", 1))
                if k == "processor":
                    n_logical += 1
                if k in ("model name", "vendor_id", "cpu family", "model", "stepping", "microcode") and k not in fields:
                    fields[k] = v
    except OSError:
        pass
    name = fields.get("model name") or platform.processor() or "unknown"
    extra = ", ".join(f"{k} {fields[k]}" for k in ("vendor_id", "cpu family", "model", "stepping", "microcode")
                      if k in fields)
    return f"{name} ({extra}; {n_logical} logical CPUs visible)" if extra else name


def forward_totals(cfg, fused_out_proj=True):
    """Algorithmic FLOPs and compulsory HBM bytes of one LM forward (bf16, eb=2).

    Per block, bytes: norm_conv (read x, write x_conv), in_proj (read x_conv and W, write
    projs), SSM (read dt/x/b, write y), slot state pre-pass (read k, v), slot_gate (read
    q/k/v/gate, write output), rowln (read and write combined; absent when the LayerNorm is
    folded into out_proj), out_proj (read combined, W and the residual, write the
    residual).  FLOPs: in_proj, out_proj and the slot contractions (dense C x C count).
    Plus embedding, the two final LayerNorms (norm_final, norm_f: one fused pass, read and
    write once) and the tied head (read x and the embedding, write the logits)."""
    eb = 2
    T = cfg["B"] * cfg["L"]
    dm, ds, H, C, V = cfg["d_model"], cfg["d_state"], cfg["num_heads"], cfg["chunk"], 50304
    hd, P = dm // H, 3 * ds + 4 * dm
    rowln = 0 if fused_out_proj else 2 * (ds + dm)
    blk_bytes = T * eb * (2 * dm + (dm + P) + 4 * ds + 2 * dm + 5 * dm + rowln + (ds + 3 * dm)) \
        + eb * (P * dm + dm * (ds + dm))
    blk_flops = 2 * T * dm * P + 2 * T * (ds + dm) * dm + T * H * (4 * C * hd + 4 * hd * hd)
    n = cfg["n_layers"]
    tail_bytes = T * eb * dm * (1 + 2 + 1) + V * dm * eb + T * V * eb
    tail_flops = 2 * T * dm * V
    return n * blk_flops + tail_flops, n * blk_bytes + tail_bytes


# Calls whose kernels bench.py times (hdcmamba_amd._ops wrapper names).
KERNELS = ("norm_conv", "ssm", "slot_state", "slot_gate", "rowln", "rowln2", "rowln_gemm")


def _mean(xs):
    return sum(xs) / len(xs)


def kernel_table(cfg, tokens, times):
    """Per-kernel durations (microseconds, mean over launches) and roofline fractions from
    the dispatch-timed calls `times` ({call: [[ms of each kernel of the call] per call]}).

    Algorithmic HBM bytes per token (eb = element bytes): norm_conv 2 dm eb (read x, write
    x_conv); SSM 4 ds eb (read dt, x, b; write y); slot_state 2 dm eb (read k, v); slot_gate
    5 dm eb (read q, k, v, gate; write the gated output) -- also the bytes of the slot
    operator as a whole (state pre-pass + segment scan + gate pass); rowln 2 dm eb.
    out_proj (rowln_gemm) is MFMA-bound: 2 T (ds + dm) dm FLOPs against the bf16 peak."""
    eb = 2 if cfg["dtype_name"] == "bf16" else 4
    dm, ds = cfg["d_model"], cfg["d_state"]

    def hbm(us, nbytes, launches, **extra):
        gbs = nbytes / (us * 1e-6) / 1e9
        return {"us": round(us, 2), "launches": launches, "bytes_per_launch": nbytes, "bound": "hbm",
                "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4), **extra}

    out = {}
    if "norm_conv" in times:
        c = times["norm_conv"]
        out["norm_conv"] = hbm(_mean([k[0] for k in c]) * 1e3, 2 * dm * eb * tokens, len(c))
    if "ssm" in times:
        c = times["ssm"]
        per = [round(_mean([k[i] for k in c]) * 1e3, 2) for i in range(len(c[0]))]
        out["ssm"] = hbm(sum(per), 4 * ds * eb * tokens, len(c), kernels_us=per,
                         note="sum of the SSM's kernels")
    if "slot_state" in times:
        c = [k for k in times["slot_state"] if len(k) == 2]  # pre-pass + scan (more than one segment)
        if c:
            out["slot_state"] = hbm(_mean([k[0] for k in c]) * 1e3, 2 * dm * eb * tokens, len(c))
            out["slot_scan"] = {"us": round(_mean([k[1] for k in c]) * 1e3, 2), "launches": len(c)}
    if "slot_gate" in times:
        c = times["slot_gate"]
        out["slot_gate"] = hbm(_mean([k[0] for k in c]) * 1e3, 5 * dm * eb * tokens, len(c))
    if "slot_gate" in out and "slot_state" in out:
        us = out["slot_state"]["us"] + out["slot_scan"]["us"] + out["slot_gate"]["us"]
        out["slot_op"] = hbm(us, 5 * dm * eb * tokens, out["slot_gate"]["launches"],
                             note="slot_state + slot_scan + slot_gate against the gate pass's bytes")
    if "rowln" in times:
        c = times["rowln"]
        out["rowln"] = hbm(_mean([k[0] for k in c]) * 1e3, 2 * dm * eb * tokens, len(c))
    if "rowln2" in times:  # norm_final and norm_f in one pass
        c = times["rowln2"]
        out["rowln2"] = hbm(_mean([k[0] for k in c]) * 1e3, 2 * dm * eb * tokens, len(c))
    if "rowln_gemm" in times:
        c = times["rowln_gemm"]
        us = _mean([k[0] for k in c]) * 1e3
        fl = 2 * tokens * (ds + dm) * dm
        tfs = fl / (us * 1e-6) / 1e12
        out["out_proj"] = {"us": round(us, 2), "launches": len(c), "flops_per_launch": fl, "bound": "mfma",
                           "TFLOP/s": round(tfs, 1), "frac": round(tfs / MFMA_PEAK_TFS, 4),
                           "note": "rowln_gemm: out_proj with the folded row LayerNorm and the residual"}
    return out


def roofline_of(k, traffic, profile_us=None):
    """The bench line's roofline object for one kernel_table entry; with `profile_us` (the
    kernel's mean duration in the committed rocprofv3 kernel trace of this bench command),
    also the fraction that duration gives."""
    if k["bound"] == "mfma":
        r = {"bound": "mfma", "achieved": k["TFLOP/s"], "peak": MFMA_PEAK_TFS, "unit": "TFLOP/s",
             "frac": k["frac"], "traffic": traffic, "us": k["us"], "flops_per_launch": k["flops_per_launch"]}
        work, peak, scale = k["flops_per_launch"], MFMA_PEAK_TFS, 1e12
    else:
        r = {"bound": "hbm", "achieved": k["GB/s"], "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": k["frac"],
             "traffic": traffic, "us": k["us"], "bytes_per_launch": k["bytes_per_launch"]}
        work, peak, scale = k["bytes_per_launch"], HBM_PEAK_GBS, 1e9
    if profile_us:
        r["profile_us"] = profile_us
        r["profile_frac"] = round(work / (profile_us * 1e-6) / scale / peak, 4)
    return r


PROFILES = os.path.join(ROOT, "profiles")
TRAFFIC_SUMMARY = os.path.join(PROFILES, "lm_c4_forward_traffic.md")
STATS_SUMMARY = os.path.join(PROFILES, "lm_c4_forward_kernel_stats.md")
MFMA_SUMMARY = os.path.join(PROFILES, "lm_c4_forward_mfma.md")
SOURCE_KEY = "kernel_sources_sha256:"
COPY_CALIB_BYTES = 64 << 20  # the counter runs' calibration copy (see main)

# bench.py kernel key -> start of the kernel's name in rocprofv3 output (template arguments
# removed); the out_proj GEMM of the forward is the statistics variant (EPI_ROWSTATS = 2)
KERNEL_NAMES = {"norm_conv": "norm_conv_kernel<", "ssm": "ssm_scan_kernel<", "slot_state": "slot_state_kernel<",
                "slot_scan": "slot_scan_kernel<", "slot_gate": "slot_gate_kernel<", "rowln": "rowln_kernel<",
                "rowln2": "rowln2_kernel<",
                "out_proj": "gemm_bt_kernel<2,"}


def _short_name(n):
    n = n.replace("void ", "").replace("(anonymous namespace)::", "")
    return n.split("(")[0]


def _kernel_key(name):
    for key, prefix in KERNEL_NAMES.items():
        if name.startswith(prefix):
            return key
    return None


def source_hash():
    """sha256 over the HIP sources and headers the library's kernels are built from and the
    package's Python (which decides the launch sequence): a stored profile is used only while
    these are unchanged."""
    import glob
    import hashlib

    h = hashlib.sha256()
    files = sorted(glob.glob(os.path.join(ROOT, "hdcmamba_amd", "csrc", "*.hip")) +
                   glob.glob(os.path.join(ROOT, "hdcmamba_amd", "csrc", "*.h")) +
                   glob.glob(os.path.join(ROOT, "hdcmamba_amd", "*.py")) +
                   [os.path.join(ROOT, "include", "hdcm.h")])
    for path in files:
        h.update(os.path.basename(path).encode())
        with open(path, "rb") as f:
            h.update(f.read())
    return h.hexdigest()


def _metric_lines(metric, values):
    """Machine-readable lines of a profile summary: '<metric>: <kernel> <value>'."""
    return [f"{metric}: {k} {v}" for k, v in sorted(values.items())]


def stored_metric(path, metric):
    """{kernel: value} of `metric` in a committed profile summary, or {} when the summary is
    missing or was made from other kernel sources than the ones in this tree."""
    if not os.path.exists(path):
        return {}
    vals, src = {}, None
    with open(path) as f:
        for line in f:
            if line.startswith(SOURCE_KEY):
                src = line.split(":", 1)[1].strip()
            elif line.startswith(metric + ":"):
                f = line.split(":", 1)[1].split()
                if len(f) == 2:  # '<kernel> <value>' (older summaries held one bare number)
                    vals[f[0]] = float(f[1])
    return vals if src == source_hash() else {}


def _read_pmc(path):
    """{(dispatch id): {counter: value}, ...} and {dispatch id: short kernel name} of a
    rocprofv3 --pmc counter_collection.csv."""
    import collections
    import csv

    vals, names = collections.defaultdict(dict), {}
    with open(path) as f:
        for r in csv.DictReader(f):
            d = int(r["Dispatch_Id"])
            vals[d][r["Counter_Name"]] = float(r["Counter_Value"])
            names[d] = _short_name(r["Kernel_Name"])
    return vals, names


def pmc_summary(fetch_csv, write_csv, copy_bytes):
    """Per-kernel HBM bytes per dispatch from two rocprofv3 --pmc runs (FETCH_SIZE and
    WRITE_SIZE, KiB per dispatch).  Each counter is scaled by bytes / counter reading of the
    runtime's copy kernel for the copy of known size (`copy_bytes`) in the same run.
    Returns markdown text."""
    import collections

    def read(path, counter):
        vals, names = _read_pmc(path)
        agg = collections.defaultdict(list)
        for d, c in vals.items():
            if counter in c:
                agg[names[d]].append(c[counter])
        return agg

    def scale(agg, counter):
        cands = [v for v in agg.get("__amd_rocclr_copyBuffer", []) if v > 0.25 * copy_bytes / 1024]
        if not cands:
            raise SystemExit(f"no copy kernel of ~{copy_bytes} bytes in the {counter} run")
        return copy_bytes / (max(cands) * 1024)

    fa, wa = read(fetch_csv, "FETCH_SIZE"), read(write_csv, "WRITE_SIZE")
    ff, fw = scale(fa, "FETCH_SIZE"), scale(wa, "WRITE_SIZE")
    lines = ["| kernel | dispatches | FETCH_SIZE KiB | WRITE_SIZE KiB | HBM MB per dispatch (scaled) |",
             "|---|---:|---:|---:|---:|"]
    out, keyed = {}, {}
    for k in sorted(set(fa) & set(wa), key=lambda k: -sum(fa[k]) / len(fa[k])):
        f, w = sum(fa[k]) / len(fa[k]), sum(wa[k]) / len(wa[k])
        out[k] = (f * ff + w * fw) * 1024
        lines.append(f"| {k[:70]} | {len(fa[k])} | {f:.1f} | {w:.1f} | {out[k] / 1e6:.2f} |")
        key = _kernel_key(k)
        if key:
            keyed[key] = round(out[k])
    head = [f"copy calibration ({copy_bytes} bytes): FETCH_SIZE x {ff:.4f}, WRITE_SIZE x {fw:.4f}", "",
            f"{SOURCE_KEY} {source_hash()}"] + _metric_lines("traffic_bytes_per_launch", keyed) + [""]
    return "\n".join(head + lines) + "\n"


def mfma_summary(pmc_csv):
    """Per-kernel MFMA use from a rocprofv3 --pmc run of MfmaUtil (rocprofiler's derived metric:
    SQ_VALU_MFMA_BUSY_CYCLES over GRBM_GUI_ACTIVE x SIMDs, percent), SQ_INSTS_VALU_MFMA_MOPS_BF16
    and SQ_INSTS_VALU_MFMA_MOPS_F32 (x 512 = FLOPs).  Returns markdown text."""
    import collections

    vals, names = _read_pmc(pmc_csv)
    agg = collections.defaultdict(lambda: collections.defaultdict(list))
    for d, c in vals.items():
        for ctr, v in c.items():
            agg[names[d]][ctr].append(v)
    lines = ["| kernel | dispatches | MFMA busy % | bf16 MFMA GFLOP per dispatch | fp32 MFMA GFLOP per dispatch |",
             "|---|---:|---:|---:|---:|"]
    keyed, order = {}, []
    for k, c in agg.items():
        if "MfmaUtil" not in c:
            continue
        util = sum(c["MfmaUtil"]) / len(c["MfmaUtil"])
        bf = sum(c.get("SQ_INSTS_VALU_MFMA_MOPS_BF16", [0])) / max(1, len(c.get("SQ_INSTS_VALU_MFMA_MOPS_BF16", [0]))) * 512
        f32 = sum(c.get("SQ_INSTS_VALU_MFMA_MOPS_F32", [0])) / max(1, len(c.get("SQ_INSTS_VALU_MFMA_MOPS_F32", [0]))) * 512
        order.append((-util, k, len(c["MfmaUtil"]), util, bf, f32))
        key = _kernel_key(k)
        if key:
            keyed[key] = round(util / 100, 4)
    for _, k, n, util, bf, f32 in sorted(order):
        if util > 0 or bf > 0:
            lines.append(f"| {k[:70]} | {n} | {util:.1f} | {bf / 1e9:.2f} | {f32 / 1e9:.3f} |")
    head = [f"{SOURCE_KEY} {source_hash()}"] + _metric_lines("mfma_busy", keyed) + [""]
    return "\n".join(head + lines) + "\n"


def trace_summary(trace_csv, steps, warmup, layers=24, capture_warmup=2):
    """Per-kernel mean durations of a rocprofv3 --kernel-trace run of this bench by phase: the
    recorded graph's replays (warmup + steps forwards after the capture's warm-up forwards) and
    the event-timed eager forwards (the last min(steps, 5)), for the kernels launched once per
    layer.  Returns markdown text with 'graph_us' and 'timed_us' lines."""
    import collections
    import csv

    k_steps = max(1, min(steps, 5))
    fwd = capture_warmup + warmup + steps + 1 + k_steps  # forwards of the run, in order
    by = collections.defaultdict(list)
    with open(trace_csv) as f:
        for r in csv.DictReader(f):
            key = _kernel_key(_short_name(r["Kernel_Name"]))
            if key:
                by[key].append((int(r["Start_Timestamp"]), int(r["End_Timestamp"])))
    lines = ["| kernel | launches | all (us) | graph replays (us) | timed eager forwards (us) |",
             "|---|---:|---:|---:|---:|"]
    graph, timed = {}, {}
    for key in KERNEL_NAMES:
        v = sorted(by.get(key, []))
        if len(v) != fwd * layers:
            continue
        d = [(e - s) / 1e3 for s, e in v]
        g = d[capture_warmup * layers:(capture_warmup + warmup + steps) * layers]
        t = d[(fwd - k_steps) * layers:]
        graph[key], timed[key] = round(sum(g) / len(g), 2), round(sum(t) / len(t), 2)
        lines.append(f"| {key} | {len(d)} | {sum(d) / len(d):.2f} | {graph[key]:.2f} | {timed[key]:.2f} |")
    head = ([f"{SOURCE_KEY} {source_hash()}"] + _metric_lines("graph_us", graph) + _metric_lines("timed_us", timed)
            + [""])
    return "\n".join(head + lines) + "\n"


def stats_summary(stats_csv):
    """Markdown table of a rocprofv3 --kernel-trace --stats kernel_stats.csv, with the mean
    duration of the bench's kernels as machine-readable lines."""
    import csv

    with open(stats_csv) as f:
        rows = list(csv.DictReader(f))
    lines = ["| kernel | calls | avg us | share |", "|---|---:|---:|---:|"]
    keyed = {}
    for r in rows:
        name = _short_name(r["Name"])
        avg = float(r["AverageNs"]) / 1e3
        lines.append(f"| {name[:70]} | {r['Calls']} | {avg:.1f} | {float(r['Percentage']):.1f}% |")
        key = _kernel_key(name)
        if key and key not in keyed:
            keyed[key] = round(avg, 2)
    head = [f"{SOURCE_KEY} {source_hash()}"] + _metric_lines("avg_us", keyed) + [""]
    return "\n".join(head + lines) + "\n"


def cpu_baseline(model, ids_gpu, cfg, runs=3, run_cap_s=90.0):
    """The CPU oracle on the same weights and inputs: one warm-up (embedding, the first block,
    final norms and logits at the full sequence length), then ``runs`` timed forwards of the
    whole model (embedding, every block, final norms, logits), as the reference's benchmark
    method for the full models (1 warm-up + 3 runs).  A run whose blocks would exceed
    ``run_cap_s`` times the rest of its blocks by extrapolation from their mean (recorded in
    ``sample``).  ``value`` is tokens/s over the mean run."""
    import torch

    import oracle

    threads = len(os.sched_getaffinity(0))  # every core this process may run on
    torch.set_num_threads(threads)
    sd = {k: v.detach().cpu() for k, v in model.state_dict().items()}
    L = cfg["L"]
    ids = ids_gpu[:1, :L].cpu()
    bcfg = oracle.BlockCfg(cfg["d_model"], cfg["d_state"], cfg["num_heads"], cfg["chunk"])
    n_layers = cfg["n_layers"]
    F = torch.nn.functional
    blocks = [{k[len(pre):]: v for k, v in sd.items() if k.startswith(pre)}
              for pre in (f"backbone.layers.{i}." for i in range(n_layers))]

    def tail(x):
        x = F.layer_norm(x, (cfg["d_model"],), sd["backbone.norm_final.weight"], sd["backbone.norm_final.bias"])
        x = F.layer_norm(x, (cfg["d_model"],), sd["norm_f.weight"], sd["norm_f.bias"])
        return F.linear(x, sd["embedding.weight"])

    def forward(nb):
        """(seconds, blocks run): embedding, up to nb blocks (stopping at the cap), tail."""
        t0 = time.perf_counter()
        x = F.embedding(ids, sd["embedding.weight"])
        t_blocks, done = 0.0, 0
        for i in range(nb):
            tb = time.perf_counter()
            x = oracle.block_forward(blocks[i], x, bcfg)
            t_blocks += time.perf_counter() - tb
            done += 1
            if t_blocks > run_cap_s:
                break
        tail(x)
        t = time.perf_counter() - t0
        return t + (t_blocks / done) * (nb - done), done

    t_start = time.perf_counter()
    forward(1)  # warm-up: every op at full size
    times, done = [], n_layers
    for _ in range(runs):
        t, d = forward(n_layers)
        times.append(t)
        done = min(done, d)
    mean = sum(times) / len(times)
    sample = (f"CPU oracle (plain PyTorch, bf16) on the same weights, B=1, L={L}: 1 warm-up (embedding, one "
              f"block, final norms, logits), then {runs} timed forwards of the whole model (embedding, "
              f"{n_layers} blocks, final norms, logits)"
              + ("" if done == n_layers else f"; {done} of {n_layers} blocks timed per run, the rest extrapolated"))
    return {"value": round(L / mean, 1), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": sample, "cpu_model": _cpu_model(), "run_seconds": [round(t, 2) for t in times],
            "seconds_measured": round(time.perf_counter() - t_start, 2)}


def cpu_baseline_block(model, x_gpu, cfg, warmup=3, runs=10):
    """The CPU oracle's block forward on the same weights and input: ``warmup`` untimed and
    ``runs`` timed forwards (the reference benchmark's count for single blocks).  ``value``
    is tokens/s over the mean run."""
    import torch

    import oracle

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    sd = {k: v.detach().cpu() for k, v in model.state_dict().items()}
    x = x_gpu.cpu()
    bcfg = oracle.BlockCfg(cfg["d_model"], cfg["d_state"], cfg["num_heads"], cfg["chunk"])
    t_start = time.perf_counter()
    for _ in range(warmup):
        oracle.block_forward(sd, x, bcfg)
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        oracle.block_forward(sd, x, bcfg)
        times.append(time.perf_counter() - t0)
    mean = sum(times) / len(times)
    return {"value": round(x.shape[0] * x.shape[1] / mean, 1), "unit": "tokens/s", "cores": threads,
            "kind": "port",
            "sample": (f"CPU oracle (plain PyTorch, {str(x.dtype).replace('torch.', '')}) block forward on the same "
                       f"weights and input, B={x.shape[0]}, L={x.shape[1]}: {warmup} warm-ups, {runs} timed runs"),
            "cpu_model": _cpu_model(), "run_seconds": [round(t, 3) for t in times],
            "seconds_measured": round(time.perf_counter() - t_start, 2)}


def cpu_baseline_decode(lm, ids_gpu, cfg, L, prefill_layers=2, steps=16):
    """The CPU oracle on the decode workload's weights: the prefill of ``prefill_layers``
    blocks at the full B x L timed and extrapolated to every block (marked so), then one
    warm-up and ``steps`` timed decode steps of the whole model (embedding, every block's
    recurrent step, final norms, tied head; oracle.block_step).  The decode cost does not
    depend on the states' values, so blocks past the timed prefill start from zero states of
    the same shapes.  ``value`` is decode tokens/s (B per step)."""
    import torch

    import oracle

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    F = torch.nn.functional
    t_start = time.perf_counter()
    sd = {k: v.detach().cpu() for k, v in lm.state_dict().items()}
    ids = ids_gpu.cpu()
    B, n_layers, dm = ids.shape[0], cfg["n_layers"], cfg["d_model"]
    bcfg = oracle.BlockCfg(dm, cfg["d_state"], cfg["num_heads"], cfg["chunk"])
    blocks = [{k[len(pre):]: v for k, v in sd.items() if k.startswith(pre)}
              for pre in (f"backbone.layers.{i}." for i in range(n_layers))]
    emb = sd["embedding.weight"]
    steps = min(steps, ids.shape[1] - L - 1)  # token ids past the prefill: a warm-up step, then the timed ones
    t0 = time.perf_counter()
    x = F.embedding(ids[:, :L], emb)
    states = []
    for i in range(prefill_layers):
        x, st = oracle.block_prefill_state(blocks[i], x, bcfg)
        states.append(st)
        print(f"cpu baseline: prefill block {i} done at {time.perf_counter() - t0:.1f} s", file=sys.stderr, flush=True)
    t_pre = time.perf_counter() - t0
    del x
    H, hd, ds = bcfg.num_heads, bcfg.head_dim, bcfg.d_state
    for _ in range(prefill_layers, n_layers):
        states.append({"conv": torch.zeros(B, 3, dm, dtype=emb.dtype), "h": torch.zeros(B, ds),
                       "S_prev": torch.zeros(B, H, hd, hd), "S_intra": torch.zeros(B, H, hd, hd),
                       "pos": states[0]["pos"]})

    def step(t):
        x = F.embedding(ids[:, L + t], emb)
        for i in range(n_layers):
            x = oracle.block_step(blocks[i], x, states[i], bcfg)
        x = F.layer_norm(x.float(), (dm,), sd["backbone.norm_final.weight"].float(),
                         sd["backbone.norm_final.bias"].float()).to(emb.dtype)
        x = F.layer_norm(x.float(), (dm,), sd["norm_f.weight"].float(), sd["norm_f.bias"].float()).to(emb.dtype)
        return F.linear(x, emb)

    step(0)
    t0 = time.perf_counter()
    for t in range(1, steps + 1):
        step(t)
        if t % 4 == 0:
            print(f"cpu baseline: decode step {t} at {time.perf_counter() - t0:.1f} s", file=sys.stderr, flush=True)
    t_dec = time.perf_counter() - t0
    pre_full = t_pre / prefill_layers * n_layers
    return {"value": round(B * steps / t_dec, 1), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": (f"CPU oracle (plain PyTorch, bf16) on the same weights: {steps} timed decode steps of the "
                       f"whole {n_layers}-layer model at B={B} (oracle.block_step per block, final norms, tied "
                       f"head) after one warm-up step; prefill of {prefill_layers} blocks at B={B}, L={L} timed "
                       f"and extrapolated to {n_layers} blocks"),
            "prefill_tokens_per_s": round(B * L / pre_full, 1), "prefill_extrapolated": True,
            "prefill_seconds_measured": round(t_pre, 2), "decode_seconds": round(t_dec, 2),
            "cpu_model": _cpu_model(), "seconds_measured": round(time.perf_counter() - t_start, 2)}


def decode_bench(args, torch, cfg, make_lm, lm_input, dev):
    """Prefill, then time decode steps (B tokens per step) replayed from the captured graph."""
    B, L = cfg["B"], cfg["L"]
    steps = args.steps if args.steps != 10 else 128
    warm = max(args.warmup, 2)
    lm = make_lm("lm_c5").to(torch.bfloat16).to(dev)
    from hdcmamba_amd import _ops, set_fused_out_proj, set_fused_step_front
    set_fused_out_proj(lm, args.fused_out_proj == "on")
    set_fused_step_front(lm, args.fused_step_front == "on")
    ids = lm_input("lm_c5", B=B, L=L + warm + steps + 1).to(dev)
    with torch.no_grad():
        lm.prefill(ids[:, :256])  # warm the prefill kernels and GEMM handles
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        _, states = lm.prefill(ids[:, :L])
        torch.cuda.synchronize()
        t_prefill = time.perf_counter() - t0
        runner = lm if args.eager else lm.capture_decode(states)
        step = (lambda tok: lm.step(tok, states)) if args.eager else runner.step
        for t in range(warm):
            step(ids[:, L + t].contiguous())
        torch.cuda.synchronize()
        toks = [ids[:, L + warm + t].contiguous() for t in range(steps)]
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for tok in toks:
            step(tok)
        torch.cuda.synchronize()
        sec = time.perf_counter() - t0
        # Per-kernel durations of the step's custom kernels: HIP events from their own dispatch
        # timestamps over a few eager steps (launches inside a graph replay carry no events).
        step_kernels = ("norm_conv_in_proj_step", "norm_conv_step", "skinny_gemm", "mixer_step", "rowln_gemm")
        _ops.timer.active = set(step_kernels)
        for t in range(min(8, steps)):
            lm.step(toks[t], states)
        torch.cuda.synchronize()
        _ops.timer.active = set()
        step_times = _ops.timer.collect()
    # bytes one step must move: every parameter once (the tied head counted once) plus the
    # carried states: slot, one fp32 state read and one written per token (S_intra between the
    # tokens of a chunk, S_prev at its first and last), plus S_prev read again at a chunk's
    # last token (1/C of the steps); SSM h read and written; the conv history's 3 rows read and
    # written (shifted)
    param_bytes = sum(p.numel() * p.element_size() for p in lm.parameters())
    st = states[0]
    C = lm.backbone.layers[0].chunk_size
    state_bytes = len(states) * ((2 + 1 / C) * st.S_prev.numel() * 4 + 2 * st.h.numel() * 4
                                 + 2 * st.conv.numel() * 2)
    ms = sec / steps * 1e3
    gbs = (param_bytes + state_bytes) / (ms * 1e-3) / 1e9
    # per layer: the front streams the in_proj weight, the mixer reads and writes one fp32 slot
    # state per (sequence, head), out_proj streams its weight (the rows they read and write
    # are a few hundred KB)
    dm, ds, H = cfg["d_model"], cfg["d_state"], cfg["num_heads"]
    hd = dm // H
    P = 3 * ds + 4 * dm
    step_bytes = {"norm_conv_in_proj_step": P * dm * 2, "mixer_step": 2 * B * H * hd * hd * 4,
                  "rowln_gemm": dm * (ds + dm) * 2}
    step_kernel_table = {}
    for name, calls in step_times.items():
        flat = [k[0] for k in calls if k]
        if not flat:
            continue
        us = _mean(flat) * 1e3
        entry = {"us": round(us, 2), "launches": len(flat)}
        if name in step_bytes:
            g = step_bytes[name] / (us * 1e-6) / 1e9
            entry.update(bytes_per_launch=step_bytes[name], bound="hbm", **{"GB/s": round(g, 1)},
                         frac=round(g / HBM_PEAK_GBS, 4))
        step_kernel_table[name] = entry
    out = {
        "metric": "decode tokens/sec on 1 MI355X, B=16 after an L=8192 prefill",
        "value": round(B * steps / sec, 1), "unit": "tokens/s", "n_gpus": 1, "steps": steps, "warmup": warm,
        "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic: uniform random token ids, random-init weights",
        "config": {"workload": "48-layer d_model=2048 HdcMamba LM, prefill B=16 L=8192 then single-token decode",
                   "d_model": 2048, "d_state": 128, "num_heads": 32, "chunk": 64, "layers": 48, "vocab": 50304,
                   "global_batch": B, "prefill_len": L, "graph": not args.eager,
                   "fused_out_proj": args.fused_out_proj == "on", "fused_step_front": args.fused_step_front == "on"},
        "roofline": {"kernel": "whole decode step", "bound": "hbm", "achieved": round(gbs, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "bytes_per_launch": param_bytes + state_bytes},
        "prefill_tokens_per_s": round(B * L / t_prefill, 1),
        "kernels": step_kernel_table,
        "kernel_timing": ("HIP events from each custom kernel's own dispatch timestamps over eager decode "
                          "steps after the timed replays (norm_conv_in_proj_step: the LayerNorm + conv + "
                          "in_proj front; mixer_step; rowln_gemm: out_proj with the folded LayerNorm and "
                          "the residual); mean per launch; bytes: the streamed weight or the slot states"),
        "step_front_timeouts": _ops.step_timeouts(dev) if args.fused_step_front == "on" else None,
        "cpu_baseline": cpu_baseline_decode(lm, ids, cfg, L) if args.cpu_baseline == "on" else None,
        "gpu": torch.cuda.get_device_name(0),
    }
    print(json.dumps(out), flush=True)


def train_bench(args, torch, cfg, make_lm, lm_input, dev):
    """Training steps of the headline LM as the reference's trainer runs them
    (train_fineweb.py:161-179): bf16 model under autocast, cross-entropy on fp32 logits,
    backward, AdamW step.  `--differentiable-mixer` also trains in_proj, the LN+conv, A_log
    and the GroupNorm (the reference's kernels have no backward)."""
    import torch.nn.functional as F
    from hdcmamba_amd import set_differentiable_mixer

    L = cfg["L"]
    steps = args.steps if args.steps != 10 else 3
    warm = max(args.warmup if args.warmup != 3 else 2, 1)
    lm = make_lm("lm_c4").to(torch.bfloat16).to(dev).train()
    set_differentiable_mixer(lm, args.differentiable_mixer)
    opt = torch.optim.AdamW(lm.parameters(), lr=1e-4, betas=(0.9, 0.95), weight_decay=0.1)
    ids = lm_input("lm_c4", B=cfg["B"], L=L + 1).to(dev)

    def step():
        opt.zero_grad(set_to_none=True)
        with torch.amp.autocast("cuda", dtype=torch.bfloat16):
            logits = lm(ids[:, :-1])
            loss = F.cross_entropy(logits.view(-1, logits.size(-1)).float(), ids[:, 1:].reshape(-1))
        loss.backward()
        opt.step()
        return loss

    for _ in range(warm):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        loss = step()
    torch.cuda.synchronize()
    sec = time.perf_counter() - t0
    tokens = cfg["B"] * L * steps
    out = {
        "metric": "training tokens/sec on 1 MI355X at L=32768 (forward, loss, backward, AdamW)",
        "value": round(tokens / sec, 1), "unit": "tokens/s", "n_gpus": 1, "steps": steps, "warmup": warm,
        "ms_per_step": round(sec / steps * 1e3, 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic: uniform random token ids, random-init weights",
        "config": {"workload": "24-layer d_model=1024 HdcMamba LM training step, B=1, L=32768",
                   "differentiable_mixer": bool(args.differentiable_mixer), "optimizer": "AdamW",
                   "loss": "cross-entropy on fp32 logits (train_fineweb.py:170-171)"},
        "loss": round(float(loss), 4),
        "peak_memory_GiB": round(torch.cuda.max_memory_allocated() / 2 ** 30, 1),
        "gpu": torch.cuda.get_device_name(0),
    }
    print(json.dumps(out), flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--differentiable-mixer", action="store_true",
                    help="lm_c4_train: train the SSM, slot and gate parameters too")
    ap.add_argument("--workload", default="lm_c4",
                    choices=["lm_c4", "lm_c3", "block_c1", "block_c2", "lm_c5_decode", "lm_c4_train"],
                    help="lm_c5_decode: 48-layer d_model=2048 LM, prefill B=16 x 8192, then timed "
                         "single-token decode steps (a separate measurement, not the headline line)")
    ap.add_argument("--eager", action="store_true", help="lm_c5_decode: step from Python instead of "
                    "replaying the captured decode graph")
    ap.add_argument("--graph", default="on", choices=["on", "off"],
                    help="LM workloads: time replays of the forward recorded as a HIP graph "
                         "(on) or eager forwards (off)")
    ap.add_argument("--tuned-gemms", default="on", choices=["on", "off"],
                    help="run in_proj/out_proj/LM head on the hipBLASLt/rocBLAS solutions recorded "
                         "in hdcmamba_amd/tuned/gemm_gfx950.csv (TunableOp, tuning off)")
    ap.add_argument("--fused-out-proj", default="on", choices=["on", "off"],
                    help="LM workloads: the LayerNorm of `combined`, out_proj and the residual add as one "
                         "GEMM with the LayerNorm in its epilogue (on) or a row LayerNorm kernel and addmm (off)")
    ap.add_argument("--fused-step-front", default="on", choices=["on", "off"],
                    help="lm_c5_decode: each block's LayerNorm + conv and in_proj of the token as one launch "
                         "(on) or as two kernels (off)")
    ap.add_argument("--cpu-baseline", default="on", choices=["on", "off"])
    ap.add_argument("--cpu-runs", type=int, default=3, help="timed CPU-oracle forwards after one warm-up")
    ap.add_argument("--pmc-summary", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="print the HBM traffic table of two rocprofv3 --pmc runs of this bench "
                         "(FETCH_SIZE, WRITE_SIZE) and exit; needs no GPU")
    ap.add_argument("--stats-summary", metavar="KERNEL_STATS_CSV",
                    help="print the per-kernel table of a rocprofv3 --stats run and exit")
    ap.add_argument("--trace-summary", metavar="KERNEL_TRACE_CSV",
                    help="print the per-phase kernel durations of a rocprofv3 --kernel-trace run of this bench "
                         "(made with the --steps and --warmup given here) and exit")
    ap.add_argument("--mfma-summary", metavar="PMC_CSV",
                    help="print the MFMA-use table of a rocprofv3 --pmc MfmaUtil SQ_INSTS_VALU_MFMA_MOPS_BF16 "
                         "SQ_INSTS_VALU_MFMA_MOPS_F32 run of this bench and exit; needs no GPU")
    args = ap.parse_args()
    if args.stats_summary:
        sys.stdout.write(stats_summary(args.stats_summary))
        return
    if args.mfma_summary:
        sys.stdout.write(mfma_summary(args.mfma_summary))
        return
    if args.trace_summary:
        sys.stdout.write(trace_summary(args.trace_summary, args.steps, args.warmup))
        return
    if args.pmc_summary:
        # scaled by the 64 MiB calibration copy a forward run of bench.py makes first
        sys.stdout.write(pmc_summary(*args.pmc_summary, copy_bytes=COPY_CALIB_BYTES))
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one MI355X (got --gpus {args.gpus}, WORLD_SIZE {world}); runs on "
              "several GPUs are not part of this build.", file=sys.stderr)
        sys.exit(2)

    import torch

    from cfgs import WORKLOADS, block_input, lm_input, make_block, make_lm
    from hdcmamba_amd import _ops, set_fused_out_proj
    from hdcmamba_amd.gemm_tuning import use_tuned_gemms

    n_tuned = use_tuned_gemms() if args.tuned_gemms == "on" else 0

    dev = torch.device("cuda:0")
    if args.workload == "lm_c5_decode":
        return decode_bench(args, torch, WORKLOADS["lm_c5"], make_lm, lm_input, dev)
    if args.workload == "lm_c4_train":
        return train_bench(args, torch, WORKLOADS["lm_c4"], make_lm, lm_input, dev)
    cfg = dict(WORKLOADS[args.workload])
    cfg["dtype_name"] = "bf16" if cfg["dtype"] == torch.bfloat16 else "fp32"
    if args.workload.startswith("lm"):
        model = make_lm(args.workload).to(cfg["dtype"]).to(dev)
        set_fused_out_proj(model, args.fused_out_proj == "on")
        inp = lm_input(args.workload).to(dev)
        workload = (f"{cfg['n_layers']}-layer d_model={cfg['d_model']} HdcMamba LM forward, "
                    f"B={cfg['B']}, L={cfg['L']}")
    else:
        model = make_block(args.workload).to(cfg["dtype"]).to(dev)
        inp = block_input(args.workload).to(dev)
        workload = f"one HdcMamba block forward, B={cfg['B']}, L={cfg['L']}, d_model={cfg['d_model']}"
    tokens = cfg["B"] * cfg["L"]

    # A device copy of known size outside the timed regions: the rocprofv3 counter runs of this
    # command scale FETCH_SIZE and WRITE_SIZE by what they read for it (--pmc-summary).
    calib = torch.empty(COPY_CALIB_BYTES // 2, dtype=torch.bfloat16, device=dev)
    torch.empty_like(calib).copy_(calib)
    del calib

    use_graph = args.graph == "on" and args.workload.startswith("lm")
    with torch.no_grad():
        runner = model.capture_forward(inp) if use_graph else model
        for _ in range(args.warmup):
            runner(inp)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            runner(inp)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        # Per-kernel durations: every custom kernel of k_steps eager forwards records a pair of
        # HIP events from its own dispatch timestamps (hdcm_time_launches; launches inside a
        # graph replay cannot carry events).  The events add nothing to the stream, so these
        # forwards also give the eager rate.
        # The scan runs in sequence with the slot kernels here, as in the recorded graph, so each
        # kernel is timed alone (eager forwards otherwise overlap it with the slot pre-pass).
        k_steps = max(1, min(args.steps, 5))
        from hdcmamba_amd.model import HdcMamba9v3Block
        overlap = HdcMamba9v3Block.ssm_overlap
        HdcMamba9v3Block.ssm_overlap = "none"
        model(inp)
        torch.cuda.synchronize()
        _ops.timer.active = set(KERNELS)
        t2 = time.perf_counter()
        for _ in range(k_steps):
            model(inp)
        torch.cuda.synchronize()
        t3 = time.perf_counter()
        _ops.timer.active = set()
        HdcMamba9v3Block.ssm_overlap = overlap
    times = _ops.timer.collect()
    sec = t1 - t0
    ms_per_step = sec / args.steps * 1e3
    value = tokens * args.steps / sec
    eager_ms = (t3 - t2) / k_steps * 1e3
    kernels = kernel_table(cfg, tokens, times)
    # figures of the committed rocprofv3 summaries of this command (profiles/), when they were
    # made from the kernel sources in this tree: HBM bytes per launch (FETCH_SIZE + WRITE_SIZE),
    # mean kernel-trace durations, MFMA busy fractions
    stored = args.workload == "lm_c4" and args.fused_out_proj == "on"
    traffic = stored_metric(TRAFFIC_SUMMARY, "traffic_bytes_per_launch") if stored else {}
    prof_us = stored_metric(STATS_SUMMARY, "timed_us") if stored else {}
    graph_us = stored_metric(STATS_SUMMARY, "graph_us") if stored else {}
    mfma = stored_metric(MFMA_SUMMARY, "mfma_busy") if stored else {}
    for k, v in kernels.items():
        if k in prof_us:
            v["profile_us"] = prof_us[k]
        if k in graph_us:
            v["graph_us"] = graph_us[k]
        if k in mfma:
            v["mfma_busy"] = mfma[k]
    roofline = roofline_of(kernels["slot_gate"], traffic.get("slot_gate"), prof_us.get("slot_gate"))
    # the slot operator as a whole (state pre-pass, segment scan, gate pass) against the
    # gate pass's algorithmic bytes (q, k, v, gate read once, output written once)
    roofline_slot_op = None
    if "slot_op" in kernels:
        parts = ("slot_state", "slot_scan", "slot_gate")
        op_traffic = sum(traffic[p] for p in parts) if all(p in traffic for p in parts) else None
        op_us = round(sum(prof_us[p] for p in parts), 2) if all(p in prof_us for p in parts) else None
        roofline_slot_op = roofline_of(kernels["slot_op"], op_traffic, op_us)
    # the fused out_proj (LayerNorm folded into the GEMM) is the largest kernel of this build by
    # time; it is MFMA-bound, so its roofline is FLOPs against the bf16 dense peak
    roofline_out_proj = None
    if "out_proj" in kernels:
        roofline_out_proj = roofline_of(kernels["out_proj"], traffic.get("out_proj"), prof_us.get("out_proj"))
        if "out_proj" in mfma:
            roofline_out_proj["mfma_busy"] = mfma["out_proj"]

    forward_summary = None
    if args.workload.startswith("lm"):
        fl, by = forward_totals(cfg, args.fused_out_proj == "on")
        sec_step = ms_per_step * 1e-3
        forward_summary = {"TFLOP": round(fl / 1e12, 2), "TFLOP/s": round(fl / sec_step / 1e12, 1),
                           "frac_bf16_mfma_peak": round(fl / sec_step / 2.5e15, 4),
                           "GB": round(by / 1e9, 2), "GB/s": round(by / sec_step / 1e9, 1),
                           "frac_hbm_peak": round(by / sec_step / 8e12, 4)}

    cpu = None
    if args.cpu_baseline == "on":
        cpu = (cpu_baseline(model, inp, cfg, runs=args.cpu_runs) if args.workload.startswith("lm")
               else cpu_baseline_block(model, inp, cfg))

    out = {
        "metric": "forward tokens/sec on 1 MI355X at L=32768; achieved HBM GB/s % of peak",
        "value": round(value, 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": cfg["dtype_name"],
        "data": "synthetic: uniform random token ids / N(0,1) inputs, random-init weights",
        "config": {"workload": workload, "d_model": cfg["d_model"], "d_state": cfg["d_state"],
                   "num_heads": cfg["num_heads"], "chunk": cfg["chunk"], "layers": cfg.get("n_layers", 1),
                   "vocab": 50304 if args.workload.startswith("lm") else None,
                   "global_batch": cfg["B"], "seq_len": cfg["L"], "parallelism": "none (1 GPU)",
                   "fused_out_proj": args.fused_out_proj == "on"},
        "roofline": dict(kernel="slot_gate (slot memory + GroupNorm + gate pass)", **roofline),
        "roofline_slot_op": (dict(kernel="slot operator: slot_state + slot_scan + slot_gate", **roofline_slot_op)
                             if roofline_slot_op else None),
        "roofline_out_proj": (dict(kernel="rowln_gemm: out_proj with the folded LayerNorm and the residual",
                                   **roofline_out_proj) if roofline_out_proj else None),
        "cpu_baseline": cpu,
        "kernels": kernels,
        "forward": forward_summary,
        "timing": {"steps": "HIP graph replays of the whole forward" if use_graph else "eager forwards",
                   "kernels": (f"HIP events recorded by each custom kernel's own dispatch (begin and end "
                               f"timestamps, hipExtLaunchKernel) over {k_steps} eager forwards with the scan in "
                               f"sequence with the slot kernels (as in the recorded graph); mean per launch. "
                               f"profile_us: the same launches in the committed kernel trace; graph_us: that "
                               f"trace's graph replays"),
                   "eager_ms_per_step": round(eager_ms, 3)},
        "gemm_solutions": (f"TunableOp file, {n_tuned} recorded GEMM signatures" if n_tuned
                           else "library default heuristics"),
        "gpu": torch.cuda.get_device_name(0),
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
