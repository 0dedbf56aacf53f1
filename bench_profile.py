"""Per-stage figures of the Arctic forward from rocprofv3 output.

Subcommands:

    python bench_profile.py run
        One forward of the bench workload (config 5) plus one elementwise
        multiply that reads and writes CAL_BYTES, for `rocprofv3
        --kernel-trace` or `--pmc FETCH_SIZE` / `--pmc WRITE_SIZE` to
        observe (the program goes right after `--`).

    python bench_profile.py summarize [--trace DIR] [--fetch DIR] [--write DIR]
        Reads the CSV output of those runs and prints a markdown summary with
        one row per forward stage, ending in a fenced JSON block that
        bench.py reads for `roofline.traffic`.

    python bench_profile.py gemm
        The config-3 GEMM pair (T = 65536: 384 -> 1536 + GELU, then
        1536 -> 384 + residual + LayerNorm; f32 activations, int8 weights,
        through tzh_linear_w8) three times, for `rocprofv3` passes.

    python bench_profile.py counters DIR [DIR ...]
        Per-kernel averages of the counters in those runs' CSV output, with
        unit busy/stall fractions (see COUNTER_NOTES).

Dispatches are mapped to forward stages by kernel and launch order: both
LayerNorm GEMMs are linear_pipe_kernel<2> (with f32 activations the k = 384
one has a tile configuration of its own); the one launched after attention
is attn_out_ln and the one after ffn1_gelu is ffn2_ln; mlp_fused_kernel, the
fused feed-forward block, is the stage ffn, in its O-projection mode
(template argument 1) the stage attn_ffn and in its QKV mode (2) the stage
qkv; mlp_tail_kernel, which finishes the rows of a split last round,
belongs to the stage before it.  The
pieces of a split partial round (the residual-only GEMM) and their row
LayerNorm belong to the LayerNorm GEMM launched just before them.

FETCH_SIZE and WRITE_SIZE (KiB per dispatch, summed over the L2 channels)
are scaled by what they read for the calibration multiply, whose true traffic
is CAL_BYTES read and CAL_BYTES written.
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import re
import sys

CAL_BYTES = 1 << 30
STAGES = ("pack_ids", "embed_ln", "qkv", "attention", "attn_out_ln", "attn_ffn", "ffn", "ffn1_gelu", "ffn2_ln",
          "cls_l2")


def epi_of(kernel: str) -> int | None:
    """Epilogue template argument of a linear_pipe_kernel dispatch (mangled
    or demangled name), None for other kernels."""
    m = re.search(r"linear_pipe_kernelILi(\d)E|linear_pipe_kernel<(\d),", kernel)
    if not m:
        return None
    return int(m.group(1) or m.group(2))


def stage_of(kernel: str, prev: str | None) -> str | None:
    """Forward stage of a dispatch of `kernel`, given the previous stage."""
    if "pack_ids_kernel" in kernel:
        return "pack_ids"
    if "embed_ln_kernel" in kernel:
        return "embed_ln"
    if "attn_varlen_kernel" in kernel or "attn_varlen_f32_kernel" in kernel:
        return "attention"
    if "cls_l2_kernel" in kernel:
        return "cls_l2"
    if "mlp_fused_kernel" in kernel:
        # the template mode (mangled ...kernelILi<mode>E...): 1 the O-projection
        # mode, 2 the QKV mode, 0 the feed-forward block alone
        if "ILi1E" in kernel or "<1>" in kernel:
            return "attn_ffn"
        return "qkv" if ("ILi2E" in kernel or "<2>" in kernel) else "ffn"
    if "mlp_tail_kernel" in kernel:  # the rows of the fused kernel's split last round
        return prev if prev in ("attn_ffn", "ffn") else None
    epi = epi_of(kernel)
    if epi == 0:
        return "qkv"
    if epi == 1:
        return "ffn1_gelu"
    if epi == 2:  # (after its own stage: a repeated launch of a timing forward)
        return ("attn_out_ln" if prev == "attention" else "ffn2_ln" if prev == "ffn1_gelu"
                else prev if prev in ("attn_out_ln", "ffn2_ln") else None)
    if epi == 3 or "ln_rows_kernel" in kernel:
        return prev if prev in ("attn_out_ln", "ffn2_ln") else None
    return None


def _rows(directory: str, suffix: str) -> list[dict]:
    files = sorted(glob.glob(os.path.join(directory, "**", f"*{suffix}"), recursive=True))
    if not files:
        raise FileNotFoundError(f"no *{suffix} under {directory}")
    rows = []
    for f in files:
        with open(f, newline="") as fh:
            rows.extend(csv.DictReader(fh))
    return rows


def _instances(seq):
    """Groups (kernel name, value) dispatches in launch order into stage
    instances per forward precision: {"fp32" | "fp16": {stage: [summed
    value of each instance]}}.  A forward runs from one pack_ids dispatch to
    the next; its precision is that of its attention kernel.  A dispatch that
    continues the previous stage (the pieces of a split LayerNorm round, the
    fused kernel's split-round rows) adds to that stage's current instance.  Forwards that launch a stage
    twice in a row (bench.py's per-launch timing forwards repeat each stage)
    are left out, so that instances and averages are those of plain
    forwards."""
    out = {}
    fwd, prec, prev, repeated = {}, None, None, False

    def flush():
        if prec is not None and not repeated:
            tgt = out.setdefault(prec, {})
            for k, v in fwd.items():
                tgt.setdefault(k, []).extend(v)

    for name, v in seq:
        st = stage_of(name, prev)
        if st is None:
            continue
        if st == "pack_ids":
            flush()
            fwd, prec, repeated = {}, None, False
        if st == "attention":
            prec = "fp32" if "attn_varlen_f32_kernel" in name else "fp16"
        if st == prev and (epi_of(name) == 3 or "ln_rows_kernel" in name or "mlp_tail_kernel" in name):
            fwd[st][-1] += v
        else:
            repeated = repeated or st == prev
            fwd.setdefault(st, []).append(v)
        prev = st
    flush()
    return out


def trace_stats(directory: str) -> dict:
    """{precision: {stage: (instances, average microseconds of kernel time
    per instance)}} from a kernel trace."""
    rows = sorted(_rows(directory, "kernel_trace.csv"), key=lambda r: int(r["Dispatch_Id"]))
    acc = _instances((r["Kernel_Name"], (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-3) for r in rows)
    return {p: {k: (len(v), sum(v) / len(v)) for k, v in a.items()} for p, a in acc.items()}


def counter_stats(directory: str, counter: str) -> tuple[dict, float]:
    """({stage: average counter value per stage instance}, the calibration multiply's value)."""
    per_dispatch = {}
    for r in _rows(directory, "counter_collection.csv"):
        if r["Counter_Name"] != counter:
            continue
        d = int(r["Dispatch_Id"])
        name, v = per_dispatch.get(d, (r["Kernel_Name"], 0.0))
        per_dispatch[d] = (name, v + float(r["Counter_Value"]))
    cal = 0.0
    for d in sorted(per_dispatch):
        name, v = per_dispatch[d]
        if "elementwise_kernel" in name:  # the calibration multiply (and torch's fills)
            cal = max(cal, v)
    acc = _instances(per_dispatch[d] for d in sorted(per_dispatch))
    return {p: {k: sum(v) / len(v) for k, v in a.items()} for p, a in acc.items()}, cal


COMMANDS = """Commands (on one MI355X; rocprofv3 runs from /tmp with TMPDIR=/tmp and
PYTHONPATH=<repo>, the program right after `--`):

    rocprofv3 --kernel-trace --stats --output-format csv -d <out>/trace -o fwd -- \\
        python3 <repo>/bench.py --steps 5 --warmup 2 --no-cpu-baseline --forward-only > <out>/trace.log
    rocprofv3 --pmc FETCH_SIZE --output-format csv -d <out>/fetch -o f -- \\
        python3 <repo>/bench_profile.py run
    rocprofv3 --pmc WRITE_SIZE --output-format csv -d <out>/write -o w -- \\
        python3 <repo>/bench_profile.py run
    python3 <repo>/bench_profile.py summarize \\
        --trace <out>/trace --fetch <out>/fetch --write <out>/write --bench-log <out>/trace.log
"""


def kernel_stats_table(directory: str, top: int = 10) -> list[str]:
    """rocprofv3's --stats kernel summary as a markdown table."""
    rows = _rows(directory, "kernel_stats.csv")
    rows.sort(key=lambda r: -float(r["TotalDurationNs"]))
    out = ["| kernel | calls | avg us | total ms | % |", "|---|---:|---:|---:|---:|"]
    for r in rows[:top]:
        out.append(f"| `{r['Name'][:96]}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.1f} | "
                   f"{float(r['TotalDurationNs']) / 1e6:.2f} | {float(r['Percentage']):.1f} |")
    return out


def forward_sum_us(stages: dict) -> float | None:
    """Kernel time of one forward: every stage's average times its launches
    per forward (pack_ids runs once per forward)."""
    n_fwd = (stages.get("pack_ids") or {}).get("instances") or 0
    if not n_fwd:
        return None
    return sum(v["avg_us"] * v["instances"] / n_fwd for v in stages.values() if v["instances"] and v["avg_us"])


def bench_line(path: str | None) -> dict:
    """The JSON line a bench.py run printed into `path` ({} if none)."""
    if not path:
        return {}
    try:
        for line in open(path):
            if line.startswith("{") and '"metric"' in line:
                return json.loads(line)
    except OSError:
        pass
    return {}


def summarize(trace: str | None, fetch: str | None, write: str | None, bench_log: str | None = None) -> str:
    out = ["# Per-stage profile: int8 Arctic-embed-xs forward, batch 256 x seq 512", "", COMMANDS]
    data: dict = {}
    times = trace_stats(trace) if trace else {}
    f_stats, f_cal = counter_stats(fetch, "FETCH_SIZE") if fetch else ({}, 0.0)
    w_stats, w_cal = counter_stats(write, "WRITE_SIZE") if write else ({}, 0.0)
    cal_kib = CAL_BYTES / 1024.0
    f_scale = cal_kib / f_cal if f_cal else None
    w_scale = cal_kib / w_cal if w_cal else None
    if fetch or write:
        out.append(f"Calibration: an elementwise multiply over {CAL_BYTES} bytes read FETCH_SIZE {f_cal:.0f} KiB "
                   f"(scale {f_scale if f_scale is None else round(f_scale, 4)}) and WRITE_SIZE {w_cal:.0f} KiB "
                   f"(scale {w_scale if w_scale is None else round(w_scale, 4)}); per-stage bytes below are "
                   "counter x scale.")
        out.append("")
    for prec in ("fp32", "fp16"):
        t = times.get(prec, {})
        fs, ws = f_stats.get(prec, {}), w_stats.get(prec, {})
        if not (t or fs or ws):
            continue
        key = "stages" if prec == "fp32" else "stages_fp16"
        data[key] = {}
        out.append(f"{prec} forward ({'the default: f32 activations' if prec == 'fp32' else 'opt-in f16 activations'}):")
        out.append("")
        out.append("| stage | instances | avg us | HBM read MB | HBM write MB |")
        out.append("|---|---:|---:|---:|---:|")
        for st in STAGES:
            n, us = t.get(st, (0, float("nan")))
            if n == 0 and st not in fs and st not in ws:
                continue  # a stage this precision does not run (fused or split feed-forward)
            rd = fs[st] * 1024 * f_scale if st in fs and f_scale else None
            wr = ws[st] * 1024 * w_scale if st in ws and w_scale else None
            data[key][st] = {"instances": n, "avg_us": None if n == 0 else round(us, 2),
                             "read_bytes": None if rd is None else int(rd),
                             "write_bytes": None if wr is None else int(wr)}
            out.append(f"| {st} | {n} | {us:.1f} | {'' if rd is None else f'{rd / 1e6:.1f}'} | "
                       f"{'' if wr is None else f'{wr / 1e6:.1f}'} |")
        out.append("")
    data["calibration"] = {"bytes": CAL_BYTES, "fetch_kib": f_cal, "write_kib": w_cal}
    b = bench_line(bench_log)
    if trace and b:
        # rocprofv3's kernel times against the bench's own clock, same process
        steps = {"fp32": b.get("ms_per_step"), "fp16": (b.get("fp16_forward") or {}).get("ms_per_step")}
        out.append("Reconciliation with the bench line of the same trace run (kernel times summed per "
                   "forward against the bench's timed step):")
        out.append("")
        out.append("| forward | kernel sum per forward, ms | bench ms_per_step | kernel sum / step |")
        out.append("|---|---:|---:|---:|")
        for prec, key in (("fp32", "stages"), ("fp16", "stages_fp16")):
            tot = forward_sum_us(data.get(key, {}))
            st = steps[prec]
            if tot and st:
                out.append(f"| {prec} | {tot / 1000:.3f} | {st:.3f} | {tot / 1000 / st:.3f} |")
        out.append("")
        data["reconciliation"] = {prec: {"kernel_sum_ms": round((forward_sum_us(data.get(key, {})) or 0) / 1000, 4),
                                         "ms_per_step": steps[prec]}
                                  for prec, key in (("fp32", "stages"), ("fp16", "stages_fp16"))}
    if trace:
        out += ["The fp32 forward runs each layer's O-projection, its LayerNorm and the feed-forward",
                "block as one kernel (mlp_fused_kernel<1>, stage attn_ffn, with mlp_tail_kernel for a",
                "split last round) and its QKV projection on the same kernel's QKV mode",
                "(mlp_fused_kernel<2>, stage qkv); the fp16 forward runs linear_pipe_kernel for QKV,",
                "the O-projection and the GEMM pair (attn_out_ln, ffn1_gelu, ffn2_ln), whose two",
                "LayerNorm GEMMs are both linear_pipe_kernel<2>; the rows above separate them by",
                "launch order.  The stage rows average the plain forwards of the trace run.  The",
                "counter runs (bench_profile.py run) make one fp32 forward.  rocprofv3's own kernel",
                "summary of the trace run (bench.py: the fp16 forward first, 5 timed + 2 warmup, then",
                "the fp32 one, 5 timed + 2 warmup + 3 with per-launch events, which issue each stage",
                "10 times back to back):", ""]
        out += kernel_stats_table(trace)
    out += ["", "```json", json.dumps(data, indent=1), "```", ""]
    return "\n".join(out)


def load_traffic(path: str) -> dict:
    """The JSON block of a summary written by `summarize` ({} if absent)."""
    try:
        text = open(path).read()
    except OSError:
        return {}
    start = text.find("```json")
    if start < 0:
        return {}
    end = text.find("```", start + 7)
    return json.loads(text[start + 7:end])


def run() -> None:
    import numpy as np
    import torch

    import tenzor_amd
    from tenzor_amd import synth
    from tenzor_amd.arctic import ModelWeights, forwardBatch

    cfg = synth.Config()
    ctx = tenzor_amd.Context(0)
    model = ModelWeights.fromHost(ctx, synth.quantize(synth.make_arctic_f32(1, cfg)), cfg)
    ids, lengths = synth.make_batch(5, 256, 512)
    d_ids = torch.from_numpy(ids.view(np.int32)).cuda()
    out = torch.empty((256, cfg.hidden_size), device="cuda")
    forwardBatch(out, d_ids, lengths, model)
    torch.cuda.synchronize()
    src = torch.ones(CAL_BYTES // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    torch.mul(src, 2.0, out=dst)  # reads and writes CAL_BYTES
    torch.cuda.synchronize()
    print("forward and calibration multiply done", flush=True)


def gemm() -> None:
    """Config 3 three times: f32 X [65536, 384] -> 1536 + GELU (f32), then
    1536 -> 384 + residual (X) + LayerNorm (f32); int8 weights."""
    import ctypes as C

    import numpy as np
    import torch

    import tenzor_amd
    from tenzor_amd import _abi, check, lib

    ctx = tenzor_amd.Context(0)
    T, K, N1 = 65536, 384, 1536
    rng = np.random.default_rng(9)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    X = dev(rng.standard_normal((T, K)).astype(np.float32))
    H = torch.empty((T, N1), dtype=torch.float32, device="cuda")
    Y = torch.empty((T, K), dtype=torch.float32, device="cuda")
    Q1 = dev(rng.integers(-127, 128, size=(N1, K)).astype(np.int8))
    Q2 = dev(rng.integers(-127, 128, size=(K, N1)).astype(np.int8))
    S1 = dev(np.full(N1, 0x211F, np.int16))  # f16 0.01
    S2 = dev(np.full(K, 0x211F, np.int16))
    B1, B2 = dev(np.zeros(N1, np.float32)), dev(np.zeros(K, np.float32))
    G, Bt = dev(np.ones(K, np.float32)), dev(np.zeros(K, np.float32))
    for _ in range(3):
        check(lib().tzh_linear_w8(ctx.handle, X.data_ptr(), _abi.F32, Q1.data_ptr(), S1.data_ptr(), B1.data_ptr(),
                                  H.data_ptr(), _abi.F32, T, K, N1, _abi.EPI_BIAS_GELU, None, _abi.F32, None, None,
                                  0.0))
        check(lib().tzh_linear_w8(ctx.handle, H.data_ptr(), _abi.F32, Q2.data_ptr(), S2.data_ptr(), B2.data_ptr(),
                                  Y.data_ptr(), _abi.F32, T, N1, K, _abi.EPI_BIAS_RES_LN, X.data_ptr(), _abi.F32,
                                  G.data_ptr(), Bt.data_ptr(), C.c_float(1e-12)))
    torch.cuda.synchronize()
    print("config-3 GEMM pair done", flush=True)


def nodes() -> None:
    """Times the eval node kinds (softmax, layernorm, transpose) at sizes
    well above the caches and prints HBM throughput by algorithmic bytes
    (each element read once and written once)."""
    import numpy as np
    import torch

    from tenzor_amd.expr import LayerNormExpr, Tensor, evalInto

    rng = np.random.default_rng(0)
    x = Tensor(torch.from_numpy(rng.standard_normal((16384, 4096)).astype(np.float32)).cuda())
    g = Tensor(torch.ones(4096, device="cuda"))
    b = Tensor(torch.zeros(4096, device="cuda"))
    a = Tensor(torch.from_numpy(rng.standard_normal((64, 512, 12, 32)).astype(np.float32)).cuda())
    cases = [("softmax last axis [16384, 4096] f32", x.softmax(-1), x.numel()),
             ("softmax axis 0 [16384, 4096] f32", x.softmax(0), x.numel()),
             ("layernorm last dim [16384, 4096] f32", LayerNormExpr(x, g, b, 1), x.numel()),
             ("transpose 0213 [64, 512, 12, 32] f32", a.transpose((0, 2, 1, 3)), a.numel())]
    for name, e, n in cases:
        out = torch.empty(e.shape, device="cuda")
        for _ in range(3):
            evalInto(e, out)
        torch.cuda.synchronize()
        s, t = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(20):
            evalInto(e, out)
        t.record()
        torch.cuda.synchronize()
        us = s.elapsed_time(t) / 20 * 1e3
        print(f"{name}: {us:.1f} us, {2 * n * 4 / us / 1e3:.0f} GB/s", flush=True)


# MI355X: 8 XCDs of 32 CUs, 4 SIMDs per CU.  GRBM_GUI_ACTIVE is summed over
# the XCDs; TA/TD/TCP `_sum` counters over one instance per CU; the SQ
# cycle counters over the SIMDs (MFMA busy) or the CUs (LDS active).
COUNTER_NOTES = {
    "TA_TA_BUSY_sum": ("TA busy", 256),
    "TD_TD_BUSY_sum": ("TD busy", 256),
    "TD_TC_STALL_sum": ("TD stalled by the L1 (TC)", 256),
    "TA_ADDR_STALLED_BY_TC_CYCLES_sum": ("TA address stalled by the L1", 256),
    "TCP_PENDING_STALL_CYCLES_sum": ("L1 waiting for L2 data", 256),
    "SQ_VALU_MFMA_BUSY_CYCLES": ("MFMA busy (per SIMD)", 1024),
    "SQ_LDS_IDX_ACTIVE": ("LDS active (indexed ops)", 256),
}


def counters(dirs: list[str]) -> str:
    per = {}
    for d in dirs:
        disp = {}
        for r in _rows(d, "counter_collection.csv"):
            key = (r["Dispatch_Id"], r["Counter_Name"])
            disp[key] = (r["Kernel_Name"], disp.get(key, ("", 0.0))[1] + float(r["Counter_Value"]))
        for (did, cname), (kname, v) in disp.items():
            k = kname.replace("(anonymous namespace)::", "").split("(")[0][:150]
            per.setdefault(k, {}).setdefault(cname, {})[(d, did)] = v
    out = []
    for k, cs in per.items():
        if not any(x in k for x in ("linear_pipe_kernel", "ln_rows_kernel", "attn_varlen", "mlp_fused_kernel")):
            continue
        out.append(f"### `{k}`")
        out.append("")
        out.append("| counter | per dispatch | fraction of GPU-active cycles |")
        out.append("|---|---:|---:|")
        for cname in sorted(cs):
            vals = cs[cname]
            avg = sum(vals.values()) / len(vals)
            frac = ""
            if cname in COUNTER_NOTES:
                # GRBM_GUI_ACTIVE of the same dispatches (same pass)
                dispatches = list(vals)
                g = [cs.get("GRBM_GUI_ACTIVE", {}).get(dk) for dk in dispatches]
                g = [x for x in g if x]
                if g:
                    label, inst = COUNTER_NOTES[cname]
                    frac = f"{avg / inst / (sum(g) / len(g) / 8):.0%} ({label})"
            out.append(f"| {cname} | {avg:.4g} | {frac} |")
        out.append("")
    return "\n".join(out) + "\n"


def kernels(trace: str, fetch: str | None, write: str | None, fetch_scale: float, write_scale: float) -> str:
    """Per-kernel table of a run that is not a forward (config 2 or 3):
    average duration from the trace, FETCH_SIZE / WRITE_SIZE per dispatch
    times the calibration scales (measured in the forward's calibration
    multiply: 1 GiB read gives FETCH_SIZE 0.5 GiB, 1 GiB written WRITE_SIZE
    1 GiB)."""
    def norm(k):
        return k.replace("(anonymous namespace)::", "").split("(")[0][:120]

    times = {}
    for r in _rows(trace, "kernel_trace.csv"):
        times.setdefault(norm(r["Kernel_Name"]), []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-3)
    cnt = {}
    for d, counter in ((fetch, "FETCH_SIZE"), (write, "WRITE_SIZE")):
        if not d:
            continue
        per = {}
        for r in _rows(d, "counter_collection.csv"):
            if r["Counter_Name"] != counter:
                continue
            key = int(r["Dispatch_Id"])
            name, v = per.get(key, (norm(r["Kernel_Name"]), 0.0))
            per[key] = (name, v + float(r["Counter_Value"]))
        for name, v in per.values():
            cnt.setdefault(name, {}).setdefault(counter, []).append(v)
    out = ["| kernel | calls | avg us | HBM read MB | HBM write MB |", "|---|---:|---:|---:|---:|"]
    for k, v in sorted(times.items(), key=lambda kv: -sum(kv[1])):
        c = cnt.get(k, {})
        rd = sum(c["FETCH_SIZE"]) / len(c["FETCH_SIZE"]) * 1024 * fetch_scale / 1e6 if "FETCH_SIZE" in c else None
        wr = sum(c["WRITE_SIZE"]) / len(c["WRITE_SIZE"]) * 1024 * write_scale / 1e6 if "WRITE_SIZE" in c else None
        out.append(f"| `{k}` | {len(v)} | {sum(v) / len(v):.1f} | {'' if rd is None else f'{rd:.1f}'} | "
                   f"{'' if wr is None else f'{wr:.1f}'} |")
    return "\n".join(out) + "\n"


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    sub.add_parser("run")
    sub.add_parser("gemm")
    sub.add_parser("nodes")
    s = sub.add_parser("summarize")
    s.add_argument("--trace")
    s.add_argument("--fetch")
    s.add_argument("--write")
    s.add_argument("--bench-log", help="the output of the traced bench.py run (its JSON line)")
    c = sub.add_parser("counters")
    c.add_argument("dirs", nargs="+")
    k = sub.add_parser("kernels")
    k.add_argument("--trace", required=True)
    k.add_argument("--fetch")
    k.add_argument("--write")
    k.add_argument("--fetch-scale", type=float, default=2.0)
    k.add_argument("--write-scale", type=float, default=1.0)
    a = ap.parse_args(argv)
    if a.cmd == "run":
        run()
    elif a.cmd == "gemm":
        gemm()
    elif a.cmd == "nodes":
        nodes()
    elif a.cmd == "counters":
        sys.stdout.write(counters(a.dirs))
    elif a.cmd == "kernels":
        sys.stdout.write(kernels(a.trace, a.fetch, a.write, a.fetch_scale, a.write_scale))
    else:
        sys.stdout.write(summarize(a.trace, a.fetch, a.write, a.bench_log))
    return 0


if __name__ == "__main__":
    sys.exit(main())
