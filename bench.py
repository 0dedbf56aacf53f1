"""Headline benchmark: int8 Arctic-embed-xs forward, batch 256 x seq 512
(lengths U[16,512], padded with id 0), CLS pooling + L2, on one MI355X, in
the reference's f32 arithmetic.

    python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--no-cpu-baseline]
    python bench.py --precision fp16         # the opt-in f16-activation forward
    python bench.py --workload chain         # config 2: exp((A + b) * c), 16384^2
    python bench.py --workload gemm3         # config 3: the int8 GEMM pair, T = 65536
    python bench.py --workload embed-docs    # the embed command's document path

Prints one JSON line.  A step is one forward of the whole batch with the
padded token ids already resident in HBM; `value` counts real (unpadded)
tokens.  `roofline` describes the dominant kernel (by total time in the
forward), timed inside the forward with HIP events recorded around every
launch on the forward's own stream; `cpu_baseline` times the C restatement of the reference's
batch-parallel CPU forward (forwardBatchParallel) on a sample of the same
batch on the host cores.  The default (forward) line also carries `chain`
and `gemm3`: configs 2 and 3 measured in the same run (value, time per
step, roofline fraction of their kernels and their own CPU baselines), the
same figures their own workloads print.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0      # MI355X HBM3E
F16_PEAK_TFLOPS = 2500.0   # MI355X dense fp16 MFMA
SEED_WEIGHTS, SEED_BATCH = 1, 5
BATCH, SEQ = 256, 512
TRAFFIC_PROFILE = "arctic_b256_stage_profile.md"


KERNELS = {
    # f32 forward: the fused kernel's QKV mode (X in registers, weights streamed through LDS); fp16:
    # linear_pipe_kernel
    "qkv": "mlp_fused_kernel<2> (fp32; linear_pipe_kernel with --precision fp16): bias, 384 -> 1152",
    "attention": "attn_varlen_f32_kernel (attn_varlen_kernel with --precision fp16)",
    "attn_out_ln": "linear_pipe_kernel bias+residual+LayerNorm, 384 -> 384, 64-row tiles, two workgroups per CU",
    "ffn1_gelu": "linear_pipe_kernel bias+GELU, 384 -> 1536",
    "ffn2_ln": "linear_pipe_kernel bias+residual+LayerNorm, 1536 -> 384, + split last round "
               "(linear_pipe_kernel residual pieces, ln_rows_kernel)",
    "ffn": "mlp_fused_kernel: the feed-forward block in one kernel, 384 -> 1536 + GELU -> 384 + residual + "
           "LayerNorm, the intermediate kept on chip",
    "attn_ffn": "mlp_fused_kernel<1>: O-projection 384 -> 384 + residual + LayerNorm, then the feed-forward "
                "block (384 -> 1536 + GELU -> 384 + residual + LayerNorm) in one kernel, h1 and the intermediate "
                "kept on chip",
    "embed_ln": "embed_ln_kernel", "pack_ids": "pack_ids_kernel", "cls_l2": "cls_l2_kernel",
}


TIMING_REPS = 10  # launches of each stage between two events in the per-stage timing


def host_facts():
    """(threads the CPU baseline uses, nproc, CPU model).  The threads are the
    CPUs this process may run on, at most 16: the GPU box's CPU share for
    one GPU."""
    nproc = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return min(16, nproc), nproc, model


def load_traffic(path: str) -> dict:
    """The JSON block of a profile summary written by bench_profile.py
    (its `summarize` subcommand); {} if absent."""
    try:
        text = open(path).read()
    except OSError:
        return {}
    start = text.find("```json")
    if start < 0:
        return {}
    end = text.find("```", start + 7)
    return json.loads(text[start + 7:end])


def stage_work(T, lengths, es=4):
    """Algorithmic (flops, HBM bytes) of one launch of each forward stage.

    Bytes follow the reference's op boundaries in f32 (the per-token figures
    of the measurement plan: QKV 6144, attention core 6144, O-proj + residual
    + LayerNorm 4608, FFN1 + GELU 7680, FFN2 + residual + LayerNorm 9216,
    embeddings 4608 bytes per token) plus the int8 weights, f16 scales and
    f32 biases the launch reads.  The f32 forward moves exactly those
    activation bytes; the f16 one about half (bytes_moved, es = 2)."""
    H, I = 384, 1536
    w = {}
    for name, K, N, per_tok, res in (("qkv", H, 3 * H, 6144, False), ("attn_out_ln", H, H, 4608, True),
                                     ("ffn1_gelu", H, I, 7680, False), ("ffn2_ln", I, H, 9216, True)):
        weights = N * K + N * (2 + 4) + (2 * N * 4 if res else 0)
        moved = T * K * es + T * N * es + (T * N * es if res else 0) + weights
        w[name] = (2.0 * T * K * N, float(T * per_tok + weights), float(moved))
    # the fused feed-forward block: the two linears' op-boundary bytes (the
    # reference writes and re-reads the intermediate); it moves X in, Y out,
    # X again as the residual, and reads its f16 weight pack
    f1, f2 = w["ffn1_gelu"], w["ffn2_ln"]
    w["ffn"] = (f1[0] + f2[0], f1[1] + f2[1], float(3 * T * H * es + 2 * (2 * H * I)))
    # ... preceded by the O-projection + LayerNorm (op-boundary bytes of the
    # three linears; it moves the context and h in and h out)
    o = w["attn_out_ln"]
    w["attn_ffn"] = (o[0] + f1[0] + f2[0], o[1] + f1[1] + f2[1], float(3 * T * H * es + 2 * (2 * H * I + H * H)))
    L2 = float((lengths.astype(np.float64) ** 2).sum())
    # per head QK^T and PV: 2 * L^2 * 32 flops each; 12 heads
    w["attention"] = (4.0 * L2 * H, float(T * 6144), float(T * 3 * H * es + T * H * es))
    # word/position/type rows (f32) gathered per token, LayerNorm, one row out
    w["embed_ln"] = (0.0, float(T * 4608), float(T * H * 4 * 3 + T * H * es))
    w["pack_ids"] = (0.0, float(T * 4 * 3), float(T * 4 * 3))
    w["cls_l2"] = (0.0, float(len(lengths) * H * (4 + 4)), float(len(lengths) * H * (es + 4)))
    return w


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--forward-only", action="store_true",
                    help="leave configs 2 and 3 out of the forward line (for kernel traces of the forward alone)")
    ap.add_argument("--cpu-sample-stride", type=int, default=1, help="every k-th sequence of the batch")
    ap.add_argument("--workload", choices=["forward", "chain", "gemm3", "embed-docs"], default="forward")
    ap.add_argument("--precision", choices=["fp32", "fp16"], default="fp32",
                    help="forward activations: fp32 (the reference's arithmetic) or the opt-in fp16")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the forward is data-parallel over "
              "sequences and multi-GPU runs are not part of this build", file=sys.stderr)
        sys.exit(2)

    import torch

    import tenzor_amd
    from tenzor_amd import synth
    from tenzor_amd.arctic import ModelWeights, forwardBatch

    assert torch.cuda.is_available(), "bench.py needs the GPU"
    if args.workload == "embed-docs":
        return embed_docs(args)
    if args.workload == "chain":
        print(json.dumps(chain(args)), flush=True)
        return
    if args.workload == "gemm3":
        print(json.dumps(gemm3(args)), flush=True)
        return
    cfg = synth.Config()
    weights = synth.quantize(synth.make_arctic_f32(SEED_WEIGHTS, cfg))  # N(0,0.02), gamma 1, beta 0
    ctx = tenzor_amd.Context(0)
    model = ModelWeights.fromHost(ctx, weights, cfg)
    ids, lengths = synth.make_batch(SEED_BATCH, BATCH, SEQ)
    d_ids = torch.from_numpy(ids.view(np.int32)).cuda()
    out = torch.empty((BATCH, cfg.hidden_size), device="cuda")
    real_tokens = int(lengths.sum())

    def timed_steps(steps, warmup):
        for _ in range(warmup):
            forwardBatch(out, d_ids, lengths, model)
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(steps):
            forwardBatch(out, d_ids, lengths, model)
        e.record()
        torch.cuda.synchronize()
        return s.elapsed_time(e) * 1e-3

    # the other precision first (a labelled extra), then the measured one
    other = "fp16" if args.precision == "fp32" else "fp32"
    model.set_precision("float16" if other == "fp16" else "float32")
    other_s = timed_steps(max(5, args.steps // 2), 2)
    other_steps = max(5, args.steps // 2)
    model.set_precision("float32" if args.precision == "fp32" else "float16")
    elapsed = timed_steps(args.steps, args.warmup)
    ms_per_step = elapsed / args.steps * 1e3
    value = real_tokens * args.steps / elapsed
    assert torch.isfinite(out).all()

    # per-kernel durations inside the forward: HIP events around every stage
    # on the forward's own stream (tzh_arctic_set_timing), each stage issued
    # TIMING_REPS times back to back between its events so that the cost of
    # an event (a dispatch wait after each, about 15-20 us) is spread over
    # the repetitions, as in a forward's own back-to-back launches
    model.set_timing(True, reps=TIMING_REPS)
    per_stage = {}
    n_timed = 3
    for _ in range(n_timed):
        forwardBatch(out, d_ids, lengths, model)
        for name, us in model.launch_times():
            per_stage.setdefault(name, []).append(us)
    model.set_timing(False)
    T = real_tokens
    es = 4 if args.precision == "fp32" else 2
    work = stage_work(T, lengths, es)
    stages = {}
    for name, v in per_stage.items():
        launches_per_fwd = len(v) // n_timed
        avg_us = sum(v) / len(v)
        flops, byts, byts16 = work.get(name, (0.0, 0.0, 0.0))
        roof_us = max(flops / (F16_PEAK_TFLOPS * 1e12), byts / (HBM_PEAK_GBS * 1e9)) * 1e6
        stages[name] = dict(avg_us=avg_us, launches=launches_per_fwd, total_us=avg_us * launches_per_fwd,
                            flops=flops, bytes=byts, bytes16=byts16, roof_us=roof_us,
                            bound="mfma" if flops / (F16_PEAK_TFLOPS * 1e12) > byts / (HBM_PEAK_GBS * 1e9) else "hbm")
    dom_name = max(stages, key=lambda k: stages[k]["total_us"])
    dom = stages[dom_name]
    secs = dom["avg_us"] * 1e-6
    if dom["bound"] == "hbm":
        achieved, peak, unit = dom["bytes"] / secs / 1e9, HBM_PEAK_GBS, "GB/s"
    else:
        achieved, peak, unit = dom["flops"] / secs / 1e12, F16_PEAK_TFLOPS, "TFLOP/s"
    fwd_roof_us = sum(st["roof_us"] * st["launches"] for st in stages.values())
    # HBM bytes per launch of that stage, measured by rocprofv3 FETCH_SIZE and
    # WRITE_SIZE passes over the same workload (calibrated against a known
    # copy; see bench_profile.py) and committed with the profile
    measured = load_traffic(os.path.join(ROOT, "profiles", TRAFFIC_PROFILE)).get("stages", {}).get(dom_name, {})
    traffic = None
    if measured.get("read_bytes") is not None and measured.get("write_bytes") is not None:
        traffic = measured["read_bytes"] + measured["write_bytes"]

    line = {
        "metric": "tokens/sec int8 arctic-embed-xs b256 s512, 1 GPU; % of HBM/MFMA roofline",
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.precision,
        "arithmetic": ("f32 activations in HBM; every product of f32 operands on the MFMA from exact f16 hi/lo "
                       "splits (int8 codes exact in f16), f32 accumulation, f32 softmax/LayerNorm statistics"
                       if args.precision == "fp32" else
                       "opt-in: activations rounded to f16 between kernels, f16 MFMA operands, f32 accumulation"),
        "data": "synthetic",
        "config": {
            "workload": "int8-weight Arctic-embed-xs forward (6 layers, hidden 384, 12 heads, FFN 1536), "
                        "batch 256, seq 512 padded, lengths U[16,512], CLS + L2",
            "global_batch": BATCH,
            "seq_len": SEQ,
            "real_tokens_per_step": real_tokens,
            "padded_tokens_per_step": BATCH * SEQ,
            "weights": "int8 per-output-channel symmetric, f16 scales; embeddings/LayerNorm f32",
            "parallelism": "single GPU",
        },
        "roofline": {
            "kernel": f"{dom_name} ({KERNELS[dom_name]}, T={T})",
            "bound": dom["bound"],
            "achieved": round(achieved, 2),
            "peak": peak,
            "unit": unit,
            "frac": round(achieved / peak, 4),
            "traffic": traffic,
            "traffic_source": f"profiles/{TRAFFIC_PROFILE}" if traffic is not None else None,
            "avg_us": round(dom["avg_us"], 2),
            "algorithmic_bytes": int(dom["bytes"]),
            "algorithmic_flops": int(dom["flops"]),
            "bytes_moved": int(dom["bytes16"]),
            "moved_GBps": round(dom["bytes16"] / secs / 1e9, 1),
            # the f32 products run as f16 MFMAs on the hi/lo halves: two per
            # product in the GEMMs, three in attention; the matrix cores'
            # share of that work
            "mfma_frac_f32_split": round((3.0 if dom_name == "attention" else 2.0) * dom["flops"] / secs / 1e12 /
                                         F16_PEAK_TFLOPS, 4),
        },
        "forward_roofline_frac": round(fwd_roof_us / (ms_per_step * 1e3), 4),
        "stage_us": {k: round(v["avg_us"], 1) for k, v in stages.items()},
        "padded_equivalent_tokens_per_s": round(BATCH * SEQ * args.steps / elapsed, 1),
        f"{other}_forward": {"value": round(real_tokens * other_steps / other_s, 1), "unit": "tokens/s",
                             "ms_per_step": round(other_s / other_steps * 1e3, 4), "steps": other_steps},
    }

    if not args.no_cpu_baseline:
        import oracle

        threads, nproc, cpu_model = host_facts()
        sel = np.arange(0, BATCH, args.cpu_sample_stride)
        flat, offs = synth.packed(ids[sel], lengths[sel])
        hw = synth.HostWeights(weights, cfg)
        t0 = time.perf_counter()
        oracle.arctic_forward_batch(hw, flat, offs, lengths[sel], nthreads=threads)
        dt = time.perf_counter() - t0
        line["cpu_baseline"] = {
            "value": round(float(lengths[sel].sum()) / dt, 1),
            "unit": "tokens/s",
            "cores": threads,
            "nproc": nproc,
            "cpu": cpu_model,
            "kind": "port",
            "sample": f"{len(sel)} of the {BATCH} sequences (every {args.cpu_sample_stride}th, "
                      f"{int(lengths[sel].sum())} real tokens), C restatement of forwardBatchParallel "
                      f"(f32, OpenMP over sequences), {dt:.1f} s",
        }
    model.deinit()
    del d_ids, out
    torch.cuda.empty_cache()
    # configs 2 and 3 in the same run (their own workloads print the full
    # line): value, time per step, roofline fraction and CPU baseline each
    for name, fn in () if args.forward_only else (("chain", chain), ("gemm3", gemm3)):
        sub = fn(argparse.Namespace(steps=args.steps, warmup=args.warmup, no_cpu_baseline=args.no_cpu_baseline))
        line[name] = {k: sub[k] for k in ("metric", "value", "unit", "ms_per_step", "dtype", "config", "roofline")}
        if "kernels" in sub:
            line[name]["kernels"] = sub["kernels"]
        if "cpu_baseline" in sub:
            line[name]["cpu_baseline"] = sub["cpu_baseline"]
        torch.cuda.empty_cache()
    print(json.dumps(line), flush=True)


CHAIN_N = 16384
CHAIN_BYTES = 3 * CHAIN_N * CHAIN_N * 4 + CHAIN_N * 4  # A, c read, out written, b read once


def kernel_events(launch, reps):
    """Average device duration (us) of `launch()` bracketed by events on
    torch's current stream, the stream the library enqueues on (tzh_ctx made
    with the torch stream).  A GPU spin (torch.cuda._sleep) is queued ahead
    of each pair of events, so that the host's time to issue the launch (a
    Python call that builds and uploads its program) passes while the GPU
    spins instead of between the two events."""
    import torch

    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    for a, b in ev:
        torch.cuda._sleep(2_000_000)
        a.record()
        launch()
        b.record()
    torch.cuda.synchronize()
    return sum(a.elapsed_time(b) for a, b in ev) / reps * 1e3


def chain(args):
    """Config 2: out = exp((A + b) * c), A and c f32 [16384, 16384], b a row
    vector [16384] broadcast over rows, all U(-1, 1) from a seed; one
    tenzor.eval per step (one generated kernel, one pass over memory).
    The CPU baseline is the reference executor's three passes with two
    temporaries (executor.zig:49-196, restated in oracle.c), single-threaded
    as the executor is, on a band of rows."""
    import torch

    import tenzor_amd
    from tenzor_amd.expr import BinaryExpr, Tensor, evalInto

    n = CHAIN_N
    g = torch.Generator(device="cuda").manual_seed(12)
    A = torch.rand(n, n, device="cuda", generator=g) * 2 - 1
    b = torch.rand(n, device="cuda", generator=g) * 2 - 1
    c = torch.rand(n, n, device="cuda", generator=g) * 2 - 1
    out = torch.empty_like(A)
    ctx = tenzor_amd.Context(0)
    expr = BinaryExpr("add", Tensor(A), Tensor(b)).mul(Tensor(c)).exp()
    step = lambda: evalInto(expr, out, ctx)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(args.steps):
        step()
    e.record()
    torch.cuda.synchronize()
    elapsed = s.elapsed_time(e) * 1e-3
    assert bool(torch.isfinite(out).all())
    kern_us = kernel_events(step, 10)
    achieved = CHAIN_BYTES / (kern_us * 1e-6) / 1e9
    line = {
        "metric": "GB/s (algorithmic bytes), fused elementwise chain exp((A + b) * c), f32 16384^2, 1 GPU; "
                  "% of HBM roofline",
        "value": round(CHAIN_BYTES * args.steps / elapsed / 1e9, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic",
        "config": {"workload": "config 2: tenzor.eval of BinaryExpr(.add, A, b).mul(c).exp(), A, c f32 [16384, 16384], "
                               "b f32 [16384] broadcast over rows, U(-1, 1)", "parallelism": "single GPU",
                   "algorithmic_bytes": CHAIN_BYTES},
        "roofline": {"kernel": "tzh_chain (generated single-pass chain kernel)", "bound": "hbm",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None, "avg_us": round(kern_us, 2),
                     "algorithmic_bytes": CHAIN_BYTES},
    }
    if not args.no_cpu_baseline:
        import oracle

        _, nproc, cpu_model = host_facts()
        rows = 8192
        An, bn, cn = A[:rows].cpu().numpy(), b.cpu().numpy(), c[:rows].cpu().numpy()
        from tenzor_amd.expr import to_tape

        class _H:
            def __init__(self, a):
                self.a = a
                self.shape = a.shape
                self.dtype = torch.float32

            def is_contiguous(self):
                return True

        nodes, _ = to_tape(BinaryExpr("add", Tensor(_H(An)), Tensor(_H(bn))).mul(Tensor(_H(cn))).exp())
        t0 = time.perf_counter()
        rc, ref = oracle.eval_tape(nodes, [An, bn, cn], np.float32)
        dt = time.perf_counter() - t0
        assert rc == 0
        got = out[:rows].cpu().numpy()
        ulp = np.abs(got.view(np.int32).astype(np.int64) - ref.view(np.int32).astype(np.int64)).max()
        sample_bytes = 3 * rows * n * 4 + n * 4
        line["cpu_baseline"] = {
            "value": round(sample_bytes / dt / 1e9, 3), "unit": "GB/s", "cores": 1, "nproc": nproc, "cpu": cpu_model,
            "kind": "port",
            "sample": f"rows 0..{rows - 1} of A and c ({sample_bytes / 1e9:.2f} GB algorithmic), the executor's three "
                      f"passes with two temporaries (oracle.c), one thread; {dt:.1f} s; GPU vs CPU on the sample: "
                      f"max {int(ulp)} ulp",
        }
    ctx.close()
    return line


def gemm3(args):
    """Config 3: X f32 [65536, 384] N(0, 1) @ W1 int8 [1536, 384] + bias + GELU
    -> f32 [65536, 1536]; then @ W2 int8 [384, 1536] + bias + residual (X) +
    LayerNorm (eps 1e-12) -> f32 [65536, 384].  Codes U{-127..127}, scales
    U(0.001, 0.02) rounded to f16, biases U(-0.1, 0.1), gamma 1, beta 0.
    One step is the pair; `value` counts tokens (rows of X).  The CPU
    baseline is matmul_w8a32 + GELU + matmul_w8a32 + residual + LayerNorm
    restated in oracle.c, one thread (the reference's GEMM is
    single-threaded), on a sample of rows."""
    import ctypes as C

    import torch

    import oracle
    import tenzor_amd
    from tenzor_amd import _abi, check, lib

    T, K, N1 = 65536, 384, 1536
    rng = np.random.default_rng(3)
    X = torch.randn(T, K, generator=torch.Generator().manual_seed(3)).numpy()

    def wts(seed, n, k):
        r = np.random.default_rng(seed)
        q = r.integers(-127, 128, size=(n, k)).astype(np.int8)
        sc = np.array([oracle.f32_to_f16(v) for v in r.uniform(0.001, 0.02, n).astype(np.float32)], np.uint16)
        return q, sc, r.uniform(-0.1, 0.1, n).astype(np.float32)

    q1, s1, b1 = wts(31, N1, K)
    q2, s2, b2 = wts(32, K, N1)
    gamma, beta = np.ones(K, np.float32), np.zeros(K, np.float32)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    Xd, Hd, Yd = dev(X), torch.empty((T, N1), device="cuda"), torch.empty((T, K), device="cuda")
    Q1, S1, B1 = dev(q1), dev(s1.view(np.int16)), dev(b1)
    Q2, S2, B2, G, Bt = dev(q2), dev(s2.view(np.int16)), dev(b2), dev(gamma), dev(beta)
    ctx = tenzor_amd.Context(0)

    def g1():
        check(lib().tzh_linear_w8(ctx.handle, Xd.data_ptr(), _abi.F32, Q1.data_ptr(), S1.data_ptr(), B1.data_ptr(),
                                  Hd.data_ptr(), _abi.F32, T, K, N1, _abi.EPI_BIAS_GELU, None, _abi.F32, None, None,
                                  0.0))

    def g2():
        check(lib().tzh_linear_w8(ctx.handle, Hd.data_ptr(), _abi.F32, Q2.data_ptr(), S2.data_ptr(), B2.data_ptr(),
                                  Yd.data_ptr(), _abi.F32, T, N1, K, _abi.EPI_BIAS_RES_LN, Xd.data_ptr(), _abi.F32,
                                  G.data_ptr(), Bt.data_ptr(), C.c_float(1e-12)))

    for _ in range(args.warmup):
        g1()
        g2()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(args.steps):
        g1()
        g2()
    e.record()
    torch.cuda.synchronize()
    elapsed = s.elapsed_time(e) * 1e-3
    # per-launch durations (each call also re-tiles its int8 codes into the
    # kernel's layout in the context scratch: a separate small kernel)
    us1, us2 = kernel_events(g1, 10), kernel_events(g2, 10)
    flops = 2.0 * T * K * N1
    bytes1 = 4.0 * T * (K + N1) + N1 * K + N1 * (2 + 4)
    bytes2 = 4.0 * T * (N1 + K + K) + K * N1 + K * (2 + 4) + 2 * K * 4
    roof = []
    for name, us, byts in (("gemm1 bias+GELU 384->1536", us1, bytes1), ("gemm2 bias+residual+LN 1536->384", us2, bytes2)):
        t_hbm, t_mfma = byts / (HBM_PEAK_GBS * 1e9), flops / (F16_PEAK_TFLOPS * 1e12)
        roof.append(dict(kernel=name, avg_us=round(us, 2), bound="hbm" if t_hbm >= t_mfma else "mfma",
                         algorithmic_bytes=int(byts), frac=round(max(t_hbm, t_mfma) / (us * 1e-6), 4),
                         achieved=round(byts / (us * 1e-6) / 1e9, 1)))
    dom = max(roof, key=lambda r: r["avg_us"])
    line = {
        "metric": "tokens/sec, int8-weight GEMM pair (384->1536 + GELU, 1536->384 + residual + LayerNorm), "
                  "f32 activations, T = 65536, 1 GPU; % of HBM roofline",
        "value": round(T * args.steps / elapsed, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic",
        "config": {"workload": "config 3: X f32 [65536, 384] N(0,1); W1 int8 [1536, 384], W2 int8 [384, 1536], "
                               "per-row f16 scales U(0.001, 0.02), biases U(-0.1, 0.1); GELU; residual X; "
                               "LayerNorm gamma 1 beta 0 eps 1e-12", "parallelism": "single GPU"},
        "roofline": {"kernel": dom["kernel"], "bound": dom["bound"], "achieved": dom["achieved"],
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": dom["frac"], "traffic": None,
                     "avg_us": dom["avg_us"], "algorithmic_bytes": dom["algorithmic_bytes"]},
        "kernels": roof,
    }
    if not args.no_cpu_baseline:
        _, nproc, cpu_model = host_facts()
        rows = np.sort(rng.choice(T, 4096, replace=False))
        t0 = time.perf_counter()
        h = oracle.gelu(oracle.matmul_w8a32(X[rows], q1, s1, b1))
        ref = oracle.layernorm(X[rows] + oracle.matmul_w8a32(h, q2, s2, b2), gamma, beta, 1e-12)
        dt = time.perf_counter() - t0
        err = float(np.abs(Yd.cpu().numpy()[rows] - ref).max())
        line["cpu_baseline"] = {
            "value": round(len(rows) / dt, 1), "unit": "tokens/s", "cores": 1, "nproc": nproc, "cpu": cpu_model,
            "kind": "port",
            "sample": f"{len(rows)} random rows of X through the pair (oracle.c: matmul_w8a32, GELU, matmul_w8a32, "
                      f"residual, LayerNorm), one thread; {dt:.1f} s; GPU vs CPU on the sample: max-abs {err:.2e}",
        }
    ctx.close()
    return line


DOCS = 256


def embed_docs(args):
    """The embed command's document path (main.zig:786-933) over DOCS
    synthetic documents per step: host tokenization, chunking, one batched
    forward over every chunk, chunk mean + L2.  A step starts from host
    text and ends with the embeddings in HBM; `value` counts pieces
    (tokens before chunking).  Piece counts ~ U[16, 4000], avoiding 511..920
    (one over-long chunk in the reference, an error here)."""
    import torch

    import tenzor_amd
    from tenzor_amd import synth
    from tenzor_amd.arctic import ModelWeights, embedDocuments, forwardBatch
    from tenzor_amd.tokenizer import Tokenizer

    cfg = synth.Config()
    weights = synth.quantize(synth.make_arctic_f32(SEED_WEIGHTS, cfg))
    ctx = tenzor_amd.Context(0)
    model = ModelWeights.fromHost(ctx, weights, cfg)
    vocab_bytes, words = synth.make_vocab(SEED_BATCH)
    tok = Tokenizer.init()
    tok.loadVocabFromBytes(vocab_bytes)
    rng = np.random.default_rng(SEED_BATCH)
    sizes = rng.integers(16, 4001, size=DOCS)
    sizes = np.where((sizes > 510) & (sizes < 921), sizes + 410, sizes)
    docs = [synth.make_text(int(1000 + i), words, int(n), plain=True) for i, n in enumerate(sizes)]
    out = torch.empty((DOCS, cfg.hidden_size), device="cuda")
    for _ in range(args.warmup):
        counts = embedDocuments(out, docs, tok, model)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        embedDocuments(out, docs, tok, model)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    assert torch.isfinite(out).all()
    pieces = int(sizes.sum())

    # the same chunks through the forward alone, ids already in HBM
    from tenzor_amd.tokenizer import chunk_count

    chunk_ids, chunk_lens = [], []
    for d in docs:
        p = tok.encodeRaw(d)
        for k in range(chunk_count(len(p))):
            c = np.concatenate([[101], p[460 * k:min(460 * k + 510, len(p))], [102]]).astype(np.uint32)
            chunk_ids.append(c)
            chunk_lens.append(len(c))
    flat = torch.from_numpy(np.concatenate(chunk_ids).view(np.int32)).cuda()
    cout = torch.empty((len(chunk_lens), cfg.hidden_size), device="cuda")
    forwardBatch(cout, flat, chunk_lens, model)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(args.steps):
        forwardBatch(cout, flat, chunk_lens, model)
    e.record()
    torch.cuda.synchronize()
    fwd_ms = s.elapsed_time(e) / args.steps

    line = {
        "metric": "documents/sec, embed document path (tokenize, 510/50 chunks, int8 arctic-embed-xs, mean + L2), 1 GPU",
        "value": round(DOCS * args.steps / elapsed, 1),
        "unit": "documents/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic",
        "config": {
            "workload": f"{DOCS} synthetic documents of U[16,4000] pieces (511..920 moved up by 410), "
                        "synthetic 30522-line vocabulary",
            "pieces_per_step": pieces,
            "chunks_per_step": int(counts.sum()),
            "chunk_tokens_per_step": int(sum(chunk_lens)),
            "parallelism": "single GPU",
        },
        "pieces_per_s": round(pieces * args.steps / elapsed, 1),
        "forward_only_ms": round(fwd_ms, 4),
        "host_and_pooling_share": round(1 - fwd_ms / (elapsed / args.steps * 1e3), 4),
    }
    if not args.no_cpu_baseline:
        import oracle
        from oracle import wordpiece as wp

        threads, nproc, cpu_model = host_facts()
        hw = synth.HostWeights(weights, cfg)
        sample = list(range(0, DOCS, 32))
        starts = np.concatenate([[0], np.cumsum(counts)])
        sel = [j for d in sample for j in range(int(starts[d]), int(starts[d + 1]))]
        flat_s = np.concatenate([chunk_ids[j] for j in sel]).astype(np.uint32)
        lens_s = np.array([chunk_lens[j] for j in sel], np.int32)
        offs = np.concatenate([[0], np.cumsum(lens_s)[:-1]]).astype(np.int64)
        t0 = time.perf_counter()
        emb = oracle.arctic_forward_batch(hw, flat_s, offs, lens_s, nthreads=threads)
        k = 0
        for d in sample:
            n = int(counts[d])
            wp.chunk_mean_l2(emb[k:k + n])
            k += n
        dt = time.perf_counter() - t0
        line["cpu_baseline"] = {
            "value": round(len(sample) / dt, 2),
            "unit": "documents/s",
            "cores": threads,
            "nproc": nproc,
            "cpu": cpu_model,
            "kind": "port",
            "sample": f"{len(sample)} of the {DOCS} documents ({len(sel)} chunks), C restatement of the forward "
                      f"+ the pooling; tokenization not timed; {dt:.1f} s",
        }
    print(json.dumps(line), flush=True)
    tok.deinit()
    model.deinit()


if __name__ == "__main__":
    main()
