"""Headline benchmark: int8 Arctic-embed-xs forward, batch 256 x seq 512
(lengths U[16,512], padded with id 0), CLS pooling + L2, on one MI355X.

    python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--no-cpu-baseline]

Prints one JSON line.  A step is one forward of the whole batch with the
padded token ids already resident in HBM; `value` counts real (unpadded)
tokens.  `roofline` describes the dominant kernel (by total time in the
forward), timed alone with HIP events on the stream the forward uses, at the
same shape; `cpu_baseline` times the C restatement of the reference's
batch-parallel CPU forward (forwardBatchParallel) on a sample of the same
batch on the host cores.
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


def gemm_shapes(T):
    """(name, K, N, epilogue, flops, algorithmic HBM bytes) per layer of the
    forward, at f16 activation boundaries (A read once, C written once,
    int8 weights + f16 scales + f32 bias read once, residual read once)."""
    out = []
    for name, K, N, epi, res in (("qkv", 384, 1152, 0, False), ("attn_out_ln", 384, 384, 2, True),
                                 ("ffn1_gelu", 384, 1536, 1, False), ("ffn2_ln", 1536, 384, 2, True)):
        flops = 2.0 * T * K * N
        byts = T * K * 2 + T * N * 2 + (T * N * 2 if res else 0) + N * K + N * (2 + 4) + (2 * N * 4 if res else 0)
        out.append((name, K, N, epi, flops, byts))
    return out


def time_kernel(fn, iters=20, warmup=3):
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(iters):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / iters * 1e-3  # seconds


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-sample-stride", type=int, default=1, help="every k-th sequence of the batch")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the forward is data-parallel over "
              "sequences and multi-GPU runs are not part of this build", file=sys.stderr)
        sys.exit(2)

    import ctypes as C

    import torch

    import tenzor_amd
    from tenzor_amd import _abi, check, lib, synth
    from tenzor_amd.arctic import ModelWeights, forwardBatch

    assert torch.cuda.is_available(), "bench.py needs the GPU"
    cfg = synth.Config()
    weights = synth.quantize(synth.make_arctic_f32(SEED_WEIGHTS, cfg))  # N(0,0.02), gamma 1, beta 0
    ctx = tenzor_amd.Context(0)
    model = ModelWeights.fromHost(ctx, weights, cfg)
    ids, lengths = synth.make_batch(SEED_BATCH, BATCH, SEQ)
    d_ids = torch.from_numpy(ids.view(np.int32)).cuda()
    out = torch.empty((BATCH, cfg.hidden_size), device="cuda")
    real_tokens = int(lengths.sum())

    for _ in range(args.warmup):
        forwardBatch(out, d_ids, lengths, model)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(args.steps):
        forwardBatch(out, d_ids, lengths, model)
    e.record()
    torch.cuda.synchronize()
    elapsed = s.elapsed_time(e) * 1e-3
    ms_per_step = elapsed / args.steps * 1e3
    value = real_tokens * args.steps / elapsed
    assert torch.isfinite(out).all()

    # per-GEMM standalone timing at the forward's shapes (same kernels, same stream)
    T = real_tokens
    gemms = []
    X = torch.randn(T, 1536, device="cuda").half()
    R = torch.randn(T, 384, device="cuda").half()
    Y = torch.empty(T, 1536, device="cuda", dtype=torch.half)
    G, Bt = torch.ones(384, device="cuda"), torch.zeros(384, device="cuda")
    for name, K, N, epi, flops, byts in gemm_shapes(T):
        W = torch.randint(-127, 128, (N, K), dtype=torch.int8, device="cuda")
        S = torch.full((N,), int(np.float16(0.01).view(np.int16)), dtype=torch.int16, device="cuda")
        B = torch.zeros(N, device="cuda")
        fn = lambda: check(lib().tzh_linear_w8(ctx.handle, X.data_ptr(), _abi.F16, W.data_ptr(), S.data_ptr(),
                                               B.data_ptr(), Y.data_ptr(), _abi.F16, T, K, N, epi,
                                               R.data_ptr() if epi == 2 else None, _abi.F16, G.data_ptr(),
                                               Bt.data_ptr(), 1e-12))
        t = time_kernel(fn)
        roof_t = max(flops / (F16_PEAK_TFLOPS * 1e12), byts / (HBM_PEAK_GBS * 1e9))
        gemms.append(dict(name=name, seconds=t, flops=flops, bytes=byts, roof_t=roof_t,
                          bound="mfma" if flops / (F16_PEAK_TFLOPS * 1e12) > byts / (HBM_PEAK_GBS * 1e9) else "hbm"))
    dom = max(gemms, key=lambda g: g["seconds"])
    if dom["bound"] == "hbm":
        achieved, peak, unit = dom["bytes"] / dom["seconds"] / 1e9, HBM_PEAK_GBS, "GB/s"
    else:
        achieved, peak, unit = dom["flops"] / dom["seconds"] / 1e12, F16_PEAK_TFLOPS, "TFLOP/s"

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
        "dtype": "fp16",
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
            "kernel": f"gemm_w8 {dom['name']} (T={T}, K,N from the layer)",
            "bound": dom["bound"],
            "achieved": round(achieved, 2),
            "peak": peak,
            "unit": unit,
            "frac": round(achieved / peak, 4),
            "traffic": None,
            "avg_us": round(dom["seconds"] * 1e6, 2),
        },
        "forward_roofline_frac": round(6 * sum(g["roof_t"] for g in gemms) / (ms_per_step * 1e-3), 4),
        "gemm_us": {g["name"]: round(g["seconds"] * 1e6, 1) for g in gemms},
        "padded_equivalent_tokens_per_s": round(BATCH * SEQ * args.steps / elapsed, 1),
    }

    if not args.no_cpu_baseline:
        import oracle

        threads = min(16, os.cpu_count() or 1)
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
            "kind": "port",
            "sample": f"{len(sel)} of the {BATCH} sequences (every {args.cpu_sample_stride}th, "
                      f"{int(lengths[sel].sum())} real tokens), C restatement of forwardBatchParallel, "
                      f"{dt:.1f} s",
        }
    print(json.dumps(line), flush=True)
    model.deinit()


if __name__ == "__main__":
    main()
