"""Headline benchmark: int8 Arctic-embed-xs forward, batch 256 x seq 512
(lengths U[16,512], padded with id 0), CLS pooling + L2, on one MI355X.

    python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--no-cpu-baseline]
    python bench.py --workload embed-docs    # the embed command's document path

Prints one JSON line.  A step is one forward of the whole batch with the
padded token ids already resident in HBM; `value` counts real (unpadded)
tokens.  `roofline` describes the dominant kernel (by total time in the
forward), timed inside the forward with HIP events recorded around every
launch on the forward's own stream; `cpu_baseline` times the C restatement of the reference's
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
TRAFFIC_PROFILE = "arctic_b256_stage_profile.md"


KERNELS = {
    "qkv": "linear_pipe_kernel bias, 384 -> 1152",
    "attention": "attn_varlen_kernel",
    "attn_out_ln": "linear_pipe_kernel bias+residual+LayerNorm, 384 -> 384, 64-row tiles, two workgroups per CU",
    "ffn1_gelu": "linear_pipe_kernel bias+GELU, 384 -> 1536",
    "ffn2_ln": "linear_pipe_kernel bias+residual+LayerNorm, 1536 -> 384, + split last round "
               "(linear_pipe_kernel residual pieces, ln_rows_kernel)",
    "embed_ln": "embed_ln_kernel", "pack_ids": "pack_ids_kernel", "cls_l2": "cls_l2_kernel",
}


def stage_work(T, lengths):
    """Algorithmic (flops, HBM bytes) of one launch of each forward stage.

    Bytes follow the reference's op boundaries in f32 (the per-token figures
    of the measurement plan: QKV 6144, attention core 6144, O-proj + residual
    + LayerNorm 4608, FFN1 + GELU 7680, FFN2 + residual + LayerNorm 9216,
    embeddings 4608 bytes per token) plus the int8 weights, f16 scales and
    f32 biases the launch reads; this build moves f16 activations, so its
    actual traffic is about half (reported separately as bytes_f16)."""
    H, I = 384, 1536
    w = {}
    for name, K, N, per_tok, res in (("qkv", H, 3 * H, 6144, False), ("attn_out_ln", H, H, 4608, True),
                                     ("ffn1_gelu", H, I, 7680, False), ("ffn2_ln", I, H, 9216, True)):
        weights = N * K + N * (2 + 4) + (2 * N * 4 if res else 0)
        f16 = T * K * 2 + T * N * 2 + (T * N * 2 if res else 0) + weights
        w[name] = (2.0 * T * K * N, float(T * per_tok + weights), float(f16))
    L2 = float((lengths.astype(np.float64) ** 2).sum())
    # per head QK^T and PV: 2 * L^2 * 32 flops each; 12 heads
    w["attention"] = (4.0 * L2 * H, float(T * 6144), float(T * 3 * H * 2 + T * H * 2))
    # word/position/type rows (f32) gathered per token, LayerNorm, one row out
    w["embed_ln"] = (0.0, float(T * 4608), float(T * H * 4 * 3 + T * H * 2))
    w["pack_ids"] = (0.0, float(T * 4 * 3), float(T * 4 * 3))
    w["cls_l2"] = (0.0, float(len(lengths) * H * (4 + 4)), float(len(lengths) * H * (2 + 4)))
    return w


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-sample-stride", type=int, default=1, help="every k-th sequence of the batch")
    ap.add_argument("--workload", choices=["forward", "embed-docs"], default="forward")
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

    # per-kernel durations inside the forward: HIP events around every launch
    # on the forward's own stream (tzh_arctic_set_timing)
    model.set_timing(True)
    per_stage = {}
    n_timed = 3
    for _ in range(n_timed):
        forwardBatch(out, d_ids, lengths, model)
        for name, us in model.launch_times():
            per_stage.setdefault(name, []).append(us)
    model.set_timing(False)
    T = real_tokens
    work = stage_work(T, lengths)
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
    # copy; see profile_summary.py) and committed with the profile
    from tenzor_amd.profile_summary import load_traffic

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
            "bytes_f16": int(dom["bytes16"]),
            "achieved_f16_GBps": round(dom["bytes16"] / secs / 1e9, 1),
        },
        "forward_roofline_frac": round(fwd_roof_us / (ms_per_step * 1e3), 4),
        "stage_us": {k: round(v["avg_us"], 1) for k, v in stages.items()},
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
        "dtype": "fp16",
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

        threads = min(16, os.cpu_count() or 1)
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
            "kind": "port",
            "sample": f"{len(sample)} of the {DOCS} documents ({len(sel)} chunks), C restatement of the forward "
                      f"+ the pooling; tokenization not timed; {dt:.1f} s",
        }
    print(json.dumps(line), flush=True)
    tok.deinit()
    model.deinit()


if __name__ == "__main__":
    main()
