"""Benchmark of the int8 projection + paged-attention decode path on one MI355X.

Default workload: TinyLlama-1.1B-shaped int8 decode at batch 1,
random-init weights N(0, 0.02) quantized per row (lm_head int8 too), a 512-token random
prompt prefilled on the GPU, then greedy decode steps. A "step" is one decode step of the
batch (one pia_model_decode call: every layer, the LM head, argmax, token fed back).

Also reported (same line): the batch-32 paged decode of configs[2] (contexts U[128, 2048],
blocks assigned by a random permutation of the pool), the dominant kernel's roofline from
HIP events on the library's stream, and the CPU baseline (the oracle's restatement of the
reference's rayon + AVX2 path) timed on a bounded sample on this host.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-b32] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "paged-infer_amd"))
import pia  # noqa: E402

METRIC = "int8 decode tok/s (B=1,32) + int8 GEMV HBM GB/s as % of ~8 TB/s peak"
# HBM bytes per launch of the gate/up projection at batch 1, from rocprofv3 FETCH_SIZE and
# WRITE_SIZE runs scaled by a 256 MiB copy (profiles/decode_b1_projection_traffic.md).
TRAFFIC_GATE_UP_B1 = 23_420_000
HBM_PEAK_GBS = 8000.0
SEED = 2024


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def host_cores() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(n, int(os.environ.get("OMP_NUM_THREADS", n))))


def decode_loop(model, toks, positions, tables, steps, bs, mgr=None):
    """Greedy decode `steps` steps; returns the final tokens. Blocks are pre-mapped."""
    toks = list(toks)
    positions = list(positions)
    for _ in range(steps):
        _, am = model.decode(toks, positions, tables, want_logits=False)
        toks = am.tolist()
        positions = [p + 1 for p in positions]
    return toks, positions


def profile_pass(model, toks, pos, tables, steps):
    """Per-class device time of `steps` decode steps: HIP events around every launch on the
    library's stream (eager launches behind a short device spin so the host enqueues ahead and
    each event pair brackets only its kernel). Same inputs and kernels as the timed replays."""
    model.profile(True)
    n = len(pia.Model.PROFILE_CLASSES)
    acc, by, calls = np.zeros(n), np.zeros(n), np.zeros(n)
    for _ in range(steps):
        _, am = model.decode(toks, pos, tables, want_logits=False)
        ms, b, c = model.profile_get()
        acc += ms
        by += b
        calls += c
        toks = am.tolist()
        pos = [p + 1 for p in pos]
    model.profile(False)
    per = {name: {"ms_per_step": acc[i] / steps, "bytes_per_launch": by[i] / max(calls[i], 1),
                  "us_per_launch": 1e3 * acc[i] / max(calls[i], 1), "launches_per_step": calls[i] / steps}
           for i, name in enumerate(pia.Model.PROFILE_CLASSES)}
    return dict(classes=per, gemv_ms=sum(acc[i] for i in range(5)) / steps, attn_ms=acc[5] / steps,
                other_ms=acc[6] / steps, gemv_bytes=sum(by[i] for i in range(5)) / steps, attn_bytes=by[5] / steps)


def run_b1(ctx, cfg, weights, steps, warmup, prompt_len=512):
    bs = 16
    total_tokens = prompt_len + warmup + 2 * steps + 8
    nb = (total_tokens + bs - 1) // bs
    table = list(range(nb))
    model = pia.Model(ctx, cfg, weights)
    model.kv_alloc(nb, bs)
    prompt = np.random.default_rng(SEED).integers(0, cfg.vocab, prompt_len).tolist()
    t0 = time.perf_counter()
    _, tok = model.prefill(prompt, 0, table, want_logits=False)
    ctx.sync()
    prefill_s = time.perf_counter() - t0
    toks, pos = decode_loop(model, [tok], [prompt_len], [table], warmup, bs)
    # Timed region: K greedy decode steps, each a replay of the captured decode graph.
    ctx.sync()
    t0 = time.perf_counter()
    toks, pos = decode_loop(model, toks, pos, [table], steps, bs)
    ctx.sync()
    elapsed = time.perf_counter() - t0
    prof = profile_pass(model, toks, pos, [table], min(steps, 20))
    kv_state = model.kv_download() if os.environ.get("BENCH_CPU", "1") == "1" else None
    # Per-launch device time of each projection class on the model's own weights (graph of the
    # class's launches over all layers; agrees with rocprofv3 --kernel-trace averages).
    prof["launch"] = {}
    for cls in ("qkv", "o", "gate_up", "down", "lm_head"):
        us, by = model.bench_class(cls, 1)
        prof["launch"][cls] = {"us": round(us, 3), "bytes": by, "GB/s": round(by / us / 1e3, 1)}
    res = dict(tok_s=steps / elapsed, ms_per_step=1e3 * elapsed / steps, prefill_tok_s=prompt_len / prefill_s,
               last_tok=toks[0], last_pos=pos[0], table=table, nb=nb, weight_bytes=model.weight_bytes(), **prof)
    model.close()
    return res, kv_state


def run_b32(ctx, cfg, weights, steps, warmup, batch=32):
    bs = 16
    rng = np.random.default_rng(SEED + 32)
    ctxs = rng.integers(128, 2049, batch)
    need = [(int(c) + warmup + steps + 8 + bs - 1) // bs for c in ctxs]
    nb = sum(need)
    perm = rng.permutation(nb).tolist()
    tables, k = [], 0
    for n in need:
        tables.append(perm[k:k + n])
        k += n
    model = pia.Model(ctx, cfg, weights)
    model.kv_alloc(nb, bs)
    first = []
    t0 = time.perf_counter()
    for b in range(batch):
        prompt = rng.integers(0, cfg.vocab, int(ctxs[b])).tolist()
        _, t = model.prefill(prompt, 0, tables[b], want_logits=False)
        first.append(t)
    ctx.sync()
    prefill_s = time.perf_counter() - t0
    toks, pos = decode_loop(model, first, [int(c) for c in ctxs], tables, warmup, bs)
    ctx.sync()
    t0 = time.perf_counter()
    toks, pos = decode_loop(model, toks, pos, tables, steps, bs)
    ctx.sync()
    elapsed = time.perf_counter() - t0
    prof = profile_pass(model, toks, pos, tables, min(steps, 5))
    gemv_ms, attn_ms, gemv_bytes, attn_bytes = prof["gemv_ms"], prof["attn_ms"], prof["gemv_bytes"], prof["attn_bytes"]
    gu = prof["classes"]["gate_up"]
    model.close()
    return dict(tok_s=batch * steps / elapsed, ms_per_step=1e3 * elapsed / steps,
                prefill_tok_s=float(np.sum(ctxs)) / prefill_s, mean_ctx=float(np.mean(ctxs)),
                gemv_gbs=(gemv_bytes / 1e9) / (gemv_ms / 1e3) if gemv_ms else None,
                attn_gbs=(attn_bytes / 1e9) / (attn_ms / 1e3) if attn_ms else None,
                gemv_ms=gemv_ms, attn_ms=attn_ms,
                gate_up_gbs=gu["bytes_per_launch"] / (gu["us_per_launch"] * 1e3))


SWEEP_SHAPES = [  # (name, rows, cols) of the fused projections
    ("tl.qkv", 2560, 2048), ("tl.o", 2048, 2048), ("tl.gate_up", 11264, 2048), ("tl.down", 2048, 5632),
    ("tl.lm_head", 32000, 2048), ("l3.qkv", 6144, 4096), ("l3.o", 4096, 4096), ("l3.gate_up", 28672, 4096),
    ("l3.down", 4096, 14336), ("l3.lm_head", 128256, 4096)]


def gemv_sweep(ctx, batch=1, reps=20):
    """Per-shape int8 projection time: `reps` launches captured in one graph, HIP events around
    a replay (pia_bench_projection). Bytes are the algorithmic bytes of one launch."""
    out = {}
    for name, rows, cols in SWEEP_SHAPES:
        us, by = pia.bench_projection(ctx, rows, cols, batch, reps)
        out[name] = {"us": round(us, 2), "GB/s": round(by / us / 1e3, 1), "frac": round(by / us / 1e3 / HBM_PEAK_GBS, 3)}
    return out


def cpu_baseline(cfg, weights, b1, kv_state, budget_s=15.0):
    """The oracle (C++ restatement of the reference's rayon + AVX2 path) decoding at batch 1
    from the GPU run's KV state, on this host's cores, for a bounded number of steps."""
    sys.path.insert(0, str(ROOT))
    from oracle import oracle as orc
    cores = host_cores()
    orc.set_threads(cores)
    om = orc.OracleModel(cfg, weights)
    tok, pos, table, nb = b1["last_tok"], b1["last_pos"], b1["table"], b1["nb"]
    kv = kv_state
    t0 = time.perf_counter()
    lc = om.decode([tok], [pos], [table], kv, nb, 16)
    one = time.perf_counter() - t0
    n = int(max(2, min(200, budget_s / max(one, 1e-3))))
    tok = orc.argmax(lc[0])
    pos += 1
    t0 = time.perf_counter()
    for _ in range(n):
        lc = om.decode([tok], [pos], [table], kv, nb, 16)
        tok = orc.argmax(lc[0])
        pos += 1
    el = time.perf_counter() - t0
    return {"value": n / el, "unit": "tok/s", "cores": cores, "kind": "port",
            "sample": f"{n} greedy decode steps at batch 1 (TinyLlama shape, int8 incl. lm_head) from the GPU "
                      f"run's KV state at position {b1['last_pos']}, oracle/ref_cpu.cpp with {cores} threads, "
                      f"avx2={bool(orc.lib().orc_have_avx2())}"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-b32", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--sweep", action="store_true", help="also time each projection shape alone")
    ap.add_argument("--only-b32", action="store_true", help="run only the batch-32 decode (profiling aid)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only copy one 256 MiB KV block 3 times (k_copy_block: known bytes, for PMC scaling)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the int8 decode path is built and measured on a single MI355X; "
              "multi-GPU sharding is design-only (DESIGN.md). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if args.no_cpu:
        os.environ["BENCH_CPU"] = "0"

    cfg = pia.TINYLLAMA
    log("building synthetic TinyLlama int8 weights")
    weights = pia.synth_weights(cfg, seed=SEED)
    ctx = pia.Context(0)
    if args.copy_calibration:
        lay = pia.KvLayout(1, 2, 32768, 8, 128)  # one block = 32768*8*2*128 floats = 256 MiB
        buf = ctx.empty((2 * 32768 * 8 * 2 * 128,), np.float32)
        for _ in range(3):
            pia.check(pia.lib().pia_kv_copy_block_dev(ctx.h, buf.ptr, lay, 0, 1, None))
        ctx.sync()
        print(json.dumps({"copy_calibration": {"bytes_read": 1 << 28, "bytes_written": 1 << 28, "launches": 3}}))
        return
    if args.only_b32:
        b32 = run_b32(ctx, cfg, weights, args.steps, args.warmup)
        print(json.dumps({"b32": b32}), flush=True)
        return
    log("B=1 decode")
    b1, kv_state = run_b1(ctx, cfg, weights, args.steps, args.warmup)
    # Dominant kernel of the step: the gate/up projection (largest share of the step's time).
    dom = b1["launch"]["gate_up"]
    dom_gbs = dom["GB/s"]
    out = {
        "metric": METRIC,
        "value": round(b1["tok_s"], 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(b1["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8w-f32",
        "data": "synthetic (seeded N(0,0.02) weights -> per-row int8; uniform random prompt)",
        "config": {"workload": "tinyllama-1.1b-shape int8 decode, batch 1, 512-token prompt (configs[1])",
                   "batch": 1, "prompt_tokens": 512, "block_size": 16, "lm_head": "int8",
                   "weight_bytes": b1["weight_bytes"], "prefill_tok_s": round(b1["prefill_tok_s"], 1),
                   "gemv_ms_per_step": round(b1["gemv_ms"], 4), "attention_ms_per_step": round(b1["attn_ms"], 4),
                   "other_ms_per_step": round(b1["other_ms"], 4)},
        "roofline": {"bound": "hbm", "achieved": round(dom_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(dom_gbs / HBM_PEAK_GBS, 4), "traffic": TRAFFIC_GATE_UP_B1,
                     "kernel": "k_gemv gate/up (11264 x 2048 int8, fused RMSNorm + SwiGLU), batch 1",
                     "algorithmic_bytes_per_launch": int(dom["bytes"]), "us_per_launch": dom["us"],
                     "timing": "HIP events around a graph replay of the 22 gate/up launches of a step "
                               "(model weights, fused RMSNorm + SwiGLU), on the library stream"},
        "projections_b1": b1["launch"],
        "step_breakdown_ms": {k: round(v["ms_per_step"], 4) for k, v in b1["classes"].items()},
    }
    if not args.no_b32:
        log("B=32 paged decode")
        b32 = run_b32(ctx, cfg, weights, max(5, args.steps // 4), max(2, args.warmup // 2))
        out["b32"] = {k: (round(v, 3) if isinstance(v, float) else v) for k, v in b32.items()}
    if args.sweep:
        log("GEMV shape sweep")
        out["gemv_sweep_b1"] = gemv_sweep(ctx, 1)
    if not args.no_cpu:
        log("CPU baseline")
        out["cpu_baseline"] = cpu_baseline(cfg, weights, b1, kv_state)
    ctx.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
