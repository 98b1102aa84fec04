"""Benchmark of the int8 projection + paged-attention decode path on one MI355X.

Default workload: TinyLlama-1.1B-shaped int8 decode at batch 1,
random-init weights N(0, 0.02) quantized per row (lm_head int8 too), a 512-token random
prompt prefilled on the GPU, then greedy decode steps. A "step" is one decode step of the
batch (one pia_model_decode call: every layer, the LM head, argmax, token fed back).

Also reported (same line): the batch-32 paged decode of configs[2] (contexts U[128, 2048],
blocks assigned by a random permutation of the pool), the dominant kernel's roofline from
HIP events on the library's stream, and the CPU baseline (the oracle's restatement of the
reference's rayon + AVX2 path) timed on a bounded sample on this host.

Also (same line): device sampling latency per mode, the cost of a speculative verification
pass against a plain step, and checkpoint loading throughput.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-b32] [--no-cpu] [--no-extras]
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
TRAFFIC_GATE_UP_B1 = 23_450_000
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 matrix-core peak, TOP/s
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
    first_tokens, first_pos, first_argmax = list(toks), list(pos), None
    for _ in range(steps):
        _, am = model.decode(toks, pos, tables, want_logits=False)
        if first_argmax is None:
            first_argmax = am.tolist()
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
                other_ms=acc[6] / steps, gemv_bytes=sum(by[i] for i in range(5)) / steps, attn_bytes=by[5] / steps,
                first_tokens=first_tokens, first_pos=first_pos, first_argmax=first_argmax)


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
    # Per-class time of a step from graph replays: each projection class's launches (above)
    # times its launches per step; attention and the small kernels are what is left of the
    # timed step.
    ms_step = 1e3 * elapsed / steps
    layers = cfg.layers
    gb = {cls: round(prof["launch"][cls]["us"] * (1 if cls == "lm_head" else layers) / 1e3, 4)
          for cls in ("qkv", "o", "gate_up", "down", "lm_head")}
    gb["attention_and_rest"] = round(ms_step - sum(gb.values()), 4)
    prof["graph_breakdown"] = gb
    # Whole-step HBM rate: every weight byte and the KV bytes attention reads, per timed step.
    step_bytes = model.weight_bytes() + prof["attn_bytes"]
    prof["step_hbm"] = {"bytes_per_step": int(step_bytes), "GB/s": round(step_bytes / ms_step / 1e6, 1),
                        "frac": round(step_bytes / ms_step / 1e6 / HBM_PEAK_GBS, 4)}
    # The Llama-3-8B LM head (128256 x 4096 int8, 525 MB) at batch 1: the largest single GEMV
    # of the configurations, long enough to show the kernel's streaming rate.
    us, by = pia.bench_projection(ctx, 128256, 4096, 1, 10)
    prof["big_gemv"] = {"rows": 128256, "cols": 4096, "us": round(us, 2), "bytes": by, "GB/s": round(by / us / 1e3, 1),
                        "frac": round(by / us / 1e3 / HBM_PEAK_GBS, 4)}
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
    state = dict(toks=prof["first_tokens"], pos=prof["first_pos"], tables=tables, nb=nb,
                 gpu_argmax=prof["first_argmax"],
                 kv=model.kv_download() if os.environ.get("BENCH_CPU", "1") == "1" else None)
    model.close()
    return state, dict(tok_s=batch * steps / elapsed, ms_per_step=1e3 * elapsed / steps,
                prefill_tok_s=float(np.sum(ctxs)) / prefill_s, mean_ctx=float(np.mean(ctxs)),
                gemv_gbs=(gemv_bytes / 1e9) / (gemv_ms / 1e3) if gemv_ms else None,
                attn_gbs=(attn_bytes / 1e9) / (attn_ms / 1e3) if attn_ms else None,
                gemv_ms=gemv_ms, attn_ms=attn_ms,
                gate_up_gbs=gu["bytes_per_launch"] / (gu["us_per_launch"] * 1e3))


def _timed(ctx, fn, reps):
    fn()
    ctx.sync()
    t0 = time.perf_counter()
    for _ in range(reps):
        fn()
    ctx.sync()
    return (time.perf_counter() - t0) / reps


def run_sampling(ctx, vocab, reps=20):
    """Device sampling (Sampler::sample) over TinyLlama-vocabulary logits: microseconds per
    call (host clock around `reps` back-to-back calls on the library stream), per mode, batch
    and setting."""
    rng = np.random.default_rng(SEED + 7)
    res = {}
    for batch in (1, 32):
        logits = (rng.standard_normal((batch, vocab)) * 2.0).astype(np.float32)
        dl, do = ctx.to_device(logits), ctx.empty((batch,), np.int32)
        dr = ctx.to_device(np.array([pia.rng_new(i) for i in range(batch)], np.uint64))
        for name, prm in (("t0.8_p0.9_k40", (0.8, 0.9, 40)), ("t1.0_full_vocab", (1.0, 1.0, 0))):
            dp = ctx.to_device(pia.sampling_array([prm] * batch))
            for mode, mname in ((pia.SAMPLE_REFERENCE, "reference_order"), (pia.SAMPLE_EXACT_SUMS, "exact_sums")):
                call = lambda: pia.check(pia.lib().pia_sample_dev(ctx.h, do.ptr, dl.ptr, vocab, batch, vocab, dp.ptr,
                                                                   dr.ptr, mode, None))
                res[f"b{batch}_{name}_{mname}_us"] = round(1e6 * _timed(ctx, call, reps), 1)
            dp.free()
        for d in (dl, do, dr):
            d.free()
    return res


def run_spec_verify(ctx, cfg, weights, prompt_len=512, reps=20):
    """Cost of one speculative verification pass (pia_model_verify_groups) of the held token
    plus K drafts of one sequence at context 512, against a plain batch-1 step (K = 0)."""
    bs = 16
    nb = (prompt_len + 64 + bs - 1) // bs
    table = list(range(nb))
    model = pia.Model(ctx, cfg, weights)
    model.kv_alloc(nb, bs)
    prompt = np.random.default_rng(SEED + 11).integers(0, cfg.vocab, prompt_len).tolist()
    _, tok = model.prefill(prompt, 0, table, want_logits=False)
    res = {}
    for k in (0, 1, 4, 8):
        group = [(prompt_len, [tok] + prompt[:k], table)]
        res[f"k{k}_ms_per_pass"] = round(1e3 * _timed(ctx, lambda: model.verify_groups(group), reps), 4)
    res["k4_cost_vs_k0"] = round(res["k4_ms_per_pass"] / res["k0_ms_per_pass"], 3)
    model.close()
    return res


def run_loader(ctx, cfg, layers=4):
    """pia_model_load_safetensors on a TinyLlama-shaped bf16 checkpoint cut to `layers` layers
    (same per-layer shapes, full embedding and LM head), written to /dev/shm: seconds and
    checkpoint GB/s, int8 (device quantizer) and f32."""
    import struct
    hd = cfg.hidden // cfg.heads
    kvd = cfg.kv_heads * hd
    rng = np.random.default_rng(SEED + 13)

    def bf(shape):
        n = int(np.prod(shape))
        return pia.f32_to_bf16((rng.standard_normal(n, dtype=np.float32) * 0.02).reshape(shape))

    shapes = {"model.embed_tokens.weight": (cfg.vocab, cfg.hidden), "model.norm.weight": (cfg.hidden,),
              "lm_head.weight": (cfg.vocab, cfg.hidden)}
    for i in range(layers):
        p = f"model.layers.{i}"
        shapes.update({f"{p}.input_layernorm.weight": (cfg.hidden,),
                       f"{p}.post_attention_layernorm.weight": (cfg.hidden,),
                       f"{p}.self_attn.q_proj.weight": (cfg.hidden, cfg.hidden),
                       f"{p}.self_attn.k_proj.weight": (kvd, cfg.hidden),
                       f"{p}.self_attn.v_proj.weight": (kvd, cfg.hidden),
                       f"{p}.self_attn.o_proj.weight": (cfg.hidden, cfg.hidden),
                       f"{p}.mlp.gate_proj.weight": (cfg.inter, cfg.hidden),
                       f"{p}.mlp.down_proj.weight": (cfg.hidden, cfg.inter),
                       f"{p}.mlp.up_proj.weight": (cfg.inter, cfg.hidden)})
    header, off = {}, 0
    for name, shp in shapes.items():
        n = 2 * int(np.prod(shp))
        header[name] = {"dtype": "BF16", "shape": list(shp), "data_offsets": [off, off + n]}
        off += n
    hj = json.dumps(header).encode()
    hj += b" " * (-len(hj) % 8)
    path = Path("/dev/shm") / f"pia_bench_{os.getpid()}.safetensors"
    try:
        with open(path, "wb") as f:
            f.write(struct.pack("<Q", len(hj)))
            f.write(hj)
            for shp in shapes.values():
                f.write(bf(shp).tobytes())
        lcfg = pia.LlamaConfig(cfg.hidden, layers, cfg.heads, cfg.kv_heads, cfg.inter, cfg.vocab)
        res = {"checkpoint_bytes": off, "layers": layers}
        for quant in ("int8", "f32"):
            t0 = time.perf_counter()
            m = pia.Model.from_safetensors(ctx, path, lcfg, quantization=quant, lm_head_int8=quant == "int8")
            ctx.sync()
            dt = time.perf_counter() - t0
            m.close()
            res[f"{quant}_s"] = round(dt, 3)
            res[f"{quant}_GB_per_s"] = round(off / dt / 1e9, 2)
        return res
    finally:
        path.unlink(missing_ok=True)


def run_c4_prefill(ctx, cfg, weights, seqs=8, seq_len=2048):
    """`seqs` sequences of `seq_len` uniform-random tokens prefilled one after the
    other (prefill_batched per sequence, src/model.rs:1222-1255), each into its own block table
    drawn from a random permutation of the pool. Reports prompt tokens/s and the matrix-core
    utilisation of the projection GEMMs (useful int8 ops 2*M*rows*cols over their device time)."""
    bs = 16
    nbs = (seq_len + bs - 1) // bs
    rng = np.random.default_rng(SEED + 4)
    perm = rng.permutation(seqs * nbs).tolist()
    tables = [perm[i * nbs:(i + 1) * nbs] for i in range(seqs)]
    prompts = [rng.integers(0, cfg.vocab, seq_len).tolist() for _ in range(seqs)]
    model = pia.Model(ctx, cfg, weights)
    model.kv_alloc(seqs * nbs, bs)
    model.prefill(prompts[0][:256], 0, tables[0], want_logits=False)  # warm-up (allocations, code load)
    ctx.sync()
    t0 = time.perf_counter()
    first = [model.prefill(p, 0, t, want_logits=False)[1] for p, t in zip(prompts, tables)]
    ctx.sync()
    elapsed = time.perf_counter() - t0
    # Per-class device time of one more prefill of sequence 0 (same inputs, eager, HIP events).
    model.profile(True)
    model.prefill(prompts[0], 0, tables[0], want_logits=False)
    ms, _, calls = model.profile_get()
    model.profile(False)
    hd = cfg.head_dim
    kvd = cfg.kv_heads * hd
    per_layer = {"qkv": (cfg.hidden + 2 * kvd) * cfg.hidden, "o": cfg.hidden * cfg.hidden,
                 "gate_up": 2 * cfg.inter * cfg.hidden, "down": cfg.hidden * cfg.inter}
    names = pia.Model.PROFILE_CLASSES
    proj_ops = sum(2.0 * seq_len * per_layer[k] * cfg.layers for k in per_layer)
    proj_ms = sum(ms[names.index(k)] for k in per_layer)
    classes = {}
    for k in per_layer:
        i = names.index(k)
        ops = 2.0 * seq_len * per_layer[k] * cfg.layers
        classes[k] = {"ms": round(ms[i], 3), "TOP/s": round(ops / (ms[i] * 1e-3) / 1e12, 1)}
    classes["attention"] = {"ms": round(ms[names.index("attention")], 3)}
    classes["other"] = {"ms": round(ms[names.index("other")], 3)}
    achieved = proj_ops / (proj_ms * 1e-3) / 1e12
    model.close()
    return dict(tok_s=seqs * seq_len / elapsed, ms_per_seq=1e3 * elapsed / seqs, first_tokens=first,
                gemm_tops=achieved, gemm_frac=achieved / INT8_PEAK_TOPS, classes=classes,
                tables=tables, prompts=prompts)


def run_c5(ctx, steps, warmup, seed=SEED + 5):
    """Llama-3-8B-shaped int8 decode at batch 64 with prefix sharing and COW.

    Per prefix group g (4 groups of one random 1024-token prefix): 8 parent sequences admit
    prefix_g + an 8-token parent tail through the KvCacheManager's PrefixCache (the first
    misses and prefills 1032 tokens, then publishes the 64 full prefix blocks; the other 7 hit
    them and prefill only their 8 tail tokens); each parent forks 2 children, which share the
    parent's partially filled tail block; each child then writes its 256 unique random prompt
    tokens starting mid-block, so ensure_writable copies the shared tail block (copy-on-write,
    on the device) before the child's prefill. Parents are released; the 64 children decode
    `steps` greedy steps at batch 64. Returns tok/s plus the state needed by the CPU leg."""
    cfg = pia.LLAMA3_8B
    bs, groups, parents, kids, prefix_len, tail_len, uniq = 16, 4, 8, 2, 1024, 8, 256
    log("synthesizing Llama-3-8B-shape int8 weights")
    weights = pia.synth_weights(cfg, seed=seed)
    rng = np.random.default_rng(seed)
    n_child = groups * parents * kids
    prompt_total = prefix_len + tail_len + uniq
    per_child = (prompt_total + warmup + steps + 2 * bs) // bs + 1
    total_blocks = groups * (prefix_len // bs + parents) + n_child * per_child
    model = pia.Model(ctx, cfg, weights)
    model.kv_alloc(total_blocks, bs)
    kvm = pia.KvCacheManager(total_blocks, bs, prefix_cache=True)
    tick = 0
    t0 = time.perf_counter()
    prefill_tokens = 0
    children = []  # (seq_id, Table, prompt)
    parent_ids = []
    for g in range(groups):
        prefix = rng.integers(0, cfg.vocab, prefix_len).tolist()
        for p in range(parents):
            pid = 1000 + g * parents + p
            tail = rng.integers(0, cfg.vocab, tail_len).tolist()
            toks = prefix + tail
            tick += 1
            got = kvm.admit(pid, toks, tick)
            assert got is not None, "KV pool too small for the c5 workload"
            table, (cached, _, _) = got
            model.prefill(toks[cached:], cached, table.blocks(), want_logits=False)
            prefill_tokens += len(toks) - cached
            kvm.publish(table)
            parent_ids.append(pid)
            for k in range(kids):
                cid = g * parents * kids + p * kids + k
                tick += 1
                ct = kvm.fork(table, cid, tick)
                children.append((cid, ct, toks + rng.integers(0, cfg.vocab, uniq).tolist()))
    # Children: copy-on-write of the shared tail block, then prefill of the unique tokens.
    first = []
    for cid, ct, toks in children:
        pos0 = prefix_len + tail_len
        kvm.ensure_writable(cid, ct, pos0, ctx, model.kv_ptr, model.layout)
        while len(ct) * bs < prompt_total:
            tick += 1
            assert kvm.append_block(cid, ct, tick)
        _, t = model.prefill(toks[pos0:], pos0, ct.blocks(), want_logits=False)
        prefill_tokens += uniq
        first.append(t)
    ctx.sync()
    prefill_s = time.perf_counter() - t0
    for pid in parent_ids:
        kvm.release(pid)
    # Map every block the decode steps will write (append_block on the same manager).
    for cid, ct, _ in children:
        while len(ct) * bs < prompt_total + warmup + 2 * steps + 8:
            tick += 1
            assert kvm.append_block(cid, ct, tick)
    stats = kvm.stats()
    tables = [ct.blocks() for _, ct, _ in children]
    toks, pos = decode_loop(model, first, [prompt_total] * n_child, tables, warmup, bs)
    ctx.sync()
    t0 = time.perf_counter()
    toks, pos = decode_loop(model, toks, pos, tables, steps, bs)
    ctx.sync()
    elapsed = time.perf_counter() - t0
    prof = profile_pass(model, toks, pos, tables, 3)
    # Logical KV bytes one decode step reads (every entry's mapped window, all layers) and the
    # compulsory bytes (each distinct physical block read once).
    distinct = set()
    logical = 0
    for t, p in zip(tables, pos):
        nb_used = p // bs + 1
        distinct.update(t[:nb_used])
        logical += (p + 1) * cfg.layers * cfg.kv_heads * 2 * cfg.head_dim * 4
    compulsory = len(distinct) * bs * cfg.layers * cfg.kv_heads * 2 * cfg.head_dim * 4
    res = dict(tok_s=n_child * steps / elapsed, ms_per_step=1e3 * elapsed / steps, batch=n_child, steps=steps,
               prefill_tok_s=prefill_tokens / prefill_s, prefill_tokens=prefill_tokens,
               weight_bytes=model.weight_bytes(), kv_logical_bytes_per_step=logical,
               kv_compulsory_bytes_per_step=compulsory,
               gemv_ms=prof["gemv_ms"], attn_ms=prof["attn_ms"], other_ms=prof["other_ms"],
               gemv_gbs=(prof["gemv_bytes"] / 1e9) / (prof["gemv_ms"] / 1e3),
               attn_logical_gbs=(logical / 1e9) / (prof["attn_ms"] / 1e3),
               prefix_cache={k: stats[k] for k in ("hits", "misses", "inserts", "tokens_saved", "cow_copies")},
               first_argmax=prof["first_argmax"])
    state = dict(cfg=cfg, weights=weights, toks=prof["first_tokens"], pos=prof["first_pos"], tables=tables,
                 nb=total_blocks, kv=model.kv_download() if os.environ.get("BENCH_CPU", "1") == "1" else None)
    model.close()
    return res, state


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


def cpu_decode_baseline(cfg, weights, toks, pos, tables, nb, kv, gpu_argmax, budget_s, label):
    """The oracle decoding one batch step after another from the GPU run's KV state (same
    tokens, positions and block tables), on this host's cores, for about `budget_s` seconds.
    Also checks the first step's greedy tokens against the GPU's for the same inputs."""
    sys.path.insert(0, str(ROOT))
    from oracle import oracle as orc
    cores = host_cores()
    orc.set_threads(cores)
    om = orc.OracleModel(cfg, weights)
    b = len(toks)
    t0 = time.perf_counter()
    lc = om.decode(toks, pos, tables, kv, nb, 16)
    one = time.perf_counter() - t0
    first = [orc.argmax(lc[i]) for i in range(b)]
    match = sum(int(x == int(y)) for x, y in zip(first, gpu_argmax))
    n = int(max(1, min(200, budget_s / max(one, 1e-3)))) - 1
    tk, ps = first, [p + 1 for p in pos]
    t1 = time.perf_counter()
    for _ in range(n):
        lc = om.decode(tk, ps, tables, kv, nb, 16)
        tk = [orc.argmax(lc[i]) for i in range(b)]
        ps = [p + 1 for p in ps]
    el = (time.perf_counter() - t1) if n else one
    steps = n if n else 1
    return {"value": b * steps / el, "unit": "tok/s", "cores": cores, "kind": "port",
            "sample": f"{steps} greedy decode steps at batch {b} ({label}) from the GPU run's KV state, "
                      f"oracle/ref_cpu.cpp with {cores} threads, avx2={bool(orc.lib().orc_have_avx2())}",
            "first_step_argmax_match": f"{match}/{b}"}


def cpu_prefill_baseline(cfg, weights, prompt, budget_s=10.0):
    """The oracle's prefill_batched (32-token chunks, as the reference) over the first tokens of
    one configs[3] prompt, for about `budget_s` seconds."""
    sys.path.insert(0, str(ROOT))
    from oracle import oracle as orc
    cores = host_cores()
    orc.set_threads(cores)
    om = orc.OracleModel(cfg, weights)
    nb = len(prompt) // 16 + 1
    kv = np.zeros(orc.kv_floats(cfg, nb, 16), np.float32)
    table = list(range(nb))
    t0 = time.perf_counter()
    om.prefill(prompt[:32], 0, table, kv, nb, 16)
    one = time.perf_counter() - t0
    n = int(max(1, min(len(prompt) // 32 - 1, budget_s / max(one, 1e-3))))
    t0 = time.perf_counter()
    om.prefill(prompt[32:32 + 32 * n], 32, table, kv, nb, 16)
    el = time.perf_counter() - t0
    return {"value": 32 * n / el, "unit": "tok/s", "cores": cores, "kind": "port",
            "sample": f"prefill of prompt tokens 32..{32 + 32 * n} of one configs[3] sequence (32-token chunks), "
                      f"oracle/ref_cpu.cpp with {cores} threads"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-b32", action="store_true", help="skip configs[2] (batch-32 paged decode)")
    ap.add_argument("--no-c4", action="store_true", help="skip configs[3] (8 x 2048-token prefill)")
    ap.add_argument("--no-c5", action="store_true", help="skip configs[4] (Llama-3-8B batch 64, prefix + COW)")
    ap.add_argument("--c5-steps", type=int, default=128)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extras", action="store_true",
                    help="skip the sampling / speculative-verification / checkpoint-loading measurements")
    ap.add_argument("--sweep", action="store_true", help="also time each projection shape alone")
    ap.add_argument("--only-b32", action="store_true", help="run only the batch-32 decode (profiling aid)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only copy one 256 MiB KV block 3 times (k_copy_block: known bytes, for PMC scaling)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the int8 decode path is built and measured on a single MI355X; "
              "multi-GPU sharding is not built (every box has one GPU). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if args.no_cpu:
        os.environ["BENCH_CPU"] = "0"
    cpu = not args.no_cpu

    cfg = pia.TINYLLAMA
    ctx = pia.Context(0)
    if args.copy_calibration:
        lay = pia.KvLayout(1, 2, 32768, 8, 128)  # one block = 32768*8*2*128 floats = 256 MiB
        buf = ctx.empty((2 * 32768 * 8 * 2 * 128,), np.float32)
        for _ in range(3):
            pia.check(pia.lib().pia_kv_copy_block_dev(ctx.h, buf.ptr, lay, 0, 1, None))
        ctx.sync()
        print(json.dumps({"copy_calibration": {"bytes_read": 1 << 28, "bytes_written": 1 << 28, "launches": 3}}))
        return
    log("building synthetic TinyLlama int8 weights")
    weights = pia.synth_weights(cfg, seed=SEED)
    if args.only_b32:
        _, b32 = run_b32(ctx, cfg, weights, args.steps, args.warmup)
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
        # Eager pass, one event pair per launch: overstates every class a little (the events
        # and the device spin are not free); the graph-replay figures below sum to the step.
        "step_breakdown_eager_ms": {k: round(v["ms_per_step"], 4) for k, v in b1["classes"].items()},
        "step_breakdown_graph_ms": b1["graph_breakdown"],
        "step_hbm": b1["step_hbm"],
        "lm_head_llama3_b1": b1["big_gemv"],
    }
    if cpu:
        log("CPU baseline (batch 1)")
        out["cpu_baseline"] = cpu_decode_baseline(cfg, weights, b1["first_tokens"], b1["first_pos"], [b1["table"]],
                                                  b1["nb"], kv_state, b1["first_argmax"], 15.0,
                                                  "TinyLlama shape, int8 incl. lm_head")
        kv_state = None
    if not args.no_b32:
        log("B=32 paged decode (configs[2])")
        st32, b32 = run_b32(ctx, cfg, weights, max(5, args.steps // 4), max(2, args.warmup // 2))
        out["b32"] = {k: (round(v, 3) if isinstance(v, float) else v) for k, v in b32.items()}
        if cpu:
            log("CPU baseline (batch 32)")
            out["b32"]["cpu_baseline"] = cpu_decode_baseline(cfg, weights, st32["toks"], st32["pos"], st32["tables"],
                                                             st32["nb"], st32["kv"], st32["gpu_argmax"], 10.0,
                                                             "TinyLlama shape, configs[2] contexts and tables")
        st32 = None
    if not args.no_extras:
        log("device sampling, speculative verification, checkpoint loading")
        out["sampling_us"] = run_sampling(ctx, cfg.vocab)
        out["spec_verify"] = run_spec_verify(ctx, cfg, weights)
        out["loader"] = run_loader(ctx, cfg)
    if not args.no_c4:
        log("8 x 2048-token prefill (configs[3])")
        c4 = run_c4_prefill(ctx, cfg, weights)
        prompt0 = c4.pop("prompts")[0]
        c4.pop("tables")
        out["c4_prefill"] = {k: (round(v, 4) if isinstance(v, float) else v) for k, v in c4.items()}
        out["c4_prefill"]["mfma_roofline"] = {"bound": "mfma", "achieved": round(c4["gemm_tops"], 1),
                                              "peak": INT8_PEAK_TOPS, "unit": "TOP/s (useful int8 ops)",
                                              "frac": round(c4["gemm_frac"], 4)}
        if cpu:
            log("CPU baseline (prefill)")
            out["c4_prefill"]["cpu_baseline"] = cpu_prefill_baseline(cfg, weights, prompt0)
    if args.sweep:
        log("GEMV shape sweep")
        out["gemv_sweep_b1"] = gemv_sweep(ctx, 1)
    weights = None
    if not args.no_c5:
        log("Llama-3-8B batch-64 decode with prefix sharing + COW (configs[4])")
        c5, st5 = run_c5(ctx, args.c5_steps, 4)
        out["c5_llama3_8b_b64"] = {k: (round(v, 3) if isinstance(v, float) else v) for k, v in c5.items()}
        if cpu:
            log("CPU baseline (Llama-3-8B batch 64)")
            out["c5_llama3_8b_b64"]["cpu_baseline"] = cpu_decode_baseline(
                st5["cfg"], st5["weights"], st5["toks"], st5["pos"], st5["tables"], st5["nb"], st5["kv"],
                c5["first_argmax"], 20.0, "Llama-3-8B shape, configs[4] prefix-shared tables")
        out["c5_llama3_8b_b64"].pop("first_argmax")
        st5 = None
    ctx.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
