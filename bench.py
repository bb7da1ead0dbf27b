#!/usr/bin/env python3
"""bench.py — routed-expert MoE decode at K3 scale on one MI355X.

Workload (one "step" = one decode token through the whole stack):
  a 60-layer stack of MoE layers, hidden 7168, 384 experts of intermediate
  2048, top-16 sigmoid routing from fp32 routers ~N(0, 0.02), experts in the
  2-stage x 4096-entry residual VQ with 12-bit codes (3.00 bits per weight),
  fp16 codebooks ~N(0, 0.02), fp16 row scales ~U(0.01, 0.05), uniformly
  random codes. Each layer keeps 64 of its 384 expert records resident in
  HBM (60 x 64 records, about 63.5 GB), and its e_score_correction_bias
  lifts those 64 so that every selection hits the cache. The token's hidden
  state enters layer L+1 as h + moe_L(h). Inputs live in HBM before timing.

Reported:
  value        MoE-layer tokens/s (tokens x layers / wall time of the
               timed steps, HIP events on the compute stream); one step's
               launches are captured as a HIP graph and replayed per token
               (--no-graph: launched from the host)
  roofline     the expert matvec kernel: algorithmic bytes (codes + row
               scales of the 16 selected experts) / its launch time from HIP
               events bracketing each launch, against 8 TB/s
  cpu_baseline the reference's own CPU path (oracle/_ref) on the VQ3R twin
               of a K3 layer (3 x 256 entries, the same 3.00 bits per
               weight), 16 of 64 experts routed per token (1.06 GB of
               records rotating through DRAM), over the host CPUs this
               process may use (at most 16, one GPU's share of the box),
               with a one-thread row beside it

The default run also measures the other configurations, each in a child
process of its own (the same code as --workload), and carries their lines
in "workloads": single-expert, kimi-decode, kimi-prefill (and its exact
mode), k3-miss, table-slots.

Workloads (--workload), each printing its own JSON line:
  single-expert one expert's SwiGLU FFN on one token (hidden 2304,
                intermediate 1024), rotating over 128 resident records
                (341 MB, beyond the 256 MB MALL)
  kimi-prefill  512 tokens through a Kimi-Linear-shape MoE layer stack
                (hidden 2304, 256 experts of intermediate 1024, top-8
                softmax, Zipf(1.1)-skewed expert loads, 8-bit shared expert)
  kimi-decode   one decode token through 26 Kimi-Linear-shape layers (all
                256 expert records of each resident, Q8G shared expert)
  vq-encode     the encoder (waste_vq_encode) on one K3 gate matrix, 2 x 4096
                and 3 x 256 codebooks
  k3-miss       32 decode tokens (one per sequence) through 4 K3 layers,
                an HBM cache of 0.69 of the stack's records, misses copied
                from pinned host memory on the copy stream; passes without
                lookahead, with lookahead, and all resident
  table-slots   the reference's dispatch-table slots mvq_rows_f32 and
                kda_step through waste_register_hip, called as the engine
                calls them (host pointers), beside the reference's own
                AVX-512 slots on the host
"""
from __future__ import annotations

import argparse
import json
import os
import shutil
import sys
import tempfile
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
sys.path.insert(0, os.path.join(HERE, "tests", "golden"))

METRIC = "MoE-layer tokens/s + achieved HBM GB/s (% of peak), K3-scale RVQ, 1 MI355X"
TRAFFIC_FILE = os.path.join(HERE, "profiles", "k_vq_lut_k3_decode_traffic.json")
TRAFFIC_SINGLE = os.path.join(HERE, "profiles", "k_vq_rows_single_expert_traffic.json")
TRAFFIC_KIMI = os.path.join(HERE, "profiles", "k_vq_lut_kimi_decode_traffic.json")
TRAFFIC_PREFILL = {"fp16": ("k_vq_run_f16", os.path.join(HERE, "profiles", "k_vq_run_f16_kimi_prefill_traffic.json")),
                   "exact": ("k_vq_mfma_run", os.path.join(HERE, "profiles", "k_vq_mfma_run_kimi_prefill_traffic.json"))}
HBM_PEAK_GBS = 8000.0
H, I, E, K = 7168, 2048, 384, 16
S, EN = 2, 4096


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def rec_layout():
    gate = (I // 64) * (H // 8) * 64 * 3
    down = (H // 64) * (I // 8) * 64 * 3
    scales = 2 * (2 * I + H)
    raw = 48 + 2 * gate + down + scales
    return gate, down, scales, (raw + 4095) // 4096 * 4096


def pair_bytes():
    gate, down, scales, _ = rec_layout()
    return 2 * gate + down + scales            # codes + row scales per (token, expert)


def layer_bytes():
    # codes+scales of K experts, the fp32 router, the layer's codebooks,
    # the bias, x in and y out
    return K * pair_bytes() + E * H * 4 + 3 * S * EN * 8 * 2 + E * 4 + 2 * H * 4


ROUTERS = {
    "cert": "certified (fast exact-sum logits with error bounds; rows whose bounds leave the picks or their order "
            "open recomputed in the reference's sequential order: the reference's picks by construction)",
    "fast": "fast (fixed-order tree logits, picks not certified)",
    "strict": "strict (every logit summed sequentially: bit-exact logits)",
}


def setup(layers, resident, seed=1234, router="cert"):
    import warp_amd
    gate, down, scales_b, rec_bytes = rec_layout()
    ctx = warp_amd.Context(hidden=H, inter=I, n_experts=E, top_k=K, n_layers=layers, fmt="VQ12",
                           renorm=True, routed_scale=1.0, max_tokens=1, rec_bytes=rec_bytes,
                           cache_bytes=layers * resident * rec_bytes, router_strict=router == "strict",
                           router_fast=router == "fast")
    rng = np.random.Generator(np.random.PCG64(seed))
    t0 = time.time()
    for L in range(layers):
        books = rng.normal(0.0, 0.02, size=(3 * S, EN, 8)).astype(np.float16).view(np.uint16)
        ctx.set_codebooks(L, L * 3 * S, books)
        router = rng.standard_normal((E, H), dtype=np.float32) * np.float32(0.02)
        res_ids = rng.permutation(E)[:resident]
        bias = np.zeros(E, np.float32)
        bias[res_ids] = 1.0                         # resident experts always win
        ctx.set_router(L, router, bias)
        for e in res_ids:
            sc = rng.uniform(0.01, 0.05, size=2 * I + H).astype(np.float16).view(np.uint16)
            ctx.put_expert_synth(L, int(e), int(rng.integers(1 << 62)), sc)
        if L % 10 == 9:
            log(f"bench: {L + 1}/{layers} layers resident ({time.time() - t0:.1f}s)")
    ctx.sync()
    return ctx, rec_bytes


def run_gpu(args):
    from warp_amd.device import Buf, Event
    ctx, rec_bytes = setup(args.layers, args.resident, router=args.router)
    ctx.set_matvec_path(args.matvec_path)
    n_in = max(args.steps, args.warmup, 1)
    X = Buf.of(np.random.default_rng(7).standard_normal((n_in, H), dtype=np.float32))
    bufs = [Buf.empty(H), Buf.empty(H)]
    stream = ctx.stream

    def step(s):
        # token s enters from its own staged input; h <- h + moe_L(h)
        x = X.ptr + (s % n_in) * H * 4
        for L in range(args.layers):
            out = bufs[L & 1]
            ctx.moe_decode(L, x, out, resid_dev=x)
            x = out.ptr

    if args.calibrate_copy_mib:
        from warp_amd.device import D2D, check, rt
        n = args.calibrate_copy_mib << 20
        src, dst = Buf(n), Buf(n)
        check(rt().hipMemcpy(dst.ptr, src.ptr, n, D2D), "calibration copy")
        src.free()
        dst.free()
    log(f"bench: warmup {args.warmup} steps")
    for s in range(args.warmup):
        step(s)
    ctx.sync()
    timed = step
    graph = None
    if args.graph:
        # one step captured as a HIP graph (its 4 x layers launches), replayed
        # per token after the token's input is copied into its input buffer
        from warp_amd.device import D2D, Graph, copy_async
        stage = Buf.empty(H)

        def body():
            x = stage.ptr
            for L in range(args.layers):
                out = bufs[L & 1]
                ctx.moe_decode(L, x, out, resid_dev=x)
                x = out.ptr

        graph = Graph(stream, body)

        def timed(s):
            copy_async(stage.ptr, X.ptr + (s % n_in) * H * 4, H * 4, D2D, stream)
            graph.launch()

        for s in range(args.warmup):
            timed(s)
        ctx.sync()
    e0, e1 = Event(), Event()
    rs0 = ctx.route_stats()
    # timed steps: nothing but the layers on the stream
    log(f"bench: timing {args.steps} steps of {args.layers} layers" + (" (graph replays)" if graph else ""))
    t0 = time.perf_counter()
    e0.record(stream)
    for s in range(args.steps):
        timed(s)
    e1.record(stream)
    e1.synchronize()
    ctx.sync()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_ms(e1)
    rs1 = ctx.route_stats()
    routings = args.steps * args.layers
    args.route_recompute = {"routings": routings, "recomputed": rs1["recomputed"] - rs0["recomputed"],
                            "rows": rs1["rows"] - rs0["rows"],
                            "rate": round((rs1["recomputed"] - rs0["recomputed"]) / routings, 4)}
    args.router_cost = None
    if args.router == "cert":
        # what the certificate costs: the same steps from the fast logits'
        # picks, uncertified, in this process on the same inputs
        ctx.set_router_fast(True)
        g2 = Graph(stream, body) if graph is not None else None

        def timed_fast(s):
            if g2 is None:
                step(s)
                return
            copy_async(stage.ptr, X.ptr + (s % n_in) * H * 4, H * 4, D2D, stream)
            g2.launch()

        for s in range(args.warmup):
            timed_fast(s)
        ctx.sync()
        f0, f1 = Event(), Event()
        f0.record(stream)
        for s in range(args.steps):
            timed_fast(s)
        f1.record(stream)
        f1.synchronize()
        ms_fast = f0.elapsed_ms(f1)
        if g2 is not None:
            g2.free()
        ctx.set_router_fast(False)
        args.router_cost = {"certified_ms_per_step": round(ms / args.steps, 4),
                            "uncertified_ms_per_step": round(ms_fast / args.steps, 4),
                            "overhead": round(ms / ms_fast - 1.0, 4)}
        log(f"bench: certified selection {ms / args.steps:.3f} ms/step, uncertified {ms_fast / args.steps:.3f} "
            f"ms/step ({100 * (ms / ms_fast - 1):.1f}% overhead), recompute rate {args.route_recompute['rate']}")
    # the same steps again with HIP events around each expert-matvec and
    # router launch, for the per-kernel durations
    log("bench: per-launch timing pass")
    ctx.set_timing(True)
    for s in range(args.steps):
        step(s)
    ctx.sync()
    kms, kn = ctx.get_timing()
    ctx.set_timing(False)
    args.kernel = ctx.matvec_kernel(0)
    out = bufs[(args.layers - 1) & 1].numpy()
    assert np.isfinite(out).all(), "non-finite hidden state after the stack"
    st = ctx.cache_stats()
    if graph is not None:
        graph.free()
    ctx.close()
    return ms, wall, kms, kn, st


def kernels_sha256():
    import hashlib
    with open(os.path.join(HERE, "warp_amd", "csrc", "kernels.hip"), "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()


def measured_traffic(kernel, launches, path=TRAFFIC_FILE):
    """HBM traffic per launch of the expert matvec from the committed counter
    summary (L2-to-memory read requests by size, write requests), when it
    was taken on this kernel from this very kernels.hip (its sha256 is
    recorded with the counters); None otherwise, with the reason. launches:
    the launch names the summary must hold ("fused", or "gate_up" and
    "down")."""
    try:
        with open(path) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None, "no counter summary"
    if t.get("kernel") != kernel:
        return None, f"counters were taken on {t.get('kernel')}"
    if t.get("kernels_sha256") != kernels_sha256():
        return None, "counters were taken on another build of kernels.hip"
    if any(k not in t for k in launches):
        return None, "the counter summary does not hold these launches"
    return {k: t[k]["read_bytes"] + t[k]["write_bytes"] for k in launches} | {"source": t["source"]}, None


def matvec_roofline(kms, kn, b0, b1, kernel):
    """The expert matvec's roofline terms from the per-launch timing classes:
    class 0 alone is the fused launch (gate/up, down and combine in one),
    else class 0 the gate/up and class 1 the down launches. b0, b1: the
    algorithmic bytes (codes and row scales of the picks) of gate/up and of
    down for one token; kernel: the one the context ran (matvec_kernel)."""
    fused = kn[0] > 0 and kn[1] == 0
    if fused:
        t = kms[0]
        nbytes = kn[0] * (b0 + b1)
        per = {"bytes_per_launch": {"fused": b0 + b1},
               "avg_launch_us": {"fused": round(kms[0] / kn[0] * 1e3, 2)},
               "what": kernel + " (gate/up, down and combine of the routed experts in one launch per layer)"}
    else:
        t = kms[0] + kms[1]
        nbytes = kn[0] * b0 + kn[1] * b1
        per = {"bytes_per_launch": {"gate_up": b0, "down": b1},
               "avg_launch_us": {"gate_up": round(kms[0] / max(kn[0], 1) * 1e3, 2),
                                 "down": round(kms[1] / max(kn[1], 1) * 1e3, 2)},
               "what": kernel + " (expert matvec, gate/up and down launches)"}
    achieved = nbytes / (t / 1e3) / 1e9 if t > 0 else None
    return kernel, fused, achieved, per


def cpu_threads():
    """Host CPUs for the reference's pool: those this process may run on, at
    most 16 (one GPU's share of the GPU box's cores), or WARP_BENCH_CPU_THREADS."""
    env = int(os.environ.get("WARP_BENCH_CPU_THREADS", "0"))
    if env > 0:
        return env
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def twin_dir(args, name, spec):
    """The container of a VQ3R twin, written once per bench run into the
    run's twin directory (shared by the child processes), or into a fresh
    temporary directory."""
    import container as ct
    root = args.twin_dir or tempfile.mkdtemp(prefix="warp_twin_")
    d = os.path.join(root, name)
    if os.path.exists(os.path.join(d, "manifest.json")):
        return d, False
    log(f"bench: writing the VQ3R twin container {name} for the CPU baseline")
    model = ct.build(spec)
    tmp = d + ".tmp"
    shutil.rmtree(tmp, ignore_errors=True)
    os.makedirs(tmp)
    ct.write(model, tmp)
    del model
    os.replace(tmp, d)
    return d, not args.twin_dir


def ref_rows(d, cache_bytes, warm, one, units, seconds, describe):
    """The reference (oracle/_ref) on container d over cpu_threads() and over
    one thread (half the time): warm(ref) fills its cache, one(ref, i) is
    call i of the timed loop, each worth `units`. Returns the cpu_baseline
    object."""
    from oracle import pyoracle as po
    rows = []
    for threads, secs in ((cpu_threads(), seconds), (1, seconds / 2)):
        ref = po.Ref(d, cache_bytes=cache_bytes, n_threads=threads)
        used, isa = ref.threads(), ref.backend()
        warm(ref)
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < secs:
            one(ref, n)
            n += 1
        dt = time.perf_counter() - t0
        ref.close(reset_pool=True)
        rows.append((n * units / dt, n, dt, used, isa))
    (v, n, dt, used, isa), (v1, n1, dt1, _, _) = rows
    all_row = {"value": v, "cores": used, "sample": describe["sample"].format(n=n * units, threads=used, secs=dt,
                                                                              isa=isa)}
    one_row = {"value": v1, "cores": 1, "sample": describe["sample"].format(n=n1 * units, threads=1, secs=dt1,
                                                                            isa=isa)}
    best = all_row if v >= v1 else one_row
    return {"value": best["value"], "unit": describe["unit"], "cores": best["cores"], "kind": "reference",
            "isa": isa, "sample": best["sample"], "chosen": "the better of the two rows",
            "all_threads": all_row, "one_thread": one_row}


def k3_twin_spec():
    import container as ct
    # 64 experts of the K3 shape (1.06 GB of records), top-16 by a random
    # router; the reference's loader requires a shared expert: Q4G g128
    return ct.Spec(hidden=H, inter=I, experts=64, top_k=K, layers=1, fmt="VQ3R", bias=False, renorm=True,
                   routed_scale=1.0, shared_bits=4, shared_group=128, subnormals=False, keep_codes=False, seed=99)


def cpu_baseline(args, seconds):
    """The reference's moe_layer on the VQ3R twin of a K3 layer."""
    from oracle import pyoracle as po
    if not os.path.exists(po.REF_LIB):
        return None
    d, own = twin_dir(args, "k3_vq3r_64", k3_twin_spec())
    rng = np.random.default_rng(3)
    xs = rng.standard_normal((64, H), dtype=np.float32)

    def warm(ref):
        for t in range(24):                        # the first tokens fill the reference's cache
            ref.moe_layer(0, xs[t % 64], 64, K, H)

    def one(ref, i):
        ref.moe_layer(0, xs[i % 64], 64, K, H)
    res = ref_rows(d, 64 * 17_000_000 + (64 << 20), warm, one, 1, seconds, {
        "unit": "MoE-layer tokens/s",
        "sample": "{n} decode tokens through a K3-shape layer (H 7168, I 2048, top-16 of 64 experts, 1.06 GB of "
                  "records rotating through DRAM) in the reference's VQ3R format (3x256, 3.00 bits/weight, the "
                  "twin of the 2x4096 format it cannot load), its own moe_layer ({isa} LUT build + gather apply) "
                  "over {threads} threads, {secs:.1f}s; its loader requires a shared expert, so each token also "
                  "runs a Q4G shared expert (about 8% of the bytes) that the GPU workload does not have"})
    if own:
        shutil.rmtree(os.path.dirname(d), ignore_errors=True)
    return res


# ---- config 1: one expert's FFN, decode ----------------------------------------------------

N_SINGLE = 128        # resident records the single-expert workload rotates over (341 MB)


def run_single_expert(args):
    """One step = one graph replay of N_SINGLE consecutive single-expert FFNs
    (one per resident record, one token each)."""
    import warp_amd
    from warp_amd.device import Buf, Event, Graph
    gate, down, scales_b, rec_bytes = kimi_rec_layout()
    ctx = warp_amd.Context(hidden=KH, inter=KI, n_experts=N_SINGLE, top_k=1, n_layers=1, fmt="VQ12", renorm=False,
                           routed_scale=1.0, max_tokens=1, rec_bytes=rec_bytes, cache_bytes=N_SINGLE * rec_bytes)
    rng = np.random.Generator(np.random.PCG64(1357))
    ctx.set_codebooks(0, 0, rng.normal(0.0, 0.02, size=(3 * S, EN, 8)).astype(np.float16).view(np.uint16))
    for e in range(N_SINGLE):
        sc = rng.uniform(0.01, 0.05, size=2 * KI + KH).astype(np.float16).view(np.uint16)
        ctx.put_expert_synth(0, e, int(rng.integers(1 << 62)), sc)
    ctx.set_matvec_path(args.matvec_path)
    X = Buf.of(rng.standard_normal((N_SINGLE, KH), dtype=np.float32))
    Y = Buf.empty((N_SINGLE, KH))

    def body():
        for e in range(N_SINGLE):
            ctx.expert_ffn(0, e, X.ptr + e * KH * 4, Y.ptr + e * KH * 4)

    for _ in range(args.warmup):
        body()
    ctx.sync()
    graph = Graph(ctx.stream, body) if args.graph else None
    run = graph.launch if graph else body
    for _ in range(args.warmup):
        run()
    ctx.sync()
    e0, e1 = Event(), Event()
    log(f"bench: timing {args.steps} passes over {N_SINGLE} single-expert FFNs")
    t0 = time.perf_counter()
    e0.record(ctx.stream)
    for _ in range(args.steps):
        run()
    e1.record(ctx.stream)
    e1.synchronize()
    ctx.sync()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_ms(e1)
    ctx.set_timing(True)
    body()
    body()
    ctx.sync()
    kms, kn = ctx.get_timing()
    ctx.set_timing(False)
    ctx_kernel = ctx.matvec_kernel(0, expert_ffn=True)
    assert np.isfinite(Y.numpy()).all(), "non-finite expert output"
    if graph is not None:
        graph.free()
    ctx.close()
    n_ffn = args.steps * N_SINGLE
    us_ffn = ms * 1e3 / n_ffn
    pair = 2 * gate + down + scales_b
    b0 = 2 * gate + 2 * 2 * KI
    b1 = down + 2 * KH
    achieved = (kn[0] * b0 + kn[1] * b1) / ((kms[0] + kms[1]) / 1e3) / 1e9 if kn[0] and kn[1] else None
    ffn_gbs = pair / (us_ffn * 1e-6) / 1e9
    kernel = ctx_kernel
    tr, tr_why = measured_traffic(kernel, ("gate_up", "down"), TRAFFIC_SINGLE)
    traffic = round((kn[0] * tr["gate_up"] + kn[1] * tr["down"]) / max(kn[0] + kn[1], 1)) if tr else None
    return {
        "metric": "single-expert SwiGLU FFN decode tokens/s (one expert per token), 1 MI355X",
        "value": round(n_ffn / (ms / 1e3), 1),
        "unit": "expert-FFN tokens/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms / args.steps, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp32",
        "data": "synthetic (random codes, codebooks and scales of the Kimi-Linear expert shape)",
        "launch": (f"{N_SINGLE} FFNs captured as one HIP graph and replayed per step" if graph
                   else "host launches"),
        "config": {"workload": f"single routed expert SwiGLU FFN, decode batch 1, rotating over {N_SINGLE} resident "
                               f"records ({N_SINGLE * pair / 1e6:.0f} MB)",
                   "hidden": KH, "inter": KI, "records": N_SINGLE, "format": "RVQ 2x4096 12-bit codes (3.00 b/w)",
                   "parallelism": "single GPU"},
        "us_per_ffn": round(us_ffn, 3),
        "ffn_bytes": pair,
        "ffn_hbm_gbs": round(ffn_gbs, 1),
        "ffn_hbm_frac": round(ffn_gbs / HBM_PEAK_GBS, 4),
        "roofline": {"bound": "hbm", "achieved": None if achieved is None else round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": None if achieved is None else round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_per_launch": tr if tr else {"unmeasured": tr_why},
                     "kernel": kernel + " (expert matvec, gate/up and down launches)",
                     "bytes_per_launch": {"gate_up": b0, "down": b1},
                     "avg_launch_us": {"gate_up": round(kms[0] / max(kn[0], 1) * 1e3, 2),
                                       "down": round(kms[1] / max(kn[1], 1) * 1e3, 2)}},
        "published_reference_gpu": {"value_gbs": 405.3, "what": "one expert matrix [1024x2304] VQ3R (2.4 MB), "
                                    "kernel only, on an RTX 5060 Ti (third party), docs/LEARNED.md:2910"},
        "wall_s": round(wall, 3),
        "cpu_baseline": None if args.no_cpu else cpu_baseline_single(args, args.cpu_seconds),
    }


def cpu_baseline_single(args, seconds):
    """The reference's per-expert FFN (gate and up tables and applies, SiLU,
    down matvec, as moe_layer runs each routed expert) on the VQ3R twin,
    rotating over 400 records (1.07 GB)."""
    from oracle import pyoracle as po
    import container as ct
    if not os.path.exists(po.REF_LIB):
        return None
    n_rec = 400
    spec = ct.Spec(hidden=KH, inter=KI, experts=n_rec, top_k=1, layers=1, fmt="VQ3R", renorm=False,
                   routed_scale=1.0, shared_bits=8, shared_group=32, subnormals=False, keep_codes=False, seed=95)
    d, own = twin_dir(args, "kimi_vq3r_400", spec)
    x = np.random.default_rng(3).standard_normal(KH, dtype=np.float32)

    def warm(ref):
        for e in range(n_rec):
            ref.expert_ffn(0, e, x, KH)

    def one(ref, i):
        ref.expert_ffn(0, i % n_rec, x, KH)
    res = ref_rows(d, n_rec * 2_700_000 + (64 << 20), warm, one, 1, seconds, {
        "unit": "expert-FFN tokens/s",
        "sample": "{n} single-expert FFNs (H 2304, I 1024) rotating over 400 records (1.07 GB) in the reference's "
                  "VQ3R format (3x256, 3.00 bits/weight), its own per-expert path of moe_layer ({isa} LUT builds, "
                  "gather applies, SiLU, down matvec) over {threads} threads, {secs:.1f}s"})
    if own:
        shutil.rmtree(os.path.dirname(d), ignore_errors=True)
    return res


# ---- Kimi-Linear-shape prefill (a second workload, not the headline line) ----------------

KH, KI, KE, KK, KIS = 2304, 1024, 256, 8, 1024      # hidden, inter, experts, top-k, shared inter


def kimi_rec_layout():
    gate = (KI // 64) * (KH // 8) * 64 * 3
    down = (KH // 64) * (KI // 8) * 64 * 3
    scales = 2 * (2 * KI + KH)
    raw = 48 + 2 * gate + down + scales
    return gate, down, scales, (raw + 4095) // 4096 * 4096


def zipf_bias(router, X, s=1.1, seed=5, iters=80):
    """A per-expert bias (the e_score_correction_bias the reference's selection
    adds, src/model.c:2723-2745) under which the tokens-per-expert counts of
    top-8 softmax routing of X follow Zipf(s) over a random ranking of the
    experts (counts capped at one pick per token and expert): fitted on the
    host by raising each expert's bias by the log ratio of its target count
    to its count."""
    T = X.shape[0]
    logits = X.astype(np.float64) @ router.astype(np.float64).T
    logits -= logits.max(1, keepdims=True)
    sc = np.exp(logits)
    sc /= sc.sum(1, keepdims=True)
    z = (np.arange(KE) + 1.0) ** -s
    target = z / z.sum() * T * KK
    for _ in range(20):                      # cap at T, spread the excess over the rest
        over = target > T
        if not over.any():
            break
        excess = (target[over] - T).sum()
        target[over] = T
        target[~over] += excess * target[~over] / target[~over].sum()
    want = target[np.random.default_rng(seed).permutation(KE)]      # expert e's target count
    step = float(np.std(sc))
    b = np.zeros(KE)
    for _ in range(iters):
        pick = np.argpartition(-(sc + b), KK, axis=1)[:, :KK]
        cnt = np.bincount(pick.ravel(), minlength=KE)
        b += 0.5 * step * (np.log(want + 0.5) - np.log(cnt + 0.5))
    return b.astype(np.float32)


def run_prefill(args):
    import warp_amd
    from warp_amd.hip import ROUTE_SOFTMAX
    from warp_amd.device import Buf, Event, Graph
    T, layers = args.tokens, args.layers
    gate, down, scales_b, rec_bytes = kimi_rec_layout()
    ctx = warp_amd.Context(hidden=KH, inter=KI, n_experts=KE, top_k=KK, n_layers=layers, fmt="VQ12",
                           renorm=True, routed_scale=1.0, router_act=ROUTE_SOFTMAX, max_tokens=T,
                           rec_bytes=rec_bytes, cache_bytes=layers * KE * rec_bytes,
                           prefill_fp16=args.prefill == "fp16")
    rng = np.random.Generator(np.random.PCG64(4321))
    X = rng.standard_normal((T, KH), dtype=np.float32)
    shared_bytes = kimi_layers(ctx, layers, rng, lambda L, router: zipf_bias(router, X, seed=5 + L))
    Xd = Buf.of(X)
    outs = [Buf.empty((T, KH)) for _ in range(layers)]
    # the routing of the timed input: distinct experts and pairs per layer
    distinct = []
    for L in range(layers):
        route, _ = ctx.moe_chunk(L, Xd.ptr, outs[L].ptr, T, want_route=True)
        distinct.append(len(np.unique(route)))
    counts = np.sort(np.bincount(route.ravel(), minlength=KE))[::-1]

    def step():
        for L in range(layers):
            ctx.moe_chunk(L, Xd.ptr, outs[L].ptr, T)

    for _ in range(args.warmup):
        step()
    ctx.sync()
    # every record resident and no routes asked for: a chunk queues its work
    # and returns, so one step can be captured and replayed
    graph = Graph(ctx.stream, step) if args.graph else None
    run = graph.launch if graph else step
    for _ in range(args.warmup):
        run()
    ctx.sync()
    e0, e1 = Event(), Event()
    stream = ctx.stream
    log(f"bench: timing {args.steps} prefill steps of {T} tokens x {layers} layers" +
        (" (graph replays)" if graph else ""))
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(args.steps):
        run()
    e1.record(stream)
    e1.synchronize()
    ctx.sync()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_ms(e1)
    for L in range(layers):
        assert np.isfinite(outs[L].numpy()).all(), "non-finite prefill output"
    if graph:
        graph.free()
    ctx.close()
    pair_bytes = 2 * gate + down + scales_b
    per_layer = (np.mean(distinct) * pair_bytes + shared_bytes + KE * KH * 4 + 3 * S * EN * 8 * 2 + KE * 4
                 + 2 * T * KH * 4)
    flops = 2 * 3 * KH * KI * T * KK + 2 * 3 * KH * KIS * T
    sec = ms / 1e3
    n_lt = args.steps * layers
    gbs = per_layer * n_lt / sec / 1e9
    tfs = flops * n_lt / sec / 1e12
    # the routed launches' HBM bytes per launch (one gate+up and one down per layer)
    pk, ppath = TRAFFIC_PREFILL[args.prefill]
    tr, tr_why = measured_traffic(pk, ("gate_up", "down"), ppath)
    traffic = round((tr["gate_up"] + tr["down"]) / 2) if tr else None
    return {
        "metric": "MoE-layer prefill tokens/s, Kimi-Linear shape, 1 MI355X",
        "value": round(T * n_lt / sec, 1),
        "unit": "MoE-layer tokens/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms / args.steps, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp16" if args.prefill == "fp16" else "fp32",
        "launch": "one step (every layer's chunk) captured as a HIP graph and replayed" if graph else "host launches",
        "data": "synthetic (random codes, codebooks, scales, shared expert and routers of the Kimi-Linear shapes; "
                "a per-expert bias that skews tokens per expert towards Zipf(1.1))",
        "config": {"workload": f"Kimi-Linear-shape MoE layer, prefill of {T} tokens, {layers}-layer stack",
                   "hidden": KH, "inter": KI, "experts": KE, "top_k": KK, "routing": "softmax + bias",
                   "shared_expert": "Q8G group 32, intermediate 1024", "tokens": T, "layers": layers,
                   "format": "RVQ 2x4096 12-bit codes (3.00 b/w)", "parallelism": "single GPU"},
        "per_layer": {"distinct_experts": round(float(np.mean(distinct)), 1), "pairs": T * KK,
                      "tokens_on_busiest_5": counts[:5].tolist(), "algorithmic_bytes": int(per_layer),
                      "useful_flops": int(flops)},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_per_launch": tr if tr else {"unmeasured": tr_why},
                     "kernel": pk + " (routed experts, one gate+up and one down launch per layer)",
                     "what": "algorithmic bytes of the layer (records of the distinct experts picked, shared "
                             "expert, router, codebooks, activations) over the step time: HBM-bound, the "
                             "arithmetic intensity (about 85 FLOP/B) is below the bf16 ridge"},
        "mfma": {"achieved": round(tfs, 2), "peak": 2500.0, "unit": "TFLOP/s",
                 "frac": round(tfs / 2500.0, 5),
                 "note": "useful FLOPs (2 x 3 x H x I per pair, plus the shared expert); " +
                         ("the expert products run one fp16 operand per position (stages added) against x's fp16 "
                          "high half" if args.prefill == "fp16" else
                          "the expert products run fp16 hi/lo halves of x and every stage on the matrix cores, "
                          "2 x stages times the useful MFMA work")},
        "precision": ("fp16 operands, fp32 accumulation (outputs within 2e-3 of the reference)"
                      if args.prefill == "fp16" else "exact products (outputs within 1e-4 of the reference)"),
        "wall_s": round(wall, 3),
        "cpu_baseline": None if args.no_cpu else cpu_baseline_prefill(args, args.cpu_seconds, T),
    }


def kimi_layers(ctx, layers, rng, bias_of):
    """Codebooks, router (+ bias_of(L, router)), all 256 expert records and
    the Q8G g32 shared expert of each Kimi-Linear-shape layer; returns the
    shared expert's bytes per layer."""
    import container as ct
    shared_bytes = 0
    t0 = time.time()
    for L in range(layers):
        books = rng.normal(0.0, 0.02, size=(3 * S, EN, 8)).astype(np.float16).view(np.uint16)
        ctx.set_codebooks(L, L * 3 * S, books)
        router = rng.standard_normal((KE, KH), dtype=np.float32) * np.float32(0.02)
        ctx.set_router(L, router, bias_of(L, router))
        for e in range(KE):
            sc = rng.uniform(0.01, 0.05, size=2 * KI + KH).astype(np.float16).view(np.uint16)
            ctx.put_expert_synth(L, e, int(rng.integers(1 << 62)), sc)
        sh = [ct.quant_rows(rng, M, N, 8, 32, (1e-4, 3e-4)) for M, N in ((KIS, KH), (KIS, KH), (KH, KIS))]
        ctx.set_shared(L, 8, 32, KIS, [np.ascontiguousarray(q[0]) for q in sh],
                       [np.ascontiguousarray(q[1]) for q in sh], [q[2] for q in sh])
        shared_bytes = sum(q[0].nbytes + q[1].nbytes for q in sh)
        if L % 8 == 7:
            log(f"bench: {L + 1}/{layers} Kimi-Linear layers set up ({time.time() - t0:.1f}s)")
    ctx.sync()
    return shared_bytes


def run_kimi_decode(args):
    """One step = one decode token through a stack of Kimi-Linear-shape MoE
    layers (every expert record resident), h <- h + moe(h)."""
    import warp_amd
    from warp_amd.hip import ROUTE_SOFTMAX
    from warp_amd.device import Buf, Event
    layers = args.layers
    gate, down, scales_b, rec_bytes = kimi_rec_layout()
    ctx = warp_amd.Context(hidden=KH, inter=KI, n_experts=KE, top_k=KK, n_layers=layers, fmt="VQ12",
                           renorm=True, routed_scale=1.0, router_act=ROUTE_SOFTMAX, max_tokens=1,
                           rec_bytes=rec_bytes, cache_bytes=layers * KE * rec_bytes)
    rng = np.random.Generator(np.random.PCG64(8642))
    shared_bytes = kimi_layers(ctx, layers, rng, lambda L, router: None)
    ctx.set_matvec_path(args.matvec_path)
    n_in = max(args.steps, args.warmup, 1)
    X = Buf.of(rng.standard_normal((n_in, KH), dtype=np.float32))
    bufs = [Buf.empty(KH), Buf.empty(KH)]

    def step(s):
        x = X.ptr + (s % n_in) * KH * 4
        for L in range(layers):
            out = bufs[L & 1]
            ctx.moe_decode(L, x, out, resid_dev=x)
            x = out.ptr

    for s in range(args.warmup):
        step(s)
    ctx.sync()
    timed, graph = step, None
    if args.graph:
        from warp_amd.device import D2D, Graph, copy_async
        stage = Buf.empty(KH)

        def body():
            x = stage.ptr
            for L in range(layers):
                out = bufs[L & 1]
                ctx.moe_decode(L, x, out, resid_dev=x)
                x = out.ptr

        graph = Graph(ctx.stream, body)

        def timed(s):
            copy_async(stage.ptr, X.ptr + (s % n_in) * KH * 4, KH * 4, D2D, ctx.stream)
            graph.launch()

        for s in range(args.warmup):
            timed(s)
        ctx.sync()
    e0, e1 = Event(), Event()
    log(f"bench: timing {args.steps} decode steps of {layers} Kimi-Linear layers")
    t0 = time.perf_counter()
    e0.record(ctx.stream)
    for s in range(args.steps):
        timed(s)
    e1.record(ctx.stream)
    e1.synchronize()
    ctx.sync()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_ms(e1)
    ctx.set_timing(True)
    for s in range(args.steps):
        step(s)
    ctx.sync()
    kms, kn = ctx.get_timing()
    ctx.set_timing(False)
    mv_kernel = ctx.matvec_kernel(0)
    assert np.isfinite(bufs[(layers - 1) & 1].numpy()).all(), "non-finite hidden state after the stack"
    if graph is not None:
        graph.free()
    ctx.close()
    n_lt = args.steps * layers
    b0 = KK * (2 * gate + 2 * 2 * KI)
    b1 = KK * (down + 2 * KH)
    kernel, fused, achieved, per = matvec_roofline(kms, kn, b0, b1, mv_kernel)
    tr, tr_why = measured_traffic(kernel, ("fused",) if fused else ("gate_up", "down"), TRAFFIC_KIMI)
    traffic = None
    if tr:
        traffic = tr["fused"] if fused else round((kn[0] * tr["gate_up"] + kn[1] * tr["down"]) /
                                                  max(kn[0] + kn[1], 1))
    per_layer = (KK * (2 * gate + down + scales_b) + shared_bytes + KE * KH * 4 + 3 * S * EN * 8 * 2 + KE * 4
                 + 2 * KH * 4)
    layer_gbs = per_layer * n_lt / (ms / 1e3) / 1e9
    return {
        "metric": "MoE-layer decode tokens/s, Kimi-Linear shape, 1 MI355X",
        "value": round(n_lt / (ms / 1e3), 2),
        "unit": "MoE-layer tokens/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms / args.steps, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp32",
        "data": "synthetic (random codes, codebooks, scales, shared expert and routers of the Kimi-Linear shapes)",
        "launch": "one step captured as a HIP graph and replayed per token" if args.graph else "host launches",
        "config": {"workload": f"Kimi-Linear-shape MoE layer, decode batch 1, {layers}-layer stack",
                   "hidden": KH, "inter": KI, "experts": KE, "top_k": KK, "routing": "softmax",
                   "shared_expert": "Q8G group 32, intermediate 1024", "layers": layers,
                   "format": "RVQ 2x4096 12-bit codes (3.00 b/w)", "parallelism": "single GPU"},
        "layer_bytes": int(per_layer),
        "layer_hbm_gbs": round(layer_gbs, 1),
        "layer_hbm_frac": round(layer_gbs / HBM_PEAK_GBS, 4),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_per_launch": tr if tr else {"unmeasured": tr_why},
                     "kernel": per["what"],
                     "bytes_per_launch": per["bytes_per_launch"],
                     "avg_launch_us": per["avg_launch_us"],
                     "router_avg_us": round(kms[2] / max(kn[2], 1) * 1e3, 2)},
        "wall_s": round(wall, 3),
        "cpu_baseline": None if args.no_cpu else cpu_baseline_kimi_decode(args, args.cpu_seconds),
    }


def kimi_twin(args):
    """The VQ3R twin of two Kimi-Linear-shape layers (2 x 256 records, 1.37 GB
    rotating through DRAM), with a Q8G g32 shared expert."""
    import container as ct
    spec = ct.Spec(hidden=KH, inter=KI, experts=KE, top_k=KK, layers=2, fmt="VQ3R", renorm=True, routed_scale=1.0,
                   shared_bits=8, shared_group=32, subnormals=False, keep_codes=False, seed=97)
    return twin_dir(args, "kimi_vq3r_2x256", spec)


KIMI_CACHE = 2 * KE * 2_700_000 + (64 << 20)


def cpu_baseline_kimi_decode(args, seconds):
    """The reference's moe_layer on the VQ3R twin of two Kimi-Linear layers,
    alternating layers token by token."""
    from oracle import pyoracle as po
    if not os.path.exists(po.REF_LIB):
        return None
    d, own = kimi_twin(args)
    xs = np.random.default_rng(3).standard_normal((64, KH), dtype=np.float32)

    def warm(ref):
        for t in range(128):                       # fills the reference's cache
            ref.moe_layer(t & 1, xs[t % 64], KE, KK, KH)

    def one(ref, i):
        ref.moe_layer(i & 1, xs[i % 64], KE, KK, KH)
    res = ref_rows(d, KIMI_CACHE, warm, one, 1, seconds, {
        "unit": "MoE-layer tokens/s",
        "sample": "{n} decode tokens through two Kimi-Linear-shape layers in turn (H 2304, I 1024, top-8 of 256 "
                  "experts, Q8G shared expert; 1.37 GB of records) in the reference's VQ3R format (3x256, 3.00 "
                  "bits/weight), its own moe_layer ({isa}) over {threads} threads, {secs:.1f}s; the reference "
                  "routes with sigmoid scores (softmax is not in it)"})
    if own:
        shutil.rmtree(os.path.dirname(d), ignore_errors=True)
    return res


def cpu_baseline_prefill(args, seconds, T):
    """The reference's moe_chunk on the VQ3R twin of two Kimi-Linear layers,
    chunks of 64 tokens (its prefill chunk, src/model.h:285), alternating
    layers."""
    from oracle import pyoracle as po
    if not os.path.exists(po.REF_LIB):
        return None
    d, own = kimi_twin(args)
    chunk = 64
    Xs = np.random.default_rng(3).standard_normal((8, chunk, KH), dtype=np.float32)

    def warm(ref):
        for t in range(8):
            ref.moe_chunk(t & 1, Xs[t], KK, KH)

    def one(ref, i):
        ref.moe_chunk(i & 1, Xs[i % 8], KK, KH)
    res = ref_rows(d, KIMI_CACHE, warm, one, chunk, seconds, {
        "unit": "MoE-layer tokens/s",
        "sample": "{n} prefill tokens in chunks of 64 through two Kimi-Linear-shape layers in turn (H 2304, I 1024, "
                  "top-8 of 256 experts, Q8G shared expert) in the reference's VQ3R format (3x256, 3.00 "
                  "bits/weight), its own moe_chunk ({isa}) over {threads} threads, {secs:.1f}s; the reference routes "
                  "with sigmoid scores (softmax is not in it)"})
    if own:
        shutil.rmtree(os.path.dirname(d), ignore_errors=True)
    return res


def cpu_baseline_miss(args, seconds, T):
    """The reference's moe_chunk on the VQ3R twin of a K3 layer (64 experts)
    with its expert cache holding half of them: a T-token batch picks about
    all 64, so about half of every chunk's distinct records miss and are
    read from the container (page cache) by its bank_fetch
    (src/model.c:1767-1795, src/ecache.c:596-669)."""
    from oracle import pyoracle as po
    if not os.path.exists(po.REF_LIB):
        return None
    d, own = twin_dir(args, "k3_vq3r_64", k3_twin_spec())
    Xs = np.random.default_rng(4).standard_normal((4, T, H), dtype=np.float32)

    def warm(ref):
        ref.moe_chunk(0, Xs[0], K, H)

    def one(ref, i):
        ref.moe_chunk(0, Xs[i % 4], K, H)
    res = ref_rows(d, 32 * 16_600_000, warm, one, T, seconds, {
        "unit": "MoE-layer tokens/s",
        "sample": "{n} decode tokens in batches of " + str(T) + " through a K3-shape layer (H 7168, I 2048, top-16 "
                  "of 64 experts) in the reference's VQ3R format, its own moe_chunk ({isa}) over {threads} "
                  "threads, {secs:.1f}s, with its expert cache at 32 records (half of the 64 the batch picks): "
                  "misses read from the container through its bank_fetch, served by the host's page cache, so "
                  "this prices the CPU path's compute plus a host memory copy, not a storage read"})
    if own:
        shutil.rmtree(os.path.dirname(d), ignore_errors=True)
    return res


MISS_METRIC = "MoE-layer tokens/s with half the selected expert records missing from HBM, K3-scale, 1 MI355X"


def miss_pool(ctx, layers, seed=99):
    """Every expert record of the stack in pinned host memory, as the
    cache's host tier holds them: one random code payload varied per record
    by a byte XOR (any 12-bit code is a valid index), per-record header and
    fp16 row scales ~U(0.01, 0.05)."""
    import struct
    import container as ct
    gate, down, scales_b, rec_bytes = rec_layout()
    pool = ctx.host_alloc(layers * E * rec_bytes)
    rng = np.random.Generator(np.random.PCG64(seed))
    tmpl = rng.integers(0, 256, size=rec_bytes, dtype=np.uint8)
    offs = (ct.HDR, ct.HDR + gate, ct.HDR + 2 * gate, ct.HDR + 2 * gate + down)
    for L in range(layers):
        for e in range(E):
            i = L * E + e
            r = pool[i * rec_bytes:(i + 1) * rec_bytes]
            np.bitwise_xor(tmpl, np.uint8((i * 37 + 11) & 0xFF), out=r)
            r[:ct.HDR] = np.frombuffer(struct.pack("<IHHBBHHHIIIIIIII", ct.MAGIC_EXPERT, L, e, ct.FMT_CODE["VQ12"],
                                                   0, L * 3 * S, 0, 0, rec_bytes // ct.ALIGN, *offs, 0, 0, 0),
                                       np.uint8)
            r[offs[3]:offs[3] + scales_b] = rng.uniform(0.01, 0.05, size=scales_b // 2).astype(np.float16).view(
                np.uint8)
        log(f"bench: host tier, {L + 1}/{layers} layers of records")
    return pool, rec_bytes


def h2d_peak(pool, nbytes=1 << 30, reps=3):
    """The pinned host-to-device copy rate of this box: the best of a few
    synchronous copies of `nbytes` from the host tier."""
    from warp_amd.device import Buf, H2D, check, rt
    dst = Buf(nbytes)
    best = 0.0
    for _ in range(reps):
        t0 = time.perf_counter()
        check(rt().hipMemcpy(dst.ptr, pool.ctypes.data, nbytes, H2D), "H2D calibration copy")
        best = max(best, nbytes / (time.perf_counter() - t0) / 1e9)
    dst.free()
    return best


def run_miss(args):
    """One step = one batch of T decode tokens (one per sequence, ragged
    sequences) through `layers` K3 layers, h <- h + moe(h). The HBM cache
    holds a fraction of the stack's records; the rest stream in from pinned
    host memory on the copy stream. Three passes over the same inputs: no
    lookahead, lookahead (each token's top-16 predicted for layer L+1 from
    layer L's input, fetched while layer L computes), and every record
    resident (the compute alone)."""
    import warp_amd
    from warp_amd.device import Buf, Event
    T, layers = args.tokens, args.layers
    rng = np.random.Generator(np.random.PCG64(2468))
    books = [rng.normal(0.0, 0.02, size=(3 * S, EN, 8)).astype(np.float16).view(np.uint16) for _ in range(layers)]
    routers = [rng.standard_normal((E, H), dtype=np.float32) * np.float32(0.02) for _ in range(layers)]
    n_in = args.warmup + args.steps
    X = Buf.of(rng.standard_normal((n_in, T, H), dtype=np.float32))
    outs = [Buf.empty((T, H)) for _ in range(layers)]
    slots = int(round(args.cache_frac * layers * E))
    pool, rec_bytes = None, None

    def open_pass(n_slots, lookahead):
        nonlocal pool, rec_bytes
        _, _, _, rb = rec_layout()
        ctx = warp_amd.Context(hidden=H, inter=I, n_experts=E, top_k=K, n_layers=layers, fmt="VQ12", renorm=True,
                               routed_scale=1.0, max_tokens=T, rec_bytes=rb, cache_bytes=n_slots * rb,
                               lookahead=lookahead)
        for L in range(layers):
            ctx.set_codebooks(L, L * 3 * S, books[L])
            ctx.set_router(L, routers[L], np.zeros(E, np.float32))
        if pool is None:
            pool, rec_bytes = miss_pool(ctx, layers)
        base = pool.ctypes.data
        ctx.set_fetch_host(lambda L, e: base + (L * E + e) * rec_bytes)
        return ctx

    def run_pass(ctx, name):
        def step(s):
            h = X.ptr + s * T * H * 4
            for L in range(layers):
                ctx.moe_chunk(L, h, outs[L].ptr, T, resid_dev=h)
                h = outs[L].ptr
        for s in range(args.warmup):
            step(s)
        ctx.sync()
        st0 = ctx.cache_stats()
        e0, e1 = Event(), Event()
        log(f"bench: {name}: timing {args.steps} steps of {T} tokens x {layers} layers")
        t0 = time.perf_counter()
        e0.record(ctx.stream)
        for s in range(args.steps):
            step(args.warmup + s)
        e1.record(ctx.stream)
        e1.synchronize()
        ctx.sync()
        wall = time.perf_counter() - t0
        ms = e0.elapsed_ms(e1)
        st1 = ctx.cache_stats()
        d = {k: st1[k] - st0[k] for k in ("hits", "misses", "spec_issued", "bytes_read", "evictions")}
        n_lt = args.steps * layers
        sel = d["hits"] + d["misses"]
        out = outs[layers - 1].numpy()
        assert np.isfinite(out).all(), "non-finite hidden state after the stack"
        return {"tokens_per_s": round(T * n_lt / (wall), 1), "ms_per_layer": round(wall * 1e3 / n_lt, 3),
                "event_ms_per_layer": round(ms / n_lt, 3),
                "miss_rate": round(d["misses"] / max(sel, 1), 4),
                "records_per_layer": round(sel / n_lt, 1),
                "fetched_per_layer": round((d["misses"] + d["spec_issued"]) / n_lt, 1),
                "spec_per_layer": round(d["spec_issued"] / n_lt, 1),
                "h2d_gb_per_layer": round(d["bytes_read"] / n_lt / 1e9, 4),
                "h2d_gbs": round(d["bytes_read"] / wall / 1e9, 2)}

    res = {}
    ctx = open_pass(slots, 0)
    peak = h2d_peak(pool)
    log(f"bench: pinned host-to-device copy {peak:.1f} GB/s")
    res["no_lookahead"] = run_pass(ctx, "no lookahead")
    ctx.close()
    ctx = open_pass(slots, args.lookahead)
    res["lookahead"] = run_pass(ctx, f"lookahead {args.lookahead} per token")
    ctx.close()
    ctx = open_pass(layers * E, 0)
    for L in range(layers):
        ctx.prefetch(L, np.arange(E))
    ctx.sync()
    res["resident"] = run_pass(ctx, "all resident")
    ctx.close()
    ctx.host_free(pool)
    la = res["lookahead"]
    copy_ms = la["h2d_gb_per_layer"] / peak * 1e3
    return {
        "metric": MISS_METRIC,
        "value": la["tokens_per_s"],
        "unit": "MoE-layer tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(la["ms_per_layer"] * layers, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (random codes, codebooks, scales and routers of the K3 shapes; uniform routing)",
        "config": {"workload": f"K3-scale MoE layer, {T}-token decode batch (one token per sequence), "
                               f"{layers}-layer stack, HBM cache of {slots} records ({args.cache_frac:.2f} of the "
                               "stack), misses from pinned host memory",
                   "hidden": H, "inter": I, "experts": E, "top_k": K, "tokens": T, "layers": layers,
                   "cache_slots": slots, "record_bytes": rec_layout()[3], "lookahead_per_token": args.lookahead,
                   "parallelism": "single GPU"},
        "passes": res,
        "roofline": {"bound": "host-to-device copy", "achieved": la["h2d_gbs"], "peak": round(peak, 2),
                     "unit": "GB/s", "frac": round(la["h2d_gbs"] / peak, 4), "traffic": None,
                     "peak_source": "best of 3 synchronous 1 GiB copies from the pinned host tier"},
        "layer_ms_bounds": {"copy_at_peak": round(copy_ms, 3), "compute_resident": res["resident"]["ms_per_layer"],
                            "measured": la["ms_per_layer"]},
        "cpu_baseline": None if args.no_cpu else cpu_baseline_miss(args, args.cpu_seconds, T),
    }


VALU_PEAK_OPS = 78.6e12   # fp32 vector operations/s: the 157.3 TFLOP/s vector peak counts an FMA as 2


def run_vq_encode(args):
    """The encoder (waste_vq_encode) on one K3 gate matrix: 2048 x 7168
    weights = 1,835,008 vectors of 8, N(0, 1), on device buffers; the
    3 x 256 codebooks of the reference's own format and the 2 x 4096 of the
    12-bit format. A step encodes the whole matrix."""
    import warp_amd.hip as wh
    from warp_amd.device import Buf, Event, check, rt
    n = I * H // 8
    rng = np.random.Generator(np.random.PCG64(97))
    X = Buf.of(rng.standard_normal((n, 8), dtype=np.float32))
    resid = Buf.empty((n, 8))
    codes = Buf.empty((n, 3), np.uint16)
    res = {}
    for S_, E_ in ((3, 256), (2, 4096)):
        books = Buf.of(rng.standard_normal((S_, E_, 8), dtype=np.float32))

        def step():
            rc = wh.lib().warp_hip_vq_encode_dev(X.ptr, n, books.ptr, S_, E_, resid.ptr, codes.ptr, None)
            if rc:
                raise wh.WarpHipError(rc, "vq_encode_dev")
        for _ in range(args.warmup):
            step()
        check(rt().hipDeviceSynchronize(), "sync")
        e0, e1 = Event(), Event()
        e0.record(None)
        for _ in range(args.steps):
            step()
        e1.record(None)
        e1.synchronize()
        ms = e0.elapsed_ms(e1) / args.steps
        ops = n * S_ * E_ * 25.0                     # per entry: 8 subtract, 8 multiply, 8 add, 1 compare
        res[f"{S_}x{E_}"] = {"ms_per_matrix": round(ms, 3), "vectors_per_s": round(n / (ms / 1e3), 1),
                             "valu_ops_per_s": ops / (ms / 1e3), "valu_frac": round(ops / (ms / 1e3) / VALU_PEAK_OPS, 4)}
        log(f"bench: vq-encode {S_}x{E_}: {ms:.3f} ms per matrix")
        books.free()
    main = res["3x256"]                               # the reference's format, beside its CPU encoder
    cpu = None if args.no_cpu else cpu_baseline_encode(args.cpu_seconds)
    return {
        "metric": "VQ-encoded vectors/s (waste_vq_encode, 8-dim vectors), 1 MI355X",
        "value": main["vectors_per_s"],
        "unit": "vectors/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": main["ms_per_matrix"],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp32",
        "data": "synthetic (N(0,1) vectors and codebooks)",
        "config": {"workload": "encode one K3 gate matrix (2048 x 7168 weights, 1,835,008 vectors of 8) with "
                               "3 x 256 codebooks (the reference's format); 2 x 4096 (16-bit codes) beside it",
                   "vectors": n, "parallelism": "single GPU"},
        "passes": {k: {kk: (round(vv, 1) if isinstance(vv, float) and kk != "valu_frac" else vv)
                       for kk, vv in v.items()} for k, v in res.items()},
        "roofline": {"bound": "valu", "achieved": round(main["valu_ops_per_s"] / 1e12, 2),
                     "peak": round(VALU_PEAK_OPS / 1e12, 2), "unit": "T fp32 vector ops/s",
                     "frac": main["valu_frac"], "traffic": None,
                     "kernel": "k_vq_encode_stage (a scan of every codebook entry per vector and stage)"},
        "cpu_baseline": cpu,
    }


def cpu_baseline_encode(seconds):
    """The reference's waste_vq_encode (oracle/_ref) on the 3 x 256 case."""
    import ctypes
    from oracle import pyoracle as po
    if not os.path.exists(po.REF_LIB):
        return None
    L = ctypes.CDLL(po.REF_LIB)
    L.waste_vq_encode.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                  ctypes.c_int, ctypes.c_void_p, ctypes.c_int]
    L.waste_vq_encode.restype = None
    threads = cpu_threads()
    rng = np.random.default_rng(98)
    m = 1 << 16
    X = rng.standard_normal((m, 8), dtype=np.float32)
    books = rng.standard_normal((3, 256, 8), dtype=np.float32)
    out = np.empty((m, 3), np.uint8)
    L.waste_vq_encode(X.ctypes.data, m, books.ctypes.data, 3, 256, 8, out.ctypes.data, threads)
    k, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        L.waste_vq_encode(X.ctypes.data, m, books.ctypes.data, 3, 256, 8, out.ctypes.data, threads)
        k += 1
    dt = time.perf_counter() - t0
    return {"value": k * m / dt, "unit": "vectors/s", "cores": threads, "kind": "reference",
            "sample": f"{k} calls of waste_vq_encode on {m} vectors with 3 x 256 codebooks (the reference's "
                      f"8-bit codes; it has no 4096-entry encoder) over {threads} threads, {dt:.1f}s"}


# ---- the dispatch table's slots as the engine calls them -------------------------------------

def _tables():
    """ctypes types of the reference's dispatch table (src/waste_backend.h:67-90)
    and mvq_arg (src/simd.h:35-39)."""
    import ctypes as C

    class MvqArg(C.Structure):
        _fields_ = [("y", C.c_void_p), ("W", C.c_void_p), ("ws", C.c_void_p), ("xq", C.c_void_p),
                    ("xs", C.c_void_p), ("in_", C.c_int), ("ng", C.c_int), ("group", C.c_int), ("bits", C.c_int),
                    ("rowbytes", C.c_size_t)]

    class Table(C.Structure):
        _fields_ = [("kda_step", C.c_void_p), ("short_conv_step", C.c_void_p), ("rmsnorm_gated", C.c_void_p),
                    ("mvq_rows_f32", C.c_void_p), ("lutb_range", C.c_void_p), ("on_device", C.c_int)]
    slot = C.CFUNCTYPE(None, C.c_int, C.c_int, C.c_void_p)
    kda = C.CFUNCTYPE(None, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                      C.c_void_p, C.c_void_p, C.c_void_p)
    return MvqArg, Table, slot, kda


def _time_calls(fn, seconds, min_calls=5):
    n, t0 = 0, time.perf_counter()
    while n < min_calls or time.perf_counter() - t0 < seconds:
        fn()
        n += 1
    return (time.perf_counter() - t0) / n, n


# (name, rows, in, bits, group): a Kimi-Linear shared expert's gate rows, a
# quantised K3 router, a K3 trunk projection, a slice of a K3 lm_head
MVQ_SHAPES = [("kimi_shared_gate_q8g32", 1024, 2304, 8, 32), ("k3_router_q8g128", 384, 7168, 8, 128),
              ("k3_proj_q8g128", 7168, 7168, 8, 128), ("k3_lm_head_slice_q8g128", 16384, 7168, 8, 128)]
KDA_SHAPES = [("kimi_linear_kda_h32_k128_v128", 32, 128, 128)]


def run_table_slots(args):
    """The reference's dispatch-table slots as its engine calls them, with
    host pointers: mvq_rows_f32 (run_rows hands a device backend the whole row
    range in one call, src/model.c:356-360) and kda_step (one decode step of
    every head, src/kda.c:26-68), through the table waste_register_hip fills,
    against the same slots of the reference's own table (oracle/_ref,
    waste_backend_init's AVX-512 build) on this host: its mvq rows split over
    the host threads in 64-row ranges as its pool splits them, and over one
    thread; its kda_step on one thread, as the engine calls it."""
    import ctypes as C
    from concurrent.futures import ThreadPoolExecutor
    import warp_amd
    from oracle import pyoracle as po
    MvqArg, Table, Slot, Kda = _tables()
    t = Table()
    assert warp_amd.lib().waste_register_hip(C.byref(t)), "no gfx950 device"
    dev_mvq, dev_kda = Slot(t.mvq_rows_f32), Kda(t.kda_step)
    ref_mvq = ref_kda = None
    isa = None
    if not args.no_cpu and os.path.exists(po.REF_LIB):
        R = C.CDLL(po.REF_LIB)
        R.waste_backend_init.argtypes = [C.c_uint]
        R.waste_backend_init(0)
        R.waste_backend_name.restype = C.c_char_p
        isa = R.waste_backend_name().decode()
        rt = Table.in_dll(R, "waste_k")
        ref_mvq, ref_kda = Slot(rt.mvq_rows_f32), Kda(rt.kda_step)
    threads = cpu_threads()
    pool = ThreadPoolExecutor(threads)          # the reference's pool keeps its threads too
    secs = max(0.5, args.cpu_seconds / 8)
    rng = np.random.default_rng(42)
    out = {"mvq_rows_f32": {}, "kda_step": {}}
    for name, rows, n, bits, group in MVQ_SHAPES:
        ng = n // group
        W = rng.integers(-127, 128, size=(rows, n), dtype=np.int8)
        ws = rng.uniform(0.002, 0.02, size=(rows, ng)).astype(np.float16).view(np.uint16)
        x = rng.standard_normal(n).astype(np.float32)
        yd, yc = np.empty(rows, np.float32), np.empty(rows, np.float32)
        ad = MvqArg(yd.ctypes.data, W.ctypes.data, ws.ctypes.data, None, x.ctypes.data, n, ng, group, bits, n)
        ac = MvqArg(yc.ctypes.data, W.ctypes.data, ws.ctypes.data, None, x.ctypes.data, n, ng, group, bits, n)
        pd, pc = C.cast(C.pointer(ad), C.c_void_p), C.cast(C.pointer(ac), C.c_void_p)
        dev_mvq(0, rows, pd)                                      # the device mirror of W is made once
        s_dev, k_dev = _time_calls(lambda: dev_mvq(0, rows, pd), secs)
        nbytes = rows * (n + 2 * ng)
        row = {"rows": rows, "in": n, "bits": bits, "group": group, "weight_bytes": nbytes,
               "device_us_per_call": round(s_dev * 1e6, 1), "device_calls": k_dev,
               "device_weight_gbs": round(nbytes / s_dev / 1e9, 1)}
        if ref_mvq is not None:
            ref_mvq(0, rows, pc)
            assert np.allclose(yd, yc, rtol=1e-4, atol=1e-3 * float(np.max(np.abs(yc)))), name

            step = max(64, (rows // threads + 63) // 64 * 64)
            cut = [(b, min(b + step, rows)) for b in range(0, rows, step)]

            def pooled():
                for f in [pool.submit(ref_mvq, b, e, pc) for b, e in cut]:
                    f.result()
            s_cpu, _ = _time_calls(pooled, secs)
            s_one, _ = _time_calls(lambda: ref_mvq(0, rows, pc), secs / 2)
            row.update({"cpu_us_per_call": round(s_cpu * 1e6, 1), "cpu_threads": threads,
                        "cpu_one_thread_us_per_call": round(s_one * 1e6, 1),
                        "speedup_vs_cpu": round(min(s_cpu, s_one) / s_dev, 2)})
        out["mvq_rows_f32"][name] = row
        log(f"bench: mvq slot {name}: device {s_dev * 1e6:.1f} us" +
            (f", reference {row['cpu_us_per_call']:.1f} us ({threads} threads) / "
             f"{row['cpu_one_thread_us_per_call']:.1f} us (1)" if "cpu_us_per_call" in row else ""))
        warp_amd.lib().waste_hip_release_host_buffers()
    for name, Hh, Kk, Vv in KDA_SHAPES:
        q, k = rng.standard_normal((Hh, Kk)).astype(np.float32), rng.standard_normal((Hh, Kk)).astype(np.float32)
        v = rng.standard_normal((Hh, Vv)).astype(np.float32)
        g = -np.abs(rng.standard_normal((Hh, Kk))).astype(np.float32) * 0.1
        beta = rng.uniform(0.1, 0.9, Hh).astype(np.float32)
        S0 = (rng.standard_normal((Hh, Kk, Vv)) * 0.1).astype(np.float32)
        o = np.empty((Hh, Vv), np.float32)
        scratch = np.empty(Vv, np.float32)              # waste_kda_step's u [V]
        Sd, Sc = S0.copy(), S0.copy()
        ptrs = lambda S_: [a.ctypes.data for a in (q, k, v, g, beta)] + [S_.ctypes.data, o.ctypes.data,
                                                                          scratch.ctypes.data]
        pd_, pc_ = ptrs(Sd), ptrs(Sc)
        s_dev, k_dev = _time_calls(lambda: dev_kda(Hh, Kk, Vv, *pd_), secs)
        sbytes = Hh * Kk * Vv * 4
        row = {"H": Hh, "K": Kk, "V": Vv, "state_bytes": sbytes, "device_us_per_call": round(s_dev * 1e6, 1),
               "device_calls": k_dev}
        if ref_kda is not None:
            s_one, _ = _time_calls(lambda: ref_kda(Hh, Kk, Vv, *pc_), secs)
            row.update({"cpu_one_thread_us_per_call": round(s_one * 1e6, 1),
                        "speedup_vs_cpu": round(s_one / s_dev, 2)})
        out["kda_step"][name] = row
        log(f"bench: kda slot {name}: device {s_dev * 1e6:.1f} us" +
            (f", reference {row['cpu_one_thread_us_per_call']:.1f} us (1 thread)" if ref_kda is not None else ""))
    dstat, fstat = (C.c_uint64(), C.c_uint64())
    warp_amd.lib().warp_hip_table_stats(C.byref(dstat), C.byref(fstat))
    main = out["mvq_rows_f32"]["k3_proj_q8g128"]
    return {
        "metric": "dispatch-table slot calls/s as the engine calls them (host pointers), 1 MI355X",
        "value": round(1.0 / (main["device_us_per_call"] / 1e6), 1),
        "unit": "mvq_rows_f32 calls/s (K3 trunk projection, 7168 x 7168 Q8G g128)",
        "n_gpus": 1, "steps": None, "warmup": 1, "ms_per_step": round(main["device_us_per_call"] / 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8 x fp32",
        "data": "synthetic (random Q8G rows, fp16 scales, N(0,1) activations; KDA inputs and state)",
        "config": {"workload": "the mvq_rows_f32 and kda_step slots of the reference's table through "
                               "waste_register_hip, per call: inputs host to device, kernel, outputs back",
                   "parallelism": "single GPU"},
        "slots": out, "cpu_isa": isa, "fallback_calls": fstat.value,
        "roofline": {"bound": "hbm", "achieved": main["device_weight_gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(main["device_weight_gbs"] / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "k_mvq through the mvq_rows_f32 slot, whole call (copies and wait included)"},
        "cpu_baseline": None if ref_mvq is None else {
            "value": round(1.0 / (min(main["cpu_us_per_call"], main["cpu_one_thread_us_per_call"]) / 1e6), 1),
            "unit": "mvq_rows_f32 calls/s", "cores": threads if main["cpu_us_per_call"] <=
            main["cpu_one_thread_us_per_call"] else 1, "kind": "reference",
            "sample": f"the reference's {isa} mvq_rows_f32 slot on the same rows, split in 64-row ranges over "
                      f"{threads} threads and on one thread (the better kept)"},
    }


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--workload", choices=["k3-decode", "single-expert", "kimi-prefill", "k3-miss", "kimi-decode",
                                           "vq-encode", "table-slots"],
                    default="k3-decode",
                    help="k3-decode (the headline line), single-expert (one expert's FFN, decode), kimi-prefill "
                         "(a 512-token Kimi-Linear-shape prefill), k3-miss (a 32-token K3 decode batch with half its "
                         "expert records streamed from host), kimi-decode (Kimi-Linear-shape decode, batch 1, with "
                         "its shared expert), vq-encode (the encoder on one K3 matrix) or table-slots (the "
                         "dispatch table's mvq_rows_f32 and kda_step slots as the engine calls them)")
    ap.add_argument("--only", action="store_true",
                    help="k3-decode: the headline line alone, without the other configurations' children")
    ap.add_argument("--twin-dir", default=None,
                    help="directory for the CPU baselines' twin containers (shared by the children of one run)")
    ap.add_argument("--child-timeout", type=float, default=420.0,
                    help="seconds allowed to each other configuration's child process")
    ap.add_argument("--tokens", type=int, default=None,
                    help="tokens per step: kimi-prefill (default 512), k3-miss (default 32)")
    ap.add_argument("--cache-frac", type=float, default=0.69,
                    help="k3-miss: HBM cache slots as a fraction of the stack's records")
    ap.add_argument("--lookahead", type=int, default=4,
                    help="k3-miss: experts of layer L+1 predicted per token from layer L's input")
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--layers", type=int, default=None,
                    help="layers in the stack: k3-decode 60, kimi-prefill 4, k3-miss 4, kimi-decode 26")
    ap.add_argument("--resident", type=int, default=64, help="expert records per layer kept in HBM")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="seconds of the reference's CPU path per baseline (the one-thread row gets half)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-graph", dest="graph", action="store_false",
                    help="k3-decode, kimi-decode: launch every kernel from the host instead of replaying one "
                         "captured step")
    ap.add_argument("--router", choices=sorted(ROUTERS), default="cert",
                    help="K3 decode: cert = certified selection (the reference's picks by construction), fast = "
                         "the fast logits' picks uncertified, strict = every logit in the reference's sequential "
                         "order")
    ap.add_argument("--matvec-path", choices=["auto", "mfma", "fused", "gather"], default="auto",
                    help="expert matvec kernel: auto = the LUT kernel (the row kernel for one expert), mfma = "
                         "decode-then-dot on the matrix cores, fused = the LUT kernel's gate/up, down and combine in "
                         "one launch per layer, gather = decode-then-dot with codebook gathers")
    ap.add_argument("--prefill", choices=["exact", "fp16"], default="fp16",
                    help="kimi-prefill: the expert products' precision: fp16 (the configuration's decode-to-16-bit + "
                         "MFMA design: stages added into one fp16 operand against x's fp16 high half, outputs within "
                         "2e-3) or exact (fp16 hi/lo halves of x, every stage a product of its own, within 1e-4); "
                         "the default run also times the exact mode in a child of its own")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="before timing, one device-to-device copy of this many MiB (a known-size "
                         "kernel for scaling the profiler's traffic counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one MI355X; --gpus {args.gpus} is not supported: the path runs on a "
              "single GPU (experts would shard across GPUs by owner, with an all-to-all of token groups "
              "for prefill; not built)", file=sys.stderr)
        sys.exit(2)

    if args.workload == "single-expert":
        print(json.dumps(run_single_expert(args)))
        return
    if args.workload == "kimi-prefill":
        args.layers = args.layers or 4
        args.tokens = args.tokens or 512
        print(json.dumps(run_prefill(args)))
        return
    if args.workload == "vq-encode":
        print(json.dumps(run_vq_encode(args)))
        return
    if args.workload == "table-slots":
        print(json.dumps(run_table_slots(args)))
        return
    if args.workload == "kimi-decode":
        args.layers = args.layers or 26
        print(json.dumps(run_kimi_decode(args)))
        return
    if args.workload == "k3-miss":
        args.layers = args.layers or 4
        args.tokens = args.tokens or 32
        print(json.dumps(run_miss(args)))
        return
    args.layers = args.layers or 60
    workloads = {}
    if not args.twin_dir:
        # one directory of twin containers for the whole run, removed at exit
        import atexit
        args.twin_dir = tempfile.mkdtemp(prefix="warp_bench_twins_")
        atexit.register(shutil.rmtree, args.twin_dir, True)
    if not args.only:
        # the other configurations first, each in a child process, before this
        # process touches the GPU
        workloads = run_children(args)
    ms, wall, kms, kn, st = run_gpu(args)
    steps, layers = args.steps, args.layers
    layer_tokens = steps * layers
    value = layer_tokens / (ms / 1e3)
    # the expert matvec: class 0 gate+up launches, class 1 down launches
    gate, down, scales_b, _ = rec_layout()
    b0 = K * (2 * gate + 2 * 2 * I)               # codes + gate/up row scales per gate/up launch
    b1 = K * (down + 2 * H)                       # codes + down row scales per down launch
    kernel, fused, achieved, per = matvec_roofline(kms, kn, b0, b1, args.kernel)
    layer_gbs = layer_bytes() * layer_tokens / (ms / 1e3) / 1e9
    tr, tr_why = measured_traffic(kernel, ("fused",) if fused else ("gate_up", "down"))
    traffic = None
    if tr:
        traffic = tr["fused"] if fused else round((kn[0] * tr["gate_up"] + kn[1] * tr["down"]) /
                                                  max(kn[0] + kn[1], 1))
    cpu = None if args.no_cpu else cpu_baseline(args, args.cpu_seconds)
    rec = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "MoE-layer tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms / steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (random codes, codebooks, scales and routers of the K3 shapes)",
        "launch": "one step captured as a HIP graph and replayed per token" if args.graph else "host launches",
        "router": ROUTERS[args.router],
        "router_recompute": args.route_recompute if args.router == "cert" else None,
        "router_cost": args.router_cost,
        "config": {"workload": "K3-scale MoE decode layer, batch 1, 60-layer stack",
                   "hidden": H, "inter": I, "experts": E, "top_k": K, "layers": layers,
                   "format": "RVQ 2x4096 12-bit codes (3.00 b/w)", "resident_per_layer": args.resident,
                   "parallelism": "single GPU"},
        "layer_hbm_gbs": round(layer_gbs, 1),
        "layer_hbm_frac": round(layer_gbs / HBM_PEAK_GBS, 4),
        "layer_bytes": layer_bytes(),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_per_launch": tr if tr else {"unmeasured": tr_why},
                     "kernel": per["what"],
                     "timing": "HIP events around each launch on the compute stream, in a second pass of the "
                               "same steps",
                     "bytes_per_launch": per["bytes_per_launch"],
                     "avg_launch_us": per["avg_launch_us"],
                     "router_avg_us": round(kms[2] / max(kn[2], 1) * 1e3, 2)},
        "cache": {"hits": st["hits"], "misses": st["misses"], "resident": st["resident"]},
        "wall_s": round(wall, 3),
        "cpu_baseline": cpu,
        "workloads": workloads,
    }
    print(json.dumps(rec))


# (key, workload, extra arguments): the prefill twice, in the precision
# mode asked for and in the exact mode (its CPU baseline is the same)
CHILDREN = [("single_expert", "single-expert", []), ("kimi_decode", "kimi-decode", []),
            ("kimi_prefill", "kimi-prefill", []), ("kimi_prefill_exact", "kimi-prefill", ["--prefill", "exact", "--no-cpu"]),
            ("k3_miss", "k3-miss", []), ("table_slots", "table-slots", [])]


def run_children(args):
    """The other configurations (the prefill in both precision modes), each `bench.py --workload X` in a child
    process (its own HIP context and memory), with this run's step counts
    and CPU-baseline seconds; a child that fails is reported, not fatal."""
    import subprocess
    out = {}
    for key, wl, extra in CHILDREN:
        if key == "kimi_prefill_exact" and args.prefill == "exact":
            continue
        cmd = [sys.executable, os.path.abspath(__file__), "--workload", wl, "--twin-dir", args.twin_dir,
               "--cpu-seconds", str(args.cpu_seconds), "--matvec-path", args.matvec_path,
               "--prefill", args.prefill]
        if wl == "k3-miss":
            cmd += ["--steps", "8", "--warmup", "2"]
        else:
            cmd += ["--steps", str(args.steps), "--warmup", str(args.warmup)]
        if args.no_cpu:
            cmd.append("--no-cpu")
        if not args.graph:
            cmd.append("--no-graph")
        cmd += extra
        log(f"bench: configuration {key} in a child process")
        t0 = time.perf_counter()
        try:
            r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=None, text=True, timeout=args.child_timeout)
            lines = [l for l in r.stdout.splitlines() if l.startswith("{")]
            if r.returncode == 0 and lines:
                out[key] = json.loads(lines[-1])
                out[key]["child_wall_s"] = round(time.perf_counter() - t0, 1)
            else:
                out[key] = {"error": f"exit status {r.returncode}", "stdout_tail": r.stdout[-400:]}
        except subprocess.TimeoutExpired:
            out[key] = {"error": f"did not finish in {args.child_timeout:.0f}s"}
        log(f"bench: configuration {key}: " + ("ok" if "error" not in out[key] else out[key]["error"]))
    # the two prefill modes share their CPU baseline (the same 512 tokens
    # through the reference's moe_chunk), measured once
    fp, ex = out.get("kimi_prefill"), out.get("kimi_prefill_exact")
    if fp and ex and "error" not in fp and "error" not in ex and fp.get("cpu_baseline") and not ex.get("cpu_baseline"):
        ex["cpu_baseline"] = dict(fp["cpu_baseline"], shared_with="kimi_prefill")
    return out


if __name__ == "__main__":
    main()
