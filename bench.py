#!/usr/bin/env python3
"""Decode throughput of lgml's ragged continuous-batching path on one MI355X.

Default workload ("C2"): a Llama-3-8B-shaped model
(32 layers, d 4096, 32 / 8 heads, head 128, FFN 14336, vocab 128256) with
N(0, 0.02) weights quantized Q4_K_M (output and attn_v / ffn_down of the
more_bits layers Q6_K), f16 KV in 64-cell blocks; 64 slots with prompt
lengths U[128, 4096]; continuous batching: a request's decode budget is
U[64, 2048]; a finished request's slot is taken by a new one whose prompt
(U[128, 4096]) is prefilled in 512-token chunks mixed into the decode
passes. The run starts in the steady state of that process: each initial
request has already decoded part of its budget (what is left is U[1,
budget]), so requests finish and join from the first steps on, also in a
20-step run. The initial contexts are filled with synthetic KV (the
attention reads cost the same whatever the values); joining prompts run
the real prefill. One step = one pass of the engine (E:flush): the next
token of every decoding slot plus the prompt chunks of joining slots.

--workload c3: the same 8B model with prefix
caching. A 2048-token system prefix is prefilled once and its 32 blocks
are published; 64 requests of prefix + a unique suffix U[16, 512] attach
those blocks (refcounts up to 64) and run only their suffixes; joins do
the same, their suffix prefilled in 512-token chunks mixed into the
decode pass (a pass carries the decode tokens and at most 512 prompt
tokens). Attention bytes are reported both logical (every sequence's own
context, the §8(d) figure the roofline uses) and unique (the shared
prefix once).

--workload c5: the same loop on a 30B-A3B-shaped
qwen3moe (48 layers, d 2048, 32 / 4 heads, head 128, 128 experts of width
768, top-8 softmax routing, router logits N(0, 1), Q4_K), prompts
U[256, 8192]: tokens are grouped by expert for the grouped Q4_K expert
products.

--workload c4: a Gemma-4-style model (26 layers,
d 2560, 8 / 4 heads of 256, 5 sliding-window layers with a 1024-token ring
per slot to 1 global layer, GeGLU FFN 10240, vocab 262144 tied, Q8_0), 32
slots with contexts U[1024, 16384] decoding (no joins: every budget
outlasts the run).

value = decoded tokens / wall seconds of the K timed steps of the mixed
phase (continuous batching with joins; inputs resident in HBM; the
per-step host plan upload and the sampled ids read back are inside; no
instrumentation). config.decode_only is a second timed phase of K steps
in which every pass is pure decode at full occupancy (finished slots are
refilled with already-prefilled requests). The engine runs ahead by one
pass (the next pass is planned and queued before the previous one's
tokens are read back; decode tokens go from pass to pass on the device);
--sync reads every pass back first. roofline = the paged attention kernel
(the dominant kernel: ~80% of a C2 step's bytes): its algorithmic bytes
(K + V of every visible cell, q in, out) per launch over its duration,
timed with HIP events on the pass's stream during min(K, 16) further decode
steps, against 8 TB/s. prefill_roofline = the weight products of one
512-token prompt chunk (a joining request's pass) against the MFMA peak.
cpu_baseline = the C oracle (oracle/) timed on a bounded sample of the same
step on the host cores.
"""
import argparse
import json
import os
import sys
import time


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=4)
    ap.add_argument("--seed", type=int, default=20261201)
    ap.add_argument("--slots", type=int, default=0, help="slots (0 = the workload's)")
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="c2")
    ap.add_argument("--bps", type=int, default=0, help="KV blocks per attention work item (0 = auto)")
    ap.add_argument("--ring-bps", type=int, default=0,
                    help="KV blocks per work item through the sliding-window rings (0 = auto)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-decode-phase", action="store_true",
                    help="skip the pure-decode timed phase (config.decode_only)")
    ap.add_argument("--quiet", action="store_true")
    ap.add_argument("--sync", action="store_true",
                    help="read each pass's tokens back before launching the next (no run-ahead)")
    ap.add_argument("--streams", type=int, default=0,
                    help="1, or 2: a pass as two halves at once on two streams (0 = the workload's)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="BYTES",
                    help="only run a plain device copy of BYTES, 8 times (the known-size kernel "
                         "that scales the FETCH_SIZE / WRITE_SIZE counters); prints nothing")
    ap.add_argument("--read-probe", type=int, default=0, metavar="BYTES",
                    help="only time a plain streaming read (f32 row sums of BYTES of f16 in "
                         "rows of 4096) and a device copy of BYTES, 10 times each after 2 "
                         "untimed: the practical HBM ceilings the kernels' GB/s compare with; "
                         "prints both")
    ap.add_argument("--act", choices=("ggml", "exact"), default="ggml",
                    help="arithmetic of the quantized weight products: ggml (the reference CPU "
                         "path's: X quantized to Q8_K / Q8_0 per block, integer block dots; "
                         "default) or exact (f32-accurate X as f16 hi + lo halves)")
    ap.add_argument("--graph-probe", action="store_true",
                    help="only time one decode pass of the workload's model at 64 contexts "
                         "U[128, 4000] three ways: eager, as a captured HIP graph replayed "
                         "(same plan), and the capture itself; prints the three")
    ap.add_argument("--product", default="", metavar="TYPE:MxK:N",
                    help="only run one weight product (q4 / q6 / q8, M x K weights, N rows), "
                         "5 times after 2 untimed calls: the subject of the products' counter "
                         "passes; prints its mean time")
    return ap.parse_args()


HBM_PEAK = 8.0e12      # MI355X HBM3E, bytes/s
MFMA_PEAK = 2.5e15     # MI355X dense f16 MFMA, flop/s (the products' arithmetic)
PREFILL_CHUNK = 512    # lua/lgml/engine.lua:57 UBATCH
WORKLOADS = {
    "c2": dict(shape="c2", prompt=(128, 4096),
               metric="decode tok/s, 64 ragged seqs, Llama-3-8B-shape Q4_K; paged-attn HBM GB/s %",
               text="C2: Llama-3-8B shape, Q4_K_M, f16 KV, 64 ragged slots, prompts U[128,4096], "
                    "continuous batching from the steady state (budgets U[64,2048], initial "
                    "requests part-way through theirs; joins prefilled in 512-token chunks)"),
    "c3": dict(shape="c2", prompt=(16, 512), prefix=2048, chunk_cap=True,
               metric="decode tok/s, 64 seqs on a shared 2048-token prefix, Llama-3-8B-shape "
                      "Q4_K; paged-attn HBM GB/s %",
               text="C3: Llama-3-8B shape, Q4_K_M, f16 KV, 64 slots sharing a 2048-token prefix "
                    "(32 refcounted blocks) + unique suffixes U[16,512], continuous batching "
                    "from the steady state (budgets U[64,2048]); a join attaches the prefix and "
                    "prefills its suffix in 512-token chunks mixed into the decode ubatch"),
    "c4": dict(shape="c4", prompt=(1024, 16384), slots=32, joins=False,
               metric="decode tok/s, 32 slots, Gemma-4-style SWA ring Q8_0; paged-attn HBM GB/s %",
               text="C4: Gemma-4-style, 26 layers (5 sliding-window 1024-token rings per slot : 1 "
                    "global), d 2560, 8/4 heads of 256, GeGLU 10240, vocab 262144 tied, Q8_0, f16 "
                    "KV, 32 slots, contexts U[1024,16384], decode only (no joins)"),
    "c5": dict(shape="c5", prompt=(256, 8192),
               metric="decode tok/s, 64 ragged seqs, 30B-A3B-shape MoE Q4_K; paged-attn HBM GB/s %",
               text="C5: 30B-A3B-shaped qwen3moe, 128 experts x 768, top-8 softmax routing, Q4_K, "
                    "f16 KV, 64 ragged slots, prompts U[256,8192], continuous batching from the "
                    "steady state (budgets U[64,2048]; joins prefilled in 512-token chunks), "
                    "tokens grouped by expert"),
}
HERE = os.path.dirname(os.path.abspath(__file__))
# HBM bytes per paged-attention launch of this workload, from rocprofv3
# FETCH_SIZE / WRITE_SIZE passes scaled by a copy kernel (see the file).
TRAFFIC_FILE = os.path.join(HERE, "profiles", "paged_attn_traffic.json")


def log(args, *a):
    if not args.quiet:
        print(*a, file=sys.stderr, flush=True)


def host_cpu():
    """(CPU model, logical CPUs this process may run on, online CPUs)."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = os.cpu_count() or 1
    return model, usable, os.cpu_count() or usable


def cpu_baseline(hp, contexts, seed, args):
    """The C oracle on one decode step of the workload's shape: 1 of the
    n_layer layers plus the output head (a sliding and a global layer, for
    a gemma shape), all sequences at the workload's contexts (synthetic KV),
    timed on the host cores; scaled to a full step."""
    import numpy as np

    from lgml_amd import workload
    from oracle import core, models

    E, V = hp["n_embd"], hp["n_vocab"]
    threads = core.threads()
    S = len(contexts)
    B = 64
    nbs = [(c + 1 + B - 1) // B for c in contexts]
    gemma = bool(hp.get("gemma"))
    R = workload.ring_blocks(hp, 1) if gemma else 0
    n_cells = max(sum(nbs), S * R) * B
    row = hp["n_head_kv"] * hp["head_dim"]
    rng = np.random.default_rng(seed)
    kp = [rng.integers(0x3000, 0x3c00, size=(n_cells, row), dtype=np.uint16)]
    vp = [rng.integers(0x3000, 0x3c00, size=(n_cells, row), dtype=np.uint16)]
    bt = np.full((S, max(nbs)), -1, np.int32)
    o = 0
    for i, nb in enumerate(nbs):
        bt[i, :nb] = np.arange(o, o + nb)
        o += nb
    rt = np.arange(S * R, dtype=np.int32).reshape(S, R) if gemma else None
    ids = rng.integers(0, V, size=S).astype(np.int32)
    b = core.BatchDesc([1] * S, contexts, bt, B, ids, list(range(S)), ring_tab=rt)
    shape = WORKLOADS[args.workload]["shape"]

    def one_layer(shp):
        """Mean seconds of a 1-layer pass (embeddings, layer, head), repeated
        until ~8 s of samples; the model's output matrix."""
        ohp, w = models.build(shp, seed=seed, n_layer=1, init="normal")
        om = core.OracleModel(dict(ohp, act_quant=bool(hp.get("act_quant"))), w)
        reps, t_all = 0, 0.0
        while reps < 2 or (t_all < 8.0 and reps < 20):
            t0 = time.time()
            om.forward(kp, vp, b)
            t_all += time.time() - t0
            reps += 1
        return t_all / reps, reps, t_all, w["output"]

    kinds = [("layer", shape, hp["n_layer"])]
    if gemma:
        n_glob = sum(1 - workload.gemma_layer(hp, il)["swa"] for il in range(hp["n_layer"]))
        kinds = [("sliding layer", shape, hp["n_layer"] - n_glob),
                 ("global layer", dict(models.SHAPES[shape], swa_period=1), n_glob)]
    passes = [one_layer(shp) for _, shp, _ in kinds]
    out = passes[0][3]
    x = rng.standard_normal((S, E)).astype(np.float32)
    t0 = time.time()
    (core.mul_mat_q8 if hp.get("act_quant") else core.mul_mat)(out[1], out[0], V, E, x)
    t_head = time.time() - t0
    t_step = t_head
    parts = []
    for (name, _, n), (t_pass, reps, t_all, _) in zip(kinds, passes):
        t_layer = max(t_pass - t_head, 1e-9)
        t_step += n * t_layer
        parts.append("%d x %s (%.2f s; %d passes, %.1f s)" % (n, name, t_layer, reps, t_all))
    model, usable, online = host_cpu()
    return {"value": S / t_step, "unit": "tok/s", "cores": threads, "kind": "port",
            "cpu_model": model, "nproc": usable, "cpus_online": online,
            "sample": "oracle/ (C, OpenMP, %d threads on %d usable of %d online CPUs, %s) "
                      "1-layer decode passes of the %s shape at %d sequences (contexts as the "
                      "GPU run, synthetic KV), output head %.1f s; step = head + %s"
                      % (threads, usable, online, model, args.workload.upper(), S, t_head,
                         " + ".join(parts))}


def traffic_of(path, args):
    """Measured HBM bytes per attention launch (profiles/paged_attn_traffic.json)
    and the algorithmic bytes of the steps they were counted on (a short run:
    other contexts than this run's traced steps), when measured on this
    workload; else (None, None)."""
    try:
        with open(path) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None, None
    if (t.get("seed") != args.seed or t.get("slots") != args.slots or
            t.get("bench_workload") != args.workload):
        return None, None
    return t.get("bytes_per_launch"), t.get("algorithmic_bytes_per_launch")


def product_flops(hp, n_tokens, n_out):
    """Flops of the weight products of one pass of n_tokens tokens with
    n_out logit rows: 2 x (weights each token multiplies) per token
    (routed experts: the n_used picks of each token and the router)."""
    E, H, Hkv, D, F, V, L = (hp[k] for k in ("n_embd", "n_head", "n_head_kv", "head_dim", "n_ff",
                                             "n_vocab", "n_layer"))
    from lgml_amd import workload
    per_tok = 0
    for il in range(L):
        has_wv = not hp.get("gemma") or workload.gemma_layer(hp, il)["has_wv"]
        per_tok += (H * D + Hkv * D * (2 if has_wv else 1)) * E + E * H * D
        if hp.get("n_expert"):
            per_tok += hp["n_expert"] * E + hp["n_used"] * 3 * hp["n_ff_exp"] * E
        else:
            per_tok += 3 * F * E
    return 2.0 * (per_tok * n_tokens + V * E * n_out)


def product_only(spec, act):
    """One weight product of seeded random weights (lgmlh_gen_normal, as the
    benched models) on N(0, 1) rows, run 2 + 5 times, in the arithmetic act."""
    import torch
    from lgml_amd import hip
    L = hip.lib()
    name, mk, n = spec.split(":")
    ty = {"q4": hip.Q4_K, "q6": hip.Q6_K, "q8": hip.Q8_0}[name]
    M, K = (int(v) for v in mk.split("x"))
    N = int(n)
    st = torch.cuda.current_stream().cuda_stream
    raw = torch.empty(L.lgmlh_row_size(ty, K) * M, dtype=torch.uint8, device="cuda")
    hip.check(L.lgmlh_gen_normal(20261201, ty, M, K, 0.0, 0.02, raw.data_ptr(), st))
    w = torch.empty(L.lgmlh_repacked_bytes(ty, M, K), dtype=torch.uint8, device="cuda")
    hip.check(L.lgmlh_repack(ty, M, K, raw.data_ptr(), w.data_ptr(), st))
    g = torch.Generator(device="cuda")
    g.manual_seed(1)
    x = torch.randn(N, K, device="cuda", generator=g)
    y = torch.empty(N, M, device="cuda")
    nb = L.lgmlh_mul_mat_workspace(ty, M, K, N)
    ws = torch.empty(max(nb, 1), dtype=torch.uint8, device="cuda")

    def call():
        fn = L.lgmlh_mul_mat_ggml if act == "ggml" else L.lgmlh_mul_mat
        hip.check(fn(ty, w.data_ptr(), M, K, x.data_ptr(), hip.F32, N, y.data_ptr(),
                     hip.EPI_NONE, None, ws.data_ptr(), nb, st))
    call()
    call()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(5):
        call()
    e1.record()
    torch.cuda.synchronize()
    print("product %s (%s): %.1f us" % (spec, act, e0.elapsed_time(e1) * 1e3 / 5))
    return 0


def read_probe(nbytes):
    """The practical HBM ceilings on this box: a streaming read (torch's f32
    row sums of f16 rows of 4096 values: 5.9-6.4 TB/s, where one sum over
    the whole buffer reaches only 3.6) and a device copy, each of nbytes,
    timed with events over 10 runs after 2 untimed ones."""
    import torch
    a = torch.empty(nbytes // 2, dtype=torch.float16, device="cuda").fill_(1.0)
    b = torch.empty_like(a)
    rows = a.view(-1, 4096)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for name, fn, moved in (("read", lambda: rows.sum(1, dtype=torch.float32), nbytes),
                            ("copy", lambda: b.copy_(a), 2 * nbytes)):
        fn()
        fn()
        torch.cuda.synchronize()
        e0.record()
        for _ in range(10):
            fn()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / 10
        print("%s of %d B: %.1f us, %.0f GB/s (bytes moved %d)" % (name, nbytes, us, moved / us / 1e3,
                                                                  moved))
    return 0


def graph_probe(args):
    """What a captured graph of the decode pass would save: the pass run
    eagerly (lgmlh_forward launches kernel after kernel), a capture of the
    same call replayed (every replay checked equal to the eager logits, with
    eager passes between replays), and the wall time of capturing and
    instantiating it. A plan changes every step (lengths, work items, grid
    sizes), so a graph would be captured again per pass."""
    import numpy as np
    import torch

    from lgml_amd import runtime, workload
    wl = WORKLOADS[args.workload]
    hp = dict(workload.SHAPES[wl["shape"]])
    if hp.get("gemma"):
        print("--graph-probe runs the paged-only workloads (c2, c3, c5)", file=sys.stderr)
        return 2
    hp["act_quant"] = args.act == "ggml"
    S, nbk = 64, (4000 + 64 + 63) // 64
    model = runtime.DeviceModel(hp, runtime.generated_weights(
        hp, args.seed, workload.policy(hp["wtype"], hp["n_layer"])), S * nbk * 64)
    g = torch.Generator(device="cuda")
    g.manual_seed(args.seed)
    for t in model.kpools + model.vpools:
        t.view(torch.float16).uniform_(-1.0, 1.0, generator=g)
    rng = workload.Lcg(args.seed)
    npast = [rng.int(128, 4000) for _ in range(S)]
    ids = np.array([rng.int(0, hp["n_vocab"] - 1) for _ in range(S)], np.int32)
    bt = (np.arange(S, dtype=np.int32)[:, None] * nbk + np.arange(nbk, dtype=np.int32)[None, :])
    plan = model.plan([1] * S, npast, bt, ids)
    out = torch.empty((S, hp["n_vocab"]), dtype=torch.float32, device="cuda")
    for _ in range(3):
        model.forward(plan, logits=out)
    torch.cuda.synchronize()
    ref = out.clone()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def timed(fn, n=20):
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n

    eager = timed(lambda: model.forward(plan, logits=out))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    caps = []
    for _ in range(3):
        graph = torch.cuda.CUDAGraph()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        with torch.cuda.graph(graph, stream=side):
            model.forward(plan, logits=out)
        torch.cuda.synchronize()
        caps.append((time.perf_counter() - t0) * 1e3)
    for i in range(4):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        if not torch.equal(out, ref):
            print("replay %d differs from the eager pass" % i, file=sys.stderr)
            return 1
        model.forward(plan, logits=out)
    replay = timed(graph.replay)
    if not torch.equal(out, ref):
        print("the timed replays differ from the eager pass", file=sys.stderr)
        return 1
    print("%s decode pass, 64 sequences: eager %.3f ms, graph replay %.3f ms (%.3f ms less), "
          "capture + instantiate %s ms" % (args.workload, eager, replay, eager - replay,
                                            " / ".join("%.2f" % c for c in caps)))
    return 0


def main():
    args = parse()
    if args.graph_probe:
        return graph_probe(args)
    if args.read_probe:
        return read_probe(args.read_probe)
    if args.calibrate_copy:
        import torch
        n = args.calibrate_copy // 4
        a = torch.empty(n, dtype=torch.float32, device="cuda").fill_(1.0)
        b = torch.empty_like(a)
        torch.cuda.synchronize()
        for _ in range(8):
            b.copy_(a)
        torch.cuda.synchronize()
        return 0
    if args.product:
        return product_only(args.product, args.act)
    if args.gpus != 1:
        print("bench.py measures one GPU: every GPU box here has one, and the multi-GPU "
              "sharding of this path is design only; run with --gpus 1",
              file=sys.stderr)
        return 2
    import numpy as np
    import torch

    from lgml_amd import engine, hip, runtime, workload

    wl = WORKLOADS[args.workload]
    hp = dict(workload.SHAPES[wl["shape"]])
    hp["act_quant"] = args.act == "ggml"
    ty = workload.policy(hp["wtype"], hp["n_layer"])
    rng = workload.Lcg(args.seed)
    S = args.slots = args.slots or wl.get("slots", 64)
    plo, phi = wl["prompt"]
    prefix_n = wl.get("prefix", 0)
    n_trace = min(args.steps, 16)
    joins_on = wl.get("joins", True)
    # without joins every budget outlasts the warmup, timed and traced steps
    n_run = args.warmup + 2 * args.steps + n_trace + 8
    budget = (64, 2048) if joins_on else (n_run,) * 2
    max_ctx = prefix_n + phi + budget[1] + 64
    # the shared prefix is stored once; a probe prefill chunk and margin
    n_cells = ((S * (max_ctx - prefix_n) + prefix_n + 4 * PREFILL_CHUNK + 63) // 64) * 64
    # sliding layers: a ring per slot, sized for 512-token passes
    ring_cells = S * workload.ring_blocks(hp, engine.UBATCH) * 64 if hp.get("gemma") else 0
    log(args, "building the model on the device ...")
    t0 = time.time()
    model = runtime.DeviceModel(hp, runtime.generated_weights(hp, args.seed, ty), n_cells,
                                ring_cells=ring_cells)
    model.ring_blocks_per_split = args.ring_bps
    torch.cuda.synchronize()
    log(args, "model ready in %.1f s; pool %d cells (%.1f GB KV)" % (
        time.time() - t0, n_cells, n_cells * 2 * 2 * hp["n_head_kv"] * hp["head_dim"] *
        hp["n_layer"] / 1e9))
    # Synthetic KV for the initial contexts: small f16 values in every cell.
    g = torch.Generator(device="cuda")
    g.manual_seed(args.seed)
    for t in model.kpools + model.vpools:
        t.view(torch.float16).uniform_(-1.0, 1.0, generator=g)

    trace = runtime.EventTrace(n_trace * hp["n_layer"] * 8 + 64,
                               hip.TRACE_ATTN | hip.TRACE_GEMM | hip.TRACE_EXPERTS)
    n_streams = 1 if args.sync else (args.streams or wl.get("streams", 1))
    # C3: a pass carries the decode tokens and at most one 512-token chunk
    max_tokens = S + PREFILL_CHUNK if wl.get("chunk_cap") else None
    eng = engine.Engine(model, S, blocks_per_split=args.bps, run_ahead=not args.sync,
                        streams=n_streams, prefix_cache=prefix_n > 0, max_tokens=max_tokens)
    prefix = [rng.int(0, hp["n_vocab"] - 1) for _ in range(prefix_n)]
    if prefix_n:
        # the system prefix, prefilled once for real and published
        r0 = engine.Request(prefix + [rng.int(0, hp["n_vocab"] - 1)], 1)
        eng.submit(r0)
        while not r0.done:
            eng.step()
        eng.drain()
        log(args, "prefix of %d tokens prefilled and published (%d keys)" % (
            prefix_n, len(eng.infos)))

    def new_request(prefilled):
        """A request of the workload. prefilled: its prompt's KV is already
        in its cells (synthetic), and it is part-way through its budget
        (the steady state); else it joins and its prompt is prefilled for
        real (after the shared prefix's blocks, with prefix caching)."""
        n = rng.int(plo, phi)
        prompt = prefix + [rng.int(0, hp["n_vocab"] - 1) for _ in range(n)]
        b = rng.int(*budget)
        r = engine.Request(prompt, rng.int(1, b) if prefilled and joins_on else b)
        eng.submit(r)
        if prefilled:
            eng.seqs.reserve(r.seq, len(prompt))
            r.seq.n_past = len(prompt)
            r.fed = len(prompt)
            r.out = [prompt[-1]]
            r.max_new += 1
        return r

    for _ in range(S):
        new_request(True)
    contexts0 = [r.seq.n_past for r in eng.active]
    joins = [0]
    mode = ["mixed"]

    def top_up():
        """Refill finished slots: joining requests (the mixed phase), or
        already-prefilled ones (the pure-decode phase)."""
        while joins_on and len(eng.active) < S:
            new_request(mode[0] == "decode")
            joins[0] += 1

    def step(record):
        """One engine step; (requests that got a token, whether a pass was
        read back: a run-ahead engine's first step after a drain reads none)."""
        eng.trace = trace if record else None
        done = eng.passes
        got = eng.step()
        top_up()
        return got, eng.passes > done

    def drain():
        got = eng.drain()
        top_up()
        return got

    wbytes = workload.weight_bytes(hp, S)
    xbytes = workload.expert_bytes(hp, S)
    cellb = 2 * hp["n_head_kv"] * hp["head_dim"] * 2  # K+V bytes per cell and layer
    swa = list(model.swa)

    def bytes_of(plan):
        """(attention bytes of each layer, step bytes, unique attention bytes
        of a layer) of a pass: K + V of every cell a query group sees (a
        sliding layer: at most the window - 1 + the pass's tokens), q in and
        out; the step adds the weights and the new cells' K + V. Unique:
        each pool cell once, however many sequences share its block."""
        seq_n = plan.seq_n.astype(np.int64)
        n_kv = plan.seq_npast.astype(np.int64) + seq_n
        N = int(seq_n.sum())
        qo = N * hp["n_head"] * hp["head_dim"] * 4 * 2
        full = int(n_kv.sum()) * cellb
        win = int(np.minimum(n_kv, hp.get("n_swa", 0) - 1 + seq_n).sum()) * cellb
        per_layer = [(win if sl else full) + qo for sl in swa]
        used = {}
        for s, nk in enumerate(n_kv):
            for i in range(int((nk + 63) // 64)):
                b = int(plan.block_tab[s, i])
                used[b] = max(used.get(b, 0), int(min(64, nk - 64 * i)))
        uniq = sum(used.values()) * cellb + qo
        return per_layer, wbytes + sum(per_layer) + N * cellb * len(swa), uniq

    def timed(n_steps):
        """n_steps timed steps; every pass launched in them is read back in
        them (the run-ahead engine's last one by the drain). Returns (wall,
        decoded, prefill tokens, joins, per-pass step bytes)."""
        decoded = prefill_tok = 0
        step_bytes = []
        joins[0] = 0
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(n_steps + 1):
            if i < n_steps:
                got, read = step(False)
            else:
                n0 = eng.passes
                got = drain()
                read = eng.passes > n0
            if not read:
                continue
            decoded += len(got)
            for pl in eng.last_plans:  # a pass split over two streams has two plans
                seq_n = pl.seq_n
                prefill_tok += int(seq_n[seq_n > 1].sum())
            step_bytes.append(sum(bytes_of(pl)[1] for pl in eng.last_plans)
                              - wbytes * (len(eng.last_plans) - 1))
        torch.cuda.synchronize()
        return time.perf_counter() - t0, decoded, prefill_tok, joins[0], step_bytes

    for _ in range(args.warmup):
        step(False)
    drain()
    # the mixed phase: continuous batching with joins (value)
    wall, decoded, prefill_tok, n_joins, step_bytes = timed(args.steps)
    log(args, "mixed phase: %d steps, %.1f tok/s, %d joins, %d prefill tokens" % (
        args.steps, decoded / wall, n_joins, prefill_tok))
    # the pure-decode phase: finished slots are refilled with prefilled
    # requests; untimed steps first finish the prompts still in flight
    mode[0] = "decode"
    dec = None
    if not args.no_decode_phase and joins_on:
        for _ in range(64):
            if all(r.fed >= len(r.feed) for r in eng.active):
                break
            step(False)
        drain()
        dwall, ddec, dpre, _, dbytes = timed(args.steps)
        dec = {"value": ddec / dwall, "ms_per_step": dwall * 1e3 / args.steps,
               "decoded_tokens": ddec, "prefill_tokens": dpre,
               "step_GBps": sum(dbytes) / dwall / 1e9,
               "step_roofline_frac": sum(dbytes) / dwall / HBM_PEAK}
        log(args, "decode phase: %.1f tok/s" % dec["value"])
    # the traced steps run as one pass on one stream: the events time the
    # attention kernels themselves, with nothing else running beside them
    attn_bytes, uniq_bytes, decode_pass = [], [], []
    eng.n_streams = 1
    for _ in range(n_trace):
        step(True)
        pl = eng.launched_plan
        pb = bytes_of(pl)
        attn_bytes.append(pb[0])
        uniq_bytes.append(pb[2])
        decode_pass.append(bool((pl.seq_n <= 1).all()))
    drain()

    def per_pass(ts):
        """The recorded spans of one kind, split by pass (the same number
        of launches of a kind in every pass)."""
        k = len(ts) // n_trace
        return [ts[i * k:(i + 1) * k] for i in range(n_trace)]
    # The kernel figures come from the decode passes among the traced ones.
    keep = [i for i in range(n_trace) if decode_pass[i]]
    if len(keep) < n_trace // 2:
        keep = list(range(n_trace))
    at_p = per_pass(trace.times_ms(hip.TRACE_ATTN))
    gt_p = per_pass(trace.times_ms(hip.TRACE_GEMM))
    xt_p = per_pass(trace.times_ms(hip.TRACE_EXPERTS))
    at = [t for i in keep for t in at_p[i]]
    n_att = len(at)
    tot_bytes = sum(sum(attn_bytes[i][:len(at_p[i])]) for i in keep)
    tot_uniq = sum(uniq_bytes[i] * len(at_p[i]) for i in keep)
    attn_gbs = tot_bytes / (sum(at) / 1e3) if at else 0.0
    avg_attn_ms = sum(at) / max(n_att, 1)
    attn_bytes_per_launch = tot_bytes / max(n_att, 1)  # algorithmic, these steps
    traffic = traffic_of(TRAFFIC_FILE, args)
    gemm_ms = sum(sum(gt_p[i]) + sum(xt_p[i]) for i in keep) / len(keep)
    exp_ms = sum(sum(xt_p[i]) for i in keep) / len(keep)

    # One 512-token prompt chunk alone (a joining request's prefill pass):
    # the weight products against the MFMA peak.
    pre = None
    try:
        c = engine.Seq(eng.seqs)
        eng.seqs.reserve(c, PREFILL_CHUNK)
        bt = np.array([c.blocks], np.int32)
        ids = np.array([rng.int(0, hp["n_vocab"] - 1) for _ in range(PREFILL_CHUNK)], np.int32)
        rt = None
        if eng.ring_blocks:
            rt = np.arange(eng.ring_blocks, dtype=np.int32)[None]  # slot 0's ring
        plan = model.plan([PREFILL_CHUNK], [0], bt, ids, args.bps, ring_tab=rt)
        for rep in range(3):
            trace.reset()
            model.forward(plan, trace=trace if rep == 2 else None)
        g_ms = sum(trace.times_ms(hip.TRACE_GEMM)) + sum(trace.times_ms(hip.TRACE_EXPERTS))
        fl = product_flops(hp, PREFILL_CHUNK, 1)
        pre = {"bound": "mfma", "kernel": "qgemm_kernel (all weight products of the pass)",
               "achieved": fl / (g_ms / 1e3) / 1e12, "peak": MFMA_PEAK / 1e12,
               "unit": "TFLOP/s", "frac": fl / (g_ms / 1e3) / MFMA_PEAK,
               "tokens": PREFILL_CHUNK, "gemm_ms": g_ms, "flops": fl}
        eng.seqs.free(c)
        # the probe wrote slot 0's ring: no engine pass runs after it
    except Exception as e:  # report, do not hide the decode numbers
        pre = {"error": repr(e)}

    ms_step = wall * 1e3 / args.steps
    step_gbs = sum(step_bytes) / wall
    result = {
        "metric": wl["metric"],
        "value": decoded / wall,
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "%s weights, %s, f16 KV, f32 accumulate" % (
            hp["wtype"].replace("q8_0", "Q8_0"),
            "X quantized per block as ggml's CPU path (Q8_%s), integer block dots" % (
                "0" if hp["wtype"] == "q8_0" else "K") if args.act == "ggml"
            else "f32-accurate X (f16 hi + lo)"),
        "data": "synthetic (seeded random-init weights, LCG prompts, synthetic initial KV)",
        "config": {
            "workload": wl["text"],
            "slots": S, "seed": args.seed, "decoded_tokens": decoded,
            "prefill_tokens": prefill_tok, "joins": n_joins,
            "mean_context": float(np.mean(contexts0)),
            "act": args.act,
            "engine": "sync" if args.sync else "run-ahead, %d stream%s" % (
                n_streams, "s" if n_streams > 1 else ""),
            "decode_only": dec,
        },
        "roofline": {
            "bound": "hbm", "kernel": "paged_attn_kernel + merge_kernel (per layer)",
            "achieved": attn_gbs / 1e9, "peak": HBM_PEAK / 1e9, "unit": "GB/s",
            "frac": attn_gbs / HBM_PEAK, "traffic": traffic[0],
            "traffic_algorithmic_bytes": traffic[1],
            "bytes_per_launch": attn_bytes_per_launch,
            "avg_launch_ms": avg_attn_ms, "launches": n_att,
        },
        "step_roofline": {
            "bytes_per_step": sum(step_bytes) / len(step_bytes),
            "achieved_GBps": step_gbs / 1e9, "frac": step_gbs / HBM_PEAK,
            "gemm_ms_per_step": gemm_ms, "attn_ms_per_step": sum(at) / len(keep),
            "traced_steps": len(keep),
            "gemm_GBps": wbytes / (gemm_ms / 1e3) / 1e9 if gemm_ms else None,
        },
        "prefill_roofline": pre,
    }
    if prefix_n:
        # logical (each sequence's context; the roofline's figure) against
        # unique (the shared prefix read from HBM once) attention bytes
        result["roofline"]["unique_bytes_per_launch"] = tot_uniq / max(n_att, 1)
        result["roofline"]["logical_bytes_per_launch"] = tot_bytes / max(n_att, 1)
        result["roofline"]["unique_GBps"] = tot_uniq / (sum(at) / 1e3) / 1e9 if at else None
        result["config"]["prefix_tokens"] = prefix_n
        result["config"]["prefix_hits"] = eng.hits
    if xbytes:
        # grouped expert products: expected distinct experts' bytes per step
        result["step_roofline"].update({
            "expert_bytes_per_step": xbytes, "expert_ms_per_step": exp_ms,
            "expert_GBps": xbytes / (exp_ms / 1e3) / 1e9 if exp_ms else None})
    if not args.no_cpu_baseline:
        log(args, "timing the CPU oracle sample ...")
        try:
            result["cpu_baseline"] = cpu_baseline(hp, contexts0, args.seed, args)
        except Exception as e:  # report, do not hide the GPU number
            result["cpu_baseline"] = {"error": repr(e)}
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
