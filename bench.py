#!/usr/bin/env python3
"""Decode throughput of lgml's ragged continuous-batching path on one MI355X.

Default workload ("C2"): a Llama-3-8B-shaped model
(32 layers, d 4096, 32 / 8 heads, head 128, FFN 14336, vocab 128256) with
N(0, 0.02) weights quantized Q4_K_M (output and attn_v / ffn_down of the
more_bits layers Q6_K), f16 KV in 64-cell blocks; 64 slots with prompt
lengths U[128, 4096]; continuous batching: every request has a decode budget
U[64, 2048]; a finished request's slot is taken by a new one whose prompt
(U[128, 4096]) is prefilled in 512-token chunks mixed into the decode passes.
The initial 64 contexts are filled with synthetic KV (the attention reads
cost the same whatever the values); joining prompts run the real prefill.
One step = one pass of the engine (E:flush): the next token of every
decoding slot plus the prompt chunks of joining slots.

--workload c5: the same loop on a 30B-A3B-shaped
qwen3moe (48 layers, d 2048, 32 / 4 heads, head 128, 128 experts of width
768, top-8 softmax routing, router logits N(0, 1), Q4_K), prompts
U[256, 8192]: tokens are grouped by expert for the grouped Q4_K expert
products.

--workload c4: a Gemma-4-style model (26 layers,
d 2560, 8 / 4 heads of 256, 5 sliding-window layers with a 1024-token ring
per slot to 1 global layer, GeGLU FFN 10240, vocab 262144 tied, Q8_0), 32
slots with contexts U[1024, 16384] decoding 128 steps (no joins: every
budget outlasts the run).

value = decoded tokens / wall seconds of the K timed steps (inputs resident
in HBM; the per-step host plan upload and the 64 sampled ids read back are
inside; no instrumentation). The engine runs ahead by one pass (the next
pass is planned and queued before the previous one's tokens are read back;
decode tokens go from pass to pass on the device); --sync reads every pass
back before the next. roofline = the paged attention kernel (the
dominant kernel: ~80% of the step's bytes): its algorithmic bytes (K + V of
every visible cell, q in, out) per launch over its duration, timed with HIP
events on the pass's stream during min(K, 16) further steps (the decode
passes among them), against 8 TB/s. cpu_baseline = the C oracle (oracle/)
timed on a bounded sample of the same step on the host cores.
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
    ap.add_argument("--quiet", action="store_true")
    ap.add_argument("--sync", action="store_true",
                    help="read each pass's tokens back before launching the next (no run-ahead)")
    ap.add_argument("--streams", type=int, default=0,
                    help="1, or 2: a pass as two halves at once on two streams (0 = the workload's)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="BYTES",
                    help="only run a plain device copy of BYTES, 8 times (the known-size kernel "
                         "that scales the FETCH_SIZE / WRITE_SIZE counters); prints nothing")
    return ap.parse_args()


HBM_PEAK = 8.0e12  # MI355X HBM3E, bytes/s
WORKLOADS = {
    "c2": dict(prompt=(128, 4096),
               metric="decode tok/s, 64 ragged seqs, Llama-3-8B-shape Q4_K; paged-attn HBM GB/s %",
               text="C2: Llama-3-8B shape, Q4_K_M, f16 KV, 64 ragged slots, prompts U[128,4096], "
                    "continuous batching (budgets U[64,2048], joins prefilled in 512-token chunks)"),
    "c4": dict(prompt=(1024, 16384), slots=32, joins=False,
               metric="decode tok/s, 32 slots, Gemma-4-style SWA ring Q8_0; paged-attn HBM GB/s %",
               text="C4: Gemma-4-style, 26 layers (5 sliding-window 1024-token rings per slot : 1 "
                    "global), d 2560, 8/4 heads of 256, GeGLU 10240, vocab 262144 tied, Q8_0, f16 "
                    "KV, 32 slots, contexts U[1024,16384], decode only (no joins)"),
    "c5": dict(prompt=(256, 8192),
               metric="decode tok/s, 64 ragged seqs, 30B-A3B-shape MoE Q4_K; paged-attn HBM GB/s %",
               text="C5: 30B-A3B-shaped qwen3moe, 128 experts x 768, top-8 softmax routing, Q4_K, "
                    "f16 KV, 64 ragged slots, prompts U[256,8192], continuous batching (budgets "
                    "U[64,2048], joins prefilled in 512-token chunks), tokens grouped by expert"),
}
HERE = os.path.dirname(os.path.abspath(__file__))
# HBM bytes per paged-attention launch of this workload, from rocprofv3
# FETCH_SIZE / WRITE_SIZE passes scaled by a copy kernel (see the file).
TRAFFIC_FILE = os.path.join(HERE, "profiles", "paged_attn_traffic.json")


def log(args, *a):
    if not args.quiet:
        print(*a, file=sys.stderr, flush=True)


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

    def one_layer(shape):
        """Mean seconds of a 1-layer pass (embeddings, layer, head), repeated
        until ~8 s of samples; the model's output matrix."""
        ohp, w = models.build(shape, seed=seed, n_layer=1, init="normal")
        om = core.OracleModel(ohp, w)
        reps, t_all = 0, 0.0
        while reps < 2 or (t_all < 8.0 and reps < 20):
            t0 = time.time()
            om.forward(kp, vp, b)
            t_all += time.time() - t0
            reps += 1
        return t_all / reps, reps, t_all, w["output"]

    kinds = [("layer", args.workload, hp["n_layer"])]
    if gemma:
        n_glob = sum(1 - workload.gemma_layer(hp, il)["swa"] for il in range(hp["n_layer"]))
        kinds = [("sliding layer", args.workload, hp["n_layer"] - n_glob),
                 ("global layer", dict(models.SHAPES[args.workload], swa_period=1), n_glob)]
    passes = [one_layer(shape) for _, shape, _ in kinds]
    out = passes[0][3]
    x = rng.standard_normal((S, E)).astype(np.float32)
    t0 = time.time()
    core.mul_mat(out[1], out[0], V, E, x)
    t_head = time.time() - t0
    t_step = t_head
    parts = []
    for (name, _, n), (t_pass, reps, t_all, _) in zip(kinds, passes):
        t_layer = max(t_pass - t_head, 1e-9)
        t_step += n * t_layer
        parts.append("%d x %s (%.2f s; %d passes, %.1f s)" % (n, name, t_layer, reps, t_all))
    return {"value": S / t_step, "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": "oracle/ (C, OpenMP) 1-layer decode passes of the %s shape at %d sequences "
                      "(contexts as the GPU run, synthetic KV), output head %.1f s; step = head + "
                      "%s" % (args.workload.upper(), S, t_head, " + ".join(parts))}


def traffic_of(path, args):
    """Measured HBM bytes per attention launch (profiles/paged_attn_traffic.json),
    when measured on this workload; else None."""
    try:
        with open(path) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    if (t.get("seed") != args.seed or t.get("slots") != args.slots or
            t.get("bench_workload") != args.workload):
        return None
    return t.get("bytes_per_launch")


def main():
    args = parse()
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
    if args.gpus != 1:
        print("bench.py measures one GPU: every GPU box here has one, and the multi-GPU "
              "sharding of this path is design only (see DESIGN.md); run with --gpus 1",
              file=sys.stderr)
        return 2
    import numpy as np
    import torch

    from lgml_amd import engine, hip, runtime, workload

    wl = WORKLOADS[args.workload]
    hp = dict(workload.SHAPES[args.workload])
    ty = workload.policy(hp["wtype"], hp["n_layer"])
    rng = workload.Lcg(args.seed)
    S = args.slots = args.slots or wl.get("slots", 64)
    plo, phi = wl["prompt"]
    n_trace = min(args.steps, 16)
    joins_on = wl.get("joins", True)
    # without joins every budget outlasts the warmup, timed and traced steps
    budget = (64, 2048) if joins_on else (args.warmup + args.steps + n_trace + 2,) * 2
    max_ctx = phi + budget[1] + 64
    n_cells = ((S * max_ctx + 63) // 64) * 64
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
    eng = engine.Engine(model, S, blocks_per_split=args.bps, run_ahead=not args.sync,
                        streams=n_streams)

    def new_request(prefilled):
        n = rng.int(plo, phi)
        prompt = [rng.int(0, hp["n_vocab"] - 1) for _ in range(n)]
        r = engine.Request(prompt, rng.int(*budget))
        eng.submit(r)
        if prefilled:
            eng.seqs.reserve(r.seq, n)
            r.seq.n_past = n
            r.fed = n
            r.out = [prompt[-1]]
            r.max_new += 1
        return r

    for _ in range(S):
        new_request(True)
    contexts0 = [r.seq.n_past for r in eng.active]
    joins = [0]

    def top_up():
        while joins_on and len(eng.active) < S:
            new_request(False)
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

    for _ in range(args.warmup):
        step(False)
    drain()
    torch.cuda.synchronize()
    trace.reset()
    decoded = prefill_tok = 0
    wbytes = workload.weight_bytes(hp, S)
    xbytes = workload.expert_bytes(hp, S)
    cellb = 2 * hp["n_head_kv"] * hp["head_dim"] * 2  # K+V bytes per cell and layer
    swa = list(model.swa)

    def bytes_of(plan):
        """(attention bytes of each layer, step bytes) of a pass: K + V of
        every cell a query group sees (a sliding layer: at most the window
        - 1 + the pass's tokens), q in and out; the step adds the weights and
        the new cells' K + V."""
        seq_n = plan.seq_n.astype(np.int64)
        n_kv = plan.seq_npast.astype(np.int64) + seq_n
        N = int(seq_n.sum())
        qo = N * hp["n_head"] * hp["head_dim"] * 4 * 2
        full = int(n_kv.sum()) * cellb
        win = int(np.minimum(n_kv, hp.get("n_swa", 0) - 1 + seq_n).sum()) * cellb
        per_layer = [(win if sl else full) + qo for sl in swa]
        return per_layer, wbytes + sum(per_layer) + N * cellb * len(swa)

    # The timed steps run without instrumentation (value, ms_per_step); the
    # kernel times come from n_trace more steps with HIP events around
    # each attention launch group and weight product.
    step_bytes = []
    joins[0] = 0
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    # every pass launched in the timed region is read back in it (the
    # run-ahead engine's last one by the drain)
    for i in range(args.steps + 1):
        if i < args.steps:
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
    wall = time.perf_counter() - t0
    # the traced steps run as one pass on one stream: the events time the
    # attention kernels themselves, with nothing else running beside them
    attn_bytes, decode_pass = [], []
    eng.n_streams = 1
    for _ in range(n_trace):
        step(True)
        pl = eng.launched_plan
        attn_bytes.append(bytes_of(pl)[0])
        decode_pass.append(bool((pl.seq_n <= 1).all()))
    drain()

    def per_pass(ts):
        """The recorded spans of one kind, split by pass (the same number
        of launches of a kind in every pass)."""
        k = len(ts) // n_trace
        return [ts[i * k:(i + 1) * k] for i in range(n_trace)]
    # The kernel figures come from the decode passes among the traced ones:
    # a joining prompt's 512-token chunk is a prefill pass, another regime
    # (its attention reads each block once per group of 16 / G tokens).
    keep = [i for i in range(n_trace) if decode_pass[i]]
    if len(keep) < n_trace // 2:
        keep = list(range(n_trace))
    at_p = per_pass(trace.times_ms(hip.TRACE_ATTN))
    gt_p = per_pass(trace.times_ms(hip.TRACE_GEMM))
    xt_p = per_pass(trace.times_ms(hip.TRACE_EXPERTS))
    at = [t for i in keep for t in at_p[i]]
    n_att = len(at)
    tot_bytes = sum(sum(attn_bytes[i][:len(at_p[i])]) for i in keep)
    attn_gbs = tot_bytes / (sum(at) / 1e3) if at else 0.0
    avg_attn_ms = sum(at) / max(n_att, 1)
    gemm_ms = sum(sum(gt_p[i]) + sum(xt_p[i]) for i in keep) / len(keep)
    exp_ms = sum(sum(xt_p[i]) for i in keep) / len(keep)
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
        "dtype": "%s weights, f16 KV, f32 accumulate" % hp["wtype"].replace("q8_0", "Q8_0"),
        "data": "synthetic (seeded random-init weights, LCG prompts, synthetic initial KV)",
        "config": {
            "workload": wl["text"],
            "slots": S, "seed": args.seed, "decoded_tokens": decoded,
            "prefill_tokens": prefill_tok, "joins": joins[0],
            "mean_context": float(np.mean(contexts0)),
            "engine": "sync" if args.sync else "run-ahead, %d stream%s" % (
                n_streams, "s" if n_streams > 1 else ""),
        },
        "roofline": {
            "bound": "hbm", "kernel": "paged_attn_kernel + merge_kernel (per layer)",
            "achieved": attn_gbs / 1e9, "peak": HBM_PEAK / 1e9, "unit": "GB/s",
            "frac": attn_gbs / HBM_PEAK, "traffic": traffic_of(TRAFFIC_FILE, args),
            "avg_launch_ms": avg_attn_ms, "launches": n_att,
        },
        "step_roofline": {
            "bytes_per_step": sum(step_bytes) / len(step_bytes),
            "achieved_GBps": step_gbs / 1e9, "frac": step_gbs / HBM_PEAK,
            "gemm_ms_per_step": gemm_ms, "attn_ms_per_step": sum(at) / len(keep),
            "traced_steps": len(keep),
            "gemm_GBps": wbytes / (gemm_ms / 1e3) / 1e9 if gemm_ms else None,
        },
    }
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
