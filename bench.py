"""Benchmark of the Granite 4.2 8B non-GEMM layer ops on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick]

Headline (`value`): achieved HBM GB/s of one prefill step at T = 512 tokens
embedding gather + fused residual-add/RMSNorm with FP8
output + SwiGLU with FP8 output + RoPE with the int8 paged-KV write, i.e.
ideal (algorithmic) bytes of the step / measured time of the step. Inputs are
resident in HBM; 8 distinct input sets rotate so the 256 MB Infinity Cache
does not serve repeated iterations.

Also reported (extra keys): each op's µs, GB/s and fraction of the 8 TB/s
peak at T = 1, 8, 512 and 8192; the µs of a 40-layer batch-1 decode step
(161 launches replayed as one HIP graph); the bandwidth-stress sequence
(config 5); and the CPU baseline (the oracle, one core, on a bounded sample).

Timing: HIP events recorded on the stream the kernels are launched on (torch's
current stream, handed to the library with granite4_set_stream), bracketing
K back-to-back steps after W warmup steps, with torch.cuda.synchronize() on
both sides.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "tests"))

H, I, HQ, HK, D = 4096, 12800, 32, 8, 128
VOCAB = 100352
PEAK_GBS = 8000.0  # MI355X HBM3E
ROTATE_BYTES = 320e6  # distinct bytes per timed replay: more than the 256 MB Infinity Cache

# Algorithmic bytes per token (BASELINE.md section 3 / the survey's 8(d)).
B_EMBED = 4 * H + 4
B_NORM_FP8 = 7 * H
B_NORM_BF16 = 8 * H
B_SWIGLU_FP8 = 5 * I
B_SWIGLU_BF16 = 6 * I
B_ROPE_COMMON = (HQ + 2 * HK) * D * 2 + 2 * 64 * 4 + HQ * D * 2 + 4  # qkv R, cos/sin R, q_rot W, pt
B_ROPE = {16: B_ROPE_COMMON + 2 * HK * D * 2,
          8: B_ROPE_COMMON + 2 * HK * D + 2 * HK * 4,
          "k5v4g32": B_ROPE_COMMON + HK * (80 + 64) + 2 * HK * 4 * 4}


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "layerops_prefill_T512_hbm_traffic.md")


def profiled_traffic(kernel, path=TRAFFIC_PROFILE):
    """HBM bytes per dispatch of `kernel` from the committed rocprofv3 summary
    (two --pmc runs of `bench.py --only t512`: FETCH_SIZE, then WRITE_SIZE, KiB
    per dispatch). The table's scaled columns (MiB fetched x2.0 and written
    x1.0, the factors the known-size copy probe gives these counters) are
    summed. None if the summary has no row for the kernel."""
    try:
        for line in open(path):
            cells = [c.strip() for c in line.strip().strip("|").split("|")]
            if len(cells) >= 6 and cells[0].strip("`").startswith(kernel):
                return int((float(cells[4]) + float(cells[5])) * (1 << 20))
    except (OSError, ValueError):
        pass
    return None


def per_launch_extra(op):
    return {"norm_fp8": 2 * H + 4, "norm_bf16": 2 * H, "swiglu_fp8": 4}.get(op, 0)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--quick", action="store_true", help="headline + decode only")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", choices=["t512", "t8192", "decode", "t8", "stress", "tN", "probe", "floor", "t1",
                                       "attn", "gemm", "decode_gemv", "decode_trace",
                                       "layer_steps", "multi_step", "fp8_trace"],
                    help="run one configuration and print its detail (profiling runs)")
    ap.add_argument("--T", type=int, default=1024, help="token count for --only tN")
    ap.add_argument("--attn-case", default=None, help="run only this bench_attn case")
    ap.add_argument("--gemm-case", default=None,
                    help="run only this bench_gemm case, as T512:name or T8192:name")
    ap.add_argument("--trace-summary", default=None, metavar="KERNEL_TRACE_CSV",
                    help="summarise a rocprofv3 kernel trace of --only decode_trace (no GPU)")
    args = ap.parse_args()
    if args.trace_summary:
        print(json.dumps(summarize_decode_trace(args.trace_summary)), flush=True)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (the non-GEMM layer ops are "
              "token-parallel; see DESIGN.md for how they would shard). Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    import torch
    from pkg import layerops
    L = layerops()
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.init()
    stream = torch.cuda.current_stream()
    L.use_stream(stream)
    dev = "cuda"
    gen = torch.Generator(device=dev)
    gen.manual_seed(0x6A4)

    def randn(shape, std=1.0, mean=0.0):
        t = torch.empty(shape, dtype=torch.float32, device=dev).normal_(mean, std, generator=gen)
        return t.to(torch.bfloat16)

    def timed(fn, steps, warmup, sets, replays=3):
        """ms per fn() call: `steps` calls over rotating input sets captured in
        one HIP graph, replayed `replays` times between two events on the
        launch stream (no host launch cost inside the timed region)."""
        for i in range(warmup):
            fn(sets[i % len(sets)])
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        cap = torch.cuda.Stream()
        cap.wait_stream(stream)
        with torch.cuda.stream(cap):
            L.use_stream(cap)
            with torch.cuda.graph(g, stream=cap):
                for i in range(steps):
                    fn(sets[i % len(sets)])
        L.use_stream(stream)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(replays):
            g.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        del g
        return e0.elapsed_time(e1) / (steps * replays)  # ms

    cos_t, sin_t = L.rope_tables(1e7, D, 65536)
    emb = randn((VOCAB, H), std=0.02)
    gamma = randn((H,), std=0.1, mean=1.0)
    work = L.fp8_workspace()

    def prefill_sets(T, nsets, bits, group, pos0):
        sets = []
        pages = (T + 15) // 16
        for s in range(nsets):
            res = randn((T, H))
            ch = torch.randperm(H, generator=gen, device=dev)[: H // 100]
            res[:, ch] = (res[:, ch].float() * 20).to(torch.bfloat16)
            st = {
                "tok": torch.randint(0, VOCAB, (T,), generator=gen, device=dev, dtype=torch.int32),
                "emb_out": torch.empty((T, H), dtype=torch.bfloat16, device=dev),
                "res": res, "branch": randn((T, H)),
                "res_out": torch.empty((T, H), dtype=torch.bfloat16, device=dev),
                "codes_h": torch.empty((T, H), dtype=torch.uint8, device=dev),
                "scale": torch.empty(1, dtype=torch.float32, device=dev),
                "gu": randn((T, 2 * I)),
                "codes_i": torch.empty((T, I), dtype=torch.uint8, device=dev),
                "qkv": randn((T, (HQ + 2 * HK) * D)),
                "q_rot": torch.empty((T, HQ * D), dtype=torch.bfloat16, device=dev),
                "arena": L.KvArena(bits, HK, (pos0 % 16) + pages * 16 + 16, group=group),
                "pos0": pos0,
            }
            # fresh contiguous pages of the pool, page table by position
            stride = st["arena"].stride
            pt = torch.full((pos0 + T,), -1, dtype=torch.int32)
            pt[pos0:] = torch.arange(T, dtype=torch.int32) + (pos0 % 16)
            st["pt"] = pt.to(dev)
            assert int(pt[-1]) < stride
            sets.append(st)
        return sets

    def op_embed(s):
        T = s["res"].shape[0]
        L.call("granite4_embed_rows", s["tok"], T, emb, VOCAB, H, 1.0, s["emb_out"])

    def op_norm_fp8(s):
        T = s["res"].shape[0]
        L.call("granite4_add_rmsnorm_fp8", s["res"], s["branch"], 1.0, gamma, 1e-5, T, H,
               s["res_out"], s["codes_h"], s["scale"], work)

    def op_swiglu_fp8(s):
        T = s["gu"].shape[0]
        L.call("granite4_swiglu_fp8", s["gu"], T, I, s["codes_i"], s["scale"], work, None)

    def op_rope(s):
        qkv = s["qkv"]
        L.rope_append(s["arena"], qkv[:, :HQ * D], qkv[:, HQ * D:(HQ + HK) * D],
                      qkv[:, (HQ + HK) * D:], cos_t, sin_t, base_pos=s["pos0"], d_pt=s["pt"],
                      k_round_bf16=False, q_rot=s["q_rot"])

    def op_step(s):
        op_embed(s)
        op_norm_fp8(s)
        op_swiglu_fp8(s)
        op_rope(s)

    def rotation(b, steps):
        """Input sets for an op of b bytes per call such that one replay of
        the timed graph touches more than ROTATE_BYTES distinct bytes of the
        op's own buffers (more than the 256 MB Infinity Cache holds), and
        the graph's call count: every set once per replay, at least `steps`
        calls."""
        n = max(2, -(-int(ROTATE_BYTES) // int(b)))
        return n, n * max(1, -(-steps // n))

    def measure_ops(T, bits, group, pos0, rope_key, steps, warmup):
        ops = (("embed", op_embed, B_EMBED * T),
               ("add_rmsnorm_fp8", op_norm_fp8, B_NORM_FP8 * T + per_launch_extra("norm_fp8")),
               ("swiglu_fp8", op_swiglu_fp8, B_SWIGLU_FP8 * T + per_launch_extra("swiglu_fp8")),
               (f"rope_append_{rope_key}", op_rope, B_ROPE[rope_key] * T))
        step_bytes = sum(b for _, _, b in ops)
        nsets = max(rotation(b, steps)[0] for _, _, b in ops + (("step", None, step_bytes),))
        sets = prefill_sets(T, nsets, bits, group, pos0)
        out = {}
        for name, fn, b in ops:
            n, calls = rotation(b, steps)
            ms = timed(fn, calls, warmup, sets[:n])
            gbs = b / (ms * 1e-3) / 1e9
            out[name] = {"us": round(ms * 1e3, 3), "bytes": int(b), "GBps": round(gbs, 1),
                         "frac_peak": round(gbs / PEAK_GBS, 4), "sets": n,
                         "rotated_MB": round(n * b / 1e6, 1)}
        n, calls = rotation(step_bytes, steps)
        ms = timed(op_step, calls, warmup, sets[:n])
        out["step"] = {"us": round(ms * 1e3, 3), "bytes": int(step_bytes),
                       "GBps": round(step_bytes / (ms * 1e-3) / 1e9, 1), "sets": n,
                       "rotated_MB": round(n * step_bytes / 1e6, 1)}
        del sets
        torch.cuda.empty_cache()
        return out

    result_extra = {}

    if args.only:
        if args.only == "t512":
            r = measure_ops(512, 8, 128, 0, 8, args.steps, args.warmup)
        elif args.only == "t8192":
            r = measure_ops(8192, 5, 32, 57344, "k5v4g32", args.steps, args.warmup)
        elif args.only == "probe":
            r = bench_probe(torch, L, stream, timed)
        elif args.only == "t1":
            r = bench_t1_ops(torch, L, randn, timed, cos_t, sin_t, emb, gamma)
        elif args.only == "floor":
            r = bench_floor(torch, L, timed, work)
        elif args.only == "tN":
            r = measure_ops(args.T, 8, 128, 0, 8, args.steps, args.warmup)
        elif args.only == "decode_gemv":
            r = bench_decode_gemv(torch, L, gen, cos_t, sin_t, emb, gamma, stream)
        elif args.only == "fp8_trace":
            r = bench_fp8_trace(torch, L, randn, gamma)
        elif args.only == "layer_steps":
            r = bench_layer_steps(torch, L, gen, cos_t, sin_t, emb, gamma, stream)
        elif args.only == "multi_step":
            r = bench_layer_steps(torch, L, gen, cos_t, sin_t, emb, gamma, stream, prefill=False)
        elif args.only == "decode_trace":
            r = bench_decode_gemv(torch, L, gen, cos_t, sin_t, emb, gamma, stream,
                                  trace_replays=25)
        elif args.only == "decode":
            r = {"decode_T1": bench_decode(torch, L, randn, cos_t, sin_t, emb, gamma, stream, args),
                 "decode_T1_with_attention": bench_decode(torch, L, randn, cos_t, sin_t, emb, gamma,
                                                          stream, args, with_attn=True)}
        elif args.only == "t8":
            r = bench_multi8(torch, L, randn, cos_t, sin_t, gamma, work, gen, stream, timed, args)
        elif args.only == "attn":
            r = bench_attn(torch, L, randn, gen, timed, args)
        elif args.only == "gemm":
            r = bench_gemm(torch, L, gen, timed, work, args)
        else:
            r = bench_stress(torch, L, randn, cos_t, sin_t, gamma, stream)
        print(json.dumps({"only": args.only, "detail": r}), flush=True)
        return

    # ---------------------------------------------------------------- headline: T = 512
    # First, so that its 8 GB of weights are allocated from fresh device memory.
    log("config 1 with the decode GEMVs: non-GEMM overhead of the fused batch-1 decode step")
    result_extra["decode_T1_gemv"] = bench_decode_gemv(torch, L, gen, cos_t, sin_t, emb, gamma,
                                                       stream)
    log(json.dumps(result_extra["decode_T1_gemv"]))

    log("config 3: prefill T=512 (embed + add_rmsnorm_fp8 + swiglu_fp8 + rope_int8)")
    c3 = measure_ops(512, 8, 128, 0, 8, args.steps, args.warmup)
    log(json.dumps(c3))
    result_extra["prefill_T512"] = c3

    # ---------------------------------------------------------------- decode T = 1, 40 layers
    log("config 1: 40-layer batch-1 decode step as one HIP graph")
    decode = bench_decode(torch, L, randn, cos_t, sin_t, emb, gamma, stream, args)
    log(json.dumps(decode))
    result_extra["decode_T1"] = decode

    log("config 1: each op alone at T=1")
    result_extra["decode_T1_ops"] = bench_t1_ops(torch, L, randn, timed, cos_t, sin_t, emb, gamma)
    log(json.dumps(result_extra["decode_T1_ops"]))

    log("the fixed floor under the T=512 ops (launch, grid synchronisation, same-size copies)")
    result_extra["floor_T512"] = bench_floor(torch, L, timed, work)
    log(json.dumps(result_extra["floor_T512"]))

    if not args.quick:
        log("config 1 + attention: the decode step with the split-KV attention per layer")
        result_extra["decode_T1_with_attention"] = bench_decode(torch, L, randn, cos_t, sin_t, emb,
                                                                gamma, stream, args, with_attn=True)
        log(json.dumps(result_extra["decode_T1_with_attention"]))
        log("config 2: T=8 sessions")
        result_extra["decode_T8"] = bench_multi8(torch, L, randn, cos_t, sin_t, gamma, work, gen,
                                                 stream, timed, args)
        log(json.dumps(result_extra["decode_T8"]))
        log("config 4: prefill T=8192, RoPE at 57344.., K5V4 group 32")
        result_extra["prefill_T8192"] = measure_ops(8192, 5, 32, 57344, "k5v4g32",
                                                    max(5, args.steps // 2), 2)
        log(json.dumps(result_extra["prefill_T8192"]))
        log("config 5: bandwidth stress, 40 layers x T=32768, bf16")
        result_extra["stress_T32768"] = bench_stress(torch, L, randn, cos_t, sin_t, gamma, stream)
        log(json.dumps(result_extra["stress_T32768"]))

        log("split-KV decode attention over the paged pool (next row: the KV consumer)")
        result_extra["attn_decode"] = bench_attn(torch, L, randn, gen, timed, args)
        log(json.dumps(result_extra["attn_decode"]))

        log("FP8 GEMMs with the layer ops fused into their epilogues (next row)")
        result_extra["gemm_fused"] = bench_gemm(torch, L, gen, timed, work, args)
        log(json.dumps(result_extra["gemm_fused"]))

    log("bandwidth probe (achievable read / copy rate on this device)")
    result_extra["probe"] = bench_probe(torch, L, stream, timed)
    log(json.dumps(result_extra["probe"]))

    # ---------------------------------------------------------------- CPU baseline
    cpu = None if args.no_cpu else cpu_baseline()
    if cpu is not None:
        log(json.dumps(cpu))

    dom = c3["swiglu_fp8"]
    line = {
        "metric": "achieved HBM GB/s (% of peak) for fused layer ops at T=1 and T=512; "
                  "µs/decode step",
        "value": c3["step"]["GBps"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(c3["step"]["us"] / 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded torch RNG; N(0,1) hidden with 1% x20 outlier channels)",
        "config": {"workload": "prefill T=512, one layer: embed + add_rmsnorm_fp8 + swiglu_fp8 "
                               "+ rope_append int8 paged KV",
                   "T": 512, "H": H, "I": I, "Hq": HQ, "Hk": HK, "head_dim": D,
                   "kv": "int8 per (head,token)", "page": 16},
        "roofline": {"bound": "hbm", "kernel": "swiglu_fp8 (single launch: swiglu_fp8_fused_kernel)",
                     "achieved": dom["GBps"], "peak": PEAK_GBS, "unit": "GB/s",
                     "frac": round(dom["GBps"] / PEAK_GBS, 4),
                     "traffic": profiled_traffic("swiglu_fp8_fused_kernel"),
                     "traffic_source": "profiles/layerops_prefill_T512_hbm_traffic.md"},
        "cpu_baseline": cpu,
        "measured_probe_GBps": result_extra["probe"],
        "T1_ops": {k: {"us": v["us"], "GBps": v["GBps"], "frac_peak": v["frac_peak"]}
                   for k, v in result_extra["decode_T1_ops"].items()},
        "T512_ops": {k: {"us": v["us"], "GBps": v["GBps"], "frac_peak": v.get("frac_peak")}
                     for k, v in c3.items()},
        "decode_us_per_step": result_extra["decode_T1_gemv"]["with_attention"]["fused_us"],
        "decode_non_gemm_overhead_us": {
            "with_attention": result_extra["decode_T1_gemv"]["with_attention"][
                "non_gemm_overhead_fused_us"],
            "config1_ops_in_gemvs": result_extra["decode_T1_gemv"]["config1_non_gemm_overhead_us"],
            "gemvs_rope_append_launch": result_extra["decode_T1_gemv"][
                "non_gemm_overhead_fused_us"],
            "standalone_ops_graph_us": decode["graph_us_per_step"]},
        "detail": result_extra,
    }
    print(json.dumps(line), flush=True)


def bench_decode(torch, L, randn, cos_t, sin_t, emb, gamma, stream, args, layers=40,
                 with_attn=False):
    """161 launches: embed, then per layer add_rmsnorm (attention residual),
    rope + bf16 KV append at *d_pos, add_rmsnorm (FFN residual), SwiGLU.
    with_attn adds the split-KV attention of the appended pool (split +
    combine, 241 launches): the KV read of a 4322-position context."""
    dev = "cuda"
    stride = 8192
    pos = torch.tensor([4321], dtype=torch.int32, device=dev)
    toks = torch.randint(0, VOCAB, (8192,), dtype=torch.int32, device=dev)
    pt = torch.randperm(stride, device=dev).to(torch.int32)
    res = torch.empty((1, H), dtype=torch.bfloat16, device=dev)
    normed = torch.empty_like(res)
    act = torch.empty((1, I), dtype=torch.bfloat16, device=dev)
    q_rot = torch.empty((1, HQ * D), dtype=torch.bfloat16, device=dev)
    attn_out = torch.empty((1, HQ * D), dtype=torch.bfloat16, device=dev)
    scratch = torch.empty(L.call_size("granite4_attn_split_scratch_bytes", HQ, 1, stride),
                          dtype=torch.uint8, device=dev)
    per = []
    for _ in range(layers):
        per.append({"b_attn": randn((1, H)), "b_ffn": randn((1, H)), "gu": randn((1, 2 * I)),
                    "q": randn((1, HQ * D)), "k": randn((1, HK * D)), "v": randn((1, HK * D)),
                    "arena": L.KvArena(16, HK, stride)})

    def step():
        L.call("granite4_embed_at_pos", toks, pos, emb, VOCAB, H, 1.0, res)
        for p in per:
            a = p["arena"]
            L.call("granite4_add_rmsnorm", res, p["b_attn"], 1.0, gamma, 1e-5, 1, H, res, normed)
            L.call("granite4_rope_append_at_pos", p["q"], p["k"], p["v"], cos_t, sin_t, 65536,
                   pos, pt, HQ, HK, D, 16, 128, q_rot, a.k, a.v, a.k_scale, a.v_scale, stride)
            if with_attn:
                L.call("granite4_attn_paged", q_rot, 1, HQ, HK, D, 1.0 / 128, a.k, a.v, None, None,
                       16, 128, stride, 0, pos, pt, None, None, 0, 0, scratch, attn_out)
            L.call("granite4_add_rmsnorm", res, p["b_ffn"], 1.0, gamma, 1e-5, 1, H, res, normed)
            L.call("granite4_swiglu", p["gu"], 1, I, act)

    # eager timing (launch-bound: includes host launch cost)
    for _ in range(3):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    n_eager = 10
    for _ in range(n_eager):
        step()
    torch.cuda.synchronize()
    eager_us = (time.perf_counter() - t0) / n_eager * 1e6

    # graph capture on a side stream, replay on it
    g = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cap):
        L.use_stream(cap)
        step()  # warm the side stream
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=cap):
            step()
    L.use_stream(stream)
    torch.cuda.synchronize()
    for _ in range(5):
        g.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    reps = 50
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    graph_us = e0.elapsed_time(e1) / reps * 1e3
    ideal = B_EMBED + layers * (2 * B_NORM_BF16 + B_SWIGLU_BF16 + B_ROPE[16])
    if with_attn:
        ideal += layers * (int(pos.item()) + 1) * HK * kv_bytes_per_position(16, 128)
    return {"layers": layers, "launches": 1 + (6 if with_attn else 4) * layers,
            "graph_us_per_step": round(graph_us, 2),
            "eager_us_per_step": round(eager_us, 2), "ideal_bytes": ideal,
            "ideal_us_at_peak": round(ideal / PEAK_GBS / 1e3, 3)}


def bench_t1_ops(torch, L, randn, timed, cos_t, sin_t, emb, gamma, nsets=8):
    """BASELINE config 1's ops one at a time at T = 1 (bf16 outputs), each
    timed as the prefill ops are (a graph of back-to-back calls over rotating
    input sets): µs per call, algorithmic bytes and GB/s. At this size every
    op is one launch's fixed cost (see bench_floor)."""
    dev = "cuda"
    stride = 8192
    toks = torch.randint(0, VOCAB, (8192,), dtype=torch.int32, device=dev)
    pt = torch.randperm(stride, device=dev).to(torch.int32)
    sets = []
    for i in range(nsets):
        sets.append({"pos": torch.tensor([1000 + 7 * i], dtype=torch.int32, device=dev),
                     "res": randn((1, H)), "br": randn((1, H)),
                     "res_out": torch.empty((1, H), dtype=torch.bfloat16, device=dev),
                     "normed": torch.empty((1, H), dtype=torch.bfloat16, device=dev),
                     "gu": randn((1, 2 * I)), "act": torch.empty((1, I), dtype=torch.bfloat16,
                                                                 device=dev),
                     "q": randn((1, HQ * D)), "k": randn((1, HK * D)), "v": randn((1, HK * D)),
                     "q_rot": torch.empty((1, HQ * D), dtype=torch.bfloat16, device=dev),
                     "arena": L.KvArena(16, HK, stride)})
    ops = {
        "embed": (lambda s: L.call("granite4_embed_at_pos", toks, s["pos"], emb, VOCAB, H, 1.0,
                                   s["res_out"]), B_EMBED),
        "add_rmsnorm": (lambda s: L.call("granite4_add_rmsnorm", s["res"], s["br"], 1.0, gamma,
                                         1e-5, 1, H, s["res_out"], s["normed"]),
                        B_NORM_BF16 + per_launch_extra("norm_bf16")),
        "swiglu": (lambda s: L.call("granite4_swiglu", s["gu"], 1, I, s["act"]), B_SWIGLU_BF16),
        "rope_append_bf16": (lambda s: L.call(
            "granite4_rope_append_at_pos", s["q"], s["k"], s["v"], cos_t, sin_t, 65536, s["pos"],
            pt, HQ, HK, D, 16, 128, s["q_rot"], s["arena"].k, s["arena"].v, None, None, stride),
            B_ROPE[16]),
    }
    out = {}
    for name, (fn, b) in ops.items():
        ms = timed(fn, 40, 4, sets)
        gbs = b / (ms * 1e-3) / 1e9
        out[name] = {"us": round(ms * 1e3, 3), "bytes": int(b), "GBps": round(gbs, 2),
                     "frac_peak": round(gbs / PEAK_GBS, 5)}
    return out


def graph_us(torch, L, stream, step, reps=20):
    """µs per step() replayed as one HIP graph (captured on a side stream)."""
    g = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cap):
        L.use_stream(cap)
        step()
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=cap):
            step()
    L.use_stream(stream)
    torch.cuda.synchronize()
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    del g
    return e0.elapsed_time(e1) / reps * 1e3


def graphs_us(torch, L, stream, steps, rounds=5, reps=20):
    """µs per step for each of several steps (name -> function), each captured
    once as a HIP graph on a side stream, then timed round-robin over
    `rounds` rounds of `reps` replays; the median round of each. Interleaving
    keeps slow drifts of the clock (and the box) out of the differences
    between steps."""
    graphs = {}
    cap = torch.cuda.Stream()
    for name, step in steps.items():
        g = torch.cuda.CUDAGraph()
        cap.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(cap):
            L.use_stream(cap)
            step()
            torch.cuda.synchronize()
            with torch.cuda.graph(g, stream=cap):
                step()
        L.use_stream(stream)
        torch.cuda.synchronize()
        graphs[name] = g
    times = {name: [] for name in steps}
    for _ in range(rounds):
        for name, g in graphs.items():
            for _ in range(3):
                g.replay()
            torch.cuda.synchronize()
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                g.replay()
            e1.record()
            torch.cuda.synchronize()
            times[name].append(e0.elapsed_time(e1) / reps * 1e3)
    del graphs
    return {name: sorted(t)[len(t) // 2] for name, t in times.items()}


def paired_diff_us(torch, L, stream, base, other, pairs=41, reps=6):
    """µs per step of other() minus base(), each captured once as a HIP
    graph: `pairs` back-to-back pairs of timed blocks of `reps` replays (the
    order inside a pair alternating), the difference taken within each pair.
    Returns the median, 10th and 90th percentile of the per-pair differences
    and the median step times."""
    graphs = []
    cap = torch.cuda.Stream()
    for step in (base, other):
        g = torch.cuda.CUDAGraph()
        cap.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(cap):
            L.use_stream(cap)
            step()
            torch.cuda.synchronize()
            with torch.cuda.graph(g, stream=cap):
                step()
        L.use_stream(stream)
        torch.cuda.synchronize()
        graphs.append(g)

    def block(g):
        g.replay()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps * 1e3

    diffs, tb, to = [], [], []
    for i in range(pairs):
        if i % 2 == 0:
            b = block(graphs[0])
            o = block(graphs[1])
        else:
            o = block(graphs[1])
            b = block(graphs[0])
        diffs.append(o - b)
        tb.append(b)
        to.append(o)
    del graphs
    q = np.percentile(diffs, [10, 50, 90])
    return {"median_us": round(float(q[1]), 1), "p10_us": round(float(q[0]), 1),
            "p90_us": round(float(q[2]), 1), "pairs": pairs, "reps": reps,
            "base_us": round(float(np.median(tb)), 1), "other_us": round(float(np.median(to)), 1)}


def bench_decode_gemv(torch, L, gen, cos_t, sin_t, emb, gamma, stream, layers=40,
                      trace_replays=0):
    """Batch-1 decode step with its GEMVs (fp8 weight rows of the 8B model:
    q|k|v 6144 x 4096, o 4096 x 4096, gate and up 12800 x 4096, down 4096 x
    12800; 199 MB per layer, random e4m3 codes), three ways, each replayed as
    one HIP graph:
      plain    the GEMVs alone (no norm, RoPE, KV write, SwiGLU, residual);
      unfused  the reference's decode order: RMSNorm, q|k|v GEMV, RoPE + bf16
               KV append, O GEMV + residual, RMSNorm, gate/up GEMV + SwiGLU,
               down GEMV + residual (7 launches per layer);
      fused    RMSNorm as the GEMV prologue, SwiGLU and residual as epilogues,
               RoPE + KV append a launch of its own (5 per layer). Also timed:
               the same without the RoPE launches, and with RoPE + append in
               the q|k|v GEMV's epilogue (one workgroup per head: 48 of them,
               slower than the separate launch).
      config1  BASELINE config 1's ops (embed, add+RMSNorm, SwiGLU, RoPE on
               Q/K; no KV write) all inside the GEMVs: norm prologues, RoPE in
               the q|k|v epilogue, SwiGLU and residual epilogues (4 per layer).
    with attention: the same with the split-KV attention of each layer, the
    KV append inside the attention launch.
    The non-GEMM overhead of a step is its time minus the plain step's."""
    dev = "cuda"
    stride = 8192
    pos = torch.tensor([4321], dtype=torch.int32, device=dev)
    toks = torch.randint(0, VOCAB, (8192,), dtype=torch.int32, device=dev)
    pt = torch.randperm(stride, device=dev).to(torch.int32)

    def codes(*shape):
        c = torch.randint(0, 0x7F, shape, generator=gen, device=dev, dtype=torch.int32)
        sign = torch.randint(0, 2, shape, generator=gen, device=dev, dtype=torch.int32) << 7
        return (c | sign).to(torch.uint8)

    def bf(*shape):
        return torch.randn(shape, generator=gen, device=dev).to(torch.bfloat16)

    per = []
    for _ in range(layers):
        per.append({"wq": codes(HQ * D, H), "wk": codes(HK * D, H), "wv": codes(HK * D, H),
                    "wo": codes(H, HQ * D), "wg": codes(I, H), "wu": codes(I, H),
                    "wd": codes(H, I), "arena": L.KvArena(16, HK, stride)})
    hidden = bf(H)
    normed = bf(H)
    q, k, v = bf(HQ * D), bf(HK * D), bf(HK * D)
    q_rot = bf(HQ * D)
    attn_out = bf(HQ * D)
    act = bf(I)
    g_out, u_out, o_out = bf(I), bf(I), bf(H)
    sc = 1.0 / 512

    def plain():
        for p in per:
            L.call("granite4_gemv_qkv", normed, p["wq"], p["wk"], p["wv"], sc, sc, sc, HQ * D,
                   HK * D, HK * D, H, q, k, v)
            L.call("granite4_gemv_fp8w", attn_out, p["wo"], sc, H, HQ * D, o_out)
            L.call("granite4_gemv_qkv", normed, p["wg"], p["wu"], None, sc, sc, 0.0, I, I, 0, H,
                   g_out, u_out, None)
            L.call("granite4_gemv_fp8w", act, p["wd"], sc, H, I, o_out)

    def rope(p):
        a = p["arena"]
        L.call("granite4_rope_append_at_pos", q, k, v, cos_t, sin_t, 65536, pos, pt, HQ, HK, D,
               16, 128, q_rot, a.k, a.v, a.k_scale, a.v_scale, stride)

    def unfused():
        L.call("granite4_embed_at_pos", toks, pos, emb, VOCAB, H, 1.0, hidden)
        for p in per:
            L.call("granite4_kernel_rmsnorm", hidden, gamma, 1e-5, 1, H, normed)
            L.call("granite4_gemv_qkv", normed, p["wq"], p["wk"], p["wv"], sc, sc, sc, HQ * D,
                   HK * D, HK * D, H, q, k, v)
            rope(p)
            L.call("granite4_gemv_fp8w_resid", attn_out, p["wo"], sc, hidden, 1.0, H, HQ * D,
                   hidden)
            L.call("granite4_kernel_rmsnorm", hidden, gamma, 1e-5, 1, H, normed)
            L.call("granite4_kernel_silu_gate_up", p["wg"], p["wu"], normed, sc, sc, I, H, act)
            L.call("granite4_gemv_fp8w_resid", act, p["wd"], sc, hidden, 1.0, H, I, hidden)

    def fused():
        L.call("granite4_embed_at_pos", toks, pos, emb, VOCAB, H, 1.0, hidden)
        for p in per:
            a = p["arena"]
            L.call("granite4_gemv_rmsnorm_qkv_rope_append", hidden, gamma, 1e-5, p["wq"], p["wk"],
                   p["wv"], sc, sc, sc, cos_t, sin_t, 65536, pos, pt, HQ, HK, 16, 128, q_rot,
                   a.k, a.v, a.k_scale, a.v_scale, stride)
            L.call("granite4_gemv_fp8w_resid", attn_out, p["wo"], sc, hidden, 1.0, H, HQ * D,
                   hidden)
            L.call("granite4_gemv_rmsnorm_silu_gate_up", hidden, gamma, 1e-5, p["wg"], p["wu"],
                   sc, sc, I, H, act)
            L.call("granite4_gemv_fp8w_resid", act, p["wd"], sc, hidden, 1.0, H, I, hidden)

    def fused_split(with_rope):
        def step():
            L.call("granite4_embed_at_pos", toks, pos, emb, VOCAB, H, 1.0, hidden)
            for p in per:
                L.call("granite4_gemv_rmsnorm_qkv", hidden, gamma, 1e-5, p["wq"], p["wk"], p["wv"],
                       sc, sc, sc, HQ * D, HK * D, HK * D, H, q, k, v)
                if with_rope:
                    rope(p)
                L.call("granite4_gemv_fp8w_resid", attn_out, p["wo"], sc, hidden, 1.0, H, HQ * D,
                       hidden)
                L.call("granite4_gemv_rmsnorm_silu_gate_up", hidden, gamma, 1e-5, p["wg"],
                       p["wu"], sc, sc, I, H, act)
                L.call("granite4_gemv_fp8w_resid", act, p["wd"], sc, hidden, 1.0, H, I, hidden)
        return step

    attn_scr = torch.empty(L.call_size("granite4_attn_split_scratch_bytes", HQ, 1, stride),
                           dtype=torch.uint8, device=dev)

    def attn(p, qq):
        a = p["arena"]
        L.call("granite4_attn_paged", qq, 1, HQ, HK, D, 1.0 / 128, a.k, a.v, None, None, 16, 128,
               stride, 0, pos, pt, None, None, 0, 0, attn_scr, attn_out)

    def plain_attn():
        # the GEMVs and the attention alone: no norm, RoPE, KV append, SwiGLU, residual
        for p in per:
            L.call("granite4_gemv_qkv", normed, p["wq"], p["wk"], p["wv"], sc, sc, sc, HQ * D,
                   HK * D, HK * D, H, q, k, v)
            attn(p, q)
            L.call("granite4_gemv_fp8w", attn_out, p["wo"], sc, H, HQ * D, o_out)
            L.call("granite4_gemv_qkv", normed, p["wg"], p["wu"], None, sc, sc, 0.0, I, I, 0, H,
                   g_out, u_out, None)
            L.call("granite4_gemv_fp8w", act, p["wd"], sc, H, I, o_out)

    def unfused_attn():
        L.call("granite4_embed_at_pos", toks, pos, emb, VOCAB, H, 1.0, hidden)
        for p in per:
            L.call("granite4_kernel_rmsnorm", hidden, gamma, 1e-5, 1, H, normed)
            L.call("granite4_gemv_qkv", normed, p["wq"], p["wk"], p["wv"], sc, sc, sc, HQ * D,
                   HK * D, HK * D, H, q, k, v)
            rope(p)
            attn(p, q_rot)
            L.call("granite4_gemv_fp8w_resid", attn_out, p["wo"], sc, hidden, 1.0, H, HQ * D,
                   hidden)
            L.call("granite4_kernel_rmsnorm", hidden, gamma, 1e-5, 1, H, normed)
            L.call("granite4_kernel_silu_gate_up", p["wg"], p["wu"], normed, sc, sc, I, H, act)
            L.call("granite4_gemv_fp8w_resid", act, p["wd"], sc, hidden, 1.0, H, I, hidden)

    def fused_attn():
        # every non-GEMM op inside a GEMV or the attention launch: norm prologues,
        # RoPE + KV append in the attention, SwiGLU and residual epilogues
        L.call("granite4_embed_at_pos", toks, pos, emb, VOCAB, H, 1.0, hidden)
        for p in per:
            a = p["arena"]
            L.call("granite4_gemv_rmsnorm_qkv", hidden, gamma, 1e-5, p["wq"], p["wk"], p["wv"],
                   sc, sc, sc, HQ * D, HK * D, HK * D, H, q, k, v)
            L.call("granite4_attn_decode_append", q, k, v, cos_t, sin_t, 65536, pos, pt, HQ, HK,
                   1.0 / 128, a.k, a.v, a.k_scale, a.v_scale, 16, 128, stride, attn_scr,
                   attn_out)
            L.call("granite4_gemv_fp8w_resid", attn_out, p["wo"], sc, hidden, 1.0, H, HQ * D,
                   hidden)
            L.call("granite4_gemv_rmsnorm_silu_gate_up", hidden, gamma, 1e-5, p["wg"], p["wu"],
                   sc, sc, I, H, act)
            L.call("granite4_gemv_fp8w_resid", act, p["wd"], sc, hidden, 1.0, H, I, hidden)

    k_rot = bf(HK * D)

    # The library's whole decode step (granite4_decode_step): RoPE in the
    # q|k|v GEMV epilogue, the KV append in the attention, norm prologues,
    # SwiGLU and residual epilogues.
    dstep = L.DecodeStep(
        [{"attn_norm": gamma, "ffn_norm": gamma, "wq": p["wq"], "wk": p["wk"], "wv": p["wv"],
          "wo": p["wo"], "wg": p["wg"], "wu": p["wu"], "wd": p["wd"], "sq": sc, "sk": sc,
          "sv": sc, "so": sc, "sg": sc, "su": sc, "sd": sc, "cache_k": p["arena"].k,
          "cache_v": p["arena"].v} for p in per],
        H, I, HQ, HK, VOCAB, emb, cos_t, sin_t, eps=1e-5, emb_mult=1.0, resid_mult=1.0,
        attn_scale=1.0 / 128, kv_bits=16, kv_group=128, kv_stride=stride)

    def fused_attn_rot():
        dstep(toks, pos, pt)

    def fused_attn_parts(rope_gemv):
        # breakdown: the fused GEMVs with plain attention (no KV append);
        # rope_gemv selects the q|k|v GEMV with the RoPE epilogue
        def step():
            L.call("granite4_embed_at_pos", toks, pos, emb, VOCAB, H, 1.0, hidden)
            for p in per:
                if rope_gemv:
                    L.call("granite4_gemv_rmsnorm_qkv_rope", hidden, gamma, 1e-5, p["wq"],
                           p["wk"], p["wv"], sc, sc, sc, cos_t, sin_t, 65536, pos, HQ, HK, H,
                           q_rot, k_rot, v)
                    attn(p, q_rot)
                else:
                    L.call("granite4_gemv_rmsnorm_qkv", hidden, gamma, 1e-5, p["wq"], p["wk"],
                           p["wv"], sc, sc, sc, HQ * D, HK * D, HK * D, H, q, k, v)
                    attn(p, q)
                L.call("granite4_gemv_fp8w_resid", attn_out, p["wo"], sc, hidden, 1.0, H,
                       HQ * D, hidden)
                L.call("granite4_gemv_rmsnorm_silu_gate_up", hidden, gamma, 1e-5, p["wg"],
                       p["wu"], sc, sc, I, H, act)
                L.call("granite4_gemv_fp8w_resid", act, p["wd"], sc, hidden, 1.0, H, I, hidden)
        return step

    def fused_rope_epilogue():
        # config 1's ops (embed, add+RMSNorm, SwiGLU, RoPE on Q/K) all inside
        # the decode GEMVs: the embedding in the first q|k|v GEMV's prologue,
        # RoPE in the q|k|v epilogue, no KV write
        for i, p in enumerate(per):
            if i == 0:
                L.call("granite4_gemv_embed_rmsnorm_qkv_rope", toks, emb, VOCAB, 1.0, hidden, gamma,
                       1e-5, p["wq"], p["wk"], p["wv"], sc, sc, sc, cos_t, sin_t, 65536, pos, HQ,
                       HK, H, q_rot, k_rot, v)
            else:
                L.call("granite4_gemv_rmsnorm_qkv_rope", hidden, gamma, 1e-5, p["wq"], p["wk"],
                       p["wv"], sc, sc, sc, cos_t, sin_t, 65536, pos, HQ, HK, H, q_rot, k_rot, v)
            L.call("granite4_gemv_fp8w_resid", attn_out, p["wo"], sc, hidden, 1.0, H, HQ * D,
                   hidden)
            L.call("granite4_gemv_rmsnorm_silu_gate_up", hidden, gamma, 1e-5, p["wg"], p["wu"],
                   sc, sc, I, H, act)
            L.call("granite4_gemv_fp8w_resid", act, p["wd"], sc, hidden, 1.0, H, I, hidden)

    if trace_replays:
        # Kernel-trace mode: the plain and config-1 steps only, replayed
        # alternately, for a rocprofv3 kernel trace whose per-step kernel
        # duration sums (summarize_decode_trace) give the overhead without
        # the graph-timing noise of the launches around them.
        t = graphs_us(torch, L, stream, {"plain": plain, "config1": fused_rope_epilogue},
                      rounds=trace_replays, reps=1)
        del per
        torch.cuda.empty_cache()
        return {"layers": layers, "replays_each": trace_replays, "graph_us": t,
                "config1_non_gemm_overhead_us": round(t["config1"] - t["plain"], 1)}

    t = graphs_us(torch, L, stream, {
        "plain": plain, "plain_attn": plain_attn, "unfused_attn": unfused_attn,
        "parts_norope": fused_attn_parts(False), "parts_rope": fused_attn_parts(True),
        "rope_epi": fused_rope_epilogue, "fused_attn_ropeattn": fused_attn,
        "fused_attn": fused_attn_rot, "unfused": unfused, "qkv_rope_kernel": fused,
        "fused_norope": fused_split(False), "fused": fused_split(True)})
    t_plain, t_plain_attn, t_unfused_attn = t["plain"], t["plain_attn"], t["unfused_attn"]
    t_parts_norope, t_parts_rope, t_rope_epi = t["parts_norope"], t["parts_rope"], t["rope_epi"]
    t_fused_attn_ropeattn, t_fused_attn = t["fused_attn_ropeattn"], t["fused_attn"]
    t_unfused, t_qkv_rope_kernel = t["unfused"], t["qkv_rope_kernel"]
    t_fused_norope, t_fused = t["fused_norope"], t["fused"]
    # Config 1's overhead again as paired differences (plain and config-1
    # step timed back to back, 41 pairs): the median is steadier than the
    # difference of two separately taken medians.
    paired = paired_diff_us(torch, L, stream, plain, fused_rope_epilogue)
    wbytes = layers * (HQ * D + 2 * HK * D + 2 * I) * H + layers * H * (HQ * D + I)
    del per
    torch.cuda.empty_cache()
    return {"layers": layers, "weight_bytes": wbytes,
            "plain_gemv_us": round(t_plain, 1),
            "plain_gemv_GBps": round(wbytes / (t_plain * 1e-6) / 1e9, 1),
            "unfused_us": round(t_unfused, 1), "fused_us": round(t_fused, 1),
            "non_gemm_overhead_unfused_us": round(t_unfused - t_plain, 1),
            "non_gemm_overhead_fused_us": round(t_fused - t_plain, 1),
            "config1_fused_us": round(t_rope_epi, 1),
            "config1_non_gemm_overhead_us": paired["median_us"],
            "config1_non_gemm_overhead_paired": paired,
            "config1_non_gemm_overhead_rounds_us": round(t_rope_epi - t_plain, 1),
            "fused_gemvs_without_rope_us": round(t_fused_norope, 1),
            "rope_append_launches_us": round(t_fused - t_fused_norope, 1),
            "fused_qkv_rope_one_launch_us": round(t_qkv_rope_kernel, 1),
            "with_attention": {
                "context": int(pos.item()) + 1, "kv": "bf16",
                "plain_gemv_attn_us": round(t_plain_attn, 1),
                "unfused_us": round(t_unfused_attn, 1), "fused_us": round(t_fused_attn, 1),
                "non_gemm_overhead_unfused_us": round(t_unfused_attn - t_plain_attn, 1),
                "non_gemm_overhead_fused_us": round(t_fused_attn - t_plain_attn, 1),
                "fused_rope_in_attention_us": round(t_fused_attn_ropeattn, 1),
                "breakdown_us": {
                    "norm_swiglu_resid_embed": round(t_parts_norope - t_plain_attn, 1),
                    "rope_epilogue": round(t_parts_rope - t_parts_norope, 1),
                    "kv_append_in_attention": round(t_fused_attn - t_parts_rope, 1)},
                "launches_per_step": {"plain": 5 * layers, "unfused": 1 + 8 * layers,
                                      "fused": 1 + 5 * layers}},
            "launches_per_step": {"plain": 4 * layers, "unfused": 1 + 7 * layers,
                                  "fused": 1 + 5 * layers}}


def summarize_decode_trace(path, layers=40):
    """Per-step kernel time of the plain and config-1 decode steps from a
    rocprofv3 kernel trace (CSV) of `bench.py --only decode_trace`.

    A dispatch of gemv_kernel<0, 0, ...> (no prologue, plain output) belongs
    to the plain step; every other gemv_kernel (norm / embed prologues,
    residual, SwiGLU and RoPE epilogues) to the config-1 step. Each step is
    4 * layers dispatches; the k-th group of each class is the k-th replay.
    The overhead is the config-1 step's summed kernel durations minus the
    plain step's: the time the fused ops add inside the GEMVs, without the
    launch gaps (both steps launch 4 * layers kernels)."""
    import csv
    rows = []
    with open(path, newline="") as fh:
        for rec in csv.DictReader(fh):
            name = rec.get("Kernel_Name") or rec.get("KernelName") or ""
            if "gemv_kernel" not in name:
                continue
            t0 = int(rec.get("Start_Timestamp") or rec.get("BeginNs"))
            t1 = int(rec.get("End_Timestamp") or rec.get("EndNs"))
            rows.append((t0, t1, "gemv_kernel<0, 0," in name or "gemv_kernelILi0ELi0E" in name))
    rows.sort()
    per = 4 * layers
    def med(v):
        v = sorted(v)
        return v[len(v) // 2]

    steps, slots = {}, {}
    for cls, plain in (("plain", True), ("config1", False)):
        d = [t1 - t0 for t0, t1, p in rows if p == plain]
        n = len(d) // per
        steps[cls] = [sum(d[i * per:(i + 1) * per]) / 1e3 for i in range(n)]
        # the median duration of each of the step's 4 * layers launches over
        # the replays, summed: robust to the odd slow dispatch
        slots[cls] = sum(med([d[i * per + j] for i in range(n)]) for j in range(per)) / 1e3
    n = min(len(steps["plain"]), len(steps["config1"]))
    diff = sorted(steps["config1"][i] - steps["plain"][i] for i in range(n))
    return {"replays": n, "layers": layers,
            "plain_kernel_us_per_step": round(med(steps["plain"]), 1),
            "config1_kernel_us_per_step": round(med(steps["config1"]), 1),
            "config1_non_gemm_overhead_us": {
                "per_launch_medians": round(slots["config1"] - slots["plain"], 2),
                "median": round(med(diff), 2), "min": round(diff[0], 2),
                "max": round(diff[-1], 2), "p10": round(diff[n // 10], 2),
                "p90": round(diff[(9 * n) // 10], 2)}}


def bench_multi8(torch, L, randn, cos_t, sin_t, gamma, work, gen, stream, timed, args):
    """Config 2: 8 sessions at random positions in [0, 65536), own page tables,
    FP8 norm / SwiGLU outputs, int8 KV; per-layer op times."""
    dev = "cuda"
    n = 8
    pool_pages = 8 * 4096 + 64
    stride = pool_pages * 16
    rs = np.random.default_rng(2)
    pos = rs.integers(0, 65536, n).astype(np.int32)
    perm = torch.randperm(pool_pages, generator=gen, device=dev).to(torch.int32)
    # session i owns pages perm[i*4096:(i+1)*4096]; its position p -> row
    pts = []
    for i in range(n):
        pages = perm[i * 4096:(i + 1) * 4096].to(torch.int64)
        rows = (pages[:, None] * 16 + torch.arange(16, device=dev)[None, :]).reshape(-1)
        pts.append(rows.to(torch.int32).contiguous())
    M = L.multi_rows_struct()
    m = M()
    m.n = n
    for i in range(n):
        m.pos[i] = int(pos[i])
        m.pt[i] = pts[i].data_ptr()
    d_m = torch.from_numpy(np.frombuffer(bytes(m), np.uint8).copy()).to(dev)
    arena = L.KvArena(8, HK, stride)
    sets = []
    for _ in range(8):
        sets.append({"res": randn((n, H)), "branch": randn((n, H)), "gu": randn((n, 2 * I)),
                     "q": randn((n, HQ * D)), "k": randn((n, HK * D)), "v": randn((n, HK * D)),
                     "res_out": torch.empty((n, H), dtype=torch.bfloat16, device=dev),
                     "codes_h": torch.empty((n, H), dtype=torch.uint8, device=dev),
                     "codes_i": torch.empty((n, I), dtype=torch.uint8, device=dev),
                     "q_rot": torch.empty((n, HQ * D), dtype=torch.bfloat16, device=dev),
                     "scale": torch.empty(1, dtype=torch.float32, device=dev)})

    def norm(s):
        L.call("granite4_add_rmsnorm_fp8", s["res"], s["branch"], 1.0, gamma, 1e-5, n, H,
               s["res_out"], s["codes_h"], s["scale"], work)

    def swiglu(s):
        L.call("granite4_swiglu_fp8", s["gu"], n, I, s["codes_i"], s["scale"], work, None)

    def rope(s):
        L.call("granite4_multi_rope_append", s["q"], s["k"], s["v"], cos_t, sin_t, d_m, n, HQ, HK,
               D, 8, arena.k, arena.v, arena.k_scale, arena.v_scale, stride, s["q_rot"])

    out = {}
    for name, fn in (("add_rmsnorm_fp8", norm), ("swiglu_fp8", swiglu),
                     ("multi_rope_append_int8", rope)):
        out[name + "_us"] = round(timed(fn, 200, 20, sets) * 1e3, 3)
    out["layer_us"] = round(2 * out["add_rmsnorm_fp8_us"] + out["swiglu_fp8_us"] +
                            out["multi_rope_append_int8_us"], 3)
    return out


def bench_fp8_trace(torch, L, randn, gamma):
    """Per-workgroup timestamps of the single-launch FP8 kernels, from a
    measurement build of the library (build.py --define G4_TRACE_FP8, loaded
    with G4_LAYEROPS_LIB): µs after the first workgroup's start, [min,
    median, max] over the workgroups, of the last of 4 calls. Marks: start,
    first part held, all held / streamed once, grid maximum known, (swiglu:
    held part encoded), end."""
    work = L.fp8_workspace(65536)
    off = L.fp8_work_bytes(0)
    out = {}

    def marks(n):
        torch.cuda.synchronize()
        tr = work[off:off + 8 * 8 * 1024].view(torch.int64).cpu().numpy().reshape(-1, 8)[:, :n]
        tr = tr[tr[:, 0] > 0]
        if len(tr) == 0:
            return "no marks: load a build made with --define G4_TRACE_FP8"
        rel = (tr - tr[:, 0].min()) / 100.0
        return {"workgroups": len(tr),
                "marks_us": [[round(float(np.min(rel[:, i])), 1), round(float(np.median(rel[:, i])), 1),
                              round(float(np.max(rel[:, i])), 1)] for i in range(n)]}

    gu = [randn((8192, 2 * I)) for _ in range(2)]
    codes = torch.empty((8192, I), dtype=torch.uint8, device="cuda")
    scale = torch.empty(1, dtype=torch.float32, device="cuda")
    for i in range(4):
        if i == 3:
            work[off:].zero_()
        L.call("granite4_swiglu_fp8", gu[i % 2], 8192, I, codes, scale, work, None)
    out["swiglu_fp8_T8192"] = marks(6)
    del gu, codes
    for T in (8192, 4096, 512):
        xs = [randn((T, H)) for _ in range(2)]
        br = randn((T, H))
        ro = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
        c = torch.empty((T, H), dtype=torch.uint8, device="cuda")
        for i in range(4):
            if i == 3:
                work[off:].zero_()
            L.call("granite4_add_rmsnorm_fp8", xs[i % 2], br, 1.0, gamma, 1e-5, T, H, ro, c, scale,
                   work)
        out[f"add_rmsnorm_fp8_T{T}"] = marks(5)
    return out


def bench_layer_steps(torch, L, gen, cos_t, sin_t, emb, gamma, stream, prefill=True):
    """The engine's batched layer sequences through their single calls:
    granite4_prefill_layers (forward_prefill, one chunk) per layer at T=512
    (config 3: int8 KV, positions 0..511) and T=8192 (config 4: K5V4 group
    32, positions 57344..65535, attending to every earlier position), and granite4_decode_step_multi
    (forward_multi_step) for config 2's 8 sessions at random positions in
    [0, 65536) over 40 layers (int8 KV, each session's page table over its
    own 4096 pages of the pool). Both activation forms; random fp8 weights of
    the 8B shapes (q|k|v and gate|up one block each). Each timed as a HIP
    graph (graphs_us). prefill=False times the multi-session step only."""
    dev = "cuda"

    def codes(*shape):
        c = torch.randint(0, 0x7F, shape, generator=gen, device=dev, dtype=torch.int32)
        sign = torch.randint(0, 2, shape, generator=gen, device=dev, dtype=torch.int32) << 7
        return (c | sign).to(torch.uint8)

    def layers(n, bits, group, stride):
        out = []
        for _ in range(n):
            wqkv = codes((HQ + 2 * HK) * D, H)
            wgu = codes(2 * I, H)
            a = L.KvArena(bits, HK, stride, group=group)
            out.append({"attn_norm": gamma, "ffn_norm": gamma, "wq": wqkv[:HQ * D],
                        "wk": wqkv[HQ * D:(HQ + HK) * D], "wv": wqkv[(HQ + HK) * D:],
                        "wo": codes(H, HQ * D), "wg": wgu[:I], "wu": wgu[I:], "wd": codes(H, I),
                        "sq": 1 / 512, "sk": 1 / 512, "sv": 1 / 512, "so": 1 / 512,
                        "sg": 1 / 512, "su": 1 / 512, "sd": 1 / 512, "cache_k": a.k,
                        "cache_v": a.v, "k_scale": a.k_scale, "v_scale": a.v_scale, "_a": a})
        return out

    out = {}
    toks = torch.randint(0, VOCAB, (65536,), dtype=torch.int32, device=dev, generator=gen)
    nl = 4
    for T, bits, group, pos0, key in ((512, 8, 128, 0, "T512_int8"),
                                      (8192, 5, 32, 57344, "T8192_k5v4g32"))[:2 if prefill else 0]:
        # one sequence, arena row = position: the chunk at pos0 attends to
        # all pos0 earlier positions (zero-filled codes and scales)
        stride, pt = pos0 + T, None
        ly = layers(nl, bits, group, stride)
        st = L.LayerSteps(ly, H, I, HQ, HK, VOCAB, emb, cos_t, sin_t, T, eps=1e-5,
                          resid_mult=0.22, kv_bits=bits, kv_group=group, kv_stride=stride)
        t = graphs_us(torch, L, stream, {
            "fp8": lambda: st.prefill(toks, pos0, T, pt, L.OPS_FP8),
            "bf16": lambda: st.prefill(toks, pos0, T, pt, L.OPS_BF16)}, rounds=3, reps=3)
        out[f"prefill_{key}"] = {"layers_timed": nl,
                                 "fp8_us_per_layer": round(t["fp8"] / nl, 1),
                                 "bf16_us_per_layer": round(t["bf16"] / nl, 1)}
        del st, ly
        torch.cuda.empty_cache()
    n, pages_per = 8, 4096
    pool_pages = n * pages_per
    stride = pool_pages * 16
    ly = layers(40, 8, 128, stride)
    rs = np.random.default_rng(5)
    pos = rs.integers(0, 65536, n).astype(np.int32)
    perm = torch.randperm(pool_pages, generator=gen, device=dev).to(torch.int64)
    pts = [(perm[i * pages_per:(i + 1) * pages_per, None] * 16 +
            torch.arange(16, device=dev)[None, :]).reshape(-1).to(torch.int32).contiguous()
           for i in range(n)]
    tok_rows = [torch.randint(0, VOCAB, (65536,), dtype=torch.int32, device=dev, generator=gen)
                for _ in range(n)]
    M = L.multi_rows_struct()()
    M.n = n
    for i in range(n):
        M.pos[i] = int(pos[i])
        M.pt[i] = pts[i].data_ptr()
        M.tok[i] = tok_rows[i].data_ptr()
    d_m = torch.from_numpy(np.frombuffer(bytes(M), np.uint8).copy()).to(dev)
    st = L.LayerSteps(ly, H, I, HQ, HK, VOCAB, emb, cos_t, sin_t, n, eps=1e-5, resid_mult=0.22,
                      kv_bits=8, kv_group=128, kv_stride=stride)
    t = graphs_us(torch, L, stream, {"fp8": lambda: st.multi(d_m, n, L.OPS_FP8),
                                     "bf16": lambda: st.multi(d_m, n, L.OPS_BF16)},
                  rounds=3, reps=3)
    ctx = int(pos.sum()) + n
    out["decode_T8_multi_40_layers"] = {
        "sessions": n, "positions": [int(p) for p in pos], "fp8_us": round(t["fp8"], 1),
        "bf16_us": round(t["bf16"], 1),
        "weight_GB": round(40 * ((HQ + 2 * HK) * D * H + 2 * I * H + H * HQ * D + H * I) / 1e9, 2),
        "kv_read_GB": round(40 * ctx * HK * 2 * (D + 4) / 1e9, 2)}
    del st, ly
    torch.cuda.empty_cache()
    return out


def kv_bytes_per_position(bits, group):
    """K row + V row + f32 scales of one KV head at one position."""
    kb, vb = {16: (256, 256), 8: (128, 128), 4: (64, 64), 5: (80, 64)}[bits]
    return kb + vb + (0 if bits == 16 else 2 * 4 * (D // group))


FP8_MFMA_PEAK_TFLOPS = 5000.0  # MI355X dense FP8 matrix-core peak
BF16_MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 matrix-core peak


def bench_gemm(torch, L, gen, timed, work, args):
    """FP8 x FP8 GEMMs (granite4_gemm_fp8*) at the layer's shapes, T = 512 and
    8192: the gate|up projection with SwiGLU -> FP8 fused into its epilogue
    against the same GEMM storing bf16 gate|up followed by granite4_swiglu_fp8,
    and the O projection with the residual epilogue + RMSNorm -> FP8 against
    the GEMM storing the bf16 branch followed by granite4_add_rmsnorm_fp8.
    Random e4m3 codes (finite), two rotating input sets. TFLOP/s counts 2 M N K
    per GEMM; the roofline is the 5 PFLOP/s dense FP8 matrix-core peak."""
    dev = "cuda"
    out = {}

    def codes(shape):
        c = torch.randint(0, 0x7F, shape, generator=gen, device=dev, dtype=torch.int32)
        sign = torch.randint(0, 2, shape, generator=gen, device=dev, dtype=torch.int32) << 7
        return (c | sign).to(torch.uint8)

    only = getattr(args, "gemm_case", None)
    for T in (512, 8192):
        if only and not only.startswith(f"T{T}:"):
            continue
        sets = []
        for _ in range(2):
            sets.append({
                "a": codes((T, H)), "act_a": codes((T, I)),
                "w_gu": codes((2 * I, H)), "w_o": codes((H, H)), "w_d": codes((H, I)),
                "act": torch.empty((T, I), dtype=torch.bfloat16, device=dev),
                "codes_i": torch.empty((T, I), dtype=torch.uint8, device=dev),
                "gu": torch.empty((T, 2 * I), dtype=torch.bfloat16, device=dev),
                "hidden": torch.randn((T, H), generator=gen, device=dev).to(torch.bfloat16),
                "branch": torch.empty((T, H), dtype=torch.bfloat16, device=dev),
                "res_out": torch.empty((T, H), dtype=torch.bfloat16, device=dev),
                "codes_h": torch.empty((T, H), dtype=torch.uint8, device=dev),
                "scale": torch.empty(1, dtype=torch.float32, device=dev),
                "gamma": torch.ones(H, dtype=torch.bfloat16, device=dev),
                "hid_a": torch.randn((T, H), generator=gen, device=dev).to(torch.bfloat16),
                "qkv_out": torch.empty((T, 6144), dtype=torch.bfloat16, device=dev),
                "gu_f32": torch.empty((T, 2 * I), dtype=torch.float32, device=dev),
            })

        a_sc = torch.full((1,), 0.01, dtype=torch.float32, device=dev)

        def gu_fused(s):
            L.call("granite4_gemm_fp8_swiglu", s["a"], H, a_sc, s["w_gu"], T, I, H, 0.01, 0.01,
                   s["act"], s["codes_i"], s["scale"], work)

        def gu_unfused(s):
            L.gemm_fp8(s["a"], a_sc, s["w_gu"], out=s["gu"], scales=(0.01, 0.01, 0.01))
            L.call("granite4_swiglu_fp8", s["gu"], T, I, s["codes_i"], s["scale"], work, None)

        def o_fused(s):
            L.call("granite4_gemm_fp8_residual_rmsnorm_fp8", s["a"], H, a_sc, s["w_o"], T, H, H,
                   0.01, s["hidden"], 1.0, s["gamma"], 1e-5, s["codes_h"], s["scale"], work)

        def o_unfused(s):
            L.gemm_fp8(s["a"], a_sc, s["w_o"], out=s["branch"], scales=(0.01, 0.01, 0.01))
            L.call("granite4_add_rmsnorm_fp8", s["hidden"], s["branch"], 1.0, s["gamma"], 1e-5, T,
                   H, s["res_out"], s["codes_h"], s["scale"], work)

        def down(s):
            L.gemm_fp8(s["act_a"], a_sc, s["w_d"], out=s["hidden"], out_kind=L.GEMM_RESIDUAL,
                       scales=(0.01, 0.01, 0.01), residual=s["hidden"])

        # The reference's own prefill GEMM form (granite4_prefill_gemm: bf16
        # activations x fp8 weights), at the same shapes.
        def ref_qkv(s):
            L.prefill_gemm(s["hid_a"], s["w_gu"][:6144], out=s["qkv_out"],
                           scales=(0.01, 0.01, 0.01), segs=(4096, 5120))

        def ref_gu_f32(s):
            L.prefill_gemm(s["hid_a"], s["w_gu"], out_kind=L.GEMM_F32, out=s["gu_f32"],
                           scales=(0.01, 0.01, 0.01))

        def ref_down(s):
            L.prefill_gemm(s["act"], s["w_d"], out_kind=L.GEMM_RESIDUAL, out=s["hidden"],
                           scales=(0.01, 0.01, 0.01), residual=s["hidden"])

        steps = 10 if T == 512 else 4
        res = {}
        for name, fn, flops in (("gate_up_swiglu_fp8_fused", gu_fused, 2.0 * T * 2 * I * H),
                                ("gate_up_then_swiglu_fp8", gu_unfused, 2.0 * T * 2 * I * H),
                                ("o_residual_rmsnorm_fp8_fused", o_fused, 2.0 * T * H * H),
                                ("o_then_add_rmsnorm_fp8", o_unfused, 2.0 * T * H * H),
                                ("down_residual", down, 2.0 * T * H * I),
                                ("bf16A_qkv_bf16", ref_qkv, 2.0 * T * 6144 * H),
                                ("bf16A_gate_up_f32", ref_gu_f32, 2.0 * T * 2 * I * H),
                                ("bf16A_down_residual", ref_down, 2.0 * T * H * I)):
            if only and only != f"T{T}:{name}":
                continue
            ms = timed(fn, steps, 2, sets, replays=2)
            tf = flops / (ms * 1e-3) / 1e12
            res[name] = {"us": round(ms * 1e3, 2), "TFLOPs": round(tf, 1)}
            if name.startswith("bf16A"):
                res[name]["frac_bf16_peak"] = round(tf / BF16_MFMA_PEAK_TFLOPS, 4)
            else:
                res[name]["frac_fp8_peak"] = round(tf / FP8_MFMA_PEAK_TFLOPS, 4)
        out[f"T{T}"] = res
        del sets
        torch.cuda.empty_cache()
    return out


def bench_attn(torch, L, randn, gen, timed, args):
    """Split-KV decode attention (granite4_attn_paged) over one layer's paged
    pool: batch-1 decode at 8K and 32K context (bf16, int8, K5V4 group 32) and
    8 sessions at positions U[0, 65536) with their own page tables (int8).
    Algorithmic bytes: the KV rows and scales every query row attends to, plus
    q, out and the page-table entries. Input sets rotate past the 256 MB
    Infinity Cache (each layer's KV is cold in a real step)."""
    dev = "cuda"
    cases = [("T1_ctx8192_bf16", 1, 8192, 16, 128), ("T1_ctx8192_int8", 1, 8192, 8, 128),
             ("T1_ctx8192_k5v4g32", 1, 8192, 5, 32), ("T1_ctx32768_int8", 1, 32768, 8, 128),
             ("T8_sessions_ctx65536_int8", 8, 65536, 8, 128)]
    out = {}
    for name, rows, ctx, bits, group in cases:
        if getattr(args, "attn_case", None) and name != args.attn_case:
            continue
        stride = ctx
        pages = stride // 16
        kb, vb = {16: (256, 256), 8: (128, 128), 4: (64, 64), 5: (80, 64)}[bits]
        multi = rows > 1
        if multi:
            pos = torch.randint(0, ctx, (rows,), generator=gen, device=dev, dtype=torch.int32)
        else:
            pos = torch.tensor([ctx - 1], dtype=torch.int32, device=dev)
        lens = (pos.cpu().long() + 1)
        set_bytes = HK * stride * (kb + vb)
        nsets = max(2, min(8, -(-640 * 2 ** 20 // set_bytes)))
        sets = []
        for _ in range(nsets):
            st = {}
            if bits == 16:
                st["k"] = randn((HK * stride * D,), std=0.5)
                st["v"] = randn((HK * stride * D,))
                st["ks"] = st["vs"] = None
            else:
                st["k"] = torch.randint(0, 256, (HK * stride * kb,), generator=gen, device=dev,
                                        dtype=torch.uint8)
                st["v"] = torch.randint(0, 256, (HK * stride * vb,), generator=gen, device=dev,
                                        dtype=torch.uint8)
                ng = D // group
                st["ks"] = torch.rand((HK * stride * ng,), generator=gen, device=dev) * 0.005
                st["vs"] = torch.rand((HK * stride * ng,), generator=gen, device=dev) * 0.1
            st["q"] = randn((rows, HQ * D))
            tables = [(torch.randperm(pages, generator=gen, device=dev).to(torch.int32)[:, None] * 16 +
                       torch.arange(16, device=dev, dtype=torch.int32)).reshape(-1)
                      for _ in range(rows if multi else 1)]
            st["tables"] = tables
            st["pt"] = None if multi else tables[0]
            st["row_pos"] = pos if multi else None
            st["row_pt"] = (torch.tensor([t.data_ptr() for t in tables], dtype=torch.int64,
                                         device=dev) if multi else None)
            sets.append(st)
        d_pos = None if multi else pos
        scratch = torch.empty(L.call_size("granite4_attn_split_scratch_bytes", HQ, rows, stride),
                              dtype=torch.uint8, device=dev)
        o = torch.empty((rows, HQ * D), dtype=torch.bfloat16, device=dev)

        def fn(s):
            L.call("granite4_attn_paged", s["q"], rows, HQ, HK, D, 1.0 / 128, s["k"], s["v"],
                   s["ks"], s["vs"], bits, group, stride, 0, d_pos, s["pt"], s["row_pos"],
                   s["row_pt"], 0, 0, scratch, o)

        ms = timed(fn, 20, 3, sets)
        kv = int(sum(int(n) for n in lens)) * HK * kv_bytes_per_position(bits, group)
        b = kv + 2 * rows * HQ * D * 2 + int(sum(int(n) for n in lens)) * 4
        gbs = b / (ms * 1e-3) / 1e9
        out[name] = {"us": round(ms * 1e3, 3), "bytes": b, "GBps": round(gbs, 1),
                     "frac_peak": round(gbs / PEAK_GBS, 4), "sets": nsets}
        del sets, scratch
        torch.cuda.empty_cache()
    # Causal prefill attention over the pool: T = 512 from position 0 (int8, config
    # 3's shape) and T = 8192 at positions 57344.. (K5V4 group 32, config 4's shape).
    # MFMA-bound: the figure is TFLOP/s of the QK^T and PV products over the
    # causal (lower-triangular) key ranges.
    for name, T, pos0, bits, group in (("prefill_T512_int8", 512, 0, 8, 128),
                                       ("prefill_T8192_at57344_k5v4g32", 8192, 57344, 5, 32)):
        if getattr(args, "attn_case", None) and name != args.attn_case:
            continue
        stride = pos0 + T
        kb, vb = {16: (256, 256), 8: (128, 128), 4: (64, 64), 5: (80, 64)}[bits]
        ng = D // group
        st = {"k": torch.randint(0, 256, (HK * stride * kb,), generator=gen, device=dev,
                                 dtype=torch.uint8),
              "v": torch.randint(0, 256, (HK * stride * vb,), generator=gen, device=dev,
                                 dtype=torch.uint8),
              "ks": torch.rand((HK * stride * ng,), generator=gen, device=dev) * 0.005,
              "vs": torch.rand((HK * stride * ng,), generator=gen, device=dev) * 0.1,
              "q": randn((T, HQ * D)),
              "pt": (torch.randperm(stride // 16, generator=gen, device=dev).to(torch.int32)[:, None] * 16 +
                     torch.arange(16, device=dev, dtype=torch.int32)).reshape(-1)}
        o = torch.empty((T, HQ * D), dtype=torch.bfloat16, device=dev)

        def fnp(s):
            L.call("granite4_prefill_attn", s["q"], T, HQ, HK, D, 1.0 / 128, s["k"], s["v"], s["ks"],
                   s["vs"], bits, group, stride, pos0, s["pt"], 0, o)

        steps = 20 if T <= 512 else 3
        ms = timed(fnp, steps, 1, [st])
        keys = sum(pos0 + r + 1 for r in range(T))
        flops = 4.0 * HQ * D * keys
        out[name] = {"us": round(ms * 1e3, 3), "TFLOPs": round(flops / (ms * 1e-3) / 1e12, 2),
                     "frac_bf16_peak": round(flops / (ms * 1e-3) / 2.5e15, 4)}
        del st
        torch.cuda.empty_cache()
    return out


def bench_probe(torch, L, stream, timed):
    """Streaming read / copy probe (the reference's kernels_bench.cu pattern):
    the achievable HBM rate here, and known-size kernels for calibrating the
    FETCH_SIZE / WRITE_SIZE counters. 32 MB and 512 MB buffers, 4 rotating sets."""
    out = {}
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    for mb in (32, 512):
        nb = mb << 20
        sets = [(torch.ones(nb, dtype=torch.uint8, device="cuda"),
                 torch.empty(nb, dtype=torch.uint8, device="cuda")) for _ in range(4)]
        for mode, name, mult in ((2, "read_nt", 1), (3, "copy_nt", 2), (0, "read", 1),
                                 (1, "copy", 2)):
            ms = timed(lambda st, m=mode: L.call("granite4_bw_probe", st[0],
                                                  sink if m in (0, 2) else st[1], nb, m, 2048),
                       8, 2, sets)
            out[f"{name}_{mb}MB_GBps"] = round(mult * nb / (ms * 1e-3) / 1e9, 1)
        del sets
        torch.cuda.empty_cache()
    return out


def bench_floor(torch, L, timed, work, T=512):
    """The fixed floor under the T=512 ops, each measured as the ops are (a
    graph of back-to-back calls over 8 rotating buffer sets): an empty launch;
    one grid synchronisation with no data; and, per op, a kernel that only
    reads the op's input bytes and writes its output bytes in one launch
    (1024 workgroups, every load in flight), without and with one grid
    synchronisation between the loads and the stores."""
    out = {}
    steps = 40
    one = torch.zeros(16, dtype=torch.uint8, device="cuda")
    for blocks in (1, 512, 1024):
        ms = timed(lambda st, b=blocks: L.call("granite4_floor_probe", None, 0, None, 0, None, 0, b),
                   steps, 4, [None])
        out[f"empty_{blocks}wg_us"] = round(ms * 1e3, 3)
    for blocks in (512, 1024):
        ms = timed(lambda st, b=blocks: L.call("granite4_floor_probe", one, 0, one, 0, work, 2, b),
                   steps, 4, [None])
        out[f"sync_only_{blocks}wg_us"] = round(ms * 1e3, 3)
    ops = {"embed": (2 * H * T, 2 * H * T),
           "add_rmsnorm_fp8": (4 * H * T + 2 * H, 3 * H * T),
           "swiglu_fp8": (4 * I * T, I * T),
           "rope_append_8": (((HQ + 2 * HK) * D * 2 + 512 + 4) * T,
                             (HQ * D * 2 + 2 * HK * D + 2 * HK * 4) * T)}
    for name, (rb, wb) in ops.items():
        rb16, wb16 = (rb + 15) // 16 * 16, (wb + 15) // 16 * 16
        sets = [(torch.ones(rb16, dtype=torch.uint8, device="cuda"),
                 torch.empty(wb16, dtype=torch.uint8, device="cuda")) for _ in range(8)]
        r = {"read_B": rb, "write_B": wb}
        for mode, key in ((1, "copy"), (2, "copy_sync")):
            ms = timed(lambda st, m=mode: L.call("granite4_floor_probe", st[0], rb16, st[1], wb16,
                                                  work, m, 1024), steps, 4, sets)
            r[f"{key}_us"] = round(ms * 1e3, 3)
            r[f"{key}_frac_peak"] = round((rb + wb) / (ms * 1e-3) / 1e9 / PEAK_GBS, 4)
        out[name] = r
        del sets
        torch.cuda.empty_cache()
    return out


def bench_stress(torch, L, randn, cos_t, sin_t, gamma, stream, layers=40, T=32768):
    dev = "cuda"
    res = randn((T, H))
    branch = randn((T, H))
    normed = torch.empty_like(res)
    gu = randn((T, 2 * I))
    act = torch.empty((T, I), dtype=torch.bfloat16, device=dev)
    qkv = randn((T, (HQ + 2 * HK) * D))
    q_rot = torch.empty((T, HQ * D), dtype=torch.bfloat16, device=dev)
    arena = L.KvArena(16, HK, T)
    pt = torch.arange(T, dtype=torch.int32, device=dev)

    def layer():
        L.call("granite4_add_rmsnorm", res, branch, 1.0, gamma, 1e-5, T, H, res, normed)
        L.rope_append(arena, qkv[:, :HQ * D], qkv[:, HQ * D:(HQ + HK) * D], qkv[:, (HQ + HK) * D:],
                      cos_t, sin_t, base_pos=0, d_pt=pt, q_rot=q_rot)
        L.call("granite4_add_rmsnorm", res, branch, 1.0, gamma, 1e-5, T, H, res, normed)
        L.call("granite4_swiglu", gu, T, I, act)

    layer()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(layers):
        layer()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1)
    per_layer = (2 * B_NORM_BF16 + B_SWIGLU_BF16 + B_ROPE[16]) * T
    total = per_layer * layers
    return {"layers": layers, "T": T, "ms": round(ms, 3), "bytes": total,
            "GBps": round(total / (ms * 1e-3) / 1e9, 1),
            "frac_peak": round(total / (ms * 1e-3) / 1e9 / PEAK_GBS, 4)}


def cpu_baseline(budget_s=16.0):
    """The oracle (scalar C, oracle/g4_cpu_step.c) on the headline workload
    itself: the whole T=512 step (embed from the full 100352-row table,
    add+RMSNorm -> FP8, SwiGLU -> FP8, RoPE + int8 KV), about budget_s / 2
    seconds on one thread, then the same on every core of the box's share,
    the step split by token rows with the FP8 scales agreed between two
    barriers. Inputs are built before the timed loop; GB/s in the GPU's
    ideal-byte units (value = all cores)."""
    import ctypes
    import oracle_lib as ol
    fn = ol.lib.g4o_cpu_step_bench
    fn.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_double, ctypes.POINTER(ctypes.c_double)]
    fn.restype = ctypes.c_int
    T = 512
    step_bytes = T * (B_EMBED + B_NORM_FP8 + B_SWIGLU_FP8 + B_ROPE[8]) + \
        per_launch_extra("norm_fp8") + per_launch_extra("swiglu_fp8")
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    # The GPU box's CPU share is 16 cores per GPU: use all of them (fewer if
    # the process may run on fewer).
    cores = max(1, min(avail, 16))
    wall = ctypes.c_double()
    n1 = fn(T, 1, budget_s / 2, ctypes.byref(wall))
    t1 = wall.value
    nt = fn(T, cores, budget_s / 2, ctypes.byref(wall))
    tt = wall.value
    if n1 <= 0 or nt <= 0:
        return None
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(step_bytes * nt / tt / 1e9, 3), "unit": "GB/s", "cores": cores,
            "kind": "port", "cpu": model, "hardware_concurrency": os.cpu_count(),
            "affinity_cores": avail,
            "one_core_GBps": round(step_bytes * n1 / t1 / 1e9, 3),
            "ms_per_step_one_core": round(t1 / n1 * 1e3, 2),
            "ms_per_step_all_cores": round(tt / nt * 1e3, 2),
            "sample": f"the full T=512 step (BASELINE config 3: embed from the [100352][4096] "
                      f"table, add_rmsnorm + FP8, SwiGLU + FP8, RoPE + int8 paged KV) with the "
                      f"scalar C oracle: {n1} steps on one thread in {t1:.1f} s, then {nt} steps "
                      f"on {cores} threads (rows split across threads) in {tt:.1f} s"}


if __name__ == "__main__":
    main()
