"""Decode benchmark: batch-1 4-bit (MLX affine, group 64) LM decode on one
MI355X at a bf16 KV cache prefilled to 2048 positions, Qwen2-0.5B shape
(24 layers, hidden 896, 14/2 heads of 64, SwiGLU 4864, vocab 151936, tied
head, greedy argmax), random-init weights N(0, 0.02) quantized on the GPU.

A step is one decode token: embed(previous argmax) -> 24 layers -> final
norm -> LM head -> argmax, with the token fed back on the device.  Every
step decodes at position 2048 (the cache length is reset before each step,
so the appended row is rewritten in place and the context stays 2048).

Prints one JSON line (see the keys below).  `value` is tokens/s over the
timed region.  `roofline` prices the step kernel against HBM: algorithmic
bytes per token (4-bit weights incl. the tied head at 0.5625 B/param, biases
and norms, the KV read of 2048 rows and the one-row append) divided by the
kernel's average launch duration, which events recorded around every launch
on the launch stream measure inside the timed region (with the persistent
schedule a step is one launch).  `traffic` is the HBM bytes per launch that
rocprofv3's FETCH_SIZE/WRITE_SIZE counters measured for this workload,
scaled by a plain copy's reading (profiles/); null for other workloads.
`cpu_baseline` times the oracle (the CPU restatement in oracle/, OpenMP over
output rows) on the host cores on a bounded sample of the same workload.
"""
import argparse
import importlib
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "tests"))

METRIC = "LM decode tokens/s @bs1 ctx2048 (4-bit) + achieved HBM GB/s % of peak"
HBM_PEAK_GBS = 8000.0


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--ctx", type=int, default=2048)
    p.add_argument("--mode", choices=["auto", "kernels", "persistent", "direct"], default="auto")
    p.add_argument("--cpu-seconds", type=float, default=10.0, help="bound of the CPU baseline sample")
    p.add_argument("--no-cpu", action="store_true")
    return p.parse_args()


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the decode path runs on a single MI355X "
              "(multi-GPU sharding is described in DESIGN.md, not launched)", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch

    ming = importlib.import_module("ming-tts-serve_amd")
    S = importlib.import_module("ming-tts-serve_amd.synthetic")
    spec = S.QWEN2_05B
    ctx = ming.Context(0)
    t0 = time.time()
    syn = S.SyntheticLm(ctx, spec, seed=0, quant=True)
    m = syn.model()
    m.set_mode({"auto": ming.LM_AUTO, "kernels": ming.LM_KERNELS, "persistent": ming.LM_PERSISTENT,
                "direct": ming.LM_PERSISTENT_DIRECT}[args.mode])
    cache = S.KvCache(spec, args.ctx + 1)
    cache.fill_random(args.ctx, seed=1)
    torch.cuda.synchronize()
    print(f"[bench] setup {time.time() - t0:.1f}s", file=sys.stderr, flush=True)

    tok = torch.tensor([1234], dtype=torch.int32, device="cuda")

    def step():
        cache.kv.len = args.ctx
        m.step(cache.kv, token=tok, argmax=tok)

    for _ in range(args.warmup):
        step()
    ctx.sync()
    # the library launches on torch's current stream (Context binds it), so
    # these events bracket each launch on its own stream
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for i in range(args.steps):
        ev[i][0].record()
        step()
        ev[i][1].record()
    e1.record()
    torch.cuda.synchronize()
    ctx.sync()
    ms = e0.elapsed_time(e1) / args.steps
    launch_ms = sum(a.elapsed_time(b) for a, b in ev) / args.steps
    tok_s = 1000.0 / ms
    bytes_tok = S.lm_bytes_per_token(spec, args.ctx)
    achieved = bytes_tok / (launch_ms * 1e-3) / 1e9

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(ming, S, syn, cache, args)

    out = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init N(0,0.02) weights quantized to MLX affine 4-bit/g64; KV cache N(0,1))",
        "config": {
            "workload": f"Qwen2-0.5B-shaped 24-layer 4-bit LM decode step, bs1, ctx {args.ctx}, greedy argmax "
                        f"over 151936",
            "weights": "MLX affine u32 4-bit, group 64, bf16 scales/biases, global scale 1.0",
            "kv_cache": "bf16 in place",
            "schedule": args.mode,
            "global_batch": 1,
            "seq_len": args.ctx,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(args),
            "bytes_per_launch": bytes_tok,
            "launch_ms": round(launch_ms, 5),
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


def measured_traffic(args):
    """HBM bytes per launch from the committed rocprofv3 counter runs, for
    the workload they were taken on (ctx 2048, persistent schedule)."""
    path = os.path.join(ROOT, "profiles", "decode_tagged_kernel_ctx2048_traffic.json")
    if args.ctx != 2048 or args.mode not in ("auto", "persistent") or not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f)["traffic_bytes_per_dispatch"]


def cpu_baseline(ming, S, syn, cache, args):
    """Oracle decode steps on the host cores at the same context, for about
    args.cpu_seconds (at least one step)."""
    import numpy as np

    import oracle
    from lmkit import oracle_model, oracle_step

    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1)
    oracle.set_threads(threads)
    cfg, layers, norm, head = oracle_model(syn)
    kc, vc = cache.host()
    tok = 1234
    n = 0
    t0 = time.time()
    while True:
        x = oracle.embed(head, tok)
        tok, _, _, _, _ = oracle_step(cfg, layers, norm, head, x, args.ctx, kc, vc)
        n += 1
        if time.time() - t0 >= args.cpu_seconds:
            break
    dt = time.time() - t0
    return {
        "value": round(n / dt, 3),
        "unit": "tokens/s",
        "cores": oracle.get_threads(),
        "kind": "port",
        "sample": f"{n} decode tokens of the same 24-layer 4-bit model at ctx {args.ctx} "
                  f"({dt:.1f} s, C restatement of the MLX CPU graph, OpenMP over output rows)",
    }


if __name__ == "__main__":
    main()
