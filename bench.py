"""Decode benchmark: batch-1 4-bit (MLX affine, group 64) LM decode on one
MI355X over a bf16 KV cache prefilled to 2048 positions, Qwen2-0.5B shape
(24 layers, hidden 896, 14/2 heads of 64, SwiGLU 4864, vocab 151936, tied
head, greedy argmax), random-init weights N(0, 0.02) quantized on the GPU.

A step is one decode token: embed(previous argmax) -> 24 layers -> final
norm -> LM head -> argmax, with the token fed back on the device.  The cache
grows by one row per step: the warm-up steps decode the positions just
before 2048 and the K timed steps positions 2048 .. 2048 + K - 1.

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

Two more workloads print a line of the same form (`--workload`):
  cfm   one flow-head sample per step (cfmSample: 10 CFG Euler steps through
        8 DiT blocks, hidden 1024, 16 x 64 heads, ff 4096, 6 rows; bf16
        weights N(0, 0.02)); roofline over the weight bytes of a sample.
        --mode kernels|persistent picks the launch path or the persistent
        kernel (auto: the launch path); --stamps with persistent prints the
        per-stage timing from the kernel's stamps.
  c4    one sample of config 4's adaLN flow head per step (4 blocks, hidden
        896, 14 x 64 heads, ff 3584, a patch of 4 frames x 64, 10 CFG Euler
        steps; the modulations of all steps are computed once per sample).
  loop  one token of the TTS loop per step (sampleLatents: flow head,
        aggregator, a hidden-only 4-bit LM decode step and the stop head),
        the per-token time being the difference of a K-step and a 1-step run
        after the same prompt prefill; roofline over the token's weight and
        KV bytes.
  server  config 5's multi-request decode: --seqs sequences (16 or 64) with
        contexts drawn uniform in [128, 4096] (seed 0) over a paged bf16 KV
        cache advance one token per step (each fed its own argmax) through
        the batched 4-bit step (MFMA GEMMs, paged attention), and the DiT
        flow head samples every sequence's latent from its hidden state
        (ming_cfm_sample_batch: 10 CFG Euler steps through 8 blocks, bf16;
        --lm-only leaves it out); value is tokens/s over all sequences;
        roofline over the step's weight bytes (4-bit LM once, the flow head's
        bf16 weights once per Euler step) plus every sequence's KV read and
        append.
  gemv  config 2's isolated 4-bit GEMV sweep (ming_qgemv): [in x out] =
        [896x896], [896x128], [896x4864], [4864x896], [896x151936] at global
        scales 1, 0.5 and 3, weights quantized on the GPU from N(0, 0.02), x
        N(0, 1).  Each shape's matrix is replicated into copies totalling more
        than 512 MB that the dispatches cycle through, so every dispatch reads
        its weights from HBM, not from the 256 MB MALL; --steps dispatches are
        queued behind a device fill so that they run back to back, and the
        time per dispatch is the events' span over them (host-bound entries
        are flagged).  value is the GB/s of the [896x151936] head shape at
        g = 1; every entry is listed under `sweep`.
  dit   the flow head's four block kernels one at a time (ming_dit_single:
        A rms + q/k/v + rotary + attention, B out_proj + residual, C rms +
        ff1 + gelu, D ff2 + residual) at the reference shape (R = 2 x 3
        rows, hidden 1024, ff 4096), --steps dispatches of each kernel
        cycling through copies of its weights that total more than
        --rotate-mb (so each dispatch's weights come from HBM: the 16 real
        blocks' q/k/v alone, 100 MB, would sit in the 256 MB MALL), queued
        behind a device fill; value is the four kernels' weight bytes over
        their summed time per dispatch.
  prefill one 512-token prompt per step through ming_lm_prefill (one
        batched chunk of up to 512 rows over a paged cache, causal); value is prompt
        tokens/s; roofline over the weights once per chunk plus the causal
        KV reads and appends.
  c1    config 1's generate job per step: the bf16 Qwen2-0.5B-shaped LM
        (random-init bf16 weights N(0, 0.02), vocab 151936), a 64-token prompt
        of uniform ids fed one position at a time, then 128 greedy ids with the
        argmax fed back on the device (ming_lm_generate), the cache emptied at
        the start of each job; value is greedy ids/s over the whole job;
        roofline over the bf16 weight bytes of each of the job's 191 steps
        plus its KV reads and appends.
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
METRIC_CFM = "flow-head samples/s (cfmSample: 10 CFG Euler steps, 8 DiT blocks, hidden 1024, bf16) + achieved GB/s"
METRIC_C4 = "adaLN flow-head samples/s (config 4: 4 blocks, hidden 896, 4-frame patch, 10 CFG Euler steps, bf16) + achieved GB/s"
METRIC_DIT = "DiT block kernels achieved GB/s (fused.single A-D, weights rotated through HBM, bf16)"
METRIC_GEMV = "4-bit GEMV achieved GB/s (MLX affine g64, [896x151936] head shape, weights rotated through HBM)"
GEMV_SHAPES = [(896, 896), (896, 128), (896, 4864), (4864, 896), (896, 151936)]  # [in, out]
METRIC_C1 = ("LM generate greedy tokens/s (config 1: bf16 Qwen2-0.5B, 64-token prompt + 128 greedy steps, bs1) "
             "+ achieved HBM GB/s")
METRIC_LOOP = "TTS tokens/s (sampleLatents step: flow head + aggregator + 4-bit LM decode + stop head) + achieved GB/s"
HBM_PEAK_GBS = 8000.0
# the 4-bit paths' arithmetic: MLX-affine 4-bit weights, bf16 activations, f32 accumulation
DTYPE_W4 = "w4a16 (4-bit weights, bf16 activations, f32 accumulate)"


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--workload", choices=["lm", "c1", "cfm", "c4", "loop", "server", "prefill", "vae", "gemv", "dit"],
                   default="lm")
    p.add_argument("--shape", type=int, default=-1, help="gemv workload: one shape of the sweep (index), default all")
    p.add_argument("--rotate-mb", type=float, default=512.0, help="gemv and dit workloads: distinct weight bytes each kernel cycles through")
    p.add_argument("--weight-sets", type=int, default=1,
                   help="cfm workload: samples cycle through this many flow heads of distinct weights (202 MB per "
                        "Euler step each), so with 2 or more each sample's first reads come from HBM")
    p.add_argument("--seqs", type=int, default=64, help="server workload: concurrent sequences")
    p.add_argument("--lm-only", action="store_true", help="server workload: no DiT head")
    p.add_argument("--prompt", type=int, default=512, help="prefill workload: prompt tokens")
    p.add_argument("--latents", type=int, default=100, help="vae workload: latents per decode")
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--ctx", type=int, default=2048)
    p.add_argument("--mode", choices=["auto", "kernels", "persistent", "direct", "xcd"], default="auto")
    p.add_argument("--cpu-seconds", type=float, default=10.0, help="bound of the CPU baseline sample")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--stamps", action="store_true",
                   help="cfm workload with --mode persistent, or lm with the persistent schedule: per-stage timing "
                        "from the device stamps (stderr, after the timed run)")
    p.add_argument("--cooperative", action="store_true",
                   help="lm/loop: cooperative persistent launch (default: ordinary launch, the bench owns the device)")
    return p.parse_args()


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the decode path runs on a single MI355X "
              "(multi-GPU sharding is described in DESIGN.md, not launched)", file=sys.stderr)
        sys.exit(2)
    if args.workload == "cfm":
        return bench_cfm(args)
    if args.workload == "loop":
        return bench_loop(args)
    if args.workload == "c4":
        return bench_c4(args)
    if args.workload == "server":
        return bench_server(args)
    if args.workload == "prefill":
        return bench_prefill(args)
    if args.workload == "vae":
        return bench_vae(args)
    if args.workload == "c1":
        return bench_c1(args)
    if args.workload == "gemv":
        return bench_gemv(args)
    if args.workload == "dit":
        return bench_dit(args)
    import torch

    ming = importlib.import_module("ming-tts-serve_amd")
    S = importlib.import_module("ming-tts-serve_amd.synthetic")
    spec = S.QWEN2_05B
    ctx = ming.Context(0)
    ctx.set_exclusive(not args.cooperative)
    t0 = time.time()
    syn = S.SyntheticLm(ctx, spec, seed=0, quant=True)
    m = syn.model()
    m.set_mode({"auto": ming.LM_AUTO, "kernels": ming.LM_KERNELS, "persistent": ming.LM_PERSISTENT,
                "direct": ming.LM_PERSISTENT_DIRECT, "xcd": ming.LM_PERSISTENT_XCD}[args.mode])
    # the cache is prefilled so that the timed steps decode at positions ctx .. ctx + steps - 1:
    # the warm-up steps append the rows just before ctx, and every step appends one row
    start = max(1, args.ctx - args.warmup)
    cache = S.KvCache(spec, args.ctx + args.steps + 1)
    cache.fill_random(start, seed=1)
    torch.cuda.synchronize()
    print(f"[bench] setup {time.time() - t0:.1f}s", file=sys.stderr, flush=True)

    tok = torch.tensor([1234], dtype=torch.int32, device="cuda")

    def step():
        m.step(cache.kv, token=tok, argmax=tok)

    while cache.len < args.ctx:
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
    assert cache.len == args.ctx + args.steps
    ms = e0.elapsed_time(e1) / args.steps
    launch_ms = sum(a.elapsed_time(b) for a, b in ev) / args.steps
    tok_s = 1000.0 / ms
    # mean algorithmic bytes over the timed positions ctx .. ctx + steps - 1
    bytes_tok = int(round(sum(S.lm_bytes_per_token(spec, args.ctx + i) for i in range(args.steps)) / args.steps))
    achieved = bytes_tok / (launch_ms * 1e-3) / 1e9

    if args.stamps and args.mode in ("auto", "persistent", "direct", "xcd"):
        lm_stage_report(ctx, m, spec, cache, step, args.ctx)

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(ming, S, syn, cache, args)

    out = {
        "metric": METRIC if args.ctx == 2048 else METRIC.replace("ctx2048", f"ctx{args.ctx}"),
        "value": round(tok_s, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": DTYPE_W4,
        "data": "synthetic (random-init N(0,0.02) weights quantized to MLX affine 4-bit/g64; KV cache N(0,1))",
        "config": {
            "workload": f"Qwen2-0.5B-shaped 24-layer 4-bit LM decode, bs1, {args.steps} greedy steps over a KV cache "
                        f"prefilled to {args.ctx} (positions {args.ctx}..{args.ctx + args.steps - 1}), argmax over "
                        f"151936 fed back on the device",
            "weights": "MLX affine u32 4-bit, group 64, bf16 scales/biases, global scale 1.0",
            "arithmetic": "4-bit weights unpacked in registers, bf16 activations and KV cache, f32 accumulation",
            "kv_cache": "bf16 in place",
            "schedule": args.mode if args.mode != "auto" else f"auto ({lm_schedule(args)})",
            "launch": "cooperative" if args.cooperative else "ordinary (device held by this process alone)",
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
    m.close()
    ctx.close()
    print(json.dumps(out), flush=True)


def lm_stage_report(ctx, m, spec, cache, step, pos, reps=5):
    """Per-stage timing of the persistent decode step from its device stamps
    (ming_lm_model_profile: every workgroup stamps each stage's input arrival
    and its done, wall clock at 100 MHz), printed to stderr.  Per stage, over
    layers 2 .. L-3 and `reps` steps (medians over steps, means over layers):
    exchange = the previous stage's last done -> the median worker's arrival,
    work = the median worker's arrival -> its done, span = the previous
    stage's last done -> this stage's last done (the stage's share of the
    step), and the hubs' legs of the two normalised hand-offs."""
    import ctypes

    import numpy as np
    import torch

    ns, g = ctypes.c_int32(), ctypes.c_int32()
    ctx.check(ctx.L.ming_lm_model_profile_shape(m.h, ctypes.byref(ns), ctypes.byref(g)))
    ns, g = ns.value, g.value
    L, nh = spec.n_layers, 8
    st = torch.zeros((ns, g), dtype=torch.int64, device="cuda")
    runs = []
    for _ in range(reps):
        st.zero_()
        cache.kv.len = pos  # each profiled step decodes position pos again
        ctx.check(ctx.L.ming_lm_model_profile(m.h, ctypes.c_void_p(st.data_ptr())))
        step()
        ctx.sync()
        ctx.check(ctx.L.ming_lm_model_profile(m.h, ctypes.c_void_p(0)))
        runs.append(st.cpu().numpy().astype(np.float64))
    slot = lambda l, s: 1 + 2 * (5 * l + s)
    names = ("q/k/v", "attention", "o_proj", "gate/up", "down")
    rows = {n: [] for n in names}
    hubs = {"q/k/v": [], "o_proj": [], "gate/up": []}
    head = []
    for T in runs:
        T = T / 100.0  # ticks -> us
        W = T[:, nh:]
        prev_done = None
        seq = [(l, s) for l in range(L) for s in range(5)]
        for i, (l, s) in enumerate(seq):
            arr, done = W[slot(l, s)], W[slot(l, s) + 1]
            on = (arr > 0) & (done > 0)
            if i > 0:
                pl, ps = seq[i - 1]
                pd = W[slot(pl, ps) + 1]
                prev_done = pd[pd > 0].max()
                if 2 <= l < L - 2 and on.any():
                    rows[names[s]].append((np.median(arr[on]) - prev_done, np.median(done[on] - arr[on]),
                                           done[on].max() - prev_done))
                    if s in (0, 2, 3):
                        H = T[:, :nh]
                        ha, hd = H[slot(l, s)], H[slot(l, s) + 1]
                        if (ha > 0).all() and (hd > 0).all():
                            hubs[names[s]].append((ha.max() - prev_done, hd.max() - ha.max(),
                                                   np.median(arr[on]) - hd.max()))
        ha, hd = W[slot(L, 0)], W[slot(L, 0) + 1]
        ld = W[slot(L - 1, 4) + 1]
        on = (ha > 0) & (hd > 0)
        if on.any():
            head.append((np.median(ha[on]) - ld[ld > 0].max(), np.median(hd[on] - ha[on]),
                         hd[on].max() - ld[ld > 0].max()))
    print(f"[lm stages] position {pos}, {reps} steps; us per layer (mean over layers 2..{L - 3}): "
          f"exchange = previous stage's last done -> median arrival, work = median arrival -> done, "
          f"span = previous stage's last done -> last done", file=sys.stderr)
    total = 0.0
    for n in names:
        if not rows[n]:
            continue
        a = np.array(rows[n])
        total += a[:, 2].mean()
        extra = ""
        if hubs.get(n):
            h = np.array(hubs[n])
            extra = (f"   hubs: last producer -> hub holds the input {h[:, 0].mean():5.2f}, image built and flagged "
                     f"{h[:, 1].mean():5.2f}, flag -> median worker {h[:, 2].mean():5.2f}")
        print(f"[lm stages] {n:10s} exchange {a[:, 0].mean():5.2f}  work {a[:, 1].mean():5.2f}  "
              f"span {a[:, 2].mean():5.2f}{extra}", file=sys.stderr)
    print(f"[lm stages] layer total {total:.2f} us", file=sys.stderr)
    if head:
        h = np.array(head)
        print(f"[lm stages] head       exchange {h[:, 0].mean():5.2f}  work {h[:, 1].mean():5.2f}  "
              f"span {h[:, 2].mean():5.2f}", file=sys.stderr)


def lm_schedule(args):
    """The decode schedule a step runs: MING_LM_AUTO takes the XCD-local one
    (4-bit model, attention splits of 384 positions on at most 31 workers of
    one XCD slot) unless MING_LM_XCD=0, else the first persistent one."""
    if args.mode != "auto":
        return args.mode
    fits = args.ctx + args.steps + 1 <= 31 * 384 and os.environ.get("MING_LM_XCD", "1") != "0"
    return "xcd" if fits else "persistent"


def measured_traffic(args):
    """HBM bytes per launch from the committed rocprofv3 counter runs, for
    the workload they were taken on (ctx 2048, each persistent schedule)."""
    name = {"xcd": "decode_xcd_kernel", "persistent": "decode_tagged_kernel"}.get(lm_schedule(args))
    path = os.path.join(ROOT, "profiles", f"{name}_ctx2048_traffic.json")
    if args.ctx != 2048 or name is None or not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f)["traffic_bytes_per_dispatch"]


def profile_traffic(name):
    """HBM bytes per sample of a flow-head workload from its committed
    rocprofv3 counter runs (profiles/<name>_traffic.json), or None."""
    path = os.path.join(ROOT, "profiles", name + "_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f)["traffic_bytes_per_sample"]


def host_threads():
    return int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1)


def cpu_baseline(ming, S, syn, cache, args):
    """Oracle decode steps on the host cores at the same context, for about
    args.cpu_seconds on all threads, then about half that on one thread (at
    least one step each).  The oracle is a scalar C restatement of the MLX CPU
    graph (per-element dequantization in f32, OpenMP over output rows), not an
    optimised CPU decoder."""
    import oracle
    from lmkit import oracle_model, oracle_step

    cfg, layers, norm, head = oracle_model(syn)
    kc, vc = cache.host()

    def run(threads, seconds):
        oracle.set_threads(threads)
        tok, n, t0 = 1234, 0, time.time()
        while True:
            x = oracle.embed(head, tok)
            tok, _, _, _, _ = oracle_step(cfg, layers, norm, head, x, args.ctx, kc, vc)
            n += 1
            if time.time() - t0 >= seconds:
                break
        return n, time.time() - t0

    n, dt = run(host_threads(), args.cpu_seconds)
    cores = oracle.get_threads()
    n1, dt1 = run(1, args.cpu_seconds / 2)
    return {
        "value": round(n / dt, 3),
        "unit": "tokens/s",
        "cores": cores,
        "kind": "port",
        "sample": f"{n} decode tokens of the same 24-layer 4-bit model at ctx {args.ctx} "
                  f"({dt:.1f} s, scalar C restatement of the MLX CPU graph, OpenMP over output rows)",
        "single_core": {"value": round(n1 / dt1, 3), "unit": "tokens/s", "cores": 1,
                        "sample": f"{n1} decode tokens on one thread ({dt1:.1f} s)"},
    }


# ---- multi-request decode ------------------------------------------------------------

METRIC_SERVER = ("multi-request decode tokens/s (config 5: 4-bit LM, paged bf16 KV, ragged ctx 128..4096) "
                 "+ achieved HBM GB/s")


def bench_server(args):
    import numpy as np
    import torch

    ming = importlib.import_module("ming-tts-serve_amd")
    S = importlib.import_module("ming-tts-serve_amd.synthetic")
    spec = S.QWEN2_05B
    n = args.seqs
    ctx = ming.Context(0)
    t0 = time.time()
    syn = S.SyntheticLm(ctx, spec, seed=0, quant=True)
    m = syn.model()
    lens = [int(v) for v in np.random.default_rng(0).integers(128, 4096 + 1, n)]
    pps = (max(lens) + args.warmup + args.steps + 1 + 63) // 64
    batch = ming.LmBatch(m, n, pps * 64)
    pk = S.PagedKv(spec, n, pps, seed=0)
    pk.fill_device(lens, seed=1)
    tok = torch.tensor([int(t) for t in ming.synth_uniform_i32(0, "server.tok", n, spec.vocab)], dtype=torch.int32,
                       device="cuda")
    dit = not args.lm_only
    if dit:
        dspec = S.MING_DIT
        flow = S.SyntheticFlow(ctx, dspec, seed=1, parts=("cfm",))
        cfm = flow.cfm_model()
        dev = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda().view(torch.bfloat16)
        hid = torch.empty((n, spec.hidden), dtype=torch.bfloat16, device="cuda")
        hist = dev(ming.synth_normal_bf16(2, "server.hist", n * dspec.latent)).reshape(n, dspec.latent)
        noise = dev(ming.synth_normal_bf16(3, "server.noise", n * dspec.latent)).reshape(n, dspec.latent)
        sde = dev(ming.synth_normal_bf16(4, "server.sde", n * 10 * dspec.latent)).reshape(n, 10, dspec.latent)
        lat = torch.empty((n, dspec.latent), dtype=torch.bfloat16, device="cuda")
    torch.cuda.synchronize()
    print(f"[bench] server setup {time.time() - t0:.1f}s ({n} sequences, {pps} pages each)", file=sys.stderr,
          flush=True)

    def step():
        if dit:  # the flow head samples each sequence's latent from its hidden state
            batch.step(pk, pk.table, pk.pos, tokens=tok, hidden=hid, argmax=tok)
            cfm.sample_batch(n, hid, hist, noise, sde, 2.0, 0.25, 1.0, lat)
        else:
            batch.step(pk, pk.table, pk.pos, tokens=tok, argmax=tok)

    for _ in range(args.warmup):
        step()
    ctx.sync()
    start = [p + args.warmup for p in lens]
    ms = timed_events(step, args.steps, 0)
    ctx.sync()
    assert pk.pos.cpu().tolist() == [p + args.steps for p in start]
    kv_row = spec.n_layers * 2 * spec.kvd * 2
    fixed = S.lm_bytes_per_token(spec, 0) - kv_row
    mean_ctx = float(np.mean(start)) + (args.steps - 1) / 2.0
    nbytes = int(fixed + n * (mean_ctx + 1) * kv_row)
    if dit:
        nbytes += cfm_bytes_per_sample(S.MING_DIT)
    achieved = nbytes / (ms * 1e-3) / 1e9
    cpu = None
    if not args.no_cpu:
        import oracle
        from lmkit import oracle_model, oracle_step

        oracle.set_threads(int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1))
        cfg, layers, norm, head = oracle_model(syn)
        done, t1, i = 0, time.time(), 0
        while True:  # sequences in turn, each at its own context, one token each
            pos = int(pk.pos[i].item())
            kc, vc = pk.gather(i, pos)
            kcc = np.zeros(kc.shape[:2] + (pos + 1, kc.shape[3]), np.uint16)
            vcc = np.zeros_like(kcc)
            kcc[:, :, :pos], vcc[:, :, :pos] = kc, vc
            oracle_step(cfg, layers, norm, head, oracle.embed(head, int(tok[i].item())), pos, kcc, vcc)
            done += 1
            i = (i + 1) % n
            if time.time() - t1 >= args.cpu_seconds:
                break
        dt = time.time() - t1
        cpu = {"value": round(done / dt, 3), "unit": "tokens/s", "cores": oracle.get_threads(), "kind": "port",
               "sample": f"{done} decode tokens of sequences 0..{min(done, n) - 1} at their own contexts "
                         f"({dt:.1f} s, C restatement of the batch-1 graph, one sequence at a time)"}
    line = base_line(METRIC_SERVER, n * 1000.0 / ms, "tokens/s", args, ms,
                     {"workload": f"{n} concurrent sequences, one decode token each per step, contexts uniform in "
                                  f"[128, 4096] (seed 0, mean {mean_ctx:.0f}) advancing during the run; Qwen2-0.5B "
                                  f"-shaped 24-layer 4-bit LM, paged bf16 KV (64-position pages), greedy argmax" +
                                  ("; DiT flow head per token (10 CFG Euler steps, 8 blocks, hidden 1024, bf16) on "
                                   "every sequence's hidden state" if dit else "; LM only"),
                      "global_batch": n, "seq_len": int(round(mean_ctx))},
                     {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                      "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None, "bytes_per_launch": nbytes,
                      "launch_ms": round(ms, 5)},
                     cpu, "synthetic (random-init N(0,0.02) weights quantized to MLX affine 4-bit/g64; KV N(0,1))",
                     dtype=DTYPE_W4 if not dit else DTYPE_W4 + "; flow head bf16")
    close_all(cfm if dit else None, batch, m, ctx)
    print(json.dumps(line), flush=True)


METRIC_PREFILL = "prompt prefill tokens/s (4-bit LM, causal, paged bf16 KV) + achieved HBM GB/s"


def bench_prefill(args):
    import numpy as np
    import torch

    ming = importlib.import_module("ming-tts-serve_amd")
    S = importlib.import_module("ming-tts-serve_amd.synthetic")
    spec = S.QWEN2_05B
    L = args.prompt
    ctx = ming.Context(0)
    syn = S.SyntheticLm(ctx, spec, seed=0, quant=True)
    m = syn.model()
    pps = (L + 63) // 64
    rows = min(L, 512)  # the prompt in chunks of up to 512 rows
    batch = ming.LmBatch(m, rows, pps * 64)
    pk = S.PagedKv(spec, 1, pps, seed=0)
    ids = ming.synth_uniform_i32(0, "prefill.prompt", L, spec.vocab)
    tok = torch.tensor([int(t) for t in ids], dtype=torch.int32, device="cuda")
    hid = torch.empty((L, spec.hidden), dtype=torch.bfloat16, device="cuda")
    row = pk.table[0].contiguous()
    ms = timed_events(lambda: batch.prefill(pk, row, 0, tokens=tok, hidden=hid), args.steps, args.warmup)
    ctx.sync()
    kv_row = spec.n_layers * 2 * spec.kvd * 2
    chunks = (L + rows - 1) // rows
    nbytes = int(chunks * (S.lm_bytes_per_token(spec, 0) - kv_row) + kv_row * (L * (L + 1) // 2 + L))
    achieved = nbytes / (ms * 1e-3) / 1e9
    cpu = None
    if not args.no_cpu:
        import oracle
        from lmkit import oracle_model, oracle_step

        oracle.set_threads(int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1))
        cfg, layers, norm, head = oracle_model(syn)
        kc = np.zeros((spec.n_layers, spec.kv_heads, L, spec.head_dim), np.uint16)
        vc = np.zeros_like(kc)
        done, t1 = 0, time.time()
        while done < L:  # the oracle prefills row by row (its cache grows like the reference's)
            oracle_step(cfg, layers, norm, head, oracle.embed(head, int(ids[done])), done, kc, vc)
            done += 1
            if time.time() - t1 >= args.cpu_seconds:
                break
        dt = time.time() - t1
        cpu = {"value": round(done / dt, 3), "unit": "tokens/s", "cores": oracle.get_threads(), "kind": "port",
               "sample": f"the first {done} rows of the same prompt, one position at a time ({dt:.1f} s, "
                         f"C restatement of the layer graph)"}
    line = base_line(METRIC_PREFILL, L * 1000.0 / ms, "tokens/s", args, ms,
                     {"workload": f"one {L}-token prompt (uniform ids, seed 0) from position 0 through the 24-layer "
                                  f"4-bit Qwen2-0.5B-shaped LM, causal, paged bf16 KV, {chunks} chunk(s) of <= {rows} rows",
                      "global_batch": 1, "seq_len": L},
                     {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                      "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None, "bytes_per_launch": nbytes,
                      "launch_ms": round(ms, 5)},
                     cpu, "synthetic (random-init N(0,0.02) weights quantized to MLX affine 4-bit/g64)",
                     dtype=DTYPE_W4)
    close_all(batch, m, ctx)
    print(json.dumps(line), flush=True)


C1_PROMPT, C1_STEPS = 64, 128


def c1_bytes_per_step(spec, pos):
    """Algorithmic HBM bytes of one bf16 decode step at position pos: every
    linear and the tied head at 2 B/param, biases and norms, the KV read of
    the pos cached rows and the one-row append."""
    H, I, kvd, L = spec.hidden, spec.inter, spec.kvd, spec.n_layers
    per_layer = H * H * 2 + 2 * kvd * H + 3 * H * I
    small = L * (2 * H + (H + 2 * kvd)) * 2 + H * 2
    kv_row = L * 2 * kvd * 2
    return (per_layer * L + spec.vocab * H) * 2 + small + kv_row * pos + kv_row


def bench_c1(args):
    import numpy as np
    import torch

    ming = importlib.import_module("ming-tts-serve_amd")
    S = importlib.import_module("ming-tts-serve_amd.synthetic")
    spec = S.QWEN2_05B
    ctx = ming.Context(0)
    ctx.set_exclusive(not args.cooperative)
    t0 = time.time()
    syn = S.SyntheticLm(ctx, spec, seed=0, quant=False)
    m = syn.model()
    m.set_mode({"auto": ming.LM_AUTO, "kernels": ming.LM_KERNELS, "persistent": ming.LM_PERSISTENT,
                "direct": ming.LM_PERSISTENT_DIRECT, "xcd": ming.LM_PERSISTENT_XCD}[args.mode])
    ids = [int(t) for t in ming.synth_uniform_i32(0, "c1.prompt", C1_PROMPT, spec.vocab)]
    ptok = torch.tensor(ids, dtype=torch.int32, device="cuda")
    cache = S.KvCache(spec, C1_PROMPT + C1_STEPS)
    toks = torch.zeros(C1_STEPS + 1, dtype=torch.int32, device="cuda")
    print(f"[bench c1] setup {time.time() - t0:.1f}s", file=sys.stderr, flush=True)
    nsteps = C1_PROMPT + C1_STEPS - 1
    # events around every step of the timed jobs (the library launches on torch's current stream)
    ev = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(nsteps)]
          for _ in range(args.steps)]

    def job(evs=None):
        cache.kv.len = 0
        toks[0:1].copy_(ptok[C1_PROMPT - 1:])
        for i in range(nsteps):
            if evs:
                evs[i][0].record()
            if i < C1_PROMPT - 1:  # prompt rows
                m.step(cache.kv, token=ptok[i:i + 1])
            else:  # one greedy step: argmax of step k is the input of step k + 1, on the device
                k = i - (C1_PROMPT - 1)
                m.generate(cache.kv, 1, toks[k:])
            if evs:
                evs[i][1].record()

    for _ in range(args.warmup):
        job()
    torch.cuda.synchronize()
    first = toks.cpu().numpy().copy()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for j in range(args.steps):
        job(ev[j])
    e1.record()
    torch.cuda.synchronize()
    ctx.sync()
    assert cache.len == C1_PROMPT + C1_STEPS - 1
    if args.warmup:
        assert np.array_equal(first, toks.cpu().numpy()), "greedy ids differ between jobs"
    ms = e0.elapsed_time(e1) / args.steps
    per = np.array([[a.elapsed_time(b) for a, b in evj] for evj in ev])  # ms per step launch
    launch_ms = float(per.mean())
    prompt_ms = float(per[:, :C1_PROMPT - 1].sum(axis=1).mean())
    nbytes = sum(c1_bytes_per_step(spec, p) for p in range(nsteps))
    achieved = nbytes / nsteps / (launch_ms * 1e-3) / 1e9
    cpu = None
    if not args.no_cpu:
        import oracle
        from lmkit import oracle_model, oracle_step

        oracle.set_threads(host_threads())
        cfg, layers, norm, head = oracle_model(syn)
        kc = np.zeros((spec.n_layers, spec.kv_heads, C1_PROMPT + C1_STEPS, spec.head_dim), np.uint16)
        vc = np.zeros_like(kc)
        done, feed, t1 = 0, ids[0], time.time()
        while done < C1_PROMPT + C1_STEPS - 1:  # the same job, one position at a time, until the bound
            am, _, _, _, _ = oracle_step(cfg, layers, norm, head, oracle.embed(head, feed), done, kc, vc)
            done += 1
            feed = ids[done] if done < C1_PROMPT else am
            if time.time() - t1 >= args.cpu_seconds:
                break
        dt = time.time() - t1
        cpu = {"value": round(done / dt, 3), "unit": "tokens/s (steps of the job)", "cores": oracle.get_threads(),
               "kind": "port",
               "sample": f"the first {done} of the job's {C1_PROMPT + C1_STEPS - 1} steps (prompt rows, then greedy "
                         f"ids fed back) ({dt:.1f} s, scalar C restatement of the MLX CPU graph, OpenMP over output "
                         f"rows); the GPU's steps/s over the whole job is {(C1_PROMPT + C1_STEPS - 1) * 1000.0 / ms:.1f}"}
    line = base_line(METRIC_C1, C1_STEPS * 1000.0 / ms, "tokens/s", args, ms,
                     {"workload": f"config 1 generate job: bf16 Qwen2-0.5B-shaped LM (24 layers, hidden 896, 14/2 heads, "
                                  f"inter 4864, vocab 151936, tied head), {C1_PROMPT}-token uniform prompt (seed 0) fed "
                                  f"one position at a time, then {C1_STEPS} greedy ids fed back on the device; one job "
                                  f"per step, cache emptied at its start",
                      "global_batch": 1, "seq_len": C1_PROMPT + C1_STEPS,
                      "schedule": args.mode if args.mode != "auto" else
                      f"auto ({'xcd' if os.environ.get('MING_LM_XCD', '1') != '0' else 'persistent'})",
                      "prompt_ms": round(prompt_ms, 3),
                      "greedy_steps_tok_s": round(C1_STEPS * 1000.0 / (ms - prompt_ms), 2),
                      "steps_per_job": C1_PROMPT + C1_STEPS - 1},
                     {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                      "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                      "bytes_per_launch": int(round(nbytes / nsteps)), "launch_ms": round(launch_ms, 5),
                      "bytes_per_job": nbytes},
                     cpu, "synthetic (random-init bf16 weights N(0,0.02), uniform prompt ids)")
    close_all(m, ctx)
    print(json.dumps(line), flush=True)


METRIC_VAE = "VAE decoder latents/s (fc1, 4x upsample, 24-layer sliding-window Qwen2, ISTFT head; f32 graph) + achieved TFLOP/s"
MFMA_F32_PEAK_TFLOPS = 157.3


def vae_flops(spec, T):
    """Algorithmic FLOPs of one decode of T latents: every linear (2 per weight per row), the
    window attention (q.k and p.v over at most `window` keys) and the irfft as a matrix product."""
    F = T * spec.patch
    H, kvd, I = spec.hidden, spec.kvd, spec.inter
    layer = H * H * 2 + 2 * kvd * H + 3 * H * I
    keys = sum(min(i + 1, spec.window) for i in range(F))
    attn = 2 * 2 * keys * spec.heads * spec.head_dim
    return (2 * T * H * spec.latent + 2 * F * layer * spec.n_layers + spec.n_layers * attn
            + 2 * F * (spec.n_fft + 2) * H + 2 * F * (spec.n_fft + 2) * spec.n_fft)


def bench_vae(args):
    import numpy as np
    import torch

    ming = importlib.import_module("ming-tts-serve_amd")
    S = importlib.import_module("ming-tts-serve_amd.synthetic")
    spec, T = S.MING_VAE, args.latents
    ctx = ming.Context(0)
    syn = S.SyntheticVae(ctx, spec, seed=0)
    m = syn.model(T)
    lat = torch.from_numpy(ming.synth_normal_bf16(0, "vae.latents", T * spec.latent).view(np.int16)).cuda().view(
        torch.bfloat16)
    wave = torch.empty(T * spec.patch * spec.hop, dtype=torch.float32, device="cuda")
    ms = timed_events(lambda: m.decode(T, lat, wave), args.steps, args.warmup)
    ctx.sync()
    flops = vae_flops(spec, T)
    achieved = flops / (ms * 1e-3) / 1e12
    cpu = None
    if not args.no_cpu:
        import oracle
        from vaekit import oracle_vae

        oracle.set_threads(int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1))
        om = oracle_vae(syn)
        lat_h = lat.view(torch.int16).cpu().numpy().view(np.uint16).reshape(T, spec.latent)
        chunk, n, t1 = min(T, 8), 0, time.time()
        while time.time() - t1 < args.cpu_seconds:  # fragments of 8 latents until the sample bound
            oracle.vae_decode(om, lat_h[:chunk])
            n += chunk
        dt = time.time() - t1
        cpu = {"value": round(n / dt, 4), "unit": "latents/s", "cores": oracle.get_threads(), "kind": "port",
               "sample": f"{n // chunk} fragments of {chunk} latents ({chunk * spec.patch} frames each) through the "
                         f"same decoder ({dt:.1f} s, C restatement of the f32 graph)"}
    line = base_line(METRIC_VAE, T * 1000.0 / ms, "latents/s", args, ms,
                     {"workload": f"one fragment of {T} latents ({T * spec.patch} frames, "
                                  f"{T * spec.patch * spec.hop / 44100:.2f} s of 44.1 kHz audio) through the VAE "
                                  f"decoder: fc1 64->896, 4x upsample, 24-layer Qwen2-0.5B-shaped stack with a "
                                  f"64-row sliding window, head 896->3530, ISTFT n_fft 3528 / hop 882",
                      "global_batch": 1, "seq_len": T * spec.patch},
                     {"bound": "mfma", "achieved": round(achieved, 2), "peak": MFMA_F32_PEAK_TFLOPS,
                      "unit": "TFLOP/s", "frac": round(achieved / MFMA_F32_PEAK_TFLOPS, 4), "traffic": None,
                      "flops_per_launch": flops, "launch_ms": round(ms, 5)},
                     cpu, "synthetic (random-init N(0,0.02) bf16 weights, periodic Hann window; latents N(0,1))")
    line["dtype"] = "f32"
    close_all(m, ctx)
    print(json.dumps(line), flush=True)


# ---- flow head -----------------------------------------------------------------------

def cfm_bytes_per_sample(spec):
    """bf16 weight bytes one cfmSample reads: per Euler step the blocks, x_emb
    (for y) and the final layer; once c_emb and x_emb (for the history)."""
    D, H, lat = spec.hidden, spec.lm_hidden, spec.latent
    per_step = spec.cfm_blocks * spec.block_params() + D * lat + D + lat * D + lat + D
    once = D * H + D + D * lat
    return 2 * (10 * per_step + once)


def timed_events(fn, steps, warmup):
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def base_line(metric, value, unit, args, ms, config, roofline, cpu, data, dtype="bf16"):
    return {"metric": metric, "value": round(value, 3), "unit": unit, "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": dtype, "data": data, "config": config, "roofline": roofline,
            "cpu_baseline": cpu}


def close_all(*handles):
    """Destroy the library handles in the order given (models before their
    context) while the runtime is whole, instead of at interpreter exit."""
    for h in handles:
        if h is not None:
            h.close()


def gemv_bytes(K, N):
    """Algorithmic bytes of one 4-bit GEMV: u32 nibbles (0.5 B/param), bf16
    scale and bias per group of 64 (0.0625 B/param), the bf16 input row and
    the bf16 output row."""
    return N * K // 2 + N * (K // 64) * 4 + 2 * K + 2 * N


def bench_gemv(args):
    import ctypes

    import numpy as np
    import torch

    ming = importlib.import_module("ming-tts-serve_amd")
    ctx = ming.Context(0)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda().view(torch.bfloat16)
    shapes = GEMV_SHAPES if args.shape < 0 else [GEMV_SHAPES[args.shape]]
    # a device fill long enough for the host to queue every dispatch behind it
    blocker = torch.empty(1 << 30, dtype=torch.int32, device="cuda")
    sweep, head = [], None
    for K, N in shapes:
        nbytes = gemv_bytes(K, N)
        wbytes = N * K // 2 + N * (K // 64) * 4
        R = max(2, -(-int(args.rotate_mb * 2 ** 20) // wbytes))
        w = dev(ming.synth_normal_bf16(1, f"gemv.w.{K}x{N}", N * K, 0.0, 0.02)).reshape(N, K)
        x = dev(ming.synth_normal_bf16(2, f"gemv.x.{K}", K))
        y = torch.empty(N, dtype=torch.bfloat16, device="cuda")
        for g in (1.0, 0.5, 3.0):
            wq = torch.empty((R, N, K // 8), dtype=torch.int32, device="cuda")
            sc = torch.empty((R, N, K // 64), dtype=torch.bfloat16, device="cuda")
            bi = torch.empty((R, N, K // 64), dtype=torch.bfloat16, device="cuda")
            ctx.quantize(w, wq[0], sc[0], bi[0], global_scale=g)
            wq[1:] = wq[0]
            sc[1:] = sc[0]
            bi[1:] = bi[0]
            tx, ty = ming.tensor(x), ming.tensor(y)
            refs = [(ctypes.byref(ming.tensor(wq[r], ming.DT_U32)), ctypes.byref(ming.tensor(sc[r])),
                     ctypes.byref(ming.tensor(bi[r]))) for r in range(R)]
            f, h = ctx.L.ming_qgemv, ctx.h

            def run(n, start=0):
                for i in range(n):
                    a = refs[(start + i) % R]
                    st = f(h, ctypes.byref(tx), a[0], a[1], a[2], ctypes.c_float(g), 64, 4, ctypes.byref(ty))
                    if st:
                        ctx.check(st)

            # the warm-up reads copies the timed dispatches come to last (or, with fewer copies than
            # dispatches, a cycle longer than the MALL), so no timed read is a cache hit
            nwarm = min(R, max(args.warmup, 1))
            run(nwarm, start=R - nwarm)
            torch.cuda.synchronize()
            b0, b1, e1 = (torch.cuda.Event(enable_timing=True) for _ in range(3))
            b0.record()
            for _ in range(4):
                blocker.fill_(7)
            b1.record()
            t0 = time.perf_counter()
            run(args.steps)
            host_s = time.perf_counter() - t0
            e1.record()
            torch.cuda.synchronize()
            ctx.sync()
            ms = b1.elapsed_time(e1) / args.steps
            blocked_ms = b0.elapsed_time(b1)
            gbs = nbytes / (ms * 1e-3) / 1e9
            ent = {"in": K, "out": N, "global_scale": g, "us": round(ms * 1e3, 3), "GB/s": round(gbs, 1),
                   "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes": nbytes, "copies": R,
                   "host_bound": host_s * 1e3 > blocked_ms}
            sweep.append(ent)
            print(f"[gemv] [{K}x{N}] g={g}: {ent['us']} us/dispatch, {ent['GB/s']} GB/s "
                  f"({100 * ent['frac']:.1f}% of HBM), {R} copies, host {host_s * 1e3:.2f} ms vs blocker "
                  f"{blocked_ms:.2f} ms", file=sys.stderr, flush=True)
            if (K, N) == (896, 151936) and g == 1.0:
                head = ent
            del wq, sc, bi, refs
        del w, x, y
    if head is None:
        head = sweep[0]
    cpu = None
    if not args.no_cpu:
        import oracle

        oracle.set_threads(host_threads())
        K, N = head["in"], head["out"]
        w = ming.synth_normal_bf16(1, f"gemv.w.{K}x{N}", N * K, 0.0, 0.02).reshape(N, K)
        wq, s_, b_ = oracle.quantize(w)
        L = oracle.Linear(wq, s_, b_)
        xh = ming.synth_normal_bf16(2, f"gemv.x.{K}", K)
        n, t0 = 0, time.time()
        while True:
            oracle.linear(L, xh)
            n += 1
            if time.time() - t0 >= min(args.cpu_seconds, 10.0):
                break
        dt = time.time() - t0
        cpu = {"value": round(gemv_bytes(K, N) * n / dt / 1e9, 3), "unit": "GB/s", "cores": oracle.get_threads(),
               "kind": "port", "sample": f"{n} GEMVs [{K}x{N}] ({dt:.1f} s, C restatement: per-element dequant, "
                                         f"f32 accumulate, OpenMP over output rows)"}
    line = base_line(METRIC_GEMV, head["GB/s"], "GB/s", args, head["us"] * 1e-3,
                     {"workload": f"4-bit GEMV [{head['in']}x{head['out']}] at g = {head['global_scale']}, one "
                                  f"dispatch per step over {head['copies']} weight copies (> {args.rotate_mb:.0f} MB)",
                      "weights": "MLX affine u32 4-bit, group 64, bf16 scales/biases, fp32 global scale",
                      "shapes": [f"{k}x{n}" for k, n in shapes], "global_batch": 1, "seq_len": 1},
                     {"bound": "hbm", "achieved": head["GB/s"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                      "frac": head["frac"], "traffic": None, "bytes_per_launch": head["bytes"],
                      "launch_ms": round(head["us"] * 1e-3, 6)},
                     cpu, "synthetic (N(0,0.02) weights quantized on the GPU; x N(0,1))", dtype=DTYPE_W4)
    line["sweep"] = sweep
    close_all(ctx)
    print(json.dumps(line), flush=True)


def bench_dit(args):
    import ctypes

    import numpy as np
    import torch

    ming = importlib.import_module("ming-tts-serve_amd")
    S = importlib.import_module("ming-tts-serve_amd.synthetic")
    spec = S.MING_DIT
    ctx = ming.Context(0)
    flow = S.SyntheticFlow(ctx, spec, seed=1)
    D, F, B, L = spec.hidden, spec.ff, 2, 3
    R = B * L
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda().view(torch.bfloat16)
    x = dev(ming.synth_normal_bf16(1, "bench.dit.x", R * D)).reshape(R, D)
    half = spec.head_dim // 2
    cos = torch.empty((L, half), dtype=torch.float32, device="cuda")
    sin = torch.empty((L, half), dtype=torch.float32, device="cuda")
    ctx.rotary_table(spec.inv_freq(), L, cos, sin)
    bf = lambda *sh: torch.empty(sh, dtype=torch.bfloat16, device="cuda")
    out = dict(qkv=bf(3, R, D), att=bf(R, D), x1=bf(R, D), hh=bf(R, F), x2=bf(R, D))
    o = ming.DitOut(*(out[k].data_ptr() for k in ("qkv", "att", "x1", "hh", "x2")))
    cfg = spec.cfg()
    ctx.dit_block(cfg, flow.cfm_blocks[0], x, B, L, cos, sin, o)  # the inputs of stages B and D
    ctx.sync()
    qkv_tmp, res = bf(3, R, D), bf(R * max(D, F))
    src = flow.cfm_blocks[0]
    pre = "flowloss.cfm.model.blocks.0"
    lins = {0: (("wq", "attn.to_q"), ("wk", "attn.to_k"), ("wv", "attn.to_v")), 1: (("wo", "attn.to_out.0"),),
            2: (("w1", "mlp.ff.0.0"),), 3: (("w2", "mlp.ff.2"),)}
    inp = {0: None, 1: out["att"], 2: None, 3: out["hh"]}
    xin = {0: x, 1: x, 2: out["x1"], 3: out["x1"]}
    wbytes = {0: 3 * (D * D + D) * 2 + D * 2, 1: (D * D + D) * 2, 2: (F * D + F) * 2 + D * 2, 3: (D * F + D) * 2}
    names = {0: "A q/k/v + attention", 1: "B out_proj + residual", 2: "C ff1 + gelu", 3: "D ff2 + residual"}
    blocker = torch.empty(1 << 30, dtype=torch.int32, device="cuda")
    f, h = ctx.L.ming_dit_single, ctx.h
    stages, tot_b, tot_us = [], 0, 0.0
    for ki in range(4):
        # copies of this kernel's weight matrices (block 0's values) totalling > --rotate-mb
        nrot = max(2, -(-int(args.rotate_mb * 2 ** 20) // wbytes[ki]))
        big = {fld: flow.dev[f"{pre}.{key}.weight"].unsqueeze(0).repeat(nrot, 1, 1) for fld, key in lins[ki]}
        blocks = []
        for r in range(nrot):
            nb = ming.DitBlockW.from_buffer_copy(src)
            for fld, _ in lins[ki]:
                setattr(nb, fld, ming.linear(big[fld][r]))
            blocks.append(nb)
        args_k = [(h, ki, ctypes.byref(cfg), ctypes.byref(blocks[i]), ming.ptr(xin[ki]), ming.ptr(inp[ki]), B, L,
                   ming.ptr(cos), ming.ptr(sin), ming.ptr(qkv_tmp), ming.ptr(res)) for i in range(len(blocks))]

        def run(n):
            for i in range(n):
                st = f(*args_k[i % len(blocks)])
                if st:
                    ctx.check(st)

        run(args.warmup)
        torch.cuda.synchronize()
        b0, b1, e1 = (torch.cuda.Event(enable_timing=True) for _ in range(3))
        b0.record()
        for _ in range(8):
            blocker.fill_(ki)
        b1.record()
        t0 = time.perf_counter()
        run(args.steps)
        host_s = time.perf_counter() - t0
        e1.record()
        torch.cuda.synchronize()
        ctx.sync()
        us = b1.elapsed_time(e1) * 1e3 / args.steps
        gbs = wbytes[ki] / (us * 1e-6) / 1e9
        stages.append({"kernel": names[ki], "us": round(us, 3), "weight_bytes": wbytes[ki], "GB/s": round(gbs, 1),
                       "frac": round(gbs / HBM_PEAK_GBS, 4), "copies": nrot,
                       "host_bound": host_s * 1e3 > b0.elapsed_time(b1)})
        del big, blocks, args_k
        tot_b += wbytes[ki]
        tot_us += us
        print(f"[dit] {names[ki]}: {us:.2f} us/dispatch, {gbs:.1f} GB/s ({100 * gbs / HBM_PEAK_GBS:.1f}% of HBM)",
              file=sys.stderr, flush=True)
    achieved = tot_b / (tot_us * 1e-6) / 1e9
    line = base_line(METRIC_DIT, achieved, "GB/s", args, tot_us * 1e-3,
                     {"workload": "the four DiT block kernels of the flow head at the reference shape (R = 2 x 3 "
                                  "rows, hidden 1024, 16 x 64 heads, ff 4096), one dispatch of each per step, "
                                  f"each cycling through copies of its weights totalling > {args.rotate_mb:.0f} MB",
                      "global_batch": 1, "seq_len": L},
                     {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                      "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None, "bytes_per_launch": tot_b,
                      "launch_ms": round(tot_us * 1e-3, 6)},
                     None, "synthetic (random-init N(0,0.02) bf16 DiT weights; x N(0,1))")
    line["stages"] = stages
    close_all(ctx)
    print(json.dumps(line), flush=True)


def bench_cfm(args):
    import numpy as np
    import torch

    ming = importlib.import_module("ming-tts-serve_amd")
    S = importlib.import_module("ming-tts-serve_amd.synthetic")
    spec = S.MING_DIT
    ctx = ming.Context(0)
    if not args.cooperative:
        ctx.set_exclusive(True)  # the bench holds the device: the persistent flow head launches ordinarily
    flow = S.SyntheticFlow(ctx, spec, seed=1, parts=("cfm",))
    mode = {"auto": ming.CFM_AUTO, "kernels": ming.CFM_KERNELS, "persistent": ming.CFM_PERSISTENT}.get(
        args.mode, ming.CFM_AUTO)
    m = flow.cfm_model()
    try:  # does the persistent kernel fit this device (AUTO takes it where it does)?
        m.set_mode(ming.CFM_PERSISTENT)
        fits = True
    except ming.MingError:
        fits = False
    m.set_mode(mode)
    persistent = mode == ming.CFM_PERSISTENT or (mode == ming.CFM_AUTO and fits)
    others = []  # further weight sets, cycled sample by sample
    for i in range(1, max(1, args.weight_sets)):
        f = S.SyntheticFlow(ctx, spec, seed=1 + i, parts=("cfm",))
        others.append((f, f.cfm_model()))
        others[-1][1].set_mode(mode)
    models = [m] + [o[1] for o in others]
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda().view(torch.bfloat16)
    host = {k: ming.synth_normal_bf16(s, "bench." + k, n) for k, s, n in
            (("z", 1, spec.lm_hidden), ("hist", 2, spec.latent), ("noise", 3, spec.latent), ("sde", 4, 10 * spec.latent))}
    z, hist, noise, sde = (dev(host[k]) for k in ("z", "hist", "noise", "sde"))
    out = torch.empty(spec.latent, dtype=torch.bfloat16, device="cuda")
    turn = [0]

    def one():
        models[turn[0] % len(models)].sample(z, hist, noise, sde, 2.0, 0.25, 0.0, out)
        turn[0] += 1

    ms = timed_events(one, args.steps, args.warmup)
    if args.stamps and args.mode == "persistent":
        cfm_stage_report(ctx, m, spec, lambda: m.sample(z, hist, noise, sde, 2.0, 0.25, 0.0, out))
    nbytes = cfm_bytes_per_sample(spec)
    achieved = nbytes / (ms * 1e-3) / 1e9
    cpu = None
    if not args.no_cpu:
        import oracle
        from ditkit import oracle_cfm

        oracle.set_threads(int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1))
        oc = oracle_cfm(flow)
        n, t0 = 0, time.time()
        while True:
            oracle.cfm_sample(oc, host["z"], host["hist"], host["noise"], host["sde"].reshape(10, -1), 2.0, 0.0)
            n += 1
            if time.time() - t0 >= args.cpu_seconds:
                break
        dt = time.time() - t0
        cpu = {"value": round(n / dt, 4), "unit": "samples/s", "cores": oracle.get_threads(), "kind": "port",
               "sample": f"{n} flow-head samples of the same weights ({dt:.1f} s, C restatement of the MLX graph)"}
    line = base_line(METRIC_CFM, 1000.0 / ms, "samples/s", args, ms,
                     {"workload": "flow head of one token: 10 CFG Euler steps through 8 DiT blocks (hidden 1024, "
                                  "16x64 heads, ff 4096), rows 2 halves x 3 positions", "global_batch": 1, "seq_len": 3,
                      "weight_sets": len(models)},
                     {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                      "frac": round(achieved / HBM_PEAK_GBS, 4),
                      "traffic": profile_traffic("cfm_persistent_ref_shape") if persistent else None,
                      "bytes_per_launch": nbytes, "launch_ms": round(ms, 5)},
                     cpu, "synthetic (random-init N(0,0.02) bf16 DiT weights; z, history, noise N(0,1))")
    close_all(*models, ctx)
    print(json.dumps(line), flush=True)


def cfm_stage_report(ctx, m, spec, run):
    """Per-stage timing of the persistent flow head (ming_cfm_model_profile
    stamps of the first worker over 5 samples, medians), printed to stderr:
    for each of a block's four stage images, the wait from the worker's own
    outputs of the stage before to its slice's inputs (hand-off), its slice
    work, the wait for every slice of the image plus the copy into LDS
    (deliver), and the stage's compute up to its outputs."""
    import numpy as np
    import torch

    nb, steps = spec.cfm_blocks, 10
    nflag = steps * nb * 4
    st = torch.zeros((6, nflag), dtype=torch.int64, device="cuda")
    res = []
    for _ in range(5):
        st.zero_()
        m.profile(st)
        run()
        ctx.sync()
        m.profile(None)
        res.append(st.cpu().numpy().astype(np.float64) / 100.0)  # wall_clock64 ticks at 100 MHz -> us
    a = np.median(np.stack(res), axis=0)
    pub, got, sent, recvd, fin = a[0], a[1], a[2], a[3], a[4]
    names = ("rms1 rows -> q/k/v", "attention rows -> out_proj", "rms2 rows -> ff1", "ff1 rows -> ff2")
    print("[cfm stages] image k of a block, first worker: its outputs of the stage before -> its slice's inputs "
          "(hand-off) -> its slice published (slice) -> every slice, image in LDS (deliver) -> its outputs (compute); "
          "us, median of 5 samples, mean over blocks", file=sys.stderr)
    total = 0.0
    for k in range(4):
        idx = np.array([(s * nb + b) * 4 + k for s in range(steps) for b in range(nb) if k > 0 or b > 0])
        h, sl, d, c = recvd[idx] - sent[idx - 1], pub[idx] - recvd[idx], got[idx] - pub[idx], sent[idx] - got[idx]
        total += h.mean() + sl.mean() + d.mean() + c.mean()
        print(f"[cfm stages] {names[k]:28s} hand-off {h.mean():5.2f}  slice {sl.mean():5.2f}  deliver {d.mean():5.2f}"
              f"  compute {c.mean():5.2f}", file=sys.stderr)
    head = [got[((s + 1) * nb) * 4] - sent[(s * nb + nb - 1) * 4 + 3] for s in range(steps - 1)]
    print(f"[cfm stages] per block {total:.2f} us; a step's last ff2 outputs -> the next step's first image in LDS "
          f"(final layer, embed) {np.mean(head):.2f} us; first image -> last final layer {fin[steps - 1] - got[0]:.1f} us",
          file=sys.stderr)


def bench_c4(args):
    import numpy as np
    import torch

    ming = importlib.import_module("ming-tts-serve_amd")
    S = importlib.import_module("ming-tts-serve_amd.synthetic")
    spec = S.MING_ADALN
    ctx = ming.Context(0)
    syn = S.SyntheticAdaln(ctx, spec, seed=1)
    m = syn.model()
    F, lat = spec.frames, spec.latent
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda().view(torch.bfloat16)
    host = {k: ming.synth_normal_bf16(s, "bench." + k, n) for k, s, n in
            (("z", 1, spec.lm_hidden), ("noise", 3, F * lat), ("sde", 4, 10 * F * lat))}
    z, noise, sde = (dev(host[k]) for k in ("z", "noise", "sde"))
    out = torch.empty((F, lat), dtype=torch.bfloat16, device="cuda")
    ms = timed_events(lambda: m.sample(z, noise, sde, 2.0, 0.25, 0.0, out), args.steps, args.warmup)
    nbytes = spec.sample_weight_bytes()
    achieved = nbytes / (ms * 1e-3) / 1e9
    cpu = None
    if not args.no_cpu:
        import oracle
        from ditkit import oracle_adaln

        oracle.set_threads(int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1))
        om = oracle_adaln(syn)
        n, t0 = 0, time.time()
        while True:
            oracle.adaln_sample(om, host["z"], host["noise"].reshape(F, lat), host["sde"].reshape(10, F, lat), 2.0,
                                0.0)
            n += 1
            if time.time() - t0 >= args.cpu_seconds:
                break
        dt = time.time() - t0
        cpu = {"value": round(n / dt, 4), "unit": "samples/s", "cores": oracle.get_threads(), "kind": "port",
               "sample": f"{n} adaLN flow-head samples of the same weights ({dt:.1f} s, C restatement)"}
    line = base_line(METRIC_C4, 1000.0 / ms, "samples/s", args, ms,
                     {"workload": "config 4 adaLN flow head: 4 DiT blocks (hidden 896, 14x64 heads, ff 3584) with "
                                  "adaLN-Zero modulation from silu(t_emb + c_emb(z)), a 4-frame x 64 patch, "
                                  "10 CFG Euler steps, rows 2 halves x 4 frames", "global_batch": 1, "seq_len": F},
                     {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                      "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": profile_traffic("adaln_c4_flow_head"),
                      "bytes_per_launch": nbytes, "launch_ms": round(ms, 5)},
                     cpu, "synthetic (random-init N(0,0.02) bf16 weights; z, noise N(0,1))")
    close_all(m, ctx)
    print(json.dumps(line), flush=True)


# ---- whole per-token loop ------------------------------------------------------------

def bench_loop(args):
    import numpy as np
    import torch

    ming = importlib.import_module("ming-tts-serve_amd")
    S = importlib.import_module("ming-tts-serve_amd.synthetic")
    lspec, dspec = S.QWEN2_05B, S.MING_DIT
    ctx = ming.Context(0)
    ctx.set_exclusive(not args.cooperative)
    lm = S.SyntheticLm(ctx, lspec, seed=0, quant=True)
    lmm = lm.model()
    flow = S.SyntheticFlow(ctx, dspec, seed=1)
    cfm, agg = flow.cfm_model(), flow.agg_model()
    H, lat, L = lspec.hidden, dspec.latent, 16
    K = max(2, args.steps)
    never = torch.tensor([20.0, 0.0], dtype=torch.bfloat16, device="cuda")  # stop bias: the loop runs K steps
    emb = torch.from_numpy(ming.synth_normal_bf16(5, "bench.embeds", L * H, 0.0, 0.5).view(np.int16).reshape(L, H))
    emb = emb.cuda().view(torch.bfloat16)
    bank = torch.empty((K, 11, lat), dtype=torch.bfloat16, device="cuda")
    ctx.noise_bank(7, K, lat, bank)
    lats = torch.empty((K, lat), dtype=torch.bfloat16, device="cuda")

    def run(n):
        cache = S.KvCache(lspec, L + n + 2)
        torch.cuda.synchronize()
        t = time.perf_counter()
        done, _ = ctx.sample_latents(lmm, cfm, agg, flow.lin_w("stop_head"), never, emb, cache.kv, bank,
                                     ming.SampleParams(n, 2.0, 0.25, 0.0), lats)
        dt = time.perf_counter() - t
        ctx.sync()  # a device wait that gave up fails the run instead of timing it
        return dt, done

    for _ in range(max(1, args.warmup // 10)):
        run(2)
    t1, _ = run(1)
    tk, done = run(K)
    ms = (tk - t1) / (done - 1) * 1e3
    lm_bytes = S.lm_bytes_per_token(lspec, L + K // 2) - lspec.vocab * lspec.hidden * 0.5625  # no head in the loop
    nbytes = int(lm_bytes + cfm_bytes_per_sample(dspec) + 2 * (dspec.agg_blocks * dspec.block_params() +
                 dspec.hidden * lat + dspec.hidden * H + 3 * dspec.hidden + H) + 2 * (2 * H + 2))
    achieved = nbytes / (ms * 1e-3) / 1e9
    cpu = None
    if not args.no_cpu:
        cpu = loop_cpu_baseline(ming, lm, flow, args)
    line = base_line(METRIC_LOOP, 1000.0 / ms, "tokens/s", args, ms,
                     {"workload": f"one sampleLatents step after a {L}-row prompt: flow head (8 blocks x 10 Euler "
                                  "steps), aggregator (8 blocks), Qwen2-0.5B-shaped 24-layer 4-bit LM decode "
                                  "(hidden only), stop head", "global_batch": 1, "seq_len": L + K,
                      "launch": "cooperative" if args.cooperative else "ordinary (device held by this process alone)"},
                     {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                      "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None, "bytes_per_launch": nbytes,
                      "launch_ms": round(ms, 5)},
                     cpu, "synthetic (random-init N(0,0.02) weights, LM quantized to MLX affine 4-bit/g64; "
                          "prompt rows N(0,0.25); noise bank N(0,1))")
    # one whole call with one step: workspace set-up, the prompt's prefill, the first latent
    line["first_latent_ms"] = round(t1 * 1e3, 3)
    line["dtype"] = DTYPE_W4 + "; flow head and aggregator bf16"
    close_all(cfm, agg, lmm, ctx)
    print(json.dumps(line), flush=True)


def loop_cpu_baseline(ming, lm, flow, args):
    """The oracle's per-token work (stop head, flow head, aggregator, LM
    decode step) on the host cores, for about args.cpu_seconds (>= 1 token)."""
    import numpy as np

    import oracle
    from ditkit import oracle_agg, oracle_cfm
    from lmkit import oracle_model, oracle_step

    oracle.set_threads(int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1))
    cfg, layers, norm, head = oracle_model(lm)
    oc, oa = oracle_cfm(flow), oracle_agg(flow)
    stop = oracle.Linear(flow.hostw["stop_head.weight"])
    H, lat = lm.spec.hidden, flow.spec.latent
    kc = np.zeros((lm.spec.n_layers, lm.spec.kv_heads, 64, lm.spec.head_dim), np.uint16)
    vc = np.zeros_like(kc)
    z = ming.synth_normal_bf16(9, "bench.z", H)
    hist = np.zeros(lat, np.uint16)
    noise = ming.synth_normal_bf16(10, "bench.noise", 11 * lat).reshape(11, lat)
    n, t0 = 0, time.time()
    while n < 60:
        oracle.stop_prob(stop, flow.hostw["stop_head.bias"], z)
        latent, _ = oracle.cfm_sample(oc, z, hist, noise[0], noise[1:], 2.0, 0.0)
        x = oracle.aggregate(oa, latent)
        _, z, _, _, _ = oracle_step(cfg, layers, norm, head, x, n, kc, vc)
        hist = latent
        n += 1
        if time.time() - t0 >= args.cpu_seconds:
            break
    dt = time.time() - t0
    return {"value": round(n / dt, 4), "unit": "tokens/s", "cores": oracle.get_threads(), "kind": "port",
            "sample": f"{n} TTS tokens of the same models ({dt:.1f} s; the oracle's LM step includes its head)"}


if __name__ == "__main__":
    main()
