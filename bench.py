"""Benchmark: paged decode attention + KV append on one MI355X.

A step is one decode step of the BASELINE.json north-star workload
(configs[2], Llama-3-8B shape): for each of the 32 layers, every one of the
256 sequences appends its new K/V token and attends over its whole context
(seq_len + 1 keys) -- one pkv_decode_attention launch per layer.  Inputs are
resident in HBM before the timed region.

Prints ONE JSON line (rank 0).  `value` = tokens/s = batch / step time;
`roofline` = the decode kernel's algorithmic bytes per launch over its
average launch duration (HIP events on the launch stream) against the 8 TB/s
HBM peak; `cpu_baseline` = the oracle's CPU restatement of the reference
decode math timed on this host on a bounded sample (see --cpu-layers).
"""
from __future__ import annotations

import argparse
import ctypes
import dataclasses
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.join(ROOT, "ai-engine_amd"), os.path.join(ROOT, "oracle")]

METRIC = "decode attn+KV-append tokens/s and achieved HBM GB/s, Llama-3-8B shape, 1 GPU"
HBM_PEAK_GBPS = 8000.0
# GPU against CPU agreement of attention outputs: north star's fp32 tolerance
TOLERANCE = {"abs": 1e-3, "rel": 2e-3}


def agreement(gpu, ref):
    """(every |gpu - ref| <= abs + rel |ref|, the largest |gpu - ref| / bound)."""
    import numpy as np
    gpu = np.asarray(gpu, np.float64)
    ref = np.asarray(ref, np.float64)
    bound = TOLERANCE["abs"] + TOLERANCE["rel"] * np.abs(ref)
    worst = float(np.max(np.abs(gpu - ref) / bound)) if ref.size else 0.0
    return bool(worst <= 1.0), worst

CONFIGS = {
    # name: (shape attr, batch, ctx_lo, ctx_hi, description)
    "cfg1": ("CFG1", 8, 128, 1024, "Llama-3.2-1B decode: 16 layers, 32q/8kv heads, hd 64, bs 16, "
             "f16 KV, B=8, ctx U[128,1024], 2048 blocks/layer"),
    "cfg2d": ("CFG2", 56, 256, 2048, "TinyLlama-1.1B decode part: 22 layers, 32q/4kv heads, hd 64, "
              "bs 16, f16 KV, B=56, ctx U[256,2048]"),
    "cfg3": ("CFG3", 256, 512, 4096, "Llama-3-8B decode: 32 layers, 32q/8kv heads, hd 128, bs 16, "
             "bf16 KV, B=256, ctx U[512,4096], pool 1.2x live tokens"),
    "cfg4": ("CFG4", 128, 2048, 8192, "Llama-3-70B layers 0-39: 40 layers, 64q/8kv heads, hd 128, "
             "bs 16, bf16 KV, B=128, ctx U[2048,8192], pool 1.2x live tokens"),
}


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def host_cpu() -> dict:
    """The host the CPU baseline ran on: model name, logical CPUs of the
    machine and the CPUs this process may run on."""
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
    return {"cpu_model": model, "nproc": os.cpu_count() or 1, "usable_cpus": usable}


def timed_passes(fn, args):
    """Runs fn() at least args.cpu_layers times and for at least
    args.cpu_seconds; returns (seconds per pass, passes, last result)."""
    n, res, t0 = 0, None, time.time()
    while n < max(1, args.cpu_layers) or (time.time() - t0 < args.cpu_seconds and n < 100000):
        res = fn()
        n += 1
    return (time.time() - t0) / n, n, res


def copy_ceiling(dev, cache=None, used=None, gib: int = 2, reps: int = 10) -> dict:
    """The HBM copy ceiling on this GPU: the faster of a plain device-to-device
    copy of `gib` GiB (torch copy_, i.e. hipMemcpyAsync) and, given a pool,
    the library's block-copy kernel moving up to 1,024 blocks (all layers,
    K and V) from the blocks in `used` into blocks no table references.
    Both move far more than the 256 MB Infinity Cache; read + written bytes
    over the average time, HIP events."""
    import numpy as np
    import torch
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def timed(fn):
        for _ in range(2):
            fn()
        torch.cuda.synchronize()
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    n = (gib << 30) // 4
    src = torch.ones(n, dtype=torch.int32, device=dev)
    dst = torch.empty_like(src)
    ms = timed(lambda: dst.copy_(src))
    del src, dst
    torch.cuda.empty_cache()
    res = {"GBps": round(2 * (gib << 30) / (ms / 1e3) / 1e9, 1),
           "method": f"torch copy_ of {gib} GiB (read + write counted), {reps} reps"}
    if cache is not None:
        # random (seeded) sources and destinations, as the block churn uses:
        # a copy between two ranges at a constant offset streams slower
        # (5.0 against 6.1 TB/s measured), so it would understate the ceiling
        used = np.unique(np.asarray(used, np.int32))
        free = np.setdiff1d(np.arange(cache.num_blocks, dtype=np.int32), used)
        m = int(min(1024, free.size, used.size))
        if m > 0:
            rng = np.random.default_rng(7)
            s_t = torch.from_numpy(rng.permutation(used)[:m].astype(np.int32)).to(dev)
            d_t = torch.from_numpy(rng.permutation(free)[:m].astype(np.int32)).to(dev)
            ms_b = timed(lambda: cache.copy_blocks(s_t, d_t))
            moved = 2 * m * cache.block_bytes * 2 * cache.n_layers
            gbps_b = moved / (ms_b / 1e3) / 1e9
            res["copy_blocks_GBps"] = round(gbps_b, 1)
            res["torch_copy_GBps"] = res["GBps"]
            res["method"] = (f"max of torch copy_ of {gib} GiB and pkv_copy_blocks of {m} random "
                             f"blocks x {cache.n_layers} layers K+V into random free blocks "
                             f"({moved / 1e9:.2f} GB moved), read + write counted, {reps} reps")
            res["GBps"] = round(max(res["GBps"], gbps_b), 1)
    return res


def read_ceiling(dev, cache, used, reps: int = 10) -> dict:
    """The read ceiling of the decode's own access pattern: pkv_pool_read_blocks
    streams every block the tables reference (32 KiB per layer's K or V for
    the Llama-3-8B shape, in random pool order, every layer) with nothing
    else to do; bytes read over the average time, HIP events.  A read-only
    kernel such as decode is bounded by this rate, where a copy (read +
    write) is not."""
    import numpy as np
    import torch
    blocks = torch.from_numpy(np.unique(np.asarray(used, np.int32))).to(dev)
    acc = torch.zeros(1, dtype=torch.int64, device=dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for _ in range(2):
        cache.read_blocks(blocks, out=acc)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(reps):
        cache.read_blocks(blocks, out=acc)
    e1.record()
    torch.cuda.synchronize()
    cache.check()
    ms = e0.elapsed_time(e1) / reps
    nbytes = int(blocks.numel()) * cache.block_bytes * 2 * cache.n_layers
    return {"GBps": round(nbytes / (ms / 1e3) / 1e9, 1),
            "method": (f"pkv_pool_read_blocks of the {blocks.numel()} blocks the tables reference, "
                       f"{cache.n_layers} layers K+V ({nbytes / 1e9:.2f} GB read), {reps} reps"),
            "kernel": "pkv::read_blocks_kernel", "kernel_avg_us": round(ms * 1e3, 1)}


def timed_steps(step, n, stream):
    """Times n calls of step(i) on `stream` with a HIP event at every step
    boundary: returns (mean ms per step, {median, p10, p90} of the steps)."""
    import numpy as np
    import torch
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(n + 1)]
    torch.cuda.synchronize()
    marks[0].record(stream)
    for i in range(n):
        step(i)
        marks[i + 1].record(stream)
    torch.cuda.synchronize()
    per = np.array([marks[i].elapsed_time(marks[i + 1]) for i in range(n)])
    dist = {"median": round(float(np.median(per)), 4),
            "p10": round(float(np.percentile(per, 10)), 4),
            "p90": round(float(np.percentile(per, 90)), 4)}
    return marks[0].elapsed_time(marks[n]) / n, dist


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="cfg3",
                    choices=sorted(CONFIGS) + ["cfg2", "cfg5", "sample", "gather", "append"])
    ap.add_argument("--rope", action="store_true",
                    help="decode configs and cfg2: q and the new k/v arrive in f32 before the "
                         "rotary embedding, which the decode kernel applies "
                         "(pkv_decode_attention_rope) and the chunk store applies to k and q "
                         "(pkv_append_rope)")
    ap.add_argument("--serial", action="store_true",
                    help="cfg2: time eager launches on one stream only (default: the step as "
                         "a HIP graph with each layer's decode on a second stream)")
    ap.add_argument("--unfused", action="store_true",
                    help="cfg2: store the chunk's K/V with a separate pkv_append launch")
    ap.add_argument("--separate", action="store_true",
                    help="cfg2: separate prefill and decode launches per layer (default: one "
                         "pkv_mixed_attention launch per layer)")
    ap.add_argument("--kv-dtype", choices=["f32", "f16", "bf16"], default=None,
                    help="decode configs: pool dtype instead of the config's (f32 is the "
                         "reference's KvPool dtype)")
    ap.add_argument("--logits", choices=["bf16", "f32"], default="bf16",
                    help="sample: the logits' dtype (f32: genuine f32 values, which take the "
                         "bucket kernel; bf16: the runs of equal 16-bit values)")
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--cpu-layers", type=int, default=2,
                    help="minimum layer passes of the CPU baseline sample (0 = skip it)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="the CPU baseline repeats its sample for at least this long")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--replicas", type=int, default=0,
                    help="pool replicas rotated across steps so that every step reads its K/V "
                         "from HBM, not the 256 MB Infinity Cache (0 = auto: >= 1 GB per "
                         "rotation)")
    ap.add_argument("--no-secondary", dest="secondary", action="store_false",
                    help="cfg3: skip the in-process runs of cfg1, cfg2, cfg4, cfg5, append "
                         "and sample_f32 reported under 'secondary' in the same line")
    ap.add_argument("--graph", choices=["auto", "on", "off"], default="auto",
                    help="replay each step as a captured HIP graph (auto: when a layer's "
                         "launch moves < 128 MB, i.e. launch overhead would show)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build runs on one GPU only: the paged-KV path has no "
                                   "inter-GPU exchange here (sequences or kv heads would "
                                   "shard across GPUs with no exchange; not built); "
                                   "run with --gpus 1"}))
        return 2

    import numpy as np
    import torch

    import pagedkv
    from pagedkv import workload as wl

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        return 1
    dev = torch.device("cuda", 0)
    if args.config == "cfg5":
        return emit(churn(args, dev))
    if args.config == "cfg2":
        return emit(mix(args, dev))
    if args.config == "sample":
        return emit(sample_bench(args, dev))
    if args.config == "gather":
        return gather_bench(args, dev)
    if args.config == "append":
        return emit(append_bench(args, dev))
    res = decode_bench(args, dev)
    if (args.config == "cfg3" and args.secondary and "error" not in res
            and not (args.rope or args.kv_dtype)):
        res["secondary"] = secondary(args, dev)
    return emit(res)


def emit(res: dict) -> int:
    """Prints the one result line; exit status 1 when it carries an error."""
    print(json.dumps(res), flush=True)
    return 1 if "error" in res else 0


def secondary(args, dev) -> dict:
    """The other hot-path workloads, timed right after the headline: cfg1 and
    cfg4 decode, the cfg2 prefill+decode mix, the cfg5 block churn
    (copy-on-write, eviction, in-place compaction, with the full-pool
    validation outside timing), the KV append line and exact token selection
    over 256 rows of f32 logits (pkv_sample_exact), up to 10 timed steps
    after 2 warmup steps, no CPU baseline.  Each runs in a child process of
    its own, exactly as `bench.py --config NAME` (its pool allocated in a
    fresh process, as in a standalone run: allocated in this process after
    the headline's pool was freed, cfg4's pool landed on slower HBM
    placements, 465.7-468.7 us per layer against 441.4-461.2 us for every
    fresh-process run).  A failure is recorded under that config's name and
    does not touch the headline figures."""
    import subprocess

    import torch
    torch.cuda.synchronize()
    torch.cuda.empty_cache()  # the headline's tensors, before the children allocate
    runs = {"cfg1": ["--config", "cfg1"], "cfg2": ["--config", "cfg2"],
            "cfg4": ["--config", "cfg4"], "cfg5": ["--config", "cfg5"],
            "append": ["--config", "append"],
            "sample_f32": ["--config", "sample", "--logits", "f32"]}
    steps = max(1, min(args.steps, 10))
    out = {}
    for name, cfg_args in runs.items():
        cmd = [sys.executable, os.path.abspath(__file__), *cfg_args, "--steps", str(steps),
               "--warmup", "2", "--cpu-layers", "0", "--seed", str(args.seed)]
        t0 = time.time()
        try:
            p = subprocess.run(cmd, capture_output=True, text=True, timeout=900)
            lines = [l for l in p.stdout.splitlines() if l.startswith("{")]
            r = json.loads(lines[-1]) if lines else {
                "error": f"exit status {p.returncode}: {p.stderr.strip()[-400:]}"}
        except Exception as e:  # recorded, the headline stands
            r = {"error": f"{type(e).__name__}: {e}"}
        if "error" in r:
            out[name] = {"error": r["error"]}
            log(f"[bench] secondary {name}: {r['error']}")
            continue
        keep = ("bound", "achieved", "unit", "frac", "kernel", "kernel_avg_us")
        out[name] = {"value": r["value"], "unit": r["unit"], "ms_per_step": r["ms_per_step"],
                     "steps": r["steps"], "warmup": r["warmup"], "dtype": r["dtype"],
                     "workload": r["config"]["workload"],
                     "roofline": {k: r["roofline"][k] for k in keep},
                     "wall_s": round(time.time() - t0, 1)}
        for extra in ("roofline_prefill", "roofline_decode", "read_ceiling_GBps", "validation",
                      "cow", "compaction", "bit_exact", "fast", "greedy"):
            if extra in r:
                v = r[extra]
                out[name][extra] = ({k: v[k] for k in keep} if extra.startswith("roofline_")
                                    else v)
            elif extra == "read_ceiling_GBps" and "read_ceiling" in r.get("roofline", {}):
                out[name][extra] = r["roofline"]["read_ceiling"]["GBps"]
        log(f"[bench] secondary {name}: {r['value']} {r['unit']}, "
            f"{r['roofline']['kernel']} frac {r['roofline']['frac']}")
    return out


def decode_bench(args, dev) -> dict:
    """Decode configs (cfg1, cfg2d, cfg3, cfg4): every layer of one decode
    step over the batch as pkv_decode_attention calls (fused append of the
    new token), replayed as HIP graphs when launches are small.  Returns
    the result line as a dict ({"error": ...} on a failed check)."""
    import numpy as np
    import torch

    import pagedkv
    from pagedkv import workload as wl

    shape_attr, B, lo, hi, desc = CONFIGS[args.config]
    shape = getattr(wl, shape_attr)
    if args.kv_dtype:
        # another pool dtype on the same shape (f32: the reference's own KvPool)
        shape = dataclasses.replace(shape, dtype={"f32": wl.F32, "f16": wl.F16,
                                                  "bf16": wl.BF16}[args.kv_dtype])
        desc += f" [KV pool in {args.kv_dtype}]"
    L, H, KVH, hd, bs = shape.n_layers, shape.n_head, shape.n_kv_head, shape.head_dim, shape.block_size
    tdt = pagedkv.torch_dtype(shape.dtype)
    num_blocks = 2048 if args.config == "cfg1" else None
    batch = wl.decode_batch(shape, B, lo, hi, args.seed, num_blocks=num_blocks)
    bytes_step = wl.decode_bytes(shape, batch.ctx)
    bytes_launch = bytes_step / L
    # A step whose K/V fit the Infinity Cache would be timed from cache on
    # the next step: rotate `reps` full pool replicas (layers r*L .. r*L+L-1).
    reps = args.replicas or max(1, min(8, math.ceil(1.0e9 / bytes_step)))
    use_graph = args.graph == "on" or (args.graph == "auto" and bytes_launch < 128e6)
    log(f"[bench] {args.config}: B={B} ctx mean {batch.ctx.mean():.0f} max {batch.ctx.max()} "
        f"pool {batch.num_blocks} blocks x {L} layers x {reps} replica(s), "
        f"{'graph' if use_graph else 'eager'} launches")

    cache = pagedkv.PagedKvCache(L * reps, batch.num_blocks, bs, KVH, hd, tdt)
    cache.fill_normal(args.seed)
    g = torch.Generator(device=dev)
    g.manual_seed(args.seed)
    idt = torch.float32 if args.rope else tdt  # the reference's activations are f32
    q = (torch.randn((L, B, H, hd), generator=g, device=dev, dtype=torch.float32)
         / math.sqrt(hd)).to(idt)
    k_new = torch.randn((L, B, KVH, hd), generator=g, device=dev, dtype=torch.float32).to(idt)
    v_new = torch.randn((L, B, KVH, hd), generator=g, device=dev, dtype=torch.float32).to(idt)
    out = torch.empty((L, B, H * hd), dtype=tdt, device=dev)
    tables = torch.from_numpy(np.where(batch.tables < 0, 0, batch.tables).astype(np.int32)).to(dev)
    ctx_lens = torch.from_numpy(batch.context_lens).to(dev)
    max_ctx = int(batch.context_lens.max())
    cache.reserve_decode(B, H, max_ctx)
    torch.cuda.synchronize()

    lib = pagedkv.lib()
    stream = torch.cuda.current_stream(dev)
    sp = int(stream.cuda_stream) or None
    h = cache.handle
    odt = pagedkv.pkv_dtype(tdt)
    scale = 1.0 / math.sqrt(hd)
    ptrs = [(q[l].data_ptr(), out[l].data_ptr(), k_new[l].data_ptr(), v_new[l].data_ptr())
            for l in range(L)]
    tp, cp, mbps = tables.data_ptr(), ctx_lens.data_ptr(), tables.shape[1]

    rope = None
    if args.rope:
        # Llama-3 rotary base; q/k rotated at position seq_len inside the kernel
        rope = pagedkv.Rope(hd, 500000.0, max_ctx + 1)
        e = 2 if tdt != torch.float32 else 4
        # f32 q and new k/v read instead of the pool dtype, plus one cos/sin row
        bytes_launch += B * (H + 2 * KVH) * hd * (4 - e) + B * hd * 4
        bytes_step = bytes_launch * L

    def launch(l: int, r: int, s) -> None:
        qp, op, kp, vp = ptrs[l]
        if rope is not None:
            rc = lib.pkv_decode_attention_rope(h, r * L + l, rope.handle, None, pagedkv.F32, qp,
                                               op, odt, tp, mbps, cp, max_ctx, B, H, scale, kp,
                                               vp, s)
        else:
            rc = lib.pkv_decode_attention(h, r * L + l, qp, op, odt, tp, mbps, cp, max_ctx, B, H,
                                          scale, kp, vp, s)
        if rc:
            pagedkv._lib.check(rc, h)

    def eager_step(i: int) -> None:
        for l in range(L):
            launch(l, i % reps, sp)

    step = eager_step
    if use_graph:
        # One graph per replica: the L decode calls of a step (main kernel +
        # split-context merge each), replayed in rotation.
        cap = torch.cuda.Stream(dev)
        graphs = []
        for r in range(reps):
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr, stream=cap):
                cs = int(torch.cuda.current_stream(dev).cuda_stream)
                for l in range(L):
                    launch(l, r, cs)
            graphs.append(gr)
        torch.cuda.synchronize()

        def step(i: int) -> None:
            graphs[i % reps].replay()

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    cache.check()
    if use_graph:
        # a graph replay against eager launches of the same step: bit-identical
        step(0)
        torch.cuda.synchronize()
        ref_out = out.clone()
        eager_step(0)
        torch.cuda.synchronize()
        graph_ok = bool(torch.equal(ref_out.view(torch.int16), out.view(torch.int16)))
        log(f"[bench] graph replay == eager launch: {graph_ok}")
        if not graph_ok:
            cache.close()
            return {"error": "graph replay differs from eager launches"}

    ms_step, step_dist = timed_steps(step, args.steps, stream)

    # Dominant-kernel duration: the library records HIP events on the launch
    # stream right before and after each call's main decode kernel (not the
    # split-context merge); eager launches over the same replica rotation.
    n_kt = max(1, min(args.steps, 5))
    cache.profile(True)
    for i in range(n_kt):
        eager_step(i)
    torch.cuda.synchronize()
    kern_total_ms, kern_n = cache.profile_read()
    cache.profile(False)
    kern_avg_ms = kern_total_ms / max(1, kern_n)
    cache.check()

    tok_s = B / (ms_step / 1e3)
    gbps_step = bytes_step / (ms_step / 1e3) / 1e9
    gbps_kernel = bytes_launch / (kern_avg_ms / 1e3) / 1e9
    used_blocks = batch.tables[batch.tables >= 0]
    ceiling = copy_ceiling(dev, cache, used_blocks)
    log(f"[bench] copy ceiling: {ceiling['GBps']:.0f} GB/s ({ceiling['method']})")
    rceil = read_ceiling(dev, cache, used_blocks)
    log(f"[bench] read ceiling: {rceil['GBps']:.0f} GB/s ({rceil['method']})")
    log(f"[bench] {ms_step:.3f} ms/step, {tok_s:.0f} tok/s, step {gbps_step:.0f} GB/s, "
        f"decode kernel avg {kern_avg_ms * 1e3:.1f} us over {kern_n} launches ({gbps_kernel:.0f} GB/s)")

    traffic = None
    prof = os.path.join(ROOT, "profiles", f"decode_{args.config}_traffic.json")
    if os.path.exists(prof):
        with open(prof) as f:
            tr = json.load(f)
        if (tr.get("seed") == args.seed and tr.get("config") == args.config
                and not args.kv_dtype and not args.rope):
            traffic = tr.get("bytes_per_launch")  # measured for the config's own dtype

    cpu = None
    if args.cpu_layers > 0 and not args.rope:
        # layer 0 of replica 0 (the CPU sample's layer) once more with an f32
        # output, so the agreement check sees the fp32 result and not its
        # rounding to the pool dtype (bf16 alone moves it by up to 2^-8
        # relative); the fused append stores the same row again
        out0 = torch.empty((1, B, H * hd), dtype=torch.float32, device=dev)
        qp, _, kp0, vp0 = ptrs[0]
        rc = lib.pkv_decode_attention(h, 0, qp, out0.data_ptr(), pagedkv.F32, tp, mbps, cp,
                                      max_ctx, B, H, scale, kp0, vp0, sp)
        if rc:
            pagedkv._lib.check(rc, h)
        torch.cuda.synchronize()
        cpu = cpu_baseline(cache, batch, shape, args, q, k_new, v_new, out0, log)

    result = {
        "metric": METRIC,
        "value": round(tok_s, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "step_ms": step_dist,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {wl.BF16: "bf16", wl.F16: "f16", wl.F32: "f32"}[shape.dtype],
        "data": "synthetic (seeded N(0,1) K/V/Q, random block tables)",
        "config": {"workload": f"{args.config}: {desc}"
                               + (" + fused RoPE (f32 q/k/v in)" if args.rope else ""),
                   "batch": B, "layers": L,
                   "mean_context": round(float(batch.ctx.mean()), 1), "seed": args.seed,
                   "num_blocks": batch.num_blocks, "pool_replicas": reps,
                   "launch": "hip graph" if use_graph else "eager", "parallelism": "single GPU"},
        "hbm_gbps": round(gbps_step, 1),
        "roofline": {"bound": "hbm", "achieved": round(gbps_kernel, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(gbps_kernel / HBM_PEAK_GBPS, 4),
                     "traffic": traffic, "kernel": "pkv::decode_kernel",
                     "kernel_avg_us": round(kern_avg_ms * 1e3, 2),
                     "algorithmic_bytes_per_launch": int(bytes_launch),
                     "read_ceiling": rceil,
                     "frac_of_read_ceiling": round(gbps_kernel / rceil["GBps"], 4),
                     "copy_ceiling": dict(ceiling, note="read + write rate of a copy; not a "
                                                        "bound for a read-only kernel")},
        "cpu_baseline": cpu,
    }
    if rope is not None:
        rope.close()
    cache.close()
    return result


def append_bench(args, dev) -> dict:
    """KvPool::write (attention.rs:57-83) at a bandwidth-relevant size on
    cfg3's layer shape (8 kv heads, hd 128, bf16, bs 16, a 44,256-block
    pool): 65,536 token rows (256 prompt chunks of 256) scattered to random
    pool slots by one pkv_append call.  value = GB/s of the K and V rows read
    and written; bit-exact against the oracle's closed-form write on a
    sample of rows, untouched rows checked unchanged.  A 512 MiB
    device-to-device copy of known size runs in the same process as the
    calibration point of HBM counters."""
    import numpy as np
    import torch

    import pagedkv
    from pagedkv import workload as wl

    KVH, hd, bs, nb, N = 8, 128, 16, 44256, 65536
    cache = pagedkv.PagedKvCache(1, nb, bs, KVH, hd, torch.bfloat16)
    cache.fill_normal(args.seed)
    slots_np = wl.permutation(args.seed ^ 0xA99, nb * bs)[:N].astype(np.int32)
    g = torch.Generator(device=dev)
    g.manual_seed(args.seed)
    k = torch.randn((N, KVH, hd), generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn((N, KVH, hd), generator=g, device=dev).to(torch.bfloat16)
    slots = torch.from_numpy(slots_np).to(dev)
    before = cache.read_bytes(0, pagedkv.K)
    pool = cache.layer(0)
    for _ in range(max(1, args.warmup)):
        pool.append(k, v, slots)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        pool.append(k, v, slots)
    e1.record()
    torch.cuda.synchronize()
    cache.check()
    ms = e0.elapsed_time(e1) / args.steps
    row = KVH * hd * 2
    gbytes = N * row * 2 * 2   # K and V rows, read and written
    # calibration copy of known size (its dispatch carries 512 MiB each way)
    cal_src = torch.ones((512 << 20) // 4, dtype=torch.int32, device=dev)
    cal_dst = torch.empty_like(cal_src)
    cal_dst.copy_(cal_src)
    torch.cuda.synchronize()
    del cal_src, cal_dst
    # bit-exact: the pool equals the oracle's write of the same rows
    kh = k.cpu().view(torch.int16).numpy().view(np.uint16)
    vh = v.cpu().view(torch.int16).numpy().view(np.uint16)
    exp = before.view(np.uint16).reshape(nb * bs, KVH, hd).copy()
    exp[slots_np] = kh
    got = cache.read_bytes(0, pagedkv.K).view(np.uint16).reshape(nb * bs, KVH, hd)
    ok = bool(np.array_equal(got, exp))
    gotv = cache.read_bytes(0, pagedkv.V).view(np.uint16).reshape(nb * bs, KVH, hd)
    ok &= bool(np.array_equal(gotv[slots_np], vh))
    log(f"[bench] append: {N} rows, {ms * 1e3:.1f} us ({gbytes / (ms / 1e3) / 1e9:.0f} GB/s), "
        f"pool bytes equal the oracle's write: {ok}")
    if not ok:
        cache.close()
        return {"error": "append differs from the oracle"}
    cpu = None
    if args.cpu_layers > 0:
        kp = before.view(np.uint16).reshape(nb * bs, KVH, hd).copy()
        vp = kp.copy()

        def write_all():
            # the closed form of KvPool::write for these rows: row i to slot
            # slots[i], K and V, in place (no per-row pool copy)
            kp[slots_np] = kh
            vp[slots_np] = vh
        dt, passes, _ = timed_passes(write_all, args)
        cpu = {"value": round(gbytes / dt / 1e9, 3), "unit": "GB/s", "cores": 1, "host": host_cpu(),
               "kind": "port",
               "sample": (f"numpy scatter of the same {N} K and V rows to their slots (the "
                          f"closed form of KvPool::write, in place), one thread, {passes} "
                          f"passes of {dt * 1e3:.1f} ms")}
    res = {
        "metric": "KV append (KvPool::write) GB/s, Llama-3-8B layer shape, 1 GPU",
        "value": round(gbytes / (ms / 1e3) / 1e9, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": max(1, args.warmup), "ms_per_step": round(ms, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) rows, random distinct slots)",
        "config": {"workload": f"append: {N} rows (8 kv heads x hd 128 bf16) to random slots of a "
                               f"{nb}-block pool, one pkv_append call", "seed": args.seed,
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(gbytes / (ms / 1e3) / 1e9, 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gbytes / (ms / 1e3) / 1e9 / HBM_PEAK_GBPS, 4), "traffic": None,
                     "kernel": "pkv::append_kernel", "kernel_avg_us": round(ms * 1e3, 2),
                     "algorithmic_bytes_per_launch": gbytes},
        "cpu_baseline": cpu,
        "bit_exact": ok,
    }
    cache.close()
    return res


def gather_bench(args, dev) -> int:
    """KvPool::gather_seq (attention.rs:85-97), the per-row gather of the
    reference's decode step (transformer.rs:277), on cfg3's layer shape: the
    K and V rows of each of the 256 sequences (ctx + 1 tokens) copied out of
    the pool in table order by pkv_gather_seq, one call per sequence, the
    256 calls replayed as a HIP graph.  value = GB/s of read + written bytes;
    checked bit-exact against the oracle on a sample of sequences."""
    import numpy as np
    import torch

    import oracle
    import pagedkv
    from pagedkv import workload as wl

    shape = wl.CFG3
    B, bs, KVH, hd = 256, shape.block_size, shape.n_kv_head, shape.head_dim
    batch = wl.decode_batch(shape, B, 512, 4096, args.seed)
    cache = pagedkv.PagedKvCache(1, batch.num_blocks, bs, KVH, hd, torch.bfloat16)
    cache.fill_normal(args.seed)
    lens = (batch.ctx + 1).astype(np.int64)
    tables = [torch.from_numpy(np.ascontiguousarray(batch.tables[b, :-(-int(lens[b]) // bs)]))
              .to(dev) for b in range(B)]
    outs = [(torch.empty((int(n), KVH, hd), dtype=torch.bfloat16, device=dev),
             torch.empty((int(n), KVH, hd), dtype=torch.bfloat16, device=dev)) for n in lens]
    lib = pagedkv.lib()
    h = cache.handle

    def calls(sp):
        for b in range(B):
            rc = lib.pkv_gather_seq(h, 0, tables[b].data_ptr(), int(lens[b]),
                                    outs[b][0].data_ptr(), outs[b][1].data_ptr(), sp)
            if rc:
                pagedkv._lib.check(rc, h)

    cap = torch.cuda.Stream(dev)
    gr = torch.cuda.CUDAGraph()
    calls(int(torch.cuda.current_stream(dev).cuda_stream) or None)
    torch.cuda.synchronize()
    with torch.cuda.graph(gr, stream=cap):
        calls(int(torch.cuda.current_stream(dev).cuda_stream))
    for _ in range(max(1, args.warmup)):
        gr.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        gr.replay()
    e1.record()
    torch.cuda.synchronize()
    cache.check()
    ms = e0.elapsed_time(e1) / args.steps
    row = KVH * hd * 2
    gbytes = int(lens.sum()) * row * 2 * 2  # K and V rows, read and written
    # bit-exact against the oracle's closed form on a sample of sequences
    nd = np.uint16
    kp = cache.read_bytes(0, pagedkv.K).view(nd).reshape(batch.num_blocks, bs, KVH, hd)
    vp = cache.read_bytes(0, pagedkv.V).view(nd).reshape(batch.num_blocks, bs, KVH, hd)
    ok = True
    for b in range(0, B, 51):
        rk, rv = oracle.gather_seq(kp, vp, bs, batch.tables[b].astype(np.uint32), int(lens[b]))
        gk = outs[b][0].cpu().view(torch.int16).numpy().view(np.uint16)
        gv = outs[b][1].cpu().view(torch.int16).numpy().view(np.uint16)
        ok &= np.array_equal(gk, rk) and np.array_equal(gv, rv)
    log(f"[bench] gather: {B} sequences, {int(lens.sum())} rows, {ms * 1e3:.1f} us per step "
        f"({gbytes / (ms / 1e3) / 1e9:.0f} GB/s), oracle bit-exact: {ok}")
    if not ok:
        print(json.dumps({"error": "gather differs from the oracle"}))
        return 1
    # the same rows by one pkv_gather_varlen call (no reference counterpart),
    # checked equal to the per-sequence outputs
    mb = max(t.numel() for t in tables)
    vt = torch.zeros((B, mb), dtype=torch.int32, device=dev)
    for b in range(B):
        vt[b, :tables[b].numel()] = tables[b]
    total = int(lens.sum())
    cu = torch.from_numpy(np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)).to(dev)
    vk = torch.empty((total, KVH, hd), dtype=torch.bfloat16, device=dev)
    vv = torch.empty_like(vk)
    sp0 = int(torch.cuda.current_stream(dev).cuda_stream) or None

    def varlen():
        rc = lib.pkv_gather_varlen(h, 0, vt.data_ptr(), mb, cu.data_ptr(), B, total,
                                   vk.data_ptr(), vv.data_ptr(), sp0)
        if rc:
            pagedkv._lib.check(rc, h)
    for _ in range(max(1, args.warmup)):
        varlen()
    torch.cuda.synchronize()
    e0.record()
    for _ in range(args.steps):
        varlen()
    e1.record()
    torch.cuda.synchronize()
    cache.check()
    ms_varlen = e0.elapsed_time(e1) / args.steps
    same = all(torch.equal(vk[int(c0):int(c0) + int(n)], outs[b][0]) and
               torch.equal(vv[int(c0):int(c0) + int(n)], outs[b][1])
               for b, (c0, n) in enumerate(zip(np.concatenate([[0], np.cumsum(lens)])[:-1], lens)))
    log(f"[bench] gather_varlen (one call): {ms_varlen * 1e3:.1f} us "
        f"({gbytes / (ms_varlen / 1e3) / 1e9:.0f} GB/s), equal to the per-sequence calls: {same}")
    if not same:
        print(json.dumps({"error": "gather_varlen differs from gather_seq"}))
        return 1
    cpu = None
    if args.cpu_layers > 0:
        tb = batch.tables.astype(np.uint32)
        rows = iter(range(1 << 30))
        per, n, _ = timed_passes(
            lambda: [oracle.gather_seq(kp, vp, bs, tb[b], int(lens[b]))
                     for b in [next(rows) % B]], args)
        mean_b = gbytes / B
        cpu = {"value": round(mean_b / per / 1e9, 2), "unit": "GB/s", "cores": 1, "host": host_cpu(), "kind": "port",
               "sample": f"oracle gather_seq (closed-form index copy) of one sequence per pass, "
                         f"{n} passes of {per * 1e3:.2f} ms"}
    res = {
        "metric": "KvPool::gather_seq GB/s (read + written), Llama-3-8B layer shape, 1 GPU",
        "value": round(gbytes / (ms / 1e3) / 1e9, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) pool, random block tables)",
        "config": {"workload": f"gather: {B} sequences of cfg3 (ctx U[512, 4096]), one layer, "
                               f"8 kv heads x hd 128, bs 16, one call per sequence in a HIP graph",
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(gbytes / (ms / 1e3) / 1e9, 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gbytes / (ms / 1e3) / 1e9 / HBM_PEAK_GBPS, 4), "traffic": None,
                     "kernel": "pkv::gather_kernel", "kernel_avg_us": round(ms * 1e3 / B, 2),
                     "algorithmic_bytes_per_launch": gbytes // B},
        "varlen_one_call": {"us": round(ms_varlen * 1e3, 2),
                            "GBps": round(gbytes / (ms_varlen / 1e3) / 1e9, 1),
                            "kernel": "pkv::gather_varlen_kernel"},
        "cpu_baseline": cpu,
    }
    print(json.dumps(res), flush=True)
    cache.close()
    return 0


def sample_bench(args, dev) -> dict:
    """Token selection on the device (sample.rs:12-55 as the engine calls it,
    engine.rs:145-162): 256 rows of Llama-3's 128,256-entry vocabulary in
    bf16 (--logits f32: genuine f32 values), every row sampled at temperature
    0.8 (seed 42, no top-k / top-p, as the engine's sample_cfg).  value =
    rows/s of pkv_sample_exact, which reproduces sample.rs's f32 arithmetic
    bit for bit (checked against the oracle's f32 restatement); the faster
    pkv_sample (exact probability mass, equal tokens except where the
    reference's f32 rounding alone moves the pick) and greedy rows are timed
    beside it.  roofline = one read of the logits per launch against HBM
    peak."""
    import numpy as np
    import torch

    import oracle
    import pagedkv

    B, V = 256, 128256
    f32 = args.logits == "f32"
    g = torch.Generator(device=dev)
    g.manual_seed(args.seed)
    logits = torch.randn((B, V), generator=g, device=dev) * 3.0
    if not f32:
        logits = logits.to(torch.bfloat16)
    ldt = pagedkv.F32 if f32 else pagedkv.BF16
    temps = torch.full((B,), 0.8, device=dev)
    out = torch.empty(B, dtype=torch.int32, device=dev)
    lib = pagedkv.lib()
    sp = int(torch.cuda.current_stream(dev).cuda_stream) or None

    def run(t, exact=False, rows=B, o=None):
        fn = lib.pkv_sample_exact if exact else lib.pkv_sample
        rc = fn(logits.data_ptr(), ldt, V, rows, V,
                t.data_ptr() if t is not None else None, 0, float("nan") if exact else 1.0, 42,
                (o if o is not None else out).data_ptr(), sp)
        if rc:
            pagedkv._lib.check(rc, None)

    def time_it(t, exact=False, rows=B, o=None):
        for _ in range(max(1, args.warmup)):
            run(t, exact, rows, o)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.steps):
            run(t, exact, rows, o)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / args.steps

    ms_exact = time_it(temps, exact=True)
    got_exact = out.cpu().numpy().copy()
    routes = torch.empty(B, dtype=torch.int32, device=dev)
    pagedkv.sample(logits, temps, routes=routes)
    rnames = ("argmax", "buckets", "runs", "sort")
    route_counts = {rnames[k]: int(v) for k, v in
                    enumerate(torch.bincount(routes.long().cpu(), minlength=4).tolist()) if v}
    ms = time_it(temps)
    got = out.cpu().numpy().copy()
    ms_greedy = time_it(None)
    greedy = out.cpu().numpy().copy()
    x32 = logits.float().cpu().numpy()
    # parity on a few rows: greedy exact; sampled equal to the exact-arithmetic
    # restatement unless its running sum is within 1e-6 of r
    # and the exact path equal to the f32 restatement (the reference's arithmetic)
    ok = True
    for b in range(0, B, 37):
        ok &= int(greedy[b]) == oracle.argmax(x32[b])
        tok, margin = oracle.sample(x32[b], 0.8, precise=True)
        ok &= int(got[b]) == tok or margin < 1e-6
        ok &= int(got_exact[b]) == oracle.sample(x32[b], 0.8)[0]
    log(f"[bench] sample: exact {ms_exact * 1e3:.1f} us (rows by kernel: {route_counts}), "
        f"fast {ms * 1e3:.1f} us sampled, {ms_greedy * 1e3:.1f} us greedy for {B} x {V} "
        f"{args.logits} rows; oracle check {'ok' if ok else 'FAILED'}")
    if not ok:
        return {"error": "token selection differs from the oracle"}
    rbytes = B * V * (4 if f32 else 2) + B * 4
    # small batches (the split path: each row over several workgroups), the
    # first rows of the same logits; checked against the full batch's tokens
    small, small_exact = {}, {}
    for sb in (1, 8, 32):
        o2 = torch.empty(sb, dtype=torch.int32, device=dev)
        for exact, dst, ref in ((False, small, got), (True, small_exact, got_exact)):
            us = time_it(temps, exact, sb, o2) * 1e3
            same = bool(np.array_equal(o2.cpu().numpy(), ref[:sb]))
            dst[str(sb)] = {"us": round(us, 2), "same_tokens_as_full_batch": same}
            ok &= same
    log(f"[bench] sample, small batches (us): "
        + ", ".join(f"{k} rows exact {small_exact[k]['us']} / fast {v['us']}"
                    for k, v in small.items()))
    if not ok:
        return {"error": "small-batch tokens differ from the full batch's"}
    cpu = None
    if args.cpu_layers > 0:
        # the reference procedure (sort, f32 softmax, running sum) on host rows
        rows = iter(range(1 << 30))
        per, n, _ = timed_passes(lambda: oracle.sample(x32[next(rows) % B], 0.8), args)
        cpu = {"value": round(1.0 / per, 1), "unit": "rows/s", "cores": 1, "host": host_cpu(), "kind": "port",
               "sample": f"oracle sample() (stable sort + f32 softmax + running sum, as "
                         f"sample.rs) of one {V}-entry row, {n} passes of {per * 1e3:.1f} ms"}
    res = {
        "metric": "on-device token selection rows/s (sample.rs at T=0.8), Llama-3 vocabulary, 1 GPU",
        "value": round(B / (ms_exact / 1e3), 1), "unit": "rows/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_exact, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": args.logits,
        "data": "synthetic (seeded N(0, 9) logits" + (", genuine f32 values)" if f32 else ")"),
        "config": {"workload": f"sample: {B} rows x {V} {args.logits} logits, temperature 0.8, "
                               f"seed 42",
                   "entry_point": "pkv_sample_exact (bit-identical to sample.rs)",
                   "rows_by_kernel": route_counts,
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(rbytes / (ms_exact / 1e3) / 1e9, 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(rbytes / (ms_exact / 1e3) / 1e9 / HBM_PEAK_GBPS, 4),
                     "traffic": None,
                     "kernel": "pkv::sample_bucket_kernel" if f32 else "pkv::sample_runs_kernel",
                     "kernel_avg_us": round(ms_exact * 1e3, 2),
                     "algorithmic_bytes_per_launch": rbytes},
        "small_batches_exact": small_exact,
        "fast": {"entry_point": "pkv_sample (exact probability mass; equal tokens except where "
                                "the reference's f32 rounding alone moves the pick)",
                 "us": round(ms * 1e3, 2), "rows_per_s": round(B / (ms / 1e3), 1),
                 "GBps": round(rbytes / (ms / 1e3) / 1e9, 1), "small_batches": small},
        "greedy": {"us": round(ms_greedy * 1e3, 2),
                   "GBps": round(rbytes / (ms_greedy / 1e3) / 1e9, 1)},
        "cpu_baseline": cpu,
    }
    return res


def cpu_baseline(cache, batch, shape, args, q, k_new, v_new, out, log):
    """Times the oracle's CPU restatement of the reference decode math
    (append + attention per layer, OpenMP over (sequence, kv head)) on layer
    0's data copied to host, repeated for a bounded sample (timed_passes),
    scaled to a full step."""
    import numpy as np
    import oracle
    import pagedkv
    from pagedkv import workload as wl

    threads = args.cpu_threads or min(16, os.cpu_count() or 1)
    nd = np.float32 if shape.dtype == wl.F32 else np.uint16
    shp = (cache.num_blocks, cache.block_size, cache.n_kv_head, cache.head_dim)
    t_copy = time.time()
    kp = cache.read_bytes(0, pagedkv.K).view(nd).reshape(shp)
    vp = cache.read_bytes(0, pagedkv.V).view(nd).reshape(shp)

    def host(t):
        t = t.contiguous().cpu()
        if nd is np.uint16:
            return t.view(__import__("torch").int16).numpy().view(np.uint16)
        return t.numpy()

    qh, knh, vnh = host(q[0]), host(k_new[0]), host(v_new[0])
    tables = np.where(batch.tables < 0, 0, batch.tables).astype(np.int32)
    cl = batch.context_lens
    log(f"[bench] cpu baseline: host copy {time.time() - t_copy:.1f}s, {threads} threads")
    scale = 1.0 / math.sqrt(shape.head_dim)
    oracle.lib()
    dt, passes, res = timed_passes(
        lambda: oracle.decode_inplace(kp, vp, shape.dtype, shape.block_size, tables, cl, qh, knh,
                                      vnh, scale, n_threads=threads), args)
    step_s = dt * shape.n_layers
    # sanity: the CPU result agrees with the GPU's layer-0 output
    gpu0 = out[0].float().cpu().numpy()
    agree, worst = agreement(gpu0, res)
    log(f"[bench] cpu baseline: {dt:.2f} s/layer -> {batch.batch / step_s:.1f} tok/s "
        f"(gpu/cpu layer-0 agreement: {agree}, max |err| / bound {worst:.3f})")
    res_cpu = {"value": round(batch.batch / step_s, 2), "unit": "tok/s", "cores": threads, "host": host_cpu(),
               "kind": "port",
               "sample": (f"layer 0 of the same workload ({batch.batch} seqs, append + attention), "
                          f"{passes} passes of {dt * 1e3:.1f} ms, scaled x{shape.n_layers} layers"),
               "agrees_with_gpu": agree, "tolerance": TOLERANCE,
               "max_err_over_bound": round(worst, 4)}
    # The reference's own costs where they fit in a bounded sample: an f32
    # pool, a full K and V pool copy per appended row (slice_assign), then
    # gather / pad / GQA repeat / masked SDPA, one thread.
    if kp.size * 4 <= (256 << 20):
        kf = wl.widen(kp, shape.dtype).reshape(shp).astype(np.float32)
        vf = wl.widen(vp, shape.dtype).reshape(shp).astype(np.float32)
        qf, knf, vnf = (wl.widen(x, shape.dtype).astype(np.float32) for x in (qh, knh, vnh))
        seq = (cl - 1).astype(np.int64)
        fdt, fpasses, _ = timed_passes(
            lambda: oracle.decode_step_faithful_f32(kf, vf, shape.block_size, tables, seq, seq,
                                                    qf, knf, vnf, scale), args)
        fstep = fdt * shape.n_layers
        log(f"[bench] cpu reference-faithful: {fdt:.2f} s/layer -> "
            f"{batch.batch / fstep:.2f} tok/s")
        res_cpu["reference_faithful"] = {
            "value": round(batch.batch / fstep, 3), "unit": "tok/s", "cores": 1, "host": host_cpu(),
            "kind": "port",
            "sample": (f"layer 0, f32 pool of {kp.size * 4 >> 20} MiB per K, a full K and V pool "
                       f"copy per appended row (slice_assign) then gather/pad/mask/sdpa, "
                       f"{fpasses} passes of {fdt * 1e3:.0f} ms, scaled x{shape.n_layers} layers")}
    return res_cpu


def mix(args, dev) -> dict:
    """TinyLlama-1.1B continuous-batching mix (22
    layers, 32q/4kv heads, hd 64, bs 16, f16).  Per layer: the 8 sequences
    in chunked prefill store their 256-token chunk (pkv_append) and attend
    it causally over prior context U[0,1024] (pkv_prefill_attention); the
    56 decoding sequences (context U[256,2048]) append one token and attend
    (pkv_decode_attention, fused append).  value = tokens advanced per
    second (8*256 + 56 per step).  roofline = the prefill kernel's
    algorithmic flops (unmasked query-key pairs) over its average duration
    against 2.5 PFLOP/s dense f16; the decode kernel's HBM roofline beside."""
    import numpy as np
    import torch

    import pagedkv
    from pagedkv import workload as wl

    shape = wl.CFG2
    L, H, KVH, hd, bs = shape.n_layers, shape.n_head, shape.n_kv_head, shape.head_dim, shape.block_size
    NP, C, ND = 8, 256, 56
    m = wl.mix_batch(shape, NP, C, 0, 1024, ND, 256, 2048, args.seed)
    T = NP * C
    log(f"[bench] cfg2: {NP} prefill chunks of {C} (priors {m.prior.tolist()}), {ND} decode "
        f"(ctx mean {m.ctx.mean():.0f}), pool {m.num_blocks} blocks x {L} layers")
    tdt = torch.float16
    cache = pagedkv.PagedKvCache(L, m.num_blocks, bs, KVH, hd, tdt)
    cache.fill_normal(args.seed)
    g = torch.Generator(device=dev)
    g.manual_seed(args.seed)

    def rnd(*shp, sc=1.0):
        return (torch.randn(shp, generator=g, device=dev, dtype=torch.float32) * sc).to(tdt)

    sc = 1.0 / math.sqrt(hd)
    # with --rope the inputs are the f32 projections before rotation (the
    # reference's activations) and the rotary embedding is part of the step
    qp, kc, vc = rnd(L, T, H, hd, sc=sc), rnd(L, T, KVH, hd), rnd(L, T, KVH, hd)
    qd, kd, vd = rnd(L, ND, H, hd, sc=sc), rnd(L, ND, KVH, hd), rnd(L, ND, KVH, hd)
    if args.rope:
        qp, kc, vc, qd, kd, vd = (t.float() for t in (qp, kc, vc, qd, kd, vd))
        qrot = torch.empty((T, H, hd), dtype=tdt, device=dev)
    outp = torch.empty((L, T, H * hd), dtype=tdt, device=dev)
    outd = torch.empty((L, ND, H * hd), dtype=tdt, device=dev)
    tables = np.where(m.tables < 0, 0, m.tables).astype(np.int32)
    ptab = torch.from_numpy(np.ascontiguousarray(tables[:NP])).to(dev)
    dtab = torch.from_numpy(np.ascontiguousarray(tables[NP:])).to(dev)
    slots = torch.from_numpy(m.chunk_slots()).to(dev)
    cu = torch.from_numpy(m.cu_q_lens).to(dev)
    pctx_np = (m.prior + m.chunk).astype(np.int32)
    dctx_np = (m.ctx + 1).astype(np.int32)
    pctx, dctx = torch.from_numpy(pctx_np).to(dev), torch.from_numpy(dctx_np).to(dev)
    max_p, max_d = int(pctx_np.max()), int(dctx_np.max())
    mbps = tables.shape[1]
    cache.reserve_decode(ND, H, max_d)
    rope = None
    if args.rope:
        rope = pagedkv.Rope(hd, 10000.0, max(max_p, max_d) + 1)
        ppos = torch.from_numpy(np.concatenate(
            [np.arange(p, p + c, dtype=np.int32) for p, c in zip(m.prior, m.chunk)])).to(dev)
    torch.cuda.synchronize()

    lib = pagedkv.lib()
    stream = torch.cuda.current_stream(dev)
    sp = int(stream.cuda_stream) or None
    h = cache.handle
    odt = pagedkv.pkv_dtype(tdt)
    chk = pagedkv._lib.check

    def append(l):
        if rope is not None:   # k rotated + stored, v stored, q rotated: one launch
            rc = lib.pkv_append_rope(h, l, rope.handle, ppos.data_ptr(), pagedkv.F32,
                                     kc[l].data_ptr(), vc[l].data_ptr(), slots.data_ptr(), T,
                                     qp[l].data_ptr(), qrot.data_ptr(), H, sp)
        else:
            rc = lib.pkv_append(h, l, kc[l].data_ptr(), vc[l].data_ptr(), slots.data_ptr(), T, sp)
        if rc:
            chk(rc, h)

    def prefill(l):
        q = qrot if rope is not None else qp[l]
        rc = lib.pkv_prefill_attention(h, l, q.data_ptr(), outp[l].data_ptr(), odt,
                                       cu.data_ptr(), pctx.data_ptr(), ptab.data_ptr(), mbps, NP, C,
                                       max_p, H, sc, sp)
        if rc:
            chk(rc, h)

    def prefill_store(l):
        # the chunk's K/V stored by the prefill launch itself
        rc = lib.pkv_prefill_attention_append(h, l, qp[l].data_ptr(), outp[l].data_ptr(), odt,
                                              cu.data_ptr(), pctx.data_ptr(), ptab.data_ptr(),
                                              mbps, NP, C, max_p, H, sc, kc[l].data_ptr(),
                                              vc[l].data_ptr(), sp)
        if rc:
            chk(rc, h)

    fused_store = rope is None and not args.unfused

    def chunk(l):
        if fused_store:
            prefill_store(l)
        else:
            append(l)
            prefill(l)

    def decode(l, on=None):
        st = on if on is not None else sp
        if rope is not None:
            rc = lib.pkv_decode_attention_rope(h, l, rope.handle, None, pagedkv.F32,
                                               qd[l].data_ptr(), outd[l].data_ptr(), odt,
                                               dtab.data_ptr(), mbps, dctx.data_ptr(), max_d, ND,
                                               H, sc, kd[l].data_ptr(), vd[l].data_ptr(), st)
        else:
            rc = lib.pkv_decode_attention(h, l, qd[l].data_ptr(), outd[l].data_ptr(), odt,
                                          dtab.data_ptr(), mbps, dctx.data_ptr(), max_d, ND, H,
                                          sc, kd[l].data_ptr(), vd[l].data_ptr(), st)
        if rc:
            chk(rc, h)

    # Per layer the prefill rows' and the decode rows' attention are
    # independent (an engine forks them after the QKV projection and joins
    # before the output projection): the decode runs on a second stream
    # (default priority) between a fork and a join event of each layer.
    dec_stream = torch.cuda.Stream(dev)
    dsp = int(dec_stream.cuda_stream)
    forks = [torch.cuda.Event() for _ in range(L)]
    joins = [torch.cuda.Event() for _ in range(L)]

    def step_serial():
        for l in range(L):
            chunk(l)
            decode(l)

    def step_overlap():
        for l in range(L):
            forks[l].record(stream)
            dec_stream.wait_event(forks[l])
            decode(l, dsp)
            chunk(l)
            joins[l].record(dec_stream)
            stream.wait_event(joins[l])

    # the decode's split-context partials live in the pool workspace, which a
    # split prefill would share: overlap only when the prefill does not split
    overlap_ok = cache.prefill_workspace_bytes(NP, H, C, max_p) == 0

    # One launch per layer for both batches (pkv_mixed_attention): the
    # prefill and decode workgroups share the CUs.  The argument structs are
    # built once; the stream is the call's own argument.
    use_mixed = not args.serial and not args.separate and fused_store
    pbs = [pagedkv._lib.PrefillBatch(qp[l].data_ptr(), outp[l].data_ptr(), odt, cu.data_ptr(),
                                     pctx.data_ptr(), ptab.data_ptr(), mbps, NP, C, max_p,
                                     kc[l].data_ptr(), vc[l].data_ptr()) for l in range(L)]
    dbs = [pagedkv._lib.DecodeBatch(qd[l].data_ptr(), outd[l].data_ptr(), odt, dtab.data_ptr(),
                                    mbps, dctx.data_ptr(), max_d, ND, kd[l].data_ptr(),
                                    vd[l].data_ptr()) for l in range(L)]

    def mixed(l):
        rc = lib.pkv_mixed_attention(h, l, ctypes.byref(pbs[l]), ctypes.byref(dbs[l]), H, sc, sp)
        if rc:
            chk(rc, h)

    def step_mixed():
        for l in range(L):
            mixed(l)

    dists = {}

    def time_steps(fn):
        for _ in range(args.warmup):
            fn()
        ms, dists[fn] = timed_steps(lambda i: fn(), args.steps, stream)
        return ms

    def capture(fn):
        # the library calls take the stream pointer `sp`: point it at the
        # capture stream while fn is recorded
        nonlocal stream, sp
        cap = torch.cuda.Stream(dev)
        cap.wait_stream(stream)
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        saved = (stream, sp)
        with torch.cuda.graph(gr, stream=cap):
            stream, sp = cap, int(cap.cuda_stream)
            fn()
        stream, sp = saved
        torch.cuda.synchronize()
        return gr

    ms_serial = time_steps(step_serial)   # eager, one stream
    step_fn = step_serial
    ms_graph_serial = None
    ms_graph_separate = None
    schedule = "eager launches, one stream"
    ms_step = ms_serial
    if not args.serial:
        # the step as a HIP graph, each layer's decode forked onto a second
        # stream when allowed; one replay must reproduce an eager step's
        # outputs bit for bit (both kernels are deterministic and the step's
        # appends rewrite the same rows)
        step_serial()
        torch.cuda.synchronize()
        ref_p, ref_d = outp.clone(), outd.clone()
        g_serial = capture(step_serial)
        g_step = capture(step_overlap) if overlap_ok else g_serial
        outp.zero_()
        outd.zero_()
        g_step.replay()
        torch.cuda.synchronize()
        if not (torch.equal(outp, ref_p) and torch.equal(outd, ref_d)):
            if rope is not None:
                rope.close()
            cache.close()
            return {"error": "graph replay differs from eager launches"}
        ms_graph_serial = time_steps(g_serial.replay)
        step_fn = g_step.replay
        ms_step = time_steps(step_fn)
        schedule = ("HIP graph; per layer the decode on a second stream, forked and joined "
                    "around the prefill" if overlap_ok else "HIP graph, one stream")
        if use_mixed:
            ms_graph_separate = ms_step
            # one eager mixed step must equal the separate launches bit for
            # bit, and so must a replay of its graph
            outp.zero_()
            outd.zero_()
            step_mixed()
            torch.cuda.synchronize()
            same = torch.equal(outp, ref_p) and torch.equal(outd, ref_d)
            g_mixed = capture(step_mixed)
            outp.zero_()
            outd.zero_()
            g_mixed.replay()
            torch.cuda.synchronize()
            if not (same and torch.equal(outp, ref_p) and torch.equal(outd, ref_d)):
                if rope is not None:
                    rope.close()
                cache.close()
                return {"error": "mixed launches differ from separate launches"}
            step_fn = g_mixed.replay
            ms_step = time_steps(step_fn)
            schedule = ("HIP graph, one pkv_mixed_attention launch per layer (prefill and "
                        "decode workgroups in one grid, then the split-context merge)")
        del ref_p, ref_d
    cache.check()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    n_kt = max(1, min(args.steps, 5))

    def kernel_ms(fn):
        cache.profile(True)
        for _ in range(n_kt):
            for l in range(L):
                fn(l)
        torch.cuda.synchronize()
        tot, n = cache.profile_read()
        cache.profile(False)
        return tot / max(1, n), n

    pre_ms, pre_n = kernel_ms(prefill_store if fused_store else prefill)
    dec_ms, dec_n = kernel_ms(decode)
    mix_ms = kernel_ms(mixed)[0] if use_mixed else None
    t0.record(stream)
    for _ in range(n_kt):
        for l in range(L):
            append(l)
    t1.record(stream)
    torch.cuda.synchronize()
    app_ms = t0.elapsed_time(t1) / (n_kt * L)
    cache.check()

    flops = wl.prefill_flops(shape, m.prior, m.chunk)
    pbytes = wl.prefill_bytes(shape, m.prior, m.chunk)
    dbytes = wl.decode_bytes(shape, m.ctx, 1)
    # chunk append: k and v read and written (+ q read and written with --rope)
    ib = 4 if rope is not None else 2
    abytes = T * KVH * hd * 2 * (ib + 2) + 4 * T
    if rope is not None:
        abytes += T * H * hd * (ib + 2) + 4 * T
    tflops = flops / (pre_ms / 1e3) / 1e12
    dec_gbps = dbytes / (dec_ms / 1e3) / 1e9
    tok_s = (T + ND) / (ms_step / 1e3)
    # decode flops: q.k and p.v over every key of every query head
    dflops = 4 * H * hd * int((m.ctx + 1).sum())
    roof_pre = {"bound": "mfma", "achieved": round(tflops, 2), "peak": 2500.0,
                "unit": "TFLOP/s", "frac": round(tflops / 2500.0, 4), "traffic": None,
                "kernel": "pkv::prefill_kernel", "kernel_avg_us": round(pre_ms * 1e3, 2),
                "algorithmic_flops_per_launch": flops, "algorithmic_bytes_per_launch": pbytes}
    roof = roof_pre
    if mix_ms is not None:
        mtf = (flops + dflops) / (mix_ms / 1e3) / 1e12
        roof = {"bound": "mfma", "achieved": round(mtf, 2), "peak": 2500.0, "unit": "TFLOP/s",
                "frac": round(mtf / 2500.0, 4), "traffic": None, "kernel": "pkv::mixed_kernel",
                "kernel_avg_us": round(mix_ms * 1e3, 2),
                "algorithmic_flops_per_launch": flops + dflops,
                "algorithmic_bytes_per_launch": pbytes + dbytes,
                "hbm_GBps": round((pbytes + dbytes) / (mix_ms / 1e3) / 1e9, 1)}
        log(f"[bench] mixed kernel {mix_ms * 1e3:.1f} us per layer ({mtf:.1f} TFLOP/s, "
            f"{roof['hbm_GBps']:.0f} GB/s); separate launches, graph: {ms_graph_separate:.3f} ms")
    log(f"[bench] {ms_step:.3f} ms/step ({schedule}; eager serial {ms_serial:.3f}, graph serial "
        f"{ms_graph_serial if ms_graph_serial is None else round(ms_graph_serial, 3)}), "
        f"{tok_s:.0f} tok/s; per layer: prefill {pre_ms * 1e3:.1f} us "
        f"({tflops:.1f} TFLOP/s), decode {dec_ms * 1e3:.1f} us ({dec_gbps:.0f} GB/s), "
        f"chunk append {app_ms * 1e3:.1f} us")

    cpu = None
    if args.cpu_layers > 0 and rope is None:
        import oracle
        threads = args.cpu_threads or min(16, os.cpu_count() or 1)
        shp = (m.num_blocks, bs, KVH, hd)
        kp = cache.read_bytes(0, pagedkv.K).view(np.uint16).reshape(shp)
        vp = cache.read_bytes(0, pagedkv.V).view(np.uint16).reshape(shp)

        def host(t):
            return t.contiguous().cpu().view(torch.int16).numpy().view(np.uint16)

        hq, hk, hv = host(qp[0]), host(kc[0]), host(vc[0])
        dq, dk, dv = host(qd[0]), host(kd[0]), host(vd[0])
        oracle.lib()

        def one_layer():
            return (oracle.prefill_inplace(kp, vp, wl.F16, bs, tables[:NP], m.cu_q_lens, pctx_np,
                                           hq, hk, hv, sc, n_threads=threads),
                    oracle.decode_inplace(kp, vp, wl.F16, bs, tables[NP:], dctx_np, dq, dk, dv,
                                          sc, n_threads=threads))
        dt, passes, (rp, rd) = timed_passes(one_layer, args)
        gp, gd = outp[0].float().cpu().numpy(), outd[0].float().cpu().numpy()
        agree_p, worst_p = agreement(gp, rp)
        agree_d, worst_d = agreement(gd, rd)
        agree, worst = agree_p and agree_d, max(worst_p, worst_d)
        log(f"[bench] cpu baseline: {dt:.2f} s/layer (gpu/cpu layer-0 agreement: {agree}, "
            f"max |err| / bound {worst:.3f})")
        cpu = {"value": round((T + ND) / (dt * L), 2), "unit": "tok/s", "cores": threads, "host": host_cpu(),
               "kind": "port",
               "sample": (f"layer 0 of the same mix (chunk store + causal prefill of {NP}x{C}, "
                          f"append + decode of {ND}), {passes} passes of {dt * 1e3:.1f} ms, "
                          f"scaled x{L} layers"),
               "agrees_with_gpu": agree, "tolerance": TOLERANCE,
               "max_err_over_bound": round(worst, 4)}
        cpu["reference_faithful"] = mix_faithful(m, tables, kp, vp, (hq, hk, hv), (dq, dk, dv),
                                                 NP, C, ND, L, sc)

    res = {
        "metric": "continuous-batching mix tokens/s (chunked prefill + decode), TinyLlama-1.1B shape, 1 GPU",
        "value": round(tok_s, 1), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 4), "step_ms": dists[step_fn],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f16",
        "data": "synthetic (seeded N(0,1) K/V/Q, random block tables)",
        "config": {"workload": "cfg2: 22 layers, 32q/4kv heads, hd 64, bs 16, f16 KV; 8 chunked "
                               "prefills of 256 over prior U[0,1024] + 56 decodes, ctx U[256,2048]"
                               + (" + RoPE (f32 q/k/v in: pkv_append_rope, "
                                  "pkv_decode_attention_rope)" if rope is not None else ""),
                   "priors": m.prior.tolist(), "mean_decode_context": round(float(m.ctx.mean()), 1),
                   "seed": args.seed, "num_blocks": m.num_blocks, "parallelism": "single GPU"},
        "roofline": roof,
        "roofline_prefill": roof_pre,
        "roofline_decode": {"bound": "hbm", "achieved": round(dec_gbps, 1), "peak": HBM_PEAK_GBPS,
                            "unit": "GB/s", "frac": round(dec_gbps / HBM_PEAK_GBPS, 4),
                            "kernel": "pkv::decode_kernel", "kernel_avg_us": round(dec_ms * 1e3, 2),
                            "algorithmic_bytes_per_launch": dbytes},
        "append": {"us": round(app_ms * 1e3, 2), "GBps": round(abytes / (app_ms / 1e3) / 1e9, 1),
                   "rope": rope is not None},
        "schedule": schedule,
        "chunk_store": ("fused into the prefill launch (pkv_prefill_attention_append)"
                        if fused_store else "separate launch (append us above)"),
        "ms_per_step_eager_serial": round(ms_serial, 4),
        "ms_per_step_graph_serial": None if ms_graph_serial is None else round(ms_graph_serial, 4),
        "ms_per_step_graph_separate": (None if ms_graph_separate is None
                                       else round(ms_graph_separate, 4)),
        "cpu_baseline": cpu,
    }
    if rope is not None:
        rope.close()
    cache.close()
    return res


def mix_faithful(m, tables, kp, vp, chunk_rows, decode_rows, NP, C, ND, L, scale):
    """The reference's own costs for cfg2's layer 0, one thread: f32 pools
    (its KvPool dtype); every stored row -- the 8 x 256 chunk tokens and the
    56 decode tokens -- first copies the whole K and V pool (slice_assign,
    attention.rs:73-80; transformer.rs:173-177 for the prompt); each chunk
    attends densely, every query over all prior + C keys under an additive
    causal mask (transformer.rs:139-148,180-196); the decode rows gather, pad,
    mask and run sdpa (transformer.rs:271-292).  Bounded sample: the chunk
    attention of all 8 sequences without copies, 16 timed pool copies
    (scaled to the 2,048 chunk rows), and the decode part with its 56
    copies; the sum is scaled x22 layers.  A lower bound of the reference:
    it has no prior-context prefill and would prefill each whole prompt."""
    import numpy as np
    import oracle
    from pagedkv import workload as wl

    kf = wl.widen(kp, wl.F16).astype(np.float32).reshape(kp.shape)
    vf = wl.widen(vp, wl.F16).astype(np.float32).reshape(vp.shape)
    hq, hk, hv = (wl.widen(x, wl.F16).astype(np.float32) for x in chunk_rows)
    dq, dk, dv = (wl.widen(x, wl.F16).astype(np.float32) for x in decode_rows)
    bs = kp.shape[1]
    cu = m.cu_q_lens
    t0 = time.time()
    for s_ in range(NP):
        rows = slice(int(cu[s_]), int(cu[s_ + 1]))
        oracle.prefill_chunk_faithful_f32(kf, vf, bs, tables[s_].astype(np.uint32), int(m.prior[s_]),
                                          hq[rows], hk[rows], hv[rows], scale, n_copies=0)
    t_attn = time.time() - t0
    rows0 = slice(int(cu[0]), int(cu[1]))
    n_cp = 16
    t0 = time.time()
    oracle.prefill_chunk_faithful_f32(kf, vf, bs, tables[0].astype(np.uint32), int(m.prior[0]),
                                      hq[rows0][:n_cp], hk[rows0][:n_cp], hv[rows0][:n_cp], scale,
                                      n_copies=n_cp)
    t_cp16 = time.time() - t0   # 16 pool copies + a 16-query attention
    t0 = time.time()
    oracle.prefill_chunk_faithful_f32(kf, vf, bs, tables[0].astype(np.uint32), int(m.prior[0]),
                                      hq[rows0][:n_cp], hk[rows0][:n_cp], hv[rows0][:n_cp], scale,
                                      n_copies=0)
    per_copy = max(0.0, t_cp16 - (time.time() - t0)) / n_cp
    seq = m.ctx.astype(np.int64)
    t0 = time.time()
    oracle.decode_step_faithful_f32(kf, vf, bs, tables[NP:].astype(np.uint32), seq, seq, dq, dk, dv,
                                    scale)
    t_dec = time.time() - t0
    layer_s = t_attn + NP * C * per_copy + t_dec
    log(f"[bench] cpu reference-faithful: chunk attention {t_attn:.2f} s, pool copy "
        f"{per_copy * 1e3:.1f} ms x {NP * C}, decode {t_dec:.2f} s -> {layer_s:.1f} s/layer")
    return {"value": round((NP * C + ND) / (layer_s * L), 4), "unit": "tok/s", "cores": 1,
            "host": host_cpu(), "kind": "port",
            "sample": (f"layer 0, f32 pool of {kf.nbytes >> 20} MiB per K: dense masked attention "
                       f"of the {NP} chunks ({t_attn:.1f} s), {n_cp} full K+V pool copies timed "
                       f"({per_copy * 1e3:.1f} ms each, x{NP * C} chunk rows), decode of {ND} "
                       f"rows with their pool copies ({t_dec:.1f} s); scaled x{L} layers")}


def churn(args, dev) -> dict:
    """block-manager churn on the Llama-3-8B KV shape
    (32 layers, 8 KV heads, hd 128, bs 16, bf16; 65,536 blocks = 128 GiB).
    Pool at 60% occupancy in sequences of U[1, 256] blocks (host allocator).
    One step: 512 copy-on-write block copies from seeded fork events
    (pkv_copy_blocks), eviction of a random 25% of sequences (host only),
    and compaction of the surviving blocks into a contiguous prefix under a
    random remap (pkv_compact, in place).  Reports device time and GB/s of
    the copy and compaction kernels (bytes moved counted twice: read+write)."""
    import numpy as np
    import torch

    import pagedkv
    from pagedkv import workload as wl

    L, KVH, hd, bs, N = 32, 8, 128, 16, 65536
    cache = pagedkv.PagedKvCache(L, N, bs, KVH, hd, torch.bfloat16)
    cache.fill_normal(args.seed)
    alloc = pagedkv.BlockAllocator(N, bs)
    target = int(0.6 * N)
    seqs, live, i = [], 0, 0
    while live < target:
        nb = int(wl.randint(args.seed + i, 1, 1, 256)[0])
        nb = min(nb, target - live)
        t = pagedkv.BlockTable()
        alloc.ensure_capacity(t, nb * bs)
        seqs.append(t)
        live += nb
        i += 1
    # fork events: a random block of a random (pre-fork) sequence is copied to
    # a fresh block; no destination is also a source (the CoW contract)
    r = wl.splitmix64(args.seed ^ 0xF04C, 2 * 512)
    src, dst = [], []
    n_parents = len(seqs)
    for k in range(512):
        t = seqs[int(r[2 * k] % np.uint64(n_parents))]
        blocks = t.blocks
        src.append(blocks[int(r[2 * k + 1] % np.uint64(len(blocks)))])
        child = pagedkv.BlockTable()
        alloc.ensure_capacity(child, bs)
        dst.append(child.blocks[0])
        seqs.append(child)
    s_t = torch.tensor(src, dtype=torch.int32, device=dev)
    d_t = torch.tensor(dst, dtype=torch.int32, device=dev)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for _ in range(max(1, args.warmup)):
        cache.copy_blocks(s_t, d_t)  # idempotent: same src -> same dst
    torch.cuda.synchronize()
    reps = max(1, args.steps)
    cache.profile(True)
    e0.record()
    for _ in range(reps):
        cache.copy_blocks(s_t, d_t)
    e1.record()
    torch.cuda.synchronize()
    cow_ms = e0.elapsed_time(e1) / reps
    cow_kms, cow_n = cache.profile_read()
    cow_kms /= max(1, cow_n)
    cow_bytes = 2 * 512 * cache.block_bytes * 2 * L
    cache.check()
    # validation (untimed): every live block, copies included, holds the
    # bytes the fill wrote into its original block
    origin = np.arange(N, dtype=np.int32)
    origin[np.asarray(dst)] = origin[np.asarray(src)]
    live_ids = np.concatenate([np.array(t.blocks, np.int32) for t in seqs if len(t)])
    t0 = time.time()
    bad_cow = cache.verify_normal(args.seed, live_ids, origin[live_ids])
    verify_s = time.time() - t0
    # eviction of a random 25% of sequences
    order = wl.permutation(args.seed ^ 0xE51C, len(seqs))
    n_evict = len(seqs) // 4
    for j in order[:n_evict]:
        alloc.release(seqs[j])
    survivors = [seqs[j] for j in order[n_evict:]]
    surv = np.concatenate([np.array(t.blocks, np.int32) for t in survivors if len(t)])
    n_surv = surv.size
    remap = wl.permutation(args.seed ^ 0xC0DE, n_surv).astype(np.int32)
    # warm-up: move one free block onto another (loads the kernel; no live data moves)
    free_ids = np.setdiff1d(np.arange(N, dtype=np.int32), surv)
    cache.compact(free_ids[:1], free_ids[1:2])
    torch.cuda.synchronize()
    cache.profile_read()
    # compaction forward (survivors -> remap) and back, alternately: every
    # call moves the same blocks; the average covers host planning, plan
    # upload and kernel of one call
    comp_reps = max(2, reps)
    comp_ms = comp_wall_ms = 0.0
    for k in range(comp_reps):
        a_, b_ = (surv, remap) if k % 2 == 0 else (remap, surv)
        torch.cuda.synchronize()
        t0 = time.time()
        e0.record()
        cache.compact(a_, b_)
        e1.record()
        torch.cuda.synchronize()
        comp_wall_ms += (time.time() - t0) * 1e3
        comp_ms += e0.elapsed_time(e1)
    comp_ms /= comp_reps
    comp_wall_ms /= comp_reps
    comp_kms, comp_n = cache.profile_read()
    comp_kms /= max(1, comp_n)
    cache.profile(False)
    if comp_reps % 2 == 0:
        cache.compact(surv, remap)  # untimed: end on a forward compaction
    moved = int((surv != remap).sum())
    comp_bytes = 2 * moved * cache.block_bytes * 2 * L
    cache.check()
    # validation (untimed): block remap[i] holds what survivor surv[i] held
    t0 = time.time()
    bad_comp = cache.verify_normal(args.seed, remap, origin[surv])
    verify_s += time.time() - t0
    validation = {"validated": bad_cow == 0 and bad_comp == 0,
                  "mismatches": int(bad_cow + bad_comp),
                  "blocks_checked": int(live_ids.size + remap.size),
                  "method": "device recomputation of every live block's fill bytes "
                            "(counter hash of seed, layer, K/V, original block, element) "
                            "after the CoW copies and after compaction",
                  "seconds": round(verify_s, 2)}
    log(f"[bench] cfg5 validation: {validation['mismatches']} mismatching 16-byte chunks in "
        f"{validation['blocks_checked']} blocks x {2 * L} slabs ({verify_s:.1f} s)")
    step_ms = cow_ms + comp_ms
    log(f"[bench] cfg5: CoW {cow_ms:.3f} ms ({cow_bytes / (cow_ms / 1e3) / 1e9:.0f} GB/s), "
        f"compaction {comp_ms:.2f} ms incl. host plan + upload, kernel {comp_kms:.2f} ms "
        f"({comp_bytes / (comp_kms / 1e3) / 1e9:.0f} GB/s)")

    traffic = None
    prof = os.path.join(ROOT, "profiles", "churn_cfg5_traffic.json")
    if os.path.exists(prof):
        with open(prof) as f:
            tr = json.load(f)
        if tr.get("seed") == args.seed:
            traffic = tr.get("bytes_per_launch")

    cpu = None
    if args.cpu_layers > 0:
        cpu = churn_cpu_baseline(cache, args)

    res = {
        "metric": "block churn: copy-on-write + compaction GB/s (bytes moved x2), Llama-3-8B KV, 1 GPU",
        "value": round((cow_bytes + comp_bytes) / (step_ms / 1e3) / 1e9, 1), "unit": "GB/s",
        "n_gpus": 1, "steps": reps, "warmup": max(1, args.warmup), "ms_per_step": round(step_ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) pool, seeded fork/evict/remap events)",
        "config": {"workload": "cfg5: 32 layers x 8 kv heads x hd 128, bs 16, bf16, 65536 blocks, "
                               "60% occupancy, 512 CoW copies, 25% eviction, compaction",
                   "live_blocks": live, "sequences": len(seqs), "survivor_blocks": int(n_surv),
                   "seed": args.seed, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(comp_bytes / (comp_kms / 1e3) / 1e9, 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(comp_bytes / (comp_kms / 1e3) / 1e9 / HBM_PEAK_GBPS, 4),
                     "traffic": traffic, "kernel": "pkv::compact_kernel",
                     "kernel_avg_us": round(comp_kms * 1e3, 1),
                     "algorithmic_bytes_per_launch": comp_bytes},
        "validation": validation,
        "cow": {"copies": 512, "ms": round(cow_ms, 4), "kernel_ms": round(cow_kms, 4),
                "GBps": round(cow_bytes / (cow_ms / 1e3) / 1e9, 1)},
        "compaction": {"moved_blocks": moved, "calls": comp_reps,
                       "ms_incl_host_plan_and_upload": round(comp_ms, 3),
                       "ms_wall_incl_plan": round(comp_wall_ms, 3), "kernel_ms": round(comp_kms, 3),
                       "GBps": round(comp_bytes / (comp_ms / 1e3) / 1e9, 1)},
        "cpu_baseline": cpu,
    }
    cache.close()
    return res


def churn_cpu_baseline(cache, args):
    """The oracle's closed-form compaction (memcpy of every moved block, K
    and V; single thread) on a 1-layer, 8,192-block pool of the same block
    shape with a 45 % survivor remap like cfg5's, repeated for a bounded
    sample; GB/s counts bytes moved x2 as the GPU figure does."""
    import numpy as np
    import oracle
    from pagedkv import workload as wl

    nb = 8192
    bb = cache.block_bytes
    pool = np.zeros(2 * nb * bb, dtype=np.uint8)
    pool[::4096] = 1
    perm = wl.permutation(args.seed ^ 0xCB, nb)
    n_surv = int(nb * 0.6 * 0.75)
    src = perm[:n_surv].astype(np.int32)
    dst = wl.permutation(args.seed ^ 0xCD, n_surv).astype(np.int32)
    oracle.lib()
    dt, passes, _ = timed_passes(lambda: oracle.compact(pool, 1, bb, src, dst), args)
    moved = int((src != dst).sum())
    gbps = 2 * moved * bb * 2 / dt / 1e9
    log(f"[bench] cpu baseline: compaction of {moved} blocks in {dt * 1e3:.1f} ms -> {gbps:.2f} GB/s")
    return {"value": round(gbps, 2), "unit": "GB/s", "cores": 1, "host": host_cpu(), "kind": "port",
            "sample": (f"closed-form compaction (memcpy) of {moved} of 8192 blocks, 1 layer K+V, "
                       f"{passes} passes of {dt * 1e3:.1f} ms")}


if __name__ == "__main__":
    sys.exit(main())
