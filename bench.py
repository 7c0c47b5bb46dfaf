"""FlexAttention benchmark on one MI355X.

    python bench.py [--steps K] [--warmup W] [--config ns|c2|c3|c4|c5|decode] [--others c2,c3,c4,c5] [--no-cpu]

The headline workload (default ns) is causal attention B4 H32 S8192 D128 in
bf16, the shape the 50 % / 35 % targets are set on; the other workloads
(C2 causal S2048, C3 sliding window, C4 GQA + ALiBi + soft-cap, C5 packed
documents) are timed after it and reported as extra keys.
A step is one forward + backward pass (fa_fwd and fa_bwd through the C ABI,
outputs preallocated, inputs resident in HBM) over one batch of synthetic
inputs; for these bf16 workloads fa_bwd is two launches (the dQ kernel, which
also computes Delta = rowsum(O dO), then dK/dV).  Throughput counts only
unmasked (query, key) pairs P per (batch, head): fwd 4*D*P, bwd 10*D*P,
fwd+bwd 14*D*P FLOPs (recomputation is not credited).

Prints ONE JSON line.  ``value`` is the fwd+bwd effective TFLOP/s; the line
also carries the forward figure, per-kernel times, the public
``flex_attention`` forward + autograd backward time on the same inputs, the
roofline of the dominant kernel (HIP events on the launch stream; HBM bytes
per launch from profiles/traffic.json only when that file was measured on the
current kernel sources) and the CPU baseline: the oracle's C restatement of
the reference's tiled algorithm, timed on a bounded sample of heads of the
same workload on this host.  ``gemm_reference`` times torch's bf16 GEMM
(hipBLASLt, 8192^3) on the same GPU in the same run: the board runs at its
power limit under sustained matrix-core load, so that figure is the practical
ceiling the attention figures are read against.  ``--power`` samples socket
power and GFX clocks (amd-smi) while each kernel runs back to back.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "pallas-flexattn_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np  # noqa: E402

METRIC = "effective TFLOP/s fwd and fwd+bwd (unmasked FLOPs), % of bf16 MFMA peak"
PEAK_BF16_TFLOPS = 2516.6  # MI355X dense bf16 MFMA: 256 CU x 4 SIMD x 1024 FLOP/clk x 2.4 GHz ("2.5 PFLOP/s")
PEAK_FP8_TFLOPS = 5033.2   # dense fp8 MFMA, twice the bf16 rate ("5.0 PFLOP/s")


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def doc_lengths(rng, S):
    out, tot = [], 0
    while tot < S:
        n = int(rng.integers(256, 4097))
        n = min(n, S - tot)
        out.append(n)
        tot += n
    return out


def make_config(name):
    """Workload definitions (shapes, masks, score mods, seeds)."""
    import pallas_flexattn as pf
    if name == "c2":
        return dict(workload="causal fwd+bwd B8 H16 S2048 D128 bf16 (q,k,v ~ 0.5*N(0,1))", B=8, Hq=16, Hkv=16,
                    S=2048, D=128, seed=1, scale_in=0.5, mask=pf.causal_mask, window=(-1, 0), docs=None,
                    score=None)
    if name == "c3":
        return dict(workload="sliding-window-1024 causal fwd+bwd B4 H32 S8192 D128 bf16", B=4, Hq=32, Hkv=32,
                    S=8192, D=128, seed=2, scale_in=1.0, mask=pf.sliding_window_mask(1023, 0),
                    window=(1023, 0), docs=None, score=None)
    if name == "c4":
        return dict(workload="GQA causal + ALiBi + softcap50 fwd+bwd B4 Hq32 Hkv8 S4096 D128 bf16", B=4, Hq=32,
                    Hkv=8, S=4096, D=128, seed=3, scale_in=1.0, mask=pf.causal_mask, window=(-1, 0), docs=None,
                    score=pf.compose_score_mods(pf.alibi_score_mod(32), pf.softcap_score_mod(50.0)))
    if name == "c5":
        rng = np.random.default_rng(4)
        lens = [doc_lengths(rng, 16384) for _ in range(2)]
        dm = pf.document_mask(lens)
        return dict(workload="packed-document causal fwd+bwd B2 H16 S16384 D128 bf16", B=2, Hq=16, Hkv=16,
                    S=16384, D=128, seed=4, scale_in=1.0, mask=pf.and_masks(dm, pf.causal_mask), window=(-1, 0),
                    docs=dm.doc_ids, score=None)
    if name == "ns":
        return dict(workload="causal fwd+bwd B4 H32 S8192 D128 bf16", B=4, Hq=32, Hkv=32, S=8192, D=128, seed=5,
                    scale_in=1.0, mask=pf.causal_mask, window=(-1, 0), docs=None, score=None)
    raise SystemExit(f"unknown config {name}")


def count_pairs(cfg):
    """Unmasked (q, k) pairs summed over batch rows, per head (exact)."""
    S = cfg["S"]
    left, right = cfg["window"]
    q = np.arange(S, dtype=np.int64)
    lo = np.zeros(S, np.int64) if left < 0 else np.maximum(q - left, 0)
    hi = np.full(S, S - 1, np.int64) if right < 0 else np.minimum(q + right, S - 1)
    if cfg["docs"] is None:
        return int(np.sum(hi - lo + 1)) * cfg["B"]
    total = 0
    for b in range(cfg["B"]):
        d = cfg["docs"][min(b, cfg["docs"].shape[0] - 1)]
        starts = np.searchsorted(d, d, side="left")
        ends = np.searchsorted(d, d, side="right") - 1
        a, z = np.maximum(lo, starts), np.minimum(hi, ends)
        total += int(np.sum(np.maximum(z - a + 1, 0)))
    return total


def gen_inputs(cfg):
    rng = np.random.default_rng(cfg["seed"])
    B, Hq, Hkv, S, D = cfg["B"], cfg["Hq"], cfg["Hkv"], cfg["S"], cfg["D"]
    q = rng.standard_normal((B, Hq, S, D), dtype=np.float32) * cfg["scale_in"]
    k = rng.standard_normal((B, Hkv, S, D), dtype=np.float32) * cfg["scale_in"]
    v = rng.standard_normal((B, Hkv, S, D), dtype=np.float32) * cfg["scale_in"]
    do = rng.standard_normal((B, Hq, S, D), dtype=np.float32)
    return q, k, v, do


def time_region(fn, iters, stream):
    import torch
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(iters):
        fn()
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) / iters


def cpu_baseline(cfg, arrays, pairs_per_head, target_s):
    """The oracle's C restatement of the reference's tiled fwd + 3-kernel bwd
    (every tile computed, as the reference does), on a bounded sample of
    (batch, head) programs."""
    from oracle import tiled
    from oracle.bf16 import round_bf16
    B, Hq, S, D = cfg["B"], cfg["Hq"], cfg["S"], cfg["D"]
    if cfg["Hq"] != cfg["Hkv"] or cfg["score"] is not None or cfg["docs"] is not None:
        return None  # the reference algorithm has no GQA / score mods / document masks
    q, k, v, do = (round_bf16(a) for a in arrays)
    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or os.cpu_count() or 1
    threads = min(threads, os.cpu_count() or threads)

    def run(nh):
        t0 = time.perf_counter()
        o, lse = tiled.fwd(q, k, v, 128, 64, window=cfg["window"], bf16=True, nthreads=threads, bh_range=(0, nh))
        tiled.bwd(q, k, v, o, lse, do, 128, 64, window=cfg["window"], bf16=True, nthreads=threads,
                  bh_range=(0, nh))
        return time.perf_counter() - t0

    t1 = run(min(threads, B * Hq))
    per_head = t1 / min(threads, B * Hq)
    nh = int(max(1, min(B * Hq, target_s / max(per_head, 1e-6))))
    nh = max(min(threads, B * Hq), (nh // threads) * threads) if nh >= threads else nh
    t = run(nh)
    flops = 14.0 * D * pairs_per_head * nh / B  # pairs_per_head sums over batch rows
    return {"value": flops / t / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"{nh} of {B * Hq} (batch, head) programs, fwd + 3-kernel bwd over all tiles, "
                      f"{t:.1f} s; same unmasked-FLOP count as the GPU value"}


def bench_decode(args):
    """Decoding-shaped forward: one query per (batch, q head) against a long
    KV cache, bf16, no mask (B8 Hq32 Hkv8 Skv32768 D128).  HBM-bound: the
    metric is KV-cache bytes read per second by split-KV flex_decode (the
    query heads of each GQA group packed into one tile, so K / V are read once
    per group), next to the same cache paged (64 pages of 512 keys per row,
    shuffled) and the unsplit forward."""
    import torch
    import pallas_flexattn as pf
    B, Hq, Hkv, Sq, Skv, D = 8, 32, 8, 1, 32768, 128
    g = torch.Generator(device="cuda").manual_seed(6)
    q = torch.randn(B, Hq, Sq, D, device="cuda", generator=g).to(torch.bfloat16)
    k = torch.randn(B, Hkv, Skv, D, device="cuda", generator=g).to(torch.bfloat16)
    v = torch.randn(B, Hkv, Skv, D, device="cuda", generator=g).to(torch.bfloat16)
    ps = 512
    npg = Skv // ps
    perm = torch.randperm(B * npg, generator=torch.Generator().manual_seed(7)).view(B, npg).to(torch.int32)
    kc = k.view(B, Hkv, npg, ps, D).permute(0, 2, 1, 3, 4).reshape(B * npg, Hkv, ps, D)[perm.view(-1).argsort()]
    vc = v.view(B, Hkv, npg, ps, D).permute(0, 2, 1, 3, 4).reshape(B * npg, Hkv, ps, D)[perm.view(-1).argsort()]
    kc, vc = kc.contiguous(), vc.contiguous()
    pt = perm.cuda()
    stream = torch.cuda.current_stream()
    split = lambda: pf.flex_decode(q, k, v, enable_gqa=True)  # noqa: E731
    paged = lambda: pf.flex_decode(q, kc, vc, enable_gqa=True, page_table=pt)  # noqa: E731
    plain = lambda: pf.flex_attention(q, k, v, enable_gqa=True)  # noqa: E731
    o_s, o_p = split(), paged()
    torch.cuda.synchronize()
    if not torch.equal(o_s, o_p):
        raise SystemExit("paged and contiguous decode differ")
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < 0.5:
        split()
        paged()
        plain()
        torch.cuda.synchronize()
    ms_split = time_region(split, args.steps, stream)
    ms_paged = time_region(paged, args.steps, stream)
    ms_plain = time_region(plain, args.steps, stream)
    kv_bytes = 2.0 * B * Hkv * Skv * D * 2
    gbs = kv_bytes / (ms_split * 1e-3) / 1e9
    out = {
        "metric": "KV-cache read bandwidth, decode forward (split-KV)", "value": round(gbs, 1), "unit": "GB/s",
        "n_gpus": 1, "steps": args.steps, "ms_per_step": round(ms_split, 4), "higher_is_better": True,
        "dtype": "bf16", "data": "synthetic (torch normals rounded to bf16)",
        "config": {"workload": "decode B8 Hq32 Hkv8 Sq1 Skv32768 D128 bf16, no mask", "B": B, "Hq": Hq, "Hkv": Hkv,
                   "Sq": Sq, "Skv": Skv, "D": D},
        "paged_ms": round(ms_paged, 4), "paged_gbs": round(kv_bytes / (ms_paged * 1e-3) / 1e9, 1),
        "page_size": ps,
        "unsplit_forward_ms": round(ms_plain, 4),
        "roofline": {"kernel": "fwd (split-KV, GQA-packed) + merge", "bound": "hbm", "achieved": round(gbs, 1),
                     "peak": 8000.0, "unit": "GB/s", "frac": round(gbs / 8000.0, 4), "traffic": None},
    }
    print(json.dumps(out), flush=True)


def sources_sha256():
    """Hash of the HIP sources and the C ABI header: identifies the kernels a
    counter measurement was taken on."""
    import hashlib
    h = hashlib.sha256()
    csrc = os.path.join(ROOT, "pallas-flexattn_amd", "csrc")
    for name in sorted(os.listdir(csrc)):
        if name.endswith((".h", ".hip")):
            with open(os.path.join(csrc, name), "rb") as f:
                h.update(name.encode() + b"\0" + f.read())
    with open(os.path.join(ROOT, "include", "flexattn.h"), "rb") as f:
        h.update(f.read())
    return h.hexdigest()


def gemm_reference(steps, stream):
    """The bf16 GEMM torch runs through hipBLASLt, 8192 x 8192 x 8192, timed the
    same way on the same GPU: what a plain library GEMM reaches on this board
    under its power limit, next to the attention kernels."""
    import torch
    n = 8192
    a = torch.randn(n, n, device="cuda", dtype=torch.bfloat16)
    b = torch.randn(n, n, device="cuda", dtype=torch.bfloat16)
    c = torch.empty(n, n, device="cuda", dtype=torch.bfloat16)
    fn = lambda: torch.matmul(a, b, out=c)  # noqa: E731
    warm(fn, min_s=0.2)
    ms = time_region(fn, steps, stream)
    tf = 2.0 * n ** 3 / (ms * 1e-3) / 1e12
    return {"workload": "bf16 GEMM 8192 x 8192 x 8192 (torch.matmul, hipBLASLt)", "ms": round(ms, 4),
            "tflops": round(tf, 2), "pct_peak": round(100 * tf / PEAK_BF16_TFLOPS, 2)}


def amd_smi_sample():
    """(socket power W, mean GFX clock MHz over the XCDs) from one amd-smi
    reading, or None."""
    import re
    import subprocess
    try:
        out = subprocess.run(["amd-smi", "metric", "-p", "-c"], capture_output=True, text=True, timeout=10).stdout
    except (OSError, subprocess.SubprocessError):
        return None
    pw = re.search(r"SOCKET_POWER:\s*([0-9.]+)\s*W", out)
    clks, in_gfx = [], False
    for line in out.splitlines():
        t = line.strip()
        if re.match(r"GFX_\d+:", t):
            in_gfx = True
        elif in_gfx and t.startswith("CLK:"):
            m = re.match(r"CLK:\s*([0-9.]+)\s*MHz", t)
            if m:
                clks.append(float(m.group(1)))
            in_gfx = False
    if not pw or not clks:
        return None
    return float(pw.group(1)), sum(clks) / len(clks)


def power_profile(fns, seconds=2.5):
    """Runs each (name, fn) back to back for `seconds` while amd-smi samples the
    socket power and GFX clocks; the first 0.8 s (clock ramp) is left out.
    Returns {name: {"watts": median, "mhz": median, "samples": n, "ms": per call}}."""
    import threading
    import torch
    res = {}
    for name, fn in fns:
        samples, stop = [], [False]

        def sampler():
            while not stop[0]:
                t = time.perf_counter()
                s = amd_smi_sample()
                if s is not None:
                    samples.append((t, s))
                time.sleep(0.05)

        th = threading.Thread(target=sampler)
        t0 = time.perf_counter()
        th.start()
        n = 0
        while time.perf_counter() - t0 < seconds:
            fn()
            n += 1
            if n % 4 == 0:
                torch.cuda.synchronize()
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        stop[0] = True
        th.join()
        vals = [s for t, s in samples if t0 + 0.8 < t < t1]
        if vals:
            w = sorted(v[0] for v in vals)[len(vals) // 2]
            mhz = sorted(v[1] for v in vals)[len(vals) // 2]
            res[name] = {"watts": w, "mhz": round(mhz), "samples": len(vals), "ms": round((t1 - t0) * 1e3 / n, 4)}
        else:
            res[name] = {"watts": None, "mhz": None, "samples": 0, "ms": round((t1 - t0) * 1e3 / n, 4)}
        log(f"power {name}: {res[name]}")
    return res


def measured_traffic(config, kernel):
    """HBM bytes per launch of `kernel` at `config` from profiles/traffic.json,
    only if it was measured on the current kernel sources (else None)."""
    tpath = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(tpath):
        return None
    with open(tpath) as f:
        table = json.load(f)
    if table.get("sources_sha256") != sources_sha256():
        return None
    return table.get(f"{config}/{kernel}")


def warm(fn, min_steps=3, min_s=0.5):
    """Untimed steps until the GPU clock has settled (at least min_steps and
    min_s seconds); returns the count."""
    import torch
    n, t0 = 0, time.perf_counter()
    while n < min_steps or time.perf_counter() - t0 < min_s:
        fn()
        n += 1
        if n % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    return n


def setup(name, dev, numpy_inputs):
    """Inputs (bf16 on the GPU), the device-built block mask and a Runner for a
    workload.  numpy_inputs: seeded numpy normals (as the CPU baseline uses);
    otherwise torch normals drawn on the GPU with the same seed (same
    distribution, no host round trip)."""
    import torch
    import pallas_flexattn as pf
    from pallas_flexattn.flash_attn import Runner
    cfg = make_config(name)
    B, Hq, Hkv, S, D = cfg["B"], cfg["Hq"], cfg["Hkv"], cfg["S"], cfg["D"]
    arrays = None
    if numpy_inputs:
        arrays = gen_inputs(cfg)
        tq, tk, tv, tdo = (torch.from_numpy(a).to(dev, torch.bfloat16) for a in arrays)
    else:
        g = torch.Generator(device=dev).manual_seed(cfg["seed"])
        sc = cfg["scale_in"]
        tq, tk, tv = ((torch.randn(B, h, S, D, device=dev, generator=g) * sc).to(torch.bfloat16)
                      for h in (Hq, Hkv, Hkv))
        tdo = torch.randn(B, Hq, S, D, device=dev, generator=g).to(torch.bfloat16)
    bmask = pf.create_block_mask(cfg["mask"], B, Hq, S, S, 128, device=dev)
    runner = Runner(tq, tk, tv, tdo, score_mod=cfg["score"], block_mask=bmask)
    return cfg, arrays, (tq, tk, tv, tdo), bmask, runner


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=None,
                    help="untimed warm-up steps (default: at least 3 steps and 0.5 s, so the GPU clock has "
                         "settled before the timed steps; the count used is reported)")
    ap.add_argument("--config", default="ns",
                    help="headline workload: ns (causal B4 H32 S8192 D128, default), c2, c3, c4, c5, decode")
    ap.add_argument("--others", default="c2,c3,c4,c5",
                    help="further workloads reported as extra keys (fwd and fwd+bwd TFLOP/s); '' for none")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--profile-kernel", choices=("fwd", "dkdv", "dq", "bwd", "copy"), default=None,
                    help="run only this kernel --profile-iters times and exit (for rocprofv3 counter passes; "
                         "bwd = fa_bwd, the dQ kernel with Delta fused then dK/dV; "
                         "copy = a 256 MiB device copy used to calibrate FETCH_SIZE / WRITE_SIZE)")
    ap.add_argument("--profile-iters", type=int, default=3)
    ap.add_argument("--power", action="store_true",
                    help="run the forward, dK/dV, dQ, the whole step and a bf16 GEMM back to back for a few "
                         "seconds each while amd-smi samples socket power and GFX clocks; print them and exit")
    ap.add_argument("--dense-ref", action="store_true",
                    help="also time the headline shape with no mask (every tile live) and report the time "
                         "fraction next to the live-block fraction (sparse-proportionality check)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one MI355X: --gpus {args.gpus} is not supported (run with --gpus 1)",
              file=sys.stderr)
        sys.exit(2)

    import torch
    import pallas_flexattn as pf
    from pallas_flexattn.flash_attn import Runner

    if args.config == "decode":
        bench_decode(args)
        return

    if args.profile_kernel == "copy":
        src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(args.profile_iters):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"profile: {args.profile_iters} copies of 256 MiB")
        return

    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    cfg, arrays, (tq, tk, tv, tdo), bmask, runner = setup(args.config, dev, numpy_inputs=not args.no_cpu)
    B, Hq, Hkv, S, D = cfg["B"], cfg["Hq"], cfg["Hkv"], cfg["S"], cfg["D"]
    log(f"config {args.config}: {cfg['workload']}")
    pairs = count_pairs(cfg)  # per head, summed over batch rows
    flop_fwd = 4.0 * D * pairs * Hq
    flop_bwd = 10.0 * D * pairs * Hq

    if args.power:
        import torch
        n = 8192
        ga = torch.randn(n, n, device="cuda", dtype=torch.bfloat16)
        gb = torch.randn(n, n, device="cuda", dtype=torch.bfloat16)
        gc = torch.empty(n, n, device="cuda", dtype=torch.bfloat16)
        runner.fwd()
        runner.preprocess()
        idle = [amd_smi_sample() for _ in range(5)]
        idle = [x for x in idle if x]
        res = power_profile((("fwd", runner.fwd), ("bwd_dkdv", runner.dkdv), ("bwd_dq", runner.dq_),
                             ("step", runner.step), ("gemm_bf16_8192", lambda: torch.matmul(ga, gb, out=gc))))
        flops = {"fwd": flop_fwd, "bwd_dkdv": 8.0 * D * pairs * Hq, "bwd_dq": 6.0 * D * pairs * Hq,
                 "step": flop_fwd + flop_bwd, "gemm_bf16_8192": 2.0 * n ** 3}
        for k, v in res.items():
            v["tflops"] = round(flops[k] / (v["ms"] * 1e-3) / 1e12, 1)
            v["pct_peak"] = round(100 * v["tflops"] / PEAK_BF16_TFLOPS, 2)
        print(json.dumps({"config": cfg["workload"], "idle": {"watts": idle[0][0] if idle else None,
                                                              "mhz": round(idle[0][1]) if idle else None},
                          "kernels": res}))
        return

    if args.profile_kernel:
        runner.fwd()
        runner.preprocess()
        fn = {"fwd": runner.fwd, "dkdv": runner.dkdv, "dq": runner.dq_, "bwd": runner.bwd}[args.profile_kernel]
        for _ in range(args.profile_iters):
            fn()
        torch.cuda.synchronize()
        log(f"profile: {args.profile_kernel} x {args.profile_iters} on {args.config}")
        return

    # block mask build: on the host and on the GPU (median of 5 device builds,
    # each ending in the copy of the tables to the host), bit-identical
    t0 = time.perf_counter()
    host_bmask = pf.create_block_mask(cfg["mask"], B, Hq, S, S, 128)
    mask_host_ms = (time.perf_counter() - t0) * 1e3
    builds = []
    for _ in range(5):
        t0 = time.perf_counter()
        pf.create_block_mask(cfg["mask"], B, Hq, S, S, 128, device=dev)
        builds.append((time.perf_counter() - t0) * 1e3)
    mask_ms = sorted(builds)[2]
    if not all(np.array_equal(getattr(bmask, f), getattr(host_bmask, f))
               for f in ("num_blocks_in_row", "col_indices", "kv_num_blocks", "kv_indices", "full_kv_num_blocks",
                         "full_kv_indices", "q_num_blocks", "q_indices", "full_q_num_blocks", "full_q_indices")):
        raise SystemExit("device and host block masks differ")

    # per-kernel times: the forward, the whole backward, and the staged
    # kernels (Delta pass, dK/dV, dQ reading Delta), each after its own short
    # warm-up; the dQ kernel with Delta fused takes about bwd - bwd_dkdv.
    # They run before the headline steps, so those start on a GPU whose clock
    # has left its idle state, as in a training loop.
    kernels = {}
    for name, fn in (("fwd", runner.fwd), ("bwd", runner.bwd), ("bwd_preprocess", runner.preprocess),
                     ("bwd_dkdv", runner.dkdv), ("bwd_dq", runner.dq_)):
        warm(fn, min_steps=2, min_s=0.05)
        kernels[name] = time_region(fn, args.steps, stream)
    ms_fwd = kernels["fwd"]
    algo = {"fwd": flop_fwd, "bwd_dkdv": 8.0 * D * pairs * Hq, "bwd_dq": 6.0 * D * pairs * Hq}
    dom = max(("fwd", "bwd_dkdv", "bwd_dq"), key=lambda n: kernels[n])
    achieved = algo[dom] / (kernels[dom] * 1e-3) / 1e12
    fwd_tflops = flop_fwd / (ms_fwd * 1e-3) / 1e12

    # the public API on the same inputs: flex_attention forward + autograd
    # backward (plans, tables and device arrays cached after the first call)
    qq, kk, vv = (t.detach().requires_grad_() for t in (tq, tk, tv))

    def api_step():
        o = pf.flex_attention(qq, kk, vv, score_mod=cfg["score"], block_mask=bmask, enable_gqa=Hq != Hkv)
        torch.autograd.grad(o, (qq, kk, vv), tdo)

    warm(api_step, min_s=0.1)
    api_ms = time_region(api_step, args.steps, stream)
    del qq, kk, vv

    # the headline: W untimed steps, then exactly K timed steps
    if args.warmup is None:
        args.warmup = warm(runner.step)
    else:
        for _ in range(args.warmup):
            runner.step()
    torch.cuda.synchronize()
    log(f"warmup done ({args.warmup} steps)")
    ms_step = time_region(runner.step, args.steps, stream)
    torch.cuda.synchronize()
    log(f"timed {args.steps} steps: {ms_step:.3f} ms/step")
    fwdbwd_tflops = (flop_fwd + flop_bwd) / (ms_step * 1e-3) / 1e12
    log(f"flex_attention fwd+bwd: {api_ms:.3f} ms/step (Runner {ms_step:.3f})")

    # the fp8 forward on the same workload: q, k, v quantised once (timed
    # apart), then the fp8 kernel alone, inputs resident in HBM
    fp8 = None
    if D in (64, 128):
        from pallas_flexattn.fp8 import Fp8Runner, quantize_fp8

        def quant():
            return quantize_fp8(tq), quantize_fp8(tk), quantize_fp8(tv, transpose=True)

        q8, k8, v8 = quant()
        warm(quant, min_s=0.1)
        quant_ms = time_region(quant, args.steps, stream)
        fr = Fp8Runner(q8, k8, v8, score_mod=cfg["score"], block_mask=bmask, enable_gqa=Hq != Hkv)
        warm(fr.fwd, min_s=0.2)
        fp8_ms = time_region(fr.fwd, args.steps, stream)
        fp8_tflops = flop_fwd / (fp8_ms * 1e-3) / 1e12
        fp8 = {"workload": cfg["workload"].replace("fwd+bwd", "fwd").replace("bf16", "fp8 e4m3 (128-row block scales)"),
               "ms": round(fp8_ms, 4), "tflops": round(fp8_tflops, 2),
               "pct_fp8_peak": round(100 * fp8_tflops / PEAK_FP8_TFLOPS, 2), "peak_tflops": PEAK_FP8_TFLOPS,
               "speedup_vs_bf16_fwd": round(ms_fwd / fp8_ms, 3), "quantize_qkv_ms": round(quant_ms, 4)}
        log(f"fp8 forward: {fp8_ms:.3f} ms ({fp8_tflops:.1f} TFLOP/s, {ms_fwd / fp8_ms:.2f}x bf16); "
            f"quantise q, k, v {quant_ms:.3f} ms")
        del fr, q8, k8, v8

    sparsity = None
    if args.dense_ref:
        dense = Runner(tq, tk, tv, tdo, score_mod=cfg["score"])
        warm(dense.step, min_s=0.1)
        dense_ms = time_region(dense.step, args.steps, stream)
        del dense
        live = 1.0 - bmask.sparsity
        sparsity = {"live_block_fraction": round(live, 4), "dense_ms_per_step": round(dense_ms, 4),
                    "time_fraction": round(ms_step / dense_ms, 4)}
        log(f"dense reference {dense_ms:.3f} ms/step; time fraction {ms_step / dense_ms:.3f} vs live blocks {live:.3f}")

    cpu = None
    if not args.no_cpu:
        log("cpu baseline ...")
        cpu = cpu_baseline(cfg, arrays, pairs, args.cpu_seconds)
        log("cpu baseline done")
    del arrays, runner, tq, tk, tv, tdo

    others = {}
    for name in [n for n in args.others.split(",") if n and n != args.config]:
        ocfg, _, _, obm, orun = setup(name, dev, numpy_inputs=False)
        warm(orun.step, min_s=0.1)
        oms = time_region(orun.step, args.steps, stream)
        orun.fwd()
        ofwd = time_region(orun.fwd, args.steps, stream)
        opairs = count_pairs(ocfg)
        of, ob = 4.0 * ocfg["D"] * opairs * ocfg["Hq"], 10.0 * ocfg["D"] * opairs * ocfg["Hq"]
        others[name] = {"workload": ocfg["workload"], "ms_per_step": round(oms, 4), "fwd_ms": round(ofwd, 4),
                        "fwdbwd_tflops": round((of + ob) / (oms * 1e-3) / 1e12, 2),
                        "fwdbwd_pct_peak": round(100 * (of + ob) / (oms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 2),
                        "fwd_tflops": round(of / (ofwd * 1e-3) / 1e12, 2),
                        "fwd_pct_peak": round(100 * of / (ofwd * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 2),
                        "live_block_fraction": round(1.0 - obm.sparsity, 4)}
        log(f"{name}: {others[name]['fwdbwd_tflops']} TFLOP/s fwd+bwd, {others[name]['fwd_tflops']} fwd")
        del orun, obm
        torch.cuda.empty_cache()

    gemm = gemm_reference(args.steps, stream) if not args.profile_kernel else None
    log(f"bf16 GEMM reference: {gemm['tflops']} TFLOP/s ({gemm['pct_peak']} % of peak)")

    out = {
        "metric": METRIC,
        "value": round(fwdbwd_tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded normals rounded to bf16)",
        "config": {"workload": cfg["workload"], "B": B, "Hq": Hq, "Hkv": Hkv, "S": S, "D": D,
                   "mask_block": 128, "live_tiles": bmask.live_tiles(),
                   "live_tiles_per_head": bmask.live_tiles() / (bmask.table_shape[0] * bmask.table_shape[1]),
                   "reference_executed_tiles_per_head": ((S + 127) // 128) ** 2,
                   "unmasked_pairs_per_head": pairs / B},
        "fwdbwd_pct_peak": round(100 * fwdbwd_tflops / PEAK_BF16_TFLOPS, 2),
        "fwd_tflops": round(fwd_tflops, 2),
        "fwd_pct_peak": round(100 * fwd_tflops / PEAK_BF16_TFLOPS, 2),
        "kernel_ms": {k: round(v, 4) for k, v in kernels.items()},
        "flex_attention_ms_per_step": round(api_ms, 4),
        "block_mask_build_ms": round(mask_ms, 3),
        "block_mask_build_host_ms": round(mask_host_ms, 2),
        "roofline": {"kernel": dom, "bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": measured_traffic(args.config, dom)},
        "cpu_baseline": cpu,
        "fp8_forward": fp8,
        "other_configs": others,
        "gemm_reference": gemm,
    }
    if sparsity is not None:
        out["sparsity_check"] = sparsity
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
