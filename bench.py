"""Benchmark of the PrunePath sparse-MoE MLP hot path on one MI355X.

Metric: MoE-MLP decode us/layer + HBM GB/s (bs=1); prefill
tokens/s + MFMA util.

* step = one decode MoE-MLP layer call: H=1536, E=16 experts of
  G=384 neurons, bf16 packed weights, fp32 router, tau=0.70, a fresh x ~N(0,1) per
  step. Steps rotate over 16 independent random-init layers (16 x 56.6 MB of decode
  records > the 256 MB MALL) so weights stream from HBM. Steps are captured in a
  HIP graph and replayed; inputs are resident in HBM before timing starts.
  value = us per layer-step (lower is better).
* roofline (decode kernel, HBM-bound): algorithmic bytes per step =
  k*3*H*G*2 (selected experts' gate/up/down records) + Epad*H*4 (fp32 router) +
  H*4 (x) + H*2 (out), k = experts the step selects (measured per step).
* prefill: N=2048 tokens, tau=0.70; tokens/s of the whole
  prefill path and MFMA utilisation of the two grouped GEMMs
  (FLOPs = P*6*H*G over selected pairs P, no padding) against 2.5 PFLOP/s bf16 dense.
* cpu_baseline: the reference's own CPU path, restated op for op in torch fp32
  (oracle/torch_masked.py: dense gate/up over all neurons, softmax_thresholding, the
  expert mask, down), timed on this host at 1, 2, 4, ... threads up to the allowed
  count, median of >= 20 runs after warm-up, for decode bs=1, bs=16/64 (tau 0.95, Zipf
  bias) and prefill 2048 (tau 0.70); each configuration reports its fastest thread
  count; value = decode bs=1 at its fastest, us per layer-token; cores = that count.
* roofline.traffic: HBM bytes per decode launch from rocprofv3 FETCH_SIZE and
  WRITE_SIZE (two --pmc runs of this script with --calibrate-copy-mib), each scaled
  by the ratio of known bytes to the same counter on a plain elementwise pass of
  known size; read from profiles/decode16_hbm_traffic.txt (written from the output
  of --pmc-summary), null when that file is absent.
"""
from __future__ import annotations

import argparse
import importlib
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, os.path.join(ROOT, "tests", "golden")):
    if p not in sys.path:
        sys.path.insert(0, p)

H, I, E, G = 1536, 6144, 16, 384
PEAK_HBM_GBS = 8000.0
PEAK_BF16_TFLOPS = 2500.0
METRIC = "MoE-MLP decode µs/layer + HBM GB/s (bs=1); prefill tokens/s + MFMA util"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--layers", type=int, default=16, help="independent weight sets rotated per step")
    ap.add_argument("--tau", type=float, default=0.70)
    ap.add_argument("--prefill-tokens", type=int, default=2048)
    ap.add_argument("--prefill-reps", type=int, default=20)
    ap.add_argument("--prefill-zipf", action="store_true",
                    help="prefill section with the config-3 router bias (log Zipf(1.2)), e.g. for profiling small batches")
    ap.add_argument("--cpu-runs", type=int, default=20, help="timed calls per CPU-baseline configuration")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the small-batch (config 3) and E=192/G=32 side measurements")
    ap.add_argument("--side", default="all",
                    help="side sections to run, comma-separated: eager, small, e192, masked, stack (default all)")
    ap.add_argument("--small-batch-only", action="store_true",
                    help="run only the config-3 small-batch section (both paths) and print its numbers")
    ap.add_argument("--grid", type=int, default=0, help="decode workgroups (0 = library default)")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="run 5 plain elementwise passes (torch.neg, fp32) over this many MiB first "
                         "(counter calibration for --pmc)")
    ap.add_argument("--calibrate-only", action="store_true",
                    help="run only the --calibrate-copy-mib pass (a profiler run of its own)")
    ap.add_argument("--pmc-summary", default=None,
                    help="summarise rocprofv3 --pmc csv output under this directory and exit")
    return ap.parse_args()


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "decode16_hbm_traffic.txt")


def pmc_summary(d):
    """Per-kernel mean of each counter per dispatch from rocprofv3 csv output; the
    calibration pass (kernel name containing 'neg') gives bytes-per-counter-unit."""
    import collections
    import csv
    import glob
    files = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        sys.exit(f"no counter_collection.csv under {d}")
    agg = collections.defaultdict(lambda: collections.defaultdict(float))
    disp = collections.defaultdict(set)
    for f in files:
        for r in csv.DictReader(open(f)):
            k = r["Kernel_Name"]
            agg[k][r["Counter_Name"]] += float(r["Counter_Value"])
            disp[k].add(r["Dispatch_Id"])
    calib = {}
    for k, cs in sorted(agg.items(), key=lambda kv: -len(disp[kv[0]])):
        n = len(disp[k])
        line = " ".join(f"{c}={v / n:.6g}" for c, v in sorted(cs.items()))
        print(f"{n:6d} dispatches  {line}  {k[:90]}")
        if "neg" in k:
            calib = {c: v / n for c, v in cs.items()}
    return calib


def read_traffic():
    if not os.path.exists(TRAFFIC_FILE):
        return None
    for line in open(TRAFFIC_FILE):
        if line.startswith("hbm_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def _allowed_threads() -> int:
    """Cores this process may use: the affinity mask, capped by OMP_NUM_THREADS when set
    (the GPU box grants each job a share of the host)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    omp = os.environ.get("OMP_NUM_THREADS")
    return max(1, min(n, int(omp))) if omp and omp.isdigit() else n


def cpu_baseline(args):
    """The reference's CPU path (oracle/torch_masked.py, torch fp32, op for op
    src/openpangu_moe_origin.py:96-118 + src/MoEBlock_origin.py:188-212) on the BASELINE
    shapes: median wall time of >= 20 calls after 3 warm-up calls, per configuration and
    thread count (1, 2, 4, ... up to the threads this process may use). Each
    configuration reports its fastest thread count (more threads are not always faster:
    a one-token layer is a few GEMVs); value and cores are decode bs=1's fastest. Prefill
    below 8 threads runs a 256-token sample per call (the dense layer's time is linear in
    tokens), scaled to 2048 tokens."""
    import numpy as np
    import torch

    import inputs as gi
    from oracle.torch_masked import MaskedLayer
    w = gi.layer_weights(0)
    plain = MaskedLayer(w["w_gate"], w["w_up"], w["w_down"], w["w_router"], w["expert_ids"])
    zipf = MaskedLayer(w["w_gate"], w["w_up"], w["w_down"], w["w_router"], w["expert_ids"], bias=gi.zipf_bias(E))
    rng = np.random.default_rng(5)
    cfgs = [("decode_bs1", 1, 0.70, plain), ("bs16", 16, 0.95, zipf), ("bs64", 64, 0.95, zipf),
            ("prefill2048", 2048, 0.70, plain)]
    n_all = _allowed_threads()
    sweep = sorted({t for t in (1, 2, 4, 8, 16, 32, 64) if t < n_all} | {n_all})
    out = {}
    t_start = time.perf_counter()
    for threads in sweep:
        torch.set_num_threads(threads)
        for name, n, tau, layer in cfgs:
            n_run = 256 if (threads < 8 and n > 256) else n
            x = torch.from_numpy(rng.standard_normal((n_run, H)).astype(np.float32))
            for _ in range(3):
                layer(x, tau)
            ts = []
            for _ in range(args.cpu_runs):
                t0 = time.perf_counter()
                layer(x, tau)
                ts.append(time.perf_counter() - t0)
            us = float(np.median(ts)) * 1e6 * (n / n_run)
            c = out.setdefault(name, {"tokens": n, "tau": tau, "router_bias": "zipf(1.2)" if layer is zipf else None,
                                      "by_threads": {}})
            c["by_threads"][str(threads)] = {"us_per_call": us, "us_per_token": us / n, "runs": args.cpu_runs,
                                             "sample_tokens_per_call": n_run}
    torch.set_num_threads(n_all)
    for c in out.values():
        best = min(c["by_threads"], key=lambda t: c["by_threads"][t]["us_per_call"])
        c["best_threads"] = int(best)
        c["best"] = c["by_threads"][best]
    d = out["decode_bs1"]
    return {"value": d["best"]["us_per_call"], "unit": "us/layer", "cores": d["best_threads"], "kind": "port",
            "sample": (f"oracle/torch_masked.py (torch fp32 dense masked layer, the reference's CPU path), "
                       f"H={H} E={E} G={G}; median of {args.cpu_runs} calls per configuration and thread count "
                       f"({', '.join(map(str, sweep))}) after 3 warm-up calls; value = decode bs=1 tau 0.70 at its "
                       f"fastest thread count ({d['best_threads']}); "
                       f"{time.perf_counter() - t_start:.1f} s of CPU work in total"),
            "threads_allowed": n_all, "cpu_model": _cpu_model(),
            "torch_cpu_capability": torch.backends.cpu.get_cpu_capability(), "configs": out}


def eager_decode(pkg, ops, torch, layer, x, E, G, tau, dev, g, reps=2000):
    """Host cost of one eager (not graph-captured) bs = 1 decode call through each layer a
    caller can use: the C ABI over ctypes, the torch.library op
    (torch.ops.prunepath.moe_decode_into) and the TauSparseMoE module. Per path: `reps`
    calls back to back after 50 warm-up calls; host_us = time to issue them / reps (no
    synchronisation inside the loop), wall_us = time until the GPU has finished them /
    reps. The kernel itself takes ~11.5 us, so a host_us above that is the host's bound."""
    import ctypes
    packed, rp, ws = layer
    H = x.numel()
    out = torch.empty(1, H, dtype=torch.bfloat16, device=dev)
    lib = pkg._lib.lib()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    xp, rpp, pp, op, wsp = (ctypes.c_void_p(t.data_ptr()) for t in (x, rp, packed, out, ws))
    tau_c = ctypes.c_float(tau)

    def abi():
        rc = lib.pp_moe_decode(xp, 0, H, rpp, None, E, G, tau_c, pp, op, wsp, 0, stream)
        if rc != 0:
            raise RuntimeError("pp_moe_decode: %d" % rc)

    x2 = x.reshape(1, H)
    top = pkg._lib.torch_ops().moe_decode_into

    def torch_op():
        top(x2, rp, None, E, G, float(tau), packed, ws, out, 0)

    I = E * G
    mod = pkg.TauSparseMoE(H, I, E, G, tau).to(dev)
    with torch.no_grad():
        mod.load_from_masked(torch.randn(I, H, device=dev, generator=g) * 0.02,
                             torch.randn(I, H, device=dev, generator=g) * 0.02,
                             torch.randn(H, I, device=dev, generator=g) * 0.02,
                             torch.randn(E, H, device=dev, generator=g) * 0.02,
                             torch.arange(I, device=dev) // G)
    x3 = x.reshape(1, 1, H)

    def module():
        with torch.no_grad():
            mod(x3)

    res = {"reps": reps, "note": "eager bs=1 decode calls back to back, steady state (one untimed pass of "
                                 "every path first); host_us = issue time per call, wall_us = time per call "
                                 "until the GPU finished"}
    paths = (("c_abi_ctypes", abi), ("torch_op", torch_op), ("module", module))
    # the first few thousand module calls of a process run ~3x slower on the host (measured:
    # 30 us against 11 us per call in a second pass over the same paths), so every path gets
    # one untimed pass of `reps` calls before the timed one
    for _, fn in paths:
        for _ in range(reps):
            fn()
    torch.cuda.synchronize()
    for name, fn in paths:
        for _ in range(50):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        t1 = time.perf_counter()
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        res[name] = {"host_us": (t1 - t0) * 1e6 / reps, "wall_us": (t2 - t0) * 1e6 / reps}
    del mod
    return res


def small_batch(ops, gi, torch, np, layers, dev, g, reps=1):
    """Config 3 (bs 16 and 64, tau 0.95, Zipf(1.2) router bias): both paths, graph-replayed
    (32 calls per graph over the rotating weight sets), `reps` timed replays (median)."""
    extra = {}
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    Epad = (E + 15) // 16 * 16
    # config 3: small-batch decode, bs 16 and 64, tau 0.95, Zipf(1.2) router bias;
    # bytes = union of the selected experts' records + router + x
    # two paths: the one-launch batch kernel (pp_moe_decode_batch, what TauSparseMoE
    # runs for 2 <= N <= 64) and the five-kernel prefill pipeline on the same tokens
    bias = torch.from_numpy(gi.zipf_bias(E)).to(dev)
    bwsq = torch.empty(ops.decode_batch_workspace_bytes(H, E, G), dtype=torch.uint8, device=dev)
    for nb in (16, 64):
        R = 32
        xq = torch.randn(R, nb, H, device=dev, generator=g)
        wsq = torch.empty(ops.prefill_workspace_bytes(nb, H, E, G), dtype=torch.uint8, device=dev)
        outq = torch.empty(nb, H, dtype=torch.bfloat16, device=dev)
        union = []
        for r in range(R):
            packed, rp, _ = layers[r % len(layers)]
            m = ops.route(xq[r], rp, E, 0.95, bias=bias, want_logits=False)["mask"]
            union.append(int((m.sum(0) > 0).sum()))
        u = float(np.mean(union))
        byt = u * 3 * H * G * 2 + Epad * H * 4 + nb * H * 4 + nb * H * 2

        def call_batch(r):
            packed, rp, wsd = layers[r % len(layers)]
            ops.moe_decode_batch(xq[r], rp, bias, E, G, 0.95, packed, wsd, bwsq, out=outq)

        def call_prefill(r):
            packed, rp, _ = layers[r % len(layers)]
            ops.moe_prefill(xq[r], rp, bias, E, G, 0.95, packed, workspace=wsq, out=outq)

        for key, call in ((f"bs{nb}", call_batch), (f"bs{nb}_prefill", call_prefill)):
            for r in range(R):
                call(r)
            torch.cuda.synchronize()
            gq = torch.cuda.CUDAGraph()
            sq = torch.cuda.Stream()
            sq.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(sq):
                with torch.cuda.graph(gq, stream=sq):
                    for r in range(R):
                        call(r)
            torch.cuda.current_stream().wait_stream(sq)
            gq.replay()
            torch.cuda.synchronize()
            e0.record()
            gq.replay()
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1000.0 / R
            extra[key] = {"us_per_layer": us, "tokens_per_s": nb / (us * 1e-6), "experts_hit_mean": u,
                          "hbm_gbs": byt / (us * 1e-6) / 1e9, "frac": byt / (us * 1e-6) / (PEAK_HBM_GBS * 1e9),
                          "tau": 0.95, "router_bias": "zipf(1.2)",
                          "path": "pp_moe_decode_batch (one launch)" if call is call_batch else
                                  "pp_moe_prefill (route, bucket, gate/up, down, combine)"}
        for lid in range(len(layers)):  # the batch calls left the decode workspaces healthy
            assert ops.decode_state(layers[lid][2], E)["error"] == 0
    return extra


def mfma_ceiling(pkg, torch, iters=200, reps=20):
    """bf16 MFMA rate on register operands (libpp_bench.so, measurement support built beside
    the library): one 8-wave workgroup per CU, the dense GEMMs' 4 x 2 wave tile of
    v_mfma_f32_32x32x16_bf16, random-sign and all-zero operands. The chip's clock under MFMA
    load depends on the operand bits, so this is the rate the GEMMs' MFMA work can reach on
    data like theirs; `iters` sets a launch near their length (tens of us)."""
    import ctypes

    import numpy as np
    lib = ctypes.CDLL(os.path.join(os.path.dirname(pkg.__file__), "libpp_bench.so"))
    lib.ppb_mfma_rate.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                  ctypes.POINTER(ctypes.c_float)]
    grid = torch.cuda.get_device_properties(0).multi_processor_count
    flops = grid * 8.0 * iters * 8 * 32768.0
    res = {"grid": grid, "waves_per_cu": 8, "iters": iters, "launches": reps}
    for name, mode in (("random_sign", 1), ("zero", 0)):
        ms = (ctypes.c_float * reps)()
        rc = lib.ppb_mfma_rate(grid, iters, mode, reps, ms)
        if rc:
            raise RuntimeError(f"ppb_mfma_rate: HIP error {rc}")
        med = float(np.median(np.frombuffer(ms, dtype=np.float32)))
        res[name] = {"us_per_launch": med * 1e3, "tflops": flops / (med * 1e-3) / 1e12,
                     "frac_of_peak": flops / (med * 1e-3) / 1e12 / PEAK_BF16_TFLOPS}
    return res


def main():
    args = parse()
    if args.pmc_summary:
        pmc_summary(args.pmc_summary)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (every box has one MI355X); "
              "--gpus must be 1", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import inputs as gi
    pkg = importlib.import_module("prune_path_openpangu-embedded-1b_amd")
    ops = pkg.ops
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    if args.calibrate_copy_mib > 0:
        n = args.calibrate_copy_mib * (1 << 20) // 4
        src = torch.randn(n, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
        print(f"calibration: 5 x torch.neg over {args.calibrate_copy_mib} MiB fp32 "
              f"(reads {n * 4} B, writes {n * 4} B per dispatch)", file=sys.stderr)
        del src, dst
    if args.calibrate_only:
        return

    # ---------------- layers (random init, packed once; reference-layout copies not kept)
    layers = []
    g = torch.Generator(device=dev)
    for l in range(args.layers):
        g.manual_seed(1000 + l)
        wg = torch.randn(I, H, device=dev, generator=g) * 0.02
        wu = torch.randn(I, H, device=dev, generator=g) * 0.02
        wd = torch.randn(H, I, device=dev, generator=g) * 0.02
        wr = torch.randn(E, H, device=dev, generator=g) * 0.02
        perm = torch.randperm(I, device=dev, generator=g).to(torch.int32)  # random balanced partition
        packed = ops.pack_experts(wg, wu, wd, E, G, perm=perm, layout="linear")
        rp = ops.pack_router(wr, layout="linear")
        ws = ops.decode_workspace(H, E, dev)
        layers.append((packed, rp, ws))
        del wg, wu, wd
    torch.cuda.synchronize()

    if args.small_batch_only:
        print(json.dumps({"small_batch": small_batch(ops, gi, torch, np, layers, dev, g, reps=5)}))
        return

    # ---------------- decode: inputs resident, per-step k from an untimed pass of the batch
    # kernel, whose routing is the decode kernel's own code (dec16_logits, sel16_wave: the
    # same logits bits and selection for the same x), so that no decode-kernel dispatch
    # runs outside the graph-replayed warm-up and timed steps
    K, W = args.steps, args.warmup
    xs = torch.randn(K + W, H, device=dev, generator=g)
    outs = torch.empty(K + W, H, dtype=torch.bfloat16, device=dev)
    ks = np.zeros(K + W, dtype=np.int64)
    bws = torch.empty(ops.decode_batch_workspace_bytes(H, E, G), dtype=torch.uint8, device=dev)
    for l in range(len(layers)):
        packed, rp, ws = layers[l]
        steps = np.arange(W + (l - W) % len(layers), W + K, len(layers))  # the steps that use layer l
        for c in range(0, len(steps), 64):
            idx = torch.from_numpy(steps[c:c + 64]).to(dev)
            mask = torch.empty(len(idx), E, dtype=torch.uint8, device=dev)
            ops.moe_decode_batch(xs[idx], rp, None, E, G, args.tau, packed, ws, bws, mask_out=mask)
            ks[steps[c:c + 64]] = mask.sum(1).cpu().numpy()
        assert ops.decode_state(ws, E)["error"] == 0
    ks = ks[W:]
    del bws

    def capture(lo, hi):
        graph = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            with torch.cuda.graph(graph, stream=s):
                for i in range(lo, hi):
                    packed, rp, ws = layers[i % len(layers)]
                    ops.moe_decode(xs[i], rp, None, E, G, args.tau, packed, ws, grid=args.grid,
                                   out=outs[i:i + 1])
        torch.cuda.current_stream().wait_stream(s)
        return graph

    g_warm = capture(0, W) if W > 0 else None
    g_time = capture(W, W + K)
    if g_warm is not None:
        g_warm.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    g_time.replay()
    e1.record()
    torch.cuda.synchronize()
    dec_ms = e0.elapsed_time(e1)
    us_per_step = dec_ms * 1000.0 / K
    Epad = (E + 15) // 16 * 16
    bytes_steps = ks * 3 * H * G * 2 + Epad * H * 4 + H * 4 + H * 2
    gbs = float(bytes_steps.mean()) / (us_per_step * 1e-6) / 1e9

    # ---------------- prefill (config 4)
    prefill = None
    if not args.no_prefill:
        N = args.prefill_tokens
        R = args.prefill_reps
        pbias = torch.from_numpy(gi.zipf_bias(E)).to(dev) if args.prefill_zipf else None
        xp = torch.randn(R, N, H, device=dev, generator=g)
        wsp = torch.empty(ops.prefill_workspace_bytes(N, H, E, G), dtype=torch.uint8, device=dev)
        outp = torch.empty(N, H, dtype=torch.bfloat16, device=dev)
        for r in range(2):
            packed, rp, _ = layers[r % len(layers)]
            ops.moe_prefill(xp[r], rp, pbias, E, G, args.tau, packed, workspace=wsp, out=outp)
        torch.cuda.synchronize()
        gp = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            with torch.cuda.graph(gp, stream=s):
                for r in range(R):
                    packed, rp, _ = layers[r % len(layers)]
                    ops.moe_prefill(xp[r], rp, pbias, E, G, args.tau, packed, workspace=wsp, out=outp)
        torch.cuda.current_stream().wait_stream(s)
        gp.replay()
        torch.cuda.synchronize()
        e0.record()
        gp.replay()
        e1.record()
        torch.cuda.synchronize()
        pf_ms = e0.elapsed_time(e1) / R
        # pairs per call (routing is deterministic): from the route stage
        P = 0
        for r in range(R):
            packed, rp, _ = layers[r % len(layers)]
            P += int(ops.route(xp[r], rp, E, args.tau, bias=pbias, want_logits=False)["count"].sum())
        P_mean = P / R
        # the two grouped GEMMs alone, graph-replayed on a fixed bucket layout
        packed, rp, _ = layers[0]
        xb = xp[0].to(torch.bfloat16)
        rt = ops.route(xb, rp, E, args.tau, bias=pbias, want_logits=False)
        bk = ops.bucket(rt["mask"], rt["gates"])
        P0 = int(rt["count"].sum())
        act = ops.expert_gateup(xb, packed, E, G, bk)
        y = ops.expert_down(act, packed, H, E, G, bk)
        torch.cuda.synchronize()

        def time_graph(fn, reps=R):
            gg = torch.cuda.CUDAGraph()
            ss = torch.cuda.Stream()
            ss.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(ss):
                with torch.cuda.graph(gg, stream=ss):
                    for _ in range(reps):
                        fn()
            torch.cuda.current_stream().wait_stream(ss)
            gg.replay()
            torch.cuda.synchronize()
            e0.record()
            gg.replay()
            e1.record()
            torch.cuda.synchronize()
            return e0.elapsed_time(e1) / reps

        lib = pkg._lib.lib()
        import ctypes

        def gateup_call():
            s_ = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            pkg._lib.check(lib.pp_expert_gateup(ctypes.c_void_p(xb.data_ptr()), H, G, ctypes.c_void_p(packed.data_ptr()),
                                                E, ctypes.c_void_p(bk["token_ids"].data_ptr()),
                                                ctypes.c_void_p(bk["pair_gates"].data_ptr()),
                                                ctypes.c_void_p(bk["tiles"].data_ptr()),
                                                ctypes.c_void_p(bk["meta"].data_ptr()), bk["max_tiles"],
                                                ctypes.c_void_p(act.data_ptr()), s_), "gateup")

        def down_call():
            s_ = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            pkg._lib.check(lib.pp_expert_down(ctypes.c_void_p(act.data_ptr()), H, G, ctypes.c_void_p(packed.data_ptr()),
                                              E, ctypes.c_void_p(bk["tiles"].data_ptr()),
                                              ctypes.c_void_p(bk["meta"].data_ptr()), bk["max_tiles"],
                                              ctypes.c_void_p(y.data_ptr()), s_), "down")

        gu_ms = time_graph(gateup_call)
        dn_ms = time_graph(down_call)
        fl_gu = 4.0 * P0 * H * G
        fl_dn = 2.0 * P0 * H * G
        prefill = {
            "tokens": N, "tau": args.tau, "router_bias": "zipf(1.2)" if args.prefill_zipf else None,
            "pairs_mean": P_mean, "ms_per_call": pf_ms,
            "tokens_per_s": N / (pf_ms * 1e-3),
            "gemm_flops": fl_gu + fl_dn,
            "gateup_us": gu_ms * 1e3, "down_us": dn_ms * 1e3,
            "gateup_tflops": fl_gu / (gu_ms * 1e-3) / 1e12, "down_tflops": fl_dn / (dn_ms * 1e-3) / 1e12,
            "mfma_util": (fl_gu + fl_dn) / ((gu_ms + dn_ms) * 1e-3) / (PEAK_BF16_TFLOPS * 1e12),
            "layer_mfma_util": (6.0 * P_mean * H * G) / (pf_ms * 1e-3) / (PEAK_BF16_TFLOPS * 1e12),
        }
        # the MFMA rate reachable on random bf16 operands, beside the GEMMs' own rate
        ceil = mfma_ceiling(pkg, torch)
        prefill["mfma_ceiling"] = ceil
        prefill["mfma_util_of_ceiling"] = ((fl_gu + fl_dn) / ((gu_ms + dn_ms) * 1e-3) / 1e12
                                           / ceil["random_sign"]["tflops"])

    # ---------------- side measurements (not the headline value)
    extra = None
    sides = set(args.side.split(","))

    def want(name):
        return "all" in sides or name in sides

    if not args.no_extra:
        extra = {}
        if want("eager"):
            extra["eager_decode"] = eager_decode(pkg, ops, torch, layers[0], xs[0], E, G, args.tau, dev, g)
        if want("small"):
            extra.update(small_batch(ops, gi, torch, np, layers, dev, g))
        if want("e192"):
            # real-checkpoint shape: E=192 experts of G=32, one layer, decode bs=1 and prefill 2048
            E2, G2 = 192, 32
            l192 = []
            NS = 8
            for l in range(NS):
                g.manual_seed(2000 + l)
                wg = torch.randn(I, H, device=dev, generator=g) * 0.02
                wu = torch.randn(I, H, device=dev, generator=g) * 0.02
                wd = torch.randn(H, I, device=dev, generator=g) * 0.02
                wr = torch.randn(E2, H, device=dev, generator=g) * 0.02
                perm = torch.randperm(I, device=dev, generator=g).to(torch.int32)
                l192.append((ops.pack_experts(wg, wu, wd, E2, G2, perm=perm, layout="linear"),
                             ops.pack_router(wr, layout="linear"), ops.decode_workspace(H, E2, dev)))
                del wg, wu, wd
            R = 64
            xd = torch.randn(R, H, device=dev, generator=g)
            od = torch.empty(R, H, dtype=torch.bfloat16, device=dev)
            kk = []
            for r in range(R):
                packed, rp, ws = l192[r % NS]
                ops.moe_decode(xd[r], rp, None, E2, G2, args.tau, packed, ws, out=od[r:r + 1])
                kk.append(ops.decode_state(ws, E2)["k"])
            gd = torch.cuda.CUDAGraph()
            sd_ = torch.cuda.Stream()
            sd_.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(sd_):
                with torch.cuda.graph(gd, stream=sd_):
                    for r in range(R):
                        packed, rp, ws = l192[r % NS]
                        ops.moe_decode(xd[r], rp, None, E2, G2, args.tau, packed, ws, out=od[r:r + 1])
            torch.cuda.current_stream().wait_stream(sd_)
            gd.replay()
            torch.cuda.synchronize()
            e0.record()
            gd.replay()
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1000.0 / R
            k2 = float(np.mean(kk))
            byt = k2 * 3 * H * G2 * 2 + 192 * H * 4 + H * 6
            extra["e192_g32_decode"] = {"us_per_layer": us, "k_mean": k2, "hbm_gbs": byt / (us * 1e-6) / 1e9,
                                        "weight_sets": NS}
            # the same shape's prefill (2048 tokens): G = 32 takes the dense form (router logits,
            # selection, dense gate/up over every neuron with the gate 0 for unselected experts,
            # dense down), one pass; calls rotate over the weight sets, graph-replayed like the
            # configured shape's prefill
            if not args.no_prefill:
                Np, Rp = args.prefill_tokens, 2 * NS
                xp2 = torch.randn(Rp, Np, H, device=dev, generator=g)
                wsp = torch.empty(ops.prefill_workspace_bytes(Np, H, E2, G2), dtype=torch.uint8, device=dev)
                opf = torch.empty(Np, H, dtype=torch.bfloat16, device=dev)
                P2 = 0
                for r in range(Rp):
                    packed, rp, _ = l192[r % NS]
                    P2 += int(ops.route(xp2[r], rp, E2, args.tau)["count"].sum())
                    ops.moe_prefill(xp2[r], rp, None, E2, G2, args.tau, packed, workspace=wsp, out=opf)
                torch.cuda.synchronize()
                gq = torch.cuda.CUDAGraph()
                sq = torch.cuda.Stream()
                sq.wait_stream(torch.cuda.current_stream())
                with torch.cuda.stream(sq):
                    with torch.cuda.graph(gq, stream=sq):
                        for r in range(Rp):
                            packed, rp, _ = l192[r % NS]
                            ops.moe_prefill(xp2[r], rp, None, E2, G2, args.tau, packed, workspace=wsp, out=opf)
                torch.cuda.current_stream().wait_stream(sq)
                gq.replay()
                torch.cuda.synchronize()
                e0.record()
                gq.replay()
                e1.record()
                torch.cuda.synchronize()
                ms2 = e0.elapsed_time(e1) / Rp
                P2 /= Rp
                dense_fl = 6.0 * Np * H * (E2 * G2)
                extra["e192_g32_prefill"] = {
                    "tokens": Np, "tau": args.tau, "pairs_mean": P2, "ms_per_call": ms2,
                    "tokens_per_s": Np / (ms2 * 1e-3), "form": "dense (G % 64 != 0)", "weight_sets": NS,
                    "layer_mfma_util": 6.0 * P2 * H * G2 / (ms2 * 1e-3) / (PEAK_BF16_TFLOPS * 1e12),
                    "dense_flops": dense_fl,
                    "dense_mfma_util": dense_fl / (ms2 * 1e-3) / (PEAK_BF16_TFLOPS * 1e12)}
                del wsp, opf, xp2, gq
            del l192
        if want("masked"):
            # masked training path: the expert gating of MoELayer.forward and its backward on
            # a training batch of 16 x 1024 tokens, bf16 activations [16384, 6144] (200 MB per
            # tensor, beyond the MALL); bytes = activations read + written (+ gates)
            torch.cuda.empty_cache()
            Nt = 16384
            ids = torch.randperm(I, device=dev, generator=g) % E
            lay = ops.masked_gate_layout(ids, E)
            inter = torch.randn(Nt, I, device=dev, generator=g).to(torch.bfloat16)
            d_o = torch.randn(Nt, I, device=dev, generator=g).to(torch.bfloat16)
            gts = torch.rand(Nt, E, device=dev, generator=g)
            mg = {}
            for name, fn, byt in (
                    ("fwd", lambda: ops.masked_gate_fwd(inter, gts, lay[0]), 2 * Nt * I * 2 + Nt * E * 4),
                    ("bwd", lambda: ops.masked_gate_bwd(d_o, inter, gts, *lay), 3 * Nt * I * 2 + 2 * Nt * E * 4)):
                fn()
                torch.cuda.synchronize()
                R = 10
                gm = torch.cuda.CUDAGraph()
                sm = torch.cuda.Stream()
                sm.wait_stream(torch.cuda.current_stream())
                with torch.cuda.stream(sm):
                    with torch.cuda.graph(gm, stream=sm):
                        for _ in range(R):
                            fn()
                torch.cuda.current_stream().wait_stream(sm)
                gm.replay()
                torch.cuda.synchronize()
                e0.record()
                gm.replay()
                e1.record()
                torch.cuda.synchronize()
                us = e0.elapsed_time(e1) * 1000.0 / R
                mg[name] = {"us": us, "hbm_gbs": byt / (us * 1e-6) / 1e9, "frac": byt / (us * 1e-6) / 1e9 / PEAK_HBM_GBS}
                del gm
            extra["masked_gate_train"] = {"rows": Nt, "intermediate": I, "experts": E, "dtype": "bf16", **mg}
            del inter, d_o, gts
        if want("stack"):
            # config 5: 26-layer decoder-shaped stack, 1024-token prompt + 128 greedy steps
            torch.cuda.empty_cache()
            extra["decoder_stack"] = pkg.decoder_stack.run(prompt_len=1024, steps=128, layers=26, tau=args.tau)

    # ---------------- CPU baseline: the reference's dense masked layer, torch fp32 on the host
    cpu = None if args.no_cpu else cpu_baseline(args)

    res = {
        "metric": METRIC, "value": us_per_step, "unit": "us/layer", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": us_per_step / 1000.0, "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "decode bs=1, one MoE-MLP layer per step (BASELINE config 2)",
                   "hidden": H, "experts": E, "group_size": G, "tau": args.tau, "batch": 1,
                   "weight_sets": args.layers, "router": "fp32", "x": "fresh N(0,1) fp32 per step"},
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": gbs / PEAK_HBM_GBS, "traffic": read_traffic(),
                     "bytes_per_step": float(bytes_steps.mean()), "k_mean": float(ks.mean()),
                     "k_min": int(ks.min()), "k_max": int(ks.max())},
        "decode": {"us_per_layer": us_per_step, "hbm_gbs": gbs, "k_mean": float(ks.mean())},
        "prefill": prefill,
        "side": extra,
        "cpu_baseline": cpu,
    }
    print(json.dumps(res))


if __name__ == "__main__":
    main()
