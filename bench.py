"""Benchmark: NN evals/s of the HIP backend on b18c384nbt fp16, 19x19, batch 256
with inputs resident in HBM, called through the C
ABI (kgh_forward_device, which replays a captured HIP graph for repeated
forwards); the matrix-core roofline of the 3x3 conv kernel measured with HIP
events on the handle's stream around every conv launch of eager forwards of
the same workload, run right after the timed steps; and the same-run CPU
baseline (the oracle: a restatement of KataGo's Eigen backend).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
    python bench.py --config 3 --batch 1      # C3 latency at batch 1

Prints one JSON line.
"""
import argparse
import json
import os
import sys
import tempfile
import threading
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_FP16_TFLOPS = 2500.0  # MI355X dense fp16 matrix-core peak (datasheet)
PEAK_FP32_TFLOPS = 157.3  # MI355X dense fp32 matrix-core peak
CFG_INDEX = 2              # headline: b18c384nbt fp16 19x19 batch 256


def conv_flops(layers, hw):
    """Algorithmic FLOPs per eval split into 3x3 convs, 1x1 convs and the rest:
    2*k*k*Cin*Cout*HW per conv; 2*in*out per matmul, times HW inside
    transformer blocks (per-position projections); attention
    2*HW*HW*(dq + dv) per head."""
    f3 = f1 = other = 0.0
    per_position = 0  # matmul records still to come inside a transformer block
    for rec in layers:
        if rec["op"] == 13:  # attention: i = heads, kvHeads, dq, dv
            heads, dq, dv = int(rec["i"][0]), int(rec["i"][2]), int(rec["i"][3])
            other += 2.0 * hw * hw * (dq + dv) * heads
            per_position = 4
        elif rec["op"] == 14:  # ffn: linear1, gate, linear2
            per_position = 3 if int(rec["i"][2]) else 2
        elif rec["op"] == 4 and per_position > 0:
            other += 2.0 * int(rec["i"][0]) * int(rec["i"][1]) * hw
            per_position -= 1
            continue
        if rec["op"] == 1:
            ky, kx, ci, co = (int(v) for v in rec["i"][:4])
            f = 2.0 * ky * kx * ci * co * hw
            if ky == 3 and kx == 3:
                f3 += f
            elif ky == 1 and kx == 1:
                f1 += f
            else:
                other += f
        elif rec["op"] == 4:
            other += 2.0 * int(rec["i"][0]) * int(rec["i"][1])
    return f3, f1, other


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "conv3x3_b18c384nbt_b256_fp16_traffic.md")


def measured_traffic():
    """HBM-side bytes per 3x3 conv launch, from the committed rocprofv3
    FETCH_SIZE/WRITE_SIZE summary (scaled by a plain-copy calibration); None
    when the summary is absent."""
    import re
    try:
        text = open(TRAFFIC_PROFILE).read()
    except OSError:
        return None
    m = re.search(r"^traffic_bytes_per_launch:\s*(\d+)", text, re.M)
    return int(m.group(1)) if m else None


_VENDOR_GEMM = r"""
import json, torch
n, iters = %d, %d
a = torch.randn(n, n, dtype=torch.float16, device="cuda")
b = torch.randn(n, n, dtype=torch.float16, device="cuda")
for _ in range(5):
    c = a @ b
torch.cuda.synchronize()
e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
e0.record()
for _ in range(iters):
    c = a @ b
e1.record()
torch.cuda.synchronize()
print(json.dumps({"ms": e0.elapsed_time(e1) / iters}))
"""


def vendor_gemm_rate(n=8192, iters=40):
    """Sustained fp16 matrix-core rate of the vendor GEMM (torch.matmul ->
    hipBLASLt) on random N(0,1) operands, n x n x n, timed with events on
    torch's stream. Random operands matter: with constant operands the matrix
    cores run near the 2.5 PFLOP/s datasheet peak, with random data the chip's
    power limit lowers the clock, which caps every fp16 kernel on the box.
    Runs in a child process started before this process touches the GPU
    (torch's HIP runtime and libkatago_hip's cannot share one process)."""
    import subprocess
    try:
        out = subprocess.run([sys.executable, "-c", _VENDOR_GEMM % (n, iters)], capture_output=True, text=True, timeout=300)
        ms = json.loads(out.stdout.strip().splitlines()[-1])["ms"]
    except Exception as e:  # reported, not fatal: the bench line stands without it
        return {"tflops": None, "what": f"torch.matmul fp16 {n}^3 random operands: failed ({type(e).__name__})"}
    return {"tflops": round(2.0 * n ** 3 / (ms * 1e-3) / 1e12, 1), "what": f"torch.matmul fp16 {n}x{n}x{n}, random N(0,1) operands"}


# CPU threads this process may keep busy on a GPU box: its share of the host
# is 16 CPUs per GPU, whatever the host's own core count is.
BOX_CPU_SHARE = 16


def cpu_baseline(path, seconds_target=15.0):
    """The oracle (fp32 Eigen-algorithm restatement) on T host threads, each
    running forwards of batch 8, as the reference's Eigen deployment runs one
    single-threaded forward per server thread (eigenbackend.cpp:8-9). T is
    every core of the affinity set, up to the GPU box's CPU share; the host's
    hardware_concurrency and the affinity set size are reported beside it."""
    from katago_amd import modelgen
    from oracle import oracle
    host_cores = os.cpu_count() or 1
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = host_cores
    threads = max(1, min(affinity, BOX_CPU_SHARE))
    om = oracle.OracleModel(path)
    sp, gl = modelgen.synthetic_inputs(2000 + CFG_INDEX, 8)
    t0 = time.perf_counter()
    om.forward(sp[:1], gl[:1])
    per_row = time.perf_counter() - t0
    iters = int(max(1, min(4, seconds_target / max(per_row * 8, 1e-3))))
    done = [0]
    lock = threading.Lock()

    def work():
        for _ in range(iters):
            om.forward(sp, gl)
            with lock:
                done[0] += 8

    ths = [threading.Thread(target=work) for _ in range(threads)]
    t0 = time.perf_counter()
    for t in ths:
        t.start()
    for t in ths:
        t.join()
    wall = time.perf_counter() - t0
    value = done[0] / wall
    return {"value": round(value, 3), "unit": "evals/s", "cores": threads, "kind": "port",
            "host_hardware_concurrency": host_cores, "affinity_cores": affinity,
            "per_thread": round(value / threads, 3),
            "sample": f"b18c384nbt fp32, Eigen-algorithm restatement (oracle/eigen_oracle.cpp), {threads} threads x "
                      f"{iters} forwards x batch 8 = {done[0]} evals in {wall:.1f} s; threads = the affinity set "
                      f"({affinity} of the host's {host_cores}) capped at the box's CPU share of {BOX_CPU_SHARE} per GPU"}


def latency(h, call, lm, cfg, batch=1, steps=200):
    """Batch-1 latency: each forward timed alone on the host clock (launch to
    synchronize), inputs resident in HBM; and the same through the host-memory
    entry point (featurized row in pageable host memory -> pinned staging ->
    H2D -> forward -> D2H), as a KataGo search thread waiting on one
    evaluation sees it."""
    import numpy as np
    from katago_amd import modelgen, nn
    lat = []
    for _ in range(steps):
        t0 = time.perf_counter()
        call()
        h.synchronize()
        lat.append(time.perf_counter() - t0)
    q = lambda a, p: round(1000.0 * float(np.percentile(a, p)), 4)
    sp, gl = modelgen.synthetic_inputs(cfg.input_seed, 1, board_sizes=cfg.board_sizes)

    def host_path(low_latency):
        ctx = nn.ComputeContext(lm, 19, 19, use_fp16=cfg.fp16, auto_tune=False, low_latency=low_latency)
        ch = nn.ComputeHandle(ctx, max_batch=1)
        for _ in range(5):
            ch.get_output(sp, gl)
        host = []
        for _ in range(steps):
            t0 = time.perf_counter()
            ch.get_output(sp, gl)
            host.append(time.perf_counter() - t0)
        ch.close()
        ctx.close()
        return {"p50": q(host, 50), "p90": q(host, 90), "min": q(host, 0)}

    out = {"hbm_resident_ms": {"p50": q(lat, 50), "p90": q(lat, 90), "min": q(lat, 0)},
           "pcie_inclusive_ms": host_path(False)}
    if cfg.fp16 and batch <= 16:
        # The same with hipLowLatency (split-K 3x3 convs): device-resident
        # inputs on a one-row device handle, and the host-memory path.
        h.set_low_latency(True)
        for _ in range(5):
            call()
        h.synchronize()
        fast = []
        for _ in range(steps):
            t0 = time.perf_counter()
            call()
            h.synchronize()
            fast.append(time.perf_counter() - t0)
        h.set_low_latency(False)
        out["low_latency"] = {"hbm_resident_ms": {"p50": q(fast, 50), "p90": q(fast, 90), "min": q(fast, 0)},
                              "pcie_inclusive_ms": host_path(True),
                              "what": "hipLowLatency: split-K 3x3 convolutions (up to 8 workgroups per board and 64 "
                                      "output channels, fp32 partial sums added in a fixed order)"}
    out.update({"forwards": steps, "what": "one board per forward, host wall clock from launch to synchronize"})
    return out


def _fixture_positions(batch):
    """Positions of KataGo's own random games (tests/golden/featurize_golden.json.gz)
    in 19x19 tensors, repeated up to `batch`."""
    import gzip
    with gzip.open(os.path.join(ROOT, "tests", "golden", "featurize_golden.json.gz"), "rt") as f:
        fixtures = [fx for fx in json.load(f)["positions"] if fx["nnx"] == 19 and fx["nny"] == 19]
    return [fixtures[i % len(fixtures)] for i in range(batch)]


def featurize_rate(batch, seconds=2.0):
    """Rows/s of the featurizer (kgn_featurize: chains, ladders on three
    boards, pass-alive area, history and rule features of NNInputs::fillRowV7)
    on one thread and on the box's CPU share."""
    from katago_amd import nn
    pos = nn.Positions(_fixture_positions(batch))
    out = {}
    for threads in (1, BOX_CPU_SHARE):
        nn.featurize(pos, 19, 19, num_threads=threads)
        rows, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < seconds:
            nn.featurize(pos, 19, 19, num_threads=threads)
            rows += batch
        out[f"threads_{threads}"] = round(rows / (time.perf_counter() - t0), 1)
    out["unit"] = "rows/s"
    out["what"] = (f"{batch}-row batches of 19x19 positions from seeded random games (tests/golden/featurize_golden.json.gz), "
                   "NHWC rows identical to KataGo's NNInputs::fillRowV7")
    return out


def featurize_serve_rate(lm, cfg, batch, rounds=30, servers=2):
    """Positions in, network outputs out: one thread featurizes batches
    (kgn_featurize on BOX_CPU_SHARE - servers threads) into a queue, and
    `servers` threads, each with its own handle on the device (as KataGo's
    server threads per GPU), run them through getOutput (pinned staging, H2D,
    forward, D2H), so one batch's host packing and copies overlap another's
    forward."""
    import queue
    from katago_amd import nn
    pos = nn.Positions(_fixture_positions(batch))
    ctx = nn.ComputeContext(lm, 19, 19, use_fp16=cfg.fp16, auto_tune=False)
    handles = [nn.ComputeHandle(ctx, max_batch=batch) for _ in range(servers)]
    q = queue.Queue(maxsize=servers + 1)
    first = nn.featurize(pos, 19, 19)
    for h in handles:
        h.get_output(*first)  # warm up (graph capture)

    done = [0] * servers
    errors = []

    def produce():
        try:
            for _ in range(rounds):
                q.put(nn.featurize(pos, 19, 19, num_threads=max(1, BOX_CPU_SHARE - servers)))
        except Exception as e:  # re-raised below; the servers still get their end marks
            errors.append(e)
        finally:
            for _ in range(servers):
                q.put(None)

    def serve(i):
        try:
            while True:
                item = q.get()
                if item is None:
                    break
                handles[i].get_output(*item)
                done[i] += batch
        except Exception as e:  # re-raised below, after every thread ended
            errors.append(e)
            while q.get() is not None:  # let the producer finish
                pass

    threads = [threading.Thread(target=produce)] + [threading.Thread(target=serve, args=(i,)) for i in range(servers)]
    t0 = time.perf_counter()
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    secs = time.perf_counter() - t0
    for h in handles:
        h.close()
    ctx.close()
    if errors:
        raise errors[0]
    return {"value": round(sum(done) / secs, 1), "unit": "evals/s", "batches": rounds, "server_threads": servers,
            "path": "positions -> kgn_featurize (host) -> getOutput (pinned staging, H2D, forward, D2H) -> rows, "
                    "featurizing overlapped with the device, two server threads with a handle each"}


def serve_rate(lm, cfg, batch, server_threads=2, rounds=40):
    """Evals/s with rows coming from host memory through the batching
    evaluator (NNEvaluator's serve loop): 2*batch native client threads keep
    both server threads' batches full; each batch is packed into pinned
    memory, copied to the device, run, copied back and unpacked. Not the
    headline value, which has inputs resident in HBM."""
    from katago_amd import modelgen, nn
    sp, gl = modelgen.synthetic_inputs(cfg.input_seed, batch, board_sizes=cfg.board_sizes)
    ev = nn.Evaluator(lm, max_batch=batch, use_fp16=cfg.fp16, num_server_threads=server_threads)
    clients = server_threads * batch
    ev.run_clients(sp, gl, num_clients=clients, evals_per_client=2)  # warm up (graph capture per handle)
    ev.clear_stats()
    secs, _ = ev.run_clients(sp, gl, num_clients=clients, evals_per_client=rounds)
    rows, batches = ev.stats()
    ev.close()
    print(f"bench: serve {rows} rows in {batches} batches, {secs:.3f} s", file=sys.stderr, flush=True)
    return {"value": round(rows / secs, 2), "unit": "evals/s", "server_threads": server_threads, "clients": clients,
            "avg_batch": round(rows / max(batches, 1), 1),
            "path": "featurized rows in host memory -> NNEvaluator batching -> pinned staging -> H2D -> forward -> D2H -> rows"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--model-dir", default=None)
    ap.add_argument("--config", type=int, default=CFG_INDEX,
                    help="BASELINE.json config index; 2 (default) is the headline, 4 the transformer trunk")
    ap.add_argument("--no-autotune", action="store_true", help="keep the built-in kernel choices")
    ap.add_argument("--batch", type=int, default=0, help="boards per forward instead of the config's (not the headline line)")
    ap.add_argument("--latency", action="store_true", help="also time single forwards (always on at --batch 1)")
    ap.add_argument("--no-latency", action="store_true", help="skip the single-forward timing even at --batch 1")
    ap.add_argument("--low-latency", action="store_true",
                    help="run the timed forwards in the handle's low-latency mode (split-K 3x3 convs; batch <= 16)")
    ap.add_argument("--no-serve", action="store_true",
                    help="skip the PCIe-inclusive measurement through the batching evaluator")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run 5 plain device copies of MIB MiB (torch), to scale rocprofv3 FETCH_SIZE/WRITE_SIZE")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU. Rows are independent and weights replicated, so N GPUs run N independent "
              "handles with no communication; this build does not launch multi-GPU runs.", file=sys.stderr)
        sys.exit(2)

    if args.copy_calibration:
        import torch
        nbytes = args.copy_calibration << 20
        src = torch.ones(nbytes, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": nbytes, "copies": 5}), flush=True)
        return

    # Before anything here initialises the GPU.
    vendor = vendor_gemm_rate() if args.config == CFG_INDEX and not args.batch else None

    import numpy as np
    from katago_amd import modelgen, nn

    cfg = modelgen.configs()[args.config]
    batch, hw = (args.batch or cfg.batch), 19 * 19
    model_dir = args.model_dir or os.path.join(tempfile.gettempdir(), "katago_amd_models")
    path = modelgen.ensure_model(model_dir, cfg)
    print(f"bench: model {path}", file=sys.stderr, flush=True)

    lm = nn.LoadedModel(path)
    dm = nn.DeviceModel(lm, use_fp16=cfg.fp16)
    h = nn.DeviceHandle(dm, batch)
    if args.low_latency:
        h.set_low_latency(True)
    # Tile choices as a backend handle makes them at creation (the on-device
    # autotuner); the table goes to stderr.
    tuning = "" if args.no_autotune else h.autotune()
    print("bench: autotuned conv shapes (ky kx cinPad cout M gated residual maskedResidual variant name best_us "
          "heuristic_us):\n" + tuning, file=sys.stderr, flush=True)
    f3, f1, fother = conv_flops(dm.layers, hw)
    flops_per_eval = f3 + f1 + fother

    sp, gl = modelgen.synthetic_inputs(cfg.input_seed, batch, board_sizes=cfg.board_sizes)
    d_sp = nn.DeviceBuffer.from_array(sp)
    d_gl = nn.DeviceBuffer.from_array(gl)
    d_sym = nn.DeviceBuffer.from_array(np.zeros(batch, np.int32))
    d_opt = nn.DeviceBuffer.from_array(np.zeros(batch, np.float32))
    d_out = nn.DeviceBuffer(batch * h.row_floats * 4)
    call = lambda: h.forward_device(batch, d_sp.ptr, d_gl.ptr, d_sym.ptr, d_opt.ptr, d_out.ptr)

    for _ in range(args.warmup):
        call()
    h.synchronize()
    print(f"bench: warmup {args.warmup} done", file=sys.stderr, flush=True)

    # Timed steps: the production path (repeated forwards replay a captured
    # HIP graph).
    h.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        call()
    h.synchronize()
    elapsed = time.perf_counter() - t0
    out = d_out.to_array(np.float32, (batch, h.row_floats))
    assert np.isfinite(out).all(), "non-finite outputs"
    # Kernel timing: the same forwards launched eagerly with HIP events
    # recorded on the handle's stream around every conv launch.
    prof_steps = max(1, min(args.steps, 10))
    h.set_profiling(True)
    for _ in range(prof_steps):
        call()
    h.synchronize()
    ms3, n3, fl3 = h.profile(0)
    ms1, n1, fl1 = h.profile(1)
    per_kernel = h.profile_kernels()
    h.set_profiling(False)
    # Every conv kernel together (3x3 and 1x1): the conv-kernel fraction of the
    # dense peak as the target defines it, direct-conv FLOPs over conv time.
    conv_frac = (fl3 + fl1) / ((ms3 + ms1) * 1e-3) / 1e12 if ms3 + ms1 > 0 else 0.0

    evals = batch * args.steps
    value = evals / elapsed
    print(f"bench: {args.steps} steps in {elapsed:.3f} s; profiled {prof_steps} eager steps: 3x3 conv {n3} launches "
          f"{ms3:.2f} ms total, 1x1 conv {n1} launches {ms1:.2f} ms total", file=sys.stderr, flush=True)
    headline = args.config == CFG_INDEX and batch == cfg.batch
    # Roofline kernel: the 3x3 conv for the convolutional nets, the 1x1
    # (per-position GEMM) kernel for a transformer trunk; the figures cover
    # every launch of that kind, and the name lists the kernels that ran
    # (as the launches recorded them), the one with the most time first.
    peak = PEAK_FP16_TFLOPS if cfg.fp16 else PEAK_FP32_TFLOPS
    kind = 0 if ms3 >= ms1 else 1
    ms_k, n_k, fl_k = (ms3, n3, fl3) if kind == 0 else (ms1, n1, fl1)
    ran = sorted((r for r in per_kernel if r[0] == kind), key=lambda r: -r[2])
    kname = "; ".join(f"{r[4]} x{r[1] // prof_steps}" for r in ran) + " per forward"
    avg_ms = ms_k / max(n_k, 1)
    achieved = (fl_k / max(n_k, 1)) / (avg_ms * 1e-3) / 1e12 if n_k else 0.0
    name = cfg.arch.name.replace("-synthetic", "")
    boards = "x".join(str(b) for b in cfg.board_sizes)
    result = {
        "metric": ("NN evals/sec, b18c384nbt fp16 19x19 batch 256; % of fp16 MFMA peak" if headline else
                   f"NN evals/sec, {name} {'fp16' if cfg.fp16 else 'fp32'} 19x19 batch {batch}"),
        "value": round(value, 2),
        "unit": "evals/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1000.0 * elapsed / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16" if cfg.fp16 else "fp32",
        "data": f"synthetic (seeded random-weight {name}, seeded synthetic positions)",
        "config": {"workload": f"C{args.config}: {name} {'fp16' if cfg.fp16 else 'fp32'} boards {boards} in 19x19, batch {batch}, "
                               f"symmetry 0, inputs resident in HBM",
                   "global_batch": batch, "board": "19x19", "parallelism": "none (1 GPU)",
                   "autotuned_shapes": len([l for l in tuning.splitlines() if l.strip()]),
                   **({"low_latency": True} if args.low_latency else {})},
        "mfma_frac_end_to_end": round(value * flops_per_eval / (peak * 1e12), 4),
        "gflop_per_eval": round(flops_per_eval / 1e9, 3),
        "conv_frac": {"achieved": round(conv_frac, 2), "peak": peak, "unit": "TFLOP/s",
                      "frac": round(conv_frac / peak, 4), "frac_3x3": round((fl3 / (ms3 * 1e-3) / 1e12) / peak, 4) if ms3 else None,
                      "frac_1x1": round((fl1 / (ms1 * 1e-3) / 1e12) / peak, 4) if ms1 else None,
                      "ms_3x3": round(ms3 / prof_steps, 4), "ms_1x1": round(ms1 / prof_steps, 4),
                      "what": "sum of direct-conv FLOPs of every 3x3 and 1x1 conv launch over the sum of their durations "
                              "(HIP events), per forward"},
        "kernels_per_forward": [{"kernel": r[4], "kind": ("3x3", "1x1", "other")[r[0]], "launches": r[1] // prof_steps,
                                 "us_per_launch": round(1000.0 * r[2] / r[1], 2),
                                 "tflops": round(r[3] / (r[2] * 1e-3) / 1e12, 1) if r[2] > 0 else None} for r in per_kernel],
        "roofline": {"bound": "mfma", "kernel": kname, "achieved": round(achieved, 2),
                     "peak": peak, "unit": "TFLOP/s", "frac": round(achieved / peak, 4),
                     "traffic": measured_traffic() if headline else None, "avg_launch_ms": round(avg_ms, 5), "launches": n_k,
                     "timing": f"HIP events around each launch over {prof_steps} eager forwards after the timed steps"},
    }
    if vendor is not None:
        # The same kernel against what a vendor fp16 GEMM sustains on this box
        # with random operands (power-limited clock), beside the datasheet peak.
        result["roofline"]["vendor_gemm_sustained"] = vendor
        if vendor["tflops"]:
            result["roofline"]["frac_of_vendor_gemm"] = round(achieved / vendor["tflops"], 4)
    if (batch == 1 or args.latency) and not args.no_latency:
        result["latency"] = latency(h, call, lm, cfg, batch)
    if not args.no_serve and batch > 1:
        result["pcie_inclusive"] = serve_rate(lm, cfg, batch)
        if cfg.arch.num_input == 22 and cfg.arch.num_global == 19:  # the inputs of fillRowV7
            result["featurize"] = featurize_rate(batch)
            result["featurize_plus_serve"] = featurize_serve_rate(lm, cfg, batch)
    if not args.no_cpu:
        print("bench: timing CPU baseline", file=sys.stderr, flush=True)
        result["cpu_baseline"] = cpu_baseline(path)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
