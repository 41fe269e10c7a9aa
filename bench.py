"""Benchmark of the FlashPrefill gfx950 path on the headline workload (config 3).

One step = one full ``flash_prefill_varlen_func`` call (plan -> pool K ->
search -> block-sparse attention) over a 131072-token single sequence with
Llama-3-8B head shapes (32 q / 8 kv heads, d = 128, bf16, causal, block 128),
inputs resident in HBM. Prints ONE JSON line (rank 0); each field is defined
where main() fills it in.

    python bench.py [--gpus 1] [--steps 10] [--warmup 3]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = ("128K prefill attn latency (ms) + effective TFLOPS, speedup vs dense at 1 MI355X")
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_FP32_TFLOPS = 157.3    # MI355X dense fp32 MFMA (config 1 runs fp32 inputs)
PEAK_HBM_GBPS = 8000.0
MAX_GFX_MHZ = 2400.0         # MI355X shader clock ceiling (amd-smi gfx max_clk); the bf16 peak is quoted at it


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", type=int, default=3,
                    help="3 (default): the bench line (with configs 1, 2, 4 and 5 as "
                         "sub-reports); 1, 2, 4 or 5: that config's report line alone (1: CPU "
                         "oracle at 4K fp32, 2: Llama shapes at 4K/16K/32K, 4: Qwen2.5 varlen "
                         "ragged, 5: 64K decoder-layer attention block)")
    ap.add_argument("--seq-len", type=int, default=131072)
    ap.add_argument("--seed", type=int, default=128)
    ap.add_argument("--alpha", type=float, default=0.18)
    ap.add_argument("--no-dense", action="store_true", help="skip the dense baselines")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--no-clock", action="store_true",
                    help="skip the shader-clock / socket-power sampling (amd-smi child "
                         "processes); for runs under rocprofv3, whose preloaded library would "
                         "start the GPU in every child process")
    ap.add_argument("--no-configs", action="store_true",
                    help="leave out the configs 1, 2, 4 and 5 sub-reports of the bench line")
    ap.add_argument("--cpu-seconds", type=float, default=20.0,
                    help="time budget of the CPU baseline sample")
    ap.add_argument("--collect-traffic", action="store_true",
                    help="measure the attention, pooling and search kernels' bytes per "
                         "launch beyond L2 with two rocprofv3 --pmc passes (read and write "
                         "request counts by size, checked on a 1 GiB copy), and write the "
                         "summaries under profiles/")
    ap.add_argument("--traffic-probe", action="store_true",
                    help=argparse.SUPPRESS)  # child of --collect-traffic: one attention + one copy
    ap.add_argument("--power", action="store_true",
                    help="run the attention stage back to back for --power-seconds while "
                         "sampling socket power with amd-smi; print time, power and energy "
                         "per launch")
    ap.add_argument("--power-seconds", type=float, default=4.0)
    ap.add_argument("--attn-sweep", action="store_true",
                    help="attention stage alone at 128K over selection settings: a window sweep "
                         "(alpha 1, last-n 0; linear fit of time against blocks per row gives "
                         "the per-block and per-row cost), the bench setting, a near-dense "
                         "alpha and every block (alpha 0); one JSON line per setting, for "
                         "clock counters under rocprofv3")
    return ap.parse_args()


def timed(fn, reps, stream=None):
    """Average milliseconds of fn() over reps, with HIP events on the current stream."""
    import torch
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    s.record()
    for _ in range(reps):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / reps


COPY_BYTES = 1 << 30  # check copy: 1 GiB read + 1 GiB written


ATTN_KERNEL = "k_attn"


def attn_kernel_name():
    return ATTN_KERNEL


def traffic_file(S):
    return os.path.join(ROOT, "profiles", f"attn_traffic_llama{S // 1024}k_{ATTN_KERNEL}.json")


def stage_traffic_file(S):
    return os.path.join(ROOT, "profiles", f"search_pool_traffic_llama{S // 1024}k.json")


def traffic_probe(args):
    """One call of each stage (plan, pool, search, attention) on the bench
    input and one plain 1 GiB copy, for the counter passes of
    --collect-traffic."""
    import torch
    from flashprefill_amd import synth
    from flashprefill_amd.runtime import FlashPrefillCall
    dev = torch.device("cuda:0")
    spec = synth.llama_spec(args.seq_len, seed=args.seed)
    q, k, v, cu = synth.make_inputs(spec, device=dev)
    o = torch.empty_like(q)
    call = FlashPrefillCall(q, k, v, o, cu, args.seq_len, alpha=args.alpha)
    call.plan(); call.pool(); call.search()
    call.attn()
    src = torch.empty(COPY_BYTES // 4, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    print("traffic probe done", flush=True)


# L2 -> fabric request counters of one pass each (at most 4 TCC counters per
# pass). On gfx950 with this ROCm, reads leave L2 as 128-byte requests that
# FETCH_SIZE counts as 64 bytes (its 128-byte term, TCC_BUBBLE, reads 0: a
# kernel reading exactly 1 GiB with coalesced 16-byte loads reports 0.5 GiB),
# so read bytes come from the raw counts; writes are 64-byte requests, which
# WRITE_SIZE counts correctly.
TRAFFIC_PASSES = {
    "read": ["TCC_EA0_RDREQ_sum", "TCC_EA0_RDREQ_32B_sum", "TCC_EA0_RDREQ_64B_sum"],
    "write": ["TCC_EA0_WRREQ_sum", "TCC_EA0_WRREQ_64B_sum"],
}


def traffic_bytes(kind, c):
    """Bytes from one dispatch's counters (dict name -> value)."""
    if kind == "read":
        n, n32, n64 = c["TCC_EA0_RDREQ_sum"], c["TCC_EA0_RDREQ_32B_sum"], c["TCC_EA0_RDREQ_64B_sum"]
        return 32.0 * n32 + 64.0 * n64 + 128.0 * (n - n32 - n64)
    n, n64 = c["TCC_EA0_WRREQ_sum"], c["TCC_EA0_WRREQ_64B_sum"]
    return 32.0 * (n - n64) + 64.0 * n64


def collect_traffic(args):
    """Two rocprofv3 counter passes over --traffic-probe (started as child
    processes; this process never touches the GPU): L2 -> fabric read and
    write request counts of the attention, pooling and search dispatches,
    converted to bytes by request size. The 1 GiB copy in the same pass is
    the check: its read and write bytes must come out at 1 GiB each."""
    import csv
    import glob
    import subprocess
    import tempfile
    probe = [sys.executable, "-u", os.path.abspath(__file__), "--traffic-probe",
             "--seq-len", str(args.seq_len), "--seed", str(args.seed), "--alpha", str(args.alpha)]
    res = {}
    for kind, ctrs in TRAFFIC_PASSES.items():
        with tempfile.TemporaryDirectory() as td:
            cmd = ["rocprofv3", "--pmc"] + ctrs + ["--output-format", "csv", "-d", td, "-o", "p",
                                                   "--"] + probe
            print("bench: " + " ".join(cmd), file=sys.stderr, flush=True)
            r = subprocess.run(["timeout", "-s", "KILL", "300"] + cmd, capture_output=True, text=True)
            if r.returncode != 0:
                raise SystemExit(f"rocprofv3 pass {kind} failed ({r.returncode}): {r.stderr[-800:]}")
            disp = {}  # (stage, dispatch id) -> {counter: value}
            for f in glob.glob(f"{td}/**/*counter_collection.csv", recursive=True):
                for row in csv.DictReader(open(f)):
                    name = row["Kernel_Name"]
                    key = ("attn" if f"fp::{attn_kernel_name()}<" in name else
                           "pool" if "fp::k_pool<" in name else
                           "search" if "fp::k_search<" in name else
                           "copy" if "copy" in name.lower() else None)
                    if key is None or row["Counter_Name"] not in ctrs:
                        continue
                    d = disp.setdefault((key, int(row["Dispatch_Id"])), {})
                    d[row["Counter_Name"]] = d.get(row["Counter_Name"], 0.0) + float(row["Counter_Value"])
            byts = {}
            for (key, did), c in sorted(disp.items(), key=lambda x: x[0][1]):
                if all(x in c for x in ctrs):
                    byts.setdefault(key, []).append(traffic_bytes(kind, c))
            if "attn" not in byts or "copy" not in byts:
                raise SystemExit(f"pass {kind}: dispatches not found ({sorted(byts)})")
            # the last dispatch of each stage; the probe's last copy is the 1 GiB one
            # (earlier copy kernels are the input conversions)
            res[kind] = {st: v[-1] for st, v in byts.items() if st != "copy"}
            res[kind]["copy_check"] = byts["copy"][-1] / COPY_BYTES
    rd, wr = res["read"], res["write"]
    method = ("rocprofv3 --pmc " + " ".join(TRAFFIC_PASSES["read"]) + " (read bytes = 128 x "
              "128-byte + 64 x 64-byte + 32 x 32-byte requests), then --pmc " +
              " ".join(TRAFFIC_PASSES["write"]) + " (write bytes = 64 x 64-byte + 32 x 32-byte "
              "requests), over python -u bench.py --traffic-probe")
    out = {
        "kernel": attn_kernel_name(), "workload": f"bench.py config 3, seq_len {args.seq_len}, "
        f"seed {args.seed}, alpha {args.alpha}",
        "command": "python bench.py --collect-traffic", "method": method,
        "check": {"copy_1GiB_read_ratio": rd["copy_check"], "copy_1GiB_write_ratio": wr["copy_check"]},
        "fetch_bytes": rd["attn"], "write_bytes": wr["attn"],
        "traffic_bytes": rd["attn"] + wr["attn"],
    }
    os.makedirs(os.path.dirname(traffic_file(args.seq_len)), exist_ok=True)
    with open(traffic_file(args.seq_len), "w") as fh:
        json.dump(out, fh, indent=1)
    print(json.dumps(out), flush=True)
    stages = {"workload": out["workload"], "command": out["command"], "method": method,
              "check": out["check"]}
    for st, kern in (("pool", "k_pool"), ("search", "k_search")):
        if st in rd and st in wr:
            stages[kern] = {"fetch_bytes": rd[st], "write_bytes": wr[st],
                            "traffic_bytes": rd[st] + wr[st]}
    with open(stage_traffic_file(args.seq_len), "w") as fh:
        json.dump(stages, fh, indent=1)
    print(json.dumps(stages), flush=True)


def power_run(args):
    """Attention launches back to back on the bench input for --power-seconds,
    socket power sampled every 0.2 s with `amd-smi metric -p` in a thread (a
    child process per sample; this process owns the GPU). Median power over
    the run (the first two samples dropped), HIP-event time per launch, and
    their product: energy per launch."""
    import statistics
    import subprocess
    import threading
    import torch
    from flashprefill_amd import synth
    from flashprefill_amd.runtime import FlashPrefillCall
    dev = torch.device("cuda:0")
    spec = synth.llama_spec(args.seq_len, seed=args.seed)
    q, k, v, cu = synth.make_inputs(spec, device=dev)
    o = torch.empty_like(q)
    call = FlashPrefillCall(q, k, v, o, cu, args.seq_len, alpha=args.alpha)
    call.plan(); call.pool(); call.search(); call.attn()
    torch.cuda.synchronize()
    watts, stop = [], threading.Event()

    def sample():
        while not stop.is_set():
            r = subprocess.run(["amd-smi", "metric", "-p", "-g", "0", "--csv"],
                               capture_output=True, text=True)
            rows = [ln.split(",") for ln in r.stdout.strip().splitlines() if ln]
            if len(rows) >= 2 and "socket_power" in rows[0]:
                try:
                    watts.append(float(rows[1][rows[0].index("socket_power")]))
                except ValueError:
                    pass
            stop.wait(0.2)

    th = threading.Thread(target=sample)
    th.start()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    n, t0 = 0, time.time()
    e0.record()
    while time.time() - t0 < args.power_seconds:
        for _ in range(20):
            call.attn()
        torch.cuda.synchronize()
        n += 20
    e1.record()
    torch.cuda.synchronize()
    stop.set()
    th.join()
    ms = e0.elapsed_time(e1) / n
    w = statistics.median(watts[2:]) if len(watts) > 2 else None
    print(json.dumps({"kernel": attn_kernel_name(), "workload": f"bench.py config 3, seq_len "
                      f"{args.seq_len}, seed {args.seed}, alpha {args.alpha}",
                      "launches": n, "ms_per_launch": round(ms, 4), "power_samples": len(watts),
                      "socket_power_W_median": w,
                      "energy_J_per_launch": round(w * ms / 1e3, 3) if w else None}), flush=True)


def clock_under_load(stage, seconds):
    """The shader clock (MHz, mean over the XCDs' gfx clocks) and socket power
    (W) while `stage` runs back to back for `seconds`: medians of samples of
    `amd-smi metric -c` / `-p` taken every 0.2 s in a thread (a child process
    per sample; this process owns the GPU), the first two dropped. None where
    amd-smi is not available."""
    import shutil
    import statistics
    import subprocess
    import threading
    import torch
    if shutil.which("amd-smi") is None:
        return None
    clk, watts, stop = [], [], threading.Event()

    def read(flag):
        r = subprocess.run(["amd-smi", "metric", flag, "-g", "0", "--csv"], capture_output=True,
                           text=True, timeout=20)
        rows = [ln.split(",") for ln in r.stdout.strip().splitlines() if ln]
        return dict(zip(rows[0], rows[1])) if len(rows) >= 2 else {}

    def sample():
        while not stop.is_set():
            try:
                c = read("-c")
                g = [float(v) for kk, v in c.items() if kk.startswith("gfx_") and
                     kk.endswith("_clk") and v.replace(".", "", 1).isdigit()]
                if g:
                    clk.append(sum(g) / len(g))
                p = read("-p").get("socket_power", "")
                if p.replace(".", "", 1).isdigit():
                    watts.append(float(p))
            except (OSError, subprocess.SubprocessError, ValueError):
                pass
            stop.wait(0.2)

    th = threading.Thread(target=sample)
    th.start()
    t0 = time.time()
    while time.time() - t0 < seconds:
        for _ in range(10):
            stage()
        torch.cuda.synchronize()
    stop.set()
    th.join()
    if len(clk) < 3:
        return None
    return {"gfx_mhz": round(statistics.median(clk[2:]), 1),
            "socket_W": round(statistics.median(watts[2:]), 1) if len(watts) > 2 else None,
            "samples": len(clk)}


def attn_sweep(args):
    """Attention stage at --seq-len over several selections (see --attn-sweep)."""
    import statistics
    import torch
    from flashprefill_amd import synth
    from flashprefill_amd.runtime import FlashPrefillCall
    dev = torch.device("cuda:0")
    S = args.seq_len
    spec = synth.llama_spec(S, seed=args.seed)
    q, k, v, cu = synth.make_inputs(spec, device=dev)
    o = torch.empty_like(q)
    rows = spec.num_q_heads * ((S + 127) // 128)
    fit = []
    cases = [dict(alpha=1.0, window_size=w, last_n_block=0) for w in (1, 2, 4, 8, 16, 32, 64)]
    cases += [dict(alpha=args.alpha, window_size=4, last_n_block=2),
              dict(alpha=0.01, window_size=4, last_n_block=2),
              dict(alpha=0.0, window_size=4, last_n_block=2)]
    for cs in cases:
        call = FlashPrefillCall(q, k, v, o, cu, S, **cs)
        call.plan(); call.pool(); call.search(); call.attn()
        n = int(call.counts()[:, :rows // spec.num_q_heads].sum().item())
        ms = median([timed(call.attn, 3 if cs["alpha"] else 1) for _ in range(3)])
        rec = dict(cs, blocks=n, blocks_per_row=round(n / rows, 3), ms_attn=round(ms, 4),
                   executed_tflops=round(4 * 128 * 128 * spec.head_dim * n / ms / 1e9, 1))
        print(json.dumps(rec), flush=True)
        if cs["alpha"] == 1.0:
            fit.append((n / rows, ms))
    xs, ys = [x for x, _ in fit], [y for _, y in fit]
    mx, my = statistics.mean(xs), statistics.mean(ys)
    slope = sum((x - mx) * (y - my) for x, y in zip(xs, ys)) / sum((x - mx) ** 2 for x in xs)
    # one row per (head, q-block); time per row and per block in slot units:
    # rows * cost / (2 workgroups per CU x CUs)
    slots = 2 * torch.cuda.get_device_properties(dev).multi_processor_count
    print(json.dumps({"window_sweep_fit": {
        "us_per_block_per_slot": round(slope * 1e3 * slots / rows, 3),
        "us_per_row_per_slot": round((my - slope * mx) * 1e3 * slots / rows, 3),
        "slots": slots}}), flush=True)


def dense_causal_flops(S, Hq, d):
    return 2.0 * d * Hq * S * (S + 1)


def cpu_baseline(q, k, v, alpha, budget_s):
    """The oracle (a CPU restatement of the reference algorithm) on a bounded
    sample of the same workload: every query head, q-blocks visited from the
    last one down in strides of 32, until ``budget_s`` seconds are used.
    Rate = dense-causal FLOPs of the sampled rows / CPU time (same unit as
    ``value``)."""
    import torch
    from oracle import flashprefill_oracle as O
    torch.set_num_threads(cpu_threads())
    S, Hq, d = q.shape
    nb = (S + 127) // 128
    qc, kc, vc = q.cpu(), k.cpu(), v.cpu()
    t0 = time.perf_counter()
    mk = O.pool_k(kc)
    rows_done, flops = 0, 0.0
    stride_rows = [i for i in range(nb - 1, -1, -32)]
    for i in stride_rows:
        rows = [(h, i) for h in range(Hq)]
        O.flashprefill_rows(qc, kc, vc, rows, alpha=alpha, attention_sink=2, window=4,
                            last_n=2, native=False, mk=mk)
        rows_done += len(rows)
        q0, q1 = i * 128, min(S, (i + 1) * 128)
        flops += Hq * 4.0 * d * sum(range(q0 + 1, q1 + 1))
        if time.perf_counter() - t0 > budget_s:
            break
    el = time.perf_counter() - t0
    return {
        "value": flops / el / 1e12,
        "unit": "TFLOP/s (effective)",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"oracle (pool K of all {nb} blocks, then score+select+attention) on "
                   f"{rows_done} (head, q-block) rows of the same 128K input: all {Hq} heads x "
                   f"q-blocks {nb - 1}, {nb - 33}, ... ; {el:.1f} s on "
                   f"{platform.processor() or platform.machine()}, os.cpu_count()={os.cpu_count()}"),
    }


def median(xs):
    xs = sorted(xs)
    return xs[len(xs) // 2]


def measure(q, k, v, cu, seq_lens, alpha, steps, warmup, dense_baselines, dense_reps=3,
            rounds=1, min_region_ms=0.0):
    """Time one operator configuration (HIP events on the launch stream):
    the public entry point flash_prefill_varlen_func (its cached workspace
    and argument handling included: what a caller pays per call), the same
    call on a prebuilt descriptor, the plan, search and attention stages,
    density, and the dense baselines (this kernel with every causal block
    selected, torch SDPA flash per sequence with the KV heads expanded;
    each the median of ``dense_reps`` timings). With ``rounds`` > 1 the
    public and prebuilt calls are timed alternately that many times (``steps``
    calls each) and the medians are reported: short configurations otherwise
    carry the first timed region's ramp-up (their first round runs up to
    ~10 % slower). With ``min_region_ms`` the number of calls per timed
    region is raised until the region lasts about that long (a 4K call is
    ~0.1 ms: five calls make a 0.5 ms region, where launch jitter and the
    clock's ramp weigh in); the count used is reported as ``steps``."""
    import torch
    from flashprefill_amd import flash_prefill_varlen_func
    from flashprefill_amd.runtime import FlashPrefillCall
    T, Hq, d = q.shape
    Hkv = k.shape[1]
    S_max = max(seq_lens)
    o = torch.empty_like(q)

    def public_call():
        flash_prefill_varlen_func(q, k, v, o, cu, S_max, alpha, 128, 2, 4, 2)

    call = FlashPrefillCall(q, k, v, o, cu, S_max, alpha=alpha, attention_sink=2,
                            window_size=4, last_n_block=2)
    for _ in range(warmup):
        public_call()
        call.run()
    torch.cuda.synchronize()
    if min_region_ms > 0:
        est = timed(call.run, 3)
        steps = max(steps, min(400, math.ceil(min_region_ms / max(est, 1e-3))))
    print("bench: timing", file=sys.stderr, flush=True)
    pub_ms, pre_ms = [], []
    for _ in range(rounds):
        pub_ms.append(timed(public_call, steps))
        pre_ms.append(timed(call.run, steps))
    ms_total, ms_prebuilt = median(pub_ms), median(pre_ms)

    # t_search is pool + score + select, the search of the reference's path
    # (its block-table setup is orchestration); the plan kernel, which builds
    # the work tables of both the search and the attention, is timed apart
    # and reported beside it
    def search_stage():
        call.pool()
        call.search()

    ms_plan = timed(call.plan, max(3, steps))
    ms_search = timed(search_stage, max(3, steps))
    # the same split inside full calls: events around the plan, the search
    # stages and the attention of each staged call (same kernels as call.run())
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(max(3, steps))]
    torch.cuda.synchronize()
    for e4 in ev:
        e4[0].record()
        call.plan()
        e4[1].record()
        search_stage()
        e4[2].record()
        call.attn()
        e4[3].record()
    torch.cuda.synchronize()
    in_call_plan = sum(e4[0].elapsed_time(e4[1]) for e4 in ev) / len(ev)
    in_call_search = sum(e4[1].elapsed_time(e4[2]) for e4 in ev) / len(ev)
    in_call_total = sum(e4[0].elapsed_time(e4[3]) for e4 in ev) / len(ev)
    ms_pool = timed(call.pool, max(3, steps))
    ms_score = timed(call.search, max(3, steps))
    ms_attn = timed(call.attn, max(3, steps))
    assert call.status() == 0
    tile, _, _, _ = call.seq_tables()
    n_exec = int(call.counts()[:, :tile[-1]].sum().item())
    causal_blocks = sum(Hq * ((s + 127) // 128) * ((s + 127) // 128 + 1) // 2 for s in seq_lens)
    exec_tflops = 4.0 * 128 * 128 * d * n_exec / (ms_attn * 1e-3) / 1e12
    dense_flops = sum(dense_causal_flops(s, Hq, d) for s in seq_lens)
    out = {
        "steps": steps, "rounds": rounds,
        "ms_total": ms_total, "ms_total_prebuilt_call": ms_prebuilt,
        "ms_search": ms_search, "ms_attn": ms_attn,
        "ms_pool": ms_pool, "ms_score": ms_score, "ms_plan": ms_plan,
        "search_share": ms_search / ms_total,
        "search_share_incl_plan": (ms_search + ms_plan) / ms_total, "executed_blocks": n_exec,
        "in_call_split": {"ms_plan": in_call_plan, "ms_search": in_call_search,
                          "ms_total": in_call_total,
                          "search_share": in_call_search / in_call_total,
                          "search_share_incl_plan": (in_call_plan + in_call_search) / in_call_total},
        "density": n_exec / causal_blocks, "executed_tflops": exec_tflops,
        "mfma_frac": exec_tflops / PEAK_BF16_TFLOPS,
        "effective_tflops": dense_flops / (ms_total * 1e-3) / 1e12,
        "search_algorithmic_GBps": (q.numel() + k.numel()) * q.element_size() /
                                   (ms_search * 1e-3) / 1e9,
        "dense": {},
    }
    if not dense_baselines:
        return out
    print("bench: dense baselines", file=sys.stderr, flush=True)
    dense = out["dense"]
    o2 = torch.empty_like(q)
    dcall = FlashPrefillCall(q, k, v, o2, cu, S_max, alpha=0.0, attention_sink=2,
                             window_size=4, last_n_block=2)
    dcall.plan(); dcall.pool(); dcall.search()
    dcall.attn()
    dense["own_all_blocks_attn_ms"] = median([timed(dcall.attn, 1) for _ in range(dense_reps)])
    dense["own_all_blocks_tflops"] = dense_flops / (dense["own_all_blocks_attn_ms"] * 1e-3) / 1e12
    del o2, dcall
    try:
        from torch.nn.attention import SDPBackend, sdpa_kernel
        offs = [0]
        for s_ in seq_lens:
            offs.append(offs[-1] + s_)
        parts = []
        for b in range(len(seq_lens)):
            a0, a1 = offs[b], offs[b + 1]
            parts.append((q[a0:a1].transpose(0, 1).unsqueeze(0),
                          k[a0:a1].repeat_interleave(Hq // Hkv, dim=1).transpose(0, 1).unsqueeze(0),
                          v[a0:a1].repeat_interleave(Hq // Hkv, dim=1).transpose(0, 1).unsqueeze(0)))

        def sdpa_all():
            for qh, kh, vh in parts:
                torch.nn.functional.scaled_dot_product_attention(qh, kh, vh, is_causal=True)

        with sdpa_kernel([SDPBackend.FLASH_ATTENTION]):
            sdpa_all()
            dense["sdpa_flash_ms"] = median([timed(sdpa_all, 1) for _ in range(dense_reps)])
        dense["sdpa_flash_tflops"] = dense_flops / (dense["sdpa_flash_ms"] * 1e-3) / 1e12
        del parts
    except Exception as exc:  # the flash backend is the only one that fits long sequences
        dense["sdpa_flash_error"] = f"{type(exc).__name__}: {exc}"[:200]
    cands = [x for x in (dense.get("sdpa_flash_ms"), dense.get("own_all_blocks_attn_ms")) if x]
    dense["reps"] = dense_reps
    if cands:
        dense["fastest_dense_ms"] = min(cands)
        dense["speedup_vs_dense"] = min(cands) / ms_total
    return out


def _rounded(x):
    if isinstance(x, float):
        return round(x, 4)
    if isinstance(x, dict):
        return {k: _rounded(v) for k, v in x.items()}
    return x


def cpu_threads():
    """Host threads for the CPU baseline: the box's CPU share (OMP_NUM_THREADS
    when set, else os.cpu_count())."""
    return max(1, int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1)))


def config1_report(args):
    """Config 1 (4096 tokens, 8 q / 2 kv heads, d = 64, fp32, seed 0, sinks
    and 16 stripe columns): the oracle, i.e. the CPU restatement of the
    reference's native forward (ops/flashprefill_native_forward.py:405-499),
    timed in full on the host: median of 5 runs after 1 warm-up."""
    import torch
    from flashprefill_amd import synth
    from oracle import flashprefill_oracle as O
    torch.set_num_threads(cpu_threads())
    spec = synth.config1_spec(seed=0)
    q, k, v, _ = synth.make_inputs(spec)
    qb, kb, vb = q.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0)
    times = []
    for rep in range(6):
        t0 = time.perf_counter()
        res = O.flash_prefill(qb, kb, vb, 128, 2, 4, args.alpha, 2, 0)
        if rep:
            times.append((time.perf_counter() - t0) * 1e3)
    sel = res.traces[0].sel
    nb = sel.shape[-1]
    S, Hq, d = q.shape
    ms = median(times)
    gpu = {}
    if torch.cuda.is_available():
        # the same call on the GPU (fp32 kernels), for the GPU / CPU ratio
        from flashprefill_amd import flash_prefill
        dev = torch.device("cuda:0")
        qd, kd, vd = qb.to(dev), kb.to(dev), vb.to(dev)
        od = torch.empty_like(qd)

        def gpu_call():
            flash_prefill(qd, kd, vd, od, 128, 2, 4, args.alpha, 2, 0)

        gpu_call()
        gpu_ms = timed(gpu_call, 20)
        err = (od[0].cpu() - res.out[0]).abs()
        # the attention stage alone (fp32 MFMA kernel) on the same input in
        # the batched layout: executed block FLOPs / its time, against the
        # fp32 MFMA peak
        from flashprefill_amd.runtime import FlashPrefillCall
        call = FlashPrefillCall(qd[0], kd[0], vd[0], torch.empty_like(qd[0]), None, S,
                                alpha=args.alpha, attention_sink=2, window_size=4,
                                last_n_block=2, native_normalize=True, batch=1,
                                uniform_seq_len=S)
        call.run()
        n_exec = int(call.counts()[:, :nb].sum().item())
        attn_ms = timed(call.attn, 20)
        exec_tf = 4.0 * 128 * 128 * d * n_exec / (attn_ms * 1e-3) / 1e12
        eff_tf = dense_causal_flops(S, Hq, d) / (gpu_ms * 1e-3) / 1e12
        gpu = {"gpu_ms": gpu_ms, "gpu_effective_tflops": eff_tf,
               "gpu_effective_frac_of_fp32_mfma_peak": eff_tf / PEAK_FP32_TFLOPS,
               "gpu_attn_ms": attn_ms, "gpu_executed_tflops": exec_tf,
               "gpu_attn_frac_of_fp32_mfma_peak": exec_tf / PEAK_FP32_TFLOPS,
               "fp32_mfma_peak_tflops": PEAK_FP32_TFLOPS,
               "gpu_speedup_vs_cpu": ms / gpu_ms,
               "gpu_vs_cpu_max_abs_diff": f"{float(err.max()):.3e}", "gpu_dtype": "fp32"}
    return _rounded({**gpu,
        "case": "config 1: 4096 tokens, 8 q / 2 kv heads, d 64, fp32, native forward, alpha "
                f"{args.alpha}", "cpu_ms_median": ms, "cpu_ms_runs": times,
        "cpu_effective_tflops": dense_causal_flops(S, Hq, d) / (ms * 1e-3) / 1e12,
        "density": int(sel.sum()) / (Hq * nb * (nb + 1) // 2), "cores": torch.get_num_threads(),
        "cpu": f"{platform.processor() or platform.machine()}, os.cpu_count()={os.cpu_count()}",
        "kind": "port (oracle/flashprefill_oracle.py flash_prefill)"})


def config_cases(config):
    from flashprefill_amd import synth
    if config == 2:
        return [(synth.llama_spec(S, seed=seed), 0.18, f"{S // 1024}K")
                for S, seed in ((4096, 4), (16384, 16), (32768, 32))]
    if config == 3:
        # config 3's shapes at 262144 tokens: the length of the reference's
        # 256K headline (README.md:6)
        return [(synth.llama_spec(262144, seed=256), 0.18, "256K, config 3 shapes")]
    if config == 4:
        return [(synth.qwen_varlen_spec(), 0.08,
                 "ragged {256K, 64K, 17K, 3K, 1K}, Qwen2.5-7B heads")]
    if config == "tp":
        # one rank's share of config 3 under tensor parallelism over heads
        # (what vLLM runs, README.md:33): 32 / TP query and 8 / TP KV heads at
        # the full 128K length, for TP = 8 and 4
        return [(synth.SynthSpec(seq_lens=(131072,), num_q_heads=32 // tp, num_kv_heads=8 // tp,
                                 head_dim=128, seed=128), 0.18,
                 f"128K, one TP = {tp} rank ({32 // tp} q / {8 // tp} kv heads)") for tp in (8, 4)]
    raise SystemExit(f"--config {config}: 1, 2, 3, 4 or 5")


def config_results(config, steps, warmup, dense):
    """Configs 2 (Llama shapes at 4K / 16K / 32K) and 4 (Qwen2.5 varlen
    ragged batch), config 3 at 256K and one tensor-parallel rank's share of
    config 3 ("tp"): one result per case."""
    import torch
    from flashprefill_amd import synth
    dev = torch.device("cuda:0")
    results = []
    for spec, alpha, name in config_cases(config):
        print(f"bench: config {config} {name}", file=sys.stderr, flush=True)
        q, k, v, cu = synth.make_inputs(spec, device=dev)
        r = measure(q, k, v, cu, list(spec.seq_lens), alpha, steps, warmup, dense, rounds=3,
                    min_region_ms=20.0)
        r.update({"case": name, "seq_lens": list(spec.seq_lens), "num_q_heads": spec.num_q_heads,
                  "num_kv_heads": spec.num_kv_heads, "head_dim": spec.head_dim, "alpha": alpha,
                  "seed": spec.seed})
        results.append(_rounded(r))
        del q, k, v, cu
        torch.cuda.empty_cache()
    return results


def other_config(args):
    """One JSON report line for config 1, 2, 4 or 5 alone."""
    if args.config == 5:
        print(json.dumps(decoder_layer_report(args)), flush=True)
        return
    if args.config == 1:
        print(json.dumps({"report": "config 1", **config1_report(args)}), flush=True)
        return
    results = config_results(args.config, args.steps, args.warmup, not args.no_dense)
    print(json.dumps({"report": f"config {args.config}", "n_gpus": 1, "dtype": "bf16",
                      "data": "synthetic (flashprefill_amd/synth.py)",
                      "attention_kernel": attn_kernel_name(), "results": results}), flush=True)


def decoder_layer_report(args):
    """Config 5: one prefill attention block at 64K tokens (hidden
    4096, 32 q / 4 kv heads, d = 128, bf16, RoPE theta 1e6, random-init
    weights, no q/k norm, as the config describes it): QKV projection -> RoPE ->
    FlashPrefill (varlen signature, cu_seqlens = [0, S]) -> O projection."""
    import torch
    from flashprefill_amd import flash_prefill_varlen_func
    from flashprefill_amd.attention_layer import PrefillAttention
    from flashprefill_amd.runtime import FlashPrefillCall
    dev = torch.device("cuda:0")
    S, hidden, Hq, Hkv, d, alpha = 65536, 4096, 32, 4, 128, 0.12
    layer = PrefillAttention(hidden, Hq, Hkv, d, rope_theta=1e6, alpha=alpha, device=dev, seed=5)
    g = torch.Generator(device=dev).manual_seed(5)
    x = torch.randn(S, hidden, generator=g, device=dev).to(torch.bfloat16)
    cu = torch.tensor([0, S], dtype=torch.int32, device=dev)
    for _ in range(args.warmup):
        layer(x, cu, S)
    ms_layer = timed(lambda: layer(x, cu, S), args.steps)
    ms_qkv = timed(lambda: layer.project_qkv(x, cu), args.steps)
    q, k, v = layer.project_qkv(x, cu)
    o = torch.empty_like(q)
    ms_attn = timed(lambda: flash_prefill_varlen_func(q, k, v, o, cu, S, alpha), args.steps)
    ms_oproj = timed(lambda: o.view(S, Hq * d) @ layer.w_o.t(), args.steps)
    call = FlashPrefillCall(q, k, v, torch.empty_like(q), cu, S, alpha=alpha)
    call.run()
    torch.cuda.synchronize()
    nb = S // 128
    n_exec = int(call.counts()[:, :nb].sum().item())
    density = n_exec / (Hq * nb * (nb + 1) // 2)
    del call
    # the op inside the block in the three forms of the other configs: times,
    # executed TFLOP/s and MFMA fraction, search share, and the dense
    # baselines (own kernel with every block, SDPA flash) at this shape. With
    # random-init weights the block scores are unstructured and every block
    # is selected (density 1.0): the op runs dense here.
    op = measure(q, k, v, cu, [S], alpha, args.steps, args.warmup, not args.no_dense,
                 dense_reps=1 if args.no_dense else 3)
    op_keys = ("ms_total", "ms_search", "ms_attn", "ms_plan", "search_share",
               "search_share_incl_plan", "executed_tflops", "mfma_frac", "effective_tflops",
               "density", "dense")
    rep = {"report": "config 5", "n_gpus": 1, "dtype": "bf16",
           "data": "synthetic: hidden states ~ N(0,1), random-init weights (seed 5); the "
                   "unstructured scores select every block (density 1.0)",
           "attention_kernel": attn_kernel_name(),
           "config": {"seq_len": S, "hidden": hidden, "num_q_heads": Hq, "num_kv_heads": Hkv,
                      "head_dim": d, "rope_theta": 1e6, "alpha": alpha, "qk_norm": False},
           "ms_layer": ms_layer, "ms_qkv_proj_rope": ms_qkv, "ms_flashprefill": ms_attn,
           "ms_o_proj": ms_oproj, "attention_share": ms_attn / ms_layer, "density": density,
           "qkv_proj_tflops": 2.0 * S * hidden * (Hq + 2 * Hkv) * d / (ms_qkv * 1e-3) / 1e12,
           "op": {kk: op[kk] for kk in op_keys if kk in op}}
    if not args.no_dense:
        from torch.nn.attention import SDPBackend, sdpa_kernel
        qh = q.transpose(0, 1).unsqueeze(0)
        kh = k.repeat_interleave(Hq // Hkv, dim=1).transpose(0, 1).unsqueeze(0)
        vh = v.repeat_interleave(Hq // Hkv, dim=1).transpose(0, 1).unsqueeze(0)
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION]):
            torch.nn.functional.scaled_dot_product_attention(qh, kh, vh, is_causal=True)
            ms_dense = median([timed(lambda: torch.nn.functional.scaled_dot_product_attention(
                qh, kh, vh, is_causal=True), 1) for _ in range(3)])
        rep["ms_dense_attention_sdpa_flash"] = ms_dense
        rep["ms_layer_with_dense_attention"] = ms_layer - ms_attn + ms_dense
        rep["layer_speedup_vs_dense"] = rep["ms_layer_with_dense_attention"] / ms_layer
        own = op["dense"].get("own_all_blocks_attn_ms")
        if own:
            rep["op_speedup_vs_own_dense_kernel"] = own / ms_attn
    return _rounded(rep)


def main():
    args = parse()
    if args.collect_traffic:
        collect_traffic(args)
        return
    if args.traffic_probe:
        traffic_probe(args)
        return
    if args.power:
        power_run(args)
        return
    if args.attn_sweep:
        attn_sweep(args)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (one MI355X per box); "
              "--gpus N with N > 1 is not supported", file=sys.stderr)
        sys.exit(2)
    import torch
    from flashprefill_amd import synth

    if args.config != 3:
        other_config(args)
        return
    S = args.seq_len
    spec = synth.llama_spec(S, seed=args.seed)
    print(f"bench: generating {S}-token structured input on cuda:0", file=sys.stderr, flush=True)
    q, k, v, cu = synth.make_inputs(spec, device=torch.device("cuda:0"))
    Hq, Hkv, d = spec.num_q_heads, spec.num_kv_heads, spec.head_dim
    r = measure(q, k, v, cu, [S], args.alpha, args.steps, args.warmup, not args.no_dense)
    ms_total, ms_search, ms_attn = r["ms_total"], r["ms_search"], r["ms_attn"]
    n_exec, density, exec_tflops, eff_tflops = (r["executed_blocks"], r["density"],
                                                r["executed_tflops"], r["effective_tflops"])
    search_gbps = r["search_algorithmic_GBps"]
    dense = r["dense"]

    # shader clock and socket power while the attention, then the search,
    # runs back to back: both stages run below the 2.4 GHz clock ceiling,
    # held there by the card's power limit
    clock = None
    if not args.no_clock:
        print("bench: clock under load", file=sys.stderr, flush=True)
        from flashprefill_amd.runtime import FlashPrefillCall
        ccall = FlashPrefillCall(q, k, v, torch.empty_like(q), cu, S, alpha=args.alpha)
        ccall.plan(); ccall.pool(); ccall.search(); ccall.attn()

        def search_only():
            ccall.pool()
            ccall.search()
        clock = {"attention": clock_under_load(ccall.attn, 2.0),
                 "search": clock_under_load(search_only, 2.0),
                 "max_gfx_mhz": MAX_GFX_MHZ,
                 "method": "amd-smi metric -c (mean of the 8 XCDs' gfx clocks) and -p every 0.2 s "
                           "while the stage runs back to back for 2 s; medians"}
        del ccall

    cpu = None
    if not args.no_cpu:
        print("bench: CPU baseline (oracle sample)", file=sys.stderr, flush=True)
        cpu = cpu_baseline(q, k, v, args.alpha, args.cpu_seconds)

    # HBM roofline of the pooling and search kernels: algorithmic bytes per
    # launch (pool: read K, write pooled K; search: read Q and pooled K, write
    # the index lists and counts) and the measured HBM traffic, over each
    # kernel's own time
    elt = q.element_size()
    nb = (S + 127) // 128
    algo = {"k_pool": k.numel() * elt + nb * Hkv * d * elt,
            "k_search": q.numel() * elt + nb * Hkv * d * elt + 4 * (n_exec + Hq * nb)}
    stage_ms = {"k_pool": r["ms_pool"], "k_search": r["ms_score"]}
    stage_traffic = {}
    stf = stage_traffic_file(S)
    if os.path.exists(stf):
        with open(stf) as fh:
            sj = json.load(fh)
        if str(S) in sj.get("workload", ""):
            stage_traffic = {kk: sj[kk]["traffic_bytes"] for kk in ("k_pool", "k_search")
                             if kk in sj}
    search_roofline = {"bound": "hbm", "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                       "traffic_source": os.path.relpath(stf, ROOT) if stage_traffic else None,
                       "kernels": {}}
    for kk in ("k_pool", "k_search"):
        ach = algo[kk] / (stage_ms[kk] * 1e-3) / 1e9
        ent = {"ms": round(stage_ms[kk], 4), "algorithmic_bytes": int(algo[kk]),
               "achieved": round(ach, 1), "frac": round(ach / PEAK_HBM_GBPS, 4)}
        if kk in stage_traffic:
            ent["traffic"] = int(stage_traffic[kk])
            ent["traffic_GBps"] = round(stage_traffic[kk] / (stage_ms[kk] * 1e-3) / 1e9, 1)
        search_roofline["kernels"][kk] = ent
    # the fused search is compute-bound rather than HBM-bound: its score MFMAs
    # (every causal (q-block, k-block) pair, 128 rows x d each) against the
    # bf16 MFMA peak, and its exp2 rate (128 per pair below the diagonal, 1 on it)
    pairs = Hq * nb * (nb + 1) // 2
    score_flops = 2 * 128 * d * pairs
    n_exp2 = Hq * (128 * nb * (nb - 1) // 2 + nb)
    score_tf = score_flops / (stage_ms["k_search"] * 1e-3) / 1e12
    search_roofline["kernels"]["k_search"]["compute"] = {
        "score_mfma_flops": int(score_flops), "score_mfma_tflops": round(score_tf, 1),
        "frac_of_bf16_mfma_peak": round(score_tf / PEAK_BF16_TFLOPS, 4),
        "exp2": int(n_exp2), "exp2_per_ns": round(n_exp2 / (stage_ms["k_search"] * 1e6), 1)}

    traffic, traffic_src = None, None
    tf = traffic_file(S)
    if os.path.exists(tf):
        with open(tf) as fh:
            tj = json.load(fh)
        if tj.get("kernel") == attn_kernel_name() and str(S) in tj.get("workload", ""):
            traffic = int(tj["traffic_bytes"])
            traffic_src = os.path.relpath(tf, ROOT)

    line = {
        "metric": METRIC,
        "value": round(eff_tflops, 3),
        "unit": "TFLOP/s (effective: dense-causal FLOPs / time per prefill)",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_total, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": ("synthetic: seeded structured Q/K/V ~ N(0,1)/sqrt(d) with sinks, 64 stripe "
                 "runs, rotary local band, topic segments, 8 hot blocks/head "
                 "(flashprefill_amd/synth.py)"),
        "config": {"workload": "config 3: 131072-token single-sequence prefill attention, "
                               "Llama-3-8B heads", "seq_len": S, "num_q_heads": Hq,
                   "num_kv_heads": Hkv, "head_dim": d, "block_size": 128, "alpha": args.alpha,
                   "attention_sink": 2, "window_size": 4, "last_n_block": 2, "seed": args.seed},
        # t_search = pool + score + select; the plan kernel (work tables of
        # both stages) is t_plan, and the shares including it are reported too
        "t_search_ms": round(ms_search, 4),
        "t_plan_ms": round(r["ms_plan"], 4),
        "t_attn_ms": round(ms_attn, 4),
        "search_share": round(ms_search / ms_total, 4),
        "search_share_in_call": round(r["in_call_split"]["search_share"], 4),
        "search_share_incl_plan": round(r["search_share_incl_plan"], 4),
        "search_share_incl_plan_in_call": round(r["in_call_split"]["search_share_incl_plan"], 4),
        "density": round(density, 5),
        "executed_blocks": n_exec,
        "executed_tflops": round(exec_tflops, 2),
        "search_algorithmic_GBps": round(search_gbps, 1),
        "dense": {k2: (round(v2, 4) if isinstance(v2, float) else v2) for k2, v2 in dense.items()},
        "roofline": {"bound": "mfma", "kernel": f"fp::{attn_kernel_name()} (block-sparse attention)",
                     "achieved": round(exec_tflops, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(exec_tflops / PEAK_BF16_TFLOPS, 4),
                     "traffic": traffic, "traffic_unit": "bytes per launch beyond L2 (read + "
                     "write requests by size)", "traffic_source": traffic_src,
                     "algorithmic_kv_bytes": n_exec * 2 * 128 * d * q.element_size()},
        "search_roofline": search_roofline,
        "clock": clock,
        "cpu_baseline": cpu,
    }
    if clock and clock["attention"]:
        # the same achieved rate against the peak scaled to the clock the
        # attention holds under the power limit (the nominal frac above stays
        # the reported one)
        line["roofline"]["frac_at_measured_clock"] = round(
            exec_tflops / (PEAK_BF16_TFLOPS * clock["attention"]["gfx_mhz"] / MAX_GFX_MHZ), 4)
    if not args.no_configs:
        # the other configs, measured in the same run after the headline
        # (their inputs are generated after the 128K tensors are freed)
        del q, k, v, cu
        torch.cuda.empty_cache()
        sub_steps, sub_warmup = min(args.steps, 5), min(args.warmup, 2)
        configs = {}
        for c in (2, 4):
            configs[f"config_{c}"] = config_results(c, sub_steps, sub_warmup, not args.no_dense)
        configs["config_3_256k"] = config_results(3, sub_steps, sub_warmup, not args.no_dense)
        configs["config_3_tp_ranks"] = config_results("tp", sub_steps, sub_warmup,
                                                      not args.no_dense)
        print("bench: config 5", file=sys.stderr, flush=True)
        sub = argparse.Namespace(steps=sub_steps, warmup=sub_warmup, no_dense=args.no_dense)
        configs["config_5"] = decoder_layer_report(sub)
        if not args.no_cpu:
            print("bench: config 1 (CPU oracle)", file=sys.stderr, flush=True)
            configs["config_1"] = config1_report(args)
        line["configs"] = configs
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
