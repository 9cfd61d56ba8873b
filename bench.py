"""Benchmark of the per-step sampling path on one MI355X.

Workload (the large-batch full-vocabulary top-p configuration): 256 rows x
248,320 binary32 logits of 2*t_3 (Student-t, nu = 3), top-k disabled, top-p
0.95, temperature 1.0, Gumbel draw (version 3), per-row seeds, top-20 logprobs
per row. A step is one yskn_smp_sample call over the 256 rows, inputs resident
in HBM; three input buffers rotate so that the 256 MB Infinity Cache does not
serve a step from the previous one.

Prints one JSON line: rows/s (value), us per step, the dominant kernel's
achieved HBM bandwidth against the MI355X peak (8 TB/s) from HIP events on the
launch stream (with the median and p10/p90 of per-launch event intervals), and
the CPU oracle's rows/s on a bounded sample of the same rows (the reference
algorithm restated in C: full sort, serial binary64 tail), on one thread and
on every host core.

Extra keys time the other four workloads (single row with 1,024 draws,
speculative verify of 8 rows, bf16 penalties, 64 heterogeneous rows) as
microseconds per call with their algorithmic bandwidth; they are reported
beside the headline, not in it.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "yasakani-for-mac_amd"))

METRIC = "µs/sampling step and rows/sec at V=248,320; achieved HBM GB/s vs peak"
PEAK_GBS = 8000.0
ROWS, V = 256, 248_320
ALG_BYTES = ROWS * V * 4  # one read of the logits per step


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="time budget of the CPU oracle sample (1 thread)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-configs", action="store_true", help="skip the per-workload extra keys")
    ap.add_argument("--only-config", type=int, default=0,
                    help="time only workload N (1..4) and print its line (profiling)")
    ap.add_argument("--profile-copy", action="store_true",
                    help="run a plain device copy of the workload's size (counter calibration)")
    ap.add_argument("--dump-logits", metavar="PATH",
                    help="write the workload's logits (rows x V binary32, row-major) to PATH and exit; "
                         "lib/smp_bench --logits PATH replays them without Python")
    return ap.parse_args()


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def host_threads() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def cpu_baseline(x_host, seeds, positions, budget_s, threads=1):
    """Rows/s of the C oracle (full sort, serial binary64 tail, top-20
    logprobs) on a bounded prefix of the rows; `threads` rows at a time."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from concurrent.futures import ThreadPoolExecutor

    import yskn_oracle as O

    def one(r):
        p = O.params_from_thousandths(1000, 950, 0, top_k=0, seed=seeds[r], extension=True)
        tok = O.sample(x_host[r], int(positions[r]), p)
        O.top_logprobs(x_host[r], 20)
        return tok

    done, ids = 0, []
    t0 = time.perf_counter()
    with ThreadPoolExecutor(max_workers=threads) as pool:
        while done < x_host.shape[0]:
            batch = list(range(done, min(x_host.shape[0], done + threads)))
            ids.extend(pool.map(one, batch))
            done += len(batch)
            if time.perf_counter() - t0 > budget_s and done >= 4:
                break
    dt = time.perf_counter() - t0
    return done / dt, done, ids


def event_times(torch, stream, launch, n):
    """Per-launch intervals (us) between events recorded around n back-to-back
    launches on `stream`, and the whole interval. A spin kernel is queued
    first so that every launch is enqueued before the device reaches it: the
    intervals are device time (with the gaps between launches), not host
    call overhead."""
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(n + 1)]
    if hasattr(torch.cuda, "_sleep"):
        torch.cuda._sleep(50_000_000)
    evs[0].record(stream)
    for i in range(n):
        launch(i)
        evs[i + 1].record(stream)
    torch.cuda.synchronize()
    per = [evs[i].elapsed_time(evs[i + 1]) * 1e3 for i in range(n)]
    return per, evs[0].elapsed_time(evs[n]) * 1e3


def pct(v, q):
    import numpy as np

    return float(np.percentile(np.asarray(v, float), q))


def small_configs(torch, yskn_smp, synth, only=0, steps=30, warmup=5):
    """Microseconds per call of the four smaller workloads, each a single
    C-ABI call on device-resident inputs, timed by HIP events on the launch
    stream; bandwidth is the algorithmic bytes (one read of the logits plus
    side inputs) over the median call."""
    import numpy as np

    import ctypes as C

    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream()
    res = {}

    def record(name, fn, alg_bytes, workload, extra=None):
        for i in range(warmup):
            fn(i)
        torch.cuda.synchronize()
        per, tot = event_times(torch, stream, fn, steps)
        med = pct(per, 50)
        r = {"workload": workload, "us_per_call_median": med, "us_per_call_p10": pct(per, 10),
             "us_per_call_p90": pct(per, 90), "us_per_call_mean": tot / steps,
             "algorithmic_bytes": alg_bytes, "achieved_gbs": alg_bytes / med / 1e3,
             "frac_of_hbm_peak": alg_bytes / med / 1e3 / PEAK_GBS}
        if extra:
            r.update(extra)
        res[name] = r

    L = yskn_smp.load_library()
    sptr = C.c_void_p(stream.cuda_stream)

    def prepared(name, *args):
        """One C call with arguments built once (device-resident inputs and
        outputs), so that the timed loop measures the launches only."""
        f = getattr(L, name)

        def call(i):
            st = f(*args)
            if st != 0:
                raise RuntimeError(L.yskn_smp_last_error().decode())
        return call

    def vp(t):
        return C.c_void_p(t.data_ptr())

    # 1: single row, 1,024 draws in one launch (and one draw)
    if only in (0, 1):
        x = synth.single_row(dev)
        d = yskn_smp.DeviceSampler(1, synth.V_SMALL)
        d.set_params(yskn_smp.SamplingParameters(temperature_milli=1000, top_p_milli=950, top_k=20, seed=0))
        pos = torch.arange(1024, dtype=torch.int64, device=dev).reshape(1, 1024)
        ids = torch.empty((1, 1024), dtype=torch.int32, device=dev)
        keep1 = {}
        aux1 = d._aux(1, dev, keep1, top20=True)
        record("single_row_1024_draws",
               prepared("yskn_smp_sample", d.h, vp(x), d._dtype(x), 1, synth.V_SMALL, synth.V_SMALL, vp(pos), 1024,
                        vp(ids), C.byref(aux1), sptr),
               synth.V_SMALL * 4, "1 x 151,936 f32, top-k 20, top-p 0.95, T 1.0, 1,024 positions in one call")
        p1 = torch.zeros((1, 1), dtype=torch.int64, device=dev)
        aux0 = yskn_smp.CAux()
        record("single_row_one_draw",
               prepared("yskn_smp_sample", d.h, vp(x), d._dtype(x), 1, synth.V_SMALL, synth.V_SMALL, vp(p1), 1,
                        vp(ids), C.byref(aux0), sptr),
               synth.V_SMALL * 4, "1 x 151,936 f32, top-k 20, top-p 0.95, T 1.0, one draw")
    # 2: speculative verify, 8 rows
    if only in (0, 2):
        tgt, _ = synth.spec_verify(8, dev)
        d2 = yskn_smp.DeviceSampler(8, synth.V_LARGE)
        d2.set_params(yskn_smp.SamplingParameters(temperature_milli=1000, top_p_milli=950, top_k=20, seed=0x5EC))
        drafts = torch.zeros(7, dtype=torch.int32, device=dev)
        base = torch.tensor([10_000], dtype=torch.int64, device=dev)
        eos = torch.zeros(1, dtype=torch.int32, device=dev)
        vids = torch.empty(8, dtype=torch.int32, device=dev)
        vres = torch.empty(5, dtype=torch.int32, device=dev)
        aux2 = yskn_smp.CAux()
        record("spec_verify_8",
               prepared("yskn_smp_verify", d2.h, vp(tgt), d2._dtype(tgt), 8, synth.V_LARGE, synth.V_LARGE,
                        vp(drafts), vp(base), vp(eos), 0, vp(vids), vp(vres), C.byref(aux2), None, sptr),
               8 * synth.V_LARGE * 4, "verify 8 x 248,320 f32, top-k 20, top-p 0.95, accept rule on the device")
    # 3: penalties, bf16
    if only in (0, 3):
        xb, hist = synth.penalties(dev)
        d3 = yskn_smp.DeviceSampler(1, synth.V_LARGE)
        d3.set_params(yskn_smp.SamplingParameters(temperature_milli=700, top_p_milli=900, min_p_milli=50,
                                                  top_k=20, seed=31, repetition_penalty=1.05,
                                                  presence_penalty=0.5, frequency_penalty=0.3))
        p3 = torch.zeros(1, dtype=torch.int64, device=dev)
        ids3 = torch.empty(1, dtype=torch.int32, device=dev)
        keep3 = {}
        aux3 = d3._aux(1, dev, keep3, history=hist.reshape(1, -1))
        record("penalties_bf16",
               prepared("yskn_smp_sample", d3.h, vp(xb), d3._dtype(xb), 1, synth.V_LARGE, synth.V_LARGE, vp(p3), 1,
                        vp(ids3), C.byref(aux3), sptr),
               synth.V_LARGE * 2 + hist.numel() * 4,
               "1 x 248,320 bf16 + 8,192 history ids, rep 1.05 pres 0.5 freq 0.3, T 0.7 top-p 0.9 min-p 0.05",
               {"kernels_per_call": 2})
    # 4: 64 heterogeneous rows
    if only in (0, 4):
        xs = synth.batched(64, dev)
        pr = synth.batched_params(64)
        d4 = yskn_smp.DeviceSampler(64, synth.V_LARGE, extended_top_k=True)
        d4.set_params([yskn_smp.SamplingParameters(temperature_milli=p["temperature_milli"],
                                                   top_p_milli=p["top_p_milli"], min_p_milli=p["min_p_milli"],
                                                   top_k=p["top_k"], seed=p["seed"]) for p in pr])
        p4 = torch.tensor([p["position"] for p in pr], dtype=torch.int64, device=dev)
        ids4 = torch.empty(64, dtype=torch.int32, device=dev)
        aux4 = yskn_smp.CAux()
        record("batched_heterogeneous_64",
               prepared("yskn_smp_sample", d4.h, vp(xs), d4._dtype(xs), 64, synth.V_LARGE, synth.V_LARGE, vp(p4), 1,
                        vp(ids4), C.byref(aux4), sptr),
               64 * synth.V_LARGE * 4,
               "64 x 248,320 f32, per-row T / top-p / min-p, top-k cycling 1, 20, 50, disabled",
               {"path_stats_after": None})
        res["batched_heterogeneous_64"]["path_stats_after"] = d4.stats()
    return res


def main():
    a = parse()
    if a.only_config:
        import torch

        import yskn_smp
        from yskn_smp import synth

        torch.cuda.set_device(0)
        print(json.dumps(small_configs(torch, yskn_smp, synth, a.only_config, a.steps, a.warmup)))
        return
    if a.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {a.gpus} is not supported "
              "(rows shard across GPUs with no exchange; see DESIGN.md)", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch

    import yskn_smp
    from yskn_smp import synth

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if a.profile_copy:
        src = torch.empty(ALG_BYTES // 4, dtype=torch.float32, device=dev).uniform_()
        dst = torch.empty_like(src)
        for _ in range(a.warmup + a.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"profile_copy_bytes": ALG_BYTES, "launches": a.warmup + a.steps}))
        return

    print(f"generating {ROWS} x {V} logits (2*t3) on the GPU", file=sys.stderr, flush=True)
    x0 = synth.large_batch(ROWS, dev)
    if a.dump_logits:
        x0.cpu().numpy().tofile(a.dump_logits)
        print(json.dumps({"dumped": a.dump_logits, "rows": ROWS, "vocab": V}))
        return
    bufs = [x0, x0.clone(), x0.clone()]
    seeds = synth.large_batch_seeds(ROWS)
    positions = torch.arange(1, ROWS + 1, dtype=torch.int64, device=dev)
    smp = yskn_smp.DeviceSampler(ROWS, V, extended_top_k=True)
    smp.set_params([yskn_smp.SamplingParameters(temperature_milli=1000, top_p_milli=950, top_k=0,
                                                min_p_milli=0, seed=s) for s in seeds])
    # outputs allocated once; the timed loop allocates nothing
    out = smp.sample(bufs[0], positions, n_logprobs=20)
    smp.sync()
    first_ids = out["ids"].cpu().numpy().astype(np.uint32).reshape(-1)

    import ctypes as C

    L = yskn_smp.load_library()
    aux = yskn_smp.CAux()
    aux.n_logprobs = 20
    aux.logprob_ids, aux.logprobs = out["logprob_ids"].data_ptr(), out["logprobs"].data_ptr()
    stream = torch.cuda.current_stream()
    sptr = C.c_void_p(stream.cuda_stream)
    pos_ptr, ids_ptr = positions.data_ptr(), out["ids"].data_ptr()

    # the launch arguments are prepared once: the timed loop is one C call
    # per step, so that the host stays ahead of the device
    fn = L.yskn_smp_sample
    aux_ref = C.byref(aux)
    args = [(smp.h, C.c_void_p(bufs[j].data_ptr()), 0, ROWS, V, V, C.c_void_p(pos_ptr), 1,
             C.c_void_p(ids_ptr), aux_ref, sptr) for j in range(3)]

    def step(i):
        st = fn(*args[i % 3])
        if st != 0:
            raise RuntimeError(L.yskn_smp_last_error().decode())

    print(f"warmup {a.warmup} steps", file=sys.stderr, flush=True)
    for i in range(a.warmup):
        step(i)
    torch.cuda.synchronize()
    # HIP events on the launch stream bracket the timed launches: their
    # interval over the number of launches is the average launch duration
    # (back to back, so it includes the gaps between launches)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    print(f"timing {a.steps} steps", file=sys.stderr, flush=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    for i in range(a.steps):
        step(i)
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    smp.sync()
    stats = smp.stats()
    avg_launch_s = float(ev0.elapsed_time(ev1)) / 1e3 / a.steps
    ms_per_step = wall * 1e3 / a.steps
    rows_per_s = ROWS * a.steps / wall
    achieved = ALG_BYTES / avg_launch_s / 1e9
    # per-launch distribution: an event after every launch (a separate pass,
    # so that the headline interval carries no extra event records)
    per, _ = event_times(torch, stream, step, a.steps)

    cpu = None
    cpu_all = None
    parity = None
    if not a.no_cpu:
        print("CPU oracle sample (1 thread, then every core)", file=sys.stderr, flush=True)
        x_host = x0.cpu().numpy()
        pos_host = positions.cpu().numpy()
        rps, n, cpu_ids = cpu_baseline(x_host, seeds, pos_host, a.cpu_seconds, 1)
        parity = bool(np.array_equal(first_ids[:n], np.array(cpu_ids, np.uint32)))
        model = cpu_model()
        cpu = {"value": rps, "unit": "rows/s", "cores": 1, "kind": "port",
               "sample": f"first {n} of the {ROWS} rows: sample (full sort, serial binary64 tail) "
                         f"+ top-20 logprobs per row, C oracle (-O3), 1 thread on {model}"}
        nt = min(host_threads(), 64)
        rps_all, n_all, ids_all = cpu_baseline(x_host, seeds, pos_host, a.cpu_seconds, nt)
        parity = parity and bool(np.array_equal(first_ids[:n_all], np.array(ids_all, np.uint32)))
        cpu_all = {"value": rps_all, "unit": "rows/s", "cores": nt, "kind": "port",
                   "sample": f"first {n_all} rows, one row per thread, {nt} threads on {model}"}
    configs = None
    if not a.no_configs:
        print("timing the other workloads", file=sys.stderr, flush=True)
        configs = small_configs(torch, yskn_smp, synth)
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "large_batch_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")
    res = {
        "metric": METRIC,
        "value": rows_per_s,
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": ms_per_step,
        "us_per_step": ms_per_step * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "large_batch_top_p: 256 x 248,320 f32 logits (2*t_3), top-k disabled, "
                               "top-p 0.95, T 1.0, Gumbel v3, per-row seeds, top-20 logprobs",
                   "rows": ROWS, "vocab": V},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / PEAK_GBS, "traffic": traffic,
                     "traffic_source": "profiles/large_batch_traffic.json: rocprofv3 --pmc FETCH_SIZE and "
                                       "WRITE_SIZE in separate runs, scaled by a plain copy (not measured "
                                       "in this run)",
                     "kernel_us": avg_launch_s * 1e6,
                     "launch_us_median": pct(per, 50), "launch_us_p10": pct(per, 10),
                     "launch_us_p90": pct(per, 90)},
        "cpu_baseline": cpu,
        "cpu_baseline_all_cores": cpu_all,
        "other_workloads": configs,
        "parity_with_oracle": parity,
        "path_stats": stats,
    }
    print(json.dumps(res))


if __name__ == "__main__":
    main()
