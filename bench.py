"""Benchmark of the per-step sampling path on one MI355X.

Workload (the large-batch full-vocabulary top-p configuration): 256 rows x
248,320 binary32 logits of 2*t_3 (Student-t, nu = 3), top-k disabled, top-p
0.95, temperature 1.0, Gumbel draw (version 3), per-row seeds, top-20 logprobs
per row. A step is one yskn_smp_sample call over the 256 rows, inputs resident
in HBM; three input buffers rotate so that the 256 MB Infinity Cache does not
serve a step from the previous one.

Prints one JSON line: rows/s (value), us per step, the dominant kernel's
achieved HBM bandwidth against the MI355X peak (8 TB/s) from HIP events on the
launch stream, and the CPU oracle's rows/s on a bounded sample of the same rows
(the reference algorithm restated in C: full sort, serial binary64 tail).
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
    ap.add_argument("--profile-copy", action="store_true",
                    help="run a plain device copy of the workload's size (counter calibration)")
    ap.add_argument("--dump-logits", metavar="PATH",
                    help="write the workload's logits (rows x V binary32, row-major) to PATH and exit; "
                         "lib/smp_bench --logits PATH replays them without Python")
    return ap.parse_args()


def cpu_baseline(x_host, seeds, positions, budget_s):
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import yskn_oracle as O

    done, ids = 0, []
    t0 = time.perf_counter()
    while done < x_host.shape[0]:
        p = O.params_from_thousandths(1000, 950, 0, top_k=0, seed=seeds[done], extension=True)
        ids.append(O.sample(x_host[done], int(positions[done]), p))
        O.top_logprobs(x_host[done], 20)
        done += 1
        if time.perf_counter() - t0 > budget_s and done >= 4:
            break
    dt = time.perf_counter() - t0
    return done / dt, done, ids


def main():
    a = parse()
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

    cpu = None
    parity = None
    if not a.no_cpu:
        print("CPU oracle sample", file=sys.stderr, flush=True)
        x_host = x0.cpu().numpy()
        rps, n, cpu_ids = cpu_baseline(x_host, seeds, positions.cpu().numpy(), a.cpu_seconds)
        parity = bool(np.array_equal(first_ids[:n], np.array(cpu_ids, np.uint32)))
        cpu = {"value": rps, "unit": "rows/s", "cores": 1, "kind": "port",
               "sample": f"first {n} of the {ROWS} rows: sample (full sort, serial binary64 tail) "
                         f"+ top-20 logprobs per row, C oracle, 1 thread"}
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
                     "kernel_us": avg_launch_s * 1e6},
        "cpu_baseline": cpu,
        "parity_with_oracle": parity,
        "path_stats": stats,
    }
    print(json.dumps(res))


if __name__ == "__main__":
    main()
