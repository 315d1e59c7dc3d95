"""Benchmark of the stride-aware elementwise + reduction path on one MI355X.

Metric: achieved HBM GB/s, and the fraction of MI355X's 8 TB/s peak, for
f32 add, axis-sum and argmax.  One step = one pass of the hot path over the BASELINE configs
that metric names:
    C1  add      f32, 16,777,216 elements U(-1,1), seed 0            12 B/elem
    C4  sum      axis=-1 of an (8192, 8192) f32 N(0,1) array, seed 0   4 B/elem + 4 B/row
    C4  argmax   axis=1 of the same array -> int64                    4 B/elem + 8 B/row
Inputs are resident in HBM before timing.  Each op is launched K times back-to-back between two
HIP events on the stream it runs on, with outputs preallocated (out=) and the inputs rotated
over 4 device copies, so every launch streams its inputs from HBM rather than from the 256 MB
Infinity Cache.  `value` = algorithmic bytes of the step / summed average launch time.  `cpu_baseline` times the CPU oracle (single-threaded C restatement of
musapy's CPU path) on the same step.

    python bench.py [--steps K] [--warmup W] [--all] [--no-cpu] [--only add|sum|argmax|copy]
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

import numpy as np

PEAK_GBS = 8000.0  # MI355X HBM3E


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--all", action="store_true", help="also time every BASELINE config (table on stderr)")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--only", choices=["add", "sum", "argmax", "copy"],
                   help="launch one step op (or the calibration copy) warmup+steps times and exit; "
                        "the program run under rocprofv3 --pmc for the HBM traffic figures")
    return p.parse_args()


TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "hbm_traffic_step_kernels.md")


def measured_traffic():
    """HBM bytes per launch of each step kernel, from the committed rocprofv3 --pmc summary:
    FETCH_SIZE and WRITE_SIZE (KiB per dispatch, one pass each) scaled by what the same counters
    read for a plain copy of known size.  Rows look like `| key | kernel | ... | bytes |`."""
    out = {}
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                m = re.match(r"\|\s*(add|sum|argmax)\s*\|.*\|\s*([0-9]+)\s*\|\s*$", line)
                if m:
                    out[m.group(1)] = int(m.group(2))
    except OSError:
        pass
    return out


COPIES = 4  # input copies rotated between launches (4 x the working set >> the 256 MB MALL)


class Timer:
    """HIP events on device 0's stream (the stream every op below is launched on)."""

    def __init__(self, ms):
        self.ms = ms
        self.t = ms._core._Timer(0)

    def run(self, launches):
        """Launches back-to-back between two events; returns the average launch time (ms).
        `host_ms` keeps the host time per launch of the same loop (the time to enqueue it)."""
        self.t.start()
        h0 = time.perf_counter()
        for f in launches:
            f()
        self.host_ms = (time.perf_counter() - h0) * 1e3 / len(launches)
        self.t.stop()
        return self.t.elapsed_ms() / len(launches)


def _copies(ms, host, n=COPIES):
    return [ms.from_numpy(host) for _ in range(n)]


def step_ops(ms):
    """The three ops of one step, each as a function of the launch index (inputs rotate)."""
    rng = np.random.default_rng(0)
    a = rng.uniform(-1, 1, 16_777_216).astype(np.float32)
    b = rng.uniform(-1, 1, 16_777_216).astype(np.float32)
    x = np.random.default_rng(0).standard_normal((8192, 8192), dtype=np.float32)
    A, B, X = _copies(ms, a), _copies(ms, b), _copies(ms, x)
    C = ms.from_numpy(np.zeros_like(a))
    S = ms.from_numpy(np.zeros(8192, np.float32))
    I = ms.from_numpy(np.zeros(8192, np.int64))
    n = 8192 * 8192
    ops = [
        ("add", "C1 add f32 16,777,216", lambda i: ms.add(A[i % COPIES], B[i % COPIES], out=C), 12 * 16_777_216),
        ("sum", "C4 sum axis=-1 (8192,8192) f32", lambda i: ms.sum(X[i % COPIES], axis=-1, out=S),
         4 * n + 4 * 8192),
        ("argmax", "C4 argmax axis=1 (8192,8192) f32", lambda i: ms.argmax(X[i % COPIES], axis=1, out=I),
         4 * n + 8 * 8192),
    ]
    # calibration: a plain copy of a unit-stride view starting 4 KiB in (page- and line-aligned,
    # so no cache line is shared between workgroups): one vectorised copy kernel
    m = 16_777_216 - 1024
    ops.append(("copy", "calibration copy f32 16,776,192",
                lambda i: ms.contiguous(ms.slice(A[i % COPIES], [(1024, 16_777_216, 1)])), 8 * m))
    host = {"a": a, "b": b, "x": x}
    return ops, host


def all_config_ops(ms, host_legs=False):
    """Every BASELINE config op (for the per-config table); inputs rotate over 3 copies.

    Rows are (name, gpu launch of launch index i, algorithmic bytes, cpu leg).  With `host_legs`
    the BASELINE config rows carry a cpu leg: a function that runs the CPU oracle (the
    single-threaded C restatement of musapy's CPU path) once on the same host inputs and returns
    the algorithmic bytes it covered.  The widened rows carry none."""
    K = 3
    R = None
    if host_legs:
        sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
        from oracle import reference as R

    def leg(f, nbytes):
        return (lambda: (f(), nbytes)[1]) if R is not None else None

    rng = np.random.default_rng(0)
    ops = []
    a64 = rng.uniform(-1, 1, 67_108_864).astype(np.float32)
    b64 = rng.uniform(-1, 1, 67_108_864).astype(np.float32)
    A64, B64 = _copies(ms, a64, K), _copies(ms, b64, K)
    ops.append(("C1-64M add f32 67,108,864", lambda i: ms.add(A64[i % K], B64[i % K]), 12 * 67_108_864,
                leg(lambda: R.binary("add", a64, b64), 12 * 67_108_864)))
    ops.append(("full sum f32 64M", lambda i: ms.sum(A64[i % K]), 4 * 67_108_864 + 4,
                leg(lambda: R.reduce(a64, "sum"), 4 * 67_108_864 + 4)))
    ops.append(("full argmax f32 64M", lambda i: ms.argmax(A64[i % K]), 4 * 67_108_864 + 8,
                leg(lambda: R.reduce(a64, "argmax"), 4 * 67_108_864 + 8)))
    # the same whole-array reductions at 4x the size: the fixed end-of-launch hand-over amortised
    a256 = np.random.default_rng(1).uniform(-1, 1, 268_435_456).astype(np.float32)
    A256 = _copies(ms, a256, K)
    ops.append(("full sum f32 256M", lambda i: ms.sum(A256[i % K]), 4 * 268_435_456 + 4,
                leg(lambda: R.reduce(a256, "sum"), 4 * 268_435_456 + 4)))
    ops.append(("full argmax f32 256M", lambda i: ms.argmax(A256[i % K]), 4 * 268_435_456 + 8,
                leg(lambda: R.reduce(a256, "argmax"), 4 * 268_435_456 + 8)))
    r = np.random.default_rng(0)
    ca, cb = r.uniform(-1, 1, (4096, 1)).astype(np.float32), r.uniform(-1, 1, (8192,)).astype(np.float32)
    CA, CB = _copies(ms, ca, K), _copies(ms, cb, K)
    nb = 4 * 33_554_432 + 4 * 4096 + 4 * 8192
    ops.append(("C2 broadcast add (4096,1)+(8192,)", lambda i: ms.add(CA[i % K], CB[i % K]), nb,
                leg(lambda: R.binary("add", ca, cb), nb)))
    xh = np.random.default_rng(0).uniform(-4, 4, (8192, 4096)).astype(np.float32)
    xt = [ms.transpose(c) for c in _copies(ms, xh, K)]
    ops.append(("C2 exp transposed (8192,4096)^T", lambda i: ms.exp(xt[i % K]), 8 * 33_554_432,
                leg(lambda: R.unary("exp", xh.T), 8 * 33_554_432)))
    r = np.random.default_rng(0)
    i64h = r.integers(-1000, 1001, (2048, 2048, 4), dtype=np.int64)
    f64h = r.standard_normal((2048, 2048, 4))
    i64, f64 = _copies(ms, i64h, K), _copies(ms, f64h, K)
    N = 16_777_216
    sh = i64h.astype(np.float64) + f64h  # the host inputs of the later C3 steps (values only feed timing)
    ch = np.clip(sh, -1.0, 1.0)
    fh = ch.astype(np.float32)
    ops.append(("C3 add i64+f64->f64 (cast+add)", lambda i: ms.add(i64[i % K], f64[i % K]), 24 * N,
                leg(lambda: R.binary("add", i64h, f64h), 24 * N)))
    s = [ms.add(i64[k], f64[k]) for k in range(K)]
    ops.append(("C3 clamp f64", lambda i: ms.clamp(s[i % K], -1.0, 1.0), 16 * N,
                leg(lambda: R.clamp(sh, -1.0, 1.0), 16 * N)))
    c = [ms.clamp(s[k], -1.0, 1.0) for k in range(K)]
    ops.append(("C3 astype f64->f32", lambda i: ms.astype(c[i % K], "f32"), 12 * N,
                leg(lambda: R.cast(ch, "f32"), 12 * N)))
    f = [ms.astype(c[k], "f32") for k in range(K)]
    ops.append(("C3 astype f32->bf16", lambda i: ms.astype(f[i % K], "bf16"), 6 * N,
                leg(lambda: R.cast(fh, "bf16"), 6 * N)))
    ops.append(("C3 astype f32->f16", lambda i: ms.astype(f[i % K], "f16"), 6 * N,
                leg(lambda: R.cast(fh, "f16"), 6 * N)))
    Xh = np.random.default_rng(0).standard_normal((8192, 8192), dtype=np.float32)
    X = _copies(ms, Xh, K)
    n = 8192 * 8192
    ops.append(("C4 sum axis=0", lambda i: ms.sum(X[i % K], axis=0), 4 * n + 4 * 8192,
                leg(lambda: R.reduce(Xh, "sum", 0), 4 * n + 4 * 8192)))
    ops.append(("C4 mean axis=-1", lambda i: ms.mean(X[i % K], axis=-1), 4 * n + 4 * 8192,
                leg(lambda: R.reduce(Xh, "mean", -1), 4 * n + 4 * 8192)))
    ops.append(("C4 mean axis=0", lambda i: ms.mean(X[i % K], axis=0), 4 * n + 4 * 8192,
                leg(lambda: R.reduce(Xh, "mean", 0), 4 * n + 4 * 8192)))
    ops.append(("C4 max axis=(0,1)", lambda i: ms.max(X[i % K], axis=(0, 1)), 4 * n + 4,
                leg(lambda: R.reduce(Xh, "max", (0, 1)), 4 * n + 4)))
    ops.append(("C4 argmin axis=1", lambda i: ms.argmin(X[i % K], axis=1), 4 * n + 8 * 8192,
                leg(lambda: R.reduce(Xh, "argmin", 1), 4 * n + 8 * 8192)))
    yh = np.random.default_rng(0).random((1024, 65536))
    y = _copies(ms, yh, K)
    ops.append(("C5 cumsum f64 (1024,65536) axis=1", lambda i: ms.cumsum(y[i % K], axis=1), 16 * 1024 * 65536,
                leg(lambda: R.cumsum(yh, axis=1), 16 * 1024 * 65536)))
    if R is not None:
        # musapy's literal CPU cumsum re-sums the prefix for every output (O(L^2) per row); rows
        # are independent and cost the same, so one row's rate is the whole array's
        ops.append(("C5 cumsum f64, literal O(L^2) CPU form (1 of 1024 rows)", None, 16 * 65536,
                    leg(lambda: R.cumsum(yh[:1], axis=1, literal=True), 16 * 65536)))
    r = np.random.default_rng(0)
    z = (r.standard_normal((16, 1024, 1024), dtype=np.float32)
         + 1j * r.standard_normal((16, 1024, 1024), dtype=np.float32)).astype(np.complex64)
    Z = _copies(ms, z, K)
    ops.append(("C5 c64 sum axis=(1,2)", lambda i: ms.sum(Z[i % K], axis=(1, 2)), 8 * 16 * 1024 * 1024 + 128,
                leg(lambda: R.reduce(z, "sum", (1, 2)), 8 * 16 * 1024 * 1024 + 128)))
    # widened rows: comparisons (1-byte bool output) and complex elementwise
    M = 16 * 1024 * 1024
    ops.append(("cmp lt f32 64M -> bool", lambda i: ms.lt(A64[i % K], B64[i % K]), 9 * 67_108_864, None))
    ops.append(("cmp eq f64 16M -> bool", lambda i: ms.eq(s[i % K], c[i % K]), 17 * N, None))
    Z2 = [ms.neg(Z[(k + 1) % K]) for k in range(K)]
    ops.append(("cmp eq c64 16M -> bool", lambda i: ms.eq(Z[i % K], Z2[i % K]), 17 * M, None))
    ops.append(("c64 mul 16M", lambda i: ms.mul(Z[i % K], Z2[i % K]), 24 * M, None))
    ops.append(("c64 div 16M", lambda i: ms.div(Z[i % K], Z2[i % K]), 24 * M, None))
    ops.append(("c64 abs 16M -> f32", lambda i: ms.abs(Z[i % K]), 12 * M, None))
    ops.append(("astype f32->c64 64M", lambda i: ms.astype(A64[i % K], "c64"), 12 * 67_108_864, None))
    W = [ms.astype(Z[k], "c128") for k in range(K)]
    W2 = [ms.astype(Z2[k], "c128") for k in range(K)]
    ops.append(("c128 mul 16M", lambda i: ms.mul(W[i % K], W2[i % K]), 48 * M, None))
    ops.append(("c128 div 16M", lambda i: ms.div(W[i % K], W2[i % K]), 48 * M, None))
    # contiguous() materialisation: 2-D transpose (transpose2d entry point), 3-D permute, flip
    ops.append(("contiguous X^T f32 (8192,8192)", lambda i: ms.contiguous(ms.transpose(X[i % K])), 8 * n, None))
    P = _copies(ms, np.random.default_rng(1).standard_normal((8192, 128, 64), dtype=np.float32), K)
    ops.append(("contiguous permute(2,0,1) f32 (8192,128,64)",
                lambda i: ms.contiguous(ms.permute(P[i % K], [2, 0, 1])), 8 * n, None))
    ops.append(("contiguous flip axis=1 f32 (8192,8192)", lambda i: ms.contiguous(ms.flip(X[i % K], 1)), 8 * n,
                None))
    wm = (r.standard_normal((4096, 4096)) + 1j * r.standard_normal((4096, 4096))).astype(np.complex128)
    WM = _copies(ms, wm, K)
    ops.append(("contiguous ^T c128 (4096,4096)", lambda i: ms.contiguous(ms.transpose(WM[i % K])),
                32 * 4096 * 4096, None))
    return ops


def interop_costs(ms):
    """DLPack exchange: host time of a zero-copy export + import of a device array (no device
    work), and the rate of importing a host (NumPy) tensor, which is a PCIe copy."""
    a = ms.from_numpy(np.zeros((4096, 4096), np.float32))
    v = ms.transpose(a)
    for _ in range(100):
        ms.from_dlpack(v)
    n = 2000
    t0 = time.perf_counter()
    for _ in range(n):
        ms.from_dlpack(v)
    us = (time.perf_counter() - t0) * 1e6 / n
    h = np.random.default_rng(0).standard_normal((8192, 8192), dtype=np.float32)
    ms.from_dlpack(h)
    ms.synchronize()
    t0 = time.perf_counter()
    for _ in range(3):
        ms.from_dlpack(h)
    ms.synchronize()
    gbs = 3 * h.nbytes / (time.perf_counter() - t0) / 1e9
    return {"dlpack_roundtrip_us": round(us, 2), "host_import_GBps_pcie": round(gbs, 2)}


def host_cpu():
    """The host the CPU baseline ran on: CPU model and logical CPU count (one thread is used)."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "nproc": os.cpu_count(), "threads_used": 1}


def cpu_baseline(host):
    """The CPU oracle (single thread) on the same step; returns (GB/s, seconds, sample)."""
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import reference as R

    n = 8192 * 8192
    algo = 12 * 16_777_216 + (4 * n + 4 * 8192) + (4 * n + 8 * 8192)
    reps = 0
    t0 = time.perf_counter()
    while True:
        R.binary("add", host["a"], host["b"])
        R.reduce(host["x"], "sum", -1)
        R.reduce(host["x"], "argmax", 1)
        reps += 1
        el = time.perf_counter() - t0
        if el > 8.0 or reps >= 10:
            break
    return algo * reps / el / 1e9, el / reps, f"the full step (C1 add 16M + C4 sum axis=-1 + C4 argmax axis=1), {reps} passes"


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}): this build runs on single-GPU "
              f"boxes. Elementwise ops and axis reductions shard over the non-reduced dims with no exchange; a "
              f"whole-array reduction adds one exchange of a scalar per GPU.", file=sys.stderr)
        sys.exit(2)
    import musapy_amd as ms

    timer = Timer(ms)
    ops, host = step_ops(ms)
    if args.only:
        key, name, fn, bytes_ = next(o for o in ops if o[0] == args.only)
        for i in range(args.warmup + args.steps):
            fn(i)
        ms.synchronize()
        print(json.dumps({"only": key, "op": name, "launches": args.warmup + args.steps, "algo_bytes": bytes_}),
              flush=True)
        return
    ops = [o for o in ops if o[0] != "copy"]
    for _, name, fn, _ in ops:  # warm-up (first launches load code objects, fill the memory pool)
        for i in range(max(args.warmup, 1)):
            fn(i)
    ms.synchronize()
    per_op = {}
    t0 = time.perf_counter()
    ms.synchronize()
    # K steps: each op is launched K times back-to-back between two events (inputs rotate over
    # COPIES device copies, so every launch streams from HBM)
    for _, name, fn, _ in ops:
        per_op[name] = timer.run([(lambda i=i, fn=fn: fn(i)) for i in range(args.steps)])
    ms.synchronize()
    wall = time.perf_counter() - t0
    table = {}
    keys = {}
    total_bytes, total_ms = 0, 0.0
    for key, name, fn, bytes_ in ops:
        t = float(per_op[name])
        table[name] = {"ms": round(t, 5), "algo_bytes": bytes_, "GBps": round(bytes_ / t / 1e6, 1),
                       "frac_peak": round(bytes_ / t / 1e6 / PEAK_GBS, 4)}
        keys[name] = key
        total_bytes += bytes_
        total_ms += t
    dom = max(table, key=lambda k: table[k]["ms"])
    traffic = measured_traffic().get(keys[dom])
    value = total_bytes / total_ms / 1e6
    line = {
        "metric": "achieved HBM GB/s (and % of MI355X peak) for f32 add, axis-sum, argmax",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(total_ms, 5),
        "wall_ms_per_step": round(wall * 1e3 / args.steps, 3),
        "timing": f"HIP events around {args.steps} back-to-back launches per op, inputs rotated over {COPIES} copies",
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (numpy default_rng seed 0, BASELINE.json C1/C4 distributions)",
        "config": {"workload": "C1 add f32 16,777,216 + C4 sum axis=-1 + C4 argmax axis=1 on (8192,8192) f32",
                   "parallelism": "single GPU"},
        "frac_of_peak": round(value / PEAK_GBS, 4),
        "ops": table,
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": table[dom]["GBps"], "peak": PEAK_GBS,
                     "unit": "GB/s", "frac": table[dom]["frac_peak"], "traffic": traffic,
                     "algo_bytes": table[dom]["algo_bytes"],
                     "traffic_source": os.path.relpath(TRAFFIC_FILE, os.path.dirname(os.path.abspath(__file__)))
                     if traffic is not None else None},
    }
    if not args.no_cpu:
        v, sec, sample = cpu_baseline(host)
        line["cpu_baseline"] = {"value": round(v, 3), "unit": "GB/s", "cores": 1, "kind": "port",
                                "sample": sample, "seconds_per_pass": round(sec, 3), "host": host_cpu()}
    if args.all:
        rows = []
        for name, fn, bytes_, cpu in all_config_ops(ms, host_legs=not args.no_cpu):
            row = {"op": name}
            if fn is not None:
                fn(0)
                ms.synchronize()
                t = timer.run([(lambda i=i, fn=fn: fn(i)) for i in range(20)])
                row.update({"ms": round(t, 5), "GBps": round(bytes_ / t / 1e6, 1),
                            "frac_peak": round(bytes_ / t / 1e6 / PEAK_GBS, 4), "host_ms": round(timer.host_ms, 5)})
            if cpu is not None:  # the CPU oracle once on the same host inputs, one thread
                t0 = time.perf_counter()
                covered = cpu()
                row["cpu_GBps"] = round(covered / (time.perf_counter() - t0) / 1e9, 3)
            rows.append(row)
            print(json.dumps(row), file=sys.stderr, flush=True)
        line["all_configs"] = rows
        line["interop"] = interop_costs(ms)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
