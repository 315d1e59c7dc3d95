"""Benchmark of the stride-aware elementwise + reduction path on one MI355X.

Metric: achieved HBM GB/s, and the fraction of MI355X's 8 TB/s peak, for
f32 add, axis-sum and argmax.  One step = one pass of the hot path over the BASELINE configs
that metric names:
    C1  add      f32, 16,777,216 elements U(-1,1), seed 0            12 B/elem
    C4  sum      axis=-1 of an (8192, 8192) f32 N(0,1) array, seed 0   4 B/elem + 4 B/row
    C4  argmax   axis=1 of the same array -> int64                    4 B/elem + 8 B/row
Inputs are resident in HBM before timing.  Each op is launched K times back-to-back between two
HIP events on the stream it runs on, with outputs preallocated (out=) and inputs and outputs
rotated over 4 device buffers, so every launch streams from HBM rather than from the 256 MB
Infinity Cache.  `value` = algorithmic bytes of the step / summed average launch time.
`mall_flushed` repeats the step with each launch timed alone after 768 MB of other traffic.  `cpu_baseline` times the CPU oracle (single-threaded C restatement of
musapy's CPU path) on the same step.

    python bench.py [--steps K] [--warmup W] [--all] [--no-cpu] [--only KEY]
"""
from __future__ import annotations

import argparse
import gc
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
    p.add_argument("--keys", metavar="K1,K2", help="with --all: time only these config keys")
    p.add_argument("--only", metavar="KEY",
                   help="launch one op warmup+steps times and exit (a step op: add, sum, argmax; the "
                        "calibration copy: copy; or a config key of --all, e.g. cumsum, max01): the "
                        "program run under rocprofv3 --pmc for the HBM traffic figures")
    return p.parse_args()


TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "hbm_traffic_step_kernels.md")


STEP_TRACE_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "kernel_trace_bench_step.md")


def profiled_kernel_us(key):
    """Average kernel duration (us) of step op `key` in the committed rocprofv3 kernel trace of the
    default bench (profiles/kernel_trace_bench_step.md), found through the kernel name the
    traffic summary gives for that key; None when either file lacks it."""
    name = None
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                m = re.match(r"\|\s*(add|sum|argmax)\s*\|\s*`([^`]+)`", line)
                if m and m.group(1) == key:
                    name = m.group(2)
        if name is None:
            return None
        with open(STEP_TRACE_FILE) as f:
            for line in f:
                cells = [c.strip() for c in line.strip().strip("|").split("|")]
                if len(cells) >= 4 and cells[0] == f"`{name}`":
                    return float(cells[3])  # the first row of that kernel: the step's grid
    except (OSError, ValueError):
        return None
    return None


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
ROTATED_BYTES = 512 << 20  # per --all row: at least this many bytes of inputs over the rotated copies


class Timer:
    """HIP events on device 0's stream (the stream every op below is launched on)."""

    def __init__(self, ms):
        self.ms = ms
        self.t = ms._core._Timer(0)

    def run(self, launches):
        """Launches back-to-back between two events; returns the average launch time (ms).
        `host_ms` keeps the host time per launch of the same loop (the time to enqueue it)."""
        gc.disable()  # a collection inside the loop would stall the launches and idle the GPU
        try:
            self.t.start()
            h0 = time.perf_counter()
            for f in launches:
                f()
            self.host_ms = (time.perf_counter() - h0) * 1e3 / len(launches)
            self.t.stop()
        finally:
            gc.enable()
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
    # outputs rotate over as many buffers as the inputs, so no launch writes the lines the previous
    # one left in the Infinity Cache
    C = [ms.from_numpy(np.zeros_like(a)) for _ in range(COPIES)]
    S = [ms.from_numpy(np.zeros(8192, np.float32)) for _ in range(COPIES)]
    I = [ms.from_numpy(np.zeros(8192, np.int64)) for _ in range(COPIES)]
    n = 8192 * 8192
    ops = [
        ("add", "C1 add f32 16,777,216", lambda i: ms.add(A[i % COPIES], B[i % COPIES], out=C[i % COPIES]),
         12 * 16_777_216),
        ("sum", "C4 sum axis=-1 (8192,8192) f32", lambda i: ms.sum(X[i % COPIES], axis=-1, out=S[i % COPIES]),
         4 * n + 4 * 8192),
        ("argmax", "C4 argmax axis=1 (8192,8192) f32",
         lambda i: ms.argmax(X[i % COPIES], axis=1, out=I[i % COPIES]), 4 * n + 8 * 8192),
    ]
    # calibration: a plain copy of a unit-stride view starting 4 KiB in (page- and line-aligned,
    # so no cache line is shared between workgroups): one vectorised copy kernel
    m = 16_777_216 - 1024
    ops.append(("copy", "calibration copy f32 16,776,192",
                lambda i: ms.contiguous(ms.slice(A[i % COPIES], [(1024, 16_777_216, 1)])), 8 * m))
    host = {"a": a, "b": b, "x": x}
    return ops, host


def all_config_ops(ms, host_legs=False):
    """Every BASELINE config op (for the per-config table), built one at a time.

    Rows are (key, name, build).  build() uploads that op's inputs and returns (gpu launch of
    launch index i, algorithmic bytes, cpu leg).  Each row rotates over K copies of its inputs and
    keeps its last K outputs alive, with K = max(4, what makes the rotated inputs at least 512 MB),
    so consecutive launches read and write lines the 256 MB Infinity Cache does not hold.  With
    `host_legs` the BASELINE config rows carry a cpu leg: a function that runs the CPU oracle (the
    single-threaded C restatement of musapy's CPU path) once on the same host inputs and returns
    the algorithmic bytes it covered.  The widened rows carry none.  `key` names the op for
    `--only` (the program profiled under rocprofv3 --pmc)."""
    R = None
    if host_legs:
        sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
        from oracle import reference as R

    def leg(f, nbytes):
        return (lambda: (f(), nbytes)[1]) if R is not None else None

    N = 16_777_216
    M = 16 * 1024 * 1024
    n = 8192 * 8192
    cache = {}

    def get(name, make):
        if name not in cache:
            cache[name] = make()
        return cache[name]

    def ncopies(*hosts):
        """Copies to rotate: at least 4, and at least 512 MB of inputs over all copies."""
        per = sum(h.nbytes for h in hosts)
        return max(4, -(-ROTATED_BYTES // per))

    def a64():
        return get("a64", lambda: np.random.default_rng(0).uniform(-1, 1, 67_108_864).astype(np.float32))

    def b64():
        def mk():
            r = np.random.default_rng(0)
            r.uniform(-1, 1, 67_108_864)
            return r.uniform(-1, 1, 67_108_864).astype(np.float32)
        return get("b64", mk)

    def a256():
        return get("a256", lambda: np.random.default_rng(1).uniform(-1, 1, 268_435_456).astype(np.float32))

    def c2():
        def mk():
            r = np.random.default_rng(0)
            return r.uniform(-1, 1, (4096, 1)).astype(np.float32), r.uniform(-1, 1, (8192,)).astype(np.float32)
        return get("c2", mk)

    def c3():
        def mk():
            r = np.random.default_rng(0)
            i64h = r.integers(-1000, 1001, (2048, 2048, 4), dtype=np.int64)
            f64h = r.standard_normal((2048, 2048, 4))
            sh = i64h.astype(np.float64) + f64h  # host inputs of the later C3 steps (values only feed timing)
            ch = np.clip(sh, -1.0, 1.0)
            return i64h, f64h, sh, ch, ch.astype(np.float32)
        return get("c3", mk)

    def xh():
        return get("x", lambda: np.random.default_rng(0).standard_normal((8192, 8192), dtype=np.float32))

    def zh():
        def mk():
            r = np.random.default_rng(0)
            return (r.standard_normal((16, 1024, 1024), dtype=np.float32)
                    + 1j * r.standard_normal((16, 1024, 1024), dtype=np.float32)).astype(np.complex64)
        return get("z", mk)

    def up(h, k):
        return _copies(ms, h, k)

    def row(fn, nbytes, cpu=None, k=COPIES):
        if fn is None:
            return None, nbytes, cpu
        # keep the last k results alive, so consecutive launches write k + 1 different output
        # blocks instead of the one the memory pool would hand back (whose lines the Infinity
        # Cache still holds)
        ring = [None] * k

        def g(i):
            ring[i % k] = fn(i)
        g.ring = k
        return g, nbytes, cpu

    def b_add64():
        k = ncopies(a64(), b64())
        A, B = up(a64(), k), up(b64(), k)
        return row(lambda i: ms.add(A[i % k], B[i % k]), 12 * 67_108_864,
                   leg(lambda: R.binary("add", a64(), b64()), 12 * 67_108_864), k)

    def b_sum64():
        k = ncopies(a64())
        A = up(a64(), k)
        return row(lambda i: ms.sum(A[i % k]), 4 * 67_108_864 + 4, leg(lambda: R.reduce(a64(), "sum"), 4 * 67_108_864 + 4),
                   k)

    def b_argmax64():
        k = ncopies(a64())
        A = up(a64(), k)
        return row(lambda i: ms.argmax(A[i % k]), 4 * 67_108_864 + 8,
                   leg(lambda: R.reduce(a64(), "argmax"), 4 * 67_108_864 + 8), k)

    def b_sum256():
        k = ncopies(a256())
        A = up(a256(), k)
        return row(lambda i: ms.sum(A[i % k]), 4 * 268_435_456 + 4,
                   leg(lambda: R.reduce(a256(), "sum"), 4 * 268_435_456 + 4), k)

    def b_argmax256():
        k = ncopies(a256())
        A = up(a256(), k)
        return row(lambda i: ms.argmax(A[i % k]), 4 * 268_435_456 + 8,
                   leg(lambda: R.reduce(a256(), "argmax"), 4 * 268_435_456 + 8), k)

    def b_bcast():
        ca, cb = c2()
        # the broadcast operands are small (48 KB); what streams is the 128 MB output, which the
        # ring below rotates over k buffers
        k = ncopies(np.empty(33_554_432, np.float32))
        CA, CB = up(ca, k), up(cb, k)
        nb = 4 * 33_554_432 + 4 * 4096 + 4 * 8192
        return row(lambda i: ms.add(CA[i % k], CB[i % k]), nb, leg(lambda: R.binary("add", ca, cb), nb), k)

    def b_expT():
        h = get("xe", lambda: np.random.default_rng(0).uniform(-4, 4, (8192, 4096)).astype(np.float32))
        k = ncopies(h)
        xt = [ms.transpose(c) for c in up(h, k)]
        return row(lambda i: ms.exp(xt[i % k]), 8 * 33_554_432, leg(lambda: R.unary("exp", h.T), 8 * 33_554_432), k)

    def b_xTc2():
        # the copy of C2's transposed view (what exp adds to it: b_expT against this row)
        h = get("xe", lambda: np.random.default_rng(0).uniform(-4, 4, (8192, 4096)).astype(np.float32))
        k = ncopies(h)
        xt = [ms.transpose(c) for c in up(h, k)]
        return row(lambda i: ms.contiguous(xt[i % k]), 8 * 33_554_432, k=k)

    def b_exp32():
        # exp of a contiguous array of C2's size (the transcendental's cost without the transpose)
        h = get("xe", lambda: np.random.default_rng(0).uniform(-4, 4, (8192, 4096)).astype(np.float32))
        k = ncopies(h)
        X = up(h, k)
        return row(lambda i: ms.exp(X[i % k]), 8 * 33_554_432, k=k)

    def b_c3add():
        i64h, f64h, _, _, _ = c3()
        k = ncopies(i64h, f64h)
        I, F = up(i64h, k), up(f64h, k)
        return row(lambda i: ms.add(I[i % k], F[i % k]), 24 * N, leg(lambda: R.binary("add", i64h, f64h), 24 * N), k)

    def c3_dev(stage, k):
        i64h, f64h, _, _, _ = c3()
        s_ = []
        for j in range(k):  # one upload at a time: k copies of the stage, not of every input
            s_.append(ms.add(ms.from_numpy(i64h), ms.from_numpy(f64h)))
        if stage == "s":
            return s_
        c_ = [ms.clamp(x, -1.0, 1.0) for x in s_]
        del s_
        if stage == "c":
            return c_
        return [ms.astype(x, "f32") for x in c_]

    def b_clamp():
        sh = c3()[2]
        k = ncopies(sh)
        s_ = c3_dev("s", k)
        return row(lambda i: ms.clamp(s_[i % k], -1.0, 1.0), 16 * N, leg(lambda: R.clamp(sh, -1.0, 1.0), 16 * N), k)

    def b_f64f32():
        ch = c3()[3]
        k = ncopies(ch)
        c_ = c3_dev("c", k)
        return row(lambda i: ms.astype(c_[i % k], "f32"), 12 * N, leg(lambda: R.cast(ch, "f32"), 12 * N), k)

    def b_bf16():
        fh = c3()[4]
        k = ncopies(fh)
        f_ = c3_dev("f", k)
        return row(lambda i: ms.astype(f_[i % k], "bf16"), 6 * N, leg(lambda: R.cast(fh, "bf16"), 6 * N), k)

    def b_f16():
        fh = c3()[4]
        k = ncopies(fh)
        f_ = c3_dev("f", k)
        return row(lambda i: ms.astype(f_[i % k], "f16"), 6 * N, leg(lambda: R.cast(fh, "f16"), 6 * N), k)

    def b_c4(kind, axis, nbytes):
        def b():
            k = ncopies(xh())
            X = up(xh(), k)
            return row(lambda i: getattr(ms, kind)(X[i % k], axis=axis), nbytes,
                       leg(lambda: R.reduce(xh(), kind, axis), nbytes), k)
        return b

    def b_cumsum():
        yh = get("y", lambda: np.random.default_rng(0).random((1024, 65536)))
        k = ncopies(yh)
        Y = up(yh, k)
        return row(lambda i: ms.cumsum(Y[i % k], axis=1), 16 * 1024 * 65536,
                   leg(lambda: R.cumsum(yh, axis=1), 16 * 1024 * 65536), k)

    def b_cumsum_literal():
        # musapy's literal CPU cumsum re-sums the prefix for every output (O(L^2) per row); rows
        # are independent and cost the same, so one row's rate is the whole array's
        yh = get("y", lambda: np.random.default_rng(0).random((1024, 65536)))
        return row(None, 16 * 65536, leg(lambda: R.cumsum(yh[:1], axis=1, literal=True), 16 * 65536))

    def b_copy64():
        # C5's bytes (512 MB in, 512 MB out) as a plain copy: the rate a read-once, write-once f64
        # stream reaches, beside the chained scan (a unit-stride view 1024 elements in, so that
        # contiguous() copies)
        m = 1024 * 65536
        h = get("y", lambda: np.random.default_rng(0).random((1024, 65536))).reshape(-1)
        h = np.concatenate([np.zeros(1024), h])
        k = ncopies(h)
        Y = up(h, k)
        return row(lambda i: ms.contiguous(ms.slice(Y[i % k], [(1024, 1024 + m, 1)])), 16 * m, k=k)

    def b_csum():
        k = ncopies(zh())
        Z = up(zh(), k)
        nb = 8 * 16 * 1024 * 1024 + 128
        return row(lambda i: ms.sum(Z[i % k], axis=(1, 2)), nb, leg(lambda: R.reduce(zh(), "sum", (1, 2)), nb), k)

    def b_lt():
        k = ncopies(a64(), b64())
        A, B = up(a64(), k), up(b64(), k)
        return row(lambda i: ms.lt(A[i % k], B[i % k]), 9 * 67_108_864, k=k)

    def b_eqf64():
        k = ncopies(c3()[2], c3()[3])
        s_, c_ = c3_dev("s", k), c3_dev("c", k)
        return row(lambda i: ms.eq(s_[i % k], c_[i % k]), 17 * N, k=k)

    def zpair(k):
        Z = up(zh(), k)
        return Z, [ms.neg(Z[(j + 1) % k]) for j in range(k)]

    def b_eqc64():
        k = ncopies(zh(), zh())
        Z, Z2 = zpair(k)
        return row(lambda i: ms.eq(Z[i % k], Z2[i % k]), 17 * M, k=k)

    def b_cmul(op, dt):
        def b():
            k = ncopies(zh(), zh())
            Z, Z2 = zpair(k)
            if dt == "c128":
                Z, Z2 = [ms.astype(z, "c128") for z in Z], [ms.astype(z, "c128") for z in Z2]
            return row(lambda i: getattr(ms, op)(Z[i % k], Z2[i % k]), (48 if dt == "c128" else 24) * M, k=k)
        return b

    def b_cabs():
        k = ncopies(zh())
        Z = up(zh(), k)
        return row(lambda i: ms.abs(Z[i % k]), 12 * M, k=k)

    def b_f32c64():
        k = ncopies(a64())
        A = up(a64(), k)
        return row(lambda i: ms.astype(A[i % k], "c64"), 12 * 67_108_864, k=k)

    def b_xT():
        k = ncopies(xh())
        X = up(xh(), k)
        return row(lambda i: ms.contiguous(ms.transpose(X[i % k])), 8 * n, k=k)

    def b_perm():
        ph = np.random.default_rng(1).standard_normal((8192, 128, 64), dtype=np.float32)
        k = ncopies(ph)
        P = up(ph, k)
        return row(lambda i: ms.contiguous(ms.permute(P[i % k], [2, 0, 1])), 8 * n, k=k)

    def b_flip():
        k = ncopies(xh())
        X = up(xh(), k)
        return row(lambda i: ms.contiguous(ms.flip(X[i % k], 1)), 8 * n, k=k)

    def b_c128T():
        r = np.random.default_rng(2)
        wm = (r.standard_normal((4096, 4096)) + 1j * r.standard_normal((4096, 4096))).astype(np.complex128)
        k = ncopies(wm)
        WM = up(wm, k)
        return row(lambda i: ms.contiguous(ms.transpose(WM[i % k])), 32 * 4096 * 4096, k=k)

    return [
        ("add64", "C1-64M add f32 67,108,864", b_add64),
        ("sum64", "full sum f32 64M", b_sum64),
        ("argmax64", "full argmax f32 64M", b_argmax64),
        ("sum256", "full sum f32 256M", b_sum256),
        ("argmax256", "full argmax f32 256M", b_argmax256),
        ("bcast", "C2 broadcast add (4096,1)+(8192,)", b_bcast),
        ("expT", "C2 exp transposed (8192,4096)^T", b_expT),
        ("xTc2", "contiguous of C2's transposed view f32 (8192,4096)^T", b_xTc2),
        ("exp32", "exp f32 contiguous (8192,4096)", b_exp32),
        ("c3add", "C3 add i64+f64->f64 (fused promotion)", b_c3add),
        ("clamp", "C3 clamp f64", b_clamp),
        ("f64f32", "C3 astype f64->f32", b_f64f32),
        ("bf16", "C3 astype f32->bf16", b_bf16),
        ("f16", "C3 astype f32->f16", b_f16),
        ("sum0", "C4 sum axis=0", b_c4("sum", 0, 4 * n + 4 * 8192)),
        ("mean1", "C4 mean axis=-1", b_c4("mean", -1, 4 * n + 4 * 8192)),
        ("mean0", "C4 mean axis=0", b_c4("mean", 0, 4 * n + 4 * 8192)),
        ("max01", "C4 max axis=(0,1)", b_c4("max", (0, 1), 4 * n + 4)),
        ("argmin1", "C4 argmin axis=1", b_c4("argmin", 1, 4 * n + 8 * 8192)),
        ("cumsum", "C5 cumsum f64 (1024,65536) axis=1", b_cumsum),
        ("cumsum_literal", "C5 cumsum f64, literal O(L^2) CPU form (1 of 1024 rows)", b_cumsum_literal),
        ("copy64", "contiguous f64 67,108,864 (C5's bytes as a plain copy)", b_copy64),
        ("csum", "C5 c64 sum axis=(1,2)", b_csum),
        ("lt", "cmp lt f32 64M -> bool", b_lt),
        ("eqf64", "cmp eq f64 16M -> bool", b_eqf64),
        ("eqc64", "cmp eq c64 16M -> bool", b_eqc64),
        ("c64mul", "c64 mul 16M", b_cmul("mul", "c64")),
        ("c64div", "c64 div 16M", b_cmul("div", "c64")),
        ("c64abs", "c64 abs 16M -> f32", b_cabs),
        ("f32c64", "astype f32->c64 64M", b_f32c64),
        ("c128mul", "c128 mul 16M", b_cmul("mul", "c128")),
        ("c128div", "c128 div 16M", b_cmul("div", "c128")),
        ("xT", "contiguous X^T f32 (8192,8192)", b_xT),
        ("permute", "contiguous permute(2,0,1) f32 (8192,128,64)", b_perm),
        ("flip", "contiguous flip axis=1 f32 (8192,8192)", b_flip),
        ("c128T", "contiguous ^T c128 (4096,4096)", b_c128T),
    ]


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


def mall_flushed(ms, ops, timer, steps):
    """Each op launched `steps` times, every launch timed alone by HIP events right after 768 MB of
    other traffic (an add over three 256 MB buffers) has replaced what the 256 MB Infinity Cache
    held: a cold-cache figure beside the back-to-back one.  Returns {name: median ms}: the median,
    because a single launch timed alone can catch a host-side stall (one such launch under a
    profiler read 10x the others and turned the average into a figure of the stall)."""
    h = np.full(67_108_864, 1.0, np.float32)
    F = [ms.from_numpy(h) for _ in range(3)]
    del h
    per = {}
    for _, name, fn, _ in ops:
        t = []
        for i in range(steps):
            ms.add(F[0], F[1], out=F[2])
            t.append(timer.run([lambda i=i, fn=fn: fn(i)]))
        per[name] = float(np.median(t))
    return per


def run_only(ms, key, warmup, steps):
    """--only KEY: launch one op warmup+steps times (the program rocprofv3 --pmc profiles)."""
    if key in ("add", "sum", "argmax", "copy"):
        ops, _ = step_ops(ms)
        key, name, fn, bytes_ = next(o for o in ops if o[0] == key)
    else:
        rows = {k: (n, b) for k, n, b in all_config_ops(ms)}
        if key not in rows:
            print(f"unknown --only key {key!r}; config keys: {', '.join(rows)}", file=sys.stderr)
            sys.exit(2)
        name, build = rows[key]
        fn, bytes_, _ = build()
        if fn is None:
            print(f"--only {key}: a CPU-only row", file=sys.stderr)
            sys.exit(2)
    for i in range(warmup + steps):
        fn(i)
    ms.synchronize()
    print(json.dumps({"only": key, "op": name, "launches": warmup + steps, "algo_bytes": bytes_}), flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}): this build runs on single-GPU "
              f"boxes. Elementwise ops and axis reductions shard over the non-reduced dims with no exchange; a "
              f"whole-array reduction adds one exchange of a scalar per GPU.", file=sys.stderr)
        sys.exit(2)
    import musapy_amd as ms

    timer = Timer(ms)
    if args.only:
        run_only(ms, args.only, args.warmup, args.steps)
        return
    ops, host = step_ops(ms)
    ops = [o for o in ops if o[0] != "copy"]
    for _, name, fn, _ in ops:  # warm-up (first launches load code objects, fill the memory pool)
        for i in range(max(args.warmup, 1)):
            fn(i)
    ms.synchronize()
    per_op = {}
    t0 = time.perf_counter()
    ms.synchronize()
    # K steps: each op is launched K times back-to-back between two events (inputs and outputs
    # rotate over COPIES device buffers, so every launch streams from HBM)
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
    cold = mall_flushed(ms, ops, timer, args.steps)
    cold_ms = sum(cold.values())
    line = {
        "metric": "achieved HBM GB/s (and % of MI355X peak) for f32 add, axis-sum, argmax",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(total_ms, 5),
        "wall_ms_per_step": round(wall * 1e3 / args.steps, 3),
        "timing": f"HIP events around {args.steps} back-to-back launches per op, inputs and outputs rotated over "
                  f"{COPIES} buffers",
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (numpy default_rng seed 0, BASELINE.json C1/C4 distributions)",
        "config": {"workload": "C1 add f32 16,777,216 + C4 sum axis=-1 + C4 argmax axis=1 on (8192,8192) f32",
                   "parallelism": "single GPU"},
        "frac_of_peak": round(value / PEAK_GBS, 4),
        "ops": table,
        "mall_flushed": {"value": round(total_bytes / cold_ms / 1e6, 1), "ms_per_step": round(cold_ms, 5),
                         "ops_ms": {k: round(v, 5) for k, v in cold.items()},
                         "method": "each launch timed alone by HIP events after 768 MB of other traffic "
                                   "(add over three 256 MB buffers) flushed the Infinity Cache; median "
                                   "per op"},
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": table[dom]["GBps"], "peak": PEAK_GBS,
                     "unit": "GB/s", "frac": table[dom]["frac_peak"], "traffic": traffic,
                     "algo_bytes": table[dom]["algo_bytes"],
                     "frac_basis": "event time: HIP events on the op's stream around the back-to-back launches, "
                                   "averaged (includes the gap between launches); kernel durations from "
                                   "rocprofv3 are in profiles/kernel_trace_bench_step.md",
                     "traffic_source": os.path.relpath(TRAFFIC_FILE, os.path.dirname(os.path.abspath(__file__)))
                     if traffic is not None else None},
    }
    kus = profiled_kernel_us(keys[dom])
    if kus:
        line["roofline"]["profiled_kernel_us"] = kus
        line["roofline"]["frac_by_profiled_kernel_time"] = round(table[dom]["algo_bytes"] / (kus * 1e3) / PEAK_GBS, 4)
    if not args.no_cpu:
        v, sec, sample = cpu_baseline(host)
        line["cpu_baseline"] = {"value": round(v, 3), "unit": "GB/s", "cores": 1, "kind": "port",
                                "sample": sample, "seconds_per_pass": round(sec, 3), "host": host_cpu()}
    if args.all:
        del ops, host
        rows = []
        wanted = set(args.keys.split(",")) if args.keys else None
        for key, name, build in all_config_ops(ms, host_legs=not args.no_cpu):
            if wanted is not None and key not in wanted:
                continue
            gc.collect()  # free the previous row's device arrays before this row is timed
            fn, bytes_, cpu = build()
            row = {"op": name, "key": key}
            if fn is not None:
                # fill the output ring and the memory pool before timing: the ring holds k results, so
                # the pool reaches its k + 1 blocks per row only at launch k + 1 (with 8 warm-up launches,
                # the first row of a new size class with k = 8 paid a hipMalloc inside its timed loop)
                for i in range(max(8, 2 * getattr(fn, "ring", 0))):
                    fn(i)
                ms.synchronize()
                t = timer.run([(lambda i=i, fn=fn: fn(i)) for i in range(20)])
                row.update({"ms": round(t, 5), "GBps": round(bytes_ / t / 1e6, 1),
                            "frac_peak": round(bytes_ / t / 1e6 / PEAK_GBS, 4), "host_ms": round(timer.host_ms, 5)})
            if cpu is not None:  # the CPU oracle once on the same host inputs, one thread
                t0 = time.perf_counter()
                covered = cpu()
                row["cpu_GBps"] = round(covered / (time.perf_counter() - t0) / 1e9, 3)
            rows.append(row)
            del fn, cpu
            print(json.dumps(row), file=sys.stderr, flush=True)
        line["all_configs"] = rows
        line["interop"] = interop_costs(ms)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
