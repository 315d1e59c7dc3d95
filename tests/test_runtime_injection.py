"""The op layer's error paths, driven on the CPU through the runtime's test hooks.

The runtime layer sends every HIP call through a call table.  `mpy_rt_set_backend(HOST)` swaps in
a host-memory table (one fake device; memory from the C heap; streams, events and synchronizes
as no-ops; kernel launches without effect), and `mpy_rt_inject(call, code, skip, count)` makes
chosen calls fail.  This is the counterpart of the reference's mock runtime
(rust/musapy-core/src/musa_ffi.rs:154-355) and of its error tests: a failing MUSA call is a
StreamError (musa_ffi.rs:369-380), an allocation failure an OutOfMemoryError (buffer.rs:176-185),
a launch error a KernelError (musa_ffi.rs:383-408), and a failing synchronize poisons the stream
(stream.rs:311-377).  Results computed under the fake are meaningless; only errors, poison marks
and allocation counts are checked.

Each scenario runs in a child process (the backend is process-wide).  The same scenarios run a
second time against a build whose host code carries AddressSanitizer and
UndefinedBehaviorSanitizer, together with a sweep of operators over many layouts, so the host
code's unwinding and planning paths are checked for memory and UB errors.  On a machine with a
GPU the fake backend is refused and these tests skip.
"""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "musapy_amd"))
import build as _build  # noqa: E402  (musapy_amd/build.py)

SCENARIOS = r'''
import ctypes, json, os, sys
import numpy as np
import musapy_amd as ms

lib = ctypes.CDLL(os.path.join(os.path.dirname(ms.__file__), "libmusapy_hip.so"))
MALLOC, MEMCPY, SYNC, LAUNCH, FAULT, EVENT, STREAM = range(7)
if lib.mpy_rt_set_backend(1) != 0:
    print(json.dumps({"skip": "the host backend is refused here (a HIP device is present)"}))
    sys.exit(0)
results = {"module": ms.__file__, "asan": hasattr(ctypes.CDLL(None), "__asan_init")}


def live():
    return ms.mem_stats()["live_bytes"] if isinstance(ms.mem_stats(), dict) else ms.mem_stats()[0]


def expect(name, exc, fn):
    try:
        fn()
    except Exception as e:  # noqa: BLE001
        results.setdefault(name, []).append([type(e).__name__, str(e)])
        return e
    results.setdefault(name, []).append(["none", ""])
    return None


def case(fn):
    name = fn.__name__
    try:
        fn(name)
    except Exception as e:  # noqa: BLE001
        results.setdefault(name, []).append(["unexpected " + type(e).__name__, str(e)])
    finally:
        for c in range(7):
            lib.mpy_rt_inject(c, 0, 0, 0)


A = np.arange(24, dtype=np.float32).reshape(4, 6)


@case
def launch(name):
    a = ms.from_numpy(A)
    lib.mpy_rt_inject(LAUNCH, 98, 0, 1)
    expect(name, ms.KernelError, lambda: ms.add(a, a))
    expect(name, None, lambda: ms.add(a, a))          # the error was reported once
    lib.mpy_rt_inject(LAUNCH, 98, 1, 1)               # the second launch of a two-launch op
    expect(name, None, lambda: ms.sum(a, 0))
    expect(name, ms.KernelError, lambda: ms.sum(a, 0))


@case
def sync(name):
    s = ms.Stream()
    with ms.stream(s):
        a = ms.from_numpy(A)
        b = ms.mul(a, a)
        lib.mpy_rt_inject(SYNC, 700, 0, 1)
        expect(name, ms.StreamError, lambda: s.synchronize())
        results[name + "_poisoned"] = bool(s.is_poisoned)
        expect(name, None, lambda: b.numpy())         # poison marks the stream, it does not refuse work
        expect(name, None, lambda: ms.add(b, a).numpy())


@case
def fault(name):
    s = ms.Stream()
    with ms.stream(s):
        a = ms.from_numpy(A)
        lib.mpy_rt_inject(FAULT, 2, 0, 1)
        ms.add(a, a)
        expect(name, None, lambda: s.synchronize())   # no bounded wait queued: the word is not read
        results[name + "_clean"] = not bool(s.is_poisoned)
        ms.cumsum(a, 1)
        expect(name, ms.KernelError, lambda: s.synchronize())
        results[name + "_poisoned"] = bool(s.is_poisoned)
        ms.cumsum(a, 1)
        expect(name, None, lambda: s.synchronize())   # the word was cleared by the read


@case
def oom(name):
    before = live()
    lib.mpy_rt_inject(MALLOC, 2, 0, 1)                 # one miss fails: the cache is emptied, the retry succeeds
    expect(name, None, lambda: ms.from_numpy(np.zeros(1 << 20, np.float32)))
    lib.mpy_rt_inject(MALLOC, 2, 0, 2)                 # the retry fails as well
    expect(name, ms.OutOfMemoryError, lambda: ms.from_numpy(np.zeros((1 << 20) + 64, np.float32)))
    a = ms.from_numpy(A)
    lib.mpy_rt_inject(MALLOC, 2, 0, 2)
    expect(name, ms.OutOfMemoryError, lambda: ms.contiguous(ms.transpose(a, (1, 0))).numpy())
    del a
    ms.synchronize()
    results[name + "_live_delta"] = live() - before


@case
def memcpy(name):
    before = live()
    lib.mpy_rt_inject(MEMCPY, 1, 0, 1)
    expect(name, ms.StreamError, lambda: ms.from_numpy(A))
    a = ms.from_numpy(A)
    lib.mpy_rt_inject(MEMCPY, 1, 0, 1)
    expect(name, ms.StreamError, lambda: a.numpy())
    expect(name, None, lambda: a.numpy())
    del a
    ms.synchronize()
    results[name + "_live_delta"] = live() - before


@case
def stream(name):
    lib.mpy_rt_inject(STREAM, 1, 0, 1)
    expect(name, ms.StreamError, lambda: ms.Stream())
    expect(name, None, lambda: ms.Stream())


@case
def event(name):
    before = live()
    s1, s2 = ms.Stream(), ms.Stream()
    with ms.stream(s1):
        x = ms.from_numpy(A)
        a = ms.add(x, x)                                # `a` was last written on s1
    with ms.stream(s2):
        lib.mpy_rt_inject(EVENT, 1, 0, 1)               # the cross-stream wait before reading `a`
        expect(name, ms.StreamError, lambda: ms.add(a, a))
        expect(name, None, lambda: ms.add(a, a).numpy())
    lib.mpy_rt_inject(EVENT, 1, 0, 4)                   # the free of `a` cannot order itself by event
    del a, x
    ms.synchronize()
    results[name + "_live_delta"] = live() - before


@case
def debug_ctx(name):
    """Debug mode records an OpContext per op (op_builder.rs:507-521); a failing synchronize names
    the oldest pending op (stream.rs:367-373) and a clean one clears them."""
    ms.set_debug(False)
    s = ms.Stream()
    with ms.stream(s):
        a = ms.from_numpy(A)
        ms.add(a, a)
        results[name + "_off_pending"] = s.pending_count
        ms.set_debug(True)
        b = ms.mul(a, a)
        ms.sum(b, 0)
        results[name + "_on_pending"] = s.pending_count
        lib.mpy_rt_inject(SYNC, 700, 0, 1)
        expect(name, ms.StreamError, lambda: s.synchronize())
        results[name + "_after_fail"] = s.pending_count      # a failed synchronize keeps them
        expect(name, None, lambda: s.synchronize())
        results[name + "_after_clean"] = s.pending_count
        ms.cumsum(a, 1)
        lib.mpy_rt_inject(FAULT, 1, 0, 1)
        expect(name, ms.KernelError, lambda: s.synchronize())
        ms.set_debug(False)
        with ms.debug():
            results[name + "_ctx_on"] = ms._core._is_debug()
            with ms.debug():
                pass
            results[name + "_ctx_nested"] = ms._core._is_debug()
        results[name + "_ctx_off"] = ms._core._is_debug()
        results[name + "_stream_id"] = s.id


@case
def device_sync(name):
    """ms.synchronize() reads the fault word of every stream with bounded waits queued and poisons
    only the stream that reports one."""
    s1, s2 = ms.Stream(), ms.Stream()
    with ms.stream(s1):
        a = ms.from_numpy(A)
        ms.cumsum(a, 1)                                 # bounded waits on s1
    with ms.stream(s2):
        b = ms.from_numpy(A)
        ms.add(b, b)                                    # none on s2
    lib.mpy_rt_inject(FAULT, 1, 0, 1)
    expect(name, ms.KernelError, lambda: ms.synchronize())
    results[name + "_poisoned"] = [bool(s1.is_poisoned), bool(s2.is_poisoned)]
    expect(name, None, lambda: ms.synchronize())


if "--sweep" in sys.argv:
    rng = np.random.default_rng(5)
    shapes = [(), (1,), (7,), (3, 5), (4, 1, 6), (2, 3, 4, 5), (0, 3), (5, 0)]
    n = 0
    for sh in shapes:
        x = ms.from_numpy(rng.standard_normal(sh).astype(np.float32))
        y = ms.from_numpy(rng.standard_normal(sh).astype(np.float32))
        views = [x]
        if len(sh) >= 2:
            views += [ms.transpose(x, tuple(reversed(range(len(sh))))), ms.flip(x, len(sh) - 1)]
        for v in views:
            for op in (ms.add, ms.sub, ms.mul, ms.div, ms.lt, ms.eq):
                op(v, v); n += 1
            ms.add(v, ms.array(2.0, "f32")); ms.exp(v); ms.abs(v); ms.clamp(v, -1.0, 1.0); n += 4
            for dt in ("f64", "f16", "bf16", "i64", "c64", "c128"):
                ms.astype(v, dt); n += 1
            ms.contiguous(v); n += 1
            for fn in (ms.sum, ms.max, ms.argmin, ms.mean, ms.prod):
                if v.size:
                    fn(v); n += 1
                for ax in range(len(sh)):
                    if v.shape[ax] or fn in (ms.sum, ms.prod, ms.mean):
                        fn(v, ax); n += 1
            for ax in range(len(sh)):
                ms.cumsum(v, ax); n += 1
        if len(sh) >= 2:
            ms.add(x, ms.from_numpy(np.ones(sh[-1], np.float32))); n += 1
            if sh[0]:
                ms.index_select(x, 0, sh[0] - 1); n += 1
    z = ms.from_numpy(np.ones((3, 4), np.complex128))
    ms.mul(z, z); ms.div(z, z); ms.abs(z); ms.eq(z, z); ms.transpose(z, (1, 0)).numpy(); n += 5
    ms.synchronize()
    results["sweep_ops"] = n

print(json.dumps(results))
'''


def _run(env, extra=(), cwd=ROOT):
    # `python -c` puts the working directory first on sys.path: it selects the package copy
    r = subprocess.run([sys.executable, "-c", SCENARIOS, *extra], env=env, cwd=cwd, stdout=subprocess.PIPE,
                       stderr=subprocess.PIPE, text=True, timeout=600)
    assert r.returncode == 0, f"child exited {r.returncode}\n{r.stdout[-3000:]}\n{r.stderr[-6000:]}"
    out = json.loads(r.stdout.strip().splitlines()[-1])
    if "skip" in out:
        pytest.skip(out["skip"])
    return out, r.stderr


@pytest.fixture(scope="module")
def plain():
    if not os.path.exists(_build.core_path()):
        pytest.skip("the native extension is not built")
    env = dict(os.environ)
    env["PYTHONPATH"] = ROOT + os.pathsep + env.get("PYTHONPATH", "")
    res = _run(env)[0]
    assert res["module"].startswith(os.path.join(ROOT, "musapy_amd")) and not res["asan"]
    return res


def _kinds(res, name):
    return [k for k, _ in res[name]]


def test_launch_error_is_kernel_error_and_reported_once(plain):
    assert _kinds(plain, "launch") == ["KernelError", "none", "none", "KernelError"]


def test_sync_error_poisons_and_later_work_runs(plain):
    assert _kinds(plain, "sync") == ["StreamError", "none", "none"]
    assert plain["sync_poisoned"] is True


def test_wait_fault_read_only_after_bounded_waits(plain):
    assert _kinds(plain, "fault") == ["none", "KernelError", "none"]
    assert plain["fault_clean"] is True and plain["fault_poisoned"] is True
    assert "device wait expired" in plain["fault"][1][1]


def test_debug_mode_attributes_stream_failures_to_the_oldest_op(plain):
    assert _kinds(plain, "debug_ctx") == ["StreamError", "none", "KernelError"]
    assert plain["debug_ctx_off_pending"] == 0
    assert plain["debug_ctx_on_pending"] == 2
    assert plain["debug_ctx_after_fail"] == 2 and plain["debug_ctx_after_clean"] == 0
    sid = plain["debug_ctx_stream_id"]
    msg = plain["debug_ctx"][0][1]
    assert f"| failed op: op 'mul' on stream {sid}, inputs=[(4, 6) f32, (4, 6) f32] at <string>:" in msg, msg
    assert "(debug_ctx)" in msg, msg
    assert f"failed op: op 'cumsum' on stream {sid}, inputs=[(4, 6) f32]" in plain["debug_ctx"][2][1]
    assert plain["debug_ctx_ctx_on"] is True and plain["debug_ctx_ctx_nested"] is True
    assert plain["debug_ctx_ctx_off"] is False


def test_device_synchronize_reports_the_faulting_stream(plain):
    assert _kinds(plain, "device_sync") == ["KernelError", "none"]
    assert plain["device_sync_poisoned"] == [True, False]


def test_allocation_failure_retries_then_raises(plain):
    assert _kinds(plain, "oom") == ["none", "OutOfMemoryError", "OutOfMemoryError"]
    assert plain["oom_live_delta"] == 0


def test_copy_failure_is_stream_error_and_frees(plain):
    assert _kinds(plain, "memcpy") == ["StreamError", "StreamError", "none"]
    assert plain["memcpy_live_delta"] == 0


def test_stream_create_failure(plain):
    assert _kinds(plain, "stream") == ["StreamError", "none"]


def test_event_failure_in_cross_stream_wait(plain):
    assert _kinds(plain, "event") == ["StreamError", "none"]
    assert plain["event_live_delta"] == 0


def _stale(target):
    if not os.path.exists(target):
        return True
    t = os.path.getmtime(target)
    roots = [os.path.join(ROOT, "musapy_amd", "csrc"), os.path.join(ROOT, "include")]
    files = [os.path.join(ROOT, "musapy_amd", "__init__.py"), os.path.join(ROOT, "musapy_amd", "build.py")]
    for r in roots:
        for d, _, names in os.walk(r):
            files += [os.path.join(d, n) for n in names]
    return any(os.path.getmtime(f) > t for f in files)


def test_sanitized_host_code():
    """The same scenarios plus an operator sweep under ASan + UBSan (clang's runtime)."""
    try:
        _build.asan_runtime()
    except RuntimeError as e:
        pytest.skip(str(e))
    core = os.path.join(_build.sanitized_dir(), "musapy_amd", os.path.basename(_build.core_path()))
    if _stale(core):
        _build.build_sanitized(verbose=False)
    env = _build.sanitizer_env()
    res, err = _run(env, ["--sweep"], cwd=_build.sanitized_dir())
    assert res["asan"] and os.path.dirname(res["module"]) == os.path.dirname(core), res["module"]
    assert "runtime error" not in err and "AddressSanitizer" not in err, err[-6000:]
    assert _kinds(res, "launch") == ["KernelError", "none", "none", "KernelError"]
    assert _kinds(res, "oom") == ["none", "OutOfMemoryError", "OutOfMemoryError"]
    assert _kinds(res, "event") == ["StreamError", "none"]
    assert res["sweep_ops"] > 300
