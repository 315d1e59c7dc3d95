"""DLPack exchange and the NumPy protocols on the GPU.

* musapy_amd -> musapy_amd through the capsule protocol: zero copy (same device pointer),
  strides and offsets of views kept, every dtype, unversioned and versioned capsules, lifetime
  (the producer's buffer outlives the producer object), stream ordering across streams.
* host tensors (NumPy) are copied in; ``np.asarray`` reads back; NumPy ufuncs on device arrays
  run the device op, and mixing in host data raises (strict policy).
* PyTorch-ROCm, both directions, in a child process that imports torch first so that torch and
  this backend share one HIP runtime (a process that loads this backend's runtime first and
  torch's copy second would hold two).
"""
import gc
import os
import subprocess
import sys

import numpy as np
import pytest

import musapy_amd as ms
from tests.conftest import assert_bits_equal

pytestmark = pytest.mark.gpu
RNG = np.random.default_rng(99)
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DTYPES = [np.bool_, np.int8, np.int16, np.int32, np.int64, np.uint8, np.uint16, np.uint32, np.uint64, np.float16,
          np.float32, np.float64, np.complex64, np.complex128]


def rand(shape, dt):
    raw = RNG.integers(0, 256, int(np.prod(shape)) * np.dtype(dt).itemsize, dtype=np.uint8)
    if dt == np.bool_:
        raw &= 1
    return raw.view(dt).reshape(shape)


@pytest.mark.parametrize("dt", DTYPES, ids=lambda d: np.dtype(d).name)
def test_roundtrip_zero_copy_views(dt):
    x = rand((7, 12, 5), dt)
    A = ms.from_numpy(x)
    views = [
        (A, x),
        (ms.transpose(A), x.T),
        (ms.flip(A, 1), x[:, ::-1]),
        (A[2:, 3:11:2, 1], x[2:, 3:11:2, 1]),
        (A[4], x[4]),
        (A[1, 2, 3], x[1, 2, 3]),
    ]
    for v, want in views:
        b = ms.from_dlpack(v)
        assert b.data_ptr == v.data_ptr
        assert b.shape == v.shape and b.strides == v.strides and b.dtype == v.dtype
        assert_bits_equal(b.numpy(), want, f"{np.dtype(dt).name} view", nan_bits=True)
    assert A.__dlpack_device__() == (10, 0)


def test_capsule_protocol_details():
    A = ms.from_numpy(np.arange(12, dtype=np.float32).reshape(3, 4))
    cap = A.__dlpack__()
    assert type(cap).__name__ == "PyCapsule" and "dltensor" in repr(cap)
    capv = A.__dlpack__(max_version=(1, 0))
    assert "dltensor_versioned" in repr(capv)
    del cap, capv  # unconsumed capsules release the array through their deleters
    legacy = A.__dlpack__(max_version=(0, 8))
    assert "dltensor_versioned" not in repr(legacy)
    del legacy
    with pytest.raises(BufferError):
        A.__dlpack__(dl_device=(1, 0))
    A.__dlpack__(dl_device=(10, 0))
    C = ms.from_dlpack(A, copy=True)
    assert C.data_ptr != A.data_ptr and C.tolist() == A.tolist()
    with pytest.raises(TypeError):
        ms.from_dlpack([1, 2, 3])


def test_lifetime_and_release():
    gc.collect()
    ms.synchronize()
    base = ms.mem_stats()["live_bytes"]
    x = RNG.standard_normal((1024, 1024)).astype(np.float32)
    A = ms.from_numpy(x)
    B = ms.from_dlpack(ms.transpose(A))
    del A  # the producer object goes; the adopted view keeps the memory alive
    gc.collect()
    assert_bits_equal(B.numpy(), x.T, "after producer deleted")
    assert_bits_equal(ms.sum(B, axis=0).numpy(), ms.sum(ms.from_numpy(x), axis=1).numpy(), "ops on adopted view")
    del B
    caps = [ms.from_numpy(x).__dlpack__() for _ in range(3)]  # never consumed
    del caps
    gc.collect()
    ms.synchronize()
    assert ms.mem_stats()["live_bytes"] <= base


def test_stream_ordering_between_producer_and_consumer():
    s1, s2 = ms.Stream(), ms.Stream()
    x = RNG.standard_normal(1 << 22).astype(np.float32)
    with ms.stream(s1):
        X = ms.from_numpy(x)
        Y = ms.exp(ms.add(X, X))  # queued on s1
    with ms.stream(s2):
        Z = ms.from_dlpack(Y)  # s2 waits for s1's write before using the memory
        assert Z.stream == s2
        S = ms.neg(Z)
    got = S.numpy()
    want = -np.exp(x + x)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.max(np.abs(got - want) / np.maximum(np.abs(want), 1e-30)) < 1e-6


def test_host_tensors_and_numpy_protocols():
    x = RNG.standard_normal((33, 17)).astype(np.float64)
    A = ms.from_dlpack(x)  # host producer: copied to the device
    assert A.device == "hip:0" and A.dtype == "f64"
    assert_bits_equal(A.numpy(), x, "host import")
    with pytest.raises(BufferError):
        ms.from_dlpack(x, copy=False)
    assert_bits_equal(np.asarray(A), x, "np.asarray")
    assert np.asarray(A, dtype=np.float32).dtype == np.float32
    B = ms.from_numpy(RNG.standard_normal((33, 17)))
    r = np.add(A, B)
    assert isinstance(r, ms.Array)
    assert_bits_equal(r.numpy(), x + B.numpy(), "np.add on device arrays")
    assert isinstance(np.less(A, B), ms.Array) and np.less(A, B).dtype == "b1"
    assert_bits_equal(np.negative(A).numpy(), -x, "np.negative", nan_bits=True)
    out = ms.from_numpy(np.zeros_like(x))
    np.multiply(A, B, out=(out,))
    assert_bits_equal(out.numpy(), x * B.numpy(), "np.multiply out=")
    with pytest.raises(ms.DeviceError):
        np.add(A, x)
    with pytest.raises(TypeError):
        np.arctan2(A, B)


TORCH_SCRIPT = r"""
import sys
import torch  # first: one HIP runtime (torch's) serves both libraries in this process
import numpy as np
sys.path.insert(0, sys.argv[1])
import musapy_amd as ms

maps = open("/proc/self/maps").read()
libs = {l.split()[-1] for l in maps.splitlines() if "libamdhip64" in l}
assert len(libs) == 1, libs
print("hip runtimes:", libs, flush=True)
dev = torch.device("cuda:0")
g = torch.Generator(device="cpu").manual_seed(5)

# torch -> musapy_amd: zero copy, strided views, values
t = torch.randn(256, 384, generator=g).to(dev)
for name, v in (("contig", t), ("T", t.t()), ("slice", t[3:200:3, 5:])):
    a = ms.from_dlpack(v)
    assert a.data_ptr == v.data_ptr(), name
    assert a.shape == tuple(v.shape) and list(a.strides) == list(v.stride()), name
    assert np.array_equal(a.numpy(), v.cpu().numpy()), name
    s = ms.sum(a, axis=1).numpy()
    assert np.allclose(s, v.sum(dim=1).cpu().numpy(), rtol=1e-5, atol=1e-4), name
print("torch->ms ok", flush=True)

# musapy_amd writes into torch-owned memory through out=
o = torch.empty(256, 384, device=dev)
ms.add(ms.from_dlpack(t), ms.from_dlpack(t), out=ms.from_dlpack(o))
torch.cuda.synchronize()
ms.synchronize()
assert torch.equal(o, t + t)
print("out= into torch memory ok", flush=True)

# musapy_amd -> torch: zero copy, views, dtypes
x = np.random.default_rng(1).standard_normal((64, 96)).astype(np.float32)
A = ms.from_numpy(x)
T = torch.from_dlpack(A)
assert T.device.type == "cuda" and T.data_ptr() == A.data_ptr
assert np.array_equal(T.cpu().numpy(), x)
V = torch.from_dlpack(ms.transpose(A))
assert tuple(V.stride()) == (1, 96) and np.array_equal(V.cpu().numpy(), x.T)
del A
import gc; gc.collect()
assert np.array_equal(T.cpu().numpy(), x)  # torch keeps the buffer alive
for npdt, tdt in ((np.float64, torch.float64), (np.int64, torch.int64), (np.int32, torch.int32),
                  (np.uint8, torch.uint8), (np.bool_, torch.bool), (np.float16, torch.float16),
                  (np.complex64, torch.complex64), (np.complex128, torch.complex128)):
    h = (np.random.default_rng(2).standard_normal(50) * 10).astype(npdt)
    tt = torch.from_dlpack(ms.from_numpy(h))
    assert tt.dtype == tdt, (npdt, tt.dtype)
    assert np.array_equal(tt.cpu().numpy(), h), npdt
    back = ms.from_dlpack(torch.from_numpy(h).to(dev))
    assert np.array_equal(back.numpy(), h), npdt
bf = torch.randn(40, generator=g).to(torch.bfloat16).to(dev)
mb = ms.from_dlpack(bf)
assert mb.dtype == "bf16" and np.array_equal(mb.numpy(), bf.view(torch.int16).cpu().numpy().view(np.uint16))
print("ms->torch ok", flush=True)

# ordering: torch's pending work on its stream is complete before a musapy_amd op reads it
big = torch.zeros(1 << 24, device=dev)
big.add_(1.0).mul_(3.0)
m = ms.from_dlpack(big)
assert abs(float(ms.sum(m).numpy()) - 3.0 * (1 << 24)) <= 8.0
print("ordering ok", flush=True)
"""


def test_torch_interop_in_one_runtime():
    r = subprocess.run([sys.executable, "-c", TORCH_SCRIPT, ROOT], capture_output=True, text=True, timeout=300)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
