"""CPU-side tests of the C ABI: the library loads, exports every declared entry
point, and the host logic (errors, argument checks, top_k_reduce) behaves like the
reference.  No kernel runs here."""
import ctypes
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "vector_hip.h")


def _declared():
    txt = open(HEADER).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(vhip_[a-z0-9_]+)\s*\(", txt)))


def test_library_exports_every_declared_symbol():
    import vector_hip as vh

    lib = ctypes.CDLL(vh.library_path())
    names = _declared()
    assert len(names) >= 40
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"


def _dt_needed(path):
    """DT_NEEDED entries of an ELF64 little-endian shared library, read from its dynamic section."""
    import struct

    data = open(path, "rb").read()
    assert data[:4] == b"\x7fELF" and data[4] == 2 and data[5] == 1, "not an ELF64 little-endian file"
    shoff, = struct.unpack_from("<Q", data, 0x28)
    shentsize, shnum = struct.unpack_from("<HH", data, 0x3A)
    secs = [struct.unpack_from("<IIQQQQIIQQ", data, shoff + i * shentsize) for i in range(shnum)]
    dyn = [s for s in secs if s[1] == 6]  # SHT_DYNAMIC
    assert len(dyn) == 1, "no dynamic section"
    _, _, _, _, off, size, link, _, _, _ = dyn[0]
    stroff = secs[link][4]
    out = []
    for i in range(0, size, 16):
        tag, val = struct.unpack_from("<qQ", data, off + i)
        if tag == 0:
            break
        if tag == 1:  # DT_NEEDED
            end = data.index(b"\0", stroff + val)
            out.append(data[stroff + val:end].decode())
    return out


def test_no_torch_or_oracle_in_product():
    """The product neither imports nor links the oracle (test infrastructure only) or torch: the
    Python binding, every native source, and the built library's DT_NEEDED list."""
    import vector_hip as vh

    pkg = os.path.dirname(vh.__file__)
    srcs = [os.path.join(pkg, f) for f in os.listdir(pkg) if f.endswith(".py")]
    csrc = os.path.join(os.path.dirname(pkg), "csrc")
    srcs += [os.path.join(csrc, f) for f in os.listdir(csrc)]
    srcs += [os.path.join(ROOT, "include", f) for f in os.listdir(os.path.join(ROOT, "include"))]
    assert len(srcs) > 20
    for path in srcs:
        src = open(path).read()
        for bad in ("import oracle", "from oracle", "vh_oracle", "import torch", "torch/"):
            assert bad not in src, f"{path} names {bad!r}"
    needed = _dt_needed(vh.library_path())
    assert any(n.startswith("libamdhip64") for n in needed), needed
    assert not [n for n in needed if "oracle" in n or "torch" in n or "c10" in n], needed


def test_device_count_is_nonnegative():
    import vector_hip as vh

    assert vh.CudaDeviceContext.device_count() >= 0


def test_insufficient_devices_error():
    """distributed_knn.rs:470-494, ddp/mod.rs:106-122, integration_tests.rs:163-177."""
    import vector_hip as vh

    avail = vh.CudaDeviceContext.device_count()
    data = np.array([1, 2, 3, 4], np.float32)
    with pytest.raises(vh.InsufficientDevices) as ei:
        vh.DistributedKnnEngine.try_new(data, 2, avail + 100, vh.GpuShardMode.Sharded, vh.DistanceMetric.L2Squared)
    assert ei.value.requested == avail + 100 and ei.value.available == avail
    with pytest.raises(vh.InsufficientDevices) as ei:
        vh.DistributedKMeansEngine.try_new(avail + 10)
    assert ei.value == vh.InsufficientDevices(avail + 10, avail)


def test_invalid_config_errors():
    import vector_hip as vh

    with pytest.raises(vh.InvalidConfig):
        vh.DistributedKnnEngine.emulator(np.zeros(4, np.float32), 2, 0)
    with pytest.raises(vh.InvalidConfig):
        vh.CudaKnnEngine(np.zeros(5, np.float32), 2)  # length not a multiple of dimension
    h = ctypes.c_void_p()
    lib = ctypes.CDLL(vh.library_path())
    lib.vhip_knn_create.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_void_p]
    assert lib.vhip_knn_create(None, 0, 4, 42, 0, ctypes.byref(h)) == -5  # unknown metric
    assert lib.vhip_knn_create(None, 0, 0, 0, 0, ctypes.byref(h)) == -5   # dimension 0


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="checks the no-GPU error path")
def test_no_gpu_is_an_error_not_a_fallback():
    import vector_hip as vh

    with pytest.raises((vh.HardwareNotAvailable, vh.DeviceNotFound)):
        vh.CudaKnnEngine(np.zeros((4, 2), np.float32), 2)


def test_top_k_reduce_matches_reference_kats_and_oracle(oracle):
    """collective.rs:239-282 known answers, and agreement with the oracle's restatement
    (same BinaryHeap rules) on random lists with ties."""
    import vector_hip as vh

    R = vh.SearchResult
    m = vh.CollectiveOps.top_k_reduce([[R(0, 1.0), R(1, 5.0)], [R(10, 0.5), R(11, 4.0)]], 2)
    assert [r.id for r in m] == [10, 0]
    assert vh.CollectiveOps.top_k_reduce([], 5) == []
    assert vh.CollectiveOps.top_k_reduce([[R(0, 1.0)]], 0) == []
    m = vh.CollectiveOps.top_k_reduce([[R(0, .85), R(1, .40)], [R(2, .95), R(3, .70)]], 3,
                                      vh.DistanceMetric.CosineSimilarity)
    assert [r.id for r in m] == [2, 0, 3]
    m = vh.CollectiveOps.top_k_reduce([[R(0, 2.0)], [R(1, 1.0)]], 10)
    assert [r.id for r in m] == [1, 0]
    rng = np.random.default_rng(1)
    for trial in range(20):
        lists = []
        for r in range(3):
            n = rng.integers(0, 12)
            ids = rng.integers(0, 1000, n)
            d = rng.integers(0, 6, n).astype(np.float32)  # many ties
            lists.append((ids, d))
        k = int(rng.integers(1, 10))
        metric = "cosine" if trial % 2 else "l2"
        oi, od = oracle.top_k_reduce(lists, k, metric)
        got = vh.CollectiveOps.top_k_reduce([[R(int(a), float(b)) for a, b in zip(*l)] for l in lists], k,
                                            vh.DistanceMetric.CosineSimilarity if trial % 2 else
                                            vh.DistanceMetric.L2Squared)
        assert [r.id for r in got] == list(oi) and np.allclose([r.distance for r in got], od)


def test_device_context_emulator_descriptor():
    """CudaDeviceContext.with_ordinal / new (device.rs:120-221) return a software-emulator
    descriptor for an ordinal with no usable device; with_ordinal_strict raises.  A descriptor
    runs nothing: an engine on that ordinal raises instead of falling back to the CPU."""
    import vector_hip as vh

    missing = vh.CudaDeviceContext.device_count() + 100
    c = vh.CudaDeviceContext.with_ordinal(missing)
    assert not c.is_hardware_available() and c.device_id() == missing and c.total_memory_bytes() == 0
    s = vh.CudaDeviceContext.software_emulator(3)
    assert not s.is_hardware_available() and s.device_id() == 3
    with pytest.raises((vh.DeviceNotFound, vh.HardwareNotAvailable)) as ei:
        vh.CudaDeviceContext.with_ordinal_strict(missing)
    if isinstance(ei.value, vh.DeviceNotFound):
        assert ei.value.ordinal == missing
    with pytest.raises((vh.DeviceNotFound, vh.HardwareNotAvailable)):
        vh.CudaKnnEngine.with_ordinal(np.zeros((4, 2), np.float32), 2, vh.DistanceMetric.L2Squared, missing)
