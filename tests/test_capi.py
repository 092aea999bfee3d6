"""C ABI of include/mnb.h, checked without a GPU: the library loads, exports
every declared entry point, reports sizes, and rejects bad arguments with the
documented status codes before touching the device."""
import ctypes

import numpy as np
import pytest

MNB_OK, NULLP, SHAPE, ATTR, UNSUP, WORK, HIP, NODEV, ALLOC = range(9)


def _desc(pkg, K=256, N=64, bits=4, bs=32, acc=0, zp=0):
    return pkg.MnbDesc(K, N, bits, bs, acc, zp)


def test_library_exports_every_header_function(pkg):
    L = pkg.library()
    names = pkg.header_functions()
    assert names == sorted([
        "mnb_plan_create", "mnb_plan_create_device", "mnb_plan_destroy", "mnb_workspace_bytes",
        "mnb_run", "mnb_run_path", "mnb_run_ex", "mnb_select_path", "mnb_status_str",
        "mnb_last_error", "mnb_weight_bytes", "mnb_version", "mnb_qdq_repack",
        "mnb_plan_create_gate_up", "mnb_rmsnorm_workspace_bytes", "mnb_run_rmsnorm",
        "mnb_run_no_alloc", "mnb_kernel_name", "mnb_kernel_workspace_bytes", "mnb_run_kernel",
        "mnb_plan_device_bytes",
        "mnb_stream_read", "mnb_stream_read_grid"])
    for name in names:
        assert hasattr(L, name), name


def test_version_and_status_strings(pkg):
    L = pkg.library()
    assert L.mnb_version().decode().startswith("mnb-gfx950")
    texts = {L.mnb_status_str(s).decode() for s in range(9)}
    assert len(texts) == 9
    assert L.mnb_status_str(99).decode() == "unknown status"


@pytest.mark.parametrize("cfg", ["c1", "c2", "c3", "c4"])
def test_weight_bytes_match_measurement_contract(pkg, cfg):
    """mnb_weight_bytes + A + Y equals the algorithmic bytes the roofline uses."""
    p = pkg.workloads.CONFIGS[cfg].projections[0]
    wb = pkg.weight_bytes(p.K, p.N, p.block_size, p.has_zero_points)
    assert wb == p.weight_bytes()
    expected = {"c1": (1, 10_518_528), "c2": (1, 31_498_240), "c3": (1, 37_691_392),
                "c4": (2048, 76_021_760)}[cfg]
    assert p.algorithmic_bytes(expected[0]) == expected[1]


def test_c5_layer_stack_bytes(pkg):
    c5 = pkg.workloads.CONFIGS["c5"]
    per_layer = sum(p.algorithmic_bytes(1) for p in c5.projections)
    assert per_layer * c5.layers == 3_743_940_608


@pytest.mark.parametrize("field,value,status", [
    ("bits", 3, UNSUP), ("bits", 8, UNSUP), ("block_size", 24, ATTR), ("block_size", 8, ATTR),
    ("K", 0, SHAPE), ("N", -1, SHAPE), ("accuracy_level", 7, ATTR), ("has_zero_points", 2, ATTR),
])
def test_plan_create_rejects_bad_attributes(pkg, field, value, status):
    L = pkg.library()
    d = _desc(pkg)
    setattr(d, field, value)
    plan = ctypes.c_void_p()
    B = np.zeros(64 * 8 * 16, np.uint8)
    S = np.zeros(64 * 8, np.float32)
    rc = L.mnb_plan_create(ctypes.byref(d), B.ctypes.data, S.ctypes.data, None, ctypes.byref(plan))
    assert rc == status
    assert not plan.value
    assert L.mnb_weight_bytes(ctypes.byref(d), ctypes.byref(ctypes.c_size_t())) == status


def test_plan_create_null_and_zero_point_consistency(pkg):
    L = pkg.library()
    plan = ctypes.c_void_p()
    B = np.zeros(64 * 8 * 16, np.uint8)
    S = np.zeros(64 * 8, np.float32)
    Z = np.zeros(64 * 4, np.uint8)
    d = _desc(pkg)
    assert L.mnb_plan_create(None, B.ctypes.data, S.ctypes.data, None, ctypes.byref(plan)) == NULLP
    assert L.mnb_plan_create(ctypes.byref(d), None, S.ctypes.data, None, ctypes.byref(plan)) == NULLP
    assert L.mnb_plan_create(ctypes.byref(d), B.ctypes.data, None, None, ctypes.byref(plan)) == NULLP
    assert L.mnb_plan_create(ctypes.byref(d), B.ctypes.data, S.ctypes.data, None, None) == NULLP
    # zero points given but not declared, and declared but not given
    assert L.mnb_plan_create(ctypes.byref(d), B.ctypes.data, S.ctypes.data, Z.ctypes.data,
                             ctypes.byref(plan)) == UNSUP
    dz = _desc(pkg, zp=1)
    assert L.mnb_plan_create(ctypes.byref(dz), B.ctypes.data, S.ctypes.data, None,
                             ctypes.byref(plan)) == NULLP
    assert L.mnb_plan_create_device(ctypes.byref(dz), B.ctypes.data, S.ctypes.data, None,
                                    ctypes.byref(plan)) == NULLP


def test_run_and_queries_reject_null_plan(pkg):
    L = pkg.library()
    x = ctypes.c_size_t()
    p = ctypes.c_int()
    assert L.mnb_run(None, 1, None, None, None, 0, None) == NULLP
    assert L.mnb_run_path(None, 1, None, None, None, 0, None, 1) == NULLP
    assert L.mnb_run_ex(None, 1, None, None, None, None, 0, None, 1) == NULLP
    assert L.mnb_workspace_bytes(None, 1, ctypes.byref(x)) == NULLP
    assert L.mnb_select_path(None, 1, ctypes.byref(p)) == NULLP
    assert L.mnb_run_no_alloc(None, 1, None, None, None) == NULLP
    assert L.mnb_plan_destroy(None) == MNB_OK
    assert L.mnb_plan_device_bytes(None, ctypes.byref(x)) == NULLP
    assert L.mnb_run_rmsnorm(None, 1, None, None, 1e-5, None, None, 0, None) == NULLP
    assert L.mnb_rmsnorm_workspace_bytes(None, 1, ctypes.byref(x)) == NULLP


def test_stream_probes_validate_before_the_device(pkg):
    """The read probes reject null buffers, empty or oversized reads, bad
    grids and a short output before any HIP call (fake non-null pointers are
    never dereferenced on these paths)."""
    L = pkg.library()
    fake = ctypes.c_void_p(0x1000)
    assert L.mnb_stream_read(None, 1024, fake, 2048, None) == NULLP
    assert L.mnb_stream_read(fake, 0, fake, 2048, None) == SHAPE
    assert L.mnb_stream_read(fake, 1024, fake, 100, None) == WORK
    assert L.mnb_stream_read_grid(fake, 1024, None, 2048, 224, 512, None) == NULLP
    assert L.mnb_stream_read_grid(fake, 1 << 31, fake, 2048, 224, 512, None) == SHAPE
    for wgs, threads in ((224, 500), (224, 0), (224, 2048), (0, 512), (70000, 64)):
        assert L.mnb_stream_read_grid(fake, 1024, fake, 1 << 20, wgs, threads, None) == SHAPE
    assert L.mnb_stream_read_grid(fake, 1024, fake, 1791, 224, 512, None) == WORK


def test_gate_up_plan_validates_before_the_device(pkg):
    """mnb_plan_create_gate_up checks both weights' pointers and the doubled
    row count before any HIP call."""
    L = pkg.library()
    plan = ctypes.c_void_p()
    B = np.zeros(64 * 8 * 16, np.uint8)
    S = np.zeros(64 * 8, np.float32)
    Z = np.zeros(64 * 4, np.uint8)
    P = lambda a: a.ctypes.data
    d = _desc(pkg)
    assert L.mnb_plan_create_gate_up(ctypes.byref(d), P(B), P(S), None, None, P(S), None,
                                     ctypes.byref(plan)) == NULLP
    assert L.mnb_plan_create_gate_up(ctypes.byref(d), P(B), P(S), None, P(B), P(S), None,
                                     None) == NULLP
    dz = _desc(pkg, zp=1)
    assert L.mnb_plan_create_gate_up(ctypes.byref(dz), P(B), P(S), P(Z), P(B), P(S), None,
                                     ctypes.byref(plan)) == NULLP
    assert L.mnb_plan_create_gate_up(ctypes.byref(d), P(B), P(S), P(Z), P(B), P(S), None,
                                     ctypes.byref(plan)) == UNSUP
    big = _desc(pkg, N=(1 << 29) + 1)
    assert L.mnb_plan_create_gate_up(ctypes.byref(big), P(B), P(S), None, P(B), P(S), None,
                                     ctypes.byref(plan)) == SHAPE
    assert not plan.value


def test_plan_create_without_gpu_reports_no_device(pkg):
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    L = pkg.library()
    d = _desc(pkg)
    plan = ctypes.c_void_p()
    B = np.zeros(64 * 8 * 16, np.uint8)
    S = np.zeros(64 * 8, np.float32)
    rc = L.mnb_plan_create(ctypes.byref(d), B.ctypes.data, S.ctypes.data, None, ctypes.byref(plan))
    assert rc == NODEV
    assert not plan.value


def test_python_operator_validates_sizes(pkg):
    op = pkg.MatMulNBits(256, 64, 4, 32)
    with pytest.raises(ValueError, match="onnx_light_cpu_amd::MatMulNBits: B has"):
        op.prepare(np.zeros(10, np.uint8), np.zeros(64 * 8, np.float32))
    with pytest.raises(ValueError, match="scales has"):
        op.prepare(np.zeros(64 * 8 * 16, np.uint8), np.zeros(3, np.float32))
    with pytest.raises(ValueError, match="zero_points has"):
        op.prepare(np.zeros(64 * 8 * 16, np.uint8), np.zeros(64 * 8, np.float32),
                   np.zeros(5, np.uint8))
    bad = pkg.MatMulNBits(256, 64, 3, 32)
    with pytest.raises(ValueError, match="unsupported"):
        bad.prepare(np.zeros(64 * 8 * 16, np.uint8), np.zeros(64 * 8, np.float32))


@pytest.mark.parametrize("K,N,bs,zp", [(96, 5, 32, True), (256, 3, 64, False), (160, 7, 32, True)])
def test_gate_up_interleave_reads_exactly_the_inputs(pkg, K, N, bs, zp):
    """Without a GPU, mnb_plan_create_gate_up still interleaves the two weights
    on the host before the device check: on exactly-sized inputs (odd block
    counts, an odd number of rows) it reports MNB_ERR_NO_DEVICE. Under the
    host-sanitizer build (`make -C onnx-light-cpu_amd sanitize-test`) any read
    past an input or write past the interleaved copies aborts the run."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    L = pkg.library()
    nb = (K + bs - 1) // bs
    rng = np.random.default_rng(K + N)
    mk = lambda n, dt: (rng.integers(0, 256, n).astype(dt) if dt == np.uint8
                        else rng.random(n).astype(dt))
    Bg, Bu = mk(N * nb * bs // 2, np.uint8), mk(N * nb * bs // 2, np.uint8)
    Sg, Su = mk(N * nb, np.float32), mk(N * nb, np.float32)
    Zg = mk(N * ((nb + 1) // 2), np.uint8) if zp else None
    Zu = mk(N * ((nb + 1) // 2), np.uint8) if zp else None
    d = pkg.MnbDesc(K, N, 4, bs, 0, 1 if zp else 0)
    plan = ctypes.c_void_p()
    P = lambda a: None if a is None else a.ctypes.data
    assert L.mnb_plan_create_gate_up(ctypes.byref(d), P(Bg), P(Sg), P(Zg), P(Bu), P(Su), P(Zu),
                                     ctypes.byref(plan)) == NODEV
    assert not plan.value
