"""Registration boundary, mirroring the reference's registration tests
(unittests/cc/test_onnx_light_kernel_registration.cc:30-198): inventory
contents, no mutation while collecting, duplicate rejection, dispatch keys,
usage log, and the operator adapter's argument errors (raised on the host
before any device work)."""
import pytest


def test_inventory_lists_matmul_nbits(pkg):
    inv = pkg.registered_kernels()
    assert inv == [{
        "domain": "com.microsoft", "op_type": "MatMulNBits", "device": pkg.DEVICE_GPU,
        "kernel_name": "onnx_light_cpu_amd::MatMulNBitsKernel", "types": [pkg.DTYPE_FLOAT],
        "since_version": 1, "until_version": None}]


def test_collecting_does_not_install(pkg):
    pkg.host_library().olc_amd_clear_dispatch_table()
    pkg.registered_kernels()
    assert pkg.dispatch_keys() == []
    pkg.register_kernels()
    assert pkg.dispatch_keys() == ["com.microsoft:MatMulNBits@2"]
    # registering again in a new pass replaces, as onnx-light's table does
    pkg.register_kernels()
    assert pkg.dispatch_keys() == ["com.microsoft:MatMulNBits@2"]


def test_duplicate_in_one_pass_throws(pkg):
    with pytest.raises(ValueError, match="duplicate registration for domain 'com.microsoft', "
                                         "operator 'MatMulNBits', device 2"):
        pkg.register_pass(["MatMulNBits", "MatMulNBits"])
    with pytest.raises(ValueError, match="unknown operator"):
        pkg.register_pass(["Gemm"])
    pkg.register_pass(["MatMulNBits"])


def _run(pkg, attrs, inputs, out=None):
    return pkg.run_node("com.microsoft", "MatMulNBits", attrs, inputs, out)


ATTRS = {"K": 64, "N": 8, "bits": 4, "block_size": 32}


def _inputs(pkg, a_type=1, b_type=2, s_type=1, zp=None, g_idx=False, bias=None, n_b=8 * 32):
    # device pointers are never dereferenced: every case fails validation first
    dev = pkg.DEVICE_GPU
    ins = [(0x1000, a_type, dev, [1, 64]), (0x2000, b_type, dev, [n_b]),
           (0x3000, s_type, dev, [8, 2])]
    if zp or g_idx or bias:
        ins.append(zp if zp else (None, 2, dev, [0]))
    if g_idx or bias:
        ins.append((0x5000, 6, dev, [64]) if g_idx else (None, 6, dev, [0]))
    if bias:
        ins.append(bias)
    return ins


@pytest.mark.parametrize("attrs,msg", [
    ({"N": 8, "bits": 4, "block_size": 32}, "missing attribute 'K'"),
    ({"K": 64, "N": 8, "bits": 8, "block_size": 32}, "only bits=4 is supported"),
    ({"K": 64, "N": 8, "bits": 4, "block_size": 48}, "block_size must be a power of two"),
    ({"K": 64, "N": 8, "bits": 4, "block_size": 32, "accuracy_level": 9}, "accuracy_level"),
])
def test_adapter_attribute_errors(pkg, attrs, msg):
    pkg.register_kernels()
    with pytest.raises(ValueError, match="onnx_light_cpu_amd::MatMulNBitsKernel: " + msg):
        _run(pkg, attrs, _inputs(pkg))


@pytest.mark.parametrize("kw,msg", [
    ({"a_type": 10}, "input A must be float"),
    ({"b_type": 1}, "input B must be uint8"),
    ({"s_type": 10}, "input scales must be float"),
    ({"n_b": 7}, "B must have"),
    ({"g_idx": True}, "input g_idx is not supported"),
    ({"bias": (0x6000, 6, 2, [8])}, "input bias must be float"),
    ({"bias": (0x6000, 1, 2, [7])}, "bias must have N=8 elements"),
    ({"bias": (0x6000, 1, 1, [8])}, "bias must be in device memory"),
    ({"zp": (0x4000, 1, 2, [8])}, "zero_points must be uint8"),
    ({"zp": (0x4000, 2, 2, [3])}, "zero_points must have"),
])
def test_adapter_input_errors_and_usage_log(pkg, kw, msg):
    import torch
    pkg.register_kernels()
    pkg.clear_used_kernel_names()
    out = torch.empty(8)
    with pytest.raises(ValueError, match=msg):
        _run(pkg, ATTRS, _inputs(pkg, **kw), out)
    # Run() records usage first, as the reference kernels do (kernel_usage.cc:36-42)
    assert pkg.used_kernel_names() == ["onnx_light_cpu_amd::MatMulNBitsKernel"]


def test_usage_recording_switch(pkg):
    import torch
    pkg.register_kernels()
    pkg.clear_used_kernel_names()
    pkg.set_kernel_usage_recording(False)
    try:
        with pytest.raises(ValueError):
            _run(pkg, ATTRS, _inputs(pkg, a_type=10), torch.empty(8))
        assert pkg.used_kernel_names() == []
    finally:
        pkg.set_kernel_usage_recording(True)


def test_unregistered_operator(pkg):
    with pytest.raises(ValueError, match="no kernel for 'ai.onnx:MatMul'"):
        pkg.run_node("", "MatMul", {}, [], None)
