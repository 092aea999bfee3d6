"""onnx-light-cpu_amd: MatMulNBits (com.microsoft, bits=4) for AMD MI355X.

Python mirror of the operator over the C ABI in ``include/mnb.h``
(``libmnb.so``, gfx950 HIP kernels) and of the registration entry points in
``libolc_amd.so`` (C++ host side). The mirror follows the reference's Python
surface: ``register_kernels()`` / ``registered_kernels()`` /
``used_kernel_names()`` (onnx_light_cpu/_register.py:263-379) and an
operator object whose errors are ``ValueError`` with the reference's
``"<library>::<Kernel>: ..."`` message style
(onnx_light_cpu/kernels/math/matmul_kernel.cc:38-41).

There is no CPU fallback: if ``libmnb.so`` is missing or no gfx950 device is
current, every compute call raises.
"""
from __future__ import annotations

import ctypes
import os
import pathlib

import numpy as np

from . import workloads  # noqa: F401  (re-exported for bench and tests)

HERE = pathlib.Path(__file__).resolve().parent
ROOT = HERE.parent
# The built libraries: in-tree, or the directory ONNX_LIGHT_CPU_AMD_LIB_DIR
# names (the host-sanitizer build of `make -C onnx-light-cpu_amd sanitize`).
LIB_DIR = pathlib.Path(os.environ.get("ONNX_LIGHT_CPU_AMD_LIB_DIR", str(HERE)))
LIB_PATH = LIB_DIR / "libmnb.so"
HOST_LIB_PATH = LIB_DIR / "libolc_amd.so"
HEADER_PATH = ROOT / "include" / "mnb.h"

KERNEL_PREFIX = "onnx_light_cpu_amd::MatMulNBits"

STATUS = {
    0: "MNB_OK", 1: "MNB_ERR_NULL_POINTER", 2: "MNB_ERR_BAD_SHAPE", 3: "MNB_ERR_BAD_ATTRIBUTE",
    4: "MNB_ERR_UNSUPPORTED", 5: "MNB_ERR_WORKSPACE", 6: "MNB_ERR_HIP", 7: "MNB_ERR_NO_DEVICE",
    8: "MNB_ERR_ALLOC",
}
PATH_AUTO, PATH_GEMV, PATH_GEMM, PATH_GENERIC, PATH_EXACT, PATH_PREFILL = 0, 1, 2, 3, 4, 5
# MNB_KERNEL_* of include/mnb.h (mnb_run_kernel)
(KERNEL_GEMV_M1, KERNEL_GEMV_SMALL_M, KERNEL_GEMV_MFMA, KERNEL_DECODE_FRAG, KERNEL_GEMM,
 KERNEL_PREFILL, KERNEL_GEMV, KERNEL_GENERIC, KERNEL_STREAM, KERNEL_GEMV_FRAG) = range(1, 11)


class MnbDesc(ctypes.Structure):
    _fields_ = [("K", ctypes.c_int64), ("N", ctypes.c_int64), ("bits", ctypes.c_int32),
                ("block_size", ctypes.c_int32), ("accuracy_level", ctypes.c_int32),
                ("has_zero_points", ctypes.c_int32)]


_lib = None


def library():
    """Loads libmnb.so (built in-tree by ``make -C onnx-light-cpu_amd``)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built; run __graft_entry__.build()")
        L = ctypes.CDLL(str(LIB_PATH))
        vp, i64, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_size_t
        L.mnb_plan_create.argtypes = [ctypes.POINTER(MnbDesc), vp, vp, vp, ctypes.POINTER(vp)]
        L.mnb_plan_create_device.argtypes = [ctypes.POINTER(MnbDesc), vp, vp, vp,
                                             ctypes.POINTER(vp)]
        L.mnb_plan_create_gate_up.argtypes = [ctypes.POINTER(MnbDesc), vp, vp, vp, vp, vp, vp,
                                              ctypes.POINTER(vp)]
        L.mnb_rmsnorm_workspace_bytes.argtypes = [vp, i64, ctypes.POINTER(sz)]
        L.mnb_run_rmsnorm.argtypes = [vp, i64, vp, vp, ctypes.c_float, vp, vp, sz, vp]
        L.mnb_plan_destroy.argtypes = [vp]
        L.mnb_plan_device_bytes.argtypes = [vp, ctypes.POINTER(sz)]
        L.mnb_workspace_bytes.argtypes = [vp, i64, ctypes.POINTER(sz)]
        L.mnb_run.argtypes = [vp, i64, vp, vp, vp, sz, vp]
        L.mnb_run_path.argtypes = [vp, i64, vp, vp, vp, sz, vp, ctypes.c_int]
        L.mnb_run_ex.argtypes = [vp, i64, vp, vp, vp, vp, sz, vp, ctypes.c_int]
        L.mnb_run_no_alloc.argtypes = [vp, i64, vp, vp, vp]
        i32 = ctypes.c_int32
        L.mnb_qdq_repack.argtypes = [i64, i64, i32, i32, vp, vp, vp, vp, vp, vp,
                                     ctypes.POINTER(i32)]
        L.mnb_select_path.argtypes = [vp, i64, ctypes.POINTER(ctypes.c_int)]
        L.mnb_status_str.argtypes = [ctypes.c_int]
        L.mnb_status_str.restype = ctypes.c_char_p
        L.mnb_last_error.restype = ctypes.c_char_p
        L.mnb_weight_bytes.argtypes = [ctypes.POINTER(MnbDesc), ctypes.POINTER(sz)]
        L.mnb_version.restype = ctypes.c_char_p
        L.mnb_kernel_name.argtypes = [vp, i64, sz]
        L.mnb_kernel_name.restype = ctypes.c_char_p
        L.mnb_kernel_workspace_bytes.argtypes = [vp, i64, ctypes.c_int, ctypes.c_int,
                                                 ctypes.c_int, ctypes.POINTER(sz)]
        L.mnb_run_kernel.argtypes = [vp, i64, vp, vp, vp, sz, vp, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_int]
        L.mnb_stream_read.argtypes = [vp, sz, vp, sz, vp]
        L.mnb_stream_read_grid.argtypes = [vp, sz, vp, sz, ctypes.c_int, ctypes.c_int, vp]
        for name in ("mnb_plan_create", "mnb_plan_create_device", "mnb_plan_destroy",
                     "mnb_workspace_bytes", "mnb_run", "mnb_run_path", "mnb_select_path",
                     "mnb_weight_bytes", "mnb_run_ex", "mnb_qdq_repack",
                     "mnb_plan_create_gate_up", "mnb_rmsnorm_workspace_bytes",
                     "mnb_run_rmsnorm", "mnb_run_no_alloc", "mnb_kernel_workspace_bytes",
                     "mnb_run_kernel", "mnb_stream_read", "mnb_stream_read_grid",
                     "mnb_plan_device_bytes"):
            getattr(L, name).restype = ctypes.c_int
        _lib = L
    return _lib


def header_functions():
    """Names of the functions declared in include/mnb.h."""
    import re
    text = HEADER_PATH.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(mnb_\w+)\s*\(", text, re.M)))


class MatMulNBitsError(ValueError):
    """Raised for a non-OK status (the reference throws std::invalid_argument)."""

    def __init__(self, status: int, what: str):
        self.status = status
        L = library()
        detail = L.mnb_last_error().decode() if status in (6, 7, 8) else ""
        msg = f"{KERNEL_PREFIX}: {what}: {L.mnb_status_str(status).decode()}"
        if detail:
            msg += f" ({detail})"
        super().__init__(msg)


def _check(status: int, what: str):
    if status != 0:
        raise MatMulNBitsError(status, what)


def _host_ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _dev_ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


class MatMulNBits:
    """One MatMulNBits node: attributes at construction, constants at prepare().

    Mirrors the operator contract of ONNX Runtime's com.microsoft::MatMulNBits
    (attributes K, N, bits, block_size, accuracy_level; inputs A, B, scales,
    zero_points, bias). The ``g_idx`` input is rejected.
    """

    domain = "com.microsoft"
    op_type = "MatMulNBits"

    def __init__(self, K: int, N: int, bits: int = 4, block_size: int = 32,
                 accuracy_level: int = 0):
        self.desc = MnbDesc(K, N, bits, block_size, accuracy_level, 0)
        self._plan = ctypes.c_void_p()
        self._keep = ()
        self._work = None
        self._kwork = None

    # -- constants ---------------------------------------------------------
    def prepare(self, B, scales, zero_points=None):
        """Uploads host (numpy) constants once; the plan owns device copies."""
        self.release()
        self.desc.has_zero_points = int(zero_points is not None)
        B = np.ascontiguousarray(B, dtype=np.uint8)
        scales = np.ascontiguousarray(scales, dtype=np.float32)
        zp = None if zero_points is None else np.ascontiguousarray(zero_points, dtype=np.uint8)
        self._check_sizes(B.size, scales.size, None if zp is None else zp.size)
        _check(library().mnb_plan_create(ctypes.byref(self.desc), _host_ptr(B), _host_ptr(scales),
                                         _host_ptr(zp), ctypes.byref(self._plan)),
               "prepare")
        return self

    def prepare_device(self, dB, dScales, dZeroPoints=None):
        """Borrows device (torch) constants; the tensors are kept referenced."""
        self.release()
        self.desc.has_zero_points = int(dZeroPoints is not None)
        self._check_sizes(dB.numel(), dScales.numel(),
                          None if dZeroPoints is None else dZeroPoints.numel())
        _check(library().mnb_plan_create_device(ctypes.byref(self.desc), _dev_ptr(dB),
                                                _dev_ptr(dScales), _dev_ptr(dZeroPoints),
                                                ctypes.byref(self._plan)),
               "prepare_device")
        self._keep = (dB, dScales, dZeroPoints)
        return self

    def _check_sizes(self, b, s, z):
        d = self.desc
        if d.block_size <= 0 or d.K <= 0 or d.N <= 0:
            return  # the C ABI reports the attribute error
        nb = (d.K + d.block_size - 1) // d.block_size
        if b != d.N * nb * (d.block_size // 2):
            raise ValueError(f"{KERNEL_PREFIX}: B has {b} bytes, expected N*nb*bs/2 = "
                             f"{d.N * nb * (d.block_size // 2)}")
        if s != d.N * nb:
            raise ValueError(f"{KERNEL_PREFIX}: scales has {s} elements, expected {d.N * nb}")
        if z is not None and z != d.N * ((nb + 1) // 2):
            raise ValueError(f"{KERNEL_PREFIX}: zero_points has {z} bytes, expected "
                             f"{d.N * ((nb + 1) // 2)}")

    def release(self):
        if self._plan:
            library().mnb_plan_destroy(self._plan)
            self._plan = ctypes.c_void_p()
        self._keep = ()

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass

    # -- compute -----------------------------------------------------------
    def select_path(self, M: int) -> int:
        p = ctypes.c_int()
        _check(library().mnb_select_path(self._plan, M, ctypes.byref(p)), "select_path")
        return p.value

    @classmethod
    def from_qdq(cls, x, x_scale, x_zero_point=None, *, K: int, N: int, signed: bool,
                 block_size: int = 0, axis=None, accuracy_level: int = 0):
        """The MatMulNBits node for MatMul(A, DequantizeLinear(x, x_scale,
        x_zero_point)) with constant weights (see qdq_to_matmul_nbits), prepared."""
        attrs, B, S, Z = qdq_to_matmul_nbits(x, x_scale, x_zero_point, K=K, N=N, signed=signed,
                                             block_size=block_size, axis=axis)
        return cls(K, N, 4, attrs["block_size"], accuracy_level).prepare(B, S, Z)

    def __call__(self, A, out=None, path: int = PATH_AUTO, stream=None, bias=None):
        """Y[..., M, N] = A[..., M, K] * W^T on A's device (a torch CUDA tensor)."""
        import torch
        if not self._plan:
            raise ValueError(f"{KERNEL_PREFIX}: prepare() was not called")
        if not A.is_cuda or A.dtype != torch.float32:
            raise ValueError(f"{KERNEL_PREFIX}: A must be a float32 device tensor")
        if A.shape[-1] != self.desc.K:
            raise ValueError(f"{KERNEL_PREFIX}: A's last dimension {A.shape[-1]} != K "
                             f"{self.desc.K}")
        A2 = A.reshape(-1, self.desc.K).contiguous()
        M = A2.shape[0]
        if out is None:
            out = torch.empty(*A.shape[:-1], self.desc.N, device=A.device, dtype=torch.float32)
        if not out.is_contiguous() or out.numel() != M * self.desc.N:
            raise ValueError(f"{KERNEL_PREFIX}: out must be contiguous [..., M, N]")
        s = stream if stream is not None else torch.cuda.current_stream(A.device)
        if bias is not None and (bias.numel() != self.desc.N or not bias.is_contiguous()):
            raise ValueError(f"{KERNEL_PREFIX}: bias must be a contiguous [N] tensor")
        work = self.workspace(M, A.device, path)
        _check(library().mnb_run_ex(self._plan, M, _dev_ptr(A2), _dev_ptr(bias), _dev_ptr(out),
                                    _dev_ptr(work), 0 if work is None else work.numel(),
                                    ctypes.c_void_p(s.cuda_stream), path),
               "run")
        return out

    def run_rmsnorm(self, X, gamma, eps: float = 1e-5, out=None, stream=None):
        """Y = this node applied to RMSNormalization(X) (last axis, scale
        gamma [K]), the normalization fused into the run (mnb_run_rmsnorm)."""
        import torch
        if not self._plan:
            raise ValueError(f"{KERNEL_PREFIX}: prepare() was not called")
        K = self.desc.K
        if (not X.is_cuda or X.dtype != torch.float32 or X.shape[-1] != K
                or gamma.numel() != K or gamma.dtype != torch.float32):
            raise ValueError(f"{KERNEL_PREFIX}: X must be float32 [..., K] and gamma float32 [K] "
                             "device tensors")
        X2 = X.reshape(-1, K).contiguous()
        g = gamma.contiguous()
        M = X2.shape[0]
        if out is None:
            out = torch.empty(*X.shape[:-1], self.desc.N, device=X.device, dtype=torch.float32)
        n = ctypes.c_size_t()
        _check(library().mnb_rmsnorm_workspace_bytes(self._plan, M, ctypes.byref(n)),
               "rmsnorm workspace")
        if self._work is None or self._work.numel() < n.value or self._work.device != X.device:
            self._work = torch.empty(max(n.value, 1), dtype=torch.uint8, device=X.device)
        s = stream if stream is not None else torch.cuda.current_stream(X.device)
        _check(library().mnb_run_rmsnorm(self._plan, M, _dev_ptr(X2), _dev_ptr(g), float(eps),
                                         _dev_ptr(out), _dev_ptr(self._work), self._work.numel(),
                                         ctypes.c_void_p(s.cuda_stream)),
               "run_rmsnorm")
        return out

    def kernel_name(self, M: int, workspace_bytes=None) -> str:
        """The main kernel a run of M rows launches, with workspace_bytes of
        workspace (default: what workspace_bytes(M) asks for)."""
        n = self.workspace_bytes(M) if workspace_bytes is None else workspace_bytes
        return library().mnb_kernel_name(self._plan, M, n).decode()

    def run_kernel(self, A, kernel: int, p0: int = 0, p1: int = 0, out=None, stream=None):
        """One run with a chosen kernel and launch shape (mnb_run_kernel: tuning
        and cross-checks; plain plans, no bias)."""
        import torch
        A2 = A.reshape(-1, self.desc.K).contiguous()
        M = A2.shape[0]
        if out is None:
            out = torch.empty(M, self.desc.N, device=A.device, dtype=torch.float32)
        n = ctypes.c_size_t()
        _check(library().mnb_kernel_workspace_bytes(self._plan, M, kernel, p0, p1,
                                                    ctypes.byref(n)), "kernel workspace")
        work = None
        if n.value > 0:
            if self._kwork is None or self._kwork.numel() < n.value or self._kwork.device != A.device:
                self._kwork = torch.empty(n.value, dtype=torch.uint8, device=A.device)
            work = self._kwork
        s = stream if stream is not None else torch.cuda.current_stream(A.device)
        _check(library().mnb_run_kernel(self._plan, M, _dev_ptr(A2), _dev_ptr(out), _dev_ptr(work),
                                        0 if work is None else work.numel(),
                                        ctypes.c_void_p(s.cuda_stream), kernel, p0, p1),
               "run_kernel")
        return out

    def device_bytes(self) -> int:
        """Device memory the plan owns (mnb_plan_device_bytes)."""
        n = ctypes.c_size_t()
        _check(library().mnb_plan_device_bytes(self._plan, ctypes.byref(n)), "device_bytes")
        return n.value

    def workspace_bytes(self, M: int) -> int:
        n = ctypes.c_size_t()
        _check(library().mnb_workspace_bytes(self._plan, M, ctypes.byref(n)), "workspace_bytes")
        return n.value

    def workspace(self, M: int, device, path: int = PATH_AUTO):
        """Device workspace for M rows, kept and grown across calls (not during capture)."""
        import torch
        need = self.workspace_bytes(M) if path != PATH_GENERIC else 0
        if need == 0:
            return None
        if self._work is None or self._work.numel() < need or self._work.device != device:
            self._work = torch.empty(need, dtype=torch.uint8, device=device)
        return self._work

    run = __call__


class GateUpSiLU(MatMulNBits):
    """Gated-MLP front half as one plan: H[..., M, N] = silu(A Wg^T) * (A Wu^T)
    for a gate and an up MatMulNBits weight of the same shape (K, N =
    intermediate size, block_size, zero-point presence). The C ABI's
    mnb_plan_create_gate_up interleaves the two weights' rows once; every call
    needs the workspace (kept by the object). The unfused graph it replaces is
    two MatMulNBits nodes, Sigmoid and two Muls."""

    op_type = "MatMulNBitsGateUpSiLU"

    def prepare(self, Bg, Sg, Zg, Bu, Su, Zu):
        """Uploads host (numpy) gate and up constants once, rows interleaved."""
        self.release()
        if (Zg is None) != (Zu is None):
            raise ValueError(f"{KERNEL_PREFIX}: gate and up must both have zero points or neither")
        self.desc.has_zero_points = int(Zg is not None)
        arrs = []
        for B, S, Z in ((Bg, Sg, Zg), (Bu, Su, Zu)):
            B = np.ascontiguousarray(B, dtype=np.uint8)
            S = np.ascontiguousarray(S, dtype=np.float32)
            Z = None if Z is None else np.ascontiguousarray(Z, dtype=np.uint8)
            self._check_sizes(B.size, S.size, None if Z is None else Z.size)
            arrs += [B, S, Z]
        _check(library().mnb_plan_create_gate_up(ctypes.byref(self.desc),
                                                 *[_host_ptr(a) for a in arrs],
                                                 ctypes.byref(self._plan)),
               "prepare")
        return self

    def prepare_device(self, *args, **kwargs):
        raise NotImplementedError(f"{KERNEL_PREFIX}: gate/up plans are built from host weights")

    def __call__(self, A, out=None, path: int = PATH_AUTO, stream=None, bias=None):
        if bias is not None:
            raise ValueError(f"{KERNEL_PREFIX}: a gate/up plan takes no bias")
        return super().__call__(A, out=out, path=path, stream=stream)

    def workspace(self, M: int, device, path: int = PATH_AUTO):
        import torch
        need = self.workspace_bytes(M)
        if self._work is None or self._work.numel() < need or self._work.device != device:
            self._work = torch.empty(need, dtype=torch.uint8, device=device)
        return self._work

    run = __call__


def weight_bytes(K, N, block_size, has_zero_points, bits=4) -> int:
    d = MnbDesc(K, N, bits, block_size, 0, int(has_zero_points))
    b = ctypes.c_size_t()
    _check(library().mnb_weight_bytes(ctypes.byref(d), ctypes.byref(b)), "weight_bytes")
    return b.value


# ---- registration mirror (onnx_light_cpu/_register.py:263-379) over libolc_amd.so ----

_host = None


def qdq_to_matmul_nbits(x, x_scale, x_zero_point=None, *, K: int, N: int, signed: bool,
                        block_size: int = 0, axis=None):
    """Constant DequantizeLinear -> MatMul weight as MatMulNBits inputs.

    x: uint8 array, the ONNX packing of an INT4 (signed) or UINT4 [K, N] tensor
    (low nibble first); x_scale: float32 [ceil(K/block_size), N] (blocked along
    K, axis 0), [N] (per column, axis 1) or one value; x_zero_point: packed
    like x with x_scale's shape, or None. Runs the C++ recognizer
    (host/qdq_matmul.cc) over the C ABI's mnb_qdq_repack. Returns
    (attributes, B, scales, zero_points or None).
    """
    import numpy as np
    H = host_library()
    x = np.ascontiguousarray(x, dtype=np.uint8)
    sc = np.ascontiguousarray(x_scale, dtype=np.float32)
    zp = None if x_zero_point is None else np.ascontiguousarray(x_zero_point, dtype=np.uint8)
    bs_out = block_size if block_size > 0 else K
    nb = -(-K // bs_out)
    B = np.empty((N, nb, bs_out // 2), np.uint8)
    S = np.empty((N, nb), np.float32)
    Z = np.empty((N, (nb + 1) // 2), np.uint8)
    dims = (ctypes.c_int64 * max(1, sc.ndim))(*sc.shape)
    out_bs = ctypes.c_int64()
    has_zp = ctypes.c_int()
    _host_check(H.olc_amd_dequantize_linear_to_matmul_nbits(
        22 if signed else 21, K, N, _host_ptr(x), _host_ptr(sc), sc.ndim, dims, _host_ptr(zp),
        0 if axis is None else 1, 0 if axis is None else axis, block_size,
        ctypes.byref(out_bs), _host_ptr(B), B.size, _host_ptr(S), S.size, _host_ptr(Z), Z.size,
        ctypes.byref(has_zp)))
    attrs = {"K": K, "N": N, "bits": 4, "block_size": out_bs.value}
    return attrs, B, S, (Z if has_zp.value else None)


def host_library():
    """Loads libolc_amd.so, the C++ registration boundary and operator adapter."""
    global _host
    if _host is None:
        if not HOST_LIB_PATH.exists():
            raise RuntimeError(f"{HOST_LIB_PATH} is not built; run __graft_entry__.build()")
        library()  # libmnb.so first: libolc_amd.so links against it
        H = ctypes.CDLL(str(HOST_LIB_PATH))
        H.olc_amd_last_error.restype = ctypes.c_char_p
        for name in ("olc_amd_register_all_kernels", "olc_amd_register_matmul_nbits_kernel"):
            getattr(H, name).restype = ctypes.c_int
        H.olc_amd_register_pass.argtypes = [ctypes.c_char_p]
        H.olc_amd_register_pass.restype = ctypes.c_int
        for name in ("olc_amd_registered_kernels", "olc_amd_used_kernel_names",
                     "olc_amd_dispatch_keys"):
            getattr(H, name).argtypes = [ctypes.c_char_p, ctypes.c_size_t]
            getattr(H, name).restype = ctypes.c_size_t
        H.olc_amd_set_usage_recording.argtypes = [ctypes.c_int]
        vp, i64p, i32p = ctypes.c_void_p, ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int32)
        H.olc_amd_run_node.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_int, ctypes.c_int,
                                       ctypes.POINTER(ctypes.c_char_p), i64p, ctypes.c_int,
                                       ctypes.POINTER(vp), i32p, i32p, i32p, i64p, vp,
                                       ctypes.c_int64, vp, ctypes.c_size_t, vp]
        H.olc_amd_run_node.restype = ctypes.c_int
        H.olc_amd_kernel_create.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_int,
                                            ctypes.c_int, ctypes.POINTER(ctypes.c_char_p), i64p]
        H.olc_amd_kernel_create.restype = vp
        H.olc_amd_kernel_run.argtypes = [vp, ctypes.c_int, ctypes.POINTER(vp), i32p, i32p, i32p,
                                         i64p, vp, ctypes.c_int64, vp, ctypes.c_size_t, vp]
        H.olc_amd_kernel_run.restype = ctypes.c_int
        H.olc_amd_kernel_destroy.argtypes = [vp]
        H.olc_amd_dequantize_linear_to_matmul_nbits.argtypes = [
            ctypes.c_int, ctypes.c_int64, ctypes.c_int64, vp, vp, ctypes.c_int, i64p, vp,
            ctypes.c_int, ctypes.c_int64, ctypes.c_int64, i64p, vp, ctypes.c_size_t, vp,
            ctypes.c_size_t, vp, ctypes.c_size_t, ctypes.POINTER(ctypes.c_int)]
        H.olc_amd_dequantize_linear_to_matmul_nbits.restype = ctypes.c_int
        _host = H
    return _host


def _host_string(fn):
    n = fn(None, 0)
    buf = ctypes.create_string_buffer(n)
    fn(buf, n)
    return buf.value.decode()


def _host_check(rc):
    if rc != 0:
        raise ValueError(host_library().olc_amd_last_error().decode())


def register_kernels():
    """Installs this library's kernels into the dispatch table (RegisterAllKernels)."""
    _host_check(host_library().olc_amd_register_all_kernels())


def register_pass(op_types):
    """One registration pass over the listed operators; duplicates raise ValueError."""
    _host_check(host_library().olc_amd_register_pass(",".join(op_types).encode()))


def registered_kernels():
    """Inventory of registrations (CollectRegisteredKernels), without installing anything."""
    out = []
    for line in _host_string(host_library().olc_amd_registered_kernels).splitlines():
        domain, op, device, name, types, since, until = line.split("\t")
        out.append({"domain": domain, "op_type": op, "device": int(device), "kernel_name": name,
                    "types": [int(t) for t in types.split(",") if t],
                    "since_version": None if since == "-1" else int(since),
                    "until_version": None if until == "-1" else int(until)})
    return out


def dispatch_keys():
    return _host_string(host_library().olc_amd_dispatch_keys).splitlines()


def used_kernel_names():
    return _host_string(host_library().olc_amd_used_kernel_names).splitlines()


def clear_used_kernel_names():
    host_library().olc_amd_clear_used_kernel_names()


def set_kernel_usage_recording(enabled: bool):
    host_library().olc_amd_set_usage_recording(int(bool(enabled)))


DEVICE_CPU, DEVICE_GPU = 1, 2
DTYPE_FLOAT, DTYPE_UINT8 = 1, 2


def _attr_arrays(attrs):
    names = (ctypes.c_char_p * max(1, len(attrs)))(*[k.encode() for k in attrs])
    vals = (ctypes.c_int64 * max(1, len(attrs)))(*attrs.values())
    return names, vals


def _input_arrays(inputs):
    n = len(inputs)
    ptrs = (ctypes.c_void_p * max(1, n))(*[None if p is None else p for p, _, _, _ in inputs])
    types = (ctypes.c_int32 * max(1, n))(*[t for _, t, _, _ in inputs])
    devs = (ctypes.c_int32 * max(1, n))(*[d for _, _, d, _ in inputs])
    ranks = (ctypes.c_int32 * max(1, n))(*[len(s) for _, _, _, s in inputs])
    flat = [d for _, _, _, s in inputs for d in s]
    dims = (ctypes.c_int64 * max(1, len(flat)))(*flat)
    return n, ptrs, types, devs, ranks, dims


def run_node(domain, op_type, attrs, inputs, out, stream=None, device=DEVICE_GPU,
             workspace=None):
    """Runs one node through the dispatch table, as onnx-light's RunNode would.

    inputs: list of (pointer or None, dtype, device, shape) tuples; out: a
    contiguous float32 torch tensor receiving Y; workspace: a device torch
    tensor the run may use as scratch (RuntimeContext's workspace allocator),
    or None.
    """
    H = host_library()
    names, vals = _attr_arrays(attrs)
    n, ptrs, types, devs, ranks, dims = _input_arrays(inputs)
    s = None if stream is None else ctypes.c_void_p(stream)
    _host_check(H.olc_amd_run_node(
        domain.encode(), op_type.encode(), device, len(attrs), names, vals, n, ptrs, types, devs,
        ranks, dims, None if out is None else ctypes.c_void_p(out.data_ptr()),
        0 if out is None else out.numel(),
        None if workspace is None else ctypes.c_void_p(workspace.data_ptr()),
        0 if workspace is None else workspace.numel() * workspace.element_size(), s))
    return out


class NodeKernel:
    """One kernel object from the dispatch table, kept across runs the way a
    session keeps a node's kernel; runs may come from several threads at once,
    each with its own stream, output and workspace."""

    def __init__(self, domain, op_type, attrs, device=DEVICE_GPU):
        H = host_library()
        names, vals = _attr_arrays(attrs)
        self._h = H.olc_amd_kernel_create(domain.encode(), op_type.encode(), device, len(attrs),
                                          names, vals)
        if not self._h:
            raise ValueError(H.olc_amd_last_error().decode())

    def run(self, inputs, out, stream=None, workspace=None):
        H = host_library()
        n, ptrs, types, devs, ranks, dims = _input_arrays(inputs)
        s = None if stream is None else ctypes.c_void_p(stream)
        _host_check(H.olc_amd_kernel_run(
            ctypes.c_void_p(self._h), n, ptrs, types, devs, ranks, dims,
            ctypes.c_void_p(out.data_ptr()), out.numel(),
            None if workspace is None else ctypes.c_void_p(workspace.data_ptr()),
            0 if workspace is None else workspace.numel() * workspace.element_size(), s))
        return out

    def close(self):
        if self._h:
            host_library().olc_amd_kernel_destroy(ctypes.c_void_p(self._h))
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
