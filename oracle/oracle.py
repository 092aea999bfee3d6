"""MatMulNBits CPU oracle, Python side -- TEST INFRASTRUCTURE ONLY.

ctypes wrappers over ``oracle/libmnb_oracle.so`` (this repo's C restatement,
``mnb_oracle.c``) and, when it was built, ``oracle/_ref/libolc_ref.so`` (the
onnx-light-cpu reference's own sources plus ``ref_shim.cc``). Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import this
module, and only as the checker; the product path never does.

Reference anchors for what each function restates are in ``mnb_oracle.h``.
"""
from __future__ import annotations

import ctypes
import os
import pathlib

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
ORACLE_SO = HERE / "libmnb_oracle.so"
REF_SO = HERE / "_ref" / "libolc_ref.so"

_c_i64 = ctypes.c_int64
_c_ptr = ctypes.c_void_p


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


_lib = None
_ref = None


def lib():
    """The C oracle; raises if it was not built (``make -C oracle oracle``)."""
    global _lib
    if _lib is None:
        if not ORACLE_SO.exists():
            raise RuntimeError(f"oracle not built: {ORACLE_SO} (run make -C oracle oracle)")
        L = ctypes.CDLL(str(ORACLE_SO))
        sig5 = [_c_i64, _c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, ctypes.c_int]
        for name in ("mnbo_matmul_nbits_f64", "mnbo_matmul_nbits_ref_f32",
                     "mnbo_matmul_nbits_fused_f32", "mnbo_abs_dot_f64"):
            getattr(L, name).argtypes = sig5
            getattr(L, name).restype = None
        L.mnbo_dequantize.argtypes = [_c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr, _c_ptr, _c_ptr]
        L.mnbo_nibble.argtypes = [_c_ptr, _c_i64]
        L.mnbo_nibble.restype = ctypes.c_int
        L.mnbo_f32_to_f16_array.argtypes = [_c_ptr, _c_ptr, _c_i64]
        L.mnbo_f16_to_f32_array.argtypes = [_c_ptr, _c_ptr, _c_i64]
        L.mnbo_execution_block_count.argtypes = [_c_i64, ctypes.c_double, _c_i64]
        L.mnbo_execution_block_count.restype = _c_i64
        _lib = L
    return _lib


def ref_available() -> bool:
    return REF_SO.exists()


def ref():
    """The reference build (oracle/_ref); raises if absent."""
    global _ref
    if _ref is None:
        if not REF_SO.exists():
            raise RuntimeError(f"reference build absent: {REF_SO}")
        R = ctypes.CDLL(str(REF_SO))
        R.olcref_int4_matmul.argtypes = [_c_ptr, ctypes.c_int, _c_ptr, ctypes.c_int, _c_ptr,
                                         _c_i64, _c_i64, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64]
        R.olcref_matmul_f32.argtypes = [_c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr, ctypes.c_int,
                                        _c_ptr, ctypes.c_int]
        R.olcref_matmul_f32.restype = ctypes.c_int
        R.olcref_f32_to_f16_bits.argtypes = [ctypes.c_float]
        R.olcref_f32_to_f16_bits.restype = ctypes.c_uint16
        _ref = R
    return _ref


def default_threads() -> int:
    return max(1, min(16, os.cpu_count() or 1))


def _check(K, N, bs, A, B, scales, zp):
    nb = (K + bs - 1) // bs
    A = np.ascontiguousarray(A, dtype=np.float32)
    B = np.ascontiguousarray(B, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    assert A.ndim == 2 and A.shape[1] == K, A.shape
    assert B.size == N * nb * (bs // 2), (B.shape, N, nb, bs)
    assert scales.size == N * nb
    if zp is not None:
        zp = np.ascontiguousarray(zp, dtype=np.uint8)
        assert zp.size == N * ((nb + 1) // 2)
    return A, B, scales, zp


def matmul_nbits_f64(A, B, scales, zp, K, N, bs, threads=None):
    """Exact-product fp64 oracle, [M, N] float64."""
    A, B, scales, zp = _check(K, N, bs, A, B, scales, zp)
    Y = np.empty((A.shape[0], N), np.float64)
    lib().mnbo_matmul_nbits_f64(A.shape[0], K, N, bs, _ptr(A), _ptr(B), _ptr(scales), _ptr(zp),
                                _ptr(Y), threads or default_threads())
    return Y


def abs_dot_f64(A, B, scales, zp, K, N, bs, threads=None):
    """sum_k |A[m,k]| |W[n,k]| in fp64: the rounding-error scale of each output."""
    A, B, scales, zp = _check(K, N, bs, A, B, scales, zp)
    Y = np.empty((A.shape[0], N), np.float64)
    lib().mnbo_abs_dot_f64(A.shape[0], K, N, bs, _ptr(A), _ptr(B), _ptr(scales), _ptr(zp),
                           _ptr(Y), threads or default_threads())
    return Y


def matmul_nbits_ref_f32(A, B, scales, zp, K, N, bs, threads=None):
    """Reference-order fp32 (dequantize, then k-ascending mul+add per output)."""
    A, B, scales, zp = _check(K, N, bs, A, B, scales, zp)
    Y = np.empty((A.shape[0], N), np.float32)
    lib().mnbo_matmul_nbits_ref_f32(A.shape[0], K, N, bs, _ptr(A), _ptr(B), _ptr(scales),
                                    _ptr(zp), _ptr(Y), threads or default_threads())
    return Y


def matmul_nbits_fused_f32(A, B, scales, zp, K, N, bs, threads=None):
    """Fused unpack -> scale -> fp32 accumulate (the CPU int4_gemv), [M, N] float32."""
    A, B, scales, zp = _check(K, N, bs, A, B, scales, zp)
    Y = np.empty((A.shape[0], N), np.float32)
    lib().mnbo_matmul_nbits_fused_f32(A.shape[0], K, N, bs, _ptr(A), _ptr(B), _ptr(scales),
                                      _ptr(zp), _ptr(Y), threads or default_threads())
    return Y


def dequantize(B, scales, zp, K, N, bs):
    """W [N, K] float32 = (q - zp) * scale."""
    _, B, scales, zp = _check(K, N, bs, np.zeros((1, K), np.float32), B, scales, zp)
    W = np.empty((N, K), np.float32)
    lib().mnbo_dequantize(K, N, bs, _ptr(B), _ptr(scales), _ptr(zp), _ptr(W))
    return W


def dequantize_linear_4bit(x_packed, K, N, signed, scale, zp=None, block_size=0, axis=None):
    """ONNX DequantizeLinear of a constant 4-bit MatMul weight: W [K, N] float32.

    Restates the ONNX operator (opset 21 blocked quantization): element (k, n)
    of x is element k*N + n of the row-major flattening, nibble (i & 1) of
    byte i // 2, low nibble first, signed nibbles two's complement -- the
    packing the reference's ReadPacked4Bit reads
    (onnx_light_cpu/impl/math/gemm/vnni/integer_gemm_vnni.h:42-47, .cc:60-65).
    y = (x - zero_point) * scale, with the scale (and zero point) of element
    (k, n) at [k // block_size, n] when block_size > 0 (axis 0), at [n] for
    per-axis scales along axis 1, or the single value of a per-tensor scale;
    an absent zero point is 0. Plain numpy, one element at a time in effect.
    """
    xb = np.asarray(x_packed, np.uint8).ravel()
    idx = np.arange(K * N)
    q = ((xb[idx >> 1] >> ((idx & 1) * 4)) & 0xF).astype(np.int64)
    if signed:
        q = np.where(q >= 8, q - 16, q)
    q = q.reshape(K, N)
    sc = np.asarray(scale, np.float32)
    if zp is not None:
        zb = np.asarray(zp, np.uint8).ravel()
        zi = np.arange(sc.size)
        z = ((zb[zi >> 1] >> ((zi & 1) * 4)) & 0xF).astype(np.int64)
        if signed:
            z = np.where(z >= 8, z - 16, z)
        z = z.reshape(sc.shape)
    else:
        z = np.zeros(sc.shape, np.int64)
    if block_size > 0:
        rows = np.arange(K) // block_size
        s_full, z_full = sc[rows, :], z[rows, :]
    elif sc.size == N and sc.ndim == 1:
        s_full, z_full = np.broadcast_to(sc, (K, N)), np.broadcast_to(z, (K, N))
    else:
        s_full = np.full((K, N), sc.ravel()[0], np.float32)
        z_full = np.full((K, N), z.ravel()[0], np.int64)
    return ((q - z_full).astype(np.float32) * s_full).astype(np.float32)


def silu_mul_f64(g, u):
    """silu(g) * u = g * sigmoid(g) * u in fp64, sigmoid(g) = 1 / (1 + exp(-g)):
    the Sigmoid -> Mul -> Mul subgraph of a gated MLP that the gate/up plan
    fuses (docs/next_steps/2026/2026_08_qwen3_inference.rst:371-377 lists the
    fusion; the ONNX Sigmoid and Mul operators define the values). sigmoid
    is taken as 1 / (1 + exp(-g)) for g >= 0 and exp(g) / (1 + exp(g)) below,
    which neither overflows nor cancels."""
    g = np.asarray(g, np.float64)
    u = np.asarray(u, np.float64)
    e = np.exp(-np.abs(g))
    sig = np.where(g >= 0, 1.0 / (1.0 + e), e / (1.0 + e))
    return g * sig * u


def gate_up_silu_f64(A, Bg, Sg, Zg, Bu, Su, Zu, K, N, bs, threads=None):
    """H [M, N] fp64 = silu(A * Wg^T) * (A * Wu^T), both products from the
    pinned fp64 MatMulNBits restatement (matmul_nbits_f64)."""
    g = matmul_nbits_f64(A, Bg, Sg, Zg, K, N, bs, threads)
    u = matmul_nbits_f64(A, Bu, Su, Zu, K, N, bs, threads)
    return silu_mul_f64(g, u)


def rmsnorm_f64(X, gamma, eps):
    """ONNX RMSNormalization-23 over the last axis in fp64:
    X / sqrt(mean(X^2) + eps) * gamma (the schema the roadmap targets,
    docs/next_steps/2026/2026_08_qwen3_inference.rst:143, 282)."""
    X = np.asarray(X, np.float64)
    ms = np.mean(X * X, axis=-1, keepdims=True)
    return X / np.sqrt(ms + eps) * np.asarray(gamma, np.float64)


def f32_to_f16_bits(x):
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.empty(x.size, np.uint16)
    lib().mnbo_f32_to_f16_array(_ptr(x), _ptr(out), x.size)
    return out


def f16_bits_to_f32(h):
    h = np.ascontiguousarray(h, dtype=np.uint16).ravel()
    out = np.empty(h.size, np.float32)
    lib().mnbo_f16_to_f32_array(_ptr(h), _ptr(out), h.size)
    return out


def execution_block_count(total, cost, threads):
    return int(lib().mnbo_execution_block_count(total, cost, threads))


# ---- reference build wrappers (oracle/_ref) ----

def ref_matmul_f32(A, W, threads=1, trans_b=True):
    """Reference MatMulPlan<float>: Y = A @ W^T with W [N, K] passed as trans_b,
    or (trans_b=False) Y = A @ W with W [K, N], the orientation of an ONNX
    MatMul's B input."""
    A = np.ascontiguousarray(A, dtype=np.float32)
    W = np.ascontiguousarray(W, dtype=np.float32)
    M, K = A.shape
    N = W.shape[0] if trans_b else W.shape[1]
    Y = np.empty((M, N), np.float32)
    algo = ref().olcref_matmul_f32(M, N, K, _ptr(A), _ptr(W), int(trans_b), _ptr(Y), threads)
    return Y, algo


def ref_int4_matmul(a_packed, a_signed, b_packed, b_signed, rows, cols, depth, a_zp, b_zp):
    """Reference IntegerMatMul4Bit2D: int32 [rows, cols]."""
    a_packed = np.ascontiguousarray(a_packed, dtype=np.uint8)
    b_packed = np.ascontiguousarray(b_packed, dtype=np.uint8)
    a_zp = np.ascontiguousarray(np.atleast_1d(a_zp), dtype=np.int32)
    b_zp = np.ascontiguousarray(np.atleast_1d(b_zp), dtype=np.int32)
    C = np.empty((rows, cols), np.int32)
    ref().olcref_int4_matmul(_ptr(a_packed), int(a_signed), _ptr(b_packed), int(b_signed),
                             _ptr(C), rows, cols, depth, _ptr(a_zp), a_zp.size, _ptr(b_zp),
                             b_zp.size)
    return C


def ref_f32_to_f16_bits(x):
    R = ref()
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    return np.array([R.olcref_f32_to_f16_bits(float(v)) for v in x], dtype=np.uint16)


# ---- error metrics used by the parity tests ----

def normwise_max_error(y, y_ref):
    """max_i |y_i - yref_i| / max_i |yref_i| (the GEMV tolerance's metric)."""
    y = np.asarray(y, np.float64)
    y_ref = np.asarray(y_ref, np.float64)
    denom = np.max(np.abs(y_ref))
    if denom == 0:
        return float(np.max(np.abs(y - y_ref)))
    return float(np.max(np.abs(y - y_ref)) / denom)


def l2_rel_error(y, y_ref):
    """||y - yref||_2 / ||yref||_2 (the GEMM tolerance's metric)."""
    y = np.asarray(y, np.float64)
    y_ref = np.asarray(y_ref, np.float64)
    denom = np.linalg.norm(y_ref)
    if denom == 0:
        return float(np.linalg.norm(y - y_ref))
    return float(np.linalg.norm(y - y_ref) / denom)
