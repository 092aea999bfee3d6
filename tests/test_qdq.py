"""QDQ front-end (CPU): constant DequantizeLinear -> MatMul mapped onto
MatMulNBits by host/qdq_matmul.cc over the C ABI's mnb_qdq_repack.

The repacked weights must dequantize (oracle.dequantize, the MatMulNBits
definition) to exactly the float weights ONNX DequantizeLinear defines
(oracle.dequantize_linear_4bit). That restatement is pinned here by a
hand-computed case and, where the reference build is present, by the
reference's own packed-4-bit integer GEMM (IntegerMatMul4Bit2D), which reads
the same ONNX packing and per-column zero points.
"""
import ctypes

import numpy as np
import pytest


def _pack(vals):
    """ONNX 4-bit packing of small integers (two's complement for negatives)."""
    v = (np.asarray(vals, np.int64).ravel() & 0xF).astype(np.uint8)
    if v.size % 2:
        v = np.append(v, 0)
    return (v[0::2] | (v[1::2] << 4)).astype(np.uint8)


def _random_qdq(rng, K, N, signed, bs, with_zp, per="block"):
    lo, hi = (-8, 8) if signed else (0, 16)
    x = rng.integers(lo, hi, size=(K, N))
    if per == "block":
        shape = (-(-K // bs), N)
    elif per == "column":
        shape = (N,)
    else:
        shape = (1,)
    scale = rng.uniform(0.001, 0.05, size=shape).astype(np.float32)
    zp = rng.integers(lo, hi, size=shape) if with_zp else None
    return x, _pack(x), scale, (None if zp is None else _pack(zp)), zp


def test_dequantize_linear_hand_case(orc):
    """The ONNX definition worked by hand: (x - zp) * scale per block of K."""
    K, N, bs = 32, 2, 16
    x = np.array([[(k + 3 * n) % 16 - 8 for n in range(N)] for k in range(K)])
    scale = np.array([[0.5, 0.25], [2.0, 1.0]], np.float32)
    zp = np.array([[-1, 3], [0, -8]])
    want = np.empty((K, N), np.float32)
    for k in range(K):
        for n in range(N):
            want[k, n] = (x[k, n] - zp[k // bs, n]) * scale[k // bs, n]
    got = orc.dequantize_linear_4bit(_pack(x), K, N, True, scale, _pack(zp), bs)
    np.testing.assert_array_equal(got, want)
    # first element low nibble, second high: x[0,0] = -8 -> 0x8, x[0,1] = -5 -> 0xB
    assert _pack(x)[0] == 0xB8


@pytest.mark.parametrize("signed", [True, False])
@pytest.mark.parametrize("with_zp", [True, False])
@pytest.mark.parametrize("K,N,bs", [(64, 6, 16), (96, 5, 32), (300, 7, 128), (128, 33, 64),
                                    (1, 3, 16), (257, 1, 32)])
def test_blocked_repack_dequantizes_exactly(pkg, orc, signed, with_zp, K, N, bs):
    rng = np.random.default_rng(K * 31 + N * 7 + bs + signed + 2 * with_zp)
    _, xp, scale, zpp, _ = _random_qdq(rng, K, N, signed, bs, with_zp)
    attrs, B, S, Z = pkg.qdq_to_matmul_nbits(xp, scale, zpp, K=K, N=N, signed=signed,
                                             block_size=bs, axis=0)
    assert attrs == {"K": K, "N": N, "bits": 4, "block_size": bs}
    # INT4 without zero points needs no MatMulNBits zero-point input (default 8)
    assert (Z is None) == (signed and not with_zp)
    W_onnx = orc.dequantize_linear_4bit(xp, K, N, signed, scale, zpp, bs)
    W_nbits = orc.dequantize(B, S, Z, K, N, bs)
    np.testing.assert_array_equal(W_nbits, W_onnx.T)
    # padding nibbles past K in the last block are zero
    nb = -(-K // bs)
    if K % bs:
        tail = B.reshape(N, nb * bs // 2)[:, (K + 1) // 2:]
        assert not tail.any()


@pytest.mark.parametrize("per", ["column", "tensor"])
@pytest.mark.parametrize("signed,with_zp", [(True, True), (False, False), (False, True)])
def test_per_column_and_per_tensor_map_to_one_block(pkg, orc, per, signed, with_zp):
    K, N = 64, 9
    rng = np.random.default_rng(5 + signed + 2 * with_zp + (per == "tensor") * 4)
    _, xp, scale, zpp, _ = _random_qdq(rng, K, N, signed, 0, with_zp, per=per)
    attrs, B, S, Z = pkg.qdq_to_matmul_nbits(xp, scale, zpp, K=K, N=N, signed=signed,
                                             axis=1 if per == "column" else None)
    assert attrs["block_size"] == K and S.shape == (N, 1)
    W_onnx = orc.dequantize_linear_4bit(xp, K, N, signed, scale, zpp, 0)
    np.testing.assert_array_equal(orc.dequantize(B, S, Z, K, N, K), W_onnx.T)


@pytest.mark.parametrize("kw,msg", [
    (dict(block_size=16, axis=1), "blocked quantization must run along K"),
    (dict(block_size=24, axis=0), "block_size must be a power of two >= 16"),
    (dict(block_size=16, axis=0, scale_shape=(3, 5)), r"x_scale must be \[ceil"),
    (dict(block_size=0, axis=0, scale_shape=(5,)), "per-axis scales must run along N"),
    (dict(block_size=0, K=48, scale_shape=(5,), axis=1),
     "per-column and per-tensor scales map to one block of K, so K must be a power of two"),
])
def test_rejections_name_the_reason(pkg, kw, msg):
    K = kw.get("K", 64)
    N = 5
    shape = kw.get("scale_shape", (-(-K // 16), N))
    x = _pack(np.zeros((K, N), np.int64))
    scale = np.ones(shape, np.float32)
    with pytest.raises(ValueError, match="DequantizeLinearToMatMulNBits: " + msg):
        pkg.qdq_to_matmul_nbits(x, scale, None, K=K, N=N, signed=True,
                                block_size=kw["block_size"], axis=kw["axis"])


def test_c_abi_statuses(pkg):
    L = pkg.library()
    u8 = np.zeros(64, np.uint8)
    f = np.ones(8, np.float32)
    has = ctypes.c_int32()
    P = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    assert L.mnb_qdq_repack(32, 2, 16, 1, None, P(f), None, P(u8), P(f), P(u8),
                            ctypes.byref(has)) == 1  # MNB_ERR_NULL_POINTER
    assert L.mnb_qdq_repack(32, 2, 48, 1, P(u8), P(f), None, P(u8), P(f), P(u8),
                            ctypes.byref(has)) == 3  # MNB_ERR_BAD_ATTRIBUTE
    assert L.mnb_qdq_repack(0, 2, 16, 1, P(u8), P(f), None, P(u8), P(f), P(u8),
                            ctypes.byref(has)) == 2  # MNB_ERR_BAD_SHAPE


@pytest.mark.parametrize("signed", [True, False])
def test_against_reference_integer_gemm(pkg, orc, signed):
    """Per-column QDQ weights (scale 1) times integer activations: the repacked
    MatMulNBits weights give exactly the reference's IntegerMatMul4Bit2D over
    the original ONNX-packed weight with per-column zero points."""
    if not orc.ref_available():
        pytest.skip("reference build (oracle/_ref) not present")
    K, N, M = 64, 10, 3
    rng = np.random.default_rng(40 + signed)
    x, xp, _, zpp, zp = _random_qdq(rng, K, N, signed, 0, True, per="column")
    a = rng.integers(0, 16, size=(M, K))
    C = orc.ref_int4_matmul(_pack(a), False, xp, signed, M, N, K, 0, zp.astype(np.int32))
    scale = np.ones(N, np.float32)
    _, B, S, Z = pkg.qdq_to_matmul_nbits(xp, scale, zpp, K=K, N=N, signed=signed, axis=1)
    y = orc.matmul_nbits_f64(a.astype(np.float32), B, S, Z, K, N, K)
    np.testing.assert_array_equal(y, C.astype(np.float64))
