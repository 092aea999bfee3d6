"""Pins the CPU oracle (oracle/mnb_oracle.c) before it is trusted as the checker.

Each oracle function is checked against something other than its own formula:
  - golden fixtures written by the reference's compiled code (tests/golden):
    its fp32 MatMul engine on the dequantized weights, its packed-4-bit integer
    GEMM, its fp32 -> fp16 conversion;
  - the reference build itself, live, where oracle/_ref is present;
  - numpy's independent float16 rounding;
  - closed forms, invariants and brute force on tiny shapes.
"""
import pathlib

import numpy as np
import pytest

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"


def _cases(npz):
    names = sorted({k.split("/")[0] for k in npz.files})
    for name in names:
        K, N, bs, M = (int(v) for v in npz[f"{name}/attrs"])
        zp = npz[f"{name}/zero_points"] if f"{name}/zero_points" in npz.files else None
        yield name, K, N, bs, M, npz[f"{name}/A"], npz[f"{name}/B"], npz[f"{name}/scales"], zp


# ---- nibble order ---------------------------------------------------------

def test_nibble_order_all_bytes(orc):
    """Low nibble is element 0 (integer_gemm_vnni.cc:60-65), for every byte value."""
    L = orc.lib()
    for b in range(256):
        buf = np.array([b], np.uint8)
        assert L.mnbo_nibble(buf.ctypes.data, 0) == (b & 0xF)
        assert L.mnbo_nibble(buf.ctypes.data, 1) == (b >> 4)


def test_dequantize_layout_brute_force(orc):
    """W[n, k] against per-element decoding of the [N, nb, bs/2] layout."""
    K, N, bs = 40, 3, 16  # nb = 3, K tail of 8 inside the last block, odd nb
    rng = np.random.default_rng(1)
    nb = 3
    B = rng.integers(0, 256, (N, nb, bs // 2), dtype=np.uint8)
    S = rng.uniform(0.1, 1, (N, nb)).astype(np.float32)
    Z = rng.integers(0, 256, (N, 2), dtype=np.uint8)
    W = orc.dequantize(B, S, Z, K, N, bs)
    for n in range(N):
        for k in range(K):
            b, j = divmod(k, bs)
            byte = int(B[n, b, j // 2])
            q = byte & 0xF if j % 2 == 0 else byte >> 4
            zb = int(Z[n, b // 2])
            z = zb & 0xF if b % 2 == 0 else zb >> 4
            assert W[n, k] == np.float32(q - z) * S[n, b]


# ---- golden fixtures from the reference's own code ------------------------

def test_ref_order_matches_reference_engine_bit_exact(orc):
    """The reference-order fp32 mode equals MatMulPlan<float>/GemmSkinnyM output."""
    d = np.load(GOLDEN / "ref_matmul.npz")
    n_cases = 0
    for name, K, N, bs, M, A, B, S, Z in _cases(d):
        assert int(d[f"{name}/gemm_algorithm"]) == 2  # GemmAlgorithm::kSkinnyM
        y = orc.matmul_nbits_ref_f32(A, B, S, Z, K, N, bs, threads=1)
        np.testing.assert_array_equal(y, d[f"{name}/Y_reference_engine"], err_msg=name)
        n_cases += 1
    assert n_cases == 6


def test_fp64_oracle_within_summation_bound_of_reference_engine(orc):
    """|y_ref - y64| <= (K+1) u sum|a||w| (recursive fp32 summation, u = 2^-24)."""
    d = np.load(GOLDEN / "ref_matmul.npz")
    for name, K, N, bs, M, A, B, S, Z in _cases(d):
        y64 = orc.matmul_nbits_f64(A, B, S, Z, K, N, bs)
        bound = (K + 1) * 2.0 ** -24 * orc.abs_dot_f64(A, B, S, Z, K, N, bs)
        err = np.abs(d[f"{name}/Y_reference_engine"].astype(np.float64) - y64)
        assert np.all(err <= bound), name


def test_integer_cases_match_reference_int4_gemm_exactly(orc):
    """Integer-valued MatMulNBits == IntegerMatMul4Bit2D with per-column zero points."""
    d = np.load(GOLDEN / "int4_kat.npz")
    for name, K, N, bs, M, A, B, S, Z in _cases(d):
        y64 = orc.matmul_nbits_f64(A, B, S, Z, K, N, bs)
        np.testing.assert_array_equal(y64, d[f"{name}/C_reference_int4"].astype(np.float64),
                                      err_msg=name)
        y32 = orc.matmul_nbits_ref_f32(A, B, S, Z, K, N, bs)
        np.testing.assert_array_equal(y32.astype(np.float64), y64, err_msg=name)
        yf = orc.matmul_nbits_fused_f32(A, B, S, Z, K, N, bs)
        np.testing.assert_array_equal(yf.astype(np.float64), y64, err_msg=name)


def test_f16_conversion_matches_reference_and_numpy(orc):
    d = np.load(GOLDEN / "f16.npz")
    x = d["x"]
    bits = orc.f32_to_f16_bits(x)
    np.testing.assert_array_equal(bits, d["bits_reference"])
    # numpy's float16 cast is an independent round-to-nearest-even implementation
    with np.errstate(over="ignore"):
        np.testing.assert_array_equal(bits, x.astype(np.float16).view(np.uint16))
    back = orc.f16_bits_to_f32(bits)
    finite = np.isfinite(back)
    np.testing.assert_array_equal(back[finite],
                                  bits[finite].view(np.float16).astype(np.float32))


def test_every_f16_bit_pattern_round_trips(orc):
    h = np.arange(0x10000, dtype=np.uint32).astype(np.uint16)
    f = orc.f16_bits_to_f32(h)
    ok = ~np.isnan(f)
    np.testing.assert_array_equal(f[ok], h[ok].view(np.float16).astype(np.float32))
    np.testing.assert_array_equal(orc.f32_to_f16_bits(f[ok]), h[ok])


# ---- live reference build, where present -----------------------------------

def test_reference_int4_known_answers(ref_lib):
    """The reference's own IntegerPacked4Bit tests (test_integer_gemm_vnni.cc:354-380),
    run on the reference build: junk high nibbles ignored, modulo-2^32 correction."""
    a = np.array([0x32, 0xF4], np.uint8)  # {2, 3, 4}, unused high nibble 0xF
    b = np.array([0x65, 0x87], np.uint8)  # {5, 6, 7}, unused high nibble 0x8
    c = ref_lib.ref_int4_matmul(a, False, b, False, 1, 1, 3, [0], [0])
    assert int(c[0, 0]) == 2 * 5 + 3 * 6 + 4 * 7
    packed = np.array([0xA0], np.uint8)
    c = ref_lib.ref_int4_matmul(packed, False, packed, False, 1, 1, 1, [-2000000000],
                                [-2000000000])
    assert int(c[0, 0]) & 0xFFFFFFFF == (2000000000 * 2000000000) & 0xFFFFFFFF


def test_ref_order_matches_live_reference_engine(orc, ref_lib):
    rng = np.random.default_rng(3)
    for K, N, bs, M in ((256, 130, 32, 1), (1024, 70, 128, 3), (96, 200, 32, 2)):
        nb = (K + bs - 1) // bs
        B = rng.integers(0, 256, (N, nb, bs // 2), dtype=np.uint8)
        S = rng.uniform(0.005, 0.02, (N, nb)).astype(np.float32)
        Z = rng.integers(0, 256, (N, (nb + 1) // 2), dtype=np.uint8)
        A = rng.standard_normal((M, K)).astype(np.float32)
        y_ref, algo = ref_lib.ref_matmul_f32(A, orc.dequantize(B, S, Z, K, N, bs))
        assert algo == 2
        np.testing.assert_array_equal(orc.matmul_nbits_ref_f32(A, B, S, Z, K, N, bs), y_ref)


# ---- brute force, closed forms, invariants ---------------------------------

def test_fp64_oracle_brute_force_tiny(orc):
    rng = np.random.default_rng(11)
    for K, N, bs, M, has_zp in ((5, 2, 16, 2, True), (33, 3, 32, 1, False), (64, 2, 16, 3, True)):
        nb = (K + bs - 1) // bs
        B = rng.integers(0, 256, (N, nb, bs // 2), dtype=np.uint8)
        S = rng.uniform(0.1, 2, (N, nb)).astype(np.float32)
        Z = rng.integers(0, 256, (N, (nb + 1) // 2), dtype=np.uint8) if has_zp else None
        A = rng.standard_normal((M, K)).astype(np.float32)
        y = orc.matmul_nbits_f64(A, B, S, Z, K, N, bs)
        flat = B.reshape(N, -1)
        for m in range(M):
            for n in range(N):
                acc = 0.0
                for k in range(K):
                    byte = int(flat[n, k // 2])
                    q = (byte >> (4 * (k % 2))) & 0xF
                    blk = k // bs
                    if Z is None:
                        z = 8
                    else:
                        zb = int(Z[n, blk // 2])
                        z = (zb >> (4 * (blk % 2))) & 0xF
                    acc += float(A[m, k]) * (q - z) * float(S[n, blk])
                assert abs(y[m, n] - acc) <= 1e-12 * (1 + abs(acc))


def test_closed_forms(orc):
    K, N, bs = 256, 9, 64
    rng = np.random.default_rng(2)
    A = rng.standard_normal((3, K)).astype(np.float32)
    S = rng.uniform(0.1, 1, (N, 4)).astype(np.float32)
    # q == zp everywhere -> exactly 0 in every mode
    B = np.full((N, 4, 32), 0x99, np.uint8)
    Z = np.full((N, 2), 0x99, np.uint8)
    for f in (orc.matmul_nbits_f64, orc.matmul_nbits_ref_f32, orc.matmul_nbits_fused_f32):
        assert np.all(f(A, B, S, Z, K, N, bs) == 0)
    # absent zero points mean 8
    B8 = np.full((N, 4, 32), 0x88, np.uint8)
    assert np.all(orc.matmul_nbits_f64(A, B8, S, None, K, N, bs) == 0)
    # block_size == K is per-channel quantization: y = s * sum a (q - z)
    Bk = rng.integers(0, 256, (N, 1, K // 2), dtype=np.uint8)
    Sk = rng.uniform(0.1, 1, (N, 1)).astype(np.float32)
    Zk = rng.integers(0, 16, (N, 1), dtype=np.uint8)
    q = np.empty((N, K))
    q[:, 0::2] = Bk.reshape(N, -1) & 0xF
    q[:, 1::2] = Bk.reshape(N, -1) >> 4
    expect = (A.astype(np.float64) @ (q - Zk.astype(np.float64)).T) * Sk[:, 0].astype(np.float64)
    np.testing.assert_allclose(orc.matmul_nbits_f64(A, Bk, Sk, Zk, K, N, K), expect, rtol=1e-12,
                               atol=1e-12)


def test_invariants(orc):
    K, N, bs, M = 512, 31, 32, 5
    rng = np.random.default_rng(4)
    nb = K // bs
    B = rng.integers(0, 256, (N, nb, bs // 2), dtype=np.uint8)
    S = rng.uniform(0.005, 0.02, (N, nb)).astype(np.float32)
    Z = rng.integers(0, 256, (N, (nb + 1) // 2), dtype=np.uint8)
    A = rng.standard_normal((M, K)).astype(np.float32)
    y = orc.matmul_nbits_f64(A, B, S, Z, K, N, bs)
    # linearity: scaling A by 2 is exact
    np.testing.assert_array_equal(orc.matmul_nbits_f64(2 * A, B, S, Z, K, N, bs), 2 * y)
    # permuting weight rows permutes output columns
    perm = rng.permutation(N)
    np.testing.assert_array_equal(orc.matmul_nbits_f64(A, B[perm], S[perm], Z[perm], K, N, bs),
                                  y[:, perm])
    # rows of A are independent
    for m in range(M):
        np.testing.assert_array_equal(orc.matmul_nbits_f64(A[m:m + 1], B, S, Z, K, N, bs)[0],
                                      y[m])
    # the fp32 modes agree with fp64 to the fp32 summation bound
    scale = orc.abs_dot_f64(A, B, S, Z, K, N, bs)
    for f in (orc.matmul_nbits_ref_f32, orc.matmul_nbits_fused_f32):
        err = np.abs(f(A, B, S, Z, K, N, bs) - y)
        assert np.all(err <= K * 2.0 ** -24 * scale + 1e-30)
    # threading does not change results (contiguous column ranges, same order)
    np.testing.assert_array_equal(orc.matmul_nbits_ref_f32(A, B, S, Z, K, N, bs, threads=1),
                                  orc.matmul_nbits_ref_f32(A, B, S, Z, K, N, bs, threads=7))


def test_execution_block_count_cases(orc):
    """ExecutionBlockCount (impl/execution.h:72-94): grain 2^15 work units."""
    assert orc.execution_block_count(0, 1.0, 8) == 0
    assert orc.execution_block_count(100, 1.0, 1) == 1
    assert orc.execution_block_count(100, 1.0, 8) == 1          # 100 units < grain
    assert orc.execution_block_count(4, 2 ** 15, 8) == 4         # capped by total
    assert orc.execution_block_count(100, 2 ** 15, 8) == 8       # capped by threads
    assert orc.execution_block_count(100, 2 ** 14, 64) == 50     # capped by useful blocks
