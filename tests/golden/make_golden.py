"""Writes the golden fixtures in this directory from the reference's own code.

Run in the build container, where oracle/_ref/libolc_ref.so was compiled from
the onnx-light-cpu sources (``make -C oracle ref``). The fixtures are data only:
seeded inputs plus the outputs of three reference functions.

* ``ref_matmul.npz`` -- MatMulNBits inputs and the reference fp32 engine's
  result on the dequantized weights: ``MatMulPlan<float>`` with ``trans_b``
  (onnx_light_cpu/impl/math/gemm/gemm_plan.h:161-195), which runs GemmSkinnyM
  (impl/math/gemm_kernel.cc:1208-1258) for these shapes. The dequantization
  W = (q - zp) * scale is the operator's definition, one fp32 rounding.
* ``int4_kat.npz`` -- integer-valued MatMulNBits cases (A integers in [-8, 7],
  scales 1, one block per row) and the exact int32 result of the reference's
  packed-4-bit GEMM ``IntegerMatMul4Bit2D`` (vnni/integer_gemm_vnni.h:52-55)
  with per-column zero points: the same sum computed by independent code.
* ``f16.npz`` -- fp32 values around every rounding boundary and the
  reference's ``FloatToFloat16Bits`` (impl/math/half_conversion.h:42-78).

Usage: python tests/golden/make_golden.py
"""
import pathlib
import sys

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))

import __graft_entry__  # noqa: E402

orc = __graft_entry__.load_oracle()
pkg = __graft_entry__.load_package()
W = pkg.workloads

# (name, K, N, block_size, zero points, M, sigma)
MATMUL_CASES = [
    ("k64_n7_bs32_zp_m1", 64, 7, 32, True, 1, 1.0),
    ("k96_n65_bs32_nozp_m3", 96, 65, 32, False, 3, 1.0),
    ("k256_n40_bs64_zp_m2", 256, 40, 64, True, 2, 0.5),
    ("k100_n33_bs16_zp_m1", 100, 33, 16, True, 1, 1.0),   # K tail inside the last block
    ("k512_n24_bs128_zp_m4", 512, 24, 128, True, 4, 1.0),
    ("k384_n16_bs128_nozp_m1", 384, 16, 128, False, 1, 2.0),  # odd block count: junk zp nibble
]


def pack_nibbles(q):
    """Packs integer nibbles [..., 2n] low-first; an odd tail gets 0xA in the unused nibble."""
    q = np.asarray(q, dtype=np.uint8)
    if q.shape[-1] % 2:
        q = np.concatenate([q, np.full(q.shape[:-1] + (1,), 0xA, np.uint8)], axis=-1)
    return (q[..., 0::2] & 0xF) | ((q[..., 1::2] & 0xF) << 4)


def make_matmul():
    out = {}
    for i, (name, K, N, bs, zp, M, sigma) in enumerate(MATMUL_CASES):
        p = W.Projection(name, K, N, bs, zp, sigma)
        B, S, Z = W.make_weights(p, 1000 + i)
        A = W.make_activations(M, K, sigma, 2000 + i)
        Wd = orc.dequantize(B, S, Z, K, N, bs)
        Y, algo = orc.ref_matmul_f32(A, Wd)
        out[f"{name}/A"] = A
        out[f"{name}/B"] = B
        out[f"{name}/scales"] = S
        if Z is not None:
            out[f"{name}/zero_points"] = Z
        out[f"{name}/attrs"] = np.array([K, N, bs, M], np.int64)
        out[f"{name}/Y_reference_engine"] = Y
        out[f"{name}/gemm_algorithm"] = np.array(algo, np.int64)
    np.savez_compressed(HERE / "ref_matmul.npz", **out)


def make_int4_kat():
    rng = np.random.default_rng(77)
    out = {}
    for i, (K, N, M) in enumerate([(17, 5, 1), (64, 9, 3), (65, 4, 2), (128, 33, 2)]):
        a = rng.integers(-8, 8, size=(M, K))
        q = rng.integers(0, 16, size=(N, K))
        zp = rng.integers(0, 16, size=N)
        # MatMulNBits operands: one block of K per row (block_size padded to K rounded up
        # to an even power of two), scales 1, zero point nibble per row.
        bs = 16
        while bs < K:
            bs *= 2
        qpad = np.concatenate([q, np.zeros((N, bs - K), np.int64)], axis=1)
        B = pack_nibbles(qpad).reshape(N, 1, bs // 2)
        Z = pack_nibbles(zp.reshape(N, 1)).reshape(N, 1)
        S = np.ones((N, 1), np.float32)
        # Reference: A packed signed [M, K], B^T packed unsigned [K, N], per-column zp.
        a_packed = pack_nibbles((a & 0xF).reshape(-1))
        bt_packed = pack_nibbles(q.T.reshape(-1))
        C = orc.ref_int4_matmul(a_packed, True, bt_packed, False, M, N, K, [0],
                                zp.astype(np.int32))
        tag = f"k{K}_n{N}_m{M}"
        out[f"{tag}/A"] = a.astype(np.float32)
        out[f"{tag}/B"] = B
        out[f"{tag}/scales"] = S
        out[f"{tag}/zero_points"] = Z
        out[f"{tag}/attrs"] = np.array([K, N, bs, M], np.int64)
        out[f"{tag}/C_reference_int4"] = C
    np.savez_compressed(HERE / "int4_kat.npz", **out)


def make_f16():
    vals = [0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, 1e6, -1e6, np.inf, -np.inf,
            2.0 ** -14, 2.0 ** -24, 2.0 ** -25, 1.5 * 2.0 ** -25, 2.0 ** -26, 3 * 2.0 ** -25,
            6.1e-5, 5.96e-8, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 1.0 + 2.0 ** -12]
    rng = np.random.default_rng(5)
    scaled = (rng.standard_normal(2000) * 10 ** rng.uniform(-9, 5, 2000)).astype(np.float32)
    raw = rng.integers(0, 2 ** 32, 2000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    x = np.concatenate([np.array(vals, np.float32), scaled, raw])
    x = x[~np.isnan(x)]
    np.savez_compressed(HERE / "f16.npz", x=x, bits_reference=orc.ref_f32_to_f16_bits(x))


if __name__ == "__main__":
    if not orc.ref_available():
        sys.exit("oracle/_ref/libolc_ref.so is not built (make -C oracle ref)")
    make_matmul()
    make_int4_kat()
    make_f16()
    for f in sorted(HERE.glob("*.npz")):
        print(f.name, f.stat().st_size, "bytes")
