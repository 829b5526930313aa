"""Pins of the oracle's restatements for the optional artifact encodings:
Q4G16Tile (q4_g16.h, q4_g16.cpp, q4_g16_evex.cpp, q4_g16_avx2.cpp) and the
Q8_0 gate rows (q8_0_matmul with matrix scales, q8_0.cpp:160-193, as
run_q8_gate_tail calls it, weights.inl:1015-1034). Each is checked against
the reference build in oracle/_ref where it is built, and against closed
forms (dequantized float64 dot products, the packer's rounding bound)."""
import numpy as np
import pytest

from oracle import q35_oracle as orc

need_ref = pytest.mark.skipif(not orc.ref_available(), reason="oracle/_ref (the reference build) is not built here")
AUTO, SCALAR = 0, 1  # Q8_0Backend (q8_0.h:23-31)


def rand_g16(rng, rows, nb):
    t = np.zeros((rows // 8, nb), orc.G16)
    t["qs"] = rng.integers(0, 256, size=(rows // 8, nb, 128), dtype=np.uint8)
    t["d"] = rng.lognormal(0.0, 0.5, size=(rows // 8, nb, 2, 8)).astype(np.float16).view(np.uint16)
    return t


def g16_dense(t, rows, nb):
    return np.stack([orc.g16_dequantize_row(t, r, nb) for r in range(rows)]).astype(np.float64)


def test_g16_pack_rounding_bound():
    """Every weight dequantizes to within half a step of its own 16-column
    half's scale, and the largest magnitude of each half is exact up to the
    binary16 rounding of its scale: the nibble order and the d[half][row]
    placement both have to be right for that."""
    rng = np.random.default_rng(3)
    rows, cols = 24, 96
    w = rng.standard_normal((rows, cols)).astype(np.float32)
    t = orc.g16_pack(w)
    deq = g16_dense(t, rows, cols // 32)
    halves = np.abs(w.reshape(rows, cols // 16, 16)).max(axis=2)
    step = (halves / 7.0).astype(np.float16).astype(np.float64)
    bound = np.repeat(step, 16).reshape(rows, cols) * 0.5 + 1e-7
    assert np.all(np.abs(deq - w) <= bound + np.abs(w) * 2e-3)


def test_g16_matmul_closed_form():
    rng = np.random.default_rng(4)
    rows, nb, count = 40, 6, 5
    t = rand_g16(rng, rows, nb)
    x = rng.standard_normal((count, nb * 32)).astype(np.float32)
    act = orc.q8_quantize_1(x).reshape(count, nb)
    got = orc.g16_matmul(t, act, rows, count, nb)
    a = (act["qs"].astype(np.float64) * act["scales"].astype(np.float64)).reshape(count, nb * 32)
    want = a @ g16_dense(t, rows, nb).T
    mag = np.abs(a) @ np.abs(g16_dense(t, rows, nb)).T
    assert np.all(np.abs(got - want) <= 1e-5 * mag + 1e-6)


@need_ref
def test_g16_dequant_matches_reference():
    rng = np.random.default_rng(5)
    rows, nb = 16, 4
    t = rand_g16(rng, rows, nb)
    r = orc.ref()
    for row in range(rows):
        want = np.zeros(nb * 32, np.float32)
        r.ref_q4_g16_dequantize_row(orc.ptr(t), row, orc.ptr(want), nb)
        assert np.array_equal(orc.g16_dequantize_row(t, row, nb), want)


@need_ref
@pytest.mark.parametrize("count", [1, 3, 16, 21])
def test_g16_matmul_matches_reference(count):
    """The SIMD paths (AVX2 matvec, AVX-512 VNNI wide tiles) use the same fma
    chain as the restatement: bit-identical. The scalar path rounds the
    product before the add, so it agrees to float rounding only."""
    rng = np.random.default_rng(6 + count)
    rows, nb = 64, 8
    t = rand_g16(rng, rows, nb)
    x = rng.standard_normal((count, nb * 32)).astype(np.float32)
    act = orc.q8_quantize_1(x)
    got = orc.g16_matmul(t, act, rows, count, nb)
    r = orc.ref()
    for backend in (AUTO, SCALAR):
        want = np.zeros((count, rows), np.float32)
        if count == 1:
            r.ref_q4_g16_matvec(orc.ptr(t), orc.ptr(act), orc.ptr(want), rows, nb, backend)
        else:
            packed = np.zeros(((count + 15) // 16) * nb * 640, np.uint8)
            r.ref_q4_g16_pack_activations(orc.ptr(act), orc.ptr(packed), count, nb)
            r.ref_q4_g16_matmul(orc.ptr(t), orc.ptr(packed), orc.ptr(want), rows, count, nb, rows, backend)
        if backend == AUTO and r.ref_backend_resolve(AUTO) != SCALAR:
            assert np.array_equal(got, want), (backend, np.abs(got - want).max())
        else:
            np.testing.assert_allclose(got, want, rtol=1e-5, atol=2e-6 * np.abs(want).max())


@need_ref
@pytest.mark.parametrize("count", [1, 4, 7])
def test_q8_rows_match_reference(count):
    rng = np.random.default_rng(20 + count)
    rows, cols = 32, 256
    w = (rng.standard_normal((rows, cols)) * 0.05).astype(np.float32)
    blocks8, mscales = orc.q8_rows_pack(w)
    x = rng.standard_normal((count, cols)).astype(np.float32)
    act = orc.q8_quantize_1(x)
    got = orc.q8_matmul(blocks8, mscales, act, rows, count, cols // 32)
    # the reference takes Q8_0 activation blocks: the same codes and binary16 scale
    v8, _ = orc.q8_rows_pack(x)
    r = orc.ref()
    want = np.zeros((count, rows), np.float32)
    r.ref_q8_0_matmul(orc.ptr(blocks8), orc.ptr(v8), orc.ptr(want), rows, count, cols // 32, rows, AUTO,
                      orc.ptr(mscales))
    np.testing.assert_allclose(got, want, rtol=2e-6, atol=1e-6)
    # closed form over the dequantized rows
    wd = blocks8["qs"].astype(np.float64) * mscales[..., None]
    ad = act["qs"].reshape(count, -1, 32).astype(np.float64) * act["scales"].reshape(count, -1, 1)
    dense = np.einsum("tbi,rbi->tr", ad, wd)
    assert np.all(np.abs(got - dense) <= 1e-5 * np.abs(dense).max() + 1e-6)
