"""Pins of the oracle functions that the whole-step goldens only exercise
indirectly: the attention KV store's binary16 rounding, CpuEngine's RoPE
tables, and the logistic functions of the linear-attention gates.

- q35o_attention_float_to_half (full_attention.cpp:18-46) against the
  reference build's attention_cache_store_f16 (scalar and auto-selected
  backends) on 2^20 seeded values and the subnormal, overflow, infinity, NaN
  and halfway edges, and against IEEE round-to-nearest-even (numpy) for every
  finite value;
- q35o_rope_tables (cpu_engine.inl:339-352) against the FP64 closed form
  cos/sin(p * theta^(-2i / rope_dim)), exactly at p = 0 and for i = 0 (an
  integer angle), and the theta / exponent it uses against the geometric
  ratio between neighbouring frequencies;
- q35o_sigmoid / q35o_softplus (weights.inl:656-678) against FP64 closed
  forms over their whole range, including both sides of the branch points.
"""
import numpy as np
import pytest


def edge_values():
    v = [0.0, -0.0, np.inf, -np.inf, 65504.0, 65519.99, 65520.0, -65520.0, 1e10, 6.1035156e-05, 6.0e-05,
         5.9604645e-08, 2.9802322e-08, 2.9802326e-08, 1e-9, -1e-7, 1.0, 1.0009766, 1.00048828125, 1.00146484375,
         2049.0, 2051.0, 3.0517578e-05]
    bits = [0x7fc00000, 0x7f800001, 0xffc00000, 0x7fffffff, 0x7fa00000, 0x00000001, 0x807fffff, 0x38800000,
            0x387fffff, 0x33000000, 0x33000001, 0x477fe000, 0x477fefff, 0x477ff000]
    return np.concatenate([np.array(v, np.float32), np.array(bits, np.uint32).view(np.float32)])


def seeded_values():
    rng = np.random.default_rng(20)
    n = 1 << 20
    out = np.empty(n, np.float32)
    out[: n // 2] = rng.standard_normal(n // 2).astype(np.float32) * np.float32(
        2.0) ** rng.integers(-30, 20, n // 2).astype(np.float32)
    # arbitrary bit patterns, NaNs included
    out[n // 2:] = rng.integers(0, 1 << 32, n - n // 2, dtype=np.uint64).astype(np.uint32).view(np.float32)
    return out


def test_attention_float_to_half_matches_reference_and_ieee(orc):
    x = np.concatenate([seeded_values(), edge_values()])
    got = orc.f16_bits(x)
    finite = np.isfinite(x)
    # IEEE binary16 round-to-nearest-even for every finite value (overflow to inf)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(got[finite], want[finite])
    # infinities keep their sign; every NaN becomes the quiet NaN of its sign
    inf = np.isinf(x)
    np.testing.assert_array_equal(got[inf], np.where(x[inf] > 0, 0x7c00, 0xfc00).astype(np.uint16))
    nan = np.isnan(x)
    sign = (x[nan].view(np.uint32) >> 16) & 0x8000
    np.testing.assert_array_equal(got[nan], (sign | 0x7e00).astype(np.uint16))
    if not orc.ref_available():
        pytest.skip("reference build (oracle/_ref) not present")
    r = orc.ref()
    for backend in (1, 0):  # Q8_0Backend::scalar, auto_select
        out = np.zeros(x.size, np.uint16)
        r.ref_attention_cache_store_f16(orc.ptr(x), orc.ptr(out), x.size, backend)
        sel = np.ones(x.size, bool) if backend == 1 else ~nan  # SIMD converts keep NaN payloads
        np.testing.assert_array_equal(got[sel], out[sel], err_msg=f"backend {backend}")


@pytest.mark.parametrize("theta,rope_dim", [(10000000.0, 64), (10000.0, 32), (1000000.0, 128)])
def test_rope_tables_closed_form(orc, theta, rope_dim):
    positions = 8200
    cs, sn = orc.rope_tables(theta, rope_dim, positions)
    half = rope_dim // 2
    p = np.arange(positions, dtype=np.float64)[:, None]
    i = np.arange(half, dtype=np.float64)[None, :]
    angle = p * np.power(float(theta), -2.0 * i / rope_dim)
    # the FP32 angle carries the rounding of theta^x (1 ulp) times p: bound
    # the table by it (|d cos| <= |d angle|)
    tol = 4 * np.finfo(np.float32).eps * np.maximum(angle, 1.0)
    assert np.all(np.abs(cs - np.cos(angle)) <= tol)
    assert np.all(np.abs(sn - np.sin(angle)) <= tol)
    # position 0: angle 0 exactly; frequency 0: the angle is the position itself
    np.testing.assert_array_equal(cs[0], np.ones(half, np.float32))
    np.testing.assert_array_equal(sn[0], np.zeros(half, np.float32))
    np.testing.assert_allclose(cs[:, 0], np.cos(np.arange(positions, dtype=np.float64)), atol=2e-7)
    # neighbouring frequencies differ by theta^(-2 / rope_dim): read the
    # inverse frequencies off position 1 (angle = inv_freq, small enough for asin)
    inv = np.arcsin(sn[1].astype(np.float64))
    ok = inv < 1.0
    ratio = inv[1:][ok[1:]] / inv[:-1][ok[1:]]
    np.testing.assert_allclose(ratio, theta ** (-2.0 / rope_dim), rtol=1e-5)


def test_sigmoid_softplus_fp64(orc):
    xs = np.concatenate([np.linspace(-60, 60, 24001), [-20.0001, -20.0, -19.9999, 19.9999, 20.0, 20.0001, 0.0, -0.0,
                                                        1e-8, -1e-8, 88.0, -87.0, -103.0]]).astype(np.float32)
    sig = np.array([orc.lib.q35o_sigmoid(float(v)) for v in xs], np.float64)
    sp = np.array([orc.lib.q35o_softplus(float(v)) for v in xs], np.float64)
    x = xs.astype(np.float64)
    sig_ref = np.where(x >= 0, 1.0 / (1.0 + np.exp(-x)), np.exp(x) / (1.0 + np.exp(x)))
    sp_ref = np.logaddexp(0.0, x)
    np.testing.assert_allclose(sig, sig_ref, rtol=4e-7, atol=1e-45)
    # softplus: the reference returns x above 20 and exp(x) below -20, exact
    # to FP32 there (the dropped terms are below half an ulp)
    np.testing.assert_allclose(sp, sp_ref, rtol=4e-7, atol=1e-45)
    assert np.all(sp[xs > 20] == xs[xs > 20])
    lo = xs < -20
    np.testing.assert_allclose(sp[lo], np.exp(x[lo]), rtol=2.0 ** -23, atol=1e-45)  # expf: within 1 ulp
