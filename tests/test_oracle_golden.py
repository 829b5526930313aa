"""The CPU oracle against the golden vectors the reference build wrote
(tests/golden/make_golden.py). Integer and byte outputs bit-exact; the DOT4
FP32 projections bit-exact (same fma chain as the reference's avx2 path);
FP32 kernels within 1e-5 relative (the reference SIMD paths reorder sums)."""
import os

import numpy as np
import pytest

with np.load(os.path.join(os.path.dirname(__file__), "golden", "kernels.npz")) as _f:
    G = {k: np.ascontiguousarray(_f[k]) for k in _f.files}


def rel(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - b)) / max(np.max(np.abs(b)), 1e-30))


def test_h128_basis_known_answer(orc):
    """tests/q4_quantizer_test.cpp:12-19: H128 of x_i = (i - 64)/32, block 0, default seed."""
    x = (np.arange(128) - 64) * 0.03125
    y = orc.h128_transform(x.astype(np.float32))
    np.testing.assert_allclose(y, G["h128_basis_fixture"], atol=1e-6)


def test_half_conversion(orc):
    got = np.array([orc.lib.q35o_float_to_half(float(v)) for v in G["half_in"]], np.uint16)
    assert np.array_equal(got, G["half_out"])


def test_q8_quantizers(orc):
    x = G["q8_in"]
    x4 = orc.q8_quantize_4(x)
    for f in ("qs", "sums"):
        assert np.array_equal(x4[f], G["q8_x4"][f])
    assert np.array_equal(x4["scales"].view(np.uint32), G["q8_x4"]["scales"].view(np.uint32))
    x1 = orc.q8_quantize_1(x[3])
    assert np.array_equal(x1["qs"], G["q8_x1"]["qs"]) and np.array_equal(x1["sums"], G["q8_x1"]["sums"])


def test_h128_prepare(orc):
    h4 = orc.h128_prepare_4(G["h128_in"])
    for f in ("qs", "sums"):
        assert np.array_equal(h4[f], G["h128_x4"][f])
    assert np.array_equal(h4["scales"].view(np.uint32), G["h128_x4"]["scales"].view(np.uint32))
    h1 = orc.h128_prepare_1(G["h128_in"][5])
    assert np.array_equal(h1["qs"], G["h128_x1"]["qs"])
    assert np.array_equal(h1["scales"].view(np.uint32), G["h128_x1"]["scales"].view(np.uint32))


def test_dot4_pack_and_projections(orc):
    rows, blocks = 64, 32
    packed = orc.dot4_pack(G["dot4_canon"], rows, blocks)
    assert np.array_equal(packed.view(np.uint8), G["dot4_packed"].view(np.uint8))
    mm = orc.dot4_matmul(packed, G["h128_x4"], rows, 8, blocks)
    assert np.array_equal(mm.view(np.uint32), G["dot4_matmul"].view(np.uint32))
    mv = orc.dot4_matvec(packed, G["h128_x1"], rows, blocks)
    assert np.array_equal(mv.view(np.uint32), G["dot4_matvec"].view(np.uint32))
    import ctypes
    val, idx = ctypes.c_float(), ctypes.c_size_t()
    counts = np.ascontiguousarray(G["dot4_counts"], np.int32)
    orc.lib.q35o_dot4_argmax(orc.ptr(packed), orc.ptr(G["h128_x1"]), orc.ptr(counts), 1.3, 0, rows, blocks,
                             ctypes.byref(val), ctypes.byref(idx))
    assert idx.value == int(G["dot4_argmax"][0])
    assert np.float32(val.value) == G["dot4_argmax_value"][0]


def test_delta_rows(orc):
    st, out = orc.delta_rows(G["delta_state"].reshape(-1), G["delta_q"], G["delta_k"], G["delta_v"],
                             G["delta_alpha"], G["delta_beta"], 128, 128)
    assert rel(st, G["delta_state_out"].reshape(-1)) < 1e-5
    assert rel(out, G["delta_out"].reshape(-1)) < 1e-5


def test_attention_decode(orc):
    out = orc.attention_decode(G["attn_q"], G["attn_gate"], G["attn_keys"], G["attn_values"], 8, 2, 256)
    assert rel(out, G["attn_out"]) < 1e-5


def test_activation_ops(orc):
    x, w = G["act_x"], G["act_w"]
    rn = np.zeros_like(x)
    orc.lib.q35o_rms_norm(orc.ptr(x), orc.ptr(w), orc.ptr(rn), 4, 256, 1e-6, 1.0)
    assert rel(rn, G["rms_out"]) < 1e-5
    l2 = x.copy()
    orc.lib.q35o_l2_normalize(orc.ptr(l2), 4, 256, 1e-6, 0.0883883476)
    assert rel(l2, G["l2_out"]) < 1e-5
    sm = np.zeros(256, np.float32)
    orc.lib.q35o_silu_mul(orc.ptr(np.ascontiguousarray(x[0])), orc.ptr(np.ascontiguousarray(x[1])), orc.ptr(sm), 256)
    assert rel(sm, G["silu_mul_out"]) < 1e-5
    ch, kern = 256, 4
    km = np.ascontiguousarray(G["conv_w"])
    st = G["conv_state"].copy()
    out = np.zeros(ch, np.float32)
    orc.lib.q35o_conv1d_silu(orc.ptr(st), 2, orc.ptr(G["conv_x"]), orc.ptr(km), orc.ptr(out), ch, kern)
    assert rel(out, G["conv_out"]) < 1e-5
    assert np.array_equal(st, G["conv_state_out"])
    rp = np.ascontiguousarray(x[:2]).copy()
    orc.lib.q35o_rope(orc.ptr(rp), 2, 128, 64, orc.ptr(G["rope_cos"]), orc.ptr(G["rope_sin"]))
    assert rel(rp, G["rope_out"]) < 1e-5
