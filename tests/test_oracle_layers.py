"""The oracle's layer steps against the reference's own layer composition.

q35o_linear_attention_row and q35o_full_attention_row (oracle/q35_oracle.c,
the restated linear_step / full_step the whole oracle step runs) are checked
against run_linear_attention_step and prepare_full_attention_row +
run_full_attention_step themselves (src/runtime/layers.inl:36-395), built from
the reference's sources into oracle/_ref/libq35ref_layers.so the way the
reference's tests/head_runtime_test.cpp builds its runtime tests. Both run
from the same projected rows (return_core), over chained steps, so the conv
ring, the recurrent state and the KV rows are compared too.

With the scalar backend every fp32 order matches except the reference's
per-head RMSNorm and L2 norm helpers, which always take the auto-selected
kernels (weights.inl:1544-1566): the tolerance is a few ulp (1e-5 relative
to each vector's scale), not a block-flip envelope. The V rows are binary16
and must match bit for bit; the K rows pass through that norm, so a handful
of their elements may round one binary16 ulp apart. A planted mistake in the oracle side of the
comparison (the q scale, the GQA head order, the RoPE rows) fails it."""
import ctypes
import os

import numpy as np
import pytest

from oracle import q35_oracle as orc

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LAYERS_SO = os.path.join(ROOT, "oracle", "_ref", "libq35ref_layers.so")
P = ctypes.c_void_p
SCALAR = 1  # Q8_0Backend::scalar (q8_0.h:23-31)


@pytest.fixture(scope="module")
def refl():
    if not os.path.exists(LAYERS_SO):
        pytest.skip("oracle/_ref/libq35ref_layers.so is built by __graft_entry__.build() next to the reference")
    r = ctypes.CDLL(LAYERS_SO)
    r.refl_linear_attention_row.restype = ctypes.c_int
    r.refl_linear_attention_row.argtypes = [ctypes.c_int] * 6 + [ctypes.c_float] + [P] * 5 + [
        ctypes.POINTER(ctypes.c_size_t), P, P, P, ctypes.c_char_p, ctypes.c_size_t]
    r.refl_full_attention_row.restype = ctypes.c_int
    r.refl_full_attention_row.argtypes = [ctypes.c_int] * 5 + [ctypes.c_float] + [P] * 4 + [
        ctypes.c_size_t, ctypes.c_int, P, P, P, P, ctypes.c_char_p, ctypes.c_size_t]
    return r


def ptr(a):
    return a.ctypes.data_as(P)


def close(got, want, what, tol=1e-5):
    scale = max(1e-30, float(np.abs(want).max()))
    err = float(np.abs(got.astype(np.float64) - want.astype(np.float64)).max()) / scale
    assert err <= tol, f"{what}: max error {err:.3g} of the vector's scale"


def dims(k_heads=4, v_heads=4, heads=4, kv_heads=2):
    return orc.dims_from(dict(n_layers=1, hidden=256, intermediate=256, vocab=64, n_heads=heads, n_kv_heads=kv_heads,
                              head_dim=256, rope_dim=64, rope_theta=10000000.0, rms_eps=1e-6, lin_kernel=4,
                              lin_k_heads=k_heads, lin_v_heads=v_heads, lin_k_dim=128, lin_v_dim=128,
                              sign_seed=orc.SIGN_SEED))


def run_linear(refl, d, steps, seed, backend, mutate=None):
    rng = np.random.default_rng(seed)
    q_dim, v_dim = d.lin_k_heads * d.lin_k_dim, d.lin_v_heads * d.lin_v_dim
    ch = 2 * q_dim + v_dim
    conv_w = (rng.standard_normal((ch, d.lin_kernel)) * 0.4).astype(np.float32)  # [channels][kernel]
    norm_w = (1.0 + rng.standard_normal(d.lin_v_dim) * 0.1).astype(np.float32)
    a_log = (rng.standard_normal(d.lin_v_heads) * 0.5).astype(np.float32)
    dt_bias = (rng.standard_normal(d.lin_v_heads) * 0.5).astype(np.float32)
    layer = orc.Layer()
    layer.is_linear = 1
    layer.conv_w, layer.lin_norm, layer.a_log, layer.dt_bias = ptr(conv_w), ptr(norm_w), ptr(a_log), ptr(dt_bias)
    km = np.ascontiguousarray(conv_w.T)  # pack_conv1d_kernel_major (weights.inl:532-544)
    o_conv = np.zeros((d.lin_kernel - 1) * ch, np.float32)
    r_conv = o_conv.copy()
    o_rec = (rng.standard_normal(d.lin_v_heads * d.lin_v_dim * d.lin_k_dim) * 0.02).astype(np.float32)
    r_rec = o_rec.copy()
    o_ring, r_ring = ctypes.c_size_t(0), ctypes.c_size_t(0)
    err = ctypes.create_string_buffer(256)
    for n in range(steps):
        proj = rng.standard_normal(ch + v_dim + 2 * d.lin_v_heads).astype(np.float32)
        o_core = np.zeros(v_dim, np.float32)
        r_core = np.zeros(v_dim, np.float32)
        o_in = mutate(proj, d) if mutate else proj
        assert orc.lib.q35o_linear_attention_row(ctypes.byref(d), ctypes.byref(layer), ptr(o_conv),
                                                 ctypes.byref(o_ring), ptr(o_rec), ptr(o_in), ptr(o_core)) == 0
        assert refl.refl_linear_attention_row(backend, d.lin_k_heads, d.lin_v_heads, d.lin_k_dim, d.lin_v_dim,
                                              d.lin_kernel, d.rms_eps, ptr(km), ptr(norm_w), ptr(dt_bias),
                                              ptr(a_log), ptr(r_conv), ctypes.byref(r_ring), ptr(r_rec), ptr(proj),
                                              ptr(r_core), err, 256) == 0, err.value
        close(o_core, r_core, f"linear core, step {n}")
        close(o_rec, r_rec, f"recurrent state, step {n}")
        np.testing.assert_array_equal(o_conv.view(np.uint32), r_conv.view(np.uint32), err_msg=f"conv ring, step {n}")
        assert o_ring.value == r_ring.value


@pytest.mark.parametrize("k_heads,v_heads", [(4, 4), (2, 4)])
@pytest.mark.parametrize("backend", [SCALAR, 0])
def test_linear_attention_row_matches_reference(refl, k_heads, v_heads, backend):
    """Six chained rows: conv ring, gates, L2 norms (q x 1/sqrt(128)), GQA
    repeat (2 key heads for 4 value heads), the delta rule, the gated
    RMSNorm and SiLU(z)."""
    run_linear(refl, dims(k_heads, v_heads), 6, seed=3 + k_heads, backend=backend)


def run_full(refl, d, steps, seed, backend, mutate=None):
    rng = np.random.default_rng(seed)
    hd, kvw = d.head_dim, d.n_kv_heads * d.head_dim
    q_norm = (rng.standard_normal(hd) * 0.1).astype(np.float32)
    k_norm = (rng.standard_normal(hd) * 0.1).astype(np.float32)
    layer = orc.Layer()
    layer.is_linear = 0
    layer.q_norm, layer.k_norm = ptr(q_norm), ptr(k_norm)
    cs, sn = orc.rope_tables(d.rope_theta, d.rope_dim, steps)
    o_k = np.zeros((steps, kvw), np.uint16)
    o_v = np.zeros_like(o_k)
    r_k, r_v = o_k.copy(), o_v.copy()
    err = ctypes.create_string_buffer(256)
    for pos in range(steps):
        proj = rng.standard_normal((d.n_heads + d.n_kv_heads) * hd * 2).astype(np.float32)
        o_core = np.zeros(d.n_heads * hd, np.float32)
        r_core = np.zeros_like(o_core)
        o_in = mutate(proj, d) if mutate else proj
        assert orc.lib.q35o_full_attention_row(ctypes.byref(d), ctypes.byref(layer), ptr(o_k), ptr(o_v), pos,
                                               ptr(cs[pos]), ptr(sn[pos]), ptr(o_in), ptr(o_core)) == 0
        assert refl.refl_full_attention_row(backend, d.n_heads, d.n_kv_heads, hd, d.rope_dim, d.rms_eps,
                                            ptr(q_norm), ptr(k_norm), ptr(r_k), ptr(r_v), steps, pos,
                                            ptr(cs[pos]), ptr(sn[pos]), ptr(proj), ptr(r_core), err, 256) == 0, \
            err.value
        # K passes the reference's auto-kernel RMSNorm first: one binary16 ulp
        ulp = np.abs(o_k[pos].astype(np.int32) - r_k[pos].astype(np.int32))
        assert ulp.max() <= 1 and (ulp > 0).sum() <= 4, f"K row {pos}: {int((ulp > 0).sum())} elements differ"
        np.testing.assert_array_equal(o_v[pos], r_v[pos], err_msg=f"V row {pos}")
        # a flipped K element moves its scores by ~2^-11 of q.k: looser only then
        close(o_core, r_core, f"attention core, position {pos}", 1e-5 if ulp.max() == 0 else 1e-4)
        o_k[pos] = r_k[pos]  # both caches hold the same history for the next position


@pytest.mark.parametrize("heads,kv_heads", [(4, 2), (8, 2)])
@pytest.mark.parametrize("backend", [SCALAR, 0])
def test_full_attention_row_matches_reference(refl, heads, kv_heads, backend):
    """Seven positions: q/gate de-interleave, q/k RMSNorm (1 + w), split-half
    RoPE on the first 64 dims, the binary16 K/V append and the sigmoid-gated
    GQA attention over every cached row."""
    run_full(refl, dims(heads=heads, kv_heads=kv_heads), 7, seed=11 + heads, backend=backend)


def test_planted_mistakes_fail(refl):
    """The comparison has teeth: inputs altered the way a dropped term or a
    transposed operand would alter them fail it."""
    def swap_kv_heads(proj, d):  # the two K heads exchanged
        p = proj.copy()
        hd = d.head_dim
        k0 = d.n_heads * hd * 2
        p[k0:k0 + hd], p[k0 + hd:k0 + 2 * hd] = proj[k0 + hd:k0 + 2 * hd].copy(), proj[k0:k0 + hd].copy()
        return p

    def scale_beta(proj, d):  # the b gate row of the first value head altered
        p = proj.copy()
        q_dim, v_dim = d.lin_k_heads * d.lin_k_dim, d.lin_v_heads * d.lin_v_dim
        p[2 * q_dim + v_dim + v_dim] += 0.5
        return p

    with pytest.raises(AssertionError):
        run_full(refl, dims(heads=4, kv_heads=2), 3, seed=5, backend=SCALAR, mutate=swap_kv_heads)
    with pytest.raises(AssertionError):
        run_linear(refl, dims(4, 4), 2, seed=5, backend=SCALAR, mutate=scale_beta)
