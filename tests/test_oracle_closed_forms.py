"""Closed-form and brute-force pins of the CPU oracle, independent of the
reference build: Sylvester Hadamard with independently derived sign words,
bijections, FP64 recomputation, quantizer invariants, ring-buffer semantics,
split-K merge identity, and batched == unbatched for the whole step."""
import numpy as np
import pytest

MASK = (1 << 64) - 1


def splitmix(x):
    x = (x + 0x9e3779b97f4a7c15) & MASK
    x = ((x ^ (x >> 30)) * 0xbf58476d1ce4e5b9) & MASK
    x = ((x ^ (x >> 27)) * 0x94d049bb133111eb) & MASK
    return x ^ (x >> 31)


def signs(block, seed):
    out = []
    for w in range(2):
        s = splitmix((seed + block * 0x9e3779b97f4a7c15 + w * 0xd1b54a32d192ed03) & MASK)
        out += [-1.0 if (s >> b) & 1 else 1.0 for b in range(64)]
    return np.array(out)


def sylvester(n):
    h = np.array([[1.0]])
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    return h


@pytest.mark.parametrize("block", [0, 1, 27])
def test_h128_is_sylvester_times_signs(orc, block):
    h = sylvester(128)
    d = signs(block, orc.SIGN_SEED)
    r = np.stack([orc.h128_transform(np.eye(128, dtype=np.float32)[i], block) for i in range(128)], 1)
    want = (h * d[None, :]) * np.float64(np.float32(0.08838834764831844055))
    assert np.array_equal(r.astype(np.float64), want)
    np.testing.assert_allclose(r.astype(np.float64) @ r.T.astype(np.float64), np.eye(128), atol=1e-6)


def test_q8_quantizer_invariants(orc):
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(32 * 64) * rng.uniform(0.01, 10, 32 * 64)).astype(np.float32)
    x[:32] = 0
    q = orc.q8_quantize_1(x)
    for b in range(64):
        v = x[b * 32:(b + 1) * 32].astype(np.float64)
        codes = q["qs"][b].astype(np.int64)
        amax = np.abs(v).max()
        assert q["sums"][b] == codes.sum()
        if amax == 0:
            assert np.all(codes == 0) and q["scales"][b][0] == 0
            continue
        assert np.float16(np.float32(amax) / np.float32(127)) == np.float16(q["scales"][b][0])
        assert np.abs(codes).max() == 127 and np.all(np.abs(codes) <= 127)
        step = amax / 127
        assert np.all(np.abs(codes * step - v) <= 0.5 * step * (1 + 1e-6))


def test_dot4_bijection_and_dequant(orc):
    rng = np.random.default_rng(1)
    rows, blocks = 24, 5
    canon = orc.random_q4_blocks(rng, rows, blocks * 32)
    packed = orc.dot4_pack(canon, rows, blocks)
    assert np.array_equal(orc.dot4_unpack(packed, rows, blocks).view(np.uint8), canon.view(np.uint8))
    for row in (0, 13, 23):
        got = orc.dot4_dequantize_row(packed, row, blocks)
        lo = (canon["qs"][row] & 15).astype(np.float64) - 8
        hi = (canon["qs"][row] >> 4).astype(np.float64) - 8
        vals = np.concatenate([lo, hi], axis=1)  # GGML Q4_0: low nibbles are values 0..15
        want = vals * canon["d"][row].view(np.float16).astype(np.float64)[:, None]
        assert np.array_equal(got.astype(np.float64), want.reshape(-1))


def test_block_dots_and_matvec_fp64(orc):
    rng = np.random.default_rng(2)
    rows, blocks = 16, 7
    canon = orc.random_q4_blocks(rng, rows, blocks * 32)
    packed = orc.dot4_pack(canon, rows, blocks)
    x = rng.standard_normal(blocks * 32).astype(np.float32)
    act = orc.q8_quantize_1(x)
    codes = act["qs"].reshape(-1)
    dots = orc.dot4_block_dots(packed, codes, rows, blocks)
    w = np.stack([orc.dot4_dequantize_row(packed, r, blocks) for r in range(rows)])
    wint = np.concatenate([(canon["qs"] & 15).astype(np.int64) - 8, (canon["qs"] >> 4).astype(np.int64) - 8], axis=2)
    want = np.einsum("rbk,bk->rb", wint, codes.reshape(blocks, 32).astype(np.int64))
    assert np.array_equal(dots, want)
    mv = orc.dot4_matvec(packed, act, rows, blocks)
    full = (w.astype(np.float64).reshape(rows, blocks, 32) * (codes.reshape(blocks, 32) *
            act["scales"][:, 0, None].astype(np.float64))).sum((1, 2))
    np.testing.assert_allclose(mv, full, rtol=1e-5, atol=1e-5 * np.abs(full).max())


def test_delta_rule_outer_product_form(orc):
    rng = np.random.default_rng(3)
    h, d = 3, 128
    s = rng.standard_normal((h, d, d)) * 0.1
    q = rng.standard_normal((h, d)); k = rng.standard_normal((h, d)) * 0.1; v = rng.standard_normal((h, d))
    al = rng.uniform(0.2, 1, h); be = rng.uniform(0, 1, h)
    st, out = orc.delta_rows(s.astype(np.float32).reshape(-1), q.astype(np.float32), k.astype(np.float32),
                             v.astype(np.float32), al.astype(np.float32), be.astype(np.float32), d, d)
    s32 = s.astype(np.float32).astype(np.float64)
    q32, k32, v32 = (a.astype(np.float32).astype(np.float64) for a in (q, k, v))
    a32, b32 = al.astype(np.float32).astype(np.float64), be.astype(np.float32).astype(np.float64)
    dec = a32[:, None, None] * s32
    new = dec + b32[:, None, None] * np.einsum("hi,hj->hij", v32 - np.einsum("hij,hj->hi", dec, k32), k32)
    np.testing.assert_allclose(st.reshape(h, d, d), new, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(out.reshape(h, d), np.einsum("hij,hj->hi", new, q32), rtol=1e-4, atol=1e-5)


def _attn64(q, g, keys, vals, heads, kvh, hd):
    kf = keys.view(np.float16).astype(np.float64)
    vf = vals.view(np.float16).astype(np.float64)
    out = np.zeros(heads * hd)
    for h in range(heads):
        kv = h // (heads // kvh)
        s = kf[:, kv * hd:(kv + 1) * hd] @ q[h * hd:(h + 1) * hd] / np.sqrt(hd)
        p = np.exp(s - s.max())
        p /= p.sum()
        out[h * hd:(h + 1) * hd] = (p @ vf[:, kv * hd:(kv + 1) * hd]) / (1 + np.exp(-g[h * hd:(h + 1) * hd]))
    return out


def test_attention_fp64_and_split_merge(orc):
    rng = np.random.default_rng(4)
    heads, kvh, hd, seq = 4, 2, 256, 300
    keys = rng.standard_normal((seq, kvh * hd)).astype(np.float16).view(np.uint16)
    vals = rng.standard_normal((seq, kvh * hd)).astype(np.float16).view(np.uint16)
    q = rng.standard_normal(heads * hd).astype(np.float32)
    g = rng.standard_normal(heads * hd).astype(np.float32)
    got = orc.attention_decode(q, g, keys, vals, heads, kvh, hd)
    want = _attn64(q.astype(np.float64), g.astype(np.float64), keys, vals, heads, kvh, hd)
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-5)
    # split-K partials merged with merge_attention_partial (full_attention_tiled.cpp:66-78)
    kf, vf = keys.view(np.float16).astype(np.float64), vals.view(np.float16).astype(np.float64)
    h, kv = 1, 0
    m, l, acc = 0.0, 0.0, np.zeros(hd)
    for lo in range(0, seq, 128):
        s = kf[lo:lo + 128, :hd] @ q[h * hd:(h + 1) * hd] / 16.0
        om = s.max(); p = np.exp(s - om); ol = p.sum(); ov = p @ vf[lo:lo + 128, :hd]
        if l == 0:
            m, l, acc = om, ol, ov
            continue
        mm = max(m, om)
        a, b = np.exp(m - mm), np.exp(om - mm)
        acc, l, m = a * acc + b * ov, a * l + b * ol, mm
    merged = acc / l / (1 + np.exp(-g[h * hd:(h + 1) * hd].astype(np.float64)))
    np.testing.assert_allclose(merged, want[h * hd:(h + 1) * hd], rtol=1e-9, atol=1e-12)


def test_conv_ring_equals_causal_convolution(orc):
    rng = np.random.default_rng(5)
    ch, kern, steps = 16, 4, 9
    w = rng.standard_normal((ch, kern)).astype(np.float32)
    km = np.ascontiguousarray(w.T)
    xs = rng.standard_normal((steps, ch)).astype(np.float32)
    state = np.zeros((kern - 1) * ch, np.float32)
    for t in range(steps):
        out = np.zeros(ch, np.float32)
        orc.lib.q35o_conv1d_silu(orc.ptr(state), t % (kern - 1), orc.ptr(np.ascontiguousarray(xs[t])), orc.ptr(km),
                                 orc.ptr(out), ch, kern)
        hist = np.zeros((kern, ch))
        for j in range(kern):
            src = t - (kern - 1) + j
            if src >= 0:
                hist[j] = xs[src]
        z = (hist * w.T.astype(np.float64)).sum(0)
        np.testing.assert_allclose(out, z / (1 + np.exp(-z)), rtol=1e-5, atol=1e-6)


def test_norms_rope_silu_fp64(orc):
    rng = np.random.default_rng(6)
    x = rng.standard_normal((3, 256)).astype(np.float32)
    w = (rng.standard_normal(256) * 0.1).astype(np.float32)
    y = np.zeros_like(x)
    orc.lib.q35o_rms_norm(orc.ptr(x), orc.ptr(w), orc.ptr(y), 3, 256, 1e-6, 1.0)
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt((x64 ** 2).mean(1, keepdims=True) + 1e-6) * (1 + w.astype(np.float64))
    np.testing.assert_allclose(y, want, rtol=1e-5, atol=1e-6)
    z = x.copy()
    orc.lib.q35o_l2_normalize(orc.ptr(z), 3, 256, 1e-6, 0.5)
    np.testing.assert_allclose(z, 0.5 * x64 / np.sqrt((x64 ** 2).sum(1, keepdims=True) + 1e-6), rtol=1e-5)
    r = x[:1].copy()
    c = rng.standard_normal(16).astype(np.float32)
    s = rng.standard_normal(16).astype(np.float32)
    orc.lib.q35o_rope(orc.ptr(r), 1, 256, 32, orc.ptr(c), orc.ptr(s))
    a, b = x64[0, :16], x64[0, 16:32]
    np.testing.assert_allclose(r[0, :16], a * c - b * s, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(r[0, 16:32], b * c + a * s, rtol=1e-5, atol=1e-6)
    assert np.array_equal(r[0, 32:], x[0, 32:])
    o = np.zeros(256, np.float32)
    orc.lib.q35o_silu_mul(orc.ptr(np.ascontiguousarray(x[0])), orc.ptr(np.ascontiguousarray(x[1])), orc.ptr(o), 256)
    np.testing.assert_allclose(o, x64[0] / (1 + np.exp(-x64[0])) * x64[1], rtol=1e-5, atol=1e-6)


def test_step_batched_equals_unbatched(orc):
    """cpu_batch_model_test.cpp:84-108 pattern: a row's logits do not depend on its batch mates."""
    from tests.model_util import build_small_model, small_dims
    d, sched = small_dims()
    t = build_small_model(d, sched, seed=9)
    m = orc.OracleModel(d, sched, t)
    prompts = np.random.default_rng(7).integers(0, d["vocab"], size=(3, 6)).astype(np.int32)
    batched = [m.new_state(16, p) for p in prompts]
    single = [m.new_state(16, p) for p in prompts]
    for step in range(6):
        _, lb, _ = m.step(batched, prompts[:, step], want_logits=True)
        for r in range(3):
            _, ls, _ = m.step([single[r]], prompts[r:r + 1, step], want_logits=True)
            assert np.array_equal(lb[r], ls[0])
