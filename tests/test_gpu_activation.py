"""The stand-alone activation entry points (include/q35_hip.h, activation
ops; activation.h:9-77, full_attention.h:22-26) against the CPU oracle on
seeded inputs, including the edges each reference function names:
- q35_rms_norm_f32: Qwen's (1 + w) offset and a plain offset 0, odd widths;
- q35_l2_normalize_f32: in place, with an output scale, a zero row;
- q35_causal_conv1d_silu_f32: several tokens through the ring (each advances
  it), a strided input, a channel sub-range (other channels untouched);
- q35_silu_mul_f32: the exponent range on both sides of zero;
- q35_rope_f32: split-half rotation of the first rope_dim dims only;
- q35_attention_cache_store_f16: round-to-nearest-even, subnormals,
  overflow, signed zero and quiet NaN, bit-exact.
FP32 results are within 1e-5 relative (the GPU's reduction order and
device exp differ in the last bits); stores, ring updates and binary16 bits
are exact."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def close(got, want, rtol=1e-5, what=""):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    floor = rtol * (np.max(np.abs(want)) if want.size else 0.0)
    assert np.all(np.abs(got - want) <= rtol * np.abs(want) + floor), what


@pytest.mark.parametrize("rows,width,offset", [(5, 1024, 1.0), (3, 256, 0.0), (2, 130, 1.0)])
def test_rms_norm(q, ctx, orc, rows, width, offset):
    rng = np.random.default_rng(width)
    x = rng.standard_normal((rows, width)).astype(np.float32) * 3
    w = rng.standard_normal(width).astype(np.float32) * 0.2
    out = ctx.array(shape=(rows, width), dtype=np.float32)
    print(f"rms_norm {rows}x{width} offset {offset}", flush=True)
    q.rms_norm_f32(ctx, ctx.array(x), ctx.array(w), out, rows, width, 1e-6, offset)
    close(out.download(), orc.rms_norm(x, w, 1e-6, offset))


def test_l2_normalize(q, ctx, orc):
    rng = np.random.default_rng(3)
    x = rng.standard_normal((6, 128)).astype(np.float32)
    x[2] = 0.0  # eps keeps a zero row finite
    dx = ctx.array(x)
    print("l2_normalize", flush=True)
    q.l2_normalize_f32(ctx, dx, 6, 128, 1e-6, 1.0 / np.sqrt(128.0))
    want = x.copy()
    orc.lib.q35o_l2_normalize(orc.ptr(want), 6, 128, 1e-6, 1.0 / np.sqrt(128.0))
    got = dx.download()
    close(got, want)
    assert np.all(got[2] == 0.0)


def test_causal_conv1d_ring_stride_and_range(q, ctx, orc):
    rng = np.random.default_rng(4)
    ch, kern, batch, stride = 300, 4, 5, 320
    begin, end = 17, 260
    state = rng.standard_normal((kern - 1, ch)).astype(np.float32)
    x = rng.standard_normal((batch, stride)).astype(np.float32)
    w = rng.standard_normal((kern, ch)).astype(np.float32) * 0.5
    ring = 2
    dstate, dout = ctx.array(state), ctx.array(np.full((batch, ch), 7.0, np.float32))
    print("conv1d: 5 tokens, strided input, channels [17, 260)", flush=True)
    q.causal_conv1d_silu_f32(ctx, dstate, ring, ctx.array(x), ctx.array(w), dout, ch, kern, batch=batch,
                             input_stride=stride, channel_begin=begin, channel_end=end)
    want_state, want_out, r = state.copy(), np.full((batch, ch), 7.0, np.float32), ring
    for t in range(batch):
        o = np.zeros(ch, np.float32)
        st = want_state.copy()
        orc.lib.q35o_conv1d_silu(orc.ptr(st), r, orc.ptr(np.ascontiguousarray(x[t, :ch])), orc.ptr(w), orc.ptr(o),
                                 ch, kern)
        want_state[:, begin:end] = st[:, begin:end]
        want_out[t, begin:end] = o[begin:end]
        r = (r + 1) % (kern - 1)
    got_state, got_out = dstate.download(), dout.download()
    np.testing.assert_array_equal(got_state, want_state)  # raw inputs into the ring, other channels untouched
    close(got_out, want_out)
    np.testing.assert_array_equal(got_out[:, :begin], want_out[:, :begin])


def test_silu_mul(q, ctx, orc):
    rng = np.random.default_rng(5)
    g = np.concatenate([rng.standard_normal(4000) * 6, [0.0, -0.0, 40.0, -40.0, 88.0, -90.0]]).astype(np.float32)
    u = rng.standard_normal(g.size).astype(np.float32)
    out = ctx.array(shape=(g.size,), dtype=np.float32)
    print("silu_mul", flush=True)
    q.silu_mul_f32(ctx, ctx.array(g), ctx.array(u), out, g.size)
    close(out.download(), orc.silu_mul(g, u))


@pytest.mark.parametrize("rope_dim", [64, 256, 2])
def test_rope(q, ctx, orc, rope_dim):
    rng = np.random.default_rng(rope_dim)
    heads, hd = 6, 256
    x = rng.standard_normal((heads, hd)).astype(np.float32)
    cs, sn = orc.rope_tables(10000000.0, rope_dim, 700)
    c, s = np.ascontiguousarray(cs[613]), np.ascontiguousarray(sn[613])
    dx = ctx.array(x)
    print(f"rope dim {rope_dim}", flush=True)
    q.rope_f32(ctx, dx, heads, hd, rope_dim, ctx.array(c), ctx.array(s))
    want = x.copy()
    orc.lib.q35o_rope(orc.ptr(want), heads, hd, rope_dim, orc.ptr(c), orc.ptr(s))
    got = dx.download()
    close(got, want)
    np.testing.assert_array_equal(got[:, rope_dim:], x[:, rope_dim:])


def test_attention_cache_store_f16(q, ctx, orc):
    rng = np.random.default_rng(6)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * np.float32(2.0) ** rng.integers(-28, 18, 100000),
                        np.array([0.0, -0.0, np.inf, -np.inf, 65504, 65520, 1e-8, -6e-8, np.nan], np.float32),
                        np.array([0x7fa00000, 0xffc00001, 0x33000001, 0x387fffff, 0x477fefff], np.uint32).view(
                            np.float32)]).astype(np.float32)
    out = ctx.array(shape=(x.size,), dtype=np.uint16)
    print("attention_cache_store_f16", flush=True)
    q.attention_cache_store_f16(ctx, ctx.array(x), out, x.size)
    np.testing.assert_array_equal(out.download(), orc.f16_bits(x))
