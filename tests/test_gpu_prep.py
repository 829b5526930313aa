"""Activation preparation parity on the GPU: int8 codes, sums and FP32 scales
bit-exact against the oracle (q4_0.cpp:149-235, q4_h128.cpp:259-401)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("cols", [128, 1024, 2048, 3584])
@pytest.mark.parametrize("vectors", [4, 16])
def test_h128_prepare_4(q, ctx, orc, cols, vectors):
    rng = np.random.default_rng(cols + vectors)
    x = rng.standard_normal((vectors, cols)).astype(np.float32)
    x[0, :32] = 0.0            # zero block: scale 0, inverse 0
    x[1, 5] = 1e30 if vectors > 1 else 0.0
    want = orc.h128_prepare_4(x)
    dx = ctx.array(x)
    out = ctx.array(shape=want.shape, dtype=orc.Q8X4)
    print(f"h128 prepare_4 cols={cols} vectors={vectors}", flush=True)
    q.q4_h128_prepare_activations_4(ctx, dx, out, vectors, cols)
    got = out.download()
    assert np.array_equal(got["qs"], want["qs"])
    assert np.array_equal(got["sums"], want["sums"])
    assert np.array_equal(got["scales"].view(np.uint32), want["scales"].view(np.uint32))


@pytest.mark.parametrize("cols", [1024, 3584])
def test_h128_prepare_1(q, ctx, orc, cols):
    rng = np.random.default_rng(cols)
    x = (rng.standard_normal(cols) * 3).astype(np.float32)
    want = orc.h128_prepare_1(x)
    out = ctx.array(shape=want.shape, dtype=orc.Q8X1)
    q.q4_h128_prepare_activation_1(ctx, ctx.array(x), out, cols)
    got = out.download()
    for f in ("qs", "sums"):
        assert np.array_equal(got[f], want[f])
    assert np.array_equal(got["scales"].view(np.uint32), want["scales"].view(np.uint32))


def test_identity_quantize(q, ctx, orc):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((16, 1024)).astype(np.float32)
    # exact .5 ties after scaling round away from zero
    x[2, :32] = np.linspace(-127, 127, 32, dtype=np.float32) / 2.0
    want4 = orc.q8_quantize_4(x)
    out4 = ctx.array(shape=want4.shape, dtype=orc.Q8X4)
    q.q8_0_quantize_vectors_4(ctx, ctx.array(x), out4, 16, 32)
    got4 = out4.download()
    assert np.array_equal(got4["qs"], want4["qs"]) and np.array_equal(got4["sums"], want4["sums"])
    assert np.array_equal(got4["scales"].view(np.uint32), want4["scales"].view(np.uint32))
    want1 = orc.q8_quantize_1(x[3])
    out1 = ctx.array(shape=want1.shape, dtype=orc.Q8X1)
    q.q8_0_quantize_vector_1(ctx, ctx.array(x[3]), out1, 32)
    got1 = out1.download()
    assert np.array_equal(got1["qs"], want1["qs"]) and np.array_equal(got1["sums"], want1["sums"])
