"""q35_q4_dot4_matmul_noalloc (the entry point that allocates nothing: its
scratch is a fixed 16 MiB device array per GPU) against q35_q4_dot4_matmul,
called through the C ABI on the same inputs: bit-identical outputs on two
calls in a row, the second on a smaller shape (the array keeps the first
call's contents), stride padding untouched, and the size limit and argument
errors reported without touching the output."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _problem(orc, rng, rows, blocks, vectors):
    packed = orc.dot4_pack(orc.random_q4_blocks(rng, rows, blocks * 32), rows, blocks)
    x = rng.standard_normal((vectors, blocks * 32)).astype(np.float32)
    return packed, orc.h128_prepare_4(x)


def _call(q, ctx, fn, dm, da, out, rows, vectors, blocks, stride):
    return fn(ctx.handle, dm.ptr, da.ptr, out.ptr, rows, vectors, blocks, stride)


# (rows, blocks, vectors, stride): a 4B down projection shape (K split 32 ways,
# 48-token chunks), then a smaller one with a ragged token count and padding,
# then four vectors (the GEMV, no scratch)
SHAPES = [(2560, 288, 132, 2560), (1032, 40, 20, 1039), (520, 36, 4, 523)]


def test_two_calls_match_allocating_entry_point(q, ctx, orc):
    for i, (rows, blocks, vectors, stride) in enumerate(SHAPES):
        rng = np.random.default_rng(900 + i)
        packed, act = _problem(orc, rng, rows, blocks, vectors)
        dm, da = ctx.array(packed), ctx.array(act)
        init = np.full((vectors, stride), -77.0, np.float32)
        ref, got = ctx.array(init), ctx.array(init)
        print(f"noalloc call {i}: rows={rows} blocks={blocks} vectors={vectors} stride={stride}", flush=True)
        ctx.check(_call(q, ctx, q.lib.q35_q4_dot4_matmul, dm, da, ref, rows, vectors, blocks, stride), "matmul")
        ctx.check(_call(q, ctx, q.lib.q35_q4_dot4_matmul_noalloc, dm, da, got, rows, vectors, blocks, stride),
                  "matmul_noalloc")
        want, have = ref.download(), got.download()
        np.testing.assert_array_equal(have.view(np.uint32), want.view(np.uint32))
        assert np.all(have[:, rows:] == -77.0)
        # the contraction itself, against the oracle's reference fma chain
        exact = orc.dot4_matmul(packed, act, rows, vectors, blocks)
        assert np.max(np.abs(have[:, :rows] - exact)) <= 1e-5 * np.abs(exact).max()


def test_limits_and_errors(q, ctx, orc):
    rng = np.random.default_rng(7)
    packed, act = _problem(orc, rng, 64, 4, 4)
    dm, da = ctx.array(packed), ctx.array(act)
    out = ctx.array(np.full((4, 64), 5.0, np.float32))
    fn = q.lib.q35_q4_dot4_matmul_noalloc
    print("noalloc: rejected shapes", flush=True)
    # 16384 rows x 288 blocks at 8 vectors: 32 K splits x 16 tokens x 16384
    # rows of FP32 partials (32 MiB) exceed the array; rejected before any
    # launch (up to 4 vectors run the GEMV, which uses no scratch)
    assert _call(q, ctx, fn, dm, da, out, 16384, 8, 288, 16384) == 5  # Q35_ERR_UNSUPPORTED
    assert b"static scratch" in q.lib.q35_context_last_error(ctx.handle)
    assert _call(q, ctx, fn, dm, da, out, 64, 6, 4, 64) == 1  # vector count % 4
    assert _call(q, ctx, fn, dm, da, out, 60, 4, 4, 64) == 1  # rows % 8
    assert fn(ctx.handle, dm.ptr, da.ptr, ctypes.c_void_p(), 64, 4, 4, 64) == 1  # no output
    ctx.synchronize()
    assert np.all(out.download() == 5.0)
