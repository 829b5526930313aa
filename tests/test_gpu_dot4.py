"""Q4-G32-DOT4 GEMV/GEMM parity on the GPU (config 1 and edge shapes).

Bar: int32 block dots bit-exact; the exact-mode FP32 outputs bit-exact (same
fma chain as q4_dot4.cpp:43-56); production split-K outputs within 1e-5
relative (north-star bar 1e-3); argmax indices exact."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _problem(orc, rng, rows, cols, vectors):
    canon = orc.random_q4_blocks(rng, rows, cols)
    packed = orc.dot4_pack(canon, rows, cols // 32)
    x = rng.standard_normal((vectors, cols)).astype(np.float32)
    return packed, x


@pytest.mark.parametrize("vectors", [4, 16])
def test_config1_matmul_h128(q, ctx, orc, vectors):
    rng = np.random.default_rng(3701 + vectors)
    rows, cols = 3584, 1024
    packed, x = _problem(orc, rng, rows, cols, vectors)
    act = orc.h128_prepare_4(x)
    want = orc.dot4_matmul(packed, act, rows, vectors, cols // 32)
    dm, da = ctx.array(packed), ctx.array(act)
    out = ctx.array(shape=(vectors, rows), dtype=np.float32)
    print(f"config1 matmul B={vectors}", flush=True)
    q.q4_dot4_matmul(ctx, dm, da, out, rows, vectors, cols // 32, rows, exact=True)
    got = out.download()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    q.q4_dot4_matmul(ctx, dm, da, out, rows, vectors, cols // 32, rows)
    fast = out.download()
    scale = np.abs(want).max()
    assert np.max(np.abs(fast - want)) <= 1e-5 * scale
    # int32 block dots, bit-exact against the brute-force oracle
    dots = ctx.array(shape=(vectors, rows, cols // 32), dtype=np.int32)
    q.q4_dot4_block_dots(ctx, dm, da, dots, rows, vectors, cols // 32)
    got_dots = dots.download()
    for t in (0, vectors - 1):
        codes, _, _ = orc.x4_vector(act, t)
        assert np.array_equal(got_dots[t], orc.dot4_block_dots(packed, codes, rows, cols // 32))


def test_config1_matvec_b1(q, ctx, orc):
    rng = np.random.default_rng(1701)
    rows, cols = 3584, 1024
    packed, x = _problem(orc, rng, rows, cols, 1)
    act = orc.q8_quantize_1(x[0])
    want = orc.dot4_matvec(packed, act, rows, cols // 32)
    dm, da = ctx.array(packed), ctx.array(act)
    out = ctx.array(shape=(rows,), dtype=np.float32)
    print("config1 matvec B=1", flush=True)
    q.q4_dot4_matvec(ctx, dm, da, out, rows, cols // 32)
    got = out.download()
    # the single-launch dot4 GEMV runs the reference's chain: bit-exact
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("rows,blocks,count", [(8, 1, 1), (200, 112, 2), (3584, 32, 3), (1032, 288, 4),
                                               (64, 129, 1), (2560, 80, 4)])
def test_small_count_gemv_exact(q, ctx, orc, rows, blocks, count):
    """One to four vectors run the single-launch dot4 GEMV: X1 rows
    (matvec, matmul_x1) and an X4 group (matmul, 4 vectors) give the oracle's
    block-order chain (q4_dot4.cpp:43-56) bit for bit, over one and several
    128-block passes and a ragged last pass; outputs beyond `rows` in the
    strided layout stay untouched."""
    rng = np.random.default_rng(rows * 7 + blocks + count)
    packed, x = _problem(orc, rng, rows, blocks * 32, count)
    x1 = np.stack([orc.q8_quantize_1(x[i]) for i in range(count)])
    want = np.stack([orc.dot4_matvec(packed, x1[i], rows, blocks) for i in range(count)])
    dm = ctx.array(packed)
    stride = rows + 3
    out = ctx.array(np.full((count, stride), 7.0, np.float32))
    print(f"small-count GEMV rows={rows} blocks={blocks} count={count}", flush=True)
    q.q4_dot4_matmul_x1(ctx, dm, ctx.array(x1), out, rows, count, blocks, stride)
    got = out.download()
    assert np.all(got[:, rows:] == 7.0)
    np.testing.assert_array_equal(got[:, :rows].view(np.uint32), want.view(np.uint32))
    if count == 1:
        one = ctx.array(shape=(rows,), dtype=np.float32)
        q.q4_dot4_matvec(ctx, dm, ctx.array(x1[0]), one, rows, blocks)
        np.testing.assert_array_equal(one.download().view(np.uint32), want[0].view(np.uint32))
    if count == 4:
        act = orc.h128_prepare_4(x)
        want4 = orc.dot4_matmul(packed, act, rows, 4, blocks)
        out4 = ctx.array(shape=(4, stride), dtype=np.float32)
        q.q4_dot4_matmul(ctx, dm, ctx.array(act), out4, rows, 4, blocks, stride)
        np.testing.assert_array_equal(out4.download()[:, :rows].view(np.uint32), want4.view(np.uint32))


@pytest.mark.parametrize("rows,blocks,vectors,stride", [(8, 1, 4, 8), (24, 3, 8, 31), (200, 112, 12, 207),
                                                        (1032, 32, 64, 1032), (64, 4, 20, 64)])
def test_edge_shapes(q, ctx, orc, rows, blocks, vectors, stride):
    rng = np.random.default_rng(rows * 7 + blocks)
    packed, x = _problem(orc, rng, rows, blocks * 32, vectors)
    act = orc.q8_quantize_4(x)
    want = orc.dot4_matmul(packed, act, rows, vectors, blocks, stride)
    dm, da = ctx.array(packed), ctx.array(act)
    init = np.full((vectors, stride), -123.0, np.float32)
    out = ctx.array(init)
    print(f"edge rows={rows} blocks={blocks} vectors={vectors}", flush=True)
    q.q4_dot4_matmul(ctx, dm, da, out, rows, vectors, blocks, stride, exact=True)
    got = out.download()
    assert np.array_equal(got[:, :rows].view(np.uint32), want[:, :rows].view(np.uint32))
    assert np.all(got[:, rows:] == -123.0), "wrote past `rows` into the stride padding"


def test_extreme_codes(q, ctx, orc):
    """All-15 / all-0 codes with +-127 activations (the reference test's patterns 0 and 1)."""
    rows, blocks, vectors = 64, 64, 4
    for pattern in (0, 1):
        canon = np.zeros((rows, blocks), orc.Q4_0)
        canon["qs"] = 255 if pattern == 0 else 0
        canon["d"] = np.float16(1.0).view(np.uint16)
        packed = orc.dot4_pack(canon, rows, blocks)
        act = np.zeros((vectors // 4, blocks), orc.Q8X4)
        act["qs"] = -128 if pattern == 0 else 127
        act["sums"] = act["qs"].reshape(vectors // 4, blocks, 4, 32).astype(np.int32).sum(-1)
        act["scales"] = 0.001
        want = orc.dot4_matmul(packed, act, rows, vectors, blocks)
        dm, da = ctx.array(packed), ctx.array(act)
        out = ctx.array(shape=(vectors, rows), dtype=np.float32)
        q.q4_dot4_matmul(ctx, dm, da, out, rows, vectors, blocks, rows, exact=True)
        assert np.array_equal(out.download(), want)


def test_argmax_batch_penalty(q, ctx, orc):
    """Fused greedy head: per-row penalty and lowest-index ties (cpu_engine_greedy.inl:45-57)."""
    rng = np.random.default_rng(11)
    rows, cols, vectors = 4096, 1024, 8
    packed, x = _problem(orc, rng, rows, cols, vectors)
    act = orc.q8_quantize_4(x)
    logits = orc.dot4_matmul(packed, act, rows, vectors, cols // 32)
    counts = (rng.random((vectors, rows)) < 0.05).astype(np.int32) * 2
    pen = np.array([1.0, 1.05, 1.3, 1.0, 2.0, 1.0, 1.1, 1.0], np.float32)
    adj = logits.copy()
    for v in range(vectors):
        m = (counts[v] > 0) & (pen[v] > 1)
        adj[v, m] = np.where(adj[v, m] > 0, adj[v, m] / pen[v], adj[v, m] * pen[v])
    want = adj.argmax(1)
    dm, da, dc, dp = ctx.array(packed), ctx.array(act), ctx.array(counts), ctx.array(pen)
    idx = ctx.array(shape=(vectors,), dtype=np.int32)
    val = ctx.array(shape=(vectors,), dtype=np.float32)
    q.q4_dot4_argmax_batch(ctx, dm, da, dc, dp, rows, vectors, cols // 32, idx, val)
    got = idx.download()
    # every row's logit is one fp32 fma chain in block order, as in the
    # reference: the winning value and index are exact
    np.testing.assert_array_equal(got, want)
    np.testing.assert_array_equal(val.download(), adj[np.arange(vectors), want])
    # exact ties go to the lowest index
    canon = np.zeros((16, 1), orc.Q4_0)
    canon["qs"] = 0x99
    canon["d"] = np.float16(1.0).view(np.uint16)
    tpk = orc.dot4_pack(canon, 16, 1)
    tact = np.zeros((1, 1), orc.Q8X4)
    tact["qs"] = 1
    tact["sums"] = 32
    tact["scales"] = 1.0
    q.q4_dot4_argmax_batch(ctx, ctx.array(tpk), ctx.array(tact), None, None, 16, 4, 1, idx, val)
    assert np.all(idx.download()[:4] == 0)


@pytest.mark.parametrize("rows,cols,vectors", [(1000, 1024, 16), (4096, 1024, 40), (2056, 2560, 64), (520, 4096, 4)])
def test_argmax_head_shapes(q, ctx, orc, rows, cols, vectors):
    """Greedy head over ragged row groups (rows % 64 != 0), one to four token
    tiles and widths whose staged activations do or do not fit in LDS (the
    streaming kernel and its fallback): exact index and value against the
    oracle's logits (argmax with lowest-index ties)."""
    rng = np.random.default_rng(rows + cols + vectors)
    packed, x = _problem(orc, rng, rows, cols, vectors)
    act = orc.q8_quantize_4(x)
    logits = orc.dot4_matmul(packed, act, rows, vectors, cols // 32)
    counts = (rng.random((vectors, rows)) < 0.1).astype(np.int32)
    pen = np.where(np.arange(vectors) % 3 == 1, 1.5, 1.0).astype(np.float32)
    adj = logits.copy()
    for v in range(vectors):
        m = (counts[v] > 0) & (pen[v] > 1)
        adj[v, m] = np.where(adj[v, m] > 0, adj[v, m] / pen[v], adj[v, m] * pen[v])
    want = adj.argmax(1)
    idx = ctx.array(shape=(vectors,), dtype=np.int32)
    val = ctx.array(shape=(vectors,), dtype=np.float32)
    print(f"argmax head rows={rows} cols={cols} B={vectors}", flush=True)
    q.q4_dot4_argmax_batch(ctx, ctx.array(packed), ctx.array(act), ctx.array(counts), ctx.array(pen), rows, vectors,
                           cols // 32, idx, val)
    np.testing.assert_array_equal(idx.download(), want)
    np.testing.assert_array_equal(val.download(), adj[np.arange(vectors), want])


@pytest.mark.parametrize("rows,blocks,vectors", [(2560, 288, 300), (3584, 32, 512), (200, 112, 132), (1032, 80, 68),
                                                  (16392, 40, 100), (200, 8, 4136)])
def test_dense_matches_split_launches(q, ctx, orc, rows, blocks, vectors):
    """Above 64 vectors q4_dot4_matmul runs the dense GEMM (every K block of a
    64-row group in one wavefront, the split structure folded in registers);
    its rows must equal the 64-vector split launches bit for bit, here with
    32, 4 and 14 K splits, a ragged row group and ragged token groups; 16392
    rows give a tall matrix whose last 64-row group holds one 8-row tile.
    4136 vectors are a 4096-vector chunk and a 40-vector one, which the dense
    GEMM runs with one token tile per wavefront (its form at 64 rows)."""
    rng = np.random.default_rng(rows + vectors)
    packed, x = _problem(orc, rng, rows, blocks * 32, vectors)
    act = orc.h128_prepare_4(x)
    dm, da = ctx.array(packed), ctx.array(act)
    stride = rows + 4
    dense = ctx.array(np.full((vectors, stride), -5.0, np.float32))
    print(f"dense rows={rows} blocks={blocks} vectors={vectors}", flush=True)
    q.q4_dot4_matmul(ctx, dm, da, dense, rows, vectors, blocks, stride)
    got = dense.download()
    assert np.all(got[:, rows:] == -5.0)
    for t0 in range(0, vectors, 64):
        n = min(64, vectors - t0)
        # up to four vectors would run the GEMV's single chains: launch eight
        # (the group twice) and keep the first rows, which are batch-invariant
        sub = act[t0 // 4:(t0 + n) // 4]
        n_run = 8 if n <= 4 else n
        part = ctx.array(shape=(n_run, stride), dtype=np.float32)
        q.q4_dot4_matmul(ctx, dm, ctx.array(np.concatenate([sub, sub]) if n <= 4 else sub), part, rows, n_run,
                         blocks, stride)
        np.testing.assert_array_equal(got[t0:t0 + n, :rows].view(np.uint32), part.download()[:n, :rows].view(np.uint32),
                                      err_msg=f"vectors {t0}..{t0 + n}")
    want = orc.dot4_matmul(packed, act, rows, vectors, blocks)
    assert np.max(np.abs(got[:, :rows] - want)) <= 1e-5 * np.abs(want).max()


@pytest.mark.parametrize("count", [5, 8, 70])
def test_matmul_x1_rows(q, ctx, orc, count):
    """q4_dot4_matmul_x1 (q4_dot4.h:15-18): independently prepared X1 rows
    give the bits of the X4 path on the same vectors (every count, the dense
    path above 64), and each row equals the oracle's matvec within 1e-5."""
    rng = np.random.default_rng(4100 + count)
    rows, cols = 520, 1024
    packed, x = _problem(orc, rng, rows, cols, count)
    x1 = np.stack([orc.h128_prepare_1(x[i]) for i in range(count)])
    dm = ctx.array(packed)
    stride = rows + 8
    out = ctx.array(np.full((count, stride), 3.0, np.float32))
    print(f"matmul_x1 count={count}", flush=True)
    q.q4_dot4_matmul_x1(ctx, dm, ctx.array(x1), out, rows, count, cols // 32, stride)
    got = out.download()
    assert np.all(got[:, rows:] == 3.0)
    assert q.lib.q35_q4_dot4_has_x1_tile(count) == 1
    if count % 4 == 0:
        ref = ctx.array(shape=(count, stride), dtype=np.float32)
        q.q4_dot4_matmul(ctx, dm, ctx.array(orc.h128_prepare_4(x)), ref, rows, count, cols // 32, stride)
        np.testing.assert_array_equal(got[:, :rows].view(np.uint32), ref.download()[:, :rows].view(np.uint32))
    for i in (0, count - 1):
        want = orc.dot4_matvec(packed, x1[i], rows, cols // 32)
        assert np.max(np.abs(got[i, :rows] - want)) <= 1e-5 * np.abs(want).max()
