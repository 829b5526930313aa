"""CPU pins of the stage-parity checker's own helpers (tests/test_gpu_stage_parity.py):
the numpy DOT4 unpack and FP64 projection reference against the C oracle's
q35o_dot4_matmul (the reference's scalar_row chain), and the A16 <-> X4 code
layouts against each other."""
import numpy as np

from tests.test_gpu_stage_parity import Dot4, a16_rows, x4_rows


def test_dot4_reference_matches_oracle_chain(orc):
    rng = np.random.default_rng(11)
    rows, cols, tokens = 48, 256, 8
    packed = orc.dot4_pack(orc.random_q4_blocks(rng, rows, cols), rows, cols // 32)
    x = rng.standard_normal((tokens, cols)).astype(np.float32)
    act = orc.h128_prepare_4(x)
    want = orc.dot4_matmul(packed, act, rows, tokens, cols // 32)
    codes, scales = x4_rows(act, tokens)
    got = Dot4(packed.view(np.uint8).ravel(), rows, cols).rows_for(codes, scales)
    # FP64 over exact block dots vs the FP32 block-order chain: rounding only
    assert np.max(np.abs(got - want)) <= 1e-5 * np.max(np.abs(want))
    # a planted mistake in the unpack (one nibble order swapped) is caught
    bad = Dot4(packed.view(np.uint8).ravel(), rows, cols)
    bad.w = bad.w[:, :, ::-1].copy()
    assert np.max(np.abs(bad.rows_for(codes, scales) - want)) > 1e-2 * np.max(np.abs(want))


def test_a16_layout_inverts_to_x4(orc):
    rng = np.random.default_rng(12)
    rows, cols = 20, 128
    x = rng.standard_normal((24, cols)).astype(np.float32)
    act = orc.h128_prepare_4(x)
    codes, scales = x4_rows(act, 24)
    nb, tiles = cols // 32, 2
    # build the A16 words: tile, block, lane = token + 16 * k-group, 8 codes each
    a16 = np.zeros((tiles, nb, 64, 8), np.int8)
    sc = np.zeros((tiles, nb, 16), np.float32)
    for t in range(rows):
        for b in range(nb):
            for g in range(4):
                a16[t // 16, b, t % 16 + 16 * g] = codes[t, b * 32 + 8 * g:b * 32 + 8 * g + 8]
            sc[t // 16, b, t % 16] = scales[t, b]
    got_c, got_s = a16_rows(a16.view(np.uint64).ravel(), sc.ravel(), rows, nb)
    np.testing.assert_array_equal(got_c, codes[:rows])
    np.testing.assert_array_equal(got_s, scales[:rows])
