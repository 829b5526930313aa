"""Pins of the sampling restatement (oracle/sampling.py) that the GPU engine's
sampled decoding is checked against: the C++ standard's known answer for
std::mt19937, libstdc++'s uniform_real_distribution<float> boundary, and
token-for-token agreement with the reference engine's own sampled decoding
(sample_token_from_logits, layers.inl:491-600, through CpuEngine built in
oracle/_ref) over penalties, temperatures, top_k (including 0 = every token)
and top_p."""
import os

import numpy as np
import pytest

from oracle import q35_oracle as orc
from oracle.sampling import MT19937, sample_token, uniform_float


def test_mt19937_known_answer():
    rng = MT19937()
    for _ in range(9999):
        rng()
    assert rng() == 4123659995  # [rand.predef]: the 10000th output of mt19937


def test_uniform_float_stays_below_one():
    class Fixed:
        def __init__(self, v):
            self.v = v

        def __call__(self):
            return self.v

    assert uniform_float(Fixed(0)) == 0.0
    assert uniform_float(Fixed(2 ** 31)) == np.float32(0.5)
    top = uniform_float(Fixed(2 ** 32 - 1))  # float(2^32 - 1) rounds to 2^32
    assert top < 1.0 and top == np.nextafter(np.float32(1), np.float32(0))


@pytest.fixture(scope="module")
def model_dir(q, tmp_path_factory):
    import json

    import bench
    from tests.model_util import write_0p8b_artifact

    path = str(tmp_path_factory.mktemp("m08s"))
    d, _, art = write_0p8b_artifact(q, path, 1, 0.02)
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(bench.CONFIG_08B, f)
    return d, path, art


@pytest.mark.skipif(not orc.ref_available(), reason="oracle/_ref (the reference build) is not built here")
@pytest.mark.parametrize("temperature,top_p,top_k,penalty,seed", [(0.7, 0.8, 20, 1.05, 1234), (1.0, 1.0, 0, 1.0, 7),
                                                                  (0.6, 0.95, 0, 1.3, 99), (0.0, 1.0, 0, 1.2, 5),
                                                                  (1.2, 0.5, 3, 1.0, 31)])
def test_restatement_matches_reference_engine(model_dir, temperature, top_p, top_k, penalty, seed):
    """The reference CpuEngine samples a request (its logits callback reports
    every raw logits row); the restatement, fed those rows and the request's
    counts (prompt tokens plus the tokens sampled so far, cpu_engine.inl:376-378,
    :464), draws the same tokens from the same seed."""
    d, path, art = model_dir
    prompt = np.random.default_rng(seed).integers(0, d.vocab, size=12).astype(np.int32)
    new = 12
    want, logits = orc.ref_engine_sample(path, art, prompt, new, d.vocab, temperature, top_p, top_k, penalty, seed)
    counts = np.bincount(prompt, minlength=d.vocab).astype(np.int32)
    mt = MT19937(seed)
    for s in range(new):
        got = sample_token(logits[s], counts, temperature, top_p, top_k, penalty, mt)
        assert got == want[s], (s, got, want[s])
        counts[want[s]] += 1
