"""Restatement of the reference's sampled decoding for tests: std::mt19937
(the C++ standard's MT19937 with init_genrand seeding), libstdc++'s
uniform_real_distribution<float> over it (one 32-bit draw: float(x) / 2^32,
kept below 1), and sample_token_from_logits (src/runtime/layers.inl:491-600).
TEST INFRASTRUCTURE ONLY: the product samples in the engine
(qwen35-cpu_amd/csrc/engine.cpp) from device candidate lists.

Pins (tests/test_oracle_sampling.py): the C++ standard's known answer for
mt19937 (the 10000th output of a default-seeded engine is 4123659995,
[rand.predef]), and token-for-token agreement with the reference's own
sample_token_from_logits built in oracle/_ref."""
import math

import numpy as np


class MT19937:
    """std::mt19937: 624-word state, init_genrand seeding, tempered outputs."""

    def __init__(self, seed=5489):
        self.mt = [0] * 624
        self.mt[0] = seed & 0xFFFFFFFF
        for i in range(1, 624):
            prev = self.mt[i - 1]
            self.mt[i] = (1812433253 * (prev ^ (prev >> 30)) + i) & 0xFFFFFFFF
        self.index = 624

    def _twist(self):
        mt = self.mt
        for i in range(624):
            y = (mt[i] & 0x80000000) | (mt[(i + 1) % 624] & 0x7FFFFFFF)
            v = mt[(i + 397) % 624] ^ (y >> 1)
            if y & 1:
                v ^= 0x9908B0DF
            mt[i] = v
        self.index = 0

    def __call__(self):
        if self.index >= 624:
            self._twist()
        y = self.mt[self.index]
        self.index += 1
        y ^= y >> 11
        y ^= (y << 7) & 0x9D2C5680
        y ^= (y << 15) & 0xEFC60000
        y ^= y >> 18
        return y & 0xFFFFFFFF


def uniform_float(rng):
    """uniform_real_distribution<float>(0, 1)(rng) in libstdc++: generate_canonical
    with one 32-bit draw, float(x) / 2^32, kept below 1."""
    r = np.float32(rng()) / np.float32(4294967296.0)
    if r >= np.float32(1.0):
        r = np.nextafter(np.float32(1.0), np.float32(0.0))
    return r


def sample_token(raw_logits, counts, temperature, top_p, top_k, penalty, rng):
    """sample_token_from_logits (layers.inl:491-600) in float32, in the
    reference's order of operations. Candidate ties sort by lower token."""
    raw = np.asarray(raw_logits, np.float32)
    cnt = np.asarray(counts)
    if temperature <= 1.0e-6:
        v = raw.copy()
        if penalty > 1.0:
            m = cnt > 0
            v[m] = np.where(v[m] > 0, v[m] / np.float32(penalty), v[m] * np.float32(penalty))
        return int(np.argmax(v))  # first maximum, as argmax_index
    v = raw.copy()
    if penalty > 1.0:
        m = cnt > 0
        v[m] = np.where(v[m] > 0, v[m] / np.float32(penalty), v[m] * np.float32(penalty))
    v = v * (np.float32(1.0) / np.float32(temperature))
    order = np.lexsort((np.arange(v.size), -v.astype(np.float64)))
    if 0 < top_k < v.size:
        order = order[:top_k]
    vals = v[order]
    max_logit = np.float32(vals.max())
    probs = np.array([np.float32(math.exp(float(np.float32(x - max_logit)))) for x in vals], np.float32)
    denom = np.float32(0.0)
    for p in probs:
        denom = np.float32(denom + p)
    if not denom > 0:
        return int(order[0])
    probs = (probs / denom).astype(np.float32)
    keep = probs.size
    if top_p < 1.0:
        cumulative = np.float32(0.0)
        keep = 0
        while keep < probs.size:
            cumulative = np.float32(cumulative + probs[keep])
            if cumulative >= np.float32(top_p):
                keep += 1
                break
            keep += 1
        keep = max(1, min(keep, probs.size))
    probs = probs[:keep]
    renorm = np.float32(0.0)
    for p in probs:
        renorm = np.float32(renorm + p)
    if not renorm > 0:
        return int(order[0])
    probs = (probs / renorm).astype(np.float32)
    r = uniform_float(rng)
    cumulative = np.float32(0.0)
    for i in range(probs.size):
        cumulative = np.float32(cumulative + probs[i])
        if r <= cumulative or i + 1 == probs.size:
            return int(order[i])
    return int(order[-1])
