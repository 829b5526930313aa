"""The CPU oracle's whole decode step (q35o_forward_batch, the restatement of
forward_batch, cpu_engine.inl:201-325) on the random-init 0.8B artifact
against the reference CpuEngine's teacher-forced logits
(tests/golden/engine_0p8b.npz). Activation quantization makes any two
implementations with different reduction orders drift apart through binary16
scale flips; the reference's scalar and auto-selected backends themselves
differ by the envelope stored in the golden. The oracle must stay within 1.5x
that envelope of the reference's production (auto) backend."""
import os

import numpy as np
import pytest

from tests.model_util import (artifact_tensors, check_within_envelope, golden_0p8b, reference_envelope,
                              teacher_forced_probe_logits, write_0p8b_artifact)

ROWS = 2


@pytest.fixture(scope="module", params=["q4", "g16q8"])
def artifact(q, tmp_path_factory, request):
    """Both artifact variants: Q4 throughout, and the G16 tied head with Q8_0
    gate rows (weights.inl:724-734, :1700-1747), each with its reference golden."""
    g = golden_0p8b(request.param)
    d, sched, path = write_0p8b_artifact(q, str(tmp_path_factory.mktemp("m08")), int(g["seed"][0]),
                                         float(g["weight_std"][0]), request.param)
    yield d, sched, path, g
    os.remove(path)


def test_oracle_within_reference_envelope(orc, artifact):
    d, sched, path, g = artifact
    m = orc.OracleModel(d.as_dict(), sched, artifact_tensors(path))
    seq = g["forced_sequence"][:ROWS]
    states = [m.new_state(seq.shape[1] + 1, seq[r, :1]) for r in range(ROWS)]

    def step(i, tokens):
        _, lg, _ = m.step(states, tokens, 1.0, True)
        for r in range(ROWS):
            states[r]["counts"][seq[r, i + 1]] += 1
        return lg

    got, top = teacher_forced_probe_logits(step, seq, g["probe_index"])
    check_within_envelope(got, g, ROWS)
    env_max = reference_envelope(g)[0]
    ref_top = g["forced_b0_top_index"][:ROWS, :, 0]
    margin = g["forced_b0_top_values"][:ROWS, :, 0] - g["forced_b0_top_values"][:ROWS, :, 1]
    clear = margin > 2 * env_max
    assert np.array_equal(top[clear], ref_top[clear])
