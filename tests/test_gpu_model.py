"""Whole decode step on the GPU against the oracle's restatement of
forward_batch (cpu_engine.inl:201-325) on a small hybrid model: greedy tokens
identical (margin-aware), raw logits within 1e-2 max-abs; graph replay
identical to eager launches."""
import numpy as np
import pytest

from tests.model_util import build_small_model, hip_greedy, oracle_greedy, small_dims, upload_model

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def small(q, ctx):
    d, sched = small_dims()
    tensors = build_small_model(d, sched, seed=5)
    model = upload_model(q, ctx, d, sched, tensors)
    yield d, sched, tensors, model
    model.close()


def test_greedy_tokens_and_logits(q, ctx, orc, small):
    d, sched, tensors, model = small
    prompts = np.random.default_rng(1).integers(0, d["vocab"], size=(5, 24)).astype(np.int32)
    print("small model: oracle", flush=True)
    want, want_lg = oracle_greedy(d, sched, tensors, prompts, 8, want_logits=True)
    print("small model: HIP", flush=True)
    got, got_lg = hip_greedy(q, ctx, d, sched, tensors, prompts, 8, want_logits=True, model=model)
    assert np.max(np.abs(got_lg[:, 0] - want_lg[:, 0])) < 1e-2
    # teacher-forced comparison is not available here, so compare while the
    # sequences agree, requiring agreement wherever the oracle's margin is clear
    for r in range(prompts.shape[0]):
        for n in range(8):
            top2 = np.sort(want_lg[r, n])[-2:]
            if got[r, n] != want[r, n]:
                assert top2[1] - top2[0] < 1e-2, (r, n)
                break
            assert np.max(np.abs(got_lg[r, n] - want_lg[r, n])) < 1e-2, (r, n)


def test_greedy_path_matches_logits_path(q, ctx, small):
    d, sched, tensors, model = small
    prompts = np.random.default_rng(2).integers(0, d["vocab"], size=(4, 10)).astype(np.int32)
    greedy = hip_greedy(q, ctx, d, sched, tensors, prompts, 6, model=model)
    via_logits, _ = hip_greedy(q, ctx, d, sched, tensors, prompts, 6, want_logits=True, model=model)
    assert np.array_equal(greedy, via_logits)


def test_graph_replay_equals_eager(q, ctx, small):
    d, sched, tensors, model = small
    prompts = np.random.default_rng(3).integers(0, d["vocab"], size=(3, 12)).astype(np.int32)
    a, la = hip_greedy(q, ctx, d, sched, tensors, prompts, 5, want_logits=True, use_graphs=True, model=model)
    b, lb = hip_greedy(q, ctx, d, sched, tensors, prompts, 5, want_logits=True, use_graphs=False, model=model)
    assert np.array_equal(a, b) and np.array_equal(la, lb)


def test_penalty_and_page_sizes(q, ctx, orc, small):
    d, sched, tensors, model = small
    prompts = np.random.default_rng(4).integers(0, 64, size=(2, 20)).astype(np.int32)
    want, want_lg = oracle_greedy(d, sched, tensors, prompts, 6, penalty=1.3, want_logits=True)
    for pt in (1, 16, 64):
        got = hip_greedy(q, ctx, d, sched, tensors, prompts, 6, penalty=1.3, page_tokens=pt, model=model)
        for r in range(2):
            for n in range(6):
                if got[r, n] != want[r, n]:
                    top2 = np.sort(want_lg[r, n])[-2:]
                    assert top2[1] - top2[0] < 5e-2
                    break
