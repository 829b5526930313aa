"""The G16 head (Q4G16Tile, q4_g16_matmul_wide order) at the 0.8B hidden
width, where 16-token tiles of staged activations fit the head workgroup's
LDS only three at a time: batches above 48 rows run as several launches at
one grid. Greedy tokens must equal argmax of the logits path, and both must
follow the oracle."""
import numpy as np
import pytest

from tests.model_util import build_small_model, hip_greedy, oracle_envelope, small_dims, upload_model

pytestmark = pytest.mark.gpu


def test_g16_head_token_chunks(q, ctx, orc):
    d, _ = small_dims()
    d = dict(d, hidden=1024, intermediate=512, n_layers=2)
    sched = np.array([1, 0], np.uint8)
    tensors = build_small_model(d, sched, seed=11, head_g16=True, q8_gates=True)
    model = upload_model(q, ctx, d, sched, tensors)
    try:
        prompts = np.random.default_rng(12).integers(0, d["vocab"], size=(52, 3)).astype(np.int32)
        print("g16 head: 52 rows, HIP greedy", flush=True)
        greedy = hip_greedy(q, ctx, d, sched, tensors, prompts, 3, model=model)
        print("g16 head: HIP logits path", flush=True)
        via, lg = hip_greedy(q, ctx, d, sched, tensors, prompts, 3, want_logits=True, model=model)
        assert np.array_equal(greedy, via)
        assert np.array_equal(via[:, 0], np.argmax(lg[:, 0], axis=1))
        print("g16 head: oracle and its envelope", flush=True)
        want_lg, want, env_max, env_mean = oracle_envelope(d, sched, tensors, prompts, 3)
        diff = np.abs(lg[:, 0] - want_lg[:, 0])
        print(f"g16 head: envelope max {env_max:.4f} mean {env_mean:.5f}; HIP vs oracle max {diff.max():.4f} "
              f"mean {diff.mean():.5f}", flush=True)
        assert diff.max() <= 1.5 * env_max + 1e-3 and diff.mean() <= 1.5 * env_mean + 1e-4
        top2 = np.sort(want_lg[:, 0], axis=1)[:, -2:]
        clear = top2[:, 1] - top2[:, 0] > env_max
        assert np.array_equal(via[clear, 0], want[clear, 0])
    finally:
        model.close()
