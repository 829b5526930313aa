"""The engine's packed scheduler against the reference's alternating one
(cpu_engine_scheduler.inl:64-80: a decode batch or one prefill chunk per
step), both in serving mode. With packed_steps, q35_engine_step runs the
decode batch and the next prompt chunks of up to max_prefill_requests
requests in one packed step. Without it the reference's rule holds: with
max_prefill_requests > 1 only short selected readouts share a prefill step
(shared_prefill, cpu_engine.inl:628-666). Every request must end with the
same tokens as under the plain alternating schedule, a logits-callback
request must see bit-identical raw logits at every position (its state and
KV agree throughout), and the selected readouts the same values, for
greedy, sampled, forced and selected-readout requests. The counters
(CpuEngineStats) record the packed and shared steps; physical_kv_bytes
follows the pages the requests hold."""
import numpy as np
import pytest

from tests.model_util import build_small_model, small_dims, upload_model

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def small(q, ctx):
    d, sched = small_dims()
    tensors = build_small_model(d, sched, seed=13)
    model = upload_model(q, ctx, d, sched, tensors)
    yield d, model
    model.close()


def run(q, model, d, packed, prefill_requests):
    rng = np.random.default_rng(31)
    prompts = [rng.integers(0, d["vocab"], size=n).astype(np.int32) for n in (37, 5, 90, 18, 64, 11)]
    eng = q.Engine(model, max_resident_requests=4, max_context=160, max_decode_batch_size=4, prefill_chunk_size=24,
                   page_tokens=16, max_prefill_requests=prefill_requests, packed_steps=packed, max_queued_requests=8)
    seen, selected = [], {}

    def cb(index, forced, logits):
        seen.append(logits.view(np.uint32).copy())
        return True

    def readout(key):
        def fn(index, forced, values):
            selected[key] = values.view(np.uint32).copy()
            return True
        return fn

    # two short selected readouts (cpu_engine.inl:628-631) first: admitted
    # together, they lead the prefill rotation
    ids = [eng.submit_spec(p, max_new_tokens=1, temperature=0.0, forced_output_tokens=[7],
                           selected_logit_tokens=[2, 9, 2, 40], selected_logits_callback=readout(k))
           for k, p in enumerate((prompts[1], prompts[5]))]
    ids += [eng.submit(prompts[0], max_new_tokens=12),
           eng.submit_spec(prompts[1], max_new_tokens=10, temperature=0.8, top_p=0.9, top_k=20, seed=5),
           eng.submit_spec(prompts[2], max_new_tokens=9, temperature=0.0, repetition_penalty=1.1,
                           logits_callback=cb),
           eng.submit(prompts[3], max_new_tokens=14, repetition_penalty=1.2),
           eng.submit_spec(prompts[4], max_new_tokens=6, temperature=1.1, top_k=0, seed=9),
           eng.submit_spec(prompts[5], max_new_tokens=5, forced_output_tokens=[3, 1, 4, 1, 5])]
    read = {rid: [] for rid in ids}
    for _ in range(2000):
        eng.step()
        for rid in ids:
            read[rid] += eng.read_output(rid).tolist()
        if all(eng.terminal(i) and len(read[i]) == eng.result(i)[1].size for i in ids):
            break
    outs = []
    for rid in ids:
        res, toks = eng.result(rid)
        assert res.status == q.REQ_STATUS_INV["complete"], (packed, prefill_requests, rid, res.status)
        assert read[rid] == toks.tolist()  # every token handed out once, in order
        outs.append(toks.tolist())
    stats = eng.stats()
    for rid in ids:
        eng.release(rid)
    assert eng.stats()["physical_kv_bytes"] == 0
    eng.close()
    return outs, seen, stats, selected


def test_packed_and_shared_steps_equal_alternating(q, ctx, small):
    d, model = small
    print("engine: alternating schedule", flush=True)
    base, base_seen, base_stats, base_sel = run(q, model, d, False, 1)
    assert base_stats["packed_ticks"] == 0 and base_stats["shared_prefill_ticks"] == 0
    assert base_stats["batch_ticks"] > 0 and base_stats["batch_rows"] >= base_stats["batch_ticks"]
    assert base_stats["lm_head_batches"] >= base_stats["batch_ticks"]
    assert sorted(base_sel) == [0, 1]
    for packed, shared in ((True, 1), (False, 3), (True, 3)):
        print(f"engine: packed={packed} max_prefill_requests={shared}", flush=True)
        outs, seen, stats, sel = run(q, model, d, packed, shared)
        assert outs == base, (packed, shared)
        assert len(seen) == len(base_seen)
        for a, b in zip(seen, base_seen):
            np.testing.assert_array_equal(a, b)
        for k in (0, 1):
            np.testing.assert_array_equal(sel[k], base_sel[k])
        assert (stats["packed_ticks"] > 0) == packed
        # without packed steps only the two short readouts share a step
        assert (stats["shared_prefill_ticks"] > 0) == (shared > 1)
        if not packed and shared > 1:
            assert stats["shared_prefill_requests"] == 2 * stats["shared_prefill_ticks"]
        if packed:
            assert stats["packed_rows"] > stats["packed_ticks"]


def test_stats_count_forwards_and_pages(q, ctx, small):
    d, model = small
    n_layers = d["n_layers"]
    eng = q.Engine(model, max_resident_requests=2, max_context=64, max_decode_batch_size=2, prefill_chunk_size=32,
                   page_tokens=16)
    a = eng.submit(np.arange(20, dtype=np.int32), max_new_tokens=4)
    b = eng.submit(np.arange(5, dtype=np.int32), max_new_tokens=4)
    eng.prefill_batch([a, b])
    s0 = eng.stats()
    # one chunk each: a forward per chunk (4 projections and a state batch per
    # layer, the greedy head); pages 2 + 1 of K and V rows per full layer
    assert s0["lm_head_batches"] == 2 and s0["greedy_lm_head_batches"] == 2
    assert s0["projection_batches"] == 2 * (4 * n_layers + 1) and s0["state_batches"] == 2 * n_layers
    page_bytes = 16 * d["n_kv_heads"] * d["head_dim"] * 2 * 2 * 1  # one full-attention layer
    assert s0["physical_kv_bytes"] == 3 * page_bytes
    assert s0["resident_requests"] == 2 and s0["queued_requests"] == 0
    eng.advance_batch([a, b])
    s1 = eng.stats()
    assert s1["batch_ticks"] == 1 and s1["batch_rows"] == 2
    assert s1["projection_batches"] - s0["projection_batches"] == 4 * n_layers + 1
    eng.close()
