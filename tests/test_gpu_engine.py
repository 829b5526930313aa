"""The request-level engine (q35_engine_*, the CpuEngine mirror) on the small
hybrid model: ragged prompts prefilled together, one by one in chunks, or by
the serving scheduler all give the oracle's greedy tokens; stop ids, cancel,
release, KV page accounting and the reference's error contract
(cpu_engine.inl:832-1017, tests/cpu_engine_test.cpp patterns)."""
import numpy as np
import pytest

from tests.model_util import build_small_model, oracle_greedy, small_dims, upload_model

pytestmark = pytest.mark.gpu

NEW = 6


@pytest.fixture(scope="module")
def small(q, ctx):
    d, sched = small_dims()
    tensors = build_small_model(d, sched, seed=11)
    model = upload_model(q, ctx, d, sched, tensors)
    rng = np.random.default_rng(21)
    prompts = [rng.integers(0, d["vocab"], size=n).astype(np.int32) for n in (3, 17, 1, 9)]
    refs = [oracle_greedy(d, sched, tensors, p[None, :], NEW, want_logits=True) for p in prompts]
    yield d, sched, tensors, model, prompts, refs
    model.close()


def check_tokens(got, ref):
    """Equal to the oracle's greedy tokens up to the first near-tie."""
    want, logits = ref
    for n in range(NEW):
        if got[n] != want[0, n]:
            top2 = np.sort(logits[0, n])[-2:]
            assert top2[1] - top2[0] < 1e-2, (n, got, want)
            return


def test_prefill_batch_then_advance_batch(q, small):
    d, sched, tensors, model, prompts, refs = small
    eng = q.Engine(model, max_resident_requests=4, max_context=64, max_decode_batch_size=4, page_tokens=16)
    ids = [eng.submit(p, max_new_tokens=NEW) for p in prompts]
    eng.prefill_batch(ids)
    for _ in range(NEW - 1):
        eng.advance_batch(ids)
    for rid, ref in zip(ids, refs):
        res, toks = eng.result(rid)
        assert res.status == q.REQ_STATUS_INV["complete"] and toks.size == NEW
        assert res.decode_forwards == NEW - 1
        check_tokens(toks, ref)
    eng.close()


def test_chunked_advance_matches(q, small):
    d, sched, tensors, model, prompts, refs = small
    eng = q.Engine(model, max_resident_requests=2, max_context=64, max_decode_batch_size=2,
                   prefill_chunk_size=4, page_tokens=4, use_graphs=False)
    for p, ref in zip(prompts, refs):
        rid = eng.submit(p, max_new_tokens=NEW)
        while eng.result(rid)[0].status == q.REQ_STATUS_INV["prefill"]:
            eng.advance(rid)
        while eng.result(rid)[0].status == q.REQ_STATUS_INV["decode"]:
            eng.advance(rid)
        res, toks = eng.result(rid)
        assert res.prefill_tokens == p.size and res.committed_tokens >= p.size
        check_tokens(toks, ref)
        eng.release(rid)
    eng.close()


def test_scheduler_step_drains(q, small):
    d, sched, tensors, model, prompts, refs = small
    # two resident slots for four requests: admission must wait for retirement
    eng = q.Engine(model, max_resident_requests=2, max_context=64, max_decode_batch_size=2,
                   prefill_chunk_size=5, page_tokens=16)
    ids = [eng.submit(p, max_new_tokens=NEW) for p in prompts]
    for _ in range(500):
        if not eng.step():
            break
    for rid, ref in zip(ids, refs):
        res, toks = eng.result(rid)
        assert res.status == q.REQ_STATUS_INV["complete"], res.status
        check_tokens(toks, ref)
    eng.close()


def test_stop_cancel_release_and_errors(q, small):
    d, sched, tensors, model, prompts, refs = small
    st = q.REQ_STATUS_INV
    eng = q.Engine(model, max_resident_requests=3, max_context=32, max_decode_batch_size=2, page_tokens=16)
    free0 = q.lib.q35_runtime_free_pages(eng._rt())
    # the stop id is the oracle's second token: generation ends before it, without it (select(), cpu_engine.inl:441-487)
    want, logits = refs[1]
    stop = int(want[0, 1])
    first = list(want[0]).index(stop)
    a = eng.submit(prompts[1], max_new_tokens=NEW, stop_token_ids=[stop])
    eng.prefill_batch([a])
    while eng.result(a)[0].status == st["decode"]:
        eng.advance_batch([a])
    res, toks = eng.result(a)
    margins = [np.diff(np.sort(logits[0, n])[-2:])[0] for n in range(first + 1)]
    if min(margins) > 1e-2:
        assert res.status == st["complete"] and toks.tolist() == want[0, :first].tolist()
    b = eng.submit(prompts[0], max_new_tokens=NEW)
    eng.cancel(b)
    assert eng.result(b)[0].status == st["cancelled"]
    with pytest.raises(q.Q35Error):
        eng.advance(b)  # not active
    with pytest.raises(q.Q35Error):
        eng.advance(999)  # unknown id
    c = eng.submit(prompts[2], max_new_tokens=NEW)
    eng.prefill_batch([c])
    with pytest.raises(q.Q35Error):
        eng.advance_batch([c, c])  # duplicate rows
    with pytest.raises(q.Q35Error):
        eng.submit(np.array([d["vocab"]], np.int32))  # token out of range
    with pytest.raises(q.Q35Error):
        eng.submit(prompts[1], max_new_tokens=40)  # exceeds max_context
    eng.advance_batch([c])  # still usable after rejected calls
    assert eng.result(c)[1].size == 2
    for rid in (a, b, c):
        eng.release(rid)
    with pytest.raises(q.Q35Error):
        eng.result(a)
    assert q.lib.q35_runtime_free_pages(eng._rt()) == free0  # every KV page back in the pool
    eng.close()
