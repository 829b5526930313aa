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


def test_step_timing_keeps_graph_steps(q, small):
    """q35_runtime_set_step_timing brackets each step's graph replay with HIP
    events: the steps keep their tokens (the graphs still run), every decode
    step is counted once, and the GPU time it sums is positive and below the
    wall time of the same steps."""
    import time
    d, sched, tensors, model, prompts, refs = small
    eng = q.Engine(model, max_resident_requests=4, max_context=64, max_decode_batch_size=4, page_tokens=16)
    ids = [eng.submit(p, max_new_tokens=NEW) for p in prompts]
    eng.prefill_batch(ids)
    eng.advance_batch(ids)  # the step's graph is captured outside the timed steps
    eng.set_step_timing(True)
    t = time.perf_counter()
    for _ in range(NEW - 2):
        eng.advance_batch(ids)
    wall_ms = (time.perf_counter() - t) * 1000.0
    gpu_ms, steps = eng.step_timing()
    print(f"step timing: {gpu_ms:.3f} ms of GPU time in {wall_ms:.3f} ms over {steps} steps", flush=True)
    assert steps == NEW - 2
    assert 0.0 < gpu_ms < wall_ms
    eng.set_step_timing(False)
    assert eng.step_timing() == (0.0, 0)
    for rid, ref in zip(ids, refs):
        res, toks = eng.result(rid)
        assert res.status == q.REQ_STATUS_INV["complete"] and toks.size == NEW
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


def serve(eng, ids, steps=500, read=1 << 20):
    """Drives a serving-mode engine through step(), reading every request's
    output after each step as server.cpp:275-300 does: the tokens read."""
    got = {i: [] for i in ids}
    for _ in range(steps):
        eng.step()
        for i in ids:
            got[i] += eng.read_output(i, read).tolist()
        if all(eng.terminal(i) and len(got[i]) == eng.result(i)[1].size for i in ids):
            break
    return got


def test_scheduler_step_drains(q, small):
    d, sched, tensors, model, prompts, refs = small
    # serving mode, two resident slots for four queued requests: admission
    # waits for retirement
    eng = q.Engine(model, max_resident_requests=2, max_context=64, max_decode_batch_size=2,
                   prefill_chunk_size=5, page_tokens=16, max_queued_requests=4)
    ids = [eng.submit(p, max_new_tokens=NEW) for p in prompts]
    st = eng.stats()
    assert st["queued_requests"] == 4 and st["resident_requests"] == 0  # queued requests hold no device state
    got = serve(eng, ids, read=2)
    for rid, ref in zip(ids, refs):
        res, toks = eng.result(rid)
        assert res.status == q.REQ_STATUS_INV["complete"], res.status
        check_tokens(toks, ref)
        assert got[rid] == toks.tolist()
        assert res.queue_ms >= 0.0
    assert eng.stats()["resident_requests"] == 0  # terminal requests retire at once in serving mode
    eng.close()


def test_serving_mode_contract(q, small):
    """CpuEngine's two modes (cpu_engine.inl:832-948,
    cpu_engine_scheduler.inl:2-127): step and read_output only in serving
    mode, advance and advance_batch only outside it; the record limit and
    the bounded queue; stop sequences longer than the output buffer are
    rejected; a request whose unread output reaches max_buffered_tokens is
    not scheduled until read_output drains it; a token that may start a stop
    sequence is held back by read_output until the next token resolves it."""
    d, sched, tensors, model, prompts, refs = small
    E = q.Q35Error
    direct = q.Engine(model, max_resident_requests=2, max_context=64, max_decode_batch_size=2, page_tokens=16)
    a = direct.submit(prompts[1], max_new_tokens=NEW)
    with pytest.raises(E, match="step requires serving mode"):
        direct.step()
    with pytest.raises(E, match="read_output requires serving mode"):
        direct.read_output(a)
    direct.submit(prompts[0], max_new_tokens=NEW)
    with pytest.raises(E):
        direct.submit(prompts[2], max_new_tokens=NEW)  # direct mode: at most max_resident_requests records
    direct.close()
    with pytest.raises(E):
        q.Engine(model, max_resident_requests=1, max_context=64, max_decode_batch_size=2, page_tokens=16,
                 max_queued_requests=2, max_buffered_tokens=0)

    eng = q.Engine(model, max_resident_requests=1, max_context=64, max_decode_batch_size=2, page_tokens=16,
                   max_queued_requests=2, max_buffered_tokens=2)
    with pytest.raises(E, match="Queue full or stop sequence"):
        eng.submit_spec(prompts[0], NEW, temperature=0.0, stop_sequences=[[1, 2, 3]])
    a = eng.submit(prompts[1], max_new_tokens=NEW)
    b = eng.submit(prompts[3], max_new_tokens=NEW)
    with pytest.raises(E, match="Queue full"):
        eng.submit(prompts[0], max_new_tokens=NEW)
    with pytest.raises(E, match="Serving mode must be driven through step"):
        eng.advance(a)
    with pytest.raises(E, match="Serving mode must be driven through step"):
        eng.advance_batch([a])
    for _ in range(20):
        eng.step()
    res, toks = eng.result(a)
    assert toks.size == 2 and res.status == q.REQ_STATUS_INV["decode"]  # two unread tokens: a waits
    assert eng.result(b)[0].status == q.REQ_STATUS_INV["queued"]  # one resident slot
    assert eng.read_output(a, 1).tolist() == toks[:1].tolist()
    for _ in range(20):
        eng.step()
    assert eng.result(a)[1].size == 3  # one token of room, one more token
    got = serve(eng, [a, b])
    for rid, k in ((a, 1), (b, 3)):
        res, toks = eng.result(rid)
        assert res.status == q.REQ_STATUS_INV["complete"]
        check_tokens(toks, refs[k])
    assert [int(t) for t in eng.result(a)[1][:1]] + got[a] == eng.result(a)[1].tolist()
    assert got[b] == eng.result(b)[1].tolist()
    eng.close()

    # a stop sequence [t2, x] with x never generated after t2: read_output
    # holds t2 back until the next token shows the sequence does not match
    eng = q.Engine(model, max_resident_requests=2, max_context=64, max_decode_batch_size=2, page_tokens=16,
                   max_queued_requests=2)
    free = serve(eng, [eng.submit(prompts[1], max_new_tokens=NEW)])
    toks = list(free.values())[0]
    stop = [toks[2], (toks[3] + 1) % d["vocab"]]
    c = eng.submit_spec(prompts[1], NEW, temperature=0.0, repetition_penalty=1.0, stop_sequences=[stop])
    seen = []
    for _ in range(50):
        eng.step()
        n = eng.result(c)[1].size
        if n == 3:
            seen.append(eng.read_output(c).tolist())
        if n == 4:
            seen.append(eng.read_output(c).tolist())
            break
    assert seen == [toks[:2], toks[2:4]], (seen, toks)
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
