"""Prefix cache of the engine (CpuEngine::register_prefix / find_prefix,
cpu_engine_prefix.inl:11-96; CpuRequestSpec::prefix restored in initialize,
cpu_engine.inl:386-407) on the small hybrid model.

Chunked prefill leaves the state that single-token steps leave, bit for bit,
so a request that restores a prefix snapshot and shares its KV pages must
produce exactly the tokens of the same request prefilled from scratch: with
the prefix ending inside a page (the shared tail page is copied on the first
write, kv_pages.h:52-60) or on a page boundary, with two requests sharing one
prefix in the same decode batch, and for a complete hit (prompt == prefix)
whose first token comes from its own greedy head on the stored hidden row
(cpu_engine.inl:711-726), with and without a repetition penalty. The
from-scratch tokens are themselves checked against the CPU oracle, so a
prefix hit is tied to the restated reference step, not only to this engine.
In serving mode the same holds for automatic prefixes (register_prefix_tokens):
built once by the first request, attached by the requests that waited.""" 
import numpy as np
import pytest

from tests.model_util import build_small_model, oracle_greedy, small_dims, upload_model

pytestmark = pytest.mark.gpu

NEW = 6


@pytest.fixture(scope="module", params=["q4", "g16q8"])
def small(q, ctx, request):
    """The small hybrid model, with the default encodings and with the G16
    tied head plus Q8 gate rows (a complete hit runs the head itself)."""
    d, sched = small_dims()
    alt = request.param == "g16q8"
    tensors = build_small_model(d, sched, seed=13, head_g16=alt, q8_gates=alt)
    model = upload_model(q, ctx, d, sched, tensors)
    model.oracle = (d, sched, tensors)
    yield d, model
    model.close()


def engine(q, model, **kw):
    cfg = dict(max_resident_requests=4, max_context=96, max_decode_batch_size=4, prefill_chunk_size=8,
               page_tokens=16, use_graphs=False)
    cfg.update(kw)
    return q.Engine(model, **cfg)


def drain(q, eng, ids):
    """Prefill every request, then decode them together until all finish."""
    eng.prefill_batch([i for i in ids if q.REQ_STATUS[eng.result(i)[0].status] == "prefill"])
    while True:
        active = [i for i in ids if q.REQ_STATUS[eng.result(i)[0].status] == "decode"]
        if not active:
            break
        eng.advance_batch(active)
    return [eng.result(i) for i in ids]


def reference_tokens(q, model, prompts, penalty=1.0):
    """The tokens of the same requests prefilled from scratch on the HIP
    engine, each checked against the CPU oracle's greedy decode
    (oracle/q35_oracle.c, the restated reference step)."""
    eng = engine(q, model)
    ids = [eng.submit(p, NEW, penalty) for p in prompts]
    out = [toks for _, toks in drain(q, eng, ids)]
    eng.close()
    d, sched, tensors = model.oracle
    for p, toks in zip(prompts, out):
        np.testing.assert_array_equal(toks, oracle_greedy(d, sched, tensors, p[None, :], NEW, penalty)[0])
    return out


@pytest.mark.parametrize("plen", [24, 32])
def test_prefix_hit_equals_full_prefill(q, small, plen):
    d, model = small
    rng = np.random.default_rng(plen)
    shared = rng.integers(0, d["vocab"], size=plen).astype(np.int32)
    prompts = [np.concatenate([shared, rng.integers(0, d["vocab"], size=n).astype(np.int32)]) for n in (9, 14)]
    want = reference_tokens(q, model, prompts)
    eng = engine(q, model)
    free0 = eng.free_pages()
    print(f"prefix hit plen={plen}", flush=True)
    h = eng.register_prefix(shared, "tenant-a")
    assert h != 0
    ids = [eng.submit(p, NEW, prefix=h) for p in prompts]
    results = drain(q, eng, ids)
    for (res, toks), ref, p in zip(results, want, prompts):
        np.testing.assert_array_equal(toks, ref)
        assert res.cached_prefix_tokens == plen
        assert res.prefill_tokens == p.size - plen
    # the prefix's pages stay shared and intact: a third request still matches
    rid = eng.submit(prompts[0], NEW, prefix=h)
    np.testing.assert_array_equal(drain(q, eng, [rid])[0][1], want[0])
    for i in ids + [rid]:
        eng.release(i)
    eng.release_prefix(h)
    # only the cached prefix's own pages remain allocated
    assert eng.free_pages() == free0 - (plen + 15) // 16
    st = eng.prefix_stats()
    assert st["prefix_builds"] == 1 and st["prefix_hits"] == 3 and st["prefix_entries"] == 1
    eng.close()


@pytest.mark.parametrize("penalty", [1.0, 1.3])
def test_complete_hit_runs_its_own_head(q, small, penalty):
    d, model = small
    prompt = np.random.default_rng(7).integers(0, d["vocab"], size=21).astype(np.int32)
    want = reference_tokens(q, model, [prompt], penalty)[0]
    eng = engine(q, model)
    print(f"complete prefix hit penalty={penalty}", flush=True)
    h = eng.register_prefix(prompt, "tenant-a")
    rid = eng.submit(prompt, NEW, penalty, prefix=h)
    res, toks = drain(q, eng, [rid])[0]
    np.testing.assert_array_equal(toks, want)
    assert res.cached_prefix_tokens == prompt.size and res.prefill_tokens == 0
    eng.close()


def test_find_dedup_evict_and_errors(q, small):
    d, model = small
    t = np.random.default_rng(3).integers(0, d["vocab"], size=40).astype(np.int32)
    eng = engine(q, model)
    free0 = eng.free_pages()
    print("prefix find / dedup / errors", flush=True)
    h16 = eng.register_prefix(t[:16], "a")
    h24 = eng.register_prefix(t[:24], "a")
    assert eng.register_prefix(t[:24], "a") == h24  # exact tokens and namespace: the same snapshot
    assert eng.find_prefix(t[:30], "a") == (h24, 24)
    assert eng.find_prefix(t[:20], "a") == (h16, 16)
    assert eng.find_prefix(t, "b") == (0, 0)
    assert eng.find_prefix(t[1:], "a") == (0, 0)
    with pytest.raises(q.Q35Error):
        eng.submit(t[1:30], NEW, prefix=h24)  # the prompt does not start with the prefix
    with pytest.raises(q.Q35Error):
        eng.register_prefix(t[:8], "")  # a trust namespace is required
    for h in (h16, h24, h24, h24, h16):  # register x3 + find x2 pins
        eng.release_prefix(h)
    with pytest.raises(q.Q35Error):
        eng.release_prefix(h24)  # no pins left
    assert eng.prefix_stats()["prefix_builds"] == 2
    eng.close()
    # a budget that holds one prefix: the unpinned one is evicted for the next
    eng = engine(q, model, max_prefix_bytes=1_000_000)
    free0 = eng.free_pages()
    a = eng.register_prefix(t[:16], "a")
    with pytest.raises(q.Q35Error):
        eng.register_prefix(t[:12], "a")  # the pinned prefix cannot be evicted
    eng.release_prefix(a)
    b = eng.register_prefix(t[:12], "a")
    st = eng.prefix_stats()
    assert st["prefix_evictions"] == 1 and st["prefix_entries"] == 1
    assert eng.find_prefix(t, "a") == (b, 12)
    assert eng.free_pages() == free0 - 1
    eng.close()


def serve(eng, ids):
    """Drives a serving-mode engine through step() and read_output."""
    got = {i: [] for i in ids}
    for _ in range(500):
        eng.step()
        for i in ids:
            got[i] += eng.read_output(i).tolist()
        if all(eng.terminal(i) and len(got[i]) == eng.result(i)[1].size for i in ids):
            break
    return got


@pytest.mark.parametrize("plen", [40, 48])
def test_automatic_prefix_single_flight(q, small, plen):
    """register_prefix_tokens in serving mode (cpu_engine_singleflight.inl:
    same_build, prefix_admissible, publish_prefix; cpu_engine.inl:737-760): of
    three queued requests sharing a plen-token prefix, the first is admitted
    and builds it, the other two wait while it is building (not admitted
    although slots are free), then attach the published prefix. Every
    request's tokens equal the cold run's bit for bit; the builder reports
    plen newly written tokens, the others plen cached ones. A prefix ending
    inside a page (40) leaves a shared tail page that the builder itself
    copies on its next write."""
    d, model = small
    rng = np.random.default_rng(17 + plen)
    shared = rng.integers(0, d["vocab"], size=plen).astype(np.int32)
    prompts = [np.concatenate([shared, rng.integers(0, d["vocab"], size=n).astype(np.int32)]) for n in (9, 14, 5)]
    # the cold run on the same engine in direct mode, tied to the oracle up to
    # the first near-tie (greedy top-2 margin below 0.1: the kernels and the
    # oracle round differently inside the 1e-3 stage tolerance)
    cold = engine(q, model)
    want = [toks for _, toks in drain(q, cold, [cold.submit(p, NEW) for p in prompts])]
    cold.close()
    dd, sched, tensors = model.oracle
    for p, toks in zip(prompts, want):
        ref, lg = oracle_greedy(dd, sched, tensors, p[None, :], NEW, 1.0, want_logits=True)
        for n in range(NEW):
            if toks[n] != ref[0, n]:
                top2 = np.sort(lg[0, n])[-2:]
                assert top2[1] - top2[0] < 0.1, (n, toks, ref[0])
                break
    eng = engine(q, model, max_queued_requests=8, max_prefill_requests=3)
    print(f"automatic prefix plen={plen}", flush=True)
    ids = [eng.submit_spec(p, NEW, temperature=0.0, repetition_penalty=1.0, register_prefix_tokens=plen,
                           trust_namespace="tenant-s") for p in prompts]
    eng.step()  # admits only the builder: the others share its build
    st = eng.stats()
    assert st["resident_requests"] == 1 and st["queued_requests"] == 2
    got = serve(eng, ids)
    for k, (rid, ref) in enumerate(zip(ids, want)):
        res, toks = eng.result(rid)
        assert res.status == q.REQ_STATUS_INV["complete"]
        np.testing.assert_array_equal(toks, ref)
        assert got[rid] == toks.tolist()
        if k == 0:
            assert res.prefix_written_tokens == plen and res.cached_prefix_tokens == 0
        else:
            assert res.cached_prefix_tokens == plen and res.prefill_tokens == prompts[k].size - plen
    ps = eng.prefix_stats()
    assert ps["prefix_builds"] == 1 and ps["prefix_hits"] == 2 and ps["prefix_entries"] == 1
    h, n = eng.find_prefix(prompts[1], "tenant-s")
    assert n == plen
    eng.release_prefix(h)
    with pytest.raises(q.Q35Error):  # automatic builds need a namespace
        eng.submit_spec(prompts[0], NEW, register_prefix_tokens=plen)
    eng.close()
    direct = engine(q, model)
    with pytest.raises(q.Q35Error):  # and serving mode
        direct.submit_spec(prompts[0], NEW, register_prefix_tokens=plen, trust_namespace="t")
    direct.close()
