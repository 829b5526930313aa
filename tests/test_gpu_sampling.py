"""Sampled decoding on the GPU (sample_token_from_logits, layers.inl:491-600;
select, cpu_engine.inl:441-487) on the small hybrid model.

The device selects each row's top_k candidates of the penalized,
temperature-scaled logits; the engine finishes softmax, top_p and the draw on
the host. Checks:
- candidate lists bit-exact against a numpy restatement of the same rows
  (penalty, scaling, descending order with ties to the lower token);
- every sampled token equal to oracle/sampling.py's restatement (pinned
  against the reference engine in tests/test_oracle_sampling.py) applied to
  the raw logits the request's logits callback saw and the request's counts,
  from the same seed -- with top_k on the device path, top_k 0 on the full-row
  path, temperature 0 with a callback, and rows of different kinds in one batch;
- forced output tokens, callback arguments and failures, stop sequences."""
import numpy as np
import pytest

from oracle.sampling import MT19937, sample_token
from tests.model_util import build_small_model, small_dims, upload_model

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", params=["q4", "g16q8"])
def small(q, ctx, request):
    """The small hybrid model with the default encodings, and with the G16
    tied head plus Q8 gate rows (the head_candidates path must use the
    head's own tile format)."""
    d, sched = small_dims()
    alt = request.param == "g16q8"
    tensors = build_small_model(d, sched, seed=17, head_g16=alt, q8_gates=alt)
    model = upload_model(q, ctx, d, sched, tensors)
    yield d, model
    model.close()


def test_head_candidates_equal_step_logits(q, small):
    """q35_runtime_head_candidates (the first token after a prefill or on a
    complete prefix hit) runs the head on a stored final hidden row: its raw
    logits and candidates must equal the logits path of the step that
    produced the row, bit for bit, and q35_runtime_head its argmax."""
    d, model = small
    rt = q.Runtime(model, max_slots=1, max_batch=1, max_context=32, page_tokens=16, use_graphs=False)
    prompt = np.random.default_rng(21).integers(0, d["vocab"], size=6).astype(np.int32)
    slot = rt.slot_alloc(prompt)
    table = np.array([[rt.page_alloc()]], np.int32)
    print("head_candidates vs step logits", flush=True)
    for t in range(prompt.size):
        last = t == prompt.size - 1
        res = rt.step([slot], [t], [prompt[t]], table, logits=last)
    want = res[1][0]
    hidden = rt.last_hidden(1)[0]
    cand, raw = rt.head_candidates(slot, hidden, 64, 1.0, raw_logits=True)
    np.testing.assert_array_equal(raw.view(np.uint32), want.view(np.uint32))
    order = np.lexsort((np.arange(want.size), -want.astype(np.float64)))[:64]
    np.testing.assert_array_equal(cand["token"], order)
    np.testing.assert_array_equal(cand["value"].view(np.uint32), want[order].view(np.uint32))
    assert rt.head(slot, hidden) == int(order[0])
    rt.close()


def engine(q, model, **kw):
    cfg = dict(max_resident_requests=4, max_context=96, max_decode_batch_size=4, prefill_chunk_size=8,
               page_tokens=16, use_graphs=True)
    cfg.update(kw)
    return q.Engine(model, **cfg)


def drain(q, eng, ids):
    """Runs the requests to the end; a call that reports a failed row (the
    reference's advance_batch returns false, cpu_engine.inl:1006-1013) still
    leaves the other rows advanced, so the loop goes on."""
    while True:
        states = {i: q.REQ_STATUS[eng.result(i)[0].status] for i in ids}
        pre = [i for i in ids if states[i] == "prefill"]
        active = [i for i in ids if states[i] == "decode"]
        if not pre and not active:
            return [eng.result(i) for i in ids]
        try:
            if pre:
                eng.prefill_batch(pre)
            else:
                eng.advance_batch(active)
        except q.Q35Error:
            pass


def test_candidates_match_restatement(q, small):
    d, model = small
    rt = q.Runtime(model, max_slots=3, max_batch=3, max_context=64, page_tokens=16, use_graphs=False)
    rng = np.random.default_rng(5)
    prompts = [rng.integers(0, d["vocab"], size=n).astype(np.int32) for n in (5, 9, 3)]
    slots = [rt.slot_alloc(p) for p in prompts]
    table = np.array([[rt.page_alloc()] for _ in slots], np.int32)
    pos = np.zeros(3, np.int32)
    toks = np.array([p[0] for p in prompts], np.int32)
    top_k = np.array([1, 20, 64], np.int32)
    inv_t = np.array([1.0, 1 / 0.7, 1 / 1.3], np.float32)
    pen = np.array([1.3, 1.05, 1.0], np.float32)
    print("candidate lists vs restatement", flush=True)
    for step in range(3):
        cand, raw = rt.step_candidates(slots, pos, toks, table, top_k, inv_t, penalties=pen, raw_logits=True)
        for r in range(3):
            v = raw[r].copy()
            counts = rt.slot_counts(slots[r])
            if pen[r] > 1:
                m = counts > 0
                v[m] = np.where(v[m] > 0, v[m] / pen[r], v[m] * pen[r])
            v = (v * inv_t[r]).astype(np.float32)
            order = np.lexsort((np.arange(v.size), -v.astype(np.float64)))[:top_k[r]]
            np.testing.assert_array_equal(cand[r]["token"][:top_k[r]], order)
            np.testing.assert_array_equal(cand[r]["value"][:top_k[r]].view(np.uint32), v[order].view(np.uint32))
            assert np.all(cand[r]["token"][top_k[r]:] == -1)
        pos += 1
        toks = cand["token"][:, 0].astype(np.int32)
    rt.close()


CONFIGS = [(0.7, 0.8, 20, 1.05, 1234), (1.0, 1.0, 0, 1.0, 7), (0.0, 1.0, 0, 1.2, 5), (1.2, 0.5, 3, 1.0, 31),
           (0.8, 0.9, 64, 1.1, 2)]


@pytest.mark.parametrize("temperature,top_p,top_k,penalty,seed", CONFIGS)
def test_engine_sampling_matches_restatement(q, small, temperature, top_p, top_k, penalty, seed):
    d, model = small
    vocab = d["vocab"]
    prompt = np.random.default_rng(seed).integers(0, vocab, size=11).astype(np.int32)
    new = 10
    seen = {}

    def callback(index, forced, logits):
        assert forced == -1 and logits.size == vocab
        seen[index] = logits
        return True

    eng = engine(q, model)
    print(f"sampling t={temperature} p={top_p} k={top_k} pen={penalty}", flush=True)
    rid = eng.submit_spec(prompt, new, temperature, top_p, top_k, penalty, seed, logits_callback=callback)
    res, toks = drain(q, eng, [rid])[0]
    assert q.REQ_STATUS[res.status] == "complete" and toks.size == new
    counts = np.bincount(prompt, minlength=vocab)
    mt = MT19937(seed)
    for s in range(new):
        want = sample_token(seen[s], counts, temperature, top_p, top_k, penalty, mt)
        assert toks[s] == want, (s, toks[s], want)
        counts[toks[s]] += 1
    eng.close()


def test_mixed_batch_keeps_greedy_rows_exact(q, small):
    """A greedy row decoded beside sampled rows (the step takes the candidate
    path for the whole batch) gives the tokens of an all-greedy run."""
    d, model = small
    rng = np.random.default_rng(9)
    p_greedy, p_a, p_b = (rng.integers(0, d["vocab"], size=n).astype(np.int32) for n in (7, 13, 4))
    eng = engine(q, model)
    want = drain(q, eng, [eng.submit(p_greedy, 8, 1.1)])[0][1]
    eng.close()
    eng = engine(q, model)
    print("mixed greedy + sampled batch", flush=True)
    ids = [eng.submit(p_greedy, 8, 1.1), eng.submit_spec(p_a, 8, 0.9, 0.9, 40, 1.0, 3),
           eng.submit_spec(p_b, 8, 1.1, 1.0, 0, 1.2, 4)]
    results = drain(q, eng, ids)
    np.testing.assert_array_equal(results[0][1], want)
    assert all(r.status == q.REQ_STATUS_INV["complete"] for r, _ in results)
    eng.close()


def test_forced_callback_failure_and_stop_sequences(q, small):
    d, model = small
    rng = np.random.default_rng(12)
    prompt = rng.integers(0, d["vocab"], size=6).astype(np.int32)
    forced = rng.integers(0, d["vocab"], size=5).astype(np.int32)
    calls = []

    def record(index, forced_token, logits):
        calls.append((index, forced_token))
        return True

    eng = engine(q, model)
    print("forced tokens, callbacks, stop sequences", flush=True)
    rid = eng.submit_spec(prompt, 5, 0.7, 0.8, 20, 1.0, 1, forced_output_tokens=forced, logits_callback=record)
    res, toks = drain(q, eng, [rid])[0]
    np.testing.assert_array_equal(toks, forced)  # forced_output_tokens replace the draw (cpu_engine.inl:456-457)
    assert calls == [(i, int(forced[i])) for i in range(5)]
    eng.release(rid)  # finished requests keep their slots until released
    # a callback that fails fails its request only
    bad = eng.submit_spec(prompt, 4, 0.7, 0.8, 20, 1.0, 1, logits_callback=lambda i, f, lg: i < 2)
    good = eng.submit(prompt, 4)
    results = drain(q, eng, [bad, good])
    assert results[0][0].status == q.REQ_STATUS_INV["failed"] and results[0][1].size == 2
    assert results[1][0].status == q.REQ_STATUS_INV["complete"]
    eng.release(bad)
    eng.release(good)
    # a stop sequence is trimmed from the output and completes the request
    rid = eng.submit(prompt, 8)
    free = drain(q, eng, [rid])[0][1]
    eng.release(rid)
    stop = free[3:5]
    rid = eng.submit_spec(prompt, 8, 0.0, 1.0, 0, 1.0, 0, stop_sequences=[stop])
    res, toks = drain(q, eng, [rid])[0]
    np.testing.assert_array_equal(toks, free[:3])
    assert res.status == q.REQ_STATUS_INV["complete"]
    with pytest.raises(q.Q35Error):
        eng.submit_spec(prompt, 5, 0.7, 0.8, 20, 1.0, 1, forced_output_tokens=forced[:3])  # not max_new tokens
    with pytest.raises(q.Q35Error):
        eng.submit_spec(prompt, 5, 0.7, 0.0, 20, 1.0, 1)  # top_p must be in (0, 1]
    eng.close()


class ModuloConstraint:
    """A stateful CpuSamplingConstraint: output token i must be congruent to
    i (mod 3); apply masks the rest with -inf, accept records the token."""

    def __init__(self):
        self.accepted = []

    def allowed(self, vocab):
        return np.arange(vocab) % 3 == len(self.accepted) % 3

    def apply(self, logits):
        logits[~self.allowed(logits.size)] = -np.inf
        return True

    def accept(self, token):
        if token % 3 != len(self.accepted) % 3:
            return False
        self.accepted.append(token)
        return True


@pytest.mark.parametrize("temperature,top_p,top_k,penalty,seed", [(0.0, 1.0, 0, 1.2, 1), (0.9, 0.8, 0, 1.1, 41),
                                                                   (1.2, 1.0, 16, 1.0, 7)])
def test_constraint_matches_restatement(q, small, temperature, top_p, top_k, penalty, seed):
    """select() with a sampling constraint (cpu_engine.inl:441-465): the
    logits callback sees the raw row, the constraint masks it, the token is
    chosen from the masked row (greedy argmax after the penalty, or the full
    row draw), and accept sees every token: equal to the restatement applied
    to the masked raw rows, from the same seed."""
    d, model = small
    vocab = d["vocab"]
    prompt = np.random.default_rng(seed + 100).integers(0, vocab, size=9).astype(np.int32)
    new, seen = 8, {}
    cons = ModuloConstraint()

    def callback(index, forced, logits):
        seen[index] = logits
        return True

    eng = engine(q, model)
    print(f"constraint t={temperature} p={top_p} k={top_k}", flush=True)
    rid = eng.submit_spec(prompt, new, temperature, top_p, top_k, penalty, seed, logits_callback=callback,
                          sampling_constraint=cons)
    res, toks = drain(q, eng, [rid])[0]
    assert q.REQ_STATUS[res.status] == "complete" and toks.size == new
    assert cons.accepted == toks.tolist()
    counts = np.bincount(prompt, minlength=vocab)
    mt = MT19937(seed)
    for s in range(new):
        masked = seen[s].copy()
        masked[np.arange(vocab) % 3 != s % 3] = -np.inf
        want = sample_token(masked, counts, temperature, top_p, top_k, penalty, mt)
        assert toks[s] == want and toks[s] % 3 == s % 3, (s, toks[s], want)
        counts[toks[s]] += 1
    eng.close()


def test_selected_readout_and_contract(q, small, request):
    """A selected readout (selected_logit_tokens + selected_logits_callback,
    one forced token) gets the head's values at the given token IDs, in
    order and with duplicates: bit-equal to the full row a logits callback
    sees for the same prompt. Combinations the reference rejects are
    rejected (cpu_engine.inl:866-875)."""
    d, model = small
    vocab = d["vocab"]
    prompt = np.random.default_rng(77).integers(0, vocab, size=10).astype(np.int32)
    sel = np.array([5, 3, 5, vocab - 1, 0], np.int32)
    eng = engine(q, model)
    g16 = request.node.callspec.params["small"] == "g16q8"
    full, got = {}, {}
    rid = eng.submit_spec(prompt, 1, 0.0, 1.0, 0, 1.0, 0, forced_output_tokens=[7],
                          logits_callback=lambda i, f, lg: full.setdefault(i, lg) is not None)
    drain(q, eng, [rid])
    kw = dict(forced_output_tokens=[7], selected_logit_tokens=sel,
              selected_logits_callback=lambda i, f, v: got.setdefault(i, (f, v)) is not None)
    if g16:  # the selected readout needs a Q4 DOT4 head (layers.inl:417-421)
        with pytest.raises(q.Q35Error):
            eng.submit_spec(prompt, 1, 0.0, 1.0, 0, 1.0, 0, **kw)
        eng.close()
        return
    sid = eng.submit_spec(prompt, 1, 0.0, 1.0, 0, 1.0, 0, **kw)
    res, toks = drain(q, eng, [sid])[0]
    assert q.REQ_STATUS[res.status] == "complete" and toks.tolist() == [7]
    forced, values = got[0]
    assert forced == 7
    np.testing.assert_array_equal(values.view(np.uint32), full[0][sel].view(np.uint32))
    cons = ModuloConstraint()
    for kw in (dict(forced_output_tokens=[7], sampling_constraint=cons),
               dict(forced_output_tokens=[7], selected_logit_tokens=sel, sampling_constraint=cons,
                    selected_logits_callback=lambda *a: True),
               dict(forced_output_tokens=[7], selected_logit_tokens=sel, logits_callback=lambda *a: True,
                    selected_logits_callback=lambda *a: True),
               dict(forced_output_tokens=[7], selected_logit_tokens=sel),
               dict(forced_output_tokens=[7], selected_logit_tokens=[vocab], selected_logits_callback=lambda *a: True)):
        with pytest.raises(q.Q35Error):
            eng.submit_spec(prompt, 1, 0.0, 1.0, 0, 1.0, 0, **kw)
    with pytest.raises(q.Q35Error):  # a selected readout reads one token
        eng.submit_spec(prompt, 2, 0.0, 1.0, 0, 1.0, 0, forced_output_tokens=[7, 7], selected_logit_tokens=sel,
                        selected_logits_callback=lambda *a: True)
    eng.close()
