"""Packed steps (q35_runtime_step_segments) and prefill chunks above 64 rows.

A packed step carries decode rows and prompt chunks of several requests in
one pass (the reference packs prefill segments of several requests into one
projection, prefill.inl:683-696, and alternates them with decode batches,
cpu_engine_scheduler.inl:64-80). Above 64 rows the projections run the dense
GEMM, prompt segments run the DeltaNet chunk scan and the tiled attention;
every row must still carry exactly the bits that separate calls give it:
- a long chunked prefill equals one single-token step per position (the
  token after the prompt, then bit-identical decode logits);
- a packed step of decode rows plus prompt chunks equals the decode step and
  the prefill calls run separately (tokens, then bit-identical logits of the
  decode steps that follow, so state and KV agree too);
- the sampled head of a packed step equals step_candidates / head_candidates;
- malformed segment lists are rejected before any launch."""
import numpy as np
import pytest

from tests.model_util import build_small_model, small_dims, upload_model

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", params=["q4", "g16_q8gates"])
def small(q, ctx, request):
    d, sched = small_dims()
    alt = request.param != "q4"
    tensors = build_small_model(d, sched, seed=5, head_g16=alt, q8_gates=alt)
    model = upload_model(q, ctx, d, sched, tensors)
    yield d, model
    model.close()


class Req:
    """A request on a runtime: slot, page table, prompt."""

    def __init__(self, rt, prompt, ctx_len):
        self.prompt = np.asarray(prompt, np.int32)
        self.slot = rt.slot_alloc(self.prompt)
        self.table = np.zeros(rt.max_pages, np.int32)
        for p in range((ctx_len + rt.cfg.page_tokens - 1) // rt.cfg.page_tokens):
            self.table[p] = rt.page_alloc()

    def seg(self, pos0, tokens, count_input=0, want=1):
        return dict(slot=self.slot, pos0=pos0, tokens=np.asarray(tokens, np.int32), page_table=self.table,
                    count_input=count_input, want_token=want)


def decode_logits(rt, reqs, pos, inp, steps):
    """`steps` decode steps of all requests in one batch: the logits of each."""
    out = []
    table = np.stack([r.table for r in reqs])
    for n in range(steps):
        tok, lg = rt.step([r.slot for r in reqs], [p + n for p in pos], inp, table, count_input=[1] * len(reqs),
                          logits=True)
        out.append(lg)
        inp = tok
    return out


@pytest.mark.parametrize("chunks", [[300], [130, 70, 1, 99], [65]])
def test_long_chunks_equal_single_steps(q, ctx, small, chunks):
    d, model = small
    plen, new = sum(chunks), 4
    prompt = np.random.default_rng(len(chunks)).integers(0, d["vocab"], size=plen).astype(np.int32)
    ctx_len = plen + new + 8
    rt = q.Runtime(model, max_slots=2, max_batch=16, max_context=ctx_len, max_step_rows=320)
    a, b = Req(rt, prompt, ctx_len), Req(rt, prompt, ctx_len)
    print(f"packed: chunks {chunks}", flush=True)
    pos, tok_a = 0, None
    for c in chunks:
        tok_a = rt.prefill(a.slot, pos, prompt[pos:pos + c], a.table)
        pos += c
    for t in range(plen):
        tok_b = int(rt.step([b.slot], [t], [prompt[t]], b.table[None, :])[0])
    assert tok_a == tok_b
    la = decode_logits(rt, [a, b], [plen, plen], np.array([tok_a, tok_b], np.int32), new)
    for n, lg in enumerate(la):
        np.testing.assert_array_equal(lg[0].view(np.uint32), lg[1].view(np.uint32), err_msg=f"decode step {n}")
    rt.close()


@pytest.mark.parametrize("layout", ["wide", "narrow"])
def test_packed_step_equals_separate_calls(q, ctx, small, layout):
    """Decode rows of two requests and prompt chunks of two others in one step
    (242 rows: more than 64, so prompt rows run the chunk scan and the tiled
    attention; 30 rows: one token group) against the decode step and the two
    prefill calls run one after another. At hidden 256 neither case fills the
    chip with dense-GEMM waves (gemm_dense_fits), so both run the split GEMMs;
    test_gpu_config5.py checks the dense GEMM in a packed step at 4B shapes."""
    d, model = small
    rng = np.random.default_rng(11)
    plens = [40, 70, 150, 90] if layout == "wide" else [40, 70, 20, 8]
    prompts = [rng.integers(0, d["vocab"], size=n).astype(np.int32) for n in plens]
    ctx_len = 200
    runs = []
    for packed in (False, True):
        rt = q.Runtime(model, max_slots=4, max_batch=16, max_context=ctx_len, max_step_rows=256)
        reqs = [Req(rt, p, ctx_len) for p in prompts]
        # A and B: prompts done, first tokens known
        first = [rt.prefill(r.slot, 0, r.prompt, r.table) for r in reqs[:2]]
        print(f"packed step ({layout}, packed={packed})", flush=True)
        if packed:
            segs = [reqs[0].seg(plens[0], [first[0]], count_input=1), reqs[1].seg(plens[1], [first[1]], count_input=1),
                    reqs[2].seg(0, prompts[2]), reqs[3].seg(0, prompts[3])]
            toks = [int(t) for t in rt.step_segments(segs)]
        else:
            dec = rt.step([reqs[0].slot, reqs[1].slot], plens[:2], first, np.stack([reqs[0].table, reqs[1].table]),
                          count_input=[1, 1])
            toks = [int(dec[0]), int(dec[1]), rt.prefill(reqs[2].slot, 0, prompts[2], reqs[2].table),
                    rt.prefill(reqs[3].slot, 0, prompts[3], reqs[3].table)]
        pos = [plens[0] + 1, plens[1] + 1, plens[2], plens[3]]
        lg = decode_logits(rt, reqs, pos, np.array(toks, np.int32), 3)
        runs.append((toks, lg))
        rt.close()
    assert runs[0][0] == runs[1][0]
    for n, (x, y) in enumerate(zip(runs[0][1], runs[1][1])):
        np.testing.assert_array_equal(x.view(np.uint32), y.view(np.uint32), err_msg=f"decode step {n}")


def test_packed_sampling_equals_candidates(q, ctx, small):
    d, model = small
    rng = np.random.default_rng(12)
    prompts = [rng.integers(0, d["vocab"], size=n).astype(np.int32) for n in (30, 100)]
    ctx_len, samp = 160, [(5, 1.0 / 0.7), (9, 1.0 / 1.3)]
    results = []
    for packed in (False, True):
        rt = q.Runtime(model, max_slots=2, max_batch=16, max_context=ctx_len, max_step_rows=128)
        a, b = Req(rt, prompts[0], ctx_len), Req(rt, prompts[1], ctx_len)
        first = rt.prefill(a.slot, 0, a.prompt, a.table)
        print(f"packed sampling (packed={packed})", flush=True)
        if packed:
            cands, raw = rt.step_segments([a.seg(30, [first], count_input=1), b.seg(0, prompts[1])], sampling=samp,
                                          raw_logits=True)
        else:
            ca, ra = rt.step_candidates([a.slot], [30], [first], a.table[None, :], samp[0][0], samp[0][1],
                                        count_input=[1], raw_logits=True)
            rt.prefill(b.slot, 0, prompts[1], b.table)
            hidden = rt.last_hidden(1)[0]
            cb, rb = rt.head_candidates(b.slot, hidden, samp[1][0], samp[1][1], raw_logits=True)
            cands, raw = np.stack([ca[0], cb]), np.stack([ra[0], rb])
        results.append((cands, raw))
        rt.close()
    np.testing.assert_array_equal(results[0][1].view(np.uint32), results[1][1].view(np.uint32))
    np.testing.assert_array_equal(results[0][0]["token"], results[1][0]["token"])
    np.testing.assert_array_equal(results[0][0]["value"].view(np.uint32), results[1][0]["value"].view(np.uint32))


def test_segment_errors(q, ctx, small):
    d, model = small
    rt = q.Runtime(model, max_slots=3, max_batch=4, max_context=64, max_step_rows=40)
    a, b = Req(rt, [1, 2, 3], 64), Req(rt, [4, 5], 64)
    bad = [
        [a.seg(0, [1, 2, 3]), a.seg(3, [4])],                 # one slot twice
        [a.seg(0, np.ones(41, np.int32))],                    # rows above max_step_rows
        [a.seg(0, [1, 2, 3], want=0)],                        # no head row
        [a.seg(62, [1, 2, 3])],                               # past max_context
        [dict(a.seg(0, [1]), tokens=np.array([d["vocab"]], np.int32))],  # token out of range
        [dict(b.seg(0, [1]), slot=2)],                        # a slot never allocated
    ]
    print("segment errors", flush=True)
    for segs in bad:
        with pytest.raises(q.Q35Error):
            rt.step_segments(segs)
    # a valid step still runs afterwards
    out = rt.step_segments([a.seg(0, [1, 2, 3]), b.seg(0, [4, 5])])
    assert np.all((out >= 0) & (out < d["vocab"]))
    rt.close()
