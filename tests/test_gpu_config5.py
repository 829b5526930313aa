"""Config 5 on the GPU: the 4B shapes (hidden 2560, 16 query / 4 KV heads,
16 key / 32 value linear heads, MLP 9216), 4 layers (3 GatedDeltaNet : 1
gated attention) and a 4096-token vocabulary so that the CPU oracle finishes
in seconds, random-init Q4 weights N(0, 0.02).
- 64 decode rows at contexts ~U[128, 8192]: every row of the batched step is
  bit-identical (logits, then the next step's logits) to the same row stepped
  alone (the batch-invariance pattern of the reference's
  tests/cpu_batch_model_test.cpp:84-108). Each row has a twin slot prefilled
  with the same prompt; the twins step alone.
- A 1536-token prompt prefilled in one chunk (dense GEMM, tiled attention,
  chunk scan) equals 1536 single-token steps: the next token, then the
  bit-identical logits of two decode steps.
- The first generated tokens equal the oracle's (q35o_forward_batch), up to
  the first position whose top-2 margin is below 0.05.
- Config 5's packed step itself: the 64 decode rows and a 2048-position chunk
  of a 4096-token prompt in one q35_runtime_step_segments pass, twice, equal
  to the same rows run as separate decode steps and prefill calls (raw logits
  bit for bit, the prompt's token, and the logits of the steps after)."""
import os

import numpy as np
import pytest

from tests.model_util import artifact_tensors

pytestmark = pytest.mark.gpu

PAGE = 16


@pytest.fixture(scope="module")
def m4b(q, ctx, tmp_path_factory):
    d, _ = q.model_dims(2)
    d.n_layers, d.vocab = 4, 4096
    sched = np.array([1, 1, 1, 0], np.uint8)
    path = os.path.join(str(tmp_path_factory.mktemp("c5")), "model.q35h128")
    print("config 5: writing the 4-layer 4B-shaped artifact", flush=True)
    q.write_random_artifact(path, d, sched, seed=7, weight_std=0.02)
    model = q.Model(ctx, d, sched, artifact=path)
    yield d, sched, model, path
    model.close()
    os.remove(path)


def pages_for(rt, n_tokens):
    table = np.zeros(rt.max_pages, np.int32)
    for p in range((n_tokens + PAGE - 1) // PAGE):
        table[p] = rt.page_alloc()
    return table


def prefill(rt, slot, prompt, table, chunk=2048):
    tok = None
    for c0 in range(0, prompt.size, chunk):
        tok = rt.prefill(slot, c0, prompt[c0:c0 + chunk], table)
    return tok


def test_64_rows_equal_rows_alone(q, ctx, m4b):
    d, sched, model, _ = m4b
    rows, steps = 64, 2
    rng = np.random.default_rng(55)
    lens = rng.integers(128, 8193, size=rows)
    rt = q.Runtime(model, max_slots=2 * rows, max_batch=rows, max_context=8192 + 8, page_tokens=PAGE,
                   max_step_rows=2048)
    twins = []
    print(f"config 5: prefilling 2 x {rows} prompts (contexts {lens.min()}..{lens.max()})", flush=True)
    for r in range(rows):
        prompt = rng.integers(0, d.vocab, size=int(lens[r])).astype(np.int32)
        pair = []
        for _ in range(2):
            slot = rt.slot_alloc(prompt)
            table = pages_for(rt, int(lens[r]) + steps)
            pair.append((slot, table, prefill(rt, slot, prompt, table)))
        assert pair[0][2] == pair[1][2], r
        twins.append(pair)
    pos = lens.astype(np.int32)
    tok_a = np.array([t[0][2] for t in twins], np.int32)
    tok_b = tok_a.copy()
    table_a = np.stack([t[0][1] for t in twins])
    for n in range(steps):
        print(f"config 5: batched step {n}", flush=True)
        out_a, lg_a = rt.step([t[0][0] for t in twins], pos + n, tok_a, table_a, count_input=[1] * rows, logits=True)
        for r in range(rows):
            s, table, _ = twins[r][1]
            out_b, lg_b = rt.step([s], [pos[r] + n], [tok_b[r]], table[None, :], count_input=[1], logits=True)
            np.testing.assert_array_equal(lg_a[r].view(np.uint32), lg_b[0].view(np.uint32),
                                          err_msg=f"row {r} (context {lens[r]}) step {n}")
            tok_b[r] = out_b[0]
        np.testing.assert_array_equal(out_a, tok_b)
        tok_a = out_a
    rt.close()


def test_1536_token_chunk_equals_single_steps(q, ctx, m4b):
    d, sched, model, _ = m4b
    plen = 1536
    prompt = np.random.default_rng(56).integers(0, d.vocab, size=plen).astype(np.int32)
    rt = q.Runtime(model, max_slots=2, max_batch=16, max_context=plen + 8, page_tokens=PAGE, max_step_rows=plen)
    a, b = rt.slot_alloc(prompt), rt.slot_alloc(prompt)
    ta, tb = pages_for(rt, plen + 3), pages_for(rt, plen + 3)
    print(f"config 5: {plen}-token prompt in one chunk", flush=True)
    tok_a = rt.prefill(a, 0, prompt, ta)
    print(f"config 5: {plen} single steps", flush=True)
    for t in range(plen):
        tok_b = int(rt.step([b], [t], [prompt[t]], tb[None, :])[0])
    assert tok_a == tok_b
    inp = np.array([tok_a, tok_b], np.int32)
    for n in range(2):
        out, lg = rt.step([a, b], [plen + n] * 2, inp, np.stack([ta, tb]), count_input=[1, 1], logits=True)
        np.testing.assert_array_equal(lg[0].view(np.uint32), lg[1].view(np.uint32), err_msg=f"decode step {n}")
        inp = out
    rt.close()


def test_first_tokens_equal_oracle(q, ctx, orc, m4b):
    d, sched, model, path = m4b
    rng = np.random.default_rng(57)
    prompts = [rng.integers(0, d.vocab, size=6).astype(np.int32) for _ in range(2)]
    new = 3
    om = orc.OracleModel(d, sched, artifact_tensors(path))
    print("config 5: oracle greedy", flush=True)
    states = [om.new_state(16, p) for p in prompts]
    want = np.zeros((2, new), np.int32)
    want_lg = np.zeros((2, new, d.vocab), np.float32)
    for t in range(prompts[0].size):
        out, lg, _ = om.step(states, [p[t] for p in prompts], want_logits=True)
    for n in range(new):
        want[:, n], want_lg[:, n] = out, lg
        if n + 1 < new:
            out, lg, _ = om.step(states, out, want_logits=True)
    rt = q.Runtime(model, max_slots=2, max_batch=8, max_context=16, page_tokens=PAGE)
    slots = [rt.slot_alloc(p) for p in prompts]
    tables = np.stack([pages_for(rt, 16) for _ in prompts])
    got = np.zeros((2, new), np.int32)
    got[:, 0] = [rt.prefill(s, 0, p, t) for s, p, t in zip(slots, prompts, tables)]
    for n in range(1, new):
        got[:, n] = rt.step(slots, [prompts[0].size + n - 1] * 2, got[:, n - 1], tables, count_input=[1, 1])
    rt.close()
    for r in range(2):
        for n in range(new):
            if got[r, n] != want[r, n]:
                top2 = np.sort(want_lg[r, n])[-2:]
                assert top2[1] - top2[0] < 0.05, (r, n, got[r], want[r], top2)
                break


@pytest.fixture(scope="module")
def m4b_wide(q, ctx, tmp_path_factory):
    """The same 4-layer 4B-shaped model with a 32,768-token vocabulary: the
    head streams 47 MB of tiles over many workgroups."""
    d, _ = q.model_dims(2)
    d.n_layers, d.vocab = 4, 32768
    sched = np.array([1, 1, 1, 0], np.uint8)
    path = os.path.join(str(tmp_path_factory.mktemp("c5w")), "model.q35h128")
    print("config 5: writing the 4-layer 4B-shaped artifact, vocab 32768", flush=True)
    q.write_random_artifact(path, d, sched, seed=9, weight_std=0.02)
    model = q.Model(ctx, d, sched, artifact=path)
    yield d, model
    model.close()
    os.remove(path)


def test_packed_step_equals_separate_calls(q, ctx, m4b_wide):
    """Config 5's packed step: 64 decode rows at contexts ~U[128, 8192] and a
    4096-token prompt in two 2048-position chunks, each chunk packed with one
    decode step of the 64 rows into a single q35_runtime_step_segments pass of
    2112 rows (dense GEMM, flash prompt attention, DeltaNet chunk scan and
    decode attention in one step; prefill.inl:683-696 packs segments, and
    cpu_engine_scheduler.inl:64-80 is the alternation the packing replaces).
    Against twin slots run as separate decode steps and prefill calls:
    - every decode row's raw logits are bit-identical in both packed steps;
    - the prompt's next token equals the twin's chunked prefill and 4096
      single-token steps of a third slot;
    - every row's logits of the two decode steps after (65 one-row segments,
      so the head takes two launches) are bit-identical to the separate
      steps', so recurrent state, conv ring and KV rows agree too."""
    d, model = m4b_wide
    rows, plen, chunk = 64, 4096, 2048
    rng = np.random.default_rng(58)
    lens = rng.integers(128, 8193, size=rows)
    rt = q.Runtime(model, max_slots=2 * rows + 3, max_batch=rows, max_context=8192 + 8, page_tokens=PAGE,
                   max_step_rows=rows + chunk)
    print(f"config 5 packed: prefilling 2 x {rows} prompts (contexts {lens.min()}..{lens.max()})", flush=True)
    dec = []  # per row: (slot A, slot B, table A, table B, first token)
    for r in range(rows):
        prompt = rng.integers(0, d.vocab, size=int(lens[r])).astype(np.int32)
        sa, sb = rt.slot_alloc(prompt), rt.slot_alloc(prompt)
        ta, tb = pages_for(rt, int(lens[r]) + 4), pages_for(rt, int(lens[r]) + 4)
        fa, fb = prefill(rt, sa, prompt, ta), prefill(rt, sb, prompt, tb)
        assert fa == fb, r
        dec.append((sa, sb, ta, tb, fa))
    prompt = rng.integers(0, d.vocab, size=plen).astype(np.int32)
    pa, pb, pc = rt.slot_alloc(prompt), rt.slot_alloc(prompt), rt.slot_alloc(prompt)
    tpa, tpb, tpc = (pages_for(rt, plen + 4) for _ in range(3))
    pos = lens.astype(np.int32)
    tok_a = np.array([x[4] for x in dec], np.int32)
    tok_b = tok_a.copy()
    greedy = [(1, 1.0)]
    p_tok_a = p_tok_b = None
    for n in range(plen // chunk):
        c0 = n * chunk
        last = c0 + chunk == plen
        dsegs = [dict(slot=x[0], pos0=int(pos[r] + n), tokens=[int(tok_a[r])], page_table=x[2], count_input=1)
                 for r, x in enumerate(dec)]
        pseg = dict(slot=pa, pos0=c0, tokens=prompt[c0:c0 + chunk], page_table=tpa, want_token=int(last))
        # the prompt chunk first in one step, last in the other
        segs = [pseg] + dsegs if n == 0 else dsegs + [pseg]
        print(f"config 5 packed: step {n} ({len(segs)} segments, {rows + chunk} rows)", flush=True)
        cands, raw = rt.step_segments(segs, sampling=greedy * len(segs), raw_logits=True)
        at = 1 if n == 0 else 0
        out_a = cands["token"][at:at + rows, 0]
        raw_a = raw[at:at + rows]
        if last:
            p_tok_a = int(cands["token"][0 if n == 0 else rows, 0])
        out_b, raw_b = rt.step([x[1] for x in dec], pos + n, tok_b, np.stack([x[3] for x in dec]),
                               count_input=[1] * rows, logits=True)
        for r in range(rows):
            np.testing.assert_array_equal(raw_a[r].view(np.uint32), raw_b[r].view(np.uint32),
                                          err_msg=f"decode row {r} (context {lens[r] + n}) in packed step {n}")
        np.testing.assert_array_equal(out_a, out_b)
        p_tok_b = rt.prefill(pb, c0, prompt[c0:c0 + chunk], tpb)
        tok_a, tok_b = out_a.astype(np.int32), out_b.astype(np.int32)
    print(f"config 5 packed: {plen} single steps of the prompt", flush=True)
    for t in range(plen):
        p_tok_c = int(rt.step([pc], [t], [prompt[t]], tpc[None, :])[0])
    assert p_tok_a == p_tok_b == p_tok_c, (p_tok_a, p_tok_b, p_tok_c)
    # two decode steps of all 65 requests: packed one-row segments against
    # the separate 64-row step and the prompt request's own step
    pos = pos + plen // chunk
    p_in = np.array([p_tok_a, p_tok_b, p_tok_c], np.int32)
    for n in range(2):
        print(f"config 5 packed: decode step {n} after the prompt", flush=True)
        segs = [dict(slot=x[0], pos0=int(pos[r] + n), tokens=[int(tok_a[r])], page_table=x[2], count_input=1)
                for r, x in enumerate(dec)]
        segs.append(dict(slot=pa, pos0=plen + n, tokens=[int(p_in[0])], page_table=tpa, count_input=1))
        cands, raw_a = rt.step_segments(segs, sampling=greedy * len(segs), raw_logits=True)
        out_b, raw_b = rt.step([x[1] for x in dec], pos + n, tok_b, np.stack([x[3] for x in dec]),
                               count_input=[1] * rows, logits=True)
        pt_b, praw_b = rt.step([pb], [plen + n], [p_in[1]], tpb[None, :], count_input=[1], logits=True)
        pt_c, praw_c = rt.step([pc], [plen + n], [p_in[2]], tpc[None, :], count_input=[1], logits=True)
        for r in range(rows):
            np.testing.assert_array_equal(raw_a[r].view(np.uint32), raw_b[r].view(np.uint32),
                                          err_msg=f"decode row {r} after the prompt, step {n}")
        np.testing.assert_array_equal(raw_a[rows].view(np.uint32), praw_b[0].view(np.uint32),
                                      err_msg=f"prompt row, step {n}")
        np.testing.assert_array_equal(praw_b[0].view(np.uint32), praw_c[0].view(np.uint32),
                                      err_msg=f"prompt row against single steps, step {n}")
        np.testing.assert_array_equal(cands["token"][:rows, 0], out_b)
        tok_a, tok_b = cands["token"][:rows, 0].astype(np.int32), out_b.astype(np.int32)
        p_in = np.array([cands["token"][rows, 0], pt_b[0], pt_c[0]], np.int32)
        assert p_in[0] == p_in[1] == p_in[2], p_in
    rt.close()
