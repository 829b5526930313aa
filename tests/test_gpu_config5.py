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
  the first position whose top-2 margin is below 0.05."""
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
