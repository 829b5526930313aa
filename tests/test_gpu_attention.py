"""Paged gated GQA attention decode parity on the GPU (config 3): B=16, context
lengths U[64, 4096], 8 query / 2 KV heads, head_dim 256, FP16 K/V in 16-token
pages with shuffled page tables, sigmoid gate. Bar: 1e-3 relative."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _case(rng, batch, heads, kv_heads, hd, lens, page_tokens):
    kvw = kv_heads * hd
    pages_per = [(n + page_tokens - 1) // page_tokens for n in lens]
    total = sum(pages_per)
    perm = rng.permutation(total).astype(np.int32)
    max_pages = max(pages_per)
    table = np.zeros((batch, max_pages), np.int32)
    o = 0
    for b in range(batch):
        table[b, :pages_per[b]] = perm[o:o + pages_per[b]]
        o += pages_per[b]
    k_pool = rng.standard_normal((total, page_tokens, kvw)).astype(np.float16).view(np.uint16)
    v_pool = rng.standard_normal((total, page_tokens, kvw)).astype(np.float16).view(np.uint16)
    qv = rng.standard_normal((batch, heads * hd)).astype(np.float32)
    gates = rng.standard_normal((batch, heads * hd)).astype(np.float32)
    return table, k_pool, v_pool, qv, gates, max_pages


def _run(q, ctx, orc, batch, heads, kv_heads, lens, page_tokens, seed):
    hd = 256
    rng = np.random.default_rng(seed)
    lens = np.asarray(lens, np.int32)
    table, k_pool, v_pool, qv, gates, max_pages = _case(rng, batch, heads, kv_heads, hd, lens, page_tokens)
    out = ctx.array(shape=(batch, heads * hd), dtype=np.float32)
    print(f"attention batch={batch} heads={heads}/{kv_heads} max_len={lens.max()}", flush=True)
    q.attention_decode_paged(ctx, ctx.array(qv), ctx.array(gates), ctx.array(k_pool), ctx.array(v_pool),
                             ctx.array(table), max_pages, ctx.array(lens), page_tokens, out, batch, heads,
                             kv_heads, hd, 1.0 / 16.0)
    got = out.download()
    for b in range(batch):
        rows = np.concatenate([k_pool[p] for p in table[b]])[:lens[b]]
        vrows = np.concatenate([v_pool[p] for p in table[b]])[:lens[b]]
        want = orc.attention_decode(qv[b], gates[b], rows, vrows, heads, kv_heads, hd)
        err = np.max(np.abs(got[b] - want)) / max(np.max(np.abs(want)), 1e-30)
        assert err < 1e-3, (b, lens[b], err)


def test_config3(q, ctx, orc):
    rng = np.random.default_rng(64)
    lens = rng.integers(64, 4097, size=16)
    _run(q, ctx, orc, 16, 8, 2, lens, 16, 1)


@pytest.mark.parametrize("lens,page_tokens", [([1, 2, 255, 256, 257], 16), ([17, 300], 256), ([513], 1)])
def test_edges(q, ctx, orc, lens, page_tokens):
    _run(q, ctx, orc, len(lens), 8, 2, lens, page_tokens, 7)


def test_gqa_group_sizes(q, ctx, orc):
    for heads, kv in ((4, 4), (4, 2), (16, 2)):
        _run(q, ctx, orc, 3, heads, kv, [40, 700, 1], 16, heads * 10 + kv)
