"""The vocabulary head, exactly: the step's logits against the oracle's head
on the step's own head input (the identity-basis A16 codes and scales the
final norm wrote, read back through the stage trace), bit for bit.
- Q4 DOT4 head: each row is q4_dot4_matvec's single block-order fma chain
  (q4_dot4.cpp:43-56), restated by q35o_dot4_matvec;
- G16 head (Q4G16Tile): per block the two 16-column halves chained as half 0
  then half 1 (q4_g16_matmul_wide, q4_g16_evex.cpp:25-49), restated by
  q35o_g16_matmul; at the 1024-wide model three 16-token tiles fit the head
  workgroup's LDS, so 52 rows run as two launches at one grid.
Batches of 1, 17 and 52 rows; the greedy head of the same step (a second
runtime fed the same tokens) must give argmax of the exact logits, lowest
index on ties."""
import numpy as np
import pytest

from tests.model_util import build_small_model, small_dims, upload_model
from tests.test_gpu_stage_parity import a16_rows

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", params=["q4", "g16"])
def wide(q, ctx, request):
    d, _ = small_dims()
    d = dict(d, hidden=1024, intermediate=512, n_layers=2)
    sched = np.array([1, 0], np.uint8)
    g16 = request.param == "g16"
    tensors = build_small_model(d, sched, seed=19, head_g16=g16)
    model = upload_model(q, ctx, d, sched, tensors)
    yield d, model, tensors, g16
    model.close()


def x1_blocks(codes, scales):
    """int8 codes [rows][nb*32] and scales [rows][nb] -> X1 blocks [rows][nb]."""
    rows, nb = scales.shape
    out = np.zeros((rows, nb), np.dtype([("scales", "<f4", (1,)), ("sums", "<i2", (1,)), ("qs", "i1", (32,)),
                                         ("pad", "<i2")]))
    q = codes.reshape(rows, nb, 32)
    out["qs"] = q
    out["scales"][..., 0] = scales
    out["sums"][..., 0] = q.astype(np.int32).sum(axis=2)
    return out


@pytest.mark.parametrize("rows", [1, 17, 52])
def test_head_logits_exact(q, ctx, orc, wide, rows):
    d, model, tensors, g16 = wide
    H, vocab = d["hidden"], d["vocab"]
    toks = np.random.default_rng(rows).integers(0, vocab, size=rows).astype(np.int32)
    results = []
    for logits in (True, False):
        rt = q.Runtime(model, max_slots=rows, max_batch=64, max_context=16, page_tokens=16, use_graphs=False)
        slots = [rt.slot_alloc(toks[i:i + 1]) for i in range(rows)]
        table = np.array([[rt.page_alloc()] for _ in range(rows)], np.int32)
        if logits:
            rt.set_trace(True)
        print(f"head exact: {'G16' if g16 else 'Q4'} rows={rows} logits={logits}", flush=True)
        res = rt.step(slots, [0] * rows, toks, table, logits=logits)
        if logits:
            tiles = (rows + 15) // 16
            codes_u64 = rt.trace(d["n_layers"], q.TRACE["CODES_HEAD"], np.uint64)
            scales = rt.trace(d["n_layers"], q.TRACE["SCALES_HEAD"], np.float32)
            codes, sc = a16_rows(codes_u64[: tiles * (H // 32) * 64], scales[: tiles * (H // 32) * 16], rows, H // 32)
            results.append((res[1], x1_blocks(codes, sc)))
        else:
            results.append(res)
        rt.close()
    (lg, x1), greedy = results
    head = tensors["model.language_model.embed_tokens.weight"][2]
    if g16:
        want = orc.g16_matmul(np.ascontiguousarray(head), x1.reshape(-1), vocab, rows, H // 32)
    else:
        want = np.stack([orc.dot4_matvec(np.ascontiguousarray(head), x1[i], vocab, H // 32) for i in range(rows)])
    np.testing.assert_array_equal(lg.view(np.uint32), want.view(np.uint32))
    np.testing.assert_array_equal(greedy, np.argmax(want, axis=1))
