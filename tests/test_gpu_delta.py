"""GatedDeltaNet decode update parity on the GPU (config 2): B=16 requests,
16 heads, d_k = d_v = 128, fp32 state N(0, 0.02); 1 step and 64 chained steps.
Bar: 1e-3 relative (north star) on outputs and state."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

B, H, D = 16, 16, 128


def _inputs(rng):
    q = rng.standard_normal((B, H, D)).astype(np.float32)
    k = rng.standard_normal((B, H, D)).astype(np.float32)
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((B, H, D)).astype(np.float32)
    beta = (1 / (1 + np.exp(-rng.standard_normal((B, H))))).astype(np.float32)
    alpha = np.exp(-np.log1p(np.exp(rng.standard_normal((B, H))))).astype(np.float32)
    return q, k, v, alpha, beta


def _rel(a, b):
    return np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30)


@pytest.mark.parametrize("steps", [1, 64])
def test_config2_batch(q, ctx, orc, steps):
    rng = np.random.default_rng(2 + steps)
    state0 = (rng.standard_normal((B, H, D, D)) * 0.02).astype(np.float32)
    dev_state = ctx.array(state0)
    ptrs = ctx.array(np.array([dev_state.address + b * H * D * D * 4 for b in range(B)], np.uint64))
    ref_state = state0.copy()
    out = ctx.array(shape=(B, H, D), dtype=np.float32)
    print(f"config2 steps={steps}", flush=True)
    for s in range(steps):
        qq, kk, vv, al, be = _inputs(rng)
        bufs = [ctx.array(a) for a in (qq, kk, vv, al, be)]
        q.gated_delta_net_update_batch(ctx, ptrs, *bufs, out, B, H, D, D)
        want = np.zeros((B, H, D), np.float32)
        for b in range(B):
            new_state, o = orc.delta_rows(ref_state[b].reshape(-1), qq[b], kk[b], vv[b], al[b], be[b], D, D)
            ref_state[b] = new_state.reshape(H, D, D)
            want[b] = o.reshape(H, D)
        if s == steps - 1 or s % 16 == 0:
            assert _rel(out.download(), want) < 1e-3, f"output step {s}"
    assert _rel(dev_state.download(), ref_state) < 1e-3


def test_rows_api_partial_range(q, ctx, orc):
    """gated_delta_net_update_rows on a sub-range of flattened rows (delta_net.h:18-31)."""
    rng = np.random.default_rng(9)
    heads, kd, vd = 4, 64, 96
    state = (rng.standard_normal((heads, vd, kd)) * 0.1).astype(np.float32)
    qq = rng.standard_normal((heads, kd)).astype(np.float32)
    kk = rng.standard_normal((heads, kd)).astype(np.float32) * 0.1
    vv = rng.standard_normal((heads, vd)).astype(np.float32)
    al = rng.uniform(0.5, 1.0, heads).astype(np.float32)
    be = rng.uniform(0.0, 1.0, heads).astype(np.float32)
    begin, end = 37, 300
    want_state, want_out = orc.delta_rows(state.reshape(-1), qq, kk, vv, al, be, kd, vd, begin, end)
    ds, dout = ctx.array(state), ctx.array(np.zeros(heads * vd, np.float32))
    q.gated_delta_net_update_rows(ctx, ds, ctx.array(qq), ctx.array(kk), ctx.array(vv), ctx.array(al),
                                  ctx.array(be), dout, heads, kd, vd, begin, end)
    assert _rel(ds.download().reshape(-1), want_state) < 1e-5
    got = dout.download()
    assert _rel(got[begin:end], want_out[begin:end]) < 1e-4
    assert np.all(got[:begin] == 0) and np.all(got[end:] == 0)
