"""The reference-side C++ binding (qwen35-cpu_amd/binding/hip_engine.hpp)
running: tests/binding/serve_binding.cpp fills the reference's own
ModelProfile for the random-init 0.8B-shaped artifact, loads it through
HipModel::load (rope width, layer schedule and sign seed derived as the
binding derives them), creates a HipEngine in serving mode and drives it as
the reference's server does (src/server.cpp:255-300: submit, step(),
read_output() after every step, release when terminal), with automatic
prefix registration on the requests that share a prompt head. Every
request's tokens must equal the Python engine's on the same artifact (the
same C engine in direct mode, whose tokens the oracle tests tie to the
restated reference step), and the shared head must be built once and hit
by the requests that waited for it.

The program is compiled by __graft_entry__.build() where the reference's
headers are present; this test runs the built program."""
import os
import subprocess

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "binding", "_build", "serve_binding")


@pytest.mark.skipif(not os.path.exists(BIN), reason="serve_binding is built by __graft_entry__.build() next to the "
                                                    "reference headers, and is not built")
def test_binding_serving_loop_tokens(q, ctx, tmp_path):
    d, sched = q.model_dims(0)
    path = str(tmp_path / "model_0p8b.q35h128")
    print("binding: writing the random-init 0.8B artifact", flush=True)
    q.write_random_artifact(path, d, sched, seed=31, weight_std=0.02)
    rng = np.random.default_rng(32)
    head = rng.integers(0, d.vocab, size=48).astype(np.int32)
    prompts = [np.concatenate([head, rng.integers(0, d.vocab, size=n).astype(np.int32)]) for n in (7, 30, 12)]
    prompts += [rng.integers(0, d.vocab, size=n).astype(np.int32) for n in (5, 40, 23)]
    req = tmp_path / "requests.txt"
    req.write_text("".join(" ".join(str(int(t)) for t in p) + "\n" for p in prompts))
    new = 9
    args = [BIN, path, str(req), "resident=4", "queued=8", "batch=4", "prefill_requests=2", f"max_new={new}",
            "register=48", "ns=tenant", "read=3", "context=256"]
    print("binding: " + " ".join(os.path.basename(a) for a in args), flush=True)
    r = subprocess.run(args, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-3000:]
    lines = r.stdout.strip().splitlines()
    got, cached = {}, {}
    for ln in lines[:-1]:
        f = ln.split()
        assert f[0] == "request" and f[2] == "complete", ln
        got[int(f[1])] = [int(x) for x in f[3:-1]]
        cached[int(f[1])] = int(f[-1].split("=")[1])
    stats = dict(kv.split("=") for kv in lines[-1].split()[1:])
    print("binding: " + lines[-1], flush=True)
    # the same requests on the Python mirror of the same engine, direct mode
    model = q.Model(ctx, d, sched, artifact=path)
    eng = q.Engine(model, max_resident_requests=len(prompts), max_context=256, max_decode_batch_size=len(prompts),
                   page_tokens=16)
    ids = [eng.submit(p, max_new_tokens=new) for p in prompts]
    eng.prefill_batch(ids)
    while True:
        active = [i for i in ids if q.REQ_STATUS[eng.result(i)[0].status] == "decode"]
        if not active:
            break
        eng.advance_batch(active)
    want = {k: eng.result(i)[1].tolist() for k, i in enumerate(ids)}
    eng.close()
    model.close()
    assert got == want
    # the 48-token head: built by the first request that reached it, hit by the two that waited
    assert int(stats["builds"]) == 1 and int(stats["hits"]) == 2
    assert sorted(cached[k] for k in range(3)) == [0, 48, 48]
    assert all(cached[k] == 0 for k in range(3, 6))
