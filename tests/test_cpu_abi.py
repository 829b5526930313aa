"""CPU-side checks of the C ABI and its host logic (no kernel launches):
every function include/q35_hip.h declares is exported by libq35hip.so and bound
by the Python package; the host-only artifact generator writes the reference's
Q35H128 v1 format with its weights packed exactly as the oracle's restatement
of the reference packer (and the reference packer itself, when its build is
present) packs the same FP32 rows; the dims presets match the reference's
text_architecture shapes."""
import os
import re
import subprocess

import numpy as np
import pytest

from tests.model_util import fnv1a, read_artifact

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "q35_hip.h")
LIB = os.path.join(ROOT, "qwen35-cpu_amd", "libq35hip.so")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^[A-Za-z_][\w \*]*?\b(q35_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_header_parses():
    names = declared()
    assert len(names) > 60
    for must in ("q35_q4_dot4_matmul", "q35_gated_delta_net_update_rows", "q35_attention_decode_paged",
                 "q35_runtime_step", "q35_engine_advance_batch"):
        assert must in names


def test_library_exports_every_declared_symbol():
    if not os.path.exists(LIB):
        pytest.skip("libq35hip.so not built")
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True, check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    missing = [n for n in declared() if n not in exported]
    assert not missing, missing


def test_python_binding_covers_the_header(q):
    import ctypes
    for n in declared():
        f = getattr(q.lib, n)
        assert isinstance(f, ctypes._CFuncPtr)
        assert f.argtypes is not None, f"{n} has no argtypes in the binding"


def test_dims_presets(q):
    """text_architecture (profile_loader.cpp:439-462) shapes and the 3:1 schedule."""
    want = {0: (24, 1024, 3584, 8, 2, 16), 1: (24, 2048, 6144, 8, 2, 16), 2: (32, 2560, 9216, 16, 4, 32)}
    for preset, (layers, hidden, inter, heads, kvh, vh) in want.items():
        d, sched = q.model_dims(preset)
        assert (d.n_layers, d.hidden, d.intermediate, d.n_heads, d.n_kv_heads, d.lin_v_heads) == \
            (layers, hidden, inter, heads, kvh, vh)
        assert d.vocab == 248320 and d.head_dim == 256 and d.rope_dim == 64 and d.lin_k_heads == 16
        assert sched.tolist() == [0 if (i + 1) % 4 == 0 else 1 for i in range(layers)]


@pytest.fixture(scope="module")
def tiny_artifact(q, tmp_path_factory):
    from tests.model_util import small_dims
    d, sched = small_dims()
    dims = q.ModelDims(**{k: d[k] for k in [f for f, _ in q.ModelDims._fields_]})
    path = str(tmp_path_factory.mktemp("art") / "tiny.q35h128")
    q.write_random_artifact(path, dims, sched, seed=7, weight_std=0.05)
    return d, sched, path


def test_artifact_format_and_checksums(tiny_artifact):
    d, sched, path = tiny_artifact
    head, t = read_artifact(path)
    assert head["dims"] == (d["n_layers"], d["hidden"], d["intermediate"], d["vocab"])
    assert head["seed"] == d["sign_seed"]
    for name, x in t.items():
        assert fnv1a(x["data"]) == x["checksum"], name
        assert int(np.prod(x["shape"])) == x["elems"], name
        if x["enc"] in (5, 6):
            rows, cols = x["shape"]
            assert len(x["data"]) == rows // 8 * cols // 32 * 144, name
        else:
            assert x["enc"] == 0 and len(x["data"]) == 4 * x["elems"], name
    assert t["model.language_model.embed_tokens.weight"]["enc"] == 5  # identity basis, tied head
    assert t["model.language_model.layers.0.linear_attn.in_proj_all.weight"]["enc"] == 6


def test_artifact_weights_match_oracle_packer(q, orc, tiny_artifact):
    d, sched, path = tiny_artifact
    _, t = read_artifact(path)
    for name in ("model.language_model.layers.0.linear_attn.in_proj_all.weight",
                 "model.language_model.layers.3.self_attn.qkv_proj.weight",
                 "model.language_model.layers.1.mlp.down_proj.weight"):
        rows, cols = t[name]["shape"]
        x = q.random_weight_rows(name, 7, 0, rows, cols, 0.05)
        want = orc.dot4_pack(orc.h128_quantize_matrix(x), rows, cols // 32)
        assert want.tobytes() == t[name]["data"], name
    name = "model.language_model.embed_tokens.weight"
    rows, cols = t[name]["shape"]
    x = q.random_weight_rows(name, 7, 0, rows, cols, 0.05)
    assert orc.dot4_pack(orc.q4_quantize(x), rows, cols // 32).tobytes() == t[name]["data"]


def test_artifact_weights_match_reference_packer(q, orc, tiny_artifact):
    if not orc.ref_available():
        pytest.skip("reference build oracle/_ref not present")
    import ctypes
    r = orc.ref()
    d, sched, path = tiny_artifact
    _, t = read_artifact(path)
    name = "model.language_model.layers.2.mlp.gate_up_proj.weight"
    rows, cols = t[name]["shape"]
    x = q.random_weight_rows(name, 7, 0, rows, cols, 0.05)
    canon = np.zeros((rows, cols // 32), orc.Q4_0)
    assert r.ref_q4_h128_quantize_matrix(ctypes.c_void_p(x.ctypes.data), ctypes.c_void_p(canon.ctypes.data),
                                         rows, cols, d["sign_seed"]) == 1
    packed = np.zeros((rows // 8, cols // 32), orc.Q4X8)
    r.ref_q4_dot4_pack_rows_8(ctypes.c_void_p(canon.ctypes.data), ctypes.c_void_p(packed.ctypes.data), rows,
                              cols // 32)
    assert packed.tobytes() == t[name]["data"]


def test_generator_rows_are_deterministic_and_seeded(q):
    a = q.random_weight_rows("w", 3, 10, 4, 64, 0.02)
    b = q.random_weight_rows("w", 3, 0, 14, 64, 0.02)[10:]
    c = q.random_weight_rows("w", 4, 10, 4, 64, 0.02)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    big = q.random_weight_rows("v", 1, 0, 256, 1024, 1.0)
    assert abs(big.mean()) < 0.01 and abs(big.std() - 1) < 0.01


def test_prefill_chunk_token_count_matches_reference_vectors(q):
    """q35_prefill_chunk_token_count against the schedules and single values of
    the reference's tests/prefill_chunk_test.cpp:20-30 (host-only, no GPU)."""
    f = q.lib.q35_prefill_chunk_token_count

    def schedule(total, chunk, expected):
        pos = 0
        for count in expected:
            if f(pos, total - pos, chunk) != count:
                return False
            pos += count
        return pos == total

    assert schedule(579, 512, [128, 384, 67])
    assert schedule(579, 128, [128, 128, 128, 128, 67])
    assert schedule(129, 64, [64, 64, 1])
    assert schedule(221, 96, [96, 32, 64, 29])
    assert schedule(127, 512, [127])
    assert schedule(128, 512, [128])
    assert schedule(129, 512, [128, 1])
    assert f(74, 505, 512) == 54 and f(221, 358, 512) == 291 and f(512, 67, 512) == 67
    assert f(0, 0, 512) == 0 and f(0, 10, 0) == 0
