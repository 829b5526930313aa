"""Small hybrid models for whole-step parity: weights packed by the oracle's
restatement of the reference packer, run by the oracle and by the HIP runtime."""
from __future__ import annotations

import os
import struct

import numpy as np

from oracle import q35_oracle as orc

SEED = orc.SIGN_SEED


def small_dims():
    """4 layers (3 GatedDeltaNet : 1 gated attention), GQA on both paths."""
    d = dict(n_layers=4, hidden=256, intermediate=512, vocab=1024, n_heads=4, n_kv_heads=2, head_dim=256,
             rope_dim=64, rope_theta=10000000.0, rms_eps=1e-6, lin_kernel=4, lin_k_heads=2, lin_v_heads=4,
             lin_k_dim=128, lin_v_dim=128, sign_seed=SEED)
    sched = np.array([1, 1, 1, 0], np.uint8)
    return d, sched


def _h128_dot4(rng, rows, cols, std):
    w = (rng.standard_normal((rows, cols)) * std).astype(np.float32)
    return orc.dot4_pack(orc.h128_quantize_matrix(w), rows, cols // 32)


def build_small_model(d, sched, seed=0, std=0.1, head_std=0.2, head_g16=False, q8_gates=False):
    """{hf_name: (encoding, shape, payload)} in the Q35H128 artifact naming.
    The scales keep the layers (not the tied embedding) in charge of the next
    token, so greedy tokens vary from step to step. head_g16 stores the tied
    embedding as Q4G16Tile (encoding 8); q8_gates moves each linear layer's
    b and a rows into a Q8_0 linear_attn.in_proj_ba tensor (encoding 7)."""
    rng = np.random.default_rng(seed)
    H, I, hd = d["hidden"], d["intermediate"], d["head_dim"]
    q_dim = d["lin_k_heads"] * d["lin_k_dim"]
    v_dim = d["lin_v_heads"] * d["lin_v_dim"]
    ch = 2 * q_dim + v_dim
    t = {}

    def f32(name, shape, values):
        t[name] = (0, list(shape), np.ascontiguousarray(values, np.float32).reshape(shape))

    def q4(name, rows, cols):
        t[name] = (6, [rows, cols], _h128_dot4(rng, rows, cols, std))

    head = (rng.standard_normal((d["vocab"], H)) * head_std).astype(np.float32)
    if head_g16:
        t["model.language_model.embed_tokens.weight"] = (8, [d["vocab"], H], orc.g16_pack(head))
    else:
        t["model.language_model.embed_tokens.weight"] = (5, [d["vocab"], H],
                                                         orc.dot4_pack(orc.q4_quantize(head), d["vocab"], H // 32))
    f32("model.language_model.norm.weight", [H], rng.standard_normal(H) * 0.1)
    for i in range(d["n_layers"]):
        p = f"model.language_model.layers.{i}."
        f32(p + "input_layernorm.weight", [H], rng.standard_normal(H) * 0.1)
        f32(p + "post_attention_layernorm.weight", [H], rng.standard_normal(H) * 0.1)
        q4(p + "mlp.gate_up_proj.weight", 2 * I, H)
        q4(p + "mlp.down_proj.weight", H, I)
        if sched[i]:
            if q8_gates:
                q4(p + "linear_attn.in_proj_all.weight", ch + v_dim, H)
                gw = (rng.standard_normal((2 * d["lin_v_heads"], H)) * std).astype(np.float32)
                t[p + "linear_attn.in_proj_ba.weight"] = (7, [2 * d["lin_v_heads"], H], orc.q8_rows_pack(gw)[0])
            else:
                q4(p + "linear_attn.in_proj_all.weight", ch + v_dim + 2 * d["lin_v_heads"], H)
            f32(p + "linear_attn.conv1d.weight", [ch, 1, d["lin_kernel"]],
                rng.standard_normal(ch * d["lin_kernel"]) * 0.3)
            q4(p + "linear_attn.out_proj.weight", H, v_dim)
            f32(p + "linear_attn.norm.weight", [d["lin_v_dim"]], 1.0 + rng.standard_normal(d["lin_v_dim"]) * 0.1)
            f32(p + "linear_attn.A_log", [d["lin_v_heads"]], np.log(rng.uniform(1, 16, d["lin_v_heads"])))
            f32(p + "linear_attn.dt_bias", [d["lin_v_heads"]], rng.standard_normal(d["lin_v_heads"]) * 0.5)
        else:
            q4(p + "self_attn.qkv_proj.weight", 2 * d["n_heads"] * hd + 2 * d["n_kv_heads"] * hd, H)
            q4(p + "self_attn.o_proj.weight", H, d["n_heads"] * hd)
            f32(p + "self_attn.q_norm.weight", [hd], rng.standard_normal(hd) * 0.1)
            f32(p + "self_attn.k_norm.weight", [hd], rng.standard_normal(hd) * 0.1)
    return t


def oracle_greedy(d, sched, tensors, prompts, new_tokens, penalty=1.0, want_logits=False):
    """Prefill token by token, then greedy decode; returns tokens [B, new] (+ logits)."""
    m = orc.OracleModel(d, sched, tensors)
    prompts = np.asarray(prompts, np.int32)
    b, plen = prompts.shape
    states = [m.new_state(plen + new_tokens + 1, prompts[r]) for r in range(b)]
    out = np.zeros((b, new_tokens), np.int32)
    logits = []
    for t in range(plen):
        tok, lg, _ = m.step(states, prompts[:, t], penalty, want_logits and t == plen - 1)
    out[:, 0] = tok
    if want_logits:
        logits.append(lg)
    for r in range(b):
        states[r]["counts"][tok[r]] += 1
    for n in range(1, new_tokens):
        tok, lg, _ = m.step(states, out[:, n - 1], penalty, want_logits)
        out[:, n] = tok
        if want_logits:
            logits.append(lg)
        for r in range(b):
            states[r]["counts"][tok[r]] += 1
    return (out, np.stack(logits, 1)) if want_logits else out


def upload_model(q, ctx, d, sched, tensors):
    dims = q.ModelDims(**{k: d[k] for k in [f for f, _ in q.ModelDims._fields_]})
    model = q.Model(ctx, dims, sched)
    for name, (enc, shape, payload) in tensors.items():
        model.upload(name, enc, shape, payload)
    model.finalize()
    return model


def hip_greedy(q, ctx, d, sched, tensors, prompts, new_tokens, penalty=1.0, want_logits=False,
               use_graphs=True, page_tokens=16, model=None, fused=None):
    """Same schedule as oracle_greedy on the HIP runtime (fused: the fused
    decode projections on or off; None keeps the runtime's default)."""
    model = model or upload_model(q, ctx, d, sched, tensors)
    prompts = np.asarray(prompts, np.int32)
    b, plen = prompts.shape
    ctx_len = plen + new_tokens + 8
    rt = q.Runtime(model, max_slots=b, max_batch=b, max_context=ctx_len, page_tokens=page_tokens,
                   use_graphs=use_graphs)
    if fused is not None:
        rt.set_fused(fused)
    slots = np.array([rt.slot_alloc(prompts[r]) for r in range(b)], np.int32)
    table = np.zeros((b, rt.max_pages), np.int32)
    npages = 0

    def ensure(pos):
        nonlocal npages
        while npages * page_tokens <= pos:
            for r in range(b):
                table[r, npages] = rt.page_alloc()
            npages += 1

    pen = np.full(b, penalty, np.float32)
    out = np.zeros((b, new_tokens), np.int32)
    logits = []
    for t in range(plen):
        ensure(t)
        last = t == plen - 1
        res = rt.step(slots, np.full(b, t), prompts[:, t], table, np.zeros(b, np.uint8), pen,
                      logits=want_logits and last)
        tok = res[0] if (want_logits and last) else res
        if want_logits and last:
            logits.append(res[1])
    out[:, 0] = tok
    for n in range(1, new_tokens):
        pos = plen + n - 1
        ensure(pos)
        res = rt.step(slots, np.full(b, pos), out[:, n - 1], table, np.ones(b, np.uint8), pen, logits=want_logits)
        if want_logits:
            out[:, n] = res[0]
            logits.append(res[1])
        else:
            out[:, n] = res
    rt.close()
    return (out, np.stack(logits, 1)) if want_logits else out


def fnv1a(b):
    h = 0xcbf29ce484222325
    for x in np.frombuffer(b, np.uint8):
        h = ((h ^ int(x)) * 0x100000001b3) & ((1 << 64) - 1)
    return h


def read_artifact(path):
    """Q35H128 v1 reader (src/weights/q4_h128_artifact.cpp layout), independent of the library."""
    raw = open(path, "rb").read()
    assert raw[:8] == b"Q35H128\0"
    version, endian, header, align = struct.unpack_from("<4I", raw, 8)
    assert (version, endian, header, align) == (1, 0x01020304, 96, 64)
    count, dir_off, dir_bytes, data_off, seed = struct.unpack_from("<5Q", raw, 24)
    layers, hidden, inter, vocab = struct.unpack_from("<4I", raw, 64)
    tensors, pos = {}, dir_off
    for _ in range(count):
        name_size, rank, enc, transform, group, zero = struct.unpack_from("<6I", raw, pos)
        tseed, elems, off, size, checksum = struct.unpack_from("<5Q", raw, pos + 24)
        name = raw[pos + 64:pos + 64 + name_size].decode()
        shape = struct.unpack_from(f"<{rank}Q", raw, pos + 64 + name_size)
        pos += 64 + name_size + 8 * rank
        assert off % 64 == 0 and off >= data_off and off + size <= len(raw) and zero == 0
        tensors[name] = dict(enc=enc, transform=transform, group=group, seed=tseed, elems=elems, shape=shape,
                             data=raw[off:off + size], checksum=checksum)
    assert pos == dir_off + dir_bytes
    return dict(seed=seed, dims=(layers, hidden, inter, vocab)), tensors


def artifact_tensors(path):
    """{hf_name: (encoding, shape, payload bytes as uint8)} of a Q35H128 file."""
    _, t = read_artifact(path)
    return {k: (v["enc"], list(v["shape"]), np.frombuffer(v["data"], np.uint8)) for k, v in t.items()}


GOLDEN_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
GOLDEN_0P8B = os.path.join(GOLDEN_DIR, "engine_0p8b.npz")


def golden_0p8b(variant="q4"):
    """Reference-engine greedy tokens and top-8 logits (tests/golden/make_engine_golden.py);
    variant "g16q8" is the artifact with the G16 head and Q8 gate rows."""
    path = GOLDEN_0P8B if variant == "q4" else os.path.join(GOLDEN_DIR, f"engine_0p8b_{variant}.npz")
    with np.load(path) as f:
        return {k: np.ascontiguousarray(f[k]) for k in f.files}


def write_0p8b_artifact(q, directory, seed, weight_std, variant="q4"):
    d, sched = q.model_dims(0)
    path = os.path.join(directory, "model.q35h128")
    alt = variant != "q4"
    q.write_random_artifact(path, d, sched, seed=seed, weight_std=weight_std, head_g16=alt, q8_gates=alt)
    return d, sched, path


def check_against_golden(tokens, logits_at, g, tol):
    """tokens [B, N] must equal the reference's up to each row's first
    near-tie (top-2 gap below 2*tol); logits_at(row, step, index[8]) gives our
    raw logits at the reference's top-8 indices, which must agree within tol
    for every position compared."""
    ref_tok, top_v, top_i = g["tokens"], g["top_values"], g["top_index"]
    compared = 0
    for r in range(ref_tok.shape[0]):
        for n in range(ref_tok.shape[1]):
            got = logits_at(r, n, top_i[r, n])
            assert np.max(np.abs(got - top_v[r, n])) < tol, (r, n, got, top_v[r, n])
            compared += 1
            if tokens[r, n] != ref_tok[r, n]:
                assert top_v[r, n, 0] - top_v[r, n, 1] < 2 * tol, (r, n)
                break
    return compared


def oracle_envelope(d, sched, tensors, prompts, new_tokens, penalty=1.0, want=None):
    """The model's own quantization noise: the oracle against itself with the
    RMSNorm epsilon moved by 10%, a last-ulp change of every norm. Activation
    quantization rounds each 32-value block's scale to binary16, so such a
    change flips whole blocks wherever a scale sits on a rounding boundary,
    and the flips compound through the recurrent state. Returns
    (logits, tokens, max_abs, mean_abs) of the unperturbed run and the
    perturbed run's distance from it."""
    if want is None:
        want = oracle_greedy(d, sched, tensors, prompts, new_tokens, penalty, want_logits=True)
    tok, lg = want
    d2 = dict(d)
    d2["rms_eps"] = d["rms_eps"] * 1.1
    _, lg2 = oracle_greedy(d2, sched, tensors, prompts, new_tokens, penalty, want_logits=True)
    diff = np.abs(lg2[:, 0] - lg[:, 0])
    return lg, tok, float(diff.max()), float(diff.mean())


def reference_envelope(g):
    """The reference's own cross-ISA spread in the 0.8B golden: its scalar
    Q8_0 backend against the host's auto-selected one, over the probe logits
    of every teacher-forced position. Returns (max_abs, mean_abs,
    mean_abs of the first four positions)."""
    diff = np.abs(g["forced_b1_probe"] - g["forced_b0_probe"])
    return float(diff.max()), float(diff.mean()), float(diff[:, :4].mean())


def check_within_envelope(got, g, rows):
    """Probe logits [rows][steps][P] against the reference's auto backend:
    no further than 1.5x the reference's own scalar-vs-auto spread, overall
    and over the first four positions (where flips have not compounded yet).
    Returns (max_abs, mean_abs)."""
    env_max, env_mean, env_early = reference_envelope(g)
    diff = np.abs(got - g["forced_b0_probe"][:rows])
    print(f"vs reference: max {diff.max():.4f} mean {diff.mean():.5f} early {diff[:, :4].mean():.5f} "
          f"(reference scalar vs auto: max {env_max:.4f} mean {env_mean:.5f} early {env_early:.5f})", flush=True)
    assert diff.max() <= 1.5 * env_max
    assert diff.mean() <= 1.5 * env_mean
    assert diff[:, :4].mean() <= 1.5 * env_early
    return float(diff.max()), float(diff.mean())


def teacher_forced_probe_logits(step_fn, seq, probe_index):
    """Feeds seq[:, i] at position i for i < len-1 through step_fn(i, tokens)
    -> logits [rows][vocab]; returns logits at probe_index [rows][len-1][P]
    and the argmax tokens [rows][len-1]."""
    rows, n = seq.shape
    out = np.zeros((rows, n - 1, probe_index.size), np.float32)
    top = np.zeros((rows, n - 1), np.int32)
    for i in range(n - 1):
        lg = step_fn(i, seq[:, i])
        out[:, i] = lg[:, probe_index]
        top[:, i] = np.argmax(lg, axis=1)
    return out, top
