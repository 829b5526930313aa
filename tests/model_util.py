"""Small hybrid models for whole-step parity: weights packed by the oracle's
restatement of the reference packer, run by the oracle and by the HIP runtime."""
from __future__ import annotations

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


def build_small_model(d, sched, seed=0, std=0.1, head_std=0.2):
    """{hf_name: (encoding, shape, payload)} in the Q35H128 artifact naming.
    The scales keep the layers (not the tied embedding) in charge of the next
    token, so greedy tokens vary from step to step."""
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
               use_graphs=True, page_tokens=16, model=None):
    """Same schedule as oracle_greedy on the HIP runtime."""
    model = model or upload_model(q, ctx, d, sched, tensors)
    prompts = np.asarray(prompts, np.int32)
    b, plen = prompts.shape
    ctx_len = plen + new_tokens + 8
    rt = q.Runtime(model, max_slots=b, max_batch=b, max_context=ctx_len, page_tokens=page_tokens,
                   use_graphs=use_graphs)
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
