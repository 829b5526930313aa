"""Stage-wise teacher-forced parity of the decode step: the random-init 0.8B
model at config-4 size (16 requests, 512-token random prompts, 8 decode
steps fed with the GPU's own greedy tokens).

The runtime's stage trace (q35_runtime_set_trace) keeps every stage's input
and output, so each stage is restarted on the CPU oracle from the GPU's own
input and rounding differences cannot compound: a stage bug shows at its own
size instead of hiding inside a whole-model envelope. Checked at every layer
and step:
- int8 codes and scales bit-exact at every quantization point: the H128
  preparation of the in, out, gate_up and down projection inputs
  (q4_h128_prepare_activations_4, q4_h128.cpp:326-401) and the identity-basis
  preparation of the head input (q8_0_quantize_vectors_4, q4_0.cpp:149-180);
- FP32 stage outputs within 1e-3 relative (|gpu - ref| <= 1e-3 |ref| + 1e-3
  rms(ref) per row): both RMSNorms; every projection's rows against the exact
  int32 block dots times the binary16 scales, accumulated in FP64; the
  DeltaNet step (conv ring, gates, state update, gated norm) from
  run_linear_attention_step's restatement (q35o_linear_attention_row); the
  attention prep and output from prepare_full_attention_row +
  run_full_attention_step's restatement over the GPU's own KV pages; the
  SiLU gating;
- the residual adds exactly the projection rows it is given (bit-exact);
- head logits from the GPU's final hidden row within 1e-2 max-abs of the
  oracle's head (the reference's block-order chain).
All rows are checked on the first step, two rows per later step (the CPU
side of the full check is the slow part)."""
import os

import numpy as np
import pytest

from tests.model_util import artifact_tensors, write_0p8b_artifact

pytestmark = pytest.mark.gpu

B, PROMPT, STEPS, PAGE = 16, 512, 8, 16
RTOL = 1e-3


@pytest.fixture(scope="module", params=["q4", "g16q8"])
def m08(q, ctx, orc, tmp_path_factory, request):
    print(f"0.8B ({request.param}): writing the random-init artifact", flush=True)
    d, sched, path = write_0p8b_artifact(q, str(tmp_path_factory.mktemp("stage")), 1, 0.02, request.param)
    model = q.Model(ctx, d, sched, artifact=path)
    tensors = artifact_tensors(path)
    om = orc.OracleModel(d, sched, tensors)
    yield d, sched, model, tensors, om
    model.close()
    os.remove(path)


def assert_close(gpu, ref, what, rtol=RTOL):
    gpu = np.asarray(gpu, np.float64)
    ref = np.asarray(ref, np.float64)
    floor = rtol * np.sqrt(np.mean(ref * ref)) if ref.size else 0.0
    err = np.abs(gpu - ref)
    bad = err > rtol * np.abs(ref) + floor
    assert not bad.any(), f"{what}: {bad.sum()} of {bad.size} outside 1e-3 (max err {err.max():.3g}, floor {floor:.3g})"


def a16_rows(codes_u64, scales, rows, nb):
    """A16 activations (tile, block, lane = token + 16 * k-group) -> int8
    codes [rows][nb * 32] and scales [rows][nb]."""
    tiles = (rows + 15) // 16
    c = codes_u64.reshape(tiles, nb, 4, 16).view(np.int8).reshape(tiles, nb, 4, 16, 8)
    codes = c.transpose(0, 3, 1, 2, 4).reshape(tiles * 16, nb * 32)[:rows]
    sc = scales.reshape(tiles, nb, 16).transpose(0, 2, 1).reshape(tiles * 16, nb)[:rows]
    return codes, sc


def x4_rows(act4, rows):
    """Reference X4 blocks [rows / 4][nb] -> int8 codes [rows][nb * 32] and scales [rows][nb]."""
    nb = act4.shape[1]
    codes = act4["qs"].reshape(rows // 4, nb, 4, 32).transpose(0, 2, 1, 3).reshape(rows, nb * 32)
    scales = act4["scales"].transpose(0, 2, 1).reshape(rows, nb)
    return codes, scales


class Dot4:
    """A DOT4 matrix as (u - 8) codes [rows][K] and binary16 row scales
    [rows][K / 32] (q4_dot4.h:5-6: qs[32t + 4r + j] = u[r][8t + j] | u[r][8t + 4 + j] << 4)."""

    def __init__(self, payload, rows, cols):
        nb = cols // 32
        t = np.frombuffer(payload, np.uint8).reshape(rows // 8, nb, 144)
        self.scale = t[:, :, :16].copy().view(np.float16).astype(np.float64).transpose(0, 2, 1).reshape(rows, nb)
        qs = t[:, :, 16:].reshape(rows // 8, nb, 4, 8, 4)  # [tile][block][t][r][j]
        lo, hi = (qs & 15).astype(np.int8), (qs >> 4).astype(np.int8)
        u = np.concatenate([lo, hi], axis=4)  # [tile][block][t][r][j | 4 + j] = column 8t + (0..7)
        codes = (u.transpose(0, 3, 1, 2, 4).reshape(rows, nb, 32) - 8).astype(np.float32)
        self.w = np.ascontiguousarray(codes.transpose(1, 0, 2))  # [block][row][32]
        self.rows, self.nb = rows, nb

    def rows_for(self, codes, scales):
        """FP64 reference of the projection: sum over blocks of the exact
        int32 block dot times half(d_row) * s_token."""
        a = np.ascontiguousarray(codes.astype(np.float32).reshape(-1, self.nb, 32).transpose(1, 2, 0))
        dots = np.matmul(self.w, a).astype(np.float64)  # [block][row][token], exact in FP32
        return np.einsum("brt,rb,tb->tr", dots, self.scale, scales.astype(np.float64))


def check_codes(orc, gpu_codes, gpu_scales, fp32_rows, nb, what, h128=True):
    act = orc.h128_prepare_4(fp32_rows) if h128 else orc.q8_quantize_4(fp32_rows)
    want_c, want_s = x4_rows(act, fp32_rows.shape[0])
    got_c, got_s = a16_rows(gpu_codes, gpu_scales, fp32_rows.shape[0], nb)
    np.testing.assert_array_equal(got_c, want_c, err_msg=f"{what} codes")
    np.testing.assert_array_equal(got_s.view(np.uint32), want_s.view(np.uint32), err_msg=f"{what} scales")
    return got_c, got_s


def test_decode_stages_against_oracle(q, orc, m08):
    d, sched, model, tensors, om = m08
    H, I, V = d.hidden, d.intermediate, d.vocab
    kvw = d.n_kv_heads * d.head_dim
    q_dim, v_dim = d.lin_k_heads * d.lin_k_dim, d.lin_v_heads * d.lin_v_dim
    ch = 2 * q_dim + v_dim
    pfx = "model.language_model.layers."
    mats = {}

    def mat(name, rows, cols):
        if name not in mats:
            mats[name] = Dot4(tensors[name][2], rows, cols)
        return mats[name]

    ctx_len = PROMPT + STEPS + 8
    rt = q.Runtime(model, max_slots=B, max_batch=B, max_context=ctx_len, page_tokens=PAGE, use_graphs=False)
    rng = np.random.default_rng(2024)
    prompts = rng.integers(0, V, size=(B, PROMPT)).astype(np.int32)
    slots = np.array([rt.slot_alloc(prompts[r]) for r in range(B)], np.int32)
    table = np.array([[rt.page_alloc() for _ in range(rt.max_pages)] for _ in range(B)], np.int32)
    print("prefilling 16 x 512 tokens", flush=True)
    tokens = np.zeros(B, np.int32)
    for r in range(B):
        for p0 in range(0, PROMPT, 16):
            tokens[r] = rt.prefill(int(slots[r]), p0, prompts[r, p0:p0 + 16], table[r])
    rt.set_trace(True)
    layer_pos = {}
    li = fi = 0
    for l in range(d.n_layers):
        layer_pos[l] = (li, fi)
        li, fi = (li + 1, fi) if sched[l] else (li, fi + 1)
    for step in range(STEPS):
        pos = PROMPT + step
        toks, logits = rt.step(slots, np.full(B, pos), tokens, table, np.ones(B, np.uint8), logits=True)
        rows = np.arange(B) if step == 0 else np.array([(2 * step) % B, (2 * step + 1) % B])
        print(f"step {step}: checking rows {rows.tolist()} of every layer", flush=True)

        def tr(layer, name, dtype=np.float32):
            return rt.trace(layer, q.TRACE[name], dtype)

        for l in range(d.n_layers):
            p = f"{pfx}{l}."
            lin = bool(sched[l])
            w_in = tensors[p + "input_layernorm.weight"][2].view(np.float32)
            w_post = tensors[p + "post_attention_layernorm.weight"][2].view(np.float32)
            x_in = tr(l, "X_IN").reshape(B, H)
            normed = tr(l, "NORMED_IN").reshape(B, H)
            assert_close(normed[rows], orc.rms_norm(x_in[rows], w_in, d.rms_eps, 1.0), f"L{l} input norm")
            codes, scales = check_codes(orc, tr(l, "CODES_IN", np.uint64), tr(l, "SCALES_IN"), normed, H // 32,
                                        f"L{l} in-proj input")
            in_name = p + ("linear_attn.in_proj_all.weight" if lin else "self_attn.qkv_proj.weight")
            in_rows = tensors[in_name][1][0]
            proj = tr(l, "PROJ_IN").reshape(B, in_rows)
            assert_close(proj[rows], mat(in_name, in_rows, H).rows_for(codes[rows], scales[rows]), f"L{l} in-proj")
            if lin:
                li, _ = layer_pos[l]
                gates = tr(l, "GATES")
                if gates is not None:  # Q8 gate rows over the identity-basis input (run_q8_gate_tail)
                    gates = gates.reshape(B, -1)
                    ba = tensors[p + "linear_attn.in_proj_ba.weight"]
                    blocks8 = np.ascontiguousarray(ba[2]).view(orc.Q8_0).reshape(ba[1][0], H // 32)
                    ms = blocks8["d"].view(np.float16).astype(np.float32)
                    act1 = orc.q8_quantize_1(normed.ravel())
                    want = orc.q8_matmul(blocks8, ms, act1, ba[1][0], B, H // 32)
                    np.testing.assert_array_equal(gates.view(np.uint32), want.view(np.uint32), err_msg=f"L{l} gates")
                    proj = np.concatenate([proj, gates], axis=1)
                conv_b = tr(l, "CONV_BEFORE").reshape(B, d.lin_kernel, ch)
                conv_a = tr(l, "CONV_AFTER").reshape(B, d.lin_kernel, ch)
                st_b = tr(l, "STATE_BEFORE").reshape(B, -1)
                st_a = tr(l, "STATE_AFTER").reshape(B, -1)
                core = tr(l, "CORE").reshape(B, v_dim)
                for r in rows:
                    # the reference ring: the last kernel-1 inputs oldest first at ring index 0
                    hist = np.stack([conv_b[r, (pos + 1 + k) % d.lin_kernel] for k in range(d.lin_kernel - 1)])
                    c_ref, conv_ref, ring, st_ref = om.linear_row(l, hist, 0, st_b[r], proj[r])
                    assert_close(core[r], c_ref, f"L{l} row {r} DeltaNet output")
                    assert_close(st_a[r], st_ref, f"L{l} row {r} DeltaNet state")
                    np.testing.assert_array_equal(conv_a[r, pos % d.lin_kernel], proj[r, :ch],
                                                  err_msg=f"L{l} conv ring")
            else:
                _, fi = layer_pos[l]
                kpool = tr(l, "K_POOL", np.uint16).reshape(-1, PAGE, kvw)
                vpool = tr(l, "V_POOL", np.uint16).reshape(-1, PAGE, kvw)
                core = tr(l, "CORE").reshape(B, d.n_heads * d.head_dim)
                for r in rows:
                    keys = kpool[table[r]].reshape(-1, kvw)[:pos + 1]
                    vals = vpool[table[r]].reshape(-1, kvw)[:pos + 1]
                    c_ref, k_ref, v_ref = om.full_row(l, keys, vals, pos, proj[r])
                    assert_close(core[r], c_ref, f"L{l} row {r} attention output")
                    k_new = k_ref.reshape(-1, kvw)[pos].view(np.float16).astype(np.float32)
                    v_new = v_ref.reshape(-1, kvw)[pos].view(np.float16).astype(np.float32)
                    assert_close(keys[pos].view(np.float16).astype(np.float32), k_new, f"L{l} row {r} new key")
                    assert_close(vals[pos].view(np.float16).astype(np.float32), v_new, f"L{l} row {r} new value")
            width = v_dim if lin else d.n_heads * d.head_dim
            c_codes, c_scales = check_codes(orc, tr(l, "CODES_CORE", np.uint64), tr(l, "SCALES_CORE"), core,
                                            width // 32, f"L{l} out-proj input")
            out_name = p + ("linear_attn.out_proj.weight" if lin else "self_attn.o_proj.weight")
            proj_out = tr(l, "PROJ_OUT").reshape(B, H)
            assert_close(proj_out[rows], mat(out_name, H, width).rows_for(c_codes[rows], c_scales[rows]),
                         f"L{l} out-proj")
            x_mid = tr(l, "X_MID").reshape(B, H)
            np.testing.assert_array_equal(x_mid.view(np.uint32), (x_in + proj_out).view(np.uint32),
                                          err_msg=f"L{l} residual")
            normed_p = tr(l, "NORMED_POST").reshape(B, H)
            assert_close(normed_p[rows], orc.rms_norm(x_mid[rows], w_post, d.rms_eps, 1.0), f"L{l} post norm")
            g_codes, g_scales = check_codes(orc, tr(l, "CODES_POST", np.uint64), tr(l, "SCALES_POST"), normed_p,
                                            H // 32, f"L{l} gate_up input")
            gu = tr(l, "GATE_UP").reshape(B, 2 * I)
            assert_close(gu[rows], mat(p + "mlp.gate_up_proj.weight", 2 * I, H).rows_for(g_codes[rows], g_scales[rows]),
                         f"L{l} gate_up")
            silu = tr(l, "SILU").reshape(B, I)
            assert_close(silu[rows], orc.silu_mul(gu[rows, :I], gu[rows, I:]), f"L{l} silu")
            d_codes, d_scales = check_codes(orc, tr(l, "CODES_DOWN", np.uint64), tr(l, "SCALES_DOWN"), silu, I // 32,
                                            f"L{l} down input")
            down = tr(l, "DOWN").reshape(B, H)
            assert_close(down[rows], mat(p + "mlp.down_proj.weight", H, I).rows_for(d_codes[rows], d_scales[rows]),
                         f"L{l} down")
            nxt = tr(l + 1, "X_IN") if l + 1 < d.n_layers else tr(d.n_layers, "X_FINAL")
            np.testing.assert_array_equal(nxt.reshape(B, H).view(np.uint32), (x_mid + down).view(np.uint32),
                                          err_msg=f"L{l} second residual")
        # final norm and the head
        fl = d.n_layers
        x_fin = tr(fl, "X_FINAL").reshape(B, H)
        hidden = tr(fl, "HIDDEN").reshape(B, H)
        w_fin = tensors["model.language_model.norm.weight"][2].view(np.float32)
        assert_close(hidden[rows], orc.rms_norm(x_fin[rows], w_fin, d.rms_eps, 1.0), "final norm")
        check_codes(orc, tr(fl, "CODES_HEAD", np.uint64), tr(fl, "SCALES_HEAD"), hidden, H // 32, "head input",
                    h128=False)
        emb = tensors["model.language_model.embed_tokens.weight"]
        for r in rows[:1]:  # the oracle's scalar head: ~0.3 s per row
            act1 = orc.q8_quantize_1(hidden[r])
            if emb[0] == 8:
                want = orc.g16_matmul(np.ascontiguousarray(emb[2]).view(orc.G16), act1, V, 1, H // 32)[0]
            else:
                want = orc.dot4_matvec(np.ascontiguousarray(emb[2]).view(orc.Q4X8), act1, V, H // 32)
            err = np.abs(logits[r] - want).max()
            assert err <= 1e-2, f"step {step} row {r}: head logits max-abs {err}"
        assert np.array_equal(toks, np.argmax(logits, axis=1))
        tokens = toks
    rt.set_trace(False)
    rt.close()
