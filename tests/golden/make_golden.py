"""Write the golden vectors in tests/golden/ from the reference build in
oracle/_ref (compiled from the reference's own sources by oracle/Makefile).

Run in the container that has the reference checkout:
    make -C oracle ref && python tests/golden/make_golden.py
Every input is seeded; every expected output comes from a reference function
(or, for the H128 basis, from the reference's own known-answer program
tests/q4_quantizer_test.cpp --basis-fixture).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import q35_oracle as orc  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))
AUTO, SCALAR, AVX2 = 0, 1, 2


def ptr(a):
    return ctypes.c_void_p(a.ctypes.data)


def main():
    assert orc.ref_available(), "build oracle/_ref first: make -C oracle ref"
    r = orc.ref()
    rng = np.random.default_rng(20261201)
    g = {}

    # --- the reference's own H128 known answer (tests/q4_quantizer_test.cpp:12-19)
    txt = subprocess.check_output([os.path.join(orc.REF_DIR, "q4_quantizer_test"), "--basis-fixture"], text=True)
    g["h128_basis_fixture"] = np.array([float(v) for v in txt.split()], np.float32)

    # --- binary16 conversions on a spread of floats incl. subnormals/ties/specials
    f = np.concatenate([rng.standard_normal(2000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 2000),
                        np.array([0.0, -0.0, 65504.0, 65520.0, 6.0e-8, 2.98e-8, 5.96e-8, 1e-10, np.inf, -np.inf],
                                 np.float32)]).astype(np.float32)
    g["half_in"] = f
    g["half_out"] = np.array([r.ref_float_to_half(float(v)) for v in f], np.uint16)

    # --- identity int8 quantization (q4_0.cpp:149-235), scalar semantics
    x = rng.standard_normal((8, 256)).astype(np.float32)
    x[1, :32] = np.linspace(-127, 127, 32, dtype=np.float32) / 2.0  # exact .5 ties
    x[2, :32] = 0.0
    x4 = np.zeros((2, 8), orc.Q8X4)
    r.ref_q8_0_quantize_vectors_4(ptr(x), ptr(x4), 8, 8, SCALAR)
    x1 = np.zeros(8, orc.Q8X1)
    r.ref_q8_0_quantize_vector_1(ptr(x[3]), ptr(x1), 8, SCALAR)
    g["q8_in"], g["q8_x4"], g["q8_x1"] = x, x4, x1

    # --- H128 activation preparation (q4_h128.cpp:259-401), production dispatch
    xh = (rng.standard_normal((8, 1024)) * 2).astype(np.float32)
    h4 = np.zeros((2, 32), orc.Q8X4)
    assert r.ref_q4_h128_prepare_activations_4(ptr(xh), ptr(h4), 8, 1024, orc.SIGN_SEED, AUTO) == 1
    h1 = np.zeros(32, orc.Q8X1)
    assert r.ref_q4_h128_prepare_activation_1(ptr(xh[5]), ptr(h1), 1024, orc.SIGN_SEED, AUTO) == 1
    g["h128_in"], g["h128_x4"], g["h128_x1"] = xh, h4, h1

    # --- DOT4 pack and projections (q4_dot4.cpp), avx2 path = scalar fma order
    rows, blocks = 64, 32
    canon = orc.random_q4_blocks(rng, rows, blocks * 32)
    packed = np.zeros((rows // 8, blocks), orc.Q4X8)
    r.ref_q4_dot4_pack_rows_8(ptr(canon), ptr(packed), rows, blocks)
    mm = np.zeros((8, rows), np.float32)
    r.ref_q4_dot4_matmul(ptr(packed), ptr(h4), ptr(mm), rows, 8, blocks, rows, AVX2)
    mv = np.zeros(rows, np.float32)
    r.ref_q4_dot4_matvec(ptr(packed), ptr(h1), ptr(mv), rows, blocks, AVX2)
    counts = (rng.random(rows) < 0.3).astype(np.int32)
    val, idx = ctypes.c_float(), ctypes.c_uint64()
    r.ref_q4_dot4_argmax(ptr(packed), ptr(h1), ptr(counts), 1.3, 0, rows, blocks, AVX2,
                         ctypes.byref(val), ctypes.byref(idx))
    g["dot4_canon"], g["dot4_packed"], g["dot4_matmul"], g["dot4_matvec"] = canon, packed, mm, mv
    g["dot4_counts"], g["dot4_argmax"] = counts, np.array([idx.value], np.int64)
    g["dot4_argmax_value"] = np.array([val.value], np.float32)

    # --- GatedDeltaNet rows (delta_net.cpp:63-98), production dispatch
    heads, kd, vd = 2, 128, 128
    st = (rng.standard_normal((heads, vd, kd)) * 0.02).astype(np.float32)
    q = rng.standard_normal((heads, kd)).astype(np.float32)
    k = rng.standard_normal((heads, kd)).astype(np.float32)
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    k /= np.linalg.norm(k, axis=1, keepdims=True)
    v = rng.standard_normal((heads, vd)).astype(np.float32)
    al = rng.uniform(0.3, 1.0, heads).astype(np.float32)
    be = rng.uniform(0.0, 1.0, heads).astype(np.float32)
    st2 = st.copy()
    out = np.zeros((heads, vd), np.float32)
    r.ref_gated_delta_net_update_rows(ptr(st2), ptr(q), ptr(k), ptr(v), ptr(al), ptr(be), ptr(out), heads, kd, vd,
                                      0, heads * vd, AUTO)
    g.update(delta_state=st, delta_q=q, delta_k=k, delta_v=v, delta_alpha=al, delta_beta=be,
             delta_state_out=st2, delta_out=out)

    # --- paged GQA attention decode (full_attention.cpp:283-332) over row pointers
    heads, kvh, hd, seq = 8, 2, 256, 40
    keys = rng.standard_normal((seq, kvh * hd)).astype(np.float16).view(np.uint16)
    vals = rng.standard_normal((seq, kvh * hd)).astype(np.float16).view(np.uint16)
    qa = rng.standard_normal(heads * hd).astype(np.float32)
    ga = rng.standard_normal(heads * hd).astype(np.float32)
    krow = (ctypes.c_void_p * seq)(*[keys.ctypes.data + i * keys.strides[0] for i in range(seq)])
    vrow = (ctypes.c_void_p * seq)(*[vals.ctypes.data + i * vals.strides[0] for i in range(seq)])
    scores = np.zeros(heads * seq, np.float32)
    ao = np.zeros(heads * hd, np.float32)
    r.ref_causal_attention_decode_gqa_pairs(ptr(qa), ptr(ga), ctypes.cast(krow, ctypes.c_void_p),
                                            ctypes.cast(vrow, ctypes.c_void_p), ptr(scores), ptr(ao), seq,
                                            heads * hd, kvh * hd, seq, heads, kvh, hd, 1.0 / 16.0, 0, heads // 2,
                                            AUTO)
    g.update(attn_q=qa, attn_gate=ga, attn_keys=keys, attn_values=vals, attn_out=ao)

    # --- activation ops (activation.cpp), production dispatch
    a = rng.standard_normal((4, 256)).astype(np.float32)
    w = rng.standard_normal(256).astype(np.float32) * 0.1
    rn = np.zeros_like(a)
    r.ref_rms_norm_f32(ptr(a), ptr(w), ptr(rn), 4, 256, 1e-6, 1.0, AUTO)
    l2 = a.copy()
    r.ref_l2_normalize_f32(ptr(l2), 4, 128 * 2, 1e-6, 0.0883883476, AUTO)
    sm = np.zeros(256, np.float32)
    r.ref_silu_mul_f32(ptr(a[0]), ptr(a[1]), ptr(sm), 256, AUTO)
    ch, kern = 256, 4
    cstate = rng.standard_normal((kern - 1) * ch).astype(np.float32)
    cw = (rng.standard_normal(kern * ch) * 0.3).astype(np.float32)
    cx = rng.standard_normal(ch).astype(np.float32)
    cst = cstate.copy()
    cout = np.zeros(ch, np.float32)
    r.ref_causal_conv1d_silu_f32(ptr(cst), 2, ptr(cx), ch, ptr(cw), ptr(cout), 1, ch, kern, AUTO)
    rp = a[:2].copy()
    cs = rng.standard_normal(32).astype(np.float32)
    sn = rng.standard_normal(32).astype(np.float32)
    r.ref_rope_f32(ptr(rp), 2, 128, 64, ptr(cs), ptr(sn), AUTO)
    g.update(act_x=a, act_w=w, rms_out=rn, l2_out=l2, silu_mul_out=sm, conv_state=cstate, conv_w=cw, conv_x=cx,
             conv_state_out=cst, conv_out=cout, rope_cos=cs, rope_sin=sn, rope_out=rp)

    np.savez_compressed(os.path.join(OUT, "kernels.npz"), **g)
    print("wrote", os.path.join(OUT, "kernels.npz"), sum(v.nbytes for v in g.values()), "bytes")


if __name__ == "__main__":
    main()
